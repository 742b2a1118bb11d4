"""Calls into the HIP C ABI with torch-allocated device buffers (test helper)."""
from __future__ import annotations

import ctypes as C

import numpy as np


def _dev(torch, a):
    if a is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def conv_desc(N, n, c, h, w, oc, kh, kw, sh=1, sw=1, ph=0, pw=0, group=1, act=0, algo=0, oh=None, ow=None):
    if oh is None:
        oh = (h + 2 * ph - kh) // sh + 1
    if ow is None:
        ow = (w + 2 * pw - kw) // sw + 1
    d = N.ConvDesc(n, c, h, w, oc, oh, ow, kh, kw, sh, sw, ph, pw, group, act, algo, 0)
    return d


def run_conv(N, torch, d, x, w, bias=None, res=None):
    """Pack weights, size the workspace, run spinn_hip_conv; returns (y, algo)."""
    L = N.lib()
    algo = L.spinn_hip_conv_select_algo(C.byref(d))
    assert algo > 0, algo
    d.algo = algo
    xd, wd, bd, rd = _dev(torch, x), _dev(torch, w), _dev(torch, bias), _dev(torch, res)
    yd = torch.full((d.n, d.oc, d.oh, d.ow), float("nan"), device="cuda", dtype=torch.float32)
    psz = L.spinn_hip_conv_packed_size(C.byref(d))
    pk = None
    if psz:
        pk = torch.empty(psz // 4, device="cuda", dtype=torch.float32)
        N.check(L.spinn_hip_conv_pack_weights(C.byref(d), _p(wd), _p(pk), None), "pack")
    wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
    ws = torch.empty(max(wsz // 4, 1), device="cuda", dtype=torch.float32) if wsz else None
    rc = L.spinn_hip_conv(C.byref(d), _p(xd), _p(wd), _p(pk), _p(bd), _p(rd), _p(yd), _p(ws), wsz, None)
    N.check(rc, "spinn_hip_conv")
    torch.cuda.synchronize()
    return yd.cpu().numpy(), algo


def run_gemm(N, torch, a, b, c=None, alpha=1.0, beta=1.0, trans_a=0, trans_b=0, batch=1):
    """spinn_hip_gemm on numpy operands (batched when batch > 1: a, b have a leading batch axis)."""
    L = N.lib()
    if batch > 1:
        m = a.shape[2] if trans_a else a.shape[1]
        k = a.shape[1] if trans_a else a.shape[2]
        n = b.shape[1] if trans_b else b.shape[2]
    else:
        m = a.shape[1] if trans_a else a.shape[0]
        k = a.shape[0] if trans_a else a.shape[1]
        n = b.shape[0] if trans_b else b.shape[1]
    c_mode = 0
    if c is not None:
        c_mode = 1 if c.size == n else 2
    d = N.GemmDesc(m, n, k, trans_a, trans_b, c_mode, alpha, beta, batch, 0,
                   m * k if batch > 1 else 0, k * n if batch > 1 else 0, m * n if batch > 1 else 0)
    ad, bd, cd = _dev(torch, a), _dev(torch, b), _dev(torch, c)
    shape = (batch, m, n) if batch > 1 else (m, n)
    yd = torch.full(shape, float("nan"), device="cuda", dtype=torch.float32)
    wsz = L.spinn_hip_gemm_workspace_size(C.byref(d))
    ws = torch.empty(max(wsz // 4, 1), device="cuda", dtype=torch.float32) if wsz else None
    N.check(L.spinn_hip_gemm(C.byref(d), _p(ad), _p(bd), _p(cd), _p(yd), _p(ws), wsz, None), "spinn_hip_gemm")
    torch.cuda.synchronize()
    return yd.cpu().numpy()
