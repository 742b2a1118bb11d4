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


def _out(torch, shape, offset=0):
    """A NaN-filled device buffer of `shape`; offset > 0 starts it `offset`
    floats into a larger allocation (a pointer that is not 16-byte aligned)."""
    n = int(np.prod(shape))
    base = torch.full((n + offset,), float("nan"), device="cuda", dtype=torch.float32)
    return base[offset:].view(*shape) if len(shape) else base[offset:]


def _in(torch, a, offset=0):
    a = np.ascontiguousarray(a, np.float32)
    t = _out(torch, a.shape, offset)
    t.copy_(torch.from_numpy(a))
    return t


def _done(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_binary(N, torch, op, a, b, out_shape, offset=0):
    ad, bd = _in(torch, a, offset), _in(torch, b, offset)
    yd = _out(torch, out_shape, offset)
    rc = N.lib().spinn_hip_binary(op, _p(ad), a.size, _p(bd), b.size, _p(yd), int(np.prod(out_shape)), None)
    N.check(rc, "spinn_hip_binary")
    return _done(torch, yd)


def run_unary(N, torch, op, x, offset=0):
    xd = _in(torch, x, offset)
    yd = _out(torch, x.shape, offset)
    N.check(N.lib().spinn_hip_unary(op, _p(xd), _p(yd), x.size, None), "spinn_hip_unary")
    return _done(torch, yd)


def run_batchnorm(N, torch, x, scale, bias, mean, var, eps, offset=0):
    xd = _in(torch, x, offset)
    sd, bd, md, vd = (_in(torch, v) for v in (scale, bias, mean, var))
    yd = _out(torch, x.shape, offset)
    spatial = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    rc = N.lib().spinn_hip_batchnorm(x.shape[0], x.shape[1], spatial, _p(xd), _p(sd), _p(bd), _p(md), _p(vd), eps,
                                     _p(yd), None)
    N.check(rc, "spinn_hip_batchnorm")
    return _done(torch, yd)


def run_softmax(N, torch, x, axis):
    axis %= x.ndim
    xd = _in(torch, x)
    yd = _out(torch, x.shape)
    outer, inner = int(np.prod(x.shape[:axis])), int(np.prod(x.shape[axis + 1:]))
    N.check(N.lib().spinn_hip_softmax(outer, x.shape[axis], inner, _p(xd), _p(yd), None), "spinn_hip_softmax")
    return _done(torch, yd)


def _blocks(N, pieces):
    arr = (N.BlockCopy * len(pieces))()
    for i, (src, dst, src_row, src_off, dst_row, dst_off, ln) in enumerate(pieces):
        arr[i] = N.BlockCopy(src.data_ptr(), dst.data_ptr(), src_row, src_off, dst_row, dst_off, ln)
    return arr


def run_concat(N, torch, xs, axis, offset=0):
    """Concat as op_concat lays it out: one block copy per input."""
    axis %= xs[0].ndim
    outer, inner = int(np.prod(xs[0].shape[:axis])), int(np.prod(xs[0].shape[axis + 1:]))
    shape = list(xs[0].shape)
    shape[axis] = sum(x.shape[axis] for x in xs)
    yd = _out(torch, shape, offset)
    row = shape[axis] * inner
    devs, pieces, off = [], [], 0
    for x in xs:
        xd = _in(torch, x, offset)
        devs.append(xd)
        ln = x.shape[axis] * inner
        pieces.append((xd, yd, ln, 0, row, off, ln))
        off += ln
    N.check(N.lib().spinn_hip_block_copy(_blocks(N, pieces), len(pieces), outer, None), "spinn_hip_block_copy")
    return _done(torch, yd)


def run_split(N, torch, x, sizes, axis):
    axis %= x.ndim
    outer, inner = int(np.prod(x.shape[:axis])), int(np.prod(x.shape[axis + 1:]))
    xd = _in(torch, x)
    row = x.shape[axis] * inner
    ys, pieces, off = [], [], 0
    for s in sizes:
        shape = list(x.shape)
        shape[axis] = s
        yd = _out(torch, shape)
        ys.append(yd)
        pieces.append((xd, yd, row, off, s * inner, 0, s * inner))
        off += s * inner
    N.check(N.lib().spinn_hip_block_copy(_blocks(N, pieces), len(pieces), outer, None), "spinn_hip_block_copy")
    return [_done(torch, y) for y in ys]


def run_transpose(N, torch, x, perm):
    xd = _in(torch, x)
    yd = _out(torch, [x.shape[p] for p in perm] if perm is not None else x.shape[::-1])
    dims = (C.c_int64 * x.ndim)(*x.shape)
    pm = (C.c_int32 * x.ndim)(*perm) if perm is not None else None
    N.check(N.lib().spinn_hip_transpose(x.ndim, dims, pm, _p(xd), _p(yd), None), "spinn_hip_transpose")
    return _done(torch, yd)


def run_resize(N, torch, x, oh, ow, offset=0):
    n, c, h, w = x.shape
    xd = _in(torch, x, offset)
    yd = _out(torch, (n, c, oh, ow))
    N.check(N.lib().spinn_hip_resize_nearest(n * c, h, w, oh, ow, _p(xd), _p(yd), None), "spinn_hip_resize_nearest")
    return _done(torch, yd)


def run_reduce_mean(N, torch, x, outer, dim, inner, offset=0):
    xd = _in(torch, x, offset)
    yd = _out(torch, (outer * inner,))
    N.check(N.lib().spinn_hip_reduce_mean(outer, dim, inner, _p(xd), _p(yd), None), "spinn_hip_reduce_mean")
    return _done(torch, yd)


def run_maxpool(N, torch, x, oh, ow, kh, kw, sh, sw, ph, pw):
    n, c, h, w = x.shape
    xd = _in(torch, x)
    yd = _out(torch, (n, c, oh, ow))
    d = N.PoolDesc(n, c, h, w, oh, ow, kh, kw, sh, sw, ph, pw)
    N.check(N.lib().spinn_hip_maxpool2d(C.byref(d), _p(xd), _p(yd), None), "spinn_hip_maxpool2d")
    return _done(torch, yd)
