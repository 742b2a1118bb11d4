"""GPU parity of the wave-K kernels (32 x 32 or 16 x 16 output tiles, K split
over the workgroup's waves, operands streamed straight into MFMA registers)
forced onto conv and Gemm shapes through spinn_hip_tune_force_tiles(ts, ts, 0)
for both tile edges: every
B-operand gather (1x1 pointwise, tap-ordered, (c,kh,kw) with 1x1 / 3x3 / 7x7 /
runtime windows), the raw-weight (16-byte k loads) and packed-weight A paths,
groups, ragged M / N / K edges, every fused post-op; Gemm in all transpose
combinations with 16-byte and scalar k loads, both C forms and batches.
Against the oracle and float64, absolute tolerance."""
import ctypes as C
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import conv_desc, run_conv, run_gemm

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[32, 16], ids=["ts32", "ts16"])
def force_wavek(hip, request):
    L = hip.lib()
    L.spinn_hip_tune_force_tiles(request.param, request.param, 0)
    try:
        yield request.param
    finally:
        L.spinn_hip_tune_force_tiles(0, 0, 0)


# (name, n, c, h, w, oc, k, stride, pad, group, act)
CONV = [
    ("pw_1x1_add_relu", 1, 256, 14, 14, 1024, 1, 1, 0, 1, 5),
    ("pw_1x1_k2048", 1, 2048, 7, 7, 512, 1, 1, 0, 1, 1),
    ("pw_ragged", 3, 20, 6, 10, 37, 1, 1, 0, 1, 3),           # K 20, M 37, N 180
    ("pw_grouped", 2, 64, 8, 8, 64, 1, 1, 0, 2, 4),
    ("tap_3x3", 1, 64, 56, 56, 64, 3, 1, 1, 1, 1),            # the Conv3x3+BN+ReLU layer
    ("tap_3x3_s2", 1, 128, 28, 28, 128, 3, 2, 1, 1, 1),
    ("tap_3x3_c512_7x7", 1, 512, 7, 7, 512, 3, 1, 1, 1, 5),
    ("tap_grouped", 2, 64, 14, 14, 64, 3, 1, 1, 4, 1),        # 16 channels per group
    ("gather_3x3_c3", 1, 3, 17, 19, 83, 3, 1, 1, 1, 3),
    ("gather_7x7_stem", 1, 3, 64, 64, 64, 7, 2, 3, 1, 1),
    ("gather_1x1_s2", 2, 24, 28, 28, 40, 1, 2, 0, 1, 0),      # strided 1x1: not the pointwise gather
    ("gather_5x5", 1, 8, 19, 21, 12, 5, 1, 2, 1, 2),          # runtime window, CLIP
    ("gather_3x3_c40", 1, 40, 20, 20, 48, 3, 1, 1, 1, 5),     # 40 channels: (c,kh,kw) order
]


@pytest.mark.parametrize("case", CONV, ids=[c[0] for c in CONV])
def test_wavek_conv(hip, torch_gpu, force_wavek, case):
    name, n, c, h, w, oc, k, s, p, g, act = case
    print(f"[wavek conv ts{force_wavek}] {name}", flush=True)
    d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, g, act, hip.ALGO_IMPLICIT_GEMM)
    assert hip.lib().spinn_hip_conv_workspace_size(C.byref(d)) == 0
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c // g, k, k)) * np.sqrt(2.0 / (c // g * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, d.oh, d.ow)).astype(np.float32) if act in (4, 5) else None
    y, _ = run_conv(hip, torch_gpu, d, x, wt, b, r)
    od = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
    assert_parity(y, O.conv2d(od, x, wt, b, r), what=f"wavek {name} vs oracle")
    assert_parity(y, O.conv2d_f64(od, x, wt, b, r), what=f"wavek {name} vs float64")


@pytest.mark.parametrize("mnk", [(1, 1000, 2048), (32, 1000, 2048), (3136, 256, 64), (784, 512, 128),
                                 (196, 1024, 256)], ids=str)
def test_wavek_gemm_sweep(hip, torch_gpu, force_wavek, mnk):
    m, n, k = mnk
    rng = np.random.default_rng(m * 7 + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    c = rng.normal(0, 0.01, n).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, c, trans_b=1)
    assert_parity(y, O.gemm(a, b, c, trans_b=1), what=f"wavek gemm {mnk} vs oracle")
    assert_parity(y, O.gemm_f64(a, b, c, trans_b=1), what=f"wavek gemm {mnk} vs float64")


@pytest.mark.parametrize("k", [29, 64, 300], ids=["k29_scalar", "k64", "k300"])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("cmode", [0, 1, 2])
def test_wavek_gemm_transposes(hip, torch_gpu, force_wavek, ta, tb, cmode, k):
    m, n = 37, 45
    rng = np.random.default_rng(200 + 4 * ta + 2 * tb + cmode + k)
    a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if tb else (k, n)).astype(np.float32)
    c = None if cmode == 0 else rng.uniform(-1, 1, n if cmode == 1 else (m, n)).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb)
    assert_parity(y, O.gemm_f64(a, b, c, alpha=0.5, beta=2.0, trans_a=ta, trans_b=tb), what="vs float64")


def test_wavek_matmul_batched(hip, torch_gpu, force_wavek):
    bt, m, n, k = 3, 33, 40, 72
    rng = np.random.default_rng(19)
    a = rng.uniform(-1, 1, (bt, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (bt, k, n)).astype(np.float32)
    y = run_gemm(hip, torch_gpu, a, b, alpha=1.0, beta=0.0, batch=bt)
    assert_parity(y, O.matmul(a, b), what="wavek batched matmul vs oracle")


def test_wavek_repeats_bit_identical(hip, torch_gpu, force_wavek):
    """The cross-wave sum runs in a fixed order: repeated calls are bit-identical."""
    n, c, h, w, oc = 1, 1024, 14, 14, 256
    d = conv_desc(hip, n, c, h, w, oc, 1, 1, 1, 1, 0, 0, 1, 1, hip.ALGO_IMPLICIT_GEMM)
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, 1, 1)) * np.sqrt(2.0 / c)).astype(np.float32)
    outs = [run_conv(hip, torch_gpu, d, x, wt)[0] for _ in range(3)]
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("case", [("pw_packed_only", 1, 256, 14, 14, 512, 1, 1, 0, 1, 5),
                                  ("tap_packed_only", 1, 64, 28, 28, 96, 3, 1, 1, 1, 1)], ids=lambda c: c[0])
def test_wavek_conv_packed_weights_only(hip, torch_gpu, force_wavek, case):
    """Without the raw weights (w = NULL) the kernel reads the packed W^T layout
    (tap-ordered for 16-channel multiples) instead of 16-byte loads along k."""
    name, n, c, h, w, oc, k, s, p, g, act = case
    torch = torch_gpu
    L = hip.lib()
    d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, g, act, hip.ALGO_IMPLICIT_GEMM)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c // g, k, k)) * np.sqrt(2.0 / (c // g * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, d.oh, d.ow)).astype(np.float32) if act in (4, 5) else None
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
    xd, wd, bd, rd = dev(x), dev(wt), dev(b), dev(r)
    pk = torch.empty(L.spinn_hip_conv_packed_size(C.byref(d)) // 4, device="cuda")
    hip.check(L.spinn_hip_conv_pack_weights(C.byref(d), hip.ptr(wd), hip.ptr(pk), None), "pack")
    y = torch.full((n, oc, d.oh, d.ow), float("nan"), device="cuda")
    hip.check(L.spinn_hip_conv(C.byref(d), hip.ptr(xd), None, hip.ptr(pk), hip.ptr(bd), hip.ptr(rd), hip.ptr(y),
                               None, 0, None), "conv")
    torch.cuda.synchronize()
    od = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
    assert_parity(y.cpu().numpy(), O.conv2d(od, x, wt, b, r), what=f"wavek {name} vs oracle")
