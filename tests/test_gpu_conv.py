"""GPU parity of spinn_hip_conv against the oracle (restated SPINN conv, fp32)
and the float64 closed form, through the C ABI.

Shapes cover every kernel path: tap-ordered implicit GEMM (C/g % 16 == 0),
the (c,kh,kw) gather for small channel counts, 1x1 stride 1/2, split-K for
small grids, grouped implicit GEMM, the direct (depthwise) kernel and
Winograd F(2x2,3x3) / F(4x4,3x3), with each fused post-op code (none, ReLU,
CLIP, SiLU, Add, Add+ReLU). Every case is held to the absolute bound.
"""
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import conv_desc, run_conv

pytestmark = pytest.mark.gpu

# (name, n, c, h, w, oc, k, stride, pad, group, act, algo)
CASES = [
    ("cfg0_conv3x3_relu", 1, 64, 56, 56, 64, 3, 1, 1, 1, 1, 0),
    ("stem7x7_s2", 2, 3, 64, 64, 64, 7, 2, 3, 1, 1, 0),
    ("pw1x1_add_relu", 2, 256, 14, 14, 1024, 1, 1, 0, 1, 5, 0),
    ("pw1x1_s2_none", 2, 256, 28, 28, 512, 1, 2, 0, 1, 0, 0),
    ("pw1x1_ragged_k", 3, 20, 6, 10, 37, 1, 1, 0, 1, 3, 0),     # float4 pixel runs, K tail, images inside a tile
    ("pw1x1_grouped", 2, 64, 8, 8, 64, 1, 1, 0, 2, 1, 0),
    ("pw1x1_splitk", 1, 1024, 7, 8, 256, 1, 1, 0, 1, 5, 0),
    ("pw1x1_odd_plane", 2, 64, 7, 7, 96, 1, 1, 0, 1, 1, 0),     # 49-pixel planes: gather loader
    ("oc16_3x3_32row_tile", 2, 16, 40, 40, 16, 3, 1, 1, 1, 3, 0),   # <= 32 output channels: 32 x 128 tiles
    ("oc32_pw_add_relu", 2, 48, 20, 20, 32, 1, 1, 0, 1, 5, 0),
    ("stem_c3_oc16_s2", 2, 3, 64, 64, 16, 3, 2, 1, 1, 3, 0),
    ("oc24_splitk", 1, 512, 7, 7, 24, 3, 1, 1, 1, 1, 0),
    ("stem3x3_direct", 2, 3, 64, 64, 16, 3, 2, 1, 1, 3, 3),        # few-input-channel stem kernel
    ("stem7x7_direct", 1, 3, 40, 40, 64, 7, 2, 3, 1, 1, 3),
    # 7x7 stride-2 stems on the row-per-workgroup MFMA kernel (LDS-staged window)
    ("stem7x7_224_res", 2, 3, 224, 224, 64, 7, 2, 3, 1, 5, 0),         # ResNet stem shape, residual + ReLU
    ("stem7x7_224_b1_split", 1, 3, 224, 224, 64, 7, 2, 3, 1, 1, 0),    # 112 rows: two workgroups per row
    ("stem7x7_c1_oc40_ragged", 3, 1, 37, 45, 40, 7, 2, 3, 1, 3, 0),   # one channel, 40 of 64 rows, 23-pixel rows
    ("stem7x7_c4_ow128", 1, 4, 30, 256, 64, 7, 2, 3, 1, 1, 0),         # four channels, 128-pixel rows
    ("stem7x7_oc24_few_rows", 1, 3, 56, 56, 24, 7, 2, 3, 1, 1, 0),     # 28 rows, one channel block: no row split
    ("stem7x7_ow129_fallback", 1, 3, 9, 258, 64, 7, 2, 3, 1, 1, 0),    # 129-pixel rows: generic implicit GEMM
    # stem epilogue: bias from LDS, residual loads batched (no-residual and residual variants)
    ("stem7x7_224_b8", 8, 3, 224, 224, 64, 7, 2, 3, 1, 1, 0),          # 896 rows
    ("stem7x7_c2_res_ragged", 24, 2, 48, 90, 48, 7, 2, 3, 1, 5, 0),    # 576 rows of 45 pixels, 48 channels
    ("stem7x7_c1_oc40_silu", 34, 1, 64, 64, 40, 7, 2, 3, 1, 3, 0),     # 1088 rows of 32 pixels, SiLU
    ("stem_c1_direct_oc20_res", 1, 1, 33, 35, 20, 3, 1, 1, 1, 5, 3),  # partial 16-channel chunk, residual
    # 3x3 stride-2 stems on the row-per-workgroup 16x16x4 MFMA kernel (rows <= 320 pixels,
    # grids of at least 4 rows per CU: 1024 rows on 256 CUs)
    ("stem3_mfma_640_b4", 4, 3, 640, 640, 16, 3, 2, 1, 1, 3, 3),      # YOLOv10n stem shape, 320-pixel rows
    ("stem3_mfma_c1_oc5_res", 64, 1, 33, 47, 5, 3, 2, 1, 1, 5, 3),    # one channel, 5 of 16 rows, residual
    ("stem3_mfma_c4_pad0", 56, 4, 40, 66, 16, 3, 2, 0, 1, 1, 3),      # four channels, no padding
    ("stem3_mfma_c2_oc12_odd", 96, 2, 21, 29, 12, 3, 2, 1, 1, 0, 3),  # two channels, 11 x 15 outputs
    ("stem3_fma_640_b1", 1, 3, 640, 640, 16, 3, 2, 1, 1, 3, 3),       # 320 rows: the FMA stem kernel
    ("stem3_fma_ow321_fallback", 1, 3, 8, 642, 16, 3, 2, 1, 1, 3, 3), # 321-pixel rows: the FMA stem kernel
    # AUTO's small-grid choices: 16 x 16 wave-K tiles for a 3x3 gather with K 1152 over 200 tiles and for
    # 1x1 convs with K 64 / 128; F(2x2,3x3) for 512 channels over 16 4x4 tiles
    ("auto_wavek16_3x3_k1152", 1, 128, 20, 20, 128, 3, 1, 1, 1, 3, 0),
    ("auto_wavek16_1x1_k64", 1, 64, 40, 40, 64, 1, 1, 0, 1, 3, 0),
    ("auto_wavek16_1x1_k128_add", 1, 128, 20, 20, 128, 1, 1, 0, 1, 4, 0),
    ("auto_f23_c512_b4", 4, 512, 7, 7, 512, 3, 1, 1, 1, 1, 0),
    ("direct_group1_general", 1, 6, 10, 12, 5, 3, 1, 1, 1, 1, 3),      # C > 4: general direct kernel
    ("conv3x3_s2", 2, 128, 28, 28, 128, 3, 2, 1, 1, 1, 0),
    ("ragged_silu_c3", 1, 3, 17, 19, 83, 3, 1, 1, 1, 3, 0),
    ("add_only", 1, 32, 9, 11, 48, 3, 1, 1, 1, 4, 0),
    ("splitk_7x7grid", 1, 512, 7, 7, 512, 3, 1, 1, 1, 1, 0),
    ("gemm_grouped", 2, 64, 14, 14, 64, 3, 1, 1, 4, 1, 0),
    ("depthwise_s2_silu", 2, 32, 20, 20, 32, 3, 2, 1, 32, 3, 0),
    ("depthwise7x7", 1, 24, 20, 20, 24, 7, 1, 3, 24, 3, 0),
    ("depthwise_add_pe", 2, 128, 20, 20, 128, 3, 1, 1, 128, 4, 0),   # PSA pe conv: residual fused
    ("depthwise_ragged_s1", 3, 16, 37, 45, 16, 3, 1, 1, 16, 1, 0),   # tiles past the plane edge
    ("depthwise5x5_s1", 1, 8, 19, 70, 8, 5, 1, 2, 8, 0, 0),
    ("depthwise_s2_ragged", 2, 12, 41, 67, 12, 3, 2, 1, 12, 3, 0),
    ("depthwise_large_plane", 1, 4, 160, 161, 4, 3, 1, 1, 4, 1, 0),   # 5 x 6 tiles, ragged right edge
    ("depthwise_tiny_planes", 4, 96, 7, 5, 96, 3, 1, 1, 96, 4, 0),    # 384 planes of one partial tile, residual
    ("grouped_direct_cg2", 1, 16, 12, 12, 8, 3, 1, 1, 8, 1, 0),      # two input channels per group: general kernel
    # one wave per plane and run of row bands (4-pixel quads across the row, neighbours by lane permute)
    ("dw_wave_w256", 1, 8, 9, 256, 8, 3, 1, 1, 8, 3, 0),              # 64 quads: one band per wave
    ("dw_wave_w252_rows_ragged", 2, 4, 14, 252, 4, 3, 1, 1, 4, 1, 0), # 63 quads, last band 2 rows
    ("dw_wave_5x5_w36", 2, 16, 13, 36, 16, 5, 1, 2, 16, 0, 0),       # 9 quads: 7 bands per wave
    ("dw_wave_7x7_w44_res", 2, 8, 11, 44, 8, 7, 1, 3, 8, 4, 0),      # 11 quads, residual fused
    ("dw_wave_s2_w84", 3, 16, 27, 84, 16, 3, 2, 1, 16, 1, 0),        # 42-wide output: scalar stores, half-empty last quad
    ("dw_wave_s2_w200_add_relu", 1, 8, 10, 200, 8, 3, 2, 1, 8, 5, 0),
    ("dw_wave_80x80_silu", 2, 20, 80, 80, 20, 3, 1, 1, 20, 3, 0),    # YOLOv10n plane: 3 bands per wave
    ("dw_fallback_w260", 1, 4, 6, 260, 4, 3, 1, 1, 4, 1, 0),         # 65 quads: per-thread kernel
    ("winograd_add_relu", 2, 64, 28, 28, 64, 3, 1, 1, 1, 5, 2),
    ("winograd_odd", 1, 16, 15, 13, 8, 3, 1, 1, 1, 1, 2),
    ("winograd_c256", 1, 256, 14, 14, 256, 3, 1, 1, 1, 1, 2),
    ("winograd43_add_relu", 2, 64, 28, 28, 64, 3, 1, 1, 1, 5, 4),   # F(4x4,3x3)
    ("winograd43_odd", 1, 16, 15, 13, 8, 3, 1, 1, 1, 1, 4),          # partial 4x4 tiles at both edges
    ("winograd43_c256", 1, 256, 14, 14, 256, 3, 1, 1, 1, 1, 4),
    ("winograd43_c512_add", 2, 512, 7, 7, 512, 3, 1, 1, 1, 4, 4),
    ("winograd43_p0_silu", 1, 8, 10, 12, 40, 3, 1, 0, 1, 3, 4),      # no padding: 8x10 output
    ("winograd43_batch5_c3_add", 5, 3, 9, 11, 7, 3, 1, 1, 1, 4, 4),   # a 64-tile group spans 7 images
    ("winograd43_batch3_res", 3, 12, 20, 24, 20, 3, 1, 1, 1, 5, 4),    # residual + ReLU, 30 tiles per image
    ("winograd43_large_plane", 1, 4, 126, 126, 6, 3, 1, 1, 1, 1, 4),   # 32 x 32 tiles per plane
    # act 2 (CLIP) is a declared code that applies nothing (SPINN/graph_opt.h:33)
    ("clip_conv3x3", 2, 64, 14, 14, 64, 3, 1, 1, 1, 2, 0),
    ("clip_pw1x1_splitk", 1, 1024, 7, 8, 256, 1, 1, 0, 1, 2, 0),
    ("clip_winograd43", 1, 128, 28, 28, 128, 3, 1, 1, 1, 2, 4),
    ("clip_depthwise", 1, 32, 20, 20, 32, 3, 1, 1, 32, 2, 0),
]


def _inputs(seed, n, c, h, w, oc, k, group, act, oh, ow):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c // group, k, k)) * np.sqrt(2.0 / (c // group * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, oh, ow)).astype(np.float32) if act in (4, 5) else None
    return x, wt, b, r


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_conv_parity(hip, torch_gpu, case):
    name, n, c, h, w, oc, k, s, p, g, act, algo = case
    print(f"[conv] {name}", flush=True)
    d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, g, act, algo)
    x, wt, b, r = _inputs(zlib.crc32(name.encode()), n, c, h, w, oc, k, g, act, d.oh, d.ow)
    y, used = run_conv(hip, torch_gpu, d, x, wt, b, r)
    od = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
    ref = O.conv2d(od, x, wt, b, r)
    assert_parity(y, ref, what=f"{name} (algo {used}) vs oracle")
    assert_parity(y, O.conv2d_f64(od, x, wt, b, r), what=f"{name} vs float64")


def test_conv_no_bias_raw_accumulator(hip, torch_gpu):
    """act NONE, no bias: the raw accumulator the reference's packed path returns."""
    n, c, h, w, oc = 2, 64, 12, 12, 96
    d = conv_desc(hip, n, c, h, w, oc, 3, 3, 1, 1, 1, 1)
    x, wt, _, _ = _inputs(7, n, c, h, w, oc, 3, 1, 0, d.oh, d.ow)
    y, _ = run_conv(hip, torch_gpu, d, x, wt)
    ref = O.conv2d(O.conv_desc(n, c, h, w, oc, 3, 3, 1, 1, 1, 1), x, wt, as_shipped=True)
    assert_parity(y, ref, what="raw accumulator")


def test_conv_bad_args(hip):
    import ctypes as C
    L = hip.lib()
    d = conv_desc(hip, 1, 6, 8, 8, 4, 3, 3, group=4)  # C not divisible by group
    assert L.spinn_hip_conv_select_algo(C.byref(d)) == hip.SPINN_HIP_EINVAL
    d = conv_desc(hip, 1, 8, 8, 8, 8, 3, 3, act=5)
    # residual required for ADD_RELU
    rc = L.spinn_hip_conv(C.byref(d), C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), None, None, C.c_void_p(16),
                          None, 0, None)
    assert rc == hip.SPINN_HIP_EINVAL


@pytest.mark.parametrize("shape", [(1, 1024, 7, 8, 256, 1, 0, 5), (1, 512, 7, 7, 512, 3, 1, 1)],
                         ids=["pw1x1_splitk", "conv3x3_splitk"])
def test_splitk_repeats_bit_identical(hip, torch_gpu, shape):
    """Split-K sums its partials in a fixed order: repeated calls on one workspace
    (left holding the previous call's partials) give bit-identical outputs."""
    import ctypes as C
    torch = torch_gpu
    n, c, h, w, oc, k, p, act = shape
    L = hip.lib()
    d = conv_desc(hip, n, c, h, w, oc, k, k, 1, 1, p, p, 1, act, hip.ALGO_IMPLICIT_GEMM)
    L.spinn_hip_tune_force_tiles(64, 64, 4)  # 64 x 64 tiles, K split 4 ways over workgroups
    try:
        _splitk_repeats(hip, torch, L, d, shape)
    finally:
        L.spinn_hip_tune_force_tiles(0, 0, 0)


def _splitk_repeats(hip, torch, L, d, shape):
    import ctypes as C
    n, c, h, w, oc, k, p, act = shape
    wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
    assert wsz > 0, "shape no longer splits K; pick one that does"
    x, wt, b, r = _inputs(11, n, c, h, w, oc, k, 1, act, d.oh, d.ow)
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
    xd, wd, bd, rd = dev(x), dev(wt), dev(b), dev(r)
    pk = torch.empty(L.spinn_hip_conv_packed_size(C.byref(d)) // 4, device="cuda")
    hip.check(L.spinn_hip_conv_pack_weights(C.byref(d), hip.ptr(wd), hip.ptr(pk), None), "pack")
    ws = torch.full((wsz // 4,), float("nan"), device="cuda", dtype=torch.float32)
    ref = O.conv2d(O.conv_desc(n, c, h, w, oc, k, k, 1, 1, p, p, 1, act), x, wt, b, r)
    outs = []
    for i in range(3):
        y = torch.full((n, oc, d.oh, d.ow), float("nan"), device="cuda")
        hip.check(L.spinn_hip_conv(C.byref(d), hip.ptr(xd), hip.ptr(wd), hip.ptr(pk), hip.ptr(bd), hip.ptr(rd),
                                   hip.ptr(y), hip.ptr(ws), wsz, None), "conv")
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        assert_parity(outs[-1], ref, what=f"split-K call {i}")
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
