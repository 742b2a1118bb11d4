"""F(4x4,3x3) Winograd in one launch (wino4_fused_kernel): input transform into LDS,
the 36 component GEMMs on MFMA with the accumulators in registers, output transform
and epilogue from LDS, no workspace. Checked against the oracle (restated SPINN conv,
SPINN/run_time/ops/conv/conv2d.c:92-232) and float64, with the three-launch F(4x4,3x3)
path on the same shapes, over ragged channel counts (a partial last 4-channel slice),
output channels not a multiple of 32, fewer than 32 tiles, pads 0 and 2, rows that
take the float4 and the scalar stores, residual, ReLU and SiLU; plus the full-size
ResNet-101 and YOLOv10n layers, bit-identical repeats and the workspace query."""
import ctypes as C
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import conv_desc, run_conv

pytestmark = pytest.mark.gpu

F43 = 4  # SPINN_CONV_ALGO_WINOGRAD_F43

# (name, n, c, h, w, oc, pad, act)
CASES = [
    ("c64_28_add_relu", 2, 64, 28, 28, 64, 1, 5),
    ("c16_odd_15x13_oc8", 1, 16, 15, 13, 8, 1, 1),        # partial tiles at both edges, scalar stores
    ("c6_ragged_slice_oc40", 3, 6, 12, 16, 40, 1, 0),     # C % 4 != 0, two channel blocks (second partial)
    ("c5_p0_silu", 1, 5, 10, 12, 33, 0, 3),               # no padding: 8x10 output
    ("c3_p2_add", 2, 3, 9, 11, 7, 2, 4),                  # pad 2: 11x13 output, residual, no post-op
    ("c128_28_relu", 2, 128, 28, 28, 128, 1, 1),
    ("c32_tiles_lt_32", 1, 32, 8, 8, 64, 1, 1),           # 4 tiles: one partial workgroup
    ("c40_80x80_silu", 1, 40, 80, 80, 48, 1, 3),          # 400 tiles per image
    ("c1_single_channel", 2, 1, 17, 20, 16, 1, 1),
]


def _inputs(seed, n, c, h, w, oc, act, oh, ow):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, 3, 3)) * np.sqrt(2.0 / (c * 9))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, oh, ow)).astype(np.float32) if act in (4, 5) else None
    return x, wt, b, r


@pytest.fixture
def fused_mode(hip):
    L = hip.lib()
    yield L.spinn_hip_tune_winograd_fused
    L.spinn_hip_tune_winograd_fused(-1)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_parity_and_three_launch(hip, torch_gpu, fused_mode, case):
    name, n, c, h, w, oc, p, act = case
    print(f"[wino fused] {name}", flush=True)
    L = hip.lib()
    d = conv_desc(hip, n, c, h, w, oc, 3, 3, 1, 1, p, p, 1, act, F43)
    x, wt, b, r = _inputs(zlib.crc32(name.encode()), n, c, h, w, oc, act, d.oh, d.ow)
    od = O.conv_desc(n, c, h, w, oc, 3, 3, 1, 1, p, p, 1, act)
    ref = O.conv2d(od, x, wt, b, r)
    ref64 = O.conv2d_f64(od, x, wt, b, r)
    fused_mode(1)
    assert L.spinn_hip_conv_workspace_size(C.byref(d)) == 0, "the fused kernel needs no workspace"
    y1, _ = run_conv(hip, torch_gpu, d, x, wt, b, r)
    y1b, _ = run_conv(hip, torch_gpu, d, x, wt, b, r)
    assert np.array_equal(y1, y1b), "fused launches are deterministic"
    assert_parity(y1, ref, what=f"{name} fused vs oracle")
    assert_parity(y1, ref64, what=f"{name} fused vs float64")
    fused_mode(0)
    assert L.spinn_hip_conv_workspace_size(C.byref(d)) > 0
    y3, _ = run_conv(hip, torch_gpu, d, x, wt, b, r)
    assert_parity(y1, y3, what=f"{name} fused vs three launches")


@pytest.mark.parametrize("shape", [(32, 64, 56, 56, 64, 1), (8, 32, 160, 160, 32, 3), (32, 128, 28, 28, 128, 1)],
                         ids=["resnet101_b32_64c_56", "yolov10n_b8_32c_160", "resnet101_b32_128c_28"])
def test_fused_full_size_layers(hip, torch_gpu, fused_mode, shape):
    """The full-size layers the per-shape rule sends to the fused kernel."""
    n, c, h, w, oc, act = shape
    print(f"[wino fused] full size {shape}", flush=True)
    fused_mode(1)
    d = conv_desc(hip, n, c, h, w, oc, 3, 3, 1, 1, 1, 1, 1, act, F43)
    x, wt, b, r = _inputs(n * 1000 + c, n, c, h, w, oc, act, d.oh, d.ow)
    y, _ = run_conv(hip, torch_gpu, d, x, wt, b, r)
    od = O.conv_desc(n, c, h, w, oc, 3, 3, 1, 1, 1, 1, 1, act)
    assert_parity(y, O.conv2d(od, x, wt, b, r), what=f"{shape} fused vs oracle")


def test_rule_picks_fused_for_few_channels(hip, fused_mode):
    L = hip.lib()
    fused_mode(-1)
    few = conv_desc(hip, 32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1, 1, F43)
    many = conv_desc(hip, 32, 256, 14, 14, 256, 3, 3, 1, 1, 1, 1, 1, 1, F43)
    assert L.spinn_hip_conv_workspace_size(C.byref(few)) == 0
    assert L.spinn_hip_conv_workspace_size(C.byref(many)) > 0
