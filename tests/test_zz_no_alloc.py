"""spinn_hip_conv_noalloc (scratch in the library's fixed device array) against
spinn_hip_conv (scratch in a caller workspace) through the C ABI: the same
kernels run on the same operands, so the outputs must be bit-identical. Each
case makes two calls in a row, the second on a smaller input, and also checks
the oracle's parity bar."""
import ctypes as C
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import conv_desc

pytestmark = pytest.mark.gpu

# pairs of (n, c, h, w, oc, k, stride, pad, group, act, algo): a larger call, then a smaller one;
# "splitk" pairs run with 64 x 64 tiles and K split 4 ways over workgroups (partials in the scratch)
PAIRS = [
    ("splitk_then_smaller_splitk", (1, 1024, 7, 8, 256, 1, 1, 0, 1, 5, 1), (1, 512, 7, 7, 512, 3, 1, 1, 1, 1, 1)),
    ("f43_b32_then_f43_b2", (32, 256, 14, 14, 256, 3, 1, 1, 1, 1, 4), (2, 128, 28, 28, 128, 3, 1, 1, 1, 5, 4)),
    ("f23_then_splitk", (8, 128, 28, 28, 128, 3, 1, 1, 1, 3, 2), (1, 2048, 7, 7, 512, 1, 1, 0, 1, 1, 1)),
    ("auto_stem_then_depthwise", (4, 3, 224, 224, 64, 7, 2, 3, 1, 1, 0), (1, 32, 20, 20, 32, 3, 2, 1, 32, 3, 0)),
    # stream-K under the per-shape rule: the 392-tile layer takes extra workgroups, the
    # 1568-tile one has whole-tile workgroups do the parts; arrival counters and partial
    # slots stay in the shared scratch between the calls
    ("streamk_wgs_then_streamk_parts", (32, 1024, 14, 14, 256, 1, 1, 0, 1, 1, 1),
     (32, 256, 14, 14, 1024, 1, 1, 0, 1, 5, 1)),
]


def _operands(torch, L, hip, case, seed):
    n, c, h, w, oc, k, s, p, group, act, algo = case
    d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, group, act, algo)
    d.algo = L.spinn_hip_conv_select_algo(C.byref(d))
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c // group, k, k)) * np.sqrt(2.0 / (c // group * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, d.oh, d.ow)).astype(np.float32) if act in (4, 5) else None
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
    xd, wd, bd, rd = dev(x), dev(wt), dev(b), dev(r)
    psz = L.spinn_hip_conv_packed_size(C.byref(d))
    pk = None
    if psz:
        pk = torch.empty(psz // 4, device="cuda")
        hip.check(L.spinn_hip_conv_pack_weights(C.byref(d), hip.ptr(wd), hip.ptr(pk), None), "pack")
    ref = O.conv2d(O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, group, act), x, wt, b, r)
    return d, (xd, wd, pk, bd, rd), ref


CASES = [(p, -1) for p in PAIRS] + [(p, 2) for p in PAIRS if p[0].startswith("streamk")]


@pytest.mark.parametrize("pair,streamk", CASES,
                         ids=[p[0] + ("_exchange_memory" if m == 2 else "") for p, m in CASES])
def test_noalloc_matches_workspace_entry_point(hip, torch_gpu, pair, streamk):
    L = hip.lib()
    if "splitk" in pair[0]:
        L.spinn_hip_tune_force_tiles(64, 64, 4)
    L.spinn_hip_tune_streamk(streamk)  # 2: parts' sums through memory even where they share an L2
    try:
        _compare_pair(hip, torch_gpu, L, pair)
    finally:
        L.spinn_hip_tune_force_tiles(0, 0, 0)
        L.spinn_hip_tune_streamk(-1)
    assert L.spinn_hip_device_status() == 0


def _compare_pair(hip, torch, L, pair):
    name, big, small = pair
    for i, case in enumerate((big, small)):
        d, (xd, wd, pk, bd, rd), ref = _operands(torch, L, hip, case, zlib.crc32(f"{name}{i}".encode()))
        wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
        print(f"[noalloc] {name} call {i}: algo={d.algo} scratch={wsz}", flush=True)
        assert wsz <= hip.NOALLOC_SCRATCH_BYTES
        if "splitk" in name or name.startswith("streamk"):
            assert wsz > 0, "the split-K / stream-K pair must use the scratch"
        ws = torch.empty(max(wsz // 4, 1), device="cuda") if wsz else None
        y_ws = torch.full((d.n, d.oc, d.oh, d.ow), float("nan"), device="cuda")
        y_na = torch.full((d.n, d.oc, d.oh, d.ow), float("nan"), device="cuda")
        hip.check(L.spinn_hip_conv(C.byref(d), hip.ptr(xd), hip.ptr(wd), hip.ptr(pk), hip.ptr(bd), hip.ptr(rd),
                                   hip.ptr(y_ws), hip.ptr(ws), wsz, None), "spinn_hip_conv")
        hip.check(L.spinn_hip_conv_noalloc(C.byref(d), hip.ptr(xd), hip.ptr(wd), hip.ptr(pk), hip.ptr(bd),
                                           hip.ptr(rd), hip.ptr(y_na), None), "spinn_hip_conv_noalloc")
        torch.cuda.synchronize()
        a, b = y_ws.cpu().numpy(), y_na.cpu().numpy()
        assert np.array_equal(a, b), f"{name} call {i}: outputs differ"
        assert_parity(b, ref, what=f"{name} call {i} vs oracle")


def test_noalloc_rejects_oversized_scratch(hip, torch_gpu):
    """A conv whose scratch exceeds the fixed array is refused before any launch."""
    L = hip.lib()
    # F(4x4,3x3) in three launches at 16 x 128 x 112 x 112: V and M are 2 x 231 MB
    # (128 channels stay off the one-launch form, which needs no scratch)
    d = conv_desc(hip, 16, 128, 112, 112, 128, 3, 3, 1, 1, 1, 1, 1, 1, 4)
    assert L.spinn_hip_conv_workspace_size(C.byref(d)) > hip.NOALLOC_SCRATCH_BYTES
    rc = L.spinn_hip_conv_noalloc(C.byref(d), C.c_void_p(256), C.c_void_p(256), C.c_void_p(256), None, None,
                                  C.c_void_p(256), None)
    assert rc == hip.SPINN_HIP_EWORKSPACE
