"""Data-parallel + stream-K implicit-GEMM conv launches.

Whole tiles run one workgroup each; the tiles left after an even share per CU
are cut along K, and the part of each such tile that arrives last sums all
parts in K order and applies the epilogue, inside the same launch. Checked
against the oracle (restated SPINN conv, SPINN/run_time/ops/conv/conv2d.c:92-232)
with the split forced on and off, for every B-operand loader, both tile shapes,
ragged M / N / K edges, both ways of placing the parts (extra workgroups, or
parts done by whole-tile workgroups first) and XCDs without remaining tiles;
plus bit-identical
repeats (also over a workspace filled with garbage, which the arrival counters
must ignore) and HIP-graph replays of one captured launch.
"""
import ctypes as C
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import conv_desc

pytestmark = pytest.mark.gpu

# (name, n, c, h, w, oc, k, stride, pad, act); tiles of 64 x 64 (32 x 128 for
# <= 32 output channels) on 256 CUs
CASES = [
    # extra workgroups (at most two whole tiles per CU, > 64 remaining tiles)
    ("pw_1024to256_14_b32", 32, 1024, 14, 14, 256, 1, 1, 0, 1),     # 392 tiles: 256 whole + 136 cut
    ("tap3x3_256_14_b32", 32, 256, 14, 14, 256, 3, 1, 1, 1),        # 392 tiles of 144 slices, tap gather
    ("gen3x3_ragged_silu", 32, 24, 17, 19, 83, 3, 1, 1, 3),          # (c,kh,kw) gather, M 83, K 216
    ("gen1x1_s2_none", 16, 256, 28, 28, 512, 1, 2, 0, 0),           # 392 tiles, ragged last column tile
    # parts done by whole-tile workgroups
    ("pw_256to1024_14_b32_res", 32, 256, 14, 14, 1024, 1, 1, 0, 5),  # 1568 tiles, 4 parts per remaining tile
    ("tap3x3_128_28_b32", 32, 128, 28, 28, 128, 3, 1, 1, 1),        # 784 tiles, 8 parts
    ("stem7x7_s2", 20, 3, 64, 64, 64, 7, 2, 3, 1),                   # K 147, 2 parts
    ("pw_oc32_tile32x128_res", 100, 128, 20, 20, 32, 1, 1, 0, 5),    # 32 x 128 tiles
    ("three_remaining_tiles", 37, 512, 16, 28, 64, 1, 1, 0, 3),      # 259 tiles: five XCDs without parts
]


def _inputs(seed, n, c, h, w, oc, k, act, oh, ow):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, k, k)) * np.sqrt(2.0 / (c * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, oh, ow)).astype(np.float32) if act in (4, 5) else None
    return x, wt, b, r


class _Conv:
    """One conv layer's device operands, run through spinn_hip_conv."""

    def __init__(self, hip, torch, case):
        name, n, c, h, w, oc, k, s, p, act = case
        self.hip, self.torch, self.L = hip, torch, hip.lib()
        self.d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, 1, act, hip.ALGO_IMPLICIT_GEMM)
        self.x, self.wt, self.b, self.r = _inputs(zlib.crc32(name.encode()), n, c, h, w, oc, k, act,
                                                  self.d.oh, self.d.ow)
        dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
        self.xd, self.wd, self.bd, self.rd = dev(self.x), dev(self.wt), dev(self.b), dev(self.r)
        self.pk = torch.empty(max(self.L.spinn_hip_conv_packed_size(C.byref(self.d)) // 4, 1), device="cuda")
        hip.check(self.L.spinn_hip_conv_pack_weights(C.byref(self.d), hip.ptr(self.wd), hip.ptr(self.pk), None),
                  "pack")
        self.od = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, 1, act)

    def ws_bytes(self):
        return self.L.spinn_hip_conv_workspace_size(C.byref(self.d))

    def run(self, ws, stream=None):
        torch = self.torch
        y = torch.full((self.d.n, self.d.oc, self.d.oh, self.d.ow), float("nan"), device="cuda")
        wsz = self.ws_bytes()
        self.hip.check(self.L.spinn_hip_conv(C.byref(self.d), self.hip.ptr(self.xd), self.hip.ptr(self.wd),
                                             self.hip.ptr(self.pk), self.hip.ptr(self.bd), self.hip.ptr(self.rd),
                                             self.hip.ptr(y), self.hip.ptr(ws), wsz, stream), "spinn_hip_conv")
        return y

    def oracle(self):
        return O.conv2d(self.od, self.x, self.wt, self.b, self.r)


@pytest.fixture
def streamk_mode(hip):
    L = hip.lib()
    yield L.spinn_hip_tune_streamk
    L.spinn_hip_tune_streamk(-1)
    L.spinn_hip_tune_streamk_tries(-1)
    L.spinn_hip_tune_force_tiles(0, 0, 0)


@pytest.mark.parametrize("exchange", [1, 2], ids=["exchange_l2", "exchange_memory"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_streamk_parity_and_repeats(hip, torch_gpu, streamk_mode, case, exchange):
    torch = torch_gpu
    print(f"[streamk] {case[0]} exchange {exchange}", flush=True)
    cv = _Conv(hip, torch, case)
    ref = cv.oracle()
    # the MFMA tile engine on the tile shape the rule gives these channel counts
    # (the wave-K kernel, which small grids would otherwise take, kept out)
    oc = case[5]
    hip.lib().spinn_hip_tune_force_tiles(*((32, 128) if oc <= 32 else (64, 64)), 0)
    # split forced off: whole tiles only
    streamk_mode(0)
    ws0 = torch.empty(max(cv.ws_bytes() // 4, 1), device="cuda")
    y_off = cv.run(ws0)
    torch.cuda.synchronize()
    assert_parity(y_off.cpu().numpy(), ref, what=f"{case[0]} stream-K off vs oracle")
    # split forced on: every grid whose tile count is not a multiple of the CUs;
    # parts exchange their sums through the XCD's L2 (where spinn_hip_init
    # confirmed the placement) or through memory
    streamk_mode(exchange)
    wsz = cv.ws_bytes()
    assert wsz > 0, "case does not take the stream-K launch; pick another shape"
    ws = torch.zeros(wsz // 4, device="cuda")
    outs = []
    for i in range(3):
        if i == 2:
            # arbitrary bytes in the counters and partial slots: counters of another
            # epoch count as zero
            g = torch.Generator(device="cpu").manual_seed(5)
            ws.copy_(torch.randint(-2**31, 2**31 - 1, (wsz // 4,), generator=g, dtype=torch.int32)
                     .view(torch.float32).cuda())
        y = cv.run(ws)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        assert_parity(outs[-1], ref, what=f"{case[0]} stream-K call {i} vs oracle")
    assert np.array_equal(outs[0], outs[1]), "repeated stream-K launches differ"
    assert np.array_equal(outs[0], outs[2]), "stream-K launch over a garbage workspace differs"
    assert hip.lib().spinn_hip_device_status() == 0, "an arrival reported a failure"


def test_streamk_arrival_failure_is_reported(hip, torch_gpu, streamk_mode):
    """With the arrival rounds set to 0 from the host (every kernel still exits
    normally), no part of a cut tile can claim its counter: those tiles stay
    unwritten and spinn_hip_device_status reports it once; whole tiles are
    still right. Restored, the same launch is complete and reports nothing."""
    torch = torch_gpu
    L = hip.lib()
    streamk_mode(1)
    cv = _Conv(hip, torch, CASES[0])
    ref = cv.oracle()
    wsz = cv.ws_bytes()
    assert wsz > 0
    ws = torch.zeros(wsz // 4, device="cuda")
    assert L.spinn_hip_device_status() == 0
    L.spinn_hip_tune_streamk_tries(0)
    try:
        y = cv.run(ws)  # output pre-filled with NaN
        torch.cuda.synchronize()
    finally:
        L.spinn_hip_tune_streamk_tries(-1)
    assert L.spinn_hip_device_status() == hip.SPINN_HIP_EDEVICE
    assert L.spinn_hip_device_status() == 0, "the report is cleared once read"
    yb = y.cpu().numpy()
    unwritten = np.isnan(yb)
    assert unwritten.any(), "cut tiles must stay unwritten when no arrival completes"
    written = ~unwritten
    assert np.abs(yb[written] - ref[written]).max() <= 1e-3, "whole tiles are unaffected"
    y = cv.run(ws)
    torch.cuda.synchronize()
    assert L.spinn_hip_device_status() == 0
    assert_parity(y.cpu().numpy(), ref, what="stream-K after the failure report")


def test_streamk_rule_picks_remainder_split(hip, torch_gpu, streamk_mode):
    """Under the per-shape rule the 392-tile ResNet-101 layer takes the split and
    the balanced 6272-tile one (24.5 tiles per CU) does not."""
    L = hip.lib()
    streamk_mode(-1)
    d = conv_desc(hip, 32, 1024, 14, 14, 256, 1, 1, 1, 1, 0, 0, 1, 1, hip.ALGO_IMPLICIT_GEMM)
    assert L.spinn_hip_conv_workspace_size(C.byref(d)) > 0
    d = conv_desc(hip, 32, 64, 56, 56, 256, 1, 1, 1, 1, 0, 0, 1, 1, hip.ALGO_IMPLICIT_GEMM)
    assert L.spinn_hip_conv_workspace_size(C.byref(d)) == 0


def test_streamk_graph_replays(hip, torch_gpu, streamk_mode):
    """One captured stream-K launch (its counters' epoch fixed in the graph)
    replayed several times, with eager launches of the same layer and other
    work in between: every replay equals the eager result bit for bit."""
    torch = torch_gpu
    L = hip.lib()
    streamk_mode(1)
    cv = _Conv(hip, torch, CASES[0])
    wsz = cv.ws_bytes()
    ws = torch.zeros(wsz // 4, device="cuda")
    eager = cv.run(ws)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    st = C.c_void_p()
    hip.check(L.spinn_hip_stream_create(C.byref(st)), "stream")
    y = torch.full_like(eager, float("nan"))
    gexec = C.c_void_p()
    try:
        hip.check(L.spinn_hip_graph_capture_begin(st), "capture begin")
        rc = L.spinn_hip_conv(C.byref(cv.d), hip.ptr(cv.xd), hip.ptr(cv.wd), hip.ptr(cv.pk), hip.ptr(cv.bd),
                              hip.ptr(cv.rd), hip.ptr(y), hip.ptr(ws), wsz, st)
        hip.check(L.spinn_hip_graph_capture_end(st, C.byref(gexec)), "capture end")
        hip.check(rc, "conv under capture")
        for i in range(4):
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            hip.check(L.spinn_hip_graph_launch(gexec, st), "graph launch")
            hip.check(L.spinn_hip_stream_sync(st), "sync")
            assert np.array_equal(y.cpu().numpy(), ref), f"graph replay {i} differs from the eager launch"
            # eager launches of the same layer (new epochs) between replays
            e2 = cv.run(ws)
            torch.cuda.synchronize()
            assert np.array_equal(e2.cpu().numpy(), ref)
    finally:
        if gexec:
            L.spinn_hip_graph_destroy(gexec)
        L.spinn_hip_stream_destroy(st)
