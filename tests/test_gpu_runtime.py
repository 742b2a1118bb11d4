"""End-to-end GPU parity: ENNF models through spinn_load / spinn_plan / spinn_run
(every conv, Gemm and glue op on the device, activations in one HBM arena)
against the oracle's CPU run of the same file and input."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from spinn_amd import ennf as E
from spinn_amd import models
from spinn_amd import native as N
from spinn_amd.runtime import Session
from tests.conftest import assert_parity

pytestmark = pytest.mark.gpu


def _run_both(tmp_path, g, x, name, policy=N.POLICY_AUTO, graph=False, winograd_oracle=False):
    path = g.write(tmp_path / f"{name}.ennf")
    out_shape = g.dims(g.outputs[0])
    with Session(path, policy=policy, graph=graph) as s:
        y = s.run(x)
        y2 = s.run(x)  # a second run over the same arena must reproduce the first
    ref = O.Model(path, winograd=winograd_oracle).run(x, out_shape)
    return y, y2, ref


def test_conv_bn_relu_model(hip, tmp_path):
    g, x = models.conv_bn_relu(seed=0)
    y, y2, ref = _run_both(tmp_path, g, x, "cfg0")
    assert_parity(y, ref, what="conv+bn+relu")
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("mnk", models.GEMM_SWEEP[:3], ids=str)
def test_gemm_model(hip, tmp_path, mnk):
    g, a = models.gemm_model(*mnk, seed=1)
    y, _, ref = _run_both(tmp_path, g, a, "gemm")
    assert_parity(y, ref, what=f"gemm {mnk}")


def test_vgg_stack_small(hip, tmp_path):
    sched = [(16, 32), (16, 32), (32, 16), (32, 16)]
    g, x = models.vgg_stack(batch=2, seed=3, in_c=16, schedule=sched)
    y, _, ref = _run_both(tmp_path, g, x, "vgg_small")
    assert_parity(y, ref, what="vgg small", scale_by_ref=True)


def test_vgg_stack_winograd_policy(hip, tmp_path):
    sched = [(32, 28), (32, 28), (64, 14), (64, 14)]
    g, x = models.vgg_stack(batch=2, seed=4, in_c=32, schedule=sched)
    y, _, ref = _run_both(tmp_path, g, x, "vgg_wino", policy=N.POLICY_WINOGRAD)
    assert_parity(y, ref, what="vgg winograd vs im2col oracle", scale_by_ref=True)


def test_resnet50_b1(hip, tmp_path):
    g, x = models.resnet(batch=1, seed=5, blocks=models.RESNET50_BLOCKS, hw=96)
    y, y2, ref = _run_both(tmp_path, g, x, "r50")
    assert_parity(y, ref, what="resnet50@96 b1", scale_by_ref=True)
    assert np.array_equal(y, y2)


def test_resnet101_b1(hip, tmp_path):
    g, x = models.resnet101(batch=1, seed=0)
    y, _, ref = _run_both(tmp_path, g, x, "r101")
    print(f"[r101 b1] |ref|max={np.abs(ref).max():.3e}", flush=True)
    assert_parity(y, ref, what="resnet101 b1", scale_by_ref=True)


def test_resnet101_b4_winograd_f43_and_f23(hip, tmp_path):
    """Batch 4: AUTO runs the 3x3 stride-1 convs of stages 1-3 (64@56x56, 128@28x28,
    256@14x14) as Winograd F(4x4,3x3) and stage 4's (512@7x7, 16 4x4 tiles) as
    F(2x2,3x3); the 101-layer result stays within the bound of the oracle's direct
    (im2col) convolution."""
    g, x = models.resnet101(batch=4, seed=2)
    algos = []
    L = N.lib()
    for nd in (n for n in g.nodes if n.op == E.OP_CONV):
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, _, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        d = N.ConvDesc(n, c, h, w, oc, oh, ow, kh, kw, p["strides"][0], p["strides"][1], p["pads"][0], p["pads"][1],
                       p["group"] or 1, p["act"], 0, 0)
        algos.append(L.spinn_hip_conv_select_algo(C.byref(d)))
    assert algos.count(N.ALGO_WINOGRAD_F43) == 28 and algos.count(N.ALGO_WINOGRAD) == 2
    y, y2, ref = _run_both(tmp_path, g, x, "r101b4")
    print(f"[r101 b4] |ref|max={np.abs(ref).max():.3e}", flush=True)
    assert_parity(y, ref, what="resnet101 b4 with F(4x4,3x3)", scale_by_ref=True)
    assert np.array_equal(y, y2)


def test_resnet101_b8_small_grid_tiles(hip, tmp_path):
    """Batch 8: the grids under two tiles per CU take the small-grid tile rules - 16 x 16
    wave-K tiles for the K = 64 1x1 layer at 56x56, 32 x 32 for the 1024-deep 1x1 layers at
    14x14, unsplit 64 x 64 tiles for 200-tile grids, F(2x2,3x3) for 512@7x7 - and the graph
    replays the eager result bit for bit; the 101-layer output stays within the bound of
    the oracle's direct convolution."""
    g, x = models.resnet101(batch=8, seed=5)
    algos = []
    L = N.lib()
    for nd in (n for n in g.nodes if n.op == E.OP_CONV):
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, _, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        d = N.ConvDesc(n, c, h, w, oc, oh, ow, kh, kw, p["strides"][0], p["strides"][1], p["pads"][0], p["pads"][1],
                       p["group"] or 1, p["act"], 0, 0)
        algos.append(L.spinn_hip_conv_select_algo(C.byref(d)))
    assert algos.count(N.ALGO_WINOGRAD) == 2
    path = g.write(tmp_path / "r101b8.ennf")
    with Session(path) as s:
        y = s.run(x)
    with Session(path, graph=True) as s:
        replays = [s.run(x) for _ in range(2)]
    ref = O.Model(path).run(x, g.dims(g.outputs[0]))
    print(f"[r101 b8] |ref|max={np.abs(ref).max():.3e}", flush=True)
    assert_parity(y, ref, what="resnet101 b8 (AUTO) vs oracle", scale_by_ref=True)
    for r in replays:
        assert np.array_equal(r, y)


def test_resnet101_b1_graph_replay(hip, tmp_path):
    g, x = models.resnet101(batch=1, seed=0)
    path = g.write(tmp_path / "r101g.ennf")
    with Session(path) as s:
        y_eager = s.run(x)
    with Session(path, graph=True) as s:
        outs = [s.run(x) for _ in range(3)]
    for o in outs:
        assert np.array_equal(o, y_eager)


def _input_region_reused(s) -> bool:
    """Whether the plan places another tensor inside input 0's arena region (the
    reference planner frees it after its last consumer,
    SPINN/run_time/spinn_memory_planner.c:231-238)."""
    t_in = s.tensor(s.input_id)
    lo, hi = t_in.offset, t_in.offset + t_in.size
    return any(tid != s.input_id and off < hi and off + s.tensor(tid).size > lo
               for tid, off in s.offsets().items())


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
@pytest.mark.parametrize("model", ["resnet50_96_b2", "yolov10n_320_b2_tail"])
def test_resident_runs_restore_input(hip, tmp_path, model, graph):
    """Input staged once, then three spinn_run_resident steps: each step restores
    input 0 into its arena region before the node loop (the reference copies the
    input on every spinn_run, SPINN/run_time/spinn_runtime.c:302-306), so runs 2
    and 3 equal run 1 bit for bit and the oracle within the bar, although the plan
    hands the input's region to later activations."""
    if model == "resnet50_96_b2":
        g, x = models.resnet(batch=2, seed=11, blocks=models.RESNET50_BLOCKS, hw=96)
    else:
        g, x = models.yolov10n(batch=2, seed=12, hw=320, postprocess=True)
    path = g.write(tmp_path / f"{model}.ennf")
    print(f"[resident] {model} graph={graph}", flush=True)
    with Session(path, graph=graph) as s:
        assert _input_region_reused(s), "the plan must reuse the input region for this test to mean anything"
        with pytest.raises(N.SpinnError):
            s.run_resident()  # nothing staged yet
        y_host = s.run(x)
        s.upload_input(x)
        outs = []
        for _ in range(3):
            s.run_resident()
            outs.append(s.download(s.output_id))
        # a host-copy run in between must not disturb the staged input
        s.run(np.zeros_like(x))
        s.run_resident()
        outs.append(s.download(s.output_id))
    for i, o in enumerate(outs):
        assert np.array_equal(o.view(np.uint32), y_host.view(np.uint32)), f"resident run {i + 1} differs"
    if model == "resnet50_96_b2":
        ref = O.Model(path).run(x, g.dims(g.outputs[0]))
        assert_parity(outs[1], ref, what=f"{model} resident run 2", scale_by_ref=True)
        assert_parity(outs[2], ref, what=f"{model} resident run 3", scale_by_ref=True)


@pytest.mark.parametrize("batch,hw", [(1, 640), (2, 320)], ids=["b1_640", "b2_320"])
def test_yolov10n(hip, tmp_path, batch, hw):
    """The detector: fused Conv+SiLU / Conv+Add, depthwise, unfused Add / Split /
    Concat / MaxPool 5x5 / Resize / attention (Reshape, Transpose, MatMul,
    Softmax) and the decoded head (DFL Softmax + conv, Sub / Add / Mul with
    broadcast anchors and strides, Sigmoid), output [B, 84, anchors]."""
    g, x = models.yolov10n(batch=batch, seed=7, hw=hw)
    print(f"[yolov10n] b{batch} {hw}x{hw}", flush=True)
    y, y2, ref = _run_both(tmp_path, g, x, f"y10_b{batch}")
    assert_parity(y, ref, what=f"yolov10n b{batch}@{hw}", scale_by_ref=True)
    assert np.array_equal(y, y2)
    assert_parity(y[:, 4:], ref[:, 4:], what="class scores")


def test_yolov10n_b16_graph_replay(hip, tmp_path):
    g, x = models.yolov10n(batch=16, seed=8)
    path = g.write(tmp_path / "y10_b16.ennf")
    print("[yolov10n] b16 640 eager + graph", flush=True)
    with Session(path) as s:
        y_eager = s.run(x)
    with Session(path, graph=True) as s:
        outs = [s.run(x) for _ in range(3)]
    for o in outs:
        assert np.array_equal(o, y_eager)
    ref = O.Model(path).run(x, g.dims(g.outputs[0]))
    assert_parity(y_eager, ref, what="yolov10n b16", scale_by_ref=True)


VIEW_OPS = (E.OP_RESHAPE, E.OP_FLATTEN, E.OP_IDENTITY, E.OP_UNSQUEEZE)


def _views(s):
    """(view nodes, those whose output shares its input's device address)."""
    c = s.c
    views = [c.nodes[k] for k in range(c.num_nodes) if c.nodes[k].op_type in VIEW_OPS]
    shared = [nd for nd in views if c.tensors[nd.input_ids[0]].data == c.tensors[nd.output_ids[0]].data]
    return len(views), len(shared)


def _folded_transposes(s):
    """(Transpose nodes, those a MatMul reads transposed in their place)."""
    c = s.c
    tr = [k for k in range(c.num_nodes) if c.nodes[k].op_type == E.OP_TRANSPOSE]
    mm = [k for k in range(c.num_nodes) if c.nodes[k].op_type == E.OP_MATMUL]
    if not c.node_folded:  # folding switched off: no tables
        assert not c.node_tsrc
        return len(tr), 0
    folded = [k for k in tr if c.node_folded[k]]
    reads = sum(1 for j in mm for q in range(2) if c.node_tsrc[2 * j + q] >= 0)
    assert reads == len(folded)
    return len(tr), len(folded)


def _folded_scales(s):
    """MatMuls that write a folded Mul's output with its scalar as alpha."""
    c = s.c
    if not c.node_tdst:
        return 0
    n = 0
    for j in range(c.num_nodes):
        if c.node_tdst[j] >= 0:
            assert c.nodes[j].op_type == E.OP_MATMUL
            muls = [k for k in range(c.num_nodes) if c.nodes[k].op_type == E.OP_MUL
                    and c.nodes[k].output_ids[0] == c.node_tdst[j]]
            assert len(muls) == 1 and c.node_folded[muls[0]]
            n += 1
    return n


@pytest.mark.parametrize("batch,tail", [(1, False), (1, True), (2, False)], ids=["b1_head", "b1_tail", "b2_head"])
def test_view_nodes_read_in_place(hip, tmp_path, batch, tail):
    """Reshape / Flatten / Identity / Unsqueeze copy their input unless the tensors share
    bytes. At plan time an output whose input bytes no node overwrites before the output's
    last reader takes the input's device address, so the node launches nothing; a Transpose
    of the last two axes read only by a MatMul is folded into it (the Gemm reads the
    Transpose's input with its transpose flag). YOLOv10n has both in its attention and head;
    eager and graph-replayed runs agree bit for bit, and the head's output matches the oracle."""
    g, x = models.yolov10n(batch=batch, seed=21, hw=320, postprocess=tail)
    path = g.write(tmp_path / f"y10_views_{batch}_{tail}.ennf")
    print(f"[views] yolov10n b{batch} 320 tail={tail}", flush=True)
    with Session(path) as s:
        n_views, n_shared = _views(s)
        n_tr, n_folded = _folded_transposes(s)
        n_scales = _folded_scales(s)
        y = s.run(x)
    with Session(path, graph=True) as sg:
        yg = [sg.run(x) for _ in range(2)]
    print(f"[views] {n_shared} of {n_views} view nodes read in place, {n_folded} of {n_tr} Transposes folded, "
          f"{n_scales} scalar Muls folded", flush=True)
    assert n_shared >= 1 and n_folded >= 1
    for o in yg:
        assert np.array_equal(o, y)
    if not tail:
        ref = O.Model(path).run(x, g.dims(g.outputs[0]))
        assert_parity(y, ref, what=f"yolov10n b{batch}@320 with in-place views", scale_by_ref=True)


def test_plan_fold_off_keeps_every_copy(hip, tmp_path, monkeypatch):
    """SPINN_PLAN_FOLD=0 at plan time keeps every view copy and Transpose (each tensor in its
    own bytes, as the planner placed it); the output matches the folded plan's within the
    bar (the Gemm reads the folded operands in the other orientation)."""
    g, x = models.yolov10n(batch=1, seed=22, hw=320)
    path = g.write(tmp_path / "y10_nofold.ennf")
    with Session(path) as s:
        assert _views(s)[1] >= 1 and _folded_transposes(s)[1] >= 1
        y_fold = s.run(x)
    monkeypatch.setenv("SPINN_PLAN_FOLD", "0")
    with Session(path) as s:
        assert _views(s)[1] == 0 and _folded_transposes(s)[1] == 0 and _folded_scales(s) == 0
        y = s.run(x)
    assert_parity(y, y_fold, what="yolov10n b1@320 unfolded vs folded", scale_by_ref=True)


def test_graph_mode_failed_node_is_not_replayed(hip, tmp_path):
    """A node that fails host-side validation during graph capture leaves no graph
    behind: every later graph-mode run captures again and reports the failure
    again, instead of replaying a graph without that node and returning 0."""
    rng = np.random.default_rng(0)
    g = E.Graph()
    x = g.input("x", (1, 8, 8, 8))
    r = g.tensor("r", (1, 8, 8, 8))
    g.node(E.OP_RELU, [x], [r])
    # 4 weight channels for an 8-channel input with group 1: op_conv2d refuses it
    w = g.weight("w", rng.standard_normal((8, 4, 3, 3)).astype(np.float32))
    y = g.tensor("y", (1, 8, 8, 8))
    g.node(E.OP_CONV, [r, w], [y], E.conv_params(3, 3, pads=(1, 1, 1, 1)))
    g.output(y)
    path = g.write(tmp_path / "bad_conv.ennf")
    L = N.lib()
    s = Session(path, plan=False)
    try:
        assert L.spinn_plan(s.ctx, 0) < 0  # the prepare pass already refuses the conv
        L.spinn_set_graph_mode(s.ctx, 1)
        xin = np.ones((1, 8, 8, 8), np.float32)
        for i in range(2):
            with pytest.raises(N.SpinnError):
                s.run(xin)
            assert s.c.last_error_node == 1, i
    finally:
        s.close()


def test_cli_driver_protocol(hip, tmp_path):
    """spinn_amd/bin/spinn_run on the Conv3x3+BN+ReLU model: the reference CLI's
    protocol (SPINN/run_time/main.c:17-139) - synthetic input x[i] = i/1000, 3
    warm-ups then best / average, the `SPINN Result:` line parsed the way
    SPINN/ennf2c/verify_three_way.py:29-44 parses it, and the SPINN_DUMP binary
    dump of the output - against the oracle on the same input. The synthetic
    input reaches 200, so the outputs reach the hundreds and the max-abs bound
    is taken relative to max|ref|."""
    import os
    import subprocess
    from spinn_amd import build
    g, _ = models.conv_bn_relu(seed=0)
    path = g.write(tmp_path / "cfg0.ennf")
    dump = tmp_path / "out.bin"
    env = dict(os.environ, SPINN_DUMP=str(dump))
    for extra in ([], ["5"], ["5", "--graph"]):
        print(f"[cli] spinn_run {' '.join(extra)}", flush=True)
        r = subprocess.run([str(build.CLI), str(path), *extra], capture_output=True, text=True, env=env,
                           timeout=60)
        assert r.returncode == 0, r.stderr[-2000:]
        line = next(l for l in r.stdout.splitlines() if l.startswith("SPINN Result:"))
        vals = np.array([float(v) for v in line[len("SPINN Result:"):].split()])
        n_in = int(np.prod(g.dims(g.inputs[0])))
        x = (np.arange(n_in, dtype=np.float32) / np.float32(1000)).reshape(g.dims(g.inputs[0]))
        ref = O.Model(path).run(x, g.dims(g.outputs[0]))
        dumped = np.fromfile(dump, np.float32).reshape(ref.shape)
        assert_parity(dumped, ref, what=f"cli dump {extra}", scale_by_ref=True)
        assert vals.size == ref.size
        assert np.abs(vals - dumped.ravel()).max() <= 5e-7 + 1e-6 * np.abs(dumped).max()  # %.6f print
        if extra:
            assert "Warmup: 3, Runs: 5" in r.stderr and "Best:" in r.stderr and "Avg:" in r.stderr
