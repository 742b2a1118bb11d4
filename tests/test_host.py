"""CPU tests of the host side: ENNF format, the native loader, the planner
(against the reference planner's offsets), the operator registry's error
conventions and the exported C ABI. No GPU calls."""
import ctypes as C
import re
import struct
from pathlib import Path

import numpy as np
import pytest

from spinn_amd import ennf as E
from spinn_amd import models

ROOT = Path(__file__).resolve().parents[1]
GOLD = ROOT / "tests" / "golden"


def test_struct_sizes(native):
    assert C.sizeof(native.ENNFHeader) == 64
    assert C.sizeof(native.ConvDesc) == 17 * 4
    assert len(E.conv_params(3, 3)) == 44
    assert len(E.pool_params(3, 3, 2, 2)) == 48
    assert len(E.gemm_params()) == 12
    assert len(E.reduce_params([2, 3])) == 36


def test_ennf_roundtrip(tmp_path):
    g, x = models.resnet(batch=2, seed=4, blocks=(1, 1, 1, 1), hw=32, num_classes=10)
    path = g.write(tmp_path / "m.ennf")
    m = E.read(path)
    h = m["header"]
    assert h["magic"] == E.ENNF_MAGIC and h["version_major"] == 2
    assert h["num_nodes"] == len(g.nodes) and h["num_tensors"] == len(g.tensors)
    assert h["reserved"][0] == 64  # dense weight-entry table right after the header
    assert h["weight_data_offset"] % 16 == 0
    assert m["inputs"] == g.inputs and m["outputs"] == g.outputs
    for nd, gn in zip(m["nodes"], g.nodes):
        assert nd["op"] == gn.op and nd["inputs"] == gn.inputs and nd["outputs"] == gn.outputs
        assert nd["params"] == gn.params and nd["flags"] == gn.flags
    # reference counts are those of the graph before fusion (SPINN/onnx2ennf.c:232-241)
    ids = {t.name: t.id for t in g.tensors}
    ref = {t.id: 0 for t in g.tensors}
    for n in g.onnx.nodes:
        for i in n.inputs:
            ref[ids[i]] += 1
    for t in g.tensors:
        mt = m["tensors"][t.id]
        assert mt["dims"] == t.dims and mt["ref_count"] == ref[t.id] and mt["is_weight"] == int(t.is_weight)
        if t.is_weight:
            assert np.array_equal(m["weights"][t.id], t.data)
    # the fused residual is the conv's last input, with ADD_RELU in params.reserved
    convs = [nd for nd in m["nodes"] if nd["op"] == E.OP_CONV]
    res = [nd for nd in convs if E.unpack_conv_params(nd["params"])["act"] == E.ACT_ADD_RELU]
    assert len(res) == 4 and all(len(nd["inputs"]) == 4 for nd in res)


def test_resnet101_fusion_mix():
    """67 RELU / 33 ADD_RELU / 4 NONE convs, as the reference's fusion leaves ResNet-101."""
    g, _ = models.resnet101(batch=1, seed=0)
    acts = [E.unpack_conv_params(n.params)["act"] for n in g.nodes if n.op == E.OP_CONV]
    assert len(acts) == 104
    assert acts.count(E.ACT_RELU) == 67 and acts.count(E.ACT_ADD_RELU) == 33 and acts.count(E.ACT_NONE) == 4
    flops = sum(f for _, f in models.conv_flops(g))
    assert abs(flops / 1e9 - 15.599) < 0.01  # 15.60 GFLOP of convolution per image


def _load_ctx(native, path):
    L = native.lib()
    ctx = L.spinn_load(str(path).encode())
    assert ctx
    return L, ctx


def test_native_loader_parses_model(native, tmp_path):
    g, _ = models.vgg_stack(batch=2, seed=3, in_c=16, schedule=[(16, 32), (32, 16)])
    path = g.write(tmp_path / "v.ennf")
    L, ctx = _load_ctx(native, path)
    try:
        c = ctx.contents
        assert c.num_nodes == len(g.nodes) and c.num_tensors == len(g.tensors)
        assert c.input_ids[0] == g.inputs[0] and c.output_ids[0] == g.outputs[0]
        for i, nd in enumerate(g.nodes):
            n = c.nodes[i]
            assert n.op_type == nd.op and n.num_inputs == len(nd.inputs)
            assert list(n.input_ids[:n.num_inputs]) == nd.inputs
            assert C.string_at(n.params, n.params_size) == nd.params
        for t in g.tensors:
            ct = c.tensors[t.id]
            assert tuple(ct.dims[:ct.ndim]) == t.dims and ct.size == 4 * t.elem_count
            if t.is_weight:
                p = L.spinn_get_weight(ctx, t.id)
                got = np.frombuffer(C.string_at(p, t.data.nbytes), np.float32).reshape(t.dims)
                assert np.array_equal(got, t.data)
    finally:
        L.spinn_free(ctx)


@pytest.mark.parametrize("name,maker", [
    ("conv0", lambda: models.conv_bn_relu(seed=0)[0]),
    ("resnet101_b1", lambda: models.resnet101(batch=1, seed=0)[0]),
    ("resnet101_b4", lambda: models.resnet101(batch=4, seed=0)[0]),
    ("vgg_b2", lambda: models.vgg_stack(batch=2, seed=3, in_c=16, schedule=[(16, 32), (16, 32), (32, 16), (32, 16)])[0]),
    ("gemm_32", lambda: models.gemm_model(32, 1000, 2048, seed=1)[0]),
    ("yolov10n_b1", lambda: models.yolov10n(batch=1, seed=0)[0]),
    ("yolov10n_b2_320", lambda: models.yolov10n(batch=2, seed=0, hw=320)[0]),
])
def test_planner_matches_reference(native, tmp_path, name, maker):
    """Offsets and peak equal the reference planner's (golden, from its compiled code)."""
    z = np.load(GOLD / "planner_offsets.npz", allow_pickle=False)
    path = maker().write(tmp_path / f"{name}.ennf")
    L, ctx = _load_ctx(native, path)
    try:
        peak = L.spinn_plan_memory(ctx, 0)
        assert peak == int(z[f"{name}_peak"][0])
        c = ctx.contents
        ids = z[f"{name}_ids"].tolist()
        got = [c.tensors[i].offset for i in ids]
        assert got == z[f"{name}_offsets"].tolist()
        # invariants: 16-byte alignment, inside the peak
        for i in ids:
            t = c.tensors[i]
            assert t.offset % 16 == 0 and t.offset + t.size <= peak
        _check_no_live_overlap(c)
    finally:
        L.spinn_free(ctx)
    # a cap below the peak fails like the reference (SPINN_MEM_ERR_NOMEM)
    L, ctx = _load_ctx(native, path)
    try:
        assert L.spinn_plan_memory(ctx, max(16, peak // 2)) == int(z[f"{name}_capped_rc"][0]) == -2
    finally:
        L.spinn_free(ctx)


def _check_no_live_overlap(c):
    """Replays node order: tensors alive at the same time never share bytes."""
    n_t = c.num_tensors
    remaining = [c.tensors[i].ref_count for i in range(n_t)]
    outputs = {c.output_ids[i] for i in range(c.header.num_outputs)}
    live = {c.input_ids[i] for i in range(c.header.num_inputs)}

    def span(i):
        t = c.tensors[i]
        return t.offset, t.offset + ((t.size + 15) & ~15)

    for k in range(c.num_nodes):
        nd = c.nodes[k]
        for o in nd.output_ids[:nd.num_outputs]:
            t = c.tensors[o]
            if t.is_weight or t.size == 0:
                continue
            a0, a1 = span(o)
            for l in live:
                b0, b1 = span(l)
                assert a1 <= b0 or b1 <= a0, f"tensor {o} overlaps live tensor {l}"
            live.add(o)
        for i in nd.input_ids[:nd.num_inputs]:
            t = c.tensors[i]
            if t.is_weight or t.size == 0 or i in outputs:
                continue
            if remaining[i] > 0:
                remaining[i] -= 1
                if remaining[i] == 0:
                    live.discard(i)


def test_loader_rejects_bad_files(native, tmp_path):
    L = native.lib()
    bad = tmp_path / "bad.ennf"
    data = bytearray(models.conv_bn_relu(seed=0)[0].to_bytes())
    data[0:4] = b"XXXX"
    bad.write_bytes(bytes(data))
    assert not L.spinn_load(str(bad).encode())
    assert not L.spinn_load(str(tmp_path / "missing.ennf").encode())
    trunc = tmp_path / "trunc.ennf"
    trunc.write_bytes(bytes(data[:50]))
    assert not L.spinn_load(str(trunc).encode())


def test_dispatch_conventions(native):
    """op >= 512 -> -1; an unregistered op is skipped with 0; bad arity -> -1
    (SPINN/run_time/spinn_ops.c:210-228, ops/conv/conv2d.c:95)."""
    L = native.lib()
    empty = (C.POINTER(native.SpinnTensor) * 1)()
    assert L.spinn_dispatch_op(600, empty, 0, None, 0, empty, 0) == -1
    assert L.spinn_dispatch_op(1, empty, 0, None, 0, empty, 0) == 0  # Abs: not served by this runtime
    assert L.spinn_dispatch_op(E.OP_CONV, empty, 1, None, 0, empty, 1) == -1
    assert L.spinn_dispatch_op(E.OP_GEMM, empty, 1, None, 0, empty, 1) == -1
    for op in (E.OP_CONV, E.OP_GEMM, E.OP_MATMUL, E.OP_MAXPOOL, E.OP_REDUCEMEAN, E.OP_RESHAPE, E.OP_FLATTEN,
               E.OP_GAP, E.OP_ADD, E.OP_SUB, E.OP_MUL, E.OP_DIV, E.OP_RELU, E.OP_SIGMOID, E.OP_BN, E.OP_SOFTMAX,
               E.OP_CONCAT, E.OP_SPLIT, E.OP_TRANSPOSE, E.OP_RESIZE):
        assert L.spinn_op_registered(op) == 1
    # unfused nodes keep the reference's arity checks
    for op in (E.OP_ADD, E.OP_SUB, E.OP_MUL, E.OP_DIV):
        assert L.spinn_dispatch_op(op, empty, 1, None, 0, empty, 1) == -1
    assert L.spinn_dispatch_op(E.OP_BN, empty, 4, None, 0, empty, 1) == -1
    for op in (E.OP_RELU, E.OP_SIGMOID, E.OP_SOFTMAX, E.OP_CONCAT, E.OP_SPLIT, E.OP_TRANSPOSE, E.OP_RESIZE):
        assert L.spinn_dispatch_op(op, empty, 0, None, 0, empty, 1) == -1


def test_conv_algo_selection(native):
    L = native.lib()

    def algo(*a):
        n, c, h, w, oc, k, s, p, g = a
        oh = (h + 2 * p - k) // s + 1
        d = native.ConvDesc(n, c, h, w, oc, oh, oh, k, k, s, s, p, p, g, 0, 0, 0)
        return L.spinn_hip_conv_select_algo(C.byref(d))

    assert algo(32, 256, 14, 14, 256, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43
    assert algo(32, 128, 28, 28, 128, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43
    assert algo(1, 256, 14, 14, 256, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM  # 16 4x4 tiles: too few
    assert algo(2, 256, 14, 14, 256, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM  # 32
    assert algo(4, 256, 14, 14, 256, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43   # 64
    assert algo(32, 64, 56, 56, 64, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43    # 64 channels, 6272 4x4 tiles
    assert algo(1, 64, 56, 56, 64, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM    # 64 channels, 196 4x4 tiles
    assert algo(2, 64, 56, 56, 64, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM    # 392: below 512
    assert algo(4, 64, 56, 56, 64, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43     # 784
    assert algo(32, 512, 7, 7, 512, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43    # 128 4x4 tiles
    assert algo(1, 512, 7, 7, 512, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM    # 4
    assert algo(4, 512, 7, 7, 512, 3, 1, 1, 1) == native.ALGO_WINOGRAD         # 16 tiles at K = 512: F(2,3)
    assert algo(8, 512, 7, 7, 512, 3, 1, 1, 1) == native.ALGO_WINOGRAD         # 32
    assert algo(12, 512, 7, 7, 512, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43    # 48
    assert algo(1, 128, 28, 28, 128, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM  # 49 4x4 tiles
    assert algo(4, 256, 20, 20, 64, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM   # 64 out: 100 tiles
    assert algo(16, 256, 20, 20, 64, 3, 1, 1, 1) == native.ALGO_WINOGRAD_F43   # 400 tiles
    assert algo(8, 32, 80, 80, 32, 3, 1, 1, 1) == native.ALGO_IMPLICIT_GEMM    # 32 channels
    assert algo(1, 256, 14, 14, 256, 3, 2, 1, 1) == native.ALGO_IMPLICIT_GEMM
    assert algo(1, 128, 20, 20, 128, 3, 2, 1, 128) == native.ALGO_DIRECT
    assert algo(16, 3, 640, 640, 16, 3, 2, 1, 1) == native.ALGO_DIRECT          # RGB stem into 16 channels
    assert algo(32, 3, 224, 224, 64, 7, 2, 3, 1) == native.ALGO_IMPLICIT_GEMM   # ResNet stem: matrix cores
    assert algo(1, 6, 8, 8, 4, 3, 1, 1, 4) == native.SPINN_HIP_EINVAL  # C % group != 0

    def workspace(*a):
        n, c, h, w, oc, k, s, p, g = a
        oh = (h + 2 * p - k) // s + 1
        d = native.ConvDesc(n, c, h, w, oc, oh, oh, k, k, s, s, p, p, g, 0, native.ALGO_IMPLICIT_GEMM, 0)
        return L.spinn_hip_conv_workspace_size(C.byref(d))

    # batch-1 grids under 256 CUs: the wave-K kernel needs no workspace, split K does
    assert workspace(1, 128, 20, 20, 128, 3, 1, 1, 1) == 0       # K 1152 over 200 16x16 tiles: wave-K
    assert workspace(1, 256, 20, 20, 64, 3, 1, 1, 1) > 0         # K 2304: split K
    assert workspace(1, 256, 14, 14, 256, 3, 1, 1, 1) > 0        # 208 16x16 tiles: split K
    assert workspace(1, 128, 20, 20, 256, 1, 1, 0, 1) == 0       # 1x1, K 128: wave-K
    assert workspace(4, 1024, 14, 14, 256, 1, 1, 0, 1) == 0      # K 1024 over 52 tiles: wave-K, no split
    assert workspace(8, 1024, 14, 14, 512, 1, 1, 0, 1) == 0      # 200 tiles: 64 x 64 unsplit
    assert workspace(8, 2048, 7, 7, 512, 1, 1, 0, 1) > 0         # K 2048 over 56 tiles: split K
    # 16 splits of 16 tiles fill the CUs; 16 splits of 8 tiles would not: 32 splits of 144
    assert workspace(1, 256, 14, 14, 256, 3, 1, 1, 1) == 16 * 256 * 196 * 4
    assert workspace(1, 512, 7, 7, 512, 3, 1, 1, 1) == 32 * 512 * 49 * 4


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(spinn_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol(native):
    names = _declared_functions()
    assert len(names) >= 40
    L = C.CDLL(str(native.LIB_PATH))
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes signature table covers the header
    assert not (names - set(native.exported_symbols()) - {"spinn_op_registered"}), \
        names - set(native.exported_symbols())


def test_bench_refuses_multi_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_traffic_summary_scaling(tmp_path, monkeypatch):
    """The counter reduction: calibration factors from the known-size copy/fill,
    first launch of each dropped, only conv_igemm_kernel dispatches averaged."""
    import sys
    sys.path.insert(0, str(ROOT))
    import bench

    kib = bench.CALIB_BYTES // 1024

    def write(name, rows):
        lines = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"]
        lines += [f"{i},{k},X,{v}" for i, (k, v) in enumerate(rows)]
        (tmp_path / f"{name}_counter_collection.csv").write_text("\n".join(lines) + "\n")

    # counters read half the copy's true bytes and the fill's exactly; cold first launches differ
    write("calib_FETCH_SIZE", [("fill_u32_kernel", 7), ("fill_u32_kernel", 5), ("copy_kernel", 999),
                               ("copy_kernel", kib / 2), ("copy_kernel", kib / 2)])
    write("calib_WRITE_SIZE", [("fill_u32_kernel", 1), ("fill_u32_kernel", kib), ("fill_u32_kernel", kib),
                               ("copy_kernel", kib)])
    write("r101_FETCH_SIZE", [("void conv_igemm_kernel<64>", 100.0), ("maxpool_kernel", 5000.0),
                              ("void conv_igemm_kernel<128>", 300.0)])
    write("r101_WRITE_SIZE", [("void conv_igemm_kernel<64>", 10.0), ("void conv_igemm_kernel<128>", 30.0)])
    monkeypatch.setattr(bench, "igemm_algorithmic_bytes", lambda b, p: 1.0)
    s = bench.traffic_summary(tmp_path, 32, "auto", [])
    assert s["calibration"]["fetch_factor"] == 2.0 and s["calibration"]["write_factor"] == 1.0
    assert s["dispatches"] == 2
    assert s["fetch_bytes_per_launch"] == 200 * 1024 * 2
    assert s["write_bytes_per_launch"] == 20 * 1024
    assert s["traffic_bytes_per_launch"] == 200 * 1024 * 2 + 20 * 1024


def test_bench_roofline_trace_summary(tmp_path):
    """The roofline-pass trace reduction: a shape's calls start after its weight packing,
    a split-K call's reduction launch counts into that call, other kernels are ignored,
    and the per-launch mean is weighted by each shape's layer count."""
    import json
    import sys
    sys.path.insert(0, str(ROOT))
    import bench

    rows, t = [], 0

    def k(name, us):
        nonlocal t
        rows.append((name, t, t + int(us * 1000)))
        t += int(us * 1000) + 500

    k("void spinn::fill_random_kernel(float*, unsigned long)", 3.0)  # before any shape: ignored
    k("void spinn::conv_pack_wt_kernel(float const*, float*)", 2.0)
    k("void spinn::conv_pack_kcopy_kernel(float const*, float*)", 1.0)
    for _ in range(4):  # shape 1: split-K, 10 + 2 us per call
        k("void spinn::conv_igemm_kernel<64, 64, 16, spinn::Im2colTapLoader<64, 16>, true, 0>(spinn::ConvKArgs)", 10.0)
        k("void spinn::conv_splitk_reduce_kernel(float const*, int)", 2.0)
    k("void spinn::conv_pack_wt_kernel(float const*, float*)", 2.0)
    for _ in range(4):  # shape 2: one kernel of 30 us per call
        k("void spinn::conv_igemm_sk_kernel<64, 64, 16, spinn::Pointwise1x1Loader<64, 16>, 1, 1>(spinn::ConvKArgs, "
          "spinn::SkSched)", 30.0)
    k("void spinn::xcc_id_kernel(unsigned int*)", 4.0)  # ignored
    lines = ["Kernel_Name,Start_Timestamp,End_Timestamp"] + [f'"{n}",{a},{b}' for n, a, b in rows]
    (tmp_path / "trace.csv").write_text("\n".join(lines) + "\n")
    (tmp_path / "pass.json").write_text(json.dumps({
        "launch_us": 26.0, "gflop_per_launch": 2.6, "achieved": 100.0,
        "shapes": [{"layer": "a", "count": 1, "us": 12.0}, {"layer": "b", "count": 3, "us": 30.0}]}) + "\n")
    md = bench.roofline_trace_summary(tmp_path / "trace.csv", tmp_path / "pass.json")
    assert "| a | 1 | conv_igemm_kernel | 4 | 12.00 | 12.00 | +0.0 % |" in md
    assert "| b | 3 | conv_igemm_sk_kernel | 4 | 30.00 | 30.00 | +0.0 % |" in md
    # (12 * 1 + 30 * 3) / 4 = 25.5 us; 2.6 GFLOP / 25.5 us = 102.0 TFLOP/s
    assert "rocprof 25.50 us, bench.py 25.50 us" in md and "rocprof 102.0 TFLOP/s" in md


def _hdr_fields(data):
    """(entry table offset, graph meta offset, tensor meta offset) of an ENNF image."""
    f = E._HDR.unpack_from(data, 0)
    return f[16], f[11], f[13]


def _crafted(tmp_path, name, patch):
    g, _ = models.conv_bn_relu(seed=0)
    data = bytearray(g.to_bytes())
    patch(g, data)
    p = tmp_path / f"{name}.ennf"
    p.write_bytes(bytes(data))
    return g, p


def test_loader_rejects_inconsistent_metadata(native, tmp_path):
    """Metadata that would size a launch or a copy wrongly is refused at load:
    an element count that is not the product of the dims, a byte size past 32
    bits, ndim above 8, graph input / output ids past the tensor table."""
    L = native.lib()
    meta = E._META.size

    def elem_count_off_by_one(g, d):
        _, _, mo = _hdr_fields(d)
        off = mo + g.inputs[0] * meta + 36
        struct.pack_into("<I", d, off, struct.unpack_from("<I", d, off)[0] + 1)

    def huge_dims(g, d):
        _, _, mo = _hdr_fields(d)
        off = mo + g.inputs[0] * meta
        struct.pack_into("<B8II", d, off + 3, 2, 65536, 65536, 0, 0, 0, 0, 0, 0, 0)

    def ndim_nine(g, d):
        _, _, mo = _hdr_fields(d)
        struct.pack_into("<B", d, mo + g.inputs[0] * meta + 3, 9)

    def output_id_past_table(g, d):
        _, gm, _ = _hdr_fields(d)
        n_in = struct.unpack_from("<H", d, gm)[0]
        struct.pack_into("<H", d, gm + 2 + 2 * n_in + 2, len(g.tensors))

    def input_id_past_table(g, d):
        _, gm, _ = _hdr_fields(d)
        struct.pack_into("<H", d, gm + 2, 0xFFFF)

    for name, patch in [("count", elem_count_off_by_one), ("huge", huge_dims), ("ndim", ndim_nine),
                        ("out_id", output_id_past_table), ("in_id", input_id_past_table)]:
        _, p = _crafted(tmp_path, name, patch)
        assert not L.spinn_load(str(p).encode()), name
    # the unpatched file still loads
    _, p = _crafted(tmp_path, "ok", lambda g, d: None)
    ctx = L.spinn_load(str(p).encode())
    assert ctx
    L.spinn_free(ctx)


def test_plan_rejects_short_weight_payload(native, tmp_path):
    """A weight whose payload in the file is shorter than its tensor is refused by
    spinn_plan before any device work (no host over-read by the upload)."""
    L = native.lib()

    def short_weight(g, d):
        eo, _, _ = _hdr_fields(d)
        wid = next(t.id for t in g.tensors if t.is_weight and t.data.size > 4)
        off = eo + wid * E._ENTRY.size + 8
        struct.pack_into("<I", d, off, struct.unpack_from("<I", d, off)[0] - 4)

    _, p = _crafted(tmp_path, "short", short_weight)
    ctx = L.spinn_load(str(p).encode())
    assert ctx
    try:
        assert L.spinn_plan(ctx, 0) == -1
    finally:
        L.spinn_free(ctx)


def test_headline_layer_list_matches_resnet101():
    """The per-layer GPU parity list is exactly ResNet-101's distinct conv layers."""
    from tests.test_gpu_headline import R101_LAYERS
    g, _ = models.resnet101(batch=1, seed=0)
    seen = {}
    for nd in g.nodes:
        if nd.op != E.OP_CONV:
            continue
        p = E.unpack_conv_params(nd.params)
        _, c, h, w = g.dims(nd.inputs[0])
        oc, _, k, _ = g.dims(nd.inputs[1])
        key = (c, h, w, oc, k, p["strides"][0], p["pads"][0], p["act"])
        seen[key] = seen.get(key, 0) + 1
    assert {tuple(l[:8]): l[8] for l in R101_LAYERS} == seen
