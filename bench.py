#!/usr/bin/env python3
"""Benchmark: ResNet-101 v1.5 fp32 forward on one MI355X through the ENNF runtime.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward pass of ResNet-101 (batch 32, 224x224, random-init with
BN folded) through spinn_run over a single HBM arena, with the input already
in HBM (spinn_run_resident: each step copies the staged input into its arena
region device to device, as the reference's spinn_run copies its host input on
every call, then replays the node loop from a HIP graph). Prints ONE JSON line:

  value             images/s at batch 32 (whole job = the one GPU)
  images_per_s_b1   images/s at batch 1 (same protocol)
  roofline          the implicit-GEMM conv kernel: direct-conv FLOPs of the
                    layers it runs / their summed kernel time, each layer's
                    kernel launched 10 times back to back between two HIP
                    events on its stream with random operands, against the
                    157.3 TFLOP/s fp32 MFMA peak (achieved_node_events: the
                    same ratio from HIP events recorded around every node of K
                    profiled model passes; frac_of_layer_rooflines: against
                    each layer's own MFMA-or-HBM bound)
  conv_*            the per-node-event aggregate over every conv layer
                    (Winograd layers credited at the direct-conv FLOP count)
  other_configs     config 0 (one Conv3x3+BN+ReLU), the Gemm sweep, the VGG
                    3x3 stack (implicit GEMM vs Winograd), YOLOv10n at batch 1
                    and 16 with operator families and the depthwise layers'
                    achieved HBM bandwidth (live back-to-back launches)
  cpu_baseline      the oracle's restatement of SPINN's CPU path (specified
                    epilogue) on this host's cores and on 4 threads, plus the
                    reference's own runtime as shipped when built; ResNet-101
                    batch 1, a bounded sample

Per-layer GFLOP/s and % of peak go to the --layers-out JSON file (per node,
from events) and the Markdown file beside it (per distinct layer shape, from
back-to-back launches, with Winograd's executed FLOPs).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "conv-layer fp32 GFLOP/s (% MFMA peak); ResNet-101 images/sec @ b1/b32, 1 GPU"
PEAK_FP32_MFMA = 157.3e12  # MI355X dense fp32 matrix peak, FLOP/s
ALGO_NAMES = {1: "implicit_gemm", 2: "winograd", 3: "direct", 4: "winograd_f43"}


def host_threads() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def host_cpu() -> str:
    """CPU model and physical core count of this host, from lscpu."""
    try:
        info = dict(l.split(":", 1) for l in subprocess.run(["lscpu"], capture_output=True, text=True,
                                                             timeout=10).stdout.splitlines() if ":" in l)
        sockets = int(info.get("Socket(s)", "1").strip() or 1)
        cores = int(info.get("Core(s) per socket", "0").strip() or 0) * sockets
        return f"{info.get('Model name', '?').strip()}, {cores} physical cores, {os.cpu_count()} logical"
    except Exception:
        return "unknown"


def _cpu_run(kind: str, model: Path, in_shape, out_shape, seconds: float, threads: int) -> dict | None:
    """One oracle.cpu_bench process (the OpenMP thread count is fixed per process)."""
    env = dict(os.environ, OMP_NUM_THREADS=str(threads))
    cmd = [sys.executable, "-m", "oracle.cpu_bench", "--kind", kind, "--model", str(model),
           "--in-shape", ",".join(map(str, in_shape)), "--out-shape", ",".join(map(str, out_shape)),
           "--seconds", str(seconds)]
    try:
        r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=seconds * 6 + 120)
    except subprocess.TimeoutExpired:
        return None
    if r.returncode != 0:
        print(r.stderr[-2000:], file=sys.stderr)
        return None
    res = json.loads(r.stdout.strip().splitlines()[-1])
    res["images_per_s"] = res["batch"] / (res["avg_ms"] / 1e3)
    return res


def cpu_baseline(model_b1: Path, in_shape, out_shape, seconds: float, label: str = "ResNet-101") -> dict | None:
    """The CPU path timed on this host: the oracle's C restatement of SPINN's algorithm
    (im2col + packed 6x16 AVX2 GEMM tiles, K block 256, N block 128, OpenMP over tiles,
    with the epilogue as the reference specifies it) on all the host threads available,
    then on 4 threads (the thread count of SPINN/OPTIMIZATION_PROGRESS.md:4), and the
    reference's own runtime as shipped (oracle/_ref, which drops bias / activation /
    residual on group-1 convs, SPINN/run_time/ops/mm/gemm_kernel.c:497-590) when built.
    Protocol of SPINN/run_time/main.c:42,83-108: 3 warm-ups, then runs until the time
    budget is spent; mean wall time per run including the input and output copies."""
    threads = host_threads()
    port = _cpu_run("port", model_b1, in_shape, out_shape, seconds, threads)
    if port is None:
        return None
    out = {"value": round(port["images_per_s"], 3), "unit": "images/s", "cores": threads, "kind": "port",
           "sample": (f"{label} batch {port['batch']} forward through the restated SPINN CPU path (specified "
                      f"epilogue), {port['runs']} runs after 3 warm-up (reference CLI protocol), ~{seconds:.0f} s "
                      f"budget, OpenMP {threads} threads; best {port['best_ms']:.1f} ms, mean "
                      f"{port['avg_ms']:.1f} ms per forward"),
           "host": host_cpu()}
    if threads != 4:
        p4 = _cpu_run("port", model_b1, in_shape, out_shape, seconds / 2, 4)
        if p4:
            out["threads_4"] = {"value": round(p4["images_per_s"], 3), "best_ms": round(p4["best_ms"], 2),
                                "avg_ms": round(p4["avg_ms"], 2), "runs": p4["runs"]}
    if (ROOT / "oracle" / "_ref" / "libspinn_ref.so").exists():
        ref = _cpu_run("reference", model_b1, in_shape, out_shape, seconds / 2, threads)
        if ref:
            out["reference_as_shipped"] = {
                "value": round(ref["images_per_s"], 3), "best_ms": round(ref["best_ms"], 2),
                "avg_ms": round(ref["avg_ms"], 2), "runs": ref["runs"], "threads": threads,
                "note": "the reference's own runtime built from its sources; it skips the epilogue of group-1 "
                        "convs, so it does less work than the specified path"}
    return out


def conv_table(g):
    """Per Conv node: (node index, descriptor fields, direct-conv FLOPs)."""
    from spinn_amd import ennf as E
    rows = []
    for i, nd in enumerate(g.nodes):
        if nd.op != E.OP_CONV:
            continue
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, cg, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        rows.append(dict(node=i, n=n, c=c, h=h, w=w, oc=oc, oh=oh, ow=ow, kh=kh, kw=kw, sh=p["strides"][0],
                         sw=p["strides"][1], ph=p["pads"][0], pw=p["pads"][1], group=p["group"] or 1,
                         act=p["act"], flops=2.0 * n * oc * oh * ow * cg * kh * kw))
    return rows


def algo_of(N, r, policy) -> int:
    import ctypes as C
    d = N.ConvDesc(r["n"], r["c"], r["h"], r["w"], r["oc"], r["oh"], r["ow"], r["kh"], r["kw"], r["sh"], r["sw"],
                   r["ph"], r["pw"], r["group"], r["act"], 0, 0)
    a = N.lib().spinn_hip_conv_select_algo(C.byref(d))
    if a in (N.ALGO_WINOGRAD, N.ALGO_WINOGRAD_F43) and policy == N.POLICY_IGEMM:
        return N.ALGO_IMPLICIT_GEMM
    if a == N.ALGO_IMPLICIT_GEMM and policy == N.POLICY_WINOGRAD and r["kh"] == 3 and r["kw"] == 3 \
            and r["sh"] == 1 and r["sw"] == 1 and r["group"] == 1:
        return N.ALGO_WINOGRAD_F43
    return a


def profiled_node_ms(N, Session, path, x, policy, steps: int, warmup: int):
    """Mean per-node device time (ms) over `steps` eager runs, from HIP events
    recorded on the runtime's stream before and after every node."""
    L = N.lib()
    L.spinn_set_profiling(1)
    s = Session(path, policy=policy, graph=False)
    s.upload_input(x)
    for _ in range(warmup):
        s.run_resident()
    acc = None
    for _ in range(steps):
        s.run_resident()
        t = s.node_times()
        acc = t if acc is None else acc + t
    s.close()
    L.spinn_set_profiling(0)
    return acc / steps


def suite(N, Session, models, reps: int = 100, yolo_cpu: dict | None = None) -> dict:
    """The other benchmark configurations, each on its own:
    cfg0   single fused Conv3x3+BN+ReLU 1x64x56x56 through spinn_hip_conv
           (kernel time: 20 launches in a HIP graph replayed between events;
           us_host_launches: back-to-back host launches, which the host's launch
           rate bounds at these sizes) and through spinn_run with host copies;
    gemm   the Gemm sweep (transB=1, bias vector, alpha=beta=1) through spinn_hip_gemm,
           against the MFMA roofline or, for arithmetic intensity under the
           19.7 flop/B ridge, the HBM roofline;
    vgg    the 8-layer 3x3 stack at batch 8 under the implicit-GEMM and the
           Winograd policy: images/s, direct-conv-equivalent TFLOP/s and how far
           the two outputs are apart (relative L2);
    yolo   YOLOv10n 640x640 at batch 1 and 16 (see yolo_bench)."""
    import ctypes as C
    from spinn_amd.devbuf import DeviceBuffer, time_cold, time_graph, time_launches
    L = N.lib()
    out = {}
    g, x = models.conv_bn_relu(seed=0)
    conv = g.nodes[0]  # the fused Conv: inputs x, folded weight, folded bias
    wt, bias = g.tensors[conv.inputs[1]].data, g.tensors[conv.inputs[2]].data
    d = N.ConvDesc(1, 64, 56, 56, 64, 56, 56, 3, 3, 1, 1, 1, 1, 1, N.ACT_RELU, 0, 0)
    d.algo = L.spinn_hip_conv_select_algo(C.byref(d))
    bx, bw, bb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(wt), DeviceBuffer.from_array(bias)
    by = DeviceBuffer(4 * 64 * 56 * 56)
    bp = DeviceBuffer(L.spinn_hip_conv_packed_size(C.byref(d)))
    wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
    bws = DeviceBuffer(wsz) if wsz else None
    N.check(L.spinn_hip_conv_pack_weights(C.byref(d), bw.ptr, bp.ptr, None), "pack")
    conv0 = lambda st: L.spinn_hip_conv(C.byref(d), bx.ptr, bw.ptr, bp.ptr, bb.ptr, None, by.ptr,  # noqa: E731
                                        bws.ptr if bws else None, wsz, st)
    ms = time_graph(conv0, 20)
    ms_host = time_launches(lambda: conv0(None), 2 * reps)
    flops = 2.0 * 64 * 56 * 56 * 64 * 9
    byts = 4.0 * (x.size + wt.size + bias.size + 64 * 56 * 56)
    tmp = Path(tempfile.mkdtemp(prefix="spinn_suite_"))
    with Session(g.write(tmp / "cfg0.ennf")) as s0:
        for _ in range(5):
            s0.run(x)
        t0 = time.perf_counter()
        for _ in range(reps):
            s0.run(x)
        run_ms = (time.perf_counter() - t0) / reps * 1e3
    out["cfg0_conv3x3_bn_relu"] = {"kernel_us": round(ms * 1e3, 3),
                                   "us_host_launches": round(ms_host * 1e3, 3),
                                   "gflops": round(flops / (ms * 1e-3) / 1e9, 1),
                                   "frac_mfma_peak": round(flops / (ms * 1e-3) / PEAK_FP32_MFMA, 4),
                                   "roofline_us": round(max(flops / PEAK_FP32_MFMA, byts / 8e12) * 1e6, 3),
                                   "spinn_run_ms_with_host_copies": round(run_ms, 4)}
    for b_ in (bx, bw, bb, by, bp) + ((bws,) if bws else ()):
        b_.free()
    gemms = []
    fa, fb = DeviceBuffer(FLUSH_BYTES), DeviceBuffer(FLUSH_BYTES)
    flush = lambda: N.check(L.spinn_hip_copy(fb.ptr, fa.ptr, FLUSH_BYTES, None), "flush")  # noqa: E731
    for (m, n, k) in models.GEMM_SWEEP:
        rng = np.random.default_rng(m * 7 + n)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
        c = rng.normal(0, 0.01, n).astype(np.float32)
        gd = N.GemmDesc(m, n, k, 0, 1, 1, 1.0, 1.0, 1, 0, 0, 0, 0)
        ba, bb2, bc, by2 = (DeviceBuffer.from_array(a), DeviceBuffer.from_array(b), DeviceBuffer.from_array(c),
                            DeviceBuffer(4 * m * n))
        wsz = L.spinn_hip_gemm_workspace_size(C.byref(gd))
        bws = DeviceBuffer(wsz) if wsz else None
        gemm = lambda st: L.spinn_hip_gemm(C.byref(gd), ba.ptr, bb2.ptr, bc.ptr, by2.ptr,  # noqa: E731
                                           bws.ptr if bws else None, wsz, st)
        ms = time_graph(gemm, 20)
        ms_host = time_launches(lambda: gemm(None), reps)
        f = 2.0 * m * n * k
        byts = 4.0 * (m * k + n * k + n + m * n)
        bound = "hbm" if f / byts < PEAK_FP32_MFMA / 8e12 else "mfma"
        frac = (byts / (ms * 1e-3) / 8e12) if bound == "hbm" else (f / (ms * 1e-3) / PEAK_FP32_MFMA)
        ent = {"mnk": [m, n, k], "us": round(ms * 1e3, 3), "us_host_launches": round(ms_host * 1e3, 3),
               "gflops": round(f / (ms * 1e-3) / 1e9, 1),
               "gbps": round(byts / (ms * 1e-3) / 1e9, 1), "bound": bound, "frac_roofline": round(frac, 4)}
        if bound == "hbm":
            # back to back, the 8 MB weight matrix stays in the 256 MB Infinity Cache (MALL);
            # after a 512 MiB copy it comes from HBM
            ms_c = time_cold(lambda: L.spinn_hip_gemm(C.byref(gd), ba.ptr, bb2.ptr, bc.ptr, by2.ptr,
                                                      bws.ptr if bws else None, wsz, None), flush, 20)
            ent["us_mall_resident"] = ent["us"]
            ent["us_after_flush"] = round(ms_c * 1e3, 3)
            ent["frac_hbm_after_flush"] = round(byts / (ms_c * 1e-3) / 8e12, 4)
        gemms.append(ent)
        for b_ in (ba, bb2, bc, by2) + ((bws,) if bws else ()):
            b_.free()
    fa.free()
    fb.free()
    out["gemm_sweep"] = gemms
    gv, xv = models.vgg_stack(batch=8, seed=0)
    pv = gv.write(tmp / "vgg_b8.ennf")
    vgg_flops = sum(f for _, f in models.conv_flops(gv))
    res = {}
    outs = {}
    for name, pol in (("implicit_gemm", N.POLICY_IGEMM), ("winograd", N.POLICY_WINOGRAD)):
        with Session(pv, policy=pol, graph=True) as sv:
            yv = sv.run(xv)
            sv.upload_input(xv)
            msv = time_steps(sv, max(10, reps // 10), 3, ref=yv)
            outs[name] = yv
        res[name] = {"ms": round(msv, 4), "images_per_s": round(8 / (msv * 1e-3), 1),
                     "tflops_direct_equiv": round(vgg_flops / (msv * 1e-3) / 1e12, 2)}
    dv = outs["winograd"].astype(np.float64) - outs["implicit_gemm"]
    res["winograd_vs_igemm_rel_l2"] = float(np.linalg.norm(dv) / np.linalg.norm(outs["implicit_gemm"]))
    res["winograd_vs_igemm_max_abs"] = float(np.abs(dv).max())
    res["output_max_abs"] = float(np.abs(outs["implicit_gemm"]).max())
    res["gflop_direct_equiv"] = round(vgg_flops / 1e9, 2)
    out["vgg3x3_stack_b8"] = res
    out["yolov10n"] = yolo_bench(N, Session, models, tmp, reps)
    out["yolov10n"]["cpu_baseline_b1"] = yolo_cpu
    return out


def _op_family(N, nd, g, policy) -> str:
    from spinn_amd import ennf as E
    if nd.op == E.OP_CONV:
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, cg, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        r = dict(n=n, c=c, h=h, w=w, oc=oc, oh=oh, ow=ow, kh=kh, kw=kw, sh=p["strides"][0], sw=p["strides"][1],
                 ph=p["pads"][0], pw=p["pads"][1], group=p["group"] or 1, act=p["act"])
        return "conv_" + ALGO_NAMES.get(algo_of(N, r, policy), "?")
    return {E.OP_ADD: "add", E.OP_SUB: "sub", E.OP_MUL: "mul", E.OP_CONCAT: "concat", E.OP_SPLIT: "split",
            E.OP_MAXPOOL: "maxpool", E.OP_RESIZE: "resize", E.OP_RESHAPE: "reshape", E.OP_TRANSPOSE: "transpose",
            E.OP_MATMUL: "matmul", E.OP_SOFTMAX: "softmax", E.OP_SIGMOID: "sigmoid", E.OP_TOPK: "topk",
            E.OP_REDUCEMAX: "reducemax", E.OP_GATHER_ELEMENTS: "gather_elements", E.OP_TILE: "tile",
            E.OP_UNSQUEEZE: "unsqueeze", E.OP_FLATTEN: "flatten", E.OP_MOD: "mod", E.OP_DIV: "div",
            E.OP_CAST: "cast"}.get(nd.op, f"op{nd.op}")


def copy_nodes_live(N, g, reps: int = 10) -> dict:
    """Achieved bandwidth of a graph's Concat and Split nodes: each node's block copies,
    built as the runtime's op_concat / op_split builds them (runs of dims[axis] * inner
    elements per outer index, SPINN/run_time/ops/tensor/concat.c:5-26, split.c:5-26), are
    launched through spinn_hip_block_copy `reps` times in a HIP graph replayed between HIP
    events; bytes = every element read once and written once."""
    import ctypes as C
    import struct
    from spinn_amd import ennf as E
    from spinn_amd.devbuf import DeviceBuffer, time_graph
    L = N.lib()
    out = {}
    for op, name in ((E.OP_CONCAT, "concat"), (E.OP_SPLIT, "split")):
        nodes = [nd for nd in g.nodes if nd.op == op]
        if not nodes:
            continue
        tot_ms = tot_b = 0.0
        for nd in nodes:
            axis = struct.unpack_from("<i", nd.params)[0] if len(nd.params) >= 4 else 0
            src = nd.inputs if op == E.OP_CONCAT else [nd.inputs[0]]
            dst = [nd.outputs[0]] if op == E.OP_CONCAT else nd.outputs
            dims = g.dims(src[0])
            axis = axis + len(dims) if axis < 0 else axis
            outer = int(np.prod(dims[:axis])) if axis > 0 else 1
            inner = int(np.prod(dims[axis + 1:])) if axis + 1 < len(dims) else 1
            pieces = src if op == E.OP_CONCAT else dst
            lens = [g.dims(t)[axis] * inner for t in pieces]
            row = sum(lens)
            whole = DeviceBuffer(4 * outer * row)
            parts = [DeviceBuffer(4 * outer * n) for n in lens]
            blocks = (N.BlockCopy * len(lens))()
            off = 0
            for i, (n, b) in enumerate(zip(lens, parts)):
                if op == E.OP_CONCAT:
                    blocks[i] = N.BlockCopy(b.ptr, whole.ptr, n, 0, row, off, n)
                else:
                    blocks[i] = N.BlockCopy(whole.ptr, b.ptr, row, off, n, 0, n)
                off += n
            def launch(st, blocks=blocks, nb=len(lens), outer=outer):
                rc = 0
                for i0 in range(0, nb, 16):  # SPINN_HIP_MAX_BLOCKS per launch, as op_concat / op_split do
                    sub = C.cast(C.byref(blocks, i0 * C.sizeof(N.BlockCopy)), C.POINTER(N.BlockCopy))
                    rc = rc or L.spinn_hip_block_copy(sub, min(16, nb - i0), outer, st)
                return rc
            ms = time_graph(launch, reps)
            tot_ms += ms
            tot_b += 2 * 4.0 * outer * row
            for b in parts + [whole]:
                b.free()
        out[name] = {"nodes": len(nodes), "bytes": int(tot_b), "kernel_us": round(tot_ms * 1e3, 1),
                     "achieved": round(tot_b / (tot_ms * 1e-3) / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(tot_b / (tot_ms * 1e-3) / 8e12, 4)}
    return out


def yolo_bench(N, Session, models, tmp: Path, reps: int) -> dict:
    """YOLOv10n 640x640 at batch 1 and 16, the whole exported graph including the
    TopK post-processing tail (output [B, 300, 6]): images/s (graph replay, input
    resident), direct-conv-equivalent conv TFLOP/s, and at batch 16 the device
    time per operator family from HIP events around every node."""
    res = {}
    for b in (1, 16):
        g, x = models.yolov10n(batch=b, seed=0, postprocess=True)
        path = g.write(tmp / f"y10_b{b}.ennf")
        with Session(path, graph=True) as s:
            yh = s.run(x)
            s.upload_input(x)
            ms = time_steps(s, max(20, reps // 2) if b == 1 else max(10, reps // 10), 3, ref=yh)
        gf = sum(f for _, f in models.conv_flops(g))
        ent = {"ms": round(ms, 4), "images_per_s": round(b / (ms * 1e-3), 1),
               "conv_tflops_direct_equiv": round(gf / (ms * 1e-3) / 1e12, 2), "conv_gflop": round(gf / 1e9, 3)}
        if b == 16:
            node_ms = profiled_node_ms(N, Session, path, x, N.POLICY_AUTO, 5, 2)
            fam = {}
            for i, nd in enumerate(g.nodes):
                k = _op_family(N, nd, g, N.POLICY_AUTO)
                f = fam.setdefault(k, [0, 0.0])
                f[0] += 1
                f[1] += float(node_ms[i])
            dw = [r for r in conv_table(g) if r["group"] > 1 and r["group"] == r["c"] == r["oc"]]
            dw_ms, _, dw_b, n_dw = conv_kernels_live(N, dw, N.ALGO_DIRECT)
            if dw_ms > 0:
                ent["depthwise_bandwidth"] = {
                    "layers": n_dw, "bytes": int(dw_b), "kernel_us": round(dw_ms * 1e3, 1),
                    "achieved": round(dw_b / (dw_ms * 1e-3) / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                    "frac": round(dw_b / (dw_ms * 1e-3) / 8e12, 4),
                    "method": "input + weights + bias + output (+ residual) bytes of the depthwise layers / their "
                              "kernel time, each layer launched 10x back to back in a HIP graph replayed between "
                              "HIP events"}
            ent["copy_bandwidth"] = copy_nodes_live(N, g)
            ent["node_ms_total"] = round(float(node_ms.sum()), 4)
            ent["families_ms"] = {k: {"nodes": v[0], "ms": round(v[1], 4)}
                                  for k, v in sorted(fam.items(), key=lambda kv: -kv[1][1])}
        res[f"b{b}"] = ent
        print(f"[bench] yolov10n b{b}: {ms:.3f} ms", file=sys.stderr, flush=True)
    return res


TRAFFIC_FILE = ROOT / "profiles" / "conv_igemm_traffic_resnet101_b32.json"
FLUSH_BYTES = 512 << 20  # twice the 256 MB Infinity Cache


def fill_random(buf, seed: int, scale: float = 1.0) -> None:
    """Fill a DeviceBuffer with float32 values uniform in [-scale, scale).
    Timed operands are never zero- or constant-filled: the matrix cores draw less
    power on such data and the chip holds a higher clock, which on MI355X made
    batch-32 conv layers 9-24 % faster than on random operands."""
    n = buf.nbytes // 4
    rng = np.random.default_rng(seed)
    chunk = 1 << 24
    host = np.empty(n, np.float32)
    for i in range(0, n, chunk):
        host[i:i + chunk] = rng.uniform(-scale, scale, min(chunk, n - i)).astype(np.float32)
    buf.upload(host)
CALIB_BYTES = 256 << 20


def calibration_kernels() -> None:
    """Known-size traffic for scaling the FETCH_SIZE / WRITE_SIZE counters:
    three 256 MiB fills (write only) then three 256 MiB device copies (read +
    write) through the library's own kernels."""
    from spinn_amd import native as N
    from spinn_amd.devbuf import DeviceBuffer
    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")
    a, b = DeviceBuffer(CALIB_BYTES), DeviceBuffer(CALIB_BYTES)
    for _ in range(3):
        N.check(L.spinn_hip_fill_u32(a.ptr, 7, CALIB_BYTES, None), "fill")
    for _ in range(3):
        N.check(L.spinn_hip_copy(b.ptr, a.ptr, CALIB_BYTES, None), "copy")
    N.check(L.spinn_hip_stream_sync(None), "sync")
    a.free()
    b.free()
    print("[bench] calibration kernels done", flush=True)


def small_launches(reps: int = 20) -> None:
    """Launches for a kernel profiler: the Conv3x3+BN+ReLU 1x64x56x56 layer, the five Gemm
    sweep shapes (transB=1, bias vector) and YOLOv10n's 13 depthwise layers at batch 16,
    `reps` launches each on the null stream (run it under rocprofv3 --kernel-trace --stats)."""
    import ctypes as C
    from spinn_amd import models
    from spinn_amd import native as N
    from spinn_amd.devbuf import DeviceBuffer
    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")
    g, x = models.conv_bn_relu(seed=0)
    rows = conv_table(g)
    gy, _ = models.yolov10n(batch=16, seed=0)
    rows += [r for r in conv_table(gy) if r["group"] > 1 and r["group"] == r["c"] == r["oc"]]
    nbytes = lambda *dims: 4 * int(np.prod(dims))  # noqa: E731
    for r in rows:
        d = N.ConvDesc(*(r[f] for f in CONV_FIELDS), 0, 0)
        d.algo = L.spinn_hip_conv_select_algo(C.byref(d))
        bx = DeviceBuffer(nbytes(r["n"], r["c"], r["h"], r["w"]))
        bw = DeviceBuffer(nbytes(r["oc"], r["c"] // r["group"], r["kh"], r["kw"]))
        bb = DeviceBuffer(nbytes(r["oc"]))
        by = DeviceBuffer(nbytes(r["n"], r["oc"], r["oh"], r["ow"]))
        br = DeviceBuffer(nbytes(r["n"], r["oc"], r["oh"], r["ow"])) if r["act"] in (4, 5) else None
        for i, b_ in enumerate((bx, bw, bb, by) + ((br,) if br else ())):
            fill_random(b_, seed=21 + i, scale=0.05 if b_ is bw else 1.0)
        psz = L.spinn_hip_conv_packed_size(C.byref(d))
        bp = DeviceBuffer(psz) if psz else None
        if bp:
            N.check(L.spinn_hip_conv_pack_weights(C.byref(d), bw.ptr, bp.ptr, None), "pack")
        wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
        ws = DeviceBuffer(wsz) if wsz else None
        for _ in range(reps):
            N.check(L.spinn_hip_conv(C.byref(d), bx.ptr, bw.ptr, bp.ptr if bp else None, bb.ptr,
                                     br.ptr if br else None, by.ptr, ws.ptr if ws else None, wsz, None), "conv")
        N.check(L.spinn_hip_stream_sync(None), "sync")
        for b_ in (bx, bw, bb, by, br, bp, ws):
            if b_:
                b_.free()
    for (m, n, k) in models.GEMM_SWEEP:
        gd = N.GemmDesc(m, n, k, 0, 1, 1, 1.0, 1.0, 1, 0, 0, 0, 0)
        ba, bb2, bc, by2 = DeviceBuffer(4 * m * k), DeviceBuffer(4 * n * k), DeviceBuffer(4 * n), DeviceBuffer(4 * m * n)
        for i, b_ in enumerate((ba, bb2, bc)):
            fill_random(b_, seed=31 + i, scale=1.0 if b_ is ba else 0.05)
        wsz = L.spinn_hip_gemm_workspace_size(C.byref(gd))
        ws = DeviceBuffer(wsz) if wsz else None
        for _ in range(reps):
            N.check(L.spinn_hip_gemm(C.byref(gd), ba.ptr, bb2.ptr, bc.ptr, by2.ptr, ws.ptr if ws else None, wsz,
                                     None), "gemm")
        N.check(L.spinn_hip_stream_sync(None), "sync")
        for b_ in (ba, bb2, bc, by2, ws):
            if b_:
                b_.free()
    print("[bench] small-config launches done", flush=True)


def clock_probe(reps: int = 200) -> None:
    """Launches for a clock comparison under rocprofv3 --pmc GRBM_GUI_ACTIVE GRBM_COUNT
    --kernel-trace: the 1024 -> 256 1x1 conv at 14x14, batch 32 (implicit GEMM), `reps`
    times on zero-filled operands, then `reps` times on random ones. Cycles per
    dispatch over the dispatch's duration compare the clock the chip holds on each."""
    import ctypes as C
    from spinn_amd import native as N
    from spinn_amd.devbuf import DeviceBuffer
    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")
    n, c, hw, oc = 32, 1024, 14, 256
    d = N.ConvDesc(n, c, hw, hw, oc, hw, hw, 1, 1, 1, 1, 0, 0, 1, 1, N.ALGO_IMPLICIT_GEMM, 0)
    bufs = [DeviceBuffer(4 * v) for v in (n * c * hw * hw, oc * c, oc, n * oc * hw * hw)]
    bx, bw, bb, by = bufs
    bp = DeviceBuffer(L.spinn_hip_conv_packed_size(C.byref(d)))
    wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
    ws = DeviceBuffer(wsz) if wsz else None
    for label in ("zeros", "random"):
        for i, b_ in enumerate(bufs):
            if label == "zeros":
                N.check(L.spinn_hip_fill_u32(b_.ptr, 0, b_.nbytes, None), "fill")
            else:
                fill_random(b_, seed=5 + i, scale=0.05 if i == 1 else 1.0)
        N.check(L.spinn_hip_conv_pack_weights(C.byref(d), bw.ptr, bp.ptr, None), "pack")
        N.check(L.spinn_hip_stream_sync(None), "sync")
        print(f"[bench] clock probe: {reps} launches on {label} operands", flush=True)
        for _ in range(reps):
            N.check(L.spinn_hip_conv(C.byref(d), bx.ptr, bw.ptr, bp.ptr, bb.ptr, None, by.ptr,
                                     ws.ptr if ws else None, wsz, None), "conv")
        N.check(L.spinn_hip_stream_sync(None), "sync")
    for b_ in bufs + [bp] + ([ws] if ws else []):
        b_.free()


def clock_summary(d: Path) -> str:
    """Per-dispatch GRBM_COUNT cycles and kernel-trace durations of a --clock-probe run
    (the first 20 launches of each half dropped)."""
    import csv
    cc = list(csv.DictReader(open(next(d.glob("*_counter_collection.csv")))))
    kt = list(csv.DictReader(open(next(d.glob("*_kernel_trace.csv")))))
    dur = {r["Dispatch_Id"]: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"]), r["Kernel_Name"]) for r in kt}
    cyc = {}
    for r in cc:
        if r["Counter_Name"] == "GRBM_COUNT":
            cyc[r["Dispatch_Id"]] = float(r["Counter_Value"])
    rows = sorted((int(k), dur[k][0], v) for k, v in cyc.items() if k in dur and "conv_igemm" in dur[k][1])
    half = len(rows) // 2
    lines = ["| operands | dispatches | mean duration us | mean GRBM_COUNT cycles | cycles / ns |", "|---|---|---|---|---|"]
    for name, part in (("zeros", rows[:half][20:]), ("random", rows[half:][20:])):
        du = sum(p[1] for p in part) / len(part)
        cy = sum(p[2] for p in part) / len(part)
        lines.append(f"| {name} | {len(part)} | {du / 1e3:.2f} | {cy:.0f} | {cy / du:.3f} |")
    return "\n".join(lines) + "\n"


COMPARE_LAYERS = [  # (n, c, h, w, oc, k, stride, pad, act): ResNet-101 batch-32 layers
    (32, 256, 14, 14, 1024, 1, 1, 0, 5),
    (32, 1024, 14, 14, 256, 1, 1, 0, 1),
    (32, 64, 56, 56, 64, 3, 1, 1, 1),
]


def gemm_compare(reps: int = 5) -> None:
    """Launches for the PMC comparison of the MFMA engine: three ResNet-101
    batch-32 conv layers through spinn_hip_conv (implicit GEMM, per-shape tiles),
    an 8192^3 fp32 Gemm through spinn_hip_gemm, and the same Gemm through torch
    (hipBLASLt), `reps` launches each; run it under rocprofv3 --pmc."""
    import ctypes as C
    import torch
    from spinn_amd import native as N
    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")
    P = lambda t: None if t is None else C.c_void_p(t.data_ptr())  # noqa: E731
    g = torch.Generator(device="cuda").manual_seed(0)
    for (n, c, h, w, oc, k, s, p, act) in COMPARE_LAYERS:
        oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
        d = N.ConvDesc(n, c, h, w, oc, oh, ow, k, k, s, s, p, p, 1, act, N.ALGO_IMPLICIT_GEMM, 0)
        x = torch.rand(n, c, h, w, device="cuda", generator=g)
        wt = torch.randn(oc, c, k, k, device="cuda", generator=g) * (2.0 / (c * k * k)) ** 0.5
        b = torch.zeros(oc, device="cuda")
        r = torch.rand(n, oc, oh, ow, device="cuda", generator=g) if act in (4, 5) else None
        y = torch.empty(n, oc, oh, ow, device="cuda")
        pk = torch.empty(max(L.spinn_hip_conv_packed_size(C.byref(d)) // 4, 1), device="cuda")
        N.check(L.spinn_hip_conv_pack_weights(C.byref(d), P(wt), P(pk), None), "pack")
        wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
        ws = torch.empty(max(wsz // 4, 1), device="cuda")
        for _ in range(reps):
            N.check(L.spinn_hip_conv(C.byref(d), P(x), P(wt), P(pk), P(b), P(r), P(y), P(ws), wsz, None), "conv")
    m = 8192
    a = torch.rand(m, m, device="cuda", generator=g)
    bb = torch.rand(m, m, device="cuda", generator=g)
    yy = torch.empty(m, m, device="cuda")
    gd = N.GemmDesc(m, m, m, 0, 0, 0, 1.0, 0.0, 1, 0, 0, 0, 0)
    for _ in range(reps):
        N.check(L.spinn_hip_gemm(C.byref(gd), P(a), P(bb), None, P(yy), None, 0, None), "gemm")
    torch.backends.cuda.matmul.allow_tf32 = False
    for _ in range(reps):
        torch.matmul(a, bb, out=yy)
    torch.cuda.synchronize()
    # hipBLASLt on the GEMM shapes of the conv layers (M = OC, N = batch*OH*OW, K = C*KH*KW)
    lib_us = {}
    for (m_, n_, k_) in [(1024, 6272, 256), (256, 6272, 1024), (64, 100352, 576), (256, 6272, 2304),
                         (512, 1568, 4608)]:
        a2 = torch.rand(m_, k_, device="cuda", generator=g)
        b2 = torch.rand(k_, n_, device="cuda", generator=g)
        y2 = torch.empty(m_, n_, device="cuda")
        for _ in range(3):
            torch.matmul(a2, b2, out=y2)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch.matmul(a2, b2, out=y2)
        e1.record()
        torch.cuda.synchronize()
        lib_us[f"{m_}x{n_}x{k_}"] = round(e0.elapsed_time(e1) / 20 * 1e3, 2)
    print(json.dumps({"gemm_compare": True, "torch_fp32_matmul_us": lib_us}), flush=True)


def executed_flops(r, algo: int) -> float:
    """MFMA FLOPs a layer actually executes: the direct count for the implicit GEMM
    and the direct kernels; for Winograd F(m x m, 3x3) the (m+2)^2 batched GEMMs of
    OC x C over T = N * ceil(OH/m) * ceil(OW/m) tiles (the transforms are not counted)."""
    from spinn_amd import native as N
    m = {N.ALGO_WINOGRAD: 2, N.ALGO_WINOGRAD_F43: 4}.get(algo)
    if m is None:
        return r["flops"]
    tiles = r["n"] * -(-r["oh"] // m) * -(-r["ow"] // m)
    return 2.0 * (m + 2) ** 2 * r["oc"] * r["c"] * tiles


CONV_FIELDS = ("n", "c", "h", "w", "oc", "oh", "ow", "kh", "kw", "sh", "sw", "ph", "pw", "group", "act")


def conv_layers_live(N, rows, algo_for, reps: int = 10) -> list:
    """Live kernel time of every distinct conv layer shape in `rows`: launched through
    spinn_hip_conv with the algorithm `algo_for(row)` names, `reps` times back to back
    inside a HIP graph replayed between two HIP events on the stream the kernels run
    on, so the figure carries no host launch gap or event between the launches, unlike
    the per-node event pass.
    One entry per shape: the row, its count, algorithm, ms per launch (all of the
    layer's kernels), direct and executed FLOPs and algorithmic bytes (input, weights,
    bias, output, residual; fp32, each once)."""
    import ctypes as C
    from spinn_amd.devbuf import DeviceBuffer, time_graph
    L = N.lib()
    if not rows:
        return []
    shapes = {}
    for r in rows:
        shapes.setdefault(tuple(r[f] for f in CONV_FIELDS), []).append(r)
    nbytes = lambda *dims: 4 * int(np.prod(dims))  # noqa: E731
    bufs = dict(x=max(nbytes(r["n"], r["c"], r["h"], r["w"]) for r in rows),
                y=max(nbytes(r["n"], r["oc"], r["oh"], r["ow"]) for r in rows),
                w=max(nbytes(r["oc"], r["c"] // r["group"], r["kh"], r["kw"]) for r in rows),
                b=max(nbytes(r["oc"]) for r in rows))
    bufs["r"] = bufs["y"]
    dev = {k: DeviceBuffer(v) for k, v in bufs.items()}
    scale = dict(x=1.0, y=1.0, w=0.05, b=0.1, r=1.0)
    for i, (k, b) in enumerate(dev.items()):
        fill_random(b, seed=11 + i, scale=scale[k])
    out = []
    try:
        for key, rs in shapes.items():
            r = rs[0]
            algo = algo_for(r)
            d = N.ConvDesc(*key, algo, 0)
            psz = L.spinn_hip_conv_packed_size(C.byref(d))
            pk = DeviceBuffer(psz) if psz else None
            wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
            ksplit = ""
            if wsz and algo == N.ALGO_IMPLICIT_GEMM:
                # a workspace without the stream-K split means split-K partials
                L.spinn_hip_tune_streamk(0)
                ksplit = "split-K" if L.spinn_hip_conv_workspace_size(C.byref(d)) else "stream-K"
                L.spinn_hip_tune_streamk(-1)
            ws = DeviceBuffer(wsz) if wsz else None
            if pk:
                N.check(L.spinn_hip_conv_pack_weights(C.byref(d), dev["w"].ptr, pk.ptr, None), "pack")
            has_res = r["act"] in (4, 5)
            res = dev["r"].ptr if has_res else None
            launch = lambda st: L.spinn_hip_conv(C.byref(d), dev["x"].ptr, dev["w"].ptr,  # noqa: E731
                                                 pk.ptr if pk else None, dev["b"].ptr, res, dev["y"].ptr,
                                                 ws.ptr if ws else None, wsz, st)
            # the better of two graph-timed runs: the first can catch the clock still ramping
            # up after the host-side set-up
            ms = min(time_graph(launch, reps), time_graph(launch, reps))
            byts = (nbytes(r["n"], r["c"], r["h"], r["w"]) + nbytes(r["oc"], r["c"] // r["group"], r["kh"], r["kw"])
                    + nbytes(r["oc"]) + nbytes(r["n"], r["oc"], r["oh"], r["ow"]) * (2 if has_res else 1))
            out.append(dict(row=r, count=len(rs), algo=algo, ms=ms, flops=r["flops"],
                            exec_flops=executed_flops(r, algo), bytes=byts, split=ksplit))
            for buf in (pk, ws):
                if buf:
                    buf.free()
    finally:
        for b in dev.values():
            b.free()
    return out


def conv_kernels_live(N, rows, algo: int, reps: int = 10):
    """(kernel ms summed over the layers, direct-conv FLOPs, algorithmic bytes, number of
    layers) of `rows` run with one algorithm, from conv_layers_live."""
    res = conv_layers_live(N, rows, lambda r: algo, reps)
    return (sum(e["ms"] * e["count"] for e in res), sum(e["flops"] * e["count"] for e in res),
            sum(e["bytes"] * e["count"] for e in res), sum(e["count"] for e in res))


def layers_markdown(live: list, batch: int, policy: str) -> str:
    """Per-layer table of one conv pass (one row per distinct layer shape)."""
    lines = [f"# ResNet-101 v1.5 fp32 conv layers, batch {batch}, policy {policy}", "",
             "Each distinct layer shape launched 10x back to back through `spinn_hip_conv` inside a HIP graph "
             "replayed between HIP events "
             "(`bench.py`, conv_layers_live). GFLOP = direct-convolution count 2*N*OC*OH*OW*C*KH*KW; "
             "exec GFLOP = MFMA work actually issued (Winograd F(4x4,3x3): 36 GEMMs over 4x4 output tiles, "
             "transforms not counted). K split: split-K (partials reduced by a second launch) or stream-K "
             "(whole tiles plus the remaining tiles cut along K, finished in the same launch). "
             "% peak against 157.3 TFLOP/s fp32 MFMA. Operands are random (uniform), never zero-filled. "
             "MB = algorithmic bytes (input, weights, bias, output, residual, each once); bound = the longer of "
             "the direct FLOPs at MFMA peak and MB at 8 TB/s (executed FLOPs for Winograd), and % bound = that "
             "time over the measured one.", "",
             "| layer (C,H,W -> OC, k/s, act) | x | algo | K split | GFLOP | exec GFLOP | MB | us / launch | "
             "TFLOP/s direct | % peak direct | % peak executed | bound | % bound |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    tf = te = tt = 0.0
    for e in live:
        r = e["row"]
        t = e["ms"] * 1e-3
        lines.append(f"| {r['c']},{r['h']},{r['w']} -> {r['oc']}, {r['kh']}x{r['kw']}/s{r['sh']}, {r['act']} | "
                     f"{e['count']} | {ALGO_NAMES.get(e['algo'], e['algo'])} | {e['split']} | "
                     f"{e['flops'] / 1e9:.2f} | {e['exec_flops'] / 1e9:.2f} | {e['bytes'] / 1e6:.1f} | "
                     f"{e['ms'] * 1e3:.1f} | "
                     f"{e['flops'] / t / 1e12:.1f} | {100 * e['flops'] / t / PEAK_FP32_MFMA:.1f} | "
                     f"{100 * e['exec_flops'] / t / PEAK_FP32_MFMA:.1f} | "
                     f"{'hbm' if e['bytes'] / 8e12 > e['exec_flops'] / PEAK_FP32_MFMA else 'mfma'} | "
                     f"{100 * max(e['bytes'] / 8e12, e['exec_flops'] / PEAK_FP32_MFMA) / t:.1f} |")
        tf += e["flops"] * e["count"]
        te += e["exec_flops"] * e["count"]
        tt += e["ms"] * 1e-3 * e["count"]
    lines += ["", f"All {sum(e['count'] for e in live)} conv layers: {tt * 1e3:.3f} ms of kernel time, "
                  f"{tf / 1e9:.1f} GFLOP direct ({tf / tt / 1e12:.1f} TFLOP/s, "
                  f"{100 * tf / tt / PEAK_FP32_MFMA:.1f} % of peak), {te / 1e9:.1f} GFLOP executed "
                  f"({te / tt / 1e12:.1f} TFLOP/s, {100 * te / tt / PEAK_FP32_MFMA:.1f} % of peak)."]
    return "\n".join(lines) + "\n"


def igemm_algorithmic_bytes(batch: int, policy: str) -> float:
    """Mean algorithmic bytes per implicit-GEMM conv launch of ResNet-101 at
    `batch`: input + weights + bias + output (+ residual for the fused add),
    each read or written once, fp32."""
    from spinn_amd import models
    from spinn_amd import native as N
    pol = {"auto": N.POLICY_AUTO, "igemm": N.POLICY_IGEMM, "winograd": N.POLICY_WINOGRAD}[policy]
    g, _ = models.resnet101(batch=batch, seed=0)
    alg = []
    for r in conv_table(g):
        if algo_of(N, r, pol) != N.ALGO_IMPLICIT_GEMM:
            continue
        x = r["n"] * r["c"] * r["h"] * r["w"]
        w = r["oc"] * (r["c"] // r["group"]) * r["kh"] * r["kw"]
        y = r["n"] * r["oc"] * r["oh"] * r["ow"]
        res = y if r["act"] in (4, 5) else 0
        alg.append(4.0 * (x + w + r["oc"] + y + res))
    return sum(alg) / len(alg)


def traffic_summary(d: Path, batch: int, policy: str, commands: list) -> dict:
    """Reduce the four rocprofv3 --pmc counter CSVs under `d` (calib_{FETCH,WRITE}_SIZE
    from the calibration kernels, r101_{FETCH,WRITE}_SIZE from --profile-pass) to
    calibrated HBM-side bytes per implicit-GEMM conv dispatch (conv_igemm_kernel, its
    data-parallel + stream-K form conv_igemm_sk_kernel and the 7x7 stem's stem7_mfma_kernel;
    split-K reductions not counted)."""
    import csv

    def rows(name):
        with open(d / f"{name}_counter_collection.csv") as f:
            return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in csv.DictReader(f)]

    kib = CALIB_BYTES / 1024

    def calib(counter, kind):
        v = [x for n, x in rows(f"calib_{counter}") if kind in n.lower()]
        v = v[1:] if len(v) > 1 else v  # first launch of each warms the caches
        return sum(v) / len(v)

    f_fetch = kib / calib("FETCH_SIZE", "copy")
    f_write = kib / calib("WRITE_SIZE", "fill")
    per = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        v = [x for n, x in rows(f"r101_{counter}")
             if "conv_igemm_kernel" in n or "conv_igemm_sk_kernel" in n or "stem7_mfma_kernel" in n]
        per[counter] = (len(v), sum(v) / len(v))
    fetch_b = per["FETCH_SIZE"][1] * 1024 * f_fetch
    write_b = per["WRITE_SIZE"][1] * 1024 * f_write
    return {
        "kernel": f"conv_igemm_kernel / conv_igemm_sk_kernel / stem7_mfma_kernel (all instantiations), implicit-GEMM layers of "
                  f"ResNet-101 v1.5 fp32 "
                  f"batch {batch}",
        "conv_policy": policy, "batch": batch, "commands": commands,
        "calibration": {"method": "256 MiB fills (spinn_hip_fill_u32) and 256 MiB device copies (spinn_hip_copy) "
                                  "under the same counters (bench.py --calibration-kernels); factor = true KiB / "
                                  "counter KiB, first launch of each dropped",
                        "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4)},
        "dispatches": per["FETCH_SIZE"][0],
        "fetch_kib_per_dispatch_raw": round(per["FETCH_SIZE"][1], 1),
        "write_kib_per_dispatch_raw": round(per["WRITE_SIZE"][1], 1),
        "fetch_bytes_per_launch": round(fetch_b), "write_bytes_per_launch": round(write_b),
        "traffic_bytes_per_launch": round(fetch_b + write_b),
        "algorithmic_bytes_per_launch": round(igemm_algorithmic_bytes(batch, policy)),
        "note": "FETCH_SIZE / WRITE_SIZE count traffic between the L2s and the memory fabric, so hits in the "
                "Infinity Cache (MALL) count as HBM traffic here",
    }


def measured_traffic(batch: int, policy: str):
    """Calibrated HBM-side bytes per implicit-GEMM launch from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes, when they match this workload."""
    if not TRAFFIC_FILE.exists():
        return None
    d = json.loads(TRAFFIC_FILE.read_text())
    if d.get("batch") != batch or d.get("conv_policy") != policy:
        return None
    return d.get("traffic_bytes_per_launch")


def _kernel_label(name: str) -> str:
    """A rocprofv3 kernel name without its argument list and namespaces."""
    import re
    n = name.replace("(anonymous namespace)::", "").replace("spinn::", "")
    n = re.sub(r"\((?:[A-Za-z_:]*Args|[^()]*)\)$", "", n)
    return n.replace("void ", "").strip()


def trace_summary(path: Path, passes: int) -> str:
    """Markdown tables (kernel family, then instantiation + grid) from a rocprofv3
    --kernel-trace CSV; `passes` divides totals into per-pass figures."""
    import collections
    import csv
    with open(path) as f:
        rows = list(csv.DictReader(f))
    inst = collections.defaultdict(list)
    for r in rows:
        grid = tuple(int(r.get(f"Grid_Size_{a}", 1) or 1) for a in "XYZ")
        wg = tuple(int(r.get(f"Workgroup_Size_{a}", 1) or 1) for a in "XYZ")
        groups = tuple(g // w for g, w in zip(grid, wg))
        inst[(_kernel_label(r["Kernel_Name"]), groups, wg[0] * wg[1] * wg[2])].append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    fam = collections.defaultdict(lambda: [0, 0.0])
    for (name, _, _), v in inst.items():
        f_ = fam[name.split("<")[0]]
        f_[0] += len(v)
        f_[1] += sum(v)
    total = sum(t for _, t in fam.values())
    out = [f"| kernel family | calls | total us / pass | avg us | % |", "|---|---|---|---|---|"]
    for name, (n, t) in sorted(fam.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| {name} | {n} | {t / passes:.1f} | {t / n:.2f} | {100 * t / total:.1f} |")
    out += ["", "| instantiation | workgroups (x,y,z) | threads | calls | avg us | min us | total us / pass |",
            "|---|---|---|---|---|---|---|"]
    for (name, groups, thr), v in sorted(inst.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| `{name}` | {groups} | {thr} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | "
                   f"{sum(v) / passes:.1f} |")
    return "\n".join(out)


def roofline_trace_summary(trace: Path, pass_json: Path) -> str:
    """Markdown comparison of a rocprofv3 --kernel-trace CSV of `bench.py --roofline-pass`
    with the per-shape times that run printed (its JSON line in `pass_json`): per layer
    shape, the mean kernel time per spinn_hip_conv call over every call the trace holds
    (the warm-up call, the unmeasured first replay and both timed runs: 122 calls; a
    split-K call's reduction launch included) beside the pass's own figure (the better
    of its two timed runs), then the count-weighted mean per launch, which is what the
    bench line's `launch_us` is. A shape's calls lie between its weight packing
    (`conv_pack_*`) and the next shape's."""
    import csv
    line = json.loads(pass_json.read_text().strip().splitlines()[-1])
    with open(trace) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    segs, cur, in_pack = [], None, False
    for r in rows:
        name = _kernel_label(r["Kernel_Name"])
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if name.startswith("conv_pack_"):
            if not in_pack:
                cur = {"main": None, "calls": 0, "us": 0.0}
                segs.append(cur)
            in_pack = True
            continue
        in_pack = False
        if cur is None or not name.startswith(("conv_igemm", "conv_splitk_reduce", "stem7_mfma")):
            continue
        base = name.split("<")[0]
        if cur["main"] is None:
            cur["main"] = base
        if base == cur["main"]:
            cur["calls"] += 1
        cur["us"] += us
    shapes = line["shapes"]
    if len(segs) != len(shapes):
        raise SystemExit(f"{len(segs)} packed segments in the trace against {len(shapes)} shapes in the pass")
    out = ["| layer (C,H,W -> OC, k/s, act) | x | kernel | calls traced | rocprof us / call | bench.py us / launch | diff |",
           "|---|---|---|---|---|---|---|"]
    wt = wb = n = 0.0
    for sh, sg in zip(shapes, segs):
        t = sg["us"] / max(sg["calls"], 1)
        out.append(f"| {sh['layer']} | {sh['count']} | {sg['main']} | {sg['calls']} | {t:.2f} | {sh['us']:.2f} | "
                   f"{100 * (t - sh['us']) / sh['us']:+.1f} % |")
        wt += t * sh["count"]
        wb += sh["us"] * sh["count"]
        n += sh["count"]
    out += ["", f"Count-weighted mean per launch over {int(n)} layers: rocprof {wt / n:.2f} us, bench.py "
                f"{wb / n:.2f} us (`launch_us` {line['launch_us']}), {100 * (wt - wb) / wb:+.1f} %; "
                f"{line['gflop_per_launch']:.3f} GFLOP per launch -> rocprof {line['gflop_per_launch'] / (wt / n) * 1e3:.1f} "
                f"TFLOP/s, bench.py {line['achieved']} TFLOP/s."]
    return "\n".join(out)


def pmc_summary(d: Path) -> str:
    """Per-dispatch averages of the rocprofv3 --pmc counter CSVs under `d`
    (every *_counter_collection.csv), for the spinn kernels, plus derived ratios."""
    import collections
    import csv
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    for p in sorted(d.glob("*_counter_collection.csv")):
        per = collections.defaultdict(dict)
        with open(p) as f:
            for r in csv.DictReader(f):
                if "spinn::" not in r["Kernel_Name"]:
                    continue
                key = (_kernel_label(r["Kernel_Name"]), int(r["Grid_Size"]), int(r["Workgroup_Size"]))
                per[(key, r["Dispatch_Id"])][r["Counter_Name"]] = float(r["Counter_Value"])
        for (key, _), cs in per.items():
            for c, v in cs.items():
                vals[key][c].append(v)
    out = []
    for (name, grid, wg), cs in vals.items():
        if "SQ_WAVES" not in cs or "conv_pack" in name:
            continue
        a = {c: sum(v) / len(v) for c, v in cs.items()}
        waves = a["SQ_WAVES"]
        out.append(f"### `{name}`, {grid // wg} workgroups of {wg} threads")
        out.append("")
        out.append("| counter | per dispatch | per wave |")
        out.append("|---|---|---|")
        for c in sorted(a):
            if c == "GRBM_GUI_ACTIVE":
                continue
            out.append(f"| {c} | {a[c]:.0f} | {a[c] / waves:.1f} |")
        mf = a.get("SQ_INSTS_MFMA")
        if mf:
            out.append("")
            ratios = []
            if "SQ_INSTS_VALU" in a:
                ratios.append(f"VALU instructions other than MFMA per MFMA: {(a['SQ_INSTS_VALU'] - mf) / mf:.2f}")
            if "SQ_INSTS_LDS" in a:
                ratios.append(f"LDS instructions per MFMA: {a['SQ_INSTS_LDS'] / mf:.2f}")
            if "SQ_INSTS_VMEM_RD" in a:
                ratios.append(f"vector-memory reads per MFMA: {a['SQ_INSTS_VMEM_RD'] / mf:.2f}")
            if "SQ_INSTS_SALU" in a:
                ratios.append(f"scalar ALU instructions per MFMA: {a['SQ_INSTS_SALU'] / mf:.2f}")
            if "SQ_WAIT_INST_ANY" in a and "SQ_WAVE_CYCLES" in a:
                ratios.append(f"SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES: {a['SQ_WAIT_INST_ANY'] / a['SQ_WAVE_CYCLES']:.2f}")
            if "SQ_WAIT_INST_LDS" in a and "SQ_WAVE_CYCLES" in a:
                ratios.append(f"SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES: {a['SQ_WAIT_INST_LDS'] / a['SQ_WAVE_CYCLES']:.3f}")
            out += [f"- {x}" for x in ratios]
        out.append("")
    return "\n".join(out)


FAMILY_COUNTERS = ("SQ_WAVES", "SQ_BUSY_CU_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU",
                   "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_LDS_BANK_CONFLICT")


def family_counters_summary(d: Path, tags: list) -> str:
    """Per kernel family of each workload tag: rocprofv3 runs `{tag}_sq` (--pmc with the
    FAMILY_COUNTERS), `{tag}_FETCH_SIZE` and `{tag}_WRITE_SIZE` (each with --kernel-trace),
    plus `calib_FETCH_SIZE` / `calib_WRITE_SIZE` (bench.py --calibration-kernels) for the
    byte scale. Reports, per dispatch: mean duration, executed MFMA rate (busy cycles x 64
    fp32 flops per cycle and SIMD: v_mfma_f32_32x32x2f32 is 4096 flops in 64 cycles,
    16x16x4f32 2048 in 32) against the 157.3 TFLOP/s peak, non-MFMA VALU / LDS / vector-memory
    instructions per MFMA, LDS bank conflicts, and calibrated fetched / written MB and their
    rate (L2-to-fabric traffic: Infinity Cache hits count as memory traffic)."""
    import collections
    import csv

    def load(name):
        p = d / f"{name}_counter_collection.csv"
        if not p.exists():
            return None
        per = collections.defaultdict(dict)
        with open(p) as f:
            for r in csv.DictReader(f):
                if "spinn::" not in r["Kernel_Name"] and "rocclr" not in r["Kernel_Name"]:
                    continue
                e = per[r["Dispatch_Id"]]
                e["name"] = _kernel_label(r["Kernel_Name"]).split("<")[0]
                e["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                e[r["Counter_Name"]] = float(r["Counter_Value"])
        return per

    def calib(counter, kind):
        per = load(f"calib_{counter}")
        v = [e[counter] for _, e in sorted(per.items(), key=lambda kv: int(kv[0])) if kind in e["name"].lower()]
        v = v[1:] if len(v) > 1 else v
        return (CALIB_BYTES / 1024) / (sum(v) / len(v))

    f_fetch, f_write = calib("FETCH_SIZE", "copy"), calib("WRITE_SIZE", "fill")
    out = [f"Byte scale from the 256 MiB copy / fill calibration: FETCH_SIZE x {f_fetch:.3f}, "
           f"WRITE_SIZE x {f_write:.3f}.", ""]
    for tag in tags:
        fam = collections.defaultdict(lambda: collections.defaultdict(list))
        for part in ("sq", "FETCH_SIZE", "WRITE_SIZE"):
            per = load(f"{tag}_{part}")
            if per is None:
                continue
            for e in per.values():
                for k, v in e.items():
                    if k != "name":
                        fam[e["name"]][f"{part}:{k}"].append(v)
        out += [f"### {tag}", "",
                "| kernel family | dispatches | mean us | MFMA TFLOP/s executed | % of MFMA peak | VALU / MFMA | "
                "LDS / MFMA | VMEM rd / MFMA | LDS bank conflicts / dispatch | fetched MB | written MB | GB/s |",
                "|---|---|---|---|---|---|---|---|---|---|---|---|"]
        rows = []
        for name, cs in fam.items():
            m = lambda k: (sum(cs[k]) / len(cs[k])) if cs.get(k) else None  # noqa: E731
            us = m("sq:us") or m("FETCH_SIZE:us")
            if not us:
                continue
            busy, mf = m("sq:SQ_VALU_MFMA_BUSY_CYCLES"), m("sq:SQ_INSTS_MFMA")
            tf = busy * 64 / (us * 1e-6) / 1e12 if busy else 0.0
            fmb = m("FETCH_SIZE:FETCH_SIZE")
            wmb = m("WRITE_SIZE:WRITE_SIZE")
            fmb = fmb * 1024 * f_fetch / 1e6 if fmb is not None else None
            wmb = wmb * 1024 * f_write / 1e6 if wmb is not None else None
            rate = (fmb + wmb) / us * 1e3 if fmb is not None and wmb is not None else None
            per_mf = lambda k: f"{(m(k) - (mf if k.endswith('VALU') else 0)) / mf:.2f}" if mf and m(k) is not None else "-"  # noqa: E731,E501
            rows.append((us * len(cs.get("sq:us", cs.get("FETCH_SIZE:us", []))),
                         f"| {name} | {len(cs.get('sq:us', []))} | {us:.2f} | {tf:.1f} | {100 * tf / 157.3:.1f} | "
                         f"{per_mf('sq:SQ_INSTS_VALU')} | {per_mf('sq:SQ_INSTS_LDS')} | {per_mf('sq:SQ_INSTS_VMEM_RD')} | "
                         f"{(m('sq:SQ_LDS_BANK_CONFLICT') or 0):.0f} | "
                         f"{'-' if fmb is None else f'{fmb:.2f}'} | {'-' if wmb is None else f'{wmb:.2f}'} | "
                         f"{'-' if rate is None else f'{rate:.0f}'} |"))
        out += [r for _, r in sorted(rows, key=lambda x: -x[0])] + [""]
    return "\n".join(out)


ENGINE_SCAN_SHAPES = [(1024, 14), (256, 14), (256, 56)]  # (output channels, plane edge) at batch 32
ENGINE_SCAN_K = [64, 128, 256, 512, 1024, 2048]


def engine_scan(reps: int = 10) -> None:
    """Graph-timed 1x1 convs at batch 32 over input depths K (64x64 tiles, no K split):
    time(K) = fixed + slope*K separates a launch's fixed cost (prologue, epilogue
    stores, ramp) from the K loop's steady MFMA rate. One JSON line per shape."""
    import ctypes as C
    from spinn_amd import native as N
    from spinn_amd.devbuf import DeviceBuffer, time_graph
    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")
    for (oc, hw) in ENGINE_SCAN_SHAPES:
        res = []
        for c in ENGINE_SCAN_K:
            n = 32
            d = N.ConvDesc(n, c, hw, hw, oc, hw, hw, 1, 1, 1, 1, 0, 0, 1, 1, N.ALGO_IMPLICIT_GEMM, 0)
            bufs = [DeviceBuffer(4 * v) for v in (n * c * hw * hw, oc * c, oc, n * oc * hw * hw)]
            for i, b_ in enumerate(bufs):
                fill_random(b_, seed=41 + i, scale=0.05 if i == 1 else 1.0)
            bx, bw, bb, by = bufs
            bp = DeviceBuffer(L.spinn_hip_conv_packed_size(C.byref(d)))
            N.check(L.spinn_hip_conv_pack_weights(C.byref(d), bw.ptr, bp.ptr, None), "pack")
            L.spinn_hip_tune_force_tiles(64, 64, 0)
            try:
                ms = time_graph(lambda st: L.spinn_hip_conv(C.byref(d), bx.ptr, bw.ptr, bp.ptr, bb.ptr, None, by.ptr,
                                                            None, 0, st), reps)
            finally:
                L.spinn_hip_tune_force_tiles(0, 0, 0)
            fl = 2.0 * n * oc * hw * hw * c
            res.append({"K": c, "us": round(ms * 1e3, 2), "tflops": round(fl / ms / 1e9, 1)})
            for b_ in bufs + [bp]:
                b_.free()
        ks = [r["K"] for r in res[-3:]]
        ts = [r["us"] for r in res[-3:]]
        slope = (ts[-1] - ts[0]) / (ks[-1] - ks[0])
        fixed = ts[0] - slope * ks[0]
        steady = 2.0 * 32 * oc * hw * hw / (slope * 1e-6) / 1e12
        print(json.dumps({"engine_scan": f"1x1 conv, batch 32, {oc} output channels, {hw}x{hw}",
                          "tiles_64x64": ((oc + 63) // 64) * ((32 * hw * hw + 63) // 64), "points": res,
                          "fit_over_last_three": {"fixed_us": round(fixed, 2), "us_per_k": round(slope, 4),
                                                  "steady_tflops": round(steady, 1)}}), flush=True)
    # tile edge: the two 14x14 ResNet-101 layer shapes and an 8192^3 Gemm, 64x64 vs 128x128 tiles
    for (c, oc) in ((256, 1024), (1024, 256)):
        n, hw = 32, 14
        d = N.ConvDesc(n, c, hw, hw, oc, hw, hw, 1, 1, 1, 1, 0, 0, 1, 1, N.ALGO_IMPLICIT_GEMM, 0)
        bufs = [DeviceBuffer(4 * v) for v in (n * c * hw * hw, oc * c, oc, n * oc * hw * hw)]
        for i, b_ in enumerate(bufs):
            fill_random(b_, seed=51 + i, scale=0.05 if i == 1 else 1.0)
        bx, bw, bb, by = bufs
        bp = DeviceBuffer(L.spinn_hip_conv_packed_size(C.byref(d)))
        N.check(L.spinn_hip_conv_pack_weights(C.byref(d), bw.ptr, bp.ptr, None), "pack")
        out = {}
        for t in (64, 128):
            L.spinn_hip_tune_force_tiles(t, t, 0)
            try:
                ms = time_graph(lambda st: L.spinn_hip_conv(C.byref(d), bx.ptr, bw.ptr, bp.ptr, bb.ptr, None, by.ptr,
                                                            None, 0, st), reps)
            finally:
                L.spinn_hip_tune_force_tiles(0, 0, 0)
            out[f"{t}x{t}"] = {"us": round(ms * 1e3, 2), "tflops": round(2.0 * n * oc * hw * hw * c / ms / 1e9, 1)}
        print(json.dumps({"engine_scan": f"tile edge, 1x1 conv batch 32 {c}->{oc} at 14x14", **out}), flush=True)
        for b_ in bufs + [bp]:
            b_.free()
    m = 8192
    ba, bb2, by2 = DeviceBuffer(4 * m * m), DeviceBuffer(4 * m * m), DeviceBuffer(4 * m * m)
    for i, b_ in enumerate((ba, bb2)):
        fill_random(b_, seed=61 + i)
    gd = N.GemmDesc(m, m, m, 0, 0, 0, 1.0, 0.0, 1, 0, 0, 0, 0)
    out = {}
    for t in (64, 128):
        L.spinn_hip_tune_force_tiles(t, t, 0)
        try:
            ms = time_graph(lambda st: L.spinn_hip_gemm(C.byref(gd), ba.ptr, bb2.ptr, None, by2.ptr, None, 0, st), 2,
                            replays=2)
        finally:
            L.spinn_hip_tune_force_tiles(0, 0, 0)
        out[f"{t}x{t}"] = {"us": round(ms * 1e3, 1), "tflops": round(2.0 * m ** 3 / ms / 1e9, 1)}
    print(json.dumps({"engine_scan": "tile edge, Gemm 8192^3", **out}), flush=True)
    for b_ in (ba, bb2, by2):
        b_.free()


class StepMismatch(RuntimeError):
    pass


def time_steps(sess, steps: int, warmup: int, ref: np.ndarray | None = None) -> float:
    """Mean wall time of one resident step (ms). Every step restores input 0 into its
    arena region from the staged device copy (spinn_run_resident) and runs the node
    loop. The output of the first step (and `ref`, the host-copy path's output for
    the same input, when given) must equal the output after the timed steps bit for
    bit, so every timed step computed the stated input."""
    sess.run_resident()
    first = sess.download(sess.output_id)
    if ref is not None and not np.array_equal(first.view(np.uint32), np.asarray(ref).view(np.uint32)):
        raise StepMismatch("resident step output differs from spinn_run with host copies")
    for _ in range(warmup):
        sess.run_resident()
    t0 = time.perf_counter()
    for _ in range(steps):
        sess.run_resident()  # returns after the runtime's stream is idle
    ms = (time.perf_counter() - t0) / steps * 1e3
    last = sess.download(sess.output_id)
    if not np.array_equal(first.view(np.uint32), last.view(np.uint32)):
        raise StepMismatch("output after the timed steps differs from the first step's")
    return ms


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--policy", choices=["auto", "igemm", "winograd"], default="auto")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="launch nodes one by one (for profilers)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="only the per-node-event pass at batch B (warmup + steps, eager launches): the run a "
                         "kernel profiler wraps, so its kernel statistics cover exactly the measured launches")
    ap.add_argument("--profile-model", choices=["resnet101", "yolov10n"], default="resnet101",
                    help="model of --profile-pass (yolov10n: the 640x640 detector with its TopK tail)")
    ap.add_argument("--layers-out", default=str(ROOT / "gpurun_out" / "bench_layers.json"))
    ap.add_argument("--no-suite", action="store_true", help="skip the config-0 / Gemm sweep / VGG measurements")
    ap.add_argument("--gemm-compare", action="store_true",
                    help="only the launches of the MFMA-engine PMC comparison (three ResNet-101 conv layers, an "
                         "8192^3 Gemm here and through torch/hipBLASLt)")
    ap.add_argument("--small-launches", action="store_true",
                    help="only launch the config-0 conv, the Gemm sweep and the YOLOv10n b16 depthwise layers "
                         "20x each (for rocprofv3 --kernel-trace --stats)")
    ap.add_argument("--clock-probe", action="store_true",
                    help="one conv launched 200x on zero then on random operands (run under rocprofv3 --pmc "
                         "GRBM_GUI_ACTIVE GRBM_COUNT --kernel-trace)")
    ap.add_argument("--clock-summary", metavar="DIR", help="table of a --clock-probe run's counters (no GPU)")
    ap.add_argument("--calibration-kernels", action="store_true",
                    help="only run the known-size fill/copy kernels that scale the HBM byte counters")
    ap.add_argument("--traffic-summary", metavar="DIR",
                    help="reduce rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE CSVs in DIR to the traffic file (no GPU)")
    ap.add_argument("--roofline-pass", action="store_true",
                    help="only the live implicit-GEMM launches behind `roofline` at batch B (what a kernel "
                         "profiler wraps to check its average launch duration), printed as one JSON line")
    ap.add_argument("--roofline-trace", metavar="CSV",
                    help="compare a rocprofv3 kernel trace of --roofline-pass with that run's JSON line "
                         "(--roofline-json; no GPU)")
    ap.add_argument("--roofline-json", metavar="FILE", help="the --roofline-pass output, for --roofline-trace")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="print markdown tables of a rocprofv3 kernel-trace CSV (no GPU)")
    ap.add_argument("--passes", type=int, default=1, help="passes in the traced run, for --trace-summary")
    ap.add_argument("--pmc-summary", metavar="DIR",
                    help="print per-dispatch averages of the rocprofv3 --pmc CSVs in DIR (no GPU)")
    ap.add_argument("--family-counters", metavar="DIR",
                    help="per-kernel-family counter table of the rocprofv3 runs in DIR (no GPU; see "
                         "family_counters_summary)")
    ap.add_argument("--tags", default="r101b32,r101b1,y10b16", help="workload tags for --family-counters")
    ap.add_argument("--engine-scan", action="store_true",
                    help="time 1x1 convs at batch 32 over K to split fixed cost from the K loop's rate")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: measures one GPU; --gpus {a.gpus} is not supported (the conv path would "
              "shard by batch, each GPU running the whole model on its images with no collective)",
              file=sys.stderr)
        return 2
    if a.clock_summary:
        print(clock_summary(Path(a.clock_summary)), end="")
        return 0
    if a.clock_probe:
        clock_probe()
        return 0
    if a.calibration_kernels:
        calibration_kernels()
        return 0
    if a.small_launches:
        small_launches()
        return 0
    if a.gemm_compare:
        gemm_compare()
        return 0
    if a.trace_summary:
        print(trace_summary(Path(a.trace_summary), a.passes))
        return 0
    if a.roofline_trace:
        print(roofline_trace_summary(Path(a.roofline_trace), Path(a.roofline_json)))
        return 0
    if a.pmc_summary:
        print(pmc_summary(Path(a.pmc_summary)))
        return 0
    if a.family_counters:
        print(family_counters_summary(Path(a.family_counters), a.tags.split(",")))
        return 0
    if a.engine_scan:
        engine_scan()
        return 0
    if a.traffic_summary:
        cmds = [f"rocprofv3 --pmc {c} --output-format csv -d {a.traffic_summary} -o {o}_{c} -- python -u bench.py {f}"
                for c in ("FETCH_SIZE", "WRITE_SIZE")
                for o, f in (("calib", "--calibration-kernels"),
                             ("r101", f"--profile-pass --steps 2 --warmup 1 --no-cpu --batch {a.batch}"))]
        s = traffic_summary(Path(a.traffic_summary), a.batch, a.policy, cmds)
        TRAFFIC_FILE.write_text(json.dumps(s, indent=1) + "\n")
        print(json.dumps(s))
        return 0

    from spinn_amd import models
    from spinn_amd import native as N
    from spinn_amd.runtime import Session

    policy = {"auto": N.POLICY_AUTO, "igemm": N.POLICY_IGEMM, "winograd": N.POLICY_WINOGRAD}[a.policy]
    tmp = Path(tempfile.mkdtemp(prefix="spinn_bench_"))
    t_gen = time.perf_counter()
    g1, x1 = models.resnet101(batch=1, seed=0)
    p1 = g1.write(tmp / "r101_b1.ennf")
    gB, xB = models.resnet101(batch=a.batch, seed=0)
    pB = gB.write(tmp / f"r101_b{a.batch}.ennf")
    print(f"[bench] models written in {time.perf_counter() - t_gen:.1f}s", file=sys.stderr, flush=True)

    # CPU baselines first, before this process touches the GPU.
    cpu = cpu_y10 = None
    if not a.no_cpu:
        cpu = cpu_baseline(p1, g1.dims(g1.inputs[0]), g1.dims(g1.outputs[0]), a.cpu_seconds)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
        if not a.no_suite:
            gy, _ = models.yolov10n(batch=1, seed=0, postprocess=True)
            py = gy.write(tmp / "y10_cpu_b1.ennf")
            cpu_y10 = cpu_baseline(py, gy.dims(gy.inputs[0]), gy.dims(gy.outputs[0]), a.cpu_seconds / 2,
                                   label="YOLOv10n 640x640")
            print(f"[bench] yolov10n cpu baseline: {cpu_y10}", file=sys.stderr, flush=True)

    L = N.lib()
    N.check(L.spinn_hip_init(0), "spinn_hip_init")

    if a.roofline_pass:
        rows = [r for r in conv_table(gB) if algo_of(N, r, policy) == N.ALGO_IMPLICIT_GEMM]
        live = conv_layers_live(N, rows, lambda r: algo_of(N, r, policy))
        ms = sum(e["ms"] * e["count"] for e in live)
        fl = sum(e["flops"] * e["count"] for e in live)
        n = sum(e["count"] for e in live)
        tf = fl / (ms * 1e-3) / 1e12
        lab = lambda r: f"{r['c']},{r['h']},{r['w']} -> {r['oc']}, {r['kh']}x{r['kw']}/s{r['sh']}, {r['act']}"  # noqa: E731
        print(json.dumps({"roofline_pass": True, "batch": a.batch, "layers": n, "launch_us": round(ms / n * 1e3, 2),
                          "gflop_per_launch": fl / n / 1e9, "achieved": round(tf, 3),
                          "frac": round(tf * 1e12 / PEAK_FP32_MFMA, 4),
                          "shapes": [{"layer": lab(e["row"]), "count": e["count"], "us": round(e["ms"] * 1e3, 3),
                                      "split": e["split"]} for e in live]}))
        return 0
    if a.profile_pass and a.profile_model == "yolov10n":
        gy, xy = models.yolov10n(batch=a.batch, seed=0, postprocess=True)
        py = gy.write(tmp / f"y10_b{a.batch}.ennf")
        node_ms = profiled_node_ms(N, Session, py, xy, policy, a.steps, a.warmup)
        fam = {}
        for i, nd in enumerate(gy.nodes):
            f = fam.setdefault(_op_family(N, nd, gy, policy), [0, 0.0])
            f[0] += 1
            f[1] += float(node_ms[i])
        print(json.dumps({"profile_pass": True, "model": "yolov10n+tail", "batch": a.batch, "steps": a.steps,
                          "warmup": a.warmup, "node_ms_total": float(node_ms.sum()),
                          "families_ms": {k: {"nodes": v[0], "ms": round(v[1], 4)} for k, v in
                                          sorted(fam.items(), key=lambda kv: -kv[1][1])}}))
        return 0
    if a.profile_pass:
        node_ms = profiled_node_ms(N, Session, pB, xB, policy, a.steps, a.warmup)
        rows = conv_table(gB)
        fam = {}
        for r in rows:
            algo = ALGO_NAMES.get(algo_of(N, r, policy), "?")
            f = fam.setdefault(algo, [0, 0.0, 0.0])
            f[0] += 1
            f[1] += r["flops"]
            f[2] += float(node_ms[r["node"]])
        print(json.dumps({"profile_pass": True, "batch": a.batch, "steps": a.steps, "warmup": a.warmup,
                          "node_ms_total": float(node_ms.sum()),
                          "families": {k: {"layers": v[0], "gflop": v[1] / 1e9, "ms": v[2],
                                           "tflops": v[1] / (v[2] * 1e-3) / 1e12} for k, v in fam.items()}}))
        return 0

    # ---- batch B, graph replay, input resident ----
    sB = Session(pB, policy=policy, graph=not a.no_graph)
    yB_host = sB.run(xB)  # host in, host out: the reference's spinn_run protocol
    sB.upload_input(xB)
    ms_B = time_steps(sB, a.steps, a.warmup, ref=yB_host)
    print(f"[bench] b{a.batch}: {ms_B:.3f} ms/step", file=sys.stderr, flush=True)
    # PCIe-inclusive rate (host input in, logits out) for reference
    t0 = time.perf_counter()
    for _ in range(max(3, a.steps // 4)):
        sB.run(xB)
    ms_B_h2d = (time.perf_counter() - t0) / max(3, a.steps // 4) * 1e3
    sB.close()

    # ---- per-node device time from HIP events around every node ----
    node_ms = profiled_node_ms(N, Session, pB, xB, policy, a.steps, 2)

    # ---- batch 1 ----
    s1 = Session(p1, policy=policy, graph=not a.no_graph)
    y1_host = s1.run(x1)
    s1.upload_input(x1)
    ms_1 = time_steps(s1, max(a.steps, 50), a.warmup, ref=y1_host)
    s1.close()
    print(f"[bench] b1: {ms_1:.3f} ms/step", file=sys.stderr, flush=True)

    other = None if a.no_suite else suite(N, Session, models, yolo_cpu=cpu_y10)
    if other is not None:
        print(f"[bench] suite: {json.dumps(other)}", file=sys.stderr, flush=True)

    rows = conv_table(gB)
    layers = []
    tot_f = tot_t = ig_f = ig_t = 0.0
    n_ig = 0
    for r in rows:
        ms = float(node_ms[r["node"]])
        algo = algo_of(N, r, policy)
        gf = r["flops"] / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        layers.append(dict(node=r["node"], shape=f"{r['c']}x{r['h']}x{r['w']}->{r['oc']}x{r['oh']}x{r['ow']}",
                           k=f"{r['kh']}x{r['kw']}/s{r['sh']}", act=r["act"], algo=ALGO_NAMES.get(algo, str(algo)),
                           gflop=r["flops"] / 1e9, ms=ms, gflops=gf, frac_peak=gf * 1e9 / PEAK_FP32_MFMA))
        tot_f += r["flops"]
        tot_t += ms
        if algo == N.ALGO_IMPLICIT_GEMM:
            ig_f += r["flops"]
            ig_t += ms
            n_ig += 1
    all_ms = float(node_ms.sum())
    conv_tflops = tot_f / (tot_t * 1e-3) / 1e12
    ig_node_tflops = ig_f / (ig_t * 1e-3) / 1e12 if ig_t > 0 else 0.0
    live = conv_layers_live(N, rows, lambda r: algo_of(N, r, policy))
    ig_live = [e for e in live if e["algo"] == N.ALGO_IMPLICIT_GEMM]
    ig_live_ms = sum(e["ms"] * e["count"] for e in ig_live)
    ig_live_f = sum(e["flops"] * e["count"] for e in ig_live)
    ig_tflops = ig_live_f / (ig_live_ms * 1e-3) / 1e12 if ig_live_ms > 0 else ig_node_tflops
    # each layer's own roofline: MFMA time or HBM time (algorithmic bytes at 8 TB/s), whichever is longer
    ig_bound_ms = sum(max(e["flops"] / PEAK_FP32_MFMA, e["bytes"] / 8e12) * 1e3 * e["count"] for e in ig_live)
    ig_hbm_layers = sum(e["count"] for e in ig_live if e["bytes"] / 8e12 > e["flops"] / PEAK_FP32_MFMA)
    live_ms = sum(e["ms"] * e["count"] for e in live)
    live_f = sum(e["flops"] * e["count"] for e in live)
    live_ef = sum(e["exec_flops"] * e["count"] for e in live)
    print(f"[bench] implicit-GEMM kernels: {ig_live_ms:.3f} ms per pass back to back "
          f"({ig_tflops:.1f} TFLOP/s), {ig_t:.3f} ms in the per-node event pass ({ig_node_tflops:.1f}); "
          f"all conv kernels {live_ms:.3f} ms", file=sys.stderr, flush=True)
    out_layers = Path(a.layers_out)
    out_layers.parent.mkdir(parents=True, exist_ok=True)
    out_layers.write_text(json.dumps(dict(batch=a.batch, policy=a.policy, node_ms_total=all_ms,
                                          conv_ms_total=tot_t, layers=layers), indent=1))
    out_layers.with_suffix(".md").write_text(layers_markdown(live, a.batch, a.policy))

    ips = a.batch / (ms_B * 1e-3)
    line = {
        "metric": METRIC,
        "value": round(ips, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_B, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init ResNet-101, BN folded; input U[-1,1])",
        "config": {"workload": f"ResNet-101 v1.5 fp32 forward, batch {a.batch}, 3x224x224, ENNF through "
                               f"spinn_run over one HBM arena, input staged in HBM and copied into the arena "
                               f"each step (device to device, counted in the step), "
                               f"{'per-node launches' if a.no_graph else 'HIP-graph replay'}",
                   "batch": a.batch, "image": [3, 224, 224], "conv_layers": len(rows), "conv_policy": a.policy},
        "step_check": "each timed loop's output after its last step equals its first step's and spinn_run's "
                      "with host copies, bit for bit (b32, b1, VGG and YOLOv10n loops)",
        "images_per_s_b1": round(1e3 / ms_1, 2),
        "ms_per_step_b1": round(ms_1, 4),
        "images_per_s_with_host_copies": round(a.batch / (ms_B_h2d * 1e-3), 2),
        "conv_tflops_aggregate": round(conv_tflops, 3),
        "conv_frac_mfma_peak": round(conv_tflops * 1e12 / PEAK_FP32_MFMA, 4),
        "conv_share_of_node_time": round(tot_t / all_ms, 4) if all_ms > 0 else None,
        "conv_kernels": {
            "ms_per_pass": round(live_ms, 4),
            "gflop_direct": round(live_f / 1e9, 2), "gflop_executed": round(live_ef / 1e9, 2),
            "tflops_direct_equiv": round(live_f / (live_ms * 1e-3) / 1e12, 2),
            "frac_mfma_peak_direct_equiv": round(live_f / (live_ms * 1e-3) / PEAK_FP32_MFMA, 4),
            "tflops_executed": round(live_ef / (live_ms * 1e-3) / 1e12, 2),
            "frac_mfma_peak_executed": round(live_ef / (live_ms * 1e-3) / PEAK_FP32_MFMA, 4),
            "winograd_layers": sum(e["count"] for e in live if e["algo"] in (N.ALGO_WINOGRAD, N.ALGO_WINOGRAD_F43)),
            "method": "every conv layer's kernels launched 10x back to back in a HIP graph replayed between HIP "
                      "events; direct = "
                      "2*N*OC*OH*OW*C*KH*KW (Winograd credited at the direct count), executed = the MFMA work "
                      "issued (Winograd: (m+2)^2 tile GEMMs, transforms not counted)"},
        "roofline": {"bound": "mfma", "achieved": round(ig_tflops, 3), "peak": PEAK_FP32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": round(ig_tflops * 1e12 / PEAK_FP32_MFMA, 4),
                     "traffic": measured_traffic(a.batch, a.policy),
                     "kernel": f"conv_igemm_kernel / conv_igemm_sk_kernel / stem7_mfma_kernel (implicit-GEMM conv, {n_ig} layers, "
                               f"batch {a.batch})",
                     "launch_us": round(ig_live_ms / max(n_ig, 1) * 1e3, 2),
                     "achieved_node_events": round(ig_node_tflops, 3),
                     "frac_of_layer_rooflines": round(ig_bound_ms / ig_live_ms, 4) if ig_live_ms > 0 else None,
                     "hbm_bound_layers": ig_hbm_layers,
                     "method": "direct-conv FLOPs of the implicit-GEMM layers / their kernel time, each "
                               "layer's kernel launched 10x back to back in a HIP graph replayed between HIP events, "
                               "operands random (achieved_node_events: per-node events inside the model pass; "
                               "frac_of_layer_rooflines: sum over the layers of max(FLOPs / MFMA peak, algorithmic "
                               "bytes / 8 TB/s) / their summed kernel time; hbm_bound_layers: layers whose bytes "
                               "take longer than their FLOPs at peak)"},
        "cpu_baseline": cpu,
        "other_configs": other,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
