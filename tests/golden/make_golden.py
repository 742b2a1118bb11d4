"""Write the golden fixtures in tests/golden/ from the reference's own CPU code.

Runs only where the reference sources exist: it builds oracle/_ref/libspinn_ref.so
with oracle/Makefile (the reference's run_time C sources compiled in place) and
calls the reference functions on small seeded inputs. Each fixture is an .npz
of inputs and the reference's outputs (no code), loaded with allow_pickle=False.

    python tests/golden/make_golden.py [planner conv epilogue gemm winograd tensor_ops postproc models converter]

Fixtures:
  planner_offsets.npz   spinn_load + spinn_plan_memory offsets and peak for
                        generated ENNF models (SPINN/run_time/spinn_memory_planner.c)
  conv_raw.npz          op_conv2d, group == 1: the shipped packed path returns the
                        raw accumulator (bias / act / residual dropped,
                        SPINN/run_time/ops/mm/gemm_kernel.c:497-590)
  conv_grouped.npz      op_conv2d, group > 1: full epilogue (sgemm_nn path)
  epilogue.npz          sgemm_nn with bias and every act code (gemm_kernel.c:304-339)
  gemm.npz              op_gemm (transB, bias vector / matrix) and op_matmul (batched)
  winograd.npz          winograd_pack_weight + winograd_conv_3x3 (SPINN/run_time/ops/conv/winograd.c)
                        on the identity KAT of SPINN/run_time/test_winograd2.c:56-63 and a seeded case
  tensor_ops.npz        op_add / op_sub / op_mul / op_div (modulo broadcast), op_relu, op_sigmoid,
                        op_batch_norm, op_softmax, op_concat, op_split, op_transpose, op_resize and
                        op_maxpool 5x5 s1 p2 on small seeded inputs (the unfused nodes of a detector)
  postproc.npz          op_reduce_max, op_topk (ties, signed zeros), op_gather_elements, op_tile,
                        op_cast, op_mod / op_div on int64, int32 and fp32, op_unsqueeze: the
                        detector's post-processing tail on small seeded inputs
  models_as_shipped.npz spinn_load + spinn_plan + spinn_run of generated models (YOLOv10n at
                        64x64, a 4-block ResNet at 64x64, batch 2): the reference's output and an input fingerprint
  converter.npz         SHA-256 (and, for small files, the bytes) of the reference converter's
                        output (SPINN/onnx2ennf.c, oracle/_ref/onnx2ennf) for the .onnx files of
                        converter_cases.CASES, unwritten parameter bytes zeroed
"""
from __future__ import annotations

import ctypes as C
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from spinn_amd import models  # noqa: E402
from spinn_amd.native import SpinnTensor, SpinnContext  # noqa: E402  (same struct layout as the reference's)

REF_LIB = ROOT / "oracle" / "_ref" / "libspinn_ref.so"
TENSOR_OPS = ("op_add", "op_sub", "op_mul", "op_div", "op_relu", "op_sigmoid", "op_batch_norm", "op_softmax",
              "op_concat", "op_split", "op_transpose", "op_resize", "op_maxpool")
POSTPROC_OPS = ("op_reduce_max", "op_topk", "op_gather_elements", "op_tile", "op_cast", "op_mod", "op_unsqueeze")
FP = C.POINTER(C.c_float)


def ref_lib() -> C.CDLL:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "-j8", "ref"], check=True)
    L = C.CDLL(str(REF_LIB))
    L.spinn_load.restype = C.c_void_p
    L.spinn_load.argtypes = [C.c_char_p]
    L.spinn_plan_memory.argtypes = [C.c_void_p, C.c_uint32]
    L.spinn_free.argtypes = [C.c_void_p]
    sig = [C.POINTER(C.POINTER(SpinnTensor)), C.c_int, C.c_void_p, C.c_uint16, C.POINTER(C.POINTER(SpinnTensor)),
           C.c_int]
    for f in ("op_conv2d", "op_gemm", "op_matmul") + TENSOR_OPS + POSTPROC_OPS:
        getattr(L, f).argtypes = sig
        getattr(L, f).restype = C.c_int
    L.sgemm_nn.argtypes = [C.c_int, C.c_int, C.c_int, FP, C.c_int, FP, C.c_int, FP, C.c_int, FP, C.c_int, FP]
    L.winograd_pack_weight.restype = C.c_void_p
    L.winograd_pack_weight.argtypes = [FP, C.c_int, C.c_int]
    L.winograd_conv_3x3.argtypes = [FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, FP, C.c_int,
                                    C.c_int, FP, C.c_int, C.c_int, C.c_int]
    L.winograd_conv_3x3.restype = C.c_int
    return L


def _fp(a):
    return None if a is None else a.ctypes.data_as(FP)


_ENNF_DT = {np.dtype(np.float32): 1, np.dtype(np.int32): 6, np.dtype(np.int64): 7}


def tensor(arr: np.ndarray, keep: list) -> SpinnTensor:
    t = SpinnTensor()
    t.dtype = _ENNF_DT[arr.dtype]
    t.ndim = arr.ndim
    for i, d in enumerate(arr.shape):
        t.dims[i] = d
    t.elem_count = arr.size
    t.size = arr.nbytes
    t.data = arr.ctypes.data
    keep.append(arr)
    return t


def call_op(L, name, ins, params: bytes, outs):
    keep = []
    tin = [tensor(a, keep) for a in ins]
    tout = [tensor(a, keep) for a in outs]
    pin = (C.POINTER(SpinnTensor) * len(tin))(*[C.pointer(t) for t in tin])
    pout = (C.POINTER(SpinnTensor) * len(tout))(*[C.pointer(t) for t in tout])
    pbuf = C.create_string_buffer(params, len(params)) if params else None
    rc = getattr(L, name)(pin, len(tin), C.cast(pbuf, C.c_void_p) if pbuf else None, len(params), pout, len(tout))
    assert rc == 0, (name, rc)
    # packed weights the reference cached on the weight tensor are its own to free; leak-free enough for a script


def planner(L):
    cases = {
        "conv0": models.conv_bn_relu(seed=0)[0],
        "resnet101_b1": models.resnet101(batch=1, seed=0)[0],
        "resnet101_b4": models.resnet101(batch=4, seed=0)[0],
        "vgg_b2": models.vgg_stack(batch=2, seed=3, in_c=16, schedule=[(16, 32), (16, 32), (32, 16), (32, 16)])[0],
        "gemm_32": models.gemm_model(32, 1000, 2048, seed=1)[0],
        "yolov10n_b1": models.yolov10n(batch=1, seed=0)[0],
        "yolov10n_b2_320": models.yolov10n(batch=2, seed=0, hw=320)[0],
    }
    out = {}
    tmp = HERE / "_tmp_planner.ennf"
    for name, g in cases.items():
        g.write(tmp)
        ctx = L.spinn_load(str(tmp).encode())
        assert ctx
        peak = L.spinn_plan_memory(ctx, 0)
        cp = C.cast(ctx, C.POINTER(SpinnContext)).contents
        ids, offs = [], []
        for i in range(cp.num_tensors):
            t = cp.tensors[i]
            if not t.is_weight and t.size > 0:
                ids.append(i)
                offs.append(t.offset)
        # also the capped plan that must fail with SPINN_MEM_ERR_NOMEM
        ctx2 = L.spinn_load(str(tmp).encode())
        capped = L.spinn_plan_memory(ctx2, max(16, peak // 2))
        L.spinn_free(ctx2)
        L.spinn_free(ctx)
        out[f"{name}_ids"] = np.array(ids, np.int32)
        out[f"{name}_offsets"] = np.array(offs, np.int64)
        out[f"{name}_peak"] = np.array([peak], np.int64)
        out[f"{name}_capped_rc"] = np.array([capped], np.int64)
    tmp.unlink()
    np.savez_compressed(HERE / "planner_offsets.npz", **out)


def conv_cases(L):
    from spinn_amd.ennf import conv_params
    rng = np.random.default_rng(1234)
    raw, grouped = {}, {}
    # (n, c, h, w, oc, k, stride, pad, group, act)
    specs = [
        (1, 8, 9, 9, 6, 3, 1, 1, 1, 1),
        (2, 5, 7, 6, 7, 3, 2, 1, 1, 5),
        (1, 16, 8, 8, 13, 1, 1, 0, 1, 0),
        (1, 4, 11, 11, 8, 1, 2, 0, 1, 3),
        (1, 3, 15, 15, 8, 7, 2, 3, 1, 1),
        (2, 8, 10, 10, 8, 3, 1, 1, 8, 3),   # depthwise, SiLU
        (1, 6, 9, 9, 6, 3, 2, 1, 6, 1),     # depthwise stride 2
        (1, 8, 6, 6, 12, 3, 1, 1, 4, 5),    # grouped, residual
        (1, 4, 7, 7, 4, 5, 1, 2, 4, 0),     # depthwise 5x5
    ]
    for i, (n, c, h, w, oc, k, s, p, g, act) in enumerate(specs):
        oh = (h + 2 * p - k) // s + 1
        ow = (w + 2 * p - k) // s + 1
        x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
        wt = rng.normal(0, 0.3, (oc, c // g, k, k)).astype(np.float32)
        b = rng.normal(0, 0.1, oc).astype(np.float32)
        r = rng.uniform(-1, 1, (n, oc, oh, ow)).astype(np.float32) if act in (4, 5) else None
        y = np.zeros((n, oc, oh, ow), np.float32)
        ins = [x, wt, b] + ([r] if r is not None else [])
        call_op(L, "op_conv2d", ins, conv_params(k, k, s, s, (p, p, p, p), g, act), [y])
        d = raw if g == 1 else grouped
        d[f"c{i}_spec"] = np.array([n, c, h, w, oc, k, s, p, g, act], np.int32)
        d[f"c{i}_x"], d[f"c{i}_w"], d[f"c{i}_b"], d[f"c{i}_y"] = x, wt, b, y
        if r is not None:
            d[f"c{i}_r"] = r
    np.savez_compressed(HERE / "conv_raw.npz", **raw)
    np.savez_compressed(HERE / "conv_grouped.npz", **grouped)


def epilogue(L):
    rng = np.random.default_rng(99)
    out = {}
    M, N, K = 7, 37, 11
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.normal(0, 0.5, M).astype(np.float32)
    r = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    out["a"], out["b"], out["bias"], out["r"] = a, b, bias, r
    for act in (0, 1, 2, 3, 4, 5):
        y = np.zeros((M, N), np.float32)
        L.sgemm_nn(M, N, K, _fp(a), K, _fp(b), N, _fp(y), N, _fp(bias), act, _fp(r))
        out[f"y_act{act}"] = y
    np.savez_compressed(HERE / "epilogue.npz", **out)


def tensor_ops(L):
    """The unfused operators on small seeded inputs: each case stores its inputs,
    the params it was called with and the reference's outputs."""
    import struct
    from spinn_amd.ennf import pool_params
    rng = np.random.default_rng(2024)
    out = {}

    def u(*shape, lo=-2.0, hi=2.0):
        return rng.uniform(lo, hi, shape).astype(np.float32)

    def case(name, op, ins, params, out_shapes):
        ys = [np.zeros(sh, np.float32) for sh in out_shapes]
        call_op(L, op, ins, params, ys)
        for i, a in enumerate(ins):
            out[f"{name}_in{i}"] = a
        for i, y in enumerate(ys):
            out[f"{name}_out{i}"] = y
        out[f"{name}_params"] = np.frombuffer(params, np.uint8).copy() if params else np.zeros(0, np.uint8)

    axis = lambda a: struct.pack("<i", a)  # noqa: E731
    case("add_same", "op_add", [u(2, 3, 9), u(2, 3, 9)], b"", [(2, 3, 9)])
    case("add_bcast", "op_add", [u(2, 3, 4), u(4)], b"", [(2, 3, 4)])
    case("sub_anchor", "op_sub", [u(1, 2, 12), u(3, 2, 12)], b"", [(3, 2, 12)])
    case("mul_stride", "op_mul", [u(2, 4, 12), u(1, 12)], b"", [(2, 4, 12)])
    case("mul_scalar", "op_mul", [u(3, 11), np.array([0.17677669], np.float32)], b"", [(3, 11)])
    case("mul_same", "op_mul", [u(5, 13), u(5, 13)], b"", [(5, 13)])
    den = u(4, 5)
    den[0, :3] = [0.0, 4e-7, -5e-7]
    case("div_eps", "op_div", [u(4, 5), den], b"", [(4, 5)])
    case("relu", "op_relu", [u(3, 7, 5)], b"", [(3, 7, 5)])
    case("sigmoid", "op_sigmoid", [u(2, 19, lo=-9, hi=9)], b"", [(2, 19)])
    c = 3
    case("batch_norm", "op_batch_norm",
         [u(2, c, 5, 5), u(c, lo=0.5, hi=1.5), u(c, lo=-0.2, hi=0.2), u(c, lo=-0.1, hi=0.1), u(c, lo=0.5, hi=1.5)],
         struct.pack("<ffB3x", 1e-3, 0.9, 0), [(2, c, 5, 5)])
    case("softmax_last", "op_softmax", [u(6, 21, lo=-5, hi=5)], axis(-1), [(6, 21)])
    case("softmax_short", "op_softmax", [u(4, 5)], axis(1), [(4, 5)])
    case("softmax_mid", "op_softmax", [u(2, 16, 4, 10, lo=-4, hi=4)], axis(1), [(2, 16, 4, 10)])
    case("concat_c", "op_concat", [u(2, 2, 3, 3), u(2, 4, 3, 3), u(2, 1, 3, 3)], axis(1), [(2, 7, 3, 3)])
    case("concat_last", "op_concat", [u(1, 5, 6), u(1, 5, 2), u(1, 5, 3)], axis(2), [(1, 5, 11)])
    case("split_c", "op_split", [u(2, 6, 4, 4)], struct.pack("<iI", 1, 2), [(2, 2, 4, 4), (2, 4, 4, 4)])
    case("split_qkv", "op_split", [u(1, 2, 8, 5)], struct.pack("<iI", 2, 3),
         [(1, 2, 2, 5), (1, 2, 2, 5), (1, 2, 4, 5)])

    def perm_params(perm):
        return bytes(list(perm) + [0] * (8 - len(perm)) + [len(perm), 0, 0, 0])

    case("transpose_dfl", "op_transpose", [u(2, 4, 6, 5)], perm_params((0, 2, 1, 3)), [(2, 6, 4, 5)])
    case("transpose_last2", "op_transpose", [u(2, 3, 4, 5)], perm_params((0, 1, 3, 2)), [(2, 3, 5, 4)])
    case("transpose_rev", "op_transpose", [u(3, 7)], b"", [(7, 3)])
    case("resize_2x", "op_resize", [u(1, 3, 4, 5)], b"", [(1, 3, 8, 10)])
    case("resize_odd", "op_resize", [u(2, 2, 5, 3)], b"", [(2, 2, 7, 8)])
    case("maxpool_sppf", "op_maxpool", [u(1, 3, 7, 7)], pool_params(5, 5, 1, 1, (2, 2, 2, 2)), [(1, 3, 7, 7)])
    np.savez_compressed(HERE / "tensor_ops.npz", **out)


def postproc(L):
    """The detector post-processing operators (the exported YOLOv10 tail) on
    small seeded inputs: ReduceMax, TopK (with ties and signed zeros), GatherElements
    (negative and out-of-range indices, int64 and int32), Tile (int64 and fp32),
    Cast, Mod / Div on int64 and fp32 Mod, Unsqueeze."""
    import struct
    rng = np.random.default_rng(2025)
    out = {}

    def case(name, op, ins, params, outs):
        ys = [np.zeros(sh, dt) for sh, dt in outs]
        call_op(L, op, ins, params, ys)
        for i, a in enumerate(ins):
            out[f"{name}_in{i}"] = a
        for i, y in enumerate(ys):
            out[f"{name}_out{i}"] = y
        out[f"{name}_params"] = np.frombuffer(params, np.uint8).copy() if params else np.zeros(0, np.uint8)

    f32, i64, i32 = np.float32, np.int64, np.int32
    # ReduceMax: ties, signed zeros, an all-negative row
    x = np.round(rng.uniform(-1, 1, (1, 37, 80)), 1).astype(f32)
    x[0, 0, :] = -0.0
    x[0, 1, :5] = [0.0, -0.0, 0.0, -0.0, 0.0]
    x[0, 1, 5:] = -1.0
    x[0, 2, :] = -np.abs(x[0, 2, :]) - 0.5
    case("reduce_max_scores", "op_reduce_max", [x], struct.pack("<8iBBBB", -1, *([0] * 7), 1, 0, 0, 0),
         [((1, 37), f32)])
    case("reduce_max_rows", "op_reduce_max", [rng.uniform(-3, 3, (5, 9)).astype(f32)], b"", [((5,), f32)])
    # TopK: two rows, values on a coarse grid so many values tie; +0.0 and -0.0 mixed in
    tk = np.round(rng.uniform(-1, 1, (2, 700)), 2).astype(f32)
    tk[0, ::7] = 0.0
    tk[0, 3::7] = -0.0
    tk[1, 100:400] = 0.5
    topk_params = struct.pack("<iBB2x", -1, 1, 1)
    case("topk_ties", "op_topk", [tk, np.array([300], i64)], topk_params, [((2, 300), f32), ((2, 300), i64)])
    case("topk_all", "op_topk", [rng.uniform(-1, 1, (1, 50)).astype(f32), np.array([50], i64)], topk_params,
         [((1, 50), f32), ((1, 50), i64)])
    case("topk_flat", "op_topk", [rng.uniform(0, 1, (1, 6000)).astype(f32), np.array([300], i64)], topk_params,
         [((1, 300), f32), ((1, 300), i64)])
    # GatherElements: the detector's two forms, with negative and out-of-range indices
    data = rng.uniform(-1, 1, (1, 37, 4)).astype(f32)
    idx = rng.integers(-37, 37, (1, 10, 4)).astype(i64)
    idx[0, 0, :] = [40, -40, 36, -1]
    gparams = lambda a: struct.pack("<ii", a, 0)  # noqa: E731
    case("gather_boxes", "op_gather_elements", [data, idx], gparams(1), [((1, 10, 4), f32)])
    data = rng.uniform(-1, 1, (2, 5, 6)).astype(f32)
    idx = rng.integers(0, 6, (2, 5, 3)).astype(i32)
    case("gather_last_i32", "op_gather_elements", [data, idx], gparams(-1), [((2, 5, 3), f32)])
    data = rng.uniform(-1, 1, (6, 4)).astype(f32)
    case("gather_axis0", "op_gather_elements", [data, rng.integers(0, 6, (3, 4)).astype(i64)], gparams(0),
         [((3, 4), f32)])
    # Tile: the detector's index broadcast and an fp32 2-D tile
    case("tile_idx", "op_tile", [rng.integers(0, 8400, (1, 10, 1)).astype(i64), np.array([1, 1, 80], i64)], b"",
         [((1, 10, 80), i64)])
    case("tile_f32", "op_tile", [rng.uniform(-1, 1, (2, 3)).astype(f32), np.array([2, 2], i64)], b"",
         [((4, 6), f32)])
    # Cast: int64 -> fp32 (one value needs rounding), fp32 -> int64 (truncation), int32 <-> int64
    ci = np.array([0, 1, -7, 79, 2 ** 40 + 1, -(2 ** 31), 16777217], i64)
    case("cast_i64_f32", "op_cast", [ci], struct.pack("<BB2x", 1, 0), [((7,), f32)])
    case("cast_f32_i64", "op_cast", [np.array([0.0, 1.9, -1.9, 79.5, -0.0, 123456.7], f32)],
         struct.pack("<BB2x", 7, 0), [((6,), i64)])
    case("cast_i32_i64", "op_cast", [np.array([5, -5, 2 ** 31 - 1], i32)], struct.pack("<BB2x", 7, 0), [((3,), i64)])
    case("cast_i64_i32", "op_cast", [np.array([5, -5, 2 ** 33 + 7], i64)], struct.pack("<BB2x", 6, 0), [((3,), i32)])
    # Mod / Div: label = index mod nc, anchor = index / nc (scalar divisor), negatives, a zero divisor
    flat = rng.integers(0, 24000, (1, 300)).astype(i64)
    nc = np.array(80, i64)
    case("mod_labels", "op_mod", [flat, nc.reshape(())], b"", [((1, 300), i64)])
    case("div_anchor", "op_div", [flat, nc.reshape(())], b"", [((1, 300), i64)])
    sa = np.array([7, -7, 7, -7, 5, 0], i64)
    sb = np.array([3, 3, -3, -3, 0, 4], i64)
    case("mod_signs", "op_mod", [sa, sb], b"", [((6,), i64)])
    case("div_signs", "op_div", [sa, sb], b"", [((6,), i64)])
    case("mod_i32", "op_mod", [sa.astype(i32), np.array([4], i32)], b"", [((6,), i32)])
    case("mod_f32", "op_mod", [np.array([5.5, -5.5, 7.25, 1e-3, -0.0], f32), np.array([2.0, 2.0, -2.5], f32)], b"",
         [((5,), f32)])
    case("unsqueeze", "op_unsqueeze", [rng.integers(0, 99, (1, 7)).astype(i64), np.array([-1], i64)], b"",
         [((1, 7, 1), i64)])
    np.savez_compressed(HERE / "postproc.npz", **out)


MODEL_CASES = {
    # name: (generator, kwargs) - small enough that input and output stay a few KB
    "yolov10n_64": ("yolov10n", dict(batch=1, seed=5, hw=64)),
    "resnet_64": ("resnet", dict(batch=2, seed=6, blocks=(1, 1, 1, 1), hw=64, num_classes=10)),
    "yolov10n_64_post": ("yolov10n", dict(batch=1, seed=5, hw=64, postprocess=True)),
}


def models_as_shipped(L):
    """Whole ENNF models through the reference's spinn_load / spinn_plan /
    spinn_run: its output is the as-shipped one (group==1 convs drop the
    epilogue), which the oracle reproduces with oracle_set_as_shipped(1)."""
    L.spinn_plan.argtypes = [C.c_void_p, C.c_uint32]
    L.spinn_run.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    out = {}
    tmp = HERE / "_tmp_model.ennf"
    for name, (gen, kw) in MODEL_CASES.items():
        g, x = getattr(models, gen)(**kw)
        g.write(tmp)
        ctx = L.spinn_load(str(tmp).encode())
        assert ctx and L.spinn_plan(ctx, 0) == 0
        y = np.zeros(g.dims(g.outputs[0]), np.float32)
        assert L.spinn_run(ctx, x.ctypes.data, y.ctypes.data) == 0
        L.spinn_free(ctx)
        # the generator recreates the input from the seed; keep a fingerprint to catch drift
        out[f"{name}_x_sum"] = np.array([x.astype(np.float64).sum(), x.ravel()[0], x.ravel()[-1]])
        out[f"{name}_y"] = y
    tmp.unlink()
    np.savez_compressed(HERE / "models_as_shipped.npz", **out)


def gemm(L):
    from spinn_amd.ennf import gemm_params
    rng = np.random.default_rng(7)
    out = {}
    specs = [(1, 40, 64, 0, 1, 1), (9, 33, 20, 0, 1, 1), (12, 10, 16, 1, 0, 2), (5, 6, 7, 1, 1, 0), (32, 50, 96, 0, 1, 1)]
    for i, (m, n, k, ta, tb, cm) in enumerate(specs):
        a = rng.uniform(-1, 1, (k, m) if ta else (m, k)).astype(np.float32)
        b = (rng.standard_normal((n, k) if tb else (k, n)) / np.sqrt(k)).astype(np.float32)
        c = None if cm == 0 else rng.normal(0, 0.1, n if cm == 1 else (m, n)).astype(np.float32)
        y = np.zeros((m, n), np.float32)
        call_op(L, "op_gemm", [a, b] + ([c] if c is not None else []), gemm_params(1.0, 1.0, ta, tb), [y])
        out[f"g{i}_spec"] = np.array([m, n, k, ta, tb, cm], np.int32)
        out[f"g{i}_a"], out[f"g{i}_b"], out[f"g{i}_y"] = a, b, y
        if c is not None:
            out[f"g{i}_c"] = c
    a = rng.uniform(-1, 1, (3, 5, 8)).astype(np.float32)
    b = rng.uniform(-1, 1, (3, 8, 6)).astype(np.float32)
    y = np.zeros((3, 5, 6), np.float32)
    call_op(L, "op_matmul", [a, b], b"", [y])
    out["mm_a"], out["mm_b"], out["mm_y"] = a, b, y
    np.savez_compressed(HERE / "gemm.npz", **out)


def winograd(L):
    out = {}
    # identity KAT (SPINN/run_time/test_winograd2.c:56-63): 4x4 input 1..16, 3x3 kernel = centre tap, pad 1
    x = np.arange(1, 17, dtype=np.float32).reshape(1, 1, 4, 4)
    w = np.zeros((1, 1, 3, 3), np.float32)
    w[0, 0, 1, 1] = 1.0
    rng = np.random.default_rng(5)
    cases = [("kat", x, w, None)]
    x2 = rng.uniform(-1, 1, (1, 6, 8, 8)).astype(np.float32)
    w2 = rng.normal(0, 0.3, (5, 6, 3, 3)).astype(np.float32)
    b2 = rng.normal(0, 0.1, 5).astype(np.float32)
    cases.append(("rand", x2, w2, b2))
    for name, xx, ww, bb in cases:
        n, c, h, wd = xx.shape
        oc = ww.shape[0]
        U = L.winograd_pack_weight(_fp(ww), oc, c)
        y = np.zeros((n, oc, h, wd), np.float32)
        rc = L.winograd_conv_3x3(_fp(xx), n, c, h, wd, U, oc, _fp(bb), 1, 1, _fp(y), h, wd, 1)
        assert rc == 0, rc
        out[f"{name}_x"], out[f"{name}_w"], out[f"{name}_y"] = xx, ww, y
        if bb is not None:
            out[f"{name}_b"] = bb
    np.savez_compressed(HERE / "winograd.npz", **out)


def converter(_L):
    """SHA-256 of the reference converter's output (SPINN/onnx2ennf.c, built by `make -C oracle ref`)
    for each graph of converter_cases.CASES, written as an .onnx file by spinn_amd.onnx, with the
    parameter bytes the converter leaves unwritten zeroed; the small files are kept whole."""
    import os
    import subprocess
    import tempfile

    from tests.golden import converter_cases as CC
    exe = HERE.parents[1] / "oracle" / "_ref" / "onnx2ennf"
    out = {}
    with tempfile.TemporaryDirectory() as td:
        for name, (make, env, _kw) in CC.CASES.items():
            src, dst = Path(td) / f"{name}.onnx", Path(td) / f"{name}.ennf"
            src.write_bytes(make().to_onnx())
            subprocess.run([str(exe), str(src), str(dst)], check=True, stdout=subprocess.DEVNULL,
                           env={**os.environ, **env})
            buf = CC.mask_unset(dst.read_bytes())
            out[f"{name}_sha256"] = CC.digest(buf)
            out[f"{name}_size"] = np.array([len(buf)], np.int64)
            if len(buf) < 64 * 1024:
                out[f"{name}_bytes"] = np.frombuffer(buf, np.uint8)
    np.savez_compressed(HERE / "converter.npz", **out)


def main():
    L = ref_lib()
    steps = {"planner": planner, "conv": conv_cases, "epilogue": epilogue, "gemm": gemm, "winograd": winograd,
             "tensor_ops": tensor_ops, "postproc": postproc, "models": models_as_shipped, "converter": converter}
    for name in sys.argv[1:] or list(steps):
        steps[name](L)
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
