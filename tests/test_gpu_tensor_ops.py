"""GPU parity of the unfused-node kernels (spinn_hip_binary / unary / batchnorm /
softmax / block_copy / transpose / resize_nearest, and maxpool 5x5 s1) through
the C ABI: against the reference's own outputs (tests/golden/tensor_ops.npz),
against the oracle at detector-head sizes, on both the float4 and the scalar
paths (16-byte aligned and misaligned buffers), and on the edge cases."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_parity
from tests.hipops import (run_batchnorm, run_binary, run_concat, run_maxpool, run_reduce_mean, run_resize, run_softmax,
                          run_split, run_transpose, run_unary)
from tests.test_oracle import _ROUNDED, _params_axis, _tensor_op_cases

pytestmark = pytest.mark.gpu

BIN = {"add": 0, "sub": 1, "mul": 2, "div": 3}


def _hip_tensor_op(N, torch, name, ins, prm, out_shapes):
    op = name.split("_")[0]
    if op in BIN:
        return [run_binary(N, torch, BIN[op], ins[0], ins[1], out_shapes[0])]
    if op in ("relu", "sigmoid"):
        return [run_unary(N, torch, {"relu": 0, "sigmoid": 1}[op], ins[0])]
    if op == "batch":
        eps = float(np.frombuffer(prm[:4].tobytes(), np.float32)[0])
        return [run_batchnorm(N, torch, *ins, eps)]
    if op == "softmax":
        return [run_softmax(N, torch, ins[0], _params_axis(prm, -1))]
    if op == "concat":
        return [run_concat(N, torch, ins, _params_axis(prm, 0))]
    if op == "split":
        ax = _params_axis(prm, 0)
        return run_split(N, torch, ins[0], [sh[ax] for sh in out_shapes], ax)
    if op == "transpose":
        nd = ins[0].ndim
        return [run_transpose(N, torch, ins[0], list(prm[:nd]) if prm.size else None)]
    if op == "resize":
        return [run_resize(N, torch, ins[0], *out_shapes[0][2:])]
    if op == "maxpool":
        return [run_maxpool(N, torch, ins[0], *out_shapes[0][2:], 5, 5, 1, 1, 2, 2)]
    raise AssertionError(name)


@pytest.mark.parametrize("case", list(_tensor_op_cases()), ids=lambda c: c[0])
def test_matches_reference_fixture(hip, torch_gpu, case):
    name, ins, prm, outs = case
    print(f"[tensor-op] fixture {name}", flush=True)
    got = _hip_tensor_op(hip, torch_gpu, name, ins, prm, [o.shape for o in outs])
    for g, ref in zip(got, outs):
        if name in _ROUNDED or name.startswith("div"):
            np.testing.assert_allclose(g, ref, rtol=2e-6, atol=1e-7)
        else:
            np.testing.assert_array_equal(g, ref)


@pytest.mark.parametrize("offset", [0, 1], ids=["vec4", "scalar"])
def test_binary_broadcasts(hip, torch_gpu, offset):
    rng = np.random.default_rng(11 + offset)
    b16 = rng.uniform(-2, 2, (16, 4, 8400)).astype(np.float32)
    strides = rng.uniform(8, 32, (1, 8400)).astype(np.float32)
    anchors = rng.uniform(0, 80, (1, 2, 8400)).astype(np.float32)
    lt = rng.uniform(0, 9, (16, 2, 8400)).astype(np.float32)
    cases = [("mul", b16, strides, b16.shape), ("sub", anchors, lt, lt.shape), ("add", lt, anchors, lt.shape),
             ("mul", np.array([0.1767767], np.float32), b16, b16.shape), ("add", lt, lt, lt.shape),
             ("div", lt, anchors, lt.shape)]
    for op, a, b, shape in cases:
        print(f"[tensor-op] binary {op} {a.shape} {b.shape} offset {offset}", flush=True)
        y = run_binary(hip, torch_gpu, BIN[op], a, b, shape, offset=offset)
        ref = O.binary(op, a, b, shape)
        if op == "div":
            np.testing.assert_allclose(y, ref, rtol=1e-6)
        else:
            np.testing.assert_array_equal(y, ref)
    # odd element counts (no float4 path even when aligned)
    a = rng.uniform(-1, 1, 1001).astype(np.float32)
    b = rng.uniform(-1, 1, 7).astype(np.float32)
    np.testing.assert_array_equal(run_binary(hip, torch_gpu, 0, a, b, (1001,), offset), O.binary("add", a, b, (1001,)))


@pytest.mark.parametrize("offset", [0, 1], ids=["vec4", "scalar"])
def test_unary_and_batchnorm(hip, torch_gpu, offset):
    rng = np.random.default_rng(21 + offset)
    x = rng.uniform(-12, 12, (16, 80, 8400 // 4)).astype(np.float32)
    for op, name in ((0, "relu"), (1, "sigmoid"), (2, "silu")):
        print(f"[tensor-op] unary {name} offset {offset}", flush=True)
        y = run_unary(hip, torch_gpu, op, x, offset)
        if op == 0:
            np.testing.assert_array_equal(y, O.unary(name, x))
        else:
            np.testing.assert_allclose(y, O.unary(name, x), rtol=2e-6, atol=1e-7)
    for shape in ((2, 64, 40, 40), (3, 5, 7, 3), (4, 6)):
        print(f"[tensor-op] batchnorm {shape} offset {offset}", flush=True)
        xb = rng.uniform(-3, 3, shape).astype(np.float32)
        c = shape[1]
        p = [rng.uniform(0.5, 1.5, c).astype(np.float32) for _ in range(4)]
        y = run_batchnorm(hip, torch_gpu, xb, *p, 1e-3, offset)
        assert_parity(y, O.batchnorm(xb, *p, eps=1e-3), what=f"batchnorm {shape}")


@pytest.mark.parametrize("shape,axis", [
    ((32, 400, 400), -1),         # attention rows (batch 16 x 2 heads)
    ((3, 8400), -1),              # one long row per wave
    ((5, 1), -1),                 # dim 1
    ((7, 37), -1),                # dim < wave size
    ((16, 16, 4, 8400), 1),       # DFL: softmax over 16 bins, inner 33600
    ((2, 3, 5), 0),               # outer 1
    ((9, 64), -1),                # one value per lane
    ((9, 65), -1),                # two per lane, the second in lane 0 only
    ((6, 200), -1),               # four per lane, partial
    ((4, 1024), -1),              # sixteen per lane: the register form's longest row
    ((3, 1025), -1),              # one past it: the running (max, sum) form
    ((3, 32, 4, 10), 1),          # columns of 32
    ((2, 33, 12), 1),             # columns of 33: the running form
    ((4, 5, 7), 1),               # columns of 5, inner 7: one column per thread
    ((2, 16, 6, 2), 1),           # columns of 16, inner 12
], ids=["attn", "long", "dim1", "short", "dfl", "outer1", "dim64", "dim65", "dim200", "dim1024", "dim1025",
        "cols32", "cols33", "cols5", "cols16"])
def test_softmax(hip, torch_gpu, shape, axis):
    print(f"[tensor-op] softmax {shape} axis {axis}", flush=True)
    rng = np.random.default_rng(len(shape) * 100 + shape[-1])
    x = rng.uniform(-8, 8, shape).astype(np.float32)
    y = run_softmax(hip, torch_gpu, x, axis)
    ref = O.softmax(x, axis)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(y.sum(axis=axis), 1.0, rtol=1e-5)


@pytest.mark.parametrize("offset", [0, 1], ids=["vec4", "scalar"])
def test_concat_split(hip, torch_gpu, offset):
    rng = np.random.default_rng(31 + offset)
    head = [rng.uniform(-1, 1, (16, 144, n)).astype(np.float32) for n in (6400, 1600, 400)]
    print(f"[tensor-op] concat head offset {offset}", flush=True)
    np.testing.assert_array_equal(run_concat(hip, torch_gpu, head, 2, offset), O.concat(head, 2))
    c2f = [rng.uniform(-1, 1, (2, 32, 80, 80)).astype(np.float32) for _ in range(4)]
    np.testing.assert_array_equal(run_concat(hip, torch_gpu, c2f, 1, offset), O.concat(c2f, 1))
    odd = [rng.uniform(-1, 1, (3, k, 5)).astype(np.float32) for k in (1, 2, 3)]
    np.testing.assert_array_equal(run_concat(hip, torch_gpu, odd, 1, offset), O.concat(odd, 1))
    print("[tensor-op] split", flush=True)
    qkv = rng.uniform(-1, 1, (16, 2, 128, 400)).astype(np.float32)
    for got, ref in zip(run_split(hip, torch_gpu, qkv, [32, 32, 64], 2), O.split(qkv, [32, 32, 64], 2)):
        np.testing.assert_array_equal(got, ref)
    box = rng.uniform(-1, 1, (2, 144, 8400)).astype(np.float32)
    for got, ref in zip(run_split(hip, torch_gpu, box, [64, 80], 1), O.split(box, [64, 80], 1)):
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("shape,perm", [
    ((32, 32, 400), (0, 2, 1)),        # q^T: tiled batched 2-D path, ragged 400
    ((1, 2, 400, 400), (0, 1, 3, 2)),  # attention^T
    ((16, 4, 16, 8400), (0, 2, 1, 3)),  # DFL: general path, contiguous inner
    ((1, 84, 8400), (0, 2, 1)),        # head output -> [8400, 84]
    ((3, 5, 7, 2), (3, 0, 2, 1)),      # general
    ((33, 65), None),                  # reversed dims (no perm), 2-D tiled
    ((4, 1, 6), (1, 0, 2)),            # only a size-1 dim moves: a copy
    ((2, 3, 4), (0, 1, 2)),            # identity
], ids=["qT", "attnT", "dfl", "head", "general", "rev", "unit", "identity"])
def test_transpose(hip, torch_gpu, shape, perm):
    print(f"[tensor-op] transpose {shape} {perm}", flush=True)
    x = np.random.default_rng(int(np.prod(shape)) % 1000).uniform(-1, 1, shape).astype(np.float32)
    p = perm if perm is not None else tuple(range(len(shape)))[::-1]
    np.testing.assert_array_equal(run_transpose(hip, torch_gpu, x, perm), O.transpose(x, p))


def test_resize_and_sppf_pool(hip, torch_gpu):
    rng = np.random.default_rng(41)
    # exact 2x (the two-per-thread form, then odd width and a misaligned input: the general form),
    # other scales
    for shape, oh, ow, off in (((1, 256, 20, 20), 40, 40, 0), ((16, 128, 40, 40), 80, 80, 0),
                               ((3, 5, 7, 10), 14, 20, 0), ((2, 3, 4, 5), 8, 10, 0), ((2, 3, 4, 6), 8, 12, 1),
                               ((2, 3, 5, 3), 7, 8, 0), ((1, 2, 6, 6), 3, 4, 0)):
        print(f"[tensor-op] resize {shape} -> {oh}x{ow} offset {off}", flush=True)
        x = rng.uniform(-1, 1, shape).astype(np.float32)
        np.testing.assert_array_equal(run_resize(hip, torch_gpu, x, oh, ow, off), O.resize_nearest(x, oh, ow))
    x = rng.uniform(-1, 1, (16, 128, 20, 20)).astype(np.float32)
    print("[tensor-op] maxpool 5x5 s1 p2", flush=True)
    np.testing.assert_array_equal(run_maxpool(hip, torch_gpu, x, 20, 20, 5, 5, 1, 1, 2, 2),
                                  O.maxpool(x, 20, 20, 5, 5, 1, 1, 2, 2))


@pytest.mark.parametrize("shape,k,s,p", [
    ((32, 64, 112, 112), 3, 2, 1),  # ResNet stem pool at batch 32
    ((2, 5, 17, 16), 3, 2, 1),      # odd height: the last window hangs over the pad
    ((1, 3, 8, 8), 2, 2, 0),        # VGG-style 2x2 (runtime window)
    ((2, 4, 9, 11), 3, 1, 1),
    ((1, 2, 10, 9), 7, 3, 3),
    ((3, 2, 6, 7), 5, 1, 2),
    ((16, 128, 20, 20), 5, 1, 2),   # YOLOv10n SPPF pool at batch 16 (band/quad kernel)
    ((2, 3, 13, 12), 5, 1, 2),      # odd number of output rows per band pair
    ((1, 2, 9, 256), 3, 1, 1),      # one band of 64 quads per wave
    ((2, 3, 7, 12), 3, 2, 1),       # stride 2, last quad half past the row
    ((1, 4, 11, 36), 3, 1, 1),      # 9 quads: 7 bands per wave, lanes 63 idle
], ids=["r101-b32", "odd", "2x2", "3x3s1", "7x7s3", "5x5s1", "sppf-b16", "5x5-odd", "w256", "s2-w12",
        "w36"])
def test_maxpool_shapes(hip, torch_gpu, shape, k, s, p):
    """Bit-exact against the oracle, including NaN inputs (never selected: the reference keeps
    the running max unless val > max, SPINN/run_time/ops/pool/maxpool.c:36) and -inf."""
    n, c, h, w = shape
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    print(f"[tensor-op] maxpool {shape} k{k} s{s} p{p}", flush=True)
    x = np.random.default_rng(n * c + h).uniform(-1, 1, shape).astype(np.float32)
    flat = x.reshape(-1)
    flat[::97] = np.nan
    flat[5::89] = -np.inf
    np.testing.assert_array_equal(run_maxpool(hip, torch_gpu, x, oh, ow, k, k, s, s, p, p),
                                  O.maxpool(x, oh, ow, k, k, s, s, p, p))


@pytest.mark.parametrize("outer,dim,inner,offset,exact", [
    (32 * 2048, 49, 1, 0, True),  # ResNet-101 global average pool at batch 32 (7x7 map)
    (2048, 49, 1, 0, True),       # batch 1
    (300, 7, 1, 0, True),         # last block of 44 rows
    (257, 62, 1, 0, True),        # even rows: padded LDS stride, one row in the last block
    (5, 63, 1, 0, True),          # longest staged row
    (9, 1, 1, 0, True),
    (40, 64, 1, 0, False),        # one wave per row, shuffle-tree sum
    (3, 1000, 1, 0, False),
    (100, 49, 1, 1, False),       # input not 16-byte aligned: the wave kernel
    (4, 9, 17, 0, True),          # inner > 1: one thread per output, sequential sum
], ids=["gap-b32", "gap-b1", "ragged", "even", "d63", "d1", "wave64", "wave1000", "unaligned", "strided"])
def test_reduce_mean(hip, torch_gpu, outer, dim, inner, offset, exact):
    """The staged-row and strided kernels sum each row in the reference's order from 0
    (SPINN/run_time/ops/reduce/reduce_mean.c:68-72): bit-exact. Rows longer than 63 floats
    (or an unaligned input) take the wave kernel, whose shuffle tree reorders the additions:
    within 1e-6 absolute on inputs in [-1, 1]."""
    print(f"[tensor-op] reduce_mean outer={outer} dim={dim} inner={inner} offset={offset}", flush=True)
    x = np.random.default_rng(outer + dim + inner).uniform(-1, 1, outer * dim * inner).astype(np.float32)
    got = run_reduce_mean(hip, torch_gpu, x, outer, dim, inner, offset)
    want = O.reduce_mean(x, outer, dim, inner)
    if exact:
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)


def test_bad_arguments(hip, torch_gpu):
    L = hip.lib()
    buf = torch_gpu.zeros(64, device="cuda")
    p = C.c_void_p(buf.data_ptr())
    assert L.spinn_hip_binary(7, p, 4, p, 4, p, 4, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_binary(0, p, 0, p, 4, p, 4, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_binary(0, p, 4, p, 4, p, 0, None) == 0
    assert L.spinn_hip_binary(0, p, 4, p, 4, p, 1 << 33, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_unary(9, p, p, 4, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_softmax(2, 0, 3, p, p, None) == 0
    dims = (C.c_int64 * 3)(2, 2, 2)
    assert L.spinn_hip_transpose(3, dims, (C.c_int32 * 3)(0, 0, 1), p, p, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_transpose(3, dims, (C.c_int32 * 3)(0, 1, 3), p, p, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_transpose(9, dims, None, p, p, None) == hip.SPINN_HIP_EINVAL
    blocks = (hip.BlockCopy * 17)()
    assert L.spinn_hip_block_copy(blocks, 17, 1, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_resize_nearest(1, 0, 4, 4, 4, p, p, None) == hip.SPINN_HIP_EINVAL
    torch_gpu.cuda.synchronize()


@pytest.mark.parametrize("nbytes,src_off,dst_off", [
    (16, 0, 0),
    (59_000_000, 0, 0),           # a detector-head Reshape at batch 16
    (4 * 4096 * 4097, 0, 0),
    (4 * 1000 + 8, 0, 0),         # not a multiple of 16 bytes
    (4 * 1000, 4, 8),             # misaligned ends
    (4 * 1000, 16, 32),           # aligned offsets inside the buffers
])
def test_device_copy(hip, torch_gpu, nbytes, src_off, dst_off):
    """spinn_hip_copy (Reshape / Flatten / Identity, the resident runs' input restore)
    copies exactly `nbytes` bytes at any size and alignment and leaves the bytes
    around the destination run untouched."""
    print(f"[tensor-op] copy bytes={nbytes} src_off={src_off} dst_off={dst_off}", flush=True)
    L = hip.lib()
    n = (nbytes + src_off + 64) // 4 + 16
    rng = np.random.default_rng(nbytes % 1000 + src_off)
    src_h = rng.integers(0, 2**31, n, dtype=np.int64).astype(np.int32)
    src = torch_gpu.from_numpy(src_h).cuda()
    dst = torch_gpu.full(((nbytes + dst_off + 64) // 4 + 16,), -7, dtype=torch_gpu.int32, device="cuda")
    hip.check(L.spinn_hip_copy(C.c_void_p(dst.data_ptr() + dst_off), C.c_void_p(src.data_ptr() + src_off),
                               C.c_size_t(nbytes), None), "spinn_hip_copy")
    torch_gpu.cuda.synchronize()
    got = dst.cpu().numpy().view(np.uint8)
    want = np.full(got.shape, 0, np.uint8)
    want[:] = np.frombuffer(np.full(got.size // 4, -7, np.int32).tobytes(), np.uint8)
    want[dst_off:dst_off + nbytes] = src_h.view(np.uint8)[src_off:src_off + nbytes]
    np.testing.assert_array_equal(got, want)
