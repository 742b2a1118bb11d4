"""GPU parity of the detector post-processing operators (ReduceMax, TopK,
GatherElements, Tile, Cast, integer Div / Mod) through the C ABI: bit for bit
against the reference's own operators (tests/golden/postproc.npz) and against
the oracle at detector sizes; then the whole YOLOv10n graph with its exported
TopK tail through spinn_run, the tail checked bit for bit against the oracle's
tail applied to the device's own pre-TopK tensor."""
import ctypes as C
import struct

import numpy as np
import pytest

from oracle import oracle as O
from spinn_amd import models
from spinn_amd.runtime import Session
from tests.conftest import assert_parity
from tests.test_oracle import _postproc_cases, oracle_postproc

pytestmark = pytest.mark.gpu

_DT = {np.dtype(np.float32): 1, np.dtype(np.int32): 6, np.dtype(np.int64): 7}


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _p(t):
    return C.c_void_p(t.data_ptr())


def _empty(torch, shape, dtype):
    tdt = {np.dtype(np.float32): torch.float32, np.dtype(np.int32): torch.int32,
           np.dtype(np.int64): torch.int64}[np.dtype(dtype)]
    t = torch.empty(tuple(shape), dtype=tdt, device="cuda")
    t.view(torch.uint8).fill_(0xA5)  # poison: every element must be written
    return t


def device_postproc(N, torch, name, ins, prm, out_shapes, out_dtypes):
    """Run the device operator a fixture case exercises; returns numpy outputs."""
    L = N.lib()
    d_in = [_dev(torch, a) for a in ins]
    outs = [_empty(torch, s, dt) for s, dt in zip(out_shapes, out_dtypes)]
    if name.startswith("reduce_max"):
        rc = L.spinn_hip_reduce_max(outs[0].numel(), ins[0].size // outs[0].numel(), _p(d_in[0]), _p(outs[0]), None)
    elif name.startswith("topk"):
        n = ins[0].shape[-1]
        k = out_shapes[0][-1]
        rc = L.spinn_hip_topk(ins[0].size // n, n, k, _p(d_in[0]), _p(outs[0]), _p(outs[1]), None)
    elif name.startswith("gather"):
        axis = struct.unpack("<i", prm[:4])[0] % ins[0].ndim
        d = N.GatherDesc()
        d.ndim, d.axis, d.index_dtype = ins[0].ndim, axis, _DT[ins[1].dtype]
        for i in range(ins[0].ndim):
            d.in_dims[i], d.out_dims[i] = ins[0].shape[i], out_shapes[0][i]
        rc = L.spinn_hip_gather_elements(C.byref(d), _p(d_in[0]), _p(d_in[1]), _p(outs[0]), None)
    elif name.startswith("tile"):
        nd = ins[0].ndim
        rc = L.spinn_hip_tile(nd, (C.c_int64 * nd)(*ins[0].shape), (C.c_int64 * nd)(*out_shapes[0]),
                              ins[0].dtype.itemsize, _p(d_in[0]), _p(outs[0]), None)
    elif name.startswith("cast"):
        rc = L.spinn_hip_cast(_DT[ins[0].dtype], _DT[np.dtype(out_dtypes[0])], ins[0].size, _p(d_in[0]), _p(outs[0]),
                              None)
    elif name.startswith("mod") or name.startswith("div"):
        op = N.BINARY_MOD if name.startswith("mod") else N.BINARY_DIV
        rc = L.spinn_hip_binary_typed(op, _DT[ins[0].dtype], _p(d_in[0]), ins[0].size, _p(d_in[1]), ins[1].size,
                                      _p(outs[0]), outs[0].numel(), None)
    elif name == "unsqueeze":
        rc = L.spinn_hip_copy(_p(outs[0]), _p(d_in[0]), ins[0].nbytes, None)
    else:
        raise KeyError(name)
    N.check(rc, name)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("case", _postproc_cases(), ids=lambda c: c[0])
def test_postproc_matches_reference(hip, torch_gpu, case):
    name, ins, prm, outs = case
    print(f"[postproc] {name}", flush=True)
    got = device_postproc(hip, torch_gpu, name, ins, prm, [o.shape for o in outs], [o.dtype for o in outs])
    for g, ref in zip(got, outs):
        assert g.shape == ref.shape and g.dtype == ref.dtype
        np.testing.assert_array_equal(g.view(np.uint8), ref.view(np.uint8))


@pytest.mark.parametrize("rows,n,k,grid", [(16, 8400, 300, 0.01), (2, 24000, 300, 0.05), (3, 1024, 1024, 0.25),
                                          (1, 97, 1, 0.0), (4, 5000, 700, 0.0), (1, 24000, 300, 0.5),
                                          (3, 100003, 7, 0.001), (2, 9000, 1, 0.0), (2, 8192, 300, 0.01),
                                          (1, 8193, 64, 0.01), (2, 16384, 300, 0.05), (1, 32768, 1024, 0.01),
                                          (1, 32769, 300, 0.01)])
def test_topk_detector_sizes(hip, torch_gpu, rows, n, k, grid):
    """Sizes of the detector tail (8400 anchors, 300 x 80 candidates, batch 16),
    k = n, k = 1 and k > 512, long rows, with values on a grid so ties are everywhere (a
    0.5 grid leaves five distinct values); rows of 8, 16 and 32 chunks of 1024 and one
    element past each (the register-resident kernels and the streaming one beyond)."""
    print(f"[topk] rows={rows} n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k)
    x = rng.uniform(-1, 1, (rows, n)).astype(np.float32)
    if grid:
        x = (np.round(x / grid) * grid).astype(np.float32)
    x[:, ::11] = -0.0
    ref_v, ref_i = O.topk(x, k)
    got_v, got_i = device_postproc(hip, torch_gpu, "topk", [x, np.array([k], np.int64)], b"",
                                   [(rows, k), (rows, k)], [np.float32, np.int64])
    np.testing.assert_array_equal(got_i, ref_i)
    np.testing.assert_array_equal(got_v.view(np.uint32), ref_v.view(np.uint32))


def _sampled_positions(n):
    """The elements the register TopK kernels sample for their threshold: thread t of 1024
    reads element (t mod chunks) * 1024 + t, chunks = n // 1024."""
    t = np.arange(1024)
    return (t % (n // 1024)) * 1024 + t


@pytest.mark.parametrize("rows,n,k,layout", [
    (16, 8400, 300, "uniform"), (2, 24000, 300, "uniform"), (1, 24000, 300, "sigmoid"),
    (1, 24000, 300, "descending"), (1, 24000, 300, "ascending"), (1, 24000, 300, "top_at_samples"),
    (1, 4096, 512, "uniform"), (2, 32768, 1, "uniform"), (1, 5000, 300, "sigmoid"),
    (1, 8192, 300, "top_off_samples")])
def test_topk_sampled_threshold(hip, torch_gpu, rows, n, k, layout):
    """Continuous values, where the register kernels take the sampled threshold (one count
    pass, then only the keys >= the sample's q-th largest are sorted), and layouts that defeat
    the sample: the row's largest values exactly at the sampled elements (too few keys pass,
    so the full selection runs) or everywhere else; sorted rows; k = 1 and k = 512."""
    print(f"[topk] sampled rows={rows} n={n} k={k} {layout}", flush=True)
    rng = np.random.default_rng(n + k + len(layout))
    if layout == "sigmoid":
        x = 1.0 / (1.0 + np.exp(-rng.normal(-6.0, 2.0, (rows, n))))
    elif layout in ("descending", "ascending"):
        x = np.sort(rng.uniform(0, 1, (rows, n)), axis=1)
        if layout == "descending":
            x = x[:, ::-1]
    else:
        x = rng.uniform(-1, 1, (rows, n))
        s = _sampled_positions(n)
        if layout == "top_at_samples":
            x[:, s] += 10.0
        elif layout == "top_off_samples":
            x += 10.0
            x[:, s] -= 10.0
    x = np.ascontiguousarray(x, dtype=np.float32)
    ref_v, ref_i = O.topk(x, k)
    got_v, got_i = device_postproc(hip, torch_gpu, "topk", [x, np.array([k], np.int64)], b"",
                                   [(rows, k), (rows, k)], [np.float32, np.int64])
    np.testing.assert_array_equal(got_i, ref_i)
    np.testing.assert_array_equal(got_v.view(np.uint32), ref_v.view(np.uint32))


@pytest.mark.parametrize("rows,block", [(8400, 80), (7, 80), (33, 16), (513, 48), (5, 256), (9, 20)],
                         ids=["b1_scores", "few_rows", "b16", "b48", "b256", "b20_one_lane"])
def test_reduce_max_short_rows(hip, torch_gpu, rows, block):
    """Rows of up to 256 floats: four lanes per row (blocks of a multiple of 16) or one,
    with ties everywhere (a 0.25 grid) and zeros of both signs, so the element kept must be
    the first maximal one, bit for bit as the reference's scan."""
    print(f"[reduce_max] rows={rows} block={block}", flush=True)
    rng = np.random.default_rng(rows + block)
    x = (np.round(rng.uniform(-1, 1, (rows, block)) * 4) / 4).astype(np.float32)
    x[x == 0] = np.where(rng.random(int((x == 0).sum())) < 0.5, -0.0, 0.0).astype(np.float32)
    got = device_postproc(hip, torch_gpu, "reduce_max", [x], b"", [(rows,)], [np.float32])[0]
    np.testing.assert_array_equal(got.view(np.uint32), O.reduce_max(x, rows).reshape(rows).view(np.uint32))


def test_reduce_gather_tile_detector_sizes(hip, torch_gpu):
    rng = np.random.default_rng(3)
    scores = np.round(rng.uniform(0, 1, (16, 8400, 80)), 3).astype(np.float32)
    got = device_postproc(hip, torch_gpu, "reduce_max", [scores], b"", [(16, 8400)], [np.float32])[0]
    np.testing.assert_array_equal(got.view(np.uint32), O.reduce_max(scores, 16 * 8400).reshape(16, 8400).view(np.uint32))
    idx = rng.integers(0, 8400, (16, 300, 1)).astype(np.int64)
    t = device_postproc(hip, torch_gpu, "tile", [idx], b"", [(16, 300, 80)], [np.int64])[0]
    np.testing.assert_array_equal(t, np.tile(idx, (1, 1, 80)))
    g = device_postproc(hip, torch_gpu, "gather", [scores, t], struct.pack("<ii", 1, 0), [(16, 300, 80)],
                        [np.float32])[0]
    np.testing.assert_array_equal(g, np.take_along_axis(scores, t, 1))


def test_postproc_bad_arguments(hip):
    L = hip.lib()
    one = C.c_void_p(16)
    assert L.spinn_hip_topk(1, 10, 11, one, one, one, None) == hip.SPINN_HIP_EINVAL        # k > n
    assert L.spinn_hip_topk(1, 4000, 1025, one, one, one, None) == hip.SPINN_HIP_EUNSUPPORTED
    assert L.spinn_hip_reduce_max(4, 0, one, one, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_cast(1, 11, 4, one, one, None) == hip.SPINN_HIP_EUNSUPPORTED       # to float64
    assert L.spinn_hip_binary_typed(hip.BINARY_MOD, 11, one, 1, one, 1, one, 1, None) == hip.SPINN_HIP_EUNSUPPORTED
    d = hip.GatherDesc()
    d.ndim, d.axis, d.index_dtype = 2, 1, 7
    d.in_dims[0], d.in_dims[1], d.out_dims[0], d.out_dims[1] = 2, 5, 3, 5                  # dim 0 past the data
    assert L.spinn_hip_gather_elements(C.byref(d), one, one, one, None) == hip.SPINN_HIP_EINVAL
    assert L.spinn_hip_tile(2, (C.c_int64 * 2)(0, 3), (C.c_int64 * 2)(2, 3), 4, one, one, None) == hip.SPINN_HIP_EINVAL


def _tail_numpy(pre, nc=80, max_det=300):
    """The exported tail on one image's decoded head [4 + nc, A] with the oracle's operators."""
    yt = np.ascontiguousarray(pre.T)
    boxes, scores = yt[:, :4], yt[:, 4:]
    best = O.reduce_max(scores, scores.shape[0])
    _, i1 = O.topk(best[None], max_det)
    i1 = i1[0]
    s1 = scores[i1]
    s2, i2 = O.topk(s1.reshape(1, -1), max_det)
    i2 = i2[0]
    lab = O.binary_typed("mod", i2, np.array([nc], np.int64), i2.shape)
    anc = O.binary_typed("div", i2, np.array([nc], np.int64), i2.shape)
    return np.concatenate([boxes[i1][anc], s2[0][:, None], lab[:, None].astype(np.float32)], 1)


@pytest.mark.parametrize("batch,hw", [(1, 640), (2, 320), (16, 640)])
def test_yolov10n_with_topk_tail(hip, tmp_path, batch, hw):
    """Whole detector incl. the TopK tail on the device; graph replay reproduces
    eager. The tail is checked bit for bit against the oracle's operators applied
    to the decoded head the device computes for the same model without the tail
    (the same kernels on the same inputs, so the same bits; the head tensor of
    the full model is recycled by the arena planner once the tail has read it)."""
    print(f"[yolov10n+tail] b{batch}@{hw}", flush=True)
    g, x = models.yolov10n(batch=batch, seed=7, hw=hw, postprocess=True)
    gp, xp = models.yolov10n(batch=batch, seed=7, hw=hw, postprocess=False)
    assert np.array_equal(x, xp)
    path = g.write(tmp_path / "y10post.ennf")
    pp = gp.write(tmp_path / "y10pre.ennf")
    with Session(path) as s:
        y = s.run(x)
    with Session(path, graph=True) as sg:
        yg = sg.run(x)
        yg2 = sg.run(x)
    with Session(pp) as sp:
        pre = sp.run(x)
    assert y.shape == (batch, 300, 6)
    assert np.array_equal(y, yg) and np.array_equal(yg, yg2)
    for b in range(batch):
        np.testing.assert_array_equal(y[b], _tail_numpy(pre[b]))
    if batch == 1:
        # and the decoded head is within tolerance of the oracle's
        ref_pre = O.Model(pp).run(x, gp.dims(gp.outputs[0]))
        assert_parity(pre, ref_pre, what="decoded head before the tail", scale_by_ref=True)
