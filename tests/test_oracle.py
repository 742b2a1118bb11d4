"""Pins the oracle (CPU restatement of the reference's conv/GEMM path).

Each check is chosen so that a plausible mistake in the restatement fails it:
  * the reference's own outputs on seeded inputs (golden fixtures written by
    tests/golden/make_golden.py from the reference's compiled C code):
    raw accumulator of the shipped group==1 path, grouped/depthwise convs with
    the full epilogue, the sgemm_nn epilogue for every act code, op_gemm,
    op_matmul, and the reference Winograd;
  * the reference's known-answer tests: the Winograd identity KAT
    (SPINN/run_time/test_winograd2.c:56-63) and the direct / im2col /
    Winograd agreement case of SPINN/run_time/test_winograd.c:64-75;
  * closed forms: float64 direct convolution and GEMM, and the float64
    library routine torch.nn.functional.conv2d (CPU);
  * the BN fold against BatchNorm applied after the convolution;
  * a whole ENNF model run by the oracle against a float64 torch
    interpretation of the same graph.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from spinn_amd import ennf as E
from spinn_amd import models
from tests.conftest import assert_parity, errors

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLD / name, allow_pickle=False)


# ---------------- golden fixtures from the reference ----------------

def test_conv_raw_accumulator_matches_reference():
    """group == 1: the reference's packed path returns the raw accumulator."""
    z = _load("conv_raw.npz")
    ids = sorted({k.split("_")[0] for k in z.files})
    assert ids
    for i in ids:
        n, c, h, w, oc, k, s, p, g, act = z[f"{i}_spec"].tolist()
        d = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
        r = z[f"{i}_r"] if f"{i}_r" in z.files else None
        y = O.conv2d(d, z[f"{i}_x"], z[f"{i}_w"], z[f"{i}_b"], r, as_shipped=True)
        ma, rel, _ = errors(y, z[f"{i}_y"])
        assert ma <= 1e-5 and rel <= 1e-6, (i, ma, rel)
        # and the specified epilogue really differs from the shipped output when it applies
        if act != 0:
            spec = O.conv2d(d, z[f"{i}_x"], z[f"{i}_w"], z[f"{i}_b"], r)
            assert np.abs(spec - z[f"{i}_y"]).max() > 1e-3


def test_conv_grouped_matches_reference():
    """group > 1: full epilogue (bias, residual, ReLU/SiLU) as the reference applies it."""
    z = _load("conv_grouped.npz")
    for i in sorted({k.split("_")[0] for k in z.files}):
        n, c, h, w, oc, k, s, p, g, act = z[f"{i}_spec"].tolist()
        d = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
        r = z[f"{i}_r"] if f"{i}_r" in z.files else None
        y = O.conv2d(d, z[f"{i}_x"], z[f"{i}_w"], z[f"{i}_b"], r)
        ma, rel, _ = errors(y, z[f"{i}_y"])
        assert ma <= 1e-5 and rel <= 1e-6, (i, ma, rel)


@pytest.mark.parametrize("act", [0, 1, 2, 3, 4, 5])
def test_epilogue_matches_reference(act):
    """sgemm_nn epilogue, every act code (CLIP=2 is declared but applies nothing)."""
    z = _load("epilogue.npz")
    a, b, bias, r = z["a"], z["b"], z["bias"], z["r"]
    m, k = a.shape
    n = b.shape[1]
    # the GEMM as a 1x1 convolution over a 1 x n image: W = a [m,k,1,1], X = b [1,k,1,n]
    d = O.conv_desc(1, k, 1, n, m, 1, 1, act=act)
    y = O.conv2d(d, np.ascontiguousarray(b.reshape(1, k, 1, n)), np.ascontiguousarray(a.reshape(m, k, 1, 1)), bias,
                 np.ascontiguousarray(r.reshape(1, m, 1, n)) if act in (4, 5) else None)
    ma, rel, _ = errors(y.reshape(m, n), z[f"y_act{act}"])
    assert ma <= 1e-5 and rel <= 1e-6, (ma, rel)
    # closed form of the specified order: v = acc + bias; ADD*: + R; RELU*: max0; SILU: v/(1+e^-v)
    v = a.astype(np.float64) @ b.astype(np.float64) + bias[:, None]
    if act in (4, 5):
        v = v + r
    if act in (1, 5):
        v = np.maximum(v, 0)
    elif act == 3:
        v = v / (1 + np.exp(-v))
    assert_parity(z[f"y_act{act}"], v, what="reference epilogue vs closed form")


def test_gemm_matches_reference():
    z = _load("gemm.npz")
    for i in sorted({k.split("_")[0] for k in z.files if k.startswith("g")}):
        m, n, k, ta, tb, cm = z[f"{i}_spec"].tolist()
        c = z[f"{i}_c"] if f"{i}_c" in z.files else None
        y = O.gemm(z[f"{i}_a"], z[f"{i}_b"], c, 1.0, 1.0, ta, tb)
        ma, rel, _ = errors(y, z[f"{i}_y"])
        assert ma <= 1e-5 and rel <= 1e-6, (i, ma, rel)
        assert_parity(y, O.gemm_f64(z[f"{i}_a"], z[f"{i}_b"], c, 1.0, 1.0, ta, tb), what="vs float64")
    y = O.matmul(z["mm_a"], z["mm_b"])
    assert np.abs(y - z["mm_y"]).max() <= 1e-5


def test_winograd_matches_reference_and_kat():
    z = _load("winograd.npz")
    # identity KAT: Y == X exactly (SPINN/run_time/test_winograd2.c:56-63)
    x, w = z["kat_x"], z["kat_w"]
    d = O.conv_desc(1, 1, 4, 4, 1, 3, 3, 1, 1, 1, 1, act=1)
    y = O.winograd(d, x, w)
    assert np.array_equal(y, x)
    assert np.array_equal(z["kat_y"], x)
    # seeded case with bias and ReLU against the reference's Winograd
    x, w, b = z["rand_x"], z["rand_w"], z["rand_b"]
    n, c, h, ww = x.shape
    d = O.conv_desc(n, c, h, ww, w.shape[0], 3, 3, 1, 1, 1, 1, act=1)
    y = O.winograd(d, x, w, b)
    ma, rel, _ = errors(y, z["rand_y"])
    assert ma <= 1e-5 and rel <= 1e-6
    assert_parity(y, O.conv2d_f64(d, x, w, b), what="winograd vs direct float64")


def test_winograd_direct_im2col_agree_reference_case():
    """SPINN/run_time/test_winograd.c:64-75: C=2, H=W=4, OC=3, X[i]=i+1,
    W[i]=(i%5-2)*0.5, bias {1,2,3}, pad 1; direct, im2col and Winograd agree."""
    x = (np.arange(2 * 16, dtype=np.float32) + 1).reshape(1, 2, 4, 4)
    w = (((np.arange(3 * 2 * 9) % 5) - 2) * 0.5).astype(np.float32).reshape(3, 2, 3, 3)
    b = np.array([1, 2, 3], np.float32)
    d = O.conv_desc(1, 2, 4, 4, 3, 3, 3, 1, 1, 1, 1)
    direct = O.conv2d_f64(d, x, w, b)
    assert np.abs(O.conv2d(d, x, w, b) - direct).max() < 1e-4
    assert np.abs(O.winograd(d, x, w, b) - direct).max() < 1e-4
    # exact integer-valued answer: the weights are multiples of 0.5 and X integral
    assert np.array_equal(np.round(direct * 2), direct * 2)


# ---------------- closed forms ----------------

CONV_SHAPES = [
    (2, 16, 12, 12, 24, 3, 1, 1, 1, 1),
    (1, 3, 21, 17, 10, 7, 2, 3, 1, 3),
    (2, 32, 9, 9, 40, 1, 2, 0, 1, 0),
    (1, 24, 10, 10, 24, 3, 2, 1, 24, 3),
    (1, 16, 8, 8, 32, 3, 1, 1, 4, 5),
    (3, 8, 5, 7, 6, 3, 1, 0, 1, 4),
]


@pytest.mark.parametrize("spec", CONV_SHAPES, ids=[str(s) for s in CONV_SHAPES])
def test_oracle_conv_vs_float64_and_torch(spec):
    import torch
    import torch.nn.functional as F
    n, c, h, w, oc, k, s, p, g, act = spec
    rng = np.random.default_rng(sum(spec))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = rng.normal(0, 0.4, (oc, c // g, k, k)).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    d = O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, g, act)
    r = rng.uniform(-1, 1, (n, oc, d.oh, d.ow)).astype(np.float32) if act in (4, 5) else None
    y = O.conv2d(d, x, wt, b, r)
    ref64 = O.conv2d_f64(d, x, wt, b, r)
    assert_parity(y, ref64, what="oracle vs float64 direct")
    t = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(wt).double(), torch.from_numpy(b).double(), s, p,
                 1, g)
    if r is not None:
        t = t + torch.from_numpy(r).double()
    if act in (1, 5):
        t = torch.relu(t)
    elif act == 3:
        t = t * torch.sigmoid(t)
    assert_parity(ref64, t.numpy(), rel_l2=1e-12, max_abs=1e-10, what="float64 direct vs torch float64")


def test_oracle_gemm_vs_float64():
    rng = np.random.default_rng(3)
    for (m, n, k) in models.GEMM_SWEEP[:2] + [(19, 23, 5)]:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
        c = rng.normal(0, 0.01, n).astype(np.float32)
        assert_parity(O.gemm(a, b, c, trans_b=1), a.astype(np.float64) @ b.T.astype(np.float64) + c)


def test_bn_fold_closed_form():
    """Conv with folded weights == BatchNorm(conv) (SPINN/graph_opt.c:181-198)."""
    rng = np.random.default_rng(11)
    oc, c = 8, 5
    w = models.kaiming(rng, oc, c, 3, 3)
    gamma, beta, mean, var = models.bn_params(rng, oc)
    w2, b2 = models.fold_bn(w, None, gamma, beta, mean, var)
    x = rng.uniform(-1, 1, (2, c, 7, 7)).astype(np.float32)
    d = O.conv_desc(2, c, 7, 7, oc, 3, 3, 1, 1, 1, 1)
    conv = O.conv2d_f64(d, x, w)
    bn = (conv - mean[None, :, None, None]) / np.sqrt(var.astype(np.float64) + 1e-5)[None, :, None, None] \
        * gamma[None, :, None, None] + beta[None, :, None, None]
    assert_parity(O.conv2d_f64(d, x, w2, b2), bn, max_abs=1e-5, rel_l2=1e-6)


# ---------------- unfused graph nodes ----------------

def _params_axis(prm, default):
    return int(np.frombuffer(prm[:4].tobytes(), np.int32)[0]) if prm.size >= 4 else default


def _oracle_tensor_op(name, ins, prm, out_shapes):
    """Run the oracle's restatement of the fixture's operator."""
    op = name.split("_")[0]
    if op in ("add", "sub", "mul", "div"):
        return [O.binary(op, ins[0], ins[1], out_shapes[0])]
    if op in ("relu", "sigmoid"):
        return [O.unary(op, ins[0])]
    if op == "batch":
        eps = float(np.frombuffer(prm[:4].tobytes(), np.float32)[0])
        return [O.batchnorm(*ins, eps=eps)]
    if op == "softmax":
        return [O.softmax(ins[0], _params_axis(prm, -1))]
    if op == "concat":
        return [O.concat(ins, _params_axis(prm, 0))]
    if op == "split":
        ax = _params_axis(prm, 0)
        return O.split(ins[0], [sh[ax] for sh in out_shapes], ax)
    if op == "transpose":
        nd = ins[0].ndim
        perm = list(prm[:nd]) if prm.size else list(range(nd))[::-1]
        return [O.transpose(ins[0], perm)]
    if op == "resize":
        return [O.resize_nearest(ins[0], *out_shapes[0][2:])]
    if op == "maxpool":
        return [O.maxpool(ins[0], *out_shapes[0][2:], 5, 5, 1, 1, 2, 2)]
    raise AssertionError(name)


def _tensor_op_cases():
    f = _load("tensor_ops.npz")
    names = sorted({k.rsplit("_", 1)[0] for k in f.files})
    for name in names:
        ins = [f[f"{name}_in{i}"] for i in range(8) if f"{name}_in{i}" in f.files]
        outs = [f[f"{name}_out{i}"] for i in range(8) if f"{name}_out{i}" in f.files]
        yield name, ins, f[f"{name}_params"], outs


# the reference vectorises exp (Cephes polynomial) and BatchNorm's FMA in blocks
# of 8, so those outputs agree to rounding; every other operator moves or
# combines values with one IEEE operation each and must agree bit for bit
_ROUNDED = {"sigmoid", "softmax_last", "softmax_short", "softmax_mid", "batch_norm"}


@pytest.mark.parametrize("case", list(_tensor_op_cases()), ids=lambda c: c[0])
def test_tensor_ops_match_reference(case):
    name, ins, prm, outs = case
    got = _oracle_tensor_op(name, ins, prm, [o.shape for o in outs])
    assert len(got) == len(outs)
    for g, ref in zip(got, outs):
        assert g.shape == ref.shape
        if name in _ROUNDED:
            np.testing.assert_allclose(g, ref, rtol=2e-6, atol=1e-7)
        else:
            np.testing.assert_array_equal(g, ref)


def test_tensor_ops_closed_forms():
    """The same operators against float64 numpy / torch definitions."""
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(5)
    x = rng.uniform(-3, 3, (2, 16, 4, 9)).astype(np.float32)
    xd = x.astype(np.float64)
    e = np.exp(xd - xd.max(1, keepdims=True))
    np.testing.assert_allclose(O.softmax(x, 1), e / e.sum(1, keepdims=True), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(O.unary("sigmoid", x), 1 / (1 + np.exp(-xd)), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(O.unary("silu", x), xd / (1 + np.exp(-xd)), rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(O.unary("relu", x), np.maximum(x, 0))
    sc, bi, mu, var = (rng.uniform(0.5, 1.5, 16).astype(np.float32) for _ in range(4))
    bn = F.batch_norm(torch.from_numpy(xd), torch.from_numpy(mu.astype(np.float64)),
                      torch.from_numpy(var.astype(np.float64)), torch.from_numpy(sc.astype(np.float64)),
                      torch.from_numpy(bi.astype(np.float64)), False, 0.0, 1e-5).numpy()
    np.testing.assert_allclose(O.batchnorm(x, sc, bi, mu, var, 1e-5), bn, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(O.transpose(x, (0, 2, 1, 3)), x.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(O.transpose(x, (3, 1, 0, 2)), x.transpose(3, 1, 0, 2))
    parts = O.split(x, [3, 5, 8], 1)
    np.testing.assert_array_equal(np.concatenate(parts, 1), x)
    np.testing.assert_array_equal(O.concat(parts[::-1], 1), np.concatenate(parts[::-1], 1))
    up = F.interpolate(torch.from_numpy(x), scale_factor=2, mode="nearest").numpy()
    np.testing.assert_array_equal(O.resize_nearest(x, 8, 18), up)
    b = rng.uniform(-1, 1, 9).astype(np.float32)
    np.testing.assert_array_equal(O.binary("sub", x, b, x.shape), x - b)
    np.testing.assert_array_equal(O.binary("mul", b, x, x.shape), b * x)
    np.testing.assert_array_equal(O.binary("div", x, b, x.shape), x / np.where(np.abs(b) < 1e-6, 1e-6, b))


# ---------------- whole model ----------------

def _torch_graph(g_path, x):
    """Interpret an ENNF file with float64 torch ops (independent of the oracle)."""
    import torch
    import torch.nn.functional as F
    m = E.read(g_path)
    vals = {m["inputs"][0]: torch.from_numpy(x).double()}
    W = {k: torch.from_numpy(np.array(v)).double() for k, v in m["weights"].items()}

    def v(t):
        return vals[t] if t in vals else W[t]

    for nd in m["nodes"]:
        ins = nd["inputs"]
        out_dims = m["tensors"][nd["outputs"][0]]["dims"]
        axis = int(np.frombuffer(nd["params"][:4], np.int32)[0]) if len(nd["params"]) >= 4 else None
        if nd["op"] == E.OP_CONV:
            p = E.unpack_conv_params(nd["params"])
            act = p["act"]
            has_res = act in (4, 5)
            nreal = len(ins) - (1 if has_res else 0)
            bias = W[ins[2]] if nreal > 2 else None
            y = F.conv2d(vals[ins[0]], W[ins[1]], bias, p["strides"][:2], p["pads"][:2], 1, p["group"])
            if has_res:
                y = y + vals[ins[-1]]
            if act in (1, 5):
                y = torch.relu(y)
            elif act == 3:
                y = y * torch.sigmoid(y)
        elif nd["op"] == E.OP_MAXPOOL:
            kh, kw = np.frombuffer(nd["params"][:4], np.uint16)
            sh, sw = np.frombuffer(nd["params"][8:12], np.uint16)
            ph, pw = np.frombuffer(nd["params"][16:20], np.uint16)
            y = F.max_pool2d(vals[ins[0]], (int(kh), int(kw)), (int(sh), int(sw)), (int(ph), int(pw)))
        elif nd["op"] == E.OP_REDUCEMEAN:
            y = vals[ins[0]].mean(dim=(2, 3), keepdim=True)
        elif nd["op"] == E.OP_RESHAPE:
            y = vals[ins[0]].reshape(out_dims)
        elif nd["op"] == E.OP_GEMM:
            y = vals[ins[0]] @ W[ins[1]].T + W[ins[2]]
        elif nd["op"] in (E.OP_ADD, E.OP_SUB, E.OP_MUL):
            a, b = v(ins[0]), v(ins[1])
            y = a + b if nd["op"] == E.OP_ADD else a - b if nd["op"] == E.OP_SUB else a * b
        elif nd["op"] == E.OP_SIGMOID:
            y = torch.sigmoid(vals[ins[0]])
        elif nd["op"] == E.OP_SOFTMAX:
            y = torch.softmax(vals[ins[0]], dim=axis)
        elif nd["op"] == E.OP_CONCAT:
            y = torch.cat([v(t) for t in ins], dim=axis)
        elif nd["op"] == E.OP_SPLIT:
            sizes = [m["tensors"][o]["dims"][axis] for o in nd["outputs"]]
            for o, part in zip(nd["outputs"], torch.split(vals[ins[0]], sizes, dim=axis)):
                vals[o] = part
            continue
        elif nd["op"] == E.OP_TRANSPOSE:
            nd_ = vals[ins[0]].dim()
            y = vals[ins[0]].permute(*list(nd["params"][:nd_]))
        elif nd["op"] == E.OP_MATMUL:
            y = vals[ins[0]] @ vals[ins[1]]
        elif nd["op"] == E.OP_RESIZE:
            y = F.interpolate(vals[ins[0]], size=out_dims[2:], mode="nearest")
        else:
            raise AssertionError(nd["op"])
        assert tuple(y.shape) == tuple(out_dims), (nd["op"], y.shape, out_dims)
        vals[nd["outputs"][0]] = y
    return vals[m["outputs"][0]].numpy()


def test_oracle_yolov10n_matches_torch_float64(tmp_path):
    """The detector graph (unfused Add / Split / Concat / Transpose / MatMul /
    Softmax / Resize / Sigmoid / Sub / Mul nodes around the fused convs) at
    256x256, batch 2: every node's output against float64 torch."""
    g, x = models.yolov10n(batch=2, seed=3, hw=256)
    path = g.write(tmp_path / "y10_256.ennf")
    y = O.Model(path).run(x, g.dims(g.outputs[0]))
    ref = _torch_graph(path, x)
    assert_parity(y, ref, what="oracle yolov10n vs torch float64", scale_by_ref=True)
    # boxes are pixel coordinates on the 8/16/32 strides grid, scores in (0, 1)
    assert y.shape == (2, 84, 32 * 32 + 16 * 16 + 8 * 8)
    assert np.all((y[:, 4:] > 0) & (y[:, 4:] < 1))


def test_oracle_model_matches_torch_float64(tmp_path):
    g, x = models.resnet(batch=2, seed=2, blocks=(1, 2, 1, 1), hw=64, num_classes=37)
    path = g.write(tmp_path / "tiny_resnet.ennf")
    y = O.Model(path).run(x, g.dims(g.outputs[0]))
    assert_parity(y, _torch_graph(path, x), what="oracle model vs torch float64", scale_by_ref=True)


@pytest.mark.parametrize("name", ["yolov10n_64", "resnet_64", "yolov10n_64_post"])
def test_oracle_model_as_shipped_matches_reference_runtime(name):
    """Whole models through the reference's own spinn_load / spinn_plan /
    spinn_run (tests/golden/models_as_shipped.npz): the oracle's model runner
    with the as-shipped switch (group==1 convs drop bias/act/residual, as
    SPINN/run_time/ops/mm/gemm_kernel.c:497-590 does) reproduces the
    reference's output, so node order, operand wiring and every unfused
    operator of the runner are pinned end to end."""
    import tempfile
    gen, kw = {"yolov10n_64": ("yolov10n", dict(batch=1, seed=5, hw=64)),
               "resnet_64": ("resnet", dict(batch=2, seed=6, blocks=(1, 1, 1, 1), hw=64, num_classes=10)),
               "yolov10n_64_post": ("yolov10n", dict(batch=1, seed=5, hw=64, postprocess=True))}[name]
    f = _load("models_as_shipped.npz")
    g, x = getattr(models, gen)(**kw)
    fp = f[f"{name}_x_sum"]
    assert np.isclose(x.astype(np.float64).sum(), fp[0]) and x.ravel()[0] == fp[1] and x.ravel()[-1] == fp[2]
    with tempfile.TemporaryDirectory() as td:
        m = O.Model(g.write(Path(td) / "m.ennf"))
        O.lib().oracle_set_as_shipped(1)
        try:
            y = m.run(x, g.dims(g.outputs[0]))
        finally:
            O.lib().oracle_set_as_shipped(0)
        m.close()
    ref = f[f"{name}_y"]
    assert_parity(y, ref, max_abs=1e-5, rel_l2=1e-6, what=f"{name} as-shipped vs reference spinn_run", scale_by_ref=True)


# ---------------------------------------------------------------------------
# Detector post-processing (the exported YOLOv10 tail): oracle vs the
# reference's own operators, bit for bit, and vs numpy closed forms.
# ---------------------------------------------------------------------------
def _postproc_cases():
    f = np.load(GOLD / "postproc.npz", allow_pickle=False)
    names = sorted({k.rsplit("_", 1)[0] for k in f.files})
    out = []
    for n in names:
        ins = [f[f"{n}_in{i}"] for i in range(8) if f"{n}_in{i}" in f.files]
        outs = [f[f"{n}_out{i}"] for i in range(8) if f"{n}_out{i}" in f.files]
        out.append((n, ins, f[f"{n}_params"].tobytes(), outs))
    return out


def oracle_postproc(name, ins, prm, outs):
    """Run the oracle function a fixture case exercises (shared with the GPU tests)."""
    import struct
    if name.startswith("reduce_max"):
        return [O.reduce_max(ins[0], outs[0].size).reshape(outs[0].shape)]
    if name.startswith("topk"):
        return list(O.topk(ins[0], int(ins[1][0])))
    if name.startswith("gather"):
        axis = struct.unpack("<i", prm[:4])[0]
        return [O.gather_elements(ins[0], ins[1], axis)]
    if name.startswith("tile"):
        return [O.tile(ins[0], outs[0].shape)]
    if name.startswith("cast"):
        return [O.cast(ins[0], outs[0].dtype)]
    if name.startswith("mod") or name.startswith("div"):
        op = "mod" if name.startswith("mod") else "div"
        return [O.binary_typed(op, ins[0], ins[1], outs[0].shape)]
    if name == "unsqueeze":
        return [ins[0].reshape(outs[0].shape).copy()]
    raise KeyError(name)


@pytest.mark.parametrize("case", _postproc_cases(), ids=lambda c: c[0])
def test_postproc_oracle_matches_reference(case):
    name, ins, prm, outs = case
    got = oracle_postproc(name, ins, prm, outs)
    assert len(got) == len(outs)
    for g, ref in zip(got, outs):
        assert g.shape == ref.shape and g.dtype == ref.dtype, (name, g.shape, ref.shape, g.dtype, ref.dtype)
        np.testing.assert_array_equal(g.view(np.uint8), ref.view(np.uint8))  # bit for bit, signed zeros included


def test_postproc_closed_forms():
    """TopK = stable descending argsort; GatherElements = take_along_axis; Tile,
    Cast, C-style integer Div / Mod and fmod against numpy."""
    rng = np.random.default_rng(11)
    x = np.round(rng.uniform(-1, 1, (3, 500)), 2).astype(np.float32)  # many ties
    v, i = O.topk(x, 120)
    ref_i = np.argsort(-x, axis=1, kind="stable")[:, :120]
    np.testing.assert_array_equal(i, ref_i)
    np.testing.assert_array_equal(v, np.take_along_axis(x, ref_i, 1))
    np.testing.assert_array_equal(O.reduce_max(x, 3), x.max(1))
    d = rng.uniform(-1, 1, (2, 9, 5)).astype(np.float32)
    ix = rng.integers(0, 9, (2, 4, 5)).astype(np.int64)
    np.testing.assert_array_equal(O.gather_elements(d, ix, 1), np.take_along_axis(d, ix, 1))
    np.testing.assert_array_equal(O.gather_elements(d, ix - 9, 1), np.take_along_axis(d, ix, 1))  # negative wrap
    t = rng.integers(0, 100, (1, 6, 1)).astype(np.int64)
    np.testing.assert_array_equal(O.tile(t, (2, 6, 80)), np.tile(t, (2, 1, 80)))
    a = rng.integers(-24000, 24000, 64).astype(np.int64)
    b = rng.integers(1, 90, 64).astype(np.int64) * rng.choice([-1, 1], 64)
    np.testing.assert_array_equal(O.binary_typed("div", a, b, (64,)), np.trunc(a / b).astype(np.int64))
    np.testing.assert_array_equal(O.binary_typed("mod", a, b, (64,)), np.fmod(a, b))
    fa = rng.uniform(-9, 9, 40).astype(np.float32)
    fb = rng.uniform(0.5, 3, 40).astype(np.float32)
    np.testing.assert_array_equal(O.binary_typed("mod", fa, fb, (40,)), np.fmod(fa, fb))
    np.testing.assert_array_equal(O.cast(a, np.float32), a.astype(np.float32))
    np.testing.assert_array_equal(O.cast(fa, np.int64), np.trunc(fa).astype(np.int64))
