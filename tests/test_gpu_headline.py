"""GPU parity at the full sizes of the headline workloads, against the oracle (the
restated SPINN CPU path: im2col + packed 6x16 GEMM + the specified epilogue,
SPINN/run_time/ops/conv/conv2d.c:92-232, SPINN/run_time/ops/mm/gemm_kernel.c:304-339):

* ResNet-101 v1.5 at batch 32 end to end under AUTO - the workload the benchmark's
  images/s is measured on, with its Winograd F(4x4,3x3) layers and split-K layers -
  eager and replayed from a HIP graph as the benchmark runs it;
* each of its 24 distinct conv layer shapes at batch 32 through spinn_hip_conv with
  one seeded input into both paths, held to the absolute bound (max-abs 1e-3,
  relative L2 1e-4);
* the VGG-style 3x3 stack at batch 8 (64@112 ... 512@14) under the implicit-GEMM,
  Winograd and AUTO policies.
"""
import ctypes as C
import zlib

import numpy as np
import pytest

from oracle import oracle as O
from spinn_amd import ennf as E
from spinn_amd import models
from spinn_amd import native as N
from spinn_amd.runtime import Session
from tests.conftest import assert_parity
from tests.hipops import conv_desc, run_conv

pytestmark = pytest.mark.gpu

# The 24 distinct conv layers of ResNet-101 v1.5 at 224x224:
# (c, h, w, oc, k, stride, pad, act, occurrences); tests/test_host.py checks this
# list against the generated model.
R101_LAYERS = [
    (3, 224, 224, 64, 7, 2, 3, 1, 1),
    (64, 56, 56, 64, 1, 1, 0, 1, 1),
    (64, 56, 56, 64, 3, 1, 1, 1, 3),
    (64, 56, 56, 256, 1, 1, 0, 0, 1),
    (64, 56, 56, 256, 1, 1, 0, 5, 3),
    (256, 56, 56, 64, 1, 1, 0, 1, 2),
    (256, 56, 56, 128, 1, 1, 0, 1, 1),
    (128, 56, 56, 128, 3, 2, 1, 1, 1),
    (256, 56, 56, 512, 1, 2, 0, 0, 1),
    (128, 28, 28, 512, 1, 1, 0, 5, 4),
    (512, 28, 28, 128, 1, 1, 0, 1, 3),
    (128, 28, 28, 128, 3, 1, 1, 1, 3),
    (512, 28, 28, 256, 1, 1, 0, 1, 1),
    (256, 28, 28, 256, 3, 2, 1, 1, 1),
    (512, 28, 28, 1024, 1, 2, 0, 0, 1),
    (256, 14, 14, 1024, 1, 1, 0, 5, 23),
    (1024, 14, 14, 256, 1, 1, 0, 1, 22),
    (256, 14, 14, 256, 3, 1, 1, 1, 22),
    (1024, 14, 14, 512, 1, 1, 0, 1, 1),
    (512, 14, 14, 512, 3, 2, 1, 1, 1),
    (1024, 14, 14, 2048, 1, 2, 0, 0, 1),
    (512, 7, 7, 2048, 1, 1, 0, 5, 3),
    (2048, 7, 7, 512, 1, 1, 0, 1, 2),
    (512, 7, 7, 512, 3, 1, 1, 1, 2),
]


def _layer_id(l):
    c, h, w, oc, k, s, p, act, _ = l
    return f"{c}x{h}x{w}-{oc}k{k}s{s}a{act}"


def _conv_algos(g):
    """(algo, K split?) AUTO picks for every conv node of an ENNF graph: an
    implicit GEMM that needs a workspace cuts some of its tiles along K (split-K
    partials, or the stream-K remainder tiles finished in the same launch)."""
    L = N.lib()
    out = []
    for nd in (n for n in g.nodes if n.op == E.OP_CONV):
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, _, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        d = N.ConvDesc(n, c, h, w, oc, oh, ow, kh, kw, p["strides"][0], p["strides"][1], p["pads"][0], p["pads"][1],
                       p["group"] or 1, p["act"], 0, 0)
        algo = L.spinn_hip_conv_select_algo(C.byref(d))
        d.algo = algo
        split = algo == N.ALGO_IMPLICIT_GEMM and L.spinn_hip_conv_workspace_size(C.byref(d)) > 0
        out.append((algo, split))
    return out


def test_resnet101_b32_end_to_end(hip, tmp_path):
    """The benchmark's workload: 104 convs (30 as F(4x4,3x3) Winograd, the implicit-GEMM
    layers whose tile grids do not divide evenly over the CUs with tiles cut along K),
    maxpool, global average pool and the 2048->1000 FC at batch 32; eager, then three
    graph replays bit-identical to it."""
    g, x = models.resnet101(batch=32, seed=21)
    algos = _conv_algos(g)
    n_f43 = sum(a == N.ALGO_WINOGRAD_F43 for a, _ in algos)
    n_split = sum(s for _, s in algos)
    print(f"[r101 b32] convs={len(algos)} f43={n_f43} k_split={n_split}", flush=True)
    assert len(algos) == 104 and n_f43 == 30 and n_split >= 4
    path = g.write(tmp_path / "r101b32.ennf")
    with Session(path) as s:
        y = s.run(x)
    with Session(path, graph=True) as s:
        replays = [s.run(x) for _ in range(3)]
    ref = O.Model(path).run(x, g.dims(g.outputs[0]))
    assert_parity(y, ref, what="resnet101 b32 (AUTO) vs oracle", scale_by_ref=True)
    for r in replays:
        assert np.array_equal(r, y)


@pytest.mark.parametrize("layer", R101_LAYERS, ids=[_layer_id(l) for l in R101_LAYERS])
def test_resnet101_b32_layer(hip, torch_gpu, layer):
    """One ResNet-101 conv layer at batch 32 under AUTO (the algorithm, tile and K split
    the benchmark runs) against the oracle's conv of the same seeded operands."""
    c, h, w, oc, k, s, p, act, _ = layer
    n = 32
    d = conv_desc(hip, n, c, h, w, oc, k, k, s, s, p, p, 1, act, 0)
    rng = np.random.default_rng(zlib.crc32(_layer_id(layer).encode()))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, k, k)) * np.sqrt(2.0 / (c * k * k))).astype(np.float32)
    b = rng.normal(0, 0.1, oc).astype(np.float32)
    r = rng.uniform(-1, 1, (n, oc, d.oh, d.ow)).astype(np.float32) if act in (4, 5) else None
    L = hip.lib()
    algo = L.spinn_hip_conv_select_algo(C.byref(d))
    d.algo = algo
    wsz = L.spinn_hip_conv_workspace_size(C.byref(d))
    d.algo = 0
    print(f"[r101 layer] {_layer_id(layer)} b32 algo={algo} workspace={wsz}", flush=True)
    y, used = run_conv(hip, torch_gpu, d, x, wt, b, r)
    ref = O.conv2d(O.conv_desc(n, c, h, w, oc, k, k, s, s, p, p, 1, act), x, wt, b, r)
    assert_parity(y, ref, what=f"{_layer_id(layer)} b32 (algo {used}) vs oracle")


@pytest.mark.parametrize("policy", [N.POLICY_IGEMM, N.POLICY_WINOGRAD, N.POLICY_AUTO],
                         ids=["igemm", "winograd", "auto"])
def test_vgg_stack_b8_full(hip, tmp_path, policy):
    """Eight Conv3x3+BN+ReLU layers at batch 8, 64@112 ... 512@14 with 2x2 max pools,
    under one conv policy, against the oracle's im2col convolution."""
    g, x = models.vgg_stack(batch=8, seed=11)
    path = g.write(tmp_path / "vgg8.ennf")
    with Session(path, policy=policy) as s:
        y = s.run(x)
    ref = O.Model(path).run(x, g.dims(g.outputs[0]))
    assert_parity(y, ref, what=f"vgg stack b8 policy {policy} vs oracle")
