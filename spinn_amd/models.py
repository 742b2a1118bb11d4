"""Seeded synthetic models for the benchmark configurations.

Every model is built the way an exporter leaves it (spinn_amd.onnx.OnnxGraph:
Conv, BatchNormalization, Relu, Add, Sigmoid, Mul, ... with value_info for
every intermediate) and converted to ENNF exactly as the reference converter
and graph optimizer do it (spinn_amd.onnx.convert; SPINN/onnx2ennf.c,
SPINN/graph_opt.c). The returned ENNF graph keeps its source as `g.onnx`, so
the same model can be written as an .onnx file and fed to the reference
converter. Weights are random-init, drawn from numpy's PCG64 generator with a
fixed seed so that the CPU and GPU paths see identical bytes:

  * conv weights: Kaiming normal, std = sqrt(2 / fan_in), fan_in = C/g*KH*KW;
  * BatchNorm: gamma ~ U(0.5,1.5), beta ~ N(0,0.1), mean ~ N(0,0.1),
    var ~ U(0.5,1.5), eps = 1e-5. ResNet and VGG carry BatchNormalization
    nodes, which the converter folds into the conv in float32
    (SPINN/graph_opt.c:181-198):
        f = gamma / sqrtf(var + eps);  W'[oc] = W[oc] * f;  b' = f * (b - mean) + beta.
    YOLOv10n is exported the way its framework exports it, with BN already
    folded into conv weight and bias by the same float32 formula (`fold_bn`).
"""
from __future__ import annotations

import numpy as np

from . import ennf as E
from . import onnx as X
from .onnx import ONNX_INT64, OnnxGraph

BN_EPS = np.float32(1e-5)


def fold_bn(w: np.ndarray, b: np.ndarray | None, gamma, beta, mean, var, eps=BN_EPS):
    """Conv+BN fold in float32 (SPINN/graph_opt.c:181-198)."""
    w = np.asarray(w, np.float32)
    oc = w.shape[0]
    f = (np.asarray(gamma, np.float32) / np.sqrt(np.asarray(var, np.float32) + np.float32(eps))).astype(np.float32)
    w2 = (w.reshape(oc, -1) * f[:, None]).astype(np.float32).reshape(w.shape)
    b_old = np.zeros(oc, np.float32) if b is None else np.asarray(b, np.float32)
    b2 = (f * (b_old - np.asarray(mean, np.float32)) + np.asarray(beta, np.float32)).astype(np.float32)
    return w2, b2


def bn_params(rng: np.random.Generator, oc: int):
    gamma = rng.uniform(0.5, 1.5, oc).astype(np.float32)
    beta = rng.normal(0.0, 0.1, oc).astype(np.float32)
    mean = rng.normal(0.0, 0.1, oc).astype(np.float32)
    var = rng.uniform(0.5, 1.5, oc).astype(np.float32)
    return gamma, beta, mean, var


def kaiming(rng: np.random.Generator, oc: int, cg: int, kh: int, kw: int) -> np.ndarray:
    std = np.sqrt(2.0 / (cg * kh * kw))
    return (rng.standard_normal((oc, cg, kh, kw)) * std).astype(np.float32)


def _out_hw(h, w, kh, kw, sh, sw, ph, pw):
    return (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


def add_conv_bn(g: OnnxGraph, rng, name: str, x: str, oc: int, k: int, stride: int = 1, pad: int = 0,
                group: int = 1, act: int = E.ACT_NONE, residual: str | None = None, bn: bool = True,
                bias: bool = False, fold: bool = False) -> str:
    """Append Conv [+ BatchNormalization] [+ its activation / residual nodes]; returns the last
    output. `act` names the post-op the converter will fuse: RELU -> Relu, SILU -> Sigmoid +
    Mul, ADD -> Add(residual, y), ADD_RELU -> Add(y, residual) + Relu. `fold` folds the BN at
    build time (an exporter that fuses BN itself) instead of emitting a BatchNormalization node."""
    n, c, h, w = g.dims(x)
    cg = c // group
    wt = kaiming(rng, oc, cg, k, k)
    b = rng.normal(0.0, 0.01, oc).astype(np.float32) if bias else None
    bnp = bn_params(rng, oc) if bn else None
    if bnp is not None and fold:
        wt, b = fold_bn(wt, b, *bnp)
        bnp = None
    oh, ow = _out_hw(h, w, k, k, stride, stride, pad, pad)
    ins = [x, g.weight(f"{name}.weight", wt)]
    if b is not None:
        ins.append(g.weight(f"{name}.bias", b))
    shape = (n, oc, oh, ow)
    y = g.value(f"{name}.conv", shape)
    g.node("Conv", ins, [y], dilations=[1, 1], group=group, kernel_shape=[k, k], pads=[pad] * 4,
           strides=[stride, stride])
    if bnp is not None:
        gamma, beta, mean, var = bnp
        prm = [g.weight(f"{name}.bn.{t}", v) for t, v in
               (("weight", gamma), ("bias", beta), ("running_mean", mean), ("running_var", var))]
        z = g.value(f"{name}.bn", shape)
        g.node("BatchNormalization", [y] + prm, [z], epsilon=float(BN_EPS), momentum=0.9)
        y = z
    if act == E.ACT_RELU:
        z = g.value(f"{name}.relu", shape)
        g.node("Relu", [y], [z])
        y = z
    elif act == E.ACT_SILU:
        sg = g.value(f"{name}.sigmoid", shape)
        g.node("Sigmoid", [y], [sg])
        z = g.value(f"{name}.silu", shape)
        g.node("Mul", [y, sg], [z])
        y = z
    elif act in (E.ACT_ADD, E.ACT_ADD_RELU):
        assert residual is not None
        z = g.value(f"{name}.add", shape)
        g.node("Add", [residual, y] if act == E.ACT_ADD else [y, residual], [z])
        y = z
        if act == E.ACT_ADD_RELU:
            z = g.value(f"{name}.relu", shape)
            g.node("Relu", [y], [z])
            y = z
    else:
        assert act == E.ACT_NONE and residual is None
    return y


def _convert(og: OnnxGraph) -> E.Graph:
    g = X.convert(og)
    g.onnx = og
    return g


def conv_bn_relu(seed: int = 0, n: int = 1, c: int = 64, hw: int = 56, oc: int = 64):
    """Single Conv3x3(s1,p1)+BN+ReLU (input 1x64x56x56 U[-1,1]), one fused Conv after conversion."""
    rng = np.random.default_rng(seed)
    g = OnnxGraph()
    x = g.input("x", (n, c, hw, hw))
    g.output(add_conv_bn(g, rng, "conv", x, oc, 3, 1, 1, act=E.ACT_RELU))
    xin = rng.uniform(-1.0, 1.0, (n, c, hw, hw)).astype(np.float32)
    return _convert(g), xin


GEMM_SWEEP = [(1, 1000, 2048), (32, 1000, 2048), (3136, 256, 64), (784, 512, 128), (196, 1024, 256)]


def gemm_model(m: int, n: int, k: int, seed: int = 0):
    """Y = A B^T + bias: A ~ U(-1,1) [M,K] (model input), B ~ N(0,1/K) [N,K], bias ~ N(0,0.01) [N]."""
    rng = np.random.default_rng(seed)
    g = OnnxGraph()
    a = g.input("A", (m, k))
    b = g.weight("B", (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    c = g.weight("bias", rng.normal(0.0, 0.01, n).astype(np.float32))
    y = g.value("Y", (m, n))
    g.node("Gemm", [a, b, c], [y], alpha=1.0, beta=1.0, transB=1)
    g.output(y)
    ain = rng.uniform(-1.0, 1.0, (m, k)).astype(np.float32)
    return _convert(g), ain


RESNET101_BLOCKS = (3, 4, 23, 3)
RESNET50_BLOCKS = (3, 4, 6, 3)


def resnet(batch: int = 1, seed: int = 0, blocks=RESNET101_BLOCKS, hw: int = 224, num_classes: int = 1000):
    """ResNet v1.5 (stride in the 3x3) with BatchNormalization nodes, converted.

    Block node order: conv1, conv2, downsample, conv3, Add, Relu. The residual
    Add+Relu fuses into whichever conv comes later in node order with its
    partner already computed (SPINN/graph_opt.c:350-374): conv3 for every
    block (the downsample conv of a stage's first block runs before it and
    carries no post-op). Tail: ReduceMean over (H,W) keepdims, Reshape to
    [B,2048], Gemm(transB=1) to the logits.
    """
    rng = np.random.default_rng(seed)
    g = OnnxGraph()
    x = g.input("input", (batch, 3, hw, hw))
    t = add_conv_bn(g, rng, "stem", x, 64, 7, 2, 3, act=E.ACT_RELU)
    n, c, h, w = g.dims(t)
    oh, ow = _out_hw(h, w, 3, 3, 2, 2, 1, 1)
    p = g.value("maxpool.out", (n, c, oh, ow))
    g.node("MaxPool", [t], [p], ceil_mode=0, kernel_shape=[3, 3], pads=[1, 1, 1, 1], strides=[2, 2])
    t = p
    for si, (nb, width) in enumerate(zip(blocks, (64, 128, 256, 512))):
        for bi in range(nb):
            stride = 2 if (bi == 0 and si > 0) else 1
            name = f"layer{si + 1}.{bi}"
            a = add_conv_bn(g, rng, f"{name}.conv1", t, width, 1, 1, 0, act=E.ACT_RELU)
            b = add_conv_bn(g, rng, f"{name}.conv2", a, width, 3, stride, 1, act=E.ACT_RELU)
            if bi == 0:
                ident = add_conv_bn(g, rng, f"{name}.downsample", t, width * 4, 1, stride, 0, act=E.ACT_NONE)
            else:
                ident = t
            t = add_conv_bn(g, rng, f"{name}.conv3", b, width * 4, 1, 1, 0, act=E.ACT_ADD_RELU, residual=ident)
    n, c, h, w = g.dims(t)
    m = g.value("mean.out", (n, c, 1, 1))
    g.node("ReduceMean", [t], [m], axes=[2, 3], keepdims=1)
    shape = g.weight("flatten.shape", np.array([n, c], np.int64))
    f = g.value("flatten.out", (n, c))
    g.node("Reshape", [m, shape], [f])
    fw = g.weight("fc.weight", (rng.standard_normal((num_classes, c)) / np.sqrt(c)).astype(np.float32))
    fb = g.weight("fc.bias", rng.normal(0.0, 0.01, num_classes).astype(np.float32))
    y = g.value("logits", (n, num_classes))
    g.node("Gemm", [f, fw, fb], [y], alpha=1.0, beta=1.0, transB=1)
    g.output(y)
    xin = np.random.default_rng(seed + 1).uniform(-1.0, 1.0, (batch, 3, hw, hw)).astype(np.float32)
    return _convert(g), xin


def resnet101(batch: int = 1, seed: int = 0):
    return resnet(batch, seed, RESNET101_BLOCKS)


VGG_SCHEDULE = [(64, 112), (64, 112), (128, 56), (128, 56), (256, 28), (256, 28), (512, 14), (512, 14)]


def vgg_stack(batch: int = 8, seed: int = 0, in_c: int = 64, schedule=VGG_SCHEDULE):
    """8 chained Conv3x3(s1,p1)+BN+ReLU, 2x2/2 MaxPool between resolutions."""
    rng = np.random.default_rng(seed)
    g = OnnxGraph()
    x = g.input("x", (batch, in_c, schedule[0][1], schedule[0][1]))
    t = x
    for i, (oc, res) in enumerate(schedule):
        n, c, h, w = g.dims(t)
        if h != res:
            assert h == 2 * res
            p = g.value(f"pool{i}.out", (n, c, res, res))
            g.node("MaxPool", [t], [p], ceil_mode=0, kernel_shape=[2, 2], pads=[0, 0, 0, 0], strides=[2, 2])
            t = p
        t = add_conv_bn(g, rng, f"conv{i}", t, oc, 3, 1, 1, act=E.ACT_RELU)
    g.output(t)
    xin = np.random.default_rng(seed + 1).uniform(-1.0, 1.0, g.dims(x)).astype(np.float32)
    return _convert(g), xin


def _plain_conv(g: OnnxGraph, rng, name: str, x: str, oc: int, k: int = 1, bias: bool = True,
                weight: np.ndarray | None = None) -> str:
    """A bare nn.Conv2d (no BatchNorm, no activation) with PyTorch's default
    init: weight and bias ~ U(-1/sqrt(fan_in), 1/sqrt(fan_in))."""
    n, c, h, w = g.dims(x)
    bound = 1.0 / np.sqrt(c * k * k)
    if weight is None:
        weight = rng.uniform(-bound, bound, (oc, c, k, k)).astype(np.float32)
    ins = [x, g.weight(f"{name}.weight", weight)]
    if bias:
        ins.append(g.weight(f"{name}.bias", rng.uniform(-bound, bound, oc).astype(np.float32)))
    oh, ow = _out_hw(h, w, k, k, 1, 1, k // 2, k // 2)
    y = g.value(f"{name}.out", (n, oc, oh, ow))
    g.node("Conv", ins, [y], dilations=[1, 1], group=1, kernel_shape=[k, k], pads=[k // 2] * 4, strides=[1, 1])
    return y


def yolov10n(batch: int = 1, seed: int = 0, hw: int = 640, nc: int = 80, postprocess: bool = False,
             max_det: int = 300):
    """YOLOv10n (width 0.25, depth 0.33; ultralytics yolov10n.yaml) as the
    exporter leaves the detector, converted, up to the
    one-to-one head's decoded output [B, 4 + nc, anchors] (boxes x1y1x2y2 in
    pixels, class scores after Sigmoid), i.e. before the TopK post-processing.

    BN is folded into every conv at export (conv weight and bias); each
    Conv-BN-SiLU is Conv -> Sigmoid -> Mul, which the converter fuses into one
    Conv with act SILU (SPINN/graph_opt.c:431-496); convs built with act=False
    carry no post-op, except where their single consumer is an Add whose other
    operand already exists - the PSA block's pe, proj and ffn.1 convs - which
    fuse it as act ADD (SPINN/graph_opt.c:304-421). The Bottleneck / CIB
    shortcut Adds follow a SiLU conv and stay unfused Add nodes. Node order is
    the export's execution order.
    """
    rng = np.random.default_rng(seed)
    g = OnnxGraph()
    x = g.input("images", (batch, 3, hw, hw))
    uid = [0]

    def nm(s):
        uid[0] += 1
        return f"{s}#{uid[0]}"

    def conv(name, t, oc, k=1, s=1, group=1, act=E.ACT_SILU, residual=None):
        return add_conv_bn(g, rng, name, t, oc, k, s, k // 2, group, act, residual, fold=True)

    def split(name, t, sizes, axis=1):
        dims = g.dims(t)
        outs = []
        for i, sz in enumerate(sizes):
            d = list(dims)
            d[axis] = sz
            outs.append(g.value(f"{name}.out{i}", tuple(d)))
        sw = g.weight(nm(f"{name}.split"), np.array(sizes, np.int64))
        g.node("Split", [t, sw], outs, axis=axis)
        return outs

    def concat(name, ts, axis=1):
        d = list(g.dims(ts[0]))
        d[axis] = sum(g.dims(t)[axis] for t in ts)
        y = g.value(f"{name}.out", tuple(d))
        g.node("Concat", ts, [y], axis=axis)
        return y

    def binary(op, name, a, b):
        da, db = g.dims(a), g.dims(b)
        y = g.value(f"{name}.out", da if int(np.prod(da)) >= int(np.prod(db)) else db)
        g.node(op, [a, b], [y])
        return y

    def reshape(name, t, dims):
        sw = g.weight(nm(f"{name}.shape"), np.array(dims, np.int64))
        y = g.value(f"{name}.out", tuple(dims))
        g.node("Reshape", [t, sw], [y])
        return y

    def transpose(name, t, perm):
        d = g.dims(t)
        y = g.value(f"{name}.out", tuple(d[p] for p in perm))
        g.node("Transpose", [t], [y], perm=list(perm))
        return y

    def c2f(name, t, c2, n, shortcut):
        c = c2 // 2
        y = split(f"{name}.split", conv(f"{name}.cv1", t, 2 * c), [c, c])
        for i in range(n):
            a = conv(f"{name}.m.{i}.cv1", y[-1], c, 3)
            b = conv(f"{name}.m.{i}.cv2", a, c, 3)
            y.append(binary("Add", f"{name}.m.{i}.add", y[-1], b) if shortcut else b)
        return conv(f"{name}.cv2", concat(f"{name}.cat", y), c2)

    def scdown(name, t, c2):
        return conv(f"{name}.cv2", conv(f"{name}.cv1", t, c2), c2, 3, 2, group=c2, act=E.ACT_NONE)

    def sppf(name, t, c2):
        n_, c1, h, w = g.dims(t)
        y = [conv(f"{name}.cv1", t, c1 // 2)]
        for i in range(3):
            p = g.value(f"{name}.m{i}.out", g.dims(y[-1]))
            g.node("MaxPool", [y[-1]], [p], ceil_mode=0, kernel_shape=[5, 5], pads=[2, 2, 2, 2], strides=[1, 1])
            y.append(p)
        return conv(f"{name}.cv2", concat(f"{name}.cat", y), c2)

    def psa(name, t):
        n_, c1, h, w = g.dims(t)
        c = c1 // 2
        heads, key_dim, head_dim = c // 64, 32, 64
        a, b = split(f"{name}.split", conv(f"{name}.cv1", t, 2 * c), [c, c])
        qkv = conv(f"{name}.attn.qkv", b, c + 2 * heads * key_dim, act=E.ACT_NONE)
        qkv = reshape(f"{name}.attn.view", qkv, (n_, heads, 2 * key_dim + head_dim, h * w))
        q, k, v = split(f"{name}.attn.split", qkv, [key_dim, key_dim, head_dim], axis=2)
        qt = transpose(f"{name}.attn.qT", q, (0, 1, 3, 2))
        s = g.value(f"{name}.attn.scores", (n_, heads, h * w, h * w))
        g.node("MatMul", [qt, k], [s])
        scale = g.weight(nm(f"{name}.attn.scale"), np.array(key_dim ** -0.5, np.float32))
        s = binary("Mul", f"{name}.attn.scaled", s, scale)
        p = g.value(f"{name}.attn.softmax", g.dims(s))
        g.node("Softmax", [s], [p], axis=-1)
        pt = transpose(f"{name}.attn.pT", p, (0, 1, 3, 2))
        o = g.value(f"{name}.attn.av", (n_, heads, head_dim, h * w))
        g.node("MatMul", [v, pt], [o])
        o = reshape(f"{name}.attn.view2", o, (n_, c, h, w))
        vv = reshape(f"{name}.attn.v", v, (n_, c, h, w))
        x2 = conv(f"{name}.attn.pe", vv, c, 3, group=c, act=E.ACT_ADD, residual=o)
        b = conv(f"{name}.attn.proj", x2, c, act=E.ACT_ADD, residual=b)
        f = conv(f"{name}.ffn.0", b, 2 * c)
        b = conv(f"{name}.ffn.1", f, c, act=E.ACT_ADD, residual=b)
        return conv(f"{name}.cv2", concat(f"{name}.cat", [a, b]), c1)

    def c2fcib(name, t, c2):
        c = c2 // 2
        y = split(f"{name}.split", conv(f"{name}.cv1", t, 2 * c), [c, c])
        m = conv(f"{name}.m.0.cv1.0", y[-1], c, 3, group=c)
        m = conv(f"{name}.m.0.cv1.1", m, 2 * c)
        m = conv(f"{name}.m.0.cv1.2", m, 2 * c, 7, group=2 * c)  # RepVGGDW, 3x3 branch merged at export
        m = conv(f"{name}.m.0.cv1.3", m, c)
        m = conv(f"{name}.m.0.cv1.4", m, c, 3, group=c)
        y.append(binary("Add", f"{name}.m.0.add", y[-1], m))
        return conv(f"{name}.cv2", concat(f"{name}.cat", y), c2)

    def upsample(name, t):
        n_, c, h, w = g.dims(t)
        sc = g.weight(nm(f"{name}.scales"), np.array([1, 1, 2, 2], np.float32))
        y = g.value(f"{name}.out", (n_, c, 2 * h, 2 * w))
        g.node("Resize", [t, "", sc], [y], coordinate_transformation_mode="asymmetric", mode="nearest",
               nearest_mode="floor")
        return y

    # backbone
    t = conv("model.0", x, 16, 3, 2)
    t = conv("model.1", t, 32, 3, 2)
    t = c2f("model.2", t, 32, 1, True)
    t = conv("model.3", t, 64, 3, 2)
    p3 = c2f("model.4", t, 64, 2, True)
    t = scdown("model.5", p3, 128)
    p4 = c2f("model.6", t, 128, 2, True)
    t = scdown("model.7", p4, 256)
    t = c2f("model.8", t, 256, 1, True)
    t = sppf("model.9", t, 256)
    p5 = psa("model.10", t)
    # neck
    t = concat("model.12", [upsample("model.11", p5), p4])
    h13 = c2f("model.13", t, 128, 1, False)
    t = concat("model.15", [upsample("model.14", h13), p3])
    o3 = c2f("model.16", t, 64, 1, False)
    t = concat("model.18", [conv("model.17", o3, 64, 3, 2), h13])
    o4 = c2f("model.19", t, 128, 1, False)
    t = concat("model.21", [scdown("model.20", o4, 128), p5])
    o5 = c2fcib("model.22", t, 256)
    # one-to-one v10Detect head
    reg_max, c2h, c3h = 16, 64, max(64, min(nc, 100))
    levels = []
    for i, (f, stride) in enumerate(zip((o3, o4, o5), (8, 16, 32))):
        pre = f"model.23.one2one_cv"
        n_, ch, h, w = g.dims(f)
        bx = conv(f"{pre}2.{i}.0", f, c2h, 3)
        bx = conv(f"{pre}2.{i}.1", bx, c2h, 3)
        bx = _plain_conv(g, rng, f"{pre}2.{i}.2", bx, 4 * reg_max)
        cl = conv(f"{pre}3.{i}.0.0", f, ch, 3, group=ch)
        cl = conv(f"{pre}3.{i}.0.1", cl, c3h)
        cl = conv(f"{pre}3.{i}.1.0", cl, c3h, 3, group=c3h)
        cl = conv(f"{pre}3.{i}.1.1", cl, c3h)
        cl = _plain_conv(g, rng, f"{pre}3.{i}.2", cl, nc)
        lv = concat(f"model.23.cat{i}", [bx, cl])
        levels.append((reshape(f"model.23.view{i}", lv, (n_, 4 * reg_max + nc, h * w)), h, w, stride))
    xcat = concat("model.23.cat", [lv for lv, _, _, _ in levels], axis=2)
    na = g.dims(xcat)[2]
    box, cls = split("model.23.split", xcat, [4 * reg_max, nc])
    sig = g.value("model.23.sigmoid.out", g.dims(cls))
    g.node("Sigmoid", [cls], [sig])
    d = reshape("model.23.dfl.view", box, (batch, 4, reg_max, na))
    d = transpose("model.23.dfl.t", d, (0, 2, 1, 3))
    sm = g.value("model.23.dfl.softmax", g.dims(d))
    g.node("Softmax", [d], [sm], axis=1)
    dist = _plain_conv(g, rng, "model.23.dfl.conv", sm, 1, bias=False,
                       weight=np.arange(reg_max, dtype=np.float32).reshape(1, reg_max, 1, 1))
    dist = reshape("model.23.dfl.view2", dist, (batch, 4, na))
    lt, rb = split("model.23.chunk", dist, [2, 2])
    ax, ay, st = [], [], []
    for _, h, w, stride in levels:
        gy, gx = np.meshgrid(np.arange(h, dtype=np.float32) + 0.5, np.arange(w, dtype=np.float32) + 0.5,
                             indexing="ij")
        ax.append(gx.ravel())
        ay.append(gy.ravel())
        st.append(np.full(h * w, stride, np.float32))
    anchors = g.weight("model.23.anchors", np.stack([np.concatenate(ax), np.concatenate(ay)])[None].astype(np.float32))
    strides = g.weight("model.23.strides", np.concatenate(st)[None].astype(np.float32))
    x1y1 = binary("Sub", "model.23.x1y1", anchors, lt)
    x2y2 = binary("Add", "model.23.x2y2", anchors, rb)
    dbox = binary("Mul", "model.23.dbox", concat("model.23.xyxy", [x1y1, x2y2]), strides)
    y = concat("model.23.out", [dbox, sig])
    if postprocess:
        y = _v10_postprocess(g, y, batch, na, nc, max_det, nm, split, transpose, concat)
    g.output(y)
    xin = np.random.default_rng(seed + 1).uniform(0.0, 1.0, (batch, 3, hw, hw)).astype(np.float32)
    return _convert(g), xin


def _v10_postprocess(g: OnnxGraph, y: str, batch: int, na: int, nc: int, max_det: int, nm, split, transpose,
                     concat) -> str:
    """The exported one-to-one post-process after the decoded head [B, 4 + nc, A]:
    per-anchor best score, TopK anchors, gather of their boxes and class scores,
    TopK over anchor x class, label = index mod nc, anchor = index / nc, final
    box gather; output [B, k, 6] = (x1, y1, x2, y2, score, label). The node
    sequence is the one the ONNX export carries (Transpose, Split, ReduceMax, TopK,
    Unsqueeze, Tile, GatherElements, Flatten, TopK, Mod, Div, Cast, Concat)."""
    i64 = ONNX_INT64
    pre = "model.23.post"
    yt = transpose(f"{pre}.t", y, (0, 2, 1))                       # [B, A, 4 + nc]
    boxes, scores = split(f"{pre}.split", yt, [4, nc], axis=2)
    best = g.value(f"{pre}.max", (batch, na))
    g.node("ReduceMax", [scores], [best], axes=[-1], keepdims=0)
    k1 = min(max_det, na)
    kt = g.weight(nm(f"{pre}.k"), np.array([max_det], np.int64))

    def topk(name, t, k):
        v = g.value(f"{name}.values", g.dims(t)[:-1] + (k,))
        ix = g.value(f"{name}.indices", g.dims(t)[:-1] + (k,), i64)
        g.node("TopK", [t, kt], [v, ix], axis=-1, largest=1, sorted=1)
        return v, ix

    def unsqueeze(name, t):
        u = g.value(f"{name}.out", g.dims(t) + (1,), g.elem_type(t))
        g.node("Unsqueeze", [t, g.weight(nm(f"{name}.axes"), np.array([-1], np.int64))], [u])
        return u

    def tile(name, t, reps):
        d = g.dims(t)
        u = g.value(f"{name}.out", tuple(a * r for a, r in zip(d, reps)), g.elem_type(t))
        g.node("Tile", [t, g.weight(nm(f"{name}.repeats"), np.array(reps, np.int64))], [u])
        return u

    def gather(name, data, idx):
        u = g.value(f"{name}.out", g.dims(idx))
        g.node("GatherElements", [data, idx], [u], axis=1)
        return u

    def int_op(op, name, t, divisor):
        u = g.value(f"{name}.out", g.dims(t), i64)
        g.node(op, [t, divisor], [u], **({"fmod": 0} if op == "Mod" else {}))
        return u

    _, i1 = topk(f"{pre}.topk0", best, k1)
    i1u = unsqueeze(f"{pre}.unsq0", i1)
    boxes1 = gather(f"{pre}.gather0", boxes, tile(f"{pre}.tile0", i1u, (1, 1, 4)))
    scores1 = gather(f"{pre}.gather1", scores, tile(f"{pre}.tile1", i1u, (1, 1, nc)))
    flat = g.value(f"{pre}.flat", (batch, k1 * nc))
    g.node("Flatten", [scores1], [flat], axis=1)
    k2 = min(max_det, k1 * nc)
    s2, i2 = topk(f"{pre}.topk1", flat, k2)
    ncw = g.weight(nm(f"{pre}.nc"), np.array(nc, np.int64))
    labels = int_op("Mod", f"{pre}.mod", i2, ncw)
    anchor = int_op("Div", f"{pre}.div", i2, ncw)
    lab = unsqueeze(f"{pre}.unsq1", labels)
    labf = g.value(f"{pre}.cast.out", g.dims(lab))
    g.node("Cast", [lab], [labf], to=1)
    boxes2 = gather(f"{pre}.gather2", boxes1, tile(f"{pre}.tile2", unsqueeze(f"{pre}.unsq2", anchor), (1, 1, 4)))
    return concat(f"{pre}.out", [boxes2, unsqueeze(f"{pre}.unsq3", s2), labf], axis=2)


def conv_flops(g: E.Graph) -> list:
    """Per-Conv-node direct-convolution FLOPs 2*N*OC*OH*OW*(C/g)*KH*KW (node index, flops)."""
    out = []
    for i, nd in enumerate(g.nodes):
        if nd.op != E.OP_CONV:
            continue
        p = E.unpack_conv_params(nd.params)
        n, c, h, w = g.dims(nd.inputs[0])
        oc, cg, kh, kw = g.dims(nd.inputs[1])
        _, _, oh, ow = g.dims(nd.outputs[0])
        out.append((i, 2.0 * n * oc * oh * ow * cg * kh * kw))
    return out
