"""ENNF model files: a graph builder/writer and a reader.

The writer lays a file out the way the reference converter does
(SPINN/onnx2ennf.c:258-518):

    [ENNF_Header 64 B]
    [dense ENNF_WeightEntry table, one 16 B entry per tensor id]   <- header.reserved[0]
    [graph meta: u16 n_in, u16 in_ids[], u16 n_out, u16 out_ids[]]
    [node table: ENNF_NodeBase, u16 input_ids[], u16 output_ids[], params]
    [ENNF_TensorMeta table, 44 B per tensor]
    [zero padding to 16 B]
    [weight blob, tensors back to back in id order]                 <- header.weight_data_offset

A `Graph` here is the converted, post-fusion graph (spinn_amd.onnx.convert
builds it from an exporter-shaped graph as the reference converter does): BN
folded into the conv weights and bias, the fused post-op code in
ENNF_ConvParams.reserved, the residual appended as the conv's last input,
ENNF_NODE_FLAG_FUSED on convs that carry an activation or residual, and the
reference counts of the graph before fusion (onnx2ennf.c:232-241) in
`ref_counts`; without them the writer counts the node inputs naming each
tensor.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

ENNF_MAGIC = 0x454E4E46
DT_FLOAT32, DT_INT32, DT_INT64 = 1, 6, 7
_NP_DTYPE = {DT_FLOAT32: np.float32, DT_INT32: np.int32, DT_INT64: np.int64}

# op ids (SPINN/ennf_op_types.h numeric values)
OP_ADD, OP_DIV, OP_MUL, OP_SUB = 4, 23, 39, 50
OP_CONV, OP_AVGPOOL, OP_GAP, OP_MAXPOOL = 60, 80, 81, 85
OP_BN, OP_RELU, OP_SIGMOID, OP_SOFTMAX = 100, 130, 133, 134
OP_GEMM, OP_MATMUL = 160, 161
OP_CONCAT, OP_FLATTEN, OP_IDENTITY, OP_RESHAPE = 183, 189, 193, 197
OP_RESIZE, OP_SPLIT, OP_TRANSPOSE, OP_REDUCEMEAN = 198, 206, 211, 235
OP_MOD, OP_CAST, OP_GATHER_ELEMENTS, OP_TILE, OP_TOPK, OP_UNSQUEEZE, OP_REDUCEMAX = 38, 180, 191, 209, 210, 214, 234

ACT_NONE, ACT_RELU, ACT_CLIP, ACT_SILU, ACT_ADD, ACT_ADD_RELU = 0, 1, 2, 3, 4, 5
NODE_FLAG_FUSED = 1

_HDR = struct.Struct("<IHHIIIIHHHHIIIII3I")
_NODE = struct.Struct("<HBBHBB")
_META = struct.Struct("<HBB8IIBB2x")
_ENTRY = struct.Struct("<HHIII")
assert _HDR.size == 64 and _NODE.size == 8 and _META.size == 44 and _ENTRY.size == 16


def conv_params(kh: int, kw: int, sh: int = 1, sw: int = 1, pads=(0, 0, 0, 0), group: int = 1,
                act: int = ACT_NONE, dilations=(1, 1), auto_pad: int = 0) -> bytes:
    """ENNF_ConvParams (44 B); pads in ONNX order (h_begin, w_begin, h_end, w_end)."""
    p8 = list(pads) + [0] * (8 - len(pads))
    return struct.pack("<4H4H8H4HHBB", kh, kw, 0, 0, sh, sw, 0, 0, *p8, dilations[0], dilations[1], 0, 0,
                       group, auto_pad, act)


def pool_params(kh: int, kw: int, sh: int, sw: int, pads=(0, 0, 0, 0)) -> bytes:
    """ENNF_PoolParams (48 B)."""
    p8 = list(pads) + [0] * (8 - len(pads))
    return struct.pack("<4H4H8H4HBBBBi", kh, kw, 0, 0, sh, sw, 0, 0, *p8, 1, 1, 0, 0, 0, 0, 0, 0, 0)


def gemm_params(alpha: float = 1.0, beta: float = 1.0, trans_a: int = 0, trans_b: int = 0) -> bytes:
    """ENNF_GemmParams (12 B)."""
    return struct.pack("<ffBB2x", alpha, beta, trans_a, trans_b)


def axis_params(axis: int) -> bytes:
    """ENNF_SoftmaxParams / ENNF_ConcatParams / ENNF_FlattenParams (4 B)."""
    return struct.pack("<i", axis)


def split_params(axis: int, num_outputs: int) -> bytes:
    """ENNF_SplitParams (8 B); the piece sizes travel as the int64 second input."""
    return struct.pack("<iI", axis, num_outputs)


def transpose_params(perm) -> bytes:
    """ENNF_TransposeParams (12 B): perm[8], num_dims, 3 reserved."""
    p = list(perm) + [0] * (8 - len(perm))
    return struct.pack("<8BB3x", *p, len(perm))


def batchnorm_params(eps: float = 1e-5, momentum: float = 0.9) -> bytes:
    """ENNF_BatchNormParams (12 B)."""
    return struct.pack("<ffB3x", eps, momentum, 0)


def reduce_params(axes, keepdims: int = 1) -> bytes:
    """ENNF_ReduceParams (36 B)."""
    a = list(axes) + [0] * (8 - len(axes))
    return struct.pack("<8iBBBB", *a, len(axes), keepdims, 0, 0)


def topk_params(axis: int = -1, largest: int = 1, sorted_: int = 1) -> bytes:
    """ENNF_TopKParams (8 B); K travels as the int64 second input."""
    return struct.pack("<iBB2x", axis, largest, sorted_)


def gather_params(axis: int) -> bytes:
    """ENNF_GatherParams (8 B): axis, batch_dims."""
    return struct.pack("<ii", axis, 0)


def cast_params(to_type: int) -> bytes:
    """ENNF_CastParams (4 B)."""
    return struct.pack("<BB2x", to_type, 0)


@dataclass
class Tensor:
    id: int
    name: str
    dims: tuple
    dtype: int = DT_FLOAT32
    data: np.ndarray | None = None

    @property
    def is_weight(self) -> bool:
        return self.data is not None

    @property
    def elem_count(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n


@dataclass
class Node:
    op: int
    inputs: list
    outputs: list
    params: bytes = b""
    flags: int = 0


@dataclass
class Graph:
    tensors: list = field(default_factory=list)
    nodes: list = field(default_factory=list)
    inputs: list = field(default_factory=list)
    outputs: list = field(default_factory=list)
    opset: int = 17
    ref_counts: list | None = None   # per tensor id; None: count the node inputs naming each tensor
    flags: int = 0                   # ENNF_Header.flags

    def tensor(self, name: str, dims, dtype: int = DT_FLOAT32, data: np.ndarray | None = None) -> int:
        if data is not None:
            data = np.ascontiguousarray(data, dtype=_NP_DTYPE[dtype])
            if len(dims) == 0 and data.size == 1:
                data = data.reshape(())  # ONNX scalar initializer: ndim 0, one element
            assert tuple(data.shape) == tuple(dims), (name, data.shape, dims)
        t = Tensor(len(self.tensors), name, tuple(int(d) for d in dims), dtype, data)
        self.tensors.append(t)
        return t.id

    def weight(self, name: str, data: np.ndarray, dtype: int = DT_FLOAT32) -> int:
        return self.tensor(name, data.shape, dtype, data)

    def input(self, name: str, dims) -> int:
        tid = self.tensor(name, dims)
        self.inputs.append(tid)
        return tid

    def output(self, tid: int) -> None:
        self.outputs.append(tid)

    def node(self, op: int, inputs, outputs, params: bytes = b"", flags: int = 0) -> None:
        self.nodes.append(Node(op, list(inputs), list(outputs), params, flags))

    def dims(self, tid: int) -> tuple:
        return self.tensors[tid].dims

    # ---- serialisation ----
    def to_bytes(self) -> bytes:
        ref = self.ref_counts
        if ref is None:
            ref = [0] * len(self.tensors)
            for n in self.nodes:
                for i in n.inputs:
                    ref[i] += 1
        nt = len(self.tensors)
        entry_off = _HDR.size
        graph_meta_off = entry_off + nt * _ENTRY.size
        gm = struct.pack("<H", len(self.inputs)) + b"".join(struct.pack("<H", i) for i in self.inputs)
        gm += struct.pack("<H", len(self.outputs)) + b"".join(struct.pack("<H", i) for i in self.outputs)
        node_off = graph_meta_off + len(gm)
        nb = bytearray()
        for n in self.nodes:
            nb += _NODE.pack(n.op, len(n.inputs), len(n.outputs), len(n.params), n.flags, 0)
            nb += b"".join(struct.pack("<H", i) for i in n.inputs)
            nb += b"".join(struct.pack("<H", i) for i in n.outputs)
            nb += n.params
        meta_off = node_off + len(nb)
        mb = bytearray()
        for t in self.tensors:
            dims = list(t.dims) + [0] * (8 - len(t.dims))
            mb += _META.pack(t.id, t.dtype, len(t.dims), *dims, t.elem_count & 0xFFFFFFFF,
                             1 if t.is_weight else 0, ref[t.id] & 0xFF)
        weight_off = (meta_off + len(mb) + 15) & ~15
        pad = weight_off - (meta_off + len(mb))
        entries = bytearray()
        blob = bytearray()
        n_weights = 0
        for t in self.tensors:
            raw = t.data.tobytes() if t.is_weight else b""
            n_weights += 1 if t.is_weight else 0
            if raw:
                entries += _ENTRY.pack(t.id, 0, len(blob), len(raw), 0)
                blob += raw
            else:  # activations and empty initializers: a zero entry (onnx2ennf.c:451-456, 500)
                entries += _ENTRY.pack(t.id, 0, 0, 0, 0)
        hdr = _HDR.pack(ENNF_MAGIC, 2, 0, len(self.nodes), nt, n_weights, len(blob), len(self.inputs),
                        len(self.outputs), self.opset, self.flags, graph_meta_off, node_off, meta_off, weight_off, 0,
                        entry_off, 0, 0)
        return bytes(hdr) + bytes(entries) + gm + bytes(nb) + bytes(mb) + b"\0" * pad + bytes(blob)

    def write(self, path) -> Path:
        path = Path(path)
        path.write_bytes(self.to_bytes())
        return path


def read(path_or_bytes) -> dict:
    """Parse an ENNF file into plain Python structures (used by tests and tools)."""
    buf = path_or_bytes if isinstance(path_or_bytes, (bytes, bytearray)) else Path(path_or_bytes).read_bytes()
    h = _HDR.unpack_from(buf, 0)
    keys = ["magic", "version_major", "version_minor", "num_nodes", "num_tensors", "num_weights",
            "total_weight_bytes", "num_inputs", "num_outputs", "opset_version", "flags", "graph_meta_offset",
            "node_table_offset", "tensor_meta_offset", "weight_data_offset", "string_table_offset"]
    hdr = dict(zip(keys, h[:16]))
    hdr["reserved"] = list(h[16:])
    if hdr["magic"] != ENNF_MAGIC:
        raise ValueError("bad ENNF magic")
    off = hdr["graph_meta_offset"]
    (n_in,) = struct.unpack_from("<H", buf, off)
    ins = list(struct.unpack_from(f"<{n_in}H", buf, off + 2))
    off += 2 + 2 * n_in
    (n_out,) = struct.unpack_from("<H", buf, off)
    outs = list(struct.unpack_from(f"<{n_out}H", buf, off + 2))
    nodes = []
    off = hdr["node_table_offset"]
    for _ in range(hdr["num_nodes"]):
        op, ni, no, ps, fl, _r = _NODE.unpack_from(buf, off)
        off += 8
        ii = list(struct.unpack_from(f"<{ni}H", buf, off))
        off += 2 * ni
        oo = list(struct.unpack_from(f"<{no}H", buf, off))
        off += 2 * no
        params = bytes(buf[off:off + ps])
        off += ps
        nodes.append(dict(op=op, inputs=ii, outputs=oo, params=params, flags=fl))
    tensors = {}
    off = hdr["tensor_meta_offset"]
    for _ in range(hdr["num_tensors"]):
        m = _META.unpack_from(buf, off)
        off += 44
        tid, dt, nd = m[0], m[1], m[2]
        tensors[tid] = dict(id=tid, dtype=dt, dims=tuple(m[3:3 + nd]), elem_count=m[11], is_weight=m[12],
                            ref_count=m[13])
    weights = {}
    eoff = hdr["reserved"][0]
    for tid, t in tensors.items():
        e = _ENTRY.unpack_from(buf, eoff + tid * 16)
        if t["is_weight"] and e[3] > 0:
            start = hdr["weight_data_offset"] + e[2]
            arr = np.frombuffer(bytes(buf[start:start + e[3]]), dtype=_NP_DTYPE.get(t["dtype"], np.uint8))
            weights[tid] = arr.reshape(t["dims"]) if t["dtype"] in _NP_DTYPE else arr
    return dict(header=hdr, inputs=ins, outputs=outs, nodes=nodes, tensors=tensors, weights=weights)


def unpack_conv_params(b: bytes) -> dict:
    v = struct.unpack("<4H4H8H4HHBB", b[:44])
    return dict(kernel_shape=v[0:4], strides=v[4:8], pads=v[8:16], dilations=v[16:20], group=v[20],
                auto_pad=v[21], act=v[22])
