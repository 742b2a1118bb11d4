"""ctypes bindings of the native library (libspinn.so).

Two layers are exposed, matching include/spinn_hip.h and include/spinn_runtime.h:

* the HIP compute C ABI (``spinn_hip_conv``, ``spinn_hip_gemm``, glue ops and the
  memory/stream/event plumbing) - every pointer is a device address;
* the host runtime (``spinn_load`` / ``spinn_plan`` / ``spinn_run`` /
  ``spinn_free``) that executes ENNF models over an HBM arena.

``lib()`` raises if the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libspinn.so"
CLI_PATH = PKG / "bin" / "spinn_run"

# ---- constants mirrored from the headers ----
SPINN_HIP_OK = 0
SPINN_HIP_EINVAL = -1
SPINN_HIP_EUNSUPPORTED = -2
SPINN_HIP_EWORKSPACE = -3
SPINN_HIP_EDEVICE = -4
NOALLOC_SCRATCH_BYTES = 128 << 20  # SPINN_HIP_NOALLOC_SCRATCH_BYTES

ALGO_AUTO, ALGO_IMPLICIT_GEMM, ALGO_WINOGRAD, ALGO_DIRECT, ALGO_WINOGRAD_F43 = 0, 1, 2, 3, 4
ACT_NONE, ACT_RELU, ACT_CLIP, ACT_SILU, ACT_ADD, ACT_ADD_RELU = 0, 1, 2, 3, 4, 5
ENNF_MAX_DIMS = 8
POLICY_AUTO, POLICY_IGEMM, POLICY_WINOGRAD = 0, 1, 2
BINARY_ADD, BINARY_SUB, BINARY_MUL, BINARY_DIV, BINARY_MOD = 0, 1, 2, 3, 4
TOPK_MAX_K = 1024
UNARY_RELU, UNARY_SIGMOID, UNARY_SILU = 0, 1, 2
MAX_BLOCKS = 16


class ConvDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n", "c", "h", "w", "oc", "oh", "ow", "kh", "kw", "sh", "sw", "ph", "pw",
        "group", "act", "algo", "reserved")]


class GemmDesc(C.Structure):
    _fields_ = [
        ("m", C.c_int32), ("n", C.c_int32), ("k", C.c_int32),
        ("trans_a", C.c_int32), ("trans_b", C.c_int32), ("c_mode", C.c_int32),
        ("alpha", C.c_float), ("beta", C.c_float),
        ("batch", C.c_int32), ("reserved", C.c_int32),
        ("stride_a", C.c_int64), ("stride_b", C.c_int64), ("stride_y", C.c_int64),
    ]


class PoolDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n", "c", "h", "w", "oh", "ow", "kh", "kw", "sh", "sw", "ph", "pw")]


class GatherDesc(C.Structure):
    _fields_ = [("ndim", C.c_int32), ("axis", C.c_int32), ("index_dtype", C.c_int32), ("reserved", C.c_int32),
                ("in_dims", C.c_int64 * 8), ("out_dims", C.c_int64 * 8)]


class BlockCopy(C.Structure):
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p), ("src_row", C.c_int64), ("src_off", C.c_int64),
                ("dst_row", C.c_int64), ("dst_off", C.c_int64), ("len", C.c_int64)]


class SpinnTensor(C.Structure):
    _fields_ = [
        ("id", C.c_uint16), ("dtype", C.c_uint8), ("ndim", C.c_uint8),
        ("dims", C.c_uint32 * ENNF_MAX_DIMS), ("elem_count", C.c_uint32),
        ("is_weight", C.c_uint8), ("ref_count", C.c_uint8),
        ("size", C.c_uint32), ("offset", C.c_uint32),
        ("data", C.c_void_p), ("packed_data", C.c_void_p),
    ]


class SpinnNode(C.Structure):
    _fields_ = [
        ("op_type", C.c_uint16), ("num_inputs", C.c_uint8), ("num_outputs", C.c_uint8),
        ("input_ids", C.c_uint16 * 8), ("output_ids", C.c_uint16 * 8),
        ("params_size", C.c_uint16), ("params", C.c_void_p),
    ]


class ENNFHeader(C.Structure):
    _pack_ = 1
    _fields_ = [
        ("magic", C.c_uint32), ("version_major", C.c_uint16), ("version_minor", C.c_uint16),
        ("num_nodes", C.c_uint32), ("num_tensors", C.c_uint32), ("num_weights", C.c_uint32),
        ("total_weight_bytes", C.c_uint32), ("num_inputs", C.c_uint16), ("num_outputs", C.c_uint16),
        ("opset_version", C.c_uint16), ("flags", C.c_uint16),
        ("graph_meta_offset", C.c_uint32), ("node_table_offset", C.c_uint32),
        ("tensor_meta_offset", C.c_uint32), ("weight_data_offset", C.c_uint32),
        ("string_table_offset", C.c_uint32), ("reserved", C.c_uint32 * 3),
    ]


class SpinnArena(C.Structure):
    _fields_ = [("base", C.c_void_p), ("capacity", C.c_size_t), ("peak_usage", C.c_size_t)]


class SpinnContext(C.Structure):
    _fields_ = [
        ("header", ENNFHeader),
        ("input_ids", C.c_uint16 * 16), ("output_ids", C.c_uint16 * 16),
        ("tensors", C.POINTER(SpinnTensor)), ("num_tensors", C.c_uint32),
        ("nodes", C.POINTER(SpinnNode)), ("num_nodes", C.c_uint32),
        ("arena", SpinnArena),
        ("ennf_fp", C.c_void_p), ("weight_base_offset", C.c_uint32),
        ("weight_cache", C.POINTER(C.c_void_p)), ("num_weights", C.c_uint32),
        ("flags", C.c_uint16),
        ("stream", C.c_void_p), ("weight_pool", C.c_void_p), ("weight_pool_bytes", C.c_size_t),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("last_error", C.c_int), ("last_error_node", C.c_int),
        ("graph_exec", C.c_void_p), ("use_graph", C.c_int), ("prof_state", C.c_void_p),
        ("conv_policy", C.c_int),
        ("input_stage", C.c_void_p), ("input_staged", C.c_int),
        ("node_folded", C.POINTER(C.c_uint8)), ("node_tsrc", C.POINTER(C.c_int32)),
        ("node_tdst", C.POINTER(C.c_int32)), ("node_alpha", C.POINTER(C.c_float)),
    ]


_lib = None

# name -> (restype, argtypes)
_SIGS = {
    "spinn_hip_conv": (C.c_int, [C.POINTER(ConvDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "spinn_hip_conv_noalloc": (C.c_int, [C.POINTER(ConvDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_conv_select_algo": (C.c_int, [C.POINTER(ConvDesc)]),
    "spinn_hip_conv_workspace_size": (C.c_size_t, [C.POINTER(ConvDesc)]),
    "spinn_hip_conv_packed_size": (C.c_size_t, [C.POINTER(ConvDesc)]),
    "spinn_hip_conv_pack_weights": (C.c_int, [C.POINTER(ConvDesc), C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_gemm": (C.c_int, [C.POINTER(GemmDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_void_p, C.c_size_t, C.c_void_p]),
    "spinn_hip_gemm_workspace_size": (C.c_size_t, [C.POINTER(GemmDesc)]),
    "spinn_hip_maxpool2d": (C.c_int, [C.POINTER(PoolDesc), C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_reduce_mean": (C.c_int, [C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_copy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "spinn_hip_device_status": (C.c_int, []),
    "spinn_hip_tune_streamk_tries": (None, [C.c_int]),
    "spinn_hip_tune_winograd_fused": (None, [C.c_int]),
    "spinn_hip_binary": (C.c_int, [C.c_int, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64,
                                   C.c_void_p]),
    "spinn_hip_unary": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "spinn_hip_batchnorm": (C.c_int, [C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_float, C.c_void_p, C.c_void_p]),
    "spinn_hip_softmax": (C.c_int, [C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_block_copy": (C.c_int, [C.POINTER(BlockCopy), C.c_int, C.c_int64, C.c_void_p]),
    "spinn_hip_transpose": (C.c_int, [C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int32), C.c_void_p,
                                      C.c_void_p, C.c_void_p]),
    "spinn_hip_resize_nearest": (C.c_int, [C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                           C.c_void_p, C.c_void_p]),
    "spinn_hip_reduce_max": (C.c_int, [C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_topk": (C.c_int, [C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_gather_elements": (C.c_int, [C.POINTER(GatherDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_tile": (C.c_int, [C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_int, C.c_void_p,
                                 C.c_void_p, C.c_void_p]),
    "spinn_hip_cast": (C.c_int, [C.c_int, C.c_int, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "spinn_hip_binary_typed": (C.c_int, [C.c_int, C.c_int, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
                                         C.c_int64, C.c_void_p]),
    "spinn_hip_init": (C.c_int, [C.c_int]),
    "spinn_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "spinn_hip_malloc": (C.c_int, [C.POINTER(C.c_void_p), C.c_size_t]),
    "spinn_hip_free": (C.c_int, [C.c_void_p]),
    "spinn_hip_memcpy_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "spinn_hip_memcpy_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "spinn_hip_fill_u32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_size_t, C.c_void_p]),
    "spinn_hip_stream_create": (C.c_int, [C.POINTER(C.c_void_p)]),
    "spinn_hip_stream_destroy": (C.c_int, [C.c_void_p]),
    "spinn_hip_stream_sync": (C.c_int, [C.c_void_p]),
    "spinn_hip_event_create": (C.c_int, [C.POINTER(C.c_void_p)]),
    "spinn_hip_event_destroy": (C.c_int, [C.c_void_p]),
    "spinn_hip_event_record": (C.c_int, [C.c_void_p, C.c_void_p]),
    "spinn_hip_event_elapsed_ms": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]),
    "spinn_hip_graph_capture_begin": (C.c_int, [C.c_void_p]),
    "spinn_hip_graph_capture_end": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "spinn_hip_graph_launch": (C.c_int, [C.c_void_p, C.c_void_p]),
    "spinn_hip_graph_destroy": (C.c_int, [C.c_void_p]),
    "spinn_hip_error_string": (C.c_char_p, [C.c_int]),
    "spinn_hip_version": (C.c_char_p, []),
    "spinn_hip_tune_force_tiles": (None, [C.c_int, C.c_int, C.c_int]),
    "spinn_hip_tune_streamk": (None, [C.c_int]),
    # host runtime
    "spinn_load": (C.POINTER(SpinnContext), [C.c_char_p]),
    "spinn_plan": (C.c_int, [C.POINTER(SpinnContext), C.c_uint32]),
    "spinn_run": (C.c_int, [C.POINTER(SpinnContext), C.c_void_p, C.c_void_p]),
    "spinn_free": (None, [C.POINTER(SpinnContext)]),
    "spinn_profile_dump": (None, []),
    "spinn_get_weight": (C.c_void_p, [C.POINTER(SpinnContext), C.c_uint16]),
    "spinn_plan_memory": (C.c_int, [C.POINTER(SpinnContext), C.c_uint32]),
    "spinn_dispatch_op": (C.c_int, [C.c_uint16, C.POINTER(C.POINTER(SpinnTensor)), C.c_int, C.c_void_p,
                                    C.c_uint16, C.POINTER(C.POINTER(SpinnTensor)), C.c_int]),
    "spinn_tensor_upload": (C.c_int, [C.POINTER(SpinnContext), C.c_uint16, C.c_void_p, C.c_size_t]),
    "spinn_tensor_download": (C.c_int, [C.POINTER(SpinnContext), C.c_uint16, C.c_void_p, C.c_size_t]),
    "spinn_run_resident": (C.c_int, [C.POINTER(SpinnContext)]),
    "spinn_stage_input": (C.c_int, [C.POINTER(SpinnContext), C.c_void_p, C.c_size_t]),
    "spinn_input_stage_ptr": (C.c_void_p, [C.POINTER(SpinnContext)]),
    "spinn_set_graph_mode": (C.c_int, [C.POINTER(SpinnContext), C.c_int]),
    "spinn_node_times": (C.c_int, [C.POINTER(SpinnContext), C.POINTER(C.c_float), C.c_int]),
    "spinn_op_registered": (C.c_int, [C.c_uint16]),
    "spinn_set_conv_policy": (C.c_int, [C.POINTER(SpinnContext), C.c_int]),
    "spinn_set_profiling": (None, [C.c_int]),
}


class NativeMissing(RuntimeError):
    pass


def lib() -> C.CDLL:
    """The loaded native library; raises NativeMissing if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise NativeMissing(f"{LIB_PATH} is missing: run `python -m spinn_amd.build` first")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


class SpinnError(RuntimeError):
    def __init__(self, code: int, what: str):
        msg = lib().spinn_hip_error_string(code)
        super().__init__(f"{what} failed: {code} ({msg.decode() if msg else '?'})")
        self.code = code


def check(code: int, what: str) -> None:
    if code != 0:
        raise SpinnError(code, what)


def ptr(t) -> C.c_void_p | None:
    """Device pointer of a torch tensor (or None)."""
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())
