"""ctypes binding of libmoehip.so (include/moe_hip.h, include/moe_safetensors.h).

This is the Python view of the C ABI that a Swift (or any FFI) caller binds;
tests and bench.py drive the library through it with device buffers owned by
PyTorch. There is no fallback: if the library is missing, loading fails with
an error naming the build step.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoehip.so")

MOE_OK, MOE_ERR_INVALID, MOE_ERR_UNSUPPORTED, MOE_ERR_WORKSPACE, MOE_ERR_HIP = range(5)
MOE_F32, MOE_F16, MOE_BF16 = 0, 1, 2
MOE_SOFTMAX_THEN_TOPK, MOE_TOPK_THEN_SOFTMAX, MOE_SIGMOID_TOPK = 0, 1, 2
MOE_ACT_SWIGLU, MOE_ACT_GPTOSS, MOE_ACT_GEGLU, MOE_ACT_RELU2 = 0, 1, 2, 3
MOE_PATH_NONE, MOE_PATH_DECODE1, MOE_PATH_GEMV, MOE_PATH_GEMV_MMA, MOE_PATH_GEMM = range(5)
PATH_NAMES = {MOE_PATH_NONE: "none", MOE_PATH_DECODE1: "decode1", MOE_PATH_GEMV: "gemv",
              MOE_PATH_GEMV_MMA: "gemv_mma", MOE_PATH_GEMM: "gemm"}
(MOE_ST_F32, MOE_ST_F16, MOE_ST_BF16, MOE_ST_I32, MOE_ST_U32, MOE_ST_I64, MOE_ST_U64, MOE_ST_I8,
 MOE_ST_U8) = range(9)
MOE_ST_MAX_DIMS = 8

EXPORTS = [
    "moe_last_error_string", "moe_version", "moe_validate_qproj", "moe_validate_layer",
    "moe_derive_bits", "moe_router_logits", "moe_router_logits_q", "moe_router_topk",
    "moe_router_topk_scaled",
    "moe_dispatch_workspace_bytes",
    "moe_dispatch_plan", "moe_dequantize_affine", "moe_expert_matmul_workspace_bytes",
    "moe_expert_matmul", "moe_activation_apply", "moe_unpermute", "moe_layer_workspace_bytes",
    "moe_layer_forward", "moe_layer_forward_routed", "moe_layer_forward_residual",
    "moe_layer_path", "moe_layer_forward_noalloc", "moe_layer_noalloc_max_bytes", "moe_add_rmsnorm", "moe_mxfp4_to_affine", "moe_layer_create", "moe_layer_destroy",
    "moe_layer_decode", "moe_layer_decode_many",
    "moe_st_open", "moe_st_close", "moe_st_count", "moe_st_name", "moe_st_info", "moe_st_read_host",
    "moe_st_upload", "moe_st_is_quantized", "moe_st_stacked_bytes", "moe_st_load_stacked",
    "moe_st_load_stacked_many", "moe_st_mxfp4_bytes", "moe_st_load_mxfp4",
]


class MoeError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"moe status {status}: {msg}")
        self.status = status


class QProj(C.Structure):
    _fields_ = [
        ("weight", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
        ("out_bias", C.c_void_p),
        ("bits", C.c_int32), ("group_size", C.c_int32), ("sb_dtype", C.c_int32),
        ("n", C.c_int32), ("k", C.c_int32), ("n_experts", C.c_int32),
    ]


class LayerDesc(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32),
        ("intermediate", C.c_int32), ("act_dtype", C.c_int32),
        ("router_weight", C.c_void_p), ("router_dtype", C.c_int32), ("router_bias", C.c_void_p),
        ("gating", C.c_int32), ("norm_topk_prob", C.c_int32), ("expert_bias", C.c_void_p),
        ("gate", QProj), ("up", QProj), ("down", QProj),
        ("activation", C.c_int32), ("act_alpha", C.c_float), ("act_limit", C.c_float),
        ("has_shared", C.c_int32),
        ("shared_gate", QProj), ("shared_up", QProj), ("shared_down", QProj),
        ("shared_gate_weight", C.c_void_p),
        ("logit_scale", C.c_float), ("routed_scale", C.c_float), ("expert_scale", C.c_void_p),
        ("router_q", QProj), ("shared_gate_q", QProj),
    ]


class LayerPaths(C.Structure):
    _fields_ = [("gate_up", C.c_int32), ("down", C.c_int32), ("shared_gate_up", C.c_int32),
                ("shared_down", C.c_int32)]

    def names(self) -> dict:
        return {f: PATH_NAMES[getattr(self, f)] for f, _ in self._fields_}


class LayerTrace(C.Structure):
    _fields_ = [
        ("logits", C.c_void_p), ("topk_idx", C.c_void_p), ("topk_weight", C.c_void_p),
        ("perm", C.c_void_p), ("offsets", C.c_void_p), ("events", C.c_void_p * 4),
    ]


_lib = None


def load():
    """Load libmoehip.so (built by ffai_amd.build.build())."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(LIB_PATH)
    vp, i32, sz, st = C.c_void_p, C.c_int32, C.c_size_t, C.c_void_p
    lib.moe_last_error_string.restype = C.c_char_p
    lib.moe_version.restype = C.c_char_p
    lib.moe_validate_qproj.argtypes = [C.POINTER(QProj)]
    lib.moe_validate_layer.argtypes = [C.POINTER(LayerDesc)]
    lib.moe_derive_bits.argtypes = [C.c_int64, C.c_int64, i32, C.POINTER(i32)]
    lib.moe_router_logits.argtypes = [vp, i32, i32, i32, vp, i32, vp, i32, vp, st]
    lib.moe_router_logits_q.argtypes = [vp, i32, i32, i32, C.POINTER(QProj), vp, i32, vp, st]
    lib.moe_router_topk.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, st]
    lib.moe_router_topk_scaled.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, C.c_float,
                                           C.c_float, vp, vp, vp, st]
    lib.moe_dispatch_workspace_bytes.argtypes = [i32, i32, i32]
    lib.moe_dispatch_workspace_bytes.restype = sz
    lib.moe_dispatch_plan.argtypes = [vp, i32, i32, i32, vp, vp, vp, vp, vp, sz, st]
    lib.moe_dequantize_affine.argtypes = [vp, vp, vp, i32, i32, i32, C.c_int64, vp, i32, st]
    lib.moe_expert_matmul_workspace_bytes.argtypes = [C.POINTER(QProj), i32, i32]
    lib.moe_expert_matmul_workspace_bytes.restype = sz
    lib.moe_expert_matmul.argtypes = [C.POINTER(QProj), vp, i32, vp, i32, i32, vp, vp, vp, sz, st]
    lib.moe_activation_apply.argtypes = [vp, vp, vp, C.c_int64, i32, i32, C.c_float, C.c_float, st]
    lib.moe_unpermute.argtypes = [vp, vp, vp, i32, i32, i32, vp, i32, st]
    lib.moe_layer_workspace_bytes.argtypes = [C.POINTER(LayerDesc), i32]
    lib.moe_layer_workspace_bytes.restype = sz
    lib.moe_layer_forward.argtypes = [C.POINTER(LayerDesc), vp, i32, vp, vp, sz,
                                      C.POINTER(LayerTrace), st]
    lib.moe_layer_forward_routed.argtypes = [C.POINTER(LayerDesc), vp, vp, i32, vp, vp, sz,
                                             C.POINTER(LayerTrace), st]
    lib.moe_layer_forward_residual.argtypes = [C.POINTER(LayerDesc), vp, vp, vp, C.c_float, i32,
                                               vp, vp, vp, sz, C.POINTER(LayerTrace), st]
    lib.moe_layer_path.argtypes = [C.POINTER(LayerDesc), i32, C.POINTER(LayerPaths)]
    lib.moe_layer_forward_noalloc.argtypes = [C.POINTER(LayerDesc), vp, i32, vp,
                                              C.POINTER(LayerTrace), st]
    lib.moe_layer_noalloc_max_bytes.argtypes = []
    lib.moe_layer_noalloc_max_bytes.restype = sz
    lib.moe_add_rmsnorm.argtypes = [vp, vp, vp, C.c_float, i32, i32, i32, vp, vp, st]
    lib.moe_mxfp4_to_affine.argtypes = [vp, vp, C.c_int64, vp, vp, vp, i32, st]
    lib.moe_layer_create.argtypes = [C.POINTER(LayerDesc), C.POINTER(vp)]
    lib.moe_layer_destroy.argtypes = [vp]
    lib.moe_layer_destroy.restype = None
    lib.moe_layer_decode.argtypes = [vp, vp, vp, st]
    lib.moe_layer_decode_many.argtypes = [vp, vp, i32, vp, st]
    lib.moe_st_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    lib.moe_st_close.argtypes = [vp]
    lib.moe_st_close.restype = None
    lib.moe_st_count.argtypes = [vp]
    lib.moe_st_count.restype = C.c_int64
    lib.moe_st_name.argtypes = [vp, C.c_int64]
    lib.moe_st_name.restype = C.c_char_p
    lib.moe_st_info.argtypes = [vp, C.c_char_p, C.POINTER(i32), C.POINTER(i32),
                                C.POINTER(C.c_int64), C.POINTER(sz)]
    lib.moe_st_read_host.argtypes = [vp, C.c_char_p, vp, sz]
    lib.moe_st_upload.argtypes = [vp, C.c_char_p, vp, sz, st]
    lib.moe_st_is_quantized.argtypes = [vp, C.c_char_p]
    lib.moe_st_is_quantized.restype = i32
    lib.moe_st_stacked_bytes.argtypes = [vp, C.c_char_p, i32, C.POINTER(sz)]
    lib.moe_st_load_stacked.argtypes = [vp, C.c_char_p, i32, vp, sz, C.POINTER(QProj), st]
    lib.moe_st_load_stacked_many.argtypes = [vp, i32, C.POINTER(C.c_char_p), i32, C.POINTER(vp),
                                             C.POINTER(sz), C.POINTER(QProj), st]
    lib.moe_st_mxfp4_bytes.argtypes = [vp, C.c_char_p, i32, C.POINTER(sz), C.POINTER(sz)]
    lib.moe_st_load_mxfp4.argtypes = [vp, C.c_char_p, i32, vp, sz, vp, sz, C.POINTER(QProj), st]
    for name in ["moe_validate_qproj", "moe_validate_layer", "moe_derive_bits", "moe_router_logits",
                 "moe_router_logits_q", "moe_router_topk", "moe_router_topk_scaled", "moe_dispatch_plan",
                 "moe_dequantize_affine", "moe_expert_matmul", "moe_activation_apply",
                 "moe_unpermute", "moe_layer_forward", "moe_layer_forward_routed",
                 "moe_layer_forward_residual", "moe_layer_path", "moe_layer_forward_noalloc",
                 "moe_add_rmsnorm", "moe_mxfp4_to_affine",
                 "moe_layer_create", "moe_layer_decode",
                 "moe_layer_decode_many", "moe_st_open", "moe_st_info", "moe_st_read_host",
                 "moe_st_upload", "moe_st_stacked_bytes", "moe_st_load_stacked",
                 "moe_st_load_stacked_many", "moe_st_mxfp4_bytes", "moe_st_load_mxfp4"]:
        getattr(lib, name).restype = C.c_int
    _lib = lib
    return lib


def check(status: int):
    if status != MOE_OK:
        raise MoeError(status, load().moe_last_error_string().decode())
    return status


def last_error() -> str:
    return load().moe_last_error_string().decode()
