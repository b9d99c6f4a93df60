"""ctypes binding of the C ABI declared in include/bghip.h.

The library is loaded from the package directory (built in-tree by
``python -m browsergrad_amd.build``).  There is no CPU fallback: if the
library is missing or the device cannot be opened, every entry point raises
``KernelError`` -- the HIP realizer either runs on the GPU or fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from .errors import KernelError

LIB_PATH = Path(__file__).resolve().parent / "libbghip.so"

BG_MAX_RANK = 8
BG_FUSED_MAX_INPUTS = 8
BG_FUSED_MAX_OPS = 32
BG_FUSED_MAX_IMMS = 16

# status codes
BG_OK, BG_E_INVALID, BG_E_HANDLE, BG_E_DTYPE, BG_E_SHAPE, BG_E_OOM, BG_E_HIP, BG_E_UNSUPPORTED = range(8)

# dtypes
BG_F32, BG_F16, BG_BF16, BG_BOOL, BG_I32, BG_I64, BG_U8, BG_F64 = range(8)
DTYPE_CODES = {
    "float32": BG_F32, "float16": BG_F16, "bfloat16": BG_BF16, "bool": BG_BOOL,
    "int32": BG_I32, "int64": BG_I64, "uint8": BG_U8, "float64": BG_F64,
}
DTYPE_NAMES = {v: k for k, v in DTYPE_CODES.items()}
DTYPE_SIZES = {BG_F32: 4, BG_F16: 2, BG_BF16: 2, BG_BOOL: 1, BG_I32: 4, BG_I64: 8, BG_U8: 1, BG_F64: 8}

# fused opcodes
OPS = {
    "ADD": 0, "MUL": 1, "DIV": 2, "NEG": 3, "EXP": 4, "LOG": 5,
    "MAX": 6, "MIN": 7, "CMP_EQ": 8, "CMP_NE": 9, "CMP_LT": 10, "CMP_LE": 11,
    "CMP_GT": 12, "CMP_GE": 13, "WHERE": 14, "IMM": 15, "ROUND_F16": 16,
    "ROUND_BF16": 17, "SUB": 18, "TANH": 19, "SQRT": 20, "RECIP": 21, "ABS": 22,
    "COPY": 23,
}
RED_NONE, RED_SUM, RED_MAX, RED_MEAN, RED_MIN = range(5)
ACT_NONE, ACT_RELU, ACT_GELU_TANH = range(3)

handle_t = C.c_uint64


class FusedOp(C.Structure):
    _fields_ = [("code", C.c_int32), ("a", C.c_int32), ("b", C.c_int32), ("c", C.c_int32)]


class FusedDesc(C.Structure):
    _fields_ = [
        ("n_inputs", C.c_int32),
        ("inputs", C.POINTER(handle_t)),
        ("in_strides", C.POINTER(C.c_int64)),
        ("n_ops", C.c_int32),
        ("ops", C.POINTER(FusedOp)),
        ("n_imms", C.c_int32),
        ("imms", C.POINTER(C.c_double)),
        ("rank", C.c_int32),
        ("shape", C.POINTER(C.c_int64)),
        ("out_dtype", C.c_int32),
        ("reduce_op", C.c_int32),
        ("reduce_keepdims", C.c_int32),
    ]


class MatmulDesc(C.Structure):
    _fields_ = [
        ("a", handle_t), ("b", handle_t), ("bias", handle_t),
        ("batch", C.c_int64), ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
        ("lda", C.c_int64), ("ldb", C.c_int64), ("ldc", C.c_int64),
        ("stride_a", C.c_int64), ("stride_b", C.c_int64), ("stride_c", C.c_int64),
        ("offset_a", C.c_int64), ("offset_b", C.c_int64),
        ("trans_b", C.c_int32), ("in_dtype", C.c_int32), ("out_dtype", C.c_int32),
        ("round_f16", C.c_int32), ("act", C.c_int32), ("reserved", C.c_int32),
    ]


class MatmulExt(C.Structure):
    _fields_ = [
        ("residual", handle_t), ("a_dtype", C.c_int32), ("b_dtype", C.c_int32),
        ("reserved", C.c_int32 * 4),
    ]


class LaunchRecord(C.Structure):
    _fields_ = [
        ("kernel", C.c_char * 160), ("grid", C.c_int64 * 3), ("block", C.c_int32 * 3),
        ("dynamic_lds", C.c_int64), ("static_lds", C.c_int64), ("vgprs", C.c_int32), ("scratch", C.c_int32),
        ("max_threads", C.c_int32), ("reserved", C.c_int32),
    ]


class AttentionDesc(C.Structure):
    _fields_ = [
        ("q", handle_t), ("k", handle_t), ("v", handle_t),
        ("batch", C.c_int64), ("heads", C.c_int64), ("sq", C.c_int64), ("sk", C.c_int64), ("d", C.c_int64),
        ("q_off", C.c_int64), ("k_off", C.c_int64), ("v_off", C.c_int64),
        ("q_sb", C.c_int64), ("q_sh", C.c_int64), ("q_ss", C.c_int64),
        ("k_sb", C.c_int64), ("k_sh", C.c_int64), ("k_ss", C.c_int64),
        ("v_sb", C.c_int64), ("v_sh", C.c_int64), ("v_ss", C.c_int64),
        ("o_sb", C.c_int64), ("o_sh", C.c_int64), ("o_ss", C.c_int64),
        ("scale", C.c_float), ("causal", C.c_int32), ("in_dtype", C.c_int32),
        ("out_dtype", C.c_int32), ("round_scores", C.c_int32), ("reserved", C.c_int32),
    ]


BG_PLAN_MAX_LAUNCHES = 4


class LaunchPlanEntry(C.Structure):
    _fields_ = [
        ("family", C.c_char * 48), ("n_targs", C.c_int32), ("targs", C.c_int32 * 8), ("block", C.c_int32 * 3),
        ("grid", C.c_int64 * 3),
    ]


class LaunchPlan(C.Structure):
    _fields_ = [
        ("n_launches", C.c_int32), ("tile_m", C.c_int32), ("tile_n", C.c_int32), ("tile_k", C.c_int32),
        ("k_slices", C.c_int32), ("reserved", C.c_int32), ("lds_bytes", C.c_int64), ("workspace_bytes", C.c_int64),
        ("launch", LaunchPlanEntry * BG_PLAN_MAX_LAUNCHES),
    ]


class Snapshot(C.Structure):
    _fields_ = [
        ("current_owned_bytes", C.c_int64), ("peak_owned_bytes", C.c_int64),
        ("total_allocated_bytes", C.c_int64), ("total_released_bytes", C.c_int64),
        ("alive_handle_count", C.c_int64), ("pending_profile_count", C.c_int64),
        ("pass_profile_count", C.c_int64), ("pool_cached_bytes", C.c_int64),
        ("pool_hits", C.c_int64), ("pool_misses", C.c_int64),
        ("timing_mode", C.c_int32), ("timestamp_query_available", C.c_int32),
    ]


class OptimArgs(C.Structure):
    """bg_optim_args: the scalar arguments of one optimizer update."""
    _fields_ = [("lr", C.c_double), ("beta1", C.c_double), ("beta2", C.c_double), ("eps", C.c_double),
                ("weight_decay", C.c_double), ("step", C.c_int64)]


class ConvDesc(C.Structure):
    """bg_conv_desc: one convolution of the plan route (any rank, transposed or not)."""
    _fields_ = [("op", C.c_int32), ("transposed", C.c_int32), ("spatial", C.c_int32), ("pad0", C.c_int32),
                ("n", C.c_int64), ("c_in", C.c_int64), ("c_out", C.c_int64), ("groups", C.c_int64),
                ("in_", C.c_int64 * 3), ("out", C.c_int64 * 3), ("k", C.c_int64 * 3), ("stride", C.c_int64 * 3),
                ("pad", C.c_int64 * 3), ("dilation", C.c_int64 * 3), ("output_pad", C.c_int64 * 3),
                ("a", handle_t), ("b", handle_t), ("bias", handle_t)]


CONV_OPS = {"forward": 0, "backward_input": 1, "backward_weight": 2, "backward_bias": 3}


# bg_optimizer_update kinds (BG_OPT_*), keyed by the reference's plan op names.
OPTIM_KINDS = {
    "SGD_UPDATE": 0, "ADAMW_UPDATE_M": 1, "ADAMW_UPDATE_V": 2, "ADAMW_UPDATE_PARAM": 3,
    "ADAM_UPDATE_M": 4, "ADAM_UPDATE_V": 5, "ADAM_UPDATE_PARAM": 6,
}


class PassProfile(C.Structure):
    _fields_ = [("label", C.c_char * 48), ("gpu_ms", C.c_double), ("bytes", C.c_int64), ("flops", C.c_int64)]


ctx_p = C.c_void_p
P64 = C.POINTER(C.c_int64)
PH = C.POINTER(handle_t)

# name -> (restype, argtypes); every function declared in include/bghip.h.
SIGNATURES = {
    "bg_ctx_create": (C.c_int, [C.c_int, C.c_int, C.POINTER(ctx_p)]),
    "bg_ctx_destroy": (C.c_int, [ctx_p]),
    "bg_last_error": (C.c_char_p, [ctx_p]),
    "bg_dtype_from_name": (C.c_int, [C.c_char_p]),
    "bg_dtype_size": (C.c_int64, [C.c_int]),
    "bg_synchronize": (C.c_int, [ctx_p]),
    "bg_version": (C.c_char_p, []),
    "bg_upload": (C.c_int, [ctx_p, C.c_void_p, C.c_size_t, P64, C.c_int, C.c_int, PH]),
    "bg_materialize": (C.c_int, [ctx_p, handle_t, C.c_void_p, C.c_size_t]),
    "bg_release": (C.c_int, [ctx_p, handle_t]),
    "bg_handle_info": (C.c_int, [ctx_p, handle_t, P64, C.POINTER(C.c_int), C.POINTER(C.c_int), P64]),
    "bg_alive_handles": (C.c_int, [ctx_p, P64]),
    "bg_resource_snapshot": (C.c_int, [ctx_p, C.POINTER(Snapshot)]),
    "bg_flush_profiles": (C.c_int, [ctx_p, C.POINTER(PassProfile), C.c_int, C.POINTER(C.c_int)]),
    "bg_set_profiling": (C.c_int, [ctx_p, C.c_int]),
    "bg_matmul": (C.c_int, [ctx_p, handle_t, handle_t, C.c_int64, C.c_int64, C.c_int64, C.c_int, PH]),
    "bg_fused_elementwise": (C.c_int, [ctx_p, PH, C.c_int, C.POINTER(FusedOp), C.c_int, P64, C.c_int, C.c_int, PH]),
    "bg_cast": (C.c_int, [ctx_p, handle_t, C.c_int, C.c_int, P64, C.c_int, PH]),
    "bg_flash_attention": (C.c_int, [ctx_p, handle_t, handle_t, handle_t, handle_t, C.c_int64, C.c_int64,
                                     C.c_int64, C.c_int64, C.c_int64, C.c_float, C.c_int, PH]),
    "bg_matmul_ex": (C.c_int, [ctx_p, C.POINTER(MatmulDesc), PH]),
    "bg_plan_inspect": (C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "bg_set_launch_log": (C.c_int, [ctx_p, C.c_int]),
    "bg_take_launch_log": (C.c_int, [ctx_p, C.POINTER(LaunchRecord), C.c_int, C.POINTER(C.c_int)]),
    "bg_matmul_ex2": (C.c_int, [ctx_p, C.POINTER(MatmulDesc), C.POINTER(MatmulExt), PH]),
    "bg_matmul_noalloc": (C.c_int, [ctx_p, C.POINTER(MatmulDesc), C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]),
    "bg_fused_ex": (C.c_int, [ctx_p, C.POINTER(FusedDesc), PH]),
    "bg_attention_ex": (C.c_int, [ctx_p, C.POINTER(AttentionDesc), PH]),
    "bg_layer_norm": (C.c_int, [ctx_p, handle_t, handle_t, handle_t, C.c_int64, C.c_int64, C.c_float, C.c_int, PH]),
    "bg_layer_norm_backward_input": (C.c_int, [ctx_p, handle_t, handle_t, handle_t, C.c_int64, C.c_int64,
                                               C.c_float, PH]),
    "bg_layer_norm_backward_weight": (C.c_int, [ctx_p, handle_t, handle_t, C.c_int64, C.c_int64, C.c_float, PH]),
    "bg_layer_norm_backward_bias": (C.c_int, [ctx_p, handle_t, C.c_int64, C.c_int64, PH]),
    "bg_optimizer_update": (C.c_int, [ctx_p, C.c_int, C.POINTER(handle_t), C.c_int, C.POINTER(OptimArgs),
                                      C.c_int64, PH]),
    "bg_conv1d": (C.c_int, [ctx_p, handle_t, handle_t, handle_t] + [C.c_int64] * 10 + [C.c_int, PH]),
    "bg_conv1d_backward_input": (C.c_int, [ctx_p, handle_t, handle_t] + [C.c_int64] * 10 + [C.c_int, PH]),
    "bg_conv1d_backward_weight": (C.c_int, [ctx_p, handle_t, handle_t] + [C.c_int64] * 10 + [C.c_int, PH]),
    "bg_conv1d_backward_bias": (C.c_int, [ctx_p, handle_t] + [C.c_int64] * 3 + [C.c_int, PH]),
    "bg_conv2d": (C.c_int, [ctx_p, handle_t, handle_t, handle_t] + [C.c_int64] * 16 + [C.c_int, PH]),
    "bg_conv2d_backward_input": (C.c_int, [ctx_p, handle_t, handle_t] + [C.c_int64] * 16 + [C.c_int, PH]),
    "bg_conv2d_backward_weight": (C.c_int, [ctx_p, handle_t, handle_t] + [C.c_int64] * 16 + [C.c_int, PH]),
    "bg_conv2d_backward_bias": (C.c_int, [ctx_p, handle_t] + [C.c_int64] * 4 + [C.c_int, PH]),
    "bg_conv_ex": (C.c_int, [ctx_p, C.POINTER(ConvDesc), PH]),
    "bg_copy_strided": (C.c_int, [ctx_p, handle_t, C.c_int64, P64, P64, C.c_int, PH]),
    "bg_reshape": (C.c_int, [ctx_p, handle_t, P64, C.c_int, PH]),
    "bg_reduce_last": (C.c_int, [ctx_p, handle_t, C.c_int64, C.c_int64, C.c_int, C.c_int, PH]),
    "bg_run_tensor_plan": (C.c_int, [ctx_p, C.c_char_p, P64, PH, C.c_int, C.c_int, C.c_void_p, C.c_size_t, PH]),
    "bg_run_tensor_plan_semantic": (C.c_int, [ctx_p, C.c_char_p, C.c_char_p, P64, PH, C.c_int, C.c_int,
                                              C.c_void_p, C.c_size_t, PH]),
    "bg_softmax_last": (C.c_int, [ctx_p, handle_t, C.c_int64, C.c_int64, C.c_int, PH]),
    "bg_device_ptr": (C.c_int, [ctx_p, handle_t, C.POINTER(C.c_void_p)]),
    "bg_matmul_launch_plan": (C.c_int, [C.POINTER(MatmulDesc), C.POINTER(LaunchPlan), C.c_char_p, C.c_size_t]),
    "bg_attention_launch_plan": (C.c_int, [C.POINTER(AttentionDesc), C.POINTER(LaunchPlan), C.c_char_p,
                                           C.c_size_t]),
    "bg_stream": (C.c_int, [ctx_p, C.POINTER(C.c_void_p)]),
}

# Exported for tests only (not part of include/bghip.h).
EXTRA_SIGNATURES = {
    "bg_fused_codegen_selftest": (C.c_int, [C.c_char_p, C.c_size_t]),
}

_LIB = None


def load_library(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libbghip.so and attach signatures.  Raises KernelError if absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise KernelError(
            f"HIP bridge: {p} is not built. Run `python -m browsergrad_amd.build` "
            f"(there is no CPU fallback for the HIP realizer)."
        )
    lib = C.CDLL(str(p))
    for name, (res, args) in {**SIGNATURES, **EXTRA_SIGNATURES}.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def i64_array(vals) -> C.Array:
    vals = [int(v) for v in vals]
    return (C.c_int64 * max(1, len(vals)))(*vals)


def handle_array(vals) -> C.Array:
    vals = [int(v) for v in vals]
    return (handle_t * max(1, len(vals)))(*vals)
