"""ctypes bindings for libonnxruntime_ep_mlx_amd.so (the C ABI in include/pa_mi355x.h).

The library is the product: there is no Python or CPU fallback.  ``load()`` raises if the
shared library has not been built (``python -c "import __graft_entry__ as g; g.build()"``).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
# ONNXRUNTIME_EP_MLX_AMD_LIB selects another build of the same library (side-by-side builds).
LIB_PATH = Path(os.environ.get("ONNXRUNTIME_EP_MLX_AMD_LIB",
                               PKG_ROOT / "lib" / "libonnxruntime_ep_mlx_amd.so"))

PA_DTYPE_FLOAT16 = 1
PA_DTYPE_BFLOAT16 = 2
PA_DTYPE_FLOAT32 = 3
PA_DTYPE_FP8_E4M3 = 4
PA_DTYPE_INT8 = 5
PA_DTYPE_INT4 = 6
PA_INT32_DTYPE = 10
PA_INT8_DTYPE = 11
PA_UINT8_DTYPE = 12
PA_INT64_DTYPE = 13

PA_QUANT_NONE = 0
PA_QUANT_PER_TENSOR = 1
PA_QUANT_PER_CHANNEL = 2
QUANT_TYPES = {"NONE": PA_QUANT_NONE, "PER_TENSOR": PA_QUANT_PER_TENSOR,
               "PER_CHANNEL": PA_QUANT_PER_CHANNEL}

PA_STATIC_SCRATCH_BYTES = 64 << 20  # include/pa_mi355x.h

PA_OK = 0
PA_ERR_INVALID_ARGUMENT = 1
PA_ERR_UNSUPPORTED = 2
PA_ERR_HIP = 3
PA_ERR_OUT_OF_MEMORY = 4

# Every function the header declares, in declaration order (checked by the CPU test suite).
EXPORTS = (
    "pa_last_error", "pa_version",
    "pa_pool_create", "pa_pool_destroy", "pa_pool_k_ptr", "pa_pool_v_ptr",
    "pa_pool_k_scale_ptr", "pa_pool_v_scale_ptr", "pa_pool_bytes",
    "pa_rotary_append", "pa_reshape_and_cache",
    "pa_attention_workspace_bytes", "pa_attention_workspace_bytes_ex",
    "pa_attention", "pa_attention_ex",
    "pa_paged_attention_workspace_bytes", "pa_paged_attention", "pa_paged_attention_static",
    "pa_paged_attention_claim",
    "pa_group_query_attention_workspace_bytes", "pa_group_query_attention",
    "pa_group_query_attention_claim",
)


class PaCache(C.Structure):
    _fields_ = [
        ("key_cache", C.c_void_p), ("value_cache", C.c_void_p),
        ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
        ("num_blocks", C.c_int64), ("block_size", C.c_int32), ("kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("dtype", C.c_int),
        ("k_quant_type", C.c_int32), ("v_quant_type", C.c_int32),
    ]


class PaBatch(C.Structure):
    _fields_ = [
        ("cumulative_sequence_length", C.c_void_p), ("past_seqlens", C.c_void_p),
        ("block_table", C.c_void_p), ("slot_mapping", C.c_void_p),
        ("batch", C.c_int32), ("max_blocks", C.c_int32), ("num_tokens", C.c_int32),
        ("max_query_len", C.c_int32), ("flags", C.c_uint32), ("max_context_len", C.c_int32),
    ]


PA_BATCH_NEW_ROWS_IN_CACHE = 1
PA_BATCH_SLOTS_DISTINCT = 2


class PaAttn(C.Structure):
    _fields_ = [
        ("num_heads", C.c_int32), ("scale", C.c_float), ("softcap", C.c_float),
        ("local_window_size", C.c_int32), ("is_causal", C.c_int32), ("head_sink", C.c_void_p),
        ("v_head_size", C.c_int32),
    ]


class PaNode(C.Structure):
    _fields_ = [
        ("num_heads", C.c_int32), ("kv_num_heads", C.c_int32), ("scale", C.c_float),
        ("softcap", C.c_float), ("local_window_size", C.c_int32), ("do_rotary", C.c_int32),
        ("rotary_interleaved", C.c_int32), ("rotary_offset", C.c_int32),
        ("is_causal", C.c_int32), ("qk_norm_epsilon", C.c_float),
        ("v_head_size", C.c_int32), ("kv_cache_layout_latent", C.c_int32),
    ]


class PaIO(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("num_tokens", C.c_int32), ("query_hidden", C.c_int32),
        ("query", C.c_void_p), ("key", C.c_void_p), ("value", C.c_void_p),
        ("cache", PaCache),
        ("cumulative_sequence_length", C.c_void_p), ("past_seqlens", C.c_void_p),
        ("block_table", C.c_void_p), ("batch", C.c_int32), ("max_blocks", C.c_int32),
        ("cos_cache", C.c_void_p), ("sin_cache", C.c_void_p),
        ("rotary_positions", C.c_int64), ("rotary_half", C.c_int32),
        ("slot_mapping", C.c_void_p), ("head_sink", C.c_void_p),
        ("q_norm_weight", C.c_void_p), ("k_norm_weight", C.c_void_p),
        ("host_cumulative_sequence_length", C.c_void_p), ("host_past_seqlens", C.c_void_p),
        ("host_block_table", C.c_void_p), ("host_slot_mapping", C.c_void_p),
        ("output", C.c_void_p), ("key_cache_out", C.c_void_p), ("value_cache_out", C.c_void_p),
        ("max_query_len", C.c_int32), ("max_context_len", C.c_int32),
    ]


class PaGqaNode(C.Structure):
    _fields_ = [
        ("num_heads", C.c_int32), ("kv_num_heads", C.c_int32), ("scale", C.c_float),
        ("softcap", C.c_float), ("local_window_size", C.c_int32), ("do_rotary", C.c_int32),
        ("rotary_interleaved", C.c_int32), ("is_causal", C.c_int32),
        ("qk_norm_epsilon", C.c_float), ("smooth_softmax", C.c_int32),
        ("sliding_window_cache", C.c_int32), ("qk_output", C.c_int32),
    ]


class PaGqaIO(C.Structure):
    _fields_ = [
        ("dtype", C.c_int), ("batch", C.c_int32), ("seq", C.c_int32),
        ("query_hidden", C.c_int32), ("kv_seq", C.c_int32),
        ("query", C.c_void_p), ("key", C.c_void_p), ("value", C.c_void_p),
        ("past_key", C.c_void_p), ("past_value", C.c_void_p), ("past_capacity", C.c_int32),
        ("present_key", C.c_void_p), ("present_value", C.c_void_p),
        ("present_capacity", C.c_int32),
        ("seqlens_k", C.c_void_p), ("host_seqlens_k", C.c_void_p),
        ("total_sequence_length", C.c_int64),
        ("cos_cache", C.c_void_p), ("sin_cache", C.c_void_p),
        ("rotary_positions", C.c_int64), ("rotary_half", C.c_int32),
        ("position_ids", C.c_void_p), ("host_position_ids", C.c_void_p),
        ("position_cols", C.c_int32),
        ("attention_bias", C.c_void_p), ("bias_batch", C.c_int32), ("bias_heads", C.c_int32),
        ("head_sink", C.c_void_p), ("q_norm_weight", C.c_void_p), ("k_norm_weight", C.c_void_p),
        ("output", C.c_void_p),
        ("cache_dtype", C.c_int), ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
        ("k_quant_type", C.c_int32), ("v_quant_type", C.c_int32),
        ("output_qk", C.c_void_p),
    ]


class PaGqaNodeInfo(C.Structure):
    _fields_ = [
        ("num_inputs", C.c_int32), ("num_outputs", C.c_int32),
        ("input_present", C.c_int32 * 16), ("input_dtype", C.c_int32 * 16),
        ("input_rank", C.c_int32 * 16), ("input_shape", (C.c_int64 * 4) * 16),
        ("output_present", C.c_int32 * 4), ("output_dtype", C.c_int32 * 4),
        ("output_rank", C.c_int32 * 4), ("output_shape", (C.c_int64 * 4) * 4),
        ("num_heads", C.c_int32), ("kv_num_heads", C.c_int32), ("do_rotary", C.c_int32),
        ("is_causal", C.c_int32), ("local_window_size", C.c_int32),
        ("sliding_window_cache", C.c_int32), ("kv_cache_bit_width", C.c_int32),
        ("smooth_softmax", C.c_int32), ("qk_output", C.c_int32), ("softcap", C.c_float),
        ("k_quant_type", C.c_int32), ("v_quant_type", C.c_int32),
    ]


class PaNodeInfo(C.Structure):
    _fields_ = [
        ("num_inputs", C.c_int32), ("num_outputs", C.c_int32),
        ("input_present", C.c_int32 * 17), ("input_dtype", C.c_int32 * 17),
        ("input_rank", C.c_int32 * 17), ("input_shape", (C.c_int64 * 4) * 17),
        ("output_present", C.c_int32 * 3), ("output_dtype", C.c_int32 * 3),
        ("output_rank", C.c_int32 * 3), ("output_shape", (C.c_int64 * 4) * 3),
        ("num_heads", C.c_int32), ("kv_num_heads", C.c_int32), ("v_head_size", C.c_int32),
        ("rotary_offset", C.c_int32), ("do_rotary", C.c_int32),
        ("local_window_size", C.c_int32), ("is_causal", C.c_int32),
        ("has_scale_attr", C.c_int32), ("softcap", C.c_float),
        ("kv_cache_layout_latent", C.c_int32),
        ("k_quant_type", C.c_int32), ("v_quant_type", C.c_int32),
        ("k_cache_dtype", C.c_int32), ("v_cache_dtype", C.c_int32),
    ]


class PagedAttentionError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero status; the message is pa_last_error()."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(the HIP extension is required; there is no fallback)")
    lib = C.CDLL(os.fspath(LIB_PATH))
    P, I32, I64, SZ = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
    sig = {
        "pa_last_error": (C.c_char_p, []),
        "pa_version": (C.c_char_p, []),
        "pa_pool_create": (C.c_int, [I64, I32, I32, I32, C.c_int, C.POINTER(P)]),
        "pa_pool_destroy": (C.c_int, [P]),
        "pa_pool_k_ptr": (P, [P]), "pa_pool_v_ptr": (P, [P]),
        "pa_pool_k_scale_ptr": (P, [P]), "pa_pool_v_scale_ptr": (P, [P]),
        "pa_pool_bytes": (I64, [P]),
        "pa_rotary_append": (C.c_int, [C.POINTER(PaCache), C.POINTER(PaBatch), I32, C.c_int,
                                       P, P, P, P, P, P, P, I64, I32, I32, I32, P, P, C.c_float,
                                       P]),
        "pa_reshape_and_cache": (C.c_int, [C.POINTER(PaCache), C.POINTER(PaBatch), C.c_int,
                                           P, P, P]),
        "pa_attention_workspace_bytes": (SZ, [C.POINTER(PaCache), C.POINTER(PaBatch),
                                              C.POINTER(PaAttn)]),
        "pa_attention_workspace_bytes_ex": (SZ, [C.POINTER(PaCache), C.POINTER(PaBatch),
                                                 C.POINTER(PaAttn), C.c_int, I32, I32]),
        "pa_attention": (C.c_int, [C.POINTER(PaCache), C.POINTER(PaBatch), C.POINTER(PaAttn),
                                   C.c_int, P, P, P, P, P, SZ, P]),
        "pa_attention_ex": (C.c_int, [C.POINTER(PaCache), C.POINTER(PaBatch), C.POINTER(PaAttn),
                                      C.c_int, P, P, P, P, P, SZ, I32, I32, P]),
        "pa_paged_attention_workspace_bytes": (SZ, [C.POINTER(PaNode), C.POINTER(PaIO)]),
        "pa_paged_attention": (C.c_int, [C.POINTER(PaNode), C.POINTER(PaIO), P, SZ, P]),
        "pa_paged_attention_static": (C.c_int, [C.POINTER(PaNode), C.POINTER(PaIO), P]),
        "pa_paged_attention_claim": (C.c_int, [C.POINTER(PaNodeInfo), C.c_char_p, SZ]),
        "pa_group_query_attention_workspace_bytes": (SZ, [C.POINTER(PaGqaNode),
                                                          C.POINTER(PaGqaIO)]),
        "pa_group_query_attention": (C.c_int, [C.POINTER(PaGqaNode), C.POINTER(PaGqaIO), P, SZ,
                                               P]),
        "pa_group_query_attention_claim": (C.c_int, [C.POINTER(PaGqaNodeInfo), C.c_char_p, SZ]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != PA_OK:
        msg = load().pa_last_error().decode("utf-8", "replace")
        raise PagedAttentionError(rc, msg)
