"""MI355X (gfx950) paged GQA KV-cache attention behind the com.microsoft::PagedAttention surface.

The compute lives in lib/libonnxruntime_ep_mlx_amd.so (hand-written HIP kernels behind a C ABI,
include/pa_mi355x.h).  This package is a thin ctypes + torch mirror of the operator interface;
importing it loads the library and fails loudly if it has not been built.
"""
from . import _capi
from ._capi import PagedAttentionError, load
from .ops import (PagePool, attention, group_query_attention, group_query_attention_claim,
                  paged_attention, pa_dtype,
                  reshape_and_cache, rotary_append)

load()

__all__ = [
    "PagePool", "PagedAttentionError", "attention", "group_query_attention",
    "group_query_attention_claim", "load", "pa_dtype",
    "paged_attention",
    "reshape_and_cache", "rotary_append", "_capi",
]
