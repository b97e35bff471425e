"""Workspace sizing of multi-token batches over operand images (host only, no GPU).

The planned prefill writes operand images (fp16 key and value rows laid out as the kernel's LDS
operands, 32 KiB per 64-key step of every (sequence, kv-head) at head 128) into the workspace.
They are sized by the live context of the call -- the host metadata's longest past + new tokens,
the caller's max_context_len, or GroupQueryAttention's total_sequence_length -- not by the
block-table or present capacity.  These cases check that the image region is planned and has the
live size, and that a region beyond the 2 GiB image limit (byte-coded pages: int8 / int4 / fp8)
is planned for groups of sequences that fit it rather than dropped.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from onnxruntime_ep_mlx_amd import _capi as capi

FAKE = 0x1000  # device pointers are never dereferenced by the size queries
STEP_BYTES = 2 * 64 * 128 * 2  # one 64-key image step at head 128 (keys + values, fp16)


def _gqa(total, cap, B=8, S=512, H=32, KV=8, d=128, cache=capi.PA_DTYPE_INT8):
    host = np.full(B, total - 1, np.int32)
    node = capi.PaGqaNode(H, KV, 0.0, 0.0, -1, 0, 0, 1, 1e-6, 0)
    io = capi.PaGqaIO(dtype=capi.PA_DTYPE_BFLOAT16, batch=B, seq=S, query_hidden=H * d,
                      kv_seq=S, query=FAKE, key=FAKE, value=FAKE, past_key=FAKE,
                      past_value=FAKE + 64, past_capacity=cap, present_key=FAKE,
                      present_value=FAKE + 64, present_capacity=cap, seqlens_k=FAKE,
                      host_seqlens_k=host.ctypes.data, total_sequence_length=total,
                      output=FAKE, cache_dtype=cache, k_scale=FAKE, v_scale=FAKE,
                      k_quant_type=capi.PA_QUANT_PER_CHANNEL,
                      v_quant_type=capi.PA_QUANT_PER_CHANNEL)
    return node, io, host


def test_gqa_integer_present_images_follow_total_not_capacity():
    """Advisor case: batch 8, kv 8, capacity 131072, head 128, a 2048-key call: the images are
    8 * 8 * 32 steps (64 MiB), not 8 * 8 * 2048 steps (4 GiB, beyond the image limit)."""
    lib = capi.load()
    B, KV, total, cap = 8, 8, 2048, 131072
    node, io, keep = _gqa(total, cap, B=B, KV=KV)
    n = lib.pa_group_query_attention_workspace_bytes(C.byref(node), C.byref(io))
    live = B * KV * (total // 64) * STEP_BYTES
    assert live <= n < live + (256 << 20), n
    # the same call at a small capacity plans the same images
    node2, io2, keep2 = _gqa(total, total, B=B, KV=KV)
    n2 = lib.pa_group_query_attention_workspace_bytes(C.byref(node2), C.byref(io2))
    assert abs(n - n2) < (1 << 20), (n, n2)


def _paged(past, nq, max_blocks, bs=16, KV=8, H=64, d=128, host=True, bound=0,
           cache=capi.PA_DTYPE_FP8_E4M3):
    B = len(past)
    cum = np.concatenate([[0], np.cumsum([nq] * B)]).astype(np.int32)
    past = np.asarray(past, np.int32)
    nb = B * max_blocks
    bt = np.arange(nb, dtype=np.int32).reshape(B, max_blocks)
    keep = [cum, past, bt]
    c = capi.PaCache(FAKE, FAKE, FAKE, FAKE, nb, bs, KV, d, cache)
    T = int(cum[-1])
    io = capi.PaIO(capi.PA_DTYPE_BFLOAT16, T, H * d, FAKE, FAKE, FAKE, c, FAKE, FAKE, FAKE,
                   B, max_blocks, None, None, 0, 0, None, None, None, None,
                   cum.ctypes.data if host else None, past.ctypes.data if host else None,
                   bt.ctypes.data if host else None, None, FAKE, None, None,
                   nq if not host else 0, bound)
    node = capi.PaNode(H, KV, 0.0, 0.0, -1, 0, 0, 0, 1, 1e-6)
    return node, io, keep


def test_paged_fp8_images_follow_live_context_with_host_metadata():
    """fp8 pages, batch 16, kv 8, a 65,536-position block table (4096 pages of 16) and live
    contexts of at most 1,064 keys: 17 image steps per (sequence, kv-head)."""
    lib = capi.load()
    past = [1000, 40, 700, 3] * 4
    node, io, keep = _paged(past, 64, 4096)
    n = lib.pa_paged_attention_workspace_bytes(C.byref(node), C.byref(io))
    live = 16 * 8 * -(-(1000 + 64) // 64) * STEP_BYTES
    assert live <= n < live + (256 << 20), n


def test_paged_images_follow_the_callers_context_bound():
    lib = capi.load()
    past = [1000, 40, 700, 3] * 4
    node, io, keep = _paged(past, 64, 4096, host=False, bound=1064)
    n = lib.pa_paged_attention_workspace_bytes(C.byref(node), C.byref(io))
    live = 16 * 8 * 17 * STEP_BYTES
    assert live <= n < live + (256 << 20), n
    # without a bound the images cover the block-table capacity (65,536 positions: 1,024 steps,
    # 256 MiB per sequence), 4 GiB for the batch: the planned launch runs on groups of 8
    # sequences, the workspace holding the images of one group (2 GiB) and its plan
    node0, io0, keep0 = _paged(past, 64, 4096, host=False, bound=0)
    n0 = lib.pa_paged_attention_workspace_bytes(C.byref(node0), C.byref(io0))
    group = 8 * 8 * 1024 * STEP_BYTES
    assert group == 1 << 31
    assert group <= n0 < group + (64 << 20), n0


def test_context_bound_below_the_host_metadata_is_refused():
    lib = capi.load()
    node, io, keep = _paged([1000, 40], 64, 128, bound=500)
    rc = lib.pa_paged_attention(C.byref(node), C.byref(io), C.c_void_p(0x2000), 1 << 40, None)
    msg = lib.pa_last_error().decode()
    assert rc == capi.PA_ERR_INVALID_ARGUMENT and "max_context_len" in msg, msg
    node, io, keep = _paged([1000, 40], 64, 128, bound=-1)
    rc = lib.pa_paged_attention(C.byref(node), C.byref(io), C.c_void_p(0x2000), 1 << 40, None)
    assert rc == capi.PA_ERR_INVALID_ARGUMENT
