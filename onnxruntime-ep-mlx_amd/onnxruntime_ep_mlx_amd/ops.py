"""torch-facing mirror of the com.microsoft::PagedAttention operator on MI355X.

``paged_attention`` takes the operator's inputs in the reference's order and meaning
(query, key, value, key_cache, value_cache, cumulative_sequence_length, past_seqlens,
block_table, cos_cache, sin_cache, slot_mapping, head_sink, q_norm_weight, k_norm_weight,
k_scale, v_scale, attention_metadata; rust/src/ops/attention.rs:3857-4382) and its attributes
(num_heads, kv_num_heads, scale, softcap, local_window_size, do_rotary, rotary_interleaved,
rotary_offset, is_causal, qk_norm_epsilon).  Caches are updated in place, as the reference
writes ORT's input buffers back (engine.rs:1212-1357); the return value is
(output, key_cache, value_cache) so callers can bind the optional cache outputs to the same
storage.  torch only provides device memory and the stream; all compute runs in
libonnxruntime_ep_mlx_amd.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _capi as capi

_DTYPES = {
    torch.float16: capi.PA_DTYPE_FLOAT16,
    torch.bfloat16: capi.PA_DTYPE_BFLOAT16,
    torch.float32: capi.PA_DTYPE_FLOAT32,
    torch.float8_e4m3fn: capi.PA_DTYPE_FP8_E4M3,
    # integer cache storage (kv_cache.rs:8-13): int8 codes, uint8 = two int4 codes per byte
    torch.int8: capi.PA_DTYPE_INT8,
    torch.uint8: capi.PA_DTYPE_INT4,
}


def pa_dtype(t: torch.dtype) -> int:
    try:
        return _DTYPES[t]
    except KeyError:
        raise TypeError(f"PagedAttention: unsupported dtype {t}") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _need_cuda(name: str, t: torch.Tensor | None) -> None:
    if t is not None and not t.is_cuda:
        raise ValueError(f"PagedAttention: {name} must be a device tensor")


def _contig(name: str, t: torch.Tensor | None) -> None:
    if t is not None and not t.is_contiguous():
        raise ValueError(f"PagedAttention: {name} must be contiguous")


@dataclass
class _Workspace:
    buf: torch.Tensor | None = None

    def get(self, nbytes: int, device: torch.device) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        return self.buf


_ws = _Workspace()


def _quant(mode) -> int:
    if isinstance(mode, str):
        if mode not in capi.QUANT_TYPES:
            raise ValueError(f"unknown quantization type {mode!r}")
        return capi.QUANT_TYPES[mode]
    return int(mode)


def cache_desc(key_cache: torch.Tensor, value_cache: torch.Tensor,
               k_scale: torch.Tensor | None = None,
               v_scale: torch.Tensor | None = None, *, head_dim: int | None = None,
               k_quant_type="NONE", v_quant_type="NONE") -> capi.PaCache:
    """Cache descriptor.  Integer caches (torch.int8 / torch.uint8 = int4) take fp32 scales
    with k_quant_type / v_quant_type "PER_TENSOR" ([1]) or "PER_CHANNEL" ([kv_heads, head]);
    an int4 cache's last dimension is ceil(head / 2), so pass head_dim for odd heads."""
    if key_cache.dim() != 4 or (value_cache is not None and key_cache.shape != value_cache.shape):
        raise ValueError("key_cache must be [num_blocks,block_size,kv_num_heads,head_size]")
    if value_cache is not None and key_cache.dtype != value_cache.dtype:
        raise ValueError("key/value caches must share one storage dtype")
    nb, bs, kv, width = key_cache.shape
    dt = pa_dtype(key_cache.dtype)
    if head_dim is None:
        head_dim = 2 * width if dt == capi.PA_DTYPE_INT4 else width
    elif (head_dim + 1) // 2 != width if dt == capi.PA_DTYPE_INT4 else head_dim != width:
        raise ValueError("key_cache must be [num_blocks,block_size,kv_num_heads,head_size]")
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if t is not None:
            if t.dtype != torch.float32:
                raise ValueError(f"{name} must be float32")
            _need_cuda(name, t)
            _contig(name, t)
    return capi.PaCache(_ptr(key_cache), _ptr(value_cache), _ptr(k_scale), _ptr(v_scale),
                        nb, bs, kv, head_dim, dt, _quant(k_quant_type), _quant(v_quant_type))


def batch_desc(cum: torch.Tensor, past: torch.Tensor, block_table: torch.Tensor,
               num_tokens: int, slot_mapping: torch.Tensor | None = None,
               max_query_len: int = 0, flags: int = 0,
               max_context_len: int = 0) -> capi.PaBatch:
    for name, t in (("cumulative_sequence_length", cum), ("past_seqlens", past),
                    ("block_table", block_table), ("slot_mapping", slot_mapping)):
        if t is not None and t.dtype != torch.int32:
            raise ValueError(f"input {name} must be int32")
        _contig(name, t)
    return capi.PaBatch(_ptr(cum), _ptr(past), _ptr(block_table), _ptr(slot_mapping),
                        cum.numel() - 1, block_table.shape[1], num_tokens, max_query_len, flags,
                        max_context_len)


def attn_desc(num_heads: int, scale: float = 0.0, softcap: float = 0.0,
              local_window_size: int = -1, is_causal: int = 1,
              head_sink: torch.Tensor | None = None) -> capi.PaAttn:
    return capi.PaAttn(num_heads, scale, softcap, local_window_size, is_causal, _ptr(head_sink))


class PagePool:
    """HBM page pool behind the cache tensors (pa_pool_*); exposes K/V as torch views."""

    def __init__(self, num_blocks: int, block_size: int, kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device: torch.device | str = "cuda"):
        lib = capi.load()
        self.device = torch.device(device)
        self.head_dim = head_dim
        width = (head_dim + 1) // 2 if dtype == torch.uint8 else head_dim  # int4: two per byte
        self.shape = (num_blocks, block_size, kv_heads, width)
        self.dtype = dtype
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            capi.check(lib.pa_pool_create(num_blocks, block_size, kv_heads, head_dim,
                                          pa_dtype(dtype), C.byref(h)))
        self._h = h
        self.key_cache = self._view(lib.pa_pool_k_ptr(h), self.shape, dtype)
        self.value_cache = self._view(lib.pa_pool_v_ptr(h), self.shape, dtype)
        self.k_scale = self.v_scale = None
        if dtype == torch.float8_e4m3fn:
            self.k_scale = self._view(lib.pa_pool_k_scale_ptr(h), (num_blocks, kv_heads),
                                      torch.float32)
            self.v_scale = self._view(lib.pa_pool_v_scale_ptr(h), (num_blocks, kv_heads),
                                      torch.float32)

    def _view(self, ptr: int, shape, dtype) -> torch.Tensor:
        # Wrap the pool's device memory as a tensor without copying (DLPack-free: a
        # storage from the raw pointer via torch's UntypedStorage is not public, so use
        # the __cuda_array_interface__ protocol).
        n = 1
        for s in shape:
            n *= s
        itemsize = torch.empty((), dtype=dtype).element_size()
        holder = _DevPtr(ptr, n * itemsize, self.device)
        raw = torch.as_tensor(holder, device=self.device)
        return raw.view(dtype).view(*shape)

    def close(self) -> None:
        if getattr(self, "_h", None):
            torch.cuda.synchronize(self.device)
            capi.load().pa_pool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _DevPtr:
    """Minimal __cuda_array_interface__ exporter for a raw device allocation (uint8)."""

    def __init__(self, ptr: int, nbytes: int, device: torch.device):
        self.__cuda_array_interface__ = {
            "shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 3,
            "strides": None, "stream": None,
        }


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, cum: torch.Tensor, past: torch.Tensor,
                      block_table: torch.Tensor, slot_mapping: torch.Tensor | None = None,
                      k_scale: torch.Tensor | None = None,
                      v_scale: torch.Tensor | None = None, slots_distinct: bool = False, *,
                      k_quant_type="NONE", v_quant_type="NONE") -> None:
    """Append key/value rows to the pages (last writer wins on shared slots unless the caller
    asserts `slots_distinct`, which skips that check)."""
    lib = capi.load()
    for n, t in (("key", key), ("value", value), ("key_cache", key_cache)):
        _need_cuda(n, t)
        _contig(n, t)
    kv = key_cache.shape[2]
    cache = cache_desc(key_cache, value_cache, k_scale, v_scale,
                       head_dim=key.shape[-1] // kv, k_quant_type=k_quant_type,
                       v_quant_type=v_quant_type)
    batch = batch_desc(cum, past, block_table, key.shape[0], slot_mapping, 0,
                       capi.PA_BATCH_SLOTS_DISTINCT if slots_distinct else 0)
    capi.check(lib.pa_reshape_and_cache(C.byref(cache), C.byref(batch), pa_dtype(key.dtype),
                                        _ptr(key), _ptr(value), _stream(key.device)))


def rotary_append(query, key, value, key_cache, value_cache, cum, past, block_table, *,
                  num_heads, cos_cache=None, sin_cache=None, rotary_offset=0,
                  rotary_interleaved=0, q_norm_weight=None, k_norm_weight=None,
                  qk_norm_epsilon=1e-6, slot_mapping=None, k_scale=None, v_scale=None,
                  slots_distinct=False, k_quant_type="NONE", v_quant_type="NONE"):
    """Fused RMSNorm + RoPE + append.  Returns the transformed (query, key) rows."""
    lib = capi.load()
    cache = cache_desc(key_cache, value_cache, k_scale, v_scale,
                       head_dim=key.shape[-1] // key_cache.shape[2], k_quant_type=k_quant_type,
                       v_quant_type=v_quant_type)
    batch = batch_desc(cum, past, block_table, key.shape[0], slot_mapping, 0,
                       capi.PA_BATCH_SLOTS_DISTINCT if slots_distinct else 0)
    transform = cos_cache is not None or q_norm_weight is not None
    q_out = torch.empty_like(query) if transform else query
    k_out = torch.empty_like(key) if transform else key
    rot_pos = cos_cache.shape[0] if cos_cache is not None else 0
    rot_half = cos_cache.shape[1] if cos_cache is not None else 0
    capi.check(lib.pa_rotary_append(
        C.byref(cache), C.byref(batch), num_heads, pa_dtype(query.dtype), _ptr(query),
        _ptr(key), _ptr(value), _ptr(q_out) if transform else None,
        _ptr(k_out) if transform else None, _ptr(cos_cache), _ptr(sin_cache), rot_pos,
        rot_half, rotary_offset, rotary_interleaved, _ptr(q_norm_weight), _ptr(k_norm_weight),
        qk_norm_epsilon, _stream(query.device)))
    return q_out, k_out


def attention(q, k_new, v_new, key_cache, value_cache, cum, past, block_table, *, num_heads,
              scale=0.0, softcap=0.0, local_window_size=-1, is_causal=1, head_sink=None,
              k_scale=None, v_scale=None, max_query_len=0, kind=0, chunk=0, out=None,
              new_rows_in_cache=False, k_quant_type="NONE", v_quant_type="NONE",
              max_context_len=0):
    """Attention over the (already appended) paged cache; kind/chunk force a kernel family.
    new_rows_in_cache: the caller appended k_new/v_new into distinct block-table slots.
    max_context_len: bound on every sequence's past + new tokens (0 = the block-table capacity)."""
    lib = capi.load()
    cache = cache_desc(key_cache, value_cache, k_scale, v_scale,
                       head_dim=q.shape[-1] // num_heads, k_quant_type=k_quant_type,
                       v_quant_type=v_quant_type)
    batch = batch_desc(cum, past, block_table, q.shape[0], None, max_query_len,
                       capi.PA_BATCH_NEW_ROWS_IN_CACHE if new_rows_in_cache else 0,
                       max_context_len)
    attn = attn_desc(num_heads, scale, softcap, local_window_size, is_causal, head_sink)
    act = pa_dtype(q.dtype)
    nbytes = lib.pa_attention_workspace_bytes_ex(C.byref(cache), C.byref(batch), C.byref(attn),
                                                 act, kind, chunk)
    ws = _ws.get(nbytes, q.device)
    if out is None:
        out = torch.empty_like(q)
    capi.check(lib.pa_attention_ex(C.byref(cache), C.byref(batch), C.byref(attn), act, _ptr(q),
                                   _ptr(k_new), _ptr(v_new), _ptr(out), _ptr(ws), nbytes, kind,
                                   chunk, _stream(q.device)))
    return out


def paged_attention(query, key, value, key_cache, value_cache, cumulative_sequence_length,
                    past_seqlens, block_table, cos_cache=None, sin_cache=None,
                    slot_mapping=None, head_sink=None, q_norm_weight=None, k_norm_weight=None,
                    k_scale=None, v_scale=None, attention_metadata=None, *, num_heads,
                    kv_num_heads, scale=0.0, softcap=0.0, local_window_size=-1, do_rotary=0,
                    rotary_interleaved=0, rotary_offset=0, is_causal=1, qk_norm_epsilon=1e-6,
                    k_quant_type="NONE", v_quant_type="NONE", v_head_size=0,
                    kv_cache_layout="SEPARATE", validate=True, output=None,
                    key_cache_out=None, value_cache_out=None, max_query_len=0,
                    max_context_len=0, static_scratch=False):
    """com.microsoft::PagedAttention on MI355X (operator-level entry, pa_paged_attention).

    ``attention_metadata`` is accepted and ignored, like the reference
    (test_attention_contracts.py:338-367).  With ``validate`` the int32 metadata is copied to
    the host and checked with the reference's rules (attention.rs:3934-3990), which is what the
    reference does every step; without it the device copies are trusted.  ``key`` and
    ``value`` both None means packed QKV: ``query`` is [T, (num_heads + 2 kv_num_heads) * head].
    Integer caches (torch.int8, torch.uint8 = int4) take ``k_scale``/``v_scale`` with
    ``k_quant_type``/``v_quant_type`` "PER_TENSOR" or "PER_CHANNEL".
    ``kv_cache_layout="LATENT"``: one kv head, ``value`` and ``value_cache`` None; the values are
    the first ``v_head_size`` dims of the (rotated) key rows and the output is
    [T, num_heads * v_head_size].
    Outputs 1/2: the input caches are always updated in place; ``key_cache_out`` /
    ``value_cache_out`` given as tensors of their own receive a copy of the updated caches
    (outputs bound onto the inputs need nothing), and are returned in place of the inputs.
    ``max_query_len`` (0 = derive it) bounds every sequence's new tokens: it picks the kernel
    family without a device read when ``validate`` is False.  ``max_context_len`` (0 = derive
    it from the host metadata, else the block-table capacity) bounds every sequence's past + new
    tokens: it sizes the operand images of multi-token batches by the live context.
    ``static_scratch``: call pa_paged_attention_static, which allocates nothing (its workspace
    is the library's per-GPU static scratch, shared by every call on that GPU).
    """
    if kv_cache_layout not in ("SEPARATE", "LATENT"):
        raise ValueError("kv_cache_layout must be SEPARATE or LATENT")
    latent = kv_cache_layout == "LATENT"
    del attention_metadata
    lib = capi.load()
    if query.dim() != 2:
        raise ValueError("query must have rank 2")
    for n, t in (("query", query), ("key", key), ("value", value), ("key_cache", key_cache),
                 ("value_cache", value_cache), ("key_cache_out", key_cache_out),
                 ("value_cache_out", value_cache_out)):
        _need_cuda(n, t)
        _contig(n, t)
    for n, out_t, in_t in (("key_cache_out", key_cache_out, key_cache),
                           ("value_cache_out", value_cache_out, value_cache)):
        if out_t is not None and (in_t is None or out_t.shape != in_t.shape
                                  or out_t.dtype != in_t.dtype):
            raise ValueError(f"PagedAttention: {n} must match its cache's shape and dtype")
    packed = not latent and key is None and value is None
    head = query.shape[1] // (num_heads + 2 * kv_num_heads if packed else num_heads)
    v_head = v_head_size or head
    node = capi.PaNode(num_heads, kv_num_heads, scale, softcap, local_window_size, do_rotary,
                       rotary_interleaved, rotary_offset, is_causal, qk_norm_epsilon,
                       v_head_size, int(latent))
    host = {}
    if validate:
        for name, t in (("cum", cumulative_sequence_length), ("past", past_seqlens),
                        ("bt", block_table), ("slots", slot_mapping)):
            host[name] = None if t is None else t.detach().to("cpu").contiguous()
    if output is None:
        output = query.new_empty((query.shape[0], num_heads * v_head))
    cache = cache_desc(key_cache, value_cache, k_scale, v_scale, head_dim=head,
                       k_quant_type=k_quant_type, v_quant_type=v_quant_type)
    io = capi.PaIO(
        pa_dtype(query.dtype), query.shape[0], query.shape[1], _ptr(query), _ptr(key),
        _ptr(value), cache, _ptr(cumulative_sequence_length), _ptr(past_seqlens),
        _ptr(block_table), cumulative_sequence_length.numel() - 1, block_table.shape[1],
        _ptr(cos_cache) if do_rotary else None, _ptr(sin_cache) if do_rotary else None,
        cos_cache.shape[0] if (do_rotary and cos_cache is not None) else 0,
        cos_cache.shape[1] if (do_rotary and cos_cache is not None) else 0,
        _ptr(slot_mapping), _ptr(head_sink), _ptr(q_norm_weight), _ptr(k_norm_weight),
        _ptr(host.get("cum")), _ptr(host.get("past")), _ptr(host.get("bt")),
        _ptr(host.get("slots")), _ptr(output), _ptr(key_cache_out), _ptr(value_cache_out),
        max_query_len, max_context_len)
    if static_scratch:
        capi.check(lib.pa_paged_attention_static(C.byref(node), C.byref(io),
                                                 _stream(query.device)))
    else:
        nbytes = lib.pa_paged_attention_workspace_bytes(C.byref(node), C.byref(io))
        ws = _ws.get(nbytes, query.device)
        capi.check(lib.pa_paged_attention(C.byref(node), C.byref(io), _ptr(ws), nbytes,
                                          _stream(query.device)))
    return (output, key_cache if key_cache_out is None else key_cache_out,
            value_cache if value_cache_out is None else value_cache_out)


def group_query_attention(query, key, value, past_key, past_value, seqlens_k,
                          total_sequence_length, cos_cache=None, sin_cache=None,
                          position_ids=None, attention_bias=None, head_sink=None, k_scale=None,
                          v_scale=None, q_norm_weight=None, k_norm_weight=None, *, num_heads,
                          kv_num_heads, scale=0.0, softcap=0.0, local_window_size=-1,
                          do_rotary=0, rotary_interleaved=0, is_causal=1, qk_norm_epsilon=1e-6,
                          smooth_softmax=0, k_quant_type="NONE", v_quant_type="NONE",
                          present="new", present_key=None, present_value=None, validate=True,
                          output=None, sliding_window_cache=0, qk_output=0, output_qk=None):
    """com.microsoft::GroupQueryAttention on MI355X (pa_group_query_attention), inputs in the
    operator's order (query, key, value, past_key, past_value, seqlens_k,
    total_sequence_length, cos_cache, sin_cache, position_ids, attention_bias, head_sink,
    k_scale, v_scale, q_norm_weight, k_norm_weight; attention.rs:932-1454).

    ``key``/``value`` None: packed QKV query [B, S, (H + 2 KV) * head].  ``key``/``value`` with
    a zero-length sequence axis: no new rows (the past is attended as is).  ``past_key`` None:
    the first prompt, no past.  Integer caches (torch.int8, or torch.uint8 = int4 rows of
    ceil(head / 2) bytes) take ``k_scale``/``v_scale`` with "PER_TENSOR" / "PER_CHANNEL".
    ``present`` selects outputs 1/2: "new" allocates [B, KV, max(past capacity, total), row]
    (the operator's own contract), "shared" updates ``past_key``/``past_value`` in place
    (outputs bound onto the inputs: capacity stays), "omitted" returns None for both;
    ``present_key``/``present_value`` given explicitly are used as the "new" buffers.
    ``validate``: copy seqlens_k (and position_ids) to the host for the reference's checks.
    ``sliding_window_cache``: the caches are rings of the past capacity (``local_window_size``
    > 0); "new" presents then take the past's capacity.  ``qk_output`` 1 / 2 writes the
    scores / probabilities [B, H, S, total] into ``output_qk`` (allocated when None).
    Returns (output, present_key, present_value), plus output_qk when ``qk_output`` is set."""
    lib = capi.load()
    if query.dim() != 3:
        raise ValueError("query must have rank 3 [batch, sequence, hidden]")
    if present not in ("new", "shared", "omitted"):
        raise ValueError("present must be 'new', 'shared' or 'omitted'")
    for n, t in (("query", query), ("key", key), ("value", value), ("past_key", past_key),
                 ("past_value", past_value), ("k_scale", k_scale), ("v_scale", v_scale),
                 ("position_ids", position_ids), ("attention_bias", attention_bias),
                 ("present_key", present_key), ("present_value", present_value)):
        _need_cuda(n, t)
        _contig(n, t)
    if seqlens_k.dtype != torch.int32:
        raise ValueError("input seqlens_k must be int32")
    if position_ids is not None and position_ids.dtype != torch.int64:
        raise ValueError("GroupQueryAttention: position_ids must be int64 [batch,>=sequence]")
    B, S = query.shape[0], query.shape[1]
    packed = key is None and value is None
    head = query.shape[2] // (num_heads + 2 * kv_num_heads if packed else num_heads)
    kv_seq = S if packed else key.shape[1]
    total = int(total_sequence_length)
    # without a past the caches use the activation dtype (kv_cache.rs:24)
    cache_dt = past_key.dtype if past_key is not None else query.dtype
    width = (head + 1) // 2 if cache_dt == torch.uint8 else head
    past_cap = past_key.shape[2] if past_key is not None else 0
    if present == "shared":
        if past_key is None:
            raise ValueError("GroupQueryAttention: present='shared' needs past_key/past_value")
        present_key, present_value = past_key, past_value
    elif present == "new" and present_key is None:
        shape = (B, kv_num_heads, past_cap if sliding_window_cache else max(past_cap, total), width)
        present_key = torch.empty(shape, dtype=cache_dt, device=query.device)
        present_value = torch.empty(shape, dtype=cache_dt, device=query.device)
    elif present == "omitted":
        present_key = present_value = None
    host = seqlens_k.detach().to("cpu").contiguous() if validate else None
    host_pid = (position_ids.detach().to("cpu").contiguous()
                if validate and position_ids is not None else None)
    if output is None:
        output = query.new_empty((B, S, num_heads * head))
    cache_code = 0 if cache_dt == query.dtype else pa_dtype(cache_dt)
    if qk_output and output_qk is None:
        output_qk = query.new_empty((B, num_heads, S, total))
    node = capi.PaGqaNode(num_heads, kv_num_heads, scale, softcap, local_window_size, do_rotary,
                          rotary_interleaved, is_causal, qk_norm_epsilon, smooth_softmax,
                          int(sliding_window_cache), int(qk_output))
    rot = do_rotary and cos_cache is not None
    io = capi.PaGqaIO(
        dtype=pa_dtype(query.dtype), batch=B, seq=S, query_hidden=query.shape[2], kv_seq=kv_seq,
        query=_ptr(query), key=_ptr(key), value=_ptr(value), past_key=_ptr(past_key),
        past_value=_ptr(past_value), past_capacity=past_cap, present_key=_ptr(present_key),
        present_value=_ptr(present_value),
        present_capacity=present_key.shape[2] if present_key is not None else 0,
        seqlens_k=_ptr(seqlens_k), host_seqlens_k=_ptr(host), total_sequence_length=total,
        cos_cache=_ptr(cos_cache) if do_rotary else None,
        sin_cache=_ptr(sin_cache) if do_rotary else None,
        rotary_positions=cos_cache.shape[0] if rot else 0,
        rotary_half=cos_cache.shape[1] if rot else 0,
        position_ids=_ptr(position_ids), host_position_ids=_ptr(host_pid),
        position_cols=position_ids.shape[1] if position_ids is not None else 0,
        attention_bias=_ptr(attention_bias),
        bias_batch=attention_bias.shape[0] if attention_bias is not None else 0,
        bias_heads=attention_bias.shape[1] if attention_bias is not None else 0,
        head_sink=_ptr(head_sink), q_norm_weight=_ptr(q_norm_weight),
        k_norm_weight=_ptr(k_norm_weight), output=_ptr(output), cache_dtype=cache_code,
        k_scale=_ptr(k_scale), v_scale=_ptr(v_scale), k_quant_type=_quant(k_quant_type),
        v_quant_type=_quant(v_quant_type), output_qk=_ptr(output_qk) if qk_output else None)
    if attention_bias is not None and (attention_bias.dim() != 4
                                       or attention_bias.shape[2] != S
                                       or attention_bias.shape[3] != total):
        raise ValueError("GroupQueryAttention: attention_bias must broadcast to "
                         "[batch,heads,sequence,total]")
    nbytes = lib.pa_group_query_attention_workspace_bytes(C.byref(node), C.byref(io))
    ws = _ws.get(max(nbytes, 1), query.device)
    capi.check(lib.pa_group_query_attention(C.byref(node), C.byref(io), _ptr(ws), nbytes,
                                            _stream(query.device)))
    if qk_output:
        return output, present_key, present_value, output_qk
    return output, present_key, present_value


def group_query_attention_claim(info: "capi.PaGqaNodeInfo") -> tuple[bool, str]:
    """pa_group_query_attention_claim: (claimed, reason)."""
    buf = C.create_string_buffer(512)
    ok = capi.load().pa_group_query_attention_claim(C.byref(info), buf, len(buf))
    return bool(ok), buf.value.decode()
