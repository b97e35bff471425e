"""Host-side GroupQueryAttention logic (CPU only, no device work): the claim predicate
pa_group_query_attention_claim (group_query_attention_claim, attention.rs:2407-2628, plus
kv_cache::claim kv_cache.rs:16-108) and the operator's input checks that fail before any device
call (gqa_batched's length rules :614-631, :665-672, the rotary rows :523-584, the bias shape
:636-655, the present capacity of a growing cache :632).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from onnxruntime_ep_mlx_amd import _capi as capi
from onnxruntime_ep_mlx_amd import group_query_attention_claim

BF16, F32 = capi.PA_DTYPE_BFLOAT16, capi.PA_DTYPE_FLOAT32
I32, I64 = capi.PA_INT32_DTYPE, capi.PA_INT64_DTYPE


def _node(B=4, S=1, H=32, KV=8, d=128, cap=4096, dtype=BF16, rotary=True, packed=False,
          past=True, present=True, cache_dtype=None):
    """A Llama-shaped decode node: query [B, S, H*d], key/value [B, S, KV*d], past/present
    [B, KV, cap, d], seqlens_k [B], total [1], cos/sin [8192, d/2]."""
    n = capi.PaGqaNodeInfo()
    cache_dtype = dtype if cache_dtype is None else cache_dtype
    width = (d + 1) // 2 if cache_dtype == capi.PA_UINT8_DTYPE else d
    shapes = {0: [B, S, (H + 2 * KV) * d if packed else H * d], 1: [B, S, KV * d],
              2: [B, S, KV * d], 3: [B, KV, cap, width], 4: [B, KV, cap, width], 5: [B],
              6: [1], 7: [8192, d // 2], 8: [8192, d // 2]}
    dts = {0: dtype, 1: dtype, 2: dtype, 3: cache_dtype, 4: cache_dtype, 5: I32, 6: I32,
           7: dtype, 8: dtype}
    n.num_inputs = 9 if rotary else 7
    for i in range(n.num_inputs):
        if (packed and i in (1, 2)) or (not past and i in (3, 4)):
            continue
        n.input_present[i] = 1
        n.input_dtype[i] = dts[i]
        n.input_rank[i] = len(shapes[i])
        for j, s in enumerate(shapes[i]):
            n.input_shape[i][j] = s
    n.num_outputs = 3 if present else 1
    for o in range(n.num_outputs):
        n.output_present[o] = 1
        n.output_dtype[o] = dtype if o == 0 else cache_dtype
    n.output_rank[0] = 3
    n.num_heads, n.kv_num_heads = H, KV
    n.do_rotary = int(rotary)
    n.is_causal = 1
    n.local_window_size = -1
    return n


def _set_input(n, i, dtype, shape):
    n.num_inputs = max(n.num_inputs, i + 1)
    n.input_present[i] = 1
    n.input_dtype[i] = dtype
    n.input_rank[i] = len(shape)
    for j, s in enumerate(shape):
        n.input_shape[i][j] = s


def test_claim_accepts_decode_prefill_packed_and_first_prompt():
    assert group_query_attention_claim(_node()) == (True, "")
    assert group_query_attention_claim(_node(S=64, cap=8192))[0]
    assert group_query_attention_claim(_node(packed=True))[0]
    assert group_query_attention_claim(_node(past=False, S=128))[0]
    assert group_query_attention_claim(_node(present=False))[0]


def test_claim_accepts_optional_inputs():
    n = _node(B=2, S=3)
    _set_input(n, 9, I64, [2, 8])                  # position_ids [B, >= S]
    _set_input(n, 10, BF16, [2, 1, 3, 4096])       # attention_bias
    _set_input(n, 11, BF16, [32])                  # head_sink
    _set_input(n, 14, BF16, [128])                 # q_norm_weight
    _set_input(n, 15, BF16, [128])                 # k_norm_weight
    n.smooth_softmax = 1
    n.softcap = 30.0
    assert group_query_attention_claim(n) == (True, "")


def test_claim_accepts_integer_caches():
    for storage, bits in ((capi.PA_INT8_DTYPE, 8), (capi.PA_UINT8_DTYPE, 4)):
        n = _node(cache_dtype=storage)
        n.kv_cache_bit_width = bits
        n.k_quant_type = n.v_quant_type = capi.PA_QUANT_PER_CHANNEL
        _set_input(n, 12, F32, [8, 128])
        _set_input(n, 13, F32, [8, 128])
        assert group_query_attention_claim(n) == (True, ""), bits


def _with(mutate):
    n = _node()
    mutate(n)
    return n


@pytest.mark.parametrize("mutate,reason", [
    # sliding_window_cache and output_qk rules (attention.rs:2455-2473, :2589-2590, :2730-2748)
    (lambda n: setattr(n, "sliding_window_cache", 1),
     "sliding_window_cache=1 requires local_window_size > 0"),
    (lambda n: (setattr(n, "sliding_window_cache", 1), setattr(n, "local_window_size", 64),
                setattr(n, "num_outputs", 1)),
     "sliding_window_cache requires present key/value outputs"),
    (lambda n: (setattr(n, "sliding_window_cache", 1), setattr(n, "local_window_size", 8192)),
     "sliding-window key cache capacity must be at least local_window_size"),
    (lambda n: (setattr(n, "sliding_window_cache", 1), setattr(n, "local_window_size", 64),
                n.input_shape[4].__setitem__(2, 32)),
     "sliding-window value cache capacity must be at least local_window_size"),
    (lambda n: (setattr(n, "sliding_window_cache", 1), setattr(n, "local_window_size", 64),
                n.input_shape[3].__setitem__(2, -1)),
     "sliding-window key cache capacity must be at least local_window_size"),
    (lambda n: (setattr(n, "sliding_window_cache", 1), setattr(n, "local_window_size", 64),
                setattr(n, "qk_output", 1), setattr(n, "num_outputs", 4),
                n.output_present.__setitem__(3, 1), n.output_dtype.__setitem__(3, BF16),
                n.output_rank.__setitem__(3, 4)),
     "sliding_window_cache with QK diagnostics is unsupported"),
    (lambda n: (setattr(n, "qk_output", 2), setattr(n, "num_outputs", 4),
                n.output_present.__setitem__(3, 1), n.output_dtype.__setitem__(3, BF16),
                n.output_rank.__setitem__(3, 4), n.output_shape[3].__setitem__(1, 16)),
     "output_qk must be [batch,num_heads,sequence_length,total_sequence_length]"),
    (lambda n: (setattr(n, "qk_output", 1), setattr(n, "num_outputs", 4),
                n.output_present.__setitem__(3, 1), n.output_dtype.__setitem__(3, F32),
                n.output_rank.__setitem__(3, 4)),
     "output_qk must be [batch,num_heads,sequence_length,total_sequence_length]"),
    # the reference's own reasons
    (lambda n: setattr(n, "num_outputs", 5), "requires 1 to 4 outputs"),
    (lambda n: n.output_present.__setitem__(2, 0), "present_key and present_value must both"),
    (lambda n: setattr(n, "is_causal", 2), "causal must be 0 or 1"),
    (lambda n: setattr(n, "local_window_size", 0), "local_window_size must be -1 or positive"),
    (lambda n: (setattr(n, "is_causal", 0), setattr(n, "local_window_size", 8)),
     "bidirectional GroupQueryAttention requires local_window_size=-1"),
    (lambda n: n.input_present.__setitem__(4, 0), "past_key and past_value must be provided"),
    (lambda n: n.output_dtype.__setitem__(0, capi.PA_DTYPE_FP8_E4M3), "MLX float dtype"),
    (lambda n: (setattr(n, "num_inputs", 7)), "7-input GroupQueryAttention requires do_rotary=0"),
    (lambda n: n.input_present.__setitem__(2, 0), "Q/K/V must be either all separate or packed"),
    (lambda n: n.input_dtype.__setitem__(1, capi.PA_DTYPE_FLOAT16), "input 1 must have"),
    (lambda n: n.input_dtype.__setitem__(5, I64), "input 5 must have int32 dtype"),
    (lambda n: setattr(n, "kv_num_heads", 5), "positive multiple of kv_num_heads"),
    (lambda n: n.input_shape[0].__setitem__(2, 4001), "query hidden size must match head count"),
    (lambda n: setattr(n, "kv_cache_bit_width", 8), "kv_cache_bit_width must agree"),
    (lambda n: n.input_shape[1].__setitem__(2, 512), "key/value must match query batch"),
    (lambda n: n.input_shape[3].__setitem__(1, 4), "past cache must be [batch,kv_num_heads"),
    (lambda n: n.input_shape[4].__setitem__(2, 100), "past key/value cache shapes must match"),
    (lambda n: n.input_rank.__setitem__(6, 2), "total_sequence_length must be scalar or [1]"),
    (lambda n: (n.input_shape[7].__setitem__(1, 80), n.input_shape[8].__setitem__(1, 80)),
     "rotary caches must have matching"),
    (lambda n: _set_input(n, 9, I32, [4, 1]), "position_ids must be int64"),
    (lambda n: _set_input(n, 10, BF16, [4, 1, 1]), "attention_bias (input 10) must have rank 4"),
    (lambda n: _set_input(n, 10, BF16, [4, 3, 1, 10]), "attention_bias must broadcast"),
    (lambda n: _set_input(n, 11, BF16, [16]), "head_sink must be [num_heads]"),
    (lambda n: _set_input(n, 14, BF16, [128]), "input 15 lacks tensor type/shape info"),
    (lambda n: _set_input(n, 15, BF16, [128]), "q_norm_weight and k_norm_weight"),
    (lambda n: (_set_input(n, 14, BF16, [64]), _set_input(n, 15, BF16, [64])),
     "Q/K norm weight 14 must have shape [head_size=128]"),
    (lambda n: setattr(n, "smooth_softmax", 2), "smooth_softmax must be -1"),
    (lambda n: setattr(n, "qk_output", 1), "enabled exactly when output_qk is present"),
    (lambda n: setattr(n, "softcap", float("inf")), "softcap must be finite"),
    (lambda n: n.input_dtype.__setitem__(3, capi.PA_INT8_DTYPE),
     "output 1 must retain its cache dtype"),
    (lambda n: [a.__setitem__(i, capi.PA_INT8_DTYPE)
                for a, i in ((n.input_dtype, 3), (n.input_dtype, 4), (n.output_dtype, 1),
                             (n.output_dtype, 2))],
     "integer k cache requires PER_TENSOR or PER_CHANNEL quantization"),
])
def test_claim_declines_with_reasons(mutate, reason):
    ok, why = group_query_attention_claim(_with(mutate))
    assert not ok and reason in why, why


def test_claim_accepts_sliding_and_qk_forms():
    n = _node()
    n.sliding_window_cache, n.local_window_size = 1, 4096
    assert group_query_attention_claim(n)[0]
    for mode in (1, 2):
        n = _node()
        n.qk_output, n.num_outputs = mode, 4
        n.output_present[3] = 1
        n.output_dtype[3] = BF16
        n.output_rank[3] = 4
        for j, v in enumerate([4, 32, 1, -1]):  # total_sequence_length symbolic
            n.output_shape[3][j] = v
        assert group_query_attention_claim(n)[0], group_query_attention_claim(n)[1]


def test_claim_sliding_integer_alignment():
    """Sliding integer rings need 16-byte rows (attention.rs:2589-2590): head % 16 for int8,
    head % 32 for int4."""
    for bits, dt, head, ok in ((8, capi.PA_INT8_DTYPE, 16, True), (8, capi.PA_INT8_DTYPE, 24, False),
                               (4, capi.PA_UINT8_DTYPE, 32, True), (4, capi.PA_UINT8_DTYPE, 48, False),
                               (4, capi.PA_UINT8_DTYPE, 16, False)):
        n = _node(cache_dtype=dt, d=head, rotary=False)
        n.kv_cache_bit_width = bits
        n.k_quant_type = n.v_quant_type = capi.PA_QUANT_PER_TENSOR
        _set_input(n, 12, F32, [1])
        _set_input(n, 13, F32, [1])
        n.sliding_window_cache, n.local_window_size = 1, 8
        got, why = group_query_attention_claim(n)
        assert got == ok, (bits, head, why)
        if not ok:
            assert "pinned 16-byte alignment" in why, why


def test_claim_integer_cache_rules():
    n = _node(cache_dtype=capi.PA_UINT8_DTYPE, d=127)
    n.input_shape[0][2] = 32 * 127
    for i in (1, 2):
        n.input_shape[i][2] = 8 * 127
    n.kv_cache_bit_width = 4
    n.k_quant_type = n.v_quant_type = capi.PA_QUANT_PER_TENSOR
    _set_input(n, 12, F32, [1])
    _set_input(n, 13, F32, [1])
    for i in (7, 8):
        n.input_shape[i][1] = 63
    ok, why = group_query_attention_claim(n)
    assert not ok and "even logical head size" in why, why
    n = _node(cache_dtype=capi.PA_INT8_DTYPE)
    n.kv_cache_bit_width = 8
    n.k_quant_type = n.v_quant_type = capi.PA_QUANT_PER_CHANNEL
    _set_input(n, 12, F32, [8, 64])
    _set_input(n, 13, F32, [8, 128])
    ok, why = group_query_attention_claim(n)
    assert not ok and "k_scale must contain 1024 elements" in why, why


# ------------------------------------------------------------------ operator input checks
FAKE = 0x1000  # never dereferenced: every case below fails before any device work


def _io(B=2, S=1, H=8, KV=2, d=64, seqlens=(9, 5), total=None, cap=32, present_cap=None,
        shared=True, kv_seq=None, past=True):
    host = np.asarray(seqlens, np.int32)
    total = int(host.max()) + 1 if total is None else total
    node = capi.PaGqaNode(H, KV, 0.0, 0.0, -1, 0, 0, 1, 1e-6, 0)
    pres = FAKE if shared else FAKE + 0x10000
    io = capi.PaGqaIO(dtype=BF16, batch=B, seq=S, query_hidden=H * d,
                      kv_seq=S if kv_seq is None else kv_seq, query=FAKE, key=FAKE, value=FAKE,
                      past_key=FAKE if past else None, past_value=FAKE + 64 if past else None,
                      past_capacity=cap if past else 0, present_key=pres,
                      present_value=pres + 64,
                      present_capacity=(max(cap if past else 0, total) if present_cap is None
                                        else present_cap),
                      seqlens_k=FAKE, host_seqlens_k=host.ctypes.data,
                      total_sequence_length=total, output=FAKE)
    return node, io, host


def _run(node, io):
    lib = capi.load()
    nbytes = lib.pa_group_query_attention_workspace_bytes(C.byref(node), C.byref(io))
    rc = lib.pa_group_query_attention(C.byref(node), C.byref(io), C.c_void_p(FAKE),
                                      max(nbytes, 1), None)
    return rc, lib.pa_last_error().decode()


def test_growing_present_must_have_the_grown_capacity():
    node, io, keep = _io(seqlens=(40, 5), cap=32, shared=False, present_cap=32)
    rc, err = _run(node, io)
    assert rc != 0 and "max(past capacity,total_sequence_length)" in err, err


def test_shared_present_cannot_grow():
    node, io, keep = _io(seqlens=(40, 5), cap=40, shared=True)
    io.past_capacity = 32
    rc, err = _run(node, io)
    assert rc != 0 and "exceeds available past cache" in err, err


def test_first_prompt_needs_no_past_but_later_calls_do():
    node, io, keep = _io(S=4, seqlens=(9, 5), past=False, shared=False)
    rc, err = _run(node, io)
    assert rc != 0 and "exceeds available past cache" in err, err  # past 6 without a past


def test_ragged_lengths_only_on_the_first_prompt():
    # total != S and a length below S
    node, io, keep = _io(S=4, seqlens=(9, 1), cap=16)
    rc, err = _run(node, io)
    assert rc != 0 and "invalid per-batch or maximum sequence lengths" in err, err


def test_empty_key_value_needs_a_past():
    node, io, keep = _io(kv_seq=0, past=False, shared=False)
    rc, err = _run(node, io)
    assert rc != 0 and "K/V must match Q sequence or be empty" in err, err


def test_position_ids_outside_the_rotary_rows():
    node, io, keep = _io(S=2, seqlens=(9, 5), cap=16)
    node.do_rotary = 1
    io.cos_cache = io.sin_cache = FAKE
    io.rotary_positions, io.rotary_half = 64, 32
    pid = np.array([[3, 4], [63, 64]], np.int64)  # flat form: 64 is past the last row
    io.position_ids, io.host_position_ids, io.position_cols = FAKE, pid.ctypes.data, 2
    rc, err = _run(node, io)
    assert rc != 0 and "position_ids exceed the supplied cache" in err, err
    # first prompt (total == S): only pid[0] is read, as an offset
    node, io, keep2 = _io(S=4, seqlens=(3, 3), past=False, shared=False)
    node.do_rotary = 1
    io.cos_cache = io.sin_cache = FAKE
    io.rotary_positions, io.rotary_half = 64, 32
    pid = np.array([[61, 0, 0, 0], [0, 0, 0, 0]], np.int64)
    io.position_ids, io.host_position_ids, io.position_cols = FAKE, pid.ctypes.data, 4
    rc, err = _run(node, io)
    assert rc != 0 and "position_ids exceed the supplied cache" in err, err


def test_rotary_positions_beyond_the_cache():
    node, io, keep = _io(S=1, seqlens=(30, 5), cap=32)
    node.do_rotary = 1
    io.cos_cache = io.sin_cache = FAKE
    io.rotary_positions, io.rotary_half = 16, 32
    rc, err = _run(node, io)
    assert rc != 0 and "requested positions exceed the supplied cache" in err, err


def test_bias_must_broadcast():
    node, io, keep = _io()
    io.attention_bias, io.bias_batch, io.bias_heads = FAKE, 2, 3
    rc, err = _run(node, io)
    assert rc != 0 and "attention_bias must broadcast" in err, err
