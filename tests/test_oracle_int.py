"""Pins of the oracle's integer (int8 / int4) KV-cache restatement (QuantizedCache,
kv_cache.rs:110-256), each independent of the oracle's own code:

- hand-derived codes for the reference's tie / saturation / zero-scale vectors
  (test_quantized_kv.py:478-491), for both widths and both encode rules;
- numpy float32 arithmetic (IEEE division / multiplication, np.rint half-to-even, np.clip)
  around exact rounding ties at adjacent float32 values (test_quantized_kv.py:322-341), which
  separates the paged divide rule from the GroupQueryAttention reciprocal rule;
- int4 nibble layout known bytes (test_quantized_kv.py:1-6 docstring: +8 bias, even channel
  low nibble, unused high nibble 8) and decode known values;
- exact round trips (codes times powers of two);
- cache-level invariants (only slot rows change) and fp64 attention over the decoded pages,
  plus the reference's known answer for a page written before any read
  (test_quantized_kv.py:539-556).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import F16, F32, I4, I8, PER_CHANNEL, PER_TENSOR
from pa_cases import int_scales, make_case

TIES = np.array([-1024, -128.5, -8.5, -7.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 6.5, 7.5, 126.5,
                 127.5, 1024, 0], np.float32)
# Codes at scale 1, derived by hand: clip to the range, round half to even.
TIES_I8 = [-128, -128, -8, -8, -2, -2, 0, 0, 2, 2, 6, 8, 126, 127, 127, 0]
TIES_I4 = [-8, -8, -8, -8, -2, -2, 0, 0, 2, 2, 6, 7, 7, 7, 7, 0]


@pytest.mark.parametrize("reciprocal", [False, True])
def test_int_code_ties_and_saturation(reciprocal):
    for bits, want in ((8, TIES_I8), (4, TIES_I4)):
        got = [orc.int_code(float(x), 1.0, bits, reciprocal) for x in TIES]
        assert got == want, (bits, got)


def test_int_code_zero_scale_rules():
    # paged: divide, zero scale -> code 0 (kv_cache.rs:186-188)
    for bits in (8, 4):
        assert [orc.int_code(float(x), 0.0, bits, False) for x in TIES] == [0] * len(TIES)
    # GQA: reciprocal of a zero scale is read as 1 (kv_cache.rs:180-181, 189-191)
    assert [orc.int_code(float(x), 0.0, 8, True) for x in TIES] == TIES_I8
    assert [orc.int_code(float(x), 0.0, 4, True) for x in TIES] == TIES_I4


def test_int_code_negative_ties_are_symmetric():
    for bits in (8, 4):
        lo, hi = (-128, 127) if bits == 8 else (-8, 7)
        for x in TIES:
            want = int(np.clip(np.rint(-np.float64(x)), lo, hi))  # -x is exact in float32
            assert orc.int_code(float(-x), 1.0, bits, False) == want


def _half_boundary_values(scale):
    centers = np.array([-128.5, -127.5, -8.5, -7.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 6.5, 7.5,
                        126.5, 127.5], np.float32) * np.float32(scale)
    return np.stack([np.nextafter(centers, -np.inf, dtype=np.float32), centers,
                     np.nextafter(centers, np.inf, dtype=np.float32)], -1).reshape(-1)


@pytest.mark.parametrize("scale", [0.3, 0.7, 1.1, -0.3])
@pytest.mark.parametrize("bits", [8, 4])
def test_int_code_matches_ieee_float32_at_rounding_ties(scale, bits):
    s = np.float32(scale)
    x = _half_boundary_values(s)
    lo, hi = (-128, 127) if bits == 8 else (-8, 7)
    paged = np.clip(np.rint(x / s), lo, hi).astype(int)                    # IEEE fp32 divide
    gqa = np.clip(np.rint(x * (np.float32(1) / s)), lo, hi).astype(int)    # fp32 reciprocal
    got_p = np.array([orc.int_code(float(v), float(s), bits, False) for v in x])
    got_g = np.array([orc.int_code(float(v), float(s), bits, True) for v in x])
    np.testing.assert_array_equal(got_p, paged)
    np.testing.assert_array_equal(got_g, gqa)


def test_divide_and_reciprocal_rules_disagree_somewhere():
    """The two encode rules differ at some tie-adjacent float32 inputs, so the tests above
    distinguish a divide from a reciprocal multiply."""
    diffs = 0
    for scale in (0.3, 0.7, 1.1, -0.3):
        s = np.float32(scale)
        for v in _half_boundary_values(s):
            diffs += orc.int_code(float(v), float(s), 8, False) != \
                orc.int_code(float(v), float(s), 8, True)
    assert diffs > 0


@pytest.mark.parametrize("codes,want", [
    ([-8, 7], [0xF0]), ([7, -8], [0x0F]), ([0, 0], [0x88]), ([1, 2, 3], [0xA9, 0x8B]),
    ([-1], [0x87]), ([3, -3, 5, -5], [0x5B, 0x3D]),
])
def test_int4_nibble_layout_known_bytes(codes, want):
    row = orc.int_encode_row(np.asarray(codes, np.float32), [1.0], 4)
    assert row.tolist() == want


def test_int8_row_is_twos_complement_codes():
    x = np.array([-128, -1, 0, 1, 127, 3.5, -3.5], np.float32)
    row = orc.int_encode_row(x, [1.0], 8)
    assert row.view(np.uint8).tolist() == [0x80, 0xFF, 0x00, 0x01, 0x7F, 0x04, 0xFC]


def test_int_decode_known_values():
    got8 = orc.int_decode_row(np.array([0x80, 0x7F, 0x00, 0xFF], np.uint8), 4, [0.5], 8)
    assert got8.tolist() == [-64.0, 63.5, 0.0, -0.5]
    got4 = orc.int_decode_row(np.array([0xA9, 0x8B], np.uint8), 3, [2.0], 4)
    assert got4.tolist() == [2.0, 4.0, 6.0]  # nibbles 9, 10, 11 minus 8, times 2; pad dropped
    per = orc.int_decode_row(np.array([0xF0], np.uint8), 2, [0.25, 3.0], 4, per_channel=True)
    assert per.tolist() == [-2.0, 21.0]


@pytest.mark.parametrize("bits,d", [(8, 16), (8, 128), (4, 16), (4, 7)])
@pytest.mark.parametrize("per_channel", [False, True])
def test_int_round_trip_exact(bits, d, per_channel):
    rng = np.random.default_rng(bits * 100 + d)
    lo, hi = (-128, 127) if bits == 8 else (-8, 7)
    codes = rng.integers(lo, hi + 1, d)
    scale = (2.0 ** rng.integers(-6, 3, d)).astype(np.float32) if per_channel else \
        np.array([0.125], np.float32)
    x = (codes * (scale if per_channel else scale[0])).astype(np.float32)
    for reciprocal in (False, True):  # powers of two: divide and reciprocal agree exactly
        row = orc.int_encode_row(x, scale, bits, per_channel, reciprocal)
        back = orc.int_decode_row(row, d, scale, bits, per_channel)
        np.testing.assert_array_equal(back, x)


def _reference_geometry(bits, head=16, modes=(PER_CHANNEL, PER_CHANNEL), seed=818, **kw):
    """The reference's integer PagedAttention geometry (test_quantized_kv.py:344-362): 4 heads,
    2 kv heads, 6 blocks of 4, three sequences with new lengths [2, 0, 1] and pasts [3, 1, 2]."""
    return make_case(4, 2, head, 6, 4, 3, dtype=F16, cache_dtype=I8 if bits == 8 else I4,
                     seed=seed, new_lens=[2, 0, 1], past=[3, 1, 2], max_blocks=2,
                     int_modes=modes, **kw)


@pytest.mark.parametrize("bits,head", [(8, 16), (4, 16), (4, 7)])
@pytest.mark.parametrize("modes", [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL),
                                   (PER_TENSOR, PER_CHANNEL)])
def test_int_append_changes_only_slot_rows(bits, head, modes):
    c = _reference_geometry(bits, head, modes)
    kc, vc = orc.reshape_and_cache(c["key"], c["value"], F16, c["key_cache"], c["value_cache"],
                                   c["cache_dtype"], c["cum"], c["past"], c["block_table"],
                                   k_scale=c["k_scale"], v_scale=c["v_scale"], k_mode=modes[0],
                                   v_mode=modes[1], head_dim=head)
    bs, KV = 4, 2
    touched = set()
    for b in range(3):
        for j in range(c["cum"][b + 1] - c["cum"][b]):
            pos = c["past"][b] + j
            slot = c["block_table"][b, pos // bs] * bs + pos % bs
            touched.add(slot)
            t = c["cum"][b] + j
            for kh in range(KV):
                for side, (cache, src, sc, mode) in enumerate((
                        (kc, c["key"], c["k_scale"], modes[0]),
                        (vc, c["value"], c["v_scale"], modes[1]))):
                    x = orc.decode(src[t, kh * head:(kh + 1) * head], F16)
                    pc = mode == PER_CHANNEL
                    want = orc.int_encode_row(x, sc[kh] if pc else sc, bits, pc)
                    np.testing.assert_array_equal(cache[slot // bs, slot % bs, kh], want)
    flat_k = kc.reshape(-1, KV, kc.shape[-1])
    old_k = c["key_cache"].reshape(-1, KV, kc.shape[-1])
    for slot in range(flat_k.shape[0]):
        if slot not in touched:
            np.testing.assert_array_equal(flat_k[slot], old_k[slot])


def _decoded_cache(cache, scale, mode, bits, head):
    nb, bs, KV, _ = cache.shape
    out = np.empty((nb, bs, KV, head), np.float32)
    for i in range(nb):
        for j in range(bs):
            for kh in range(KV):
                pc = mode == PER_CHANNEL
                out[i, j, kh] = orc.int_decode_row(cache[i, j, kh], head,
                                                   scale[kh] if pc else scale, bits, pc)
    return out


def _fp64_reference(c, kc, vc, head, softcap=0.0, window=-1, causal=1, sink=None):
    """softmax(scale q.k) v in float64 over every position read from the decoded pages."""
    bits = 8 if c["cache_dtype"] == I8 else 4
    K = _decoded_cache(kc, c["k_scale"], c["k_quant"], bits, head).astype(np.float64)
    V = _decoded_cache(vc, c["v_scale"], c["v_quant"], bits, head).astype(np.float64)
    H, KV, bs = c["num_heads"], c["kv_num_heads"], kc.shape[1]
    q = orc.decode(c["query"], F16).astype(np.float64).reshape(-1, H, head)
    out = np.zeros((q.shape[0], H * head))
    scale = 1.0 / np.sqrt(np.float32(head))
    for b in range(len(c["cum"]) - 1):
        s0, s1 = c["cum"][b], c["cum"][b + 1]
        total = c["past"][b] + s1 - s0
        pos = np.arange(total)
        rows = (c["block_table"][b, pos // bs], pos % bs)
        for i, t in enumerate(range(s0, s1)):
            rp = c["past"][b] + i
            vis = np.ones(total, bool)
            if causal:
                vis &= pos <= rp
            if window > 0:
                vis &= pos >= rp - window + 1
            for h in range(H):
                kh = h // (H // KV)
                logits = (K[rows][:, kh] @ q[t, h]) * float(np.float32(scale))
                if softcap:
                    cap = float(np.float32(softcap))  # the fp32 attribute value
                    logits = cap * np.tanh(logits / cap)
                logits = np.where(vis, logits, -np.inf)
                m = logits.max() if sink is None else max(logits.max(), sink[h])
                w = np.exp(logits - m)
                den = w.sum() + (0.0 if sink is None else np.exp(sink[h] - m))
                out[t, h * head:(h + 1) * head] = (w @ V[rows][:, kh]) / den
    return out


@pytest.mark.parametrize("bits,head", [(8, 16), (4, 16), (4, 7)])
@pytest.mark.parametrize("modes", [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL)])
@pytest.mark.parametrize("causal,window,softcap", [(1, -1, 0.0), (0, 2, 0.7)])
def test_int_attention_matches_fp64_over_decoded_pages(bits, head, modes, causal, window,
                                                       softcap):
    c = _reference_geometry(bits, head, modes, causal=causal, window=window, softcap=softcap)
    out, _, kc, vc = orc.paged_attention_op(c)
    ref = _fp64_reference(c, kc, vc, head, softcap, window, causal)
    np.testing.assert_allclose(out, ref, rtol=1e-9, atol=1e-9)


def test_int_attention_reads_new_rows_quantised_from_the_pages():
    """Known answer (test_quantized_kv.py:539-556): every page starts at code 0 (0x88 for int4),
    q = k = 0 and v = 1 at scale 1, token 1 writes slot 0, token 0 and 2 skip; every read sees
    v = 1 wherever slot 0 is visible, so the first output row is exactly 1."""
    for bits in (8, 4):
        c = _reference_geometry(bits, 16, (PER_TENSOR, PER_TENSOR), slot_mapping=[-1, 0, -1])
        c["cum"] = np.array([0, 1, 1, 3], np.int32)
        c["past"] = np.zeros(3, np.int32)
        c["block_table"] = np.zeros((3, 2), np.int32)
        for name in ("key_cache", "value_cache"):
            c[name] = np.full_like(c[name], 0 if bits == 8 else 0x88)
        c["query"] = orc.encode(np.zeros((3, 4 * 16)), F16)
        c["key"] = orc.encode(np.zeros((3, 2 * 16)), F16)
        c["value"] = orc.encode(np.ones((3, 2 * 16)), F16)
        c["k_scale"] = np.array([1.0], np.float32)
        c["v_scale"] = np.array([1.0], np.float32)
        out, out_t, _, _ = orc.paged_attention_op(c)
        assert np.all(out[0] == 1.0)


def test_gqa_int_cache_uses_the_reciprocal_rule():
    """GroupQueryAttention integer caches: the rows written equal the reciprocal-rule encode,
    which differs from the paged divide rule where a per-channel scale is zero."""
    rng = np.random.default_rng(5)
    B, S, H, KV, d, cap = 2, 2, 4, 2, 32, 6
    for bits in (8, 4):
        width = d if bits == 8 else d // 2
        q = orc.encode(rng.standard_normal((B, S, H * d)), F32)
        k = orc.encode(rng.standard_normal((B, S, KV * d)), F32)
        v = orc.encode(rng.standard_normal((B, S, KV * d)), F32)
        raw = np.int8 if bits == 8 else np.uint8
        pk = rng.integers(-128 if bits == 8 else 0, 128 if bits == 8 else 256,
                          (B, KV, cap, width)).astype(raw)
        pv = pk.copy()
        ks, vs = int_scales(KV, d, PER_CHANNEL, 0), int_scales(KV, d, PER_CHANNEL, 1)
        seqlens = np.array([3, 5], np.int32)
        out, pk2, pv2 = orc.gqa_contiguous(F32, q, k, v, pk, pv, seqlens, H, KV, d, 0.125,
                                           cache_dtype=I8 if bits == 8 else I4, k_scale=ks,
                                           v_scale=vs, k_mode=PER_CHANNEL, v_mode=PER_CHANNEL)
        zero_channel_seen = False
        for b in range(B):
            past = seqlens[b] + 1 - S
            for j in range(S):
                for kh in range(KV):
                    x = k[b, j, kh * d:(kh + 1) * d]
                    want = orc.int_encode_row(x, ks[kh], bits, True, True)
                    np.testing.assert_array_equal(pk2[b, kh, past + j], want)
                    divide = orc.int_encode_row(x, ks[kh], bits, True, False)
                    zero_channel_seen |= not np.array_equal(want, divide)
        assert zero_channel_seen
        assert np.isfinite(out).all()
