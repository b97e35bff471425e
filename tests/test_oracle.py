"""Pins for the CPU oracle (CPU only).

The reference ships no golden vectors for this path (every input is seeded at test time), so
each oracle function is pinned by something other than its own formula:
  converters  -> numpy / torch dtype casts (and every 16-bit / 8-bit pattern)
  RoPE        -> torch-CPU fp16/bf16 arithmetic evaluating the reference's rotate_half
                 formulation (test_paged_attention.py:29-48), special angles, fp64 rotation
  RMSNorm     -> the reference's numpy formula in float64 (test_paged_attention.py:101-103)
  append      -> byte invariants and the reference's duplicate-slot known answer
                 (test_paged_attention.py:605-659), skip/overwrite slot rules
  attention   -> torch fp64 scaled_dot_product_attention, closed forms (single key, uniform
                 keys, two-key softcap, sink), block-table relabelling and GQA==MHA invariance
  fp8         -> torch.float8_e4m3fn casts
  GQA (C1)    -> torch fp64 SDPA and equivalence with the paged restatement
  CPU baseline-> the fp64 contiguous restatement at fp32 tolerance
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import _oracle as orc
from _oracle import BF16, E4M3, F16, F32
from pa_cases import make_case


# ------------------------------------------------------------------------------ converters
def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 5.96e-8, 2.98e-8,
            6.1e-5, 3.0e38, -3.0e38, float("inf"), float("-inf"), 1.00390625, 1.01171875]
    rng = np.random.default_rng(0)
    r = np.concatenate([
        np.array(vals, np.float32),
        rng.standard_normal(20000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),
        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    return r[np.isfinite(r) | np.isinf(r)]


def test_bf16_encode_matches_torch():
    x = _special_f32()
    ours = orc.encode(x, BF16)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


def test_bf16_decode_all_patterns():
    raw = np.arange(2**16, dtype=np.uint32).astype(np.uint16)
    ours = orc.decode(raw, BF16)
    theirs = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16).float().numpy()
    finite = np.isfinite(theirs)
    assert np.array_equal(ours[finite], theirs[finite])
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))


def test_f16_encode_matches_numpy():
    x = _special_f32()
    ours = orc.encode(x, F16)
    theirs = x.astype(np.float16)
    assert np.array_equal(ours.view(np.uint16)[~np.isnan(theirs)],
                          theirs.view(np.uint16)[~np.isnan(theirs)])
    # exact halfway cases between adjacent halves, including subnormals
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    assert np.array_equal(orc.encode(mids, F16).view(np.uint16),
                          mids.astype(np.float16).view(np.uint16))


def test_f16_decode_all_patterns():
    raw = np.arange(2**16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    ours = orc.decode(raw, F16)
    theirs = raw.astype(np.float32)
    finite = np.isfinite(theirs)
    assert np.array_equal(ours[finite], theirs[finite])
    assert np.array_equal(np.isinf(ours), np.isinf(theirs))


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = orc.decode(codes, E4M3)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(theirs)
    assert np.array_equal(ours[ok], theirs[ok])
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    assert orc.decode(np.array([0x7e], np.uint8), E4M3)[0] == 448.0


def test_e4m3_encode_matches_torch_in_range_and_saturates():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(50000) * 50, rng.standard_normal(50000) * 0.01,
                        np.array([0.0, -0.0, 448.0, -448.0, 2.0**-9, 2.0**-10, 3 * 2.0**-10])])
    x = x.astype(np.float32)
    x = x[np.abs(x) <= 448]
    ours = orc.encode(x, E4M3)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)
    big = np.array([449.0, 1e6, float("inf"), -500.0, -float("inf")], np.float32)
    assert list(orc.encode(big, E4M3)) == [0x7e, 0x7e, 0x7e, 0xfe, 0xfe]
    assert orc.encode(np.array([np.nan], np.float32), E4M3)[0] == 0x7f


# ------------------------------------------------------------------------------ RoPE
def _ref_rope_torch(x, cos, sin, pos, interleaved, tdt):
    """The reference's _apply_rope (test_paged_attention.py:29-48) in torch tensors of the
    activation dtype: x * c + rotate_half(x) * s, every op rounding to that dtype."""
    x = torch.as_tensor(x).to(tdt)
    c, s = torch.as_tensor(cos[pos]).to(tdt), torch.as_tensor(sin[pos]).to(tdt)
    if not interleaved:
        c = torch.cat([c, c], -1)
        s = torch.cat([s, s], -1)
        d = x.shape[-1] // 2
        rot = torch.cat([-x[..., d:], x[..., :d]], -1)
    else:
        c = torch.repeat_interleave(c, 2, -1)
        s = torch.repeat_interleave(s, 2, -1)
        rot = torch.empty_like(x)
        rot[..., 0::2] = -x[..., 1::2]
        rot[..., 1::2] = x[..., 0::2]
    return x * c[:, None, :] + rot * s[:, None, :]


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("interleaved", [0, 1])
@pytest.mark.parametrize("theta", [10000.0, 500000.0])
def test_rope_matches_reference_formula_in_dtype(dtype, interleaved, theta):
    from pa_cases import rotary_cache
    rng = np.random.default_rng(7)
    rows, heads, d = 40, 3, 64
    x = orc.encode(rng.standard_normal((rows, heads, d)) * 2, dtype)
    cos, sin = rotary_cache(5000, d, theta, dtype)
    pos = rng.integers(0, 5000, rows).astype(np.int32)
    ours = orc.rope_rows(x, heads, d, pos, cos, sin, 0, interleaved, dtype)
    tdt = torch.float16 if dtype == F16 else torch.bfloat16
    want = _ref_rope_torch(orc.decode(x, dtype), orc.decode(cos, dtype), orc.decode(sin, dtype),
                           pos, interleaved, tdt)
    want_raw = orc.encode(want.float().numpy(), dtype)
    assert np.array_equal(ours, want_raw)


def test_rope_special_angles_and_offset():
    rng = np.random.default_rng(8)
    d, half = 32, 8
    x = orc.encode(rng.standard_normal((2, 1, d)), BF16)
    one, zero = orc.encode(np.ones((1, half)), BF16), orc.encode(np.zeros((1, half)), BF16)
    pos = np.zeros(2, np.int32)
    same = orc.rope_rows(x, 1, d, pos, one, zero, 8, 0, BF16)
    assert np.array_equal(same, x)  # angle 0 is the identity
    quarter = orc.rope_rows(x, 1, d, pos, zero, one, 8, 0, BF16)
    xf, qf = orc.decode(x, BF16), orc.decode(quarter, BF16)
    assert np.array_equal(qf[..., 8:16], -xf[..., 16:24])  # o1 = -x2
    assert np.array_equal(qf[..., 16:24], xf[..., 8:16])   # o2 = x1
    assert np.array_equal(qf[..., :8], xf[..., :8]) and np.array_equal(qf[..., 24:], xf[..., 24:])


def test_rope_fp32_is_a_rotation():
    rng = np.random.default_rng(9)
    d = 64
    x = rng.standard_normal((16, 2, d)).astype(np.float32)
    ang = rng.uniform(0, 2 * np.pi, (16, d // 2))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    out = orc.rope_rows(x, 2, d, np.arange(16), cos, sin, 0, 0, F32)
    x64 = x.astype(np.float64)
    c, s = cos.astype(np.float64)[:, None], sin.astype(np.float64)[:, None]
    want = np.concatenate([x64[..., :32] * c - x64[..., 32:] * s,
                           x64[..., 32:] * c + x64[..., :32] * s], -1)
    assert np.max(np.abs(out - want)) < 1e-5
    assert np.allclose(np.linalg.norm(out, axis=-1), np.linalg.norm(x64, axis=-1), rtol=1e-5)


def test_rms_norm_matches_reference_numpy_formula():
    rng = np.random.default_rng(10)
    d = 64
    x = orc.encode(rng.standard_normal((8, 4, d)), F16)
    w = orc.encode(np.linspace(0.75, 1.25, d), F16)
    ours = orc.decode(orc.rms_norm_rows(x, 4, d, w, 1e-5, F16), F16)
    xf = orc.decode(x, F16).astype(np.float64)
    want = xf / np.sqrt(np.mean(xf * xf, -1, keepdims=True) + 1e-5) * orc.decode(w, F16)
    assert np.max(np.abs(ours - want) / (np.abs(want) + 1e-3)) < 2 * 2.0**-10


# ------------------------------------------------------------------------------ append
def _append_case(seed, **kw):
    return make_case(4, 2, 16, 12, 4, 3, dtype=F16, seed=seed, **kw)


def test_append_writes_exactly_the_slot_rows():
    c = _append_case(3)
    kc, vc = orc.reshape_and_cache(c["key"], c["value"], F16, c["key_cache"], c["value_cache"],
                                   F16, c["cum"], c["past"], c["block_table"])
    bs = 4
    touched = np.zeros(c["key_cache"].shape[:2], bool)
    for b in range(3):
        for j in range(c["cum"][b + 1] - c["cum"][b]):
            p = c["past"][b] + j
            blk, off = c["block_table"][b, p // bs], p % bs
            touched[blk, off] = True
            t = c["cum"][b] + j
            assert np.array_equal(kc[blk, off].reshape(-1).view(np.uint16),
                                  c["key"][t].view(np.uint16))
            assert np.array_equal(vc[blk, off].reshape(-1).view(np.uint16),
                                  c["value"][t].view(np.uint16))
    assert np.array_equal(kc[~touched].view(np.uint16), c["key_cache"][~touched].view(np.uint16))
    assert np.array_equal(vc[~touched].view(np.uint16),
                          c["value_cache"][~touched].view(np.uint16))


def test_append_duplicate_slots_known_answer():
    # test_paged_attention.py:605-659: two tokens into slot 0 -> key 2s and value 4s remain
    kc = np.zeros((2, 16, 1, 64), np.float16)
    vc = np.zeros_like(kc)
    k = np.stack([np.full(64, 1), np.full(64, 2)]).astype(np.float16)
    v = np.stack([np.full(64, 3), np.full(64, 4)]).astype(np.float16)
    kc2, vc2 = orc.reshape_and_cache(k, v, F16, kc, vc, F16, np.array([0, 2], np.int32),
                                     np.array([0], np.int32), np.array([[0, 1]], np.int32),
                                     slot_mapping=np.array([0, 0], np.int32))
    assert np.all(kc2[0, 0, 0] == 2) and np.all(vc2[0, 0, 0] == 4)
    assert np.all(kc2[0, 1:] == 0) and np.all(kc2[1] == 0)


def test_append_skip_slots_leave_cache_untouched():
    c = _append_case(4)
    T = c["query"].shape[0]
    kc, vc = orc.reshape_and_cache(c["key"], c["value"], F16, c["key_cache"], c["value_cache"],
                                   F16, c["cum"], c["past"], c["block_table"],
                                   slot_mapping=np.full(T, -1, np.int32))
    assert np.array_equal(kc.view(np.uint16), c["key_cache"].view(np.uint16))


def test_append_fp8_quantises_with_block_scales():
    rng = np.random.default_rng(12)
    kc = np.zeros((4, 4, 2, 8), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.array([[0.5, 0.0], [1.0, 2.0], [0.25, 4.0], [1.0, 1.0]], np.float32)
    vs = ks[::-1].copy()
    k = orc.encode(rng.standard_normal((2, 16)) * 3, BF16)
    v = orc.encode(rng.standard_normal((2, 16)) * 3, BF16)
    slots = np.array([5, 9], np.int32)  # blocks 1 and 2
    kc2, vc2 = orc.reshape_and_cache(k, v, BF16, kc, vc, E4M3, np.array([0, 2], np.int32),
                                     np.array([0], np.int32), np.array([[0, 1, 2, 3]], np.int32),
                                     slot_mapping=slots, k_scale=ks, v_scale=vs)
    kf = orc.decode(k, BF16).reshape(2, 2, 8)
    for t, slot in enumerate(slots):
        blk, off = divmod(int(slot), 4)
        for h in range(2):
            sc = ks[blk, h]
            want = (np.zeros(8, np.uint8) if sc == 0 else torch.from_numpy(
                np.clip(kf[t, h] / sc, -448, 448).astype(np.float32)).to(
                torch.float8_e4m3fn).view(torch.uint8).numpy())
            assert np.array_equal(kc2[blk, off, h], want)


# ------------------------------------------------------------------------------ attention
def _torch_sdpa_reference(case):
    """Independent evaluation: gather per-sequence keys (cache for p < past, new rows after),
    repeat KV heads, torch fp64 scaled_dot_product_attention with an explicit mask."""
    c = case
    H, KV, d = c["num_heads"], c["kv_num_heads"], c["head_dim"]
    dt = c["dtype"]
    kc, vc = orc.reshape_and_cache(c["key"], c["value"], dt, c["key_cache"], c["value_cache"],
                                   dt, c["cum"], c["past"], c["block_table"],
                                   slot_mapping=c.get("slot_mapping"))
    kcf, vcf = orc.decode(kc, dt).astype(np.float64), orc.decode(vc, dt).astype(np.float64)
    q = orc.decode(c["query"], dt).astype(np.float64)
    kn = orc.decode(c["key"], dt).astype(np.float64)
    vn = orc.decode(c["value"], dt).astype(np.float64)
    bs = kc.shape[1]
    scale = c.get("scale") or float(np.float32(1) / np.sqrt(np.float32(d)))
    out = np.zeros((q.shape[0], H * d))
    for b in range(len(c["cum"]) - 1):
        s0, s1 = c["cum"][b], c["cum"][b + 1]
        nq, past = s1 - s0, int(c["past"][b])
        if nq == 0:
            continue
        total = past + nq
        keys = np.zeros((total, KV, d))
        vals = np.zeros((total, KV, d))
        for p in range(total):
            if p < past:
                blk, off = c["block_table"][b, p // bs], p % bs
                keys[p], vals[p] = kcf[blk, off], vcf[blk, off]
            else:
                keys[p] = kn[s0 + p - past].reshape(KV, d)
                vals[p] = vn[s0 + p - past].reshape(KV, d)
        qh = torch.from_numpy(q[s0:s1].reshape(nq, H, d).transpose(1, 0, 2).copy())
        kh = torch.from_numpy(np.repeat(keys, H // KV, 1).transpose(1, 0, 2).copy())
        vh = torch.from_numpy(np.repeat(vals, H // KV, 1).transpose(1, 0, 2).copy())
        rows = past + np.arange(nq)[:, None]
        cols = np.arange(total)[None, :]
        allow = np.ones((nq, total), bool)
        if c.get("is_causal", 1):
            allow &= cols <= rows
        w = c.get("local_window_size", -1)
        if w > 0:
            allow &= cols >= rows - w + 1
        o = torch.nn.functional.scaled_dot_product_attention(
            qh[None], kh[None], vh[None], attn_mask=torch.from_numpy(allow)[None, None],
            scale=scale)
        out[s0:s1] = o[0].numpy().transpose(1, 0, 2).reshape(nq, H * d)
    return out


@pytest.mark.parametrize("H,KV,d", [(4, 2, 16), (4, 4, 32), (8, 2, 64), (2, 1, 128)])
@pytest.mark.parametrize("causal,window", [(1, -1), (0, -1), (1, 3), (0, 2)])
def test_attention_matches_torch_sdpa_fp64(H, KV, d, causal, window):
    c = make_case(H, KV, d, 24, 4, 3, dtype=F16, seed=H * d + causal + window, causal=causal,
                  window=window)
    ours, _, _, _ = orc.paged_attention_op(c)
    want = _torch_sdpa_reference(c)
    assert np.max(np.abs(ours - want)) < 1e-12


def test_attention_slot_remap_uses_new_rows():
    # with remapped slots the new positions still attend to the new rows, and cached prefix
    # rows overwritten by the remap are read back (test_paged_attention.py:321-376)
    c = make_case(4, 2, 64, 8, 16, 1, dtype=F16, seed=418, new_lens=[5], past=[37])
    c["slot_mapping"] = (c["block_table"][0, 0] * 16 + np.arange(5)).astype(np.int32)
    ours, _, _, _ = orc.paged_attention_op(c)
    assert np.max(np.abs(ours - _torch_sdpa_reference(c))) < 1e-12


def test_attention_closed_forms():
    # single visible key: output equals that value row
    c = make_case(2, 1, 32, 4, 4, 1, dtype=F32, seed=1, new_lens=[1], past=[0])
    out, _, _, _ = orc.paged_attention_op(c)
    v = c["value"].astype(np.float64)
    assert np.allclose(out[0, :32], v[0], atol=0) and np.allclose(out[0, 32:], v[0], atol=0)
    # identical keys: uniform weights -> mean of the visible values
    c = make_case(1, 1, 8, 4, 4, 1, dtype=F32, seed=2, new_lens=[1], past=[7])
    c["key_cache"][:] = 0.5
    c["key"][:] = 0.5
    out, _, kc, vc = orc.paged_attention_op(c)
    vals = [vc[c["block_table"][0, p // 4], p % 4, 0] for p in range(7)] + [c["value"][0]]
    assert np.allclose(out[0], np.mean(np.array(vals, np.float64), 0), rtol=1e-12, atol=1e-12)


def test_attention_sink_and_softcap_closed_forms():
    # one key with score s and a sink logit z: output = v * e^s / (e^s + e^z)
    c = make_case(1, 1, 4, 2, 4, 1, dtype=F32, seed=3, new_lens=[1], past=[0], scale=1.0)
    c["query"][:] = [[1.0, 0.0, 0.0, 0.0]]
    c["key"][:] = [[0.7, 0.0, 0.0, 0.0]]
    c["head_sink_f32"] = np.array([0.2], np.float32)
    out, _, _, _ = orc.paged_attention_op(c)
    s = 0.7
    want = c["value"][0].astype(np.float64) * math.exp(s) / (math.exp(s) + math.exp(0.2))
    assert np.allclose(out[0], want, rtol=1e-6)
    # two keys with softcap: weights e^{c tanh(s_i/c)}
    c = make_case(1, 1, 4, 2, 4, 1, dtype=F32, seed=4, new_lens=[1], past=[1], scale=1.0,
                  softcap=2.0)
    c["query"][:] = [[1.0, 0.0, 0.0, 0.0]]
    c["key"][:] = [[3.0, 0.0, 0.0, 0.0]]
    blk = c["block_table"][0, 0]
    c["key_cache"][blk, 0, 0] = [1.5, 0.0, 0.0, 0.0]
    out, _, _, vc = orc.paged_attention_op(c)
    w0, w1 = math.exp(2 * math.tanh(1.5 / 2)), math.exp(2 * math.tanh(3.0 / 2))
    want = (vc[blk, 0, 0].astype(np.float64) * w0 + c["value"][0] * w1) / (w0 + w1)
    assert np.allclose(out[0], want, rtol=1e-6)


def test_attention_invariant_to_block_relabelling_and_gqa_repeat():
    c = make_case(8, 2, 32, 16, 4, 2, dtype=F16, seed=21)
    base, _, _, _ = orc.paged_attention_op(c)
    perm = np.random.default_rng(5).permutation(16)
    inv = np.argsort(perm)
    c2 = dict(c)
    c2["key_cache"] = c["key_cache"][perm].copy()
    c2["value_cache"] = c["value_cache"][perm].copy()
    c2["block_table"] = inv[c["block_table"]].astype(np.int32)
    relabelled, _, _, _ = orc.paged_attention_op(c2)
    assert np.array_equal(base, relabelled)
    # GQA == MHA over KV heads repeated g times
    c3 = dict(c)
    g = 4
    rep = lambda a, shape: np.repeat(a.reshape(shape), g, axis=-2)
    T = c["key"].shape[0]
    c3["kv_num_heads"] = 8
    c3["key"] = rep(c["key"], (T, 2, 32)).reshape(T, 8 * 32).copy()
    c3["value"] = rep(c["value"], (T, 2, 32)).reshape(T, 8 * 32).copy()
    c3["key_cache"] = np.repeat(c["key_cache"], g, axis=2).copy()
    c3["value_cache"] = np.repeat(c["value_cache"], g, axis=2).copy()
    mha, _, _, _ = orc.paged_attention_op(c3)
    assert np.max(np.abs(mha - base)) < 1e-12


def test_fp8_attention_dequantises_code_times_scale():
    c = make_case(4, 2, 16, 8, 4, 2, dtype=BF16, cache_dtype=E4M3, seed=31)
    out, _, kc, vc = orc.paged_attention_op(c)
    # equivalent bf16/fp32 problem: dequantise every page, then read all positions from pages
    kf = orc.decode(kc, E4M3) * c["k_scale"][:, None, :, None]
    vf = orc.decode(vc, E4M3) * c["v_scale"][:, None, :, None]
    q = orc.decode(c["query"], BF16)
    H, KV, d, bs = 4, 2, 16, 4
    for b in range(2):
        s0, s1 = c["cum"][b], c["cum"][b + 1]
        nq, past = s1 - s0, int(c["past"][b])
        tot = past + nq
        keys = np.stack([kf[c["block_table"][b, p // bs], p % bs] for p in range(tot)])
        vals = np.stack([vf[c["block_table"][b, p // bs], p % bs] for p in range(tot)])
        qh = torch.from_numpy(q[s0:s1].reshape(nq, H, d).transpose(1, 0, 2).astype(np.float64))
        kh = torch.from_numpy(np.repeat(keys, 2, 1).transpose(1, 0, 2).astype(np.float64))
        vh = torch.from_numpy(np.repeat(vals, 2, 1).transpose(1, 0, 2).astype(np.float64))
        allow = np.arange(tot)[None, :] <= (past + np.arange(nq))[:, None]
        o = torch.nn.functional.scaled_dot_product_attention(
            qh[None], kh[None], vh[None], attn_mask=torch.from_numpy(allow)[None, None],
            scale=float(np.float32(1) / np.sqrt(np.float32(d))))
        want = o[0].numpy().transpose(1, 0, 2).reshape(nq, H * d)
        assert np.max(np.abs(out[s0:s1] - want)) < 1e-6


# ------------------------------------------------------------------------------ GQA (C1)
def test_gqa_contiguous_c1_matches_torch_and_paged():
    rng = np.random.default_rng(1)
    H, KV, d, past = 8, 2, 64, 128
    q = rng.standard_normal((1, 1, H * d)).astype(np.float32)
    k = rng.standard_normal((1, 1, KV * d)).astype(np.float32)
    v = rng.standard_normal((1, 1, KV * d)).astype(np.float32)
    pk = rng.standard_normal((1, KV, past + 1, d)).astype(np.float32)
    pv = rng.standard_normal((1, KV, past + 1, d)).astype(np.float32)
    out, pk2, pv2 = orc.gqa_contiguous(F32, q, k, v, pk, pv, np.array([past]), H, KV, d, 0.125)
    assert np.array_equal(pk2[0, :, past], k.reshape(KV, d))
    qh = torch.from_numpy(q.reshape(1, H, d).transpose(1, 0, 2).astype(np.float64))
    kh = torch.from_numpy(np.repeat(pk2[0], 4, 0).astype(np.float64))
    vh = torch.from_numpy(np.repeat(pv2[0], 4, 0).astype(np.float64))
    o = torch.nn.functional.scaled_dot_product_attention(qh[None], kh[None], vh[None],
                                                         scale=0.125)
    want = o[0].numpy().transpose(1, 0, 2).reshape(1, 1, H * d)
    assert np.max(np.abs(out - want)) < 1e-12
    # the same problem through the paged restatement
    bs = 16
    nb = 9
    kc = np.zeros((nb, bs, KV, d), np.float32)
    vc = np.zeros_like(kc)
    for p in range(past):
        kc[p // bs, p % bs], vc[p // bs, p % bs] = pk[0, :, p], pv[0, :, p]
    case = dict(num_heads=H, kv_num_heads=KV, head_dim=d, dtype=F32, cache_dtype=F32,
                cum=np.array([0, 1], np.int32), past=np.array([past], np.int32),
                block_table=np.arange(nb, dtype=np.int32)[None], query=q.reshape(1, -1),
                key=k.reshape(1, -1), value=v.reshape(1, -1), key_cache=kc, value_cache=vc,
                scale=0.125)
    paged, _, _, _ = orc.paged_attention_op(case)
    assert np.max(np.abs(paged.reshape(out.shape) - out)) < 1e-12


def test_cpu_baseline_matches_fp64_restatement():
    rng = np.random.default_rng(2)
    B, H, KV, d = 3, 8, 2, 64
    ctx = np.array([5, 130, 77], np.int32)
    off = np.concatenate([[0], np.cumsum(ctx)[:-1]]).astype(np.int64)
    k = orc.encode(rng.standard_normal((ctx.sum(), KV, d)), BF16)
    v = orc.encode(rng.standard_normal((ctx.sum(), KV, d)), BF16)
    q = orc.encode(rng.standard_normal((B, H, d)), BF16)
    got = orc.cpu_gqa_decode(BF16, q, k, v, off, ctx, H, KV, d, 0.125, 4)
    for b in range(B):
        pk = np.ascontiguousarray(k[off[b]:off[b] + ctx[b]].transpose(1, 0, 2))[None]
        pv = np.ascontiguousarray(v[off[b]:off[b] + ctx[b]].transpose(1, 0, 2))[None]
        # treat the last row as the "new" token so seqlens_k = ctx - 1
        want, _, _ = orc.gqa_contiguous(BF16, q[b].reshape(1, 1, H * d),
                                        np.ascontiguousarray(pk[0, :, -1]).reshape(1, 1, -1),
                                        np.ascontiguousarray(pv[0, :, -1]).reshape(1, 1, -1),
                                        pk, pv, np.array([ctx[b] - 1]), H, KV, d, 0.125)
        assert orc.rel_l2(got[b].reshape(-1), want.reshape(-1)) < 1e-5


# The CPU path timed beside the GPU (pa_cpu_baseline.c): the same attention over contiguous K/V
# gathered from the pages after the append, in fp32 accumulation -- equal to the oracle's fp64
# result to fp32 rounding, for decode (one row per sequence) and causal prefill chunks.
@pytest.mark.parametrize("new", [[1, 1, 1], [5, 17, 1]], ids=["decode", "prefill"])
def test_cpu_baseline_matches_oracle(new):
    from pa_cases import make_case
    B, bs, mb = 3, 16, 6
    case = make_case(8, 2, 64, B * mb, bs, B, dtype=orc.BF16, seed=12, new_lens=new,
                     past=[40, 9, 70], max_blocks=mb, std=1.0)
    ref, _, kc, vc = orc.paged_attention_op(case)
    cum, past = case["cum"], case["past"]
    ks, vs, offs, off = [], [], [], 0
    for b in range(B):
        total = int(past[b] + cum[b + 1] - cum[b])
        pos = np.arange(total)
        slots = case["block_table"][b, pos // bs] * bs + pos % bs
        ks.append(kc.reshape(-1, 2, 64)[slots])
        vs.append(vc.reshape(-1, 2, 64)[slots])
        offs.append(off)
        off += total
    k, v = np.ascontiguousarray(np.concatenate(ks)), np.ascontiguousarray(np.concatenate(vs))
    scale = float(1.0 / np.sqrt(np.float32(64)))
    if max(new) == 1:
        q = case["query"].reshape(B, 8, 64).copy()
        out = orc.cpu_gqa_decode(orc.BF16, q, k, v, offs, past + 1, 8, 2, 64, scale, 3)
    else:
        out = orc.cpu_gqa_prefill(orc.BF16, case["query"], k, v, offs, cum[:-1],
                                  np.diff(cum), past, 8, 2, 64, scale, 3)
    assert orc.rel_l2(out.reshape(ref.shape), ref) <= 1e-5
