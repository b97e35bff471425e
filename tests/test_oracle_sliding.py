"""Pins of the oracle's GroupQueryAttention sliding_window_cache and output_qk restatements
(orc_gqa_batched with sliding / qk_mode), by independent evaluations on the CPU.

sliding_window_cache (attention.rs:1139-1330): the oracle runs call after call, each call's
present fed back as the next past, and is compared with a numpy model that keeps the whole
history of the sequence and evaluates each call in float64 at absolute positions:
  * output: softmax over the keys in the causal window [pos - W + 1, pos] of the history, with
    the bias at the key's absolute column and the sink in the denominator;
  * present: the ring as a procedure -- append the new rows, and while more than the capacity
    are stored drop the oldest `gap` = capacity - W + 1 rows -- then zero rows.  That count is
    also the reference test's own `resident` formula (test_composed_attention.py:316-317,
    _models.py:310-312), checked beside it.
The calls cross the wrap point several times, with single-token and multi-token calls, calls
whose window needs rows the ring drops (the staged view), fp32 rotary at absolute positions, and
integer rings (codes compared exactly, attention through code * scale).

output_qk (attention.rs:771-785, :833-839): mode 1 holds the scaled, softcapped, biased logits
where visible and 0 elsewhere; mode 2 the probabilities (sink in the denominator); columns past
each sequence's length are 0.  Checked against numpy on the oracle's own present (pinned by the
GroupQueryAttention oracle pins), and through the invariant out = probabilities . values.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F32, I8, PER_CHANNEL, PER_TENSOR
from gqa_cases import gqa_case, run_oracle
from pa_cases import int_scales


def ring_rows(total, cap, window):
    """Rows the ring keeps for a sequence of `total` rows: the reference test's formula."""
    gap = cap - window + 1
    return total if total <= cap else total - gap * ((total - cap + gap - 1) // gap)


def rope64(x, pos, cos, sin):
    """Non-interleaved rotary in float64 on the first 2 * half dims at integer positions."""
    half = cos.shape[1]
    c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
    x = x.astype(np.float64).copy()
    x1, x2 = x[..., :half].copy(), x[..., half:2 * half].copy()
    x[..., :half] = x1 * c - x2 * s
    x[..., half:2 * half] = x2 * c + x1 * s
    return x


def run_sliding_calls(steps, *, B=2, H=4, KV=2, d=16, cap=7, W=3, rotary=False, bias=False,
                      sink=False, softcap=0.0, seed=0, cache_dtype=0):
    """Feed the oracle call after call (steps: new rows per call) and check every call against
    the full-history model."""
    rng = np.random.default_rng(seed)
    g = H // KV
    dt = F32
    scale = float(np.float32(1 / np.sqrt(d)))
    quant = cache_dtype != 0
    ks = int_scales(KV, d, PER_CHANNEL, 0) if quant else None
    vs = int_scales(KV, d, PER_TENSOR, 1) if quant else None
    if quant:
        ks = np.where(ks == 0, 0.5, ks).astype(np.float32)  # no zero-scale channel here
    w = d
    raw = np.int8 if quant else np.float32
    past_k = np.zeros((B, KV, cap, w), raw)
    past_v = np.zeros((B, KV, cap, w), raw)
    hist_k = [np.zeros((0, KV, d)) for _ in range(B)]  # history as attended (decoded) rows
    hist_v = [np.zeros((0, KV, d)) for _ in range(B)]
    ring_k = [np.zeros((0, KV, w), raw) for _ in range(B)]  # the ring as a procedure
    ring_v = [np.zeros((0, KV, w), raw) for _ in range(B)]
    lengths = np.zeros(B, np.int64)
    gap = cap - W + 1
    max_len = sum(steps) + 4
    cos = sin = None
    if rotary:
        ang = np.arange(max_len)[:, None] * (1.0 / 10000 ** (np.arange(d // 2) / (d // 2)))
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    sinks = rng.standard_normal(H).astype(np.float32) if sink else None
    for call, S in enumerate(steps):
        lengths += S
        total = int(lengths.max())
        q = rng.standard_normal((B, S, H * d)).astype(np.float32)
        k = rng.standard_normal((B, S, KV * d)).astype(np.float32)
        v = rng.standard_normal((B, S, KV * d)).astype(np.float32)
        bias_arr = rng.uniform(-2, 2, (B, 1, S, total)).astype(np.float32) if bias else None
        out, pk, pv = orc.gqa_batched(
            dt, q, k, v, past_k, past_v, (lengths - 1).astype(np.int32), total, H, KV, d,
            scale=scale, window=W, causal=1, cos=cos, sin=sin, bias=bias_arr, head_sink=sinks,
            softcap=softcap, cache_dtype=cache_dtype, k_scale=ks, v_scale=vs,
            k_mode=PER_CHANNEL if quant else 0, v_mode=PER_TENSOR if quant else 0, sliding=1)
        for b in range(B):
            p = int(lengths[b]) - S
            kb = k[b].reshape(S, KV, d).astype(np.float64)
            if rotary:
                kb = np.stack([rope64(kb[j], p + j, cos, sin) for j in range(S)])
            vb = v[b].reshape(S, KV, d).astype(np.float64)
            if quant:  # stored codes (the reciprocal rule), attended as code * scale
                kc = np.stack([orc.int_encode_row(kb[j, kh], ks[kh], 8, per_channel=True,
                                                  reciprocal=True)
                               for j in range(S) for kh in range(KV)]).reshape(S, KV, w)
                vc = np.stack([orc.int_encode_row(vb[j, kh], vs, 8, per_channel=False,
                                                  reciprocal=True)
                               for j in range(S) for kh in range(KV)]).reshape(S, KV, w)
                kb = kc.astype(np.float64) * ks[None].astype(np.float64)
                vb = vc.astype(np.float64) * vs.astype(np.float64)
            else:
                kc, vc = kb.astype(np.float32), vb.astype(np.float32)
            hist_k[b] = np.concatenate([hist_k[b], kb])
            hist_v[b] = np.concatenate([hist_v[b], vb])
            ring_k[b] = np.concatenate([ring_k[b], kc.astype(raw)])
            ring_v[b] = np.concatenate([ring_v[b], vc.astype(raw)])
            while ring_k[b].shape[0] > cap:
                ring_k[b], ring_v[b] = ring_k[b][gap:], ring_v[b][gap:]
            n = ring_k[b].shape[0]
            assert n == ring_rows(int(lengths[b]), cap, W)
            # present: the ring, then zero rows (rotated keys: the model rotates in float64,
            # the oracle in fp32 with one rounding)
            if rotary:
                np.testing.assert_allclose(pk[b, :, :n], ring_k[b].transpose(1, 0, 2),
                                           rtol=1e-6, atol=1e-6)
            else:
                np.testing.assert_array_equal(pk[b, :, :n], ring_k[b].transpose(1, 0, 2))
            np.testing.assert_array_equal(pv[b, :, :n], ring_v[b].transpose(1, 0, 2))
            assert not pk[b, :, n:].any() and not pv[b, :, n:].any()
            # output: window attention over the whole history at absolute positions
            for i in range(S):
                pos = p + i
                qi = q[b, i].reshape(H, d).astype(np.float64)
                if rotary:
                    qi = rope64(qi, pos, cos, sin)
                lo = max(0, pos - W + 1)
                for h in range(H):
                    keys = hist_k[b][lo:pos + 1, h // g]
                    s = scale * keys @ qi[h]
                    if softcap:
                        s = softcap * np.tanh(s / softcap)
                    if bias:
                        s = s + bias_arr[b, 0, i, lo:pos + 1]
                    z = np.concatenate([s, [sinks[h]]]) if sink else s
                    e = np.exp(z - z.max())
                    pr = e[: len(s)] / e.sum()
                    want = pr @ hist_v[b][lo:pos + 1, h // g]
                    got = out[b, i, h * d:(h + 1) * d]
                    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6,
                                               err_msg=f"call {call} b {b} row {i} head {h}")
        past_k, past_v = pk, pv


def test_ring_rows_formula_is_the_dropping_procedure():
    for cap in range(1, 12):
        for W in range(1, cap + 1):
            gap = cap - W + 1
            n = 0
            for total in range(1, 60):
                n += 1
                while n > cap:
                    n -= gap
                assert n == ring_rows(total, cap, W), (cap, W, total)


def test_sliding_decode_calls_across_wraps():
    run_sliding_calls([1] * 20, cap=7, W=3)


def test_sliding_window_equals_capacity():
    # W = capacity (gap 1): the ring keeps the last `capacity` rows after every call
    run_sliding_calls([1] * 12 + [3, 1], cap=5, W=5, seed=1)


def test_sliding_multi_token_calls_staged_view():
    # calls of 3 and 5 rows: the window needs rows the ring drops in the same call
    run_sliding_calls([4, 3, 5, 1, 3, 5, 2, 1, 5], cap=6, W=4, seed=2)


def test_sliding_first_prompt_longer_than_the_ring():
    run_sliding_calls([9, 1, 1, 4], cap=5, W=2, seed=3)


def test_sliding_rotary_bias_sink_softcap():
    run_sliding_calls([3, 1, 1, 2, 1, 1, 4, 1], cap=6, W=3, rotary=True, bias=True, sink=True,
                      softcap=2.5, seed=4)


def test_sliding_int8_ring():
    run_sliding_calls([2, 1, 1, 3, 1, 1, 1, 2], cap=5, W=3, seed=5, cache_dtype=I8)


def test_sliding_rotary_without_bias_rounds_per_op():
    """bf16 rotary without bias or position ids rotates with per-op rounding (gqa_rope), with a
    bias in fp32 (gqa_rope_f32, attention.rs:1222-1228): the stored key rows differ."""
    c0 = gqa_case(BF16, 1, 2, 2, 1, 16, [40], cap=8, window=4, rotary=True, seed=7)
    c0["sliding"] = 1
    c1 = dict(c0)
    c1["bias"] = np.zeros((1, 1, 2, 41), np.uint16)  # an all-zero bias: only the rounding differs
    _, pk0, _ = run_oracle(c0)
    _, pk1, _ = run_oracle(c1)
    assert not np.array_equal(pk0, pk1)
    # the new rows sit at ring rows [before, before + 2) = [kept, after) of the present
    n = ring_rows(41, 8, 4)
    assert not pk0[0, 0, n:].any()


# ------------------------------------------------------------------------------ output_qk
QK_FORMS = {
    "ragged_first_prompt_smooth": dict(dtype=F32, B=3, S=5, H=4, KV=2, d=8, seqlens=[4, 2, 3],
                                       smooth=1),
    "later_call_bias_sink_softcap": dict(dtype=F32, B=2, S=2, H=4, KV=2, d=8, seqlens=[6, 9],
                                         cap=10, bias_shape=(2, 4, 2, 10), sink=True,
                                         softcap=2.0),
    "window_growing": dict(dtype=F32, B=2, S=3, H=2, KV=1, d=8, seqlens=[7, 4], cap=6,
                           window=3),
    "non_causal": dict(dtype=F32, B=1, S=3, H=2, KV=2, d=8, seqlens=[6], cap=6, causal=0),
}


@pytest.mark.parametrize("form", sorted(QK_FORMS))
@pytest.mark.parametrize("mode", [1, 2])
def test_output_qk_against_numpy(form, mode):
    kw = dict(QK_FORMS[form])
    c = gqa_case(kw.pop("dtype"), kw.pop("B"), kw.pop("S"), kw.pop("H"), kw.pop("KV"),
                 kw.pop("d"), kw.pop("seqlens"), seed=11 + mode, **kw)
    c["qk_mode"] = mode
    out, pk, pv, qk = run_oracle(c)
    B, S, H, KV, d, total = c["B"], c["S"], c["H"], c["KV"], c["d"], c["total"]
    g = H // KV
    dec = lambda a: orc.decode(a, c["dtype"]).astype(np.float64)
    q = dec(c["q"]).reshape(B, S, H, d)
    keys, vals = dec(pk), dec(pv)
    for b in range(B):
        length = int(c["seqlens"][b]) + 1
        qp = max(length - S, 0)
        for i in range(S):
            end = min(qp + i + 1, length) if c["causal"] else length
            start = 0
            if c["window"] > 0:
                start = max(0, min(qp + i, length - 1) - c["window"] + 1)
            for h in range(H):
                s = c["scale"] * keys[b, h // g, :length] @ q[b, i, h]
                if c["softcap"]:
                    s = c["softcap"] * np.tanh(s / c["softcap"])
                if c.get("bias") is not None:
                    bb = dec(c["bias"])
                    s = s + bb[b if bb.shape[0] > 1 else 0, h if bb.shape[1] > 1 else 0, i, :length]
                vis = (np.arange(length) >= start) & (np.arange(length) < end)
                z = np.where(vis, s, -np.inf)
                sk = dec(c["sink"])[h] if c.get("sink") is not None else (0.0 if c["smooth"] else None)
                zz = np.concatenate([z, [sk]]) if sk is not None else z
                e = np.exp(zz - zz.max())
                pr = e[:length] / e.sum()
                want = np.zeros(total)
                want[:length] = np.where(vis, s, 0.0) if mode == 1 else pr
                np.testing.assert_allclose(qk[b, h, i], want, rtol=1e-6, atol=1e-9)
                if mode == 2:  # the probabilities are the ones the output uses
                    np.testing.assert_allclose(out[b, i, h * d:(h + 1) * d],
                                               qk[b, h, i, :length] @ vals[b, h // g, :length],
                                               rtol=1e-9, atol=1e-12)
