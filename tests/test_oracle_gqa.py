"""Pins for the oracle's GroupQueryAttention restatement (orc_gqa_batched) and for the fixed
RMSNorm reduction order (orc_sum_squares).  CPU only.

orc_gqa_batched is a loop over visible-key bounds.  It is checked here against an independent
evaluation written the way the reference builds its graph (gqa_batched, attention.rs:586-848):
present caches as concatenations [past[:past] | new[:new_rows] | past[length:cap] | zeros]
padded to max(cap, total); masks as arange comparisons (causal_mask_topleft :308-326,
causal_window_mask :328-359); logits in fp64 with softcap then the bias; a sink as an extra
softmax column that is dropped (attention_probs_with_sink :100-118); the rotary rows taken with
the reference's position rule (gqa_rotary_rows :538-584), in torch fp32 arithmetic rounded once
(gqa_rope_f32) or through the already-pinned per-op rope (gqa_rope).  Closed forms cover the
sink, smooth_softmax, the bias and right-padded prompt rows; agreement with the shared-buffer
restatement orc_gqa_contiguous covers the plain decode/prefill forms.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import _oracle as orc
from _oracle import BF16, F16, F32, I4, I8, PER_CHANNEL
from gqa_cases import FORMS, form_case, gqa_case, run_oracle


# ------------------------------------------------------------------------- RMSNorm order
def test_sum_squares_exact_for_representable_sums():
    # small integers: every partial sum is exact, so any order gives numpy's sum
    rng = np.random.default_rng(1)
    for d in (8, 64, 100, 128, 256, 640):
        x = rng.integers(-30, 31, d).astype(np.float32)
        assert orc.sum_squares(x, F32) == float(np.sum(x.astype(np.float64) ** 2))


def _fixed_order_f64(x: np.ndarray) -> float:
    """The documented order, evaluated with numpy: lane partials p[l] over x[l::64] by fused
    multiply-adds (exact in fp64 for bf16 inputs, then one rounding to fp32), then the XOR
    butterfly over distances 32..1."""
    p = np.zeros(64, np.float32)
    for start in range(0, x.size, 64):
        chunk = x[start:start + 64].astype(np.float64)
        lanes = np.arange(chunk.size)
        p[lanes] = (p[lanes].astype(np.float64) + chunk * chunk).astype(np.float32)
    for o in (32, 16, 8, 4, 2, 1):
        p = (p + p[np.arange(64) ^ o]).astype(np.float32)
    assert np.all(p == p[0])
    return float(p[0])


def test_sum_squares_follows_the_device_order():
    rng = np.random.default_rng(2)
    seq_differs = 0
    for trial in range(50):
        d = (64, 128, 256)[trial % 3]
        raw = orc.encode(rng.standard_normal(d) * 3.0, BF16)
        x = orc.decode(raw, BF16)
        got = orc.sum_squares(raw, BF16)
        assert got == _fixed_order_f64(x)
        seq = np.float32(0)
        for v in x:
            seq = np.float32(seq + np.float32(v * v))
        seq_differs += int(seq != got)
    # the order is observable: a sequential sum gives other fp32 results on these inputs
    assert seq_differs > 0


# ------------------------------------------------------------------------- GQA restatement
def _rope_torch_f32(x, cos_rows, sin_rows, half, interleaved, dtype):
    """gqa_rope_f32: fp32 operations, one rounding to T.  x [n, heads, d] decoded floats,
    cos/sin rows [n, half]."""
    xt = torch.from_numpy(x.astype(np.float32))
    c = torch.from_numpy(cos_rows.astype(np.float32))[:, None, :]
    s = torch.from_numpy(sin_rows.astype(np.float32))[:, None, :]
    if interleaved:
        a, b = xt[..., 0:2 * half:2], xt[..., 1:2 * half:2]
    else:
        a, b = xt[..., :half], xt[..., half:2 * half]
    o1, o2 = a * c - b * s, b * c + a * s
    out = xt.clone()
    if interleaved:
        out[..., 0:2 * half:2], out[..., 1:2 * half:2] = o1, o2
    else:
        out[..., :half], out[..., half:2 * half] = o1, o2
    return orc.decode(orc.encode(out.numpy(), dtype), dtype)


def _rotary_positions(pid, total, S, b, qp):
    if pid is None:
        return qp + np.arange(S)
    if total == S:
        return pid.reshape(-1)[0] + np.arange(S)
    return pid.reshape(-1)[b * S:(b + 1) * S]


def _graph_reference(case):
    """The independent evaluation described in the module docstring.  Returns (out fp64
    [B, S, H*d], present_k raw, present_v raw)."""
    c = case
    dt, B, S, H, KV, d = c["dtype"], c["B"], c["S"], c["H"], c["KV"], c["d"]
    g = H // KV
    total = c["total"]
    lengths = c["seqlens"].astype(np.int64) + 1
    kv_seq = 0 if c["k"] is None else c["k"].shape[1]
    cap = 0 if c["pk"] is None else c["pk"].shape[2]
    capacity = max(cap, total)
    cdt = c.get("cache_dtype", 0)
    quant = cdt in (I8, I4)
    zero_code = 0x88 if cdt == I4 else 0
    f32rope = c.get("pid") is not None or kv_seq == 0
    outs, pks, pvs = [], [], []
    for b in range(B):
        length = int(lengths[b])
        qp = max(length - S, 0)
        past = length if kv_seq == 0 else qp
        new_rows = 0 if kv_seq == 0 else length - past
        q = orc.decode(c["q"][b], dt).reshape(S, H, d)
        if c.get("q_norm") is not None:
            q = orc.decode(orc.rms_norm_rows(c["q"][b].reshape(S * H, d), 1, d, c["q_norm"],
                                             1e-6, dt), dt).reshape(S, H, d)
        k = None
        if kv_seq:
            k = orc.decode(c["k"][b], dt).reshape(kv_seq, KV, d)
            if c.get("k_norm") is not None:
                k = orc.decode(orc.rms_norm_rows(c["k"][b].reshape(kv_seq * KV, d), 1, d,
                                                 c["k_norm"], 1e-6, dt), dt).reshape(kv_seq, KV, d)
        if c.get("cos") is not None:
            pos = _rotary_positions(c.get("pid"), total, S, b, qp)
            cosf, sinf = orc.decode(c["cos"], dt), orc.decode(c["sin"], dt)
            half = cosf.shape[1]
            if f32rope:
                q = _rope_torch_f32(q, cosf[pos], sinf[pos], half, c.get("interleaved", 0), dt)
                if k is not None:
                    k = _rope_torch_f32(k, cosf[pos], sinf[pos], half, c.get("interleaved", 0),
                                        dt)
            else:
                q = orc.decode(orc.rope_rows(orc.encode(q, dt), H, d, pos, c["cos"], c["sin"],
                                             0, c.get("interleaved", 0), dt), dt)
                if k is not None:
                    k = orc.decode(orc.rope_rows(orc.encode(k, dt), KV, d, pos, c["cos"],
                                                 c["sin"], 0, c.get("interleaved", 0), dt), dt)
        # present: [past rows | new rows | past tail | zero codes] (attention.rs:735-818)
        width = c["pk"].shape[3] if c["pk"] is not None else d
        raw_t = orc.RAW[cdt or dt]
        pk_b = c["pk"][b] if c["pk"] is not None else np.zeros((KV, 0, width), raw_t)
        pv_b = c["pv"][b] if c["pv"] is not None else np.zeros((KV, 0, width), raw_t)
        v = c["v"][b] if kv_seq else None
        if quant:
            bits = 8 if cdt == I8 else 4
            enc_k = np.stack([
                np.stack([_int_row(k[j, h], c["k_scale"], c["k_mode"], h, bits)
                          for j in range(new_rows)]) if new_rows else np.zeros((0, width), raw_t)
                for h in range(KV)])
            vf = orc.decode(v, dt).reshape(kv_seq, KV, d) if kv_seq else None
            enc_v = np.stack([
                np.stack([_int_row(vf[j, h], c["v_scale"], c["v_mode"], h, bits)
                          for j in range(new_rows)]) if new_rows else np.zeros((0, width), raw_t)
                for h in range(KV)])
        else:
            enc_k = orc.encode(k[:new_rows], dt).transpose(1, 0, 2) if new_rows else \
                np.zeros((KV, 0, d), raw_t)
            enc_v = v.reshape(kv_seq, KV, d)[:new_rows].transpose(1, 0, 2) if new_rows else \
                np.zeros((KV, 0, d), raw_t)
        stored_k = np.concatenate([pk_b[:, :past], enc_k], 1)
        stored_v = np.concatenate([pv_b[:, :past], enc_v], 1)
        if length < cap:
            tail_k, tail_v = pk_b[:, length:], pv_b[:, length:]
        else:
            tail_k = np.full((KV, capacity - length, width), zero_code, raw_t)
            tail_v = tail_k.copy()
        pres_k = np.concatenate([stored_k, tail_k], 1) if kv_seq else pk_b
        pres_v = np.concatenate([stored_v, tail_v], 1) if kv_seq else pv_b
        pad = capacity - pres_k.shape[1]
        if pad > 0:
            z = np.full((KV, pad, width), zero_code, raw_t)
            pres_k, pres_v = np.concatenate([pres_k, z], 1), np.concatenate([pres_v, z], 1)
        pks.append(pres_k)
        pvs.append(pres_v)
        # attention over the stored rows
        if quant:
            bits = 8 if cdt == I8 else 4
            ak = np.stack([_int_decode(stored_k[h], c["k_scale"], c["k_mode"], h, bits, d)
                           for h in range(KV)])
            av = np.stack([_int_decode(stored_v[h], c["v_scale"], c["v_mode"], h, bits, d)
                           for h in range(KV)])
        else:
            ak, av = orc.decode(stored_k, dt), orc.decode(stored_v, dt)
        qt = torch.from_numpy(q.astype(np.float64)).permute(1, 0, 2)              # [H, S, d]
        kt = torch.from_numpy(np.repeat(ak.astype(np.float64), g, 0))            # [H, L, d]
        vt = torch.from_numpy(np.repeat(av.astype(np.float64), g, 0))
        logits = (qt @ kt.transpose(1, 2)) * float(np.float32(c["scale"]))
        if c.get("softcap", 0.0) > 0:
            cp = float(np.float32(c["softcap"]))
            logits = cp * torch.tanh(logits / cp)
        if c.get("bias") is not None:
            bb = 0 if c["bias"].shape[0] == 1 else b
            bias = orc.decode(c["bias"][bb], dt)[:, :, :length].astype(np.float64)
            logits = logits + torch.from_numpy(bias)
        key_pos = np.arange(length)[None, :]
        q_pos = qp + np.arange(S)[:, None]
        window = c.get("window", -1)
        if window > 0:
            lower = np.minimum(np.arange(qp - window + 1, qp + S - window + 1),
                               length - window)[:, None]
            allow = (key_pos <= q_pos) & (lower <= key_pos)
        elif c.get("causal", 1):
            allow = key_pos <= q_pos
        else:
            allow = np.ones((S, length), bool)
        logits = logits.masked_fill(~torch.from_numpy(allow)[None], float("-inf"))
        sink = None
        if c.get("sink") is not None:
            sink = orc.decode(c["sink"], dt).astype(np.float64)
        elif c.get("smooth", 0) == 1:
            sink = np.zeros(H)
        if sink is not None:
            col = torch.from_numpy(sink)[:, None, None].expand(H, S, 1)
            probs = torch.softmax(torch.cat([logits, col], 2), 2)[:, :, :length]
        else:
            probs = torch.softmax(logits, 2)
        outs.append((probs @ vt).permute(1, 0, 2).reshape(S, H * d).numpy())
    return np.stack(outs), np.stack(pks), np.stack(pvs)


def _int_row(x, scale, mode, h, bits):
    d = x.size
    out = np.zeros(d if bits == 8 else (d + 1) // 2, np.int8 if bits == 8 else np.uint8)
    sc = scale[h] if mode == PER_CHANNEL else scale
    orc.lib().orc_int_encode_row(orc._p(np.ascontiguousarray(x, np.float32)), d,
                                 orc._p(np.ascontiguousarray(sc, np.float32)),
                                 int(mode == PER_CHANNEL), bits, 1, orc._p(out))
    return out


def _int_decode(rows, scale, mode, h, bits, d):
    sc = np.asarray(scale[h] if mode == PER_CHANNEL else scale, np.float32).reshape(-1)
    if bits == 8:
        codes = rows.astype(np.float32)
    else:
        lo, hi = (rows & 15).astype(np.int32) - 8, (rows >> 4).astype(np.int32) - 8
        codes = np.stack([lo, hi], -1).reshape(rows.shape[0], -1)[:, :d].astype(np.float32)
    return codes * (sc if sc.size > 1 else sc[0])


@pytest.mark.parametrize("form", list(FORMS))
def test_gqa_batched_matches_the_reference_graph(form):
    c = form_case(form)
    out, pk, pv = run_oracle(c)
    want, wk, wv = _graph_reference(c)
    assert np.array_equal(pk.view(np.uint8), wk.view(np.uint8)), "present_key"
    assert np.array_equal(pv.view(np.uint8), wv.view(np.uint8)), "present_value"
    assert np.max(np.abs(out - want)) < 1e-10


def test_gqa_batched_agrees_with_the_shared_buffer_restatement():
    for dtype, S, window, softcap in ((F32, 1, -1, 0.0), (F16, 5, 40, 0.0), (F16, 5, -1, 25.0)):
        c = gqa_case(dtype, 2, S, 8, 2, 64, [70, 159], cap=160, seed=S, window=window,
                     softcap=softcap, std=0.5)
        out, pk, pv = run_oracle(c, present_cap=160)
        ref, rpk, rpv = orc.gqa_contiguous(dtype, c["q"], c["k"], c["v"], c["pk"], c["pv"],
                                           c["seqlens"], 8, 2, 64, c["scale"], softcap=softcap,
                                           window=window)
        assert np.array_equal(pk, rpk) and np.array_equal(pv, rpv)
        assert np.max(np.abs(out - ref)) < 1e-12


def test_gqa_batched_closed_forms():
    # zero queries: every visible key scores 0
    H, KV, d = 2, 1, 8
    # (1) smooth_softmax: weights 1 / (n + 1) -> sum of the visible values / (n + 1)
    c = gqa_case(F32, 1, 1, H, KV, d, [5], cap=8, seed=3, smooth=1)
    c["q"][:] = 0
    out, pk, pv = run_oracle(c)
    vals = pv[0, 0, :6].astype(np.float64)
    assert np.allclose(out[0, 0, :d], vals.sum(0) / 7, rtol=1e-13, atol=1e-13)
    # (2) head sink z: weights 1 / (n + e^z)
    c = gqa_case(F32, 1, 1, H, KV, d, [5], cap=8, seed=4, sink=True)
    c["q"][:] = 0
    out, pk, pv = run_oracle(c)
    z = c["sink"].astype(np.float64)
    for h in range(H):
        want = pv[0, 0, :6].astype(np.float64).sum(0) / (6 + np.exp(z[h]))
        assert np.allclose(out[0, 0, h * d:(h + 1) * d], want, rtol=1e-13, atol=1e-13)
    # (3) bias log(w_p): weights proportional to w_p
    c = gqa_case(F32, 1, 1, H, KV, d, [5], cap=8, seed=5, bias_shape=(1, 1, 1, 6))
    c["q"][:] = 0
    w = np.array([1, 2, 3, 4, 5, 6], np.float64)
    c["bias"] = np.log(w).astype(np.float32).reshape(1, 1, 1, 6)
    out, pk, pv = run_oracle(c)
    wf = np.exp(c["bias"].astype(np.float64).reshape(6))
    want = (wf[:, None] * pv[0, 0, :6].astype(np.float64)).sum(0) / wf.sum()
    assert np.allclose(out[0, 0, :d], want, rtol=1e-12)
    # (4) ragged first prompt: a right-padded row (i >= length) sees every stored key; with
    # zero queries its output is the mean of the stored values
    c = gqa_case(F32, 2, 6, H, KV, d, [5, 2], seed=6)
    c["q"][:] = 0
    out, pk, pv = run_oracle(c)
    assert pk.shape[2] == 6
    mean1 = pv[1, 0, :3].astype(np.float64).mean(0)
    for i in range(3, 6):
        assert np.allclose(out[1, i, :d], mean1, rtol=1e-13, atol=1e-13)
    # rows of the second sequence beyond its length stay zero codes in the present
    assert np.all(pk[1, :, 3:] == 0) and np.all(pv[1, :, 3:] == 0)


def test_gqa_batched_window_lower_bound_clamps_to_last_key():
    # causal_window_mask: lower = min(query_past + i - w + 1, length - w); for right-padded
    # rows the window ends at the last stored key (attention.rs:348-351)
    c = gqa_case(F32, 1, 8, 1, 1, 4, [4], seed=7, window=2)
    c["q"][:] = 0
    out, pk, pv = run_oracle(c)
    v = pv[0, 0].astype(np.float64)
    for i in range(8):
        lo = min(i - 2 + 1, 5 - 2)
        hi = min(i, 4)
        want = v[max(lo, 0):hi + 1].mean(0)
        assert np.allclose(out[0, i], want, rtol=1e-13, atol=1e-13), i


def test_gqa_batched_rejects_what_the_reference_rejects():
    # past beyond the supplied capacity
    c = gqa_case(F16, 1, 1, 2, 1, 8, [9], cap=4, seed=8)
    with pytest.raises(AssertionError):
        run_oracle(c)
    # rotary positions beyond the cos/sin rows
    c = gqa_case(F16, 1, 2, 2, 1, 8, [3], cap=4, seed=9, rotary=True,
                 pid=np.array([[100, 101]]))
    with pytest.raises(AssertionError):
        run_oracle(c)
