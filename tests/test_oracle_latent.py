"""Pins of the oracle's LATENT-layout restatement (attention.rs:4058-4062, :4210-4213: one kv
head, values are the first v_head_size dims of the rotated key rows, output
[T, H * v_head_size]):

- equivalence with the pinned SEPARATE path: a SEPARATE case whose value rows are the rotated
  key rows and whose value cache is a copy of the key cache gives the same scores, so its
  first v_head_size output dims per head are the LATENT output;
- the reference's hand-computed LATENT known answer (test_paged_attention.py:669-759), restated
  in numpy float32 with its own tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import F16
from pa_cases import make_latent_case


@pytest.mark.parametrize("rotary", [0, 1])
@pytest.mark.parametrize("d,vd,H", [(16, 8, 2), (64, 48, 4), (72, 64, 8)])
def test_latent_equals_separate_with_values_from_rotated_keys(rotary, d, vd, H):
    c = make_latent_case(H, d, vd, 24, 4, 3, dtype=F16, seed=d + vd + rotary,
                         new_lens=[2, 1, 3], past=[5, 0, 9], max_blocks=8, do_rotary=rotary,
                         rot_dim=min(16, d - 8) if rotary else None,
                         rotary_offset=8 if rotary else 0,
                         scale=0.2)
    latent, _, kc_lat, _ = orc.paged_attention_op(c)

    sep = dict(c)
    sep.pop("latent")
    sep.pop("v_head_size")
    k_rot = c["key"]
    if rotary:
        pos = np.concatenate([c["past"][b] + np.arange(c["cum"][b + 1] - c["cum"][b])
                              for b in range(3)])
        k_rot = orc.rope_rows(c["key"], 1, d, pos, c["cos_cache"], c["sin_cache"], 8, 0, F16)
    sep["value"] = k_rot
    sep["value_cache"] = c["key_cache"].copy()
    full, _, kc_sep, vc_sep = orc.paged_attention_op(sep)
    np.testing.assert_array_equal(kc_lat, kc_sep)      # identical key appends
    np.testing.assert_array_equal(vc_sep, kc_sep)      # so the separate values mirror the keys
    T = c["query"].shape[0]
    want = full.reshape(T, H, d)[:, :, :vd].reshape(T, H * vd)
    np.testing.assert_array_equal(latent, want)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def test_latent_reference_known_answer():
    """test_paged_attention.py:669-759 restated: h=2, kv=1, d=16, vd=8, rot=8 at offset 8,
    two new tokens over past 3, block table [[1, 0, 2]], scale 0.2, float32 reference math,
    the reference's own tolerance (2e-2)."""
    h, kv, d, vd, rot, nb, blk = 2, 1, 16, 8, 8, 3, 4
    nt, past_len, offset, scale = 2, 3, 8, 0.2
    rng = np.random.default_rng(291)
    q = (rng.standard_normal((nt, h * d)) * 0.2).astype(np.float16)
    k = (rng.standard_normal((nt, d)) * 0.2).astype(np.float16)
    kc = (rng.standard_normal((nb, blk, kv, d)) * 0.2).astype(np.float16)
    bt = np.array([[1, 0, 2]], dtype=np.int32)
    half = rot // 2
    inv = 1.0 / (10000.0 ** (np.arange(half) / half))
    angles = np.arange(nb * blk)[:, None] * inv[None, :]
    cos = np.cos(angles).astype(np.float16)
    sin = np.sin(angles).astype(np.float16)

    def rope(x, pos):
        out = x.copy()
        c = np.concatenate([cos[pos], cos[pos]], -1).astype(np.float32)[:, None, :]
        s = np.concatenate([sin[pos], sin[pos]], -1).astype(np.float32)[:, None, :]
        sl = x[..., offset:offset + rot]
        out[..., offset:offset + rot] = sl * c + _rotate_half(sl) * s
        return out

    positions = np.arange(past_len, past_len + nt)
    qh = rope(q.reshape(nt, h, d).astype(np.float32), positions)
    kh = rope(k.reshape(nt, kv, d).astype(np.float32), positions)
    keys = np.empty((past_len + nt, d), np.float32)
    for logical in range(past_len):
        keys[logical] = kc[bt[0, logical // blk], logical % blk, 0]
    keys[past_len:] = kh[:, 0]
    scores = np.einsum("thd,kd->htk", qh, keys) * scale
    cols = np.arange(past_len + nt)[None, :]
    rows = (past_len + np.arange(nt))[:, None]
    scores = np.where((cols > rows)[None], -np.inf, scores)
    probs = np.exp(scores - scores.max(-1, keepdims=True))
    probs /= probs.sum(-1, keepdims=True)
    expected = np.einsum("htk,kv->thv", probs, keys[:, :vd]).reshape(nt, h * vd)

    case = dict(num_heads=h, kv_num_heads=kv, head_dim=d, dtype=F16, cache_dtype=F16,
                cum=np.array([0, nt], np.int32), past=np.array([past_len], np.int32),
                block_table=bt, query=q, key=k, key_cache=kc, cos_cache=cos, sin_cache=sin,
                rotary_offset=offset, scale=scale, latent=True, v_head_size=vd)
    out, out_t, kc_out, _ = orc.paged_attention_op(case)
    np.testing.assert_allclose(out_t.astype(np.float32), expected, rtol=2e-2, atol=2e-2)
    expected_cache = kc.copy()
    for i in range(nt):
        logical = past_len + i
        expected_cache[bt[0, logical // blk], logical % blk, 0] = kh[i, 0].astype(np.float16)
    np.testing.assert_allclose(kc_out.astype(np.float32), expected_cache.astype(np.float32),
                               rtol=2e-3, atol=2e-3)
