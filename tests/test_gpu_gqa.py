"""GroupQueryAttention on contiguous caches (pa_group_query_attention) against the oracle's
contiguous GQA restatement (orc_gqa_contiguous: gqa_batched, attention.rs:586-848, and the
reference's ORT-CPU-semantics reference test_gqa_position_cache.py:104-126).

Bars: present rows bit-exact; outputs rel-L2 <= 1e-5 (fp32) and
<= 2e-3 against the T-rounded oracle output for fp16/bf16.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, F32
from pa_cases import from_torch, rotary_cache, to_torch

pytestmark = pytest.mark.gpu


def gqa_case(B, S, H, KV, d, cap, seqlens, dtype, seed, std=1.0):
    rng = np.random.default_rng(seed)
    enc = lambda shape: orc.encode(rng.standard_normal(shape) * std, dtype)
    return dict(q=enc((B, S, H * d)), k=enc((B, S, KV * d)), v=enc((B, S, KV * d)),
                pk=enc((B, KV, cap, d)), pv=enc((B, KV, cap, d)),
                seqlens=np.asarray(seqlens, np.int32))


def run_gqa(c, dtype, H, KV, **kw):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    T = {n: to_torch(c[n], dtype) for n in ("q", "k", "v", "pk", "pv")}
    sl = torch.from_numpy(c["seqlens"]).cuda()
    extra = {n: to_torch(c[n], dtype) for n in ("cos", "sin", "sink") if n in c}
    kw.setdefault("present", "shared")
    out, pk, pv = ep.group_query_attention(
        T["q"], T["k"], T["v"], T["pk"], T["pv"], sl, int(c["seqlens"].max()) + 1,
        cos_cache=extra.get("cos"), sin_cache=extra.get("sin"), head_sink=extra.get("sink"),
        num_heads=H, kv_num_heads=KV, do_rotary=int("cos" in c), **kw)
    torch.cuda.synchronize()
    return from_torch(out, dtype), from_torch(pk, dtype), from_torch(pv, dtype)


def check_against_oracle(c, dtype, H, KV, d, scale, tol, **kw):
    ref, rpk, rpv = orc.gqa_contiguous(dtype, c["q"], c["k"], c["v"], c["pk"], c["pv"],
                                       c["seqlens"], H, KV, d, scale, **kw)
    out, pk, pv = run_gqa(c, dtype, H, KV, scale=scale,
                          softcap=kw.get("softcap", 0.0), local_window_size=kw.get("window", -1))
    assert np.array_equal(pk, rpk), "present_key differs"
    assert np.array_equal(pv, rpv), "present_value differs"
    got = orc.decode(out, dtype).astype(np.float64)
    if dtype == F32:
        err = orc.rel_l2(got, ref)
    else:
        err = orc.rel_l2(got, orc.decode(orc.encode(ref.astype(np.float32), dtype), dtype))
    assert err <= tol, err


# fp32, batch 1, 8 q / 2 kv heads, d 64, past 128 + 1 new, scale 1/8
def test_gqa_c1_fp32():
    c = gqa_case(1, 1, 8, 2, 64, 129, [128], F32, seed=1)
    check_against_oracle(c, F32, 8, 2, 64, 0.125, 1e-5)


# decode on the streaming matrix-core kernel (g * seq <= 16): ragged lengths, both dtypes
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("d,H,KV", [(128, 32, 8), (64, 8, 2)])
def test_gqa_decode_mfma(dtype, d, H, KV):
    rng = np.random.default_rng(d + H)
    B, cap = 5, 1536
    seqlens = rng.integers(0, cap, size=B)
    seqlens[0] = cap - 1
    c = gqa_case(B, 1, H, KV, d, cap, seqlens, dtype, seed=int(seqlens.sum()))
    check_against_oracle(c, dtype, H, KV, d, float(1 / np.sqrt(d)), 2e-3)


# multi-token queries (g * seq > 16: VALU kernel), fp32 and fp16, window and softcap
@pytest.mark.parametrize("dtype,window,softcap", [(F32, -1, 0.0), (F16, 40, 0.0),
                                                  (F16, -1, 25.0)])
def test_gqa_prefill_valu(dtype, window, softcap):
    B, S, cap = 2, 5, 160
    c = gqa_case(B, S, 8, 2, 64, cap, [70, 159], dtype, seed=7, std=0.5)
    check_against_oracle(c, dtype, 8, 2, 64, 0.125, 1e-5 if dtype == F32 else 2e-3,
                         window=window, softcap=softcap)


# RoPE on the new rows at positions seqlens_k + 1 - S + i (theta 500000, bf16): the expected
# output is the contiguous oracle on query/key rows rotated by the oracle's RoPE restatement
def test_gqa_rotary_bf16():
    B, S, H, KV, d, cap = 3, 1, 16, 4, 128, 600
    seqlens = np.array([599, 10, 300], np.int32)
    c = gqa_case(B, S, H, KV, d, cap, seqlens, BF16, seed=11)
    c["cos"], c["sin"] = rotary_cache(cap + 8, d, 500000.0, BF16)
    pos = (np.repeat(seqlens + 1 - S, S) + np.tile(np.arange(S), B)).astype(np.int32)
    qr = orc.rope_rows(c["q"].reshape(B * S, H * d), H, d, pos, c["cos"], c["sin"], 0, 0, BF16)
    kr = orc.rope_rows(c["k"].reshape(B * S, KV * d), KV, d, pos, c["cos"], c["sin"], 0, 0, BF16)
    ref, rpk, rpv = orc.gqa_contiguous(BF16, qr.reshape(c["q"].shape), kr.reshape(c["k"].shape),
                                       c["v"], c["pk"], c["pv"], seqlens, H, KV, d,
                                       float(1 / np.sqrt(d)))
    out, pk, pv = run_gqa(c, BF16, H, KV)
    assert np.array_equal(pk, rpk)
    assert np.array_equal(pv, rpv)
    got = orc.decode(out, BF16).astype(np.float64)
    assert orc.rel_l2(got, orc.decode(orc.encode(ref.astype(np.float32), BF16), BF16)) <= 2e-3
