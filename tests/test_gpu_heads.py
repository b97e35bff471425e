"""Heads 96 and 256 on the matrix cores: the streaming decode (decode_balanced_kernel<T, 96 | 256>)
and the LDS-shared prefill kernel (prefill_kernel<T, 96 | 256>).

The reference's direct kernel takes heads 64/96/128/256 (attention.rs:4140); its head-256 tests
(test_paged_attention.py:245-247, :289-318) are mirrored in test_gpu_paged_attention.py and now
reach this kernel for their decode-shaped batches.  Here: ragged decode batches in both dtypes,
rotary, softcap + sink, local window, page sizes 16/32/64, two query tokens per sequence
(g * nq <= 16), long contexts split over many segments (merged), a negative scale, the
kernel-level entry forced to the streaming decode (kind 1), which fails for a head size the
kernel does not take, and multi-token batches on the prefill kernel (the planned launch at
head 256 is in test_gpu_paged_attention.py::test_prefill_planned).

Bars as everywhere: caches bit-exact, outputs rel-L2 <= 2e-3 against the T-rounded oracle
(<= 4e-3 against its fp64 output).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16
from pa_cases import from_torch, make_case, run_gpu_op, to_torch

pytestmark = pytest.mark.gpu


def check(case, tol=2e-3):
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    assert np.array_equal(kc, kc_ref) and np.array_equal(vc, vc_ref), "caches differ"
    dt = case["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    err = orc.rel_l2(got, orc.decode(ref_t, dt))
    assert err <= tol, err
    assert orc.rel_l2(got, ref) <= 2 * tol


def decode_case(d, dtype, seed, B=8, H=16, KV=4, bs=16, ctx_hi=700, nq=1, **kw):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(nq + 1, ctx_hi, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    return make_case(H, KV, d, B * mb + 3, bs, B, dtype=dtype, seed=seed, new_lens=[nq] * B,
                     past=ctx - nq, max_blocks=mb, std=1.0, **kw)


@pytest.mark.parametrize("d", [96, 256])
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("variant", ["plain", "rotary", "softcap_sink", "window", "block32",
                                     "block64", "two_tokens", "negative_scale"])
def test_decode_heads(d, dtype, variant):
    kw = {}
    if variant == "rotary":
        kw = dict(do_rotary=1, theta=10000.0)
    elif variant == "softcap_sink":
        kw = dict(softcap=30.0, head_sink=np.linspace(-1, 2, 16))
    elif variant == "window":
        kw = dict(window=100)
    elif variant == "block32":
        kw = dict(bs=32)
    elif variant == "block64":
        kw = dict(bs=64)
    elif variant == "two_tokens":
        kw = dict(nq=2)
    elif variant == "negative_scale":
        kw = dict(scale=-float(1 / np.sqrt(d)))
    check(decode_case(d, dtype, seed=d + len(variant), **kw))


# long contexts: one sequence far longer than the others, split over many segments
@pytest.mark.parametrize("d", [96, 256])
def test_decode_heads_long_context(d):
    B, bs = 4, 16
    ctx = np.array([12000, 300, 4100, 77])
    mb = int((ctx.max() + bs - 1) // bs)
    case = make_case(8, 1, d, B * mb, bs, B, dtype=BF16, seed=d, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, std=1.0, do_rotary=1, theta=500000.0)
    check(case)


@pytest.mark.parametrize("d", [96, 256])
def test_kernel_level_streaming_decode(d):
    """pa_attention_ex with kind 1 over appended pages takes the streaming decode: the same
    output as the automatic choice, and within the bar of the oracle."""
    import torch
    import onnxruntime_ep_mlx_amd as ep
    case = decode_case(d, BF16, seed=7 * d, B=6, H=32, KV=8)
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value", "key_cache",
                                              "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                         I["past"], I["block_table"])
    outs = [ep.attention(t["query"], t["key"], t["value"], t["key_cache"], t["value_cache"],
                         I["cum"], I["past"], I["block_table"], num_heads=32, max_query_len=1,
                         kind=kind) for kind in (1, 0)]
    torch.cuda.synchronize()
    a, b = (from_torch(o, BF16) for o in outs)
    assert np.array_equal(a, b)
    got = orc.decode(a, BF16).astype(np.float64)
    assert orc.rel_l2(got, orc.decode(ref_t, BF16)) <= 2e-3


# multi-token batches (more than 16 grouped rows: the LDS-shared prefill kernel): ragged chunks,
# an empty sequence, causal / window / softcap / sink, both dtypes
@pytest.mark.parametrize("d", [96, 256])
@pytest.mark.parametrize("dtype,variant", [(BF16, "plain"), (F16, "plain"), (BF16, "window"),
                                           (F16, "softcap_sink"), (BF16, "non_causal"),
                                           (BF16, "block32")])
def test_prefill_heads(d, dtype, variant):
    rng = np.random.default_rng(d + len(variant))
    B, H, KV = 4, 16, 4
    bs = 32 if variant == "block32" else 16
    new_lens = [37, 0, 70, 5]
    past = rng.integers(0, 600, size=B)
    mb = int((past.max() + max(new_lens) + bs - 1) // bs)
    kw = {}
    if variant == "window":
        kw = dict(window=50)
    elif variant == "softcap_sink":
        kw = dict(softcap=20.0, head_sink=np.linspace(-1, 1, H))
    elif variant == "non_causal":
        kw = dict(causal=0)
    check(make_case(H, KV, d, B * mb + 5, bs, B, dtype=dtype, seed=d + len(variant),
                    new_lens=new_lens, past=past, max_blocks=mb, std=1.0, **kw))
