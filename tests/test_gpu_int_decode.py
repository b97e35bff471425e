"""Integer (int8 / int4) pages on the streaming matrix-core decode
(decode_balanced_kernel<T, 64 | 128, CAP, kDcI8 | kDcI4>) against the oracle.

The codes convert exactly to fp16 and the products run in fp16; per-tensor key scales enter the
score scale, per-channel key scales the query operands (fp16 after a per-row power-of-two
normalisation), value scales the epilogue and the partial merge (QuantizedCache::decode,
kv_cache.rs:222-256: values are code x scale).  Cases: both widths, heads 64 / 128, the three
scale layouts of the reference's tests (per-channel cycles with a zero channel), both activation
dtypes, rotary, softcap + sink, local window, pages of 32, two query tokens, long contexts split
over segments (merged), a negative scale, and the kernel-level entry forced to the streaming
decode.

Bars: cache bytes bit-exact; outputs rel-L2 <= 2e-3 against the oracle rounded to T (<= 4e-3
against its fp64 output).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, I4, I8, PER_CHANNEL, PER_TENSOR
from pa_cases import from_torch, make_case, run_gpu_op, to_torch

pytestmark = pytest.mark.gpu

MODES = [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL), (PER_CHANNEL, PER_TENSOR)]
MODE_IDS = ["tensor", "channel", "mixed"]


def check(case, tol=2e-3):
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    np.testing.assert_array_equal(kc, kc_ref)
    np.testing.assert_array_equal(vc, vc_ref)
    dt = case["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    err = orc.rel_l2(got, orc.decode(ref_t, dt))
    assert err <= tol, err
    assert orc.rel_l2(got, ref) <= 2 * tol


def int_case(bits, d, seed, dtype=BF16, modes=(PER_CHANNEL, PER_CHANNEL), B=8, H=16, KV=4,
             bs=16, ctx_hi=900, nq=1, ctx=None, **kw):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(nq + 1, ctx_hi, size=B) if ctx is None else np.asarray(ctx)
    mb = int((ctx.max() + bs - 1) // bs)
    return make_case(H, KV, d, B * mb + 3, bs, B, dtype=dtype,
                     cache_dtype=I8 if bits == 8 else I4, seed=seed, new_lens=[nq] * B,
                     past=ctx - nq, max_blocks=mb, std=1.0, int_modes=modes, **kw)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("modes", MODES, ids=MODE_IDS)
def test_int_decode_scale_layouts(bits, d, modes):
    check(int_case(bits, d, seed=bits + d + modes[0] * 3 + modes[1], modes=modes))


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("variant", ["fp16", "rotary", "softcap_sink", "window", "block32",
                                     "two_tokens", "negative_scale", "gqa8"])
def test_int_decode_variants(bits, variant):
    kw, dtype = {}, BF16
    if variant == "fp16":
        dtype = F16
    elif variant == "rotary":
        kw = dict(do_rotary=1, theta=500000.0)
    elif variant == "softcap_sink":
        kw = dict(softcap=30.0, head_sink=np.linspace(-1, 2, 16))
    elif variant == "window":
        kw = dict(window=100)
    elif variant == "block32":
        kw = dict(bs=32)
    elif variant == "two_tokens":
        kw = dict(nq=2)
    elif variant == "negative_scale":
        kw = dict(scale=-float(1 / np.sqrt(128)))
    elif variant == "gqa8":
        kw = dict(H=64, KV=8)  # g = 8
    check(int_case(bits, 128, seed=bits * 10 + len(variant), dtype=dtype, **kw))


# long contexts split over many segments: the partial merge applies the value scales
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("modes", [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL)],
                         ids=["tensor", "channel"])
def test_int_decode_long_context(bits, modes):
    check(int_case(bits, 128, seed=bits + 77, modes=modes, B=4, H=8, KV=1,
                   ctx=[12000, 300, 4100, 77]))


@pytest.mark.parametrize("bits", [8, 4])
def test_int_kernel_level_streaming_decode(bits):
    """pa_attention_ex with kind 1 over appended integer pages takes the streaming decode: the
    same output as the automatic choice, within the bar of the oracle."""
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import QUANT_NAMES
    case = int_case(bits, 128, seed=bits + 5, B=6, H=32, KV=8)
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    cd = case["cache_dtype"]
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value")}
    kc, vc = to_torch(case["key_cache"], cd), to_torch(case["value_cache"], cd)
    ks, vs = (torch.from_numpy(case[n]).cuda() for n in ("k_scale", "v_scale"))
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    qn = dict(k_quant_type=QUANT_NAMES[case["k_quant"]], v_quant_type=QUANT_NAMES[case["v_quant"]])
    ep.reshape_and_cache(t["key"], t["value"], kc, vc, I["cum"], I["past"], I["block_table"],
                         None, ks, vs, **qn)
    outs = [ep.attention(t["query"], t["key"], t["value"], kc, vc, I["cum"], I["past"],
                         I["block_table"], num_heads=32, k_scale=ks, v_scale=vs,
                         max_query_len=1, kind=kind, **qn) for kind in (1, 0)]
    torch.cuda.synchronize()
    a, b = (from_torch(o, BF16) for o in outs)
    assert np.array_equal(a, b)
    got = orc.decode(a, BF16).astype(np.float64)
    assert orc.rel_l2(got, orc.decode(ref_t, BF16)) <= 2e-3


# Precision of the bias-carrying key operands: scores are sums of q~ x (code + bias) (bias 1152
# for int8, 1032 for int4) with bias x sum(q~) taken off afterwards, so the fp32 rounding of the
# sums scales with bias x sum|q~| rather than with the score.  Peaky softmaxes (queries 8x larger,
# logits spanning tens of units) and keys at code 0 except one outlier channel (per-tensor int4,
# scores nearly all from that channel) put the most weight on that rounding.
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("modes", [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL)],
                         ids=["tensor", "channel"])
def test_int_decode_peaky_softmax(bits, modes):
    case = int_case(bits, 128, seed=bits * 7 + modes[0], modes=modes, B=6, H=16, KV=4)
    q = orc.decode(case["query"], BF16) * 8.0
    case["query"] = orc.encode(q, BF16)
    check(case)


@pytest.mark.parametrize("d", [64, 128])
def test_int4_per_tensor_outlier_channel(d):
    case = int_case(4, d, seed=31 + d, modes=(PER_TENSOR, PER_TENSOR), B=6, H=16, KV=4)
    kc = np.full_like(case["key_cache"], 0x88)  # code 0 in both nibbles
    rng = np.random.default_rng(d)
    codes = rng.integers(-8, 8, size=kc.shape[:3])  # channel 0 (low nibble of byte 0)
    kc[..., 0] = ((codes + 8) | (8 << 4)).astype(np.uint8)
    case["key_cache"] = kc
    q = orc.decode(case["query"], BF16).reshape(case["query"].shape[0], 16, d)
    q[:, :, 0] *= 16.0  # the outlier channel dominates the scores
    case["query"] = orc.encode(q.reshape(-1, 16 * d), BF16)
    check(case)
