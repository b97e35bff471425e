"""Multi-token batches over integer (int8 / int4) pages on the matrix-core prefill, on the GPU
through the C ABI, against the oracle.

At heads 64, 96, 128 and 256 a batch with more than one query row per sequence over integer
pages runs the planned prefill over operand images: the plan launch copies each 64-key step's
key and value codes into fp16 images (every int8 / int4 code is exact in fp16), the prefill
kernel multiplies the key scales into the query rows (with a power-of-two factor per row that
keeps the products inside fp16), takes the scores and P.V on fp16 matrix cores and applies the
value scales to the output per dimension.  Scales follow the reference's tests
(test_quantized_kv.py:73-78: per-tensor 0.125 / 0.25, per-channel cycles with a zero channel);
geometry and draws follow test_paged_attention.py:182-208 at prefill lengths.

Bars: cache bytes bit-exact; outputs rel-L2 <= 2e-3 against the oracle rounded to T and
<= 4e-3 against its float64 result.  The kernel-level entry pins the path: kind 2 (prefill
matrix-core kernel) forced runs, matches the automatic choice bit for bit, and agrees with the
VALU kernel (kind 3); kind 2 with a forced split-K chunk is refused.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, I4, I8, PER_CHANNEL, PER_TENSOR
from pa_cases import QUANT_NAMES, from_torch, make_case, run_gpu_op, to_torch

pytestmark = pytest.mark.gpu

MODES = {"tensor": (PER_TENSOR, PER_TENSOR), "channel": (PER_CHANNEL, PER_CHANNEL),
         "mixed": (PER_TENSOR, PER_CHANNEL)}


def _rounded(ref, dtype):
    return orc.decode(orc.encode(ref.astype(np.float32), dtype), dtype).astype(np.float64)


def prefill_case(d, bits, mode, dtype, H=8, KV=2, seed=0, **kw):
    """Four sequences: prefill chunks of 150, 0, 37 and 200 rows over pasts of 300, 50, 0, 500
    (blocks of 16, 48 per sequence, pool shuffled)."""
    kw.setdefault("new_lens", [150, 0, 37, 200])
    kw.setdefault("past", [300, 50, 0, 500])
    return make_case(H, KV, d, 4 * 48, 16, 4, dtype=dtype, cache_dtype=I8 if bits == 8 else I4,
                     seed=seed + 31 * d + bits, max_blocks=48, int_modes=MODES[mode], **kw)


def _check_rows(got, ref, ref_t, cum, dtype):
    want_t = _rounded(ref_t if ref_t is not None else ref, dtype)
    for b in range(len(cum) - 1):
        rows = slice(int(cum[b]), int(cum[b + 1]))
        if rows.stop == rows.start:
            continue
        err_t = orc.rel_l2(got[rows], want_t[rows])
        err64 = orc.rel_l2(got[rows], ref[rows])
        assert err_t <= 2e-3, (b, err_t)
        assert err64 <= 4e-3, (b, err64)


def check_op(case):
    print(f"int-prefill case H={case['num_heads']} KV={case['kv_num_heads']} "
          f"d={case['head_dim']} cache={orc.NAMES[case['cache_dtype']]} "
          f"act={orc.NAMES[case['dtype']]} softcap={case['softcap']} "
          f"window={case['local_window_size']}", flush=True)
    ref, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    np.testing.assert_array_equal(kc, kc_ref)
    np.testing.assert_array_equal(vc, vc_ref)
    got = orc.decode(out, case["dtype"]).astype(np.float64)
    _check_rows(got, ref, None, case["cum"], case["dtype"])
    return ref, kc_ref, vc_ref


@pytest.mark.parametrize("d,bits,mode,dtype", [
    (128, 8, "channel", BF16), (128, 4, "tensor", F16), (128, 8, "mixed", F16),
    (128, 4, "channel", BF16), (64, 8, "mixed", BF16), (64, 4, "channel", F16),
    (96, 8, "tensor", BF16), (96, 4, "mixed", F16), (256, 8, "channel", BF16),
    (256, 4, "tensor", F16)],
    ids=["d128-i8-channel-bf16", "d128-i4-tensor-fp16", "d128-i8-mixed-fp16",
         "d128-i4-channel-bf16", "d64-i8-mixed-bf16", "d64-i4-channel-fp16",
         "d96-i8-tensor-bf16", "d96-i4-mixed-fp16", "d256-i8-channel-bf16",
         "d256-i4-tensor-fp16"])
def test_int_prefill_operator(d, bits, mode, dtype):
    check_op(prefill_case(d, bits, mode, dtype))


# softcap with a local window and sink logits; large keys (codes saturate, scores far from 1)
@pytest.mark.parametrize("d,bits,dtype", [(128, 8, BF16), (256, 4, BF16), (96, 8, F16),
                                          (64, 4, BF16)])
def test_int_prefill_softcap_window_sink(d, bits, dtype):
    H = 8
    c = prefill_case(d, bits, "channel", dtype, H=H, softcap=30.0, window=260,
                     head_sink=np.linspace(-1.0, 1.0, H))
    check_op(c)


@pytest.mark.parametrize("d,bits,std", [(128, 8, 4.0), (128, 4, 0.02), (256, 8, 8.0)])
def test_int_prefill_magnitudes(d, bits, std):
    check_op(prefill_case(d, bits, "mixed", BF16, std=std, value_std=std * 3))


# 7:1 head group, one long chunk, a sequence of one row (decode among prefills)
@pytest.mark.parametrize("bits", [8, 4])
def test_int_prefill_group7_ragged(bits):
    check_op(prefill_case(128, bits, "channel", F16, H=14, KV=2, new_lens=[1, 300, 5, 64],
                          past=[600, 0, 250, 10]))


def _attention(case, kc, vc, kind, chunk=0):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    dt, cdt = case["dtype"], case["cache_dtype"]
    I = lambda k: torch.from_numpy(np.ascontiguousarray(case[k], np.int32)).cuda()
    out = ep.attention(to_torch(case["query"], dt), to_torch(case["key"], dt),
                       to_torch(case["value"], dt), to_torch(kc, cdt), to_torch(vc, cdt),
                       I("cum"), I("past"), I("block_table"), num_heads=case["num_heads"],
                       softcap=case["softcap"], local_window_size=case["local_window_size"],
                       k_scale=torch.from_numpy(case["k_scale"]).cuda(),
                       v_scale=torch.from_numpy(case["v_scale"]).cuda(),
                       k_quant_type=QUANT_NAMES[case["k_quant"]],
                       v_quant_type=QUANT_NAMES[case["v_quant"]], kind=kind, chunk=chunk,
                       new_rows_in_cache=True)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("d,bits,dtype", [(128, 8, BF16), (64, 4, F16), (256, 8, F16),
                                          (96, 4, BF16)])
def test_int_prefill_kernel_level_kinds(d, bits, dtype):
    import torch
    c = prefill_case(d, bits, "mixed", dtype)
    print(f"int-prefill kinds d={d} bits={bits} act={orc.NAMES[dtype]}", flush=True)
    ref, _, kc, vc = orc.paged_attention_op(c)
    auto = _attention(c, kc, vc, 0)
    mx = _attention(c, kc, vc, 2)
    valu = _attention(c, kc, vc, 3)
    assert torch.equal(auto, mx)  # the automatic choice is the matrix-core prefill
    for out in (mx, valu):
        got = orc.decode(from_torch(out, dtype), dtype).astype(np.float64)
        _check_rows(got, ref, None, c["cum"], dtype)
    with pytest.raises(Exception, match="over operand images only"):
        _attention(c, kc, vc, 2, chunk=64)


# rows of 768 and 1024 elements over all kv-heads: the append quantises them in two pieces
@pytest.mark.parametrize("d,bits", [(96, 8), (128, 4), (128, 8)])
def test_int_prefill_wide_rows(d, bits):
    check_op(prefill_case(d, bits, "channel", BF16, H=16, KV=8, new_lens=[40, 3, 0, 77],
                          past=[100, 5, 9, 300]))


# GroupQueryAttention over contiguous integer caches ([B, KV, cap, d] codes): multi-token
# queries at heads 64-256 run the same image prefill, the images gathered from the present rows
@pytest.mark.parametrize("bits,d,present", [(8, 128, "shared"), (4, 64, "new"), (8, 256, "new"),
                                            (4, 96, "shared")])
def test_int_gqa_contiguous_multi_token(bits, d, present):
    from gqa_cases import gqa_case
    from test_gpu_gqa_forms import check as gqa_check
    c = gqa_case(BF16, 3, 64, 16, 4, d, [200, 63, 150], cap=256, seed=bits + d,
                 cache_dtype=I8 if bits == 8 else I4, modes=(PER_CHANNEL, PER_TENSOR), std=0.5)
    gqa_check(c, present=present)
