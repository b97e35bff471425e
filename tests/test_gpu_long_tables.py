"""Multi-token batches over byte-coded pages (fp8 e4m3, int8, int4) whose block tables span
65,536 positions while the live contexts are short, on the GPU through the C ABI, against the
oracle.

The planned prefill's operand images (fp16 rows of every 64-key step of every (sequence,
kv-head), 32 KiB per step at head 128) are sized by the live context: the host metadata's
longest past + new tokens, or the caller's max_context_len.  Sized by the block-table capacity,
16 sequences x 8 kv-heads x 1,024 steps would need 4 GiB -- beyond the 2 GiB image limit -- and
these batches would fall to the VALU kernel; now they run the matrix-core prefill over images.
Where the caller's bound itself makes the images too large, the planned prefill runs on groups
of sequences whose images fit, one launch per group over the same image region.
The block tables repeat valid pool blocks past each sequence's live pages (the reference's
validation checks only the blocks a sequence needs, attention.rs:3975-3987).

Bars: cache bytes bit-exact; outputs rel-L2 <= 2e-3 against the oracle rounded to T and
<= 4e-3 against its float64 result, per sequence.  A call whose context exceeds the caller's
bound (device metadata only) leaves those sequences' rows unwritten and the others exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, E4M3, F16, I4, I8
from pa_cases import QUANT_NAMES, from_torch, make_case, run_gpu_op, to_torch

pytestmark = pytest.mark.gpu

SPAN_BLOCKS = 4096  # 65,536 positions of 16-row pages


def long_table_case(cache_dtype, dtype=BF16, B=16, KV=8, H=16, d=128, bs=16, seed=0):
    rng = np.random.default_rng(seed + 5)
    new = rng.integers(40, 160, size=B)
    past = rng.integers(0, 1100, size=B)
    live = int(-(-(past + new).max() // bs))
    c = make_case(H, KV, d, B * live, bs, B, dtype=dtype, cache_dtype=cache_dtype,
                  seed=seed + 31, new_lens=new, past=past, max_blocks=live)
    bt = c["block_table"]
    c["block_table"] = np.ascontiguousarray(np.resize(bt, (B, SPAN_BLOCKS)), np.int32)
    c["block_table"][:, :live] = bt  # live pages as drawn, the rest repeats valid block ids
    return c


def _check(case, out, kc, vc, skip=()):
    ref, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    np.testing.assert_array_equal(kc, kc_ref)
    np.testing.assert_array_equal(vc, vc_ref)
    got = orc.decode(out, case["dtype"]).astype(np.float64)
    want_t = orc.decode(orc.encode(ref.astype(np.float32), case["dtype"]),
                        case["dtype"]).astype(np.float64)
    cum = case["cum"]
    for b in range(len(cum) - 1):
        rows = slice(int(cum[b]), int(cum[b + 1]))
        if b in skip or rows.stop == rows.start:
            continue
        assert orc.rel_l2(got[rows], want_t[rows]) <= 2e-3, b
        assert orc.rel_l2(got[rows], ref[rows]) <= 4e-3, b


@pytest.mark.parametrize("cache_dtype,dtype", [(E4M3, BF16), (E4M3, F16), (I8, BF16), (I4, F16)],
                         ids=["fp8-bf16", "fp8-fp16", "int8-bf16", "int4-fp16"])
def test_long_block_table_prefill_over_live_images(cache_dtype, dtype):
    case = long_table_case(cache_dtype, dtype)
    print(f"long-table case {orc.NAMES[cache_dtype]} act={orc.NAMES[dtype]} B=16 KV=8 d=128 "
          f"span={SPAN_BLOCKS * 16}", flush=True)
    out, kc, vc = run_gpu_op(case)
    _check(case, out, kc, vc)


def test_long_block_table_with_callers_context_bound():
    """Device metadata only: the caller's max_context_len sizes the images."""
    case = long_table_case(E4M3, BF16, seed=3)
    mc = int((case["past"] + np.diff(case["cum"])).max())
    mq = int(np.diff(case["cum"]).max())
    print(f"long-table case fp8 bound={mc}", flush=True)
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=mq, max_context_len=mc)
    _check(case, out, kc, vc)


def test_context_bound_below_a_sequence_leaves_its_rows():
    """A bound below one sequence's context (device metadata only): that sequence's rows stay
    as they were (no access outside the images), every other sequence is exact."""
    case = long_table_case(E4M3, BF16, seed=4)
    tot = case["past"] + np.diff(case["cum"])
    b_long = int(np.argmax(tot))
    mc = int(np.sort(tot)[-2])  # below the longest only
    assert tot[b_long] > mc
    mq = int(np.diff(case["cum"]).max())
    print(f"long-table case fp8 short bound={mc} (sequence {b_long} has {int(tot[b_long])})",
          flush=True)
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=mq, max_context_len=mc)
    _check(case, out, kc, vc, skip=(b_long,))


@pytest.mark.parametrize("cache_dtype,dtype", [(E4M3, BF16), (I8, BF16), (I4, F16)],
                         ids=["fp8-bf16", "int8-bf16", "int4-fp16"])
def test_oversized_images_run_in_sequence_groups(cache_dtype, dtype):
    """The caller bounds the context by the whole block-table span (65,536 positions): images of
    12 sequences x 8 kv-heads x 1,024 64-key steps (3 GiB) exceed the 2 GiB image limit, so the
    planned prefill runs on groups of 8 and 4 sequences over one 2 GiB image region instead of
    dropping to the VALU kernel.  The kernel-level call that admits only the planned prefill
    (kind 2 over byte-coded pages) gives the operator's output bit for bit."""
    import torch
    import onnxruntime_ep_mlx_amd as ep
    case = long_table_case(cache_dtype, dtype, B=12, seed=11)
    assert "cos_cache" not in case
    mq = int(np.diff(case["cum"]).max())
    mc = SPAN_BLOCKS * 16
    print(f"grouped-images case {orc.NAMES[cache_dtype]} act={orc.NAMES[dtype]} B=12 KV=8 "
          f"bound={mc}", flush=True)
    out, kc, vc = run_gpu_op(case, validate=False, max_query_len=mq, max_context_len=mc)
    _check(case, out, kc, vc)
    # the same attention through the kernel-level entry on the updated caches
    cdt = case["cache_dtype"]
    t = {n: to_torch(case[n], dtype) for n in ("query", "key", "value")}
    I = {n: torch.from_numpy(np.ascontiguousarray(case[n], np.int32)).cuda()
         for n in ("cum", "past", "block_table")}
    again = ep.attention(t["query"], t["key"], t["value"], to_torch(kc, cdt), to_torch(vc, cdt),
                         I["cum"], I["past"], I["block_table"], num_heads=case["num_heads"],
                         k_scale=torch.from_numpy(case["k_scale"]).cuda(),
                         v_scale=torch.from_numpy(case["v_scale"]).cuda(),
                         k_quant_type=QUANT_NAMES[case.get("k_quant", 0)],
                         v_quant_type=QUANT_NAMES[case.get("v_quant", 0)],
                         max_query_len=mq, kind=2, new_rows_in_cache=True, max_context_len=mc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out, from_torch(again, dtype))
