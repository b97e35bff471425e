"""GPU parity of the planned prefill over operand images (heads 64, 96, 128 and 256).

When every 64-key step of values is read by at least four 128-row blocks (g * max_query_len >=
512 grouped query rows per sequence) the plan launch writes, once per (sequence, kv-head) and
64-key step, the key rows gathered from the pages and the value rows converted to fp16 under a
power-of-two scale of the step, both in the prefill kernel's LDS operand layout; the prefill
kernel stages them into LDS with direct loads and brings each step's values and its output
accumulator to one exponent.  Checked against the oracle rounded to T (rel-L2 <= 2e-3) and
against its float64 result (<= 4e-3), twice per case (bit-identical calls): both activation
dtypes, values far above and below the fp16 range, a few rows 1000x and 2^100 x larger than the
rest late in long sequences (step exponents rising and falling, the accumulator moved up and
down, and steps negligible against the output), block sizes 32 and 8 (keys addressed row by
row), new rows read from the inputs instead of the pages, softcap + window, sink logits, an
empty sequence, ragged chunks and a 7:1 head group.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16
from pa_cases import make_case, to_torch, from_torch

pytestmark = pytest.mark.gpu


def _run(case, dtype, nq, new_rows_in_cache):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    H = case["num_heads"]
    t = {n: to_torch(case[n], dtype) for n in ("query", "key", "value", "key_cache",
                                               "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    if new_rows_in_cache:
        ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                             I["past"], I["block_table"])
    hs = to_torch(case["head_sink"], dtype) if case.get("head_sink") is not None else None
    outs = [ep.attention(t["query"], t["key"], t["value"], t["key_cache"], t["value_cache"],
                         I["cum"], I["past"], I["block_table"], num_heads=H, max_query_len=nq,
                         kind=2, head_sink=hs, softcap=case["softcap"],
                         local_window_size=case["local_window_size"],
                         new_rows_in_cache=new_rows_in_cache) for _ in range(2)]
    torch.cuda.synchronize()
    return outs


def _check(case, dtype, nq, new_rows_in_cache):
    import torch
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    outs = _run(case, dtype, nq, new_rows_in_cache)
    cum = case["cum"]
    ref_d = orc.decode(ref_t, dtype)
    for out in outs:
        got = orc.decode(from_torch(out, dtype), dtype)
        # every sequence on its own (output magnitudes differ by up to 2^100 between them)
        for b in range(len(cum) - 1):
            rows = slice(int(cum[b]), int(cum[b + 1]))
            if rows.stop == rows.start:
                continue
            err_t = orc.rel_l2(got[rows], ref_d[rows])
            err64 = orc.rel_l2(got[rows].astype(np.float64), ref[rows])
            assert err_t <= 2e-3, (b, err_t)
            assert err64 <= 4e-3, (b, err64)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("d,dtype,bs,in_cache,vstd,softcap,window,sink,hot", [
    (128, BF16, 16, True, None, 0.0, -1, True, None),
    (128, F16, 16, True, None, 0.0, -1, True, None),
    (128, BF16, 16, True, 1e6, 0.0, -1, False, None),
    (128, BF16, 16, True, 1e-6, 0.0, -1, False, None),
    (128, BF16, 16, True, None, 0.0, -1, False, 1000.0),
    (128, BF16, 16, True, None, 0.0, -1, False, 2.0 ** 100),
    (128, BF16, 32, True, None, 30.0, 2900, True, None),
    (128, BF16, 8, False, None, 0.0, -1, False, None),
    (128, F16, 8, False, None, 0.0, -1, True, None),
    (64, BF16, 16, True, None, 0.0, -1, True, None),
    (64, F16, 8, False, None, 30.0, 2900, False, None),
    (64, BF16, 16, True, None, 0.0, -1, False, 2.0 ** 100),
    (256, BF16, 16, True, None, 0.0, -1, True, None),
    (256, F16, 32, True, None, 30.0, 2900, False, None),
    (256, BF16, 8, False, 1e6, 0.0, -1, True, None),
    (256, BF16, 16, True, None, 0.0, -1, False, 1000.0),
    (96, BF16, 16, True, None, 0.0, -1, True, None),
    (96, F16, 8, False, 300.0, 30.0, 2900, False, None),
    (96, BF16, 32, True, None, 0.0, -1, False, 2.0 ** 100)],
    ids=["bf16_sink", "f16_sink", "bf16_large_v", "bf16_tiny_v", "bf16_hot_rows",
         "bf16_extreme_rows",
         "bf16_block32_softcap_window", "bf16_block8_new_rows_from_inputs",
         "f16_block8_new_rows_from_inputs_sink", "d64_bf16_sink",
         "d64_f16_block8_softcap_window", "d64_bf16_extreme_rows", "d256_bf16_sink",
         "d256_f16_block32_softcap_window", "d256_bf16_block8_large_v_sink",
         "d256_bf16_hot_rows", "d96_bf16_sink", "d96_f16_block8_large_v_softcap_window",
         "d96_bf16_block32_extreme_rows"])
def test_prefill_images(d, dtype, bs, in_cache, vstd, softcap, window, sink, hot):
    rng = np.random.default_rng(5 + bs)
    B, H, KV, nq = 24, 32, 8, 128  # g * nq = 512 rows: 4 row blocks per sequence
    new_lens = np.full(B, nq)
    new_lens[3] = 0
    new_lens[9] = 77
    past = rng.integers(0, 600, size=B)
    past[[4, 20]] = [2900, 4000]  # items over the split threshold
    past[11] = 0
    mb = int((past.max() + nq + bs - 1) // bs)
    case = make_case(H, KV, d, B * mb, bs, B, dtype=dtype, seed=5 + bs, new_lens=new_lens,
                     past=past, max_blocks=mb, std=1.0, value_std=vstd, softcap=softcap,
                     window=window, head_sink=(rng.standard_normal(H) if sink else None))
    if hot is not None:
        # rows 2000..2015 and 3500..3515 of the two long sequences (in the middle and late)
        vc = orc.decode(case["value_cache"], dtype)
        for b in (4, 20):
            for pos in (2000, 3500):
                if pos < past[b]:
                    blk = case["block_table"][b, pos // bs]
                    vc[blk, pos % bs: pos % bs + 16] *= hot
        case["value_cache"] = orc.encode(vc, dtype)
    _check(case, dtype, nq, in_cache)


def test_prefill_images_group7_ragged():
    """Qwen-style 7:1 head groups (28 query / 4 kv heads), ragged 100..200-token chunks (up to
    11 row blocks per sequence), pasts up to 3000."""
    rng = np.random.default_rng(41)
    B, H, KV, d, bs = 16, 28, 4, 128, 16
    new_lens = rng.integers(100, 201, size=B)
    past = rng.integers(0, 3000, size=B)
    nq = int(new_lens.max())
    mb = int((past.max() + nq + bs - 1) // bs)
    case = make_case(H, KV, d, B * mb, bs, B, dtype=BF16, seed=41, new_lens=new_lens,
                     past=past, max_blocks=mb, std=1.0)
    _check(case, BF16, nq, True)


@pytest.mark.parametrize("d,B", [(128, 16), (64, 16), (96, 16), (128, 4), (256, 4)],
                         ids=["d128_images", "d64_images", "d96_images", "d128_in_loop",
                              "d256_in_loop"])
def test_step_with_a_huge_low_probability_value(d, B):
    """One key per (sequence, kv-head) carries a value row 2^40 times the others with a score
    ~42 below them (probability ~2^-60): its image step must not lose the ordinary values of
    the same step, which hold the attention mass of every row (a single exponent per step would
    put them 2^-40 below the step's largest value, under fp16's range).  Such steps keep raw bf16
    values and take their P.V product in bf16.  16 sequences fill the planned launch over images
    (heads 64/96/128; head 256 keeps one exponent per step: values more than 2^-29 below a step's
    largest lose bits there); 4 sequences take the grid launch without images, whose kernel
    multiplies raw bf16 values.  Per-sequence bars."""
    rng = np.random.default_rng(77 + d)
    H, KV, nq, bs = 32, 8, 128, 16
    past = np.resize(np.array([300, 450, 120, 600]), B)
    mb = int((past.max() + nq + bs - 1) // bs)
    case = make_case(H, KV, d, B * mb, bs, B, dtype=BF16, seed=77 + d, new_lens=np.full(B, nq),
                     past=past, max_blocks=mb, std=1.0)
    q = orc.decode(case["query"], BF16).reshape(-1, H, d)
    q[:, :, 0] = 4.0
    case["query"] = orc.encode(q.reshape(-1, H * d), BF16)
    kc = orc.decode(case["key_cache"], BF16)
    vc = orc.decode(case["value_cache"], BF16)
    for b in range(B):
        pos = 100
        blk, row = case["block_table"][b, pos // bs], pos % bs
        kc[blk, row] = 0.0
        kc[blk, row, :, 0] = -120.0 * np.sqrt(d / 128.0)
        vc[blk, row] = rng.standard_normal((KV, d)) * 2.0 ** 40
    case["key_cache"] = orc.encode(kc, BF16)
    case["value_cache"] = orc.encode(vc, BF16)
    _check(case, BF16, nq, True)
