"""GroupQueryAttention forms that run on the matrix-core kernels (pa_group_query_attention through
the C ABI) against the oracle's restatement orc_gqa_batched (gqa_batched, attention.rs:586-848):

  * decode batches over int8 / int4 present caches on the streaming decode in contiguous-row
    addressing (codes read per lane from the rows of each (sequence, kv-head));
  * an additive attention_bias (attention.rs:308-359 masks, bias added after the scale and
    softcap) on the streaming decode and on prefill_kernel at heads 64 / 96 / 128 / 256, in
    every broadcast shape, with softcap, window and sink, over bf16 / fp16 and integer presents;
  * ragged first prompts (sequences shorter than the padded query rows: per-sequence key counts)
    on the prefill kernels (planned launch, operand images, int8 presents) and the streaming
    decode.

Bars: present caches bit-exact; outputs rel-L2 <= 2e-3 against the T-rounded oracle output and
<= 4e-3 against its fp64 output (the check of test_gpu_gqa_forms).
"""
from __future__ import annotations

import numpy as np
import pytest

from _oracle import BF16, F16, I4, I8, PER_CHANNEL, PER_TENSOR
from gqa_cases import gqa_case
from test_gpu_gqa_forms import check

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- integer presents, decode
@pytest.mark.parametrize("cache", [I8, I4], ids=["int8", "int4"])
@pytest.mark.parametrize("dtype,d,H,KV", [(BF16, 128, 32, 8), (F16, 64, 16, 2)],
                         ids=["bf16_d128", "fp16_d64"])
@pytest.mark.parametrize("modes", [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL),
                                   (PER_CHANNEL, PER_TENSOR)], ids=["pt", "pc", "pc_pt"])
def test_int_present_decode_streaming(cache, dtype, d, H, KV, modes):
    # capacity 1000 (not a multiple of the 32-key step): the longest sequence's last step reads
    # rows past the capacity, which re-read its last row
    rng = np.random.default_rng(d + cache + 3 * modes[0] + modes[1])
    B, cap = 6, 1000
    seqlens = rng.integers(8, cap - 2, size=B)
    seqlens[0] = cap - 2
    c = gqa_case(dtype, B, 1, H, KV, d, seqlens, cap=cap, seed=d + cache, rotary=True,
                 theta=500000.0, cache_dtype=cache, modes=modes)
    check(c, present="shared")


@pytest.mark.parametrize("cache", [I8, I4], ids=["int8", "int4"])
@pytest.mark.parametrize("variant", ["new_present", "window_sink_softcap", "rows4"])
def test_int_present_decode_streaming_forms(cache, variant):
    rng = np.random.default_rng(31 + cache + len(variant))
    B, H, KV, d, cap = 5, 32, 8, 128, 700
    seqlens = rng.integers(40, cap - 5, size=B)
    kw = dict(cap=cap, rotary=True, theta=500000.0, cache_dtype=cache,
              modes=(PER_CHANNEL, PER_CHANNEL))
    S = 1
    if variant == "window_sink_softcap":
        kw.update(window=100, sink=True, softcap=20.0)
    if variant == "rows4":  # 4 new rows x g = 4: 16 grouped rows, still the streaming decode
        S = 4
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, seed=41 + cache, **kw)
    check(c, present="new" if variant == "new_present" else "shared")


# ------------------------------------------------------------------------------ bias, decode
@pytest.mark.parametrize("d", [64, 96, 128, 256])
@pytest.mark.parametrize("shape", ["b_h", "1_1", "b_1", "1_h"])
def test_bias_decode_streaming(d, shape):
    rng = np.random.default_rng(d + len(shape))
    B, H, KV, cap = 4, 16, 4, 600
    seqlens = rng.integers(10, cap - 1, size=B)
    total = int(seqlens.max()) + 1
    bshape = {"b_h": (B, H, 1, total), "1_1": (1, 1, 1, total), "b_1": (B, 1, 1, total),
              "1_h": (1, H, 1, total)}[shape]
    c = gqa_case(BF16 if d != 96 else F16, B, 1, H, KV, d, seqlens, cap=cap, seed=d + 5,
                 rotary=True, theta=500000.0, bias_shape=bshape)
    check(c, present="shared")


@pytest.mark.parametrize("variant", ["softcap_sink", "window", "smooth", "int8", "int4", "rows4"])
def test_bias_decode_streaming_forms(variant):
    rng = np.random.default_rng(50 + len(variant))
    B, H, KV, d, cap = 5, 32, 8, 128, 900
    seqlens = rng.integers(10, cap - 4, size=B)
    S = 4 if variant == "rows4" else 1
    total = int(seqlens.max()) + 1
    kw = dict(cap=cap, rotary=True, theta=500000.0, bias_shape=(B, H, S, total))
    if variant == "softcap_sink":
        kw.update(softcap=15.0, sink=True)
    elif variant == "window":
        kw.update(window=64)
    elif variant == "smooth":
        kw.update(smooth=1)
    elif variant in ("int8", "int4"):
        kw.update(cache_dtype=I8 if variant == "int8" else I4, modes=(PER_CHANNEL, PER_TENSOR))
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, seed=60 + len(variant), **kw)
    check(c, present="shared")


# ------------------------------------------------------------------------ bias, multi-token
@pytest.mark.parametrize("d", [64, 96, 128, 256])
@pytest.mark.parametrize("variant", ["chunk", "window_softcap", "first_prompt"])
def test_bias_multi_token_prefill(d, variant):
    rng = np.random.default_rng(d + 7 * len(variant))
    B, S, H, KV = 3, 48, 16, 4
    if variant == "first_prompt":
        seqlens = np.full(B, S - 1)
        c = gqa_case(BF16, B, S, H, KV, d, seqlens, seed=d + 70, rotary=True, theta=500000.0,
                     bias_shape=(B, 1, S, S))
        check(c)
        return
    seqlens = rng.integers(S, 500, size=B)
    total = int(seqlens.max()) + 1
    kw = dict(cap=517, rotary=True, theta=500000.0, bias_shape=(1, H, S, total))
    if variant == "window_softcap":
        kw.update(window=77, softcap=12.0, sink=True)
    c = gqa_case(F16 if d == 96 else BF16, B, S, H, KV, d, seqlens, seed=d + 71, **kw)
    check(c, present="shared")


def test_bias_multi_token_planned_launch():
    # enough (sequence, kv-head, 128-row block) items for the planned launch, one long item split
    rng = np.random.default_rng(78)
    B, S, H, KV, d = 16, 128, 32, 8, 128
    seqlens = rng.integers(S, 400, size=B)
    seqlens[3] = 2999
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, cap=3000, seed=78, rotary=True,
                 theta=500000.0, bias_shape=(B, 1, S, 3000))
    check(c, present="shared")


# ------------------------------------------------------------------------ ragged first prompts
@pytest.mark.parametrize("dtype,d", [(BF16, 128), (F16, 128), (BF16, 64), (F16, 96),
                                     (BF16, 256)], ids=["bf16_128", "fp16_128", "bf16_64",
                                                        "fp16_96", "bf16_256"])
def test_ragged_first_prompt_prefill(dtype, d):
    rng = np.random.default_rng(d + dtype)
    B, S, H, KV = 4, 96, 16, 4
    seqlens = rng.integers(5, S - 1, size=B)
    seqlens[0] = S - 1
    c = gqa_case(dtype, B, S, H, KV, d, seqlens, seed=d + 80, rotary=True, theta=500000.0,
                 pid=np.zeros((B, S), np.int64))
    check(c)


def test_ragged_first_prompt_planned_launch():
    # 16 sequences x 8 kv-heads x 2 row blocks: the planned launch over operand images
    rng = np.random.default_rng(90)
    B, S, H, KV, d = 16, 64, 32, 8, 128
    seqlens = rng.integers(3, S - 1, size=B)
    seqlens[5] = S - 1
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, seed=90, rotary=True, theta=500000.0,
                 pid=np.zeros((B, S), np.int64))
    check(c)


@pytest.mark.parametrize("cache", [I8, I4], ids=["int8", "int4"])
def test_ragged_first_prompt_int_presents(cache):
    # integer presents: the planned launch over code images, with per-sequence key counts
    rng = np.random.default_rng(95 + cache)
    B, S, H, KV, d = 6, 64, 16, 4, 128
    seqlens = rng.integers(3, S - 1, size=B)
    seqlens[2] = S - 1
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, cap=S, seed=95 + cache, rotary=True,
                 theta=500000.0, cache_dtype=cache, modes=(PER_CHANNEL, PER_CHANNEL))
    check(c)


def test_ragged_first_prompt_decode_rows():
    # 4 query rows x g = 4: the streaming decode with per-sequence key counts
    B, S, H, KV, d = 5, 4, 16, 4, 128
    seqlens = np.array([3, 0, 1, 2, 3])
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, seed=99, rotary=True, theta=500000.0,
                 pid=np.zeros((B, S), np.int64))
    check(c)
