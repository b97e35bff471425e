"""Multi-token batches over fp8 e4m3 pages on the matrix-core prefill, on the GPU through the C
ABI, against the oracle.

At heads 64, 96, 128 and 256 a batch with more than one query row per sequence over fp8 pages
(per-(block, kv-head) fp32 scales) runs the planned prefill over operand images: the plan launch
dequantises each 64-key step's key and value rows (e4m3 code x page scale in fp32) and writes
them as fp16 under one power of two per step for the keys and one for the values; the prefill
kernel takes the query rows to fp16 under a power of two per row, the scores and P.V on fp16
matrix cores, and each step's key exponent into its softmax scale.  Pages follow the config 5
draw (N(0,1) quantised with scale amax / 448 per (block, kv-head)); some cases spread the page
scales over many binades within one step (keys 2^+-6, values 2^+-40) or move them far from 1.

Bars: cache bytes bit-exact; outputs rel-L2 <= 2e-3 against the oracle rounded to T and
<= 4e-3 against its float64 result, per sequence.  The kernel-level entry pins the path: kind 2
forced runs, matches the automatic choice bit for bit, and agrees with the VALU kernel (kind 3).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, E4M3, F16
from pa_cases import from_torch, make_case, run_gpu_op, to_torch

pytestmark = pytest.mark.gpu


def _rounded(ref, dtype):
    return orc.decode(orc.encode(ref.astype(np.float32), dtype), dtype).astype(np.float64)


def _check_rows(got, ref, cum, dtype):
    want_t = _rounded(ref, dtype)
    for b in range(len(cum) - 1):
        rows = slice(int(cum[b]), int(cum[b + 1]))
        if rows.stop == rows.start:
            continue
        err_t = orc.rel_l2(got[rows], want_t[rows])
        err64 = orc.rel_l2(got[rows], ref[rows])
        assert err_t <= 2e-3, (b, err_t)
        assert err64 <= 4e-3, (b, err64)


def fp8_case(d, dtype, H=8, KV=2, bs=16, seed=0, kspread=0, vspread=0, smult=1.0, **kw):
    """Four sequences: prefill chunks of 150, 0, 37 and 200 rows over pasts of 300, 50, 0, 500.
    kspread / vspread: page scales times 2^U(-spread, spread) per (block, kv-head); smult: all
    page scales times smult."""
    kw.setdefault("new_lens", [150, 0, 37, 200])
    kw.setdefault("past", [300, 50, 0, 500])
    mb = (768 + bs - 1) // bs
    c = make_case(H, KV, d, 4 * mb, bs, 4, dtype=dtype, cache_dtype=E4M3,
                  seed=seed + 7 * d + bs, max_blocks=mb, **kw)
    rng = np.random.default_rng(seed + 99)
    for name, spread in (("k_scale", kspread), ("v_scale", vspread)):
        f = np.exp2(rng.uniform(-spread, spread, c[name].shape)) if spread else 1.0
        c[name] = (c[name] * f * smult).astype(np.float32)
    return c


def check_op(case):
    print(f"fp8-prefill case H={case['num_heads']} KV={case['kv_num_heads']} "
          f"d={case['head_dim']} act={orc.NAMES[case['dtype']]} "
          f"bs={case['key_cache'].shape[1]} softcap={case['softcap']} "
          f"window={case['local_window_size']}", flush=True)
    ref, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case)
    np.testing.assert_array_equal(kc, kc_ref)
    np.testing.assert_array_equal(vc, vc_ref)
    got = orc.decode(out, case["dtype"]).astype(np.float64)
    _check_rows(got, ref, case["cum"], case["dtype"])


@pytest.mark.parametrize("d,dtype", [(128, BF16), (128, F16), (64, BF16), (64, F16),
                                     (96, BF16), (96, F16), (256, BF16), (256, F16)],
                         ids=["d128-bf16", "d128-fp16", "d64-bf16", "d64-fp16", "d96-bf16",
                              "d96-fp16", "d256-bf16", "d256-fp16"])
def test_fp8_prefill_operator(d, dtype):
    check_op(fp8_case(d, dtype))


@pytest.mark.parametrize("d,bs", [(128, 32), (128, 8), (96, 8), (256, 32)])
def test_fp8_prefill_block_sizes(d, bs):
    check_op(fp8_case(d, BF16, bs=bs))


@pytest.mark.parametrize("d,dtype", [(128, BF16), (256, F16), (64, BF16), (96, BF16)])
def test_fp8_prefill_softcap_window_sink(d, dtype):
    H = 8
    check_op(fp8_case(d, dtype, H=H, softcap=30.0, window=260,
                      head_sink=np.linspace(-1.0, 1.0, H)))


# page scales spread over many binades inside one step, or all far from 1
@pytest.mark.parametrize("d,dtype,kspread,vspread,smult", [
    (128, BF16, 6, 40, 1.0), (128, F16, 6, 10, 1.0), (64, BF16, 3, 60, 1.0),
    (128, BF16, 0, 0, 2.0 ** 90), (128, BF16, 0, 0, 2.0 ** -90), (256, BF16, 4, 40, 1.0)],
    ids=["spread-bf16", "spread-fp16", "spread-d64", "large", "small", "spread-d256"])
def test_fp8_prefill_scales(d, dtype, kspread, vspread, smult):
    # large / small scales: the keys' scale is held at 1 (scores stay O(1)), the values' moved
    c = fp8_case(d, dtype, kspread=kspread, vspread=vspread)
    if smult != 1.0:
        c["v_scale"] = (c["v_scale"] * np.float32(smult)).astype(np.float32)
    check_op(c)


# 7:1 head group, ragged chunks, a sequence of one row among prefills
def test_fp8_prefill_group7_ragged():
    check_op(fp8_case(128, F16, H=14, KV=2, new_lens=[1, 300, 5, 64], past=[600, 0, 250, 10]))


def _attention(case, kc, vc, kind):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    dt = case["dtype"]
    I = lambda k: torch.from_numpy(np.ascontiguousarray(case[k], np.int32)).cuda()
    out = ep.attention(to_torch(case["query"], dt), to_torch(case["key"], dt),
                       to_torch(case["value"], dt), to_torch(kc, E4M3), to_torch(vc, E4M3),
                       I("cum"), I("past"), I("block_table"), num_heads=case["num_heads"],
                       softcap=case["softcap"], local_window_size=case["local_window_size"],
                       k_scale=torch.from_numpy(case["k_scale"]).cuda(),
                       v_scale=torch.from_numpy(case["v_scale"]).cuda(), kind=kind,
                       new_rows_in_cache=True)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("d,dtype", [(128, BF16), (64, F16), (256, BF16), (96, F16)])
def test_fp8_prefill_kernel_level_kinds(d, dtype):
    import torch
    c = fp8_case(d, dtype, kspread=2, vspread=8)
    print(f"fp8-prefill kinds d={d} act={orc.NAMES[dtype]}", flush=True)
    ref, _, kc, vc = orc.paged_attention_op(c)
    auto = _attention(c, kc, vc, 0)
    mx = _attention(c, kc, vc, 2)
    valu = _attention(c, kc, vc, 3)
    assert torch.equal(auto, mx)  # the automatic choice is the matrix-core prefill
    for out in (mx, valu):
        got = orc.decode(from_torch(out, dtype), dtype).astype(np.float64)
        _check_rows(got, ref, c["cum"], dtype)


# rows of 768 and 1024 elements over all kv-heads: the append quantises them in two pieces
@pytest.mark.parametrize("d", [96, 128])
def test_fp8_prefill_wide_rows(d):
    check_op(fp8_case(d, BF16, H=16, KV=8, new_lens=[40, 3, 0, 77], past=[100, 5, 9, 300]))
