"""GPU parity: the HIP path through the C ABI against the CPU oracle on identical seeded inputs.

Bars: cache bytes after append bit-exact; outputs within
rel-L2 <= 2e-3 (fp16/bf16) or <= 1e-5 (fp32).  For fp16/bf16 the output is compared with the
oracle's output rounded to the activation dtype (the reference returns T), and additionally
with the unrounded float64 result at twice the bar.  Geometries mirror the reference's
tests/ops/test_paged_attention.py cases (cited per test) plus the BASELINE.json configs.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, E4M3, F16, F32
from pa_cases import make_case, run_gpu_op

pytestmark = pytest.mark.gpu

TOL = {F16: 2e-3, BF16: 2e-3, F32: 1e-5}


def check(case, validate=True, tol=None):
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case, validate=validate)
    assert np.array_equal(kc, kc_ref), "key cache differs from the oracle"
    assert np.array_equal(vc, vc_ref), "value cache differs from the oracle"
    dt = case["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    bar = TOL[dt] if tol is None else tol
    if dt == F32:
        err = orc.rel_l2(got, ref)
        assert err <= bar, f"rel-L2 {err:.3e} > {bar}"
    else:
        err_t = orc.rel_l2(got, orc.decode(ref_t, dt))
        err64 = orc.rel_l2(got, ref)
        assert err_t <= bar, f"rel-L2 vs T-rounded oracle {err_t:.3e} > {bar}"
        assert err64 <= 2 * bar, f"rel-L2 vs fp64 oracle {err64:.3e} > {2 * bar}"
    return out


# test_paged_attention.py:239-242 (GQA/MHA/MQA x batch 1/3, d=16, block 4)
@pytest.mark.parametrize("H,KV", [(4, 2), (4, 4), (8, 2), (2, 1)], ids=["gqa", "mha", "gqa8", "mqa"])
@pytest.mark.parametrize("batch", [1, 3])
def test_core(H, KV, batch):
    check(make_case(H, KV, 16, 8 * batch, 4, batch, dtype=F16, seed=H * 10 + KV + batch))


# same geometries at MFMA-kernel head sizes, both activation dtypes
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [F16, BF16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("H,KV", [(4, 2), (8, 2), (2, 1), (8, 8)])
def test_core_mfma(d, dtype, H, KV):
    check(make_case(H, KV, d, 32, 16, 3, dtype=dtype, seed=d + H + KV))


# test_paged_attention.py:245-247 (head 256)
@pytest.mark.parametrize("kv", [1, 4])
def test_head256(kv):
    check(make_case(24, kv, 256, 4, 64, 1, dtype=F16, seed=256 + kv))


# test_paged_attention.py:250-280 (causal x window decode replay)
@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("window", [-1, 1, 3])
@pytest.mark.parametrize("d", [16, 64])
def test_mask_variants(causal, window, d):
    for nt in (3, 1, 2, 1):
        check(make_case(4, 2, d, 4, 4, 1, dtype=F16, seed=943 + nt, new_lens=[nt], past=[5],
                        causal=causal, window=window))


# test_paged_attention.py:284-286 (multi-block gather)
@pytest.mark.parametrize("blk", [2, 8, 16])
def test_multiblock(blk):
    check(make_case(8, 2, 32, 16, blk, 2, dtype=F16, seed=blk + 7))
    check(make_case(8, 2, 64, 16, blk, 2, dtype=BF16, seed=blk + 8))


# test_paged_attention.py:289-318 (long context x 1/5/8 queries)
@pytest.mark.parametrize("past", [4095, 16383])
@pytest.mark.parametrize("queries", [1, 5, 8])
@pytest.mark.parametrize("geom", [(24, 4, 256, 256), (8, 2, 128, 16)], ids=["d256", "d128"])
def test_long_context(past, queries, geom):
    H, KV, d, blk = geom
    blocks = (past + queries + blk - 1) // blk
    check(make_case(H, KV, d, blocks, blk, 1, dtype=F16, seed=412, new_lens=[queries],
                    past=[past]), tol=3e-3 if d == 256 else None)


# test_paged_attention.py:321-376 (slot_mapping normal / overwrite / skip, caches exact)
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("mapping", ["normal", "overwrite", "skip"])
@pytest.mark.parametrize("d", [64, 128])
def test_cache_overlay(causal, mapping, d):
    queries, past = 5, 1022
    base = make_case(4, 2, d, 8, 256, 1, dtype=F16, seed=417, new_lens=[queries], past=[past],
                     causal=causal)
    slots = None
    if mapping == "skip":
        slots = np.full(queries, -1, np.int32)
    elif mapping == "overwrite":
        slots = (base["block_table"][0, 0] * 256 + np.arange(queries)).astype(np.int32)
    if slots is not None:
        base["slot_mapping"] = slots
    check(base)


# test_paged_attention.py:605-659 (duplicate slots: the last token's row stays)
def test_duplicate_slots_known_answer():
    case = make_case(1, 1, 64, 2, 16, 1, dtype=F16, seed=42, new_lens=[2], past=[0])
    case["query"] = np.ones((2, 64), np.float16)
    case["key"] = np.stack([np.full(64, 1), np.full(64, 2)]).astype(np.float16)
    case["value"] = np.stack([np.full(64, 3), np.full(64, 4)]).astype(np.float16)
    case["slot_mapping"] = np.array([0, 0], np.int32)
    out, kc, vc = run_gpu_op(case)
    assert np.all(kc[0, 0, 0] == np.float16(2)) and np.all(vc[0, 0, 0] == np.float16(4))
    check(case)


# duplicate slots through the block table (no slot mapping): sequence 2's new positions land on
# the block sequence 0 writes, at overlapping offsets, and sequence 1's row names one block twice,
# so its later positions overwrite its earlier ones.  The last writer in token order must win
# (sequential scatter); the host metadata shows the slots are not distinct, so the append runs
# its block-table last-writer check.
@pytest.mark.parametrize("dtype", [F16, BF16], ids=["fp16", "bf16"])
def test_block_table_duplicate_slots(dtype):
    case = make_case(4, 2, 64, 12, 16, 3, dtype=dtype, seed=91, new_lens=[5, 20, 7],
                     past=[3, 10, 3], max_blocks=4, std=1.0)
    case["block_table"] = np.array([[0, 1, 2, 3], [4, 4, 5, 6], [0, 8, 9, 10]], np.int32)
    check(case)


# test_paged_attention.py:663-666 (RoPE neox / gptj) + the BASELINE.json bf16 theta=500000 rotary
@pytest.mark.parametrize("interleaved", [0, 1], ids=["neox", "gptj"])
@pytest.mark.parametrize("H,KV,d,dtype", [(4, 2, 16, F16), (2, 1, 64, F16), (32, 8, 128, BF16)])
def test_rotary(interleaved, H, KV, d, dtype):
    check(make_case(H, KV, d, 16, 4 if d < 128 else 16, 2, dtype=dtype, do_rotary=1,
                    interleaved=interleaved, theta=500000.0 if dtype == BF16 else 10000.0,
                    seed=H + d + interleaved))


@pytest.mark.parametrize("offset,rot", [(8, 16), (0, 32), (16, 32)])
def test_partial_rotary_offset(offset, rot):
    check(make_case(4, 2, 64, 16, 16, 2, dtype=BF16, do_rotary=1, rot_dim=rot,
                    rotary_offset=offset, seed=offset + rot))


# test_paged_attention.py:855-983 (slot_mapping, head_sink, q/k norm, attention_metadata)
@pytest.mark.parametrize("dtype", [F16, BF16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("d", [8, 64])
def test_optional_inputs(dtype, d):
    case = make_case(4, 2, d, 4, 4, 1, dtype=dtype, seed=129, new_lens=[2], past=[3],
                     slot_mapping=[3, 9], head_sink=[-0.5, 0.25, 1.0, -1.0], qk_norm=True,
                     std=1.0)
    case["block_table"] = np.array([[2, 0, 1, 3]], np.int32)
    check(case)


@pytest.mark.parametrize("softcap", [0.0, 5.0, 30.0])
@pytest.mark.parametrize("d", [16, 128])
def test_softcap_and_sink(softcap, d):
    check(make_case(8, 2, d, 64, 16, 3, dtype=BF16, seed=77, softcap=softcap,
                    head_sink=np.linspace(-1, 2, 8), std=1.0))


# a negative softmax scale (an attribute value the reference passes through unchanged): the
# kernels take |scale| and move the sign into the query operands -- MFMA decode, the prefill
# kernel, the VALU kernel (d 16), softcap, and fp8 pages
@pytest.mark.parametrize("d,dtype,cache,nq,softcap", [
    (128, BF16, None, 1, 0.0), (128, F16, None, 40, 0.0), (16, F16, None, 3, 0.0),
    (128, BF16, None, 1, 5.0), (128, BF16, E4M3, 1, 0.0)],
    ids=["decode", "prefill", "valu", "softcap", "fp8"])
def test_negative_scale(d, dtype, cache, nq, softcap):
    rng = np.random.default_rng(d + nq)
    B, bs = 3, 16
    past = rng.integers(100, 900, size=B)
    mb = int((past.max() + nq + bs - 1) // bs)
    check(make_case(8, 2, d, B * mb + 2, bs, B, dtype=dtype, cache_dtype=cache, seed=d + nq,
                    new_lens=[nq] * B, past=past, max_blocks=mb, std=1.0, softcap=softcap,
                    scale=-0.11))


# GroupQueryAttention decode, fp32, B=1, 8q/2kv, d=64, past 128 + 1 new,
# no rotary, scale 1/8 -- the GPU paged path on the equivalent pages must agree with the
# contiguous-KV (ORT CPU semantics) restatement to rel-L2 <= 1e-5.
def test_c1_gqa_fp32_against_contiguous():
    rng = np.random.default_rng(1)
    H, KV, d, past = 8, 2, 64, 128
    q = rng.standard_normal((1, 1, H * d)).astype(np.float32)
    k = rng.standard_normal((1, 1, KV * d)).astype(np.float32)
    v = rng.standard_normal((1, 1, KV * d)).astype(np.float32)
    pk = rng.standard_normal((1, KV, past + 1, d)).astype(np.float32)
    pv = rng.standard_normal((1, KV, past + 1, d)).astype(np.float32)
    ref, _, _ = orc.gqa_contiguous(F32, q, k, v, pk, pv, np.array([past]), H, KV, d, 0.125)
    bs = 16
    nb = (past + 1 + bs - 1) // bs
    kc = np.zeros((nb, bs, KV, d), np.float32)
    vc = np.zeros_like(kc)
    for p in range(past):
        kc[p // bs, p % bs] = pk[0, :, p]
        vc[p // bs, p % bs] = pv[0, :, p]
    case = dict(num_heads=H, kv_num_heads=KV, head_dim=d, dtype=F32, cache_dtype=F32,
                cum=np.array([0, 1], np.int32), past=np.array([past], np.int32),
                block_table=np.arange(nb, dtype=np.int32)[None], query=q.reshape(1, H * d),
                key=k.reshape(1, KV * d), value=v.reshape(1, KV * d), key_cache=kc,
                value_cache=vc, scale=0.125, is_causal=1, local_window_size=-1, softcap=0.0)
    import onnxruntime_ep_mlx_amd as ep
    import torch
    from pa_cases import to_torch, from_torch
    t = {n: to_torch(case[n], F32) for n in ("query", "key", "value", "key_cache", "value_cache")}
    I = lambda a: torch.from_numpy(a).cuda()
    out, kc_t, vc_t = ep.paged_attention(
        t["query"], t["key"], t["value"], t["key_cache"], t["value_cache"], I(case["cum"]),
        I(case["past"]), I(case["block_table"]), num_heads=H, kv_num_heads=KV, scale=0.125)
    torch.cuda.synchronize()
    got = from_torch(out, F32).reshape(ref.shape)
    err = orc.rel_l2(got, ref)
    assert err <= 1e-5, err
    # present cache rows equal the contiguous present rows
    kc_g = from_torch(kc_t, F32)
    assert np.array_equal(kc_g[past // bs, past % bs], k.reshape(KV, d))


# BASELINE.json config 3 geometry (Llama-3-8B decode), reduced batch for the oracle
@pytest.mark.parametrize("kind", [0, 3], ids=["auto", "generic"])
def test_c3_geometry_reduced_batch(kind):
    rng = np.random.default_rng(3)
    B, bs = 8, 16
    ctx = rng.integers(512, 8193, size=B)
    max_blocks = int((ctx.max() + bs - 1) // bs)
    case = make_case(32, 8, 128, B * max_blocks, bs, B, dtype=BF16, seed=3, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=max_blocks, do_rotary=1, theta=500000.0, std=1.0)
    if kind == 0:
        check(case)
        return
    # force the generic kernel through the kernel-level entry points
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value", "key_cache",
                                              "value_cache", "cos_cache", "sin_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    qr, kr = ep.rotary_append(t["query"], t["key"], t["value"], t["key_cache"],
                              t["value_cache"], I["cum"], I["past"], I["block_table"],
                              num_heads=32, cos_cache=t["cos_cache"], sin_cache=t["sin_cache"])
    out = ep.attention(qr, kr, t["value"], t["key_cache"], t["value_cache"], I["cum"],
                       I["past"], I["block_table"], num_heads=32, max_query_len=1, kind=3)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(t["key_cache"], BF16), kc_ref)
    err = orc.rel_l2(orc.decode(from_torch(out, BF16), BF16), orc.decode(ref_t, BF16))
    assert err <= 2e-3, err


# split-K invariance: every chunk size gives the oracle's answer (chunked MFMA and VALU kernels)
@pytest.mark.parametrize("chunk", [32, 64, 256, 1024])
@pytest.mark.parametrize("kind", [4, 3], ids=["mfma_chunked", "generic"])
def test_split_k_chunks(chunk, kind):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    rng = np.random.default_rng(11)
    B, bs = 4, 16
    ctx = rng.integers(100, 3000, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    case = make_case(16, 4, 128, B * mb, bs, B, dtype=BF16, seed=11, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, std=1.0)
    ref, ref_t, kc_ref, _ = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value", "key_cache",
                                              "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                         I["past"], I["block_table"])
    out = ep.attention(t["query"], t["key"], t["value"], t["key_cache"], t["value_cache"],
                       I["cum"], I["past"], I["block_table"], num_heads=16, max_query_len=1,
                       kind=kind, chunk=chunk)
    torch.cuda.synchronize()
    err = orc.rel_l2(orc.decode(from_torch(out, BF16), BF16), orc.decode(ref_t, BF16))
    assert err <= 2e-3, err


# LDS-shared prefill kernel through the kernel-level entries: ragged multi-token queries (one
# sequence empty), split-K chunks, page sizes that do or do not hold whole 16-key tiles, new
# rows read from the pages or from the caller's rows, windows and softcap
@pytest.mark.parametrize("chunk", [0, 32, 96, 512])
@pytest.mark.parametrize("new_rows_in_cache", [False, True])
@pytest.mark.parametrize("bs,d,dtype,window,softcap", [
    (16, 128, BF16, -1, 0.0), (8, 128, F16, -1, 0.0), (32, 64, BF16, 100, 0.0),
    (16, 64, F16, -1, 20.0)], ids=["bs16_d128", "bs8_d128", "bs32_d64_window", "d64_softcap"])
def test_prefill_kernel_level(chunk, new_rows_in_cache, bs, d, dtype, window, softcap):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    rng = np.random.default_rng(20 + bs + d)
    B, H, KV = 4, 14, 2
    new_lens = [37, 0, 70, 5]
    past = rng.integers(0, 600, size=B)
    mb = int((past.max() + max(new_lens) + bs - 1) // bs)
    case = make_case(H, KV, d, B * mb, bs, B, dtype=dtype, seed=20 + bs + d, new_lens=new_lens,
                     past=past, max_blocks=mb, std=1.0, window=window, softcap=softcap)
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], dtype) for n in ("query", "key", "value", "key_cache",
                                               "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                         I["past"], I["block_table"])
    outs = {}
    for kind in (2, 4):
        outs[kind] = ep.attention(t["query"], t["key"], t["value"], t["key_cache"],
                                  t["value_cache"], I["cum"], I["past"], I["block_table"],
                                  num_heads=H, max_query_len=max(new_lens), kind=kind,
                                  chunk=chunk, local_window_size=window, softcap=softcap,
                                  new_rows_in_cache=new_rows_in_cache)
    torch.cuda.synchronize()
    for kind, out in outs.items():
        got = orc.decode(from_torch(out, dtype), dtype)
        err = orc.rel_l2(got, orc.decode(ref_t, dtype))
        assert err <= 2e-3, (kind, err)
        assert orc.rel_l2(got.astype(np.float64), ref) <= 4e-3, kind


# planned prefill (library-chosen plan with at least two workgroups per CU, 512 items here on a
# 256-CU MI355X): units ordered longest first, items past the split threshold run as two halves
# merged afterwards, one sequence without new tokens (no items), and a sink logit that only the
# merge of the split items folds in for those rows.  The halves' partials are fp16 rows scaled
# by a power of two per row: values far outside the fp16 range (bf16 values ~1e6) and far below
# its normal range (~1e-6) must merge within the same bar.
@pytest.mark.parametrize("d,dtype,sink,vstd,softcap,window", [
    (64, BF16, False, None, 0.0, -1), (128, F16, True, None, 0.0, -1),
    (128, BF16, True, 1e6, 0.0, -1), (64, BF16, False, 1e-6, 0.0, -1),
    (128, BF16, True, None, 30.0, 2900), (256, BF16, True, None, 0.0, -1),
    (96, F16, False, None, 30.0, 2900)],
    ids=["d64_bf16", "d128_f16_sink", "d128_bf16_large_v", "d64_bf16_tiny_v",
         "d128_bf16_softcap_window", "d256_bf16_sink", "d96_f16_softcap_window_grid"])
def test_prefill_planned(d, dtype, sink, vstd, softcap, window):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    rng = np.random.default_rng(71 + d)
    B, H, KV, bs, nq = 64, 32, 8, 16, 16
    new_lens = np.full(B, nq)
    new_lens[5] = 0
    past = rng.integers(0, 300, size=B)
    past[[17, 63]] = [2600, 3500]  # items longer than the 2048-key threshold
    mb = int((past.max() + nq + bs - 1) // bs)
    case = make_case(H, KV, d, B * mb, bs, B, dtype=dtype, seed=71 + d, new_lens=new_lens,
                     past=past, max_blocks=mb, std=1.0, value_std=vstd, softcap=softcap,
                     window=window, head_sink=(rng.standard_normal(H) if sink else None))
    ref, ref_t, _, _ = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], dtype) for n in ("query", "key", "value", "key_cache",
                                               "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                         I["past"], I["block_table"])
    hs = to_torch(case["head_sink"], dtype) if sink else None
    outs = [ep.attention(t["query"], t["key"], t["value"], t["key_cache"], t["value_cache"],
                         I["cum"], I["past"], I["block_table"], num_heads=H, max_query_len=nq,
                         kind=2, head_sink=hs, softcap=softcap, local_window_size=window,
                         new_rows_in_cache=True) for _ in range(2)]
    torch.cuda.synchronize()
    for out in outs:
        got = orc.decode(from_torch(out, dtype), dtype)
        assert orc.rel_l2(got, orc.decode(ref_t, dtype)) <= 2e-3
        assert orc.rel_l2(got.astype(np.float64), ref) <= 4e-3
    # the unit order inside a histogram bucket may differ between calls; the rows may not
    assert torch.equal(outs[0], outs[1])


# balanced decode kernel through the kernel-level entries: segments that split sequences,
# sequences of one step, the separate partial merge, and both sources of the new rows
@pytest.mark.parametrize("new_rows_in_cache", [False, True])
@pytest.mark.parametrize("B,lo,hi", [(4, 100, 3000), (64, 1, 40), (37, 1, 9000)])
def test_balanced_decode_kernel_level(new_rows_in_cache, B, lo, hi):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    rng = np.random.default_rng(B + lo)
    bs = 16
    ctx = rng.integers(lo, hi + 1, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    case = make_case(32, 8, 128, B * mb, bs, B, dtype=BF16, seed=B + hi, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, std=1.0)
    ref, ref_t, kc_ref, _ = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value", "key_cache",
                                              "value_cache")}
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], t["key_cache"], t["value_cache"], I["cum"],
                         I["past"], I["block_table"])
    outs = []
    for _ in range(2):  # twice: the workspace left by one call must not leak into the next
        outs.append(ep.attention(t["query"], t["key"], t["value"], t["key_cache"],
                                 t["value_cache"], I["cum"], I["past"], I["block_table"],
                                 num_heads=32, max_query_len=1, kind=1,
                                 new_rows_in_cache=new_rows_in_cache))
    torch.cuda.synchronize()
    for out in outs:
        err = orc.rel_l2(orc.decode(from_torch(out, BF16), BF16), orc.decode(ref_t, BF16))
        assert err <= 2e-3, err
    assert torch.equal(outs[0], outs[1])


# batches beyond one wavefront: the 64-way sequence search takes two levels (append, generic
# kernel) and the balanced decode scans sequences in several 64-wide chunks; decode and mixed
# decode/prefill, with rotary so the query rows go through the append kernel too
@pytest.mark.parametrize("B,mixed", [(65, False), (300, False), (150, True)])
def test_large_batch(B, mixed):
    rng = np.random.default_rng(B)
    bs, mb = 16, 12
    new = rng.integers(1, 5, size=B) if mixed else np.ones(B, np.int64)
    past = np.array([rng.integers(0, mb * bs - n + 1) for n in new])
    check(make_case(8, 2, 128, B * mb, bs, B, dtype=BF16, seed=B, new_lens=new, past=past,
                    max_blocks=mb, do_rotary=1, std=1.0))


# BASELINE.json config 4 geometry (Qwen2.5-7B chunked prefill), reduced
@pytest.mark.parametrize("dtype", [BF16, F16], ids=["bf16", "fp16"])
def test_c4_prefill_reduced(dtype):
    rng = np.random.default_rng(4)
    B, bs, chunk = 2, 16, 64
    past = rng.integers(0, 700, size=B)
    mb = int((past.max() + chunk + bs - 1) // bs)
    check(make_case(28, 4, 128, B * mb, bs, B, dtype=dtype, seed=4, new_lens=[chunk] * B,
                    past=past, max_blocks=mb, std=1.0))


# BASELINE.json config 5 geometry (fp8 e4m3 pages, per-(block, kv-head) scales), reduced
@pytest.mark.parametrize("ctx", [1, 300, 4096])
def test_c5_fp8_reduced(ctx):
    bs = 16
    mb = (ctx + bs - 1) // bs
    check(make_case(64, 8, 128, 2 * mb + 2, bs, 2, dtype=BF16, cache_dtype=E4M3, seed=5,
                    new_lens=[1, 1], past=[ctx - 1, max(ctx - 5, 0)], max_blocks=mb, std=1.0))


# fp8 pages on the matrix-core decode: both activation dtypes, d 64/128, softcap, two-token
# queries (g * nq <= 16), page sizes 8 (VALU fallback), 16 and 32, many-way split sequences
@pytest.mark.parametrize("dtype,d,bs,softcap,nq", [
    (BF16, 128, 16, 0.0, 1), (F16, 128, 16, 0.0, 1), (BF16, 64, 16, 0.0, 1),
    (BF16, 128, 32, 0.0, 1), (BF16, 128, 8, 0.0, 1), (BF16, 128, 16, 30.0, 1),
    (F16, 128, 16, 0.0, 2)])
def test_fp8_pages_decode(dtype, d, bs, softcap, nq):
    rng = np.random.default_rng(d + bs + nq)
    B = 5
    ctx = rng.integers(40, 1500, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    check(make_case(16, 4, d, B * mb + 3, bs, B, dtype=dtype, cache_dtype=E4M3,
                    seed=int(ctx.sum()), new_lens=[nq] * B, past=ctx - nq, max_blocks=mb,
                    std=1.0, softcap=softcap))


# fp8 decode at BASELINE.json config 5's per-sequence shape (64 q / 8 kv heads, 32768 keys),
# two sequences: the fp8 streaming kernel against the VALU kernel on identical pages, plus the
# oracle on one sequence
def test_fp8_long_context_matches_valu():
    import torch
    import onnxruntime_ep_mlx_amd as ep
    from pa_cases import to_torch, from_torch
    bs, ctx, B = 16, 32768, 2
    mb = ctx // bs
    case = make_case(64, 8, 128, B * mb + 2, bs, B, dtype=BF16, cache_dtype=E4M3, seed=55,
                     new_lens=[1] * B, past=[ctx - 1, ctx - 1001], max_blocks=mb, std=1.0)
    ref, ref_t, kc_ref, vc_ref = orc.paged_attention_op(case)
    t = {n: to_torch(case[n], BF16) for n in ("query", "key", "value")}
    kc, vc = to_torch(case["key_cache"], E4M3), to_torch(case["value_cache"], E4M3)
    ks, vs = (torch.from_numpy(case[n]).cuda() for n in ("k_scale", "v_scale"))
    I = {n: torch.from_numpy(case[n]).cuda() for n in ("cum", "past", "block_table")}
    ep.reshape_and_cache(t["key"], t["value"], kc, vc, I["cum"], I["past"], I["block_table"],
                         k_scale=ks, v_scale=vs)
    outs = [ep.attention(t["query"], t["key"], t["value"], kc, vc, I["cum"], I["past"],
                         I["block_table"], num_heads=64, max_query_len=1, kind=kind,
                         k_scale=ks, v_scale=vs) for kind in (1, 3)]
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(kc, E4M3), kc_ref)
    g1, g3 = (orc.decode(from_torch(o, BF16), BF16).astype(np.float64) for o in outs)
    assert orc.rel_l2(g1, orc.decode(ref_t, BF16)) <= 2e-3
    assert orc.rel_l2(g1, g3) <= 2e-3


# q/k RMSNorm on the C3 decode batch shape (bf16, 64 sequences, 32 / 8 heads, d 128, RoPE theta
# 500000): the normalised and rotated key rows in the pages are bit-exact, since the device and
# the oracle sum the squares in one fixed order (64 fma partials, then an XOR butterfly)
def test_qk_norm_c3_decode_batch():
    rng = np.random.default_rng(3)
    B, bs = 64, 16
    ctx = rng.integers(512, 2049, size=B)
    mb = int((ctx.max() + bs - 1) // bs)
    case = make_case(32, 8, 128, B * mb, bs, B, dtype=BF16, seed=3, new_lens=[1] * B,
                     past=ctx - 1, max_blocks=mb, do_rotary=1, theta=500000.0, qk_norm=True,
                     std=1.0)
    check(case)
