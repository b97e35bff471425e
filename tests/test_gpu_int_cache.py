"""Integer (int8 / int4) KV caches, packed QKV and head sizes off the matrix-core path, on the
GPU through the C ABI, against the oracle.

The integer cases mirror the reference's tests/ops/test_quantized_kv.py (paged: :344-556, GQA:
:81-195): its geometry (4 heads / 2 kv heads, 6 blocks of 4, new lengths [2, 0, 1] over pasts
[3, 1, 2]), its scales (per-tensor 0.125 / 0.25, per-channel cycles with a zero channel), live
scale changes between steps, tie / saturation / zero-scale values, values one float32 ulp
either side of rounding ties, norm before quantisation, and a page written before any read.

Bars: cache bytes bit-exact (integer codes and untouched bytes alike); outputs rel-L2 <= 2e-3
against the oracle rounded to T (<= 1e-5 for fp32).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, F32, I4, I8, PER_CHANNEL, PER_TENSOR
from pa_cases import (QUANT_NAMES, from_torch, int_scales, make_case, run_gpu_op, to_torch,
                      torch_dtype)

pytestmark = pytest.mark.gpu

MODES = [(PER_TENSOR, PER_TENSOR), (PER_CHANNEL, PER_CHANNEL), (PER_TENSOR, PER_CHANNEL)]
MODE_IDS = ["tensor", "channel", "mixed"]


def _rounded(ref, dtype):
    return orc.decode(orc.encode(ref.astype(np.float32), dtype), dtype).astype(np.float64)


def check_op(case, packed=False, tol=2e-3):
    print(f"int-cache case H={case['num_heads']} d={case['head_dim']} "
          f"cache={orc.NAMES[case['cache_dtype']]} packed={packed}", flush=True)
    ref, _, kc_ref, vc_ref = orc.paged_attention_op(case)
    out, kc, vc = run_gpu_op(case, packed=packed)
    np.testing.assert_array_equal(kc, kc_ref)
    np.testing.assert_array_equal(vc, vc_ref)
    got = orc.decode(out, case["dtype"]).astype(np.float64)
    want = ref if case["dtype"] == F32 else _rounded(ref, case["dtype"])
    err = orc.rel_l2(got, want)
    assert err <= (1e-5 if case["dtype"] == F32 else tol), err
    return out, kc, vc


def reference_case(bits, head=16, modes=(PER_CHANNEL, PER_CHANNEL), slots=True, dtype=F16,
                   **kw):
    """test_quantized_kv.py:344-392 geometry; slots = the reference's explicit slot mapping
    (token 0 and 1 of sequence 0 at their block-table slots, token 2 skipped)."""
    c = make_case(4, 2, head, 6, 4, 3, dtype=dtype, cache_dtype=I8 if bits == 8 else I4,
                  seed=818 + head + bits, new_lens=[2, 0, 1], past=[3, 1, 2], max_blocks=2,
                  int_modes=modes, **kw)
    if slots:
        bt = c["block_table"]
        c["slot_mapping"] = np.array([bt[0, 0] * 4 + 3, bt[0, 1] * 4, -1], np.int32)
    return c


# test_paged_integer_live_physical_cache (test_quantized_kv.py:448-466): two steps, the second
# with changed live scales and flipped resident bytes.
@pytest.mark.parametrize("bits,head", [(8, 16), (4, 16), (4, 7)], ids=["i8", "i4", "i4-odd"])
@pytest.mark.parametrize("packed", [False, True], ids=["sep", "packed"])
@pytest.mark.parametrize("modes", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("slots", [False, True], ids=["table", "slots"])
def test_paged_integer_live_physical_cache(bits, head, packed, modes, slots):
    c = reference_case(bits, head, modes, slots)
    for step in range(2):
        if step:
            c["k_scale"] = c["k_scale"] * np.float32(1.125)
            c["v_scale"] = c["v_scale"] * np.float32(1.25)
            c["key_cache"] = c["key_cache"] ^ np.array(3, c["key_cache"].dtype)
            c["value_cache"] = c["value_cache"] ^ np.array(7, c["value_cache"].dtype)
        check_op(c, packed=packed)


# test_paged_integer_rotary_sink_and_local (:469-475): rotary, head sink, softcap 0.7, masks
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("causal,window", [(1, -1), (1, 2), (0, -1), (0, 2)])
def test_paged_integer_rotary_sink_and_local(bits, causal, window):
    c = reference_case(bits, 16, causal=causal, window=window, softcap=0.7,
                       head_sink=np.linspace(-0.5, 0.5, 4))
    rng = np.random.default_rng(3)
    c["cos_cache"] = orc.encode(rng.uniform(0.5, 1.5, (16, 8)), F16)
    c["sin_cache"] = orc.encode(rng.uniform(-0.5, 0.5, (16, 8)), F16)
    check_op(c)


# test_paged_integer_ties_saturation_zero_scale (:478-491)
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("scale", [1.0, 0.0, 0.3])
def test_paged_integer_ties_saturation_zero_scale(bits, scale):
    c = reference_case(bits, 16, (PER_TENSOR, PER_TENSOR), slots=False)
    values = np.array([-1024, -128.5, -8.5, -7.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 6.5, 7.5,
                       126.5, 127.5, 1024, 0], np.float32)
    c["key"] = orc.encode(np.resize(values, c["key"].shape), F16)
    c["value"] = orc.encode(-np.resize(values, c["value"].shape), F16)
    c["k_scale"] = np.array([scale], np.float32)
    c["v_scale"] = np.array([scale], np.float32)
    check_op(c)


# test_integer_fp32_half_boundary_arithmetic (:322-341, paged=True): float32 values one ulp
# either side of exact rounding ties.  fp32 activations keep them exact, so the kernel's division
# must be the IEEE one; fp16 activations follow the reference test as written.
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("dtype", [F32, F16], ids=["fp32", "fp16"])
def test_paged_integer_half_boundary_arithmetic(bits, dtype):
    for scale in map(np.float32, [0.3, 0.7, 1.1, -0.3]):
        c = reference_case(bits, 16, (PER_TENSOR, PER_TENSOR), dtype=dtype)
        centers = np.array([-128.5, -127.5, -8.5, -7.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 6.5,
                            7.5, 126.5, 127.5], np.float32) * scale
        values = np.stack([np.nextafter(centers, -np.inf, dtype=np.float32), centers,
                           np.nextafter(centers, np.inf, dtype=np.float32)], -1).reshape(-1)
        c["query"] = orc.encode(np.zeros(c["query"].shape), dtype)
        c["key"] = orc.encode(np.resize(values, c["key"].shape), dtype)
        c["value"] = orc.encode(np.resize(values, c["value"].shape), dtype)
        c["k_scale"] = np.array([scale], np.float32)
        c["v_scale"] = np.array([scale], np.float32)
        check_op(c)


# test_paged_integer_qk_norm_before_quantization (:526-536)
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_integer_qk_norm_before_quantization(bits):
    c = reference_case(bits, 16, (PER_TENSOR, PER_TENSOR), qk_norm=True)
    c["query"] = orc.encode(np.resize(np.array([0.25, -0.5, 0.75, 1]), c["query"].shape), F16)
    c["key"] = orc.encode(np.resize(np.array([1, 0.5, -0.25, -0.75]), c["key"].shape), F16)
    c["q_norm"] = orc.encode(np.ones(16), F16)
    c["k_norm"] = orc.encode(np.ones(16), F16)
    check_op(c)


# test_paged_integer_shared_page_write_before_any_read (:539-556): known answer, row 0 == 1
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_integer_shared_page_write_before_any_read(bits):
    c = reference_case(bits, 16, (PER_TENSOR, PER_TENSOR))
    c["cum"] = np.array([0, 1, 1, 3], np.int32)
    c["past"] = np.zeros(3, np.int32)
    c["block_table"] = np.zeros((3, 2), np.int32)
    c["slot_mapping"] = np.array([-1, 0, -1], np.int32)
    for name in ("key_cache", "value_cache"):
        c[name] = np.full_like(c[name], 0 if bits == 8 else 0x88)
    c["query"] = orc.encode(np.zeros(c["query"].shape), F16)
    c["key"] = orc.encode(np.zeros(c["key"].shape), F16)
    c["value"] = orc.encode(np.ones(c["value"].shape), F16)
    c["k_scale"] = np.array([1.0], np.float32)
    c["v_scale"] = np.array([1.0], np.float32)
    out, _, _ = check_op(c)
    assert np.all(orc.decode(out[0], F16) == 1.0)


# test_integer_cache_bfloat16_preserves_fp32_scales (:558-596): bf16 activations
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_integer_bfloat16(bits):
    check_op(reference_case(bits, 16, dtype=BF16))


# a decode batch at the Llama-3-8B head geometry on integer pages (streaming matrix-core decode)
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_integer_decode_batch(bits):
    rng = np.random.default_rng(bits)
    B, bs = 6, 16
    past = rng.integers(200, 1500, B)
    c = make_case(32, 8, 128, 6 * 96, bs, B, dtype=BF16, cache_dtype=I8 if bits == 8 else I4,
                  seed=bits, new_lens=[1] * B, past=past, max_blocks=96,
                  int_modes=(PER_CHANNEL, PER_TENSOR), std=1.0)
    check_op(c)


# pa_reshape_and_cache with integer pages, duplicate slots (last writer wins)
@pytest.mark.parametrize("bits", [8, 4])
def test_reshape_and_cache_integer_duplicate_slots(bits):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    c = reference_case(bits, 16, (PER_CHANNEL, PER_TENSOR))
    bt = c["block_table"]
    slots = np.array([bt[1, 0] * 4 + 1, bt[1, 0] * 4 + 1, bt[2, 1] * 4 + 2], np.int32)
    kc_ref, vc_ref = orc.reshape_and_cache(c["key"], c["value"], F16, c["key_cache"],
                                           c["value_cache"], c["cache_dtype"], c["cum"],
                                           c["past"], bt, slot_mapping=slots,
                                           k_scale=c["k_scale"], v_scale=c["v_scale"],
                                           k_mode=PER_CHANNEL, v_mode=PER_TENSOR, head_dim=16)
    cd = c["cache_dtype"]
    kc, vc = to_torch(c["key_cache"], cd), to_torch(c["value_cache"], cd)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()
    ep.reshape_and_cache(to_torch(c["key"], F16), to_torch(c["value"], F16), kc, vc,
                         i32(c["cum"]), i32(c["past"]), i32(bt), i32(slots),
                         torch.from_numpy(c["k_scale"]).cuda(),
                         torch.from_numpy(c["v_scale"]).cuda(),
                         k_quant_type="PER_CHANNEL", v_quant_type="PER_TENSOR")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_torch(kc, cd), kc_ref)
    np.testing.assert_array_equal(from_torch(vc, cd), vc_ref)


def test_integer_cache_requires_scales_and_modes():
    import torch
    import onnxruntime_ep_mlx_amd as ep
    c = reference_case(8, 16, (PER_TENSOR, PER_TENSOR))
    c.pop("v_scale")
    with pytest.raises(ep.PagedAttentionError, match="quantized v cache requires a scale"):
        run_gpu_op(c)
    c = reference_case(8, 16, (PER_TENSOR, PER_TENSOR))
    c["k_quant"] = 0
    with pytest.raises(ep.PagedAttentionError, match="PER_TENSOR or PER_CHANNEL"):
        run_gpu_op(c)
    torch.cuda.synchronize()


# ------------------------------------------------------------------------- GroupQueryAttention
def gqa_int_case(bits, dtype, modes, seed, B=2, S=2, H=4, KV=2, d=32, cap=6, seqlens=(3, 5)):
    """test_quantized_kv.py:81-195 (_gqa): batch 2, 2 new rows, capacity 6, per-channel scales
    of 2 kv heads x 32 channels, resident rows holding codes."""
    rng = np.random.default_rng(seed)
    enc = lambda shape: orc.encode(rng.standard_normal(shape) * 0.7, dtype)
    width = d if bits == 8 else d // 2
    c = dict(q=enc((B, S, H * d)), k=enc((B, S, KV * d)), v=enc((B, S, KV * d)),
             seqlens=np.asarray(seqlens, np.int32), bits=bits, d=d, H=H, KV=KV,
             k_scale=int_scales(KV, d, modes[0], 0), v_scale=int_scales(KV, d, modes[1], 1),
             modes=modes)
    if bits == 8:
        c["pk"] = rng.integers(-128, 128, (B, KV, cap, width), dtype=np.int8)
        c["pv"] = rng.integers(-128, 128, (B, KV, cap, width), dtype=np.int8)
    else:
        c["pk"] = rng.integers(0, 256, (B, KV, cap, width), dtype=np.uint8)
        c["pv"] = rng.integers(0, 256, (B, KV, cap, width), dtype=np.uint8)
    return c


def run_gqa_int(c, dtype, packed=False, **kw):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    cd = I8 if c["bits"] == 8 else I4
    q, k, v = (to_torch(c[n], dtype) for n in ("q", "k", "v"))
    if packed:
        q, k, v = torch.cat([q, k, v], dim=2).contiguous(), None, None
    pk, pv = to_torch(c["pk"], cd), to_torch(c["pv"], cd)
    out, pk, pv = ep.group_query_attention(
        q, k, v, pk, pv, torch.from_numpy(c["seqlens"]).cuda(), int(c["seqlens"].max()) + 1,
        num_heads=c["H"], kv_num_heads=c["KV"], scale=float(1 / np.sqrt(c["d"])),
        k_scale=torch.from_numpy(c["k_scale"]).cuda(),
        v_scale=torch.from_numpy(c["v_scale"]).cuda(),
        k_quant_type=QUANT_NAMES[c["modes"][0]], v_quant_type=QUANT_NAMES[c["modes"][1]],
        present=kw.pop("present", "shared"), **kw)
    torch.cuda.synchronize()
    return from_torch(out, dtype), from_torch(pk, cd), from_torch(pv, cd)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("dtype", [F32, F16], ids=["fp32", "fp16"])
@pytest.mark.parametrize("packed", [False, True], ids=["sep", "packed"])
@pytest.mark.parametrize("modes", MODES, ids=MODE_IDS)
def test_gqa_integer_live_cache_scales(bits, dtype, packed, modes):
    c = gqa_int_case(bits, dtype, modes, seed=bits + 10 * int(packed))
    print(f"gqa int{bits} {orc.NAMES[dtype]} packed={packed} modes={modes}", flush=True)
    ref, rpk, rpv = orc.gqa_contiguous(dtype, c["q"], c["k"], c["v"], c["pk"], c["pv"],
                                       c["seqlens"], c["H"], c["KV"], c["d"],
                                       float(np.float32(1 / np.sqrt(c["d"]))),
                                       cache_dtype=I8 if bits == 8 else I4,
                                       k_scale=c["k_scale"], v_scale=c["v_scale"],
                                       k_mode=modes[0], v_mode=modes[1])
    out, pk, pv = run_gqa_int(c, dtype, packed=packed)
    np.testing.assert_array_equal(pk, rpk)
    np.testing.assert_array_equal(pv, rpv)
    got = orc.decode(out, dtype).astype(np.float64)
    want = ref if dtype == F32 else _rounded(ref, dtype)
    assert orc.rel_l2(got, want) <= (1e-5 if dtype == F32 else 2e-3)


def test_gqa_int4_odd_head_is_refused():
    import onnxruntime_ep_mlx_amd as ep
    c = gqa_int_case(4, F32, (PER_TENSOR, PER_TENSOR), seed=3, d=31)
    c["pk"] = np.zeros((2, 2, 6, 16), np.uint8)
    c["pv"] = np.zeros((2, 2, 6, 16), np.uint8)
    with pytest.raises(ep.PagedAttentionError, match="even logical head size"):
        run_gqa_int(c, F32)


# ------------------------------------------------------------------ packed QKV, any head size
@pytest.mark.parametrize("dtype,d,H,KV,rotary", [
    (BF16, 128, 32, 8, 1),   # decode on the balanced MFMA kernel, rotated q/k from the copy
    (F16, 64, 8, 2, 0),      # no rotary: the append copies the packed rows out
    (F16, 128, 28, 4, 1),    # multi-token (chunked MFMA kernel)
])
def test_paged_packed_qkv_float_cache(dtype, d, H, KV, rotary):
    new_lens = [1, 1, 1, 1] if H == 32 else [3, 1, 4, 2]
    c = make_case(H, KV, d, 256, 16, 4, dtype=dtype, seed=d + H, new_lens=new_lens,
                  do_rotary=rotary, theta=500000.0)
    check_op(c, packed=True)


@pytest.mark.parametrize("d", [7, 20, 40, 96, 200])
def test_paged_head_sizes_off_the_matrix_core_path(d):
    c = make_case(8, 2, d, 64, 16, 3, dtype=F16, seed=d, do_rotary=int(d % 4 == 0),
                  rot_dim=d // 2 if d % 4 == 0 else None)
    check_op(c)


def test_gqa_packed_qkv_float_cache():
    import torch
    import onnxruntime_ep_mlx_amd as ep
    rng = np.random.default_rng(11)
    B, S, H, KV, d, cap = 3, 1, 32, 8, 128, 700
    enc = lambda shape: orc.encode(rng.standard_normal(shape), BF16)
    q, k, v = enc((B, S, H * d)), enc((B, S, KV * d)), enc((B, S, KV * d))
    pk, pv = enc((B, KV, cap, d)), enc((B, KV, cap, d))
    seqlens = np.array([650, 12, 699], np.int32)
    ref, rpk, rpv = orc.gqa_contiguous(BF16, q, k, v, pk, pv, seqlens, H, KV, d,
                                       float(np.float32(1 / np.sqrt(d))))
    qkv = torch.cat([to_torch(q, BF16), to_torch(k, BF16), to_torch(v, BF16)], 2).contiguous()
    out, tpk, tpv = ep.group_query_attention(
        qkv, None, None, to_torch(pk, BF16), to_torch(pv, BF16),
        torch.from_numpy(seqlens).cuda(), int(seqlens.max()) + 1, num_heads=H, kv_num_heads=KV)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(tpk, BF16), rpk)
    assert np.array_equal(from_torch(tpv, BF16), rpv)
    got = orc.decode(from_torch(out, BF16), BF16).astype(np.float64)
    assert orc.rel_l2(got, _rounded(ref, BF16)) <= 2e-3
