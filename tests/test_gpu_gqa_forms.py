"""GroupQueryAttention forms on the GPU (pa_group_query_attention through the C ABI) against
the oracle's full restatement orc_gqa_batched (gqa_batched, attention.rs:586-848): first
prompts without a past (ragged, right-padded rows), growing present caches, no new key/value
rows, position ids (offset and flattened forms, fp32 rotation), additive attention bias,
smooth_softmax and head sinks, q/k RMSNorm, integer caches with zero-code tails, packed QKV,
present outputs new / bound onto the past / omitted, and device-only metadata.

Bars: present caches bit-exact; outputs rel-L2 <= 2e-3 against the T-rounded oracle output for
fp16/bf16 (and <= 4e-3 against its fp64 output), <= 1e-5 for fp32.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, F32
from gqa_cases import FORMS, form_case, gqa_case, run_oracle
from pa_cases import from_torch, to_torch, torch_dtype

pytestmark = pytest.mark.gpu


def run_device(c, present="new", packed=False, validate=True):
    import torch
    import onnxruntime_ep_mlx_amd as ep
    dt = c["dtype"]
    cdt = c["cache_dtype"] or dt
    T = lambda x, code=dt: None if x is None else to_torch(x, code)
    F = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()
    B, S, H, KV, d = c["B"], c["S"], c["H"], c["KV"], c["d"]
    if c["k"] is None:  # no new rows: empty key/value [B, 0, KV * d]
        k = torch.empty((B, 0, KV * d), dtype=torch_dtype(dt), device="cuda")
        v = torch.empty_like(k)
    else:
        k, v = T(c["k"]), T(c["v"])
    q = T(c["q"])
    if packed:
        q, k, v = torch.cat([q, k, v], 2).contiguous(), None, None
    modes = {0: "NONE", 1: "PER_TENSOR", 2: "PER_CHANNEL"}
    print(f"gqa B={B} S={S} H={H} KV={KV} d={d} {orc.NAMES[dt]} present={present} "
          f"packed={packed} validate={validate}", flush=True)
    out, pk, pv = ep.group_query_attention(
        q, k, v, T(c["pk"], cdt), T(c["pv"], cdt), F(c["seqlens"]), c["total"],
        cos_cache=T(c.get("cos")), sin_cache=T(c.get("sin")), position_ids=F(c.get("pid")),
        attention_bias=T(c.get("bias")), head_sink=T(c.get("sink")),
        k_scale=F(c.get("k_scale")), v_scale=F(c.get("v_scale")),
        q_norm_weight=T(c.get("q_norm")), k_norm_weight=T(c.get("k_norm")),
        num_heads=H, kv_num_heads=KV, scale=c["scale"], softcap=c["softcap"],
        local_window_size=c["window"], do_rotary=int(c.get("cos") is not None),
        is_causal=c["causal"], smooth_softmax=c["smooth"],
        k_quant_type=modes[c.get("k_mode", 0)], v_quant_type=modes[c.get("v_mode", 0)],
        present=present, validate=validate)
    torch.cuda.synchronize()
    return (from_torch(out, dt), None if pk is None else from_torch(pk, cdt),
            None if pv is None else from_torch(pv, cdt))


def check(c, present="new", packed=False, validate=True):
    cap = 0 if c["pk"] is None else c["pk"].shape[2]
    ref, rpk, rpv = run_oracle(c, present_cap=cap if present == "shared" else None)
    out, pk, pv = run_device(c, present=present, packed=packed, validate=validate)
    if present != "omitted":
        assert pk.shape == rpk.shape, (pk.shape, rpk.shape)
        assert np.array_equal(pk.view(np.uint8), rpk.view(np.uint8)), "present_key differs"
        assert np.array_equal(pv.view(np.uint8), rpv.view(np.uint8)), "present_value differs"
    else:
        assert pk is None and pv is None
    dt = c["dtype"]
    got = orc.decode(out, dt).astype(np.float64)
    if dt == F32:
        err = orc.rel_l2(got, ref)
        assert err <= 1e-5, err
    else:
        err = orc.rel_l2(got, orc.decode(orc.encode(ref.astype(np.float32), dt), dt))
        assert err <= 2e-3, err
        assert orc.rel_l2(got, ref) <= 4e-3


@pytest.mark.parametrize("form", list(FORMS))
def test_forms_new_present(form):
    check(form_case(form))


# outputs bound onto the past buffers (capacity stays) and outputs omitted
@pytest.mark.parametrize("form", ["no_new_rows", "bias_smooth", "bias_heads_sink_softcap",
                                  "position_ids_flat", "qk_norm", "non_causal"])
@pytest.mark.parametrize("present", ["shared", "omitted"])
def test_forms_shared_and_omitted_present(form, present):
    check(form_case(form), present=present)


# the same forms from device-only metadata (no host copies of seqlens_k / position_ids)
@pytest.mark.parametrize("form", ["ragged_first_prompt", "growing_window", "no_new_rows",
                                  "position_ids_flat", "int4_growing"])
def test_forms_device_only_metadata(form):
    check(form_case(form), validate=False)


# decode batches on the streaming matrix-core kernel (head 128 / 64, g <= 16): smooth_softmax,
# head sink, no new rows, position ids and q/k norm
@pytest.mark.parametrize("variant", ["smooth", "sink", "no_new_rows", "position_ids", "qk_norm"])
@pytest.mark.parametrize("dtype,d,H,KV", [(BF16, 128, 32, 8), (F16, 64, 16, 2)],
                         ids=["bf16_d128", "fp16_d64"])
def test_decode_forms_on_matrix_cores(variant, dtype, d, H, KV):
    rng = np.random.default_rng(d + len(variant))
    B, cap = 6, 1024
    seqlens = rng.integers(8, cap - 1, size=B)
    kw = dict(cap=cap, rotary=True, theta=500000.0)
    if variant == "smooth":
        kw["smooth"] = 1
    elif variant == "sink":
        kw["sink"] = True
    elif variant == "no_new_rows":
        kw["kv_seq"] = 0
    elif variant == "position_ids":
        kw["pid"] = rng.integers(0, cap, size=(B, 3))
    elif variant == "qk_norm":
        kw["qk_norm"] = True
    c = gqa_case(dtype, B, 1, H, KV, d, seqlens, seed=d + len(variant), **kw)
    check(c, present="shared")


# multi-token queries over a long past and a first prompt (bf16, head 128)
@pytest.mark.parametrize("first", [False, True], ids=["chunk", "first_prompt"])
def test_multi_token_head128(first):
    if first:
        c = gqa_case(BF16, 3, 96, 16, 4, 128, [95, 40, 70], seed=5, rotary=True,
                     theta=500000.0, pid=np.zeros((3, 96), np.int64))
    else:
        c = gqa_case(BF16, 2, 64, 16, 4, 128, [600, 350], cap=640, seed=6, rotary=True,
                     theta=500000.0)
    check(c)


def test_packed_qkv_with_position_ids_and_qk_norm():
    rng = np.random.default_rng(12)
    c = gqa_case(BF16, 2, 3, 16, 4, 128, [200, 90], cap=256, seed=12, rotary=True,
                 pid=rng.integers(0, 256, size=(2, 3)), qk_norm=True)
    check(c, packed=True)


def test_attention_bias_on_a_decode_batch():
    # a bias routes the call to the VALU kernel even for decode-shaped batches
    c = gqa_case(F16, 4, 1, 16, 4, 128, [300, 17, 511, 64], cap=512, seed=13,
                 bias_shape=(4, 16, 1, 512))
    check(c, present="shared")


# Multi-token GroupQueryAttention on the LDS-shared prefill kernels in contiguous-cache addressing
# (head 128: prefill_mx_kernel, other heads: prefill_kernel): chunks over a past, growing and
# shared presents, a window, a sink, capacities that are not multiples of the key step (the
# last steps read row by row), and a first prompt with every sequence full length.
@pytest.mark.parametrize("d", [64, 96, 128, 256])
@pytest.mark.parametrize("variant", ["chunk_new", "chunk_shared", "window_sink", "first_full"])
def test_multi_token_prefill_kernels(d, variant):
    rng = np.random.default_rng(d + len(variant))
    B, S, H, KV = 3, 48, 16, 4
    if variant == "first_full":
        c = gqa_case(BF16, B, S, H, KV, d, [S - 1] * B, seed=d, rotary=True, theta=500000.0)
        check(c)
        return
    seqlens = rng.integers(S, 500, size=B)
    kw = dict(cap=517, rotary=True, theta=500000.0)
    if variant == "window_sink":
        kw.update(window=77, sink=True)
    c = gqa_case(F16 if variant == "window_sink" else BF16, B, S, H, KV, d, seqlens,
                 seed=d + 1, **kw)
    check(c, present="shared" if variant == "chunk_shared" else "new")


# enough (sequence, kv-head, 128-row block) items for the planned launch (split halves merged)
def test_multi_token_prefill_planned_launch():
    rng = np.random.default_rng(77)
    B, S, H, KV, d = 16, 128, 32, 8, 128
    seqlens = rng.integers(S, 400, size=B)
    seqlens[3] = 2999  # one long item that splits
    c = gqa_case(BF16, B, S, H, KV, d, seqlens, cap=3000, seed=77, rotary=True, theta=500000.0)
    check(c, present="shared")
