"""GroupQueryAttention sliding_window_cache rings and output_qk diagnostics on the GPU
(pa_group_query_attention through the C ABI) against the oracle (orc_gqa_batched with sliding /
qk_mode, pinned in test_oracle_sliding.py).

Rings (attention.rs:1139-1368): calls are chained -- each call's present is the next call's
past, on the device and in the oracle independently -- across several wrap points, with decode
calls on the streaming matrix-core decode (bf16/fp16, heads 64/128), multi-token calls on the
prefill kernels (including calls whose window needs rows the ring drops in the same call),
int8 / int4 rings, a bias (absolute columns) with fp32 rotary, sink and softcap on the VALU
kernel, presents of their own and bound onto the past, and device-only metadata.

output_qk (attention.rs:771-785): modes 1 and 2 over first prompts, later calls with bias, sink
and softcap, windows, bidirectional rows, integer presents and decode batches.

Bars: presents bit-exact; outputs rel-L2 <= 2e-3 against the T-rounded oracle for fp16/bf16
(<= 4e-3 against its fp64 output), <= 1e-5 for fp32; diagnostics rel-L2 per sequence and head
<= 2e-3 against the T-rounded oracle (fp32: 1e-5), exact zeros where the oracle has them.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from _oracle import BF16, F16, F32, I4, I8, PER_CHANNEL, PER_TENSOR
from gqa_cases import gqa_case, run_oracle
from pa_cases import from_torch, to_torch

pytestmark = pytest.mark.gpu

MODES = {0: "NONE", 1: "PER_TENSOR", 2: "PER_CHANNEL"}


def run_device(c, pk_dev, pv_dev, present="new", validate=True, qk=0):
    """One call on the device; pk_dev / pv_dev: the past rings (torch).  Returns the output (raw
    numpy), the present rings (torch) and the diagnostics (raw numpy) when qk is set."""
    import torch
    import onnxruntime_ep_mlx_amd as ep
    dt = c["dtype"]
    cdt = c["cache_dtype"] or dt
    T = lambda x, code=dt: None if x is None else to_torch(x, code)
    F = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()
    print(f"gqa sliding={c.get('sliding', 0)} qk={qk} B={c['B']} S={c['S']} H={c['H']} "
          f"KV={c['KV']} d={c['d']} {orc.NAMES[dt]} cache={orc.NAMES[cdt]} window={c['window']} "
          f"present={present} validate={validate}", flush=True)
    res = ep.group_query_attention(
        T(c["q"]), T(c["k"]), T(c["v"]), pk_dev, pv_dev, F(c["seqlens"]), c["total"],
        cos_cache=T(c.get("cos")), sin_cache=T(c.get("sin")), position_ids=F(c.get("pid")),
        attention_bias=T(c.get("bias")), head_sink=T(c.get("sink")),
        k_scale=F(c.get("k_scale")), v_scale=F(c.get("v_scale")),
        q_norm_weight=T(c.get("q_norm")), k_norm_weight=T(c.get("k_norm")),
        num_heads=c["H"], kv_num_heads=c["KV"], scale=c["scale"], softcap=c["softcap"],
        local_window_size=c["window"], do_rotary=int(c.get("cos") is not None),
        is_causal=c["causal"], smooth_softmax=c["smooth"],
        k_quant_type=MODES[c.get("k_mode", 0)], v_quant_type=MODES[c.get("v_mode", 0)],
        present=present, validate=validate, sliding_window_cache=c.get("sliding", 0),
        qk_output=qk)
    torch.cuda.synchronize()
    out = from_torch(res[0], dt)
    return (out, res[1], res[2]) + ((from_torch(res[3], dt),) if qk else ())


def check_out(got_raw, ref, dt, what=""):
    got = orc.decode(got_raw, dt).astype(np.float64)
    if dt == F32:
        assert orc.rel_l2(got, ref) <= 1e-5, what
    else:
        assert orc.rel_l2(got, orc.decode(orc.encode(ref.astype(np.float32), dt), dt)) <= 2e-3, what
        assert orc.rel_l2(got, ref) <= 4e-3, what


def chain(steps, *, dtype=BF16, B=3, H=8, KV=2, d=128, cap=64, W=40, start=None, cache_dtype=0,
          modes=(PER_CHANNEL, PER_TENSOR), present="new", validate=True, seed=0, **kw):
    """Calls of steps[i] new rows each, every present fed back as the next past; lengths start
    at `start` (per sequence) so the first calls already run on full rings."""
    import torch
    rng = np.random.default_rng(seed)
    start = np.asarray(start if start is not None else rng.integers(0, 3 * cap, size=B), np.int64)
    c0 = gqa_case(dtype, B, steps[0], H, KV, d, start + steps[0] - 1, cap=cap, window=W,
                  cache_dtype=cache_dtype, modes=modes, seed=seed, **kw)
    c0["sliding"] = 1
    # the first past rings: each sequence's ring_end(start) rows of random content, zero codes after
    gap = cap - W + 1
    zero = 0x88 if cache_dtype == I4 else 0
    pk, pv = c0["pk"].copy(), c0["pv"].copy()
    for b in range(B):
        n = int(start[b]) if start[b] <= cap else int(start[b] - gap * ((start[b] - cap + gap - 1) // gap))
        pk.view(np.uint8)[b, :, n:] = zero
        pv.view(np.uint8)[b, :, n:] = zero
    cdt = cache_dtype or dtype
    dev_k, dev_v = to_torch(pk, cdt), to_torch(pv, cdt)
    lengths = start.copy()
    for call, S in enumerate(steps):
        lengths = lengths + S
        c = gqa_case(dtype, B, S, H, KV, d, lengths - 1, cap=cap, window=W,
                     cache_dtype=cache_dtype, modes=modes, seed=seed + 100 * (call + 1), **kw)
        c["sliding"] = 1
        c["pk"], c["pv"] = pk, pv
        ref, pk, pv = run_oracle(c)
        out, dk, dv = run_device(c, dev_k, dev_v, present=present, validate=validate)
        assert np.array_equal(from_torch(dk, cdt).view(np.uint8), pk.view(np.uint8)), call
        assert np.array_equal(from_torch(dv, cdt).view(np.uint8), pv.view(np.uint8)), call
        check_out(out, ref, dtype, f"call {call}")
        if present == "new":
            dev_k, dev_v = dk, dv  # a fresh buffer each call
        else:
            assert dk.data_ptr() == dev_k.data_ptr()


@pytest.mark.parametrize("dtype,d,H,KV", [(BF16, 128, 32, 8), (F16, 64, 16, 2)],
                         ids=["bf16_d128", "fp16_d64"])
@pytest.mark.parametrize("present", ["new", "shared"])
def test_sliding_decode_chain(dtype, d, H, KV, present):
    chain([1] * 30, dtype=dtype, d=d, H=H, KV=KV, B=4, cap=64, W=40, present=present,
          start=[0, 23, 64, 150], seed=d)


@pytest.mark.parametrize("present", ["new", "shared"])
def test_sliding_multi_token_chain(present):
    # 17-row calls on a ring of 48 with window 24 (gap 25): windows need rows the call drops
    chain([17, 5, 17, 1, 17, 9, 17], B=3, H=16, KV=4, cap=48, W=24, start=[0, 40, 95],
          present=present, seed=1)


@pytest.mark.parametrize("cache_dtype,modes", [(I8, (PER_CHANNEL, PER_TENSOR)),
                                               (I4, (PER_TENSOR, PER_CHANNEL))],
                         ids=["int8", "int4"])
def test_sliding_integer_rings(cache_dtype, modes):
    chain([1] * 6 + [9, 1, 9], dtype=BF16, B=3, H=8, KV=2, d=128, cap=40, W=16,
          start=[3, 39, 120], cache_dtype=cache_dtype, modes=modes, seed=2)


def test_sliding_bias_rotary_sink_softcap():
    """A bias (absolute columns), which also switches the rotary to fp32; sink and softcap."""
    B, S = 2, 3
    for call, start in enumerate(([10, 70], [70, 131])):
        start = np.asarray(start)
        total = int((start + S).max())
        c = gqa_case(F16, B, S, 8, 2, 64, start + S - 1, cap=32, window=12, rotary=True,
                     bias_shape=(B, 1, S, total), sink=True, softcap=4.0, seed=3 + call)
        c["sliding"] = 1
        ref, pk, pv = run_oracle(c)
        out, dk, dv = run_device(c, to_torch(c["pk"], F16), to_torch(c["pv"], F16))
        assert np.array_equal(from_torch(dk, F16), pk) and np.array_equal(from_torch(dv, F16), pv)
        check_out(out, ref, F16)


def test_sliding_fp32_and_device_only_metadata():
    chain([1, 1, 4, 1], dtype=F32, B=2, H=4, KV=2, d=64, cap=20, W=8, start=[5, 44],
          validate=False, seed=4)


def test_sliding_rejections():
    import torch
    import onnxruntime_ep_mlx_amd as ep
    c = gqa_case(BF16, 1, 1, 4, 1, 64, [9], cap=8, window=4, seed=5)
    T = lambda x: to_torch(x, BF16)
    lens = torch.tensor([9], dtype=torch.int32, device="cuda")
    common = dict(num_heads=4, kv_num_heads=1, sliding_window_cache=1)
    with pytest.raises(RuntimeError, match="sliding cache requires 0 < local_window_size <= capacity"):
        ep.group_query_attention(T(c["q"]), T(c["k"]), T(c["v"]), T(c["pk"]), T(c["pv"]), lens,
                                 10, local_window_size=9, **common)
    empty = torch.empty((1, 0, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="non-sliding past"):
        ep.group_query_attention(T(c["q"]), empty, empty, T(c["pk"]), T(c["pv"]), lens, 10,
                                 local_window_size=4, **common)
    bad = torch.tensor([0], dtype=torch.int32, device="cuda")  # length 1 < rows 2
    q2 = T(np.concatenate([c["q"], c["q"]], axis=1))
    k2 = T(np.concatenate([c["k"], c["k"]], axis=1))
    with pytest.raises(RuntimeError, match="invalid sliding sequence lengths"):
        ep.group_query_attention(q2, k2, k2, T(c["pk"]), T(c["pv"]), bad, 1,
                                 local_window_size=4, **common)


# ------------------------------------------------------------------------------ output_qk
QK_CASES = {
    "first_prompt_ragged_smooth": dict(dtype=BF16, B=3, S=24, H=8, KV=2, d=64,
                                       seqlens=[23, 9, 15], smooth=1),
    "later_bias_sink_softcap": dict(dtype=F16, B=2, S=3, H=8, KV=4, d=64, seqlens=[40, 77],
                                    cap=80, bias_shape=(2, 8, 3, 78), sink=True, softcap=5.0),
    "window_growing_rotary": dict(dtype=BF16, B=2, S=5, H=4, KV=1, d=128, seqlens=[60, 33],
                                  cap=56, window=20, rotary=True),
    "non_causal_fp32": dict(dtype=F32, B=2, S=4, H=4, KV=2, d=32, seqlens=[20, 13], cap=24,
                            causal=0),
    "int8_present": dict(dtype=BF16, B=2, S=2, H=8, KV=2, d=64, seqlens=[30, 17], cap=32,
                         cache_dtype=I8, modes=(PER_CHANNEL, PER_TENSOR)),
    "decode_d128": dict(dtype=BF16, B=4, S=1, H=32, KV=8, d=128, seqlens=[700, 12, 300, 1023],
                        cap=1024, rotary=True, theta=500000.0),
}


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name", sorted(QK_CASES))
def test_output_qk(name, mode):
    kw = dict(QK_CASES[name])
    c = gqa_case(kw.pop("dtype"), kw.pop("B"), kw.pop("S"), kw.pop("H"), kw.pop("KV"),
                 kw.pop("d"), kw.pop("seqlens"), seed=7 + mode, **kw)
    c["qk_mode"] = mode
    ref, pk, pv, qk_ref = run_oracle(c)
    dt, cdt = c["dtype"], c["cache_dtype"] or c["dtype"]
    T = lambda x: None if x is None else to_torch(x, cdt)
    out, dk, dv, qk = run_device(c, T(c["pk"]), T(c["pv"]), qk=mode)
    assert np.array_equal(from_torch(dk, cdt).view(np.uint8), pk.view(np.uint8))
    assert np.array_equal(from_torch(dv, cdt).view(np.uint8), pv.view(np.uint8))
    check_out(out, ref, dt)
    got = orc.decode(qk, dt).astype(np.float64)
    want = orc.decode(orc.encode(qk_ref.astype(np.float32), dt), dt).astype(np.float64)
    assert not got[qk_ref == 0].any(), "masked keys and columns past the length must be 0"
    bar = 1e-5 if dt == F32 else 2e-3
    for b in range(c["B"]):
        for h in range(c["H"]):
            assert orc.rel_l2(got[b, h], want[b, h]) <= bar, (b, h)
