"""GroupQueryAttention problems shared by the oracle pins and the GPU parity tests: raw inputs
(numpy storage arrays as in _oracle), attributes, and the oracle call (orc_gqa_batched)."""
from __future__ import annotations

import numpy as np

import _oracle as orc
from _oracle import BF16, F16, F32, I4, I8, PER_CHANNEL, PER_TENSOR
from pa_cases import int_scales, rotary_cache


def gqa_case(dtype, B, S, H, KV, d, seqlens, *, cap=None, kv_seq=None, total=None, seed=0,
             rotary=False, theta=10000.0, pid=None, bias_shape=None, sink=False, smooth=0,
             qk_norm=False, window=-1, softcap=0.0, causal=1, cache_dtype=0,
             modes=(PER_TENSOR, PER_TENSOR), std=1.0):
    """One GroupQueryAttention problem: raw inputs, attributes and the oracle call's kwargs."""
    rng = np.random.default_rng(seed)
    seqlens = np.asarray(seqlens, np.int32)
    total = int(seqlens.max()) + 1 if total is None else total
    kv_seq = S if kv_seq is None else kv_seq
    enc = lambda shape, s=std: orc.encode(rng.standard_normal(shape) * s, dtype)
    c = dict(dtype=dtype, B=B, S=S, H=H, KV=KV, d=d, seqlens=seqlens, total=total,
             scale=float(np.float32(1 / np.sqrt(d))), window=window, softcap=softcap,
             causal=causal, smooth=smooth, cache_dtype=cache_dtype)
    c["q"] = enc((B, S, H * d))
    c["k"] = enc((B, kv_seq, KV * d)) if kv_seq else None
    c["v"] = enc((B, kv_seq, KV * d)) if kv_seq else None
    if cap:
        if cache_dtype == I8:
            c["pk"] = rng.integers(-128, 128, (B, KV, cap, d), dtype=np.int8)
            c["pv"] = rng.integers(-128, 128, (B, KV, cap, d), dtype=np.int8)
        elif cache_dtype == I4:
            c["pk"] = rng.integers(0, 256, (B, KV, cap, (d + 1) // 2), dtype=np.uint8)
            c["pv"] = rng.integers(0, 256, (B, KV, cap, (d + 1) // 2), dtype=np.uint8)
        else:
            c["pk"], c["pv"] = enc((B, KV, cap, d)), enc((B, KV, cap, d))
    else:
        c["pk"] = c["pv"] = None
    if cache_dtype:
        c["k_scale"] = int_scales(KV, d, modes[0], 0)
        c["v_scale"] = int_scales(KV, d, modes[1], 1)
        c["k_mode"], c["v_mode"] = modes
    if rotary:
        c["cos"], c["sin"] = rotary_cache(max(total, cap or 0) + 16, d, theta, dtype)
    c["pid"] = None if pid is None else np.ascontiguousarray(pid, np.int64)
    c["bias"] = None if bias_shape is None else enc(bias_shape, 2.0)
    c["sink"] = enc((H,), 1.0) if sink else None
    if qk_norm:
        c["q_norm"] = orc.encode(np.linspace(0.75, 1.25, d), dtype)
        c["k_norm"] = orc.encode(np.linspace(1.25, 0.75, d), dtype)
    return c


def run_oracle(c, present_cap=None):
    """The oracle on a case: (out, present_k, present_v) (+ the diagnostics with qk_mode)."""
    return orc.gqa_batched(
        c["dtype"], c["q"], c["k"], c["v"], c["pk"], c["pv"], c["seqlens"], c["total"], c["H"],
        c["KV"], c["d"], scale=c["scale"], present_cap=present_cap, softcap=c["softcap"],
        window=c["window"], causal=c["causal"], cos=c.get("cos"), sin=c.get("sin"),
        position_ids=c.get("pid"), bias=c.get("bias"), head_sink=c.get("sink"),
        smooth=c["smooth"], q_norm=c.get("q_norm"), k_norm=c.get("k_norm"),
        cache_dtype=c["cache_dtype"], k_scale=c.get("k_scale"), v_scale=c.get("v_scale"),
        k_mode=c.get("k_mode", 0), v_mode=c.get("v_mode", 0), sliding=c.get("sliding", 0),
        qk_mode=c.get("qk_mode", 0))


FORMS = {
    # first prompt, no past, ragged lengths (right-padded rows), position ids offset form
    "ragged_first_prompt": dict(dtype=BF16, B=3, S=12, H=4, KV=2, d=32, seqlens=[11, 4, 8],
                                rotary=True, pid=np.array([[3] * 12, [0] * 12, [0] * 12])),
    # growing cache: capacity 20 < total 24 (query_past 20 fits the capacity), window 6
    "growing_window": dict(dtype=F16, B=2, S=4, H=4, KV=1, d=16, seqlens=[23, 19], cap=20,
                           window=6),
    # no new key/value rows (kv_seq 0): the past alone, fp32 rope of the queries
    "no_new_rows": dict(dtype=BF16, B=2, S=3, H=4, KV=2, d=32, seqlens=[9, 14], cap=16,
                        kv_seq=0, rotary=True),
    # additive bias [B, 1, S, total] and smooth_softmax
    "bias_smooth": dict(dtype=F16, B=2, S=3, H=4, KV=2, d=16, seqlens=[10, 6], cap=12,
                        bias_shape=(2, 1, 3, 11), smooth=1),
    # bias [1, H, S, total], head sink and softcap
    "bias_heads_sink_softcap": dict(dtype=BF16, B=2, S=2, H=4, KV=2, d=16, seqlens=[7, 5],
                                    cap=8, bias_shape=(1, 4, 2, 8), sink=True, softcap=3.0),
    # later call with position ids: the first B*S flattened ids (second axis wider than S)
    "position_ids_flat": dict(dtype=BF16, B=2, S=2, H=4, KV=2, d=32, seqlens=[6, 9], cap=10,
                              rotary=True, pid=np.array([[4, 5, 20, 21], [7, 8, 22, 23]])),
    # q/k RMSNorm before the rotation
    "qk_norm": dict(dtype=BF16, B=2, S=2, H=4, KV=2, d=64, seqlens=[5, 9], cap=10,
                    rotary=True, qk_norm=True),
    # integer caches that grow: zero codes 0 (int8) and 0x88 (int4) beyond the stored rows
    "int8_growing": dict(dtype=F16, B=2, S=2, H=4, KV=2, d=16, seqlens=[7, 4], cap=6,
                         cache_dtype=I8, modes=(PER_CHANNEL, PER_TENSOR)),
    "int4_growing": dict(dtype=F32, B=2, S=2, H=4, KV=2, d=16, seqlens=[7, 4], cap=6,
                         cache_dtype=I4, modes=(PER_TENSOR, PER_CHANNEL)),
    # bidirectional attention over the whole stored sequence
    "non_causal": dict(dtype=F32, B=2, S=3, H=2, KV=1, d=8, seqlens=[5, 8], cap=9, causal=0),
}




def form_case(form, **over):
    kw = dict(FORMS[form])
    kw.update(over)
    return gqa_case(kw.pop("dtype"), kw.pop("B"), kw.pop("S"), kw.pop("H"), kw.pop("KV"),
                    kw.pop("d"), kw.pop("seqlens"), seed=kw.pop("seed", len(form)), **kw)
