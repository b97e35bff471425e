"""Seeded PagedAttention cases shared by the CPU and GPU tests.

Shapes and draws follow the reference's own test inputs (tests/ops/test_paged_attention.py:
182-208: numpy default_rng(seed), new lengths in [1, 4], past uniform within capacity, values
N(0,1)*0.3, block_table = permutation of the pool), with the dtype and geometry as parameters.
bf16 values are produced with the oracle's RNE encoder (pinned against torch in test_oracle).
"""
from __future__ import annotations

import numpy as np

import _oracle as orc
from _oracle import BF16, E4M3, F16, F32, I4, I8, PER_CHANNEL, PER_TENSOR, RAW


def rotary_cache(positions: int, rot_dim: int, theta: float, dtype: int):
    """cos/sin [positions, rot_dim/2] built in float64 then rounded to dtype (the structured
    cache the reference's tests and _models.rotary_caches build, _models.py:261-266)."""
    half = rot_dim // 2
    inv = 1.0 / (theta ** (np.arange(half, dtype=np.float64) / half))
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return orc.encode(np.cos(ang), dtype), orc.encode(np.sin(ang), dtype)


def fp8_pages(rng, shape, scale_mult=1.0):
    """e4m3 pages with per-(block, kv-head) fp32 scales: x ~ N(0,1), scale = amax/448."""
    nb, bs, kv, d = shape
    x = rng.standard_normal(shape).astype(np.float32) * scale_mult
    amax = np.abs(x).max(axis=(1, 3))  # [nb, kv]
    scale = (amax / 448.0).astype(np.float32)
    scale[scale == 0] = 1.0
    codes = orc.encode(x / scale[:, None, :, None], E4M3)
    return codes, scale


def int_scales(KV, d, mode, side):
    """Integer-cache scales as the reference's tests draw them (test_quantized_kv.py:73-78):
    per-tensor 0.125 (k) / 0.25 (v); per-channel a cycle of eight values, zero included, rolled
    by the side, shaped [KV, d]."""
    if mode == PER_TENSOR:
        return np.array([0.125 if side == 0 else 0.25], np.float32)
    pattern = np.array([0.125, 0.25, 0.5, 1, 0.0625, 0.375, 2, 0], np.float32)
    return np.roll(np.resize(pattern, (KV, 1, d)), side, axis=-1).reshape(KV, d).copy()


def make_case(H, KV, d, nb, bs, batch, *, dtype=F16, cache_dtype=None, seed=0, new_lens=None,
              past=None, max_blocks=None, do_rotary=0, interleaved=0, theta=10000.0,
              rot_dim=None, rotary_offset=0, slot_mapping=None, head_sink=None, qk_norm=False,
              softcap=0.0, window=-1, causal=1, scale=0.0, std=0.3, value_std=None,
              int_modes=(PER_CHANNEL, PER_CHANNEL)):
    rng = np.random.default_rng(seed)
    cache_dtype = dtype if cache_dtype is None else cache_dtype
    if max_blocks is None:
        max_blocks = nb // batch
    cap = max_blocks * bs
    if new_lens is None:
        new_lens = rng.integers(1, min(4, cap) + 1, size=batch)
    new_lens = np.asarray(new_lens, np.int32)
    if past is None:
        past = np.array([rng.integers(0, cap - nl + 1) for nl in new_lens])
    past = np.asarray(past, np.int32)
    cum = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
    T = int(cum[-1])
    vstd = std if value_std is None else value_std

    def draw(shape, s):
        return orc.encode(rng.standard_normal(shape) * s, dtype)

    case = dict(num_heads=H, kv_num_heads=KV, head_dim=d, dtype=dtype, cache_dtype=cache_dtype,
                cum=cum, past=past, softcap=softcap, local_window_size=window, is_causal=causal,
                scale=scale)
    case["query"] = draw((T, H * d), std)
    case["key"] = draw((T, KV * d), std)
    case["value"] = draw((T, KV * d), vstd)
    if cache_dtype == E4M3:
        case["key_cache"], case["k_scale"] = fp8_pages(rng, (nb, bs, KV, d))
        case["value_cache"], case["v_scale"] = fp8_pages(rng, (nb, bs, KV, d))
    elif cache_dtype in (I8, I4):
        # random resident codes (test_quantized_kv.py:357-359) and the reference's scales
        width = d if cache_dtype == I8 else (d + 1) // 2
        for side, name in enumerate(("key", "value")):
            if cache_dtype == I8:
                case[f"{name}_cache"] = rng.integers(-128, 128, (nb, bs, KV, width), dtype=np.int8)
            else:
                case[f"{name}_cache"] = rng.integers(0, 256, (nb, bs, KV, width), dtype=np.uint8)
            case["kv"[side] + "_scale"] = int_scales(KV, d, int_modes[side], side)
        case["k_quant"], case["v_quant"] = int_modes
    else:
        case["key_cache"] = draw((nb, bs, KV, d), std)
        case["value_cache"] = draw((nb, bs, KV, d), vstd)
    case["block_table"] = rng.permutation(nb)[: batch * max_blocks].astype(np.int32).reshape(
        batch, max_blocks)
    if do_rotary:
        rd = d if rot_dim is None else rot_dim
        case["cos_cache"], case["sin_cache"] = rotary_cache(cap + 8, rd, theta, dtype)
        case["rotary_offset"] = rotary_offset
        case["rotary_interleaved"] = interleaved
    if slot_mapping is not None:
        case["slot_mapping"] = np.asarray(slot_mapping, np.int32)
    if head_sink is not None:
        hs = orc.encode(np.asarray(head_sink, np.float32), dtype)
        case["head_sink"] = hs
        case["head_sink_f32"] = orc.decode(hs, dtype)
    if qk_norm:
        case["q_norm"] = orc.encode(np.linspace(0.75, 1.25, d), dtype)
        case["k_norm"] = orc.encode(np.linspace(1.25, 0.75, d), dtype)
        case["qk_norm_epsilon"] = 1e-5
    return case


# ----------------------------------------------------------------------------- torch bridging

def torch_dtype(code: int):
    import torch
    return {F16: torch.float16, BF16: torch.bfloat16, F32: torch.float32,
            E4M3: torch.float8_e4m3fn, I8: torch.int8, I4: torch.uint8}[code]


def to_torch(raw: np.ndarray, code: int, device="cuda"):
    import torch
    raw = np.ascontiguousarray(raw)
    if code == BF16:
        t = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16)
    elif code == E4M3:
        t = torch.from_numpy(raw).view(torch.float8_e4m3fn)
    else:
        t = torch.from_numpy(raw)
    return t.to(device)


def from_torch(t, code: int) -> np.ndarray:
    import torch
    t = t.detach().cpu().contiguous()
    if code == BF16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if code == E4M3:
        return t.view(torch.uint8).numpy()
    return t.numpy()


QUANT_NAMES = {0: "NONE", PER_TENSOR: "PER_TENSOR", PER_CHANNEL: "PER_CHANNEL"}


def run_gpu_op(case: dict, validate=True, device="cuda", packed=False, max_query_len=0,
               cache_outputs="omitted", static_scratch=False, max_context_len=0):
    """Run the operator-level entry (pa_paged_attention) on the GPU for a case.  packed: hand
    Q, K and V over as one [T, (H + 2 KV) * d] query with key = value = None.
    cache_outputs: "omitted" (outputs 1/2 absent), "aliased" (bound onto the input caches) or
    "separate" (buffers of their own, pre-filled with a garbage pattern); with "separate" the
    return value also holds the input caches after the call: (out, kc_out, vc_out, kc_in, vc_in).
    """
    import torch
    import onnxruntime_ep_mlx_amd as ep
    dt, cdt = case["dtype"], case["cache_dtype"]
    T = lambda k, code=dt: None if case.get(k) is None else to_torch(case[k], code, device)
    I = lambda k: None if case.get(k) is None else torch.from_numpy(
        np.ascontiguousarray(case[k], np.int32)).to(device)
    F = lambda k: None if case.get(k) is None else torch.from_numpy(case[k]).to(device)
    kc, vc = T("key_cache", cdt), T("value_cache", cdt)
    q, k, v = T("query"), T("key"), T("value")
    if packed:
        q, k, v = torch.cat([q, k, v], dim=1).contiguous(), None, None
    kco = vco = None
    if cache_outputs == "aliased":
        kco, vco = kc, vc
    elif cache_outputs == "separate":
        kco = torch.full_like(kc.view(torch.uint8), 0x5A).view(kc.dtype)
        vco = None if vc is None else torch.full_like(vc.view(torch.uint8), 0xA5).view(vc.dtype)
    kc_in, vc_in = kc, vc
    out, kc, vc = ep.paged_attention(
        q, k, v, kc, vc, I("cum"), I("past"), I("block_table"),
        T("cos_cache"), T("sin_cache"), I("slot_mapping"), T("head_sink"), T("q_norm"),
        T("k_norm"), F("k_scale"), F("v_scale"), None,
        num_heads=case["num_heads"], kv_num_heads=case["kv_num_heads"],
        scale=case.get("scale", 0.0), softcap=case.get("softcap", 0.0),
        local_window_size=case.get("local_window_size", -1),
        do_rotary=int("cos_cache" in case), rotary_interleaved=case.get("rotary_interleaved", 0),
        rotary_offset=case.get("rotary_offset", 0), is_causal=case.get("is_causal", 1),
        qk_norm_epsilon=case.get("qk_norm_epsilon", 1e-6),
        k_quant_type=QUANT_NAMES[case.get("k_quant", 0)],
        v_quant_type=QUANT_NAMES[case.get("v_quant", 0)],
        v_head_size=case.get("v_head_size", 0),
        kv_cache_layout="LATENT" if case.get("latent") else "SEPARATE", validate=validate,
        key_cache_out=kco, value_cache_out=vco, max_query_len=max_query_len,
        max_context_len=max_context_len, static_scratch=static_scratch)
    torch.cuda.synchronize()
    res = (from_torch(out, dt), from_torch(kc, cdt), None if vc is None else from_torch(vc, cdt))
    if cache_outputs == "separate":
        res += (from_torch(kc_in, cdt), None if vc_in is None else from_torch(vc_in, cdt))
    return res


def make_latent_case(H, d, vd, nb, bs, batch, **kw):
    """LATENT layout case (kv_num_heads 1, no value input or value cache)."""
    c = make_case(H, 1, d, nb, bs, batch, **kw)
    c.pop("value")
    c.pop("value_cache")
    c["latent"] = True
    c["v_head_size"] = vd
    return c
