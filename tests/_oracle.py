"""ctypes access to the CPU oracle (oracle/build/libpa_oracle.so) for the test suite.

Test infrastructure only: the oracle is the checker, never the thing measured or shipped.
Arrays are numpy "raw storage" arrays: float16 for fp16, uint16 bit patterns for bf16,
float32 for fp32, uint8 codes for fp8 e4m3.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
LIB = ORACLE_DIR / "build" / "libpa_oracle.so"

F16, BF16, F32, E4M3, I8, I4 = 1, 2, 3, 4, 5, 6
RAW = {F16: np.float16, BF16: np.uint16, F32: np.float32, E4M3: np.uint8, I8: np.int8,
       I4: np.uint8}
NAMES = {F16: "fp16", BF16: "bf16", F32: "fp32", E4M3: "e4m3", I8: "int8", I4: "int4"}
PER_TENSOR, PER_CHANNEL = 1, 2

_lib = None


class GqaArgs(C.Structure):
    """orc_gqa_args (oracle/pa_oracle.h)."""
    _fields_ = [(n, C.c_int) for n in ("dtype", "batch", "seq", "kv_seq", "num_heads",
                                       "kv_heads", "head_dim")] + [
        ("query", C.c_void_p), ("key", C.c_void_p), ("value", C.c_void_p),
        ("past_k", C.c_void_p), ("past_v", C.c_void_p), ("past_cap", C.c_int),
        ("present_k", C.c_void_p), ("present_v", C.c_void_p), ("present_cap", C.c_int),
        ("seqlens_k", C.c_void_p), ("total", C.c_int64),
        ("cos_cache", C.c_void_p), ("sin_cache", C.c_void_p), ("cos_rows", C.c_int64),
        ("rot_half", C.c_int), ("interleaved", C.c_int),
        ("position_ids", C.c_void_p), ("bias", C.c_void_p), ("bias_b", C.c_int),
        ("bias_h", C.c_int), ("head_sink", C.c_void_p), ("smooth", C.c_int),
        ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("norm_eps", C.c_float),
        ("scale", C.c_float), ("softcap", C.c_float), ("window", C.c_int), ("causal", C.c_int),
        ("cache_dtype", C.c_int), ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
        ("k_mode", C.c_int), ("v_mode", C.c_int),
        ("sliding", C.c_int), ("qk_mode", C.c_int), ("qk_out", C.c_void_p),
    ]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", os.fspath(ORACLE_DIR)], check=True)
        L = C.CDLL(os.fspath(LIB))
        P, I32, I64, F = C.c_void_p, C.c_int, C.c_int64, C.c_float
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [F]
        L.orc_bf16_to_f32.restype = F
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [F]
        L.orc_f16_to_f32.restype = F
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_e4m3.restype = C.c_uint8
        L.orc_f32_to_e4m3.argtypes = [F]
        L.orc_e4m3_to_f32.restype = F
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_encode.argtypes = [P, P, I64, I32]
        L.orc_decode.argtypes = [P, P, I64, I32]
        L.orc_rms_norm_rows.argtypes = [P, I64, I32, I32, P, F, I32]
        L.orc_rope_rows.restype = I32
        L.orc_rope_rows.argtypes = [P, I64, I32, I32, P, P, P, I64, I32, I32, I32, I32]
        L.orc_int_code.restype = I32
        L.orc_int_code.argtypes = [F, F, I32, I32]
        L.orc_int_encode_row.argtypes = [P, I32, P, I32, I32, I32, P]
        L.orc_int_decode_row.argtypes = [P, I32, P, I32, I32, P]
        L.orc_reshape_and_cache.restype = I32
        L.orc_reshape_and_cache.argtypes = [P, P, I32, P, P, I32, P, P, I32, I32, P, P, P, I32,
                                            I32, P, I64, I32, I32, I32]
        L.orc_paged_attention.restype = I32
        L.orc_paged_attention.argtypes = [P, P, P, I32, P, P, I32, P, P, I32, I32, P, P, P, I32,
                                          I32, I64, I32, I32, I32, I32, F, F, I32, I32, P, P, I32]
        L.orc_paged_attention_op.restype = I32
        L.orc_paged_attention_op.argtypes = [I32, I32, P, P, P, I64, P, P, P, P, I32, I32, I64,
                                             I32, P, P, P, I32, I32, P, P, I64, I32, I32, I32, P,
                                             P, P, P, F, I32, I32, I32, F, F, I32, I32, P, P,
                                             I32]
        L.orc_gqa_contiguous.restype = I32
        L.orc_gqa_contiguous.argtypes = [I32, P, P, P, P, P, I32, I32, I32, I32, I32, I32, P, F,
                                         F, I32, I32, P, I32, P, P, I32, I32]
        L.orc_gqa_batched.restype = I32
        L.orc_gqa_batched.argtypes = [C.POINTER(GqaArgs), P]
        L.orc_sum_squares.restype = F
        L.orc_sum_squares.argtypes = [P, I64, I32, I32]
        L.orc_cpu_gqa_decode.restype = I32
        L.orc_cpu_gqa_decode.argtypes = [I32, P, P, P, P, P, I32, I32, I32, I32, F, P, I32]
        L.orc_cpu_gqa_prefill.restype = I32
        L.orc_cpu_gqa_prefill.argtypes = [I32, P, P, P, P, P, P, P, I32, I32, I32, I32, F, P,
                                          I32]
        _lib = L
    return _lib


def _p(a):
    """Pointer argument for a C call.  data_as keeps a reference to the array, so a temporary
    made inline in the call's argument list stays alive until the call returns."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def encode(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, RAW[dtype])
    lib().orc_encode(_p(x), _p(out), x.size, dtype)
    return out


def decode(raw: np.ndarray, dtype: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw)
    out = np.empty(raw.shape, np.float32)
    lib().orc_decode(_p(raw), _p(out), raw.size, dtype)
    return out


def rms_norm_rows(x: np.ndarray, heads: int, head_dim: int, weight: np.ndarray, eps: float,
                  dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x).copy()
    rows = x.size // (heads * head_dim)
    lib().orc_rms_norm_rows(_p(x), rows, heads, head_dim, _p(np.ascontiguousarray(weight)),
                            eps, dtype)
    return x


def rope_rows(x: np.ndarray, heads: int, head_dim: int, positions: np.ndarray, cos: np.ndarray,
              sin: np.ndarray, offset: int, interleaved: int, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x).copy()
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    rc = lib().orc_rope_rows(_p(x), pos.size, heads, head_dim, _p(pos), _p(cos), _p(sin),
                             cos.shape[0], cos.shape[1], offset, interleaved, dtype)
    assert rc == 0, rc
    return x


def int_code(x: float, scale: float, bits: int, reciprocal: bool = False) -> int:
    return lib().orc_int_code(x, scale, bits, int(reciprocal))


def int_encode_row(x, scale, bits, per_channel=False, reciprocal=False) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    scale = np.ascontiguousarray(scale, np.float32)
    d = x.shape[-1]
    out = np.empty(d if bits == 8 else (d + 1) // 2, np.uint8)
    lib().orc_int_encode_row(_p(x), d, _p(scale), int(per_channel), bits, int(reciprocal),
                             _p(out))
    return out.view(np.int8) if bits == 8 else out


def int_decode_row(codes, head_dim, scale, bits, per_channel=False) -> np.ndarray:
    codes = np.ascontiguousarray(codes).view(np.uint8)
    scale = np.ascontiguousarray(scale, np.float32)
    out = np.empty(head_dim, np.float32)
    lib().orc_int_decode_row(_p(codes), head_dim, _p(scale), int(per_channel), bits, _p(out))
    return out


def head_dim_of(cache: np.ndarray, cache_dtype: int, head_dim: int | None = None) -> int:
    """Logical head size of a [nb, bs, KV, width] cache (int4 width = ceil(d / 2))."""
    if head_dim is not None:
        return head_dim
    return cache.shape[3] * 2 if cache_dtype == I4 else cache.shape[3]


def reshape_and_cache(key, value, act_dtype, kc, vc, cache_dtype, cum, past, bt,
                      slot_mapping=None, k_scale=None, v_scale=None, k_mode=0, v_mode=0,
                      head_dim=None):
    kc, vc = kc.copy(), vc.copy()
    nb, bs, kv, _ = kc.shape
    d = head_dim_of(kc, cache_dtype, head_dim)
    rc = lib().orc_reshape_and_cache(
        _p(key), _p(value), act_dtype, _p(kc), _p(vc), cache_dtype, _p(k_scale), _p(v_scale),
        k_mode, v_mode, _p(cum), _p(past), _p(bt), len(cum) - 1, bt.shape[1], _p(slot_mapping),
        nb, bs, kv, d)
    assert rc == 0, rc
    return kc, vc


def paged_attention_op(case: dict, *, return_cache=True):
    """Run the whole operator on a case dict (see pa_cases.make_case).  A case without a
    value_cache (and value) is the LATENT layout with v_head_size output dims."""
    c = case
    kc = c["key_cache"].copy()
    vc = None if c.get("value_cache") is None else c["value_cache"].copy()
    nb, bs, kv, _ = kc.shape
    d = head_dim_of(kc, c["cache_dtype"], c.get("head_dim"))
    vd = c.get("v_head_size", 0) or d
    T = c["query"].shape[0]
    H = c["num_heads"]
    out = np.zeros((T, H * vd), np.float64)
    out_t = np.zeros((T, H * vd), RAW[c["dtype"]])
    cos, sin = c.get("cos_cache"), c.get("sin_cache")
    sink = c.get("head_sink_f32")
    rc = lib().orc_paged_attention_op(
        c["dtype"], c["cache_dtype"], _p(c["query"]), _p(c["key"]), _p(c.get("value")), T, _p(kc),
        _p(vc), _p(c.get("k_scale")), _p(c.get("v_scale")), c.get("k_quant", 0),
        c.get("v_quant", 0), nb, bs, _p(c["cum"]), _p(c["past"]),
        _p(c["block_table"]), len(c["cum"]) - 1, c["block_table"].shape[1], _p(cos), _p(sin),
        0 if cos is None else cos.shape[0], 0 if cos is None else cos.shape[1],
        c.get("rotary_offset", 0), c.get("rotary_interleaved", 0), _p(c.get("slot_mapping")),
        _p(sink), _p(c.get("q_norm")), _p(c.get("k_norm")), c.get("qk_norm_epsilon", 1e-6), H,
        kv, d, c.get("scale", 0.0) or float(np.float32(1.0) / np.sqrt(np.float32(d))),
        c.get("softcap", 0.0), c.get("local_window_size", -1), c.get("is_causal", 1), _p(out),
        _p(out_t), vd)
    assert rc == 0, rc
    return out, out_t, kc, vc


def paged_attention(q, k_new, v_new, act_dtype, kc, vc, cache_dtype, cum, past, bt, H, scale,
                    softcap=0.0, window=-1, causal=1, head_sink=None, k_scale=None,
                    v_scale=None, k_mode=0, v_mode=0, head_dim=None):
    nb, bs, kv, _ = kc.shape
    d = head_dim_of(kc, cache_dtype, head_dim)
    out = np.zeros((q.shape[0], H * d), np.float64)
    rc = lib().orc_paged_attention(
        _p(q), _p(k_new), _p(v_new), act_dtype, _p(kc), _p(vc), cache_dtype, _p(k_scale),
        _p(v_scale), k_mode, v_mode, _p(cum), _p(past), _p(bt), len(cum) - 1, bt.shape[1], nb,
        bs, H, kv, d, scale, softcap, window, causal, _p(head_sink), _p(out), 0)
    assert rc == 0, rc
    return out


def gqa_contiguous(dtype, q, k, v, pk, pv, seqlens_k, H, KV, d, scale, softcap=0.0, window=-1,
                   causal=1, cache_dtype=0, k_scale=None, v_scale=None, k_mode=0, v_mode=0):
    B, S = q.shape[0], q.shape[1]
    pk, pv = pk.copy(), pv.copy()
    out = np.zeros((B, S, H * d), np.float64)
    rc = lib().orc_gqa_contiguous(dtype, _p(q), _p(k), _p(v), _p(pk), _p(pv), B, S, H, KV, d,
                                  pk.shape[2], _p(np.ascontiguousarray(seqlens_k, np.int32)),
                                  scale, softcap, window, causal, _p(out), cache_dtype,
                                  _p(k_scale), _p(v_scale), k_mode, v_mode)
    assert rc == 0, rc
    return out, pk, pv


def sum_squares(x: np.ndarray, dtype: int) -> float:
    """orc_sum_squares of one row (the fixed RMSNorm reduction order)."""
    x = np.ascontiguousarray(x)
    return float(lib().orc_sum_squares(_p(x), 0, x.size, dtype))


def gqa_batched(dtype, q, k, v, past_k, past_v, seqlens_k, total, H, KV, d, *, scale,
                present_cap=None, softcap=0.0, window=-1, causal=1, cos=None, sin=None,
                interleaved=0, position_ids=None, bias=None, head_sink=None, smooth=0,
                q_norm=None, k_norm=None, norm_eps=1e-6, cache_dtype=0, k_scale=None,
                v_scale=None, k_mode=0, v_mode=0, sliding=0, qk_mode=0):
    """orc_gqa_batched: every GroupQueryAttention form on contiguous caches.  q [B, S, H*d];
    k/v [B, kv_seq, KV*d] or None (kv_seq 0); past_k/v [B, KV, cap, w] or None.  sliding: the
    sliding_window_cache ring (present capacity = past capacity); qk_mode 1 / 2: output_qk.
    Returns (out float64 [B, S, H*d], present_k, present_v), plus the float64 diagnostics
    [B, H, S, total] when qk_mode is set."""
    B, S = q.shape[0], q.shape[1]
    kv_seq = 0 if k is None else k.shape[1]
    cap = 0 if past_k is None else past_k.shape[2]
    if present_cap is None:
        present_cap = cap if sliding else max(cap, int(total))
    qk = np.zeros((B, H, S, int(total)), np.float64) if qk_mode else None
    w = d if not cache_dtype else (d if cache_dtype == I8 else (d + 1) // 2)
    raw = RAW[cache_dtype or dtype]
    pres_k = np.zeros((B, KV, present_cap, w), raw)
    pres_v = np.zeros((B, KV, present_cap, w), raw)
    out = np.zeros((B, S, H * d), np.float64)
    keep = []

    def ptr(x, dt=None):
        if x is None:
            return None
        x = np.ascontiguousarray(x, dt) if dt is not None else np.ascontiguousarray(x)
        keep.append(x)
        return x.ctypes.data

    a = GqaArgs(dtype=dtype, batch=B, seq=S, kv_seq=kv_seq, num_heads=H, kv_heads=KV,
                head_dim=d, query=ptr(q), key=ptr(k), value=ptr(v), past_k=ptr(past_k),
                past_v=ptr(past_v), past_cap=cap, present_k=pres_k.ctypes.data,
                present_v=pres_v.ctypes.data, present_cap=present_cap,
                seqlens_k=ptr(seqlens_k, np.int32), total=int(total), cos_cache=ptr(cos),
                sin_cache=ptr(sin), cos_rows=0 if cos is None else cos.shape[0],
                rot_half=0 if cos is None else cos.shape[1], interleaved=interleaved,
                position_ids=ptr(position_ids, np.int64), bias=ptr(bias),
                bias_b=0 if bias is None else bias.shape[0],
                bias_h=0 if bias is None else bias.shape[1], head_sink=ptr(head_sink),
                smooth=smooth, q_norm=ptr(q_norm), k_norm=ptr(k_norm), norm_eps=norm_eps,
                scale=scale, softcap=softcap, window=window, causal=causal,
                cache_dtype=cache_dtype, k_scale=ptr(k_scale, np.float32),
                v_scale=ptr(v_scale, np.float32), k_mode=k_mode, v_mode=v_mode,
                sliding=sliding, qk_mode=qk_mode, qk_out=None if qk is None else qk.ctypes.data)
    rc = lib().orc_gqa_batched(C.byref(a), out.ctypes.data)
    assert rc == 0, rc
    if qk_mode:
        return out, pres_k, pres_v, qk
    return out, pres_k, pres_v


def cpu_gqa_decode(dtype, q, k, v, kv_offset, ctx, H, KV, d, scale, threads):
    B = len(ctx)
    out = np.zeros((B, H, d), np.float32)
    rc = lib().orc_cpu_gqa_decode(dtype, _p(q), _p(k), _p(v),
                                  _p(np.ascontiguousarray(kv_offset, np.int64)),
                                  _p(np.ascontiguousarray(ctx, np.int32)), B, H, KV, d, scale,
                                  _p(out), threads)
    assert rc == 0, rc
    return out


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def cpu_gqa_prefill(dtype, q, k, v, kv_offset, q_start, nq, past, H, KV, d, scale, threads):
    """CPU path of chunked prefill (causal GQA over contiguous K/V); q is [T, H * d]."""
    B = len(nq)
    out = np.zeros((q.shape[0], H, d), np.float32)
    rc = lib().orc_cpu_gqa_prefill(dtype, _p(q), _p(k), _p(v),
                                   _p(np.ascontiguousarray(kv_offset, np.int64)),
                                   _p(np.ascontiguousarray(q_start, np.int32)),
                                   _p(np.ascontiguousarray(nq, np.int32)),
                                   _p(np.ascontiguousarray(past, np.int32)), B, H, KV, d, scale,
                                   _p(out), threads)
    assert rc == 0, rc
    return out
