#!/usr/bin/env python3
"""Benchmark: paged GQA decode step at the Llama-3-8B shape.

One step = the hot path over one batch through the operator entry pa_paged_attention: host
validation of the int32 metadata, fused RoPE + KV append of the 64 new tokens, and the balanced
split-K paged decode on matrix cores.  Inputs are synthetic (seeded N(0,1), bf16) and resident in
HBM before timing.

  value      = algorithmic KV bytes per step / step time (GB/s); KV bytes = 4096 * sum(ctx)
  roofline   = the attention launch (pa_attention_ex: balanced decode kernel + partial merge
               kernel, same stream) timed with events on that stream: KV bytes / launch time vs
               8 TB/s
  cpu_baseline = the oracle's threaded contiguous-KV GQA decode (ORT CPU semantics) on a
               bounded sample of the same sequences, scaled to the full batch by KV bytes

--config c4 / c5 measure BASELINE.json configs 4 (chunked prefill, Qwen2.5-7B shape: value =
TFLOP/s of the causal attention FLOPs, roofline vs the 2.5 PFLOP/s dense bf16 MFMA peak) and 5
(fp8 e4m3 pages, B=16, ctx 32768: value = GB/s of fp8 KV bytes, roofline vs 8 TB/s) the same way;
their lines carry their own metric names; their CPU baselines are the same CPU path on one
sequence (causal prefill chunk / fp8 pages dequantised to fp32).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config c3|c4|c5]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, os.fspath(ROOT / "onnxruntime-ep-mlx_amd"))

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-ms", type=float, default=200.0,
                    help="after the --warmup steps, further untimed steps until this much wall "
                         "time has passed: the first ~20 ms of sustained load after an idle GPU "
                         "run ~10 %% slower (C4: 290 vs 255-260 us per step)")
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--chunk", type=int, default=0, help="split-K chunk (0 = library default)")
    ap.add_argument("--cpu-sample", type=int, default=16, help="sequences in the CPU sample")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 1 GiB device copies (known bytes) to scale HBM counters")
    ap.add_argument("--config", choices=("c3", "c4", "c5"), default="c3",
                    help="c3 (default): BASELINE.json config 3; c4 / c5: configs 4 / 5")
    ap.add_argument("--head-dim", type=int, default=128, choices=(64, 96, 128, 256),
                    help="c3 / c4: the same batch at another head size (128 = the config)")
    ap.add_argument("--cache-dtype", default="bf16", choices=("bf16", "int8", "int4", "fp8"),
                    help="c3 / c4: the same batch over int8 / int4 pages with per-channel "
                         "fp32 scales (bf16 = the config); c4 also over fp8 e4m3 pages")
    ap.add_argument("--gqa", action="store_true",
                    help="c3 only: the same decode batch through GroupQueryAttention "
                         "(pa_group_query_attention) over contiguous presents [64, 8, 8192, 128] "
                         "updated in place, --cache-dtype bf16 / int8 / int4")
    ap.add_argument("--latent", type=int, default=0, metavar="HEADS",
                    help="c3 only: the config 3 contexts through the LATENT layout (MLA: one "
                         "kv-head of 576-dim rows, values = their first 512 dims, RoPE on the last "
                         "64) with HEADS query heads (16 or 128)")
    ap.add_argument("--bias", action="store_true",
                    help="with --gqa: an attention_bias [64, 1, 1, total] (bf16 N(0,1))")
    return ap.parse_args()


def load_traffic(name="decode_c3_traffic.json"):
    """HBM bytes per attention launch from the committed counter summary, if present."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    with open(path) as f:
        t = json.load(f)
    return t.get("hbm_bytes_per_launch")


def build_workload(torch, ep, seed, d=128, cache="bf16"):
    import numpy as np
    rng = np.random.default_rng(seed)
    B, H, KV, bs, nb = 64, 32, 8, 16, 40000
    ctx = rng.integers(512, 8193, size=B).astype(np.int32)
    mb = 8192 // bs
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((B, mb), np.int32)
    used = 0
    for b in range(B):
        n = (int(ctx[b]) + bs - 1) // bs
        bt[b, :n] = perm[used:used + n]
        bt[b, n:] = perm[used]
        used += n
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(seed)
    ks = vs = None
    if cache == "bf16":
        kc = torch.empty((nb, bs, KV, d), dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        for t in (kc, vc):  # fill in slices to bound the fp32 temporary
            for i in range(0, nb, 5000):
                t[i:i + 5000] = torch.randn((min(5000, nb - i), bs, KV, d), generator=g,
                                            device=dev).to(torch.bfloat16)
    else:
        # integer codes uniform over the code range, per-channel scales [KV, d] of N(0,1) / 64
        width, dt = (d, torch.int8) if cache == "int8" else ((d + 1) // 2, torch.uint8)
        lo, hi = (-128, 128) if cache == "int8" else (0, 256)
        kc = torch.randint(lo, hi, (nb, bs, KV, width), generator=g, device=dev, dtype=dt)
        vc = torch.randint(lo, hi, (nb, bs, KV, width), generator=g, device=dev, dtype=dt)
        ks = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
        vs = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
    half = d // 2
    inv = 1.0 / (500000.0 ** (torch.arange(half, dtype=torch.float64) / half))
    ang = torch.arange(8192 + 8, dtype=torch.float64)[:, None] * inv[None, :]
    cos = ang.cos().to(torch.bfloat16).to(dev)
    sin = ang.sin().to(torch.bfloat16).to(dev)
    q = torch.randn((B, H * d), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, KV * d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, KV * d), generator=g, device=dev).to(torch.bfloat16)
    w = dict(B=B, T=B, mq=1, H=H, KV=KV, d=d, bs=bs, nb=nb, ctx=ctx, bt_np=bt, kc=kc, vc=vc,
             cos=cos, sin=sin, q=q, k=k, v=v, ks=ks, vs=vs, cache=cache,
             quant="NONE" if cache == "bf16" else "PER_CHANNEL")
    w["cum"] = torch.arange(B + 1, dtype=torch.int32, device=dev)
    w["past"] = torch.from_numpy(ctx - 1).to(dev)
    w["bt"] = torch.from_numpy(bt).to(dev)
    return w


def build_prefill_workload(torch, seed=4, d=128, cache="bf16"):
    """bf16, 8 sequences each appending a 512-token chunk over a cached
    context U[0, 4096], 28 query / 4 kv heads, d 128, block 16, causal within the chunk, packed
    cumulative_sequence_length, values N(0,1).  No rotary (the config names none).
    cache int8 / int4: the same batch over integer pages (codes uniform over the code range,
    per-channel fp32 scales [KV, d] of U[0.5, 1.5) / 64); fp8: over e4m3 pages, N(0,1) quantised
    with scale amax / 448 per (block, kv-head) as config 5 draws them."""
    import numpy as np
    rng = np.random.default_rng(seed)
    B, H, KV, bs, chunk = 8, 28, 4, 16, 512
    past = rng.integers(0, 4097, size=B).astype(np.int32)
    mb = (4096 + chunk + bs - 1) // bs
    nb = B * mb
    bt = rng.permutation(nb).astype(np.int32).reshape(B, mb)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(seed)
    ks = vs = None
    if cache == "bf16":
        kc = torch.randn((nb, bs, KV, d), generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn((nb, bs, KV, d), generator=g, device=dev).to(torch.bfloat16)
    elif cache == "fp8":
        kc = torch.empty((nb, bs, KV, d), dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.empty_like(kc)
        ks = torch.empty((nb, KV), dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        for t, sc in ((kc, ks), (vc, vs)):
            x = torch.randn((nb, bs, KV, d), generator=g, device=dev)
            sc.copy_((x.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-12))
            t.copy_((x / sc[:, None, :, None]).to(torch.float8_e4m3fn))
    else:
        width, dt = (d, torch.int8) if cache == "int8" else (d // 2, torch.uint8)
        lo, hi = (-128, 128) if cache == "int8" else (0, 256)
        kc = torch.randint(lo, hi, (nb, bs, KV, width), generator=g, device=dev, dtype=dt)
        vc = torch.randint(lo, hi, (nb, bs, KV, width), generator=g, device=dev, dtype=dt)
        ks = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
        vs = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
    T = B * chunk
    w = dict(B=B, T=T, mq=chunk, H=H, KV=KV, d=d, bs=bs, nb=nb, ctx=past + chunk, bt_np=bt,
             kc=kc, vc=vc, cos=None, sin=None, ks=ks, vs=vs, cache=cache,
             quant="PER_CHANNEL" if cache in ("int8", "int4") else "NONE",
             q=torch.randn((T, H * d), generator=g, device=dev).to(torch.bfloat16),
             k=torch.randn((T, KV * d), generator=g, device=dev).to(torch.bfloat16),
             v=torch.randn((T, KV * d), generator=g, device=dev).to(torch.bfloat16))
    w["cum"] = torch.arange(0, T + 1, chunk, dtype=torch.int32, device=dev)
    w["past"] = torch.from_numpy(past).to(dev)
    w["bt"] = torch.from_numpy(bt).to(dev)
    # causal attention FLOPs: QK and PV, 2 * 2 * H * d per visible (query, key) pair
    w["flops"] = sum(4.0 * H * d * (chunk * int(p) + chunk * (chunk + 1) / 2) for p in past)
    return w


def build_fp8_workload(torch, seed=5):
    """e4m3 K/V pages with per-(block, kv-head) fp32 scales, bf16 query,
    batch 16, 64 query / 8 kv heads, d 128, context 32768 per sequence, block 16, random block
    tables, values N(0,1) quantised with scale amax/448 per (block, kv-head)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    B, H, KV, d, bs, ctx = 16, 64, 8, 128, 16, 32768
    nbs = ctx // bs
    nb = B * nbs + 64
    bt = rng.permutation(nb)[: B * nbs].astype(np.int32).reshape(B, nbs)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.empty((nb, bs, KV, d), dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((nb, KV), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    for t, sc in ((kc, ks), (vc, vs)):
        for i in range(0, nb, 4096):  # slices bound the fp32 temporary
            n = min(4096, nb - i)
            x = torch.randn((n, bs, KV, d), generator=g, device=dev)
            s_ = (x.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-12)
            sc[i:i + n] = s_
            t[i:i + n] = (x / s_[:, None, :, None]).to(torch.float8_e4m3fn)
    w = dict(B=B, T=B, mq=1, H=H, KV=KV, d=d, bs=bs, nb=nb, ctx=np.full(B, ctx, np.int32),
             bt_np=bt, kc=kc, vc=vc, ks=ks, vs=vs, cos=None, sin=None,
             q=torch.randn((B, H * d), generator=g, device=dev).to(torch.bfloat16),
             k=torch.randn((B, KV * d), generator=g, device=dev).to(torch.bfloat16),
             v=torch.randn((B, KV * d), generator=g, device=dev).to(torch.bfloat16))
    w["cum"] = torch.arange(B + 1, dtype=torch.int32, device=dev)
    w["past"] = torch.full((B,), ctx - 1, dtype=torch.int32, device=dev)
    w["bt"] = torch.from_numpy(bt).to(dev)
    return w


class GqaStep:
    """GroupQueryAttention over the config 3 decode batch: contiguous presents [B, KV, 8192, d]
    (bf16, or int8 / int4 codes with per-channel scales) updated in place, seqlens_k = ctx - 1,
    one new token per sequence rotated at position ctx - 1; one ctypes call per step."""

    def __init__(self, torch, w, cache, bias):
        import numpy as np
        from onnxruntime_ep_mlx_amd import _capi as capi
        self.lib, self.capi = capi.load(), capi
        dev = torch.device("cuda", 0)
        g = torch.Generator(device=dev).manual_seed(11)
        B, H, KV, d, cap = w["B"], w["H"], w["KV"], w["d"], 8192
        if cache == "bf16":
            self.pk = torch.empty((B, KV, cap, d), dtype=torch.bfloat16, device=dev)
            self.pv = torch.empty_like(self.pk)
            for t in (self.pk, self.pv):
                for b in range(0, B, 8):
                    t[b:b + 8] = torch.randn((8, KV, cap, d), generator=g,
                                             device=dev).to(torch.bfloat16)
            ks = vs = None
            code, quant = 0, capi.PA_QUANT_NONE
        else:
            width, dt = (d, torch.int8) if cache == "int8" else (d // 2, torch.uint8)
            lo, hi = (-128, 128) if cache == "int8" else (0, 256)
            self.pk = torch.randint(lo, hi, (B, KV, cap, width), generator=g, device=dev,
                                    dtype=dt)
            self.pv = torch.randint(lo, hi, (B, KV, cap, width), generator=g, device=dev,
                                    dtype=dt)
            ks = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
            vs = (torch.rand((KV, d), generator=g, device=dev) + 0.5) / 64.0
            code = capi.PA_DTYPE_INT8 if cache == "int8" else capi.PA_DTYPE_INT4
            quant = capi.PA_QUANT_PER_CHANNEL
        self.keep = [ks, vs]
        self.seqlens = torch.from_numpy((w["ctx"] - 1).astype(np.int32)).to(dev)
        self.host = np.ascontiguousarray((w["ctx"] - 1).astype(np.int32))
        self.q = w["q"].view(B, 1, H * d)
        self.k = w["k"].view(B, 1, KV * d)
        self.v = w["v"].view(B, 1, KV * d)
        self.out = torch.empty_like(self.q)
        total = int(w["ctx"].max())  # the longest sequence after the new token
        self.bias = (torch.randn((B, 1, 1, total), generator=g, device=dev).to(torch.bfloat16)
                     if bias else None)
        ptr = lambda t: None if t is None else t.data_ptr()
        self.node = capi.PaGqaNode(H, KV, 0.0, 0.0, -1, 1, 0, 1, 1e-6, 0, 0, 0)
        self.io = capi.PaGqaIO(
            dtype=capi.PA_DTYPE_BFLOAT16, batch=B, seq=1, query_hidden=H * d, kv_seq=1,
            query=ptr(self.q), key=ptr(self.k), value=ptr(self.v), past_key=ptr(self.pk),
            past_value=ptr(self.pv), past_capacity=cap, present_key=ptr(self.pk),
            present_value=ptr(self.pv), present_capacity=cap, seqlens_k=ptr(self.seqlens),
            host_seqlens_k=self.host.ctypes.data, total_sequence_length=total,
            cos_cache=ptr(w["cos"]), sin_cache=ptr(w["sin"]),
            rotary_positions=w["cos"].shape[0], rotary_half=w["cos"].shape[1],
            attention_bias=ptr(self.bias), bias_batch=B if bias else 0,
            bias_heads=1 if bias else 0, output=ptr(self.out), cache_dtype=code,
            k_scale=ptr(ks), v_scale=ptr(vs), k_quant_type=quant, v_quant_type=quant)
        self.ws_bytes = self.lib.pa_group_query_attention_workspace_bytes(C.byref(self.node),
                                                                         C.byref(self.io))
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream().cuda_stream

    def __call__(self):
        self.capi.check(self.lib.pa_group_query_attention(
            C.byref(self.node), C.byref(self.io), self.ws.data_ptr(), self.ws_bytes,
            self.stream))


class LatentStep:
    """The config 3 decode contexts (B=64, ctx U[512,8192] seed 3, block 16) through the LATENT
    layout: one kv-head of 576-dim key rows whose first 512 dims are the values (MLA), H query
    heads, RoPE (theta 10000) on dims 512..575, one new row per sequence; one ctypes call per step
    (pa_paged_attention)."""

    def __init__(self, torch, seed, H):
        import numpy as np
        from onnxruntime_ep_mlx_amd import _capi as capi
        from onnxruntime_ep_mlx_amd.ops import cache_desc
        self.lib, self.capi = capi.load(), capi
        rng = np.random.default_rng(seed)
        B, D, VD, bs = 64, 576, 512, 16
        self.ctx = rng.integers(512, 8193, size=B).astype(np.int32)
        mb = 8192 // bs
        nb = int(sum((int(c) + bs - 1) // bs for c in self.ctx)) + 64
        perm = rng.permutation(nb).astype(np.int32)
        bt = np.zeros((B, mb), np.int32)
        used = 0
        for b in range(B):
            n = (int(self.ctx[b]) + bs - 1) // bs
            bt[b, :n] = perm[used:used + n]
            bt[b, n:] = perm[used]
            used += n
        dev = torch.device("cuda", 0)
        g = torch.Generator(device=dev).manual_seed(seed)
        self.kc = torch.randn((nb, bs, 1, D), generator=g, device=dev).to(torch.bfloat16)
        half = 32
        inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float64) / half))
        ang = torch.arange(8192 + 8, dtype=torch.float64)[:, None] * inv[None, :]
        self.cos = ang.cos().to(torch.bfloat16).to(dev)
        self.sin = ang.sin().to(torch.bfloat16).to(dev)
        self.q = torch.randn((B, H * D), generator=g, device=dev).to(torch.bfloat16)
        self.k = torch.randn((B, D), generator=g, device=dev).to(torch.bfloat16)
        self.out = torch.empty((B, H * VD), dtype=torch.bfloat16, device=dev)
        self.cum = torch.arange(B + 1, dtype=torch.int32, device=dev)
        self.past = torch.from_numpy(self.ctx - 1).to(dev)
        self.bt = torch.from_numpy(bt).to(dev)
        self.host = {"cum": np.arange(B + 1, dtype=np.int32),
                     "past": np.ascontiguousarray(self.ctx - 1), "bt": bt}
        self.node = capi.PaNode(H, 1, float(1 / np.sqrt(192)), 0.0, -1, 1, 0, VD, 1, 1e-6, VD, 1)
        self.io = capi.PaIO(
            capi.PA_DTYPE_BFLOAT16, B, H * D, self.q.data_ptr(), self.k.data_ptr(), None,
            cache_desc(self.kc, None, head_dim=D), self.cum.data_ptr(), self.past.data_ptr(),
            self.bt.data_ptr(), B, mb, self.cos.data_ptr(), self.sin.data_ptr(),
            self.cos.shape[0], half, None, None, None, None, self.host["cum"].ctypes.data,
            self.host["past"].ctypes.data, self.host["bt"].ctypes.data, None,
            self.out.data_ptr())
        self.ws_bytes = self.lib.pa_paged_attention_workspace_bytes(C.byref(self.node),
                                                                    C.byref(self.io))
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream().cuda_stream

    def __call__(self):
        self.capi.check(self.lib.pa_paged_attention(C.byref(self.node), C.byref(self.io),
                                                    self.ws.data_ptr(), self.ws_bytes,
                                                    self.stream))


def latent_main(args, torch):
    """--latent H: a variant line (not the driver's default line).  value = latent-row bytes read
    per step (sum ctx x 576 x 2, each row once for all heads) / step time."""
    step = LatentStep(torch, args.seed, args.latent)
    kv_bytes = float(step.ctx.sum()) * 576 * 2
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_w = time.perf_counter()
    while (time.perf_counter() - t_w) * 1e3 < args.warmup_ms:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": f"LATENT (MLA 576/512) paged decode GB/s (latent-row bytes), config 3 "
                  f"contexts, {args.latent} query heads",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "us_per_step": round(ms * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 latent rows and queries; random block tables)",
        "config": {"workload": "pa_paged_attention, kv_cache_layout LATENT: RoPE + append of one "
                               "latent row per sequence + attention of every head over the rows",
                   "batch": 64, "num_heads": args.latent, "kv_heads": 1, "head_dim": 576,
                   "v_head_size": 512, "block_size": 16, "ctx": "U[512,8192]",
                   "sum_ctx": int(step.ctx.sum()), "latent_bytes_per_step": int(kv_bytes)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole call (append + latent_kernel + split_reduce_kernel)"},
        "cpu_baseline": None}), flush=True)


def gqa_main(args, torch, ep):
    """--gqa: the config 3 decode batch through GroupQueryAttention (a variant line, not the
    driver's default line).  value = KV bytes of the codes or rows read per step / step time."""
    w = build_workload(torch, ep, args.seed, 128, "bf16")
    step = GqaStep(torch, w, args.cache_dtype, args.bias)
    elem = {"bf16": 2, "int8": 1, "int4": 0.5}[args.cache_dtype]
    kv_bytes = float(w["ctx"].sum()) * w["KV"] * w["d"] * 2 * elem
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_w = time.perf_counter()
    while (time.perf_counter() - t_w) * 1e3 < args.warmup_ms:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    what = f"{args.cache_dtype} presents" + (", attention_bias [64,1,1,total]" if args.bias else "")
    print(json.dumps({
        "metric": f"GroupQueryAttention decode GB/s (KV bytes), config 3 batch, {what}",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "us_per_step": round(ms * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if args.cache_dtype == "bf16" else f"bf16 x {args.cache_dtype}",
        "data": "synthetic (seeded N(0,1) bf16 rows or uniform codes; N(0,1) q/k/v)",
        "config": {"workload": "pa_group_query_attention: RoPE + present append + streaming "
                               "decode over contiguous presents, one token per sequence",
                   "batch": w["B"], "num_heads": w["H"], "kv_heads": w["KV"], "head_dim": w["d"],
                   "present_capacity": 8192, "ctx": "U[512,8192]",
                   "sum_ctx": int(w["ctx"].sum()), "kv_bytes_per_step": int(kv_bytes),
                   "cache_dtype": args.cache_dtype, "attention_bias": bool(args.bias)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole GroupQueryAttention call (append + decode + merge)"},
        "cpu_baseline": None}), flush=True)


class Step:
    """Pre-built C-ABI argument blocks so the timed loop is one ctypes call per step.

    step()      : pa_paged_attention -- the operator entry (RoPE + append + attention), with
                  the int32 metadata validated on the host every step as the reference does.
    append() /
    attention() : the same work through the kernel-level entries, used to time the attention
                  launch on its own for the roofline.
    """

    def __init__(self, torch, ep, w, chunk, kind=1):
        import numpy as np
        from onnxruntime_ep_mlx_amd import _capi as capi
        from onnxruntime_ep_mlx_amd.ops import attn_desc, batch_desc, cache_desc
        self.lib = capi.load()
        self.capi = capi
        self.w = w
        self.act = capi.PA_DTYPE_BFLOAT16
        self.stream = torch.cuda.current_stream().cuda_stream
        self.out = torch.empty_like(w["q"])
        rotary = w["cos"] is not None
        ptr = lambda t: None if t is None else t.data_ptr()
        # operator-level blocks
        self.host = {n: np.ascontiguousarray(w[n].cpu().numpy()) for n in ("cum", "past", "bt")}
        self.node = capi.PaNode(w["H"], w["KV"], 0.0, 0.0, -1, int(rotary), 0, 0, 1, 1e-6)
        self.io = capi.PaIO(
            self.act, w["T"], w["H"] * w["d"], w["q"].data_ptr(), w["k"].data_ptr(),
            w["v"].data_ptr(), cache_desc(w["kc"], w["vc"], w["ks"], w["vs"], head_dim=w["d"],
                                          k_quant_type=w.get("quant", "NONE"),
                                          v_quant_type=w.get("quant", "NONE")),
            w["cum"].data_ptr(), w["past"].data_ptr(), w["bt"].data_ptr(), w["B"],
            w["bt"].shape[1], ptr(w["cos"]), ptr(w["sin"]), w["cos"].shape[0] if rotary else 0,
            w["cos"].shape[1] if rotary else 0, None, None, None, None,
            self.host["cum"].ctypes.data, self.host["past"].ctypes.data,
            self.host["bt"].ctypes.data, None, self.out.data_ptr())
        self.op_ws_bytes = self.lib.pa_paged_attention_workspace_bytes(C.byref(self.node),
                                                                       C.byref(self.io))
        self.op_ws = torch.empty(max(self.op_ws_bytes, 1), dtype=torch.uint8, device="cuda")
        # kernel-level blocks
        self.cache = cache_desc(w["kc"], w["vc"], w["ks"], w["vs"], head_dim=w["d"],
                                k_quant_type=w.get("quant", "NONE"),
                                v_quant_type=w.get("quant", "NONE"))
        self.batch = batch_desc(w["cum"], w["past"], w["bt"], w["T"], None, w["mq"],
                                capi.PA_BATCH_NEW_ROWS_IN_CACHE)
        self.attn = attn_desc(w["H"])
        self.rotary = rotary
        self.q_out = torch.empty_like(w["q"]) if rotary else w["q"]
        self.k_out = torch.empty_like(w["k"]) if rotary else w["k"]
        self.chunk = chunk
        self.kind = kind
        self.ws_bytes = self.lib.pa_attention_workspace_bytes_ex(
            C.byref(self.cache), C.byref(self.batch), C.byref(self.attn), self.act, kind, chunk)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device="cuda")

    def __call__(self):
        rc = self.lib.pa_paged_attention(C.byref(self.node), C.byref(self.io),
                                         self.op_ws.data_ptr(), self.op_ws_bytes, self.stream)
        self.capi.check(rc)

    def append(self):
        w = self.w
        rot = self.rotary
        rc = self.lib.pa_rotary_append(
            C.byref(self.cache), C.byref(self.batch), w["H"], self.act, w["q"].data_ptr(),
            w["k"].data_ptr(), w["v"].data_ptr(), self.q_out.data_ptr() if rot else None,
            self.k_out.data_ptr() if rot else None, w["cos"].data_ptr() if rot else None,
            w["sin"].data_ptr() if rot else None, w["cos"].shape[0] if rot else 0,
            w["cos"].shape[1] if rot else 0, 0, 0, None, None, 0.0, self.stream)
        self.capi.check(rc)

    def attention(self):
        w = self.w
        rc = self.lib.pa_attention_ex(
            C.byref(self.cache), C.byref(self.batch), C.byref(self.attn), self.act,
            self.q_out.data_ptr(), self.k_out.data_ptr(), w["v"].data_ptr(),
            self.out.data_ptr(), self.ws.data_ptr(), self.ws_bytes, self.kind, self.chunk,
            self.stream)
        self.capi.check(rc)


def cpu_info():
    """Threads the CPU path may use and the host's CPU model.  The threads are the CPUs this
    process may run on (its affinity mask), capped by OMP_NUM_THREADS when the job sets it: a GPU
    box grants each GPU's job a share of the host's cores and states it that way."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(allowed, int(env)) if env.isdigit() and int(env) > 0 else allowed
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(threads, 1), model, os.cpu_count() or 1


def _timed(fn, seconds, max_reps=10000):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            return el / reps, reps, el


def _host_pages(torch, w, sample):
    """The sampled sequences' pages copied to the host as a small paged pool (their blocks in
    block-table order) plus each sequence's block ids in it: the input of the CPU gather."""
    import numpy as np
    bs = w["bs"]
    ids, local, base = [], [], 0
    for b in sample:
        n = (int(w["ctx"][b]) + bs - 1) // bs
        ids.append(w["bt_np"][b, :n].astype(np.int64))
        local.append(np.arange(base, base + n))
        base += n
    sel = torch.from_numpy(np.concatenate(ids)).cuda()
    raw = lambda t: t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16)
    kp = raw(w["kc"]).index_select(0, sel).cpu().numpy()
    vp = raw(w["vc"]).index_select(0, sel).cpu().numpy()
    sc = None
    if w["ks"] is not None:
        sc = (w["ks"].index_select(0, sel).cpu().numpy(), w["vs"].index_select(0, sel).cpu().numpy())
    return kp, vp, sc, local


def _gather(w, kp, vp, sc, local, sample):
    """CPU page -> contiguous gather of the sampled sequences ([sum ctx, KV, d] K and V); fp8
    pages are dequantised to fp32 (code * block scale) on the way, as a CPU GQA needs."""
    import numpy as np
    bs, KV, d = w["bs"], w["KV"], w["d"]
    ks, vs, offs, off = [], [], [], 0
    for b, blk in zip(sample, local):
        c = int(w["ctx"][b])
        kk = kp[blk].reshape(-1, KV, d)[:c]
        vv = vp[blk].reshape(-1, KV, d)[:c]
        if sc is not None:
            import _oracle as orc
            kscale = np.repeat(sc[0][blk], bs, axis=0)[:c, :, None]
            vscale = np.repeat(sc[1][blk], bs, axis=0)[:c, :, None]
            kk = orc.decode(np.ascontiguousarray(kk), orc.E4M3) * kscale
            vv = orc.decode(np.ascontiguousarray(vv), orc.E4M3) * vscale
        ks.append(kk)
        vs.append(vv)
        offs.append(off)
        off += c
    return (np.ascontiguousarray(np.concatenate(ks)), np.ascontiguousarray(np.concatenate(vs)),
            offs)


def cpu_baseline(torch, w, step, n_seq, seconds, config="c3"):
    """The CPU path (the oracle directory's threaded contiguous-KV GQA, ORT CPU semantics, fp32
    accumulation) on a bounded sample of the same workload, on this host's cores.  The page ->
    contiguous gather it needs is timed on its own and reported beside it, not inside value."""
    import numpy as np
    sys.path.insert(0, os.fspath(ROOT / "tests"))
    import _oracle as orc
    threads, model, host_cpus = cpu_info()
    B, H, KV, d = w["B"], w["H"], w["KV"], w["d"]
    sample = list(range(min(n_seq, B)))
    kp, vp, sc, local = _host_pages(torch, w, sample)
    k, v, offs = _gather(w, kp, vp, sc, local, sample)
    gather_s, _, _ = _timed(lambda: _gather(w, kp, vp, sc, local, sample), min(seconds, 3.0), 50)
    dt = orc.F32 if sc is not None else orc.BF16
    if dt == orc.F32:
        k, v = k.astype(np.float32), v.astype(np.float32)
    scale = float(1.0 / np.sqrt(np.float32(d)))
    ctxs = [int(w["ctx"][b]) for b in sample]
    if config == "c4":
        mq = w["mq"]
        q = step.q_out[: len(sample) * mq].view(torch.int16).cpu().numpy().view(np.uint16)
        q = np.ascontiguousarray(q)
        past = [c - mq for c in ctxs]
        starts = [i * mq for i in range(len(sample))]
        run = lambda: orc.cpu_gqa_prefill(dt, q, k, v, offs, starts, [mq] * len(sample), past,
                                          H, KV, d, scale, threads)
    else:
        q = step.q_out[sample].view(torch.int16).cpu().numpy().view(np.uint16).reshape(
            len(sample), H, d).copy()
        if dt == orc.F32:
            q = orc.decode(q, orc.BF16)
        run = lambda: orc.cpu_gqa_decode(dt, q, k, v, offs, ctxs, H, KV, d, scale, threads)
    per, reps, el = _timed(run, seconds)
    what = {"c3": "contiguous bf16 KV", "c4": "contiguous bf16 KV, causal 512-row chunks",
            "c5": "contiguous KV dequantised from e4m3 pages to fp32"}[config]
    info = {"cores": threads, "kind": "port", "cpu_model": model, "host_cpus": host_cpus,
            "gather_ms_sample": round(gather_s * 1e3, 2)}
    desc = (f"first {len(sample)} of {B} sequences (sum ctx {sum(ctxs)}), {reps} reps in "
            f"{el:.1f} s, {what} gathered from the pages (gather timed apart: "
            f"{gather_s * 1e3:.1f} ms for the sample), fp32 accumulation, {threads} threads")
    if config == "c4":
        fl = sum(4.0 * H * d * (w["mq"] * (c - w["mq"]) + w["mq"] * (w["mq"] + 1) / 2)
                 for c in ctxs)
        return {"value": round(fl / per / 1e12, 4), "unit": "TFLOP/s", **info,
                "ms_per_step_full_batch": round(per * w["flops"] / fl * 1e3, 1),
                "sample": desc}
    elem = 1 if config == "c5" else 2
    sample_bytes = float(sum(ctxs)) * KV * d * 2 * elem
    full_bytes = float(w["ctx"].sum()) * KV * d * 2 * elem
    return {"value": round(sample_bytes / per / 1e9, 3),
            "unit": "GB/s (fp8 KV bytes)" if config == "c5" else "GB/s (KV bytes)", **info,
            "us_per_step_full_batch": round(per * full_bytes / sample_bytes * 1e6, 1),
            "gather_us_full_batch": round(gather_s * full_bytes / sample_bytes * 1e6, 1),
            "sample": desc}


MFMA_BF16_PEAK_TFLOPS = 2500.0


def other_config_line(args, w, ms_step, attn_ms, kv_bytes, cpu=None):
    """JSON line of BASELINE.json configs 4 and 5 (not the driver's default line)."""
    common = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "warmup_extra_steps": args.warmup_extra, "ms_per_step": round(ms_step, 4), "us_per_step": round(ms_step * 1e3, 1),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "cpu_baseline": cpu}
    if args.config == "c4":
        tf_step = w["flops"] / (ms_step * 1e-3) / 1e12
        tf_attn = w["flops"] / (attn_ms * 1e-3) / 1e12
        return {
            "metric": "chunked-prefill paged attention TFLOP/s (causal QK+PV FLOPs)",
            "value": round(tf_step, 2), "unit": "TFLOP/s", **common, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) bf16 pages and q/k/v; random block tables)",
            "config": {
                "workload": "chunked prefill, Qwen2.5-7B shape (BASELINE.json config 4): append "
                            "of 8 x 512 new tokens + causal paged attention over past "
                            "U[0,4096]",
                "batch": w["B"], "tokens": w["T"], "num_heads": w["H"], "kv_heads": w["KV"],
                "head_dim": w["d"], "block_size": w["bs"], "pasts": [int(x) for x in
                                                                     w["ctx"] - w["mq"]],
                "flops_per_step": w["flops"], "kv_bytes_read": int(kv_bytes),
                "entry": "pa_paged_attention (host-validated metadata)"},
            "roofline": {
                "bound": "mfma", "achieved": round(tf_attn, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tf_attn / MFMA_BF16_PEAK_TFLOPS, 4),
                "traffic": (load_traffic("prefill_c4_traffic.json")
                            if w["d"] == 128 and w.get("cache", "bf16") == "bf16" else None),
                "kernel": "pa_attention (planned prefill over operand images: plan + image "
                          "launch, prefill_mx_kernel, merge of split items)",
                "us_per_launch": round(attn_ms * 1e3, 1)},
        }
    gbs = kv_bytes / (ms_step * 1e-3) / 1e9
    attn_gbs = kv_bytes / (attn_ms * 1e-3) / 1e9
    return {
        "metric": "fp8 paged GQA decode µs/step + achieved HBM GB/s (fp8 KV bytes), B=16, "
                  "ctx 32768",
        "value": round(gbs, 2), "unit": "GB/s", **common, "dtype": "bf16 x e4m3",
        "tokens_per_s": round(w["B"] / (ms_step * 1e-3), 1),
        "data": "synthetic (seeded N(0,1) quantised to e4m3 with amax/448 block scales)",
        "config": {
            "workload": "long-context fp8 paged decode (BASELINE.json config 5): append + "
                        "split-K paged attention over e4m3 pages",
            "batch": w["B"], "num_heads": w["H"], "kv_heads": w["KV"], "head_dim": w["d"],
            "block_size": w["bs"], "ctx": 32768, "kv_bytes_per_step": int(kv_bytes),
            "entry": "pa_paged_attention (host-validated metadata)"},
        "roofline": {
            "bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic("decode_fp8_c5_traffic.json"),
            "kernel": "pa_attention (decode_balanced_kernel fp8 + balanced_merge_kernel)",
            "us_per_launch": round(attn_ms * 1e3, 1)},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(decode shards by sequence or kv-head with no exchange between GPUs)",
              file=sys.stderr)
        sys.exit(2)
    if args.config == "c5" and args.cache_dtype != "bf16":
        print("bench.py: --cache-dtype applies to c3 and c4 (c5 is the e4m3 config)",
              file=sys.stderr)
        sys.exit(2)
    if args.config == "c3" and args.cache_dtype == "fp8":
        print("bench.py: the fp8 decode batch is config 5 (--config c5)", file=sys.stderr)
        sys.exit(2)
    if args.gqa and (args.config != "c3" or args.cache_dtype == "fp8" or args.head_dim != 128):
        print("bench.py: --gqa takes the config 3 batch at head 128 with bf16 / int8 / int4 "
              "presents", file=sys.stderr)
        sys.exit(2)
    if args.latent and (args.config != "c3" or args.gqa or args.latent not in (16, 128)):
        print("bench.py: --latent takes 16 or 128 heads over the config 3 contexts",
              file=sys.stderr)
        sys.exit(2)
    if args.bias and not args.gqa:
        print("bench.py: --bias applies to --gqa", file=sys.stderr)
        sys.exit(2)
    import torch
    import onnxruntime_ep_mlx_amd as ep
    torch.cuda.set_device(0)
    if args.gqa:
        gqa_main(args, torch, ep)
        return
    if args.latent:
        latent_main(args, torch)
        return
    if args.config == "c3":
        w = build_workload(torch, ep, args.seed, args.head_dim, args.cache_dtype)
        step = Step(torch, ep, w, args.chunk, kind=1 if args.cache_dtype == "bf16" else 0)
    elif args.config == "c4":
        w = build_prefill_workload(torch, d=args.head_dim, cache=args.cache_dtype)
        step = Step(torch, ep, w, args.chunk, kind=0)
    else:
        w = build_fp8_workload(torch)
        step = Step(torch, ep, w, args.chunk, kind=0)
    # bytes per K or V element: fp8 / int8 pages 1, int4 pages 1/2, bf16 2
    kv_elem = {"int8": 1, "int4": 0.5}.get(w.get("cache"), 1 if w["ks"] is not None else 2)
    kv_bytes = float(w["ctx"].sum()) * w["KV"] * w["d"] * 2 * kv_elem

    if args.calibrate_copy:
        # Plain copies of exactly 1 GiB (read 1 GiB, write 1 GiB): the reference dispatches
        # for scaling FETCH_SIZE / WRITE_SIZE counter readings to bytes.
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    extra, t_w = 0, time.perf_counter()
    while (time.perf_counter() - t_w) * 1e3 < args.warmup_ms:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        extra += 10
    args.warmup_extra = extra

    # whole-step timing
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps

    # dominant launch: the attention call on the same stream, timed per launch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for a, b in evs:
        step.append()
        a.record()
        step.attention()
        b.record()
    torch.cuda.synchronize()
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    attn_gbs = kv_bytes / (attn_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu_baseline and w.get("cache", "bf16") == "bf16":
        n_seq = {"c3": args.cpu_sample, "c4": 1, "c5": 1}[args.config]
        cpu = cpu_baseline(torch, w, step, n_seq, args.cpu_seconds, args.config)

    if args.config != "c3":
        line = other_config_line(args, w, ms_step, attn_ms, kv_bytes, cpu)
        cache = w.get("cache", "bf16")
        if w["d"] != 128 or cache != "bf16":  # not config 4 itself: say so in the line
            what = f"head_dim {w['d']}" + ("" if cache == "bf16" else f", {cache} pages")
            line["metric"] += f" ({what} variant of config 4)"
            line["config"]["cache_dtype"] = cache
            if cache in ("int8", "int4"):
                line["dtype"] = f"bf16 x {cache} (fp16 code images, fp16 MFMA)"
                line["data"] = ("synthetic (seeded uniform integer codes, per-channel scales; "
                                "N(0,1) bf16 q/k/v; random block tables)")
            elif cache == "fp8":
                line["dtype"] = "bf16 x e4m3 (fp16 images of the dequantised rows, fp16 MFMA)"
                line["data"] = ("synthetic (seeded N(0,1) quantised to e4m3 with amax/448 "
                                "block scales; N(0,1) bf16 q/k/v; random block tables)")
        print(json.dumps(line), flush=True)
        return

    gbs = kv_bytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": "paged GQA decode µs/step + achieved HBM GB/s (KV bytes) at B=64, ctx≤8k",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_extra_steps": args.warmup_extra,
        "ms_per_step": round(ms_step, 4),
        "us_per_step": round(ms_step * 1e3, 1),
        "tokens_per_s": round(w["B"] / (ms_step * 1e-3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 pages, q/k/v; random block tables)",
        "config": {
            "workload": "paged GQA decode, Llama-3-8B shape (BASELINE.json config 3): RoPE + KV "
                        "append + split-K paged attention per step",
            "batch": w["B"], "num_heads": w["H"], "kv_heads": w["KV"], "head_dim": w["d"],
            "block_size": w["bs"], "pool_blocks": w["nb"], "ctx": "U[512,8192]",
            "sum_ctx": int(w["ctx"].sum()), "kv_bytes_per_step": int(kv_bytes),
            "rotary_theta": 500000.0, "entry": "pa_paged_attention (host-validated metadata)",
        },
        "roofline": {
            "bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": load_traffic() if (w["d"] == 128 and w["cache"] == "bf16") else None,
            "kernel": "pa_attention (decode_balanced_kernel + balanced_merge_kernel)",
            "us_per_launch": round(attn_ms * 1e3, 1),
        },
        "cpu_baseline": cpu,
    }
    if w["d"] != 128 or w["cache"] != "bf16":  # not config 3 itself: say so in the line
        what = f"head_dim {w['d']}" + ("" if w["cache"] == "bf16" else f", {w['cache']} pages")
        line["metric"] += f" ({what} variant of config 3)"
        line["config"]["workload"] = (f"config 3 decode batch at {what}: RoPE + KV append + "
                                      "split-K paged attention per step")
        line["config"]["cache_dtype"] = w["cache"]
        if w["cache"] != "bf16":
            if w["d"] not in (64, 128):  # byte-coded pages stream at heads 64 / 128 only
                line["roofline"]["kernel"] = ("pa_attention (attn_generic_kernel + "
                                              "split_reduce_kernel)")
            line["dtype"] = f"bf16 x {w['cache']}"
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
