// pa_tiles.hpp — the 16x16x32 MFMA tile step shared by the paged decode and prefill kernels:
// per-lane operand layouts, one 32-key step of online-softmax attention for a 16-row group,
// and the row set-up / epilogue (final rows or split-K partials).
//
// Scores are computed transposed, S^T = K_tile . Q^T (A = 16 keys x 32 dims straight from the
// page rows, B = Q^T held in registers), so lane l ends with S[key 4*(l/16)+i][row l%16] of each
// 16-key tile -- exactly the A-operand layout that P needs for O += P . V.  The value operand
// (8 keys x 1 dim per lane) is assembled from 8 value-row slices; output column n of N-tile j
// is head dim DL*n + j.  P is split into hi + lo 16-bit parts (two MFMAs), so the PV product
// keeps ~16 mantissa bits.
#pragma once

#include "pa_device.hpp"

namespace pa {
namespace {

// One lane's slice of one value row: DL = D/16 elements (D/32 words); 64 and 128 as vectors.
template <int D>
struct VRow {
  uint32_t w[D / 32];
  __device__ uint32_t word(int i) const { return w[i]; }
};
template <>
struct VRow<64> {
  u32x2 w;
  __device__ uint32_t word(int i) const { return w[i]; }
};
template <>
struct VRow<128> {
  u32x4 w;
  __device__ uint32_t word(int i) const { return w[i]; }
};

template <int D>
__device__ __forceinline__ VRow<D> ld_vrow(const char* ptr);
template <>
__device__ __forceinline__ VRow<64> ld_vrow<64>(const char* ptr) {
  return VRow<64>{*reinterpret_cast<const u32x2*>(ptr)};
}
template <>
__device__ __forceinline__ VRow<128> ld_vrow<128>(const char* ptr) {
  return VRow<128>{*reinterpret_cast<const u32x4*>(ptr)};
}

__device__ __forceinline__ u32x4 ld16(const char* ptr) {
  return *reinterpret_cast<const u32x4*>(ptr);
}

// Streaming (non-temporal, `nt`) loads for key/value page rows that one pass reads once.  On
// gfx950 a contiguous 2 GiB read runs 7-10% faster with nt loads than with plain ones (e.g.
// 6.35 vs 5.82 TB/s at 8192 workgroups), since the streamed lines do not displace reused ones.
__device__ __forceinline__ u32x4 ld16s(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
}
__device__ __forceinline__ u32x2 ld8s(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(ptr));
}
__device__ __forceinline__ uint32_t ld4s(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(ptr));
}
template <int D>
__device__ __forceinline__ VRow<D> ld_vrow_s(const char* ptr) {
  if constexpr (D == 64) {
    return VRow<64>{ld8s(ptr)};
  } else if constexpr (D == 128) {
    return VRow<128>{ld16s(ptr)};
  } else if constexpr (D % 128 == 0) {  // 16-byte pieces (the slice is 16-byte aligned)
    VRow<D> r;
#pragma unroll
    for (int i = 0; i < D / 128; ++i) {
      const u32x4 v = ld16s(ptr + 16 * i);
#pragma unroll
      for (int k = 0; k < 4; ++k) r.w[4 * i + k] = v[k];
    }
    return r;
  } else if constexpr (D == 96) {  // 12-byte slices, 4-byte aligned: one dwordx3 load
    VRow<D> r;
    __builtin_memcpy(r.w, __builtin_assume_aligned(ptr, 4), 12);
    return r;
  } else {  // 4-byte words
    VRow<D> r;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) r.w[i] = ld4s(ptr + 4 * i);
    return r;
  }
}

template <int D>
struct Step {
  u32x4 k[2][D / 32];  // tile A / tile B key rows, 8 dims per k-step
  VRow<D> v[8];        // value rows: keys 4G+e of tile A (e<4) and of tile B (e>=4)
};

// Wave-uniform description of the (sequence, kv-head, chunk) being processed.
struct WaveInfo {
  const char* kc;  // key cache (bytes)
  const char* vc;
  const char* kn;  // new key rows (bytes)
  const char* vn;
  int b, kh, s0, pastb, total, cache_limit;
  int bs, bs_shift;  // block size, log2 if a power of two else -1
  int max_blocks, num_tokens;
  int64_t num_blocks;
  int64_t rowb;      // bytes between consecutive cache rows (kv_heads * D * 2; contiguous: D * 2)
  int first_bi;      // first block-table index of the chunk
  const int32_t* bt; // this sequence's block-table row
  int64_t hoff;      // byte offset of the kv-head's slice in a row (contiguous caches: 0)
  // Contiguous [batch, kv_heads, cap, D] caches (GroupQueryAttention present): row of key 0 of
  // this (sequence, kv-head), and cap; lin_row0 < 0 for pages.
  int64_t lin_row0;
  int lin_cap;
};

__device__ __forceinline__ int div_bs(int x, const WaveInfo& w) {
  return w.bs_shift >= 0 ? (x >> w.bs_shift) : x / w.bs;
}
__device__ __forceinline__ int mod_bs(int x, const WaveInfo& w) {
  return w.bs_shift >= 0 ? (x & (w.bs - 1)) : x % w.bs;
}

// Byte offset of key/value row `pos` for this lane (any block size), choosing the cache page
// (positions < cache_limit) or the new rows.  Positions past the end clamp to the last real
// row; block ids are clamped into the pool, so malformed metadata cannot fault.
__device__ __forceinline__ const char* row_ptr(const WaveInfo& w, int pos, bool value, int D) {
  if (pos >= w.total) pos = w.total - 1;
  if (w.lin_row0 >= 0)  // contiguous cache holding every key (total <= cap)
    return (value ? w.vc : w.kc) + (w.lin_row0 + max(pos, 0)) * w.rowb;
  if (pos < w.cache_limit) {
    const int bi = min(div_bs(pos, w), w.max_blocks - 1);
    int64_t blk = w.bt[bi];
    blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
    return (value ? w.vc : w.kc) + (blk * w.bs + mod_bs(pos, w)) * w.rowb + w.hoff;
  }
  int64_t tok = min(max((int64_t)w.s0 + (pos - w.pastb), (int64_t)0), (int64_t)w.num_tokens - 1);
  return (value ? w.vn : w.kn) + tok * w.rowb + w.hoff;
}

// Block-table window: lane i holds the page id of block first + i.
struct PageWindow {
  int first;
  int ids;
};

__device__ __forceinline__ void window_at(PageWindow& pw, const WaveInfo& w, int bi, int lane) {
  pw.first = bi;
  pw.ids = w.bt[min(bi + lane, w.max_blocks - 1)];
}

// Byte offset (from the cache base) of the first row of the 16-key tile starting at key t.
__device__ __forceinline__ int64_t tile_base(const WaveInfo& w, PageWindow& pw, int t, int lane,
                                             int D) {
  if (w.lin_row0 >= 0) return (w.lin_row0 + t) * w.rowb;  // contiguous cache
  const int bi = min(div_bs(t, w), w.max_blocks - 1);
  if (bi < pw.first || bi >= pw.first + 64) window_at(pw, w, bi, lane);
  int64_t blk = __builtin_amdgcn_readlane(pw.ids, bi - pw.first);
  blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
  return (blk * w.bs + mod_bs(t, w)) * w.rowb + w.hoff;
}

// Regroup 8 value rows (lane holds DL dims of each) into the MFMA B-operand of N-tile j:
// 8 keys x head dim DL*c + j.
template <typename TT, int D>
__device__ __forceinline__ typename TT::vec8 value_operand(const Step<D>& st, int j) {
  u32x4 w;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t lo = st.v[2 * m].word(j >> 1), hi = st.v[2 * m + 1].word(j >> 1);
    // One byte permute: low halves (even j) or high halves (odd j) of the two rows.
    w[m] = __builtin_amdgcn_perm(hi, lo, (j & 1) ? 0x07060302u : 0x05040100u);
  }
  return __builtin_bit_cast(typename TT::vec8, w);
}

// Zero this lane's value rows of a step that lie at or past `total` (rows re-read past the
// sequence end take no part even if their bytes are not finite).
template <int D>
__device__ __forceinline__ void clear_tail_rows(Step<D>& st, int t0, int total, int G) {
  if (t0 + 32 <= total) return;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (t0 + 16 * (e >> 2) + 4 * G + (e & 3) >= total) st.v[e] = VRow<D>{};
}

// Row state of one 16-row group.
template <typename TT, int D>
struct RowState {
  typename TT::vec8 qv[D / 32];
  f32x4 o[D / 16];
  float m_run;   // running max of row c (log2 units); identical across the 4 lane groups
  float l_part;  // this lane's share of the row-c denominator
  int vis_lo, vis_hi;
};

// SC: fp8 pages, whose key codes score as ks * (q . code) and whose value codes weigh in as
// vs * code; ks/vs are the page scales of tile A (keys t0..t0+15) and tile B.
//
// The key operand `k` holds the two 16-key tiles (A: keys t0..t0+15, B: t0+16..t0+31), 16 bytes
// per lane and k-step; `vop(j)` returns the value operand of N-tile j (8 keys x head dim
// DL*c + j, keys in the order the scores come out: 4G+i of tile A, then of tile B).
//
// MASK = false: the caller knows every key of the step is visible to every valid row of the
// group (rows past the end of the sequence have zero queries and are never stored), so the
// per-score position tests are skipped.
//
// The step is split into three pieces -- scores, the (rare) lazy rescale, probabilities and
// the PV product -- so that attend_groups can run the middle piece once for several row
// groups and leave the exponentials of one group and the PV MFMAs of another in one basic
// block for the scheduler to interleave.

// Scores of the step in log2 units (masked to -inf where not visible); returns this lane's max.
//
// `kop(tile, s)` returns the key operand of k-step s of tile 0 (keys t0..t0+15) or 1.
// BIAS: bx[e] (an additive bias in log2 units for score e of the lane: key t0 + 16 (e / 4) +
// 4 G + e % 4) is added after the scale and softcap, before the position masks.
template <typename TT, int D, bool CAP, bool SC, bool MASK, bool FOLD = false, bool KOFF = false,
          bool BIAS = false, typename KeyOp>
__device__ __forceinline__ float step_scores(const RowState<TT, D>& rs, KeyOp kop, int t0,
                                             int end, int G, float scale_log2, float scale,
                                             float cap, float ksA, float ksB, float (&x)[8],
                                             bool masked = true, float koff = 0.0f,
                                             const float* bx = nullptr) {
  constexpr int KS = D / 32;
  f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    sa = TT::mfma(kop(0, s), rs.qv[s], sa);
    sb = TT::mfma(kop(1, s), rs.qv[s], sb);
  }
  // KOFF: every score of the row carries koff (key operands offset by a constant): removed in
  // the FMA that applies the tile's factor.
  static_assert(!KOFF || SC, "offset keys come with page factors");
  if constexpr (SC && CAP) {
    if constexpr (KOFF) {
      const float ka = koff * ksA, kb = koff * ksB;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sa[e] = __builtin_fmaf(sa[e], ksA, -ka);
        sb[e] = __builtin_fmaf(sb[e], ksB, -kb);
      }
    } else {
      sa *= ksA;
      sb *= ksB;
    }
  }
  // Page scales (SC) fold into the log2-domain score scale: one product per tile.  FOLD (no
  // softcap, no page scales, scale_log2 >= 0): x keeps the raw products, the scale multiplies
  // only their maximum here and enters each exponent through one FMA in step_probs.
  static_assert(!FOLD || (!CAP && !SC && !BIAS), "FOLD takes plain scaled scores");
  const float xa = SC ? ksA * scale_log2 : scale_log2, xb = SC ? ksB * scale_log2 : scale_log2;
  const float kxa = KOFF ? koff * xa : 0.0f, kxb = KOFF ? koff * xb : 0.0f;
  const float cap_k = CAP ? scale / cap : 0.0f, cap_l2 = cap * kLog2e;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sv = (e < 4) ? sa[e & 3] : sb[e & 3];
    if constexpr (CAP)
      x[e] = softcap_log2(sv, cap_k, cap_l2);
    else if constexpr (FOLD)
      x[e] = sv;
    else if constexpr (KOFF)
      x[e] = __builtin_fmaf(sv, (e < 4) ? xa : xb, -((e < 4) ? kxa : kxb));
    else
      x[e] = sv * ((e < 4) ? xa : xb);
    if constexpr (BIAS) x[e] += bx[e];
  }
  // `masked` (wave-uniform) is false when the caller knows every key of the step is visible to
  // every valid row: one scalar branch instead of the per-score position tests.
  // Positions [vis_lo, min(end, vis_hi)) of the row: one unsigned range test per score, the
  // differences taken modulo 2^32 (the span is below 3 * 2^30, a position below vis_lo lands
  // above it); three compares per score kept their masks in scalar registers.
  if constexpr (MASK) {
    if (masked) {
      const int hi_pos = min(end, rs.vis_hi);
      const unsigned span = hi_pos > rs.vis_lo ? (unsigned)hi_pos - (unsigned)rs.vis_lo : 0u;
      const unsigned rel = (unsigned)(t0 + 4 * G) - (unsigned)rs.vis_lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned off = 16 * (e >> 2) + (e & 3);
        x[e] = (rel + off < span) ? x[e] : kNegInf;
      }
    }
  }
  float lmax = kNegInf;
#pragma unroll
  for (int e = 0; e < 8; ++e) lmax = fmaxf(lmax, x[e]);
  if constexpr (FOLD) lmax *= scale_log2;
  return lmax;
}

// Lazy rescale: the running max only moves when a score exceeds it by more than 2^8.
template <typename TT, int D>
__device__ __forceinline__ bool needs_rescale(const RowState<TT, D>& rs, float lmax) {
  return lmax > rs.m_run + 8.0f;
}

template <typename TT, int D>
__device__ __forceinline__ void rescale_rows(RowState<TT, D>& rs, float lmax, int G) {
  constexpr int DL = D / 16;
  float rmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
  rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
  const float m_new = fmaxf(rs.m_run, rmax);
  const float alpha = (m_new == kNegInf) ? 1.0f : exp2f(rs.m_run - m_new);
  rs.l_part *= alpha;
  rs.m_run = m_new;
  float ar[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * G + i, 64);
#pragma unroll
  for (int j = 0; j < DL; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) rs.o[j][i] *= ar[i];
}

// Probabilities of the step as the PV A operand, split into hi + lo 16-bit parts.
//
// They use the hardware base-2 exponential (v_exp_f32) without the denormal-range rescaling of
// exp2f: arguments are <= 8 (lazy max) and a probability below 2^-126 of the row maximum adds
// nothing to an fp32 sum that holds the maximum's own 1.
template <typename TT, int D, bool FOLD, bool SC>
__device__ __forceinline__ void step_probs(RowState<TT, D>& rs, const float (&x)[8],
                                           float scale_log2, float vsA, float vsB,
                                           typename TT::vec8& phi, typename TT::vec8& plo8) {
  // FOLD: x holds the raw scores of step_scores<..., FOLD = true>
  const float msafe = (rs.m_run == kNegInf) ? 0.0f : rs.m_run;
  float pv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pv[e] = __builtin_amdgcn_exp2f(FOLD ? __builtin_fmaf(x[e], scale_log2, -msafe) : x[e] - msafe);
    rs.l_part += pv[e];
  }
  if constexpr (SC) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] *= (e < 4) ? vsA : vsB;  // l_part keeps the unscaled sum
  }
  TT::split8(pv, phi, plo8);
}

// SPLIT = false: P enters the P.V product once, rounded to T (fp16 keeps 11 bits; used for
// integer pages, whose value operands are exact small integers).
template <typename TT, int D, bool CAP, bool SC, bool MASK = true, bool SPLIT = true,
          bool KOFF = false, bool BIAS = false, typename KeyOp, typename ValueOp>
__device__ __forceinline__ void attend_step_ops(RowState<TT, D>& rs, KeyOp kop, ValueOp vop,
                                                int t0, int end, int G, float scale_log2,
                                                float scale, float cap, float ksA, float ksB,
                                                float vsA, float vsB, bool masked = true,
                                                float koff = 0.0f, const float* bx = nullptr) {
  using vec8 = typename TT::vec8;
  constexpr int DL = D / 16;
  float x[8];
  const float lmax = step_scores<TT, D, CAP, SC, MASK, false, KOFF, BIAS>(
      rs, kop, t0, end, G, scale_log2, scale, cap, ksA, ksB, x, masked, koff, bx);
  if (__any(needs_rescale(rs, lmax))) rescale_rows(rs, lmax, G);
  if constexpr (SPLIT) {
    vec8 phi, plo8;
    step_probs<TT, D, false, SC>(rs, x, scale_log2, vsA, vsB, phi, plo8);
#pragma unroll
    for (int j = 0; j < DL; ++j) {
      const vec8 vb = vop(j);
      rs.o[j] = TT::mfma(phi, vb, rs.o[j]);
      rs.o[j] = TT::mfma(plo8, vb, rs.o[j]);
    }
  } else {
    const float msafe = (rs.m_run == kNegInf) ? 0.0f : rs.m_run;
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv[e] = __builtin_amdgcn_exp2f(x[e] - msafe);
      rs.l_part += pv[e];
      if constexpr (SC) pv[e] *= (e < 4) ? vsA : vsB;
    }
    const vec8 pp = TT::cvt8(pv);
#pragma unroll
    for (int j = 0; j < DL; ++j) rs.o[j] = TT::mfma(pp, vop(j), rs.o[j]);
  }
}

template <typename TT, int D, bool CAP, bool SC, bool MASK = true, typename ValueOp>
__device__ __forceinline__ void attend_step(RowState<TT, D>& rs, const u32x4 (&k)[2][D / 32],
                                            ValueOp vop, int t0, int end, int G,
                                            float scale_log2, float scale, float cap, float ksA,
                                            float ksB, float vsA, float vsB, bool masked = true) {
  using vec8 = typename TT::vec8;
  attend_step_ops<TT, D, CAP, SC, MASK>(
      rs, [&](int tile, int s) { return __builtin_bit_cast(vec8, k[tile][s]); }, vop, t0, end, G,
      scale_log2, scale, cap, ksA, ksB, vsA, vsB, masked);
}

// NG row groups against the same step: all scores first, one branch for the rare rescale, then
// every group's probabilities and PV MFMAs in one block, each value operand built once.
// Without softcap or bias the scale folds into the exponents (step_scores FOLD), which takes
// scale_log2 >= 0: the caller moves the sign of a negative scale into the query operands.
// BIAS: bx[j] holds group j's additive bias of the lane's scores (log2 units, step_scores).
template <typename TT, int D, bool CAP, bool MASK, int NG, bool BIAS = false, typename KeyOp,
          typename ValueOp>
__device__ __forceinline__ void attend_groups_ops(RowState<TT, D> (&rs)[NG], KeyOp kop,
                                                  ValueOp vop, int t0, int end, int G,
                                                  float scale_log2, float scale, float cap,
                                                  const float (*bx)[8] = nullptr) {
  using vec8 = typename TT::vec8;
  constexpr int DL = D / 16;
  constexpr bool FOLD = !CAP && !BIAS;
  float x[NG][8], lmax[NG];
  bool any = false;
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    lmax[j] = step_scores<TT, D, CAP, false, MASK, FOLD, false, BIAS>(
        rs[j], kop, t0, end, G, scale_log2, scale, cap, 1.f, 1.f, x[j], true, 0.0f,
        BIAS ? bx[j] : nullptr);
    any = any || needs_rescale(rs[j], lmax[j]);
  }
  if (__any(any)) {
#pragma unroll
    for (int j = 0; j < NG; ++j)
      if (__any(needs_rescale(rs[j], lmax[j]))) rescale_rows(rs[j], lmax[j], G);
  }
  vec8 phi[NG], plo[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j)
    step_probs<TT, D, FOLD, false>(rs[j], x[j], scale_log2, 1.f, 1.f, phi[j], plo[j]);
#pragma unroll
  for (int n = 0; n < DL; ++n) {
    const vec8 vb = vop(n);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      rs[j].o[n] = TT::mfma(phi[j], vb, rs[j].o[n]);
      rs[j].o[n] = TT::mfma(plo[j], vb, rs[j].o[n]);
    }
  }
}

template <typename TT, int D, bool CAP, bool MASK, int NG, bool BIAS = false, typename ValueOp>
__device__ __forceinline__ void attend_groups(RowState<TT, D> (&rs)[NG],
                                              const u32x4 (&k)[2][D / 32], ValueOp vop, int t0,
                                              int end, int G, float scale_log2, float scale,
                                              float cap, const float (*bx)[8] = nullptr) {
  using vec8 = typename TT::vec8;
  attend_groups_ops<TT, D, CAP, MASK, NG, BIAS>(
      rs, [&](int tile, int s) { return __builtin_bit_cast(vec8, k[tile][s]); }, vop, t0, end, G,
      scale_log2, scale, cap, bx);
}

// One 32-key step held in registers as loaded (value rows regrouped here).
template <typename TT, int D, bool CAP, bool SC = false>
__device__ __forceinline__ void compute_step(RowState<TT, D>& rs, const Step<D>& st, int t0,
                                             int end, int G, float scale_log2, float scale,
                                             float cap, float ksA = 1.f, float ksB = 1.f,
                                             float vsA = 1.f, float vsB = 1.f,
                                             bool masked = true) {
  attend_step<TT, D, CAP, SC>(
      rs, st.k, [&](int j) { return value_operand<TT, D>(st, j); }, t0, end, G, scale_log2,
      scale, cap, ksA, ksB, vsA, vsB, masked);
}

// Past length of sequence b, clamped so that past + nq stays within the cache capacity.  The host
// rejects such metadata when it validates; trusted device metadata then cannot push 32-bit key
// positions past the capacity (or overflow them), and valid metadata is unchanged.
__device__ __forceinline__ int clamped_past(const AttnParams& p, int b, int nq) {
  const int cap = p.linear_cap > 0
                      ? p.linear_cap
                      : (int)min((int64_t)p.max_blocks * p.block_size, (int64_t)(INT32_MAX / 2));
  return min(max(p.past[b], 0), max(cap - nq, 0));
}

// Keys of sequence b: past + query rows, bounded by key_limit[b] when given (GroupQueryAttention
// first prompts whose sequences are shorter than the padded query rows).
__device__ __forceinline__ int seq_total(const AttnParams& p, int b, int pastb, int nq) {
  const int t = pastb + nq;
  return p.key_limit ? min(t, max(p.key_limit[b], 0)) : t;
}

// GroupQueryAttention's additive bias [bias_b, bias_h, bias_rows, bias_cols] in T for one query
// row: query qi of sequence b at head h (a size-1 batch or head dimension broadcasts); key
// position pos reads column pos + off clamped into [0, cols), the VALU kernel's rule.
struct BiasRow {
  const uint16_t* row;
  int off, last;
};
__device__ __forceinline__ BiasRow bias_row_of(const AttnParams& p, int b, int h, int qi) {
  const int64_t r = ((int64_t)(p.bias_b == 1 ? 0 : b) * p.bias_h + (p.bias_h == 1 ? 0 : h)) *
                        p.bias_rows + qi;
  BiasRow br;
  br.row = reinterpret_cast<const uint16_t*>(p.bias) + r * p.bias_cols;
  br.off = p.bias_col_off ? p.bias_col_off[b] : 0;
  br.last = p.bias_cols - 1;
  return br;
}
// The bias of this lane's 8 scores of a 32-key step (keys t0 + 16 (e / 4) + 4 G + e % 4) as
// stored (two per word), and in log2 units.
__device__ __forceinline__ void bias_load(const BiasRow& br, int t0, int G, uint32_t (&raw)[4]) {
  uint32_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    v[e] = br.row[min(max(t0 + 16 * (e >> 2) + 4 * G + (e & 3) + br.off, 0), br.last)];
#pragma unroll
  for (int i = 0; i < 4; ++i) raw[i] = v[2 * i] | (v[2 * i + 1] << 16);
}
template <typename TT>
__device__ __forceinline__ void bias_log2(const uint32_t (&raw)[4], float (&bx)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    bx[e] = TT::to_f32((typename TT::raw)(raw[e >> 1] >> (16 * (e & 1)))) * kLog2e;
}

__device__ __forceinline__ WaveInfo make_wave(const AttnParams& p, int D, int b, int kh, int s0,
                                              int pastb, int total) {
  WaveInfo w;
  w.kc = reinterpret_cast<const char*>(p.key_cache);
  w.vc = reinterpret_cast<const char*>(p.value_cache);
  w.kn = reinterpret_cast<const char*>(p.k_new);
  w.vn = reinterpret_cast<const char*>(p.v_new);
  w.b = b;
  w.kh = kh;
  w.s0 = s0;
  w.pastb = pastb;
  w.total = total;
  w.cache_limit = (p.read_all_from_cache || p.new_rows_in_cache) ? total : pastb;
  w.bs = p.block_size;
  w.bs_shift = (p.block_size & (p.block_size - 1)) == 0 ? __builtin_ctz(p.block_size) : -1;
  w.max_blocks = p.max_blocks;
  w.num_tokens = p.num_tokens;
  w.num_blocks = p.num_blocks;
  w.rowb = (int64_t)p.kv_heads * D * 2;
  w.first_bi = 0;
  w.bt = p.block_table + (int64_t)b * p.max_blocks;
  w.hoff = (int64_t)kh * D * 2;
  w.lin_row0 = -1;
  w.lin_cap = 0;
  if (p.linear_cap > 0) {
    w.rowb = (int64_t)D * 2;
    w.hoff = 0;
    w.lin_row0 = ((int64_t)b * p.kv_heads + kh) * p.linear_cap;
    w.lin_cap = p.linear_cap;
    w.bs = 16;  // rows of 16-key tiles are consecutive
    w.bs_shift = 4;
    w.cache_limit = total;
  }
  return w;
}

// Rows row0 .. row0+15 of kv-head kh: this lane's MFMA column is row r = row0 + c, i.e. query
// token r / g and head kh*g + r % g.  `qxor` is XORed into every query word (0x80008000 flips
// the sign of every element).
template <typename TT, int D>
__device__ __forceinline__ void init_rows(RowState<TT, D>& rs, const AttnParams& p,
                                          const WaveInfo& w, int row0, int R, int g, int c,
                                          int G, uint32_t qxor = 0) {
  using vec8 = typename TT::vec8;
  const int r = row0 + c;
  const bool rvalid = r < R;
  const int qi = rvalid ? r / g : 0;
  const int h = w.kh * g + (rvalid ? r % g : 0);
  const int rpos = w.pastb + qi;
  rs.vis_lo = p.window > 0 ? rpos - p.window + 1 : 0;
  rs.vis_hi = rvalid ? (p.causal ? rpos + 1 : w.total) : -1;
  const char* qrow = reinterpret_cast<const char*>(p.q) +
                     (((int64_t)(w.s0 + qi) * p.num_heads + h) * D + 8 * G) * 2;
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    const u32x4 v = rvalid ? (ld16(qrow + 64 * s) ^ qxor) : u32x4{0, 0, 0, 0};
    rs.qv[s] = __builtin_bit_cast(vec8, v);
  }
#pragma unroll
  for (int j = 0; j < D / 16; ++j) rs.o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  rs.m_run = kNegInf;
  rs.l_part = 0.0f;
}

// Epilogue: rows 4G+i of this lane's O registers.  final: normalise (with the sink) and write
// the output row in T; otherwise write the partial (O, m, l) at part_index(row): fp32, or with
// `half_part` fp16 rows scaled by 2^-e (e from the row's largest |O|, clamped to [-64, 126]: every
// element of a finite fp32 row fits, and l * 2^-e stays a normal float since l >= 1 for a row
// with any visible key) with e folded into the row's (m, l) as (m + e, l * 2^-e).  A log-sum-exp
// merge over (m, l, O) gives the same result for either form: the factors 2^e cancel between
// the weighted O and the denominator, the sink term included.
// TO: the output type (the products' type TT unless they run in another one); vsc: per-dim
// factors of the lane's DL output dims in final rows (integer pages' value scales), or null.
template <typename TT, int D, typename TO = TT, typename PartIndex>
__device__ __forceinline__ void store_rows(const RowState<TT, D>& rs, const AttnParams& p, int kh,
                                           int s0, int row0, int R, int g, int c, int G,
                                           float sink_c, bool final, PartIndex part_index,
                                           bool half_part = false, const float* vsc = nullptr) {
  constexpr int DL = D / 16;
  float l_row = rs.l_part + __shfl_xor(rs.l_part, 16, 64);
  l_row += __shfl_xor(l_row, 32, 64);
  int ex[4] = {0, 0, 0, 0};
  if (!final && half_part) {
    // Row 4G+i lives in the 16 lanes of group G (DL dims each): max over j, then over c.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < DL; ++j) mx = fmaxf(mx, fabsf(rs.o[j][i]));
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      ex[i] = min(max(__builtin_amdgcn_frexp_expf(mx), -64), 126);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rr = row0 + 4 * G + i;
    const float mi = __shfl(rs.m_run, 4 * G + i, 64);
    const float li = __shfl(l_row, 4 * G + i, 64);
    const float si = __shfl(sink_c, 4 * G + i, 64);  // sink logit of row rr (log2 units)
    if (rr >= R) continue;
    const int oqi = rr / g, oh = kh * g + rr % g;
    const int64_t t = s0 + oqi;
    if (final) {
      const float f = finalize_factor(mi, li, si);
      typename TO::raw vals[DL];
#pragma unroll
      for (int j = 0; j < DL; ++j) vals[j] = TO::from_f32(rs.o[j][i] * f * (vsc ? vsc[j] : 1.0f));
      typename TO::raw* dst =
          reinterpret_cast<typename TO::raw*>(p.out) + (t * p.num_heads + oh) * D + DL * c;
      if constexpr (DL == 8) {
        u32x4 pk;
#pragma unroll
        for (int m = 0; m < 4; ++m)
          pk[m] = (uint32_t)vals[2 * m] | ((uint32_t)vals[2 * m + 1] << 16);
        *reinterpret_cast<u32x4*>(dst) = pk;
      } else {
#pragma unroll
        for (int j = 0; j < DL; ++j) dst[j] = vals[j];
      }
    } else if (half_part) {
      const int64_t pi = part_index(t, oh, rr - row0);
      uint32_t w[DL / 2];
#pragma unroll
      for (int m = 0; m < DL / 2; ++m) {
        const _Float16 a = (_Float16)__builtin_ldexpf(rs.o[2 * m][i], -ex[i]);
        const _Float16 b = (_Float16)__builtin_ldexpf(rs.o[2 * m + 1][i], -ex[i]);
        w[m] = (uint32_t)__builtin_bit_cast(uint16_t, a) |
               ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
      }
      char* dst = reinterpret_cast<char*>(p.part_o) + (pi * D + DL * c) * 2;
      if constexpr (DL % 8 == 0) {
#pragma unroll
        for (int m = 0; m < DL / 8; ++m)
          reinterpret_cast<u32x4*>(dst)[m] = u32x4{w[4 * m], w[4 * m + 1], w[4 * m + 2], w[4 * m + 3]};
      } else if constexpr (DL == 4) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
      } else {
#pragma unroll
        for (int m = 0; m < DL / 2; ++m) reinterpret_cast<uint32_t*>(dst)[m] = w[m];
      }
      if (c == 0) {
        p.part_ml[pi * 2 + 0] = mi + (float)ex[i];
        p.part_ml[pi * 2 + 1] = __builtin_ldexpf(li, -ex[i]);
      }
    } else {
      const int64_t pi = part_index(t, oh, rr - row0);
      float* dst = p.part_o + pi * D + DL * c;
#pragma unroll
      for (int j = 0; j < DL; ++j) dst[j] = rs.o[j][i];
      if (c == 0) {
        p.part_ml[pi * 2 + 0] = mi;
        p.part_ml[pi * 2 + 1] = li;
      }
    }
  }
}

}  // namespace
}  // namespace pa
