// pa_decode.hip — split-K paged GQA decode on gfx950 matrix cores.
//
// Replaces the reference's direct Metal vector kernel and its two-pass partition/reduce
// (paged_attention.rs:31-143, launcher :229-334) and, for bf16, the dense gather + SDPA
// fallback (attention.rs:4192-4319) that the reference takes for every non-fp16 decode.
//
// Work unit: one wavefront per (sequence, kv-head, 16-row group, context chunk).  The
// wavefront serves every grouped query row of its kv-head -- rows r = (query token i, head hh)
// with r = i*g + hh, up to 16 at a time -- from ONE pass over the pages, so each K/V byte is
// read from HBM once per kv-head instead of once per query head (the reference re-reads it g
// times).
//
// Per 32-key step (two 16-key tiles A and B):
//   S^T = K_tile . Q^T   v_mfma_f32_16x16x32 (A = 16 keys x 32 dims straight from the page
//                        rows, 16 bytes per lane; B = Q^T held in registers for the chunk).
//                        Lane l ends with S[key 4*(l/16)+i][row l%16], i = 0..3, per tile.
//   online softmax       base 2, per row, lazy rescale: the running max only moves when a
//                        score exceeds it by more than 2^8, so the O rescale (and its
//                        cross-lane exchange) is rare.
//   O += P . V           v_mfma_f32_16x16x32: A = P exactly in the layout S came out in (row
//                        l%16, keys 4*(l/16)+0..3 of tile A and of tile B), B = V.  The value
//                        operand needs 8 keys x 1 dim per lane; lanes read 8 full value rows
//                        (16 lanes cover one 256-byte row) and regroup them with byte permutes,
//                        assigning output column n of N-tile j to head dim DL*n + j.  P is
//                        split into hi + lo 16-bit parts (two MFMAs) so the PV product keeps
//                        ~16 mantissa bits; the reference accumulates PV in fp32.
//
// Memory pipeline: steps whose 32 keys all sit in cached pages (and whose 16-key tiles each lie
// in one page, i.e. block_size % 16 == 0) run in a software-pipelined loop -- the next step's
// 16 KiB (bf16, d=128) is loaded into a second register set while the current step computes,
// with the page id taken from a register (v_readlane) so addresses are a scalar page base plus a
// fixed lane offset.  The remaining steps (the ones holding the new tokens, or any step when the
// block size is not a multiple of 16) take a per-lane addressed path without prefetch.
//
// Split-K: each chunk writes (m, l, O) partials; pa_attn_generic.hip's reduce merges them.  A
// sequence that fits one chunk writes its final rows directly.
#include <algorithm>
#include <type_traits>

#include "pa_tiles.hpp"

namespace pa {
namespace {

// fp8 (e4m3) pages: the same rows as loaded, one byte per element.  Key chunk h of a lane holds
// dims 64h + 16G .. +15 (k-steps 2h and 2h+1); value row e holds the lane's D/16 dims.
template <int D>
struct RawV8;
template <>
struct RawV8<64> {
  uint32_t w;
};
template <>
struct RawV8<128> {
  u32x2 w;
};
template <int D>
struct Step8 {
  u32x4 k[2][D / 64];
  RawV8<D> v[8];
  float sc;  // lane l: scale of (l & 2 ? value : key) page of tile (l & 1)
};

// Four e4m3 codes -> four bf16 (exact: every e4m3 value is a bf16 value) as two packed words,
// one gfx950 v_cvt_scalef32_pk_bf16_fp8 per code pair (scale 1.0: no scaling; all 65536 code
// pairs in both word positions checked on the device against an exact decode, NaN codes stay
// NaN).  For fp16 activations the same values are packed as fp16 (also exact: |x| <= 448, and
// the e4m3 subnormals are fp16 normals), so the MFMA operands match the query's type.
template <typename TT>
__device__ __forceinline__ u32x2 e4m3x4_widen(uint32_t w) {
  if constexpr (TT::code == PA_DTYPE_FLOAT16) {
    return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))};
  } else {
    return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))};
  }
}

// Key operand of k-step s of tile `tile`, widened from the codes as it is needed: chunk h = s/2
// of the lane's key codes holds k-steps 2h (words 0, 1) and 2h + 1 (words 2, 3).
template <typename TT, int D>
__device__ __forceinline__ typename TT::vec8 key_operand8(const Step8<D>& r, int tile, int s) {
  const u32x4& w = r.k[tile][s >> 1];
  const int t = s & 1;
  const u32x2 a = e4m3x4_widen<TT>(w[2 * t]), b = e4m3x4_widen<TT>(w[2 * t + 1]);
  return __builtin_bit_cast(typename TT::vec8, u32x4{a[0], a[1], b[0], b[1]});
}

// Value operand of N-tile j (8 keys x head dim (D/16)*c + j) straight from the code rows: one
// byte permute gathers dims j and j + 1 (j even) of value rows 2m and 2m + 1, and one
// conversion per N-tile turns a code pair into word m.  The permute of j and j + 1 is the same
// expression, so the two N-tiles share it.
template <typename TT, int D>
__device__ __forceinline__ typename TT::vec8 value_operand8(const Step8<D>& r, int j) {
  u32x4 w;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t lo, hi;
    if constexpr (D == 128) {
      lo = r.v[2 * m].w[j >> 2];
      hi = r.v[2 * m + 1].w[j >> 2];
    } else {
      lo = r.v[2 * m].w;
      hi = r.v[2 * m + 1].w;
    }
    // Bytes (row 2m, dim j'), (row 2m+1, dim j'), (row 2m, dim j'+1), (row 2m+1, dim j'+1) with
    // j' = j & ~1 within the word.
    const uint32_t pair = __builtin_amdgcn_perm(hi, lo, (j & 2) ? 0x07030602u : 0x05010400u);
    const u32x2 both = e4m3x4_widen<TT>(pair);  // (j & 1) picks one; the other folds away
    w[m] = (j & 1) ? both[1] : both[0];
  }
  return __builtin_bit_cast(typename TT::vec8, w);
}

// Integer pages (kv_cache.rs:222-256: values are code x scale).  The products run in fp16 on the
// exact codes: 0x64XX is the fp16 value 1024 + XX, so a biased code byte XX becomes its code with
// one packed subtraction -- int8: XX = code ^ 0x80, minus 1152; int4: XX = nibble = code + 8,
// minus 1032 (both exact: the results are small integers).  Key operands skip the subtraction:
// they hold code + bias, and the bias times the row's query sum (int_query's offset, the same for
// every key of the row) leaves each score in the FMA that scales it.  The scales enter outside
// the products: per-tensor key scales in the score scale, per-channel ones in the query operands,
// value scales in the epilogue (balanced_merge_kernel for split rows).
typedef _Float16 f16x2c __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f16pair_sub(uint32_t w, float bias) {
  const f16x2c v = __builtin_bit_cast(f16x2c, w) - f16x2c{(_Float16)bias, (_Float16)bias};
  return __builtin_bit_cast(uint32_t, v);
}
// w * a + b on both fp16 halves (exact here: w / 16 and the difference are fp16 integers).
__device__ __forceinline__ uint32_t f16pair_fma(uint32_t w, float a, float b) {
  const f16x2c v = __builtin_bit_cast(f16x2c, w) * f16x2c{(_Float16)a, (_Float16)a} +
                   f16x2c{(_Float16)b, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// int8 pages: Step8 layout (one byte per code).  Key operand of k-step s: words 2 (s & 1) and
// 2 (s & 1) + 1 of chunk s / 2, as in key_operand8.
template <int D>
__device__ __forceinline__ f16x8 key_operand_i8(const Step8<D>& r, int tile, int s) {
  const u32x4& w = r.k[tile][s >> 1];
  const int t = s & 1;
  const uint32_t a = w[2 * t] ^ 0x80808080u, b = w[2 * t + 1] ^ 0x80808080u;
  u32x4 o;  // code + 1152
  o[0] = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
  o[1] = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
  o[2] = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  o[3] = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  return __builtin_bit_cast(f16x8, o);
}

// Value operand of N-tile j (8 keys x head dim (D/16) c + j): word m pairs dim j of value rows
// 2m and 2m + 1 (byte j & 3 of word j >> 2 of each row slice).
template <int D>
__device__ __forceinline__ f16x8 value_operand_i8(const Step8<D>& r, int j) {
  const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + (j & 3)) << 16) | (uint32_t)(j & 3);
  u32x4 o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t lo, hi;
    if constexpr (D == 128) {
      lo = r.v[2 * m].w[j >> 2];
      hi = r.v[2 * m + 1].w[j >> 2];
    } else {
      lo = r.v[2 * m].w;
      hi = r.v[2 * m + 1].w;
    }
    o[m] = f16pair_sub(__builtin_amdgcn_perm(hi, lo, sel) ^ 0x64806480u, 1152.f);
  }
  return __builtin_bit_cast(f16x8, o);
}

// int4 pages: rows of D/2 bytes, byte i = dims 2i (low nibble) and 2i + 1 (high nibble).  Keys:
// lane group G holds the D/4 dims (D/4) G .. of its row in one D/8-byte piece (16 lanes x 4
// groups read whole row slices), word s of it = the 8 dims (D/4) G + 8 s .. of k-step s (the
// query operands take the same dims); value row e: the lane's D/16 dims in D/32 bytes (D = 64:
// two bytes in the low half of the word).
template <int D>
struct Step4 {
  uint32_t k[2][D / 32];
  uint32_t v[8];
};

template <int D>
__device__ __forceinline__ f16x8 key_operand_i4(const Step4<D>& r, int tile, int s) {
  const uint32_t x = r.k[tile][s];
  const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  u32x4 o;  // code + 1032
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + m) << 16) | (uint32_t)m;
    o[m] = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
  }
  return __builtin_bit_cast(f16x8, o);
}

// Value operand of N-tile j: byte j / 2 of value rows 2m and 2m + 1 into the two halves of word
// m (one byte permute), the nibble of dim j kept in place under the exponent of 1024 (one
// and-or): low nibbles (even j) read 1024 + code + 8, high nibbles (odd j) 1024 + 16 (code + 8),
// both brought back to the exact code by one packed fp16 operation.
template <int D>
__device__ __forceinline__ f16x8 value_operand_i4(const Step4<D>& r, int j) {
  const int byte = j >> 1;
  const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
  u32x4 o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t t = __builtin_amdgcn_perm(r.v[2 * m + 1], r.v[2 * m], sel);
    if (j & 1)
      o[m] = f16pair_fma((t & 0x00F000F0u) | 0x64006400u, 0.0625f, -72.f);
    else
      o[m] = f16pair_sub((t & 0x000F000Fu) | 0x64006400u, 1032.f);
  }
  return __builtin_bit_cast(f16x8, o);
}

// Integer pages: a piece's query rows as fp16 operands.  Per-channel key scales multiply the
// query dims they meet (q_d * s_d, fp32); the row is then scaled by 2^(14 - e), e the exponent
// of its largest |value| (so the row fits fp16 and keeps 11 bits), and the returned factor
// 2^(e - 14) -- times a per-tensor key scale -- restores the scores.  Lanes c, c + 16, c + 32,
// c + 48 hold row c; the lane's dims of k-step q are 64 (q / 2) + 16 G + 8 (q % 2) .. + 7 (int8),
// (D / 4) G + 8 q .. + 7 (int4).
// koff: bias x the sum of the row's fp16 query operands (the key operands hold code + bias).
template <typename TT, int D, bool I4>
__device__ __forceinline__ float int_query(RowState<TF16, D>& rs, const u32x4 (&qr)[D / 32],
                                           const AttnParams& p, int kh, int G, float bias,
                                           float& koff) {
  const bool pc = p.k_quant == PA_QUANT_PER_CHANNEL;
  float qf[D / 32][8];
  float mx = 0.0f;
#pragma unroll
  for (int q = 0; q < D / 32; ++q) {
    float sc[8];
    if (pc) {
      const float* sp = p.k_scale + (int64_t)kh * D + (I4 ? (D / 4) * G + 8 * q
                                                           : 64 * (q >> 1) + 16 * G + 8 * (q & 1));
      const f32x4 a = *reinterpret_cast<const f32x4*>(sp);
      const f32x4 b = *reinterpret_cast<const f32x4*>(sp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = a[i];
        sc[4 + i] = b[i];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t w = qr[q][e >> 1];
      const float v = TT::to_f32((typename TT::raw)((e & 1) ? (w >> 16) : (w & 0xffffu)));
      qf[q][e] = pc ? v * sc[e] : v;
      mx = fmaxf(mx, fabsf(qf[q][e]));
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const int ex = mx > 0.0f ? max(__builtin_amdgcn_frexp_expf(mx), -100) : 0;
  const float up = __builtin_ldexpf(1.0f, 14 - ex);
  float qsum = 0.0f;
#pragma unroll
  for (int q = 0; q < D / 32; ++q) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = qf[q][e] * up;
    rs.qv[q] = TF16::cvt8(t);
#pragma unroll
    for (int e = 0; e < 8; ++e) qsum += (float)rs.qv[q][e];
  }
  qsum += __shfl_xor(qsum, 16, 64);
  qsum += __shfl_xor(qsum, 32, 64);
  koff = bias * qsum;
  return __builtin_ldexpf(1.0f, ex - 14) * (pc ? 1.0f : p.k_scale[0]);
}

// Fast path: all 32 keys cached, 16-key tiles page-aligned.  The page id of each tile comes
// from lane (tile_block - first_bi) of `btv` (this chunk's block-table entries, one per lane).
template <int D>
__device__ __forceinline__ void load_fast(const WaveInfo& w, int btv, uint32_t koff,
                                          uint32_t voff, int t0, Step<D>& st) {
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const int tp = t0 + 16 * tile;
    int64_t blk = __builtin_amdgcn_readlane(btv, div_bs(tp, w) - w.first_bi);
    blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
    const int64_t tb = (blk * w.bs + mod_bs(tp, w)) * w.rowb + (int64_t)w.kh * D * 2;
    const char* kb = w.kc + tb;
    const char* vb = w.vc + tb;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) st.k[tile][s] = ld16(kb + koff + 64 * s);
#pragma unroll
    for (int e = 0; e < 4; ++e) st.v[4 * tile + e] = ld_vrow<D>(vb + voff + e * w.rowb);
  }
}

template <int D>
__device__ __forceinline__ void load_edge(const WaveInfo& w, int c, int G, int t0, Step<D>& st) {
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const char* kb = row_ptr(w, t0 + 16 * tile + c, false, D) + 16 * G;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) st.k[tile][s] = ld16(kb + 64 * s);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int pos = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
    st.v[e] = ld_vrow<D>(row_ptr(w, pos, true, D) + (D / 16) * 2 * c);
  }
}

// ----------------------------------------------------------------------------- shared driver

// Walk keys [t_begin, t_last) for one (sequence, kv-head) with NG 16-row groups `rs`; t_begin
// is a multiple of 32.  Every loaded step serves all NG groups (NG x fewer key/value reads per
// query row).  Steps entirely inside cached pages go through the pipelined fast loop in
// sub-ranges of at most 1024 keys (one block-table entry per lane covers a sub-range); the rest
// take the per-lane addressed path.  `end` masks keys at or beyond it.
//
// The fast loop keeps DEPTH steps in registers: DEPTH-1 steps are in flight while one
// computes.  Loads are always issued (past the last step they re-read the last step, which the
// caches serve), so every path through an iteration issues the same loads and the compiler's
// vmcnt waits only drain the step about to be computed.
template <typename TT, int D, bool CAP, int DEPTH, int NG>
__device__ __forceinline__ void run_range(WaveInfo w, RowState<TT, D> (&rs)[NG], int t_begin,
                                          int t_last, int end, int lane, int c, int G,
                                          float scale_log2, float scale, float cap) {
  static_assert(DEPTH == 2 || DEPTH == 3, "pipeline depth");
  const uint32_t koff = (uint32_t)(c * w.rowb + 16 * G);
  const uint32_t voff = (uint32_t)(4 * G * w.rowb + (D / 16) * 2 * c);
  int fast_lim = t_begin;
  if (w.bs % 16 == 0) {
    fast_lim = min(t_last, w.cache_limit);
    // Every key of the sequence is in the pages: the last (partial) step comes from the pages
    // too, its keys past the end masked and its page ids clamped into the pool.
    if (w.cache_limit >= w.total) fast_lim = t_begin + ((t_last - t_begin + 31) / 32) * 32;
  }
  int t0 = t_begin;
  Step<D> ring[DEPTH];
  while (t0 + 32 <= fast_lim) {
    const int nfast = (min(fast_lim, t0 + 1024) - t0) / 32;
    w.first_bi = div_bs(t0, w);
    const int btv = w.bt[min(w.first_bi + lane, w.max_blocks - 1)];
    const int last = t0 + 32 * (nfast - 1);
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i) load_fast<D>(w, btv, koff, voff, min(t0 + 32 * i, last), ring[i]);
    for (int k = 0; k < nfast; k += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        load_fast<D>(w, btv, koff, voff, min(t0 + 32 * (k + i + DEPTH - 1), last),
                     ring[(i + DEPTH - 1) % DEPTH]);
        if (k + i < nfast) {
          const int ts = t0 + 32 * (k + i);
          clear_tail_rows<D>(ring[i], ts, w.total, G);
#pragma unroll
          for (int j = 0; j < NG; ++j)
            compute_step<TT, D, CAP>(rs[j], ring[i], ts, end, G, scale_log2, scale, cap);
        }
      }
    }
    t0 += 32 * nfast;
  }
  Step<D>& sA = ring[0];
  for (; t0 < t_last; t0 += 32) {
    load_edge<D>(w, c, G, t0, sA);
#pragma unroll
    for (int j = 0; j < NG; ++j)
      compute_step<TT, D, CAP>(rs[j], sA, t0, end, G, scale_log2, scale, cap);
  }
}

// ----------------------------------------------------------------------------- chunked kernel
// One wavefront per (context chunk, kv-head, NG 16-row groups, sequence); kv-head fastest in the
// grid so the wavefronts reading the same pages run together.  Used when a sequence has more
// than 16 grouped query rows (multi-token queries, chunked prefill); partials at (token, head,
// chunk).  NG = 1: two wavefronts per SIMD (the d=128 ring fits 256 registers).  NG > 1
// (prefill): every loaded key/value step serves 16 * NG query rows, one wavefront per SIMD.
template <typename TT, int D, bool CAP, int NG>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(NG == 1 ? 2 : 1, NG == 1 ? 2 : 1))) void
decode_chunked_kernel(const AttnParams p) {
  const int kh = blockIdx.x % p.kv_heads, rgroup = blockIdx.x / p.kv_heads;
  const int ngroups = gridDim.x / p.kv_heads;
  const int split = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x, c = lane & 15, G = lane >> 4;
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int nq = s1 - s0;
  if (nq <= 0) return;
  const int pastb = clamped_past(p, b, nq);
  const int total = seq_total(p, b, pastb, nq);
  const int start = split * p.chunk;
  if (start >= total) return;
  const int end = min(start + p.chunk, total);
  const int g = p.num_heads / p.kv_heads;
  const int R = g * nq;
  const WaveInfo w = make_wave(p, D, b, kh, s0, pastb, total);
  const bool single = (start == 0 && end == total);
  // Metadata beyond the planned capacity (total > max_blocks * block_size) leaves no partial
  // buffer to write into; such rows are left unwritten rather than faulting.
  if (!single && p.part_o == nullptr) return;
  for (int row0 = 16 * NG * rgroup; row0 < R; row0 += 16 * NG * ngroups) {
    RowState<TT, D> rs[NG];
    // Keys outside every row's causal/window range are skipped (whole 32-key steps).
    int lo_any = INT32_MAX, hi_any = -1;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      init_rows<TT, D>(rs[j], p, w, row0 + 16 * j, R, g, c, G);
      if (row0 + 16 * j + c < R) lo_any = min(lo_any, rs[j].vis_lo);
      hi_any = max(hi_any, rs[j].vis_hi);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      lo_any = min(lo_any, __shfl_xor(lo_any, o, 64));
      hi_any = max(hi_any, __shfl_xor(hi_any, o, 64));
    }
    const int t_first = max(start, (lo_any / 32) * 32);
    const int t_last = min(end, hi_any);
    run_range<TT, D, CAP, 2, NG>(w, rs, t_first, t_last, end, lane, c, G, p.scale_log2, p.scale,
                                 p.softcap);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int r0 = row0 + 16 * j;
      if (r0 >= R) break;
      const int rc = min(r0 + c, R - 1);
      const float sink_c = sink_logit<TT>(p, kh * g + rc % g);
      store_rows<TT, D>(rs[j], p, kh, s0, r0, R, g, c, G, sink_c, single,
                        [&](int64_t t, int oh, int) {
                          return (t * p.num_heads + oh) * p.max_splits + split;
                        });
    }
  }
}

// ----------------------------------------------------------------------------- balanced kernel
// Decode with at most 16 grouped query rows per sequence.  Every sequence contributes
// n_b = ceil((total_b - first_b) / 32) steps of 32 keys (first_b: first key any row can see);
// the steps of all sequences, in order, are cut into `nseg` contiguous segments of equal length
// (the last ones may be shorter or empty), and the
// wavefront for (segment, kv-head) walks its segment across sequence boundaries.  Each
// wavefront does the same work and the kv-heads of a segment are adjacent in the grid, so all
// wavefronts finish together and the ones sharing pages read them together.  A sequence
// covered by one segment is written directly; otherwise each covering segment s writes a
// partial at slot s + b (unique: segments of b are consecutive and the next sequence starts in
// the segment where b ends or in the next one), merged by balanced_merge_kernel.

struct SeqSteps {
  int s0, nq, pastb, total, first, n;  // first: first key step start (multiple of 32)
};

// All three metadata loads are issued before any test (index clamped; p.batch >= 1), so a
// lookup costs one memory round trip.
__device__ __forceinline__ SeqSteps seq_steps(const AttnParams& p, int b) {
  SeqSteps q{0, 0, 0, 0, 0, 0};
  const int bb = min(b, p.batch - 1);
  const int c0 = p.cum[bb], c1 = p.cum[bb + 1], pb = p.past[bb];
  const bool live = b < p.batch;
  q.s0 = live ? min(max(c0, 0), p.num_tokens) : 0;
  const int s1 = live ? min(max(c1, q.s0), p.num_tokens) : 0;
  // Keys are clamped to the cache capacity (metadata the host checked never reaches it), which
  // bounds the batch's step count for the 32-bit step indices of the streaming kernel.
  const int cap = p.linear_cap > 0 ? p.linear_cap
                                   : (int)min((int64_t)p.max_blocks * p.block_size,
                                              (int64_t)(INT32_MAX / 2));
  q.nq = min(s1 - q.s0, cap);
  const bool any = q.nq > 0;
  q.pastb = any ? min(max(pb, 0), cap - q.nq) : 0;
  q.total = any ? q.pastb + q.nq : 0;
  if (p.key_limit && any) q.total = min(q.total, max(p.key_limit[bb], 0));
  q.first = (any && p.window > 0) ? (max(0, q.pastb - p.window + 1) / 32) * 32 : 0;
  q.n = any ? max(q.total - q.first + 31, 0) / 32 : 0;
  return q;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// Wave-uniform (readlane, so the compiler keeps it in scalar registers).
__device__ __forceinline__ int64_t total_steps(const AttnParams& p, int lane) {
  int64_t S = 0;
  for (int base = 0; base < p.batch; base += 64) {
    const int n = seq_steps(p, base + lane).n;
    S += __builtin_amdgcn_readlane(wave_incl_scan(n, lane), 63);
  }
  return S;
}

// Segments are L = ceil(S / nseg) steps long, so empty segments can only trail the list and
// every segment between the first and last one covering a sequence holds part of it.
__device__ __forceinline__ int64_t seg_len(int64_t S, int nseg) { return (S + nseg - 1) / nseg; }

// Merge the nparts partials of (sequence b, kv-head kh), stored at slots f+b .. f+nparts-1+b,
// into the final rows.  Thread t (of 256) handles row t / 16 and DS = D / 16 consecutive head
// dims.  Up to KB pieces are loaded together (every load issued before any is used; indices
// clamped into range, surplus pieces weighted zero), so a sequence of up to KB partials -- at
// the config 3 batch every one -- costs one memory round trip.
template <typename TT, int D>
__device__ __forceinline__ void merge_pieces(const AttnParams& p, int b, int kh, int s0, int R,
                                             int g, int f, int nparts, int tid) {
  constexpr int DS = D / 16;           // dims per thread
  constexpr int KB = D > 128 ? 6 : 96 / DS;  // pieces per batch (~96 registers of partials)
  static_assert(DS % 2 == 0, "pairs of dims");
  const int r = tid >> 4, slice = tid & 15;
  if (r >= R) return;
  float M = kNegInf, lsum = 0.0f;
  float acc[DS];
#pragma unroll
  for (int e = 0; e < DS; ++e) acc[e] = 0.0f;
  for (int k0 = 0; k0 < nparts; k0 += KB) {
    float2 ml[KB];
    float o[KB][DS];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int k = min(k0 + j, nparts - 1);
      const int64_t row = (((int64_t)f + k + b) * p.kv_heads + kh) * 16 + r;
      ml[j] = *reinterpret_cast<const float2*>(p.part_ml + row * 2);
      const float* src = p.part_o + row * D + slice * DS;
      if constexpr (DS % 4 == 0) {
#pragma unroll
        for (int v = 0; v < DS / 4; ++v) {
          const f32x4 x = reinterpret_cast<const f32x4*>(src)[v];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[j][4 * v + e] = x[e];
        }
      } else {
#pragma unroll
        for (int v = 0; v < DS / 2; ++v) {
          const float2 x = reinterpret_cast<const float2*>(src)[v];
          o[j][2 * v] = x.x;
          o[j][2 * v + 1] = x.y;
        }
      }
    }
    float mn = M;
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (k0 + j < nparts) mn = fmaxf(mn, ml[j].x);
    // mn == -inf (every piece so far saw only masked keys) leaves a = w = 0 below.
    const float a = (M == kNegInf) ? 0.0f : exp2f(M - mn);
    lsum *= a;
#pragma unroll
    for (int e = 0; e < DS; ++e) acc[e] *= a;
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const float w = (k0 + j < nparts && ml[j].x != kNegInf) ? exp2f(ml[j].x - mn) : 0.0f;
      lsum += ml[j].y * w;
#pragma unroll
      for (int e = 0; e < DS; ++e) acc[e] += o[j][e] * w;
    }
    M = mn;
  }
  const int h = kh * g + r % g;
  const int64_t t = s0 + r / g;
  const float fct = finalize_factor(M, lsum, sink_logit<TT>(p, h));
  if (p.v_quant == PA_QUANT_PER_TENSOR || p.v_quant == PA_QUANT_PER_CHANNEL) {
    // integer pages: the partials are in code units; scale each output dim
    const bool pc = p.v_quant == PA_QUANT_PER_CHANNEL;
#pragma unroll
    for (int e = 0; e < DS; ++e)
      acc[e] *= pc ? p.v_scale[(int64_t)kh * D + slice * DS + e] : p.v_scale[0];
  }
  uint32_t w[DS / 2];
#pragma unroll
  for (int m = 0; m < DS / 2; ++m)
    w[m] = (uint32_t)TT::from_f32(acc[2 * m] * fct) |
           ((uint32_t)TT::from_f32(acc[2 * m + 1] * fct) << 16);
  uint32_t* out = reinterpret_cast<uint32_t*>(reinterpret_cast<typename TT::raw*>(p.out) +
                                              (t * p.num_heads + h) * D + slice * DS);
  if constexpr (DS % 8 == 0) {
#pragma unroll
    for (int v = 0; v < DS / 8; ++v)
      reinterpret_cast<u32x4*>(out)[v] = u32x4{w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]};
  } else if constexpr (DS == 4) {
    *reinterpret_cast<u32x2*>(out) = u32x2{w[0], w[1]};
  } else {
#pragma unroll
    for (int m = 0; m < DS / 2; ++m) out[m] = w[m];
  }
}

// Up to 64 consecutive sequences, lane l describing sequence base + l.
struct SeqWin {
  int base;
  SeqSteps q;
  int P;  // first flattened step of this lane's sequence
};

// Wave-uniform position in the flattened step list.  The sequence fields a cursor needs on every
// step are read from the window lanes only when it enters a sequence, and the key position t
// advances by 32 per step, so moving to the next step costs a few scalar instructions.  Step
// indices are 32-bit: sequences are clamped to the cache capacity (seq_steps) and the host
// bounds batch * (capacity / 32 + 1) below 2^31.
struct Cursor {
  int f;      // flattened step
  int pend;   // one past the last step of the sequence holding step f
  int u;      // sub-segment holding step f
  int ub;     // one past that sub-segment's last step
  int bl;     // window lane of the sequence
  int t;      // first key position of step f
  int kh;     // kv-head of sub-segment u
  int total;  // keys of the sequence
  int lim;    // keys below lim are read from the pages
};

__device__ __forceinline__ int sub_segment_kh(int u, int u0, int x, int kv_heads) {
  const int kh = x + (u - u0);  // mix <= kv_heads
  return kh >= kv_heads ? kh - kv_heads : kh;
}

__device__ __forceinline__ int lane_of(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

__device__ __forceinline__ void cursor_seq(Cursor& c, const SeqWin& sw, const AttnParams& p) {
  const int pend_l = sw.P + sw.q.n;
  const uint64_t m = __ballot(sw.q.n > 0 && pend_l > c.f);
  c.bl = m ? __builtin_ctzll(m) : 63;
  c.pend = lane_of(pend_l, c.bl);
  c.total = lane_of(sw.q.total, c.bl);
  c.lim = (p.read_all_from_cache || p.new_rows_in_cache) ? c.total : lane_of(sw.q.pastb, c.bl);
  c.t = lane_of(sw.q.first, c.bl) + 32 * (c.f - lane_of(sw.P, c.bl));
}

__device__ __forceinline__ Cursor cursor_at(const SeqWin& sw, const AttnParams& p, int f, int L,
                                            int x, int u0) {
  Cursor c;
  c.f = f;
  c.u = f / L;
  c.ub = (c.u + 1) * L;
  c.kh = sub_segment_kh(c.u, u0, x, p.kv_heads);
  cursor_seq(c, sw, p);
  return c;
}

// Next step, or stay on the last one (hi - 1): look-ahead cursors re-read it.  Returns true
// when the sequence or the kv-head changed.
__device__ __forceinline__ bool cursor_next(Cursor& c, const SeqWin& sw, const AttnParams& p,
                                            int hi, int L, int x, int u0) {
  if (c.f + 1 >= hi) return false;
  ++c.f;
  c.t += 32;
  bool changed = false;
  if (c.f >= c.pend) {
    cursor_seq(c, sw, p);
    changed = true;
  }
  if (c.f >= c.ub) {
    ++c.u;
    c.ub += L;
    c.kh = sub_segment_kh(c.u, u0, x, p.kv_heads);
    changed = true;
  }
  return changed;
}

// Block-table entries of a step: lane l holds the entry of key t + (l & 31) (index clamped into
// the table row; entries past the sequence are never used for addressing).
__device__ __forceinline__ int load_step_blocks(const AttnParams& p, const SeqWin& sw,
                                                const Cursor& c, int lane, int bs_shift) {
  // Contiguous caches have no block table: the load still happens (same count on every path)
  // and its value is unused.
  if (p.linear_cap > 0) return p.cum[0];
  const int bi = min((c.t + (lane & 31)) >> bs_shift, p.max_blocks - 1);
  return p.block_table[(int64_t)(sw.base + c.bl) * p.max_blocks + bi];
}

// Address of key/value row `pos` (t <= pos < total) of a step, branch-free: a cache page when
// pos < lim (page id from lane pos - t of `btl`, clamped into the pool), else the new row of the
// packed batch (token s0 + pos - pastb).
__device__ __forceinline__ const char* stream_row(const AttnParams& p, const Cursor& c, int btl,
                                                  int pos, int s0, int pastb, const char* cache,
                                                  const char* fresh, uint32_t rowb, uint32_t hoff,
                                                  int bs_shift) {
  const int blk = min(max(__shfl(btl, pos - c.t, 64), 0), (int)min(p.num_blocks - 1,
                                                                      (int64_t)INT32_MAX));
  const uint32_t crow = ((uint32_t)blk << bs_shift) + (uint32_t)(pos & (p.block_size - 1));
  const uint32_t tok = (uint32_t)min(max(s0 + (pos - pastb), 0), p.num_tokens - 1);
  const bool in_cache = pos < c.lim;
  const char* base = in_cache ? cache : fresh;
  const uint64_t row = in_cache ? crow : tok;
  return base + row * rowb + hoff;
}

// Page rows through buffer loads: one scalar descriptor per 16-row tile (base address in
// SGPRs) and offsets fixed per lane, so addressing a step costs scalar instructions only.
// Streaming (nt) loads, like ld16s.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const char* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ u32x4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}
__device__ __forceinline__ u32x2 bld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 2));
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 2);
}

// One lane's value-row slice (D/8 bytes at voff of the row at soff) through buffer loads.
template <int D>
__device__ __forceinline__ VRow<D> bld_vrow(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff) {
  if constexpr (D == 64) {
    return VRow<64>{bld8(r, voff, soff)};
  } else if constexpr (D == 128) {
    return VRow<128>{bld16(r, voff, soff)};
  } else if constexpr (D % 128 == 0) {
    VRow<D> v;
#pragma unroll
    for (int i = 0; i < D / 128; ++i) {
      const u32x4 x = bld16(r, voff + 16 * i, soff);
#pragma unroll
      for (int k = 0; k < 4; ++k) v.w[4 * i + k] = x[k];
    }
    return v;
  } else if constexpr (D == 96) {  // one dwordx3 load (4-byte aligned slice)
    const u32x3 x =
        __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 2));
    return VRow<D>{{x[0], x[1], x[2]}};
  } else {
    VRow<D> v;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) v.w[i] = bld4(r, voff + 4 * i, soff);
    return v;
  }
}

// Page id of tile `tile` of a step (lane 16 * tile of `btl`), clamped into the pool, and the
// byte offset of the tile's first row from the pool base.
__device__ __forceinline__ uint64_t tile_row_bytes(const AttnParams& p, const Cursor& c, int btl,
                                                   int tile, int bs_shift, uint32_t rowb,
                                                   int64_t& blk) {
  blk = min(max((int64_t)__builtin_amdgcn_readlane(btl, 16 * tile), (int64_t)0),
            (int64_t)p.num_blocks - 1);
  const uint64_t row0 =
      (uint64_t)((blk << bs_shift) + ((c.t + 16 * tile) & (p.block_size - 1)));
  return row0 * rowb;
}

// Cache kinds of the streaming decode: pages in the activation dtype, fp8 e4m3, int8, int4;
// kDcLin marks integer codes in a contiguous cache and kDcBias an additive attention bias
// (GroupQueryAttention presents and attention_bias).
enum DecodeCache { kDcT = 0, kDcFp8 = 1, kDcI8 = 2, kDcI4 = 3, kDcLin = 4, kDcBias = 8 };
// The cache dtype of a decode form (kDcT: -1, caches in the activation dtype).
constexpr int decode_cache_dtype(int ck) {
  return (ck & 3) == kDcI4 ? PA_DTYPE_INT4
         : (ck & 3) == kDcI8 ? PA_DTYPE_INT8
         : (ck & 3) == kDcFp8 ? PA_DTYPE_FP8_E4M3
                              : -1;
}

template <typename TT, int D, int CK>
using RingStep = typename std::conditional<
    (CK & 3) == kDcT, Step<D>,
    typename std::conditional<(CK & 3) == kDcI4, Step4<D>, Step8<D>>::type>::type;

// Per-lane constants of the streaming loads.
struct LaneOffs {
  uint32_t koff, voff;  // key / value offsets of this lane inside a 16-row tile (bytes)
  uint32_t rowb;        // bytes per cache row
};

// Per-lane pointers of the query row and sink logit the data cursor's (sequence, kv-head)
// needs; recomputed only when that cursor changes sequence or kv-head.  MFMA column c is row
// r = c (rows past R repeat the last one; their scores never reach an output).  Query k-step q
// covers dims 32q + 8G .. (bf16 pages), 64(q/2) + 16G + 8(q%2) .. (fp8 / int8 pages, matching
// the key chunks) or (D/4)G + 8q .. (int4 pages); the lane part of that offset is folded in
// here, the q part is a constant.
struct QueryPtrs {
  const char* q;
  const char* sink;
  BiasRow br;  // BIAS: the bias row of row r
};
// QL: the query layout (0 pages in T, 1 fp8 / int8 pages, 2 int4 pages)
template <int D, int QL, bool BIAS = false>
__device__ __forceinline__ QueryPtrs query_ptrs(const AttnParams& p, const SeqWin& sw,
                                                const Cursor& c, int g, int lane) {
  const int cl = lane & 15, G = lane >> 4;
  const int s0 = lane_of(sw.q.s0, c.bl), nq = lane_of(sw.q.nq, c.bl);
  const int r = max(min(cl, g * nq - 1), 0);
  const int rq = r / g, rh = r - rq * g;
  QueryPtrs o;
  o.q = reinterpret_cast<const char*>(p.q) +
        ((int64_t)(s0 + rq) * p.num_heads + c.kh * g + rh) * D * 2 +
        (QL == 1 ? 32 : QL == 2 ? D / 2 : 16) * G;
  // Sink logit input of that row's head (a harmless read of the query when there is none).
  o.sink = p.head_sink ? reinterpret_cast<const char*>(p.head_sink) + (c.kh * g + rh) * 2
                       : reinterpret_cast<const char*>(p.q);
  if constexpr (BIAS) o.br = bias_row_of(p, sw.base + c.bl, c.kh * g + rh, rq);
  return o;
}

// fp8 pages (every row in the pages, block size a multiple of 16): per tile D/64 16-byte key
// chunks (dims 64h + 16G ..) and four D/16-byte value rows per lane, plus the page scales.
template <int D, bool SCALES = true>
__device__ __forceinline__ void load_step8(const AttnParams& p, const Cursor& c, int btl, int lane,
                                           int bs_shift, const LaneOffs& lo, Step8<D>& st) {
  const uint32_t hoff = (uint32_t)c.kh * D;
  const char* kc = reinterpret_cast<const char*>(p.key_cache);
  const char* vc = reinterpret_cast<const char*>(p.value_cache);
  int64_t blk[2];
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const uint64_t off = tile_row_bytes(p, c, btl, tile, bs_shift, lo.rowb, blk[tile]) + hoff;
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kc + off), rv = rows_rsrc(vc + off);
#pragma unroll
    for (int h = 0; h < D / 64; ++h) st.k[tile][h] = bld16(rk, lo.koff + 64 * h, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (D == 128)
        st.v[4 * tile + e].w = bld8(rv, lo.voff, e * lo.rowb);
      else
        st.v[4 * tile + e].w = bld4(rv, lo.voff, e * lo.rowb);
    }
  }
  if constexpr (SCALES) {
    const float* sp = (lane & 2) ? p.v_scale : p.k_scale;
    st.sc = sp[((lane & 1) ? blk[1] : blk[0]) * p.kv_heads + c.kh];
  }
}

// int4 pages: per tile one D/8-byte key piece (the lane group's D/4 dims) and four D/32-byte
// value row slices per lane.
template <int D>
__device__ __forceinline__ void load_step4(const AttnParams& p, const Cursor& c, int btl, int lane,
                                           int bs_shift, const LaneOffs& lo, Step4<D>& st) {
  const uint32_t hoff = (uint32_t)c.kh * (D / 2);
  const char* kc = reinterpret_cast<const char*>(p.key_cache);
  const char* vc = reinterpret_cast<const char*>(p.value_cache);
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    int64_t blk;
    const uint64_t off = tile_row_bytes(p, c, btl, tile, bs_shift, lo.rowb, blk) + hoff;
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kc + off), rv = rows_rsrc(vc + off);
    if constexpr (D == 128) {
      const u32x4 x = bld16(rk, lo.koff, 0);
#pragma unroll
      for (int m = 0; m < 4; ++m) st.k[tile][m] = x[m];
    } else {
      const u32x2 x = bld8(rk, lo.koff, 0);
      st.k[tile][0] = x[0];
      st.k[tile][1] = x[1];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (D == 128)
        st.v[4 * tile + e] = bld4(rv, lo.voff, e * lo.rowb);
      else
        st.v[4 * tile + e] =
            (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rv, lo.voff, e * lo.rowb, 2);
    }
  }
}

// Contiguous integer caches [batch, kv_heads, cap, RB bytes] (GroupQueryAttention presents):
// the same per-lane pieces as load_step8 / load_step4, addressed per lane from the rows of
// (sequence, kv-head); rows past the sequence end re-read its last row (finite codes, weighted
// zero), so no load leaves the sequence's rows.
template <int D, int CK, typename ST>
__device__ __forceinline__ void load_step_linear(const AttnParams& p, const SeqWin& sw,
                                                 const Cursor& c, int lane, ST& st) {
  constexpr int RB = CK == kDcI4 ? D / 2 : D;  // bytes per row
  const int cl = lane & 15, G = lane >> 4;
  const int last = c.total - 1;
  const int64_t r0 = ((int64_t)(sw.base + c.bl) * p.kv_heads + c.kh) * p.linear_cap;
  const char* kc = reinterpret_cast<const char*>(p.key_cache) + r0 * RB;
  const char* vc = reinterpret_cast<const char*>(p.value_cache) + r0 * RB;
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    const int tp = c.t + 16 * tile;
    const char* kr = kc + (int64_t)min(tp + cl, last) * RB;
    if constexpr (CK == kDcI4) {
      if constexpr (D == 128) {
        const u32x4 x = ld16s(kr + 16 * G);
#pragma unroll
        for (int m = 0; m < 4; ++m) st.k[tile][m] = x[m];
      } else {
        const u32x2 x = ld8s(kr + 8 * G);
        st.k[tile][0] = x[0];
        st.k[tile][1] = x[1];
      }
    } else {
#pragma unroll
      for (int h = 0; h < D / 64; ++h) st.k[tile][h] = ld16s(kr + 16 * G + 64 * h);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const char* vr = vc + (int64_t)min(tp + 4 * G + e, last) * RB + (RB / 16) * cl;
      if constexpr (CK == kDcI4) {
        if constexpr (D == 128)
          st.v[4 * tile + e] = ld4s(vr);
        else
          st.v[4 * tile + e] =
              (uint32_t)__builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(vr));
      } else {
        if constexpr (D == 128)
          st.v[4 * tile + e].w = ld8s(vr);
        else
          st.v[4 * tile + e].w = ld4s(vr);
      }
    }
  }
}

// All loads of one step: K and V rows of both 16-key tiles and the query rows of the step's
// (sequence, kv-head).  Every path issues the same number of loads, so the compiler's vmcnt
// waits only drain the step about to be computed.  Rows past the sequence end re-read the last
// row (or stay in the last page).
template <typename TT, int D, int CK>
__device__ __forceinline__ void load_stream_step(const AttnParams& p, const SeqWin& sw,
                                                 const Cursor& c, int btl, int lane, int bs_shift,
                                                 const LaneOffs& lo, const QueryPtrs& qp,
                                                 bool qload, RingStep<TT, D, CK>& st,
                                                 u32x4 (&qv)[D / 32], typename TT::raw& sk) {
  constexpr int QL = (CK & 3) == kDcT ? 0 : (CK & 3) == kDcI4 ? 2 : 1;  // query layout
  const int cl = lane & 15, G = lane >> 4;
  if constexpr ((CK & kDcLin) != 0) {
    load_step_linear<D, CK & 3>(p, sw, c, lane, st);
  } else if constexpr (CK == kDcI8 || CK == kDcI4) {
    if constexpr (CK == kDcI8)
      load_step8<D, false>(p, c, btl, lane, bs_shift, lo, st);
    else
      load_step4<D>(p, c, btl, lane, bs_shift, lo, st);
  } else if constexpr (CK == kDcFp8) {
    load_step8<D, true>(p, c, btl, lane, bs_shift, lo, st);
  } else {
    constexpr int DL = D / 16;
    const uint32_t hoff = (uint32_t)c.kh * D * 2;
    const char* kc = reinterpret_cast<const char*>(p.key_cache);
    const char* vc = reinterpret_cast<const char*>(p.value_cache);
    const int last = c.total - 1;
    if (p.linear_cap > 0) {
      // Contiguous cache: rows of (b, kh) follow each other; rows past the end re-read the last.
      const int64_t r0 = ((int64_t)(sw.base + c.bl) * p.kv_heads + c.kh) * p.linear_cap;
      const uint32_t rs = (uint32_t)D * 2;
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        const int tp = c.t + 16 * tile;
        const char* kr = kc + (uint64_t)(r0 + min(tp + cl, last)) * rs;
#pragma unroll
        for (int q = 0; q < D / 32; ++q) st.k[tile][q] = ld16s(kr + 16 * G + 64 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          st.v[4 * tile + e] =
              ld_vrow_s<D>(vc + (uint64_t)(r0 + min(tp + 4 * G + e, last)) * rs + DL * 2 * cl);
      }
    } else if (bs_shift >= 4 && min(c.t + 31, last) < c.lim) {
      // Every row in the pages and each 16-key tile inside one page.
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        int64_t blk;
        const uint64_t off = tile_row_bytes(p, c, btl, tile, bs_shift, lo.rowb, blk) + hoff;
        const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kc + off), rv = rows_rsrc(vc + off);
#pragma unroll
        for (int q = 0; q < D / 32; ++q) st.k[tile][q] = bld16(rk, lo.koff + 64 * q, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) st.v[4 * tile + e] = bld_vrow<D>(rv, lo.voff, e * lo.rowb);
      }
    } else {
      const char* kn = reinterpret_cast<const char*>(p.k_new);
      const char* vn = reinterpret_cast<const char*>(p.v_new);
      const int s0 = lane_of(sw.q.s0, c.bl), pastb = lane_of(sw.q.pastb, c.bl);
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        const int tp = c.t + 16 * tile;
        const char* kr = stream_row(p, c, btl, min(tp + cl, last), s0, pastb, kc, kn, lo.rowb,
                                    hoff, bs_shift);
#pragma unroll
        for (int q = 0; q < D / 32; ++q) st.k[tile][q] = ld16s(kr + 16 * G + 64 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const char* vr = stream_row(p, c, btl, min(tp + 4 * G + e, last), s0, pastb, vc, vn,
                                      lo.rowb, hoff, bs_shift);
          st.v[4 * tile + e] = ld_vrow_s<D>(vr + DL * 2 * cl);
        }
      }
    }
  }
  // Query rows and sink only for a step that starts a piece (the compute cursor takes them
  // there and nowhere else).
  if (qload) {
#pragma unroll
    for (int q = 0; q < D / 32; ++q)
      qv[q] = ld16(qp.q + (QL == 1 ? 128 * (q >> 1) + 16 * (q & 1) : QL == 2 ? 16 * q : 64 * q));
    sk = *reinterpret_cast<const typename TT::raw*>(qp.sink);
  }
}

// Stream the flattened steps [lo, hi) of one window through a DEPTH-deep register ring.  Three
// cursors run over the same step list: block-table entries are fetched 2 * (DEPTH - 1) steps
// ahead of the compute, key/value/query rows DEPTH - 1 steps ahead, so a sequence or kv-head
// boundary costs no pipeline refill.  A piece (one sequence, one sub-segment) is finished when
// the compute cursor leaves it: final rows when the piece covers its whole sequence, else a
// partial at slot u + b.  Steps whose keys are visible to every row of the piece skip the
// per-score position tests.
template <typename TT, int D, bool CAP, int CK, int DEPTH>
__device__ __forceinline__ void stream_range(const AttnParams& p, const SeqWin& sw, int lo, int hi,
                                             int L, int x, int u0, int lane) {
  constexpr bool F8 = (CK & 3) != kDcT;  // byte-coded pages
  constexpr int QL = (CK & 3) == kDcT ? 0 : (CK & 3) == kDcI4 ? 2 : 1;  // query layout
  constexpr bool BIAS = (CK & kDcBias) != 0;  // additive bias (GroupQueryAttention)
  constexpr bool INT = (CK & 3) >= kDcI8;  // integer codes: fp16 products
  constexpr int CB = CK & 3;               // the code kind (kDcLin: contiguous addressing)
  using MT = typename std::conditional<INT, TF16, TT>::type;  // the products' type
  using vec8 = typename MT::vec8;
  const int c = lane & 15, G = lane >> 4;
  const int g = p.num_heads / p.kv_heads;
  const int bs_shift = __builtin_ctz(p.block_size);  // power of two (host dispatch)
  const int K = hi - lo;
  // bytes per row of one kv-head, and of one key chunk / value slice unit
  constexpr int RB = CB == kDcT ? 2 * D : CB == kDcI4 ? D / 2 : D;
  LaneOffs lofs;
  lofs.rowb = (uint32_t)p.kv_heads * RB;
  lofs.koff = (uint32_t)c * lofs.rowb + (CB == kDcI4 ? D / 8 : 16) * G;
  lofs.voff = (uint32_t)(4 * G) * lofs.rowb + (uint32_t)(RB / 16) * c;

  // Block ids run BA steps ahead of the compute in a ring of NBT entries: 2 * (DEPTH - 1) ahead
  // in DEPTH entries, or, with a one-step ring (rows loaded in the step that uses them), one
  // step ahead in two entries.  The loop body is unrolled U times so every ring index is a
  // compile-time constant.
  constexpr int BA = DEPTH > 1 ? 2 * (DEPTH - 1) : 1;
  constexpr int NBT = DEPTH > 1 ? DEPTH : 2;
  constexpr int U = DEPTH > 1 ? DEPTH : 2;
  Cursor cc = cursor_at(sw, p, lo, L, x, u0);
  Cursor cd = cc, cb = cc;
  QueryPtrs qp = query_ptrs<D, QL, BIAS>(p, sw, cd, g, lane);
  RingStep<TT, D, CK> st[DEPTH];
  u32x4 qr[DEPTH][D / 32];
  typename TT::raw skr[DEPTH];
  uint32_t braw[BIAS ? DEPTH : 1][4];  // BIAS: the lane's 8 bias values of each ring step
  int btr[NBT];
  // Prologue: block ids of steps 0 .. DEPTH-2, their rows, block ids of steps DEPTH-1 .. BA-1.
#pragma unroll
  for (int j = 0; j < DEPTH - 1; ++j) {
    btr[j % NBT] = load_step_blocks(p, sw, cb, lane, bs_shift);
    cursor_next(cb, sw, p, hi, L, x, u0);
  }
  bool qload = true;  // the data cursor's step starts a piece
#pragma unroll
  for (int j = 0; j < DEPTH - 1; ++j) {
    load_stream_step<TT, D, CK>(p, sw, cd, btr[j % NBT], lane, bs_shift, lofs, qp, qload, st[j],
                                qr[j], skr[j]);
    if constexpr (BIAS) bias_load(qp.br, cd.t, G, braw[j]);
    qload = cursor_next(cd, sw, p, hi, L, x, u0);
    if (qload) qp = query_ptrs<D, QL, BIAS>(p, sw, cd, g, lane);
  }
#pragma unroll
  for (int j = DEPTH - 1; j < BA; ++j) {
    btr[j % NBT] = load_step_blocks(p, sw, cb, lane, bs_shift);
    cursor_next(cb, sw, p, hi, L, x, u0);
  }

  RowState<MT, D> rs;
  float row_f = 1.0f;  // integer pages: this row's score factor (query normalisation x key scale)
  float koff = 0.0f;   // integer pages: the key-operand bias times the row's query sum
  int pc_bl = -1, pc_u = -1;  // the piece being computed
  int pc_kh = 0, pc_total = 0;
  int full_lo = 0, full_hi = 0;  // steps [t, t + 32) inside [full_lo, full_hi) need no masks
  float pc_sink = kNegInf;       // sink logit of row c
  auto finish = [&]() {
    const int b = sw.base + pc_bl;
    const int P = lane_of(sw.P, pc_bl), n = lane_of(sw.q.n, pc_bl);
    const bool final = P >= pc_u * L && P + n <= (pc_u + 1) * L;
    const int64_t slot = (int64_t)pc_u + b;
    float vsc[D / 16];  // integer pages: value scales of the lane's output dims
    if constexpr (INT) {
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
        vsc[j] = p.v_quant == PA_QUANT_PER_CHANNEL ? p.v_scale[(int64_t)pc_kh * D + (D / 16) * c + j]
                                                   : p.v_scale[0];
    }
    store_rows<MT, D, TT>(rs, p, pc_kh, lane_of(sw.q.s0, pc_bl), 0, g * lane_of(sw.q.nq, pc_bl), g,
                          c, G, pc_sink, final,
                          [&](int64_t, int, int rloc) { return (slot * p.kv_heads + pc_kh) * 16 + rloc; },
                          false, INT ? vsc : nullptr);
  };

  for (int k = 0; k < K; k += U) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      // Rows of step k+i+DEPTH-1 (block ids fetched BA-DEPTH+1 iterations ago), then the block
      // ids of step k+i+BA.
      const int sd_slot = (i + DEPTH - 1) % DEPTH;
      const int bt_use = (i + DEPTH - 1) % NBT, bt_load = (i + BA) % NBT;
      const int cs = i % DEPTH;  // ring slot of the step computed now
      load_stream_step<TT, D, CK>(p, sw, cd, btr[bt_use], lane, bs_shift, lofs, qp, qload,
                                  st[sd_slot], qr[sd_slot], skr[sd_slot]);
      if constexpr (BIAS) bias_load(qp.br, cd.t, G, braw[BIAS ? sd_slot : 0]);
      qload = cursor_next(cd, sw, p, hi, L, x, u0);
      if (qload) qp = query_ptrs<D, QL, BIAS>(p, sw, cd, g, lane);
      btr[bt_load] = load_step_blocks(p, sw, cb, lane, bs_shift);
      cursor_next(cb, sw, p, hi, L, x, u0);
      if (k + i < K) {
        if (cc.bl != pc_bl || cc.u != pc_u) {
          if (pc_bl >= 0) finish();
          pc_bl = cc.bl;
          pc_u = cc.u;
          pc_kh = cc.kh;
          pc_total = cc.total;
          pc_sink = p.head_sink ? TT::to_f32(skr[cs]) * kLog2e : (p.smooth_softmax ? 0.0f : kNegInf);
          const int nq = lane_of(sw.q.nq, cc.bl), pastb = lane_of(sw.q.pastb, cc.bl);
          const int R = g * nq;
          const bool rvalid = c < R;
          const int rpos = pastb + (rvalid ? c / g : 0);
          rs.vis_lo = p.window > 0 ? rpos - p.window + 1 : 0;
          rs.vis_hi = rvalid ? (p.causal ? rpos + 1 : pc_total) : -1;
          // Every valid row (positions pastb .. pastb + nq - 1) sees keys [full_lo, full_hi):
          // its window and, when causal, the keys up to itself.
          full_lo = p.window > 0 ? pastb + nq - p.window : 0;
          full_hi = p.causal ? min(pastb + 1, pc_total) : pc_total;
          if constexpr (INT)
            row_f = int_query<TT, D, CB == kDcI4>(rs, qr[cs], p, pc_kh, G, CB == kDcI8 ? 1152.f : 1032.f,
                                     koff);
          else
#pragma unroll
            for (int q = 0; q < D / 32; ++q) rs.qv[q] = __builtin_bit_cast(vec8, qr[cs][q]);
#pragma unroll
          for (int j = 0; j < D / 16; ++j) rs.o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
          rs.m_run = kNegInf;
          rs.l_part = 0.0f;
        }
        const int t0 = cc.t;
        const bool masked = !(t0 >= full_lo && t0 + 32 <= full_hi);
        // (generic: instantiated only for pages in the activation dtype, where it is called)
        auto run = [&](auto& cur, float ksA, float ksB, float vsA, float vsB) {
          if (t0 + 32 > pc_total) {
            // Value rows past the sequence end (re-read rows) take no part, even if not finite.
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int pos = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
              if (pos >= pc_total) cur.v[e] = VRow<D>{};
            }
          }
          compute_step<TT, D, CAP, false>(rs, cur, t0, pc_total, G, p.scale_log2, p.scale,
                                          p.softcap, ksA, ksB, vsA, vsB, masked);
        };
        float bx[8];  // BIAS: the step's bias in log2 units
        if constexpr (BIAS) bias_log2<TT>(braw[cs], bx);
        if constexpr (INT) {
          // Codes are finite: rows past the end weigh in with probability 0 as they are.
          auto& cur = st[cs];
          attend_step_ops<MT, D, CAP, true, true, false, true, BIAS>(
              rs,
              [&](int tile, int s) {
                if constexpr (CB == kDcI8) return key_operand_i8<D>(cur, tile, s);
                else return key_operand_i4<D>(cur, tile, s);
              },
              [&](int j) {
                if constexpr (CB == kDcI8) return value_operand_i8<D>(cur, j);
                else return value_operand_i4<D>(cur, j);
              },
              t0, pc_total, G, p.scale_log2, p.scale, p.softcap, row_f, row_f, 1.f, 1.f, masked,
              koff, bx);
        } else if constexpr (F8) {
          // Page scales of tiles A and B (lanes 0..3); a tile wholly past the end weighs zero
          // (its page id, and so its scale, is not a real one).
          Step8<D>& cur = st[cs];
          const int sc = __builtin_bit_cast(int, cur.sc);
          const bool b_live = t0 + 16 < pc_total;
          if (t0 + 32 > pc_total) {
            // Value rows past the sequence end (re-read rows) take no part, even if not finite.
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int pos = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
              if (pos >= pc_total) cur.v[e] = RawV8<D>{};
            }
          }
          attend_step_ops<TT, D, CAP, true>(
              rs, [&](int tile, int s) { return key_operand8<TT, D>(cur, tile, s); },
              [&](int j) { return value_operand8<TT, D>(cur, j); }, t0, pc_total, G,
              p.scale_log2, p.scale, p.softcap,
              __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc, 0)),
              b_live ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc, 1)) : 0.f,
              __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc, 2)),
              b_live ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc, 3)) : 0.f, masked);
        } else if constexpr (BIAS) {
          Step<D>& cur = st[cs];
          clear_tail_rows<D>(cur, t0, pc_total, G);
          attend_step_ops<TT, D, CAP, false, true, true, false, true>(
              rs, [&](int tile, int s) { return __builtin_bit_cast(vec8, cur.k[tile][s]); },
              [&](int j) { return value_operand<TT, D>(cur, j); }, t0, pc_total, G, p.scale_log2,
              p.scale, p.softcap, 1.f, 1.f, 1.f, 1.f, masked, 0.0f, bx);
        } else {
          run(st[cs], 1.f, 1.f, 1.f, 1.f);
        }
        cursor_next(cc, sw, p, hi, L, x, u0);
      }
    }
  }
  if (pc_bl >= 0) finish();
}

// Decode with at most 16 grouped query rows per sequence.  Every sequence contributes
// n_b = ceil((total_b - first_b) / 32) steps of 32 keys (first_b: first key any row can see); the
// steps of all sequences, in order, are cut into p.max_splits sub-segments of L = ceil(S /
// max_splits) steps (empty ones only at the end).  Sub-segment u of kv-head h is walked by
// wavefront (x, seg) with seg = u / mix and x = (h - u % mix) mod kv_heads: each wavefront walks
// `mix` consecutive sub-segments, each for the next kv-head, so every wavefront reads the same
// share of every kv-head's bytes (whose HBM speed differs by their address) and all finish
// together.  A sequence inside one sub-segment is written directly; otherwise each covering
// sub-segment u writes a partial at slot u + b (unique: the sub-segments of b are consecutive
// and the next sequence starts in the one where b ends or later), merged by
// balanced_merge_kernel.
// Ring depth (steps held in registers) of the streaming decode.  bf16/fp16 pages: 2 -- each step
// is 16 KiB per wavefront, and the smaller ring needs fewer registers (C3 attention launch
// 179 us against 185 us at depth 3).  Head 256: 1 (a 32 KiB step; depth 2 spills ~80 registers
// and measured 378 us against 359 us on the C3 batch at head 256).  fp8 pages: 3 (8 KiB steps;
// depths 2-5 measured within noise of each other).
#ifndef PA_DECODE_DEPTH
#define PA_DECODE_DEPTH 2
#endif
#ifndef PA_DECODE_DEPTH8
#define PA_DECODE_DEPTH8 3
#endif
// int4 pages: 2 -- with two wavefronts per SIMD (decode_waves) the smaller ring holds as many
// bytes in flight per SIMD and needs fewer registers (C3 batch 99.1 -> 97.4 us per launch).
#ifndef PA_DECODE_DEPTH_I4
#define PA_DECODE_DEPTH_I4 2
#endif
#ifndef PA_DECODE_DEPTH_I8
#define PA_DECODE_DEPTH_I8 3
#endif
template <typename TT, int D, bool CAP, int CK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    (CK & kDcBias) ? 1 : decode_waves(decode_cache_dtype(CK), D),
    (CK & kDcBias) ? 1 : decode_waves(decode_cache_dtype(CK), D)))) void
decode_balanced_kernel(const AttnParams p) {
  // Workgroup = W wavefronts (one per SIMD of a CU) for W consecutive kv-heads of one segment:
  // the kv-head slices of each page row are then fetched through one CU together, which the
  // memory system serves measurably faster than the same slices fetched from W different CUs.
  const int W = blockDim.x >> 6;
  const int nx = p.kv_heads / W;             // head groups
  const int nseg = p.max_splits / p.mix;     // segments; the grid holds nx * nseg workgroups
  // Workgroups go round-robin to the 8 XCDs (id % 8).  Runs of 8 consecutive ids share a head
  // group, so every XCD serves every head group: with the head group as the fastest index the
  // groups were tied to one XCD parity each, and the odd-XCD half finished ~5 us later.
  const int id = blockIdx.x;
  int hg, seg;
  if (nseg % 8 == 0) {
    hg = (id >> 3) % nx;
    seg = ((id >> 3) / nx) * 8 + (id & 7);
  } else {
    hg = id % nx;
    seg = id / nx;
  }
  // The wavefront index is wave-uniform; readfirstlane tells the compiler, so the kv-head and
  // every page address derived from it stay in scalar registers.
  const int x = __builtin_amdgcn_readfirstlane(hg * W + (int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int M = p.mix;
  // Step counts fit 32 bits: sequences are clamped to the cache capacity and the host bounds
  // batch * (capacity / 32 + 1) below 2^31.
  const int64_t S = total_steps(p, lane);
  if (S <= 0) return;
  const int L = (int)seg_len(S, p.max_splits);
  const int u0 = seg * M;
  const int gs = (int)min(S, (int64_t)L * u0), ge = (int)min(S, (int64_t)L * (u0 + M));
  if (gs >= ge) return;
  int carry = 0;
  for (int base = 0; base < p.batch && carry < ge; base += 64) {
    SeqWin sw;
    sw.base = base;
    sw.q = seq_steps(p, base + lane);
    const int incl = wave_incl_scan(sw.q.n, lane);
    sw.P = carry + (incl - sw.q.n);
    const int chunk_total = __builtin_amdgcn_readlane(incl, 63);
    const int lo = max(gs, carry), hi = min(ge, carry + chunk_total);
    if (lo < hi)
      stream_range<TT, D, CAP, CK, (CK & 3) == kDcI4 ? PA_DECODE_DEPTH_I4 : (CK & 3) == kDcI8 ? PA_DECODE_DEPTH_I8 : (CK & 3) != kDcT ? PA_DECODE_DEPTH8 : (D > 128 ? 1 : PA_DECODE_DEPTH)>(p, sw, lo, hi, L, x,
                                                                           u0, lane);
    carry += chunk_total;
  }
}

// Merge the partials of every (kv-head, sequence) split across segments (one workgroup each).
// A device-scope fence per piece inside the decode kernel (to let the last piece merge) writes
// back the XCD's L2 and measured far slower than this separate launch.
template <typename TT, int D>
__global__ __launch_bounds__(256) void balanced_merge_kernel(const AttnParams p) {
  const int kh = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int nseg = p.max_splits;
  const int g = p.num_heads / p.kv_heads;
  // Prefix of steps up to b, b's own metadata and the total, one parallel pass over sequences.
  int64_t S = 0, Pb = 0;
  int nb = 0, s0 = 0, nq = 0;
  for (int base = 0; base < p.batch; base += 64) {
    const SeqSteps q = seq_steps(p, base + lane);
    const int incl = wave_incl_scan(q.n, lane);
    if (b >= base && b < base + 64) {
      const int src = b - base;
      Pb = S + __shfl(incl - q.n, src, 64);
      nb = __shfl(q.n, src, 64);
      s0 = __shfl(q.s0, src, 64);
      nq = __shfl(q.nq, src, 64);
    }
    S += __shfl(incl, 63, 64);
  }
  if (nb <= 0 || S <= 0) return;
  const int64_t seg_l = seg_len(S, nseg);
  const int f = (int)(Pb / seg_l);
  const int nparts = (int)((Pb + nb - 1) / seg_l) - f + 1;
  if (nparts <= 1) return;  // written directly by the decode kernel
  merge_pieces<TT, D>(p, b, kh, s0, g * nq, g, f, nparts, (int)threadIdx.x);
}

template <typename TT, int D, bool CAP>
void launch_balanced_ck(const AttnParams& p, dim3 grid, dim3 block, int ck, hipStream_t s) {
  switch (ck) {
    case kDcFp8: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcFp8>), grid, block, 0, s, p); break;
    case kDcI8: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI8>), grid, block, 0, s, p); break;
    case kDcI4: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI4>), grid, block, 0, s, p); break;
    case kDcI8 | kDcLin: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI8 | kDcLin>), grid, block, 0, s, p); break;
    case kDcI4 | kDcLin: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI4 | kDcLin>), grid, block, 0, s, p); break;
    case kDcBias: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcBias>), grid, block, 0, s, p); break;
    case kDcI8 | kDcLin | kDcBias: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI8 | kDcLin | kDcBias>), grid, block, 0, s, p); break;
    case kDcI4 | kDcLin | kDcBias: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcI4 | kDcLin | kDcBias>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((decode_balanced_kernel<TT, D, CAP, kDcT>), grid, block, 0, s, p); break;
  }
}

// ck: DecodeCache kind of the pages (the streaming decode); the chunked kernel takes kDcT only.
template <typename TT, int D>
hipError_t launch_d(const AttnParams& p, dim3 grid, dim3 block, bool balanced, int ck,
                    hipStream_t s) {
  if constexpr (D != 64 && D != 128) {
    // Heads 96 / 256: the streaming decode on pages in the activation dtype only.
    if (!balanced || (ck != kDcT && ck != kDcBias)) return hipErrorInvalidValue;
    if (ck == kDcBias) {
      if (p.softcap > 0.0f)
        hipLaunchKernelGGL((decode_balanced_kernel<TT, D, true, kDcBias>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((decode_balanced_kernel<TT, D, false, kDcBias>), grid, block, 0, s, p);
    } else if (p.softcap > 0.0f) {
      hipLaunchKernelGGL((decode_balanced_kernel<TT, D, true, kDcT>), grid, block, 0, s, p);
    } else {
      hipLaunchKernelGGL((decode_balanced_kernel<TT, D, false, kDcT>), grid, block, 0, s, p);
    }
    return hipGetLastError();
  } else if (balanced) {
    if (p.softcap > 0.0f)
      launch_balanced_ck<TT, D, true>(p, grid, block, ck, s);
    else
      launch_balanced_ck<TT, D, false>(p, grid, block, ck, s);
  } else if (p.ng > 1) {
    // NG row groups per wavefront: 4 at d=64, 2 at d=128 (what fits the register file).
    constexpr int NG = D == 64 ? 4 : 2;
    if (p.softcap > 0.0f)
      hipLaunchKernelGGL((decode_chunked_kernel<TT, D, true, NG>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((decode_chunked_kernel<TT, D, false, NG>), grid, dim3(64), 0, s, p);
  } else {
    if (p.softcap > 0.0f)
      hipLaunchKernelGGL((decode_chunked_kernel<TT, D, true, 1>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((decode_chunked_kernel<TT, D, false, 1>), grid, dim3(64), 0, s, p);
  }
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_t(const AttnParams& p, dim3 grid, dim3 block, bool balanced, int ck,
                    hipStream_t s) {
  switch (p.head_dim) {
    case 64: return launch_d<TT, 64>(p, grid, block, balanced, ck, s);
    case 96: return launch_d<TT, 96>(p, grid, block, balanced, ck, s);
    case 128: return launch_d<TT, 128>(p, grid, block, balanced, ck, s);
    case 256: return launch_d<TT, 256>(p, grid, block, balanced, ck, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool balanced_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype, int block_size) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (head_dim != 64 && head_dim != 96 && head_dim != 128 && head_dim != 256) return false;
  if (block_size <= 0 || (block_size & (block_size - 1)) != 0) return false;
  if (cache_dtype == act) return true;
  // byte-coded pages (fp8, int8, int4): 16-key tiles inside one page, heads 64 / 128
  return (cache_dtype == PA_DTYPE_FP8_E4M3 || cache_dtype == PA_DTYPE_INT8 ||
          cache_dtype == PA_DTYPE_INT4) &&
         block_size >= 16 && (head_dim == 64 || head_dim == 128);
}

bool decode_mfma_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (cache_dtype != act) return false;
  return head_dim == 64 || head_dim == 128;
}

// Chunked launch (p.max_splits chunks of p.chunk keys): any number of query rows.
hipError_t launch_decode_mfma(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                              hipStream_t s) {
  if (!decode_mfma_supported(p.head_dim, act, cache_dtype)) return hipErrorInvalidValue;
  if (p.linear_cap > 0) return hipErrorInvalidValue;  // paged caches only
  if (p.batch <= 0) return hipSuccess;
  const int g = p.num_heads / p.kv_heads;
  const int mq = p.max_query_len > 0 ? p.max_query_len : p.num_tokens;
  if (p.ng != 1 && p.ng != (p.head_dim == 64 ? 4 : 2)) return hipErrorInvalidValue;
  const int rows_per_wave = 16 * p.ng;
  const int row_groups = (int)std::min<int64_t>(((int64_t)g * mq + rows_per_wave - 1) / rows_per_wave,
                                                (int64_t)(INT32_MAX / p.kv_heads));
  dim3 grid(p.kv_heads * row_groups, p.max_splits, p.batch);
  if (act == PA_DTYPE_FLOAT16) return launch_t<TF16>(p, grid, dim3(64), false, kDcT, s);
  return launch_t<TBF16>(p, grid, dim3(64), false, kDcT, s);
}

// The partial merge of the balanced decode, for the head size of the decode launch.
template <typename TT>
hipError_t launch_merge(const AttnParams& p, hipStream_t s) {
  const dim3 grid(p.kv_heads, p.batch), block(256);
  switch (p.head_dim) {
    case 64: hipLaunchKernelGGL((balanced_merge_kernel<TT, 64>), grid, block, 0, s, p); break;
    case 96: hipLaunchKernelGGL((balanced_merge_kernel<TT, 96>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((balanced_merge_kernel<TT, 128>), grid, block, 0, s, p); break;
    case 256: hipLaunchKernelGGL((balanced_merge_kernel<TT, 256>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Balanced launch: p.max_splits holds the segment count; every sequence must have at most 16
// grouped query rows (g * query length <= 16).  Launches the decode and the partial merge.
hipError_t launch_decode_balanced(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                                  hipStream_t s) {
  if (!balanced_supported(p.head_dim, act, cache_dtype, p.block_size)) return hipErrorInvalidValue;
  int ck = cache_dtype == PA_DTYPE_FP8_E4M3 ? kDcFp8
           : cache_dtype == PA_DTYPE_INT8   ? kDcI8
           : cache_dtype == PA_DTYPE_INT4   ? kDcI4
                                            : kDcT;
  const bool coded = ck != kDcT;
  if (coded != (p.read_all_from_cache != 0)) return hipErrorInvalidValue;
  // contiguous caches: in the activation dtype or integer codes (GroupQueryAttention presents)
  if (coded && (p.k_scale == nullptr || p.v_scale == nullptr ||
                (p.linear_cap > 0 && ck == kDcFp8)))
    return hipErrorInvalidValue;
  if (ck >= kDcI8 && p.linear_cap > 0) ck |= kDcLin;
  // an additive bias (GroupQueryAttention): caches in the activation dtype or integer codes
  if (p.bias != nullptr) {
    if (ck == kDcFp8 || (ck >= kDcI8 && p.linear_cap <= 0)) return hipErrorInvalidValue;
    ck |= kDcBias;
  }
  if ((ck & 3) >= kDcI8 && ((p.k_quant != PA_QUANT_PER_TENSOR && p.k_quant != PA_QUANT_PER_CHANNEL) ||
                      (p.v_quant != PA_QUANT_PER_TENSOR && p.v_quant != PA_QUANT_PER_CHANNEL)))
    return hipErrorInvalidValue;
  if (p.batch <= 0) return hipSuccess;
  if (p.part_o == nullptr || p.mix < 1 || p.mix > p.kv_heads || p.max_splits % p.mix != 0)
    return hipErrorInvalidValue;
  const int W = p.kv_heads % 4 == 0 ? 4 : p.kv_heads % 2 == 0 ? 2 : 1;
  dim3 grid((p.kv_heads / W) * (p.max_splits / p.mix)), block(64 * W);
  hipError_t e = (act == PA_DTYPE_FLOAT16) ? launch_t<TF16>(p, grid, block, true, ck, s)
                                           : launch_t<TBF16>(p, grid, block, true, ck, s);
  if (e != hipSuccess) return e;
  return act == PA_DTYPE_FLOAT16 ? launch_merge<TF16>(p, s) : launch_merge<TBF16>(p, s);
}

}  // namespace pa
