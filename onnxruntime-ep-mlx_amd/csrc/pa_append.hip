// pa_append.hip — fused Q/K RMSNorm + rotary embedding + KV append (reshape_and_cache).
//
// Replaces the reference's per-sequence MLX graph (attention.rs:4021-4120): split heads,
// mlx_fast_rms_norm (:4045-4049), rope_with_offset -> gqa_rope (:3812-3855, :459-503), the
// host-side slot rule (:4064-4079) and mlx_scatter_single into the flattened cache
// (:4080-4120).  One workgroup per packed token; one wavefront per head row.
//
// Bit-exactness: every rotary multiply / subtract / add rounds to the activation dtype on its
// own (the reference composes separate MLX ops in T), using integer RNE for bf16 and the IEEE
// v_cvt_f16_f32 for fp16; contraction into FMA is disabled for the fp32 variant.
// Duplicate slots: a token skips its write when any later token maps to the same slot, so the
// cache ends up holding the last token's row, as sequential scatter does.
// Integer caches (int8, int4 nibble pairs) store sat(RNE(x / scale)) codes of the final T row
// (QuantizedCache::encode, kv_cache.rs:170-219).

#include "pa_device.hpp"

#pragma clang fp contract(off)

namespace pa {
namespace {

// gqa_rope_f32 terms: fp32 products and their sum or difference, each rounded on its own (the
// pragma above keeps them apart; the HIP __f*_rn helpers are compiled outside it, and their
// products and sums were fused -- down to one fp16 rounding of a*c - b*s through v_fma_mix).
__device__ __forceinline__ float rot_sub32(float a, float c, float b, float s) {
  const float x = a * c, y = b * s;
  return x - y;
}
__device__ __forceinline__ float rot_add32(float a, float c, float b, float s) {
  const float x = a * c, y = b * s;
  return x + y;
}

template <typename TT>
__device__ __forceinline__ float ldv(const void* p, int64_t i) {
  return TT::to_f32(reinterpret_cast<const typename TT::raw*>(p)[i]);
}
template <typename TT>
__device__ __forceinline__ void stv(void* p, int64_t i, float v) {
  reinterpret_cast<typename TT::raw*>(p)[i] = TT::from_f32(v);
}
template <typename TT>
__device__ __forceinline__ float rnd(float v) {
  return TT::to_f32(TT::from_f32(v));
}

// Cache slot of logical position `logical` of sequence b; -1 when its block-table entry is
// out of range.
__device__ __forceinline__ int64_t slot_at(const AppendParams& p, int b, int64_t logical) {
  const int64_t bi = logical / p.block_size;
  if (bi < 0 || bi >= p.max_blocks) return -1;
  const int64_t blk = p.block_table[(int64_t)b * p.max_blocks + bi];
  if (blk < 0 || blk >= p.num_blocks) return -1;
  return blk * p.block_size + logical % p.block_size;
}


// Last-writer rule without a slot mapping: whether a later token writes `slot` (block blk =
// slot / bs, offset slot % bs) of token position `pos` in sequence b.  A later token u can only
// be a new position of sequence b (after pos) or of a later sequence whose block-table entry
// for u's block is blk, at offset slot % bs of that block -- so the workgroup scans the
// block-table entries that cover the new positions of sequences b.. (O(T / bs + B) per token)
// instead of every later token.  Called by the whole workgroup (256 threads).
__device__ bool later_block_dup(const AppendParams& p, int b, int64_t pos, int64_t slot) {
  constexpr int NT = 256;
  __shared__ int pre[NT + 1];   // prefix of block-entry counts over a chunk of sequences
  __shared__ int k0s[NT];       // first block index of each sequence's new positions
  __shared__ int64_t ps_s[NT];  // first new position (past, clamped at 0)
  __shared__ int n_s[NT];       // new-token count
  __shared__ int wsum[NT / 64];
  const int tid = threadIdx.x;
  const int64_t bs = p.block_size;
  const int64_t blk = slot / bs, off = slot % bs;
  bool dup = false;
  for (int base = b; base < p.batch; base += NT) {
    const int sq = base + tid;
    int k0 = 0, nk = 0, n = 0;
    int64_t ps = 0;
    if (sq < p.batch) {
      n = p.cum[sq + 1] - p.cum[sq];
      ps = (int64_t)max(p.past[sq], 0);
      if (n > 0) {
        const int64_t k1 = min((ps + n - 1) / bs, (int64_t)p.max_blocks - 1);
        k0 = (int)min(ps / bs, (int64_t)p.max_blocks);
        nk = k1 >= k0 ? (int)(k1 - k0 + 1) : 0;
      }
    }
    k0s[tid] = k0;
    ps_s[tid] = ps;
    n_s[tid] = n;
    // Inclusive scan of nk: wave scans, then the totals of the earlier wavefronts.
    int x = nk;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if ((tid & 63) >= o) x += y;
    }
    if ((tid & 63) == 63) wsum[tid >> 6] = x;
    __syncthreads();
    for (int w = 0; w < (tid >> 6); ++w) x += wsum[w];
    pre[tid + 1] = x;
    if (tid == 0) pre[0] = 0;
    __syncthreads();
    const int total = pre[NT];
    for (int j = tid; j < total; j += NT) {
      int lo = 0, hi = NT - 1;  // sequence i of entry j: pre[i] <= j < pre[i + 1]
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= j) lo = mid; else hi = mid - 1;
      }
      const int sq2 = base + lo;
      const int k = k0s[lo] + (j - pre[lo]);
      if ((int64_t)p.block_table[(int64_t)sq2 * p.max_blocks + k] == blk) {
        const int64_t pp = (int64_t)k * bs + off;
        if (pp >= ps_s[lo] && pp < ps_s[lo] + n_s[lo] && (sq2 > b || pp > pos)) dup = true;
      }
    }
    __syncthreads();  // the next chunk rewrites the tables
  }
  return __syncthreads_or(dup);
}

// Normalise + rotate one head row in place of `dst` (reads from src).  Executed by one wave.
// Destinations: dst/dst2 receive the row in T (either may be null); q8 (may be null) receives
// the fp8 code e4m3_sat(x / q8_scale), zero scale -> 0.
template <typename TT>
__device__ void process_row(const AppendParams& p, const void* src, int64_t src_base, void* dst,
                            int64_t dst_base, void* dst2, int64_t dst2_base, uint8_t* q8,
                            int64_t q8_base, float q8_scale, const void* norm_w, int64_t pos,
                            int lane) {
  const int D = p.head_dim;
  float inv = 1.0f;
  if (norm_w) {
    const float acc = sum_squares([&](int e) { return ldv<TT>(src, src_base + e); }, D, lane);
    inv = 1.0f / __builtin_sqrtf(acc / (float)D + p.norm_eps);
  }
  auto fetch = [&](int e) -> float {
    float v = ldv<TT>(src, src_base + e);
    if (norm_w) v = rnd<TT>(rnd<TT>(v * inv) * ldv<TT>(norm_w, e));
    return v;
  };
  auto put = [&](int e, float v) {
    if (dst) stv<TT>(dst, dst_base + e, v);
    if (dst2) stv<TT>(dst2, dst2_base + e, v);
    if (q8) q8[q8_base + e] = q8_scale == 0.0f ? 0 : (uint8_t)f32_to_e4m3_sat(v / q8_scale);
  };
  // A position outside the supplied cos/sin rows is rejected by host validation; unvalidated
  // calls copy such rows unrotated instead of reading past the cache.
  const int half = (p.cos_cache && pos >= 0 && pos < p.rotary_positions) ? p.rotary_half : 0;
  const int off = p.rotary_offset;
  for (int i = lane; i < half; i += 64) {
    float c = ldv<TT>(p.cos_cache, pos * half + i);
    float s = ldv<TT>(p.sin_cache, pos * half + i);
    int e1 = p.rotary_interleaved ? off + 2 * i : off + i;
    int e2 = p.rotary_interleaved ? off + 2 * i + 1 : off + half + i;
    float a = fetch(e1), b = fetch(e2);
    float o1, o2;
    if (p.rope_fp32) {  // each operation rounded to fp32, one rounding to T (gqa_rope_f32)
      o1 = rnd<TT>(rot_sub32(a, c, b, s));
      o2 = rnd<TT>(rot_add32(b, c, a, s));
    } else {
      o1 = rnd<TT>(rnd<TT>(a * c) - rnd<TT>(b * s));
      o2 = rnd<TT>(rnd<TT>(b * c) + rnd<TT>(a * s));
    }
    put(e1, o1);
    put(e2, o2);
  }
  // Elements outside the rotated range: plain copies.  16-bit rows with 16-byte aligned pieces
  // (e.g. the LATENT layout's 512 latent dims beside a 64-dim rotary range) move 8 elements per
  // lane and access, the bits unchanged; otherwise element by element.
  using raw = typename TT::raw;
  const int rot_lo = off, rot_hi = off + 2 * half;
  if (sizeof(raw) == 2 && !norm_w && !q8 && D % 8 == 0 && rot_lo % 8 == 0 && rot_hi % 8 == 0 &&
      ((src_base | dst_base | (dst2 ? dst2_base : 0)) & 7) == 0 &&
      ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
        reinterpret_cast<uintptr_t>(dst2)) & 15) == 0) {
    const raw* s16 = reinterpret_cast<const raw*>(src) + src_base;
    for (int e = 8 * lane; e < D; e += 512) {
      if (e >= rot_lo && e < rot_hi) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(s16 + e);
      if (dst) *reinterpret_cast<u32x4*>(reinterpret_cast<raw*>(dst) + dst_base + e) = v;
      if (dst2) *reinterpret_cast<u32x4*>(reinterpret_cast<raw*>(dst2) + dst2_base + e) = v;
    }
    return;
  }
  for (int e = lane; e < D; e += 64) {
    if (e >= off && e < off + 2 * half) continue;
    put(e, fetch(e));
  }
}

// Cache storage kinds of the append kernel.
enum CacheKind { kCacheT = 0, kCacheFp8 = 1, kCacheI8 = 2, kCacheI4 = 3 };

// Integer code of x (QuantizedCache::encode, kv_cache.rs:170-199): paged caches divide by the
// scale and store 0 for a zero scale; GroupQueryAttention caches multiply by the fp32
// reciprocal with a zero scale read as 1.  Then clip to the code range and round half to even
// (the clip bounds are integers, so clip-then-round equals round-then-clip).  NaN -> 0.
__device__ __forceinline__ int int_code(float x, float s, bool reciprocal, float lo, float hi) {
  float y;
  if (reciprocal) {
    const float r = 1.0f / (s == 0.0f ? 1.0f : s);
    y = x * r;
  } else {
    y = s == 0.0f ? 0.0f : x / s;
  }
  if (y != y) return 0;
  return (int)__builtin_rintf(fminf(fmaxf(y, lo), hi));
}

// Integer-cache row writer.  Each output element's final value (normalised, rotated, rounded
// to T exactly as process_row does) is recomputed by the lane that stores it, so an int4 byte
// (two channels) needs no exchange between lanes.  out (may be null) receives the T row.
template <typename TT, int CK>
__device__ void int_row(const AppendParams& p, const void* src, int64_t sbase, void* out,
                        int64_t obase, uint8_t* cache, int64_t cbase, const float* sc,
                        bool per_channel, int kh, const void* norm_w, bool rotate,
                        int64_t pos, int lane) {
  const int D = p.head_dim;
  float inv = 1.0f;
  if (norm_w) {
    const float acc = sum_squares([&](int e) { return ldv<TT>(src, sbase + e); }, D, lane);
    inv = 1.0f / __builtin_sqrtf(acc / (float)D + p.norm_eps);
  }
  const int half =
      (rotate && p.cos_cache && pos >= 0 && pos < p.rotary_positions) ? p.rotary_half : 0;
  const int off = p.rotary_offset;
  auto fetch = [&](int e) -> float {
    float v = ldv<TT>(src, sbase + e);
    if (norm_w) v = rnd<TT>(rnd<TT>(v * inv) * ldv<TT>(norm_w, e));
    return v;
  };
  auto value = [&](int e) -> float {
    const int r = e - off;
    if (r < 0 || r >= 2 * half) return fetch(e);
    const bool first = p.rotary_interleaved ? (r & 1) == 0 : r < half;
    const int i = p.rotary_interleaved ? (r >> 1) : (first ? r : r - half);
    const int e1 = p.rotary_interleaved ? off + 2 * i : off + i;
    const int e2 = p.rotary_interleaved ? off + 2 * i + 1 : off + half + i;
    const float c = ldv<TT>(p.cos_cache, pos * half + i);
    const float s = ldv<TT>(p.sin_cache, pos * half + i);
    const float a = fetch(e1), b = fetch(e2);
    if (p.rope_fp32)
      return first ? rnd<TT>(rot_sub32(a, c, b, s)) : rnd<TT>(rot_add32(b, c, a, s));
    return first ? rnd<TT>(rnd<TT>(a * c) - rnd<TT>(b * s))
                 : rnd<TT>(rnd<TT>(b * c) + rnd<TT>(a * s));
  };
  const bool recip = p.quant_reciprocal != 0;
  const float s0 = (cache && !per_channel) ? sc[0] : 0.0f;
  auto scale_of = [&](int e) -> float { return per_channel ? sc[(int64_t)kh * D + e] : s0; };
  if (CK == kCacheI4) {
    const int W = (D + 1) >> 1;
    for (int j = lane; j < W; j += 64) {
      const int e0 = 2 * j, e1 = 2 * j + 1;
      const float v0 = value(e0);
      const float v1 = e1 < D ? value(e1) : 0.0f;
      if (out) {
        stv<TT>(out, obase + e0, v0);
        if (e1 < D) stv<TT>(out, obase + e1, v1);
      }
      if (cache) {
        const int c0 = int_code(v0, scale_of(e0), recip, -8.0f, 7.0f) + 8;
        const int c1 = e1 < D ? int_code(v1, scale_of(e1), recip, -8.0f, 7.0f) + 8 : 8;
        cache[cbase + j] = (uint8_t)(c0 | (c1 << 4));
      }
    }
  } else {
    for (int e = lane; e < D; e += 64) {
      const float v = value(e);
      if (out) stv<TT>(out, obase + e, v);
      if (cache) cache[cbase + e] = (uint8_t)(int8_t)int_code(v, scale_of(e), recip, -128.0f, 127.0f);
    }
  }
}

template <typename TT, int CK>
__global__ __launch_bounds__(256) void rotary_append_kernel(const AppendParams p) {
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool linear = p.linear_cap > 0;
  int seq_b;
  int64_t pos, rpos;      // storage position, rotary position
  bool kv_store = true;   // GroupQueryAttention: this row is one of the stored new rows
  if (linear) {
    // GroupQueryAttention: [batch, seq] query rows at query_past + j, query_past =
    // max(length - seq, 0); the first length - query_past key/value rows are stored there.
    seq_b = t / p.gqa_seq;
    const int j = t % p.gqa_seq;
    const int len = p.seqlens_k[seq_b] + 1;
    const int qp = max(len - p.gqa_seq, 0);
    pos = (int64_t)qp + j;
    kv_store = p.gqa_kv_rows != 0 && j < len - qp;
    rpos = pos;
    if (p.ring_cap > 0) {  // sliding_window_cache: row before + j of the staged view
      const RingGeom rg = ring_geom(len, p.gqa_seq, p.ring_cap, p.ring_window);
      pos = (int64_t)rg.before + j;
      rpos = (int64_t)rg.p + j;
      kv_store = p.gqa_kv_rows != 0;
    }
    if (p.position_ids)
      rpos = p.pos_offset_form ? p.position_ids[0] + j
                               : p.position_ids[(int64_t)seq_b * p.gqa_seq + j];
    if (p.meta_out && t == 0 && blockIdx.y == 0)
      for (int i = threadIdx.x; i <= p.batch; i += blockDim.x) {
        p.meta_out[kMetaCum + i] = i * p.gqa_seq;  // cum
        if (i < p.batch) {
          const int li = p.seqlens_k[i] + 1;
          if (p.ring_cap > 0) {
            const RingGeom rg = ring_geom(li, p.gqa_seq, p.ring_cap, p.ring_window);
            p.meta_out[meta_past(p.batch) + i] = rg.before;                 // past (view rows)
            p.meta_out[meta_keys(p.batch) + i] = rg.before + p.gqa_seq;     // key count
            p.meta_out[meta_colofs(p.batch) + i] = rg.p - rg.before;        // bias column offset
          } else {
            p.meta_out[meta_past(p.batch) + i] = max(li - p.gqa_seq, 0);  // past (query_past)
            p.meta_out[meta_keys(p.batch) + i] = li;                       // key count
          }
        }
      }
  } else {
    const SeqPos sp = seq_pos_of_token(p.cum, p.past, p.batch, t);
    seq_b = sp.b;
    pos = (int64_t)max(sp.past, 0) + (t - sp.start);
    rpos = pos;
  }
  const int D = p.head_dim;
  const bool transform = p.cos_cache != nullptr || p.q_norm != nullptr || p.copy_rows;

  // Workgroups with blockIdx.y >= 1 take four query head rows each, one per wavefront, so
  // every head row of every token is in flight at once.
  if (blockIdx.y > 0) {
    const int h = (blockIdx.y - 1) * 4 + wave;
    if (p.do_q && transform && h < p.num_heads)
      process_row<TT>(p, p.query, (int64_t)t * p.q_ld + (int64_t)h * D, p.q_out,
                      ((int64_t)t * p.num_heads + h) * D, nullptr, 0, nullptr, 0, 0.0f,
                      p.q_norm, rpos, lane);
    return;
  }
  if (linear && p.gqa_kv_rows == 0) return;  // no new key/value rows in this call

  // blockIdx.y == 0: this token's key/value rows.  Cache slot and last-writer rule first.
  int64_t slot;
  if (linear)  // rows of one (b, kv-head) are distinct
    slot = (kv_store && pos >= 0 && pos < p.linear_cap) ? pos : -1;
  else
    slot = p.slot_mapping ? (int64_t)p.slot_mapping[t] : slot_at(p, seq_b, pos);
  if (!linear && slot >= p.num_blocks * p.block_size) slot = -1;
  bool later_dup = false;
  if (slot >= 0 && !p.slots_distinct && !linear) {
    if (p.slot_mapping) {
      for (int u = t + 1 + threadIdx.x; u < p.num_tokens; u += blockDim.x)
        if ((int64_t)p.slot_mapping[u] == slot) later_dup = true;
    } else {
      later_dup = later_block_dup(p, seq_b, pos, slot);
    }
  }
  const bool write_cache = slot >= 0 && !__syncthreads_or(later_dup);

  // 3. key rows: transform into k_out and/or the cache row; value rows: copy / quantise
  // Cache row width per kv-head in storage units: int4 packs two channels per byte.
  const int Dc = CK == kCacheI4 ? (D + 1) >> 1 : D;
  const int64_t crow = (int64_t)p.kv_heads * Dc;
  // LATENT layout: no value input and no value cache (values are read from the key rows).
  const bool write_v = write_cache && p.value != nullptr && p.value_cache != nullptr;
  void* const v_out = p.value != nullptr ? p.v_out : nullptr;
  // Plain copies (no rotary/norm, cache in the activation dtype, paged): the token's key row
  // and value row -- all kv-heads, contiguous in the input and in the slot -- move 16 bytes per
  // lane across the whole workgroup when every address is 16-byte aligned.
  bool copied = false;
  if (CK == kCacheT && !transform && !linear) {
    using raw = typename TT::raw;
    const int64_t row_bytes = (int64_t)p.kv_heads * D * (int64_t)sizeof(raw);
    const char* ks = reinterpret_cast<const char*>(p.key) + (int64_t)t * p.k_ld * sizeof(raw);
    const char* vs = p.value ? reinterpret_cast<const char*>(p.value) + (int64_t)t * p.v_ld * sizeof(raw)
                             : nullptr;
    char* kd = write_cache ? reinterpret_cast<char*>(p.key_cache) + slot * row_bytes : nullptr;
    char* vd = write_v ? reinterpret_cast<char*>(p.value_cache) + slot * row_bytes : nullptr;
    char* vo = v_out ? reinterpret_cast<char*>(v_out) + (int64_t)t * row_bytes : nullptr;
    const uintptr_t align = (uintptr_t)row_bytes | (uintptr_t)ks | (uintptr_t)vs | (uintptr_t)kd |
                            (uintptr_t)vd | (uintptr_t)vo;
    if ((align & 15) == 0) {
      for (int64_t o = (int64_t)threadIdx.x * 16; o < row_bytes; o += (int64_t)blockDim.x * 16) {
        if (kd) *reinterpret_cast<u32x4*>(kd + o) = *reinterpret_cast<const u32x4*>(ks + o);
        if (vd || vo) {
          const u32x4 x = *reinterpret_cast<const u32x4*>(vs + o);
          if (vd) *reinterpret_cast<u32x4*>(vd + o) = x;
          if (vo) *reinterpret_cast<u32x4*>(vo + o) = x;
        }
      }
      copied = true;
    }
  }
  for (int kh = wave; kh < p.kv_heads && !copied; kh += 4) {
    const int64_t kbase = (int64_t)t * p.k_ld + (int64_t)kh * D;
    const int64_t vbase = (int64_t)t * p.v_ld + (int64_t)kh * D;
    const int64_t obase = ((int64_t)t * p.kv_heads + kh) * D;  // k_out / v_out rows
    const int64_t cbase = linear ? (((int64_t)seq_b * p.kv_heads + kh) * p.linear_cap + slot) * Dc
                                 : slot * crow + (int64_t)kh * Dc;
    if (CK == kCacheT) {
      if (transform) {
        void* k_dst = p.k_out ? p.k_out : (write_cache ? p.key_cache : nullptr);
        int64_t k_base = p.k_out ? obase : cbase;
        void* k_dst2 = (p.k_out && write_cache) ? p.key_cache : nullptr;
        if (k_dst)
          process_row<TT>(p, p.key, kbase, k_dst, k_base, k_dst2, cbase, nullptr, 0, 0.0f,
                          p.k_norm, rpos, lane);
      } else if (write_cache) {
        const typename TT::raw* ks = reinterpret_cast<const typename TT::raw*>(p.key);
        typename TT::raw* kd = reinterpret_cast<typename TT::raw*>(p.key_cache);
        for (int e = lane; e < D; e += 64) kd[cbase + e] = ks[kbase + e];
      }
      if (write_v || v_out) {
        const typename TT::raw* vs = reinterpret_cast<const typename TT::raw*>(p.value);
        typename TT::raw* vd = reinterpret_cast<typename TT::raw*>(p.value_cache);
        typename TT::raw* vo = reinterpret_cast<typename TT::raw*>(v_out);
        for (int e = lane; e < D; e += 64) {
          const typename TT::raw x = vs[vbase + e];
          if (write_v) vd[cbase + e] = x;
          if (vo) vo[obase + e] = x;
        }
      }
    } else if (CK == kCacheFp8) {
      // fp8 cache: the (rotated) key row goes to k_out when transforming and is quantised
      // from registers; values are quantised from the input rows.
      const int64_t blk = write_cache ? slot / p.block_size : 0;
      const float ks = write_cache ? p.k_scale[blk * p.kv_heads + kh] : 0.0f;
      const float vsc = write_cache ? p.v_scale[blk * p.kv_heads + kh] : 0.0f;
      uint8_t* kd = write_cache ? reinterpret_cast<uint8_t*>(p.key_cache) : nullptr;
      uint8_t* vd = reinterpret_cast<uint8_t*>(p.value_cache);
      if (transform) {
        if (p.k_out || kd)
          process_row<TT>(p, p.key, kbase, p.k_out, obase, nullptr, 0, kd, cbase, ks, p.k_norm,
                          rpos, lane);
      } else if (write_cache) {
        for (int e = lane; e < D; e += 64) {
          float kx = ldv<TT>(p.key, kbase + e);
          kd[cbase + e] = ks == 0.0f ? 0 : (uint8_t)f32_to_e4m3_sat(kx / ks);
        }
      }
      if (write_v || v_out)
        for (int e = lane; e < D; e += 64) {
          float vx = ldv<TT>(p.value, vbase + e);
          if (write_v) vd[cbase + e] = vsc == 0.0f ? 0 : (uint8_t)f32_to_e4m3_sat(vx / vsc);
          if (v_out) stv<TT>(v_out, obase + e, vx);
        }
    } else {
      uint8_t* kd = write_cache ? reinterpret_cast<uint8_t*>(p.key_cache) : nullptr;
      uint8_t* vd = write_v ? reinterpret_cast<uint8_t*>(p.value_cache) : nullptr;
      if (kd || (transform && p.k_out))
        int_row<TT, CK>(p, p.key, kbase, transform ? p.k_out : nullptr, obase, kd, cbase,
                        p.k_scale, p.k_quant == PA_QUANT_PER_CHANNEL, kh, p.k_norm, true, rpos,
                        lane);
      if (vd || v_out)  // values are neither normalised nor rotated
        int_row<TT, CK>(p, p.value, vbase, v_out, obase, vd, cbase, p.v_scale,
                        p.v_quant == PA_QUANT_PER_CHANNEL, kh, nullptr, false, pos, lane);
    }
  }
}

// Plain append: no rotary or norm, cache in the activation dtype, paged, every token's slot
// distinct (no last-writer rule) and every row 16-byte aligned.  One wavefront per token: the
// key and value rows (all kv-heads, contiguous in the input and in the slot) are loaded 16
// bytes per lane before the slot lookup resolves, then stored; up to kCopyChunks * 1 KiB per row.
constexpr int kCopyChunks = 4;
__global__ __launch_bounds__(256) void copy_append_kernel(const AppendParams p, int row_bytes) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= p.num_tokens) return;  // whole wavefront
  const char* ks = reinterpret_cast<const char*>(p.key) + (int64_t)t * p.k_ld * 2;
  const char* vs = reinterpret_cast<const char*>(p.value) + (int64_t)t * p.v_ld * 2;
  u32x4 kr[kCopyChunks], vr[kCopyChunks];
#pragma unroll
  for (int i = 0; i < kCopyChunks; ++i) {
    const int o = (i * 64 + lane) * 16;
    if (o < row_bytes) {
      kr[i] = *reinterpret_cast<const u32x4*>(ks + o);
      vr[i] = *reinterpret_cast<const u32x4*>(vs + o);
    }
  }
  const SeqPos sp = seq_pos_of_token(p.cum, p.past, p.batch, t);
  const int64_t pos = (int64_t)max(sp.past, 0) + (t - sp.start);
  int64_t slot = p.slot_mapping ? (int64_t)p.slot_mapping[t] : slot_at(p, sp.b, pos);
  if (slot >= p.num_blocks * p.block_size) slot = -1;
  if (slot < 0) return;
  char* kd = reinterpret_cast<char*>(p.key_cache) + slot * row_bytes;
  char* vd = reinterpret_cast<char*>(p.value_cache) + slot * row_bytes;
#pragma unroll
  for (int i = 0; i < kCopyChunks; ++i) {
    const int o = (i * 64 + lane) * 16;
    if (o < row_bytes) {
      *reinterpret_cast<u32x4*>(kd + o) = kr[i];
      *reinterpret_cast<u32x4*>(vd + o) = vr[i];
    }
  }
}

// Quantising append for byte-coded pages (int8, int4, fp8 e4m3): no rotary or norm, paged,
// every token's slot distinct, 16-bit activations, head_dim % 8 == 0.  One wavefront per token,
// lane l takes elements 8 l .. 8 l + 7 of each 512-element piece of the token's key and value rows
// (all kv-heads, contiguous in the input and in the slot): one 16-byte load per row, the codes
// of int_code / f32_to_e4m3_sat (the per-row kernel's arithmetic, so the bytes are identical),
// one 8-byte (int8, fp8) or 4-byte (int4) store.  The first piece's rows load before the slot
// lookup resolves.
template <typename TT, int CK>
__global__ __launch_bounds__(256) void quant_append_kernel(const AppendParams p) {
  static_assert(CK != kCacheT, "byte-coded pages");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= p.num_tokens) return;  // whole wavefront
  const int D = p.head_dim, n = p.kv_heads * D;
  using raw = typename TT::raw;
  const raw* ks = reinterpret_cast<const raw*>(p.key) + (int64_t)t * p.k_ld;
  const raw* vs = reinterpret_cast<const raw*>(p.value) + (int64_t)t * p.v_ld;
  u32x4 kx = u32x4{0u, 0u, 0u, 0u}, vx = kx;
  if (8 * lane < n) {
    kx = *reinterpret_cast<const u32x4*>(ks + 8 * lane);
    vx = *reinterpret_cast<const u32x4*>(vs + 8 * lane);
  }
  const SeqPos sp = seq_pos_of_token(p.cum, p.past, p.batch, t);
  const int64_t pos = (int64_t)max(sp.past, 0) + (t - sp.start);
  int64_t slot = p.slot_mapping ? (int64_t)p.slot_mapping[t] : slot_at(p, sp.b, pos);
  if (slot >= p.num_blocks * p.block_size) slot = -1;
  if (slot < 0) return;
  constexpr int EB = CK == kCacheI4 ? 4 : 8;  // code bytes per 8 elements
  uint8_t* kd = reinterpret_cast<uint8_t*>(p.key_cache) + slot * (int64_t)(n / 8 * EB);
  uint8_t* vd = reinterpret_cast<uint8_t*>(p.value_cache) + slot * (int64_t)(n / 8 * EB);
  const int64_t blk = slot / p.block_size;
  const bool recip = p.quant_reciprocal != 0;
  const bool kpc = p.k_quant == PA_QUANT_PER_CHANNEL, vpc = p.v_quant == PA_QUANT_PER_CHANNEL;
  for (int e0 = 8 * lane; e0 < n; e0 += 512) {
    if (e0 != 8 * lane) {
      kx = *reinterpret_cast<const u32x4*>(ks + e0);
      vx = *reinterpret_cast<const u32x4*>(vs + e0);
    }
    const int kh = e0 / D;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
      const u32x4 x = side ? vx : kx;
      const float* sc = side ? p.v_scale : p.k_scale;
      const bool pc = side ? vpc : kpc;
      uint32_t code[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = TT::to_f32((uint16_t)(x[i >> 1] >> (16 * (i & 1))));
        if constexpr (CK == kCacheFp8) {
          const float s8 = sc[blk * p.kv_heads + kh];
          code[i] = s8 == 0.0f ? 0u : f32_to_e4m3_sat(v / s8);
        } else {
          const float si = sc[pc ? e0 + i : 0];  // per channel: [kv_heads, D] = element order
          code[i] = CK == kCacheI4
                        ? (uint32_t)(int_code(v, si, recip, -8.0f, 7.0f) + 8)
                        : (uint32_t)(uint8_t)(int8_t)int_code(v, si, recip, -128.0f, 127.0f);
        }
      }
      uint8_t* dst = (side ? vd : kd) + e0 / 8 * EB;
      if constexpr (CK == kCacheI4) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w |= (code[2 * j] | (code[2 * j + 1] << 4)) << (8 * j);
        *reinterpret_cast<uint32_t*>(dst) = w;
      } else {
        u32x2 w = u32x2{0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i >> 2] |= (code[i] & 0xffu) << (8 * (i & 3));
        *reinterpret_cast<u32x2*>(dst) = w;
      }
    }
  }
}

}  // namespace

template <typename TT>
void launch_append_t(const AppendParams& p, pa_dtype cache_dtype, dim3 grid, dim3 block,
                     hipStream_t s) {
  switch (cache_dtype) {
    case PA_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL((rotary_append_kernel<TT, kCacheFp8>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_INT8:
      hipLaunchKernelGGL((rotary_append_kernel<TT, kCacheI8>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_INT4:
      hipLaunchKernelGGL((rotary_append_kernel<TT, kCacheI4>), grid, block, 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((rotary_append_kernel<TT, kCacheT>), grid, block, 0, s, p);
      break;
  }
}

// ------------------------------------------------------------------- sliding_window_cache rings
// Byte moves of the GroupQueryAttention ring (attention.rs:1139-1368), one workgroup per
// (sequence, kv-head, chunk of rows), 16 bytes per thread when rows are 16-byte multiples (else
// one byte).  stage: history rows [0, before) of the past ring -> rows [0, before) of the staged
// view (capacity cap + seq); present: rows [0, after) of the present ring <- view rows
// [seed, seed + after), rows [after, cap) <- zero codes (int4: 0x88).  The present may be the past
// buffer itself: the present pass runs after the attention, and reads only the view.
constexpr int kRingRowsPerGroup = 64;
template <bool V16>
__global__ __launch_bounds__(256) void ring_move_kernel(RingParams r) {
  const int bh = blockIdx.x, b = bh / r.kv_heads;
  const int len = r.seqlens_k[b] + 1;
  const RingGeom g = ring_geom(len, r.seq, r.cap, r.window);
  const int row0 = blockIdx.y * kRingRowsPerGroup;
  const int64_t rb = r.row_bytes;
  for (int side = 0; side < 2; ++side) {
    const char* src = side ? r.src_v : r.src_k;
    char* dst = side ? r.dst_v : r.dst_k;
    const int64_t spitch = (int64_t)(r.present ? r.cap + r.seq : r.cap) * rb;  // rows of a (b, kh)
    const int64_t dpitch = (int64_t)(r.present ? r.cap : r.cap + r.seq) * rb;
    src += bh * spitch;
    dst += bh * dpitch;
    // rows [row0, row1) of this group: stage copies [0, before); present copies [0, after) from
    // view row seed and zero-fills [after, cap)
    const int nrows = r.present ? r.cap : g.before;
    const int row1 = min(row0 + kRingRowsPerGroup, nrows);
    if (row0 >= row1) continue;
    const int copy_end = r.present ? min(row1, g.after) : row1;
    const int64_t soff = r.present ? (int64_t)g.seed * rb : 0;
    constexpr int U = V16 ? 16 : 1;
    const int64_t a0 = row0 * rb, a_copy = max((int64_t)copy_end * rb, a0), a1 = row1 * rb;
    for (int64_t o = a0 + (int64_t)threadIdx.x * U; o < a1; o += 256 * U) {
      if constexpr (V16) {
        u32x4 v = u32x4{r.zero, r.zero, r.zero, r.zero};
        if (o < a_copy) v = *reinterpret_cast<const u32x4*>(src + soff + o);
        *reinterpret_cast<u32x4*>(dst + o) = v;
      } else {
        dst[o] = o < a_copy ? src[soff + o] : (char)(r.zero & 0xff);
      }
    }
  }
}

hipError_t launch_ring_move(const RingParams& r, hipStream_t s) {
  if (r.batch <= 0 || r.kv_heads <= 0 || r.cap <= 0 || r.window <= 0 || r.window > r.cap ||
      r.seq <= 0 || r.row_bytes <= 0)
    return hipErrorInvalidValue;
  // rows of a group: present [0, cap); stage [0, before) with before <= cap
  const dim3 grid((unsigned)((int64_t)r.batch * r.kv_heads),
                  (r.cap + kRingRowsPerGroup - 1) / kRingRowsPerGroup);
  const uintptr_t al = (uintptr_t)r.src_k | (uintptr_t)r.src_v | (uintptr_t)r.dst_k |
                       (uintptr_t)r.dst_v | (uintptr_t)r.row_bytes;
  if ((al & 15) == 0)
    hipLaunchKernelGGL((ring_move_kernel<true>), grid, dim3(256), 0, s, r);
  else
    hipLaunchKernelGGL((ring_move_kernel<false>), grid, dim3(256), 0, s, r);
  return hipGetLastError();
}

hipError_t launch_rotary_append(const AppendParams& p, pa_dtype act, pa_dtype cache_dtype,
                                hipStream_t s) {
  if (p.num_tokens <= 0) return hipSuccess;
  const bool transform = p.cos_cache != nullptr || p.q_norm != nullptr || p.copy_rows;
  const int q_groups = (p.do_q && transform) ? (p.num_heads + 3) / 4 : 0;
  dim3 grid(p.num_tokens, 1 + q_groups), block(256);
  if (cache_dtype != act && cache_dtype != PA_DTYPE_FP8_E4M3 && cache_dtype != PA_DTYPE_INT8 &&
      cache_dtype != PA_DTYPE_INT4)
    return hipErrorInvalidValue;
  if (cache_dtype == act && act != PA_DTYPE_FLOAT32 && !transform && p.linear_cap <= 0 &&
      p.slots_distinct && p.key && p.value && p.key_cache && p.value_cache && !p.v_out) {
    // 16-bit elements: every row start (input stride, slot stride) must be 16-byte aligned.
    const int64_t row_bytes = (int64_t)p.kv_heads * p.head_dim * 2;
    const uintptr_t align = (uintptr_t)p.key | (uintptr_t)p.value | (uintptr_t)p.key_cache |
                            (uintptr_t)p.value_cache | (uintptr_t)(p.k_ld * 2) |
                            (uintptr_t)(p.v_ld * 2) | (uintptr_t)row_bytes;
    if ((align & 15) == 0 && row_bytes <= kCopyChunks * 64 * 16) {
      hipLaunchKernelGGL(copy_append_kernel, dim3((p.num_tokens + 3) / 4), dim3(256), 0, s, p,
                         (int)row_bytes);
      return hipGetLastError();
    }
  }
  const bool coded = cache_dtype == PA_DTYPE_INT8 || cache_dtype == PA_DTYPE_INT4 ||
                     cache_dtype == PA_DTYPE_FP8_E4M3;
  if (coded && (act == PA_DTYPE_FLOAT16 || act == PA_DTYPE_BFLOAT16) && !transform &&
      p.linear_cap <= 0 && p.slots_distinct && p.key && p.value && p.key_cache &&
      p.value_cache && p.k_scale && p.v_scale && !p.v_out && p.head_dim % 8 == 0) {
    // 16-byte input rows, 8-byte (int4: 4-byte) code rows
    const uintptr_t in_align = (uintptr_t)p.key | (uintptr_t)p.value | (uintptr_t)(p.k_ld * 2) |
                               (uintptr_t)(p.v_ld * 2);
    const uintptr_t out_align = (uintptr_t)p.key_cache | (uintptr_t)p.value_cache;
    if ((in_align & 15) == 0 && (out_align & (cache_dtype == PA_DTYPE_INT4 ? 3 : 7)) == 0) {
      const dim3 qg((p.num_tokens + 3) / 4);
      const bool h = act == PA_DTYPE_FLOAT16;
      switch (cache_dtype) {
        case PA_DTYPE_INT8:
          if (h) hipLaunchKernelGGL((quant_append_kernel<TF16, kCacheI8>), qg, dim3(256), 0, s, p);
          else hipLaunchKernelGGL((quant_append_kernel<TBF16, kCacheI8>), qg, dim3(256), 0, s, p);
          break;
        case PA_DTYPE_INT4:
          if (h) hipLaunchKernelGGL((quant_append_kernel<TF16, kCacheI4>), qg, dim3(256), 0, s, p);
          else hipLaunchKernelGGL((quant_append_kernel<TBF16, kCacheI4>), qg, dim3(256), 0, s, p);
          break;
        default:
          if (h) hipLaunchKernelGGL((quant_append_kernel<TF16, kCacheFp8>), qg, dim3(256), 0, s, p);
          else hipLaunchKernelGGL((quant_append_kernel<TBF16, kCacheFp8>), qg, dim3(256), 0, s, p);
          break;
      }
      return hipGetLastError();
    }
  }
  switch (act) {
    case PA_DTYPE_FLOAT16: launch_append_t<TF16>(p, cache_dtype, grid, block, s); break;
    case PA_DTYPE_BFLOAT16: launch_append_t<TBF16>(p, cache_dtype, grid, block, s); break;
    case PA_DTYPE_FLOAT32: launch_append_t<TF32>(p, cache_dtype, grid, block, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pa
