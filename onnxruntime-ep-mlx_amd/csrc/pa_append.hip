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

#include "pa_device.hpp"

#pragma clang fp contract(off)

namespace pa {
namespace {

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

// Per-lane slot of token u (the last-writer scan; u differs between lanes).
__device__ __forceinline__ int64_t token_slot_lane(const AppendParams& p, int u) {
  if (p.slot_mapping) return (int64_t)p.slot_mapping[u];
  const int b = seq_of_token_lane(p.cum, p.batch, u);
  return slot_at(p, b, (int64_t)max(p.past[b], 0) + (u - p.cum[b]));
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
    float acc = 0.0f;
    for (int e = lane; e < D; e += 64) {
      float v = ldv<TT>(src, src_base + e);
      acc += v * v;
    }
    // Reduction order differs from a sequential sum; fp32 sums of <=256 squares of values that
    // are already in T agree with the sequential order to well under one T ulp of the result.
    acc = wave_sum(acc);
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
    float o1 = rnd<TT>(rnd<TT>(a * c) - rnd<TT>(b * s));
    float o2 = rnd<TT>(rnd<TT>(b * c) + rnd<TT>(a * s));
    put(e1, o1);
    put(e2, o2);
  }
  for (int e = lane; e < D; e += 64) {
    if (e >= off && e < off + 2 * half) continue;
    put(e, fetch(e));
  }
}

template <typename TT, bool FP8>
__global__ __launch_bounds__(256) void rotary_append_kernel(const AppendParams p) {
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool linear = p.linear_cap > 0;
  int seq_b;
  int64_t pos;
  if (linear) {
    // GroupQueryAttention: [batch, seq] query rows; past_b = seqlens_k[b] + 1 - seq.
    seq_b = t / p.gqa_seq;
    pos = (int64_t)p.seqlens_k[seq_b] + 1 - p.gqa_seq + (t % p.gqa_seq);
    if (p.meta_out && t == 0 && blockIdx.y == 0)
      for (int i = threadIdx.x; i <= p.batch; i += blockDim.x) {
        p.meta_out[i] = i * p.gqa_seq;  // cum
        if (i < p.batch) p.meta_out[p.batch + 1 + i] = max(p.seqlens_k[i] + 1 - p.gqa_seq, 0);
      }
  } else {
    const SeqPos sp = seq_pos_of_token(p.cum, p.past, p.batch, t);
    seq_b = sp.b;
    pos = (int64_t)max(sp.past, 0) + (t - sp.start);
  }
  const int D = p.head_dim;
  const bool transform = p.cos_cache != nullptr || p.q_norm != nullptr;


  // Workgroups with blockIdx.y >= 1 take four query head rows each, one per wavefront, so
  // every head row of every token is in flight at once.
  if (blockIdx.y > 0) {
    const int h = (blockIdx.y - 1) * 4 + wave;
    if (p.do_q && transform && h < p.num_heads) {
      int64_t base = ((int64_t)t * p.num_heads + h) * D;
      process_row<TT>(p, p.query, base, p.q_out, base, nullptr, 0, nullptr, 0, 0.0f, p.q_norm,
                      pos, lane);
    }
    return;
  }

  // blockIdx.y == 0: this token's key/value rows.  Cache slot and last-writer rule first.
  int64_t slot;
  if (linear)
    slot = (pos >= 0 && pos < p.linear_cap) ? pos : -1;  // rows of one (b, kv-head) are distinct
  else
    slot = p.slot_mapping ? (int64_t)p.slot_mapping[t] : slot_at(p, seq_b, pos);
  if (!linear && slot >= p.num_blocks * p.block_size) slot = -1;
  bool later_dup = false;
  if (slot >= 0 && !p.slots_distinct && !linear) {
    for (int u = t + 1 + threadIdx.x; u < p.num_tokens; u += blockDim.x)
      if (token_slot_lane(p, u) == slot) later_dup = true;
  }
  const bool write_cache = slot >= 0 && !__syncthreads_or(later_dup);

  // 3. key rows: transform into k_out and/or the cache row; value rows: copy / quantise
  const int64_t row = (int64_t)p.kv_heads * D;
  for (int kh = wave; kh < p.kv_heads; kh += 4) {
    int64_t sbase = (int64_t)t * row + (int64_t)kh * D;
    int64_t cbase = linear ? (((int64_t)seq_b * p.kv_heads + kh) * p.linear_cap + slot) * D
                           : slot * row + (int64_t)kh * D;
    if (!FP8) {
      if (transform) {
        void* k_dst = p.k_out ? p.k_out : (write_cache ? p.key_cache : nullptr);
        int64_t k_base = p.k_out ? sbase : cbase;
        void* k_dst2 = (p.k_out && write_cache) ? p.key_cache : nullptr;
        if (k_dst)
          process_row<TT>(p, p.key, sbase, k_dst, k_base, k_dst2, cbase, nullptr, 0, 0.0f,
                          p.k_norm, pos, lane);
      } else if (write_cache) {
        const typename TT::raw* ks = reinterpret_cast<const typename TT::raw*>(p.key);
        typename TT::raw* kd = reinterpret_cast<typename TT::raw*>(p.key_cache);
        for (int e = lane; e < D; e += 64) kd[cbase + e] = ks[sbase + e];
      }
      if (write_cache) {
        const typename TT::raw* vs = reinterpret_cast<const typename TT::raw*>(p.value);
        typename TT::raw* vd = reinterpret_cast<typename TT::raw*>(p.value_cache);
        for (int e = lane; e < D; e += 64) vd[cbase + e] = vs[sbase + e];
      }
    } else {
      // fp8 cache: the (rotated) key row goes to k_out when transforming and is quantised
      // from registers; values are quantised from the input rows.
      const int64_t blk = write_cache ? slot / p.block_size : 0;
      const float ks = write_cache ? p.k_scale[blk * p.kv_heads + kh] : 0.0f;
      const float vsc = write_cache ? p.v_scale[blk * p.kv_heads + kh] : 0.0f;
      uint8_t* kd = write_cache ? reinterpret_cast<uint8_t*>(p.key_cache) : nullptr;
      uint8_t* vd = reinterpret_cast<uint8_t*>(p.value_cache);
      if (transform) {
        if (p.k_out || kd)
          process_row<TT>(p, p.key, sbase, p.k_out, sbase, nullptr, 0, kd, cbase, ks, p.k_norm,
                          pos, lane);
      } else if (write_cache) {
        for (int e = lane; e < D; e += 64) {
          float kx = ldv<TT>(p.key, sbase + e);
          kd[cbase + e] = ks == 0.0f ? 0 : (uint8_t)f32_to_e4m3_sat(kx / ks);
        }
      }
      if (write_cache) {
        for (int e = lane; e < D; e += 64) {
          float vx = ldv<TT>(p.value, sbase + e);
          vd[cbase + e] = vsc == 0.0f ? 0 : (uint8_t)f32_to_e4m3_sat(vx / vsc);
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_rotary_append(const AppendParams& p, pa_dtype act, pa_dtype cache_dtype,
                                hipStream_t s) {
  if (p.num_tokens <= 0) return hipSuccess;
  const bool transform = p.cos_cache != nullptr || p.q_norm != nullptr;
  const int q_groups = (p.do_q && transform) ? (p.num_heads + 3) / 4 : 0;
  dim3 grid(p.num_tokens, 1 + q_groups), block(256);
  const bool fp8 = cache_dtype == PA_DTYPE_FP8_E4M3;
  switch (act) {
    case PA_DTYPE_FLOAT16:
      if (fp8)
        hipLaunchKernelGGL((rotary_append_kernel<TF16, true>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((rotary_append_kernel<TF16, false>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_BFLOAT16:
      if (fp8)
        hipLaunchKernelGGL((rotary_append_kernel<TBF16, true>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((rotary_append_kernel<TBF16, false>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_FLOAT32:
      if (fp8)
        hipLaunchKernelGGL((rotary_append_kernel<TF32, true>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((rotary_append_kernel<TF32, false>), grid, block, 0, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pa
