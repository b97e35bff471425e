// pa_attn_generic.hip — VALU paged attention for every dtype/shape, plus the split-K reduce.
//
// One wavefront per (packed query token, query head, context chunk).  Lanes split head_dim;
// each key costs one cross-lane sum.  This is the fp32 path (the ORT CPU GQA parity config)
// and the fallback for shapes the MFMA kernels do not cover, including integer (int8/int4)
// pages, whose keys/values are code * scale in fp32; it is not the hot path.
//
// Semantics restated from _paged_ref (test_paged_attention.py:127-155) and the dense
// fallback (attention.rs:4192-4319): positions < past read the cache pages through the block
// table, positions >= past read the new rows; causal keeps keys p <= past + row; a window keeps
// p >= past + row - window + 1; softcap s -> c*tanh(s/c); a head sink adds exp(sink) to the
// denominator only (attention_probs_with_sink :100-118).  Softmax runs in base 2 on
// x = s*log2(e), which is the same function.
#include <type_traits>

#include "pa_device.hpp"

namespace pa {

namespace {

// Element e of a cache row starting at storage index `base`, widened to fp32.  `scale` is the
// fp8 per-(block, kv-head) scale or the integer per-tensor / per-channel scale of element e.
template <typename CT>
struct CacheRead;

template <>
struct CacheRead<TF16> {
  __device__ static float at(const void* c, int64_t base, int e, float) {
    return f16_to_f32(reinterpret_cast<const uint16_t*>(c)[base + e]);
  }
};
template <>
struct CacheRead<TBF16> {
  __device__ static float at(const void* c, int64_t base, int e, float) {
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(c)[base + e]);
  }
};
template <>
struct CacheRead<TF32> {
  __device__ static float at(const void* c, int64_t base, int e, float) {
    return reinterpret_cast<const float*>(c)[base + e];
  }
};
struct Fp8Cache {};
template <>
struct CacheRead<Fp8Cache> {
  __device__ static float at(const void* c, int64_t base, int e, float scale) {
    return e4m3_to_f32(reinterpret_cast<const uint8_t*>(c)[base + e]) * scale;
  }
};
// Integer caches: QuantizedCache::decode (kv_cache.rs:222-256), code * scale in fp32.
struct I8Cache {};
template <>
struct CacheRead<I8Cache> {
  __device__ static float at(const void* c, int64_t base, int e, float scale) {
    return (float)reinterpret_cast<const int8_t*>(c)[base + e] * scale;
  }
};
struct I4Cache {};
template <>
struct CacheRead<I4Cache> {
  __device__ static float at(const void* c, int64_t base, int e, float scale) {
    const uint32_t byte = reinterpret_cast<const uint8_t*>(c)[base + (e >> 1)];
    return (float)((int)((byte >> ((e & 1) * 4)) & 15u) - 8) * scale;
  }
};

// Keys of sequence b: past + query rows, bounded by key_limit[b] when given (GroupQueryAttention
// sequences shorter than the query rows of a ragged first prompt) and by the capacity of a
// contiguous cache (unvalidated lengths never address another sequence's rows).
__device__ __forceinline__ int64_t seq_keys(const AttnParams& p, int b, int64_t pastb, int nq) {
  int64_t t = pastb + nq;
  if (p.key_limit) t = min(t, (int64_t)max(p.key_limit[b], 0));
  return p.linear_cap > 0 ? min(t, (int64_t)p.linear_cap) : t;
}

template <typename CT>
constexpr bool kIntCache = false;
template <>
constexpr bool kIntCache<I8Cache> = true;
template <>
constexpr bool kIntCache<I4Cache> = true;

// Elements per lane: NE = 4 covers head_dim <= 256, NE = 10 head_dim <= 640 (latent heads).
template <typename TT, typename CT, int NE>
__global__ __launch_bounds__(64) void attn_generic_kernel(const AttnParams p) {
  const int split = blockIdx.x, h = blockIdx.y, t = blockIdx.z;
  const int lane = threadIdx.x;
  const int D = p.head_dim;
  const int VD = p.v_head_dim;  // value / output head size (< D only for the LATENT layout)
  const int b = seq_of_token(p.cum, p.batch, t);
  const int s0 = p.cum[b];
  const int nq = p.cum[b + 1] - s0;
  const int64_t pastb = max(p.past[b], 0);
  const int64_t total = seq_keys(p, b, pastb, nq);
  const int64_t start = (int64_t)split * p.chunk;
  if (nq <= 0 || start >= total) return;
  const int64_t end = min(start + (int64_t)p.chunk, total);
  const int g = p.num_heads / p.kv_heads;
  const int kh = h / g;
  const int64_t rp = pastb + (t - s0);
  int64_t lo = start, hi = end;
  if (p.causal) hi = min(hi, rp + 1);
  // window end point: the row's position, or the last key for rows past it (a right-padded
  // first prompt, causal_window_mask attention.rs:328-353)
  if (p.window > 0) lo = max(lo, min(rp, total - 1) - p.window + 1);
  const typename TT::raw* bias_row =
      p.bias ? reinterpret_cast<const typename TT::raw*>(p.bias) +
                   ((((int64_t)(p.bias_b == 1 ? 0 : b) * p.bias_h + (p.bias_h == 1 ? 0 : h)) *
                         p.bias_rows + (t - s0)) * p.bias_cols)
             : nullptr;
  // bias column of key position pos: pos + the sequence's offset (sliding-window rings)
  const int64_t bias_off = p.bias_col_off ? p.bias_col_off[b] : 0;

  const int64_t row = (int64_t)p.kv_heads * D;
  // Cache rows in storage units: int4 holds two channels per byte.
  const int Dc = std::is_same<CT, I4Cache>::value ? (D + 1) >> 1 : D;
  const int64_t crow = (int64_t)p.kv_heads * Dc;
  float qv[NE], o[NE], ksv[NE], vsv[NE];
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    int e = lane + 64 * k;
    qv[k] = e < D ? TT::to_f32(reinterpret_cast<const typename TT::raw*>(
                        p.q)[((int64_t)t * p.num_heads + h) * D + e])
                  : 0.0f;
    o[k] = 0.0f;
    ksv[k] = vsv[k] = 1.0f;
    if (kIntCache<CT> && e < D) {
      ksv[k] = p.k_scale[p.k_quant == PA_QUANT_PER_CHANNEL ? (int64_t)kh * D + e : 0];
      vsv[k] = p.v_scale[p.v_quant == PA_QUANT_PER_CHANNEL ? (int64_t)kh * D + e : 0];
    }
  }
  float m = kNegInf, l = 0.0f;
  const float cap = p.softcap;
  for (int64_t pos = lo; pos < hi; ++pos) {
    const void *kb, *vb;
    int64_t off;
    float ks = 1.0f, vs = 1.0f;
    bool from_cache = pos < pastb || p.read_all_from_cache || p.linear_cap > 0;
    if (p.linear_cap > 0) {
      // contiguous [batch, kv_heads, cap, head_dim] cache holding the new rows too
      off = (((int64_t)b * p.kv_heads + kh) * p.linear_cap + pos) * Dc;
      kb = p.key_cache;
      vb = p.v_from_key ? p.key_cache : p.value_cache;
    } else if (from_cache) {
      int64_t bi = pos / p.block_size;
      int64_t blk = p.block_table[(int64_t)b * p.max_blocks + min(bi, (int64_t)p.max_blocks - 1)];
      blk = min(max(blk, (int64_t)0), p.num_blocks - 1);
      off = (blk * p.block_size + pos % p.block_size) * crow + (int64_t)kh * Dc;
      kb = p.key_cache;
      vb = p.v_from_key ? p.key_cache : p.value_cache;
      if (std::is_same<CT, Fp8Cache>::value) {
        ks = p.k_scale[blk * p.kv_heads + kh];
        vs = p.v_scale[blk * p.kv_heads + kh];
      }
    } else {
      int64_t tok = min(max((int64_t)s0 + (pos - pastb), (int64_t)0), (int64_t)p.num_tokens - 1);
      off = tok * row + (int64_t)kh * D;
      kb = p.k_new;
      vb = p.v_from_key ? p.k_new : p.v_new;
    }
    float part = 0.0f;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int e = lane + 64 * k;
      if (e < D) {
        float kv = from_cache ? CacheRead<CT>::at(kb, off, e, kIntCache<CT> ? ksv[k] : ks)
                              : TT::to_f32(reinterpret_cast<const typename TT::raw*>(kb)[off + e]);
        part += qv[k] * kv;
      }
    }
    float s = wave_sum(part) * p.scale;
    if (cap > 0.0f) s = cap * tanhf(s / cap);
    if (bias_row) s += TT::to_f32(bias_row[min(max(pos + bias_off, (int64_t)0), (int64_t)p.bias_cols - 1)]);
    float x = s * kLog2e;
    float mn = fmaxf(m, x);
    float alpha = (m == kNegInf) ? 0.0f : exp2f(m - mn);
    float w = exp2f(x - mn);
    l = l * alpha + w;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int e = lane + 64 * k;
      if (e < VD) {
        float vv = from_cache ? CacheRead<CT>::at(vb, off, e, kIntCache<CT> ? vsv[k] : vs)
                              : TT::to_f32(reinterpret_cast<const typename TT::raw*>(vb)[off + e]);
        o[k] = o[k] * alpha + w * vv;
      }
    }
    m = mn;
  }

  const bool single = (start == 0 && end == total);
  if (!single && p.part_o == nullptr) return;  // beyond planned capacity: nothing to write into
  if (single) {
    float f = finalize_factor(m, l, sink_logit<TT>(p, h));
    typename TT::raw* out = reinterpret_cast<typename TT::raw*>(p.out);
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int e = lane + 64 * k;
      if (e < VD) out[((int64_t)t * p.num_heads + h) * VD + e] = TT::from_f32(o[k] * f);
    }
  } else {
    int64_t pi = ((int64_t)t * p.num_heads + h) * p.max_splits + split;
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      int e = lane + 64 * k;
      if (e < VD) p.part_o[pi * D + e] = o[k];
    }
    if (lane == 0) {
      p.part_ml[pi * 2 + 0] = m;
      p.part_ml[pi * 2 + 1] = l;
    }
  }
}

#ifndef PA_MERGE_ROUND
#define PA_MERGE_ROUND 4  // eight per round measured slower
#endif

// Merge the per-chunk partials of one (token, head): global max, rescaled sums, divide.
// Partial rows have stride head_dim; outputs hold v_head_dim values per head.  A workgroup of
// NT threads (one or four wavefronts) per (head, token): thread x takes the value elements x,
// x + NT, ... (NE of them); with four wavefronts each thread's loads of a round of split rows
// are few and all in flight together (few (head, token) pairs), with one the workgroups are
// cheaper (many pairs).  Every wavefront computes the split weights itself (no exchange between
// them).  Each element sums its split rows in split order.
template <typename TT, int NE, int NT>
__global__ __launch_bounds__(NT) void split_reduce_kernel(const AttnParams p) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int D = p.head_dim;
  const int VD = p.v_head_dim;
  const int b = seq_of_token(p.cum, p.batch, t);
  const int nq = p.cum[b + 1] - p.cum[b];
  const int64_t total = seq_keys(p, b, max(p.past[b], 0), nq);
  if (nq <= 0) return;
  const int nsplit = (int)min((total + p.chunk - 1) / p.chunk, (int64_t)p.max_splits);
  if (nsplit <= 1) return;  // the attention kernel already wrote the final row
  const int64_t base = ((int64_t)t * p.num_heads + h) * p.max_splits;
  const float2* ml = reinterpret_cast<const float2*>(p.part_ml) + base;
  // Lanes hold the (m, l) of splits lane, lane+64, ...: one parallel load instead of a chain.
  float M = kNegInf;
  for (int s = lane; s < nsplit; s += 64) M = fmaxf(M, ml[s].x);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  float L = 0.0f;
  for (int s = lane; s < nsplit; s += 64) {
    const float2 v = ml[s];
    if (v.x != kNegInf) L += v.y * exp2f(v.x - M);
  }
  L = wave_sum(L);
  const float f = finalize_factor(M, L, sink_logit<TT>(p, h));
  typename TT::raw* out = reinterpret_cast<typename TT::raw*>(p.out);
  const float* po = p.part_o + base * D;
  float acc[NE];
#pragma unroll
  for (int q = 0; q < NE; ++q) acc[q] = 0.0f;
  for (int s0 = 0; s0 < nsplit; s0 += 64) {
    // every lane stays active through the shuffles: split weights live one per lane
    float wl = 0.0f;
    if (s0 + lane < nsplit) {
      const float ms = ml[s0 + lane].x;
      wl = (ms == kNegInf) ? 0.0f : exp2f(ms - M);
    }
    const int n = min(64, nsplit - s0);
    // PA_MERGE_ROUND split rows per round, their loads issued together
    constexpr int RND = PA_MERGE_ROUND;
    int k = 0;
    for (; k + RND <= n; k += RND) {
      float v[RND][NE];
#pragma unroll
      for (int u = 0; u < RND; ++u) {
        const float* row = po + (int64_t)(s0 + k + u) * D;
#pragma unroll
        for (int q = 0; q < NE; ++q) {
          const int e = tid + NT * q;
          v[u][q] = e < VD ? row[e] : 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < RND; ++u) {
        const float wk = __shfl(wl, k + u, 64);
#pragma unroll
        for (int q = 0; q < NE; ++q) acc[q] += v[u][q] * wk;
      }
    }
    for (; k < n; ++k) {
      const float wk = __shfl(wl, k, 64);
      const float* row = po + (int64_t)(s0 + k) * D;
#pragma unroll
      for (int q = 0; q < NE; ++q) {
        const int e = tid + NT * q;
        if (e < VD) acc[q] += row[e] * wk;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NE; ++q) {
    const int e = tid + NT * q;
    if (e < VD) out[((int64_t)t * p.num_heads + h) * VD + e] = TT::from_f32(acc[q] * f);
  }
}

// Lanes hold head_dim / 64 elements: 4 up to 256, 10 up to 640.
constexpr int kMaxHeadDim = 640;
template <int NE>
constexpr bool ne_covers(int d) { return d <= 64 * NE; }

template <typename TT, int NE>
hipError_t launch_generic_ne(const AttnParams& p, pa_dtype cache_dtype, hipStream_t s) {
  dim3 grid(p.max_splits, p.num_heads, p.num_tokens), block(64);
  switch (cache_dtype) {
    case PA_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL((attn_generic_kernel<TT, Fp8Cache, NE>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_INT8:
      hipLaunchKernelGGL((attn_generic_kernel<TT, I8Cache, NE>), grid, block, 0, s, p);
      break;
    case PA_DTYPE_INT4:
      hipLaunchKernelGGL((attn_generic_kernel<TT, I4Cache, NE>), grid, block, 0, s, p);
      break;
    default:
      if (cache_dtype != TT::code) return hipErrorInvalidValue;
      hipLaunchKernelGGL((attn_generic_kernel<TT, TT, NE>), grid, block, 0, s, p);
      break;
  }
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_generic_t(const AttnParams& p, pa_dtype cache_dtype, hipStream_t s) {
  return ne_covers<4>(p.head_dim) ? launch_generic_ne<TT, 4>(p, cache_dtype, s)
                                  : launch_generic_ne<TT, 10>(p, cache_dtype, s);
}

// ------------------------------------------------------------------------------ output_qk
// GroupQueryAttention's QK diagnostics (output 3, attention.rs:771-785, :833-839) over a
// contiguous present [batch, kv_heads, linear_cap, D]: row (b, h, i) of qk [batch, num_heads,
// seq, cols] holds, for key j < the sequence's key count, the score s_j = scale * q.k_j
// (softcapped, plus the bias) where row i sees key j (mode 1), or its probability
// exp(s_j - m) / (sum of the visible exp(s - m) + exp(sink - m)) (mode 2), and 0 everywhere else
// (masked keys, columns past the key count).  One workgroup per row, keys spread over the
// threads, each a full dot product in fp32 from the row in LDS; mode 2 takes a maxima-and-sums
// pass before the writing pass.  Rows sit at b * seq + i of q (seq = max_query_len); past[b] is
// the sequence's query_past and keys[b] its key count.
constexpr int kQkThreads = 256;
template <typename TT, typename CT>
__global__ __launch_bounds__(kQkThreads) void gqa_qk_kernel(const AttnParams p, void* qk, int mode,
                                                            int64_t cols, const int32_t* keys) {
  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int S = p.max_query_len, D = p.head_dim, g = p.num_heads / p.kv_heads, kh = h / g;
  __shared__ float qs[kMaxHeadDim];
  __shared__ float red_m[kQkThreads / 64], red_l[kQkThreads / 64];
  const int64_t t = (int64_t)b * S + i;
  for (int e = tid; e < D; e += kQkThreads)
    qs[e] = TT::to_f32(reinterpret_cast<const typename TT::raw*>(p.q)[(t * p.num_heads + h) * D + e]);
  __syncthreads();
  const int64_t qp = max(p.past[b], 0);
  const int64_t length = min((int64_t)max(keys[b], 0), (int64_t)p.linear_cap);
  int64_t hi = length, lo = 0;
  if (p.causal) hi = min(hi, qp + i + 1);
  if (p.window > 0) lo = max((int64_t)0, min(qp + i, length - 1) - p.window + 1);
  const int Dc = std::is_same<CT, I4Cache>::value ? (D + 1) >> 1 : D;
  const int64_t base0 = ((int64_t)b * p.kv_heads + kh) * p.linear_cap * Dc;
  const bool kpc = p.k_quant == PA_QUANT_PER_CHANNEL;
  const typename TT::raw* bias_row =
      p.bias ? reinterpret_cast<const typename TT::raw*>(p.bias) +
                   ((((int64_t)(p.bias_b == 1 ? 0 : b) * p.bias_h + (p.bias_h == 1 ? 0 : h)) *
                         p.bias_rows + i) * p.bias_cols)
             : nullptr;
  auto score = [&](int64_t j) {
    float dot = 0.0f;
    for (int e = 0; e < D; ++e) {
      const float ks = kIntCache<CT> ? p.k_scale[kpc ? (int64_t)kh * D + e : 0] : 1.0f;
      dot += qs[e] * CacheRead<CT>::at(p.key_cache, base0 + j * Dc, e, ks);
    }
    float sc = dot * p.scale;
    if (p.softcap > 0.0f) sc = p.softcap * tanhf(sc / p.softcap);
    if (bias_row) sc += TT::to_f32(bias_row[min(j, (int64_t)p.bias_cols - 1)]);
    return sc;
  };
  // mode 2: the row's maximum (with the sink) and denominator, in base 2
  float m = kNegInf, l = 0.0f;
  if (mode == 2) {
    for (int64_t j = lo + tid; j < hi; j += kQkThreads) {
      const float x = score(j) * kLog2e, mn = fmaxf(m, x);
      l = l * (m == kNegInf ? 0.0f : exp2f(m - mn)) + exp2f(x - mn);
      m = mn;
    }
    // combine (m, l) over the wavefront, then over the wavefronts
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float m2 = __shfl_xor(m, o, 64), l2 = __shfl_xor(l, o, 64), mn = fmaxf(m, m2);
      l = (mn == kNegInf) ? 0.0f
                          : l * (m == kNegInf ? 0.0f : exp2f(m - mn)) +
                                l2 * (m2 == kNegInf ? 0.0f : exp2f(m2 - mn));
      m = mn;
    }
    if ((tid & 63) == 0) red_m[tid >> 6] = m, red_l[tid >> 6] = l;
    __syncthreads();
    m = kNegInf;
    l = 0.0f;
    for (int w = 0; w < kQkThreads / 64; ++w) {
      const float mn = fmaxf(m, red_m[w]);
      l = (mn == kNegInf) ? 0.0f
                          : l * (m == kNegInf ? 0.0f : exp2f(m - mn)) +
                                red_l[w] * (red_m[w] == kNegInf ? 0.0f : exp2f(red_m[w] - mn));
      m = mn;
    }
    const float sk = sink_logit<TT>(p, h);
    const float mm = fmaxf(m, sk);
    l = (mm == kNegInf) ? 0.0f
                        : l * (m == kNegInf ? 0.0f : exp2f(m - mm)) +
                              (sk == kNegInf ? 0.0f : exp2f(sk - mm));
    m = mm;
  }
  typename TT::raw* row = reinterpret_cast<typename TT::raw*>(qk) + ((((int64_t)b * p.num_heads + h) * S + i) * cols);
  for (int64_t j = tid; j < cols; j += kQkThreads) {
    float v = 0.0f;
    if (j >= lo && j < hi) {
      const float sc = score(j);
      v = mode == 1 ? sc : (l > 0.0f ? exp2f(sc * kLog2e - m) / l : 0.0f);
    }
    row[j] = TT::from_f32(v);
  }
}

template <typename TT>
hipError_t launch_qk_t(const AttnParams& p, pa_dtype cache_dtype, void* qk, int mode, int64_t cols,
                       const int32_t* keys, hipStream_t s) {
  const dim3 grid(p.max_query_len, p.num_heads, p.batch), block(kQkThreads);
  switch (cache_dtype) {
    case PA_DTYPE_INT8:
      hipLaunchKernelGGL((gqa_qk_kernel<TT, I8Cache>), grid, block, 0, s, p, qk, mode, cols, keys);
      break;
    case PA_DTYPE_INT4:
      hipLaunchKernelGGL((gqa_qk_kernel<TT, I4Cache>), grid, block, 0, s, p, qk, mode, cols, keys);
      break;
    default:
      if (cache_dtype != TT::code) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gqa_qk_kernel<TT, TT>), grid, block, 0, s, p, qk, mode, cols, keys);
      break;
  }
  return hipGetLastError();
}

template <typename TT>
void launch_reduce_t(const AttnParams& p, hipStream_t s) {
  dim3 grid(p.num_heads, p.num_tokens);
  // four wavefronts per pair up to 4096 pairs (16 per CU), one beyond (LATENT decode at 16
  // heads, 1024 pairs: merge 14.4 -> 8.4 us; at 128 heads, 8192 pairs: 22.3 us with one,
  // 26.7 us with four)
  if ((int64_t)p.num_heads * p.num_tokens <= 4096) {
    if (p.v_head_dim <= 256)
      hipLaunchKernelGGL((split_reduce_kernel<TT, 1, 256>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((split_reduce_kernel<TT, 3, 256>), grid, dim3(256), 0, s, p);
  } else if (p.v_head_dim <= 256) {
    hipLaunchKernelGGL((split_reduce_kernel<TT, 4, 64>), grid, dim3(64), 0, s, p);
  } else {
    hipLaunchKernelGGL((split_reduce_kernel<TT, 10, 64>), grid, dim3(64), 0, s, p);
  }
}

}  // namespace

hipError_t launch_attn_generic(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                               hipStream_t s) {
  if (p.num_tokens <= 0) return hipSuccess;
  if (p.head_dim > kMaxHeadDim || p.v_head_dim < 1 || p.v_head_dim > p.head_dim)
    return hipErrorInvalidValue;
  switch (act) {
    case PA_DTYPE_FLOAT16: return launch_generic_t<TF16>(p, cache_dtype, s);
    case PA_DTYPE_BFLOAT16: return launch_generic_t<TBF16>(p, cache_dtype, s);
    case PA_DTYPE_FLOAT32: return launch_generic_t<TF32>(p, cache_dtype, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gqa_qk(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype, void* qk,
                         int mode, int64_t cols, const int32_t* keys, hipStream_t s) {
  if (p.batch <= 0 || p.max_query_len <= 0) return hipSuccess;
  if (p.head_dim > kMaxHeadDim || p.linear_cap <= 0 || (mode != 1 && mode != 2) || cols <= 0 ||
      !keys || !qk || p.max_query_len > 65535 || p.num_heads > 65535 || p.batch > 65535)
    return hipErrorInvalidValue;
  switch (act) {
    case PA_DTYPE_FLOAT16: return launch_qk_t<TF16>(p, cache_dtype, qk, mode, cols, keys, s);
    case PA_DTYPE_BFLOAT16: return launch_qk_t<TBF16>(p, cache_dtype, qk, mode, cols, keys, s);
    case PA_DTYPE_FLOAT32: return launch_qk_t<TF32>(p, cache_dtype, qk, mode, cols, keys, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_split_reduce(const AttnParams& p, pa_dtype act, hipStream_t s) {
  if (p.num_tokens <= 0 || p.max_splits <= 1) return hipSuccess;
  if (p.head_dim > kMaxHeadDim || p.v_head_dim < 1 || p.v_head_dim > p.head_dim)
    return hipErrorInvalidValue;
  switch (act) {
    case PA_DTYPE_FLOAT16: launch_reduce_t<TF16>(p, s); break;
    case PA_DTYPE_BFLOAT16: launch_reduce_t<TBF16>(p, s); break;
    case PA_DTYPE_FLOAT32: launch_reduce_t<TF32>(p, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pa
