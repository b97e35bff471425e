// pa_decode.hip — split-K paged GQA decode on gfx950 matrix cores.
//
// Replaces the reference's direct Metal vector kernel and its two-pass partition/reduce
// (paged_attention.rs:31-143, launcher :229-334) and, for bf16, the dense gather + SDPA
// fallback (attention.rs:4192-4319) that the reference takes for every non-fp16 decode.
//
// Work unit: one wavefront per (sequence, kv-head, context chunk).  The wavefront serves every
// grouped query row of its kv-head — rows r = (query token i, head hh) with r = i*g + hh, up
// to 16 at a time — from ONE pass over the pages, so each K/V byte is read from HBM once per
// kv-head instead of once per query head (the reference re-reads it g times).
//
// Per 32-token step (two 16-token tiles A and B):
//   S^T = K_tile . Q^T   v_mfma_f32_16x16x32 (A = 16 keys x 32 dims straight from the page row,
//                        16 bytes per lane; B = Q^T held in registers for the whole chunk).
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
// Split-K: each chunk writes (m, l, O) partials; pa_attn_generic.hip's reduce merges them.
// A sequence that fits one chunk writes its final rows directly.
//
// HBM traffic per step and kv-head: 16 KiB of K/V rows (bf16, d=128), each byte read once.
// The next step's rows are loaded before the current step is computed (two register sets).
#include <algorithm>

#include "pa_device.hpp"

namespace pa {
namespace {

template <int D>
struct VRow;  // one lane's slice of one value row: DL = D/16 elements
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
__device__ __forceinline__ VRow<D> load_vrow(const uint16_t* ptr);
template <>
__device__ __forceinline__ VRow<64> load_vrow<64>(const uint16_t* ptr) {
  VRow<64> r;
  r.w = *reinterpret_cast<const u32x2*>(ptr);
  return r;
}
template <>
__device__ __forceinline__ VRow<128> load_vrow<128>(const uint16_t* ptr) {
  VRow<128> r;
  r.w = *reinterpret_cast<const u32x4*>(ptr);
  return r;
}

template <int D>
struct Step {
  static constexpr int KS = D / 32;
  u32x4 k[2][KS];  // tile A / tile B key rows, 8 dims per k-step
  VRow<D> v[8];    // value rows: keys 4G+e of tile A (e<4) and of tile B (e>=4)
};

template <typename TT, int D>
struct DecodeCtx {
  const AttnParams& p;
  const uint16_t* kc;
  const uint16_t* vc;
  const uint16_t* kn;
  const uint16_t* vn;
  int b, kh, s0, nq;
  int pastb, total, cache_limit;
  int64_t row;  // elements between consecutive cache rows (kv_heads * D)
  int c, G;
  int first_bi;
  int btv;      // lane i: block_table[b, first_bi + i]
  bool aligned; // block_size % 16 == 0: a 16-key tile never straddles two pages

  __device__ int64_t clamp_blk(int64_t blk) const {
    return min(max(blk, (int64_t)0), p.num_blocks - 1);
  }

  // Element offset of key/value row `pos` (per-lane, any block size); `is_cache` tells the
  // caller which base pointer applies.  Positions past the end clamp to the last real row.
  __device__ int64_t row_offset(int pos, bool& is_cache) const {
    if (pos >= total) pos = total - 1;
    if (pos < cache_limit) {
      is_cache = true;
      int bi = min(pos / p.block_size, p.max_blocks - 1);
      int64_t blk = clamp_blk(p.block_table[(int64_t)b * p.max_blocks + bi]);
      return (blk * p.block_size + pos % p.block_size) * row + (int64_t)kh * D;
    }
    is_cache = false;
    int64_t tok = min(max((int64_t)s0 + (pos - pastb), (int64_t)0), (int64_t)p.num_tokens - 1);
    return tok * row + (int64_t)kh * D;
  }

  __device__ void load_generic(int t0, Step<D>& st) const {
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      bool cache;
      int64_t off = row_offset(t0 + 16 * tile + c, cache);
      const uint16_t* base = (cache ? kc : kn) + off + 8 * G;
#pragma unroll
      for (int s = 0; s < Step<D>::KS; ++s)
        st.k[tile][s] = *reinterpret_cast<const u32x4*>(base + 32 * s);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bool cache;
      int pos = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
      int64_t off = row_offset(pos, cache);
      st.v[e] = load_vrow<D>((cache ? vc : vn) + off + (D / 16) * c);
    }
  }

  // All 32 keys are cached and each 16-key tile lies in one page: the page id is wave-uniform
  // (read from a register with v_readlane), so addresses are a scalar base + lane offset.
  __device__ void load_fast(int t0, Step<D>& st) const {
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      int tp = t0 + 16 * tile;
      int64_t blk = clamp_blk(__builtin_amdgcn_readlane(btv, tp / p.block_size - first_bi));
      int64_t tbase = (blk * p.block_size + tp % p.block_size) * row + (int64_t)kh * D;
      const uint16_t* kb = kc + tbase + (int64_t)c * row + 8 * G;
#pragma unroll
      for (int s = 0; s < Step<D>::KS; ++s)
        st.k[tile][s] = *reinterpret_cast<const u32x4*>(kb + 32 * s);
      const uint16_t* vb = vc + tbase + (int64_t)(4 * G) * row + (D / 16) * c;
#pragma unroll
      for (int e = 0; e < 4; ++e) st.v[4 * tile + e] = load_vrow<D>(vb + (int64_t)e * row);
    }
  }

  __device__ void load(int t0, Step<D>& st) const {
    if (aligned && t0 + 32 <= cache_limit)
      load_fast(t0, st);
    else
      load_generic(t0, st);
  }
};

// Regroup 8 value rows (lane holds DL dims of each) into DL MFMA B-operands of 8 keys x 1 dim.
template <typename TT, int D>
__device__ __forceinline__ typename TT::vec8 value_operand(const Step<D>& st, int j) {
  u32x4 w;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t lo = st.v[2 * m].word(j >> 1), hi = st.v[2 * m + 1].word(j >> 1);
    w[m] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
  }
  return __builtin_bit_cast(typename TT::vec8, w);
}

template <typename TT, int D>
__global__ __launch_bounds__(64) void decode_mfma_kernel(const AttnParams p) {
  constexpr int KS = D / 32;
  constexpr int DL = D / 16;
  using vec8 = typename TT::vec8;
  const int split = blockIdx.x, b = blockIdx.z;
  const int kh = blockIdx.y % p.kv_heads, rgroup = blockIdx.y / p.kv_heads;
  const int ngroups = gridDim.y / p.kv_heads;
  const int lane = threadIdx.x, c = lane & 15, G = lane >> 4;

  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int nq = s1 - s0;
  if (nq <= 0) return;
  const int pastb = max(p.past[b], 0);
  const int total = pastb + nq;
  const int start = split * p.chunk;
  if (start >= total) return;
  const int end = min(start + p.chunk, total);
  const int g = p.num_heads / p.kv_heads;
  const int R = g * nq;

  DecodeCtx<TT, D> ctx{p};
  ctx.kc = reinterpret_cast<const uint16_t*>(p.key_cache);
  ctx.vc = reinterpret_cast<const uint16_t*>(p.value_cache);
  ctx.kn = reinterpret_cast<const uint16_t*>(p.k_new);
  ctx.vn = reinterpret_cast<const uint16_t*>(p.v_new);
  ctx.b = b;
  ctx.kh = kh;
  ctx.s0 = s0;
  ctx.nq = nq;
  ctx.pastb = pastb;
  ctx.total = total;
  ctx.cache_limit = p.read_all_from_cache ? total : pastb;
  ctx.row = (int64_t)p.kv_heads * D;
  ctx.c = c;
  ctx.G = G;
  ctx.aligned = (p.block_size % 16) == 0;
  ctx.first_bi = start / p.block_size;
  {
    int bi = min(ctx.first_bi + lane, p.max_blocks - 1);
    ctx.btv = p.block_table[(int64_t)b * p.max_blocks + bi];
  }
  const uint16_t* qp = reinterpret_cast<const uint16_t*>(p.q);
  const float scale_log2 = p.scale_log2;
  const float cap = p.softcap;

  for (int row0 = 16 * rgroup; row0 < R; row0 += 16 * ngroups) {
    // This lane's MFMA column: query row r = row0 + c.
    const int r = row0 + c;
    const bool rvalid = r < R;
    const int qi = rvalid ? r / g : 0;
    const int h = kh * g + (rvalid ? r % g : 0);
    const int rpos = pastb + qi;
    int vis_lo = p.window > 0 ? rpos - p.window + 1 : 0;
    int vis_hi = p.causal ? rpos + 1 : total;
    if (!rvalid) vis_hi = -1;

    vec8 qv[KS];
    {
      const uint16_t* qrow = qp + ((int64_t)(s0 + qi) * p.num_heads + h) * D + 8 * G;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4 w = rvalid ? *reinterpret_cast<const u32x4*>(qrow + 32 * s) : u32x4{0, 0, 0, 0};
        qv[s] = __builtin_bit_cast(vec8, w);
      }
    }

    f32x4 o[DL];
#pragma unroll
    for (int j = 0; j < DL; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf;  // running max of row c (log2 units); identical across G
    float l_part = 0.0f;    // this lane's share of the row-c denominator

    auto compute = [&](int t0, const Step<D>& st) {
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sa = TT::mfma(__builtin_bit_cast(vec8, st.k[0][s]), qv[s], sa);
        sb = TT::mfma(__builtin_bit_cast(vec8, st.k[1][s]), qv[s], sb);
      }
      float x[8];
      float lmax = kNegInf;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int pos = t0 + 16 * (e >> 2) + 4 * G + (e & 3);
        float sv = (e < 4) ? sa[e & 3] : sb[e & 3];
        float xv;
        if (cap > 0.0f)
          xv = cap * tanhf(sv * p.scale / cap) * kLog2e;
        else
          xv = sv * scale_log2;
        const bool vis = pos < end && pos >= vis_lo && pos < vis_hi;
        x[e] = vis ? xv : kNegInf;
        lmax = fmaxf(lmax, x[e]);
      }
      if (__any(lmax > m_run + 8.0f)) {
        float rmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
        const float m_new = fmaxf(m_run, rmax);
        const float alpha = (m_new == kNegInf) ? 1.0f : exp2f(m_run - m_new);
        l_part *= alpha;
        m_run = m_new;
        float ar[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * G + i, 64);
#pragma unroll
        for (int j = 0; j < DL; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[j][i] *= ar[i];
      }
      const float msafe = (m_run == kNegInf) ? 0.0f : m_run;
      float pv[8], plo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = exp2f(x[e] - msafe);
        l_part += pv[e];
      }
      vec8 phi = TT::cvt8(pv);
#pragma unroll
      for (int e = 0; e < 8; ++e) plo[e] = pv[e] - TT::back(phi[e]);
      vec8 plo8 = TT::cvt8(plo);
#pragma unroll
      for (int j = 0; j < DL; ++j) {
        vec8 vb = value_operand<TT, D>(st, j);
        o[j] = TT::mfma(phi, vb, o[j]);
        o[j] = TT::mfma(plo8, vb, o[j]);
      }
    };

    // Keys outside every row's causal/window range are skipped (whole 32-key steps).
    int lo_any = rvalid ? vis_lo : INT32_MAX;
    int hi_any = vis_hi;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      lo_any = min(lo_any, __shfl_xor(lo_any, o, 64));
      hi_any = max(hi_any, __shfl_xor(hi_any, o, 64));
    }
    const int t_first = max(start, (lo_any / 32) * 32);
    const int t_last = min(end, hi_any);  // exclusive
    Step<D> sA, sB;
    int t0 = t_first;
    if (t0 < t_last) {
      ctx.load(t0, sA);
      while (true) {
        if (t0 + 32 < t_last) ctx.load(t0 + 32, sB);
        compute(t0, sA);
        t0 += 32;
        if (t0 >= t_last) break;
        if (t0 + 32 < t_last) ctx.load(t0 + 32, sA);
        compute(t0, sB);
        t0 += 32;
        if (t0 >= t_last) break;
      }
    }

    // Row totals: sum the four lane groups' partial denominators of row c, then fetch the
    // (m, l) of the rows this lane's O registers hold (rows 4G+i).
    float l_row = l_part + __shfl_xor(l_part, 16, 64);
    l_row += __shfl_xor(l_row, 32, 64);
    const bool single = (start == 0 && end == total);
    // Metadata beyond the planned capacity (total > max_blocks * block_size) leaves no
    // partial buffer to write into; such rows are left unwritten rather than faulting.
    if (!single && p.part_o == nullptr) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + 4 * G + i;
      const float mi = __shfl(m_run, 4 * G + i, 64);
      const float li = __shfl(l_row, 4 * G + i, 64);
      if (rr >= R) continue;
      const int oqi = rr / g, oh = kh * g + rr % g;
      const int64_t t = s0 + oqi;
      if (single) {
        const float f = finalize_factor(mi, li, sink_logit<TT>(p, oh));
        typename TT::raw vals[DL];
#pragma unroll
        for (int j = 0; j < DL; ++j) vals[j] = TT::from_f32(o[j][i] * f);
        typename TT::raw* dst =
            reinterpret_cast<typename TT::raw*>(p.out) + (t * p.num_heads + oh) * D + DL * c;
#pragma unroll
        for (int j = 0; j < DL; ++j) dst[j] = vals[j];
      } else {
        const int64_t pi = (t * p.num_heads + oh) * p.max_splits + split;
        float* dst = p.part_o + pi * D + DL * c;
#pragma unroll
        for (int j = 0; j < DL; ++j) dst[j] = o[j][i];
        if (c == 0) {
          p.part_ml[pi * 2 + 0] = mi;
          p.part_ml[pi * 2 + 1] = li;
        }
      }
    }
  }
}

template <typename TT>
hipError_t launch_t(const AttnParams& p, int row_groups, hipStream_t s) {
  dim3 grid(p.max_splits, p.kv_heads * row_groups, p.batch), block(64);
  switch (p.head_dim) {
    case 64: hipLaunchKernelGGL((decode_mfma_kernel<TT, 64>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((decode_mfma_kernel<TT, 128>), grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (cache_dtype != act) return false;
  return head_dim == 64 || head_dim == 128;
}

hipError_t launch_decode_mfma(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                              hipStream_t s) {
  if (!decode_mfma_supported(p.head_dim, act, cache_dtype)) return hipErrorInvalidValue;
  if (p.batch <= 0) return hipSuccess;
  const int g = p.num_heads / p.kv_heads;
  const int mq = p.max_query_len > 0 ? p.max_query_len : p.num_tokens;
  const int row_groups = (int)std::min<int64_t>(((int64_t)g * mq + 15) / 16, 65535 / p.kv_heads);
  if (act == PA_DTYPE_FLOAT16) return launch_t<TF16>(p, row_groups, s);
  return launch_t<TBF16>(p, row_groups, s);
}

}  // namespace pa
