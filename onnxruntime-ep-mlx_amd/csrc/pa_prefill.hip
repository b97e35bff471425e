// pa_prefill.hip — chunked-prefill attention over the paged cache on gfx950 matrix cores.
//
// Replaces the reference's prefill route, the dense fallback (attention.rs:4192-4319) that
// gathers the pages, concatenates the new rows and runs SDPA with native GQA heads for more
// than 8 query tokens (:4235-4253, paged_sdpa :3786-3809).
//
// Work unit: one workgroup of 4 wavefronts per (sequence, kv-head, block of 64*NG grouped query
// rows, context chunk).  Rows r = (query token i, head hh) with r = i*g + hh, as in the decode
// kernels; wavefront w owns rows row0 + 16*NG*w + 16*j, j < NG, and computes them with the
// shared 16x16x32 tile step (pa_tiles.hpp).
//
// Every 32-key step is fetched from the pages once per workgroup, the four wavefronts taking a
// quarter each (key tile A, key tile B, the first and the second half of the value dims), and
// written to LDS as the per-lane MFMA operand images the tile step consumes -- value rows
// already regrouped into the B-operand layout.  Each wavefront then reads its operands with
// 16-byte LDS reads, consecutive lanes at consecutive addresses (conflict free).  Against every
// wavefront streaming the step by itself this cuts the L2->CU bytes 4x and does the value
// regroup once per workgroup instead of once per wavefront.
//
// Pipeline: two LDS buffers and one barrier per step.  In iteration k the wavefronts compute
// step k from buffer k&1, then write step k+1 (whose global loads were issued one iteration
// earlier) into buffer (k+1)&1 -- last read in iteration k-1, before the previous barrier --
// and issue the global loads of step k+2.  Two workgroups share a CU (two wavefronts per SIMD),
// so one computes while the other waits at its barrier.
//
// Keys come from the pages when the step lies below the cache limit and the block size is a
// multiple of 16 (one page per 16-key tile, page ids from a block-table window held one entry
// per lane); other steps (new rows not yet in the pages, odd block sizes) address every row on
// its own.  Value rows at or past the sequence end are zeroed and their scores masked.
#include "pa_tiles.hpp"

namespace pa {
namespace {

// One wavefront's quarter of a step: 16-key tile T = role & 1 of the keys (roles 0, 1) or of the
// values (roles 2, 3), loaded as 4 pieces of D/8 bytes per lane -- the same instruction
// sequence for every role, only the bases and strides differ:
//   key role:   row c of the tile, dims 8G..8G+7 of each 32-dim k-step (16 bytes per k-step);
//   value role: rows 4G..4G+3 of the tile, the lane's DL = D/16 dims DL*c ..
// r[] holds the pieces in order (key k-step s = 16-byte item s; value row e = words HW*e ..).
template <int D>
struct Quarter {
  static constexpr int PW = D / 32;  // words per piece
  uint32_t r[4 * PW];
  __device__ u32x4 item(int s) const { return u32x4{r[4 * s], r[4 * s + 1], r[4 * s + 2], r[4 * s + 3]}; }
  __device__ uint32_t vword(int e, int wi) const { return r[PW * e + wi]; }
};

template <int D>
__device__ __forceinline__ void load_piece(uint32_t* r, const char* ptr) {
  if constexpr (D == 128) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(ptr);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = v[i];
  } else {
    const u32x2 v = *reinterpret_cast<const u32x2*>(ptr);
    r[0] = v[0];
    r[1] = v[1];
  }
}

// Per-lane geometry of a role: piece s sits at row `row0 + s * row_step` of the tile and byte
// `col0 + (s >> 1) * col_a + (s & 1) * col_b` of that row's kv-head slice.
struct RoleGeom {
  bool value;
  int row0, row_step;
  int col0, col_a, col_b;
};

template <int D>
__device__ __forceinline__ RoleGeom role_geom(int role, int c, int G) {
  RoleGeom g;
  g.value = role >= 2;
  if (g.value) {
    g.row0 = 4 * G;
    g.row_step = 1;
    g.col0 = (D / 16) * 2 * c;
    g.col_a = g.col_b = 0;
  } else {
    g.row0 = c;
    g.row_step = 0;
    g.col0 = 16 * G;
    g.col_a = D == 128 ? 128 : 64;  // k-step pairs (d=128) / k-steps (d=64)
    g.col_b = D == 128 ? 64 : 8;    // next k-step (d=128) / second half of a k-step (d=64)
  }
  return g;
}

// PW words of one value row slice at ptr (4-byte aligned; 16-byte aligned when PW % 4 == 0).
template <int PW>
__device__ __forceinline__ void load_words(uint32_t* r, const char* ptr) {
  if constexpr (PW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < PW / 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(ptr + 16 * i);
#pragma unroll
      for (int k = 0; k < 4; ++k) r[4 * i + k] = v[k];
    }
  } else {
    __builtin_memcpy(r, __builtin_assume_aligned(ptr, 4), 4 * PW);
  }
}

// Issue this wavefront's loads of the step at key t0.
template <int D>
__device__ __forceinline__ void load_quarter(const WaveInfo& w, PageWindow& pw, const RoleGeom& rg,
                                             int role, int t0, int lane, Quarter<D>& q) {
  const int t = t0 + 16 * (role & 1);
  // With every key in the pages the last (partial) step comes from them too: rows past the end
  // are masked / zeroed and page ids are clamped into the pool.
  // (Contiguous caches: only steps whose 32 rows all lie inside the capacity.)
  const bool paged = w.bs % 16 == 0 && (t0 + 32 <= w.cache_limit || w.cache_limit >= w.total) &&
                     (w.lin_row0 < 0 || t0 + 32 <= w.lin_cap);
  if constexpr (D != 64 && D != 128) {
    // Other heads: key role = KS 16-byte k-step items of row c; value role = the lane's D/8
    // bytes of rows 4G .. 4G+3.
    constexpr int KS = D / 32, PW = D / 32;
    const int c = lane & 15, G = lane >> 4;
    const int64_t tb = paged ? tile_base(w, pw, t, lane, D) : 0;
    if (!rg.value) {
      const char* rp = paged ? w.kc + tb + (int64_t)c * w.rowb : row_ptr(w, t + c, false, D);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 v = ld16(rp + 16 * G + 64 * s);
#pragma unroll
        for (int k = 0; k < 4; ++k) q.r[4 * s + k] = v[k];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const char* rp = paged ? w.vc + tb + (int64_t)(4 * G + e) * w.rowb
                               : row_ptr(w, t + 4 * G + e, true, D);
        load_words<PW>(q.r + PW * e, rp + (D / 16) * 2 * c);
      }
    }
    return;
  }
  if (paged) {
    const char* base = (rg.value ? w.vc : w.kc) + tile_base(w, pw, t, lane, D) +
                       (int64_t)rg.row0 * w.rowb + rg.col0;
    const int64_t rstep = rg.row_step * w.rowb;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      load_piece<D>(q.r + Quarter<D>::PW * s,
                    base + s * rstep + (s >> 1) * rg.col_a + (s & 1) * rg.col_b);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      load_piece<D>(q.r + Quarter<D>::PW * s,
                    row_ptr(w, t + rg.row0 + s * rg.row_step, rg.value, D) + rg.col0 +
                        (s >> 1) * rg.col_a + (s & 1) * rg.col_b);
  }
}

// Write this wavefront's quarter of the step at key t0 into LDS buffer `buf` ([item][lane]):
// items 0 .. 2*KS-1 are the key operands (tile, k-step), items 2*KS + j the value operands of
// N-tile j.  Word m of a value operand combines value rows 2m and 2m+1 of the step (rows 4G+i
// of tile A for m < 2, of tile B for m >= 2), so value role T writes words 2T, 2T+1 of every
// N-tile.
template <int D>
__device__ __forceinline__ void store_quarter(u32x4 (*buf)[64], Quarter<D>& q, int role, int t0,
                                              int total, int lane, int G) {
  constexpr int KS = D / 32, DL = D / 16;
  const int T = role & 1;
  if (role < 2) {
#pragma unroll
    for (int s = 0; s < KS; ++s) buf[T * KS + s][lane] = q.item(s);
  } else {
    if (t0 + 32 > total) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (t0 + 16 * T + 4 * G + e >= total)
#pragma unroll
          for (int i = 0; i < Quarter<D>::PW; ++i) q.r[Quarter<D>::PW * e + i] = 0u;
    }
#pragma unroll
    for (int j = 0; j < DL; ++j) {
      u32x2 half;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t lo = q.vword(2 * m, j >> 1), hi = q.vword(2 * m + 1, j >> 1);
        // one byte permute: the low (even j) or high (odd j) halves of the two rows
        half[m] = __builtin_amdgcn_perm(hi, lo, (j & 1) ? 0x07060302u : 0x05040100u);
      }
      reinterpret_cast<u32x2*>(&buf[2 * KS + j][lane])[T] = half;
    }
  }
}

// Two workgroups per CU; one at head 256, whose row state and step operands need the larger
// register budget.  BIAS: GroupQueryAttention's additive attention bias (AttnParams::bias), each
// lane's 8 values per group and step loaded one step ahead (one workgroup per CU from head 128
// on: two spilled ~25 registers).
template <typename TT, int D, bool CAP, int NG, bool BIAS = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    (D > 128 || (BIAS && D == 128)) ? 1 : 2, (D > 128 || (BIAS && D == 128)) ? 1 : 2))) void
prefill_kernel(const AttnParams p) {
  using vec8 = typename TT::vec8;
  constexpr int KS = D / 32, DL = D / 16, NI = 2 * KS + DL;
  constexpr int ROWS = 64 * NG;  // grouped query rows per workgroup
  __shared__ u32x4 lds[2][NI][64];
  // Grid x: (row block, sequence, kv-head) with (sequence, kv-head) fastest and the row blocks
  // in reverse, so the last blocks of each chunk (the most keys under the causal mask) start
  // first.  Grid y: context chunk (split-K).
  int rb, kh, b, split = blockIdx.y, part = 0, item = 0, ustart = 0, uend = 0;
  if (p.plan_items > 0) {
    // Planned: this workgroup's unit, longest first (both loads in one round trip).
    const int nunits = p.plan_info[0];
    const int4 u = reinterpret_cast<const int4*>(p.plan)[min((int)blockIdx.x, p.plan_items * 2 - 1)];
    if ((int)blockIdx.x >= nunits) return;
    item = u.x;
    part = u.y;
    ustart = u.z;
    uend = u.w;
    kh = item % p.kv_heads;
    rb = (item / p.kv_heads) % p.plan_rbs;
    b = item / (p.kv_heads * p.plan_rbs);
  } else {
    const int units = p.batch * p.kv_heads;
    const int unit = blockIdx.x % units;
    rb = (int)(gridDim.x / units) - 1 - (int)(blockIdx.x / units);
    kh = unit % p.kv_heads;
    b = unit / p.kv_heads;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, c = lane & 15, G = lane >> 4;
  // Everything up to the first barrier is uniform over the workgroup.
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int nq = s1 - s0;
  const int g = p.num_heads / p.kv_heads;
  const int R = g * nq;
  const int row0 = rb * ROWS;
  if (row0 >= R) return;
  const int pastb = clamped_past(p, b, nq);
  const int total = seq_total(p, b, pastb, nq);
  int start, end;
  bool single;
  if (p.plan_items > 0) {
    start = ustart;
    end = max(ustart, min(uend, total));
    single = part == 0;
  } else {
    start = split * p.chunk;
    if (start >= total) return;
    end = start + min(p.chunk, total - start);
    single = start == 0 && end == total;
  }
  // Metadata beyond the planned capacity leaves no partial buffer: rows stay unwritten.
  if (!single && p.part_o == nullptr) return;
  // Keys any row of the workgroup can see.
  const int r_last = min(row0 + ROWS, R) - 1;
  const int hi = p.causal ? pastb + r_last / g + 1 : total;
  const int lo = p.window > 0 ? max(0, pastb + row0 / g - p.window + 1) : 0;
  const int t_first = max(start, (lo / 32) * 32);
  const int t_last = min(end, hi);
  const int nsteps = t_last > t_first ? (t_last - t_first + 31) / 32 : 0;

  const WaveInfo w = make_wave(p, D, b, kh, s0, pastb, total);
  // This wavefront's rows and the keys they can see (steps outside are not computed).
  const int wrow0 = row0 + 16 * NG * wave;
  // A negative softmax scale moves its sign into the query operands (attend_groups takes a
  // scale that is not negative).
  const uint32_t qxor = p.scale < 0.0f ? 0x80008000u : 0u;
  const float scale = fabsf(p.scale), scale_log2 = fabsf(p.scale_log2);
  RowState<TT, D> rs[NG];
#pragma unroll
  for (int j = 0; j < NG; ++j) init_rows<TT, D>(rs[j], p, w, wrow0 + 16 * j, R, g, c, G, qxor);
  // Keys visible to some row [any_lo, any_hi) and to every row [all_lo, all_hi) of the wave.
  int any_lo = 0, any_hi = -1, all_lo = 0, all_hi = -1;
  if (wrow0 < R) {
    const int qf = wrow0 / g, ql = (min(wrow0 + 16 * NG, R) - 1) / g;
    any_hi = p.causal ? pastb + ql + 1 : total;
    all_hi = min(end, p.causal ? pastb + qf + 1 : total);
    any_lo = p.window > 0 ? pastb + qf - p.window + 1 : 0;
    all_lo = p.window > 0 ? pastb + ql - p.window + 1 : 0;
  }

  // bias rows of this lane in each group (rows past R read row R - 1: never stored)
  BiasRow brow[NG];
  uint32_t bnext[BIAS ? NG : 1][4];
  if constexpr (BIAS) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int r = min(wrow0 + 16 * j + c, R - 1);
      brow[j] = bias_row_of(p, b, kh * g + r % g, r / g);
      if (nsteps > 0) bias_load(brow[j], t_first, G, bnext[j]);
    }
  }

  PageWindow pw;
  window_at(pw, w, min(div_bs(t_first, w), w.max_blocks - 1), lane);
  const RoleGeom rg = role_geom<D>(wave, c, G);
  Quarter<D> q;
  if (nsteps > 0) {
    load_quarter<D>(w, pw, rg, wave, t_first, lane, q);
    store_quarter<D>(lds[0], q, wave, t_first, total, lane, G);
    if (nsteps > 1) load_quarter<D>(w, pw, rg, wave, t_first + 32, lane, q);
  }
  __syncthreads();
  for (int k = 0; k < nsteps; ++k) {
    const int t0 = t_first + 32 * k;
    float bx[NG][8];
    if constexpr (BIAS) {
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        bias_log2<TT>(bnext[j], bx[j]);
        if (k + 1 < nsteps) bias_load(brow[j], t0 + 32, G, bnext[j]);
      }
    }
    if constexpr (D > 128) {
      // Heads above 128: operands read from LDS where they are used (the row state of two
      // groups already takes most of the register file).
      if (t0 < any_hi && t0 + 32 > any_lo) {
        const int bsel = k & 1;
        auto kl = [&](int tile, int s) {
          return __builtin_bit_cast(vec8, lds[bsel][tile * KS + s][lane]);
        };
        auto vl = [&](int n) { return __builtin_bit_cast(vec8, lds[bsel][2 * KS + n][lane]); };
        if (t0 >= all_lo && t0 + 32 <= all_hi)
          attend_groups_ops<TT, D, CAP, false, NG, BIAS>(rs, kl, vl, t0, end, G, scale_log2,
                                                         scale, p.softcap, bx);
        else
          attend_groups_ops<TT, D, CAP, true, NG, BIAS>(rs, kl, vl, t0, end, G, scale_log2,
                                                        scale, p.softcap, bx);
      }
    } else if (t0 < any_hi && t0 + 32 > any_lo) {
      u32x4 kop[2][KS];
      u32x4 vop[DL];
#pragma unroll
      for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int s = 0; s < KS; ++s) kop[tile][s] = lds[k & 1][tile * KS + s][lane];
#pragma unroll
      for (int j = 0; j < DL; ++j) vop[j] = lds[k & 1][2 * KS + j][lane];
      auto vb = [&](int n) { return __builtin_bit_cast(vec8, vop[n]); };
      if (t0 >= all_lo && t0 + 32 <= all_hi)
        attend_groups<TT, D, CAP, false, NG, BIAS>(rs, kop, vb, t0, end, G, scale_log2, scale,
                                                   p.softcap, bx);
      else
        attend_groups<TT, D, CAP, true, NG, BIAS>(rs, kop, vb, t0, end, G, scale_log2, scale,
                                                  p.softcap, bx);
    }
    if (k + 1 < nsteps) store_quarter<D>(lds[(k + 1) & 1], q, wave, t0 + 32, total, lane, G);
    if (k + 2 < nsteps) load_quarter<D>(w, pw, rg, wave, t0 + 64, lane, q);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int r0 = wrow0 + 16 * j;
    if (r0 >= R) break;
    const int rc = min(r0 + c, R - 1);
    const float sink_c = sink_logit<TT>(p, kh * g + rc % g);
    store_rows<TT, D>(rs[j], p, kh, s0, r0, R, g, c, G, sink_c, single,
                      [&](int64_t t, int oh, int rloc) {
                        if (p.plan_items > 0)
                          return ((int64_t)item * 2 + part - 1) * ROWS + (r0 - row0) + rloc;
                        return (t * p.num_heads + oh) * p.max_splits + split;
                      },
                      p.plan_items > 0);
  }
}

// ----------------------------------------------------------------------------- d = 128 kernel
// The head-128 prefill kernel on 32x32x16 matrix-core tiles, 64 keys per step.
//
// Workgroup: 4 wavefronts, 128 grouped query rows of one (sequence, kv-head) -- wavefront w owns
// rows row0 + 32 w + c, c = lane % 32 -- over a key range, two workgroups per CU.  Both products
// run transposed, so every lane holds one query row:
//   scores  S^T[key][row] = K . Q^T   (A = 32 keys x 16 dims from LDS, B = Q^T in registers):
//           lane l gets row c, keys 8 i + 4 h + j (h = l / 32, register 4 i + j) of a 32-key block;
//   output  O^T[dim][row] = V^T . P^T (A = 32 dims x 16 keys from LDS, B = P^T in registers):
//           lane l accumulates row c, dims 8 i + 4 h + j of each 32-dim tile.
// The probabilities of key slice t (keys 16 t .. 16 t + 15) are then registers 8 (t % 2) .. + 7
// of score block t / 2 as they come out of the score product, in the key order
// {4 h + j, 8 + 4 h + j} that the value images are written in.  Row maxima, sums and the lazy
// rescale need no cross-lane traffic except one swap between the lane halves.
//
// P . V runs in fp16: probabilities are <= 2^8 (lazy maximum) and convert with round to nearest
// even; bf16 value rows convert exactly to fp16 after a power-of-two scale 2^-s per 32-dim
// quarter, chosen from the largest value seen so far in that quarter (s = exponent - 15, so the
// largest converted value lies in [2^14, 2^15)).  When a step raises a quarter's s the output
// accumulated for that quarter is scaled by the exact power of two 2^(s_old - s_new); the
// epilogue multiplies by 2^s.  Values below 2^-29 of their quarter's maximum lose precision (fp16
// subnormal range), far below the rounding of the fp32 sums.  fp16 activations use their value
// rows as they are.
//
// Steps are fetched once per workgroup: wavefront w loads keys 16 w .. 16 w + 15 of the step (one
// page when the block size is a multiple of 16) and the values of dims 32 w .. 32 w + 31 for all
// 64 keys, converts and regroups them in registers and writes the per-lane MFMA operand images to
// LDS.  Two LDS buffers, one barrier per step, the global loads of step k + 2 in flight while step
// k computes.
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

constexpr int kMxKeys = 64;  // keys per step

template <typename TT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32<TBF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<TF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Both lane halves' value of x (lanes l and l ^ 32 hold the same query row).
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  // lanes 0..31: r[1] is lane l + 32's x; lanes 32..63: r[0] is lane l - 32's x
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// Largest step below the accumulator's exponent that the planned prefill's images take through
// the probabilities (scaled by at most 2^-kImgPShift, so probabilities down to 2^(kImgPShift - 14)
// of the lazy maximum stay fp16-normal).
constexpr int kImgPShift = 4;
// Wide steps of bf16 value images: a step whose nonzero values span kImgWideSpan or more binades
// (some would go subnormal in fp16 under the step's single exponent) keeps its values as raw bf16
// and is tagged in its exponent word (vstep = s + kImgWideTag); the prefill kernel takes its P.V
// product in bf16 with the probabilities split into bf16 hi + lo parts.
constexpr int kImgWideSpan = 29;
constexpr int kImgWideTag = 1 << 24;

// Maximum of a float over the wavefront (butterfly).
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Maximum of a non-negative value over the wavefront (DPP row steps, then the row broadcasts).
__device__ __forceinline__ int wave_max_nonneg(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));  // row_mirror
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false));  // row_bcast:15
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

// One LDS buffer: the operand images of a step of 32 KB keys (KB = 2 for the in-loop staging).
//   k[kb][ks][lane]: key 32 kb + lane % 32, dims 16 ks + 8 (lane / 32) .. + 7 (score A operand)
//   v[t][nt][slot]:  slot mx_vslot(lane) holds dim 32 nt + lane % 32, keys
//                    16 t + {4 h + e, 8 + 4 h + e}, h = lane / 32 (output A operand, fp16)
//   vs[nt]:          the value scale exponent s of quarter nt for this step
// Every staging write and every operand read touches 16 distinct 16-byte bank groups per
// 16 lanes (the value slots are XOR-swizzled for the staging writes; mx_vslot keeps the reads a
// permutation of the image).
template <int KB, int D = 128>
struct MxBufT {
  u32x4 k[KB][D / 16][64];
  u32x4 v[2 * KB][D / 32][64];
  int vs[4];
  int pad[12];
};
using MxBuf = MxBufT<2>;

__device__ __forceinline__ int mx_vslot(int lane) { return lane ^ ((lane >> 4) & 3); }

// This wavefront's share of a step's rows, as loaded.
//   keys:   key 16 w + lane % 16, bytes 64 i + 16 (lane / 16) .. + 15 of its row slice, i < 4
//   values: keys 16 t + 4 hh + e and 16 t + 8 + 4 hh + e (e < 4; t = lane / 16,
//           hh = lane / 8 % 2), dims 32 w + 4 (lane % 8) .. + 3
struct MxStage {
  u32x4 k[4];
  u32x2 v[8];
};

// Issue the loads of the step at key t0.  Page rows come straight from the pages when the step
// lies below the cache limit (or every key is in the pages) and the block size is a multiple of
// 16: the 16 keys of a group then share one page.  Other steps address every row on its own.
// Value rows at or past the end are zeroed when stored (mx_store).
template <typename TT>
__device__ __forceinline__ void mx_load(const WaveInfo& w, PageWindow& pw, int wave, int lane,
                                        int t0, MxStage& st) {
  constexpr int D = 128;
  const int kr = lane & 15, cq = lane >> 4;
  const int dg = lane & 7, hh = (lane >> 3) & 1, t = lane >> 4;
  const int64_t koff = w.hoff + 16 * cq;
  const int64_t voff = w.hoff + (32 * wave + 4 * dg) * 2;
  const bool paged = w.bs % 16 == 0 && (t0 + kMxKeys <= w.cache_limit || w.cache_limit >= w.total) &&
                     (w.lin_row0 < 0 || t0 + kMxKeys <= w.lin_cap);
  if (paged) {
    // pool row of the first key of each 16-key group (wave-uniform), from the block-table window
    // (contiguous caches: consecutive rows)
    int64_t grp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (w.lin_row0 >= 0) {
        grp[q] = w.lin_row0 + t0 + 16 * q;
        continue;
      }
      const int bi = min(div_bs(t0 + 16 * q, w), w.max_blocks - 1);
      if (bi < pw.first || bi >= pw.first + 64) window_at(pw, w, bi, lane);
      int64_t blk = __builtin_amdgcn_readlane(pw.ids, bi - pw.first);
      blk = min(max(blk, (int64_t)0), w.num_blocks - 1);
      grp[q] = blk * w.bs + mod_bs(t0 + 16 * q, w);
    }
    const char* kb = w.kc + (grp[wave] + kr) * w.rowb + koff;
#pragma unroll
    for (int i = 0; i < 4; ++i) st.k[i] = ld16(kb + 64 * i);
    const int64_t vrow = (t == 0 ? grp[0] : t == 1 ? grp[1] : t == 2 ? grp[2] : grp[3]) + 4 * hh;
    const char* vb = w.vc + vrow * w.rowb + voff;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      st.v[e] = *reinterpret_cast<const u32x2*>(vb + (e + 4 * (e >> 2)) * w.rowb);
  } else {
    const char* kb = row_ptr(w, t0 + 16 * wave + kr, false, D) + 16 * cq;
#pragma unroll
    for (int i = 0; i < 4; ++i) st.k[i] = ld16(kb + 64 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = 16 * t + 4 * hh + (e & 3) + 8 * (e >> 2);
      st.v[e] = *reinterpret_cast<const u32x2*>(row_ptr(w, t0 + key, true, D) +
                                                (32 * wave + 4 * dg) * 2);
    }
  }
}

// Convert (bf16 values: to fp16 under this quarter's running scale) and regroup this
// wavefront's share of the step at t0 into LDS buffer `buf`.  s_run: the quarter's running scale
// exponent (wave-uniform), updated here.
template <typename TT>
__device__ __forceinline__ void mx_store(MxBuf& buf, MxStage& st, int wave, int lane, int t0,
                                         int total, int& s_run) {
  const int kr = lane & 15, cq = lane >> 4;
  const int dg = lane & 7, hh = (lane >> 3) & 1, t = lane >> 4;
  // keys: bytes 64 i + 16 cq = 16-byte chunk dc = 4 i + cq -> slice dc / 2, half dc % 2
  const int kk = 16 * wave + kr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int dc = 4 * i + cq;
    buf.k[kk >> 5][dc >> 1][32 * (dc & 1) + (kk & 31)] = st.k[i];
  }
  // values: rows at or past the end take no part (their bytes may be anything): a row mask
  // folded into the conversion (no branch, so the staging interleaves with the MFMAs)
  uint32_t keep[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    keep[e] = (t0 + 16 * t + 4 * hh + (e & 3) + 8 * (e >> 2) < total) ? 0xffffffffu : 0u;
  if constexpr (!std::is_same<TT, TBF16>::value) {
#pragma unroll
    for (int e = 0; e < 8; ++e) st.v[e] = u32x2{st.v[e][0] & keep[e], st.v[e][1] & keep[e]};
  } else {
    // largest biased exponent of the quarter's step, then s = max(s_run, exponent - 141): the
    // largest value maps into [2^14, 2^15) of fp16 (bf16 exponent e -> fp16 exponent e - 112 - s)
    uint32_t mx = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const u16x2 a = __builtin_bit_cast(u16x2, st.v[e][m] & (keep[e] & 0x7fff7fffu));
        mx = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, mx), a));
      }
    const int emax = wave_max_nonneg((int)(max(mx & 0xffffu, mx >> 16) >> 7));
    s_run = max(s_run, max(emax - 141, -112));
    const unsigned short bias = (unsigned short)((112 + s_run) << 7);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t x = st.v[e][m] & keep[e];
        u16x2 a = __builtin_bit_cast(u16x2, x & 0x7fff7fffu);
        a = __builtin_elementwise_sub_sat(a, u16x2{bias, bias});
        a = a << (unsigned short)3;
        st.v[e][m] = (x & 0x80008000u) | __builtin_bit_cast(uint32_t, a);
      }
  }
  // regroup: dims 4 dg + 2 m (+1) of the 8 keys -> full slots of image (t, nt = wave), lane'
  // 32 hh + 4 dg + 2 m (+1); element e' of a slot is row e' (keys 4 hh + e', then 8 + 4 hh + ...)
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    u32x4 lo, hi;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      lo[e2] = __builtin_amdgcn_perm(st.v[2 * e2 + 1][m], st.v[2 * e2][m], 0x05040100u);
      hi[e2] = __builtin_amdgcn_perm(st.v[2 * e2 + 1][m], st.v[2 * e2][m], 0x07060302u);
    }
    const int lp = 32 * hh + 4 * dg + 2 * m;
    buf.v[t][wave][mx_vslot(lp)] = lo;
    buf.v[t][wave][mx_vslot(lp + 1)] = hi;
  }
  buf.vs[wave] = s_run;  // every lane writes the same word: no branch
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Wait for every outstanding vector-memory operation of this wavefront (the step's direct LDS
// loads) -- vmcnt(0), expcnt and lgkmcnt left at their maxima.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Image staging: this wavefront's quarter of the step at t0 goes straight from the step's
// operand image (AttnParams::vimg, the LDS buffer image byte for byte) to LDS buffer `buf`:
// direct LDS loads of 1 KiB items (4 KB per wavefront), 16 bytes per lane, no register round trip.
template <int KB, int D>
__device__ __forceinline__ void img_issue(MxBufT<KB, D>& buf, int wave, int lane, int t0,
                                          const char* img_hb) {
  constexpr int SB = img_step_bytes(D);
  static_assert(sizeof(MxBufT<KB, D>::k) + sizeof(MxBufT<KB, D>::v) == SB && 32 * KB == img_keys(D),
                "image = LDS operands");
  constexpr int PW = SB / 4;  // bytes per wavefront
  const char* src = img_hb + (int64_t)(t0 / img_keys(D)) * SB + PW * wave + 16 * lane;
  char* dst = reinterpret_cast<char*>(&buf.k[0][0][0]) + PW * wave;
#pragma unroll
  for (int i = 0; i < PW / 1024; ++i)
    __builtin_amdgcn_global_load_lds(src + 1024 * i, (lds_ptr_t)(dst + 1024 * i), 16, 0, 0);
}

// IMG: value operands from the per-(sequence, kv-head) value images (AttnParams::vimg), staged
// by direct LDS loads one step ahead; otherwise loaded, converted and regrouped in the loop.
#ifndef PA_IMG_WAVES
#define PA_IMG_WAVES 2
#endif
// INTC: integer pages (images of fp16 codes): per-channel / per-tensor key scales fold into the
// query, normalised per row by a power of two whose exponent joins the row's softmax scale; the
// scores run on fp16 products; value scales multiply the output per dim before normalisation.
// F8S: fp8 pages (images of the dequantised rows in fp16, keys and values each under a per-step
// power of two): the query rows go to fp16 under a per-row power of two as for INTC, and each
// step's key exponent joins the softmax scale of the step.
template <typename TT, bool CAP, bool IMG, int D = 128, bool INTC = false, bool F8S = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, IMG && D <= 128 ? PA_IMG_WAVES : 2))) void
prefill_mx_kernel(const AttnParams p) {
  static_assert(!(INTC || F8S) || IMG, "byte-coded pages over images only");
  using KT = typename std::conditional<INTC || F8S, TF16, TT>::type;  // score operand type
  // bf16 pages over images: steps may be wide (raw bf16 values, see kImgWideTag).  Head 256 keeps
  // one loop (its image kernel is at the register limit; a second loop instance spills).
  constexpr bool kWide = IMG && !INTC && !F8S && std::is_same<TT, TBF16>::value && D <= 128;
  constexpr int ROWS = kPrefillRows;
  static_assert(ROWS == 128, "four wavefronts of 32 rows");
  static_assert(IMG ? img_head(D) : D == 128, "images at heads 64 / 96 / 128 / 256, in-loop staging at 128");
  // key blocks of 32 per step: image steps of img_keys(D) keys, or 64 keys staged in the loop;
  // KS 16-dim k-steps of the score product, NQ 32-dim output tiles
  constexpr int KB = IMG ? img_keys(D) / 32 : 2, KEYS = 32 * KB, KS = D / 16, NQ = D / 32;
  using Buf = MxBufT<KB, D>;
  __shared__ Buf lds[2];
  int rb, kh, b, split = blockIdx.y, part = 0, item = 0, ustart = 0, uend = 0;
  if (p.plan_items > 0) {
    const int nunits = p.plan_info[0];
    const int4 u = reinterpret_cast<const int4*>(p.plan)[min((int)blockIdx.x, p.plan_items * 2 - 1)];
    if ((int)blockIdx.x >= nunits) return;
    item = u.x;
    part = u.y;
    ustart = u.z;
    uend = u.w;
    kh = item % p.kv_heads;
    rb = (item / p.kv_heads) % p.plan_rbs;
    b = item / (p.kv_heads * p.plan_rbs);
  } else {
    const int units = p.batch * p.kv_heads;
    const int unit = blockIdx.x % units;
    rb = (int)(gridDim.x / units) - 1 - (int)(blockIdx.x / units);
    kh = unit % p.kv_heads;
    b = unit / p.kv_heads;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int nq = s1 - s0;
  const int g = p.num_heads / p.kv_heads;
  const int R = g * nq;
  const int row0 = rb * ROWS;
  if (row0 >= R) return;
  const int pastb = clamped_past(p, b, nq);
  const int total = seq_total(p, b, pastb, nq);
  int start, end;
  bool single;
  if (p.plan_items > 0) {
    start = ustart;
    end = max(ustart, min(uend, total));
    single = part == 0;
  } else {
    start = split * p.chunk;
    if (start >= total) return;
    end = start + min(p.chunk, total - start);
    single = start == 0 && end == total;
  }
  if (!single && p.part_o == nullptr) return;
  const int r_last = min(row0 + ROWS, R) - 1;
  const int hi_all = p.causal ? pastb + r_last / g + 1 : total;
  const int lo_all = p.window > 0 ? max(0, pastb + row0 / g - p.window + 1) : 0;
  const int t_first = max(start, (lo_all / KEYS) * KEYS);
  const int t_last = min(end, hi_all);
  const int nsteps = t_last > t_first ? (t_last - t_first + KEYS - 1) / KEYS : 0;

  const WaveInfo w = make_wave(p, D, b, kh, s0, pastb, total);
  // This lane's query row and the keys it sees.
  const int r = row0 + 32 * wave + c;
  const bool rvalid = r < R;
  const int qi = rvalid ? r / g : 0, head = kh * g + (rvalid ? r % g : 0);
  const int rpos = pastb + qi;
  const int vis_lo = p.window > 0 ? rpos - p.window + 1 : 0;
  const int vis_hi = rvalid ? (p.causal ? rpos + 1 : total) : -1;
  const uint32_t qxor = p.scale < 0.0f ? 0x80008000u : 0u;
  const float scale = fabsf(p.scale);
  // the row's log2-domain score scale and softcap factor (per lane for integer pages)
  float scale_log2 = fabsf(p.scale_log2);
  float cap_k = CAP ? scale / p.softcap : 0.0f;
  const float cap_l2 = p.softcap * kLog2e;
  u32x4 qv[KS];
  {
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       (((int64_t)(s0 + qi) * p.num_heads + head) * D + 8 * h) * 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qv[ks] = rvalid ? (ld16(qrow + 32 * ks) ^ qxor) : u32x4{0u, 0u, 0u, 0u};
    if constexpr (INTC || F8S) {
      // q * key scale in fp32 (dims 16 ks + 8 h + e of this lane), scaled by 2^-er so the bound
      // max|q| (the row) x max|scale| (the kv-head) lies below 2^14, then fp16 (RNE), one product
      // at a time: scores = 2^er * (q16 . codes).  fp8 pages: no scale here (the images hold the
      // dequantised keys), max|scale| = 1.
      const bool kpc = INTC && p.k_quant == PA_QUANT_PER_CHANNEL;
      float mq = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          mq = fmaxf(mq, fabsf(TT::to_f32((uint16_t)(qv[ks][e >> 1] >> (16 * (e & 1))))));
      mq = fmaxf(mq, other_half(mq));
      float ms = 1.0f;
      if constexpr (INTC) {
        if (kpc) {
          ms = 0.0f;
          for (int d = lane; d < D; d += 64) ms = fmaxf(ms, fabsf(p.k_scale[(int64_t)kh * D + d]));
          ms = wave_max_f(ms);
        } else {
          ms = fabsf(p.k_scale[0]);
        }
      }
      const float bound = mq * ms;
      const int er = bound > 0.0f ? __builtin_amdgcn_frexp_expf(bound) - 14 : 0;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int d0 = 16 * ks + 8 * h + 2 * m;
          const float s0v = INTC ? p.k_scale[kpc ? (int64_t)kh * D + d0 : 0] : 1.0f;
          const float s1v = INTC ? p.k_scale[kpc ? (int64_t)kh * D + d0 + 1 : 0] : 1.0f;
          const float a = TT::to_f32((uint16_t)qv[ks][m]) * s0v;
          const float c = TT::to_f32((uint16_t)(qv[ks][m] >> 16)) * s1v;
          const f16x2v ph = __builtin_convertvector(
              f32x2v{__builtin_ldexpf(a, -er), __builtin_ldexpf(c, -er)}, f16x2v);
          qv[ks][m] = __builtin_bit_cast(uint32_t, ph);
          __builtin_amdgcn_sched_barrier(0);  // the scale loads a pair at a time (registers)
        }
      scale_log2 = __builtin_ldexpf(scale_log2, er);
      cap_k = __builtin_ldexpf(cap_k, er);
    }
  }
  // Keys visible to some row [any_lo, any_hi) and to every row [all_lo, all_hi) of the wave.
  int any_lo = 0, any_hi = -1, all_lo = 0, all_hi = -1;
  {
    const int wr0 = row0 + 32 * wave;
    if (wr0 < R) {
      const int qf = wr0 / g, ql = (min(wr0 + 32, R) - 1) / g;
      any_hi = p.causal ? pastb + ql + 1 : total;
      all_hi = min(end, p.causal ? pastb + qf + 1 : total);
      any_lo = p.window > 0 ? pastb + qf - p.window + 1 : 0;
      all_lo = p.window > 0 ? pastb + ql - p.window + 1 : 0;
    }
  }
  f32x16 o[NQ];
#pragma unroll
  for (int nt = 0; nt < NQ; ++nt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[nt][i] = 0.0f;
  float m_run = kNegInf, l_part = 0.0f;
  // Value scale exponents the output quarters are accumulated in, and this wavefront's running
  // scale of the quarter it stages (bf16 values; fp16 values are used unscaled).
  constexpr int kS0 = std::is_same<TT, TBF16>::value ? -112 : 0;
  int sv[NQ];
#pragma unroll
  for (int nt = 0; nt < NQ; ++nt) sv[nt] = kS0;

  // Scores of the step at t0 from LDS buffer `buf`: two 32-key blocks, their accumulation chains
  // interleaved.
  auto scores = [&](const Buf& buf, f32x16(&sc)[KB]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[kb][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sc[kb] = mfma32<KT>(buf.k[kb][ks][lane], qv[ks], sc[kb]);
  };
  // Online softmax of the step at t0 over its scores, then O += P . V from buffer `buf`.
  // IMG: the accumulator's value exponent (output in units of 2^s_acc; no step seen yet: far below
  // any step's) -- each step's image holds its values in units of 2^sj.
  int s_acc = -(1 << 29);
  // WT: std::true_type in the loop instance for (sequence, kv-head) pairs with wide steps (see
  // kImgWideTag), std::false_type otherwise (the branch on a step's tag costs the common loop
  // registers, so it lives in a loop of its own)
  auto attend = [&](auto WT, const f32x16(&sc)[KB], int t0, const Buf& buf, int sj, int ek) __attribute__((always_inline)) {
    constexpr bool kWideLoop = kWide && decltype(WT)::value;
    // the step's score scale (fp8 pages: its keys are in units of 2^ek)
    const float sl2 = F8S ? __builtin_ldexpf(scale_log2, ek) : scale_log2;
    const float ck = F8S ? __builtin_ldexpf(cap_k, ek) : cap_k;
    float x[KB][16];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = sc[kb][i];
        if constexpr (CAP) v = softcap_log2(v, ck, cap_l2);
        x[kb][i] = v;
      }
    // per-score position tests only on steps some row does not see whole (one scalar branch):
    // key positions [vis_lo, min(end, vis_hi)) of this row, one unsigned range test each (three
    // compares per score kept their masks in scalar registers and spilled them).  Differences
    // taken modulo 2^32: the span is below 3 * 2^30 and a position below vis_lo lands above it.
    if (!(t0 >= all_lo && t0 + KEYS <= all_hi)) {
      const int hi_pos = min(end, vis_hi);
      const unsigned span = hi_pos > vis_lo ? (unsigned)hi_pos - (unsigned)vis_lo : 0u;
      const unsigned rel = (unsigned)(t0 + 4 * h) - (unsigned)vis_lo;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const unsigned off = 32 * kb + 8 * (i >> 2) + (i & 3);
          x[kb][i] = (rel + off < span) ? x[kb][i] : kNegInf;
        }
    }
    float lmax = kNegInf;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) lmax = fmaxf(lmax, x[kb][i]);
    lmax = fmaxf(lmax, other_half(lmax));
    if constexpr (!CAP) lmax *= sl2;
    if (__any(lmax > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, lmax);
      const float alpha = (m_run == kNegInf || m_new == kNegInf) ? 1.0f : exp2f(m_run - m_new);
      l_part *= alpha;
      m_run = m_new;
#pragma unroll
      for (int nt = 0; nt < NQ; ++nt) o[nt] *= alpha;
    }
    // value scales of this step: the output quarters follow a raised s exactly
    if constexpr (!IMG) {
      const int4 vs4 = *reinterpret_cast<const int4*>(buf.vs);
      const int vsn[4] = {__builtin_amdgcn_readfirstlane(vs4.x),
                          __builtin_amdgcn_readfirstlane(vs4.y),
                          __builtin_amdgcn_readfirstlane(vs4.z),
                          __builtin_amdgcn_readfirstlane(vs4.w)};
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        if (vsn[nt] != sv[nt]) {
          const float f = __builtin_ldexpf(1.0f, sv[nt] - vsn[nt]);
          o[nt] *= f;
          sv[nt] = vsn[nt];
        }
    }
    // IMG: bring the step's values and the accumulator to one exponent.  A step up to
    // kImgPShift below the accumulator enters through its probabilities, scaled by 2^-dsh (exact:
    // an offset in the exponent, and row sums weigh the fp16 probabilities by 2^dsh); otherwise
    // the accumulator moves to the step's exponent by an exact power of two -- upwards only while
    // that cannot overflow, which a step 2^-100 below output values that large could need: such a
    // step's values are negligible against the output and count in the row sums only.
    int dsh = 0;
    bool pv_on = true;
    bool wide = false;
    if constexpr (IMG) {
      if constexpr (kWideLoop) {  // raw bf16 values (see kImgWideTag); sj is the step's exponent
        wide = sj > kImgWideTag / 2;
        if (wide) sj -= kImgWideTag;
      }
      int d = __builtin_amdgcn_readfirstlane(s_acc - sj);
      bool up_ok = true;
      if (d > 84) {  // moving up by 2^d: only if the largest |output| stays below 2^120
        float om = 0.0f;
#pragma unroll
        for (int nt = 0; nt < NQ; ++nt)
#pragma unroll
          for (int i = 0; i < 16; ++i) om = fmaxf(om, fabsf(o[nt][i]));
        om = wave_max_f(om);
        up_ok = __builtin_amdgcn_readfirstlane(__builtin_ldexpf(om, min(d, 300)) <= 0x1p120f ? 1 : 0);
      }
      if (d < 0 || (d > kImgPShift && up_ok)) {
        const float f = __builtin_ldexpf(1.0f, d);
#pragma unroll
        for (int nt = 0; nt < NQ; ++nt) o[nt] *= f;
        s_acc = sj;
        d = 0;
      }
      pv_on = d <= kImgPShift;
      dsh = pv_on ? d : 0;
    }
    if (IMG && !pv_on) {
      const float m0 = (m_run == kNegInf) ? 0.0f : m_run;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          l_part += __builtin_amdgcn_exp2f(CAP ? x[kb][i] - m0 : __builtin_fmaf(x[kb][i], sl2, -m0));
      return;
    }
    if constexpr (kWideLoop) {
      if (wide) {
        // P.V in bf16 against the raw bf16 values: the probabilities in units of 2^-s_acc (the
        // output's units; exact powers of two) as bf16 hi parts, then the remainders as bf16 lo
        // parts (about 16 bits together), one operand set at a time in the registers the fp16
        // path uses; the row sum takes the probabilities themselves
        const float m0 = (m_run == kNegInf) ? 0.0f : m_run;
        // the value operands through an index the compiler cannot equate with the fp16 path's,
        // so their LDS reads are not hoisted above the branch (all of them live at once)
        int vl = lane;
        asm volatile("" : "+v"(vl));
        u32x4 pw[2 * KB];
#pragma unroll
        for (int part = 0; part < 2; ++part) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int m = 0; m < 8; ++m) {
              float pe[2];
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const float xv = x[kb][2 * m + j];
                const float pv = __builtin_amdgcn_exp2f(CAP ? xv - m0 : __builtin_fmaf(xv, sl2, -m0));
                if (part == 0) l_part += pv;
                pe[j] = __builtin_ldexpf(pv, -s_acc);
              }
              // hi = RNE bf16 of pe; lo = bf16 of pe - hi (hi read back exactly from its bits)
              const uint32_t hw = __builtin_bit_cast(
                  uint32_t, __builtin_convertvector(f32x2v{pe[0], pe[1]}, bf16x2v));
              uint32_t w = hw;
              if (part == 1) {
                const float h0 = __builtin_bit_cast(float, hw << 16);
                const float h1 = __builtin_bit_cast(float, hw & 0xffff0000u);
                w = __builtin_bit_cast(uint32_t,
                                       __builtin_convertvector(f32x2v{pe[0] - h0, pe[1] - h1}, bf16x2v));
              }
              pw[2 * kb + (m >> 2)][m & 3] = w;
            }
#pragma unroll
          for (int t = 0; t < 2 * KB; ++t)
#pragma unroll
            for (int nt = 0; nt < NQ; ++nt) o[nt] = mfma32<TBF16>(buf.v[t][nt][vl], pw[t], o[nt]);
        }
        return;
      }
    }
    const float msafe = ((m_run == kNegInf) ? 0.0f : m_run) + (float)dsh;
    const _Float16 lw = (_Float16)(float)(1 << dsh);
    u32x4 pb[2 * KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float pv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(CAP ? x[kb][i] - msafe
                                           : __builtin_fmaf(x[kb][i], sl2, -msafe));
      }
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const f16x2v ph = __builtin_convertvector(
              f32x2v{pv[8 * half + 2 * m], pv[8 * half + 2 * m + 1]}, f16x2v);
          pb[2 * kb + half][m] = __builtin_bit_cast(uint32_t, ph);
          // the row sum adds the fp16 probabilities the P.V product takes
          l_part = __builtin_amdgcn_fdot2(ph, f16x2v{lw, lw}, l_part, false);
        }
    }
#pragma unroll
    for (int t = 0; t < 2 * KB; ++t)
#pragma unroll
      for (int nt = 0; nt < NQ; ++nt)
        o[nt] = mfma32<TF16>(buf.v[t][nt][IMG ? lane : mx_vslot(lane)], pb[t], o[nt]);
  };
  // Steps some row of this wavefront sees.
  auto seen = [&](int t0) { return t0 < any_hi && t0 + KEYS > any_lo; };

  if constexpr (IMG) {
    const int64_t hb = (int64_t)b * p.kv_heads + kh;
    const char* img_hb = p.vimg + hb * p.img_steps * (int64_t)img_step_bytes(D);
    const int32_t* vstep_hb = p.vstep + hb * p.img_steps;
    // Direct LDS loads of step k + 1 into the other buffer while step k computes (every
    // wavefront finished reading that buffer before the barrier that ended iteration k - 1).
    // The value exponent of step k + 1 is loaded with its operands, at the start of iteration k,
    // so its latency hides under the step's compute like theirs.
    auto steps = [&](auto WT) __attribute__((always_inline)) {
      int sj = 0, sj_next = 0;
      if (nsteps > 0) {
        img_issue(lds[0], wave, lane, t_first, img_hb);
        sj_next = vstep_hb[t_first / KEYS];
      }
      wait_vmem();
      __syncthreads();
      for (int k = 0; k < nsteps; ++k) {
        const int t0 = t_first + KEYS * k;
        sj = __builtin_amdgcn_readfirstlane(sj_next);
        int ek = 0;
        if constexpr (F8S) {  // fp8 pages: key exponent above, value exponent below
          ek = sj >> 16;
          sj = (int)(int16_t)(sj & 0xffff);
        }
        if (k + 1 < nsteps) {
          img_issue(lds[(k + 1) & 1], wave, lane, t0 + KEYS, img_hb);
          sj_next = vstep_hb[t0 / KEYS + 1];
        }
        if (seen(t0)) {
          f32x16 sc[KB];
          scores(lds[k & 1], sc);
          attend(WT, sc, t0, lds[k & 1], sj, ek);
        }
        wait_vmem();
        __syncthreads();
      }
    };
    // pairs whose images hold a wide step (flag == this call's epoch) take the loop that reads
    // the step tags; stale flags of earlier calls hold other epochs
    if (kWide && __builtin_amdgcn_readfirstlane(p.img_wide[hb]) == p.img_epoch)
      steps(std::true_type{});
    else
      steps(std::false_type{});
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt) sv[nt] = s_acc;
  } else {
    PageWindow pw;
    window_at(pw, w, min(div_bs(t_first, w), w.max_blocks - 1), lane);
    MxStage st;
    int s_stage = kS0;
    if (nsteps > 0) {
      mx_load<TT>(w, pw, wave, lane, t_first, st);
      mx_store<TT>(lds[0], st, wave, lane, t_first, total, s_stage);
      if (nsteps > 1) mx_load<TT>(w, pw, wave, lane, t_first + KEYS, st);
    }
    __syncthreads();
    for (int k = 0; k < nsteps; ++k) {
      const int t0 = t_first + KEYS * k;
      if (seen(t0)) {
        f32x16 sc[KB];
        scores(lds[k & 1], sc);
        attend(std::false_type{}, sc, t0, lds[k & 1], 0, 0);
      }
      if (k + 1 < nsteps) mx_store<TT>(lds[(k + 1) & 1], st, wave, lane, t0 + KEYS, total, s_stage);
      if (k + 2 < nsteps) mx_load<TT>(w, pw, wave, lane, t0 + 2 * KEYS, st);
      __syncthreads();
    }
  }

  // Epilogue: row r's output in true units is o[nt] * 2^sv[nt]; lanes l and l ^ 32 hold dims
  // 8 i + 4 h + j of each quarter.
  if constexpr (INTC) {  // value scales per dim (per channel) or one per tensor
    const bool vpc = p.v_quant == PA_QUANT_PER_CHANNEL;
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[nt][4 * i + j] *= p.v_scale[vpc ? (int64_t)kh * D + 32 * nt + 8 * i + 4 * h + j : 0];
      __builtin_amdgcn_sched_barrier(0);  // the scale loads one quarter at a time (registers)
    }
  }
  const float l_row = l_part + other_half(l_part);
  if (!rvalid) return;
  const int64_t tok = s0 + qi;
  const float sink_c = sink_logit<TT>(p, head);
  if (single) {
    const float f = finalize_factor(m_run, l_row, sink_c);
    typename TT::raw* dst = reinterpret_cast<typename TT::raw*>(p.out) + (tok * p.num_heads + head) * D;
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt) {
      const float fq = __builtin_ldexpf(f, sv[nt]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x2 pk;
#pragma unroll
        for (int m = 0; m < 2; ++m)
          pk[m] = (uint32_t)TT::from_f32(o[nt][4 * i + 2 * m] * fq) |
                  ((uint32_t)TT::from_f32(o[nt][4 * i + 2 * m + 1] * fq) << 16);
        *reinterpret_cast<u32x2*>(dst + 32 * nt + 8 * i + 4 * h) = pk;
      }
    }
  } else if (p.plan_items == 0) {
    // split-K chunk of the grid-order launch: fp32 partial (O, m, l) for split_reduce_kernel
    const int64_t pi = (tok * p.num_heads + head) * p.max_splits + split;
    float* dstf = p.part_o + pi * D;
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = __builtin_ldexpf(o[nt][4 * i + j], sv[nt]);
        *reinterpret_cast<f32x4*>(dstf + 32 * nt + 8 * i + 4 * h) = v4;
      }
    if (h == 0) {
      p.part_ml[pi * 2 + 0] = m_run;
      p.part_ml[pi * 2 + 1] = l_row;
    }
  } else {
    // fp16 partial row scaled by 2^-e (e from the row's largest |O|), e folded into (m, l)
    float mx = 0.0f;
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt) {
      float q = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) q = fmaxf(q, fabsf(o[nt][i]));
      mx = fmaxf(mx, __builtin_ldexpf(q, sv[nt]));
    }
    mx = fmaxf(mx, other_half(mx));
    const int ex = min(max(__builtin_amdgcn_frexp_expf(mx), -64), 126);
    const int64_t pi = ((int64_t)item * 2 + part - 1) * ROWS + (r - row0);
    char* dstb = reinterpret_cast<char*>(p.part_o) + pi * D * 2;
#pragma unroll
    for (int nt = 0; nt < NQ; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x2 pk;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const _Float16 a = (_Float16)__builtin_ldexpf(o[nt][4 * i + 2 * m], sv[nt] - ex);
          const _Float16 bb = (_Float16)__builtin_ldexpf(o[nt][4 * i + 2 * m + 1], sv[nt] - ex);
          pk[m] = (uint32_t)__builtin_bit_cast(uint16_t, a) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, bb) << 16);
        }
        *reinterpret_cast<u32x2*>(dstb + (32 * nt + 8 * i + 4 * h) * 2) = pk;
      }
    if (h == 0) {
      p.part_ml[pi * 2 + 0] = m_run + (float)ex;
      p.part_ml[pi * 2 + 1] = __builtin_ldexpf(l_row, -ex);
    }
  }
}

// ----------------------------------------------------------------------------- planned prefill
// Split threshold of the plan: items with more visible keys than PA_PLAN_SPLIT_PCT percent of a
// slot's even share of all keys (and at least PA_PLAN_SPLIT_MIN keys) run as two halves.
// C4 attention launch by threshold: 25 % 393 us, 35 % 392-395, 45 % 372-382, 60 % 391-396,
// 80 % 388-389, 100 % 384-389; with the fp16 partials: 30 % 354-357, 38 % 356, 45 % 340-344,
// 55 % 342-343.
#ifndef PA_PLAN_SPLIT_PCT
#define PA_PLAN_SPLIT_PCT 45
#endif
#ifndef PA_PLAN_SPLIT_MIN
#define PA_PLAN_SPLIT_MIN 2048
#endif
// Visible key range [first, end) of item i (the keys some row of the row block can see), the
// same bounds the prefill kernel derives; end < 0 when the row block holds no rows.
struct ItemKeys {
  int first, end;
};
__device__ __forceinline__ ItemKeys item_keys(const AttnParams& p, int i) {
  const int g = p.num_heads / p.kv_heads;
  const int rb = (i / p.kv_heads) % p.plan_rbs, b = i / (p.kv_heads * p.plan_rbs);
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int R = g * (s1 - s0);
  const int row0 = rb * kPrefillRows;
  if (row0 >= R) return ItemKeys{0, -1};
  const int pastb = clamped_past(p, b, s1 - s0);
  const int total = seq_total(p, b, pastb, s1 - s0);
  // Operand images cover img_steps steps of every (sequence, kv-head): a sequence with more keys
  // (beyond the caller's context bound) gets no work, so nothing reads past its images.
  if (p.img_steps > 0 && total > p.img_steps * p.plan_step) return ItemKeys{0, -1};
  const int r_last = min(row0 + kPrefillRows, R) - 1;
  const int hi = p.causal ? pastb + r_last / g + 1 : total;
  const int lo = p.window > 0 ? max(0, pastb + row0 / g - p.window + 1) : 0;
  const int first = (lo / p.plan_step) * p.plan_step;
  return ItemKeys{first, max(first, min(total, hi))};
}

// One workgroup: the work units of every item, longest first.  An item whose visible keys
// exceed PA_PLAN_SPLIT_PCT % of a slot's even share of all keys (plan_slots workgroup slots) is
// split into two
// halves at a 32-key boundary.  Units are ordered by a counting sort on their 32-key step count
// (LDS histogram, descending); the order inside a bucket is whatever the atomics give, which
// changes nothing in the results (every unit writes its own rows or partial).
//
// With operand images, workgroups 1.. of the same launch write the images (image_steps), which
// need nothing from the plan: they cost no launch of their own and run on other CUs while
// workgroup 0 plans.

// Operand images (AttnParams::vimg): each img_keys(D)-key step of (sequence, kv-head) holds the
// step's LDS operand buffer of prefill_mx_kernel byte for byte, so the kernel's staging is a plain
// copy:
//   keys (img_keys(D) x D x 2 bytes): item (kb, ks), lane l holds bytes 32 ks + 16 (l / 32) ..
//   + 15 of the row slice of key 32 kb + l % 32 -- the rows gathered from the pages (or the
//   caller's new rows);
//   values (as many bytes): the rows converted to fp16 under the step's scale 2^-s -- bf16 values: s puts
//   the step's largest |value| into [2^14, 2^15) of fp16 (exact conversion; values below 2^-29 of
//   it lose bits in the fp16 subnormal range); fp16 values: s = 0 -- regrouped through LDS into
//   the P.V A-operand layout: item (t, nt), lane l holds dim 32 nt + l % 32 of keys 16 t + 4 h + e
//   and then 16 t + 8 + 4 h + e (e < 4, h = l / 32).
// Rows at or past the sequence end are zero.  Steps of img_keys(D) keys, NT / 256 consecutive
// steps per workgroup, 256 threads each: thread (row r, piece q) moves 16-byte chunks
// dc = CH q .. CH q + CH - 1 of key and value row r; key chunk dc goes to item (kb = r / 32,
// ks = dc / 2), lane 32 (dc % 2) + r % 32.  The step's exponent goes to vstep.
// One group of NT / 256 image steps of one (sequence, kv-head): id -> (step group, kv-head,
// sequence); the rows are loaded into registers by img_load and written out by img_store.
template <int NT, int D>
struct ImgGroup {
  // PCS threads per row, each moving CH of the row's D / 8 16-byte chunks
  static constexpr int KEYS = img_keys(D), PCS = 256 / KEYS, CH = (D / 8) / PCS;
  static_assert(CH * PCS * 8 == D, "whole chunks per thread");
  u32x4 kx[CH], vx[CH];
  float ks, vs;  // fp8 pages: the row's key / value page scales
  int64_t hb;
  int j, r, q;
  bool step_live;
};

// Page codes of integer caches (KC: kImgI8 / kImgI4) load as 32-bit words and widen exactly to
// fp16 (int8 codes; int4 nibbles, low nibble first, biased by +8), so the images hold the codes
// and the scales apply outside the products.  fp8 pages (kImgF8) load their e4m3 codes (words 0
// and 1 of each chunk) and the row's page scales; img_store dequantises them (code x scale in
// fp32) and writes keys and values as fp16 under per-step powers of two.
constexpr int kImgT = 0, kImgI8 = 1, kImgI4 = 2, kImgF8 = 3;
template <int KC>
__device__ __forceinline__ uint32_t f16_pair(int a, int b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)b) << 16);
}
template <int KC, int CH>
__device__ __forceinline__ void load_codes(const char* row, bool live, u32x4 (&x)[CH]) {
  if constexpr (KC == kImgI8) {
    // 8 codes per 16-byte fp16 chunk: two words
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      uint32_t w[2];
#pragma unroll
      for (int k = 0; k < 2; ++k)
        w[k] = live ? reinterpret_cast<const uint32_t*>(row)[2 * i + k] : 0u;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int c0 = (int8_t)(w[k] & 0xff), c1 = (int8_t)((w[k] >> 8) & 0xff);
        const int c2 = (int8_t)((w[k] >> 16) & 0xff), c3 = (int8_t)(w[k] >> 24);
        x[i][2 * k] = f16_pair<KC>(c0, c1);
        x[i][2 * k + 1] = f16_pair<KC>(c2, c3);
      }
    }
  } else {
    // 8 codes per chunk: one word of nibbles
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const uint32_t w = live ? reinterpret_cast<const uint32_t*>(row)[i] : 0x88888888u;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        x[i][k] = f16_pair<KC>((int)((w >> (8 * k)) & 15u) - 8, (int)((w >> (8 * k + 4)) & 15u) - 8);
    }
  }
}

template <int NT, int D, int KC>
__device__ __forceinline__ void img_load(const AttnParams& p, int id, ImgGroup<NT, D>& g) {
  constexpr int SPW = NT / 256, KEYS = img_keys(D), PCS = ImgGroup<NT, D>::PCS;
  constexpr int CH = ImgGroup<NT, D>::CH;
  const int nj = (p.img_steps + SPW - 1) / SPW;
  const int jb = id % nj, kh = (id / nj) % p.kv_heads, b = min(id / (nj * p.kv_heads), p.batch - 1);
  const int s0 = min(max(p.cum[b], 0), p.num_tokens);
  const int s1 = min(max(p.cum[b + 1], s0), p.num_tokens);
  const int pastb = clamped_past(p, b, s1 - s0);
  const int total = seq_total(p, b, pastb, s1 - s0);
  const int tid = threadIdx.x;
  g.j = jb * SPW + tid / 256;
  g.step_live = s1 > s0 && g.j < p.img_steps && g.j * KEYS < total;
  g.hb = (int64_t)b * p.kv_heads + kh;
  g.r = (tid & 255) / PCS;
  g.q = tid % PCS;
  WaveInfo w = make_wave(p, D, b, kh, s0, pastb, total);
  const int pos = g.j * KEYS + g.r;
  const bool live = g.step_live && pos < total;
  if constexpr (KC == kImgT) {
    const char* ks = live ? row_ptr(w, pos, false, D) + 16 * CH * g.q : nullptr;
    const char* vs = live ? row_ptr(w, pos, true, D) + 16 * CH * g.q : nullptr;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      g.kx[i] = live ? ld16(ks + 16 * i) : u32x4{0u, 0u, 0u, 0u};
      g.vx[i] = live ? ld16(vs + 16 * i) : u32x4{0u, 0u, 0u, 0u};
    }
  } else {
    // code rows: D bytes (int8, fp8) or D / 2 (int4) per kv-head
    constexpr int RB = KC == kImgI4 ? D / 2 : D;
    w.rowb = w.lin_row0 >= 0 ? RB : (int64_t)p.kv_heads * RB;
    w.hoff = w.lin_row0 >= 0 ? 0 : (int64_t)kh * RB;
    const int cb = (KC == kImgI4 ? 4 : 8) * CH * g.q;  // bytes before this thread's codes
    const char* ks = live ? row_ptr(w, pos, false, D) + cb : nullptr;
    const char* vs = live ? row_ptr(w, pos, true, D) + cb : nullptr;
    if constexpr (KC == kImgF8) {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const u32x2 kw = live ? reinterpret_cast<const u32x2*>(ks)[i] : u32x2{0u, 0u};
        const u32x2 vw = live ? reinterpret_cast<const u32x2*>(vs)[i] : u32x2{0u, 0u};
        g.kx[i] = u32x4{kw[0], kw[1], 0u, 0u};
        g.vx[i] = u32x4{vw[0], vw[1], 0u, 0u};
      }
      // page scales of the row's block (paged caches only: every row is read from the pages)
      g.ks = g.vs = 0.0f;
      if (live) {
        const int bi = min(div_bs(pos, w), w.max_blocks - 1);
        const int64_t blk = min(max((int64_t)w.bt[bi], (int64_t)0), w.num_blocks - 1);
        g.ks = p.k_scale[blk * p.kv_heads + kh];
        g.vs = p.v_scale[blk * p.kv_heads + kh];
      }
    } else {
      load_codes<KC, CH>(ks, live, g.kx);
      load_codes<KC, CH>(vs, live, g.vx);
    }
  }
}

// fp8 pages: the largest |e4m3 code| of a thread's chunks (the magnitude order of e4m3 is the
// integer order of its low seven bits), then as fp32.  A NaN code (0x7f) counts as the largest
// finite magnitude, 0x7e = 448, so the step's exponent still keeps its finite values in fp16 range
// (the NaN itself converts to an fp16 NaN).
template <int CH>
__device__ __forceinline__ float f8_chunks_absmax(const u32x4 (&x)[CH]) {
  using u8x4 = unsigned char __attribute__((ext_vector_type(4)));
  u8x4 m = u8x4{0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < CH; ++i)
#pragma unroll
    for (int k = 0; k < 2; ++k)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(u8x4, x[i][k] & 0x7f7f7f7fu));
  const unsigned c = max(max((unsigned)m[0], (unsigned)m[1]), max((unsigned)m[2], (unsigned)m[3]));
  return e4m3_to_f32(min(c, 0x7eu));
}

// fp8 pages: 8 e4m3 codes (words 0, 1 of x) times f (page scale x 2^-s) as 4 fp16 pairs (RNE).
// Each code pair widens exactly to fp16 with one v_cvt_scalef32_pk_f16_fp8 at scale 1.0 (the
// decode's widening: every e4m3 value is an fp16 value, NaN stays NaN), then to fp32.
__device__ __forceinline__ u32x4 f8_chunk_f16(const u32x4& x, float f) {
  const f16x2v c[4] = {
      __builtin_bit_cast(f16x2v, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[0], 1.0f, false)),
      __builtin_bit_cast(f16x2v, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[0], 1.0f, true)),
      __builtin_bit_cast(f16x2v, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[1], 1.0f, false)),
      __builtin_bit_cast(f16x2v, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[1], 1.0f, true))};
  u32x4 o;
#pragma unroll
  for (int m = 0; m < 4; ++m)
    o[m] = __builtin_bit_cast(
        uint32_t, __builtin_convertvector(f32x2v{(float)c[m][0] * f, (float)c[m][1] * f}, f16x2v));
  return o;
}

// Exponent s of a step whose largest |value| is mx: mx * 2^-s lies in [2^14, 2^15) of fp16; the
// biased form (s + 256 > 0, 0 for a step of zeros) takes the group maximum as an integer.
__device__ __forceinline__ int f8_step_exp_biased(float mx) {
  return mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) - 15 + 256 : 0;
}

template <typename TT, int NT, int D, int KC>
__device__ __forceinline__ void img_store(const AttnParams& p, ImgGroup<NT, D>& g,
                                          uint32_t (*rows)[img_keys(D)][D / 2 + 1], int* emax) {
  constexpr int KB = img_keys(D) / 32, CH = ImgGroup<NT, D>::CH, NQ = D / 32;
  constexpr int SB = img_step_bytes(D);
  // bf16 pages take a per-step scale; fp16 pages and integer codes (exact in fp16) go as they are
  constexpr bool BF = std::is_same<TT, TBF16>::value && KC == kImgT;
  const int tid = threadIdx.x, grp = tid / 256, r = g.r, q = g.q;
  char* dst = p.vimg + (g.hb * p.img_steps + g.j) * (int64_t)SB;
  auto store_keys = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int dc = CH * q + i;
      *reinterpret_cast<u32x4*>(dst + ((((r >> 5) * (D / 16) + (dc >> 1)) * 64) + 32 * (dc & 1) + (r & 31)) * 16) =
          g.kx[i];
    }
  };
  if (KC != kImgF8 && g.step_live) store_keys();
  // the step's largest biased exponent of |value| (bf16; every wavefront of a group, then LDS)
  int e = 0, ek = 0;
  if constexpr (KC == kImgF8) {  // values and keys: exponents of the dequantised maxima
    e = wave_max_nonneg(f8_step_exp_biased(f8_chunks_absmax<CH>(g.vx) * fabsf(g.vs)));
    ek = wave_max_nonneg(f8_step_exp_biased(f8_chunks_absmax<CH>(g.kx) * fabsf(g.ks)));
  }
  if constexpr (BF) {
    // largest magnitude and smallest nonzero magnitude (zeros read as 0x7fff), as bit patterns
    uint32_t mx = 0, mn = 0x7fff7fffu;
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u16x2 a = __builtin_bit_cast(u16x2, g.vx[i][m] & 0x7fff7fffu);
        mx = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, mx), a));
        const u16x2 z = __builtin_bit_cast(u16x2, (a == (unsigned short)0)) & (unsigned short)0x7fff;
        mn = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, mn), a + z));
      }
    e = wave_max_nonneg((int)(max(mx & 0xffffu, mx >> 16) >> 7));
    // 255 - the smallest nonzero biased exponent (a max, so the group reduction is one atomicMax)
    ek = wave_max_nonneg(255 - (int)(min(mn & 0xffffu, mn >> 16) >> 7));
  }
  if (tid < 2 * (NT / 256)) emax[tid] = 0;
  __syncthreads();
  if ((tid & 63) == 0) {
    atomicMax(&emax[grp], e);
    if (KC == kImgF8 || BF) atomicMax(&emax[NT / 256 + grp], ek);
  }
  __syncthreads();
  // bf16: s = emax - 141 puts the largest value into [2^14, 2^15) of fp16; fp16: s = 0.  A wide
  // bf16 step (nonzero values kImgWideSpan or more binades apart) keeps its values as they are.
  int sc = BF ? max(emax[grp] - 141, -112) : 0;
  // (heads up to 128: the prefill kernel at head 256 has no loop for wide steps)
  const bool wide = BF && D <= 128 && emax[grp] - (255 - emax[NT / 256 + grp]) >= kImgWideSpan;
  if constexpr (KC == kImgF8) {
    // fp8: code x page scale x 2^-s in fp16 (keys under their own s), both exponents to vstep
    const int sv = emax[grp] > 0 ? emax[grp] - 256 : 0;
    const int sk = emax[NT / 256 + grp] > 0 ? emax[NT / 256 + grp] - 256 : 0;
    const float fk = __builtin_ldexpf(g.ks, -sk), fv = __builtin_ldexpf(g.vs, -sv);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      g.kx[i] = f8_chunk_f16(g.kx[i], fk);
      g.vx[i] = f8_chunk_f16(g.vx[i], fv);
    }
    if (g.step_live) store_keys();
    sc = (int)((uint32_t)sk << 16 | ((uint32_t)sv & 0xffffu));
  }
  if (wide) {
    sc += kImgWideTag;
    if (g.step_live && (tid & 255) == 0) p.img_wide[g.hb] = p.img_epoch;
  }
  if (BF && !wide) {
    // bf16 exponent E -> fp16 exponent E - 112 - s: subtract (112 + s) << 7 from the magnitude
    // bits (saturating: values below the fp16 range flush towards zero), shift into place
    const unsigned short bias = (unsigned short)((112 + sc) << 7);
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        u16x2 a = __builtin_bit_cast(u16x2, g.vx[i][m] & 0x7fff7fffu);
        a = __builtin_elementwise_sub_sat(a, u16x2{bias, bias});
        a = a << (unsigned short)3;
        g.vx[i][m] = (g.vx[i][m] & 0x80008000u) | __builtin_bit_cast(uint32_t, a);
      }
  }
#pragma unroll
  for (int i = 0; i < CH; ++i)
#pragma unroll
    for (int m = 0; m < 4; ++m) rows[grp][r][4 * (CH * q + i) + m] = g.vx[i][m];
  __syncthreads();
  if (g.step_live) {
    if ((tid & 255) == 0) p.vstep[g.hb * p.img_steps + g.j] = sc;
    // value regroup: task (t, h, nt, dim pair dp) -> slots of lanes 32 h + 2 dp (+1) of item
    // (t, nt)
    char* vdst = dst + SB / 2;
    constexpr int NTASK = 64 * KB * NQ;  // (t < 2 KB, h < 2, nt < NQ, dp < 16)
#pragma unroll
    for (int rep = 0; rep < (NTASK + 255) / 256; ++rep) {
      const int task = (tid & 255) + 256 * rep;
      if (task >= NTASK) break;
      const int dp = task & 15, h = (task >> 4) & 1, nt = (task >> 5) % NQ, t = (task >> 5) / NQ;
      u32x4 lo, hi;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        // elements 2 e2, 2 e2 + 1: keys 16 t + 4 h + (e & 3) + 8 (e >> 2)
        const int ka = 16 * t + 4 * h + ((2 * e2) & 3) + 8 * ((2 * e2) >> 2);
        const uint32_t wa = rows[grp][ka][16 * nt + dp], wb = rows[grp][ka + 1][16 * nt + dp];
        lo[e2] = __builtin_amdgcn_perm(wb, wa, 0x05040100u);
        hi[e2] = __builtin_amdgcn_perm(wb, wa, 0x07060302u);
      }
      u32x4* o = reinterpret_cast<u32x4*>(vdst + (NQ * t + nt) * 1024) + 32 * h + 2 * dp;
      o[0] = lo;
      o[1] = hi;
    }
  }
}

// Image workgroup `id`: one group of NT / 256 steps.  (A persistent variant, each workgroup
// loading its next group before writing the current one, measured no faster.)
template <typename TT, int NT, int D, int KC>
__device__ __forceinline__ void image_steps(const AttnParams& p, int id) {
  constexpr int SPW = NT / 256;
  __shared__ uint32_t rows[SPW][img_keys(D)][D / 2 + 1];  // fp16 value rows, one word = two dims
  __shared__ int emax[2 * SPW];  // per step: value exponent, then (fp8 pages) key exponent
  const int nj = (p.img_steps + SPW - 1) / SPW;
  if (id >= nj * p.kv_heads * p.batch) return;
  ImgGroup<NT, D> g;
  img_load<NT, D, KC>(p, id, g);
  img_store<TT, NT, D, KC>(p, g, rows, emax);
}

template <int NT, typename TT, int IMGD, int KC = kImgT>
__global__ __launch_bounds__(NT) void prefill_plan_kernel(const AttnParams p) {
  if constexpr (IMGD > 0) {  // head size of the operand images; KC: the pages' element kind
    if (blockIdx.x > 0) {
      image_steps<TT, NT, IMGD, KC>(p, (int)blockIdx.x - 1);
      return;
    }
  }
  constexpr int NB = 1024;  // buckets of 32-key steps (the last one holds everything longer)
  __shared__ int hist[NB];
  __shared__ unsigned long long total_keys;
  const int tid = threadIdx.x;
  for (int i = tid; i < NB; i += NT) hist[i] = 0;
  if (tid == 0) total_keys = 0;
  __syncthreads();
  // The key ranges of this thread's first kCached items stay in registers for the later passes
  // (each costs two dependent metadata loads).
  constexpr int kCached = 4;
  ItemKeys cached[kCached];
  auto keys = [&](int j, int i) { return j < kCached ? cached[j] : item_keys(p, i); };
  unsigned long long mine = 0;
  for (int i = tid, j = 0; i < p.plan_items; i += NT, ++j) {
    const ItemKeys k = item_keys(p, i);
#pragma unroll
    for (int c = 0; c < kCached; ++c)
      if (c == j) cached[c] = k;
    if (k.end >= 0) mine += (unsigned long long)(k.end - k.first);
  }
  // Wave sums first: one LDS atomic per wavefront instead of one per thread on one address.
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) mine += __shfl_xor(mine, o, 64);
  if ((tid & 63) == 0) atomicAdd(&total_keys, mine);
  __syncthreads();
  const long long thr = max((long long)PA_PLAN_SPLIT_MIN,
                           (long long)(total_keys * PA_PLAN_SPLIT_PCT / 100) / max(p.plan_slots, 1));
  const int step = p.plan_step;
  auto bucket = [&](int len) { return NB - 1 - min((len + step - 1) / step, NB - 1); };
  auto split_of = [&](const ItemKeys& k) {
    return k.end - k.first > thr && k.end - k.first >= 2 * step;
  };
  // Halves split at a key-step boundary.
  auto mid_of = [&](const ItemKeys& k) {
    return k.first + (((k.end - k.first + step - 1) / step + 1) / 2) * step;
  };
  for (int i = tid, j = 0; i < p.plan_items; i += NT, ++j) {
    const ItemKeys k = keys(j, i);
    if (k.end < 0) {
      p.plan_split[i] = 0;
      continue;
    }
    const bool sp = split_of(k);
    p.plan_split[i] = sp ? 1 : 0;
    if (sp) {
      const int mid = mid_of(k);
      atomicAdd(&hist[bucket(mid - k.first)], 1);
      atomicAdd(&hist[bucket(k.end - mid)], 1);
    } else {
      atomicAdd(&hist[bucket(k.end - k.first)], 1);
    }
  }
  __syncthreads();
  {  // exclusive scan of the histogram, one bucket per thread: wave scans, then the wave sums
    static_assert(NT == NB && NT % 64 == 0 && NT / 64 <= 64, "one bucket per thread");
    __shared__ int wsum[NT / 64];
    const int lane = tid & 63, wave = tid >> 6;
    const int c = hist[tid];
    int x = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (wave == 0) {
      int v = lane < NT / 64 ? wsum[lane] : 0;
#pragma unroll
      for (int o = 1; o < NT / 64; o <<= 1) {
        const int y = __shfl_up(v, o, 64);
        if (lane >= o) v += y;
      }
      if (lane < NT / 64) wsum[lane] = v;
    }
    __syncthreads();
    const int excl = x - c + (wave > 0 ? wsum[wave - 1] : 0);
    hist[tid] = excl;
    if (tid == NT - 1) p.plan_info[0] = excl + c;
  }
  __syncthreads();
  int4* plan = reinterpret_cast<int4*>(p.plan);
  for (int i = tid, j = 0; i < p.plan_items; i += NT, ++j) {
    const ItemKeys k = keys(j, i);
    if (k.end < 0) continue;
    if (split_of(k)) {
      const int mid = mid_of(k);
      plan[atomicAdd(&hist[bucket(mid - k.first)], 1)] = int4{i, 1, k.first, mid};
      plan[atomicAdd(&hist[bucket(k.end - mid)], 1)] = int4{i, 2, mid, k.end};
    } else {
      plan[atomicAdd(&hist[bucket(k.end - k.first)], 1)] = int4{i, 0, k.first, k.end};
    }
  }
}

// Merge the two halves of each split item: one workgroup per kPrefillMergeRows rows of an
// item's row block, D/8 lanes per row (16 bytes of fp16 each); every load of the workgroup is
// issued before the first is used, so the merge costs one memory latency after the split flag.  The halves'
// partials are fp16 rows scaled by a power of two folded into their (m, l) (store_rows with
// half_part): the log-sum-exp merge below takes them as they are.
constexpr int kPrefillMergeRows = 32;
// Threads of a merge workgroup at head size D: D / 8 per row, as many rows per pass as divide
// kPrefillMergeRows within 256 threads (head 96: 12 x 16 = 192).
__host__ __device__ constexpr int merge_rows_per_pass(int D) {
  return (256 / (D / 8)) >= 32 ? 32 : (256 / (D / 8)) >= 16 ? 16 : 8;
}
__host__ __device__ constexpr int merge_threads(int D) { return (D / 8) * merge_rows_per_pass(D); }
template <typename TT, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(const AttnParams p) {
  constexpr int QPR = D / 8;              // lanes per row, 8 elements (16 bytes of fp16) each
  constexpr int RPP = merge_rows_per_pass(D);  // rows per pass
  constexpr int NP = kPrefillMergeRows / RPP;
  static_assert(kPrefillRows % kPrefillMergeRows == 0 && kPrefillMergeRows % RPP == 0, "merge tiling");
  constexpr int CH = kPrefillRows / kPrefillMergeRows;
  const int i = blockIdx.x / CH;
  if (!p.plan_split[i]) return;
  const int g = p.num_heads / p.kv_heads;
  const int kh = i % p.kv_heads, rb = (i / p.kv_heads) % p.plan_rbs;
  const int b = i / (p.kv_heads * p.plan_rbs);
  const int row0 = rb * kPrefillRows;
  const int q = threadIdx.x % QPR;
  const int rbase = (blockIdx.x % CH) * kPrefillMergeRows + threadIdx.x / QPR;
  // Every load in one round trip: the sequence bounds, both halves' (m, l) and rows, the sink.
  // Rows past the block's last row read in-bounds workspace rows and store nothing.
  const int cb0 = p.cum[b], cb1 = p.cum[b + 1];
  float2 a[NP], c[NP];
  u32x4 ha[NP], hc[NP];  // fp16 partial rows (store_rows, half_part)
  float sk[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int r = rbase + j * RPP;
    const int64_t r0 = ((int64_t)i * 2) * kPrefillRows + r, r1 = r0 + kPrefillRows;
    a[j] = reinterpret_cast<const float2*>(p.part_ml)[r0];
    c[j] = reinterpret_cast<const float2*>(p.part_ml)[r1];
    ha[j] = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(p.part_o) + r0 * D * 2)[q];
    hc[j] = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(p.part_o) + r1 * D * 2)[q];
    sk[j] = sink_logit<TT>(p, kh * g + (row0 + r) % g);
  }
  const int s0 = min(max(cb0, 0), p.num_tokens);
  const int s1 = min(max(cb1, s0), p.num_tokens);
  const int rows = min(kPrefillRows, g * (s1 - s0) - row0);
  auto widen = [](uint32_t w2, int e) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w2 >> (16 * e)));
  };
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int r = rbase + j * RPP;
    if (r >= rows) continue;
    const float M = fmaxf(a[j].x, c[j].x);
    const float wa = (a[j].x == kNegInf) ? 0.0f : exp2f(a[j].x - M);
    const float wc = (c[j].x == kNegInf) ? 0.0f : exp2f(c[j].x - M);
    const int rr = row0 + r;
    const int h = kh * g + rr % g;
    const int64_t t = s0 + rr / g;
    const float f = finalize_factor(M, a[j].y * wa + c[j].y * wc, sk[j]);
    u32x4 pk;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float lo = (widen(ha[j][m], 0) * wa + widen(hc[j][m], 0) * wc) * f;
      const float hi = (widen(ha[j][m], 1) * wa + widen(hc[j][m], 1) * wc) * f;
      pk[m] = (uint32_t)TT::from_f32(lo) | ((uint32_t)TT::from_f32(hi) << 16);
    }
    *reinterpret_cast<u32x4*>(reinterpret_cast<typename TT::raw*>(p.out) +
                              (t * p.num_heads + h) * D + 8 * q) = pk;
  }
}

// Page kinds of the prefill launch: pages in the activation dtype, integer codes, fp8 codes.
constexpr int kPkT = 0, kPkInt = 1, kPkF8 = 2;

template <typename TT, int D>
hipError_t launch_d(const AttnParams& p, dim3 grid, hipStream_t s, int pk = kPkT) {
  constexpr int NG = kPrefillGroups;
  if (p.bias != nullptr) {
    // GroupQueryAttention's additive bias: prefill_kernel at every head size, pages in the
    // activation dtype, no operand images
    if (p.vimg != nullptr || pk != kPkT) return hipErrorInvalidValue;
    if (p.softcap > 0.0f)
      hipLaunchKernelGGL((prefill_kernel<TT, D, true, NG, true>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((prefill_kernel<TT, D, false, NG, true>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
  }
  if constexpr (img_head(D)) {
    if (p.vimg != nullptr) {
      if (pk == kPkInt) {
        if (p.softcap > 0.0f)
          hipLaunchKernelGGL((prefill_mx_kernel<TT, true, true, D, true>), grid, dim3(256), 0, s, p);
        else
          hipLaunchKernelGGL((prefill_mx_kernel<TT, false, true, D, true>), grid, dim3(256), 0, s, p);
      } else if (pk == kPkF8) {
        if (p.softcap > 0.0f)
          hipLaunchKernelGGL((prefill_mx_kernel<TT, true, true, D, false, true>), grid, dim3(256), 0, s, p);
        else
          hipLaunchKernelGGL((prefill_mx_kernel<TT, false, true, D, false, true>), grid, dim3(256), 0, s, p);
      } else if (p.softcap > 0.0f) {
        hipLaunchKernelGGL((prefill_mx_kernel<TT, true, true, D>), grid, dim3(256), 0, s, p);
      } else {
        hipLaunchKernelGGL((prefill_mx_kernel<TT, false, true, D>), grid, dim3(256), 0, s, p);
      }
      return hipGetLastError();
    }
  }
  if (pk != kPkT) return hipErrorInvalidValue;  // byte-coded pages run over images only
  // Head 128 without images: fp16 pages on the 32x32 kernel with in-loop staging (fp16 values as
  // they are); bf16 pages on prefill_kernel below, whose P.V takes the raw bf16 values (hi + lo
  // probabilities) -- the in-loop fp16 conversion of bf16 values keeps a running power of two per
  // quarter, under which values 2^-29 below the largest seen so far lose bits.
  if constexpr (D == 128 && !std::is_same<TT, TBF16>::value) {
    const bool cap = p.softcap > 0.0f;
    if (cap) {
      hipLaunchKernelGGL((prefill_mx_kernel<TT, true, false>), grid, dim3(256), 0, s, p);
    } else {
      hipLaunchKernelGGL((prefill_mx_kernel<TT, false, false>), grid, dim3(256), 0, s, p);
    }
    return hipGetLastError();
  }
  if (p.softcap > 0.0f)
    hipLaunchKernelGGL((prefill_kernel<TT, D, true, NG>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((prefill_kernel<TT, D, false, NG>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename TT>
hipError_t launch_t(const AttnParams& p, dim3 grid, hipStream_t s, int pk = kPkT) {
  switch (p.head_dim) {
    case 64: return launch_d<TT, 64>(p, grid, s, pk);
    case 96: return launch_d<TT, 96>(p, grid, s, pk);
    case 128: return launch_d<TT, 128>(p, grid, s, pk);
    case 256: return launch_d<TT, 256>(p, grid, s, pk);
    default: return hipErrorInvalidValue;
  }
}

// The merge of the planned prefill's split items (heads whose rows tile the merge workgroup).
template <typename TT>
hipError_t launch_prefill_merge(const AttnParams& p, hipStream_t s) {
  const dim3 grid(p.plan_items * (kPrefillRows / kPrefillMergeRows));
  switch (p.head_dim) {
    case 64: hipLaunchKernelGGL((prefill_merge_kernel<TT, 64>), grid, dim3(merge_threads(64)), 0, s, p); break;
    case 96: hipLaunchKernelGGL((prefill_merge_kernel<TT, 96>), grid, dim3(merge_threads(96)), 0, s, p); break;
    case 128: hipLaunchKernelGGL((prefill_merge_kernel<TT, 128>), grid, dim3(merge_threads(128)), 0, s, p); break;
    case 256: hipLaunchKernelGGL((prefill_merge_kernel<TT, 256>), grid, dim3(merge_threads(256)), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

// Planned prefill: plan (one workgroup), the prefill kernel over 2 * plan_items unit slots
// (workgroups past the planned count exit at once), then the merge of the split items.
hipError_t launch_prefill_planned(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                                  hipStream_t s) {
  // byte-coded pages (integer, fp8): over operand images of their rows only
  const bool coded = prefill_coded_supported(p.head_dim, act, cache_dtype);
  const int pk = !coded ? kPkT : cache_dtype == PA_DTYPE_FP8_E4M3 ? kPkF8 : kPkInt;
  if (coded ? (p.vimg == nullptr || !p.k_scale || !p.v_scale)
           : (!prefill_mfma_supported(p.head_dim, act, cache_dtype) ||
              !prefill_planned_supported(p.head_dim)))
    return hipErrorInvalidValue;
  if (p.plan_items <= 0 || p.plan_rbs <= 0 || !p.plan || !p.plan_info ||
      !p.plan_split || !p.part_o || !p.part_ml || p.max_splits != 1)
    return hipErrorInvalidValue;
  if ((int64_t)p.plan_items * (kPrefillRows / kPrefillMergeRows) > INT32_MAX) return hipErrorInvalidValue;
  // Operand images: written by workgroups 1.. of the plan launch.
  constexpr int kPlanThreads = 1024;
  const bool img = p.vimg != nullptr;
  if (img && (!img_head(p.head_dim) || !p.vstep || p.img_steps <= 0))
    return hipErrorInvalidValue;
  const int64_t nimg = img ? (int64_t)p.batch * p.kv_heads *
                                 ((p.img_steps + kPlanThreads / 256 - 1) / (kPlanThreads / 256))
                           : 0;
  if (nimg + 1 > INT32_MAX) return hipErrorInvalidValue;
  const dim3 pg((unsigned)(1 + nimg));
  auto plan = [&](auto tt, auto dd, auto kc) {
    using T_ = decltype(tt);
    constexpr int D_ = decltype(dd)::value, KC_ = decltype(kc)::value;
    hipLaunchKernelGGL((prefill_plan_kernel<kPlanThreads, T_, D_, KC_>), pg, dim3(kPlanThreads), 0,
                       s, p);
  };
  using I0 = std::integral_constant<int, 0>;
  if (!img) {
    plan(TBF16{}, I0{}, I0{});
  } else {
    auto by_kind = [&](auto tt, auto dd) {
      if (cache_dtype == PA_DTYPE_INT8)
        plan(tt, dd, std::integral_constant<int, kImgI8>{});
      else if (cache_dtype == PA_DTYPE_INT4)
        plan(tt, dd, std::integral_constant<int, kImgI4>{});
      else if (cache_dtype == PA_DTYPE_FP8_E4M3)
        plan(tt, dd, std::integral_constant<int, kImgF8>{});
      else
        plan(tt, dd, std::integral_constant<int, kImgT>{});
    };
    auto by_head = [&](auto tt) {
      switch (p.head_dim) {
        case 64: by_kind(tt, std::integral_constant<int, 64>{}); break;
        case 96: by_kind(tt, std::integral_constant<int, 96>{}); break;
        case 128: by_kind(tt, std::integral_constant<int, 128>{}); break;
        default: by_kind(tt, std::integral_constant<int, 256>{}); break;
      }
    };
    if (act == PA_DTYPE_FLOAT16)
      by_head(TF16{});
    else
      by_head(TBF16{});
  }
  const dim3 grid(2 * p.plan_items, 1);
  hipError_t e = act == PA_DTYPE_FLOAT16 ? launch_t<TF16>(p, grid, s, pk)
                                         : launch_t<TBF16>(p, grid, s, pk);
  if (e != hipSuccess) return e;
  return act == PA_DTYPE_FLOAT16 ? launch_prefill_merge<TF16>(p, s)
                                 : launch_prefill_merge<TBF16>(p, s);
}

// Byte-coded pages (int8 / int4 codes with fp32 scales, fp8 e4m3 with per-(block, kv-head)
// scales) on the planned prefill over operand images.
bool prefill_coded_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (cache_dtype != PA_DTYPE_INT8 && cache_dtype != PA_DTYPE_INT4 &&
      cache_dtype != PA_DTYPE_FP8_E4M3)
    return false;
  return img_head(head_dim);
}

bool prefill_mfma_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype) {
  if (act != PA_DTYPE_FLOAT16 && act != PA_DTYPE_BFLOAT16) return false;
  if (cache_dtype != act) return false;
  return head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256;
}

// The planned launch merges split items with D/8 lanes per row (merge_threads).
bool prefill_planned_supported(int head_dim) {
  return head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 256;
}

// Grid: one workgroup per (row block, sequence, kv-head) and context chunk (p.max_splits
// chunks of p.chunk keys).
hipError_t launch_prefill_mfma(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                               hipStream_t s) {
  if (!prefill_mfma_supported(p.head_dim, act, cache_dtype)) return hipErrorInvalidValue;
  if (p.batch <= 0) return hipSuccess;
  if (p.chunk < 32 || p.chunk % 32 != 0 || p.max_splits < 1) return hipErrorInvalidValue;
  const int g = p.num_heads / p.kv_heads;
  const int mq = p.max_query_len > 0 ? p.max_query_len : p.num_tokens;
  const int64_t rbs = ((int64_t)g * mq + kPrefillRows - 1) / kPrefillRows;
  const int64_t units = (int64_t)p.batch * p.kv_heads;
  if (rbs * units > INT32_MAX || p.max_splits > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(rbs * units), p.max_splits);
  if (act == PA_DTYPE_FLOAT16) return launch_t<TF16>(p, grid, s);
  return launch_t<TBF16>(p, grid, s);
}

}  // namespace pa
