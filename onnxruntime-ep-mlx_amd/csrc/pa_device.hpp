// pa_device.hpp — device-side helpers shared by the gfx950 kernels: dtype traits, exact
// conversions, MFMA wrappers and the kernel parameter blocks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_mi355x.h"

namespace pa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ------------------------------------------------------------------------------ conversions
// Integer round-to-nearest-even conversions: the rotary/append path must produce the exact bits
// of the CPU restatement, so these do not depend on instruction selection.
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// IEEE binary16 conversion of the hardware (v_cvt_f16_f32) is round-to-nearest-even.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// OCP e4m3fn (bias 7, no infinities, 0x7f/0xff NaN, max 448).
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 15u, m = c & 7u;
  float v;
  if (e == 0)
    v = (float)m * 0.001953125f;  // m * 2^-9
  else
    v = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  if (e == 15 && m == 7) v = __builtin_nanf("");
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | s);
}
// Saturating round-to-nearest-even encode; same arithmetic as the CPU restatement.
__device__ __forceinline__ uint32_t f32_to_e4m3_sat(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t s = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7fu;
  float af = __builtin_bit_cast(float, a);
  if (af >= 448.0f) return s | 0x7eu;
  if (a == 0) return s;
  int E = (int)(a >> 23) - 127;  // floor(log2) for normals; subnormal fp32 clamps below
  if (E < -6) E = -6;
  float q = __builtin_rintf(__builtin_ldexpf(af, 3 - E));
  if (q >= 16.0f) {
    E += 1;
    q = 8.0f;
  }
  uint32_t qi = (uint32_t)q;
  if (qi < 8u) return s | qi;
  return s | ((uint32_t)(E + 7) << 3) | (qi - 8u);
}

// ------------------------------------------------------------------------------ dtype traits
struct TF16 {
  using raw = uint16_t;
  using vec8 = f16x8;
  static constexpr int code = PA_DTYPE_FLOAT16;
  __device__ static float to_f32(raw h) { return f16_to_f32(h); }
  __device__ static raw from_f32(float f) { return f32_to_f16_rne(f); }
  __device__ static f32x4 mfma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static vec8 cvt8(const float* x) {
    vec8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)x[i];
    return r;
  }
  __device__ static float back(_Float16 v) { return (float)v; }
  // x = hi + lo with hi and lo fp16 (probabilities split for the P.V product).  hi rounds toward
  // zero (one packed conversion per pair), so x - hi is exact in fp32; lo rounds the same way,
  // leaving an error below 2^-20 of x.
  __device__ static void split8(const float (&x)[8], vec8& hi, vec8& lo) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const auto h = __builtin_amdgcn_cvt_pkrtz(x[2 * m], x[2 * m + 1]);
      const auto l = __builtin_amdgcn_cvt_pkrtz(x[2 * m] - (float)h[0], x[2 * m + 1] - (float)h[1]);
      hi[2 * m] = h[0];
      hi[2 * m + 1] = h[1];
      lo[2 * m] = l[0];
      lo[2 * m + 1] = l[1];
    }
  }
};

struct TBF16 {
  using raw = uint16_t;
  using vec8 = bf16x8;
  static constexpr int code = PA_DTYPE_BFLOAT16;
  __device__ static float to_f32(raw h) { return bf16_to_f32(h); }
  __device__ static raw from_f32(float f) { return f32_to_bf16_rne(f); }
  __device__ static f32x4 mfma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static vec8 cvt8(const float* x) {
    vec8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)x[i];
    return r;
  }
  __device__ static float back(__bf16 v) { return (float)v; }
  // x = hi + lo with hi and lo bf16 (probabilities split for the P.V product): hi is x rounded
  // to nearest even (one packed conversion per pair), read back exactly from its bit pattern,
  // and lo = round(x - hi).  Writing the read-back as bit operations keeps the compiler from
  // re-deriving each hi element with a conversion of its own.
  __device__ static void split8(const float (&x)[8], vec8& hi, vec8& lo) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x2 h = __builtin_convertvector(f32x2{x[2 * m], x[2 * m + 1]}, bf16x2);
      const uint32_t w = __builtin_bit_cast(uint32_t, h);
      const float h0 = __builtin_bit_cast(float, w << 16), h1 = __builtin_bit_cast(float, w & 0xffff0000u);
      const bf16x2 l = __builtin_convertvector(f32x2{x[2 * m] - h0, x[2 * m + 1] - h1}, bf16x2);
      hi[2 * m] = h[0];
      hi[2 * m + 1] = h[1];
      lo[2 * m] = l[0];
      lo[2 * m + 1] = l[1];
    }
  }
};

struct TF32 {
  using raw = float;
  static constexpr int code = PA_DTYPE_FLOAT32;
  __device__ static float to_f32(raw h) { return h; }
  __device__ static raw from_f32(float f) { return f; }
};

// ------------------------------------------------------------------------------ wave helpers
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum of squares of a D-element row with one fixed rounding order (restated by the CPU oracle,
// orc_rms_norm_rows): lane l folds elements l, l + 64, ... with fused multiply-adds in that order,
// then the 64 lane sums meet in an XOR butterfly over lane distances 32, 16, ..., 1 (both lanes of
// a pair add the same two values, so every lane ends with the same sum).
template <typename Load>
__device__ __forceinline__ float sum_squares(Load ld, int D, int lane) {
  float acc = 0.0f;
  for (int e = lane; e < D; e += 64) {
    const float v = ld(e);
    acc = __builtin_fmaf(v, v, acc);
  }
  return wave_sum(acc);
}

// Sequence index of packed token t: largest b with cum[b] <= t (cum monotone, cum[0] <= t).
// A 64-way search run by the whole wavefront (t wave-uniform): each level has every lane test
// one evenly spaced candidate, so batch <= 64 costs one memory round trip and batch <= 4096
// two, where a binary search pays log2(batch) dependent loads.
__device__ __forceinline__ int seq_of_token(const int32_t* cum, int batch, int t) {
  const int lane = threadIdx.x & 63;
  int lo = 0, n = batch;  // answer in [lo, lo + n)
  while (n > 64) {
    const int step = (n + 63) / 64;
    const int j = lo + lane * step;
    const uint64_t ok = __ballot(j < lo + n && __ldg(&cum[j]) <= t);
    const int k = ok ? 63 - __builtin_clzll(ok) : 0;  // last candidate at or below t
    const int nlo = lo + k * step;
    n = min(step, lo + n - nlo);
    lo = nlo;
  }
  const uint64_t ok = __ballot(lane < n && __ldg(&cum[lo + lane]) <= t);
  return ok ? lo + 63 - __builtin_clzll(ok) : lo;
}

// seq_of_token plus cum[b] and past[b], fetched in the same round trip as the last level.
struct SeqPos {
  int b, start, past;
};
__device__ __forceinline__ SeqPos seq_pos_of_token(const int32_t* cum, const int32_t* past,
                                                   int batch, int t) {
  const int lane = threadIdx.x & 63;
  int lo = 0, n = batch;
  while (n > 64) {
    const int step = (n + 63) / 64;
    const int j = lo + lane * step;
    const uint64_t ok = __ballot(j < lo + n && __ldg(&cum[j]) <= t);
    const int k = ok ? 63 - __builtin_clzll(ok) : 0;
    const int nlo = lo + k * step;
    n = min(step, lo + n - nlo);
    lo = nlo;
  }
  const bool in = lane < n;
  const int cj = in ? __ldg(&cum[lo + lane]) : 0;
  const int pj = in ? __ldg(&past[lo + lane]) : 0;
  const uint64_t ok = __ballot(in && cj <= t);
  const int k = ok ? 63 - __builtin_clzll(ok) : 0;
  return SeqPos{lo + k, __shfl(cj, k, 64), __shfl(pj, k, 64)};
}

// ------------------------------------------------------------------------------ parameters
struct AppendParams {
  const void* query;
  const void* key;
  const void* value;
  void* q_out;
  void* k_out;
  void* key_cache;
  void* value_cache;
  const float* k_scale;
  const float* v_scale;
  const void* cos_cache;
  const void* sin_cache;
  const void* q_norm;
  const void* k_norm;
  const int32_t* cum;
  const int32_t* past;
  const int32_t* block_table;
  const int32_t* slot_mapping;
  int64_t num_blocks;
  int64_t rotary_positions;
  int32_t block_size, kv_heads, head_dim, num_heads;
  int32_t batch, max_blocks, num_tokens;
  int32_t rotary_half, rotary_offset, rotary_interleaved;
  int32_t do_q;  // process query rows (rotary/norm) into q_out
  float norm_eps;
  int32_t slots_distinct;  // no two tokens share a slot: skip the last-writer check
  // Contiguous (GroupQueryAttention) caches: [batch, kv_heads, linear_cap, head_dim]; token t is
  // query row j = t % gqa_seq of sequence b = t / gqa_seq, length = seqlens_k[b] + 1, at position
  // query_past + j with query_past = max(length - gqa_seq, 0); its key/value row is stored there
  // when j < length - query_past (and gqa_kv_rows, i.e. the call has new key/value rows).
  // meta_out (if set) receives cum [batch + 1], past = query_past [batch] and the key count
  // length [batch] for the attention that follows.
  int32_t linear_cap;  // 0: paged cache
  int32_t gqa_seq;
  int32_t gqa_kv_rows;
  const int32_t* seqlens_k;
  int32_t* meta_out;
  // Rotary position overrides (GroupQueryAttention position_ids, int64 [batch, pos_cols]): row j
  // of sequence b rotates at pid[0] + j (pos_offset_form: a first prompt) or at pid[b * gqa_seq
  // + j] (the flattened ids).  rope_fp32: rotate in fp32 and round once (gqa_rope_f32).
  const int64_t* position_ids;
  int32_t pos_offset_form;
  int32_t rope_fp32;
  // Input row strides in elements (packed QKV rows are (H + 2 KV) * D wide).  With copy_rows
  // the query/key rows go to q_out/k_out and the value rows to v_out (contiguous [T, heads * D])
  // even when nothing rotates or normalises them.
  int64_t q_ld, k_ld, v_ld;
  void* v_out;
  int32_t copy_rows;
  // Integer caches: scale layout per side (PA_QUANT_PER_TENSOR / PA_QUANT_PER_CHANNEL) and the
  // encode rule: 0 divides by the scale (zero scale -> code 0), 1 multiplies by its reciprocal
  // (zero scale read as 1).
  int32_t k_quant, v_quant;
  int32_t quant_reciprocal;
  // GroupQueryAttention sliding_window_cache (ring_cap > 0, linear mode): a sequence of length
  // len has p = len - gqa_seq past rows, of which the ring holds before = ring_end(p); row j
  // rotates at position p + j and is stored at row before + j of the staged view (capacity
  // linear_cap = ring_cap + gqa_seq).  meta_out then also receives the ring geometry
  // (ring_meta).
  int32_t ring_cap, ring_window;
};

// Rows a sliding_window_cache ring of capacity cap and window w holds for a sequence of len rows
// (attention.rs:1166-1181): len while it fits, else len less whole multiples of gap = cap - w + 1.
__host__ __device__ __forceinline__ int ring_end(int64_t len, int cap, int w) {
  if (len <= cap) return (int)len;
  const int64_t gap = (int64_t)cap - w + 1;
  return (int)(len - gap * ((len - cap + gap - 1) / gap));
}

// Ring geometry of one sequence: p past rows (absolute), `before` held before the call, `after`
// after it, and the staged-view row of the present's first row (seed = before - (after - seq)).
struct RingGeom {
  int p, before, after, seed;
};
__host__ __device__ __forceinline__ RingGeom ring_geom(int len, int seq, int cap, int w) {
  RingGeom g;
  g.p = len - seq > 0 ? len - seq : 0;
  g.before = ring_end(g.p, cap, w);
  g.after = ring_end((int64_t)g.p + seq, cap, w);
  g.seed = g.before - (g.after - seq);
  return g;
}

// Metadata the append writes for the attention (GroupQueryAttention, meta_out): cum [B + 1],
// past [B], key count [B], then for rings the bias column offset p - before [B] (a view row's
// absolute position minus the row), seed [B] and after [B].
constexpr int kMetaCum = 0;
__host__ __device__ constexpr int meta_past(int B) { return B + 1; }
__host__ __device__ constexpr int meta_keys(int B) { return 2 * B + 1; }
__host__ __device__ constexpr int meta_colofs(int B) { return 3 * B + 1; }
__host__ __device__ constexpr int meta_ints(int B) { return 4 * B + 1; }

struct AttnParams {
  const void* q;
  const void* k_new;
  const void* v_new;
  const void* key_cache;
  const void* value_cache;
  const float* k_scale;
  const float* v_scale;
  const int32_t* cum;
  const int32_t* past;
  const int32_t* block_table;
  const void* head_sink;
  void* out;
  float* part_o;   // [num_tokens, H, max_splits, D]
  float* part_ml;  // [num_tokens, H, max_splits, 2]  (m in log2 units, l)
  int64_t num_blocks;
  int32_t block_size, kv_heads, head_dim, num_heads;
  int32_t batch, max_blocks, num_tokens;
  int32_t chunk, max_splits;
  int32_t max_query_len;  // host bound on new tokens per sequence (row-group count)
  float scale;       // softmax scale applied to q.k
  float scale_log2;  // scale * log2(e)
  float softcap;     // 0 = off
  int32_t window;    // <= 0 = off
  int32_t causal;
  int32_t read_all_from_cache;  // fp8 rule: every position from the pages
  // The append that ran before this call left every new key/value row in its cache slot
  // (block-table slots, no duplicates), so new positions may be read from the pages.
  int32_t new_rows_in_cache;
  int32_t mix;  // balanced decode: sub-segments (each for another kv-head) per wavefront
  int32_t ng;   // chunked kernel: 16-row groups per wavefront (1 or 4)
  // Contiguous caches [batch, kv_heads, linear_cap, head_dim] (GroupQueryAttention present
  // buffers; the new rows are already in them): position pos of (b, kv-head kh) is row
  // (b * kv_heads + kh) * linear_cap + pos.  0: paged cache.
  int32_t linear_cap;
  int32_t k_quant, v_quant;  // integer caches: PA_QUANT_PER_TENSOR / PA_QUANT_PER_CHANNEL
  // LATENT layout (kv_heads == 1): the value of a position is the first v_head_dim dims of its
  // key row (key cache / k_new); outputs are [T, H * v_head_dim].  v_head_dim == head_dim and
  // v_from_key == 0 otherwise.
  int32_t v_head_dim;
  int32_t v_from_key;
  // Planned prefill (plan_items > 0): item i = (sequence, row block, kv-head) with
  // i = (b * plan_rbs + rb) * kv_heads + kh.  The plan kernel writes the work units longest first
  // -- plan[4u .. 4u+3] = (item, part, first key, end key), part 0 a whole item, 1 / 2 the halves
  // of an item split in two -- the unit count at plan_info[0] and plan_split[i] = 1 for split
  // items, whose halves leave fp16 partials (rows scaled by a power of two) at rows
  // (2 i + part - 1) * kPrefillRows + row.  plan_step: the prefill kernel's key step (32 or 64);
  // item key ranges start and split at multiples of it.
  int32_t plan_items, plan_rbs, plan_slots, plan_step;
  // GroupQueryAttention forms (VALU kernel; the others take none of them): key_limit[b] bounds
  // the keys of sequence b (its length, below past + query rows for a ragged first prompt); bias
  // [bias_b, bias_h, bias_rows, bias_cols] in T is added to the scaled (softcapped) score of row i
  // of sequence b, head h, key p at ((b | 0) * bias_h + (h | 0)) * bias_rows + i) * bias_cols + p;
  // smooth_softmax: a zero sink logit when head_sink is NULL.
  const int32_t* key_limit;
  const void* bias;
  int32_t bias_b, bias_h, bias_rows, bias_cols;
  // bias column of key position pos of sequence b: pos + bias_col_off[b] (sliding_window_cache:
  // the staged view's rows are not absolute positions); NULL: pos
  const int32_t* bias_col_off;
  int32_t smooth_softmax;
  int32_t* plan;
  int32_t* plan_info;
  int32_t* plan_split;
  // Operand images of the planned prefill (vimg != NULL): for every img_keys(head_dim)-key step
  // of (sequence b, kv-head kh), the key rows gathered and the value rows converted to fp16, both
  // laid out as the prefill kernel's LDS operands, at
  // vimg + ((b * kv_heads + kh) * img_steps + step) * img_step_bytes(head_dim); vstep[same index]
  // is the step's power-of-two value exponent s (image element = value * 2^-s).
  char* vimg;
  int32_t* vstep;
  int32_t img_steps;
  // per (sequence, kv-head): set to img_epoch (a per-call number) by the image writer when a step
  // of the pair is wide (bf16 values kept raw, see the image writer); any other value: none
  int32_t* img_wide;
  int32_t img_epoch;
};

// Image geometry of the planned prefill: kImgKeys keys x d dims of 16-bit keys and values per
// step (the prefill kernel's key step over images: 32 or 64).
#ifndef PA_IMG_KEYS
#define PA_IMG_KEYS 64
#endif
constexpr int kImgKeys = PA_IMG_KEYS;
static_assert(kImgKeys == 32 || kImgKeys == 64, "image steps of one or two 32-key blocks");
// Keys per image step at head size d (head 256: 32, so a step's operands and the output rows
// fit the register budget of two wavefronts per SIMD), and the bytes of one step's image.
__host__ __device__ constexpr int img_keys(int d) { return d > 128 ? 32 : kImgKeys; }
__host__ __device__ constexpr int img_step_bytes(int d) { return 2 * img_keys(d) * d * 2; }
// Wavefronts per SIMD of the streaming decode over caches of this dtype (the grid holds that many
// segments per SIMD).  int4 codes: two -- their decode is bound by instruction issue (the code
// widening), and a second wavefront fills the first one's memory waits; its kernel fits 256
// VGPRs without spilling (the bias variant keeps one wavefront per SIMD and runs the grid in two
// rounds).  int8 at two spills ~34 VGPRs and stays at one.
#ifndef PA_DECODE_WAVES_I4
#define PA_DECODE_WAVES_I4 2
#endif
#ifndef PA_DECODE_WAVES_I8
#define PA_DECODE_WAVES_I8 1
#endif
// Pages in the activation dtype: two at head 64 (201 VGPRs; its 8 KiB steps keep few bytes in
// flight per wavefront: C3-shaped batch 113.5 -> 100.8 us per launch), one at head 96 (two: 163.5
// -> 170.0 us) and at heads 128 / 256 (bound by what the memory system delivers; above 256
// VGPRs).
// fp8 pages: one (two at ring depth 2, 229 VGPRs: C5 launch 185.6 -> 201.4 us).
#ifndef PA_DECODE_WAVES_F8
#define PA_DECODE_WAVES_F8 1
#endif
#ifndef PA_DECODE_WAVES_D96
#define PA_DECODE_WAVES_D96 1
#endif
#ifndef PA_DECODE_WAVES_D64
#define PA_DECODE_WAVES_D64 2
#endif
__host__ __device__ constexpr int decode_waves(int cache_dtype, int head_dim) {
  return cache_dtype == PA_DTYPE_INT4        ? PA_DECODE_WAVES_I4
         : cache_dtype == PA_DTYPE_INT8      ? PA_DECODE_WAVES_I8
         : cache_dtype == PA_DTYPE_FP8_E4M3  ? PA_DECODE_WAVES_F8
         : head_dim == 96                    ? PA_DECODE_WAVES_D96
         : head_dim == 64                    ? PA_DECODE_WAVES_D64
                                             : 1;
}
// Heads the planned prefill runs over operand images.
__host__ __device__ constexpr bool img_head(int d) {
  return d == 64 || d == 96 || d == 128 || d == 256;
}

// Softcapped score in log2 units for the matrix-core kernels: cap * tanh(y) * log2(e), y = v * k
// with k = scale / cap, from the identity tanh(y) = sign(y) (1 - e) / (1 + e), e = exp(-2 |y|):
// one exponential and one reciprocal (about one ulp each, ~2^-22 absolute in tanh: far below
// the resolution of bf16 / fp16 scores) instead of a division and the library tanh per score.
// |y| large: e = 0, tanh = +-1; NaN stays NaN.
__device__ __forceinline__ float softcap_log2(float v, float k, float cap_log2) {
  const float y = v * k;
  const float e = __builtin_amdgcn_exp2f(-2.0f * kLog2e * fabsf(y));
  const float t = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
  return __builtin_copysignf(t, y) * cap_log2;
}

// Final normalisation shared by every attention kernel: the factor that turns an output
// accumulated relative to running max m (log2 units) with running sum l into the result,
// folding in an optional sink logit that only enters the denominator.
__device__ __forceinline__ float finalize_factor(float m, float l, float sink_x) {
  float mm = fmaxf(m, sink_x);
  if (mm == kNegInf) return 0.0f;
  float f = (m == kNegInf) ? 0.0f : exp2f(m - mm);
  float lt = l * f + ((sink_x == kNegInf) ? 0.0f : exp2f(sink_x - mm));
  return lt > 0.0f ? f / lt : 0.0f;
}

template <typename TT>
__device__ __forceinline__ float sink_logit(const AttnParams& p, int h) {
  if (!p.head_sink) return p.smooth_softmax ? 0.0f : kNegInf;
  return TT::to_f32(reinterpret_cast<const typename TT::raw*>(p.head_sink)[h]) * kLog2e;
}

// Prefill kernel geometry: 16-row groups per wavefront, and grouped query rows per workgroup
// of 4 wavefronts.
constexpr int kPrefillGroups = 2;
constexpr int kPrefillRows = 64 * kPrefillGroups;

// Keys per step of the prefill kernel for a head size: 64 for the head-128 kernel on 32x32
// tiles, 32 for the head-64 kernel on 16x16 tiles.
inline int prefill_key_step(int head_dim) { return head_dim == 128 ? 64 : 32; }

// Launchers (defined in the .hip files).
// GroupQueryAttention sliding_window_cache ring moves (pa_append.hip): present == 0 stages the
// past ring's history rows into the view; present == 1 writes the present ring from the view.
struct RingParams {
  const int32_t* seqlens_k;
  const char* src_k;
  const char* src_v;
  char* dst_k;
  char* dst_v;
  int64_t row_bytes;  // bytes of one stored row of one kv-head
  int32_t batch, kv_heads, seq, cap, window;
  int32_t present;
  uint32_t zero;  // zero code in every byte (int4: 0x88888888)
};
hipError_t launch_ring_move(const RingParams& r, hipStream_t s);
hipError_t launch_rotary_append(const AppendParams& p, pa_dtype act, pa_dtype cache_dtype,
                                hipStream_t s);
hipError_t launch_attn_generic(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                               hipStream_t s);
hipError_t launch_decode_mfma(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                              hipStream_t s);
hipError_t launch_decode_balanced(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                                  hipStream_t s);
hipError_t launch_prefill_mfma(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                               hipStream_t s);
// Planned prefill: plan kernel, prefill kernel over the planned units, merge of split items.
hipError_t launch_prefill_planned(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype,
                                  hipStream_t s);
hipError_t launch_split_reduce(const AttnParams& p, pa_dtype act, hipStream_t s);
// LATENT layout on matrix cores (pa_latent.hip); partials merged by launch_split_reduce.
bool latent_mfma_supported(int head_dim, int v_head_dim, pa_dtype act, pa_dtype cache_dtype);
// 16-row groups per LATENT workgroup for H heads and max_query_len mq.
inline int latent_row_groups(int heads, int mq) { return (int64_t)heads * mq >= 32 ? 2 : 1; }
hipError_t launch_latent(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype, hipStream_t s);
// GroupQueryAttention output_qk diagnostics (pa_attn_generic.hip): mode 1 scores, 2 probabilities
// into qk [batch, num_heads, max_query_len, cols]; keys[b]: the sequence's key count.
hipError_t launch_gqa_qk(const AttnParams& p, pa_dtype act, pa_dtype cache_dtype, void* qk,
                         int mode, int64_t cols, const int32_t* keys, hipStream_t s);
bool decode_mfma_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype);
// Balanced (streaming) decode: fp16/bf16 activations, d in {64, 96, 128, 256}, power-of-two
// pages, pages in the activation dtype or (d 64 / 128) fp8 e4m3 with at least 16 rows per page.
bool balanced_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype, int block_size);
bool prefill_mfma_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype);
bool prefill_coded_supported(int head_dim, pa_dtype act, pa_dtype cache_dtype);
bool prefill_planned_supported(int head_dim);

}  // namespace pa
