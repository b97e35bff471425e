/*
 * pa_oracle.c — CPU restatement of the reference's paged GQA KV-cache attention path.
 *
 * TEST INFRASTRUCTURE ONLY (see pa_oracle.h).  Compiled with -ffp-contract=off so that every
 * float operation rounds on its own, which the per-op rounding rules below depend on.
 */
#include "pa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---------------------------------------------------------------- converters (IEEE / OCP) */

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                                   /* normal half: >= 2^-14 */
    uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
  }
  if (a <= 0x33000000u) return sign; /* <= 2^-25: rounds (ties-to-even) to zero */
  uint32_t e = a >> 23;
  uint32_t m = (a & 0x7fffffu) | 0x800000u;
  uint32_t shift = 126u - e; /* value in units of 2^-24 is m >> shift */
  uint32_t q = m >> shift;
  uint32_t rem = m & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

float orc_e4m3_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7) return NAN;
  float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

uint8_t orc_f32_to_e4m3(float f) {
  if (isnan(f)) return 0x7f;
  uint8_t s = signbit(f) ? 0x80 : 0x00;
  float a = fabsf(f);
  if (a >= 448.0f) return s | 0x7e;
  if (a == 0.0f) return s;
  int e2;
  frexpf(a, &e2);
  int E = e2 - 1; /* floor(log2 a) */
  if (E < -6) E = -6;
  /* quantum 2^(E-3); dividing by a power of two is exact, rintf rounds ties to even */
  float q = rintf(ldexpf(a, 3 - E));
  if (q >= 16.0f) { /* rounded up into the next binade */
    E += 1;
    q = 8.0f;
  }
  if (q < 8.0f) return s | (uint8_t)q; /* subnormal (only possible when E == -6) */
  return s | (uint8_t)(((E + 7) << 3) | ((int)q - 8));
}

/* --------------------------------------------------------- integer caches (a11) */
/* QuantizedCache::encode (kv_cache.rs:170-199): divisor = scale, or 1 where scale == 0; the
 * paged rule divides and then writes 0 where scale == 0 (:186-188), the GQA rule multiplies by
 * fp32(1 / divisor) (:189-191); then mlx_clip to the code range and mlx_round (half to even). */
int orc_int_code(float x, float scale, int bits, int reciprocal) {
  float divisor = scale == 0.0f ? 1.0f : scale;
  float y;
  if (reciprocal) {
    float r = 1.0f / divisor;
    y = x * r;
  } else {
    y = scale == 0.0f ? 0.0f : x / divisor;
  }
  if (isnan(y)) return 0;
  float lo = bits == 4 ? -8.0f : -128.0f, hi = bits == 4 ? 7.0f : 127.0f;
  if (y < lo) y = lo;
  if (y > hi) y = hi;
  return (int)rintf(y); /* default rounding mode: to nearest, ties to even */
}

/* int4 packing (kv_cache.rs:196-219): biased = code + 8, an odd row padded with 8, byte =
 * low + 16 * high over (even, odd) channel pairs. */
void orc_int_encode_row(const float* x, int head_dim, const float* scale, int per_channel,
                        int bits, int reciprocal, uint8_t* dst) {
  if (bits == 8) {
    for (int e = 0; e < head_dim; ++e)
      dst[e] = (uint8_t)(int8_t)orc_int_code(x[e], scale[per_channel ? e : 0], 8, reciprocal);
    return;
  }
  for (int j = 0; j < (head_dim + 1) / 2; ++j) {
    int e0 = 2 * j, e1 = 2 * j + 1;
    int lo = orc_int_code(x[e0], scale[per_channel ? e0 : 0], 4, reciprocal) + 8;
    int hi = e1 < head_dim ? orc_int_code(x[e1], scale[per_channel ? e1 : 0], 4, reciprocal) + 8
                           : 8;
    dst[j] = (uint8_t)(lo + 16 * hi);
  }
}

/* QuantizedCache::decode (kv_cache.rs:222-256): int4 splits (byte & 15, byte >> 4), slices to
 * head_dim and subtracts 8; both widths multiply by the scale in fp32. */
void orc_int_decode_row(const uint8_t* src, int head_dim, const float* scale, int per_channel,
                        int bits, float* out) {
  for (int e = 0; e < head_dim; ++e) {
    float code = bits == 8 ? (float)(int8_t)src[e]
                           : (float)((e & 1 ? src[e / 2] >> 4 : src[e / 2] & 15) - 8);
    out[e] = code * scale[per_channel ? e : 0];
  }
}

static inline int is_int_dt(int dt) { return dt == ORC_I8 || dt == ORC_I4; }
/* storage units (elements, or int4 bytes) of one kv-head row */
static inline int cache_width(int dt, int head_dim) {
  return dt == ORC_I4 ? (head_dim + 1) / 2 : head_dim;
}

static inline float ld(const void* p, int64_t i, int dt) {
  switch (dt) {
    case ORC_F16: return orc_f16_to_f32(((const uint16_t*)p)[i]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)p)[i]);
    case ORC_E4M3: return orc_e4m3_to_f32(((const uint8_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static inline void st(void* p, int64_t i, float v, int dt) {
  switch (dt) {
    case ORC_F16: ((uint16_t*)p)[i] = orc_f32_to_f16(v); break;
    case ORC_BF16: ((uint16_t*)p)[i] = orc_f32_to_bf16(v); break;
    case ORC_E4M3: ((uint8_t*)p)[i] = orc_f32_to_e4m3(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

/* round a float to dtype and back (identity for fp32) */
static inline float rd(float v, int dt) {
  switch (dt) {
    case ORC_F16: return orc_f16_to_f32(orc_f32_to_f16(v));
    case ORC_BF16: return orc_bf16_to_f32(orc_f32_to_bf16(v));
    default: return v;
  }
}

static inline int esize(int dt) { return dt == ORC_F32 ? 4 : dt == ORC_E4M3 ? 1 : 2; }

void orc_encode(const float* src, void* dst, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) st(dst, i, src[i], dtype);
}

void orc_decode(const void* src, float* dst, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) dst[i] = ld(src, i, dtype);
}

/* ------------------------------------------------------------------ RMSNorm (a4, optional) */
/* attention.rs:4045-4049 calls mlx_fast_rms_norm(x, w, eps): fp32 sum of squares, then the
 * normalised value is rounded to T and multiplied by the weight in T.  The sum of squares has
 * one fixed rounding order, the device's: 64 partial sums p[l] fold elements l, l + 64, ...
 * with fused multiply-adds in that order, then an XOR butterfly over distances 32, 16, ..., 1
 * replaces p[l] by p[l] + p[l ^ o] (a sum MLX leaves unspecified; any fp32 order is within its
 * contract, this one makes the normalised rows bit-exact). */
static float orc_sum_squares_f(const float* v, int head_dim) {
  float p[64], q[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int e = l; e < head_dim; e += 64) acc = fmaf(v[e], v[e], acc);
    p[l] = acc;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ o];
    memcpy(p, q, sizeof p);
  }
  return p[0];
}

float orc_sum_squares(const void* x, int64_t base, int head_dim, int dtype) {
  float* v = (float*)malloc((size_t)(head_dim > 0 ? head_dim : 1) * sizeof(float));
  if (!v) return NAN;
  for (int e = 0; e < head_dim; ++e) v[e] = ld(x, base + e, dtype);
  float r = orc_sum_squares_f(v, head_dim);
  free(v);
  return r;
}

void orc_rms_norm_rows(void* x, int64_t rows, int heads, int head_dim, const void* weight,
                       float eps, int dtype) {
  for (int64_t r = 0; r < rows * heads; ++r) {
    int64_t base = r * head_dim;
    float acc = orc_sum_squares(x, base, head_dim, dtype);
    float inv = 1.0f / sqrtf(acc / (float)head_dim + eps);
    for (int i = 0; i < head_dim; ++i) {
      float v = rd(ld(x, base + i, dtype) * inv, dtype);
      st(x, base + i, v * ld(weight, i, dtype), dtype);
    }
  }
}

/* ------------------------------------------------------------------------- RoPE (a5) */
/* gqa_rope (attention.rs:459-503): non-interleaved o1 = x1*c - x2*s, o2 = x2*c + x1*s on the
 * rotary slice [offset, offset + 2*half); interleaved on (even, odd) pairs; every multiply,
 * subtract and add is a separate MLX op in the activation dtype, so each rounds to T.  The
 * cos/sin rows are the supplied cache rows at absolute positions (cos_sin_row :523-535). */
int orc_rope_rows(void* x, int64_t rows, int heads, int head_dim, const int32_t* positions,
                  const void* cos_cache, const void* sin_cache, int64_t cos_rows, int half,
                  int offset, int interleaved, int dtype) {
  if (offset < 0 || offset + 2 * half > head_dim) return 1;
  for (int64_t r = 0; r < rows; ++r) {
    int64_t pos = positions[r];
    if (pos < 0 || pos >= cos_rows) return 2;
    for (int h = 0; h < heads; ++h) {
      int64_t base = (r * heads + h) * (int64_t)head_dim + offset;
      for (int i = 0; i < half; ++i) {
        float c = ld(cos_cache, pos * half + i, dtype);
        float s = ld(sin_cache, pos * half + i, dtype);
        int64_t i1 = interleaved ? base + 2 * i : base + i;
        int64_t i2 = interleaved ? base + 2 * i + 1 : base + half + i;
        float a = ld(x, i1, dtype), b = ld(x, i2, dtype);
        float o1 = rd(rd(a * c, dtype) - rd(b * s, dtype), dtype);
        float o2 = rd(rd(b * c, dtype) + rd(a * s, dtype), dtype);
        st(x, i1, o1, dtype);
        st(x, i2, o2, dtype);
      }
    }
  }
  return 0;
}

/* ---------------------------------------------------------------- append / scatter (a6) */

static int token_slot(const int32_t* cum, const int32_t* past, const int32_t* bt, int b,
                      int max_blocks, const int32_t* slot_mapping, int j, int block_size,
                      int64_t* slot) {
  int64_t t = cum[b] + j;
  if (slot_mapping) {
    *slot = slot_mapping[t];
    return 0;
  }
  int64_t logical = (int64_t)past[b] + j;
  *slot = (int64_t)bt[(int64_t)b * max_blocks + logical / block_size] * block_size +
          logical % block_size;
  return 0;
}

/* Paged quantised encode, restating kv_cache.rs:170-192 (x / scale, zero scale -> 0) with the
 * fp8 e4m3 saturating RNE cast in place of the int8 clip/round. */
static uint8_t quant_e4m3(float x, float scale) {
  if (scale == 0.0f) return 0;
  return orc_f32_to_e4m3(x / scale);
}

int orc_reshape_and_cache(const void* key, const void* value, int act_dtype, void* key_cache,
                          void* value_cache, int cache_dtype, const float* k_scale,
                          const float* v_scale, int k_mode, int v_mode, const int32_t* cum,
                          const int32_t* past, const int32_t* block_table, int batch,
                          int max_blocks, const int32_t* slot_mapping, int64_t num_blocks,
                          int block_size, int kv_heads, int head_dim) {
  int64_t row = (int64_t)kv_heads * head_dim;
  int width = cache_width(cache_dtype, head_dim);
  float* tmp = NULL;
  if (is_int_dt(cache_dtype)) {
    tmp = (float*)malloc((size_t)head_dim * sizeof(float));
    if (!tmp) return 4;
  }
  for (int b = 0; b < batch; ++b) {
    int nq = cum[b + 1] - cum[b];
    for (int j = 0; j < nq; ++j) {
      int64_t slot;
      token_slot(cum, past, block_table, b, max_blocks, slot_mapping, j, block_size, &slot);
      if (slot < 0) continue;
      if (slot >= num_blocks * block_size) {
        free(tmp);
        return 3;
      }
      int64_t t = cum[b] + j;
      if (is_int_dt(cache_dtype)) {
        int bits = cache_dtype == ORC_I8 ? 8 : 4;
        for (int kh = 0; kh < kv_heads; ++kh)
          for (int side = 0; side < (value_cache ? 2 : 1); ++side) {
            const void* src = side ? value : key;
            const float* sc = side ? v_scale : k_scale;
            int pc = (side ? v_mode : k_mode) == ORC_QUANT_PER_CHANNEL;
            uint8_t* dst = (uint8_t*)(side ? value_cache : key_cache) +
                           (slot * kv_heads + kh) * (int64_t)width;
            for (int i = 0; i < head_dim; ++i)
              tmp[i] = ld(src, t * row + (int64_t)kh * head_dim + i, act_dtype);
            orc_int_encode_row(tmp, head_dim, pc ? sc + (int64_t)kh * head_dim : sc, pc, bits, 0,
                               dst);
          }
      } else if (cache_dtype == ORC_E4M3) {
        int64_t blk = slot / block_size;
        for (int kh = 0; kh < kv_heads; ++kh) {
          float ks = k_scale[blk * kv_heads + kh];
          float vs = value_cache ? v_scale[blk * kv_heads + kh] : 0.0f;
          for (int i = 0; i < head_dim; ++i) {
            int64_t src = t * row + (int64_t)kh * head_dim + i;
            int64_t dst = slot * row + (int64_t)kh * head_dim + i;
            ((uint8_t*)key_cache)[dst] = quant_e4m3(ld(key, src, act_dtype), ks);
            if (value_cache)
              ((uint8_t*)value_cache)[dst] = quant_e4m3(ld(value, src, act_dtype), vs);
          }
        }
      } else {
        int es = esize(cache_dtype);
        memcpy((char*)key_cache + slot * row * es, (const char*)key + t * row * es,
               (size_t)(row * es));
        if (value_cache) /* LATENT: no value cache */
          memcpy((char*)value_cache + slot * row * es, (const char*)value + t * row * es,
                 (size_t)(row * es));
      }
    }
  }
  free(tmp);
  return 0;
}

/* ----------------------------------------------------------------------- attention (a8) */

/* Element e of the kv-head row at storage index `base` (block blk, kv-head kh), as the
 * attention reads it: T, fp8 code * block scale, or integer code * scale (fp32). */
static double cache_elem(const void* cache, int cache_dtype, const float* scales, int mode,
                         int64_t blk, int kv_heads, int kh, int head_dim, int64_t base, int e) {
  if (cache_dtype == ORC_E4M3) {
    float v = orc_e4m3_to_f32(((const uint8_t*)cache)[base + e]) * scales[blk * kv_heads + kh];
    return (double)v;
  }
  if (is_int_dt(cache_dtype)) {
    const uint8_t* row = (const uint8_t*)cache + base;
    float code = cache_dtype == ORC_I8 ? (float)(int8_t)row[e]
                                       : (float)((e & 1 ? row[e / 2] >> 4 : row[e / 2] & 15) - 8);
    float s = scales[mode == ORC_QUANT_PER_CHANNEL ? (int64_t)kh * head_dim + e : 0];
    return (double)(code * s);
  }
  return (double)ld(cache, base + e, cache_dtype);
}

int orc_paged_attention(const void* q, const void* k_new, const void* v_new, int act_dtype,
                        const void* key_cache, const void* value_cache, int cache_dtype,
                        const float* k_scale, const float* v_scale, int k_mode, int v_mode,
                        const int32_t* cum, const int32_t* past, const int32_t* block_table,
                        int batch, int max_blocks, int64_t num_blocks, int block_size,
                        int num_heads, int kv_heads, int head_dim, float scale, float softcap,
                        int window, int causal, const float* head_sink, double* out,
                        int v_head_dim) {
  (void)num_blocks;
  int g = num_heads / kv_heads;
  int d = head_dim;
  /* LATENT (value_cache == NULL): values are the first vd dims of the key rows
   * (attention.rs:4058-4062 for new rows, :4210-4213 for cached rows). */
  int latent = value_cache == NULL;
  int vd = v_head_dim > 0 ? v_head_dim : d;
  if (latent) {
    value_cache = key_cache;
    v_new = k_new;
  }
  int64_t row = (int64_t)kv_heads * d;
  int width = cache_width(cache_dtype, d);
  int64_t crow = (int64_t)kv_heads * width;
  int quant = cache_dtype == ORC_E4M3 || is_int_dt(cache_dtype);
  int failed = 0;
  for (int b = 0; b < batch; ++b) {
    int s0 = cum[b], nq = cum[b + 1] - cum[b];
    if (nq <= 0) continue;
    int64_t pastb = past[b], total = pastb + nq;
    /* Every (query row, head) pair is computed on its own, in the same sequential order
     * whichever thread takes it, so the results do not depend on the thread count. */
#pragma omp parallel reduction(| : failed)
    {
      double* scores = (double*)malloc((size_t)total * sizeof(double));
      double* qrow = (double*)malloc((size_t)d * sizeof(double));
      if (!scores || !qrow) failed = 1;
#pragma omp for collapse(2) schedule(dynamic, 1)
    for (int i = 0; i < nq; ++i) {
      for (int h = 0; h < num_heads; ++h) {
        if (!scores || !qrow) continue;
        int64_t t = s0 + i, rp = pastb + i;
        int kh = h / g;
        const int64_t qbase = (t * num_heads + h) * (int64_t)d;
        for (int e = 0; e < d; ++e) qrow[e] = (double)ld(q, qbase + e, act_dtype);
        double m = -INFINITY;
        for (int64_t p = 0; p < total; ++p) {
          int visible = (!causal || p <= rp) && (window <= 0 || p >= rp - window + 1);
          if (!visible) {
            scores[p] = -INFINITY;
            continue;
          }
          double dot = 0.0;
          if (p < pastb || quant) {
            int64_t blk = block_table[(int64_t)b * max_blocks + p / block_size];
            int64_t base = (blk * block_size + p % block_size) * crow + (int64_t)kh * width;
            for (int e = 0; e < d; ++e)
              dot += qrow[e] * cache_elem(key_cache, cache_dtype, k_scale, k_mode, blk,
                                          kv_heads, kh, d, base, e);
          } else {
            int64_t base = (s0 + (p - pastb)) * row + (int64_t)kh * d;
            for (int e = 0; e < d; ++e) dot += qrow[e] * (double)ld(k_new, base + e, act_dtype);
          }
          double s = (double)scale * dot;
          if (softcap > 0.0f) s = (double)softcap * tanh(s / (double)softcap);
          scores[p] = s;
          if (s > m) m = s;
        }
        double sink = head_sink ? (double)head_sink[h] : -INFINITY;
        double mm = m > sink ? m : sink;
        double l = 0.0;
        double* o = out + (t * num_heads + h) * (int64_t)vd;
        for (int e = 0; e < vd; ++e) o[e] = 0.0;
        if (mm == -INFINITY) continue; /* nothing visible: the sum==0 guard leaves zeros */
        for (int64_t p = 0; p < total; ++p) {
          if (scores[p] == -INFINITY) continue;
          double w = exp(scores[p] - mm);
          l += w;
          if (p < pastb || quant) {
            int64_t blk = block_table[(int64_t)b * max_blocks + p / block_size];
            int64_t base = (blk * block_size + p % block_size) * crow + (int64_t)kh * width;
            for (int e = 0; e < vd; ++e)
              o[e] += w * cache_elem(value_cache, cache_dtype, v_scale, v_mode, blk, kv_heads, kh,
                                     d, base, e);
          } else {
            int64_t base = (s0 + (p - pastb)) * row + (int64_t)kh * d;
            for (int e = 0; e < vd; ++e) o[e] += w * (double)ld(v_new, base + e, act_dtype);
          }
        }
        if (head_sink) l += exp(sink - mm);
        if (l != 0.0)
          for (int e = 0; e < vd; ++e) o[e] /= l;
      }
    }
      free(scores);
      free(qrow);
    }
  }
  return failed ? 4 : 0;
}

int orc_paged_attention_op(int act_dtype, int cache_dtype, const void* query, const void* key,
                           const void* value, int64_t num_tokens, void* key_cache,
                           void* value_cache, const float* k_scale, const float* v_scale,
                           int k_mode, int v_mode, int64_t num_blocks, int block_size, const int32_t* cum,
                           const int32_t* past, const int32_t* block_table, int batch,
                           int max_blocks, const void* cos_cache, const void* sin_cache,
                           int64_t cos_rows, int rot_half, int rot_offset, int interleaved,
                           const int32_t* slot_mapping, const float* head_sink,
                           const void* q_norm, const void* k_norm, float norm_eps,
                           int num_heads, int kv_heads, int head_dim, float scale,
                           float softcap, int window, int causal, double* out, void* out_t,
                           int v_head_dim) {
  int es = esize(act_dtype);
  size_t qbytes = (size_t)num_tokens * num_heads * head_dim * es;
  size_t kbytes = (size_t)num_tokens * kv_heads * head_dim * es;
  void* qr = malloc(qbytes ? qbytes : 1);
  void* kr = malloc(kbytes ? kbytes : 1);
  int32_t* pos = (int32_t*)malloc((size_t)(num_tokens ? num_tokens : 1) * sizeof(int32_t));
  int rc = 0;
  if (!qr || !kr || !pos) {
    rc = 4;
    goto done;
  }
  memcpy(qr, query, qbytes);
  memcpy(kr, key, kbytes);
  for (int b = 0; b < batch; ++b)
    for (int t = cum[b]; t < cum[b + 1]; ++t) pos[t] = past[b] + (t - cum[b]);
  if (q_norm) {
    orc_rms_norm_rows(qr, num_tokens, num_heads, head_dim, q_norm, norm_eps, act_dtype);
    orc_rms_norm_rows(kr, num_tokens, kv_heads, head_dim, k_norm, norm_eps, act_dtype);
  }
  if (cos_cache) {
    rc = orc_rope_rows(qr, num_tokens, num_heads, head_dim, pos, cos_cache, sin_cache, cos_rows,
                       rot_half, rot_offset, interleaved, act_dtype);
    if (!rc)
      rc = orc_rope_rows(kr, num_tokens, kv_heads, head_dim, pos, cos_cache, sin_cache,
                         cos_rows, rot_half, rot_offset, interleaved, act_dtype);
    if (rc) goto done;
  }
  rc = orc_reshape_and_cache(kr, value, act_dtype, key_cache, value_cache, cache_dtype, k_scale,
                             v_scale, k_mode, v_mode, cum, past, block_table, batch, max_blocks,
                             slot_mapping, num_blocks, block_size, kv_heads, head_dim);
  if (rc) goto done;
  rc = orc_paged_attention(qr, kr, value, act_dtype, key_cache, value_cache, cache_dtype, k_scale,
                           v_scale, k_mode, v_mode, cum, past, block_table, batch, max_blocks,
                           num_blocks, block_size, num_heads, kv_heads, head_dim, scale, softcap,
                           window, causal, head_sink, out, v_head_dim);
  if (!rc && out_t) {
    int64_t n = num_tokens * (int64_t)num_heads * (v_head_dim > 0 ? v_head_dim : head_dim);
    for (int64_t i = 0; i < n; ++i) st(out_t, i, (float)out[i], act_dtype);
  }
done:
  free(qr);
  free(kr);
  free(pos);
  return rc;
}

/* ------------------------------------------------------------ contiguous GQA (C1 semantic) */
/* test_gqa_position_cache.py:104-126: past_b = total_b - S with total_b = seqlens_k[b] + 1;
 * new rows land at [past_b, total_b); row i attends to [max(0, end - window), end) with
 * end = past_b + i + 1 when causal (else total_b); GQA head map kv = h / (H / KV). */
int orc_gqa_contiguous(int dtype, const void* query, const void* key, const void* value,
                       void* present_k, void* present_v, int batch, int seq, int num_heads,
                       int kv_heads, int head_dim, int cap, const int32_t* seqlens_k,
                       float scale, float softcap, int window, int causal, double* out,
                       int cache_dtype, const float* k_scale, const float* v_scale, int k_mode,
                       int v_mode) {
  int g = num_heads / kv_heads, d = head_dim;
  int quant = is_int_dt(cache_dtype);
  int width = quant ? cache_width(cache_dtype, d) : d;
  int bits = cache_dtype == ORC_I8 ? 8 : 4;
  int kpc = k_mode == ORC_QUANT_PER_CHANNEL, vpc = v_mode == ORC_QUANT_PER_CHANNEL;
  double* scores = (double*)malloc((size_t)(cap > 0 ? cap : 1) * sizeof(double));
  float* tmp = (float*)malloc((size_t)d * sizeof(float));
  float* kd = (float*)malloc((size_t)d * sizeof(float));
  if (!scores || !tmp || !kd) {
    free(scores);
    free(tmp);
    free(kd);
    return 4;
  }
  int rc = 0;
  /* row p of (b, kh) of a present cache, widened as the attention reads it */
  #define PRESENT_ROW(buf, sc, pc, p, outrow)                                                  \
    do {                                                                                      \
      int64_t r_ = ((int64_t)b * kv_heads + kh) * cap + (p);                                  \
      if (quant)                                                                              \
        orc_int_decode_row((const uint8_t*)(buf) + r_ * width, d,                             \
                           (pc) ? (sc) + (int64_t)kh * d : (sc), (pc), bits, (outrow));       \
      else                                                                                    \
        for (int e_ = 0; e_ < d; ++e_) (outrow)[e_] = ld((buf), r_ * d + e_, dtype);          \
    } while (0)
  for (int b = 0; b < batch && !rc; ++b) {
    int total = seqlens_k[b] + 1;
    int pastb = total - seq;
    if (pastb < 0 || total > cap) {
      rc = 5;
      break;
    }
    for (int j = 0; j < seq; ++j)
      for (int kh = 0; kh < kv_heads; ++kh) {
        int64_t src = (((int64_t)b * seq + j) * kv_heads + kh) * d;
        int64_t dst = ((int64_t)b * kv_heads + kh) * cap + pastb + j;
        if (quant) {
          for (int side = 0; side < 2; ++side) {
            const void* in = side ? value : key;
            const float* sc = side ? v_scale : k_scale;
            int pc = side ? vpc : kpc;
            for (int e = 0; e < d; ++e) tmp[e] = ld(in, src + e, dtype);
            orc_int_encode_row(tmp, d, pc ? sc + (int64_t)kh * d : sc, pc, bits, 1,
                               (uint8_t*)(side ? present_v : present_k) + dst * width);
          }
        } else {
          for (int e = 0; e < d; ++e) {
            st(present_k, dst * d + e, ld(key, src + e, dtype), dtype);
            st(present_v, dst * d + e, ld(value, src + e, dtype), dtype);
          }
        }
      }
    for (int i = 0; i < seq; ++i)
      for (int h = 0; h < num_heads; ++h) {
        int kh = h / g;
        int end = causal ? pastb + i + 1 : total;
        if (end > total) end = total;
        int start = window > 0 ? (end - window > 0 ? end - window : 0) : 0;
        int64_t qb = (((int64_t)b * seq + i) * num_heads + h) * d;
        double m = -INFINITY;
        for (int p = start; p < end; ++p) {
          PRESENT_ROW(present_k, k_scale, kpc, p, kd);
          double dot = 0.0;
          for (int e = 0; e < d; ++e) dot += (double)ld(query, qb + e, dtype) * (double)kd[e];
          double s = (double)scale * dot;
          if (softcap > 0.0f) s = (double)softcap * tanh(s / (double)softcap);
          scores[p] = s;
          if (s > m) m = s;
        }
        double* o = out + qb;
        for (int e = 0; e < d; ++e) o[e] = 0.0;
        double l = 0.0;
        for (int p = start; p < end; ++p) {
          double w = exp(scores[p] - m);
          l += w;
          PRESENT_ROW(present_v, v_scale, vpc, p, kd);
          for (int e = 0; e < d; ++e) o[e] += w * (double)kd[e];
        }
        if (l != 0.0)
          for (int e = 0; e < d; ++e) o[e] /= l;
      }
  }
  #undef PRESENT_ROW
  free(scores);
  free(tmp);
  free(kd);
  return rc;
}

/* ------------------------------------------------------------ GroupQueryAttention (all forms) */
/* RMSNorm of one row held as T values in floats (orc_rms_norm_rows on a single row). */
static void norm_row(float* v, int d, const void* weight, float eps, int dtype) {
  float acc = orc_sum_squares_f(v, d);
  float inv = 1.0f / sqrtf(acc / (float)d + eps);
  for (int i = 0; i < d; ++i) v[i] = rd(rd(v[i] * inv, dtype) * ld(weight, i, dtype), dtype);
}

/* gqa_rope (per-op T rounding) or gqa_rope_f32 (fp32 ops, one rounding) of one row at cos/sin
 * row pos (attention.rs:459-521). */
static void rope_row(float* v, int64_t pos, const void* cos, const void* sin, int half,
                     int interleaved, int f32, int dtype) {
  for (int i = 0; i < half; ++i) {
    float c = ld(cos, pos * half + i, dtype), s = ld(sin, pos * half + i, dtype);
    int i1 = interleaved ? 2 * i : i, i2 = interleaved ? 2 * i + 1 : half + i;
    float a = v[i1], b = v[i2];
    if (f32) {
      float ac = a * c, bs = b * s, bc = b * c, as = a * s;
      v[i1] = rd(ac - bs, dtype);
      v[i2] = rd(bc + as, dtype);
    } else {
      v[i1] = rd(rd(a * c, dtype) - rd(b * s, dtype), dtype);
      v[i2] = rd(rd(b * c, dtype) + rd(a * s, dtype), dtype);
    }
  }
}

static int gqa_one_sequence(const orc_gqa_args* a, int b, double* out) {
  const int S = a->seq, H = a->num_heads, KV = a->kv_heads, d = a->head_dim;
  const int dt = a->dtype, g = H / KV;
  const int cdt = a->cache_dtype ? a->cache_dtype : dt;
  const int quant = is_int_dt(cdt), bits = cdt == ORC_I8 ? 8 : 4;
  const int w = quant ? cache_width(cdt, d) : d;
  const size_t row_bytes = quant ? (size_t)w : (size_t)w * esize(dt);
  const int Pc = a->present_cap, C0 = a->past_k ? a->past_cap : 0;
  const int f32rope = a->position_ids != NULL || a->kv_seq == 0;
  const int kpc = a->k_mode == ORC_QUANT_PER_CHANNEL, vpc = a->v_mode == ORC_QUANT_PER_CHANNEL;
  float* row = (float*)malloc((size_t)(d > 0 ? d : 1) * sizeof(float));
  float* qrow = (float*)malloc((size_t)(d > 0 ? d : 1) * sizeof(float));
  double* sc = (double*)malloc((size_t)(Pc > 0 ? Pc : 1) * sizeof(double));
  if (!row || !qrow || !sc) {
    free(row);
    free(qrow);
    free(sc);
    return 4;
  }
  int rc = 0;
  do {
    const int length = a->seqlens_k[b] + 1;
    const int qp = length - S > 0 ? length - S : 0;
    const int past = a->kv_seq == 0 ? length : qp;
    const int new_rows = a->kv_seq == 0 ? 0 : length - past;
    if (past > C0 || length > Pc) {
      rc = 5;
      break;
    }
    /* present = [past rows | new rows | past tail | zero codes] */
    for (int kh = 0; kh < KV; ++kh)
      for (int side = 0; side < 2; ++side) {
        const uint8_t* src = (const uint8_t*)(side ? a->past_v : a->past_k);
        uint8_t* dst = (uint8_t*)(side ? a->present_v : a->present_k);
        for (int r = 0; r < Pc; ++r) {
          uint8_t* o = dst + (((size_t)b * KV + kh) * Pc + r) * row_bytes;
          if (r < C0 && !(r >= past && r < length))
            memcpy(o, src + (((size_t)b * KV + kh) * C0 + r) * row_bytes, row_bytes);
          else
            memset(o, cdt == ORC_I4 ? 0x88 : 0, row_bytes);
        }
      }
    for (int j = 0; j < S; ++j) {
      int64_t rp = qp + j;
      if (a->position_ids)
        rp = a->total == S ? a->position_ids[0] + j : a->position_ids[(int64_t)b * S + j];
      if (a->cos_cache && (rp < 0 || rp >= a->cos_rows)) {
        rc = 6;
        break;
      }
      if (j >= new_rows) continue;
      for (int kh = 0; kh < KV; ++kh) {
        const int64_t src = (((int64_t)b * a->kv_seq + j) * KV + kh) * d;
        const int64_t dst_row = ((int64_t)b * KV + kh) * Pc + past + j;
        for (int side = 0; side < 2; ++side) {
          const void* in = side ? a->value : a->key;
          for (int e = 0; e < d; ++e) row[e] = ld(in, src + e, dt);
          if (!side && a->k_norm) norm_row(row, d, a->k_norm, a->norm_eps, dt);
          if (!side && a->cos_cache)
            rope_row(row, rp, a->cos_cache, a->sin_cache, a->rot_half, a->interleaved, f32rope,
                     dt);
          void* pres = side ? a->present_v : a->present_k;
          if (quant) {
            const float* s = side ? a->v_scale : a->k_scale;
            const int pc = side ? vpc : kpc;
            orc_int_encode_row(row, d, pc ? s + (int64_t)kh * d : s, pc, bits, 1,
                               (uint8_t*)pres + dst_row * w);
          } else {
            for (int e = 0; e < d; ++e) st(pres, dst_row * d + e, row[e], dt);
          }
        }
      }
    }
    if (rc) break;
    for (int i = 0; i < S; ++i) {
      int64_t rp = qp + i;
      if (a->position_ids)
        rp = a->total == S ? a->position_ids[0] + i : a->position_ids[(int64_t)b * S + i];
      /* visible keys [lo, hi) of this row (causal_mask_topleft / causal_window_mask) */
      int hi = a->causal ? qp + i + 1 : length;
      if (hi > length) hi = length;
      int lo = 0;
      if (a->window > 0) {
        int l1 = qp + i - a->window + 1, l2 = length - a->window;
        lo = l1 < l2 ? l1 : l2;
        if (lo < 0) lo = 0;
      }
      for (int h = 0; h < H; ++h) {
        const int kh = h / g;
        const int64_t qb = (((int64_t)b * S + i) * H + h) * d;
        for (int e = 0; e < d; ++e) qrow[e] = ld(a->query, qb + e, dt);
        if (a->q_norm) norm_row(qrow, d, a->q_norm, a->norm_eps, dt);
        if (a->cos_cache)
          rope_row(qrow, rp, a->cos_cache, a->sin_cache, a->rot_half, a->interleaved, f32rope,
                   dt);
        double m = -INFINITY;
        for (int p = lo; p < hi; ++p) {
          const int64_t r = ((int64_t)b * KV + kh) * Pc + p;
          if (quant)
            orc_int_decode_row((const uint8_t*)a->present_k + r * w, d,
                               kpc ? a->k_scale + (int64_t)kh * d : a->k_scale, kpc, bits, row);
          else
            for (int e = 0; e < d; ++e) row[e] = ld(a->present_k, r * d + e, dt);
          double dot = 0.0;
          for (int e = 0; e < d; ++e) dot += (double)qrow[e] * (double)row[e];
          double s = (double)a->scale * dot;
          if (a->softcap > 0.0f) s = (double)a->softcap * tanh(s / (double)a->softcap);
          if (a->bias) {
            const int bb = a->bias_b == 1 ? 0 : b, bh = a->bias_h == 1 ? 0 : h;
            s += (double)ld(a->bias, (((int64_t)bb * a->bias_h + bh) * S + i) * a->total + p, dt);
          }
          sc[p] = s;
          if (s > m) m = s;
        }
        double sink = -INFINITY;
        if (a->head_sink) sink = (double)ld(a->head_sink, h, dt);
        else if (a->smooth) sink = 0.0;
        if (sink > m) m = sink;
        double* o = out + qb;
        for (int e = 0; e < d; ++e) o[e] = 0.0;
        double l = sink == -INFINITY ? 0.0 : exp(sink - m);
        for (int p = lo; p < hi; ++p) l += exp(sc[p] - m);
        if (a->qk_mode) {
          /* diagnostics row (b, h, i): visible logits or probabilities, zero elsewhere */
          double* qk = a->qk_out + (((int64_t)b * H + h) * S + i) * a->total;
          for (int64_t p = 0; p < a->total; ++p) qk[p] = 0.0;
          for (int p = lo; p < hi; ++p) qk[p] = a->qk_mode == 1 ? sc[p] : exp(sc[p] - m) / l;
        }
        for (int p = lo; p < hi; ++p) {
          const double wgt = exp(sc[p] - m);
          const int64_t r = ((int64_t)b * KV + kh) * Pc + p;
          if (quant)
            orc_int_decode_row((const uint8_t*)a->present_v + r * w, d,
                               vpc ? a->v_scale + (int64_t)kh * d : a->v_scale, vpc, bits, row);
          else
            for (int e = 0; e < d; ++e) row[e] = ld(a->present_v, r * d + e, dt);
          for (int e = 0; e < d; ++e) o[e] += wgt * (double)row[e];
        }
        if (l != 0.0)
          for (int e = 0; e < d; ++e) o[e] /= l;
      }
    }
  } while (0);
  free(row);
  free(qrow);
  free(sc);
  return rc;
}

/* sliding_window_cache (attention.rs:1139-1330).  The ring of capacity C holds the last
 * cache_end(L) rows of a sequence of length L at [0, cache_end(L)): cache_end(L) = L while
 * L <= C, else L - gap * ceil((L - C) / gap) with gap = C - window + 1 (:1166-1181).  A call with
 * p = length - S past rows attends its S new rows over the staged view [past rows [0, before) |
 * new rows] (before = cache_end(p)) with the causal window of causal_window_mask (:1288-1290;
 * the reference narrows the view to the kept rows when that holds the window, :1183-1192, which
 * masks the same keys), bias columns at absolute positions p - before + j (:1292-1301), and
 * writes the present [the last after = cache_end(p + S) rows of the view | zero codes]
 * (:1338-1368).  RoPE rotates at absolute positions p + i, in fp32 with position ids or a bias
 * (:1222-1228). */
static int cache_end(int64_t L, int C, int W) {
  if (L <= C) return (int)L;
  const int64_t gap = (int64_t)C - W + 1, over = L - C;
  return (int)(L - gap * ((over + gap - 1) / gap));
}

static int gqa_sliding_sequence(const orc_gqa_args* a, int b, double* out) {
  const int S = a->seq, H = a->num_heads, KV = a->kv_heads, d = a->head_dim;
  const int dt = a->dtype, g = H / KV, C = a->past_cap, W = a->window;
  const int cdt = a->cache_dtype ? a->cache_dtype : dt;
  const int quant = is_int_dt(cdt), bits = cdt == ORC_I8 ? 8 : 4;
  const int w = quant ? cache_width(cdt, d) : d;
  const size_t row_bytes = quant ? (size_t)w : (size_t)w * esize(dt);
  const int f32rope = a->position_ids != NULL || a->bias != NULL;
  const int kpc = a->k_mode == ORC_QUANT_PER_CHANNEL, vpc = a->v_mode == ORC_QUANT_PER_CHANNEL;
  if (!a->past_k || a->present_cap != C || W <= 0 || W > C || a->kv_seq != S) return 7;
  const int length = a->seqlens_k[b] + 1;
  const int p = length - S;
  if (p < 0) return 7;
  const int before = cache_end(p, C, W), after = cache_end((int64_t)p + S, C, W);
  const int seed = before - (after - S); /* view row of the present's first row */
  const int L = before + S;               /* rows of the staged view */
  uint8_t* view_k = (uint8_t*)malloc((size_t)KV * L * row_bytes);
  uint8_t* view_v = (uint8_t*)malloc((size_t)KV * L * row_bytes);
  float* row = (float*)malloc((size_t)d * sizeof(float));
  float* qrow = (float*)malloc((size_t)d * sizeof(float));
  double* sc = (double*)malloc((size_t)L * sizeof(double));
  int rc = 0;
  if (!view_k || !view_v || !row || !qrow || !sc) rc = 4;
  for (int kh = 0; kh < KV && !rc; ++kh)
    for (int side = 0; side < 2; ++side) {
      const uint8_t* src = (const uint8_t*)(side ? a->past_v : a->past_k);
      uint8_t* view = side ? view_v : view_k;
      memcpy(view + (size_t)kh * L * row_bytes, src + ((size_t)b * KV + kh) * C * row_bytes,
             (size_t)before * row_bytes);
    }
  /* the new rows, normalised, rotated and encoded as stored */
  for (int j = 0; j < S && !rc; ++j) {
    int64_t rp = (int64_t)p + j;
    if (a->position_ids)
      rp = a->total == S ? a->position_ids[0] + j : a->position_ids[(int64_t)b * S + j];
    if (a->cos_cache && (rp < 0 || rp >= a->cos_rows)) {
      rc = 6;
      break;
    }
    for (int kh = 0; kh < KV; ++kh) {
      const int64_t src = (((int64_t)b * S + j) * KV + kh) * d;
      for (int side = 0; side < 2; ++side) {
        const void* in = side ? a->value : a->key;
        for (int e = 0; e < d; ++e) row[e] = ld(in, src + e, dt);
        if (!side && a->k_norm) norm_row(row, d, a->k_norm, a->norm_eps, dt);
        if (!side && a->cos_cache)
          rope_row(row, rp, a->cos_cache, a->sin_cache, a->rot_half, a->interleaved, f32rope, dt);
        uint8_t* dst = (side ? view_v : view_k) + ((size_t)kh * L + before + j) * row_bytes;
        if (quant) {
          const float* s = side ? a->v_scale : a->k_scale;
          const int pc = side ? vpc : kpc;
          orc_int_encode_row(row, d, pc ? s + (int64_t)kh * d : s, pc, bits, 1, dst);
        } else {
          for (int e = 0; e < d; ++e) st(dst, e, row[e], dt);
        }
      }
    }
  }
  /* attention of the S query rows over the view */
  for (int i = 0; i < S && !rc; ++i) {
    int64_t rp = (int64_t)p + i;
    if (a->position_ids)
      rp = a->total == S ? a->position_ids[0] + i : a->position_ids[(int64_t)b * S + i];
    const int qpos = before + i;
    const int lo = qpos - W + 1 > 0 ? qpos - W + 1 : 0, hi = qpos + 1;
    for (int h = 0; h < H; ++h) {
      const int kh = h / g;
      const int64_t qb = (((int64_t)b * S + i) * H + h) * d;
      for (int e = 0; e < d; ++e) qrow[e] = ld(a->query, qb + e, dt);
      if (a->q_norm) norm_row(qrow, d, a->q_norm, a->norm_eps, dt);
      if (a->cos_cache)
        rope_row(qrow, rp, a->cos_cache, a->sin_cache, a->rot_half, a->interleaved, f32rope, dt);
      double m = -INFINITY;
      for (int j = lo; j < hi; ++j) {
        const uint8_t* kr = view_k + ((size_t)kh * L + j) * row_bytes;
        if (quant)
          orc_int_decode_row(kr, d, kpc ? a->k_scale + (int64_t)kh * d : a->k_scale, kpc, bits, row);
        else
          for (int e = 0; e < d; ++e) row[e] = ld(kr, e, dt);
        double dot = 0.0;
        for (int e = 0; e < d; ++e) dot += (double)qrow[e] * (double)row[e];
        double s = (double)a->scale * dot;
        if (a->softcap > 0.0f) s = (double)a->softcap * tanh(s / (double)a->softcap);
        if (a->bias) {
          const int bb = a->bias_b == 1 ? 0 : b, bh = a->bias_h == 1 ? 0 : h;
          const int64_t col = (int64_t)p - before + j; /* absolute key position */
          s += (double)ld(a->bias, (((int64_t)bb * a->bias_h + bh) * S + i) * a->total + col, dt);
        }
        sc[j] = s;
        if (s > m) m = s;
      }
      double sink = -INFINITY;
      if (a->head_sink) sink = (double)ld(a->head_sink, h, dt);
      else if (a->smooth) sink = 0.0;
      if (sink > m) m = sink;
      double* o = out + qb;
      for (int e = 0; e < d; ++e) o[e] = 0.0;
      double l = sink == -INFINITY ? 0.0 : exp(sink - m);
      for (int j = lo; j < hi; ++j) {
        const double wgt = exp(sc[j] - m);
        l += wgt;
        const uint8_t* vr = view_v + ((size_t)kh * L + j) * row_bytes;
        if (quant)
          orc_int_decode_row(vr, d, vpc ? a->v_scale + (int64_t)kh * d : a->v_scale, vpc, bits, row);
        else
          for (int e = 0; e < d; ++e) row[e] = ld(vr, e, dt);
        for (int e = 0; e < d; ++e) o[e] += wgt * (double)row[e];
      }
      if (l != 0.0)
        for (int e = 0; e < d; ++e) o[e] /= l;
    }
  }
  /* present: the last `after` rows of the view, then zero codes */
  for (int kh = 0; kh < KV && !rc; ++kh)
    for (int side = 0; side < 2; ++side) {
      const uint8_t* view = side ? view_v : view_k;
      uint8_t* dst = (uint8_t*)(side ? a->present_v : a->present_k) +
                     ((size_t)b * KV + kh) * C * row_bytes;
      memcpy(dst, view + ((size_t)kh * L + seed) * row_bytes, (size_t)after * row_bytes);
      memset(dst + (size_t)after * row_bytes, cdt == ORC_I4 ? 0x88 : 0,
             (size_t)(C - after) * row_bytes);
    }
  free(view_k);
  free(view_v);
  free(row);
  free(qrow);
  free(sc);
  return rc;
}

int orc_gqa_batched(const orc_gqa_args* a, double* out) {
  int rc = 0;
  /* sequences are independent (each writes its own present rows and output rows) */
  #pragma omp parallel for schedule(dynamic, 1) reduction(max : rc)
  for (int b = 0; b < a->batch; ++b) {
    int r = a->sliding ? gqa_sliding_sequence(a, b, out) : gqa_one_sequence(a, b, out);
    if (r > rc) rc = r;
  }
  return rc;
}
