/*
 * pa_oracle.h — CPU restatement of the reference's paged GQA KV-cache attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library, and only as the checker (or the timed CPU baseline).  The product
 * (onnxruntime-ep-mlx_amd/) never links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference
 * root).  The reference itself (Rust + MLX + Metal) cannot be built here: no rustc/cargo, no
 * ORT headers, no MLX, no Metal.
 *
 * Pins (what checks each function independently of its own formula) live in
 * tests/test_oracle.py: numpy/torch dtype casts for the converters, torch-CPU bf16/fp16
 * arithmetic evaluating the reference's rotate_half formulation for RoPE, byte invariants and
 * the reference's duplicate-slot known answer for append, torch's fp64
 * scaled_dot_product_attention plus closed forms for attention, and torch.float8_e4m3fn for
 * the fp8 encoder.
 */
#ifndef PA_ORACLE_H
#define PA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F16 = 1, ORC_BF16 = 2, ORC_F32 = 3, ORC_E4M3 = 4, ORC_I8 = 5, ORC_I4 = 6 };
/* Integer cache scale layouts (k_quant_type / v_quant_type): one scale, or [kv_heads, d]. */
enum { ORC_QUANT_NONE = 0, ORC_QUANT_PER_TENSOR = 1, ORC_QUANT_PER_CHANNEL = 2 };

/* Scalar converters (round-to-nearest-even from IEEE-754 / OCP FP8 definitions). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
uint8_t orc_f32_to_e4m3(float f); /* RNE, saturating to +-448, NaN -> 0x7f */
float orc_e4m3_to_f32(uint8_t c);

/* Integer KV code of one value (QuantizedCache::encode, kv_cache.rs:170-199; byte equations of
 * test_quantized_kv.py:22-37): reciprocal = 0 is the paged rule x / scale with a zero scale
 * giving 0; reciprocal = 1 is the GroupQueryAttention (MLAS) rule x * fp32(1 / scale) with a zero
 * scale read as 1.  Clip to [-2^(bits-1), 2^(bits-1) - 1], round half to even.  NaN -> 0. */
int orc_int_code(float x, float scale, int bits, int reciprocal);
/* One kv-head row of head_dim values -> int8 codes, or int4 bytes (code + 8, channel 2i in the
 * low nibble, 2i+1 in the high nibble, an odd row's last high nibble 8).  scale points at the
 * single per-tensor scale or at this row's head_dim channel scales (per_channel). */
void orc_int_encode_row(const float* x, int head_dim, const float* scale, int per_channel,
                        int bits, int reciprocal, uint8_t* dst);
/* QuantizedCache::decode (kv_cache.rs:222-256): code * scale in fp32. */
void orc_int_decode_row(const uint8_t* src, int head_dim, const float* scale, int per_channel,
                        int bits, float* out);

/* Bulk converters between float32 and a storage dtype. */
void orc_encode(const float* src, void* dst, int64_t n, int dtype);
void orc_decode(const void* src, float* dst, int64_t n, int dtype);

/* In-place RMSNorm over head_dim of rows [rows, heads, head_dim] (mlx_fast_rms_norm at
 * attention.rs:4045-4049; numpy form test_paged_attention.py:101-103), with the sum of squares
 * of orc_sum_squares (64 fma partials over a stride of 64, then an XOR butterfly 32..1). */
float orc_sum_squares(const void* x, int64_t base, int head_dim, int dtype);
void orc_rms_norm_rows(void* x, int64_t rows, int heads, int head_dim, const void* weight,
                       float eps, int dtype);

/* In-place rotary embedding with per-op rounding to dtype (gqa_rope attention.rs:459-503,
 * rope_with_offset :3812-3855, cos_sin_row :523-535). positions[rows]. */
int orc_rope_rows(void* x, int64_t rows, int heads, int head_dim, const int32_t* positions,
                  const void* cos_cache, const void* sin_cache, int64_t cos_rows, int half,
                  int offset, int interleaved, int dtype);

/* Slot rule + scatter (attention.rs:4064-4120; test_paged_attention.py:117-126).
 * cache_dtype == ORC_E4M3 quantises x / scale[block, kv-head] (zero scale -> 0); ORC_I8 / ORC_I4
 * store integer codes (paged divide rule) with per-tensor or per-channel scales given by
 * k_mode / v_mode (ORC_QUANT_*); int4 rows are (head_dim + 1) / 2 bytes. */
int orc_reshape_and_cache(const void* key, const void* value, int act_dtype, void* key_cache,
                          void* value_cache, int cache_dtype, const float* k_scale,
                          const float* v_scale, int k_mode, int v_mode, const int32_t* cum,
                          const int32_t* past,
                          const int32_t* block_table, int batch, int max_blocks,
                          const int32_t* slot_mapping, int64_t num_blocks, int block_size,
                          int kv_heads, int head_dim);

/* Attention after append, in double (_paged_ref test_paged_attention.py:127-155, dense
 * fallback attention.rs:4192-4319, sink/softcap :79-118). q/k_new/v_new are the rotated rows in
 * act_dtype.  head_sink: fp32 [H] or NULL.  out: [num_tokens, H*head_dim] doubles.
 * Quantised caches (fp8, int8, int4) read every position, new rows included, from the pages
 * (attention.rs:4192-4195).  value_cache == NULL is the LATENT layout: values are the first
 * v_head_dim (0 = head_dim) dims of the key rows and out is [num_tokens, H*v_head_dim]. */
int orc_paged_attention(const void* q, const void* k_new, const void* v_new, int act_dtype,
                        const void* key_cache, const void* value_cache, int cache_dtype,
                        const float* k_scale, const float* v_scale, int k_mode, int v_mode,
                        const int32_t* cum,
                        const int32_t* past, const int32_t* block_table, int batch,
                        int max_blocks, int64_t num_blocks, int block_size, int num_heads,
                        int kv_heads, int head_dim, float scale, float softcap, int window,
                        int causal, const float* head_sink, double* out, int v_head_dim);

/* Whole operator: norm + rope + append + attention (paged_attention_op attention.rs:3857-4382
 * and _paged_ref test_paged_attention.py:63-157).  Caches are updated in place.
 * out_t (may be NULL) receives the output rounded to act_dtype. */
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
                           int v_head_dim);

/* Contiguous-cache GroupQueryAttention (ORT CPU semantics as restated by the reference's
 * test_gqa_position_cache.py:88-126 and gqa_batched attention.rs:586-848):
 * query [B,S,H*d], key/value [B,S,KV*d], present_k/v [B,KV,cap,d] (past in, present out),
 * seqlens_k[b] = total_b - 1.  Computes in double.  out [B,S,H*d].
 * cache_dtype ORC_I8 / ORC_I4 (0 = dtype): integer present caches [B,KV,cap,width] holding codes
 * of the reciprocal (MLAS) rule; attention reads code * scale of every row. */
int orc_gqa_contiguous(int dtype, const void* query, const void* key, const void* value,
                       void* present_k, void* present_v, int batch, int seq, int num_heads,
                       int kv_heads, int head_dim, int cap, const int32_t* seqlens_k,
                       float scale, float softcap, int window, int causal, double* out,
                       int cache_dtype, const float* k_scale, const float* v_scale, int k_mode,
                       int v_mode);

/* GroupQueryAttention on contiguous caches, every form of gqa_batched (attention.rs:586-848,
 * reached from group_query_attention_op :932-1454): per sequence length = seqlens_k[b] + 1,
 * query_past = max(length - seq, 0), past = kv_seq == 0 ? length : query_past; query rows sit
 * at query_past + i (ragged first prompts: right-padded rows beyond the length); RMSNorm of q/k
 * (qk norm), then RoPE at query_past + i or at the position ids (first prompt, total == seq:
 * pid[0] + i; later: pid_flat[b * seq + i]) — in fp32 with one rounding when position ids are
 * given or kv_seq == 0 (gqa_rope_f32), per-op T rounding otherwise (gqa_rope); the present is
 * [past rows | new rows | past tail | zero codes] of present_cap rows; attention over the
 * present's first length rows with the top-left causal rule key <= query_past + i, the window
 * lower bound min(query_past + i - w + 1, length - w) (:328-359), scale, softcap, + bias
 * [b|1, h|1, i, key], and a sink logit (head_sink, or 0 for smooth_softmax) in the denominator
 * only (:100-118).  Computes in double; out [B, S, H * d]. */
typedef struct orc_gqa_args {
  int dtype, batch, seq, kv_seq, num_heads, kv_heads, head_dim;
  const void* query;   /* [B, S, H * d] */
  const void* key;     /* [B, kv_seq, KV * d] (unused when kv_seq == 0) */
  const void* value;
  const void* past_k;  /* [B, KV, past_cap, w] or NULL (no past) */
  const void* past_v;
  int past_cap;
  void* present_k;     /* out [B, KV, present_cap, w] */
  void* present_v;
  int present_cap;
  const int32_t* seqlens_k;
  int64_t total;
  const void* cos_cache; /* [cos_rows, rot_half] or NULL (no rotary) */
  const void* sin_cache;
  int64_t cos_rows;
  int rot_half, interleaved;
  const int64_t* position_ids; /* flattened [B, >= S] or NULL */
  const void* bias;            /* [bias_b, bias_h, S, total] in T or NULL */
  int bias_b, bias_h;
  const void* head_sink;       /* [H] in T or NULL */
  int smooth;
  const void* q_norm;          /* [d] in T or NULL */
  const void* k_norm;
  float norm_eps, scale, softcap;
  int window, causal;
  int cache_dtype;             /* 0 (= dtype), ORC_I8 or ORC_I4 */
  const float* k_scale;
  const float* v_scale;
  int k_mode, v_mode;
  /* sliding_window_cache (attention.rs:1139-1330): past and present are rings of capacity
   * past_cap (present_cap must equal it) holding the last cache_end(length) rows; window > 0 */
  int sliding;
  /* qk_output (attention.rs:771-785): 1 the visible logits (scaled, softcapped, biased; 0 where
   * masked), 2 the probabilities, into qk_out [B, H, S, total] (columns >= length are 0) */
  int qk_mode;
  double* qk_out;
} orc_gqa_args;
int orc_gqa_batched(const orc_gqa_args* a, double* out);

/* CPU baseline (pa_cpu_baseline.c): the same contiguous GQA decode in fp32 accumulation over
 * all requested threads, one task per (sequence, kv-head).  k/v: [sum_b ctx_b, KV, d] packed
 * per sequence at row offsets kv_offset[b]; q [B, H, d]; out [B, H, d] float. */
int orc_cpu_gqa_decode(int dtype, const void* q, const void* k, const void* v,
                       const int64_t* kv_offset, const int32_t* ctx, int batch, int num_heads,
                       int kv_heads, int head_dim, float scale, float* out, int threads);

/* The CPU path for chunked prefill (bench.py config 4): causal GQA over contiguous K/V
 * ([past + nq, kv_heads, head_dim] per sequence at kv_offset), query rows q_start[b] ..
 * q_start[b] + nq[b] - 1 at positions past[b] .., fp32 accumulation, `threads` pthreads. */
int orc_cpu_gqa_prefill(int dtype, const void* q, const void* k, const void* v,
                        const int64_t* kv_offset, const int32_t* q_start, const int32_t* nq,
                        const int32_t* past, int batch, int num_heads, int kv_heads,
                        int head_dim, float scale, float* out, int threads);

#ifdef __cplusplus
}
#endif

#endif
