/*
 * pa_mi355x.h — C ABI of the MI355X (gfx950) paged GQA KV-cache attention library.
 *
 * This is the seam the reference plugin EP crosses when it runs com.microsoft::PagedAttention:
 * there the op handler builds an MLX graph (scatter into the flattened cache, page gather,
 * SDPA, or a custom Metal vector kernel); here the same inputs are handed, as plain device
 * pointers and sizes, to hand-written HIP kernels.  Nothing in this header uses torch, HIP or
 * ORT types; hipStream_t is passed as the opaque `pa_stream_t`.
 *
 * Conventions
 *   - Every entry point returns 0 on success or a PA_ERR_* code; pa_last_error() returns the
 *     thread-local message of the last failure.  Messages raised while validating operator
 *     metadata start with "PagedAttention:" like the reference's errors
 *     (rust/src/ops/attention.rs:3938-3990).
 *   - All tensor pointers are device pointers unless the field name starts with host_.
 *   - No entry point allocates device memory except pa_pool_create; split-K partials live in
 *     a caller-provided workspace sized by pa_attention_workspace_bytes.
 *   - Work is enqueued on `stream`; nothing synchronises the host unless stated.
 *
 * Layouts (identical to the ORT operator contract the reference claims,
 * rust/src/ops/attention.rs:4537-4560 and tests/ops/test_paged_attention.py:161-178):
 *   query            [num_tokens, num_heads * head_dim]           activation dtype T
 *   key, value       [num_tokens, kv_heads * head_dim]            T
 *   key/value_cache  [num_blocks, block_size, kv_heads, head_dim] T (or e4m3 with per-(block,
 *                    kv-head) fp32 scales for the fp8 cache, a build-defined extension)
 *   cumulative_sequence_length [batch + 1] int32, past_seqlens [batch] int32,
 *   block_table      [batch, max_blocks] int32, slot_mapping [num_tokens] int32 (-1 = skip)
 *   cos/sin cache    [positions, rotary_dim / 2] T
 *   output           [num_tokens, num_heads * head_dim] T
 */
#ifndef PA_MI355X_H
#define PA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pa_stream_t; /* hipStream_t; NULL = the null stream */

typedef enum pa_dtype {
  PA_DTYPE_FLOAT16 = 1,
  PA_DTYPE_BFLOAT16 = 2,
  PA_DTYPE_FLOAT32 = 3,
  PA_DTYPE_FP8_E4M3 = 4, /* OCP e4m3fn, cache storage only */
  /* Integer cache storage (ORT int8 / uint8 "int4" caches, kv_cache.rs:110-256): */
  PA_DTYPE_INT8 = 5, /* one signed code per channel */
  PA_DTYPE_INT4 = 6  /* uint8 bytes of two (code + 8) nibbles: channel 2i low, 2i+1 high; an
                        odd head's last high nibble is 8; a row is (head_dim + 1) / 2 bytes */
} pa_dtype;

/* Scale layout of one side of an integer cache ("k_quant_type" / "v_quant_type"). */
#define PA_QUANT_NONE 0
#define PA_QUANT_PER_TENSOR 1  /* one fp32 scale */
#define PA_QUANT_PER_CHANNEL 2 /* fp32 [kv_heads, head_dim] */

#define PA_OK 0
#define PA_ERR_INVALID_ARGUMENT 1
#define PA_ERR_UNSUPPORTED 2
#define PA_ERR_HIP 3
#define PA_ERR_OUT_OF_MEMORY 4

/* Thread-local text of the last failure on this thread ("" if none).
 * Replaces the OrtStatus message path of the reference's FFI guard (rust/src/lib.rs:53-80). */
const char* pa_last_error(void);
const char* pa_version(void);

/* ------------------------------------------------------------------------------------------ */
/* Page pool: the HBM slab behind the cache tensors.  Replaces the MLX-backed "MLX" device
 * OrtAllocator that hands out the cache tensors (rust/src/device.rs:415-486, created by
 * factory.rs:266-286).  One hipMalloc per side, [num_blocks, block_size, kv_heads, head_dim]
 * elements ((head_dim + 1) / 2 bytes per kv-head row for PA_DTYPE_INT4). */
typedef struct pa_pool pa_pool;

int pa_pool_create(int64_t num_blocks, int32_t block_size, int32_t kv_heads, int32_t head_dim,
                   pa_dtype cache_dtype, pa_pool** out_pool);
int pa_pool_destroy(pa_pool* pool);
void* pa_pool_k_ptr(const pa_pool* pool);
void* pa_pool_v_ptr(const pa_pool* pool);
/* fp8 pools only: per-(block, kv-head) fp32 scales, [num_blocks, kv_heads]; NULL otherwise. */
float* pa_pool_k_scale_ptr(const pa_pool* pool);
float* pa_pool_v_scale_ptr(const pa_pool* pool);
int64_t pa_pool_bytes(const pa_pool* pool);

/* ------------------------------------------------------------------------------------------ */
/* Descriptors shared by the kernel-level entry points. */

/* A paged KV cache (inputs 3/4 of PagedAttention, attention.rs:3922-3932).
 * Integer caches (inputs 14/15 = k_scale/v_scale, QuantizedCache kv_cache.rs:110-256): a new
 * row is stored as codes sat(RNE(x / scale)) (zero scale -> code 0) and every key/value the
 * attention reads, the new rows included, is code * scale in fp32 read back from the pages. */
typedef struct pa_cache {
  void* key_cache;
  void* value_cache; /* NULL: the LATENT layout, each position's value is the first
                        v_head_size dims of its key row (attention.rs:4058-4062, :4210-4213) */
  const float* k_scale; /* fp8: [num_blocks, kv_heads]; int8/int4: see k_quant_type */
  const float* v_scale; /* fp8: [num_blocks, kv_heads]; int8/int4: see v_quant_type */
  int64_t num_blocks;
  int32_t block_size;
  int32_t kv_heads;
  int32_t head_dim; /* logical head size (int4 rows hold (head_dim + 1) / 2 bytes) */
  pa_dtype dtype;   /* storage dtype: T, PA_DTYPE_FP8_E4M3, PA_DTYPE_INT8 or PA_DTYPE_INT4 */
  int32_t k_quant_type; /* PA_QUANT_*: integer caches only (PA_QUANT_NONE otherwise) */
  int32_t v_quant_type;
} pa_cache;

/* Packed var-length batch metadata (inputs 5/6/7/10, attention.rs:3934-3990). */
typedef struct pa_batch {
  const int32_t* cumulative_sequence_length; /* [batch + 1] */
  const int32_t* past_seqlens;               /* [batch] */
  const int32_t* block_table;                /* [batch, max_blocks] */
  const int32_t* slot_mapping;               /* [num_tokens] or NULL */
  int32_t batch;
  int32_t max_blocks;
  int32_t num_tokens;
  /* Host-known upper bound of new tokens per sequence; selects decode vs prefill kernels
   * without a device read.  0 means "unknown" and is treated as num_tokens. */
  int32_t max_query_len;
  uint32_t flags; /* PA_BATCH_* bits */
  /* Host-known upper bound of past + new tokens of any one sequence.  It sizes the operand images
   * of the planned prefill (part of the workspace) by the live context instead of the block-table
   * capacity.  0 means "unknown" and is treated as max_blocks * block_size.  The caller
   * guarantees the bound: the query rows of a sequence whose context exceeds it may be left
   * unwritten (no access outside the buffers). */
  int32_t max_context_len;
} pa_batch;

/* The caller guarantees that every new key/value row was written to its block-table slot on
 * this stream before the attention call (pa_rotary_append / pa_reshape_and_cache without a
 * slot_mapping) and that no two tokens share a slot, so new positions may be read from the
 * pages.  pa_paged_attention sets this itself when its host metadata proves it. */
#define PA_BATCH_NEW_ROWS_IN_CACHE 1u

/* The caller guarantees that no two new tokens map to the same cache slot, so the append
 * skips its last-writer-wins check (a scan over later tokens).  pa_paged_attention sets this
 * itself when its host metadata proves it. */
#define PA_BATCH_SLOTS_DISTINCT 2u

/* Attention attributes (attention.rs:3857-3870, 4255-4311; attr_scale :448-453). */
typedef struct pa_attn {
  int32_t num_heads;
  float scale;               /* 0 -> 1/sqrt(head_dim) */
  float softcap;             /* 0 -> off; else softcap * tanh(s / softcap) */
  int32_t local_window_size; /* -1 -> off; else keys >= row - window + 1 */
  int32_t is_causal;         /* 1: key p visible to row r iff p <= past + r */
  const void* head_sink;     /* [num_heads] in activation dtype, or NULL */
  int32_t v_head_size;       /* 0 -> head_dim; smaller only for a LATENT cache; q/out rows are
                                [num_heads * head_dim] / [num_heads * v_head_size] */
} pa_attn;

/* ------------------------------------------------------------------------------------------ */
/* Kernel-level entry points (what the op handler calls once metadata is validated). */

/* KV append, optionally fused with Q/K RMSNorm and rotary embedding (a4/a5/a6 of the path).
 * Replaces the per-sequence rope_with_offset + mlx_scatter_single loop of
 * attention.rs:4021-4120 (gqa_rope :459-503, cos_sin_row :523-535, slot rule :4064-4079).
 *   query/key/value      [num_tokens, heads * head_dim] in act_dtype
 *   q_out / k_out        rotated (and normalised) query/key rows, same layout; may alias
 *                        query/key; may be NULL when no rotation/normalisation is requested
 *   cos_cache/sin_cache  [rotary_positions, rotary_half] act_dtype, or NULL (no rotary)
 *   q_norm/k_norm        [head_dim] act_dtype, or NULL
 * Cache rows are written in token order: when two tokens target one slot, the later token's
 * row is the one left in the cache (test_paged_attention.py:117-126, :605-659).  Every
 * elementwise rotary/norm step rounds to act_dtype, as the reference's per-op MLX graph does. */
int pa_rotary_append(const pa_cache* cache, const pa_batch* batch, int32_t num_heads,
                     pa_dtype act_dtype, const void* query, const void* key, const void* value,
                     void* q_out, void* k_out, const void* cos_cache, const void* sin_cache,
                     int64_t rotary_positions, int32_t rotary_half, int32_t rotary_offset,
                     int32_t rotary_interleaved, const void* q_norm, const void* k_norm,
                     float norm_eps, pa_stream_t stream);

/* Pure reshape_and_cache: bit copy of key/value rows into their slots (or fp8 quantisation
 * x / scale, zero scale -> 0, RNE, saturate to +-448; or integer codes, see pa_cache).  Same
 * slot and ordering rules. */
int pa_reshape_and_cache(const pa_cache* cache, const pa_batch* batch, pa_dtype act_dtype,
                         const void* key, const void* value, pa_stream_t stream);

/* Workspace (bytes) needed by pa_attention for split-K partials. */
size_t pa_attention_workspace_bytes(const pa_cache* cache, const pa_batch* batch,
                                    const pa_attn* attn);
/* Workspace (bytes) needed by pa_attention_ex for the given kind / chunk. */
size_t pa_attention_workspace_bytes_ex(const pa_cache* cache, const pa_batch* batch,
                                       const pa_attn* attn, pa_dtype act_dtype, int32_t kind,
                                       int32_t chunk_tokens);

/* Attention over the paged cache after append.  Keys/values at positions < past come from the
 * cache pages; positions >= past come from k_new/v_new (the rotated new rows), exactly as the
 * reference's _paged_ref and its patched Metal kernel do (attention.rs:4161-4190,
 * paged_attention.rs:46-74).  fp8 and integer caches read every position from the pages (the
 * quantised rule of attention.rs:4192-4194).  q: [num_tokens, num_heads*head_dim]; out
 * likewise.
 * Dispatch (fp16/bf16 activations at head sizes 64, 96, 128 and 256 run on matrix cores):
 *   - decode batches, (num_heads/kv_heads) * max_query_len <= 16 with a power-of-two block size:
 *     the streaming (stream-K) decode over pages in T, and at heads 64/128 over fp8, int8 and
 *     int4 pages of at least 16 rows;
 *   - other batches over pages in T: the LDS-shared prefill kernel (128 grouped query rows per
 *     workgroup; the planned launch -- longest-first units, long items split in two -- once the
 *     batch fills two workgroups per compute unit, over operand images when each (sequence,
 *     kv-head) has at least 4 row blocks);
 *   - other batches over fp8 / int8 / int4 pages: the planned prefill over operand images (fp16
 *     rows of the live context, within 2 GiB of workspace; larger batches run it on groups of
 *     sequences whose images fit, one launch per group);
 *   - the LATENT layout (one kv-head, values = the first v_head_size key dims) with the cache in
 *     the activation dtype, key rows of a multiple of 32 dims up to 640 and values of 128, 256
 *     or 512 dims (MLA 576 / 512): its matrix-core kernel, all heads served by one read of each
 *     row per 16 grouped query rows;
 *   - fp32 activations, other head sizes, other LATENT shapes and forced split-K chunks over
 *     byte-coded pages: the VALU kernel.
 * batch->max_query_len = 0 is read as num_tokens. */
int pa_attention(const pa_cache* cache, const pa_batch* batch, const pa_attn* attn,
                 pa_dtype act_dtype, const void* q, const void* k_new, const void* v_new,
                 void* out, void* workspace, size_t workspace_bytes, pa_stream_t stream);

/* Same contract, forcing one kernel family (for parity tests and benchmarks).
 * kind: 0 = automatic, 1 = decode MFMA (balanced segments when every sequence has at most 16
 * grouped query rows, else chunked split-K), 2 = LDS-shared prefill kernel (planned launch when
 * the batch fills the GPU and chunk_tokens is 0, else split-K chunks), 3 = generic VALU,
 * 4 = decode MFMA with chunked split-K forced.  A kind that does not cover the dtype / head size
 * returns PA_ERR_UNSUPPORTED.  The LATENT layout takes 0 (its matrix-core kernel where that
 * covers the shape) or 3.
 * chunk_tokens: split-K chunk for the chunked/generic kernels (multiple of 32; 0 = automatic). */
int pa_attention_ex(const pa_cache* cache, const pa_batch* batch, const pa_attn* attn,
                    pa_dtype act_dtype, const void* q, const void* k_new, const void* v_new,
                    void* out, void* workspace, size_t workspace_bytes, int32_t kind,
                    int32_t chunk_tokens, pa_stream_t stream);

/* ------------------------------------------------------------------------------------------ */
/* Operator-level entry: the Compute body of com.microsoft::PagedAttention
 * (paged_attention_op, attention.rs:3857-4382), minus ORT tensor plumbing. */

typedef struct pa_paged_attention_node {
  int32_t num_heads;          /* "num_heads" */
  int32_t kv_num_heads;       /* "kv_num_heads" */
  float scale;                /* "scale" (0 = default) */
  float softcap;              /* "softcap" */
  int32_t local_window_size;  /* "local_window_size" (-1) */
  int32_t do_rotary;          /* "do_rotary" */
  int32_t rotary_interleaved; /* "rotary_interleaved" */
  int32_t rotary_offset;      /* "rotary_offset" */
  int32_t is_causal;          /* "is_causal" (1) */
  float qk_norm_epsilon;      /* "qk_norm_epsilon" (1e-6) */
  int32_t v_head_size;        /* "v_head_size" (0 = head_size) */
  /* "kv_cache_layout" == "LATENT": kv_num_heads 1, inputs 2/4 (value, value_cache) absent,
   * values are the first v_head_size dims of the (rotated) key rows, output
   * [num_tokens, num_heads * v_head_size]. */
  int32_t kv_cache_layout_latent;
} pa_paged_attention_node;

typedef struct pa_paged_attention_io {
  pa_dtype dtype;              /* T */
  int32_t num_tokens;          /* query.shape[0] */
  int32_t query_hidden;        /* query.shape[1]; key == value == NULL: packed QKV, query is
                                  [num_tokens, (num_heads + 2 * kv_num_heads) * head] */
  const void* query;           /* input 0 */
  const void* key;             /* input 1 (NULL: packed) */
  const void* value;           /* input 2 (NULL: packed, or LATENT) */
  pa_cache cache;              /* inputs 3/4 (+14/15 for fp8 / integer cache scales) */
  const int32_t* cumulative_sequence_length; /* input 5, device */
  const int32_t* past_seqlens; /* input 6, device */
  const int32_t* block_table;  /* input 7, device */
  int32_t batch;               /* input 5 length - 1 */
  int32_t max_blocks;          /* input 7 shape[1] */
  const void* cos_cache;       /* input 8 */
  const void* sin_cache;       /* input 9 */
  int64_t rotary_positions;    /* input 8 shape[0] */
  int32_t rotary_half;         /* input 8 shape[1] */
  const int32_t* slot_mapping; /* input 10, device, or NULL */
  const void* head_sink;       /* input 11 or NULL */
  const void* q_norm_weight;   /* input 12 or NULL */
  const void* k_norm_weight;   /* input 13 or NULL */
  /* Host copies of inputs 5/6/7/10.  The reference reads these on the host every step
   * (read_int_input, attention.rs:3733-3753); when given they are validated with the
   * reference's rules and error messages.  When NULL the device copies are trusted (kernels
   * still clamp every index so malformed metadata cannot fault). */
  const int32_t* host_cumulative_sequence_length;
  const int32_t* host_past_seqlens;
  const int32_t* host_block_table;
  const int32_t* host_slot_mapping;
  void* output;                /* output 0 */
  /* Outputs 1/2 (key_cache_out / value_cache_out).  The input caches are always updated in
   * place.  NULL (output omitted) or the input cache's own address (the output bound onto the
   * input, ORT's shared-buffer binding): nothing more is written.  A distinct buffer of the
   * cache's shape and dtype receives a copy of the whole updated cache (engine.rs:110-126
   * full-copy path, attention.rs:4336-4380).  value_cache_out must be NULL for LATENT. */
  void* key_cache_out;
  void* value_cache_out;
  /* Host-known bound on the new tokens of any one sequence (max of cum[b+1] - cum[b]); 0 =
   * unknown.  It selects the kernel family and sizes the workspace without a device read.
   * With host_cumulative_sequence_length it must be >= the largest query length there (else
   * PA_ERR_INVALID_ARGUMENT); without it the caller guarantees the bound, and query rows beyond
   * it are left unwritten (no access outside the buffers).  0 without host metadata: the bound
   * is num_tokens. */
  int32_t max_query_len;
  /* Host-known bound on past + new tokens of any one sequence (max of past[b] + cum[b+1] -
   * cum[b]); 0 = unknown.  It sizes the workspace's operand images of multi-token batches by the
   * live context rather than by max_blocks * block_size.  With host metadata the exact maximum is
   * used and a smaller bound is refused (PA_ERR_INVALID_ARGUMENT); without it the caller
   * guarantees the bound, and query rows of a sequence beyond it may be left unwritten (no access
   * outside the buffers).  0 without host metadata: the block-table capacity. */
  int32_t max_context_len;
} pa_paged_attention_io;

/* Workspace bytes for one call.  The size depends on the shapes (num_tokens, batch,
 * max_blocks, heads, head size, dtypes, block size) and on the query-length bound (io's
 * max_query_len, else the host cumulative lengths, else num_tokens); a caller that always passes
 * the same max_query_len (its largest chunk) may size the workspace once per shape. */
size_t pa_paged_attention_workspace_bytes(const pa_paged_attention_node* node,
                                          const pa_paged_attention_io* io);
int pa_paged_attention(const pa_paged_attention_node* node, const pa_paged_attention_io* io,
                       void* workspace, size_t workspace_bytes, pa_stream_t stream);

/* Allocation-free variant of pa_paged_attention.  It has no counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same contract as pa_paged_attention, except that the
 * workspace is a scratch buffer of PA_STATIC_SCRATCH_BYTES inside the library's code object on
 * each GPU (a file-scope __device__ array, resident until the process ends): a call whose
 * workspace (pa_paged_attention_workspace_bytes) exceeds it returns PA_ERR_UNSUPPORTED before
 * any device work.  No hipMalloc / hipFree or other allocating routine is called.  Every call
 * on one GPU shares that GPU's scratch: calls that overlap on one GPU (different streams, or
 * host threads) race and must be serialised by the caller; calls in stream order do not.  The
 * kernels need no cleared scratch (everything they read is written earlier in the same call). */
#define PA_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int pa_paged_attention_static(const pa_paged_attention_node* node,
                              const pa_paged_attention_io* io, pa_stream_t stream);

/* Operator-level entry: com.microsoft::GroupQueryAttention on contiguous caches
 * (group_query_attention_op / gqa_batched, attention.rs:932-1454 and :586-848).
 * Per sequence b, with length = seqlens_k[b] + 1 (the reference's rules, attention.rs:614-672):
 *   query_past = max(length - seq, 0); the seq query rows sit at positions query_past + i;
 *   kv_seq == seq: the first length - query_past new key/value rows are stored at
 *   [query_past, length) (a ragged first prompt, total_sequence_length == seq, stores only
 *   `length` rows); kv_seq == 0: no new rows, the past already holds all `length` keys.
 *   Row i attends keys [0, length) with the top-left causal rule p <= query_past + i, the
 *   window rule p >= min(query_past + i, length - 1) - window + 1, an optional additive bias,
 *   softcap, and a sink logit (head_sink, or 0 for smooth_softmax) in the denominator only.
 *   present = [the length stored rows | past rows [length, past_capacity) | zero codes up to
 *   present_capacity] (int4 zero codes are 0x88 bytes).
 * Caches: present_key == past_key (the shared-buffer binding): updated in place, capacity
 * past_capacity.  present_key of its own ([batch, kv_heads, present_capacity, head] with
 * present_capacity = max(past_capacity, total_sequence_length), the growing present): past rows
 * are copied in first.  present_key NULL (output omitted): the present lives in the workspace.
 * past_key NULL (no past inputs): every sequence must be a first prompt.
 * RoPE (do_rotary) rotates the query rows and the stored key rows at their positions with the
 * supplied cache rows, each operation rounded to T like the reference's composed graph; with
 * position_ids (input 9: first prompt, total_sequence_length == seq: rows pid[0] + i of every
 * sequence; later calls: pid_flat[b * seq + i]) or kv_seq == 0 the rotation runs in fp32 and
 * rounds once (gqa_rope_f32, attention.rs:506-521).  Messages of invalid inputs start with
 * "GroupQueryAttention:".  Integer present caches (cache_dtype PA_DTYPE_INT8 / PA_DTYPE_INT4,
 * "kv_cache_bit_width" 8 / 4) encode the new rows as sat(RNE(x * (1 / scale))) with a zero scale
 * read as 1 (the MLAS reciprocal rule, kv_cache.rs:183-190) and attend over code * scale.
 * sliding_window_cache = 1 (attention.rs:1139-1368): past_key / past_value are rings of capacity
 * past_capacity >= local_window_size > 0 (present_capacity must equal it; the present is the
 * past buffer itself or one of its own, never omitted; kv_seq == seq).  A sequence of length L
 * holds its last ring_end(L) rows at rows [0, ring_end(L)): L while L <= capacity, else L less
 * whole multiples of gap = capacity - window + 1.  A call with p = length - seq past rows
 * attends the staged view [the ring's ring_end(p) rows | the seq new rows] under the causal
 * window (new row i at absolute position p + i, rotated there; RoPE in fp32 with position ids or
 * a bias; bias columns at absolute positions) and writes the present [the view's last
 * ring_end(p + seq) rows | zero codes].  The view lives in the workspace.
 * qk_output = 1 / 2 (attention.rs:771-785, :833-839; not with sliding_window_cache): output_qk
 * receives, per (sequence, head, query row), the scaled, softcapped, biased scores where the row
 * sees the key (1) or the probabilities with the sink in the denominator (2), 0 elsewhere and in
 * the columns past the sequence's length; computed on the VALU after the attention.
 * Kernels: fp16/bf16 decode batches (num_heads/kv_heads * seq <= 16) run the streaming
 * matrix-core decode -- heads 64/96/128/256 over presents in the activation dtype, heads 64/128
 * over int8 / int4 presents (codes read per lane from the contiguous rows) -- with or without an
 * attention_bias; multi-token batches at those heads run the matrix-core prefill (int8 / int4
 * presents over operand images of the codes; with a bias prefill_kernel, which takes it at every
 * head size, over presents in the activation dtype); ragged first prompts (sequences shorter than
 * seq) bound each sequence's keys on the same kernels.  fp32 activations, other head sizes and a
 * bias on a multi-token batch over int8 / int4 presents run the VALU kernel. */
typedef struct pa_gqa_node {
  int32_t num_heads;          /* "num_heads" */
  int32_t kv_num_heads;       /* "kv_num_heads" */
  float scale;                /* "scale" (0 = 1/sqrt(head)) */
  float softcap;              /* "softcap" */
  int32_t local_window_size;  /* "local_window_size" (-1) */
  int32_t do_rotary;          /* "do_rotary" */
  int32_t rotary_interleaved; /* "rotary_interleaved" */
  int32_t is_causal;          /* "causal" (1) */
  float qk_norm_epsilon;      /* "qk_norm_epsilon" (1e-6) */
  int32_t smooth_softmax;     /* "smooth_softmax" == 1: a zero sink logit for every head */
  int32_t sliding_window_cache; /* "sliding_window_cache" (0): ring caches, see below */
  int32_t qk_output;          /* "qk_output" (0): 1 scores, 2 probabilities into output_qk */
} pa_gqa_node;

typedef struct pa_gqa_io {
  pa_dtype dtype;            /* T */
  int32_t batch;             /* query.shape[0] */
  int32_t seq;               /* query.shape[1] (query rows per sequence) */
  int32_t query_hidden;      /* query.shape[2] = num_heads * head (packed: (H + 2 KV) * head) */
  int32_t kv_seq;            /* key.shape[1]: seq, or 0 (no new rows; needs a past) */
  const void* query;         /* input 0 [batch, seq, query_hidden] */
  const void* key;           /* input 1 [batch, kv_seq, kv_heads * head] (NULL with value NULL
                                and kv_seq == seq: packed QKV; unread when kv_seq == 0) */
  const void* value;         /* input 2 */
  const void* past_key;      /* input 3 [batch, kv_heads, past_capacity, stored head] or NULL */
  const void* past_value;    /* input 4 */
  int32_t past_capacity;     /* input 3 shape[2] (0 when absent) */
  void* present_key;         /* output 1 (== past_key, a buffer of its own, or NULL) */
  void* present_value;       /* output 2 */
  int32_t present_capacity;  /* output 1 shape[2] (ignored when present_key is NULL) */
  const int32_t* seqlens_k;  /* input 5 [batch], device */
  const int32_t* host_seqlens_k; /* host copy of input 5 (enables validation) or NULL */
  int64_t total_sequence_length; /* input 6 (host scalar) */
  const void* cos_cache;     /* input 7 [positions, rotary_dim / 2] */
  const void* sin_cache;     /* input 8 */
  int64_t rotary_positions;
  int32_t rotary_half;
  const int64_t* position_ids;      /* input 9 [batch, position_cols] int64, device, or NULL */
  const int64_t* host_position_ids; /* host copy of input 9 (validation) or NULL */
  int32_t position_cols;
  const void* attention_bias; /* input 10 [bias_batch, bias_heads, seq, total_sequence_length]
                                 in T (additive, after scale and softcap), or NULL */
  int32_t bias_batch;         /* 1 or batch */
  int32_t bias_heads;         /* 1 or num_heads */
  const void* head_sink;     /* input 11 [num_heads] or NULL */
  const void* q_norm_weight; /* inputs 14/15 [head] or NULL */
  const void* k_norm_weight;
  void* output;              /* output 0 [batch, seq, num_heads * head] */
  pa_dtype cache_dtype;      /* present storage: 0 (= T), PA_DTYPE_INT8 or PA_DTYPE_INT4 */
  const float* k_scale;      /* inputs 12/13 for integer caches, see pa_cache */
  const float* v_scale;
  int32_t k_quant_type;      /* PA_QUANT_* ("k_quant_type" / "v_quant_type") */
  int32_t v_quant_type;
  void* output_qk;           /* output 3 [batch, num_heads, seq, total_sequence_length] in T
                                (qk_output 1 / 2), else NULL */
} pa_gqa_io;

size_t pa_group_query_attention_workspace_bytes(const pa_gqa_node* node, const pa_gqa_io* io);
int pa_group_query_attention(const pa_gqa_node* node, const pa_gqa_io* io, void* workspace,
                             size_t workspace_bytes, pa_stream_t stream);

/* Claim predicate for a PagedAttention node (paged_attention_claim, attention.rs:4384-4645,
 * plus kv_cache::claim kv_cache.rs:16-108), restricted to what this build executes.
 * Host only; no device work.  Returns 1 (claimed) or 0 (declined, reason written). */
typedef struct pa_node_info {
  int32_t num_inputs;          /* 8..17 */
  int32_t num_outputs;         /* 1..3 */
  int32_t input_present[17];
  int32_t input_dtype[17];     /* pa_dtype, or PA_INT32_DTYPE / PA_INT8_DTYPE / PA_UINT8_DTYPE */
  int32_t input_rank[17];
  int64_t input_shape[17][4];
  int32_t output_present[3];
  int32_t output_dtype[3];
  int32_t output_rank[3];
  int64_t output_shape[3][4];
  int32_t num_heads, kv_num_heads, v_head_size, rotary_offset, do_rotary, local_window_size;
  int32_t is_causal, has_scale_attr;
  float softcap;
  int32_t kv_cache_layout_latent; /* "kv_cache_layout" == "LATENT" */
  /* "k_quant_type"/"v_quant_type": PA_QUANT_* (absent = PA_QUANT_NONE, any other string -1) */
  int32_t k_quant_type, v_quant_type;
  /* "k_cache_dtype"/"v_cache_dtype": 0 when absent or empty, PA_DTYPE_FLOAT16 "float16",
   * PA_DTYPE_BFLOAT16 "bfloat16", PA_DTYPE_INT8 "int8", PA_DTYPE_INT4 "int4", -1 otherwise */
  int32_t k_cache_dtype, v_cache_dtype;
} pa_node_info;
#define PA_INT32_DTYPE 10
#define PA_INT8_DTYPE 11
#define PA_UINT8_DTYPE 12

int pa_paged_attention_claim(const pa_node_info* node, char* reason, size_t reason_len);

/* Claim predicate for a GroupQueryAttention node (group_query_attention_claim,
 * attention.rs:2407-2754, plus kv_cache::claim kv_cache.rs:16-108 for the present caches),
 * restricted to what pa_group_query_attention executes: sliding_window_cache and the output_qk
 * diagnostics (output 3) are declined with their reason.  Host only.  Returns 1 (claimed) or 0
 * (declined, reason written). */
typedef struct pa_gqa_node_info {
  int32_t num_inputs;          /* 7..16 */
  int32_t num_outputs;         /* 1..4 */
  int32_t input_present[16];
  int32_t input_dtype[16];     /* pa_dtype, or PA_INT32_DTYPE / PA_INT8_DTYPE / PA_UINT8_DTYPE /
                                  PA_INT64_DTYPE */
  int32_t input_rank[16];
  int64_t input_shape[16][4];  /* -1: unknown (symbolic) dimension */
  int32_t output_present[4];
  int32_t output_dtype[4];
  int32_t output_rank[4];
  int64_t output_shape[4][4];
  int32_t num_heads, kv_num_heads, do_rotary, is_causal, local_window_size;
  int32_t sliding_window_cache, kv_cache_bit_width, smooth_softmax, qk_output;
  float softcap;
  /* "k_quant_type"/"v_quant_type": PA_QUANT_* (absent = PA_QUANT_NONE, any other string -1) */
  int32_t k_quant_type, v_quant_type;
} pa_gqa_node_info;
#define PA_INT64_DTYPE 13

int pa_group_query_attention_claim(const pa_gqa_node_info* node, char* reason, size_t reason_len);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PA_MI355X_H */
