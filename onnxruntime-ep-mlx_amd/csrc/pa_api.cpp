// pa_api.cpp — host side of the C ABI declared in include/pa_mi355x.h.
//
// Mirrors the reference's PagedAttention operator surface (attention.rs:3857-4382 handler,
// :4384-4645 claim) with its validation rules and "PagedAttention:" error messages, and
// dispatches to the gfx950 kernels.  No torch, no ORT types; every device buffer is provided by
// the caller except the page pool.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "pa_device.hpp"
#include "pa_mi355x.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(PA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t elem_size(pa_dtype d) {
  switch (d) {
    case PA_DTYPE_FLOAT16:
    case PA_DTYPE_BFLOAT16: return 2;
    case PA_DTYPE_FLOAT32: return 4;
    case PA_DTYPE_FP8_E4M3:
    case PA_DTYPE_INT8: return 1;
    case PA_DTYPE_INT4: return 0;  // two channels per byte: use cache_head_bytes
  }
  return 0;
}

bool is_int_cache(pa_dtype d) { return d == PA_DTYPE_INT8 || d == PA_DTYPE_INT4; }

// Bytes of one kv-head's row in a cache of storage dtype d.
size_t cache_head_bytes(pa_dtype d, int head_dim) {
  if (d == PA_DTYPE_INT4) return (size_t)(head_dim + 1) / 2;
  return elem_size(d) * (size_t)head_dim;
}

bool is_act(pa_dtype d) {
  return d == PA_DTYPE_FLOAT16 || d == PA_DTYPE_BFLOAT16 || d == PA_DTYPE_FLOAT32;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Largest head size any kernel serves (the VALU kernel; matrix cores take 64, 96, 128, 256).
constexpr int kMaxHeadDim = 640;

// ---------------------------------------------------------------------------- descriptor checks
int check_cache(const pa_cache* c, pa_dtype act) {
  if (!c) return fail(PA_ERR_INVALID_ARGUMENT, "cache descriptor is NULL");
  if (c->num_blocks <= 0 || c->block_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: caches require matching positive block geometry");
  if (c->kv_heads <= 0 || c->head_dim <= 0 || c->head_dim > kMaxHeadDim)
    return fail(PA_ERR_UNSUPPORTED, "head_dim %d unsupported (1..%d)", c->head_dim,
                kMaxHeadDim);
  if (!c->key_cache) return fail(PA_ERR_INVALID_ARGUMENT, "key_cache pointer is NULL");
  // value_cache == NULL is the LATENT layout (values read from the key rows).
  if (!c->value_cache && c->dtype != act)
    return fail(PA_ERR_UNSUPPORTED, "quantized LATENT cache contract is not supported");
  if (c->dtype == PA_DTYPE_FP8_E4M3) {
    if (!c->k_scale || !c->v_scale)
      return fail(PA_ERR_INVALID_ARGUMENT, "fp8 cache requires k_scale and v_scale");
  } else if (is_int_cache(c->dtype)) {
    // kv_cache.rs:37-60: integer caches need PER_TENSOR / PER_CHANNEL fp32 scales.
    for (int side = 0; side < 2; ++side) {
      const int mode = side ? c->v_quant_type : c->k_quant_type;
      if (mode != PA_QUANT_PER_TENSOR && mode != PA_QUANT_PER_CHANNEL)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "integer %s cache requires PER_TENSOR or PER_CHANNEL quantization",
                    side ? "v" : "k");
      if (!(side ? c->v_scale : c->k_scale))
        return fail(PA_ERR_INVALID_ARGUMENT, "quantized %s cache requires a scale tensor",
                    side ? "v" : "k");
    }
  } else if (c->dtype != act) {
    return fail(PA_ERR_UNSUPPORTED,
                "cache dtype must equal the activation dtype or be fp8 / int8 / int4");
  }
  if (!is_act(act)) return fail(PA_ERR_UNSUPPORTED, "activation dtype must be fp16/bf16/fp32");
  if (c->num_blocks * (int64_t)c->block_size > INT32_MAX)
    return fail(PA_ERR_UNSUPPORTED, "cache has more than 2^31 slots");
  return PA_OK;
}

int check_batch(const pa_batch* bt) {
  if (!bt) return fail(PA_ERR_INVALID_ARGUMENT, "batch descriptor is NULL");
  if (bt->batch < 1)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: cumulative_sequence_length must have length batch+1");
  if (bt->num_tokens < 0 || bt->max_blocks < 1)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: inconsistent cumulative lengths, past lengths or block table");
  if (!bt->cumulative_sequence_length || !bt->past_seqlens || !bt->block_table)
    return fail(PA_ERR_INVALID_ARGUMENT, "metadata pointers are NULL");
  return PA_OK;
}

// ---------------------------------------------------------------------------- attention plan
// kind: 1 decode MFMA (balanced segments when every sequence has <= 16 grouped query rows,
// chunked otherwise), 2 prefill MFMA, 3 generic VALU, 4 decode MFMA forced chunked.
// Balanced decode: sub-segments per wavefront, each for the next kv-head.  Mixing kv-heads
// within a wavefront evens out the different HBM speeds of the kv-heads' byte ranges.
#ifndef PA_DECODE_MIX
#define PA_DECODE_MIX 1
#endif
constexpr int kDecodeMix = PA_DECODE_MIX;

struct Plan {
  int kind;
  bool balanced;
  int chunk;
  int max_splits;    // chunk count (chunked/generic) or sub-segment count (balanced)
  int mix;           // balanced: sub-segments per wavefront
  int ng;            // chunked MFMA kernel: 16-row groups per wavefront
  size_t part_rows;  // rows of fp32 partials in the workspace
  // Planned prefill: items (sequence, row block, kv-head), row blocks per sequence.
  int64_t plan_items = 0;
  int plan_rbs = 0;
  // Planned head-128 prefill with operand images: 64-key steps per (sequence, kv-head) of the
  // image region (0: no images).
  int img_steps = 0;
  // Byte-coded pages whose images of the whole batch exceed the image limit: the planned launch
  // runs on groups of sub_batch sequences in turn, the workspace sized for one group (0: the
  // whole batch in one launch).
  int sub_batch = 0;
};

// Sequences one planned launch covers.
int64_t plan_batch(const pa_batch* b, const Plan& pl) {
  return pl.sub_batch > 0 ? std::min<int64_t>(pl.sub_batch, b->batch) : b->batch;
}

// Operand images of the planned prefill: taken when every key step of the images is read
// by at least kImgMinRowBlocks row blocks (the images are written once and read by each), within
// kImgMaxBytes of workspace.  PA_PREFILL_IMAGES=0 at build time keeps the in-loop conversion.
#ifndef PA_PREFILL_IMAGES
#define PA_PREFILL_IMAGES 1
#endif
#ifndef PA_IMG_WAVES
#define PA_IMG_WAVES 2
#endif
constexpr int64_t kImgMinRowBlocks = 4;
// LATENT kernel: context chunks sized for this many workgroups per CU
#ifndef PA_LATENT_TARGET
#define PA_LATENT_TARGET 2
#endif
constexpr int64_t kImgMaxBytes = (int64_t)1 << 31;

int max_ctx_bound(const pa_cache* c, const pa_batch* b) {
  int64_t v = (int64_t)b->max_blocks * c->block_size;
  return (int)std::min<int64_t>(v, INT32_MAX / 2);
}

// Compute units of the current device (256 when no device is visible: sizing only).
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Per-sequence query and past lengths from host metadata (pa_paged_attention's host_* inputs),
// when the caller gave them: they size the LATENT kernel's context chunks.
struct HostLens {
  const int32_t* cum = nullptr;
  const int32_t* past = nullptr;
};

#ifndef PA_LATENT_PLAN
#define PA_LATENT_PLAN 1
#endif
// Price of a partial-row byte against a key byte in latent_chunk: the merge streams its rows
// slower than the kernel streams keys (MLA decode at 16 heads, config 3 contexts: weight 1
// 142.2 us per step, 2 137.8 us, 3 137.4 us).
#ifndef PA_LATENT_MERGE_W
#define PA_LATENT_MERGE_W 3.0
#endif
// Resident workgroups assumed by latent_chunk, in multiples of the real count: the estimate
// leaves out each workgroup's fixed cost (query load, first steps' latency, partial rows), and
// a doubled count picks the chunk that measured best (MLA decode at 16 heads, config 3
// contexts, step: x1 (chunk 640) 135.8 us, x2 (480) 124.9 us, x3 (416) 139.9 us, x4 (352)
// 152.6 us; 128 heads unchanged at the 992-key cap).
#ifndef PA_LATENT_SLOTS_X
#define PA_LATENT_SLOTS_X 2.0
#endif
#ifndef PA_LATENT_ODD_SPLITS
#define PA_LATENT_ODD_SPLITS 1
#endif
constexpr int kLatPlanMaxBatch = 4096;  // batches beyond this keep the capacity rule (host cost)

// LATENT kernel: the context chunk (a multiple of 32 keys in [256, cap]) that minimises the
// estimated launch time for the host's per-sequence key counts, in units of one 32-key step of a
// workgroup: the work of all workgroups spread over `slots` resident ones, plus half a
// workgroup's length for the last dispatch round, plus the partial rows of split sequences (fp32
// O, m, l written by the kernel and read by the merge) priced as PA_LATENT_MERGE_W key bytes.
int latent_chunk(const pa_cache* c, const pa_batch* b, const pa_attn* a, const HostLens& hl,
                 int ng, int64_t slots, int cap) {
  const int D = c->head_dim;
  const int64_t H = a->num_heads;
  double best = 0.0;
  int pick = 0;
  for (int ch = 256; ch <= cap; ch += 32) {
    int64_t work = 0, part_rows = 0;
    for (int i = 0; i < b->batch; ++i) {
      const int64_t nq = (int64_t)hl.cum[i + 1] - hl.cum[i];
      if (nq <= 0) continue;
      const int64_t tot = std::max<int64_t>((int64_t)std::max(hl.past[i], 0) + nq, 1);
      const int64_t rbs = (H * nq + 16 * ng - 1) / (16 * ng);
      const int64_t n = (tot + ch - 1) / ch;
      work += rbs * ((tot + 31) / 32 + n);  // steps + one step of set-up per workgroup
      if (n > 1) part_rows += n * H * nq;
    }
    const double merge =
        PA_LATENT_MERGE_W * (double)part_rows * (D * 4 + 8) * 2 / ((double)slots * 32 * D * 2);
    const double est = (double)work / (double)slots + (ch / 32 + 1) * 0.5 + merge;
    if (pick == 0 || est < best) {
      best = est;
      pick = ch;
    }
  }
  return pick;
}

// images: the planned head-128 prefill may use operand images (off where the workspace is
// bounded, pa_paged_attention_static).  bias: GroupQueryAttention's attention bias is present
// (its streaming decode runs one wavefront per SIMD at every cache dtype).
Plan make_plan(const pa_cache* c, const pa_batch* b, const pa_attn* a, pa_dtype act, int kind,
               int chunk, bool linear = false, int linear_cap = 0, bool images = true,
               bool bias = false, const HostLens& hl = HostLens()) {
  Plan pl{};
  // The LATENT layout (values = leading dims of the key rows): its matrix-core kernel (kind 5)
  // where it covers the head sizes and dtypes, else the VALU kernel.
  if (c->value_cache == nullptr || (a->v_head_size > 0 && a->v_head_size != c->head_dim)) {
    const int vd = a->v_head_size > 0 ? a->v_head_size : c->head_dim;
    kind = (kind == 0 && c->kv_heads == 1 &&
            pa::latent_mfma_supported(c->head_dim, vd, act, c->dtype))
               ? 5
               : 3;
  }
  const int g = a->num_heads / c->kv_heads;
  const int mq = b->max_query_len > 0 ? b->max_query_len : std::max(b->num_tokens, 1);
  const bool mfma = pa::decode_mfma_supported(c->head_dim, act, c->dtype);
  // The balanced (streaming) decode addresses rows with 32-bit row indices and shifts, and
  // numbers the 32-key steps of the whole batch with 32-bit indices: every sequence is clamped
  // to the cache capacity on the device, so batch * (capacity / 32 + 1) bounds the step count.
  const int64_t cap = linear_cap > 0 ? linear_cap : (int64_t)b->max_blocks * c->block_size;
  // (contiguous caches: in the activation dtype or integer codes)
  const bool bal_ok = (int64_t)g * mq <= 16 &&
                      pa::balanced_supported(c->head_dim, act, c->dtype, c->block_size) &&
                      !(linear && c->dtype != act && !is_int_cache(c->dtype)) &&
                      (int64_t)c->num_blocks * c->block_size <= (int64_t)UINT32_MAX &&
                      (int64_t)std::max(b->batch, 0) * (cap / 32 + 2) < (int64_t)INT32_MAX;
  // Byte-coded pages (int8 / int4 codes, fp8 e4m3 paged): multi-token batches on the planned
  // prefill over operand images of the pages when the images may be used and fit (else the VALU
  // kernel).
  const bool intc = PA_PREFILL_IMAGES && images &&
                    pa::prefill_coded_supported(c->head_dim, act, c->dtype) &&
                    !(linear && c->dtype == PA_DTYPE_FP8_E4M3);
  // Contiguous caches: the streaming decode, the LDS-shared prefill kernels, or VALU.
  if (kind == 0 && linear)
    kind = bal_ok ? 1 : (pa::prefill_mfma_supported(c->head_dim, act, c->dtype) || intc) ? 2 : 3;
  if (kind == 0) {
    if (bal_ok || (mfma && (int64_t)g * mq <= 16))
      kind = 1;
    else if (pa::prefill_mfma_supported(c->head_dim, act, c->dtype))
      kind = 2;
    else if (mfma)
      kind = 1;
    else if (intc)
      kind = 2;
    else
      kind = 3;
  }
  // byte-coded pages run the prefill kernel only over images, i.e. the planned launch
  if (kind == 2 && pa::prefill_coded_supported(c->head_dim, act, c->dtype) && (!intc || chunk > 0))
    kind = 3;
  pl.kind = kind;
  pl.balanced = kind == 1 && bal_ok;
  if (kind == 4) pl.kind = 1;
  // Longest context a sequence can have: the contiguous capacity, or the block table's.
  const int ctx = std::max(
      linear_cap > 0 ? std::min(linear_cap, INT32_MAX / 2) : max_ctx_bound(c, b), 1);
  if (pl.balanced) {
    // decode_waves wavefronts per SIMD on every CU, each walking kDecodeMix sub-segments.
    pl.chunk = 32;
    pl.mix = std::min(kDecodeMix, c->kv_heads);
    const int waves = bias ? 1 : pa::decode_waves(c->dtype, c->head_dim);
    pl.max_splits = pl.mix * std::max(1, 4 * waves * device_cus() / c->kv_heads);
    pl.part_rows = (size_t)(pl.max_splits + b->batch) * c->kv_heads * 16;
    return pl;
  }
  // Chunked MFMA kernel: several 16-row groups per wavefront once a sequence has >= 64 grouped
  // query rows (prefill chunks), so each loaded key/value step serves more rows (4 groups at
  // d=64, 2 at d=128: what fits the register file).
  pl.ng = (pl.kind == 1 && (int64_t)g * mq >= 64) ? (c->head_dim == 64 ? 4 : 2) : 1;
  if (chunk <= 0 && kind == 2) {
    // Prefill workgroups (4 wavefronts, pa::kPrefillRows grouped query rows each): split the
    // context only when they cannot fill two workgroups per CU.
    const int64_t rbs = ((int64_t)g * mq + pa::kPrefillRows - 1) / pa::kPrefillRows;
    const int64_t units = (int64_t)b->batch * c->kv_heads * rbs;
    const int64_t target = 2 * (int64_t)device_cus();
    if ((units >= target || intc) && units <= (int64_t)INT32_MAX / 4 &&
        pa::prefill_planned_supported(c->head_dim)) {
      // Enough workgroups for every slot: planned units, longest first, long items split in two
      // (the tail of uneven row blocks otherwise idles ~28% of the slots at the C4 shape).
      pl.chunk = (int)std::min<int64_t>(((int64_t)ctx + 31) / 32 * 32, INT32_MAX / 2);
      pl.max_splits = 1;
      pl.plan_items = units;
      pl.plan_rbs = (int)rbs;
      pl.part_rows = (size_t)units * 2 * pa::kPrefillRows;
      if (PA_PREFILL_IMAGES && images && pa::img_head(c->head_dim) &&
          (rbs >= kImgMinRowBlocks || intc)) {
        // images of the live context: the caller's bound on past + new tokens, else the capacity
        const int ik = pa::img_keys(c->head_dim);
        const int64_t live =
            b->max_context_len > 0 ? std::min<int64_t>(b->max_context_len, ctx) : (int64_t)ctx;
        const int64_t steps = (live + ik - 1) / ik;
        const int64_t per_seq = (int64_t)c->kv_heads * steps * pa::img_step_bytes(c->head_dim);
        if ((int64_t)b->batch * per_seq <= kImgMaxBytes && steps <= 65535 &&
            b->batch <= 65535) {
          pl.img_steps = (int)steps;
        } else if (intc && !linear && per_seq <= kImgMaxBytes && steps <= 65535) {
          // byte-coded pages: groups of sequences whose images fit, one planned launch each
          pl.sub_batch = (int)std::min<int64_t>(kImgMaxBytes / per_seq, 65535);
          pl.img_steps = (int)steps;
          const int64_t sub_units = (int64_t)pl.sub_batch * c->kv_heads * rbs;
          pl.plan_items = sub_units;
          pl.part_rows = (size_t)sub_units * 2 * pa::kPrefillRows;
        }
      }
      if (!(intc && pl.img_steps == 0)) return pl;
      pl = Plan{};  // byte-coded pages whose images do not fit: see below
      pl.kind = 2;
    } else if (units >= target) {
      chunk = (int)std::min<int64_t>(((int64_t)ctx + 31) / 32 * 32, INT32_MAX / 2);
    } else {
      const int64_t splits = (target + units - 1) / units;
      int64_t ch = (ctx + splits - 1) / splits;
      const int64_t step = pa::prefill_key_step(c->head_dim);
      chunk = (int)std::min<int64_t>(std::max<int64_t>((ch + step - 1) / step * step, 256),
                                     INT32_MAX / 2);
    }
  }
  // Byte-coded pages that did not get the planned launch over images: the VALU kernel.
  if (pl.kind == 2 && pa::prefill_coded_supported(c->head_dim, act, c->dtype)) {
    kind = 3;
    pl.kind = 3;
    pl.ng = 1;
  }
  if (chunk <= 0) {
    // Work units without split-K: (sequence, kv-head, row groups) for the MFMA kernel,
    // (token, head) for the VALU kernel.  Split the context only when they cannot fill the
    // GPU (~2048 one-per-SIMD wavefronts for NG = 4, ~4096 otherwise).
    const int64_t rows_pw = 16 * pl.ng;
    // LATENT kernel: workgroups of 4 wavefronts per 16 grouped rows, one or two per CU
    const int64_t units =
        pl.kind == 1   ? (int64_t)b->batch * c->kv_heads * (((int64_t)g * mq + rows_pw - 1) / rows_pw)
        : pl.kind == 5 ? (int64_t)b->batch * (((int64_t)g * mq + 16 * pa::latent_row_groups(g, mq) - 1) /
                                             (16 * pa::latent_row_groups(g, mq)))
                       : (int64_t)std::max(b->num_tokens, 1) * a->num_heads;
    const int64_t target =
        pl.kind == 5 ? PA_LATENT_TARGET * (int64_t)device_cus() : pl.ng > 1 ? 2048 : 4096;
    if (pl.kind == 5 && PA_LATENT_PLAN && hl.cum && hl.past && b->batch <= kLatPlanMaxBatch &&
        c->block_size >= 16) {
      // workgroups resident per CU: two at 128 value dims with one row group, else one
      const int vd = a->v_head_size > 0 ? a->v_head_size : c->head_dim;
      const int ng = pa::latent_row_groups(g, mq);
      const int64_t slots =
          (int64_t)(PA_LATENT_SLOTS_X * (vd <= 128 && ng == 1 ? 2 : 1) * device_cus());
      chunk = latent_chunk(c, b, a, hl, ng, slots,
                           std::max(256, 63 * c->block_size / 32 * 32));
    } else if (units >= target) {
      chunk = (int)std::min<int64_t>(((int64_t)ctx + 31) / 32 * 32, INT32_MAX / 2);
    } else {
      const int64_t splits = (target + units - 1) / units;
      int64_t ch = (ctx + splits - 1) / splits;
      ch = ((ch + 31) / 32) * 32;
      chunk = (int)std::min<int64_t>(std::max<int64_t>(ch, 256), 1024);
    }
  }
  chunk = std::max(32, chunk / 32 * 32);
  // the LATENT kernel holds one window of 64 page ids per chunk
  if (pl.kind == 5 && c->block_size >= 16)
    chunk = std::min(chunk, std::max(32, 63 * c->block_size / 32 * 32));
  pl.chunk = chunk;
  pl.max_splits = (int)std::max<int64_t>(1, ((int64_t)ctx + chunk - 1) / chunk);
  // LATENT grid (row blocks, splits, sequences): workgroups go to the 8 XCDs round-robin by
  // linear id, so with an even split count the same splits of every sequence land on the same
  // XCDs (the early splits, which every sequence has, piling onto some of them).  An odd count
  // (the extra workgroups exit at once) cycles each split over all XCDs: 16-head MLA decode over
  // the config 3 contexts at 512-key chunks (16 splits) 160.3 -> 128.6 us per step.
  if (pl.kind == 5 && PA_LATENT_ODD_SPLITS && pl.max_splits > 1 && pl.max_splits % 2 == 0 &&
      pl.max_splits < 65535)
    ++pl.max_splits;
  pl.part_rows = pl.max_splits > 1
                     ? (size_t)std::max(b->num_tokens, 0) * a->num_heads * pl.max_splits
                     : 0;
  return pl;
}

// Bytes of the partial rows: fp32 elements, except the planned prefill's halves, which are
// stored as fp16 rows scaled by a power of two (store_rows with half_part).
size_t part_o_bytes(const pa_cache* c, const Plan& pl) {
  const size_t es = pl.plan_items > 0 ? 2 : sizeof(float);
  return align256(pl.part_rows * c->head_dim * es);
}

// Workspace: [partial O | partial (m, l)].
// Planned prefill adds [unit list (2 per item, 4 int32 each) | unit count | split flag per item].
// Operand images add [images | step value exponents].
size_t plan_bytes(const Plan& pl) {
  return align256((size_t)pl.plan_items * 2 * 4 * sizeof(int32_t)) + 256 +
         align256((size_t)pl.plan_items * sizeof(int32_t));
}
size_t image_bytes(const pa_cache* c, const pa_batch* b, const Plan& pl) {
  if (pl.img_steps == 0) return 0;
  const size_t hb = (size_t)plan_batch(b, pl) * c->kv_heads;
  return align256(hb * pl.img_steps * pa::img_step_bytes(c->head_dim)) +
         align256(hb * pl.img_steps * sizeof(int32_t)) + align256(hb * sizeof(int32_t));
}

// Per-call number of the image writer's wide-step flags (AttnParams::img_wide): never 0, so a
// zeroed flag array reads as "no wide step".
int32_t next_img_epoch() {
  static std::atomic<uint32_t> epoch{0};
  uint32_t e = epoch.fetch_add(1, std::memory_order_relaxed) + 1;
  if ((e & 0x7fffffffu) == 0) e = epoch.fetch_add(1, std::memory_order_relaxed) + 1;
  return (int32_t)(e & 0x7fffffffu);
}
size_t workspace_for(const pa_cache* c, const pa_batch* b, const pa_attn*, const Plan& pl) {
  if (pl.part_rows == 0) return 0;
  size_t n = part_o_bytes(c, pl) + align256(pl.part_rows * 2 * sizeof(float));
  if (pl.plan_items > 0) n += plan_bytes(pl) + image_bytes(c, b, pl);
  return n;
}

// Options of one attention call beyond the public descriptors.
struct RunOpts {
  bool new_rows_in_cache = false;  // new rows sit in their block-table slots (see AttnParams)
  int linear_cap = 0;              // contiguous [batch, kv_heads, cap, d] caches (GQA present)
  // GroupQueryAttention forms (see AttnParams): per-sequence key counts, additive bias, zero sink
  const int32_t* key_limit = nullptr;
  const void* bias = nullptr;
  int bias_b = 0, bias_h = 0, bias_rows = 0, bias_cols = 0;
  const int32_t* bias_col_off = nullptr;  // per-sequence bias column offsets (sliding rings)
  bool smooth_softmax = false;
  bool images = true;  // operand images allowed (see make_plan)
  HostLens host;       // host metadata lengths (LATENT chunk sizing)
};

// Operand images for a call with these options: not with a bias (the matrix-core kernels that
// take one -- the streaming decode and prefill_kernel -- read the cache rows themselves), so
// byte-coded multi-token batches with a bias run on the VALU kernel.
bool plan_images(const RunOpts& o) { return o.images && o.bias == nullptr; }

int run_attention(const pa_cache* c, const pa_batch* b, const pa_attn* a, pa_dtype act,
                  const void* q, const void* kn, const void* vn, void* out, void* ws,
                  size_t ws_bytes, int kind, int chunk, hipStream_t s, RunOpts opts = RunOpts()) {
  int rc = check_cache(c, act);
  if (rc) return rc;
  if ((rc = check_batch(b))) return rc;
  if (!a) return fail(PA_ERR_INVALID_ARGUMENT, "attention descriptor is NULL");
  if (a->num_heads <= 0 || a->num_heads % c->kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "PagedAttention: bad num_heads/kv_num_heads");
  if (b->num_tokens == 0) return PA_OK;
  // Quantised caches (fp8, int8, int4) read every position from the pages.
  const bool quant = c->dtype == PA_DTYPE_FP8_E4M3 || is_int_cache(c->dtype);
  const bool latent = c->value_cache == nullptr;
  const int vd = a->v_head_size > 0 ? a->v_head_size : c->head_dim;
  if (!latent && vd != c->head_dim)
    return fail(PA_ERR_INVALID_ARGUMENT, "SEPARATE layout requires equal key and value head sizes");
  if (vd > c->head_dim)
    return fail(PA_ERR_INVALID_ARGUMENT, "LATENT v_head_size must not exceed head_size");
  if (!q || !out || (!quant && (!kn || (!vn && !latent))))
    return fail(PA_ERR_INVALID_ARGUMENT, "q/k_new/v_new/out pointers are NULL");
  if (kind < 0 || kind > 4) return fail(PA_ERR_INVALID_ARGUMENT, "unknown kernel kind %d", kind);
  if (latent && kind != 0 && kind != 3)
    return fail(PA_ERR_UNSUPPORTED,
                "the LATENT layout runs on its matrix-core kernel (automatic choice) or the VALU "
                "kernel only");
  if (kind == 4 && !pa::decode_mfma_supported(c->head_dim, act, c->dtype))
    return fail(PA_ERR_UNSUPPORTED, "decode MFMA kernel does not cover this dtype/head_dim");
  if (kind == 1 && !pa::decode_mfma_supported(c->head_dim, act, c->dtype)) {
    const int g = a->num_heads / c->kv_heads;
    const int mq = b->max_query_len > 0 ? b->max_query_len : std::max(b->num_tokens, 1);
    if (!((int64_t)g * mq <= 16 &&
          pa::balanced_supported(c->head_dim, act, c->dtype, c->block_size)))
      return fail(PA_ERR_UNSUPPORTED, "decode MFMA kernel does not cover this dtype/head_dim");
  }
  if (kind == 2 && !pa::prefill_mfma_supported(c->head_dim, act, c->dtype) &&
      !pa::prefill_coded_supported(c->head_dim, act, c->dtype))
    return fail(PA_ERR_UNSUPPORTED, "prefill MFMA kernel does not cover this dtype/head_dim");
  if (!(a->softcap >= 0.0f) || !std::isfinite(a->softcap))
    return fail(PA_ERR_INVALID_ARGUMENT, "softcap must be finite and non-negative");
  Plan pl = make_plan(c, b, a, act, kind, chunk, opts.linear_cap > 0, opts.linear_cap,
                      plan_images(opts), opts.bias != nullptr, opts.host);
  if (kind == 2 && pl.kind != 2 && pa::prefill_coded_supported(c->head_dim, act, c->dtype))
    return fail(PA_ERR_UNSUPPORTED,
                "prefill MFMA kernel: byte-coded pages run on it over operand images only (planned "
                "launch, automatic chunking, images within the workspace)");
  if (opts.linear_cap > 0 && !(pl.balanced || pl.kind == 2 || pl.kind == 3))
    return fail(PA_ERR_UNSUPPORTED,
                "contiguous caches run on the streaming decode, prefill or VALU kernels only");
  size_t need = workspace_for(c, b, a, pl);
  if (need > 0 && (!ws || ws_bytes < need))
    return fail(PA_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes, got %zu", need,
                ws_bytes);

  pa::AttnParams p{};
  p.q = q;
  p.k_new = kn;
  p.v_new = vn;
  p.key_cache = c->key_cache;
  p.value_cache = c->value_cache;
  p.k_scale = c->k_scale;
  p.v_scale = c->v_scale;
  p.cum = b->cumulative_sequence_length;
  p.past = b->past_seqlens;
  p.block_table = b->block_table;
  p.head_sink = a->head_sink;
  p.out = out;
  p.part_o = need ? reinterpret_cast<float*>(ws) : nullptr;
  p.part_ml = need ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + part_o_bytes(c, pl))
                   : nullptr;
  if (pl.plan_items > 0) {
    char* base = reinterpret_cast<char*>(ws) + part_o_bytes(c, pl) +
                 align256(pl.part_rows * 2 * sizeof(float));
    p.plan = reinterpret_cast<int32_t*>(base);
    base += align256((size_t)pl.plan_items * 2 * 4 * sizeof(int32_t));
    p.plan_info = reinterpret_cast<int32_t*>(base);
    p.plan_split = reinterpret_cast<int32_t*>(base + 256);
    p.plan_items = (int32_t)pl.plan_items;
    p.plan_rbs = pl.plan_rbs;
    // workgroups resident per CU: two, three for the 32-key image kernel (148 VGPRs, 33 KB LDS),
    // one for the bias kernel from head 128 on
    p.plan_slots = (pl.img_steps > 0 && pa::img_keys(c->head_dim) == 32 && c->head_dim <= 128
                        ? PA_IMG_WAVES
                    : opts.bias && c->head_dim >= 128 ? 1
                                                      : 2) * device_cus();
    p.plan_step = pl.img_steps > 0 ? pa::img_keys(c->head_dim) : pa::prefill_key_step(c->head_dim);
    if (pl.img_steps > 0) {
      const size_t hb = (size_t)plan_batch(b, pl) * c->kv_heads;
      char* img = base + plan_bytes(pl) - align256((size_t)pl.plan_items * 2 * 4 * sizeof(int32_t));
      p.vimg = img;
      img += align256(hb * pl.img_steps * pa::img_step_bytes(c->head_dim));
      p.vstep = reinterpret_cast<int32_t*>(img);
      img += align256(hb * pl.img_steps * sizeof(int32_t));
      p.img_wide = reinterpret_cast<int32_t*>(img);
      p.img_epoch = next_img_epoch();
      p.img_steps = pl.img_steps;
    }
  }
  p.num_blocks = c->num_blocks;
  p.block_size = c->block_size;
  p.kv_heads = c->kv_heads;
  p.head_dim = c->head_dim;
  p.num_heads = a->num_heads;
  p.batch = b->batch;
  p.max_blocks = b->max_blocks;
  p.num_tokens = b->num_tokens;
  p.chunk = pl.chunk;
  p.max_splits = pl.max_splits;
  p.mix = pl.mix;
  p.linear_cap = opts.linear_cap;
  p.ng = pl.ng > 0 ? pl.ng : 1;
  p.max_query_len = b->max_query_len > 0 ? b->max_query_len : b->num_tokens;
  p.scale = a->scale != 0.0f ? a->scale : 1.0f / std::sqrt((float)c->head_dim);
  p.scale_log2 = p.scale * pa::kLog2e;
  p.softcap = a->softcap;
  p.window = a->local_window_size;
  p.causal = a->is_causal ? 1 : 0;
  p.read_all_from_cache = quant ? 1 : 0;
  p.k_quant = c->k_quant_type;
  p.v_quant = c->v_quant_type;
  p.v_head_dim = vd;
  p.v_from_key = latent ? 1 : 0;
  p.new_rows_in_cache =
      (opts.new_rows_in_cache || ((b->flags & PA_BATCH_NEW_ROWS_IN_CACHE) && !b->slot_mapping))
          ? 1
          : 0;
  p.key_limit = opts.key_limit;
  p.bias = opts.bias;
  p.bias_b = opts.bias_b;
  p.bias_h = opts.bias_h;
  p.bias_rows = opts.bias_rows;
  p.bias_cols = opts.bias_cols;
  p.bias_col_off = opts.bias_col_off;
  p.smooth_softmax = opts.smooth_softmax ? 1 : 0;

  hipError_t e;
  if (pl.balanced) {
    e = pa::launch_decode_balanced(p, act, c->dtype, s);  // attention + partial merge
    if (e != hipSuccess) return hip_fail(e, "balanced decode launch");
    return PA_OK;
  }
  switch (pl.kind) {
    case 1: e = pa::launch_decode_mfma(p, act, c->dtype, s); break;
    case 2:
      if (pl.sub_batch > 0) {
        // groups of sequences in turn over the same workspace (cum holds absolute token
        // offsets, so q / k / v / out stay as they are)
        e = hipSuccess;
        for (int64_t b0 = 0; b0 < b->batch && e == hipSuccess; b0 += pl.sub_batch) {
          pa::AttnParams q = p;
          const int nb = (int)std::min<int64_t>(pl.sub_batch, b->batch - b0);
          q.cum = p.cum + b0;
          q.past = p.past + b0;
          q.block_table = p.block_table + b0 * p.max_blocks;
          q.batch = nb;
          q.plan_items = (int32_t)((int64_t)nb * c->kv_heads * pl.plan_rbs);
          if (p.key_limit) q.key_limit = p.key_limit + b0;
          // fresh wide-step flags: the image slots are reused by every group
          if (b0 > 0) q.img_epoch = next_img_epoch();
          e = pa::launch_prefill_planned(q, act, c->dtype, s);
        }
      } else {
        e = pl.plan_items > 0 ? pa::launch_prefill_planned(p, act, c->dtype, s)
                              : pa::launch_prefill_mfma(p, act, c->dtype, s);
      }
      break;
    case 5: e = pa::launch_latent(p, act, c->dtype, s); break;
    default: e = pa::launch_attn_generic(p, act, c->dtype, s); break;
  }
  if (e != hipSuccess) return hip_fail(e, "attention kernel launch");
  if (pl.max_splits > 1) {
    e = pa::launch_split_reduce(p, act, s);
    if (e != hipSuccess) return hip_fail(e, "split-K reduce launch");
  }
  return PA_OK;
}

}  // namespace

// ============================================================================== C ABI
extern "C" {

const char* pa_last_error(void) { return g_last_error.c_str(); }

const char* pa_version(void) { return "onnxruntime-ep-mlx_amd 0.1.0 (gfx950)"; }

// ------------------------------------------------------------------------------ page pool
struct pa_pool {
  void* k;
  void* v;
  float* ks;
  float* vs;
  int64_t bytes;
};

int pa_pool_create(int64_t num_blocks, int32_t block_size, int32_t kv_heads, int32_t head_dim,
                   pa_dtype cache_dtype, pa_pool** out_pool) {
  if (!out_pool) return fail(PA_ERR_INVALID_ARGUMENT, "out_pool is NULL");
  *out_pool = nullptr;
  const size_t hb = head_dim > 0 ? cache_head_bytes(cache_dtype, head_dim) : 0;
  if (num_blocks <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0 || hb == 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "invalid pool geometry");
  // Integer pools hold codes only: their per-tensor / per-channel scales are operator inputs.
  size_t side = (size_t)num_blocks * block_size * kv_heads * hb;
  pa_pool* p = new pa_pool{};
  hipError_t e = hipMalloc(&p->k, side);
  if (e == hipSuccess) e = hipMalloc(&p->v, side);
  if (e == hipSuccess && cache_dtype == PA_DTYPE_FP8_E4M3) {
    size_t sb = (size_t)num_blocks * kv_heads * sizeof(float);
    e = hipMalloc(&p->ks, sb);
    if (e == hipSuccess) e = hipMalloc(&p->vs, sb);
  }
  if (e != hipSuccess) {
    (void)hipFree(p->k);
    (void)hipFree(p->v);
    (void)hipFree(p->ks);
    (void)hipFree(p->vs);
    delete p;
    return fail(PA_ERR_OUT_OF_MEMORY, "pool allocation of 2 x %zu bytes failed: %s", side,
                hipGetErrorString(e));
  }
  p->bytes = (int64_t)(2 * side);
  *out_pool = p;
  return PA_OK;
}

int pa_pool_destroy(pa_pool* p) {
  if (!p) return PA_OK;
  (void)hipFree(p->k);
  (void)hipFree(p->v);
  (void)hipFree(p->ks);
  (void)hipFree(p->vs);
  delete p;
  return PA_OK;
}

void* pa_pool_k_ptr(const pa_pool* p) { return p ? p->k : nullptr; }
void* pa_pool_v_ptr(const pa_pool* p) { return p ? p->v : nullptr; }
float* pa_pool_k_scale_ptr(const pa_pool* p) { return p ? p->ks : nullptr; }
float* pa_pool_v_scale_ptr(const pa_pool* p) { return p ? p->vs : nullptr; }
int64_t pa_pool_bytes(const pa_pool* p) { return p ? p->bytes : 0; }

// ------------------------------------------------------------------------------ append
// Operator-level append options beyond the kernel-level entry: contiguous (GroupQueryAttention)
// caches, packed-QKV input strides with contiguous copies of the rows, and the integer encode
// rule (see AppendParams).
struct AppendExtra {
  int linear_cap = 0, seq = 0;
  bool kv_rows = true;  // GroupQueryAttention: the call has new key/value rows
  const int32_t* seqlens_k = nullptr;
  int32_t* meta_out = nullptr;
  int64_t q_ld = 0, k_ld = 0, v_ld = 0;  // 0: contiguous rows
  void* v_out = nullptr;
  bool copy_rows = false;
  bool quant_reciprocal = false;
  const int64_t* position_ids = nullptr;
  bool pos_offset_form = false;
  bool rope_fp32 = false;
  int ring_cap = 0, ring_window = 0;  // sliding_window_cache rings (see AppendParams)
};

static int rotary_append_impl(const pa_cache* c, const pa_batch* b, int32_t num_heads,
                              pa_dtype act, const void* query, const void* key,
                              const void* value, void* q_out, void* k_out, const void* cos,
                              const void* sin, int64_t rot_pos, int32_t rot_half,
                              int32_t rot_offset, int32_t interleaved, const void* qn,
                              const void* kn, float eps, hipStream_t s,
                              const AppendExtra& x = AppendExtra()) {
  int rc = check_cache(c, act);
  if (rc) return rc;
  if ((rc = check_batch(b))) return rc;
  if (b->num_tokens == 0) return PA_OK;
  if (x.kv_rows && (!key || (!value && c->value_cache)))
    return fail(PA_ERR_INVALID_ARGUMENT, "key/value pointers are NULL");
  const bool rotate = cos != nullptr;
  if (rotate) {
    if (!sin || rot_half <= 0 || rot_offset < 0 || rot_offset + 2 * rot_half > c->head_dim ||
        rot_pos <= 0)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "rotary_offset + rotary_dim must not exceed head_size");
  }
  if ((qn == nullptr) != (kn == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "q_norm_weight and k_norm_weight must be provided together");
  const bool transform = rotate || qn || x.copy_rows;
  if (transform && num_heads > 0 && query && !q_out)
    return fail(PA_ERR_INVALID_ARGUMENT, "q_out is required when rotating/normalising query");
  pa::AppendParams p{};
  p.query = query;
  p.key = key;
  p.value = value;
  p.q_out = q_out;
  p.k_out = k_out;
  p.key_cache = c->key_cache;
  p.value_cache = c->value_cache;
  p.k_scale = c->k_scale;
  p.v_scale = c->v_scale;
  p.cos_cache = cos;
  p.sin_cache = sin;
  p.q_norm = qn;
  p.k_norm = kn;
  p.cum = b->cumulative_sequence_length;
  p.past = b->past_seqlens;
  p.block_table = b->block_table;
  p.slot_mapping = b->slot_mapping;
  p.num_blocks = c->num_blocks;
  p.rotary_positions = rot_pos;
  p.block_size = c->block_size;
  p.kv_heads = c->kv_heads;
  p.head_dim = c->head_dim;
  p.num_heads = num_heads;
  p.batch = b->batch;
  p.max_blocks = b->max_blocks;
  p.num_tokens = b->num_tokens;
  p.rotary_half = rotate ? rot_half : 0;
  p.rotary_offset = rotate ? rot_offset : 0;
  p.rotary_interleaved = interleaved ? 1 : 0;
  p.do_q = (query && q_out && num_heads > 0) ? 1 : 0;
  p.norm_eps = eps;
  p.slots_distinct = (b->flags & PA_BATCH_SLOTS_DISTINCT) ? 1 : 0;
  p.linear_cap = x.linear_cap;
  p.gqa_seq = x.seq;
  p.gqa_kv_rows = x.kv_rows ? 1 : 0;
  p.position_ids = x.position_ids;
  p.pos_offset_form = x.pos_offset_form ? 1 : 0;
  p.rope_fp32 = x.rope_fp32 ? 1 : 0;
  p.ring_cap = x.ring_cap;
  p.ring_window = x.ring_window;
  p.seqlens_k = x.seqlens_k;
  p.meta_out = x.meta_out;
  p.q_ld = x.q_ld ? x.q_ld : (int64_t)num_heads * c->head_dim;
  p.k_ld = x.k_ld ? x.k_ld : (int64_t)c->kv_heads * c->head_dim;
  p.v_ld = x.v_ld ? x.v_ld : (int64_t)c->kv_heads * c->head_dim;
  p.v_out = x.v_out;
  p.copy_rows = x.copy_rows ? 1 : 0;
  p.k_quant = c->k_quant_type;
  p.v_quant = c->v_quant_type;
  p.quant_reciprocal = x.quant_reciprocal ? 1 : 0;
  hipError_t e = pa::launch_rotary_append(p, act, c->dtype, s);
  if (e != hipSuccess) return hip_fail(e, "rotary/append kernel launch");
  return PA_OK;
}

int pa_rotary_append(const pa_cache* cache, const pa_batch* batch, int32_t num_heads,
                     pa_dtype act_dtype, const void* query, const void* key, const void* value,
                     void* q_out, void* k_out, const void* cos_cache, const void* sin_cache,
                     int64_t rotary_positions, int32_t rotary_half, int32_t rotary_offset,
                     int32_t rotary_interleaved, const void* q_norm, const void* k_norm,
                     float norm_eps, pa_stream_t stream) {
  return rotary_append_impl(cache, batch, num_heads, act_dtype, query, key, value, q_out, k_out,
                            cos_cache, sin_cache, rotary_positions, rotary_half, rotary_offset,
                            rotary_interleaved, q_norm, k_norm, norm_eps,
                            reinterpret_cast<hipStream_t>(stream));
}

int pa_reshape_and_cache(const pa_cache* cache, const pa_batch* batch, pa_dtype act_dtype,
                         const void* key, const void* value, pa_stream_t stream) {
  return rotary_append_impl(cache, batch, 0, act_dtype, nullptr, key, value, nullptr, nullptr,
                            nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 0.0f,
                            reinterpret_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------------------ attention
size_t pa_attention_workspace_bytes(const pa_cache* cache, const pa_batch* batch,
                                    const pa_attn* attn) {
  if (!cache || !batch || !attn || cache->kv_heads <= 0 || batch->batch <= 0) return 0;
  // Quantised storage does not name the activation dtype; the plan only needs a 16-bit one.
  pa_dtype act = (cache->dtype == PA_DTYPE_FP8_E4M3 || is_int_cache(cache->dtype))
                     ? PA_DTYPE_BFLOAT16
                     : cache->dtype;
  return workspace_for(cache, batch, attn, make_plan(cache, batch, attn, act, 0, 0));
}

size_t pa_attention_workspace_bytes_ex(const pa_cache* cache, const pa_batch* batch,
                                       const pa_attn* attn, pa_dtype act_dtype, int32_t kind,
                                       int32_t chunk_tokens) {
  if (!cache || !batch || !attn || cache->kv_heads <= 0 || batch->batch <= 0) return 0;
  return workspace_for(cache, batch, attn,
                       make_plan(cache, batch, attn, act_dtype, kind, chunk_tokens));
}

int pa_attention(const pa_cache* cache, const pa_batch* batch, const pa_attn* attn,
                 pa_dtype act_dtype, const void* q, const void* k_new, const void* v_new,
                 void* out, void* workspace, size_t workspace_bytes, pa_stream_t stream) {
  return run_attention(cache, batch, attn, act_dtype, q, k_new, v_new, out, workspace,
                       workspace_bytes, 0, 0, reinterpret_cast<hipStream_t>(stream));
}

int pa_attention_ex(const pa_cache* cache, const pa_batch* batch, const pa_attn* attn,
                    pa_dtype act_dtype, const void* q, const void* k_new, const void* v_new,
                    void* out, void* workspace, size_t workspace_bytes, int32_t kind,
                    int32_t chunk_tokens, pa_stream_t stream) {
  return run_attention(cache, batch, attn, act_dtype, q, k_new, v_new, out, workspace,
                       workspace_bytes, kind, chunk_tokens, reinterpret_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------------------ operator level
namespace {

struct OpLayout {
  int head, v_head, kv_hidden;
  bool packed, transform;
  size_t q_bytes, k_bytes, v_bytes, attn_off, total;
  pa_batch batch;
  pa_attn attn;
};

int op_layout(const pa_paged_attention_node* n, const pa_paged_attention_io* io, OpLayout* L,
              bool images = true) {
  if (!n || !io) return fail(PA_ERR_INVALID_ARGUMENT, "node/io is NULL");
  if (n->num_heads <= 0 || n->kv_num_heads <= 0 || n->num_heads % n->kv_num_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "PagedAttention: bad num_heads/kv_num_heads");
  // attention.rs:4434: key and value absent together = packed [T, (H + 2 KV) * head] query.
  const bool latent = n->kv_cache_layout_latent != 0;
  L->packed = !latent && io->key == nullptr && io->value == nullptr;
  if (latent) {
    // attention.rs:4452-4481: one kv-head, value and value_cache absent.
    if (n->kv_num_heads != 1)
      return fail(PA_ERR_INVALID_ARGUMENT, "PagedAttention: LATENT layout requires kv_num_heads=1");
    if (!io->key || io->value || io->cache.value_cache)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "PagedAttention: LATENT layout aliases value to key and requires absent "
                  "value/value_cache");
  } else {
    if (!L->packed && (io->key == nullptr || io->value == nullptr))
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "PagedAttention: key and value must both be present or both be absent");
    if (!io->cache.value_cache)
      return fail(PA_ERR_INVALID_ARGUMENT, "PagedAttention: value_cache is required");
  }
  const int qheads = L->packed ? n->num_heads + 2 * n->kv_num_heads : n->num_heads;
  if (io->query_hidden <= 0 || io->query_hidden % qheads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "query must have rank 2 and a hidden size divisible by its separate or packed "
                "head count");
  L->head = io->query_hidden / qheads;
  L->kv_hidden = L->head * n->kv_num_heads;
  if (io->cache.head_dim != L->head || io->cache.kv_heads != n->kv_num_heads)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "key_cache must be [num_blocks,block_size,kv_num_heads,head_size]");
  L->v_head = n->v_head_size > 0 ? n->v_head_size : L->head;
  if (latent && L->v_head > L->head)
    return fail(PA_ERR_INVALID_ARGUMENT, "PagedAttention: LATENT v_head_size must not exceed head_size");
  if (!latent && L->v_head != L->head)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: SEPARATE layout requires equal key and value head sizes");
  // Packed rows are copied out contiguously by the append kernel (rotated or not).
  L->transform = (n->do_rotary != 0) || io->q_norm_weight != nullptr || L->packed;
  size_t es = elem_size(io->dtype);
  const size_t T = (size_t)std::max(io->num_tokens, 0);
  L->q_bytes = L->transform ? align256(T * n->num_heads * L->head * es) : 0;
  L->k_bytes = L->transform ? align256(T * L->kv_hidden * es) : 0;
  L->v_bytes = L->packed ? align256(T * L->kv_hidden * es) : 0;
  L->attn_off = L->q_bytes + L->k_bytes + L->v_bytes;
  pa_batch& b = L->batch;
  b.cumulative_sequence_length = io->cumulative_sequence_length;
  b.past_seqlens = io->past_seqlens;
  b.block_table = io->block_table;
  b.slot_mapping = io->slot_mapping;
  b.batch = io->batch;
  b.max_blocks = io->max_blocks;
  b.num_tokens = io->num_tokens;
  b.flags = 0;
  // Query-length bound: the caller's, else the host cumulative lengths, else num_tokens.
  if (io->max_query_len < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "max_query_len must be non-negative");
  b.max_query_len = std::min(io->max_query_len, std::max(io->num_tokens, 1));
  if (b.max_query_len == 0 && io->host_cumulative_sequence_length) {
    int mq = 0;
    for (int i = 0; i < io->batch; ++i)
      mq = std::max(mq, io->host_cumulative_sequence_length[i + 1] -
                            io->host_cumulative_sequence_length[i]);
    b.max_query_len = std::max(mq, 1);
  }
  if (b.max_query_len == 0) b.max_query_len = std::max(io->num_tokens, 1);
  // Context bound (past + new tokens of any sequence): the host metadata's maximum, else the
  // caller's, else 0 (the block-table capacity).
  if (io->max_context_len < 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "max_context_len must be non-negative");
  b.max_context_len = io->max_context_len;
  if (io->host_cumulative_sequence_length && io->host_past_seqlens) {
    int64_t mc = 1;
    for (int i = 0; i < io->batch; ++i)
      mc = std::max<int64_t>(mc, (int64_t)io->host_past_seqlens[i] +
                                     io->host_cumulative_sequence_length[i + 1] -
                                     io->host_cumulative_sequence_length[i]);
    b.max_context_len = (int32_t)std::min<int64_t>(mc, INT32_MAX);
  }
  pa_attn& a = L->attn;
  a.num_heads = n->num_heads;
  a.scale = n->scale;
  a.softcap = n->softcap;
  a.local_window_size = n->local_window_size;
  a.is_causal = n->is_causal;
  a.head_sink = io->head_sink;
  a.v_head_size = L->v_head;
  L->total = L->attn_off +
             workspace_for(&io->cache, &b, &a,
                           make_plan(&io->cache, &b, &a, io->dtype, 0, 0, false, 0, images,
                                     false,
                                     HostLens{io->host_cumulative_sequence_length,
                                              io->host_past_seqlens}));
  return PA_OK;
}

// Host-side metadata validation, restating attention.rs:3934-3990 rule for rule.
int validate_host_metadata(const pa_paged_attention_node* n, const pa_paged_attention_io* io) {
  const int32_t* cum = io->host_cumulative_sequence_length;
  const int32_t* past = io->host_past_seqlens;
  const int32_t* bt = io->host_block_table;
  const int B = io->batch;
  if (B < 1)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: cumulative_sequence_length must have length batch+1");
  if (!past || !bt)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: host metadata must include past_seqlens and block_table");
  bool bad = cum[0] != 0 || cum[B] != io->num_tokens || io->max_blocks < 1;
  for (int i = 0; i < B && !bad; ++i) bad = cum[i] < 0 || cum[i] > cum[i + 1];
  for (int i = 0; i < B && !bad; ++i) bad = past[i] < 0;
  if (bad)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: inconsistent cumulative lengths, past lengths or block table");
  if (io->max_query_len > 0)
    for (int i = 0; i < B; ++i)
      if (cum[i + 1] - cum[i] > io->max_query_len)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "PagedAttention: a sequence has more new tokens (%d) than max_query_len (%d)",
                    cum[i + 1] - cum[i], io->max_query_len);
  if (io->max_context_len > 0)
    for (int i = 0; i < B; ++i)
      if ((int64_t)past[i] + cum[i + 1] - cum[i] > io->max_context_len)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "PagedAttention: a sequence has more tokens (%lld) than max_context_len (%d)",
                    (long long)past[i] + cum[i + 1] - cum[i], io->max_context_len);
  const int64_t nb = io->cache.num_blocks, bs = io->cache.block_size;
  if (io->slot_mapping) {
    const int32_t* sm = io->host_slot_mapping;
    if (!sm)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "PagedAttention: host slot_mapping is required with a device slot_mapping");
    for (int t = 0; t < io->num_tokens; ++t)
      if (sm[t] < -1 || (int64_t)sm[t] >= nb * bs)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "PagedAttention: slot_mapping must contain -1 or valid physical cache slots");
  }
  for (int i = 0; i < B; ++i) {
    int64_t total = (int64_t)past[i] + cum[i + 1] - cum[i];
    if (total > INT32_MAX || total > (int64_t)io->max_blocks * bs)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "PagedAttention: sequence exceeds block table capacity");
    int64_t needed = (total + bs - 1) / bs;
    for (int64_t j = 0; j < needed; ++j) {
      int32_t blk = bt[(int64_t)i * io->max_blocks + j];
      if (blk < 0 || blk >= nb)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "PagedAttention: block table contains an invalid physical block");
    }
    if (n->do_rotary) {
      // cos_sin_row (attention.rs:523-535) slices rows [past, past + nq) of the cache.
      int64_t nq = cum[i + 1] - cum[i];
      if (nq > 0 && (past[i] > io->rotary_positions - nq))
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "RotaryEmbedding: requested positions exceed the supplied cache");
    }
  }
  return PA_OK;
}

// True when every token's block-table slot is distinct, so after the append each new key/value
// row sits in its own slot and the attention may read new positions from the pages.
bool host_slots_distinct(const pa_paged_attention_io* io) {
  const int32_t* cum = io->host_cumulative_sequence_length;
  const int32_t* past = io->host_past_seqlens;
  const int32_t* bt = io->host_block_table;
  const int64_t bs = io->cache.block_size;
  // Sufficient and cheap (about T / block_size + B entries): no block id appears twice among the
  // block-table entries that cover the new positions, so no two slots (block * bs + row) meet.
  {
    std::vector<int32_t> blocks;
    blocks.reserve((size_t)std::max(io->num_tokens, 0) / std::max<int64_t>(bs, 1) + 2 * io->batch);
    for (int b = 0; b < io->batch; ++b) {
      if (cum[b + 1] <= cum[b]) continue;
      const int64_t first = (int64_t)past[b], last = first + (cum[b + 1] - cum[b]) - 1;
      for (int64_t bi = first / bs; bi <= last / bs; ++bi)
        blocks.push_back(bt[(int64_t)b * io->max_blocks + bi]);
    }
    std::sort(blocks.begin(), blocks.end());
    if (std::adjacent_find(blocks.begin(), blocks.end()) == blocks.end()) return true;
  }
  // Otherwise compare the slots themselves (shared blocks whose written rows differ).
  std::vector<int64_t> slots;
  slots.reserve((size_t)std::max(io->num_tokens, 0));
  for (int b = 0; b < io->batch; ++b)
    for (int t = cum[b]; t < cum[b + 1]; ++t) {
      const int64_t pos = (int64_t)past[b] + (t - cum[b]);
      slots.push_back((int64_t)bt[(int64_t)b * io->max_blocks + pos / bs] * bs + pos % bs);
    }
  std::sort(slots.begin(), slots.end());
  return std::adjacent_find(slots.begin(), slots.end()) == slots.end();
}

}  // namespace

namespace {

// Bytes of one side of the paged cache ([num_blocks, block_size, kv_heads, row bytes]).
size_t cache_side_bytes(const pa_cache& c) {
  return (size_t)c.num_blocks * c.block_size * c.kv_heads * cache_head_bytes(c.dtype, c.head_dim);
}

// Outputs 1/2 bound to buffers of their own receive the updated caches (the input caches were
// updated in place; an output bound onto its input needs nothing more).
int check_cache_outputs(const pa_paged_attention_node* n, const pa_paged_attention_io* io) {
  if (n->kv_cache_layout_latent && io->value_cache_out)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "PagedAttention: LATENT layout has no separate value cache output");
  return PA_OK;
}

int copy_cache_outputs(const pa_paged_attention_io* io, hipStream_t s) {
  const size_t bytes = cache_side_bytes(io->cache);
  const void* src[2] = {io->cache.key_cache, io->cache.value_cache};
  void* dst[2] = {io->key_cache_out, io->value_cache_out};
  for (int i = 0; i < 2; ++i) {
    if (!dst[i] || dst[i] == src[i] || !src[i]) continue;
    hipError_t e = hipMemcpyAsync(dst[i], src[i], bytes, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "cache output copy");
  }
  return PA_OK;
}

}  // namespace

size_t pa_paged_attention_workspace_bytes(const pa_paged_attention_node* node,
                                          const pa_paged_attention_io* io) {
  OpLayout L;
  if (op_layout(node, io, &L)) return 0;
  return L.total;
}

// The operator entry; images: see make_plan.
static int paged_attention_impl(const pa_paged_attention_node* n, const pa_paged_attention_io* io,
                                void* workspace, size_t workspace_bytes, pa_stream_t stream,
                                bool images) {
  OpLayout L;
  int rc = op_layout(n, io, &L, images);
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (io->host_cumulative_sequence_length && (rc = validate_host_metadata(n, io))) return rc;
  if (n->local_window_size != -1 && n->local_window_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "local_window_size must be -1 or positive");
  if (n->do_rotary && (!io->cos_cache || !io->sin_cache))
    return fail(PA_ERR_INVALID_ARGUMENT, "do_rotary=1 requires cos_cache and sin_cache inputs");
  if (n->do_rotary && n->rotary_offset % 8 != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "rotary_offset must be a multiple of 8");
  if (workspace_bytes < L.total || (L.total && !workspace))
    return fail(PA_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes, got %zu",
                L.total, workspace_bytes);
  if ((rc = check_cache_outputs(n, io))) return rc;
  if (io->num_tokens == 0) return copy_cache_outputs(io, s);
  char* ws = reinterpret_cast<char*>(workspace);
  void* q_rot = L.transform ? ws : nullptr;
  void* k_rot = L.transform ? ws + L.q_bytes : nullptr;
  void* v_rows = L.packed ? ws + L.q_bytes + L.k_bytes : nullptr;
  const void* key = io->key;
  const void* value = io->value;
  AppendExtra x;
  if (L.packed) {
    const size_t es = elem_size(io->dtype);
    const char* qkv = reinterpret_cast<const char*>(io->query);
    key = qkv + (size_t)n->num_heads * L.head * es;
    value = qkv + (size_t)(n->num_heads + n->kv_num_heads) * L.head * es;
    x.q_ld = x.k_ld = x.v_ld = io->query_hidden;
    x.v_out = v_rows;
    x.copy_rows = true;
  }
  RunOpts opts;
  opts.images = images;
  opts.host = HostLens{io->host_cumulative_sequence_length, io->host_past_seqlens};
  const bool distinct = io->slot_mapping == nullptr &&
                        io->host_cumulative_sequence_length != nullptr && host_slots_distinct(io);
  if (distinct) L.batch.flags |= PA_BATCH_SLOTS_DISTINCT;
  opts.new_rows_in_cache = distinct && io->cache.dtype == io->dtype;
  rc = rotary_append_impl(&io->cache, &L.batch, n->num_heads, io->dtype, io->query, key, value,
                          q_rot, k_rot, n->do_rotary ? io->cos_cache : nullptr,
                          n->do_rotary ? io->sin_cache : nullptr, io->rotary_positions,
                          io->rotary_half, n->rotary_offset, n->rotary_interleaved,
                          io->q_norm_weight, io->k_norm_weight, n->qk_norm_epsilon, s, x);
  if (rc) return rc;
  const void* q = L.transform ? q_rot : io->query;
  const void* kn = L.transform ? k_rot : key;
  const void* vn = L.packed ? v_rows : value;
  rc = run_attention(&io->cache, &L.batch, &L.attn, io->dtype, q, kn, vn, io->output,
                     ws + L.attn_off, workspace_bytes - L.attn_off, 0, 0, s, opts);
  if (rc) return rc;
  return copy_cache_outputs(io, s);
}

int pa_paged_attention(const pa_paged_attention_node* n, const pa_paged_attention_io* io,
                       void* workspace, size_t workspace_bytes, pa_stream_t stream) {
  return paged_attention_impl(n, io, workspace, workspace_bytes, stream, true);
}

// ------------------------------------------------------------------------------ no-alloc entry
// The scratch of pa_paged_attention_static: one array per GPU in the library's code object.  In
// host code its name is only a host-side stand-in; the device address comes from
// hipGetSymbolAddress, looked up once per device and kept in g_scratch_ptr.
namespace {

static __device__ __align__(256) unsigned char scratch[PA_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int static_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PA_ERR_UNSUPPORTED, "device %d is beyond the %d devices served", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(PA_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PA_OK;
}

}  // namespace

int pa_paged_attention_static(const pa_paged_attention_node* n, const pa_paged_attention_io* io,
                              pa_stream_t stream) {
  OpLayout L;
  int rc = op_layout(n, io, &L);
  if (rc) return rc;
  // A planned prefill whose operand images do not fit the scratch runs without them.
  bool images = true;
  if (L.total > PA_STATIC_SCRATCH_BYTES) {
    images = false;
    if ((rc = op_layout(n, io, &L, false))) return rc;
  }
  if (L.total > PA_STATIC_SCRATCH_BYTES)
    return fail(PA_ERR_UNSUPPORTED,
                "pa_paged_attention_static: the call needs %zu bytes of workspace, more than the "
                "%zu-byte static scratch",
                L.total, (size_t)PA_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = static_scratch(&ws))) return rc;
  return paged_attention_impl(n, io, ws, PA_STATIC_SCRATCH_BYTES, stream, images);
}

// ------------------------------------------------------------------------------ GQA
namespace {

// Workspace bytes of run_attention for these descriptors and options (the same plan).
size_t attention_ws(const pa_cache* c, const pa_batch* b, const pa_attn* a, pa_dtype act,
                    const RunOpts& o) {
  return workspace_for(c, b, a,
                       make_plan(c, b, a, act, 0, 0, o.linear_cap > 0, o.linear_cap,
                                 plan_images(o), o.bias != nullptr));
}

struct GqaLayout {
  int head;
  bool packed, transform;
  bool shared;      // present == past: updated in place
  bool in_ws;       // present omitted: it lives in the workspace
  bool ragged;      // some sequence may be shorter than the query rows (per-sequence key counts)
  int cap_in;       // past capacity (0 without a past)
  int cap_p;        // present capacity
  bool sliding;     // sliding_window_cache: past and present are rings of capacity cap_in
  int view_cap;     // sliding: rows per (sequence, kv-head) of the staged view (cap_in + seq)
  size_t row_bytes; // bytes of one stored row of one kv-head
  size_t q_bytes, k_bytes, v_bytes, meta_off, pres_off, pres_side, view_off, view_side, attn_off,
      total;
  pa_cache cache;
  pa_batch batch;
  pa_attn attn;
  RunOpts opts;
};

// group_query_attention_op / gqa_batched (attention.rs:932-1454, :586-848): shapes, caches and the
// workspace [rotated q | rotated k | packed v | metadata | present (when omitted) | staged view
// (sliding_window_cache) | attention].
int gqa_layout(const pa_gqa_node* n, const pa_gqa_io* io, GqaLayout* L) {
  if (!n || !io) return fail(PA_ERR_INVALID_ARGUMENT, "node/io is NULL");
  if (n->num_heads <= 0 || n->kv_num_heads <= 0 || n->num_heads % n->kv_num_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "GroupQueryAttention: bad num_heads/kv_num_heads");
  // Key and value absent together: packed [B, S, (H + 2 KV) * head] query (attention.rs:2487).
  // With kv_seq == 0 the (empty) key/value pointers are not read.
  L->packed = io->kv_seq > 0 && io->key == nullptr && io->value == nullptr;
  if (!L->packed && io->kv_seq > 0 && (io->key == nullptr || io->value == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: key and value must both be present or both be absent");
  if (io->batch < 1 || io->seq < 1)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: batch and sequence length must be positive");
  if ((io->kv_seq != io->seq && io->kv_seq != 0) ||
      (io->kv_seq == 0 && (L->packed || io->past_key == nullptr || n->sliding_window_cache)))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: K/V must match Q sequence or be empty with paired "
                "non-sliding past");
  if ((io->past_key == nullptr) != (io->past_value == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: past_key and past_value must be provided together");
  if ((io->present_key == nullptr) != (io->present_value == nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: present_key and present_value must both be provided or "
                "both omitted");
  const int qheads = L->packed ? n->num_heads + 2 * n->kv_num_heads : n->num_heads;
  if (io->query_hidden <= 0 || io->query_hidden % qheads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: query hidden size is not divisible by its head count");
  if (!is_act(io->dtype))
    return fail(PA_ERR_UNSUPPORTED, "activation dtype must be fp16/bf16/fp32");
  if (!io->query || !io->seqlens_k || !io->output)
    return fail(PA_ERR_INVALID_ARGUMENT, "GroupQueryAttention: required pointers are NULL");
  const int64_t total = io->total_sequence_length;
  if (total <= 0 || total > INT32_MAX)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: invalid per-batch or maximum sequence lengths");
  L->cap_in = io->past_key ? io->past_capacity : 0;
  if (io->past_key && io->past_capacity < 1)
    return fail(PA_ERR_INVALID_ARGUMENT, "GroupQueryAttention: past cache capacity must be positive");
  L->shared = io->present_key && io->present_key == io->past_key;
  if (L->shared != (io->present_value && io->present_value == io->past_value))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: present_key and present_value must both alias the past "
                "or neither");
  L->in_ws = io->present_key == nullptr;
  const int64_t grown = std::max<int64_t>(L->cap_in, total);
  L->sliding = n->sliding_window_cache != 0;
  L->view_cap = 0;
  if (L->sliding) {
    // rings of the past's capacity (attention.rs:1146-1165, claim :2455-2473)
    if (n->local_window_size <= 0 || !io->past_key || io->past_capacity < n->local_window_size)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: sliding cache requires 0 < local_window_size <= capacity");
    if (L->in_ws)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: sliding_window_cache requires present key/value outputs");
    if (!L->shared && io->present_capacity != io->past_capacity)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: sliding present must be [batch,kv_num_heads,past "
                  "capacity,head]");
    if (n->qk_output != 0)
      return fail(PA_ERR_UNSUPPORTED,
                  "GroupQueryAttention: sliding_window_cache with QK diagnostics is unsupported");
    L->cap_p = L->cap_in;
    L->view_cap = L->cap_in + io->seq;
  } else if (L->shared) {
    L->cap_p = L->cap_in;
  } else if (!L->in_ws) {
    if (io->present_capacity != grown)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: present must be [batch,kv_num_heads,max(past capacity,"
                  "total_sequence_length),head]");
    L->cap_p = io->present_capacity;
  } else {
    L->cap_p = (int)grown;
  }
  if ((int64_t)io->batch * n->kv_num_heads * std::max(L->cap_p, L->view_cap) > (int64_t)INT32_MAX)
    return fail(PA_ERR_UNSUPPORTED, "GroupQueryAttention: present cache has more than 2^31 rows");
  if (n->qk_output < 0 || n->qk_output > 2 || (n->qk_output != 0) != (io->output_qk != nullptr))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: qk_output must be 0, 1 or 2 and enabled exactly when "
                "output_qk is present");
  L->head = io->query_hidden / qheads;
  L->transform = (n->do_rotary != 0) || io->q_norm_weight != nullptr || L->packed;
  const int64_t T = (int64_t)io->batch * io->seq;
  const size_t es = elem_size(io->dtype);
  const bool kv_rows = io->kv_seq != 0;
  L->q_bytes = L->transform ? align256((size_t)T * n->num_heads * L->head * es) : 0;
  L->k_bytes = (L->transform && kv_rows) ? align256((size_t)T * n->kv_num_heads * L->head * es) : 0;
  L->v_bytes = L->packed ? align256((size_t)T * n->kv_num_heads * L->head * es) : 0;
  L->meta_off = L->q_bytes + L->k_bytes + L->v_bytes;
  L->pres_off = L->meta_off + align256((size_t)pa::meta_ints(io->batch) * sizeof(int32_t));
  pa_cache& c = L->cache;
  c = pa_cache{};
  c.dtype = io->cache_dtype == 0 ? io->dtype : io->cache_dtype;
  if (c.dtype != io->dtype && !is_int_cache(c.dtype))
    return fail(PA_ERR_UNSUPPORTED,
                "GroupQueryAttention: present caches must use the activation dtype, int8 or int4");
  if (c.dtype == PA_DTYPE_INT4 && L->head % 2 != 0)
    return fail(PA_ERR_UNSUPPORTED,
                "GroupQueryAttention: packed INT4 requires an even logical head size");
  L->row_bytes = cache_head_bytes(c.dtype, L->head);
  L->pres_side = L->in_ws ? align256((size_t)io->batch * n->kv_num_heads * L->cap_p * L->row_bytes) : 0;
  L->view_off = L->pres_off + 2 * L->pres_side;
  L->view_side = L->sliding ? align256((size_t)io->batch * n->kv_num_heads * L->view_cap * L->row_bytes) : 0;
  L->attn_off = L->view_off + 2 * L->view_side;
  // rows the attention addresses per (sequence, kv-head): the present, or the staged view
  const int lin_cap = L->sliding ? L->view_cap : L->cap_p;
  // The cache pointers are set per call (the present may live in the workspace).
  c.key_cache = io->present_key ? io->present_key : const_cast<void*>(io->query);
  c.value_cache = io->present_value ? io->present_value : const_cast<void*>(io->query);
  c.block_size = 16;  // geometry for the plan only: rows are addressed contiguously
  c.num_blocks = ((int64_t)io->batch * n->kv_num_heads * lin_cap + 15) / 16;
  c.kv_heads = n->kv_num_heads;
  c.head_dim = L->head;
  c.k_scale = io->k_scale;
  c.v_scale = io->v_scale;
  c.k_quant_type = is_int_cache(c.dtype) ? io->k_quant_type : PA_QUANT_NONE;
  c.v_quant_type = is_int_cache(c.dtype) ? io->v_quant_type : PA_QUANT_NONE;
  pa_batch& b = L->batch;
  b = pa_batch{};
  b.batch = io->batch;
  b.max_blocks = 1;
  b.num_tokens = (int32_t)T;
  b.max_query_len = io->seq;
  b.flags = PA_BATCH_NEW_ROWS_IN_CACHE | PA_BATCH_SLOTS_DISTINCT;
  // every sequence's keys: at most total_sequence_length (host value), within the capacity; the
  // staged view of a ring holds at most its capacity plus the new rows
  b.max_context_len = L->sliding ? lin_cap
                                 : (int32_t)std::max<int64_t>(1, std::min<int64_t>(total, L->cap_p));
  pa_attn& a = L->attn;
  a = pa_attn{};
  a.num_heads = n->num_heads;
  a.scale = n->scale;
  a.softcap = n->softcap;
  a.local_window_size = n->local_window_size;
  a.is_causal = n->is_causal;
  a.head_sink = io->head_sink;
  RunOpts& o = L->opts;
  o = RunOpts{};
  o.new_rows_in_cache = true;
  o.linear_cap = lin_cap;
  // A first prompt (total == seq) may hold sequences shorter than the query rows (right-padded
  // rows): their key counts come from seqlens_k (VALU kernel).  Otherwise every sequence has
  // query_past + seq keys and any kernel family serves it.  The pointer is set per call.
  L->ragged = total == io->seq && !L->sliding;  // rings: every sequence has length >= seq
  if (L->ragged && io->host_seqlens_k) {
    L->ragged = false;
    for (int b = 0; b < io->batch; ++b) L->ragged |= io->host_seqlens_k[b] + 1 < io->seq;
  }
  static const int32_t kPlanOnly = 0;  // non-null marker for planning; replaced before running
  o.key_limit = L->ragged ? &kPlanOnly : nullptr;
  o.bias = io->attention_bias;
  o.bias_b = io->bias_batch;
  o.bias_h = io->bias_heads;
  o.bias_rows = io->seq;
  o.bias_cols = (int)total;
  o.smooth_softmax = n->smooth_softmax == 1;
  L->total = L->attn_off + attention_ws(&c, &b, &a, io->dtype, o);
  return PA_OK;
}

// gqa_batched's length rules (attention.rs:614-631, :665-672) and its cache bound (:695-700).
int validate_gqa_lengths(const pa_gqa_io* io, const GqaLayout& L) {
  const int32_t* len = io->host_seqlens_k;
  const int64_t total = io->total_sequence_length;
  bool bad = false;
  if (L.sliding) {  // attention.rs:1142-1151
    int64_t mx = -1;
    for (int b = 0; b < io->batch; ++b) {
      const int64_t v = len[b];
      bad |= v < 0 || v >= total || v + 1 < io->seq;
      mx = std::max(mx, v);
    }
    if (bad || mx != total - 1)
      return fail(PA_ERR_INVALID_ARGUMENT, "GroupQueryAttention: invalid sliding sequence lengths");
    return PA_OK;
  }
  int64_t mx = -1;
  for (int b = 0; b < io->batch && !bad; ++b) {
    const int64_t v = len[b];
    if (v < 0 || v >= total || (total != io->seq && v + 1 < io->seq)) bad = true;
    mx = std::max(mx, v);
  }
  if (bad || mx != total - 1)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: invalid per-batch or maximum sequence lengths");
  for (int b = 0; b < io->batch; ++b) {
    const int64_t length = (int64_t)len[b] + 1;
    const int64_t qp = std::max<int64_t>(length - io->seq, 0);
    const int64_t past = io->kv_seq == 0 ? length : qp;
    if (past > L.cap_in || (!io->past_key && past != 0) || length > L.cap_p)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: sequence length exceeds available past cache");
  }
  return PA_OK;
}

// Rotary rows the call reads: positions query_past + i (cos_sin_row, attention.rs:523-535), or
// the position ids (gqa_rotary_rows :538-584).
int validate_gqa_rotary(const pa_gqa_io* io) {
  const int64_t rows = io->rotary_positions, S = io->seq;
  if (io->position_ids) {
    if (io->position_cols < S)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "GroupQueryAttention: position_ids must be int64 [batch,>=sequence]");
    const int64_t* pid = io->host_position_ids;
    if (!pid) return PA_OK;  // device ids: kernels leave rows outside the cache unrotated
    if (io->total_sequence_length == S) {
      if (pid[0] < 0 || pid[0] > rows - S)
        return fail(PA_ERR_INVALID_ARGUMENT,
                    "GroupQueryAttention: position_ids exceed the supplied cache");
    } else {
      for (int64_t i = 0; i < (int64_t)io->batch * S; ++i)
        if (pid[i] < 0 || pid[i] >= rows)
          return fail(PA_ERR_INVALID_ARGUMENT,
                      "GroupQueryAttention: position_ids exceed the supplied cache");
    }
    return PA_OK;
  }
  if (!io->host_seqlens_k) return PA_OK;
  for (int b = 0; b < io->batch; ++b) {
    const int64_t qp = std::max<int64_t>((int64_t)io->host_seqlens_k[b] + 1 - S, 0);
    if (qp > rows - S)
      return fail(PA_ERR_INVALID_ARGUMENT,
                  "RotaryEmbedding: requested positions exceed the supplied cache");
  }
  return PA_OK;
}

}  // namespace

size_t pa_group_query_attention_workspace_bytes(const pa_gqa_node* node, const pa_gqa_io* io) {
  GqaLayout L;
  if (gqa_layout(node, io, &L)) return 0;
  return L.total;
}

int pa_group_query_attention(const pa_gqa_node* n, const pa_gqa_io* io, void* workspace,
                             size_t workspace_bytes, pa_stream_t stream) {
  GqaLayout L;
  int rc = gqa_layout(n, io, &L);
  if (rc) return rc;
  if (io->host_seqlens_k && (rc = validate_gqa_lengths(io, L))) return rc;
  if (n->local_window_size != -1 && n->local_window_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: local_window_size must be -1 or positive");
  if (n->do_rotary && (!io->cos_cache || !io->sin_cache))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: do_rotary=1 requires cos_cache and sin_cache inputs");
  if (n->do_rotary && (io->rotary_half <= 0 || 2 * io->rotary_half > L.head))
    return fail(PA_ERR_INVALID_ARGUMENT,
                "GroupQueryAttention: rotary dimension must not exceed head_size");
  if (n->do_rotary && (rc = validate_gqa_rotary(io))) return rc;
  if (io->attention_bias &&
      !((io->bias_batch == 1 || io->bias_batch == io->batch) &&
        (io->bias_heads == 1 || io->bias_heads == n->num_heads)))
    return fail(PA_ERR_INVALID_ARGUMENT,
                L.sliding ? "GroupQueryAttention: sliding attention_bias requires absolute "
                            "total_sequence_length columns"
                          : "GroupQueryAttention: attention_bias must broadcast to "
                            "[batch,heads,sequence,total]");
  if (workspace_bytes < L.total || !workspace)
    return fail(PA_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes, got %zu", L.total,
                workspace_bytes);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  int32_t* meta = reinterpret_cast<int32_t*>(ws + L.meta_off);
  L.batch.cumulative_sequence_length = meta;
  L.batch.past_seqlens = meta + pa::meta_past(io->batch);
  L.batch.block_table = meta;  // unused for contiguous caches
  L.opts.key_limit = L.ragged ? meta + pa::meta_keys(io->batch) : nullptr;
  if (L.in_ws) {
    L.cache.key_cache = ws + L.pres_off;
    L.cache.value_cache = ws + L.pres_off + L.pres_side;
  }
  // A ring's staged view: [the ring's rows before the call | the new rows] per (sequence,
  // kv-head); the attention reads it and the present is written from it afterwards.
  pa::RingParams ring{};
  if (L.sliding) {
    L.cache.key_cache = ws + L.view_off;
    L.cache.value_cache = ws + L.view_off + L.view_side;
    L.opts.bias_col_off = meta + pa::meta_colofs(io->batch);
    ring.seqlens_k = io->seqlens_k;
    ring.row_bytes = (int64_t)L.row_bytes;
    ring.batch = io->batch;
    ring.kv_heads = n->kv_num_heads;
    ring.seq = io->seq;
    ring.cap = L.cap_in;
    ring.window = n->local_window_size;
    ring.zero = L.cache.dtype == PA_DTYPE_INT4 ? 0x88888888u : 0u;
    ring.src_k = reinterpret_cast<const char*>(io->past_key);
    ring.src_v = reinterpret_cast<const char*>(io->past_value);
    ring.dst_k = reinterpret_cast<char*>(L.cache.key_cache);
    ring.dst_v = reinterpret_cast<char*>(L.cache.value_cache);
    ring.present = 0;
    hipError_t e = pa::launch_ring_move(ring, s);
    if (e != hipSuccess) return hip_fail(e, "sliding-window staging");
  }
  // The present starts as [past rows | zero codes] unless it is the past buffer itself
  // (gqa_batched builds [stored | past tail | zeros], attention.rs:790-818).
  if (!L.shared && !L.sliding) {
    const size_t pitch = (size_t)L.cap_p * L.row_bytes;
    const size_t keep = (size_t)std::min(L.cap_in, L.cap_p) * L.row_bytes;
    const size_t rows = (size_t)io->batch * n->kv_num_heads;
    const int zero = L.cache.dtype == PA_DTYPE_INT4 ? 0x88 : 0;
    for (int side = 0; side < 2; ++side) {
      char* dst = reinterpret_cast<char*>(side ? L.cache.value_cache : L.cache.key_cache);
      const void* src = side ? io->past_value : io->past_key;
      hipError_t e = hipSuccess;
      if (src && keep > 0)
        e = hipMemcpy2DAsync(dst, pitch, src, (size_t)L.cap_in * L.row_bytes, keep, rows,
                             hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess && pitch > keep)
        e = hipMemset2DAsync(dst + keep, pitch, zero, pitch - keep, rows, s);
      if (e != hipSuccess) return hip_fail(e, "present cache set-up");
    }
  }
  void* q_rot = L.transform ? ws : nullptr;
  void* k_rot = L.k_bytes ? ws + L.q_bytes : nullptr;
  void* v_rows = L.packed ? ws + L.q_bytes + L.k_bytes : nullptr;
  const void* key = io->kv_seq ? io->key : nullptr;
  const void* value = io->kv_seq ? io->value : nullptr;
  AppendExtra x;
  x.linear_cap = L.sliding ? L.view_cap : L.cap_p;
  x.seq = io->seq;
  if (L.sliding) {
    x.ring_cap = L.cap_in;
    x.ring_window = n->local_window_size;
  }
  x.kv_rows = io->kv_seq != 0;
  x.seqlens_k = io->seqlens_k;
  x.meta_out = meta;
  x.quant_reciprocal = true;  // MLAS GQA encode: x * (1 / scale), zero scale read as 1
  if (n->do_rotary && io->position_ids) {
    x.position_ids = io->position_ids;
    x.pos_offset_form = io->total_sequence_length == io->seq;
  }
  // gqa_rope_f32 for position ids or an empty key/value (attention.rs:716-720); on rings for
  // position ids or a bias (:1222-1228)
  x.rope_fp32 = n->do_rotary &&
                (io->position_ids != nullptr ||
                 (L.sliding ? io->attention_bias != nullptr : io->kv_seq == 0));
  if (L.packed) {
    const size_t es = elem_size(io->dtype);
    const char* qkv = reinterpret_cast<const char*>(io->query);
    key = qkv + (size_t)n->num_heads * L.head * es;
    value = qkv + (size_t)(n->num_heads + n->kv_num_heads) * L.head * es;
    x.q_ld = x.k_ld = x.v_ld = io->query_hidden;
    x.v_out = v_rows;
    x.copy_rows = true;
  }
  rc = rotary_append_impl(&L.cache, &L.batch, n->num_heads, io->dtype, io->query, key, value,
                          q_rot, k_rot, n->do_rotary ? io->cos_cache : nullptr,
                          n->do_rotary ? io->sin_cache : nullptr, io->rotary_positions,
                          io->rotary_half, 0, n->rotary_interleaved, io->q_norm_weight,
                          io->k_norm_weight, n->qk_norm_epsilon, s, x);
  if (rc) return rc;
  const void* q = L.transform ? q_rot : io->query;
  const void* kn = k_rot ? k_rot : (key ? key : io->query);
  const void* vn = L.packed ? v_rows : (value ? value : io->query);
  rc = run_attention(&L.cache, &L.batch, &L.attn, io->dtype, q, kn, vn, io->output,
                     ws + L.attn_off, workspace_bytes - L.attn_off, 0, 0, s, L.opts);
  if (rc) return rc;
  if (L.sliding) {  // the present ring: the view's last rows, then zero codes
    ring.present = 1;
    ring.src_k = reinterpret_cast<const char*>(L.cache.key_cache);
    ring.src_v = reinterpret_cast<const char*>(L.cache.value_cache);
    ring.dst_k = reinterpret_cast<char*>(io->present_key);
    ring.dst_v = reinterpret_cast<char*>(io->present_value);
    hipError_t e = pa::launch_ring_move(ring, s);
    if (e != hipSuccess) return hip_fail(e, "sliding-window present");
  }
  if (n->qk_output != 0) {  // output 3: scores or probabilities over the present
    pa::AttnParams p{};
    p.q = q;
    p.key_cache = L.cache.key_cache;
    p.k_scale = L.cache.k_scale;
    p.k_quant = L.cache.k_quant_type;
    p.past = L.batch.past_seqlens;
    p.head_sink = io->head_sink;
    p.smooth_softmax = n->smooth_softmax == 1 ? 1 : 0;
    p.bias = io->attention_bias;
    p.bias_b = io->bias_batch;
    p.bias_h = io->bias_heads;
    p.bias_rows = io->seq;
    p.bias_cols = (int32_t)io->total_sequence_length;
    p.num_heads = n->num_heads;
    p.kv_heads = n->kv_num_heads;
    p.head_dim = L.head;
    p.batch = io->batch;
    p.max_query_len = io->seq;
    p.linear_cap = L.cap_p;
    p.scale = n->scale != 0.0f ? n->scale : 1.0f / std::sqrt((float)L.head);
    p.softcap = n->softcap;
    p.window = n->local_window_size;
    p.causal = n->is_causal ? 1 : 0;
    hipError_t e = pa::launch_gqa_qk(p, io->dtype, L.cache.dtype, io->output_qk, n->qk_output,
                                     io->total_sequence_length, meta + pa::meta_keys(io->batch), s);
    if (e != hipSuccess) return hip_fail(e, "output_qk");
  }
  return PA_OK;
}

// ------------------------------------------------------------------------------ claim
// paged_attention_claim (attention.rs:4384-4645) + kv_cache::claim (kv_cache.rs:16-108),
// restricted to the forms this build executes; declined forms name the reason.
int pa_paged_attention_claim(const pa_node_info* n, char* reason, size_t reason_len) {
  auto deny = [&](const char* fmt, ...) {
    if (reason && reason_len) {
      va_list ap;
      va_start(ap, fmt);
      vsnprintf(reason, reason_len, fmt, ap);
      va_end(ap);
    }
    return 0;
  };
  if (!n) return deny("node info is NULL");
  if (reason && reason_len) reason[0] = 0;
  const int T16 = PA_DTYPE_FLOAT16, TB16 = PA_DTYPE_BFLOAT16, I32 = PA_INT32_DTYPE;
  if (n->is_causal != 0 && n->is_causal != 1) return deny("is_causal must be 0 or 1");
  if (n->num_outputs < 1 || n->num_outputs > 3)
    return deny("PagedAttention requires 1 to 3 outputs");
  if (n->v_head_size < 0) return deny("v_head_size must be non-negative");
  if (n->rotary_offset < 0) return deny("rotary_offset must be non-negative");
  const int out_dt = n->output_dtype[0];
  if (out_dt != T16 && out_dt != TB16)
    return deny("PagedAttention is only supported for fp16/bf16 (T)");
  if (n->num_inputs < 8 || n->num_inputs > 17)
    return deny("expects 8 required inputs plus optional rotary, scheduling, normalization, "
                "and scale inputs, got %d", n->num_inputs);
  auto present = [&](int i) { return i < n->num_inputs && n->input_present[i]; };
  auto out_present = [&](int i) { return i < n->num_outputs && n->output_present[i]; };
  const bool latent = n->kv_cache_layout_latent != 0;
  const int cache_dt = present(3) ? n->input_dtype[3] : out_dt;
  const bool quantized = cache_dt == PA_INT8_DTYPE || cache_dt == PA_UINT8_DTYPE;
  if (latent && quantized) return deny("quantized LATENT cache contract is not supported");
  const bool packed = !latent && !present(1) && !present(2);
  for (int i : {0, 1}) {
    if (packed && i > 0) break;
    if (!present(i) || n->input_dtype[i] != out_dt)
      return deny("input %d must be present and share the output float dtype", i);
  }
  if (latent) {
    if (present(2) || present(4))
      return deny("LATENT layout aliases value to key and requires absent value/value_cache");
  } else if (!packed && (!present(2) || n->input_dtype[2] != out_dt)) {
    return deny("input 2 must be present and share the output float dtype");
  }
  for (int i : {5, 6, 7})
    if (!present(i) || n->input_dtype[i] != I32) return deny("input %d must be int32", i);
  const int64_t H = n->num_heads, KV = n->kv_num_heads;
  if (!(H > 0 && KV > 0 && H % KV == 0))
    return deny("num_heads (%lld) must be a positive multiple of kv_num_heads (%lld)",
                (long long)H, (long long)KV);
  if (latent && KV != 1) return deny("LATENT layout requires kv_num_heads=1");
  const int64_t qheads = packed ? H + 2 * KV : H;
  if (n->input_rank[0] != 2 || n->input_shape[0][1] <= 0 || n->input_shape[0][1] % qheads != 0)
    return deny("query must have rank 2 and a hidden size divisible by its separate or packed "
                "head count");
  const int64_t head = n->input_shape[0][1] / qheads;
  if (head > kMaxHeadDim)
    return deny("head_size %lld is not executed by this build", (long long)head);
  // kv_cache::claim (kv_cache.rs:16-108): both caches share one storage dtype; integer caches
  // need PER_TENSOR / PER_CHANNEL fp32 scales (inputs 14/15) and a matching *_cache_dtype; a
  // floating cache uses the activation dtype, NONE quantization and no scale.  fp8 e4m3 pages
  // with fp32 per-(block, kv-head) scales are this build's extension.
  if (!present(3) || (!latent && !present(4)))
    return deny("key_cache and value_cache must be present");
  if (latent && cache_dt != out_dt)
    return deny("a LATENT cache must use the activation dtype");
  for (int side = 0; side < 2; ++side) {
    const int cache_in = 3 + side, scale_in = 14 + side;
    const char* nm = side ? "v" : "k";
    const int side_dt = present(cache_in) ? n->input_dtype[cache_in] : out_dt;
    if (side_dt != cache_dt) return deny("key/value caches must share one storage dtype");
    const int mode = side ? n->v_quant_type : n->k_quant_type;
    if (quantized) {
      if (mode != PA_QUANT_PER_TENSOR && mode != PA_QUANT_PER_CHANNEL)
        return deny("integer %s cache requires PER_TENSOR or PER_CHANNEL quantization", nm);
      if (!present(scale_in)) return deny("quantized %s cache requires a scale tensor", nm);
      if (n->input_dtype[scale_in] != PA_DTYPE_FLOAT32) return deny("%s_scale must be float32", nm);
      const int rank = n->input_rank[scale_in];
      int64_t count = 1;
      bool known = rank >= 0 && rank <= 4;
      for (int d = 0; known && d < rank; ++d) {
        if (n->input_shape[scale_in][d] < 0) known = false;
        else count *= n->input_shape[scale_in][d];
      }
      const int64_t expected = mode == PA_QUANT_PER_TENSOR ? 1 : KV * head;
      if (known && count != expected)
        return deny("%s_scale must contain %lld elements", nm, (long long)expected);
      if (mode == PA_QUANT_PER_CHANNEL &&
          !(rank > 0 && rank <= 4 &&
            (n->input_shape[scale_in][rank - 1] < 0 || n->input_shape[scale_in][rank - 1] == head)))
        return deny("PagedAttention per-channel scales must end in head_size");
    } else if (cache_dt == PA_DTYPE_FP8_E4M3) {
      if (!present(scale_in) || n->input_dtype[scale_in] != PA_DTYPE_FLOAT32 ||
          n->input_rank[scale_in] != 2 || n->input_shape[scale_in][1] != KV)
        return deny("fp8 cache requires float32 %s_scale [num_blocks, kv_num_heads]", nm);
    } else if (!(cache_dt == out_dt && mode == PA_QUANT_NONE && !present(scale_in))) {
      return deny("floating %s cache requires activation dtype, NONE quantization and no scale",
                  nm);
    }
    const int logical = side ? n->v_cache_dtype : n->k_cache_dtype;
    const int expected = cache_dt == PA_INT8_DTYPE    ? PA_DTYPE_INT8
                         : cache_dt == PA_UINT8_DTYPE ? PA_DTYPE_INT4
                         : cache_dt == T16            ? T16
                         : cache_dt == TB16           ? TB16
                                                      : 0;
    if (!(logical == expected || (logical == 0 && expected != PA_DTYPE_INT4)))
      return deny("%s_cache_dtype must agree with cache storage; uint8 requires explicit int4",
                  nm);
  }
  const int64_t cache_head = cache_dt == PA_UINT8_DTYPE ? (head + 1) / 2 : head;
  const int64_t v_head = n->v_head_size == 0 ? head : n->v_head_size;
  if (v_head <= 0) return deny("effective v_head_size must be positive");
  if (!packed) {
    if (n->input_rank[1] != 2 || n->input_shape[1][1] != KV * head)
      return deny("key must be [num_tokens,kv_num_heads*head_size]");
    if (!latent && (n->input_rank[2] != 2 || n->input_shape[2][1] != KV * v_head))
      return deny("value must be [num_tokens,kv_num_heads*v_head_size]");
  }
  if (!latent && v_head != head)
    return deny("SEPARATE layout requires equal key and value head sizes");
  if (latent && v_head > head) return deny("LATENT v_head_size must not exceed head_size");
  if (latent && v_head != head && !n->has_scale_attr)
    return deny("LATENT layout with asymmetric value heads requires an explicit scale");
  for (int i : {3, 4}) {
    if (latent && i == 4) break;
    if (n->input_rank[i] != 4 || n->input_shape[i][2] != KV || n->input_shape[i][3] != cache_head)
      return deny("%s must be [num_blocks,block_size,kv_num_heads,head_size]",
                  i == 3 ? "key_cache" : "value_cache");
  }
  if (n->output_rank[0] != 2 ||
      !(n->output_shape[0][1] < 0 || n->output_shape[0][1] == H * v_head))
    return deny("output must be [num_tokens,num_heads*v_head_size]");
  if (!(n->local_window_size == -1 || n->local_window_size > 0))
    return deny("local_window_size must be -1 or positive");
  if (!std::isfinite(n->softcap) || n->softcap < 0.0f)
    return deny("softcap must be finite and non-negative");
  if (n->do_rotary) {
    if (!present(8) || !present(9))
      return deny("do_rotary=1 requires cos_cache and sin_cache inputs");
    if (n->input_dtype[8] != out_dt || n->input_dtype[9] != out_dt)
      return deny("cos_cache/sin_cache must share the output float dtype");
    if (n->input_rank[8] != 2 || n->input_rank[9] != 2 ||
        n->input_shape[8][0] != n->input_shape[9][0] ||
        n->input_shape[8][1] != n->input_shape[9][1] || n->input_shape[8][1] <= 0)
      return deny("cos/sin caches must have matching [positions,rotary_dim/2] shapes");
    const int64_t rot = n->input_shape[8][1] * 2;
    if (n->rotary_offset + rot > head)
      return deny("rotary_offset + rotary_dim must not exceed head_size");
    if (n->rotary_offset % 8 != 0) return deny("rotary_offset must be a multiple of 8");
  }
  if (present(10) &&
      !(n->input_dtype[10] == I32 && n->input_rank[10] == 1 &&
        (n->input_shape[10][0] < 0 || n->input_shape[0][0] < 0 ||
         n->input_shape[10][0] == n->input_shape[0][0])))
    return deny("slot_mapping must be int32 [num_tokens]");
  if (present(11) &&
      !(n->input_dtype[11] == out_dt && n->input_rank[11] == 1 && n->input_shape[11][0] == H))
    return deny("head_sink must be [num_heads] in activation dtype");
  if (present(12) != present(13))
    return deny("q_norm_weight and k_norm_weight must be provided together");
  if (present(12))
    for (int i : {12, 13})
      if (!(n->input_dtype[i] == out_dt && n->input_rank[i] == 1 && n->input_shape[i][0] == head))
        return deny("Q/K norm weight %d must be [head_size] in activation dtype", i);
  if (present(16) && !(n->input_dtype[16] == I32 && n->input_rank[16] == 1 &&
                       (n->input_shape[16][0] == 2 || n->input_shape[16][0] == 3)))
    return deny("attention_metadata must be int32 [2] or [3]");
  if (latent && out_present(2)) return deny("LATENT layout has no separate value cache output");
  for (int i = 1; i < std::min(n->num_outputs, 3); ++i)
    if (out_present(i) && n->output_dtype[i] != n->input_dtype[i + 2])
      return deny("cache output %d must retain cache storage dtype", i);
  return 1;
}

// group_query_attention_claim (attention.rs:2407-2754) + kv_cache::claim for contiguous caches
// (kv_cache.rs:16-108, scales at inputs 12/13), check for check in the reference's order, with
// its messages; head sizes beyond the VALU kernel's 640 are declined.
int pa_group_query_attention_claim(const pa_gqa_node_info* n, char* reason, size_t reason_len) {
  auto deny = [&](const char* fmt, ...) {
    if (reason && reason_len) {
      va_list ap;
      va_start(ap, fmt);
      vsnprintf(reason, reason_len, fmt, ap);
      va_end(ap);
    }
    return 0;
  };
  if (!n) return deny("node info is NULL");
  if (reason && reason_len) reason[0] = 0;
  auto present = [&](int i) { return i < n->num_inputs && n->input_present[i] != 0; };
  auto out_present = [&](int i) { return i < n->num_outputs && n->output_present[i] != 0; };
  auto shape = [&](int i, int d) { return n->input_shape[i][d]; };
  const int I32 = PA_INT32_DTYPE;
  if (n->num_outputs < 1 || n->num_outputs > 4) return deny("requires 1 to 4 outputs");
  if (out_present(1) != out_present(2))
    return deny("present_key and present_value must both be provided or both omitted");
  const bool sliding = n->sliding_window_cache != 0;
  if (n->is_causal != 0 && n->is_causal != 1) return deny("causal must be 0 or 1");
  const int window = n->local_window_size;
  if (!(window == -1 || window > 0)) return deny("local_window_size must be -1 or positive");
  if (n->is_causal == 0 && window != -1)
    return deny("bidirectional GroupQueryAttention requires local_window_size=-1");
  if (present(3) != present(4)) return deny("past_key and past_value must be provided together");
  const int out_dt = n->output_dtype[0];
  if (!out_present(0) || !is_act((pa_dtype)out_dt))
    return deny("output must have an MLX float dtype");
  if (n->num_inputs < 7 || n->num_inputs > 16)
    return deny("expects 7 required inputs plus optional rotary/bias/QK-norm inputs, got %d",
                n->num_inputs);
  const bool has_bias = present(10), do_rotary = n->do_rotary != 0;
  if (n->num_inputs == 7 && do_rotary)
    return deny("7-input GroupQueryAttention requires do_rotary=0 because cos/sin caches are "
                "absent");
  if (sliding) {
    if (window <= 0) return deny("sliding_window_cache=1 requires local_window_size > 0");
    if (!(out_present(1) && out_present(2)))
      return deny("sliding_window_cache requires present key/value outputs");
    if (!(present(3) && n->input_rank[3] == 4 && shape(3, 2) >= window))
      return deny("sliding-window key cache capacity must be at least local_window_size");
    if (!(present(4) && n->input_rank[4] == 4 && shape(4, 2) >= window))
      return deny("sliding-window value cache capacity must be at least local_window_size");
  }
  const bool packed = present(0) && !present(1) && !present(2);
  if (!packed && !(present(0) && present(1) && present(2)))
    return deny("Q/K/V must be either all separate or packed in input 0 with inputs 1 and 2 "
                "absent");
  const bool quantized =
      present(3) && (n->input_dtype[3] == PA_INT8_DTYPE || n->input_dtype[3] == PA_UINT8_DTYPE);
  int float_idx[10], nf = 0;
  float_idx[nf++] = 0;
  if (!packed) float_idx[nf++] = 1, float_idx[nf++] = 2;
  if (present(3) && !quantized) float_idx[nf++] = 3, float_idx[nf++] = 4;
  if (do_rotary) float_idx[nf++] = 7, float_idx[nf++] = 8;
  if (has_bias) float_idx[nf++] = 10;
  if (present(14)) float_idx[nf++] = 14, float_idx[nf++] = 15;
  for (int k = 0; k < nf; ++k) {
    const int i = float_idx[k];
    if (!present(i)) return deny("input %d lacks tensor type/shape info", i);
    if (n->input_dtype[i] != out_dt) return deny("input %d must have the output dtype", i);
  }
  for (int i = 1; i < std::min(n->num_outputs, 3); ++i)
    if (out_present(i) && n->output_dtype[i] != (present(i + 2) ? n->input_dtype[i + 2] : out_dt))
      return deny("output %d must retain its cache dtype", i);
  for (int i : {5, 6})
    if (!present(i) || n->input_dtype[i] != I32) return deny("input %d must have int32 dtype", i);
  if (has_bias && n->input_rank[10] != 4)
    return deny("attention_bias (input 10) must have rank 4, got rank %d", n->input_rank[10]);
  const int64_t nh = n->num_heads, kvh = n->kv_num_heads;
  if (!(nh > 0 && kvh > 0 && nh % kvh == 0))
    return deny("num_heads (%lld) must be a positive multiple of kv_num_heads (%lld)",
                (long long)nh, (long long)kvh);
  if (n->input_rank[0] != 3 || shape(0, 2) <= 0)
    return deny("query must have rank 3 and a positive static hidden size");
  const int64_t total_heads = packed ? nh + 2 * kvh : nh;
  if (shape(0, 2) % total_heads != 0) return deny("query hidden size must match head count");
  const int64_t head = shape(0, 2) / total_heads;
  if (head > kMaxHeadDim)
    return deny("head_size %lld is not executed by this build", (long long)head);
  // kv_cache::claim: one storage dtype; integer caches need PER_TENSOR/PER_CHANNEL fp32 scales.
  const int cache_dt = present(3) ? n->input_dtype[3] : out_dt;
  for (int side = 0; side < 2; ++side) {
    const int cache_in = 3 + side, scale_in = 12 + side;
    const char* nm = side ? "v" : "k";
    const int dt = present(cache_in) ? n->input_dtype[cache_in] : out_dt;
    if (dt != cache_dt) return deny("key/value caches must share one storage dtype");
    const int mode = side ? n->v_quant_type : n->k_quant_type;
    if (quantized) {
      if (mode != PA_QUANT_PER_TENSOR && mode != PA_QUANT_PER_CHANNEL)
        return deny("integer %s cache requires PER_TENSOR or PER_CHANNEL quantization", nm);
      if (!present(scale_in)) return deny("quantized %s cache requires a scale tensor", nm);
      if (n->input_dtype[scale_in] != PA_DTYPE_FLOAT32) return deny("%s_scale must be float32", nm);
      const int rank = n->input_rank[scale_in];
      int64_t count = 1;
      bool known = rank >= 0 && rank <= 4;
      for (int d = 0; known && d < rank; ++d) {
        if (shape(scale_in, d) < 0) known = false;
        else count *= shape(scale_in, d);
      }
      const int64_t expected = mode == PA_QUANT_PER_TENSOR ? 1 : kvh * head;
      if (known && count != expected)
        return deny("%s_scale must contain %lld elements", nm, (long long)expected);
    } else if (!(dt == out_dt && mode == PA_QUANT_NONE && !present(scale_in))) {
      return deny("floating %s cache requires activation dtype, NONE quantization and no scale",
                  nm);
    }
    if (out_present(1 + side) && n->output_dtype[1 + side] != dt)
      return deny("present %s cache must retain its input storage dtype", nm);
  }
  const int bits_expected =
      cache_dt == PA_INT8_DTYPE ? 8 : cache_dt == PA_UINT8_DTYPE ? 4 : 0;
  if (n->kv_cache_bit_width != bits_expected)
    return deny("kv_cache_bit_width must agree with cache storage");
  if (n->kv_cache_bit_width == 4 && head % 2 != 0)
    return deny("GQA packed INT4 requires an even logical head size (pinned CheckPast byte "
                "geometry)");
  if (sliding && n->kv_cache_bit_width != 0 &&
      head % (n->kv_cache_bit_width == 4 ? 32 : 16) != 0)
    return deny("sliding integer cache rows must satisfy pinned 16-byte alignment");
  const int64_t cache_head = n->kv_cache_bit_width == 4 ? (head + 1) / 2 : head;
  const int64_t qb = shape(0, 0), qs = shape(0, 1);
  if (has_bias &&
      !((shape(10, 0) < 0 || shape(10, 0) == 1 || qb < 0 || shape(10, 0) == qb) &&
        (shape(10, 1) < 0 || shape(10, 1) == 1 || shape(10, 1) == nh) &&
        (shape(10, 2) < 0 || qs < 0 || shape(10, 2) == qs)))
    return deny("attention_bias must broadcast to "
                "[batch,num_heads,sequence_length,total_sequence_length]");
  if (!packed) {
    for (int i : {1, 2}) {
      const int64_t kb = shape(i, 0), ks = shape(i, 1);
      if (!(n->input_rank[i] == 3 && shape(i, 2) == kvh * head &&
            (kb < 0 || qb < 0 || kb == qb) &&
            (ks < 0 || qs < 0 || ks == qs || (ks == 0 && present(3)))))
        return deny("key/value must match query batch, sequence length and KV head geometry");
    }
    for (int d = 0; d < 3; ++d)
      if (shape(1, d) != shape(2, d)) return deny("key/value shapes must match");
  }
  for (int i : {3, 4}) {
    if (!present(i)) continue;
    if (!(n->input_rank[i] == 4 && shape(i, 1) == kvh && shape(i, 3) == cache_head &&
          (shape(i, 0) < 0 || qb < 0 || shape(i, 0) == qb)))
      return deny("past cache must be [batch,kv_num_heads,capacity,stored_head_size]");
  }
  if (present(3))
    for (int d = 0; d < 4; ++d)
      if (shape(3, d) != shape(4, d)) return deny("past key/value cache shapes must match");
  if (!(n->input_rank[5] == 1 && (shape(5, 0) < 0 || qb < 0 || shape(5, 0) == qb)))
    return deny("seqlens_k must be [batch]");
  if (!(n->input_rank[6] == 0 || (n->input_rank[6] == 1 && shape(6, 0) == 1)))
    return deny("total_sequence_length must be scalar or [1]");
  if (do_rotary &&
      !(n->input_rank[7] == 2 && n->input_rank[8] == 2 && shape(7, 0) == shape(8, 0) &&
        shape(7, 1) == shape(8, 1) && shape(7, 1) > 0 && 2 * shape(7, 1) <= head))
    return deny("rotary caches must have matching [positions,rotary_dim/2] shapes within the "
                "head");
  if (present(9) && do_rotary &&
      !(n->input_dtype[9] == PA_INT64_DTYPE && n->input_rank[9] == 2 &&
        (shape(9, 0) < 0 || qb < 0 || shape(9, 0) == qb) &&
        (shape(9, 1) < 0 || qs < 0 || shape(9, 1) >= qs)))
    return deny("position_ids must be int64 [batch,>=sequence_length]");
  if (present(11) &&
      !(n->input_dtype[11] == out_dt && n->input_rank[11] == 1 && shape(11, 0) == nh))
    return deny("head_sink must be [num_heads] in activation dtype");
  if (present(14) != present(15))
    return deny("q_norm_weight and k_norm_weight must be provided together");
  if (present(14))
    for (int i : {14, 15})
      if (!(n->input_rank[i] == 1 && shape(i, 0) == head))
        return deny("Q/K norm weight %d must have shape [head_size=%lld]", i, (long long)head);
  if (n->smooth_softmax < -1 || n->smooth_softmax > 1)
    return deny("smooth_softmax must be -1 (schema default), 0 or 1");
  const int qk = n->qk_output;
  if (!(qk >= 0 && qk <= 2 && (qk != 0) == out_present(3)))
    return deny("qk_output must be 0, 1 or 2 and enabled exactly when output_qk is present");
  if (sliding && qk != 0) return deny("sliding_window_cache with QK diagnostics is unsupported");
  if (qk != 0 &&
      !(n->output_dtype[3] == out_dt && n->output_rank[3] == 4 &&
        (n->output_shape[3][0] < 0 || qb < 0 || n->output_shape[3][0] == qb) &&
        (n->output_shape[3][1] < 0 || n->output_shape[3][1] == nh) &&
        (n->output_shape[3][2] < 0 || qs < 0 || n->output_shape[3][2] == qs)))
    return deny("output_qk must be [batch,num_heads,sequence_length,total_sequence_length] in "
                "activation dtype");
  if (!std::isfinite(n->softcap) || n->softcap < 0.0f)
    return deny("softcap must be finite and non-negative");
  return 1;
}

}  // extern "C"
