/*
 * pa_cpu_baseline.c — the CPU path timed beside the GPU in bench.py (TEST/BENCH INFRASTRUCTURE).
 *
 * It is the contiguous-KV GroupQueryAttention decode that ORT's CPUExecutionProvider would run
 * on the gathered cache (semantics: test_gqa_position_cache.py:88-126; gqa_batched
 * attention.rs:586-848): fp32 accumulation, GQA head map kv = h / (H / KV), scale applied to the
 * dot product, max-subtracted softmax.  One task per (sequence, kv-head) so every K/V row is
 * converted once and serves all grouped query heads; tasks are spread over `threads` pthreads.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pa_oracle.h"

typedef struct {
  int dtype;
  const void* q;
  const void* k;
  const void* v;
  const int64_t* kv_offset;
  const int32_t* ctx;
  int batch, num_heads, kv_heads, head_dim;
  float scale;
  float* out;
  int next; /* guarded by lock */
  pthread_mutex_t lock;
} job_t;

static inline void load_row(const void* base, int64_t idx, int d, int dtype, float* dst) {
  if (dtype == ORC_BF16) {
    const uint16_t* s = (const uint16_t*)base + idx;
    for (int e = 0; e < d; ++e) {
      uint32_t u = (uint32_t)s[e] << 16;
      memcpy(&dst[e], &u, 4);
    }
  } else if (dtype == ORC_F16) {
    const uint16_t* s = (const uint16_t*)base + idx;
    for (int e = 0; e < d; ++e) dst[e] = orc_f16_to_f32(s[e]);
  } else {
    memcpy(dst, (const float*)base + idx, (size_t)d * sizeof(float));
  }
}

static void* worker(void* arg) {
  job_t* j = (job_t*)arg;
  int g = j->num_heads / j->kv_heads, d = j->head_dim;
  int max_ctx = 0;
  for (int b = 0; b < j->batch; ++b)
    if (j->ctx[b] > max_ctx) max_ctx = j->ctx[b];
  float* qf = (float*)malloc(sizeof(float) * (size_t)g * d);
  float* row = (float*)malloc(sizeof(float) * (size_t)d);
  float* sc = (float*)malloc(sizeof(float) * (size_t)g * (max_ctx > 0 ? max_ctx : 1));
  float* acc = (float*)malloc(sizeof(float) * (size_t)g * d);
  for (;;) {
    pthread_mutex_lock(&j->lock);
    int task = j->next++;
    pthread_mutex_unlock(&j->lock);
    if (task >= j->batch * j->kv_heads) break;
    int b = task / j->kv_heads, kh = task % j->kv_heads;
    int n = j->ctx[b];
    for (int hh = 0; hh < g; ++hh)
      load_row(j->q, ((int64_t)b * j->num_heads + kh * g + hh) * d, d, j->dtype, qf + hh * d);
    for (int p = 0; p < n; ++p) {
      load_row(j->k, ((j->kv_offset[b] + p) * j->kv_heads + kh) * (int64_t)d, d, j->dtype, row);
      for (int hh = 0; hh < g; ++hh) {
        float s = 0.0f;
        const float* qq = qf + hh * d;
        for (int e = 0; e < d; ++e) s += qq[e] * row[e];
        sc[(size_t)hh * n + p] = s * j->scale;
      }
    }
    float lsum[64];
    for (int hh = 0; hh < g; ++hh) {
      float m = -INFINITY;
      float* s = sc + (size_t)hh * n;
      for (int p = 0; p < n; ++p) m = s[p] > m ? s[p] : m;
      float l = 0.0f;
      for (int p = 0; p < n; ++p) {
        s[p] = expf(s[p] - m);
        l += s[p];
      }
      lsum[hh & 63] = l;
    }
    memset(acc, 0, sizeof(float) * (size_t)g * d);
    for (int p = 0; p < n; ++p) {
      load_row(j->v, ((j->kv_offset[b] + p) * j->kv_heads + kh) * (int64_t)d, d, j->dtype, row);
      for (int hh = 0; hh < g; ++hh) {
        float w = sc[(size_t)hh * n + p];
        float* a = acc + hh * d;
        for (int e = 0; e < d; ++e) a[e] += w * row[e];
      }
    }
    for (int hh = 0; hh < g; ++hh) {
      float inv = lsum[hh & 63] > 0.0f ? 1.0f / lsum[hh & 63] : 0.0f;
      float* o = j->out + ((int64_t)b * j->num_heads + kh * g + hh) * d;
      for (int e = 0; e < d; ++e) o[e] = acc[hh * d + e] * inv;
    }
  }
  free(qf);
  free(row);
  free(sc);
  free(acc);
  return NULL;
}

int orc_cpu_gqa_decode(int dtype, const void* q, const void* k, const void* v,
                       const int64_t* kv_offset, const int32_t* ctx, int batch, int num_heads,
                       int kv_heads, int head_dim, float scale, float* out, int threads) {
  if (num_heads / kv_heads > 64 || threads < 1) return 1;
  job_t j;
  memset(&j, 0, sizeof j);
  j.dtype = dtype;
  j.q = q;
  j.k = k;
  j.v = v;
  j.kv_offset = kv_offset;
  j.ctx = ctx;
  j.batch = batch;
  j.num_heads = num_heads;
  j.kv_heads = kv_heads;
  j.head_dim = head_dim;
  j.scale = scale;
  j.out = out;
  pthread_mutex_init(&j.lock, NULL);
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  int started = 0;
  for (int i = 0; i < threads; ++i)
    if (pthread_create(&tid[i], NULL, worker, &j) == 0) ++started;
  if (started == 0) worker(&j);
  for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
  free(tid);
  pthread_mutex_destroy(&j.lock);
  return 0;
}

/* ---------------------------------------------------------------------------- prefill */
/* Chunked prefill on the CPU path: sequence b's nq[b] query rows (tokens q_start[b] ..) sit at
 * positions past[b] .. past[b] + nq[b] - 1 and see keys 0 .. position (causal); the contiguous
 * K/V of sequence b hold past[b] + nq[b] rows from kv_offset[b].  One task per (sequence,
 * kv-head, block of kPrefillRowsCpu query rows): each key row is converted once per task and
 * serves the block's rows of all grouped heads; tasks spread over `threads` pthreads. */
enum { kPrefillRowsCpu = 16 };

typedef struct {
  int dtype;
  const void *q, *k, *v;
  const int64_t* kv_offset;
  const int32_t *q_start, *nq, *past;
  int batch, num_heads, kv_heads, head_dim, blocks_per_seq;
  float scale;
  float* out;
  int next;
  pthread_mutex_t lock;
} pjob_t;

static void* prefill_worker(void* arg) {
  pjob_t* j = (pjob_t*)arg;
  const int g = j->num_heads / j->kv_heads, d = j->head_dim, R = kPrefillRowsCpu;
  int max_total = 1;
  for (int b = 0; b < j->batch; ++b)
    if (j->past[b] + j->nq[b] > max_total) max_total = j->past[b] + j->nq[b];
  float* qf = (float*)malloc(sizeof(float) * (size_t)R * g * d);
  float* row = (float*)malloc(sizeof(float) * (size_t)d);
  float* sc = (float*)malloc(sizeof(float) * (size_t)R * g * max_total);
  float* acc = (float*)malloc(sizeof(float) * (size_t)R * g * d);
  float* lsum = (float*)malloc(sizeof(float) * (size_t)R * g);
  const int tasks = j->batch * j->kv_heads * j->blocks_per_seq;
  for (;;) {
    pthread_mutex_lock(&j->lock);
    int task = j->next++;
    pthread_mutex_unlock(&j->lock);
    if (task >= tasks) break;
    const int rb = task % j->blocks_per_seq, kh = (task / j->blocks_per_seq) % j->kv_heads;
    const int b = task / (j->blocks_per_seq * j->kv_heads);
    const int r0 = rb * R, rows = j->nq[b] - r0 < R ? j->nq[b] - r0 : R;
    if (rows <= 0) continue;
    const int past = j->past[b];
    const int n = past + r0 + rows; /* keys the block's last row sees */
    for (int r = 0; r < rows; ++r)
      for (int hh = 0; hh < g; ++hh)
        load_row(j->q, ((int64_t)(j->q_start[b] + r0 + r) * j->num_heads + kh * g + hh) * d, d,
                 j->dtype, qf + ((size_t)r * g + hh) * d);
    for (int p = 0; p < n; ++p) {
      load_row(j->k, ((j->kv_offset[b] + p) * j->kv_heads + kh) * (int64_t)d, d, j->dtype, row);
      for (int r = 0; r < rows; ++r) {
        if (p > past + r0 + r) continue;
        for (int hh = 0; hh < g; ++hh) {
          const float* qq = qf + ((size_t)r * g + hh) * d;
          float s = 0.0f;
          for (int e = 0; e < d; ++e) s += qq[e] * row[e];
          sc[((size_t)r * g + hh) * n + p] = s * j->scale;
        }
      }
    }
    for (int r = 0; r < rows; ++r) {
      const int nr = past + r0 + r + 1;
      for (int hh = 0; hh < g; ++hh) {
        float* s = sc + ((size_t)r * g + hh) * n;
        float m = -INFINITY, l = 0.0f;
        for (int p = 0; p < nr; ++p) m = s[p] > m ? s[p] : m;
        for (int p = 0; p < nr; ++p) {
          s[p] = expf(s[p] - m);
          l += s[p];
        }
        lsum[r * g + hh] = l;
      }
    }
    memset(acc, 0, sizeof(float) * (size_t)rows * g * d);
    for (int p = 0; p < n; ++p) {
      load_row(j->v, ((j->kv_offset[b] + p) * j->kv_heads + kh) * (int64_t)d, d, j->dtype, row);
      for (int r = 0; r < rows; ++r) {
        if (p > past + r0 + r) continue;
        for (int hh = 0; hh < g; ++hh) {
          const float w = sc[((size_t)r * g + hh) * n + p];
          float* a = acc + ((size_t)r * g + hh) * d;
          for (int e = 0; e < d; ++e) a[e] += w * row[e];
        }
      }
    }
    for (int r = 0; r < rows; ++r)
      for (int hh = 0; hh < g; ++hh) {
        const float l = lsum[r * g + hh], inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* o = j->out + ((int64_t)(j->q_start[b] + r0 + r) * j->num_heads + kh * g + hh) * d;
        for (int e = 0; e < d; ++e) o[e] = acc[((size_t)r * g + hh) * d + e] * inv;
      }
  }
  free(qf);
  free(row);
  free(sc);
  free(acc);
  free(lsum);
  return NULL;
}

int orc_cpu_gqa_prefill(int dtype, const void* q, const void* k, const void* v,
                        const int64_t* kv_offset, const int32_t* q_start, const int32_t* nq,
                        const int32_t* past, int batch, int num_heads, int kv_heads,
                        int head_dim, float scale, float* out, int threads) {
  if (threads < 1 || kv_heads < 1 || num_heads % kv_heads != 0) return 1;
  pjob_t j;
  memset(&j, 0, sizeof j);
  j.dtype = dtype;
  j.q = q;
  j.k = k;
  j.v = v;
  j.kv_offset = kv_offset;
  j.q_start = q_start;
  j.nq = nq;
  j.past = past;
  j.batch = batch;
  j.num_heads = num_heads;
  j.kv_heads = kv_heads;
  j.head_dim = head_dim;
  j.scale = scale;
  j.out = out;
  int mq = 1;
  for (int b = 0; b < batch; ++b)
    if (nq[b] > mq) mq = nq[b];
  j.blocks_per_seq = (mq + kPrefillRowsCpu - 1) / kPrefillRowsCpu;
  pthread_mutex_init(&j.lock, NULL);
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  int started = 0;
  for (int i = 0; i < threads; ++i)
    if (pthread_create(&tid[i], NULL, prefill_worker, &j) == 0) ++started;
  if (started == 0) prefill_worker(&j);
  for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
  free(tid);
  pthread_mutex_destroy(&j.lock);
  return 0;
}
