/*
 * refcpu_mt.c -- multi-threaded CPU restatement (TEST INFRASTRUCTURE ONLY:
 * the timed CPU baseline of bench.py and a cross-check in tests/).
 *
 * Restates the parallel decomposition of CallaghanDev.ML's
 * AccelerationMutliThreadCPU (AlwaysParallel = true, degree of parallelism =
 * logical processor count, AccelerationMutliThreadCPU.cs:17-20,61-69):
 * Parallel.For is modelled by worker threads that claim loop indices from a
 * shared atomic counter.  Inner loops are the reference's scalar loops.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "refcpu.h"

static int g_threads = 0;

int mt_num_threads(void) {
  if (g_threads > 0) return g_threads;
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

void mt_set_threads(int n) { g_threads = n; }

typedef void (*body_fn)(void *ctx, long i);

typedef struct {
  body_fn fn;
  void *ctx;
  long n;
  long next;
} pfor_t;

static void *pfor_worker(void *arg) {
  pfor_t *p = (pfor_t *)arg;
  for (;;) {
    long i = __atomic_fetch_add(&p->next, 1, __ATOMIC_RELAXED);
    if (i >= p->n) break;
    p->fn(p->ctx, i);
  }
  return NULL;
}

/* Parallel.For(0, n, body) with dynamic index claiming. */
static void parallel_for(long n, body_fn fn, void *ctx) {
  int t = mt_num_threads();
  if (t > n) t = (int)n;
  pfor_t p = {fn, ctx, n, 0};
  if (t <= 1) {
    pfor_worker(&p);
    return;
  }
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)t);
  for (int i = 1; i < t; i++) pthread_create(&th[i], NULL, pfor_worker, &p);
  pfor_worker(&p);
  for (int i = 1; i < t; i++) pthread_join(th[i], NULL);
  free(th);
}

/* ---- ProjectQKV: AccelerationMutliThreadCPU.cs:798-831 ---------------- */
typedef struct {
  const float *x, *wq, *bq, *wk, *bk, *wv, *bv;
  float *q, *k, *v;
  int in_dim, out_dim;
} qkv_ctx;

static void qkv_row(void *c_, long i) {
  qkv_ctx *c = (qkv_ctx *)c_;
  const float *xr = c->x + i * c->in_dim;
  for (int o = 0; o < c->out_dim; o++) {
    float qs = c->bq[o], ks = c->bk[o], vs = c->bv[o];
    const float *wqr = c->wq + (long)o * c->in_dim;
    const float *wkr = c->wk + (long)o * c->in_dim;
    const float *wvr = c->wv + (long)o * c->in_dim;
    for (int d = 0; d < c->in_dim; d++) {
      float xv = xr[d];
      qs += wqr[d] * xv;
      ks += wkr[d] * xv;
      vs += wvr[d] * xv;
    }
    c->q[i * c->out_dim + o] = qs;
    c->k[i * c->out_dim + o] = ks;
    c->v[i * c->out_dim + o] = vs;
  }
}

int mt_project_qkv(const float *x, const float *wq, const float *bq,
                   const float *wk, const float *bk, const float *wv,
                   const float *bv, float *q, float *k, float *v, int rows,
                   int in_dim, int out_dim) {
  qkv_ctx c = {x, wq, bq, wk, bk, wv, bv, q, k, v, in_dim, out_dim};
  parallel_for(rows, qkv_row, &c);
  return 0;
}

/* ---- ProjectOutputBatch: :2331-2359 ----------------------------------- */
typedef struct {
  const float *h, *w, *b;
  float *y;
  int in_dim, out_dim;
  int bias_last; /* BatchDotProductAddBias adds the bias after the sum */
} lin_ctx;

static void lin_row(void *c_, long i) {
  lin_ctx *c = (lin_ctx *)c_;
  const float *hr = c->h + i * c->in_dim;
  for (int j = 0; j < c->out_dim; j++) {
    const float *wr = c->w + (long)j * c->in_dim;
    float s = c->bias_last ? 0.0f : c->b[j];
    for (int d = 0; d < c->in_dim; d++) s += wr[d] * hr[d];
    c->y[i * c->out_dim + j] = c->bias_last ? s + c->b[j] : s;
  }
}

int mt_project_output_batch(const float *h, const float *w, const float *b,
                            float *y, int rows, int in_dim, int out_dim) {
  lin_ctx c = {h, w, b, y, in_dim, out_dim, 0};
  parallel_for(rows, lin_row, &c);
  return 0;
}

/* BatchDotProductAddBias: :483-528 (sum from 0, bias added last). */
int mt_batch_dot_add_bias(const float *w, const float *x, const float *b,
                          float *y, int rows, int in_dim, int out_dim) {
  lin_ctx c = {x, w, b, y, in_dim, out_dim, 1};
  parallel_for(rows, lin_row, &c);
  return 0;
}

/* ---- RoPE: :3353-3380, :3910-3985 (parallel over head x position) ----- */
typedef struct {
  float *x;
  const float *denom;
  int rows, dim, hd;
  int inverse;
} rope_ctx;

static void rope_item(void *c_, long flat) {
  rope_ctx *c = (rope_ctx *)c_;
  int head = (int)(flat / c->rows);
  int pos = (int)(flat - (long)head * c->rows);
  float *row = c->x + (long)pos * c->dim + head * c->hd;
  for (int p = 0; p < c->hd / 2; p++) {
    float theta = (float)pos / c->denom[p];
    float co = cosf(theta), si = sinf(theta);
    if (c->inverse) si = -si;
    float x0 = row[2 * p], x1 = row[2 * p + 1];
    row[2 * p] = (x0 * co) - (x1 * si);
    row[2 * p + 1] = (x0 * si) + (x1 * co);
  }
}

int mt_rope_inplace(float *x, int rows, int dim, int num_heads,
                    float base_theta, int inverse) {
  if (num_heads <= 0 || dim % num_heads) return -1;
  int hd = dim / num_heads;
  if (hd & 1) return -1;
  int pairs = hd / 2;
  if (rows == 0 || pairs == 0) return 0;
  float *denom = (float *)malloc(sizeof(float) * (size_t)pairs);
  for (int p = 0; p < pairs; p++)
    denom[p] = powf(base_theta, (2.0f * (float)p) / (float)hd);
  rope_ctx c = {x, denom, rows, dim, hd, inverse};
  parallel_for((long)num_heads * rows, rope_item, &c);
  free(denom);
  return 0;
}

/* ---- ScaledDotProductAttention: :1991-2098 (parallel over heads only;
 * value accumulated with the head dimension outer and keys inner) ------- */
typedef struct {
  const float *q, *k, *v;
  float *out;
  const uint8_t *mask;
  int lq, lk, dim, hd, causal;
  float scale;
} sdpa_ctx;

static void sdpa_head(void *c_, long head) {
  sdpa_ctx *c = (sdpa_ctx *)c_;
  int off = (int)head * c->hd;
  float *scores = (float *)malloc(sizeof(float) * (size_t)c->lk);
  for (int qi = 0; qi < c->lq; qi++) {
    int usable = c->causal ? (qi + 1 < c->lk ? qi + 1 : c->lk) : c->lk;
    float maxs = -INFINITY;
    const float *qr = c->q + (long)qi * c->dim + off;
    for (int ki = 0; ki < usable; ki++) {
      if (c->mask && !c->mask[(long)qi * c->lk + ki]) {
        scores[ki] = -INFINITY;
        continue;
      }
      const float *kr = c->k + (long)ki * c->dim + off;
      float dot = 0.0f;
      for (int d = 0; d < c->hd; d++) dot += qr[d] * kr[d];
      float s = dot * c->scale;
      scores[ki] = s;
      if (s > maxs) maxs = s;
    }
    if (isinf(maxs) && maxs < 0) continue;
    float sum = 0.0f;
    for (int ki = 0; ki < usable; ki++) {
      float s = scores[ki];
      if (isinf(s) && s < 0) {
        scores[ki] = 0.0f;
        continue;
      }
      float e = expf(s - maxs);
      scores[ki] = e;
      sum += e;
    }
    if (sum <= 0.0f || isnan(sum) || isinf(sum)) continue;
    float inv = 1.0f / sum;
    for (int d = 0; d < c->hd; d++) {
      float val = 0.0f;
      for (int ki = 0; ki < usable; ki++) {
        float w = scores[ki] * inv;
        if (w != 0.0f) val += w * c->v[(long)ki * c->dim + off + d];
      }
      c->out[(long)qi * c->dim + off + d] = val;
    }
  }
  free(scores);
}

int mt_sdpa(const float *q, const float *k, const float *v, float *out, int lq,
            int lk, int dim, int num_heads, const uint8_t *mask, int causal) {
  if (num_heads <= 0 || lq <= 0 || lk <= 0 || dim <= 0 || dim % num_heads)
    return -1;
  if (causal && lq != lk) return -2;
  int hd = dim / num_heads;
  memset(out, 0, sizeof(float) * (size_t)lq * (size_t)dim);
  sdpa_ctx c = {q, k, v, out, mask, lq, lk, dim, hd, causal, 1.0f / sqrtf((float)hd)};
  parallel_for(num_heads, sdpa_head, &c);
  return 0;
}

/* ---- ResidualLayerNorm: :1694-1740 (row-parallel) --------------------- */
typedef struct {
  const float *a, *b, *g, *be;
  float *out;
  int f;
  float eps;
} ln_ctx;

static void ln_row(void *c_, long i) {
  ln_ctx *c = (ln_ctx *)c_;
  ref_residual_layernorm(c->a + i * c->f, c->b + i * c->f, c->g, c->be,
                         c->out + i * c->f, 1, c->f, c->eps);
}

int mt_residual_layernorm(const float *a, const float *b, const float *gamma,
                          const float *beta, float *out, int rows,
                          int features, float eps) {
  ln_ctx c = {a, b, gamma, beta, out, features, eps};
  parallel_for(rows, ln_row, &c);
  return 0;
}

/* ---- decode attention over a [B, Tmax, D] cache ------------------------
 * LanguageModel.cs:365-427 is single-threaded inline host code; the
 * reference has no multi-threaded decode.  parallel = 0 runs the B
 * sequences one after another (faithful), parallel = 1 spreads them over
 * threads (a labelled extension). */
typedef struct {
  const float *q, *kc, *vc;
  const int *kv_len;
  float *out;
  int t_max, dim, heads;
  float scale;
} dec_ctx;

static void dec_item(void *c_, long b) {
  dec_ctx *c = (dec_ctx *)c_;
  long cache_off = b * (long)c->t_max * c->dim;
  ref_decode_attention(c->q + b * c->dim, c->kc + cache_off, c->vc + cache_off,
                       c->kv_len[b], c->dim, c->heads, c->scale,
                       c->out + b * c->dim);
}

int mt_decode_attention_batch(const float *q, const float *kcache,
                              const float *vcache, const int *kv_len,
                              int batch, int t_max, int dim, int num_heads,
                              float scale, float *out, int parallel) {
  dec_ctx c = {q, kcache, vcache, kv_len, out, t_max, dim, num_heads, scale};
  if (parallel) {
    parallel_for(batch, dec_item, &c);
  } else {
    for (long b = 0; b < batch; b++) dec_item(&c, b);
  }
  return 0;
}
