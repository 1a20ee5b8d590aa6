/*
 * refcpu.c -- single-threaded CPU parity oracle (TEST INFRASTRUCTURE ONLY).
 *
 * Restates the hot-path methods of CallaghanDev.ML's AccelerationCPU and the
 * LanguageModel forward / decode / generate flow, operation for operation,
 * so that on an x86-64 host with glibc libm (which .NET's MathF calls on
 * Linux) it reproduces the reference CPU manager's float32 results.  Built
 * with -O2 -ffp-contract=off so that no multiply-add is fused, matching
 * RyuJIT, which never contracts.
 *
 * Reference paths are relative to CallaghanDev.ML/ in the reference repo.
 */
#include "refcpu.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define REF_OK 0
#define REF_EINVAL (-1)
#define REF_ECAUSAL (-2)
#define REF_ENAN (-3)

/* AccelerationManagers/AccelerationCPU.cs:65-104 (Dot).  Vector<float> path
 * (8 lanes on AVX2) when length >= 2*width: lane-wise products accumulated
 * per lane, lanes summed in order, then a 4-way unrolled scalar tail and a
 * scalar remainder, all accumulating into one float in sequence. */
float ref_dot(const float *a, const float *b, int n) {
  float sum = 0.0f;
  int i = 0;
  if (n >= REF_VECTOR_WIDTH * 2) {
    int vend = n - (n % REF_VECTOR_WIDTH);
    float acc[REF_VECTOR_WIDTH];
    for (int l = 0; l < REF_VECTOR_WIDTH; l++) acc[l] = 0.0f;
    for (; i < vend; i += REF_VECTOR_WIDTH)
      for (int l = 0; l < REF_VECTOR_WIDTH; l++) acc[l] += a[i + l] * b[i + l];
    for (int l = 0; l < REF_VECTOR_WIDTH; l++) sum += acc[l];
  }
  int end4 = i + ((n - i) & ~3);
  for (; i < end4; i += 4) {
    sum += a[i] * b[i];
    sum += a[i + 1] * b[i + 1];
    sum += a[i + 2] * b[i + 2];
    sum += a[i + 3] * b[i + 3];
  }
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* AccelerationCPU.cs:107-140 (AddScaledRow): dst[i] += src[i] * scale.
 * Element-wise, so the vector and scalar forms give identical results. */
static void add_scaled_row(float *dst, const float *src, int n, float scale) {
  for (int i = 0; i < n; i++) dst[i] += src[i] * scale;
}

/* AccelerationCPU.cs:2005-2069 (ProjectQKV): q[i,o] = bQ[o] + Dot(WQ[o,:], x[i,:]),
 * likewise K and V, interleaved per output column. */
int ref_project_qkv(const float *x, const float *wq, const float *bq,
                    const float *wk, const float *bk, const float *wv,
                    const float *bv, float *q, float *k, float *v, int rows,
                    int in_dim, int out_dim) {
  if (!x || !wq || !wk || !wv || !bq || !bk || !bv) return REF_EINVAL;
  if (rows < 0 || in_dim < 0 || out_dim < 0) return REF_EINVAL;
  for (int i = 0; i < rows; i++) {
    const float *xr = x + (long)i * in_dim;
    for (int o = 0; o < out_dim; o++) {
      q[(long)i * out_dim + o] = bq[o] + ref_dot(wq + (long)o * in_dim, xr, in_dim);
      k[(long)i * out_dim + o] = bk[o] + ref_dot(wk + (long)o * in_dim, xr, in_dim);
      v[(long)i * out_dim + o] = bv[o] + ref_dot(wv + (long)o * in_dim, xr, in_dim);
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:2694-2715 (ProjectOutputBatch): y[i,j] = b[j] + Dot(W[j,:], h[i,:]). */
int ref_project_output_batch(const float *h, const float *w, const float *b,
                             float *y, int rows, int in_dim, int out_dim) {
  if (!h || !w || !b) return REF_EINVAL;
  for (int i = 0; i < rows; i++)
    for (int j = 0; j < out_dim; j++)
      y[(long)i * out_dim + j] =
          b[j] + ref_dot(w + (long)j * in_dim, h + (long)i * in_dim, in_dim);
  return REF_OK;
}

/* AccelerationCPU.cs:342-404 (BatchDotProductAddBias): y[i,j] = Dot(W[j,:], x[i,:]) + b[j]. */
int ref_batch_dot_add_bias(const float *w, const float *x, const float *b,
                           float *y, int rows, int in_dim, int out_dim) {
  if (!w || !x || !b) return REF_EINVAL;
  for (int i = 0; i < rows; i++)
    for (int j = 0; j < out_dim; j++)
      y[(long)i * out_dim + j] =
          ref_dot(w + (long)j * in_dim, x + (long)i * in_dim, in_dim) + b[j];
  return REF_OK;
}

/* Neural Network/NeuralNetwork.cs:704-716 (StableSigmoidLocal). */
static float stable_sigmoid(float x) {
  if (x >= 0.0f) {
    float z = expf(-x);
    return 1.0f / (1.0f + z);
  }
  float z = expf(x);
  return z / (1.0f + z);
}

/* Neural Network/NeuralNetwork.cs:670-702 (ApplyActivationInPlace);
 * activation ids follow Enums/ActivationType.cs:7-15
 * (None, Sigmoid, Tanh, Relu, Leakyrelu, Swish). */
void ref_activation_inplace(float *x, long n, int activation) {
  if (activation == 0) return;
  for (long i = 0; i < n; i++) {
    float t = x[i];
    switch (activation) {
      case 1: x[i] = stable_sigmoid(t); break;
      case 2: x[i] = tanhf(t); break;
      case 3: x[i] = t > 0.0f ? t : 0.0f; break;
      case 4: x[i] = t > 0.0f ? t : 0.01f * t; break;
      case 5: x[i] = t * stable_sigmoid(t); break;
      default: break;
    }
  }
}

/* AccelerationCPU.cs:4929-4980 (ApplyRotaryPositionEmbeddingHeadCoreInPlace):
 * interleaved pairs (2p, 2p+1) of one head, denom[p] = powf(base, (2p)/hd),
 * theta = pos / denom[p]; inverse negates sin. */
static void rope_head_core(float *x, int rows, int dim, int start_col,
                           int head_dim, float base_theta, int inverse) {
  int pairs = head_dim / 2;
  if (rows == 0 || pairs == 0) return;
  float *denom = (float *)malloc(sizeof(float) * (size_t)pairs);
  for (int p = 0; p < pairs; p++)
    denom[p] = powf(base_theta, (2.0f * (float)p) / (float)head_dim);
  for (int pos = 0; pos < rows; pos++) {
    float *row = x + (long)pos * dim;
    for (int p = 0; p < pairs; p++) {
      int even = start_col + 2 * p;
      float theta = (float)pos / denom[p];
      float c = cosf(theta);
      float s = sinf(theta);
      if (inverse) s = -s;
      float x0 = row[even];
      float x1 = row[even + 1];
      row[even] = (x0 * c) - (x1 * s);
      row[even + 1] = (x0 * s) + (x1 * c);
    }
  }
  free(denom);
}

/* AccelerationCPU.cs:4855-4891 (ApplyRotaryPositionEmbeddingInPlace). */
int ref_rope_inplace(float *x, int rows, int dim, int num_heads,
                     float base_theta, int inverse) {
  if (!x) return REF_EINVAL;
  if (num_heads <= 0) return REF_EINVAL;
  if (!(base_theta > 0.0f) || isinf(base_theta)) return REF_EINVAL;
  if (dim % num_heads != 0) return REF_EINVAL;
  int hd = dim / num_heads;
  if (hd & 1) return REF_EINVAL;
  for (int h = 0; h < num_heads; h++)
    rope_head_core(x, rows, dim, h * hd, hd, base_theta, inverse);
  return REF_OK;
}

/* AccelerationCPU.cs:4893-4927 (ApplyRotaryPositionEmbeddingHeadInPlace). */
int ref_rope_head_inplace(float *x, int rows, int dim, int start_col,
                          int head_dim, float base_theta, int inverse) {
  if (!x) return REF_EINVAL;
  if (start_col < 0 || head_dim < 0) return REF_EINVAL;
  if (head_dim & 1) return REF_EINVAL;
  if (!(base_theta > 0.0f) || isinf(base_theta)) return REF_EINVAL;
  if (start_col + head_dim > dim) return REF_EINVAL;
  rope_head_core(x, rows, dim, start_col, head_dim, base_theta, inverse);
  return REF_OK;
}

/* AccelerationCPU.cs:1797-1956 (ScaledDotProductAttention): per head and
 * query, keys j < usable (causal ? min(i+1, Lk) : Lk) that the mask allows;
 * scale = 1/sqrtf(d_h); three passes (scores+max, exp+sum, weighted V sum);
 * an all-masked row or a non-finite / non-positive sum leaves the row 0. */
int ref_sdpa(const float *q, const float *k, const float *v, float *out,
             int lq, int lk, int dim, int num_heads, const uint8_t *mask,
             int causal) {
  if (!q || !k || !v || !out) return REF_EINVAL;
  if (num_heads <= 0) return REF_EINVAL;
  if (lq <= 0 || lk <= 0 || dim <= 0) return REF_EINVAL;
  if (dim % num_heads != 0) return REF_EINVAL;
  if (causal && lq != lk) return REF_ECAUSAL;
  int hd = dim / num_heads;
  float scale = 1.0f / sqrtf((float)hd);
  memset(out, 0, sizeof(float) * (size_t)lq * (size_t)dim);
  float *scores = (float *)malloc(sizeof(float) * (size_t)lk);
  for (int h = 0; h < num_heads; h++) {
    int off = h * hd;
    for (int i = 0; i < lq; i++) {
      int usable = causal ? (i + 1 < lk ? i + 1 : lk) : lk;
      const float *qr = q + (long)i * dim + off;
      float *orow = out + (long)i * dim + off;
      float maxs = -INFINITY;
      for (int j = 0; j < usable; j++) {
        if (mask && !mask[(long)i * lk + j]) {
          scores[j] = -INFINITY;
          continue;
        }
        float s = ref_dot(qr, k + (long)j * dim + off, hd) * scale;
        scores[j] = s;
        if (s > maxs) maxs = s;
      }
      if (isinf(maxs) && maxs < 0) continue;
      float sum = 0.0f;
      for (int j = 0; j < usable; j++) {
        float s = scores[j];
        if (isinf(s) && s < 0) {
          scores[j] = 0.0f;
          continue;
        }
        float e = expf(s - maxs);
        scores[j] = e;
        sum += e;
      }
      if (sum <= 0.0f || isnan(sum) || isinf(sum)) continue;
      float inv = 1.0f / sum;
      for (int j = 0; j < usable; j++) {
        float w = scores[j] * inv;
        if (w == 0.0f) continue;
        add_scaled_row(orow, v + (long)j * dim + off, hd, w);
      }
    }
  }
  free(scores);
  return REF_OK;
}

/* AccelerationCPU.cs:1647-1792 (MultiHeadAttentionForward): same three
 * passes with an explicit scale, optional mask, no causal flag; an empty
 * sequence returns zeros. */
int ref_mha_forward(const float *q, const float *k, const float *v, float *out,
                    int lq, int lk, int dim, int num_heads, float scale,
                    const uint8_t *mask) {
  if (!q || !k || !v || !out) return REF_EINVAL;
  if (num_heads <= 0 || dim % num_heads != 0) return REF_EINVAL;
  int hd = dim / num_heads;
  memset(out, 0, sizeof(float) * (size_t)lq * (size_t)dim);
  if (lq == 0 || lk == 0 || hd == 0) return REF_OK;
  float *scores = (float *)malloc(sizeof(float) * (size_t)lk);
  for (int h = 0; h < num_heads; h++) {
    int off = h * hd;
    for (int i = 0; i < lq; i++) {
      const float *qr = q + (long)i * dim + off;
      float *orow = out + (long)i * dim + off;
      float maxs = -INFINITY;
      for (int j = 0; j < lk; j++) {
        if (mask && !mask[(long)i * lk + j]) {
          scores[j] = -INFINITY;
          continue;
        }
        float s = ref_dot(qr, k + (long)j * dim + off, hd) * scale;
        scores[j] = s;
        if (s > maxs) maxs = s;
      }
      if (isinf(maxs) && maxs < 0) continue;
      float sum = 0.0f;
      for (int j = 0; j < lk; j++) {
        float s = scores[j];
        if (isinf(s) && s < 0) {
          scores[j] = 0.0f;
          continue;
        }
        float e = expf(s - maxs);
        scores[j] = e;
        sum += e;
      }
      float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
      for (int j = 0; j < lk; j++) {
        float w = scores[j] * inv;
        if (w == 0.0f) continue;
        add_scaled_row(orow, v + (long)j * dim + off, hd, w);
      }
    }
  }
  free(scores);
  return REF_OK;
}

/* AccelerationCPU.cs:710-833 (Softmax): row softmax, masked entries 0, an
 * all-masked row stays 0; a NaN in a considered entry throws
 * InvalidOperationException (returned here as -3). */
int ref_softmax(const float *x, float *out, int rows, int cols,
                const uint8_t *mask) {
  memset(out, 0, sizeof(float) * (size_t)rows * (size_t)cols);
  for (int i = 0; i < rows; i++) {
    const float *r = x + (long)i * cols;
    float *o = out + (long)i * cols;
    const uint8_t *m = mask ? mask + (long)i * cols : NULL;
    float mx = -INFINITY;
    for (int j = 0; j < cols; j++) {
      if (m && !m[j]) continue;
      if (isnan(r[j])) return REF_ENAN;
      if (r[j] > mx) mx = r[j];
    }
    if (isinf(mx) && mx < 0) continue;
    float sum = 0.0f;
    for (int j = 0; j < cols; j++) {
      if (m && !m[j]) {
        o[j] = 0.0f;
        continue;
      }
      float e = expf(r[j] - mx);
      o[j] = e;
      sum += e;
    }
    if (sum <= 0.0f || isnan(sum) || isinf(sum)) continue;
    float inv = 1.0f / sum;
    for (int j = 0; j < cols; j++) o[j] *= inv;
  }
  return REF_OK;
}

/* AccelerationCPU.cs:1376-1438 (ResidualLayerNorm): LN(a + b) per row with
 * two-pass mean and biased variance, invStd = 1/sqrtf(var + eps). */
int ref_residual_layernorm(const float *a, const float *b, const float *gamma,
                           const float *beta, float *out, int rows,
                           int features, float eps) {
  if (!a || !b || !gamma || !beta || !out) return REF_EINVAL;
  for (int i = 0; i < rows; i++) {
    const float *ar = a + (long)i * features;
    const float *br = b + (long)i * features;
    float *o = out + (long)i * features;
    float mean = 0.0f;
    for (int j = 0; j < features; j++) mean += ar[j] + br[j];
    mean /= (float)features;
    float var = 0.0f;
    for (int j = 0; j < features; j++) {
      float d = (ar[j] + br[j]) - mean;
      var += d * d;
    }
    var /= (float)features;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (int j = 0; j < features; j++) {
      float n = ((ar[j] + br[j]) - mean) * inv_std;
      o[j] = gamma[j] * n + beta[j];
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:3473-3515 (EmbedTokenIds): row copy per token id;
 * an id outside [0, vocab) throws ArgumentOutOfRangeException. */
int ref_embed_tokens(const int *ids, int count, const float *table, int vocab,
                     int dim, float *out) {
  for (int i = 0; i < count; i++) {
    int t = ids[i];
    if ((unsigned)t >= (unsigned)vocab) return REF_EINVAL;
    memcpy(out + (long)i * dim, table + (long)t * dim, sizeof(float) * (size_t)dim);
  }
  return REF_OK;
}

/* AccelerationCPU.cs:1566-1586 (CreateCausalMask): mask[i,j] = (j <= i). */
void ref_causal_mask(int n, uint8_t *mask) {
  for (int i = 0; i < n; i++)
    for (int j = 0; j < n; j++) mask[(long)i * n + j] = (uint8_t)(j <= i);
}

/* ---------------------------------------------------------------------- */
/* LanguageModel flow                                                      */
/* ---------------------------------------------------------------------- */

/* Transformers/MultiTypeTransformer/TransformerBlock.cs:53-57 ->
 * AccelerationCPU.cs:1957-2002 (FFNForwardBatch) ->
 * Neural Network/NeuralNetwork.cs:629-668 (ForwardPassOnlyBatch):
 * [D -> FF (activation) -> D (None)] via BatchDotProductAddBias. */
static void ffn_forward(const ref_lm *m, const ref_lm_layer *L, const float *x,
                        int rows, float *out) {
  float *hid = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)m->ff);
  ref_batch_dot_add_bias(L->ffn_w1, x, L->ffn_b1, hid, rows, m->dim, m->ff);
  ref_activation_inplace(hid, (long)rows * m->ff, m->ffn_activation);
  ref_batch_dot_add_bias(L->ffn_w2, hid, L->ffn_b2, out, rows, m->ff, m->dim);
  free(hid);
}

/* TransformerBlock.cs:35-44 with MultiHeadAttention.cs:96-112,149-159:
 * x -> LN1(x + Wo*SDPA(RoPE(Wq x), RoPE(Wk x), Wv x)) -> LN2(h + FFN(h)). */
static void block_forward(const ref_lm *m, const ref_lm_layer *L,
                          const float *x, int n, float *y) {
  int D = m->dim;
  size_t sz = (size_t)n * (size_t)D;
  float *q = (float *)malloc(sizeof(float) * sz);
  float *k = (float *)malloc(sizeof(float) * sz);
  float *v = (float *)malloc(sizeof(float) * sz);
  float *att = (float *)malloc(sizeof(float) * sz);
  float *proj = (float *)malloc(sizeof(float) * sz);
  float *h = (float *)malloc(sizeof(float) * sz);
  float *f = (float *)malloc(sizeof(float) * sz);
  ref_project_qkv(x, L->wq, L->bq, L->wk, L->bk, L->wv, L->bv, q, k, v, n, D, D);
  ref_rope_inplace(q, n, D, m->heads, 10000.0f, 0);
  ref_rope_inplace(k, n, D, m->heads, 10000.0f, 0);
  ref_sdpa(q, k, v, att, n, n, D, m->heads, NULL, 1);
  ref_project_output_batch(att, L->wo, L->bo, proj, n, D, D);
  ref_residual_layernorm(x, proj, L->ln1_g, L->ln1_b, h, n, D, 1e-5f);
  ffn_forward(m, L, h, n, f);
  ref_residual_layernorm(h, f, L->ln2_g, L->ln2_b, y, n, D, 1e-5f);
  free(q); free(k); free(v); free(att); free(proj); free(h); free(f);
}

/* LanguageModel.cs:210-223 (ForwardHiddenFromEmbedding, causal = decoder-only). */
int ref_lm_hidden(const ref_lm *m, const float *embedded, int n, float *hidden) {
  size_t sz = (size_t)n * (size_t)m->dim;
  float *a = (float *)malloc(sizeof(float) * sz);
  float *b = (float *)malloc(sizeof(float) * sz);
  memcpy(a, embedded, sizeof(float) * sz);
  for (int l = 0; l < m->layers; l++) {
    block_forward(m, &m->layer[l], a, n, b);
    float *t = a; a = b; b = t;
  }
  memcpy(hidden, a, sizeof(float) * sz);
  free(a); free(b);
  return REF_OK;
}

/* LanguageModel.cs:585-600 (ValidateTokenSequence). */
static int validate_tokens(const ref_lm *m, const int *ids, int n) {
  if (!ids || n <= 0 || n > m->max_seq) return REF_EINVAL;
  for (int i = 0; i < n; i++)
    if ((unsigned)ids[i] >= (unsigned)m->vocab) return REF_EINVAL;
  return REF_OK;
}

/* LanguageModel.cs:112-122,192-195,225-233 (Forward -> ProjectToOutput). */
int ref_lm_forward(const ref_lm *m, const int *ids, int n, float *logits) {
  if (validate_tokens(m, ids, n)) return REF_EINVAL;
  size_t sz = (size_t)n * (size_t)m->dim;
  float *e = (float *)malloc(sizeof(float) * sz);
  float *h = (float *)malloc(sizeof(float) * sz);
  ref_embed_tokens(ids, n, m->token_embedding, m->vocab, m->dim, e);
  ref_lm_hidden(m, e, n, h);
  ref_project_output_batch(h, m->out_proj, m->out_bias, logits, n, m->dim, m->vocab);
  free(e); free(h);
  return REF_OK;
}

/* LanguageModel.cs:365-427: attention of one query row over cache rows
 * [0, key_len) with scalar sequential dots, recomputed in each of the three
 * passes exactly as the reference does. */
int ref_decode_attention(const float *q, const float *kcache,
                         const float *vcache, int key_len, int dim,
                         int num_heads, float scale, float *out) {
  int hd = dim / num_heads;
  memset(out, 0, sizeof(float) * (size_t)dim);
  for (int h = 0; h < num_heads; h++) {
    int off = h * hd;
    float maxs = -INFINITY;
    for (int j = 0; j < key_len; j++) {
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot += q[off + d] * kcache[(long)j * dim + off + d];
      float s = dot * scale;
      if (s > maxs) maxs = s;
    }
    float sum = 0.0f;
    for (int j = 0; j < key_len; j++) {
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot += q[off + d] * kcache[(long)j * dim + off + d];
      sum += expf((dot * scale) - maxs);
    }
    float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int j = 0; j < key_len; j++) {
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot += q[off + d] * kcache[(long)j * dim + off + d];
      float w = expf((dot * scale) - maxs) * inv;
      if (w == 0.0f) continue;
      for (int d = 0; d < hd; d++) out[off + d] += w * vcache[(long)j * dim + off + d];
    }
  }
  return REF_OK;
}

/* LanguageModel.cs:432-480 (ApplyRotaryPositionSingleRow). */
static void rope_single_row(float *q, float *k, int dim, int num_heads, int pos) {
  int hd = dim / num_heads;
  for (int h = 0; h < num_heads; h++) {
    int off = h * hd;
    for (int p = 0; p < hd / 2; p++) {
      int even = off + 2 * p;
      float theta = (float)pos / powf(10000.0f, (2.0f * (float)p) / (float)hd);
      float c = cosf(theta), s = sinf(theta);
      float q0 = q[even], q1 = q[even + 1];
      q[even] = (q0 * c) - (q1 * s);
      q[even + 1] = (q0 * s) + (q1 * c);
      float k0 = k[even], k1 = k[even + 1];
      k[even] = (k0 * c) - (k1 * s);
      k[even + 1] = (k0 * s) + (k1 * c);
    }
  }
}

typedef struct {
  float *keys, *values; /* [max_seq, D] */
  int length;
} layer_cache;

/* LanguageModel.cs:305-332 (ForwardDecoderTokenFromEmbedding) and
 * :334-430 (DecoderSelfAttentionStep). */
static int decoder_token(const ref_lm *m, layer_cache *caches, const float *emb,
                         int pos, float *out) {
  int D = m->dim;
  float *x = (float *)malloc(sizeof(float) * (size_t)D);
  float *q = (float *)malloc(sizeof(float) * (size_t)D);
  float *k = (float *)malloc(sizeof(float) * (size_t)D);
  float *v = (float *)malloc(sizeof(float) * (size_t)D);
  float *att = (float *)malloc(sizeof(float) * (size_t)D);
  float *proj = (float *)malloc(sizeof(float) * (size_t)D);
  float *h = (float *)malloc(sizeof(float) * (size_t)D);
  float *f = (float *)malloc(sizeof(float) * (size_t)D);
  memcpy(x, emb, sizeof(float) * (size_t)D);
  int rc = REF_OK;
  for (int l = 0; l < m->layers; l++) {
    const ref_lm_layer *L = &m->layer[l];
    layer_cache *c = &caches[l];
    if (c->length != pos || c->length >= m->max_seq) { rc = REF_EINVAL; break; }
    ref_project_qkv(x, L->wq, L->bq, L->wk, L->bk, L->wv, L->bv, q, k, v, 1, D, D);
    rope_single_row(q, k, D, m->heads, pos);
    memcpy(c->keys + (long)c->length * D, k, sizeof(float) * (size_t)D);
    memcpy(c->values + (long)c->length * D, v, sizeof(float) * (size_t)D);
    c->length++;
    int hd = D / m->heads;
    ref_decode_attention(q, c->keys, c->values, c->length, D, m->heads,
                         1.0f / sqrtf((float)hd), att);
    ref_project_output_batch(att, L->wo, L->bo, proj, 1, D, D);
    ref_residual_layernorm(x, proj, L->ln1_g, L->ln1_b, h, 1, D, 1e-5f);
    ffn_forward(m, L, h, 1, f);
    ref_residual_layernorm(h, f, L->ln2_g, L->ln2_b, x, 1, D, 1e-5f);
  }
  memcpy(out, x, sizeof(float) * (size_t)D);
  free(x); free(q); free(k); free(v); free(att); free(proj); free(h); free(f);
  return rc;
}

/* LanguageModel.cs:235-268 (ProjectLastTokenOnly): scalar sequential sums. */
static void last_token_logits(const ref_lm *m, const float *hidden, float *logits) {
  for (int o = 0; o < m->vocab; o++) {
    float s = m->out_bias[o];
    for (int e = 0; e < m->dim; e++) s += m->out_proj[(long)o * m->dim + e] * hidden[e];
    logits[o] = s;
  }
}

/* LanguageModel.cs:482-537 (Generate, decoder-only branch) with the sampler
 * (:551-584) replaced by greedy argmax, lowest index on ties. */
int ref_lm_generate_greedy(const ref_lm *m, const int *prompt, int n_prompt,
                           int max_new, int *out_tokens, int *out_len) {
  if (validate_tokens(m, prompt, n_prompt)) return REF_EINVAL;
  if (max_new < 0) return REF_EINVAL;
  int count = n_prompt;
  memcpy(out_tokens, prompt, sizeof(int) * (size_t)n_prompt);
  *out_len = count;
  if (count >= m->max_seq || max_new == 0) return REF_OK;
  int D = m->dim;
  layer_cache *caches = (layer_cache *)calloc((size_t)m->layers, sizeof(layer_cache));
  for (int l = 0; l < m->layers; l++) {
    caches[l].keys = (float *)calloc((size_t)m->max_seq * D, sizeof(float));
    caches[l].values = (float *)calloc((size_t)m->max_seq * D, sizeof(float));
  }
  float *hidden = (float *)malloc(sizeof(float) * (size_t)D);
  float *logits = (float *)malloc(sizeof(float) * (size_t)m->vocab);
  int rc = REF_OK;
  for (int pos = 0; pos < count && rc == REF_OK; pos++)
    rc = decoder_token(m, caches, m->token_embedding + (long)out_tokens[pos] * D, pos, hidden);
  for (int g = 0; g < max_new && count < m->max_seq && rc == REF_OK; g++) {
    last_token_logits(m, hidden, logits);
    int best = 0;
    for (int o = 1; o < m->vocab; o++)
      if (logits[o] > logits[best]) best = o;
    out_tokens[count++] = best;
    if (count < m->max_seq && g + 1 < max_new)
      rc = decoder_token(m, caches, m->token_embedding + (long)best * D, count - 1, hidden);
  }
  *out_len = count;
  for (int l = 0; l < m->layers; l++) {
    free(caches[l].keys);
    free(caches[l].values);
  }
  free(caches); free(hidden); free(logits);
  return rc;
}
