/*
 * refcpu_train.c -- CPU parity oracle for the rest of the training step of
 * TransformerTrainer (TEST INFRASTRUCTURE ONLY; see refcpu.h).
 *
 * Restates, operation for operation in float32 (-ffp-contract=off, as
 * refcpu.c): ResidualLayerNormForward with its cache, LayerNormBackward,
 * CrossEntropyLossAndGradient, NeuralNetwork.ComputeInputGradientBatch (the
 * FFN backward), AccumulateTokenEmbeddingGrad, the squared norms, in-place
 * scaling and SGD updates the trainer applies, and TrainBatchDiscrete's flow
 * for one bucket of equal-length sequences.
 *
 * Reference paths are relative to CallaghanDev.ML/ in the reference repo.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "refcpu.h"

#define REF_OK 0
#define REF_EINVAL (-1)

/* AccelerationCPU.cs:1440-1514 (ResidualLayerNormForward): residual = a + b,
 * mean and biased variance of each row (two passes), normalized =
 * (residual - mean) / sqrt(var + eps), out = gamma * normalized + beta. */
int ref_residual_layernorm_forward(const float *a, const float *b, const float *gamma,
                                   const float *beta, float *out, float *means, float *vars,
                                   float *normalized, float *residual, int rows, int features,
                                   float eps) {
  if (!a || !b || !gamma || !beta || !out || !means || !vars || !normalized || !residual)
    return REF_EINVAL;
  for (int i = 0; i < rows; i++) {
    const long row = (long)i * features;
    float mean = 0.0f;
    for (int j = 0; j < features; j++) {
      const float value = a[row + j] + b[row + j];
      residual[row + j] = value;
      mean += value;
    }
    mean /= (float)features;
    means[i] = mean;
    float var = 0.0f;
    for (int j = 0; j < features; j++) {
      const float d = residual[row + j] - mean;
      var += d * d;
    }
    var /= (float)features;
    vars[i] = var;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int j = 0; j < features; j++) {
      const float n = (residual[row + j] - mean) * inv_std;
      normalized[row + j] = n;
      out[row + j] = gamma[j] * n + beta[j];
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:1516-1564 (LayerNormBackward).  Per row:
 *   dGamma[j] += dOut * normalized,  dBeta[j] += dOut,
 *   dNorm = dOut * gamma[j],
 *   dVar  = sum_j dNorm * (x - mean) * -0.5 * invStd^3,
 *   dMean = sum_j dNorm * -invStd,
 *   dx    = dNorm * invStd + dVar * 2/N * (x - mean) + dMean / N.
 * dgamma and dbeta are overwritten (the reference returns new arrays). */
int ref_layernorm_backward(const float *dout, const float *normalized, const float *gamma,
                           const float *input, const float *mean, const float *var,
                           float *dinput, float *dgamma, float *dbeta, int rows, int features,
                           float eps) {
  if (!dout || !normalized || !gamma || !input || !mean || !var || !dinput || !dgamma || !dbeta)
    return REF_EINVAL;
  for (int j = 0; j < features; j++) dgamma[j] = dbeta[j] = 0.0f;
  for (int i = 0; i < rows; i++) {
    const long row = (long)i * features;
    const float inv_std = 1.0f / sqrtf(var[i] + eps);
    const float inv_std3 = inv_std * inv_std * inv_std;
    float dvar = 0.0f, dmean = 0.0f;
    const float m = mean[i];
    for (int j = 0; j < features; j++) {
      const float g = dout[row + j];
      dgamma[j] += g * normalized[row + j];
      dbeta[j] += g;
      const float dnorm = g * gamma[j];
      const float xm = input[row + j] - m;
      dvar += dnorm * xm * (-0.5f) * inv_std3;
      dmean += dnorm * (-inv_std);
    }
    const float inv_n = 1.0f / (float)features;
    const float dvar_scale = dvar * 2.0f * inv_n;
    const float dmean_scale = dmean * inv_n;
    for (int j = 0; j < features; j++) {
      const float dnorm = dout[row + j] * gamma[j];
      const float xm = input[row + j] - m;
      dinput[row + j] = dnorm * inv_std + dvar_scale * xm + dmean_scale;
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:2377-2440 (CrossEntropyLossAndGradient): for the first
 * effective_len rows, p = softmax(logits[i]) (max-shifted exp, one sum),
 * loss -= log(p[target] + 1e-10), dLogits = p / effective_len with
 * 1 / effective_len subtracted at the target; rows past effective_len keep a
 * zero gradient; loss /= effective_len.  targets[target_start + i] is row i's
 * target. */
int ref_cross_entropy(const float *logits, int rows, int out_dim, const int *targets,
                      int n_targets, int target_start, int effective_len, float *loss,
                      float *dlogits) {
  if (!logits || !targets || !loss || !dlogits) return REF_EINVAL;
  if (target_start < 0 || effective_len < 0 || (long)target_start + effective_len > n_targets)
    return REF_EINVAL;
  if (effective_len > rows) return REF_EINVAL;
  memset(dlogits, 0, sizeof(float) * (size_t)rows * out_dim);
  *loss = 0.0f;
  if (effective_len == 0) return REF_OK;
  const float inv_len = 1.0f / (float)effective_len;
  float total = 0.0f;
  for (int i = 0; i < effective_len; i++) {
    const long row = (long)i * out_dim;
    float mx = -INFINITY;
    for (int j = 0; j < out_dim; j++) mx = fmaxf(mx, logits[row + j]);
    float sum = 0.0f;
    for (int j = 0; j < out_dim; j++) {
      const float p = expf(logits[row + j] - mx);
      dlogits[row + j] = p;
      sum += p;
    }
    const float inv_sum = 1.0f / sum;
    const int t = targets[target_start + i];
    if (t < 0 || t >= out_dim) return REF_EINVAL;
    total -= logf((dlogits[row + t] * inv_sum) + 1e-10f);
    for (int j = 0; j < out_dim; j++) {
      float g = (dlogits[row + j] * inv_sum) * inv_len;
      if (j == t) g -= inv_len;
      dlogits[row + j] = g;
    }
  }
  *loss = total / (float)effective_len;
  return REF_OK;
}

static float stable_sigmoid_local(float x) { /* NeuralNetwork.cs:704-716 */
  if (x >= 0.0f) {
    const float z = expf(-x);
    return 1.0f / (1.0f + z);
  }
  const float z = expf(x);
  return z / (1.0f + z);
}

/* NeuralNetwork.cs:885-944 (FillActivationAndDerivative). */
static void act_and_derivative(float z, int type, float *a, float *d) {
  switch (type) {
    case 1: {
      const float s = stable_sigmoid_local(z);
      *a = s;
      *d = s * (1.0f - s);
      return;
    }
    case 2: {
      const float t = tanhf(z);
      *a = t;
      *d = 1.0f - (t * t);
      return;
    }
    case 3:
      *a = z > 0.0f ? z : 0.0f;
      *d = z >= 0.0f ? 1.0f : 0.0f;
      return;
    case 4:
      *a = z > 0.0f ? z : 0.01f * z;
      *d = z <= 0.0f ? 0.1f : 1.0f;
      return;
    case 5: {
      const float s = stable_sigmoid_local(z);
      *a = z * s;
      *d = s + z * s * (1.0f - s);
      return;
    }
    default:
      *a = z;
      *d = 1.0f;
      return;
  }
}

/* AccelerationCPU.cs:159-214 (MatrixMultiply): c[i, j] = Dot(a[i, :], b[:, j]). */
static void matmul(const float *a, const float *b, float *c, int m, int k, int n) {
  float *bt = (float *)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1) * (n > 0 ? n : 1));
  for (int kk = 0; kk < k; kk++)
    for (int j = 0; j < n; j++) bt[(long)j * k + kk] = b[(long)kk * n + j];
  for (int i = 0; i < m; i++)
    for (int j = 0; j < n; j++) c[(long)i * n + j] = ref_dot(a + (long)i * k, bt + (long)j * k, k);
  free(bt);
}

/* NeuralNetwork.cs:946-988 (AccumulateGradientsBatch): wg += deltas^T prev
 * (MatrixMultiply of the transposed deltas), bg[i] += column sum of deltas. */
static void accumulate_batch(const float *deltas, const float *prev, float *wg, float *bg,
                             int rows, int size, int prev_size) {
  float *dt = (float *)calloc((size_t)(rows > 0 ? rows : 1) * (size > 0 ? size : 1), sizeof(float));
  float *wd = (float *)malloc(sizeof(float) * (size_t)(size > 0 ? size : 1) * (prev_size > 0 ? prev_size : 1));
  for (int r = 0; r < rows; r++)
    for (int i = 0; i < size; i++) dt[(long)i * rows + r] = deltas[(long)r * size + i];
  matmul(dt, prev, wd, size, rows, prev_size);
  for (int i = 0; i < size; i++) {
    float b = bg[i];
    for (int r = 0; r < rows; r++) b += deltas[(long)r * size + i];
    bg[i] = b;
    for (int j = 0; j < prev_size; j++) wg[(long)i * prev_size + j] += wd[(long)i * prev_size + j];
  }
  free(dt);
  free(wd);
}

/* NeuralNetwork.cs:773-882 (ComputeInputGradientBatch) for a network with
 * n_layers weight layers: layer l maps widths[l] -> widths[l + 1] with
 * w[l] [widths[l+1], widths[l]], b[l] and activation act[l].  The forward
 * pass is recomputed (BatchDotProductAddBias, then activation and
 * derivative); deltas run from the output layer down; wgrad[l] / bgrad[l]
 * accumulate (both NULL: no accumulation); dinput [rows, widths[0]]. */
int ref_ffn_input_gradient(const float *input, const float *dout, int rows, int n_layers,
                           const int *widths, const float *const *w, const float *const *b,
                           const int *act, float *const *wgrad, float *const *bgrad,
                           float *dinput) {
  if (!input || !dout || !widths || !w || !b || !act || !dinput || n_layers < 1) return REF_EINVAL;
  if (rows == 0) return REF_OK;
  float **acts = (float **)calloc((size_t)n_layers + 1, sizeof(float *));
  float **ders = (float **)calloc((size_t)n_layers + 1, sizeof(float *));
  acts[0] = (float *)input;
  for (int l = 0; l < n_layers; l++) {
    const int in = widths[l], out = widths[l + 1];
    float *z = (float *)malloc(sizeof(float) * (size_t)rows * out);
    ref_batch_dot_add_bias(w[l], acts[l], b[l], z, rows, in, out);
    acts[l + 1] = (float *)malloc(sizeof(float) * (size_t)rows * out);
    ders[l + 1] = (float *)malloc(sizeof(float) * (size_t)rows * out);
    for (long e = 0; e < (long)rows * out; e++) act_and_derivative(z[e], act[l], &acts[l + 1][e], &ders[l + 1][e]);
    free(z);
  }
  const int out_dim = widths[n_layers];
  float *delta = (float *)malloc(sizeof(float) * (size_t)rows * out_dim);
  for (long e = 0; e < (long)rows * out_dim; e++) delta[e] = dout[e] * ders[n_layers][e];
  const int acc = wgrad && bgrad;
  if (acc) accumulate_batch(delta, acts[n_layers - 1], wgrad[n_layers - 1], bgrad[n_layers - 1], rows, out_dim, widths[n_layers - 1]);
  for (int l = n_layers - 1; l >= 1; l--) {
    const int size = widths[l], above = widths[l + 1];
    float *hid = (float *)malloc(sizeof(float) * (size_t)rows * size);
    matmul(delta, w[l], hid, rows, above, size);
    for (long e = 0; e < (long)rows * size; e++) hid[e] *= ders[l][e];
    free(delta);
    delta = hid;
    if (acc) accumulate_batch(delta, acts[l - 1], wgrad[l - 1], bgrad[l - 1], rows, size, widths[l - 1]);
  }
  matmul(delta, w[0], dinput, rows, widths[1], widths[0]);
  free(delta);
  for (int l = 1; l <= n_layers; l++) {
    free(acts[l]);
    free(ders[l]);
  }
  free(acts);
  free(ders);
  return REF_OK;
}

/* AccelerationCPU.cs:2339-2370 (AccumulateTokenEmbeddingGrad): row i of dX is
 * added to row ids[i] of the embedding gradient, rows in order. */
int ref_accumulate_token_embedding_grad(float *eg, const float *dx, const int *ids, int n, int dim,
                                        int vocab) {
  if (!eg || !dx || !ids) return REF_EINVAL;
  for (int i = 0; i < n; i++) {
    const int t = ids[i];
    if (t < 0 || t >= vocab) return REF_EINVAL;
    for (int j = 0; j < dim; j++) eg[(long)t * dim + j] += dx[(long)i * dim + j];
  }
  return REF_OK;
}

/* AccelerationCPU.cs:2493-2512 (MatrixSquaredNorm / VectorSquaredNorm). */
float ref_squared_norm(const float *x, long n) {
  float s = 0.0f;
  for (long i = 0; i < n; i++) s += x[i] * x[i];
  return s;
}

/* AccelerationCPU.cs:2514-2546 (MatrixScaleInPlace / VectorScaleInPlace). */
void ref_scale_inplace(float *x, long n, float scale) {
  for (long i = 0; i < n; i++) x[i] *= scale;
}

/* AccelerationCPU.cs:2548-2597 (MatrixUpdate / VectorUpdate): w -= lr * g. */
void ref_sgd_update(float *w, const float *g, long n, float lr) {
  for (long i = 0; i < n; i++) w[i] -= lr * g[i];
}

/* AccelerationCPU.cs:2447-2490 (MSELossAndGradient): for rows i <
 * effective_len, diff = p[i] - t[target_start + i], loss += diff^2,
 * dOutput = 2 * diff / (effective_len * out_dim); loss /= effective_len *
 * out_dim.  Rows past effective_len keep a zero gradient. */
int ref_mse_loss(const float *pred, int rows, int out_dim, const float *targets, int target_rows,
                 int target_start, int effective_len, float *loss, float *dout) {
  if (!pred || !targets || !loss || !dout) return REF_EINVAL;
  if (target_start < 0 || effective_len < 0 || (long)target_start + effective_len > target_rows ||
      effective_len > rows)
    return REF_EINVAL;
  memset(dout, 0, sizeof(float) * (size_t)rows * out_dim);
  *loss = 0.0f;
  if (effective_len == 0 || out_dim == 0) return REF_OK;
  const float inv_len = 1.0f / (float)(effective_len * out_dim);
  float total = 0.0f;
  for (int i = 0; i < effective_len; i++)
    for (int j = 0; j < out_dim; j++) {
      const float diff = pred[(long)i * out_dim + j] - targets[(long)(target_start + i) * out_dim + j];
      total += diff * diff;
      dout[(long)i * out_dim + j] = 2.0f * diff * inv_len;
    }
  *loss = total / (float)(effective_len * out_dim);
  return REF_OK;
}

/* AccelerationCPU.cs:2280-2332 (BackpropInputProjection): wg[e, f] +=
 * dX[i, e] * input[row_start + i, f], bg[e] += dX[i, e], rows in order. */
int ref_backprop_input_projection(const float *dx, const float *input, int input_rows,
                                  int input_cols, int row_start, float *wg, float *bg, int seq_len,
                                  int emb_dim, int feat_dim) {
  if (!dx || !input || !wg || !bg) return REF_EINVAL;
  if (row_start < 0 || seq_len < 0 || row_start + seq_len > input_rows || feat_dim > input_cols)
    return REF_EINVAL;
  for (int i = 0; i < seq_len; i++) {
    const float *src = input + (long)(row_start + i) * input_cols;
    for (int e = 0; e < emb_dim; e++) {
      const float d = dx[(long)i * emb_dim + e];
      for (int f = 0; f < feat_dim; f++) wg[(long)e * feat_dim + f] += d * src[f];
      bg[e] += d;
    }
  }
  return REF_OK;
}
