/*
 * refcpu_bwd.c -- CPU parity oracle for the attention backward path
 * (TEST INFRASTRUCTURE ONLY; see refcpu.h).
 *
 * Restates AccelerationCPU's MultiHeadAttentionBackward, BackpropQKV,
 * BackpropLinearProjection and BackpropOutputProjection operation for
 * operation in float32 (-ffp-contract=off, as refcpu.c).
 *
 * Reference paths are relative to CallaghanDev.ML/ in the reference repo.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "refcpu.h"

#define REF_OK 0
#define REF_EINVAL (-1)

/* AccelerationCPU.cs:1037-1280 (MultiHeadAttentionBackwardCore).  Per head
 * and query row i: scores s_j = Dot(q_i, k_j) * scale over the active keys
 * (mask[i][j] true; without a mask keys j < min(i + 1, lk) when
 * use_decoder_mask, else all), softmax weights w_j = exp(s_j - max) / sum,
 * then dV_j += w_j * dout_i, dAttn_j = dout_i . v_j, rowDot = sum_j w_j dAttn_j,
 * dDot_j = w_j (dAttn_j - rowDot) * scale, dQ_i += dDot_j k_j and
 * dK_j += dDot_j q_i (terms with dDot_j == 0 skipped).  Rows with no active
 * key, a -inf maximum or a non-positive sum contribute nothing.  Outputs are
 * overwritten. */
int ref_mha_backward(const float *q, const float *k, const float *v,
                     const float *dout, float *dq, float *dk, float *dv, int lq,
                     int lk, int dim, int num_heads, float scale,
                     const uint8_t *mask, int use_decoder_mask) {
  if (!q || !k || !v || !dout || !dq || !dk || !dv) return REF_EINVAL;
  if (num_heads <= 0 || lq < 0 || lk < 0 || dim <= 0 || dim % num_heads) return REF_EINVAL;
  const int hd = dim / num_heads;
  memset(dq, 0, sizeof(float) * (size_t)lq * dim);
  memset(dk, 0, sizeof(float) * (size_t)lk * dim);
  memset(dv, 0, sizeof(float) * (size_t)lk * dim);
  float *w = (float *)malloc(sizeof(float) * (size_t)(lk > 0 ? lk : 1));
  float *dattn = (float *)malloc(sizeof(float) * (size_t)(lk > 0 ? lk : 1));
  int *active = (int *)malloc(sizeof(int) * (size_t)(lk > 0 ? lk : 1));
  float *dqrow = (float *)malloc(sizeof(float) * (size_t)hd);
  for (int h = 0; h < num_heads; h++) {
    const int off = h * hd;
    for (int i = 0; i < lq; i++) {
      for (int d = 0; d < hd; d++) dqrow[d] = 0.0f;
      const float *qr = q + (size_t)i * dim + off;
      const float *dor = dout + (size_t)i * dim + off;
      float maxs = -INFINITY;
      int n = 0;
      if (mask) {
        for (int j = 0; j < lk; j++) {
          if (!mask[(size_t)i * lk + j]) continue;
          const float s = ref_dot(qr, k + (size_t)j * dim + off, hd) * scale;
          w[j] = s;
          active[n++] = j;
          if (s > maxs) maxs = s;
        }
      } else {
        const int visible = use_decoder_mask ? (i + 1 < lk ? i + 1 : lk) : lk;
        for (int j = 0; j < visible; j++) {
          const float s = ref_dot(qr, k + (size_t)j * dim + off, hd) * scale;
          w[j] = s;
          active[n++] = j;
          if (s > maxs) maxs = s;
        }
      }
      if (n == 0 || (isinf(maxs) && maxs < 0)) continue;
      float sum = 0.0f;
      for (int a = 0; a < n; a++) {
        const int j = active[a];
        const float e = expf(w[j] - maxs);
        w[j] = e;
        sum += e;
      }
      if (sum <= 0.0f) continue;
      const float inv = 1.0f / sum;
      for (int a = 0; a < n; a++) w[active[a]] *= inv;
      float rowdot = 0.0f;
      for (int a = 0; a < n; a++) {
        const int j = active[a];
        const float wj = w[j];
        float da = 0.0f;
        float *dvr = dv + (size_t)j * dim + off;
        const float *vr = v + (size_t)j * dim + off;
        for (int d = 0; d < hd; d++) {
          const float g = dor[d];
          dvr[d] += wj * g;
          da += g * vr[d];
        }
        dattn[j] = da;
        rowdot += wj * da;
      }
      for (int a = 0; a < n; a++) {
        const int j = active[a];
        const float ddot = w[j] * (dattn[j] - rowdot) * scale;
        if (ddot == 0.0f) continue;
        const float *kr = k + (size_t)j * dim + off;
        float *dkr = dk + (size_t)j * dim + off;
        for (int d = 0; d < hd; d++) {
          dqrow[d] += ddot * kr[d];
          dkr[d] += ddot * qr[d];
        }
      }
      float *dqr = dq + (size_t)i * dim + off;
      for (int d = 0; d < hd; d++) dqr[d] += dqrow[d];
    }
  }
  free(w);
  free(dattn);
  free(active);
  free(dqrow);
  return REF_OK;
}

/* AccelerationCPU.cs:2071-2186 (BackpropQKV): for each row i and output o,
 * bias grads += dX[i][o]; for each input d: W*Grad[o][d] += dX[i][o] * x[i][d]
 * and dInput[i][d] += dQ wq + dK wk + dV wv (one sum of three products).
 * dx is overwritten (a new array in the reference); the gradients
 * accumulate. */
int ref_backprop_qkv(const float *x, const float *dq, const float *dk,
                     const float *dv, const float *wq, const float *wk,
                     const float *wv, float *wqg, float *bqg, float *wkg,
                     float *bkg, float *wvg, float *bvg, float *dx, int rows,
                     int in_dim, int out_dim) {
  if (!x || !dq || !dk || !dv || !wq || !wk || !wv || !wqg || !bqg || !wkg ||
      !bkg || !wvg || !bvg || !dx)
    return REF_EINVAL;
  if (rows < 0 || in_dim < 0 || out_dim < 0) return REF_EINVAL;
  memset(dx, 0, sizeof(float) * (size_t)rows * in_dim);
  for (int i = 0; i < rows; i++) {
    const float *xr = x + (size_t)i * in_dim;
    float *dxr = dx + (size_t)i * in_dim;
    for (int o = 0; o < out_dim; o++) {
      const float gq = dq[(size_t)i * out_dim + o];
      const float gk = dk[(size_t)i * out_dim + o];
      const float gv = dv[(size_t)i * out_dim + o];
      bqg[o] += gq;
      bkg[o] += gk;
      bvg[o] += gv;
      const size_t wr = (size_t)o * in_dim;
      for (int d = 0; d < in_dim; d++) {
        const float xv = xr[d];
        wqg[wr + d] += gq * xv;
        wkg[wr + d] += gk * xv;
        wvg[wr + d] += gv * xv;
        dxr[d] += gq * wq[wr + d] + gk * wk[wr + d] + gv * wv[wr + d];
      }
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:2188-2229 (BackpropLinearProjection): per row i,
 * weightGrad[j][k] += dOut[i][j] * input[i][k], biasGrad[j] += dOut[i][j],
 * then dInput[i][k] += sum_j dOut[i][j] * W[j][k] (summed in j order). */
int ref_backprop_linear_projection(const float *x, const float *dy,
                                   const float *w, float *wg, float *bg,
                                   float *dx, int rows, int in_dim,
                                   int out_dim) {
  if (!x || !dy || !w || !wg || !bg || !dx) return REF_EINVAL;
  if (rows < 0 || in_dim < 0 || out_dim < 0) return REF_EINVAL;
  for (int i = 0; i < rows; i++) {
    const float *xr = x + (size_t)i * in_dim;
    const float *dyr = dy + (size_t)i * out_dim;
    for (int j = 0; j < out_dim; j++) {
      const float g = dyr[j];
      float *wgr = wg + (size_t)j * in_dim;
      for (int kk = 0; kk < in_dim; kk++) wgr[kk] += g * xr[kk];
      bg[j] += g;
    }
    for (int kk = 0; kk < in_dim; kk++) {
      float s = 0.0f;
      for (int j = 0; j < out_dim; j++) s += dyr[j] * w[(size_t)j * in_dim + kk];
      dx[(size_t)i * in_dim + kk] += s;
    }
  }
  return REF_OK;
}

/* AccelerationCPU.cs:2231-2270 (BackpropOutputProjection): as
 * BackpropLinearProjection with the product x * dLogits in the weight
 * gradient and dX overwritten (a new array). */
int ref_backprop_output_projection(const float *dl, const float *x,
                                   const float *w, float *wg, float *bg,
                                   float *dx, int rows, int out_dim,
                                   int emb_dim) {
  if (!dl || !x || !w || !wg || !bg || !dx) return REF_EINVAL;
  if (rows < 0 || out_dim < 0 || emb_dim < 0) return REF_EINVAL;
  for (int i = 0; i < rows; i++) {
    const float *dlr = dl + (size_t)i * out_dim;
    const float *xr = x + (size_t)i * emb_dim;
    for (int vv = 0; vv < out_dim; vv++) {
      const float g = dlr[vv];
      float *wgr = wg + (size_t)vv * emb_dim;
      for (int e = 0; e < emb_dim; e++) wgr[e] += xr[e] * g;
      bg[vv] += g;
    }
    for (int e = 0; e < emb_dim; e++) {
      float s = 0.0f;
      for (int vv = 0; vv < out_dim; vv++) s += dlr[vv] * w[(size_t)vv * emb_dim + e];
      dx[(size_t)i * emb_dim + e] = s;
    }
  }
  return REF_OK;
}
