// Training-step kernels of the decoder LM (TransformerTrainer.TrainBatchDiscrete,
// Transformers/MultiTypeTransformer/TransformerTrainer.cs:217-327): the
// LayerNorm forward with its cache and its backward, the cross-entropy loss
// and gradient, the token-embedding gradient, and the global-norm clipping
// and SGD update over every parameter.  All reductions run in a fixed order
// (no atomics), so a step gives the same bits on every run.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace cdml {
namespace {

constexpr int kRowCache = 32;  // most features kept in registers per lane (64 * 32 = 2048)

// Row-cache size of the LayerNorm kernels: the smallest power of two with
// 64 * RC >= features, so short rows keep few registers (high occupancy).
inline int row_cache(int f) {
  int rc = 1;
  while (64 * rc < f) rc <<= 1;
  return rc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// ResidualLayerNormForward (AccelerationCPU.cs:1440-1514) for one row per
// wave: residual = a + b, mean, biased variance (two passes), out = gamma *
// (residual - mean) * invStd + beta; mean / var / residual / normalized are
// written when non-NULL.  Element i of a lane's row cache is column
// lane + 64 i, or with V4 (features % 4 == 0, 16-byte aligned rows, RC >= 4)
// column 256 (i / 4) + 4 lane + i % 4, so that each access moves a float4.
template <int RC, bool V4>
__global__ void __launch_bounds__(256) ln_forward_kernel(const float *__restrict__ a,
                                                         const float *__restrict__ b,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta,
                                                         float *__restrict__ out,
                                                         float *__restrict__ mean_out,
                                                         float *__restrict__ var_out,
                                                         float *__restrict__ res_out,
                                                         float *__restrict__ norm_out, int rows,
                                                         int f, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const size_t base = (size_t)row * f;
  float cache[RC];
  float sum = 0.f;
  if constexpr (V4) {
#pragma unroll
    for (int i4 = 0; i4 < RC / 4; ++i4) {
      const int j = 256 * i4 + 4 * lane;
      vf4 v = {0.f, 0.f, 0.f, 0.f};
      if (j < f) v = *reinterpret_cast<const vf4 *>(a + base + j) + *reinterpret_cast<const vf4 *>(b + base + j);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cache[4 * i4 + c] = v[c];
        sum += v[c];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const int j = lane + 64 * i;
      cache[i] = j < f ? a[base + j] + b[base + j] : 0.f;
      sum += cache[i];
    }
  }
  const float mean = wave_sum(sum) / (float)f;
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    const int j = V4 ? 256 * (i >> 2) + 4 * lane + (i & 3) : lane + 64 * i;
    const float d = cache[i] - mean;
    var += j < f ? d * d : 0.f;
  }
  var = wave_sum(var) / (float)f;
  const float inv_std = 1.0f / sqrtf(var + eps);
  if constexpr (V4) {
#pragma unroll
    for (int i4 = 0; i4 < RC / 4; ++i4) {
      const int j = 256 * i4 + 4 * lane;
      if (j >= f) continue;
      const vf4 g = *reinterpret_cast<const vf4 *>(gamma + j), be = *reinterpret_cast<const vf4 *>(beta + j);
      vf4 n, y, r;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        r[c] = cache[4 * i4 + c];
        n[c] = (r[c] - mean) * inv_std;
        y[c] = g[c] * n[c] + be[c];
      }
      *reinterpret_cast<vf4 *>(out + base + j) = y;
      if (res_out) *reinterpret_cast<vf4 *>(res_out + base + j) = r;
      if (norm_out) *reinterpret_cast<vf4 *>(norm_out + base + j) = n;
    }
  } else {
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const int j = lane + 64 * i;
      if (j < f) {
        const float n = (cache[i] - mean) * inv_std;
        out[base + j] = gamma[j] * n + beta[j];
        if (res_out) res_out[base + j] = cache[i];
        if (norm_out) norm_out[base + j] = n;
      }
    }
  }
  if (lane == 0) {
    if (mean_out) mean_out[row] = mean;
    if (var_out) var_out[row] = var;
  }
}

// LayerNormBackward (AccelerationCPU.cs:1516-1564), dX part: one row per
// wave.  g = dout (+ dout2: the two gradients of a residual branch, summed
// first as MatrixAddInPlace does); normalized is recomputed from the
// residual input when not given.  Each workgroup owns ln_block_rows(RC) rows
// and writes its partial column sums of g * normalized and g to the
// workspace for ln_param_grad_kernel.
constexpr int kLnRowsPerBlock = 64;  // rows per workgroup (16 waves x 4, or 4 waves x 16 for the longest rows)
constexpr int ln_waves(int rc) { return rc >= 32 ? 4 : 16; }
// Rows per workgroup by row cache: rows of 129 .. 256 features take 32 (16
// waves x 2 rows: c5's 131072 x 256 backward 124 -> 108 us), longer rows 64
// (at 1024 features 32 rows measured 52 -> 62 us).  The workspace size
// follows it, so the choice depends on the feature count only.
constexpr int ln_block_rows(int rc) { return rc == 4 ? 32 : kLnRowsPerBlock; }
inline int ln_blocks(int rows, int features) {
  const int r = ln_block_rows(row_cache(features));
  return (rows + r - 1) / r;
}

template <int RC, int WAVES = ln_waves(RC), int ROWS = ln_block_rows(RC)>
__global__ void __launch_bounds__(64 * WAVES) ln_backward_kernel(
    const float *__restrict__ dout, const float *__restrict__ dout2,
    const float *__restrict__ normalized, const float *__restrict__ gamma,
    const float *__restrict__ x, const float *__restrict__ mean, const float *__restrict__ var,
    float *__restrict__ dx, float *__restrict__ part_g, float *__restrict__ part_b, int rows,
    int f, float eps) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = blockIdx.x * ROWS;
  float pg[RC], pb[RC];
#pragma unroll
  for (int i = 0; i < RC; ++i) pg[i] = pb[i] = 0.f;
  // Short rows (RC <= 4): the wave's U rows are handled together so that
  // their loads and reductions overlap; rows past the end are clamped for
  // the loads and contribute nothing.
  constexpr int U = RC <= 4 ? ROWS / WAVES : 1;
  const float inv_n = 1.0f / (float)f;
  for (int rr0 = wave; rr0 < ROWS; rr0 += WAVES * U) {
    float gv[U][RC], xm[U][RC], dvar[U], dmean[U], istd[U];
    size_t base[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = row0 + rr0 + WAVES * u;
      live[u] = row < rows;
      const int rc = live[u] ? row : rows - 1;
      base[u] = (size_t)rc * f;
      const float inv_std = 1.0f / sqrtf(var[rc] + eps);
      const float inv_std3 = inv_std * inv_std * inv_std;
      const float m = mean[rc];
      istd[u] = inv_std;
      dvar[u] = dmean[u] = 0.f;
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        const int j = lane + 64 * i;
        gv[u][i] = 0.f;
        xm[u][i] = 0.f;
        if (j < f) {
          float g = dout[base[u] + j];
          if (dout2) g += dout2[base[u] + j];
          const float xmj = x[base[u] + j] - m;
          const float n = normalized ? normalized[base[u] + j] : xmj * inv_std;
          if (live[u]) {
            pg[i] += g * n;
            pb[i] += g;
          }
          const float dnorm = g * gamma[j];
          dvar[u] += dnorm * xmj * (-0.5f) * inv_std3;
          dmean[u] += dnorm * (-inv_std);
          gv[u][i] = g;
          xm[u][i] = xmj;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      dvar[u] = wave_sum(dvar[u]);
      dmean[u] = wave_sum(dmean[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!live[u]) continue;
      const float dvar_scale = dvar[u] * 2.0f * inv_n;
      const float dmean_scale = dmean[u] * inv_n;
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        const int j = lane + 64 * i;
        if (j < f) dx[base[u] + j] = (gv[u][i] * gamma[j]) * istd[u] + dvar_scale * xm[u][i] + dmean_scale;
      }
    }
  }
  // the waves' column partials meet in LDS, summed in wave order
  __shared__ float rg[WAVES][64], rb[WAVES][64];
#pragma unroll
  for (int i = 0; i < RC; ++i) {
    if (64 * i >= f) break;  // uniform
    rg[wave][lane] = pg[i];
    rb[wave][lane] = pb[i];
    __syncthreads();
    const int j = lane + 64 * i;
    if (wave == 0 && j < f) {
      float sg = 0.f, sb = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        sg += rg[w][lane];
        sb += rb[w][lane];
      }
      part_g[(size_t)blockIdx.x * f + j] = sg;
      part_b[(size_t)blockIdx.x * f + j] = sb;
    }
    __syncthreads();
  }
}

// The same with float4 columns (features % 4 == 0, 16-byte aligned rows, at
// least 256 features of row cache): lane l owns columns 256 i + 4 l .. + 3,
// so every load and store moves a float4.  The column partials of the
// waves meet in LDS 256 columns at a time and two waves add them, in wave
// order, for the workspace.
template <int R4, int WAVES, int ROWS>
__global__ void __launch_bounds__(64 * WAVES) ln_backward_vec_kernel(
    const float *__restrict__ dout, const float *__restrict__ dout2,
    const float *__restrict__ normalized, const float *__restrict__ gamma,
    const float *__restrict__ x, const float *__restrict__ mean, const float *__restrict__ var,
    float *__restrict__ dx, float *__restrict__ part_g, float *__restrict__ part_b, int rows,
    int f, float eps) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = blockIdx.x * ROWS;
  constexpr int U = R4 == 1 ? ROWS / WAVES : 1;
  const float inv_n = 1.0f / (float)f;
  vf4 pg[R4], pb[R4], gm[R4];
  bool colok[R4];
#pragma unroll
  for (int i = 0; i < R4; ++i) {
    const int col = 256 * i + 4 * lane;
    colok[i] = col < f;
    gm[i] = colok[i] ? *reinterpret_cast<const vf4 *>(gamma + col) : vf4{0.f, 0.f, 0.f, 0.f};
    pg[i] = pb[i] = vf4{0.f, 0.f, 0.f, 0.f};
  }
  for (int rr0 = wave; rr0 < ROWS; rr0 += WAVES * U) {
    vf4 gv[U][R4], xm[U][R4];
    float dvar[U], dmean[U], istd[U];
    size_t base[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = row0 + rr0 + WAVES * u;
      live[u] = row < rows;
      const int rc = live[u] ? row : rows - 1;
      base[u] = (size_t)rc * f;
      const float inv_std = 1.0f / sqrtf(var[rc] + eps);
      const float inv_std3 = inv_std * inv_std * inv_std;
      const float m = mean[rc];
      istd[u] = inv_std;
      dvar[u] = dmean[u] = 0.f;
#pragma unroll
      for (int i = 0; i < R4; ++i) {
        gv[u][i] = xm[u][i] = vf4{0.f, 0.f, 0.f, 0.f};
        if (!colok[i]) continue;
        const size_t o = base[u] + 256 * i + 4 * lane;
        vf4 g = *reinterpret_cast<const vf4 *>(dout + o);
        if (dout2) g += *reinterpret_cast<const vf4 *>(dout2 + o);
        const vf4 xv = *reinterpret_cast<const vf4 *>(x + o);
        vf4 n;
        if (normalized) n = *reinterpret_cast<const vf4 *>(normalized + o);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float xmj = xv[c] - m;
          const float nj = normalized ? n[c] : xmj * inv_std;
          if (live[u]) {
            pg[i][c] += g[c] * nj;
            pb[i][c] += g[c];
          }
          const float dnorm = g[c] * gm[i][c];
          dvar[u] += dnorm * xmj * (-0.5f) * inv_std3;
          dmean[u] += dnorm * (-inv_std);
          xm[u][i][c] = xmj;
        }
        gv[u][i] = g;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      dvar[u] = wave_sum(dvar[u]);
      dmean[u] = wave_sum(dmean[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!live[u]) continue;
      const float dvar_scale = dvar[u] * 2.0f * inv_n;
      const float dmean_scale = dmean[u] * inv_n;
#pragma unroll
      for (int i = 0; i < R4; ++i) {
        if (!colok[i]) continue;
        vf4 y;
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = (gv[u][i][c] * gm[i][c]) * istd[u] + dvar_scale * xm[u][i][c] + dmean_scale;
        *reinterpret_cast<vf4 *>(dx + base[u] + 256 * i + 4 * lane) = y;
      }
    }
  }
  __shared__ vf4 rg[WAVES][64], rb[WAVES][64];
#pragma unroll
  for (int i = 0; i < R4; ++i) {
    if (256 * i >= f) break;  // uniform
    rg[wave][lane] = pg[i];
    rb[wave][lane] = pb[i];
    __syncthreads();
    if (threadIdx.x < 128) {
      const int l = threadIdx.x & 63;
      const bool isb = threadIdx.x >= 64;
      vf4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < WAVES; ++w) sum += isb ? rb[w][l] : rg[w][l];
      const int col = 256 * i + 4 * l;
      if (col < f) *reinterpret_cast<vf4 *>((isb ? part_b : part_g) + (size_t)blockIdx.x * f + col) = sum;
    }
    __syncthreads();
  }
}

// dGamma / dBeta: the row-block partials summed in a fixed order -- 64
// columns per workgroup, wave w of 16 taking blocks w, w + 16, ..., the 16
// wave sums then added in wave order -- and written, or added to the
// caller's accumulators (the trainer's VectorAccumulate).
__global__ void __launch_bounds__(1024) ln_param_grad_kernel(const float *__restrict__ part_g,
                                                             const float *__restrict__ part_b,
                                                             float *__restrict__ dgamma,
                                                             float *__restrict__ dbeta, int nblk,
                                                             int f, int accumulate) {
  __shared__ float rg[16][64], rb[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + lane;
  float sg = 0.f, sb = 0.f;
  if (j < f)
    for (int k = wave; k < nblk; k += 16) {
      sg += part_g[(size_t)k * f + j];
      sb += part_b[(size_t)k * f + j];
    }
  rg[wave][lane] = sg;
  rb[wave][lane] = sb;
  __syncthreads();
  if (wave == 0 && j < f) {
    float g = 0.f, b = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      g += rg[w][lane];
      b += rb[w][lane];
    }
    if (dgamma) dgamma[j] = accumulate ? dgamma[j] + g : g;
    if (dbeta) dbeta[j] = accumulate ? dbeta[j] + b : b;
  }
}

// First pass of the dGamma / dBeta sums for many row blocks: workgroup
// (c, s) adds the partials of blocks s * chunk .. min((s + 1) * chunk, nblk)
// - 1 for columns 64 c .. 64 c + 63 (wave w takes the slice's blocks w, w + 4,
// ..., the four wave sums then added in wave order) and writes them as row s
// of out_g / out_b, which ln_param_grad_kernel then sums.  The order is fixed,
// so results do not depend on timing.
__global__ void __launch_bounds__(256) ln_param_slice_kernel(const float *__restrict__ part_g,
                                                             const float *__restrict__ part_b,
                                                             float *__restrict__ out_g,
                                                             float *__restrict__ out_b, int nblk,
                                                             int chunk, int f) {
  __shared__ float rg[4][64], rb[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + lane;
  const int k0 = blockIdx.y * chunk, k1 = min(k0 + chunk, nblk);
  float sg = 0.f, sb = 0.f;
  if (j < f) {
    int k = k0 + wave;
    for (; k + 12 < k1; k += 16) {  // four blocks in flight per wave
      const float g0 = part_g[(size_t)k * f + j], g1 = part_g[(size_t)(k + 4) * f + j];
      const float g2 = part_g[(size_t)(k + 8) * f + j], g3 = part_g[(size_t)(k + 12) * f + j];
      const float b0 = part_b[(size_t)k * f + j], b1 = part_b[(size_t)(k + 4) * f + j];
      const float b2 = part_b[(size_t)(k + 8) * f + j], b3 = part_b[(size_t)(k + 12) * f + j];
      sg = (((sg + g0) + g1) + g2) + g3;
      sb = (((sb + b0) + b1) + b2) + b3;
    }
    for (; k < k1; k += 4) {
      sg += part_g[(size_t)k * f + j];
      sb += part_b[(size_t)k * f + j];
    }
  }
  rg[wave][lane] = sg;
  rb[wave][lane] = sb;
  __syncthreads();
  if (wave == 0 && j < f) {
    out_g[(size_t)blockIdx.y * f + j] = ((rg[0][lane] + rg[1][lane]) + rg[2][lane]) + rg[3][lane];
    out_b[(size_t)blockIdx.y * f + j] = ((rb[0][lane] + rb[1][lane]) + rb[2][lane]) + rb[3][lane];
  }
}

// Row-block count above which the dGamma / dBeta sums take two passes, and
// the first pass's slice count.
constexpr int kLnSlices = 64;
inline int ln_slices(int nblk) { return nblk > 4 * kLnSlices ? kLnSlices : 0; }

// CrossEntropyLossAndGradient (AccelerationCPU.cs:2377-2440): one workgroup per
// row.  Rows below effective_len: p = exp(l - max) / sum, loss term
// -log(p[target] + 1e-10), gradient (p / effective_len, minus 1 / effective_len
// at the target) times grad_scale; rows at or past effective_len get a zero
// gradient.  grad_scale is the trainer's ScaleMatrixLocal of a bucket
// (TransformerTrainer.cs:291-294), 1 otherwise.
__global__ void __launch_bounds__(256) ce_row_kernel(const float *__restrict__ logits, int ldl,
                                                     const int *__restrict__ targets, int rows,
                                                     int v, int effective_len, float grad_scale,
                                                     float *__restrict__ dl, int lddl,
                                                     float *__restrict__ row_loss) {
  const int row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float *l = logits + (size_t)row * ldl;
  float *g = dl + (size_t)row * lddl;
  if (row >= effective_len) {
    for (int j = t; j < v; j += 256) g[j] = 0.f;
    return;
  }
  __shared__ float red[4];
  float mx = -INFINITY;
  for (int j = t; j < v; j += 256) mx = fmaxf(mx, l[j]);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int j = t; j < v; j += 256) {
    const float e = expf(l[j] - mx);
    g[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = ((red[0] + red[1]) + red[2]) + red[3];
  const float inv_sum = 1.0f / sum;
  const float inv_len = 1.0f / (float)effective_len;
  const int target = targets[row];
  if (t == 0 && (target < 0 || target >= v)) row_loss[row] = NAN;  // surfaces as a non-finite loss
  for (int j = t; j < v; j += 256) {
    float gr = (g[j] * inv_sum) * inv_len;
    if (j == target) {
      row_loss[row] = -logf((g[j] * inv_sum) + 1e-10f);
      gr -= inv_len;
    }
    g[j] = gr * grad_scale;
  }
}

// MSELossAndGradient (AccelerationCPU.cs:2447-2490): one thread per row; rows
// below effective_len get d = 2 * diff / (effective_len * out_dim) (times
// grad_scale) and their sum of diff^2 as the row term; later rows get 0.
__global__ void __launch_bounds__(256) mse_row_kernel(const float *__restrict__ pred, int ldp,
                                                      const float *__restrict__ targets, int ldt,
                                                      int rows, int o, int effective_len,
                                                      float grad_scale, float *__restrict__ d,
                                                      int ldd, float *__restrict__ row_loss) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  float *dr = d + (size_t)row * ldd;
  if (row >= effective_len) {
    for (int j = 0; j < o; ++j) dr[j] = 0.f;
    return;
  }
  const float inv_len = 1.0f / (float)(effective_len * o);
  const float *pr = pred + (size_t)row * ldp, *tr = targets + (size_t)row * ldt;
  float s = 0.f;
  for (int j = 0; j < o; ++j) {
    const float diff = pr[j] - tr[j];
    s += diff * diff;
    dr[j] = (2.0f * diff * inv_len) * grad_scale;
  }
  row_loss[row] = s;
}

// target[i] += addend[i] (MatrixAddInPlace, AccelerationCPU.cs:522-546).
__global__ void __launch_bounds__(256) add_inplace_kernel(float *__restrict__ target,
                                                          const float *__restrict__ addend,
                                                          long long n) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    target[i] += addend[i];
}

// loss = (sum of the row terms, fixed order) / divisor, times loss_scale.
// One workgroup of 1024 threads; thread t keeps four running sums (rows
// t + 1024 (4q + r) into sum r), so four loads per thread are in flight, and
// the sums meet in a fixed tree.
__global__ void __launch_bounds__(1024) ce_loss_kernel(const float *__restrict__ row_loss, int n,
                                                       float divisor, float loss_scale,
                                                       float *__restrict__ loss) {
  __shared__ float red[1024];
  const int t = threadIdx.x;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int i = t;
  for (; i + 3 * 1024 < n; i += 4 * 1024) {
    s0 += row_loss[i];
    s1 += row_loss[i + 1024];
    s2 += row_loss[i + 2048];
    s3 += row_loss[i + 3072];
  }
  for (; i < n; i += 1024) s0 += row_loss[i];
  red[t] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
  if (t == 0) *loss = (red[0] / divisor) * loss_scale;
}

// AccumulateTokenEmbeddingGrad (AccelerationCPU.cs:2339-2370) as a gather: group
// k adds rows order[start[k] .. start[k+1]) of dx (+ dx2) to row token[k] of
// the gradient, one column per thread, rows in increasing order (the
// reference's order), so repeated tokens need no atomics.
__global__ void __launch_bounds__(256) embed_grad_kernel(float *__restrict__ eg,
                                                         const float *__restrict__ dx,
                                                         const float *__restrict__ dx2, int ldx,
                                                         const int *__restrict__ order,
                                                         const int *__restrict__ start,
                                                         const int *__restrict__ token, int dim) {
  const int k = blockIdx.x;
  const int j = blockIdx.y * 256 + threadIdx.x;
  if (j >= dim) return;
  float *dst = eg + (size_t)token[k] * dim + j;
  float v = *dst;
  for (int r = start[k]; r < start[k + 1]; ++r) {
    const size_t o = (size_t)order[r] * ldx + j;
    v += dx2 ? dx[o] + dx2[o] : dx[o];
  }
  *dst = v;
}

constexpr int kNormBlocks = 512;

// Squared norm of every parameter's gradient after `prescale` (the trainer's
// ScaleGradients by 1 / validCount, TransformerTrainer.cs:313): each block
// walks every tensor with a stride of kNormBlocks float4s and writes one
// partial per tensor.
__global__ void __launch_bounds__(256) sumsq_kernel(const cdml_param *__restrict__ params,
                                                    int count, float prescale,
                                                    float *__restrict__ partial) {
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int t = 0; t < count; ++t) {
    const float *g = params[t].grad;
    const long long n = params[t].count;
    float s = 0.f;
    if ((reinterpret_cast<uintptr_t>(g) & 15) == 0) {
      const long long n4 = n >> 2;
      for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n4; e += (long long)kNormBlocks * 256) {
        const vf4 x = reinterpret_cast<const vf4 *>(g)[e];
        const float a0 = x[0] * prescale, a1 = x[1] * prescale, a2 = x[2] * prescale, a3 = x[3] * prescale;
        s += ((a0 * a0 + a1 * a1) + a2 * a2) + a3 * a3;
      }
      for (long long e = (n4 << 2) + (long long)blockIdx.x * 256 + threadIdx.x; e < n;
           e += (long long)kNormBlocks * 256) {
        const float a = g[e] * prescale;
        s += a * a;
      }
    } else {
      for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long long)kNormBlocks * 256) {
        const float a = g[e] * prescale;
        s += a * a;
      }
    }
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) partial[(size_t)t * kNormBlocks + blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
  }
}

// ComputeGradientNorm + ClipGradients (TransformerTrainer.cs:1306-1352): the
// per-tensor sums in block order, tensors with equal consecutive group ids
// summed first (the trainer adds WQ + WK + WV + WO before adding them to the
// total), norm = sqrt(total).  result[0] = norm, result[1] = the clipping
// factor (threshold / norm when clipping and norm > threshold, else 1),
// result[2] = 1 when the norm is finite (the update runs), else 0.
__global__ void __launch_bounds__(64) norm_finalize_kernel(const cdml_param *__restrict__ params,
                                                           int count,
                                                           const float *__restrict__ partial,
                                                           int use_clipping, float threshold,
                                                           float *__restrict__ result) {
  __shared__ float tensor_sum[64];
  float total = 0.f, group_sum = 0.f;
  int group = 0;
  for (int t0 = 0; t0 < count; t0 += 64) {
    const int t = t0 + threadIdx.x;
    if (t < count) {
      float s = 0.f;
      for (int b = 0; b < kNormBlocks; ++b) s += partial[(size_t)t * kNormBlocks + b];
      tensor_sum[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int i = 0; i < 64 && t0 + i < count; ++i) {
        const int g = params[t0 + i].group;
        if (t0 + i == 0) {
          group = g;
          group_sum = tensor_sum[i];
        } else if (g == group) {
          group_sum += tensor_sum[i];
        } else {
          total += group_sum;
          group = g;
          group_sum = tensor_sum[i];
        }
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (count > 0) total += group_sum;
    const float norm = sqrtf(total);
    const bool finite = isfinite(norm);
    result[0] = norm;
    result[1] = (use_clipping && finite && norm > threshold) ? threshold / norm : 1.f;
    result[2] = finite ? 1.f : 0.f;
  }
}

// UpdateParameters (TransformerTrainer.cs:1269-1305, MatrixUpdate
// AccelerationCPU.cs:2548-2597): g' = (g * prescale) * clip (the in-place
// ScaleGradients calls, the second only when clipping applied), w -= lr * g'.
// With a non-finite norm nothing is updated (TransformerTrainer.cs:316-320).
// zero_grads: the gradients are cleared for the next step (ZeroAllGradients);
// otherwise g' is written back, as the reference's in-place scaling leaves it.
__global__ void __launch_bounds__(256) sgd_kernel(const cdml_param *__restrict__ params, int count,
                                                  float lr, float prescale,
                                                  const float *__restrict__ result, int zero_grads) {
#pragma clang fp contract(off)
  const bool run = result[2] != 0.f;
  const float clip = result[1];
  const bool clipped = clip != 1.f;
  const long long stride = (long long)gridDim.x * 256;
  for (int t = 0; t < count; ++t) {
    float *w = params[t].weight, *g = params[t].grad;
    const long long n = params[t].count;
    for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
      float gs = g[e] * prescale;
      if (clipped) gs = gs * clip;
      if (run) w[e] -= lr * gs;  // multiply and subtract rounded separately, as MatrixUpdate
      g[e] = zero_grads ? 0.f : gs;
    }
  }
}

// MatrixUpdate / VectorUpdate (AccelerationCPU.cs:2548-2597): w -= lr * g,
// the product and the difference rounded separately as in the reference.
__global__ void __launch_bounds__(256) update_kernel(float *__restrict__ w, const float *__restrict__ g,
                                                     float lr, long long n) {
#pragma clang fp contract(off)
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    w[i] -= lr * g[i];
}

// MatrixScaleInPlace / VectorScaleInPlace (AccelerationCPU.cs:2514-2546).
__global__ void __launch_bounds__(256) scale_kernel(float *__restrict__ x, float a, long long n) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    x[i] *= a;
}

// MatrixSquaredNorm / VectorSquaredNorm (AccelerationCPU.cs:2493-2512): block
// b sums the squares of elements b * 256 + t + k * kNormBlocks * 256 into a
// partial; one wave then adds the partials in block order.
__global__ void __launch_bounds__(256) sq_partial_kernel(const float *__restrict__ x, long long n,
                                                         float *__restrict__ partial) {
  __shared__ float red[4];
  float s = 0.f;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)kNormBlocks * 256)
    s += x[i] * x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

__global__ void __launch_bounds__(64) sq_final_kernel(const float *__restrict__ partial,
                                                      float *__restrict__ out) {
  float s = 0.f;
  for (int b = threadIdx.x; b < kNormBlocks; b += 64) s += partial[b];
  s = wave_sum(s);
  if (threadIdx.x == 0) out[0] = s;
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_update_f32(float *weights, const float *gradients, float learning_rate, size_t count,
                               cdml_stream stream) {
  if (count == 0) return CDML_OK;
  if (!weights || !gradients) return fail(CDML_E_INVALID, "cdml_update_f32: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  const size_t blocks = std::min<size_t>((count + 255) / 256, 8192);
  update_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(weights, gradients, learning_rate,
                                                                         (long long)count);
  return check_launch("update_kernel");
}

extern "C" int cdml_scale_f32(float *x, float scale, size_t count, cdml_stream stream) {
  if (count == 0) return CDML_OK;
  if (!x) return fail(CDML_E_INVALID, "cdml_scale_f32: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  const size_t blocks = std::min<size_t>((count + 255) / 256, 8192);
  scale_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(x, scale, (long long)count);
  return check_launch("scale_kernel");
}

extern "C" int cdml_sum_squares_workspace_size(size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_sum_squares_workspace_size: bytes is NULL");
  *bytes = (size_t)kNormBlocks * sizeof(float);
  return CDML_OK;
}

extern "C" int cdml_sum_squares(const float *x, size_t count, float *out, void *workspace,
                                size_t workspace_bytes, cdml_stream stream) {
  if (!out) return fail(CDML_E_INVALID, "cdml_sum_squares: out is NULL");
  if (count > 0 && !x) return fail(CDML_E_INVALID, "cdml_sum_squares: x is NULL");
  if (!workspace || workspace_bytes < (size_t)kNormBlocks * sizeof(float))
    return fail(CDML_E_INVALID, "cdml_sum_squares: workspace of %zu bytes needed",
                (size_t)kNormBlocks * sizeof(float));
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  float *partial = static_cast<float *>(workspace);
  sq_partial_kernel<<<dim3(kNormBlocks), dim3(256), 0, st>>>(x, (long long)count, partial);
  rc = check_launch("sq_partial_kernel");
  if (rc) return rc;
  sq_final_kernel<<<dim3(1), dim3(64), 0, st>>>(partial, out);
  return check_launch("sq_final_kernel");
}

extern "C" int cdml_residual_layernorm_fwd(const float *a, const float *b, const float *gamma,
                                           const float *beta, float *out, float *mean,
                                           float *variance, float *residual, float *normalized,
                                           int rows, int features, float eps,
                                           cdml_stream stream) {
  if (rows < 0 || features < 0)
    return fail(CDML_E_INVALID, "cdml_residual_layernorm_fwd: negative size");
  if (rows == 0 || features == 0) return CDML_OK;
  if (!a || !b || !gamma || !beta || !out)
    return fail(CDML_E_INVALID, "cdml_residual_layernorm_fwd: NULL pointer");
  if (features > 64 * kRowCache)
    return fail(CDML_E_INVALID, "cdml_residual_layernorm_fwd: more than %d features", 64 * kRowCache);
  int rc = ensure_device();
  if (rc) return rc;
  const dim3 grid((rows + 3) / 4), block(256);
  hipStream_t st = as_hip(stream);
  const int rcache = row_cache(features);
  const bool v4 = rcache >= 4 && features % 4 == 0 && aligned16(a) && aligned16(b) && aligned16(gamma) &&
                  aligned16(beta) && aligned16(out) && (!residual || aligned16(residual)) &&
                  (!normalized || aligned16(normalized));
#define CDML_LN_FWD(RC, V) ln_forward_kernel<RC, V><<<grid, block, 0, st>>>(a, b, gamma, beta, out, mean, variance, residual, normalized, rows, features, eps)
  if (v4) {
    switch (rcache) {
      case 4: CDML_LN_FWD(4, true); break;
      case 8: CDML_LN_FWD(8, true); break;
      case 16: CDML_LN_FWD(16, true); break;
      default: CDML_LN_FWD(32, true); break;
    }
  } else {
    switch (rcache) {
      case 1: CDML_LN_FWD(1, false); break;
      case 2: CDML_LN_FWD(2, false); break;
      case 4: CDML_LN_FWD(4, false); break;
      case 8: CDML_LN_FWD(8, false); break;
      case 16: CDML_LN_FWD(16, false); break;
      default: CDML_LN_FWD(32, false); break;
    }
  }
#undef CDML_LN_FWD
  return check_launch("ln_forward_kernel");
}

extern "C" int cdml_layernorm_backward_workspace_size(int rows, int features, size_t *bytes) {
  if (!bytes || rows < 0 || features < 0)
    return fail(CDML_E_INVALID, "cdml_layernorm_backward_workspace_size: bad argument");
  const size_t nblk = features > 0 ? (size_t)ln_blocks(rows, features) : 0;
  const size_t slices = nblk > (size_t)4 * kLnSlices ? kLnSlices : 0;
  *bytes = 2 * (nblk + slices) * (size_t)features * sizeof(float);
  return CDML_OK;
}

extern "C" int cdml_layernorm_backward(const float *dout, const float *dout2,
                                       const float *normalized, const float *gamma,
                                       const float *input, const float *mean,
                                       const float *variance, float *dinput, float *dgamma,
                                       float *dbeta, int rows, int features, float eps,
                                       int accumulate, void *workspace, size_t workspace_bytes,
                                       cdml_stream stream) {
  if (rows < 0 || features < 0)
    return fail(CDML_E_INVALID, "cdml_layernorm_backward: negative size");
  if (features == 0) return CDML_OK;
  if (features > 64 * kRowCache)
    return fail(CDML_E_INVALID, "cdml_layernorm_backward: more than %d features", 64 * kRowCache);
  if (!dout || !gamma || !input || !mean || !variance || !dinput)
    return fail(CDML_E_INVALID, "cdml_layernorm_backward: NULL pointer");
  size_t need = 0;
  cdml_layernorm_backward_workspace_size(rows, features, &need);
  if (need && (!workspace || workspace_bytes < need))
    return fail(CDML_E_INVALID, "cdml_layernorm_backward: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  const int nblk = ln_blocks(rows, features);
  float *pg = static_cast<float *>(workspace), *pb = pg + (size_t)nblk * features;
  const int rcache = row_cache(features);
  const bool vec = rcache >= 4 && features % 4 == 0 && aligned16(dout) && (!dout2 || aligned16(dout2)) &&
                   (!normalized || aligned16(normalized)) && aligned16(gamma) && aligned16(input) &&
                   aligned16(dinput) && aligned16(pg);
  if (rows > 0 && vec) {
#define CDML_LN_BWDV(RC) ln_backward_vec_kernel<RC / 4, ln_waves(RC), ln_block_rows(RC)><<<dim3(nblk), dim3(64 * ln_waves(RC)), 0, st>>>(dout, dout2, normalized, gamma, input, mean, variance, dinput, pg, pb, rows, features, eps)
    switch (rcache) {
      case 4: CDML_LN_BWDV(4); break;
      case 8: CDML_LN_BWDV(8); break;
      case 16: CDML_LN_BWDV(16); break;
      default: CDML_LN_BWDV(32); break;
    }
#undef CDML_LN_BWDV
    rc = check_launch("ln_backward_vec_kernel");
    if (rc) return rc;
  } else if (rows > 0) {
#define CDML_LN_BWD(RC) ln_backward_kernel<RC><<<dim3(nblk), dim3(64 * ln_waves(RC)), 0, st>>>(dout, dout2, normalized, gamma, input, mean, variance, dinput, pg, pb, rows, features, eps)
    switch (rcache) {
      case 1: CDML_LN_BWD(1); break;
      case 2: CDML_LN_BWD(2); break;
      case 4: CDML_LN_BWD(4); break;
      case 8: CDML_LN_BWD(8); break;
      case 16: CDML_LN_BWD(16); break;
      default: CDML_LN_BWD(32); break;
    }
#undef CDML_LN_BWD
    rc = check_launch("ln_backward_kernel");
    if (rc) return rc;
  }
  if (dgamma || dbeta) {
    const int slices = ln_slices(nblk);
    if (slices) {  // many row blocks: sum slices of them on many CUs first
      float *sg = pb + (size_t)nblk * features, *sb = sg + (size_t)slices * features;
      const int chunk = (nblk + slices - 1) / slices;
      ln_param_slice_kernel<<<dim3((features + 63) / 64, slices), dim3(256), 0, st>>>(pg, pb, sg, sb, nblk,
                                                                                      chunk, features);
      rc = check_launch("ln_param_slice_kernel");
      if (rc) return rc;
      ln_param_grad_kernel<<<dim3((features + 63) / 64), dim3(1024), 0, st>>>(sg, sb, dgamma, dbeta, slices,
                                                                              features, accumulate);
    } else {
      ln_param_grad_kernel<<<dim3((features + 63) / 64), dim3(1024), 0, st>>>(pg, pb, dgamma, dbeta, nblk,
                                                                              features, accumulate);
    }
    rc = check_launch("ln_param_grad_kernel");
  }
  return rc;
}

extern "C" int cdml_cross_entropy_workspace_size(int rows, size_t *bytes) {
  if (!bytes || rows < 0) return fail(CDML_E_INVALID, "cdml_cross_entropy_workspace_size: bad argument");
  *bytes = (size_t)(rows > 0 ? rows : 1) * sizeof(float);
  return CDML_OK;
}

extern "C" int cdml_cross_entropy(const float *logits, int ldl, const int *targets, int rows,
                                  int out_dim, int effective_len, float grad_scale,
                                  float loss_scale, float *loss, float *dlogits, int lddl,
                                  void *workspace, size_t workspace_bytes, cdml_stream stream) {
  if (rows < 0 || out_dim <= 0 || effective_len < 0 || effective_len > rows)
    return fail(CDML_E_INVALID, "cdml_cross_entropy: bad size");
  if (ldl < out_dim || lddl < out_dim)
    return fail(CDML_E_INVALID, "cdml_cross_entropy: row stride smaller than the row");
  if (!logits || !dlogits || !loss || (effective_len > 0 && !targets))
    return fail(CDML_E_INVALID, "cdml_cross_entropy: NULL pointer");
  if (!workspace || workspace_bytes < (size_t)(rows > 0 ? rows : 1) * sizeof(float))
    return fail(CDML_E_INVALID, "cdml_cross_entropy: workspace too small");
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  float *row_loss = static_cast<float *>(workspace);
  if (rows > 0) {
    ce_row_kernel<<<dim3(rows), dim3(256), 0, st>>>(logits, ldl, targets, rows, out_dim, effective_len,
                                                    grad_scale, dlogits, lddl, row_loss);
    rc = check_launch("ce_row_kernel");
    if (rc) return rc;
  }
  if (effective_len == 0) return cdml_zero_f32_async(loss, 1, stream);
  ce_loss_kernel<<<dim3(1), dim3(1024), 0, st>>>(row_loss, effective_len, (float)effective_len, loss_scale,
                                                 loss);
  return check_launch("ce_loss_kernel");
}

extern "C" int cdml_mse_loss(const float *pred, int ldp, const float *targets, int ldt, int rows,
                             int out_dim, int effective_len, float grad_scale, float loss_scale,
                             float *loss, float *dout, int ldd, void *workspace,
                             size_t workspace_bytes, cdml_stream stream) {
  if (rows < 0 || out_dim <= 0 || effective_len < 0 || effective_len > rows)
    return fail(CDML_E_INVALID, "cdml_mse_loss: bad size");
  if (ldp < out_dim || ldt < out_dim || ldd < out_dim)
    return fail(CDML_E_INVALID, "cdml_mse_loss: row stride smaller than the row");
  if (!pred || !dout || !loss || (effective_len > 0 && !targets))
    return fail(CDML_E_INVALID, "cdml_mse_loss: NULL pointer");
  if (!workspace || workspace_bytes < (size_t)(rows > 0 ? rows : 1) * sizeof(float))
    return fail(CDML_E_INVALID, "cdml_mse_loss: workspace too small");
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  float *row_loss = static_cast<float *>(workspace);
  if (rows > 0) {
    mse_row_kernel<<<dim3((rows + 255) / 256), dim3(256), 0, st>>>(pred, ldp, targets, ldt, rows, out_dim,
                                                                  effective_len, grad_scale, dout, ldd,
                                                                  row_loss);
    rc = check_launch("mse_row_kernel");
    if (rc) return rc;
  }
  if (effective_len == 0) return cdml_zero_f32_async(loss, 1, stream);
  ce_loss_kernel<<<dim3(1), dim3(1024), 0, st>>>(row_loss, effective_len, (float)(effective_len * out_dim),
                                                 loss_scale, loss);
  return check_launch("ce_loss_kernel");
}

extern "C" int cdml_add_inplace(float *target, const float *addend, size_t count, cdml_stream stream) {
  if (count == 0) return CDML_OK;
  if (!target || !addend) return fail(CDML_E_INVALID, "cdml_add_inplace: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  const size_t blocks = std::min<size_t>((count + 255) / 256, 8192);
  add_inplace_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(target, addend, (long long)count);
  return check_launch("add_inplace_kernel");
}

extern "C" int cdml_embedding_grad(float *grad, const float *dx, const float *dx2, int ldx,
                                   const int *order, const int *group_start,
                                   const int *group_token, int n_groups, int dim,
                                   cdml_stream stream) {
  if (n_groups < 0 || dim < 0 || ldx < dim) return fail(CDML_E_INVALID, "cdml_embedding_grad: bad size");
  if (n_groups == 0 || dim == 0) return CDML_OK;
  if (!grad || !dx || !order || !group_start || !group_token)
    return fail(CDML_E_INVALID, "cdml_embedding_grad: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  embed_grad_kernel<<<dim3(n_groups, (dim + 255) / 256), dim3(256), 0, as_hip(stream)>>>(
      grad, dx, dx2, ldx, order, group_start, group_token, dim);
  return check_launch("embed_grad_kernel");
}

extern "C" int cdml_grad_norm_workspace_size(int count, size_t *bytes) {
  if (!bytes || count < 0) return fail(CDML_E_INVALID, "cdml_grad_norm_workspace_size: bad argument");
  *bytes = (size_t)(count > 0 ? count : 1) * kNormBlocks * sizeof(float);
  return CDML_OK;
}

extern "C" int cdml_grad_norm(const cdml_param *params, int count, float prescale,
                              int use_clipping, float threshold, float *result, void *workspace,
                              size_t workspace_bytes, cdml_stream stream) {
  if (count < 0) return fail(CDML_E_INVALID, "cdml_grad_norm: negative count");
  if (!params || !result) return fail(CDML_E_INVALID, "cdml_grad_norm: NULL pointer");
  if (use_clipping && !(threshold > 0.f && std::isfinite(threshold)))
    return fail(CDML_E_INVALID, "cdml_grad_norm: clip threshold must be finite and positive");
  size_t need = 0;
  cdml_grad_norm_workspace_size(count, &need);
  if (!workspace || workspace_bytes < need)
    return fail(CDML_E_INVALID, "cdml_grad_norm: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  float *partial = static_cast<float *>(workspace);
  if (count > 0) {
    sumsq_kernel<<<dim3(kNormBlocks), dim3(256), 0, st>>>(params, count, prescale, partial);
    rc = check_launch("sumsq_kernel");
    if (rc) return rc;
  }
  norm_finalize_kernel<<<dim3(1), dim3(64), 0, st>>>(params, count, partial, use_clipping, threshold,
                                                     result);
  return check_launch("norm_finalize_kernel");
}

extern "C" int cdml_sgd_update(const cdml_param *params, int count, float learning_rate,
                               float prescale, const float *result, int zero_grads,
                               cdml_stream stream) {
  if (count < 0) return fail(CDML_E_INVALID, "cdml_sgd_update: negative count");
  if (count == 0) return CDML_OK;
  if (!params || !result) return fail(CDML_E_INVALID, "cdml_sgd_update: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  sgd_kernel<<<dim3(2048), dim3(256), 0, as_hip(stream)>>>(params, count, learning_rate, prescale, result,
                                                            zero_grads);
  return check_launch("sgd_kernel");
}
