// Fused residual add + LayerNorm (AccelerationCPU.cs:1376-1438):
//   s = a + b;  y = gamma * (s - mean(s)) / sqrt(var(s) + eps) + beta
// with the biased variance, computed in two passes over the row as the
// reference does.  One wave per row; rows up to 64 * ROW_CACHE features keep
// the residual sum in registers between the passes.
#include "common.h"

namespace cdml {
namespace {

// Row-cache size: the smallest power of two with 64 * RC >= features (up to
// 32); longer rows are re-read in the second and third passes.
inline int row_cache(int f) {
  int rc = 1;
  while (64 * rc < f && rc < 32) rc <<= 1;
  return rc;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// With V4 (features % 4 == 0, 16-byte aligned rows, every row cached, at
// least 4 cached values per lane) lane l holds columns 256 i + 4 l .. + 3, so
// every access moves a float4.
template <int ROW_CACHE>
__global__ void __launch_bounds__(256) residual_ln_v4_kernel(const float *__restrict__ a,
                                                             const float *__restrict__ b,
                                                             const float *__restrict__ gamma,
                                                             const float *__restrict__ beta,
                                                             float *__restrict__ y, int rows, int f,
                                                             float eps) {
  constexpr int R4 = ROW_CACHE / 4;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const size_t base = (size_t)row * f;
  vf4 cache[R4];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < R4; ++i) {
    const int j = 256 * i + 4 * lane;
    cache[i] = vf4{0.f, 0.f, 0.f, 0.f};
    if (j < f) cache[i] = *reinterpret_cast<const vf4 *>(a + base + j) + *reinterpret_cast<const vf4 *>(b + base + j);
    sum += (cache[i][0] + cache[i][1]) + (cache[i][2] + cache[i][3]);
  }
  const float mean = wave_sum(sum) / (float)f;
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < R4; ++i) {
    if (256 * i + 4 * lane >= f) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float d = cache[i][c] - mean;
      var += d * d;
    }
  }
  var = wave_sum(var) / (float)f;
  const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < R4; ++i) {
    const int j = 256 * i + 4 * lane;
    if (j >= f) continue;
    const vf4 g = *reinterpret_cast<const vf4 *>(gamma + j), be = *reinterpret_cast<const vf4 *>(beta + j);
    vf4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = g[c] * ((cache[i][c] - mean) * inv_std) + be[c];
    *reinterpret_cast<vf4 *>(y + base + j) = o;
  }
}

template <int ROW_CACHE>
__global__ void __launch_bounds__(256) residual_ln_kernel(const float *__restrict__ a,
                                                          const float *__restrict__ b,
                                                          const float *__restrict__ gamma,
                                                          const float *__restrict__ beta,
                                                          float *__restrict__ y, int rows, int f,
                                                          float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float *ar = a + (size_t)row * f;
  const float *br = b + (size_t)row * f;
  float *yr = y + (size_t)row * f;
  const bool cached = f <= 64 * ROW_CACHE;
  float cache[ROW_CACHE];
  float sum = 0.f;
  if (cached) {
#pragma unroll
    for (int i = 0; i < ROW_CACHE; ++i) {
      const int j = lane + 64 * i;
      cache[i] = j < f ? ar[j] + br[j] : 0.f;
      sum += cache[i];
    }
  } else {
    for (int j = lane; j < f; j += 64) sum += ar[j] + br[j];
  }
  const float mean = wave_sum(sum) / (float)f;
  float var = 0.f;
  if (cached) {
#pragma unroll
    for (int i = 0; i < ROW_CACHE; ++i) {
      const int j = lane + 64 * i;
      const float d = cache[i] - mean;
      var += j < f ? d * d : 0.f;
    }
  } else {
    for (int j = lane; j < f; j += 64) {
      const float d = (ar[j] + br[j]) - mean;
      var += d * d;
    }
  }
  var = wave_sum(var) / (float)f;
  const float inv_std = 1.0f / sqrtf(var + eps);
  if (cached) {
#pragma unroll
    for (int i = 0; i < ROW_CACHE; ++i) {
      const int j = lane + 64 * i;
      if (j < f) yr[j] = gamma[j] * ((cache[i] - mean) * inv_std) + beta[j];
    }
  } else {
    for (int j = lane; j < f; j += 64)
      yr[j] = gamma[j] * (((ar[j] + br[j]) - mean) * inv_std) + beta[j];
  }
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_residual_layernorm(const float *a, const float *b, const float *gamma,
                                       const float *beta, float *y, int rows, int features,
                                       float eps, cdml_stream stream) {
  if (rows < 0 || features < 0) return fail(CDML_E_INVALID, "cdml_residual_layernorm: negative size");
  if (rows == 0 || features == 0) return CDML_OK;
  if (!a || !b || !gamma || !beta || !y)
    return fail(CDML_E_INVALID, "cdml_residual_layernorm: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  const dim3 grid((rows + 3) / 4), block(256);
  hipStream_t st = as_hip(stream);
  const int rcache = row_cache(features);
  if (rcache >= 4 && features <= 64 * rcache && features % 4 == 0 && aligned16(a) && aligned16(b) &&
      aligned16(gamma) && aligned16(beta) && aligned16(y)) {
#define CDML_RLN4(RC) residual_ln_v4_kernel<RC><<<grid, block, 0, st>>>(a, b, gamma, beta, y, rows, features, eps)
    switch (rcache) {
      case 4: CDML_RLN4(4); break;
      case 8: CDML_RLN4(8); break;
      case 16: CDML_RLN4(16); break;
      default: CDML_RLN4(32); break;
    }
#undef CDML_RLN4
    return check_launch("residual_ln_v4_kernel");
  }
#define CDML_RLN(RC) residual_ln_kernel<RC><<<grid, block, 0, st>>>(a, b, gamma, beta, y, rows, features, eps)
  switch (rcache) {
    case 1: CDML_RLN(1); break;
    case 2: CDML_RLN(2); break;
    case 4: CDML_RLN(4); break;
    case 8: CDML_RLN(8); break;
    case 16: CDML_RLN(16); break;
    default: CDML_RLN(32); break;
  }
#undef CDML_RLN
  return check_launch("residual_ln_kernel");
}
