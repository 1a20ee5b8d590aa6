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
#define CDML_RLN(RC) residual_ln_kernel<RC><<<grid, block, 0, st>>>(a, b, gamma, beta, y, rows, features, eps)
  switch (row_cache(features)) {
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
