// Issue-rate probe for gfx950 (standalone program, not part of the library):
// how long one SIMD takes per v_mfma_f32_32x32x2_f32 when the MFMAs are
// dependent, when VALU instructions of several kinds sit between them, and
// when their A operands come from LDS.  The flash kernels' instruction budget
// is set from these figures.  Every workgroup is 256 threads (4 waves) and
// 1024 workgroups fill 256 CUs with 4 waves per SIMD unless stated.
//
// Build and run (profile_bench.py --passes probe does both):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         issue_rates.hip -o issue_rates && ./issue_rates
// Output: one line per case, "<case> <cycles per step per SIMD>", cycles at
// the 2.4 GHz peak clock from event time.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float vf4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));        \
      std::exit(1);                                                       \
    }                                                                     \
  } while (0)

__device__ __forceinline__ floatx16 mf(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// CH independent accumulator chains, 32 MFMAs per iteration.
template <int CH>
__global__ void __launch_bounds__(256) chains(float *out, int iters, float x) {
  floatx16 acc[CH];
  for (int c = 0; c < CH; ++c)
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
  const float a = x + threadIdx.x, b = x * 2.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 32 / CH; ++s)
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[c] = mf(a, b, acc[c]);
  }
  float s = 0.f;
  for (int c = 0; c < CH; ++c)
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// Per step: one MFMA (if MFMA) and N independent VALU instructions of KIND
// (0 add, 1 exp2, 2 max3, 3 fma) spread over 8 registers.
template <int KIND, int N, bool MFMA>
__global__ void __launch_bounds__(256) valu_mix(float *out, int iters, float x) {
  floatx16 acc;
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  const float a = x + threadIdx.x, b = x * 2.f, c = x * 0.25f;
  float v[8];
  for (int i = 0; i < 8; ++i) v[i] = x + i * threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      if (MFMA) acc = mf(a, b, acc);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float &t = v[j & 7];
        if (KIND == 0) t = t + c;
        else if (KIND == 1) t = __builtin_amdgcn_exp2f(t);
        else if (KIND == 2) t = __builtin_fmaxf(__builtin_fmaxf(t, c), v[(j + 1) & 7]);
        else t = t * c + 1.0f;
      }
    }
  }
  float s = 0.f;
  for (int r = 0; r < 16; ++r) s += acc[r];
  for (int i = 0; i < 8; ++i) s += v[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// A softmax-like mix: a dependent chain of 16 MFMAs, then a burst of 48
// independent adds (BURST), or the MFMAs alone (MFMA_ONLY), or the adds alone.
template <bool MFMA, bool ADDS>
__global__ void __launch_bounds__(256) burst(float *out, int iters, float x) {
  floatx16 acc;
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  const float a = x + threadIdx.x, b = x * 2.f, c = x * 0.25f;
  float v[8];
  for (int i = 0; i < 8; ++i) v[i] = x + i * threadIdx.x;
  for (int it = 0; it < iters; ++it) {
    if (MFMA) {
#pragma unroll
      for (int s = 0; s < 16; ++s) acc = mf(a, b, acc);
    }
    if (ADDS) {
#pragma unroll
      for (int j = 0; j < 48; ++j) v[j & 7] = v[j & 7] + c;
    }
  }
  float s = 0.f;
  for (int r = 0; r < 16; ++r) s += acc[r];
  for (int i = 0; i < 8; ++i) s += v[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// MFMA A operands read from LDS one group of four ahead: KIND 0 one 16-byte
// read of four consecutive keys of a column (a transposed tile), KIND 1 four
// 4-byte reads of four rows, KIND 2 registers only.
template <int KIND>
__global__ void __launch_bounds__(256) lds_operands(float *out, int iters, float x) {
  __shared__ __attribute__((aligned(16))) float lds[64 * 68 * 2];
  for (int i = threadIdx.x; i < 64 * 68 * 2; i += 256) lds[i] = x * (i & 255);
  __syncthreads();
  floatx16 acc;
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  const float b = x * 2.f;
  const int lane = threadIdx.x & 63, li = lane & 31, hf = lane >> 5;
  vf4 cur = {x, x, x, x};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      vf4 nxt;
      const int row = (it * 16 + g) & 63;
      if (KIND == 0) {
        nxt = *reinterpret_cast<const vf4 *>(&lds[li * 68 + ((row * 8 + 4 * hf) & 63)]);
      } else if (KIND == 1) {
        const float *p = &lds[(row & 31) * 36 + 4 * hf * 36 + li];
        nxt = vf4{p[0], p[36], p[72], p[108]};
      } else {
        nxt = vf4{cur.y + b, cur.z, cur.w, cur.x};
      }
      acc = mf(cur.x, b, acc);
      acc = mf(cur.y, b, acc);
      acc = mf(cur.z, b, acc);
      acc = mf(cur.w, b, acc);
      cur = nxt;
    }
  }
  float s = 0.f;
  for (int r = 0; r < 16; ++r) s += acc[r];
  out[blockIdx.x * 256 + threadIdx.x] = s + cur.x;
}

template <typename F>
static double time_ms(F launch) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int w = 0; w < 3; ++w) launch();
  CHECK(hipEventRecord(e0));
  const int reps = 5;
  for (int w = 0; w < reps; ++w) launch();
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  return ms / reps;
}

// cycles per step per SIMD at 2.4 GHz: steps = wgs * 4 waves * per-wave steps / 1024 SIMDs
static double cycles(double ms, int wgs, double steps_per_wave) {
  return ms * 1e-3 * 2.4e9 / ((double)wgs * 4 * steps_per_wave / 1024);
}

int main() {
  float *out = nullptr;
  CHECK(hipMalloc(&out, 1024 * 256 * sizeof(float)));
  const int iters = 100;
  for (int wgs : {256, 512, 1024}) {
    double m1 = time_ms([&] { chains<1><<<wgs, 256>>>(out, iters, 1e-3f); });
    double m4 = time_ms([&] { chains<4><<<wgs, 256>>>(out, iters, 1e-3f); });
    std::printf("mfma_dependent_chain waves_per_simd=%d %.1f\n", wgs / 256, cycles(m1, wgs, iters * 32.0));
    std::printf("mfma_4_chains waves_per_simd=%d %.1f\n", wgs / 256, cycles(m4, wgs, iters * 32.0));
  }
#define MIX(K, NN, M, name)                                                                    \
  std::printf("%s n=%d mfma=%d %.1f\n", name, NN, (int)M,                                      \
              cycles(time_ms([&] { valu_mix<K, NN, M><<<1024, 256>>>(out, iters, 1e-3f); }), 1024, \
                     iters * 32.0))
  MIX(0, 8, false, "v_add_f32");
  MIX(1, 8, false, "v_exp_f32");
  MIX(2, 8, false, "v_max3_f32");
  MIX(3, 8, false, "v_fma_f32");
  MIX(0, 0, true, "mfma_only");
  MIX(0, 4, true, "v_add_f32");
  MIX(0, 16, true, "v_add_f32");
  MIX(1, 4, true, "v_exp_f32");
  MIX(1, 8, true, "v_exp_f32");
  MIX(2, 8, true, "v_max3_f32");
  MIX(3, 8, true, "v_fma_f32");
#undef MIX
  for (int wgs : {256, 512, 1024}) {
    const int it = 200;
    std::printf("16_mfma_then_48_adds waves_per_simd=%d %.1f\n", wgs / 256,
                cycles(time_ms([&] { burst<true, true><<<wgs, 256>>>(out, it, 1e-3f); }), wgs, it));
    std::printf("16_mfma_only waves_per_simd=%d %.1f\n", wgs / 256,
                cycles(time_ms([&] { burst<true, false><<<wgs, 256>>>(out, it, 1e-3f); }), wgs, it));
    std::printf("48_adds_only waves_per_simd=%d %.1f\n", wgs / 256,
                cycles(time_ms([&] { burst<false, true><<<wgs, 256>>>(out, it, 1e-3f); }), wgs, it));
  }
  const char *lds_names[] = {"lds_b128_transposed", "lds_b32_rows", "registers"};
  for (int k = 0; k < 3; ++k) {
    double ms = 0;
    if (k == 0) ms = time_ms([&] { lds_operands<0><<<1024, 256>>>(out, 50, 1e-3f); });
    if (k == 1) ms = time_ms([&] { lds_operands<1><<<1024, 256>>>(out, 50, 1e-3f); });
    if (k == 2) ms = time_ms([&] { lds_operands<2><<<1024, 256>>>(out, 50, 1e-3f); });
    std::printf("mfma_operands_from_%s %.1f\n", lds_names[k], cycles(ms, 1024, 50 * 64.0));
  }
  CHECK(hipFree(out));
  return 0;
}
