// Shared helpers for the gfx950 kernels and the C-ABI implementation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "cdml.h"

namespace cdml {

// Thread-local last-error message (cdml_last_error()).
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);

// Makes the library's device current on the calling thread.
int ensure_device();

// Finds this device's copy of the static scratch behind the no-allocation
// entry points (hipGetSymbolAddress); called by cdml_init with `device`
// current.  It does not touch the thread's last error: a failure is
// described in `msg` and reported by the entry point that needs the scratch.
int noalloc_scratch_setup(int device, char *msg, size_t msg_bytes);

// Compute units of the current device (queried once; 256 on MI355X).
int num_cus();

// Checks the launch that was just enqueued.
int check_launch(const char *what);

inline hipStream_t as_hip(cdml_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch geometry for gfx950: 8 XCDs, and hardware hands workgroup i to XCD
// i % 8.  xcd_remap() turns the hardware id into a logical id such that each
// XCD receives one contiguous range of logical work, so neighbouring tiles
// (same head, same weight panel) share an L2.
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int hw_id, int padded_total) {
  const int per_xcd = padded_total / kNumXcd;
  return (hw_id % kNumXcd) * per_xcd + hw_id / kNumXcd;
}

inline int pad_to_xcd(int n) { return (n + kNumXcd - 1) / kNumXcd * kNumXcd; }

// fp32 MFMA 32x32x2: D = A(32x2) * B(2x32) + C, one block.
// Operand layout (lane l, half h = l / 32):
//   A[i][k]: i = l % 32, k = h      B[k][j]: j = l % 32, k = h
//   D[i][j]: j = l % 32, i = 8*(r/4) + 4*h + (r%4) for accumulator r = 0..15
typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native 4-float vector for register staging: unlike HIP's float4 struct it
// is always kept in registers (no private-memory copies of staging arrays).
typedef float vf4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx16 mfma32x32x2(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The forward attention launcher (flash_attn.hip) for callers that have
// validated their arguments.  With lse non-NULL it also writes each row's
// log2 softmax normaliser ([batch * heads][lq]; head dims up to 128).
// causal: key j is visible to query i iff j <= i (lq may differ from lk).
int flash_forward(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                  float *o, int ldo, float *lse, int batch, int lq, int lk, int dim, int num_heads,
                  float scale, bool causal, const uint8_t *mask, hipStream_t st);

}  // namespace cdml
