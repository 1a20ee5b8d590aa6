// Interleaved-pair rotary position embedding, in place
// (AccelerationCPU.cs:4929-4980, LanguageModel.cs:432-480,
// TransformerTrainer.cs:811-848).
//
// The per-pair denominators powf(base, 2p / head_dim) are computed on the host
// with the same float expression as the reference and passed by value, so
// every device thread forms theta = pos / denom[p] from bit-identical
// operands (the rotation angle reaches thousands of radians at long
// positions, where a one-ulp difference in denom would show in sin/cos).
#include <algorithm>
#include <cmath>

#include "common.h"

namespace cdml {
namespace {

constexpr int kMaxPairs = 256;

struct RopeArgs {
  float *x;
  const int *positions;
  int rows, ld, start_col, head_dim, num_heads, pairs;
  int inverse, pos_offset, seg_len;
  float denom[kMaxPairs];
};

__global__ void __launch_bounds__(256) rope_kernel(const RopeArgs a) {
  // (x0 cos) - (x1 sin) with both products rounded, as the reference
  // evaluates it: no fused multiply-add
#pragma clang fp contract(off)
  const long long total = (long long)a.rows * a.num_heads * a.pairs;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int p = (int)(idx % a.pairs);
    const long long rh = idx / a.pairs;
    const int head = (int)(rh % a.num_heads);
    const int row = (int)(rh / a.num_heads);
    int pos;
    if (a.positions) pos = a.positions[row];
    else pos = a.pos_offset + (a.seg_len > 0 ? row % a.seg_len : row);
    const float theta = (float)pos / a.denom[p];
    float s, c;
    sincosf(theta, &s, &c);
    if (a.inverse) s = -s;
    float *px = a.x + (size_t)row * a.ld + a.start_col + head * a.head_dim + 2 * p;
    const float x0 = px[0], x1 = px[1];
    px[0] = x0 * c - x1 * s;
    px[1] = x0 * s + x1 * c;
  }
}

// (cos, sin) of every (position, pair) with the arithmetic of rope_kernel,
// so a projection epilogue that reads the table rotates exactly as the
// in-place kernel does.
__global__ void __launch_bounds__(256) rope_table_kernel(const RopeArgs a, float2 *cs) {
  const long long total = (long long)a.rows * a.pairs;
  for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int p = (int)(idx % a.pairs);
    const int pos = (int)(idx / a.pairs);
    const float theta = (float)pos / a.denom[p];
    float s, c;
    sincosf(theta, &s, &c);
    cs[idx] = make_float2(c, s);
  }
}

// Q and K rotated together from a cdml_rope_table (the trainer's
// ApplySegmentedRotaryInPlace, TransformerTrainer.cs:811-848): blockIdx.y
// picks the matrix, each thread one unit of W floats (W = 4: two pairs moved
// as float4, the head dim a multiple of 4; W = 2: one pair) of row
// idx / units.  The rotation is rope_kernel's expression on the table's
// (cos, sin), so the bits equal cdml_rope's.
template <int W>
__global__ void __launch_bounds__(256) rope_qk_table_kernel(float *q, float *k, int rows, int ld, int units,
                                                            int head_dim, int pairs, const float2 *__restrict__ cs,
                                                            int pos_offset, int seg_len, int inverse) {
#pragma clang fp contract(off)
  float *x = blockIdx.y ? k : q;
  const unsigned total = (unsigned)rows * (unsigned)units;
  for (unsigned idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
    const unsigned row = idx / (unsigned)units;
    const int col = W * (int)(idx - row * (unsigned)units);
    const int pos = pos_offset + (seg_len > 0 ? (int)(row % (unsigned)seg_len) : (int)row);
    const int p0 = (col % head_dim) / 2;
    float *px = x + (size_t)row * ld + col;
    if constexpr (W == 4) {
      const float4 t = *reinterpret_cast<const float4 *>(cs + (size_t)pos * pairs + p0);
      const float4 v = *reinterpret_cast<const float4 *>(px);
      const float s0 = inverse ? -t.y : t.y, s1 = inverse ? -t.w : t.w;
      float4 o;
      o.x = v.x * t.x - v.y * s0;
      o.y = v.x * s0 + v.y * t.x;
      o.z = v.z * t.z - v.w * s1;
      o.w = v.z * s1 + v.w * t.z;
      *reinterpret_cast<float4 *>(px) = o;
    } else {
      const float2 t = cs[(size_t)pos * pairs + p0];
      const float s0 = inverse ? -t.y : t.y;
      const float x0 = px[0], x1 = px[1];
      px[0] = x0 * t.x - x1 * s0;
      px[1] = x0 * s0 + x1 * t.x;
    }
  }
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_rope_qk_table(float *q, float *k, int rows, int ld, int head_dim, int num_heads,
                                  const float *rope_cs, int n_pos, int pos_offset, int seg_len, int inverse,
                                  cdml_stream stream) {
  if (rows < 0 || ld < 0 || head_dim < 0 || num_heads <= 0 || n_pos < 0 || seg_len < 0 || pos_offset < 0)
    return fail(CDML_E_INVALID, "cdml_rope_qk_table: bad size");
  if (head_dim & 1) return fail(CDML_E_INVALID, "cdml_rope_qk_table: RoPE requires an even head dimension");
  if ((long long)head_dim * num_heads > ld) return fail(CDML_E_INVALID, "cdml_rope_qk_table: heads exceed the row");
  if (rows == 0 || head_dim == 0) return CDML_OK;
  if (!q || !rope_cs) return fail(CDML_E_INVALID, "cdml_rope_qk_table: NULL pointer");
  if (q == k) return fail(CDML_E_INVALID, "cdml_rope_qk_table: q and k must be different arrays");
  if (reinterpret_cast<uintptr_t>(rope_cs) % 8)
    return fail(CDML_E_INVALID, "cdml_rope_qk_table: rope_cs must be 8-byte aligned");
  const long long last = (long long)pos_offset + (seg_len > 0 ? std::min(seg_len, rows) : rows) - 1;
  if (last >= n_pos)
    return fail(CDML_E_INVALID, "cdml_rope_qk_table: position %lld outside the table's %d", last, n_pos);
  const bool v4 = head_dim % 4 == 0 && ld % 4 == 0 && aligned16(q) && (!k || aligned16(k)) && aligned16(rope_cs);
  const int width = head_dim * num_heads, units = v4 ? width / 4 : width / 2;
  if ((long long)rows * units >= (1ll << 31))
    return fail(CDML_E_INVALID, "cdml_rope_qk_table: %d rows of %d heads exceed 2^31 units", rows, num_heads);
  int rc = ensure_device();
  if (rc) return rc;
  const long long total = (long long)rows * units;
  const dim3 grid((unsigned)std::min<long long>((total + 255) / 256, 8192), k ? 2 : 1), block(256);
  const float2 *cs = reinterpret_cast<const float2 *>(rope_cs);
  if (v4)
    rope_qk_table_kernel<4><<<grid, block, 0, as_hip(stream)>>>(q, k, rows, ld, units, head_dim, head_dim / 2, cs,
                                                                pos_offset, seg_len, inverse ? 1 : 0);
  else
    rope_qk_table_kernel<2><<<grid, block, 0, as_hip(stream)>>>(q, k, rows, ld, units, head_dim, head_dim / 2, cs,
                                                                pos_offset, seg_len, inverse ? 1 : 0);
  return check_launch("rope_qk_table_kernel");
}

extern "C" int cdml_rope(float *x, int rows, int ld, int start_col, int head_dim, int num_heads,
                         float base_theta, int inverse, int pos_offset, int seg_len,
                         const int *positions, cdml_stream stream) {
  if (rows < 0 || start_col < 0 || head_dim < 0 || num_heads <= 0 || seg_len < 0)
    return fail(CDML_E_INVALID, "cdml_rope: bad size");
  if (head_dim & 1) return fail(CDML_E_INVALID, "cdml_rope: RoPE requires an even head dimension");
  if (!(base_theta > 0.f) || std::isinf(base_theta))
    return fail(CDML_E_INVALID, "cdml_rope: base_theta must be positive and finite");
  if (head_dim / 2 > kMaxPairs) return fail(CDML_E_INVALID, "cdml_rope: head_dim above %d", 2 * kMaxPairs);
  if ((long long)start_col + (long long)head_dim * num_heads > ld)
    return fail(CDML_E_INVALID, "cdml_rope: heads exceed the row");
  if (rows == 0 || head_dim == 0) return CDML_OK;
  if (!x) return fail(CDML_E_INVALID, "cdml_rope: x is NULL");
  int rc = ensure_device();
  if (rc) return rc;
  RopeArgs a{};
  a.x = x;
  a.positions = positions;
  a.rows = rows;
  a.ld = ld;
  a.start_col = start_col;
  a.head_dim = head_dim;
  a.num_heads = num_heads;
  a.pairs = head_dim / 2;
  a.inverse = inverse ? 1 : 0;
  a.pos_offset = pos_offset;
  a.seg_len = seg_len;
  for (int p = 0; p < a.pairs; ++p)
    a.denom[p] = powf(base_theta, (2.0f * (float)p) / (float)head_dim);
  long long total = (long long)rows * num_heads * a.pairs;
  long long blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  rope_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(a);
  return check_launch("rope_kernel");
}

extern "C" int cdml_rope_table(float *cs, int n_pos, int head_dim, float base_theta,
                               cdml_stream stream) {
  if (n_pos < 0 || head_dim <= 0 || (head_dim & 1))
    return fail(CDML_E_INVALID, "cdml_rope_table: n_pos >= 0 and an even head_dim > 0 required");
  if (!(base_theta > 0.f) || std::isinf(base_theta))
    return fail(CDML_E_INVALID, "cdml_rope_table: base_theta must be positive and finite");
  if (head_dim / 2 > kMaxPairs)
    return fail(CDML_E_INVALID, "cdml_rope_table: head_dim above %d", 2 * kMaxPairs);
  if (n_pos == 0) return CDML_OK;
  if (!cs) return fail(CDML_E_INVALID, "cdml_rope_table: cs is NULL");
  if (reinterpret_cast<uintptr_t>(cs) % 8)
    return fail(CDML_E_INVALID, "cdml_rope_table: cs must be 8-byte aligned");
  int rc = ensure_device();
  if (rc) return rc;
  RopeArgs a{};
  a.rows = n_pos;
  a.pairs = head_dim / 2;
  for (int p = 0; p < a.pairs; ++p)
    a.denom[p] = powf(base_theta, (2.0f * (float)p) / (float)head_dim);
  const long long total = (long long)n_pos * a.pairs;
  long long blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  rope_table_kernel<<<dim3((unsigned)blocks), dim3(256), 0, as_hip(stream)>>>(
      a, reinterpret_cast<float2 *>(cs));
  return check_launch("rope_table_kernel");
}
