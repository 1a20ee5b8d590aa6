// Single-query decode attention over a cached K/V (the device form of the
// inline loop in LanguageModel.DecoderSelfAttentionStep, LanguageModel.cs:365-427).
//
// HBM-bound: every cached K and V element is read exactly once.  The cache
// of each (sequence, head) is split into chunks of DC_CHUNK keys; one
// 256-thread workgroup owns a chunk and each of its four waves a quarter of
// it.  Inside a wave, each group of 8 lanes owns one key per step (8 keys per
// wave-step).  Lane e of a group holds the head dims
// {VW*e + 8*VW*i + c : i < NV, c < VW}, so one vector load instruction of the
// group covers 8*VW contiguous floats (a whole 128-byte line for VW = 4).
// K and V rows of a step are loaded together and the next step's rows are in
// flight while the current one is consumed: the scores are reduced across the
// 8 lanes of a group and folded into a per-group online softmax (running max,
// running sum, running output), so no workgroup barrier separates the K and V
// streams.  The eight groups of a wave and then the four waves are merged with
// the (max, sum) rescaling; a combine kernel merges the chunks.
#include <mutex>

#include "common.h"

namespace cdml {
namespace {

constexpr int DC_THREADS = 256;
constexpr int DC_CHUNK = 256;       // keys per workgroup (the partials are sized for it)
constexpr int DC_CHUNK_WIDE = 512;  // keys per workgroup when the grid stays wide

struct DecodeArgs {
  const float *q, *kc, *vc;
  const int *kv_len;
  float *o;
  float *part;  // [batch*heads][nsplit][hd + 2]: o[hd], max, sum
  int t_max, dim, heads, hd, nsplit;
  float scale_log2;
};

template <int VW>
struct VecT;
template <>
struct VecT<4> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct VecT<2> {
  typedef float type __attribute__((ext_vector_type(2)));
};

// One lane's NV vectors of a cached row (streamed once: non-temporal).
template <int VW, int NV>
__device__ __forceinline__ void load_slice(const float *__restrict__ p, float (&r)[VW * NV]) {
  typedef typename VecT<VW>::type V;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    V t = __builtin_nontemporal_load(reinterpret_cast<const V *>(p + 8 * VW * i));
#pragma unroll
    for (int c = 0; c < VW; ++c) r[VW * i + c] = t[c];
  }
}

// Merges online-softmax state (m, l, o) with a partner's (exp2 domain).
template <int EPL>
__device__ __forceinline__ void merge_state(float &m, float &l, float (&o)[EPL], float m2, float l2,
                                            const float (&o2)[EPL]) {
  const float mn = fmaxf(m, m2);
  const float mu = mn == -INFINITY ? 0.f : mn;
  const float a1 = fast_exp2(m - mu), a2 = fast_exp2(m2 - mu);
  l = l * a1 + l2 * a2;
#pragma unroll
  for (int i = 0; i < EPL; ++i) o[i] = o[i] * a1 + o2[i] * a2;
  m = mn;
}

template <int HD, int CHUNK>
__global__ void __launch_bounds__(DC_THREADS) decode_split_kernel(const DecodeArgs a) {
  constexpr int KITER = CHUNK / 4 / 8;  // steps of 8 keys per wave
  static_assert(KITER % 2 == 0, "the key loop alternates two register sets");
  constexpr int VW = HD >= 32 ? 4 : 2;  // floats per vector load
  constexpr int NV = HD / (8 * VW);     // vector loads per lane per row
  constexpr int EPL = VW * NV;          // head dims per lane (= HD / 8)
  __shared__ float red_m[4], red_l[4];
  __shared__ float red_o[4][HD];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 3, e = lane & 7;
  const int len = min(max(a.kv_len[b], 0), a.t_max);
  const int chunk0 = split * CHUNK;
  float *part = a.part + ((size_t)(b * a.heads + h) * a.nsplit + split) * (HD + 2);

  if (chunk0 >= len) {
    for (int d = threadIdx.x; d < HD + 2; d += DC_THREADS) part[d] = d == HD ? -INFINITY : 0.f;
    return;
  }

  const size_t col = (size_t)h * HD + VW * e;
  float q[EPL];
  load_slice<VW, NV>(a.q + (size_t)b * a.dim + col, q);

  const float *kb = a.kc + (size_t)b * a.t_max * a.dim + col;
  const float *vb = a.vc + (size_t)b * a.t_max * a.dim + col;
  const int key0 = chunk0 + wave * (KITER * 8) + g;

  float m = -INFINITY, l = 0.f;
  float o[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) o[i] = 0.f;

  // Rows past the cache length are clamped to its last row (the chunk holds
  // at least one valid key) and left out of the softmax below, so the loads
  // need no branch.  Two register sets alternate: the next step's K and V
  // rows are in flight while the current ones are consumed.
  const int last = len - 1;
  float k0r[EPL], v0r[EPL], k1r[EPL], v1r[EPL];
  auto step = [&](int it, const float(&kr)[EPL], const float(&vr)[EPL]) {
    const int key = key0 + it * 8;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) s += q[i] * kr[i];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (key < len) {
      s *= a.scale_log2;
      const float mn = fmaxf(m, s);
      const float alpha = fast_exp2(m - mn);  // m = -inf on the first key: 0
      const float p = fast_exp2(s - mn);
      l = l * alpha + p;
#pragma unroll
      for (int i = 0; i < EPL; ++i) o[i] = o[i] * alpha + p * vr[i];
      m = mn;
    }
  };
  load_slice<VW, NV>(kb + (size_t)min(key0, last) * a.dim, k0r);
  load_slice<VW, NV>(vb + (size_t)min(key0, last) * a.dim, v0r);
#pragma unroll
  for (int it = 0; it < KITER; it += 2) {
    const int k1 = min(key0 + (it + 1) * 8, last);
    load_slice<VW, NV>(kb + (size_t)k1 * a.dim, k1r);
    load_slice<VW, NV>(vb + (size_t)k1 * a.dim, v1r);
    step(it, k0r, v0r);
    if (it + 2 < KITER) {
      const int k2 = min(key0 + (it + 2) * 8, last);
      load_slice<VW, NV>(kb + (size_t)k2 * a.dim, k0r);
      load_slice<VW, NV>(vb + (size_t)k2 * a.dim, v0r);
    }
    step(it + 1, k1r, v1r);
  }

  // Merge the 8 key groups of the wave (lanes with equal e).
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
    float o2[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) o2[i] = __shfl_xor(o[i], off);
    merge_state<EPL>(m, l, o, __shfl_xor(m, off), __shfl_xor(l, off), o2);
  }
  if (lane == 0) {
    red_m[wave] = m;
    red_l[wave] = l;
  }
  __syncthreads();
  // Rescale each wave's output to the workgroup max before the LDS sum.
  const float M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  const float mu = M == -INFINITY ? 0.f : M;
  const float aw = fast_exp2(m - mu);
  if (g == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int c = 0; c < VW; ++c) red_o[wave][VW * e + 8 * VW * i + c] = o[VW * i + c] * aw;
  }
  __syncthreads();
  for (int d = threadIdx.x; d < HD; d += DC_THREADS)
    part[d] = red_o[0][d] + red_o[1][d] + red_o[2][d] + red_o[3][d];
  if (threadIdx.x == 0) {
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) L += red_l[w] * fast_exp2(red_m[w] - mu);
    part[HD] = M;
    part[HD + 1] = L;
  }
}

// Merges the chunks of one (sequence, head) for the head dims of
// decode_split_kernel: with M the max over the chunk maxima and
// w_s = 2^(m_s - M), o = sum_s w_s o_s / sum_s w_s l_s.  Thread t sums dim
// t % HD over every G-th chunk from t / HD, so all G*HD threads have loads in
// flight; the G partial sums meet in LDS.
template <int HD>
__global__ void __launch_bounds__(DC_THREADS) decode_combine_vec_kernel(const DecodeArgs a) {
  constexpr int G = DC_THREADS / HD;
  __shared__ float red_m[4], red_l[4];
  __shared__ float acc_s[G][HD];
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int n = a.nsplit;
  const float *part = a.part + (size_t)(b * a.heads + h) * n * (HD + 2);

  float M = -INFINITY;
  for (int s = t; s < n; s += DC_THREADS) M = fmaxf(M, part[s * (HD + 2) + HD]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  if (lane == 0) red_m[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  const float mu = M == -INFINITY ? 0.f : M;

  float l = 0.f;
  for (int s = t; s < n; s += DC_THREADS)
    l += part[s * (HD + 2) + HD + 1] * fast_exp2(part[s * (HD + 2) + HD] - mu);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
  if (lane == 0) red_l[wave] = l;

  const int d = t % HD, sg = t / HD;
  float acc = 0.f;
#pragma unroll 4
  for (int s = sg; s < n; s += G)
    acc += part[s * (HD + 2) + d] * fast_exp2(part[s * (HD + 2) + HD] - mu);
  acc_s[sg][d] = acc;
  __syncthreads();
  if (t < HD) {
    float sum = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) sum += acc_s[g][t];
    const float L = red_l[0] + red_l[1] + red_l[2] + red_l[3];
    a.o[(size_t)b * a.dim + (size_t)h * HD + t] = L > 0.f ? sum / L : 0.f;
  }
}

__global__ void __launch_bounds__(256) decode_combine_kernel(const DecodeArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int hd = a.hd;
  const float *part = a.part + (size_t)(b * a.heads + h) * a.nsplit * (hd + 2);
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, part[s * (hd + 2) + hd]);
  const float m_use = M == -INFINITY ? 0.f : M;
  float l = 0.f;
  for (int s = 0; s < a.nsplit; ++s)
    l += part[s * (hd + 2) + hd + 1] * fast_exp2(part[s * (hd + 2) + hd] - m_use);
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (int s = 0; s < a.nsplit; ++s)
      acc += part[s * (hd + 2) + d] * fast_exp2(part[s * (hd + 2) + hd] - m_use);
    a.o[(size_t)b * a.dim + (size_t)h * hd + d] = acc * inv;
  }
}

// Any head dim: one workgroup per (sequence, head, chunk), one thread per key.
__global__ void __launch_bounds__(256) decode_split_generic_kernel(const DecodeArgs a) {
  extern __shared__ float sm[];  // p[256] | red[8]
  float *pv = sm;
  float *red = sm + 256;
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, hd = a.hd;
  const int len = min(max(a.kv_len[b], 0), a.t_max);
  const int chunk0 = split * DC_CHUNK;
  float *part = a.part + ((size_t)(b * a.heads + h) * a.nsplit + split) * (hd + 2);
  if (chunk0 >= len) {
    for (int d = t; d < hd + 2; d += 256) part[d] = d == hd ? -INFINITY : 0.f;
    return;
  }
  const float *qrow = a.q + (size_t)b * a.dim + (size_t)h * hd;
  const size_t cache = (size_t)b * a.t_max * a.dim + (size_t)h * hd;
  const int key = chunk0 + t;
  float s = -INFINITY;
  if (key < len) {
    float acc = 0.f;
    const float *kr = a.kc + cache + (size_t)key * a.dim;
    for (int d = 0; d < hd; ++d) acc += qrow[d] * kr[d];
    s = acc * a.scale_log2;
  }
  float mx = s;
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((t & 63) == 0) red[t >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float m_use = M == -INFINITY ? 0.f : M;
  const float p = fast_exp2(s - m_use);
  pv[t] = p;
  float ps = p;
  for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
  if ((t & 63) == 0) red[4 + (t >> 6)] = ps;
  __syncthreads();
  const int n = min(DC_CHUNK, len - chunk0);
  for (int d = t; d < hd; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < n; ++j) acc += pv[j] * a.vc[cache + (size_t)(chunk0 + j) * a.dim + d];
    part[d] = acc;
  }
  if (t == 0) {
    part[hd] = M;
    part[hd + 1] = red[4] + red[5] + red[6] + red[7];
  }
}

bool fast_hd(int hd) { return hd == 16 || hd == 32 || hd == 64 || hd == 128 || hd == 256; }


// Partials of cdml_decode_attn_noalloc: a file-scope device array, one copy
// per GPU, that lives until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol); it uses the address hipGetSymbolAddress returned for the device.
constexpr int kScratchMaxDevices = 64;
static __device__ __align__(256) float scratch[CDML_DECODE_NOALLOC_MAX_BYTES / sizeof(float)];
static std::mutex g_scratch_mu;
static float *g_scratch_ptr[kScratchMaxDevices];

}  // namespace

// Looks up this device's copy of `scratch` once (the device is current).
int noalloc_scratch_setup(int device, char *msg, size_t msg_bytes) {
  if (device < 0 || device >= kScratchMaxDevices) {
    snprintf(msg, msg_bytes, "device %d is beyond the %d devices the no-allocation entry points track", device,
             kScratchMaxDevices);
    return CDML_E_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return CDML_OK;
  void *p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    (void)hipGetLastError();
    snprintf(msg, msg_bytes, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    return CDML_E_HIP;
  }
  g_scratch_ptr[device] = static_cast<float *>(p);
  return CDML_OK;
}

static float *noalloc_scratch_ptr(int device) {
  if (device < 0 || device >= kScratchMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace cdml

using namespace cdml;

extern "C" int cdml_decode_attn_workspace_size(int batch, int t_max, int dim, int num_heads,
                                               size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_decode_attn_workspace_size: bytes is NULL");
  if (batch < 0 || t_max < 0 || dim <= 0 || num_heads <= 0 || dim % num_heads)
    return fail(CDML_E_INVALID, "cdml_decode_attn_workspace_size: bad size");
  const int hd = dim / num_heads;
  const int nsplit = (t_max + DC_CHUNK - 1) / DC_CHUNK;
  *bytes = sizeof(float) * (size_t)batch * num_heads * (size_t)nsplit * (hd + 2);
  return CDML_OK;
}

// Validated launch of the split and combine kernels over the partials buffer
// `part` (at least cdml_decode_attn_workspace_size() bytes; every split
// writes its whole slot, so the buffer needs no clearing).
static int decode_launch(const float *q, const float *kcache, const float *vcache,
                         const int *kv_len, float *o, int batch, int t_max, int dim,
                         int num_heads, float scale, float *part, hipStream_t st) {
  DecodeArgs a{};
  a.q = q;
  a.kc = kcache;
  a.vc = vcache;
  a.kv_len = kv_len;
  a.o = o;
  a.part = part;
  a.t_max = t_max;
  a.dim = dim;
  a.heads = num_heads;
  a.hd = dim / num_heads;
  a.nsplit = (t_max + DC_CHUNK - 1) / DC_CHUNK;
  a.scale_log2 = scale * 1.4426950408889634f;
  dim3 grid(a.nsplit, num_heads, batch);
  const bool vec = fast_hd(a.hd) && dim % 4 == 0 && aligned16(q) && aligned16(kcache) &&
                   aligned16(vcache);
  if (vec) {
    // 512-key chunks while they still give the launch four workgroups per CU
    // (c4: 1.26 -> 1.23 ms); shorter caches and small batches keep 256 for
    // the parallelism.  Fewer chunks fit the partials sized for 256.
    const int nsplit_wide = (t_max + DC_CHUNK_WIDE - 1) / DC_CHUNK_WIDE;
    const bool wide = (long long)nsplit_wide * num_heads * batch >= 4LL * num_cus();
    if (wide) {
      a.nsplit = nsplit_wide;
      grid.x = nsplit_wide;
    }
    const dim3 cgrid(num_heads, batch);
#define CDML_DECODE_CASE(HDV)                                                              \
  case HDV:                                                                                \
    if (wide)                                                                              \
      decode_split_kernel<HDV, DC_CHUNK_WIDE><<<grid, DC_THREADS, 0, st>>>(a);             \
    else                                                                                   \
      decode_split_kernel<HDV, DC_CHUNK><<<grid, DC_THREADS, 0, st>>>(a);                  \
    decode_combine_vec_kernel<HDV><<<cgrid, DC_THREADS, 0, st>>>(a);                       \
    break;
    switch (a.hd) {
      CDML_DECODE_CASE(16)
      CDML_DECODE_CASE(32)
      CDML_DECODE_CASE(64)
      CDML_DECODE_CASE(128)
      default:
      CDML_DECODE_CASE(256)
    }
#undef CDML_DECODE_CASE
    return check_launch("decode_split_kernel/decode_combine_vec_kernel");
  }
  decode_split_generic_kernel<<<grid, 256, sizeof(float) * (256 + 8), st>>>(a);
  int rc = check_launch("decode_split_generic_kernel");
  if (rc) return rc;
  decode_combine_kernel<<<dim3(num_heads, batch), dim3(a.hd < 256 ? 128 : 256), 0, st>>>(a);
  return check_launch("decode_combine_kernel");
}

extern "C" int cdml_decode_attn(const float *q, const float *kcache, const float *vcache,
                                const int *kv_len, float *o, int batch, int t_max, int dim,
                                int num_heads, float scale, void *workspace,
                                size_t workspace_bytes, cdml_stream stream) {
  size_t need = 0;
  int rc = cdml_decode_attn_workspace_size(batch, t_max, dim, num_heads, &need);
  if (rc) return rc;
  if (batch == 0) return CDML_OK;
  if (t_max == 0) return cdml_zero_f32_async(o, (size_t)batch * dim, stream);
  if (!q || !kcache || !vcache || !kv_len || !o)
    return fail(CDML_E_INVALID, "cdml_decode_attn: NULL pointer");
  if (!workspace || workspace_bytes < need)
    return fail(CDML_E_INVALID, "cdml_decode_attn: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  if (batch > 65535 || num_heads > 65535)
    return fail(CDML_E_INVALID, "cdml_decode_attn: batch and heads must be <= 65535");
  rc = ensure_device();
  if (rc) return rc;
  return decode_launch(q, kcache, vcache, kv_len, o, batch, t_max, dim, num_heads, scale,
                       static_cast<float *>(workspace), as_hip(stream));
}

extern "C" int cdml_decode_attn_noalloc(const float *q, const float *kcache, const float *vcache,
                                        const int *kv_len, float *o, int batch, int t_max, int dim,
                                        int num_heads, float scale, cdml_stream stream) {
  size_t need = 0;
  int rc = cdml_decode_attn_workspace_size(batch, t_max, dim, num_heads, &need);
  if (rc) return rc;
  if (batch == 0) return CDML_OK;
  if (t_max == 0) return cdml_zero_f32_async(o, (size_t)batch * dim, stream);
  if (!q || !kcache || !vcache || !kv_len || !o)
    return fail(CDML_E_INVALID, "cdml_decode_attn_noalloc: NULL pointer");
  if (need > (size_t)CDML_DECODE_NOALLOC_MAX_BYTES)
    return fail(CDML_E_INVALID,
                "cdml_decode_attn_noalloc: the shape needs %zu bytes of partials, more than the %zu "
                "bytes of the library's static scratch; call cdml_decode_attn with a workspace",
                need, (size_t)CDML_DECODE_NOALLOC_MAX_BYTES);
  if (batch > 65535 || num_heads > 65535)
    return fail(CDML_E_INVALID, "cdml_decode_attn_noalloc: batch and heads must be <= 65535");
  rc = ensure_device();
  if (rc) return rc;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(CDML_E_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  float *part = noalloc_scratch_ptr(dev);
  if (!part) {  // cdml_init sets it up; a device made current some other way gets it here
    char msg[256];
    rc = noalloc_scratch_setup(dev, msg, sizeof(msg));
    if (rc) return fail(rc, "cdml_decode_attn_noalloc: %s", msg);
    part = noalloc_scratch_ptr(dev);
  }
  return decode_launch(q, kcache, vcache, kv_len, o, batch, t_max, dim, num_heads, scale, part,
                       as_hip(stream));
}
