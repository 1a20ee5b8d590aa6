// Whole greedy decode steps of a small decoder-only model in one launch:
// LanguageModel.Generate's per-token loop (LanguageModel.cs:482-537) with
// DecoderSelfAttentionStep (:334-430) in every post-LN block
// (TransformerBlock.cs:35-44).  A generation step of a model this small is
// two dozen dependent launches of microseconds each, so the launches, not
// the arithmetic, set its time.  Here one workgroup per sequence keeps the
// token's activations in LDS and runs every step, layer and the LM head's
// argmax itself: sequences never exchange data, so no step needs another
// workgroup.
//
// Products y = act(W x + b) run one thread per output with float4 loads,
// four in flight; attention runs one thread per (head, key) for the scores,
// one wave per head for the softmax, one thread per output column for P V.
#include "common.h"

namespace cdml {
namespace {

constexpr int kTinyThreads = 256;
constexpr int kTinyMaxDim = 256;
constexpr int kTinyMaxFF = 1024;
constexpr int kTinyMaxScores = 4096;  // heads * MaxSequenceLength

__device__ __forceinline__ float tiny_sigmoid(float x) {
  if (x >= 0.f) return 1.f / (1.f + expf(-x));
  const float z = expf(x);
  return z / (1.f + z);
}

// NeuralNetwork.cs:670-716's activations (ReLU as x > 0 ? x : 0).
__device__ __forceinline__ float tiny_act(float x, int act) {
  switch (act) {
    case CDML_ACT_SIGMOID: return tiny_sigmoid(x);
    case CDML_ACT_TANH: return tanhf(x);
    case CDML_ACT_RELU: return x > 0.f ? x : 0.f;
    case CDML_ACT_LEAKYRELU: return x > 0.f ? x : 0.01f * x;
    case CDML_ACT_SWISH: return x * tiny_sigmoid(x);
    default: return x;
  }
}

__device__ __forceinline__ float tiny_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float tiny_wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// sum_k row[k] x[k] for K % 4 == 0 (16-byte aligned row, x in LDS): four
// float4 loads in flight per iteration, one running sum per float4 lane.
__device__ __forceinline__ float tiny_dot(const float *__restrict__ row, const float *x, int K) {
  const float4 *r4 = reinterpret_cast<const float4 *>(row);
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  int i = 0;
  for (; i + 4 <= K / 4; i += 4) {
    const float4 a0 = r4[i], a1 = r4[i + 1], a2 = r4[i + 2], a3 = r4[i + 3];
    const float4 b0 = x4[i], b1 = x4[i + 1], b2 = x4[i + 2], b3 = x4[i + 3];
    acc.x += a0.x * b0.x + a1.x * b1.x + a2.x * b2.x + a3.x * b3.x;
    acc.y += a0.y * b0.y + a1.y * b1.y + a2.y * b2.y + a3.y * b3.y;
    acc.z += a0.z * b0.z + a1.z * b1.z + a2.z * b2.z + a3.z * b3.z;
    acc.w += a0.w * b0.w + a1.w * b1.w + a2.w * b2.w + a3.w * b3.w;
  }
  for (; i < K / 4; ++i) {
    const float4 a0 = r4[i], b0 = x4[i];
    acc.x += a0.x * b0.x;
    acc.y += a0.y * b0.y;
    acc.z += a0.z * b0.z;
    acc.w += a0.w * b0.w;
  }
  return (acc.x + acc.y) + (acc.z + acc.w);
}

// y[n] = act(b[n] + w[n] . x) for n < N (x and y in LDS).
__device__ __forceinline__ void tiny_linear(const float *__restrict__ w, const float *__restrict__ b,
                                            const float *x, int K, int N, float *y, int act) {
  for (int n = threadIdx.x; n < N; n += kTinyThreads)
    y[n] = tiny_act(tiny_dot(w + (size_t)n * K, x, K) + (b ? b[n] : 0.f), act);
}

// out = LayerNorm(a + c) with the biased variance in two passes (the
// reference's ResidualLayerNorm, AccelerationCPU.cs:1376-1438); wave 0.
__device__ __forceinline__ void tiny_residual_ln(const float *a, const float *c, const float *__restrict__ g,
                                                 const float *__restrict__ be, float *out, int D, float eps) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  float v[kTinyMaxDim / 64];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kTinyMaxDim / 64; ++i) {
    const int j = lane + 64 * i;
    v[i] = j < D ? a[j] + c[j] : 0.f;
    sum += v[i];
  }
  const float mean = tiny_wave_sum(sum) / (float)D;
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < kTinyMaxDim / 64; ++i) {
    const int j = lane + 64 * i;
    const float d = v[i] - mean;
    var += j < D ? d * d : 0.f;
  }
  var = tiny_wave_sum(var) / (float)D;
  const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < kTinyMaxDim / 64; ++i) {
    const int j = lane + 64 * i;
    if (j < D) out[j] = g[j] * ((v[i] - mean) * inv_std) + be[j];
  }
}

__global__ void __launch_bounds__(kTinyThreads) tiny_decode_kernel(const cdml_tiny_model m, int *tokens,
                                                                   int batch, int pos0, int n_steps) {
  __shared__ __attribute__((aligned(16))) float x[kTinyMaxDim], q[kTinyMaxDim], kv[2][kTinyMaxDim],
      att[kTinyMaxDim], h[kTinyMaxDim];
  __shared__ __attribute__((aligned(16))) float ff[2][kTinyMaxFF];
  __shared__ float sc[kTinyMaxScores];
  __shared__ float best_v[kTinyThreads / 64];
  __shared__ int best_i[kTinyThreads / 64];
  __shared__ int tok;
  const int b = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int D = m.dim, H = m.heads, hd = D / H, S = m.max_seq;
  const float scale = 1.0f / sqrtf((float)hd);
  if (t == 0) tok = tokens[b];
  __syncthreads();
  for (int s = 1; s <= n_steps; ++s) {
    const int pos = pos0 + s - 1;  // position of the token being fed
    const int nk = pos + 1;        // keys visible to it, itself included
    for (int d = t; d < D; d += kTinyThreads) x[d] = m.embedding[(size_t)tok * D + d];
    __syncthreads();
    for (int l = 0; l < m.n_layers; ++l) {
      const cdml_tiny_layer &L = m.layers[l];
      tiny_linear(L.wq, L.bq, x, D, D, q, CDML_ACT_NONE);
      tiny_linear(L.wk, L.bk, x, D, D, kv[0], CDML_ACT_NONE);
      tiny_linear(L.wv, L.bv, x, D, D, kv[1], CDML_ACT_NONE);
      __syncthreads();
      // RoPE of q and k at `pos` (AccelerationCPU.cs:4947-4975): pair p of a
      // head is columns 2p and 2p + 1, (cos, sin) from the model's table
      for (int e = t; e < D; e += kTinyThreads) {
        if (e & 1) continue;
        const float2 cs = reinterpret_cast<const float2 *>(m.rope_cs)[(size_t)pos * (hd / 2) + (e % hd) / 2];
        const float q0 = q[e], q1 = q[e + 1], k0 = kv[0][e], k1 = kv[0][e + 1];
        q[e] = q0 * cs.x - q1 * cs.y;
        q[e + 1] = q1 * cs.x + q0 * cs.y;
        kv[0][e] = k0 * cs.x - k1 * cs.y;
        kv[0][e + 1] = k1 * cs.x + k0 * cs.y;
      }
      __syncthreads();
      // append K and V as row `pos` of this sequence's caches
      float *kc = L.kcache + (size_t)b * S * D, *vc = L.vcache + (size_t)b * S * D;
      for (int d = t; d < D; d += kTinyThreads) {
        kc[(size_t)pos * D + d] = kv[0][d];
        vc[(size_t)pos * D + d] = kv[1][d];
      }
      __threadfence_block();  // the appended row is read back below
      __syncthreads();
      // scores of every head against the nk cached keys
      for (int i = t; i < H * nk; i += kTinyThreads) {
        const int hh = i / nk, j = i % nk;
        sc[hh * S + j] = tiny_dot(kc + (size_t)j * D + hh * hd, q + hh * hd, hd) * scale;
      }
      __syncthreads();
      // softmax per head: wave w takes heads w, w + 4, ...
      for (int hh = wave; hh < H; hh += kTinyThreads / 64) {
        float mx = -INFINITY;
        for (int j = lane; j < nk; j += 64) mx = fmaxf(mx, sc[hh * S + j]);
        mx = tiny_wave_max(mx);
        float sum = 0.f;
        for (int j = lane; j < nk; j += 64) {
          const float p = expf(sc[hh * S + j] - mx);
          sc[hh * S + j] = p;
          sum += p;
        }
        sum = tiny_wave_sum(sum);
        const float inv = 1.0f / sum;
        for (int j = lane; j < nk; j += 64) sc[hh * S + j] *= inv;
      }
      __syncthreads();
      // att[e] = sum_j p[head(e)][j] v_j[e]
      for (int e = t; e < D; e += kTinyThreads) {
        const float *p = sc + (e / hd) * S;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        int j = 0;
        for (; j + 4 <= nk; j += 4) {  // four V loads in flight
          a0 += p[j] * vc[(size_t)j * D + e];
          a1 += p[j + 1] * vc[(size_t)(j + 1) * D + e];
          a2 += p[j + 2] * vc[(size_t)(j + 2) * D + e];
          a3 += p[j + 3] * vc[(size_t)(j + 3) * D + e];
        }
        for (; j < nk; ++j) a0 += p[j] * vc[(size_t)j * D + e];
        att[e] = (a0 + a1) + (a2 + a3);
      }
      __syncthreads();
      tiny_linear(L.wo, L.bo, att, D, D, q, CDML_ACT_NONE);  // q is free again: the projection
      __syncthreads();
      tiny_residual_ln(x, q, L.ln1g, L.ln1b, h, D, m.eps);
      __syncthreads();
      const float *in = h;
      int width = D;
      for (int f = 0; f < L.n_ff; ++f) {
        float *out = ff[f & 1];
        tiny_linear(L.ffw[f], L.ffb[f], in, width, L.ffrows[f], out, L.ffact[f]);
        __syncthreads();
        in = out;
        width = L.ffrows[f];
      }
      tiny_residual_ln(h, in, L.ln2g, L.ln2b, x, D, m.eps);
      __syncthreads();
    }
    // LM head and greedy choice: the lowest index among the largest logits
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int n = t; n < m.vocab; n += kTinyThreads) {
      const float v = tiny_dot(m.out_w + (size_t)n * D, x, D) + m.out_b[n];
      if (v > bv || (v == bv && n < bi)) {
        bv = v;
        bi = n;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      best_v[wave] = bv;
      best_i[wave] = bi;
    }
    __syncthreads();
    if (t == 0) {
      float v = best_v[0];
      int i = best_i[0];
      for (int w = 1; w < kTinyThreads / 64; ++w)
        if (best_v[w] > v || (best_v[w] == v && best_i[w] < i)) {
          v = best_v[w];
          i = best_i[w];
        }
      if (i >= m.vocab) i = 0;  // every logit NaN: as cdml_argmax_rows
      tok = i;
      tokens[(size_t)s * batch + b] = i;
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_tiny_decode(const cdml_tiny_model *model, int *tokens, int batch, int pos0, int n_steps,
                                cdml_stream stream) {
  if (!model || !tokens) return fail(CDML_E_INVALID, "cdml_tiny_decode: NULL pointer");
  const cdml_tiny_model &m = *model;
  if (batch < 0 || n_steps < 0 || pos0 < 0) return fail(CDML_E_INVALID, "cdml_tiny_decode: negative size");
  if (batch == 0 || n_steps == 0) return CDML_OK;
  if (m.dim <= 0 || m.heads <= 0 || m.dim % m.heads || (m.dim / m.heads) % 4 || m.dim > kTinyMaxDim ||
      m.n_layers < 0 || m.vocab <= 0 || m.max_seq <= 0 || (long long)m.heads * m.max_seq > kTinyMaxScores)
    return fail(CDML_E_INVALID, "cdml_tiny_decode: model outside the fused path's limits (dim %d, heads %d, "
                "max_seq %d)", m.dim, m.heads, m.max_seq);
  if ((long long)pos0 + n_steps > m.max_seq)
    return fail(CDML_E_INVALID, "cdml_tiny_decode: positions past MaxSequenceLength");
  if (!m.embedding || !m.out_w || !m.out_b || !m.rope_cs || (m.n_layers > 0 && !m.layers))
    return fail(CDML_E_INVALID, "cdml_tiny_decode: NULL model pointer");
  if (!aligned16(m.embedding) || !aligned16(m.out_w))
    return fail(CDML_E_INVALID, "cdml_tiny_decode: embedding and LM head must be 16-byte aligned");
  int rc = ensure_device();
  if (rc) return rc;
  tiny_decode_kernel<<<dim3((unsigned)batch), dim3(kTinyThreads), 0, as_hip(stream)>>>(m, tokens, batch, pos0,
                                                                                       n_steps);
  return check_launch("tiny_decode_kernel");
}

extern "C" int cdml_tiny_layer_check(const cdml_tiny_layer *layer, int dim) {
  if (!layer) return fail(CDML_E_INVALID, "cdml_tiny_layer_check: NULL layer");
  const cdml_tiny_layer &L = *layer;
  if (L.n_ff < 1 || L.n_ff > CDML_TINY_MAX_FF)
    return fail(CDML_E_INVALID, "cdml_tiny_layer_check: %d FFN layers (1 to %d)", L.n_ff, CDML_TINY_MAX_FF);
  // Weight rows and cache rows are read as float4.
  const float *vec4[] = {L.wq, L.wk, L.wv, L.wo, L.kcache, L.vcache};
  for (const float *p : vec4)
    if (!p || !aligned16(p))
      return fail(CDML_E_INVALID, "cdml_tiny_layer_check: NULL or unaligned weight or cache pointer");
  if (!L.ln1g || !L.ln1b || !L.ln2g || !L.ln2b)  // biases may be NULL (zero)
    return fail(CDML_E_INVALID, "cdml_tiny_layer_check: NULL LayerNorm pointer");
  int width = dim;
  for (int f = 0; f < L.n_ff; ++f) {
    if (L.ffcols[f] != width || L.ffrows[f] <= 0 || L.ffrows[f] > kTinyMaxFF || L.ffrows[f] % 4)
      return fail(CDML_E_INVALID, "cdml_tiny_layer_check: FFN layer %d is %d x %d", f, L.ffrows[f], L.ffcols[f]);
    if (!L.ffw[f] || !aligned16(L.ffw[f]))
      return fail(CDML_E_INVALID, "cdml_tiny_layer_check: FFN layer %d has a NULL or unaligned pointer", f);
    if (L.ffact[f] < CDML_ACT_NONE || L.ffact[f] > CDML_ACT_SWISH)
      return fail(CDML_E_INVALID, "cdml_tiny_layer_check: FFN layer %d activation %d", f, L.ffact[f]);
    width = L.ffrows[f];
  }
  if (width != dim) return fail(CDML_E_INVALID, "cdml_tiny_layer_check: FFN output width %d != dim %d", width, dim);
  return CDML_OK;
}
