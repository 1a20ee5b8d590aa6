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
// Every phase of a step is latency-bound (a few hundred outputs whose
// operands sit in L2), so the layout is chosen for the fewest dependent
// memory round trips: each dot product (projections, scores, LM head) is
// spread over G adjacent lanes, G the smallest power of two that leaves a
// lane at most 8 float4 loads, all issued before the first is used, and
// the G partial sums meet in a butterfly of shuffles; P V splits the keys
// over kTinyThreads / D thread groups, each with 8 V loads in flight.  The
// softmax is one wave per head.
#include "common.h"

namespace cdml {
namespace {

// 512 threads per sequence: c1 generation 0.69 -> 0.64 ms against 256 (the
// projections and the LM head take one pass of dot products instead of two);
// 1024 measured 0.68 ms (the barriers cost more than the passes save)
constexpr int kTinyThreads = 512;
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

constexpr int kTinyLoads = 8;  // float4 loads in flight per lane of a dot product

// Lanes per dot product of length K (K % 4 == 0, K <= 1024): the smallest
// power of two G with K / 4 <= 8 G.
__device__ __forceinline__ int tiny_group(int K) {
  int g = 1;
  while (g < 64 && K / 4 > kTinyLoads * g) g <<= 1;
  return g;
}

// Lane `sub`'s share of row . x over float4 groups sub, sub + G, ... (16-byte
// aligned row; x in LDS); every load is issued before the first product.
__device__ __forceinline__ float tiny_dot_part(const float *__restrict__ row, const float *x, int nf4, int sub,
                                               int G) {
  const float4 *r4 = reinterpret_cast<const float4 *>(row);
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float4 a[kTinyLoads];
#pragma unroll
  for (int i = 0; i < kTinyLoads; ++i) {
    const int idx = sub + G * i;
    a[i] = idx < nf4 ? r4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < kTinyLoads; ++i) {
    const int idx = sub + G * i;
    if (idx < nf4) {
      const float4 b = x4[idx];
      acc += (a[i].x * b.x + a[i].y * b.y) + (a[i].z * b.z + a[i].w * b.w);
    }
  }
  return acc;
}

// For every o < count: emit(o, row(o) . x(o)), K-long dot products spread
// over G lanes each.  Every thread runs the same passes (the shuffles need
// whole waves); emit runs on the group's first lane.
template <class Row, class X, class Emit>
__device__ __forceinline__ void tiny_dots(int count, int K, Row row, X x, Emit emit) {
  const int G = tiny_group(K), per = kTinyThreads / G, nf4 = K / 4;
  const int sub = threadIdx.x % G, slot = threadIdx.x / G;
  for (int base = 0; base < count; base += per) {
    const int o = base + slot;
    float acc = o < count ? tiny_dot_part(row(o), x(o), nf4, sub, G) : 0.f;
    for (int off = G >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (sub == 0 && o < count) emit(o, acc);
  }
}

// y[n] = act(b[n] + w[n] . x) for n < N (x and y in LDS).
__device__ __forceinline__ void tiny_linear(const float *__restrict__ w, const float *__restrict__ b,
                                            const float *x, int K, int N, float *y, int act) {
  tiny_dots(
      N, K, [&](int n) { return w + (size_t)n * K; }, [&](int) { return x; },
      [&](int n, float v) { y[n] = tiny_act(v + (b ? b[n] : 0.f), act); });
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
  __shared__ float part[kTinyThreads];  // P V partial sums of the key groups
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
      // Q, K and V as one set of 3 D dot products
      tiny_dots(
          3 * D, D,
          [&](int o) {
            const int n = o % D;
            return (o < D ? L.wq : o < 2 * D ? L.wk : L.wv) + (size_t)n * D;
          },
          [&](int) { return x; },
          [&](int o, float v) {
            const int n = o % D;
            const float *bias = o < D ? L.bq : o < 2 * D ? L.bk : L.bv;
            (o < D ? q : o < 2 * D ? kv[0] : kv[1])[n] = v + (bias ? bias[n] : 0.f);
          });
      __syncthreads();
      // RoPE of q and k at `pos` (AccelerationCPU.cs:4947-4975): pair p of a
      // head is columns 2p and 2p + 1, (cos, sin) from the model's table
      for (int e = t; e < D; e += kTinyThreads) {
#pragma clang fp contract(off)
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
      tiny_dots(
          H * nk, hd, [&](int i) { return kc + (size_t)(i % nk) * D + (i / nk) * hd; },
          [&](int i) { return q + (i / nk) * hd; }, [&](int i, float v) { sc[(i / nk) * S + i % nk] = v * scale; });
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
      // att[e] = sum_j p[head(e)][j] v_j[e]: group g of the kTinyThreads / D thread
      // groups takes keys g, g + groups, ..., 8 V loads in flight per lane
      {
        const int groups = kTinyThreads / D, g = t / D, e = t % D;
        if (g < groups) {
          const float *p = sc + (e / hd) * S;
          float acc = 0.f;
          for (int j0 = g; j0 < nk; j0 += kTinyLoads * groups) {
            float vv[kTinyLoads];
#pragma unroll
            for (int i = 0; i < kTinyLoads; ++i) {
              const int j = j0 + i * groups;
              vv[i] = j < nk ? vc[(size_t)j * D + e] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < kTinyLoads; ++i) {
              const int j = j0 + i * groups;
              if (j < nk) acc += p[j] * vv[i];
            }
          }
          part[t] = acc;
        }
        __syncthreads();
        for (int d = t; d < D; d += kTinyThreads) {
          float v = 0.f;
          for (int gg = 0; gg < groups; ++gg) v += part[gg * D + d];
          att[d] = v;
        }
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
    tiny_dots(
        m.vocab, D, [&](int n) { return m.out_w + (size_t)n * D; }, [&](int) { return x; },
        [&](int n, float v) {
          v += m.out_b[n];
          if (v > bv || (v == bv && n < bi)) {
            bv = v;
            bi = n;
          }
        });
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
