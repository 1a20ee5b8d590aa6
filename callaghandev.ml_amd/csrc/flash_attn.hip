// Fused flash-style fp32 attention forward for gfx950 (ScaledDotProductAttention
// and MultiHeadAttentionForward of the reference, AccelerationCPU.cs:1647-1956).
//
// One 256-thread workgroup owns 128 queries of one (sequence, head); each of
// its four waves owns 32 queries for the whole key loop.  Per key tile of BN
// keys (K and V staged through double-buffered LDS, next tile prefetched into
// registers while the current one is consumed):
//
//   S^T = K Q^T     v_mfma_f32_32x32x2_f32, A = K rows from LDS (16-byte
//                   reads), B = the wave's Q held in registers for the whole
//                   loop.  Computing S transposed puts one query per lane
//                   (lane % 32) and 16 keys per lane in the accumulator, so the
//                   softmax row reductions are in-lane plus one swap between
//                   the two half-waves.
//   online softmax  running max / sum per query in the exp2 domain
//                   (scale * log2 e folded into one FMA), masked keys -inf.
//   O^T += V^T P^T  the probabilities stay in the S accumulator registers:
//                   accumulator r of a lane holds key 8*(r/4) + 4*h + r%4,
//                   exactly the key the B operand of MFMA step r needs, so
//                   P is consumed in place; V^T comes from LDS (b32 reads).
//
// Causal: tiles entirely above the diagonal are never loaded; a wave skips
// MFMA work for its 32-key sub-blocks that lie wholly in its future; heavy
// query tiles are dispatched first.  A row whose keys are all masked ends
// with sum 0 and is written as 0 (AccelerationCPU.cs:1908-1911).
#include <cfloat>

#include "common.h"

namespace cdml {
namespace {

constexpr int FA_THREADS = 256;
constexpr int FA_BM = 128;  // queries per workgroup (32 per wave)
constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
  const float *q, *k, *v;
  float *o;
  float *lse;  // optional [batch * heads][lq]: log2 of each row's softmax normaliser
  const uint8_t *mask;
  int ldq, ldk, ldv, ldo;
  int lq, lk, heads, hd;
  float scale_log2;
  int n_qt, n_bh, total, padded;
};

// Stages one BN x HD tile of K or V (rows [k0, k0+BN) of head column block
// `col0`) from global memory into registers and then into LDS.  Each
// thread's element offsets inside a tile are fixed (set once); a tile load
// adds them to the wave-uniform tile base.  Rows past lk (the sequence end)
// are clamped to row lk - 1: their scores are masked to -inf and their
// probabilities are exactly 0.
template <int HD, int BN, bool VEC>
struct KvStage {
  static constexpr int F4_ROW = HD / 4;
  static constexpr int ROWS_PER_PASS = FA_THREADS / F4_ROW;
  static constexpr int NV = BN / ROWS_PER_PASS;
  static constexpr int NS = BN * HD / FA_THREADS;
  vf4 r[VEC ? NV : 1];  // a native vector, so the prefetch stays a register load issued at the loop top
  float s[VEC ? 1 : NS];
  uint32_t off[VEC ? NV : 1];  // element offsets of this thread's rows in a tile
  int col;

  __device__ __forceinline__ void init(int ld) {
    if constexpr (VEC) {
      const int t = threadIdx.x;
      col = (t % F4_ROW) * 4;
#pragma unroll
      for (int i = 0; i < NV; ++i) off[i] = (uint32_t)((t / F4_ROW + ROWS_PER_PASS * i) * ld + col);
    }
  }

  __device__ __forceinline__ void load(const float *__restrict__ base, int ld, int k0, int lk,
                                       int hd) {
    if constexpr (VEC) {
      const float *tile = base + (size_t)k0 * ld;  // wave-uniform
      const uint32_t lim = (uint32_t)(min(lk - 1 - k0, BN - 1) * ld) + col;
#pragma unroll
      for (int i = 0; i < NV; ++i) r[i] = *reinterpret_cast<const vf4 *>(tile + min(off[i], lim));
    } else {
      const int t = threadIdx.x;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int e = t + FA_THREADS * i;
        const int row = e / HD, c = e % HD;
        const int key = k0 + row;
        s[i] = (key < lk && c < hd) ? base[(size_t)key * ld + c] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(float (*lds)[HD + 4]) {
    const int t = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
        *reinterpret_cast<vf4 *>(&lds[t / F4_ROW + ROWS_PER_PASS * i][col]) = r[i];
    } else {
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int e = t + FA_THREADS * i;
        lds[e / HD][e % HD] = s[i];
      }
    }
  }
};

// max / sum of a value over the two half-waves (lanes l and l ^ 32) with
// v_permlane32_swap: both results hold the value of lane l % 32 and of lane
// l % 32 + 32.
__device__ __forceinline__ float halves_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max of three scores.  The scores come from MFMA accumulators and are
// never signalling NaNs, so the IEEE quieting that fmaxf otherwise adds to
// each operand is dropped (one v_max3_f32 instead of five instructions).
__device__ __forceinline__ float max3_scores(float a, float b, float c) {
#pragma float_control(precise, off)
  return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// Growth of the running max (log2 units) tolerated before the output is
// rescaled: probabilities stay <= 2^8, far from fp32 overflow.
constexpr float kRescaleThreshold = 8.0f;

// Offset of accumulator register r's key inside its 32-key sub-block for a
// lane of half-wave h: 8 * (r / 4) + 4 * h + r % 4 (the 32x32 MFMA D layout).
__device__ __forceinline__ constexpr int acc_key(int r) { return 8 * (r >> 2) + (r & 3); }

template <int HD, int BN, bool CAUSAL, bool HAS_MASK, bool VEC, bool PAIR>
__global__ void __launch_bounds__(FA_THREADS, 2) flash_fwd_kernel(const FlashArgs a) {
  constexpr int NKB = BN / 32;   // 32-key sub-blocks per tile
  constexpr int NDB = HD / 32;   // 32-wide head-dim blocks of O^T
  constexpr int NQ = HD / 2;     // MFMA k-steps of Q.K
  constexpr int NKG = HD / 8;    // float4 groups of a K row slice
  constexpr int VCH = HD <= 32 ? 16 : 8;  // P.V steps whose V operands are read at once
  __shared__ __attribute__((aligned(16))) float Ks[2][BN][HD + 4];
  __shared__ __attribute__((aligned(16))) float Vs[2][BN][HD + 4];

  // Workgroup i takes (sequence, head) i % n_bh, so with workgroup i on XCD
  // i % 8 all tiles of one (sequence, head) share an XCD and its L2 whenever
  // n_bh is a multiple of 8.  Under the causal rule query tile t sees t + 1
  // key tiles:
  //  * slot p = i / n_bh is tile n_qt - 1 - p, counted from the longest row
  //    down, so every XCD receives the heaviest tiles first and the lightest
  //    last (a near-optimal greedy schedule when the launch spans several
  //    rounds of resident workgroups);
  //  * with PAIR (a launch that fits in one round), slot p runs the pair of
  //    tiles n_qt - 1 - p and p one after the other, so every workgroup has
  //    the same work (n_qt + 1 key tiles; the middle tile of an odd count
  //    runs alone) and the round finishes together.
  // Without the causal rule slot p is tile p.
  const int lid = blockIdx.x;
  const int n_bh = a.n_bh;
  const int bh = lid % n_bh;
  const int slot = lid / n_bh;
  const int npass = (PAIR && 2 * slot + 1 != a.n_qt) ? 2 : 1;
  const int b = bh / a.heads, h = bh % a.heads;
  for (int pass = 0; pass < npass; ++pass) {
  if (pass > 0) __syncthreads();  // the LDS tiles of the first pass are done with
  const int qt = CAUSAL ? (pass == 0 ? a.n_qt - 1 - slot : slot) : slot;
  const int q0 = qt * FA_BM;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, hf = lane >> 5;
  const int qw0 = q0 + wave * 32;   // first query of this wave (wave-uniform)
  const int qi = qw0 + li;          // this lane's query
  const int col0 = h * a.hd;

  const float *__restrict__ kbase = a.k + (size_t)b * a.lk * a.ldk + col0;
  const float *__restrict__ vbase = a.v + (size_t)b * a.lk * a.ldv + col0;

  // Q^T operand: register 4u + r holds q[qi][8u + 4*hf + r].
  float qreg[NQ];
  {
    const float *qrow = a.q + ((size_t)b * a.lq + min(qi, a.lq - 1)) * a.ldq + col0;
    const bool qok = qi < a.lq;
#pragma unroll
    for (int u = 0; u < HD / 8; ++u) {
      const int d = 8 * u + 4 * hf;
      if constexpr (VEC) {
        float4 t4 = *reinterpret_cast<const float4 *>(qrow + d);
        qreg[4 * u + 0] = qok ? t4.x : 0.f;
        qreg[4 * u + 1] = qok ? t4.y : 0.f;
        qreg[4 * u + 2] = qok ? t4.z : 0.f;
        qreg[4 * u + 3] = qok ? t4.w : 0.f;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) qreg[4 * u + r] = (qok && d + r < a.hd) ? qrow[d + r] : 0.f;
      }
    }
    // Q in the exp2 domain: the scores leave the MFMA as s * scale * log2(e)
#pragma unroll
    for (int i = 0; i < NQ; ++i) qreg[i] *= a.scale_log2;
  }

  const int kend = CAUSAL ? min(q0 + FA_BM, a.lk) : a.lk;
  const int n_kt = (kend + BN - 1) / BN;

  KvStage<HD, BN, VEC> sk, sv;
  sk.init(a.ldk);
  sv.init(a.ldv);
  sk.load(kbase, a.ldk, 0, a.lk, a.hd);
  sv.load(vbase, a.ldv, 0, a.lk, a.hd);
  sk.store(Ks[0]);
  sv.store(Vs[0]);
  __syncthreads();

  floatx16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
  // The reference max of this lane's query (exp2 domain) is subtracted by
  // the MFMA itself: the first step of every S^T block starts from negm,
  // -m_run in all 16 entries (0 until the first visible key sets m_run), so
  // the scores come out relative to the reference and p = exp2(score).
  float m_run = -INFINITY;
  float thr = -INFINITY;  // rescale threshold: any visible key until m_run is set
  float l_a = 0.f, l_b = 0.f;  // running sums over this half-wave's keys
  floatx16 negm = {};
  // Last key this lane may attend (the causal diagonal and the sequence end).
  const int key_last = CAUSAL ? min(qi, a.lk - 1) : a.lk - 1;

  const uint8_t *mrow = HAS_MASK ? a.mask + (size_t)min(qi, a.lq - 1) * a.lk : nullptr;

  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const int k0 = kt * BN;
    const bool more = kt + 1 < n_kt;
    // Next tile into registers.  The last iteration re-stages its own tile
    // into the idle buffer (nobody reads it again): an unconditional stage
    // keeps the staging registers out of scratch memory.
    sk.load(kbase, a.ldk, more ? k0 + BN : k0, a.lk, a.hd);
    sv.load(vbase, a.ldv, more ? k0 + BN : k0, a.lk, a.hd);

#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int kb0 = k0 + kb * 32;
      // A sub-block wholly past the sequence end or in this wave's future
      // contributes nothing (every probability would be 0): skip it.
      if (kb0 >= a.lk || (CAUSAL && kb0 > qw0 + 31)) continue;
      const float(*krow)[HD + 4] = &Ks[cur][kb * 32];
      const float(*vrow)[HD + 4] = &Vs[cur][kb * 32];

      // S^T = K Q^T; the K operand group u + 1 is read while group u multiplies.
      floatx16 sacc;
      float4 kcur = *reinterpret_cast<const float4 *>(&krow[li][4 * hf]);
#pragma unroll
      for (int u = 0; u < NKG; ++u) {
        float4 knext;
        if (u + 1 < NKG) knext = *reinterpret_cast<const float4 *>(&krow[li][8 * (u + 1) + 4 * hf]);
        sacc = mfma32x32x2(kcur.x, qreg[4 * u + 0], u == 0 ? negm : sacc);
        sacc = mfma32x32x2(kcur.y, qreg[4 * u + 1], sacc);
        sacc = mfma32x32x2(kcur.z, qreg[4 * u + 2], sacc);
        sacc = mfma32x32x2(kcur.w, qreg[4 * u + 3], sacc);
        if (u + 1 < NKG) kcur = knext;
      }
      // V^T operands of the first P.V chunk, in flight during the softmax.
      float vr[VCH][NDB];
#pragma unroll
      for (int st = 0; st < VCH; ++st)
#pragma unroll
        for (int db = 0; db < NDB; ++db) vr[st][db] = vrow[acc_key(st) + 4 * hf][db * 32 + li];

      // Masking (wave-uniform decision): the diagonal, the sequence end, a mask.
      if (HAS_MASK || kb0 + 31 > (CAUSAL ? min(qw0, a.lk - 1) : a.lk - 1)) {
        const int last_vis = key_last - kb0 - 4 * hf;  // last visible offset for this lane
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          bool ok = acc_key(r) <= last_vis;
          if (HAS_MASK) {
            const int key = min(kb0 + acc_key(r) + 4 * hf, a.lk - 1);
            ok = ok && qi < a.lq && mrow[key] != 0;
          }
          sacc[r] = ok ? sacc[r] : -INFINITY;
        }
      }
      // tile max relative to the reference (-inf: no visible key)
      float smax = max3_scores(sacc[0], sacc[1], sacc[2]);
#pragma unroll
      for (int r = 3; r < 15; r += 2) smax = max3_scores(smax, sacc[r], sacc[r + 1]);
      smax = max3_scores(smax, sacc[15], -INFINITY);
      smax = halves_max(smax);

      // Lazy rescale: the first visible key sets the reference, later only a
      // rise of more than the threshold moves it (the scores shift with it).
      const bool need = smax > thr;
      if (__builtin_amdgcn_ballot_w64(need)) {
        const bool first = m_run == -INFINITY;
        const float shift = need ? smax : 0.f;
        const float alpha = (need && !first) ? fast_exp2(-smax) : 1.0f;  // o and l are 0 before the first key
        m_run = need ? (first ? smax : m_run + smax) : m_run;
        thr = m_run == -INFINITY ? -INFINITY : kRescaleThreshold;
        l_a *= alpha;
        l_b *= alpha;
        const float nref = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sacc[r] -= shift;
          negm[r] = nref;
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(sacc[r]);
        sacc[r] = p;
        if (r & 1) l_b += p;
        else l_a += p;
      }

      // O^T += V^T P^T: accumulator r of the lane holds the probability of
      // key acc_key(r) + 4*hf, the key B-operand slot of MFMA step r needs.
#pragma unroll
      for (int ch = 0; ch < 16 / VCH; ++ch) {
        if (ch > 0) {
#pragma unroll
          for (int st = 0; st < VCH; ++st)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
              vr[st][db] = vrow[acc_key(ch * VCH + st) + 4 * hf][db * 32 + li];
        }
#pragma unroll
        for (int st = 0; st < VCH; ++st)
#pragma unroll
          for (int db = 0; db < NDB; ++db) oacc[db] = mfma32x32x2(vr[st][db], sacc[ch * VCH + st], oacc[db]);
      }
    }

    sk.store(Ks[cur ^ 1]);
    sv.store(Vs[cur ^ 1]);
    __syncthreads();
  }

  // Normalise and store: lane holds query qi, dims db*32 + 8*(r/4) + 4*hf + r%4.
  const float l_tot = halves_sum(l_a + l_b);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  // For the backward pass: p = exp2(s * scale * log2(e) - lse) recovers every
  // probability (+inf for a row with no visible key, whose p are all 0).
  if (a.lse && hf == 0 && qi < a.lq)
    a.lse[(size_t)bh * a.lq + qi] = l_tot > 0.f ? m_run + __log2f(l_tot) : INFINITY;
  if (qi < a.lq) {
    float *orow = a.o + ((size_t)b * a.lq + qi) * a.ldo + col0;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        if constexpr (VEC) {
          *reinterpret_cast<float4 *>(orow + d) =
              make_float4(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv,
                          oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (d + r < a.hd) orow[d + r] = oacc[db][4 * g + r] * inv;
        }
      }
    }
  }
  }  // pass
}

// Head dims above 128: one workgroup per (sequence, head, query), keys in
// chunks of 256 with an online softmax; correctness path only.
__global__ void __launch_bounds__(256) flash_generic_kernel(const FlashArgs a, int causal) {
  extern __shared__ float sm[];  // q[hd] | o[hd] | p[256] | red[8]
  float *qv = sm;
  float *ov = sm + a.hd;
  float *pv = ov + a.hd;
  float *red = pv + 256;
  const int row = blockIdx.x;  // b * lq + i
  const int b = row / a.lq, i = row % a.lq;
  const int h = blockIdx.y;
  const int col0 = h * a.hd;
  const int t = threadIdx.x;
  const float *qrow = a.q + ((size_t)b * a.lq + i) * a.ldq + col0;
  for (int d = t; d < a.hd; d += 256) {
    qv[d] = qrow[d];
    ov[d] = 0.f;
  }
  __syncthreads();
  const int usable = causal ? min(i + 1, a.lk) : a.lk;
  float m_run = -INFINITY, l_run = 0.f;
  for (int c0 = 0; c0 < usable; c0 += 256) {
    const int j = c0 + t;
    float s = -INFINITY;
    if (j < usable && (!a.mask || a.mask[(size_t)i * a.lk + j])) {
      const float *krow = a.k + ((size_t)b * a.lk + j) * a.ldk + col0;
      float acc = 0.f;
      for (int d = 0; d < a.hd; ++d) acc += qv[d] * krow[d];
      s = acc * a.scale_log2;
    }
    float mx = s;
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    const float p = fast_exp2(s - m_use);
    pv[t] = p;
    float ps = p;
    for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
    if ((t & 63) == 0) red[4 + (t >> 6)] = ps;
    __syncthreads();
    l_run = l_run * alpha + (red[4] + red[5] + red[6] + red[7]);
    m_run = m_new;
    const int n = min(256, usable - c0);
    for (int d = t; d < a.hd; d += 256) {
      float acc = ov[d] * alpha;
      for (int jj = 0; jj < n; ++jj)
        acc += pv[jj] * a.v[((size_t)b * a.lk + c0 + jj) * a.ldv + col0 + d];
      ov[d] = acc;
    }
    __syncthreads();
  }
  const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
  float *orow = a.o + ((size_t)b * a.lq + i) * a.ldo + col0;
  for (int d = t; d < a.hd; d += 256) orow[d] = ov[d] * inv;
}

template <int HD, int BN, bool CAUSAL, bool HAS_MASK>
void launch_tpl(FlashArgs a, bool vec, hipStream_t st) {
  // Pairs of causal tiles when one tile per workgroup would fit in a single
  // round of resident workgroups (four per CU), so that the round lasts as
  // long as its longest tile, and the pairs still give every CU two
  // workgroups (fewer would leave SIMDs with a single wave).
  const long long cus = num_cus();
  const bool pair = CAUSAL && a.n_qt > 1 && (long long)a.n_bh * a.n_qt <= 4 * cus &&
                    (long long)a.n_bh * ((a.n_qt + 1) / 2) >= 2 * cus;
  a.total = pair ? a.n_bh * ((a.n_qt + 1) / 2) : a.n_bh * a.n_qt;
  if constexpr (CAUSAL) {
    if (pair) {
      if (vec) flash_fwd_kernel<HD, BN, true, HAS_MASK, true, true><<<dim3(a.total), dim3(FA_THREADS), 0, st>>>(a);
      else flash_fwd_kernel<HD, BN, true, HAS_MASK, false, true><<<dim3(a.total), dim3(FA_THREADS), 0, st>>>(a);
      return;
    }
  }
  if (vec)
    flash_fwd_kernel<HD, BN, CAUSAL, HAS_MASK, true, false><<<dim3(a.total), dim3(FA_THREADS), 0, st>>>(a);
  else
    flash_fwd_kernel<HD, BN, CAUSAL, HAS_MASK, false, false><<<dim3(a.total), dim3(FA_THREADS), 0, st>>>(a);
}

template <int HD, int BN>
void launch_hd(const FlashArgs &a, bool causal, bool vec, hipStream_t st) {
  const bool m = a.mask != nullptr;
  if (causal) {
    if (m) launch_tpl<HD, BN, true, true>(a, vec, st);
    else launch_tpl<HD, BN, true, false>(a, vec, st);
  } else {
    if (m) launch_tpl<HD, BN, false, true>(a, vec, st);
    else launch_tpl<HD, BN, false, false>(a, vec, st);
  }
}

}  // namespace
}  // namespace cdml

using namespace cdml;

namespace cdml {

// Launches the forward kernels; the arguments are validated by the caller.
// causal here admits lq != lk (key j visible to query i iff j <= i).
int flash_forward(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                  float *o, int ldo, float *lse, int batch, int lq, int lk, int dim, int num_heads,
                  float scale, bool causal, const uint8_t *mask, hipStream_t st) {
  FlashArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.mask = mask;
  a.ldq = ldq;
  a.ldk = ldk;
  a.ldv = ldv;
  a.ldo = ldo;
  a.lq = lq;
  a.lk = lk;
  a.heads = num_heads;
  a.hd = dim / num_heads;
  a.scale_log2 = scale * kLog2e;

  const int hd = a.hd;
  if (hd > 128) {
    if (lse) return fail(CDML_E_INVALID, "flash_forward: no row statistics above head dim 128");
    a.n_qt = lq;
    size_t smem = sizeof(float) * (2 * (size_t)hd + 256 + 8);
    if (smem > 160 * 1024) return fail(CDML_E_INVALID, "cdml_sdpa_fwd: head dim %d too large", hd);
    flash_generic_kernel<<<dim3(batch * lq, num_heads), dim3(256), smem, st>>>(a, causal);
    return check_launch("flash_generic_kernel");
  }
  const int hd_pad = hd <= 32 ? 32 : (hd <= 64 ? 64 : 128);
  const bool vec = hd == hd_pad && ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && ldo % 4 == 0 &&
                   aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  a.n_qt = (lq + FA_BM - 1) / FA_BM;
  a.n_bh = batch * num_heads;
  long long total = (long long)batch * num_heads * a.n_qt;
  if (total > (1LL << 30)) return fail(CDML_E_INVALID, "cdml_sdpa_fwd: problem too large");
  a.total = (int)total;
  a.padded = pad_to_xcd(a.total);
  if (hd_pad == 32) launch_hd<32, 64>(a, causal, vec, st);
  else if (hd_pad == 64) launch_hd<64, 32>(a, causal, vec, st);
  else launch_hd<128, 32>(a, causal, vec, st);
  return check_launch("flash_fwd_kernel");
}

}  // namespace cdml

namespace {

int sdpa_fwd_impl(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv, float *o,
                  int ldo, float *lse, int batch, int lq, int lk, int dim, int num_heads, float scale,
                  int causal, const uint8_t *mask, cdml_stream stream) {
  if (batch < 0 || lq < 0 || lk < 0 || dim <= 0 || num_heads <= 0)
    return fail(CDML_E_INVALID, "cdml_sdpa_fwd: bad size (batch %d, lq %d, lk %d, dim %d, heads %d)",
                batch, lq, lk, dim, num_heads);
  if (dim % num_heads != 0)
    return fail(CDML_E_INVALID, "cdml_sdpa_fwd: dim %d not divisible by num_heads %d", dim, num_heads);
  if (causal && lq != lk)
    return fail(CDML_E_CAUSAL, "cdml_sdpa_fwd: causal attention requires lq == lk (got %d, %d)", lq, lk);
  if (ldq < dim || ldk < dim || ldv < dim || ldo < dim)
    return fail(CDML_E_INVALID, "cdml_sdpa_fwd: row stride smaller than dim");
  if ((long long)ldk * 128 > INT32_MAX || (long long)ldv * 128 > INT32_MAX)
    return fail(CDML_E_INVALID, "cdml_sdpa_fwd: row stride above %d elements", INT32_MAX / 128);
  if (batch == 0 || lq == 0) return CDML_OK;
  if (lk == 0) return fail(CDML_E_INVALID, "cdml_sdpa_fwd: lk must be >= 1");
  if (!q || !k || !v || !o) return fail(CDML_E_INVALID, "cdml_sdpa_fwd: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  return flash_forward(q, ldq, k, ldk, v, ldv, o, ldo, lse, batch, lq, lk, dim, num_heads, scale,
                       causal != 0, mask, as_hip(stream));
}

}  // namespace

extern "C" int cdml_sdpa_fwd(const float *q, int ldq, const float *k, int ldk, const float *v,
                             int ldv, float *o, int ldo, int batch, int lq, int lk, int dim,
                             int num_heads, float scale, int causal, const uint8_t *mask,
                             cdml_stream stream) {
  return sdpa_fwd_impl(q, ldq, k, ldk, v, ldv, o, ldo, nullptr, batch, lq, lk, dim, num_heads, scale,
                       causal, mask, stream);
}

extern "C" int cdml_sdpa_fwd_lse(const float *q, int ldq, const float *k, int ldk, const float *v,
                                 int ldv, float *o, int ldo, float *lse, int batch, int lq, int lk,
                                 int dim, int num_heads, float scale, int causal,
                                 const uint8_t *mask, cdml_stream stream) {
  if (!lse) return fail(CDML_E_INVALID, "cdml_sdpa_fwd_lse: lse is NULL");
  return sdpa_fwd_impl(q, ldq, k, ldk, v, ldv, o, ldo, lse, batch, lq, lk, dim, num_heads, scale, causal,
                       mask, stream);
}
