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
//                   (scale * log2 e folded into Q), masked keys -inf.
//   O^T += V^T P^T  the probabilities stay in the S accumulator registers:
//                   accumulator r of a lane holds key 8*(r/4) + 4*h + r%4,
//                   exactly the key the B operand of MFMA step r needs, so
//                   P is consumed in place; V is staged transposed in LDS,
//                   so one 16-byte read feeds four MFMA steps.
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

// Division by a launch-constant divisor d >= 1 for dividends 0 <= x < 2^31:
// x / d = (x * m) >> l with l = 31 + ceil(log2 d) and m = ceil(2^l / d) < 2^32
// (the error m * d - 2^l is below d, so x * error < 2^l for every such x).
// Block-uniform dividends keep the division on the scalar unit.
struct UDiv {
  uint32_t m;
  int l;
  static UDiv make(uint32_t d) {
    if (d == 0) d = 1;  // no launch divides by it
    int s = 0;
    while ((1ull << s) < d) ++s;
    const int l = 31 + s;
    return {(uint32_t)(((1ull << l) + d - 1) / d), l};
  }
  __device__ __forceinline__ int div(int x) const { return (int)(((uint64_t)(uint32_t)x * m) >> l); }
};

struct FlashArgs {
  const float *q, *k, *v;
  float *o;
  float *lse;  // optional [batch * heads][lq]: log2 of each row's softmax normaliser
  const uint8_t *mask;
  int ldq, ldk, ldv, ldo;
  int lq, lk, heads, hd;
  float scale_log2;
  int n_qt, n_bh, n_items;  // query tiles per sequence, (sequence, head) pairs, n_bh * n_qt
  UDiv by_bh, by_heads;     // division by n_bh and by heads
  int fast;                 // sub-blocks may skip their maximum (see try_fast)
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
  uint32_t off[VEC ? NV : 1];  // byte offsets of this thread's rows in a tile
  int col;

  __device__ __forceinline__ void init(int ld) {
    if constexpr (VEC) {
      const int t = threadIdx.x;
      col = (t % F4_ROW) * 4;
#pragma unroll
      for (int i = 0; i < NV; ++i) off[i] = 4u * (uint32_t)((t / F4_ROW + ROWS_PER_PASS * i) * ld + col);
    }
  }

  __device__ __forceinline__ void load(const float *__restrict__ base, int ld, int k0, int lk,
                                       int hd) {
    if constexpr (VEC) {
      // wave-uniform tile base plus a 32-bit per-lane byte offset (one
      // scalar-base global load per row, no 64-bit address arithmetic)
      const char *tile = reinterpret_cast<const char *>(base + (size_t)k0 * ld);
      const uint32_t lim = 4u * ((uint32_t)(min(lk - 1 - k0, BN - 1) * ld) + col);
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

// Stages one BN x HD tile of V transposed into LDS, Vt[d][key] with row pitch
// BN + 4, so that the P.V step reads the four consecutive keys of one V^T
// column it needs for four MFMA steps in a single 16-byte read.  A thread
// takes two consecutive keys of a 4-wide column group (two 16-byte global
// loads) and writes them as four 8-byte pairs Vt[c + j][2p .. 2p + 1].
// Lanes 8m .. 8m + 7 of a wave take key pairs 0..7 (of an 8-pair block) of
// column group m (of an 8-group block): the sixteen lanes of an 8-byte store
// phase then cover two column groups, whose V^T rows (4 * pitch floats apart,
// 16 banks apart) each receive eight contiguous pairs, so no two lanes share
// a bank, and each 16-byte load instruction still reads 128 contiguous bytes
// of each of 8 rows.  (With consecutive lanes on consecutive column groups
// of one key pair, sixteen lanes' rows fell on two bank groups.)  Rows past
// lk are clamped as in KvStage.
template <int HD, int BN, bool VEC>
struct VtStage {
  static constexpr int NCG = HD / 4;               // 4-wide column groups
  static constexpr int NKP = BN / 2;               // key pairs
  static constexpr int NU = NKP * NCG / FA_THREADS;  // (key pair, column group) units per thread
  static_assert(NKP % 8 == 0 && NCG % 8 == 0, "V tile blocks of 8 key pairs x 8 column groups");
  // key pair and column group of unit u (64 units per 8 x 8 block)
  __device__ __forceinline__ static int unit_kp(int u) { return (u & 7) + 8 * ((u >> 6) % (NKP / 8)); }
  __device__ __forceinline__ static int unit_cg(int u) { return ((u >> 3) & 7) + 8 * ((u >> 6) / (NKP / 8)); }
  static constexpr int NS = BN * HD / FA_THREADS;
  static_assert(NKP * NCG % FA_THREADS == 0, "V tile units must divide the workgroup");
  vf4 r[VEC ? 2 * NU : 1];
  float s[VEC ? 1 : NS];
  uint32_t off[VEC ? NU : 1];  // byte offset of each unit's first row in a tile
  int col[VEC ? NU : 1];

  __device__ __forceinline__ void init(int ld) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = threadIdx.x + FA_THREADS * i;
        col[i] = unit_cg(u) * 4;
        off[i] = 4u * (uint32_t)(2 * unit_kp(u) * ld + col[i]);
      }
    }
  }

  __device__ __forceinline__ void load(const float *__restrict__ base, int ld, int k0, int lk,
                                       int hd) {
    if constexpr (VEC) {
      const char *tile = reinterpret_cast<const char *>(base + (size_t)k0 * ld);
      const uint32_t last = (uint32_t)min(lk - 1 - k0, BN - 1) * (uint32_t)ld;
      const uint32_t row = 4u * (uint32_t)ld;
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const uint32_t lim = 4u * (last + col[i]);
        r[2 * i] = *reinterpret_cast<const vf4 *>(tile + min(off[i], lim));
        r[2 * i + 1] = *reinterpret_cast<const vf4 *>(tile + min(off[i] + row, lim));
      }
    } else {
      const int t = threadIdx.x;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int e = t + FA_THREADS * i;
        const int rw = e / HD, c = e % HD;
        const int key = k0 + rw;
        s[i] = (key < lk && c < hd) ? base[(size_t)key * ld + c] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(float (*lds)[BN + 4]) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = threadIdx.x + FA_THREADS * i;
        const int kp = 2 * unit_kp(u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          typedef float vf2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<vf2 *>(&lds[col[i] + j][kp]) = vf2{r[2 * i][j], r[2 * i + 1][j]};
        }
      }
    } else {
      const int t = threadIdx.x;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int e = t + FA_THREADS * i;
        lds[e % HD][e / HD] = s[i];
      }
    }
  }
};

// max / sum of a value over the two half-waves (lanes l and l ^ 32) with
// v_permlane32_swap: both results hold the value of lane l % 32 and of lane
// l % 32 + 32.
__device__ __forceinline__ float halves_max(float x) {
#pragma float_control(precise, off)
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));  // scores: no signalling NaN
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

// A sub-block whose per-lane probability sum stays at or below this bound is
// accumulated without looking at its maximum: no probability exceeds it, so
// nothing overflows (the running sums stay below 2^32 times the key count).
constexpr float kFastSumLimit = 4294967296.0f;  // 2^32

// Which query tiles a workgroup runs, one after the other.  Item i of a
// launch is (sequence, head) i % n_bh and, under the causal rule, query tile
// n_qt - 1 - i / n_bh (heaviest rows first), else tile i / n_bh.
//  * kOne: workgroup i runs item i.  With workgroup i on XCD i % 8, all tiles
//    of one (sequence, head) share an XCD and its L2 whenever n_bh is a
//    multiple of 8, and every XCD receives the heaviest tiles first (a
//    near-optimal greedy schedule for a launch of several rounds).
//  * kPair (causal launches that fit in one round): workgroup i runs tiles
//    n_qt - 1 - p and p of its (sequence, head), p = i / n_bh, so every
//    workgroup has the same work (n_qt + 1 key tiles; the middle tile of an
//    odd count runs alone) and the round finishes together.
// The last key tile of a workgroup's first item prefetches the first key tile
// and the Q rows of the second.
enum { kOne = 0, kPair = 1 };

struct Item {
  int bh, qt;
};

template <bool CAUSAL, int SCHED>
__device__ __forceinline__ bool item_at(const FlashArgs &a, int k, Item &it) {
  const int i = blockIdx.x;
  if (SCHED == kPair) {
    const int slot = a.by_bh.div(i);
    it.bh = i - slot * a.n_bh;
    if (k == 0) it.qt = a.n_qt - 1 - slot;
    else if (k == 1 && 2 * slot + 1 != a.n_qt) it.qt = slot;
    else return false;
    return true;
  } else if (k > 0) {
    return false;
  }
  const int slot = a.by_bh.div(i);
  it.bh = i - slot * a.n_bh;
  it.qt = CAUSAL ? a.n_qt - 1 - slot : slot;
  return true;
}

// Q^T operand of a wave: register 4u + r holds q[qi][8u + 4*hf + r], not yet
// scaled.  Rows past lq read row lq - 1: they are computed but never stored.
template <int HD, bool VEC>
__device__ __forceinline__ void load_q(float (&qreg)[HD / 2], const FlashArgs &a, int b, int col0, int qi,
                                       int hf) {
  const float *qrow = a.q + ((size_t)b * a.lq + min(qi, a.lq - 1)) * a.ldq + col0;
#pragma unroll
  for (int u = 0; u < HD / 8; ++u) {
    const int d = 8 * u + 4 * hf;
    if constexpr (VEC) {
      const vf4 t4 = *reinterpret_cast<const vf4 *>(qrow + d);
#pragma unroll
      for (int r = 0; r < 4; ++r) qreg[4 * u + r] = t4[r];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) qreg[4 * u + r] = d + r < a.hd ? qrow[d + r] : 0.f;
    }
  }
}

// The online softmax of one wave's 32 query rows (one per lane % 32) over
// 32-key sub-blocks.
template <int HD, bool HAS_MASK>
struct OnlineRows {
  static constexpr int NDB = HD / 32;     // 32-wide head-dim blocks of O^T
  static constexpr int NQ = HD / 2;       // MFMA k-steps of Q.K
  static constexpr int NKG = HD / 8;      // float4 groups of a K row slice
  // P.V steps whose V operands are read at once (8: at head dim 32 every
  // variant but the masked ones keeps four waves per SIMD)
  static constexpr int VCH = 8;
  static constexpr int NVG = VCH / 4;            // 16-byte V^T reads per chunk and head-dim block
  floatx16 oacc[NDB];
  // The reference max of this lane's query (exp2 domain) is subtracted by
  // the MFMA itself: the first step of every S^T block starts from negm,
  // -m_run in all 16 entries (0 until the first visible key sets m_run), so
  // the scores come out relative to the reference and p = exp2(score).
  floatx16 negm;
  float m_run, thr;  // thr: rescale threshold, any visible key until m_run is set
  float l_a, l_b;    // running sums over this half-wave's keys
  bool warm;         // every lane of the wave has its reference (wave-uniform)

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[db][r] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) negm[r] = 0.f;
    m_run = -INFINITY;
    thr = -INFINITY;
    l_a = l_b = 0.f;
    warm = false;
  }

  // Sets the scores of keys this lane may not attend to -inf: keys past
  // last_vis (offset within the sub-block for this lane's half), and with
  // HAS_MASK also keys whose mask byte mrow[min(kb0 + offset, key_cap)] is 0
  // or any key when !row_ok.
  __device__ __forceinline__ void apply_mask(floatx16 &sacc, int hf, int last_vis, const uint8_t *mrow, int kb0,
                                             int key_cap, bool row_ok) const {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bool ok = acc_key(r) <= last_vis;
      if (HAS_MASK) {
        const int key = min(kb0 + acc_key(r) + 4 * hf, key_cap);
        ok = ok && row_ok && mrow[key] != 0;
      }
      sacc[r] = ok ? sacc[r] : -INFINITY;
    }
  }

  // O^T += V^T P^T: accumulator r of the lane holds the probability of key
  // acc_key(r) + 4*hf, the key B-operand slot of MFMA step r needs.  vr holds
  // the first chunk's V^T operands.
  template <int VP>
  __device__ __forceinline__ void accumulate_pv(const floatx16 &p, vf4 (&vr)[NVG][NDB], const float (*vt)[VP],
                                                int key0, int li, int hf) {
#pragma unroll
    for (int ch = 0; ch < 16 / VCH; ++ch) {
      if (ch > 0) {
#pragma unroll
        for (int g = 0; g < NVG; ++g)
#pragma unroll
          for (int db = 0; db < NDB; ++db)
            vr[g][db] = *reinterpret_cast<const vf4 *>(&vt[db * 32 + li][key0 + 8 * (ch * NVG + g) + 4 * hf]);
      }
#pragma unroll
      for (int st = 0; st < VCH; ++st)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          oacc[db] = mfma32x32x2(vr[st / 4][db][st % 4], p[ch * VCH + st], oacc[db]);
    }
  }

  // The common sub-block once every row has its reference: probabilities and
  // their per-lane sum first, and only if some lane's sum is above 2^32 (a
  // score far above the reference) or NaN does the caller take the full path
  // (consume) on recomputed scores.  sacc is turned into probabilities in
  // place; on false the running state is unchanged and sacc is garbage.
  template <int VP>
  __device__ __forceinline__ bool try_fast(floatx16 &sacc, const float (*vt)[VP], int key0, int li, int hf,
                                           bool masked, int last_vis, const uint8_t *mrow, int kb0, int key_cap,
                                           bool row_ok) {
    vf4 vr[NVG][NDB];
#pragma unroll
    for (int g = 0; g < NVG; ++g)
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        vr[g][db] = *reinterpret_cast<const vf4 *>(&vt[db * 32 + li][key0 + 8 * g + 4 * hf]);
    if (HAS_MASK || masked) apply_mask(sacc, hf, last_vis, mrow, kb0, key_cap, row_ok);
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = fast_exp2(sacc[r]);
    // pairwise sum (a tree of depth 4)
    float s8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) s8[i] = sacc[2 * i] + sacc[2 * i + 1];
    const float ps = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
    if (__builtin_amdgcn_ballot_w64(!(ps <= kFastSumLimit))) return false;
    l_a += ps;
    accumulate_pv(sacc, vr, vt, key0, li, hf);
    return true;
  }

  // S^T = K Q^T for the 32 keys whose rows start at krow; the K operand group
  // u + 1 is read while group u multiplies.
  template <int KP>
  __device__ __forceinline__ floatx16 scores(const float (*krow)[KP], const float (&qreg)[NQ], int li,
                                             int hf) const {
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
    return sacc;
  }

  // Softmax of one sub-block's scores and O^T += V^T P^T.  vt: V^T rows
  // (pitch VP) whose columns key0 .. key0 + 31 are this sub-block's keys.
  // masked (wave-uniform): some key of the sub-block may be invisible (see
  // apply_mask).
  template <int VP>
  __device__ __forceinline__ void consume(floatx16 sacc, const float (*vt)[VP], int key0, int li, int hf,
                                          bool masked, int last_vis, const uint8_t *mrow, int kb0,
                                          int key_cap, bool row_ok) {
    // V^T operands of the first P.V chunk, in flight during the softmax: steps
    // 4g .. 4g + 3 take keys 8g + 4h .. 8g + 4h + 3 of column db * 32 + li.
    vf4 vr[NVG][NDB];
#pragma unroll
    for (int g = 0; g < NVG; ++g)
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        vr[g][db] = *reinterpret_cast<const vf4 *>(&vt[db * 32 + li][key0 + 8 * g + 4 * hf]);

    if (HAS_MASK || masked) apply_mask(sacc, hf, last_vis, mrow, kb0, key_cap, row_ok);
    // tile max relative to the reference (-inf: no visible key)
    // (a tree of depth 3: eight v_max3 whose inputs do not wait on each other)
    const float m0 = max3_scores(sacc[0], sacc[1], sacc[2]);
    const float m1 = max3_scores(sacc[3], sacc[4], sacc[5]);
    const float m2 = max3_scores(sacc[6], sacc[7], sacc[8]);
    const float m3 = max3_scores(sacc[9], sacc[10], sacc[11]);
    const float m4 = max3_scores(sacc[12], sacc[13], sacc[14]);
    float smax = max3_scores(max3_scores(m0, m1, m2), max3_scores(m3, m4, sacc[15]), -INFINITY);
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
      const float nref = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[r] -= shift;
        negm[r] = nref;
      }
      if (__builtin_amdgcn_ballot_w64(need && !first)) {  // not at a row's first visible key
        l_a *= alpha;
        l_b *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp2(sacc[r]);
      sacc[r] = p;
      if (r & 1) l_b += p;
      else l_a += p;
    }
    warm = !__builtin_amdgcn_ballot_w64(m_run == -INFINITY);
    accumulate_pv(sacc, vr, vt, key0, li, hf);
  }

  // Normalise and store row qi of (sequence b, head bh): the lane holds dims
  // db*32 + 8*(r/4) + 4*hf + r%4.  For the backward pass the row statistic
  // lse = m + log2(l) recovers every probability as exp2(s * scale * log2 e
  // - lse) (+inf for a row with no visible key, whose p are all 0).
  template <bool VEC>
  __device__ __forceinline__ void store(const FlashArgs &a, int bh, int b, int qi, int col0, int hf) const {
    const float l_tot = halves_sum(l_a + l_b);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
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
  }
};

template <int HD, int BN, bool CAUSAL, bool HAS_MASK, bool VEC, int SCHED>
__global__ void __launch_bounds__(FA_THREADS, 2) flash_fwd_kernel(const FlashArgs a) {
  constexpr int NKB = BN / 32;   // 32-key sub-blocks per tile
  constexpr int NQ = HD / 2;     // MFMA k-steps of Q.K
  __shared__ __attribute__((aligned(16))) float Ks[2][BN][HD + 4];
  __shared__ __attribute__((aligned(16))) float Vt[2][HD][BN + 4];  // V transposed

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, hf = lane >> 5;

  KvStage<HD, BN, VEC> sk;
  VtStage<HD, BN, VEC> sv;
  sk.init(a.ldk);
  sv.init(a.ldv);

  // The first item: its Q rows and first key tile.
  Item it;
  item_at<CAUSAL, SCHED>(a, 0, it);
  float qreg[NQ];
  {
    const int b = a.by_heads.div(it.bh), col0 = (it.bh - b * a.heads) * a.hd;
    load_q<HD, VEC>(qreg, a, b, col0, it.qt * FA_BM + wave * 32 + li, hf);
    sk.load(a.k + (size_t)b * a.lk * a.ldk + col0, a.ldk, 0, a.lk, a.hd);
    sv.load(a.v + (size_t)b * a.lk * a.ldv + col0, a.ldv, 0, a.lk, a.hd);
  }
  sk.store(Ks[0]);
  sv.store(Vt[0]);
  __syncthreads();
  int buf = 0;  // LDS buffer holding the current key tile

  for (int k = 0;; ++k) {
    const int b = a.by_heads.div(it.bh), h = it.bh - b * a.heads;
    const int q0 = it.qt * FA_BM;
    const int qw0 = q0 + wave * 32;   // first query of this wave (wave-uniform)
    const int qi = qw0 + li;          // this lane's query
    const int col0 = h * a.hd;
    const float *__restrict__ kbase = a.k + (size_t)b * a.lk * a.ldk + col0;
    const float *__restrict__ vbase = a.v + (size_t)b * a.lk * a.ldv + col0;

    // Q in the exp2 domain: the scores leave the MFMA as s * scale * log2(e)
#pragma unroll
    for (int i = 0; i < NQ; ++i) qreg[i] *= a.scale_log2;

    Item nx = it;
    const bool has_next = item_at<CAUSAL, SCHED>(a, k + 1, nx);
    const int nb = a.by_heads.div(nx.bh), ncol0 = (nx.bh - nb * a.heads) * a.hd;  // used only with has_next

    const int kend = CAUSAL ? min(q0 + FA_BM, a.lk) : a.lk;
    const int n_kt = (kend + BN - 1) / BN;

    OnlineRows<HD, HAS_MASK> rows;
    rows.init();
    // Last key this lane may attend (the causal diagonal and the sequence end).
    const int key_last = CAUSAL ? min(qi, a.lk - 1) : a.lk - 1;
    const uint8_t *mrow = HAS_MASK ? a.mask + (size_t)min(qi, a.lq - 1) * a.lk : nullptr;

    for (int kt = 0; kt < n_kt; ++kt) {
      const int cur = buf;
      const int k0 = kt * BN;
      const bool last = kt + 1 == n_kt;
      // Next tile into registers: this item's next tile, else the next
      // item's first tile.  Without a next item the last iteration re-stages
      // its own tile into the idle buffer (nobody reads it again): an
      // unconditional stage keeps the staging registers out of scratch memory.
      {
        const bool to_next = last && has_next;
        const int ks = !last ? k0 + BN : (has_next ? 0 : k0);
        sk.load(to_next ? a.k + (size_t)nb * a.lk * a.ldk + ncol0 : kbase, a.ldk, ks, a.lk, a.hd);
        sv.load(to_next ? a.v + (size_t)nb * a.lk * a.ldv + ncol0 : vbase, a.ldv, ks, a.lk, a.hd);
      }
      bool q_next = false;  // the next item's Q rows are loading

#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const int kb0 = k0 + kb * 32;
        // A sub-block wholly past the sequence end or in this wave's future
        // contributes nothing (every probability would be 0), and a wave
        // whose rows all lie past lq (the last tile of a ragged length) has
        // nothing to compute: skip.
        if (kb0 >= a.lk || qw0 >= a.lq || (CAUSAL && kb0 > qw0 + 31)) continue;
        floatx16 sacc = rows.scores(&Ks[cur][kb * 32], qreg, li, hf);
        // Q is last read by the final sub-block of the last tile: the next
        // item's Q rows load while this sub-block's softmax and P.V run.
        if (kb == NKB - 1 && last && has_next) {
          load_q<HD, VEC>(qreg, a, nb, ncol0, nx.qt * FA_BM + wave * 32 + li, hf);
          q_next = true;
        }
        // masking is needed on the diagonal and at the sequence end (wave-uniform)
        const bool masked = kb0 + 31 > (CAUSAL ? min(qw0, a.lk - 1) : a.lk - 1);
        const int last_vis = key_last - kb0 - 4 * hf;
        // Once every row has its reference, a sub-block is accumulated without
        // its maximum unless its probabilities come out unbounded; then its
        // scores are recomputed (K is still in LDS and Q in registers: a kOne
        // workgroup loads no further Q rows) for the full path.  Explicit
        // masks keep the full path (the mask reads in both paths would cost
        // the registers of a fourth wave per SIMD), and so do launches of
        // fewer than three workgroups per CU, whose waves cannot hide the wait
        // of the check before the P.V step (every paired launch is one).
        bool done = false;
        if (!HAS_MASK && SCHED == kOne && a.fast && rows.warm) {
          done = rows.try_fast(sacc, Vt[cur], kb * 32, li, hf, masked, last_vis, mrow, kb0, a.lk - 1, qi < a.lq);
          if (!done) {
            // K is read from LDS again (the compiler may not keep the first
            // scores, which would hold them live through the fast path)
            asm volatile("" ::: "memory");
            sacc = rows.scores(&Ks[cur][kb * 32], qreg, li, hf);
          }
        }
        if (!done)
          rows.consume(sacc, Vt[cur], kb * 32, li, hf, masked, last_vis, mrow, kb0, a.lk - 1, qi < a.lq);
      }
      // a wave that skipped the final sub-block loads the next Q rows here
      if (last && has_next && !q_next) load_q<HD, VEC>(qreg, a, nb, ncol0, nx.qt * FA_BM + wave * 32 + li, hf);

      sk.store(Ks[cur ^ 1]);
      sv.store(Vt[cur ^ 1]);
      __syncthreads();
      buf = cur ^ 1;
    }
    rows.template store<VEC>(a, it.bh, b, qi, col0, hf);
    if (!has_next) break;
    it = nx;
  }
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

template <int HD, int BN, bool CAUSAL, bool HAS_MASK, bool VEC>
void launch_sched(const FlashArgs &a, hipStream_t st) {
  // Pairs of causal tiles when one tile per workgroup would fit in a single
  // round of resident workgroups (four per CU), so that the round lasts as
  // long as its longest tile, and the pairs still give every CU two
  // workgroups (fewer would leave SIMDs with a single wave).  Only for
  // sequences of at most four query tiles: with more, one workgroup per tile
  // (which keeps the no-maximum sub-block path) measured 3-6% faster
  // (c2, 16 x 1024 with 8 heads of 64: 161-167 against 172-175 us; 8 x 2048
  // heads of 64: 294-296 against 310 us), while 32 x 512 heads of 64 still
  // gain 4-6% from pairs.
  const long long cus = num_cus();
  FlashArgs b = a;
  if constexpr (CAUSAL) {
    const long long pairs = (long long)a.n_bh * ((a.n_qt + 1) / 2);
    if (a.n_qt > 1 && a.n_qt <= 4 && (long long)a.n_items <= 4 * cus && pairs >= 2 * cus) {
      b.fast = 0;
      flash_fwd_kernel<HD, BN, CAUSAL, HAS_MASK, VEC, kPair><<<dim3((unsigned)pairs), dim3(FA_THREADS), 0, st>>>(b);
      return;
    }
  }
  b.fast = (long long)a.n_items >= 3 * cus;
  flash_fwd_kernel<HD, BN, CAUSAL, HAS_MASK, VEC, kOne><<<dim3(a.n_items), dim3(FA_THREADS), 0, st>>>(b);
}

template <int HD, int BN, bool CAUSAL, bool HAS_MASK>
void launch_tpl(const FlashArgs &a, bool vec, hipStream_t st) {
  if (vec) launch_sched<HD, BN, CAUSAL, HAS_MASK, true>(a, st);
  else launch_sched<HD, BN, CAUSAL, HAS_MASK, false>(a, st);
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
  a.n_bh = batch * num_heads;
  a.n_qt = (lq + FA_BM - 1) / FA_BM;
  a.by_bh = UDiv::make((uint32_t)a.n_bh);
  a.by_heads = UDiv::make((uint32_t)num_heads);
  long long total = (long long)batch * num_heads * a.n_qt;
  if (total > (1LL << 30)) return fail(CDML_E_INVALID, "cdml_sdpa_fwd: problem too large");
  a.n_items = (int)total;
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
