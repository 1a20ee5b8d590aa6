// Attention backward for gfx950: MultiHeadAttentionBackward of the reference
// (AccelerationCPU.cs:1011-1280) on fp32 MFMA.
//
// With P = softmax(S), S = scale * Q K^T per (sequence, head) under the
// causal rule (key j visible to query i iff j <= i) and/or a mask:
//   dV = P^T dO,  dP = dO V^T,  dS = P (dP - D) with D_i = sum_j P_ij dP_ij,
//   dQ = scale dS K,  dK = scale dS^T Q.
// D_i equals dO_i . O_i, so the pass runs in four launches:
//   1. the forward kernel with row statistics: O and lse_i (log2 of the
//      softmax normaliser), so that P_ij = exp2(s_ij * scale * log2 e - lse_i);
//   2. bwd_delta_kernel: D = rowsum(dO * O) per head;
//   3. flash_bwd_dkdv_kernel, key-block major: a workgroup owns 128 keys of
//      one (sequence, head), each wave 32 keys whose K and V rows stay in
//      registers; Q, dO, lse and D tiles stream through double-buffered LDS.
//      Per 32-query sub-block: S = Q K^T and dP = dO V^T land with one key
//      per lane and 16 queries per lane in registers, exactly the B operand
//      layout that dV^T += dO^T P and dK^T += Q^T dS need, so P and dS are
//      consumed in place;
//   4. flash_bwd_dq_kernel, query-block major like the forward: S^T = K Q^T
//      and dP^T = V dO^T put one query per lane, dS^T is consumed in place by
//      dQ^T += K^T dS^T.
// Every output element is written by one lane of one workgroup: no atomics,
// and the result is the same on every run.  Head dims below 128 other than
// 32 and 64, or rows that are not 16-byte aligned, run the same kernels at the
// next of 32 / 64 / 128 with zero-filled scalar loads (VEC false) and
// predicated stores; zero columns of Q, K, V and dO leave S, dP and every
// stored gradient column unchanged.  Head dims above 128 take
// flash_bwd_generic_kernel, which follows the reference's per-row loops.
#include "common.h"

namespace cdml {
namespace {

constexpr int BW_THREADS = 256;
constexpr int BW_TILE = 128;  // keys (dK/dV) or queries (dQ) per workgroup
constexpr int kBufferWord3 = 0x00020000;  // gfx9 buffer resource word 3: raw 32-bit dwords
constexpr int kCachePolicyNT = 2;         // buffer instruction cache policy: non-temporal
constexpr float kLog2e = 1.4426950408889634f;

struct BwdArgs {
  const float *q, *k, *v, *dout;
  float *dq, *dk, *dv;
  const float *o;      // forward output [batch * lq][dim] (row stride ldo)
  const float *lse;    // [batch * heads][lq]
  float *delta;        // [batch * heads][lq]
  float *ds;           // stored dS blocks (causal, lq == lk) or NULL
  long long ds_bh;     // floats of ds per (sequence, head)
  const uint8_t *mask; // [lq][lk] or NULL
  int ldq, ldk, ldv, lddo, lddq, lddk, lddv, ldo;
  int batch, lq, lk, dim, heads, hd;
  float scale, scale_log2;
  int n_tiles, total;
  // Inverse rotary embedding applied to dQ and dK as they are stored
  // (cdml_sdpa_bwd_saved_rope): rope_cs[pos * hd / 2 + p] holds (cos, sin) of
  // position pos for pair p, and a row's position is its index in its
  // sequence.  NULL: no rotation.
  const float2 *rope_cs;
};

// The inverse rotation of one pair (x0, x1) = dims (2p, 2p + 1) by (cos, sin)
// t, rounded as rope_qk_table_kernel rounds it (each product before the sum),
// so the fused form stores the same bits as a separate cdml_rope_qk_table.
__device__ __forceinline__ float2 rope_inverse_pair(float x0, float x1, float2 t) {
#pragma clang fp contract(off)
  const float s = -t.y;
  return make_float2(x0 * t.x - x1 * s, x0 * s + x1 * t.x);
}

// Offset of accumulator register r's row inside its 32-row block for a lane of
// half-wave h: 8 * (r / 4) + 4 * h + r % 4 (the 32x32 MFMA D layout).
__device__ __forceinline__ constexpr int acc_row(int r) { return 8 * (r >> 2) + (r & 3); }

// One ROWS x HD tile of a row-major matrix (rows [row0, row0 + ROWS) of the
// head's column block), global -> registers -> LDS.  Each thread's offsets
// inside a tile are fixed; rows past `nrows` are clamped to the last row
// (their contributions are masked or never stored).  Without VEC, columns at
// or past the head dim `hd` read as zero and the rest are scalar loads.
template <int HD, int ROWS, bool VEC>
struct RowStage {
  static constexpr int F4 = HD / 4;
  static constexpr int RPP = BW_THREADS / F4;
  static constexpr int NV = ROWS / RPP;
  static_assert(NV >= 1 && ROWS % RPP == 0, "tile shape");
  vf4 r[NV];
  uint32_t off[NV];
  int col;

  __device__ __forceinline__ void init(int ld) {
    const int t = threadIdx.x;
    col = (t % F4) * 4;
#pragma unroll
    for (int i = 0; i < NV; ++i) off[i] = (uint32_t)((t / F4 + RPP * i) * ld + col);
  }
  __device__ __forceinline__ void load(const float *__restrict__ base, int ld, int row0, int nrows,
                                       int hd) {
    const float *tile = base + (size_t)row0 * ld;
    const uint32_t lim = (uint32_t)(min(nrows - 1 - row0, ROWS - 1) * ld) + col;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if constexpr (VEC) {
        r[i] = *reinterpret_cast<const vf4 *>(tile + min(off[i], lim));
      } else {
        const float *p = tile + min(off[i], lim);
#pragma unroll
        for (int c = 0; c < 4; ++c) r[i][c] = col + c < hd ? p[c] : 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(float (*lds)[HD + 4]) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV; ++i) *reinterpret_cast<vf4 *>(&lds[t / F4 + RPP * i][col]) = r[i];
  }
};

// D[b, h, i] = dO_i . O_i over head h's columns; one thread per (row, head).
// D[b, h, i] = dO[b, i, head h] . O[b, i, head h].  Thread e owns float4 e of
// the flat [batch * lq, dim / 4] view, so a wave reads whole rows (coalesced);
// the HD / 4 consecutive lanes of one head sum their partials with xor
// shuffles (HD / 4 divides 64, so a head never straddles two waves).
template <int HD>
__global__ void __launch_bounds__(256) bwd_delta_kernel(const BwdArgs a) {
  constexpr int G = HD / 4;
  const int d4 = a.dim >> 2;
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long n = (long long)a.batch * a.lq * d4;
  const long long ec = e < n ? e : n - 1;  // every lane joins the shuffles
  const long long row = ec / d4;
  const int c4 = (int)(ec % d4);
  const vf4 x = *reinterpret_cast<const vf4 *>(a.dout + row * a.lddo + 4 * c4);
  const vf4 y = *reinterpret_cast<const vf4 *>(a.o + row * a.ldo + 4 * c4);
  float s = (x[0] * y[0] + x[1] * y[1]) + (x[2] * y[2] + x[3] * y[3]);
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (e < n && c4 % G == 0) {
    const int h = c4 / G;
    const int b = (int)(row / a.lq), i = (int)(row % a.lq);
    a.delta[((size_t)b * a.heads + h) * a.lq + i] = s;
  }
}

// D for any head dim and stride: thread e owns (row e / heads, head e % heads).
__global__ void __launch_bounds__(256) bwd_delta_scalar_kernel(const BwdArgs a) {
  const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
  if (e >= (long long)a.batch * a.lq * a.heads) return;
  const long long row = e / a.heads;
  const int h = (int)(e % a.heads);
  const float *x = a.dout + row * a.lddo + h * a.hd;
  const float *y = a.o + row * a.ldo + h * a.hd;
  float s = 0.f;
  for (int d = 0; d < a.hd; ++d) s += x[d] * y[d];
  const int b = (int)(row / a.lq), i = (int)(row % a.lq);
  a.delta[((size_t)b * a.heads + h) * a.lq + i] = s;
}

// dK and dV.  Workgroup i takes (sequence, head) i % n_bh and key tile
// i / n_bh: under the causal rule the first key tiles are seen by the most
// queries, so the heaviest tiles go out first on every XCD.
//
// With STORE_DS (causal, lq == lk) the kernel also writes every dS sub-block
// it forms, for flash_bwd_dq_ds_kernel: block (query block i, key block j),
// j <= i, holds 32 x 32 floats at ds + bh * ds_bh + (i (i + 1) / 2 + j) * 1024,
// query row r of the block at [32 r, 32 r + 32) with key 2s + c at 16 c + s,
// which is the A operand order of the dQ product (16 contiguous floats per
// lane).
template <int HD, int BQ, bool CAUSAL, bool HAS_MASK, bool VEC, bool STORE_DS>
__global__ void __launch_bounds__(BW_THREADS, (HD <= 32 && !HAS_MASK) ? 3 : (HD <= 64 ? 2 : 1)) flash_bwd_dkdv_kernel(const BwdArgs a) {
  constexpr int NQB = BQ / 32;  // 32-query sub-blocks per tile
  constexpr int NDB = HD / 32;  // 32-wide head-dim blocks of dK^T / dV^T
  constexpr int NKG = HD / 8;   // 8-dim groups of the Q.K and dO.V products
  __shared__ __attribute__((aligned(16))) float Qs[2][BQ][HD + 4];
  __shared__ __attribute__((aligned(16))) float Gs[2][BQ][HD + 4];  // dO
  __shared__ __attribute__((aligned(16))) float Ls[2][BQ];          // lse
  __shared__ __attribute__((aligned(16))) float Ds[2][BQ];          // D

  const int n_bh = a.batch * a.heads;
  const int bh = blockIdx.x % n_bh, kt = blockIdx.x / n_bh;
  const int b = bh / a.heads, h = bh % a.heads;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31, hf = lane >> 5;
  const int k0 = kt * BW_TILE;
  const int kw0 = k0 + wave * 32;  // first key of this wave
  const int key = kw0 + li;        // this lane's key
  const int col0 = h * (VEC ? HD : a.hd);

  // B operands of S = Q K^T and dP = dO V^T: register 4u + r holds
  // K[key][8u + 4*hf + r] (and likewise V), fixed for the whole loop.
  float kreg[HD / 2], vreg[HD / 2];
  {
    const int kr = min(key, a.lk - 1);
    const float *krow = a.k + ((size_t)b * a.lk + kr) * a.ldk + col0;
    const float *vrow = a.v + ((size_t)b * a.lk + kr) * a.ldv + col0;
#pragma unroll
    for (int u = 0; u < NKG; ++u) {
      const int d = 8 * u + 4 * hf;
      if constexpr (VEC) {
        const vf4 x = *reinterpret_cast<const vf4 *>(krow + d);
        const vf4 y = *reinterpret_cast<const vf4 *>(vrow + d);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kreg[4 * u + r] = x[r];
          vreg[4 * u + r] = y[r];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          kreg[4 * u + r] = d + r < a.hd ? krow[d + r] : 0.f;
          vreg[4 * u + r] = d + r < a.hd ? vrow[d + r] : 0.f;
        }
      }
    }
  }

  const int q_begin = CAUSAL ? k0 : 0;  // queries before k0 see none of these keys
  const int n_it = q_begin < a.lq ? (a.lq - q_begin + BQ - 1) / BQ : 0;
  const float *__restrict__ qbase = a.q + (size_t)b * a.lq * a.ldq + col0;
  const float *__restrict__ gbase = a.dout + (size_t)b * a.lq * a.lddo + col0;
  const float *__restrict__ lse = a.lse + (size_t)bh * a.lq;
  const float *__restrict__ dlt = a.delta + (size_t)bh * a.lq;

  floatx16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[db][r] = dv[db][r] = 0.f;
  const floatx16 zero = {};

  RowStage<HD, BQ, VEC> sq, sg;
  sq.init(a.ldq);
  sg.init(a.lddo);
  float lreg = 0.f, dreg = 0.f;
  // The stored dS blocks of this (sequence, head) as a buffer resource (the
  // launch keeps ds_bh * 4 bytes within 2^31), and the byte offset of this
  // lane's entries in a block (row 4 hf + acc_row(r), key li).
  const __amdgpu_buffer_rsrc_t ds_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      STORE_DS ? a.ds + (size_t)bh * a.ds_bh : nullptr, (short)0, STORE_DS ? (int)(a.ds_bh * 4) : 0, kBufferWord3);
  const int ds_lane = 4 * (4 * hf * 32 + (li & 1) * 16 + (li >> 1));
  if (n_it > 0) {
    sq.load(qbase, a.ldq, q_begin, a.lq, a.hd);
    sg.load(gbase, a.lddo, q_begin, a.lq, a.hd);
    if (t < BQ) {
      const int qq = min(q_begin + t, a.lq - 1);
      lreg = lse[qq];
      dreg = dlt[qq];
    }
    sq.store(Qs[0]);
    sg.store(Gs[0]);
    if (t < BQ) {
      Ls[0][t] = lreg;
      Ds[0][t] = dreg;
    }
  }
  __syncthreads();

  for (int it = 0; it < n_it; ++it) {
    const int cur = it & 1;
    const int qt0 = q_begin + it * BQ;
    // Next tile into registers; the last iteration re-stages its own tile
    // into the idle buffer (an unconditional stage keeps the registers out
    // of scratch memory).
    const int nxt = it + 1 < n_it ? qt0 + BQ : qt0;
    sq.load(qbase, a.ldq, nxt, a.lq, a.hd);
    sg.load(gbase, a.lddo, nxt, a.lq, a.hd);
    if (t < BQ) {
      const int qq = min(nxt + t, a.lq - 1);
      lreg = lse[qq];
      dreg = dlt[qq];
    }

#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      const int qb0 = qt0 + qb * 32;
      // Sub-blocks past the sequence end or wholly before this wave's keys
      // contribute nothing, and neither does a wave whose keys all lie past lk.
      if (qb0 >= a.lq || kw0 >= a.lk || (CAUSAL && qb0 + 31 < kw0)) continue;
      const float(*qrow)[HD + 4] = &Qs[cur][qb * 32];
      const float(*grow)[HD + 4] = &Gs[cur][qb * 32];

      // S = Q K^T and dP = dO V^T (two independent MFMA chains).
      floatx16 s, dp;
      vf4 qa = *reinterpret_cast<const vf4 *>(&qrow[li][4 * hf]);
      vf4 ga = *reinterpret_cast<const vf4 *>(&grow[li][4 * hf]);
#pragma unroll
      for (int u = 0; u < NKG; ++u) {
        vf4 qn, gn;
        if (u + 1 < NKG) {
          qn = *reinterpret_cast<const vf4 *>(&qrow[li][8 * (u + 1) + 4 * hf]);
          gn = *reinterpret_cast<const vf4 *>(&grow[li][8 * (u + 1) + 4 * hf]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s = mfma32x32x2(qa[r], kreg[4 * u + r], (u == 0 && r == 0) ? zero : s);
          dp = mfma32x32x2(ga[r], vreg[4 * u + r], (u == 0 && r == 0) ? zero : dp);
        }
        if (u + 1 < NKG) {
          qa = qn;
          ga = gn;
        }
      }

      // P = exp2(S * scale * log2 e - lse) and dS = P (dP - D), per query row
      // 8g + 4*hf + c of the sub-block (registers 4g + c).
      // (the masked and the unmasked forms are separate branches: a select
      // per element would run the mask arithmetic on every sub-block)
      const bool need = HAS_MASK || (CAUSAL && qb0 < kw0 + 31) || qb0 + 31 >= a.lq;
      if (need) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const vf4 l4 = *reinterpret_cast<const vf4 *>(&Ls[cur][qb * 32 + 8 * g + 4 * hf]);
          const vf4 d4 = *reinterpret_cast<const vf4 *>(&Ds[cur][qb * 32 + 8 * g + 4 * hf]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int r = 4 * g + c;
            const int qq = qb0 + 8 * g + 4 * hf + c;
            bool ok = qq < a.lq;
            if (CAUSAL) ok = ok && key <= qq;
            if (HAS_MASK) ok = ok && key < a.lk && a.mask[(size_t)min(qq, a.lq - 1) * a.lk + min(key, a.lk - 1)];
            const float p = ok ? fast_exp2(fmaf(s[r], a.scale_log2, -l4[c])) : 0.f;
            s[r] = p;
            dp[r] = p * (dp[r] - d4[c]);
          }
        }
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const vf4 l4 = *reinterpret_cast<const vf4 *>(&Ls[cur][qb * 32 + 8 * g + 4 * hf]);
          const vf4 d4 = *reinterpret_cast<const vf4 *>(&Ds[cur][qb * 32 + 8 * g + 4 * hf]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int r = 4 * g + c;
            const float p = fast_exp2(fmaf(s[r], a.scale_log2, -l4[c]));
            s[r] = p;
            dp[r] = p * (dp[r] - d4[c]);
          }
        }
      }
      if constexpr (STORE_DS) {
        // buffer stores: the block's byte offset in a scalar register, this
        // lane's fixed offset plus the row's immediate (one VGPR of address).
        // Non-temporal (the nt bit): the blocks stream to HBM rather than
        // sitting dirty in the caches, where the dQ pass's reads would evict
        // and write them back under its own traffic (c5 attention backward
        // 1170 -> 1146 us, c3 2902 -> 2841 us; non-temporal loads in the dQ
        // pass were slower).
        const int qi = qb0 >> 5, kj = kw0 >> 5;
        const int boff = (qi * (qi + 1) / 2 + kj) * 4096;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dp[r]), ds_rsrc, ds_lane + 128 * acc_row(r), boff,
                                                kCachePolicyNT);
      }

      // dV^T += dO^T P and dK^T += Q^T dS: MFMA step st pairs query rows
      // acc_row(st) (half 0) and acc_row(st) + 4 (half 1), the rows held by
      // register st of P and dS.
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int qr = acc_row(st) + 4 * hf;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          dv[db] = mfma32x32x2(grow[qr][db * 32 + li], s[st], dv[db]);
          dk[db] = mfma32x32x2(qrow[qr][db * 32 + li], dp[st], dk[db]);
        }
      }
    }

    sq.store(Qs[cur ^ 1]);
    sg.store(Gs[cur ^ 1]);
    if (t < BQ) {
      Ls[cur ^ 1][t] = lreg;
      Ds[cur ^ 1][t] = dreg;
    }
    __syncthreads();
  }

  // Lane li holds key `key`: register 4g + c of block db is dimension
  // db*32 + 8g + 4*hf + c.
  if (key < a.lk) {
    float *dkrow = a.dk + ((size_t)b * a.lk + key) * a.lddk + col0;
    float *dvrow = a.dv + ((size_t)b * a.lk + key) * a.lddv + col0;
    // (cos, sin) of this key's pairs, loaded before any store (a load issued
    // after a store waits for it)
    float2 cs[NDB][4][2];
    if (a.rope_cs) {
      const float2 *t = a.rope_cs + (size_t)key * (a.hd >> 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int d = db * 32 + 8 * g + 4 * hf + 2 * j;
            cs[db][g][j] = d < a.hd ? t[d >> 1] : make_float2(1.f, 0.f);
          }
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        vf4 x, y;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          x[c] = dk[db][4 * g + c] * a.scale;
          y[c] = dv[db][4 * g + c];
        }
        if (a.rope_cs) {  // dims d + c and d + c + 1 are one pair, in this lane
#pragma unroll
          for (int c = 0; c < 4; c += 2) {
            const float2 r = rope_inverse_pair(x[c], x[c + 1], cs[db][g][c >> 1]);
            x[c] = r.x;
            x[c + 1] = r.y;
          }
        }
        if constexpr (VEC) {
          *reinterpret_cast<vf4 *>(dkrow + d) = x;
          *reinterpret_cast<vf4 *>(dvrow + d) = y;
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (d + c < a.hd) {
              dkrow[d + c] = x[c];
              dvrow[d + c] = y[c];
            }
        }
      }
    }
  }
}

// dQ.  Query-tile major with the heaviest causal tiles first, as the forward.
template <int HD, int BN, bool CAUSAL, bool HAS_MASK, bool VEC>
__global__ void __launch_bounds__(BW_THREADS, 2) flash_bwd_dq_kernel(const BwdArgs a) {
  constexpr int NKB = BN / 32;
  constexpr int NDB = HD / 32;
  constexpr int NKG = HD / 8;
  __shared__ __attribute__((aligned(16))) float Ks[2][BN][HD + 4];
  __shared__ __attribute__((aligned(16))) float Vs[2][BN][HD + 4];

  const int n_bh = a.batch * a.heads;
  const int bh = blockIdx.x % n_bh;
  int qt = blockIdx.x / n_bh;
  if (CAUSAL) qt = a.n_tiles - 1 - qt;
  const int b = bh / a.heads, h = bh % a.heads;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31, hf = lane >> 5;
  const int q0 = qt * BW_TILE;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 + li;
  const int qc = min(qi, a.lq - 1);
  const int col0 = h * (VEC ? HD : a.hd);

  // B operands of S^T = K Q^T and dP^T = V dO^T: register 4u + r holds
  // Q[qi][8u + 4*hf + r] (and likewise dO).
  float qreg[HD / 2], greg[HD / 2];
  {
    const float *qrow = a.q + ((size_t)b * a.lq + qc) * a.ldq + col0;
    const float *grow = a.dout + ((size_t)b * a.lq + qc) * a.lddo + col0;
#pragma unroll
    for (int u = 0; u < NKG; ++u) {
      const int d = 8 * u + 4 * hf;
      if constexpr (VEC) {
        const vf4 x = *reinterpret_cast<const vf4 *>(qrow + d);
        const vf4 y = *reinterpret_cast<const vf4 *>(grow + d);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          qreg[4 * u + r] = x[r];
          greg[4 * u + r] = y[r];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          qreg[4 * u + r] = d + r < a.hd ? qrow[d + r] : 0.f;
          greg[4 * u + r] = d + r < a.hd ? grow[d + r] : 0.f;
        }
      }
    }
  }
  const float lse_q = a.lse[(size_t)bh * a.lq + qc];
  const float d_q = a.delta[(size_t)bh * a.lq + qc];
  const int key_last = CAUSAL ? min(qi, a.lk - 1) : a.lk - 1;
  const uint8_t *mrow = HAS_MASK ? a.mask + (size_t)qc * a.lk : nullptr;

  const int kend = CAUSAL ? min(q0 + BW_TILE, a.lk) : a.lk;
  const int n_kt = (kend + BN - 1) / BN;
  const float *__restrict__ kbase = a.k + (size_t)b * a.lk * a.ldk + col0;
  const float *__restrict__ vbase = a.v + (size_t)b * a.lk * a.ldv + col0;

  floatx16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;
  const floatx16 zero = {};

  RowStage<HD, BN, VEC> sk, sv;
  sk.init(a.ldk);
  sv.init(a.ldv);
  sk.load(kbase, a.ldk, 0, a.lk, a.hd);
  sv.load(vbase, a.ldv, 0, a.lk, a.hd);
  sk.store(Ks[0]);
  sv.store(Vs[0]);
  __syncthreads();

  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    const int k0 = kt * BN;
    const int nxt = kt + 1 < n_kt ? k0 + BN : k0;
    sk.load(kbase, a.ldk, nxt, a.lk, a.hd);
    sv.load(vbase, a.ldv, nxt, a.lk, a.hd);

#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int kb0 = k0 + kb * 32;
      if (kb0 >= a.lk || qw0 >= a.lq || (CAUSAL && kb0 > qw0 + 31)) continue;  // nothing to add
      const float(*krow)[HD + 4] = &Ks[cur][kb * 32];
      const float(*vrow)[HD + 4] = &Vs[cur][kb * 32];

      // S^T = K Q^T and dP^T = V dO^T
      floatx16 s, dp;
      vf4 ka = *reinterpret_cast<const vf4 *>(&krow[li][4 * hf]);
      vf4 va = *reinterpret_cast<const vf4 *>(&vrow[li][4 * hf]);
#pragma unroll
      for (int u = 0; u < NKG; ++u) {
        vf4 kn, vn;
        if (u + 1 < NKG) {
          kn = *reinterpret_cast<const vf4 *>(&krow[li][8 * (u + 1) + 4 * hf]);
          vn = *reinterpret_cast<const vf4 *>(&vrow[li][8 * (u + 1) + 4 * hf]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s = mfma32x32x2(ka[r], qreg[4 * u + r], (u == 0 && r == 0) ? zero : s);
          dp = mfma32x32x2(va[r], greg[4 * u + r], (u == 0 && r == 0) ? zero : dp);
        }
        if (u + 1 < NKG) {
          ka = kn;
          va = vn;
        }
      }

      // dS^T = P^T (dP^T - D); register r holds key kb0 + acc_row(r) + 4*hf.
      const bool need = HAS_MASK || kb0 + 31 > (CAUSAL ? min(qw0, a.lk - 1) : a.lk - 1);
      const int thr = key_last - kb0 - 4 * hf;
      if (need) {  // separate branches, as in the dK/dV kernel
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          bool ok = acc_row(r) <= thr;
          if (HAS_MASK) ok = ok && mrow[min(kb0 + acc_row(r) + 4 * hf, a.lk - 1)] != 0;
          const float p = ok ? fast_exp2(fmaf(s[r], a.scale_log2, -lse_q)) : 0.f;
          dp[r] = p * (dp[r] - d_q);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(fmaf(s[r], a.scale_log2, -lse_q));
          dp[r] = p * (dp[r] - d_q);
        }
      }

      // dQ^T += K^T dS^T
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int kr = acc_row(st) + 4 * hf;
#pragma unroll
        for (int db = 0; db < NDB; ++db) dq[db] = mfma32x32x2(krow[kr][db * 32 + li], dp[st], dq[db]);
      }
    }

    sk.store(Ks[cur ^ 1]);
    sv.store(Vs[cur ^ 1]);
    __syncthreads();
  }

  if (qi < a.lq) {
    float *dqrow = a.dq + ((size_t)b * a.lq + qi) * a.lddq + col0;
    float2 cs[NDB][4][2];  // (cos, sin) of this row's pairs, loaded before any store
    if (a.rope_cs) {
      const float2 *t = a.rope_cs + (size_t)qi * (a.hd >> 1);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int d = db * 32 + 8 * g + 4 * hf + 2 * j;
            cs[db][g][j] = d < a.hd ? t[d >> 1] : make_float2(1.f, 0.f);
          }
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hf;
        vf4 x;
#pragma unroll
        for (int c = 0; c < 4; ++c) x[c] = dq[db][4 * g + c] * a.scale;
        if (a.rope_cs) {
#pragma unroll
          for (int c = 0; c < 4; c += 2) {
            const float2 r = rope_inverse_pair(x[c], x[c + 1], cs[db][g][c >> 1]);
            x[c] = r.x;
            x[c + 1] = r.y;
          }
        }
        if constexpr (VEC) {
          *reinterpret_cast<vf4 *>(dqrow + d) = x;
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (d + c < a.hd) dqrow[d + c] = x[c];
        }
      }
    }
  }
}

// dQ from the dS blocks that flash_bwd_dkdv_kernel stored (causal, lq == lk,
// 16-byte aligned rows): dQ = scale dS K, one product instead of recomputing
// S and dP.  Query-tile major with the heaviest tiles first, as the forward.
// Wave w owns query block i = q0 / 32 + w; for its key blocks j <= i the A
// operand (dS[q][2s + c] in lane (q, c) for step s) is 16 contiguous floats
// per lane, loaded two blocks ahead, and K streams through double-buffered LDS
// as the B operand.  Lane d of the accumulator holds dQ[q][d] for the 16
// query rows acc_row(r) + 4 c.
template <int HD, int BN>
__global__ void __launch_bounds__(BW_THREADS, 2) flash_bwd_dq_ds_kernel(const BwdArgs a) {
  constexpr int NKB = BN / 32;
  constexpr int NDB = HD / 32;
  __shared__ __attribute__((aligned(16))) float Ks[2][BN][HD + 4];

  const int n_bh = a.batch * a.heads;
  const int bh = blockIdx.x % n_bh;
  const int qt = a.n_tiles - 1 - (int)(blockIdx.x / n_bh);
  const int b = bh / a.heads, h = bh % a.heads;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31, hf = lane >> 5;
  const int q0 = qt * BW_TILE;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 >> 5;                    // this wave's query block
  const int last = qw0 < a.lq ? qi : -1;      // its last key block (none past the end)
  const int col0 = h * HD;
  const float *__restrict__ kbase = a.k + (size_t)b * a.lk * a.ldk + col0;
  const float *__restrict__ dsw = a.ds + (size_t)bh * a.ds_bh + (size_t)qi * (qi + 1) / 2 * 1024 + li * 32 + hf * 16;

  floatx16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;

  const int kend = min(q0 + BW_TILE, a.lk);
  const int n_kt = (kend + BN - 1) / BN;
  RowStage<HD, BN, true> sk;
  sk.init(a.ldk);
  sk.load(kbase, a.ldk, 0, a.lk, HD);
  sk.store(Ks[0]);
  // dS operands two blocks ahead: cur (block j), n1 (j + 1), n2 (j + 2)
  vf4 cur[4], n1[4], n2[4];
  if (last >= 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = *reinterpret_cast<const vf4 *>(dsw + 4 * i);
  }
  if (last >= 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) n1[i] = *reinterpret_cast<const vf4 *>(dsw + 1024 + 4 * i);
  }
  __syncthreads();

  for (int kt = 0; kt < n_kt; ++kt) {
    const int lbuf = kt & 1;
    const int k0 = kt * BN;
    sk.load(kbase, a.ldk, kt + 1 < n_kt ? k0 + BN : k0, a.lk, HD);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int j = kt * NKB + kb;  // key block
      if (j > last) continue;
      if (j + 2 <= last) {
#pragma unroll
        for (int i = 0; i < 4; ++i) n2[i] = *reinterpret_cast<const vf4 *>(dsw + (size_t)(j + 2) * 1024 + 4 * i);
      }
      const float(*krow)[HD + 4] = &Ks[lbuf][kb * 32];
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float av = cur[st >> 2][st & 3];
#pragma unroll
        for (int db = 0; db < NDB; ++db) dq[db] = mfma32x32x2(av, krow[2 * st + hf][db * 32 + li], dq[db]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cur[i] = n1[i];
        n1[i] = n2[i];
      }
    }
    sk.store(Ks[lbuf ^ 1]);
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int q = qw0 + acc_row(r) + 4 * hf;
    if (q < a.lq) {
      float *dqrow = a.dq + ((size_t)b * a.lq + q) * a.lddq + col0;
#pragma unroll
      for (int db = 0; db < NDB; ++db) dqrow[db * 32 + li] = dq[db][r] * a.scale;
    }
  }
}

// dQ from the stored dS blocks for short sequences (lq <= 32 * MAXQB): one
// workgroup per (sequence, head) stages the head's whole K in LDS once; wave
// w owns query blocks w and nqb - 1 - w, so every wave has nqb + 1 key
// blocks of work (the middle block of an odd count alone) and no barrier
// follows the staging.  Operand order and the per-block product are those
// of flash_bwd_dq_ds_kernel, with the dS operands four blocks ahead (a block
// is about a thousand MFMA cycles at head dim 32, short of the load latency).
template <int HD, int MAXQB>
__global__ void __launch_bounds__(64 * (MAXQB / 2)) flash_bwd_dq_ds_short_kernel(const BwdArgs a) {
  constexpr int NDB = HD / 32;
  __shared__ __attribute__((aligned(16))) float Ks[32 * MAXQB][HD + 4];
  const int bh = blockIdx.x;
  const int b = bh / a.heads, h = bh % a.heads;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int li = lane & 31, hf = lane >> 5;
  const int nqb = (a.lq + 31) >> 5;
  const int col0 = h * HD;
  // K rows [0, 32 nqb) of the head, rows past lk clamped (their dS is 0)
  {
    const float *kbase = a.k + (size_t)b * a.lk * a.ldk + col0;
    constexpr int F4 = HD / 4;
    for (int e = t; e < 32 * nqb * F4; e += blockDim.x) {
      const int r = e / F4, c = (e % F4) * 4;
      *reinterpret_cast<vf4 *>(&Ks[r][c]) =
          *reinterpret_cast<const vf4 *>(kbase + (size_t)min(r, a.lk - 1) * a.ldk + c);
    }
  }
  __syncthreads();
  const float *__restrict__ dsbh = a.ds + (size_t)bh * a.ds_bh + li * 32 + hf * 16;
  for (int pass = 0; pass < 2; ++pass) {
    const int qi = pass == 0 ? nqb - 1 - wave : wave;
    if (pass == 1 && qi >= nqb - 1 - wave) break;  // the middle block ran in pass 0
    const float *dsw = dsbh + (size_t)qi * (qi + 1) / 2 * 1024;
    floatx16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) dq[db][r] = 0.f;
    // dS operands PF blocks ahead in a ring: block j lives in buf[j % PF]
    // (the loop is unrolled by PF, so every index is a constant and no
    // in-flight load is ever copied), and the load of block j + PF goes into
    // the buffer block j has just left.
    constexpr int PF = 4;
    vf4 buf[PF][4];
#pragma unroll
    for (int p = 0; p < PF; ++p)
      if (p <= qi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) buf[p][i] = *reinterpret_cast<const vf4 *>(dsw + (size_t)p * 1024 + 4 * i);
      }
    for (int j0 = 0; j0 <= qi; j0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int j = j0 + u;
        if (j > qi) break;
        const float(*krow)[HD + 4] = &Ks[j * 32];
#pragma unroll
        for (int st = 0; st < 16; ++st) {
          const float av = buf[u][st >> 2][st & 3];
#pragma unroll
          for (int db = 0; db < NDB; ++db) dq[db] = mfma32x32x2(av, krow[2 * st + hf][db * 32 + li], dq[db]);
        }
        if (j + PF <= qi) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            buf[u][i] = *reinterpret_cast<const vf4 *>(dsw + (size_t)(j + PF) * 1024 + 4 * i);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = qi * 32 + acc_row(r) + 4 * hf;
      if (q < a.lq) {
        float *dqrow = a.dq + ((size_t)b * a.lq + q) * a.lddq + col0;
#pragma unroll
        for (int db = 0; db < NDB; ++db) dqrow[db * 32 + li] = dq[db][r] * a.scale;
      }
    }
  }
}

// Any head dim, any strides: one workgroup per (sequence, head) walks the
// queries in order, as AccelerationCPU.cs:1092-1268 does per head, with the
// keys spread over the threads.  scratch holds two floats per key.
__global__ void __launch_bounds__(256) flash_bwd_generic_kernel(const BwdArgs a, float *scratch,
                                                                 int causal) {
  extern __shared__ float sm[];  // q_i[hd] | dout_i[hd] | red[8]
  float *qv = sm, *gv = sm + a.hd, *red = sm + 2 * a.hd;
  const int bh = blockIdx.x;
  const int b = bh / a.heads, h = bh % a.heads;
  const int t = threadIdx.x, hd = a.hd, col0 = h * hd;
  float *w = scratch + (size_t)bh * 2 * a.lk;
  float *da = w + a.lk;
  const float *K = a.k + (size_t)b * a.lk * a.ldk + col0;
  const float *V = a.v + (size_t)b * a.lk * a.ldv + col0;
  float *dK = a.dk + (size_t)b * a.lk * a.lddk + col0;
  float *dV = a.dv + (size_t)b * a.lk * a.lddv + col0;
  for (int j = t; j < a.lk; j += 256)
    for (int d = 0; d < hd; ++d) dK[(size_t)j * a.lddk + d] = dV[(size_t)j * a.lddv + d] = 0.f;

  auto block_max = [&](float x) {
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = x;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  };
  auto block_sum = [&](float x) {
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    __syncthreads();
    if ((t & 63) == 0) red[t >> 6] = x;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
  };

  for (int i = 0; i < a.lq; ++i) {
    const float *qrow = a.q + ((size_t)b * a.lq + i) * a.ldq + col0;
    const float *grow = a.dout + ((size_t)b * a.lq + i) * a.lddo + col0;
    float *dqrow = a.dq + ((size_t)b * a.lq + i) * a.lddq + col0;
    __syncthreads();
    for (int d = t; d < hd; d += 256) {
      qv[d] = qrow[d];
      gv[d] = grow[d];
    }
    __syncthreads();
    const int visible = causal ? min(i + 1, a.lk) : a.lk;
    float mx = -INFINITY;
    for (int j = t; j < visible; j += 256) {
      float s = -INFINITY;
      if (!a.mask || a.mask[(size_t)i * a.lk + j]) {
        float acc = 0.f;
        for (int d = 0; d < hd; ++d) acc += qv[d] * K[(size_t)j * a.ldk + d];
        s = acc * a.scale;
      }
      w[j] = s;
      mx = fmaxf(mx, s);
    }
    mx = block_max(mx);
    float sum = 0.f;
    if (mx != -INFINITY) {
      for (int j = t; j < visible; j += 256) {
        const float e = w[j] == -INFINITY ? 0.f : expf(w[j] - mx);
        w[j] = e;
        sum += e;
      }
    }
    sum = block_sum(sum);
    if (!(mx != -INFINITY && sum > 0.f)) {  // the row contributes nothing
      for (int d = t; d < hd; d += 256) dqrow[d] = 0.f;
      continue;
    }
    const float inv = 1.0f / sum;
    float rd = 0.f;
    for (int j = t; j < visible; j += 256) {
      const float wj = w[j] * inv;
      float g = 0.f;
      for (int d = 0; d < hd; ++d) g += gv[d] * V[(size_t)j * a.ldv + d];
      w[j] = wj;
      da[j] = g;
      rd += wj * g;
    }
    rd = block_sum(rd);
    for (int j = t; j < visible; j += 256) {
      const float wj = w[j];
      const float dd = wj * (da[j] - rd) * a.scale;
      for (int d = 0; d < hd; ++d) {
        dV[(size_t)j * a.lddv + d] += wj * gv[d];
        if (dd != 0.f) dK[(size_t)j * a.lddk + d] += dd * qv[d];
      }
      da[j] = dd;
    }
    __syncthreads();
    for (int d = t; d < hd; d += 256) {
      float acc = 0.f;
      for (int j = 0; j < visible; ++j) acc += da[j] * K[(size_t)j * a.ldk + d];
      dqrow[d] = acc;
    }
  }
}

// rows x cols block (row stride ld) set to zero.
__global__ void __launch_bounds__(256) zero_rows_kernel(float *p, long long rows, int cols, int ld) {
  const long long n = rows * cols;
  for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long long)gridDim.x * 256)
    p[(e / cols) * ld + e % cols] = 0.f;
}

int zero_rows(float *p, long long rows, int cols, int ld, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return CDML_OK;
  const long long n = rows * cols;
  zero_rows_kernel<<<dim3((unsigned)std::min<long long>((n + 255) / 256, 16384)), dim3(256), 0, st>>>(
      p, rows, cols, ld);
  return check_launch("zero_rows_kernel");
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Returns whether dQ left rotated (a.rope_cs set and a dQ kernel that
// applies it: the stored-dS dQ kernels do not, their 16 rows per lane would
// cost the table registers they need for their occupancy).
template <int HD, int BQ, int BN, bool CAUSAL, bool HAS_MASK, bool VEC>
bool launch_bwd(BwdArgs &a, hipStream_t st) {
  const int n_bh = a.batch * a.heads;
  const int kt = (a.lk + BW_TILE - 1) / BW_TILE;
  a.n_tiles = (a.lq + BW_TILE - 1) / BW_TILE;
  if constexpr (CAUSAL && !HAS_MASK && VEC && HD <= 64) {
    if (a.ds) {  // dQ from the stored dS blocks
      flash_bwd_dkdv_kernel<HD, BQ, true, false, true, true><<<dim3(n_bh * kt), dim3(BW_THREADS), 0, st>>>(a);
      constexpr int kShortQB = HD <= 32 ? 16 : 8;  // the whole K of a head in LDS: 72 KB at most
      const int nqb = (a.lq + 31) / 32;
      if (nqb <= kShortQB)
        flash_bwd_dq_ds_short_kernel<HD, kShortQB><<<dim3(n_bh), dim3(64 * ((nqb + 1) / 2)), 0, st>>>(a);
      else
        flash_bwd_dq_ds_kernel<HD, 64><<<dim3(n_bh * a.n_tiles), dim3(BW_THREADS), 0, st>>>(a);
      return false;
    }
  }
  flash_bwd_dkdv_kernel<HD, BQ, CAUSAL, HAS_MASK, VEC, false><<<dim3(n_bh * kt), dim3(BW_THREADS), 0, st>>>(a);
  flash_bwd_dq_kernel<HD, BN, CAUSAL, HAS_MASK, VEC><<<dim3(n_bh * a.n_tiles), dim3(BW_THREADS), 0, st>>>(a);
  return a.rope_cs != nullptr;
}

template <int HD, int BQ, int BN, bool VEC>
bool launch_bwd_mode(BwdArgs &a, bool causal, hipStream_t st) {
  if (causal) {
    if (a.mask) return launch_bwd<HD, BQ, BN, true, true, VEC>(a, st);
    return launch_bwd<HD, BQ, BN, true, false, VEC>(a, st);
  }
  if (a.mask) return launch_bwd<HD, BQ, BN, false, true, VEC>(a, st);
  return launch_bwd<HD, BQ, BN, false, false, VEC>(a, st);
}

template <int HD, int BQ, int BN>
bool launch_bwd_hd(BwdArgs &a, bool causal, bool vec, hipStream_t st) {
  return vec ? launch_bwd_mode<HD, BQ, BN, true>(a, causal, st) : launch_bwd_mode<HD, BQ, BN, false>(a, causal, st);
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_sdpa_bwd_workspace_size(int batch, int lq, int lk, int dim, int num_heads,
                                            size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_sdpa_bwd_workspace_size: bytes is NULL");
  if (batch < 0 || lq < 0 || lk < 0 || dim <= 0 || num_heads <= 0 || dim % num_heads)
    return fail(CDML_E_INVALID, "cdml_sdpa_bwd_workspace_size: bad size");
  const size_t f = sizeof(float), bh = (size_t)batch * num_heads;
  // O | lse | D | two floats per key for the generic kernel
  *bytes = align256(f * (size_t)batch * lq * dim) + 2 * align256(f * bh * lq) + align256(f * 2 * bh * lk);
  return CDML_OK;
}

namespace cdml {
namespace {

// Bytes of the stored-dS workspace of cdml_sdpa_bwd_saved (after D), or 0 when
// the shape does not take that path: causal, lq == lk, head dim 32 or 64.
size_t ds_bytes(int batch, int lq, int lk, int dim, int num_heads, bool causal) {
  const int hd = dim / num_heads;
  if (!causal || lq != lk || (hd != 32 && hd != 64) || lq == 0) return 0;
  const size_t nb = ((size_t)lq + 31) / 32;
  return (size_t)batch * num_heads * (nb * (nb + 1) / 2) * 1024 * sizeof(float);
}

}  // namespace
}  // namespace cdml

extern "C" int cdml_sdpa_bwd_stored_ds_workspace_size(int batch, int lq, int lk, int dim, int num_heads,
                                                      int causal, size_t *bytes) {
  int rc = cdml_sdpa_bwd_workspace_size(batch, lq, lk, dim, num_heads, bytes);
  if (rc) return rc;
  *bytes = align256(*bytes) + ds_bytes(batch, lq, lk, dim, num_heads, causal != 0);
  return CDML_OK;
}

extern "C" int cdml_sdpa_bwd_saved_workspace_size(int batch, int lq, int lk, int dim, int num_heads,
                                                  int causal, size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_sdpa_bwd_saved_workspace_size: bytes is NULL");
  if (batch < 0 || lq < 0 || lk < 0 || dim <= 0 || num_heads <= 0 || dim % num_heads)
    return fail(CDML_E_INVALID, "cdml_sdpa_bwd_saved_workspace_size: bad size");
  const size_t d = sizeof(float) * (size_t)batch * num_heads * lq;
  const size_t extra = ds_bytes(batch, lq, lk, dim, num_heads, causal != 0);
  *bytes = extra ? align256(d) + extra : d;
  return CDML_OK;
}

namespace cdml {
namespace {

// cdml_sdpa_bwd, and with o_saved / lse_saved the backward from the forward's
// saved output and row statistics (cdml_sdpa_bwd_saved): no forward pass.
int sdpa_bwd_impl(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                  const float *o_saved, int ldo_saved, const float *lse_saved, const float *dout,
                  int lddo, float *dq, int lddq, float *dk, int lddk, float *dv, int lddv, int batch,
                  int lq, int lk, int dim, int num_heads, float scale, int causal,
                  const uint8_t *mask, void *workspace, size_t workspace_bytes, cdml_stream stream,
                  const char *what, const float *rope_cs = nullptr, int rope_npos = 0) {
  const bool saved = o_saved != nullptr;
  size_t need = 0;
  int rc = cdml_sdpa_bwd_workspace_size(batch, lq, lk, dim, num_heads, &need);
  if (rc) return rc;
  if (saved) {
    need = sizeof(float) * (size_t)batch * num_heads * lq;
    if (!lse_saved || ldo_saved < dim)
      return fail(CDML_E_INVALID, "%s: saved output needs the row statistics and a row stride of at "
                  "least dim", what);
  }
  if (ldq < dim || ldk < dim || ldv < dim || lddo < dim || lddq < dim || lddk < dim || lddv < dim)
    return fail(CDML_E_INVALID, "%s: row stride smaller than dim", what);
  if ((long long)ldq * 128 > INT32_MAX || (long long)ldk * 128 > INT32_MAX ||
      (long long)ldv * 128 > INT32_MAX || (long long)lddo * 128 > INT32_MAX)
    return fail(CDML_E_INVALID, "%s: row stride above %d elements", what, INT32_MAX / 128);
  if (batch == 0 || (lq == 0 && lk == 0)) return CDML_OK;
  if ((lq && (!dq || !q || !dout)) || (lk && (!dk || !dv || !k || !v)))
    return fail(CDML_E_INVALID, "%s: NULL pointer", what);
  rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  if (lq == 0 || lk == 0) {  // nothing attends: every gradient is 0
    rc = zero_rows(dq, (long long)batch * lq, dim, lddq, st);
    if (!rc) rc = zero_rows(dk, (long long)batch * lk, dim, lddk, st);
    if (!rc) rc = zero_rows(dv, (long long)batch * lk, dim, lddv, st);
    return rc;
  }
  if (!workspace || workspace_bytes < need)
    return fail(CDML_E_INVALID, "%s: workspace of %zu bytes needed, %zu given", what, need,
                workspace_bytes);
  if ((long long)batch * num_heads * ((std::max(lq, lk) + BW_TILE - 1) / BW_TILE) > (1LL << 30))
    return fail(CDML_E_INVALID, "%s: problem too large", what);

  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.mask = mask;
  a.ldq = ldq;
  a.ldk = ldk;
  a.ldv = ldv;
  a.lddo = lddo;
  a.lddq = lddq;
  a.lddk = lddk;
  a.lddv = lddv;
  a.batch = batch;
  a.lq = lq;
  a.lk = lk;
  a.dim = dim;
  a.heads = num_heads;
  a.hd = dim / num_heads;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.rope_cs = reinterpret_cast<const float2 *>(rope_cs);
  char *ws = static_cast<char *>(workspace);
  const size_t f = sizeof(float), bh = (size_t)batch * num_heads;
  float *o = reinterpret_cast<float *>(ws);
  float *lse = reinterpret_cast<float *>(ws + align256(f * (size_t)batch * lq * dim));
  float *delta = reinterpret_cast<float *>(reinterpret_cast<char *>(lse) + align256(f * bh * lq));
  float *scratch = reinterpret_cast<float *>(reinterpret_cast<char *>(delta) + align256(f * bh * lq));
  a.o = o;
  a.ldo = dim;
  a.lse = lse;
  a.delta = delta;
  if (saved) {  // workspace holds D only
    a.o = o_saved;
    a.ldo = ldo_saved;
    a.lse = lse_saved;
    a.delta = reinterpret_cast<float *>(ws);
  }

  const int hd = a.hd;
  if (hd > 128 && saved)
    return fail(CDML_E_INVALID, "%s: saved statistics need head dim <= 128; use cdml_sdpa_bwd", what);
  if (hd > 128) {
    const size_t smem = f * (2 * (size_t)hd + 8);
    if (smem > 64 * 1024) return fail(CDML_E_INVALID, "%s: head dim %d too large", what, hd);
    flash_bwd_generic_kernel<<<dim3((unsigned)bh), dim3(256), smem, st>>>(a, scratch, causal ? 1 : 0);
    return check_launch("flash_bwd_generic_kernel");
  }
  // 1. O and the row statistics (unless the caller saved them)
  if (!saved) {
    rc = flash_forward(q, ldq, k, ldk, v, ldv, o, dim, lse, batch, lq, lk, dim, num_heads, scale,
                       causal != 0, mask, st);
    if (rc) return rc;
  }
  // 2. D = rowsum(dO * O)
  const int hd_pad = hd <= 32 ? 32 : (hd <= 64 ? 64 : 128);
  const bool vec = hd == hd_pad && ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && lddo % 4 == 0 &&
                   lddq % 4 == 0 && lddk % 4 == 0 && lddv % 4 == 0 && aligned16(q) && aligned16(k) &&
                   aligned16(v) && aligned16(dout) && aligned16(dq) && aligned16(dk) && aligned16(dv);
  if (vec && a.ldo % 4 == 0 && aligned16(a.o)) {
    const long long n = (long long)batch * lq * (dim / 4);
    const dim3 grid((unsigned)((n + 255) / 256));
    if (hd == 32) bwd_delta_kernel<32><<<grid, dim3(256), 0, st>>>(a);
    else if (hd == 64) bwd_delta_kernel<64><<<grid, dim3(256), 0, st>>>(a);
    else bwd_delta_kernel<128><<<grid, dim3(256), 0, st>>>(a);
  } else {
    const long long n = (long long)batch * lq * num_heads;
    bwd_delta_scalar_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(a);
  }
  rc = check_launch("bwd_delta_kernel");
  if (rc) return rc;
  // 3. dK, dV and 4. dQ; with room for the dS blocks after the required
  // workspace, dQ is one product over them
  if (vec && !mask) {
    const size_t extra = ds_bytes(batch, lq, lk, dim, num_heads, causal != 0);
    const size_t off = align256(need);  // the dS blocks follow the required workspace
    // (a (sequence, head)'s blocks must fit a buffer resource's 31-bit range)
    if (extra && workspace_bytes >= off + extra && extra / bh <= (size_t)INT32_MAX) {
      a.ds = reinterpret_cast<float *>(ws + off);
      a.ds_bh = (long long)(extra / sizeof(float) / bh);
    }
  }
  bool dq_rotated;
  if (hd_pad == 32) dq_rotated = launch_bwd_hd<32, 64, 64>(a, causal != 0, vec, st);
  else if (hd_pad == 64) dq_rotated = launch_bwd_hd<64, 64, 32>(a, causal != 0, vec, st);
  else dq_rotated = launch_bwd_hd<128, 32, 32>(a, causal != 0, vec, st);
  rc = check_launch("flash_bwd_dkdv_kernel / flash_bwd_dq_kernel");
  if (rc || !rope_cs || dq_rotated) return rc;
  // dK left rotated; dQ from the stored dS blocks takes the table RoPE
  return cdml_rope_qk_table(dq, nullptr, batch * lq, lddq, hd, num_heads, rope_cs, rope_npos, 0, lq, 1, stream);
}

}  // namespace
}  // namespace cdml

extern "C" int cdml_sdpa_bwd(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                             const float *dout, int lddo, float *dq, int lddq, float *dk, int lddk,
                             float *dv, int lddv, int batch, int lq, int lk, int dim, int num_heads,
                             float scale, int causal, const uint8_t *mask, void *workspace,
                             size_t workspace_bytes, cdml_stream stream) {
  return sdpa_bwd_impl(q, ldq, k, ldk, v, ldv, nullptr, 0, nullptr, dout, lddo, dq, lddq, dk, lddk, dv,
                       lddv, batch, lq, lk, dim, num_heads, scale, causal, mask, workspace,
                       workspace_bytes, stream, "cdml_sdpa_bwd");
}

extern "C" int cdml_sdpa_bwd_saved(const float *q, int ldq, const float *k, int ldk, const float *v,
                                   int ldv, const float *o, int ldo, const float *lse,
                                   const float *dout, int lddo, float *dq, int lddq, float *dk,
                                   int lddk, float *dv, int lddv, int batch, int lq, int lk, int dim,
                                   int num_heads, float scale, int causal, const uint8_t *mask,
                                   void *workspace, size_t workspace_bytes, cdml_stream stream) {
  if (!o) return fail(CDML_E_INVALID, "cdml_sdpa_bwd_saved: o is NULL");
  return sdpa_bwd_impl(q, ldq, k, ldk, v, ldv, o, ldo, lse, dout, lddo, dq, lddq, dk, lddk, dv, lddv,
                       batch, lq, lk, dim, num_heads, scale, causal, mask, workspace, workspace_bytes,
                       stream, "cdml_sdpa_bwd_saved");
}

extern "C" int cdml_sdpa_bwd_saved_rope(const float *q, int ldq, const float *k, int ldk, const float *v,
                                        int ldv, const float *o, int ldo, const float *lse,
                                        const float *dout, int lddo, float *dq, int lddq, float *dk,
                                        int lddk, float *dv, int lddv, int batch, int lq, int lk, int dim,
                                        int num_heads, float scale, int causal, const uint8_t *mask,
                                        const float *rope_cs, int n_pos, void *workspace,
                                        size_t workspace_bytes, cdml_stream stream) {
  const char *what = "cdml_sdpa_bwd_saved_rope";
  if (!o) return fail(CDML_E_INVALID, "%s: o is NULL", what);
  if (num_heads > 0 && dim > 0 && dim % num_heads == 0 && ((dim / num_heads) & 1))
    return fail(CDML_E_INVALID, "%s: RoPE requires an even head dimension", what);
  if (!rope_cs) return fail(CDML_E_INVALID, "%s: rope_cs is NULL", what);
  if (reinterpret_cast<uintptr_t>(rope_cs) % 8)
    return fail(CDML_E_INVALID, "%s: rope_cs must be 8-byte aligned", what);
  if (n_pos < std::max(lq, lk))
    return fail(CDML_E_INVALID, "%s: a %d-row table does not cover %d positions", what, n_pos, std::max(lq, lk));
  return sdpa_bwd_impl(q, ldq, k, ldk, v, ldv, o, ldo, lse, dout, lddo, dq, lddq, dk, lddk, dv, lddv,
                       batch, lq, lk, dim, num_heads, scale, causal, mask, workspace, workspace_bytes,
                       stream, what, rope_cs, n_pos);
}
