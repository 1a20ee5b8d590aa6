// fp32 MFMA GEMM for the projections of the attention path and their
// gradients:
//   C[m, n] = act(sum_k opA[m, k] * opB[k, n] + bias[n])  (+ C[m, n] when beta)
// opA is A [M, K] (row stride lda) or, transposed, A stored [K, M]; opB is the
// weight W [N, K] ([out, in], the reference's layout: y = x W^T) or, for
// gradients, B stored [K, N].  Up to three problems with the same shape run in
// one launch (the fused Q/K/V projection and its weight gradients).
//
// Forward (A [M, K], W [N, K]):                  y = x W^T    ProjectQKV, linear
// Input gradient (A = dY [M, K], B = W [K, N]):  dX = dY W    BackpropQKV, ...
// Weight gradient (A = dY stored [K, M], B = X [K, N]): dW += dY^T X, with the
//   bias gradient (row sums of opA = column sums of dY) folded into the
//   staging of opA.
//
// The MFMA inner loop is the same for every layout: both operand tiles sit in
// LDS as [rows][k] with row pitch BK + 4 floats, and every lane reads its A
// and B operands as 16-byte LDS reads that feed four v_mfma_f32_32x32x2_f32
// each.  The reduction index k is visited in the permuted order
// kappa(s, h) = 8*(s/4) + 4*h + s%4 on both operands, which leaves the sum
// unchanged.  A transposed operand is transposed on its way into LDS.
#include <algorithm>

#include "common.h"

namespace cdml {
namespace {

constexpr int BM = 128, BN = 128, BK = 32, LDSK = BK + 4;
constexpr int NTHREADS = 256;
constexpr int GROUP_M = 8;
// Epilogue selector of the tiled kernel beyond the activations: no
// activation, rotary embedding on problems 0 and 1.
constexpr int kActRope = 100;

struct GemmProblem {
  const float *a;     // opA source
  const float *w;     // opB source
  const float *bias;  // [N] or NULL
  float *c;
  float *bgrad;       // [M] += row sums of opA (transposed-A launches only), or NULL
};

struct GemmArgs {
  GemmProblem p[3];
  int lda, ldb, ldc;
  int M, N, K;
  int nprob;
  int tiles_m, tiles_n;  // tiles_n counts the tiles of one problem
  int total, padded;
  int act;
  int beta;  // 1: add the result to C
  // Split-K weight gradient with a ragged K: the tiled chunks cover rows
  // [0, ktail0) and splitk_reduce_kernel adds rows [ktail0, K) of opA^T opB
  // (and of opA's row sums) itself; 0 when K % 16 == 0.  (It fills the
  // padding before rope_cs.)
  int ktail0;
  // Rotary position embedding applied to problems 0 and 1 (Q and K) in the
  // epilogue when rope_cs is set: rope_cs[pos * rope_hd / 2 + p] holds
  // (cos, sin) of position pos for pair p; row m has position
  // rope_pos0 + (rope_seg > 0 ? m % rope_seg : m), below rope_npos.
  const float2 *rope_cs;
  int rope_hd, rope_npos, rope_pos0, rope_seg;
  // Split-K of the weight-gradient GEMMs (transposed-A launches): ksplit
  // chunks of kchunk k-tiles each; chunk c of problem p writes its partial
  // C to ws + (c * nprob + p) * M * N ([M][N], row stride N) and its partial
  // bias-gradient row sums to wsb + (c * nprob + p) * M; splitk_reduce_kernel
  // adds the chunks, in chunk order, to C and bgrad.  tiles counts the
  // output tiles of all problems (total = tiles * ksplit).
  int ksplit, kchunk, tiles;
  float *ws, *wsb;
  int small;  // split-K by wgrad_small_kernel (kchunk counts rows, not k-tiles)
  // K segments of an input-gradient launch (opB stored [K, N], one problem):
  // when kseg > 0, k-tiles [s * kseg, (s + 1) * kseg) read opA from p[s].a
  // and opB from p[s].w (s < 3), so dX = dQ WQ + dK WK + dV WV is one
  // product with K = 3 * out.  (It fills the padding before `pre`.)
  int kseg;
  // Single-problem epilogue options (store_elem): pre receives the
  // pre-activation acc + bias (forward layers whose backward needs it); dz
  // multiplies the result by act'(dz) with act = dact (the hidden deltas of
  // NeuralNetwork.ComputeInputGradientBatch); add is added last (a residual
  // gradient, MatrixAddInPlace).
  float *pre;
  const float *dz, *add;
  int ldpre, lddz, ldadd, dact;
};

// The value of lane l ^ 1 (a DPP quad permutation [1, 0, 3, 2]).
__device__ __forceinline__ float swap_pair(float y) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(y), 0xB1, 0xF, 0xF, false));
}

// Epilogue of both forward GEMM kernels with the rotary embedding of
// AccelerationCPU.cs:4947-4975 folded in.  A lane holds column n of rows
// mrow0 + 32 i + 8 (r / 4) + 4 hf + r % 4, so the pair partner of column n
// (n ^ 1; head dims are even) sits in lane li ^ 1 of the same register: one
// lane swap gives each lane both halves of its pair.  The swap runs in every
// lane; only the store is predicated.
template <int BI, int BJ>
__device__ __forceinline__ void store_rope(const GemmArgs &args, const GemmProblem &P,
                                           const floatx16 (&acc)[BI][BJ], int mrow0, int ncol0,
                                           int li, int hf) {
  // each rotation product rounded before the sum, as the reference and the
  // in-place rope kernels evaluate it: no fused multiply-add
#pragma clang fp contract(off)
  const int pairs = args.rope_hd >> 1;
  int n[BJ], pidx[BJ];
  bool odd[BJ];
  float bias[BJ];
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    n[j] = ncol0 + j * 32 + li;
    const int c = n[j] % args.rope_hd;
    pidx[j] = c >> 1;
    odd[j] = c & 1;
    bias[j] = (P.bias && n[j] < args.N) ? P.bias[n[j]] : 0.f;
  }
  // rows of block i: mb + dr(r), dr = 8 (r / 4) + 4 hf + r % 4
  auto block = [&](int i, int mb, auto position) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int dr = 8 * (r >> 2) + 4 * hf + (r & 3);
      const int m = mb + dr;
      const int pos = min(position(m, dr), args.rope_npos - 1);  // rows past M are never stored
      const float2 *cs = args.rope_cs + (size_t)pos * pairs;
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const float y = acc[i][j][r] + bias[j];
        const float yp = swap_pair(y);
        const float2 t = cs[pidx[j]];
        const float out = odd[j] ? yp * t.y + y * t.x : y * t.x - yp * t.y;
        if (m < args.M && n[j] < args.N) P.c[(size_t)m * args.ldc + n[j]] = out;
      }
    }
  };
  const int seg = args.rope_seg;
  // every row and column of this wave's blocks exists (wave-uniform)
  const bool full = mrow0 + 32 * BI <= args.M && ncol0 + 32 * BJ <= args.N;
#pragma unroll
  for (int i = 0; i < BI; ++i) {
    const int mb = mrow0 + i * 32;             // wave-uniform
    const int pb = seg > 0 ? mb % seg : mb;    // position of row mb in its segment
    if (seg <= 0 || pb + 31 < seg) {
      if (full) {
        // A whole block inside one segment: positions pos0 + pb + dr (every
        // one inside the table, which the entry point checks), no predicates,
        // and per row only wave-uniform offsets from the lane's bases.
        // The table entries of four rows are loaded before any of their
        // stores: a load issued after a store waits for it (the memory
        // counter covers both), which serialised one round trip per element.
        // (Loading a group ahead, or eight rows at once, takes the kernel past
        // 128 VGPRs and one of its two workgroups per CU.)
        const float2 *__restrict__ csb = args.rope_cs + (size_t)(args.rope_pos0 + pb + 4 * hf) * pairs;
        float *__restrict__ cb = P.c + (size_t)(mb + 4 * hf) * args.ldc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float2 t[4][BJ];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int j = 0; j < BJ; ++j) t[rr][j] = csb[(8 * g + rr) * pairs + pidx[j]];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int r = 4 * g + rr;
            float *c = cb + (size_t)(8 * g + rr) * args.ldc;
#pragma unroll
            for (int j = 0; j < BJ; ++j) {
              const float y = acc[i][j][r] + bias[j];
              const float yp = swap_pair(y);
              c[n[j]] = odd[j] ? yp * t[rr][j].y + y * t[rr][j].x : y * t[rr][j].x - yp * t[rr][j].y;
            }
          }
        }
      } else {
        block(i, mb, [&](int, int dr) { return args.rope_pos0 + pb + dr; });
      }
    } else {
      // a block across a segment boundary divides per row
      block(i, mb, [&](int m, int) { return args.rope_pos0 + m % seg; });
    }
  }
}

// The same epilogue with the (cos, sin) table staged through LDS, for full
// row tiles inside one position segment and head dims 2^(LP+1) (8 .. 64).
// The k-loop ends on a barrier, so the operand tiles in `tab` (As) are free.
// Phase i covers block i of every wave row: the workgroup copies the table
// rows of those WM x 32 output rows into tab[pair * RS + row] with coalesced
// loads (a thread keeps one pair for all its fetches, so every fetch and LDS
// write is its base plus a constant), and each lane then reads its (cos, sin)
// from LDS, which never waits on the stores (a global load issued after a
// store waits for it: one round trip per group of rows in store_rope).
// Same arithmetic, same bits as store_rope.
template <int TM, int WM, int NT, int BI, int BJ, int LP>
__device__ __forceinline__ void store_rope_lds(const GemmArgs &args, const GemmProblem &P,
                                               const floatx16 (&acc)[BI][BJ], int mseg, int wm, int mw, int nw,
                                               int li, int hf, float2 *tab) {
#pragma clang fp contract(off)
  constexpr int PAIRS = 1 << LP;
  constexpr int ROWS = WM * 32;             // table rows per phase
  constexpr int RS = ROWS + 2;              // pitch of one pair's column (float2)
  constexpr int STEP = NT / PAIRS;          // rows between a thread's fetches
  constexpr int KN = ROWS * PAIRS / NT;     // fetches per thread and phase
  constexpr int WR = TM / WM;               // tile rows per wave row
  static_assert(KN >= 1 && KN * NT == ROWS * PAIRS && (STEP % 32 == 0 || 32 % STEP == 0), "fetch shape");
  const int t = threadIdx.x;
  const int p = t & (PAIRS - 1), q0 = t >> LP;
  // table row q of a phase is tile row (q / 32) * WR + q % 32 (+ 32 i); for
  // q = q0 + k * STEP that is the lane's base row plus a constant
  const int ro0 = STEP <= 32 ? q0 : (q0 >> 5) * WR + (q0 & 31);
  const float2 *__restrict__ src = args.rope_cs + (size_t)(args.rope_pos0 + mseg + ro0) * PAIRS + p;
  float2 *wr = tab + p * RS + q0;
  float2 pre[KN];
  int n[BJ], pcol[BJ];
  float bias[BJ];
  const bool odd = li & 1;  // column parity (nw is a multiple of 32)
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    n[j] = nw + j * 32 + li;
    pcol[j] = ((n[j] & (2 * PAIRS - 1)) >> 1) * RS;
    bias[j] = (P.bias && n[j] < args.N) ? P.bias[n[j]] : 0.f;
  }
  const bool full_n = nw + 32 * BJ <= args.N;
  const float2 *tl = tab + wm * 32 + 4 * hf;  // row 8 (r / 4) + r % 4 of this lane's half
#pragma unroll
  for (int i = 0; i < BI; ++i) {
#pragma unroll
    for (int k = 0; k < KN; ++k) {
      const int qk = k * STEP;  // constant
      const int c = (qk >> 5) * WR + (STEP <= 32 ? (qk & 31) : 0) + 32 * i;
      pre[k] = src[(size_t)c * PAIRS];
    }
    if (i > 0) __syncthreads();  // phase i - 1's reads are done
#pragma unroll
    for (int k = 0; k < KN; ++k) wr[k * STEP] = pre[k];
    __syncthreads();
    const int mb = mw + i * 32;  // wave-uniform
    if (full_n) {
      float *__restrict__ cb = P.c + (size_t)(mb + 4 * hf) * args.ldc;
      // groups of four rows: the scheduling barrier keeps later groups' LDS
      // reads from being hoisted (their registers would cost the second
      // workgroup per CU)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int dr = 8 * g + rr;
          float *c = cb + (size_t)dr * args.ldc;
#pragma unroll
          for (int j = 0; j < BJ; ++j) {
            const float2 cs = tl[pcol[j] + dr];
            const float y = acc[i][j][4 * g + rr] + bias[j];
            const float yp = swap_pair(y);
            c[n[j]] = odd ? yp * cs.y + y * cs.x : y * cs.x - yp * cs.y;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        const int m = mb + 4 * hf + dr;
#pragma unroll
        for (int j = 0; j < BJ; ++j) {
          const float2 cs = tl[pcol[j] + dr];
          const float y = acc[i][j][r] + bias[j];
          const float yp = swap_pair(y);  // in every lane; only the store is predicated
          const float out = odd ? yp * cs.y + y * cs.x : y * cs.x - yp * cs.y;
          if (n[j] < args.N) P.c[(size_t)m * args.ldc + n[j]] = out;
        }
      }
    }
  }
}

__device__ __forceinline__ float stable_sigmoid(float x) {
  if (x >= 0.f) return 1.f / (1.f + expf(-x));
  const float z = expf(x);
  return z / (1.f + z);
}

// Activation and derivative codes of the derivative-from-output form
// (cdml_linear_preact without z, CDML_ACT_FROM_OUTPUT): ReLU whose zero output
// is -0 where z < 0 or z is NaN, and ReLU's derivative read from that sign.
// Leaky ReLU needs neither: its output has the sign of z, so act'(y) equals
// act'(z) with the same expression.
constexpr int kActReluMarked = 6;
constexpr int kDerivReluOut = 7;

// Activation derivative at the pre-activation z, as FillActivationAndDerivative
// (Neural Network/NeuralNetwork.cs:885-944) defines it, including its ReLU
// derivative of 1 at z = 0 and leaky-ReLU slope 0.1 for z <= 0.
__device__ __forceinline__ float act_deriv(float z, int act) {
  switch (act) {
    case CDML_ACT_SIGMOID: {
      const float s = stable_sigmoid(z);
      return s * (1.f - s);
    }
    case CDML_ACT_TANH: {
      const float t = tanhf(z);
      return 1.f - t * t;
    }
    case CDML_ACT_RELU:
      return z >= 0.f ? 1.f : 0.f;
    case CDML_ACT_LEAKYRELU:
      return z <= 0.f ? 0.1f : 1.f;
    case kDerivReluOut:  // z >= 0 exactly where the marked output is not -0
      return __float_as_int(z) < 0 ? 0.f : 1.f;
    case CDML_ACT_SWISH: {
      const float s = stable_sigmoid(z);
      return s + z * s * (1.f - s);
    }
    default:
      return 1.f;
  }
}

__device__ __forceinline__ float activate(float x, int act) {
  switch (act) {
    case CDML_ACT_SIGMOID:
      return stable_sigmoid(x);
    case CDML_ACT_TANH:
      return tanhf(x);
    case CDML_ACT_RELU:
      return x > 0.f ? x : 0.f;
    case kActReluMarked:
      return x > 0.f ? x : (x >= 0.f ? 0.f : -0.f);
    case CDML_ACT_LEAKYRELU:
      return x > 0.f ? x : 0.01f * x;
    case CDML_ACT_SWISH:
      return x * stable_sigmoid(x);
    default:
      return x;
  }
}

// Stores output (m, n) of problem P from z = acc + bias: pre <- z,
// v = act(z), v *= act'(dz) and v += add when those options are set, then
// C = v (or C + v with beta).
// The options are a compile-time switch (EPI) so that launches without them
// keep the plain epilogue.
template <bool EPI>
__device__ __forceinline__ void store_elem(const GemmArgs &args, const GemmProblem &P, int m, int n,
                                           float z, int act) {
  float v;
  if constexpr (EPI) {
    if (args.pre) args.pre[(size_t)m * args.ldpre + n] = z;
    v = activate(z, act);
    if (args.dz) v *= act_deriv(args.dz[(size_t)m * args.lddz + n], args.dact);
    if (args.add) v += args.add[(size_t)m * args.ldadd + n];
  } else {
    v = activate(z, act);
  }
  float *pc = P.c + (size_t)m * args.ldc + n;
  *pc = args.beta ? *pc + v : v;
}

inline bool has_epi(const GemmArgs &g) { return g.pre || g.dz || g.add; }

// Global -> register staging of one 128x32 tile of a row-major [rows, K]
// matrix.  VEC: K % 4 == 0 and 16-byte aligned rows, four float4 per thread;
// otherwise sixteen guarded scalars per thread.
template <bool VEC>
struct TileStage {
  float4 r[4];
  float s[16];

  __device__ __forceinline__ void load(const float *__restrict__ src, int ld, int row0, int rows,
                                       int k0, int K) {
    const int t = threadIdx.x;
    if constexpr (VEC) {
      const int c = (t & 7) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + (t >> 3) + 32 * i;
        if (row < rows && k0 + c < K)
          r[i] = *reinterpret_cast<const float4 *>(src + (size_t)row * ld + k0 + c);
        else
          r[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    } else {
      const int c = t & 31;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = row0 + (t >> 5) + 8 * i;
        s[i] = (row < rows && k0 + c < K) ? src[(size_t)row * ld + k0 + c] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(float (*lds)[LDSK]) {
    const int t = threadIdx.x;
    if constexpr (VEC) {
      const int c = (t & 7) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<float4 *>(&lds[(t >> 3) + 32 * i][c]) = r[i];
    } else {
      const int c = t & 31;
#pragma unroll
      for (int i = 0; i < 16; ++i) lds[(t >> 5) + 8 * i][c] = s[i];
    }
  }
};

// Guarded fallback of the forward layout (any K, any alignment).
template <bool VEC, bool EPI>
__global__ void __launch_bounds__(NTHREADS) gemm_nt_kernel(const GemmArgs args) {
  __shared__ __attribute__((aligned(16))) float As[2][BM][LDSK];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN][LDSK];

  const int lid = xcd_remap(blockIdx.x, args.padded);
  if (lid >= args.total) return;

  // Grouped ordering over (tiles_m, nprob * tiles_n): GROUP_M tile-rows share
  // each weight panel while it is hot in L2.
  const int tiles_n_all = args.tiles_n * args.nprob;
  const int in_group = GROUP_M * tiles_n_all;
  const int group = lid / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(args.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (lid % in_group) % gsize;
  const int tn_all = (lid % in_group) / gsize;
  const int prob = tn_all / args.tiles_n;
  const int tn = tn_all % args.tiles_n;

  const GemmProblem P = args.p[prob];
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = args.M, N = args.N, K = args.K;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, hf = lane >> 5;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  TileStage<VEC> sa, sb;
  const int nk = (K + BK - 1) / BK;
  sa.load(P.a, args.lda, m0, M, 0, K);
  sb.load(P.w, args.ldb, n0, N, 0, K);
  sa.store(As[0]);
  sb.store(Bs[0]);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      sa.load(P.a, args.lda, m0, M, (kt + 1) * BK, K);
      sb.load(P.w, args.ldb, n0, N, (kt + 1) * BK, K);
    }
#pragma unroll
    for (int u = 0; u < BK / 8; ++u) {
      float4 a4[2], b4[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a4[i] = *reinterpret_cast<const float4 *>(&As[cur][wm * 64 + i * 32 + li][u * 8 + hf * 4]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b4[j] = *reinterpret_cast<const float4 *>(&Bs[cur][wn * 64 + j * 32 + li][u * 8 + hf * 4]);
      const float av[2][4] = {{a4[0].x, a4[0].y, a4[0].z, a4[0].w},
                              {a4[1].x, a4[1].y, a4[1].z, a4[1].w}};
      const float bv[2][4] = {{b4[0].x, b4[0].y, b4[0].z, b4[0].w},
                              {b4[1].x, b4[1].y, b4[1].z, b4[1].w}};
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x2(av[i][r], bv[j][r], acc[i][j]);
    }
    if (more) {
      sa.store(As[cur ^ 1]);
      sb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  if (args.rope_cs && prob < 2) {
    store_rope<2, 2>(args, P, acc, m0 + wm * 64, n0 + wn * 64, li, hf);
    return;
  }
  // Epilogue: D[i][j] of block (bi, bj) sits at row 8*(r/4) + 4*hf + r%4,
  // column li; 32 lanes store 32 consecutive columns of one row.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + li;
    if (n >= N) continue;
    const float bias = P.bias ? P.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (m < M) store_elem<EPI>(args, P, m, n, acc[i][j][r] + bias, args.act);
      }
    }
  }
}

// Global -> LDS staging of one ROWS x BKK operand tile of the tiled kernel;
// the tile lands in LDS as [rows][k] (pitch BKK + 4) for either source layout.
//   T = false: the source is [rows][K] (k contiguous, row stride ld): each
//     thread moves 16-byte row pieces straight into LDS.  The F4R lanes of a
//     row are consecutive; the rows of a wave's 16 are interleaved, so that
//     consecutive lane quads write rows r, r + 4, r + 8, r + 12, whose 64-byte
//     pieces fall in disjoint bank ranges at pitch BKK + 4 (rows r and r + 1
//     share banks: c3's Q/K/V and output projections had 19.2 M and 6.4 M
//     conflict cycles per dispatch, now 0.5 M and 0, with the matrix pipes
//     busy 87.2% instead of 85.3% of the Q/K/V product's active cycles).
//   T = true:  the source is [K][rows] (rows contiguous, k-row stride ld):
//     each thread loads four consecutive rows of one k and stores them as four
//     LDS words.  Consecutive lanes take consecutive k, so the four stores of
//     a wave fall in distinct banks.
// Each thread's offsets are fixed for the whole K loop; rows past the end are
// clamped to the last row (T: the last four rows; rows % 4 == 0), so loads
// need no predication and clamped rows only feed results that are never
// stored.
template <int ROWS, int BKK, int NT, bool T>
struct OpStage {
  static constexpr int LD = BKK + 4;
  static constexpr int F4R = BKK / 4;   // T = false: vectors per row
  static constexpr int RPP = NT / F4R;  // T = false: rows per pass
  static constexpr int G = NT / BKK;    // T = true: four-row groups per pass
  static constexpr int NP = T ? ROWS / (4 * G) : ROWS / RPP;
  static_assert(NP >= 1 && (T ? ROWS % (4 * G) == 0 : ROWS % RPP == 0), "staging shape");
  uint32_t off[NP];
  vf4 v[NP];
  int sa, sb;  // T = false: (row, column); T = true: (k, row group)

  __device__ __forceinline__ void init(int row0, int rows, int ld) {
    const int t = threadIdx.x;
    if constexpr (T) {
      sa = t % BKK;
      sb = t / BKK;
#pragma unroll
      for (int i = 0; i < NP; ++i)
        off[i] = (uint32_t)sa * (uint32_t)ld + (uint32_t)min(row0 + 4 * (sb + G * i), rows - 4);
    } else {
      static_assert(F4R == 4 && RPP % 16 == 0, "row interleave");
      const int q = t / F4R;  // q's 16-row group keeps its rows, taken in the order 0, 4, 8, 12, 1, 5, ...
      sa = (q & ~15) | ((q & 3) << 2) | ((q >> 2) & 3);
      sb = (t % F4R) * 4;
#pragma unroll
      for (int i = 0; i < NP; ++i) off[i] = (uint32_t)min(row0 + sa + RPP * i, rows - 1) * (uint32_t)ld + sb;
    }
  }
  // First element of k-tile kt.
  static __device__ __forceinline__ const float *tile(const float *x, int kt, int ld) {
    return T ? x + (size_t)kt * BKK * ld : x + (size_t)kt * BKK;
  }
  __device__ __forceinline__ void load(const float *__restrict__ base) {
#pragma unroll
    for (int i = 0; i < NP; ++i) v[i] = *reinterpret_cast<const vf4 *>(base + off[i]);
  }
  __device__ __forceinline__ void store(float (*lds)[LD]) const {
    if constexpr (T) {
#pragma unroll
      for (int i = 0; i < NP; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) lds[4 * (sb + G * i) + c][sa] = v[i][c];
    } else {
#pragma unroll
      for (int i = 0; i < NP; ++i) *reinterpret_cast<vf4 *>(&lds[sa + RPP * i][sb]) = v[i];
    }
  }
};

// Tiled fast path (K % BKK == 0, 16-byte aligned rows, element offsets
// below 2^32; a transposed operand also needs rows % 4 == 0).  A workgroup of
// WM x WN waves computes a TM x TN tile of C, each wave a (TM/WM) x (TN/WN)
// block of 32x32 MFMA tiles.  K advances by BKK through double-buffered LDS.
// The LDS operands of group u + 1 are read while the MFMAs of group u run, and
// the k-tile after next is fetched while the current one is consumed.
// Measured on MI355X, high occupancy (four waves per SIMD with two 512-thread
// workgroups per CU) hides latency better than deeper register blocking.
//
// With TA and a bias-gradient pointer, the workgroups of the first column
// tile also sum each opA tile in LDS while it is current (every valid k-tile
// exactly once) and add the row sums to bgrad: the bias gradient of a
// weight-gradient GEMM costs no extra pass over dY.  Each thread keeps one
// partial sum (row t % TM, a 1/(NT/TM) slice of the k-tile); the slices meet
// in LDS at the end.
template <int TM, int TN, int BKK, int WM, int WN, int MINB, int ACT, bool TA, bool TB, bool EPI>
__global__ void __launch_bounds__(64 * WM * WN, MINB) gemm_tile_kernel(const GemmArgs args) {
  constexpr int NT = 64 * WM * WN;
  constexpr int LD = BKK + 4;
  constexpr int BI = TM / WM / 32, BJ = TN / WN / 32;
  static_assert(BI >= 1 && BJ >= 1, "tile shape");
  typedef OpStage<TM, BKK, NT, TA> StageA;
  typedef OpStage<TN, BKK, NT, TB> StageB;
  __shared__ __attribute__((aligned(16))) float As[2][TM][LD];
  __shared__ __attribute__((aligned(16))) float Bs[2][TN][LD];

  int lid = xcd_remap(blockIdx.x, args.padded);
  if (lid >= args.total) return;
  // Split-K: chunk-major, so the workgroups of one chunk (which share its
  // k-range of both operands) sit together on an XCD.
  int chunk = 0;
  if (args.ksplit > 1) {
    chunk = lid / args.tiles;
    lid -= chunk * args.tiles;
  }
  // Grouped ordering over (tiles_m, nprob * tiles_n): GROUP_M tile-rows share
  // each weight panel while it is hot in L2.
  const int tiles_n_all = args.tiles_n * args.nprob;
  const int in_group = GROUP_M * tiles_n_all;
  const int group = lid / in_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(args.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (lid % in_group) % gsize;
  const int tn_all = (lid % in_group) / gsize;
  // The RoPE instance keeps the problem index in a scalar register (the
  // divisions above run on the vector unit; left there, the values it keeps
  // for the staged-table epilogue cost its k-loop the VGPRs of the second
  // workgroup per CU).  Other instances allocate better without the hint.
  const int prob = ACT == kActRope ? __builtin_amdgcn_readfirstlane(tn_all / args.tiles_n) : tn_all / args.tiles_n;
  const int tn = tn_all % args.tiles_n;

  const GemmProblem P = args.p[prob];
  const int m0 = tm * TM, n0 = tn * TN;
  const int M = args.M, N = args.N, K = args.K;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, hf = lane >> 5;

  StageA sa;
  StageB sb;
  sa.init(m0, M, args.lda);
  sb.init(n0, N, args.ldb);
  floatx16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int kt0 = chunk * args.kchunk;
  const int nk = args.ksplit > 1 ? min(args.kchunk, K / BKK - kt0) : K / BKK;
  const float *__restrict__ A = StageA::tile(P.a, kt0, args.lda);
  const float *__restrict__ W = StageB::tile(P.w, kt0, args.ldb);
  // K segments exist only in the plain input-gradient instance (in the
  // epilogue instances their selects would cost the registers of the second
  // workgroup per CU); the segment of k-tile kt is wave-uniform, so choosing
  // it takes scalar selects only.
  constexpr bool SEG = TB && !TA && !EPI;
  const bool seg = SEG && args.kseg > 0;
  auto load_seg = [&](int kt) {
    const int sg = (kt >= args.kseg) + (kt >= 2 * args.kseg);
    const int kl = kt - sg * args.kseg;
    sa.load(StageA::tile(sg == 0 ? args.p[0].a : sg == 1 ? args.p[1].a : args.p[2].a, kl, args.lda));
    sb.load(StageB::tile(sg == 0 ? args.p[0].w : sg == 1 ? args.p[1].w : args.p[2].w, kl, args.ldb));
  };
  const bool bsum = TA && P.bgrad && tn == 0;
  constexpr int KCH = NT / TM;  // k slices per row for the bias-gradient sums
  static_assert(NT % TM == 0 && BKK % (4 * KCH) == 0, "bias-gradient slices");
  float bpart = 0.f;

  // k-tile 0 -> LDS, k-tile 1 -> registers
  if (SEG && seg) {
    load_seg(0);
  } else {
    sa.load(StageA::tile(A, 0, args.lda));
    sb.load(StageB::tile(W, 0, args.ldb));
  }
  sa.store(As[0]);
  sb.store(Bs[0]);
  {
    const int k1 = min(1, nk - 1);
    if (SEG && seg) {
      load_seg(k1);
    } else {
      sa.load(StageA::tile(A, k1, args.lda));
      sb.load(StageB::tile(W, k1, args.ldb));
    }
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float(*as)[LD] = &As[cur][wm * (TM / WM) + li];
    const float(*bsh)[LD] = &Bs[cur][wn * (TN / WN) + li];
    vf4 a4[BI], b4[BJ];
#pragma unroll
    for (int i = 0; i < BI; ++i) a4[i] = *reinterpret_cast<const vf4 *>(&as[i * 32][hf * 4]);
#pragma unroll
    for (int j = 0; j < BJ; ++j) b4[j] = *reinterpret_cast<const vf4 *>(&bsh[j * 32][hf * 4]);
#pragma unroll
    for (int u = 0; u < BKK / 8; ++u) {
      vf4 an[BI], bn[BJ];
      if (u + 1 < BKK / 8) {
#pragma unroll
        for (int i = 0; i < BI; ++i) an[i] = *reinterpret_cast<const vf4 *>(&as[i * 32][(u + 1) * 8 + hf * 4]);
#pragma unroll
        for (int j = 0; j < BJ; ++j) bn[j] = *reinterpret_cast<const vf4 *>(&bsh[j * 32][(u + 1) * 8 + hf * 4]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
          for (int j = 0; j < BJ; ++j) acc[i][j] = mfma32x32x2(a4[i][r], b4[j][r], acc[i][j]);
      if (u + 1 < BKK / 8) {
#pragma unroll
        for (int i = 0; i < BI; ++i) a4[i] = an[i];
#pragma unroll
        for (int j = 0; j < BJ; ++j) b4[j] = bn[j];
      }
    }
    // Stage k-tile kt + 1 (already in registers) and fetch k-tile kt + 2.
    // Past the end both are unconditional re-stages of the last tile into
    // the idle buffer, which nothing reads again: keeping them unconditional
    // keeps the staging registers out of scratch memory.
    sa.store(As[cur ^ 1]);
    sb.store(Bs[cur ^ 1]);
    if constexpr (TA) {
      if (bsum) {  // k-tile kt, stable in As[cur] until the barrier below
        const float *row = &As[cur][t % TM][(t / TM) * (BKK / KCH)];
#pragma unroll
        for (int e = 0; e < BKK / KCH; e += 4) {
          const vf4 x = *reinterpret_cast<const vf4 *>(row + e);
          bpart += (x[0] + x[1]) + (x[2] + x[3]);
        }
      }
    }
    const int k2 = min(kt + 2, nk - 1);
    if (SEG && seg) {
      load_seg(k2);
    } else {
      sa.load(StageA::tile(A, k2, args.lda));
      sb.load(StageB::tile(W, k2, args.ldb));
    }
    __syncthreads();
  }

  if constexpr (TA) {
    if (bsum) {  // uniform over the workgroup; the loop ended on a barrier
      float *red = &As[0][0][0];
      red[t] = bpart;
      __syncthreads();
      if (t < TM && m0 + t < M) {
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < KCH; ++c) s += red[t + c * TM];
        if (args.ksplit > 1)
          args.wsb[((size_t)chunk * args.nprob + prob) * M + m0 + t] = s;
        else
          P.bgrad[m0 + t] += s;
      }
    }
    if (args.ksplit > 1) {  // the partial product of this chunk, reduced later
      float *out = args.ws + ((size_t)chunk * args.nprob + prob) * (size_t)M * N;
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const int n = n0 + wn * (TN / WN) + j * 32 + li;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * (TM / WM) + i * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (m < M) out[(size_t)m * N + n] = acc[i][j][r];
          }
      }
      return;
    }
  }

  if constexpr (ACT == kActRope) {
    if (prob < 2) {
      // uniform: the whole workgroup takes one form
      const int pairs = args.rope_hd >> 1, seg = args.rope_seg;
      const int mseg = seg > 0 ? m0 % seg : m0;
      static_assert(sizeof(As) >= sizeof(float2) * 32 * (WM * 32 + 2), "RoPE table in LDS");
      // (the 128 x 128 configuration keeps store_rope: with the LDS form its
      // k-loop needs more than the 128 VGPRs of four waves per SIMD)
      const bool lds = TM == 256 && m0 + TM <= M && (seg <= 0 || mseg + TM <= seg);
      float2 *tab = reinterpret_cast<float2 *>(&As[0][0][0]);
      const int mw = m0 + wm * (TM / WM), nw = n0 + wn * (TN / WN);
      if (lds && pairs == 32)
        store_rope_lds<TM, WM, NT, BI, BJ, 5>(args, P, acc, mseg, wm, mw, nw, li, hf, tab);
      else if (lds && pairs == 16)
        store_rope_lds<TM, WM, NT, BI, BJ, 4>(args, P, acc, mseg, wm, mw, nw, li, hf, tab);
      else if (lds && pairs == 8)
        store_rope_lds<TM, WM, NT, BI, BJ, 3>(args, P, acc, mseg, wm, mw, nw, li, hf, tab);
      else if (lds && pairs == 4)
        store_rope_lds<TM, WM, NT, BI, BJ, 2>(args, P, acc, mseg, wm, mw, nw, li, hf, tab);
      else
        store_rope<BI, BJ>(args, P, acc, m0 + wm * (TM / WM), n0 + wn * (TN / WN), li, hf);
      return;
    }
  }
  // Epilogue: D[i][j] of block (bi, bj) sits at row 8*(r/4) + 4*hf + r%4,
  // column li; 32 lanes store 32 consecutive columns of one row.
  if constexpr (!EPI) {
    const int mw = m0 + wm * (TM / WM), nw = n0 + wn * (TN / WN);
    if (!args.beta && mw + TM / WM <= M && nw + TN / WN <= N) {
      // every row and column of this wave's blocks exists: no predicates, and
      // per row only a wave-uniform offset from the lane's base
      float bias[BJ];
#pragma unroll
      for (int j = 0; j < BJ; ++j) bias[j] = P.bias ? P.bias[nw + j * 32 + li] : 0.f;
      float *cb = P.c + (size_t)(mw + 4 * hf) * args.ldc + nw + li;
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float *c = cb + (size_t)(i * 32 + 8 * (r >> 2) + (r & 3)) * args.ldc;
#pragma unroll
          for (int j = 0; j < BJ; ++j)
            c[j * 32] = activate(acc[i][j][r] + bias[j], ACT == kActRope ? CDML_ACT_NONE : ACT);
        }
      return;
    }
  } else if constexpr (!TA) {
    const int mw = m0 + wm * (TM / WM), nw = n0 + wn * (TN / WN);
    if (!args.beta && mw + TM / WM <= M && nw + TN / WN <= N) {
      // The training epilogue on a whole wave block: the dz and add operands
      // of four rows are loaded before any of their stores (a load issued
      // after a store waits for it), and every address is a lane base plus a
      // wave-uniform row offset.
      float bias[BJ];
#pragma unroll
      for (int j = 0; j < BJ; ++j) bias[j] = P.bias ? P.bias[nw + j * 32 + li] : 0.f;
      const size_t lane_c = (size_t)(mw + 4 * hf) * args.ldc + nw + li;
      const size_t lane_pre = (size_t)(mw + 4 * hf) * args.ldpre + nw + li;
      const size_t lane_dz = (size_t)(mw + 4 * hf) * args.lddz + nw + li;
      const size_t lane_add = (size_t)(mw + 4 * hf) * args.ldadd + nw + li;
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float zv[4][BJ], av[4][BJ];
          if (args.dz) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
              for (int j = 0; j < BJ; ++j)
                zv[rr][j] = args.dz[lane_dz + (size_t)(i * 32 + 8 * g + rr) * args.lddz + j * 32];
          }
          if (args.add) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
              for (int j = 0; j < BJ; ++j)
                av[rr][j] = args.add[lane_add + (size_t)(i * 32 + 8 * g + rr) * args.ldadd + j * 32];
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int r = 4 * g + rr, d = i * 32 + 8 * g + rr;
#pragma unroll
            for (int j = 0; j < BJ; ++j) {
              const float z = acc[i][j][r] + bias[j];
              if (args.pre) args.pre[lane_pre + (size_t)d * args.ldpre + j * 32] = z;
              float v = activate(z, ACT == kActRope ? CDML_ACT_NONE : ACT);
              if (args.dz) v *= act_deriv(zv[rr][j], args.dact);
              if (args.add) v += av[rr][j];
              P.c[lane_c + (size_t)d * args.ldc + j * 32] = v;
            }
          }
        }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const int n = n0 + wn * (TN / WN) + j * 32 + li;
    if (n >= N) continue;
    const float bias = P.bias ? P.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < BI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * (TM / WM) + i * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (m < M) store_elem<EPI>(args, P, m, n, acc[i][j][r] + bias, ACT == kActRope ? CDML_ACT_NONE : ACT);
      }
    }
  }
}

// Few rows (decode steps, short batches: M <= MR), non-transposed operands,
// 16-byte aligned rows with K % 4 == 0.  One wave per pair of output columns
// (n, n + 1): its lanes stride over K in float4 steps, each keeping 2 x MR
// partial dot products, which xor-shuffle sums then complete in every lane.
// The kernel is short (no LDS, no MFMA tiles), so a launch costs little more
// than the bytes of W it streams; the pair is also the rotation pair of the
// fused RoPE epilogue (head dims are even).
template <int MR, bool EPI>
__global__ void __launch_bounds__(256) gemm_rows_kernel(const GemmArgs args) {
  const int prob = blockIdx.y;
  const GemmProblem P = args.p[prob];
  const int M = args.M, N = args.N, K = args.K;
  const int lane = threadIdx.x & 63;
  const int n0 = 2 * (blockIdx.x * 4 + (threadIdx.x >> 6));
  if (n0 >= N) return;
  const int n1 = min(n0 + 1, N - 1);
  const float *__restrict__ w0 = P.w + (size_t)n0 * args.ldb;
  const float *__restrict__ w1 = P.w + (size_t)n1 * args.ldb;
  float s0[MR], s1[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) s0[m] = s1[m] = 0.f;
  for (int k = 4 * lane; k < K; k += 256) {
    const float4 a = *reinterpret_cast<const float4 *>(w0 + k);
    const float4 b = *reinterpret_cast<const float4 *>(w1 + k);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const float4 x = *reinterpret_cast<const float4 *>(P.a + (size_t)m * args.lda + k);
        s0[m] += (x.x * a.x + x.y * a.y) + (x.z * a.z + x.w * a.w);
        s1[m] += (x.x * b.x + x.y * b.y) + (x.z * b.z + x.w * b.w);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s0[m] += __shfl_xor(s0[m], off);
      s1[m] += __shfl_xor(s1[m], off);
    }
  }
  // lane m stores row m
  float z0 = 0.f, z1 = 0.f;
#pragma unroll
  for (int m = 0; m < MR; ++m)
    if (lane == m) {
      z0 = s0[m];
      z1 = s1[m];
    }
  if (lane >= M) return;
  const int m = lane;
  const bool has1 = n0 + 1 < N;
  z0 += P.bias ? P.bias[n0] : 0.f;
  if (has1) z1 += P.bias ? P.bias[n0 + 1] : 0.f;
  if (args.rope_cs && prob < 2) {  // AccelerationCPU.cs:4947-4975 on the pair (n0, n0 + 1)
#pragma clang fp contract(off)
    int pos = args.rope_pos0 + (args.rope_seg > 0 ? m % args.rope_seg : m);
    pos = min(pos, args.rope_npos - 1);
    const float2 t = args.rope_cs[(size_t)pos * (args.rope_hd >> 1) + ((n0 % args.rope_hd) >> 1)];
    float *c = P.c + (size_t)m * args.ldc + n0;
    c[0] = z0 * t.x - z1 * t.y;
    if (has1) c[1] = z1 * t.x + z0 * t.y;
    return;
  }
  store_elem<EPI>(args, P, m, n0, z0, args.act);
  if (has1) store_elem<EPI>(args, P, m, n0 + 1, z1, args.act);
}

// A short reduction (K <= 16: the input projection of a time-series model,
// F features -> D), non-transposed operands, N <= 1024: thread t owns the
// four columns 4 (t % n4) .. + 3 (n4 = ceil(N / 4)) of rows t / n4,
// t / n4 + 256 / n4, ..., and keeps their K x 4 weights and biases in
// registers.  The threads of one row read the same K inputs (broadcast
// loads) and the four results leave as one float4 when the row layout
// allows it.  Every output sums its K products in k order.  TB: W is read as
// [K, N] (the input gradient dX = dY W of a layer with few outputs).
template <bool EPI, bool TB = false>
__global__ void __launch_bounds__(256) gemm_smallk_kernel(const GemmArgs args) {
  const GemmProblem P = args.p[blockIdx.y];
  const int M = args.M, N = args.N, K = args.K;
  const int n4 = (N + 3) / 4;
  const int rpp = 256 / n4;  // rows per pass of the workgroup (n4 <= 256)
  const int r = threadIdx.x / n4, n0 = (threadIdx.x % n4) * 4;
  if (r >= rpp) return;      // threads past the last whole row group
  float w[16][4], bias[4];
#pragma unroll
  for (int k = 0; k < 16; ++k)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = min(n0 + c, N - 1);
      w[k][c] = k < K ? P.w[TB ? (size_t)k * args.ldb + n : (size_t)n * args.ldb + k] : 0.f;
    }
#pragma unroll
  for (int c = 0; c < 4; ++c) bias[c] = P.bias && n0 + c < N ? P.bias[n0 + c] : 0.f;
  for (int m = blockIdx.x * rpp + r; m < M; m += gridDim.x * rpp) {
    const float *__restrict__ x = P.a + (size_t)m * args.lda;
    float z[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k < K) {
        const float xv = x[k];
#pragma unroll
        for (int c = 0; c < 4; ++c) z[c] += xv * w[k][c];
      }
    }
    float *crow = P.c + (size_t)m * args.ldc;
    if (!EPI && !args.beta && n0 + 3 < N && ((reinterpret_cast<uintptr_t>(crow + n0) & 15) == 0)) {
      vf4 y;
#pragma unroll
      for (int c = 0; c < 4; ++c) y[c] = activate(z[c] + bias[c], args.act);
      *reinterpret_cast<vf4 *>(crow + n0) = y;
      continue;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (n0 + c < N) store_elem<EPI>(args, P, m, n0 + c, z[c] + bias[c], args.act);
  }
}

// Few output columns (N <= 4: a regression head, D -> 1), non-transposed
// operands, K % 4 == 0 with 16-byte aligned rows: the 16 lanes of a group
// take every 16th float4 of one row, their partial dot products meet through
// four xor shuffles inside the group, and its first lane stores the N
// outputs.  (The tiled kernel would run a 128 x 128 MFMA tile for one live
// column.)
constexpr int kNarrowN = 4;
template <bool EPI>
__global__ void __launch_bounds__(256) gemm_narrow_n_kernel(const GemmArgs args) {
  const GemmProblem P = args.p[blockIdx.y];
  const int M = args.M, N = args.N, K4 = args.K / 4;
  const int g = threadIdx.x & 15;
  for (int m = (blockIdx.x * 256 + threadIdx.x) >> 4; m < M; m += gridDim.x * 16) {
    const float *__restrict__ x = P.a + (size_t)m * args.lda;
    float z[kNarrowN] = {0.f, 0.f, 0.f, 0.f};
    for (int i = g; i < K4; i += 16) {
      const vf4 xv = *reinterpret_cast<const vf4 *>(x + 4 * i);
#pragma unroll
      for (int n = 0; n < kNarrowN; ++n)
        if (n < N) {
          const vf4 wv = *reinterpret_cast<const vf4 *>(P.w + (size_t)n * args.ldb + 4 * i);
          z[n] += (xv[0] * wv[0] + xv[1] * wv[1]) + (xv[2] * wv[2] + xv[3] * wv[3]);
        }
    }
#pragma unroll
    for (int n = 0; n < kNarrowN; ++n)
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) z[n] += __shfl_xor(z[n], off, 16);
    if (g == 0) {
#pragma unroll
      for (int n = 0; n < kNarrowN; ++n)
        if (n < N) store_elem<EPI>(args, P, m, n, z[n] + (P.bias ? P.bias[n] : 0.f), args.act);
    }
  }
}

// Any layout, any shape (the gradient GEMMs whose sizes miss the tiled
// kernel's conditions): a 64 x 64 tile of C per 256-thread workgroup, 4 x 4
// outputs per thread, K in steps of 16 through LDS with guarded loads that
// walk each source along its contiguous dimension.
template <bool TA, bool TB, bool EPI>
__global__ void __launch_bounds__(256) gemm_any_kernel(const GemmArgs args) {
  __shared__ float As[16][65], Bs[16][65];  // [k][m], [k][n]
  const GemmProblem P = args.p[blockIdx.z];
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int M = args.M, N = args.N, K = args.K;
  const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = t; e < 1024; e += 256) {
      const int kk = TA ? e / 64 : e % 16, mm = TA ? e % 64 : e / 16;
      const int m = m0 + mm, k = k0 + kk;
      As[kk][mm] = (m < M && k < K) ? (TA ? P.a[(size_t)k * args.lda + m] : P.a[(size_t)m * args.lda + k]) : 0.f;
      const int kb = TB ? e / 64 : e % 16, nn = TB ? e % 64 : e / 16;
      const int n = n0 + nn, kq = k0 + kb;
      Bs[kb][nn] = (n < N && kq < K) ? (TB ? P.w[(size_t)kq * args.ldb + n] : P.w[(size_t)n * args.ldb + kq]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      store_elem<EPI>(args, P, m, n, acc[i][j] + (P.bias ? P.bias[n] : 0.f), args.act);
    }
  }
}

// bgrad[m] += sum_k opA[m, k] for the problems of a gemm_any_kernel launch.
template <bool TA>
__global__ void __launch_bounds__(256) op_rowsum_kernel(const GemmArgs args) {
  const GemmProblem P = args.p[blockIdx.y];
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (!P.bgrad || m >= args.M) return;
  float s = 0.f;
  for (int k = 0; k < args.K; ++k) s += TA ? P.a[(size_t)k * args.lda + m] : P.a[(size_t)m * args.lda + k];
  P.bgrad[m] += s;
}

// Sum of the split-K partials: C (+)= sum_c ws[c], bgrad += sum_c wsb[c].
// N % 4 == 0 (the tiled path's transposed staging of opB needs it), so an
// output is four consecutive columns.  LANES consecutive lanes share an
// output: lane g adds chunks g, g + LANES, ... in order, and a fixed
// xor-shuffle tree joins the sums, so the order of every addition is fixed
// (the same bits on every run) while the chunk loads of the group are in
// flight together.  The group of output e also sums bias row e.  Eight
// lanes pay off from 32 chunks on; below that one lane walks the chunks.
template <int LANES>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmArgs args) {
  constexpr int kReduceLanes = LANES;
  const int prob = blockIdx.y;
  const GemmProblem P = args.p[prob];
  const int M = args.M, N = args.N, n4 = N >> 2;
  const size_t plane = (size_t)args.nprob * M * N;
  const size_t e = ((size_t)blockIdx.x * 256 + threadIdx.x) / kReduceLanes;
  const int g = threadIdx.x % kReduceLanes;
  const size_t n_out = (size_t)M * n4;
  if (e < n_out) {
    const int m = (int)(e / n4), n = (int)(e % n4) * 4;
    const float *src = args.ws + (size_t)prob * M * N + (size_t)m * N + n;
    vf4 s = {0.f, 0.f, 0.f, 0.f};
    for (int c = g; c < args.ksplit; c += kReduceLanes) {
      const vf4 x = *reinterpret_cast<const vf4 *>(src + c * plane);
      s[0] += x[0];
      s[1] += x[1];
      s[2] += x[2];
      s[3] += x[3];
    }
    // the ragged last rows: opA stored [K, M], opB [K, N] (16-byte rows)
    for (int k = args.ktail0 + g; args.ktail0 > 0 && k < args.K; k += kReduceLanes) {
      const float av = P.a[(size_t)k * args.lda + m];
      const vf4 bv = *reinterpret_cast<const vf4 *>(P.w + (size_t)k * args.ldb + n);
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] += av * bv[q];
    }
#pragma unroll
    for (int off = kReduceLanes / 2; off > 0; off >>= 1)
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] += __shfl_xor(s[q], off);
    if (g == 0) {
      float *dst = P.c + (size_t)m * args.ldc + n;
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = args.beta ? dst[q] + s[q] : s[q];
    }
  }
  // every lane of a group runs the shuffles together (e is uniform in a group)
  if (P.bgrad && e < (size_t)M) {
    float s = 0.f;
    for (int c = g; c < args.ksplit; c += kReduceLanes)
      s += args.wsb[((size_t)c * args.nprob + prob) * M + e];
    for (int k = args.ktail0 + g; args.ktail0 > 0 && k < args.K; k += kReduceLanes)
      s += P.a[(size_t)k * args.lda + e];
#pragma unroll
    for (int off = kReduceLanes / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (g == 0) P.bgrad[e] += s;
  }
}

// Split-K plan of a weight-gradient GEMM (M = out, N = in, K = rows): enough
// chunks to give every CU two resident workgroups when the output alone has
// too few tiles, at least eight k-tiles (128 rows) per chunk (two for small
// outputs).
struct SplitPlan {
  int ksplit = 1, kchunk = 0;
  bool small = false;  // small output: wgrad_small_kernel, kchunk in rows
  size_t bytes = 0;    // workspace: ksplit * nprob * (M * N + M) floats
};

// Weight gradients whose output is too small or too oddly shaped for the
// tiled kernel (an input projection [D, 5], a regression head [1, D]) but
// whose row reduction is long: block c sums rows [c * kchunk, (c + 1) *
// kchunk) of opA^T opB (opA stored [K, M], opB [K, N]) and of opA's row
// sums into its own partial; wgrad_small_reduce_kernel adds the partials in
// block order.  Each thread owns up to kSmallPer outputs.
constexpr int kSmallPer = 16;
constexpr int kSmallOut = 256 * kSmallPer;

__global__ void __launch_bounds__(256) wgrad_small_kernel(const GemmArgs args) {
  const int chunk = blockIdx.x, prob = blockIdx.y, t = threadIdx.x;
  const GemmProblem P = args.p[prob];
  const int M = args.M, N = args.N, MN = M * N;
  const int k0 = chunk * args.kchunk, k1 = min(args.K, k0 + args.kchunk);
  float acc[kSmallPer], bacc[kSmallPer];
  int am[kSmallPer], bn[kSmallPer];
#pragma unroll
  for (int i = 0; i < kSmallPer; ++i) {
    const int e = min(t + 256 * i, MN - 1);
    am[i] = e / N;
    bn[i] = e % N;
    acc[i] = bacc[i] = 0.f;
  }
  const bool bsum = P.bgrad != nullptr;
  for (int k = k0; k < k1; ++k) {
    const float *ar = P.a + (size_t)k * args.lda;
    const float *br = P.w + (size_t)k * args.ldb;
#pragma unroll
    for (int i = 0; i < kSmallPer; ++i)
      if (t + 256 * i < MN) acc[i] += ar[am[i]] * br[bn[i]];
    if (bsum) {
#pragma unroll
      for (int i = 0; i < kSmallPer; ++i)
        if (t + 256 * i < M) bacc[i] += ar[t + 256 * i];
    }
  }
  float *out = args.ws + ((size_t)chunk * args.nprob + prob) * MN;
#pragma unroll
  for (int i = 0; i < kSmallPer; ++i)
    if (t + 256 * i < MN) out[t + 256 * i] = acc[i];
  if (bsum) {
    float *ob = args.wsb + ((size_t)chunk * args.nprob + prob) * M;
#pragma unroll
    for (int i = 0; i < kSmallPer; ++i)
      if (t + 256 * i < M) ob[t + 256 * i] = bacc[i];
  }
}

// The same weight gradients when one side is narrow (at most kNarrow): the
// input projection [D, F] (F = 5) and a regression head [O, D] (O <= 16).
// Threads run along the wide side, so each row of that operand is one
// coalesced load and the narrow side's few values of the row are broadcast
// loads; a thread keeps the narrow side's sums (and the bias row sums) in
// registers over its chunk of rows, in row order, four rows per iteration.
// OVER_M: the output rows m are wide (thread m, columns n < N narrow);
// otherwise the columns n are wide and the rows m < M narrow.
constexpr int kNarrow = 16;
template <bool OVER_M>
__global__ void __launch_bounds__(256) wgrad_narrow_kernel(const GemmArgs args) {
  const int chunk = blockIdx.x, prob = blockIdx.z;
  const GemmProblem P = args.p[prob];
  const int M = args.M, N = args.N, MN = M * N;
  const int wide = OVER_M ? M : N, narrow = OVER_M ? N : M;
  const int i = blockIdx.y * 256 + threadIdx.x;
  const int ic = min(i, wide - 1);
  const int k0 = chunk * args.kchunk, k1 = min(args.K, k0 + args.kchunk);
  const bool bsum = P.bgrad != nullptr;
  float acc[kNarrow], bacc[kNarrow];
#pragma unroll
  for (int j = 0; j < kNarrow; ++j) acc[j] = bacc[j] = 0.f;
  auto row = [&](int k) {
    const float *ar = P.a + (size_t)k * args.lda;
    const float *br = P.w + (size_t)k * args.ldb;
    if constexpr (OVER_M) {
      const float x = ar[ic];
#pragma unroll
      for (int j = 0; j < kNarrow; ++j)
        if (j < narrow) acc[j] += x * br[j];
      bacc[0] += x;
    } else {
      const float y = br[ic];
#pragma unroll
      for (int j = 0; j < kNarrow; ++j)
        if (j < narrow) {
          const float x = ar[j];
          acc[j] += x * y;
          bacc[j] += x;
        }
    }
  };
  int k = k0;
  for (; k + 4 <= k1; k += 4) {
    row(k);
    row(k + 1);
    row(k + 2);
    row(k + 3);
  }
  for (; k < k1; ++k) row(k);
  if (i >= wide) return;
  float *out = args.ws + ((size_t)chunk * args.nprob + prob) * MN;
#pragma unroll
  for (int j = 0; j < kNarrow; ++j)
    if (j < narrow) out[OVER_M ? (size_t)i * N + j : (size_t)j * N + i] = acc[j];
  if (bsum) {
    float *ob = args.wsb + ((size_t)chunk * args.nprob + prob) * M;
    if constexpr (OVER_M) {
      ob[i] = bacc[0];
    } else if (i == 0) {
#pragma unroll
      for (int j = 0; j < kNarrow; ++j)
        if (j < narrow) ob[j] = bacc[j];
    }
  }
}

// Sum of the small-output partials, kSmallLanes lanes per output: lane g adds
// chunks g, g + kSmallLanes, ... in order and a fixed xor-shuffle tree joins
// them (the same bits on every run); the group of output e also sums bias
// row e.
constexpr int kSmallLanes = 64;
__global__ void __launch_bounds__(256) wgrad_small_reduce_kernel(const GemmArgs args) {
  const int prob = blockIdx.y;
  const GemmProblem P = args.p[prob];
  const int M = args.M, N = args.N, MN = M * N;
  const int e = (blockIdx.x * 256 + threadIdx.x) / kSmallLanes;
  const int g = threadIdx.x % kSmallLanes;
  if (e < MN) {
    float s = 0.f;
    for (int c = g; c < args.ksplit; c += kSmallLanes) s += args.ws[((size_t)c * args.nprob + prob) * MN + e];
#pragma unroll
    for (int off = kSmallLanes / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (g == 0) {
      float *dst = P.c + (size_t)(e / N) * args.ldc + e % N;
      *dst = args.beta ? *dst + s : s;
    }
  }
  if (P.bgrad && e < M) {
    float s = 0.f;
    for (int c = g; c < args.ksplit; c += kSmallLanes) s += args.wsb[((size_t)c * args.nprob + prob) * M + e];
#pragma unroll
    for (int off = kSmallLanes / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (g == 0) P.bgrad[e] += s;
  }
}

// The 256 x 128 eight-wave tiles for M >= 1024, and for weight gradients
// (both operands transposed, a long row reduction split over chunks) whose
// M is a multiple of 256; 128 x 128 four-wave tiles otherwise.
inline bool big_tiles(int M, bool wgrad) { return M >= 1024 || (wgrad && M % 256 == 0); }

SplitPlan splitk_plan(int M, int N, int K, int nprob) {
  SplitPlan sp;
  const int nk = K / 16;  // whole k-tiles; the reduce or a tail launch adds a ragged tail
  sp.kchunk = nk;
  if (M <= 0 || N <= 0) return sp;
  if (nk < 1 || N % 4 || M % 4) {  // not the tiled kernel's shape
    if ((long long)M * N > kSmallOut || K < 2048) return sp;
    sp.small = true;
    // chunks of 64 rows (at most 4096 chunks): each workgroup's row loop is
    // short, so the launch is not bound by one loop's load latency
    const int bound = std::min(4096, (K + 63) / 64);
    sp.ksplit = bound;
    sp.kchunk = (K + sp.ksplit - 1) / sp.ksplit;
    sp.ksplit = (K + sp.kchunk - 1) / sp.kchunk;
    // sized for the bound, which never decreases with K: a workspace sized
    // for a caller's largest row count covers every smaller one
    sp.bytes = (size_t)bound * nprob * ((size_t)M * N + M) * sizeof(float);
    return sp;
  }
  const bool big = big_tiles(M, true);
  const int TM = big ? 256 : 128, TN = 128;
  const int tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN) * nprob;
  const int slots = big ? 512 : 1024;
  // at least eight k-tiles per chunk, or two for a small output (at most
  // 64 K elements, so a chunk's partial is at most 256 KB): a short
  // reduction into a few tiles is otherwise one workgroup's serial k-loop
  const int min_kt = (long long)M * N * nprob <= 65536 ? 2 : 8;
  const int s = std::min(slots / tiles, nk / min_kt);
  if (s <= 1) return sp;
  sp.kchunk = (nk + s - 1) / s;
  sp.ksplit = (nk + sp.kchunk - 1) / sp.kchunk;
  if (sp.ksplit <= 1) {
    sp = SplitPlan{};
    sp.kchunk = nk;
    return sp;
  }
  // sized for s (at least ksplit, and never decreasing with K, unlike
  // ksplit itself: 75 k-tiles in 3-tile chunks take 25, 74 in 2-tile chunks
  // 37), so a workspace sized for a caller's largest row count covers every
  // smaller one
  sp.bytes = (size_t)s * nprob * ((size_t)M * N + M) * sizeof(float);
  return sp;
}

// The forward tile kernel for the launch's activation.
template <int TM, int TN, int BKK, int WM, int WN, int MINB, bool EPI>
void launch_tile_act(const GemmArgs &g, dim3 grid, dim3 block, hipStream_t stream) {
  switch (g.act) {
    case CDML_ACT_NONE: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_NONE, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_SIGMOID: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_SIGMOID, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_TANH: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_TANH, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_RELU: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_RELU, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_LEAKYRELU: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_LEAKYRELU, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
    case kActReluMarked:
      if constexpr (!EPI) {  // only launches without z use it
        gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, kActReluMarked, false, false, false><<<grid, block, 0, stream>>>(g);
        break;
      }
      [[fallthrough]];
    default: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_SWISH, false, false, EPI><<<grid, block, 0, stream>>>(g); break;
  }
}

// Two tile configurations: 256 x 128 with eight waves for M >= 1024, and
// 128 x 128 with four waves for smaller M (decode rows, short sequences).
template <int TM, int TN, int BKK, int WM, int WN, int MINB, bool TA, bool TB>
int launch_tile(GemmArgs g, hipStream_t stream) {
  g.tiles_m = (g.M + TM - 1) / TM;
  g.tiles_n = (g.N + TN - 1) / TN;
  g.tiles = g.tiles_m * g.tiles_n * g.nprob;
  if (g.ksplit < 1) g.ksplit = 1;
  g.total = g.tiles * g.ksplit;
  g.padded = pad_to_xcd(g.total);
  const dim3 grid(g.padded), block(64 * WM * WN);
  if constexpr (TA || TB) {
    if (has_epi(g))
      gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_NONE, TA, TB, true><<<grid, block, 0, stream>>>(g);
    else
      gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_NONE, TA, TB, false><<<grid, block, 0, stream>>>(g);
    if (g.ksplit > 1) {
      const size_t outs = std::max((size_t)g.M * (g.N / 4), (size_t)g.M);
      if (g.ksplit >= 32)
        splitk_reduce_kernel<8><<<dim3((unsigned)((outs * 8 + 255) / 256), g.nprob), dim3(256), 0, stream>>>(g);
      else
        splitk_reduce_kernel<1><<<dim3((unsigned)((outs + 255) / 256), g.nprob), dim3(256), 0, stream>>>(g);
    }
  } else {
    if (g.rope_cs) {
      gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, kActRope, false, false, false><<<grid, block, 0, stream>>>(g);
      return CDML_OK;
    }
    if (has_epi(g)) {
      launch_tile_act<TM, TN, BKK, WM, WN, MINB, true>(g, grid, block, stream);
    } else {
      launch_tile_act<TM, TN, BKK, WM, WN, MINB, false>(g, grid, block, stream);
    }
  }
  return CDML_OK;
}

// Whether a [rows, K] (T = false) or [K, rows] (T = true) operand with row
// stride ld and base p suits the tiled kernel's staging.
bool stage_ok(const float *p, int rows, int ld, bool T, int bkk) {
  if (!aligned16(p) || ld % 4) return false;
  if (T) return rows % 4 == 0 && (unsigned long long)bkk * ld + rows < (1ull << 32);
  return (unsigned long long)rows * ld < (1ull << 32);
}

template <bool TA, bool TB>
int launch_layout(GemmArgs &g, bool fast, hipStream_t stream) {
  if (fast) return big_tiles(g.M, TA && TB) ? launch_tile<256, 128, 16, 4, 2, 2, TA, TB>(g, stream)
                                            : launch_tile<128, 128, 16, 2, 2, 2, TA, TB>(g, stream);
  const dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, g.nprob);
  if (has_epi(g)) gemm_any_kernel<TA, TB, true><<<grid, dim3(256), 0, stream>>>(g);
  else gemm_any_kernel<TA, TB, false><<<grid, dim3(256), 0, stream>>>(g);
  bool bgrad = false;
  for (int i = 0; i < g.nprob; ++i) bgrad = bgrad || g.p[i].bgrad;
  if (bgrad && g.K > 0) op_rowsum_kernel<TA><<<dim3((g.M + 255) / 256, g.nprob), dim3(256), 0, stream>>>(g);
  return CDML_OK;
}

// ta / tb: opA / opB stored transposed ([K, M] / [K, N]).
int launch_gemm(GemmArgs &g, bool ta, bool tb, hipStream_t stream, const char *what) {
  if (g.M == 0 || g.N == 0) return CDML_OK;
  if ((ta || tb) && (g.M > 65535 * 64 || g.N > 65535 * 64))
    return fail(CDML_E_INVALID, "%s: matrix too large", what);
  bool fast = g.K % 16 == 0 && g.K > 0;
  for (int i = 0; i < g.nprob; ++i)
    fast = fast && stage_ok(g.p[i].a, g.M, g.lda, ta, 16) && stage_ok(g.p[i].w, g.N, g.ldb, tb, 16);
  if (g.kseg) {  // only the tiled input-gradient kernel reads K segments
    bool ok = !ta && tb && !has_epi(g) && g.nprob == 1 && g.ksplit <= 1 && g.kseg * 16 * 3 == g.K;
    for (int i = 0; ok && i < 3; ++i)
      ok = stage_ok(g.p[i].a, g.M, g.lda, false, 16) && stage_ok(g.p[i].w, g.N, g.ldb, true, 16);
    if (!ok) return fail(CDML_E_INVALID, "%s: K segments need the tiled input-gradient kernel", what);
    fast = true;
  }
  if (ta || tb) {
    int rc;
    // A ragged K: the tiled kernel covers the whole 16-row k-tiles (it never
    // reads past them) and the last K % 16 rows are added by a second launch
    // (C += tail, bgrad += tail row sums) -- unless an epilogue must see the
    // complete sum.
    const int ktail = g.K % 16;
    bool split_tail = tb && ktail != 0 && g.K >= 16 && !g.dz && !g.add && !g.pre && g.act == CDML_ACT_NONE;
    for (int i = 0; split_tail && i < g.nprob; ++i)
      split_tail = stage_ok(g.p[i].a, g.M, g.lda, ta, 16) && stage_ok(g.p[i].w, g.N, g.ldb, tb, 16);
    if (!ta && tb && g.K <= 16 && g.K > 0 && g.M > 16 && g.N <= 1024) {  // few layer outputs
      const int rpp = 256 / ((g.N + 3) / 4);
      const dim3 grid((unsigned)std::min((g.M + rpp - 1) / rpp, 2048), (unsigned)g.nprob), block(256);
      has_epi(g) ? gemm_smallk_kernel<true, true><<<grid, block, 0, stream>>>(g)
                 : gemm_smallk_kernel<false, true><<<grid, block, 0, stream>>>(g);
      return check_launch(what);
    }
    if (ta && tb && g.small && g.ksplit > 1) {  // small output, long reduction
      if (g.N <= kNarrow)
        wgrad_narrow_kernel<true><<<dim3(g.ksplit, (g.M + 255) / 256, g.nprob), dim3(256), 0, stream>>>(g);
      else if (g.M <= kNarrow)
        wgrad_narrow_kernel<false><<<dim3(g.ksplit, (g.N + 255) / 256, g.nprob), dim3(256), 0, stream>>>(g);
      else
        wgrad_small_kernel<<<dim3(g.ksplit, g.nprob), dim3(256), 0, stream>>>(g);
      const int n = std::max(g.M * g.N, g.M) * kSmallLanes;
      wgrad_small_reduce_kernel<<<dim3((n + 255) / 256, g.nprob), dim3(256), 0, stream>>>(g);
      return check_launch(what);
    }
    if (ta && tb && split_tail && g.ksplit > 1 && !g.small && g.N % 4 == 0) {
      // split-K: the reduce adds the last K % 16 rows, no tail launch
      g.ktail0 = g.K - ktail;
      split_tail = false;
      rc = launch_layout<true, true>(g, true, stream);
    } else if (ta && tb) rc = launch_layout<true, true>(g, fast || split_tail, stream);
    else if (tb) rc = launch_layout<false, true>(g, fast || split_tail, stream);
    else rc = launch_layout<true, false>(g, false, stream);
    if (rc) return rc;
    if (split_tail) {
      const int kmain = g.K - ktail;
      GemmArgs t = g;
      t.K = ktail;
      t.beta = 1;
      t.ksplit = 1;
      for (int i = 0; i < t.nprob; ++i) {
        t.p[i].a += ta ? (size_t)kmain * g.lda : (size_t)kmain;
        t.p[i].w += tb ? (size_t)kmain * g.ldb : (size_t)kmain;
      }
      rc = ta ? launch_layout<true, true>(t, false, stream) : launch_layout<false, true>(t, false, stream);
      if (rc) return rc;
    }
    return check_launch(what);
  }
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  g.total = g.tiles_m * g.tiles_n * g.nprob;
  g.padded = pad_to_xcd(g.total);
  bool vec = (g.K % 4 == 0) && (g.lda % 4 == 0) && (g.ldb % 4 == 0);
  for (int i = 0; i < g.nprob; ++i) vec = vec && aligned16(g.p[i].a) && aligned16(g.p[i].w);
  if (g.K <= 16 && g.K > 0 && g.M > 16 && !g.rope_cs && g.N <= 1024) {
    const int rpp = 256 / ((g.N + 3) / 4);
    const dim3 grid((unsigned)std::min((g.M + rpp - 1) / rpp, 2048), (unsigned)g.nprob), block(256);
    has_epi(g) ? gemm_smallk_kernel<true><<<grid, block, 0, stream>>>(g)
               : gemm_smallk_kernel<false><<<grid, block, 0, stream>>>(g);
    return check_launch(what);
  }
  if (vec && g.N <= kNarrowN && g.K > 16 && g.M > 16 && !g.rope_cs) {
    const dim3 grid((unsigned)std::min((g.M + 15) / 16, 4096), (unsigned)g.nprob), block(256);
    has_epi(g) ? gemm_narrow_n_kernel<true><<<grid, block, 0, stream>>>(g)
               : gemm_narrow_n_kernel<false><<<grid, block, 0, stream>>>(g);
    return check_launch(what);
  }
  if (vec && g.M <= 16 && g.K > 0 && (g.rope_cs == nullptr || g.rope_hd % 2 == 0)) {
    const dim3 grid((unsigned)((g.N + 7) / 8), (unsigned)g.nprob), block(256);
    const bool epi = has_epi(g);
    if (g.M <= 4)
      epi ? gemm_rows_kernel<4, true><<<grid, block, 0, stream>>>(g)
          : gemm_rows_kernel<4, false><<<grid, block, 0, stream>>>(g);
    else
      epi ? gemm_rows_kernel<16, true><<<grid, block, 0, stream>>>(g)
          : gemm_rows_kernel<16, false><<<grid, block, 0, stream>>>(g);
    return check_launch(what);
  }
  // 256 x 128 tiles unless they would not fill one round of two workgroups
  // per CU: then 128 x 128 tiles spread the same work over twice as many
  // workgroups (16384 x 512 -> 512: 81 -> 78 us, same bits).
  const long long big_tiles_fwd = (long long)((g.M + 255) / 256) * ((g.N + 127) / 128) * g.nprob;
  if (fast && g.M >= 1024 && big_tiles_fwd >= 2 * num_cus()) {
    int rc = launch_tile<256, 128, 16, 4, 2, 2, false, false>(g, stream);
    if (rc) return rc;
  } else if (fast) {
    int rc = launch_tile<128, 128, 16, 2, 2, 2, false, false>(g, stream);
    if (rc) return rc;
  } else if (vec)
    has_epi(g) ? gemm_nt_kernel<true, true><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g)
               : gemm_nt_kernel<true, false><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g);
  else
    has_epi(g) ? gemm_nt_kernel<false, true><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g)
               : gemm_nt_kernel<false, false><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g);
  return check_launch(what);
}

// Attaches the split-K workspace of a weight-gradient launch (M = out, N =
// in, K = rows) to g; fails when the caller's workspace is smaller than
// splitk_plan asks for.
int attach_split(GemmArgs &g, void *workspace, size_t workspace_bytes, const char *what) {
  const SplitPlan sp = splitk_plan(g.M, g.N, g.K, g.nprob);
  if (sp.ksplit <= 1) return CDML_OK;
  if (!workspace || workspace_bytes < sp.bytes)
    return fail(CDML_E_INVALID, "%s: workspace of %zu bytes needed, %zu given", what, sp.bytes,
                workspace ? workspace_bytes : (size_t)0);
  if (!aligned16(workspace)) return fail(CDML_E_INVALID, "%s: workspace must be 16-byte aligned", what);
  g.ksplit = sp.ksplit;
  g.kchunk = sp.kchunk;
  g.small = sp.small ? 1 : 0;
  g.ws = static_cast<float *>(workspace);
  g.wsb = g.ws + (size_t)sp.ksplit * g.nprob * g.M * g.N;
  return CDML_OK;
}

}  // namespace
}  // namespace cdml

using namespace cdml;

extern "C" int cdml_linear_backward_workspace_size(int rows, int in_dim, int out_dim, size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_linear_backward_workspace_size: NULL pointer");
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_linear_backward_workspace_size: negative size");
  *bytes = splitk_plan(out_dim, in_dim, rows, 1).bytes;
  return CDML_OK;
}

extern "C" int cdml_backprop_qkv_workspace_size(int rows, int in_dim, int out_dim, size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_backprop_qkv_workspace_size: NULL pointer");
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_backprop_qkv_workspace_size: negative size");
  *bytes = splitk_plan(out_dim, in_dim, rows, 3).bytes;
  return CDML_OK;
}

extern "C" int cdml_project_qkv(const float *x, const float *wq, const float *bq, const float *wk,
                                const float *bk, const float *wv, const float *bv, float *q,
                                float *k, float *v, int rows, int in_dim, int out_dim,
                                cdml_stream stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_project_qkv: negative size");
  if (rows == 0 || out_dim == 0) return CDML_OK;
  if (!x || !wq || !wk || !wv || !q || !k || !v)
    return fail(CDML_E_INVALID, "cdml_project_qkv: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  // in_dim == 0: a K of zero leaves the accumulators at 0 and y = bias.
  GemmArgs g{};
  g.lda = in_dim;
  g.ldb = in_dim;
  g.ldc = out_dim;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 3;
  g.p[0] = {x, wq, bq, q, nullptr};
  g.p[1] = {x, wk, bk, k, nullptr};
  g.p[2] = {x, wv, bv, v, nullptr};
  g.act = CDML_ACT_NONE;
  return launch_gemm(g, false, false, as_hip(stream), "cdml_project_qkv");
}

extern "C" int cdml_project_qkv_rope(const float *x, const float *wq, const float *bq,
                                     const float *wk, const float *bk, const float *wv,
                                     const float *bv, float *q, float *k, float *v, int rows,
                                     int in_dim, int out_dim, int head_dim, const float *rope_cs,
                                     int n_pos, int pos_offset, int seg_len, cdml_stream stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0 || n_pos < 0 || pos_offset < 0 || seg_len < 0)
    return fail(CDML_E_INVALID, "cdml_project_qkv_rope: negative size");
  if (head_dim <= 0 || (head_dim & 1) || out_dim % head_dim)
    return fail(CDML_E_INVALID,
                "cdml_project_qkv_rope: head_dim must be even, positive and divide out_dim");
  if (rows == 0 || out_dim == 0) return CDML_OK;
  if (!x || !wq || !wk || !wv || !q || !k || !v || !rope_cs)
    return fail(CDML_E_INVALID, "cdml_project_qkv_rope: NULL pointer");
  if (reinterpret_cast<uintptr_t>(rope_cs) % 8)
    return fail(CDML_E_INVALID, "cdml_project_qkv_rope: rope_cs must be 8-byte aligned");
  const long long last_pos = (long long)pos_offset + (seg_len > 0 ? std::min(rows, seg_len) : rows) - 1;
  if (last_pos >= n_pos)
    return fail(CDML_E_INVALID, "cdml_project_qkv_rope: position %lld outside the %d-row table",
                last_pos, n_pos);
  int rc = ensure_device();
  if (rc) return rc;
  GemmArgs g{};
  g.lda = in_dim;
  g.ldb = in_dim;
  g.ldc = out_dim;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 3;
  g.p[0] = {x, wq, bq, q, nullptr};
  g.p[1] = {x, wk, bk, k, nullptr};
  g.p[2] = {x, wv, bv, v, nullptr};
  g.act = CDML_ACT_NONE;
  g.rope_cs = reinterpret_cast<const float2 *>(rope_cs);
  g.rope_hd = head_dim;
  g.rope_npos = n_pos;
  g.rope_pos0 = pos_offset;
  g.rope_seg = seg_len;
  return launch_gemm(g, false, false, as_hip(stream), "cdml_project_qkv_rope");
}

extern "C" int cdml_linear(const float *x, int ldx, const float *w, const float *b, float *y,
                           int ldy, int rows, int in_dim, int out_dim, int activation,
                           cdml_stream stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_linear: negative size");
  if (activation < CDML_ACT_NONE || activation > CDML_ACT_SWISH)
    return fail(CDML_E_INVALID, "cdml_linear: unknown activation %d", activation);
  if (rows == 0 || out_dim == 0) return CDML_OK;
  if (!x || !w || !y) return fail(CDML_E_INVALID, "cdml_linear: NULL pointer");
  if (ldx < in_dim || ldy < out_dim)
    return fail(CDML_E_INVALID, "cdml_linear: row stride smaller than the row");
  int rc = ensure_device();
  if (rc) return rc;
  GemmArgs g{};
  g.lda = ldx;
  g.ldb = in_dim;
  g.ldc = ldy;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 1;
  g.p[0] = {x, w, b, y, nullptr};
  g.act = activation;
  return launch_gemm(g, false, false, as_hip(stream), "cdml_linear");
}

namespace {

// cdml_linear_backward with the epilogue options of the input gradient:
// dx = (dY W) * act'(dz) + add (dz / add NULL: not applied; both use row
// stride lddx), or dx += dY W with accumulate_dx.
int linear_backward_impl(const float *x, int ldx, const float *dy, int lddy, const float *w,
                         const float *dz, int dact, const float *add, float *dx, int lddx,
                         float *wgrad, float *bgrad, int rows, int in_dim, int out_dim,
                         int accumulate_dx, void *workspace, size_t workspace_bytes,
                         cdml_stream stream, const char *what) {
  if (rows < 0 || in_dim < 0 || out_dim < 0) return fail(CDML_E_INVALID, "%s: negative size", what);
  if (lddy < out_dim || (dx && lddx < in_dim) || (wgrad && ldx < in_dim))
    return fail(CDML_E_INVALID, "%s: row stride smaller than the row", what);
  if (rows == 0) return CDML_OK;
  if (!dy || (dx && !w) || (wgrad && !x)) return fail(CDML_E_INVALID, "%s: NULL pointer", what);
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  if (dx && in_dim > 0) {
    // dX (+)= dY W: opA = dY [rows, out], opB = W read as [out, in]
    GemmArgs g{};
    g.lda = lddy;
    g.ldb = in_dim;
    g.ldc = lddx;
    g.M = rows;
    g.N = in_dim;
    g.K = out_dim;
    g.nprob = 1;
    g.p[0] = {dy, w, nullptr, dx, nullptr};
    g.beta = accumulate_dx ? 1 : 0;
    g.dz = dz;
    g.lddz = lddx;
    g.dact = dact;
    g.add = add;
    g.ldadd = lddx;
    rc = launch_gemm(g, false, true, st, what);
    if (rc) return rc;
  }
  if ((wgrad || bgrad) && out_dim > 0) {
    // W_grad += dY^T X: opA = dY read as [out, rows], opB = X read as
    // [rows, in]; the bias gradient rides on the staging of opA.
    GemmArgs g{};
    g.lda = lddy;
    g.ldb = ldx;
    g.ldc = in_dim;
    g.M = out_dim;
    g.N = in_dim;
    g.K = rows;
    g.nprob = 1;
    g.p[0] = {dy, x, nullptr, wgrad, bgrad};
    g.beta = 1;
    if (wgrad && in_dim > 0) {
      rc = attach_split(g, workspace, workspace_bytes, what);
      if (rc) return rc;
      rc = launch_gemm(g, true, true, st, what);
    } else if (bgrad) {
      op_rowsum_kernel<true><<<dim3((out_dim + 255) / 256, 1), dim3(256), 0, st>>>(g);
      rc = check_launch(what);
    }
    if (rc) return rc;
  }
  return CDML_OK;
}

}  // namespace

extern "C" int cdml_linear_backward(const float *x, int ldx, const float *dy, int lddy,
                                    const float *w, float *dx, int lddx, float *wgrad,
                                    float *bgrad, int rows, int in_dim, int out_dim,
                                    int accumulate_dx, void *workspace, size_t workspace_bytes,
                                    cdml_stream stream) {
  return linear_backward_impl(x, ldx, dy, lddy, w, nullptr, CDML_ACT_NONE, nullptr, dx, lddx, wgrad,
                              bgrad, rows, in_dim, out_dim, accumulate_dx, workspace, workspace_bytes,
                              stream, "cdml_linear_backward");
}

extern "C" int cdml_linear_backward_act(const float *x, int ldx, const float *dy, int lddy,
                                        const float *w, const float *dz, int activation,
                                        const float *add, float *dx, int lddx, float *wgrad,
                                        float *bgrad, int rows, int in_dim, int out_dim,
                                        void *workspace, size_t workspace_bytes,
                                        cdml_stream stream) {
  const int base = activation & ~CDML_ACT_FROM_OUTPUT;
  if (base < CDML_ACT_NONE || base > CDML_ACT_SWISH)
    return fail(CDML_E_INVALID, "cdml_linear_backward_act: unknown activation %d", activation);
  const bool from_out = (activation & CDML_ACT_FROM_OUTPUT) != 0;
  if (from_out && base != CDML_ACT_RELU && base != CDML_ACT_LEAKYRELU)
    return fail(CDML_E_INVALID, "cdml_linear_backward_act: CDML_ACT_FROM_OUTPUT needs ReLU or leaky ReLU");
  const int dact = from_out && base == CDML_ACT_RELU ? kDerivReluOut : base;
  return linear_backward_impl(x, ldx, dy, lddy, w, dz, dact, add, dx, lddx, wgrad, bgrad,
                              rows, in_dim, out_dim, 0, workspace, workspace_bytes, stream,
                              "cdml_linear_backward_act");
}

extern "C" int cdml_matmul(const float *a, int lda, const float *b, int ldb, float *c, int ldc, int m,
                           int k, int n, cdml_stream stream) {
  if (m < 0 || k < 0 || n < 0) return fail(CDML_E_INVALID, "cdml_matmul: negative size");
  if (m == 0 || n == 0) return CDML_OK;
  if (!a || !b || !c) return fail(CDML_E_INVALID, "cdml_matmul: NULL pointer");
  if (lda < k || ldb < n || ldc < n) return fail(CDML_E_INVALID, "cdml_matmul: row stride smaller than the row");
  int rc = ensure_device();
  if (rc) return rc;
  GemmArgs g{};  // k == 0: the generic kernel stores zeros
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.M = m;
  g.N = n;
  g.K = k;
  g.nprob = 1;
  g.p[0] = {a, b, nullptr, c, nullptr};
  return launch_gemm(g, false, true, as_hip(stream), "cdml_matmul");
}

extern "C" int cdml_linear_preact(const float *x, int ldx, const float *w, const float *b, float *z,
                                  float *y, int ldy, int rows, int in_dim, int out_dim,
                                  int activation, cdml_stream stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_linear_preact: negative size");
  if (activation < CDML_ACT_NONE || activation > CDML_ACT_SWISH)
    return fail(CDML_E_INVALID, "cdml_linear_preact: unknown activation %d", activation);
  if (!z && activation != CDML_ACT_RELU && activation != CDML_ACT_LEAKYRELU)
    return fail(CDML_E_INVALID, "cdml_linear_preact: z may be NULL only with ReLU or leaky ReLU");
  if (rows == 0 || out_dim == 0) return CDML_OK;
  if (!x || !w || !y) return fail(CDML_E_INVALID, "cdml_linear_preact: NULL pointer");
  if (ldx < in_dim || ldy < out_dim)
    return fail(CDML_E_INVALID, "cdml_linear_preact: row stride smaller than the row");
  int rc = ensure_device();
  if (rc) return rc;
  GemmArgs g{};
  g.lda = ldx;
  g.ldb = in_dim;
  g.ldc = ldy;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 1;
  g.p[0] = {x, w, b, y, nullptr};
  g.act = !z && activation == CDML_ACT_RELU ? kActReluMarked : activation;
  g.pre = z;
  g.ldpre = ldy;
  return launch_gemm(g, false, false, as_hip(stream), "cdml_linear_preact");
}

extern "C" int cdml_backprop_qkv(const float *x, const float *dq, const float *dk, const float *dv,
                                 const float *wq, const float *wk, const float *wv, float *wq_grad,
                                 float *bq_grad, float *wk_grad, float *bk_grad, float *wv_grad,
                                 float *bv_grad, float *dx, int rows, int in_dim, int out_dim,
                                 void *workspace, size_t workspace_bytes, cdml_stream stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0)
    return fail(CDML_E_INVALID, "cdml_backprop_qkv: negative size");
  if (rows == 0) return CDML_OK;
  if (!x || !dq || !dk || !dv || !wq || !wk || !wv || !wq_grad || !bq_grad || !wk_grad ||
      !bk_grad || !wv_grad || !bv_grad || !dx)
    return fail(CDML_E_INVALID, "cdml_backprop_qkv: NULL pointer");
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = as_hip(stream);
  if (out_dim > 0) {
    // W*_grad += d*^T X and b*_grad += column sums of d*, three problems in
    // one launch
    GemmArgs g{};
    g.lda = out_dim;
    g.ldb = in_dim;
    g.ldc = in_dim;
    g.M = out_dim;
    g.N = in_dim;
    g.K = rows;
    g.nprob = 3;
    g.p[0] = {dq, x, nullptr, wq_grad, bq_grad};
    g.p[1] = {dk, x, nullptr, wk_grad, bk_grad};
    g.p[2] = {dv, x, nullptr, wv_grad, bv_grad};
    g.beta = 1;
    if (in_dim > 0) {
      rc = attach_split(g, workspace, workspace_bytes, "cdml_backprop_qkv");
      if (rc) return rc;
      rc = launch_gemm(g, true, true, st, "cdml_backprop_qkv (weight gradients)");
    } else {
      op_rowsum_kernel<true><<<dim3((out_dim + 255) / 256, 3), dim3(256), 0, st>>>(g);
      rc = check_launch("cdml_backprop_qkv (bias gradients)");
    }
    if (rc) return rc;
  }
  if (in_dim > 0) {
    // dX = dQ WQ + dK WK + dV WV: one product over K = 3 * out_dim when the
    // tiled kernel can stage all three operand pairs (the k-loop switches
    // source at each third), else the three products accumulated in turn
    // (out_dim == 0: dX = 0)
    const float *d[3] = {dq, dk, dv};
    const float *w[3] = {wq, wk, wv};
    bool fused = out_dim > 0 && out_dim % 16 == 0 && (long long)3 * out_dim <= INT32_MAX;
    for (int s = 0; fused && s < 3; ++s)
      fused = stage_ok(d[s], rows, out_dim, false, 16) && stage_ok(w[s], in_dim, in_dim, true, 16);
    if (fused) {
      GemmArgs g{};
      g.lda = out_dim;
      g.ldb = in_dim;
      g.ldc = in_dim;
      g.M = rows;
      g.N = in_dim;
      g.K = 3 * out_dim;
      g.nprob = 1;
      for (int s = 0; s < 3; ++s) g.p[s] = {d[s], w[s], nullptr, dx, nullptr};
      g.kseg = out_dim / 16;
      return launch_gemm(g, false, true, st, "cdml_backprop_qkv (input gradient)");
    }
    for (int s = 0; s < 3; ++s) {
      GemmArgs g{};
      g.lda = out_dim;
      g.ldb = in_dim;
      g.ldc = in_dim;
      g.M = rows;
      g.N = in_dim;
      g.K = out_dim;
      g.nprob = 1;
      g.p[0] = {d[s], w[s], nullptr, dx, nullptr};
      g.beta = s > 0;
      rc = launch_gemm(g, false, true, st, "cdml_backprop_qkv (input gradient)");
      if (rc) return rc;
    }
  }
  return CDML_OK;
}
