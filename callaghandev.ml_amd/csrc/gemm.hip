// fp32 MFMA GEMM for the projections of the attention path:
//   C[m, n] = act(sum_k A[m, k] * W[n, k] + bias[n])
// A is the activation [M, K] (row stride lda), W the weight [N, K] ([out, in],
// the reference's layout), C the output [M, N] (row stride ldc).  Up to three
// problems that share A (the fused Q/K/V projection) run in one launch.
//
// Tiling for gfx950: a 256-thread workgroup computes a 128x128 tile of C; each
// of its four waves owns a 64x64 quadrant as 2x2 blocks of
// v_mfma_f32_32x32x2_f32.  K advances in steps of 32 through double-buffered
// LDS tiles (row stride 36 floats); every lane fetches its A and B operands as
// 16-byte LDS reads that feed four MFMAs each.  The reduction index k is
// visited in the permuted order kappa(s, h) = 8*(s/4) + 4*h + s%4 on both
// operands, which leaves the sum unchanged.
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
  const float *w;
  const float *bias;
  float *c;
};

struct GemmArgs {
  const float *a;
  GemmProblem p[3];
  int lda, ldc;
  int M, N, K;
  int nprob;
  int tiles_m, tiles_n;  // tiles_n counts the tiles of one problem
  int total, padded;
  int act;
  // Rotary position embedding applied to problems 0 and 1 (Q and K) in the
  // epilogue when rope_cs is set: rope_cs[pos * rope_hd / 2 + p] holds
  // (cos, sin) of position pos for pair p; row m has position
  // rope_pos0 + (rope_seg > 0 ? m % rope_seg : m), below rope_npos.
  const float2 *rope_cs;
  int rope_hd, rope_npos, rope_pos0, rope_seg;
};

// Epilogue of both GEMM kernels with the rotary embedding of
// AccelerationCPU.cs:4947-4975 folded in.  A lane holds column n of rows
// mrow0 + 32 i + 8 (r / 4) + 4 hf + r % 4, so the pair partner of column n
// (n ^ 1; head dims are even) sits in lane li ^ 1 of the same register: one
// lane swap gives each lane both halves of its pair.  The swap runs in every
// lane; only the store is predicated.
template <int BI, int BJ>
__device__ __forceinline__ void store_rope(const GemmArgs &args, const GemmProblem &P,
                                           const floatx16 (&acc)[BI][BJ], int mrow0, int ncol0,
                                           int li, int hf) {
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
#pragma unroll
  for (int i = 0; i < BI; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mrow0 + i * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
      int pos = args.rope_pos0 + (args.rope_seg > 0 ? m % args.rope_seg : m);
      pos = min(pos, args.rope_npos - 1);  // rows past M are never stored
      const float2 *cs = args.rope_cs + (size_t)pos * pairs;
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const float y = acc[i][j][r] + bias[j];
        const float yp = __shfl_xor(y, 1);
        const float2 t = cs[pidx[j]];
        const float out = odd[j] ? yp * t.y + y * t.x : y * t.x - yp * t.y;
        if (m < args.M && n[j] < args.N) P.c[(size_t)m * args.ldc + n[j]] = out;
      }
    }
  }
}

__device__ __forceinline__ float activate(float x, int act) {
  switch (act) {
    case CDML_ACT_SIGMOID:
      return x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x));
    case CDML_ACT_TANH:
      return tanhf(x);
    case CDML_ACT_RELU:
      return x > 0.f ? x : 0.f;
    case CDML_ACT_LEAKYRELU:
      return x > 0.f ? x : 0.01f * x;
    case CDML_ACT_SWISH: {
      float s = x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x));
      return x * s;
    }
    default:
      return x;
  }
}

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

template <bool VEC>
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
  sa.load(args.a, args.lda, m0, M, 0, K);
  sb.load(P.w, K, n0, N, 0, K);
  sa.store(As[0]);
  sb.store(Bs[0]);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      sa.load(args.a, args.lda, m0, M, (kt + 1) * BK, K);
      sb.load(P.w, K, n0, N, (kt + 1) * BK, K);
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
        if (m < M) P.c[(size_t)m * args.ldc + n] = activate(acc[i][j][r] + bias, args.act);
      }
    }
  }
}

// Tiled fast path (K % BKK == 0, 16-byte aligned rows, element offsets
// below 2^32).  A workgroup of WM x WN waves computes a TM x TN tile of C,
// each wave a (TM/WM) x (TN/WN) block of 32x32 MFMA tiles.  K advances by BKK
// through double-buffered LDS (row pitch BKK + 4 floats).  Every thread's
// staging rows are fixed for the whole K loop (rows past M or N are clamped
// to the last row: they feed only accumulators that are never stored), so a
// k-tile load is the wave-uniform base plus precomputed 32-bit offsets, with
// no predication.  The LDS operands of group u + 1 are read while the MFMAs of
// group u run, and the k-tile after next is fetched while the current one is
// consumed.  Measured on MI355X, high occupancy (four waves per SIMD with two
// 512-thread workgroups per CU) hides latency better than deeper register
// blocking.
template <int TM, int TN, int BKK, int WM, int WN, int MINB, int ACT>
__global__ void __launch_bounds__(64 * WM * WN, MINB) gemm_tile_kernel(const GemmArgs args) {
  constexpr int NT = 64 * WM * WN;
  constexpr int LD = BKK + 4;
  constexpr int F4R = BKK / 4;   // float4 per row of a k-tile
  constexpr int RPP = NT / F4R;  // rows per staging pass
  constexpr int NA = TM / RPP, NB = TN / RPP;
  constexpr int BI = TM / WM / 32, BJ = TN / WN / 32;
  static_assert(NA >= 1 && NB >= 1 && BI >= 1 && BJ >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float As[2][TM][LD];
  __shared__ __attribute__((aligned(16))) float Bs[2][TN][LD];

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
  const int m0 = tm * TM, n0 = tn * TN;
  const int M = args.M, N = args.N, K = args.K;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, hf = lane >> 5;

  const int srow = t / F4R, scol = (t % F4R) * 4;
  uint32_t aoff[NA], boff[NB];
#pragma unroll
  for (int i = 0; i < NA; ++i) aoff[i] = (uint32_t)min(m0 + srow + RPP * i, M - 1) * (uint32_t)args.lda + scol;
#pragma unroll
  for (int i = 0; i < NB; ++i) boff[i] = (uint32_t)min(n0 + srow + RPP * i, N - 1) * (uint32_t)K + scol;
  vf4 ra[NA], rb[NB];
  floatx16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int nk = K / BKK;
  const float *__restrict__ A = args.a;
  const float *__restrict__ W = P.w;

  // k-tile 0 -> LDS, k-tile 1 -> registers
#pragma unroll
  for (int i = 0; i < NA; ++i) ra[i] = *reinterpret_cast<const vf4 *>(A + aoff[i]);
#pragma unroll
  for (int i = 0; i < NB; ++i) rb[i] = *reinterpret_cast<const vf4 *>(W + boff[i]);
#pragma unroll
  for (int i = 0; i < NA; ++i) *reinterpret_cast<vf4 *>(&As[0][srow + RPP * i][scol]) = ra[i];
#pragma unroll
  for (int i = 0; i < NB; ++i) *reinterpret_cast<vf4 *>(&Bs[0][srow + RPP * i][scol]) = rb[i];
  {
    const int k1 = min(BKK, (nk - 1) * BKK);
#pragma unroll
    for (int i = 0; i < NA; ++i) ra[i] = *reinterpret_cast<const vf4 *>(A + k1 + aoff[i]);
#pragma unroll
    for (int i = 0; i < NB; ++i) rb[i] = *reinterpret_cast<const vf4 *>(W + k1 + boff[i]);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const float(*as)[LD] = &As[cur][wm * (TM / WM) + li];
    const float(*bs)[LD] = &Bs[cur][wn * (TN / WN) + li];
    vf4 a4[BI], b4[BJ];
#pragma unroll
    for (int i = 0; i < BI; ++i) a4[i] = *reinterpret_cast<const vf4 *>(&as[i * 32][hf * 4]);
#pragma unroll
    for (int j = 0; j < BJ; ++j) b4[j] = *reinterpret_cast<const vf4 *>(&bs[j * 32][hf * 4]);
#pragma unroll
    for (int u = 0; u < BKK / 8; ++u) {
      vf4 an[BI], bn[BJ];
      if (u + 1 < BKK / 8) {
#pragma unroll
        for (int i = 0; i < BI; ++i) an[i] = *reinterpret_cast<const vf4 *>(&as[i * 32][(u + 1) * 8 + hf * 4]);
#pragma unroll
        for (int j = 0; j < BJ; ++j) bn[j] = *reinterpret_cast<const vf4 *>(&bs[j * 32][(u + 1) * 8 + hf * 4]);
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
#pragma unroll
    for (int i = 0; i < NA; ++i) *reinterpret_cast<vf4 *>(&As[cur ^ 1][srow + RPP * i][scol]) = ra[i];
#pragma unroll
    for (int i = 0; i < NB; ++i) *reinterpret_cast<vf4 *>(&Bs[cur ^ 1][srow + RPP * i][scol]) = rb[i];
    const int k2 = min((kt + 2) * BKK, (nk - 1) * BKK);
#pragma unroll
    for (int i = 0; i < NA; ++i) ra[i] = *reinterpret_cast<const vf4 *>(A + k2 + aoff[i]);
#pragma unroll
    for (int i = 0; i < NB; ++i) rb[i] = *reinterpret_cast<const vf4 *>(W + k2 + boff[i]);
    __syncthreads();
  }

  if constexpr (ACT == kActRope) {
    if (prob < 2) {
      store_rope<BI, BJ>(args, P, acc, m0 + wm * (TM / WM), n0 + wn * (TN / WN), li, hf);
      return;
    }
  }
  // Epilogue: D[i][j] of block (bi, bj) sits at row 8*(r/4) + 4*hf + r%4,
  // column li; 32 lanes store 32 consecutive columns of one row.
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
        if (m < M) P.c[(size_t)m * args.ldc + n] = activate(acc[i][j][r] + bias, ACT);
      }
    }
  }
}

// Two tile configurations: 256 x 128 with eight waves for M >= 1024, and
// 128 x 128 with four waves for smaller M (decode rows, short sequences).
template <int TM, int TN, int BKK, int WM, int WN, int MINB>
int launch_tile(GemmArgs g, hipStream_t stream) {
  g.tiles_m = (g.M + TM - 1) / TM;
  g.tiles_n = (g.N + TN - 1) / TN;
  g.total = g.tiles_m * g.tiles_n * g.nprob;
  g.padded = pad_to_xcd(g.total);
  const dim3 grid(g.padded), block(64 * WM * WN);
  if (g.rope_cs) {
    gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, kActRope><<<grid, block, 0, stream>>>(g);
    return CDML_OK;
  }
  switch (g.act) {
    case CDML_ACT_NONE: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_NONE><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_SIGMOID: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_SIGMOID><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_TANH: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_TANH><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_RELU: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_RELU><<<grid, block, 0, stream>>>(g); break;
    case CDML_ACT_LEAKYRELU: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_LEAKYRELU><<<grid, block, 0, stream>>>(g); break;
    default: gemm_tile_kernel<TM, TN, BKK, WM, WN, MINB, CDML_ACT_SWISH><<<grid, block, 0, stream>>>(g); break;
  }
  return CDML_OK;
}

int launch_gemm(GemmArgs &g, hipStream_t stream, const char *what) {
  if (g.M == 0 || g.N == 0) return CDML_OK;
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BN - 1) / BN;
  g.total = g.tiles_m * g.tiles_n * g.nprob;
  g.padded = pad_to_xcd(g.total);
  bool vec = (g.K % 4 == 0) && (g.lda % 4 == 0) && aligned16(g.a);
  for (int i = 0; i < g.nprob; ++i) vec = vec && aligned16(g.p[i].w);
  const bool fast = vec && g.K % 16 == 0 && g.K > 0 &&
                    (unsigned long long)g.M * g.lda < (1ull << 32) &&
                    (unsigned long long)g.N * g.K < (1ull << 32);
  if (fast && g.M >= 1024) {
    int rc = launch_tile<256, 128, 16, 4, 2, 2>(g, stream);
    if (rc) return rc;
  } else if (fast) {
    int rc = launch_tile<128, 128, 16, 2, 2, 2>(g, stream);
    if (rc) return rc;
  } else if (vec)
    gemm_nt_kernel<true><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g);
  else
    gemm_nt_kernel<false><<<dim3(g.padded), dim3(NTHREADS), 0, stream>>>(g);
  return check_launch(what);
}

}  // namespace
}  // namespace cdml

using namespace cdml;

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
  if (in_dim == 0) {
    // y = bias only; a K of zero leaves the accumulators at 0.
  }
  GemmArgs g{};
  g.a = x;
  g.lda = in_dim;
  g.ldc = out_dim;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 3;
  g.p[0] = {wq, bq, q};
  g.p[1] = {wk, bk, k};
  g.p[2] = {wv, bv, v};
  g.act = CDML_ACT_NONE;
  return launch_gemm(g, as_hip(stream), "cdml_project_qkv");
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
  g.a = x;
  g.lda = in_dim;
  g.ldc = out_dim;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 3;
  g.p[0] = {wq, bq, q};
  g.p[1] = {wk, bk, k};
  g.p[2] = {wv, bv, v};
  g.act = CDML_ACT_NONE;
  g.rope_cs = reinterpret_cast<const float2 *>(rope_cs);
  g.rope_hd = head_dim;
  g.rope_npos = n_pos;
  g.rope_pos0 = pos_offset;
  g.rope_seg = seg_len;
  return launch_gemm(g, as_hip(stream), "cdml_project_qkv_rope");
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
  g.a = x;
  g.lda = ldx;
  g.ldc = ldy;
  g.M = rows;
  g.N = out_dim;
  g.K = in_dim;
  g.nprob = 1;
  g.p[0] = {w, b, y};
  g.act = activation;
  return launch_gemm(g, as_hip(stream), "cdml_linear");
}
