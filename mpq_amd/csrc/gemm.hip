// fp32 MFMA GEMM for the rank-space contractions of the VAMP / CD path.
//
//   P[s] = A[:, Ks] * op(B)[Ks, :]        (split-K partials, s = 0..splits-1)
//   C    = alpha * sum_s P[s] + beta * C  (deterministic split order)
//
// A is M x K row-major (lda).  op(B)(k, n) is B[k*ldb + n] (trans_b = 0),
// B[n*ldb + k] (trans_b = 1, e.g. V^T from V), or B[rows[k]*ldb + n] (row gather,
// used by the CD Schur update H[order[window], :]).
//
// Tiling for gfx950: 256 threads = 4 wave64s; work-group tile BM x BN, wave tile
// WM x WN built from v_mfma_f32_32x32x2_f32 (full fp32 precision).  Tiles are
// staged through LDS as [k][m] / [k][n] (each MFMA operand read is 32 consecutive
// floats), double-buffered.  Interior tiles (the rank-space products always are) run
// gemm_f32_full_kernel: no bounds checks and two K slabs of global loads in flight;
// ragged or gathered products run gemm_f32_kernel with one slab of register prefetch.
#include "gemm.h"
#include "x6_split.h"

namespace mpq {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 16;  // K slab of the default configurations (k_per_split is a multiple of 32)
constexpr int kThreads = 256;

template <int BM, int BN, int WM, int WN, bool TRANS_B, bool GATHER_B, int kBK = 16, bool PRE_C = false>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmParams p) {
  constexpr int WAVES_N = BN / WN;
  constexpr int MI = WM / 32;
  constexpr int NI = WN / 32;
  constexpr int PAD = 4;
  constexpr int LDA_S = BM + PAD;
  constexpr int LDB_S = BN + PAD;
  // per-thread loads per K slab
  constexpr int A_F4 = BM * kBK / 4 / kThreads;
  constexpr int B_F4 = BN * kBK / 4 / kThreads;
  static_assert(A_F4 >= 1 && B_F4 >= 1, "tile too small for 256 threads");

  __shared__ float As[2][kBK][LDA_S];
  __shared__ float Bs[2][kBK][LDB_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM;
  const int wn0 = (wave % WAVES_N) * WN;

  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  if (p.lower_only && n0 >= m0 + BM + p.upper_band) return;  // uniform, before any barrier
  const int split = blockIdx.z;
  const int32_t* b_rows = p.b_rows;
  if (GATHER_B && p.b_rows_group > 0) b_rows += (m0 / p.b_rows_group) * p.b_rows_group_stride;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  int64_t kend = kbeg + p.k_per_split;
  if (kend > p.K) kend = p.K;

  floatx16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // PRE_C (axpby epilogue with beta != 0): this lane's C entries are loaded before the K loop, so
  // their latency overlaps the MFMAs instead of stalling the epilogue.  Rows/columns outside C
  // read a clamped in-range entry (never used) so the loads need no branches.
  float cpre[PRE_C ? MI : 1][PRE_C ? NI : 1][PRE_C ? 16 : 1];
  if constexpr (PRE_C) {
    const int col = lane & 31;
    const int rbase = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int64_t gn = min(n0 + wn0 + j * 32 + col, p.N - 1);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t gm = min(m0 + wm0 + i * 32 + (v >> 2) * 8 + rbase + (v & 3), p.M - 1);
          cpre[i][j][v] = p.C[gm * p.ldc + gn];
        }
      }
  }

  float4 ra[A_F4];
  float4 rb[B_F4];

  // A slab: element (m, k) = A[(m0+m)*lda + k0 + k]; thread t loads float4 along k.
  auto load_a = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int t = tid + i * kThreads;
      const int m = t / (kBK / 4);
      const int kq = (t % (kBK / 4)) * 4;
      const int64_t gm = m0 + m;
      const int64_t gk = k0 + kq;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (gm < p.M) {
        const float* src = p.A + gm * p.lda + gk;
        if (gk + 3 < kend && p.a_vec4) {
          v = *reinterpret_cast<const float4*>(src);
        } else {
          if (gk + 0 < kend) v.x = src[0];
          if (gk + 1 < kend) v.y = src[1];
          if (gk + 2 < kend) v.z = src[2];
          if (gk + 3 < kend) v.w = src[3];
        }
      }
      ra[i] = v;
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int t = tid + i * kThreads;
      const int m = t / (kBK / 4);
      const int kq = (t % (kBK / 4)) * 4;
      As[buf][kq + 0][m] = ra[i].x;
      As[buf][kq + 1][m] = ra[i].y;
      As[buf][kq + 2][m] = ra[i].z;
      As[buf][kq + 3][m] = ra[i].w;
    }
  };
  auto load_b = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int t = tid + i * kThreads;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (!TRANS_B) {
        const int k = t / (BN / 4);
        const int nq = (t % (BN / 4)) * 4;
        const int64_t gk = k0 + k;
        const int64_t gn = n0 + nq;
        if (gk < kend) {
          int64_t row = gk;
          if constexpr (GATHER_B) row = b_rows[gk];
          const float* src = p.B + row * p.ldb + gn;
          if (gn + 3 < p.N && p.b_vec4) {
            v = *reinterpret_cast<const float4*>(src);
          } else {
            if (gn + 0 < p.N) v.x = src[0];
            if (gn + 1 < p.N) v.y = src[1];
            if (gn + 2 < p.N) v.z = src[2];
            if (gn + 3 < p.N) v.w = src[3];
          }
        }
      } else {
        const int n = t / (kBK / 4);
        const int kq = (t % (kBK / 4)) * 4;
        const int64_t gn = n0 + n;
        const int64_t gk = k0 + kq;
        if (gn < p.N) {
          const float* src = p.B + gn * p.ldb + gk;
          if (gk + 3 < kend && p.b_vec4) {
            v = *reinterpret_cast<const float4*>(src);
          } else {
            if (gk + 0 < kend) v.x = src[0];
            if (gk + 1 < kend) v.y = src[1];
            if (gk + 2 < kend) v.z = src[2];
            if (gk + 3 < kend) v.w = src[3];
          }
        }
      }
      rb[i] = v;
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int t = tid + i * kThreads;
      if constexpr (!TRANS_B) {
        const int k = t / (BN / 4);
        const int nq = (t % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[buf][k][nq]) = rb[i];
      } else {
        const int n = t / (kBK / 4);
        const int kq = (t % (kBK / 4)) * 4;
        Bs[buf][kq + 0][n] = rb[i].x;
        Bs[buf][kq + 1][n] = rb[i].y;
        Bs[buf][kq + 2][n] = rb[i].z;
        Bs[buf][kq + 3][n] = rb[i].w;
      }
    }
  };

  const int64_t nslab = (kend - kbeg + kBK - 1) / kBK;
  if (nslab > 0) {
    load_a(kbeg);
    load_b(kbeg);
    store_a(0);
    store_b(0);
    __syncthreads();
    for (int64_t s = 0; s < nslab; ++s) {
      const int buf = (int)(s & 1);
      if (s + 1 < nslab) {
        load_a(kbeg + (s + 1) * kBK);
        load_b(kbeg + (s + 1) * kBK);
      }
      const int kl = lane >> 5;  // operand k row within a 2-step
      const int ml = lane & 31;
#pragma unroll
      for (int kk = 0; kk < kBK; kk += 2) {
        float a[MI], b[NI];
#pragma unroll
        for (int i = 0; i < MI; ++i) a[i] = As[buf][kk + kl][wm0 + i * 32 + ml];
#pragma unroll
        for (int j = 0; j < NI; ++j) b[j] = Bs[buf][kk + kl][wn0 + j * 32 + ml];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      if (s + 1 < nslab) {
        store_a(buf ^ 1);
        store_b(buf ^ 1);
      }
      __syncthreads();
    }
  }

  // Epilogue: lane l, accumulator v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32.
  const int col = lane & 31;
  const int rbase = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int64_t gn = n0 + wn0 + j * 32 + col;
      if (gn >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t gm = m0 + wm0 + i * 32 + (v >> 2) * 8 + rbase + (v & 3);
        if (gm >= p.M) continue;
        const float val = acc[i][j][v];
        if (p.mode == kGemmPartials) {
          p.C[(int64_t)split * p.split_stride + gm * p.ldc + gn] = val;
        } else {  // kGemmAxpby, single split: C = alpha*acc + beta*C
          float* dst = p.C + gm * p.ldc + gn;
          if constexpr (PRE_C) {
            *dst = p.alpha * val + p.beta * cpre[i][j][v];
          } else {
            *dst = p.beta == 0.f ? p.alpha * val : p.alpha * val + p.beta * *dst;
          }
        }
      }
    }
  }
}

// Deterministic split-K reduction: C = alpha * sum_s P[s] + beta * C.
__global__ void splitk_reduce_kernel(const float* __restrict__ P, int splits, int64_t split_stride,
                                     int64_t M, int64_t N, float* __restrict__ C, int64_t ldc,
                                     float alpha, float beta) {
  const int64_t total = M * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / N, n = e % N;
    const float acc = sum_splits(P, splits, split_stride, m * N + n);
    float* dst = C + m * ldc + n;
    *dst = beta == 0.f ? alpha * acc : alpha * acc + beta * *dst;
  }
}

// Interior-tile variant: every M/N tile and K slab is in range and 16-byte aligned (checked by
// the host), no row gather.  Two K slabs of global loads are kept in flight (register sets R0/R1,
// the loop is unrolled by two so both sets are static), and a slab's LDS operands are all read
// before its MFMA chain, so each slab waits once for LDS and once for global memory.
template <int BM, int BN, int WM, int WN, bool TRANS_B, int HOIST = 8, bool PRE_C = false, bool GATHER_B = false>
__global__ __launch_bounds__(kThreads) void gemm_f32_full_kernel(GemmParams p) {
  static_assert(!(GATHER_B && TRANS_B), "row gather needs a row-major K x N B");
  constexpr int BK = 16;
  constexpr int WAVES_N = BN / WN;
  constexpr int MI = WM / 32;
  constexpr int NI = WN / 32;
  constexpr int LDA_S = BM + 4;
  constexpr int LDB_S = BN + 4;
  constexpr int A_F4 = BM * BK / 4 / kThreads;
  constexpr int B_F4 = BN * BK / 4 / kThreads;
  static_assert(A_F4 >= 1 && B_F4 >= 1, "tile too small for 256 threads");

  __shared__ float As[2][BK][LDA_S];
  __shared__ float Bs[2][BK][LDB_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM;
  const int wn0 = (wave % WAVES_N) * WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  if (p.lower_only && n0 >= m0 + BM + p.upper_band) return;  // uniform, before any barrier
  const int split = blockIdx.z;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  const int64_t nslab = p.k_per_split / BK;

  // per-thread global source pointers of the first slab (advanced by BK per slab)
  const float* asrc[A_F4];
  const float* bsrc[B_F4];
#pragma unroll
  for (int i = 0; i < A_F4; ++i) {
    const int t = tid + i * kThreads;
    asrc[i] = p.A + (m0 + t / (BK / 4)) * p.lda + kbeg + (t % (BK / 4)) * 4;
  }
#pragma unroll
  for (int i = 0; i < B_F4; ++i) {
    const int t = tid + i * kThreads;
    if constexpr (!TRANS_B) {
      bsrc[i] = p.B + (kbeg + t / (BN / 4)) * p.ldb + n0 + (t % (BN / 4)) * 4;
    } else {
      bsrc[i] = p.B + (n0 + t / (BK / 4)) * p.ldb + kbeg + (t % (BK / 4)) * 4;
    }
  }
  const int64_t b_step = TRANS_B ? BK : BK * p.ldb;
  // GATHER_B: K row k of B is B[b_rows[k]] (per M tile group as in gemm_f32_kernel); each thread
  // reads its slab row index in the same two-slabs-ahead prefetch as the data
  const int32_t* b_rows = p.b_rows;
  if (GATHER_B && p.b_rows_group > 0) b_rows += (m0 / p.b_rows_group) * p.b_rows_group_stride;

  float4 ra0[A_F4], rb0[B_F4], ra1[A_F4], rb1[B_F4];
  auto gload = [&](float4 (&ra)[A_F4], float4 (&rb)[B_F4], int64_t s) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) ra[i] = *reinterpret_cast<const float4*>(asrc[i] + s * BK);
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      if constexpr (GATHER_B) {
        const int t = tid + i * kThreads;
        const int64_t row = b_rows[kbeg + s * BK + t / (BN / 4)];
        rb[i] = *reinterpret_cast<const float4*>(p.B + row * p.ldb + n0 + (t % (BN / 4)) * 4);
      } else {
        rb[i] = *reinterpret_cast<const float4*>(bsrc[i] + s * b_step);
      }
    }
  };
  auto lstore = [&](const float4 (&ra)[A_F4], const float4 (&rb)[B_F4], int buf) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int t = tid + i * kThreads;
      const int m = t / (BK / 4);
      const int kq = (t % (BK / 4)) * 4;
      As[buf][kq + 0][m] = ra[i].x;
      As[buf][kq + 1][m] = ra[i].y;
      As[buf][kq + 2][m] = ra[i].z;
      As[buf][kq + 3][m] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int t = tid + i * kThreads;
      if constexpr (!TRANS_B) {
        *reinterpret_cast<float4*>(&Bs[buf][t / (BN / 4)][(t % (BN / 4)) * 4]) = rb[i];
      } else {
        const int n = t / (BK / 4);
        const int kq = (t % (BK / 4)) * 4;
        Bs[buf][kq + 0][n] = rb[i].x;
        Bs[buf][kq + 1][n] = rb[i].y;
        Bs[buf][kq + 2][n] = rb[i].z;
        Bs[buf][kq + 3][n] = rb[i].w;
      }
    }
  };

  floatx16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // PRE_C: this lane's C entries of an axpby epilogue with beta != 0, loaded before the K loop
  float cpre[PRE_C ? MI : 1][PRE_C ? NI : 1][PRE_C ? 16 : 1];
  if constexpr (PRE_C) {
    const int col = lane & 31;
    const int rbase = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int64_t gn = n0 + wn0 + j * 32 + col;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t gm = m0 + wm0 + i * 32 + (v >> 2) * 8 + rbase + (v & 3);
          cpre[i][j][v] = p.C[gm * p.ldc + gn];
        }
      }
  }

  const int kl = lane >> 5;
  const int ml = lane & 31;
  auto compute = [&](int buf) {
#pragma unroll
    for (int k0 = 0; k0 < BK / 2; k0 += HOIST) {
      float a[HOIST][MI], b[HOIST][NI];
#pragma unroll
      for (int kk = 0; kk < HOIST; ++kk) {
#pragma unroll
        for (int i = 0; i < MI; ++i) a[kk][i] = As[buf][2 * (k0 + kk) + kl][wm0 + i * 32 + ml];
#pragma unroll
        for (int j = 0; j < NI; ++j) b[kk][j] = Bs[buf][2 * (k0 + kk) + kl][wn0 + j * 32 + ml];
      }
#pragma unroll
      for (int kk = 0; kk < HOIST; ++kk)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk][i], b[kk][j], acc[i][j], 0, 0, 0);
    }
  };

  // prologue: slab 0 -> LDS buffer 0, slab 1 in flight in R1 (nslab is even)
  gload(ra0, rb0, 0);
  gload(ra1, rb1, 1);
  lstore(ra0, rb0, 0);
  __syncthreads();
  // slab s is in LDS buffer s&1; slab s+1 is in flight in R((s+1)&1).  The body covers two slabs
  // with no early exit: an exit between the halves leaves the accumulators in different registers
  // on the two paths, and the compiler then copies all of them through VGPRs every iteration,
  // which drains the MFMA pipeline (measured 88 -> 121 TFLOP/s at 128 x 14336 x 14336).
  for (int64_t s = 0; s < nslab; s += 2) {
    if (s + 2 < nslab) gload(ra0, rb0, s + 2);
    compute(0);
    lstore(ra1, rb1, 1);
    __syncthreads();
    if (s + 3 < nslab) gload(ra1, rb1, s + 3);
    compute(1);
    if (s + 2 < nslab) lstore(ra0, rb0, 0);
    __syncthreads();
  }

  const int col = lane & 31;
  const int rbase = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int64_t gn = n0 + wn0 + j * 32 + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t gm = m0 + wm0 + i * 32 + (v >> 2) * 8 + rbase + (v & 3);
        const float val = acc[i][j][v];
        if (p.mode == kGemmPartials) {
          p.C[(int64_t)split * p.split_stride + gm * p.ldc + gn] = val;
        } else {
          float* dst = p.C + gm * p.ldc + gn;
          if constexpr (PRE_C) {
            *dst = p.alpha * val + p.beta * cpre[i][j][v];
          } else {
            *dst = p.beta == 0.f ? p.alpha * val : p.alpha * val + p.beta * *dst;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// fp32 product on the bf16 matrix cores ("x6").  Every fp32 operand x is split into three bf16
// planes,
//   x0 = rn(x), x1 = rn(x - x0), x2 = rn(x - x0 - x1)   (rn: round to nearest bf16)
// with |x1| <= 2^-8 |x|, |x2| <= 2^-16 |x| and |x - x0 - x1 - x2| <= 2^-24 |x|, and the product keeps
// the six plane products of order >= 2^-16 |a||b|:
//   a b = a0 b0 + (a0 b1 + a1 b0) + (a0 b2 + a1 b1 + a2 b0) + e,   |e| <= ~2^-22.4 |a||b|
// (a1 b2 + a2 b1 + a2 b2 and the residues below the third planes), the size of one or two fp32
// roundings of the product; a product of two bf16 values is exact in the fp32 accumulator.
// v_mfma_f32_32x32x16_bf16 has 16x the flop rate of v_mfma_f32_32x32x2_f32, so the six products
// of a 32x32x16 step take 3/8 of the fp32 instruction time.
//
// Operands are packed into 128-row x 16-k tiles in MFMA fragment order: chunk c = (blk*2 + h)*32 + r
// of a tile holds row blk*32 + r at k = 16 ks + 8 h + (0..7).  B (the large, reused operand) is
// packed once as fp32 [N/128][K/16][2][256 chunks][4] (first and second four k of every chunk in two
// 4 KB halves, so a fragment is two conflict-free 16-byte LDS reads); A (small, re-formed per
// product) is split and packed as bf16 planes [ceil(M/128)][K/16][3][256][8].  A work-group
// (128 x 128 tile, one K slice, 2 x 2 waves of 64 x 64) reads each K slab as contiguous 12 KB (A,
// L2-resident) + 8 KB (B) and runs 24 MFMAs per wave per slab.  gemm_x6_ring_kernel moves the slabs
// with global_load_lds into a 4-stage LDS ring (three slabs in flight, no register staging), its
// four waves take 128 x 32 each (1 x 4), and each wave splits its own B fragments; gemm_x6_kernel (K slices of an even slab count) stages through
// registers and splits B once on its way to LDS.  Split s of tile t is block t * splits + s, so with
// 8 or 16 splits every XCD (blocks are dispatched round-robin over 8) works on one or two K slices
// and its L2 holds those slices of A.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));


// B tiles: thread per chunk (8 floats).  trans_b: op(B)(k, n) = B[n*ldb + k] (32 contiguous bytes
// per thread), else B[k*ldb + n] (lanes along n).
template <bool TRANS_B>
__global__ void x6_pack_b_kernel(const float* __restrict__ B, int64_t ldb, int64_t K, int64_t N, float* __restrict__ Bt) {
  const int64_t KS = K / 16;
  const int64_t nchunks = (N / 128) * KS * 256;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < nchunks; q += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(q & 255);
    const int64_t tk = q >> 8;  // nt * KS + ks
    const int64_t nt = tk / KS, ks = tk - nt * KS;
    const int64_t n = nt * 128 + (c >> 6) * 32 + (c & 31), k0 = ks * 16 + ((c >> 5) & 1) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = TRANS_B ? B[n * ldb + k0 + e] : B[(k0 + e) * ldb + n];
    float4* d = reinterpret_cast<float4*>(Bt) + tk * 512 + c;
    d[0] = make_float4(v[0], v[1], v[2], v[3]);
    d[256] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// A planes (of A diag(colscale) when colscale is given): thread per chunk; rows >= M are zero.
__global__ void x6_pack_a_kernel(const float* __restrict__ A, int64_t lda, int64_t M, int64_t K, uint4* __restrict__ At,
                                 const float* __restrict__ colscale) {
  const int64_t KS = K / 16;
  const int64_t nchunks = ((M + 127) / 128) * KS * 256;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < nchunks; q += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(q & 255);
    const int64_t tk = q >> 8;  // mt * KS + ks
    const int64_t mt = tk / KS, ks = tk - mt * KS;
    const int64_t m = mt * 128 + (c >> 6) * 32 + (c & 31), k0 = ks * 16 + ((c >> 5) & 1) * 8;
    float v[8];
    if (m < M) {
      const float* src = A + m * lda + k0;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = src[e];
      if (colscale) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] *= colscale[k0 + e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    uint4 h, mm, l;
    split3(v[0], v[1], h.x, mm.x, l.x);
    split3(v[2], v[3], h.y, mm.y, l.y);
    split3(v[4], v[5], h.z, mm.z, l.z);
    split3(v[6], v[7], h.w, mm.w, l.w);
    uint4* d = At + tk * 768 + c;
    d[0] = h;
    d[256] = mm;
    d[512] = l;
  }
}

// C[split] (rows < M) = A[:, K slice] * op(B)[K slice, :] from the packed operands.  Every K slice
// is an even number of 16-k slabs.
__global__ __launch_bounds__(kThreads) void gemm_x6_kernel(int64_t M, int64_t N, int64_t K, const uint4* __restrict__ At,
                                                           const float* __restrict__ Bt, float* __restrict__ C,
                                                           int64_t ldc, int64_t split_stride, int64_t k_per_split,
                                                           int splits) {
  __shared__ uint4 As[2][3][256];
  __shared__ uint4 Bs[2][3][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wmb = (wave >> 1) * 2, wnb = (wave & 1) * 2;  // 2 x 2 waves of 64 x 64
  const int64_t bid = blockIdx.x;
  const int split = (int)(bid % splits);
  const int64_t tile = bid / splits;
  const int64_t ntn = N / 128;
  const int64_t mt = tile / ntn, nt = tile - mt * ntn;
  const int64_t KS = K / 16;
  const int nslab = (int)(k_per_split / 16);
  const int64_t ks0 = (int64_t)split * nslab;
  // A slab: 768 chunks (3 planes), thread -> chunks tid + 256 j; B slab: 2 x 256 float4, thread ->
  // both halves of chunk tid
  const u32x4v* asrc = reinterpret_cast<const u32x4v*>(At) + (mt * KS + ks0) * 768 + tid;
  const f32x4v* bsrc = reinterpret_cast<const f32x4v*>(Bt) + (nt * KS + ks0) * 512 + tid;

  u32x4v qa0[3], qa1[3];
  f32x4v qb0[2], qb1[2];
  auto gload = [&](u32x4v (&qa)[3], f32x4v (&qb)[2], int64_t s) {
#pragma unroll
    for (int j = 0; j < 3; ++j) qa[j] = asrc[s * 768 + j * 256];
#pragma unroll
    for (int j = 0; j < 2; ++j) qb[j] = bsrc[s * 512 + j * 256];
  };
  auto lstore = [&](const u32x4v (&qa)[3], const f32x4v (&qb)[2], int buf) {
#pragma unroll
    for (int j = 0; j < 3; ++j) As[buf][j][tid] = __builtin_bit_cast(uint4, qa[j]);
    uint4 h, m, l;
    split3(qb[0].x, qb[0].y, h.x, m.x, l.x);
    split3(qb[0].z, qb[0].w, h.y, m.y, l.y);
    split3(qb[1].x, qb[1].y, h.z, m.z, l.z);
    split3(qb[1].z, qb[1].w, h.w, m.w, l.w);
    Bs[buf][0][tid] = h;
    Bs[buf][1][tid] = m;
    Bs[buf][2][tid] = l;
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto compute = [&](int buf) {
    bf16x8 a[3][2], b[3][2];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) {
#pragma unroll
      for (int i = 0; i < 2; ++i) a[pl][i] = __builtin_bit_cast(bf16x8, As[buf][pl][(wmb + i) * 64 + lane]);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[pl][j] = __builtin_bit_cast(bf16x8, Bs[buf][pl][(wnb + j) * 64 + lane]);
    }
    // smallest terms first; the (i, j) loop innermost keeps four independent accumulator chains
    constexpr int pa[6] = {2, 1, 0, 1, 0, 0};
    constexpr int pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
    for (int t = 0; t < 6; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[pa[t]][i], b[pb[t]][j], acc[i][j], 0, 0, 0);
  };

  // same two-slabs-in-flight schedule as gemm_f32_full_kernel
  gload(qa0, qb0, 0);
  gload(qa1, qb1, 1);
  lstore(qa0, qb0, 0);
  __syncthreads();
  for (int s = 0; s < nslab; s += 2) {
    if (s + 2 < nslab) gload(qa0, qb0, s + 2);
    compute(0);
    lstore(qa1, qb1, 1);
    __syncthreads();
    if (s + 3 < nslab) gload(qa1, qb1, s + 3);
    compute(1);
    if (s + 2 < nslab) lstore(qa0, qb0, 0);
    __syncthreads();
  }

  // lane l, accumulator v -> row 8*(v/4) + 4*(l/32) + v%4, column l%32 of the 32 x 32 block
  const int col = lane & 31, rbase = (lane >> 5) * 4;
  float* Cs = C + (int64_t)split * split_stride;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t gn = nt * 128 + (wnb + j) * 32 + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t gm = mt * 128 + (wmb + i) * 32 + (v >> 2) * 8 + rbase + (v & 3);
        if (gm < M) Cs[gm * ldc + gn] = acc[i][j][v];
      }
    }
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt bits 3:0 and 15:14).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Same product as gemm_x6_kernel with the slabs moved by global_load_lds into a ring of four LDS
// stages (three slabs in flight, no register staging).  Each stage is its own __shared__ array and
// the loops are unrolled by four, so every stage index is a constant: the compiler then tells the
// stages apart and waits only where this code waits (s_waitcnt vmcnt(n) before each barrier: all
// but the n most recent loads of this wave done, i.e. the slab about to be read).  The barrier is
// s_barrier without a fence (the fence of __syncthreads would wait for every load in flight).
// Every K slice is a positive multiple of four slabs.
template <bool kColWaves>
__global__ __launch_bounds__(kThreads) void gemm_x6_ring_kernel(int64_t M, int64_t N, int64_t K,
                                                                const uint4* __restrict__ At,
                                                                const float* __restrict__ Bt, float* __restrict__ C,
                                                                int64_t ldc, int64_t split_stride,
                                                                int64_t k_per_split, int splits) {
  constexpr int S = 4;
  constexpr int STAGE = 768 + 512;  // 16-byte slots: A planes, then the two halves of B
  constexpr int LOADS = 5;          // global_load_lds per wave per slab: 3 (A) + 2 (B)
  __shared__ uint4 st0[STAGE];
  __shared__ uint4 st1[STAGE];
  __shared__ uint4 st2[STAGE];
  __shared__ uint4 st3[STAGE];
  auto stage = [&](int slot) -> uint4* { return slot == 0 ? st0 : slot == 1 ? st1 : slot == 2 ? st2 : st3; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // wave tiles: 2 x 2 waves of 64 x 64, or (kColWaves) 1 x 4 waves of 128 x 32: every wave splits
  // only its own 32 columns of B (half the split work; the A planes, already split, are read by all
  // four).  The launch uses the 1 x 4 form: the same products in the same order (bit-identical
  // partials), 2.5-9 % less time at 128 x n x n for n = 4096, 8192 and 14336.
  constexpr int RT = kColWaves ? 4 : 2, CT = kColWaves ? 1 : 2;
  const int wmb = kColWaves ? 0 : (wave >> 1) * 2, wnb = kColWaves ? wave : (wave & 1) * 2;
  const int64_t bid = blockIdx.x;
  const int split = (int)(bid % splits);
  const int64_t tile = bid / splits;
  const int64_t ntn = N / 128;
  const int64_t mt = tile / ntn, nt = tile - mt * ntn;
  const int64_t KS = K / 16;
  const int nslab = (int)(k_per_split / 16);
  const int64_t ks0 = (int64_t)split * nslab;
  // wave w moves A slots w*192 + 64 q (q < 3) and B slots w*128 + 64 q (q < 2); lane l adds 16 l bytes
  const uint4* asrc = At + (mt * KS + ks0) * 768 + wave * 192 + lane;
  const uint4* bsrc = reinterpret_cast<const uint4*>(Bt) + (nt * KS + ks0) * 512 + wave * 128 + lane;
  auto issue = [&](int s, int slot) {
    uint4* d = stage(slot);
#pragma unroll
    for (int q = 0; q < 3; ++q)
      __builtin_amdgcn_global_load_lds(asrc + (int64_t)s * 768 + q * 64, d + wave * 192 + q * 64, 16, 0, 0);
#pragma unroll
    for (int q = 0; q < 2; ++q)
      __builtin_amdgcn_global_load_lds(bsrc + (int64_t)s * 512 + q * 64, d + 768 + wave * 128 + q * 64, 16, 0, 0);
  };
  floatx16 acc[RT][CT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  auto compute = [&](int slot) {
    const uint4* d = stage(slot);
    bf16x8 a[3][RT], b[3][CT];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int i = 0; i < RT; ++i) a[pl][i] = __builtin_bit_cast(bf16x8, d[pl * 256 + (wmb + i) * 64 + lane]);
#pragma unroll
    for (int j = 0; j < CT; ++j) {
      const float4 x = __builtin_bit_cast(float4, d[768 + (wnb + j) * 64 + lane]);
      const float4 y = __builtin_bit_cast(float4, d[768 + 256 + (wnb + j) * 64 + lane]);
      uint4 h, m, l;
      split3(x.x, x.y, h.x, m.x, l.x);
      split3(x.z, x.w, h.y, m.y, l.y);
      split3(y.x, y.y, h.z, m.z, l.z);
      split3(y.z, y.w, h.w, m.w, l.w);
      b[0][j] = __builtin_bit_cast(bf16x8, h);
      b[1][j] = __builtin_bit_cast(bf16x8, m);
      b[2][j] = __builtin_bit_cast(bf16x8, l);
    }
    constexpr int pa[6] = {2, 1, 0, 1, 0, 0};
    constexpr int pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
    for (int t = 0; t < 6; ++t)
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[pa[t]][i], b[pb[t]][j], acc[i][j], 0, 0, 0);
  };
  auto sync = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Slab t lives in stage t % 4.  Step t: wait for slab t (loads of slabs t+1, t+2 may stay in
  // flight), barrier (slab t visible; every wave is done with stage (t-1) % 4), issue slab t+3 into
  // that stage, compute slab t.
#pragma unroll
  for (int t = 0; t < S - 1; ++t) issue(t, t);
  int t0 = 0;
  for (; t0 < nslab - S; t0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS * (S - 2)));
      sync();
      issue(t0 + u + S - 1, (u + S - 1) % S);
      compute(u);
    }
  }
  // last four slabs: slab nslab - 1 is issued in the first step, then the ring drains
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS * 2));
  sync();
  issue(t0 + S - 1, S - 1);
  compute(0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS * 2));
  sync();
  compute(1);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(LOADS * 1));
  sync();
  compute(2);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  sync();
  compute(3);

  const int col = lane & 31, rbase = (lane >> 5) * 4;
  float* Cs = C + (int64_t)split * split_stride;
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < CT; ++j) {
      const int64_t gn = nt * 128 + (wnb + j) * 32 + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t gm = mt * 128 + (wmb + i) * 32 + (v >> 2) * 8 + rbase + (v & 3);
        if (gm < M) Cs[gm * ldc + gn] = acc[i][j][v];
      }
    }
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_cfg(const GemmParams& p, dim3 grid, hipStream_t stream) {
  // interior-tile kernel: whole tiles, an even number of 16-wide K slabs per split; a row gather
  // also needs its groups aligned to the 128-row M tile
  const bool gather_ok = !p.b_rows || (!p.trans_b && (p.b_rows_group == 0 || p.b_rows_group % BM == 0));
  const bool full = gather_ok && p.a_vec4 && p.b_vec4 && p.M % BM == 0 && p.N % BN == 0 &&
                    p.k_per_split % 32 == 0 && (int64_t)grid.z * p.k_per_split == p.K;
  const bool pre_c = p.mode == kGemmAxpby && p.beta != 0.f;
  if (full && p.b_rows) {
    if (pre_c) hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, false, 8, true, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, false, 8, false, true>), grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
  }
  if (full) {
    if (p.trans_b) {
      if (pre_c) hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, true, 8, true>), grid, dim3(kThreads), 0, stream, p);
      else hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      if (pre_c) hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, false, 8, true>), grid, dim3(kThreads), 0, stream, p);
      else hipLaunchKernelGGL((gemm_f32_full_kernel<BM, BN, WM, WN, false>), grid, dim3(kThreads), 0, stream, p);
    }
    return hipGetLastError();
  }
  // (the general kernel does not prefetch C: that costs it 96 VGPRs, occupancy 6 -> 2, and measured
  // slower on the CD Schur update)
  if (p.trans_b) {
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, true, false>), grid, dim3(kThreads), 0, stream, p);
  } else if (p.b_rows) {
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, false, true>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, false, false>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

int choose_splits(int64_t M, int64_t N, int64_t K, int64_t workspace_floats, int* bn_out) {
  // 128x64 tiles: the 128x128 variant needs 154 VGPRs + 128 AGPRs (one work-group per SIMD set),
  // which measured slower on every shape tried.
  const int64_t tiles_m = (M + 127) / 128;
  const int bn = 64;
  const int64_t tiles = tiles_m * ((N + bn - 1) / bn);
  int splits = 1;
  const int64_t target = 2048;  // ~8 work-groups per CU on 256 CUs (latency hiding at small M)
  while (splits < 32 && tiles * splits * 2 <= target && K / (splits * 2) >= 256 &&
         (int64_t)(splits * 2) * M * N <= workspace_floats)
    splits *= 2;
  *bn_out = bn;
  return splits;
}

hipError_t gemm_partials(GemmParams p, int splits, int bn, hipStream_t stream) {
  p.mode = splits > 1 ? kGemmPartials : p.mode;
  const int64_t kps = ((p.K + splits - 1) / splits + 31) / 32 * 32;
  p.k_per_split = kps > 0 ? kps : kBK;
  p.a_vec4 = ((reinterpret_cast<uintptr_t>(p.A) & 15u) == 0) && (p.lda % 4 == 0);
  p.b_vec4 = ((reinterpret_cast<uintptr_t>(p.B) & 15u) == 0) && (p.ldb % 4 == 0);
  (void)bn;  // one tile shape: 128 x 64 (4 waves of 64 x 32)
  dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 127) / 128), (unsigned)splits);
  return launch_cfg<128, 64, 64, 32>(p, grid, stream);
}

hipError_t splitk_reduce(const float* P, int splits, int64_t M, int64_t N, float* C, int64_t ldc,
                         float alpha, float beta, hipStream_t stream) {
  const int64_t total = M * N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, P, splits,
                     M * N, M, N, C, ldc, alpha, beta);
  return hipGetLastError();
}

bool x6_shape_ok(int64_t N, int64_t K) { return N > 0 && K > 0 && N % 128 == 0 && K % 32 == 0; }

// Split K until the grid holds about two work-groups per CU (512) or a K slice would fall below
// 32 slabs (512): more splits do not speed the product up and every split is one more partial the
// epilogues read.  128 x 14336 x 14336: 4 splits, 0.292 ms per product and 8.7 us to read the
// partials back, against 0.298 ms and 20.7 us with 16 (the down_proj layer: 2 splits 1085 ms, 4
// splits 1053-1062 ms).  128 x 4096 x 4096: 8 splits; a 14336 x 4096 gate_proj layer takes 391 ms
// against 414 ms with 16 splits, 451 ms with 4 and 619 ms with 2.
int x6_choose_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + 127) / 128) * (N / 128);
  int splits = 1;
  while (splits < 16 && tiles * splits * 2 <= 512 && K % (splits * 2 * 32) == 0 && K / (splits * 2) >= 512)
    splits *= 2;
  return splits;
}

int64_t x6_packed_a_bytes(int64_t M, int64_t K) { return ((M + 127) / 128) * 128 * K * 6; }

static unsigned grid_for(int64_t items) {
  int64_t b = (items + 255) / 256;
  return (unsigned)(b < 1 ? 1 : b > 16384 ? 16384 : b);
}

hipError_t x6_pack_b(const float* B, int64_t ldb, bool trans_b, int64_t K, int64_t N, float* Bt, hipStream_t stream) {
  const unsigned g = grid_for((N / 128) * (K / 16) * 256);
  if (trans_b) hipLaunchKernelGGL(x6_pack_b_kernel<true>, dim3(g), dim3(256), 0, stream, B, ldb, K, N, Bt);
  else hipLaunchKernelGGL(x6_pack_b_kernel<false>, dim3(g), dim3(256), 0, stream, B, ldb, K, N, Bt);
  return hipGetLastError();
}

hipError_t x6_pack_a(const float* A, int64_t lda, int64_t M, int64_t K, void* At, hipStream_t stream,
                     const float* colscale) {
  const unsigned g = grid_for(((M + 127) / 128) * (K / 16) * 256);
  hipLaunchKernelGGL(x6_pack_a_kernel, dim3(g), dim3(256), 0, stream, A, lda, M, K, static_cast<uint4*>(At),
                     colscale);
  return hipGetLastError();
}

hipError_t x6_gemm_partials(const void* At, const float* Bt, int64_t M, int64_t N, int64_t K, float* C, int64_t ldc,
                            int64_t split_stride, int splits, hipStream_t stream) {
  const int64_t kps = K / splits;
  if (!x6_shape_ok(N, K) || splits < 1 || K % splits != 0 || kps % 32 != 0) return hipErrorInvalidValue;
  const int64_t blocks = ((M + 127) / 128) * (N / 128) * splits;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  if ((kps / 16) % 4 == 0)
    hipLaunchKernelGGL(gemm_x6_ring_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, M, N, K,
                       static_cast<const uint4*>(At), Bt, C, ldc, split_stride, kps, splits);
  else
    hipLaunchKernelGGL(gemm_x6_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, M, N, K,
                       static_cast<const uint4*>(At), Bt, C, ldc, split_stride, kps, splits);
  return hipGetLastError();
}

hipError_t gemm_lower(const float* A, int64_t lda, const float* B, int64_t ldb, bool trans_b, float* C,
                      int64_t ldc, int64_t M, int64_t K, float alpha, float beta, int upper_band,
                      hipStream_t stream) {
  GemmParams p{};
  p.M = M; p.N = M; p.K = K;
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb; p.trans_b = trans_b;
  p.alpha = alpha; p.beta = beta;
  p.mode = kGemmAxpby;
  p.C = C; p.ldc = ldc;
  p.lower_only = true;
  p.upper_band = upper_band;
  return gemm_partials(p, 1, 64, stream);
}

hipError_t gemm(const float* A, int64_t lda, const float* B, int64_t ldb, bool trans_b,
                const int32_t* b_rows, float* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                float alpha, float beta, float* workspace, int64_t workspace_floats,
                hipStream_t stream) {
  int bn = 128;
  int splits = choose_splits(M, N, K, workspace ? workspace_floats : 0, &bn);
  // whole 32-k slices per split let interior tiles run gemm_f32_full_kernel
  if (K % 32 == 0)
    while (splits > 1 && K % (splits * 32) != 0) splits /= 2;
  GemmParams p{};
  p.M = M; p.N = N; p.K = K;
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb; p.trans_b = trans_b; p.b_rows = b_rows;
  p.alpha = alpha; p.beta = beta;
  if (splits == 1) {
    p.mode = kGemmAxpby;
    p.C = C; p.ldc = ldc;
    return gemm_partials(p, 1, bn, stream);
  }
  p.mode = kGemmPartials;
  p.C = workspace; p.ldc = N; p.split_stride = M * N;
  hipError_t e = gemm_partials(p, splits, bn, stream);
  if (e != hipSuccess) return e;
  return splitk_reduce(workspace, splits, M, N, C, ldc, alpha, beta, stream);
}

}  // namespace mpq

extern "C" int mpq_gemm_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
                            const float* B, int64_t ldb, int trans_b, const int32_t* b_rows,
                            float* C, int64_t ldc, float alpha, float beta, float* workspace,
                            int64_t workspace_floats, hipStream_t stream) {
  MPQ_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "mpq_gemm_f32: negative extent");
  if (M == 0 || N == 0) return mpq::kOk;
  MPQ_CHECK_ARG(A && B && C, "mpq_gemm_f32: null operand");
  MPQ_CHECK_ARG(lda >= K && ldc >= N, "mpq_gemm_f32: leading dimension too small");
  MPQ_CHECK_ARG(trans_b ? ldb >= K : ldb >= N, "mpq_gemm_f32: ldb too small");
  MPQ_CHECK_ARG(!(trans_b && b_rows), "mpq_gemm_f32: row gather needs trans_b = 0");
  MPQ_CHECK_ARG(M <= (int64_t)65535 * 128 && N <= (int64_t)0x7fffffff * 64,
                "mpq_gemm_f32: extent too large");
  MPQ_HIP_TRY(mpq::gemm(A, lda, B, ldb, trans_b != 0, b_rows, C, ldc, M, N, K, alpha, beta,
                        workspace, workspace_floats, stream));
  return mpq::kOk;
}

extern "C" int mpq_gemm_f32_split_count(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  int bn = 128;
  return mpq::choose_splits(M, N, K, (int64_t)1 << 62, &bn);
}

extern "C" int mpq_gemm_f32_splitk(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                                   int64_t ldb, int trans_b, float* partials, int splits, hipStream_t stream) {
  MPQ_CHECK_ARG(M > 0 && N > 0 && K > 0, "mpq_gemm_f32_splitk: empty product");
  MPQ_CHECK_ARG(splits >= 1 && splits <= 32, "mpq_gemm_f32_splitk: splits must be in [1, 32]");
  MPQ_CHECK_ARG(A && B && partials, "mpq_gemm_f32_splitk: null operand");
  MPQ_CHECK_ARG(lda >= K && (trans_b ? ldb >= K : ldb >= N), "mpq_gemm_f32_splitk: leading dimension too small");
  MPQ_CHECK_ARG(M <= (int64_t)65535 * 128, "mpq_gemm_f32_splitk: M too large");
  int bn = 128;
  mpq::choose_splits(M, N, K, (int64_t)1 << 62, &bn);
  mpq::GemmParams p{};
  p.M = M; p.N = N; p.K = K;
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb; p.trans_b = trans_b != 0;
  p.C = partials; p.ldc = N; p.split_stride = M * N;
  p.alpha = 1.f; p.beta = 0.f; p.mode = mpq::kGemmPartials;
  MPQ_HIP_TRY(mpq::gemm_partials(p, splits, bn, stream));
  return mpq::kOk;
}

extern "C" int mpq_gemm_x6_pack_b(int64_t K, int64_t N, const float* B, int64_t ldb, int trans_b, float* packed,
                                  hipStream_t stream) {
  MPQ_CHECK_ARG(mpq::x6_shape_ok(N, K), "mpq_gemm_x6_pack_b: needs N %% 128 == 0 and K %% 32 == 0 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  MPQ_CHECK_ARG(B && packed, "mpq_gemm_x6_pack_b: null operand");
  MPQ_CHECK_ARG(trans_b ? ldb >= K : ldb >= N, "mpq_gemm_x6_pack_b: ldb too small");
  MPQ_HIP_TRY(mpq::x6_pack_b(B, ldb, trans_b != 0, K, N, packed, stream));
  return mpq::kOk;
}

extern "C" int64_t mpq_gemm_x6_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || !mpq::x6_shape_ok(N, K)) return 0;
  const int splits = mpq::x6_choose_splits(M, N, K);
  return (mpq::x6_packed_a_bytes(M, K) + 255) / 256 * 256 + (int64_t)splits * M * N * 4;
}

extern "C" int mpq_gemm_x6(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B_packed,
                           float* C, int64_t ldc, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  MPQ_CHECK_ARG(M >= 0, "mpq_gemm_x6: negative M");
  if (M == 0) return mpq::kOk;
  MPQ_CHECK_ARG(mpq::x6_shape_ok(N, K), "mpq_gemm_x6: needs N %% 128 == 0 and K %% 32 == 0 (N=%lld K=%lld)",
                (long long)N, (long long)K);
  MPQ_CHECK_ARG(A && B_packed && C && workspace, "mpq_gemm_x6: null operand");
  MPQ_CHECK_ARG(lda >= K && ldc >= N, "mpq_gemm_x6: leading dimension too small");
  MPQ_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "mpq_gemm_x6: workspace must be 256-byte aligned");
  const int64_t need = mpq_gemm_x6_workspace_size(M, N, K);
  MPQ_CHECK_ARG(workspace_bytes >= need, "mpq_gemm_x6: workspace too small (%lld < %lld bytes)",
                (long long)workspace_bytes, (long long)need);
  const int splits = mpq::x6_choose_splits(M, N, K);
  char* ws = static_cast<char*>(workspace);
  float* P = reinterpret_cast<float*>(ws + (mpq::x6_packed_a_bytes(M, K) + 255) / 256 * 256);
  MPQ_HIP_TRY(mpq::x6_pack_a(A, lda, M, K, ws, stream));
  MPQ_HIP_TRY(mpq::x6_gemm_partials(ws, B_packed, M, N, K, P, N, M * N, splits, stream));
  MPQ_HIP_TRY(mpq::splitk_reduce(P, splits, M, N, C, ldc, 1.f, 0.f, stream));
  return mpq::kOk;
}

extern "C" int64_t mpq_rankspace_pack_floats(int64_t n) {
  return (n > 0 && mpq::x6_shape_ok(n, n)) ? 3 * n * n : 0;
}

extern "C" int mpq_rankspace_pack(int64_t n, const float* V, const float* Vs, float* packed, hipStream_t stream) {
  MPQ_CHECK_ARG(n > 0 && mpq::x6_shape_ok(n, n), "mpq_rankspace_pack: n must be a positive multiple of 128 (n=%lld)",
                (long long)n);
  MPQ_CHECK_ARG(V && Vs && packed, "mpq_rankspace_pack: null operand");
  MPQ_HIP_TRY(mpq::x6_pack_b(V, n, false, n, n, packed, stream));
  MPQ_HIP_TRY(mpq::x6_pack_b(V, n, true, n, n, packed + n * n, stream));
  MPQ_HIP_TRY(mpq::x6_pack_b(Vs, n, false, n, n, packed + 2 * n * n, stream));
  return mpq::kOk;
}

extern "C" int mpq_gemm_x6_split_count(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || !mpq::x6_shape_ok(N, K)) return 0;
  return mpq::x6_choose_splits(M, N, K);
}

extern "C" int64_t mpq_gemm_x6_packed_a_size(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 32 != 0) return 0;
  return mpq::x6_packed_a_bytes(M, K);
}

extern "C" int mpq_gemm_x6_pack_a(int64_t M, int64_t K, const float* A, int64_t lda, void* packed, hipStream_t stream) {
  MPQ_CHECK_ARG(M > 0 && K > 0 && K % 32 == 0, "mpq_gemm_x6_pack_a: needs M > 0 and K %% 32 == 0");
  MPQ_CHECK_ARG(A && packed && lda >= K, "mpq_gemm_x6_pack_a: null operand or lda < K");
  MPQ_CHECK_ARG((reinterpret_cast<uintptr_t>(packed) & 15u) == 0, "mpq_gemm_x6_pack_a: packed must be 16-byte aligned");
  MPQ_HIP_TRY(mpq::x6_pack_a(A, lda, M, K, packed, stream));
  return mpq::kOk;
}

extern "C" int mpq_gemm_x6_splitk(int64_t M, int64_t N, int64_t K, const void* A_packed, const float* B_packed,
                                  float* partials, int splits, hipStream_t stream) {
  MPQ_CHECK_ARG(M > 0 && mpq::x6_shape_ok(N, K), "mpq_gemm_x6_splitk: needs M > 0, N %% 128 == 0, K %% 32 == 0");
  MPQ_CHECK_ARG(splits >= 1 && K % splits == 0 && (K / splits) % 32 == 0,
                "mpq_gemm_x6_splitk: K / splits must be a whole multiple of 32");
  MPQ_CHECK_ARG(A_packed && B_packed && partials, "mpq_gemm_x6_splitk: null operand");
  MPQ_HIP_TRY(mpq::x6_gemm_partials(A_packed, B_packed, M, N, K, partials, N, M * N, splits, stream));
  return mpq::kOk;
}
