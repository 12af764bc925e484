// fp64 GEMM on the fp64 matrix cores (v_mfma_f64_16x16x4_f64) for the fp64 eigensolver
// (mpq_syevd_f64: trailing updates of the tridiagonalisation, the compact-WY back-transformation and
// the divide-and-conquer merge products).
//
// Tiling: a work-group of four waves computes a 128 x 64 tile of C; wave w owns the 64 x 32 sub-tile
// at rows 64 (w / 2), columns 32 (w % 2), held as 4 x 2 accumulator tiles of 16 x 16 doubles.  K
// advances in slabs of 16: every thread loads its share of the next A (128 x 16) and B (16 x 64)
// slabs into registers while the waves run the current slab's 32 MFMAs from LDS, then stores them to
// the other LDS buffer (one barrier per slab).  Both slabs sit in LDS k-major (As[k][row],
// Bs[k][col]), so an MFMA operand fragment -- lane l takes row (or column) l % 16 at k = l / 16 --
// is 16 consecutive doubles per k.  Out-of-range rows, columns and k are loaded as zeros, so any
// M, N, K and leading dimension work.
//
// Split-K (grid z) writes each K slice's tile to a partials buffer and a second kernel sums the
// slices in split order: results are bit-reproducible for a given shape.
#include "gemm_f64.h"

#include <algorithm>

namespace mpq {
namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr int kBK = 16;
constexpr int kPadA = 4;  // row pitch kBM + 4 doubles: the k rows of a slab start 8 banks apart
constexpr int kPadB = 4;
constexpr int kThreads = 256;
constexpr int kALoads = kBM * kBK / kThreads;  // 8
constexpr int kBLoads = kBK * kBN / kThreads;  // 4

enum : int { kModePartials = 0, kModeAxpby = 1 };

struct F64Params {
  int64_t M, N, K;
  const double* A;
  int64_t lda;
  const double* B;
  int64_t ldb;
  double* C;
  int64_t ldc;
  int64_t split_stride;  // partials mode: slice s at C + s * split_stride
  int64_t k_per_split;   // multiple of kBK
  double alpha, beta;
  int mode;
  int trans_b;
  int lower_only;
  int64_t upper_band;
};

__global__ __launch_bounds__(kThreads) void gemm_f64_kernel(F64Params p) {
  const int64_t m0 = (int64_t)blockIdx.y * kBM;
  const int64_t n0 = (int64_t)blockIdx.x * kBN;
  if (p.lower_only && n0 > m0 + kBM - 1 + p.upper_band) return;  // tile entirely above the band
  const int64_t k_begin = (int64_t)blockIdx.z * p.k_per_split;
  const int64_t k_end = min(p.K, k_begin + p.k_per_split);

  __shared__ double As[2][kBK][kBM + kPadA];
  __shared__ double Bs[2][kBK][kBN + kPadB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 32;
  const int fr = lane & 15;   // fragment row / column
  const int fk = lane >> 4;   // fragment k

  // C = alpha A B + beta C with alpha = +-1 and beta != 0 (the eigensolvers' updates, K = 64 or 128,
  // which are bound by this read-modify-write of C): the accumulators start from alpha beta C, read
  // before the K loop so that its latency hides behind the products (read after them it ran at
  // 1-2 TB/s), and alpha acc is the result -- the same value as alpha (A B) + beta C up to the
  // order of the fp64 sum.
  const bool c_early = p.mode == kModeAxpby && p.beta != 0.0 && (p.alpha == 1.0 || p.alpha == -1.0);
  v4d acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
      if (c_early) {
        const double ab = p.alpha * p.beta;
        const int64_t col = min(n0 + wn + 16 * j + fr, p.N - 1);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t row = min(m0 + wm + 16 * i + fk + 4 * v, p.M - 1);
          acc[i][j][v] = ab * p.C[row * p.ldc + col];
        }
      }
    }
  }

  double ra[kALoads], rb[kBLoads];
  // A slab: element e = u * 256 + tid is (row e / 16, k e % 16): 16 lanes read one row's 128 bytes
  auto load_slab = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < kALoads; ++u) {
      const int e = u * kThreads + tid;
      const int64_t gm = m0 + (e >> 4);
      const int64_t gk = k0 + (e & 15);
      ra[u] = (gm < p.M && gk < k_end) ? p.A[gm * p.lda + gk] : 0.0;
    }
    if (p.trans_b) {
      // B stored N x K: element e is (column e / 16, k e % 16)
#pragma unroll
      for (int u = 0; u < kBLoads; ++u) {
        const int e = u * kThreads + tid;
        const int64_t gn = n0 + (e >> 4);
        const int64_t gk = k0 + (e & 15);
        rb[u] = (gn < p.N && gk < k_end) ? p.B[gn * p.ldb + gk] : 0.0;
      }
    } else {
      // B stored K x N: element e is (k e / 64, column e % 64)
#pragma unroll
      for (int u = 0; u < kBLoads; ++u) {
        const int e = u * kThreads + tid;
        const int64_t gk = k0 + (e >> 6);
        const int64_t gn = n0 + (e & 63);
        rb[u] = (gn < p.N && gk < k_end) ? p.B[gk * p.ldb + gn] : 0.0;
      }
    }
  };
  auto store_slab = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kALoads; ++u) {
      const int e = u * kThreads + tid;
      As[buf][e & 15][e >> 4] = ra[u];
    }
    if (p.trans_b) {
#pragma unroll
      for (int u = 0; u < kBLoads; ++u) {
        const int e = u * kThreads + tid;
        Bs[buf][e & 15][e >> 4] = rb[u];
      }
    } else {
#pragma unroll
      for (int u = 0; u < kBLoads; ++u) {
        const int e = u * kThreads + tid;
        Bs[buf][e >> 6][e & 63] = rb[u];
      }
    }
  };

  if (k_begin < k_end) {
    load_slab(k_begin);
    store_slab(0);
    __syncthreads();
    int buf = 0;
    for (int64_t k0 = k_begin; k0 < k_end; k0 += kBK) {
      const bool more = k0 + kBK < k_end;
      if (more) load_slab(k0 + kBK);
#pragma unroll
      for (int s = 0; s < kBK / 4; ++s) {
        double a[4], b[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[buf][4 * s + fk][wm + 16 * i + fr];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = Bs[buf][4 * s + fk][wn + 16 * j + fr];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      if (more) store_slab(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }

  // accumulator element v of tile (i, j): row 16 i + lane / 16 + 4 v, column 16 j + lane % 16 (the
  // fp64 16 x 16 result interleaves its rows over the four lane groups)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn + 16 * j + fr;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = m0 + wm + 16 * i + fk + 4 * v;
        if (row >= p.M) continue;
        if (p.mode == kModePartials) {
          p.C[(int64_t)blockIdx.z * p.split_stride + row * p.ldc + col] = acc[i][j][v];
        } else if (c_early) {
          p.C[row * p.ldc + col] = p.alpha * acc[i][j][v];
        } else {
          double* c = p.C + row * p.ldc + col;
          const double prod = p.alpha * acc[i][j][v];
          *c = p.beta == 0.0 ? prod : prod + p.beta * *c;
        }
      }
    }
  }
}

// C = alpha * sum_s P[s] + beta * C, slices added in split order.
__global__ __launch_bounds__(256) void f64_reduce_kernel(const double* __restrict__ P, int splits, int64_t M,
                                                         int64_t N, double* __restrict__ C, int64_t ldc, double alpha,
                                                         double beta) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t stride = M * N;
  double s = P[idx];
  for (int k = 1; k < splits; ++k) s += P[(int64_t)k * stride + idx];
  const int64_t r = idx / N, c = idx % N;
  double* out = C + r * ldc + c;
  const double prod = alpha * s;
  *out = beta == 0.0 ? prod : prod + beta * *out;
}

hipError_t launch(const F64Params& p, int splits, hipStream_t stream) {
  const dim3 grid((unsigned)((p.N + kBN - 1) / kBN), (unsigned)((p.M + kBM - 1) / kBM), (unsigned)splits);
  hipLaunchKernelGGL(gemm_f64_kernel, grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

int f64_choose_splits(int64_t M, int64_t N, int64_t K, int64_t workspace_elems) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int64_t target = 512;  // two work-groups per CU
  if (tiles >= target || workspace_elems <= 0) return 1;
  int64_t s = (target + tiles - 1) / tiles;
  s = std::min<int64_t>(s, std::max<int64_t>(K / (4 * kBK), 1));  // each slice at least 4 slabs
  s = std::min<int64_t>(s, 64);
  while (s > 1 && s * M * N > workspace_elems) --s;
  return (int)std::max<int64_t>(s, 1);
}

hipError_t gemm_f64(const double* A, int64_t lda, const double* B, int64_t ldb, bool trans_b, double* C,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, double alpha, double beta, double* workspace,
                    int64_t workspace_elems, hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  F64Params p{};
  p.M = M;
  p.N = N;
  p.K = std::max<int64_t>(K, 0);
  p.A = A;
  p.lda = lda;
  p.B = B;
  p.ldb = ldb;
  p.trans_b = trans_b ? 1 : 0;
  p.alpha = alpha;
  p.beta = beta;
  const int splits = workspace ? f64_choose_splits(M, N, p.K, workspace_elems) : 1;
  if (splits <= 1) {
    p.C = C;
    p.ldc = ldc;
    p.mode = kModeAxpby;
    p.k_per_split = std::max<int64_t>((p.K + kBK - 1) / kBK * kBK, kBK);
    return launch(p, 1, stream);
  }
  const int64_t slabs = (p.K + kBK - 1) / kBK;
  p.k_per_split = (slabs + splits - 1) / splits * kBK;
  const int used = (int)((p.K + p.k_per_split - 1) / p.k_per_split);  // slices holding some k
  p.C = workspace;
  p.ldc = N;
  p.split_stride = M * N;
  p.mode = kModePartials;
  hipError_t e = launch(p, used, stream);
  if (e != hipSuccess) return e;
  const int64_t total = M * N;
  hipLaunchKernelGGL(f64_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, workspace, used,
                     M, N, C, ldc, alpha, beta);
  return hipGetLastError();
}

hipError_t gemm_f64_lower(const double* A, int64_t lda, const double* B, int64_t ldb, bool trans_b, double* C,
                          int64_t ldc, int64_t M, int64_t K, double alpha, double beta, int64_t upper_band,
                          hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  F64Params p{};
  p.M = M;
  p.N = M;
  p.K = std::max<int64_t>(K, 0);
  p.A = A;
  p.lda = lda;
  p.B = B;
  p.ldb = ldb;
  p.trans_b = trans_b ? 1 : 0;
  p.alpha = alpha;
  p.beta = beta;
  p.C = C;
  p.ldc = ldc;
  p.mode = kModeAxpby;
  p.k_per_split = std::max<int64_t>((p.K + kBK - 1) / kBK * kBK, kBK);
  p.lower_only = 1;
  p.upper_band = upper_band;
  return launch(p, 1, stream);
}

}  // namespace mpq

// ---- C-ABI --------------------------------------------------------------------------------------

extern "C" int64_t mpq_gemm_f64_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = mpq::f64_choose_splits(M, N, K, (int64_t)1 << 62);
  return s > 1 ? (int64_t)s * M * N * (int64_t)sizeof(double) : 0;
}

extern "C" int mpq_gemm_f64(int64_t M, int64_t N, int64_t K, const double* A, int64_t lda, const double* B,
                            int64_t ldb, int trans_b, double* C, int64_t ldc, double alpha, double beta,
                            double* workspace, int64_t workspace_bytes, hipStream_t stream) {
  MPQ_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "mpq_gemm_f64: negative dimension");
  MPQ_CHECK_ARG(M == 0 || N == 0 || (A && B && C) || K == 0, "mpq_gemm_f64: null operand");
  MPQ_CHECK_ARG(M == 0 || N == 0 || C, "mpq_gemm_f64: null C");
  MPQ_CHECK_ARG(lda >= K && ldc >= N && ldb >= (trans_b ? K : N), "mpq_gemm_f64: leading dimension too small");
  MPQ_CHECK_ARG(workspace_bytes >= 0, "mpq_gemm_f64: negative workspace size");
  MPQ_HIP_TRY(mpq::gemm_f64(A, lda, B, ldb, trans_b != 0, C, ldc, M, N, K, alpha, beta, workspace,
                            workspace ? workspace_bytes / (int64_t)sizeof(double) : 0, stream));
  return mpq::kOk;
}
