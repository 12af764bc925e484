// Two-stage tridiagonalisation for mpq_syevd (fp32, gfx950): dense -> band -> tridiagonal.
//
// The one-stage reduction (eigh.hip) reads the whole trailing matrix once per reflector, a
// symmetric matrix-vector product per column (2 n^3 / 3 bytes in total), and is bound by HBM.
// This file reduces to a band first with matrix-core products, then chases the band down to
// tridiagonal form with small cache-resident tasks:
//
// Stage 1 (dense -> band of half-bandwidth kBW = 32), one panel of 32 columns at a time:
//   * the panel below the band, P = A[r0:, c0:c0+32] (m x 32), is factorised as a tall-skinny
//     QR: Householder QR of row blocks of kLeaf rows in LDS (one work-group each), Householder QR
//     of the stacked 32 x 32 R factors in one work-group, the explicit first 32 columns Q1 of the
//     orthogonal factor (LAPACK org2r on the root, then each leaf's reflectors), and Householder
//     vectors reconstructed from Q1 (Ballard, Demmel, Grigori, Jacquelin, Nguyen, Solomonik,
//     "Reconstructing Householder vectors from tall-skinny QR", 2014): Q1 - S = L U with the
//     diagonal sign matrix S chosen during the elimination (|U_ii| >= 1, no pivoting), Y = L,
//     T = -U S Y1^-T, R = S R_tsqr, so P = (I - Y T Y^T) [R; 0];
//   * the trailing matrix takes A22 <- Q^T A22 Q as X = A22 (Y T), W = X - 1/2 Y (T^T Y^T X),
//     A22 -= Y W^T + W Y^T (LAPACK sytrd's update): X from one read of A22's lower triangle on
//     the fp32 matrix cores, the rank-64 update as bf16 x6 products.
// Stage 2 (band -> tridiagonal): bulge chasing (Schwarz 1968; Lang 1993; the task split of Haidar,
//   Ltaief and Dongarra, SC 2011).  Sweep s annihilates column s below the subdiagonal with one
//   reflector (task 0, two-sided on the 32 x 32 diagonal block below); task k >= 1 applies the
//   previous reflector from the right to the 32 x 32 block O below the band (this fills O: the
//   bulge), builds a reflector from O's first column, applies it from the left to O and
//   two-sided to the next diagonal block.  Task (s, k) touches elements of sweep s - 1 only in
//   its tasks k' <= k + 1, so the sweeps run as a pipeline: one wave per sweep, each task started
//   once the previous sweep has finished two more tasks.  A work-group's waves take consecutive
//   sweeps and hand over through LDS counters; work-groups hand over through progress counters in
//   global memory (agent-scope release / acquire), once per NW sweeps.  Every wait is bounded.
// Back-transformation of stage 2: the reflectors of the 32 sweeps of group g at chase step k act
//   on the 63 rows 32 g + 1 + 32 k .. + 62; their product is formed once as an explicit 64 x 64
//   matrix, and the eigenvector matrix takes the blocks in an order that keeps every reflector's
//   position relative to those it overlaps (groups last to first, steps in increasing order), one
//   64 x 64 x 64 MFMA product per block and 64-eigenvector slab.
//
// Band storage: AB[j * kABld + d] = A[j + d][j] for d < 64 (d <= 32 the band, d > 32 the room the
// bulges need), with zero columns past n - 1 so the last tasks read and write zeros there.
#include "eigh_band.h"
#include "gemm.h"
#include "x6_split.h"

namespace mpq {
namespace band {
namespace {

constexpr int kThr = 256;
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kProgStride = 4096;  // progress value = sweep * 4096 + tasks done (4095: finished)
constexpr int kNW = 8;             // waves (sweeps) per bulge-chasing work-group

inline int64_t al64(int64_t v) { return (v + 63) / 64 * 64; }

// ---- stage 1: tall-skinny QR of a panel -------------------------------------------------------

// Panel kernels: 1024 threads; thread (c = t % 32, s = t / 32) holds column c of rows s + 32 q
// (q < R) in registers.  The 32 threads of one row phase s are one half of a wave, so a value of
// column j reaches them by a 32-lane shuffle; the column sums over the 32 row phases are one
// reduction through LDS (double-buffered by step parity: one barrier per reflector).
constexpr int kPThr = 1024;

// Orders one wave's LDS accesses (a compiler barrier plus the wave-scope fences).
__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct PanelLds {
  float red[2][16][32];
  float rowj[2][32];
  float tau[32];
};

// Sum over the 32 row phases of every thread's `acc` (column c), into red[buf]; returns after the
// barrier with the column totals readable by every thread.
__device__ __forceinline__ void phase_reduce(PanelLds& L, int buf, float acc) {
  const int t = threadIdx.x;
  acc += __shfl_xor(acc, 32);
  if (((t >> 5) & 1) == 0) L.red[buf][t >> 6][t & 31] = acc;
  __syncthreads();
}
__device__ __forceinline__ float phase_total(const PanelLds& L, int buf, int c) {
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < 16; ++w) v += L.red[buf][w][c];
  return v;
}

// Householder QR (LAPACK geqr2) of the rows x 32 matrix held in x, k = min(rows, 32) reflectors:
// R on and above the diagonal, v below it (v_j = 1 implied), tau in L.tau.  One reduction per
// reflector gives the norm of column j and every v^T P[:, c] at once (from the unscaled column).
template <int R>
__device__ void reg_geqr2(float (&x)[R], int rows, int k, PanelLds& L) {
  const int t = threadIdx.x, c = t & 31, s = t >> 5;
  for (int j = 0; j < k; ++j) {
    const int buf = j & 1;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float xj = __shfl(x[q], j, 32);
      if (s + 32 * q > j) acc = fmaf(xj, x[q], acc);
    }
    if (s == j) L.rowj[buf][c] = x[0];  // row j of column c (j < 32: phase j, q = 0)
    phase_reduce(L, buf, acc);
    const float dc = phase_total(L, buf, c);
    const float xn2 = phase_total(L, buf, j);
    const float alpha = L.rowj[buf][j];
    float tj = 0.f, beta = alpha, scal = 0.f;
    if (xn2 > 0.f) {
      beta = -copysignf(sqrtf(fmaf(alpha, alpha, xn2)), alpha);
      tj = (beta - alpha) / beta;
      scal = 1.f / (alpha - beta);
    }
    const float w = (c > j) ? tj * (L.rowj[buf][c] + scal * dc) : 0.f;  // tau v^T P[:, c]
    // the shuffle reads column j before its own lanes rescale it (one instruction per q for all lanes)
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float xj = __shfl(x[q], j, 32);
      const int i = s + 32 * q;
      if (c > j) {
        if (i >= j) x[q] = fmaf(-(i == j ? 1.f : xj * scal), w, x[q]);
      } else if (c == j) {
        if (i > j) x[q] *= scal;
        else if (i == j) x[q] = beta;
      }
    }
    if (t == 0) L.tau[j] = tj;
  }
  __syncthreads();
}

// Leaf l of the panel: rows l kLeaf .. of P = A[r0:r0+m, c0:c0+32].  Writes its reflectors (Yl,
// rows of the panel), tau (taul[l * 32 ..], zero past k) and R (Rs rows 32 l .. 32 l + k - 1).
__global__ __launch_bounds__(kPThr) void leaf_qr_kernel(const float* __restrict__ A, int64_t lda, int64_t r0,
                                                        int64_t c0, int64_t m, float* __restrict__ Yl,
                                                        float* __restrict__ taul, float* __restrict__ Rs,
                                                        const int* __restrict__ fallback) {
  if (*fallback != 1) return;  // the Cholesky QR path produced Q1 and R
  constexpr int R = kLeaf / 32;
  __shared__ PanelLds L;
  const int t = threadIdx.x, c = t & 31, s = t >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * kLeaf;
  const int rows = (int)min((int64_t)kLeaf, m - row0);
  const int k = min(rows, 32);
  float x[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    x[q] = i < rows ? A[(r0 + row0 + i) * lda + c0 + c] : 0.f;
  }
  if (t < 32) L.tau[t] = 0.f;
  __syncthreads();
  reg_geqr2<R>(x, rows, k, L);
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    if (i < rows) Yl[(row0 + i) * 32 + c] = x[q];
    if (i < k) Rs[((int64_t)blockIdx.x * 32 + i) * 32 + c] = c >= i ? x[q] : 0.f;
  }
  if (t < 32) taul[blockIdx.x * 32 + t] = L.tau[t];
}

// Root of the TSQR: Householder QR of the stacked R factors (root_rows x 32, root_rows <= 1024),
// R (k x 32, zero below) to Rroot, and E = the first k columns of its orthogonal factor (LAPACK
// org2r; columns k..31 zero) to E (root_rows x 32).
__global__ __launch_bounds__(kPThr) void root_qr_kernel(const float* __restrict__ Rs, int root_rows,
                                                        float* __restrict__ Rroot, float* __restrict__ E,
                                                        const int* __restrict__ fallback) {
  if (*fallback != 1) return;
  constexpr int R = 32;
  __shared__ PanelLds L;
  const int t = threadIdx.x, c = t & 31, s = t >> 5;
  const int rows = root_rows;
  const int k = min(rows, 32);
  float x[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    x[q] = i < rows ? Rs[i * 32 + c] : 0.f;
  }
  if (t < 32) L.tau[t] = 0.f;
  __syncthreads();
  reg_geqr2<R>(x, rows, k, L);
  if (s < 32) Rroot[s * 32 + c] = (s < k && c >= s) ? x[0] : 0.f;  // rows 0..31 are q = 0
  // org2r: for j = k-1 .. 0, apply H_j to columns j+1 .. k-1 (rows >= j; their row j is zero, set
  // when they were finished), then column j becomes -tau_j v below the diagonal, 1 - tau_j on it
  // and zero above.
  for (int j = k - 1; j >= 0; --j) {
    const int buf = j & 1;
    const float tj = L.tau[j];
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float vj = __shfl(x[q], j, 32);
      if (s + 32 * q > j) acc = fmaf(vj, x[q], acc);
    }
    phase_reduce(L, buf, acc);
    const float w = (c > j && c < k) ? tj * phase_total(L, buf, c) : 0.f;
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const float vj = __shfl(x[q], j, 32);
      const int i = s + 32 * q;
      if (c > j && c < k) {
        if (i >= j) x[q] = fmaf(-(i == j ? 1.f : vj), w, x[q]);
      } else if (c == j) {
        x[q] = i > j ? -tj * x[q] : (i == j ? 1.f - tj : 0.f);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    if (i < rows) E[i * 32 + c] = c < k ? x[q] : 0.f;
  }
}

// Q1 rows of leaf l: Q_leaf [E_l; 0] with E_l = E rows 32 l .. 32 l + k_l - 1 (the leaf's
// reflectors applied last to first).
__global__ __launch_bounds__(kPThr) void leaf_q_kernel(const float* __restrict__ Yl, const float* __restrict__ taul,
                                                       const float* __restrict__ E, int64_t m,
                                                       float* __restrict__ Q1, const int* __restrict__ fallback) {
  if (*fallback != 1) return;
  constexpr int R = kLeaf / 32;
  __shared__ PanelLds L;
  const int t = threadIdx.x, c = t & 31, s = t >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * kLeaf;
  const int rows = (int)min((int64_t)kLeaf, m - row0);
  const int k = min(rows, 32);
  float v[R], b[R];
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    v[q] = i < rows ? Yl[(row0 + i) * 32 + c] : 0.f;
    b[q] = i < k ? E[((int64_t)blockIdx.x * 32 + i) * 32 + c] : 0.f;
  }
  for (int j = k - 1; j >= 0; --j) {
    const float tj = taul[blockIdx.x * 32 + j];
    if (tj == 0.f) continue;  // uniform
    const int buf = j & 1;
    float vj[R];
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const int i = s + 32 * q;
      const float sh = __shfl(v[q], j, 32);
      vj[q] = i == j ? 1.f : (i > j ? sh : 0.f);
      acc = fmaf(vj[q], b[q], acc);
    }
    phase_reduce(L, buf, acc);
    const float w = tj * phase_total(L, buf, c);
#pragma unroll
    for (int q = 0; q < R; ++q) b[q] = fmaf(-vj[q], w, b[q]);
  }
#pragma unroll
  for (int q = 0; q < R; ++q) {
    const int i = s + 32 * q;
    if (i < rows) Q1[(row0 + i) * 32 + c] = b[q];
  }
}

// ---- stage 1 fast path: shifted Cholesky QR, three passes ----------------------------------------
// Q1 R = P by Cholesky factorisations of 32 x 32 Gram matrices formed in fp64 (Fukaya, Kannan,
// Nakatsukasa, Yamamoto, Yanagisawa, "Shifted Cholesky QR for computing the QR factorization of
// ill-conditioned matrices", SIAM J. Sci. Comput. 2020): pass 1 factors P^T P + s I with
// s = 11 (32 m + 32 * 33) 2^-53 |P|_F^2, passes 2 and 3 refactor the Gram matrix of the current Q
// (Cholesky QR2).  R = R3 R2 R1.  When the Gram matrix of pass 2 is already within 2e-4 of I, the
// pass-2 factor is orthonormal to working precision and pass 3 is skipped (flag 2, R = R2 R1).  A
// pass whose Cholesky factorisation meets a pivot <= 0, or a last pass whose Gram matrix is not
// close to the identity, sets the panel's fallback flag to 1: then the tall-skinny Householder QR
// above runs instead (rank-deficient panels, e.g. zero panels).
constexpr int kCqTile = 256;

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const unsigned long long u = __double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
  return __longlong_as_double(((unsigned long long)hi << 32) | lo);
}

// Cholesky G = L L^T of the 32 x 32 Gram matrix in G (fp64 LDS) by wave 0, with the pass's checks
// (pass 1 adds the shift first).  Lane t holds row t in registers; pivots and the pivot column come
// by readlane (loops unrolled, register indices static).  On success the lower triangle of G holds
// L; on failure *bad = 1.
__device__ void cq_cholesky(double (*G)[33], int pass, int64_t m, int* bad) {
  const int t = threadIdx.x;
  if (t >= 64) return;  // caller checks *bad after a block barrier
  double row[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) row[c] = t < 32 ? G[t][c] : 0.0;
  if (pass == 1) {
    double tr = 0.0;
#pragma unroll
    for (int c = 0; c < 32; ++c) tr += readlane_f64(row[c], c);
    const double shift = 11.0 * (32.0 * (double)m + 32.0 * 33.0) * 0x1p-53 * tr;
#pragma unroll
    for (int c = 0; c < 32; ++c)
      if (t == c) row[c] += shift;
  }
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const double d = readlane_f64(row[i], i);
    ok = ok && d > 0.0 && (pass != 3 || (d > 0.5 && d < 2.0));
    // 1 / sqrt by the hardware estimate (v_rsq_f64, ~2^-28) and two Newton steps (full precision),
    // a shorter latency chain than sqrt followed by a division
    const double dd = ok ? d : 1.0;
    double inv = __builtin_amdgcn_rsq(dd);
    inv = inv * fma(-0.5 * dd, inv * inv, 1.5);
    inv = inv * fma(-0.5 * dd, inv * inv, 1.5);
    const double lii = dd * inv;
    const double lti = row[i] * inv;  // L[t][i] for t > i
    if (t == i) row[i] = lii;
    else if (t > i) row[i] = lti;
#pragma unroll
    for (int c = i + 1; c < 32; ++c) {
      const double lci = readlane_f64(lti, c);  // L[c][i]
      if (t >= c) row[c] = fma(-lti, lci, row[c]);
    }
  }
  if (!ok) {
    if (t == 0) *bad = 1;
    return;
  }
  if (t < 32)
#pragma unroll
    for (int c = 0; c < 32; ++c) G[t][c] = row[c];
}

// Rows of the work-group's chunk: y = p R^-1 (R upper triangular, fp64; none in pass 1) stored to
// Qout, and the partial Gram sum y^T y in fp64 (rows staged in LDS as fp64; thread (g, bi, bj)
// sums the 4 x 4 block (4 bi.., 4 bj..) over rows g (mod 4) of a tile, the four row groups are
// added in order at the end).  The last work-group to finish (atomic counter) sums the partials in
// work-group order, factors them (pass chol_pass), writes R to Rcur for the next launch and
// R_tot <- R R_tot (last pass: R_tot to Rroot in fp32), or raises the fallback flag.  Every
// work-group reads Rcur before it counts itself in, so rewriting it is safe.
constexpr int kCqLd = 34;  // fp64 row stride of the staged tile (16-byte aligned rows)
__global__ __launch_bounds__(kThr) void cq_pass_kernel(const float* __restrict__ src, int64_t ld, int64_t m,
                                                       int64_t chunk, double* __restrict__ Rcur,
                                                       int use_rcur, float* __restrict__ Qout,
                                                       double* __restrict__ Gp, int chol_pass,
                                                       double* __restrict__ Rtot, float* __restrict__ Rroot,
                                                       int* __restrict__ fallback, unsigned* __restrict__ counter) {
  if (*fallback != 0) return;
  __shared__ double sR[32][33];
  __shared__ __align__(16) double tile[kCqTile * kCqLd];
  __shared__ double G[32][33];
  __shared__ int bad, last;
  const int t = threadIdx.x;
  __shared__ double sRinv[32];
  if (use_rcur) {
    for (int e = t; e < 1024; e += kThr) sR[e >> 5][e & 31] = Rcur[e];
    if (t < 32) sRinv[t] = 1.0 / Rcur[t * 33];
  }
  __syncthreads();
  const int64_t rbeg = (int64_t)blockIdx.x * chunk;
  const int64_t rend = min(m, rbeg + chunk);
  const int grp = t >> 6, bi = (t >> 3) & 7, bj = t & 7;
  double acc[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) acc[q] = 0.0;
  for (int64_t r0 = rbeg; r0 < rend; r0 += kCqTile) {
    const int64_t r = r0 + t;
    double yd[32];
    if (r < rend) {
      float y[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) y[j] = src[r * ld + j];
      if (use_rcur) {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          double a = (double)y[j];
#pragma unroll
          for (int i = 0; i < j; ++i) a = fma(-yd[i], sR[i][j], a);
          yd[j] = a * sRinv[j];
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          y[j] = (float)yd[j];
          Qout[r * 32 + j] = y[j];
        }
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) yd[j] = (double)y[j];
    } else {
#pragma unroll
      for (int j = 0; j < 32; ++j) yd[j] = 0.0;
    }
    if (chol_pass > 0) {
#pragma unroll
      for (int j = 0; j < 32; j += 2)
        *reinterpret_cast<double2*>(&tile[t * kCqLd + j]) = make_double2(yd[j], yd[j + 1]);
      __syncthreads();
      const int rows = (int)min((int64_t)kCqTile, rend - r0);
      for (int rr = grp; rr < rows; rr += 4) {
        const double* row = &tile[rr * kCqLd];
        const double2 i01 = *reinterpret_cast<const double2*>(row + 4 * bi);
        const double2 i23 = *reinterpret_cast<const double2*>(row + 4 * bi + 2);
        const double2 j01 = *reinterpret_cast<const double2*>(row + 4 * bj);
        const double2 j23 = *reinterpret_cast<const double2*>(row + 4 * bj + 2);
        const double yi[4] = {i01.x, i01.y, i23.x, i23.y};
        const double yj[4] = {j01.x, j01.y, j23.x, j23.y};
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a * 4 + b] = fma(yi[a], yj[b], acc[a * 4 + b]);
      }
      __syncthreads();
    }
  }
  if (chol_pass == 0) return;
  {
    // the four row groups' blocks, added in group order
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) tile[grp * 1024 + (4 * bi + a) * 32 + 4 * bj + b] = acc[a * 4 + b];
    __syncthreads();
    double* gp = Gp + (int64_t)blockIdx.x * 1024;
    for (int e = t; e < 1024; e += kThr) gp[e] = ((tile[e] + tile[1024 + e]) + tile[2048 + e]) + tile[3072 + e];
  }
  // the last work-group to finish reduces and factors
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned prev = atomicAdd(counter, 1u);
    last = prev == gridDim.x - 1;
    bad = 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();  // acquire: the partials of every work-group are visible to plain loads
  // lower triangle only (the factorisation reads no other entry), partials added in work-group
  // order, 16 of them in flight per entry
  const int ng = (int)gridDim.x;
  {
    double a4[4] = {0.0, 0.0, 0.0, 0.0};
    for (int g0 = 0; g0 < ng; g0 += 16) {
      double v[4][16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = t + q * kThr;
        const bool low = (e >> 5) >= (e & 31);
#pragma unroll
        for (int u = 0; u < 16; ++u) v[q][u] = (low && g0 + u < ng) ? Gp[(int64_t)(g0 + u) * 1024 + e] : 0.0;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 16; ++u) a4[q] += v[q][u];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = t + q * kThr;
      G[e >> 5][e & 31] = a4[q];
    }
  }
  if (t == 0) *counter = 0u;  // ready for the next launch
  __syncthreads();
  // pass 2: the Gram matrix of the pass-1 factor measures how far it is from orthonormal; within
  // 2e-4 of I, the pass-2 factor is orthonormal to working precision and pass 3 is skipped
  if (chol_pass == 2) {
    double dev = 0.0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = t + q * kThr, i = e >> 5, j = e & 31;
      if (i >= j) dev = fmax(dev, fabs(G[i][j] - (i == j ? 1.0 : 0.0)));
    }
    for (int off = 32; off >= 1; off >>= 1) dev = fmax(dev, __shfl_xor(dev, off));
    if ((t & 63) == 0) sRinv[t >> 6] = dev;  // scratch (sRinv is not used after the rows)
  }
  cq_cholesky(G, chol_pass, m, &bad);
  __syncthreads();
  if (bad) {
    if (t == 0) *fallback = 1;
    return;
  }
  const bool converged =
      chol_pass == 2 && fmax(fmax(sRinv[0], sRinv[1]), fmax(sRinv[2], sRinv[3])) < 2e-4;
  // R = L^T (upper); R_tot <- R R_tot
  for (int e = t; e < 1024; e += kThr) {
    const int i = e >> 5, j = e & 31;
    Rcur[e] = j >= i ? G[j][i] : 0.0;
  }
  if (chol_pass == 1) {
    for (int e = t; e < 1024; e += kThr) {
      const int i = e >> 5, j = e & 31;
      Rtot[e] = j >= i ? G[j][i] : 0.0;
    }
    return;
  }
  for (int e = t; e < 1024; e += kThr) sR[e >> 5][e & 31] = Rtot[e];
  __syncthreads();
  for (int e = t; e < 1024; e += kThr) {
    const int i = e >> 5, j = e & 31;
    double a = 0.0;
    for (int l = i; l <= j; ++l) a = fma(G[l][i], sR[l][j], a);  // R[i][l] = L[l][i]
    Rtot[e] = j >= i ? a : 0.0;
    if (chol_pass == 3 || converged) Rroot[e] = j >= i ? (float)a : 0.f;
  }
  if (converged && t == 0) *fallback = 2;  // pass 3 returns at once; hr_kernel applies R2
}

// Householder reconstruction from Q1 (m x 32, kk = min(m, 32) columns used) and the panel's
// results.  On the Cholesky QR path Q1 still lacks the last factor (Rc, fp64): every row is first
// solved with it; after the tall-skinny fallback (flag 1) Q1 is final.  Every work-group factors
// the kk x kk top block redundantly and then handles 256 panel rows: Y row = L row (top block) or
// Q1 row U^-1, B row = Y row T (packed into BP); the reflectors go to the rows of A (row c0 + j holds Y[r][j] at
// column r0 + r, r > j).  Work-group 0 also writes T, tau and the band block
// A[r0 + i][c0 + j] = (S R)[i][j] (j >= i, zero below).
__device__ __forceinline__ void hr_q1_row(const float* __restrict__ q, const double (*sR)[33], const double* sRinv,
                                          bool apply, float (&out)[32]) {
  if (!apply) {
#pragma unroll
    for (int j = 0; j < 32; ++j) out[j] = q[j];
    return;
  }
  double yd[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    double a = (double)q[j];
#pragma unroll
    for (int i = 0; i < j; ++i) a = fma(-yd[i], sR[i][j], a);
    yd[j] = a * sRinv[j];
    out[j] = (float)yd[j];
  }
}

__global__ __launch_bounds__(kThr) void hr_kernel(const float* __restrict__ Q1, const double* __restrict__ Rc,
                                                  const int* __restrict__ fallback, const float* __restrict__ Rroot,
                                                  int64_t m, float* __restrict__ A, int64_t lda, int64_t r0,
                                                  int64_t c0, float* __restrict__ Y, float* __restrict__ BP,
                                                  float* __restrict__ Tout, float* __restrict__ tau) {
  __shared__ float LU[32][33];
  __shared__ float Xi[32][33];  // L1^-T
  __shared__ float Ts[32][33];
  __shared__ float S[32];
  __shared__ float Uinv[32];  // 1 / U[j][j]
  __shared__ double sR[32][33];
  __shared__ double sRinv[32];
  const int kk = (int)min<int64_t>(m, 32);
  const int t = threadIdx.x;
  const bool apply = *fallback != 1;
  if (apply) {
    for (int e = t; e < 1024; e += kThr) sR[e >> 5][e & 31] = Rc[e];
    if (t < 32) sRinv[t] = 1.0 / Rc[t * 33];
  }
  __syncthreads();
  if (t < 32) {
    float q[32];
    if (t < kk) hr_q1_row(Q1 + t * 32, sR, sRinv, apply, q);
#pragma unroll
    for (int j = 0; j < 32; ++j) LU[t][j] = (t < kk && j < kk) ? q[j] : 0.f;
  }
  __syncthreads();
  // LU without pivoting of Q1 - S, S_i = -sign of the current pivot (|U_ii| >= 1), then L1^-1:
  // wave 0, lane r holds row r in registers, pivot rows by readlane (loops unrolled: register
  // indices are static)
  if (t < 64) {
    float row[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) row[c] = t < 32 ? LU[t][c] : 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i < kk) {
        // pivot row i, read by every lane before any lane changes its registers
        float prow[32];
#pragma unroll
        for (int c = i; c < 32; ++c) prow[c] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(row[c]), i));
        const float si = prow[i] >= 0.f ? -1.f : 1.f;
        const float p = prow[i] - si;
        if (t == i) row[i] = p;
        if (t > i && t < kk) {
          const float l = row[i] / p;
          row[i] = l;
#pragma unroll
          for (int c = i + 1; c < 32; ++c) row[c] = fmaf(-l, prow[c], row[c]);
        }
        if (t == 0) S[i] = si;
      }
    }
    // L1^-1 (unit lower): row t = e_t - sum_{c < t} L1[t][c] (row c), rows in increasing order
    float inv[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) inv[c] = t == c ? 1.f : 0.f;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      if (c < kk) {
        float ic[32];
#pragma unroll
        for (int k = 0; k <= c; ++k) ic[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv[k]), c));
        const float l = (t > c && t < kk) ? row[c] : 0.f;
#pragma unroll
        for (int k = 0; k <= c; ++k) inv[k] = fmaf(-l, ic[k], inv[k]);
      }
    }
    if (t < 32) {
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        LU[t][c] = row[c];
        Xi[c][t] = t < kk ? inv[c] : 0.f;  // Xi = (L1^-1)^T
      }
    }
  }
  __syncthreads();
  // T = -U S Xi (upper)
  for (int e = t; e < 32 * 32; e += kThr) {
    const int i = e / 32, j = e & 31;
    float acc = 0.f;
    if (i <= j && j < kk)
      for (int l = i; l <= j; ++l) acc = fmaf(LU[i][l] * S[l], Xi[l][j], acc);
    Ts[i][j] = -acc;
  }
  if (t < 32) Uinv[t] = t < kk ? 1.0f / LU[t][t] : 0.f;
  __syncthreads();
  const int64_t r = (int64_t)blockIdx.x * kThr + t;
  if (r < m) {
    float y[32];
    if (r < kk) {
#pragma unroll
      for (int j = 0; j < 32; ++j) y[j] = j < r ? LU[r][j] : (j == r ? 1.f : 0.f);
    } else {
      float q[32];
      hr_q1_row(Q1 + r * 32, sR, sRinv, apply, q);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        float acc = j < kk ? q[j] : 0.f;
        for (int i = 0; i < j; ++i) acc = fmaf(-y[i], LU[i][j], acc);
        y[j] = j < kk ? acc * Uinv[j] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) Y[r * 32 + j] = y[j];
    // B = Y T, packed for xsym_kernel: BP[r / 32][lane (j, h = r / 16 % 2)][r % 16]
    float* bp = BP + (r >> 5) * 1024 + 512 * ((r >> 4) & 1) + (r & 15);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      float acc = 0.f;
      for (int i = 0; i <= j; ++i) acc = fmaf(y[i], Ts[i][j], acc);
      bp[16 * j] = acc;
    }
    for (int j = 0; j < kk && j < r; ++j) A[(c0 + j) * lda + r0 + r] = y[j];
  } else {  // rows m .. of the last 256-row block: zero operand rows
    float* bp = BP + (r >> 5) * 1024 + 512 * ((r >> 4) & 1) + (r & 15);
#pragma unroll
    for (int j = 0; j < 32; ++j) bp[16 * j] = 0.f;
  }
  if (blockIdx.x == 0) {
    for (int e = t; e < 32 * 32; e += kThr) Tout[e] = Ts[e / 32][e & 31];
    if (t < 32) tau[c0 + t] = t < kk ? Ts[t][t] : 0.f;
    const int rows = kk;
    for (int e = t; e < rows * 32; e += kThr) {
      const int i = e / 32, j = e & 31;
      A[(r0 + i) * lda + c0 + j] = j >= i ? S[i] * Rroot[i * 32 + j] : 0.f;
    }
  }
}

// X = the split-K partials of X = A22 (Y T) added in split order (8 loads in flight per element).
__global__ __launch_bounds__(kThr) void xsum_kernel(const float* __restrict__ P, int splits, int64_t cnt,
                                                    float* __restrict__ X) {
  const int64_t e = (int64_t)blockIdx.x * kThr + threadIdx.x;
  if (e >= cnt) return;
  float a = 0.f;
  for (int s0 = 0; s0 < splits; s0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = s0 + u < splits ? P[(int64_t)(s0 + u) * cnt + e] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) a += v[u];
  }
  X[e] = a;
}

// Partial grams over the rows of chunk g on the fp32 matrix cores: Gp[g][0] = Y^T X, and when the
// panel is the second of a pair also Gp[g][1] = Y^T Yh and Gp[g][2] = Y^T Wh (Yh, Wh: the first
// panel's Y and W from the row where this panel's rows start); np = 1 or 3 products per chunk.  Wave
// w takes rows 8 t + 2 w + h of the chunk (lane (i, h) feeds Y[row][i] and X[row][i] to MFMA step t);
// the four waves' 32 x 32 results are added through LDS in wave order.
__global__ __launch_bounds__(kThr) void gram_partial_kernel(const float* __restrict__ Y, const float* __restrict__ X,
                                                            int64_t m, int64_t chunk, float* __restrict__ Gp,
                                                            const float* __restrict__ Yh,
                                                            const float* __restrict__ Wh) {
  __shared__ float red[4][3][1024];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, i = lane & 31, h = lane >> 5;
  const bool three = Yh != nullptr;
  const int np = three ? 3 : 1;
  const int64_t rbeg = (int64_t)blockIdx.x * chunk;
  const int64_t rend = min(m, rbeg + chunk);
  floatx16 acc[3];
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[q][v] = 0.f;
  for (int64_t k0 = rbeg; k0 < rend; k0 += 64) {  // 8 steps of 8 rows, loads first
    float ya[8], xa[8], ha[8], wa[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t k = k0 + 8 * u + 2 * w + h;
      const bool in = k < rend;
      const int64_t kc = in ? k : rbeg;
      ya[u] = in ? Y[kc * 32 + i] : 0.f;
      xa[u] = in ? X[kc * 32 + i] : 0.f;
      if (three) {
        ha[u] = in ? Yh[kc * 32 + i] : 0.f;
        wa[u] = in ? Wh[kc * 32 + i] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ya[u], xa[u], acc[0], 0, 0, 0);
      if (three) {
        acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(ya[u], ha[u], acc[1], 0, 0, 0);
        acc[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(ya[u], wa[u], acc[2], 0, 0, 0);
      }
    }
  }
  for (int q = 0; q < np; ++q)
#pragma unroll
    for (int v = 0; v < 16; ++v) red[w][q][(8 * (v >> 2) + 4 * h + (v & 3)) * 32 + i] = acc[q][v];
  __syncthreads();
  for (int q = 0; q < np; ++q)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int e = t + e4 * kThr;
      Gp[((int64_t)blockIdx.x * np + q) * 1024 + e] = ((red[0][q][e] + red[1][q][e]) + red[2][q][e]) + red[3][q][e];
    }
}

// M = T^T (sum_g Gp[g]) (32 x 32): one work-group of 1024 threads, one entry each.  For the second
// panel of a pair (np = 3) X is the product of the not yet updated matrix, X = X^ - Yh G1 - Wh G2
// with G1 = (Y^T Wh)^T T and G2 = (Y^T Yh)^T T (Yh G1 + Wh G2 is the first panel's update applied to
// this panel's B = Y T); then Y^T X = S1 - S2 G1 - S3 G2 (S1 = Y^T X^, S2 = Y^T Yh, S3 = Y^T Wh), and
// G1, G2 go to Gout for w_kernel.
__global__ __launch_bounds__(1024) void m_kernel(const float* __restrict__ Gp, int ng, int np,
                                                 const float* __restrict__ T, float* __restrict__ Mout,
                                                 float* __restrict__ Gout) {
  __shared__ float S[3][32][33];
  __shared__ float Gc[2][32][33];
  __shared__ float sT[32][33];
  const int e = threadIdx.x, i = e >> 5, j = e & 31;
  sT[i][j] = T[e];
  for (int pr = 0; pr < np; ++pr) {
    float a = 0.f;
    for (int g0 = 0; g0 < ng; g0 += 16) {  // 16 loads in flight, added in partial order
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = g0 + u < ng ? Gp[((int64_t)(g0 + u) * np + pr) * 1024 + e] : 0.f;
#pragma unroll
      for (int u = 0; u < 16; ++u) a += v[u];
    }
    S[pr][i][j] = a;
  }
  __syncthreads();
  if (np == 3) {
    float g1 = 0.f, g2 = 0.f;
    for (int l = 0; l < 32; ++l) {
      g1 = fmaf(S[2][l][i], sT[l][j], g1);
      g2 = fmaf(S[1][l][i], sT[l][j], g2);
    }
    Gc[0][i][j] = g1;
    Gc[1][i][j] = g2;
    Gout[e] = g1;
    Gout[1024 + e] = g2;
    __syncthreads();
    float c = S[0][i][j];
    for (int l = 0; l < 32; ++l) c -= S[1][i][l] * Gc[0][l][j] + S[2][i][l] * Gc[1][l][j];
    __syncthreads();
    S[0][i][j] = c;
    __syncthreads();
  }
  float mv = 0.f;
  for (int l = 0; l < 32; ++l) mv = fmaf(sT[l][i], S[0][l][j], mv);
  Mout[e] = mv;
}

// W = X - 1/2 Y M and the operands of the trailing update A22 -= [Y W] [W Y]^T as three bf16 planes
// (exact split, see x6_split.h): Xp holds -[Y W], Yp holds [W Y], both in the operand order of
// v_mfma_f32_32x32x16_bf16 with ks 16-k steps (K = 16 ks), per 32-row tile T chunk (plane p, step s,
// lane l) at T * 3 ks 64 + (p ks + s) * 64 + l = row 32 T + l % 32, k = 16 s + 8 (l / 32) + 0 .. 7.
// This panel's Y fills the 8-k chunks cy .. cy + 3 of Xp (W those of Yp) and W the chunks cw .. cw + 3
// (Y those of Yp): a lone panel takes K = 64 (cy 0, cw 4); a pair of panels shares K = 128.  Row r
// goes to packed row r - row_off (the first panel of a pair packs its rows from the second panel's
// origin, row_off = 32); packed rows past m are zero, up to a multiple of 128.  Wout (optional) gets
// W in fp32.  With Gc (the second panel of a pair), X is the product of the not yet updated matrix
// and W -= Yh G1 + Wh G2 (see m_kernel).
__global__ __launch_bounds__(kThr) void w_kernel(const float* __restrict__ Mg, const float* __restrict__ Y,
                                                 const float* __restrict__ X, int64_t m, uint4* __restrict__ Xp,
                                                 uint4* __restrict__ Yp, int ks, int cy, int cw, int row_off,
                                                 float* __restrict__ Wout, const float* __restrict__ Yh,
                                                 const float* __restrict__ Wh, const float* __restrict__ Gc) {
  __shared__ float M[3][32][33];
  const int t = threadIdx.x;
  for (int e = t; e < 1024; e += kThr) M[0][e >> 5][e & 31] = Mg[e];
  if (Gc) {
    for (int e = t; e < 1024; e += kThr) {
      M[1][e >> 5][e & 31] = Gc[e];
      M[2][e >> 5][e & 31] = Gc[1024 + e];
    }
  }
  __syncthreads();
  // four threads per row: quarter q computes W's columns 8 q .. 8 q + 7 and packs chunk q of Y and W
  const int q = t & 3;
  const int64_t r = (int64_t)blockIdx.x * (kThr / 4) + (t >> 2);
  if (r >= row_off + (m - row_off + 127) / 128 * 128) return;  // packed rows: rounded up to 128
  float yq[8], wq[8];
  if (r < m) {
    float y[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) y[j] = Y[r * 32 + j];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = 8 * q + jj;
      float a = 0.f;
      for (int l = 0; l < 32; ++l) a = fmaf(y[l], M[0][l][j], a);
      wq[jj] = fmaf(-0.5f, a, X[r * 32 + j]);
      yq[jj] = y[j];
    }
    if (Gc) {
      float yh[32], wh[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        yh[j] = Yh[r * 32 + j];
        wh[j] = Wh[r * 32 + j];
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = 8 * q + jj;
        float c = 0.f;
        for (int l = 0; l < 32; ++l) c = fmaf(yh[l], M[1][l][j], fmaf(wh[l], M[2][l][j], c));
        wq[jj] -= c;
      }
    }
    if (Wout) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) Wout[r * 32 + 8 * q + jj] = wq[jj];
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      yq[jj] = 0.f;
      wq[jj] = 0.f;
    }
  }
  if (r < row_off) return;
  const int64_t pr = r - row_off;
  const int tile = 3 * ks * 64;
  uint4* xo = Xp + (pr >> 5) * tile + (pr & 31);
  uint4* yo = Yp + (pr >> 5) * tile + (pr & 31);
#pragma unroll
  for (int part = 0; part < 2; ++part) {  // chunk q of Y (part 0) and of W (part 1)
    const float* src = part == 0 ? yq : wq;  // [Y W]
    const float* srb = part == 0 ? wq : yq;  // [W Y]
    const int cc = part == 0 ? cy + q : cw + q;
    uint4 h, mm, l, hb, mb, lb;
    split3(-src[0], -src[1], h.x, mm.x, l.x);
    split3(-src[2], -src[3], h.y, mm.y, l.y);
    split3(-src[4], -src[5], h.z, mm.z, l.z);
    split3(-src[6], -src[7], h.w, mm.w, l.w);
    split3(srb[0], srb[1], hb.x, mb.x, lb.x);
    split3(srb[2], srb[3], hb.y, mb.y, lb.y);
    split3(srb[4], srb[5], hb.z, mb.z, lb.z);
    split3(srb[6], srb[7], hb.w, mb.w, lb.w);
    const int off = (cc >> 1) * 64 + (cc & 1) * 32;
    xo[off] = h;
    xo[ks * 64 + off] = mm;
    xo[2 * ks * 64 + off] = l;
    yo[off] = hb;
    yo[ks * 64 + off] = mb;
    yo[2 * ks * 64 + off] = lb;
  }
}

// The first panel of a pair updates the second panel's columns before that panel is factorised:
// A22[r][c] -= sum_k Y[r][k] W[c][k] + W[r][k] Y[c][k] for rows r < m, columns c < 32 (fp32; the rest
// of A22 takes this panel's update together with the second panel's).  8 rows per work-group.
__global__ __launch_bounds__(kThr) void colblock_kernel(float* __restrict__ A22, int64_t lda, int64_t m,
                                                        const float* __restrict__ Y, const float* __restrict__ W) {
  __shared__ float sYc[32][33], sWc[32][33], sYr[8][33], sWr[8][33];
  const int t = threadIdx.x, rr = t >> 5, c = t & 31;
  const int64_t r0 = (int64_t)blockIdx.x * 8;
  for (int e = t; e < 1024; e += kThr) {
    const int i = e >> 5, j = e & 31;
    sYc[i][j] = i < m ? Y[i * 32 + j] : 0.f;
    sWc[i][j] = i < m ? W[i * 32 + j] : 0.f;
  }
  {
    const int64_t r = r0 + rr;
    sYr[rr][c] = r < m ? Y[r * 32 + c] : 0.f;
    sWr[rr][c] = r < m ? W[r * 32 + c] : 0.f;
  }
  __syncthreads();
  const int64_t r = r0 + rr;
  if (r >= m || c >= m) return;
  float a = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) a = fmaf(sYr[rr][k], sWc[c][k], fmaf(sWr[rr][k], sYc[c][k], a));
  A22[r * lda + c] -= a;
}

// A22 += (-[Y W]) [W Y]^T on every 128 x 128 tile (ti, tj) with tj <= ti (the lower triangle and
// whole diagonal tiles; entries above the diagonal are never read).  One work-group per tile
// (triangular index), wave (wr, wc) owns the 64 x 64 quarter (two by two 32 x 32 MFMA tiles): the
// fp32 tile is loaded straight into the accumulators, then K = 16 KS (64 for one panel, 128 for a
// pair) in 16-k steps of six bf16 plane products, then stored.
template <int KS>
__global__ __launch_bounds__(kThr) void syr2k_x6_kernel(const uint4* __restrict__ Xp, const uint4* __restrict__ Yp,
                                                        float* __restrict__ A, int64_t lda, int64_t m) {
  constexpr int kTile = 3 * KS * 64;  // uint4 per 32-row tile of a packed operand
  const int64_t b = blockIdx.x;
  int64_t ti = (int64_t)((sqrt(8.0 * (double)b + 1.0) - 1.0) * 0.5);
  while ((ti + 1) * (ti + 2) / 2 <= b) ++ti;
  while (ti * (ti + 1) / 2 > b) --ti;
  const int64_t tj = b - ti * (ti + 1) / 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t R0 = 128 * ti + 64 * wr, C0 = 128 * tj + 64 * wc;
  const int col = lane & 31, rq = 4 * (lane >> 5);
  floatx16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int64_t c = C0 + 32 * y + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t r = R0 + 32 * x + 8 * (v >> 2) + rq + (v & 3);
        acc[x][y][v] = (r < m && c < m) ? A[r * lda + c] : 0.f;
      }
    }
  const uint4* xa = Xp + (R0 >> 5) * kTile + lane;
  const uint4* yb = Yp + (C0 >> 5) * kTile + lane;
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    bf16x8 av[2][3], bv[2][3];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        av[x][p] = __builtin_bit_cast(bf16x8, xa[x * kTile + (p * KS + st) * 64]);
        bv[x][p] = __builtin_bit_cast(bf16x8, yb[x * kTile + (p * KS + st) * 64]);
      }
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][0], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][1], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][1], bv[y][0], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][2], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][1], bv[y][1], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][2], bv[y][0], acc[x][y], 0, 0, 0);
      }
  }
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int64_t c = C0 + 32 * y + col;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t r = R0 + 32 * x + 8 * (v >> 2) + rq + (v & 3);
        if (r < m && c < m) A[r * lda + c] = acc[x][y][v];
      }
    }
}

// X = A22 B (B = Y T, m x 32) from the lower triangle of A22 (the trailing update keeps the lower
// triangle and the 32 x 32 diagonal blocks current), reading that triangle once.  Work-group t owns
// the lower tile (I, J), I >= J, of kTile = 64 R rows and columns and adds both of its products:
//   rows of block I: A_IJ B_J      -> partial slot J of block I,
//   rows of block J: A_IJ^T B_I    -> partial slot I of block J (I > J),
// and a diagonal tile (I = J) puts the sum of both over its lower 32 x 32 blocks (the diagonal blocks
// counted once, as stored) into slot I of block I.  Every (slot s, block K) is written by exactly one
// work-group -- tile (K, s) for s <= K, tile (s, K) for s > K -- so X = the sum over the slots in
// slot order, as xsum_kernel adds them.
//
// The four waves split the tile into 2 x 2 sub-blocks of 32 R rows.  A wave walks its sub-block in
// 32 x 32 blocks: lane (r, h) loads A[r][16 h .. 16 h + 15] (four float4) and feeds the row product
// with k = 16 h + s on MFMA step s; the same block, transposed through the wave's own LDS buffer,
// feeds the column product (lane (c, h): A[16 h + s][c]).  Both B operands come packed by hr_kernel
// (BP[32-row block][lane (j, h)][s] = B[32 blk + 16 h + s][j]).  The two waves that share a row half
// or a column half of the tile add their partials through LDS at the end.
constexpr int kXsLd = 36;  // row stride (floats) of a wave's 32 x 32 transpose buffer

struct XsBlock {
  float a[16];  // lane (r, h): A[r][16 h + s]
  float4 bi[4], bj[4];
};

template <int R>
__device__ __forceinline__ void xs_load(const float* __restrict__ A, int64_t lda, const float4* __restrict__ BP,
                                        int64_t m, int64_t R0, int64_t C0, int lane, XsBlock& x) {
  const int r = lane & 31, h = lane >> 5;
  if (R0 >= m || C0 >= m) {  // outside the matrix (the last tile row or column only)
#pragma unroll
    for (int s = 0; s < 16; ++s) x.a[s] = 0.f;
  } else {
    const int64_t row = min(R0 + r, m - 1);
    const float4* p = reinterpret_cast<const float4*>(A + row * lda + C0 + 16 * h);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 f = p[q];
      x.a[4 * q] = f.x;
      x.a[4 * q + 1] = f.y;
      x.a[4 * q + 2] = f.z;
      x.a[4 * q + 3] = f.w;
    }
    if (R0 + 32 > m || C0 + 32 > m) {  // crosses the edge: rows and columns >= m are zero
#pragma unroll
      for (int s = 0; s < 16; ++s)
        if (R0 + r >= m || C0 + 16 * h + s >= m) x.a[s] = 0.f;
    }
  }
  const float4* bi = BP + (R0 >> 5) * 256 + lane * 4;
  const float4* bj = BP + (C0 >> 5) * 256 + lane * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    x.bi[q] = bi[q];
    x.bj[q] = bj[q];
  }
}

__device__ __forceinline__ float f4e(const float4* v, int s) {
  const float4 f = v[s >> 2];
  return (s & 3) == 0 ? f.x : (s & 3) == 1 ? f.y : (s & 3) == 2 ? f.z : f.w;
}

// One wave's sub-block: 32 x 32 blocks (a, b), b outer; DIAG: a sub-block on the tile's diagonal
// (blocks above its diagonal skipped, diagonal blocks feed the row product only).
template <int R, bool DIAG>
__device__ __forceinline__ void xs_walk(const float* __restrict__ A, int64_t lda, const float4* __restrict__ BP,
                                        int64_t m, int64_t rowbase, int64_t colbase, float* tb, int lane,
                                        floatx16 (&c1)[R], floatx16 (&c2)[R]) {
  const int r = lane & 31, h = lane >> 5;
  XsBlock cur, nxt;
  xs_load<R>(A, lda, BP, m, rowbase, colbase, lane, cur);  // block (0, 0)
#pragma unroll
  for (int b = 0; b < R; ++b)
#pragma unroll
    for (int a = DIAG ? b : 0; a < R; ++a) {
      // the next block in walk order, loaded before this one's products
      const int na = a + 1 < R ? a + 1 : (DIAG ? b + 1 : 0), nb = a + 1 < R ? b : b + 1;
      if (nb < R) xs_load<R>(A, lda, BP, m, rowbase + 32 * na, colbase + 32 * nb, lane, nxt);
      const bool dblk = DIAG && a == b;
      float at[16];
      if (!dblk) {
        float4* w = reinterpret_cast<float4*>(tb + r * kXsLd + 16 * h);
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = make_float4(cur.a[4 * q], cur.a[4 * q + 1], cur.a[4 * q + 2], cur.a[4 * q + 3]);
#pragma unroll
        for (int s = 0; s < 16; ++s) at[s] = tb[(16 * h + s) * kXsLd + r];
      }
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        c1[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[s], f4e(cur.bj, s), c1[a], 0, 0, 0);
        if (!dblk) c2[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(at[s], f4e(cur.bi, s), c2[b], 0, 0, 0);
      }
      if (nb < R) cur = nxt;
    }
}

template <int R>
__device__ __forceinline__ void xs_put(float* reg, const floatx16 (&c)[R], int lane) {
#pragma unroll
  for (int a = 0; a < R; ++a)
#pragma unroll
    for (int v = 0; v < 16; ++v) reg[(a * 16 + v) * 64 + lane] = c[a][v];
}

// out[slot][rows base .. base + 32 R) = c (+ the partial in reg)
template <int R>
__device__ __forceinline__ void xs_store(float* __restrict__ P, int64_t m, int64_t slot, int64_t base,
                                         const floatx16 (&c)[R], const float* reg, int lane) {
  const int j = lane & 31, h = lane >> 5;
  float* out = P + slot * m * 32;
#pragma unroll
  for (int a = 0; a < R; ++a)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t row = base + 32 * a + 8 * (v >> 2) + 4 * h + (v & 3);
      if (row < m) out[row * 32 + j] = c[a][v] + reg[(a * 16 + v) * 64 + lane];
    }
}

template <int R>
__global__ __launch_bounds__(kThr, 2) void xsym_kernel(const float* __restrict__ A, int64_t lda,
                                                       const float4* __restrict__ BP, int64_t m,
                                                       float* __restrict__ P) {
  constexpr int SB = 32 * R, kTile = 2 * SB, kReg = R * 16 * 64;
  __shared__ float lds[4 * kReg];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int t = (int)blockIdx.x;
  int I = (int)((sqrtf(8.f * (float)t + 1.f) - 1.f) * 0.5f);
  while ((I + 1) * (I + 2) / 2 <= t) ++I;
  while (I * (I + 1) / 2 > t) --I;
  const int J = t - I * (I + 1) / 2;
  const bool diag = I == J;
  const int64_t rowbase = (int64_t)I * kTile + SB * wr, colbase = (int64_t)J * kTile + SB * wc;
  floatx16 c1[R], c2[R];
#pragma unroll
  for (int a = 0; a < R; ++a)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      c1[a][v] = 0.f;
      c2[a][v] = 0.f;
    }
  float* tb = lds + wave * kReg;
  if (!diag)
    xs_walk<R, false>(A, lda, BP, m, rowbase, colbase, tb, lane, c1, c2);
  else if (wr == wc)
    xs_walk<R, true>(A, lda, BP, m, rowbase, colbase, tb, lane, c1, c2);
  else if (wr > wc)
    xs_walk<R, false>(A, lda, BP, m, rowbase, colbase, tb, lane, c1, c2);
  __syncthreads();
  float* L0 = lds;
  float* L1 = lds + kReg;
  float* L2 = lds + 2 * kReg;
  float* L3 = lds + 3 * kReg;
  if (!diag) {
    // row half wr: (wr, 0) + (wr, 1); column half wc: (0, wc) + (1, wc)
    if (wave == 1) {
      xs_put<R>(L0, c1, lane);
      xs_put<R>(L3, c2, lane);
    } else if (wave == 3) {
      xs_put<R>(L1, c1, lane);
    } else if (wave == 0) {
      xs_put<R>(L2, c2, lane);
    }
    __syncthreads();
    const int64_t bI = (int64_t)I * kTile, bJ = (int64_t)J * kTile;
    if (wave == 0) {
      xs_store<R>(P, m, J, bI, c1, L0, lane);
    } else if (wave == 2) {
      xs_store<R>(P, m, J, bI + SB, c1, L1, lane);
      xs_store<R>(P, m, I, bJ, c2, L2, lane);
    } else if (wave == 3) {
      xs_store<R>(P, m, I, bJ + SB, c2, L3, lane);
    }
  } else {
    // rows 0 .. SB: (0, 0)'s both products + (1, 0)'s column product; rows SB ..: (1, 0)'s row
    // product + (1, 1)'s both products
    if (wave == 2) {
      xs_put<R>(L2, c2, lane);
      xs_put<R>(L1, c1, lane);
    }
    __syncthreads();
    const int64_t bI = (int64_t)I * kTile;
    if (wave == 0 || wave == 3) {
      floatx16 s[R];
#pragma unroll
      for (int a = 0; a < R; ++a) s[a] = c1[a] + c2[a];
      xs_store<R>(P, m, I, bI + (wave == 3 ? SB : 0), s, wave == 3 ? L1 : L2, lane);
    }
  }
}

// ---- stage 2: bulge chasing ------------------------------------------------------------------

// AB[j][d] = A[j + d][j] for d <= kBW inside the matrix, zero elsewhere (columns up to n + kABpad).
__global__ __launch_bounds__(kThr) void band_extract_kernel(const float* __restrict__ A, int64_t lda, int64_t n,
                                                            float* __restrict__ AB) {
  const int64_t e = (int64_t)blockIdx.x * kThr + threadIdx.x;
  if (e >= (n + kABpad) * kABld) return;
  const int64_t j = e / kABld;
  const int d = (int)(e % kABld);
  AB[e] = (d <= kBW && j + d < n) ? A[(j + d) * lda + j] : 0.f;
}

// Wave sums without LDS: rotate-and-add inside each 16-lane row (DPP row_ror 8, 4, 2, 1), then the
// row pairs and the two halves through v_permlane16_swap / v_permlane32_swap, whose two results
// hold the even/odd row (lower/upper half) of each pair, so their sum is own + partner.  Every lane
// adds the same operands (only commuted), so every lane holds the same bits.
template <int kCtrl>
__device__ __forceinline__ float ror_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float half_pair_sum(float v) {  // v + (lane ^ 32)'s v
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float wave_sum64(float v) {
  v = ror_add<0x128>(v);
  v = ror_add<0x124>(v);
  v = ror_add<0x122>(v);
  v = ror_add<0x121>(v);
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  return half_pair_sum(v);
}

// Reflector of x (32 entries, lane a of each half holds x[a]): returns tau, beta and v (v_0 = 1).
struct Refl {
  float tau, beta, scal;
};
__device__ __forceinline__ Refl make_refl(float x, int a, int h) {
  const float sq = (h == 0 && a >= 1) ? x * x : 0.f;
  const float xn2 = wave_sum64(sq);
  const float alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  Refl r{0.f, alpha, 0.f};
  if (xn2 > 0.f) {
    r.beta = -copysignf(sqrtf(fmaf(alpha, alpha, xn2)), alpha);
    r.tau = (r.beta - alpha) / r.beta;
    r.scal = 1.f / (alpha - r.beta);
  }
  return r;
}

struct BulgeArgs {
  float* AB;
  int64_t n;
  float* V2;    // stage-2 reflectors: block (g, k) at (boff(g) + k) * 1024, sweep 32 g + i at row i
  float* tau2;  // (boff(g) + k) * 32 + i
  int* gprog;   // progress of the last sweep of every NW-sweep group (global)
  int* status;  // 0 ok, 1 a wait ran out
  int64_t spin_limit;
};

__device__ __forceinline__ int64_t boff(int64_t g, int64_t K0) { return g * (K0 + 1) - g * (g - 1) / 2; }

// One wave per sweep; the NW waves of a work-group take sweeps grp NW .. grp NW + NW - 1 for
// grp = blockIdx.x, blockIdx.x + gridDim.x, ...  Cooperative launch (all work-groups resident).
// A task keeps its blocks in registers, lane (a, h) holding row a, columns cc = h + 2 q (q < 16),
// of the diagonal block D (full, mirrored from the stored lower triangle) and of the off-diagonal
// block O, and the previous reflector at the same columns.  O H_prev and D's products with v are
// row dot products (two-lane sums); H O needs columns, so O and v go through LDS (the lane then
// owns column a, rows 16 h .. 16 h + 15) and O comes back to rows for coalesced stores; y of the
// two-sided update goes through LDS as well.
__global__ __launch_bounds__(64 * kNW) void bulge_kernel(BulgeArgs args) {
  __shared__ float sO[kNW][32][33];
  __shared__ float sv[kNW][32];
  __shared__ float sy[kNW][32];
  __shared__ int lprog[kNW];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, a = lane & 31, h = lane >> 5;
  float* __restrict__ AB = args.AB;
  const int64_t n = args.n;
  const int64_t K0 = (n - 2) / kBW;
  float(*O)[33] = sO[w];
  float* vs = sv[w];
  float* ys = sy[w];
  if (lane == 0) lprog[w] = -1;
  __syncthreads();
  const int64_t nsweeps = n - 1;
  const int64_t ngroups = (nsweeps + kNW - 1) / kNW;
  for (int64_t grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
    const int64_t s = grp * kNW + w;
    if (s >= nsweeps) break;
    const int64_t K = (n - 2 - s) / kBW;                    // last chase step of this sweep
    const int64_t Kp = s > 0 ? (n - 1 - s) / kBW : 0;       // last chase step of sweep s - 1
    int seen = -1;
    float tau_prev = 0.f;
    float vp[16];  // previous reflector at this lane's columns
#pragma unroll
    for (int q = 0; q < 16; ++q) vp[q] = 0.f;
    for (int64_t k = 0; k <= K; ++k) {
      // wait until sweep s - 1 has finished its tasks up to k + 1
      if (s > 0) {
        const int need = (int)((s - 1) * kProgStride + min(k + 2, Kp + 1));
        if (seen < need) {
          int64_t it = 0;
          for (;;) {
            // relaxed polls; the acquire (for the other work-group: an L2 invalidation) only once the
            // condition holds
            int v;
            if (w > 0) {
              v = __hip_atomic_load(&lprog[w - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
              v = __hip_atomic_load(&args.gprog[grp - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (v >= need) {
              if (w > 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
              else __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
              seen = v;
              break;
            }
            if (++it > args.spin_limit ||
                ((it & 255) == 0 &&
                 __hip_atomic_load(args.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)) {
              if (lane == 0) __hip_atomic_store(args.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              return;
            }
            __builtin_amdgcn_s_sleep(2);
          }
        }
      }
      const int64_t g = s / kBW, bid = boff(g, K0) + k;
      // every load of the task is issued before the first use (one memory round trip)
      const int64_t r0 = k == 0 ? s + 1 : s + 1 + k * kBW;
      const int64_t p0 = r0 - kBW;
      // wave-uniform bases, 32-bit lane offsets (few live registers across the loads)
      float* __restrict__ ABr = AB + r0 * kABld;
      float* __restrict__ ABp = AB + p0 * kABld;
      float dv[16], ov[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int cc = h + 2 * q;
        dv[q] = ABr[a >= cc ? cc * kABld + (a - cc) : a * kABld + (cc - a)];
      }
      if (k > 0) {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int cc = h + 2 * q;
          ov[q] = ABp[cc * kABld + (a + 32 - cc)];
        }
      }
      const float x0 = k == 0 ? AB[s * kABld + 1 + a] : 0.f;
      Refl rf;
      float va;  // v[a]
      if (k == 0) {
        // column s below the subdiagonal: AB[s][1 .. 32]
        rf = make_refl(x0, a, h);
        va = a == 0 ? 1.f : x0 * rf.scal;
        if (h == 0) {
          vs[a] = va;
          AB[s * kABld + 1 + a] = a == 0 ? rf.beta : 0.f;
        }
        wave_sync();
      } else {
        // O <- O H_prev: row a dotted with v_prev
        float u = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) u = fmaf(ov[q], vp[q], u);
        u = half_pair_sum(u);
#pragma unroll
        for (int q = 0; q < 16; ++q) ov[q] = fmaf(-tau_prev * u, vp[q], ov[q]);
        // reflector from column 0 (held by the h = 0 lane of row a as ov[0]); both halves take x[a]
        const float xh = __uint_as_float(
            __builtin_amdgcn_permlane32_swap(__float_as_uint(ov[0]), __float_as_uint(ov[0]), false, false)[0]);
        const float x = h == 0 ? ov[0] : xh;
        rf = make_refl(x, a, h);
        va = a == 0 ? 1.f : x * rf.scal;
#pragma unroll
        for (int q = 0; q < 16; ++q) O[a][h + 2 * q] = ov[q];
        if (h == 0) vs[a] = va;
        wave_sync();
        // O <- H O on column a, rows 16 h .. 16 h + 15; column 0 becomes (beta, 0, ...)
        float oc[16], vv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          oc[j] = O[16 * h + j][a];
          vv[j] = vs[16 * h + j];
        }
        float z = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) z = fmaf(vv[j], oc[j], z);
        z = half_pair_sum(z);
        wave_sync();  // every column read before the result overwrites it
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int i = 16 * h + j;
          O[i][a] = a == 0 ? (i == 0 ? rf.beta : 0.f) : fmaf(-rf.tau * z, vv[j], oc[j]);
        }
        wave_sync();
        // row layout again for coalesced stores (row a, columns cc: consecutive lanes, consecutive
        // addresses)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int cc = h + 2 * q;
          ABp[cc * kABld + (a + 32 - cc)] = O[a][cc];
        }
      }
      // D <- H D H: w = D v (rows), y = tau w - tau^2 (v.w) v / 2, D -= v y^T + y v^T
      float vr[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) vr[q] = vs[h + 2 * q];
      float wr = 0.f;
#pragma unroll
      for (int q = 0; q < 16; ++q) wr = fmaf(dv[q], vr[q], wr);
      wr = half_pair_sum(wr);
      const float vw = wave_sum64(h == 0 ? va * wr : 0.f);
      const float y = rf.tau * wr - 0.5f * rf.tau * rf.tau * vw * va;
      if (h == 0) ys[a] = y;
      wave_sync();
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int cc = h + 2 * q;
        const float d = dv[q] - (va * ys[cc] + y * vr[q]);
        if (a >= cc) ABr[cc * kABld + (a - cc)] = d;
      }
      if (h == 0) args.V2[(bid * 32 + (s % kBW)) * 32 + a] = va;
      if (lane == 0) args.tau2[bid * 32 + (s % kBW)] = rf.tau;
      tau_prev = rf.tau;
#pragma unroll
      for (int q = 0; q < 16; ++q) vp[q] = vr[q];
      // the next task rewrites O, v and y in LDS only after its loads and its own barrier; order
      // this task's LDS reads before those writes
      wave_sync();
      // publish
      const int val = (int)(s * kProgStride + (k == K ? kProgStride - 1 : k + 1));
      if (w == kNW - 1) {
        if (lane == 0) __hip_atomic_store(&args.gprog[grp], val, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (lane == 0) __hip_atomic_store(&lprog[w], val, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  }
}

__global__ __launch_bounds__(kThr) void fill_int_kernel(int* __restrict__ p, int64_t count, int v) {
  const int64_t e = (int64_t)blockIdx.x * kThr + threadIdx.x;
  if (e < count) p[e] = v;
}

__global__ __launch_bounds__(kThr) void tridiag_out_kernel(const float* __restrict__ AB, int64_t n,
                                                           float* __restrict__ D, float* __restrict__ E) {
  const int64_t j = (int64_t)blockIdx.x * kThr + threadIdx.x;
  if (j >= n) return;
  D[j] = AB[j * kABld];
  if (j + 1 < n) E[j] = AB[j * kABld + 1];
}

// ---- back-transformation of stage 2 ----------------------------------------------------------

constexpr int kPtChunks = 3 * 512;  // uint4 per block: 3 bf16 planes x (2 row tiles x 4 k-steps x 64 lanes)

// Block (g, k): P = (H_31 ... H_0)^T over the window rows 32 g + 1 + 32 k .. + 63, H_i the reflector
// of sweep 32 g + i at step k (acting on window rows i .. i + 31; identity where it does not
// exist).  One work-group per block; thread (c = t % 64, q = t / 64) owns column c, rows q (mod 4)
// of M = H_31 ... H_0, then P = M^T leaves as three bf16 planes (P = P0 + P1 + P2 to 2^-24) in the
// left-operand order of v_mfma_f32_32x32x16_bf16 with the k index permuted: chunk (plane, tile,
// step, lane) holds the 8 entries P[32 tile + lane % 32][16 step + 8 (j / 4) + 4 (lane / 32) + j % 4],
// j = 0 .. 7 (the window row that k slot j of the lane stands for in q2_apply_kernel).
__global__ __launch_bounds__(kThr) void q2_build_kernel(const float* __restrict__ V2, const float* __restrict__ tau2,
                                                        int64_t n, uint4* __restrict__ Pt) {
  __shared__ float M[64][65];
  __shared__ float sv[32];
  __shared__ float red[4][64];
  const int64_t K0 = (n - 2) / kBW;
  // block index -> (g, k): boff(g) <= bid < boff(g + 1)
  const int64_t bid = blockIdx.x;
  int64_t g = 0;
  {
    int64_t lo = 0, hi = K0;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (boff(mid, K0) <= bid) lo = mid;
      else hi = mid - 1;
    }
    g = lo;
  }
  const int64_t k = bid - boff(g, K0);
  const int t = threadIdx.x, c = t & 63, q = t >> 6;
  for (int e = t; e < 64 * 64; e += kThr) M[e / 64][e & 63] = (e / 64) == (e & 63) ? 1.f : 0.f;
  __syncthreads();
  for (int i = 0; i < 32; ++i) {
    const int64_t s = g * kBW + i;
    const bool exists = s <= n - 2 && k <= (n - 2 - s) / kBW;
    const float tau = exists ? tau2[bid * 32 + i] : 0.f;
    if (tau == 0.f) continue;  // uniform
    if (t < 32) sv[t] = V2[(bid * 32 + i) * 32 + t];
    __syncthreads();
    float z = 0.f;
    for (int aa = q; aa < 32; aa += 4) z = fmaf(sv[aa], M[i + aa][c], z);
    red[q][c] = z;
    __syncthreads();
    const float zc = tau * ((red[0][c] + red[1][c]) + (red[2][c] + red[3][c]));
    for (int aa = q; aa < 32; aa += 4) M[i + aa][c] = fmaf(-sv[aa], zc, M[i + aa][c]);
    __syncthreads();
  }
  uint4* out = Pt + bid * kPtChunks;
  for (int ci = t; ci < 512; ci += kThr) {
    const int l = ci & 63, ts = ci >> 6;
    const int cc = 32 * (ts >> 2) + (l & 31), k0 = 16 * (ts & 3) + 4 * (l >> 5);
    uint32_t h[4], m[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = k0 + 2 * (j & 1) + 8 * (j >> 1);  // slots 2 j, 2 j + 1
      split3(M[kk][cc], M[kk + 1][cc], h[j], m[j], lo[j]);
    }
    out[ci] = make_uint4(h[0], h[1], h[2], h[3]);
    out[512 + ci] = make_uint4(m[0], m[1], m[2], m[3]);
    out[1024 + ci] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }
}


// Zq ((n + kQ2Pad) x ldq, row-major, zero outside the n x n matrix; column j = eigenvector j of
// the tridiagonal matrix) <- Q2 Zq: groups last to first, blocks in increasing order, each block
// Zq[lo .. lo + 63][:] <- P(g, k) Zq[lo .. lo + 63][:].  One work-group per 64 columns and one wave
// per group: four groups at once, group gl - q on wave q.  Block k of group g reads rows that
// block k - 1 of group g + 1 (wave q - 1) finishes, and its prefetch two blocks ahead the rows of
// block k + 1 of group g + 1: each wave publishes its last finished block in LDS and waits for
// its predecessor's before loading rows.  A wave keeps the whole 64 x 64 block result in
// registers (four 32 x 32 tiles; K = 64 as four 16-k steps; six bf16 plane products each): the
// finished upper half goes to memory, while the lower half, split into bf16 planes in registers,
// is the next block's upper window as it stands, because P's columns are packed in the order that
// lines each result register up with the right-operand slot holding the same row: k slot (s, h, j)
// of lane l (h = l / 32) is window row 16 s + 8 (j / 4) + 4 h + j % 4.  The window's new rows load
// from memory straight into that order.  No data passes through LDS and waves do not wait on one
// another except for rows.
constexpr int kQ2Pad = 128;  // zero rows below the matrix (prefetches past a group's end read them)
static_assert((kMaxN + kQ2Pad) * ((kMaxN + 63) / 64 * 64) * 4 < ((int64_t)1 << 31), "Zq byte offsets are int32");

struct Q2Ops {
  uint4 a01[1][2][2][3];  // P planes, k steps 0, 1 [-][row tile][k step][plane]
  uint4 a23[2][2][3];     // P planes, k steps 2, 3 [row tile][k step - 2][plane]
  uint4 b[2][4][3];    // window planes [column tile][k step][plane]
  floatx16 acc[2][2];  // block result [row tile][column tile]
  float raw[2][2][8];  // window rows (32 + 16 s' .. of a later block) [column tile][s'][slot]
};

// Zq and Pt go through buffer instructions: a lane's byte offset in a VGPR (fixed for the
// kernel), the row's or chunk's byte offset in an SGPR, no 64-bit address arithmetic per access
struct Q2Wave {
  const uint4* Pt;
  __amdgpu_buffer_rsrc_t rz;  // Zq
  int vz[2];                  // lane byte offset, column tile ct: row 4 (lane / 32), column z0 + 32 ct + lane % 32
  int ldq4;                   // bytes per row of Zq
  int roff[16];               // byte offset of row 8 (i / 4) + i % 4 (k slots 8 s + j, result registers v)
  int lane;
  int* prog;                  // LDS: last finished block of each wave in this pass
  int* status;                // global: a wait ran past its bound
  int q;
  bool failed;
};

// k steps S0, S0 + 1 of block bid's P planes (k steps 0, 1 into set SET)
template <int SET, int S0>
__device__ __forceinline__ void q2w_load_a(Q2Ops& o, const Q2Wave& w, int64_t bid) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4*>(w.Pt + bid * kPtChunks), (short)0, kPtChunks * 16, 0x00020000);
  const int vo = w.lane * 16;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int s = S0; s < S0 + 2; ++s)
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      r, vo, (p * 512 + (rt * 4 + s) * 64) * 16, 0));
        if (S0 == 0) o.a01[SET][rt][s][p] = v;
        else o.a23[rt][s - 2][p] = v;
      }
}

// window rows row0 + 16 s' + 8 (j / 4) + j % 4 + 4 h (the slots of two k steps)
__device__ __forceinline__ void q2w_load_rows(Q2Ops& o, const Q2Wave& w, int row0) {
  const int rb = row0 * w.ldq4;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int so = rb + w.roff[i];
    o.raw[0][i >> 3][i & 7] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(w.rz, w.vz[0], so, 0));
    o.raw[1][i >> 3][i & 7] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(w.rz, w.vz[1], so, 0));
  }
}

__device__ __forceinline__ void q2w_split8(const float* x, uint4& h, uint4& m, uint4& l) {
  split3(x[0], x[1], h.x, m.x, l.x);
  split3(x[2], x[3], h.y, m.y, l.y);
  split3(x[4], x[5], h.z, m.z, l.z);
  split3(x[6], x[7], h.w, m.w, l.w);
}

// k steps SB, SB + 1 of the window from the loaded rows
template <int SB>
__device__ __forceinline__ void q2w_split_rows(Q2Ops& o) {
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int s = 0; s < 2; ++s) q2w_split8(o.raw[ct][s], o.b[ct][SB + s][0], o.b[ct][SB + s][1], o.b[ct][SB + s][2]);
}

// k steps 0, 1 of the next window from the lower result tile: result register 8 s + j of the lane
// is window row 16 s + 8 (j / 4) + 4 h + j % 4 of the next block
__device__ __forceinline__ void q2w_split_lower(Q2Ops& o) {
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = o.acc[1][ct][8 * s + j];
      q2w_split8(x, o.b[ct][s][0], o.b[ct][s][1], o.b[ct][s][2]);
    }
}

// row tile RT, k step S: six plane products into both column tiles (FRESH: the first k step)
template <int SET, int RT, int S, bool FRESH>
__device__ __forceinline__ void q2w_mfma(Q2Ops& o) {
  const uint4* pa = S < 2 ? o.a01[SET][RT][S] : o.a23[RT][S - 2];
  const bf16x8 a0 = __builtin_bit_cast(bf16x8, pa[0]);
  const bf16x8 a1 = __builtin_bit_cast(bf16x8, pa[1]);
  const bf16x8 a2 = __builtin_bit_cast(bf16x8, pa[2]);
  const bf16x8 b0 = __builtin_bit_cast(bf16x8, o.b[0][S][0]);
  const bf16x8 b1 = __builtin_bit_cast(bf16x8, o.b[0][S][1]);
  const bf16x8 b2 = __builtin_bit_cast(bf16x8, o.b[0][S][2]);
  const bf16x8 d0 = __builtin_bit_cast(bf16x8, o.b[1][S][0]);
  const bf16x8 d1 = __builtin_bit_cast(bf16x8, o.b[1][S][1]);
  const bf16x8 d2 = __builtin_bit_cast(bf16x8, o.b[1][S][2]);
  floatx16 c0, c1;
  if (FRESH) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      c0[v] = 0.f;
      c1[v] = 0.f;
    }
  } else {
    c0 = o.acc[RT][0];
    c1 = o.acc[RT][1];
  }
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, d0, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, d1, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, d0, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b2, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, d2, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, d1, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b0, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, d0, c1, 0, 0, 0);
  o.acc[RT][0] = c0;
  o.acc[RT][1] = c1;
}

// result tile (both column tiles) -> rows row0 .. row0 + 31: register v is row 8 (v / 4) + 4 h + v % 4
__device__ __forceinline__ void q2w_store(const floatx16 (&c)[2], const Q2Wave& w, int row0) {
  const int rb = row0 * w.ldq4;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int so = rb + w.roff[v];
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(c[0][v]), w.rz, w.vz[0], so, 0);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(c[1][v]), w.rz, w.vz[1], so, 0);
  }
}

// wave q waits until wave q - 1 has finished its block `target` of this pass
__device__ __forceinline__ void q2w_wait(Q2Wave& w, int target) {
  if (w.q == 0 || w.failed) return;
  for (int it = 0;; ++it) {
    if (__hip_atomic_load(&w.prog[w.q - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
    if (it > (1 << 22)) {
      __hip_atomic_store(w.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w.failed = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// every lane stores the same value: no branch, so a block's work stays one scheduling region
__device__ __forceinline__ void q2w_publish(const Q2Wave& w, int k) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __hip_atomic_store(&w.prog[w.q], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSgMfma = 0x008, kSgValu = 0x002, kSgVmemRd = 0x020;

// block k of the wave's group (window rows lo0 + 32 k ..), k-step 0, 1 planes in set SET = k % 2.
// On entry: block k's P planes and block k + 1's for k steps 0, 1 (loaded or in flight), the
// window's k steps 2, 3, the rows of block k + 1's k steps 2, 3 in raw, and (k > 0) block k - 1's
// result, whose lower tile becomes this window's k steps 0, 1.  Block k + 1's k-step 2, 3 planes
// and block k + 2's k-step 0, 1 planes replace block k's as they are used.
template <bool FIRST, int SET>
__device__ __forceinline__ void q2w_block(Q2Ops& o, Q2Wave& w, int k, int nk, int lo0, int64_t base) {
  const int lo = lo0 + kBW * k;
  // One wave per SIMD issues in order, so the matrix cores stay busy only if the splits and the
  // loads sit between the products in the instruction stream: k steps 2, 3 of the upper tile
  // with the lower tile's split, k steps 2, 3 of the lower tile with block k + 1's k-step 2, 3
  // loads, k step 0 with the new rows' split (one scheduling region each).
  if (!FIRST) {
    q2w_store(o.acc[0], w, lo - kBW);  // block k - 1's upper tile is final
    q2w_publish(w, k - 1);
    __builtin_amdgcn_sched_barrier(0);
    q2w_mfma<SET, 0, 2, true>(o);
    q2w_split_lower(o);
    q2w_mfma<SET, 0, 3, false>(o);
#pragma unroll
    for (int i = 0; i < 24; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSgValu, 10, 0);
    }
  } else {
    q2w_mfma<SET, 0, 2, true>(o);
    q2w_mfma<SET, 0, 3, false>(o);
  }
  __builtin_amdgcn_sched_barrier(0);
  q2w_mfma<SET, 1, 2, true>(o);
  q2w_mfma<SET, 1, 3, false>(o);
  q2w_load_a<SET, 2>(o, w, base + min(k + 1, nk - 1));
#pragma unroll
  for (int i = 0; i < 12; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
    __builtin_amdgcn_sched_group_barrier(kSgVmemRd, 1, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  q2w_mfma<SET, 0, 0, false>(o);
  q2w_mfma<SET, 1, 0, false>(o);
  q2w_split_rows<2>(o);  // block k + 1's k steps 2, 3
#pragma unroll
  for (int i = 0; i < 24; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSgValu, 8, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // rows of block k + 2's k steps 2, 3 (block k + 1 of wave q - 1; clamped past the group's end)
  q2w_wait(w, min(k + 2, nk - 2));
  q2w_load_rows(o, w, lo0 + kBW * min(k + 2, nk - 1) + 32);
  q2w_mfma<SET, 0, 1, false>(o);
  q2w_mfma<SET, 1, 1, false>(o);
  q2w_load_a<0, 0>(o, w, base + min(k + 1, nk - 1));
#pragma unroll
  for (int i = 0; i < 22; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSgVmemRd, 2, 0);
  }
}

__global__ __launch_bounds__(256) void q2_apply_kernel(const uint4* __restrict__ Pt, float* __restrict__ Zq,
                                                       int64_t n64, int64_t ldq, int* __restrict__ status) {
  __shared__ int sprog[4];
  const int t = threadIdx.x, lane = t & 63;
  const int q = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = (int)n64;
  const int z0 = (int)blockIdx.x * 64;
  Q2Wave w;
  w.Pt = Pt;
  // every byte offset fits in 32 bits: (n + kQ2Pad) ldq 4 < 2^31 for n <= kMaxN
  w.rz = __builtin_amdgcn_make_buffer_rsrc(Zq, (short)0, (int)((n64 + kQ2Pad) * ldq * 4), 0x00020000);
  w.ldq4 = (int)ldq * 4;
  w.vz[0] = (4 * (lane >> 5) * (int)ldq + z0 + (lane & 31)) * 4;
  w.vz[1] = w.vz[0] + 32 * 4;
#pragma unroll
  for (int i = 0; i < 16; ++i) w.roff[i] = (8 * (i >> 2) + (i & 3)) * w.ldq4;
  w.lane = lane;
  w.prog = sprog;
  w.status = status;
  w.q = q;
  w.failed = false;
  const int K0 = (n - 2) / kBW;
  Q2Ops o;
  for (int gl = K0; gl >= 0; gl -= 4) {
    if (t < 4) sprog[t] = -1;
    __syncthreads();
    const int g = gl - q;
    if (g >= 0) {
      const int nk = K0 + 1 - g;
      const int64_t base = boff(g, K0);
      const int lo0 = g * kBW + 1;
      // block 0's window and block 1's new rows: rows wave q - 1 finishes by its block 1
      q2w_wait(w, min(1, nk - 2));
      q2w_load_rows(o, w, lo0);
      q2w_split_rows<0>(o);
      q2w_load_rows(o, w, lo0 + 32);
      q2w_split_rows<2>(o);
      q2w_load_a<0, 0>(o, w, base);
      q2w_load_a<0, 2>(o, w, base);
      q2w_load_rows(o, w, lo0 + 32 + kBW * min(1, nk - 1));
      q2w_block<true, 0>(o, w, 0, nk, lo0, base);
      for (int k = 1; k < nk; ++k) q2w_block<false, 0>(o, w, k, nk, lo0, base);
      // the last block: both halves are final
      const int lol = lo0 + kBW * (nk - 1);
      q2w_store(o.acc[0], w, lol);
      q2w_store(o.acc[1], w, lol + 32);
      // the last blocks' prefetches are never used: wait for them here, once per pass
      __builtin_amdgcn_s_waitcnt(0);
    }
    q2w_publish(w, 1 << 30);
    __syncthreads();
  }
}

// Z (n x n, row j = eigenvector j) -> Zq (row i = coordinate i, zero outside n x n) and back
__global__ __launch_bounds__(256) void q2_gather_kernel(const float* __restrict__ Z, int64_t n, float* __restrict__ Zq,
                                                        int64_t ldq) {
  __shared__ float tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;  // Zq tile
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t j = c0 + i, r = r0 + tx;  // Z[j][r]
    tile[i][tx] = (j < n && r < n) ? Z[j * n + r] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) Zq[(r0 + i) * ldq + c0 + tx] = tile[tx][i];
}

__global__ __launch_bounds__(256) void q2_scatter_kernel(const float* __restrict__ Zq, int64_t ldq, int64_t n,
                                                         float* __restrict__ Z) {
  __shared__ float tile[32][33];
  const int64_t j0 = (int64_t)blockIdx.y * 32, r0 = (int64_t)blockIdx.x * 32;  // Z tile
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8) {
    const int64_t r = r0 + i, j = j0 + tx;  // Zq[r][j]
    tile[i][tx] = (r < n && j < n) ? Zq[r * ldq + j] : 0.f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int64_t j = j0 + i, r = r0 + tx;
    if (j < n && r < n) Z[j * n + r] = tile[tx][i];
  }
}

}  // namespace

Layout layout(int64_t n) {
  Layout L{};
  int64_t o = 0;
  auto take = [&](int64_t elems) {
    const int64_t at = o;
    o += al64(elems);
    return at;
  };
  const int64_t nleaf = (n + kLeaf - 1) / kLeaf;
  L.Yl = take(n * 32);
  L.taul = take(nleaf * 32);
  L.Rs = take(nleaf * 32 * 32);
  L.E = take(nleaf * 32 * 32);
  L.Rroot = take(32 * 32);
  L.Q1 = take(n * 32);
  L.Y = take(n * 32);
  L.BP = take((n + 255) / 256 * 256 * 32);  // B = Y T packed for xsym_kernel, zero rows to 256
  L.X = take(n * 32);
  L.T = take(32 * 32);
  L.Gp = take(64 * 1024 * 3);
  L.Xop = take((n + 127) / 128 * 4 * (3 * 8 * 64) * 4);  // packed update operands, K <= 128 (uint4 = 4 floats)
  L.Yop = take((n + 127) / 128 * 4 * (3 * 8 * 64) * 4);
  L.Y2 = take(n * 32);   // Y of the odd panels (the first panel's Y of a pair stays in Y)
  L.Wf = take(n * 32);   // W of the first panel of a pair (fp32)
  L.G12 = take(2048);    // the pair correction's G1, G2
  L.M = take(32 * 32);
  L.px_floats = (n + 255) / 256 * n * 32;  // partial slots of X = A22 (Y T): one per tile row
  L.Px = take(L.px_floats);
  L.Gd = take(2 * 64 * 1024);   // fp64 Gram partials
  L.Rc = take(2 * 1024);        // fp64 R of the current pass
  L.Rt = take(2 * 1024);        // fp64 R_tot
  L.flags = take(n / kBW + 64); // per-panel fallback flags (int)
  L.AB = take((n + kABpad) * kABld);
  const int64_t nb = q2_blocks(n);
  L.V2 = take(nb * 32 * 32);
  L.tau2 = take(nb * 32);
  L.Pt = take(nb * kPtChunks * 4);
  L.prog = take((n + kNW) / kNW + 64);  // int progress slots + status
  L.ldq = (n + 63) / 64 * 64;
  L.Zq = take((n + kQ2Pad) * L.ldq);
  L.total = o;
  return L;
}

int sy2sb(int64_t n, float* A, int64_t lda, float* tau, float* ws, const Layout& L, hipStream_t stream) {
  // one fallback flag per panel (0: the Cholesky QR path holds), cleared up front
  int* flags = reinterpret_cast<int*>(ws + L.flags);
  const int64_t npanels = n > kBW ? (n - kBW + kBW - 1) / kBW : 0;
  if (npanels > 0) {
    hipLaunchKernelGGL(fill_int_kernel, dim3((unsigned)((npanels + 2 + kThr - 1) / kThr)), dim3(kThr), 0, stream,
                       flags, npanels + 2, 0);
    MPQ_LAUNCH_CHECK();
  }
  for (int64_t c0 = 0; c0 + kBW < n; c0 += kBW) {
    const int64_t pidx = c0 / kBW;
    const int64_t r0 = c0 + kBW, m = n - r0;
    const int64_t nleaf = (m + kLeaf - 1) / kLeaf;
    const int root_rows = (int)(32 * (nleaf - 1) + std::min<int64_t>(32, m - kLeaf * (nleaf - 1)));
    // Q1 R = P: Cholesky QR (three passes; hr_kernel applies the last factor), or the tall-skinny
    // Householder QR when it fails
    const int* fb = flags + pidx;
    int* fbw = flags + pidx;
    const float* P = A + r0 * lda + c0;
    const int64_t cq_ng = std::min<int64_t>(64, (m + kCqTile - 1) / kCqTile);
    const int64_t cq_chunk = (m + cq_ng - 1) / cq_ng;
    double* Gp = reinterpret_cast<double*>(ws + L.Gd);
    double* Rc = reinterpret_cast<double*>(ws + L.Rc);
    double* Rt = reinterpret_cast<double*>(ws + L.Rt);
    unsigned* counter = reinterpret_cast<unsigned*>(flags + npanels + 1);
    // pass p's launch solves with R_{p-1} and factors the Gram matrix of the result (R_p)
    for (int pass = 1; pass <= 3; ++pass) {
      hipLaunchKernelGGL(cq_pass_kernel, dim3((unsigned)cq_ng), dim3(kThr), 0, stream, pass <= 2 ? P : ws + L.Q1,
                         pass <= 2 ? lda : (int64_t)32, m, cq_chunk, Rc, pass > 1 ? 1 : 0, ws + L.Q1, Gp, pass, Rt,
                         ws + L.Rroot, fbw, counter);
      MPQ_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(leaf_qr_kernel, dim3((unsigned)nleaf), dim3(kPThr), 0, stream, A, lda, r0, c0, m, ws + L.Yl,
                       ws + L.taul, ws + L.Rs, fb);
    MPQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(root_qr_kernel, dim3(1), dim3(kPThr), 0, stream, ws + L.Rs, root_rows, ws + L.Rroot,
                       ws + L.E, fb);
    MPQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(leaf_q_kernel, dim3((unsigned)nleaf), dim3(kPThr), 0, stream, ws + L.Yl, ws + L.taul,
                       ws + L.E, m, ws + L.Q1, fb);
    MPQ_LAUNCH_CHECK();
    const unsigned rblocks = (unsigned)((m + kThr - 1) / kThr);
    // panels go in pairs (even panel first) sharing one trailing update; a last even panel goes alone
    const bool second = (pidx & 1) != 0;
    const bool first = !second && c0 + 2 * kBW < n;
    float* Ycur = second ? ws + L.Y2 : ws + L.Y;
    hipLaunchKernelGGL(hr_kernel, dim3(rblocks), dim3(kThr), 0, stream, ws + L.Q1, Rc, fb, ws + L.Rroot, m, A, lda,
                       r0, c0, Ycur, ws + L.BP, ws + L.T, tau);
    MPQ_LAUNCH_CHECK();
    float* A22 = A + r0 * lda + r0;
    // X = A22 (Y T): one partial slot per tile of the lower triangle's tile row / column, summed in
    // slot order; 128-wide tiles while they keep the slots within the buffer (m <= n / 2)
    const bool small = 2 * m <= n;
    const int64_t tile = small ? 128 : 256;
    const int64_t nbt = (m + tile - 1) / tile;
    if (nbt * m * 32 > L.px_floats) {
      set_error("sy2sb: %lld partial slots of %lld rows exceed the workspace", (long long)nbt, (long long)m);
      return kUnsupported;
    }
    const unsigned ntiles = (unsigned)(nbt * (nbt + 1) / 2);
    if (small)
      hipLaunchKernelGGL(xsym_kernel<2>, dim3(ntiles), dim3(kThr), 0, stream, A22, lda,
                         reinterpret_cast<const float4*>(ws + L.BP), m, ws + L.Px);
    else
      hipLaunchKernelGGL(xsym_kernel<4>, dim3(ntiles), dim3(kThr), 0, stream, A22, lda,
                         reinterpret_cast<const float4*>(ws + L.BP), m, ws + L.Px);
    MPQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(xsum_kernel, dim3((unsigned)((m * 32 + kThr - 1) / kThr)), dim3(kThr), 0, stream, ws + L.Px,
                       (int)nbt, m * 32, ws + L.X);
    MPQ_LAUNCH_CHECK();
    const int64_t ng = std::min<int64_t>(64, (m + 63) / 64);
    const int64_t chunk = ((m + ng - 1) / ng + 63) / 64 * 64;
    const int64_t ngu = (m + chunk - 1) / chunk;
    // the first panel's Y and W from this panel's first row (the second panel of a pair)
    const float* Yh = second ? ws + L.Y + 32 * 32 : nullptr;
    const float* Wh = second ? ws + L.Wf + 32 * 32 : nullptr;
    hipLaunchKernelGGL(gram_partial_kernel, dim3((unsigned)ngu), dim3(kThr), 0, stream, Ycur, ws + L.X, m, chunk,
                       ws + L.Gp, Yh, Wh);
    MPQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(m_kernel, dim3(1), dim3(1024), 0, stream, ws + L.Gp, (int)ngu, second ? 3 : 1, ws + L.T,
                       ws + L.M, ws + L.G12);
    MPQ_LAUNCH_CHECK();
    uint4* Xp = reinterpret_cast<uint4*>(ws + L.Xop);
    uint4* Yp = reinterpret_cast<uint4*>(ws + L.Yop);
    const int ks = (first || second) ? 8 : 4;
    const int cy = second ? 4 : 0, cw = first ? 8 : (second ? 12 : 4);
    const int row_off = first ? 32 : 0;
    const int64_t wrows = row_off + (m - row_off + 127) / 128 * 128;
    hipLaunchKernelGGL(w_kernel, dim3((unsigned)((4 * wrows + kThr - 1) / kThr)), dim3(kThr), 0, stream, ws + L.M, Ycur,
                       ws + L.X, m, Xp, Yp, ks, cy, cw, row_off, first ? ws + L.Wf : nullptr, Yh, Wh,
                       second ? ws + L.G12 : nullptr);
    MPQ_LAUNCH_CHECK();
    if (first) {
      // the second panel's columns now; the rest of A22 with the second panel's update
      hipLaunchKernelGGL(colblock_kernel, dim3((unsigned)((m + 7) / 8)), dim3(kThr), 0, stream, A22, lda, m, Ycur,
                         ws + L.Wf);
      MPQ_LAUNCH_CHECK();
    } else {
      // A22 -= Y W^T + W Y^T on the lower triangle and whole diagonal tiles (with the first panel's
      // part for the second panel of a pair)
      const int64_t m128 = (m + 127) / 128 * 128;
      const int64_t nt = m128 / 128;
      if (second)
        hipLaunchKernelGGL(syr2k_x6_kernel<8>, dim3((unsigned)(nt * (nt + 1) / 2)), dim3(kThr), 0, stream, Xp, Yp,
                           A22, lda, m);
      else
        hipLaunchKernelGGL(syr2k_x6_kernel<4>, dim3((unsigned)(nt * (nt + 1) / 2)), dim3(kThr), 0, stream, Xp, Yp,
                           A22, lda, m);
      MPQ_LAUNCH_CHECK();
    }
  }
  return kOk;
}

int sb2st(int64_t n, const float* A, int64_t lda, float* D, float* E, float* ws, const Layout& L,
          hipStream_t stream) {
  float* AB = ws + L.AB;
  const int64_t cnt = (n + kABpad) * kABld;
  hipLaunchKernelGGL(band_extract_kernel, dim3((unsigned)((cnt + kThr - 1) / kThr)), dim3(kThr), 0, stream, A, lda, n,
                     AB);
  MPQ_LAUNCH_CHECK();
  if (n >= 3) {
    const int64_t ngroups = (n - 1 + kNW - 1) / kNW;
    int* prog = reinterpret_cast<int*>(ws + L.prog);
    int* status = prog + ngroups;
    hipLaunchKernelGGL(fill_int_kernel, dim3((unsigned)((ngroups + 1 + kThr - 1) / kThr)), dim3(kThr), 0, stream,
                       prog, ngroups + 1, -1);
    MPQ_LAUNCH_CHECK();
    hipLaunchKernelGGL(fill_int_kernel, dim3(1), dim3(kThr), 0, stream, status, 1, 0);
    MPQ_LAUNCH_CHECK();
    BulgeArgs args{AB, n, ws + L.V2, ws + L.tau2, prog, status, (int64_t)1 << 24};
    // enough work-groups that every group of sweeps has one when the pipeline is full (about
    // n / 64 tasks per sweep in flight, two tasks apart), at most one per CU
    const int64_t want = std::max<int64_t>(1, std::min<int64_t>(ngroups, (n / kBW) / (2 * kNW) + 2));
    const unsigned G = (unsigned)std::min<int64_t>(want, 128);
    void* kargs[] = {&args};
    MPQ_HIP_TRY(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(bulge_kernel), dim3(G), dim3(64 * kNW),
                                           kargs, 0, stream));
    int st = 0;
    MPQ_HIP_TRY(hipMemcpyAsync(&st, status, sizeof(int), hipMemcpyDeviceToHost, stream));
    MPQ_HIP_TRY(hipStreamSynchronize(stream));
    if (st != 0) {
      set_error("mpq_syevd: band reduction pipeline stalled (a wait exceeded its bound)");
      set_error_code(kHipError);
      return kHipError;
    }
  }
  hipLaunchKernelGGL(tridiag_out_kernel, dim3((unsigned)((n + kThr - 1) / kThr)), dim3(kThr), 0, stream, AB, n, D, E);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

int q2_apply(int64_t n, float* Z, float* ws, const Layout& L, hipStream_t stream) {
  if (n < 3) return kOk;
  const int64_t nb = q2_blocks(n);
  uint4* Pt = reinterpret_cast<uint4*>(ws + L.Pt);
  float* Zq = ws + L.Zq;
  hipLaunchKernelGGL(q2_build_kernel, dim3((unsigned)nb), dim3(kThr), 0, stream, ws + L.V2, ws + L.tau2, n, Pt);
  MPQ_LAUNCH_CHECK();
  hipLaunchKernelGGL(q2_gather_kernel, dim3((unsigned)(L.ldq / 32), (unsigned)((n + kQ2Pad) / 32)), dim3(kThr), 0,
                     stream, Z, n, Zq, L.ldq);
  MPQ_LAUNCH_CHECK();
  int* status = reinterpret_cast<int*>(ws + L.prog) + (n - 1 + kNW - 1) / kNW + 1;
  hipLaunchKernelGGL(fill_int_kernel, dim3(1), dim3(kThr), 0, stream, status, 1, 0);
  MPQ_LAUNCH_CHECK();
  hipLaunchKernelGGL(q2_apply_kernel, dim3((unsigned)(L.ldq / 64)), dim3(kThr), 0, stream, Pt, Zq, n, L.ldq, status);
  MPQ_LAUNCH_CHECK();
  hipLaunchKernelGGL(q2_scatter_kernel, dim3((unsigned)((n + 31) / 32), (unsigned)((n + 31) / 32)), dim3(kThr), 0,
                     stream, Zq, L.ldq, n, Z);
  MPQ_LAUNCH_CHECK();
  int st = 0;
  MPQ_HIP_TRY(hipMemcpyAsync(&st, status, sizeof(int), hipMemcpyDeviceToHost, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  if (st != 0) {
    set_error("mpq_syevd: band back-transformation pipeline stalled (a wait exceeded its bound)");
    set_error_code(kHipError);
    return kHipError;
  }
  return kOk;
}

}  // namespace band
}  // namespace mpq
