// Symmetric eigendecomposition for the rank-space solvers (gfx950).
//
// Replaces the torch.linalg.eigh call of mpq/adapters/gptqmodel.py:276-310 with:
//   1. tridiagonalisation A = Q T Q^T (LAPACK sytrd, lower, blocked as latrd + syr2k) written for
//      this device: per reflector one half-storage symv kernel over the trailing matrix (only
//      64 x 64 tiles on or below the diagonal are read, each tile contributing A_t v and A_t^T v,
//      partial sums kept per tile so the result is deterministic) and one kernel that finishes
//      w = tau (A v - V W^T v - W V^T v) - tau/2 (w.v) v, applies the panel's lazy update to the
//      next column and forms the partial norms of the next reflector; every 32 reflectors the
//      trailing matrix takes the rank-64 update A -= V W^T + W V^T on the MFMA GEMM;
//   2. divide and conquer on the tridiagonal matrix (stedc.hip): T = Z^T diag(lam) Z, eigenvalues
//      ascending, Z row-major with row k = eigenvector k;
//   3. back-transformation V = Q Z: the reflectors are applied in blocks of kNB (fp64: kNB / 2) as
//      compact-WY factors I - Y Tb Y^T (Tb from the block's gram Y^T Y, LAPACK larft
//      forward/columnwise), last block first; fp32 on bf16-plane products (wy_x6.hip), fp64 on the
//      fp64 matrix cores (gemm_f64.hip).
// Output: lam ascending (n), V (n x n, row-major, column k = eigenvector k), as torch.linalg.eigh.
//
// Storage: the symmetric matrix sits in a zero-padded row-major buffer with leading dimension
// lda = n rounded up to 64, so every tile load is 16-byte aligned.  Only the lower triangle and
// the 64 x 64 diagonal tiles are kept current; column c is copied into row c when its reflector
// is formed.
// Reflector i (LAPACK's H(i) = I - tau_i v_i v_i^T, v_i[0..i] = 0, v_i[i+1] = 1) is stored in
// row i, entries i+2..n-1 -- by symmetry the same entries LAPACK's lower storage keeps in column i.
//
// fp32 with 1024 <= n <= band::kMaxN (use_two_stage) takes the two-stage reduction instead (eigh_band.hip: dense ->
// band of half-bandwidth 32 on the MFMA GEMM, band -> tridiagonal by bulge chasing); its stage-1
// reflectors sit in the rows of A the same way with v_i[i + 32] = 1, and the same compact-WY
// back-transformation applies them after the bulge-chasing reflectors.

#include <algorithm>

#include "common.h"
#include "eigh_band.h"
#include "gemm.h"
#include "gemm_f64.h"
#include "kernels.h"
#include "stedc.h"
#include "wy_x6.h"

namespace mpq {
namespace {

constexpr int kNB = 128;  // reflectors per compact-WY block of the back-transformation
constexpr int kPB = 32;   // reflectors per tridiagonalisation panel (latrd block)
constexpr int kTB = 64;   // symv tile edge
// most symv tiles per work-group (one chunk of a column strip): 4 in fp32, 8 in fp64 (measured: fp32
// n = 4096 67.6 ms per solve at 4 against 71.1 at 8 and 83.8 at 16; fp64 n = 8192 336 ms at 8, 340
// at 4, 350 at 16)
template <typename T>
constexpr int ch_max() { return sizeof(T) == 4 ? 4 : 8; }
constexpr int kThr = 256;
constexpr int kSub = 8;               // finish_kernel lanes per matrix row
constexpr int kRowsPB = kThr / kSub;  // finish_kernel rows per work-group
constexpr int kDotWG = 32;                      // symv work-groups that form the dots p, q
constexpr int kDotPerWave = (2 * kPB + 3) / 4;  // dots per wave of a dot work-group

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

// ---- element-type helpers (fp32 and fp64 share every kernel) ------------------------------------

template <typename T>
struct Vec4 {
  T x, y, z, w;
};
template <typename T>
__device__ __forceinline__ Vec4<T> load_v4(const T* p);
template <>
__device__ __forceinline__ Vec4<float> load_v4<float>(const float* p) {
  const float4 f = *reinterpret_cast<const float4*>(p);
  return {f.x, f.y, f.z, f.w};
}
template <>
__device__ __forceinline__ Vec4<double> load_v4<double>(const double* p) {
  const double2 a = *reinterpret_cast<const double2*>(p);
  const double2 b = *reinterpret_cast<const double2*>(p + 2);
  return {a.x, a.y, b.x, b.y};
}
template <typename T>
__device__ __forceinline__ T wave_sum_t(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float block_sum_t(float v, float* scratch) { return block_sum(v, scratch); }
__device__ __forceinline__ double block_sum_t(double v, double* scratch) { return block_sum_f64(v, scratch); }

// reflectors per compact-WY block of the back-transformation (the T factor's two LDS arrays:
// 2 x 128 x 129 x 4 bytes in fp32, 2 x 64 x 65 x 8 in fp64)
template <typename T>
struct NbOf;
template <>
struct NbOf<float> {
  static constexpr int value = kNB;
};
template <>
struct NbOf<double> {
  static constexpr int value = kNB / 2;
};

// out = in^T (rows x cols -> cols x rows), 32 x 32 tiles through LDS
template <typename T>
__global__ __launch_bounds__(256) void transpose_t_kernel(const T* __restrict__ in, int64_t rows, int64_t cols,
                                                          int64_t ld_in, T* __restrict__ out, int64_t ld_out) {
  __shared__ T tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = in[r * ld_in + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) out[c * ld_out + r] = tile[tx][k];
  }
}

// Operands of the rank-2 kPB panel update from the panel's reflectors V (kPB x m, rows of A) and
// W (kPB x m): X = [V^T W^T] and Yb = [W^T V^T] (m x 2 kPB each), so A -= X Yb^T.  Rows below
// `zrows` are zero (the update then starts below the panel at an aligned row and leaves the rows
// in between unchanged).  One launch per panel, 32 source columns per work-group.
template <typename T>
__global__ __launch_bounds__(256) void panel_operands_kernel(const T* __restrict__ Vp, const T* __restrict__ Wp,
                                                             int64_t m, int64_t zrows, int64_t ld, T* __restrict__ X,
                                                             T* __restrict__ Yb) {
  __shared__ T tv[kPB][33], tw[kPB][33];
  const int64_t c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int k = ty; k < kPB; k += 8) {
    const int64_t c = c0 + tx;
    const bool in = c >= zrows && c < m;
    tv[k][tx] = in ? Vp[k * ld + c] : T(0);
    tw[k][tx] = in ? Wp[k * ld + c] : T(0);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 32 * kPB; e += 256) {
    const int rr = e / kPB, k = e % kPB;
    const int64_t r = c0 + rr;
    if (r < m) {
      X[r * 2 * kPB + k] = tv[k][rr];
      X[r * 2 * kPB + kPB + k] = tw[k][rr];
      Yb[r * 2 * kPB + k] = tw[k][rr];
      Yb[r * 2 * kPB + kPB + k] = tv[k][rr];
    }
  }
}

// ---- tridiagonalisation ----------------------------------------------------------------------

// First column c of a panel, read from the lower triangle (the trailing update keeps only that
// part current) and copied into row c, where the reflector is formed: D[c] = A[c][c],
// alpha_c = A[c+1][c] and the partial sums of A[g][c]^2 for g >= c+2 (one per work-group;
// thread g = c + 256 blockIdx + tid).
template <typename T>
__global__ __launch_bounds__(kThr) void panel_start_kernel(T* __restrict__ A, int64_t lda, int64_t n,
                                                          int64_t c, T* __restrict__ D, T* __restrict__ alph,
                                                          T* __restrict__ Pn) {
  __shared__ T red[kThr / 64];
  const int64_t g = c + (int64_t)blockIdx.x * kThr + threadIdx.x;
  T sq = 0.f;
  if (g < n) {
    const T a = A[g * lda + c];
    A[c * lda + g] = a;
    if (g == c) D[c] = a;
    if (g == c + 1) alph[c] = a;
    if (g >= c + 2) sq = a * a;
  }
  const T t = block_sum_t(sq, red);
  if (threadIdx.x == 0) Pn[blockIdx.x] = t;
}

// Half-storage symv over the trailing matrix A[c+1:, c+1:] (as of the panel start) with the
// unscaled tail x of column c's reflector (x[g] = row c entry g for g >= c+2, else 0; the reflector
// is v = e_{c+1} + scale x, and the finishing kernel combines the pieces once scale is known),
// plus the dots W_j . x and V_j . x of the panel's earlier reflectors j < i (an extra row of
// kDotWG work-groups).  Tiles are 64 x 64 in global coordinates.  Work-group (x, y) takes column
// strip bj = b0 + x and row tiles bi = bj + 8y .. +7:
//   Pr[bj][rows of bi] = A_(bi,bj) x_bj          (row contributions, one value per tile row)
//   Pc[bj][y][64]      = sum_{bi > bj} A_(bi,bj)^T x_bi   (column contributions of the chunk)
//   Pvv[y][bj]         = sum x_bi^T A_(bi,bj) x_bj (x2 off the diagonal)
//   Ppq[x][64]         = dot work-group x's share of W_j . x (slots 0..i-1), V_j . x (32..32+i-1)
// No work-group waits for anything before its first tile load.
// Thread layout over a tile: column quad cq = tid % 16 (4 columns), rows r0 + 16k, r0 = tid / 16.
template <typename T>
__global__ __launch_bounds__(kThr) void symv_kernel(const T* __restrict__ A, int64_t lda, int64_t n, int64_t c,
                                                   int64_t i0, int i, const T* __restrict__ Wb,
                                                   T* __restrict__ Pr, T* __restrict__ Pc,
                                                   T* __restrict__ Pvv, T* __restrict__ Ppq, int ch_alloc,
                                                   int chl) {
  const int nblk = (int)(lda / kTB);
  const int b0 = (int)((c + 1) / kTB);
  if ((int)blockIdx.y == (int)gridDim.y - 1) {
    // dot work-groups: x < kDotWG takes strips b0 + x, b0 + x + kDotWG, ...; wave w the dots
    // d = w, w + 4, ... (d < i: W_d . x; i <= d < 2i: V_{d-i} . x), lane = entry
    if ((int)blockIdx.x >= kDotWG) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    T acc[kDotPerWave];
#pragma unroll
    for (int t = 0; t < kDotPerWave; ++t) acc[t] = 0.f;
    for (int sx = b0 + (int)blockIdx.x; sx < nblk; sx += kDotWG) {
      const int64_t g = (int64_t)sx * kTB + lane;
      const T v = (g > c + 1 && g < n) ? A[c * lda + g] : 0.f;
      T x[kDotPerWave];
#pragma unroll
      for (int t = 0; t < kDotPerWave; ++t) {
        const int d = w + 4 * t;
        const int j = d < i ? d : d - i;
        x[t] = d < 2 * i ? (d < i ? Wb[(int64_t)j * lda + g] : A[(i0 + j) * lda + g]) : 0.f;
      }
#pragma unroll
      for (int t = 0; t < kDotPerWave; ++t) acc[t] += x[t] * v;
    }
#pragma unroll
    for (int t = 0; t < kDotPerWave; ++t) {
      const int d = w + 4 * t;
      const T tot = wave_sum_t(acc[t]);
      if (lane == 0 && d < 2 * i) Ppq[(int64_t)blockIdx.x * 64 + (d < i ? d : kPB + d - i)] = tot;
    }
    return;
  }
  // odd columns walk the tiles in reverse dispatch order, so the tiles the previous column read
  // last (still in the memory-side cache) are read first
  const bool rev = (c & 1) != 0;
  const int bj = b0 + (rev ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x);
  const int ch = rev ? (int)gridDim.y - 2 - (int)blockIdx.y : (int)blockIdx.y;
  const int bi_first = bj + ch * chl;
  if (bi_first >= nblk) return;  // uniform over the work-group, before any barrier
  const int bi_end = min(bi_first + chl, nblk);
  __shared__ T red[kThr / 64];
  __shared__ T sv[(ch_max<T>() + 1) * kTB];
  __shared__ T scol[16][kTB + 1];
  const int cq = threadIdx.x & 15, r0 = threadIdx.x >> 4;
  const T* colbase = A + (int64_t)bj * kTB + 4 * cq;
  Vec4<T> cur[4], nxt[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    cur[k] = load_v4(colbase + ((int64_t)bi_first * kTB + r0 + 16 * k) * lda);
  const int nseg = 1 + bi_end - bi_first;
  for (int t = threadIdx.x; t < nseg * kTB; t += kThr) {
    const int seg = t / kTB, off = t % kTB;
    const int64_t g = (int64_t)(seg == 0 ? bj : bi_first + seg - 1) * kTB + off;
    sv[t] = (g > c + 1 && g < n) ? A[c * lda + g] : 0.f;
  }
  __syncthreads();
  T vc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) vc[u] = sv[4 * cq + u];
  T cacc[4] = {0.f, 0.f, 0.f, 0.f};
  T vav = 0.f;
  for (int bi = bi_first; bi < bi_end; ++bi) {
    if (bi + 1 < bi_end) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        nxt[k] = load_v4(colbase + ((int64_t)(bi + 1) * kTB + r0 + 16 * k) * lda);
    }
    const T* svr = sv + kTB * (1 + bi - bi_first);
    T rs[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) rs[k] = cur[k].x * vc[0] + cur[k].y * vc[1] + cur[k].z * vc[2] + cur[k].w * vc[3];
    if (bi != bj) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const T vr = svr[r0 + 16 * k];
        cacc[0] += cur[k].x * vr;
        cacc[1] += cur[k].y * vr;
        cacc[2] += cur[k].z * vr;
        cacc[3] += cur[k].w * vr;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) rs[k] += __shfl_xor(rs[k], off, 64);
    }
    if (cq == 0) {
      const T wgt = bi == bj ? 1.f : 2.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int rr = r0 + 16 * k;
        Pr[(int64_t)bj * lda + (int64_t)bi * kTB + rr] = rs[k];
        vav += wgt * rs[k] * svr[rr];
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) scol[r0][4 * cq + u] = cacc[u];
  const T vtot = block_sum_t(vav, red);  // contains the barrier that publishes scol
  if (threadIdx.x < kTB) {
    T s = 0.f;
    for (int r = 0; r < 16; ++r) s += scol[r][threadIdx.x];
    Pc[((int64_t)bj * ch_alloc + ch) * kTB + threadIdx.x] = s;
  }
  if (threadIdx.x == 0) Pvv[(int64_t)ch * nblk + bj] = vtot;
}

// Deterministic work-group sums of three values at once (one set of barriers).
template <typename T>
__device__ __forceinline__ void block_sum3(T& a, T& b, T& c, T (*scratch)[kThr / 64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  a = wave_sum_t(a);
  b = wave_sum_t(b);
  c = wave_sum_t(c);
  __syncthreads();
  if (lane == 0) {
    scratch[0][wave] = a;
    scratch[1][wave] = b;
    scratch[2][wave] = c;
  }
  __syncthreads();
  a = scratch[0][0];
  b = scratch[1][0];
  c = scratch[2][0];
  for (int w = 1; w < kThr / 64; ++w) {
    a += scratch[0][w];
    b += scratch[1][w];
    c += scratch[2][w];
  }
}

// Finish reflector i (column c = i0 + i) of the panel and, if do_next, update column c+1.  With
// r = c+1, x the unscaled tail (row c, entries >= c+2), v = e_r + scale x and u = A x (the symv):
//   A v = A[:, r] + scale u,  v^T A v = A_rr + 2 scale u_r + scale^2 x^T u,
//   p_j = W_j . v = W_j[r] + scale W_j . x,  q_j = V_j . v = V_j[r] + scale V_j . x,
//   w = tau (A v - V p - W q) + alpha2 v,  alpha2 = -tau/2 (w . v) = -tau^2/2 (v^T A v - 2 p.q)
//   W[i] = w, row c of A <- v (unit entry at r), E[c] = beta, tau[c] = tau
//   row r of A: a[g] = A[g][r] - sum_{j <= i} V_j[g] W_j[r] + W_j[g] V_j[r]  (g >= r),
//   D[r] = a[r], alph[r] = a[r+1], Pn_out[blk] = sum_{g >= r+2} a[g]^2.
// Every work-group reduces the column's scalars (|x|^2 -> tau, the dots, x^T A x, u_r) from the
// partials itself, in a fixed order, so no grid-wide step is needed.  Eight lanes per row
// g = r + 32 blockIdx + tid / 8: lane k adds the symv partials of strips b0 + k, b0 + k + 8, ...,
// chunks k, k + 8, ... and the reflectors j = k, k + 8, ...; a fixed butterfly over the eight
// lanes completes the sums.
template <typename T>
__global__ __launch_bounds__(kThr) void finish_kernel(T* __restrict__ A, int64_t lda, int64_t n, int64_t c,
                                                     int64_t i0, int i, int do_next, T* __restrict__ alph,
                                                     const T* __restrict__ Pn_in, int npn,
                                                     T* __restrict__ Pn_out, T* __restrict__ Wb,
                                                     const T* __restrict__ Pr, const T* __restrict__ Pc,
                                                     const T* __restrict__ Pvv, const T* __restrict__ Ppq,
                                                     int ch_alloc, int chl, T* __restrict__ D,
                                                     T* __restrict__ E, T* __restrict__ tau) {
  __shared__ T red3[3][kThr / 64];
  __shared__ T spq[4][64];
  __shared__ T sp[kPB], sq[kPB], svr[kPB], swr[kPB];
  const int tid = threadIdx.x, k = tid & (kSub - 1);
  const int64_t r = c + 1;
  const int64_t g = r + (int64_t)blockIdx.x * kRowsPB + (tid / kSub);
  const bool active = g < n;
  const int nblk = (int)(lda / kTB);
  const int b0 = (int)((c + 1) / kTB);
  const int ns = nblk - b0;
  const int chy = (ns + chl - 1) / chl;

  // Every global load of the kernel is issued in one batch before any of them is used: fixed-size,
  // unrolled batches from clamped in-range addresses whose values are selected afterwards.  (A
  // guarded load, or a loop that accumulates while it loads, costs a memory round trip each.)
  // Only trailing matrices above 2 kThr norm partials, kPvBatch kThr symv partials or 32 kSub
  // strips take the remainder loops below.
  constexpr int kPvBatch = 32;
  const int npv = chy * ns;  // x^T A x partials (chunk, strip); some slots hold no chunk
  const int gl = (int)min(g, n - 1);  // in-range row for the loads of inactive threads
  const int s_row = gl / kTB;
  const int nch = (nblk - s_row + chl - 1) / chl;
  const T pn_v0 = Pn_in[min(tid, npn - 1)];
  const T pn_v1 = Pn_in[min(tid + kThr, npn - 1)];
  T pq_v[kDotWG / 4];
  {
    const int slot = tid & 63, part = tid >> 6;
#pragma unroll
    for (int u = 0; u < kDotWG / 4; ++u) pq_v[u] = Ppq[(int64_t)(part * (kDotWG / 4) + u) * 64 + slot];
  }
  // partial idx = tid + kThr u sits at (chunk idx / ns, strip b0 + idx % ns); both indices step
  // by a fixed quotient and remainder (no division per element).  pv_ok bit u: the slot holds a
  // chunk (strip sx has a chunk chx when sx < ns - chl chx).
  T pv_v[kPvBatch];
  unsigned pv_ok = 0u;
  {
    const int q_step = kThr / ns, r_step = kThr % ns;
    int chx = tid / ns, sx = tid % ns;
#pragma unroll
    for (int u = 0; u < kPvBatch; ++u) {
      const int idx = tid + kThr * u;
      pv_v[u] = 0.f;
      if (idx < npv) {
        pv_v[u] = Pvv[(int64_t)chx * nblk + b0 + sx];
        if (sx < ns - chl * chx) pv_ok |= 1u << u;
      }
      sx += r_step;
      chx += q_step;
      if (sx >= ns) {
        sx -= ns;
        ++chx;
      }
    }
  }
  const T ur_c = Pc[((int64_t)b0 * ch_alloc + min(tid, chy - 1)) * kTB + (r % kTB)];
  const T ur_r = Pr[(int64_t)b0 * lda + r];
  const int jr = min(max(tid - 64, 0), max(i - 1, 0));
  const T svr_v = A[(i0 + jr) * lda + r];
  const T swr_v = Wb[(int64_t)jr * lda + r];
  const T arr = A[r * lda + r];
  T pr_v[32];
#pragma unroll
  for (int q = 0; q < 32; ++q) pr_v[q] = Pr[(int64_t)min(b0 + k + kSub * q, s_row) * lda + gl];
  T pc_v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    pc_v[q] = Pc[((int64_t)s_row * ch_alloc + min(k + kSub * q, nch - 1)) * kTB + (gl % kTB)];
  T vj[kPB / kSub], wj[kPB / kSub];
#pragma unroll
  for (int t = 0; t < kPB / kSub; ++t) {
    const int j = min(k + kSub * t, max(i - 1, 0));
    vj[t] = A[(i0 + j) * lda + gl];
    wj[t] = Wb[(int64_t)j * lda + gl];
  }
  T a_c = A[c * lda + gl];
  T a_r = A[(int64_t)gl * lda + r];  // column r, lower triangle

  // column scalars
  T xn2 = tid < npn ? pn_v0 : T(0);
  if (tid + kThr < npn) xn2 += pn_v1;
  for (int t = tid + 2 * kThr; t < npn; t += kThr) xn2 += Pn_in[t];
  T pqp = 0.f;
#pragma unroll
  for (int u = 0; u < kDotWG / 4; ++u) pqp += pq_v[u];
  T xux = 0.f;
#pragma unroll
  for (int u = 0; u < kPvBatch; ++u)
    if (pv_ok & (1u << u)) xux += pv_v[u];
  for (int idx = tid + kThr * kPvBatch; idx < npv; idx += kThr) {
    const int chx = idx / ns, sx = idx % ns;
    if (sx < ns - chl * chx) xux += Pvv[(int64_t)chx * nblk + b0 + sx];
  }
  T ur = tid < chy ? ur_c : T(0);
  if (tid == kThr - 1) ur = ur_r;  // chy < kThr - 1 (checked by the host)
  if (tid >= 64 && tid < 64 + i) {
    svr[tid - 64] = svr_v;
    swr[tid - 64] = swr_v;
  }

  // own row: symv partials (strips b0 .. s_row, chunks 0 .. nch-1 of strip s_row), the earlier
  // reflectors' entries, column r and row c
  T u = 0.f;
  if (active) {
#pragma unroll
    for (int q = 0; q < 32; ++q)
      if (b0 + k + kSub * q <= s_row) u += pr_v[q];
    for (int bj = b0 + k + 32 * kSub; bj <= s_row; bj += kSub) u += Pr[(int64_t)bj * lda + g];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (k + kSub * q < nch) u += pc_v[q];
    for (int ch = k + 4 * kSub; ch < nch; ch += kSub) u += Pc[((int64_t)s_row * ch_alloc + ch) * kTB + (g % kTB)];
  }
#pragma unroll
  for (int t = 0; t < kPB / kSub; ++t) {
    if (!(active && k + kSub * t < i)) vj[t] = wj[t] = 0.f;
  }
  if (!(active && k == 0)) a_c = a_r = 0.f;

  // column scalars: reductions (fixed order)
  spq[tid >> 6][tid & 63] = pqp;
  block_sum3(xn2, xux, ur, red3);  // its barriers also publish spq, svr, swr
  const T alpha = alph[c];
  T tau_c = 0.f, beta = alpha, scale = 0.f;
  if (xn2 != 0.f) {
    beta = -copysign(sqrt(alpha * alpha + xn2), alpha);
    tau_c = (beta - alpha) / beta;
    scale = 1.f / (alpha - beta);
  }
  if (tid < i) {
    sp[tid] = swr[tid] + scale * (spq[0][tid] + spq[1][tid] + spq[2][tid] + spq[3][tid]);
    sq[tid] = svr[tid] + scale * (spq[0][kPB + tid] + spq[1][kPB + tid] + spq[2][kPB + tid] + spq[3][kPB + tid]);
  }
  __syncthreads();
  const T yr = arr + scale * ur;
  const T vAv = arr + scale * (2.f * ur + scale * xux);
  T pq = 0.f, yr_c = yr;
  for (int j = 0; j < i; ++j) {
    pq += sp[j] * sq[j];
    yr_c -= svr[j] * sp[j] + swr[j] * sq[j];
  }
  const T alpha2 = -0.5f * tau_c * (tau_c * (vAv - 2.f * pq));
  const T w0 = tau_c * yr_c + alpha2;

  T sw = 0.f, su = 0.f;
#pragma unroll
  for (int t = 0; t < kPB / kSub; ++t) {
    const int j = k + kSub * t;
    if (j < i) {
      sw += vj[t] * sp[j] + wj[t] * sq[j];
      su += vj[t] * swr[j] + wj[t] * svr[j];
    }
  }
#pragma unroll
  for (int off = 1; off < kSub; off <<= 1) {
    u += __shfl_xor(u, off, 64);
    sw += __shfl_xor(sw, off, 64);
    su += __shfl_xor(su, off, 64);
  }
  T sqv = 0.f;
  if (active && k == 0) {
    const T vg = g == r ? 1.f : a_c * scale;
    const T wg = tau_c * ((a_r + scale * u) - sw) + alpha2 * vg;
    Wb[(int64_t)i * lda + g] = wg;
    A[c * lda + g] = vg;
    if (do_next) {
      const T a = a_r - (su + (vg * w0 + wg));
      // A[r][r] is read by every work-group above (arr): the updated diagonal goes to D only
      if (g != r) A[r * lda + g] = a;
      if (g == r) D[r] = a;
      if (g == r + 1) alph[r] = a;
      if (g >= r + 2) sqv = a * a;
    }
  }
  if (blockIdx.x == 0 && tid == 0) {
    E[c] = beta;
    tau[c] = tau_c;
  }
  if (!do_next) return;  // uniform
  T z1 = 0.f, z2 = 0.f;
  block_sum3(sqv, z1, z2, red3);
  if (tid == 0) Pn_out[blockIdx.x] = sqv;
}

// ---- back-transformation ---------------------------------------------------------------------

// Y (m x nb, row-major, m = n - i0) of reflectors i0 .. i0+nb-1: Y[r'][c] = v_{i0+c}[i0+r'], with
// v_i[i+1] = 1, v_i[r] = A[i][r] for r > i+1, 0 for r <= i.  Starting the rows at i0 (a multiple
// of the block size) keeps the GEMM operands 16-byte aligned.
template <typename T>
__global__ __launch_bounds__(256) void extract_y_kernel(const T* __restrict__ A, int64_t lda, int64_t n,
                                                        int64_t i0, int nb, int64_t off, T* __restrict__ Y) {
  const int64_t m = n - i0;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= m * nb) return;
  const int64_t rp = e / nb;
  const int c = (int)(e % nb);
  const int64_t r = i0 + rp;
  const int64_t i = i0 + c;
  T v = 0.f;
  if (r == i + off) v = 1.f;
  else if (r > i + off) v = A[i * lda + r];
  Y[e] = v;
}

// Tb (nb x nb, row-major, upper) of the compact-WY form H_0 ... H_{nb-1} = I - Y Tb Y^T from the
// gram G = Y^T Y and tau (LAPACK larft, forward, columnwise).  Tb^{-1} = diag(1/tau) + striu(G),
// so Tb = (I + N)^{-1} D with D = diag(tau), N = D striu(G) (strictly upper, nilpotent); the form
// needs no 1/tau, so tau = 0 (H = I) gives zero row and column as larft does.  Thread j < nb
// solves column j of X = (I + N)^{-1} by back substitution, x_k = -sum_{l=k+1..j} N[k][l] x_l,
// x_j = 1; Tb[k][j] = X[k][j] tau_j.  One work-group per block of reflectors: block b holds
// reflectors b NB .. b NB + nb - 1 (nb = NB except for the last, partial block), its gram at
// Gall + b NB^2 and its Tb at Tball + b NB^2 (both nb x nb, leading dimension nb); N and X in LDS
// (2 x 66 KB).
template <typename T>
__global__ __launch_bounds__(256) void larft_kernel(const T* __restrict__ Gall, const T* __restrict__ tau_all,
                                                    int64_t nrefl, T* __restrict__ Tball) {
  constexpr int NBT = NbOf<T>::value;
  const int64_t i0 = (int64_t)blockIdx.x * NBT;
  const int nb = (int)min((int64_t)NBT, nrefl - i0);
  const T* __restrict__ G = Gall + (int64_t)blockIdx.x * NBT * NBT;
  const T* __restrict__ tau = tau_all + i0;
  T* __restrict__ Tb = Tball + (int64_t)blockIdx.x * NBT * NBT;
  __shared__ T sN[NBT][NBT + 1];
  __shared__ T sX[NBT][NBT + 1];
  // 16 global loads in flight per thread (a loop of single loads waits a full memory round trip
  // per element and dominated the kernel)
  for (int e0 = threadIdx.x; e0 < NBT * NBT; e0 += 256 * 16) {
    T v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      // unconditional loads from clamped in-range indices (a guarded load becomes a branch that
      // waits for each load in turn), then a select
      const int e = e0 + 256 * u, k = e / NBT, l = e % NBT;
      const bool use = e < NBT * NBT && k < l && l < nb;
      const int kc = min(k, nb - 1), lc = min(l, nb - 1);
      const T g = G[kc * nb + lc] * tau[kc];
      v[u] = use ? g : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = e0 + 256 * u;
      if (e < NBT * NBT) sN[e / NBT][e % NBT] = v[u];
    }
  }
  __syncthreads();
  // Uniform loop bounds for every thread: sN[k][l] is then one broadcast LDS read per step and
  // sX[l][j] is conflict-free across j; x_l = 0 for l > j makes the extra terms vanish.
  // The l range starts at a multiple of 8 below k+1 (N[k][l] = 0 for l <= k, and for l >= nb)
  // and is unrolled by 8 with four partial sums, so the LDS reads of a chunk overlap.
  const int j = threadIdx.x;
  if (j < nb) {
    for (int l = 0; l < NBT; ++l) sX[l][j] = l == j ? 1.f : 0.f;
    for (int k = nb - 2; k >= 0; --k) {
      T acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int l = (k + 1) & ~7; l < nb; l += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u & 3] += sN[k][l + u] * sX[l + u][j];
      }
      if (k < j) sX[k][j] = -((acc[0] + acc[1]) + (acc[2] + acc[3]));
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nb * nb; e += blockDim.x) {
    const int k = e / nb, l = e % nb;
    Tb[e] = k <= l ? sX[k][l] * tau[l] : 0.f;
  }
}

}  // namespace
}  // namespace mpq

namespace {

using mpq::a64;

// Row-major C (M x N) = alpha A (M x K) op(B) + beta C, op(B) = B (K x N) or B^T (B: N x K), on this
// library's MFMA GEMMs (split-K partials in P when given).
int gemm_rm(const float* A, int64_t lda, const float* B, int64_t ldb, bool trans_b, float* C, int64_t ldc, int64_t M,
            int64_t N, int64_t K, float alpha, float beta, float* P, int64_t p_elems, hipStream_t stream) {
  MPQ_HIP_TRY(mpq::gemm(A, lda, B, ldb, trans_b, nullptr, C, ldc, M, N, K, alpha, beta, P, p_elems, stream));
  return mpq::kOk;
}
int gemm_rm(const double* A, int64_t lda, const double* B, int64_t ldb, bool trans_b, double* C, int64_t ldc,
            int64_t M, int64_t N, int64_t K, double alpha, double beta, double* P, int64_t p_elems,
            hipStream_t stream) {
  MPQ_HIP_TRY(mpq::gemm_f64(A, lda, B, ldb, trans_b, C, ldc, M, N, K, alpha, beta, P, p_elems, stream));
  return mpq::kOk;
}

// Trailing update A[s0:, s0:] -= [V W] [W V]^T (m x m, K = 2 kPB) on the tiles that symv and the
// column reads use: the lower triangle plus a band of kTB - 1 above the diagonal, so the 64 x 64
// diagonal tiles are whole.
int trailing_update(const float* X, const float* Yb, float* C, int64_t ldc, int64_t m, hipStream_t stream) {
  using namespace mpq;
  MPQ_HIP_TRY(gemm_lower(X, 2 * kPB, Yb, 2 * kPB, true, C, ldc, m, 2 * kPB, -1.f, 1.f, kTB - 1, stream));
  return kOk;
}
int trailing_update(const double* X, const double* Yb, double* C, int64_t ldc, int64_t m, hipStream_t stream) {
  using namespace mpq;
  MPQ_HIP_TRY(gemm_f64_lower(X, 2 * kPB, Yb, 2 * kPB, true, C, ldc, m, 2 * kPB, -1.0, 1.0, kTB - 1, stream));
  return kOk;
}

template <typename T>
hipError_t transpose_t(const T* in, int64_t rows, int64_t cols, int64_t ld_in, T* out, int64_t ld_out,
                       hipStream_t stream) {
  hipLaunchKernelGGL(mpq::transpose_t_kernel<T>, dim3((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32)),
                     dim3(256), 0, stream, in, rows, cols, ld_in, out, ld_out);
  return hipGetLastError();
}

// Workspace layout of mpq_syevd / mpq_syevd_f64 (element offsets, each region 64 elements aligned).
struct SyevdLayout {
  int64_t lda, nblk, ch_alloc, pn_stride, splits, nb, Pcap;
  int64_t A, Z, Y, Yt, W, W2, G, Tb, P, D, E, tau, alph, Pn, Wb, X, Yb, Pr, Pc, Pvv, Ppq, dc, wy1, wy3, wyw, total;
};

template <typename T>
SyevdLayout syevd_layout(int64_t n) {
  using namespace mpq;
  SyevdLayout L{};
  L.lda = a64(n);
  L.nblk = L.lda / kTB;
  L.ch_alloc = L.nblk;  // chunks of one tile at the smallest chunk length
  L.pn_stride = a64(L.lda / kRowsPB + 2);
  L.nb = NbOf<T>::value;
  int bn = 64;
  // split-K partials of the back-transformation GEMMs: W = Z Y (n x nb, K up to n) and, in fp64,
  // the grams Y^T Y (nb x nb, K up to n)
  L.splits = sizeof(T) == 4 ? std::max(choose_splits(n, L.nb, n, (int64_t)1 << 62, &bn), 1) : 1;
  int64_t o = 0;
  auto take = [&](int64_t elems) {
    const int64_t at = o;
    o += a64(elems);
    return at;
  };
  L.A = take(L.lda * L.lda);
  L.Z = take(n * n);
  L.Y = take(n * L.nb);
  L.Yt = take(n * L.nb);
  L.W = take(n * L.nb);
  L.W2 = take(n * L.nb);
  // grams and compact-WY factors of every block of reflectors
  const int64_t nblocks = std::max<int64_t>((n - 1 + L.nb - 1) / L.nb, 1);
  L.G = take(nblocks * L.nb * L.nb);
  L.Tb = take(nblocks * L.nb * L.nb);
  L.Pcap = sizeof(T) == 4 ? a64(n * L.nb) * L.splits
                          : std::max<int64_t>(n * L.nb * f64_choose_splits(n, L.nb, n, (int64_t)1 << 62),
                                              L.nb * L.nb * f64_choose_splits(L.nb, L.nb, n, (int64_t)1 << 62));
  L.P = take(L.Pcap);
  L.D = take(n);
  L.E = take(n);
  L.tau = take(n);
  L.alph = take(n);
  L.Pn = take(2 * L.pn_stride);
  L.Wb = take(kPB * L.lda);
  L.X = take(L.lda * 2 * kPB);
  L.Yb = take(L.lda * 2 * kPB);
  L.Pr = take(L.nblk * L.lda);
  L.Pc = take(L.nblk * L.ch_alloc * kTB);
  L.Pvv = take(L.nblk * L.ch_alloc);
  L.Ppq = take(kDotWG * 64);
  L.dc = take((tridiag_dc_workspace_bytes(n, (int)sizeof(T)) + (int64_t)sizeof(T) - 1) / (int64_t)sizeof(T));
  // packed operands of the fp32 back-transformation on the bf16 matrix cores
  const int64_t wyf = sizeof(T) == 4 ? wy_x6_buffer_floats(n) : 0;
  L.wy1 = take(wyf);
  L.wy3 = take(wyf);
  L.wyw = take(wyf);
  L.total = o;
  return L;
}

// A = Q T Q^T for the symmetric A (lda x lda buffer, zero padded): D, E, tau and the reflectors
// in the rows of A.  n >= 2.
template <typename T>
int sytrd(int64_t n, const SyevdLayout& L, T* base, hipStream_t stream) {
  using namespace mpq;
  const int64_t lda = L.lda;
  T* A = base + L.A;
  T* D = base + L.D;
  T* E = base + L.E;
  T* tau = base + L.tau;
  T* alph = base + L.alph;
  T* Pn = base + L.Pn;
  T* Wb = base + L.Wb;
  T* X = base + L.X;
  T* Yb = base + L.Yb;
  T* Pr = base + L.Pr;
  T* Pc = base + L.Pc;
  T* Pvv = base + L.Pvv;
  T* Ppq = base + L.Ppq;
  const int ch_alloc = (int)L.ch_alloc;
  MPQ_HIP_TRY(hipMemsetAsync(Wb, 0, (size_t)kPB * lda * sizeof(T), stream));
  for (int64_t i0 = 0; i0 < n - 1; i0 += kPB) {
    const int nbl = (int)std::min<int64_t>(kPB, n - 1 - i0);
    int npn = (int)((n - i0 + kThr - 1) / kThr);  // partial norms of the current column
    hipLaunchKernelGGL(panel_start_kernel<T>, dim3((unsigned)npn), dim3(kThr), 0, stream, A, lda, n, i0, D, alph,
                       Pn + (i0 & 1) * L.pn_stride);
    MPQ_LAUNCH_CHECK();
    for (int i = 0; i < nbl; ++i) {
      const int64_t c = i0 + i;
      const int ns = (int)L.nblk - (int)((c + 1) / kTB);
      // chunk length: ch_max tiles (fewest partials) except on small trailing matrices, where more
      // and shorter work-groups shorten the kernel
      const int chl = ns > 32 ? ch_max<T>() : 1;
      const int chy = (ns + chl - 1) / chl;
      if (chy >= kThr - 1) {
        set_error("mpq_syevd: internal chunk count %d too large", chy);
        set_error_code(kInvalidArgument);
        return kInvalidArgument;
      }
      // one extra row of work-groups forms the dots p, q
      const dim3 sgrid((unsigned)std::max(ns, kDotWG), (unsigned)(chy + 1));
      T* pn_in = Pn + (c & 1) * L.pn_stride;
      T* pn_out = Pn + ((c + 1) & 1) * L.pn_stride;
      hipLaunchKernelGGL(symv_kernel<T>, sgrid, dim3(kThr), 0, stream, A, lda, n, c, i0, i, Wb, Pr, Pc, Pvv, Ppq,
                         ch_alloc, chl);
      MPQ_LAUNCH_CHECK();
      const int do_next = (i + 1 < nbl) || (c + 1 == n - 1);
      const int fblocks = (int)((n - c - 1 + kRowsPB - 1) / kRowsPB);
      hipLaunchKernelGGL(finish_kernel<T>, dim3((unsigned)fblocks), dim3(kThr), 0, stream, A, lda, n, c, i0, i,
                         do_next, alph, pn_in, npn, pn_out, Wb, Pr, Pc, Pvv, Ppq, ch_alloc, chl, D, E, tau);
      MPQ_LAUNCH_CHECK();
      npn = fblocks;
    }
    const int64_t s0 = i0 + nbl;
    if (s0 < n - 1) {
      // trailing update A[s0:, s0:] -= V W^T + W V^T = [V W] [W V]^T (nbl == kPB here).  fp32 with
      // n % 128 == 0: the update starts at the 128-aligned row sa <= s0 with zero operand rows in
      // [sa, s0), so its square is whole 128-row tiles (the interior-tile GEMM kernel) and the rows
      // and columns in [sa, s0) get exact zero updates.
      const int64_t sa = (sizeof(T) == 4 && n % 128 == 0) ? s0 / 128 * 128 : s0;
      const int64_t m = n - sa;
      const T* Vp = A + i0 * lda + sa;
      const T* Wp = Wb + sa;
      hipLaunchKernelGGL(panel_operands_kernel<T>, dim3((unsigned)((m + 31) / 32)), dim3(256), 0, stream, Vp, Wp,
                         m, s0 - sa, lda, X, Yb);
      MPQ_LAUNCH_CHECK();
      const int rc = trailing_update(X, Yb, A + sa * lda + sa, lda, m, stream);
      if (rc != kOk) return rc;
    }
  }
  return kOk;
}

// Zb (row-major, row k = eigenvector k of the reduced matrix) <- Zb Q^T for the nrefl reflectors
// kept in the rows of A (reflector i: v_i[i + off] = 1, entries past it in row i, tau[i]), applied
// as compact-WY blocks of NB reflectors, last block first:
//    Zb[:, i0:] <- Zb[:, i0:] - ((Zb[:, i0:] Y) Tb^T) Y^T
// The grams Y^T Y of all blocks come first, then one larft launch forms every Tb.
template <typename T>
int back_transform(int64_t n, int64_t off, int64_t nrefl, const SyevdLayout& L, T* base, hipStream_t stream) {
  using namespace mpq;
  T* A = base + L.A;
  T* Z = base + L.Z;
  T* Y = base + L.Y;
  T* Yt = base + L.Yt;
  T* W = base + L.W;
  T* W2 = base + L.W2;
  T* G = base + L.G;
  T* Tb = base + L.Tb;
  T* P = base + L.P;
  T* tau = base + L.tau;
  const int64_t lda = L.lda;
  const int64_t pfl = sizeof(T) == 4 ? (L.splits > 1 ? a64(n * L.nb) * L.splits : 0) : L.Pcap;
  const int NB = (int)L.nb;
  const int64_t nblocks = nrefl > 0 ? (nrefl + NB - 1) / NB : 0;
  int rc;
  for (int64_t b = 0; b < nblocks; ++b) {
    const int64_t i0 = b * NB;
    const int nb = (int)std::min<int64_t>(NB, nrefl - i0);
    const int64_t m = n - i0;
    const int64_t cnt = m * nb;
    hipLaunchKernelGGL(extract_y_kernel<T>, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, stream, A, lda, n,
                       i0, nb, off, Y);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(transpose_t(Y, m, nb, nb, Yt, m, stream));
    if ((rc = gemm_rm(Yt, m, Y, nb, false, G + b * NB * NB, nb, nb, nb, m, T(1), T(0), P, pfl, stream)) != kOk)
      return rc;
  }
  if (nblocks > 0) {
    hipLaunchKernelGGL(larft_kernel<T>, dim3((unsigned)nblocks), dim3(256), 0, stream, G, tau, nrefl, Tb);
    MPQ_LAUNCH_CHECK();
  }
  if constexpr (sizeof(T) == 4) {
    // the blocks' products on the bf16 matrix cores (x6 planes)
    static_assert(NbOf<T>::value == kWyNB, "block size of the x6 back-transformation");
    struct Extract : WyExtractY {
      const float* A;
      int64_t lda, n, off;
      hipStream_t stream;
      int operator()(int64_t i0, int nb, float* Yo) const override {
        const int64_t cnt = (n - i0) * nb;
        hipLaunchKernelGGL(extract_y_kernel<float>, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, stream, A,
                           lda, n, i0, nb, off, Yo);
        MPQ_LAUNCH_CHECK();
        return kOk;
      }
    } ex;
    ex.A = A;
    ex.lda = lda;
    ex.n = n;
    ex.off = off;
    ex.stream = stream;
    // the grams are consumed by larft: their area is the pairs' scratch; W and W2 hold the second block
    const int64_t g_floats = std::max<int64_t>((n - 1 + L.nb - 1) / L.nb, 1) * L.nb * L.nb;
    return wy_apply_x6(n, nrefl, Tb, Z, Y, Yt, W, W2, P, (int)L.splits, G, g_floats, base + L.wy1, base + L.wy3,
                       base + L.wyw, ex, stream);
  }
  for (int64_t b = nblocks - 1; b >= 0; --b) {
    const int64_t i0 = b * NB;
    const int nb = (int)std::min<int64_t>(NB, nrefl - i0);
    const int64_t m = n - i0;
    const int64_t cnt = m * nb;
    const T* Tbb = Tb + b * NB * NB;
    hipLaunchKernelGGL(extract_y_kernel<T>, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, stream, A, lda, n,
                       i0, nb, off, Y);
    MPQ_LAUNCH_CHECK();
    if ((rc = gemm_rm(Z + i0, n, Y, nb, false, W, nb, n, nb, m, T(1), T(0), P, pfl, stream)) != kOk) return rc;
    if ((rc = gemm_rm(W, nb, Tbb, nb, true, W2, nb, n, nb, nb, T(1), T(0), nullptr, 0, stream)) != kOk) return rc;
    if ((rc = gemm_rm(W2, nb, Y, nb, true, Z + i0, n, n, m, nb, T(-1), T(1), nullptr, 0, stream)) != kOk)
      return rc;
  }
  return kOk;
}

// Two-stage path (fp32): stage 1 to a band of half-bandwidth 32, bulge chasing to tridiagonal
// form, divide and conquer, then the bulge-chasing reflectors and the stage-1 reflectors applied
// to the tridiagonal eigenvectors.  The band workspace follows the one-stage layout.
// Sizes the two-stage path handles, and those where it is the faster path on MI355X (measured per
// solve, one-stage vs two-stage: n = 1024 16.3 vs 14.0 ms, 2048 32.1 vs 28.7, 3072 50.0 vs 45.3,
// 4096 68.9 vs 62.7, 6144 125.3 vs 107.5, 8192 201.8 vs 161.5, 14336 640 vs 402; the same residuals).
bool two_stage_ok(int64_t n) { return n >= 3 && n <= mpq::band::kMaxN; }
bool use_two_stage(int64_t n, int elem) { return elem == 4 && n >= 1024 && two_stage_ok(n); }

int syevd_two_stage(int64_t n, const float* H, float* lam, float* V, float* base, const SyevdLayout& L,
                    hipStream_t stream) {
  using namespace mpq;
  const band::Layout BL = band::layout(n);
  float* bws = base + L.total;
  float* A = base + L.A;
  float* Z = base + L.Z;
  const int64_t lda = L.lda;
  MPQ_HIP_TRY(hipMemsetAsync(A, 0, (size_t)(lda * lda) * sizeof(float), stream));
  MPQ_HIP_TRY(hipMemcpy2DAsync(A, lda * sizeof(float), H, n * sizeof(float), n * sizeof(float), n,
                               hipMemcpyDeviceToDevice, stream));
  int rc;
  if ((rc = band::sy2sb(n, A, lda, base + L.tau, bws, BL, stream)) != kOk) return rc;
  if ((rc = band::sb2st(n, A, lda, base + L.D, base + L.E, bws, BL, stream)) != kOk) return rc;
  if ((rc = tridiag_dc(n, base + L.D, base + L.E, lam, Z, base + L.dc, (L.total - L.dc) * (int64_t)sizeof(float),
                       stream)) != kOk)
    return rc;
  if ((rc = band::q2_apply(n, Z, bws, BL, stream)) != kOk) return rc;
  if ((rc = back_transform<float>(n, band::kBW, n - band::kBW, L, base, stream)) != kOk) return rc;
  MPQ_HIP_TRY(transpose_t(Z, n, n, n, V, n, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  return kOk;
}

template <typename T>
int64_t syevd_workspace_elems(int64_t n) {
  const SyevdLayout L = syevd_layout<T>(n);
  return L.total + (sizeof(T) == 4 && two_stage_ok(n) ? mpq::band::layout(n).total : 0);
}

template <typename T>
int syevd_impl(int64_t n, const T* H, T* lam, T* V, void* workspace, int64_t workspace_bytes, hipStream_t stream,
               int method = 0) {
  using namespace mpq;
  MPQ_CHECK_ARG(n > 0 && n <= 46336, "mpq_syevd: n must be in [1, 46336]");
  static_assert(kDotWG % 4 == 0 && 2 * kPB <= 64 && kPB % kSub == 0, "tridiagonalisation constants");
  MPQ_CHECK_ARG(H && lam && V && workspace, "mpq_syevd: null pointer");
  MPQ_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, "mpq_syevd: workspace must be 256-byte aligned");
  const SyevdLayout L = syevd_layout<T>(n);
  const int64_t need = syevd_workspace_elems<T>(n) * (int64_t)sizeof(T);
  MPQ_CHECK_ARG(workspace_bytes >= need, "mpq_syevd: workspace too small (%lld < %lld)",
                (long long)workspace_bytes, (long long)need);
  T* base = static_cast<T*>(workspace);
  if constexpr (sizeof(T) == 4) {
    MPQ_CHECK_ARG(method >= 0 && method <= 2, "mpq_syevd_method: method must be 0 (auto), 1 or 2");
    MPQ_CHECK_ARG(method != 2 || two_stage_ok(n), "mpq_syevd_method: the two-stage path needs 3 <= n <= %lld",
                  (long long)mpq::band::kMaxN);
    if (method == 2 || (method == 0 && use_two_stage(n, 4))) return syevd_two_stage(n, H, lam, V, base, L, stream);
  }
  T* A = base + L.A;
  T* Z = base + L.Z;
  T* D = base + L.D;
  T* E = base + L.E;
  const int64_t lda = L.lda;

  // 1. tridiagonalise (zero-padded copy, leading dimension lda)
  MPQ_HIP_TRY(hipMemsetAsync(A, 0, (size_t)(lda * lda) * sizeof(T), stream));
  MPQ_HIP_TRY(hipMemcpy2DAsync(A, lda * sizeof(T), H, n * sizeof(T), n * sizeof(T), n, hipMemcpyDeviceToDevice,
                               stream));
  if (n == 1) {
    MPQ_HIP_TRY(hipMemcpyAsync(D, A, sizeof(T), hipMemcpyDeviceToDevice, stream));
  } else {
    const int rc = sytrd<T>(n, L, base, stream);
    if (rc != kOk) return rc;
  }
  // 2. tridiagonal eigenproblem
  {
    const int rc = tridiag_dc(n, D, E, lam, Z, base + L.dc, (L.total - L.dc) * (int64_t)sizeof(T), stream);
    if (rc != kOk) return rc;
  }
  // 3. Z column-major = row-major Zb with Zb = Z^T; V^T = Zb Q^T
  {
    const int rc = back_transform<T>(n, 1, n - 1, L, base, stream);
    if (rc != kOk) return rc;
  }
  // V (row-major, columns = eigenvectors) = (Zb)^T
  MPQ_HIP_TRY(transpose_t(Z, n, n, n, V, n, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  return kOk;
}

}  // namespace

extern "C" int64_t mpq_syevd_workspace_size(int64_t n) {
  if (n <= 0) return 0;
  return syevd_workspace_elems<float>(n) * 4;
}

extern "C" int mpq_syevd(int64_t n, const float* H, float* lam, float* V, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream) {
  return syevd_impl<float>(n, H, lam, V, workspace, workspace_bytes, stream);
}

extern "C" int mpq_syevd_method(int64_t n, const float* H, float* lam, float* V, void* workspace,
                                int64_t workspace_bytes, int method, hipStream_t stream) {
  return syevd_impl<float>(n, H, lam, V, workspace, workspace_bytes, stream, method);
}

extern "C" int64_t mpq_syevd_f64_workspace_size(int64_t n) {
  if (n <= 0) return 0;
  return syevd_workspace_elems<double>(n) * 8;
}

extern "C" int mpq_syevd_f64(int64_t n, const double* H, double* lam, double* V, void* workspace,
                             int64_t workspace_bytes, hipStream_t stream) {
  return syevd_impl<double>(n, H, lam, V, workspace, workspace_bytes, stream);
}
