// Divide-and-conquer eigensolver of a symmetric tridiagonal matrix (gfx950): the second stage of
// mpq_syevd / mpq_syevd_f64 (it replaces rocSOLVER stedc there).
//
// Method: Cuppen's divide and conquer with Gu and Eisenstat's stable eigenvectors (the scheme of
// LAPACK stedc / laed0-laed4, written here from the mathematics):
//   * tearing: every off-diagonal entry is a split point, T = diag(T1, T2) + beta v v^T with
//     v = e_{last of T1} + sign(beta) e_{first of T2}, so the leaves are 1 x 1 (eigenvalue
//     d_i - |e_{i-1}| - |e_i|, eigenvector 1) and every level of the binary tree is a merge;
//   * merge of two solved halves: D + rho z z^T with z the halves' eigenvector entries at the tear,
//     |z| = 1, rho = 2 |beta|; deflation of tiny rho |z_i| and of close pairs (a Givens rotation
//     zeroes one z entry) with tolerance 8 u max|D| (u the unit roundoff of the vector type);
//     the secular equation 1 + sum rho z_i^2 / (d_i - lambda) = 0 for each kept root in fp64,
//     solved relative to the nearer pole with a two-pole rational model safeguarded by bisection;
//     Loewner's formula recomputes z from the roots, so the eigenvectors
//     u_j = (zhat_i / (d_i - lambda_j))_i are orthogonal to working precision;
//   * eigenvectors of the merged block = U^T applied to the halves' eigenvectors.
// Merges of at most 512 rows run in one work-group each (all merges of a tree level in one launch).
// Larger merges run one at a time with the GPU-wide kernels below: the kept rows are gathered in
// three groups (rows from the first half only, from both halves after a rotation, from the second
// half only), so the product is two MFMA GEMMs over the nonzero halves (fp32 or fp64 matrix cores).
// Eigenvalues stay in fp64 through the tree.  Storage: Z row-major n x n, row k = eigenvector k;
// a merge of rows [s, s+m) reads and writes only the diagonal block Z[s:s+m, s:s+m].
#include "stedc.h"

#include <algorithm>
#include <vector>

#include "common.h"
#include "gemm.h"
#include "gemm_f64.h"

namespace mpq {
namespace {

constexpr int kDcThr = 256;
constexpr int kSmallMax = 512;   // largest merge handled by one work-group
constexpr int kGrp = 32;         // row-group padding of the large-merge GEMM operands
constexpr double kInvSqrt2 = 0.70710678118654752440;
constexpr double kDblEps = 2.220446049250313e-16;

template <typename T>
struct UnitRoundoff;
template <>
struct UnitRoundoff<float> {
  static constexpr double value = 5.9604644775390625e-08;  // 2^-24
};
template <>
struct UnitRoundoff<double> {
  static constexpr double value = 1.1102230246251565e-16;  // 2^-53
};

inline int64_t rup(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

__device__ __forceinline__ double block_max_f64(double v, double* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  double r = scratch[0];
  for (int w = 1; w < kDcThr / 64; ++w) r = fmax(r, scratch[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_sum_i(int v, int* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  int r = scratch[0];
  for (int w = 1; w < kDcThr / 64; ++w) r += scratch[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Root j (0-based) of f(l) = 1 + sum_i w_i / (dk_i - l), dk ascending and distinct, w_i > 0:
// lambda_j = dk[o] + tau with o the nearer pole (j or j+1; K-1 for the last root, which lies in
// (dk[K-1], dk[K-1] + sum w]).  Each step fits f near the iterate by c + s/(d_j - l) + S/(d_{j+1} - l)
// (s, S matching the derivatives of the sums over the poles left and right of the root) and takes
// the root of that model inside the bracket, else bisects.  Stops when |f| is below its rounding
// error bound or the iterate stops moving.  One wave per root: the sums over the poles are split
// across the 64 lanes (fixed reduction tree; every lane ends with the same iterate).
__device__ void secular_root_wave(const double* __restrict__ dk, const double* __restrict__ w, int K, int j,
                                  int* o_out, double* tau_out) {
  const int lane = threadIdx.x & 63;
  int o;
  double lo, hi;
  if (j < K - 1) {
    const double dj = dk[j];
    const double mid = 0.5 * (dk[j + 1] - dj);
    double fm = 0.0;
    for (int i = lane; i < K; i += 64) fm += w[i] / ((dk[i] - dj) - mid);
    fm = 1.0 + wave_sum_f64(fm);
    if (fm >= 0.0) {
      o = j;
      lo = 0.0;
      hi = mid;
    } else {
      o = j + 1;
      lo = -mid;
      hi = 0.0;
    }
  } else {
    o = K - 1;
    lo = 0.0;
    double sw = 0.0;
    for (int i = lane; i < K; i += 64) sw += w[i];
    hi = wave_sum_f64(sw);
  }
  const double dor = dk[o];
  double tau = 0.5 * (lo + hi);
  for (int it = 0; it < 80; ++it) {
    double psi = 0.0, phi = 0.0, dpsi = 0.0, dphi = 0.0;
    for (int i = lane; i < K; i += 64) {
      const double r = 1.0 / ((dk[i] - dor) - tau);
      const double t = w[i] * r;
      if (i <= j) {
        psi += t;
        dpsi += t * r;
      } else {
        phi += t;
        dphi += t * r;
      }
    }
    psi = wave_sum_f64(psi);
    phi = wave_sum_f64(phi);
    dpsi = wave_sum_f64(dpsi);
    dphi = wave_sum_f64(dphi);
    const double f = 1.0 + psi + phi;
    if (f > 0.0) hi = tau;
    else lo = tau;
    if (fabs(f) <= 4.0 * K * kDblEps * (1.0 + fabs(psi) + fabs(phi))) break;
    double tn = 0.5 * (lo + hi);
    if (j < K - 1) {
      const double Dj = (dk[j] - dor) - tau, Dj1 = (dk[j + 1] - dor) - tau;
      const double s = Dj * Dj * dpsi, S = Dj1 * Dj1 * dphi;
      const double c = f - s / Dj - S / Dj1;
      const double a1 = -(c * (Dj + Dj1) + s + S);
      const double a0 = c * Dj * Dj1 + s * Dj1 + S * Dj;
      double r1 = 0.0, r2 = 0.0;
      bool have = false;
      if (c == 0.0) {
        if (a1 != 0.0) {
          r1 = r2 = -a0 / a1;
          have = true;
        }
      } else {
        const double disc = fmax(a1 * a1 - 4.0 * c * a0, 0.0);
        const double q = -0.5 * (a1 + copysign(sqrt(disc), a1));
        if (q != 0.0) {
          r1 = q / c;
          r2 = a0 / q;
          have = true;
        }
      }
      if (have) {
        const bool in1 = tau + r1 > lo && tau + r1 < hi;
        const bool in2 = tau + r2 > lo && tau + r2 < hi;
        if (in1 && in2) tn = tau + (fabs(r1) < fabs(r2) ? r1 : r2);
        else if (in1) tn = tau + r1;
        else if (in2) tn = tau + r2;
      }
    } else {
      const double DK = -tau;
      const double s = DK * DK * dpsi;
      const double c = f - s / DK;
      if (c != 0.0) {
        const double cand = tau + DK + s / c;
        if (cand > lo && cand < hi) tn = cand;
      }
    }
    if (!(tn > lo && tn < hi)) tn = 0.5 * (lo + hi);
    if (tn == tau) break;
    tau = tn;
  }
  *o_out = o;
  *tau_out = tau;
}

// Loewner: zhat_i^2 = (lambda_{K-1} - d_i) / rho2 * prod_{j<i} (lambda_j - d_i) / (d_j - d_i)
//                     * prod_{i<=j<K-1} (lambda_j - d_i) / (d_{j+1} - d_i)   (every factor > 0),
// with lambda_j - d_i = (d_{o_j} - d_i) + tau_j; the sign is that of z_i.  The product is split over
// the 64 lanes of a wave (every lane returns the value).
__device__ double loewner_wave(const double* __restrict__ dk, const int* __restrict__ o,
                               const double* __restrict__ tau, double rho2, int K, int i, double zsign) {
  const int lane = threadIdx.x & 63;
  const double di = dk[i];
  double p = 1.0;
  for (int j = lane; j < K - 1; j += 64) p *= ((dk[o[j]] - di) + tau[j]) / (j < i ? dk[j] - di : dk[j + 1] - di);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) p *= __shfl_xor(p, off, 64);
  p *= ((dk[o[K - 1]] - di) + tau[K - 1]) / rho2;
  return copysign(sqrt(fmax(p, 0.0)), zsign);
}

// ---- tree set-up ---------------------------------------------------------------------------------

// Leaves: lam_i = d_i - |e_{i-1}| - |e_i| (every off-diagonal entry is a tear), Z_ii = 1.
template <typename T>
__global__ __launch_bounds__(256) void dc_init_kernel(int64_t n, const T* __restrict__ d, const T* __restrict__ e,
                                                      double* __restrict__ lam, T* __restrict__ Z) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  double v = (double)d[i];
  if (i > 0) v -= fabs((double)e[i - 1]);
  if (i < n - 1) v -= fabs((double)e[i]);
  lam[i] = v;
  Z[i * n + i] = T(1);
}

template <typename T>
__global__ __launch_bounds__(256) void dc_out_kernel(int64_t n, const double* __restrict__ lam, T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (T)lam[i];
}

// ---- merges of at most MAXM rows: one work-group each ---------------------------------------------

// Shared by both merge paths: z of the merge (rows < h from the first half: their entry in the
// half's last column; rows >= h: sign(beta) x their entry in the second half's first column),
// scaled by 1/sqrt(2), and the position of every row in the merged ascending order of the halves'
// eigenvalues (first half first on ties).
__device__ __forceinline__ int merged_position(const double* __restrict__ lam, int64_t s, int h, int m, int i,
                                               double di) {
  if (i < h) {
    int lo = h, hi = m;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (lam[s + mid] < di) lo = mid + 1;
      else hi = mid;
    }
    return i + (lo - h);
  }
  int lo = 0, hi = h;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (lam[s + mid] <= di) lo = mid + 1;
    else hi = mid;
  }
  return (i - h) + lo;
}

// Per-merge results the small-merge product reads (all indexed from the merge's first row s).
struct SmallOut {
  double *kD, *kZ, *kW, *dV, *rT, *zh, *inrm, *rC, *rS;
  int *rO, *pos, *slot, *rP, *rQ;  // rP, rQ: gathered slots of the rotations, in order
  int* cnt;                         // cnt[3 s] = K, cnt[3 s + 1] = number deflated, cnt[3 s + 2] = rotations
};

// Set-up of a merge of at most MAXM rows (one work-group): sort, deflation, the slots of the
// gathered rows (kept rows first) and the rotations on them, roots, Loewner z, column norms and the
// merged order.  The gather, rotation and product kernels below do the rest.
template <typename T, int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_merge_kernel(int64_t n, const int* __restrict__ nodes,
                                                                const T* __restrict__ e, double* __restrict__ lam,
                                                                const T* __restrict__ Z, double u, SmallOut so) {
  __shared__ double sD[MAXM], sZ[MAXM], kD[MAXM], kW[MAXM], kZ[MAXM], dV[MAXM], rC[MAXM], rS[MAXM];
  __shared__ int sSrc[MAXM], kSrc[MAXM], dSrc[MAXM], rP[MAXM], rQ[MAXM], slot[MAXM];
  __shared__ double red[kDcThr / 64];
  __shared__ int cnt[3];
  const int tid = threadIdx.x;
  const int64_t s = nodes[3 * blockIdx.x];
  const int m = nodes[3 * blockIdx.x + 1], h = nodes[3 * blockIdx.x + 2];
  const double beta = (double)e[s + h - 1];
  const double rho2 = 2.0 * fabs(beta);
  const double sgn = beta >= 0.0 ? 1.0 : -1.0;

  double dmax = 0.0;
  for (int i = tid; i < m; i += kDcThr) {
    const double di = lam[s + i];
    const double zi = i < h ? (double)Z[(s + i) * n + (s + h - 1)] : sgn * (double)Z[(s + i) * n + (s + h)];
    const int p = merged_position(lam, s, h, m, i, di);
    sD[p] = di;
    sZ[p] = zi * kInvSqrt2;
    sSrc[p] = i;
    dmax = fmax(dmax, fabs(di));
  }
  dmax = block_max_f64(dmax, red);  // its barriers publish sD, sZ, sSrc
  const double tol = 8.0 * u * dmax;

  // deflation scan in ascending order (one thread)
  if (tid == 0) {
    int K = 0, nd = 0, nr = 0, pj = -1, pS = 0;
    double pD = 0.0, pZ = 0.0;
    for (int t = 0; t < m; ++t) {
      const double Dt = sD[t], zt = sZ[t];
      const int st = sSrc[t];
      if (rho2 * fabs(zt) <= tol) {
        dV[nd] = Dt;
        dSrc[nd++] = st;
        continue;
      }
      if (pj < 0) {
        pj = t;
        pD = Dt;
        pZ = zt;
        pS = st;
        continue;
      }
      // |t c s| <= tol with c = z_q / tau, s = -z_p / tau, tau^2 = z_p^2 + z_q^2
      if (fabs(Dt - pD) * fabs(zt * pZ) <= tol * (zt * zt + pZ * pZ)) {
        const double tau = hypot(zt, pZ);
        const double c = zt / tau, sn = -pZ / tau;
        // rows p (deflated) <- c p + sn q, q <- -sn p + c q: z_p = 0, z_q = tau
        rP[nr] = pS;
        rQ[nr] = st;
        rC[nr] = c;
        rS[nr++] = sn;
        dV[nd] = pD * c * c + Dt * sn * sn;
        dSrc[nd++] = pS;
        pD = pD * sn * sn + Dt * c * c;
        pZ = tau;
        pS = st;
        pj = t;
      } else {
        kD[K] = pD;
        kZ[K] = pZ;
        kSrc[K++] = pS;
        pj = t;
        pD = Dt;
        pZ = zt;
        pS = st;
      }
    }
    if (pj >= 0) {
      kD[K] = pD;
      kZ[K] = pZ;
      kSrc[K++] = pS;
    }
    cnt[0] = K;
    cnt[1] = nd;
    cnt[2] = nr;
  }
  __syncthreads();
  const int K = cnt[0], nd = cnt[1], nr = cnt[2];
  // gathered row slots: kept k -> k, deflated r -> K + r
  for (int k = tid; k < K; k += kDcThr) {
    slot[kSrc[k]] = k;
    kW[k] = rho2 * kZ[k] * kZ[k];
  }
  for (int r = tid; r < nd; r += kDcThr) slot[dSrc[r]] = K + r;
  __syncthreads();
  // slots and rotations for the gather and rotation kernels
  for (int i = tid; i < m; i += kDcThr) so.slot[s + i] = slot[i];
  for (int r = tid; r < nr; r += kDcThr) {
    so.rP[s + r] = slot[rP[r]];
    so.rQ[s + r] = slot[rQ[r]];
    so.rC[s + r] = rC[r];
    so.rS[s + r] = rS[r];
  }
  for (int k = tid; k < K; k += kDcThr) {
    so.kD[s + k] = kD[k];
    so.kZ[s + k] = kZ[k];
    so.kW[s + k] = kW[k];
  }
  for (int r = tid; r < nd; r += kDcThr) so.dV[s + r] = dV[r];
  if (tid == 0) {
    so.cnt[3 * s] = K;
    so.cnt[3 * s + 1] = nd;
    so.cnt[3 * s + 2] = nr;
  }
}

// Gathered rows of the small merges: slot row = merge row i, zero outside its half.  Work-group
// (merge, 4 rows), one wave per row.
template <typename T, int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_gather_kernel(int64_t n, const int* __restrict__ nodes,
                                                                 const T* __restrict__ Z, SmallOut so,
                                                                 T* __restrict__ S) {
  const int64_t s = nodes[3 * blockIdx.x];
  const int m = nodes[3 * blockIdx.x + 1], h = nodes[3 * blockIdx.x + 2];
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= m) return;
  const int lane = threadIdx.x & 63;
  T* dst = S + s * MAXM + (int64_t)so.slot[s + i] * MAXM;
  const T* src = Z + (s + i) * n + s;
  const bool top = i < h;
  constexpr int PER = (MAXM + 63) / 64;
  T v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int c = lane + 64 * q;
    v[q] = (c < m && top == (c < h)) ? src[c] : T(0);
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int c = lane + 64 * q;
    if (c < m) dst[c] = v[q];
  }
}

// The small merges' deflation rotations on the gathered rows (one column per thread; the same
// eight-rotation prefetch as the large-merge rotation kernel).
template <typename T, int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_rotate_kernel(const int* __restrict__ nodes, SmallOut so,
                                                                 T* __restrict__ S) {
  const int64_t s = nodes[3 * blockIdx.x];
  const int m = nodes[3 * blockIdx.x + 1];
  const int c = blockIdx.y * kDcThr + threadIdx.x;
  if (c >= m) return;
  const int nr = so.cnt[3 * s + 2];
  T* __restrict__ Sb = S + s * MAXM;
  const int* __restrict__ rP = so.rP + s;
  const int* __restrict__ rQ = so.rQ + s;
  const double* __restrict__ rC = so.rC + s;
  const double* __restrict__ rS = so.rS + s;
  int last = -1;
  double lastv = 0.0;
  for (int r0 = 0; r0 < nr; r0 += 8) {
    int pv[8], qv[8];
    double av[8], bv[8], cv[8], sv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r = min(r0 + k, nr - 1);
      pv[k] = rP[r];
      qv[k] = rQ[r];
      cv[k] = rC[r];
      sv[k] = rS[r];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      av[k] = (double)Sb[(int64_t)pv[k] * MAXM + c];
      bv[k] = (double)Sb[(int64_t)qv[k] * MAXM + c];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (r0 + k >= nr) break;
      const double a = pv[k] == last ? lastv : av[k];
      const double na = cv[k] * a + sv[k] * bv[k], nb = -sv[k] * a + cv[k] * bv[k];
      Sb[(int64_t)pv[k] * MAXM + c] = (T)na;
      Sb[(int64_t)qv[k] * MAXM + c] = (T)nb;
      last = qv[k];
      lastv = (double)(T)nb;
    }
  }
}

// Roots of the small merges: one wave per root.  Work-group (merge, 4 roots).
template <int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_secular_kernel(const int* __restrict__ nodes, SmallOut so) {
  const int64_t s = nodes[3 * blockIdx.x];
  const int K = so.cnt[3 * s];
  const int j = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (j >= K) return;  // uniform over the wave
  int o;
  double tau;
  secular_root_wave(so.kD + s, so.kW + s, K, j, &o, &tau);
  if ((threadIdx.x & 63) == 0) {
    so.rO[s + j] = o;
    so.rT[s + j] = tau;
  }
}

// Loewner z of the small merges: one wave per kept pole.
template <typename T, int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_loewner_kernel(const int* __restrict__ nodes,
                                                                  const T* __restrict__ e, SmallOut so) {
  const int64_t s = nodes[3 * blockIdx.x];
  const int h = nodes[3 * blockIdx.x + 2];
  const int K = so.cnt[3 * s];
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= K) return;  // uniform over the wave
  const double rho2 = 2.0 * fabs((double)e[s + h - 1]);
  const double v = loewner_wave(so.kD + s, so.rO + s, so.rT + s, rho2, K, i, so.kZ[s + i]);
  if ((threadIdx.x & 63) == 0) so.zh[s + i] = v;
}

// Column norms of the rank-one eigenvector matrix (one wave per root) and the merged order of the
// small merges' eigenvalues (one wave per output: kept root t before the deflated values above it,
// ties among deflated by index); writes lam.
template <int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_order_kernel(const int* __restrict__ nodes, double* __restrict__ lam,
                                                                SmallOut so) {
  const int64_t s = nodes[3 * blockIdx.x];
  const int m = nodes[3 * blockIdx.x + 1];
  const int K = so.cnt[3 * s], nd = so.cnt[3 * s + 1];
  const int t = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= m) return;  // uniform over the wave
  const double* __restrict__ kD = so.kD + s;
  const double* __restrict__ rT = so.rT + s;
  const int* __restrict__ rO = so.rO + s;
  const double* __restrict__ dV = so.dV + s;
  double val;
  int c = 0;
  if (t < K) {
    const double dor = kD[rO[t]], tau = rT[t];
    double ss = 0.0;
    for (int i = lane; i < K; i += 64) {
      const double v = so.zh[s + i] / ((kD[i] - dor) - tau);
      ss += v * v;
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) so.inrm[s + t] = 1.0 / sqrt(ss);
    val = dor + tau;
    for (int r = lane; r < nd; r += 64) c += dV[r] < val;
    c += t * (lane == 0);
  } else {
    const int r = t - K;
    val = dV[r];
    for (int q = lane; q < nd; q += 64) c += (dV[q] < val) || (dV[q] == val && q < r);
    for (int j = lane; j < K; j += 64) c += kD[rO[j]] + rT[j] <= val;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
  if (lane == 0) {
    so.pos[s + t] = c;
    lam[s + c] = val;
  }
}

// Product of a small merge: output row t of the merge is root t (t < K: sum_i U[i][t] times
// gathered kept row i, U computed here from the roots) or the deflated gathered row t (t >= K),
// written to Z row s + pos[t].  Work-group (merge, 64-column panel, 32-row block); thread =
// (column, 8 rows); U in LDS for 128 kept rows at a time.
constexpr int kSpRows = 32, kSpCols = 64, kSpK = 128;
template <typename T, int MAXM>
__global__ __launch_bounds__(kDcThr) void dc_small_product_kernel(int64_t n, const int* __restrict__ nodes,
                                                                  const T* __restrict__ S, SmallOut so,
                                                                  T* __restrict__ Z) {
  __shared__ T UT[kSpRows][kSpK + 1];
  const int64_t s = nodes[3 * blockIdx.x];
  const int m = nodes[3 * blockIdx.x + 1];
  const int c0 = blockIdx.y * kSpCols, t0 = blockIdx.z * kSpRows;
  if (c0 >= m || t0 >= m) return;  // uniform
  const int K = so.cnt[3 * s];
  const T* __restrict__ Sb = S + s * MAXM;
  const int cl = threadIdx.x & (kSpCols - 1), rg = threadIdx.x / kSpCols;  // rg: rows rg*8 .. rg*8+7
  const int c = c0 + cl;
  const int cc = min(c, m - 1);
  if (t0 >= K) {  // deflated rows only: copies
    for (int r = 0; r < 8; ++r) {
      const int t = t0 + rg * 8 + r;
      if (t < m && c < m) Z[(s + so.pos[s + t]) * n + s + c] = Sb[(int64_t)t * MAXM + c];
    }
    return;
  }
  T acc[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) acc[r] = T(0);
  for (int i0 = 0; i0 < K; i0 += kSpK) {
    const int ni = min(kSpK, K - i0);
    __syncthreads();
    for (int e2 = threadIdx.x; e2 < kSpRows * kSpK; e2 += kDcThr) {
      const int r = e2 / kSpK, ii = e2 % kSpK, j = t0 + r, i = i0 + ii;
      T v = T(0);
      if (j < K && ii < ni) {
        const double dor = so.kD[s + so.rO[s + j]];
        v = (T)(so.zh[s + i] / ((so.kD[s + i] - dor) - so.rT[s + j]) * so.inrm[s + j]);
      }
      UT[r][ii] = v;
    }
    __syncthreads();
    for (int ib = 0; ib < ni; ib += 16) {
      T sv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) sv[q] = Sb[(int64_t)(i0 + min(ib + q, ni - 1)) * MAXM + cc];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[r] += UT[rg * 8 + r][ib + q] * sv[q];
      }
    }
  }
  for (int r = 0; r < 8; ++r) {
    const int t = t0 + rg * 8 + r;
    if (t >= m || c >= m) continue;
    T* dst = Z + (s + so.pos[s + t]) * n + s + c;
    *dst = t < K ? acc[r] : Sb[(int64_t)t * MAXM + c];
  }
}

// ---- merges of more than 512 rows: one merge at a time, GPU-wide kernels -------------------------

struct LargeBufs {
  double *Ds, *Zs, *kD, *kZ, *kW, *dV, *rC, *rS, *rT, *lamK, *zh, *misc;
  int *Ss, *kSrc, *kType, *kSlot, *dSrc, *rP, *rQ, *slot_of_row, *row_of_slot, *rO, *info;
  // deflation walk: non-tiny poles, their state, candidate pairs
  int *Lt, *stat, *modT, *cK, *cS0, *cS1;
  double *modD, *modZ, *cD0, *cZ0, *cD1, *cZ1;
};

// info: K, n1, n2, n3, n1p, n2p, n3p, Kc, nd, nr, Kr
enum { kiK = 0, kiN1, kiN2, kiN3, kiN1p, kiN2p, kiN3p, kiKc, kiNd, kiNr, kiKr, kiCount };

// z and the merged ascending order of one large merge (one thread per row), and per-work-group
// maxima of |D| in misc[kMiscMax + blockIdx.x].
constexpr int kMiscMax = 8;
template <typename T>
__global__ __launch_bounds__(kDcThr) void dc_sort_kernel(int64_t n, int64_t s, int m, int h, const T* __restrict__ e,
                                                         const double* __restrict__ lam, const T* __restrict__ Z,
                                                         LargeBufs b) {
  __shared__ double red[kDcThr / 64];
  const int i = blockIdx.x * kDcThr + threadIdx.x;
  const double beta = (double)e[s + h - 1];
  const double sgn = beta >= 0.0 ? 1.0 : -1.0;
  double dm = 0.0;
  if (i < m) {
    const double di = lam[s + i];
    const double zi = i < h ? (double)Z[(s + i) * n + (s + h - 1)] : sgn * (double)Z[(s + i) * n + (s + h)];
    const int p = merged_position(lam, s, h, m, i, di);
    b.Ds[p] = di;
    b.Zs[p] = zi * kInvSqrt2;
    b.Ss[p] = i;
    dm = fabs(di);
  }
  dm = block_max_f64(dm, red);
  if (threadIdx.x == 0) b.misc[kMiscMax + blockIdx.x] = dm;
}

// Exclusive prefix sum of one int per thread over the work-group; *total gets the sum.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  __syncthreads();
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < nwave; ++w) {
    if (w < wave) base += wsum[w];
    tot += wsum[w];
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

// Deflation of one large merge, row groups and slots.  The sequential rule (scan the sorted poles;
// a tiny rho |z| deflates; a pending pole p and the next pole q deflate p by a rotation when
// |t c s| <= tol, q then carrying the rotated values) is evaluated as:
//   A. the non-tiny poles in order (list L), in parallel;
//   B. the pairs (L_k, L_{k+1}) that pass the test with their original values, in parallel: a
//      pair whose first pole was not rotated into can only deflate if it is one of these;
//   C. thread 0 walks these candidate pairs in order (staged in LDS), following each chain of
//      rotations, and tests the pairs that a rotated pole reaches outside the candidates with the
//      next pole fetched from memory;
//   D. kept and deflated lists by parallel compaction.
constexpr int kWalkChunk = 512;
constexpr int kPlanThr = 1024;
template <typename T>
__global__ __launch_bounds__(kPlanThr) void dc_plan_kernel(int64_t s, int m, int h, const T* __restrict__ e, double u,
                                                           LargeBufs b) {
  __shared__ int wsum[kPlanThr / 64];
  __shared__ int grp[8];
  __shared__ int cnt[4];
  __shared__ int wk[kWalkChunk], ws0[kWalkChunk], ws1[kWalkChunk];
  __shared__ double wd0[kWalkChunk], wz0[kWalkChunk], wd1[kWalkChunk], wz1[kWalkChunk];
  const int tid = threadIdx.x;
  const double rho2 = 2.0 * fabs((double)e[s + h - 1]);
  __shared__ double wmax[kPlanThr / 64];
  double dmax = 0.0;
  for (int q = tid; q < (m + kDcThr - 1) / kDcThr; q += kPlanThr) dmax = fmax(dmax, b.misc[kMiscMax + q]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) dmax = fmax(dmax, __shfl_xor(dmax, off, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = dmax;
  __syncthreads();
  dmax = 0.0;
  for (int w = 0; w < kPlanThr / 64; ++w) dmax = fmax(dmax, wmax[w]);
  const double tol = 8.0 * u * dmax;
  auto is_small = [&](int t) { return rho2 * fabs(b.Zs[t]) <= tol; };
  auto pair_test = [&](double Dp, double zp, double Dq, double zq) {
    // |t c s| <= tol with t = Dq - Dp, c = zq / tau, s = -zp / tau, tau^2 = zp^2 + zq^2
    return fabs(Dq - Dp) * fabs(zq * zp) <= tol * (zq * zq + zp * zp);
  };
  auto half_of = [&](int src) { return src < h ? 1 : 3; };

  const double* __restrict__ Ds = b.Ds;
  const double* __restrict__ Zs = b.Zs;
  const int* __restrict__ Ss = b.Ss;
  double* __restrict__ LD = b.modD + m;  // L-ordered copies of the non-tiny poles (the second half
  double* __restrict__ LZ = b.modZ + m;  // of the mod arrays; m + nL <= 2 m <= their length)
  int* __restrict__ LS = b.Lt;
  // A
  const int cha = (m + kPlanThr - 1) / kPlanThr;
  const int a0 = min(tid * cha, m), a1 = min(a0 + cha, m);
  int nls = 0;
#pragma unroll 8
  for (int t = a0; t < a1; ++t) nls += !is_small(t);
  int nL;
  {
    int base = block_excl_scan(nls, wsum, &nL);
    for (int t = a0; t < a1; ++t) {
      const double z = Zs[t];
      if (!(rho2 * fabs(z) <= tol)) {
        LD[base] = Ds[t];
        LZ[base] = z;
        LS[base++] = Ss[t];
      }
    }
  }
  const int nsmall_mine = (a1 - a0) - nls;
  __syncthreads();
  // B
  const int npair = nL > 0 ? nL - 1 : 0;
  const int chb = (npair + kPlanThr - 1) / kPlanThr;
  const int b0 = min(tid * chb, npair), b1 = min(b0 + chb, npair);
  int ncand = 0;
#pragma unroll 8
  for (int k = b0; k < b1; ++k) ncand += pair_test(LD[k], LZ[k], LD[k + 1], LZ[k + 1]);
  int nC;
  {
    int cb = block_excl_scan(ncand, wsum, &nC);
    for (int k = b0; k < b1; ++k) {
      if (pair_test(LD[k], LZ[k], LD[k + 1], LZ[k + 1])) {
        b.cK[cb] = k;
        b.cD0[cb] = LD[k];
        b.cZ0[cb] = LZ[k];
        b.cS0[cb] = LS[k];
        b.cD1[cb] = LD[k + 1];
        b.cZ1[cb] = LZ[k + 1];
        b.cS1[cb] = LS[k + 1];
        ++cb;
      }
    }
  }
  for (int k = tid; k < nL; k += kPlanThr) b.stat[k] = 0;
  __syncthreads();
  // C (thread 0; the chain state lives in its registers across chunks)
  int nr = 0, cur = 0, ck = 0, pS = 0, pT = 0;
  bool act = false;
  double pD = 0.0, pZ = 0.0;
  // rotate pending pole L_ck (pD, pZ, pS, pT) with q = L_{ck+1} (qD, qZ, qS): L_ck deflates, q is pending
  auto rotate = [&](double qD, double qZ, int qS) {
    // z entries are below 1 in magnitude and above the tiny-z tolerance: no scaling needed
    const double tau = sqrt(qZ * qZ + pZ * pZ);
    const double it = 1.0 / tau;
    const double c = qZ * it, sn = -pZ * it;
    b.rP[nr] = pS;
    b.rQ[nr] = qS;
    b.rC[nr] = c;
    b.rS[nr++] = sn;
    b.stat[ck] = 2;
    b.modD[ck] = pD * c * c + qD * sn * sn;
    const int qT = half_of(qS);
    pD = pD * sn * sn + qD * c * c;
    pZ = tau;
    pS = qS;
    pT = (pT != qT) ? 2 : qT;
    ++ck;
    b.stat[ck] = 1;
    b.modD[ck] = pD;
    b.modZ[ck] = pZ;
    b.modT[ck] = pT;
  };
  // advance the active chain through pairs that are not candidates, up to pair `upto`
  auto extend = [&](int upto) {
    while (act && ck < upto && ck + 1 < nL) {
      const double qD = LD[ck + 1], qZ = LZ[ck + 1];
      if (pair_test(pD, pZ, qD, qZ)) {
        rotate(qD, qZ, LS[ck + 1]);
      } else {
        act = false;
        cur = ck + 1;
      }
    }
    if (act && ck + 1 >= nL) act = false;
  };
  for (int c0 = 0; c0 < nC; c0 += kWalkChunk) {
    const int cn = min(kWalkChunk, nC - c0);
    for (int i = tid; i < cn; i += kPlanThr) {
      wk[i] = b.cK[c0 + i];
      wd0[i] = b.cD0[c0 + i];
      wz0[i] = b.cZ0[c0 + i];
      ws0[i] = b.cS0[c0 + i];
      wd1[i] = b.cD1[c0 + i];
      wz1[i] = b.cZ1[c0 + i];
      ws1[i] = b.cS1[c0 + i];
    }
    __syncthreads();
    if (tid == 0) {
      for (int i = 0; i < cn; ++i) {
        const int k = wk[i];
        extend(k);
        if (k < cur) continue;
        if (!act) {  // a fresh pending pole
          pD = wd0[i];
          pZ = wz0[i];
          pS = ws0[i];
          pT = half_of(pS);
          ck = k;
        }
        if (pair_test(pD, pZ, wd1[i], wz1[i])) {
          rotate(wd1[i], wz1[i], ws1[i]);
          act = ck + 1 < nL;
        } else {
          act = false;
          cur = k + 1;
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    extend(nL);
    cnt[0] = nr;
  }
  __syncthreads();
  nr = cnt[0];
  // D
  const int chd = (nL + kPlanThr - 1) / kPlanThr;
  const int d0 = min(tid * chd, nL), d1 = min(d0 + chd, nL);
  int nk = 0, nrot_mine = 0;
  for (int k = d0; k < d1; ++k) {
    const int st = b.stat[k];
    nk += st != 2;
    nrot_mine += st == 2;
  }
  int K, nd;
  {
    int kb = block_excl_scan(nk, wsum, &K);
    for (int k = d0; k < d1; ++k) {
      const int st = b.stat[k];
      if (st == 2) continue;
      const int src = LS[k];
      b.kSrc[kb] = src;
      if (st == 1) {
        b.kD[kb] = b.modD[k];
        b.kZ[kb] = b.modZ[k];
        b.kType[kb] = b.modT[k];
      } else {
        b.kD[kb] = LD[k];
        b.kZ[kb] = LZ[k];
        b.kType[kb] = half_of(src);
      }
      ++kb;
    }
    int db = block_excl_scan(nsmall_mine + nrot_mine, wsum, &nd);
    for (int t = a0; t < a1; ++t) {
      if (is_small(t)) {
        b.dV[db] = Ds[t];
        b.dSrc[db++] = Ss[t];
      }
    }
    for (int k = d0; k < d1; ++k) {
      if (b.stat[k] == 2) {
        b.dV[db] = b.modD[k];
        b.dSrc[db++] = LS[k];
      }
    }
  }
  __syncthreads();
  // row groups: thread t takes kept entries [t ch, (t+1) ch) in order
  const int ch = (K + kPlanThr - 1) / kPlanThr;
  const int k0 = min(tid * ch, K), k1 = min(k0 + ch, K);
  int c1 = 0, c2 = 0, c3 = 0;
  for (int k = k0; k < k1; ++k) {
    const int ty = b.kType[k];
    c1 += ty == 1;
    c2 += ty == 2;
    c3 += ty == 3;
  }
  int n1, n2, n3;
  const int e1 = block_excl_scan(c1, wsum, &n1);
  const int e2 = block_excl_scan(c2, wsum, &n2);
  const int e3 = block_excl_scan(c3, wsum, &n3);
  if (tid == 0) {
    grp[0] = n1;
    grp[1] = n2;
    grp[2] = n3;
  }
  const int n1p = (n1 + kGrp - 1) / kGrp * kGrp, n2p = (n2 + kGrp - 1) / kGrp * kGrp;
  const int n3p = (n3 + kGrp - 1) / kGrp * kGrp;
  const int Kc = n1p + n2p + n3p;
  for (int t = tid; t < Kc + nd; t += kPlanThr) b.row_of_slot[t] = -1;
  __syncthreads();
  {
    int o1 = e1, o2 = n1p + e2, o3 = n1p + n2p + e3;
    for (int k = k0; k < k1; ++k) {
      const int ty = b.kType[k];
      const int sl = ty == 1 ? o1++ : (ty == 2 ? o2++ : o3++);
      b.kSlot[k] = sl;
      b.slot_of_row[b.kSrc[k]] = sl;
      b.row_of_slot[sl] = b.kSrc[k];
      b.kW[k] = rho2 * b.kZ[k] * b.kZ[k];
    }
  }
  for (int r = tid; r < nd; r += kPlanThr) {
    b.slot_of_row[b.dSrc[r]] = Kc + r;
    b.row_of_slot[Kc + r] = b.dSrc[r];
  }
  __syncthreads();
  for (int r = tid; r < nr; r += kPlanThr) {  // rotations on gathered slots
    b.rP[r] = b.slot_of_row[b.rP[r]];
    b.rQ[r] = b.slot_of_row[b.rQ[r]];
  }
  if (tid == 0) {
    b.info[kiK] = K;
    b.info[kiN1] = grp[0];
    b.info[kiN2] = grp[1];
    b.info[kiN3] = grp[2];
    b.info[kiN1p] = n1p;
    b.info[kiN2p] = n2p;
    b.info[kiN3p] = n3p;
    b.info[kiKc] = Kc;
    b.info[kiNd] = nd;
    b.info[kiNr] = nr;
    b.info[kiKr] = (K + 127) / 128 * 128;
    b.misc[0] = rho2;
  }
}

// Bbuf row t (pitch mp) = the merge row in slot t, zero outside its half; padding slots zero.
template <typename T>
__global__ __launch_bounds__(kDcThr) void dc_gather_kernel(int64_t n, int64_t s, int m, int h, const T* __restrict__ Z,
                                                           const int* __restrict__ row_of_slot, int64_t mp,
                                                           T* __restrict__ Bbuf) {
  const int t = blockIdx.x;
  const int row = row_of_slot[t];
  T* dst = Bbuf + (int64_t)t * mp;
  if (row < 0) {
    for (int c = threadIdx.x; c < m; c += kDcThr) dst[c] = T(0);
    return;
  }
  const T* src = Z + (s + row) * n + s;
  const bool top = row < h;
  for (int c = threadIdx.x; c < m; c += kDcThr) dst[c] = (top == (c < h)) ? src[c] : T(0);
}

// The deflation rotations in scan order on the gathered slots, one column per thread.  A rotation
// usually continues the previous one's second row, which is then taken from a register.
template <typename T>
__global__ __launch_bounds__(kDcThr) void dc_rotate_kernel(int m, int64_t mp, const int* __restrict__ info,
                                                           const int* __restrict__ rP, const int* __restrict__ rQ,
                                                           const double* __restrict__ rC, const double* __restrict__ rS,
                                                           T* __restrict__ Bbuf) {
  const int c = blockIdx.x * kDcThr + threadIdx.x;
  if (c >= m) return;
  const int nr = info[kiNr];
  int last = -1;
  double lastv = 0.0;
  // Rotation r's second row q is untouched by rotations < r, and its first row p is either the
  // previous rotation's q (kept in a register) or untouched: the values of eight rotations can be
  // loaded before any of them is applied.
  for (int r0 = 0; r0 < nr; r0 += 8) {
    int pv[8], qv[8];
    double av[8], bv[8], cv[8], sv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r = min(r0 + k, nr - 1);
      pv[k] = rP[r];
      qv[k] = rQ[r];
      cv[k] = rC[r];
      sv[k] = rS[r];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      av[k] = (double)Bbuf[(int64_t)pv[k] * mp + c];
      bv[k] = (double)Bbuf[(int64_t)qv[k] * mp + c];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (r0 + k >= nr) break;
      const double a = pv[k] == last ? lastv : av[k];
      const double na = cv[k] * a + sv[k] * bv[k], nb = -sv[k] * a + cv[k] * bv[k];
      Bbuf[(int64_t)pv[k] * mp + c] = (T)na;
      Bbuf[(int64_t)qv[k] * mp + c] = (T)nb;
      last = qv[k];
      lastv = (double)(T)nb;
    }
  }
}

// One wave per root.
__global__ __launch_bounds__(kDcThr) void dc_secular_kernel(const int* __restrict__ info, const double* __restrict__ kD,
                                                            const double* __restrict__ kW, int* __restrict__ rO,
                                                            double* __restrict__ rT, double* __restrict__ lamK) {
  const int K = info[kiK];
  const int j = blockIdx.x * (kDcThr / 64) + (threadIdx.x >> 6);
  if (j >= K) return;  // uniform over the wave
  int o;
  double tau;
  secular_root_wave(kD, kW, K, j, &o, &tau);
  if ((threadIdx.x & 63) == 0) {
    rO[j] = o;
    rT[j] = tau;
    lamK[j] = kD[o] + tau;
  }
}

__global__ __launch_bounds__(kDcThr) void dc_loewner_kernel(const int* __restrict__ info, const double* __restrict__ misc,
                                                            const double* __restrict__ kD, const double* __restrict__ kZ,
                                                            const int* __restrict__ rO, const double* __restrict__ rT,
                                                            double* __restrict__ zh) {
  const int K = info[kiK];
  const int i = blockIdx.x * (kDcThr / 64) + (threadIdx.x >> 6);
  if (i >= K) return;  // uniform over the wave
  const double v = loewner_wave(kD, rO, rT, misc[0], K, i, kZ[i]);
  if ((threadIdx.x & 63) == 0) zh[i] = v;
}

// Ut row j (pitch Kc) = normalised (zhat_k / (d_k - lambda_j)) in the kept rows' slots; padding
// columns and rows j >= K are zero.
template <typename T>
__global__ __launch_bounds__(kDcThr) void dc_ut_kernel(const int* __restrict__ info, const double* __restrict__ kD,
                                                       const double* __restrict__ zh, const int* __restrict__ rO,
                                                       const double* __restrict__ rT, const int* __restrict__ kSlot,
                                                       T* __restrict__ Ut) {
  __shared__ double red[kDcThr / 64];
  const int K = info[kiK], Kc = info[kiKc];
  const int j = blockIdx.x;
  T* row = Ut + (int64_t)j * Kc;
  if (j >= K) {
    for (int c = threadIdx.x; c < Kc; c += kDcThr) row[c] = T(0);
    return;
  }
  const int n1 = info[kiN1], n2 = info[kiN2], n3 = info[kiN3];
  const int n1p = info[kiN1p], n2p = info[kiN2p];
  for (int c = threadIdx.x; c < Kc; c += kDcThr) {
    const bool pad = (c >= n1 && c < n1p) || (c >= n1p + n2 && c < n1p + n2p) || c >= n1p + n2p + n3;
    if (pad) row[c] = T(0);
  }
  const double dor = kD[rO[j]], tau = rT[j];
  double ss = 0.0;
  for (int k = threadIdx.x; k < K; k += kDcThr) {
    const double v = zh[k] / ((kD[k] - dor) - tau);
    ss += v * v;
  }
  ss = block_sum_f64(ss, red);
  const double inv = 1.0 / sqrt(ss);
  for (int k = threadIdx.x; k < K; k += kDcThr) row[kSlot[k]] = (T)(zh[k] / ((kD[k] - dor) - tau) * inv);
}

// Merged order and write-back: output row t < K is root t (from Cbuf), t >= K the deflated row
// t - K (from Bbuf slot Kc + t - K).
template <typename T>
__global__ __launch_bounds__(kDcThr) void dc_scatter_kernel(int64_t n, int64_t s, int m, int64_t mp,
                                                            const int* __restrict__ info,
                                                            const double* __restrict__ lamK,
                                                            const double* __restrict__ dV, const T* __restrict__ Cbuf,
                                                            const T* __restrict__ Bbuf, double* __restrict__ lam,
                                                            T* __restrict__ Z) {
  __shared__ int ired[kDcThr / 64];
  const int K = info[kiK], nd = info[kiNd], Kc = info[kiKc];
  const int t = blockIdx.x;
  if (t >= K + nd) return;  // uniform
  double val;
  int cntv = 0;
  const T* src;
  if (t < K) {
    val = lamK[t];
    for (int r = threadIdx.x; r < nd; r += kDcThr) cntv += dV[r] < val;
    cntv = block_sum_i(cntv, ired) + t;
    src = Cbuf + (int64_t)t * mp;
  } else {
    const int r = t - K;
    val = dV[r];
    for (int q = threadIdx.x; q < nd; q += kDcThr) cntv += (dV[q] < val) || (dV[q] == val && q < r);
    for (int j = threadIdx.x; j < K; j += kDcThr) cntv += lamK[j] <= val;
    cntv = block_sum_i(cntv, ired);
    src = Bbuf + (int64_t)(Kc + r) * mp;
  }
  const int p = cntv;
  if (threadIdx.x == 0) lam[s + p] = val;
  T* dst = Z + (s + p) * n + s;
  for (int c = threadIdx.x; c < m; c += kDcThr) dst[c] = src[c];
}

template <typename T>
__global__ __launch_bounds__(256) void dc_zero_cols_kernel(int64_t rows, int64_t cols, int64_t ld, T* __restrict__ C) {
  const int64_t r = blockIdx.x;
  if (r >= rows) return;
  for (int64_t c = threadIdx.x; c < cols; c += 256) C[r * ld + c] = T(0);
}

// ---- host ----------------------------------------------------------------------------------------

struct Node {
  int s, m, h;
};

int split_of(int m) {
  if (m > kSmallMax) {
    const int h = (m + 1) / 2 + 63;
    const int hr = h / 64 * 64;
    return hr < m ? hr : m / 2;
  }
  return m / 2;
}

void build_tree(int s, int m, int depth, std::vector<std::vector<Node>>& lv) {
  if (m <= 1) return;
  const int h = split_of(m);
  if ((int)lv.size() <= depth) lv.resize(depth + 1);
  lv[depth].push_back({s, m, h});
  build_tree(s, h, depth + 1, lv);
  build_tree(s + h, m - h, depth + 1, lv);
}

struct DcLayout {
  int64_t lam, nodes, Ds, Zs, kD, kZ, kW, dV, rC, rS, rT, lamK, zh, misc;
  int64_t Ss, kSrc, kType, kSlot, dSrc, rP, rQ, slot_of_row, row_of_slot, rO, info;
  int64_t Lt, stat, modT, cK, cS0, cS1, modD, modZ, cD0, cZ0, cD1, cZ1;
  int64_t S, Ut, Cb, cnt, total;
};

DcLayout dc_layout(int64_t n, int es) {
  DcLayout L{};
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += rup(std::max<int64_t>(bytes, 1), 256);
    return at;
  };
  L.lam = take(n * 8);
  L.nodes = take((3 * n + 64) * 4);
  for (int64_t* f : {&L.Ds, &L.Zs, &L.kD, &L.kZ, &L.kW, &L.dV, &L.rC, &L.rS, &L.rT, &L.lamK, &L.zh}) *f = take(n * 8);
  for (int64_t* f : {&L.Ss, &L.kSrc, &L.kType, &L.kSlot, &L.dSrc, &L.rP, &L.rQ, &L.slot_of_row, &L.rO}) *f = take(n * 4);
  for (int64_t* f : {&L.Lt, &L.stat, &L.modT, &L.cK, &L.cS0, &L.cS1}) *f = take(n * 4);
  for (int64_t* f : {&L.cD0, &L.cZ0, &L.cD1, &L.cZ1}) *f = take(n * 8);
  for (int64_t* f : {&L.modD, &L.modZ}) *f = take(2 * n * 8);
  L.row_of_slot = take((n + 4 * kGrp) * 4);
  L.info = take(64 * 4);
  L.misc = take((kMiscMax + n / kDcThr + 8) * 8);
  L.cnt = take(3 * n * 4);
  const int64_t mp = rup(n, 4);
  const int64_t rows_b = n + 3 * kGrp;  // Kc + nd <= n + 3 (kGrp - 1)
  L.S = take(std::max(n * kSmallMax, rows_b * mp) * es);
  L.Ut = take((n > kSmallMax ? (rup(n, 128) * (n + 3 * kGrp)) : 1) * es);
  L.Cb = take((n > kSmallMax ? (rup(n, 128) * mp) : 1) * es);
  L.total = o;
  return L;
}

// Pinned staging of the node lists (grown as needed; every caller synchronises its stream before
// returning, so no copy from it is pending when it is reused; freed by
// mpq_release_thread_resources).
int* host_nodes_buf(size_t count) {
  static thread_local int* p = nullptr;
  static thread_local size_t cap = 0;
  if (count > cap) {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    cap = 0;
    if (hipHostMalloc((void**)&p, count * sizeof(int), hipHostMallocDefault) != hipSuccess) return nullptr;
    cap = count;
    track_pinned(reinterpret_cast<void**>(&p), nullptr, &cap);
  }
  return p;
}

int* host_info_buf() {
  static thread_local int* p = nullptr;
  if (!p) {
    if (hipHostMalloc((void**)&p, 64 * sizeof(int), hipHostMallocDefault) != hipSuccess) p = nullptr;
    else track_pinned(reinterpret_cast<void**>(&p), nullptr, nullptr);
  }
  return p;
}

int large_gemm(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, int64_t M, int64_t N,
               int64_t K, hipStream_t stream) {
  MPQ_HIP_TRY(gemm(A, lda, B, ldb, false, nullptr, C, ldc, M, N, K, 1.f, 0.f, nullptr, 0, stream));
  return kOk;
}

int large_gemm(const double* A, int64_t lda, const double* B, int64_t ldb, double* C, int64_t ldc, int64_t M,
               int64_t N, int64_t K, hipStream_t stream) {
  MPQ_HIP_TRY(gemm_f64(A, lda, B, ldb, false, C, ldc, M, N, K, 1.0, 0.0, nullptr, 0, stream));
  return kOk;
}

// All small merges of one size class of one tree level: set-up, gather, rotations, product.
template <typename T, int MAXM>
int small_level(int64_t n, const int* nl, int count, const T* e, double* lam, T* Z, T* S, double u, SmallOut so,
                hipStream_t stream) {
  hipLaunchKernelGGL((dc_small_merge_kernel<T, MAXM>), dim3(count), dim3(kDcThr), 0, stream, n, nl, e, lam, Z, u, so);
  const dim3 g4(count, (MAXM + 3) / 4);
  hipLaunchKernelGGL((dc_small_secular_kernel<MAXM>), g4, dim3(kDcThr), 0, stream, nl, so);
  hipLaunchKernelGGL((dc_small_loewner_kernel<T, MAXM>), g4, dim3(kDcThr), 0, stream, nl, e, so);
  hipLaunchKernelGGL((dc_small_order_kernel<MAXM>), g4, dim3(kDcThr), 0, stream, nl, lam, so);
  hipLaunchKernelGGL((dc_small_gather_kernel<T, MAXM>), dim3(count, (MAXM + 3) / 4), dim3(kDcThr), 0, stream, n, nl, Z,
                     so, S);
  hipLaunchKernelGGL((dc_small_rotate_kernel<T, MAXM>), dim3(count, (MAXM + kDcThr - 1) / kDcThr), dim3(kDcThr), 0,
                     stream, nl, so, S);
  hipLaunchKernelGGL((dc_small_product_kernel<T, MAXM>), dim3(count, (MAXM + kSpCols - 1) / kSpCols,
                                                              (MAXM + kSpRows - 1) / kSpRows),
                     dim3(kDcThr), 0, stream, n, nl, S, so, Z);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

template <typename T>
int tridiag_dc_impl(int64_t n, const T* d, const T* e, T* lam_out, T* Z, void* ws, int64_t ws_bytes,
                    hipStream_t stream) {
  MPQ_CHECK_ARG(n >= 1 && n <= (int64_t)1 << 30, "tridiagonal divide and conquer: bad order %lld", (long long)n);
  const DcLayout L = dc_layout(n, (int)sizeof(T));
  MPQ_CHECK_ARG(ws_bytes >= L.total, "tridiagonal divide and conquer: workspace too small");
  char* base = static_cast<char*>(ws);
  double* lam = reinterpret_cast<double*>(base + L.lam);
  int* nodes_d = reinterpret_cast<int*>(base + L.nodes);
  T* S = reinterpret_cast<T*>(base + L.S);
  T* Ut = reinterpret_cast<T*>(base + L.Ut);
  T* Cb = reinterpret_cast<T*>(base + L.Cb);
  LargeBufs b{};
  b.Ds = reinterpret_cast<double*>(base + L.Ds);
  b.Zs = reinterpret_cast<double*>(base + L.Zs);
  b.kD = reinterpret_cast<double*>(base + L.kD);
  b.kZ = reinterpret_cast<double*>(base + L.kZ);
  b.kW = reinterpret_cast<double*>(base + L.kW);
  b.dV = reinterpret_cast<double*>(base + L.dV);
  b.rC = reinterpret_cast<double*>(base + L.rC);
  b.rS = reinterpret_cast<double*>(base + L.rS);
  b.rT = reinterpret_cast<double*>(base + L.rT);
  b.lamK = reinterpret_cast<double*>(base + L.lamK);
  b.zh = reinterpret_cast<double*>(base + L.zh);
  b.Ss = reinterpret_cast<int*>(base + L.Ss);
  b.kSrc = reinterpret_cast<int*>(base + L.kSrc);
  b.kType = reinterpret_cast<int*>(base + L.kType);
  b.kSlot = reinterpret_cast<int*>(base + L.kSlot);
  b.dSrc = reinterpret_cast<int*>(base + L.dSrc);
  b.rP = reinterpret_cast<int*>(base + L.rP);
  b.rQ = reinterpret_cast<int*>(base + L.rQ);
  b.slot_of_row = reinterpret_cast<int*>(base + L.slot_of_row);
  b.row_of_slot = reinterpret_cast<int*>(base + L.row_of_slot);
  b.rO = reinterpret_cast<int*>(base + L.rO);
  b.info = reinterpret_cast<int*>(base + L.info);
  b.misc = reinterpret_cast<double*>(base + L.misc);
  b.Lt = reinterpret_cast<int*>(base + L.Lt);
  b.stat = reinterpret_cast<int*>(base + L.stat);
  b.modT = reinterpret_cast<int*>(base + L.modT);
  b.cK = reinterpret_cast<int*>(base + L.cK);
  b.cS0 = reinterpret_cast<int*>(base + L.cS0);
  b.cS1 = reinterpret_cast<int*>(base + L.cS1);
  b.modD = reinterpret_cast<double*>(base + L.modD);
  b.modZ = reinterpret_cast<double*>(base + L.modZ);
  b.cD0 = reinterpret_cast<double*>(base + L.cD0);
  b.cZ0 = reinterpret_cast<double*>(base + L.cZ0);
  b.cD1 = reinterpret_cast<double*>(base + L.cD1);
  b.cZ1 = reinterpret_cast<double*>(base + L.cZ1);
  SmallOut so{};  // shares the large-merge arrays: a level's small merges finish before its large ones
  so.kD = b.kD;
  so.rT = b.rT;
  so.zh = b.zh;
  so.inrm = b.lamK;
  so.rO = b.rO;
  so.kZ = b.kZ;
  so.kW = b.kW;
  so.dV = b.dV;
  so.pos = b.kSlot;
  so.slot = b.slot_of_row;
  so.rP = b.rP;
  so.rQ = b.rQ;
  so.rC = b.rC;
  so.rS = b.rS;
  so.cnt = reinterpret_cast<int*>(base + L.cnt);
  const double u = UnitRoundoff<T>::value;
  const unsigned g256 = (unsigned)((n + 255) / 256);

  hipLaunchKernelGGL(dc_init_kernel<T>, dim3(g256), dim3(256), 0, stream, n, d, e, lam, Z);
  MPQ_LAUNCH_CHECK();
  if (n > 1) {
    std::vector<std::vector<Node>> lv;
    build_tree(0, (int)n, 0, lv);
    // device node lists: per level, the small merges by size class (<= 32, <= 128, <= 512)
    std::vector<int> flat;
    struct Launch {
      int cls, offset, count;
    };
    std::vector<std::vector<Launch>> launches(lv.size());
    for (size_t dpt = 0; dpt < lv.size(); ++dpt) {
      for (int cls = 0; cls < 3; ++cls) {
        const int lim = cls == 0 ? 32 : (cls == 1 ? 128 : kSmallMax);
        const int lo = cls == 0 ? 0 : (cls == 1 ? 32 : 128);
        const int off = (int)flat.size() / 3;
        int count = 0;
        for (const Node& nd : lv[dpt]) {
          if (nd.m > lo && nd.m <= lim) {
            flat.push_back(nd.s);
            flat.push_back(nd.m);
            flat.push_back(nd.h);
            ++count;
          }
        }
        if (count) launches[dpt].push_back({cls, off, count});
      }
    }
    MPQ_CHECK_ARG((int64_t)flat.size() <= 3 * n + 64, "tridiagonal divide and conquer: node list overflow");
    if (!flat.empty()) {
      int* staged = host_nodes_buf(flat.size());
      MPQ_CHECK_ARG(staged != nullptr, "tridiagonal divide and conquer: pinned host buffer unavailable");
      std::copy(flat.begin(), flat.end(), staged);
      MPQ_HIP_TRY(hipMemcpyAsync(nodes_d, staged, flat.size() * sizeof(int), hipMemcpyHostToDevice, stream));
    }
    int* hinfo = host_info_buf();
    MPQ_CHECK_ARG(hinfo != nullptr, "tridiagonal divide and conquer: pinned host buffer unavailable");
    for (int dpt = (int)lv.size() - 1; dpt >= 0; --dpt) {
      for (const Launch& la : launches[dpt]) {
        const int* nl = nodes_d + 3 * la.offset;
        int rc;
        if (la.cls == 0) rc = small_level<T, 32>(n, nl, la.count, e, lam, Z, S, u, so, stream);
        else if (la.cls == 1) rc = small_level<T, 128>(n, nl, la.count, e, lam, Z, S, u, so, stream);
        else rc = small_level<T, kSmallMax>(n, nl, la.count, e, lam, Z, S, u, so, stream);
        if (rc != kOk) return rc;
      }
      for (const Node& nd : lv[dpt]) {
        if (nd.m <= kSmallMax) continue;
        const int64_t s = nd.s;
        const int m = nd.m, hh = nd.h;
        const int64_t mp = rup(m, 4);
        hipLaunchKernelGGL(dc_sort_kernel<T>, dim3((unsigned)((m + kDcThr - 1) / kDcThr)), dim3(kDcThr), 0, stream, n,
                           s, m, hh, e, lam, Z, b);
        hipLaunchKernelGGL(dc_plan_kernel<T>, dim3(1), dim3(kPlanThr), 0, stream, s, m, hh, e, u, b);
        MPQ_LAUNCH_CHECK();
        MPQ_HIP_TRY(hipMemcpyAsync(hinfo, b.info, kiCount * sizeof(int), hipMemcpyDeviceToHost, stream));
        MPQ_HIP_TRY(hipStreamSynchronize(stream));
        const int K = hinfo[kiK], n1p = hinfo[kiN1p], n2p = hinfo[kiN2p], n3p = hinfo[kiN3p];
        const int Kc = hinfo[kiKc], nd_ = hinfo[kiNd], Kr = hinfo[kiKr];
        MPQ_CHECK_ARG(K + nd_ == m && Kc + nd_ <= n + 3 * kGrp, "tridiagonal divide and conquer: inconsistent merge");
        T* Bbuf = S;
        hipLaunchKernelGGL(dc_gather_kernel<T>, dim3((unsigned)(Kc + nd_)), dim3(kDcThr), 0, stream, n, s, m, hh, Z,
                           b.row_of_slot, mp, Bbuf);
        MPQ_LAUNCH_CHECK();
        if (hinfo[kiNr] > 0) {
          hipLaunchKernelGGL(dc_rotate_kernel<T>, dim3((unsigned)((m + kDcThr - 1) / kDcThr)), dim3(kDcThr), 0, stream,
                             m, mp, b.info, b.rP, b.rQ, b.rC, b.rS, Bbuf);
          MPQ_LAUNCH_CHECK();
        }
        if (K > 0) {
          const unsigned gk = (unsigned)((K + kDcThr / 64 - 1) / (kDcThr / 64));
          hipLaunchKernelGGL(dc_secular_kernel, dim3(gk), dim3(kDcThr), 0, stream, b.info, b.kD, b.kW, b.rO, b.rT,
                             b.lamK);
          MPQ_LAUNCH_CHECK();
          hipLaunchKernelGGL(dc_loewner_kernel, dim3(gk), dim3(kDcThr), 0, stream, b.info, b.misc, b.kD, b.kZ,
                             b.rO, b.rT, b.zh);
          MPQ_LAUNCH_CHECK();
          hipLaunchKernelGGL(dc_ut_kernel<T>, dim3((unsigned)Kr), dim3(kDcThr), 0, stream, b.info, b.kD, b.zh, b.rO,
                             b.rT, b.kSlot, Ut);
          MPQ_LAUNCH_CHECK();
          int rc;
          // first half of the columns: groups 1 and 2; second half: groups 2 and 3
          if (n1p + n2p > 0) {
            if ((rc = large_gemm(Ut, Kc, Bbuf, mp, Cb, mp, Kr, hh, n1p + n2p, stream)) != kOk) return rc;
          } else {
            hipLaunchKernelGGL(dc_zero_cols_kernel<T>, dim3((unsigned)Kr), dim3(256), 0, stream, (int64_t)Kr,
                               (int64_t)hh, mp, Cb);
            MPQ_LAUNCH_CHECK();
          }
          if (n2p + n3p > 0) {
            if ((rc = large_gemm(Ut + n1p, Kc, Bbuf + (int64_t)n1p * mp + hh, mp, Cb + hh, mp, Kr, m - hh,
                                 n2p + n3p, stream)) != kOk)
              return rc;
          } else {
            hipLaunchKernelGGL(dc_zero_cols_kernel<T>, dim3((unsigned)Kr), dim3(256), 0, stream, (int64_t)Kr,
                               (int64_t)(m - hh), mp, Cb + hh);
            MPQ_LAUNCH_CHECK();
          }
        }
        hipLaunchKernelGGL(dc_scatter_kernel<T>, dim3((unsigned)m), dim3(kDcThr), 0, stream, n, s, m, mp, b.info,
                           b.lamK, b.dV, Cb, Bbuf, lam, Z);
        MPQ_LAUNCH_CHECK();
      }
    }
  }
  hipLaunchKernelGGL(dc_out_kernel<T>, dim3(g256), dim3(256), 0, stream, n, lam, lam_out);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

}  // namespace

int64_t tridiag_dc_workspace_bytes(int64_t n, int elem_size) {
  if (n <= 0) return 0;
  return dc_layout(n, elem_size).total;
}

int tridiag_dc(int64_t n, const float* d, const float* e, float* lam, float* Z, void* ws, int64_t ws_bytes,
               hipStream_t stream) {
  return tridiag_dc_impl<float>(n, d, e, lam, Z, ws, ws_bytes, stream);
}

int tridiag_dc(int64_t n, const double* d, const double* e, double* lam, double* Z, void* ws, int64_t ws_bytes,
               hipStream_t stream) {
  return tridiag_dc_impl<double>(n, d, e, lam, Z, ws, ws_bytes, stream);
}

}  // namespace mpq
