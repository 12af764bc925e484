// Greedy scalar coordinate-descent polish of uniform-grid codes (gfx950).
//
// Replaces mpq/polish/triton_scalar_cd.py:164-307 (uniform_scalar_diag_greedy_cd
// with the persistent sweep kernel :28-110) as dispatched from
// mpq/solver.py:299-333, plus the selection of mpq/solver.py:749-754.
//
// Semantics per row block (block_rows rows sharing one greedy order):
//   residual_u = Yu - x Vs, rhs = residual_u Vs^T, diag_j = |Vs_j|^2 (>= 1e-12)
//   per sweep: gain_j = mean_rows(rhs_j^2 / diag_j), order = stable argsort(-gain)
//   per column (in order): target = x + rhs/diag (the sweep kernel's rule; mpq_uniform_cd_sweeps_recip
//     takes the torch loop's x + rhs * (1/diag), :266), q = clamp(rint(target/s + z)),
//     accept iff res + d^2 diag - 2 rhs d + 1e-12 < res (1 + tol),
//     rhs -= d * H[col, :]
// Blocking: columns are taken in windows of 128 consecutive positions of the
// greedy order.  Inside a window one wave64 per row runs the 128 sequential
// decisions with the window's H sub-block in LDS (rank-1 updates of the window's
// own rhs entries in registers); after the window the deferred update of every
// column, rhs[r, j] -= delta[r, p] * H[order[p], j] for p = 0 .. 127 in window
// order, runs on the VALU as a sequential multiply-then-subtract chain per
// entry (schur_valu_kernel), which is exactly the per-column update order and
// rounding of the reference's sweep (its torch twin,
// mpq/polish/triton_scalar_cd.py:258-288; that loop forms the target with the reciprocal of diag,
// which the _recip entry point reproduces).  Steps whose delta is zero for
// every row of a 16-row tile are skipped (subtracting 0 * h leaves rhs as is).
// The greedy gain is summed over the block's rows in row order.  From the same
// rhs, x, codes and residual norms, a sweep here is bit-identical to the
// column-at-a-time restatement (mpq_uniform_cd_sweeps).
#include <algorithm>
#include <mutex>

#include "cd_common.h"
#include "mpq_amd.h"
#include "gemm.h"
#include "kernels.h"

namespace mpq {
namespace {

constexpr int kWin = 128;
constexpr int kRowsPerWG = 8;  // one wave64 per row

__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// gain[blk][j] = sum_{rows of blk} rhs^2 * diag_inv / rows_in_blk
__global__ __launch_bounds__(256) void gain_kernel(int64_t rows, int64_t n, int64_t block_rows,
                                                   const float* __restrict__ rhs,
                                                   const float* __restrict__ diag_inv,
                                                   float* __restrict__ gain) {
  const int64_t blk = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t r0 = blk * block_rows;
  int64_t r1 = r0 + block_rows;
  if (r1 > rows) r1 = rows;
  const float di = diag_inv[j];
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float v = rhs[r * n + j];
    acc += (v * v) * di;
  }
  gain[blk * n + j] = acc / (float)(r1 - r0);
}

// T[blk][p][q] = H[order[blk][w0 + p]][order[blk][w0 + q]] for the window (zero-padded).
__global__ __launch_bounds__(kWin) void tile_gather_kernel(int64_t n, const float* __restrict__ H,
                                                           const int32_t* __restrict__ order,
                                                           int64_t w0, int wn,
                                                           float* __restrict__ T) {
  const int64_t blk = blockIdx.y;
  const int p = blockIdx.x;
  const int q = threadIdx.x;
  const int32_t* ord = order + blk * n + w0;
  float v = 0.f;
  if (p < wn && q < wn) v = H[(int64_t)ord[p] * n + ord[q]];
  T[(blk * kWin + p) * kWin + q] = v;
}

// One window of greedy decisions; one wave per row, lane l owns positions l and l+64.
__global__ __launch_bounds__(64 * kRowsPerWG) void window_kernel(
    int64_t rows, int64_t n, int64_t block_rows, int maxq, float accept_tol,
    const int32_t* __restrict__ order, int64_t w0, int wn, const float* __restrict__ T,
    const float* __restrict__ scale, const float* __restrict__ zero, int64_t G, int64_t gs,
    const float* __restrict__ diag, const float* __restrict__ diag_inv, int recip, float* __restrict__ rhs,
    float* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ res_norm, float* __restrict__ delta,
    int* __restrict__ accepted) {
  __shared__ float Ts[kWin * kWin];
  // each wave's per-position constants (x at the window's start, scale, zero, diag), read by the
  // decision of position p with a wave-uniform LDS address: they do not depend on the decisions
  // before p, so their reads issue ahead of the sequential chain (a lane broadcast could not)
  __shared__ float Pc[kRowsPerWG][4][kWin];
  const int64_t blk = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float* Tb = T + blk * kWin * kWin;
  for (int i = threadIdx.x; i < kWin * kWin; i += blockDim.x) Ts[i] = Tb[i];
  const int64_t row = blk * block_rows + (int64_t)blockIdx.x * kRowsPerWG + wave;
  int64_t blk_end = (blk + 1) * block_rows;
  if (blk_end > rows) blk_end = rows;
  if (row >= blk_end) {
    __syncthreads();  // the tile load's barrier (every wave reaches it)
    return;
  }

  const int32_t* ord = order + blk * n + w0;
  const bool v0 = lane < wn, v1 = lane + 64 < wn;
  const int64_t c0 = v0 ? ord[lane] : 0;
  const int64_t c1 = v1 ? ord[lane + 64] : 0;
  const int64_t o0 = row * n + c0, o1 = row * n + c1;
  float rhs0 = v0 ? rhs[o0] : 0.f, rhs1 = v1 ? rhs[o1] : 0.f;
  float x0 = v0 ? x[o0] : 0.f, x1 = v1 ? x[o1] : 0.f;
  float s0 = v0 ? scale[row * G + c0 / gs] : 1.f, s1 = v1 ? scale[row * G + c1 / gs] : 1.f;
  s0 = s0 < 1e-12f ? 1e-12f : s0;
  s1 = s1 < 1e-12f ? 1e-12f : s1;
  const float z0 = v0 ? zero[row * G + c0 / gs] : 0.f, z1 = v1 ? zero[row * G + c1 / gs] : 0.f;
  const float dg0 = v0 ? diag[c0] : 1.f, dg1 = v1 ? diag[c1] : 1.f;
  const float di0 = v0 ? diag_inv[c0] : 1.f, di1 = v1 ? diag_inv[c1] : 1.f;
  int q0 = -1, q1 = -1;
  float d0 = 0.f, d1 = 0.f;
  float res = res_norm[row];
  int acc_count = 0;
  const float one_tol = 1.0f + accept_tol;
  float (*pc)[kWin] = Pc[wave];
  pc[0][lane] = x0;
  pc[0][lane + 64] = x1;
  pc[1][lane] = s0;
  pc[1][lane + 64] = s1;
  pc[2][lane] = z0;
  pc[2][lane + 64] = z1;
  pc[3][lane] = dg0;
  pc[3][lane + 64] = dg1;
  __syncthreads();  // the tile and the constants

  for (int p = 0; p < wn; ++p) {
    const int src = p & 63;
    const bool hi = p >= 64;
    const float rp = bcast(hi ? rhs1 : rhs0, src);
    const float xp = pc[0][p];
    const float sp = pc[1][p];
    const float zp = pc[2][p];
    const float dp = pc[3][p];
    // the sweep kernel's rule x + rhs / diag, or the torch loop's x + rhs * (1 / diag)
    const float target = recip ? xp + rp * bcast(hi ? di1 : di0, src) : xp + rp / dp;
    float qf = rintf(target / sp + zp);
    qf = fmaxf(fminf(qf, (float)maxq), 0.f);
    const float xq = sp * (qf - zp);
    const float dlt = xq - xp;
    float cand = res + (dlt * dlt) * dp - (2.0f * rp) * dlt;
    cand = cand < 0.f ? 0.f : cand;
    if (cand + 1e-12f < res * one_tol) {
      res = cand;
      ++acc_count;
      if (lane == src) {
        if (hi) { x1 = xq; q1 = (int)qf; d1 = dlt; }
        else { x0 = xq; q0 = (int)qf; d0 = dlt; }
      }
      const float* trow = Ts + p * kWin;
      rhs0 = rhs0 - dlt * trow[lane];
      rhs1 = rhs1 - dlt * trow[lane + 64];
    }
  }
  if (v0) {
    x[o0] = x0;
    if (q0 >= 0) q[o0] = (uint8_t)q0;
  }
  if (v1) {
    x[o1] = x1;
    if (q1 >= 0) q[o1] = (uint8_t)q1;
  }
  delta[row * kWin + lane] = v0 ? d0 : 0.f;
  delta[row * kWin + 64 + lane] = v1 ? d1 : 0.f;
  if (lane == 0) {
    res_norm[row] = res;
    accepted[row] += acc_count;
  }
}

__global__ void recip_kernel(int64_t n, const float* __restrict__ a, float* __restrict__ out) {
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n;
       j += (int64_t)gridDim.x * blockDim.x)
    out[j] = 1.0f / a[j];
}

constexpr int kSRows = 16;    // rows per work-group of the deferred update
constexpr int kSCols = 1024;  // columns per work-group (4 waves x 64 lanes x 4 columns)

// Deferred update after a window: rhs[r, j] -= delta[r, p] * H[order[p], j], p = 0 .. wn-1 in order,
// one rounding for the product and one for the difference (as the reference's column-at-a-time
// update).  Work-group = 16 rows of one row block x 1024 columns; lane = 4 consecutive columns.
// Work-groups are numbered so that the tiles sharing one block's window rows of H land on one XCD.
template <bool kVec>
__device__ __forceinline__ void load4(const float* __restrict__ row, int64_t c, int64_t n, float (&v)[4]) {
  if (kVec) {  // n % 4 == 0 and c <= n - 4
    const float4 t = *reinterpret_cast<const float4*>(row + c);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = row[c + i < n ? c + i : n - 1];
  }
}

template <bool kVec>
__global__ __launch_bounds__(256) void schur_valu_kernel(int64_t rows, int64_t n, int64_t block_rows,
                                                         int64_t rtiles, int64_t ctiles,
                                                         const int32_t* __restrict__ order, int64_t w0,
                                                         int wn, const float* __restrict__ delta,
                                                         const float* __restrict__ H,
                                                         float* __restrict__ rhs) {
  __shared__ float dT[(kWin + 1) * kSRows];  // [p][r]; slot kWin is all zero (padding steps)
  __shared__ int plist[kWin + 8];
  __shared__ int64_t hoff[kWin + 8];
  __shared__ unsigned long long masks[2];
  // XCD-aware tile numbering: hardware work-group i runs on XCD i % 8
  const int64_t total = (int64_t)gridDim.x;
  const int64_t per = total / 8;
  const int64_t id = blockIdx.x;
  const int64_t logical = id < per * 8 ? (id % 8) * per + id / 8 : id;
  const int64_t rt = logical % rtiles;
  const int64_t ct = (logical / rtiles) % ctiles;
  const int64_t blk = logical / (rtiles * ctiles);
  const int64_t r0 = blk * block_rows + rt * kSRows;
  int64_t rend = (blk + 1) * block_rows;
  if (rend > rows) rend = rows;
  const int nr = (int)(rend - r0 < kSRows ? rend - r0 : kSRows);
  if (nr <= 0) return;  // uniform over the work-group

  const int t = threadIdx.x;
  for (int e = t; e < (kWin + 1) * kSRows; e += 256) {
    const int r = e % kSRows, p = e / kSRows;
    dT[e] = (r < nr && p < wn) ? delta[(r0 + r) * kWin + p] : 0.f;
  }
  __syncthreads();
  bool active = false;
  if (t < kWin) {
#pragma unroll
    for (int r = 0; r < kSRows; ++r) active |= dT[t * kSRows + r] != 0.f;
  }
  const unsigned long long m = __ballot(active);
  if (t < kWin && (t & 63) == 0) masks[t >> 6] = m;
  __syncthreads();
  const unsigned long long m0 = masks[0], m1 = masks[1];
  const int nact = __popcll(m0) + __popcll(m1);
  if (nact == 0) return;  // uniform
  const int nact4 = (nact + 3) & ~3;
  if (t < kWin && active) {
    const int pos = t < 64 ? __popcll(m0 & ((1ull << t) - 1ull))
                           : __popcll(m0) + __popcll(m1 & ((1ull << (t - 64)) - 1ull));
    plist[pos] = t;
    hoff[pos] = (int64_t)order[blk * n + w0 + t] * n;
  }
  if (t >= nact && t < nact4 + 4) {  // padding steps (and the prefetch past the end): zero deltas, row 0 of H
    plist[t] = kWin;
    hoff[t] = 0;
  }
  __syncthreads();

  const int lane = t & 63, wave = t >> 6;
  const int64_t c0 = ct * kSCols + wave * 256 + lane * 4;
  const bool live = c0 < n;
  const int64_t cl = kVec ? (live ? c0 : n - 4) : (live ? c0 : n - 1);  // in-bounds column for idle lanes
  float a[kSRows][4];
#pragma unroll
  for (int r = 0; r < kSRows; ++r) {
    if (r < nr) {
      load4<kVec>(rhs + (r0 + r) * n, cl, n, a[r]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) a[r][i] = 0.f;
    }
  }
  float hc[4][4], hn[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) load4<kVec>(H + hoff[u], cl, n, hc[u]);
  for (int k = 0; k < nact4; k += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) load4<kVec>(H + hoff[k + 4 + u], cl, n, hn[u]);  // next group (row 0 past the end)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float* dp = dT + plist[k + u] * kSRows;
#pragma unroll
      for (int r = 0; r < kSRows; ++r) {
        const float d = dp[r];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[r][i] = a[r][i] - d * hc[u][i];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int i = 0; i < 4; ++i) hc[u][i] = hn[u][i];
    }
  }
  if (!live) return;
#pragma unroll
  for (int r = 0; r < kSRows; ++r) {
    if (r < nr) {
      float* dst = rhs + (r0 + r) * n + c0;
      if (kVec) {
        *reinterpret_cast<float4*>(dst) = make_float4(a[r][0], a[r][1], a[r][2], a[r][3]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (c0 + i < n) dst[i] = a[r][i];
      }
    }
  }
}

// q_out = improved ? q_pol : q_in; err_out likewise (mpq/solver.py:749-754).
__global__ void select_kernel(int64_t rows, int64_t n, const uint8_t* __restrict__ q_in,
                              const uint8_t* __restrict__ q_pol, const float* __restrict__ err_before,
                              const float* __restrict__ err_after, uint8_t* __restrict__ q_out,
                              float* __restrict__ err_out, int32_t* __restrict__ improved) {
  const int64_t total = rows * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / n;
    const bool imp = err_after[b] + 1e-12f < err_before[b];
    q_out[e] = imp ? q_pol[e] : q_in[e];
    if (e % n == 0) {
      if (err_out) err_out[b] = imp ? err_after[b] : err_before[b];
      if (improved) improved[b] = imp ? 1 : 0;
    }
  }
}

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

// The greedy sweeps on caller state (rhs, x, codes, residual norms, accept counts), per row block:
// gain -> stable descending order -> windows of 128 decisions -> deferred rhs update.
hipError_t run_sweeps(int64_t rows, int64_t n, int maxq, int64_t block_rows, int64_t nblocks, int sweeps,
                      float accept_tol, const float* scale, const float* zero, int64_t G, int64_t gs,
                      const float* diag, const float* diag_inv, const float* H, float* rhs, float* x,
                      uint8_t* qw, float* res_norm, int* acc, float* gain, int32_t* order, float* T,
                      float* delta, hipStream_t stream, int recip = 0) {
  const int64_t rtiles = (block_rows + kSRows - 1) / kSRows;
  const int64_t ctiles = (n + kSCols - 1) / kSCols;
  const int64_t wgs = nblocks * rtiles * ctiles;
  if (wgs > 0x7fffffffLL) return hipErrorInvalidValue;
  for (int sw = 0; sw < sweeps; ++sw) {
    hipLaunchKernelGGL(gain_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)nblocks), dim3(256), 0,
                       stream, rows, n, block_rows, rhs, diag_inv, gain);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = argsort_desc_rows(gain, nblocks, n, order, stream);
    if (e != hipSuccess) return e;
    for (int64_t w0 = 0; w0 < n; w0 += kWin) {
      const int wn = (int)std::min<int64_t>(kWin, n - w0);
      hipLaunchKernelGGL(tile_gather_kernel, dim3(kWin, (unsigned)nblocks), dim3(kWin), 0, stream, n, H,
                         order, w0, wn, T);
      hipLaunchKernelGGL(window_kernel, dim3((unsigned)((block_rows + kRowsPerWG - 1) / kRowsPerWG),
                                             (unsigned)nblocks),
                         dim3(64 * kRowsPerWG), 0, stream, rows, n, block_rows, maxq, accept_tol, order, w0,
                         wn, T, scale, zero, G, gs, diag, diag_inv, recip, rhs, x, qw, res_norm, delta, acc);
      if (n % 4 == 0)
        hipLaunchKernelGGL(schur_valu_kernel<true>, dim3((unsigned)wgs), dim3(256), 0, stream, rows, n, block_rows,
                           rtiles, ctiles, order, w0, wn, delta, H, rhs);
      else
        hipLaunchKernelGGL(schur_valu_kernel<false>, dim3((unsigned)wgs), dim3(256), 0, stream, rows, n,
                           block_rows, rtiles, ctiles, order, w0, wn, delta, H, rhs);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Workspace of mpq_uniform_cd_sweeps: diag_inv, gain, order, window tiles, deltas.
int64_t sweeps_ws_bytes(int64_t rows, int64_t n, int64_t block_rows) {
  const int64_t nblocks = (rows + block_rows - 1) / block_rows;
  return a64(n) * 4 + a64(nblocks * n) * 4 * 2 + a64(nblocks * kWin * kWin) * 4 + a64(rows * kWin) * 4;
}

struct CdPlan {
  int64_t rows, n, nblocks, nchunks;
  int splits, bn;
  int splits_x6;    // split count of the x6 products (0: shape not supported)
  int64_t ap_bytes;  // packed bf16 planes of their left operand
  int64_t bytes;
};

CdPlan cd_plan(int64_t rows, int64_t n, int64_t block_rows) {
  CdPlan c;
  c.rows = rows;
  c.n = n;
  c.nblocks = (rows + block_rows - 1) / block_rows;
  c.nchunks = (n + 1023) / 1024;
  int bn = 128;
  c.splits = choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  c.bn = bn;
  c.splits_x6 = x6_shape_ok(n, n) ? x6_choose_splits(rows, n, n) : 0;
  c.ap_bytes = c.splits_x6 > 0 ? (x6_packed_a_bytes(rows, n) + 255) / 256 * 256 : 0;
  const int64_t mat = a64(rows * n) * 4;
  int64_t b = 0;
  b += 4 * mat;                               // Yu, x, res/rhs-scratch, rhs
  b += (int64_t)std::max(c.splits, c.splits_x6) * mat;  // partials
  b += c.ap_bytes;                            // x6 planes of the left operand
  b += a64(rows * n);                         // q work (u8)
  b += 3 * a64(n) * 4;                        // diag, diag_inv, spare
  b += a64(c.nblocks * n) * 4 * 2;            // gain + order
  b += a64(c.nblocks * kWin * kWin) * 4;      // window tiles
  b += a64(rows * kWin) * 4;                  // delta
  b += 6 * a64(rows) * 4;                     // res_norm, err_before, err_after, accepted, ...
  b += a64(rows * c.nchunks) * 4;             // chunk partials
  c.bytes = b;
  return c;
}

hipError_t product_splits(const float* A, const float* B, bool trans_b, int64_t rows, int64_t n,
                          float* P, int splits, int bn, hipStream_t stream) {
  GemmParams p{};
  p.M = rows; p.N = n; p.K = n;
  p.A = A; p.lda = n; p.B = B; p.ldb = n; p.trans_b = trans_b;
  p.C = P; p.ldc = n; p.split_stride = a64(rows * n);
  p.alpha = 1.f; p.beta = 0.f; p.mode = kGemmPartials;
  return gemm_partials(p, splits, bn, stream);
}

}  // namespace

int64_t uniform_cd_workspace_bytes(int64_t rows, int64_t n, int64_t block_rows) {
  return cd_plan(rows, n, block_rows).bytes;
}

int uniform_cd_polish(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                      float accept_tol, const float* W, int64_t ldw, const float* Yu_in,
                      const uint8_t* q_in, const float* x_in, const float* scale, const float* zero,
                      int64_t gs, const float* Vs,
                      const float* H, int select, uint8_t* q_out, float* err_before_out,
                      float* err_after_out, int32_t* improved, int32_t* accepted_per_row,
                      void* workspace, int64_t workspace_bytes, hipStream_t stream,
                      const float* xprod_in = nullptr, const float* S = nullptr, const float* packed = nullptr) {
  const CdPlan pl = cd_plan(rows, n, block_rows);
  MPQ_CHECK_ARG(workspace_bytes >= pl.bytes, "uniform CD: workspace too small (%lld < %lld bytes)",
                (long long)workspace_bytes, (long long)pl.bytes);
  const int64_t G = (n + gs - 1) / gs;
  const int64_t mat = a64(rows * n) * 4;
  char* p = static_cast<char*>(workspace);
  float* Yu = (float*)p; p += mat;
  float* x = (float*)p; p += mat;
  float* scratch = (float*)p; p += mat;
  float* rhs = (float*)p; p += mat;
  float* P = (float*)p; p += (int64_t)std::max(pl.splits, pl.splits_x6) * mat;
  void* Ap = p; p += pl.ap_bytes;
  // the two full products on the packed rank-space operator (V | V^T | Vs, x6 products) when given
  const bool x6 = packed != nullptr && S != nullptr && pl.splits_x6 > 0;
  uint8_t* qw = (uint8_t*)p; p += a64(rows * n);
  float* diag = (float*)p; p += a64(n) * 4;
  float* diag_inv = (float*)p; p += a64(n) * 4;
  p += a64(n) * 4;
  float* gain = (float*)p; p += a64(pl.nblocks * n) * 4;
  int32_t* order = (int32_t*)p; p += a64(pl.nblocks * n) * 4;
  float* T = (float*)p; p += a64(pl.nblocks * kWin * kWin) * 4;
  float* delta = (float*)p; p += a64(rows * kWin) * 4;
  float* res_norm = (float*)p; p += a64(rows) * 4;
  float* err_b = (float*)p; p += a64(rows) * 4;
  float* err_a = (float*)p; p += a64(rows) * 4;
  int* acc = (int*)p; p += a64(rows) * 4;
  p += 2 * a64(rows) * 4;
  float* part = (float*)p;
  const int nchunks = (int)pl.nchunks;
  const dim3 eg((unsigned)nchunks, (unsigned)rows);
  const int64_t sstride = a64(rows * n);

  // Yu = W Vs (or given)
  if (Yu_in) {
    MPQ_HIP_TRY(hipMemcpyAsync(Yu, Yu_in, rows * n * 4, hipMemcpyDeviceToDevice, stream));
  } else {
    const float* Wc = W;
    if (ldw != n) {
      MPQ_HIP_TRY(hipMemcpy2DAsync(scratch, n * 4, W, ldw * 4, n * 4, rows, hipMemcpyDeviceToDevice, stream));
      Wc = scratch;
    }
    MPQ_HIP_TRY(product_splits(Wc, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
    MPQ_HIP_TRY(splitk_reduce(P, pl.splits, rows, n, Yu, n, 1.f, 0.f, stream));
  }
  // x (given, or from the codes); residual and its norm (= error before the polish)
  if (x_in) {
    MPQ_HIP_TRY(hipMemcpyAsync(x, x_in, rows * n * 4, hipMemcpyDeviceToDevice, stream));
  } else {
    MPQ_HIP_TRY(dequant_groups(q_in, scale, zero, G, gs, rows, n, x, stream));
  }
  MPQ_HIP_TRY(hipMemcpyAsync(qw, q_in, rows * n, hipMemcpyDeviceToDevice, stream));
  if (xprod_in) {  // x Vs from the caller
    hipLaunchKernelGGL(residual_kernel, eg, dim3(256), 0, stream, rows, n, xprod_in, 1, (int64_t)0, Yu, scratch,
                       part, nchunks);
  } else {
    MPQ_HIP_TRY(product_splits(x, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
    hipLaunchKernelGGL(residual_kernel, eg, dim3(256), 0, stream, rows, n, P, pl.splits, sstride, Yu, scratch,
                       part, nchunks);
  }
  hipLaunchKernelGGL(rows_sum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, rows,
                     nchunks, part, err_b);
  MPQ_LAUNCH_CHECK();
  MPQ_HIP_TRY(hipMemcpyAsync(res_norm, err_b, rows * 4, hipMemcpyDeviceToDevice, stream));
  MPQ_HIP_TRY(hipMemsetAsync(acc, 0, rows * 4, stream));
  // rhs = residual Vs^T (x6: (residual diag(S)) V^T, Vs = V diag(S)); diag = |Vs_j|^2
  if (x6) {
    MPQ_HIP_TRY(x6_pack_a(scratch, n, rows, n, Ap, stream, S));
    MPQ_HIP_TRY(x6_gemm_partials(Ap, packed + n * n, rows, n, n, P, n, sstride, pl.splits_x6, stream));
    MPQ_HIP_TRY(splitk_reduce(P, pl.splits_x6, rows, n, rhs, n, 1.f, 0.f, stream));
  } else {
    MPQ_HIP_TRY(product_splits(scratch, Vs, true, rows, n, P, pl.splits, pl.bn, stream));
    MPQ_HIP_TRY(splitk_reduce(P, pl.splits, rows, n, rhs, n, 1.f, 0.f, stream));
  }
  MPQ_HIP_TRY(row_sqnorm(Vs, n, n, 1e-12f, diag, stream));
  hipLaunchKernelGGL(recip_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, n, diag, diag_inv);
  MPQ_LAUNCH_CHECK();

  MPQ_HIP_TRY(run_sweeps(rows, n, maxq, block_rows, pl.nblocks, sweeps, accept_tol, scale, zero, G, gs, diag,
                         diag_inv, H, rhs, x, qw, res_norm, acc, gain, order, T, delta, stream));
  // error after the polish, from the final codes (mpq/solver.py:323-330)
  MPQ_HIP_TRY(dequant_groups(qw, scale, zero, G, gs, rows, n, x, stream));
  if (x6) {
    MPQ_HIP_TRY(x6_pack_a(x, n, rows, n, Ap, stream));
    MPQ_HIP_TRY(x6_gemm_partials(Ap, packed + 2 * n * n, rows, n, n, P, n, sstride, pl.splits_x6, stream));
  } else {
    MPQ_HIP_TRY(product_splits(x, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
  }
  hipLaunchKernelGGL(residual_kernel, eg, dim3(256), 0, stream, rows, n, P, x6 ? pl.splits_x6 : pl.splits, sstride,
                     Yu, (float*)nullptr, part, nchunks);
  hipLaunchKernelGGL(rows_sum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, rows,
                     nchunks, part, err_a);
  MPQ_LAUNCH_CHECK();
  if (err_before_out) MPQ_HIP_TRY(hipMemcpyAsync(err_before_out, err_b, rows * 4, hipMemcpyDeviceToDevice, stream));
  if (err_after_out) MPQ_HIP_TRY(hipMemcpyAsync(err_after_out, err_a, rows * 4, hipMemcpyDeviceToDevice, stream));
  if (select) {
    int64_t blocks = (rows * n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(select_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, rows, n, q_in, qw, err_b,
                       err_a, q_out, (float*)nullptr, improved);
    MPQ_LAUNCH_CHECK();
  } else {
    MPQ_HIP_TRY(hipMemcpyAsync(q_out, qw, rows * n, hipMemcpyDeviceToDevice, stream));
  }
  if (accepted_per_row) {
    MPQ_HIP_TRY(hipMemcpyAsync(accepted_per_row, acc, rows * 4, hipMemcpyDeviceToDevice, stream));
  }
  return kOk;
}

}  // namespace mpq

extern "C" int64_t mpq_uniform_cd_workspace_size(int64_t rows, int64_t n, int64_t block_rows) {
  if (rows <= 0 || n <= 0 || block_rows <= 0) return 0;
  return mpq::uniform_cd_workspace_bytes(rows, n, block_rows);
}

extern "C" int mpq_uniform_cd_polish(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                     float accept_tol, const float* W, int64_t ldw, const float* Yu,
                                     const uint8_t* q_in, const float* x_in, const float* scale,
                                     const float* zero, int64_t group_size,
                                     const float* Vs, const float* H, int select, uint8_t* q_out,
                                     float* err_before, float* err_after, int32_t* improved,
                                     int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                                     hipStream_t stream) {
  return mpq_uniform_cd_polish_ex(rows, n, maxq, block_rows, sweeps, accept_tol, W, ldw, Yu, q_in, x_in, nullptr,
                                  scale, zero, group_size, Vs, nullptr, nullptr, H, select, q_out, err_before,
                                  err_after, improved, accepted_per_row, workspace, workspace_bytes, stream);
}

extern "C" int mpq_uniform_cd_polish_ex(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                        float accept_tol, const float* W, int64_t ldw, const float* Yu,
                                        const uint8_t* q_in, const float* x_in, const float* xprod_in,
                                        const float* scale, const float* zero, int64_t group_size,
                                        const float* Vs, const float* S, const float* packed, const float* H,
                                        int select, uint8_t* q_out,
                                        float* err_before, float* err_after, int32_t* improved,
                                        int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                                        hipStream_t stream) {
  MPQ_CHECK_ARG(rows > 0 && n > 0, "mpq_uniform_cd_polish: empty problem");
  MPQ_CHECK_ARG(maxq >= 1 && maxq <= 255, "mpq_uniform_cd_polish: maxq must be in [1, 255]");
  MPQ_CHECK_ARG(block_rows >= 1 && sweeps >= 0 && group_size >= 1, "mpq_uniform_cd_polish: bad sizes");
  MPQ_CHECK_ARG(n <= 16384, "mpq_uniform_cd_polish: n <= 16384 supported (greedy-order sort in LDS)");
  MPQ_CHECK_ARG(rows <= 65535, "mpq_uniform_cd_polish: at most 65535 rows per call");
  MPQ_CHECK_ARG((W || Yu) && q_in && scale && zero && Vs && H && q_out && workspace,
                "mpq_uniform_cd_polish: null argument");
  MPQ_CHECK_ARG(!W || ldw >= n, "mpq_uniform_cd_polish: ldw < n");
  return mpq::uniform_cd_polish(rows, n, maxq, block_rows, sweeps, accept_tol, W, ldw, Yu, q_in, x_in, scale, zero,
                                group_size, Vs, H, select, q_out, err_before, err_after, improved,
                                accepted_per_row, workspace, workspace_bytes, stream, xprod_in, S, packed);
}

extern "C" int64_t mpq_uniform_cd_sweeps_workspace_size(int64_t rows, int64_t n, int64_t block_rows) {
  if (rows <= 0 || n <= 0 || block_rows <= 0) return 0;
  return mpq::sweeps_ws_bytes(rows, n, block_rows);
}

namespace mpq {
namespace {

int cd_sweeps_entry(const char* fn, int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                    float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm, int32_t* accepted,
                    const float* scale, const float* zero, int64_t group_size, const float* diag, const float* H,
                    void* workspace, int64_t workspace_bytes, hipStream_t stream, int recip = 0) {
  MPQ_CHECK_ARG(rows > 0 && n > 0, "%s: empty problem", fn);
  MPQ_CHECK_ARG(maxq >= 1 && maxq <= 255, "%s: maxq must be in [1, 255]", fn);
  MPQ_CHECK_ARG(block_rows >= 1 && sweeps >= 0 && group_size >= 1, "%s: bad sizes", fn);
  MPQ_CHECK_ARG(n <= 16384, "%s: n <= 16384 supported (greedy-order sort in LDS)", fn);
  MPQ_CHECK_ARG(rows <= 65535 * kRowsPerWG, "%s: too many rows", fn);
  MPQ_CHECK_ARG((rows + block_rows - 1) / block_rows <= 65535, "%s: too many row blocks", fn);
  MPQ_CHECK_ARG(rhs && x && q && res_norm && accepted && scale && zero && diag && H && workspace,
                "%s: null argument", fn);
  const int64_t need = sweeps_ws_bytes(rows, n, block_rows);
  MPQ_CHECK_ARG(workspace_bytes >= need, "%s: workspace too small (%lld < %lld bytes)", fn,
                (long long)workspace_bytes, (long long)need);
  const int64_t nblocks = (rows + block_rows - 1) / block_rows;
  const int64_t G = (n + group_size - 1) / group_size;
  char* p = static_cast<char*>(workspace);
  float* diag_inv = (float*)p; p += a64(n) * 4;
  float* gain = (float*)p; p += a64(nblocks * n) * 4;
  int32_t* order = (int32_t*)p; p += a64(nblocks * n) * 4;
  float* T = (float*)p; p += a64(nblocks * kWin * kWin) * 4;
  float* delta = (float*)p;
  // every workspace entry that is read is written first in the same call (diag_inv, gain, order, the
  // window tiles, and the deltas of the rows that exist), so nothing needs clearing between calls
  hipLaunchKernelGGL(recip_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, n, diag, diag_inv);
  MPQ_LAUNCH_CHECK();
  MPQ_HIP_TRY(run_sweeps(rows, n, maxq, block_rows, nblocks, sweeps, accept_tol, scale, zero, G, group_size, diag,
                         diag_inv, H, rhs, x, q, res_norm, accepted, gain, order, T, delta, stream, recip));
  return kOk;
}

}  // namespace
}  // namespace mpq

extern "C" int mpq_uniform_cd_sweeps(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                     float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                                     int32_t* accepted, const float* scale, const float* zero,
                                     int64_t group_size, const float* diag, const float* H, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  return mpq::cd_sweeps_entry("mpq_uniform_cd_sweeps", rows, n, maxq, block_rows, sweeps, accept_tol, rhs, x, q,
                              res_norm, accepted, scale, zero, group_size, diag, H, workspace, workspace_bytes,
                              stream);
}

extern "C" int mpq_uniform_cd_sweeps_recip(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                           float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                                           int32_t* accepted, const float* scale, const float* zero,
                                           int64_t group_size, const float* diag, const float* H, void* workspace,
                                           int64_t workspace_bytes, hipStream_t stream) {
  return mpq::cd_sweeps_entry("mpq_uniform_cd_sweeps_recip", rows, n, maxq, block_rows, sweeps, accept_tol, rhs, x,
                              q, res_norm, accepted, scale, zero, group_size, diag, H, workspace, workspace_bytes,
                              stream, 1);
}

// ---- allocation-free variant ------------------------------------------------------------------
// The sweeps' workspace lives in a file-scope device array, one copy per GPU, held until the
// process ends.  Its device address is looked up once per device (hipGetSymbolAddress with that
// device current) and only that address is handed to kernels; the array's name is a host-side
// stand-in in host code.  Calls that overlap on one GPU share the array and race.
namespace {

constexpr int64_t kNoAllocScratchBytes = 8ll << 20;  // 8 MiB
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = -1;
  MPQ_HIP_TRY(hipGetDevice(&dev));
  MPQ_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "mpq_uniform_cd_sweeps_noalloc: device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    MPQ_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MPQ_CHECK_ARG(p != nullptr, "mpq_uniform_cd_sweeps_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return mpq::kOk;
}

}  // namespace

extern "C" int64_t mpq_uniform_cd_sweeps_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int mpq_uniform_cd_sweeps_noalloc(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                             float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                                             int32_t* accepted, const float* scale, const float* zero,
                                             int64_t group_size, const float* diag, const float* H,
                                             hipStream_t stream) {
  MPQ_CHECK_ARG(rows > 0 && n > 0 && block_rows >= 1, "mpq_uniform_cd_sweeps_noalloc: empty problem");
  const int64_t need = mpq::sweeps_ws_bytes(rows, n, block_rows);
  MPQ_CHECK_ARG(need <= kNoAllocScratchBytes,
                "mpq_uniform_cd_sweeps_noalloc: needs %lld bytes of scratch, more than the static %lld "
                "(reduce rows or the number of row blocks, or use mpq_uniform_cd_sweeps with a workspace)",
                (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int st = scratch_for_current_device(&ws);
  if (st != mpq::kOk) return st;
  return mpq::cd_sweeps_entry("mpq_uniform_cd_sweeps_noalloc", rows, n, maxq, block_rows, sweeps, accept_tol, rhs,
                              x, q, res_norm, accepted, scale, zero, group_size, diag, H, ws, kNoAllocScratchBytes,
                              stream);
}
