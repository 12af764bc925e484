// Generic rank-space block coordinate descent (gfx950): the per-block steps of the reference's
// block_coordinate_descent_rankspace (mpq/polish/block_cd.py:332-625) for any candidate provider,
// and the device side of its providers (:628-861).
//
// The host drives the block loop (the provider is caller code); per block it runs
//   rhs    = residual_u Vs_blk^T                      (MFMA GEMM)
//   target = x_blk + rhs G_blk^-1  (gram) | x_blk + rhs diag_inv  (diag)      bcd_target_kernel
//   cand   = provider(target)                                                  *_propose kernels
//   accept = (res + d G d - 2 rhs.d)_+ + 1e-12 < res (1 + tol), d = cand - x  bcd_accept_kernel
//   residual_u -= (d . accept) Vs_blk                 (MFMA GEMM)
// Per-block metadata (bcd_prepare_kernel): the gram G = Vs_blk Vs_blk^T (fixed-order dot products),
// its Cholesky factor with the reference's diagonal-jitter retries (mpq/linear.py:121-141), the
// inverse (L L^T)^-1 and the static importance trace(G).  Blocks are at most 16 columns wide.
#include <stdint.h>

#include <algorithm>

#include "common.h"
#include "e8p12_tables.inc"
#include "mpq_amd.h"

namespace mpq {
namespace {

constexpr int kMaxBS = 16;
constexpr int kThr = 256;

// One work-group per block.  Outputs per block b: gram[b] (bs x bs), chol[b] (lower, gram metric),
// ginv[b] ((L L^T)^-1, gram metric) or ginv[b][0..bs) = 1 / max(G_ii, 1e-12) (diag metric),
// importance[b] = trace(G), status[b] = 0 or 1 (Cholesky failed after every retry).
__global__ __launch_bounds__(kThr) void bcd_prepare_kernel(int64_t R, int bs, int metric_gram,
                                                           const float* __restrict__ Vs, int64_t ldv,
                                                           float* __restrict__ gram, float* __restrict__ chol,
                                                           float* __restrict__ ginv, float* __restrict__ importance,
                                                           int* __restrict__ status) {
  __shared__ float G[kMaxBS][kMaxBS];
  __shared__ float scratch[kThr / 64];
  const int64_t b = blockIdx.x;
  const float* Vb = Vs + b * bs * ldv;
  for (int i = 0; i < bs; ++i) {
    for (int j = 0; j <= i; ++j) {
      float acc = 0.f;
      for (int64_t k = threadIdx.x; k < R; k += kThr) acc = fmaf(Vb[i * ldv + k], Vb[j * ldv + k], acc);
      acc = block_sum(acc, scratch);
      if (threadIdx.x == 0) {
        G[i][j] = acc;
        G[j][i] = acc;
      }
    }
  }
  __syncthreads();
  const int64_t o = b * bs * bs;
  for (int e = threadIdx.x; e < bs * bs; e += kThr) gram[o + e] = G[e / bs][e % bs];
  if (threadIdx.x != 0) return;
  float tr = 0.f;
  for (int i = 0; i < bs; ++i) tr += G[i][i];
  importance[b] = tr;
  if (!metric_gram) {
    for (int i = 0; i < bs; ++i) ginv[o + i] = 1.0f / fmaxf(G[i][i], 1e-12f);
    status[b] = 0;
    return;
  }
  // stabilize_cholesky: floor = max|diag| * 1e-6 + 1e-6; try k adds 2^k floor I to the matrix of the
  // previous try (six tries, then one final attempt)
  float dmax = 0.f;
  for (int i = 0; i < bs; ++i) dmax = fmaxf(dmax, fabsf(G[i][i]));
  const float floor_v = dmax * 1e-6f + 1e-6f;
  float A[kMaxBS][kMaxBS];
  float L[kMaxBS][kMaxBS];
  for (int i = 0; i < bs; ++i)
    for (int j = 0; j < bs; ++j) A[i][j] = G[i][j];
  bool ok = false;
  for (int t = 0; t <= 6 && !ok; ++t) {
    if (t > 0) {
      const float add = ldexpf(floor_v, t - 1);
      for (int i = 0; i < bs; ++i) A[i][i] = A[i][i] + add;
    }
    ok = true;
    for (int j = 0; j < bs && ok; ++j) {
      float d = A[j][j];
      for (int k = 0; k < j; ++k) d -= L[j][k] * L[j][k];
      if (!(d > 0.f)) {
        ok = false;
        break;
      }
      const float ljj = sqrtf(d);
      L[j][j] = ljj;
      for (int i = j + 1; i < bs; ++i) {
        float s = A[i][j];
        for (int k = 0; k < j; ++k) s -= L[i][k] * L[j][k];
        L[i][j] = s / ljj;
      }
      for (int i = 0; i < j; ++i) L[i][j] = 0.f;
    }
  }
  status[b] = ok ? 0 : 1;
  if (!ok) return;
  // Linv (lower), then (L L^T)^-1 = Linv^T Linv
  float Li[kMaxBS][kMaxBS];
  for (int j = 0; j < bs; ++j) {
    for (int i = 0; i < bs; ++i) Li[i][j] = 0.f;
    Li[j][j] = 1.0f / L[j][j];
    for (int i = j + 1; i < bs; ++i) {
      float s = 0.f;
      for (int k = j; k < i; ++k) s += L[i][k] * Li[k][j];
      Li[i][j] = -s / L[i][i];
    }
  }
  for (int i = 0; i < bs; ++i) {
    for (int j = 0; j < bs; ++j) {
      chol[o + i * bs + j] = L[i][j];
      float s = 0.f;
      for (int k = (i > j ? i : j); k < bs; ++k) s += Li[k][i] * Li[k][j];
      ginv[o + i * bs + j] = s;
    }
  }
}

// gain[b] = mean over rows of rhs_b G_b^-1 rhs_b^T (gram) or of sum rhs_b^2 diag_inv_b (diag); rhs
// is rows x n (all blocks).  One work-group per block, rows summed in row order.
__global__ __launch_bounds__(kThr) void bcd_gain_kernel(int64_t rows, int64_t n, int bs, int metric_gram,
                                                        const float* __restrict__ rhs, const float* __restrict__ ginv,
                                                        float* __restrict__ gain) {
  __shared__ float Gi[kMaxBS * kMaxBS];
  __shared__ float part[kThr];
  const int64_t b = blockIdx.x;
  const int64_t o = b * bs * bs;
  for (int e = threadIdx.x; e < bs * bs; e += kThr) Gi[e] = ginv[o + e];
  __syncthreads();
  float acc = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += kThr) {
    const float* h = rhs + r * n + b * bs;
    float v = 0.f;
    if (metric_gram) {
      for (int j = 0; j < bs; ++j) {
        float d = 0.f;
        for (int i = 0; i < bs; ++i) d += h[i] * Gi[i * bs + j];
        v += h[j] * d;
      }
    } else {
      for (int j = 0; j < bs; ++j) v += (h[j] * h[j]) * Gi[j];
    }
    acc += v;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int t = 0; t < kThr; ++t) s += part[t];
    gain[b] = s / (float)(rows > 0 ? rows : 1);
  }
}

// target (rows x bs) = x[:, start:start+bs] + rhs G^-1 (gram) | + rhs diag_inv (diag)
__global__ void bcd_target_kernel(int64_t rows, int64_t n, int bs, int64_t b, int metric_gram,
                                  const float* __restrict__ x, const float* __restrict__ rhs,
                                  const float* __restrict__ ginv, float* __restrict__ target) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * bs) return;
  const int64_t r = e / bs;
  const int j = (int)(e % bs);
  const float* gi = ginv + b * bs * bs;
  const float* h = rhs + r * bs;
  float u;
  if (metric_gram) {
    u = 0.f;
    for (int i = 0; i < bs; ++i) u += h[i] * gi[i * bs + j];
  } else {
    u = h[j] * gi[j];
  }
  target[e] = x[r * n + b * bs + j] + u;
}

// The accept step (mpq/polish/block_cd.py:28-42) and the state update of one block, one thread per
// row: x, res_norm, accepted and the block's index column updated in place; delta (rows x bs) gets
// the accepted moves (zero rows elsewhere) for the residual product.
__global__ void bcd_accept_kernel(int64_t rows, int64_t n, int bs, int64_t b, int64_t nb,
                                  const float* __restrict__ cand, const float* __restrict__ rhs,
                                  const float* __restrict__ gram, float accept_tol, const int64_t* __restrict__ cand_idx,
                                  float* __restrict__ x, float* __restrict__ res_norm, int64_t* __restrict__ idx,
                                  int32_t* __restrict__ accepted, float* __restrict__ delta) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* G = gram + b * bs * bs;
  float* xb = x + r * n + b * bs;
  float d[kMaxBS];
  float cross = 0.f;
  for (int j = 0; j < bs; ++j) {
    d[j] = cand[r * bs + j] - xb[j];
    cross += rhs[r * bs + j] * d[j];
  }
  float dn = 0.f;
  for (int j = 0; j < bs; ++j) {
    float dg = 0.f;
    for (int i = 0; i < bs; ++i) dg += d[i] * G[i * bs + j];
    dn += dg * d[j];
  }
  dn = fmaxf(dn, 0.f);
  const float res = res_norm[r];
  float ce = res + dn - 2.0f * cross;
  ce = fmaxf(ce, 0.f);
  const bool acc = ce + 1e-12f < res * (1.0f + accept_tol);
  for (int j = 0; j < bs; ++j) {
    if (acc) xb[j] = cand[r * bs + j];
    delta[r * bs + j] = acc ? d[j] : 0.f;
  }
  if (acc) {
    res_norm[r] = ce;
    accepted[r] += 1;
    if (idx && cand_idx) idx[r * nb + b] = cand_idx[r];
  }
}

// UniformScalarProvider.propose (block size 1): q = clamp(round(target / s + z), 0, maxq) with the
// entry's expanded scale and zero (scale floored at 1e-12), value s (q - z).
__global__ void bcd_uniform_propose_kernel(int64_t rows, int64_t n, int64_t col, int maxq,
                                           const float* __restrict__ target, const float* __restrict__ scale,
                                           const float* __restrict__ zero, float* __restrict__ vals,
                                           int64_t* __restrict__ q_out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float s = fmaxf(scale[r * n + col], 1e-12f);
  const float z = zero[r * n + col];
  float q = rintf(target[r] / s + z);
  q = fminf(fmaxf(q, 0.f), (float)maxq);
  vals[r] = s * (q - z);
  q_out[r] = (int64_t)q;
}

// UniformTopKProvider.propose: per row the candidate of topk_values[r, col, :] nearest the target
// (first on ties), and its level from topk_q when given.
__global__ void bcd_topk_scalar_propose_kernel(int64_t rows, int64_t n, int64_t col, int64_t k,
                                               const float* __restrict__ target, const float* __restrict__ vals_k,
                                               const int64_t* __restrict__ q_k, float* __restrict__ vals,
                                               int64_t* __restrict__ q_out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* c = vals_k + (r * n + col) * k;
  const float t = target[r];
  int64_t best = 0;
  float bd = (c[0] - t) * (c[0] - t);
  for (int64_t i = 1; i < k; ++i) {
    const float dd = (c[i] - t) * (c[i] - t);
    if (dd < bd || (isnan(dd) && !isnan(bd))) {
      bd = dd;
      best = i;
    }
  }
  vals[r] = c[best];
  if (q_out) q_out[r] = q_k ? q_k[(r * n + col) * k + best] : -1;
}

// E8P12 codeword of index c in the build's table layout (as the polish context's grid_kernel in
// e8p12_cd.hip): abs pattern k = c >> 8, shift branch = parity of the low byte s, sign bits s with
// bit 7 flipped when the branch and the pattern's parity differ.
__device__ __forceinline__ void e8_codeword(int c, float (&v)[8]) {
  const int k = c >> 8;
  const int s = c & 255;
  const int branch = __builtin_popcount(s) & 1;
  const int signs = s ^ (((branch ^ (int)kE8Parity[k]) & 1) << 7);
  const float sh = branch ? -0.25f : 0.25f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = 0.5f * (float)kE8Abs2[k][i];
    v[i] = sh + (((signs >> i) & 1) ? -a : a);
  }
}

constexpr int kArgRows = 32;

// E8P12Provider with the gram metric (mpq/polish/block_cd.py:702-739): per row the codeword c
// minimising |L^T t - L^T c|^2 (computed as |c L|^2 - 2 (t L).(c L); the dropped |t L|^2 is constant
// per row), first index on ties.  Work-group = 32 rows x one chunk of codewords; partial (score,
// index) per chunk, reduced in chunk order by bcd_e8_argmin_reduce_kernel.
__global__ __launch_bounds__(kThr) void bcd_e8_argmin_kernel(int64_t rows, const float* __restrict__ target,
                                                             const float* __restrict__ chol, int chunk,
                                                             float* __restrict__ pscore, int32_t* __restrict__ pidx) {
  __shared__ float tm[kArgRows][8];
  __shared__ float Ls[8][8];
  __shared__ float bs_s[kThr / 64][kArgRows];
  __shared__ int bi_s[kThr / 64][kArgRows];
  const int64_t r0 = (int64_t)blockIdx.x * kArgRows;
  const int c0 = blockIdx.y * chunk;
  if (threadIdx.x < 64) Ls[threadIdx.x / 8][threadIdx.x % 8] = chol[threadIdx.x];
  __syncthreads();
  if (threadIdx.x < kArgRows * 8) {
    const int rr = threadIdx.x / 8, j = threadIdx.x % 8;
    float s = 0.f;
    if (r0 + rr < rows)
      for (int i = 0; i < 8; ++i) s += target[(r0 + rr) * 8 + i] * Ls[i][j];
    tm[rr][j] = s;
  }
  __syncthreads();
  float best[kArgRows];
  int bidx[kArgRows];
#pragma unroll
  for (int rr = 0; rr < kArgRows; ++rr) {
    best[rr] = INFINITY;
    bidx[rr] = 0x7fffffff;
  }
  for (int c = c0 + threadIdx.x; c < c0 + chunk && c < 65536; c += kThr) {
    float v[8], cm[8];
    e8_codeword(c, v);
    float nrm = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[i] * Ls[i][j];
      cm[j] = s;
      nrm += s * s;
    }
#pragma unroll
    for (int rr = 0; rr < kArgRows; ++rr) {
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += tm[rr][j] * cm[j];
      const float sc = nrm - 2.0f * dot;
      if (sc < best[rr]) {  // codewords visited in increasing index per thread: keeps the first
        best[rr] = sc;
        bidx[rr] = c;
      }
    }
  }
  // wave then work-group minimum with the smaller index on ties
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int rr = 0; rr < kArgRows; ++rr) {
    float s = best[rr];
    int i = bidx[rr];
    for (int off = 32; off >= 1; off >>= 1) {
      const float so = __shfl_xor(s, off, 64);
      const int io = __shfl_xor(i, off, 64);
      if (so < s || (so == s && io < i)) {
        s = so;
        i = io;
      }
    }
    if (lane == 0) {
      bs_s[wave][rr] = s;
      bi_s[wave][rr] = i;
    }
  }
  __syncthreads();
  if (threadIdx.x < kArgRows && r0 + threadIdx.x < rows) {
    float s = bs_s[0][threadIdx.x];
    int i = bi_s[0][threadIdx.x];
    for (int w = 1; w < kThr / 64; ++w) {
      const float so = bs_s[w][threadIdx.x];
      const int io = bi_s[w][threadIdx.x];
      if (so < s || (so == s && io < i)) {
        s = so;
        i = io;
      }
    }
    pscore[(int64_t)blockIdx.y * rows + r0 + threadIdx.x] = s;
    pidx[(int64_t)blockIdx.y * rows + r0 + threadIdx.x] = i;
  }
}

__global__ void bcd_e8_argmin_reduce_kernel(int64_t rows, int nchunks, const float* __restrict__ pscore,
                                            const int32_t* __restrict__ pidx, float* __restrict__ vals,
                                            int64_t* __restrict__ idx) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = pscore[r];
  int i = pidx[r];
  for (int c = 1; c < nchunks; ++c) {
    const float so = pscore[(int64_t)c * rows + r];
    if (so < s) {  // chunks hold increasing indices: an equal score keeps the earlier one
      s = so;
      i = pidx[(int64_t)c * rows + r];
    }
  }
  if (i < 0 || i >= 65536) i = 0;  // every score NaN: the reference's argmin would return 0 too
  float v[8];
  e8_codeword(i, v);
  for (int j = 0; j < 8; ++j) vals[r * 8 + j] = v[j];
  idx[r] = i;
}

// E8P12TopKProvider: per row the candidate topk_idx[r, b, :] nearest the target, whitened by L
// (gram, |tL - cL|^2 clamped at 0 as the reference's select) or plain (diag); first on ties.
__global__ void bcd_e8_topk_propose_kernel(int64_t rows, int64_t nb, int64_t b, int64_t k,
                                           const int64_t* __restrict__ topk_idx, const float* __restrict__ target,
                                           const float* __restrict__ chol, float* __restrict__ vals,
                                           int64_t* __restrict__ idx) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float t[8], tm[8];
  for (int j = 0; j < 8; ++j) t[j] = target[r * 8 + j];
  float tn = 0.f;
  if (chol) {
    for (int j = 0; j < 8; ++j) {
      float s = 0.f;
      for (int i = 0; i < 8; ++i) s += t[i] * chol[i * 8 + j];
      tm[j] = s;
      tn += s * s;
    }
  }
  const int64_t* ci = topk_idx + (r * nb + b) * k;
  int64_t best = 0;
  float bd = INFINITY;
  for (int64_t q = 0; q < k; ++q) {
    int64_t c = ci[q];
    if (c < 0 || c >= 65536) c = 0;
    float v[8];
    e8_codeword((int)c, v);
    float dist = 0.f;
    if (chol) {
      float cn = 0.f, cross = 0.f;
      for (int j = 0; j < 8; ++j) {
        float s = 0.f;
        for (int i = 0; i < 8; ++i) s += v[i] * chol[i * 8 + j];
        cn += s * s;
        cross += s * tm[j];
      }
      dist = fmaxf(tn + cn - 2.0f * cross, 0.f);
    } else {
      for (int j = 0; j < 8; ++j) dist += (v[j] - t[j]) * (v[j] - t[j]);
    }
    if (dist < bd) {
      bd = dist;
      best = q;
    }
  }
  int64_t c = ci[best];
  if (c < 0 || c >= 65536) c = 0;
  float v[8];
  e8_codeword((int)c, v);
  for (int j = 0; j < 8; ++j) vals[r * 8 + j] = v[j];
  idx[r] = ci[best];
}

inline unsigned g1(int64_t n, int t = 256) { return (unsigned)((n + t - 1) / t); }

}  // namespace
}  // namespace mpq

using namespace mpq;

extern "C" int mpq_bcd_prepare(int64_t n, int64_t R, int block_size, int metric_gram, const float* Vs, float* gram,
                               float* chol, float* ginv, float* importance, int32_t* status, mpq_stream_t stream) {
  MPQ_CHECK_ARG(n > 0 && R >= 0 && block_size >= 1 && block_size <= kMaxBS && n % block_size == 0,
                "mpq_bcd_prepare: need 1 <= block_size <= %d dividing n", kMaxBS);
  MPQ_CHECK_ARG(Vs && gram && ginv && importance && status && (chol || !metric_gram), "mpq_bcd_prepare: null argument");
  hipLaunchKernelGGL(bcd_prepare_kernel, dim3((unsigned)(n / block_size)), dim3(kThr), 0, stream, R, block_size,
                     metric_gram, Vs, R, gram, chol, ginv, importance, status);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_gain(int64_t rows, int64_t n, int block_size, int metric_gram, const float* rhs,
                            const float* ginv, float* gain, mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n > 0 && block_size >= 1 && block_size <= kMaxBS && n % block_size == 0,
                "mpq_bcd_gain: bad sizes");
  MPQ_CHECK_ARG(rhs && ginv && gain, "mpq_bcd_gain: null argument");
  hipLaunchKernelGGL(bcd_gain_kernel, dim3((unsigned)(n / block_size)), dim3(kThr), 0, stream, rows, n, block_size,
                     metric_gram, rhs, ginv, gain);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_target(int64_t rows, int64_t n, int block_size, int64_t block, int metric_gram,
                              const float* x, const float* rhs, const float* ginv, float* target, mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n > 0 && block_size >= 1 && block_size <= kMaxBS && n % block_size == 0 &&
                    block >= 0 && block < n / block_size,
                "mpq_bcd_target: bad sizes");
  MPQ_CHECK_ARG(x && rhs && ginv && target, "mpq_bcd_target: null argument");
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(bcd_target_kernel, dim3(g1(rows * block_size)), dim3(256), 0, stream, rows, n, block_size, block,
                     metric_gram, x, rhs, ginv, target);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_accept(int64_t rows, int64_t n, int block_size, int64_t block, const float* cand,
                              const float* rhs, const float* gram, float accept_tol, const int64_t* cand_idx,
                              float* x, float* res_norm, int64_t* idx, int32_t* accepted, float* delta,
                              mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n > 0 && block_size >= 1 && block_size <= kMaxBS && n % block_size == 0 &&
                    block >= 0 && block < n / block_size,
                "mpq_bcd_accept: bad sizes");
  MPQ_CHECK_ARG(cand && rhs && gram && x && res_norm && accepted && delta, "mpq_bcd_accept: null argument");
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(bcd_accept_kernel, dim3(g1(rows)), dim3(256), 0, stream, rows, n, block_size, block,
                     n / block_size, cand, rhs, gram, accept_tol, cand_idx, x, res_norm, idx, accepted, delta);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_uniform_propose(int64_t rows, int64_t n, int64_t col, int maxq, const float* target,
                                       const float* scale, const float* zero, float* vals, int64_t* q,
                                       mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n > 0 && col >= 0 && col < n && maxq >= 1, "mpq_bcd_uniform_propose: bad sizes");
  MPQ_CHECK_ARG(target && scale && zero && vals && q, "mpq_bcd_uniform_propose: null argument");
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(bcd_uniform_propose_kernel, dim3(g1(rows)), dim3(256), 0, stream, rows, n, col, maxq, target,
                     scale, zero, vals, q);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_topk_scalar_propose(int64_t rows, int64_t n, int64_t col, int64_t k, const float* target,
                                           const float* vals_k, const int64_t* q_k, float* vals, int64_t* q,
                                           mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n > 0 && col >= 0 && col < n && k >= 1, "mpq_bcd_topk_scalar_propose: bad sizes");
  MPQ_CHECK_ARG(target && vals_k && vals, "mpq_bcd_topk_scalar_propose: null argument");
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(bcd_topk_scalar_propose_kernel, dim3(g1(rows)), dim3(256), 0, stream, rows, n, col, k, target,
                     vals_k, q_k, vals, q);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int64_t mpq_e8p12_metric_argmin_workspace_size(int64_t rows) {
  if (rows <= 0) return 0;
  return 16 * rows * 8;  // up to 16 chunks of (score, index)
}

extern "C" int mpq_e8p12_metric_argmin(int64_t rows, const float* target, const float* chol, float* vals,
                                       int64_t* idx, void* workspace, int64_t workspace_bytes, mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0, "mpq_e8p12_metric_argmin: negative rows");
  MPQ_CHECK_ARG(target && chol && vals && idx, "mpq_e8p12_metric_argmin: null argument");
  if (rows == 0) return kOk;
  const int64_t tiles = (rows + kArgRows - 1) / kArgRows;
  int nchunks = (int)std::min<int64_t>(16, std::max<int64_t>(1, 512 / tiles));
  MPQ_CHECK_ARG(workspace && workspace_bytes >= (int64_t)nchunks * rows * 8,
                "mpq_e8p12_metric_argmin: workspace too small");
  MPQ_CHECK_ARG(tiles <= 0x7fffffffLL, "mpq_e8p12_metric_argmin: too many rows");
  const int chunk = (65536 + nchunks - 1) / nchunks;
  float* ps = static_cast<float*>(workspace);
  int32_t* pi = reinterpret_cast<int32_t*>(ps + (int64_t)nchunks * rows);
  hipLaunchKernelGGL(bcd_e8_argmin_kernel, dim3((unsigned)tiles, (unsigned)nchunks), dim3(kThr), 0, stream, rows,
                     target, chol, chunk, ps, pi);
  hipLaunchKernelGGL(bcd_e8_argmin_reduce_kernel, dim3(g1(rows)), dim3(256), 0, stream, rows, nchunks, ps, pi, vals,
                     idx);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_bcd_e8_topk_propose(int64_t rows, int64_t nb, int64_t block, int64_t k, const int64_t* topk_idx,
                                       const float* target, const float* chol, float* vals, int64_t* idx,
                                       mpq_stream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && nb > 0 && block >= 0 && block < nb && k >= 1, "mpq_bcd_e8_topk_propose: bad sizes");
  MPQ_CHECK_ARG(topk_idx && target && vals && idx, "mpq_bcd_e8_topk_propose: null argument");
  if (rows == 0) return kOk;
  hipLaunchKernelGGL(bcd_e8_topk_propose_kernel, dim3(g1(rows)), dim3(256), 0, stream, rows, nb, block, k, topk_idx,
                     target, chol, vals, idx);
  MPQ_LAUNCH_CHECK();
  return kOk;
}
