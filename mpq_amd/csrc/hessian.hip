// Per-linear Hessian accumulation H = beta H + alpha X^T X (gfx950).
//
// The step before the per-linear solve: GPTQModel's add_batch keeps H = 2/m sum_t x_t x_t^T
// (mpq/adapters/gptqmodel.py:39 states the convention) and QUIP#'s hooks accumulate
// H = sum_t x_t x_t^T plus the column sums mu for the mean correction
// (mpq/quip_generic.py:823-921, H / ct - mu mu^T).  Both are one symmetric rank-T update per
// batch of T activations X (T x n, fp32 or bf16).
//
// SYRK on fp32 MFMA (v_mfma_f32_32x32x2_f32): 128 x 64 output tiles, only tiles on or above the
// diagonal do work; each computed element is written to (m, n) and mirrored to (n, m), so H stays
// exactly symmetric.  A = X^T needs no transpose in LDS: a K slab of X^T (128 columns of X, 16
// rows) is loaded along m with float4 reads and stored as [k][m], the layout the MFMA operand
// reads use.  Two K slabs of global loads are in flight (register sets R0/R1).
#include <hip/hip_bf16.h>

#include "common.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 64, WM = 64, WN = 32, BK = 16;
constexpr int kThreads = 256;

template <bool kBf16>
__device__ __forceinline__ float4 load4(const void* base, int64_t idx, bool ok) {
  if (!ok) return make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (kBf16) {
    const __hip_bfloat16* p = static_cast<const __hip_bfloat16*>(base) + idx;
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                       __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
  } else {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
  }
}

template <bool kBf16>
__global__ __launch_bounds__(kThreads) void syrk_kernel(const void* __restrict__ X, int64_t T, int64_t n,
                                                        int64_t ldx, float alpha, float beta,
                                                        float* __restrict__ H, int64_t ldh) {
  constexpr int WAVES_N = BN / WN;
  constexpr int MI = WM / 32, NI = WN / 32;
  constexpr int A_F4 = BM * BK / 4 / kThreads;  // 2
  constexpr int B_F4 = BN * BK / 4 / kThreads;  // 1
  __shared__ float As[2][BK][BM + 4];
  __shared__ float Bs[2][BK][BN + 4];

  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  if (n0 + BN <= m0) return;  // strictly below the diagonal: mirrored from its transpose tile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM;
  const int wn0 = (wave % WAVES_N) * WN;
  const int64_t nslab = (T + BK - 1) / BK;

  float4 ra0[A_F4], rb0[B_F4], ra1[A_F4], rb1[B_F4];
  // A(m, k) = X[k][m0 + m]: thread t loads 4 consecutive m of row k
  auto gload = [&](float4 (&ra)[A_F4], float4 (&rb)[B_F4], int64_t s) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int t = tid + i * kThreads;
      const int k = t / (BM / 4);
      const int mq = (t % (BM / 4)) * 4;
      const int64_t gk = s * BK + k;
      ra[i] = load4<kBf16>(X, gk * ldx + m0 + mq, gk < T);
    }
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int t = tid + i * kThreads;
      const int k = t / (BN / 4);
      const int nq = (t % (BN / 4)) * 4;
      const int64_t gk = s * BK + k;
      rb[i] = load4<kBf16>(X, gk * ldx + n0 + nq, gk < T);
    }
  };
  auto lstore = [&](const float4 (&ra)[A_F4], const float4 (&rb)[B_F4], int buf) {
#pragma unroll
    for (int i = 0; i < A_F4; ++i) {
      const int t = tid + i * kThreads;
      *reinterpret_cast<float4*>(&As[buf][t / (BM / 4)][(t % (BM / 4)) * 4]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_F4; ++i) {
      const int t = tid + i * kThreads;
      *reinterpret_cast<float4*>(&Bs[buf][t / (BN / 4)][(t % (BN / 4)) * 4]) = rb[i];
    }
  };

  floatx16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int kl = lane >> 5;
  const int ml = lane & 31;
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
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
  };

  gload(ra0, rb0, 0);
  if (nslab > 1) gload(ra1, rb1, 1);
  lstore(ra0, rb0, 0);
  __syncthreads();
  // Pairs of slabs with no exit inside the body (an exit between the halves makes the compiler
  // copy every accumulator through VGPRs each iteration, draining the MFMA pipeline); an odd last
  // slab, already in LDS buffer 0, is computed after the loop.
  int64_t s = 0;
  for (; s + 1 < nslab; s += 2) {
    if (s + 2 < nslab) gload(ra0, rb0, s + 2);
    compute(0);
    lstore(ra1, rb1, 1);
    __syncthreads();
    if (s + 3 < nslab) gload(ra1, rb1, s + 3);
    compute(1);
    if (s + 2 < nslab) lstore(ra0, rb0, 0);
    __syncthreads();
  }
  if (s < nslab) compute(0);

  // epilogue: elements on or above the diagonal, value written to (m, n) and (n, m)
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
        if (gn < gm) continue;
        float* dst = H + gm * ldh + gn;
        const float val = beta == 0.f ? alpha * acc[i][j][v] : alpha * acc[i][j][v] + beta * *dst;
        *dst = val;
        if (gn != gm) H[gn * ldh + gm] = val;
      }
    }
  }
}

// colsum[j] += sum_t X[t][j] (fixed order: per-thread column, rows in order).
template <bool kBf16>
__global__ __launch_bounds__(256) void colsum_kernel(const void* __restrict__ X, int64_t T, int64_t n, int64_t ldx,
                                                     float* __restrict__ colsum) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  float acc = 0.f;
  for (int64_t t = 0; t < T; ++t) {
    float v;
    if constexpr (kBf16) {
      v = __bfloat162float(static_cast<const __hip_bfloat16*>(X)[t * ldx + j]);
    } else {
      v = static_cast<const float*>(X)[t * ldx + j];
    }
    acc += v;
  }
  colsum[j] += acc;
}

}  // namespace

extern "C" int mpq_hessian_accumulate(const void* X, int x_bf16, int64_t T, int64_t n, int64_t ldx, float alpha,
                                      float beta, float* H, int64_t ldh, float* colsum, hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(T >= 0 && n > 0, "mpq_hessian_accumulate: bad shape");
  MPQ_CHECK_ARG(H && (X || T == 0), "mpq_hessian_accumulate: null pointer");
  MPQ_CHECK_ARG(n % 128 == 0, "mpq_hessian_accumulate: n must be a multiple of 128; got %lld", (long long)n);
  MPQ_CHECK_ARG(ldx >= n && ldx % 4 == 0 && ldh >= n, "mpq_hessian_accumulate: bad leading dimension");
  MPQ_CHECK_ARG(T == 0 || (reinterpret_cast<uintptr_t>(X) & (x_bf16 ? 7u : 15u)) == 0,
                "mpq_hessian_accumulate: X must be 16-byte (fp32) / 8-byte (bf16) aligned");
  MPQ_CHECK_ARG(n / 64 <= 65535, "mpq_hessian_accumulate: n too large");
  const dim3 grid((unsigned)(n / BN), (unsigned)(n / BM));
  if (x_bf16) {
    hipLaunchKernelGGL(syrk_kernel<true>, grid, dim3(kThreads), 0, stream, X, T, n, ldx, alpha, beta, H, ldh);
    if (colsum)
      hipLaunchKernelGGL(colsum_kernel<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, X, T, n, ldx,
                         colsum);
  } else {
    hipLaunchKernelGGL(syrk_kernel<false>, grid, dim3(kThreads), 0, stream, X, T, n, ldx, alpha, beta, H, ldh);
    if (colsum)
      hipLaunchKernelGGL(colsum_kernel<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, X, T, n,
                         ldx, colsum);
  }
  MPQ_LAUNCH_CHECK();
  return kOk;
}
