// Symmetric eigendecomposition for the rank-space solvers (gfx950).
//
// Replaces the torch.linalg.eigh call of mpq/adapters/gptqmodel.py:276-310 (and the fp32 use of
// mpq/adapters/quip_sharp.py:33-67) with:
//   1. rocSOLVER ssytrd (lower): A = Q T Q^T, T tridiagonal, Q = H(0) H(1) ... H(n-2) stored as
//      LAPACK reflectors (column-major view of the symmetric buffer);
//   2. rocSOLVER sstedc (divide and conquer): T = Z diag(lam) Z^T, eigenvalues ascending;
//   3. back-transformation V = Q Z on fp32 MFMA GEMMs: the reflectors are applied in blocks of
//      kNB as compact-WY factors I - Y Tb Y^T (Tb from the block's gram Y^T Y, LAPACK larft
//      forward/columnwise), last block first: two GEMMs per block instead of rocSOLVER's ormtr.
// Output: lam ascending (n), V (n x n, row-major, column k = eigenvector k), as torch.linalg.eigh.
#include <rocblas/rocblas.h>
#include <rocsolver/rocsolver.h>

#include <algorithm>

#include "common.h"
#include "gemm.h"
#include "kernels.h"

namespace mpq {
namespace {

constexpr int kNB = 128;  // reflectors per compact-WY block

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

// Y (m x nb, row-major, m = n - i0) of reflectors i0 .. i0+nb-1: Y[r'][c] = v_{i0+c}[i0+r'], with
// v_i[i+1] = 1, v_i[r] = A_col[i * n + r] for r > i+1, 0 for r <= i (A column-major).  Starting
// the rows at i0 (a multiple of the block size) keeps the GEMM operands 16-byte aligned.
__global__ __launch_bounds__(256) void extract_y_kernel(const float* __restrict__ A, int64_t n, int64_t i0, int nb,
                                                        float* __restrict__ Y) {
  const int64_t m = n - i0;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= m * nb) return;
  const int64_t rp = e / nb;
  const int c = (int)(e % nb);
  const int64_t r = i0 + rp;
  const int64_t i = i0 + c;
  float v = 0.f;
  if (r == i + 1) v = 1.f;
  else if (r > i + 1) v = A[i * n + r];
  Y[e] = v;
}

// Tb (nb x nb, row-major, upper) from the gram G = Y^T Y and tau (LAPACK larft, forward,
// columnwise): Tb[i][i] = tau_i, Tb[0:i, i] = -tau_i Tb[0:i, 0:i] G[0:i, i].  One work-group.
__global__ __launch_bounds__(256) void larft_kernel(const float* __restrict__ G, const float* __restrict__ tau,
                                                    int nb, float* __restrict__ Tb) {
  __shared__ float sT[kNB][kNB + 1];
  __shared__ float w[kNB];
  for (int e = threadIdx.x; e < nb * nb; e += blockDim.x) sT[e / nb][e % nb] = 0.f;
  __syncthreads();
  for (int i = 0; i < nb; ++i) {
    const float ti = tau[i];
    // w[0:i] = -tau_i G[0:i, i]
    for (int r = threadIdx.x; r < i; r += blockDim.x) w[r] = -ti * G[r * nb + i];
    __syncthreads();
    // T[0:i, i] = T[0:i, 0:i] w (upper triangular)
    for (int r = threadIdx.x; r < i; r += blockDim.x) {
      float acc = 0.f;
      for (int k = r; k < i; ++k) acc += sT[r][k] * w[k];
      sT[r][i] = acc;
    }
    if (threadIdx.x == 0) sT[i][i] = ti;
    __syncthreads();
  }
  for (int e = threadIdx.x; e < nb * nb; e += blockDim.x) Tb[e] = sT[e / nb][e % nb];
}

struct Handle {
  rocblas_handle h = nullptr;
  int device = -1;
};

rocblas_handle get_handle(hipStream_t stream) {
  static thread_local Handle hs[16];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return nullptr;
  if (!hs[dev].h) {
    if (rocblas_create_handle(&hs[dev].h) != rocblas_status_success) return nullptr;
    hs[dev].device = dev;
  }
  if (rocblas_set_stream(hs[dev].h, stream) != rocblas_status_success) return nullptr;
  return hs[dev].h;
}

}  // namespace
}  // namespace mpq

extern "C" int64_t mpq_syevd_workspace_size(int64_t n) {
  if (n <= 0) return 0;
  const int64_t nb = mpq::kNB;
  int bn = 128;
  const int splits = mpq::choose_splits(n, nb, n, (int64_t)1 << 62, &bn);
  // A copy, Z, Y, Y^T, W (n x nb), W2 (n x nb), gram, Tb, split partials, D, E, tau, info
  return (mpq::a64(n * n) * 2 + mpq::a64(n * nb) * 4 + mpq::a64(nb * nb) * 2 +
          mpq::a64(n * nb) * std::max(splits, 1) + mpq::a64(n) * 3 + 64) * 4;
}

extern "C" int mpq_syevd(int64_t n, const float* H, float* lam, float* V, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(n > 0 && n <= 46340, "mpq_syevd: n must be in [1, 46340]");
  MPQ_CHECK_ARG(H && lam && V && workspace, "mpq_syevd: null pointer");
  MPQ_CHECK_ARG(workspace_bytes >= mpq_syevd_workspace_size(n), "mpq_syevd: workspace too small (%lld < %lld)",
                (long long)workspace_bytes, (long long)mpq_syevd_workspace_size(n));
  rocblas_handle h = get_handle(stream);
  MPQ_CHECK_ARG(h != nullptr, "mpq_syevd: rocBLAS handle unavailable");
  const int nb_max = kNB;
  char* p = static_cast<char*>(workspace);
  float* A = (float*)p; p += a64(n * n) * 4;
  float* Z = (float*)p; p += a64(n * n) * 4;
  float* Y = (float*)p; p += a64(n * nb_max) * 4;
  float* Yt = (float*)p; p += a64(n * nb_max) * 4;
  float* W = (float*)p; p += a64(n * nb_max) * 4;
  float* W2 = (float*)p; p += a64(n * nb_max) * 4;
  float* G = (float*)p; p += a64(nb_max * nb_max) * 4;
  float* Tb = (float*)p; p += a64(nb_max * nb_max) * 4;
  int bn = 128;
  const int splits = choose_splits(n, nb_max, n, (int64_t)1 << 62, &bn);
  float* P = (float*)p; p += a64(n * nb_max) * std::max(splits, 1) * 4;
  float* D = (float*)p; p += a64(n) * 4;
  float* E = (float*)p; p += a64(n) * 4;
  float* tau = (float*)p; p += a64(n) * 4;
  rocblas_int* info = (rocblas_int*)p;
  const int ni = (int)n;

  // 1-2: tridiagonalise (the symmetric buffer read column-major) and solve the tridiagonal problem
  MPQ_HIP_TRY(hipMemcpyAsync(A, H, n * n * 4, hipMemcpyDeviceToDevice, stream));
  if (rocsolver_ssytrd(h, rocblas_fill_lower, ni, A, ni, D, E, tau) != rocblas_status_success) {
    set_error("rocsolver_ssytrd failed");
    set_error_code(kHipError);
    return kHipError;
  }
  if (rocsolver_sstedc(h, rocblas_evect_tridiagonal, ni, D, E, Z, ni, info) != rocblas_status_success) {
    set_error("rocsolver_sstedc failed");
    set_error_code(kHipError);
    return kHipError;
  }
  // Z column-major = row-major Zb with Zb = Z^T.  V^T = Zb Q^T, applied block by block:
  //   Zb[:, i0:] <- Zb[:, i0:] - ((Zb[:, i0:] Y) Tb^T) Y^T
  const int64_t nrefl = n - 1;
  for (int64_t i0 = ((nrefl - 1) / kNB) * kNB; i0 >= 0 && nrefl > 0; i0 -= kNB) {
    const int nb = (int)std::min<int64_t>(kNB, nrefl - i0);
    const int64_t m = n - i0;
    const int64_t cnt = m * nb;
    hipLaunchKernelGGL(extract_y_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, stream, A, n, i0, nb, Y);
    MPQ_LAUNCH_CHECK();
    // G = Y^T Y (nb x nb)
    MPQ_HIP_TRY(transpose_matrix(Y, m, nb, nb, Yt, m, stream));
    MPQ_HIP_TRY(gemm(Yt, m, Y, nb, false, nullptr, G, nb, nb, nb, m, 1.f, 0.f, P, a64(n * nb_max) * splits, stream));
    hipLaunchKernelGGL(larft_kernel, dim3(1), dim3(256), 0, stream, G, tau + i0, nb, Tb);
    MPQ_LAUNCH_CHECK();
    // W = Zb[:, i0:] Y  (n x nb)
    MPQ_HIP_TRY(gemm(Z + i0, n, Y, nb, false, nullptr, W, nb, n, nb, m, 1.f, 0.f, P, a64(n * nb_max) * splits,
                     stream));
    // W2 = W Tb^T  (n x nb)
    MPQ_HIP_TRY(gemm(W, nb, Tb, nb, true, nullptr, W2, nb, n, nb, nb, 1.f, 0.f, nullptr, 0, stream));
    // Zb[:, i0:] -= W2 Y^T
    MPQ_HIP_TRY(gemm(W2, nb, Y, nb, true, nullptr, Z + i0, n, n, m, nb, -1.f, 1.f, nullptr, 0, stream));
  }
  // V (row-major, columns = eigenvectors) = (Zb)^T
  MPQ_HIP_TRY(transpose_matrix(Z, n, n, n, V, n, stream));
  MPQ_HIP_TRY(hipMemcpyAsync(lam, D, n * 4, hipMemcpyDeviceToDevice, stream));
  rocblas_int hinfo = 0;
  MPQ_HIP_TRY(hipMemcpyAsync(&hinfo, info, sizeof(hinfo), hipMemcpyDeviceToHost, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  if (hinfo != 0) {
    set_error("rocsolver_sstedc did not converge (info = %d)", (int)hinfo);
    set_error_code(kNumerical);
    return kNumerical;
  }
  return kOk;
}
