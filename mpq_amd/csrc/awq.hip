// AWQ scale search for one linear (or several linears sharing their input), gfx950.
//
// The step before the per-linear solve when AWQ scaling is on (the recipe's "AWQ-style scaling"):
// mpq/awq_scale.py:491-580 (_search_best_scale) with _compute_w_mean (:49-83),
// _candidate_scales (:338-348) and _pseudo_quantize_tensor_into (:108-157).  The reference scores
// each of 20 ratios by running the inspected module; for a single linear layer the output error
// reduces to the quadratic form  sum_rows D H D^T / rows  with D = W - Wq(ratio) and
// H = X^T X / T, which is what this search evaluates:
//   1. w_mean[j] = mean_rows |W[r][j]| / (max_{group of j} |W[r][.]| + 1e-6)
//   2. per ratio r = k/20: s = clamp(x_mean^r / (w_mean^(1-r) + 1e-4), 1e-4),
//      s /= sqrt(max(s) min(s)), inf/nan -> 1
//   3. Wq = pseudo_quant(W * s) / s  (asymmetric min-max or symmetric abs-max per group)
//   4. loss(r) = sum_rows (D H) . D / rows   (split-K MFMA GEMM + fused row dots)
// All 20 losses stay on the device; the host reads them once.
#include <cmath>

#include "common.h"
#include "gemm.h"

namespace mpq {
namespace {

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

// group abs-max gmax[r][g] = max |W[r][g*gs .. (g+1)*gs)|
__global__ __launch_bounds__(256) void group_absmax_kernel(const float* __restrict__ W, int64_t rows, int64_t n,
                                                           int64_t gs, float* __restrict__ gmax) {
  const int64_t G = n / gs;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * G) return;
  const int64_t r = idx / G, g = idx % G;
  float m = 0.f;
  for (int64_t j = 0; j < gs; ++j) m = fmaxf(m, fabsf(W[r * n + g * gs + j]));
  gmax[idx] = m;
}

// w_sum[j] = sum_rows |W[r][j]| / (gmax[r][g(j)] + 1e-6), rows in order
__global__ __launch_bounds__(256) void w_sum_kernel(const float* __restrict__ W, int64_t rows, int64_t n, int64_t gs,
                                                    const float* __restrict__ gmax, float* __restrict__ w_sum) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t G = n / gs;
  const int64_t g = j / gs;
  float acc = 0.f;
  for (int64_t r = 0; r < rows; ++r) acc += fabsf(W[r * n + j]) / (gmax[r * G + g] + 1e-6f);
  w_sum[j] += acc;
}

// candidate scales for ratio k/20 (one work-group): s = clamp(x^r / (w^(1-r) + 1e-4), 1e-4),
// s /= sqrt(max * min), non-finite -> 1
__global__ __launch_bounds__(256) void candidate_scales_kernel(const float* __restrict__ x_mean,
                                                               const float* __restrict__ w_mean, int64_t n,
                                                               float ratio, float* __restrict__ s) {
  __shared__ float smax[256], smin[256];
  float mx = -INFINITY, mn = INFINITY;
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) {
    float v = powf(x_mean[j], ratio) / (powf(w_mean[j], 1.0f - ratio) + 1e-4f);
    v = v < 1e-4f ? 1e-4f : v;  // clamp(min=1e-4) keeps nan
    s[j] = v;
    mx = fmaxf(mx, v);
    mn = fminf(mn, v);
  }
  smax[threadIdx.x] = mx;
  smin[threadIdx.x] = mn;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      smax[threadIdx.x] = fmaxf(smax[threadIdx.x], smax[threadIdx.x + w]);
      smin[threadIdx.x] = fminf(smin[threadIdx.x], smin[threadIdx.x + w]);
    }
    __syncthreads();
  }
  const float norm = sqrtf(smax[0] * smin[0]);
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) {
    float v = s[j] / norm;
    if (isinf(v) || isnan(v)) v = 1.0f;
    s[j] = v;
  }
}

// D = W - pseudo_quant(W * s) / s, one wave per (row, group) (mpq/awq_scale.py:108-157 op order)
__global__ __launch_bounds__(256) void awq_delta_kernel(const float* __restrict__ W, int64_t rows, int64_t n,
                                                        int64_t gs, const float* __restrict__ s, int bits, int sym,
                                                        float* __restrict__ D) {
  const int64_t G = n / gs;
  const int64_t wid = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wid >= rows * G) return;
  const int64_t r = wid / G, g = wid % G;
  const int64_t base = r * n + g * gs;
  float vmax = -INFINITY, vmin = INFINITY, amax = 0.f;
  for (int64_t j = lane; j < gs; j += 64) {
    const float v = W[base + j] * s[g * gs + j];
    vmax = fmaxf(vmax, v);
    vmin = fminf(vmin, v);
    amax = fmaxf(amax, fabsf(v));
  }
  for (int off = 32; off > 0; off >>= 1) {
    vmax = fmaxf(vmax, __shfl_xor(vmax, off));
    vmin = fminf(vmin, __shfl_xor(vmin, off));
    amax = fmaxf(amax, __shfl_xor(amax, off));
  }
  float scale, zero = 0.f, lo, hi;
  if (!sym) {
    const float max_int = (float)((1 << bits) - 1);
    float range = vmax - vmin;
    range = range < 1e-5f ? 1e-5f : range;
    scale = range / max_int;
    zero = -rintf(vmin / scale);
    zero = zero < 0.f ? 0.f : (zero > max_int ? max_int : zero);
    lo = 0.f;
    hi = max_int;
  } else {
    const float m = amax < 1e-5f ? 1e-5f : amax;
    const float max_int = (float)((1 << (bits - 1)) - 1);
    scale = m / max_int;
    lo = -(float)(1 << (bits - 1));
    hi = max_int;
  }
  for (int64_t j = lane; j < gs; j += 64) {
    const float sj = s[g * gs + j];
    const float w = W[base + j];
    float v = w * sj;
    v = v / scale;
    v = rintf(v);
    if (!sym) v = v + zero;
    v = v < lo ? lo : (v > hi ? hi : v);
    if (!sym) v = v - zero;
    v = v * scale;
    D[base + j] = w - v / sj;
  }
}

// loss partials: part[r] = sum_j (sum_s P[s][r][j]) * D[r][j]
__global__ __launch_bounds__(256) void row_quad_kernel(int64_t n, const float* __restrict__ P, int splits,
                                                       int64_t stride, const float* __restrict__ D,
                                                       float* __restrict__ out_row) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  float acc = 0.f;
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) {
    const int64_t o = r * n + j;
    acc += sum_splits(P, splits, stride, o) * D[o];
  }
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) out_row[r] = t;
}

__global__ void loss_kernel(int64_t rows, const float* __restrict__ rowq, float* __restrict__ loss_out) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) acc += rowq[r];
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) *loss_out = t / (float)rows;
}

}  // namespace
}  // namespace mpq

extern "C" int64_t mpq_awq_workspace_size(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  int bn = 128;
  const int splits = mpq::choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  return (mpq::a64(rows * n) * (1 + splits) + mpq::a64(rows) * 2 + mpq::a64(n) * 2 + 64) * 4;
}

extern "C" int mpq_awq_w_mean(const float* W, int64_t rows, int64_t n, int64_t group_size, float* w_sum,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(rows > 0 && n > 0 && group_size >= 1 && n % group_size == 0,
                "weight shape (%lld, %lld) is not divisible by group_size=%lld", (long long)rows, (long long)n,
                (long long)group_size);
  MPQ_CHECK_ARG(W && w_sum && workspace && workspace_bytes >= a64(rows * (n / group_size)) * 4,
                "mpq_awq_w_mean: bad pointer or workspace");
  float* gmax = static_cast<float*>(workspace);
  const int64_t cnt = rows * (n / group_size);
  hipLaunchKernelGGL(group_absmax_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, stream, W, rows, n,
                     group_size, gmax);
  hipLaunchKernelGGL(w_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, W, rows, n, group_size,
                     gmax, w_sum);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_awq_search(const float* W, int64_t rows, int64_t n, const float* H, const float* x_mean,
                              const float* w_mean, int64_t group_size, int bits, int sym, float* best_scales,
                              float* losses_out, float* best_error, float* best_ratio, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(rows > 0 && n > 0 && group_size >= 1 && n % group_size == 0,
                "org_shape[-1]=%lld must be divisible by group_size=%lld", (long long)n, (long long)group_size);
  MPQ_CHECK_ARG(bits >= 2 && bits <= 8, "mpq_awq_search: bits must be in [2, 8]");
  MPQ_CHECK_ARG(W && H && x_mean && w_mean && best_scales && workspace, "mpq_awq_search: null pointer");
  MPQ_CHECK_ARG(workspace_bytes >= mpq_awq_workspace_size(rows, n), "mpq_awq_search: workspace too small");
  MPQ_CHECK_ARG(rows <= 65535 * 128LL, "mpq_awq_search: too many rows");
  int bn = 128;
  const int splits = choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  char* p = static_cast<char*>(workspace);
  float* D = (float*)p; p += a64(rows * n) * 4;
  float* P = (float*)p; p += a64(rows * n) * splits * 4;
  float* rowq = (float*)p; p += a64(rows) * 4;
  float* losses = (float*)p; p += a64(rows) * 4;  // first 20 used
  float* s = (float*)p; p += a64(n) * 4;
  float* s_best = (float*)p;
  const int64_t G = n / group_size;
  const int64_t waves = rows * G;
  for (int k = 0; k < 20; ++k) {
    const float ratio = (float)k / 20.0f;
    hipLaunchKernelGGL(candidate_scales_kernel, dim3(1), dim3(256), 0, stream, x_mean, w_mean, n, ratio, s);
    hipLaunchKernelGGL(awq_delta_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, W, rows, n,
                       group_size, s, bits, sym ? 1 : 0, D);
    MPQ_LAUNCH_CHECK();
    GemmParams gp{};
    gp.M = rows; gp.N = n; gp.K = n;
    gp.A = D; gp.lda = n; gp.B = H; gp.ldb = n; gp.trans_b = false;
    gp.C = P; gp.ldc = n; gp.split_stride = a64(rows * n);
    gp.alpha = 1.f; gp.beta = 0.f; gp.mode = kGemmPartials;
    MPQ_HIP_TRY(gemm_partials(gp, splits, bn, stream));
    hipLaunchKernelGGL(row_quad_kernel, dim3((unsigned)rows), dim3(256), 0, stream, n, P, splits, a64(rows * n), D,
                       rowq);
    hipLaunchKernelGGL(loss_kernel, dim3(1), dim3(256), 0, stream, rows, rowq, losses + k);
    MPQ_LAUNCH_CHECK();
  }
  float hl[20];
  MPQ_HIP_TRY(hipMemcpyAsync(hl, losses, sizeof(hl), hipMemcpyDeviceToHost, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  int best = -1;
  float be = INFINITY;
  for (int k = 0; k < 20; ++k) {
    if (hl[k] < be) {
      be = hl[k];
      best = k;
    }
  }
  if (best < 0) {
    set_error("AWQ scale search failed to find a valid ratio");
    set_error_code(kNumerical);
    return kNumerical;
  }
  hipLaunchKernelGGL(candidate_scales_kernel, dim3(1), dim3(256), 0, stream, x_mean, w_mean, n,
                     (float)best / 20.0f, s_best);
  MPQ_LAUNCH_CHECK();
  MPQ_HIP_TRY(hipMemcpyAsync(best_scales, s_best, n * 4, hipMemcpyDeviceToDevice, stream));
  if (losses_out) MPQ_HIP_TRY(hipMemcpyAsync(losses_out, hl, sizeof(hl), hipMemcpyHostToDevice, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  if (best_error) *best_error = be;
  if (best_ratio) *best_ratio = (float)best / 20.0f;
  return kOk;
}
