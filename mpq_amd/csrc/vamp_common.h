// Kernels shared by the uniform and E8P12 VAMP drivers (included by each driver's
// translation unit): row statistics, the r2 message, the two LMMSE epilogues,
// the rank-space error and the gamma initialisation.  Every kernel follows the
// reference's operation order (mpq/solver.py:426-703, :961-1122; mpq/linear.py).
#pragma once

#include <chrono>
#include <cstring>

#include "common.h"
#include "x6_split.h"

namespace mpq {
namespace {

constexpr int kEW = 256;             // threads per element-wise work-group
constexpr int kPer = 4;              // elements per thread
constexpr int kChunk = kEW * kPer;   // columns per work-group
constexpr float kAlphaEps = 1e-7f;
constexpr float kPrecEps = 1e-12f;

__device__ __forceinline__ float one_minus_alpha_eps() { return (float)(1.0 - 1e-7); }

struct VampStatus {
  int a1_invalid;
  int a1_nonfinite;
  int g2new_invalid;
  int g2_invalid;
  int a2_clip;
  int g1_invalid;
  int pad0, pad1;
  float a1_mean;
  float a2_mean;
  float err_mean;
  float em_mean;
  float err_sum;
  float pad2, pad3, pad4;
};

// Status handshake with the host.  The drivers read the status twice per iteration; instead of a
// device-to-host copy plus a stream synchronisation, a one-thread kernel copies the status into
// mapped, coherent pinned host memory and then publishes a sequence number behind a system-scope
// fence, and the host spins on that number.  The wait is bounded: past a time limit the host falls
// back to hipStreamSynchronize, which returns any error of the stream's earlier work.
struct StatusMailbox {
  VampStatus st;
  unsigned seq;
  unsigned pad[15];
};

// Copy the status to the mapped host mailbox, then publish its sequence number behind a
// system-scope fence (the host reads the status once it sees `seq`).  One thread.
__device__ __forceinline__ void publish_to(const VampStatus* st, StatusMailbox* box, unsigned seq) {
  box->st = *st;
  __threadfence_system();
  __hip_atomic_store(&box->seq, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// bf16 planes of this work-group's column chunk of row b, staged in s_v (column
// blockIdx.x * kChunk + i at s_v[i]), at their place in the packed left operand At of the next x6
// product (n % 16 == 0).  The producing kernels write them so the product needs no packing launch.
__device__ __forceinline__ void chunk_planes(uint4* __restrict__ At, int64_t n, int64_t b, const float* s_v) {
  const int64_t j0 = (int64_t)blockIdx.x * kChunk + 4 * threadIdx.x;
  if (j0 < n) {
    const float4 v = *reinterpret_cast<const float4*>(s_v + 4 * threadIdx.x);
    store_planes4(At, n, b, j0, v.x, v.y, v.z, v.w);
  }
}

__global__ __launch_bounds__(64) void publish_status_kernel(const VampStatus* __restrict__ src,
                                                            StatusMailbox* __restrict__ box, unsigned seq) {
  if (threadIdx.x == 0) publish_to(src, box, seq);
}

// Two mailbox slots, used by alternate sequence numbers: a status may be published (seq + 1) while the
// host has not yet read the one before it (seq), as when a driver launches the next iteration's first
// row kernel ahead of reading the current one's status.  Every driver waits for status seq before it
// launches anything that publishes seq + 2, so a slot is never rewritten before it is read.
struct HostMailbox {
  StatusMailbox* h = nullptr;  // host view of the two slots
  StatusMailbox* d = nullptr;  // device view of the same pages
  unsigned seq = 0;
  StatusMailbox* dev(unsigned s) const { return d + (s & 1u); }
};

// One mailbox per host thread (allocated on first use, freed by mpq_release_thread_resources).
inline HostMailbox* host_mailbox() {
  static thread_local HostMailbox mb;
  if (mb.h == nullptr) {
    StatusMailbox* h = nullptr;
    if (hipHostMalloc((void**)&h, 2 * sizeof(StatusMailbox),
                      hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable) != hipSuccess)
      return nullptr;
    std::memset(h, 0, 2 * sizeof(StatusMailbox));
    StatusMailbox* d = nullptr;
    if (hipHostGetDevicePointer((void**)&d, h, 0) != hipSuccess) {
      (void)hipHostFree(h);
      return nullptr;
    }
    mb.h = h;
    mb.d = d;
    track_pinned(reinterpret_cast<void**>(&mb.h), reinterpret_cast<void**>(&mb.d), nullptr);
  }
  return &mb;
}

// Wait for the status published with sequence number `seq` (by publish_status_kernel or by a
// row kernel that publishes at its end) and copy it to *out.
inline int wait_status(HostMailbox* mb, unsigned seq, VampStatus* out, hipStream_t stream) {
  const auto t0 = std::chrono::steady_clock::now();
  unsigned spins = 0;
  const StatusMailbox* box = mb->h + (seq & 1u);
  while (__atomic_load_n(&box->seq, __ATOMIC_ACQUIRE) != seq) {
    __builtin_ia32_pause();
    if ((++spins & 4095u) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::seconds(20)) {
      MPQ_HIP_TRY(hipStreamSynchronize(stream));
      if (__atomic_load_n(&box->seq, __ATOMIC_ACQUIRE) != seq) {
        set_error("VAMP status handshake: the status kernel completed but its sequence number did not arrive");
        set_error_code(kHipError);
        return kHipError;
      }
      break;
    }
  }
  std::memcpy(out, &box->st, sizeof(VampStatus));
  return kOk;
}

// Copy the device status to *out once every earlier operation on `stream` has completed.
inline int read_status(HostMailbox* mb, const VampStatus* dstatus, VampStatus* out, hipStream_t stream) {
  const unsigned seq = ++mb->seq;
  hipLaunchKernelGGL(publish_status_kernel, dim3(1), dim3(64), 0, stream, dstatus, mb->dev(seq), seq);
  MPQ_LAUNCH_CHECK();
  return wait_status(mb, seq, out, stream);
}

__device__ __forceinline__ float grp(const float* a, int64_t b, int64_t G, int64_t gs, int64_t j) {
  return a[b * G + j / gs];
}

// alpha1 = gamma * mean_j(var) per row (mpq/priors/uniform.py:191), one work-group per row.
__global__ __launch_bounds__(kEW) void row_alpha_kernel(int64_t n, const float* __restrict__ var,
                                                        const float* __restrict__ gamma,
                                                        float* __restrict__ alpha1) {
  __shared__ float red[kEW / 64];
  const int64_t b = blockIdx.x;
  float acc = 0.f;
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) acc += var[b * n + j];
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) alpha1[b] = gamma[b] * (t / (float)n);
}

// Row statistics after the denoiser (mpq/solver.py:575-615): alpha1, eta1,
// gamma2_new, damped gamma2, validity counts.  One work-group, rows looped.
__global__ __launch_bounds__(kEW) void rows_alpha1_kernel(
    int64_t rows, int64_t n, int nchunks, const float* __restrict__ var_part,
    const float* __restrict__ g1w, int has_prev, float damping, const float* __restrict__ g2prev,
    float* __restrict__ alpha1_raw, float* __restrict__ alpha1, float* __restrict__ eta1,
    float* __restrict__ g2new, float* __restrict__ g2, VampStatus* __restrict__ st, StatusMailbox* box,
    unsigned seq) {
  __shared__ float red[kEW / 64];
  int inval = 0, nonfin = 0, g2n_bad = 0, g2_bad = 0;
  float a1part = 0.f;  // this thread's rows of sum(alpha1), in row order
  const float hi = one_minus_alpha_eps();
  for (int64_t b = threadIdx.x; b < rows; b += blockDim.x) {
    float vs = var_part[b * nchunks];
    for (int c = 1; c < nchunks; ++c) vs = vs + var_part[b * nchunks + c];
    const float a1 = g1w[b] * (vs / (float)n);
    alpha1_raw[b] = a1;
    const bool fin = isfinite(a1);
    const bool valid = fin && a1 > kAlphaEps && a1 < hi;
    inval += !valid;
    nonfin += !fin;
    float a1c = a1;
    if (isnan(a1c)) a1c = 0.5f;
    else if (isinf(a1c)) a1c = a1c > 0.f ? hi : kAlphaEps;
    a1c = a1c < kAlphaEps ? kAlphaEps : (a1c > hi ? hi : a1c);
    alpha1[b] = a1c;
    a1part += a1c;
    const float e1 = g1w[b] / a1c;
    eta1[b] = e1;
    const float gn = nan_to_num_clamp_min(e1 - g1w[b], 1e-12f, 1e12f, 1e-12f, kPrecEps);
    g2new[b] = gn;
    g2n_bad += !(isfinite(gn) && gn > kPrecEps);
    float gd = gn;
    if (has_prev && damping < 1.f) {
      if (damping <= 0.f) {
        gd = g2prev[b];
      } else {
        const float p = g2prev[b] < 1e-12f ? 1e-12f : g2prev[b];
        const float q = gn < 1e-12f ? 1e-12f : gn;
        gd = expf((1.0f - damping) * logf(p) + damping * logf(q));
      }
    }
    g2[b] = gd;
    g2_bad += !(isfinite(gd) && gd > kPrecEps);
  }
  // counts: exact in fp32 for < 2^24 rows
  const float s_inval = block_sum((float)inval, red);
  const float s_nonfin = block_sum((float)nonfin, red);
  const float s_g2n = block_sum((float)g2n_bad, red);
  const float s_g2 = block_sum((float)g2_bad, red);
  const float a1sum = block_sum(a1part, red);
  if (threadIdx.x == 0) {
    st->a1_invalid = (int)s_inval;
    st->a1_nonfinite = (int)s_nonfin;
    st->g2new_invalid = (int)s_g2n;
    st->g2_invalid = (int)s_g2;
    st->a1_mean = a1sum / (float)rows;
    if (box) publish_to(st, box, seq);  // saves the launch of publish_status_kernel
  }
}

// gamma retry (mpq/solver.py:594-596).
__global__ void rows_retry_kernel(int64_t rows, const float* __restrict__ alpha1_raw, float factor,
                                  float* __restrict__ g1w) {
  const float hi = one_minus_alpha_eps();
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < rows;
       b += (int64_t)gridDim.x * blockDim.x) {
    const float a = alpha1_raw[b];
    float g = g1w[b];
    if (a <= kAlphaEps) g = g / factor;
    if (a >= hi) g = g * factor;
    g1w[b] = g < 1e-12f ? 1e-12f : g;
  }
}

// r2 message (mpq/solver.py:605-612).
__global__ __launch_bounds__(kEW) void msg_r2_kernel(int64_t n, const float* __restrict__ x1,
                                                     const float* __restrict__ r1,
                                                     const float* __restrict__ eta1,
                                                     const float* __restrict__ g1w,
                                                     const float* __restrict__ g2new, int has_prev,
                                                     float damping, const float* __restrict__ r2prev,
                                                     float* __restrict__ r2, uint4* __restrict__ planes) {
  __shared__ __attribute__((aligned(16))) float s_v[kChunk];
  const int64_t b = blockIdx.y;
  const float e1 = eta1[b], gw = g1w[b], gn = g2new[b];
  const bool damp = has_prev && damping < 1.f;
  const float keep = 1.0f - damping;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float rn = (e1 * x1[o] - gw * r1[o]) / gn;
    const float v = damp ? keep * r2prev[o] + damping * rn : rn;
    r2[o] = v;
    if (planes) s_v[e * kEW + threadIdx.x] = v;
  }
  if (planes) {  // uniform
    __syncthreads();
    chunk_planes(planes, n, b, s_v);
  }
}

// LMMSE part 1 (mpq/linear.py:44-55): from P = r2 @ V, per element
//   residual_before = Yu - P*s, denom = obs*s^2 + g2, coeff = obs*s/denom,
//   c = residual_before*coeff (input of the second product); row partial sums of
//   1/denom (alpha2), residual_after^2 and s^2/denom (EM, mpq/linear.py:74-77).
__global__ __launch_bounds__(kEW) void lmmse_epi1_kernel(
    int64_t n, const float* __restrict__ P, int splits, int64_t split_stride,
    const float* __restrict__ Yu, const float* __restrict__ S, const float* __restrict__ g2,
    float obs, float* __restrict__ c_out, float* __restrict__ part3, uint4* __restrict__ planes) {
  __shared__ float red[kEW / 64];
  __shared__ __attribute__((aligned(16))) float s_v[kChunk];
  const int64_t b = blockIdx.y;
  const int nchunks = gridDim.x;
  const float gb = g2[b];
  float sinv = 0.f, sres = 0.f, strace = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float r2v = sum_splits(P, splits, split_stride, o);
    const float sj = S[j];
    const float s2 = sj * sj;
    const float denom = obs * s2 + gb;
    const float rb = Yu[o] - r2v * sj;
    const float coeff = (obs * sj) / denom;
    c_out[o] = rb * coeff;
    if (planes) s_v[e * kEW + threadIdx.x] = rb * coeff;
    sinv += 1.0f / denom;
    const float ra = rb * (gb / denom);
    sres += ra * ra;
    strace += s2 / denom;
  }
  if (planes) {  // uniform
    __syncthreads();
    chunk_planes(planes, n, b, s_v);
  }
  const float t0 = block_sum(sinv, red);
  const float t1 = block_sum(sres, red);
  const float t2 = block_sum(strace, red);
  if (threadIdx.x == 0) {
    float* o = part3 + (b * nchunks + blockIdx.x) * 3;
    o[0] = t0;
    o[1] = t1;
    o[2] = t2;
  }
}

// Row update after LMMSE part 1 (mpq/solver.py:626-653): alpha2, eta2,
// gamma1_new, damped gamma1 (written in place), EM row statistic.
__global__ __launch_bounds__(kEW) void rows_lmmse_kernel(
    int64_t rows, int64_t n, int64_t rank, int nchunks, const float* __restrict__ part3,
    const float* __restrict__ g2, float damping, float* __restrict__ eta2,
    float* __restrict__ g1new, float* __restrict__ g1, float* __restrict__ g1w, VampStatus* __restrict__ st,
    StatusMailbox* box = nullptr, unsigned seq = 0u) {
  __shared__ float red[kEW / 64];
  const float hi = one_minus_alpha_eps();
  const float c0 = (float)(1.0 - (double)rank / (double)n);
  int clip = 0;
  float em_part = 0.f, a2_part = 0.f;  // this thread's rows, in row order
  for (int64_t b = threadIdx.x; b < rows; b += blockDim.x) {
    const float* pp = part3 + b * nchunks * 3;
    float sinv = pp[0], sres = pp[1], strace = pp[2];
    for (int c = 1; c < nchunks; ++c) {
      sinv = sinv + pp[3 * c + 0];
      sres = sres + pp[3 * c + 1];
      strace = strace + pp[3 * c + 2];
    }
    const float gb = g2[b];
    const float a2raw = c0 + (gb / (float)n) * sinv;
    clip += !(isfinite(a2raw) && a2raw > kAlphaEps && a2raw < hi);
    float a2 = a2raw;
    if (isnan(a2)) a2 = 0.5f;
    else if (isinf(a2)) a2 = a2 > 0.f ? hi : kAlphaEps;
    a2 = a2 < kAlphaEps ? kAlphaEps : (a2 > hi ? hi : a2);
    const float e2 = gb / a2;
    eta2[b] = e2;
    const float gn = nan_to_num_clamp_min(e2 - gb, 1e-12f, 1e12f, 1e-12f, kPrecEps);
    g1new[b] = gn;
    float gd = gn;
    if (damping < 1.f) {
      if (damping <= 0.f) {
        gd = g1[b];
      } else {
        const float p = g1[b] < 1e-12f ? 1e-12f : g1[b];
        const float q = gn < 1e-12f ? 1e-12f : gn;
        gd = expf((1.0f - damping) * logf(p) + damping * logf(q));
      }
    }
    g1[b] = gd;
    if (g1w) g1w[b] = gd;  // the next iteration's working gamma1 (its retries scale the copy)
    // EM statistic per row: |residual_after|^2 + trace term; alpha2 kept for stats
    eta2[rows + b] = sres + strace;
    eta2[2 * rows + b] = a2;
    em_part += sres + strace;
    a2_part += a2;
  }
  const float s_clip = block_sum((float)clip, red);
  const float em = block_sum(em_part, red);
  const float a2s = block_sum(a2_part, red);
  if (threadIdx.x == 0) {
    st->a2_clip = (int)s_clip;
    st->em_mean = em / (float)rows;
    st->a2_mean = a2s / (float)rows;
    if (box) publish_to(st, box, seq);  // saves the launch of publish_status_kernel
  }
}

// LMMSE part 2 + r1 message (mpq/linear.py:51-52, mpq/solver.py:645-653):
// x2 = r2 + sum_s P[s], r1_new = (eta2*x2 - g2*r2)/g1_new, r1 <- damped.
__global__ __launch_bounds__(kEW) void lmmse_epi2_kernel(
    int64_t n, const float* __restrict__ P, int splits, int64_t split_stride,
    const float* __restrict__ r2, const float* __restrict__ eta2, const float* __restrict__ g2,
    const float* __restrict__ g1new, float damping, float* __restrict__ r1) {
  const int64_t b = blockIdx.y;
  const float e2 = eta2[b], gb = g2[b], gn = g1new[b];
  const float keep = 1.0f - damping;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float d = sum_splits(P, splits, split_stride, o);
    const float r2v = r2[o];
    const float x2 = r2v + d;
    const float rn = (e2 * x2 - gb * r2v) / gn;
    r1[o] = damping >= 1.f ? rn : keep * r1[o] + damping * rn;
  }
}

// Rank-space error partials (mpq/linear.py:94): sum_j (Yu - sum_s P[s])^2.
// prod (optional, rows x n) receives the summed product x Vs.
__global__ __launch_bounds__(kEW) void err_epi_kernel(int64_t n, const float* __restrict__ P,
                                                      int splits, int64_t split_stride,
                                                      const float* __restrict__ Yu,
                                                      float* __restrict__ part, float* __restrict__ prod) {
  __shared__ float red[kEW / 64];
  const int64_t b = blockIdx.y;
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float v = sum_splits(P, splits, split_stride, o);
    if (prod) prod[o] = v;
    const float d = Yu[o] - v;
    acc += d * d;
  }
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) part[b * gridDim.x + blockIdx.x] = t;
}

// Row sums of chunk partials -> out[b]; st->err_mean / err_sum over rows.
__global__ __launch_bounds__(kEW) void rows_err_kernel(int64_t rows, int nchunks,
                                                       const float* __restrict__ part,
                                                       float* __restrict__ out,
                                                       VampStatus* __restrict__ st, StatusMailbox* box,
                                                       unsigned seq) {
  __shared__ float red[kEW / 64];
  float part_sum = 0.f;  // this thread's rows, in row order
  for (int64_t b = threadIdx.x; b < rows; b += blockDim.x) {
    float v = part[b * nchunks];
    for (int c = 1; c < nchunks; ++c) v = v + part[b * nchunks + c];
    out[b] = v;
    part_sum += v;
  }
  const float s = block_sum(part_sum, red);
  if (threadIdx.x == 0) {
    st->err_sum = s;
    st->err_mean = s / (float)rows;
    if (box) publish_to(st, box, seq);  // saves the launch of publish_status_kernel
  }
}

// gamma1 init (mpq/solver.py:481-483, :85-87): gamma_start * 0.25 / clamp(mean((W-x)^2), 1e-12).
__global__ __launch_bounds__(kEW) void sqdiff_part_kernel(int64_t n, const float* __restrict__ W,
                                                          int64_t ldw, const float* __restrict__ X,
                                                          int64_t ldx, float* __restrict__ part) {
  __shared__ float red[kEW / 64];
  const int64_t b = blockIdx.y;
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const float d = W[b * ldw + j] - X[b * ldx + j];
    acc += d * d;
  }
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) part[b * gridDim.x + blockIdx.x] = t;
}

__global__ __launch_bounds__(kEW) void rows_gamma_init_kernel(int64_t rows, int64_t n, int nchunks,
                                                              const float* __restrict__ part,
                                                              float gamma_start,
                                                              float* __restrict__ g1,
                                                              float* __restrict__ g1w,
                                                              VampStatus* __restrict__ st) {
  __shared__ float red[kEW / 64];
  int bad = 0;
  for (int64_t b = threadIdx.x; b < rows; b += blockDim.x) {
    float v = part[b * nchunks];
    for (int c = 1; c < nchunks; ++c) v = v + part[b * nchunks + c];
    float mse = v / (float)n;
    mse = mse < 1e-12f ? 1e-12f : mse;
    const float g = gamma_start * (0.25f / mse);
    g1[b] = g;
    if (g1w) g1w[b] = g;
    bad += !(isfinite(g) && g > kPrecEps);
  }
  const float s = block_sum((float)bad, red);
  if (threadIdx.x == 0) st->g1_invalid = (int)s;
}

// dst[r * ldd + c] = src[r * lds + c] (elements of T) for r < rows, c < cols.
template <typename T>
__global__ void copy_rows_kernel(T* __restrict__ dst, int64_t ldd, const T* __restrict__ src, int64_t lds,
                                 int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e - r * cols;
    dst[r * ldd + c] = src[r * lds + c];
  }
}

// Strided device-to-device copy of `rows` rows of `row_bytes` as one kernel (16-, 4- or 1-byte
// elements by alignment).  The solvers' small per-block copies take this instead of
// hipMemcpy*Async, whose host-side cost left the GPU idle between their short kernels.
inline hipError_t copy_rows(void* dst, int64_t ldd_bytes, const void* src, int64_t lds_bytes, int64_t rows,
                            int64_t row_bytes, hipStream_t stream) {
  if (rows <= 0 || row_bytes <= 0) return hipSuccess;
  const uintptr_t align = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                          (uintptr_t)ldd_bytes | (uintptr_t)lds_bytes | (uintptr_t)row_bytes;
  const int es = (align & 15u) == 0 ? 16 : (align & 3u) == 0 ? 4 : 1;
  const int64_t cols = row_bytes / es;
  int64_t blocks = (rows * cols + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks;
  if (es == 16)
    hipLaunchKernelGGL(copy_rows_kernel<uint4>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<uint4*>(dst), ldd_bytes / 16, static_cast<const uint4*>(src), lds_bytes / 16, rows,
                       cols);
  else if (es == 4)
    hipLaunchKernelGGL(copy_rows_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<uint32_t*>(dst), ldd_bytes / 4, static_cast<const uint32_t*>(src), lds_bytes / 4,
                       rows, cols);
  else
    hipLaunchKernelGGL(copy_rows_kernel<uint8_t>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<uint8_t*>(dst), ldd_bytes, static_cast<const uint8_t*>(src), lds_bytes, rows, cols);
  return hipGetLastError();
}

}  // namespace
}  // namespace mpq
