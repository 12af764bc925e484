// Shared helpers for the mpq_amd HIP library: error state, launch checks.
// Every kernel in this library is built for gfx950 only, with
// -ffp-contract=off: fused multiply-adds appear only where written as fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

namespace mpq {

// Status codes returned by every extern "C" entry point.
enum Status : int {
  kOk = 0,
  kInvalidArgument = -1,
  kHipError = -2,
  kUnsupported = -3,
  kNumerical = -4,
};

void set_error(const char* fmt, ...);
const char* last_error();
int last_error_code();
void set_error_code(int code);

// Registers a per-thread pinned host buffer (its host pointer slot, optionally the slot of its
// device view and of its capacity) so that mpq_release_thread_resources() frees it and clears the
// slots; registering the same slot again is a no-op.
void track_pinned(void** host, void** dev, size_t* cap);

}  // namespace mpq

#define MPQ_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      mpq::set_error(__VA_ARGS__);               \
      mpq::set_error_code(mpq::kInvalidArgument);\
      return mpq::kInvalidArgument;              \
    }                                            \
  } while (0)

#define MPQ_HIP_TRY(expr)                                                        \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess) {                                                      \
      mpq::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),      \
                     __FILE__, __LINE__);                                        \
      mpq::set_error_code(mpq::kHipError);                                       \
      return mpq::kHipError;                                                     \
    }                                                                            \
  } while (0)

#define MPQ_LAUNCH_CHECK() MPQ_HIP_TRY(hipGetLastError())

static inline int64_t mpq_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

namespace mpq {

// Deterministic work-group sum (fixed tree: lane shuffles, then waves in order).
// All threads must call it; `scratch` holds blockDim.x/64 floats.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = (blockDim.x + 63) >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = scratch[0];
  for (int w = 1; w < nwaves; ++w) total += scratch[w];
  __syncthreads();
  return total;
}

// Sum of split-K partials P[s * stride + o], s = 0..splits-1, added in split order.  The loads
// are unrolled and predicated in groups of 8 so their latencies overlap.
constexpr int kMaxSplits = 32;
__device__ __forceinline__ float sum_splits(const float* __restrict__ P, int splits, int64_t stride,
                                            int64_t o) {
  float acc = P[o];
#pragma unroll
  for (int s0 = 1; s0 < kMaxSplits; s0 += 8) {
    if (s0 >= splits) break;
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = (s0 + u < splits) ? P[(int64_t)(s0 + u) * stride + o] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < splits) acc = acc + v[u];
  }
  return acc;
}

__device__ __forceinline__ double block_sum_f64(double v, double* scratch) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = (blockDim.x + 63) >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  double total = scratch[0];
  for (int w = 1; w < nwaves; ++w) total += scratch[w];
  __syncthreads();
  return total;
}

// torch.nan_to_num + clamp_min semantics used by the VAMP precision updates.
__device__ __forceinline__ float nan_to_num_clamp_min(float x, float nan_v, float posinf_v,
                                                      float neginf_v, float lo) {
  if (isnan(x)) x = nan_v;
  else if (isinf(x)) x = x > 0.f ? posinf_v : neginf_v;
  return x < lo ? lo : x;
}

}  // namespace mpq
