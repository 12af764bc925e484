// Kernels shared by the coordinate-descent polishes (cd_uniform.hip, e8p12_cd.hip).
#pragma once

#include "common.h"

namespace mpq {
namespace {

// residual_u = Yu - P (sum of split partials), also copies it scaled for the rhs product.
__global__ __launch_bounds__(256) void residual_kernel(int64_t rows, int64_t n, const float* __restrict__ P,
                                                       int splits, int64_t split_stride,
                                                       const float* __restrict__ Yu,
                                                       float* __restrict__ res,
                                                       float* __restrict__ part, int nchunks) {
  __shared__ float red[4];
  const int64_t b = blockIdx.y;
  float acc = 0.f;
  for (int e = 0; e < 4; ++e) {
    const int64_t j = (int64_t)blockIdx.x * 1024 + e * 256 + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float v = sum_splits(P, splits, split_stride, o);
    const float r = Yu[o] - v;
    if (res) res[o] = r;
    acc += r * r;
  }
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) part[b * nchunks + blockIdx.x] = t;
}

__global__ void rows_sum_kernel(int64_t rows, int nchunks, const float* __restrict__ part,
                                float* __restrict__ out) {
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < rows;
       b += (int64_t)gridDim.x * blockDim.x) {
    float v = part[b * nchunks];
    for (int c = 1; c < nchunks; ++c) v = v + part[b * nchunks + c];
    out[b] = v;
  }
}

}  // namespace
}  // namespace mpq
