// Internal interface of the uniform-grid VAMP solver (uniform_vamp.hip).
#pragma once

#include "common.h"

#include "mpq_amd.h"

namespace mpq {

struct UniformProblem {
  int64_t rows, n;
  int maxq;
  const float* W;        // rows x n (prior centre and target)
  const float* x_init;   // rows x n RTN decision (init_from rtn; gamma1 init)
  const float* scale;    // rows x G (G = ceil(n / group_size))
  const float* zero;     // rows x G
  int64_t group_size;
  const float* V;        // n x n eigenvectors (columns)
  const float* S;        // n sqrt-eigenvalues
  int64_t ldw;           // row stride of W / x_init (elements)
  // optional products computed by the caller for all rows at once (rows x n, contiguous)
  const float* Yu_in = nullptr;   // W Vs
  const float* xr_in = nullptr;   // x_init Vs
  float* xprod_out = nullptr;     // receives x_best Vs of the returned decision
  // optional packed rank-space operator (mpq_rankspace_pack: V for r V, V for x V^T, Vs for x Vs);
  // when given, the products run on the bf16 matrix cores (x6_gemm_partials)
  const float* packed = nullptr;
};

}  // namespace mpq
