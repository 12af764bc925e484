// Internal helpers shared by the solver drivers (elementwise.hip).
#pragma once

#include "common.h"

namespace mpq {

// x = scale * (q - zero) with group-form parameters (rows x G).
hipError_t dequant_groups(const uint8_t* q, const float* scale, const float* zero, int64_t G,
                          int64_t gs, int64_t rows, int64_t n, float* x, hipStream_t stream);

// Stable descending argsort of `rows_of_keys` independent key rows of length n
// (ties: smaller index first).  n <= 16384.
hipError_t argsort_desc_rows(const float* keys, int64_t nrows, int64_t n, int32_t* order,
                             hipStream_t stream);

// out = in^T (rows x cols -> cols x rows), tiled through LDS.
hipError_t transpose_matrix(const float* in, int64_t rows, int64_t cols, int64_t ld_in, float* out,
                            int64_t ld_out, hipStream_t stream);

// out[j] = max(sum_k M[j][k]^2, floor) for an n x n matrix (row-major).
hipError_t row_sqnorm(const float* M, int64_t n, int64_t ld, float floor, float* out,
                      hipStream_t stream);

}  // namespace mpq
