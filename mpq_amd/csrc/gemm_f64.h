// Internal interface of the fp64 MFMA GEMM (gemm_f64.hip): the products of the fp64 eigensolver.
#pragma once

#include "common.h"

namespace mpq {

// Split-K count for an M x N x K fp64 product given a partials capacity (doubles); 1 when the
// product already fills the device or no workspace is given.
int f64_choose_splits(int64_t M, int64_t N, int64_t K, int64_t workspace_elems);

// Row-major C (M x N) = alpha * A (M x K) * op(B) + beta * C, op(B) = B (K x N, ldb) or B^T (B
// stored N x K, trans_b).  With a workspace of at least splits * M * N doubles the K range is split
// (f64_choose_splits) and the partials are summed in split order.  beta == 0 never reads C.
hipError_t gemm_f64(const double* A, int64_t lda, const double* B, int64_t ldb, bool trans_b, double* C,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, double alpha, double beta, double* workspace,
                    int64_t workspace_elems, hipStream_t stream);

// Lower part of a square product (M x M): C = alpha * A op(B) + beta * C on every 128 x 64 tile
// holding an entry (i, j) with j <= i + upper_band (such tiles are computed whole).
hipError_t gemm_f64_lower(const double* A, int64_t lda, const double* B, int64_t ldb, bool trans_b, double* C,
                          int64_t ldc, int64_t M, int64_t K, double alpha, double beta, int64_t upper_band,
                          hipStream_t stream);

}  // namespace mpq
