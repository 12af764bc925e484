// Internal interface of the fp32 MFMA GEMM (gemm.hip).
#pragma once

#include "common.h"

namespace mpq {

enum GemmMode : int {
  kGemmPartials = 0,  // C[split] = partial product (C = workspace, split_stride apart)
  kGemmAxpby = 1,     // single split: C = alpha * A*op(B) + beta * C
};

struct GemmParams {
  int64_t M, N, K;
  const float* A;
  int64_t lda;
  const float* B;
  int64_t ldb;
  const int32_t* b_rows;  // optional row gather of B (trans_b == false only)
  int64_t b_rows_group;   // if > 0: M tile at m0 uses b_rows + (m0 / b_rows_group) * b_rows_group_stride
  int64_t b_rows_group_stride;  //   (b_rows_group must be a multiple of the 128-row M tile)
  float* C;
  int64_t ldc;
  int64_t split_stride;
  int64_t k_per_split;
  float alpha, beta;
  int mode;
  bool trans_b;
  bool a_vec4, b_vec4;
  bool lower_only;  // square C: skip tiles whose first column is >= last row + 1 + upper_band
  int upper_band;
};

// Split-K count and N tile (always 64) for an M x N x K product with the given
// workspace capacity (floats); 1 split when no workspace.
int choose_splits(int64_t M, int64_t N, int64_t K, int64_t workspace_floats, int* bn_out);

// Launch the partial-product kernel: `splits` K slices written to p.C with
// p.split_stride apart (mode kGemmPartials), or one slice with mode kGemmAxpby.
hipError_t gemm_partials(GemmParams p, int splits, int bn, hipStream_t stream);

// C = alpha * sum_s P[s] + beta * C (fixed split order).
hipError_t splitk_reduce(const float* P, int splits, int64_t M, int64_t N, float* C, int64_t ldc,
                         float alpha, float beta, hipStream_t stream);

// Full product with the automatic split choice; `workspace` may be null (1 split).
hipError_t gemm(const float* A, int64_t lda, const float* B, int64_t ldb, bool trans_b,
                const int32_t* b_rows, float* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                float alpha, float beta, float* workspace, int64_t workspace_floats,
                hipStream_t stream);

// Lower part of a square product: C = alpha * A*op(B) + beta * C on every 128 x 64 tile holding
// an entry (i, j) with j <= i + upper_band (such tiles are computed whole).
hipError_t gemm_lower(const float* A, int64_t lda, const float* B, int64_t ldb, bool trans_b, float* C,
                      int64_t ldc, int64_t M, int64_t K, float alpha, float beta, int upper_band,
                      hipStream_t stream);

// fp32 products on the bf16 matrix cores (each operand split exactly into three bf16 planes, six
// plane products; accuracy of an fp32 product, see gemm.hip).  B is packed once into fp32 tiles of
// 128 columns x 16 k (K * N floats); A is split and packed per product (x6_packed_a_bytes).
// Shapes: N % 128 == 0, K % 32 == 0; any M (rows past M are zero in the packed A).
bool x6_shape_ok(int64_t N, int64_t K);
int x6_choose_splits(int64_t M, int64_t N, int64_t K);
int64_t x6_packed_a_bytes(int64_t M, int64_t K);
hipError_t x6_pack_b(const float* B, int64_t ldb, bool trans_b, int64_t K, int64_t N, float* Bt, hipStream_t stream);
// colscale (optional, K floats): pack the planes of A diag(colscale) instead of A.
hipError_t x6_pack_a(const float* A, int64_t lda, int64_t M, int64_t K, void* At, hipStream_t stream,
                     const float* colscale = nullptr);
// C[s] = A[:, K slice s] * op(B)[K slice s, :] for s < splits (K / splits a multiple of 32),
// C[s] at C + s * split_stride with row stride ldc.
hipError_t x6_gemm_partials(const void* At, const float* Bt, int64_t M, int64_t N, int64_t K, float* C, int64_t ldc,
                            int64_t split_stride, int splits, hipStream_t stream);

}  // namespace mpq
