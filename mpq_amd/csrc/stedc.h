// Divide-and-conquer eigensolver of a symmetric tridiagonal matrix (the second stage of
// mpq_syevd and mpq_syevd_f64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mpq {

// Device workspace (bytes) of tridiag_dc for order n and element size 4 (fp32) or 8 (fp64).
int64_t tridiag_dc_workspace_bytes(int64_t n, int elem_size);

// Eigen-decomposition T = Z^T diag(lam) Z of the tridiagonal T (diagonal d[0..n-1], off-diagonal
// e[0..n-2]): lam ascending, Z n x n row-major with row k = eigenvector k.  `ws` is 256-byte
// aligned, `ws_bytes` >= tridiag_dc_workspace_bytes(n, sizeof(T)).  Synchronises `stream` once per
// merge of more than 512 rows (the host sizes that merge's GEMMs); the caller synchronises `stream`
// before its next call on the same host thread (the node lists are staged in a per-thread pinned
// buffer).  The merge products run on this library's MFMA GEMMs (fp32 or fp64).
int tridiag_dc(int64_t n, const float* d, const float* e, float* lam, float* Z, void* ws, int64_t ws_bytes,
               hipStream_t stream);
int tridiag_dc(int64_t n, const double* d, const double* e, double* lam, double* Z, void* ws,
               int64_t ws_bytes, hipStream_t stream);

}  // namespace mpq
