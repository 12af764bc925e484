// Two-stage tridiagonalisation for mpq_syevd (fp32): internal interface of eigh_band.hip.
#pragma once

#include "common.h"

namespace mpq {
namespace band {

constexpr int kBW = 32;      // half-bandwidth of the intermediate band matrix
constexpr int kLeaf = 512;   // rows per TSQR leaf of a stage-1 panel
constexpr int kABld = 64;    // band storage: AB[j * kABld + d] = A[j + d][j], d < 2 kBW (bulge room)
constexpr int kABpad = 128;  // zero columns after column n - 1 (tasks at the end read past n)

// Largest n handled: the stacked R factors of one panel (32 rows per leaf) fit one work-group's LDS.
constexpr int64_t kMaxN = (int64_t)kLeaf * 32 + kBW;

// Number of 32-sweep groups, chase steps of group 0, and the blocks of the stage-2 reflectors
// (group g has K0 + 1 - g chase steps, K0 = (n - 2) / 32).
inline int64_t q2_groups(int64_t n) { return n >= 2 ? (n - 2) / kBW + 1 : 0; }
inline int64_t q2_blocks(int64_t n) {
  const int64_t g = q2_groups(n);
  return g * (g + 1) / 2;
}

// Element offsets (floats) of the two-stage workspace, each region 64 floats aligned.
struct Layout {
  int64_t Yl, taul, Rs, E, Rroot, Q1, Y, BP, X, T, Gp, M, Xop, Yop, Y2, Wf, G12, Px, Gd, Rc, Rt, flags, AB, V2, tau2, Pt, prog, Zq, total;
  int64_t ldq;  // leading dimension of Zq (n rounded up to 64)
  int64_t px_floats;
};
Layout layout(int64_t n);

// Stage 1: the symmetric A (full storage, row-major, leading dimension lda, zero padded) becomes
// a band matrix of half-bandwidth kBW in its lower triangle; the reflectors of panel p (rows
// 32 p .. 32 p + 31) are kept in the rows of A as the one-stage reduction keeps its own
// (v_i[i + kBW] = 1 implied, entries i + kBW + 1 .. n - 1 stored in row i), with tau[i].
int sy2sb(int64_t n, float* A, int64_t lda, float* tau, float* ws, const Layout& L, hipStream_t stream);

// Stage 2: band (lower triangle of A) -> tridiagonal D (n), E (n - 1); the reflectors of the
// chase are kept for q2_apply.  Synchronises the stream once (bulge-chasing status).
int sb2st(int64_t n, const float* A, int64_t lda, float* D, float* E, float* ws, const Layout& L,
          hipStream_t stream);

// Z (n x n, row-major, row j = eigenvector j of the tridiagonal matrix) <- Z Q2^T: the rows become
// eigenvectors of the band matrix.  Synchronises the stream once (pipeline status).
int q2_apply(int64_t n, float* Z, float* ws, const Layout& L, hipStream_t stream);

}  // namespace band
}  // namespace mpq
