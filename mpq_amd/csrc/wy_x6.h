// Compact-WY back-transformation on bf16 x6 products (wy_x6.hip): internal interface.
#pragma once

#include "common.h"

namespace mpq {

constexpr int kWyNB = 128;  // reflectors per block (the fp32 block size of eigh.hip)

// Floats of each packed operand buffer for an n x n problem (Yb1, Yb3 and Wp each take this many).
int64_t wy_x6_buffer_floats(int64_t n);

// Writes Y (m x nb, leading dimension nb, m = n - i0) of the block of nb reflectors starting at i0.
struct WyExtractY {
  virtual int operator()(int64_t i0, int nb, float* Y) const = 0;
};

// Z[:, i0 : n] <- Z[:, i0 : n] (I - Y_b Tb_b Y_b^T)^T for the blocks b = nblocks - 1 .. 0 of nrefl
// reflectors (Y_b from extract), Tb_b at Tb + b * kWyNB^2 (nb x nb, leading dimension nb), two blocks
// per pass over Z.  Z is n x n row-major.  Y, Yt, Y2 and Yt2 hold n x kWyNB floats each, P p_splits x
// a64(n x kWyNB) floats of split-K partials, scratch (at least kWyNB^2 + 64 floats; more lets the
// correction products split K) for the pairs' small products; Yb1, Yb3 and Wp wy_x6_buffer_floats(n)
// floats each (16-byte aligned).
int wy_apply_x6(int64_t n, int64_t nrefl, const float* Tb, float* Z, float* Y, float* Yt, float* Y2, float* Yt2,
                float* P, int p_splits, float* scratch, int64_t scratch_floats, void* Yb1, void* Yb3, void* Wp,
                const WyExtractY& extract, hipStream_t stream);

}  // namespace mpq
