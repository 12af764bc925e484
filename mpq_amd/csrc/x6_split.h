// Exact three-plane bf16 split of fp32 values (the operands of the x6 products in gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mpq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_bf16(float x, float y) {
  const f32x2_t v = {x, y};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));  // v_cvt_pk_bf16_f32 (RNE)
}

// Three bf16 planes of the pair (x, y), each packed low = x, high = y:
// x = rn(x) + rn(x - rn(x)) + rn(rest) up to 2^-24 |x|.
__device__ __forceinline__ void split3(float x, float y, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = pk_bf16(x, y);
  const float rx = x - __builtin_bit_cast(float, h << 16);
  const float ry = y - __builtin_bit_cast(float, h & 0xffff0000u);
  m = pk_bf16(rx, ry);
  const float sx = rx - __builtin_bit_cast(float, m << 16);
  const float sy = ry - __builtin_bit_cast(float, m & 0xffff0000u);
  l = pk_bf16(sx, sy);
}

// Planes of x[b][j0 .. j0+3] (j0 % 4 == 0, row b, K = n columns with n % 16 == 0) at their place
// in the packed left operand of an x6 product: [ceil(M/128)][n/16][3 planes][256 chunks][8 bf16],
// chunk (blk*2 + h)*32 + r holding row 128 mt + 32 blk + r at k = 16 ks + 8 h + (0..7).
__device__ __forceinline__ void store_planes4(uint4* __restrict__ At, int64_t n, int64_t b, int64_t j0, float v0,
                                              float v1, float v2, float v3) {
  const int64_t KS = n / 16;
  const int64_t mt = b >> 7;
  const int r = (int)(b & 31), blk = (int)((b >> 5) & 3);
  const int64_t ks = j0 >> 4;
  const int h = (int)((j0 >> 3) & 1), half = (int)((j0 >> 2) & 1);
  const int c = (blk * 2 + h) * 32 + r;
  uint2 hi, mi, lo;
  split3(v0, v1, hi.x, mi.x, lo.x);
  split3(v2, v3, hi.y, mi.y, lo.y);
  uint2* base = reinterpret_cast<uint2*>(At + (mt * KS + ks) * 768 + c) + half;
  base[0] = hi;
  base[512] = mi;
  base[1024] = lo;
}

}  // namespace mpq
