// GPTQ int32 packing of the integer codes and group parameters (gfx950).
//
// The step after the per-linear solve on the GPTQModel path: the MPQ codes (rows = out
// features x n = in features, uint8) and the group parameters become GPTQModel's packed
// tensors (written through patches/gptqmodel.patch:359-395 and scripts/backend_gptq.py:843,
// format GPTQ_V2):
//   qweight  int32 [n * bits / 32, rows]   codes packed along the input dimension
//   qzeros   int32 [G, rows * bits / 32]   zero points packed along the output dimension
//                                          (format v2 stores z, v1 stores z - 1)
//   scales   fp16  [G, rows]
//   g_idx    int32 [n]                     i / group_size (no act-order)
// Packing of 32 / bits values per word, value j at bit bits * j, for bits 2, 4, 8; for 3 bits,
// 32 values in 3 words: word 0 holds values 0-9 at bits 3j and the low 2 bits of value 10 at
// bits 30-31; word 1 holds bit 2 of value 10 at bit 0, values 11-20 at bits 3(j-11)+1 and the
// low bit of value 21 at bit 31; word 2 holds bits 1-2 of value 21 at bits 0-1 and values 22-31
// at bits 3(j-22)+2.  (GPTQModel's published layout; the packer itself is upstream code that
// the reference calls.)
#include <hip/hip_fp16.h>

#include "common.h"

namespace {

// Packs 32 consecutive 3-bit values v[0..31] into 3 words.
__device__ __forceinline__ void pack3(const uint32_t (&v)[32], uint32_t& w0, uint32_t& w1, uint32_t& w2) {
  w0 = 0u;
  w1 = 0u;
  w2 = 0u;
#pragma unroll
  for (int j = 0; j < 10; ++j) w0 |= v[j] << (3 * j);
  w0 |= v[10] << 30;
  w1 |= (v[10] >> 2) & 1u;
#pragma unroll
  for (int j = 11; j < 21; ++j) w1 |= v[j] << (3 * (j - 11) + 1);
  w1 |= v[21] << 31;
  w2 |= (v[21] >> 1) & 3u;
#pragma unroll
  for (int j = 22; j < 32; ++j) w2 |= v[j] << (3 * (j - 22) + 2);
}

// qweight: one thread per (32-value input group t, output column col) for 3 bits, else per
// (word, col); col is the fastest index so the int32 writes are coalesced.
__global__ __launch_bounds__(256) void pack_qweight_kernel(const uint8_t* __restrict__ q, int64_t rows, int64_t n,
                                                           int bits, int32_t* __restrict__ qweight) {
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= rows) return;
  const uint32_t mask = (1u << bits) - 1u;
  const uint8_t* src = q + col * n;
  if (bits == 3) {
    const int64_t t = blockIdx.y;  // 32 input rows
    uint32_t v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = (uint32_t)src[32 * t + j] & mask;
    uint32_t w0, w1, w2;
    pack3(v, w0, w1, w2);
    qweight[(3 * t + 0) * rows + col] = (int32_t)w0;
    qweight[(3 * t + 1) * rows + col] = (int32_t)w1;
    qweight[(3 * t + 2) * rows + col] = (int32_t)w2;
  } else {
    const int per = 32 / bits;
    const int64_t wr = blockIdx.y;
    uint32_t w = 0u;
    for (int j = 0; j < per; ++j) w |= ((uint32_t)src[wr * per + j] & mask) << (bits * j);
    qweight[wr * rows + col] = (int32_t)w;
  }
}

// qzeros (one thread per (group g, output word)), scales (fp16) and g_idx.
__global__ __launch_bounds__(256) void pack_qzeros_kernel(const float* __restrict__ zero, int64_t rows, int64_t G,
                                                          int bits, int v1, int32_t* __restrict__ qzeros) {
  const int64_t words = rows * bits / 32;
  const int64_t wc = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = blockIdx.y;
  if (wc >= words) return;
  const uint32_t mask = (1u << bits) - 1u;
  auto zval = [&](int64_t col) -> uint32_t {
    const int z = (int)rintf(zero[col * G + g]) - (v1 ? 1 : 0);
    return (uint32_t)z & mask;
  };
  if (bits == 3) {
    const int64_t t = wc / 3;  // 32 output columns
    const int which = (int)(wc % 3);
    uint32_t v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = zval(32 * t + j);
    uint32_t w0, w1, w2;
    pack3(v, w0, w1, w2);
    qzeros[g * words + wc] = (int32_t)(which == 0 ? w0 : (which == 1 ? w1 : w2));
  } else {
    const int per = 32 / bits;
    uint32_t w = 0u;
    for (int j = 0; j < per; ++j) w |= zval(wc * per + j) << (bits * j);
    qzeros[g * words + wc] = (int32_t)w;
  }
}

__global__ __launch_bounds__(256) void pack_scales_kernel(const float* __restrict__ scale, int64_t rows, int64_t G,
                                                          __half* __restrict__ scales_out) {
  const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t g = blockIdx.y;
  if (col >= rows) return;
  scales_out[g * rows + col] = __float2half(scale[col * G + g]);
}

__global__ void g_idx_kernel(int64_t n, int64_t group_size, int32_t* __restrict__ g_idx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) g_idx[i] = (int32_t)(i / group_size);
}

}  // namespace

extern "C" int mpq_gptq_pack(const uint8_t* q, const float* scale, const float* zero, int64_t rows, int64_t n,
                             int64_t group_size, int bits, int format_v1, int32_t* qweight, int32_t* qzeros,
                             void* scales_fp16, int32_t* g_idx, hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(bits == 2 || bits == 3 || bits == 4 || bits == 8, "GPTQ packing supports bits 2, 3, 4, 8; got %d",
                bits);
  MPQ_CHECK_ARG(rows > 0 && n > 0 && group_size >= 1, "mpq_gptq_pack: bad shape");
  MPQ_CHECK_ARG(n % 32 == 0 && rows % 32 == 0,
                "GPTQ packing needs in and out features divisible by 32; got %lld x %lld", (long long)rows,
                (long long)n);
  MPQ_CHECK_ARG(q && scale && zero && qweight && qzeros && scales_fp16 && g_idx, "mpq_gptq_pack: null pointer");
  MPQ_CHECK_ARG(rows <= 0x7fffffffLL * 256 && n / 32 * bits <= 65535, "mpq_gptq_pack: extent too large");
  const int64_t G = (n + group_size - 1) / group_size;
  MPQ_CHECK_ARG(G <= 65535, "mpq_gptq_pack: too many groups");
  const unsigned cb = (unsigned)((rows + 255) / 256);
  if (bits == 3) {
    hipLaunchKernelGGL(pack_qweight_kernel, dim3(cb, (unsigned)(n / 32)), dim3(256), 0, stream, q, rows, n, bits,
                       qweight);
  } else {
    hipLaunchKernelGGL(pack_qweight_kernel, dim3(cb, (unsigned)(n * bits / 32)), dim3(256), 0, stream, q, rows, n,
                       bits, qweight);
  }
  const int64_t zwords = rows * bits / 32;
  hipLaunchKernelGGL(pack_qzeros_kernel, dim3((unsigned)((zwords + 255) / 256), (unsigned)G), dim3(256), 0, stream,
                     zero, rows, G, bits, format_v1 ? 1 : 0, qzeros);
  hipLaunchKernelGGL(pack_scales_kernel, dim3(cb, (unsigned)G), dim3(256), 0, stream, scale, rows, G,
                     static_cast<__half*>(scales_fp16));
  hipLaunchKernelGGL(g_idx_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, n, group_size, g_idx);
  MPQ_LAUNCH_CHECK();
  return kOk;
}
