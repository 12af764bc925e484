// Compact-WY back-transformation Z <- Z Q^T (the eigenvector matrix times the reflectors of the
// tridiagonalisation, in blocks of kWyNB) with its three products on the bf16 matrix cores: every
// fp32 operand is split exactly into three bf16 planes and each 16-k step runs the six plane
// products whose plane indices sum to <= 2 (the x6 scheme of gemm.hip, fp32-accurate):
//   Yt = Y Tb^T               fp32 (the GEMM of gemm.hip; m x 128 x 128)
//   W2 = Z[:, i0:] Yt         split-K; Z is split in registers as it streams in, the partials are
//                             added and stored as the planes of -W2
//   Z[:, i0:] += (-W2) Y^T    in place: each fp32 tile of Z is the accumulator
// Packed operand order (both operands of v_mfma_f32_32x32x16_bf16): a matrix M (R x K) taken row
// by row, chunk (T, s, p, lane) = uint4 at ((T * KS + s) * 3 + p) * 64 + lane holding plane p of
// M[32 T + lane % 32][16 s + 8 (lane / 32) + 0 .. 7], KS = K / 16.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "wy_x6.h"
#include "gemm.h"
#include "x6_split.h"

namespace mpq {
namespace {

constexpr int kThr = 256;
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// the three planes of v (times sign) at dst (planes 64 chunks apart)
__device__ __forceinline__ void put3(uint4* __restrict__ dst, const float* v, float sign) {
  uint4 h, m, l;
  split3(sign * v[0], sign * v[1], h.x, m.x, l.x);
  split3(sign * v[2], sign * v[3], h.y, m.y, l.y);
  split3(sign * v[4], sign * v[5], h.z, m.z, l.z);
  split3(sign * v[6], sign * v[7], h.w, m.w, l.w);
  dst[0] = h;
  dst[64] = m;
  dst[128] = l;
}

// Yb3: Y by rows, the right operand of Z += (-W2) Y^T: its kWyNB reflectors fill the 16-k steps
// soff .. soff + 7 of ks3 per 32-row tile (ks3 = 16 when two blocks are applied together; Y null:
// Yb3 untouched); Yb1: Yt^T by rows (K = mpad), the right operand of W2 = Z Yt (Yt null: untouched).
// Y and Yt are m x nb (leading dimension nb); entries past m rows or nb columns are zero.
__global__ __launch_bounds__(kThr) void wy_pack_y_kernel(const float* __restrict__ Y, const float* __restrict__ Yt,
                                                         int nb, int64_t m, int64_t mpad, uint4* __restrict__ Yb1,
                                                         uint4* __restrict__ Yb3, int ks3, int soff, int tc0) {
  const int64_t n3 = Y ? mpad * 16 : 0, q1 = mpad / 8, n1 = Yt ? q1 * kWyNB : 0;
  for (int64_t it = (int64_t)blockIdx.x * kThr + threadIdx.x; it < n3 + n1; it += (int64_t)gridDim.x * kThr) {
    float v[8];
    if (it < n3) {
      const int64_t j = it >> 4;
      const int c8 = (int)(it & 15);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 8 * c8 + e;
        v[e] = (j < m && c < nb) ? Y[j * nb + c] : 0.f;
      }
      const int64_t T = j >> 5;
      const int lane = (c8 & 1) * 32 + (int)(j & 31);
      put3(Yb3 + ((T * ks3 + soff + (c8 >> 1)) * 3) * 64 + lane, v, 1.f);
    } else {
      const int64_t i2 = it - n3;
      const int c = (int)(i2 % kWyNB);
      const int64_t q = i2 / kWyNB;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t r = 8 * q + e;
        v[e] = (r < m && c < nb) ? Yt[r * nb + c] : 0.f;
      }
      const int64_t KS1 = mpad / 16;
      const int lane = (int)(q & 1) * 32 + (c & 31);
      put3(Yb1 + (((int64_t)(tc0 + (c >> 5)) * KS1 + (q >> 1)) * 3) * 64 + lane, v, 1.f);
    }
  }
}

// P[split] (n x kWyNB) = Z[:, i0 + k slice] Yt[k slice, :].  Wave w of a work-group owns rows
// 128 bx + 32 w .. + 31 and all kWyNB columns (four 32 x 32 tiles, so each split Z fragment feeds
// four tiles).  The 12 right-operand fragments of a 16-k step (12 KB) are shared by the four waves:
// the work-group loads them once into a double-buffered LDS slot while the matrix cores run the
// previous step, and the next step's Z entries load meanwhile too.  VEC: n % 4 == 0, so 8
// consecutive entries of a row are two aligned float4.
struct Z8 {
  float v[8];
};

__device__ __forceinline__ uint4 zc4() { return make_uint4(0u, 0u, 0u, 0u); }

template <bool VEC>
__device__ __forceinline__ Z8 wy_zload(const float* __restrict__ zr, int64_t k, int64_t m) {
  Z8 z;
  if (VEC && k + 8 <= m) {
    const float4 p0 = *reinterpret_cast<const float4*>(zr + k);
    const float4 p1 = *reinterpret_cast<const float4*>(zr + k + 4);
    z.v[0] = p0.x; z.v[1] = p0.y; z.v[2] = p0.z; z.v[3] = p0.w;
    z.v[4] = p1.x; z.v[5] = p1.y; z.v[6] = p1.z; z.v[7] = p1.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) z.v[e] = k + e < m ? zr[k + e] : 0.f;
  }
  return z;
}

// chunk e = (tc * 3 + p) * 64 + l of the right operand of step s
__device__ __forceinline__ const uint4* wy_bsrc(const uint4* __restrict__ Yb1, int64_t KS1, int64_t s, int e) {
  const int tc = e / 192, p = (e / 64) % 3, l = e & 63;
  return Yb1 + ((tc * KS1 + s) * 3 + p) * 64 + l;
}

template <bool VEC, int NT>
__global__ __launch_bounds__(kThr) void wy_w_kernel(const float* __restrict__ Z, int64_t n, int64_t i0, int64_t m,
                                                    const uint4* __restrict__ Yb1, int64_t KS1, int64_t kps,
                                                    float* __restrict__ P) {
  constexpr int NF = NT * 3 * 64;  // right-operand chunks of a 16-k step
  __shared__ uint4 sB[2][NF];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, hh = lane >> 5;
  const int64_t R0 = (int64_t)blockIdx.x * 128 + 32 * wave;
  const int64_t row = R0 + (lane & 31);
  const bool rok = row < n;
  const float* __restrict__ zr = Z + (rok ? row : n - 1) * n + i0;
  const int64_t s0 = (int64_t)blockIdx.y * kps / 16, s1 = min(KS1, ((int64_t)blockIdx.y * kps + kps) / 16);
  floatx16 acc[NT];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[tc][v] = 0.f;
  if (s0 < s1) {
#pragma unroll
    for (int q = 0; q < NF / 256; ++q) sB[0][t + 256 * q] = *wy_bsrc(Yb1, KS1, s0, t + 256 * q);
    Z8 zc = wy_zload<VEC>(zr, 16 * s0 + 8 * hh, m);
    __syncthreads();
    for (int64_t s = s0; s < s1; ++s) {
      const int buf = (int)((s - s0) & 1);
      const bool more = s + 1 < s1;
      uint4 nb[NF / 256];
#pragma unroll
      for (int q = 0; q < NF / 256; ++q) nb[q] = zc4();
      Z8 zn = zc;
      if (more) {
#pragma unroll
        for (int q = 0; q < NF / 256; ++q) nb[q] = *wy_bsrc(Yb1, KS1, s + 1, t + 256 * q);
        zn = wy_zload<VEC>(zr, 16 * (s + 1) + 8 * hh, m);
      }
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = rok ? zc.v[e] : 0.f;
      uint4 ph, pm, pl;
      split3(v[0], v[1], ph.x, pm.x, pl.x);
      split3(v[2], v[3], ph.y, pm.y, pl.y);
      split3(v[4], v[5], ph.z, pm.z, pl.z);
      split3(v[6], v[7], ph.w, pm.w, pl.w);
      const bf16x8 a0 = __builtin_bit_cast(bf16x8, ph), a1 = __builtin_bit_cast(bf16x8, pm),
                   a2 = __builtin_bit_cast(bf16x8, pl);
      const uint4* sb = sB[buf] + lane;
#pragma unroll
      for (int tc = 0; tc < NT; ++tc) {
        const bf16x8 b0 = __builtin_bit_cast(bf16x8, sb[(tc * 3 + 0) * 64]);
        const bf16x8 b1 = __builtin_bit_cast(bf16x8, sb[(tc * 3 + 1) * 64]);
        const bf16x8 b2 = __builtin_bit_cast(bf16x8, sb[(tc * 3 + 2) * 64]);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[tc], 0, 0, 0);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[tc], 0, 0, 0);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[tc], 0, 0, 0);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b2, acc[tc], 0, 0, 0);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[tc], 0, 0, 0);
        acc[tc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b0, acc[tc], 0, 0, 0);
      }
      if (more) {
#pragma unroll
        for (int q = 0; q < NF / 256; ++q) sB[buf ^ 1][t + 256 * q] = nb[q];
        zc = zn;
      }
      __syncthreads();  // uniform: s, s1 are the same for the whole work-group
    }
  }
  float* Ps = P + (int64_t)blockIdx.y * n * (32 * NT);
#pragma unroll
  for (int tc = 0; tc < NT; ++tc)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t r = R0 + 8 * (v >> 2) + 4 * hh + (v & 3);
      if (r < n) Ps[r * (32 * NT) + 32 * tc + (lane & 31)] = acc[tc][v];
    }
}

// W2 = the sum of the split partials (split order), stored as the planes of -W2 (the left operand
// of the update; rows past n are zero).  Thread: row 32 bx + t / 8, columns 16 (t % 8) .. + 15.
__global__ __launch_bounds__(kThr) void wy_w2_kernel(const float* __restrict__ P, int splits, int64_t n,
                                                     uint4* __restrict__ Wp, int ks, int soff, int pw, int pc0) {
  const int t = threadIdx.x;
  const int r = t >> 3, q = t & 7;
  const int64_t row = (int64_t)blockIdx.x * 32 + r;
  float o[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) o[j] = 0.f;
  if (row < n) {
    for (int sp = 0; sp < splits; ++sp) {
      const float4* src = reinterpret_cast<const float4*>(P + ((int64_t)sp * n + row) * pw + pc0 + 16 * q);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 f = src[j];
        o[4 * j] += f.x;
        o[4 * j + 1] += f.y;
        o[4 * j + 2] += f.z;
        o[4 * j + 3] += f.w;
      }
    }
  }
  uint4* dst = Wp + (((int64_t)blockIdx.x * ks + soff + q) * 3) * 64 + r;
  put3(dst, o, -1.f);
  put3(dst + 32, o + 8, -1.f);
}

// Z[r][i0 + c] += sum_k (-W2)[r][k] Y[c][k] on the 128 x 128 tile (ti, tj) (rows r < n, columns
// c < m); wave (wr, wc) owns a 64 x 64 quarter, loaded into the accumulators, K = 16 KSU (one or two
// blocks of kWyNB reflectors) in KSU 16-k steps of six plane products.  The 24 fragments of a step (4 row tiles and 4 column tiles x
// 3 planes, 24 KB) are loaded once per work-group into a double-buffered LDS slot.
template <int KSU>
__global__ __launch_bounds__(kThr, 2) void wy_upd_kernel(const uint4* __restrict__ Wp, const uint4* __restrict__ Yb3,
                                                      float* __restrict__ Z, int64_t n, int64_t i0, int64_t m,
                                                      int64_t tiles_m) {
  __shared__ uint4 sF[2][24 * 64];  // [buf][(side * 4 + tile) * 3 + plane][lane], side 0: rows, 1: columns
  const int64_t ti = blockIdx.x / tiles_m, tj = blockIdx.x - ti * tiles_m;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t R0 = 128 * ti + 64 * wr, C0 = 128 * tj + 64 * wc;
  const int col = lane & 31, rq = 4 * (lane >> 5);
  float* __restrict__ zb = Z + i0;  // entry (r, c) at zb[r * n + c]: 32-bit offsets (n^2 < 2^31)
  const int nn = (int)n;
  // thread t moves chunks e = t + 256 q (q < 6) of a step: q < 3 from the row side, q >= 3 from the
  // column side (chunk f = e / 64 = side * 12 + tile * 3 + plane)
  const uint4* srow = Wp + (4 * ti) * (KSU * 3 * 64);
  const uint4* scol = Yb3 + (4 * tj) * (KSU * 3 * 64);
  int foff[6];
#pragma unroll
  for (int q = 0; q < 6; ++q) {
    const int e = t + 256 * q, f = (e >> 6) % 12, l = e & 63;
    foff[q] = (f / 3) * (KSU * 3 * 64) + (f % 3) * 64 + l;
  }
#pragma unroll
  for (int q = 0; q < 6; ++q) sF[0][t + 256 * q] = (q < 3 ? srow : scol)[foff[q]];
  floatx16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int c = (int)(C0 + 32 * y) + col;
      const int rb = (int)(R0 + 32 * x) + rq;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = rb + 8 * (v >> 2) + (v & 3);
        acc[x][y][v] = (r < nn && c < m) ? zb[r * nn + c] : 0.f;
      }
    }
  __syncthreads();
  for (int ks = 0; ks < KSU; ++ks) {
    const int buf = ks & 1;
    uint4 nf[6];
    if (ks + 1 < KSU) {
#pragma unroll
      for (int q = 0; q < 6; ++q) nf[q] = (q < 3 ? srow : scol)[foff[q] + (ks + 1) * 3 * 64];
    }
    bf16x8 av[2][3], bv[2][3];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        av[x][p] = __builtin_bit_cast(bf16x8, sF[buf][((2 * wr + x) * 3 + p) * 64 + lane]);
        bv[x][p] = __builtin_bit_cast(bf16x8, sF[buf][((4 + 2 * wc + x) * 3 + p) * 64 + lane]);
      }
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][0], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][1], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][1], bv[y][0], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][0], bv[y][2], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][1], bv[y][1], acc[x][y], 0, 0, 0);
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[x][2], bv[y][0], acc[x][y], 0, 0, 0);
      }
    if (ks + 1 < KSU) {
#pragma unroll
      for (int q = 0; q < 6; ++q) sF[buf ^ 1][t + 256 * q] = nf[q];
    }
    __syncthreads();
  }
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int c = (int)(C0 + 32 * y) + col;
      const int rb = (int)(R0 + 32 * x) + rq;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = rb + 8 * (v >> 2) + (v & 3);
        if (r < nn && c < m) zb[r * nn + c] = acc[x][y][v];
      }
    }
}

// out (cols x rows, leading dimension rows) = in^T for in (rows x cols, leading dimension cols),
// 32 x 32 tiles through LDS
__global__ __launch_bounds__(kThr) void wy_transpose_kernel(const float* __restrict__ in, int64_t rows, int cols,
                                                            float* __restrict__ out) {
  __shared__ float tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * 32;
  const int c0 = blockIdx.y * 32;
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k;
    tile[k][tx] = (r < rows && c0 + tx < cols) ? in[r * cols + c0 + tx] : 0.f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int c = c0 + k;
    const int64_t r = r0 + tx;
    if (c < cols && r < rows) out[(int64_t)c * rows + r] = tile[tx][k];
  }
}

inline int64_t a64f(int64_t v) { return (v + 63) / 64 * 64; }

}  // namespace

int64_t wy_x6_buffer_floats(int64_t n) { return (n + 127) / 128 * 128 * 384 + 256; }

int wy_apply_x6(int64_t n, int64_t nrefl, const float* Tb, float* Z, float* Y, float* Yt, float* Y2, float* Yt2,
                float* P, int p_splits, float* scratch, int64_t scratch_floats, void* Yb1v, void* Yb3v, void* Wpv,
                const WyExtractY& extract, hipStream_t stream) {
  uint4* Yb1 = static_cast<uint4*>(Yb1v);
  uint4* Yb3 = static_cast<uint4*>(Yb3v);
  uint4* Wp = static_cast<uint4*>(Wpv);
  const int64_t nblocks = nrefl > 0 ? (nrefl + kWyNB - 1) / kWyNB : 0;
  const int64_t rows_wg = (n + 127) / 128;
  auto pack = [&](const float* Yr, const float* Ytr, int nb, int64_t m, int64_t mpad, int ks, int soff,
                  int tc0) -> int {
    const int64_t items = (Yr ? mpad * 16 : 0) + (Ytr ? mpad / 8 * kWyNB : 0);
    const int64_t g = std::min<int64_t>((items + kThr - 1) / kThr, 16384);
    hipLaunchKernelGGL(wy_pack_y_kernel, dim3((unsigned)g), dim3(kThr), 0, stream, Yr, Ytr, nb, m, mpad, Yb1, Yb3,
                       ks, soff, tc0);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  // P (S splits x n x 32 NT) = Z[:, i0:] times the NT column tiles packed in Yb1
  auto w_prod = [&](int NT, int64_t i0, int64_t m, int64_t mpad, int64_t smax) -> int64_t {
    const int64_t KS1 = mpad / 16;
    // split K so that about 1024 work-groups run, each slice a multiple of 64
    int64_t S = std::max<int64_t>(1, std::min<int64_t>({smax, mpad / 64, (1024 + rows_wg - 1) / rows_wg}));
    const int64_t kps = (mpad / S + 63) / 64 * 64;
    S = (mpad + kps - 1) / kps;
    const dim3 grid((unsigned)rows_wg, (unsigned)S);
    if (NT == 8) {
      if ((n & 3) == 0)
        hipLaunchKernelGGL((wy_w_kernel<true, 8>), grid, dim3(kThr), 0, stream, Z, n, i0, m, Yb1, KS1, kps, P);
      else
        hipLaunchKernelGGL((wy_w_kernel<false, 8>), grid, dim3(kThr), 0, stream, Z, n, i0, m, Yb1, KS1, kps, P);
    } else {
      if ((n & 3) == 0)
        hipLaunchKernelGGL((wy_w_kernel<true, 4>), grid, dim3(kThr), 0, stream, Z, n, i0, m, Yb1, KS1, kps, P);
      else
        hipLaunchKernelGGL((wy_w_kernel<false, 4>), grid, dim3(kThr), 0, stream, Z, n, i0, m, Yb1, KS1, kps, P);
    }
    return hipGetLastError() == hipSuccess ? S : -1;
  };
  // planes of -W (columns pc0 .. pc0 + 127 of the partials' pw) at the 16-k steps soff .. soff + 7 of ks
  auto w_planes = [&](int64_t S, int pw, int pc0, int ks, int soff) -> int {
    hipLaunchKernelGGL(wy_w2_kernel, dim3((unsigned)(rows_wg * 4)), dim3(kThr), 0, stream, P, (int)S, n, Wp, ks, soff,
                       pw, pc0);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  // the planes of -(Z[:, i0:] Ytr) (m x nb) at the 16-k steps soff .. soff + 7 of ks (Yb1 from Ytr)
  auto w_pass = [&](const float* Ytr, int nb, int64_t i0, int64_t m, int64_t mpad, int ks, int soff) -> int {
    int rc = pack(nullptr, Ytr, nb, m, mpad, ks, soff, 0);
    if (rc != kOk) return rc;
    const int64_t S = w_prod(4, i0, m, mpad, p_splits);
    if (S < 0) {
      set_error("wy_apply_x6: launch failed");
      return kHipError;
    }
    return w_planes(S, kWyNB, 0, ks, soff);
  };
  auto update = [&](int ks, int64_t i0, int64_t m, int64_t mpad) -> int {
    const int64_t tiles_m = mpad / 128;
    if (ks == 16)
      hipLaunchKernelGGL(wy_upd_kernel<16>, dim3((unsigned)(rows_wg * tiles_m)), dim3(kThr), 0, stream, Wp, Yb3, Z, n,
                         i0, m, tiles_m);
    else
      hipLaunchKernelGGL(wy_upd_kernel<8>, dim3((unsigned)(rows_wg * tiles_m)), dim3(kThr), 0, stream, Wp, Yb3, Z, n,
                         i0, m, tiles_m);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  int rc;
  int64_t b = nblocks - 1;
  while (b >= 0) {
    if (b >= 1) {
      // Blocks B = b and A = b - 1 in one update: with W_B = Z Yt_B and W_A' = Z Yt_A from the same Z,
      // applying B then A is Z - W_B Y_B^T - (W_A' - W_B C) Y_A^T, C = Y_B^T Yt_A, i.e.
      // Z - W_B (Y_B - Y_A C^T)^T - W_A' Y_A^T: one pass over Z with K = 2 kWyNB.
      const int64_t i0 = (b - 1) * kWyNB, i0B = b * kWyNB;
      const int nbA = kWyNB;
      const int nbB = (int)std::min<int64_t>(kWyNB, nrefl - i0B);
      const int64_t m = n - i0;
      const int64_t mpad = (m + 127) / 128 * 128;
      if (scratch_floats < (int64_t)nbB * nbA + 64 || a64f(n * kWyNB) * p_splits < (int64_t)nbB * m) {
        set_error("wy_apply_x6: scratch too small");
        return kInvalidArgument;
      }
      if ((rc = extract(i0, nbA, Y)) != kOk) return rc;
      MPQ_HIP_TRY(gemm(Y, nbA, Tb + (b - 1) * kWyNB * kWyNB, nbA, true, nullptr, Yt, nbA, m, nbA, nbA, 1.f, 0.f,
                       nullptr, 0, stream));
      // Y_B as m x nbB with its first kWyNB rows zero (its reflectors start kWyNB columns later)
      MPQ_HIP_TRY(hipMemsetAsync(Y2, 0, (size_t)kWyNB * nbB * sizeof(float), stream));
      if ((rc = extract(i0B, nbB, Y2 + (int64_t)kWyNB * nbB)) != kOk) return rc;
      MPQ_HIP_TRY(gemm(Y2, nbB, Tb + b * kWyNB * kWyNB, nbB, true, nullptr, Yt2, nbB, m, nbB, nbB, 1.f, 0.f, nullptr,
                       0, stream));
      if (p_splits >= 2) {
        // W_B and W_A' from one read of Z: the 8 column tiles of [Yt_B Yt_A]
        if ((rc = pack(nullptr, Yt2, nbB, m, mpad, 16, 0, 0)) != kOk) return rc;
        if ((rc = pack(nullptr, Yt, nbA, m, mpad, 16, 0, 4)) != kOk) return rc;
        const int64_t S = w_prod(8, i0, m, mpad, p_splits / 2);
        if (S < 0) {
          set_error("wy_apply_x6: launch failed");
          return kHipError;
        }
        if ((rc = w_planes(S, 2 * kWyNB, 0, 16, 0)) != kOk) return rc;
        if ((rc = w_planes(S, 2 * kWyNB, kWyNB, 16, 8)) != kOk) return rc;
      } else {
        if ((rc = w_pass(Yt2, nbB, i0, m, mpad, 16, 0)) != kOk) return rc;
        if ((rc = w_pass(Yt, nbA, i0, m, mpad, 16, 8)) != kOk) return rc;
      }
      // C (nbB x nbA, in scratch) = Y_B^T Yt_A through Y_B^T in P (free again); Y_B -= Y_A C^T
      hipLaunchKernelGGL(wy_transpose_kernel, dim3((unsigned)((m + 31) / 32), (unsigned)((nbB + 31) / 32)),
                         dim3(kThr), 0, stream, Y2, m, nbB, P);
      MPQ_LAUNCH_CHECK();
      float* C = scratch;
      float* gws = scratch + ((int64_t)nbB * nbA + 63) / 64 * 64;
      const int64_t gws_floats = scratch_floats - (gws - scratch);
      MPQ_HIP_TRY(gemm(P, m, Yt, nbA, false, nullptr, C, nbA, nbB, nbA, m, 1.f, 0.f, gws, gws_floats, stream));
      MPQ_HIP_TRY(gemm(Y, nbA, C, nbA, true, nullptr, Y2, nbB, m, nbB, nbA, -1.f, 1.f, gws, gws_floats, stream));
      if ((rc = pack(Y2, nullptr, nbB, m, mpad, 16, 0, 0)) != kOk) return rc;
      if ((rc = pack(Y, nullptr, nbA, m, mpad, 16, 8, 0)) != kOk) return rc;
      if ((rc = update(16, i0, m, mpad)) != kOk) return rc;
      b -= 2;
    } else {
      const int64_t i0 = b * kWyNB;
      const int nb = (int)std::min<int64_t>(kWyNB, nrefl - i0);
      const int64_t m = n - i0;
      const int64_t mpad = (m + 127) / 128 * 128;
      if ((rc = extract(i0, nb, Y)) != kOk) return rc;
      // Yt = Y Tb^T (m x nb)
      MPQ_HIP_TRY(gemm(Y, nb, Tb + b * kWyNB * kWyNB, nb, true, nullptr, Yt, nb, m, nb, nb, 1.f, 0.f, nullptr, 0,
                       stream));
      if ((rc = pack(Y, nullptr, nb, m, mpad, 8, 0, 0)) != kOk) return rc;
      if ((rc = w_pass(Yt, nb, i0, m, mpad, 8, 0)) != kOk) return rc;
      if ((rc = update(8, i0, m, mpad)) != kOk) return rc;
      b -= 1;
    }
  }
  return kOk;
}

}  // namespace mpq
