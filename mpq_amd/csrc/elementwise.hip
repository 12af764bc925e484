// Element-wise and data-movement kernels of the per-layer driver (gfx950).
//
//   mpq_gptq_find_params   GPTQ asymmetric min-max group parameters (GPTQModel
//                          Quantizer.find_params as called at
//                          mpq/adapters/gptqmodel.py:899-909)
//   mpq_uniform_rtn        RTN decision q = clamp(round(W/s) + z), x = s(q - z)
//                          (mpq/adapters/gptqmodel.py:966-969)
//   mpq_dequant            x = s(q - z)              (mpq/priors/uniform.py:302-309)
//   mpq_block_hadamard     signed block Walsh-Hadamard along rows
//                          (mpq/rotation.py:135-156, :404-438)
//   mpq_transpose          out = in^T (tiled through LDS)
//   mpq_scale_columns      out = in * scale[col]   (Vs = V * S, mpq/adapters/gptqmodel.py:890)
//   mpq_eigh_postprocess   eigenvalue floor, descending order, S = sqrt(lambda),
//                          Vs = V * S   (mpq/adapters/gptqmodel.py:302-310, :887-890)
//   argsort_desc_rows      stable descending argsort for the greedy CD order
//                          (mpq/polish/triton_scalar_cd.py:242-243)
// All HBM-bound; each is one pass over its operands.
#include "kernels.h"

namespace mpq {
namespace {

__global__ void dequant_kernel(const uint8_t* __restrict__ q, const float* __restrict__ scale,
                               const float* __restrict__ zero, int64_t G, int64_t gs, int64_t rows,
                               int64_t n, float* __restrict__ x) {
  const int64_t total = rows * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / n, j = e % n;
    const int64_t g = b * G + j / gs;
    x[e] = scale[g] * ((float)q[e] - zero[g]);
  }
}

__global__ void rtn_kernel(const float* __restrict__ W, int64_t ldw, const float* __restrict__ scale,
                           const float* __restrict__ zero, int64_t G, int64_t gs, int64_t rows,
                           int64_t n, int maxq, uint8_t* __restrict__ q, float* __restrict__ x) {
  const int64_t total = rows * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / n, j = e % n;
    const int64_t g = b * G + j / gs;
    const float s = scale[g], z = zero[g];
    float qf = rintf(W[b * ldw + j] / s) + z;
    qf = qf < 0.f ? 0.f : (qf > (float)maxq ? (float)maxq : qf);
    if (q) q[e] = (uint8_t)(int)qf;
    if (x) x[e] = s * (qf - z);
  }
}

// One work-group per (row, group): min/max over the group's columns.
__global__ __launch_bounds__(256) void find_params_kernel(const float* __restrict__ W, int64_t ldw,
                                                          int64_t n, int64_t gs, int64_t G, int maxq,
                                                          float* __restrict__ scale,
                                                          float* __restrict__ zero) {
  __shared__ float smin[4], smax[4];
  const int64_t b = blockIdx.y, g = blockIdx.x;
  const int64_t j0 = g * gs;
  int64_t j1 = j0 + gs;
  if (j1 > n) j1 = n;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t j = j0 + threadIdx.x; j < j1; j += blockDim.x) {
    const float v = W[b * ldw + j];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, off, 64));
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    smin[wave] = mn;
    smax[wave] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
      mn = fminf(mn, smin[w]);
      mx = fmaxf(mx, smax[w]);
    }
    mn = fminf(smin[0], mn);
    mx = fmaxf(smax[0], mx);
    float xmin = fminf(mn, 0.f), xmax = fmaxf(mx, 0.f);
    if (xmin == 0.f && xmax == 0.f) {
      xmin = -1.f;
      xmax = 1.f;
    }
    const float s = (xmax - xmin) / (float)maxq;
    scale[b * G + g] = s;
    zero[b * G + g] = rintf(-xmin / s);
  }
}

// Block Walsh-Hadamard (Sylvester order) of each `had`-long segment of each row,
// butterfly strides 1, 2, 4, ... exactly as mpq/rotation.py:135-156, then divided
// by sqrt(had).  forward: x*signs first; inverse: signs applied after.
__global__ __launch_bounds__(256) void block_hadamard_kernel(const float* __restrict__ in,
                                                             int64_t ld_in, float* __restrict__ out,
                                                             int64_t ld_out, int64_t width, int had,
                                                             const float* __restrict__ signs,
                                                             int inverse) {
  extern __shared__ float buf[];
  const int64_t row = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * had;
  const float* src = in + row * ld_in + c0;
  for (int i = threadIdx.x; i < had; i += blockDim.x) {
    float v = src[i];
    if (signs && !inverse) v = v * signs[c0 + i];
    buf[i] = v;
  }
  __syncthreads();
  for (int h = 1; h < had; h <<= 1) {
    for (int p = threadIdx.x; p < had / 2; p += blockDim.x) {
      const int blk = p / h, off = p % h;
      const int i0 = blk * 2 * h + off;
      const float a = buf[i0], b = buf[i0 + h];
      buf[i0] = a + b;
      buf[i0 + h] = a - b;
    }
    __syncthreads();
  }
  const float rs = sqrtf((float)had);
  float* dst = out + row * ld_out + c0;
  for (int i = threadIdx.x; i < had; i += blockDim.x) {
    float v = buf[i] / rs;
    if (signs && inverse) v = v * signs[c0 + i];
    dst[i] = v;
  }
}

__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ in, int64_t rows,
                                                        int64_t cols, int64_t ld_in,
                                                        float* __restrict__ out, int64_t ld_out) {
  __shared__ float tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = in[r * ld_in + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) out[c * ld_out + r] = tile[tx][k];
  }
}

// lam_asc (n, ascending) / V_asc (n x n, columns) -> descending, floored.
__global__ void eigh_post_kernel(const float* __restrict__ lam_asc, const float* __restrict__ V_asc,
                                 int64_t n, float floor_v, float* __restrict__ lam,
                                 float* __restrict__ S, float* __restrict__ V,
                                 float* __restrict__ Vs) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / n, j = e % n;
    float l = lam_asc[n - 1 - j];
    l = l < floor_v ? floor_v : l;
    const float s = sqrtf(l);
    const float v = V_asc[i * n + (n - 1 - j)];
    if (V) V[e] = v;
    if (Vs) Vs[e] = v * s;
    if (i == 0) {
      if (lam) lam[j] = l;
      if (S) S[j] = s;
    }
  }
}

__global__ void scale_columns_kernel(const float* __restrict__ in, int64_t rows, int64_t cols,
                                     const float* __restrict__ scale, float* __restrict__ out) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = in[e] * scale[e % cols];
}

__global__ __launch_bounds__(256) void row_sqnorm_kernel(const float* __restrict__ M, int64_t n,
                                                         int64_t ld, float floor_v,
                                                         float* __restrict__ out) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  float acc = 0.f;
  for (int64_t k = threadIdx.x; k < n; k += blockDim.x) {
    const float v = M[r * ld + k];
    acc += v * v;
  }
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) out[r] = t < floor_v ? floor_v : t;
}

// Bitonic sort of one key row in LDS: descending key, ascending index on ties.
__global__ __launch_bounds__(1024) void argsort_desc_kernel(const float* __restrict__ keys, int64_t n,
                                                            int npow2, int32_t* __restrict__ order) {
  extern __shared__ unsigned char smem[];
  float* k = reinterpret_cast<float*>(smem);
  int* id = reinterpret_cast<int*>(smem + sizeof(float) * npow2);
  const int64_t row = blockIdx.x;
  for (int i = threadIdx.x; i < npow2; i += blockDim.x) {
    if (i < n) {
      k[i] = keys[row * n + i];
      id[i] = i;
    } else {
      k[i] = -INFINITY;
      id[i] = 0x7fffffff;
    }
  }
  __syncthreads();
  for (int size = 2; size <= npow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < npow2 / 2; t += blockDim.x) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool up = (i & size) == 0;  // this block sorts "before-first"
        const float ki = k[i], kj = k[j];
        const int ii = id[i], ij = id[j];
        // "j before i" in the target order
        const bool j_first = (kj > ki) || (kj == ki && ij < ii) || (isnan(kj) && !isnan(ki));
        if (j_first == up) {
          k[i] = kj; k[j] = ki;
          id[i] = ij; id[j] = ii;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) order[row * n + i] = id[i];
}

inline unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  if (b > 16384) b = 16384;
  if (b < 1) b = 1;
  return (unsigned)b;
}

}  // namespace

hipError_t dequant_groups(const uint8_t* q, const float* scale, const float* zero, int64_t G,
                          int64_t gs, int64_t rows, int64_t n, float* x, hipStream_t stream) {
  hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(rows * n)), dim3(256), 0, stream, q, scale, zero, G,
                     gs, rows, n, x);
  return hipGetLastError();
}

hipError_t argsort_desc_rows(const float* keys, int64_t nrows, int64_t n, int32_t* order,
                             hipStream_t stream) {
  int npow2 = 1;
  while (npow2 < n) npow2 <<= 1;
  if (npow2 < 2) npow2 = 2;
  const size_t smem = (size_t)npow2 * (sizeof(float) + sizeof(int));
  hipLaunchKernelGGL(argsort_desc_kernel, dim3((unsigned)nrows), dim3(1024), smem, stream, keys, n,
                     npow2, order);
  return hipGetLastError();
}

hipError_t transpose_matrix(const float* in, int64_t rows, int64_t cols, int64_t ld_in, float* out,
                            int64_t ld_out, hipStream_t stream) {
  hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32)),
                     dim3(256), 0, stream, in, rows, cols, ld_in, out, ld_out);
  return hipGetLastError();
}

hipError_t row_sqnorm(const float* M, int64_t n, int64_t ld, float floor_v, float* out,
                      hipStream_t stream) {
  hipLaunchKernelGGL(row_sqnorm_kernel, dim3((unsigned)n), dim3(256), 0, stream, M, n, ld, floor_v, out);
  return hipGetLastError();
}

}  // namespace mpq

using namespace mpq;

extern "C" int mpq_gptq_find_params(const float* W, int64_t rows, int64_t n, int64_t ldw,
                                    int64_t group_size, int maxq, float* scale, float* zero,
                                    hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n >= 0 && group_size >= 1 && maxq >= 1, "mpq_gptq_find_params: bad shape");
  if (rows == 0 || n == 0) return kOk;
  MPQ_CHECK_ARG(W && scale && zero && ldw >= n, "mpq_gptq_find_params: bad pointer/ld");
  MPQ_CHECK_ARG(rows <= 65535, "mpq_gptq_find_params: at most 65535 rows per call");
  const int64_t G = (n + group_size - 1) / group_size;
  hipLaunchKernelGGL(find_params_kernel, dim3((unsigned)G, (unsigned)rows), dim3(256), 0, stream, W, ldw,
                     n, group_size, G, maxq, scale, zero);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_uniform_rtn(const float* W, int64_t rows, int64_t n, int64_t ldw,
                               const float* scale, const float* zero, int64_t group_size, int maxq,
                               uint8_t* q, float* x, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n >= 0 && group_size >= 1 && maxq >= 1 && maxq <= 255,
                "mpq_uniform_rtn: bad shape");
  if (rows == 0 || n == 0) return kOk;
  MPQ_CHECK_ARG(W && scale && zero && (q || x) && ldw >= n, "mpq_uniform_rtn: bad pointer/ld");
  const int64_t G = (n + group_size - 1) / group_size;
  hipLaunchKernelGGL(rtn_kernel, dim3(grid_for(rows * n)), dim3(256), 0, stream, W, ldw, scale, zero, G,
                     group_size, rows, n, maxq, q, x);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_dequant(const uint8_t* q, int64_t rows, int64_t n, const float* scale,
                           const float* zero, int64_t group_size, float* x, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n >= 0 && group_size >= 1, "mpq_dequant: bad shape");
  if (rows == 0 || n == 0) return kOk;
  MPQ_CHECK_ARG(q && scale && zero && x, "mpq_dequant: null pointer");
  const int64_t G = (n + group_size - 1) / group_size;
  MPQ_HIP_TRY(dequant_groups(q, scale, zero, G, group_size, rows, n, x, stream));
  return kOk;
}

extern "C" int mpq_block_hadamard(const float* in, int64_t ld_in, float* out, int64_t ld_out,
                                  int64_t rows, int64_t width, int64_t had_dim, const float* signs,
                                  int inverse, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && width >= 0, "mpq_block_hadamard: bad shape");
  if (rows == 0 || width == 0) return kOk;
  MPQ_CHECK_ARG(had_dim >= 1 && (had_dim & (had_dim - 1)) == 0 && had_dim <= 32768,
                "block Hadamard requires power-of-two had_dim <= 32768, got %lld", (long long)had_dim);
  MPQ_CHECK_ARG(width % had_dim == 0,
                "block Hadamard requires width divisible by had_dim; got width=%lld, had_dim=%lld",
                (long long)width, (long long)had_dim);
  MPQ_CHECK_ARG(in && out && ld_in >= width && ld_out >= width, "mpq_block_hadamard: bad pointer/ld");
  MPQ_CHECK_ARG(rows <= 65535, "mpq_block_hadamard: at most 65535 rows per call");
  hipLaunchKernelGGL(block_hadamard_kernel, dim3((unsigned)(width / had_dim), (unsigned)rows), dim3(256),
                     had_dim * sizeof(float), stream, in, ld_in, out, ld_out, width, (int)had_dim, signs,
                     inverse);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_transpose(const float* in, int64_t rows, int64_t cols, int64_t ld_in, float* out,
                             int64_t ld_out, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && cols >= 0, "mpq_transpose: bad shape");
  if (rows == 0 || cols == 0) return kOk;
  MPQ_CHECK_ARG(in && out && in != out && ld_in >= cols && ld_out >= rows, "mpq_transpose: bad pointer/ld");
  MPQ_CHECK_ARG((rows + 31) / 32 <= 65535, "mpq_transpose: too many rows");
  MPQ_HIP_TRY(transpose_matrix(in, rows, cols, ld_in, out, ld_out, stream));
  return kOk;
}

extern "C" int mpq_eigh_postprocess(const float* lam_asc, const float* V_asc, int64_t n, float floor_v,
                                    float* lam, float* S, float* V, float* Vs, hipStream_t stream) {
  MPQ_CHECK_ARG(n >= 0, "mpq_eigh_postprocess: bad shape");
  if (n == 0) return kOk;
  MPQ_CHECK_ARG(lam_asc && V_asc, "mpq_eigh_postprocess: null input");
  MPQ_CHECK_ARG(V != V_asc && Vs != V_asc, "mpq_eigh_postprocess: output must not alias V_asc");
  hipLaunchKernelGGL(eigh_post_kernel, dim3(grid_for(n * n)), dim3(256), 0, stream, lam_asc, V_asc, n,
                     floor_v, lam, S, V, Vs);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

extern "C" int mpq_scale_columns(const float* in, int64_t rows, int64_t cols, const float* scale, float* out,
                                 hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && cols >= 0, "mpq_scale_columns: bad shape");
  if (rows == 0 || cols == 0) return kOk;
  MPQ_CHECK_ARG(in && scale && out, "mpq_scale_columns: null pointer");
  hipLaunchKernelGGL(scale_columns_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, stream, in, rows, cols, scale,
                     out);
  MPQ_LAUNCH_CHECK();
  return kOk;
}

// ---- column permutations (activation order, mpq/adapters/gptqmodel.py:733-740, :1090-1095) ------

namespace {

template <typename T>
__global__ void permute_cols_kernel(const T* __restrict__ in, int64_t rows, int64_t cols,
                                    const int32_t* __restrict__ perm, T* __restrict__ out) {
  const int64_t total = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / cols, c = e - r * cols;
    out[e] = in[r * cols + perm[c]];
  }
}

__global__ void permute_sym_kernel(const float* __restrict__ in, int64_t n, const int32_t* __restrict__ perm,
                                   float* __restrict__ out) {
  const int64_t total = n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / n, j = e - i * n;
    out[e] = in[(int64_t)perm[i] * n + perm[j]];
  }
}

}  // namespace

// out[:, c] = in[:, perm[c]] for a rows x cols row-major matrix of 1- or 4-byte elements.
extern "C" int mpq_permute_columns(const void* in, int64_t rows, int64_t cols, const int32_t* perm, void* out,
                                   int elem_bytes, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && cols >= 0 && (elem_bytes == 1 || elem_bytes == 4), "mpq_permute_columns: bad shape");
  if (rows == 0 || cols == 0) return kOk;
  MPQ_CHECK_ARG(in && perm && out && in != out, "mpq_permute_columns: null or aliased pointer");
  if (elem_bytes == 4)
    hipLaunchKernelGGL(permute_cols_kernel<float>, dim3(grid_for(rows * cols)), dim3(256), 0, stream,
                       static_cast<const float*>(in), rows, cols, perm, static_cast<float*>(out));
  else
    hipLaunchKernelGGL(permute_cols_kernel<uint8_t>, dim3(grid_for(rows * cols)), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(in), rows, cols, perm, static_cast<uint8_t*>(out));
  MPQ_LAUNCH_CHECK();
  return kOk;
}

// out[i][j] = in[perm[i]][perm[j]] (n x n).
extern "C" int mpq_permute_symmetric(const float* in, int64_t n, const int32_t* perm, float* out,
                                     hipStream_t stream) {
  MPQ_CHECK_ARG(n >= 0, "mpq_permute_symmetric: bad shape");
  if (n == 0) return kOk;
  MPQ_CHECK_ARG(in && perm && out && in != out, "mpq_permute_symmetric: null or aliased pointer");
  hipLaunchKernelGGL(permute_sym_kernel, dim3(grid_for(n * n)), dim3(256), 0, stream, in, n, perm, out);
  MPQ_LAUNCH_CHECK();
  return kOk;
}
