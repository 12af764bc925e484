// E8P12 gram-metric block coordinate descent (gfx950).
//
// Replaces mpq/solver.py:369-423 (polish_e8p12_rankspace, mode "block_cd", metric
// "gram") -> mpq/polish/block_cd.py:332-625 (block_coordinate_descent_rankspace)
// with its compiled step _cd_gram_step_impl (:212-246), the greedy order of
// _batched_greedy_gain (:286-306) and stabilize_cholesky (mpq/linear.py:121-141).
//
// Semantics per row block (block_rows rows sharing one greedy order):
//   residual_u = Yu - x Vs, res = |residual_u|^2, rhs = residual_u Vs^T
//   per 8-column block j: G_j = Vs_j Vs_j^T (= H[8j.., 8j..], H = Vs Vs^T),
//     L_j = stabilized Cholesky of G_j, Gi_j = (L_j L_j^T)^-1
//   per sweep: gain_j = mean_rows(rhs_j Gi_j rhs_j^T), order = argsort(-gain)[:max_blocks]
//   per block j in order: target = x_j + rhs_j Gi_j,
//     c* = argmin_c |L_j^T (target - c)|^2 over all 65536 codewords (first index),
//     d = c* - x_j, ce = max(res + d G_j d^T - 2 rhs_j . d, 0),
//     accept iff ce + 1e-12 < res (1 + tol): x_j = c*, idx_j = c*, res = ce,
//     rhs -= d H[8j:8j+8, :]
//
// Kernels:
//   * step kernel (one launch per greedy step, all rows): grid = 32-row tiles x
//     codeword chunks.  The argmin is |L^T c|^2 - 2 (L L^T target) . c, a K = 8
//     product of the codewords with the rows' (-2 L L^T target) vectors on
//     v_mfma_f32_32x32x2_f32 (codewords on the MFMA's M side, rows on N), with the
//     per-block table |L^T c|^2 staged in LDS as the accumulator input.  Codewords
//     are generated in registers from the lattice structure (abs pattern k = idx>>8,
//     sign byte, parity-selected +-1/4 shift), never read from memory.  Each chunk
//     writes a (score, index) partial; the next launch reduces the partials
//     (earlier chunk wins ties), applies the accept test and records the delta.
//   * deferred rhs update: within a window of 16 greedy steps each step's rhs is
//     the window-start rhs minus the window's earlier deltas times 8x8 blocks of H;
//     after the window, rhs -= Delta (rows x 128) H[window rows, :] is one fp32
//     MFMA GEMM with a per-row-block row gather.
// Every work-group of a row tile computes the previous step's decision and the
// current target redundantly (identical arithmetic); only chunk 0 writes state.
// Buffers read and written by different work-groups of one launch (res, the
// step's x block and rhs) are double-buffered by step parity.
#include <algorithm>

#include "cd_common.h"
#include "e8p12_tables.inc"
#include "gemm.h"
#include "kernels.h"
#include "mpq_amd.h"
#include "x6_split.h"

namespace mpq {
namespace {

constexpr int kRT = 32;        // rows per tile
constexpr int kWS = 16;        // greedy steps per window
constexpr int kDS = 8 * kWS;   // delta row stride
constexpr int kNChunk = 16;    // codeword chunks per greedy step (work-groups per row tile)
constexpr int kCS = 65536 / kNChunk;  // codewords per chunk (LDS table of |L^T c|^2, 16 KB)
constexpr int kMeta = 192;     // G, L, Gi (8x8 each) per block
constexpr int kCodes = 65536;

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

__device__ __forceinline__ float sum8(float v) {
  // butterfly over the 8 lanes of a row group; bit-identical in all 8 lanes
  v = v + __shfl_xor(v, 1);
  v = v + __shfl_xor(v, 2);
  v = v + __shfl_xor(v, 4);
  return v;
}

// ---------------------------------------------------------------------------
// preparation (per layer): codebook grid, per-block G/L/Gi, |L^T c|^2 tables
// ---------------------------------------------------------------------------

// grid (65536 x 8) and the pattern table: the magnitudes a of abs pattern k (256 x 8), then the
// 256 pattern parities as int bits
__global__ __launch_bounds__(256) void grid_kernel(float* __restrict__ grid, float* __restrict__ pat) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int k = idx >> 8;
  const int s = idx & 255;
  const int branch = __builtin_popcount(s) & 1;
  const int signs = s ^ (((branch ^ (int)kE8Parity[k]) & 1) << 7);
  const float sh = branch ? -0.25f : 0.25f;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const float a = 0.5f * (float)kE8Abs2[k][d];
    grid[(int64_t)idx * 8 + d] = sh + (((signs >> d) & 1) ? -a : a);
    if (s == 0) pat[k * 8 + d] = a;
  }
  if (s == 0) pat[256 * 8 + k] = __int_as_float((int)kE8Parity[k]);
}

__device__ bool chol8(const float (&A)[8][8], float (&L)[8][8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float s = A[j][j];
    for (int k = 0; k < j; ++k) s = s - L[j][k] * L[j][k];
    // finiteness from the bits: this file is compiled without NaN semantics (-fno-honor-nans)
    if ((__float_as_uint(s) & 0x7f800000u) == 0x7f800000u || !(s > 0.f)) return false;
    const float d = sqrtf(s);
    L[j][j] = d;
    for (int i = j + 1; i < 8; ++i) {
      float t = A[i][j];
      for (int k = 0; k < j; ++k) t = t - L[i][k] * L[j][k];
      L[i][j] = t / d;
    }
    for (int i = 0; i < j; ++i) L[i][j] = 0.f;
  }
  return true;
}

__global__ void meta_kernel(int64_t n, int64_t nb, const float* __restrict__ H, float* __restrict__ meta,
                            int* __restrict__ fail) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= nb) return;
  float G[8][8], A[8][8], L[8][8];
  float dmax = 0.f;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      G[d][e] = H[(8 * j + d) * n + 8 * j + e];
      A[d][e] = G[d][e];
    }
    dmax = fmaxf(dmax, fabsf(G[d][d]));
  }
  // stabilize_cholesky: cumulative jitter 2^k * floor on the diagonal, 6 retries
  const float floor_v = dmax * 1e-6f + 1e-6f;
  bool ok = chol8(A, L);
  for (int k = 0; k < 6 && !ok; ++k) {
    const float add = ldexpf(floor_v, k);
#pragma unroll
    for (int d = 0; d < 8; ++d) A[d][d] = A[d][d] + add;
    ok = chol8(A, L);
  }
  if (!ok) {
    atomicAdd(fail, 1);
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int e = 0; e < 8; ++e) L[d][e] = d == e ? 1.f : 0.f;
  }
  // Gi = (L L^T)^-1 = Li^T Li with Li = L^-1 (forward substitution)
  float Li[8][8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t = (i == c) ? 1.f : 0.f;
      for (int k = c; k < i; ++k) t = t - L[i][k] * Li[k][c];
      Li[i][c] = i < c ? 0.f : t / L[i][i];
    }
  }
  float* m = meta + j * kMeta;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float gi = 0.f;
      for (int k = (d > e ? d : e); k < 8; ++k) gi = gi + Li[k][d] * Li[k][e];
      m[d * 8 + e] = G[d][e];
      m[64 + d * 8 + e] = L[d][e];
      m[128 + d * 8 + e] = gi;
    }
  }
}

// cgc[j][c] = |L_j^T c|^2 = sum_e (sum_d c_d L[d][e])^2 (mpq/polish/block_cd.py:228-230)
__global__ __launch_bounds__(256) void cgc_kernel(const float* __restrict__ grid, const float* __restrict__ meta,
                                                  float* __restrict__ cgc) {
  __shared__ float sL[64];
  const int64_t j = blockIdx.y;
  if (threadIdx.x < 64) sL[threadIdx.x] = meta[j * kMeta + 64 + threadIdx.x];
  __syncthreads();
  const int c = blockIdx.x * 256 + threadIdx.x;
  float cv[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) cv[d] = grid[(int64_t)c * 8 + d];
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float mg = cv[0] * sL[e];
#pragma unroll
    for (int d = 1; d < 8; ++d) mg = mg + cv[d] * sL[d * 8 + e];
    acc = e == 0 ? mg * mg : acc + mg * mg;
  }
  cgc[j * kCodes + c] = acc;
}

// ---------------------------------------------------------------------------
// per sweep: greedy gains and gather rows
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void e8_gain_kernel(int64_t rows, int64_t n, int64_t nb, int64_t block_rows,
                                                      const float* __restrict__ rhs, const float* __restrict__ meta,
                                                      float* __restrict__ gain) {
  const int64_t rb = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= nb) return;
  float Gi[64];
#pragma unroll
  for (int t = 0; t < 64; ++t) Gi[t] = meta[j * kMeta + 128 + t];
  const int64_t r0 = rb * block_rows;
  const int64_t r1 = std::min<int64_t>(r0 + block_rows, rows);
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    float v[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) v[d] = rhs[r * n + 8 * j + d];
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float w = v[0] * Gi[e];
#pragma unroll
      for (int d = 1; d < 8; ++d) w = w + v[d] * Gi[d * 8 + e];
      q = e == 0 ? v[e] * w : q + v[e] * w;
    }
    acc += q;
  }
  gain[rb * nb + j] = acc / (float)(r1 - r0);
}

__global__ void expand_rows_kernel(int64_t nrb, int64_t nb, const int32_t* __restrict__ order,
                                   int32_t* __restrict__ rowsidx) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nrb * nb * 8) return;
  const int64_t rb = t / (nb * 8);
  const int64_t o = t % (nb * 8);
  rowsidx[t] = 8 * order[rb * nb + o / 8] + (int32_t)(o % 8);
}

// ---------------------------------------------------------------------------
// the greedy step
// ---------------------------------------------------------------------------

struct StepArgs {
  int64_t rows, n, nb, block_rows;
  int tiles_per_rb;
  int nchunk;        // codeword chunks of this launch (gridDim.y when computing)
  int nparts;        // chunks of the previous launch (partials to reduce)
  int finalize;      // reduce and apply the decision of order position fin_t
  int fin_t, fin_slot, fin_par;
  int compute;       // run the argmin of order position t
  int t, p, w0, cur_par;
  float accept_tol;
  const int32_t* order;  // nrb x nb
  const float* meta;
  const float* cgc;      // nb x 65536
  const float* H;        // n x n
  const float* grid;     // 65536 x 8
  const float* pat;      // 256 x 8 abs-pattern magnitudes, then 256 parities (int bits)
  const float* rhs;      // rows x n, current at the window start
  float* x;              // rows x n
  int64_t* idx;          // rows x nb
  float* res;            // 2 x rows
  float* D;              // rows x kDS
  float* Rt;             // 2 x rows x 8: rhs of the step
  float* Xt;             // 2 x rows x 8: x block of the step before the decision
  float* ps;             // 2 x rows x 16 partial scores (by step parity)
  int32_t* pi;           // 2 x rows x 16 partial indices (by step parity)
  int32_t* accepted;     // rows
};

__global__ __launch_bounds__(256) void e8_cd_step_kernel(StepArgs a) {
  // s_cgc: the chunk's |L^T c|^2 for the argmin; before it, the same space holds s_D, the window's
  // deltas of the tile's rows (row r, step s, coordinate d at 8 kWS r + 8 s + d)
  __shared__ __align__(16) float s_cgc[kCS];
  static_assert(kCS >= kRT * 8 * kWS, "s_D does not fit in s_cgc");
  float* const s_D = s_cgc;
  __shared__ __align__(16) float s_abs[(kCS / 256) * 8];  // magnitudes of the chunk's kCS / 256 abs patterns
  __shared__ __align__(16) float s_H[kWS * 64];  // H[8 j_s + d][8 j + e] of the window's steps s, entry 64 s + 8 e + d
  __shared__ float s_M[128];       // block j's L (64) and Gi (64)
  __shared__ float s_u[kRT][8];
  __shared__ float s_bs[4][kRT];
  __shared__ int s_bi[4][kRT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r = tid >> 3;  // row within the tile
  const int e = tid & 7;   // coordinate
  const int gbase = lane & ~7;
  const int64_t rb = blockIdx.x / a.tiles_per_rb;
  const int64_t rloc = (int64_t)(blockIdx.x % a.tiles_per_rb) * kRT + r;
  const int64_t row_raw = rb * a.block_rows + rloc;
  const bool valid = rloc < a.block_rows && row_raw < a.rows;
  const int64_t row = valid ? row_raw : rb * a.block_rows;  // in-bounds stand-in for masked rows
  const bool writer = blockIdx.y == 0;
  const int32_t* ord = a.order + rb * a.nb;
  const int64_t rows = a.rows, n = a.n;

  // ---- loads.  Finalize: the previous step's decision needs, per row, the best of all chunks'
  // partials (in the buffer of that launch's parity: this launch's work-groups write the other one,
  // so a work-group that finishes early cannot overwrite what a later one still reads), the step's
  // x block and rhs, the residual norm and the block's gram G.  Compute: the chunk's |L^T c|^2,
  // block j's L and Gi, the window's H blocks and deltas, rhs and x of block j.  None of them reads
  // what this launch writes (block j is not the finalized block; D slots s < p - 1 were written by
  // earlier launches).  All of them are issued before the first use.
  static_assert(kCS / 4 / 256 == 4 && kWS * 64 / 256 == 4, "staging assumes 4 loads per thread");
  int jp = 0;
  float fx = 0.f, fr = 0.f, r0 = 0.f;
  float gm[8];
  float ps[16];
  int pi[16];
#pragma unroll
  for (int d = 0; d < 8; ++d) gm[d] = 0.f;
  if (a.finalize) {
    const float4* fps = reinterpret_cast<const float4*>(a.ps + (int64_t)a.fin_par * rows * 16 + row * 16);
    const int4* fpi = reinterpret_cast<const int4*>(a.pi + (int64_t)a.fin_par * rows * 16 + row * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = fps[q];
      const int4 w = fpi[q];
      ps[4 * q] = v.x; ps[4 * q + 1] = v.y; ps[4 * q + 2] = v.z; ps[4 * q + 3] = v.w;
      pi[4 * q] = w.x; pi[4 * q + 1] = w.y; pi[4 * q + 2] = w.z; pi[4 * q + 3] = w.w;
    }
    jp = ord[a.fin_t];
    const float* Gm = a.meta + (int64_t)jp * kMeta;
#pragma unroll
    for (int d = 0; d < 8; ++d) gm[d] = Gm[d * 8 + e];
    fx = a.Xt[(int64_t)a.fin_par * rows * 8 + row * 8 + e];
    fr = a.Rt[(int64_t)a.fin_par * rows * 8 + row * 8 + e];
    r0 = a.res[(int64_t)a.fin_par * rows + row];
  }
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  const int j = a.compute ? ord[a.t] : 0;
  const int c0 = blockIdx.y * kCS;
  // the magnitudes of the chunk's abs patterns (codewords are formed from their index)
  float4 ab0 = z4;
  if (tid < kCS / 256 * 2) ab0 = reinterpret_cast<const float4*>(a.pat)[c0 / 256 * 2 + tid];
  float4 cg0 = z4, cg1 = z4, cg2 = z4, cg3 = z4;
  float hv0 = 0.f, hv1 = 0.f, hv2 = 0.f, hv3 = 0.f;
  float dv[kWS - 1];
#pragma unroll
  for (int s = 0; s < kWS - 1; ++s) dv[s] = 0.f;
  float mv = 0.f, rh = 0.f, xb = 0.f;
  if (a.compute) {
    const float4* src = reinterpret_cast<const float4*>(a.cgc + (int64_t)j * kCodes + c0) + tid;
    cg0 = src[0];
    cg1 = src[256];
    cg2 = src[512];
    cg3 = src[768];
    // H block entry (s, d, e) = i = 64 s + 8 d + e, i = tid + 256 q; s = wave + 4 q is wave-uniform
    const int64_t hcol = 8 * (int64_t)j + (tid & 7);
    const int hd = (tid >> 3) & 7, hs = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t* wo = ord + a.w0 + hs;
    if (hs < a.p) hv0 = a.H[(8 * (int64_t)wo[0] + hd) * n + hcol];
    if (hs + 4 < a.p) hv1 = a.H[(8 * (int64_t)wo[4] + hd) * n + hcol];
    if (hs + 8 < a.p) hv2 = a.H[(8 * (int64_t)wo[8] + hd) * n + hcol];
    if (hs + 12 < a.p) hv3 = a.H[(8 * (int64_t)wo[12] + hd) * n + hcol];
    mv = tid < 128 ? a.meta[(int64_t)j * kMeta + 64 + tid] : 0.f;
#pragma unroll
    for (int s = 0; s < kWS - 1; ++s) dv[s] = s + 1 < a.p ? a.D[row * kDS + 8 * s + e] : 0.f;
    rh = a.rhs[row * n + 8 * (int64_t)j + e];
    xb = a.x[row * n + 8 * (int64_t)j + e];
  }

  // ---- the previous step's candidate per row (earlier chunk wins ties) and its pattern's magnitude
  // and parity, loaded here and used after the window's first part
  int bi = 0;
  float cav = 0.f;
  int cpar = 0;
  if (a.finalize) {
    float bs = ps[0];
    bi = pi[0];
#pragma unroll
    for (int c = 1; c < kNChunk; ++c) {
      if (ps[c] < bs) {
        bs = ps[c];
        bi = pi[c];
      }
    }
    cav = a.pat[8 * (bi >> 8) + e];
    cpar = __float_as_int(a.pat[2048 + (bi >> 8)]);
  }

  // ---- stage in LDS what the tile's rows share (and each row's window deltas s < p - 1)
  if (tid < kCS / 256 * 2) reinterpret_cast<float4*>(s_abs)[tid] = ab0;
  if (a.compute) {
    // H entry (s, d, e) of hv_q (i = tid + 256 q = 64 s + 8 d + e) goes to 64 s + 8 e + d
    const int ht = (tid & ~63) + 8 * (tid & 7) + ((tid >> 3) & 7);
    s_H[ht] = hv0;
    s_H[ht + 256] = hv1;
    s_H[ht + 512] = hv2;
    s_H[ht + 768] = hv3;
    if (tid < 128) s_M[tid] = mv;
    float* dr = s_D + 8 * kWS * r + e;
#pragma unroll
    for (int s = 0; s < kWS - 1; ++s)
      if (s + 1 < a.p) dr[8 * s] = dv[s];
  }
  __syncthreads();

  // ---- rhs of the step, part 1: window-start rhs minus the window's deltas s < p - 1 times H
  // blocks, in step order (the last delta is the one finalized below)
  if (a.compute) {
    const float4* dr4 = reinterpret_cast<const float4*>(s_D + 8 * kWS * r);
    const float4* hr4 = reinterpret_cast<const float4*>(s_H + 8 * e);
    for (int s = 0; s + 1 < a.p; ++s) {
      const float4 d0 = dr4[2 * s], d1 = dr4[2 * s + 1];
      const float4 h0 = hr4[16 * s], h1 = hr4[16 * s + 1];
      rh = rh - d0.x * h0.x;
      rh = rh - d0.y * h0.y;
      rh = rh - d0.z * h0.z;
      rh = rh - d0.w * h0.w;
      rh = rh - d1.x * h1.x;
      rh = rh - d1.y * h1.y;
      rh = rh - d1.z * h1.z;
      rh = rh - d1.w * h1.w;
    }
  }

  // ---- finalize: the candidate's coordinate e from its index (as grid_kernel forms the grid),
  // accept test and (chunk 0) the state updates
  float dl = 0.f;  // accepted delta of the finalized step, coordinate e
  if (a.finalize) {
    const int sb = bi & 255;
    const int branch = __builtin_popcount(sb) & 1;
    const int signs = sb ^ (((branch ^ cpar) & 1) << 7);
    const float cand = (branch ? -0.25f : 0.25f) + (((signs >> e) & 1) ? -cav : cav);
    const float fd = cand - fx;
    float dg = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) dg = dg + __shfl(fd, gbase + d) * gm[d];
    const float cross = sum8(fr * fd);
    float dn = sum8(dg * fd);
    dn = dn > 0.f ? dn : 0.f;
    float ce = (r0 + dn) - 2.0f * cross;
    ce = ce > 0.f ? ce : 0.f;
    const bool acc = ce + 1e-12f < r0 * (1.0f + a.accept_tol);
    dl = acc ? fd : 0.f;
    if (writer && valid) {
      a.D[row * kDS + 8 * a.fin_slot + e] = dl;
      if (acc) a.x[row * n + 8 * (int64_t)jp + e] = cand;
      if (e == 0) {
        a.res[(int64_t)(a.fin_par ^ 1) * rows + row] = acc ? ce : r0;
        if (acc) {
          a.idx[row * a.nb + jp] = bi;
          a.accepted[row] += 1;
        }
      }
    }
  }
  if (!a.compute) return;

  // ---- rhs of the step, part 2: the finalized delta (step p - 1 of the window), then the target
  // of order position t (block j) from block j's L and Gi
  if (a.p > 0) {
    const float* hl = s_H + 64 * (a.p - 1) + 8 * e;
#pragma unroll
    for (int d = 0; d < 8; ++d) rh = rh - __shfl(dl, gbase + d) * hl[d];
  }
  if (writer && valid) {
    a.Xt[(int64_t)a.cur_par * rows * 8 + row * 8 + e] = xb;
    a.Rt[(int64_t)a.cur_par * rows * 8 + row * 8 + e] = rh;
  }
  float tg = xb;
#pragma unroll
  for (int d = 0; d < 8; ++d) tg = tg + __shfl(rh, gbase + d) * s_M[64 + d * 8 + e];
  float tm = 0.f;  // (target L)_e
#pragma unroll
  for (int d = 0; d < 8; ++d) tm = tm + __shfl(tg, gbase + d) * s_M[d * 8 + e];
  float u = 0.f;  // (L tm)_e = (L L^T target)_e
#pragma unroll
  for (int f = 0; f < 8; ++f) u = u + s_M[e * 8 + f] * __shfl(tm, gbase + f);
  s_u[r][e] = -2.0f * u;
  __syncthreads();  // every wave is past the window loop: s_D's space takes the chunk's table
  {
    float4* dst = reinterpret_cast<float4*>(s_cgc) + tid;
    dst[0] = cg0;
    dst[256] = cg1;
    dst[512] = cg2;
    dst[768] = cg3;
  }
  __syncthreads();

  // ---- argmin over the chunk: wave w takes a quarter, 32 codewords per MFMA tile.
  // The product u . c runs on v_mfma_f32_32x32x16_bf16: codewords (multiples of 1/4 below 4, exact
  // in bf16) on the M side, the rows' u = -2 L L^T target on the N side as three exact bf16 planes
  // (u = hi + mid + lo), K = 16 holding (hi | mid) in one product and (lo | 0) in the other, each
  // k slot pairing coordinate d with plane (k / 8): every product is exact, summed in fp32.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int i = lane & 31;
  bf16x8_t bu1, bu2;
  {
    uint32_t ph[4], pm[4], plo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) split3(s_u[i][2 * q], s_u[i][2 * q + 1], ph[q], pm[q], plo[q]);
    const uint4 u1 = h ? make_uint4(pm[0], pm[1], pm[2], pm[3]) : make_uint4(ph[0], ph[1], ph[2], ph[3]);
    const uint4 u2 = h ? make_uint4(0u, 0u, 0u, 0u) : make_uint4(plo[0], plo[1], plo[2], plo[3]);
    bu1 = __builtin_bit_cast(bf16x8_t, u1);
    bu2 = __builtin_bit_cast(bf16x8_t, u2);
  }
  const int pl = __builtin_popcount(i) & 1;
  const int wq = kCS / 4;
  const int wbeg = c0 + wave * wq;
  float best = INFINITY;
  int btile = wbeg;
  floatx16 snap;
#pragma unroll
  for (int v = 0; v < 16; ++v) snap[v] = INFINITY;
  for (int kb = wbeg; kb < wbeg + wq; kb += 256) {
    const int k = kb >> 8;
    const int bp = (int)kE8Parity[k];
    // lane half h generates coordinates 4 h .. 4 h + 3 of its codeword
    const float* ak = s_abs + (k - c0 / 256) * 8 + 4 * h;
    const float a0 = ak[0], a1 = ak[1], a2 = ak[2], a3 = ak[3];
    // the codeword operand of tile th (32 codewords kb + 32 th + i)
    auto codewords = [&](int th) {
      const int shi = th * 32;
      const int s8 = shi | i;
      const int branch = (__builtin_popcount(shi) & 1) ^ pl;
      const int sg = (s8 ^ (((branch ^ bp) & 1) << 7)) >> (4 * h);
      const float sh = branch ? -0.25f : 0.25f;
      const float c0v = sh + ((sg & 1) ? -a0 : a0);
      const float c1v = sh + ((sg & 2) ? -a1 : a1);
      const float c2v = sh + ((sg & 4) ? -a2 : a2);
      const float c3v = sh + ((sg & 8) ? -a3 : a3);
      // exact bf16 pairs; the two lane halves exchange theirs so every lane holds all 8 coordinates
      const auto px = __builtin_amdgcn_permlane32_swap(pk_bf16(c0v, c1v), pk_bf16(c0v, c1v), false, false);
      const auto py = __builtin_amdgcn_permlane32_swap(pk_bf16(c2v, c3v), pk_bf16(c2v, c3v), false, false);
      return __builtin_bit_cast(bf16x8_t, make_uint4(px[0], py[0], px[1], py[1]));
    };
    auto table = [&](int th) {  // |L^T c|^2 of the tile's codewords at the lane's accumulator slots
      const float* cp = s_cgc + (kb + 32 * th - c0) + 4 * h;
      floatx16 acc;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 q = *reinterpret_cast<const float4*>(cp + 8 * g);
        acc[4 * g + 0] = q.x;
        acc[4 * g + 1] = q.y;
        acc[4 * g + 2] = q.z;
        acc[4 * g + 3] = q.w;
      }
      return acc;
    };
    // the lane's best tile so far: its minimum, its first codeword and a copy of its 16 scores,
    // kept with selects (no branch); the index inside the tile is resolved once, after the loop.
    // First index on ties: a later tile replaces only a strictly smaller minimum.
    auto keep_min = [&](const floatx16& acc, int th) {
      const float m01 = fminf(acc[0], acc[1]), m23 = fminf(acc[2], acc[3]);
      const float m45 = fminf(acc[4], acc[5]), m67 = fminf(acc[6], acc[7]);
      const float m89 = fminf(acc[8], acc[9]), mab = fminf(acc[10], acc[11]);
      const float mcd = fminf(acc[12], acc[13]), mef = fminf(acc[14], acc[15]);
      const float m = fminf(fminf(fminf(m01, m23), fminf(m45, m67)), fminf(fminf(m89, mab), fminf(mcd, mef)));
      const bool better = m < best;
      best = better ? m : best;
      btile = better ? kb + 32 * th : btile;
#pragma unroll
      for (int v = 0; v < 16; ++v) snap[v] = better ? acc[v] : snap[v];
    };
    // two tiles at a time with their own accumulators: one tile's products run on the matrix core
    // while the other's minimum runs on the vector unit
    for (int th = 0; th < 8; th += 2) {
      const bf16x8_t cwa = codewords(th), cwb = codewords(th + 1);
      floatx16 acca = table(th), accb = table(th + 1);
      acca = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cwa, bu1, acca, 0, 0, 0);
      accb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cwb, bu1, accb, 0, 0, 0);
      acca = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cwa, bu2, acca, 0, 0, 0);
      accb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cwb, bu2, accb, 0, 0, 0);
      keep_min(acca, th);
      keep_min(accb, th + 1);
    }
  }
  int bidx;
  {
    int vv = 15;
#pragma unroll
    for (int v = 14; v >= 0; --v) vv = snap[v] == best ? v : vv;
    bidx = btile + 8 * (vv >> 2) + 4 * h + (vv & 3);
  }
  // combine the two lane halves (same row, interleaved codewords), then the 4 waves
  {
    const float ob = __shfl_xor(best, 32);
    const int oi = __shfl_xor(bidx, 32);
    if (ob < best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  if (lane < 32) {
    s_bs[wave][lane] = best;
    s_bi[wave][lane] = bidx;
  }
  __syncthreads();
  if (tid < kRT) {
    float bsv = s_bs[0][tid];
    int biv = s_bi[0][tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      if (s_bs[w][tid] < bsv) {
        bsv = s_bs[w][tid];
        biv = s_bi[w][tid];
      }
    }
    const int64_t rl = (int64_t)(blockIdx.x % a.tiles_per_rb) * kRT + tid;
    const int64_t rr = rb * a.block_rows + rl;
    if (rl < a.block_rows && rr < a.rows) {
      a.ps[(int64_t)a.cur_par * rows * 16 + rr * 16 + blockIdx.y] = bsv;
      a.pi[(int64_t)a.cur_par * rows * 16 + rr * 16 + blockIdx.y] = biv;
    }
  }
}

struct CdPlan {
  int64_t nrb, nb, nchunks, bytes;
  int splits, bn;
};

CdPlan e8_cd_plan(int64_t rows, int64_t n, int64_t block_rows) {
  CdPlan c;
  c.nb = n / 8;
  c.nrb = (rows + block_rows - 1) / block_rows;
  c.nchunks = (n + 1023) / 1024;
  int bn = 128;
  c.splits = choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  c.bn = bn;
  const int64_t mat = a64(rows * n) * 4;
  int64_t b = 3 * mat;                         // Yu, residual, rhs
  b += (int64_t)c.splits * mat;                // GEMM partials
  b += a64(c.nrb * c.nb) * 4 * 2;              // gain, order
  b += a64(c.nrb * n) * 4;                     // gather rows
  b += a64(rows * kDS) * 4;                    // deltas
  b += 2 * a64(rows * 8) * 4 * 2;              // Rt, Xt
  b += 2 * a64(rows) * 4;                      // res
  b += 2 * a64(rows * 16) * 4 * 2;             // partial scores / indices, two parities
  b += 3 * a64(rows) * 4;                      // accepted, err_b, err_a
  b += a64(rows * c.nchunks) * 4;              // row partials
  c.bytes = b;
  return c;
}

hipError_t product_splits(const float* A, const float* B, bool trans_b, int64_t rows, int64_t n, float* P,
                          int splits, int bn, hipStream_t stream) {
  GemmParams p{};
  p.M = rows; p.N = n; p.K = n;
  p.A = A; p.lda = n; p.B = B; p.ldb = n; p.trans_b = trans_b;
  p.C = P; p.ldc = n; p.split_stride = a64(rows * n);
  p.alpha = 1.f; p.beta = 0.f; p.mode = kGemmPartials;
  return gemm_partials(p, splits, bn, stream);
}

int64_t ctx_bytes(int64_t n) {
  const int64_t nb = n / 8;
  return a64(n * n) * 4 + a64(nb * kMeta) * 4 + nb * kCodes * 4 + (int64_t)kCodes * 8 * 4 + (256 * 8 + 256) * 4 + 256;
}

struct Ctx {
  float* H;
  float* meta;
  float* cgc;
  float* grid;
  float* pat;
  int* fail;
};

Ctx carve_ctx(void* p, int64_t n) {
  const int64_t nb = n / 8;
  char* c = static_cast<char*>(p);
  Ctx x;
  x.H = (float*)c; c += a64(n * n) * 4;
  x.meta = (float*)c; c += a64(nb * kMeta) * 4;
  x.cgc = (float*)c; c += nb * kCodes * 4;
  x.grid = (float*)c; c += (int64_t)kCodes * 8 * 4;
  x.pat = (float*)c; c += (256 * 8 + 256) * 4;
  x.fail = (int*)c;
  return x;
}

}  // namespace
}  // namespace mpq

extern "C" int64_t mpq_e8p12_cd_context_size(int64_t n) {
  if (n <= 0 || n % 8) return 0;
  return mpq::ctx_bytes(n);
}

extern "C" int mpq_e8p12_cd_prepare(int64_t n, const float* Vs, void* ctx, int64_t ctx_bytes_given,
                                    hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(n > 0 && n % 8 == 0, "E8P12 polish expects n divisible by 8; got n=%lld", (long long)n);
  MPQ_CHECK_ARG(n / 8 <= 65535, "mpq_e8p12_cd_prepare: n too large");
  MPQ_CHECK_ARG(Vs && ctx, "mpq_e8p12_cd_prepare: null argument");
  MPQ_CHECK_ARG(ctx_bytes_given >= ctx_bytes(n), "mpq_e8p12_cd_prepare: context too small (%lld < %lld)",
                (long long)ctx_bytes_given, (long long)ctx_bytes(n));
  const Ctx c = carve_ctx(ctx, n);
  const int64_t nb = n / 8;
  // H = Vs Vs^T (the per-block grams are its 8x8 diagonal blocks)
  MPQ_HIP_TRY(gemm(Vs, n, Vs, n, true, nullptr, c.H, n, n, n, n, 1.f, 0.f, nullptr, 0, stream));
  MPQ_HIP_TRY(hipMemsetAsync(c.fail, 0, sizeof(int), stream));
  hipLaunchKernelGGL(grid_kernel, dim3(kCodes / 256), dim3(256), 0, stream, c.grid, c.pat);
  hipLaunchKernelGGL(meta_kernel, dim3((unsigned)((nb + 63) / 64)), dim3(64), 0, stream, n, nb, c.H, c.meta,
                     c.fail);
  hipLaunchKernelGGL(cgc_kernel, dim3(kCodes / 256, (unsigned)nb), dim3(256), 0, stream, c.grid, c.meta, c.cgc);
  MPQ_LAUNCH_CHECK();
  int fail = 0;
  MPQ_HIP_TRY(hipMemcpyAsync(&fail, c.fail, sizeof(int), hipMemcpyDeviceToHost, stream));
  MPQ_HIP_TRY(hipStreamSynchronize(stream));
  if (fail) {
    mpq::set_error("stabilize_cholesky: Cholesky of %d block gram(s) failed after 6 jitter retries", fail);
    mpq::set_error_code(kNumerical);
    return kNumerical;
  }
  return kOk;
}

extern "C" int64_t mpq_e8p12_cd_workspace_size(int64_t rows, int64_t n, int64_t block_rows) {
  if (rows <= 0 || n <= 0 || n % 8 || block_rows <= 0) return 0;
  return mpq::e8_cd_plan(rows, n, block_rows).bytes;
}

extern "C" int mpq_e8p12_cd_polish(int64_t rows, int64_t n, int64_t block_rows, int sweeps, int64_t max_blocks,
                                   float accept_tol, const float* W, const float* Yu_in, const float* x_in,
                                   const int64_t* idx_in, const float* Vs, const void* ctx, float* x_out,
                                   int64_t* idx_out, float* err_before_out, float* err_after_out,
                                   int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                                   hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(rows > 0 && n > 0 && n % 8 == 0, "E8P12 polish expects n divisible by 8; got n=%lld",
                (long long)n);
  MPQ_CHECK_ARG(block_rows >= 1 && sweeps >= 0, "mpq_e8p12_cd_polish: bad sizes");
  MPQ_CHECK_ARG(n / 8 <= 16384, "mpq_e8p12_cd_polish: at most 16384 blocks per row (greedy-order sort in LDS)");
  MPQ_CHECK_ARG((W || Yu_in) && x_in && idx_in && Vs && ctx && x_out && idx_out && workspace,
                "mpq_e8p12_cd_polish: null argument");
  const CdPlan pl = e8_cd_plan(rows, n, block_rows);
  MPQ_CHECK_ARG(workspace_bytes >= pl.bytes, "mpq_e8p12_cd_polish: workspace too small (%lld < %lld)",
                (long long)workspace_bytes, (long long)pl.bytes);
  const int64_t tiles_per_rb = (std::min(block_rows, rows) + kRT - 1) / kRT;
  MPQ_CHECK_ARG(pl.nrb * tiles_per_rb <= 0x7fffffff, "mpq_e8p12_cd_polish: too many rows");
  const Ctx cx = carve_ctx(const_cast<void*>(ctx), n);
  const int64_t nb = pl.nb;
  const int64_t mat = a64(rows * n) * 4;
  char* p = static_cast<char*>(workspace);
  float* Yu = (float*)p; p += mat;
  float* resid = (float*)p; p += mat;
  float* rhs = (float*)p; p += mat;
  float* P = (float*)p; p += (int64_t)pl.splits * mat;
  float* gain = (float*)p; p += a64(pl.nrb * nb) * 4;
  int32_t* order = (int32_t*)p; p += a64(pl.nrb * nb) * 4;
  int32_t* rowsidx = (int32_t*)p; p += a64(pl.nrb * n) * 4;
  float* D = (float*)p; p += a64(rows * kDS) * 4;
  float* Rt = (float*)p; p += 2 * a64(rows * 8) * 4;
  float* Xt = (float*)p; p += 2 * a64(rows * 8) * 4;
  float* res = (float*)p; p += 2 * a64(rows) * 4;
  float* ps = (float*)p; p += 2 * a64(rows * 16) * 4;   // double-buffered by step parity
  int32_t* pi = (int32_t*)p; p += 2 * a64(rows * 16) * 4;
  int32_t* acc = (int32_t*)p; p += a64(rows) * 4;
  float* err_b = (float*)p; p += a64(rows) * 4;
  float* err_a = (float*)p; p += a64(rows) * 4;
  float* part = (float*)p;
  const int nch = (int)pl.nchunks;
  const dim3 eg((unsigned)nch, (unsigned)rows);
  const int64_t sstride = a64(rows * n);

  if (Yu_in) {
    MPQ_HIP_TRY(hipMemcpyAsync(Yu, Yu_in, rows * n * 4, hipMemcpyDeviceToDevice, stream));
  } else {
    MPQ_HIP_TRY(product_splits(W, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
    MPQ_HIP_TRY(splitk_reduce(P, pl.splits, rows, n, Yu, n, 1.f, 0.f, stream));
  }
  MPQ_HIP_TRY(hipMemcpyAsync(x_out, x_in, rows * n * 4, hipMemcpyDeviceToDevice, stream));
  MPQ_HIP_TRY(hipMemcpyAsync(idx_out, idx_in, rows * nb * 8, hipMemcpyDeviceToDevice, stream));
  // residual_u, res = |residual_u|^2 (error before), rhs = residual_u Vs^T
  MPQ_HIP_TRY(product_splits(x_out, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
  hipLaunchKernelGGL(residual_kernel, eg, dim3(256), 0, stream, rows, n, P, pl.splits, sstride, Yu, resid, part,
                     nch);
  hipLaunchKernelGGL(rows_sum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, rows, nch, part,
                     err_b);
  MPQ_LAUNCH_CHECK();
  MPQ_HIP_TRY(hipMemcpyAsync(res, err_b, rows * 4, hipMemcpyDeviceToDevice, stream));
  MPQ_HIP_TRY(hipMemsetAsync(acc, 0, rows * 4, stream));
  MPQ_HIP_TRY(product_splits(resid, Vs, true, rows, n, P, pl.splits, pl.bn, stream));
  MPQ_HIP_TRY(splitk_reduce(P, pl.splits, rows, n, rhs, n, 1.f, 0.f, stream));

  const int64_t nsteps = (max_blocks > 0 && max_blocks < nb) ? max_blocks : nb;
  const int64_t row_tiles = pl.nrb * tiles_per_rb;
  // kNChunk chunks: the chunk's table takes 16 KB of LDS, so occupancy is set by registers, not LDS
  const int nchunk = kNChunk;
  const bool grouped_gemm = (block_rows % 128 == 0) || pl.nrb == 1;

  StepArgs sa{};
  sa.rows = rows; sa.n = n; sa.nb = nb; sa.block_rows = block_rows;
  sa.tiles_per_rb = (int)tiles_per_rb; sa.accept_tol = accept_tol;
  sa.order = order; sa.meta = cx.meta; sa.cgc = cx.cgc; sa.H = cx.H; sa.grid = cx.grid; sa.pat = cx.pat;
  sa.rhs = rhs; sa.x = x_out; sa.idx = idx_out; sa.res = res; sa.D = D; sa.Rt = Rt; sa.Xt = Xt;
  sa.ps = ps; sa.pi = pi; sa.accepted = acc;
  int64_t g = 0;  // global step counter: parity of the double buffers
  for (int sw = 0; sw < sweeps; ++sw) {
    hipLaunchKernelGGL(e8_gain_kernel, dim3((unsigned)((nb + 255) / 256), (unsigned)pl.nrb), dim3(256), 0, stream,
                       rows, n, nb, block_rows, rhs, cx.meta, gain);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(argsort_desc_rows(gain, pl.nrb, nb, order, stream));
    hipLaunchKernelGGL(expand_rows_kernel, dim3((unsigned)((pl.nrb * n + 255) / 256)), dim3(256), 0, stream,
                       pl.nrb, nb, order, rowsidx);
    MPQ_LAUNCH_CHECK();
    for (int64_t w0 = 0; w0 < nsteps; w0 += kWS) {
      const int wn = (int)std::min<int64_t>(kWS, nsteps - w0);
      for (int pp = 0; pp < wn; ++pp, ++g) {
        sa.finalize = pp > 0;
        sa.fin_t = (int)(w0 + pp - 1);
        sa.fin_slot = pp - 1;
        sa.fin_par = (int)((g - 1) & 1);
        sa.nparts = nchunk;
        sa.compute = 1;
        sa.t = (int)(w0 + pp);
        sa.p = pp;
        sa.w0 = (int)w0;
        sa.cur_par = (int)(g & 1);
        sa.nchunk = nchunk;
        hipLaunchKernelGGL(e8_cd_step_kernel, dim3((unsigned)row_tiles, (unsigned)nchunk), dim3(256), 0, stream,
                           sa);
      }
      sa.finalize = 1;
      sa.fin_t = (int)(w0 + wn - 1);
      sa.fin_slot = wn - 1;
      sa.fin_par = (int)((g - 1) & 1);
      sa.nparts = nchunk;
      sa.compute = 0;
      hipLaunchKernelGGL(e8_cd_step_kernel, dim3((unsigned)row_tiles, 1), dim3(256), 0, stream, sa);
      MPQ_LAUNCH_CHECK();
      // rhs[rows of rb] -= D[rows of rb] (rows x 8wn) @ H[rowsidx[rb][8 w0 : 8 (w0 + wn)], :]
      if (grouped_gemm) {
        GemmParams gp{};
        gp.M = rows; gp.N = n; gp.K = 8 * wn;
        gp.A = D; gp.lda = kDS;
        gp.B = cx.H; gp.ldb = n; gp.trans_b = false;
        gp.b_rows = rowsidx + 8 * w0; gp.b_rows_group = pl.nrb == 1 ? 0 : block_rows;
        gp.b_rows_group_stride = n;
        gp.C = rhs; gp.ldc = n; gp.alpha = -1.f; gp.beta = 1.f; gp.mode = kGemmAxpby;
        MPQ_HIP_TRY(gemm_partials(gp, 1, 64, stream));
      } else {
        for (int64_t b = 0; b < pl.nrb; ++b) {
          const int64_t r0 = b * block_rows;
          GemmParams gp{};
          gp.M = std::min<int64_t>(block_rows, rows - r0); gp.N = n; gp.K = 8 * wn;
          gp.A = D + r0 * kDS; gp.lda = kDS;
          gp.B = cx.H; gp.ldb = n; gp.trans_b = false;
          gp.b_rows = rowsidx + b * n + 8 * w0;
          gp.C = rhs + r0 * n; gp.ldc = n; gp.alpha = -1.f; gp.beta = 1.f; gp.mode = kGemmAxpby;
          MPQ_HIP_TRY(gemm_partials(gp, 1, 64, stream));
        }
      }
    }
  }
  // error after the polish (mpq/solver.py:419-422)
  MPQ_HIP_TRY(product_splits(x_out, Vs, false, rows, n, P, pl.splits, pl.bn, stream));
  hipLaunchKernelGGL(residual_kernel, eg, dim3(256), 0, stream, rows, n, P, pl.splits, sstride, Yu,
                     (float*)nullptr, part, nch);
  hipLaunchKernelGGL(rows_sum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, rows, nch, part,
                     err_a);
  MPQ_LAUNCH_CHECK();
  if (err_before_out) MPQ_HIP_TRY(hipMemcpyAsync(err_before_out, err_b, rows * 4, hipMemcpyDeviceToDevice, stream));
  if (err_after_out) MPQ_HIP_TRY(hipMemcpyAsync(err_after_out, err_a, rows * 4, hipMemcpyDeviceToDevice, stream));
  if (accepted_per_row) {
    MPQ_HIP_TRY(hipMemcpyAsync(accepted_per_row, acc, rows * 4, hipMemcpyDeviceToDevice, stream));
  }
  return kOk;
}
