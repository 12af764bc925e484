// E8P12 nearest-codeword (MAP) search on gfx950.
//
// Replaces mpq/priors/e8p12.py:541-631 (vamp_vector_map_e8p12) with its
// per-branch factorized search mpq/priors/e8p12.py:367-449, and the exact
// nearest-codeword quantizer of the codebook object (unit precision, no prior).
//
// Design: one lane per 8-dim vector; the 256 abs patterns are compile-time data
// (generated from mpq_amd/codebook.py), so each per-base score is a straight-line
// sequence over registers: shared prefix sums/minima in lexicographic order,
// one fma for the parity fix, one add for the constant; the first-index argmax
// keeps a running maximum per group of 8 bases and re-evaluates the winning
// group exactly at the end.  No memory traffic inside the search; the kernel is
// VALU-bound (38 B of HBM traffic per vector against ~5k VALU ops).
//
// Bit-exactness: every arithmetic step has the reference's operation order
// (see oracle/e8p12_map.c); the file is compiled with -ffp-contract=off.
#include "common.h"
#include "e8p12_tables.inc"

namespace {

__device__ __forceinline__ int parity8(unsigned v) { return __builtin_popcount(v & 255u) & 1; }

__device__ __forceinline__ float abs_value(int abs2) {
  // 2*|x| in {1,3,5} -> |x| in {0.5, 1.5, 2.5} (exact)
  return 0.5f * (float)abs2;
}

// Exact per-base evaluation (the oracle's loop) for the winner decode and for
// the rare lanes where a product underflows to a signed zero.
struct BaseEval {
  float score;
  unsigned sign_id;
};

__device__ __forceinline__ BaseEval eval_base(const float t[8], float cst_yn, float mhalf_g, int k) {
  float sum_abs = 0.f, min_abs = 0.f;
  int min_pos = 0;
  unsigned neg = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float a = t[i] * abs_value(kE8Abs2[k][i]);
    float aa = fabsf(a);
    if (a < 0.f) neg |= 1u << i;
    if (i == 0) {
      sum_abs = aa;
      min_abs = aa;
    } else {
      sum_abs = sum_abs + aa;
      if (aa < min_abs) {
        min_abs = aa;
        min_pos = i;
      }
    }
  }
  int mismatch = parity8(neg) != (int)kE8Parity[k];
  BaseEval out;
  out.sign_id = mismatch ? (neg ^ (1u << min_pos)) : neg;
  float linear = sum_abs - (2.0f * (float)mismatch) * min_abs;
  float cst = mhalf_g * (cst_yn + kE8SqNorm[k]);
  out.score = cst + linear;
  return out;
}

// kSplit = false: one lane per vector, 256 vectors per work-group.  kSplit = true (few vectors): 64
// vectors per work-group, one per lane, and the four waves split each vector's search -- wave p walks
// shift branch p / 2, bases 128 (p % 2) .. + 127 -- then wave 0 combines the four (best score, first
// group) pairs in index order, which is the order the one-lane search visits them in, and finishes.
template <bool kPrior, bool kVec4, bool kSplit>
__global__ __launch_bounds__(256) void e8p12_map_kernel(
    const float* __restrict__ r, int64_t n, const float* __restrict__ gamma, int64_t gamma_div,
    const float* __restrict__ center, const float* __restrict__ scale, float tau,
    int64_t* __restrict__ idx64, uint16_t* __restrict__ idx16, float* __restrict__ vals,
    float* __restrict__ err, float* __restrict__ score_out) {
  const int part = kSplit ? (int)(threadIdx.x >> 6) : 0;
  const int64_t v0 = kSplit ? (int64_t)blockIdx.x * 64 + (threadIdx.x & 63)
                            : (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (!kSplit) {
    if (v0 >= n) return;
  }
  // split: the four waves hold the same vectors, so a lane past the end stays (on the last vector)
  // until the combine; every wave reaches the barrier
  const int64_t v = v0 < n ? v0 : n - 1;

  float x[8];
  if constexpr (kVec4) {
    const float4* p = reinterpret_cast<const float4*>(r + 8 * v);
    float4 a = p[0], b = p[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = r[8 * v + i];
  }
  float g = gamma[v / gamma_div];
  float rw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rw[i] = x[i];
  if constexpr (kPrior) {
    // mpq/priors/e8p12.py:561-574: fold the Gaussian prior into (r, gamma).
    float s;
    if (scale != nullptr) {
      s = scale[v];
    } else {  // "absmax" scale of the centre block (mpq/priors/e8p12.py:53-54), exact
      s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s = fmaxf(s, fabsf(center[8 * v + i]));
    }
    s = s < 1e-12f ? 1e-12f : s;
    const float tau_c = tau > 1e-12f ? tau : 1e-12f;
    float ts = tau_c * s;
    float tau2 = ts * ts;
    float prec = 1.0f / tau2;
    float gw = g + prec;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float num = g * x[i] + prec * center[8 * v + i];
      rw[i] = num / gw;
    }
    g = gw;
  }
  const float mhalf_g = -0.5f * g;

  float best = -INFINITY;
  int best_g = 0;  // first group of MPQ_E8_GROUP bases (flattened branch*256 + k) holding `best`
  bool slow = false;

  for (int br = kSplit ? part >> 1 : 0; br < (kSplit ? (part >> 1) + 1 : 2); ++br) {
    const float off = br == 0 ? 0.25f : -0.25f;
    float y[8], t[8], u[8];
    unsigned neg = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = rw[i] - off;
      t[i] = g * y[i];
      u[i] = fabsf(t[i]);
      if (t[i] < 0.f) neg |= 1u << i;
      // A product 0.5*|t| that rounds to zero would drop a sign bit for some bases only.
      slow |= (t[i] != 0.f) && (u[i] * 0.5f == 0.f);
    }
    float yn = y[0] * y[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) yn = yn + y[i] * y[i];

    const int P = parity8(neg);
    const float mk0 = P ? -2.0f : 0.0f;  // bases with even sign parity mismatch iff P == 1
    const float mk1 = P ? 0.0f : -2.0f;
    const float cst0 = mhalf_g * (yn + kE8ClassSqNorm[0]);
    const float cst1 = mhalf_g * (yn + kE8ClassSqNorm[1]);
    const float cst2 = mhalf_g * (yn + kE8ClassSqNorm[2]);
    const float cst3 = mhalf_g * (yn + kE8ClassSqNorm[3]);
    const float cst4 = mhalf_g * (yn + kE8ClassSqNorm[4]);
    const float cst5 = mhalf_g * (yn + kE8ClassSqNorm[5]);
    const float p0_0 = u[0] * 0.5f, p0_1 = u[0] * 1.5f, p0_2 = u[0] * 2.5f;
    const float p1_0 = u[1] * 0.5f, p1_1 = u[1] * 1.5f, p1_2 = u[1] * 2.5f;
    const float p2_0 = u[2] * 0.5f, p2_1 = u[2] * 1.5f, p2_2 = u[2] * 2.5f;
    const float p3_0 = u[3] * 0.5f, p3_1 = u[3] * 1.5f, p3_2 = u[3] * 2.5f;
    const float p4_0 = u[4] * 0.5f, p4_1 = u[4] * 1.5f, p4_2 = u[4] * 2.5f;
    const float p5_0 = u[5] * 0.5f, p5_1 = u[5] * 1.5f, p5_2 = u[5] * 2.5f;
    const float p6_0 = u[6] * 0.5f, p6_1 = u[6] * 1.5f, p6_2 = u[6] * 2.5f;
    const float p7_0 = u[7] * 0.5f, p7_1 = u[7] * 1.5f, p7_2 = u[7] * 2.5f;
    const int br_group = br * (256 / MPQ_E8_GROUP);
    if constexpr (!kSplit) {
#include "e8p12_search.inc"
    } else if ((part & 1) == 0) {
#include "e8p12_search_h0.inc"
    } else {
#include "e8p12_search_h1.inc"
    }
  }
  if constexpr (kSplit) {
    __shared__ float s_best[4][64];
    __shared__ int s_bg[4][64];
    __shared__ int s_slow[4][64];
    const int lane = threadIdx.x & 63;
    s_best[part][lane] = best;
    s_bg[part][lane] = best_g;
    s_slow[part][lane] = slow ? 1 : 0;
    __syncthreads();
    if (part != 0 || v0 >= n) return;
    // index order: (branch 0, bases 0..127), (0, 128..255), (1, 0..127), (1, 128..255); a later part
    // replaces the running choice only with a strictly larger score, as the one-lane walk does
    slow = s_slow[0][lane] | s_slow[2][lane];  // per branch: the same in both of its halves
#pragma unroll
    for (int p = 1; p < 4; ++p) {
      if (s_best[p][lane] > best) {
        best = s_best[p][lane];
        best_g = s_bg[p][lane];
      }
    }
  }

  int br, k;
  if (!slow) {
    // Re-evaluate the winning group exactly; the first base scoring `best` wins.
    br = best_g / (256 / MPQ_E8_GROUP);
    const int k0 = (best_g % (256 / MPQ_E8_GROUP)) * MPQ_E8_GROUP;
    const float off = br == 0 ? 0.25f : -0.25f;
    float y[8], t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = rw[i] - off;
      t[i] = g * y[i];
    }
    float yn = y[0] * y[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) yn = yn + y[i] * y[i];
    k = k0;
    for (int j = MPQ_E8_GROUP - 1; j >= 0; --j) {
      if (eval_base(t, yn, mhalf_g, k0 + j).score == best) k = k0 + j;
    }
  } else {
    // Exact per-base sweep (never taken for normal-range inputs).
    best = -INFINITY;
    int best_k = 0;
    for (int b = 0; b < 2; ++b) {
      const float off = b == 0 ? 0.25f : -0.25f;
      float y[8], t[8];
      for (int i = 0; i < 8; ++i) {
        y[i] = rw[i] - off;
        t[i] = g * y[i];
      }
      float yn = y[0] * y[0];
      for (int i = 1; i < 8; ++i) yn = yn + y[i] * y[i];
      for (int kk = 0; kk < 256; ++kk) {
        BaseEval e = eval_base(t, yn, mhalf_g, kk);
        if (e.score > best) {
          best = e.score;
          best_k = b * 256 + kk;
        }
      }
    }
    br = best_k >> 8;
    k = best_k & 255;
  }

  // Decode the winner: recompute its sign pattern exactly.
  const float off = br == 0 ? 0.25f : -0.25f;
  float t[8];
  float yn;
  {
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = rw[i] - off;
      t[i] = g * y[i];
    }
    yn = y[0] * y[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) yn = yn + y[i] * y[i];
  }
  BaseEval e = eval_base(t, yn, mhalf_g, k);
  const unsigned s = e.sign_id ^ ((unsigned)((br ^ (int)kE8Parity[k]) & 1) << 7);
  const int idx = (k << 8) | (int)s;
  if (idx64) idx64[v] = idx;
  if (idx16) idx16[v] = (uint16_t)idx;
  if (score_out) score_out[v] = best;
  if (vals || err) {
    float c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float a = abs_value(kE8Abs2[k][i]);
      c[i] = off + (((e.sign_id >> i) & 1u) ? -a : a);
    }
    if (vals) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vals[8 * v + i] = c[i];
    }
    if (err) {
      float d0 = x[0] - c[0];
      float acc = d0 * d0;
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        float d = x[i] - c[i];
        acc = acc + d * d;
      }
      err[v] = acc;
    }
  }
}

}  // namespace

extern "C" int mpq_e8p12_map(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                             const float* center, const float* scale, float tau, int64_t* idx64,
                             uint16_t* idx16, float* vals, float* err, float* score,
                             hipStream_t stream) {
  MPQ_CHECK_ARG(n >= 0, "mpq_e8p12_map: n must be >= 0, got %lld", (long long)n);
  if (n == 0) return mpq::kOk;
  MPQ_CHECK_ARG(r != nullptr && gamma != nullptr, "mpq_e8p12_map: r and gamma are required");
  MPQ_CHECK_ARG(gamma_div >= 1, "mpq_e8p12_map: gamma_div must be >= 1");
  const bool prior = center != nullptr && tau > 0.0f;
  MPQ_CHECK_ARG(idx64 || idx16 || vals || err || score, "mpq_e8p12_map: no output requested");
  const bool vec4 = (reinterpret_cast<uintptr_t>(r) & 15u) == 0;
  // Below 2^19 vectors one lane per vector leaves SIMDs idle (2^19 / 64 lanes = 8 waves per SIMD on
  // 256 CUs): four waves per vector then, 64 vectors per work-group.
  const bool split = n < (int64_t(1) << 19);
  const int threads = 256;
  const int64_t blocks = mpq_cdiv(n, split ? 64 : threads);
  MPQ_CHECK_ARG(blocks <= 0x7fffffff, "mpq_e8p12_map: n too large");
  dim3 grid((unsigned)blocks), block(threads);
#define MPQ_E8_LAUNCH(P, V, S)                                                                  \
  hipLaunchKernelGGL((e8p12_map_kernel<P, V, S>), grid, block, 0, stream, r, n, gamma, gamma_div, \
                     center, scale, tau, idx64, idx16, vals, err, score)
#define MPQ_E8_LAUNCH2(P, V) \
  if (split) MPQ_E8_LAUNCH(P, V, true); else MPQ_E8_LAUNCH(P, V, false)
  if (prior) {
    if (vec4) { MPQ_E8_LAUNCH2(true, true); } else { MPQ_E8_LAUNCH2(true, false); }
  } else {
    if (vec4) { MPQ_E8_LAUNCH2(false, true); } else { MPQ_E8_LAUNCH2(false, false); }
  }
#undef MPQ_E8_LAUNCH2
#undef MPQ_E8_LAUNCH
  MPQ_LAUNCH_CHECK();
  return mpq::kOk;
}
