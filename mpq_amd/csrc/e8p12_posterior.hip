// E8P12 posterior (discrete MMSE denoiser) on gfx950.
//
// Replaces mpq/priors/e8p12.py:815-968 (vamp_vector_discrete_mmse_e8p12) with its
// per-branch factorized statistics mpq/priors/e8p12.py:169-308.  For every 8-block the
// posterior over the 2^16 codewords is a mixture of 512 components (2 shifts x 256
// abs patterns), each a product over coordinates of independent signs with one
// parity constraint:
//   a_i = gamma y_i b_i,  logC = sum logaddexp(a_i, -a_i),  t_i = tanh(a_i),
//   log Z_even/odd = logC + log(1 +- prod t) - log 2,
//   E[s_i] = (t_i +- prod_{j != i} t_j) / (1 +- prod t),
//   mu = off + E[s] * b,  E|c|^2 = |b|^2 + 8 off^2 + 2 off sum(mu_core).
// Mixture weights are a softmax over the 512 log-components (computed in one pass
// with a running maximum), var = (E|c|^2 - |mu|^2) / 8, and when the folded
// precision is >= 1e3 the mean snaps to the MAP codeword (var = 0).
//
// Layout: 8 lanes per 8-block.  Each coordinate's |a| takes only three values
// (b in {1/2, 3/2, 5/2}), so per branch lane c of a block computes logaddexp, log|t| and t
// for coordinate c at the three levels and stores them in LDS ([slot][block]); the lanes then
// split the 256 bases (k = c mod 8) with their own online softmax, reading the tables and the
// packed abs patterns from LDS, and merge the 8 partial states with a butterfly.
// Transcendental-bound VALU kernel.
#include "common.h"
#include "e8p12_tables.inc"

namespace {

constexpr int kThreads = 256;
constexpr int kLanes = 8;  // lanes per 8-block

__device__ __forceinline__ int slot_of(int abs2) { return abs2 >> 1; }  // 1->0, 3->1, 5->2

// log(1 - exp(x)) for x <= 0 switches from log1p(-exp(x)) to log(-expm1(x)) at -log 2
// (mpq/priors/e8p12.py:213-219)
constexpr float kLog1mexpCut = -0.69314718055994530942f;

// Hardware exp2 / log2 (v_exp_f32, v_log_f32: 1 ulp on the base-2 result) with the base change
// folded in.  exp(x) then has a relative error of about |x| * 2^-24 (6e-6 at the largest mixture
// exponents, |x| < 88, beyond which the weight underflows anyway); log(1 + y), y in [0, 1], an
// absolute error of about 1e-7.  Used for the mixture log-weights and weights, where the
// tolerance is 1e-4 relative on the posterior means; the cancelling log(-expm1(x)) near x = 0
// keeps the accurate library functions.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }
__device__ __forceinline__ float fast_log(float y) { return __builtin_amdgcn_logf(y) * 0.69314718055994530942f; }

// Merge of two partial online-softmax states (running max m, sum Z, first moments mu, second
// moment sec, offset weight wo).  Symmetric in its arguments, so both lanes of a butterfly pair
// obtain bit-identical results.
struct SoftState {
  float m, Z, sec, wo;
  float mu[8];
};

__device__ __forceinline__ void merge_state(SoftState& a, int lane_xor) {
  const float mo = __shfl_xor(a.m, lane_xor);
  const float Zo = __shfl_xor(a.Z, lane_xor);
  const float so = __shfl_xor(a.sec, lane_xor);
  const float wo = __shfl_xor(a.wo, lane_xor);
  const float mn = fmaxf(a.m, mo);
  const float fa = a.m == -INFINITY ? 0.f : expf(a.m - mn);
  const float fo = mo == -INFINITY ? 0.f : expf(mo - mn);
  a.Z = a.Z * fa + Zo * fo;
  a.sec = a.sec * fa + so * fo;
  a.wo = a.wo * fa + wo * fo;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float uo = __shfl_xor(a.mu[i], lane_xor);
    a.mu[i] = a.mu[i] * fa + uo * fo;
  }
  a.m = mn;
}

// 8 lanes per 8-block (kLanes), 32 blocks per 256-thread work-group.  Lane c of a block
// builds the three table slots of coordinate c (logaddexp, log|tanh|, tanh for |b| = 1/2, 3/2,
// 5/2) and walks the bases k = c, c + 8, ..., c + 248 of each shift branch with its own online
// softmax; the 8 partial states are merged by a butterfly at the end.
template <bool kPrior>
__global__ __launch_bounds__(kThreads) void e8p12_posterior_kernel(
    const float* __restrict__ r, int64_t n, const float* __restrict__ gamma, int64_t gamma_div,
    const float* __restrict__ center, const float* __restrict__ scale, float tau,
    const float* __restrict__ map_vals, float* __restrict__ x1_out, float* __restrict__ var_out) {
  constexpr int kBlocks = kThreads / kLanes;
  __shared__ float s_lc[24][kBlocks];
  __shared__ float s_lt[24][kBlocks];
  __shared__ float s_t[24][kBlocks];
  __shared__ unsigned s_code[256];  // bits 2i..2i+1: slot of coordinate i; bit 16: odd parity
  __shared__ float s_sq[256];

  const int tid = threadIdx.x;
  const int bl = tid / kLanes;
  const int c = tid % kLanes;
  const int64_t v = (int64_t)blockIdx.x * kBlocks + bl;
  const bool active = v < n;
  const int64_t vv = active ? v : n - 1;

  for (int k = tid; k < 256; k += kThreads) {
    unsigned w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (unsigned)slot_of(kE8Abs2[k][i]) << (2 * i);
    w |= (unsigned)(kE8Parity[k] & 1) << 16;
    s_code[k] = w;
    s_sq[k] = kE8SqNorm[k];
  }

  float rc = r[8 * vv + c];
  float g = gamma[vv / gamma_div];
  if constexpr (kPrior) {
    const float cc = center[8 * vv + c];
    float sc;
    if (scale != nullptr) {
      sc = scale[vv];
    } else {
      sc = fabsf(cc);
      sc = fmaxf(sc, __shfl_xor(sc, 1));
      sc = fmaxf(sc, __shfl_xor(sc, 2));
      sc = fmaxf(sc, __shfl_xor(sc, 4));
    }
    sc = sc < 1e-12f ? 1e-12f : sc;
    const float tau_c = tau > 1e-12f ? tau : 1e-12f;
    const float ts = tau_c * sc;
    const float prec = 1.0f / (ts * ts);
    const float gw = g + prec;
    rc = (g * rc + prec * cc) / gw;
    g = gw;
  }
  const float mhalf_g = -0.5f * g;
  const float t_hi = (float)(1.0 - 1e-7);
  const float t_lo = (float)(-1.0 + 1e-7);
  const float kLog2 = 0.69314718055994530942f;

  SoftState st;
  st.m = -INFINITY;
  st.Z = 0.f;
  st.sec = 0.f;
  st.wo = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.mu[i] = 0.f;

  for (int br = 0; br < 2; ++br) {
    const float off = br == 0 ? 0.25f : -0.25f;
    const float yc = rc - off;
    float yn = yc * yc;
    yn = yn + __shfl_xor(yn, 1);
    yn = yn + __shfl_xor(yn, 2);
    yn = yn + __shfl_xor(yn, 4);
    unsigned negmask = 0;  // bit (3 i + slot): t < 0
    const float gy = g * yc;
#pragma unroll
    for (int sl = 0; sl < 3; ++sl) {
      const float b = 0.5f + (float)sl;
      const float a = gy * b;
      const float aa = fabsf(a);
      const float lc = aa + log1pf(expf(-2.0f * aa));  // logaddexp(a, -a)
      float t = tanhf(a);
      t = t < t_lo ? t_lo : (t > t_hi ? t_hi : t);
      float at = fabsf(t);
      at = at < 1e-7f ? 1e-7f : at;
      s_lc[3 * c + sl][bl] = lc;
      s_lt[3 * c + sl][bl] = logf(at);
      s_t[3 * c + sl][bl] = t;
      if (t < 0.f) negmask |= 1u << (3 * c + sl);
    }
    negmask |= __shfl_xor(negmask, 1);
    negmask |= __shfl_xor(negmask, 2);
    negmask |= __shfl_xor(negmask, 4);
    __syncthreads();

    for (int k = c; k < 256; k += kLanes) {
      const unsigned w = s_code[k];
      int sl[8];
      float bv[8];
      unsigned bm = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int code = (int)((w >> (2 * i)) & 3u);
        sl[i] = 3 * i + code;
        bv[i] = 0.5f + (float)code;
        bm |= 1u << sl[i];
      }
      const bool even = (w >> 16) == 0u;
      float logC = s_lc[sl[0]][bl];
      float L = s_lt[sl[0]][bl];
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        logC = logC + s_lc[sl[i]][bl];
        L = L + s_lt[sl[i]][bl];
      }
      const bool neg = (__builtin_popcount(negmask & bm) & 1) != 0;
      // log(1 + prod t) for an even base, log(1 - prod t) for an odd base; |prod t| = exp(L) is
      // evaluated once and shared with the sign means below
      const bool plus_branch = even != neg;
      const float pabs = fast_exp(L);
      const float lz = plus_branch ? fast_log(1.0f + pabs)
                                   : (L < kLog1mexpCut ? fast_log(1.0f - pabs) : logf(-expm1f(L)));
      const float logZs = (logC + lz) - kLog2;
      const float sq = s_sq[k];
      const float lcomp = mhalf_g * (yn + sq) + logZs;
      // online softmax: the larger of (running max, new log-weight) contributes exp(0) = 1, so one
      // exponential per component gives the same bits as exp(m - max) and exp(lcomp - max)
      const bool up = lcomp > st.m;
      const float e = fast_exp(up ? st.m - lcomp : lcomp - st.m);
      const float resc = up ? e : 1.0f;
      const float wgt = up ? 1.0f : e;
      st.m = up ? lcomp : st.m;
      // sign means with prefix / suffix products (mpq/priors/e8p12.py:235-255)
      float tt[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) tt[i] = s_t[sl[i]][bl];
      const float prod = neg ? -pabs : pabs;
      float denom = even ? 1.0f + prod : 1.0f - prod;
      denom = fabsf(denom) > 1e-12f ? denom : 1.0f;
      const float inv = 1.0f / denom;
      float pre[8];
      float acc = 1.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pre[i] = acc;
        acc = acc * tt[i];
      }
      float suf = 1.0f;
      float mc[8];
#pragma unroll
      for (int i = 7; i >= 0; --i) {
        const float excl = pre[i] * suf;
        float smn = (even ? tt[i] + excl : tt[i] - excl) * inv;
        if (!isfinite(smn)) smn = 0.f;
        mc[i] = smn * bv[i];
        suf = suf * tt[i];
      }
      float mcsum = mc[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mcsum = mcsum + mc[i];
      const float second = (sq + 8.0f * (off * off)) + (2.0f * off) * mcsum;
      st.Z = st.Z * resc + wgt;
#pragma unroll
      for (int i = 0; i < 8; ++i) st.mu[i] = st.mu[i] * resc + wgt * mc[i];
      st.sec = st.sec * resc + wgt * second;
      st.wo = st.wo * resc + wgt * off;
    }
    __syncthreads();
  }
  merge_state(st, 1);
  merge_state(st, 2);
  merge_state(st, 4);
  if (!active) return;
  float msq = 0.f;
  float x1c = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float xi = (st.mu[i] + st.wo) / st.Z;
    msq = i == 0 ? xi * xi : msq + xi * xi;
    if (i == c) x1c = xi;
  }
  float var = ((st.sec / st.Z) - msq) / 8.0f;
  var = var < 0.f ? 0.f : var;
  if (g >= 1e3f) {
    x1c = map_vals[8 * v + c];
    var = 0.f;
  }
  x1_out[8 * v + c] = x1c;
  if (c == 0) var_out[v] = var;
}

// alpha1 = gamma1_row * mean(var1 over the row's blocks) (mpq/priors/e8p12.py:955).
__global__ __launch_bounds__(256) void row_mean_scale_kernel(const float* __restrict__ var, int64_t nb,
                                                             const float* __restrict__ gamma,
                                                             float* __restrict__ alpha) {
  __shared__ float red[4];
  const int64_t b = blockIdx.x;
  float acc = 0.f;
  for (int64_t j = threadIdx.x; j < nb; j += blockDim.x) acc += var[b * nb + j];
  const float t = mpq::block_sum(acc, red);
  if (threadIdx.x == 0) alpha[b] = gamma[b] * (t / (float)nb);
}

}  // namespace

namespace mpq {

hipError_t e8p12_posterior(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                           const float* center, const float* scale, float tau, const float* map_vals,
                           float* x1, float* var, hipStream_t stream) {
  const int64_t blocks = (n + kThreads / kLanes - 1) / (kThreads / kLanes);
  if (center != nullptr && tau > 0.f) {
    hipLaunchKernelGGL(e8p12_posterior_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, r, n,
                       gamma, gamma_div, center, scale, tau, map_vals, x1, var);
  } else {
    hipLaunchKernelGGL(e8p12_posterior_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, stream, r, n,
                       gamma, gamma_div, center, scale, tau, map_vals, x1, var);
  }
  return hipGetLastError();
}

hipError_t row_mean_scale(const float* var, int64_t rows, int64_t nb, const float* gamma, float* alpha,
                          hipStream_t stream) {
  hipLaunchKernelGGL(row_mean_scale_kernel, dim3((unsigned)rows), dim3(256), 0, stream, var, nb, gamma, alpha);
  return hipGetLastError();
}

}  // namespace mpq

extern "C" int mpq_e8p12_map(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                             const float* center, const float* scale, float tau, int64_t* idx64,
                             uint16_t* idx16, float* vals, float* err, float* score, hipStream_t stream);

extern "C" int mpq_e8p12_denoise(const float* r, int64_t rows, int64_t nb, const float* gamma,
                                 const float* center, const float* scale, float tau, float* x1, float* var,
                                 int64_t* map_idx, float* map_vals, float* alpha1, hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && nb >= 0, "mpq_e8p12_denoise: bad shape");
  const int64_t n = rows * nb;
  if (n == 0) return mpq::kOk;
  MPQ_CHECK_ARG(r && gamma && x1 && var && map_vals, "mpq_e8p12_denoise: null argument");
  MPQ_CHECK_ARG(n / 128 + 1 <= 0x7fffffff, "mpq_e8p12_denoise: too many blocks");
  int rc = mpq_e8p12_map(r, n, gamma, nb, center, scale, tau, map_idx, nullptr, map_vals, nullptr, nullptr, stream);
  if (rc != mpq::kOk) return rc;
  MPQ_HIP_TRY(mpq::e8p12_posterior(r, n, gamma, nb, center, scale, tau, map_vals, x1, var, stream));
  if (alpha1) MPQ_HIP_TRY(mpq::row_mean_scale(var, rows, nb, gamma, alpha1, stream));
  return mpq::kOk;
}
