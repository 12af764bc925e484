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
// Layout: one lane per 8-block.  Each coordinate's |a| takes only three values
// (b in {1/2, 3/2, 5/2}), so per branch a lane precomputes 24 values of logaddexp,
// log|t| and t and keeps them in LDS ([slot][lane], conflict-free); the 256 bases
// are walked with uniform (scalar) table reads.  Transcendental-bound VALU kernel.
#include "common.h"
#include "e8p12_tables.inc"

namespace {

constexpr int kThreads = 128;

struct Pattern {
  unsigned char code[8];  // 2*|b| in {1,3,5}
};

__device__ __forceinline__ int slot_of(int abs2) { return abs2 >> 1; }  // 1->0, 3->1, 5->2

__device__ __forceinline__ float log1mexp_f(float x) {
  // log(1 - exp(x)), x <= 0 (mpq/priors/e8p12.py:213-219)
  const float cutoff = -0.69314718055994530942f;
  return x < cutoff ? log1pf(-expf(x)) : logf(-expm1f(x));
}

template <bool kPrior>
__global__ __launch_bounds__(kThreads) void e8p12_posterior_kernel(
    const float* __restrict__ r, int64_t n, const float* __restrict__ gamma, int64_t gamma_div,
    const float* __restrict__ center, const float* __restrict__ scale, float tau,
    const float* __restrict__ map_vals, float* __restrict__ x1_out, float* __restrict__ var_out) {
  __shared__ float s_lc[24][kThreads];
  __shared__ float s_lt[24][kThreads];
  __shared__ float s_t[24][kThreads];
  const int lane = threadIdx.x;
  const int64_t v = (int64_t)blockIdx.x * kThreads + lane;
  const bool active = v < n;
  const int64_t vv = active ? v : n - 1;

  float rw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rw[i] = r[8 * vv + i];
  float g = gamma[vv / gamma_div];
  if constexpr (kPrior) {
    float s;
    if (scale != nullptr) {
      s = scale[vv];
    } else {
      s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s = fmaxf(s, fabsf(center[8 * vv + i]));
    }
    s = s < 1e-12f ? 1e-12f : s;
    const float tau_c = tau > 1e-12f ? tau : 1e-12f;
    const float ts = tau_c * s;
    const float prec = 1.0f / (ts * ts);
    const float gw = g + prec;
#pragma unroll
    for (int i = 0; i < 8; ++i) rw[i] = (g * rw[i] + prec * center[8 * vv + i]) / gw;
    g = gw;
  }
  const float mhalf_g = -0.5f * g;
  const float t_hi = (float)(1.0 - 1e-7);
  const float t_lo = (float)(-1.0 + 1e-7);
  const float kLog2 = 0.69314718055994530942f;

  float m = -INFINITY;  // running maximum of the log-components
  float Z = 0.f;        // sum of exp(lc - m)
  float mu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mu[i] = 0.f;
  float sec = 0.f;
  float wsum_off = 0.f;  // sum of w * offset (the constant part of mu)

  for (int br = 0; br < 2; ++br) {
    const float off = br == 0 ? 0.25f : -0.25f;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = rw[i] - off;
    float yn = y[0] * y[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) yn = yn + y[i] * y[i];
    unsigned negmask = 0;  // bit (3 i + slot): t < 0
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float gy = g * y[i];
#pragma unroll
      for (int sl = 0; sl < 3; ++sl) {
        const float b = 0.5f + (float)sl;  // 0.5, 1.5, 2.5
        const float a = gy * b;
        const float aa = fabsf(a);
        const float lc = aa + log1pf(expf(-2.0f * aa));  // logaddexp(a, -a)
        float t = tanhf(a);
        t = t < t_lo ? t_lo : (t > t_hi ? t_hi : t);
        float at = fabsf(t);
        at = at < 1e-7f ? 1e-7f : at;
        s_lc[3 * i + sl][lane] = lc;
        s_lt[3 * i + sl][lane] = logf(at);
        s_t[3 * i + sl][lane] = t;
        if (t < 0.f) negmask |= 1u << (3 * i + sl);
      }
    }
    __syncthreads();

    for (int k = 0; k < 256; ++k) {
      int sl[8];
      float bv[8];
      unsigned bm = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int code = kE8Abs2[k][i];
        sl[i] = 3 * i + slot_of(code);
        bv[i] = 0.5f * (float)code;
        bm |= 1u << sl[i];
      }
      const bool even = kE8Parity[k] == 0;
      float logC = s_lc[sl[0]][lane];
      float L = s_lt[sl[0]][lane];
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        logC = logC + s_lc[sl[i]][lane];
        L = L + s_lt[sl[i]][lane];
      }
      const bool neg = (__builtin_popcount(negmask & bm) & 1) != 0;
      // log(1 + prod t) for an even base, log(1 - prod t) for an odd base
      const bool plus_branch = even != neg;  // prod t >= 0 with "+", or prod t < 0 with "-"
      const float lz = plus_branch ? log1pf(expf(L)) : log1mexp_f(L);
      const float logZs = (logC + lz) - kLog2;
      const float cst = mhalf_g * (yn + kE8SqNorm[k]);
      const float lcomp = cst + logZs;
      // online softmax update
      const float mnew = fmaxf(m, lcomp);
      const float resc = expf(m - mnew);
      const float w = expf(lcomp - mnew);
      m = mnew;
      // sign means with prefix / suffix products (mpq/priors/e8p12.py:235-255)
      float tt[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) tt[i] = s_t[sl[i]][lane];
      const float pabs = expf(L);
      const float prod = neg ? -pabs : pabs;
      float denom = even ? 1.0f + prod : 1.0f - prod;
      denom = fabsf(denom) > 1e-12f ? denom : 1.0f;
      const float inv = 1.0f / denom;  // one division per base; the 8 sign means multiply by it
      float pre[8];
      float acc = 1.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pre[i] = acc;
        acc = acc * tt[i];
      }
      float suf = 1.0f;
      float mcsum = 0.f;
      float mc[8];
#pragma unroll
      for (int i = 7; i >= 0; --i) {
        const float excl = pre[i] * suf;
        float smn = (even ? tt[i] + excl : tt[i] - excl) * inv;
        if (!isfinite(smn)) smn = 0.f;
        mc[i] = smn * bv[i];
        suf = suf * tt[i];
      }
      mcsum = mc[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mcsum = mcsum + mc[i];
      const float second = (kE8SqNorm[k] + 8.0f * (off * off)) + (2.0f * off) * mcsum;
      Z = Z * resc + w;
#pragma unroll
      for (int i = 0; i < 8; ++i) mu[i] = mu[i] * resc + w * mc[i];
      sec = sec * resc + w * second;
      wsum_off = wsum_off * resc + w * off;
    }
    __syncthreads();
  }
  if (!active) return;
  float x1[8];
  float msq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x1[i] = (mu[i] + wsum_off) / Z;
    msq = i == 0 ? x1[i] * x1[i] : msq + x1[i] * x1[i];
  }
  float var = ((sec / Z) - msq) / 8.0f;
  var = var < 0.f ? 0.f : var;
  if (g >= 1e3f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x1[i] = map_vals[8 * v + i];
    var = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) x1_out[8 * v + i] = x1[i];
  var_out[v] = var;
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
  const int64_t blocks = (n + kThreads - 1) / kThreads;
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
