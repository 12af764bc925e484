// Uniform-grid VAMP on one row block (gfx950).
//
// Replaces mpq/solver.py:426-830 (solve_uniform_rankspace_vamp, without the
// polish, which is mpq_uniform_cd_polish) together with
//   mpq/priors/uniform.py:99-213   discrete_uniform_mmse      -> uniform_denoise_kernel
//   mpq/linear.py:10-56            linear_mmse_exact          -> GEMM + lmmse_epi1/epi2
//   mpq/linear.py:59-82            em_update_obs_precision    -> rows_lmmse_kernel + host
//   mpq/linear.py:85-94            vamp_rankspace_error       -> GEMM + err_epi_kernel
//   mpq/solver.py:833-850          _uniform_hard_decision     -> uniform_denoise_kernel<kHard*>
//
// Layout: every per-element array is rows x n row-major fp32 in HBM; codes are
// uint8.  Quantizer parameters stay in group form (rows x G) and are expanded on
// the fly.  Per-row reductions are written as fixed-order partial sums per
// 1024-column chunk, so every result is bit-reproducible run to run.
//
// Control flow is the reference's, driven from the host with two small status
// reads per iteration (after the denoiser: alpha1 / gamma2 validity; after the
// hard-state error: error mean, EM statistic).  All arithmetic follows the
// reference's operation order where it matters for decisions (scores, MAP,
// rounding); the file is compiled with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "gemm.h"
#include "kernels.h"
#include "uniform_vamp.h"
#include "vamp_common.h"

namespace mpq {
namespace {

enum DenoiseMode : int { kPosterior = 0, kHardMap = 1, kHardRoundMean = 2, kFull = 3 };
constexpr int kRegAtoms = 16;  // grids up to 4 bits keep their scores in registers

// Per element: posterior of a uniform grid a_q = s(q - z), q = 0..maxq, under the
// channel N(r1, 1/gamma) and the prior N(W, (tau*s)^2)  (mpq/priors/uniform.py:177-191): the
// first argmax of the atom scores and (MOMENTS) the softmax mean and variance.
template <bool MOMENTS>
__device__ __forceinline__ void denoise_element(float r, float c, float s, float z, float mh, float tau, int maxq,
                                                int& arg_out, float& mean_out, float& var_out) {
  float st2 = 0.f;
  if (tau > 0.f) {
    const float sc = s < 1e-12f ? 1e-12f : s;
    const float ts = tau * sc;
    st2 = ts * ts;
  }
  // score of atom q (the division is kept as a division: MAP decisions are bit-exact)
  auto score_of = [&](int q) {
    const float a = s * ((float)q - z);
    const float d = a - r;
    float score = mh * (d * d);
    if (tau > 0.f) {
      const float dc = a - c;
      score = score - (0.5f * (dc * dc)) / st2;
    }
    return score;
  };
  // pass 1: scores, max, first argmax.  Grids of up to kRegAtoms levels (4-bit) keep the scores
  // in registers for pass 2, so each score is computed once.
  float sc_reg[kRegAtoms];
  const bool in_regs = maxq < kRegAtoms;
  float mx = -INFINITY;
  int arg = 0;
  if (in_regs) {
#pragma unroll
    for (int q = 0; q < kRegAtoms; ++q) {
      sc_reg[q] = q <= maxq ? score_of(q) : -INFINITY;
      if (q <= maxq && sc_reg[q] > mx) {
        mx = sc_reg[q];
        arg = q;
      }
    }
  } else {
    for (int q = 0; q <= maxq; ++q) {
      const float score = score_of(q);
      if (score > mx) {
        mx = score;
        arg = q;
      }
    }
  }
  arg_out = arg;
  if (MOMENTS) {
    // pass 2: softmax moments
    float zsum = 0.f, m1 = 0.f, m2 = 0.f;
    if (in_regs) {
#pragma unroll
      for (int q = 0; q < kRegAtoms; ++q) {
        if (q > maxq) break;
        const float a = s * ((float)q - z);
        const float w = expf(sc_reg[q] - mx);
        zsum += w;
        m1 += w * a;
        m2 += w * (a * a);
      }
    } else {
      for (int q = 0; q <= maxq; ++q) {
        const float a = s * ((float)q - z);
        const float w = expf(score_of(q) - mx);
        zsum += w;
        m1 += w * a;
        m2 += w * (a * a);
      }
    }
    const float mean = m1 / zsum;
    const float second = m2 / zsum;
    const float var = second - mean * mean;
    mean_out = mean;
    var_out = var < 0.f ? 0.f : var;
  }
}

template <int MODE>
__global__ __launch_bounds__(kEW) void uniform_denoise_kernel(
    const float* __restrict__ r1, const float* __restrict__ gamma, const float* __restrict__ W,
    int64_t ldw, const float* __restrict__ scale, const float* __restrict__ zero, int64_t G,
    int64_t gs, int64_t n, int maxq, float tau, float* __restrict__ mean_out,
    float* __restrict__ var_part, uint8_t* __restrict__ q_out, float* __restrict__ x_out,
    uint4* __restrict__ planes) {
  __shared__ float red[kEW / 64];
  __shared__ __attribute__((aligned(16))) float s_v[(MODE == kHardMap || MODE == kHardRoundMean) ? kChunk : 4];
  const int64_t b = blockIdx.y;
  const int nchunks = gridDim.x;
  const float g = gamma[b];
  const float mh = -0.5f * g;
  float vsum = 0.f;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const float r = r1[b * n + j];
    const float c = W[b * ldw + j];
    const float s = grp(scale, b, G, gs, j);
    const float z = grp(zero, b, G, gs, j);
    int arg;
    float mean = 0.f, var = 0.f;
    denoise_element<MODE == kPosterior || MODE == kHardRoundMean || MODE == kFull>(r, c, s, z, mh, tau, maxq, arg,
                                                                                 mean, var);
    if (MODE == kPosterior) {
      mean_out[b * n + j] = mean;
      vsum += var;
    }
    if (MODE == kFull) {
      mean_out[b * n + j] = mean;
      var_part[b * n + j] = var;  // per-element variance in this mode
      reinterpret_cast<int64_t*>(q_out)[b * n + j] = arg;
      x_out[b * n + j] = s * ((float)arg - z);
    }
    if (MODE == kHardMap || MODE == kHardRoundMean) {
      int q = arg;
      if (MODE == kHardRoundMean) {
        const float sc = s < 1e-12f ? 1e-12f : s;
        float qf = rintf(mean / sc + z);
        qf = qf < 0.f ? 0.f : (qf > (float)maxq ? (float)maxq : qf);
        q = (int)qf;
      }
      q_out[b * n + j] = (uint8_t)q;
      x_out[b * n + j] = s * ((float)q - z);
      if (planes) s_v[e * kEW + threadIdx.x] = s * ((float)q - z);
    }
  }
  if (MODE == kHardMap || MODE == kHardRoundMean) {
    if (planes) {  // uniform: the planes of the hard state for its x6 product
      __syncthreads();
      chunk_planes(planes, n, b, s_v);
    }
  }
  if (MODE == kPosterior) {
    const float tot = block_sum(vsum, red);
    if (threadIdx.x == 0) var_part[b * nchunks + blockIdx.x] = tot;
  }
}

// LMMSE part 2 and the r1 message as lmmse_epi2_kernel (r1 <- damped), then, from the new r1 in
// registers, the hard decision of uniform_denoise_kernel<HMODE> with gamma = the damped gamma1 the
// row kernel wrote: one launch and one pass over r1 instead of two, the same per-element arithmetic.
template <int HMODE>
__global__ __launch_bounds__(kEW) void epi2_denoise_kernel(
    int64_t n, const float* __restrict__ P, int splits, int64_t split_stride, const float* __restrict__ r2,
    const float* __restrict__ eta2, const float* __restrict__ g2, const float* __restrict__ g1new, float damping,
    float* __restrict__ r1, const float* __restrict__ gamma, const float* __restrict__ W, int64_t ldw,
    const float* __restrict__ scale, const float* __restrict__ zero, int64_t G, int64_t gs, int maxq, float tau,
    uint8_t* __restrict__ q_out, float* __restrict__ x_out, uint4* __restrict__ planes) {
  static_assert(HMODE == kHardMap || HMODE == kHardRoundMean, "hard decision modes");
  __shared__ __attribute__((aligned(16))) float s_v[kChunk];
  const int64_t b = blockIdx.y;
  const float e2 = eta2[b], gb = g2[b], gn = g1new[b];
  const float keep = 1.0f - damping;
  const float mh = -0.5f * gamma[b];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int64_t j = (int64_t)blockIdx.x * kChunk + e * kEW + threadIdx.x;
    if (j >= n) continue;
    const int64_t o = b * n + j;
    const float d = sum_splits(P, splits, split_stride, o);
    const float r2v = r2[o];
    const float x2 = r2v + d;
    const float rn = (e2 * x2 - gb * r2v) / gn;
    const float r = damping >= 1.f ? rn : keep * r1[o] + damping * rn;
    r1[o] = r;
    const float c = W[b * ldw + j];
    const float s = grp(scale, b, G, gs, j);
    const float z = grp(zero, b, G, gs, j);
    int arg;
    float mean = 0.f, var = 0.f;
    denoise_element<HMODE == kHardRoundMean>(r, c, s, z, mh, tau, maxq, arg, mean, var);
    int q = arg;
    if (HMODE == kHardRoundMean) {
      const float sc = s < 1e-12f ? 1e-12f : s;
      float qf = rintf(mean / sc + z);
      qf = qf < 0.f ? 0.f : (qf > (float)maxq ? (float)maxq : qf);
      q = (int)qf;
    }
    q_out[o] = (uint8_t)q;
    x_out[o] = s * ((float)q - z);
    if (planes) s_v[e * kEW + threadIdx.x] = s * ((float)q - z);
  }
  if (planes) {
    __syncthreads();
    chunk_planes(planes, n, b, s_v);
  }
}

// ---------------------------------------------------------------------------
// Host driver
// ---------------------------------------------------------------------------

struct Workspace {
  float* Yu;
  float* r1;
  float* r2;
  float* r2prev;
  float* x1;  // denoiser mean; reused as the LMMSE coefficient product
  float* xs;  // hard-state dequantised values
  float* prod_cur;   // xs Vs of the current / best hard state (kept when the caller asks for it)
  float* prod_best;
  float* P;   // split-K partials
  void* Ap;   // packed bf16 planes of the left operand (x6 products)
  float* rowbuf;  // per-row arrays
  float* part;    // chunk partials (3 per row per chunk)
  uint8_t* q_cur;
  uint8_t* q_best;
  VampStatus* status;
  int splits;      // of the active product path
  int splits_f32;
  int splits_x6;   // 0 if the shape has no x6 path
  int bn;
  const float* packed;  // rank-space operator of the x6 path, or null (fp32 path)
};

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

struct Sizes {
  int64_t rows, n, nchunks, splits, splits_x6, bn;
  int64_t bytes;
};

Sizes plan(int64_t rows, int64_t n) {
  Sizes s;
  s.rows = rows;
  s.n = n;
  s.nchunks = (n + kChunk - 1) / kChunk;
  int bn = 128;
  s.splits = choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  s.splits_x6 = x6_shape_ok(n, n) ? x6_choose_splits(rows, n, n) : 0;
  s.bn = bn;
  const int64_t mat = align_up(rows * n, 64) * 4;
  int64_t bytes = 0;
  bytes += 8 * mat;                                   // Yu r1 r2 r2prev x1 xs prod_cur prod_best
  bytes += std::max(s.splits, s.splits_x6) * mat;     // P
  bytes += s.splits_x6 ? align_up(x6_packed_a_bytes(rows, n), 256) : 0;  // Ap
  bytes += align_up(32 * rows, 64) * 4;               // row arrays
  bytes += align_up(3 * rows * s.nchunks, 64) * 4;    // chunk partials
  bytes += 2 * align_up(rows * n, 256);               // q_cur q_best
  bytes += 256;                                       // status
  s.bytes = bytes;
  return s;
}

Workspace carve(void* base, const Sizes& s) {
  Workspace w{};
  char* p = static_cast<char*>(base);
  const int64_t mat = align_up(s.rows * s.n, 64) * 4;
  w.Yu = (float*)p; p += mat;
  w.r1 = (float*)p; p += mat;
  w.r2 = (float*)p; p += mat;
  w.r2prev = (float*)p; p += mat;
  w.x1 = (float*)p; p += mat;
  w.xs = (float*)p; p += mat;
  w.prod_cur = (float*)p; p += mat;
  w.prod_best = (float*)p; p += mat;
  w.P = (float*)p; p += std::max(s.splits, s.splits_x6) * mat;
  w.Ap = s.splits_x6 ? (void*)p : nullptr;
  p += s.splits_x6 ? align_up(x6_packed_a_bytes(s.rows, s.n), 256) : 0;
  w.rowbuf = (float*)p; p += align_up(32 * s.rows, 64) * 4;
  w.part = (float*)p; p += align_up(3 * s.rows * s.nchunks, 64) * 4;
  w.q_cur = (uint8_t*)p; p += align_up(s.rows * s.n, 256);
  w.q_best = (uint8_t*)p; p += align_up(s.rows * s.n, 256);
  w.status = (VampStatus*)p;
  w.splits = w.splits_f32 = (int)s.splits;
  w.splits_x6 = (int)s.splits_x6;
  w.bn = (int)s.bn;
  w.packed = nullptr;
  return w;
}

// Pinned host mirror of the device status (one per host thread, freed by
// mpq_release_thread_resources).
VampStatus* host_status() {
  static thread_local VampStatus* h = nullptr;
  if (!h) {
    if (hipHostMalloc((void**)&h, sizeof(VampStatus), hipHostMallocDefault) != hipSuccess) h = nullptr;
    else track_pinned(reinterpret_cast<void**>(&h), nullptr, nullptr);
  }
  return h;
}

}  // namespace

// Rank-space operands of the products (index into the packed operator).
enum RankOperand : int { kOpV = 0, kOpVt = 1, kOpVs = 2 };

// P = A @ op(B) as split-K partials into w.P (split_stride rows*n, w.splits of them).  With a packed
// operator the product runs on the bf16 matrix cores (A split into planes first), else on the
// fp32 MFMA kernel.
static hipError_t product(const Workspace& w, const float* A, const float* B, bool trans_b, RankOperand op,
                          int64_t rows, int64_t n, hipStream_t stream, bool a_planes_written = false) {
  if (w.packed) {
    if (!a_planes_written) {  // else the kernel that produced A wrote its planes into w.Ap
      hipError_t e = x6_pack_a(A, n, rows, n, w.Ap, stream);
      if (e != hipSuccess) return e;
    }
    return x6_gemm_partials(w.Ap, w.packed + (int64_t)op * n * n, rows, n, n, w.P, n, align_up(rows * n, 64),
                            w.splits, stream);
  }
  GemmParams p{};
  p.M = rows; p.N = n; p.K = n;
  p.A = A; p.lda = n; p.B = B; p.ldb = n; p.trans_b = trans_b; p.b_rows = nullptr;
  p.C = w.P; p.ldc = n; p.split_stride = align_up(rows * n, 64);
  p.alpha = 1.f; p.beta = 0.f;
  p.mode = w.splits > 1 ? kGemmPartials : kGemmPartials;
  return gemm_partials(p, w.splits, w.bn, stream);
}

int64_t uniform_vamp_workspace_bytes(int64_t rows, int64_t n) { return plan(rows, n).bytes; }

int uniform_vamp_solve(const UniformProblem& pr, const float* Vs, const MpqUniformVampConfig& cfg,
                       double obs_init, uint8_t* q_out, float* x_out, float* err_out,
                       float* rtn_err_out, MpqUniformVampStats* stats, void* workspace,
                       int64_t workspace_bytes, hipStream_t stream) {
  const int64_t rows = pr.rows, n = pr.n;
  const Sizes sz = plan(rows, n);
  MPQ_CHECK_ARG(workspace_bytes >= sz.bytes, "uniform VAMP: workspace too small (%lld < %lld bytes)",
                (long long)workspace_bytes, (long long)sz.bytes);
  Workspace w = carve(workspace, sz);
  if (pr.packed && w.splits_x6 > 0) {
    w.packed = pr.packed;
    w.splits = w.splits_x6;
  }
  // x6 path: the kernels producing the left operands of the products write its bf16 planes
  uint4* const planes = w.packed ? static_cast<uint4*>(w.Ap) : nullptr;
  const float* Yu = pr.Yu_in ? pr.Yu_in : w.Yu;
  VampStatus* hs = host_status();
  MPQ_CHECK_ARG(hs != nullptr, "uniform VAMP: pinned status buffer unavailable");
  const int nchunks = (int)sz.nchunks;
  const int64_t sstride = align_up(rows * n, 64);
  const dim3 eg((unsigned)nchunks, (unsigned)rows), eb(kEW);
  const int64_t G = (n + pr.group_size - 1) / pr.group_size;

  // per-row arrays
  float* g1 = w.rowbuf + 0 * rows;
  float* g1w = w.rowbuf + 1 * rows;
  float* a1raw = w.rowbuf + 2 * rows;
  float* a1 = w.rowbuf + 3 * rows;
  float* eta1 = w.rowbuf + 4 * rows;
  float* g2new = w.rowbuf + 5 * rows;
  float* g2 = w.rowbuf + 6 * rows;
  float* g2prev = w.rowbuf + 7 * rows;
  float* eta2 = w.rowbuf + 8 * rows;  // 3 * rows: eta2, EM row stat, alpha2
  float* g1new = w.rowbuf + 11 * rows;
  float* err_cur = w.rowbuf + 12 * rows;
  float* err_best = w.rowbuf + 13 * rows;

  HostMailbox* mb = host_mailbox();
  MPQ_CHECK_ARG(mb != nullptr, "uniform VAMP: mapped status mailbox unavailable");
  auto sync_status = [&]() -> int { return read_status(mb, w.status, hs, stream); };
  unsigned hard_seq = 0;  // sequence number the last hard state's row kernel published
  const float tau = cfg.prior_tau;
  int rc;

  // hard state + rank-space error of the decision for (r1, g1) -> q_cur, err_cur, status.err_mean
  // (decided: the denoiser's decision is already in q_cur / xs / planes, from epi2_denoise_kernel)
  auto hard_state = [&](const float* r, const float* g, bool decided) -> int {
    if (decided) {
    } else if (cfg.final_decision == 1) {
      hipLaunchKernelGGL(uniform_denoise_kernel<kHardRoundMean>, eg, eb, 0, stream, r, g, pr.W, pr.ldw,
                         pr.scale, pr.zero, G, pr.group_size, n, pr.maxq, tau, nullptr, nullptr,
                         w.q_cur, w.xs, planes);
    } else {
      hipLaunchKernelGGL(uniform_denoise_kernel<kHardMap>, eg, eb, 0, stream, r, g, pr.W, pr.ldw,
                         pr.scale, pr.zero, G, pr.group_size, n, pr.maxq, tau, nullptr, nullptr,
                         w.q_cur, w.xs, planes);
    }
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(product(w, w.xs, Vs, false, kOpVs, rows, n, stream, planes != nullptr));
    hipLaunchKernelGGL(err_epi_kernel, eg, eb, 0, stream, n, w.P, w.splits, sstride, Yu, w.part,
                       pr.xprod_out ? w.prod_cur : nullptr);
    // the row kernel publishes the status (hard_seq) for the wait that follows every hard state
    hard_seq = ++mb->seq;
    hipLaunchKernelGGL(rows_err_kernel, dim3(1), eb, 0, stream, rows, nchunks, w.part, err_cur, w.status, mb->dev(hard_seq),
                       hard_seq);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };

  // ---- setup ----------------------------------------------------------
  // Yu = W @ Vs (or the caller's)
  if (!pr.Yu_in) {
    // W may be strided (ldw); copy to contiguous r1 first when needed.
    const float* Wc = pr.W;
    if (pr.ldw != n) {
      MPQ_HIP_TRY(copy_rows(w.r1, n * 4, pr.W, pr.ldw * 4, rows, n * 4, stream));
      Wc = w.r1;
    }
    MPQ_HIP_TRY(product(w, Wc, Vs, false, kOpVs, rows, n, stream));
    MPQ_HIP_TRY(splitk_reduce(w.P, w.splits, rows, n, w.Yu, n, 1.f, 0.f, stream));
  }
  // RTN error (rtn_err, and the obs warm start when none is given), from x_init Vs (or the caller's)
  if (pr.xr_in) {
    hipLaunchKernelGGL(err_epi_kernel, eg, eb, 0, stream, n, pr.xr_in, 1, (int64_t)0, Yu, w.part, nullptr);
  } else {
    MPQ_HIP_TRY(copy_rows(w.xs, n * 4, pr.x_init, pr.ldw * 4, rows, n * 4, stream));
    MPQ_HIP_TRY(product(w, w.xs, Vs, false, kOpVs, rows, n, stream));
    hipLaunchKernelGGL(err_epi_kernel, eg, eb, 0, stream, n, w.P, w.splits, sstride, Yu, w.part, nullptr);
  }
  hipLaunchKernelGGL(rows_err_kernel, dim3(1), eb, 0, stream, rows, nchunks, w.part,
                     rtn_err_out ? rtn_err_out : err_cur, w.status, nullptr, 0u);
  // gamma1 init from the RTN decision
  hipLaunchKernelGGL(sqdiff_part_kernel, eg, eb, 0, stream, n, pr.W, pr.ldw, pr.x_init, pr.ldw, w.part + 0);
  hipLaunchKernelGGL(rows_gamma_init_kernel, dim3(1), eb, 0, stream, rows, n, nchunks, w.part,
                     cfg.gamma_start, g1, g1w, w.status);
  MPQ_LAUNCH_CHECK();
  if ((rc = sync_status()) != kOk) return rc;
  if (hs->g1_invalid) {
    set_error("gamma1_init invalid: expected finite and > 1e-12.");
    set_error_code(kNumerical);
    return kNumerical;
  }
  const double rtn_err_mean = (double)hs->err_mean;
  // the caller's warm start first, then the requested precision (mpq/solver.py:486-489, :147-161)
  double obs;
  if (obs_init > 0.0) obs = obs_init;
  else if (cfg.obs_precision > 0.0) obs = cfg.obs_precision;
  else {
    float m = hs->err_sum / (float)(rows * n);  // mean over all rank-space entries
    obs = 1.0 / (double)(m < 1e-12f ? 1e-12f : m);
  }
  const double obs_initial = obs;
  const bool em_active = cfg.em_obs_precision && cfg.obs_precision <= 0.0;

  // r1 init
  if (cfg.init_from == 2) {
    MPQ_HIP_TRY(hipMemsetAsync(w.r1, 0, rows * n * 4, stream));
  } else {
    const float* src = cfg.init_from == 1 ? pr.W : pr.x_init;
    MPQ_HIP_TRY(copy_rows(w.r1, n * 4, src, pr.ldw * 4, rows, n * 4, stream));
  }
  // initial hard state = best
  if ((rc = hard_state(w.r1, g1, false)) != kOk) return rc;
  if ((rc = wait_status(mb, hard_seq, hs, stream)) != kOk) return rc;
  double best_err_mean = (double)hs->err_mean;
  std::swap(w.q_cur, w.q_best);
  std::swap(err_cur, err_best);
  std::swap(w.prod_cur, w.prod_best);
  double best_obs = obs;
  int best_iter = -1, stop_iter = -1;
  int a1_retry = 0, a2_clip = 0, g2_invalid = 0;
  double obs_sum = 0.0, a1_sum = 0.0, a2_sum = 0.0;
  int n_logged = 0;
  bool has_prev = false;
  const float damping = cfg.damping;
  const float retry_factor = cfg.gamma_retry_factor > 1.000001f ? cfg.gamma_retry_factor : 1.000001f;
  const int retry_steps = cfg.gamma_retry_steps > 0 ? cfg.gamma_retry_steps : 0;
  const int iters = cfg.iters > 0 ? cfg.iters : 0;

  bool g1w_current = true;  // g1w == g1 (the row kernels that write gamma1 also write g1w)
  // posterior denoiser of (r1, g1w) + the alpha1 row kernel, which publishes its status; returns the
  // status's sequence number
  auto launch_alpha1 = [&]() -> unsigned {
    hipLaunchKernelGGL(uniform_denoise_kernel<kPosterior>, eg, eb, 0, stream, w.r1, g1w, pr.W, pr.ldw,
                       pr.scale, pr.zero, G, pr.group_size, n, pr.maxq, tau, w.x1, w.part, nullptr,
                       nullptr, nullptr);
    const unsigned seq = ++mb->seq;
    hipLaunchKernelGGL(rows_alpha1_kernel, dim3(1), eb, 0, stream, rows, n, nchunks, w.part, g1w,
                       has_prev ? 1 : 0, damping, g2prev, a1raw, a1, eta1, g2new, g2, w.status, mb->dev(seq), seq);
    return seq;
  };
  // r2 message and the first LMMSE product (obs as used by this iteration).  They write only the
  // message, the product's partials, the LMMSE mean (in x1) and its row partials, which a gamma retry
  // recomputes from scratch (the retried denoiser rewrites x1), so the loop queues them behind the
  // first denoiser pass before that pass's status is read, and the GPU has work while the host
  // waits; after a retry (g1w rescaled) they run again from the retried pass.
  auto launch_lmmse_head = [&](float obs_f) -> int {
    hipLaunchKernelGGL(msg_r2_kernel, eg, eb, 0, stream, n, w.x1, w.r1, eta1, g1w, g2new,
                       has_prev ? 1 : 0, damping, w.r2prev, w.r2, planes);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(product(w, w.r2, pr.V, false, kOpV, rows, n, stream, planes != nullptr));
    hipLaunchKernelGGL(lmmse_epi1_kernel, eg, eb, 0, stream, n, w.P, w.splits, sstride, Yu, pr.S, g2,
                       obs_f, w.x1, w.part, planes);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  unsigned ahead_seq = 0;  // the iteration's first denoiser pass, launched at the end of the one before
  for (int it = 0; it < iters; ++it) {
    // ---- denoiser with gamma retries (mpq/solver.py:559-596), from g1w = g1
    if (ahead_seq == 0) {
      if (!g1w_current) MPQ_HIP_TRY(copy_rows(g1w, 0, g1, 0, 1, rows * 4, stream));
      g1w_current = true;
    }
    const float obs_f = (float)obs;
    bool head_queued = false;  // the LMMSE head of the pass whose status is read last
    for (int attempt = 0; attempt <= retry_steps; ++attempt) {
      unsigned a1_seq = ahead_seq;
      ahead_seq = 0;
      if (a1_seq == 0) {
        a1_seq = launch_alpha1();
        MPQ_LAUNCH_CHECK();
      }
      if (attempt == 0) {
        if ((rc = launch_lmmse_head(obs_f)) != kOk) return rc;
        head_queued = true;
      }
      if ((rc = wait_status(mb, a1_seq, hs, stream)) != kOk) return rc;
      if (hs->a1_invalid == 0) break;
      if (attempt >= retry_steps) {
        if (hs->a1_nonfinite) {
          set_error("alpha1 invalid: expected all in (1e-07, 1-1e-07).");
          set_error_code(kNumerical);
          return kNumerical;
        }
        break;  // clamped alpha1 already in place (before the queued head read it)
      }
      a1_retry += hs->a1_invalid;
      hipLaunchKernelGGL(rows_retry_kernel, dim3(1), eb, 0, stream, rows, a1raw, retry_factor, g1w);
      g1w_current = false;
      head_queued = false;
      MPQ_LAUNCH_CHECK();
    }
    if (hs->g2new_invalid || hs->g2_invalid) {  // mpq/solver.py:602-604, 613-615
      ++g2_invalid;
      continue;  // the queued head's results are never read
    }
    const float a1_mean_it = hs->a1_mean;
    // ---- LMMSE
    if (!head_queued && (rc = launch_lmmse_head(obs_f)) != kOk) return rc;
    hipLaunchKernelGGL(rows_lmmse_kernel, dim3(1), eb, 0, stream, rows, n, n, nchunks, w.part, g2, damping,
                       eta2, g1new, g1, g1w, w.status);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(product(w, w.x1, pr.V, true, kOpVt, rows, n, stream, planes != nullptr));
    // ---- r1 message and the hard state of the new (r1, g1)
    if (cfg.final_decision == 1) {
      hipLaunchKernelGGL(epi2_denoise_kernel<kHardRoundMean>, eg, eb, 0, stream, n, w.P, w.splits, sstride, w.r2,
                         eta2, g2, g1new, damping, w.r1, g1, pr.W, pr.ldw, pr.scale, pr.zero, G, pr.group_size,
                         pr.maxq, tau, w.q_cur, w.xs, planes);
    } else {
      hipLaunchKernelGGL(epi2_denoise_kernel<kHardMap>, eg, eb, 0, stream, n, w.P, w.splits, sstride, w.r2, eta2,
                         g2, g1new, damping, w.r1, g1, pr.W, pr.ldw, pr.scale, pr.zero, G, pr.group_size, pr.maxq,
                         tau, w.q_cur, w.xs, planes);
    }
    MPQ_LAUNCH_CHECK();
    if ((rc = hard_state(w.r1, g1, true)) != kOk) return rc;
    std::swap(w.r2, w.r2prev);  // r2_prev <- r2
    std::swap(g2, g2prev);      // gamma2_prev <- gamma2
    has_prev = true;
    // The next iteration's first denoiser pass reads only device state (r1, gamma1, and gamma2 of
    // this iteration), so it is queued before this iteration's status is read and the GPU works
    // through the host's EM and stopping decision.  After a stop its results are never read.
    if (it + 1 < iters) {
      if (!g1w_current) MPQ_HIP_TRY(copy_rows(g1w, 0, g1, 0, 1, rows * 4, stream));
      g1w_current = true;
      ahead_seq = launch_alpha1();
      MPQ_LAUNCH_CHECK();
    }
    if ((rc = wait_status(mb, hard_seq, hs, stream)) != kOk) return rc;
    a2_clip += hs->a2_clip;
    // EM update of the observation precision (mpq/linear.py:59-82), in double like the reference
    if (em_active) {
      float den = hs->em_mean < 1e-12f ? 1e-12f : hs->em_mean;
      const double beta_new = (double)n / (double)den;
      const double beta_old = obs > 1e-12 ? obs : 1e-12;
      const double d = cfg.em_obs_precision_damping;
      double beta;
      if (d >= 1.0) beta = beta_new;
      else if (d <= 0.0) beta = beta_old;
      else beta = std::exp((1.0 - d) * std::log(beta_old) + d * std::log(beta_new > 1e-12 ? beta_new : 1e-12));
      beta = std::min(std::max(beta, cfg.em_obs_precision_min), cfg.em_obs_precision_max);
      obs = beta;
    }
    obs_sum += obs;
    a1_sum += a1_mean_it;
    a2_sum += hs->a2_mean;
    ++n_logged;
    // best iterate (mpq/solver.py:678-699)
    const double cur = (double)hs->err_mean;
    const double tol = std::max(1e-10, std::fabs(best_err_mean) * 1e-8);
    if (cur + tol < best_err_mean) {
      std::swap(w.q_cur, w.q_best);
      std::swap(err_cur, err_best);
      std::swap(w.prod_cur, w.prod_best);
      best_err_mean = cur;
      best_obs = obs;
      best_iter = it;
    } else {
      obs = best_obs;
      stop_iter = it;
      break;
    }
  }

  // a stop leaves the look-ahead pass queued: wait for its status, so that no publish to the
  // mailbox is outstanding when this call returns (a later call may run on another stream)
  if (ahead_seq != 0) {
    VampStatus unused;
    if ((rc = wait_status(mb, ahead_seq, &unused, stream)) != kOk) return rc;
  }
  // ---- outputs
  MPQ_HIP_TRY(copy_rows(q_out, 0, w.q_best, 0, 1, rows * n, stream));
  if (err_out) MPQ_HIP_TRY(copy_rows(err_out, 0, err_best, 0, 1, rows * 4, stream));
  if (pr.xprod_out)
    MPQ_HIP_TRY(copy_rows(pr.xprod_out, 0, w.prod_best, 0, 1, rows * n * 4, stream));
  if (x_out) {
    MPQ_HIP_TRY(dequant_groups(w.q_best, pr.scale, pr.zero, G, pr.group_size, rows, n, x_out, stream));
  }
  if (stats) {
    stats->iters = iters;
    stats->best_iter = best_iter;
    stats->stop_iter = stop_iter;
    stats->alpha1_retry_count = a1_retry;
    stats->alpha2_clip_count = a2_clip;
    stats->gamma2_invalid_count = g2_invalid;
    stats->obs_precision_initial = obs_initial;
    stats->obs_precision_final = obs;
    stats->obs_precision_mean = n_logged ? obs_sum / n_logged : obs;
    stats->alpha1_mean = n_logged ? a1_sum / n_logged : 0.0;
    stats->alpha2_mean = n_logged ? a2_sum / n_logged : 0.0;
    stats->best_rankspace_error_mean = best_err_mean;
    stats->rtn_rankspace_error_mean = rtn_err_mean;
  }
  return kOk;
}

}  // namespace mpq

extern "C" int64_t mpq_uniform_vamp_workspace_size(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  return mpq::uniform_vamp_workspace_bytes(rows, n);
}

extern "C" int mpq_uniform_vamp_solve(int64_t rows, int64_t n, int maxq, const float* W, int64_t ldw,
                                      const float* x_init, const float* scale, const float* zero,
                                      int64_t group_size, const float* V, const float* S,
                                      const float* Vs, const MpqUniformVampConfig* cfg,
                                      double obs_init, uint8_t* q_out, float* x_out,
                                      float* err_out, float* rtn_err_out,
                                      MpqUniformVampStats* stats, void* workspace,
                                      int64_t workspace_bytes, hipStream_t stream) {
  return mpq_uniform_vamp_solve_ex(rows, n, maxq, W, ldw, x_init, scale, zero, group_size, V, S, Vs, cfg, obs_init,
                                   nullptr, nullptr, nullptr, q_out, x_out, err_out, rtn_err_out, nullptr, stats, workspace,
                                   workspace_bytes, stream);
}

extern "C" int mpq_uniform_vamp_solve_ex(int64_t rows, int64_t n, int maxq, const float* W, int64_t ldw,
                                         const float* x_init, const float* scale, const float* zero,
                                         int64_t group_size, const float* V, const float* S,
                                         const float* Vs, const MpqUniformVampConfig* cfg,
                                         double obs_init, const float* Yu_in, const float* xr_in,
                                         const float* packed, uint8_t* q_out, float* x_out, float* err_out,
                                         float* rtn_err_out,
                                         float* xprod_out, MpqUniformVampStats* stats, void* workspace,
                                         int64_t workspace_bytes, hipStream_t stream) {
  MPQ_CHECK_ARG(rows > 0 && n > 0, "mpq_uniform_vamp_solve: empty problem");
  MPQ_CHECK_ARG(maxq >= 1 && maxq <= 255, "mpq_uniform_vamp_solve: maxq must be in [1, 255]");
  MPQ_CHECK_ARG(W && x_init && scale && zero && V && S && Vs && cfg && q_out && workspace,
                "mpq_uniform_vamp_solve: null argument");
  MPQ_CHECK_ARG(group_size >= 1, "mpq_uniform_vamp_solve: group_size must be >= 1");
  MPQ_CHECK_ARG(ldw >= n, "mpq_uniform_vamp_solve: ldw < n");
  MPQ_CHECK_ARG(rows <= 65535, "mpq_uniform_vamp_solve: at most 65535 rows per block");
  mpq::UniformProblem pr{};
  pr.rows = rows; pr.n = n; pr.maxq = maxq; pr.W = W; pr.x_init = x_init; pr.scale = scale;
  pr.zero = zero; pr.group_size = group_size; pr.V = V; pr.S = S; pr.ldw = ldw;
  pr.Yu_in = Yu_in; pr.xr_in = xr_in; pr.xprod_out = xprod_out; pr.packed = packed;
  return mpq::uniform_vamp_solve(pr, Vs, *cfg, obs_init, q_out, x_out, err_out, rtn_err_out, stats,
                                 workspace, workspace_bytes, stream);
}

extern "C" int mpq_uniform_denoise(int64_t rows, int64_t n, int maxq, const float* r1, const float* gamma,
                                   const float* center, int64_t ld_center, const float* scale,
                                   const float* zero, int64_t group_size, float tau, float* mean,
                                   float* var, int64_t* map_idx, float* map_value, float* alpha1,
                                   hipStream_t stream) {
  MPQ_CHECK_ARG(rows >= 0 && n >= 0, "mpq_uniform_denoise: bad shape");
  if (rows == 0 || n == 0) return mpq::kOk;
  MPQ_CHECK_ARG(maxq >= 1 && maxq <= 255 && group_size >= 1, "mpq_uniform_denoise: bad maxq/group_size");
  MPQ_CHECK_ARG(r1 && gamma && center && scale && zero && mean && var && map_idx && map_value,
                "mpq_uniform_denoise: null argument");
  MPQ_CHECK_ARG(ld_center >= n && rows <= 65535, "mpq_uniform_denoise: bad ld/rows");
  const int64_t G = (n + group_size - 1) / group_size;
  const dim3 eg((unsigned)((n + mpq::kChunk - 1) / mpq::kChunk), (unsigned)rows);
  hipLaunchKernelGGL(mpq::uniform_denoise_kernel<mpq::kFull>, eg, dim3(mpq::kEW), 0, stream, r1, gamma, center,
                     ld_center, scale, zero, G, group_size, n, maxq, tau, mean, var,
                     reinterpret_cast<uint8_t*>(map_idx), map_value, nullptr);
  MPQ_LAUNCH_CHECK();
  if (alpha1) {
    hipLaunchKernelGGL(mpq::row_alpha_kernel, dim3((unsigned)rows), dim3(mpq::kEW), 0, stream, n, var, gamma,
                       alpha1);
    MPQ_LAUNCH_CHECK();
  }
  return mpq::kOk;
}
