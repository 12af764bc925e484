// E8P12-prior VAMP on one row block (gfx950).
//
// Replaces mpq/solver.py:853-1138 (solve_e8p12_rankspace_vamp up to the polish, which
// is mpq_e8p12_cd_polish): the denoiser is the E8P12 posterior (mpq_e8p12_denoise),
// the linear module, EM and messages are the kernels shared with the uniform driver
// (vamp_common.h), the final decision is the factorized MAP of (r1, gamma1)
// (mpq/solver.py:1124-1138).  best_iterate (off in the recipe) is supported.
// Host control flow with two small status reads per iteration.
#include <algorithm>
#include <cmath>

#include "gemm.h"
#include "kernels.h"
#include "mpq_amd.h"
#include "vamp_common.h"

namespace mpq {

hipError_t e8p12_posterior(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                           const float* center, const float* scale, float tau, const float* map_vals,
                           float* x1, float* var, hipStream_t stream, float* var_wg);

namespace {

inline int64_t a64(int64_t v) { return (v + 63) / 64 * 64; }

// out[b] = sum_j var[b * nb + j], one work-group per row (fixed reduction order).
__global__ __launch_bounds__(kEW) void row_sum_kernel(int64_t nb, const float* __restrict__ var,
                                                      float* __restrict__ out) {
  __shared__ float red[kEW / 64];
  const int64_t b = blockIdx.x;
  float acc = 0.f;
  for (int64_t j = threadIdx.x; j < nb; j += blockDim.x) acc += var[b * nb + j];
  const float t = block_sum(acc, red);
  if (threadIdx.x == 0) out[b] = t;
}

struct E8Plan {
  int64_t rows, n, nb, nchunks;
  int splits, bn;
  int splits_x6;     // 0 if the shape has no x6 path
  int64_t ap_bytes;  // packed bf16 planes of a product's left operand (x6 path)
  int64_t bytes;
};

E8Plan e8_plan(int64_t rows, int64_t n) {
  E8Plan p;
  p.rows = rows;
  p.n = n;
  p.nb = n / 8;
  p.nchunks = (n + kChunk - 1) / kChunk;
  int bn = 128;
  p.splits = choose_splits(rows, n, n, (int64_t)1 << 62, &bn);
  p.bn = bn;
  p.splits_x6 = x6_shape_ok(n, n) ? x6_choose_splits(rows, n, n) : 0;
  p.ap_bytes = p.splits_x6 ? (x6_packed_a_bytes(rows, n) + 255) / 256 * 256 : 0;
  const int64_t mat = a64(rows * n) * 4;
  int64_t b = 7 * mat;                          // Yu r1 r2 r2prev x1 map_vals r1_best
  b += (int64_t)std::max(p.splits, p.splits_x6) * mat;  // partials
  b += p.ap_bytes;                              // packed left operand (x6 path)
  b += a64(rows * p.nb) * 4;                    // var1
  b += a64(rows * p.nb) * 8;                    // map idx
  b += a64(16 * rows) * 4;                      // row arrays
  b += a64(3 * rows * p.nchunks) * 4;           // chunk partials
  b += a64(rows * ((p.nb + 63) / 64)) * 4;      // per-work-group variance sums of the posterior
  b += 256;                                     // status
  p.bytes = b;
  return p;
}

VampStatus* host_status_e8() {
  static thread_local VampStatus* h = nullptr;
  if (!h) {
    if (hipHostMalloc((void**)&h, sizeof(VampStatus), hipHostMallocDefault) != hipSuccess) h = nullptr;
    else track_pinned(reinterpret_cast<void**>(&h), nullptr, nullptr);
  }
  return h;
}

hipError_t product(const float* A, const float* B, bool trans_b, int64_t rows, int64_t n, float* P, int splits,
                   int bn, hipStream_t stream) {
  GemmParams p{};
  p.M = rows; p.N = n; p.K = n;
  p.A = A; p.lda = n; p.B = B; p.ldb = n; p.trans_b = trans_b;
  p.C = P; p.ldc = n; p.split_stride = a64(rows * n);
  p.alpha = 1.f; p.beta = 0.f; p.mode = kGemmPartials;
  return gemm_partials(p, splits, bn, stream);
}

}  // namespace
}  // namespace mpq

extern "C" int mpq_e8p12_map(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                             const float* center, const float* scale, float tau, int64_t* idx64,
                             uint16_t* idx16, float* vals, float* err, float* score, hipStream_t stream);

extern "C" int64_t mpq_e8p12_vamp_workspace_size(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0 || n % 8) return 0;
  return mpq::e8_plan(rows, n).bytes;
}

extern "C" int mpq_e8p12_vamp_solve(int64_t rows, int64_t n, const float* Wr, const float* hat_init,
                                    const float* V, const float* S, const float* Vs, const float* prior_scale,
                                    const MpqE8P12VampConfig* cfg, double obs_init, int64_t* idx_out,
                                    float* hat_out, float* err_out, float* r1_out, float* gamma1_out,
                                    MpqE8P12VampStats* stats, void* workspace, int64_t workspace_bytes,
                                    hipStream_t stream) {
  return mpq_e8p12_vamp_solve_ex(rows, n, Wr, hat_init, V, S, Vs, prior_scale, cfg, obs_init, nullptr, idx_out,
                                 hat_out, err_out, r1_out, gamma1_out, stats, workspace, workspace_bytes, stream);
}

extern "C" int mpq_e8p12_vamp_solve_ex(int64_t rows, int64_t n, const float* Wr, const float* hat_init,
                                       const float* V, const float* S, const float* Vs, const float* prior_scale,
                                       const MpqE8P12VampConfig* cfg, double obs_init, const float* packed,
                                       int64_t* idx_out, float* hat_out, float* err_out, float* r1_out,
                                       float* gamma1_out, MpqE8P12VampStats* stats, void* workspace,
                                       int64_t workspace_bytes, hipStream_t stream) {
  using namespace mpq;
  MPQ_CHECK_ARG(rows > 0 && n > 0 && n % 8 == 0, "E8P12 solver expects n divisible by 8; got n=%lld",
                (long long)n);
  MPQ_CHECK_ARG(rows <= 65535, "mpq_e8p12_vamp_solve: at most 65535 rows per block");
  MPQ_CHECK_ARG(Wr && hat_init && V && S && Vs && cfg && idx_out && hat_out && workspace,
                "mpq_e8p12_vamp_solve: null argument");
  const E8Plan pl = e8_plan(rows, n);
  MPQ_CHECK_ARG(workspace_bytes >= pl.bytes, "mpq_e8p12_vamp_solve: workspace too small (%lld < %lld)",
                (long long)workspace_bytes, (long long)pl.bytes);
  VampStatus* hs = host_status_e8();
  MPQ_CHECK_ARG(hs != nullptr, "mpq_e8p12_vamp_solve: pinned status buffer unavailable");
  const int64_t nb = pl.nb;
  const int nchunks = (int)pl.nchunks;
  const int64_t mat = a64(rows * n) * 4;
  const int64_t sstride = a64(rows * n);
  char* p = static_cast<char*>(workspace);
  float* Yu = (float*)p; p += mat;
  float* r1 = (float*)p; p += mat;
  float* r2 = (float*)p; p += mat;
  float* r2prev = (float*)p; p += mat;
  float* x1 = (float*)p; p += mat;
  float* mvals = (float*)p; p += mat;
  float* r1_best = (float*)p; p += mat;
  float* P = (float*)p; p += (int64_t)std::max(pl.splits, pl.splits_x6) * mat;
  void* Ap = p; p += pl.ap_bytes;
  float* var1 = (float*)p; p += a64(rows * nb) * 4;
  int64_t* midx = (int64_t*)p; p += a64(rows * nb) * 8;
  float* rowbuf = (float*)p; p += a64(16 * rows) * 4;
  float* part = (float*)p; p += a64(3 * rows * nchunks) * 4;
  float* var_wg = (float*)p; p += a64(rows * ((nb + 63) / 64)) * 4;
  VampStatus* status = (VampStatus*)p;
  float* g1 = rowbuf + 0 * rows;
  float* g1w = rowbuf + 1 * rows;
  float* a1raw = rowbuf + 2 * rows;
  float* a1 = rowbuf + 3 * rows;
  float* eta1 = rowbuf + 4 * rows;
  float* g2new = rowbuf + 5 * rows;
  float* g2 = rowbuf + 6 * rows;
  float* g2prev = rowbuf + 7 * rows;
  float* eta2 = rowbuf + 8 * rows;  // 3 rows: eta2, EM row stat, alpha2
  float* g1new = rowbuf + 11 * rows;
  float* errrow = rowbuf + 12 * rows;
  float* g1_best = rowbuf + 13 * rows;
  float* varsum = rowbuf + 14 * rows;
  const dim3 eg((unsigned)nchunks, (unsigned)rows), eb(kEW);
  const float tau = cfg->prior_tau;
  const float* center = tau > 0.f ? Wr : nullptr;
  HostMailbox* mb = host_mailbox();
  MPQ_CHECK_ARG(mb != nullptr, "E8P12 VAMP: mapped status mailbox unavailable");
  auto sync_status = [&]() -> int { return read_status(mb, status, hs, stream); };
  // rank-space products: on the packed operator (x6, bf16 matrix cores) when given, else fp32 MFMA;
  // `op` indexes the packed operator (0: V for r V, 1: V for x V^T, 2: Vs for x Vs)
  const bool x6 = packed != nullptr && pl.splits_x6 > 0;
  const int nsplit = x6 ? pl.splits_x6 : pl.splits;
  uint4* const planes = x6 ? static_cast<uint4*>(Ap) : nullptr;  // written by msg_r2 / lmmse_epi1
  auto prod = [&](const float* A, const float* B, bool trans_b, int op, bool a_planes_written = false) -> hipError_t {
    if (x6) {
      if (!a_planes_written) {  // else the kernel that produced A wrote its planes into Ap
        hipError_t e = x6_pack_a(A, n, rows, n, Ap, stream);
        if (e != hipSuccess) return e;
      }
      return x6_gemm_partials(Ap, packed + (int64_t)op * n * n, rows, n, n, P, n, sstride, nsplit, stream);
    }
    return product(A, B, trans_b, rows, n, P, pl.splits, pl.bn, stream);
  };
  int rc;
  // MAP decision of (r, g) into midx / mvals and its rank-space error into errrow / status.err_mean
  // MAP decision of (r, g) and its rank-space error; with pub_seq != 0 the error row kernel also
  // publishes the status under that sequence number
  auto map_state = [&](const float* r, const float* g, unsigned pub_seq = 0u) -> int {
    int e = mpq_e8p12_map(r, rows * nb, g, nb, center, prior_scale, tau, midx, nullptr, mvals, nullptr, nullptr,
                          stream);
    if (e != kOk) return e;
    MPQ_HIP_TRY(prod(mvals, Vs, false, 2));
    hipLaunchKernelGGL(err_epi_kernel, eg, eb, 0, stream, n, P, nsplit, sstride, Yu, part, nullptr);
    hipLaunchKernelGGL(rows_err_kernel, dim3(1), eb, 0, stream, rows, nchunks, part, errrow, status,
                       pub_seq ? mb->dev(pub_seq) : nullptr, pub_seq);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };

  // ---- setup: Yu, gamma1, obs warm start
  MPQ_HIP_TRY(prod(Wr, Vs, false, 2));
  MPQ_HIP_TRY(splitk_reduce(P, nsplit, rows, n, Yu, n, 1.f, 0.f, stream));
  MPQ_HIP_TRY(prod(hat_init, Vs, false, 2));
  hipLaunchKernelGGL(err_epi_kernel, eg, eb, 0, stream, n, P, nsplit, sstride, Yu, part, nullptr);
  hipLaunchKernelGGL(rows_err_kernel, dim3(1), eb, 0, stream, rows, nchunks, part, errrow, status, nullptr, 0u);
  hipLaunchKernelGGL(sqdiff_part_kernel, eg, eb, 0, stream, n, Wr, n, hat_init, n, part);
  hipLaunchKernelGGL(rows_gamma_init_kernel, dim3(1), eb, 0, stream, rows, n, nchunks, part, cfg->gamma_start, g1,
                     nullptr,
                     status);
  MPQ_LAUNCH_CHECK();
  if ((rc = sync_status()) != kOk) return rc;
  if (hs->g1_invalid) {
    set_error("gamma1_init invalid: expected finite and > 1e-12.");
    set_error_code(kNumerical);
    return kNumerical;
  }
  double obs;
  if (cfg->obs_precision > 0.0) obs = cfg->obs_precision;
  else if (obs_init > 0.0) obs = obs_init;
  else {
    float mm = hs->err_sum / (float)(rows * n);
    obs = 1.0 / (double)(mm < 1e-12f ? 1e-12f : mm);
  }
  const double obs_initial = obs;
  const bool em_active = cfg->em_obs_precision && cfg->obs_precision <= 0.0;
  MPQ_HIP_TRY(copy_rows(r1, 0, hat_init, 0, 1, rows * n * 4, stream));

  const bool best_iterate = cfg->best_iterate != 0;
  double best_err_mean = INFINITY;
  double best_obs = obs;
  auto snapshot = [&](float* rd, float* gd, const float* rs, const float* gs) -> int {
    MPQ_HIP_TRY(copy_rows(rd, 0, rs, 0, 1, rows * n * 4, stream));
    MPQ_HIP_TRY(copy_rows(gd, 0, gs, 0, 1, rows * 4, stream));
    return kOk;
  };
  if (best_iterate) {
    // best-iterate bookkeeping (mpq/solver.py:940-958)
    if ((rc = map_state(r1, g1)) != kOk) return rc;
    if ((rc = snapshot(r1_best, g1_best, r1, g1)) != kOk) return rc;
    if ((rc = sync_status()) != kOk) return rc;
    best_err_mean = (double)hs->err_mean;
  }
  int best_iter = -1, stop_iter = -1, a1_retry = 0, a2_clip = 0, g2_invalid = 0, n_logged = 0;
  int reported_iters = cfg->iters > 0 ? cfg->iters : 0;
  double obs_sum = 0.0, a1_sum = 0.0, a2_sum = 0.0;
  bool has_prev = false;
  const float damping = cfg->damping;
  const float retry_factor = cfg->gamma_retry_factor > 1.000001f ? cfg->gamma_retry_factor : 1.000001f;
  const int retry_steps = cfg->gamma_retry_steps > 0 ? cfg->gamma_retry_steps : 0;
  const int iters = cfg->iters > 0 ? cfg->iters : 0;
  // posterior denoiser of (r1, g1w) + the alpha1 row kernel, which publishes its status under *seq
  auto launch_alpha1 = [&](unsigned* seq) -> int {
    int e = mpq_e8p12_map(r1, rows * nb, g1w, nb, center, prior_scale, tau, nullptr, nullptr, mvals, nullptr, nullptr,
                          stream);
    if (e != kOk) return e;
    // a row's variances: whole work-groups of the posterior (nb % 64 == 0), summed in the row kernel,
    // else a reduction launch of its own
    const bool wg_rows = nb % 64 == 0;
    MPQ_HIP_TRY(e8p12_posterior(r1, rows * nb, g1w, nb, center, prior_scale, tau, mvals, x1, var1, stream,
                                wg_rows ? var_wg : nullptr));
    if (!wg_rows) hipLaunchKernelGGL(row_sum_kernel, dim3((unsigned)rows), eb, 0, stream, nb, var1, varsum);
    *seq = ++mb->seq;
    hipLaunchKernelGGL(rows_alpha1_kernel, dim3(1), eb, 0, stream, rows, nb, wg_rows ? (int)(nb / 64) : 1,
                       wg_rows ? var_wg : varsum, g1w, has_prev ? 1 : 0,
                       damping, g2prev, a1raw, a1, eta1, g2new, g2, status, mb->dev(*seq), *seq);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  // r2 message and the first LMMSE product: they write only the message, the product's partials, the
  // LMMSE mean (in x1) and its row partials, which a gamma retry recomputes (the retried posterior
  // rewrites x1), so they are queued behind the first denoiser pass before its status is read
  auto launch_lmmse_head = [&](float obs_f) -> int {
    hipLaunchKernelGGL(msg_r2_kernel, eg, eb, 0, stream, n, x1, r1, eta1, g1w, g2new, has_prev ? 1 : 0, damping,
                       r2prev, r2, planes);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(prod(r2, V, false, 0, planes != nullptr));
    hipLaunchKernelGGL(lmmse_epi1_kernel, eg, eb, 0, stream, n, P, nsplit, sstride, Yu, S, g2, obs_f, x1, part,
                       planes);
    MPQ_LAUNCH_CHECK();
    return kOk;
  };
  unsigned ahead_seq = 0;  // the iteration's first denoiser pass, launched at the end of the one before
  for (int it = 0; it < iters; ++it) {
    if (ahead_seq == 0) MPQ_HIP_TRY(copy_rows(g1w, 0, g1, 0, 1, rows * 4, stream));
    const float obs_f = (float)obs;
    bool head_queued = false;  // the LMMSE head of the pass whose status is read last
    for (int attempt = 0; attempt <= retry_steps; ++attempt) {
      unsigned a1_seq = ahead_seq;
      ahead_seq = 0;
      if (a1_seq == 0 && (rc = launch_alpha1(&a1_seq)) != kOk) return rc;
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
      head_queued = false;
      MPQ_LAUNCH_CHECK();
    }
    if (hs->g2new_invalid || hs->g2_invalid) {
      ++g2_invalid;
      continue;  // the queued head's results are never read
    }
    const float a1_mean_it = hs->a1_mean;
    if (!head_queued && (rc = launch_lmmse_head(obs_f)) != kOk) return rc;
    // without best-iterate tracking the row kernel publishes this iteration's status (its EM statistic
    // and alpha2 clips are all the host reads); with it the hard state's row kernel does, after it
    const unsigned st_seq = best_iterate ? 0u : ++mb->seq;
    // the row kernel also writes the next iteration's working gamma1 (g1w = the damped gamma1)
    hipLaunchKernelGGL(rows_lmmse_kernel, dim3(1), eb, 0, stream, rows, n, n, nchunks, part, g2, damping, eta2,
                       g1new, g1, g1w, status, best_iterate ? nullptr : mb->dev(st_seq), st_seq);
    MPQ_LAUNCH_CHECK();
    MPQ_HIP_TRY(prod(x1, V, true, 1, planes != nullptr));
    hipLaunchKernelGGL(lmmse_epi2_kernel, eg, eb, 0, stream, n, P, nsplit, sstride, r2, eta2, g2, g1new, damping,
                       r1);
    MPQ_LAUNCH_CHECK();
    const unsigned wait_seq = best_iterate ? ++mb->seq : st_seq;
    if (best_iterate) {
      if ((rc = map_state(r1, g1, wait_seq)) != kOk) return rc;
    }
    std::swap(r2, r2prev);
    std::swap(g2, g2prev);
    has_prev = true;
    // The next iteration's first denoiser pass reads only device state (r1, gamma1, and gamma2 of
    // this iteration), so it is queued before this iteration's status is read.  It writes none of
    // r1, gamma1 or the MAP decision the loop keeps, so a stop (which restores the best r1, gamma1
    // and decides again) never reads its results.
    if (it + 1 < iters) {
      if ((rc = launch_alpha1(&ahead_seq)) != kOk) return rc;
    }
    if ((rc = wait_status(mb, wait_seq, hs, stream)) != kOk) return rc;
    a2_clip += hs->a2_clip;
    if (em_active) {
      const float den = hs->em_mean < 1e-12f ? 1e-12f : hs->em_mean;
      const double beta_new = (double)n / (double)den;
      const double beta_old = obs > 1e-12 ? obs : 1e-12;
      const double d = cfg->em_obs_precision_damping;
      double beta;
      if (d >= 1.0) beta = beta_new;
      else if (d <= 0.0) beta = beta_old;
      else beta = std::exp((1.0 - d) * std::log(beta_old) + d * std::log(beta_new > 1e-12 ? beta_new : 1e-12));
      beta = std::min(std::max(beta, cfg->em_obs_precision_min), cfg->em_obs_precision_max);
      obs = beta;
    }
    obs_sum += obs;
    a1_sum += a1_mean_it;
    a2_sum += hs->a2_mean;
    ++n_logged;
    if (best_iterate) {
      // keep the iterate whose MAP decision has the smallest rank-space error; stop at the
      // first iterate that does not improve and restore the best (mpq/solver.py:1083-1121)
      const double cur = (double)hs->err_mean;
      const double tol = std::max(1e-10, std::fabs(best_err_mean) * 1e-8);
      if (cur + tol < best_err_mean) {
        best_err_mean = cur;
        best_obs = obs;
        best_iter = it;
        if ((rc = snapshot(r1_best, g1_best, r1, g1)) != kOk) return rc;
      } else {
        if ((rc = snapshot(r1, g1, r1_best, g1_best)) != kOk) return rc;
        obs = best_obs;
        stop_iter = it;
        reported_iters = it + 1;
        break;
      }
    }
  }
  // ---- final MAP decision and its error (mpq/solver.py:1124-1138)
  if ((rc = map_state(r1, g1)) != kOk) return rc;
  if ((rc = sync_status()) != kOk) return rc;
  MPQ_HIP_TRY(copy_rows(idx_out, 0, midx, 0, 1, rows * nb * 8, stream));
  MPQ_HIP_TRY(copy_rows(hat_out, 0, mvals, 0, 1, rows * n * 4, stream));
  if (err_out) MPQ_HIP_TRY(copy_rows(err_out, 0, errrow, 0, 1, rows * 4, stream));
  if (r1_out) MPQ_HIP_TRY(copy_rows(r1_out, 0, r1, 0, 1, rows * n * 4, stream));
  if (gamma1_out) MPQ_HIP_TRY(copy_rows(gamma1_out, 0, g1, 0, 1, rows * 4, stream));
  if (stats) {
    stats->iters = reported_iters;
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
    stats->rankspace_error_mean = (double)hs->err_mean;
  }
  return kOk;
}
