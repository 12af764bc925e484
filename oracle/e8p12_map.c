/*
 * ORACLE — test infrastructure only.  Nothing in the product links this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * as the checker.
 *
 * CPU restatement of MPQ's factorized E8P12 MAP search:
 *   mpq/priors/e8p12.py:367-449  (_branch_factorized_map)
 *   mpq/priors/e8p12.py:541-631  (vamp_vector_map_e8p12, incl. prior folding :556-574)
 *
 * Operation order follows the reference's torch CPU evaluation exactly:
 *   a_i      = (gamma * y_i) * abs_ki                       (e8p12.py:395)
 *   y_norm   = sum_i y_i*y_i, left to right                 (:396; torch CPU sums an
 *                                                             8-wide inner dim sequentially)
 *   const    = (-0.5*gamma) * (y_norm + sqnorm_k)           (:397)
 *   sum_abs  = sum_i |a_i|, left to right                   (:400)
 *   min_abs  = min_i |a_i|, first index wins for argmin     (:403-404)
 *   parity   = popcount(a_i < 0) & 1                        (:401-402)
 *   linear   = sum_abs - 2*mismatch*min_abs                 (:409)
 *   score    = const + linear                               (:410)
 *   best     = first argmax over flattened (branch*256 + k)  (:603-607)
 *   idx      = idx_lut[branch][k][sign_id]                  (:412, :609-610)
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no vector contraction).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline int parity8(unsigned v) { return __builtin_popcount(v & 255u) & 1; }

/* One block of 8, with precision g (already prior-folded). */
static void map_one(const float *rv, float g, const float *base_abs, const float *base_sqnorm,
                    const int32_t *base_parity, const int64_t *idx_lut, int64_t *idx_out,
                    float *score_out) {
  const float offsets[2] = {0.25f, -0.25f};
  float best = -INFINITY;
  int best_flat = -1;
  int best_sign = 0;
  for (int br = 0; br < 2; ++br) {
    float y[8];
    for (int i = 0; i < 8; ++i) y[i] = rv[i] - offsets[br];
    float yn = 0.0f;
    for (int i = 0; i < 8; ++i) {
      float sq = y[i] * y[i];
      yn = (i == 0) ? sq : yn + sq;
    }
    float gy[8];
    for (int i = 0; i < 8; ++i) gy[i] = g * y[i];
    const float mhalf_g = -0.5f * g;
    for (int k = 0; k < 256; ++k) {
      const float *ab = base_abs + 8 * k;
      float sum_abs = 0.0f, min_abs = 0.0f;
      int min_pos = 0;
      unsigned neg_bits = 0;
      for (int i = 0; i < 8; ++i) {
        float a = gy[i] * ab[i];
        float aa = fabsf(a);
        if (a < 0.0f) neg_bits |= 1u << i;
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
      int mismatch = parity8(neg_bits) != base_parity[k];
      unsigned sign_id = mismatch ? (neg_bits ^ (1u << min_pos)) : neg_bits;
      float linear = sum_abs - (2.0f * (float)mismatch) * min_abs;
      float cst = mhalf_g * (yn + base_sqnorm[k]);
      float score = cst + linear;
      if (best_flat < 0 || score > best) {
        best = score;
        best_flat = br * 256 + k;
        best_sign = (int)sign_id;
      }
    }
  }
  int br = best_flat >> 8, k = best_flat & 255;
  *idx_out = idx_lut[((int64_t)br * 256 + k) * 256 + best_sign];
  if (score_out) *score_out = best;
}

/*
 * r: n x 8 fp32.  gamma: one value per `gamma_div` consecutive vectors.
 * center/scale (optional, may be NULL): prior folding of e8p12.py:561-574 with
 * tau2 = (max(tau,1e-12)*scale)^2, prec = 1/tau2, g = gamma + prec,
 * r_work = (gamma*r + prec*center) / g.
 */
void oracle_e8p12_map(const float *r, int64_t n, const float *gamma, int64_t gamma_div,
                      const float *center, const float *scale, float tau,
                      const float *base_abs, const float *base_sqnorm,
                      const int32_t *base_parity, const int64_t *idx_lut, int64_t *idx_out,
                      float *score_out) {
  const float tau_c = tau > 1e-12f ? tau : 1e-12f;
  for (int64_t v = 0; v < n; ++v) {
    float g = gamma[v / gamma_div];
    float rw[8];
    if (center != 0 && tau > 0.0f) {
      float s = scale[v] < 1e-12f ? 1e-12f : scale[v];
      float ts = tau_c * s;
      float tau2 = ts * ts;
      float prec = 1.0f / tau2;
      float gw = g + prec;
      for (int i = 0; i < 8; ++i) {
        float num = g * r[8 * v + i] + prec * center[8 * v + i];
        rw[i] = num / gw;
      }
      g = gw;
    } else {
      memcpy(rw, r + 8 * v, sizeof(rw));
    }
    map_one(rw, g, base_abs, base_sqnorm, base_parity, idx_lut, idx_out + v,
            score_out ? score_out + v : 0);
  }
}

/* Squared error ||x - grid[idx]||^2, summed left to right. */
void oracle_e8p12_sqerr(const float *x, const int64_t *idx, int64_t n, const float *grid,
                        float *err_out) {
  for (int64_t v = 0; v < n; ++v) {
    const float *c = grid + 8 * idx[v];
    float e = 0.0f;
    for (int i = 0; i < 8; ++i) {
      float d = x[8 * v + i] - c[i];
      float sq = d * d;
      e = (i == 0) ? sq : e + sq;
    }
    err_out[v] = e;
  }
}

/* Exhaustive nearest codeword over all 65536 entries in double (first index on ties). */
void oracle_e8p12_bruteforce(const float *x, int64_t n, const float *grid, int64_t *idx_out,
                             double *dist_out) {
  for (int64_t v = 0; v < n; ++v) {
    double best = INFINITY;
    int64_t bi = 0;
    for (int64_t c = 0; c < 65536; ++c) {
      double d = 0.0;
      for (int i = 0; i < 8; ++i) {
        double t = (double)x[8 * v + i] - (double)grid[8 * c + i];
        d += t * t;
      }
      if (d < best) {
        best = d;
        bi = c;
      }
    }
    idx_out[v] = bi;
    if (dist_out) dist_out[v] = best;
  }
}
