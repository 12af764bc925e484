/*
 * mpq_amd — C-ABI of the MI355X (gfx950) per-layer quantization hot path.
 *
 * Conventions (all entry points):
 *  - every buffer is caller-allocated device memory, row-major and contiguous
 *    unless a leading dimension is given, fp32 unless stated;
 *  - work is enqueued on `stream` (a hipStream_t; NULL = default stream);
 *    entry points are asynchronous except the VAMP drivers
 *    (mpq_uniform_vamp_solve, mpq_e8p12_vamp_solve), which read small status
 *    blocks back to run the reference's host-side control flow, and
 *    mpq_e8p12_cd_prepare, which reads back one failure count;
 *  - scratch memory comes from the caller (`workspace`, sized by the matching
 *    *_workspace_size query); no entry point allocates device memory;
 *  - the return value is 0 on success, MPQ_INVALID_ARGUMENT (-1) for a bad
 *    shape/argument (nothing launched), MPQ_HIP_ERROR (-2) for a HIP failure,
 *    MPQ_NUMERICAL_ERROR (-4) for the reference's numerical fail-closed checks;
 *    mpq_last_error() returns a thread-local message;
 *  - no C++ exception crosses this boundary.
 */
#ifndef MPQ_AMD_H_
#define MPQ_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mpq_stream_t; /* == hipStream_t */

#define MPQ_OK 0
#define MPQ_INVALID_ARGUMENT (-1)
#define MPQ_HIP_ERROR (-2)
#define MPQ_NUMERICAL_ERROR (-4)

/* Thread-local description of the last failed call ("" if none). */
const char* mpq_last_error(void);
int mpq_last_error_code(void);
void mpq_clear_error(void);

/*
 * Frees the calling thread's pinned host buffers (the VAMP drivers' status mailboxes and the
 * eigensolver's staging buffers); a later call that needs one allocates it again.  Waits for the
 * device to finish first.  No counterpart in the reference (its torch calls keep no such state);
 * the Python binding calls it at interpreter exit so that no library allocation outlives the
 * HIP runtime's teardown.
 */
int mpq_release_thread_resources(void);

/* ------------------------------------------------------------------------ */
/* E8P12 lattice codebook                                                   */
/* ------------------------------------------------------------------------ */

/*
 * E8P12 MAP / nearest-codeword search over n 8-dim blocks.
 * Replaces mpq/priors/e8p12.py:541-631 (vamp_vector_map_e8p12) and its
 * factorized per-branch search mpq/priors/e8p12.py:367-449; with gamma == 1 and
 * no prior it is the codebook's exact nearest-codeword quantizer
 * (cb.quantize, called at mpq/adapters/quip_sharp.py:235).
 *   r        n x 8 inputs
 *   gamma    precision, one value per `gamma_div` consecutive blocks
 *            (gamma_div = blocks per weight row for a (B, 1) gamma)
 *   center   optional n x 8 prior centre; the prior is folded in when
 *            center != NULL and tau > 0 (mpq/priors/e8p12.py:561-574)
 *   scale    optional n prior scales; NULL = abs-max of the centre block
 *   outputs (any may be NULL, at least one required):
 *            idx64 (n int64), idx16 (n uint16), vals (n x 8 codeword),
 *            err (n, ||r - codeword||^2), score (n, best log-score)
 * Indices are bit-exact with oracle/e8p12_map.c (first index on ties).
 */
int mpq_e8p12_map(const float* r, int64_t n, const float* gamma, int64_t gamma_div,
                  const float* center, const float* scale, float tau, int64_t* idx64,
                  uint16_t* idx16, float* vals, float* err, float* score, mpq_stream_t stream);

/*
 * E8P12 posterior denoiser for rows x nb 8-blocks: posterior mean x1 (rows*nb x 8),
 * per-block variance var (rows*nb), MAP index (int64, optional) and codeword
 * map_vals (rows*nb x 8), alpha1 = gamma_row * mean(var) (rows, optional).
 * Prior folding as mpq_e8p12_map.  Blocks whose folded precision is >= 1e3 snap to
 * the MAP codeword with zero variance.  Replaces mpq/priors/e8p12.py:815-968
 * (vamp_vector_discrete_mmse_e8p12, without diagnostics) and its per-branch
 * statistics mpq/priors/e8p12.py:169-308.
 */
int mpq_e8p12_denoise(const float* r, int64_t rows, int64_t nb, const float* gamma,
                      const float* center, const float* scale, float tau, float* x1, float* var,
                      int64_t* map_idx, float* map_vals, float* alpha1, mpq_stream_t stream);

/*
 * Posterior diagnostics of the E8P12 denoiser for rows x nb 8-blocks (any output may be NULL, one
 * required): logz (rows*nb) = log-partition over the 2^16 codewords, entropy (rows*nb) = entropy of
 * the posterior (mixture over the 512 components plus their sign entropies), margin (rows*nb) = gap
 * between the two largest candidate log-scores (each component's best and second-best sign
 * pattern).  Prior folding as mpq_e8p12_map.  Replaces the need_stats / return_*_blocks outputs of
 * mpq/priors/e8p12.py:815-968 (vamp_vector_discrete_mmse_e8p12) and the margin of
 * mpq/priors/e8p12.py:541-631 (vamp_vector_map_e8p12), per-branch terms mpq/priors/e8p12.py:276-305.
 */
int mpq_e8p12_posterior_stats(const float* r, int64_t rows, int64_t nb, const float* gamma,
                              const float* center, const float* scale, float tau, float* logz,
                              float* entropy, float* margin, mpq_stream_t stream);

/* Mirrors E8P12VampConfig (mpq/solver.py:59-82) without the polish fields. */
typedef struct MpqE8P12VampConfig {
  int iters;
  float damping;
  float gamma_start;
  float gamma_retry_factor;
  int gamma_retry_steps;
  float prior_tau;
  double obs_precision; /* > 0: fixed observation precision (EM off) */
  int em_obs_precision;
  double em_obs_precision_damping;
  double em_obs_precision_min;
  double em_obs_precision_max;
  int best_iterate;
} MpqE8P12VampConfig;

/* Per-solve statistics (subset of mpq/solver.py:1236-1276). */
typedef struct MpqE8P12VampStats {
  int iters;
  int best_iter;
  int stop_iter;
  int alpha1_retry_count;
  int alpha2_clip_count;
  int gamma2_invalid_count;
  double obs_precision_initial;
  double obs_precision_final;
  double obs_precision_mean;
  double alpha1_mean;
  double alpha2_mean;
  double rankspace_error_mean; /* of the final MAP decision */
} MpqE8P12VampStats;

/* Workspace bytes needed by mpq_e8p12_vamp_solve for a rows x n block. */
int64_t mpq_e8p12_vamp_workspace_size(int64_t rows, int64_t n);

/*
 * E8P12-prior VAMP on one row block, without the polish: replaces
 * mpq/solver.py:853-1138 (solve_e8p12_rankspace_vamp up to the polish) with the
 * posterior denoiser of mpq_e8p12_denoise, the LMMSE/EM/error steps shared with
 * mpq_uniform_vamp_solve and the final factorized MAP (mpq/solver.py:1124-1138).
 *   Wr, hat_init: rows x n (n % 8 == 0); V, Vs: n x n; S: n
 *   prior_scale: rows*n/8 block scales (NULL: absmax of each Wr block)
 *   idx_out: rows x n/8 int64 codeword indices, hat_out rows x n codewords,
 *   err_out (rows), r1_out (rows x n), gamma1_out (rows): optional
 *   obs_init > 0 is the warm start of the observation precision; cfg->obs_precision > 0
 *   comes before it in this solver (mpq/solver.py:893-899)
 * Reads two small status blocks per iteration (the denoiser's alpha1 checks, the LMMSE
 * row statistics), which the row kernels publish into mapped pinned host memory (the host
 * spins on a sequence number; after 20 s it falls back to hipStreamSynchronize).  The r2
 * message and first LMMSE product are queued before the first is read, the next
 * iteration's first denoiser pass before the second.  Output copies issued after the last
 * wait stay asynchronous on `stream`.
 */
int mpq_e8p12_vamp_solve(int64_t rows, int64_t n, const float* Wr, const float* hat_init,
                         const float* V, const float* S, const float* Vs, const float* prior_scale,
                         const MpqE8P12VampConfig* cfg, double obs_init, int64_t* idx_out,
                         float* hat_out, float* err_out, float* r1_out, float* gamma1_out,
                         MpqE8P12VampStats* stats, void* workspace, int64_t workspace_bytes,
                         mpq_stream_t stream);

/*
 * mpq_e8p12_vamp_solve with the packed rank-space operator of mpq_rankspace_pack (`packed`,
 * nullable): the solver's products then run as x6 products on the bf16 matrix cores (fp32
 * accuracy).  Same products as the reference's solver (mpq/solver.py:853-1138).
 */
int mpq_e8p12_vamp_solve_ex(int64_t rows, int64_t n, const float* Wr, const float* hat_init,
                            const float* V, const float* S, const float* Vs, const float* prior_scale,
                            const MpqE8P12VampConfig* cfg, double obs_init, const float* packed,
                            int64_t* idx_out, float* hat_out, float* err_out, float* r1_out,
                            float* gamma1_out, MpqE8P12VampStats* stats, void* workspace,
                            int64_t workspace_bytes, mpq_stream_t stream);

/*
 * Per-layer context of the E8P12 gram-metric polish: H = Vs Vs^T, per 8-column
 * block the gram G_j, its stabilized Cholesky factor L_j and (L_j L_j^T)^-1
 * (mpq/polish/block_cd.py:385-397, stabilize_cholesky mpq/linear.py:121-141),
 * the codebook grid and the tables |L_j^T c|^2 over all 65536 codewords
 * (mpq/polish/block_cd.py:228-230).  ctx: caller-allocated device memory of
 * mpq_e8p12_cd_context_size(n) bytes.  Returns MPQ_NUMERICAL_ERROR when a
 * Cholesky still fails after the 6 jitter retries (torch raises there).
 * Synchronises `stream` once.
 */
int64_t mpq_e8p12_cd_context_size(int64_t n);
int mpq_e8p12_cd_prepare(int64_t n, const float* Vs, void* ctx, int64_t ctx_bytes, mpq_stream_t stream);

/* Workspace bytes needed by mpq_e8p12_cd_polish. */
int64_t mpq_e8p12_cd_workspace_size(int64_t rows, int64_t n, int64_t block_rows);

/*
 * Gram-metric block coordinate descent over E8P12 codewords, every row block
 * of block_rows rows with its own greedy order: replaces mpq/solver.py:369-423
 * (polish_e8p12_rankspace, "block_cd", metric "gram") ->
 * mpq/polish/block_cd.py:332-625 with the step _cd_gram_step_impl (:212-246)
 * and the gains of _batched_greedy_gain (:286-306).
 *   targets: W (rows x n; Yu = W Vs is formed) or Yu (rows x n, W = NULL)
 *   x_in rows x n codeword values, idx_in rows x n/8 int64 codeword indices
 *   Vs n x n, ctx from mpq_e8p12_cd_prepare(n, Vs)
 *   max_blocks > 0 visits only the first max_blocks blocks of each greedy order
 *   outputs x_out, idx_out; err_before/err_after (rows, |Yu - x Vs|^2) and
 *   accepted_per_row (rows int32) may be NULL.  n/8 <= 16384.
 */
int mpq_e8p12_cd_polish(int64_t rows, int64_t n, int64_t block_rows, int sweeps, int64_t max_blocks,
                        float accept_tol, const float* W, const float* Yu, const float* x_in,
                        const int64_t* idx_in, const float* Vs, const void* ctx, float* x_out,
                        int64_t* idx_out, float* err_before, float* err_after,
                        int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                        mpq_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Dense algebra                                                            */
/* ------------------------------------------------------------------------ */

/*
 * C = alpha * A op(B) + beta * C, fp32 MFMA (v_mfma_f32_32x32x2_f32), split-K
 * with a fixed reduction order (bit-reproducible).  op(B) = B (K x N, ldb),
 * B^T (B stored N x K, trans_b = 1) or gathered rows B[b_rows[k], :].
 * Replaces the torch matmuls of mpq/linear.py:48-51, :94, mpq/solver.py:485,
 * mpq/polish/triton_scalar_cd.py:195-196.  workspace (optional) holds split-K
 * partials; with workspace_floats < 2*M*N the product runs unsplit.
 */
int mpq_gemm_f32(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                 int64_t ldb, int trans_b, const int32_t* b_rows, float* C, int64_t ldc,
                 float alpha, float beta, float* workspace, int64_t workspace_floats,
                 mpq_stream_t stream);

/*
 * C = alpha * A op(B) + beta * C in fp64 on the fp64 matrix cores (v_mfma_f64_16x16x4_f64, 128 x 64
 * tiles, split-K partials summed in a fixed order when `workspace` holds
 * mpq_gemm_f64_workspace_size(M, N, K) bytes; NULL runs the product unsplit).  The products of
 * mpq_syevd_f64, i.e. of the float64 torch.linalg.eigh in mpq/adapters/quip_sharp.py:54; exported
 * for testing the kernel on its own.
 */
int64_t mpq_gemm_f64_workspace_size(int64_t M, int64_t N, int64_t K);
int mpq_gemm_f64(int64_t M, int64_t N, int64_t K, const double* A, int64_t lda, const double* B, int64_t ldb,
                 int trans_b, double* C, int64_t ldc, double alpha, double beta, double* workspace,
                 int64_t workspace_bytes, mpq_stream_t stream);

/*
 * Split-K partial products P[s] = A[:, Ks] op(B)[Ks, :], s = 0..splits-1, written to
 * `partials` (splits x M x N, M*N apart): the kernel the VAMP drivers run for their rank-space
 * products, whose epilogues sum the partials in split order (callers that fuse their own
 * reduction use it directly).  mpq_gemm_f32_split_count gives the split count the library
 * uses for an M x N x K product.  Replaces the same torch matmuls as mpq_gemm_f32.
 */
int mpq_gemm_f32_split_count(int64_t M, int64_t N, int64_t K);
int mpq_gemm_f32_splitk(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                        int64_t ldb, int trans_b, float* partials, int splits, mpq_stream_t stream);

/*
 * fp32 products on the bf16 matrix cores ("x6"): each operand is split exactly into three bf16
 * planes and the six plane products of order >= 2^-16 |a||b| are accumulated in fp32
 * (v_mfma_f32_32x32x16_bf16), which keeps the accuracy of an fp32 product (the dropped terms are
 * below ~2^-22.4 |a||b| per multiply) at 8/3 the matrix-core rate of v_mfma_f32_32x32x2_f32.
 * The large operand op(B) (K x N, N % 128 == 0, K % 32 == 0) is packed once into fragment-ordered
 * tiles (K * N floats, mpq_gemm_x6_pack_b); mpq_gemm_x6 then forms C = A op(B) for any M, splitting
 * and packing A in `workspace` (mpq_gemm_x6_workspace_size bytes) and reducing split-K partials in
 * a fixed order.  Same products as mpq_gemm_f32 (no reference counterpart beyond those matmuls).
 */
int mpq_gemm_x6_pack_b(int64_t K, int64_t N, const float* B, int64_t ldb, int trans_b, float* packed,
                       mpq_stream_t stream);
int64_t mpq_gemm_x6_workspace_size(int64_t M, int64_t N, int64_t K);
int mpq_gemm_x6(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B_packed,
                float* C, int64_t ldc, void* workspace, int64_t workspace_bytes, mpq_stream_t stream);

/*
 * The two launches inside mpq_gemm_x6, as the VAMP solvers issue them: mpq_gemm_x6_pack_a splits
 * and packs A (mpq_gemm_x6_packed_a_size bytes, 16-byte aligned); mpq_gemm_x6_splitk writes the
 * split-K partials P[s] = A[:, Ks] op(B)[Ks, :] (splits x M x N, M*N apart; the library's split
 * count is mpq_gemm_x6_split_count, 0 when the shape has no x6 path).
 */
int mpq_gemm_x6_split_count(int64_t M, int64_t N, int64_t K);
int64_t mpq_gemm_x6_packed_a_size(int64_t M, int64_t K);
int mpq_gemm_x6_pack_a(int64_t M, int64_t K, const float* A, int64_t lda, void* packed, mpq_stream_t stream);
int mpq_gemm_x6_splitk(int64_t M, int64_t N, int64_t K, const void* A_packed, const float* B_packed,
                       float* partials, int splits, mpq_stream_t stream);

/*
 * The rank-space operator of one linear packed for the x6 products of the VAMP solvers:
 * 3 n^2 floats = [V packed for r V | V packed for x V^T | Vs packed for x Vs].
 * mpq_rankspace_pack_floats returns 0 when n has no x6 path (n % 128 != 0).  Formed once per
 * eigendecomposition and passed to mpq_uniform_vamp_solve_ex (`packed`).
 */
int64_t mpq_rankspace_pack_floats(int64_t n);
int mpq_rankspace_pack(int64_t n, const float* V, const float* Vs, float* packed, mpq_stream_t stream);

/* out = in^T (rows x cols -> cols x rows). */
int mpq_transpose(const float* in, int64_t rows, int64_t cols, int64_t ld_in, float* out,
                  int64_t ld_out, mpq_stream_t stream);

/*
 * Post-processing of an ascending eigendecomposition (lam_asc, V_asc columns):
 * eigenvalues floored at floor_v and put in descending order with their
 * vectors, S = sqrt(lam), Vs = V * S.  Replaces
 * mpq/adapters/gptqmodel.py:302-310 and :887-890 (the reference's eigh itself is
 * torch.linalg.eigh; here mpq_syevd).  Any output may be NULL.
 */
int mpq_eigh_postprocess(const float* lam_asc, const float* V_asc, int64_t n, float floor_v,
                         float* lam, float* S, float* V, float* Vs, mpq_stream_t stream);

/*
 * Symmetric eigendecomposition of H (n x n, fp32): lam ascending (n) and V (n x n, row-major,
 * column k = eigenvector k), the torch.linalg.eigh call of mpq/adapters/gptqmodel.py:276-310.
 * Blocked Householder tridiagonalisation, divide and conquer on the tridiagonal matrix (fp64
 * secular equations and Loewner vectors, merge products on the fp32 MFMA GEMM), then the
 * back-transformation V = Q Z as blocked compact-WY updates on the same GEMM; all on this
 * library's kernels.  workspace: mpq_syevd_workspace_size(n) bytes (about 24 n^2 below n = 8192,
 * about 40 n^2 from there).  Synchronises `stream` once per tridiagonal merge of more
 * than 512 rows and once at the end.
 */
int64_t mpq_syevd_workspace_size(int64_t n);
int mpq_syevd(int64_t n, const float* H, float* lam, float* V, void* workspace, int64_t workspace_bytes,
              mpq_stream_t stream);

/*
 * mpq_syevd with the reduction chosen by the caller (no counterpart in the reference, whose eigh
 * is torch.linalg.eigh): method 0 = automatic (what mpq_syevd does), 1 = the one-stage blocked
 * Householder tridiagonalisation above, 2 = the two-stage reduction (3 <= n <= 16416): dense to
 * a band of half-bandwidth 32 (panels by shifted Cholesky QR with a tall-skinny Householder QR
 * fallback, Householder vectors reconstructed from the orthogonal factor, trailing updates on the
 * MFMA GEMM), band to tridiagonal by bulge chasing (a cooperative pipeline of one wave per sweep),
 * then the chase's reflectors as explicit 64 x 64 blocks and the band reduction's reflectors as
 * compact-WY blocks applied to the tridiagonal eigenvectors.  Same output contract and workspace
 * size as mpq_syevd; the two-stage path synchronises `stream` once more (bulge-chasing status).
 */
int mpq_syevd_method(int64_t n, const float* H, float* lam, float* V, void* workspace, int64_t workspace_bytes,
                     int method, mpq_stream_t stream);

/*
 * The same decomposition in fp64 (the torch.linalg.eigh of the float64 Hessian in
 * mpq/adapters/quip_sharp.py:33-67): the one-stage kernels in double (divide-and-conquer
 * tolerances at fp64 unit roundoff), with the trailing updates, merge products and
 * back-transformation on the fp64 matrix cores (mpq_gemm_f64's kernel).
 * workspace: mpq_syevd_f64_workspace_size(n) bytes.
 */
int64_t mpq_syevd_f64_workspace_size(int64_t n);
int mpq_syevd_f64(int64_t n, const double* H, double* lam, double* V, void* workspace, int64_t workspace_bytes,
                  mpq_stream_t stream);

/* out[i][j] = in[i][j] * scale[j] (Vs = V * S, mpq/adapters/gptqmodel.py:890). */
int mpq_scale_columns(const float* in, int64_t rows, int64_t cols, const float* scale, float* out,
                      mpq_stream_t stream);

/*
 * Signed block Walsh-Hadamard along rows: forward out = H_b(in * signs) /
 * sqrt(b), inverse out = H_b(in) / sqrt(b) * signs, b = had_dim (power of two,
 * width % b == 0), Sylvester order with butterfly strides 1, 2, 4, ...
 * Replaces mpq/rotation.py:404-438 (apply_right_block_hadamard[_inverse]) and
 * its torch butterfly mpq/rotation.py:135-156.  signs may be NULL.
 */
int mpq_block_hadamard(const float* in, int64_t ld_in, float* out, int64_t ld_out, int64_t rows,
                       int64_t width, int64_t had_dim, const float* signs, int inverse,
                       mpq_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Uniform (scalar) grid                                                    */
/* ------------------------------------------------------------------------ */

/*
 * GPTQ asymmetric min-max parameters per (row, group of group_size columns):
 * xmin = min(min(w), 0), xmax = max(max(w), 0) (+-1 if both 0),
 * scale = (xmax - xmin)/maxq, zero = round(-xmin/scale).  Replaces the
 * GPTQModel quantizer.find_params calls of mpq/adapters/gptqmodel.py:899-909.
 * scale, zero: rows x ceil(n/group_size).
 */
int mpq_gptq_find_params(const float* W, int64_t rows, int64_t n, int64_t ldw, int64_t group_size,
                         int maxq, float* scale, float* zero, mpq_stream_t stream);

/*
 * RTN decision q = clamp(round(W/s) + z, 0, maxq) (uint8), x = s(q - z).
 * Replaces mpq/adapters/gptqmodel.py:966-969.  q or x may be NULL.
 */
int mpq_uniform_rtn(const float* W, int64_t rows, int64_t n, int64_t ldw, const float* scale,
                    const float* zero, int64_t group_size, int maxq, uint8_t* q, float* x,
                    mpq_stream_t stream);

/*
 * AWQ scale search for one linear (or linears sharing an input), the step before the solve:
 * mpq/awq_scale.py:491-580 (_search_best_scale) scored, for a single linear layer, by the
 * output error  sum_rows D H D^T / rows  (D = W - pseudo_quant(W s)/s, H = X^T X / T), with
 * _compute_w_mean (:49-83), _candidate_scales (:338-348), _pseudo_quantize_tensor_into
 * (:108-157), 20 ratios k/20, first minimum wins.
 *   mpq_awq_w_mean: w_sum[j] += sum_rows |W[r][j]| / (group abs-max + 1e-6) (divide by the
 *     total row count for w_mean); workspace >= rows * n/group_size floats.
 *   mpq_awq_search: W rows x n, H n x n, x_mean n (mean |x|), w_mean n; outputs best_scales (n,
 *     device), losses_out (20, device, optional), best_error / best_ratio (host pointers,
 *     optional).  Synchronises `stream` once.  n % group_size == 0.
 */
int64_t mpq_awq_workspace_size(int64_t rows, int64_t n);
int mpq_awq_w_mean(const float* W, int64_t rows, int64_t n, int64_t group_size, float* w_sum,
                   void* workspace, int64_t workspace_bytes, mpq_stream_t stream);
int mpq_awq_search(const float* W, int64_t rows, int64_t n, const float* H, const float* x_mean,
                   const float* w_mean, int64_t group_size, int bits, int sym, float* best_scales,
                   float* losses_out, float* best_error, float* best_ratio, void* workspace,
                   int64_t workspace_bytes, mpq_stream_t stream);

/*
 * Per-linear Hessian accumulation H = beta H + alpha X^T X (both triangles, exactly symmetric)
 * and optionally colsum += column sums of X: the step before the solve, GPTQModel's add_batch
 * (H = 2/m sum x x^T, mpq/adapters/gptqmodel.py:39) and QUIP#'s Hessian hooks
 * (mpq/quip_generic.py:823-921: sum x x^T and sum x, finalised as H/ct - mu mu^T).
 *   X: T x n activations (ldx >= n, ldx % 4 == 0), fp32 (x_bf16 = 0) or bf16 (x_bf16 = 1);
 *   n % 128 == 0; H: n x n fp32 (ldh).  fp32 MFMA SYRK (tiles on/above the diagonal).
 */
int mpq_hessian_accumulate(const void* X, int x_bf16, int64_t T, int64_t n, int64_t ldx, float alpha,
                           float beta, float* H, int64_t ldh, float* colsum, mpq_stream_t stream);

/*
 * GPTQModel int32 packing of the codes (the step after the solve on the GPTQModel path,
 * patches/gptqmodel.patch:359-395, scripts/backend_gptq.py:843 format GPTQ_V2):
 *   q rows x n uint8 codes (rows = out features, n = in features; both % 32 == 0),
 *   scale/zero rows x G group parameters (G = ceil(n / group_size)), bits in {2, 3, 4, 8};
 *   outputs qweight int32 [n*bits/32][rows], qzeros int32 [G][rows*bits/32] (format_v1 != 0
 *   stores zero - 1, else zero), scales fp16 [G][rows], g_idx int32 [n] = i / group_size.
 * 3-bit values are packed 32 to 3 words (GPTQModel's layout).  Parity with GPTQModel's packer:
 * the layout is its published one; the packer itself is upstream and absent.
 */
int mpq_gptq_pack(const uint8_t* q, const float* scale, const float* zero, int64_t rows, int64_t n,
                  int64_t group_size, int bits, int format_v1, int32_t* qweight, int32_t* qzeros,
                  void* scales_fp16, int32_t* g_idx, mpq_stream_t stream);

/* x = s(q - z) from uint8 codes.  Replaces mpq/priors/uniform.py:302-309 and the packed-basis
 * weight rebuild scale * (q - zero) of patches/gptqmodel.patch:381-391. */
int mpq_dequant(const uint8_t* q, int64_t rows, int64_t n, const float* scale, const float* zero,
                int64_t group_size, float* x, mpq_stream_t stream);

/*
 * Posterior of each entry over the uniform grid a_q = s(q - z), q = 0..maxq,
 * under channel N(r1, 1/gamma_row) and prior N(center, (tau*s)^2):
 * mean, var, MAP index (int64, first max) and value, alpha1 = gamma*mean(var)
 * (rows, optional).  Replaces mpq/priors/uniform.py:99-213
 * (discrete_uniform_mmse without diagnostics).
 */
int mpq_uniform_denoise(int64_t rows, int64_t n, int maxq, const float* r1, const float* gamma,
                        const float* center, int64_t ld_center, const float* scale,
                        const float* zero, int64_t group_size, float tau, float* mean, float* var,
                        int64_t* map_idx, float* map_value, float* alpha1, mpq_stream_t stream);

/* Mirrors UniformVampConfig (mpq/solver.py:35-55). */
typedef struct MpqUniformVampConfig {
  int iters;
  float damping;
  int final_decision; /* 0 = "map", 1 = "round_mean" */
  int init_from;      /* 0 = "rtn", 1 = "float", 2 = "zero" */
  float gamma_start;
  float gamma_retry_factor;
  int gamma_retry_steps;
  float prior_tau;
  double obs_precision; /* > 0: fixed observation precision (EM off) */
  int em_obs_precision;
  double em_obs_precision_damping;
  double em_obs_precision_min;
  double em_obs_precision_max;
} MpqUniformVampConfig;

/* Per-solve statistics (subset of mpq/solver.py:783-829). */
typedef struct MpqUniformVampStats {
  int iters;
  int best_iter;
  int stop_iter;
  int alpha1_retry_count;
  int alpha2_clip_count;
  int gamma2_invalid_count;
  double obs_precision_initial;
  double obs_precision_final;
  double obs_precision_mean;
  double alpha1_mean;
  double alpha2_mean;
  double best_rankspace_error_mean;
  double rtn_rankspace_error_mean;
} MpqUniformVampStats;

/* Workspace bytes needed by mpq_uniform_vamp_solve for a rows x n block. */
int64_t mpq_uniform_vamp_workspace_size(int64_t rows, int64_t n);

/*
 * Uniform-grid VAMP on one row block, without the polish: replaces
 * mpq/solver.py:426-703 (solve_uniform_rankspace_vamp up to the polish) with
 * its denoiser mpq/priors/uniform.py:99-213, LMMSE mpq/linear.py:10-56, EM
 * mpq/linear.py:59-82 and rank-space error mpq/linear.py:85-94.
 *   W (ldw), x_init: rows x n (x_init = RTN decision, also the gamma1 init)
 *   scale/zero: rows x ceil(n/group_size) group parameters
 *   V, Vs: n x n (full rank), S: n
 *   obs_init > 0 is the warm start of the observation precision; it comes before
 *   cfg->obs_precision (mpq/solver.py:486-489), else the RTN decision's error sets it
 *   q_out (rows x n uint8), x_out (optional), err_out (rows), rtn_err_out (rows, optional)
 * Reads two small status blocks per iteration (the denoiser's alpha1 checks, the hard
 * state's error), which the row kernels publish into mapped pinned host memory (the host
 * spins on a sequence number; after 20 s it falls back to hipStreamSynchronize).  The r2
 * message and first LMMSE product are queued before the first is read, the next
 * iteration's first denoiser pass before the second.  Output copies issued after the last
 * wait stay asynchronous on `stream`.
 */
int mpq_uniform_vamp_solve(int64_t rows, int64_t n, int maxq, const float* W, int64_t ldw,
                           const float* x_init, const float* scale, const float* zero,
                           int64_t group_size, const float* V, const float* S, const float* Vs,
                           const MpqUniformVampConfig* cfg, double obs_init, uint8_t* q_out,
                           float* x_out, float* err_out, float* rtn_err_out,
                           MpqUniformVampStats* stats, void* workspace, int64_t workspace_bytes,
                           mpq_stream_t stream);

/*
 * mpq_uniform_vamp_solve with products the caller formed for all rows at once (one GEMM over
 * every row block instead of one per block; the reference forms the same products per block in
 * mpq/solver.py:467-480 and the warm start in mpq/adapters/gptqmodel.py:920-941):
 *   Yu_in (optional) rows x n = W Vs, xr_in (optional) rows x n = x_init Vs;
 *   xprod_out (optional) rows x n receives x_best Vs of the returned codes (the polish's start).
 * All three are contiguous (leading dimension n).  `packed` (optional): the rank-space operator
 * from mpq_rankspace_pack; the solver's products then run as x6 products (same accuracy class
 * as the fp32 MFMA path).
 */
int mpq_uniform_vamp_solve_ex(int64_t rows, int64_t n, int maxq, const float* W, int64_t ldw,
                              const float* x_init, const float* scale, const float* zero,
                              int64_t group_size, const float* V, const float* S, const float* Vs,
                              const MpqUniformVampConfig* cfg, double obs_init, const float* Yu_in,
                              const float* xr_in, const float* packed, uint8_t* q_out, float* x_out,
                              float* err_out, float* rtn_err_out, float* xprod_out,
                              MpqUniformVampStats* stats, void* workspace, int64_t workspace_bytes,
                              mpq_stream_t stream);

/* Workspace bytes needed by mpq_uniform_cd_polish. */
int64_t mpq_uniform_cd_workspace_size(int64_t rows, int64_t n, int64_t block_rows);

/*
 * Greedy scalar coordinate-descent polish over all rows, each block of
 * block_rows rows with its own greedy column order: replaces
 * mpq/polish/triton_scalar_cd.py:164-307 (uniform_scalar_diag_greedy_cd, the
 * CUDA dispatch of mpq/solver.py:299-333) and, with select != 0, the
 * keep-if-better selection of mpq/solver.py:749-754.
 *   targets: W (ldw) rows x n (Yu = W Vs is formed) or Yu rows x n (W = NULL);
 *   q_in rows x n uint8 initial codes; x_in (optional) rows x n initial values
 *   (default: dequantised q_in); Vs, H (gram_full) n x n; outputs q_out,
 *   err_before/err_after (rows), improved (rows int32), accepted_per_row
 *   (rows int32); every output but q_out may be NULL.  n <= 16384.
 */
int mpq_uniform_cd_polish(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                          float accept_tol, const float* W, int64_t ldw, const float* Yu,
                          const uint8_t* q_in, const float* x_in, const float* scale,
                          const float* zero, int64_t group_size,
                          const float* Vs, const float* H, int select, uint8_t* q_out,
                          float* err_before, float* err_after, int32_t* improved,
                          int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                          mpq_stream_t stream);

/*
 * The greedy sweeps alone, in place on caller state: replaces the persistent
 * sweep launch of mpq/polish/triton_scalar_cd.py:113-161
 * (_launch_persistent_scalar_cd_sweep, which takes rhs_all, x_work,
 * residual_norm, order, gram and diag) together with the per-sweep greedy
 * order of :241-243.  Per row block of block_rows rows: gain_j = (sum over the
 * block's rows, in row order, of rhs^2 * (1/diag_j)) / rows_in_block, stable
 * descending order, then the column-at-a-time decisions and rank-1 updates
 * rhs -= delta * H[col, :] (product rounded, then difference rounded).
 *   rhs, x: rows x n fp32 (in/out); q: rows x n uint8 codes (in/out);
 *   res_norm: rows (in/out); accepted: rows int32, incremented by the number
 *   of accepted moves; scale/zero: rows x ceil(n/group_size); diag: n
 *   (|Vs_j|^2, already floored); H: n x n.
 * workspace: mpq_uniform_cd_sweeps_workspace_size(rows, n, block_rows) bytes.
 */
int64_t mpq_uniform_cd_sweeps_workspace_size(int64_t rows, int64_t n, int64_t block_rows);
int mpq_uniform_cd_sweeps(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                          float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                          int32_t* accepted, const float* scale, const float* zero,
                          int64_t group_size, const float* diag, const float* H, void* workspace,
                          int64_t workspace_bytes, mpq_stream_t stream);

/*
 * Column permutations of the activation-order path (desc_act, mpq/adapters/gptqmodel.py:733-740 and
 * the inverse at :1090-1095, where the reference uses index_select): mpq_permute_columns gives
 * out[:, c] = in[:, perm[c]] for a rows x cols row-major matrix of 1-byte (codes) or 4-byte (fp32)
 * elements; mpq_permute_symmetric gives out[i][j] = in[perm[i]][perm[j]] (n x n fp32).  The kernels
 * read through perm unchecked: every entry must lie in [0, cols) (resp. [0, n)), and out must not
 * overlap in.
 */
int mpq_permute_columns(const void* in, int64_t rows, int64_t cols, const int32_t* perm, void* out, int elem_bytes,
                        mpq_stream_t stream);
int mpq_permute_symmetric(const float* in, int64_t n, const int32_t* perm, float* out, mpq_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Generic rank-space block coordinate descent                              */
/* ------------------------------------------------------------------------ */

/*
 * The device steps of mpq/polish/block_cd.py:332-625 (block_coordinate_descent_rankspace) for a
 * caller-driven block loop with any candidate provider; blocks of 1 <= block_size <= 16 columns.
 * mpq_bcd_prepare: per block b of the n x R matrix Vs, the gram G_b = Vs_b Vs_b^T (gram, nb x bs x
 * bs), for metric_gram the Cholesky factor with the reference's diagonal-jitter retries
 * (stabilize_cholesky, mpq/linear.py:121-141; chol, lower) and (L L^T)^-1 (ginv), otherwise ginv[b]
 * holds 1 / max(G_ii, 1e-12); importance[b] = trace(G_b) (:398-420); status[b] = 1 where every
 * Cholesky retry failed.
 * mpq_bcd_gain: the greedy gain of every block from rhs = residual_u Vs^T (rows x n)
 * (_batched_greedy_gain, :286-306).
 * mpq_bcd_target: target = x_blk + rhs G^-1 (gram) or x_blk + rhs diag_inv (diag) (:581-585).
 * mpq_bcd_accept: the accept test and state update of one block (_cd_accept_step_impl :28-42 and
 * :600-611): x, res_norm, accepted, the block's column of idx (when given) in place; delta gets the
 * accepted moves for residual_u -= delta Vs_blk.
 */
int mpq_bcd_prepare(int64_t n, int64_t R, int block_size, int metric_gram, const float* Vs, float* gram,
                    float* chol, float* ginv, float* importance, int32_t* status, mpq_stream_t stream);
int mpq_bcd_gain(int64_t rows, int64_t n, int block_size, int metric_gram, const float* rhs, const float* ginv,
                 float* gain, mpq_stream_t stream);
int mpq_bcd_target(int64_t rows, int64_t n, int block_size, int64_t block, int metric_gram, const float* x,
                   const float* rhs, const float* ginv, float* target, mpq_stream_t stream);
int mpq_bcd_accept(int64_t rows, int64_t n, int block_size, int64_t block, const float* cand, const float* rhs,
                   const float* gram, float accept_tol, const int64_t* cand_idx, float* x, float* res_norm,
                   int64_t* idx, int32_t* accepted, float* delta, mpq_stream_t stream);

/*
 * Candidate providers of mpq/polish/block_cd.py:628-861 on the device.
 * mpq_bcd_uniform_propose: UniformScalarProvider (:628-653), column `col` of the expanded
 * scale / zero (rows x n): q = clamp(round(target / s + z), 0, maxq), value s (q - z).
 * mpq_bcd_topk_scalar_propose: UniformTopKProvider (:656-682): the nearest of the k candidates
 * vals_k[r, col, :] (rows x n x k; first on ties) and its level from q_k (nullable; -1 then).
 * mpq_e8p12_metric_argmin: E8P12Provider with the gram metric (_metric_map_assign, :702-739): per
 * row of target (rows x 8) the codeword minimising |(t - c) L|^2 over all 65536 codewords of the
 * build's table, first index on ties; workspace mpq_e8p12_metric_argmin_workspace_size(rows) bytes.
 * mpq_bcd_e8_topk_propose: E8P12TopKProvider (:778-861): the nearest of topk_idx[r, block, :]
 * (rows x nb x k codeword indices) to the target, whitened by chol (8 x 8, nullable: plain distance).
 */
int mpq_bcd_uniform_propose(int64_t rows, int64_t n, int64_t col, int maxq, const float* target,
                            const float* scale, const float* zero, float* vals, int64_t* q, mpq_stream_t stream);
int mpq_bcd_topk_scalar_propose(int64_t rows, int64_t n, int64_t col, int64_t k, const float* target,
                                const float* vals_k, const int64_t* q_k, float* vals, int64_t* q,
                                mpq_stream_t stream);
int64_t mpq_e8p12_metric_argmin_workspace_size(int64_t rows);
int mpq_e8p12_metric_argmin(int64_t rows, const float* target, const float* chol, float* vals, int64_t* idx,
                            void* workspace, int64_t workspace_bytes, mpq_stream_t stream);
int mpq_bcd_e8_topk_propose(int64_t rows, int64_t nb, int64_t block, int64_t k, const int64_t* topk_idx,
                            const float* target, const float* chol, float* vals, int64_t* idx,
                            mpq_stream_t stream);

/*
 * mpq_uniform_cd_sweeps with the RTN target formed as x + rhs * (1 / diag), the rule of the
 * reference's torch update loop (mpq/polish/triton_scalar_cd.py:258-288, target at :266, the
 * default update_backend="torch"); mpq_uniform_cd_sweeps forms x + rhs / diag like its sweep kernel
 * (:73).  Same arguments and workspace as mpq_uniform_cd_sweeps.
 */
int mpq_uniform_cd_sweeps_recip(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                                int32_t* accepted, const float* scale, const float* zero,
                                int64_t group_size, const float* diag, const float* H, void* workspace,
                                int64_t workspace_bytes, mpq_stream_t stream);

/*
 * mpq_uniform_cd_sweeps without a workspace argument and without any device
 * allocation.  No counterpart in the reference: for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The sweeps' scratch is a static device array of
 * mpq_uniform_cd_sweeps_noalloc_max_bytes() bytes (8 MiB) per GPU, held until
 * the process ends; a problem whose
 * mpq_uniform_cd_sweeps_workspace_size(rows, n, block_rows) exceeds it is
 * rejected with MPQ_INVALID_ARGUMENT.  Runs on the current device (the stream
 * must belong to it).  Every call on one GPU uses that GPU's array: calls that
 * overlap on one GPU (other threads, other streams) race.  Results are
 * bit-identical to mpq_uniform_cd_sweeps.
 */
int64_t mpq_uniform_cd_sweeps_noalloc_max_bytes(void);
int mpq_uniform_cd_sweeps_noalloc(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                                  float accept_tol, float* rhs, float* x, uint8_t* q, float* res_norm,
                                  int32_t* accepted, const float* scale, const float* zero,
                                  int64_t group_size, const float* diag, const float* H,
                                  mpq_stream_t stream);

/*
 * mpq_uniform_cd_polish with the start's product x Vs from the caller (xprod_in, rows x n,
 * contiguous; optional): mpq_uniform_vamp_solve_ex returns it for its codes, so the polish skips
 * that product (the reference recomputes it, mpq/solver.py:283-290).  With S (n singular values,
 * Vs = V diag(S)) and the packed rank-space operator (mpq_rankspace_pack; both optional, n % 128
 * == 0) its two full products (rhs = residual Vs^T, final x Vs; mpq/solver.py:291-330) run as
 * fp32-accurate bf16-plane products on the matrix cores.
 */
int mpq_uniform_cd_polish_ex(int64_t rows, int64_t n, int maxq, int64_t block_rows, int sweeps,
                             float accept_tol, const float* W, int64_t ldw, const float* Yu,
                             const uint8_t* q_in, const float* x_in, const float* xprod_in,
                             const float* scale, const float* zero, int64_t group_size,
                             const float* Vs, const float* S, const float* packed, const float* H,
                             int select, uint8_t* q_out,
                             float* err_before, float* err_after, int32_t* improved,
                             int32_t* accepted_per_row, void* workspace, int64_t workspace_bytes,
                             mpq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MPQ_AMD_H_ */
