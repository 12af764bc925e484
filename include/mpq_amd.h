/*
 * mpq_amd — C-ABI of the MI355X (gfx950) per-layer quantization hot path.
 *
 * Conventions (all entry points):
 *  - every buffer is caller-allocated device memory, row-major and contiguous,
 *    fp32 unless stated; no entry point allocates unless documented;
 *  - work is enqueued on `stream` (a hipStream_t; NULL = default stream) and is
 *    asynchronous: nothing synchronises the host;
 *  - the return value is 0 on success, MPQ_INVALID_ARGUMENT (-1) for a bad
 *    shape/argument (nothing launched), MPQ_HIP_ERROR (-2) for a HIP failure;
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

/* Thread-local description of the last failed call ("" if none). */
const char* mpq_last_error(void);
int mpq_last_error_code(void);
void mpq_clear_error(void);

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

#ifdef __cplusplus
}
#endif

#endif /* MPQ_AMD_H_ */
