// Shared helpers for the mpq_amd HIP library: error state, launch checks.
// Every kernel in this library is built for gfx950 only, with
// -ffp-contract=off: fused multiply-adds appear only where written as fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

namespace mpq {

// Status codes returned by every extern "C" entry point.
enum Status : int {
  kOk = 0,
  kInvalidArgument = -1,
  kHipError = -2,
  kUnsupported = -3,
};

void set_error(const char* fmt, ...);
const char* last_error();
int last_error_code();
void set_error_code(int code);

}  // namespace mpq

#define MPQ_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      mpq::set_error(__VA_ARGS__);               \
      mpq::set_error_code(mpq::kInvalidArgument);\
      return mpq::kInvalidArgument;              \
    }                                            \
  } while (0)

#define MPQ_HIP_TRY(expr)                                                        \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess) {                                                      \
      mpq::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),      \
                     __FILE__, __LINE__);                                        \
      mpq::set_error_code(mpq::kHipError);                                       \
      return mpq::kHipError;                                                     \
    }                                                                            \
  } while (0)

#define MPQ_LAUNCH_CHECK() MPQ_HIP_TRY(hipGetLastError())

static inline int64_t mpq_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
