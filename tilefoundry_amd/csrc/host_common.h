// Host-side helpers shared by the library's source files: the error text
// behind tfd_last_error(), launch checks, and the chunk-count dispatch of the
// GEMV templates.
#pragma once

#include <hip/hip_runtime.h>

namespace tfd_host {

// error codes returned by the entries (negative; positive values are hipError_t)
enum : int { kBadArg = -1, kBadShape = -2, kUnsupported = -3 };

extern thread_local char g_err[512];

// Record the message for tfd_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// 0, or the launch error of the last kernel (recorded under `what`).
int launched(const char* what);
// 16-byte chunks per lane (1, 2, 4, 8, 12, 16) for a length-K vector over a wave; 0 if too long.
int cmax_for(int K);
// compute units of the current device (256 if the query fails), cached per device
int compute_units();

}  // namespace tfd_host

#define TFD_CMAX_SWITCH(K, CALL)                                          \
  switch (tfd_host::cmax_for(K)) {                                        \
    case 1: { constexpr int kC = 1; CALL; break; }                        \
    case 2: { constexpr int kC = 2; CALL; break; }                        \
    case 4: { constexpr int kC = 4; CALL; break; }                        \
    case 8: { constexpr int kC = 8; CALL; break; }                        \
    case 12: { constexpr int kC = 12; CALL; break; }                      \
    case 16: { constexpr int kC = 16; CALL; break; }                      \
    default: return tfd_host::fail(tfd_host::kUnsupported, "K=%d exceeds 8192", K); \
  }
