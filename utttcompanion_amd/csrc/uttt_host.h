// Host-side helpers shared by the C-ABI entry points: error text, status codes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/uttt_amd.h"

namespace uttt {

char* last_error_buffer();

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

inline int ok() {
  last_error_buffer()[0] = '\0';
  return UTTT_OK;
}

// Status after a group of launches.
inline int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(UTTT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Readout of B rows of up to 64 tokens from saved H and W_down (chunk_update.hip): row b's
// out[t] = x[t] + LN(H[b] W_down[b])[t] for t < ntok, fp32 throughout.  h (B, 64, F) (rows past
// ntok zero), w_down (B, F, D) with row stride wd_rs, zp a (nsplit, B, 64, D) fp32 scratch; x and
// out rows of D floats, x_rs / out_rs elements apart from one row b to the next.
void launch_saved_readout(int B, int ntok, int D, int F, int nsplit, const float* h, const float* w_down,
                          int64_t wd_rs, float* zp, const float* x, int64_t x_rs, const float* ln_w,
                          const float* ln_b, float eps, float* out, int64_t out_rs, hipStream_t st);

// uttt_linear with the tile shape chosen by the caller: tile_rows 0 plans it from the shape
// (as uttt_linear does), 128 takes 128-row tiles without a k split (no workspace needed).
int linear_enqueue(const uttt_linear_args* a, hipStream_t st, int tile_rows);

}  // namespace uttt

#define UTTT_REQUIRE(cond, ...)                              \
  do {                                                       \
    if (!(cond)) return ::uttt::fail(UTTT_ERR_INVALID, __VA_ARGS__); \
  } while (0)
