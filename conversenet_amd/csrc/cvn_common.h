// Host-side helpers shared by the C-ABI translation units: error reporting, workspace carving,
// FFT plan construction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "../../include/converse2d.h"
#include "fft_device.h"

namespace cvn {

std::string& last_error_slot();

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error_slot() = buf;
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CVN_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return CVN_OK;
}

inline size_t align_up(size_t n, size_t a = 256) { return (n + a - 1) / a * a; }

// Largest transform length any generic-path kernel accepts (LDS capacity).
constexpr int kMaxFftLen = 4096;

// Decompose L into Stockham radices: 8s, then 4/2 for the rest of the power of two, then the odd
// radices with fixed butterflies, then any remaining prime factors (generic O(R^2) pass).
inline bool make_plan(int L, FftPlan* plan) {
  if (L < 1 || L > kMaxFftLen) return false;
  plan->L = L;
  plan->nst = 0;
  int n = L;
  auto push = [&](int r) {
    if (plan->nst >= kMaxStages) return false;
    plan->radix[plan->nst++] = r;
    return true;
  };
  while (n % 8 == 0) { if (!push(8)) return false; n /= 8; }
  while (n % 4 == 0) { if (!push(4)) return false; n /= 4; }
  while (n % 2 == 0) { if (!push(2)) return false; n /= 2; }
  const int odd[] = {3, 5, 7, 11, 13};
  for (int r : odd)
    while (n % r == 0) { if (!push(r)) return false; n /= r; }
  for (int f = 17; n > 1 && (int64_t)f * f <= n; f += 2)
    while (n % f == 0) { if (!push(f)) return false; n /= f; }
  if (n > 1 && !push(n)) return false;
  return true;
}

// Fused single-kernel path (converse2d_fused.hip): returns 1 and the workspace it needs when the
// padded plane (H + 2 pad, W + 2 pad) at this scale has an instantiated plan.
int fused_query(int H, int W, int pad, int scale, int64_t Cp, size_t* ws_bytes);
int fused_table(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                int H, int W, int pad, void* table, hipStream_t st);
int fused_apply(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode, int act,
                const void* table, float* out, hipStream_t st);
// CVN_DISABLE_FUSED=1 in the environment routes every call through the generic multi-pass path.
bool fused_disabled();

}  // namespace cvn
