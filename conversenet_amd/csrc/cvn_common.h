// Host-side helpers shared by the C-ABI translation units: error reporting, workspace carving,
// FFT plan construction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <atomic>
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

// Fixed-radix decomposition (8s, then 4 / 2 for the rest of the power of two, then 3, 5, 7, 11,
// 13); false if a factor is left over or the stage list overflows.
inline bool fixed_radices(int n, int* radix, int* nst, int cap) {
  *nst = 0;
  auto push = [&](int r) {
    if (*nst >= cap) return false;
    radix[(*nst)++] = r;
    return true;
  };
  while (n % 8 == 0) { if (!push(8)) return false; n /= 8; }
  while (n % 4 == 0) { if (!push(4)) return false; n /= 4; }
  while (n % 2 == 0) { if (!push(2)) return false; n /= 2; }
  const int odd[] = {3, 5, 7, 11, 13};
  for (int r : odd)
    while (n % r == 0) { if (!push(r)) return false; n /= r; }
  return n == 1;
}

inline int powmod_host(int64_t g, int64_t e, int64_t m) {
  int64_t r = 1 % m, b = g % m;
  while (e > 0) {
    if (e & 1) r = r * b % m;
    b = b * b % m;
    e >>= 1;
  }
  return (int)r;
}

// Rader setup for prime R: a primitive root g, its inverse, and the fixed-radix plan of R - 1.
inline bool make_rader(int R, RaderPlan* rp) {
  if (R - 1 > kMaxRaderLen) return false;
  for (int d = 2; d * d <= R; ++d)
    if (R % d == 0) return false;  // not prime
  if (!fixed_radices(R - 1, rp->radix, &rp->nst, kMaxInnerStages)) return false;
  int qs[16], nq = 0;
  for (int n = R - 1, d = 2; n > 1; ++d)
    if (n % d == 0) {
      qs[nq++] = d;
      while (n % d == 0) n /= d;
    }
  for (int g = 2; g < R; ++g) {
    bool prim = true;
    for (int i = 0; i < nq && prim; ++i) prim = powmod_host(g, (R - 1) / qs[i], R) != 1;
    if (prim) {
      rp->R = R;
      rp->g = g;
      rp->ginv = powmod_host(g, R - 2, R);
      return true;
    }
  }
  return false;
}

// Decompose L into Stockham radices: the fixed butterflies first, then the remaining prime factors,
// each either a Rader stage (prime R with R - 1 made of fixed radices, R - 1 <= kMaxRaderLen) or
// the generic O(R^2) pass.
inline bool make_plan(int L, FftPlan* plan) {
  if (L < 1 || L > kMaxFftLen) return false;
  plan->L = L;
  plan->nst = 0;
  plan->nrad = 0;
  int n = L;
  auto push = [&](int r) {
    if (plan->nst >= kMaxStages) return false;
    plan->radix[plan->nst++] = r;
    return true;
  };
  for (int r : {2, 3, 5, 7, 11, 13})
    while (n % r == 0) n /= r;
  int nfix = 0, fixr[kMaxStages];
  if (!fixed_radices(L / n, fixr, &nfix, kMaxStages)) return false;
  for (int i = 0; i < nfix; ++i)
    if (!push(fixr[i])) return false;
  size_t off = 0;
  for (int f = 17; n > 1; f += 2) {
    if ((int64_t)f * f > n) f = n;  // what is left is prime
    while (n % f == 0) {
      if (!push(f)) return false;
      n /= f;
      bool have = false;
      for (int r = 0; r < plan->nrad; ++r) have = have || plan->rad[r].R == f;
      if (!have && plan->nrad < kMaxRader) {
        RaderPlan rp;
        if (make_rader(f, &rp)) {
          rp.off = (int)off;
          off += rader_tab_bytes(f);
          plan->rad[plan->nrad++] = rp;
        }
      }
    }
  }
  return true;
}

// Fused single-kernel path (converse2d_fused.hip): returns 1 and the workspace it needs when the
// padded plane (H + 2 pad, W + 2 pad) at this scale has an instantiated plan (at scale > 1: when the
// upsampled plane has one).
int fused_query(int H, int W, int pad, int scale, int64_t Cp, size_t* ws_bytes);
int fused_table(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                int H, int W, int pad, int scale, void* table, hipStream_t st);
// Scratch that lets fused_apply split each plane over two workgroups (one per row group; at most
// kFusedSplitPlanes planes, where one workgroup per plane leaves most CUs idle); 0 where no split applies.
constexpr int64_t kFusedSplitPlanes = 128;
size_t fused_scratch(int64_t planes, int H, int W, int pad, int scale);
// scratch: null, or at least fused_scratch(B C, ...) bytes (then small plane counts run split)
int fused_apply(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode, int act,
                int scale, const void* table, void* scratch, float* out, hipStream_t st);
// 268 x 268 planes at scale 1 (converse2d_pfa.hip): in-place prime-factor FFTs 268 = 4 * 67 with an
// in-register Rader 67-point DFT.
bool pfa268_applies(int h, int w, int s);
// Index of Phi(u, v) (row frequency u, half-spectrum column v) in the 268 path's transfer table:
// (Cp, 67, 135, 4) = [psf plane][u mod 67][v][lane of the quad that holds bin u], so that the 16
// quads of a wave read 512 contiguous bytes per register.  The lane holding u is br(u mod 4) with
// br = [0, 2, 1, 3] (the bit-reversed output order of the quad's 4-point DFT).
__host__ __device__ inline int64_t pfa268_phi_index(int64_t cp, int v, int u) {
  const int r = u & 3;
  return ((cp * 67 + u % 67) * 135 + v) * 4 + (((r & 1) << 1) | (r >> 1));
}
// Index (in float2 units) of Phi(u, v) (row frequency u < 256, half-spectrum column v <= 128) in the
// fused kernel's table for 256 x 256 planes (the Cooley-Tukey plan in converse2d_fused.hip): per psf
// plane 64 row pairs of 259 slots, two float2 per slot (Phi at k and at k + 128).  Row frequency
// k = 2 k2 + k1 (k < 128) sits at row pair 8 (k2 mod 8) + k2 / 8, at position v of the pair for k1 = 0
// and at the odd row's position of v (256 - v; 256 for v = 0, 257 for v = 128) for k1 = 1.
// converse2d_fused.hip checks this map against its plan at compile time.
constexpr int kF256Rs = 259, kF256Slots = 64 * kF256Rs;
__host__ __device__ constexpr int64_t fused256_phi_index(int64_t cp, int v, int u) {
  const int k = u & 127, k2 = k >> 1;
  const int rp = 2 * (8 * (k2 & 7) + (k2 >> 3)) + (k & 1);
  const int pos = (rp & 1) ? (v == 0 ? 256 : (v == 128 ? 257 : 256 - v)) : v;
  return ((cp * kF256Slots + (int64_t)(rp >> 1) * kF256Rs + pos) << 1) + (u >> 7);
}
int pfa268_forward(const float* x, int64_t P, int64_t C, int64_t psf_batch, int H, int W, int pad, int mode, int act,
                   const float2* phi, float2* S, float* out, hipStream_t st);
// Scratch the 268 path needs between its passes (at least the generic path's S region).
size_t pfa268_scratch_bytes(int64_t P);
// CVN_DISABLE_FUSED=1 in the environment routes every call through the generic multi-pass path.
bool fused_disabled();

// Index of the current HIP device (0 if the query fails).
inline int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  return dev;
}
// Runs fn once per device for devices 0..63 (per-device launch attributes and occupancy queries).
// Thread-safe; concurrent first calls on one device may both run fn, so fn must be idempotent.
template <class F>
void once_per_device(std::atomic<uint64_t>& done, F fn) {
  const uint64_t bit = 1ull << (current_device() & 63);
  if (done.load(std::memory_order_acquire) & bit) return;
  fn();
  done.fetch_or(bit, std::memory_order_release);
}

// Operator path on compile-time transform lengths (converse2d_opct.hip): the LR rows (w), columns
// (h) and the HR rows / columns (w s, h s) have fixed plans.  Same scratch and table layouts as the
// generic op path; tw_* are the twiddle tables (exp(-2 pi i m / L), m < L) of each length.
bool op_ct_supported(int h, int w, int s);
int launch_op_ct(const float* x, const float* x0, int64_t P, int64_t C, int h, int w, int s, const float2* tw_w,
                 const float2* tw_h, const float2* tw_Hs, const float2* tw_Ws, const float2* kf, const float2* A,
                 float2* S, float2* S0, float2* SH, float* out, hipStream_t st);
// Module path (x0 = nearest(y)) at scale 2-4 with no padding on the same compile-time plans: LR rows,
// the module column pass (Phi times the tiled LR spectrum, inverse HR columns), HR rows with act.
// Same scratch (S, SH) and table (kPhiGeneric layout) as the generic module path.
bool module_ct_supported(int h, int w, int s, int pad);
int launch_module_ct(const float* x, int64_t P, int64_t C, int64_t psf_batch, int h, int w, int s, int act,
                     const float2* tw_w, const float2* tw_h, const float2* tw_Hs, const float2* tw_Ws,
                     const float2* phi, float2* S, float2* SH, float* out, hipStream_t st);

}  // namespace cvn
