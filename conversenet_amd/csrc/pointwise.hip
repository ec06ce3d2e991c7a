// Per-pixel channel-mixing kernels of the ConverseBlock (util_converse.py:253-323):
//   * channels-first LayerNorm (util_converse.py:63-68)
//   * 1x1 convolution (nn.Conv2d(cin, cout, 1)) on fp32 MFMA, with optional LayerNorm prologue,
//     exact-GELU epilogue and (alpha-scaled) residual add
//   * the whole conv2 branch  x + alpha * (W2 GELU(W1 LN(x) + b1) + b2)  in one kernel
//
// MFMA mapping (v_mfma_f32_16x16x4f32, wave64): a wave owns 64 pixels.  Lane l = 16 g + j loads a
// float4 of pixels p0 + 4j .. p0 + 4j + 3 of channel 4 ks + g for every k-step ks, so each float4
// component q is the B operand B[k = g][col = j] of an independent 16-pixel block (pixel
// p0 + 4 j + q).  The A operand A[row = j][k = g] comes from the weight matrix staged in LDS.  The
// accumulator of block q holds D[row = 4 g + r][col = j] in register r, so an output channel's four
// blocks are four consecutive pixels and leave as one float4 store.  For the fused two-layer
// branch the first layer's accumulators feed the second layer directly: register r of row block rb
// is the B operand of a k-step whose channel for lane group g is 16 rb + 4 g + r.
#include <math.h>

#include "cvn_common.h"

namespace cvn {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gelu_f(float v) { return gelu_fast(v); }

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// LayerNorm, channels first.  One thread per pixel; CT channels held in registers.
// ------------------------------------------------------------------------------------------------
template <int CT>
__global__ void __launch_bounds__(256) k_ln_cf(const float* __restrict__ x, int64_t HW,
                                               const float* __restrict__ w, const float* __restrict__ b,
                                               float eps, float* __restrict__ y) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= HW) return;
  const int64_t base = (int64_t)blockIdx.y * CT * HW + p;
  float v[CT];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    v[c] = x[base + c * HW];
    s += v[c];
  }
  const float u = s / (float)CT;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const float d = v[c] - u;
    q = fmaf(d, d, q);
  }
  const float den = sqrtf(q / (float)CT + eps);
#pragma unroll
  for (int c = 0; c < CT; ++c) y[base + c * HW] = fmaf(w[c], (v[c] - u) / den, b[c]);
}

__global__ void __launch_bounds__(256) k_ln_cf_any(const float* __restrict__ x, int64_t HW, int C,
                                                   const float* __restrict__ w, const float* __restrict__ b,
                                                   float eps, float* __restrict__ y) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= HW) return;
  const int64_t base = (int64_t)blockIdx.y * C * HW + p;
  float s = 0.f;
  for (int c = 0; c < C; ++c) s += x[base + c * HW];
  const float u = s / (float)C;
  float q = 0.f;
  for (int c = 0; c < C; ++c) {
    const float d = x[base + c * HW] - u;
    q = fmaf(d, d, q);
  }
  const float den = sqrtf(q / (float)C + eps);
  for (int c = 0; c < C; ++c) y[base + c * HW] = fmaf(w[c], (x[base + c * HW] - u) / den, b[c]);
}

// ------------------------------------------------------------------------------------------------
// shared pieces of the MFMA kernels
// ------------------------------------------------------------------------------------------------
// Stage W (ROWS x COLS, row-major in global) transposed into LDS: Wt[k * LD + i] = W[i][k].
template <int ROWS, int COLS, int LD>
__device__ __forceinline__ void stage_wt(const float* __restrict__ W, float* Wt) {
  for (int e = threadIdx.x; e < ROWS * COLS; e += blockDim.x) {
    const int i = e / COLS, k = e - i * COLS;
    Wt[k * LD + i] = W[e];
  }
}

// Load the wave's CIN x 64-pixel tile (float4 per k-step), zero beyond HW.
template <int CIN>
__device__ __forceinline__ void load_tile(const float* __restrict__ xb, int64_t HW, int64_t px, int g,
                                          float4 (&xv)[CIN / 4]) {
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    const int k = 4 * ks + g;
    xv[ks] = (px < HW) ? *(const float4*)(xb + (int64_t)k * HW + px) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Channels-first LayerNorm of the register tile (statistics over all CIN channels of each pixel;
// the four lane groups g hold disjoint channel subsets).
template <int CIN>
__device__ __forceinline__ void ln_tile(float4 (&xv)[CIN / 4], int g, const float* __restrict__ lw,
                                        const float* __restrict__ lb, float eps) {
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    s.x += xv[ks].x; s.y += xv[ks].y; s.z += xv[ks].z; s.w += xv[ks].w;
  }
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1) {
    s.x += __shfl_xor(s.x, m); s.y += __shfl_xor(s.y, m);
    s.z += __shfl_xor(s.z, m); s.w += __shfl_xor(s.w, m);
  }
  const float inv = 1.0f / (float)CIN;
  const float4 u = make_float4(s.x * inv, s.y * inv, s.z * inv, s.w * inv);
  float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    float d;
    d = xv[ks].x - u.x; q.x = fmaf(d, d, q.x);
    d = xv[ks].y - u.y; q.y = fmaf(d, d, q.y);
    d = xv[ks].z - u.z; q.z = fmaf(d, d, q.z);
    d = xv[ks].w - u.w; q.w = fmaf(d, d, q.w);
  }
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1) {
    q.x += __shfl_xor(q.x, m); q.y += __shfl_xor(q.y, m);
    q.z += __shfl_xor(q.z, m); q.w += __shfl_xor(q.w, m);
  }
  const float4 rs = make_float4(1.0f / sqrtf(q.x * inv + eps), 1.0f / sqrtf(q.y * inv + eps),
                                1.0f / sqrtf(q.z * inv + eps), 1.0f / sqrtf(q.w * inv + eps));
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    const int k = 4 * ks + g;
    const float ww = lw[k], bb = lb[k];
    xv[ks].x = fmaf(ww * rs.x, xv[ks].x - u.x, bb);
    xv[ks].y = fmaf(ww * rs.y, xv[ks].y - u.y, bb);
    xv[ks].z = fmaf(ww * rs.z, xv[ks].z - u.z, bb);
    xv[ks].w = fmaf(ww * rs.w, xv[ks].w - u.w, bb);
  }
}

// acc[rb][q] += W[16 rb + row][k] * x[k][block q]  over all k-steps of the register tile
template <int CIN, int COUT>
__device__ __forceinline__ void gemm_tile(const float4 (&xv)[CIN / 4], const float* Wt, int ld, int g, int j,
                                          v4f (&acc)[COUT / 16][4]) {
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    const float* wk = Wt + (4 * ks + g) * ld + j;
#pragma unroll
    for (int rb = 0; rb < COUT / 16; ++rb) {
      const float a = wk[16 * rb];
      acc[rb][0] = mfma4(a, xv[ks].x, acc[rb][0]);
      acc[rb][1] = mfma4(a, xv[ks].y, acc[rb][1]);
      acc[rb][2] = mfma4(a, xv[ks].z, acc[rb][2]);
      acc[rb][3] = mfma4(a, xv[ks].w, acc[rb][3]);
    }
  }
}

template <int COUT>
__device__ __forceinline__ void zero_acc(v4f (&acc)[COUT / 16][4]) {
#pragma unroll
  for (int rb = 0; rb < COUT / 16; ++rb)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[rb][q] = v4f{0.f, 0.f, 0.f, 0.f};
}

// Epilogue: bias, activation, optional alpha-scaled residual, float4 store.
template <int COUT>
__device__ __forceinline__ void store_tile(v4f (&acc)[COUT / 16][4], float* __restrict__ yb,
                                           const float* __restrict__ rb_ptr, int64_t HW, int64_t px, int g,
                                           const float* __restrict__ bias, int act,
                                           const float* __restrict__ res_scale) {
  if (px >= HW) return;
#pragma unroll
  for (int rb = 0; rb < COUT / 16; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 16 * rb + 4 * g + r;
      const float bo = bias ? bias[o] : 0.f;
      float4 v = make_float4(acc[rb][0][r] + bo, acc[rb][1][r] + bo, acc[rb][2][r] + bo, acc[rb][3][r] + bo);
      if (act == CVN_ACT_GELU) {
        v.x = gelu_f(v.x); v.y = gelu_f(v.y); v.z = gelu_f(v.z); v.w = gelu_f(v.w);
      }
      if (rb_ptr) {
        const float sc = res_scale ? res_scale[o] : 1.f;
        const float4 rr = *(const float4*)(rb_ptr + (int64_t)o * HW + px);
        v.x = fmaf(sc, v.x, rr.x); v.y = fmaf(sc, v.y, rr.y);
        v.z = fmaf(sc, v.z, rr.z); v.w = fmaf(sc, v.w, rr.w);
      }
      *(float4*)(yb + (int64_t)o * HW + px) = v;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// 1x1 conv (+ LN prologue) on MFMA.  Block = 4 waves = 256 pixels; grid (ceil(HW/256), B).
// ------------------------------------------------------------------------------------------------
template <int CIN, int COUT, bool LN>
__global__ void __launch_bounds__(256) k_conv1x1_mfma(const float* __restrict__ x, int64_t HW,
                                                      const float* __restrict__ W, const float* __restrict__ bias,
                                                      const float* __restrict__ lw, const float* __restrict__ lb,
                                                      float eps, int act, const float* residual,
                                                      const float* __restrict__ res_scale, float* y) {
  constexpr int LD = COUT + 16;
  __shared__ float Wt[CIN * LD];
  stage_wt<COUT, CIN, LD>(W, Wt);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int64_t b = blockIdx.y;
  const int64_t px = (int64_t)blockIdx.x * 256 + wave * 64 + 4 * j;
  const float* xb = x + b * CIN * HW;
  float4 xv[CIN / 4];
  load_tile<CIN>(xb, HW, px, g, xv);
  if (LN) ln_tile<CIN>(xv, g, lw, lb, eps);
  __syncthreads();
  v4f acc[COUT / 16][4];
  zero_acc<COUT>(acc);
  gemm_tile<CIN, COUT>(xv, Wt, LD, g, j, acc);
  store_tile<COUT>(acc, y + b * COUT * HW, residual ? residual + b * COUT * HW : nullptr, HW, px, g, bias, act,
                   res_scale);
}

// ConverseBlock conv2 branch: y = x + res_scale * (W2 GELU(W1 LN(x) + b1) + b2)
template <int C, int CM>
__global__ void __launch_bounds__(256) k_ln_mlp_mfma(const float* x, int64_t HW, const float* __restrict__ lw,
                                                     const float* __restrict__ lb, float eps,
                                                     const float* __restrict__ W1, const float* __restrict__ b1,
                                                     const float* __restrict__ W2, const float* __restrict__ b2,
                                                     const float* __restrict__ res_scale, float* y) {
  constexpr int LD1 = CM + 16;  // W1t[k][i], k < C, i < CM
  constexpr int LD2 = C + 16;   // W2t[k][i], k < CM, i < C
  __shared__ float W1t[C * LD1];
  __shared__ float W2t[CM * LD2];
  stage_wt<CM, C, LD1>(W1, W1t);
  stage_wt<C, CM, LD2>(W2, W2t);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int64_t b = blockIdx.y;
  const int64_t px = (int64_t)blockIdx.x * 256 + wave * 64 + 4 * j;
  const float* xb = x + b * C * HW;
  float4 xv[C / 4];
  load_tile<C>(xb, HW, px, g, xv);
  ln_tile<C>(xv, g, lw, lb, eps);
  __syncthreads();
  v4f h[CM / 16][4];
  zero_acc<CM>(h);
  gemm_tile<C, CM>(xv, W1t, LD1, g, j, h);
  // bias + GELU on the hidden activations (channel 16 rb + 4 g + r)
#pragma unroll
  for (int rb = 0; rb < CM / 16; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float bo = b1[16 * rb + 4 * g + r];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[rb][q][r] = gelu_f(h[rb][q][r] + bo);
    }
  v4f acc[C / 16][4];
  zero_acc<C>(acc);
#pragma unroll
  for (int rb = 0; rb < CM / 16; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float* wk = W2t + (16 * rb + 4 * g + r) * LD2 + j;
#pragma unroll
      for (int ob = 0; ob < C / 16; ++ob) {
        const float a = wk[16 * ob];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[ob][q] = mfma4(a, h[rb][q][r], acc[ob][q]);
      }
    }
  store_tile<C>(acc, y + b * C * HW, xb, HW, px, g, b2, CVN_ACT_NONE, res_scale);
}

// Plain VALU 1x1 conv for channel counts / sizes the MFMA tiles do not cover (e.g. 1 or 3 channels).
__global__ void __launch_bounds__(256) k_conv1x1_any(const float* __restrict__ x, int64_t HW, int Cin,
                                                     const float* __restrict__ W, const float* __restrict__ bias,
                                                     int Cout, int act, const float* residual,
                                                     const float* __restrict__ res_scale, float* y) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= HW) return;
  const int64_t b = blockIdx.y;
  const float* xb = x + b * Cin * HW + p;
  for (int o = 0; o < Cout; ++o) {
    float acc = bias ? bias[o] : 0.f;
    for (int c = 0; c < Cin; ++c) acc = fmaf(W[o * Cin + c], xb[(int64_t)c * HW], acc);
    if (act == CVN_ACT_GELU) acc = gelu_f(acc);
    const int64_t oi = (b * Cout + o) * HW + p;
    if (residual) acc = fmaf(res_scale ? res_scale[o] : 1.f, acc, residual[oi]);
    y[oi] = acc;
  }
}

}  // namespace cvn

using namespace cvn;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int CIN, int COUT, bool LN>
int launch_mfma(const float* x, int64_t B, int64_t HW, const float* W, const float* bias, const float* lw,
                const float* lb, float eps, int act, const float* residual, const float* res_scale, float* y,
                hipStream_t st) {
  dim3 grid((unsigned)((HW + 255) / 256), (unsigned)B);
  hipLaunchKernelGGL((k_conv1x1_mfma<CIN, COUT, LN>), grid, dim3(256), 0, st, x, HW, W, bias, lw, lb, eps, act,
                     residual, res_scale, y);
  return check_launch("1x1 conv");
}

template <bool LN>
int dispatch_mfma(int64_t Cin, int64_t Cout, const float* x, int64_t B, int64_t HW, const float* W,
                  const float* bias, const float* lw, const float* lb, float eps, int act, const float* residual,
                  const float* res_scale, float* y, hipStream_t st, bool* done) {
  *done = true;
#define CVN_CASE(ci, co) \
  if (Cin == ci && Cout == co) return launch_mfma<ci, co, LN>(x, B, HW, W, bias, lw, lb, eps, act, residual, res_scale, y, st);
  CVN_CASE(64, 64) CVN_CASE(64, 128) CVN_CASE(128, 64) CVN_CASE(128, 128) CVN_CASE(16, 64) CVN_CASE(64, 16)
  CVN_CASE(32, 32) CVN_CASE(32, 64) CVN_CASE(64, 32)
#undef CVN_CASE
  *done = false;
  return CVN_OK;
}

int conv_args_ok(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* W, int64_t Cout, int act,
                 float* y) {
  if (!x || !W || !y) return fail(CVN_ERR_ARG, "null pointer");
  if (B < 0 || Cin < 1 || Cout < 1 || HW < 0) return fail(CVN_ERR_ARG, "bad shape");
  if (act != CVN_ACT_NONE && act != CVN_ACT_GELU) return fail(CVN_ERR_ARG, "bad activation");
  if (B > 65535) return fail(CVN_ERR_UNSUPPORTED, "batch exceeds 65535");
  return CVN_OK;
}

}  // namespace

extern "C" int cvn_layernorm_cf_f32(const float* x, int64_t B, int64_t C, int64_t HW, const float* weight,
                                    const float* bias, float eps, float* y, cvn_stream_t stream) {
  if (!x || !weight || !bias || !y) return fail(CVN_ERR_ARG, "null pointer");
  if (B < 0 || C < 1 || HW < 0) return fail(CVN_ERR_ARG, "bad shape");
  if (B > 65535) return fail(CVN_ERR_UNSUPPORTED, "batch exceeds 65535");
  if (B == 0 || HW == 0) return CVN_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((HW + 255) / 256), (unsigned)B);
  switch (C) {
    case 64: hipLaunchKernelGGL(k_ln_cf<64>, grid, dim3(256), 0, st, x, HW, weight, bias, eps, y); break;
    case 128: hipLaunchKernelGGL(k_ln_cf<128>, grid, dim3(256), 0, st, x, HW, weight, bias, eps, y); break;
    case 32: hipLaunchKernelGGL(k_ln_cf<32>, grid, dim3(256), 0, st, x, HW, weight, bias, eps, y); break;
    default: hipLaunchKernelGGL(k_ln_cf_any, grid, dim3(256), 0, st, x, HW, (int)C, weight, bias, eps, y); break;
  }
  return check_launch("layernorm");
}

static int conv_impl(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* ln_w, const float* ln_b,
                     float ln_eps, const float* weight, const float* bias, int64_t Cout, int act,
                     const float* residual, const float* res_scale, float* y, hipStream_t st) {
  int rc = conv_args_ok(x, B, Cin, HW, weight, Cout, act, y);
  if (rc != CVN_OK) return rc;
  if (B == 0 || HW == 0) return CVN_OK;
  const bool vec_ok = (HW % 4 == 0) && aligned16(x) && aligned16(y) && (!residual || aligned16(residual));
  if (vec_ok) {
    bool done = false;
    if (ln_w)
      rc = dispatch_mfma<true>(Cin, Cout, x, B, HW, weight, bias, ln_w, ln_b, ln_eps, act, residual, res_scale, y,
                               st, &done);
    else
      rc = dispatch_mfma<false>(Cin, Cout, x, B, HW, weight, bias, nullptr, nullptr, 0.f, act, residual,
                                res_scale, y, st, &done);
    if (done) return rc;
  }
  if (ln_w) return fail(CVN_ERR_UNSUPPORTED, "LayerNorm-fused 1x1 conv needs an MFMA tile shape");
  dim3 grid((unsigned)((HW + 255) / 256), (unsigned)B);
  hipLaunchKernelGGL(k_conv1x1_any, grid, dim3(256), 0, st, x, HW, (int)Cin, weight, bias, (int)Cout, act,
                     residual, res_scale, y);
  return check_launch("1x1 conv");
}

extern "C" int cvn_conv1x1_f32(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* weight,
                               const float* bias, int64_t Cout, int act, const float* residual,
                               const float* res_scale, float* y, cvn_stream_t stream) {
  return conv_impl(x, B, Cin, HW, nullptr, nullptr, 0.f, weight, bias, Cout, act, residual, res_scale, y,
                   (hipStream_t)stream);
}

extern "C" int cvn_ln_conv1x1_f32(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* ln_w,
                                  const float* ln_b, float ln_eps, const float* weight, const float* bias,
                                  int64_t Cout, int act, const float* residual, const float* res_scale, float* y,
                                  cvn_stream_t stream) {
  if (!ln_w || !ln_b) return fail(CVN_ERR_ARG, "null LayerNorm parameters");
  return conv_impl(x, B, Cin, HW, ln_w, ln_b, ln_eps, weight, bias, Cout, act, residual, res_scale, y,
                   (hipStream_t)stream);
}

extern "C" int cvn_ln_mlp_residual_f32(const float* x, int64_t B, int64_t C, int64_t HW, const float* ln_w,
                                       const float* ln_b, float ln_eps, const float* w1, const float* b1,
                                       int64_t Cmid, const float* w2, const float* b2, const float* res_scale,
                                       float* y, cvn_stream_t stream) {
  if (!x || !ln_w || !ln_b || !w1 || !b1 || !w2 || !b2 || !y) return fail(CVN_ERR_ARG, "null pointer");
  if (B < 0 || HW < 0) return fail(CVN_ERR_ARG, "bad shape");
  if (B > 65535) return fail(CVN_ERR_UNSUPPORTED, "batch exceeds 65535");
  if (B == 0 || HW == 0) return CVN_OK;
  if (HW % 4 != 0 || !aligned16(x) || !aligned16(y))
    return fail(CVN_ERR_UNSUPPORTED, "fused branch needs HW %% 4 == 0 and 16-byte aligned buffers");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((HW + 255) / 256), (unsigned)B);
  if (C == 64 && Cmid == 128) {
    hipLaunchKernelGGL((k_ln_mlp_mfma<64, 128>), grid, dim3(256), 0, st, x, HW, ln_w, ln_b, ln_eps, w1, b1, w2, b2,
                       res_scale, y);
  } else if (C == 32 && Cmid == 64) {
    hipLaunchKernelGGL((k_ln_mlp_mfma<32, 64>), grid, dim3(256), 0, st, x, HW, ln_w, ln_b, ln_eps, w1, b1, w2, b2,
                       res_scale, y);
  } else {
    return fail(CVN_ERR_UNSUPPORTED, "fused branch supports (C, Cmid) in {(64,128), (32,64)}");
  }
  return check_launch("fused LN-MLP branch");
}
