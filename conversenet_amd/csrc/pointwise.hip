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

#include <algorithm>

#include "cvn_common.h"

namespace cvn {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gelu_f(float v) { return gelu_fast(v); }

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// LayerNorm, channels first.  One thread per pixel; CT channels held in registers; output stored
// non-temporal (see stq_nt).
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
  for (int c = 0; c < CT; ++c) __builtin_nontemporal_store(fmaf(w[c], (v[c] - u) / den, b[c]), &y[base + c * HW]);
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
  for (int c = 0; c < C; ++c)
    __builtin_nontemporal_store(fmaf(w[c], (x[base + c * HW] - u) / den, b[c]), &y[base + c * HW]);
}

// ------------------------------------------------------------------------------------------------
// shared pieces of the MFMA kernels.  A wave owns 16 Q pixels: lane l = 16 g + j holds pixels
// p0 + Q j .. p0 + Q j + Q - 1 (Q = 2: one float2 per channel), so per k-step the Q register
// components are the B operands of Q independent 16-pixel blocks.
// ------------------------------------------------------------------------------------------------
// Stage W (ROWS x COLS, row-major in global) transposed into LDS: Wt[k * LD + i] = W[i][k].
// Consecutive threads take consecutive rows i of one column k, so the LDS writes are contiguous.
template <int ROWS, int COLS, int LD>
__device__ __forceinline__ void stage_wt(const float* __restrict__ W, float* Wt) {
  for (int e = threadIdx.x; e < ROWS * COLS; e += blockDim.x) {
    const int k = e / ROWS, i = e - k * ROWS;
    Wt[k * LD + i] = W[i * COLS + k];
  }
}

// Stage a per-channel parameter vector into LDS (def where the pointer is null).  Read from LDS
// inside the tile loop, these stay out of the vector registers; read from global memory, the
// compiler keeps every lane's copy live across the loop.
template <int N>
__device__ __forceinline__ void stage_vec(const float* src, float def, float* dst) {
  for (int e = threadIdx.x; e < N; e += blockDim.x) dst[e] = src ? src[e] : def;
}

template <int Q>
__device__ __forceinline__ void ldq(const float* p, float (&v)[Q]) {
  if constexpr (Q == 4) {
    const float4 t = *(const float4*)p;
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else if constexpr (Q == 2) {
    const float2 t = *(const float2*)p;
    v[0] = t.x; v[1] = t.y;
  } else {
    v[0] = *p;
  }
}
template <int Q>
__device__ __forceinline__ void stq(float* p, const float (&v)[Q]) {
  if constexpr (Q == 4) *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  else if constexpr (Q == 2) *(float2*)p = make_float2(v[0], v[1]);
  else *p = v[0];
}
// The same store with the non-temporal cache policy: for outputs written once per launch and larger
// than L2, it keeps them from evicting the lines the launch still reads (the LayerNorm kernel at the
// cfg3 shape: 0.102 -> 0.078 ms; the 1x1 GEMM epilogue: 0.152 -> 0.138 ms).  The fused block tail
// keeps ordinary stores: its outputs feed the next kernel at once, and there the streaming store
// measured no gain.
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
typedef float nt_f32x2 __attribute__((ext_vector_type(2)));
template <int Q>
__device__ __forceinline__ void stq_nt(float* p, const float (&v)[Q]) {
  if constexpr (Q == 4) __builtin_nontemporal_store((nt_f32x4){v[0], v[1], v[2], v[3]}, (nt_f32x4*)p);
  else if constexpr (Q == 2) __builtin_nontemporal_store((nt_f32x2){v[0], v[1]}, (nt_f32x2*)p);
  else __builtin_nontemporal_store(v[0], p);
}

// Addressing: every access is a wave-uniform pointer (image, channel row, wave's first pixel) plus
// a 32-bit per-lane byte offset, so the compiler can use the scalar-base form of the global memory
// instructions instead of keeping a 64-bit address per access in vector registers.
__device__ __forceinline__ const float* at_off(const float* p, uint32_t off) {
  return (const float*)((const char*)p + off);
}
__device__ __forceinline__ float* at_off(float* p, uint32_t off) { return (float*)((char*)p + off); }

// Load the wave's CIN x 16Q-pixel tile (xw: channel 0 at the wave's first pixel; xoff: lane
// offset of channel g, pixel Q j), zero beyond HW.
template <int CIN, int Q>
__device__ __forceinline__ void load_tile(const float* xw, int64_t HW, bool inb, uint32_t xoff,
                                          float (&xv)[CIN / 4][Q]) {
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    if (inb) {
      ldq<Q>(at_off(xw + 4 * ks * HW, xoff), xv[ks]);
    } else {
#pragma unroll
      for (int q = 0; q < Q; ++q) xv[ks][q] = 0.f;
    }
  }
}

// Channels-first LayerNorm of the register tile (statistics over all CIN channels of each pixel;
// the four lane groups g hold disjoint channel subsets).
template <int CIN, int Q>
__device__ __forceinline__ void ln_tile(float (&xv)[CIN / 4][Q], int g, const float* lw, const float* lb,
                                        float eps) {
  const float inv = 1.0f / (float)CIN;
  float u[Q], rs[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    float s = 0.f;
#pragma unroll
    for (int ks = 0; ks < CIN / 4; ++ks) s += xv[ks][q];
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    u[q] = s * inv;
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    float v = 0.f;
#pragma unroll
    for (int ks = 0; ks < CIN / 4; ++ks) {
      const float d = xv[ks][q] - u[q];
      v = fmaf(d, d, v);
    }
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    rs[q] = 1.0f / sqrtf(v * inv + eps);
  }
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    const int k = 4 * ks + g;
    const float ww = lw[k], bb = lb[k];
#pragma unroll
    for (int q = 0; q < Q; ++q) xv[ks][q] = fmaf(ww * rs[q], xv[ks][q] - u[q], bb);
  }
}

// Keeps the compiler from moving memory operations across this point.  The GEMM loops place it
// once per k-step so that only the next step's weights are loaded ahead: without it the scheduler
// front-loads every LDS weight read of the unrolled loop, and the registers that costs halve the
// occupancy.
__device__ __forceinline__ void mem_fence_sched() { asm volatile("" ::: "memory"); }

// A copy of the (wave-uniform) plane stride that the compiler cannot see through.  Row offsets
// computed from it inside the tile loop stay per-iteration scalar arithmetic; computed from the
// kernel argument they are hoisted out of the loop as 64-bit values, which spill into vector
// registers.
__device__ __forceinline__ int64_t opaque_stride(int64_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// acc[rb][q] += W[16 rb + row][k] * x[k][block q]  over all k-steps of the register tile; the
// weights of step ks + 1 are read while step ks runs.
template <int CIN, int COUT, int Q>
__device__ __forceinline__ void gemm_tile(const float (&xv)[CIN / 4][Q], const float* Wt, int ld, int g, int j,
                                          v4f (&acc)[COUT / 16][Q]) {
  float a[2][COUT / 16];
#pragma unroll
  for (int rb = 0; rb < COUT / 16; ++rb) a[0][rb] = Wt[g * ld + j + 16 * rb];
#pragma unroll
  for (int ks = 0; ks < CIN / 4; ++ks) {
    if (ks + 1 < CIN / 4) {
      const float* wk = Wt + (4 * (ks + 1) + g) * ld + j;
#pragma unroll
      for (int rb = 0; rb < COUT / 16; ++rb) a[(ks + 1) & 1][rb] = wk[16 * rb];
    }
#pragma unroll
    for (int rb = 0; rb < COUT / 16; ++rb)
#pragma unroll
      for (int q = 0; q < Q; ++q) acc[rb][q] = mfma4(a[ks & 1][rb], xv[ks][q], acc[rb][q]);
    mem_fence_sched();
  }
}

template <int COUT, int Q>
__device__ __forceinline__ void zero_acc(v4f (&acc)[COUT / 16][Q]) {
#pragma unroll
  for (int rb = 0; rb < COUT / 16; ++rb)
#pragma unroll
    for (int q = 0; q < Q; ++q) acc[rb][q] = v4f{0.f, 0.f, 0.f, 0.f};
}

// Epilogue: bias, activation, optional alpha-scaled residual, vector store.  yw / rw: output and
// residual at channel 0 and the wave's first pixel; yoff: lane offset of channel 4 g, pixel Q j;
// bias / res_scale: per-channel vectors staged in LDS.
template <int COUT, int Q>
__device__ __forceinline__ void store_tile(v4f (&acc)[COUT / 16][Q], float* yw, const float* rw, int64_t HW,
                                           bool inb, uint32_t yoff, int g, const float* bias, int act,
                                           const float* res_scale) {
  if (!inb) return;
#pragma unroll
  for (int rb = 0; rb < COUT / 16; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 16 * rb + 4 * g + r;
      const int64_t row = (int64_t)(16 * rb + r) * HW;
      const float bo = bias[o];
      float v[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        v[q] = acc[rb][q][r] + bo;
        if (act == CVN_ACT_GELU) v[q] = gelu_f(v[q]);
      }
      if (rw) {
        const float sc = res_scale[o];
        float rr[Q];
        ldq<Q>(at_off(rw + row, yoff), rr);
#pragma unroll
        for (int q = 0; q < Q; ++q) v[q] = fmaf(sc, v[q], rr[q]);
      }
      stq_nt<Q>(at_off(yw + row, yoff), v);
    }
  }
}

// Tiles: a block of NW waves covers 16 NW Q consecutive pixels of one image; tile t is image
// t / tpb, pixels (t % tpb) 16 NW Q ...  Blocks stage the weights once and then loop over tiles
// t = blockIdx.x, blockIdx.x + gridDim.x, ...  The empty asm with a memory clobber at the top of
// each iteration keeps the compiler from hoisting the (loop-invariant) LDS weight reads into
// registers, which would cost occupancy.  Returns the wave's first pixel (wave-uniform).
__device__ __forceinline__ int64_t tile_px(int64_t t, int64_t tpb, int Q, int NW, int wave, int64_t* b) {
  *b = t / tpb;
  return (t - *b * tpb) * (16 * NW * Q) + wave * (16 * Q);
}

// ------------------------------------------------------------------------------------------------
// fp32 products on the fp16 matrix cores ("split fp16").  Every operand x is split as x = x_h + x_l,
// x_h = fp16(x) and x_l = fp16(x - x_h), both rounded toward zero (x - x_h is exact in fp32), so
// |x - x_h - x_l| < 2^-20 |x|; a product is formed as a_l b_h + a_h b_l + a_h b_h (three
// v_mfma_f32_16x16x32_f16, each product exact in the fp32 accumulator), dropping a_l b_l (< 2^-20
// |a b|).  fp16 inputs below the normal range are kept by the matrix cores (gradual underflow), so
// small values lose no relative accuracy beyond 2^-24 absolute.  A 16 x 16 x 32 block update then
// takes three of these MFMAs (8192 multiply-adds each, half the issue time of one 16x16x4 fp32 MFMA)
// instead of eight fp32 MFMAs.  fp16's range ends at 65504: a k-chunk whose activations exceed it in
// any lane of the wave is multiplied on the fp32 matrix cores instead (weights rebuilt as x_h + x_l),
// so no input range is lost.
// Operand layout of the 16x16x32 MFMA: lane l = 16 g + j holds A[row j][k = 8 g + e] and
// B[k = 8 g + e][col j], e < 8; D as for the fp32 MFMAs (lane 16 g + j: rows 4 g + r, col j).  The k
// slot 8 g + e (e = 4 hf + r) of input chunk c is channel 16 (2 c + hf) + 4 g + r: the channels lane
// group g holds in the accumulator layout (channel 16 rb + 4 g + r in register r of row block rb), so
// a layer's accumulators feed the next layer's B operand directly.
// ------------------------------------------------------------------------------------------------
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr float kF16Max = 65504.f;

__device__ __forceinline__ void split_f16(const float (&x)[8], f16x8& h, f16x8& l) {
  u32x4_t H, L;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto hp = __builtin_amdgcn_cvt_pkrtz(x[2 * i], x[2 * i + 1]);
    const auto lp = __builtin_amdgcn_cvt_pkrtz(x[2 * i] - (float)hp[0], x[2 * i + 1] - (float)hp[1]);
    H[i] = __builtin_bit_cast(unsigned, hp);
    L[i] = __builtin_bit_cast(unsigned, lp);
  }
  h = __builtin_bit_cast(f16x8, H);
  l = __builtin_bit_cast(f16x8, L);
}

// Weights (N outputs x K inputs, row-major fp32) in LDS for gemm_f16s: for input chunk c, output
// block ob and lane 16 g + j, 16 bytes of high parts (W[16 ob + j][channel of k slot 8 g + e], e < 8),
// and 1 KB further on the 16 bytes of low parts: consecutive lanes read consecutive 16-byte words.
template <int N, int K>
__device__ __forceinline__ void stage_f16s(const float* __restrict__ W, _Float16* Wl) {
  for (int e = threadIdx.x; e < N * K; e += blockDim.x) {
    const int e8 = e & 7, lj = (e >> 3) & 63, cob = e >> 9;
    const int g = lj >> 4, j = lj & 15, hf = e8 >> 2, r = e8 & 3;
    const int ob = cob % (N / 16), c = cob / (N / 16);
    const float w = W[(16 * ob + j) * K + 16 * (2 * c + hf) + 4 * g + r];
    const auto hp = __builtin_amdgcn_cvt_pkrtz(w, 0.f);
    const auto lp = __builtin_amdgcn_cvt_pkrtz(w - (float)hp[0], 0.f);
    Wl[cob * 1024 + lj * 8 + e8] = (_Float16)hp[0];
    Wl[cob * 1024 + 512 + lj * 8 + e8] = (_Float16)lp[0];
  }
}

// acc[ob][q] += W[16 ob + j][k] v[k] over all K input channels; v in the accumulator layout.
template <int K, int N, int Q>
__device__ __forceinline__ void gemm_f16s(const v4f (&v)[K / 16][Q], const _Float16* Wl, int lane,
                                          v4f (&acc)[N / 16][Q]) {
#pragma unroll
  for (int c = 0; c < K / 32; ++c) {
    float xb[Q][8];
    float mx = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xb[q][e] = v[2 * c + (e >> 2)][q][e & 3];
        mx = fmaxf(mx, fabsf(xb[q][e]));
      }
    // NaN compares false here and passes through the fp16 products as NaN
    if (__builtin_amdgcn_ballot_w64(mx > kF16Max) == 0) {
      f16x8 bh[Q], bl[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) split_f16(xb[q], bh[q], bl[q]);
#pragma unroll
      for (int ob = 0; ob < N / 16; ++ob) {
        const u32x4_t* wp = (const u32x4_t*)(Wl + (c * (N / 16) + ob) * 1024) + lane;
        const f16x8 ah = __builtin_bit_cast(f16x8, wp[0]), al = __builtin_bit_cast(f16x8, wp[64]);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          v4f t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[q], acc[ob][q], 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[q], t, 0, 0, 0);
          acc[ob][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[q], t, 0, 0, 0);
        }
        mem_fence_sched();
      }
    } else {
#pragma unroll
      for (int ob = 0; ob < N / 16; ++ob) {
        const u32x4_t* wp = (const u32x4_t*)(Wl + (c * (N / 16) + ob) * 1024) + lane;
        const f16x8 ah = __builtin_bit_cast(f16x8, wp[0]), al = __builtin_bit_cast(f16x8, wp[64]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float w = (float)ah[e] + (float)al[e];
#pragma unroll
          for (int q = 0; q < Q; ++q) acc[ob][q] = mfma4(w, xb[q][e], acc[ob][q]);
        }
        mem_fence_sched();
      }
    }
  }
}

// Loads a (channels x pixels) tile in the accumulator layout: channel 16 rb + 4 g + r in register r of
// row block rb, Q consecutive pixels per lane (zeros outside the image).
template <int N, int Q>
__device__ __forceinline__ void load_acc(const float* w, int64_t hw, bool inb, uint32_t yoff, v4f (&v)[N / 16][Q]) {
#pragma unroll
  for (int rb = 0; rb < N / 16; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float rr[Q];
      if (inb) {
        ldq<Q>(at_off(w + (int64_t)(16 * rb + r) * hw, yoff), rr);
      } else {
#pragma unroll
        for (int q = 0; q < Q; ++q) rr[q] = 0.f;
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) v[rb][q][r] = rr[q];
    }
}

// LayerNorm over the C channels of v, held in the accumulator layout (16 per lane for C = 64; the
// other lane groups of the same pixel block are lanes j + 16, j + 32, j + 48).
template <int C, int Q>
__device__ __forceinline__ void ln_acc(const v4f (&v)[C / 16][Q], const float* w, const float* bb, float eps, int g,
                                       v4f (&out)[C / 16][Q]) {
  const float inv = 1.0f / (float)C;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    float su = 0.f;
#pragma unroll
    for (int rb = 0; rb < C / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) su += v[rb][q][r];
    su += __shfl_xor(su, 16);
    su += __shfl_xor(su, 32);
    const float u = su * inv;
    float va = 0.f;
#pragma unroll
    for (int rb = 0; rb < C / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float d = v[rb][q][r] - u;
        va = fmaf(d, d, va);
      }
    va += __shfl_xor(va, 16);
    va += __shfl_xor(va, 32);
    const float rs = 1.0f / sqrtf(va * inv + eps);
#pragma unroll
    for (int rb = 0; rb < C / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 16 * rb + 4 * g + r;
        out[rb][q][r] = fmaf(w[o] * rs, v[rb][q][r] - u, bb[o]);
      }
  }
}

// ------------------------------------------------------------------------------------------------
// 1x1 conv (+ LN prologue) on MFMA.  Block = NW waves; persistent over pixel tiles.
// ------------------------------------------------------------------------------------------------
template <int CIN, int COUT, bool LN, int Q, int NW, bool F16S>
__global__ void __launch_bounds__(64 * NW) k_conv1x1_mfma(const float* __restrict__ x, int64_t HW, int64_t tpb,
                                                      int64_t ntiles, const float* __restrict__ W,
                                                      const float* __restrict__ bias, const float* __restrict__ lw,
                                                      const float* __restrict__ lb, float eps, int act,
                                                      const float* residual, const float* __restrict__ res_scale,
                                                      float* y) {
  // F16S: split-fp16 products (whole 32-channel input chunks), else fp32 MFMAs
  constexpr int LD = COUT + 16;  // (4 ks + g) LD + j + 16 rb: 16 g + j distinct banks
  __shared__ __align__(16) float Wt[F16S ? COUT * CIN : CIN * LD];
  __shared__ float prm[2 * COUT + 2 * CIN];  // bias, residual scale, LN weight, LN bias
  if constexpr (F16S) stage_f16s<COUT, CIN>(W, (_Float16*)Wt);
  else stage_wt<COUT, CIN, LD>(W, Wt);
  stage_vec<COUT>(bias, 0.f, prm);
  stage_vec<COUT>(res_scale, 1.f, prm + COUT);
  if (LN) {
    stage_vec<CIN>(lw, 1.f, prm + 2 * COUT);
    stage_vec<CIN>(lb, 0.f, prm + 2 * COUT + CIN);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, j = lane & 15;
  const uint32_t xoff = (uint32_t)(((int64_t)g * HW + Q * j) * 4);
  const uint32_t yoff = (uint32_t)(((int64_t)4 * g * HW + Q * j) * 4), yoff0 = (uint32_t)((int64_t)4 * g * HW * 4);
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    mem_fence_sched();
    const int64_t hw = opaque_stride(HW);
    int64_t b;
    const int64_t pw = tile_px(t, tpb, Q, NW, wave, &b);
    if (F16S && pw >= hw) continue;  // a wave wholly past the image end (wave-uniform)
    const bool inb = pw + Q * j < hw;
    v4f acc[COUT / 16][Q];
    zero_acc<COUT, Q>(acc);
    if constexpr (F16S) {
      v4f xv[CIN / 16][Q];
      // lanes past the image end load the wave's first pixel (valid, pw < hw), so the loads issue
      // without a branch each (measured 8 % faster here; the block tail keeps the guarded form,
      // which measured 2 % faster there); those lanes' values never reach an output
      load_acc<CIN, Q>(x + b * CIN * hw + pw, hw, true, inb ? yoff : yoff0, xv);
      if (LN) ln_acc<CIN, Q>(xv, prm + 2 * COUT, prm + 2 * COUT + CIN, eps, g, xv);
      gemm_f16s<CIN, COUT, Q>(xv, (const _Float16*)Wt, lane, acc);
    } else {
      float xv[CIN / 4][Q];
      load_tile<CIN, Q>(x + b * CIN * hw + pw, hw, inb, xoff, xv);
      if (LN) ln_tile<CIN, Q>(xv, g, prm + 2 * COUT, prm + 2 * COUT + CIN, eps);
      gemm_tile<CIN, COUT, Q>(xv, Wt, LD, g, j, acc);
    }
    store_tile<COUT, Q>(acc, y + b * COUT * hw + pw, residual ? residual + b * COUT * hw + pw : nullptr, hw, inb,
                        yoff, g, prm, act, prm + COUT);
  }
}

// ConverseBlock conv2 branch: y = x + res_scale * (W2 GELU(W1 LN(x) + b1) + b2)
template <int C, int CM, int Q, int NW>
__global__ void __launch_bounds__(64 * NW) k_ln_mlp_mfma(const float* x, int64_t HW, int64_t tpb, int64_t ntiles,
                                                     const float* __restrict__ lw, const float* __restrict__ lb,
                                                     float eps, const float* __restrict__ W1,
                                                     const float* __restrict__ b1, const float* __restrict__ W2,
                                                     const float* __restrict__ b2,
                                                     const float* __restrict__ res_scale, float* y) {
  static_assert(C % 32 == 0 && CM % 32 == 0, "split-fp16 GEMM chunks");
  __shared__ __align__(16) _Float16 W1l[2 * CM * C];  // stage_f16s layouts
  __shared__ __align__(16) _Float16 W2l[2 * C * CM];
  __shared__ float prm[CM + 4 * C];  // b1, b2, residual scale, LN weight, LN bias
  stage_f16s<CM, C>(W1, W1l);
  stage_f16s<C, CM>(W2, W2l);
  stage_vec<CM>(b1, 0.f, prm);
  stage_vec<C>(b2, 0.f, prm + CM);
  stage_vec<C>(res_scale, 1.f, prm + CM + C);
  stage_vec<C>(lw, 1.f, prm + CM + 2 * C);
  stage_vec<C>(lb, 0.f, prm + CM + 3 * C);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, j = lane & 15;
  const uint32_t yoff = (uint32_t)(((int64_t)4 * g * HW + Q * j) * 4);
  for (int64_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    mem_fence_sched();
    const int64_t hw = opaque_stride(HW);
    int64_t b;
    const int64_t pw = tile_px(t, tpb, Q, NW, wave, &b);
    const bool inb = pw + Q * j < hw;
    const float* xw = x + b * C * hw + pw;
    v4f h[CM / 16][Q];
    {
      v4f xv[C / 16][Q];
      load_acc<C, Q>(xw, hw, inb, yoff, xv);
      ln_acc<C, Q>(xv, prm + CM + 2 * C, prm + CM + 3 * C, eps, g, xv);
      zero_acc<CM, Q>(h);
      gemm_f16s<C, CM, Q>(xv, W1l, lane, h);
    }
    // bias + GELU on the hidden activations (channel 16 rb + 4 g + r)
#pragma unroll
    for (int rb = 0; rb < CM / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float bo = prm[16 * rb + 4 * g + r];
#pragma unroll
        for (int q = 0; q < Q; ++q) h[rb][q][r] = gelu_f(h[rb][q][r] + bo);
      }
    v4f acc[C / 16][Q];
    zero_acc<C, Q>(acc);
    gemm_f16s<CM, C, Q>(h, W2l, lane, acc);
    store_tile<C, Q>(acc, y + b * C * hw + pw, xw, hw, inb, yoff, g, prm + CM, CVN_ACT_NONE, prm + CM + C);
  }
}

// ConverseBlock tail in one kernel: y' = x + s1 (W0 t + b0) (the first branch's last 1x1 and its
// residual), then  out = y' + s2 (W2 GELU(W1 LN(y') + b1) + b2)  (the second branch).  y' stays in
// registers in the accumulator layout (lane group g holds channels 16 rb + 4 g + r of pixel block
// j), which is the B-operand layout of the next layer's k-steps, so neither y' nor LN(y') reaches
// memory.  out may alias x: every pixel's x is read by the lanes that later write it.  With HEAD,
// the next block's first layer follows on the same registers: th = GELU(Wh LNh(out) + bh)
// (CIN channels), so the next block does not read `out` again before its Converse2D.
struct TailArgs {
  const float* t;  // (B, CIN, HW)
  const float* x;  // (B, C, HW)
  int64_t HW, tpb, ntiles;
  const float *W0, *b0, *s1, *lw, *lb, *W1, *b1, *W2, *b2, *s2;
  float eps;
  float* y;  // (B, C, HW)
  const float *hlw, *hlb, *Wh, *bh;  // HEAD: next block's LayerNorm and 1x1 (CIN x C)
  float heps;
  float* th;  // HEAD: (B, CIN, HW)
  int t_act;  // CVN_ACT_GELU: the first layer's input is GELU(t)
};

// Stores an accumulator-layout tile (channel 16 rb + 4 g + r, Q consecutive pixels per lane).
template <int N, int Q>
__device__ __forceinline__ void store_acc(const v4f (&v)[N / 16][Q], float* yw, int64_t hw, uint32_t yoff) {
#pragma unroll
  for (int rb = 0; rb < N / 16; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float o[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) o[q] = v[rb][q][r];
      stq<Q>(at_off(yw + (int64_t)(16 * rb + r) * hw, yoff), o);
    }
}

template <int CIN, int C, int CM, int Q, int NW, bool HEAD, bool GIN>
__global__ void __launch_bounds__(64 * NW) k_conv_ln_mlp_mfma(TailArgs a) {
  static_assert(CIN % 32 == 0 && C % 32 == 0 && CM % 32 == 0, "split-fp16 GEMM chunks");
  constexpr int NP = 6 * C + CM + (HEAD ? 2 * C + CIN : 0);
  __shared__ __align__(16) _Float16 W0l[2 * C * CIN];  // stage_f16s layouts
  __shared__ __align__(16) _Float16 W1l[2 * CM * C];
  __shared__ __align__(16) _Float16 W2l[2 * C * CM];
  __shared__ __align__(16) _Float16 Whl[HEAD ? 2 * CIN * C : 8];
  __shared__ float prm[NP];  // b0, s1, LN weight, LN bias, b2, s2, b1 [, head LN weight, bias, head bias]
  stage_f16s<C, CIN>(a.W0, W0l);
  stage_f16s<CM, C>(a.W1, W1l);
  stage_f16s<C, CM>(a.W2, W2l);
  stage_vec<C>(a.b0, 0.f, prm);
  stage_vec<C>(a.s1, 1.f, prm + C);
  stage_vec<C>(a.lw, 1.f, prm + 2 * C);
  stage_vec<C>(a.lb, 0.f, prm + 3 * C);
  stage_vec<C>(a.b2, 0.f, prm + 4 * C);
  stage_vec<C>(a.s2, 1.f, prm + 5 * C);
  stage_vec<CM>(a.b1, 0.f, prm + 6 * C);
  if (HEAD) {
    stage_f16s<CIN, C>(a.Wh, Whl);
    stage_vec<C>(a.hlw, 1.f, prm + 6 * C + CM);
    stage_vec<C>(a.hlb, 0.f, prm + 7 * C + CM);
    stage_vec<CIN>(a.bh, 0.f, prm + 8 * C + CM);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, j = lane & 15;
  const uint32_t yoff = (uint32_t)(((int64_t)4 * g * a.HW + Q * j) * 4);
  for (int64_t tt = blockIdx.x; tt < a.ntiles; tt += gridDim.x) {
    mem_fence_sched();
    const int64_t hw = opaque_stride(a.HW);
    int64_t b;
    const int64_t pw = tile_px(tt, a.tpb, Q, NW, wave, &b);
    const bool inb = pw + Q * j < hw;
    // first branch's last layer: acc = W0 t (t read in the accumulator layout)
    v4f acc[C / 16][Q];
    {
      v4f tv[CIN / 16][Q];
      load_acc<CIN, Q>(a.t + b * CIN * hw + pw, hw, inb, yoff, tv);
      if (GIN) {  // t is the Converse2D output before its GELU
#pragma unroll
        for (int rb = 0; rb < CIN / 16; ++rb)
#pragma unroll
          for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int r = 0; r < 4; ++r) tv[rb][q][r] = gelu_f(tv[rb][q][r]);
      }
      zero_acc<C, Q>(acc);
      gemm_f16s<CIN, C, Q>(tv, W0l, lane, acc);
    }
    // y' = x + s1 (acc + b0), channel 16 rb + 4 g + r; x read in the same layout
    const float* xw = a.x + b * C * hw + pw;
#pragma unroll
    for (int rb = 0; rb < C / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 16 * rb + 4 * g + r;
        float rr[Q];
        if (inb) {
          ldq<Q>(at_off(xw + (int64_t)(16 * rb + r) * hw, yoff), rr);
        } else {
#pragma unroll
          for (int q = 0; q < Q; ++q) rr[q] = 0.f;
        }
        const float bo = prm[o], sc = prm[C + o];
#pragma unroll
        for (int q = 0; q < Q; ++q) acc[rb][q][r] = fmaf(sc, acc[rb][q][r] + bo, rr[q]);
      }
    // out = y' + s2 (W2 GELU(W1 LN(y') + b1) + b2)
    v4f acc2[C / 16][Q];
    {
      v4f h[CM / 16][Q];
      {
        v4f xn[C / 16][Q];
        ln_acc<C, Q>(acc, prm + 2 * C, prm + 3 * C, a.eps, g, xn);
        zero_acc<CM, Q>(h);
        gemm_f16s<C, CM, Q>(xn, W1l, lane, h);
      }
#pragma unroll
      for (int rb = 0; rb < CM / 16; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float bo = prm[6 * C + 16 * rb + 4 * g + r];
#pragma unroll
          for (int q = 0; q < Q; ++q) h[rb][q][r] = gelu_f(h[rb][q][r] + bo);
        }
      zero_acc<C, Q>(acc2);
      gemm_f16s<CM, C, Q>(h, W2l, lane, acc2);
    }
#pragma unroll
    for (int rb = 0; rb < C / 16; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 16 * rb + 4 * g + r;
        const float bo = prm[4 * C + o], sc = prm[5 * C + o];
#pragma unroll
        for (int q = 0; q < Q; ++q) acc2[rb][q][r] = fmaf(sc, acc2[rb][q][r] + bo, acc[rb][q][r]);
      }
    if (inb) store_acc<C, Q>(acc2, a.y + b * C * hw + pw, hw, yoff);
    if (HEAD) {
      // next block: th = GELU(Wh LNh(out) + bh)
      v4f hh[CIN / 16][Q];
      {
        v4f xn[C / 16][Q];
        ln_acc<C, Q>(acc2, prm + 6 * C + CM, prm + 7 * C + CM, a.heps, g, xn);
        zero_acc<CIN, Q>(hh);
        gemm_f16s<C, CIN, Q>(xn, Whl, lane, hh);
      }
#pragma unroll
      for (int rb = 0; rb < CIN / 16; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float bo = prm[8 * C + CM + 16 * rb + 4 * g + r];
#pragma unroll
          for (int q = 0; q < Q; ++q) hh[rb][q][r] = gelu_f(hh[rb][q][r] + bo);
        }
      if (inb) store_acc<CIN, Q>(hh, a.th + b * CIN * hw + pw, hw, yoff);
    }
  }
}

// Plain VALU 1x1 conv for channel counts / sizes the MFMA tiles do not cover (e.g. 1 or 3 channels,
// or pixel counts that are not a multiple of 4).  Thread = one pixel and a group of kOutGroup
// output channels (grid z); each input channel value is loaded once and feeds the whole group.
constexpr int kOutGroup = 8;
template <int PX>
__global__ void __launch_bounds__(256) k_conv1x1_any(const float* __restrict__ x, int64_t HW, int Cin,
                                                     const float* __restrict__ W, const float* __restrict__ bias,
                                                     int Cout, int act, const float* residual,
                                                     const float* __restrict__ res_scale, float* y) {
  // PX consecutive pixels per thread (4: one float4 per channel when HW % 4 == 0 and the buffers are
  // 16-byte aligned); the input-channel loop is unrolled so that several loads are in flight at once
  const int64_t p = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * PX;
  if (p >= HW) return;
  const int64_t b = blockIdx.y;
  const int o0 = blockIdx.z * kOutGroup;
  const int no = min(kOutGroup, Cout - o0);
  const float* xb = x + b * Cin * HW + p;
  float acc[kOutGroup][PX];
#pragma unroll
  for (int k = 0; k < kOutGroup; ++k)
#pragma unroll
    for (int j = 0; j < PX; ++j) acc[k][j] = (k < no && bias) ? bias[o0 + k] : 0.f;
#pragma unroll 8
  for (int c = 0; c < Cin; ++c) {
    float xv[PX];
    if constexpr (PX == 4) {
      const float4 v = *(const float4*)(xb + (int64_t)c * HW);
      xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
    } else {
      xv[0] = xb[(int64_t)c * HW];
    }
#pragma unroll
    for (int k = 0; k < kOutGroup; ++k)
      if (k < no) {
        const float wk = W[(o0 + k) * Cin + c];
#pragma unroll
        for (int j = 0; j < PX; ++j) acc[k][j] = fmaf(wk, xv[j], acc[k][j]);
      }
  }
#pragma unroll
  for (int k = 0; k < kOutGroup; ++k) {
    if (k >= no) break;
    const int o = o0 + k;
    const int64_t oi = (b * Cout + o) * HW + p;
    float v[PX];
#pragma unroll
    for (int j = 0; j < PX; ++j) {
      v[j] = acc[k][j];
      if (act == CVN_ACT_GELU) v[j] = gelu_f(v[j]);
    }
    if (residual) {
      const float sc = res_scale ? res_scale[o] : 1.f;
      if constexpr (PX == 4) {
        const float4 r = *(const float4*)(residual + oi);
        v[0] = fmaf(sc, v[0], r.x); v[1] = fmaf(sc, v[1], r.y); v[2] = fmaf(sc, v[2], r.z); v[3] = fmaf(sc, v[3], r.w);
      } else {
        v[0] = fmaf(sc, v[0], residual[oi]);
      }
    }
    if constexpr (PX == 4) *(float4*)(y + oi) = make_float4(v[0], v[1], v[2], v[3]);
    else y[oi] = v[0];
  }
}

}  // namespace cvn

using namespace cvn;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

constexpr int64_t kMaxMfmaHW = (int64_t)1 << 26;

// Tile shape per kernel: Q 16-pixel blocks per wave, NW waves per block.  Large blocks share one
// LDS copy of the weights among many waves (the weights, not the registers, bound the number of
// resident waves); the Q values are the measured best at 4 x 64 x 256 x 256.
// 1024-thread blocks cap a thread at 128 registers: the wider shapes take Q = 1 so that nothing
// spills.
template <int CIN, int COUT, bool LN>
struct ConvTile {
  // split-fp16 products for whole 32-channel input chunks (not at 128 x 128, where they would spill)
  static constexpr bool F16S = CIN % 32 == 0 && CIN + COUT < 256;
  static constexpr int Q = F16S ? (CIN + COUT >= 192 ? 1 : 2) : (CIN + COUT > 192 || (LN && CIN + COUT >= 192)) ? 1 : 2;
  static constexpr int NW = 16;
};
template <int C, int CM>
struct MlpTile {
  static constexpr int Q = 1, NW = 16;
};

// Persistent grid: as many blocks as fit on the device at once (occupancy query, cached per kernel
// and device), at most one per tile.
template <typename K>
unsigned persistent_grid(K kernel, int threads, int64_t ntiles) {
  static std::atomic<int> resident[64];
  const int dev = current_device() & 63;
  int r = resident[dev].load(std::memory_order_relaxed);
  if (r == 0) {
    int cus = 0, per_cu = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, current_device());
    (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)kernel, threads, 0);
    (void)hipGetLastError();
    r = std::max(1, cus) * std::max(1, per_cu);
    resident[dev].store(r, std::memory_order_relaxed);
  }
  return (unsigned)std::min<int64_t>(ntiles, r);
}

template <int CIN, int COUT, bool LN>
int launch_mfma(const float* x, int64_t B, int64_t HW, const float* W, const float* bias, const float* lw,
                const float* lb, float eps, int act, const float* residual, const float* res_scale, float* y,
                hipStream_t st) {
  constexpr int Q = ConvTile<CIN, COUT, LN>::Q, NW = ConvTile<CIN, COUT, LN>::NW;
  const int64_t tpb = (HW + 16 * NW * Q - 1) / (16 * NW * Q), ntiles = B * tpb;
  auto kern = k_conv1x1_mfma<CIN, COUT, LN, Q, NW, ConvTile<CIN, COUT, LN>::F16S>;
  hipLaunchKernelGGL(kern, dim3(persistent_grid(kern, 64 * NW, ntiles)), dim3(64 * NW), 0, st, x, HW, tpb, ntiles,
                     W, bias, lw, lb, eps, act, residual, res_scale, y);
  return check_launch("1x1 conv");
}

template <int C, int CM>
int launch_mlp(const float* x, int64_t B, int64_t HW, const float* ln_w, const float* ln_b, float ln_eps,
               const float* w1, const float* b1, const float* w2, const float* b2, const float* res_scale, float* y,
               hipStream_t st) {
  constexpr int Q = MlpTile<C, CM>::Q, NW = MlpTile<C, CM>::NW;
  const int64_t tpb = (HW + 16 * NW * Q - 1) / (16 * NW * Q), ntiles = B * tpb;
  auto kern = k_ln_mlp_mfma<C, CM, Q, NW>;
  hipLaunchKernelGGL(kern, dim3(persistent_grid(kern, 64 * NW, ntiles)), dim3(64 * NW), 0, st, x, HW, tpb, ntiles,
                     ln_w, ln_b, ln_eps, w1, b1, w2, b2, res_scale, y);
  return check_launch("fused LN-MLP branch");
}

template <int CIN, int C, int CM>
int launch_tail(TailArgs a, int64_t B, hipStream_t st) {
  constexpr int Q = 1, NW = 16;
  a.tpb = (a.HW + 16 * NW * Q - 1) / (16 * NW * Q);
  a.ntiles = B * a.tpb;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(persistent_grid(kern, 64 * NW, a.ntiles)), dim3(64 * NW), 0, st, a);
  };
  if (a.th)
    a.t_act == CVN_ACT_GELU ? go(k_conv_ln_mlp_mfma<CIN, C, CM, Q, NW, true, true>)
                            : go(k_conv_ln_mlp_mfma<CIN, C, CM, Q, NW, true, false>);
  else
    a.t_act == CVN_ACT_GELU ? go(k_conv_ln_mlp_mfma<CIN, C, CM, Q, NW, false, true>)
                            : go(k_conv_ln_mlp_mfma<CIN, C, CM, Q, NW, false, false>);
  return check_launch("fused block tail");
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
  // the MFMA kernels address a lane's pixels with 32-bit byte offsets within 16 channel rows
  const bool vec_ok = (HW % 4 == 0) && HW <= kMaxMfmaHW && aligned16(x) && aligned16(y) &&
                      (!residual || aligned16(residual));
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
  if ((Cout + kOutGroup - 1) / kOutGroup > 65535) return fail(CVN_ERR_UNSUPPORTED, "too many output channels");
  const bool vec = HW % 4 == 0 && aligned16(x) && aligned16(y) && (!residual || aligned16(residual));
  const int px = vec ? 4 : 1;
  dim3 grid((unsigned)((HW / px + 255) / 256), (unsigned)B, (unsigned)((Cout + kOutGroup - 1) / kOutGroup));
  if (vec)
    hipLaunchKernelGGL(k_conv1x1_any<4>, grid, dim3(256), 0, st, x, HW, (int)Cin, weight, bias, (int)Cout, act,
                       residual, res_scale, y);
  else
    hipLaunchKernelGGL(k_conv1x1_any<1>, grid, dim3(256), 0, st, x, HW, (int)Cin, weight, bias, (int)Cout, act,
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
  if (HW % 4 != 0 || HW > kMaxMfmaHW || !aligned16(x) || !aligned16(y))
    return fail(CVN_ERR_UNSUPPORTED,
                "fused branch needs HW %% 4 == 0, HW <= 2^26 and 16-byte aligned buffers");
  hipStream_t st = (hipStream_t)stream;
  if (C == 64 && Cmid == 128)
    return launch_mlp<64, 128>(x, B, HW, ln_w, ln_b, ln_eps, w1, b1, w2, b2, res_scale, y, st);
  if (C == 32 && Cmid == 64)
    return launch_mlp<32, 64>(x, B, HW, ln_w, ln_b, ln_eps, w1, b1, w2, b2, res_scale, y, st);
  return fail(CVN_ERR_UNSUPPORTED, "fused branch supports (C, Cmid) in {(64,128), (32,64)}");
}

static int tail_impl(TailArgs a, int64_t B, int64_t Ct, int64_t C, int64_t Cmid, hipStream_t st) {
  if (!a.t || !a.W0 || !a.b0 || !a.x || !a.lw || !a.lb || !a.W1 || !a.b1 || !a.W2 || !a.b2 || !a.y)
    return fail(CVN_ERR_ARG, "null pointer");
  if (a.th && (!a.hlw || !a.hlb || !a.Wh || !a.bh)) return fail(CVN_ERR_ARG, "null pointer");
  if (a.t_act != CVN_ACT_NONE && a.t_act != CVN_ACT_GELU) return fail(CVN_ERR_ARG, "bad activation %d", a.t_act);
  if (B < 0 || a.HW < 0) return fail(CVN_ERR_ARG, "bad shape");
  if (B > 65535) return fail(CVN_ERR_UNSUPPORTED, "batch exceeds 65535");
  if (a.t == a.y || (a.th && (a.th == a.x || a.th == a.y)))
    return fail(CVN_ERR_ARG, "the output may alias x only; the next block's input must be a separate buffer");
  if (B == 0 || a.HW == 0) return CVN_OK;
  if (a.HW % 4 != 0 || a.HW > kMaxMfmaHW || !aligned16(a.t) || !aligned16(a.x) || !aligned16(a.y) ||
      (a.th && !aligned16(a.th)))
    return fail(CVN_ERR_UNSUPPORTED, "fused tail needs HW %% 4 == 0, HW <= 2^26 and 16-byte aligned buffers");
  if (Ct == 128 && C == 64 && Cmid == 128) return launch_tail<128, 64, 128>(a, B, st);
  return fail(CVN_ERR_UNSUPPORTED, "fused tail supports (Ct, C, Cmid) = (128, 64, 128)");
}

extern "C" int cvn_conv_ln_mlp_residual_f32(const float* t, int t_act, int64_t B, int64_t Ct, int64_t HW,
                                            const float* w0, const float* b0, const float* res_scale1,
                                            const float* x, int64_t C, const float* ln_w, const float* ln_b,
                                            float ln_eps, const float* w1, const float* b1, int64_t Cmid,
                                            const float* w2, const float* b2, const float* res_scale2, float* y,
                                            cvn_stream_t stream) {
  TailArgs a{t, x, HW, 0, 0, w0, b0, res_scale1, ln_w, ln_b, w1, b1, w2, b2, res_scale2, ln_eps, y,
             nullptr, nullptr, nullptr, nullptr, 0.f, nullptr, t_act};
  return tail_impl(a, B, Ct, C, Cmid, (hipStream_t)stream);
}

extern "C" int cvn_conv_ln_mlp_head_f32(const float* t, int t_act, int64_t B, int64_t Ct, int64_t HW,
                                        const float* w0, const float* b0, const float* res_scale1, const float* x,
                                        int64_t C, const float* ln_w, const float* ln_b, float ln_eps,
                                        const float* w1, const float* b1, int64_t Cmid, const float* w2,
                                        const float* b2, const float* res_scale2, float* y, const float* head_ln_w,
                                        const float* head_ln_b, float head_ln_eps, const float* head_w,
                                        const float* head_b, float* t_next, cvn_stream_t stream) {
  TailArgs a{t, x, HW, 0, 0, w0, b0, res_scale1, ln_w, ln_b, w1, b1, w2, b2, res_scale2, ln_eps, y,
             head_ln_w, head_ln_b, head_w, head_b, head_ln_eps, t_next, t_act};
  if (!t_next) return fail(CVN_ERR_ARG, "null pointer");
  return tail_impl(a, B, Ct, C, Cmid, (hipStream_t)stream);
}
