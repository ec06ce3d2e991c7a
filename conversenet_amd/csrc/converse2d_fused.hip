// Converse2D forward, fused single-kernel path for scale 1: one 1024-thread workgroup per (b, c)
// plane, one HBM read of the input plane and one HBM write of the cropped output.
//
// The padded plane y (N x M) is split into two row groups, G0 = even rows and G1 = odd rows.  Per
// group (N/2 rows, processed in LDS):
//   1. load the rows with the padding index map applied on the global read, two real rows per
//      complex row ("row pair": row a in .x, row b in .y), LDS row-pair stride RS = M + 2;
//   2. forward row FFT of length M = R1 R2 R3 (pairwise coprime) in place by the prime-factor
//      algorithm.  Inside a row, sample n lives at the "3-D natural" position
//      n1 R2 R3 + n2 R3 + n3 (n_i = the Ruritanian coordinates of n), so every radix pass walks a
//      compile-time stride and needs no twiddles; frequency v ends up at position fpos(v) =
//      (v mod R1) R2 R3 + (v mod R2) R3 + (v mod R3);
//   3. Hermitian unpack of each row pair into the two half spectra: bin v in [1, M/2) of row a at
//      fpos(v), of row b at fpos(M - v); the real DC / Nyquist bins of rows a / b at slots 0 and
//      fpos(M/2) (a) and M, M + 1 (b);
//   4. forward column FFT of length N/2 = Q1 Q2 2 over the group's rows, in place, with the group
//      rows stored in the same 3-D natural order (the radix-2 axis is the row-pair axis).
// G0's spectrum is then parked in registers while G1 runs in LDS.  The radix-2 step across the
// groups (length-N column transform), the transfer function Phi and the inverse radix-2 step fold
// into one 2x2 complex map per slot, precomputed in fp64 in this kernel's slot order:
//   E' = a E + bW O,   O' = bWi E + a O,   a = Phi(k) + Phi(k + N/2), b = Phi(k) - Phi(k + N/2),
//   bW = b W^k, bWi = b W^-k, W = exp(-2 pi i / N), normalisation 1 / (N M) folded into Phi.
// Each group then runs the inverse column FFT, repacks the row pairs, runs the inverse row FFT
// (real parts = row a, imaginary parts = row b) and stores the cropped rows.
#include <math.h>

#include "cvn_common.h"

namespace cvn {

constexpr int kFT = 1024;  // threads per fused workgroup

constexpr int mod_inv(int a, int m) {
  if (m <= 1) return 0;
  for (int x = 1; x < m; ++x)
    if ((a * x) % m == 1) return x;
  return 0;
}

template <int M_, int R1_, int R2_, int R3_, int Q1_, int Q2_>
struct FusedPlan {
  static constexpr int M = M_, R1 = R1_, R2 = R2_, R3 = R3_;
  static constexpr int Q1 = Q1_, Q2 = Q2_, NH = 2 * Q1_ * Q2_, N = 2 * NH;
  static constexpr int RS = M + 2;        // row-pair stride (M/2 + 1 bins per row, two rows)
  static constexpr int NP = NH / 2;       // row pairs per group
  static constexpr int SLOTS = NP * RS;   // complex slots per group
  static constexpr int NQ = M / 2 + 1;    // half-spectrum columns
  static constexpr int ST1 = R2 * R3, ST2 = R3;  // row-axis strides (positions)
  static constexpr int CS1 = 2 * Q2, CS2 = 2;    // column-axis strides (row positions)
  static constexpr int PARK = (SLOTS + kFT - 1) / kFT;
  static_assert(R1 * R2 * R3 == M && M % 2 == 0 && NP % 2 == 1, "plan");
  // LDS: slots + int tables pa, pb (NQ each), pos (M), colsrc (M), rowsrc (2 NH)
  static constexpr size_t LDS_BYTES = (size_t)SLOTS * 8 + (size_t)(2 * NQ + 2 * M + 2 * NH) * 4;

  // position of natural sample n inside a row (Ruritanian coordinates, 3-D natural order)
  static __host__ __device__ constexpr int pos_in(int n) {
    return ((n * mod_inv((M / R1) % R1, R1)) % R1) * ST1 + ((n * mod_inv((M / R2) % R2, R2)) % R2) * ST2 +
           (R3 > 1 ? (n * mod_inv((M / R3) % R3, R3)) % R3 : 0);
  }
  // position of frequency v after the forward row transform
  static __host__ __device__ constexpr int fpos(int v) {
    return (v % R1) * ST1 + (v % R2) * ST2 + (R3 > 1 ? v % R3 : 0);
  }
  static __host__ __device__ constexpr int pa(int q) { return fpos(q); }
  static __host__ __device__ constexpr int pb(int q) { return q == 0 ? M : (q == M / 2 ? M + 1 : fpos(M - q)); }
  // row position of group row g (column transform input order) and of column frequency k (output)
  static __host__ __device__ constexpr int rpos_in(int g) {
    return ((g * mod_inv((NH / Q1) % Q1, Q1)) % Q1) * CS1 + ((g * mod_inv((NH / Q2) % Q2, Q2)) % Q2) * CS2 +
           ((g * mod_inv((NH / 2) % 2, 2)) % 2);
  }
  static __host__ __device__ constexpr int rfpos(int k) { return (k % Q1) * CS1 + (k % Q2) * CS2 + (k % 2); }
};

// Row pass A: radix R3 along the contiguous axis (positions base + m, m < R3).
template <class P, bool INV>
__device__ __forceinline__ void row_pass_a(float2* buf, int tid) {
  constexpr int R = P::R3, PER = P::M / R;
#pragma unroll 1
  for (int w = tid; w < P::NP * PER; w += kFT) {
    const int t = w / PER, i = w - t * PER;
    dft_odd_mem<R, 1, INV>(buf + t * P::RS + i * R);
  }
}

// Row pass B: the R1 x R2 prime-factor sub-grid (strides ST1, ST2) in registers, base = n3.
template <class P, bool INV>
__device__ __forceinline__ void row_pass_b(float2* buf, int tid) {
  constexpr int R1 = P::R1, R2 = P::R2, PER = P::R3;
#pragma unroll 1
  for (int w = tid; w < P::NP * PER; w += kFT) {
    const int t = w / PER, n3 = w - t * PER;
    float2* b = buf + t * P::RS + n3;
    float2 u[R1][R2];
#pragma unroll
    for (int m1 = 0; m1 < R1; ++m1)
#pragma unroll
      for (int m2 = 0; m2 < R2; ++m2) u[m1][m2] = b[m1 * P::ST1 + m2 * P::ST2];
#pragma unroll
    for (int m1 = 0; m1 < R1; ++m1) Dft<R2, INV>::run(u[m1]);
#pragma unroll
    for (int m2 = 0; m2 < R2; ++m2) {
      float2 v[R1];
#pragma unroll
      for (int m1 = 0; m1 < R1; ++m1) v[m1] = u[m1][m2];
      Dft<R1, INV>::run(v);
#pragma unroll
      for (int m1 = 0; m1 < R1; ++m1) b[m1 * P::ST1 + m2 * P::ST2] = v[m1];
    }
  }
}

// Column pass A (forward): Hermitian unpack of the row pairs, the radix-2 pair axis and the
// radix-Q1 axis (row-pair stride Q2) in registers.  Work item (q, g2); q = 0 also carries the
// Nyquist column M/2.
template <class P>
__device__ __forceinline__ void col_pass_a_fwd(float2* buf, const int* pa, const int* pb, int tid) {
  constexpr int Q1 = P::Q1, HQ = P::M / 2;
#pragma unroll 1
  for (int w = tid; w < HQ * P::Q2; w += kFT) {
    const int g2 = w / HQ, q = w - g2 * HQ;
    float2* b = buf + g2 * P::RS;
    if (q != 0) {
      const int sa = pa[q], sb = pb[q];
      float2 u0[Q1], u1[Q1];
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        const float2 zl = b[m * P::Q2 * P::RS + sa], zh = b[m * P::Q2 * P::RS + sb];
        const float2 A = make_float2(0.5f * (zl.x + zh.x), 0.5f * (zl.y - zh.y));
        const float2 B = make_float2(0.5f * (zl.y + zh.y), 0.5f * (zh.x - zl.x));
        u0[m] = cadd(A, B);
        u1[m] = csub(A, B);
      }
      Dft<Q1, false>::run(u0);
      Dft<Q1, false>::run(u1);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        b[m * P::Q2 * P::RS + sa] = u0[m];
        b[m * P::Q2 * P::RS + sb] = u1[m];
      }
    } else {
      const int sn = pa[HQ];
      float2 d0[Q1], d1[Q1], n0[Q1], n1[Q1];
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        const float2 z0 = b[m * P::Q2 * P::RS], zn = b[m * P::Q2 * P::RS + sn];
        d0[m] = make_float2(z0.x + z0.y, 0.f);
        d1[m] = make_float2(z0.x - z0.y, 0.f);
        n0[m] = make_float2(zn.x + zn.y, 0.f);
        n1[m] = make_float2(zn.x - zn.y, 0.f);
      }
      Dft<Q1, false>::run(d0);
      Dft<Q1, false>::run(d1);
      Dft<Q1, false>::run(n0);
      Dft<Q1, false>::run(n1);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        float2* r = b + m * P::Q2 * P::RS;
        r[0] = d0[m];
        r[P::M] = d1[m];
        r[sn] = n0[m];
        r[P::M + 1] = n1[m];
      }
    }
  }
}

// Column pass A (inverse): radix-Q1, inverse radix-2 pair axis, repack into complex row pairs.
template <class P>
__device__ __forceinline__ void col_pass_a_inv(float2* buf, const int* pa, const int* pb, int tid) {
  constexpr int Q1 = P::Q1, HQ = P::M / 2;
#pragma unroll 1
  for (int w = tid; w < HQ * P::Q2; w += kFT) {
    const int g2 = w / HQ, q = w - g2 * HQ;
    float2* b = buf + g2 * P::RS;
    if (q != 0) {
      const int sa = pa[q], sb = pb[q];
      float2 u0[Q1], u1[Q1];
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        u0[m] = b[m * P::Q2 * P::RS + sa];
        u1[m] = b[m * P::Q2 * P::RS + sb];
      }
      Dft<Q1, true>::run(u0);
      Dft<Q1, true>::run(u1);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        const float2 A = cadd(u0[m], u1[m]), B = csub(u0[m], u1[m]);
        b[m * P::Q2 * P::RS + sa] = make_float2(A.x - B.y, A.y + B.x);  // A + iB
        b[m * P::Q2 * P::RS + sb] = make_float2(A.x + B.y, B.x - A.y);  // conj(A) + i conj(B)
      }
    } else {
      const int sn = pa[HQ];
      float2 d0[Q1], d1[Q1], n0[Q1], n1[Q1];
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        const float2* r = b + m * P::Q2 * P::RS;
        d0[m] = r[0];
        d1[m] = r[P::M];
        n0[m] = r[sn];
        n1[m] = r[P::M + 1];
      }
      Dft<Q1, true>::run(d0);
      Dft<Q1, true>::run(d1);
      Dft<Q1, true>::run(n0);
      Dft<Q1, true>::run(n1);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        float2* r = b + m * P::Q2 * P::RS;
        r[0] = make_float2(d0[m].x + d1[m].x, d0[m].x - d1[m].x);
        r[sn] = make_float2(n0[m].x + n1[m].x, n0[m].x - n1[m].x);
      }
    }
  }
}

// Column pass B: radix Q2 along row pairs (stride 1 row pair); work item (q, g1, g3), q fastest.
template <class P, bool INV>
__device__ __forceinline__ void col_pass_b(float2* buf, const int* pa, const int* pb, int tid) {
  constexpr int Q = P::Q2;
#pragma unroll 1
  for (int w = tid; w < P::NQ * P::Q1 * 2; w += kFT) {
    const int i = w / P::NQ, q = w - i * P::NQ;
    const int g1 = i >> 1, g3 = i & 1;
    dft_odd_mem<Q, P::RS, INV>(buf + g1 * P::Q2 * P::RS + (g3 ? pb[q] : pa[q]));
  }
}

struct FusedArgs {
  const float* x;        // (P, H, W)
  const float4* tab4;    // (Cp, SLOTS): (a, bW)
  const float2* tab2;    // (Cp, SLOTS): bWi
  float* out;            // (P, H, W)
  int64_t C, psf_batch;
  int H, W, pad, mode, act;
};

__device__ __forceinline__ int fpad_src(int i, int n, int p, int mode) {
  int j = i - p;
  if (j >= 0 && j < n) return j;
  switch (mode) {
    case CVN_PAD_CIRCULAR: j %= n; return j < 0 ? j + n : j;
    case CVN_PAD_REPLICATE: return j < 0 ? 0 : n - 1;
    case CVN_PAD_REFLECT: return j < 0 ? -j : 2 * (n - 1) - j;
    default: return -1;
  }
}

__device__ __forceinline__ float fgelu(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)); }

// Rows of one group as float4 loads: wave w takes row positions w, w + 16, ...; lane l the source
// columns 4 l .. 4 l + 3.  RPW = rows per wave (rounded up).
template <class P>
struct RowIO {
  static constexpr int NW = kFT / 64;
  static constexpr int RPW = (P::NH + NW - 1) / NW;
};

template <class P>
__device__ __forceinline__ void group_prefetch(float4 (&v)[RowIO<P>::RPW], const int* srow, const float* xp,
                                               int W, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < RowIO<P>::RPW; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (rp < P::NH && 4 * lane < W) {
      const int sr = srow[rp];
      if (sr >= 0) v[i] = *(const float4*)(xp + sr * W + 4 * lane);
    }
  }
}

template <class P>
__device__ __forceinline__ void group_deposit(float2* buf, const float4 (&v)[RowIO<P>::RPW], const int (&lp)[4],
                                              int W, int wave, int lane) {
  float* fb = (float*)buf;
#pragma unroll
  for (int i = 0; i < RowIO<P>::RPW; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    if (rp < P::NH && 4 * lane < W) {
      float* r = fb + 2 * ((rp >> 1) * P::RS) + (rp & 1);
      r[2 * lp[0]] = v[i].x;
      r[2 * lp[1]] = v[i].y;
      r[2 * lp[2]] = v[i].z;
      r[2 * lp[3]] = v[i].w;
    }
  }
}

// Padding columns copied inside LDS from the interior column they replicate (or zeroed).
template <class P>
__device__ __forceinline__ void group_pad_cols(float2* buf, const int* pos, const int* colsrc, int pad, int tid) {
  if (pad == 0) return;
  const int npc = 2 * pad;
#pragma unroll 1
  for (int w = tid; w < P::NP * npc; w += kFT) {
    const int t = w / npc, c = w - t * npc;
    const int j = c < pad ? c : P::M - npc + c;
    const int sc = colsrc[j];
    float2* r = buf + t * P::RS;
    r[pos[j]] = sc >= 0 ? r[pos[pad + sc]] : make_float2(0.f, 0.f);
  }
}

// forward passes up to (not including) the last column pass
template <class P>
__device__ __forceinline__ void group_forward_passes(float2* buf, const int* pa, const int* pb, int tid) {
  row_pass_a<P, false>(buf, tid);
  __syncthreads();
  row_pass_b<P, false>(buf, tid);
  __syncthreads();
  col_pass_a_fwd<P>(buf, pa, pb, tid);
  __syncthreads();
}

template <class P>
__device__ __forceinline__ void group_inverse_store(float2* buf, const int* pa, const int* pb, const int (&lp)[4],
                                                    const int* orow, float* op, const FusedArgs& a, int wave,
                                                    int lane, int tid) {
  col_pass_b<P, true>(buf, pa, pb, tid);
  __syncthreads();
  col_pass_a_inv<P>(buf, pa, pb, tid);
  __syncthreads();
  row_pass_b<P, true>(buf, tid);
  __syncthreads();
  row_pass_a<P, true>(buf, tid);
  __syncthreads();
  const float* fb = (const float*)buf;
#pragma unroll
  for (int i = 0; i < RowIO<P>::RPW; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    if (rp < P::NH && 4 * lane < a.W) {
      const int orr = orow[rp];
      if (orr >= 0 && orr < a.H) {
        const float* r = fb + 2 * ((rp >> 1) * P::RS) + (rp & 1);
        float4 v = make_float4(r[2 * lp[0]], r[2 * lp[1]], r[2 * lp[2]], r[2 * lp[3]]);
        if (a.act == CVN_ACT_GELU) {
          v.x = fgelu(v.x); v.y = fgelu(v.y); v.z = fgelu(v.z); v.w = fgelu(v.w);
        }
        *(float4*)(op + orr * a.W + 4 * lane) = v;
      }
    }
  }
}

// Table entries of one slot, loaded DEPTH slots ahead of their use in the combine step.
constexpr int kTabDepth = 4;

template <class P>
__global__ void __launch_bounds__(kFT) k_converse2d_fused(FusedArgs a) {
  extern __shared__ float2 smem[];
  float2* buf = smem;
  int* pa = (int*)(smem + P::SLOTS);
  int* pb = pa + P::NQ;
  int* pos = pb + P::NQ;
  int* colsrc = pos + P::M;
  int* rtab = colsrc + P::M;  // 2 NH: source rows by row position (G0, G1), later output rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t plane = blockIdx.x;
  const int64_t cp = (a.psf_batch == 1) ? (plane % a.C) : plane;
  const float* xp = a.x + plane * (int64_t)a.H * a.W;
  float* op = a.out + plane * (int64_t)a.H * a.W;
  for (int q = tid; q < P::NQ; q += kFT) {
    pa[q] = P::pa(q);
    pb[q] = P::pb(q);
  }
  for (int j = tid; j < P::M; j += kFT) {
    pos[j] = P::pos_in(j);
    colsrc[j] = fpad_src(j, a.W, a.pad, a.mode);
  }
  for (int g = tid; g < P::NH; g += kFT) {
    const int rp = P::rpos_in(g);
    rtab[rp] = fpad_src(2 * g, a.H, a.pad, a.mode);
    rtab[P::NH + rp] = fpad_src(2 * g + 1, a.H, a.pad, a.mode);
  }
  int lp[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) lp[c] = P::pos_in(min(a.pad + 4 * lane + c, P::M - 1));
  __syncthreads();
  float4 pre[RowIO<P>::RPW];
  group_prefetch<P>(pre, rtab, xp, a.W, wave, lane);
  group_deposit<P>(buf, pre, lp, a.W, wave, lane);
  __syncthreads();
  group_pad_cols<P>(buf, pos, colsrc, a.pad, tid);
  __syncthreads();
  group_forward_passes<P>(buf, pa, pb, tid);
  group_prefetch<P>(pre, rtab + P::NH, xp, a.W, wave, lane);  // G1 rows arrive during G0's last pass
  col_pass_b<P, false>(buf, pa, pb, tid);
  __syncthreads();
  float2 park[P::PARK];
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) {
    const int s = tid + i * kFT;
    park[i] = (s < P::SLOTS) ? buf[s] : make_float2(0.f, 0.f);
  }
  __syncthreads();
  group_deposit<P>(buf, pre, lp, a.W, wave, lane);
  __syncthreads();
  group_pad_cols<P>(buf, pos, colsrc, a.pad, tid);
  __syncthreads();
  group_forward_passes<P>(buf, pa, pb, tid);
  col_pass_b<P, false>(buf, pa, pb, tid);
  __syncthreads();
  // radix-2 across the groups, transfer function, inverse radix-2 (table loads run kTabDepth ahead)
  const float4* t4 = a.tab4 + cp * P::SLOTS;
  const float2* t2 = a.tab2 + cp * P::SLOTS;
  float4 f4[kTabDepth];
  float2 f2[kTabDepth];
#pragma unroll
  for (int i = 0; i < kTabDepth; ++i) {
    const int s = min(tid + i * kFT, P::SLOTS - 1);
    f4[i] = t4[s];
    f2[i] = t2[s];
  }
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) {
    const int s = tid + i * kFT;
    const float4 ab = f4[i % kTabDepth];
    const float2 bi = f2[i % kTabDepth];
    if (i + kTabDepth < P::PARK) {
      const int sn = min(tid + (i + kTabDepth) * kFT, P::SLOTS - 1);
      f4[i % kTabDepth] = t4[sn];
      f2[i % kTabDepth] = t2[sn];
    }
    if (s < P::SLOTS) {
      const float2 e = park[i], o = buf[s];
      const float2 av = make_float2(ab.x, ab.y), bw = make_float2(ab.z, ab.w);
      park[i] = cadd(cmul(av, e), cmul(bw, o));
      buf[s] = cadd(cmul(bi, e), cmul(av, o));
    }
  }
  __syncthreads();
  for (int g = tid; g < P::NH; g += kFT) {  // output rows (plane row - pad) by row position
    const int rp = P::rpos_in(g);
    rtab[rp] = 2 * g - a.pad;
    rtab[P::NH + rp] = 2 * g + 1 - a.pad;
  }
  __syncthreads();
  group_inverse_store<P>(buf, pa, pb, lp, rtab + P::NH, op, a, wave, lane, tid);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) {
    const int s = tid + i * kFT;
    if (s < P::SLOTS) buf[s] = park[i];
  }
  __syncthreads();
  group_inverse_store<P>(buf, pa, pb, lp, rtab, op, a, wave, lane, tid);
}

// ----------------------------------------------------------------------------------------------
// Transfer table in the fused kernel's slot order (fp64).  One block per (psf plane, column q);
// threads over the column sub-frequency k in [0, N/2).
//   Phi(u, q) = (conj K + lambda) / (|K|^2 + lambda) / (N M),
//   K(u, q) = sum_{i,j} psf[i][j] exp(-2 pi i (u (i - kh/2) / N + q (j - kw/2) / M)).
// ----------------------------------------------------------------------------------------------
struct PhiFusedArgs {
  const float* psf;
  const float* bias;
  int64_t C;
  int kh, kw;
  double eps;
  float4* tab4;
  float2* tab2;
};

__device__ __forceinline__ double2 d_cmul(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ double2 d_root(int64_t m, int L) {  // exp(-2 pi i m / L)
  double sn, cs;
  int64_t r = m % L;
  if (r < 0) r += L;
  sincospi(-2.0 * (double)r / (double)L, &sn, &cs);
  return make_double2(cs, sn);
}

template <class P>
__global__ void __launch_bounds__(256) k_phi_fused(PhiFusedArgs a) {
  __shared__ double2 Pq[64];
  const int64_t cp = blockIdx.x / P::NQ;
  const int q = (int)(blockIdx.x - cp * P::NQ);
  const int c = (int)(cp % a.C);
  const float* psf = a.psf + cp * a.kh * a.kw;
  for (int i = threadIdx.x; i < a.kh; i += blockDim.x) {
    const double2 r = d_root(q, P::M);
    double2 e = d_root(-(int64_t)q * (a.kw / 2), P::M);
    double2 acc = make_double2(0.0, 0.0);
    for (int j = 0; j < a.kw; ++j) {
      const double t = (double)psf[i * a.kw + j];
      acc.x += t * e.x;
      acc.y += t * e.y;
      e = d_cmul(e, r);
    }
    Pq[i] = acc;
  }
  __syncthreads();
  const double lmb = 1.0 / (1.0 + exp(-((double)a.bias[c] - 9.0))) + a.eps;
  const double norm = 1.0 / ((double)P::N * (double)P::M);
  for (int k = threadIdx.x; k < P::NH; k += blockDim.x) {
    double2 ph[2];
    double2 wk = make_double2(1.0, 0.0);
    for (int h = 0; h < 2; ++h) {
      const int u = k + h * P::NH;
      const double2 r = d_root(u, P::N);
      if (h == 0) wk = r;
      double2 e = d_root(-(int64_t)u * (a.kh / 2), P::N);
      double2 K = make_double2(0.0, 0.0);
      for (int i = 0; i < a.kh; ++i) {
        const double2 t = d_cmul(e, Pq[i]);
        K.x += t.x;
        K.y += t.y;
        e = d_cmul(e, r);
      }
      const double den = (K.x * K.x + K.y * K.y + lmb) / norm;
      ph[h] = make_double2((K.x + lmb) / den, -K.y / den);
    }
    const double2 av = make_double2(ph[0].x + ph[1].x, ph[0].y + ph[1].y);
    const double2 bv = make_double2(ph[0].x - ph[1].x, ph[0].y - ph[1].y);
    const double2 bw = d_cmul(bv, wk);
    const double2 bwi = d_cmul(bv, make_double2(wk.x, -wk.y));
    const int rp = P::rfpos(k);
    const int slot = (rp >> 1) * P::RS + ((rp & 1) ? P::pb(q) : P::pa(q));
    a.tab4[cp * P::SLOTS + slot] = make_float4((float)av.x, (float)av.y, (float)bw.x, (float)bw.y);
    a.tab2[cp * P::SLOTS + slot] = make_float2((float)bwi.x, (float)bwi.y);
  }
}

// ----------------------------------------------------------------------------------------------
// host dispatch
// ----------------------------------------------------------------------------------------------
using Plan260 = FusedPlan<260, 4, 5, 13, 5, 13>;   // rows 260 = 4 5 13, columns 130 = 5 13 2
using Plan132 = FusedPlan<132, 4, 3, 11, 3, 11>;   // rows 132 = 4 3 11, columns 66 = 3 11 2

template <class P>
size_t fused_ws(int64_t Cp) {
  return align_up((size_t)Cp * P::SLOTS * sizeof(float4)) + align_up((size_t)Cp * P::SLOTS * sizeof(float2));
}

template <class P>
int fused_table_run(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                    void* table, hipStream_t st) {
  const int64_t Cp = psf_batch * C;
  float4* t4 = (float4*)table;
  float2* t2 = (float2*)((char*)table + align_up((size_t)Cp * P::SLOTS * sizeof(float4)));
  PhiFusedArgs pa{psf, bias, C, kh, kw, (double)eps, t4, t2};
  hipLaunchKernelGGL(k_phi_fused<P>, dim3((unsigned)(Cp * P::NQ)), dim3(256), 0, st, pa);
  return check_launch("fused transfer table");
}

template <class P>
int fused_apply_run(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode,
                    int act, const void* table, float* out, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute((const void*)k_converse2d_fused<P>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)P::LDS_BYTES);
    attr = true;
  }
  const int64_t Cp = psf_batch * C;
  const float4* t4 = (const float4*)table;
  const float2* t2 = (const float2*)((const char*)table + align_up((size_t)Cp * P::SLOTS * sizeof(float4)));
  FusedArgs fa{x, t4, t2, out, C, psf_batch, H, W, pad, mode, act};
  hipLaunchKernelGGL(k_converse2d_fused<P>, dim3((unsigned)(B * C)), dim3(kFT), P::LDS_BYTES, st, fa);
  return check_launch("fused converse2d");
}

// The fused kernel loads rows as float4 per lane: W must be a multiple of 4 and at most 256.
int fused_query(int H, int W, int pad, int scale, int64_t Cp, size_t* ws_bytes) {
  if (scale != 1 || W % 4 != 0 || W > 256) return 0;
  const int h = H + 2 * pad, w = W + 2 * pad;
  if (h == 260 && w == 260) { *ws_bytes = fused_ws<Plan260>(Cp); return 1; }
  if (h == 132 && w == 132) { *ws_bytes = fused_ws<Plan132>(Cp); return 1; }
  return 0;
}

int fused_table(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                int H, int W, int pad, void* table, hipStream_t st) {
  const int h = H + 2 * pad;
  if (h == 260) return fused_table_run<Plan260>(psf, bias, eps, C, psf_batch, kh, kw, table, st);
  return fused_table_run<Plan132>(psf, bias, eps, C, psf_batch, kh, kw, table, st);
}

int fused_apply(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode, int act,
                const void* table, float* out, hipStream_t st) {
  const int h = H + 2 * pad;
  if (h == 260) return fused_apply_run<Plan260>(x, B, C, H, W, psf_batch, pad, mode, act, table, out, st);
  return fused_apply_run<Plan132>(x, B, C, H, W, psf_batch, pad, mode, act, table, out, st);
}

}  // namespace cvn
