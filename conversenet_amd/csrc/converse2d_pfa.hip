// Converse2D forward for 268 x 268 padded planes (Converse-DnCNN: 256 x 256, padding 6), scale 1.
//
// Same three-pass data flow as the generic path (row transform -> column transform x Phi x inverse
// -> inverse row transform, half spectra column-major in between), but every transform is the
// in-place prime-factor FFT 268 = 4 * 67 (no twiddles): a row or column of 268 complex values sits
// in LDS at "3-D natural" positions pos_in(n) = ((3 n) mod 4) * 67 + ((17 n) mod 67), pass A runs a
// 67-point DFT along each contiguous segment of 67, pass B a 4-point DFT along stride 67, and
// frequency v ends at fpos(v) = (v mod 4) * 67 + (v mod 67).  The inverse runs the same passes with
// inverse DFTs in the opposite order, from fpos back to pos_in.
//
// The 67-point DFT is one thread's work, entirely in registers, by Rader's algorithm (primitive
// root 2): a_q = u[2^q mod 67], X_0 = u_0 + sum a, X[2^-q mod 67] = u_0 + (a (*) b)_q with the cyclic
// convolution of length 66 done as an in-register prime-factor FFT 66 = 2 * 3 * 11, a product with
// FFT(b)/66 (the generic path's Rader table for 67, built once per geometry) and the inverse FFT.
// Slot s of the 66-register array holds the convolution input a[s]; after the forward 3-axis DFT it
// holds the transform at k = kappa(s) (k = s mod 6, k = 2 s mod 11), and after the inverse 3-axis DFT
// it holds the convolution output at s again.  (C. M. Rader, Proc. IEEE 56(6), 1968; I. J. Good,
// J. R. Stat. Soc. B 20, 1958.)
#include <math.h>

#include <algorithm>

#include "cvn_common.h"

namespace cvn {
namespace pfa268 {

constexpr int L = 268, P = 67, RM = 66, NC = L / 2 + 1;  // NC: half-spectrum bins

__host__ __device__ constexpr int pos_in(int n) { return ((3 * n) % 4) * P + ((17 * n) % P); }
__host__ __device__ constexpr int fpos(int v) { return (v % 4) * P + (v % P); }
// Index tables, evaluated at compile time: gp[q] = 2^q mod 67, gq[q] = 2^-q mod 67 (34 = 2^-1), and
// kap[s] = the k with k = s (mod 6), k = 2 s (mod 11).
struct Tabs {
  int gp[RM], gq[RM], kap[RM];
  constexpr Tabs() : gp(), gq(), kap() {
    int r = 1, ri = 1;
    for (int q = 0; q < RM; ++q) {
      gp[q] = r;
      gq[q] = ri;
      r = (2 * r) % P;
      ri = (34 * ri) % P;
    }
    for (int s = 0; s < RM; ++s) {
      int k = 0;
      while (!(k % 6 == s % 6 && k % 11 == (2 * s) % 11)) ++k;
      kap[s] = k;
    }
  }
};
constexpr Tabs kT{};

// In-register 3-axis DFT of the 66 slots (axes of length 2, 3, 11; slot s has coordinates
// (s mod 2, s mod 3, 2 s mod 11), i.e. s = 33 n1 + 22 n2 + 6 n3 mod 66).
template <bool INV>
__device__ __forceinline__ void dft66_axes(float2 (&a)[RM]) {
#pragma unroll
  for (int n2 = 0; n2 < 3; ++n2)
#pragma unroll
    for (int n3 = 0; n3 < 11; ++n3) {
      float2 t[2];
#pragma unroll
      for (int n1 = 0; n1 < 2; ++n1) t[n1] = a[(33 * n1 + 22 * n2 + 6 * n3) % RM];
      Dft<2, INV>::run(t);
#pragma unroll
      for (int n1 = 0; n1 < 2; ++n1) a[(33 * n1 + 22 * n2 + 6 * n3) % RM] = t[n1];
    }
#pragma unroll
  for (int n1 = 0; n1 < 2; ++n1)
#pragma unroll
    for (int n3 = 0; n3 < 11; ++n3) {
      float2 t[3];
#pragma unroll
      for (int n2 = 0; n2 < 3; ++n2) t[n2] = a[(33 * n1 + 22 * n2 + 6 * n3) % RM];
      Dft<3, INV>::run(t);
#pragma unroll
      for (int n2 = 0; n2 < 3; ++n2) a[(33 * n1 + 22 * n2 + 6 * n3) % RM] = t[n2];
    }
#pragma unroll
  for (int n1 = 0; n1 < 2; ++n1)
#pragma unroll
    for (int n2 = 0; n2 < 3; ++n2) {
      float2 t[11];
#pragma unroll
      for (int n3 = 0; n3 < 11; ++n3) t[n3] = a[(33 * n1 + 22 * n2 + 6 * n3) % RM];
      Dft<11, INV>::run(t);
#pragma unroll
      for (int n3 = 0; n3 < 11; ++n3) a[(33 * n1 + 22 * n2 + 6 * n3) % RM] = t[n3];
    }
}

// 67-point DFT (direction given by the table: bh = FFT(b)/66 forward or its inverse-direction
// counterpart) of p[0], p[S], ..., p[66 S] in place.
template <int S>
__device__ __forceinline__ void dft67(float2* p, const float2* __restrict__ bh) {
  float2 a[RM];
  const float2 u0 = p[0];
#pragma unroll
  for (int q = 0; q < RM; ++q) a[q] = p[kT.gp[q] * S];
  dft66_axes<false>(a);
  const float2 x0 = cadd(u0, a[0]);  // slot 0 holds bin 0: sum of the a's
#pragma unroll
  for (int s = 0; s < RM; ++s) a[s] = cmul(a[s], bh[kT.kap[s]]);
  a[0] = cadd(a[0], u0);  // adds u_0 to every convolution output
  dft66_axes<true>(a);
  p[0] = x0;
#pragma unroll
  for (int q = 0; q < RM; ++q) p[kT.gq[q] * S] = a[q];
}

// pass A / pass B over `n` rows of 268 slots (row stride LD) held in LDS
template <bool INV>
__device__ __forceinline__ void pass_a(float2* buf, int n, int ld, const float2* bh, int tid, int nth) {
  for (int w = tid; w < 4 * n; w += nth) {
    const int m1 = w / n, t = w - m1 * n;  // row fastest across lanes
    dft67<1>(buf + t * ld + m1 * P, bh);
  }
}
template <bool INV>
__device__ __forceinline__ void pass_b(float2* buf, int n, int ld, int tid, int nth) {
  for (int w = tid; w < P * n; w += nth) {
    const int t = w / P, m3 = w - t * P;
    float2* b = buf + t * ld + m3;
    float2 u[4] = {b[0], b[P], b[2 * P], b[3 * P]};
    Dft<4, INV>::run(u);
    b[0] = u[0];
    b[P] = u[1];
    b[2 * P] = u[2];
    b[3 * P] = u[3];
  }
}

__device__ __forceinline__ int pad_map(int i, int n, int p, int mode) {
  int j = i - p;
  if (j >= 0 && j < n) return j;
  switch (mode) {
    case CVN_PAD_CIRCULAR: j %= n; return j < 0 ? j + n : j;
    case CVN_PAD_REPLICATE: return j < 0 ? 0 : n - 1;
    case CVN_PAD_REFLECT: return j < 0 ? -j : 2 * (n - 1) - j;
    default: return -1;
  }
}

constexpr int LD = L + 1;  // LDS row stride (odd: spreads the stride-67 pass over banks)

// Global-memory loops issue kBatch independent loads per thread before using any of them, so each
// wave keeps many requests in flight (a plain loop would wait out the full HBM latency per element).
constexpr int kBatch = 8;

// ---- row forward: padded rows 2t, 2t + 1 of the plane as one complex row; half spectrum out ----
struct RowsArgs {
  const float* x;   // (P, H, W)
  float2* S;        // (P, NC, L): column v, row r
  const float2* bh; // FFT(b)/66 forward, then inverse direction (2 x 66)
  int H, W, pad, mode, nrp;
};

__global__ void __launch_bounds__(256) k_pfa_rows_fwd(RowsArgs a) {
  extern __shared__ float2 sm[];
  float2* bh = sm;            // 66
  float2* buf = sm + 2 * RM;  // nrp rows of LD
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t plane = blockIdx.y;
  const int t0 = blockIdx.x * a.nrp;  // first row pair
  const int nrp = min(a.nrp, L / 2 - t0);
  for (int i = tid; i < RM; i += nth) bh[i] = a.bh[i];
  // per-block index tables: source column and LDS position of each padded column, source row of
  // each padded row of the block
  short* csrc = (short*)(buf + a.nrp * LD);
  short* cpos = csrc + L;
  short* rsrc = cpos + L;
  for (int n = tid; n < L; n += nth) {
    csrc[n] = (short)pad_map(n, a.W, a.pad, a.mode);
    cpos[n] = (short)pos_in(n);
  }
  for (int r = tid; r < 2 * nrp; r += nth) rsrc[r] = (short)pad_map(2 * t0 + r, a.H, a.pad, a.mode);
  __syncthreads();
  const float* xp = a.x + plane * (int64_t)a.H * a.W;
  for (int i0 = tid; i0 < nrp * L; i0 += kBatch * nth) {
    float2 v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      v[k] = make_float2(0.f, 0.f);
      if (idx < nrp * L) {
        const int t = idx / L, n = idx - t * L;
        const int sc = csrc[n], ra = rsrc[2 * t], rb = rsrc[2 * t + 1];
        if (sc >= 0) {
          if (ra >= 0) v[k].x = xp[(int64_t)ra * a.W + sc];
          if (rb >= 0) v[k].y = xp[(int64_t)rb * a.W + sc];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < nrp * L) {
        const int t = idx / L, n = idx - t * L;
        buf[t * LD + cpos[n]] = v[k];
      }
    }
  }
  __syncthreads();
  pass_a<false>(buf, nrp, LD, bh, tid, nth);
  __syncthreads();
  pass_b<false>(buf, nrp, LD, tid, nth);
  __syncthreads();
  // unpack two real rows: Ya = (Z[v] + conj Z[-v]) / 2, Yb = (Z[v] - conj Z[-v]) / (2i)
  float2* Sp = a.S + plane * (int64_t)NC * L;
  for (int idx = tid; idx < NC * 2 * nrp; idx += nth) {
    const int v = idx / (2 * nrp), rl = idx - v * 2 * nrp;
    const int t = rl >> 1;
    const float2 z = buf[t * LD + fpos(v)];
    const float2 zm = buf[t * LD + fpos(v == 0 ? 0 : L - v)];
    const float2 o = (rl & 1) == 0 ? make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y))
                                   : make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x));
    Sp[(int64_t)v * L + 2 * t0 + rl] = o;
  }
}

// ---- columns: forward transform, x Phi, inverse transform, in place on S ----
struct ColsArgs {
  float2* S;            // (P, NC, L)
  const float2* phi;    // (Cp, NC, L) natural order, 1/(L L) folded in
  const float2* bh;     // 2 x 66
  int64_t C, psf_batch;
  int ncb;              // columns per block
};

__global__ void __launch_bounds__(256) k_pfa_cols(ColsArgs a) {
  extern __shared__ float2 sm[];
  float2* bhf = sm;
  float2* bhi = sm + RM;
  float2* buf = sm + 2 * RM;
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t plane = blockIdx.y;
  const int v0 = blockIdx.x * a.ncb;
  const int ncol = min(a.ncb, NC - v0);
  const int64_t cp = a.psf_batch == 1 ? plane % a.C : plane;
  for (int i = tid; i < 2 * RM; i += nth) sm[i] = a.bh[i];
  float2* Sp = a.S + (plane * NC + v0) * (int64_t)L;
  for (int u = tid; u < L; u += nth) {
    const int pu = pos_in(u);
    for (int cb = 0; cb < ncol; cb += kBatch) {
      float2 v[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (cb + k < ncol) v[k] = Sp[(int64_t)(cb + k) * L + u];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (cb + k < ncol) buf[(cb + k) * LD + pu] = v[k];
    }
  }
  __syncthreads();
  pass_a<false>(buf, ncol, LD, bhf, tid, nth);
  __syncthreads();
  pass_b<false>(buf, ncol, LD, tid, nth);
  __syncthreads();
  const float2* ph = a.phi + (cp * NC + v0) * (int64_t)L;
  for (int u = tid; u < L; u += nth) {
    const int fu = fpos(u);
    for (int cb = 0; cb < ncol; cb += kBatch) {
      float2 f[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (cb + k < ncol) f[k] = ph[(int64_t)(cb + k) * L + u];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (cb + k < ncol) {
          float2* sl = buf + (cb + k) * LD + fu;
          *sl = cmul(*sl, f[k]);
        }
    }
  }
  __syncthreads();
  pass_b<true>(buf, ncol, LD, tid, nth);
  __syncthreads();
  pass_a<true>(buf, ncol, LD, bhi, tid, nth);
  __syncthreads();
  for (int u = tid; u < L; u += nth) {
    const int pu = pos_in(u);
    for (int c = 0; c < ncol; ++c) Sp[(int64_t)c * L + u] = buf[c * LD + pu];
  }
}

// ---- row inverse: half spectra of rows 2t, 2t + 1 -> complex row -> inverse -> crop + store ----
struct RowsInvArgs {
  const float2* S;  // (P, NC, L)
  float* out;       // (P, H, W)
  const float2* bh; // 2 x 66 (the inverse-direction table is used)
  int H, W, pad, act, nrp;
};

__global__ void __launch_bounds__(256) k_pfa_rows_inv(RowsInvArgs a) {
  extern __shared__ float2 sm[];
  float2* bh = sm;
  float2* buf = sm + 2 * RM;
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t plane = blockIdx.y;
  const int t0 = blockIdx.x * a.nrp;  // first row pair of the padded plane
  const int nrp = min(a.nrp, L / 2 - t0);
  for (int i = tid; i < RM; i += nth) bh[i] = a.bh[RM + i];
  const float2* Sp = a.S + plane * (int64_t)NC * L;
  // Z[v] = Ha[v] + i Hb[v] over the full row, with H[-v] = conj H[v]
  for (int i0 = tid; i0 < nrp * L; i0 += kBatch * nth) {
    float4 h[kBatch];  // (Ha, Hb) of rows 2t, 2t + 1 at bin |v|; row pair fastest across lanes
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < nrp * L) {
        const int v = idx / nrp, t = idx - v * nrp;
        const int vv = v <= L / 2 ? v : L - v;
        h[k] = *(const float4*)(Sp + (int64_t)vv * L + 2 * (t0 + t));
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < nrp * L) {
        const int v = idx / nrp, t = idx - v * nrp;
        const bool lo = v <= L / 2;
        const int vv = lo ? v : L - v;
        float2 ha = make_float2(h[k].x, h[k].y), hb = make_float2(h[k].z, h[k].w);
        if (vv == 0 || vv == L / 2) { ha.y = 0.f; hb.y = 0.f; }
        if (!lo) { ha.y = -ha.y; hb.y = -hb.y; }
        buf[t * LD + fpos(v)] = make_float2(ha.x - hb.y, ha.y + hb.x);
      }
    }
  }
  __syncthreads();
  pass_b<true>(buf, nrp, LD, tid, nth);
  __syncthreads();
  pass_a<true>(buf, nrp, LD, bh, tid, nth);
  __syncthreads();
  float* op = a.out + plane * (int64_t)a.H * a.W;
  for (int c = tid; c < a.W; c += nth) {
    const int pc = pos_in(c + a.pad);
    for (int rl = 0; rl < 2 * nrp; ++rl) {
      const int row = 2 * t0 + rl - a.pad;
      if (row < 0 || row >= a.H) continue;
      const float2 z = buf[(rl >> 1) * LD + pc];
      float v = (rl & 1) ? z.y : z.x;
      if (a.act == CVN_ACT_GELU) v = gelu_fast(v);
      op[(int64_t)row * a.W + c] = v;
    }
  }
}

}  // namespace pfa268

// Host side --------------------------------------------------------------------------------------
namespace {
constexpr int kRowPairs = 16;  // row pairs (complex rows) per block: 4 x 16 = 64 DFT-67 items
constexpr int kCols = 16;      // columns per block
// Rader tables, the block's rows, and (row kernel) int16 column / row index tables
size_t pfa_lds(int rows) {
  return (size_t)(2 * pfa268::RM + rows * pfa268::LD) * sizeof(float2) + (2 * pfa268::L + 2 * rows) * sizeof(short);
}
bool g_pfa_attr = false;
}  // namespace

bool pfa268_applies(int h, int w, int s, const FftPlan& plan268) {
  return h == pfa268::L && w == pfa268::L && s == 1 && plan268.nrad == 1 && plan268.rad[0].R == pfa268::P &&
         plan268.rad[0].g == 2;
}

// S: (P, NC, L) scratch; phi: (Cp, NC, L); bh: the 67-point Rader table pair (bf, bi) of the
// plan tables of length 268.
int pfa268_forward(const float* x, int64_t P, int64_t C, int64_t psf_batch, int H, int W, int pad, int mode, int act,
                   const float2* phi, const float2* bh, float2* S, float* out, hipStream_t st) {
  using namespace pfa268;
  if (!g_pfa_attr) {
    hipFuncSetAttribute((const void*)k_pfa_rows_fwd, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    hipFuncSetAttribute((const void*)k_pfa_cols, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    hipFuncSetAttribute((const void*)k_pfa_rows_inv, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    hipGetLastError();
    g_pfa_attr = true;
  }
  const int nrb = (L / 2 + kRowPairs - 1) / kRowPairs;
  RowsArgs ra{x, S, bh, H, W, pad, mode, kRowPairs};
  hipLaunchKernelGGL(k_pfa_rows_fwd, dim3(nrb, (unsigned)P), dim3(4 * kRowPairs), pfa_lds(kRowPairs), st, ra);
  int rc = check_launch("268 row pass");
  if (rc != CVN_OK) return rc;
  ColsArgs ca{S, phi, bh, C, psf_batch, kCols};
  hipLaunchKernelGGL(k_pfa_cols, dim3((NC + kCols - 1) / kCols, (unsigned)P), dim3(4 * kCols), pfa_lds(kCols), st, ca);
  if ((rc = check_launch("268 column pass")) != CVN_OK) return rc;
  RowsInvArgs ia{S, out, bh, H, W, pad, act, kRowPairs};
  hipLaunchKernelGGL(k_pfa_rows_inv, dim3(nrb, (unsigned)P), dim3(4 * kRowPairs), pfa_lds(kRowPairs), st, ia);
  return check_launch("268 inverse row pass");
}

}  // namespace cvn
