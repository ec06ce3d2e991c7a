// Converse2D operator path (converse2d.cpp:165-209: arbitrary x0, scale s > 1) on transform lengths
// fixed at compile time.  Same three passes, scratch layout and arithmetic as the generic op path
// (converse2d_generic.hip: k_rows_fwd, k_cols_op, k_rows_inv), with
//   * every Stockham pass unrolled on a compile-time radix plan (constant strides, no runtime plan),
//   * the column pass launched once per pair of mirrored alias classes instead of once per class:
//     rows are real, so after the row transforms column Ws - v of every row spectrum is the complex
//     conjugate of column v (S(t, Ws - v) = conj S(t, v), t the spatial row), and the members of
//     class w - v0 are the conjugates of the members of class v0.  The block of class v0 in [0, w/2]
//     loads each of its s HR columns from the stored half spectrum (v <= Ws/2) or as the conjugate of
//     the mirrored stored column, and stores each solved column likewise; this halves the column
//     FFTs and the spectrum traffic of the pass;
//   * rows loaded and stored as 16-byte vectors.
// Scratch (host-defined, shared with the generic path): S (P, w/2+1, h) LR half spectrum column-major,
// S0 (P, Ws/2+1, Hs) HR spectrum of x0, SH (P, Ws/2+1, Hs) the solved spectrum after the inverse
// column transforms.  Tables: the op table's K and A, each (C, Ws, Hs), and the FFT twiddles
// exp(-2 pi i m / L) (fp64-evaluated) at the start of each length's plan table.
#include <math.h>

#include "cvn_common.h"

namespace cvn {
namespace {

constexpr int kOpT = 256;  // threads per block

// Radix plans, in pass order.
template <int L>
struct OpRadices;
// Radix plans, in pass order: the first radix is 16 (its butterflies write 16 consecutive elements, one
// padded block) and every later pass has P (the product of the radices before it) a multiple of 16,
// so that the padded slots of a butterfly's legs are a compile-time offset from its first leg.
template <> struct OpRadices<64> { static constexpr int n = 2, r[2] = {16, 4}; };
template <> struct OpRadices<128> { static constexpr int n = 2, r[2] = {16, 8}; };
template <> struct OpRadices<192> { static constexpr int n = 3, r[3] = {16, 4, 3}; };
template <> struct OpRadices<256> { static constexpr int n = 2, r[2] = {16, 16}; };
template <> struct OpRadices<384> { static constexpr int n = 3, r[3] = {16, 8, 3}; };
template <> struct OpRadices<512> { static constexpr int n = 3, r[3] = {16, 16, 2}; };
template <> struct OpRadices<768> { static constexpr int n = 3, r[3] = {16, 16, 3}; };
template <> struct OpRadices<1024> { static constexpr int n = 3, r[3] = {16, 16, 4}; };

template <int L, int ST>
constexpr int op_pprod() {  // product of the radices before pass ST
  int p = 1;
  for (int i = 0; i < ST; ++i) p *= OpRadices<L>::r[i];
  return p;
}

// LDS slot of element i of a transform buffer: one spare slot after every 16, so that the strided
// writes of the Stockham passes (a butterfly's R outputs are R consecutive elements) spread over the
// banks instead of landing 16 or 8 elements apart on the same ones.
__device__ __forceinline__ int lp(int i) { return i + (i >> 4); }
__host__ __device__ constexpr int lp_size(int n) { return n + (n - 1) / 16 + 1; }

// One radix-R Stockham pass over NTR transforms of length L stored back to back in one buffer (padded
// slots), in place: every thread first reads the legs of its butterflies into registers, the block
// synchronises, and then each butterfly is twiddled, transformed and written.  P is the product of the
// radices already applied.  Butterfly i, leg j reads element i + j T (T = L / R), takes the twiddle
// exp(-+2 pi i j k / (P R)) (k = i mod P), and writes element (i - k) R + k + j P.
template <int R, int L, int P, int NTR>
struct OpPass {
  static constexpr int T = L / R, TWS = L / (P * R), TOTAL = T * NTR, NB = (TOTAL + kOpT - 1) / kOpT;
  static_assert(L % 16 == 0 && (P == 1 ? R == 16 : P % 16 == 0), "padded-offset plan");
  static_assert(P * R < L || P == T, "the last pass writes the elements it reads");

  static __device__ __forceinline__ void read(const float2* buf, float2 (&u)[NB][R], int tid) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int idx = tid + q * kOpT;
      if (idx < TOTAL) {
        const int t = idx / T, i = idx - t * T, x = t * L + i, lx = lp(x);
#pragma unroll
        for (int j = 0; j < R; ++j) u[q][j] = buf[T % 16 == 0 ? lx + j * (T + T / 16) : lp(x + j * T)];
      }
    }
  }

  template <bool INV>
  static __device__ __forceinline__ void write(float2* buf, float2 (&u)[NB][R], const float2* tw, int tid) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int idx = tid + q * kOpT;
      if (idx < TOTAL) {
        const int t = idx / T, i = idx - t * T, k = i % P;
        if constexpr (P > 1) {
#pragma unroll
          for (int j = 1; j < R; ++j) u[q][j] = cmul(u[q][j], twid<INV>(tw[j * k * TWS]));
        }
        Dft<R, INV>::run(u[q]);
        // P == 1: the 16 outputs fill one padded block; P % 16 == 0: legs P apart
        const int l0 = lp(t * L + (i - k) * R + k);
#pragma unroll
        for (int j = 0; j < R; ++j) buf[P == 1 ? l0 + j : l0 + j * (P + P / 16)] = u[q][j];
      }
    }
  }
};

// All passes of the plan on NTR transforms of length L in buf, in place.  Every thread of the block
// calls it; it synchronises twice per pass, except in the last pass, whose butterflies write the
// elements they read (P = T there), so that no other thread's reads are pending on them.
template <int L, int ST, bool INV, int NTR>
__device__ __forceinline__ void op_fft(float2* buf, const float2* tw, int tid) {
  if constexpr (ST < OpRadices<L>::n) {
    using Ps = OpPass<OpRadices<L>::r[ST], L, op_pprod<L, ST>(), NTR>;
    float2 u[Ps::NB][OpRadices<L>::r[ST]];
    Ps::read(buf, u, tid);
    if constexpr (ST + 1 < OpRadices<L>::n) __syncthreads();
    Ps::template write<INV>(buf, u, tw, tid);
    __syncthreads();
    op_fft<L, ST + 1, INV, NTR>(buf, tw, tid);
  }
}

// The passes of two plans (N1 transforms of length L1 in b1, N2 of length L2 in b2) in lockstep, two
// barriers per phase; the second plan's butterflies start on the threads after the first plan's.
template <int L1, int N1, int L2, int N2, int ST, bool INV>
__device__ __forceinline__ void op_fft_pair(float2* b1, const float2* tw1, float2* b2, const float2* tw2, int tid) {
  constexpr int n1 = OpRadices<L1>::n, n2 = OpRadices<L2>::n;
  if constexpr (ST < n1 || ST < n2) {
    constexpr int R1 = ST < n1 ? OpRadices<L1>::r[ST] : 1, R2 = ST < n2 ? OpRadices<L2>::r[ST] : 1;
    constexpr int OFF = ST < n1 ? (N1 * (L1 / R1)) % kOpT : 0;
    const int tid2 = (tid + kOpT - OFF) % kOpT;
    using P1 = OpPass<ST < n1 ? R1 : 16, L1, ST < n1 ? op_pprod<L1, ST>() : 1, N1>;
    using P2 = OpPass<ST < n2 ? R2 : 16, L2, ST < n2 ? op_pprod<L2, ST>() : 1, N2>;
    float2 u1[ST < n1 ? P1::NB : 1][ST < n1 ? R1 : 16], u2[ST < n2 ? P2::NB : 1][ST < n2 ? R2 : 16];
    if constexpr (ST < n1) P1::read(b1, u1, tid);
    if constexpr (ST < n2) P2::read(b2, u2, tid2);
    if constexpr (ST + 1 < n1 || ST + 1 < n2) __syncthreads();  // not in a phase of last passes only
    if constexpr (ST < n1) P1::template write<INV>(b1, u1, tw1, tid);
    if constexpr (ST < n2) P2::template write<INV>(b2, u2, tw2, tid2);
    __syncthreads();
    op_fft_pair<L1, N1, L2, N2, ST + 1, INV>(b1, tw1, b2, tw2, tid);
  }
}

// Work item of block `blk` of a 1-D grid of n blocks.  The dispatcher places block i on XCD i mod 8;
// when n is a multiple of 8 each XCD is given a contiguous run of n / 8 work items instead, so
// neighbouring items (row blocks of one plane whose column runs share 128-byte lines; the planes of
// one channel that read the same transfer-table columns) run on one XCD and meet in its L2.
__device__ __forceinline__ int64_t xcd_item(int64_t blk, int64_t n) {
  return (n % 8 == 0) ? (blk & 7) * (n >> 3) + (blk >> 3) : blk;
}

__device__ __forceinline__ void copy_tw(float2* dst, const float2* src, int n, int tid) {
  for (int m = tid; m < n; m += kOpT) dst[m] = src[m];
}

// ------------------------------------------------------------------------------------------------
// Rows, forward: real rows (P, nrows, L) -> half spectra S[plane][c][row], c <= L/2.  Two real rows
// per complex transform (row 2t in .x, 2t+1 in .y), unpacked after the transform.
// ------------------------------------------------------------------------------------------------
template <int L, int RPB>
__global__ void __launch_bounds__(kOpT) k_oprows_fwd(const float* __restrict__ x, int nrows, int nblk, int64_t nitems,
                                                     const float2* __restrict__ twg, float2* __restrict__ S) {
  constexpr int NTR = RPB / 2, NC = L / 2 + 1, Q = L / 4, NLD = NTR * Q;
  extern __shared__ float2 sm[];
  float2* tw = sm;
  float2* A = tw + L;
  const int tid = threadIdx.x;
  const int64_t item = xcd_item(blockIdx.x, nitems);
  const int64_t plane = item / nblk;
  const int r0 = (int)(item - plane * nblk) * RPB;
  const float* xp = x + plane * (int64_t)nrows * L;
  constexpr int IT = (NLD + kOpT - 1) / kOpT;
  float4 va[IT], vb[IT];
#pragma unroll
  for (int k = 0; k < IT; ++k) {  // every load issued before the first LDS write
    const int idx = tid + k * kOpT;
    const int t = idx / Q, c4 = idx - t * Q;
    const int ra = r0 + 2 * t;
    va[k] = vb[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (idx < NLD && ra < nrows) va[k] = *(const float4*)(xp + (int64_t)ra * L + 4 * c4);
    if (idx < NLD && ra + 1 < nrows) vb[k] = *(const float4*)(xp + (int64_t)(ra + 1) * L + 4 * c4);
  }
  copy_tw(tw, twg, L, tid);
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int idx = tid + k * kOpT;
    if (idx < NLD) {
      const int t = idx / Q, c4 = idx - t * Q;
      float2* d = A + lp(t * L + 4 * c4);  // four consecutive slots (4 c4 .. 4 c4 + 3 share a 16-block)
      d[0] = make_float2(va[k].x, vb[k].x);
      d[1] = make_float2(va[k].y, vb[k].y);
      d[2] = make_float2(va[k].z, vb[k].z);
      d[3] = make_float2(va[k].w, vb[k].w);
    }
  }
  __syncthreads();
  op_fft<L, 0, false, NTR>(A, tw, tid);
  const float2* Z = A;
  // Ya = (Z[c] + conj Z[-c]) / 2, Yb = (Z[c] - conj Z[-c]) / (2i); consecutive threads take
  // consecutive rows of one column, so each column's RPB rows are stored as one contiguous run.
  float2* Sp = S + plane * (int64_t)NC * nrows;
  for (int idx = tid; idx < NC * RPB; idx += kOpT) {
    const int c = idx / RPB, rl = idx - c * RPB;
    const int r = r0 + rl;
    if (r >= nrows) continue;
    const int t = rl >> 1;
    const float2 z = Z[lp(t * L + c)];
    const float2 zm = Z[lp(t * L + (c == 0 ? 0 : L - c))];
    const float2 v = (rl & 1) == 0 ? make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y))
                                   : make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x));
    Sp[(int64_t)c * nrows + r] = v;
  }
}

// ------------------------------------------------------------------------------------------------
// Rows, inverse: half spectra SH[plane][v][row] -> real rows (P, nrows, L), uncropped.
// ------------------------------------------------------------------------------------------------
template <int L, int RPB>
__global__ void __launch_bounds__(kOpT) k_oprows_inv(const float2* __restrict__ SH, int nrows, int nblk,
                                                     int64_t nitems, const float2* __restrict__ twg,
                                                     float* __restrict__ out, int act) {
  constexpr int NTR = RPB / 2, NC = L / 2 + 1, Q = L / 4, NST = NTR * Q;
  extern __shared__ float2 sm[];
  float2* tw = sm;
  float2* A = tw + L;
  float2* Bf = A + lp_size(NTR * L);  // the staged half spectra, Bf[rl * NC + v]
  const int tid = threadIdx.x;
  const int64_t item = xcd_item(blockIdx.x, nitems);
  const int64_t plane = item / nblk;
  const int r0 = (int)(item - plane * nblk) * RPB;
  const float2* SHp = SH + plane * (int64_t)NC * nrows;
  constexpr int IT = (NC * RPB + kOpT - 1) / kOpT;
  float2 val[IT];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int idx = tid + k * kOpT;
    const int v = idx / RPB, rl = idx - v * RPB;
    val[k] = make_float2(0.f, 0.f);
    if (idx < NC * RPB && r0 + rl < nrows) val[k] = SHp[(int64_t)v * nrows + r0 + rl];
  }
  copy_tw(tw, twg, L, tid);
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int idx = tid + k * kOpT;
    if (idx < NC * RPB) {
      const int v = idx / RPB, rl = idx - v * RPB;
      if (v == 0 || 2 * v == L) val[k].y = 0.f;  // the real part of the inverse transform
      Bf[rl * NC + v] = val[k];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < NTR * L; idx += kOpT) {
    const int t = idx / L, v = idx - t * L;
    const bool lo = v <= L / 2;
    const int vv = lo ? v : L - v;
    float2 ha = Bf[(2 * t) * NC + vv], hb = Bf[(2 * t + 1) * NC + vv];
    if (!lo) {
      ha.y = -ha.y;
      hb.y = -hb.y;
    }
    A[lp(t * L + v)] = make_float2(ha.x - hb.y, ha.y + hb.x);
  }
  __syncthreads();
  op_fft<L, 0, true, NTR>(A, tw, tid);
  const float2* Z = A;
  float* op = out + plane * (int64_t)nrows * L;
  for (int idx = tid; idx < NST; idx += kOpT) {
    const int t = idx / Q, c4 = idx - t * Q;
    const int ra = r0 + 2 * t;
    const float2* z = Z + lp(t * L + 4 * c4);  // four consecutive slots
    float2 z0 = z[0], z1 = z[1], z2 = z[2], z3 = z[3];
    if (act == CVN_ACT_GELU) {
      z0 = make_float2(gelu_fast(z0.x), gelu_fast(z0.y));
      z1 = make_float2(gelu_fast(z1.x), gelu_fast(z1.y));
      z2 = make_float2(gelu_fast(z2.x), gelu_fast(z2.y));
      z3 = make_float2(gelu_fast(z3.x), gelu_fast(z3.y));
    }
    if (ra < nrows) *(float4*)(op + (int64_t)ra * L + 4 * c4) = make_float4(z0.x, z1.x, z2.x, z3.x);
    if (ra + 1 < nrows) *(float4*)(op + (int64_t)(ra + 1) * L + 4 * c4) = make_float4(z0.y, z1.y, z2.y, z3.y);
  }
}

// ------------------------------------------------------------------------------------------------
// Columns: per (plane, alias class v0 in [0, w/2]).  LR column v0 (H points) and the S member columns
// vb = v0 + b w (HS = S H points each) are transformed forward, solved as in k_cols_op
//   m = sum_{a, b} K(u0 + a H, vb) X0(u0 + a H, vb),  d = Y(u0) - m / S^2,
//   X(u, vb) = X0(u, vb) / (Hs Ws) + A(u, vb) d,
// transformed back and stored (column vb itself, or the conjugate into column Ws - vb).
// ------------------------------------------------------------------------------------------------
struct OpColCtArgs {
  const float2* S;    // (P, NC, h)
  const float2* S0;   // (P, NCs, Hs)
  const float2* kf;   // (C, Ws, Hs)
  const float2* A;    // (C, Ws, Hs)
  float2* SH;         // (P, NCs, Hs)
  const float2* tw_h; // LR column twiddles (h entries)
  const float2* tw_H; // HR column twiddles (Hs entries)
  int64_t B, C, nitems;  // nitems = B C (w/2 + 1) blocks
  int w, Ws;
};

template <int H, int S>
__global__ void __launch_bounds__(kOpT) k_opcols(OpColCtArgs a) {
  constexpr int HS = H * S;
  extern __shared__ float2 sm[];
  float2* twh = sm;
  float2* twH = twh + H;
  float2* Y = twH + HS;
  float2* X = Y + lp_size(H);
  const int tid = threadIdx.x;
  const int NC = a.w / 2 + 1, NCs = a.Ws / 2 + 1;
  // work item (channel c, class v0, batch element bi), bi fastest: the B planes of a channel read the
  // same transfer-table columns one after the other on one XCD
  const int64_t item = xcd_item(blockIdx.x, a.nitems);
  const int64_t bi = item % a.B, cv = item / a.B;
  const int v0 = (int)(cv % NC);
  const int64_t c = cv / NC;
  const int64_t plane = bi * a.C + c;
  const float2* Sp = a.S + plane * (int64_t)NC * H;
  const float2* S0p = a.S0 + plane * (int64_t)NCs * HS;
  // loads first (LR column and the S member columns), then the twiddle copies
  constexpr int ITY = (H + kOpT - 1) / kOpT, ITX = (S * HS + kOpT - 1) / kOpT;
  float2 ly[ITY], lx[ITX];
#pragma unroll
  for (int k = 0; k < ITY; ++k) {
    const int u = tid + k * kOpT;
    ly[k] = u < H ? Sp[(int64_t)v0 * H + u] : make_float2(0.f, 0.f);
  }
#pragma unroll
  for (int k = 0; k < ITX; ++k) {
    const int idx = tid + k * kOpT;
    lx[k] = make_float2(0.f, 0.f);
    if (idx < S * HS) {
      const int b = idx / HS, u = idx - b * HS;
      const int vb = v0 + b * a.w;
      lx[k] = vb <= a.Ws / 2 ? S0p[(int64_t)vb * HS + u] : cconj(S0p[(int64_t)(a.Ws - vb) * HS + u]);
    }
  }
  static_assert(H <= kOpT, "one row class per thread");
  const float2* kf = a.kf + c * (int64_t)a.Ws * HS;
  const float2* Am = a.A + c * (int64_t)a.Ws * HS;
  copy_tw(twh, a.tw_h, H, tid);
  copy_tw(twH, a.tw_H, HS, tid);
#pragma unroll
  for (int k = 0; k < ITY; ++k)
    if (tid + k * kOpT < H) Y[lp(tid + k * kOpT)] = ly[k];
#pragma unroll
  for (int k = 0; k < ITX; ++k)
    if (tid + k * kOpT < S * HS) X[lp(tid + k * kOpT)] = lx[k];
  __syncthreads();
  op_fft<H, 0, false, 1>(Y, twh, tid);  // the LR column, then the S member columns
  op_fft<HS, 0, false, S>(X, twH, tid);
  const float inv_s2 = 1.0f / (float)(S * S);
  const float norm = 1.0f / ((float)HS * (float)a.Ws);
  if (tid < H) {
    // this thread's row class u0 = tid: its transfer-table entries (both tables requested before
    // either is used), the S x S member values, the alias-class mean and the update
    const int u0 = tid;
    float2 kv[S * S], av[S * S];
#pragma unroll
    for (int b = 0; b < S; ++b)
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const int64_t o = (int64_t)(v0 + b * a.w) * HS + u0 + aa * H;
        kv[b * S + aa] = kf[o];
        av[b * S + aa] = Am[o];
      }
    float2 x0v[S * S];
    float2 m = make_float2(0.f, 0.f);
#pragma unroll
    for (int b = 0; b < S; ++b)
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        x0v[b * S + aa] = X[lp(b * HS + u0 + aa * H)];
        const float2 t = cmul(kv[b * S + aa], x0v[b * S + aa]);
        m.x += t.x;
        m.y += t.y;
      }
    const float2 y = Y[lp(u0)];
    const float2 d = make_float2(y.x - m.x * inv_s2, y.y - m.y * inv_s2);
#pragma unroll
    for (int b = 0; b < S; ++b)
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const float2 t = cmul(av[b * S + aa], d), xv = x0v[b * S + aa];
        X[lp(b * HS + u0 + aa * H)] = make_float2(fmaf(xv.x, norm, t.x), fmaf(xv.y, norm, t.y));
      }
  }
  __syncthreads();
  op_fft<HS, 0, true, S>(X, twH, tid);
  const float2* R = X;
  // members in the stored half go to their own column; the others, as conjugates, to the mirrored
  // column Ws - vb, unless that column is a member of this same class (v0 = 0 or w/2), whose
  // block already stores it directly
  const bool self_mirror = (v0 == 0) || (2 * v0 == a.w);
  float2* SHp = a.SH + plane * (int64_t)NCs * HS;
  for (int idx = tid; idx < S * HS; idx += kOpT) {
    const int b = idx / HS, u = idx - b * HS;
    const int vb = v0 + b * a.w;
    if (vb <= a.Ws / 2)
      SHp[(int64_t)vb * HS + u] = R[lp(idx)];
    else if (!self_mirror)
      SHp[(int64_t)(a.Ws - vb) * HS + u] = cconj(R[lp(idx)]);
  }
}

// ------------------------------------------------------------------------------------------------
// Columns, module form (x0 = nearest(y), util_converse.py:165-190): per (plane, CPB consecutive HR
// columns v of the stored half), X(u, v) = Phi(u, v) Y(u mod H, v mod w) with Y the LR spectrum,
// then the inverse HR column transform; the same product and table as k_cols_module.
// ------------------------------------------------------------------------------------------------
struct ModColCtArgs {
  const float2* S;    // (P, w/2+1, H) LR row spectra
  const float2* phi;  // (Cp, Ws/2+1, Hs) module table
  float2* SH;         // (P, Ws/2+1, Hs)
  const float2* tw_h; // LR column twiddles (H entries)
  const float2* tw_H; // HR column twiddles (Hs entries)
  int64_t C, psf_batch, nitems;  // nitems = P * nblk
  int w, Ws, nblk;               // nblk = column blocks per plane
};

template <int H, int S, int CPB>
__global__ void __launch_bounds__(kOpT) k_modcols(ModColCtArgs a) {
  constexpr int HS = H * S;
  extern __shared__ float2 sm[];
  float2* twh = sm;
  float2* twH = twh + H;
  float2* Y = twH + HS;              // CPB LR columns
  float2* X = Y + lp_size(CPB * H);  // CPB HR columns
  const int tid = threadIdx.x;
  const int NC = a.w / 2 + 1, NCs = a.Ws / 2 + 1;
  // work item (plane, column block), planes of one channel adjacent (they share the table when
  // psf_batch is 1): item = (c, b, block) with the block fastest
  const int64_t item = xcd_item(blockIdx.x, a.nitems);
  const int64_t pidx = item / a.nblk;
  const int vbeg = (int)(item - pidx * a.nblk) * CPB;
  const int64_t B = a.nitems / a.nblk / a.C;
  const int64_t c = pidx / B, bi = pidx - c * B;
  const int64_t plane = bi * a.C + c;
  const int64_t cp = a.psf_batch == 1 ? c : plane;
  const int ncol = min(CPB, NCs - vbeg);
  const float2* Sp = a.S + plane * (int64_t)NC * H;
  const float2* ph = a.phi + cp * (int64_t)NCs * HS;
  constexpr int ITY = (CPB * H + kOpT - 1) / kOpT, ITX = (CPB * HS + kOpT - 1) / kOpT;
  float2 ly[ITY], lf[ITX];
#pragma unroll
  for (int k = 0; k < ITY; ++k) {
    const int idx = tid + k * kOpT;
    const int cl = idx / H, u = idx - cl * H;
    ly[k] = make_float2(0.f, 0.f);
    if (idx < CPB * H && cl < ncol) {
      const int vv = (vbeg + cl) % a.w;  // row spectra of real rows are Hermitian in the column
      ly[k] = vv <= a.w / 2 ? Sp[(int64_t)vv * H + u] : cconj(Sp[(int64_t)(a.w - vv) * H + u]);
    }
  }
#pragma unroll
  for (int k = 0; k < ITX; ++k) {
    const int idx = tid + k * kOpT;
    const int cl = idx / HS, u = idx - cl * HS;
    lf[k] = (idx < CPB * HS && cl < ncol) ? ph[(int64_t)(vbeg + cl) * HS + u] : make_float2(0.f, 0.f);
  }
  copy_tw(twh, a.tw_h, H, tid);
  copy_tw(twH, a.tw_H, HS, tid);
#pragma unroll
  for (int k = 0; k < ITY; ++k)
    if (tid + k * kOpT < CPB * H) Y[lp(tid + k * kOpT)] = ly[k];
  __syncthreads();
  op_fft<H, 0, false, CPB>(Y, twh, tid);
#pragma unroll
  for (int k = 0; k < ITX; ++k) {
    const int idx = tid + k * kOpT;
    if (idx < CPB * HS) {
      const int cl = idx / HS, u = idx - cl * HS;
      X[lp(idx)] = cmul(Y[lp(cl * H + u % H)], lf[k]);
    }
  }
  __syncthreads();
  op_fft<HS, 0, true, CPB>(X, twH, tid);
  float2* SHp = a.SH + plane * (int64_t)NCs * HS;
  for (int idx = tid; idx < ncol * HS; idx += kOpT) {
    const int cl = idx / HS, u = idx - cl * HS;
    SHp[(int64_t)(vbeg + cl) * HS + u] = X[lp(idx)];
  }
}

// Rows per block of the row passes, by length (LDS: about L + RPB L complex values, and the inverse
// pass's staging of RPB (L / 2 + 1) more; at most ~108 KB).  8 rows at 768 and 1024 points rather
// than 4: the stores of a column run then cover 64 bytes instead of 32 (reference grid at s = 3:
// 0.3215 -> 0.3145 ms; 16 rows measured 0.384 ms, the inverse pass's LDS then allowing one block per CU).
template <int L>
constexpr int op_rpb() {
  return L <= 128 ? 32 : (L <= 256 ? 16 : 8);
}
// Staging buffer of the inverse row pass: RPB rows of L / 2 + 1 bins.
template <int L>
constexpr int op_inv_bf() {
  return op_rpb<L>() * (L / 2 + 1);
}

// Dynamic LDS above 64 KiB needs the kernel's limit raised, once per device.
template <class K>
void raise_lds_limit(K kernel, std::atomic<uint64_t>& done) {
  once_per_device(done, [&] {
    (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  });
}

template <int L>
int launch_oprows_fwd(const float* x, int64_t P, int nrows, const float2* tw, float2* S, hipStream_t st) {
  constexpr int RPB = op_rpb<L>();
  const size_t lds = (size_t)(L + lp_size(RPB / 2 * L)) * sizeof(float2);
  static std::atomic<uint64_t> done{0};
  raise_lds_limit(k_oprows_fwd<L, RPB>, done);
  const int nblk = (nrows + RPB - 1) / RPB;
  hipLaunchKernelGGL((k_oprows_fwd<L, RPB>), dim3((unsigned)(nblk * P)), dim3(kOpT), lds, st, x, nrows, nblk,
                     (int64_t)nblk * P, tw, S);
  return check_launch("op row forward pass (compile-time plan)");
}

template <int L>
int launch_oprows_inv(const float2* SH, int64_t P, int nrows, const float2* tw, float* out, int act, hipStream_t st) {
  constexpr int RPB = op_rpb<L>();
  const size_t lds = (size_t)(L + lp_size(RPB / 2 * L) + op_inv_bf<L>()) * sizeof(float2);
  static std::atomic<uint64_t> done{0};
  raise_lds_limit(k_oprows_inv<L, RPB>, done);
  const int nblk = (nrows + RPB - 1) / RPB;
  hipLaunchKernelGGL((k_oprows_inv<L, RPB>), dim3((unsigned)(nblk * P)), dim3(kOpT), lds, st, SH, nrows, nblk,
                     (int64_t)nblk * P, tw, out, act);
  return check_launch("op row inverse pass (compile-time plan)");
}

template <int H, int S>
int launch_opcols(const OpColCtArgs& a, int64_t P, hipStream_t st) {
  constexpr int HS = H * S;
  const size_t lds = (size_t)(H + HS + lp_size(H) + lp_size(S * HS)) * sizeof(float2);
  static std::atomic<uint64_t> done{0};
  raise_lds_limit(k_opcols<H, S>, done);
  hipLaunchKernelGGL((k_opcols<H, S>), dim3((unsigned)a.nitems), dim3(kOpT), lds, st, a);
  return check_launch("op column pass (compile-time plan)");
}

template <int H, int S>
int launch_modcols(ModColCtArgs a, int64_t P, hipStream_t st) {
  constexpr int HS = H * S, CPB = HS >= 512 ? 1 : (HS >= 256 ? 2 : 4);
  const size_t lds = (size_t)(H + HS + lp_size(CPB * H) + lp_size(CPB * HS)) * sizeof(float2);
  a.nblk = (a.Ws / 2 + 1 + CPB - 1) / CPB;
  a.nitems = P * a.nblk;
  static std::atomic<uint64_t> done{0};
  raise_lds_limit(k_modcols<H, S, CPB>, done);
  hipLaunchKernelGGL((k_modcols<H, S, CPB>), dim3((unsigned)a.nitems), dim3(kOpT), lds, st, a);
  return check_launch("module column pass (compile-time plan)");
}

bool op_len_ok(int L) {
  switch (L) {
    case 64: case 128: case 192: case 256: case 384: case 512: case 768: case 1024: return true;
    default: return false;
  }
}

int rows_fwd_any(int L, const float* x, int64_t P, int nrows, const float2* tw, float2* S, hipStream_t st) {
  switch (L) {
    case 64: return launch_oprows_fwd<64>(x, P, nrows, tw, S, st);
    case 128: return launch_oprows_fwd<128>(x, P, nrows, tw, S, st);
    case 192: return launch_oprows_fwd<192>(x, P, nrows, tw, S, st);
    case 256: return launch_oprows_fwd<256>(x, P, nrows, tw, S, st);
    case 384: return launch_oprows_fwd<384>(x, P, nrows, tw, S, st);
    case 512: return launch_oprows_fwd<512>(x, P, nrows, tw, S, st);
    case 768: return launch_oprows_fwd<768>(x, P, nrows, tw, S, st);
    case 1024: return launch_oprows_fwd<1024>(x, P, nrows, tw, S, st);
    default: return fail(CVN_ERR_UNSUPPORTED, "no compile-time row plan for length %d", L);
  }
}

int rows_inv_any(int L, const float2* SH, int64_t P, int nrows, const float2* tw, float* out, int act,
                 hipStream_t st) {
  switch (L) {
    case 128: return launch_oprows_inv<128>(SH, P, nrows, tw, out, act, st);
    case 192: return launch_oprows_inv<192>(SH, P, nrows, tw, out, act, st);
    case 256: return launch_oprows_inv<256>(SH, P, nrows, tw, out, act, st);
    case 384: return launch_oprows_inv<384>(SH, P, nrows, tw, out, act, st);
    case 512: return launch_oprows_inv<512>(SH, P, nrows, tw, out, act, st);
    case 768: return launch_oprows_inv<768>(SH, P, nrows, tw, out, act, st);
    case 1024: return launch_oprows_inv<1024>(SH, P, nrows, tw, out, act, st);
    default: return fail(CVN_ERR_UNSUPPORTED, "no compile-time row plan for length %d", L);
  }
}

int cols_any(int h, int s, const OpColCtArgs& a, int64_t P, hipStream_t st) {
  const int key = h * 8 + s;
  switch (key) {
    case 64 * 8 + 2: return launch_opcols<64, 2>(a, P, st);
    case 64 * 8 + 3: return launch_opcols<64, 3>(a, P, st);
    case 64 * 8 + 4: return launch_opcols<64, 4>(a, P, st);
    case 128 * 8 + 2: return launch_opcols<128, 2>(a, P, st);
    case 128 * 8 + 3: return launch_opcols<128, 3>(a, P, st);
    case 128 * 8 + 4: return launch_opcols<128, 4>(a, P, st);
    case 256 * 8 + 2: return launch_opcols<256, 2>(a, P, st);
    case 256 * 8 + 3: return launch_opcols<256, 3>(a, P, st);
    case 256 * 8 + 4: return launch_opcols<256, 4>(a, P, st);
    default: return fail(CVN_ERR_UNSUPPORTED, "no compile-time column plan for h = %d, s = %d", h, s);
  }
}

int modcols_any(int h, int s, const ModColCtArgs& a, int64_t P, hipStream_t st) {
  switch (h * 8 + s) {
    case 64 * 8 + 2: return launch_modcols<64, 2>(a, P, st);
    case 64 * 8 + 3: return launch_modcols<64, 3>(a, P, st);
    case 64 * 8 + 4: return launch_modcols<64, 4>(a, P, st);
    case 128 * 8 + 2: return launch_modcols<128, 2>(a, P, st);
    case 128 * 8 + 3: return launch_modcols<128, 3>(a, P, st);
    case 128 * 8 + 4: return launch_modcols<128, 4>(a, P, st);
    case 256 * 8 + 2: return launch_modcols<256, 2>(a, P, st);
    case 256 * 8 + 3: return launch_modcols<256, 3>(a, P, st);
    case 256 * 8 + 4: return launch_modcols<256, 4>(a, P, st);
    default: return fail(CVN_ERR_UNSUPPORTED, "no compile-time column plan for h = %d, s = %d", h, s);
  }
}

bool opct_disabled() {
  static const bool off = [] {
    const char* e = getenv("CVN_DISABLE_OPCT");
    return e && e[0] == '1';
  }();
  return off;
}

}  // namespace

bool module_ct_supported(int h, int w, int s, int pad) { return pad == 0 && op_ct_supported(h, w, s); }

int launch_module_ct(const float* x, int64_t P, int64_t C, int64_t psf_batch, int h, int w, int s, int act,
                     const float2* tw_w, const float2* tw_h, const float2* tw_Hs, const float2* tw_Ws,
                     const float2* phi, float2* S, float2* SH, float* out, hipStream_t st) {
  if (!module_ct_supported(h, w, s, 0)) return fail(CVN_ERR_UNSUPPORTED, "module path: no compile-time plan");
  if ((uintptr_t)x % 16 || (uintptr_t)out % 16)
    return fail(CVN_ERR_UNSUPPORTED, "module path: compile-time kernels need 16-byte aligned planes");
  int rc;
  if ((rc = rows_fwd_any(w, x, P, h, tw_w, S, st)) != CVN_OK) return rc;
  ModColCtArgs ca;
  ca.S = S; ca.phi = phi; ca.SH = SH; ca.tw_h = tw_h; ca.tw_H = tw_Hs;
  ca.C = C; ca.psf_batch = psf_batch; ca.w = w; ca.Ws = w * s; ca.nblk = 0; ca.nitems = 0;
  if ((rc = modcols_any(h, s, ca, P, st)) != CVN_OK) return rc;
  return rows_inv_any(w * s, SH, P, h * s, tw_Ws, out, act, st);
}

bool op_ct_supported(int h, int w, int s) {
  if (opct_disabled() || s < 2 || s > 4) return false;
  if (h != 64 && h != 128 && h != 256) return false;
  return op_len_ok(w) && op_len_ok(w * s) && w % 4 == 0;
}

int launch_op_ct(const float* x, const float* x0, int64_t P, int64_t C, int h, int w, int s, const float2* tw_w,
                 const float2* tw_h, const float2* tw_Hs, const float2* tw_Ws, const float2* kf, const float2* A,
                 float2* S, float2* S0, float2* SH, float* out, hipStream_t st) {
  if (!op_ct_supported(h, w, s)) return fail(CVN_ERR_UNSUPPORTED, "op path: no compile-time plan");
  if (P > 65535) return fail(CVN_ERR_UNSUPPORTED, "B*C exceeds 65535");
  if ((uintptr_t)x % 16 || (uintptr_t)x0 % 16 || (uintptr_t)out % 16)
    return fail(CVN_ERR_UNSUPPORTED, "op path: compile-time kernels need 16-byte aligned planes");
  int rc;
  if ((rc = rows_fwd_any(w, x, P, h, tw_w, S, st)) != CVN_OK) return rc;
  if ((rc = rows_fwd_any(w * s, x0, P, h * s, tw_Ws, S0, st)) != CVN_OK) return rc;
  OpColCtArgs ca;
  ca.S = S; ca.S0 = S0; ca.kf = kf; ca.A = A; ca.SH = SH; ca.tw_h = tw_h; ca.tw_H = tw_Hs;
  ca.B = P / C; ca.C = C; ca.nitems = P * (w / 2 + 1); ca.w = w; ca.Ws = w * s;
  if ((rc = cols_any(h, s, ca, P, st)) != CVN_OK) return rc;
  return rows_inv_any(w * s, SH, P, h * s, tw_Ws, out, CVN_ACT_NONE, st);
}

}  // namespace cvn
