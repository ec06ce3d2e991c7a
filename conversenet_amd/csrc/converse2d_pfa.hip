// Converse2D forward for 268 x 268 padded planes (Converse-DnCNN: 256 x 256, padding 6), scale 1.
//
// Same three-pass data flow as the generic path (row transform -> column transform x Phi x inverse
// -> inverse row transform, half spectra column-major in between), but every transform is the
// prime-factor FFT 268 = 4 * 67 (no twiddles) on one quad of lanes: each lane holds one PFA segment
// of 67 complex values in registers, runs the 67-point DFT on it, and the 4-point DFT runs across
// the quad through DPP permutes (layout and index maps at the quad helpers below).
//
// The 67-point DFT is one thread's work, entirely in registers, by Rader's algorithm (primitive
// root 2): a_q = u[2^q mod 67], X_0 = u_0 + sum a, X[2^-q mod 67] = u_0 + (a (*) b)_q with the cyclic
// convolution of length 66 done as an in-register prime-factor FFT 66 = 2 * 3 * 11, a product with
// FFT(b)/66 (compile-time constants) and the inverse FFT.  Slot s of the 66-register array holds the
// convolution input a[s]; after the forward 3-axis DFT it holds the transform at k = kappa(s)
// (k = s mod 6, k = 2 s mod 11), and after the inverse 3-axis DFT it holds the convolution output at
// s again.  (C. M. Rader, Proc. IEEE 56(6), 1968; I. J. Good, J. R. Stat. Soc. B 20, 1958.)
#include <math.h>

#include <algorithm>

#include "cvn_common.h"

namespace cvn {
namespace pfa268 {

constexpr int L = 268, P = 67, RM = 66, NC = L / 2 + 1;  // NC: half-spectrum bins
// Between the passes a half-spectrum column occupies LP = 272 rows (2176 B, a whole number of 128-B
// lines; rows 268..271 are padding), and the row passes index LQ = 136 quads per plane (134 row
// pairs and 2 idle quads on the padding rows), so that each wave's 16 quads cover whole 128-B lines
// of every column they read or write: no line is shared between waves, each is fetched once.
constexpr int LP = 272, LQ = 136;

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

// cos and sin of 2 pi m / n by Taylor series in double at compile time (|angle| <= pi after
// reduction; 40 terms leave a truncation error far below double rounding).
struct CosSin {
  double c, s;
};
constexpr CosSin cos_sin_turn(int m, int n) {
  m %= n;
  if (2 * m >= n) m -= n;  // angle in [-pi, pi)
  const double x = 2.0 * 3.14159265358979323846 * m / n;
  double c = 0.0, s = 0.0, term = 1.0;  // term = x^k / k!
  for (int k = 0; k < 40; ++k) {
    const int r = k & 3;
    if (r == 0) c += term;
    if (r == 1) s += term;
    if (r == 2) c -= term;
    if (r == 3) s -= term;
    term = term * x / (k + 1);
  }
  return CosSin{c, s};
}
// Rader tables of the 67-point DFT (primitive root 2): b_q = W67^(2^-q mod 67), bf = FFT66(b) / 66
// (forward) and bi = FFT66(conj b) / 66 (inverse), evaluated in double at compile time and rounded
// once.  Their indices are compile-time constants in dft67_reg, so the values become instruction
// literals and occupy no registers.
struct RaderTabs {
  float bfr[RM], bfi[RM], bir[RM], bii[RM];
  constexpr RaderTabs() : bfr(), bfi(), bir(), bii() {
    double br[RM] = {}, bim[RM] = {}, wr[RM] = {}, wi[RM] = {};
    for (int q = 0; q < RM; ++q) {
      const CosSin b = cos_sin_turn(Tabs().gq[q], P), w = cos_sin_turn(q, RM);
      br[q] = b.c;
      bim[q] = -b.s;  // exp(-2 pi i gq / 67)
      wr[q] = w.c;
      wi[q] = -w.s;  // exp(-2 pi i q / 66)
    }
    for (int m = 0; m < RM; ++m) {
      double fr = 0, fi = 0, ir = 0, ii = 0;
      for (int q = 0; q < RM; ++q) {
        const int e = (q * m) % RM;
        fr += br[q] * wr[e] - bim[q] * wi[e];
        fi += br[q] * wi[e] + bim[q] * wr[e];
        ir += br[q] * wr[e] + bim[q] * wi[e];  // conj(b) w
        ii += br[q] * wi[e] - bim[q] * wr[e];
      }
      bfr[m] = (float)(fr / RM);
      bfi[m] = (float)(fi / RM);
      bir[m] = (float)(ir / RM);
      bii[m] = (float)(ii / RM);
    }
  }
};
constexpr RaderTabs kR{};

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

// 67-point DFT of the 67 registers x[0..66] in place (forward, or inverse without normalisation).
template <bool INV>
__device__ __forceinline__ void dft67_reg(float2 (&x)[P]) {
  float2 a[RM];
  const float2 u0 = x[0];
#pragma unroll
  for (int q = 0; q < RM; ++q) a[q] = x[kT.gp[q]];
  dft66_axes<false>(a);
  const float2 x0 = cadd(u0, a[0]);  // slot 0 holds bin 0: sum of the a's
#pragma unroll
  for (int s = 0; s < RM; ++s) {
    const int k = kT.kap[s];
    a[s] = cmul(a[s], INV ? make_float2(kR.bir[k], kR.bii[k]) : make_float2(kR.bfr[k], kR.bfi[k]));
  }
  a[0] = cadd(a[0], u0);  // adds u_0 to every convolution output
  dft66_axes<true>(a);
  x[0] = x0;
#pragma unroll
  for (int q = 0; q < RM; ++q) x[kT.gq[q]] = a[q];
}

// Compiler scheduling fence.  The unrolled gather loops issue kLoadChunk global loads, fence, then
// consume them: the loads of a chunk are in flight together (one memory latency per chunk), and the
// compiler can neither hoist all 67 (or 134) loads up front, which would keep every address and
// result live at once, nor serialise each load with its use to save registers.  The fence orders
// generic and global-pointer accesses only (raw buffer loads are not held back by it).
constexpr int kLoadChunk = 8;
__device__ __forceinline__ void sched_fence() { asm volatile("" ::: "memory"); }

// ---- quads: the 4 lanes 4 q .. 4 q + 3 of a wave share one complex row (or one column) ----
// Lane s of a quad holds PFA segment s (samples n with 3 n = s mod 4).  It loads the samples in
// column order c = 4 i + sig(s), sig(s) = 3 s mod 4, so the quad's loads cover 4 adjacent columns;
// register i then holds segment element m = (i + dl(s)) mod 67, dl(s) = 17 sig(s) mod 67 (a cyclic
// rotation, undone by the twiddle W67^(dl j) on the 67-point DFT's output).  The 4-point DFT across
// the segments runs across the quad's lanes through DPP quad permutes, as a radix-2 decimation in
// frequency, so its output is in bit-reversed lane order: afterwards lane k holds the bins
// v = (201 br(k) + 68 j) mod 268 (v = br(k) mod 4, v = j mod 67) in register j, br = [0, 2, 1, 3].
// The Hermitian partner -v of a bin then sits in lane [0, 1, 3, 2][k], register (67 - j) mod 67.
__device__ __forceinline__ int quad_sig(int s) { return (3 * s) & 3; }
__device__ __forceinline__ int quad_delta(int s) { return (17 * quad_sig(s)) % P; }
__device__ __forceinline__ int quad_bin(int k) { return ((k & 1) << 1) | (k >> 1); }  // br(k)

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ float2 dpp2(float2 v) {
  return make_float2(dppf<CTRL>(v.x), dppf<CTRL>(v.y));
}
// quad_perm controls: partner at distance 2 ([2, 3, 0, 1]), at distance 1 ([1, 0, 3, 2]), and the
// Hermitian partner of the bit-reversed layout ([0, 1, 3, 2])
constexpr int kX2 = 0x4E, kX1 = 0xB1, kHerm = 0xB4;

// y = (value of the partner lane) + sg * (own value): one multiply and one add with a DPP operand.
template <int CTRL>
__device__ __forceinline__ float2 quad_bfly(float2 v, float sg) {
  return make_float2(dppf<CTRL>(v.x) + sg * v.x, dppf<CTRL>(v.y) + sg * v.y);
}

// 4-point DFT across the quad for every register, radix 2 in two steps.  Forward (decimation in
// frequency, natural lane order in, bit-reversed out): a = x[s ^ 2] + (+-1) x[s] (minus in lanes 2,
// 3), lane 3 times -i, then y = a[s ^ 1] + (+-1) a[s] (minus in lanes 1, 3).  Inverse (decimation in
// time, bit-reversed in, natural out): the same steps in reverse order with +i.
template <bool INV>
__device__ __forceinline__ void quad_dft4(float2 (&x)[P], int k) {
  const float s2 = (k & 2) ? -1.f : 1.f, s1 = (k & 1) ? -1.f : 1.f;
  const bool l3 = k == 3;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    if (!INV) {
      const float2 a = quad_bfly<kX2>(x[j], s2);
      const float2 b = make_float2(l3 ? a.y : a.x, l3 ? -a.x : a.y);  // lane 3: -i a
      x[j] = quad_bfly<kX1>(b, s1);
    } else {
      const float2 c = quad_bfly<kX1>(x[j], s1);
      const float2 b = make_float2(l3 ? -c.y : c.x, l3 ? c.x : c.y);  // lane 3: +i c
      x[j] = quad_bfly<kX2>(b, s2);
    }
  }
}

// x[j] *= W67^(+-dl j) (W67 = exp(-2 pi i / 67); tw holds W67^m)
template <bool CONJ>
__device__ __forceinline__ void quad_rotate(float2 (&x)[P], const float2* tw, int dl) {
  int m = 0;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const float2 t = tw[m];
    x[j] = cmul(x[j], CONJ ? cconj(t) : t);
    m += dl;
    if (m >= P) m -= P;
    if (j % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
}

// Raw buffer stores: one wave-uniform resource per tensor and a 32-bit byte offset per lane.  A
// store whose offset lies past the resource's size is dropped by the hardware, so the conditional
// stores below need no branch (a divergent branch would make the compiler hoist the quad's DPP reads
// above it and keep them all live).
constexpr uint32_t kDrop = 0xFFFFFFF0u;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void bstore4(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}
__device__ __forceinline__ void bstore1(float v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, off, 0, 0);
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

// Shared per-block tables: W67^m and (row pass) the source column of every padded column.  The
// Rader tables are read straight from global memory: their addresses are uniform, so they arrive
// through scalar loads instead of occupying vector registers.
struct QuadTabs {
  float2 tw[P];
  short csrc[L];
};
__device__ __forceinline__ void load_quad_tabs(QuadTabs& T, int W, int pad, int mode) {
  for (int m = threadIdx.x; m < P; m += blockDim.x) {
    double sn, cs;
    sincospi(-2.0 * (double)m / (double)P, &sn, &cs);
    T.tw[m] = make_float2((float)cs, (float)sn);
  }
  if (W > 0)
    for (int n = threadIdx.x; n < L; n += blockDim.x) T.csrc[n] = (short)pad_map(n, W, pad, mode);
  __syncthreads();
}

// ---- row forward: padded rows 2t, 2t + 1 of a plane as one complex row; half spectrum out ----
// quad index g = plane * 134 + t; S (P, NC, L): column v, row r.
struct RowsArgs {
  const float* x;  // (P, H, W)
  float2* S;
  int64_t nquad;
  int H, W, pad, mode;
  uint32_t s_bytes;  // size of S (< 2^31)
};

__global__ void __launch_bounds__(256) k_pfa_rows_fwd(RowsArgs a) {
  __shared__ QuadTabs T;
  load_quad_tabs(T, a.W, a.pad, a.mode);
  const int k = threadIdx.x & 3;
  const int64_t gq = (int64_t)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
  if (gq >= a.nquad) return;  // whole quads leave together
  const int64_t plane = gq / LQ;
  const int t = (int)(gq - plane * LQ);
  // quads t = 134, 135 transform zero rows and write the padding rows 268..271
  const int ra = t < L / 2 ? pad_map(2 * t, a.H, a.pad, a.mode) : -1;
  const int rb = t < L / 2 ? pad_map(2 * t + 1, a.H, a.pad, a.mode) : -1;
  const float* xa = a.x + (plane * a.H + (ra < 0 ? 0 : ra)) * (int64_t)a.W;
  const float* xb = a.x + (plane * a.H + (rb < 0 ? 0 : rb)) * (int64_t)a.W;
  const int sig = quad_sig(k);
  float2 x[P];
#pragma unroll
  for (int i0 = 0; i0 < P; i0 += kLoadChunk) {
    // a chunk of unconditional loads from clamped (in-range) addresses, then selects: no branches
    float va[kLoadChunk], vb[kLoadChunk];
    int sv[kLoadChunk];
#pragma unroll
    for (int ii = 0; ii < kLoadChunk && i0 + ii < P; ++ii) {
      const int sc = T.csrc[4 * (i0 + ii) + sig];
      const int scc = sc < 0 ? 0 : sc;
      va[ii] = xa[scc];
      vb[ii] = xb[scc];
      sv[ii] = sc;
    }
    sched_fence();
#pragma unroll
    for (int ii = 0; ii < kLoadChunk && i0 + ii < P; ++ii)
      x[i0 + ii] = make_float2((sv[ii] >= 0 && ra >= 0) ? va[ii] : 0.f, (sv[ii] >= 0 && rb >= 0) ? vb[ii] : 0.f);
  }
  sched_fence();
  dft67_reg<false>(x);
  sched_fence();
  quad_rotate<false>(x, T.tw, quad_delta(k));
  sched_fence();
  quad_dft4<false>(x, k);
  sched_fence();
  // two real rows: Ya = (Z[v] + conj Z[-v]) / 2, Yb = (Z[v] - conj Z[-v]) / (2i)
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.S, a.s_bytes);
  const uint32_t base = (uint32_t)((plane * NC * LP + 2 * t) * 8);
  int v = (201 * quad_bin(k)) % L;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const float2 z = x[j], zm = dpp2<kHerm>(x[(P - j) % P]);
    bstore4(make_float4(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y), 0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x)), sr,
            v <= L / 2 ? base + (uint32_t)(v * LP * 8) : kDrop);
    v += 68;
    if (v >= L) v -= L;
    if (j % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
}

// ---- columns: forward transform, x Phi, inverse transform, in place on S ----
// quad index g = plane * NC + column.
struct ColsArgs {
  float2* S;          // (P, NC, LP)
  const float2* phi;  // (Cp, P, NC, 4) quad layout (pfa268_phi_index), 1/(L L) folded in
  int64_t B, C, psf_batch, nquad;
};

// Column quad handled by a thread.  With one table per channel, the quads are walked channel-major
// (the B planes of a channel one after another), and the dispatcher's round-robin over the 8 XCDs
// (workgroup i runs on XCD i % 8) is undone, so the workgroups of one XCD take consecutive runs of
// that order: a channel's 289 KB table is then fetched into an XCD's L2 once for its B planes instead
// of once per plane.
__device__ __forceinline__ int64_t cols_quad(const ColsArgs& a) {
  int64_t blk = blockIdx.x;
  const int64_t nblk = gridDim.x;
  if (a.psf_batch == 1 && nblk % 8 == 0) blk = (blk & 7) * (nblk >> 3) + (blk >> 3);
  const int64_t g = blk * (blockDim.x >> 2) + (threadIdx.x >> 2);
  if (a.psf_batch != 1 || g >= a.nquad) return g;
  const int64_t pl = g / NC;  // plane in channel-major order
  return ((pl % a.B) * a.C + pl / a.B) * NC + (g - pl * NC);
}

__global__ void __launch_bounds__(256) k_pfa_cols(ColsArgs a) {
  __shared__ QuadTabs T;
  load_quad_tabs(T, 0, 0, 0);
  const int k = threadIdx.x & 3;
  const int64_t gq = cols_quad(a);
  if (gq >= a.nquad) return;
  const int64_t plane = gq / NC;
  const int c = (int)(gq - plane * NC);
  const int64_t cp = a.psf_batch == 1 ? plane % a.C : plane;
  float2* col = a.S + gq * (int64_t)LP + quad_sig(k);
  float2 x[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    x[i] = col[4 * i];
    if (i % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
  sched_fence();
  const int dl = quad_delta(k);
  dft67_reg<false>(x);
  sched_fence();
  quad_rotate<false>(x, T.tw, dl);
  sched_fence();
  quad_dft4<false>(x, k);
  // register j of lane k multiplies by Phi at u = 201 br(k) + 68 j, stored at [cp][j][c][k]
  const float2* ph = a.phi + (cp * P * NC + c) * 4 + k;
  sched_fence();
#pragma unroll
  for (int j0 = 0; j0 < P; j0 += kLoadChunk) {
    float2 f[kLoadChunk];
#pragma unroll
    for (int jj = 0; jj < kLoadChunk && j0 + jj < P; ++jj) f[jj] = ph[(j0 + jj) * NC * 4];
    sched_fence();
#pragma unroll
    for (int jj = 0; jj < kLoadChunk && j0 + jj < P; ++jj) x[j0 + jj] = cmul(x[j0 + jj], f[jj]);
  }
  sched_fence();
  quad_dft4<true>(x, k);
  sched_fence();
  int dl2 = dl;
  asm volatile("" : "+v"(dl2));  // recompute the twiddle addresses instead of keeping the first pass's live
  quad_rotate<true>(x, T.tw, dl2);
  sched_fence();
  dft67_reg<true>(x);
  sched_fence();
#pragma unroll
  for (int i = 0; i < P; ++i) {
    col[4 * i] = x[i];
    if (i % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
}

// ---- row inverse: half spectra of rows 2t, 2t + 1 -> complex row -> inverse -> crop + store ----
struct RowsInvArgs {
  const float2* S;   // (P, NC, L)
  float* out;        // (P, H, W)
  int64_t nquad;
  int H, W, pad;
  uint32_t out_bytes;  // size of out (< 2^31)
};

template <bool GELU>
__global__ void __launch_bounds__(256) k_pfa_rows_inv(RowsInvArgs a) {
  __shared__ QuadTabs T;
  load_quad_tabs(T, 0, 0, 0);
  const int k = threadIdx.x & 3;
  const int64_t gq = (int64_t)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
  if (gq >= a.nquad) return;
  const int64_t plane = gq / LQ;
  const int t = (int)(gq - plane * LQ);  // t = 134, 135: padding rows, nothing stored
  const float2* Sp = a.S + plane * (int64_t)NC * LP + 2 * t;
  // Z[v] = Ha[v] + i Hb[v] with H[-v] = conj H[v].  (Each column is read twice by a quad, for v and for
  // -v; pairing the two reads in time cuts the reads from 1.55x to 1.0x the half spectra but made the
  // pass slower: it is latency-bound, and the pairing held more registers live.)
  float2 x[P];
  const int kb = quad_bin(k);
  int v = (201 * kb) % L;
  // v = 0 or L/2 (real bins) only for j = 0 with kb = 0 or 2; kb = 1 starts at v = 201 > L/2
  const float sg0 = (kb & 1) ? (kb == 1 ? -1.f : 1.f) : 0.f;
#pragma unroll
  for (int j0 = 0; j0 < P; j0 += kLoadChunk) {
    float4 h[kLoadChunk];
    float sg[kLoadChunk];
#pragma unroll
    for (int jj = 0; jj < kLoadChunk && j0 + jj < P; ++jj) {
      const bool lo = v <= L / 2;
      h[jj] = *(const float4*)(Sp + (int64_t)(lo ? v : L - v) * LP);
      // imaginary parts: conjugated past L/2, zero at the real bins 0 and L/2
      sg[jj] = j0 + jj == 0 ? sg0 : (lo ? 1.f : -1.f);
      v += 68;
      if (v >= L) v -= L;
    }
    sched_fence();
#pragma unroll
    for (int jj = 0; jj < kLoadChunk && j0 + jj < P; ++jj)
      x[j0 + jj] = make_float2(h[jj].x - sg[jj] * h[jj].w, sg[jj] * h[jj].y + h[jj].z);
  }
  sched_fence();
  quad_dft4<true>(x, k);
  sched_fence();
  quad_rotate<true>(x, T.tw, quad_delta(k));
  sched_fence();
  dft67_reg<true>(x);
  sched_fence();
  const int sig = quad_sig(k);
  const int r0 = t < L / 2 ? 2 * t - a.pad : -1, r1 = t < L / 2 ? r0 + 1 : -1;
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, a.out_bytes);
  const bool wa = r0 >= 0 && r0 < a.H, wb = r1 >= 0 && r1 < a.H;
  const uint32_t ba = (uint32_t)(((plane * a.H + r0) * a.W - a.pad + sig) * 4);
  const uint32_t bb = ba + (uint32_t)(a.W * 4);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int cc = 4 * i + sig - a.pad;
    const bool in = cc >= 0 && cc < a.W;
    float va = x[i].x, vb = x[i].y;
    if (GELU) {
      va = gelu_fast(va);
      vb = gelu_fast(vb);
    }
    bstore1(va, orr, in && wa ? ba + (uint32_t)(16 * i) : kDrop);
    bstore1(vb, orr, in && wb ? bb + (uint32_t)(16 * i) : kDrop);
    if (i % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
}

}  // namespace pfa268

// Host side --------------------------------------------------------------------------------------
namespace {
constexpr int kQuadsPerBlock = 64;  // 256 threads
}  // namespace

bool pfa268_applies(int h, int w, int s) { return h == pfa268::L && w == pfa268::L && s == 1; }

size_t pfa268_scratch_bytes(int64_t P) { return align_up((size_t)P * pfa268::NC * pfa268::LP * sizeof(float2)); }

// S: (P, NC, LP) scratch (pfa268_scratch_bytes); phi: (Cp, NC, L) in the quad layout.
int pfa268_forward(const float* x, int64_t P, int64_t C, int64_t psf_batch, int H, int W, int pad, int mode, int act,
                   const float2* phi, float2* S, float* out, hipStream_t st) {
  using namespace pfa268;
  const int64_t nfq = P * LQ, ncq = P * NC;
  const int64_t ncb = (ncq + kQuadsPerBlock - 1) / kQuadsPerBlock, nfb = (nfq + kQuadsPerBlock - 1) / kQuadsPerBlock;
  if (ncb > 0x7fffffff || nfb > 0x7fffffff) return fail(CVN_ERR_UNSUPPORTED, "too many planes for the 268 path");
  const int64_t s_bytes = P * NC * LP * 8, o_bytes = P * (int64_t)H * W * 4;
  if (s_bytes >= ((int64_t)1 << 31) || o_bytes >= ((int64_t)1 << 31))
    return fail(CVN_ERR_UNSUPPORTED, "the 268 path addresses its buffers with 31-bit byte offsets");
  RowsArgs ra{x, S, nfq, H, W, pad, mode, (uint32_t)s_bytes};
  hipLaunchKernelGGL(k_pfa_rows_fwd, dim3((unsigned)nfb), dim3(4 * kQuadsPerBlock), 0, st, ra);
  int rc = check_launch("268 row pass");
  if (rc != CVN_OK) return rc;
  ColsArgs ca{S, phi, P / C, C, psf_batch, ncq};
  hipLaunchKernelGGL(k_pfa_cols, dim3((unsigned)ncb), dim3(4 * kQuadsPerBlock), 0, st, ca);
  if ((rc = check_launch("268 column pass")) != CVN_OK) return rc;
  RowsInvArgs ia{S, out, nfq, H, W, pad, (uint32_t)o_bytes};
  if (act == CVN_ACT_GELU)
    hipLaunchKernelGGL(k_pfa_rows_inv<true>, dim3((unsigned)nfb), dim3(4 * kQuadsPerBlock), 0, st, ia);
  else
    hipLaunchKernelGGL(k_pfa_rows_inv<false>, dim3((unsigned)nfb), dim3(4 * kQuadsPerBlock), 0, st, ia);
  return check_launch("268 inverse row pass");
}

}  // namespace cvn
