// Converse2D forward for 268 x 268 padded planes (Converse-DnCNN: 256 x 256, padding 6), scale 1.
//
// Same three-pass data flow as the generic path (row transform -> column transform x Phi x inverse
// -> inverse row transform, half spectra column-major in between), but every transform is the
// prime-factor FFT 268 = 4 * 67 (no twiddles) held in the registers of 8 lanes, lane = 8 t + 4 e + s
// of a wave (t: transform, 8 per wave):
//   * s = 0..3 is the PFA segment: sample n = (67 s + 4 m) mod 268 is element m of segment s, and
//     bin v of the transform is bin v mod 4 of the 4-point DFT across the segments (a DPP quad
//     exchange) of bin v mod 67 of the segments' 67-point DFTs;
//   * the 67-point DFT of a segment is split over the lane pair e = 0, 1 by Rader's algorithm
//     (primitive root 2): a_q = y[2^q mod 67], Y[0] = y[0] + sum a, Y[2^-q mod 67] = y[0] + (a (*) b)_q
//     with the cyclic convolution of length 66 done as FFT_66, a product with FFT_66(b) / 66
//     (compile-time constants) and the inverse FFT_66.  FFT_66 = 2 x 33 (Good-Thomas, no twiddles):
//     the length-2 axis runs across the pair (q = 33 e + 34 r mod 66 is slot r of lane e), the
//     length-33 axis in registers as 3 x 11.
// Each lane thus holds 34 complex values (33 Rader slots and the index-0 element in lane e = 0),
// which keeps a thread near 100 registers and lets four waves share a SIMD, against two for a
// 67-value-per-lane layout; two waves per SIMD could not hide one wave's memory phase behind the
// other's arithmetic (a lone wave issues at half the paired rate).
// The gathers into Rader order and the scatters out of it go through LDS in wave-private buffers
// (8 rows or half-columns at a time), so global loads and stores stay coalesced.
// (C. M. Rader, Proc. IEEE 56(6), 1968; I. J. Good, J. R. Stat. Soc. B 20, 1958.)
#include <math.h>

#include <algorithm>

#include "cvn_common.h"

namespace cvn {
namespace pfa268 {

constexpr int L = 268, P = 67, RM = 66, NC = L / 2 + 1;  // NC: half-spectrum bins
// Between the passes a half-spectrum column occupies LP = 272 rows (rows 268..271 are zero padding),
// and the row passes index LQ = 136 row pairs per plane (134 and 2 idle pairs), so that a wave's 8
// row pairs never straddle two planes.
constexpr int LP = 272, LQ = 136;
constexpr int NR = 34;     // complex values per lane
constexpr int kTPW = 8;    // transforms per wave
constexpr int kWaves = 4;  // waves per block (256 threads)

// Index maps, evaluated at compile time.  gp[q] = 2^q, gq[q] = 2^-q (mod 67).  The in-place 33-point
// DFT (3 x 11) leaves output k = outmap[p] in slot p.  Slot p of lane e holds, before the 67-point
// DFT, the segment element min_[e][p] = gp[33 e + 34 p mod 66] and, after it, the transform at
// mout[e][p] = gq[33 e + 34 outmap[p] mod 66]; an inverse DFT's input slot p takes the forward output
// slot inv_src[p] (mout[e][inv_src[p]] = min_[e][p]).
struct Maps {
  int gp[RM], gq[RM], outmap[33], oinv[33], min_[2][33], mout[2][33], inv_src[33];
  constexpr Maps() : gp(), gq(), outmap(), oinv(), min_(), mout(), inv_src() {
    int r = 1, ri = 1;
    for (int q = 0; q < RM; ++q) {
      gp[q] = r;
      gq[q] = ri;
      r = (2 * r) % P;
      ri = (34 * ri) % P;  // 34 = 2^-1 mod 67
    }
    for (int a = 0; a < 3; ++a)
      for (int b = 0; b < 11; ++b) {
        int k = 0;
        while (!(k % 3 == a && k % 11 == b)) ++k;
        outmap[(11 * a + 3 * b) % 33] = k;
      }
    for (int p = 0; p < 33; ++p) oinv[outmap[p]] = p;
    for (int e = 0; e < 2; ++e)
      for (int p = 0; p < 33; ++p) {
        min_[e][p] = gp[(33 * e + 34 * p) % RM];
        mout[e][p] = gq[(33 * e + 34 * outmap[p]) % RM];
      }
    for (int p = 0; p < 33; ++p) inv_src[p] = oinv[(33 - p) % 33];
  }
};
constexpr Maps kM{};

// Rader tables: b_q = W67^(2^-q), bf = FFT66(b) / 66 (forward) and bi = FFT66(conj b) / 66 (inverse),
// natural bin order, evaluated in double at compile time and rounded once.  Their indices are
// compile-time constants in dft67_pair, so the values become instruction literals.
struct RaderTabs {
  float bfr[RM], bfi[RM], bir[RM], bii[RM];
  constexpr RaderTabs() : bfr(), bfi(), bir(), bii() {
    double br[RM] = {}, bim[RM] = {}, wr[RM] = {}, wi[RM] = {};
    int gq = 1;
    for (int q = 0; q < RM; ++q) {
      const CosSin b = cos_sin_turn(gq, P), w = cos_sin_turn(q, RM);
      br[q] = b.c;
      bim[q] = -b.s;  // exp(-2 pi i gq / 67)
      wr[q] = w.c;
      wi[q] = -w.s;  // exp(-2 pi i q / 66)
      gq = (34 * gq) % P;
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

// In-register 33-point DFT (Good-Thomas 3 x 11) in place on y[0..32]: slot p is input index p;
// afterwards slot p holds output outmap[p].
template <bool INV>
__device__ __forceinline__ void dft33(float2 (&y)[NR]) {
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    float2 t[11];
#pragma unroll
    for (int b = 0; b < 11; ++b) t[b] = y[(11 * a + 3 * b) % 33];
    Dft<11, INV>::run(t);
#pragma unroll
    for (int b = 0; b < 11; ++b) y[(11 * a + 3 * b) % 33] = t[b];
  }
#pragma unroll
  for (int b = 0; b < 11; ++b) {
    float2 t[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) t[a] = y[(11 * a + 3 * b) % 33];
    Dft<3, INV>::run(t);
#pragma unroll
    for (int a = 0; a < 3; ++a) y[(11 * a + 3 * b) % 33] = t[a];
  }
}

// The value of lane l ^ 4 (the other half of the Rader pair): row_shl:4 into the lanes with
// l & 4 == 0 (banks 0 and 2 of each row of 16), row_shr:4 into the others.
__device__ __forceinline__ float xor4(float v) {
  const int iv = __builtin_bit_cast(int, v);
  int r = __builtin_amdgcn_mov_dpp(iv, 0x104, 0xF, 0x5, false);  // lanes outside banks 0, 2: set below
  r = __builtin_amdgcn_update_dpp(r, iv, 0x114, 0xF, 0xA, false);
  return __builtin_bit_cast(float, r);
}
__device__ __forceinline__ float2 xor4(float2 v) { return make_float2(xor4(v.x), xor4(v.y)); }
// length-2 DFT across the pair: partner + sg own (sg = +1 in lane e = 0, -1 in lane e = 1)
__device__ __forceinline__ float2 pair_bfly(float2 v, float sg) {
  const float2 w = xor4(v);
  return make_float2(fmaf(sg, v.x, w.x), fmaf(sg, v.y, w.y));
}

// 67-point DFT of one segment held by a lane pair (forward, or inverse without normalisation).
// In: slot p < 33 holds element min_[e][p]; slot 33 holds element 0 in lane e = 0 and 0 in lane 1.
// Out: slot p holds bin mout[e][p]; slot 33 of lane 0 holds bin 0.
template <bool INV>
__device__ __forceinline__ void dft67_pair(float2 (&y)[NR], int e) {
  const float sg = e ? -1.f : 1.f;
  dft33<false>(y);
#pragma unroll
  for (int p = 0; p < 33; ++p) y[p] = pair_bfly(y[p], sg);
  const float2 u0 = y[NR - 1];
  const float2 x0 = cadd(u0, y[0]);  // lane 0, slot 0: bin 0 of FFT_66 = sum of the a's
  // the kernel transform at this lane's FFT_66 bin, b0 + e (b1 - b0) with literal b0, b1 - b0 (a select
  // between the two literals would be turned into a table lookup with spilled indices)
  const float ef = (float)e;
#pragma unroll
  for (int p = 0; p < 33; ++p) {
    const int k0 = (2 * kM.outmap[p]) % RM, k1 = (33 + 2 * kM.outmap[p]) % RM;  // FFT_66 bin of lane 0 / 1
    const float r0 = INV ? kR.bir[k0] : kR.bfr[k0], r1 = INV ? kR.bir[k1] : kR.bfr[k1];
    const float i0 = INV ? kR.bii[k0] : kR.bfi[k0], i1 = INV ? kR.bii[k1] : kR.bfi[k1];
    y[p] = cmul(y[p], make_float2(fmaf(ef, r1 - r0, r0), fmaf(ef, i1 - i0, i0)));
  }
  y[0] = cadd(y[0], u0);  // adds u_0 to every convolution output (u_0 = 0 in lane 1)
#pragma unroll
  for (int p = 0; p < 33; ++p) y[p] = pair_bfly(y[p], sg);
  float2 z[NR];
#pragma unroll
  for (int p = 0; p < 33; ++p) z[p] = y[kM.oinv[p]];  // the inverse FFT_33 takes bin p in slot p
  dft33<true>(z);
#pragma unroll
  for (int p = 0; p < 33; ++p) y[p] = z[p];
  y[NR - 1] = x0;
}

// ---- the 4-point DFT across the segments: DPP quad exchanges ----
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
template <int CTRL>
__device__ __forceinline__ float2 quad_bfly(float2 v, float sg) {
  return make_float2(dppf<CTRL>(v.x) + sg * v.x, dppf<CTRL>(v.y) + sg * v.y);
}
// Radix 2 in two steps.  Forward (decimation in frequency, natural lane order in, bit-reversed out):
// a = x[s ^ 2] + (+-1) x[s] (minus in lanes 2, 3), lane 3 times -i, then y = a[s ^ 1] + (+-1) a[s]
// (minus in lanes 1, 3); afterwards lane k holds bins v = br(k) mod 4, br = [0, 2, 1, 3].  Inverse
// (decimation in time, bit-reversed in, natural out): the same steps in reverse order with +i.
template <bool INV>
__device__ __forceinline__ void quad_dft4(float2 (&x)[NR], int k) {
  const float s2 = (k & 2) ? -1.f : 1.f, s1 = (k & 1) ? -1.f : 1.f;
  const bool l3 = k == 3;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
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
__device__ __forceinline__ int quad_bin(int k) { return ((k & 1) << 1) | (k >> 1); }  // br(k)

// element / bin index of slot p < 33 in lane e (compile-time p): two literals and a select
__device__ __forceinline__ int slot_in(int e, int p) { return e ? kM.min_[1][p] : kM.min_[0][p]; }
__device__ __forceinline__ int slot_out(int e, int p) { return e ? kM.mout[1][p] : kM.mout[0][p]; }
// sample / bin n = 67 s + 4 m (mod 268) of segment s, element m
__device__ __forceinline__ int seg_pos(int s67, int m) {
  const int n = s67 + 4 * m;
  return n >= L ? n - L : n;
}

// Compiler scheduling fence: the load loops issue kChunk global loads, fence, then consume them, so a
// chunk's loads are in flight together while the registers that hold results and addresses stay
// bounded (the compiler would otherwise hoist all 34 loads of a lane).
// opaque() hides a value from the optimiser, so index arithmetic is recomputed in each LDS phase
// instead of being kept live in 34 registers across phases.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
// pin() materialises a value at that point (the compiler would otherwise sink the arithmetic that
// consumes a chunk below the later chunks' loads and keep every loaded value live).
constexpr int kChunk = 8;
__device__ __forceinline__ void sched_fence() { asm volatile("" ::: "memory"); }
__device__ __forceinline__ void pin(float2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); }

// Scheduling wall between the phases of a pass (gather, forward transform, Phi, inverse transform,
// scatter): without it the scheduler overlaps neighbouring phases and their live values exceed the
// 128 registers that four waves per SIMD leave a thread.
__device__ __forceinline__ void phase_wall() { __builtin_amdgcn_sched_barrier(0); }

// LDS written and read back by other lanes of the same wave (wave-private buffers)
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Raw buffer stores: one wave-uniform resource per tensor and a 32-bit byte offset per lane.  A
// store whose offset lies past the resource's size is dropped by the hardware, so the conditional
// stores below need no branch.
constexpr uint32_t kDrop = 0xFFFFFFF0u;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void bstore4(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
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

// ---- row forward: padded rows 2t, 2t + 1 of a plane as one complex row; half spectrum out ----
// transform g = plane * 136 + t (t = 134, 135: zero rows, written to S's padding rows 268..271);
// S (P, NC, LP): column v, row r.
struct RowsArgs {
  const float* x;  // (P, H, W)
  float2* S;
  int64_t ntr;
  int H, W, pad, mode;
  uint32_t s_bytes;  // size of S (< 2^31)
};

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) k_pfa_rows_fwd(RowsArgs a) {
  __shared__ short csrc[L];                // source column of every padded column (-1: zero)
  __shared__ float stg[kWaves][kTPW][L];   // one row of each of the wave's 8 row pairs
  for (int n = threadIdx.x; n < L; n += blockDim.x) csrc[n] = (short)pad_map(n, a.W, a.pad, a.mode);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = lane & 3, e = (lane >> 2) & 1, tt = lane >> 3;
  const int64_t g0 = ((int64_t)blockIdx.x * kWaves + wave) * kTPW;  // the wave's first transform (wave-uniform)
  if (g0 >= a.ntr) return;                                           // whole waves leave together
  const int64_t plane = g0 / LQ;
  const int t0 = (int)(g0 - plane * LQ);
  float (*st)[L] = stg[wave];
  const int s67 = 67 * s;
  float2 y[NR];
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // h = 0: rows 2t (real parts), h = 1: rows 2t + 1 (imaginary parts)
    // stage the 8 source rows (zeros for padding row pairs and zero-padded rows), coalesced; all
    // loads are issued before the first LDS write (clamped in-range addresses, no branch)
    {
      float v[kTPW][5];  // W <= 268 < 5 * 64
#pragma unroll
      for (int i = 0; i < kTPW; ++i) {
        const int t = t0 + i;
        const int r = t < L / 2 ? pad_map(2 * t + h, a.H, a.pad, a.mode) : -1;  // wave-uniform
        const float* src = a.x + (plane * a.H + (r < 0 ? 0 : r)) * (int64_t)a.W;
#pragma unroll
        for (int j = 0; j < 5; ++j) {
          const int c = lane + 64 * j;
          const float val = src[c < a.W ? c : a.W - 1];
          v[i][j] = r < 0 ? 0.f : val;
        }
      }
#pragma unroll
      for (int i = 0; i < kTPW; ++i)
#pragma unroll
        for (int j = 0; j < 5; ++j)
          if (lane + 64 * j < a.W) st[i][lane + 64 * j] = v[i][j];
    }
    wave_lds_sync();
    const int s67h = opaque(s67), eh = opaque(e);
    // in chunks: the chunk's source-column reads, then its value reads (one LDS round trip each)
#pragma unroll
    for (int p0 = 0; p0 < NR; p0 += kChunk) {
      int sc[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk && p0 + i < NR; ++i) {
        const int p = p0 + i;
        sc[i] = csrc[p < 33 ? seg_pos(s67h, slot_in(eh, p)) : s67h];
      }
#pragma unroll
      for (int i = 0; i < kChunk && p0 + i < NR; ++i) {
        const int p = p0 + i;
        const bool zero = sc[i] < 0 || (p == NR - 1 && eh);
        const float v = st[tt][zero ? 0 : sc[i]];
        if (h == 0) y[p].x = zero ? 0.f : v; else y[p].y = zero ? 0.f : v;
      }
    }
    wave_lds_sync();
  }
  dft67_pair<false>(y, e);
  quad_dft4<false>(y, s);
  // two real rows: Ya = (Z[v] + conj Z[-v]) / 2, Yb = (Z[v] - conj Z[-v]) / (2i); the Hermitian
  // partner -v of slot p in lane (k, e) is slot p of lane (br-partner of k, 1 - e) (slot 33: same e)
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.S, a.s_bytes);
  const uint32_t base = (uint32_t)((plane * NC * LP + 2 * (t0 + tt)) * 8);
  const int v1 = (201 * quad_bin(s)) % L;
#pragma unroll
  for (int p = 0; p < NR; ++p) {
    const float2 z = y[p];
    const float2 zq = dpp2<kHerm>(z);
    const float2 zm = p < 33 ? xor4(zq) : zq;
    int v = v1 + 68 * (p < 33 ? slot_out(e, p) : 0);
    v %= L;
    const bool ok = v <= L / 2 && (p < 33 || e == 0);
    bstore4(make_float4(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y), 0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x)), sr,
            ok ? base + (uint32_t)(v * LP * 8) : kDrop);
  }
}

// ---- columns: forward transform, x Phi, inverse transform, in place on S ----
// The column pass keeps one transform per quad of lanes (each lane one PFA segment of 67 values): it
// carries two 268-point transforms and the Phi product, and with eight lanes per transform its
// staging through LDS in half-columns cost it more memory-level parallelism than the extra
// occupancy gave back (measured 0.27 ms against 0.21 ms per cfg4 layer), while for the row passes
// the 8-lane form is the faster one (0.14 / 0.16 ms against 0.18 / 0.22 ms).
namespace quad {
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

// The column pass's load loops issue kLoadChunk global loads, then sched_fence, then consume them:
// the loads of a chunk are in flight together (one memory latency per chunk), and the compiler can
// neither hoist all 67 loads up front, which would keep every address and result live at once, nor
// serialise each load with its use.
constexpr int kLoadChunk = 8;

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
template <bool INV, int J0 = 0, int J1 = P>
__device__ __forceinline__ void quad_dft4(float2 (&x)[P], int k) {
  const float s2 = (k & 2) ? -1.f : 1.f, s1 = (k & 1) ? -1.f : 1.f;
  const bool l3 = k == 3;
#pragma unroll
  for (int j = J0; j < J1; ++j) {
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

// x[j] *= W67^(+-dl j) for J0 <= j < J1 (W67 = exp(-2 pi i / 67); tw holds W67^m)
template <bool CONJ, int J0 = 0, int J1 = P>
__device__ __forceinline__ void quad_rotate(float2 (&x)[P], const float2* tw, int dl) {
  int m = (dl * J0) % P;
#pragma unroll
  for (int j = J0; j < J1; ++j) {
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

// Transfer-table entries through LDS: the quad's four entries of register j (32 contiguous bytes of
// the quad layout) are copied with global_load_lds_dwordx4 into the wave's LDS region, lane k of the
// quad copying the 16 bytes of register J0 + 2 i + (k >> 1) in instruction i, so that quad q's entry
// for register j lands at region[(j - J0) / 2 * 128 + 8 q + 4 ((j - J0) & 1) + lane]; no register holds
// it in flight (a register prefetch does not fit beside the 67 column values).  The first copy
// (registers 0 .. 33) is requested before the column loads and arrives during the forward
// transform; the second (registers 33 .. 66, overlapping the first by one so that every lane of
// every copy instruction is active: a partly masked copy made the compiler spill 105 VGPRs) after
// the first half's products, and arrives during that half's inverse 4-point DFT and rotation.  A
// wave's region is 17 KB, so two blocks of four waves fit in LDS.
constexpr int kPhiHalf = 34;  // registers per copy (even)
template <int J0, int J1>
__device__ __forceinline__ void phi_copy(const float2* ph, float2* region, int k) {
  static_assert((J1 - J0) % 2 == 0, "whole instructions: every lane copies");
#pragma unroll
  for (int i = 0; i < (J1 - J0) / 2; ++i) {
    const int j = J0 + 2 * i + (k >> 1);
    __builtin_amdgcn_global_load_lds((const void*)(ph + (int64_t)j * NC * 4 + 2 * (k & 1)),
                                     (__attribute__((address_space(3))) void*)(region + i * 128), 16, 0, 0);
  }
}
// x[j] *= Phi[j] for J0 <= j < J1, from a region filled by phi_copy<B, ...>
template <int B, int J0, int J1>
__device__ __forceinline__ void phi_product(float2 (&x)[P], const float2* region, int q, int k) {
#pragma unroll
  for (int j = J0; j < J1; ++j) x[j] = cmul(x[j], region[(j - B) / 2 * 128 + 8 * q + 4 * ((j - B) & 1) + k]);
}

__global__ void __launch_bounds__(256) k_pfa_cols(ColsArgs a) {
  __shared__ QuadTabs T;
  __shared__ __align__(16) float2 phs[kWaves][kPhiHalf / 2 * 128];  // per wave: 17 KB
  load_quad_tabs(T, 0, 0, 0);
  const int k = threadIdx.x & 3, q = (threadIdx.x & 63) >> 2;
  const int64_t gq = cols_quad(a);
  if (gq >= a.nquad) return;  // whole quads leave together; each lane copies only its own quad's entries
  const int64_t plane = gq / NC;
  const int c = (int)(gq - plane * NC);
  const int64_t cp = a.psf_batch == 1 ? plane % a.C : plane;
  // register j of lane k multiplies by Phi at u = 201 br(k) + 68 j, stored at [cp][j][c][k]
  const float2* ph = a.phi + (cp * P * NC + c) * 4;
  float2* region = phs[threadIdx.x >> 6];
  phi_copy<0, kPhiHalf>(ph, region, k);
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
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's first table half is in LDS
  phi_product<0, 0, kPhiHalf>(x, region, q, k);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // its reads are done before the region is reused
  phi_copy<P - kPhiHalf, P>(ph, region, k);
  sched_fence();
  int dl2 = dl;
  asm volatile("" : "+v"(dl2));  // recompute the twiddle addresses instead of keeping the first pass's live
  quad_dft4<true, 0, kPhiHalf>(x, k);
  quad_rotate<true, 0, kPhiHalf>(x, T.tw, dl2);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the second half
  phi_product<P - kPhiHalf, kPhiHalf, P>(x, region, q, k);
  sched_fence();
  quad_dft4<true, kPhiHalf, P>(x, k);
  quad_rotate<true, kPhiHalf, P>(x, T.tw, dl2);
  sched_fence();
  dft67_reg<true>(x);
  sched_fence();
#pragma unroll
  for (int i = 0; i < P; ++i) {
    col[4 * i] = x[i];
    if (i % kLoadChunk == kLoadChunk - 1) sched_fence();
  }
}
}  // namespace quad
// ---- row inverse: half spectra of rows 2t, 2t + 1 -> complex row -> inverse -> crop + store ----
struct RowsInvArgs {
  const float2* S;   // (P, NC, LP)
  float* out;        // (P, H, W)
  int64_t ntr;
  int H, W, pad;
};

template <bool GELU>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) k_pfa_rows_inv(RowsInvArgs a) {
  // one padded row (268 columns and 4 spare entries for lane e = 1's unused slot 33) of each of the
  // wave's 8 row pairs: every slot writes without a branch
  __shared__ float stg[kWaves][kTPW][LP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = lane & 3, e = (lane >> 2) & 1, tt = lane >> 3;
  const int64_t g0 = ((int64_t)blockIdx.x * kWaves + wave) * kTPW;
  if (g0 >= a.ntr) return;  // whole waves leave together
  const int64_t plane = g0 / LQ;
  const int t0 = (int)(g0 - plane * LQ), t = t0 + tt;
  const float2* Sp = a.S + plane * (int64_t)NC * LP + 2 * t;
  // Z[v] = Ha[v] + i Hb[v] with H[-v] = conj H[v]; slot p of lane (k, e) loads the bin whose index
  // mod 67 is min_[e][p] (the inverse 67-point DFT's input order), mod 4 br(k)
  const int v1 = (201 * quad_bin(s)) % L;
  float2 y[NR];
#pragma unroll
  for (int p0 = 0; p0 < NR; p0 += kChunk) {
    float4 hv[kChunk];
    float sg[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk && p0 + i < NR; ++i) {
      const int p = p0 + i;
      int v = v1 + 68 * (p < 33 ? slot_in(e, p) : 0);
      v %= L;
      const bool lo = v <= L / 2;
      hv[i] = *(const float4*)(Sp + (int64_t)(lo ? v : L - v) * LP);
      // imaginary parts: conjugated past L/2, zero at the real bins 0 and L/2 (no branch)
      sg[i] = (float)((v != 0) & (v != L / 2)) * (lo ? 1.f : -1.f);
    }
    sched_fence();
#pragma unroll
    for (int i = 0; i < kChunk && p0 + i < NR; ++i) {
      y[p0 + i] = make_float2(hv[i].x - sg[i] * hv[i].w, sg[i] * hv[i].y + hv[i].z);
      pin(y[p0 + i]);
    }
  }
  sched_fence();
  if (e) y[NR - 1] = make_float2(0.f, 0.f);
  phase_wall();
  quad_dft4<true>(y, s);
  dft67_pair<true>(y, e);
  phase_wall();
  // slot p now holds sample mout[e][p] of segment s: padded column 67 s + 4 mout (mod 268)
  float (*st)[LP] = stg[wave];
  const int s67 = 67 * s;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // h = 0: row 2t (real parts), h = 1: row 2t + 1 (imaginary parts)
    const int s67h = opaque(s67), eh = opaque(e);
#pragma unroll
    for (int p = 0; p < NR; ++p) {
      const int n = p < 33 ? seg_pos(s67h, slot_out(eh, p)) : (eh ? L + s : s67h);
      const float v = h ? y[p].y : y[p].x;
      st[tt][n] = GELU ? gelu_fast(v) : v;
    }
    wave_lds_sync();
    for (int i = 0; i < kTPW; ++i) {
      const int r = 2 * (t0 + i) + h - a.pad;  // wave-uniform
      if (t0 + i < L / 2 && r >= 0 && r < a.H) {
        float* dst = a.out + (plane * a.H + r) * (int64_t)a.W;
        for (int c = lane; c < a.W; c += 64) dst[c] = st[i][c + a.pad];
      }
    }
    wave_lds_sync();
  }
}

}  // namespace pfa268

// Host side --------------------------------------------------------------------------------------
namespace {
constexpr int kThreads268 = 64 * pfa268::kWaves;
constexpr int kTrPerBlock = pfa268::kWaves * pfa268::kTPW;
constexpr int kQuadsPerBlock = 64;  // column pass: 256 threads, one transform per quad
}  // namespace

bool pfa268_applies(int h, int w, int s) { return h == pfa268::L && w == pfa268::L && s == 1; }

size_t pfa268_scratch_bytes(int64_t P) { return align_up((size_t)P * pfa268::NC * pfa268::LP * sizeof(float2)); }

// S: (P, NC, LP) scratch (pfa268_scratch_bytes); phi: (Cp, 67, NC, 4) (pfa268_phi_index).
int pfa268_forward(const float* x, int64_t P, int64_t C, int64_t psf_batch, int H, int W, int pad, int mode, int act,
                   const float2* phi, float2* S, float* out, hipStream_t st) {
  using namespace pfa268;
  // the column pass copies table entries with 16-byte direct-to-LDS loads
  if ((uintptr_t)phi & 15) return fail(CVN_ERR_ARG, "the 268 path needs a 16-byte aligned transfer table");
  const int64_t nft = P * LQ, nct = P * NC;
  const int64_t nfb = (nft + kTrPerBlock - 1) / kTrPerBlock;
  if (nfb > 0x7fffffff) return fail(CVN_ERR_UNSUPPORTED, "too many planes for the 268 path");
  const int64_t s_bytes = P * NC * LP * 8;
  if (s_bytes >= ((int64_t)1 << 31)) return fail(CVN_ERR_UNSUPPORTED, "the 268 path addresses S with 31-bit byte offsets");
  RowsArgs ra{x, S, nft, H, W, pad, mode, (uint32_t)s_bytes};
  hipLaunchKernelGGL(k_pfa_rows_fwd, dim3((unsigned)nfb), dim3(kThreads268), 0, st, ra);
  int rc = check_launch("268 row pass");
  if (rc != CVN_OK) return rc;
  const int64_t ncq = (nct + kQuadsPerBlock - 1) / kQuadsPerBlock;
  quad::ColsArgs ca{S, phi, P / C, C, psf_batch, nct};
  hipLaunchKernelGGL(quad::k_pfa_cols, dim3((unsigned)ncq), dim3(4 * kQuadsPerBlock), 0, st, ca);
  if ((rc = check_launch("268 column pass")) != CVN_OK) return rc;
  RowsInvArgs ia{S, out, nft, H, W, pad};
  if (act == CVN_ACT_GELU)
    hipLaunchKernelGGL(k_pfa_rows_inv<true>, dim3((unsigned)nfb), dim3(kThreads268), 0, st, ia);
  else
    hipLaunchKernelGGL(k_pfa_rows_inv<false>, dim3((unsigned)nfb), dim3(kThreads268), 0, st, ia);
  return check_launch("268 inverse row pass");
}

}  // namespace cvn
