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
#include <stddef.h>

#include "cvn_common.h"

namespace cvn {

constexpr int kFT = 1024;  // threads per fused workgroup
typedef unsigned int v4u32_t __attribute__((ext_vector_type(4)));

// Workgroup barrier that orders LDS traffic only: global loads and stores issued before it stay in
// flight (every value a thread loads from global memory is consumed by that same thread, so no
// cross-wave ordering of global memory is needed inside the kernel).
// Raw buffer access: one SGPR resource per array, a per-lane VGPR byte offset and a wave-uniform
// SGPR byte offset, so unrolled loops need no per-iteration 64-bit address registers.  Accesses
// past num_records return zero (loads) or are dropped (stores).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float bload1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ float2 bload2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
// Output rows are written once and never read back by the kernel: stored non-temporal (cache policy
// bit NT), so they stream through L2 instead of evicting the transfer tables and the input rows that
// the other planes on the XCD are still reading (measured at cfg3: 0.238 -> 0.218 ms per call).
constexpr int kCpolNT = 2;
__device__ __forceinline__ void bstore4(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, v), r, voff, soff, kCpolNT);
}
// Rows whose byte length is not a multiple of the 128-B line (W % 32 != 0) make partial-line
// writes, which are merged in L2 with ordinary stores and not with streaming ones; so are single words.
__device__ __forceinline__ void bstore4c(float4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, v), r, voff, soff, 0);
}
__device__ __forceinline__ void bstore1(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, voff, soff, 0);
}

__device__ __forceinline__ void lds_barrier() {
  // the "memory" clobber keeps the compiler from moving LDS accesses across the barrier
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int mod_inv(int a, int m) {
  if (m <= 1) return 0;
  for (int x = 1; x < m; ++x)
    if ((a * x) % m == 1) return x;
  return 0;
}

template <int M_, int R1_, int R2_, int R3_, int Q1_, int Q2_, int RSX_ = 0>
struct FusedPlan {
  static constexpr int M = M_, R1 = R1_, R2 = R2_, R3 = R3_;
  static constexpr int Q1 = Q1_, Q2 = Q2_, NH = 2 * Q1_ * Q2_, N = 2 * NH;
  static constexpr int RS = M + 2 + RSX_;  // row-pair stride (M/2 + 1 bins per row, two rows, RSX_ spare)
  static constexpr int NP = NH / 2;       // row pairs per group
  static constexpr int SLOTS = NP * RS;   // complex slots per group
  static constexpr int NQ = M / 2 + 1;    // half-spectrum columns
  static constexpr int ST1 = R2 * R3, ST2 = R3;  // row-axis strides (positions)
  static constexpr int CS1 = 2 * Q2, CS2 = 2;    // column-axis strides (row positions)
  static constexpr int PARK = (SLOTS + kFT - 1) / kFT;  // rounds of kFT slots parked per thread
  static constexpr int SLOTS_PAD = PARK * kFT;           // group buffer padded to whole rounds
  // the first PARK_LDS rounds are parked in the LDS space left over next to the group buffer
  // LDS tables: radix-2 twiddles by row position (NH + 2 float2), int16 pa, pb, pos, a byte per
  // row-pair position saying whether it holds the odd row's bins (these four are compile-time
  // constants, copied from FusedTabs as one 16-byte-padded block of CONST_BYTES), then int16 colsrc
  static constexpr bool kCT = false;  // prime-factor passes, no twiddles
  static constexpr int TWN = 1;        // row twiddle entries (none used)
  static constexpr int TAB_TW_OFF = ((NH + 2) * 8 + (2 * NQ + M) * 2 + RS + 3) / 4 * 4;
  static constexpr int CONST_BYTES = (TAB_TW_OFF + 8 * TWN + 16) / 16 * 16;
  static constexpr int TAB_BYTES = CONST_BYTES + 2 * M;
  static constexpr int PARK_LDS_MAX = (163840 - SLOTS_PAD * 8 - TAB_BYTES - 64) / (kFT * 8);
  static constexpr int PARK_LDS = PARK_LDS_MAX < PARK ? PARK_LDS_MAX : PARK;
  static_assert(R1 * R2 * R3 == M && M % 2 == 0 && NP % 2 == 1, "plan");
  // LDS: group slots, parked rounds, int16 tables pa, pb (NQ each), pos (M), colsrc (M)
  static constexpr size_t LDS_BYTES = (size_t)SLOTS_PAD * 8 + (size_t)PARK_LDS * kFT * 8 + TAB_BYTES;

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
  // plane row of row position rp of group G (the inverse of rpos_in)
  static __host__ __device__ constexpr int plane_row(int rp, int G) {
    return 2 * (((rp / CS1) * (NH / Q1) + ((rp % CS1) >> 1) * (NH / Q2) + (rp & 1) * (NH / 2)) % NH) + G;
  }
};

// Cooley-Tukey plan for square planes of side M = A B (a power of two here: 256 = 16 x 16).
// Rows: sample n = B n1 + n2 sits at position A n2 + n1; pass A (contiguous) takes the A-point DFT
// over n1 and multiplies output k1 by W_M^(n2 k1); pass B (stride A) takes the B-point DFT over n2,
// which leaves frequency v at position v.  Columns of a group (NH = M / 2 rows, row pairs of group
// rows t and t + NP): the radix-2 step across the pair (k1), W_NH^(t k1), then NP = Q1 Q2 points over
// the row pairs t = t2 + Q2 m as Q1-point DFTs over m with W_NP^(t2 k') (column pass A) and Q2-point
// DFTs over t2 (column pass B), which leave frequency k = 2 (k' + Q1 k'') + k1 at row pair
// Q2 k' + k'' (Q1 = Q2).  The inverse runs the same steps backwards with conjugate twiddles.
template <int A_, int B_, int Q_, int RSX_>
struct CtPlan {
  static constexpr bool kCT = true;
  static constexpr int A = A_, B = B_, M = A_ * B_, N = M;
  static constexpr int NH = N / 2, NP = NH / 2, Q1 = Q_, Q2 = Q_;
  static constexpr int RS = M + 2 + RSX_;
  static constexpr int SLOTS = NP * RS;
  static constexpr int NQ = M / 2 + 1;
  static constexpr int PARK = (SLOTS + kFT - 1) / kFT;
  static constexpr int SLOTS_PAD = PARK * kFT;
  static constexpr int TWN = M;  // row twiddles W_M^j, j < M (the column twiddles are W_M^(2j), W_M^(4j))
  static constexpr int TAB_TW_OFF = ((NH + 2) * 8 + (2 * NQ + M) * 2 + RS + 3) / 4 * 4;
  static constexpr int CONST_BYTES = (TAB_TW_OFF + 8 * TWN + 16) / 16 * 16;
  static constexpr int TAB_BYTES = CONST_BYTES + 2 * M;
  static constexpr int PARK_LDS_MAX = (163840 - SLOTS_PAD * 8 - TAB_BYTES - 64) / (kFT * 8);
  static constexpr int PARK_LDS = PARK_LDS_MAX < PARK ? PARK_LDS_MAX : PARK;
  static_assert(NP == Q1 * Q2 && M % 4 == 0 && (RS & 1) == 1 && 4 * (Q1 - 1) * (Q2 - 1) < M, "plan");
  static constexpr size_t LDS_BYTES = (size_t)SLOTS_PAD * 8 + (size_t)PARK_LDS * kFT * 8 + TAB_BYTES;
  static __host__ __device__ constexpr int pos_in(int n) { return A * (n % B) + n / B; }
  static __host__ __device__ constexpr int fpos(int v) { return v; }
  static __host__ __device__ constexpr int pa(int q) { return fpos(q); }
  static __host__ __device__ constexpr int pb(int q) { return q == 0 ? M : (q == M / 2 ? M + 1 : fpos(M - q)); }
  static __host__ __device__ constexpr int rfpos(int k) {
    return 2 * (Q2 * ((k >> 1) % Q1) + (k >> 1) / Q1) + (k & 1);
  }
  static __host__ __device__ constexpr int plane_row(int rp, int G) { return 2 * ((rp >> 1) + NP * (rp & 1)) + G; }
};

// The fused kernel's plane-independent LDS tables, evaluated at compile time (twiddles in double,
// rounded once) and copied into LDS by each workgroup: radix-2 twiddles exp(-2 pi i k / N) at row
// position rfpos(k) (two zero entries past NH for the padding slots), the half-spectrum slot
// positions pa, pb, the in-row positions pos_in, and the odd-row flag per row-pair position.
template <class P>
struct alignas(16) FusedTabs {
  float w[2 * (P::NH + 2)];
  short pa[P::NQ], pb[P::NQ], pos[P::M];
  unsigned char isb[P::RS];
  float tw[2 * P::TWN];  // Cooley-Tukey plans: W_M^j (at byte offset P::TAB_TW_OFF)
  unsigned char pad[P::CONST_BYTES - P::TAB_TW_OFF - 8 * P::TWN];
  constexpr FusedTabs() : w(), pa(), pb(), pos(), isb(), tw(), pad() {
    if constexpr (P::kCT) {
      for (int j = 0; j < P::TWN; ++j) {
        const CosSin cs = cos_sin_turn(j, P::M);
        tw[2 * j] = (float)cs.c;
        tw[2 * j + 1] = (float)-cs.s;
      }
    }
    for (int k = 0; k < P::NH; ++k) {
      const CosSin cs = cos_sin_turn(k, P::N);
      w[2 * P::rfpos(k)] = (float)cs.c;
      w[2 * P::rfpos(k) + 1] = (float)-cs.s;
    }
    for (int q = 0; q < P::NQ; ++q) {
      pa[q] = (short)P::pa(q);
      pb[q] = (short)P::pb(q);
      isb[P::pb(q)] = 1;
    }
    for (int j = 0; j < P::M; ++j) pos[j] = (short)P::pos_in(j);
  }
};
template <class P>
__device__ const FusedTabs<P> kFusedTabs = FusedTabs<P>();
template <class P>
constexpr bool tabs_layout_ok() {
  return sizeof(FusedTabs<P>) == (size_t)P::CONST_BYTES && offsetof(FusedTabs<P>, tw) == (size_t)P::TAB_TW_OFF &&
         offsetof(FusedTabs<P>, pa) == (size_t)(P::NH + 2) * 8;
}

// LDS address of the Cooley-Tukey twiddle table W_M^j: after the group buffer, the parked rounds and
// the table block's first TAB_TW_OFF bytes (the layout k_converse2d_fused sets up).
template <class P>
__device__ __forceinline__ const float2* ct_tw(const float2* buf) {
  return (const float2*)((const char*)buf + (size_t)P::SLOTS_PAD * 8 + (size_t)P::PARK_LDS * kFT * 8 + P::TAB_TW_OFF);
}

// Work item w of a row pass -> (row pair t, index i < PER within the row pair).  Row pairs run fastest
// across the lanes of a wave: with the odd row-pair stride RS, the 64 row pairs of a wave then fall on
// every LDS bank (32 banks of 8 bytes for 64-bit accesses) exactly twice.  Whole blocks of 64 row
// pairs come first, each wave taking one index i of one block; the NP mod 64 remaining row pairs
// come last, row pair fastest.  (A plain i = w / NP, t = w mod NP lets a wave straddle the wrap from
// row pair NP - 1 to row pair 0, which puts three lanes on some banks.)
template <class P, int PER>
__device__ __forceinline__ void row_item(int w, int& t, int& i) {
  constexpr int T0 = P::NP / 64 * 64, RT = P::NP - T0;
  if (RT == 0 || (T0 > 0 && w < T0 * PER)) {
    const int blk = (w >> 6) / PER;
    i = (w >> 6) - blk * PER;
    t = 64 * blk + (w & 63);
  } else {
    const int v = w - T0 * PER;
    i = v / (RT > 0 ? RT : 1);
    t = T0 + (v - i * RT);
  }
}

// u[m] *= W_M^(i m) (conjugated for the inverse), the table read in two halves behind compiler fences
// so that at most half of the twiddles are held in registers at a time.
template <int A, bool INV>
__device__ __forceinline__ void ct_row_tw(float2 (&u)[A], const float2* tw, int i) {
  if (!INV) asm volatile("" ::: "memory");
#pragma unroll
  for (int m = 1; m < A / 2; ++m) u[m] = cmul(u[m], INV ? cconj(tw[i * m]) : tw[i * m]);
#pragma unroll
  for (int m = A / 2; m < A; ++m) u[m] = cmul(u[m], INV ? cconj(tw[i * m]) : tw[i * m]);
}

// Row pass A: radix R3 along the contiguous axis (positions base + m, m < R3).  Cooley-Tukey plans:
// the A-point DFT over positions A i + m with the twiddle W_M^(i m) on its outputs (forward) or
// inputs (inverse); i is wave-uniform (whole blocks of 64 row pairs), so the twiddle reads broadcast.
template <class P, bool INV>
__device__ __forceinline__ void row_pass_a(float2* buf, int tid) {
  if constexpr (P::kCT) {
    constexpr int A = P::A, PER = P::B;
    const float2* tw = ct_tw<P>(buf);
#pragma unroll 1
    for (int w = tid; w < P::NP * PER; w += kFT) {
      int t, i;
      row_item<P, PER>(w, t, i);
      float2* b = buf + t * P::RS + i * A;
      float2 u[A];
#pragma unroll
      for (int m = 0; m < A; ++m) u[m] = b[m];
      if (INV) ct_row_tw<A, true>(u, tw, i);
      Dft<A, INV>::run(u);
      if (!INV) ct_row_tw<A, false>(u, tw, i);
#pragma unroll
      for (int m = 0; m < A; ++m) b[m] = u[m];
    }
  } else {
    constexpr int R = P::R3, PER = P::M / R;
#pragma unroll 1
    for (int w = tid; w < P::NP * PER; w += kFT) {
      int t, i;
      row_item<P, PER>(w, t, i);
      dft_odd_mem<R, 1, INV>(buf + t * P::RS + i * R);
    }
  }
}

// Row pass B: the R1 x R2 prime-factor sub-grid (strides ST1, ST2) in registers, base = n3.
template <class P, bool INV>
__device__ __forceinline__ void row_pass_b(float2* buf, int tid) {
  if constexpr (P::kCT) {  // the B-point DFT over positions A m + k1, m < B
    constexpr int A = P::A, B = P::B;
#pragma unroll 1
    for (int w = tid; w < P::NP * A; w += kFT) {
      int t, k1;
      row_item<P, A>(w, t, k1);
      float2* b = buf + t * P::RS + k1;
      float2 u[B];
#pragma unroll
      for (int m = 0; m < B; ++m) u[m] = b[m * A];
      Dft<B, INV>::run(u);
#pragma unroll
      for (int m = 0; m < B; ++m) b[m * A] = u[m];
    }
    return;
  } else {
  constexpr int R1 = P::R1, R2 = P::R2, PER = P::R3;
#pragma unroll 1
  for (int w = tid; w < P::NP * PER; w += kFT) {
    int t, n3;
    row_item<P, PER>(w, t, n3);
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
}

// Column pass A (forward): Hermitian unpack of the row pairs, the radix-2 pair axis and the
// radix-Q1 axis (row-pair stride Q2) in registers.  Work item (q, g2); q = 0 also carries the
// Nyquist column M/2.
// Cooley-Tukey plans: twiddles of column pass A.  The odd pair output of row pair t = g2 + Q2 m takes
// W_NH^t = W_NH^g2 W_16^m (NH = 16 Q2) before the Q1-point DFT over m, and output k of both takes
// W_NP^(g2 k) after it.  The W_16^m are compile-time constants (tw1); the common factor W_NH^g2 commutes
// with the DFT and is folded into the odd output's table twiddle W_M^(2 g2 (1 + 2 k)) (tw2, whose even
// output twiddle is W_M^(4 g2 k)); the table reads come after a compiler fence, so they are not hoisted
// over the DFT and held in registers.
template <bool INV, int Q>
__device__ __forceinline__ void ct_col_tw1(float2 (&u)[Q]) {
  static_assert(Q == 8, "W_16 constants for an 8-point column pass");
  u[1] = tw16<INV, 1>(u[1]);
  u[2] = tw16<INV, 2>(u[2]);
  u[3] = tw16<INV, 3>(u[3]);
  u[4] = tw16<INV, 4>(u[4]);
  u[5] = tw16<INV, 5>(u[5]);
  u[6] = tw16<INV, 6>(u[6]);
  u[7] = tw16<INV, 7>(u[7]);
}
template <class P, bool INV>
__device__ __forceinline__ void ct_col_tw2(float2 (&u0)[P::Q1], float2 (&u1)[P::Q1], const float2* tw, int g2) {
  static_assert(P::NH == 16 * P::Q2 && P::M == 2 * P::NH && P::M == 4 * P::NP, "twiddle indices");
  asm volatile("" ::: "memory");
#pragma unroll
  for (int k = 0; k < P::Q1; ++k) {
    if (k > 0) {
      const float2 w0 = tw[4 * g2 * k];
      u0[k] = cmul(u0[k], INV ? cconj(w0) : w0);
    }
    const float2 w1 = tw[2 * g2 * (1 + 2 * k)];
    u1[k] = cmul(u1[k], INV ? cconj(w1) : w1);
  }
}

template <class P>
__device__ __forceinline__ void col_pass_a_fwd(float2* buf, const short* pa, const short* pb, int tid) {
  constexpr int Q1 = P::Q1, HQ = P::M / 2;
  const float2* tw = P::kCT ? ct_tw<P>(buf) : nullptr;
#pragma unroll 1
  for (int w = tid; w < HQ * P::Q2; w += kFT) {
    // row-pair group fastest across lanes: spreads the lanes of a wave over LDS banks
    const int q = w / P::Q2, g2 = w - q * P::Q2;
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
      if constexpr (P::kCT) ct_col_tw1<false>(u1);
      Dft<Q1, false>::run(u0);
      Dft<Q1, false>::run(u1);
      if constexpr (P::kCT) ct_col_tw2<P, false>(u0, u1, tw, g2);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        b[m * P::Q2 * P::RS + sa] = u0[m];
        b[m * P::Q2 * P::RS + sb] = u1[m];
      }
    } else {
      // DC (slots 0 / M) and Nyquist (slots pa[M/2] / M + 1) columns, one after the other
#pragma unroll 1
      for (int half = 0; half < 2; ++half) {
        const int src = half ? pa[HQ] : 0;
        const int da = half ? pa[HQ] : 0, db = half ? P::M + 1 : P::M;
        float2 d0[Q1], d1[Q1];
#pragma unroll
        for (int m = 0; m < Q1; ++m) {
          const float2 z = b[m * P::Q2 * P::RS + src];
          d0[m] = make_float2(z.x + z.y, 0.f);
          d1[m] = make_float2(z.x - z.y, 0.f);
        }
        if constexpr (P::kCT) ct_col_tw1<false>(d1);
        Dft<Q1, false>::run(d0);
        Dft<Q1, false>::run(d1);
        if constexpr (P::kCT) ct_col_tw2<P, false>(d0, d1, tw, g2);
#pragma unroll
        for (int m = 0; m < Q1; ++m) {
          float2* r = b + m * P::Q2 * P::RS;
          r[da] = d0[m];
          r[db] = d1[m];
        }
      }
    }
  }
}

// Column pass A (inverse): radix-Q1, inverse radix-2 pair axis, repack into complex row pairs.
template <class P>
__device__ __forceinline__ void col_pass_a_inv(float2* buf, const short* pa, const short* pb, int tid) {
  constexpr int Q1 = P::Q1, HQ = P::M / 2;
  const float2* tw = P::kCT ? ct_tw<P>(buf) : nullptr;
#pragma unroll 1
  for (int w = tid; w < HQ * P::Q2; w += kFT) {
    // row-pair group fastest across lanes: spreads the lanes of a wave over LDS banks
    const int q = w / P::Q2, g2 = w - q * P::Q2;
    float2* b = buf + g2 * P::RS;
    if (q != 0) {
      const int sa = pa[q], sb = pb[q];
      float2 u0[Q1], u1[Q1];
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        u0[m] = b[m * P::Q2 * P::RS + sa];
        u1[m] = b[m * P::Q2 * P::RS + sb];
      }
      if constexpr (P::kCT) ct_col_tw2<P, true>(u0, u1, tw, g2);
      Dft<Q1, true>::run(u0);
      Dft<Q1, true>::run(u1);
      if constexpr (P::kCT) ct_col_tw1<true>(u1);
#pragma unroll
      for (int m = 0; m < Q1; ++m) {
        const float2 A = cadd(u0[m], u1[m]), B = csub(u0[m], u1[m]);
        b[m * P::Q2 * P::RS + sa] = make_float2(A.x - B.y, A.y + B.x);  // A + iB
        b[m * P::Q2 * P::RS + sb] = make_float2(A.x + B.y, B.x - A.y);  // conj(A) + i conj(B)
      }
    } else {
      // DC (slots 0 / M -> 0) and Nyquist (slots pa[M/2] / M + 1 -> pa[M/2]) columns in turn
#pragma unroll 1
      for (int half = 0; half < 2; ++half) {
        const int sa = half ? pa[HQ] : 0, sb = half ? P::M + 1 : P::M;
        float2 d0[Q1], d1[Q1];
#pragma unroll
        for (int m = 0; m < Q1; ++m) {
          const float2* r = b + m * P::Q2 * P::RS;
          d0[m] = r[sa];
          d1[m] = r[sb];
        }
        if constexpr (P::kCT) ct_col_tw2<P, true>(d0, d1, tw, g2);
        Dft<Q1, true>::run(d0);
        Dft<Q1, true>::run(d1);
        if constexpr (P::kCT) ct_col_tw1<true>(d1);
#pragma unroll
        for (int m = 0; m < Q1; ++m) b[m * P::Q2 * P::RS + sa] = make_float2(d0[m].x + d1[m].x, d0[m].x - d1[m].x);
      }
    }
  }
}

// Column pass B: radix Q2 along row pairs (stride 1 row pair); work item (q, g1, g3), q fastest.
template <class P, bool INV>
__device__ __forceinline__ void col_pass_b(float2* buf, const short* pa, const short* pb, int tid) {
  // The half-spectrum columns sit at positions pa[q] and pb[q], which together cover every
  // position 0 .. M + 1 of a row pair exactly once, so the work items run over positions:
  // neighbouring lanes then touch neighbouring LDS words (no bank conflicts, no table lookups).
  constexpr int Q = P::Q2, NPOS = P::M + 2;
#pragma unroll 1
  for (int w = tid; w < NPOS * P::Q1; w += kFT) {
    const int g1 = w / NPOS, p = w - g1 * NPOS;
    if constexpr (P::kCT) {
      float2* b = buf + g1 * P::Q2 * P::RS + p;
      float2 u[Q];
#pragma unroll
      for (int m = 0; m < Q; ++m) u[m] = b[m * P::RS];
      Dft<Q, INV>::run(u);
#pragma unroll
      for (int m = 0; m < Q; ++m) b[m * P::RS] = u[m];
    } else {
      dft_odd_mem<Q, P::RS, INV>(buf + g1 * P::Q2 * P::RS + p);
    }
  }
}

struct FusedArgs {
  const float* x;        // (P, H, W)
  const float4* tab4;    // (Cp, SLOTS): (Phi at row frequency k, Phi at k + N/2)
  float* out;            // (P, H, W)
  int64_t B, C, psf_batch;
  int H, W, pad, mode, act;
};

// Plane handled by workgroup `blk`.  With one table per channel (psf_batch 1), planes are taken
// channel-major, and the dispatcher's round-robin over the 8 XCDs (workgroup i runs on XCD i % 8)
// is undone, so each XCD walks a contiguous run of channels: the planes that run together on one
// XCD share a few transfer tables, which then stay in that XCD's L2.
__device__ __forceinline__ int64_t fused_plane(int64_t blk, const FusedArgs& a) {
  if (a.psf_batch != 1) return blk;
  const int64_t P = a.B * a.C;
  const int64_t k = (P % 8 == 0) ? (blk & 7) * (P >> 3) + (blk >> 3) : blk;
  return (k % a.B) * a.C + k / a.B;
}

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

__device__ __forceinline__ float fgelu(float v) { return gelu_fast(v); }

// Rows of one group as float4 loads: wave w takes row positions w, w + 16, ...; lane l the source
// columns 4 l .. 4 l + 3.  RPW = rows per wave (rounded up).
template <class P>
struct RowIO {
  static constexpr int NW = kFT / 64;
  static constexpr int RPW = (P::NH + NW - 1) / NW;
};

// plane row of row position rp of group G (scalar: rp is wave-uniform)
template <class P>
__device__ __forceinline__ int plane_row(int rp, int G) {
  return P::plane_row(rp, G);
}

// Rows wider than the 256 columns the 64 lanes' float4 loads cover (the 260-point plan with no
// padding to apply: the operator path on an already padded plane).  The tail elements of a group --
// row position tr = tid / 4, column 256 + tid % 4 -- take one word per thread, loaded with the group's
// rows and deposited and stored beside them.
template <class P>
struct RowTail {
  static constexpr int TW = P::M > 256 ? P::M - 256 : 0;  // at most 4 for the 260 plan
  static constexpr bool kAny = TW > 0;
};
template <class P, bool WIDE>
__device__ __forceinline__ bool tail_item(const FusedArgs& a, int tid, int& tr, int& tc) {
  if (!WIDE || !RowTail<P>::kAny || a.W <= 256) return false;
  tr = tid >> 2;
  tc = 256 + (tid & 3);
  return tr < P::NH && tc < a.W;
}
template <class P, bool WIDE>
__device__ __forceinline__ float tail_load(__amdgpu_buffer_rsrc_t xr, const FusedArgs& a, int G, int tid) {
  int tr, tc;
  float t = 0.f;
  if (tail_item<P, WIDE>(a, tid, tr, tc)) {
    const int sr = fpad_src(plane_row<P>(tr, G), a.H, a.pad, a.mode);
    if (sr >= 0) t = bload1(xr, 4u * (uint32_t)tc, (uint32_t)(sr * a.W) * 4u);
  }
  return t;
}
template <class P>
__device__ __forceinline__ float* tail_slot(float* fb, const FusedArgs& a, int tr, int tc) {
  return fb + 2 * ((tr >> 1) * P::RS + P::pos_in(a.pad + tc)) + (tr & 1);
}

template <class P, int I0 = 0, int I1 = RowIO<P>::RPW>
__device__ __forceinline__ void group_prefetch(float4 (&v)[RowIO<P>::RPW], __amdgpu_buffer_rsrc_t xr, const FusedArgs& a,
                                               int G, int wave, int lane) {
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (rp < P::NH) {
      const int sr = fpad_src(plane_row<P>(rp, G), a.H, a.pad, a.mode);
      if (sr >= 0) v[i] = bload4(xr, 16u * lane, (uint32_t)(sr * a.W) * 4u);
    }
  }
}

template <class P, bool WIDE = false>
__device__ __forceinline__ void group_deposit(float2* buf, const float4 (&v)[RowIO<P>::RPW], const short* pos,
                                              const FusedArgs& a, float tail, int wave, int lane) {
  float* fb = (float*)buf;
  int lp[4];  // in-row positions of this lane's four columns (read here, not held across the kernel)
#pragma unroll
  for (int c = 0; c < 4; ++c) lp[c] = pos[min(a.pad + 4 * lane + c, P::M - 1)];
#pragma unroll
  for (int i = 0; i < RowIO<P>::RPW; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    if (rp < P::NH && 4 * lane < a.W) {
      float* r = fb + 2 * ((rp >> 1) * P::RS) + (rp & 1);
      r[2 * lp[0]] = v[i].x;
      r[2 * lp[1]] = v[i].y;
      r[2 * lp[2]] = v[i].z;
      r[2 * lp[3]] = v[i].w;
    }
  }
  int tr, tc;
  if (tail_item<P, WIDE>(a, 64 * wave + lane, tr, tc)) *tail_slot<P>(fb, a, tr, tc) = tail;
}

// Padding columns copied inside LDS from the interior column they replicate (or zeroed).
template <class P>
__device__ __forceinline__ void group_pad_cols(float2* buf, const short* pos, const short* colsrc, int pad, int tid) {
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
__device__ __forceinline__ void group_forward_passes(float2* buf, const short* pa, const short* pb, int tid) {
  row_pass_a<P, false>(buf, tid);
  lds_barrier();
  row_pass_b<P, false>(buf, tid);
  lds_barrier();
  col_pass_a_fwd<P>(buf, pa, pb, tid);
  lds_barrier();
}

// The same passes with G1's row loads issued a few at a time between them, so the loads never
// queue up behind each other at issue and their HBM traffic spreads over G0's compute.
template <class P, bool WIDE>
__device__ __forceinline__ void group_forward_passes_loading(float2* buf, const short* pa, const short* pb, int tid,
                                                             float4 (&pre)[RowIO<P>::RPW], float& tail,
                                                             __amdgpu_buffer_rsrc_t xr, const FusedArgs& a,
                                                             int wave, int lane) {
  constexpr int N = RowIO<P>::RPW, C1 = (N + 3) / 4, C2 = (2 * N + 3) / 4, C3 = (3 * N + 3) / 4;
  group_prefetch<P, 0, C1>(pre, xr, a, 1, wave, lane);
  tail = tail_load<P, WIDE>(xr, a, 1, 64 * wave + lane);
  row_pass_a<P, false>(buf, tid);
  lds_barrier();
  group_prefetch<P, C1, C2>(pre, xr, a, 1, wave, lane);
  row_pass_b<P, false>(buf, tid);
  lds_barrier();
  group_prefetch<P, C2, C3>(pre, xr, a, 1, wave, lane);
  col_pass_a_fwd<P>(buf, pa, pb, tid);
  lds_barrier();
  group_prefetch<P, C3, N>(pre, xr, a, 1, wave, lane);
}

// Cropped rows of group G (inverse transformed, in LDS) to the output, GELU applied on store.
template <class P, bool WIDE = false>
__device__ __forceinline__ void group_store(const float2* buf, const short* pos, __amdgpu_buffer_rsrc_t orsrc,
                                            const FusedArgs& a, int G, int wave, int lane) {
  const float* fb = (const float*)buf;
  int lp[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) lp[c] = pos[min(a.pad + 4 * lane + c, P::M - 1)];
#pragma unroll 1
  for (int i = 0; i < RowIO<P>::RPW; ++i) {
    const int rp = wave + i * RowIO<P>::NW;
    if (rp < P::NH) {
      const int orr = plane_row<P>(rp, G) - a.pad;
      if (orr >= 0 && orr < a.H && 4 * lane < a.W) {
        const float* r = fb + 2 * ((rp >> 1) * P::RS) + (rp & 1);
        float4 v = make_float4(r[2 * lp[0]], r[2 * lp[1]], r[2 * lp[2]], r[2 * lp[3]]);
        if (a.act == CVN_ACT_GELU) {
          v.x = fgelu(v.x); v.y = fgelu(v.y); v.z = fgelu(v.z); v.w = fgelu(v.w);
        }
        if (!WIDE || (a.W & 31) == 0) bstore4(v, orsrc, 16u * lane, (uint32_t)(orr * a.W) * 4u);
        else bstore4c(v, orsrc, 16u * lane, (uint32_t)(orr * a.W) * 4u);
      }
    }
  }
  int tr, tc;
  if (tail_item<P, WIDE>(a, 64 * wave + lane, tr, tc)) {
    const int orr = plane_row<P>(tr, G) - a.pad;
    if (orr >= 0 && orr < a.H) {
      float t = *tail_slot<P>(const_cast<float*>(fb), a, tr, tc);
      if (a.act == CVN_ACT_GELU) t = fgelu(t);
      bstore1(t, orsrc, 4u * (uint32_t)tc, (uint32_t)(orr * a.W) * 4u);
    }
  }
}

template <class P, bool WIDE = false>
__device__ __forceinline__ void group_inverse_store(float2* buf, const short* pa, const short* pb, const short* pos,
                                                    __amdgpu_buffer_rsrc_t orsrc, const FusedArgs& a, int G,
                                                    int wave, int lane, int tid) {
  col_pass_b<P, true>(buf, pa, pb, tid);
  lds_barrier();
  col_pass_a_inv<P>(buf, pa, pb, tid);
  lds_barrier();
  row_pass_b<P, true>(buf, tid);
  lds_barrier();
  row_pass_a<P, true>(buf, tid);
  lds_barrier();
  group_store<P, WIDE>(buf, pos, orsrc, a, G, wave, lane);
}

// Table entries of the combine step are loaded kTabBatch slots at a time.
constexpr int kTabBatch = 4;

// WIDE: rows past 256 columns (the 260 plan with no padding); a separate instantiation, so the
// padded-input kernel carries none of the row-tail code.
template <class P, bool WIDE>
__global__ void __launch_bounds__(kFT) k_converse2d_fused(FusedArgs a) {
  extern __shared__ float2 smem[];
  float2* buf = smem;
  float2* parkl = smem + P::SLOTS_PAD;  // PARK_LDS rounds of parked slots
  float2* wtab = parkl + P::PARK_LDS * kFT;  // exp(-2 pi i k / N) at row position rfpos(k)
  short* pa = (short*)(wtab + P::NH + 2);
  short* pb = pa + P::NQ;
  short* pos = pb + P::NQ;
  unsigned char* isb = (unsigned char*)(pos + P::M);  // 1 where a position holds the odd row
  short* colsrc = (short*)((char*)wtab + P::CONST_BYTES);
  static_assert(tabs_layout_ok<P>(), "LDS table block layout");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t plane = fused_plane(blockIdx.x, a);
  const int64_t cp = (a.psf_batch == 1) ? (plane % a.C) : plane;
  const uint32_t plane_bytes = (uint32_t)(a.H * a.W) * 4u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + plane * (int64_t)a.H * a.W, plane_bytes);
  const __amdgpu_buffer_rsrc_t orsrc = make_rsrc(a.out + plane * (int64_t)a.H * a.W, plane_bytes);
  const __amdgpu_buffer_rsrc_t t4r = make_rsrc(a.tab4 + cp * P::SLOTS, P::SLOTS * 16u);
  {
    const v4u32_t* src = (const v4u32_t*)&kFusedTabs<P>;
    v4u32_t* dst = (v4u32_t*)wtab;
    for (int i = tid; i < P::CONST_BYTES / 16; i += kFT) dst[i] = src[i];
  }
  for (int j = tid; j < P::M; j += kFT) colsrc[j] = fpad_src(j, a.W, a.pad, a.mode);
  float4 pre[RowIO<P>::RPW];
  group_prefetch<P>(pre, xr, a, 0, wave, lane);
  float tail = tail_load<P, WIDE>(xr, a, 0, tid);
  lds_barrier();
  group_deposit<P, WIDE>(buf, pre, pos, a, tail, wave, lane);
  lds_barrier();
  group_pad_cols<P>(buf, pos, colsrc, a.pad, tid);
  lds_barrier();
  group_forward_passes_loading<P, WIDE>(buf, pa, pb, tid, pre, tail, xr, a, wave, lane);  // G1 rows arrive meanwhile
  col_pass_b<P, false>(buf, pa, pb, tid);
  lds_barrier();
  constexpr int PL = P::PARK_LDS, PR = P::PARK - P::PARK_LDS;
  float2 park[PR > 0 ? PR : 1];
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) {
    const float2 v = buf[tid + i * kFT];  // slots past SLOTS are padding (never read back)
    if (i < PL) parkl[i * kFT + tid] = v;
    else park[i - PL] = v;
  }
  lds_barrier();
  group_deposit<P, WIDE>(buf, pre, pos, a, tail, wave, lane);
  lds_barrier();
  group_pad_cols<P>(buf, pos, colsrc, a.pad, tid);
  lds_barrier();
  group_forward_passes<P>(buf, pa, pb, tid);
  // radix-2 across the groups, transfer function, inverse radix-2.  Table entries come in batches
  // of kTabBatch slots; the first batch is requested before G1's last pass.
  // Batches are double-buffered: batch b + 1 is requested before batch b is combined.
  constexpr int NB = (P::PARK + kTabBatch - 1) / kTabBatch;
  float4 f4[2][kTabBatch];
#pragma unroll
  for (int i = 0; i < kTabBatch; ++i) f4[0][i] = bload4(t4r, 16u * tid, 16u * i * kFT);
  col_pass_b<P, false>(buf, pa, pb, tid);
  lds_barrier();
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int j = bt & 1;
    if (bt + 1 < NB) {
#pragma unroll
      for (int i = 0; i < kTabBatch; ++i)
        f4[j ^ 1][i] = bload4(t4r, 16u * tid, 16u * ((bt + 1) * kTabBatch + i) * kFT);
    }
#pragma unroll
    for (int i = 0; i < kTabBatch; ++i) {
      const int ii = bt * kTabBatch + i;
      if (ii < P::PARK) {
        const int s = tid + ii * kFT;
        const int t = s / P::RS;
        const float2 w = wtab[2 * t + isb[s - t * P::RS]];  // radix-2 twiddle of the slot's row frequency
        const float2 e = ii < PL ? parkl[ii * kFT + tid] : park[ii < PL ? 0 : ii - PL], o = buf[s];
        const float2 wo = cmul(w, o);
        const float2 y0 = cmul(make_float2(f4[j][i].x, f4[j][i].y), cadd(e, wo));
        const float2 y1 = cmul(make_float2(f4[j][i].z, f4[j][i].w), csub(e, wo));
        float2 ne = cadd(y0, y1);
        // materialise E' here: otherwise the compiler sinks its arithmetic to the unpark and keeps
        // e, o and the table entry alive across the G1 inverse
        asm volatile("" : "+v"(ne.x), "+v"(ne.y));
        if (ii < PL) parkl[ii * kFT + tid] = ne;
        else park[ii < PL ? 0 : ii - PL] = ne;
        buf[s] = cmul(cconj(w), csub(y0, y1));
      }
    }
    asm volatile("" ::: "memory");  // the batch after next may not be hoisted above this one
  }
  lds_barrier();
  group_inverse_store<P, WIDE>(buf, pa, pb, pos, orsrc, a, 1, wave, lane, tid);
  lds_barrier();
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) buf[tid + i * kFT] = i < PL ? parkl[i * kFT + tid] : park[i < PL ? 0 : i - PL];
  lds_barrier();
  group_inverse_store<P, WIDE>(buf, pa, pb, pos, orsrc, a, 0, wave, lane, tid);
}

// ----------------------------------------------------------------------------------------------
// Split form for small plane counts (at most kFusedSplitPlanes planes, where one workgroup per plane
// leaves most of the 256 CUs idle): each row group of a plane gets a workgroup of its own.
//   k_converse2d_fused_fwd: group G's rows -> its forward passes -> its spectrum (SLOTS_PAD slots in
//     the group buffer's order) to the caller's scratch.
//   k_converse2d_fused_inv: both groups' spectra -> the radix-2 step across the groups and the transfer
//     function, keeping group G's half (E' for G0, O' for G1) -> G's inverse passes and store.
// The two workgroups of a plane are 16 j + r and 16 j + 8 + r (plane 8 j + r), so they run on the
// same XCD (workgroup i goes to XCD i % 8) and the second kernel reads both spectra where the first
// wrote them.  The LDS layout is the fused kernel's; the parked rounds stay unused.
// ----------------------------------------------------------------------------------------------
__device__ __forceinline__ bool split_item(int64_t blk, int64_t planes, int64_t& plane, int& G) {
  const int r = (int)(blk & 15);
  G = r >> 3;
  plane = 8 * (blk >> 4) + (r & 7);
  return plane < planes;
}
typedef unsigned int v2u32_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bstore2(float2 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32_t, v), r, voff, soff, 0);
}

template <class P, bool WIDE>
__global__ void __launch_bounds__(kFT) k_converse2d_fused_fwd(FusedArgs a, float2* spec) {
  extern __shared__ float2 smem[];
  float2* buf = smem;
  float2* wtab = smem + P::SLOTS_PAD + P::PARK_LDS * kFT;
  short* pa = (short*)(wtab + P::NH + 2);
  short* pb = pa + P::NQ;
  short* pos = pb + P::NQ;
  short* colsrc = (short*)((char*)wtab + P::CONST_BYTES);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int64_t plane;
  int G;
  if (!split_item(blockIdx.x, a.B * a.C, plane, G)) return;  // whole workgroup: no barrier is left waiting
  const uint32_t plane_bytes = (uint32_t)(a.H * a.W) * 4u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + plane * (int64_t)a.H * a.W, plane_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(spec + (2 * plane + G) * P::SLOTS_PAD, P::SLOTS_PAD * 8u);
  float4 pre[RowIO<P>::RPW];
  group_prefetch<P>(pre, xr, a, G, wave, lane);
  const float tail = tail_load<P, WIDE>(xr, a, G, tid);
  {
    const v4u32_t* src = (const v4u32_t*)&kFusedTabs<P>;
    v4u32_t* dst = (v4u32_t*)wtab;
    for (int i = tid; i < P::CONST_BYTES / 16; i += kFT) dst[i] = src[i];
  }
  for (int j = tid; j < P::M; j += kFT) colsrc[j] = fpad_src(j, a.W, a.pad, a.mode);
  lds_barrier();
  group_deposit<P, WIDE>(buf, pre, pos, a, tail, wave, lane);
  lds_barrier();
  group_pad_cols<P>(buf, pos, colsrc, a.pad, tid);
  lds_barrier();
  group_forward_passes<P>(buf, pa, pb, tid);
  col_pass_b<P, false>(buf, pa, pb, tid);
  lds_barrier();
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) bstore2(buf[tid + i * kFT], sr, 8u * tid, 8u * i * kFT);
}

template <class P, bool WIDE>
__global__ void __launch_bounds__(kFT) k_converse2d_fused_inv(FusedArgs a, const float2* spec) {
  extern __shared__ float2 smem[];
  float2* buf = smem;
  float2* wtab = smem + P::SLOTS_PAD + P::PARK_LDS * kFT;
  short* pa = (short*)(wtab + P::NH + 2);
  short* pb = pa + P::NQ;
  short* pos = pb + P::NQ;
  unsigned char* isb = (unsigned char*)(pos + P::M);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int64_t plane;
  int G;
  if (!split_item(blockIdx.x, a.B * a.C, plane, G)) return;
  const int64_t cp = (a.psf_batch == 1) ? (plane % a.C) : plane;
  const uint32_t plane_bytes = (uint32_t)(a.H * a.W) * 4u;
  const __amdgpu_buffer_rsrc_t orsrc = make_rsrc(a.out + plane * (int64_t)a.H * a.W, plane_bytes);
  const __amdgpu_buffer_rsrc_t t4r = make_rsrc(a.tab4 + cp * P::SLOTS, P::SLOTS * 16u);
  const __amdgpu_buffer_rsrc_t er = make_rsrc(spec + 2 * plane * P::SLOTS_PAD, P::SLOTS_PAD * 8u);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(spec + (2 * plane + 1) * P::SLOTS_PAD, P::SLOTS_PAD * 8u);
  // slot rounds in batches of SB (all of them at once when there are few), the next batch's loads in
  // flight while the current one is combined
  constexpr int SB = P::PARK <= 8 ? P::PARK : kTabBatch, NB = (P::PARK + SB - 1) / SB;
  float4 f4[2][SB];
  float2 e[2][SB], o[2][SB];
  auto load = [&](int bt, int j) {
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const uint32_t r = (uint32_t)(bt * SB + i) * kFT;
      f4[j][i] = bload4(t4r, 16u * tid, 16u * r);
      e[j][i] = bload2(er, 8u * tid, 8u * r);
      o[j][i] = bload2(orr, 8u * tid, 8u * r);
    }
  };
  load(0, 0);
  {
    const v4u32_t* src = (const v4u32_t*)&kFusedTabs<P>;
    v4u32_t* dst = (v4u32_t*)wtab;
    for (int i = tid; i < P::CONST_BYTES / 16; i += kFT) dst[i] = src[i];
  }
  lds_barrier();
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int j = bt & 1;
    if (bt + 1 < NB) load(bt + 1, j ^ 1);
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int s = tid + (bt * SB + i) * kFT;
      if (bt * SB + i < P::PARK && s < P::SLOTS) {  // slots past SLOTS are padding (never read back)
        const int t = s / P::RS;
        const float2 w = wtab[2 * t + isb[s - t * P::RS]];
        const float2 wo = cmul(w, o[j][i]);
        const float2 y0 = cmul(make_float2(f4[j][i].x, f4[j][i].y), cadd(e[j][i], wo));
        const float2 y1 = cmul(make_float2(f4[j][i].z, f4[j][i].w), csub(e[j][i], wo));
        buf[s] = G == 0 ? cadd(y0, y1) : cmul(cconj(w), csub(y0, y1));
      }
    }
    asm volatile("" ::: "memory");  // the batch after next may not be hoisted above this one
  }
  lds_barrier();
  group_inverse_store<P, WIDE>(buf, pa, pb, pos, orsrc, a, G, wave, lane, tid);
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
    for (int h = 0; h < 2; ++h) {
      const int u = k + h * P::NH;
      const double2 r = d_root(u, P::N);
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
    const int rp = P::rfpos(k);
    const int slot = (rp >> 1) * P::RS + ((rp & 1) ? P::pb(q) : P::pa(q));
    a.tab4[cp * P::SLOTS + slot] =
        make_float4((float)ph[0].x, (float)ph[0].y, (float)ph[1].x, (float)ph[1].y);
  }
}

// ----------------------------------------------------------------------------------------------
// Scale s > 1 (zero-insert upsample, converse2d.cpp:104-119; nearest x0, util_converse.py:172-173):
// the high-resolution (HR) plane N x M = (h s) x (w s) has a fused plan, the low-resolution (LR)
// padded plane h x w is transformed in LDS.  By the tiling identities, the HR spectra of the
// zero-inserted y and of nearest(y) are Y(u mod h, v mod w) and Y(u mod h, v mod w) Hn(u, v), so the
// solved HR spectrum is X(u, v) = Phi(u, v) Y(u mod h, v mod w) with the module-form transfer
// function (alias-class means M over the s x s aliases (u + a h, v + b w) of a bin)
//   Phi = Hn + conj(K) (1 - M(K Hn)) / (M(|K|^2) + lambda),  Hn(u, v) = H_s(u; N) H_s(v; M),
//   H_s(u; N) = sum_{a < s} exp(-2 pi i u a / N),
// normalised by 1 / (N M).  The kernel writes X straight into the two HR groups in the fused slot
// order (E' = X(k) + X(k + N/2) for the even HR rows, O' = conj(W^k) (X(k) - X(k + N/2)) for the
// odd rows) and runs the fused inverse passes; nothing but the LR input and the HR output touches HBM.
// ----------------------------------------------------------------------------------------------
struct PhiUpArgs {
  const float* psf;
  const float* bias;
  int64_t C;
  int kh, kw, s;
  double eps;
  float4* tab4;
};

__device__ __forceinline__ double2 d_hold(int64_t u, int s, int L) {  // H_s(u; L)
  double2 acc = make_double2(0.0, 0.0);
  for (int a = 0; a < s; ++a) {
    const double2 r = d_root(u * a, L);
    acc.x += r.x;
    acc.y += r.y;
  }
  return acc;
}

// One block per (psf plane, half-spectrum column q); threads over the column sub-frequency k < N/2,
// writing (Phi(k, q), Phi(k + N/2, q)) at the slot of (k, q), in fp64.
template <class P>
__global__ void __launch_bounds__(256) k_phi_fused_up(PhiUpArgs a) {
  __shared__ double2 Pq[4][64];  // row sums of the psf at the s column aliases of q
  __shared__ double2 Hq[4];      // H_s at those columns
  const int64_t cp = blockIdx.x / P::NQ;
  const int q = (int)(blockIdx.x - cp * P::NQ);
  const int c = (int)(cp % a.C);
  const int s = a.s, h = P::N / s, w = P::M / s;
  const float* psf = a.psf + cp * a.kh * a.kw;
  for (int idx = threadIdx.x; idx < s * a.kh; idx += blockDim.x) {
    const int b = idx / a.kh, i = idx - b * a.kh;
    const int64_t qb = (q + (int64_t)b * w) % P::M;
    const double2 r = d_root(qb, P::M);
    double2 e = d_root(-qb * (a.kw / 2), P::M);
    double2 acc = make_double2(0.0, 0.0);
    for (int j = 0; j < a.kw; ++j) {
      const double t = (double)psf[i * a.kw + j];
      acc.x += t * e.x;
      acc.y += t * e.y;
      e = d_cmul(e, r);
    }
    Pq[b][i] = acc;
  }
  if (threadIdx.x < s) Hq[threadIdx.x] = d_hold((q + (int64_t)threadIdx.x * w) % P::M, s, P::M);
  __syncthreads();
  const double lmb = 1.0 / (1.0 + exp(-((double)a.bias[c] - 9.0))) + a.eps;
  const double norm = 1.0 / ((double)P::N * (double)P::M);
  const double inv_s2 = 1.0 / (double)(s * s);
  for (int k = threadIdx.x; k < P::NH; k += blockDim.x) {
    double2 ph[2];
    for (int hh = 0; hh < 2; ++hh) {
      const int u = k + hh * P::NH;
      double sk2 = 0.0;
      double2 skh = make_double2(0.0, 0.0), k00 = skh, h00 = skh;
      for (int al = 0; al < s; ++al) {
        const int64_t ua = (u + (int64_t)al * h) % P::N;
        const double2 hu = d_hold(ua, s, P::N);
        const double2 r = d_root(ua, P::N);
        double2 e = d_root(-ua * (a.kh / 2), P::N);
        double2 K[4];
        for (int b = 0; b < s; ++b) K[b] = make_double2(0.0, 0.0);
        for (int i = 0; i < a.kh; ++i) {
          for (int b = 0; b < s; ++b) {
            const double2 t = d_cmul(e, Pq[b][i]);
            K[b].x += t.x;
            K[b].y += t.y;
          }
          e = d_cmul(e, r);
        }
        for (int b = 0; b < s; ++b) {
          const double2 hn = d_cmul(hu, Hq[b]);
          const double2 kh_ = d_cmul(K[b], hn);
          sk2 += K[b].x * K[b].x + K[b].y * K[b].y;
          skh.x += kh_.x;
          skh.y += kh_.y;
          if (al == 0 && b == 0) {
            k00 = K[b];
            h00 = hn;
          }
        }
      }
      const double den = sk2 * inv_s2 + lmb;
      const double2 g = make_double2((1.0 - skh.x * inv_s2) / den, -skh.y * inv_s2 / den);
      const double2 cg = d_cmul(make_double2(k00.x, -k00.y), g);  // conj(K) g
      ph[hh] = make_double2((h00.x + cg.x) * norm, (h00.y + cg.y) * norm);
    }
    const int rp = P::rfpos(k);
    const int slot = (rp >> 1) * P::RS + ((rp & 1) ? P::pb(q) : P::pa(q));
    a.tab4[cp * P::SLOTS + slot] = make_float4((float)ph[0].x, (float)ph[0].y, (float)ph[1].x, (float)ph[1].y);
  }
}

struct FusedUpArgs {
  FusedArgs hr;        // x = LR input (P, H, W); out = HR output (P, H s, W s); H, W, pad: the HR crop
  int Hl, Wl, padl;    // LR input size and padding
  int y_off, tw_off, idx_off;  // LDS offsets (bytes) of the LR spectrum, LR twiddles, kof / qof tables
};

// Stockham radices of the LR transform length L = N / s (fixed butterflies, first to last).
template <int L> struct LrRadices;
template <> struct LrRadices<66> { static constexpr int n = 3, r0 = 2, r1 = 3, r2 = 11; };
template <> struct LrRadices<44> { static constexpr int n = 2, r0 = 4, r1 = 11, r2 = 1; };
template <> struct LrRadices<33> { static constexpr int n = 2, r0 = 3, r1 = 11, r2 = 1; };
// L = 256 / 4 on the 256 x 256 Cooley-Tukey plan
template <> struct LrRadices<64> { static constexpr int n = 3, r0 = 4, r1 = 4, r2 = 4; };

// LR twiddles exp(-2 pi i m / L), m < L, twice (the row and the column transform of a square LR
// plane), evaluated at compile time in double and rounded once.
template <int L>
struct alignas(16) LrTwTab {
  float v[4 * L];
  constexpr LrTwTab() : v() {
    for (int m = 0; m < L; ++m) {
      const CosSin cs = cos_sin_turn(m, L);
      v[2 * m] = v[2 * (m + L)] = (float)cs.c;
      v[2 * m + 1] = v[2 * (m + L) + 1] = (float)-cs.s;
    }
  }
};
template <int L>
__device__ const LrTwTab<L> kLrTw = LrTwTab<L>();

// The LR transform of `ntr` rows of length L (a -> b -> ...), compile-time radices; returns the buffer
// holding the result.
template <int L>
__device__ __forceinline__ float2* lr_fft(float2* a, float2* b, int ntr, const float2* tw, int tid) {
  using Rd = LrRadices<L>;
  stockham_pass<Rd::r0, false>(a, b, L, 1, ntr, tw, tid, kFT);
  __syncthreads();
  stockham_pass<Rd::r1, false>(b, a, L, Rd::r0, ntr, tw, tid, kFT);
  __syncthreads();
  if constexpr (Rd::n == 3) {
    stockham_pass<Rd::r2, false>(a, b, L, Rd::r0 * Rd::r1, ntr, tw, tid, kFT);
    __syncthreads();
    return b;
  }
  return a;
}

// LR padded-plane index maps use the padding map of the LR input (as the reference pads before the
// upsample, util_converse.py:144-145).
// The even-row group is parked in registers and the LDS holds one group, the slot tables and the LR
// spectrum: two workgroups per CU (8 waves per SIMD) on the 132 x 132 plan, one (4 waves per SIMD,
// 159 KB of LDS) on the 256 x 256 plan.
template <class P, int S>
__global__ void __launch_bounds__(kFT, P::kCT ? 4 : 8) k_converse2d_fused_up(FusedUpArgs ua) {
  static_assert(P::N == P::M && P::N % S == 0, "square HR plane, LR side N / S");
  constexpr int h = P::N / S, w = P::M / S, ncl = w / 2 + 1, npl = (h + 1) / 2;
  extern __shared__ float2 smem[];
  const FusedArgs& a = ua.hr;
  float2* buf = smem;
  float2* wtab = smem + P::SLOTS_PAD;
  short* pa = (short*)(wtab + P::NH + 2);
  short* pb = pa + P::NQ;
  short* pos = pb + P::NQ;
  unsigned char* isb = (unsigned char*)(pos + P::M);  // the fused kernel's table block layout
  char* base = (char*)smem;
  float2* Y = (float2*)(base + ua.y_off);      // LR half spectrum, column-major: Y[v h + u]
  float2* twl = (float2*)(base + ua.tw_off);   // exp(-2 pi i m / w), m < w
  float2* twh = twl + w;                       // exp(-2 pi i m / h), m < h
  short* kof = (short*)(base + ua.idx_off);    // column frequency k of row position rp
  short* qof = kof + P::NH;                    // half-spectrum column q of a row-pair position
  static_assert(tabs_layout_ok<P>() && w == h, "table block layout, square LR plane");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t plane = fused_plane(blockIdx.x, a);
  const int64_t cp = (a.psf_batch == 1) ? (plane % a.C) : plane;
  const uint32_t in_bytes = (uint32_t)(ua.Hl * ua.Wl) * 4u, out_bytes = (uint32_t)(a.H * a.W) * 4u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + plane * (int64_t)ua.Hl * ua.Wl, in_bytes);
  const __amdgpu_buffer_rsrc_t orsrc = make_rsrc(a.out + plane * (int64_t)a.H * a.W, out_bytes);
  const __amdgpu_buffer_rsrc_t t4r = make_rsrc(a.tab4 + cp * P::SLOTS, P::SLOTS * 16u);
  // tables: the compile-time block (radix-2 twiddles by row position, slot and in-row positions, the
  // odd-row flags) and the LR twiddles, copied; the slot -> (k, q) maps
  {
    const v4u32_t* src = (const v4u32_t*)&kFusedTabs<P>;
    v4u32_t* dst = (v4u32_t*)wtab;
    for (int i = tid; i < P::CONST_BYTES / 16; i += kFT) dst[i] = src[i];
    const float2* lt = (const float2*)kLrTw<w>.v;
    for (int m = tid; m < w + h; m += kFT) twl[m] = lt[m];
  }
  for (int k = tid; k < P::NH; k += kFT) kof[P::rfpos(k)] = (short)k;
  for (int q = tid; q < P::NQ; q += kFT) {
    qof[P::pa(q)] = (short)q;
    qof[P::pb(q)] = (short)q;
  }
  // LR padded plane as complex row pairs (row 2t in .x, 2t + 1 in .y) in buf
  float2* A = buf;
  float2* Bw = buf + npl * w;
  for (int e = tid; e < npl * w; e += kFT) {
    const int t = e / w, j = e - t * w;
    const int sc = fpad_src(j, ua.Wl, ua.padl, a.mode);
    const int r0 = fpad_src(2 * t, ua.Hl, ua.padl, a.mode);
    const int r1 = 2 * t + 1 < h ? fpad_src(2 * t + 1, ua.Hl, ua.padl, a.mode) : -1;
    float2 v = make_float2(0.f, 0.f);
    if (sc >= 0) {
      if (r0 >= 0) v.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, 4u * (uint32_t)(r0 * ua.Wl + sc), 0u, 0));
      if (r1 >= 0) v.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, 4u * (uint32_t)(r1 * ua.Wl + sc), 0u, 0));
    }
    A[e] = v;
  }
  __syncthreads();
  const float2* R = lr_fft<w>(A, Bw, npl, twl, tid);
  // Hermitian unpack of each row pair into the two rows' half spectra, column-major into Y
  for (int e = tid; e < npl * ncl; e += kFT) {
    const int t = e / ncl, v = e - t * ncl;
    const float2 zl = R[t * w + v], zh = R[t * w + (v ? w - v : 0)];
    Y[v * h + 2 * t] = make_float2(0.5f * (zl.x + zh.x), 0.5f * (zl.y - zh.y));
    if (2 * t + 1 < h) Y[v * h + 2 * t + 1] = make_float2(0.5f * (zl.y + zh.y), 0.5f * (zh.x - zl.x));
  }
  __syncthreads();
  const float2* Yr = lr_fft<h>(Y, buf, ncl, twh, tid);
  if (Yr != Y) {
    for (int e = tid; e < ncl * h; e += kFT) Y[e] = Yr[e];
    __syncthreads();
  }
  // solved HR spectrum straight into the two groups: G1 (odd HR rows) in buf, G0 (even) parked
  float2 park[P::PARK];
#pragma unroll
  for (int i0 = 0; i0 < P::PARK; ++i0) {
    const int sl = tid + i0 * kFT;
    float2 e0 = make_float2(0.f, 0.f), o1 = e0;
    if (sl < P::SLOTS) {
      const int t = sl / P::RS, p = sl - t * P::RS;
      const int rp = 2 * t + isb[p];
      const int k = kof[rp], q = qof[p];
      const float4 f = bload4(t4r, 16u * (uint32_t)sl, 0u);
      float2 yk[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int uu = (k + hh * P::NH) % h, vv = q % w;
        yk[hh] = vv < ncl ? Y[vv * h + uu] : cconj(Y[(w - vv) * h + (uu ? h - uu : 0)]);
      }
      const float2 x0 = cmul(make_float2(f.x, f.y), yk[0]), x1 = cmul(make_float2(f.z, f.w), yk[1]);
      e0 = cadd(x0, x1);
      o1 = cmul(cconj(wtab[rp]), csub(x0, x1));
    }
    park[i0] = e0;
    buf[sl] = o1;
  }
  lds_barrier();
  group_inverse_store<P>(buf, pa, pb, pos, orsrc, a, 1, wave, lane, tid);
  lds_barrier();
#pragma unroll
  for (int i = 0; i < P::PARK; ++i) buf[tid + i * kFT] = park[i];
  lds_barrier();
  group_inverse_store<P>(buf, pa, pb, pos, orsrc, a, 0, wave, lane, tid);
}

// ----------------------------------------------------------------------------------------------
// host dispatch
// ----------------------------------------------------------------------------------------------
using Plan260 = FusedPlan<260, 4, 5, 13, 5, 13, 5>;   // rows 260 = 4 5 13, columns 130 = 5 13 2
using Plan132 = FusedPlan<132, 4, 3, 11, 3, 11>;   // rows 132 = 4 3 11, columns 66 = 3 11 2
using Plan256 = CtPlan<16, 16, 8, 1>;              // rows 256 = 16 16, columns 128 = 2 8 8 (Cooley-Tukey)

// The generic table kernel writes this plan's tables through fused256_phi_index (cvn_common.h):
// check that map against the plan's slot order (the layout k_phi_fused<Plan256> writes).
constexpr bool fused256_index_ok() {
  using P = Plan256;
  if (P::RS != kF256Rs || P::SLOTS != kF256Slots) return false;
  for (int u = 0; u < P::N; ++u) {
    const int rp = P::rfpos(u % P::NH);
    // sampled columns: DC, the first bins, interior bins, and the last two (v = NQ - 1 is the Nyquist
    // column, whose odd-row slot is the pos = M + 1 special case of pb)
    constexpr int kV[] = {0, 1, 2, 37, 64, 100, P::NQ - 3, P::NQ - 2, P::NQ - 1};
    for (int v : kV) {
      const int64_t want = 2 * ((int64_t)(rp >> 1) * P::RS + ((rp & 1) ? P::pb(v) : P::pa(v))) + u / P::NH;
      if (fused256_phi_index(0, v, u) != want || fused256_phi_index(3, v, u) != want + 2 * 3 * P::SLOTS) return false;
    }
  }
  return true;
}
static_assert(fused256_index_ok(), "fused256_phi_index matches Plan256");

// The 256 x 256 plan as the up kernel uses it: the table block directly after the group buffer (the
// up kernel parks nothing in LDS; its LR spectrum takes that space), which is where the Cooley-Tukey
// passes then look for their twiddles (ct_tw).
struct Plan256Up : Plan256 {
  static constexpr int PARK_LDS = 0;
};

// LDS layout of the up kernel after the fused kernel's own regions.
struct UpLayout {
  int y_off, tw_off, idx_off;
  size_t bytes;
};
template <class P>
UpLayout up_layout(int h, int w) {
  UpLayout L;
  size_t o = align_up((size_t)P::SLOTS_PAD * 8 + P::TAB_BYTES, 16);
  L.y_off = (int)o;
  o += (size_t)(w / 2 + 1) * h * 8;
  L.tw_off = (int)o;
  o += (size_t)(w + h) * 8;
  L.idx_off = (int)o;
  o += (size_t)(P::NH + P::RS) * 2;
  L.bytes = align_up(o, 16);
  return L;
}

// The up path serves HR planes of the 132 x 132 plan from LR planes h = w = 132 / s, s in 2..4, and
// of the 256 x 256 plan from h = w = 64 at s = 4 (Converse-USRNet's first data step; at s = 2 the LR
// spectrum would not fit next to the group buffer), whose transforms use fixed radices only; the LR
// pair buffers (2 (h + 1) / 2 w) and the column transform's scratch fit in the group buffer.  Returns
// the HR plan's side, or 0.
template <class P>
bool fused_up_fits(int h, int w, size_t lds_max) {
  const int npl = (h + 1) / 2;
  if ((size_t)2 * npl * w > (size_t)P::SLOTS_PAD || (size_t)(w / 2 + 1) * h > (size_t)P::SLOTS_PAD) return false;
  return up_layout<P>(h, w).bytes <= lds_max;
}
int fused_up_plan(int H, int W, int pad, int s) {
  const int h = H + 2 * pad, w = W + 2 * pad;
  if (s < 2 || s > 4 || h != w || (W * s) % 4 != 0) return 0;
  if (h * s == Plan132::N && fused_up_fits<Plan132>(h, w, 80 * 1024)) return Plan132::N;  // two workgroups per CU
  if (h * s == Plan256Up::N && s == 4 && fused_up_fits<Plan256Up>(h, w, 160 * 1024)) return Plan256Up::N;
  return 0;
}

template <class P>
size_t fused_ws(int64_t Cp) {
  return align_up((size_t)Cp * P::SLOTS * sizeof(float4));
}

template <class P>
int fused_table_run(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                    void* table, hipStream_t st) {
  const int64_t Cp = psf_batch * C;
  float4* t4 = (float4*)table;
  PhiFusedArgs pa{psf, bias, C, kh, kw, (double)eps, t4};
  hipLaunchKernelGGL(k_phi_fused<P>, dim3((unsigned)(Cp * P::NQ)), dim3(256), 0, st, pa);
  return check_launch("fused transfer table");
}

template <class P>
size_t fused_split_bytes(int64_t planes) {
  return align_up((size_t)planes * 2 * P::SLOTS_PAD * sizeof(float2));
}

template <class P, bool WIDE>
void fused_split_launch(const FusedArgs& fa, void* scratch, hipStream_t st) {
  const unsigned grid = (unsigned)(16 * ((fa.B * fa.C + 7) / 8));
  hipLaunchKernelGGL((k_converse2d_fused_fwd<P, WIDE>), dim3(grid), dim3(kFT), P::LDS_BYTES, st, fa,
                     (float2*)scratch);
  hipLaunchKernelGGL((k_converse2d_fused_inv<P, WIDE>), dim3(grid), dim3(kFT), P::LDS_BYTES, st, fa,
                     (const float2*)scratch);
}

template <class P>
int fused_apply_run(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode,
                    int act, const void* table, void* scratch, float* out, hipStream_t st) {
  static std::atomic<uint64_t> attr{0};
  once_per_device(attr, [] {
    for (const void* k : {(const void*)k_converse2d_fused<P, false>, (const void*)k_converse2d_fused_fwd<P, false>,
                          (const void*)k_converse2d_fused_inv<P, false>})
      (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)P::LDS_BYTES);
    if constexpr (RowTail<P>::kAny) {
      for (const void* k : {(const void*)k_converse2d_fused<P, true>, (const void*)k_converse2d_fused_fwd<P, true>,
                            (const void*)k_converse2d_fused_inv<P, true>})
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)P::LDS_BYTES);
    }
    (void)hipGetLastError();
  });
  const float4* t4 = (const float4*)table;
  FusedArgs fa{x, t4, out, B, C, psf_batch, H, W, pad, mode, act};
  bool wide = false;
  if constexpr (RowTail<P>::kAny) wide = W > 256;
  if (scratch && B * C <= kFusedSplitPlanes) {
    if constexpr (RowTail<P>::kAny) {
      if (wide) fused_split_launch<P, true>(fa, scratch, st);
    }
    if (!wide) fused_split_launch<P, false>(fa, scratch, st);
    return check_launch("fused converse2d (split)");
  }
  if constexpr (RowTail<P>::kAny) {
    if (wide)
      hipLaunchKernelGGL((k_converse2d_fused<P, true>), dim3((unsigned)(B * C)), dim3(kFT), P::LDS_BYTES, st, fa);
  }
  if (!wide)
    hipLaunchKernelGGL((k_converse2d_fused<P, false>), dim3((unsigned)(B * C)), dim3(kFT), P::LDS_BYTES, st, fa);
  return check_launch("fused converse2d");
}

// The fused kernel loads rows as float4 per lane: W must be a multiple of 4 and at most 256, or 260
// on the 260-point plan with no padding (the last 4 columns go through single-word loads and stores).
// At scale > 1 the HR plane must have a fused plan (fused_up_plan).
int fused_query(int H, int W, int pad, int scale, int64_t Cp, size_t* ws_bytes) {
  if (scale != 1) {
    const int plan = fused_up_plan(H, W, pad, scale);
    if (!plan) return 0;
    *ws_bytes = plan == Plan256Up::N ? fused_ws<Plan256Up>(Cp) : fused_ws<Plan132>(Cp);
    return 1;
  }
  if (W % 4 != 0 || W > 260) return 0;  // past 256 columns only the 260 plan with no padding applies
  const int h = H + 2 * pad, w = W + 2 * pad;
  if (h == 260 && w == 260) { *ws_bytes = fused_ws<Plan260>(Cp); return 1; }
  if (h == 132 && w == 132) { *ws_bytes = fused_ws<Plan132>(Cp); return 1; }
  if (h == 256 && w == 256) { *ws_bytes = fused_ws<Plan256>(Cp); return 1; }
  return 0;
}

size_t fused_scratch(int64_t planes, int H, int W, int pad, int scale) {
  if (scale != 1 || planes > kFusedSplitPlanes) return 0;
  const int h = H + 2 * pad;
  if (h == 260) return fused_split_bytes<Plan260>(planes);
  if (h == 256) return fused_split_bytes<Plan256>(planes);
  if (h == 132) return fused_split_bytes<Plan132>(planes);
  return 0;
}

int fused_table(const float* psf, const float* bias, float eps, int64_t C, int64_t psf_batch, int kh, int kw,
                int H, int W, int pad, int scale, void* table, hipStream_t st) {
  if (scale != 1) {
    const int64_t Cp = psf_batch * C;
    PhiUpArgs pa{psf, bias, C, kh, kw, scale, (double)eps, (float4*)table};
    if (fused_up_plan(H, W, pad, scale) == Plan256Up::N)
      hipLaunchKernelGGL(k_phi_fused_up<Plan256Up>, dim3((unsigned)(Cp * Plan256Up::NQ)), dim3(256), 0, st, pa);
    else
      hipLaunchKernelGGL(k_phi_fused_up<Plan132>, dim3((unsigned)(Cp * Plan132::NQ)), dim3(256), 0, st, pa);
    return check_launch("fused transfer table (scale > 1)");
  }
  const int h = H + 2 * pad;
  if (h == 260) return fused_table_run<Plan260>(psf, bias, eps, C, psf_batch, kh, kw, table, st);
  if (h == 256) return fused_table_run<Plan256>(psf, bias, eps, C, psf_batch, kh, kw, table, st);
  return fused_table_run<Plan132>(psf, bias, eps, C, psf_batch, kh, kw, table, st);
}

template <class P>
FusedUpArgs up_args(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode,
                    int act, int scale, const void* table, float* out, size_t* lds) {
  FusedUpArgs ua;
  const UpLayout L = up_layout<P>(H + 2 * pad, W + 2 * pad);
  ua.hr = FusedArgs{x, (const float4*)table, out, B, C, psf_batch, H * scale, W * scale, pad * scale, mode, act};
  ua.Hl = H;
  ua.Wl = W;
  ua.padl = pad;
  ua.y_off = L.y_off;
  ua.tw_off = L.tw_off;
  ua.idx_off = L.idx_off;
  *lds = L.bytes;
  return ua;
}

int fused_apply(const float* x, int64_t B, int64_t C, int H, int W, int64_t psf_batch, int pad, int mode, int act,
                int scale, const void* table, void* scratch, float* out, hipStream_t st) {
  if (scale != 1) {
    static std::atomic<uint64_t> attr{0};
    once_per_device(attr, [] {
      for (const void* k : {(const void*)k_converse2d_fused_up<Plan132, 2>, (const void*)k_converse2d_fused_up<Plan132, 3>,
                            (const void*)k_converse2d_fused_up<Plan132, 4>})
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024);
      (void)hipFuncSetAttribute((const void*)k_converse2d_fused_up<Plan256Up, 4>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      (void)hipGetLastError();
    });
    const int plan = fused_up_plan(H, W, pad, scale);
    if (!plan) return fail(CVN_ERR_UNSUPPORTED, "no fused plan for this upsampling geometry");
    const dim3 grid((unsigned)(B * C));
    size_t lds = 0;
    if (plan == Plan256Up::N) {
      using P = Plan256Up;
      const FusedUpArgs ua = up_args<P>(x, B, C, H, W, psf_batch, pad, mode, act, scale, table, out, &lds);
      hipLaunchKernelGGL((k_converse2d_fused_up<P, 4>), grid, dim3(kFT), lds, st, ua);
      return check_launch("fused converse2d (scale > 1)");
    }
    using P = Plan132;
    const FusedUpArgs ua = up_args<P>(x, B, C, H, W, psf_batch, pad, mode, act, scale, table, out, &lds);
    switch (scale) {
      case 2: hipLaunchKernelGGL((k_converse2d_fused_up<P, 2>), grid, dim3(kFT), lds, st, ua); break;
      case 3: hipLaunchKernelGGL((k_converse2d_fused_up<P, 3>), grid, dim3(kFT), lds, st, ua); break;
      default: hipLaunchKernelGGL((k_converse2d_fused_up<P, 4>), grid, dim3(kFT), lds, st, ua); break;
    }
    return check_launch("fused converse2d (scale > 1)");
  }
  const int h = H + 2 * pad;
  if (h == 260) return fused_apply_run<Plan260>(x, B, C, H, W, psf_batch, pad, mode, act, table, scratch, out, st);
  if (h == 256) return fused_apply_run<Plan256>(x, B, C, H, W, psf_batch, pad, mode, act, table, scratch, out, st);
  return fused_apply_run<Plan132>(x, B, C, H, W, psf_batch, pad, mode, act, table, scratch, out, st);
}

}  // namespace cvn
