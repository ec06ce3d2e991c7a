// Device-side FFT building blocks for gfx950 (wave64): complex helpers, fixed-radix DFT butterflies,
// and a mixed-radix Stockham pass over batches of transforms held in LDS.
//
// Conventions: forward transforms use exp(-2 pi i n k / L); inverse transforms use the conjugate
// root and are unnormalised (callers fold 1/L into their spectral scale factor).  Twiddle tables
// hold exp(-2 pi i m / L) for m in [0, L), evaluated in fp64 and rounded once to fp32, so no
// fast-math sin/cos enters the transform.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cvn {

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(fmaf(a.x, b.x, -(a.y * b.y)), fmaf(a.x, b.y, a.y * b.x));
}
__device__ __forceinline__ float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
// Multiply by -i (forward) or +i (inverse).
template <bool INV>
__device__ __forceinline__ float2 rot(float2 a) {
  return INV ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}
template <bool INV>
__device__ __forceinline__ float2 twid(float2 w) {  // table entry -> direction-specific root
  return INV ? make_float2(w.x, -w.y) : w;
}

// Exact-form GELU 0.5 x (1 + erf(x / sqrt 2)) with erf from Abramowitz & Stegun, Handbook of
// Mathematical Functions, eq. 7.1.26: erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^{-z^2},
// t = 1 / (1 + p z) for z >= 0 (odd extension), |error| <= 1.5e-7.  With z = |x| / sqrt 2 and
// h = 0.5 |x| t P(t) e^{-x^2 / 2} this is GELU(x) = max(x, 0) - h for either sign of x (for x < 0,
// 0.5 x (1 - (1 - 2h/|x|)) = -h), so the 0.5 folds into the coefficients and no 1 - erf
// cancellation occurs.  Measured against the exact GELU in fp64 over [-12, 12]: |error| <= 3.3e-7,
// at about 13 instructions (two of them the hardware reciprocal and exp2).
__device__ __forceinline__ float gelu_fast(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752f, a, 1.0f));
  float p = fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
  p = fmaf(p, t, 0.5f * 1.421413741f);
  p = fmaf(p, t, 0.5f * -0.284496736f);
  p = fmaf(p, t, 0.5f * 0.254829592f);
  p *= t;
  const float e = __builtin_amdgcn_exp2f((a * (-0.5f * 1.4426950408889634f)) * a);
  return __builtin_amdgcn_fmed3f(x, 0.0f, __builtin_inff()) - (a * p) * e;
}

// Division by a block-uniform divisor d through a multiply-high with m = ceil(2^32 / d): exact for
// a * d < 2^32, which every index here satisfies (a < 2^20, d <= 4096).  Replaces the ~30-instruction
// integer division sequence in the index arithmetic of the FFT passes.
struct FastDiv {
  uint32_t m;
  int d;
};
__device__ __forceinline__ FastDiv fast_div(int d) {
  return FastDiv{d > 1 ? 0xFFFFFFFFu / (uint32_t)d + 1u : 0u, d};
}
__device__ __forceinline__ int operator/(int a, FastDiv f) {
  return f.d > 1 ? (int)__umulhi((uint32_t)a, f.m) : a;
}

// cos and sin of 2 pi m / n by Taylor series in double at compile time (|angle| <= pi after
// reduction; 40 terms leave a truncation error far below double rounding).
struct CosSin {
  double c, s;
};
constexpr CosSin cos_sin_turn(int m, int n) {
  m %= n;
  if (m < 0) m += n;
  if (4 * m % n == 0) {  // whole quarter turns exactly
    const int q = 4 * m / n;
    return CosSin{q == 0 ? 1.0 : q == 2 ? -1.0 : 0.0, q == 1 ? 1.0 : q == 3 ? -1.0 : 0.0};
  }
  if (2 * m >= n) m -= n;
  const double x = 2.0 * 3.14159265358979323846 * m / n;
  double c = 0.0, s = 0.0, term = 1.0;
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

// cos / sin of 2 pi m / R, m in [0, R), for the odd prime radices (values computed in double and
// rounded to float).
template <int R> struct Roots;
template <> struct Roots<3> {
  static constexpr float c[3] = {1.0f, -0.5f, -0.5f};
  static constexpr float s[3] = {0.0f, 0.8660254037844387f, -0.8660254037844387f};
};
template <> struct Roots<5> {
  static constexpr float c[5] = {1.0f, 0.30901699437494745f, -0.8090169943749473f,
                                 -0.8090169943749473f, 0.30901699437494745f};
  static constexpr float s[5] = {0.0f, 0.9510565162951535f, 0.5877852522924732f,
                                 -0.5877852522924732f, -0.9510565162951535f};
};
template <> struct Roots<7> {
  static constexpr float c[7] = {1.0f, 0.6234898018587336f, -0.22252093395631434f,
                                 -0.900968867902419f, -0.900968867902419f, -0.22252093395631434f,
                                 0.6234898018587336f};
  static constexpr float s[7] = {0.0f, 0.7818314824680298f, 0.9749279121818236f,
                                 0.43388373911755823f, -0.43388373911755823f,
                                 -0.9749279121818236f, -0.7818314824680298f};
};
template <> struct Roots<11> {
  static constexpr float c[11] = {1.0f, 0.8412535328311812f, 0.41541501300188644f,
                                  -0.142314838273285f, -0.654860733945285f, -0.9594929736144974f,
                                  -0.9594929736144974f, -0.654860733945285f, -0.142314838273285f,
                                  0.41541501300188644f, 0.8412535328311812f};
  static constexpr float s[11] = {0.0f, 0.5406408174555976f, 0.9096319953545183f,
                                  0.9898214418809328f, 0.7557495743542583f, 0.28173255684142967f,
                                  -0.28173255684142967f, -0.7557495743542583f, -0.9898214418809328f,
                                  -0.9096319953545183f, -0.5406408174555976f};
};
template <> struct Roots<13> {
  static constexpr float c[13] = {1.0f, 0.8854560256532099f, 0.5680647467311559f,
                                  0.120536680255323f, -0.35460488704253545f, -0.7485107481711012f,
                                  -0.970941817426052f, -0.970941817426052f, -0.7485107481711012f,
                                  -0.35460488704253545f, 0.120536680255323f, 0.5680647467311559f,
                                  0.8854560256532099f};
  static constexpr float s[13] = {0.0f, 0.4647231720437685f, 0.8229838658936564f,
                                  0.992708874098054f, 0.9350162426854148f, 0.6631226582407952f,
                                  0.23931566428755768f, -0.23931566428755768f, -0.6631226582407952f,
                                  -0.9350162426854148f, -0.992708874098054f, -0.8229838658936564f,
                                  -0.4647231720437685f};
};

// ----------------------------------------------------------------------------------------------
// In-register DFTs of a fixed radix R on u[0..R-1] (in place, natural order in and out).
// ----------------------------------------------------------------------------------------------
template <int R, bool INV> struct Dft;

template <bool INV> struct Dft<2, INV> {
  static __device__ __forceinline__ void run(float2* u) {
    float2 a = u[0], b = u[1];
    u[0] = cadd(a, b);
    u[1] = csub(a, b);
  }
};

template <bool INV> struct Dft<4, INV> {
  static __device__ __forceinline__ void run(float2* u) {
    float2 s02 = cadd(u[0], u[2]), d02 = csub(u[0], u[2]);
    float2 s13 = cadd(u[1], u[3]), d13 = rot<INV>(csub(u[1], u[3]));
    u[0] = cadd(s02, s13);
    u[2] = csub(s02, s13);
    u[1] = cadd(d02, d13);
    u[3] = csub(d02, d13);
  }
};

template <bool INV> struct Dft<8, INV> {
  static __device__ __forceinline__ void run(float2* u) {
    constexpr float r = 0.70710678118654752f;
    float2 e[4] = {u[0], u[2], u[4], u[6]};
    float2 o[4] = {u[1], u[3], u[5], u[7]};
    Dft<4, INV>::run(e);
    Dft<4, INV>::run(o);
    // o[k] *= w8^k  (w8 = exp(-+ 2 pi i / 8))
    float2 o1 = INV ? make_float2(r * (o[1].x - o[1].y), r * (o[1].x + o[1].y))
                    : make_float2(r * (o[1].x + o[1].y), r * (o[1].y - o[1].x));
    float2 o2 = rot<INV>(o[2]);
    float2 o3 = INV ? make_float2(-r * (o[3].x + o[3].y), r * (o[3].x - o[3].y))
                    : make_float2(r * (o[3].y - o[3].x), -r * (o[3].x + o[3].y));
    u[0] = cadd(e[0], o[0]);
    u[4] = csub(e[0], o[0]);
    u[1] = cadd(e[1], o1);
    u[5] = csub(e[1], o1);
    u[2] = cadd(e[2], o2);
    u[6] = csub(e[2], o2);
    u[3] = cadd(e[3], o3);
    u[7] = csub(e[3], o3);
  }
};

// 16-point DFT as 4 x 4 (Cooley-Tukey): sample 4 n1 + n2, 4-point DFTs over n1, twiddles
// W16^(n2 k1), 4-point DFTs over n2; natural order in and out.
template <bool INV, int J>
__device__ __forceinline__ float2 tw16(float2 x) {
  if constexpr (J % 16 == 0) {
    return x;
  } else if constexpr (J % 16 == 4) {
    return rot<INV>(x);
  } else {
    constexpr CosSin w = cos_sin_turn(J, 16);
    return cmul(x, make_float2((float)w.c, INV ? (float)w.s : (float)-w.s));
  }
}
template <bool INV> struct Dft<16, INV> {
  template <int N2>
  static __device__ __forceinline__ void col(float2 (&a)[4][4]) {
    a[N2][1] = tw16<INV, N2 * 1>(a[N2][1]);
    a[N2][2] = tw16<INV, N2 * 2>(a[N2][2]);
    a[N2][3] = tw16<INV, N2 * 3>(a[N2][3]);
  }
  static __device__ __forceinline__ void run(float2* u) {
    float2 a[4][4];  // a[n2][k1]
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) {
#pragma unroll
      for (int n1 = 0; n1 < 4; ++n1) a[n2][n1] = u[4 * n1 + n2];
      Dft<4, INV>::run(a[n2]);
    }
    col<1>(a);
    col<2>(a);
    col<3>(a);
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) {
      float2 v[4] = {a[0][k1], a[1][k1], a[2][k1], a[3][k1]};
      Dft<4, INV>::run(v);
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) u[k1 + 4 * k2] = v[k2];
    }
  }
};

// Odd prime radix via conjugate-pair sums: X_q = A_q -+ i B_q, X_{R-q} = A_q +- i B_q with
// A_q = u0 + sum_j cos(2 pi j q / R)(u_j + u_{R-j}),  B_q = sum_j sin(2 pi j q / R)(u_j - u_{R-j}).
template <int R, bool INV> struct DftOdd {
  static __device__ __forceinline__ void run(float2* u) {
    constexpr int H = (R - 1) / 2;
    float2 a[H], b[H];
    const float2 x0 = u[0];
    float2 sum = x0;
#pragma unroll
    for (int j = 1; j <= H; ++j) {
      a[j - 1] = cadd(u[j], u[R - j]);
      b[j - 1] = csub(u[j], u[R - j]);
      sum = cadd(sum, a[j - 1]);
    }
    u[0] = sum;  // inputs 1..R-1 are dead from here on: outputs overwrite them in place
#pragma unroll
    for (int q = 1; q <= H; ++q) {
      float2 A = x0, Bv = make_float2(0.f, 0.f);
#pragma unroll
      for (int j = 1; j <= H; ++j) {
        const int m = (j * q) % R;
        const float c = Roots<R>::c[m], s = Roots<R>::s[m];
        A.x = fmaf(c, a[j - 1].x, A.x);
        A.y = fmaf(c, a[j - 1].y, A.y);
        Bv.x = fmaf(s, b[j - 1].x, Bv.x);
        Bv.y = fmaf(s, b[j - 1].y, Bv.y);
      }
      if (!INV) {
        u[q] = make_float2(A.x + Bv.y, A.y - Bv.x);
        u[R - q] = make_float2(A.x - Bv.y, A.y + Bv.x);
      } else {
        u[q] = make_float2(A.x - Bv.y, A.y + Bv.x);
        u[R - q] = make_float2(A.x + Bv.y, A.y - Bv.x);
      }
    }
  }
};
// In-place odd-radix DFT straight from / to memory (LDS) at a compile-time stride: inputs are
// combined into conjugate-pair sums as they arrive and outputs are stored as soon as each pair
// (q, R - q) is formed, so the register footprint is ~2R floats instead of ~4R.
template <int R, int STRIDE, bool INV>
__device__ __forceinline__ void dft_odd_mem(float2* p) {
  constexpr int H = (R - 1) / 2;
  float2 a[H], b[H];
  const float2 x0 = p[0];
  float2 sum = x0;
#pragma unroll
  for (int j = 1; j <= H; ++j) {
    const float2 lo = p[j * STRIDE], hi = p[(R - j) * STRIDE];
    a[j - 1] = cadd(lo, hi);
    b[j - 1] = csub(lo, hi);
    sum = cadd(sum, a[j - 1]);
  }
  p[0] = sum;
#pragma unroll
  for (int q = 1; q <= H; ++q) {
    float2 A = x0, Bv = make_float2(0.f, 0.f);
#pragma unroll
    for (int j = 1; j <= H; ++j) {
      const int m = (j * q) % R;
      const float c = Roots<R>::c[m], s = Roots<R>::s[m];
      A.x = fmaf(c, a[j - 1].x, A.x);
      A.y = fmaf(c, a[j - 1].y, A.y);
      Bv.x = fmaf(s, b[j - 1].x, Bv.x);
      Bv.y = fmaf(s, b[j - 1].y, Bv.y);
    }
    if (!INV) {
      p[q * STRIDE] = make_float2(A.x + Bv.y, A.y - Bv.x);
      p[(R - q) * STRIDE] = make_float2(A.x - Bv.y, A.y + Bv.x);
    } else {
      p[q * STRIDE] = make_float2(A.x - Bv.y, A.y + Bv.x);
      p[(R - q) * STRIDE] = make_float2(A.x + Bv.y, A.y - Bv.x);
    }
  }
}

template <bool INV> struct Dft<3, INV> : DftOdd<3, INV> {};
template <bool INV> struct Dft<5, INV> : DftOdd<5, INV> {};
template <bool INV> struct Dft<7, INV> : DftOdd<7, INV> {};
template <bool INV> struct Dft<11, INV> : DftOdd<11, INV> {};
template <bool INV> struct Dft<13, INV> : DftOdd<13, INV> {};

// ----------------------------------------------------------------------------------------------
// FFT plan: a length L = prod(radix[i]) decomposed into Stockham passes.
// ----------------------------------------------------------------------------------------------
constexpr int kMaxStages = 24;
// Prime radices above 13 whose R - 1 factors into the fixed butterflies are computed with Rader's
// algorithm (C. M. Rader, "Discrete Fourier transforms when the number of data samples is prime",
// Proc. IEEE 56(6), 1968): with g a primitive root mod R, a_p = u_{g^p} and b_m = W^{g^-m},
//   X_0 = u_0 + sum_p a_p,   X_{g^-q} = u_0 + (a (*) b)_q   (cyclic convolution of length R - 1),
// and the convolution runs as FFT_{R-1}, a pointwise product with FFT_{R-1}(b) / (R - 1), and an
// unnormalised inverse FFT_{R-1}.  That costs O(R log R) per butterfly instead of O(R^2).
constexpr int kMaxRader = 2;        // distinct Rader primes per plan (three would exceed 4096)
constexpr int kMaxRaderLen = 256;   // R - 1 limit (bounds the LDS tables)
constexpr int kMaxInnerStages = 8;
struct RaderPlan {
  int R, g, ginv;                   // prime, primitive root mod R, its inverse mod R
  int off;                          // byte offset of this prime's tables in the Rader LDS area
  int nst;                          // inner plan of length R - 1 (fixed radices only)
  int radix[kMaxInnerStages];
};
struct FftPlan {
  int L;
  int nst;
  int radix[kMaxStages];
  int nrad;
  RaderPlan rad[kMaxRader];
};

// Tables of one Rader prime (Rm = R - 1 entries each), the same layout in global memory and LDS.
__host__ __device__ constexpr size_t rader_tab_bytes(int R) { return ((size_t)28 * (R - 1) + 15) / 16 * 16; }
// Bytes of LDS a plan's Rader tables need (0 without Rader stages).
__host__ __device__ inline size_t rader_lds_bytes(const FftPlan& plan) {
  size_t b = 0;
  for (int r = 0; r < plan.nrad; ++r) b += rader_tab_bytes(plan.rad[r].R);
  return b;
}
struct RaderTab {
  float2* tw;   // twiddles of the inner length-Rm transforms
  float2* bf;   // FFT_Rm(b) / Rm (forward direction)
  float2* bi;   // FFT_Rm(conj b) / Rm (inverse direction)
  short* gp;    // g^p mod R
  short* gq;    // g^-q mod R
};
__device__ __forceinline__ RaderTab rader_tab(char* base, const RaderPlan& rp) {
  const int Rm = rp.R - 1;
  char* b = base + rp.off;
  RaderTab t;
  t.tw = (float2*)b;
  t.bf = (float2*)(b + 8 * Rm);
  t.bi = (float2*)(b + 16 * Rm);
  t.gp = (short*)(b + 24 * Rm);
  t.gq = (short*)(b + 26 * Rm);
  return t;
}

// One radix-R Stockham pass over `ntr` transforms of length L stored back to back (src -> dst).
// p is the product of the radices already applied.  Output position of butterfly i, leg j is
// (i - k) * R + k + j * p with k = i mod p; leg j is pre-multiplied by exp(-+2 pi i j k / (p R)).
template <int R, bool INV>
__device__ __forceinline__ void stockham_pass(const float2* __restrict__ src, float2* __restrict__ dst, int L, int p,
                              int ntr, const float2* __restrict__ tw, int tid, int nth) {
  const int T = L / R;
  const int twstep = L / (p * R);
  const int total = T * ntr;
  const FastDiv fT = fast_div(T), fp = fast_div(p);
  for (int idx = tid; idx < total; idx += nth) {
    const int t = idx / fT;
    const int i = idx - t * T;
    const int k = i - (i / fp) * p;
    const float2* s = src + t * L;
    float2* d = dst + t * L;
    float2 u[R];
#pragma unroll
    for (int j = 0; j < R; ++j) u[j] = s[i + j * T];
    if (p > 1) {
#pragma unroll
      for (int j = 1; j < R; ++j) u[j] = cmul(u[j], twid<INV>(tw[j * k * twstep]));
    }
    Dft<R, INV>::run(u);
    const int j0 = (i - k) * R + k;
#pragma unroll
    for (int j = 0; j < R; ++j) d[j0 + j * p] = u[j];
  }
}

// Same pass for any radix R (runtime), O(R^2) per butterfly; used for prime factors > 13.
template <bool INV>
__device__ __forceinline__ void stockham_pass_generic(const float2* __restrict__ src, float2* __restrict__ dst, int L,
                                      int R, int p, int ntr, const float2* __restrict__ tw, int tid,
                                      int nth) {
  const int T = L / R;
  const int twstep = L / (p * R);
  const int rstep = L / R;
  const int total = T * ntr;
  const FastDiv fT = fast_div(T), fp = fast_div(p);
  for (int idx = tid; idx < total; idx += nth) {
    const int t = idx / fT;
    const int i = idx - t * T;
    const int k = i - (i / fp) * p;
    const float2* s = src + t * L;
    float2* d = dst + t * L;
    const int j0 = (i - k) * R + k;
    for (int q = 0; q < R; ++q) {
      float2 acc = make_float2(0.f, 0.f);
      int m = 0;  // (j * q) mod R
      for (int j = 0; j < R; ++j) {
        float2 v = s[i + j * T];
        if (j > 0 && p > 1) v = cmul(v, twid<INV>(tw[j * k * twstep]));
        const float2 w = twid<INV>(tw[m * rstep]);
        acc.x = fmaf(v.x, w.x, fmaf(-v.y, w.y, acc.x));
        acc.y = fmaf(v.x, w.y, fmaf(v.y, w.x, acc.y));
        m += q;
        if (m >= R) m -= R;
      }
      d[j0 + q * p] = acc;
    }
  }
}

// A fixed-radix-only plan (the inner transforms of a Rader stage) on `ntr` transforms in a / b.
template <bool INV>
__device__ __forceinline__ float2* fft_fixed(const int* radix, int nst, int L, float2* a, float2* b, int ntr, const float2* tw,
                             int tid, int nth) {
  int p = 1;
  float2* src = a;
  float2* dst = b;
  for (int st = 0; st < nst; ++st) {
    const int R = radix[st];
    switch (R) {
      case 2: stockham_pass<2, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 3: stockham_pass<3, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 4: stockham_pass<4, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 5: stockham_pass<5, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 7: stockham_pass<7, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 8: stockham_pass<8, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      case 11: stockham_pass<11, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
      default: stockham_pass<13, INV>(src, dst, L, p, ntr, tw, tid, nth); break;
    }
    __syncthreads();
    p *= R;
    float2* t = src;
    src = dst;
    dst = t;
  }
  return src;
}

// One radix-R Stockham pass (same input / output placement as stockham_pass) by Rader's algorithm.
// The NB = ntr L / R butterflies each gather their R - 1 non-zero-index legs in generator order
// into dst[b (R-1) + p]; leg 0 goes to the tail dst[NB (R-1) + b].  The inner forward and inverse
// transforms ping-pong between the first NB (R-1) slots of dst and src; with the same number of
// passes each way the convolution always ends in dst, whose tail was never touched, so the
// outputs are scattered into src.  Returns src (the pass does not swap buffers).
template <bool INV>
__device__ __forceinline__ float2* rader_pass(float2* src, float2* dst, int L, int p, int ntr, const float2* tw,
                              const RaderPlan& rp, const RaderTab& rt, int tid, int nth) {
  const int R = rp.R, Rm = R - 1, T = L / R, NB = T * ntr;
  const int twstep = L / (p * R);
  const FastDiv fRm = fast_div(Rm), fR = fast_div(R), fT = fast_div(T), fp = fast_div(p);
  float2* tail = dst + NB * Rm;
  for (int idx = tid; idx < NB * Rm; idx += nth) {
    const int b = idx / fRm, q = idx - b * Rm;
    const int t = b / fT, i = b - t * T;
    const int j = rt.gp[q];
    float2 v = src[t * L + i + j * T];
    if (p > 1) v = cmul(v, twid<INV>(tw[j * (i - (i / fp) * p) * twstep]));
    dst[idx] = v;
    if (q == 0) tail[b] = src[t * L + i];
  }
  __syncthreads();
  float2* F = fft_fixed<false>(rp.radix, rp.nst, Rm, dst, src, NB, rt.tw, tid, nth);
  const float2* bh = INV ? rt.bi : rt.bf;
  for (int idx = tid; idx < NB * Rm; idx += nth) {
    const int b = idx / fRm, m = idx - b * Rm;
    const float2 v = F[idx];
    float2 w = cmul(v, bh[m]);
    if (m == 0) {  // X_0 = u_0 + sum_p a_p; adding u_0 to bin 0 adds it to every convolution output
      const float2 u0 = tail[b];
      tail[b] = cadd(u0, v);
      w = cadd(w, u0);
    }
    F[idx] = w;
  }
  __syncthreads();
  const float2* C = fft_fixed<true>(rp.radix, rp.nst, Rm, F, F == dst ? src : dst, NB, rt.tw, tid, nth);
  for (int idx = tid; idx < NB * R; idx += nth) {
    const int b = idx / fR, r = idx - b * R;
    const int t = b / fT, i = b - t * T;
    const int k = i - (i / fp) * p;
    const int n = r == 0 ? 0 : rt.gq[r - 1];
    src[t * L + (i - k) * R + k + n * p] = r == 0 ? tail[b] : C[b * Rm + r - 1];
  }
  __syncthreads();
  return src;
}

__device__ __forceinline__ int powmod_dev(int g, int e, int m) {  // g^e mod m, binary exponentiation
  int r = 1 % m, b = g % m;
  while (e > 0) {
    if (e & 1) r = (r * b) % m;
    b = (b * b) % m;
    e >>= 1;
  }
  return r;
}

// ---- plan tables: the twiddles exp(-2 pi i m / L), m < L (fp64-evaluated, rounded once), then the
// Rader tables of each Rader prime.  Built once per geometry into global memory by build_plan_tabs
// and copied into LDS by each block with load_plan_tabs.
__host__ __device__ inline size_t plan_tw_bytes(const FftPlan& plan) { return ((size_t)8 * plan.L + 15) / 16 * 16; }
__host__ __device__ inline size_t plan_tab_bytes(const FftPlan& plan) {
  return plan_tw_bytes(plan) + rader_lds_bytes(plan);
}

// One block writes the plan's tables to `g` (16-byte aligned).  `wd` / `bd` are fp64 scratch of
// kMaxRaderLen entries each (LDS).  All threads of the block call it.
__device__ void build_plan_tabs(const FftPlan& plan, char* g, double2* wd, double2* bd, int tid, int nth) {
  float2* tw = (float2*)g;
  for (int m = tid; m < plan.L; m += nth) {
    double sn, cs;
    sincospi(-2.0 * (double)m / (double)plan.L, &sn, &cs);
    tw[m] = make_float2((float)cs, (float)sn);
  }
  char* rbase = g + plan_tw_bytes(plan);
  for (int r = 0; r < plan.nrad; ++r) {
    const RaderPlan& rp = plan.rad[r];
    const RaderTab t = rader_tab(rbase, rp);
    const int Rm = rp.R - 1;
    __syncthreads();  // wd / bd reuse across primes
    for (int m = tid; m < Rm; m += nth) {
      const int gq = powmod_dev(rp.ginv, m, rp.R);
      t.gp[m] = (short)powmod_dev(rp.g, m, rp.R);
      t.gq[m] = (short)gq;
      double sn, cs;
      sincospi(-2.0 * (double)m / (double)Rm, &sn, &cs);
      wd[m] = make_double2(cs, sn);
      t.tw[m] = make_float2((float)cs, (float)sn);
      sincospi(-2.0 * (double)gq / (double)rp.R, &sn, &cs);
      bd[m] = make_double2(cs, sn);
    }
    __syncthreads();
    for (int m = tid; m < Rm; m += nth) {
      double fr = 0.0, fi = 0.0, ir = 0.0, ii = 0.0;
      int e = 0;  // (q m) mod Rm
      for (int q = 0; q < Rm; ++q) {
        const double2 b = bd[q], w = wd[e];
        fr += b.x * w.x - b.y * w.y;
        fi += b.x * w.y + b.y * w.x;
        ir += b.x * w.x + b.y * w.y;  // conj(b) w
        ii += b.x * w.y - b.y * w.x;
        e += m;
        if (e >= Rm) e -= Rm;
      }
      const double sc = 1.0 / (double)Rm;
      t.bf[m] = make_float2((float)(fr * sc), (float)(fi * sc));
      t.bi[m] = make_float2((float)(ir * sc), (float)(ii * sc));
    }
  }
}

// Copies the plan's tables from global `g` into the block's LDS: twiddles to `tw`, Rader tables to
// `rader`.  All threads call it; the caller synchronises before use.
__device__ __forceinline__ void load_plan_tabs(const FftPlan& plan, const char* g, float2* tw, char* rader, int tid,
                                               int nth) {
  const float2* gt = (const float2*)g;
  for (int m = tid; m < plan.L; m += nth) tw[m] = gt[m];
  const int nr = (int)(rader_lds_bytes(plan) / 16);
  const float4* gr = (const float4*)(g + plan_tw_bytes(plan));
  for (int i = tid; i < nr; i += nth) ((float4*)rader)[i] = gr[i];
}

// Runs the whole plan on `ntr` transforms held in buffer a (workspace b of equal size).  Returns
// the buffer holding the result.  All threads of the block must call it; it synchronises.
// `rader` is the plan's Rader LDS area (filled by load_plan_tabs), or null when plan.nrad == 0.
template <bool INV>
__device__ __forceinline__ float2* fft_lds(const FftPlan& plan, float2* a, float2* b, int ntr, const float2* tw,
                           int tid, int nth, char* rader = nullptr) {
  int p = 1;
  float2* src = a;
  float2* dst = b;
  for (int st = 0; st < plan.nst; ++st) {
    const int R = plan.radix[st];
    int ri = -1;
    for (int r = 0; r < plan.nrad; ++r)
      if (plan.rad[r].R == R) ri = r;
    if (ri >= 0) {
      rader_pass<INV>(src, dst, plan.L, p, ntr, tw, plan.rad[ri], rader_tab(rader, plan.rad[ri]), tid, nth);
      p *= R;
      continue;  // result stays in src
    }
    switch (R) {
      case 2: stockham_pass<2, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 3: stockham_pass<3, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 4: stockham_pass<4, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 5: stockham_pass<5, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 7: stockham_pass<7, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 8: stockham_pass<8, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 11: stockham_pass<11, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      case 13: stockham_pass<13, INV>(src, dst, plan.L, p, ntr, tw, tid, nth); break;
      default: stockham_pass_generic<INV>(src, dst, plan.L, R, p, ntr, tw, tid, nth); break;
    }
    __syncthreads();
    p *= R;
    float2* t = src;
    src = dst;
    dst = t;
  }
  return src;
}

// The fixed-radix decomposition of a compile-time length L: the odd radices first, largest first
// (13, 11, 7, 5, 3), then 8s and 4 / 2 for the power of two; count 0 when L has another factor.
// Measured on the 260-point passes of the backward (13, 5, 4 against 4, 5, 13): the column pass
// 452 -> 398 us (LDS bank conflicts 2.0 -> 1.6 cycles per LDS instruction: the first pass writes
// each butterfly's R outputs to R consecutive elements, which an odd R spreads over more banks),
// the row passes 170 -> 167 and 172 -> 165 us (fewer instructions).
struct FixedRadices {
  int n;
  int r[kMaxStages];
};
constexpr FixedRadices fixed_radices_ct(int L) {
  FixedRadices f{0, {}};
  const int odd[5] = {13, 11, 7, 5, 3};
  for (int i = 0; i < 5; ++i)
    while (L % odd[i] == 0 && f.n < kMaxStages) { f.r[f.n++] = odd[i]; L /= odd[i]; }
  while (L % 8 == 0 && f.n < kMaxStages) { f.r[f.n++] = 8; L /= 8; }
  while (L % 4 == 0 && f.n < kMaxStages) { f.r[f.n++] = 4; L /= 4; }
  while (L % 2 == 0 && f.n < kMaxStages) { f.r[f.n++] = 2; L /= 2; }
  if (L != 1) f.n = 0;
  return f;
}

// fft_lds on a compile-time length L (fixed radices only): every pass's radix, stride and twiddle
// step is a constant, so each kernel carries only the butterflies its length uses.  Same twiddle
// table (exp(-2 pi i m / L), m < L) as fft_lds; the result lands in a when the pass count is even,
// in b when it is odd.
template <int L, int ST, bool INV>
__device__ __forceinline__ float2* fft_fixed_ct(float2* a, float2* b, int ntr, const float2* tw, int tid, int nth) {
  constexpr FixedRadices f = fixed_radices_ct(L);
  static_assert(f.n > 0, "length without a fixed-radix plan");
  if constexpr (ST == f.n) {
    return a;
  } else {
    constexpr int R = f.r[ST];
    constexpr int P = [] {
      int p = 1;
      for (int i = 0; i < ST; ++i) p *= fixed_radices_ct(L).r[i];
      return p;
    }();
    stockham_pass<R, INV>(a, b, L, P, ntr, tw, tid, nth);
    __syncthreads();
    return fft_fixed_ct<L, ST + 1, INV>(b, a, ntr, tw, tid, nth);
  }
}

}  // namespace cvn
