// Converse2D forward, generic multi-pass path (any plane size up to kMaxFftLen per dimension).
//
// Algorithm (per (b, c) plane; notation: y = padded input (h x w), s = scale, Hs = h s, Ws = w s,
// K = OTF of the psf at (Hs, Ws), lambda = sigmoid(bias - 9) + eps):
//   * module path (util_converse.py:142-192, x0 = nearest(y)):
//       X = Phi * tile_s(F_hw(y)),   out = crop(Re F^-1_{Hs Ws}(X))
//     with Phi = Hn + conj(K) (1 - M(K Hn)) / (M(|K|^2) + lambda), Hn the nearest-hold response
//     sum_{a<s} exp(-2 pi i u a / Hs) per axis and M the mean over the s*s alias group of a bin.
//     This is the reference solve (FR - FBC*invWBR)/lambda rewritten without the division by
//     lambda, which cancels exactly; Phi is evaluated in fp64 once per channel (or per sample).
//   * op path (converse2d.cpp:165-209, arbitrary x0):
//       X = X0 + conj(K) (tile_s(F(y)) - M(K X0)) / (M(|K|^2) + lambda),   out = Re F^-1(X).
//
// Kernels:
//   k_phi_module / k_phi_op : transfer tables in fp64 (one block per channel column class)
//   k_rows_fwd               : padding on load, R2C along rows (two real rows per complex FFT),
//                              writes the half spectrum column-major  S[plane][col][row]
//   k_cols_module            : per HR column: LR column FFT, tile, * Phi, inverse HR column FFT
//   k_cols_op                : per alias class: LR and x0 column FFTs, alias-group solve, inverse
//   k_rows_inv               : C2R along rows (two rows per complex FFT), crop + activation on store
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "cvn_common.h"

namespace cvn {

// ------------------------------------------------------------------------------------------------
// padding index map (F.pad semantics); returns -1 for a zero sample
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ int pad_src(int i, int n, int p, int mode) {
  int j = i - p;
  if (j >= 0 && j < n) return j;
  switch (mode) {
    case CVN_PAD_CIRCULAR: j %= n; return j < 0 ? j + n : j;
    case CVN_PAD_REPLICATE: return j < 0 ? 0 : n - 1;
    case CVN_PAD_REFLECT: return j < 0 ? -j : 2 * (n - 1) - j;
    default: return -1;
  }
}

__device__ __forceinline__ float gelu_exact(float v) { return gelu_fast(v); }

// Border sample q in [0, 2 pad) of a padded axis with n interior samples: padded index q (q < pad)
// or n + q (the far border).
__device__ __forceinline__ int border_idx(int q, int n, int pad) { return q < pad ? q : n + q; }

// Global-memory loops issue kBatch independent loads per thread before using any of them, so each
// wave keeps many requests in flight (a plain loop waits out the full memory latency per element).
constexpr int kBatch = 8;

__device__ __forceinline__ double2 dcmul(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ double2 dexpi(double num, double den) {  // exp(-2 pi i num / den)
  double sn, cs;
  sincospi(-2.0 * num / den, &sn, &cs);
  return make_double2(cs, sn);
}

// ------------------------------------------------------------------------------------------------
// Transfer tables (fp64 arithmetic).  One block per (psf plane, LR column class v0); threads over
// the LR row class u0.  Members of a class: (u0 + a h, v0 + b w), a, b in [0, s).
// ------------------------------------------------------------------------------------------------
struct PhiArgs {
  const float* psf;   // (Cp, kh, kw)
  const float* bias;  // (C)
  int64_t Cp;
  int C, kh, kw, s, h, w, Hs, Ws, NCs;
  int nv0;            // number of column classes handled
  double eps;
  float2* phi;        // module: (Cp, NCs, Hs);  op: A (Cp, Ws, Hs)
  float2* kf;         // op only: K (Cp, Ws, Hs)
  int layout;         // module form: kPhiGeneric (Cp, NCs, Hs), kPhiPfa268 (pfa268_phi_index) or kPhiFused256
};
// Output layouts of the module-form tables.
constexpr int kPhiGeneric = 0, kPhiPfa268 = 1, kPhiFused256 = 2;
__device__ __forceinline__ int64_t phi_out_index(const PhiArgs& a, int64_t cp, int64_t vb, int u) {
  if (a.layout == kPhiPfa268) return pfa268_phi_index(cp, (int)vb, u);
  if (a.layout == kPhiFused256) return fused256_phi_index(cp, (int)vb, u);
  return (cp * a.NCs + vb) * a.Hs + u;
}

// P[b][i] = sum_j psf[i][j] exp(-2 pi i v_b (j - kw/2) / Ws), into LDS.
__device__ void phi_row_sums(const PhiArgs& a, const float* psf, int v0, double2* P) {
  const int n = a.s * a.kh;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int b = e / a.kh, i = e - b * a.kh;
    const int64_t vb = v0 + (int64_t)b * a.w;
    double2 acc = make_double2(0.0, 0.0);
    const double2 r = dexpi((double)vb, (double)a.Ws);
    double2 ph = dexpi(-(double)(vb * (a.kw / 2) % a.Ws), (double)a.Ws);  // exp(+2 pi i vb cw / Ws)
    for (int j = 0; j < a.kw; ++j) {
      const double t = (double)psf[i * a.kw + j];
      acc.x += t * ph.x;
      acc.y += t * ph.y;
      ph = dcmul(ph, r);
    }
    P[e] = acc;
  }
}

// K(u_a, v_b) = sum_i exp(-2 pi i u_a (i - kh/2) / Hs) P[b][i]
__device__ __forceinline__ double2 phi_otf(const PhiArgs& a, const double2* P, int b, int64_t ua) {
  const double2 r = dexpi((double)ua, (double)a.Hs);
  double2 e = dexpi(-(double)(ua * (a.kh / 2) % a.Hs), (double)a.Hs);
  double2 acc = make_double2(0.0, 0.0);
  const double2* Pb = P + b * a.kh;
  for (int i = 0; i < a.kh; ++i) {
    const double2 t = dcmul(e, Pb[i]);
    acc.x += t.x;
    acc.y += t.y;
    e = dcmul(e, r);
  }
  return acc;
}

// sum_{t<s} exp(-2 pi i u t / N)
__device__ __forceinline__ double2 hold(int s, int64_t u, int N) {
  double2 acc = make_double2(1.0, 0.0);
  for (int t = 1; t < s; ++t) {
    const double2 e = dexpi((double)((u * t) % N), (double)N);
    acc.x += e.x;
    acc.y += e.y;
  }
  return acc;
}

__device__ __forceinline__ double lambda_of(const PhiArgs& a, int c) {
  const double b = (double)a.bias[c] - 9.0;
  return 1.0 / (1.0 + exp(-b)) + a.eps;
}

__global__ void k_phi_module(PhiArgs a) {
  extern __shared__ double2 Psm[];
  const int64_t cp = blockIdx.x / a.nv0;
  const int v0 = (int)(blockIdx.x - cp * a.nv0);
  const int c = (int)(cp % a.C);
  phi_row_sums(a, a.psf + cp * a.kh * a.kw, v0, Psm);
  __syncthreads();
  const double lmb = lambda_of(a, c);
  const double inv_s2 = 1.0 / ((double)a.s * a.s);
  const double norm = 1.0 / ((double)a.Hs * (double)a.Ws);
  for (int u0 = threadIdx.x; u0 < a.h; u0 += blockDim.x) {
    double2 mkh = make_double2(0.0, 0.0);
    double mk2 = 0.0;
    for (int b = 0; b < a.s; ++b) {
      const int64_t vb = v0 + (int64_t)b * a.w;
      const double2 hv = hold(a.s, vb, a.Ws);
      for (int aa = 0; aa < a.s; ++aa) {
        const int64_t ua = u0 + (int64_t)aa * a.h;
        const double2 K = phi_otf(a, Psm, b, ua);
        const double2 hn = dcmul(hold(a.s, ua, a.Hs), hv);
        const double2 kh = dcmul(K, hn);
        mkh.x += kh.x;
        mkh.y += kh.y;
        mk2 += K.x * K.x + K.y * K.y;
      }
    }
    mkh.x *= inv_s2;
    mkh.y *= inv_s2;
    const double D = mk2 * inv_s2 + lmb;
    const double2 g = make_double2((1.0 - mkh.x) / D, -mkh.y / D);  // (1 - M(K Hn)) / D
    for (int b = 0; b < a.s; ++b) {
      const int64_t vb = v0 + (int64_t)b * a.w;
      if (vb > a.Ws / 2) continue;
      const double2 hv = hold(a.s, vb, a.Ws);
      for (int aa = 0; aa < a.s; ++aa) {
        const int64_t ua = u0 + (int64_t)aa * a.h;
        const double2 K = phi_otf(a, Psm, b, ua);
        const double2 hn = dcmul(hold(a.s, ua, a.Hs), hv);
        const double2 t = dcmul(make_double2(K.x, -K.y), g);
        const double2 ph = make_double2((hn.x + t.x) * norm, (hn.y + t.y) * norm);
        a.phi[(cp * a.NCs + vb) * a.Hs + ua] = make_float2((float)ph.x, (float)ph.y);
      }
    }
  }
}

// op-path tables over the full width: kf = K, phi = conj(K) / (M(|K|^2) + lambda) / (Hs Ws)
__global__ void k_phi_op(PhiArgs a) {
  extern __shared__ double2 Psm[];
  const int64_t cp = blockIdx.x / a.nv0;
  const int v0 = (int)(blockIdx.x - cp * a.nv0);
  const int c = (int)(cp % a.C);
  phi_row_sums(a, a.psf + cp * a.kh * a.kw, v0, Psm);
  __syncthreads();
  const double lmb = lambda_of(a, c);
  const double inv_s2 = 1.0 / ((double)a.s * a.s);
  const double norm = 1.0 / ((double)a.Hs * (double)a.Ws);
  for (int u0 = threadIdx.x; u0 < a.h; u0 += blockDim.x) {
    double mk2 = 0.0;
    for (int b = 0; b < a.s; ++b)
      for (int aa = 0; aa < a.s; ++aa) {
        const double2 K = phi_otf(a, Psm, b, u0 + (int64_t)aa * a.h);
        mk2 += K.x * K.x + K.y * K.y;
      }
    const double Dinv = norm / (mk2 * inv_s2 + lmb);
    for (int b = 0; b < a.s; ++b) {
      const int64_t vb = v0 + (int64_t)b * a.w;
      for (int aa = 0; aa < a.s; ++aa) {
        const int64_t ua = u0 + (int64_t)aa * a.h;
        const double2 K = phi_otf(a, Psm, b, ua);
        const int64_t o = (cp * a.Ws + vb) * a.Hs + ua;
        a.kf[o] = make_float2((float)K.x, (float)K.y);
        a.phi[o] = make_float2((float)(K.x * Dinv), (float)(-K.y * Dinv));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Transfer tables, block-tiled form (module and op tables), scale S <= 4.  One block per (psf plane,
// chunk of vc consecutive LR column classes v0).  The block first builds, in LDS and in fp64,
// z_u = exp(-2 pi i u / Hs), the centring phase exp(+2 pi i u ch / Hs) and the hold response of
// every HR row u, the same three quantities for the chunk's HR columns vb = v0 + b w, and the psf
// row sums P[v][b][i] = sum_j psf[i][j] exp(-2 pi i vb (j - cw) / Ws).  Then one thread per alias
// class (u0, v0) evaluates the S*S members' K = phase_u * sum_i P[v][b][i] z_u^i (Horner's rule as
// four interleaved chains in z^4, four fp64 FMAs per psf row), keeps them in registers for the
// class sums, and writes the class's table entries (coalesced along u).  Same quantities and
// formulas as k_phi_module / k_phi_op.
// ------------------------------------------------------------------------------------------------
struct PhiTileLds {
  int zH, phH, hH, zW, phW, hW, P, psf, part, total;  // byte offsets
  // split-DFT form: column twiddles, fp64 psf, row twiddles per row residue, shifted psf-row sums
  int tw, psd, tr, Pt;
  int PS, NTh, Ch;  // row stride (entries) of tr and Pt, 16-row tap groups, row shift 16 Ch - kh / 2
};
__host__ __device__ inline int round4(int n) { return (n + 3) & ~3; }
// The split-DFT evaluation of the tables (phi_tile_rows16) applies: scale 1, 2 or 4, HR height a
// multiple of 16, all S (Hs / 16) row threads of an alias-class column in one block, and not the 268
// path's layout.
__host__ __device__ inline bool phi_rows16(int s, int Hs, bool q268) {
  return !q268 && (s == 1 || s == 2 || s == 4) && Hs % 16 == 0 && s * (Hs / 16) <= 256;
}
__host__ __device__ inline PhiTileLds phi_tile_lds(int s, int Hs, int kh, int kw, int vc, bool fast = false) {
  PhiTileLds L = {};
  int o = 0;
  if (fast) {
    // split-DFT form.  psf row i sits at shifted row index i' = i - kh / 2 + 16 Ch in [0, 16 NTh), so
    // that i' mod 16 is the residue of the centred row offset.  The first three regions are dead once
    // the psf-row sums are formed, and the class partial sums (s > 1) reuse them.
    const int ne = vc * s, ch = kh / 2;
    L.Ch = (ch + 15) / 16;
    L.NTh = (16 * L.Ch - ch + kh + 15) / 16;
    L.PS = 16 * L.NTh + 1;  // odd stride: the 16 row residues' and 4 members' reads spread over the banks
    L.zH = o; o += Hs * 16;
    L.tw = o; o += ne * kw * 16;
    L.psd = o; o += kw * ((kh + 1) & ~1) * 8;
    o = (o + 15) & ~15;
    L.part = 0;
    o = (s > 1 && vc * Hs * 24 > o) ? vc * Hs * 24 : o;
    o = (o + 15) & ~15;
    L.hH = o; o += (s > 1 ? Hs : 0) * 16;
    L.hW = o; o += ne * 16;
    L.tr = o; o += (Hs / 16) * L.PS * 16;
    L.Pt = o; o += ne * L.PS * 16;
    L.total = (o + 15) & ~15;
    return L;
  }
  L.zH = o; o += Hs * 16;
  L.phH = o; o += Hs * 16;
  L.hH = o; o += (s > 1 ? Hs : 0) * 16;
  L.zW = o; o += vc * s * 16;
  L.phW = o; o += vc * s * 16;
  L.hW = o; o += vc * s * 16;
  L.P = o; o += vc * s * round4(kh) * 16;
  L.psf = o; o += kh * round4(kw) * 4;
  L.total = (o + 15) & ~15;
  return L;
}

// c z + p
__device__ __forceinline__ double2 cmadd(double2 c, double2 z, double2 p) {
  return make_double2(fma(c.x, z.x, fma(-c.y, z.y, p.x)), fma(c.x, z.y, fma(c.y, z.x, p.y)));
}

// sum_{i<n4} P[i] z^i, n4 a multiple of 4: four independent Horner chains in z^4, then Horner in z
__device__ __forceinline__ double2 horner4(const double2* P, int n4, double2 z) {
  const double2 z2 = dcmul(z, z), z4 = dcmul(z2, z2);
  double2 c0 = P[n4 - 4], c1 = P[n4 - 3], c2 = P[n4 - 2], c3 = P[n4 - 1];
  for (int i = n4 - 8; i >= 0; i -= 4) {
    c0 = cmadd(c0, z4, P[i]);
    c1 = cmadd(c1, z4, P[i + 1]);
    c2 = cmadd(c2, z4, P[i + 2]);
    c3 = cmadd(c3, z4, P[i + 3]);
  }
  return cmadd(cmadd(cmadd(c3, z, c2), z, c1), z, c0);
}

// Per-block LDS tables of the tiled transfer-table kernels (k_phi_tile, k_phi_grad): row tables for
// every HR row, column tables for the chunk's HR columns vbeg + v + b w (v < nv, b < S), and the psf
// row sums P[(v S + b) kh4 + i] (rows zero-padded to kh4).  The split-DFT form (phi_split_prep) fills
// hH, hW, tr and Pt instead.
struct PhiTileView {
  double2 *zH, *phH, *hH, *zW, *phW, *hW, *P;
  double2 *tr, *Pt;
  int PS, NTh;
};
template <int S>
__device__ PhiTileView phi_tile_prep(const PhiArgs& a, unsigned char* phl, int64_t cp, int vbeg, int nv, int vc) {
  const int tid = threadIdx.x, nth = blockDim.x;
  const int Hs = a.Hs, Ws = a.Ws, kh = a.kh, kw = a.kw;
  const int kh4 = round4(kh), kw4 = round4(kw);
  const PhiTileLds L = phi_tile_lds(S, Hs, kh, kw, vc);
  PhiTileView t = {};
  t.zH = (double2*)(phl + L.zH);
  t.phH = (double2*)(phl + L.phH);
  t.hH = (double2*)(phl + L.hH);
  t.zW = (double2*)(phl + L.zW);
  t.phW = (double2*)(phl + L.phW);
  t.hW = (double2*)(phl + L.hW);
  t.P = (double2*)(phl + L.P);
  float* ps = (float*)(phl + L.psf);

  // the psf's first kPsfRegs words per thread are requested here and written to LDS after the
  // twiddle tables below, which do not depend on them, so the load latency overlaps their sincos work
  constexpr int kPsfRegs = 4;
  const float* psf = a.psf + cp * kh * kw;
  float pv[kPsfRegs];
#pragma unroll
  for (int r = 0; r < kPsfRegs; ++r) {
    const int e = tid + r * nth, i = e / kw4, j = e - i * kw4;
    pv[r] = (e < kh * kw4 && j < kw) ? psf[i * kw + j] : 0.f;
  }
  for (int u = tid; u < Hs; u += nth) {
    t.zH[u] = dexpi((double)u, (double)Hs);
    t.phH[u] = dexpi(-(double)(((int64_t)u * (kh / 2)) % Hs), (double)Hs);
    if (S > 1) t.hH[u] = hold(S, u, Hs);
  }
  for (int e = tid; e < nv * S; e += nth) {
    const int v = e / S, b = e - v * S;
    const int64_t vb = vbeg + v + (int64_t)b * a.w;
    t.zW[e] = dexpi((double)vb, (double)Ws);
    t.phW[e] = dexpi(-(double)((vb * (kw / 2)) % Ws), (double)Ws);
    t.hW[e] = hold(S, vb, Ws);
  }
#pragma unroll
  for (int r = 0; r < kPsfRegs; ++r)
    if (tid + r * nth < kh * kw4) ps[tid + r * nth] = pv[r];
  for (int e = tid + kPsfRegs * nth; e < kh * kw4; e += nth) {
    const int i = e / kw4, j = e - i * kw4;
    ps[e] = j < kw ? psf[i * kw + j] : 0.f;
  }
  __syncthreads();
  // row sums (real coefficients, same four-chain Horner); rows zero-padded to kh4
  for (int e = tid; e < nv * S * kh4; e += nth) {
    const int vbq = e / kh4, i = e - vbq * kh4;
    double2 acc = make_double2(0.0, 0.0);
    if (i < kh) {
      const double2 z = t.zW[vbq], z2 = dcmul(z, z), z4 = dcmul(z2, z2);
      const float* row = ps + i * kw4;
      double2 q[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) q[r] = make_double2((double)row[kw4 - 4 + r], 0.0);
      for (int j = kw4 - 8; j >= 0; j -= 4)
#pragma unroll
        for (int r = 0; r < 4; ++r) q[r] = cmadd(q[r], z4, make_double2((double)row[j + r], 0.0));
      acc = dcmul(cmadd(cmadd(cmadd(q[3], z, q[2]), z, q[1]), z, q[0]), t.phW[vbq]);
    }
    t.P[e] = acc;
  }
  __syncthreads();
  return t;
}

// exp(-2 pi i k / N) table index of k mod N (k may be negative); N a power of two needs no division
__device__ __forceinline__ int mod_n(int k, int N, bool pow2) {
  if (pow2) return k & (N - 1);
  k %= N;
  return k < 0 ? k + N : k;
}

// Tables of the split-DFT form, in three phases separated by barriers:
//  1. the psf in fp64, transposed (row index fastest, rows padded to an even count), and z^u = exp(-2 pi
//     i u / Hs) for every HR row (a quarter by sincospi, the rest by the exact rotations by -i, -1, i);
//     hold sums of the chunk's columns (S > 1);
//  2. column twiddles tw[m][j] = z_W^(vb (j - kw/2)) for the chunk's column members m = v S + b,
//     row twiddles tr[u1][i'] = z^(u1 (i' - 16 Ch)) per row residue u1 < Hs / 16, hold sums of every
//     HR row (S > 1), and zeroed psf-row sums;
//  3. the psf-row sums Pt[m][i'] = sum_j psf[i][j] tw[m][j] at the shifted row index
//     i' = i - kh/2 + 16 Ch (real times complex: two fp64 FMAs per tap; each task forms two rows).
// The 2-D fills give each thread one column c = tid mod C and the rows tid / C + k (nth / C), so a
// thread divides once per table rather than once per element (integer division is a ~30-instruction
// sequence here); the host guarantees kw <= nth and 16 NTh <= nth.
template <int S>
__device__ PhiTileView phi_split_prep(const PhiArgs& a, unsigned char* phl, int64_t cp, int vbeg, int nv, int vc) {
  const int tid = threadIdx.x, nth = blockDim.x;
  const int Hs = a.Hs, Ws = a.Ws, kh = a.kh, kw = a.kw, H1 = Hs >> 4;
  const int ch = kh / 2, cw = kw / 2, kh2 = (kh + 1) & ~1, nI = kh2 >> 1;
  const bool h2 = (Hs & (Hs - 1)) == 0, w2 = (Ws & (Ws - 1)) == 0;
  const PhiTileLds L = phi_tile_lds(S, Hs, kh, kw, vc, true);
  const int PS = L.PS, Ch = L.Ch, NT16 = 16 * L.NTh, nm = nv * S;
  PhiTileView t = {};
  double2* zH = (double2*)(phl + L.zH);
  double2* tw = (double2*)(phl + L.tw);
  double* psd = (double*)(phl + L.psd);
  t.hH = (double2*)(phl + L.hH);
  t.hW = (double2*)(phl + L.hW);
  t.tr = (double2*)(phl + L.tr);
  t.Pt = (double2*)(phl + L.Pt);
  t.PS = PS;
  t.NTh = L.NTh;
  // psf columns: thread column j = cj of rows rj, rj + sj, ... (threads past sj kw idle)
  const int rj = tid / kw, cj = tid - rj * kw, sj = nth / kw;
  const bool aj = rj < sj;

  // the psf's first kPsfRegs rows per thread are requested before the sincos work of the row table,
  // which does not depend on them, so the load latency overlaps it
  constexpr int kPsfRegs = 4;
  const float* psf = a.psf + cp * kh * kw;
  float pv[kPsfRegs];
#pragma unroll
  for (int r = 0; r < kPsfRegs; ++r) {
    const int i = rj + r * sj;
    pv[r] = aj && i < kh ? psf[i * kw + cj] : 0.f;
  }
  const int Q = Hs >> 2;
  for (int u = tid; u < Q; u += nth) {
    const double2 z = dexpi((double)u, (double)Hs);
    zH[u] = z;
    zH[u + Q] = make_double2(z.y, -z.x);
    zH[u + 2 * Q] = make_double2(-z.x, -z.y);
    zH[u + 3 * Q] = make_double2(-z.y, z.x);
  }
  if (S > 1)
    for (int m = tid; m < nm; m += nth) {
      const int v = m / S, b = m - v * S;
      t.hW[m] = hold(S, vbeg + v + (int64_t)b * a.w, Ws);
    }
  if (aj) {
    double* col = psd + cj * kh2;
#pragma unroll
    for (int r = 0; r < kPsfRegs; ++r)
      if (rj + r * sj < kh) col[rj + r * sj] = (double)pv[r];
    for (int i = rj + kPsfRegs * sj; i < kh; i += sj) col[i] = (double)psf[i * kw + cj];
    if (kh2 > kh && rj == 0) col[kh] = 0.0;
  }
  __syncthreads();

  if (aj)
    for (int m = rj; m < nm; m += sj) {
      const int v = m / S, b = m - v * S;
      const int k = mod_n((vbeg + v + b * a.w) * (cj - cw), Ws, w2);
      tw[m * kw + cj] = Ws == Hs ? zH[k] : dexpi((double)k, (double)Ws);
    }
  {
    const int ri = tid / NT16, ci = tid - ri * NT16, si = nth / NT16;
    if (ri < si)
      for (int u1 = ri; u1 < H1; u1 += si) t.tr[u1 * PS + ci] = zH[mod_n(u1 * (ci - 16 * Ch), Hs, h2)];
  }
  if (S > 1)
    for (int u = tid; u < Hs; u += nth) {  // hold sum sum_{t<S} z^(u t)
      double2 acc = make_double2(1.0, 0.0);
      int m = 0;
      for (int q = 1; q < S; ++q) {
        m += u;
        m -= m >= Hs ? Hs : 0;
        acc.x += zH[m].x;
        acc.y += zH[m].y;
      }
      t.hH[u] = acc;
    }
  for (int e = tid; e < nm * PS; e += nth) t.Pt[e] = make_double2(0.0, 0.0);
  __syncthreads();

  const double2* psd2 = (const double2*)psd;  // rows (2 r, 2 r + 1) of column j at psd2[j nI + r]
  const int rm = tid / nI, r = tid - rm * nI, sm = nth / nI;
  if (rm < sm)
    for (int m = rm; m < nm; m += sm) {
      const double2* twm = tw + m * kw;
      double2 a0 = make_double2(0.0, 0.0), a1 = make_double2(0.0, 0.0);
#pragma unroll 5
      for (int j = 0; j < kw; ++j) {
        const double2 p = psd2[j * nI + r], z = twm[j];
        a0.x = fma(p.x, z.x, a0.x);
        a0.y = fma(p.x, z.y, a0.y);
        a1.x = fma(p.y, z.x, a1.x);
        a1.y = fma(p.y, z.y, a1.y);
      }
      double2* Pm = t.Pt + m * PS + 2 * r - ch + 16 * Ch;
      Pm[0] = a0;
      if (2 * r + 1 < kh) Pm[1] = a1;
    }
  __syncthreads();
  return t;
}

// 16-point DFT in place, X[k] = sum_i x[i] exp(-2 pi i i k / 16), fp64: radix 4 x 4 (decimation in
// time: i = i0 + 4 i1, k = k0 + 4 k1; four 4-point DFTs over i1, twiddles w16^(i0 k0), four 4-point
// DFTs over i0).  Twiddle constants cos / sin (2 pi m / 16), m = i0 k0 <= 9.
__device__ __forceinline__ void ddft4(double2& x0, double2& x1, double2& x2, double2& x3) {
  const double2 a0 = make_double2(x0.x + x2.x, x0.y + x2.y), a1 = make_double2(x0.x - x2.x, x0.y - x2.y);
  const double2 b0 = make_double2(x1.x + x3.x, x1.y + x3.y), b1 = make_double2(x1.x - x3.x, x1.y - x3.y);
  x0 = make_double2(a0.x + b0.x, a0.y + b0.y);
  x2 = make_double2(a0.x - b0.x, a0.y - b0.y);
  x1 = make_double2(a1.x + b1.y, a1.y - b1.x);  // a1 - i b1
  x3 = make_double2(a1.x - b1.y, a1.y + b1.x);  // a1 + i b1
}
// First half of the 16-point DFT: the four 4-point DFTs over i1 and the twiddles w16^(i0 k0); the
// output X[k0 + 4 k1] is then ddft4 of x[4 k0 .. 4 k0 + 3], element k1.
__device__ __forceinline__ void ddft16_first(double2 (&x)[16]) {
  constexpr double kC[10] = {1.0, 0.92387953251128674, 0.70710678118654752, 0.38268343236508977, 0.0,
                             -0.38268343236508977, -0.70710678118654752, -0.92387953251128674, -1.0,
                             -0.92387953251128674};
  constexpr double kS[10] = {0.0, 0.38268343236508977, 0.70710678118654752, 0.92387953251128674, 1.0,
                             0.92387953251128674, 0.70710678118654752, 0.38268343236508977, 0.0,
                             -0.38268343236508977};
#pragma unroll
  for (int i0 = 0; i0 < 4; ++i0) ddft4(x[i0], x[i0 + 4], x[i0 + 8], x[i0 + 12]);  // y[i0][k0] in x[i0 + 4 k0]
#pragma unroll
  for (int i0 = 1; i0 < 4; ++i0)
#pragma unroll
    for (int k0 = 1; k0 < 4; ++k0) {
      const int m = i0 * k0;
      const double2 v = x[i0 + 4 * k0];  // times exp(-2 pi i m / 16) = (cos, -sin)
      x[i0 + 4 * k0] = m == 4 ? make_double2(v.y, -v.x)
                              : make_double2(v.x * kC[m] + v.y * kS[m], v.y * kC[m] - v.x * kS[m]);
    }
}
__device__ __forceinline__ void ddft16(double2 (&x)[16]) {
  ddft16_first(x);
#pragma unroll
  for (int k0 = 0; k0 < 4; ++k0) ddft4(x[4 * k0], x[4 * k0 + 1], x[4 * k0 + 2], x[4 * k0 + 3]);  // X[k0 + 4 k1] in x[4 k0 + k1]
  double2 t[16];
#pragma unroll
  for (int k0 = 0; k0 < 4; ++k0)
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) t[k0 + 4 * k1] = x[4 * k0 + k1];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = t[k];
}

// 1 / d in fp64 from the hardware reciprocal estimate and two Newton steps (relative error at the
// level of fp64 rounding; the table entries are rounded to fp32 afterwards).
__device__ __forceinline__ double drcp(double d) {
  double r = __builtin_amdgcn_rcp(d);
  r = fma(r, fma(-d, r, 1.0), r);
  r = fma(r, fma(-d, r, 1.0), r);
  return r;
}

// Split-DFT evaluation of the transfer function over rows (phi_rows16: Hs a multiple of 16).  One
// thread per (HR column member m, row residue u1 < H1 = Hs / 16) evaluates K at the 16 rows
// u = u1 + H1 u2 by one split step of the DFT over rows instead of 16 Horner sums: with the psf-row
// sums P_i of the column and the centred row offset i - kh/2 = i' - 16 Ch (i' the shifted row index),
// K(u) = sum_i P_i z^(u (i' - 16 Ch)), z = exp(-2 pi i / Hs), and z^(H1 u2 (i' - 16 Ch)) = w16^(u2 i')
// depends on i' mod 16 only, so K(u1 + H1 u2) = DFT16_u2( R[r] ), R[r] = sum_{i' = r mod 16} Pt[m][i']
// tr[u1][i'].  Every 16-row group of i' is summed whole (the rows past the psf are zero), so the loop
// body has compile-time register indices and LDS offsets.
__device__ __forceinline__ void phi_split_r(const PhiTileView& tv, int m, int u1, double2 (&x)[16]) {
  const double2* P = tv.Pt + m * tv.PS;
  const double2* T = tv.tr + u1 * tv.PS;
#pragma unroll
  for (int r = 0; r < 16; ++r) x[r] = make_double2(0.0, 0.0);
  for (int g = 0; g < tv.NTh; ++g, P += 16, T += 16) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = cmadd(P[r], T[r], x[r]);
      if (r % 8 == 7) __builtin_amdgcn_sched_barrier(0);  // at most 8 taps' operands in flight
    }
  }
}
__device__ __forceinline__ void phi_split_k(const PhiTileView& tv, int m, int u1, double2 (&x)[16]) {
  phi_split_r(tv, m, u1, x);
  ddft16(x);
}

// Table entries from K, the same formulas as the Horner form of k_phi_tile: with the alias class's
// sums mk2 = sum |K|^2 and mkh = sum K h_u h_v over its S x S members and rD = 1 / (mk2 / S^2 + lambda),
// module: (h_u h_v + conj K (1 - mkh / S^2) rD) / (Hs Ws) (for S = 1: (conj K + lambda) rD / (Hs Ws));
// op: K, and conj K rD / (Hs Ws).  At scale S > 1 a thread's 16 rows hold 16 / S whole alias classes
// (rows u0 + a h, h = (16 / S) H1), and the S column members of a class are the block's threads
// (v, b, u1) for b < S, which exchange their partial sums through LDS.
// LAYOUT: the table layout the S = 1 entries are written in, fixed at compile time (kPhiFused256
// also fixes Hs = 256), so that each entry's index is a per-thread base plus a constant.
template <int S, int LAYOUT = -1>
__device__ void phi_tile_rows16(const PhiArgs& a, int op, const PhiTileView& tv, double* part, int64_t cp, int vbeg,
                                int nv, double lmb) {
  const int Hs = LAYOUT == kPhiFused256 ? 256 : a.Hs, H1 = Hs >> 4;
  const double norm = 1.0 / ((double)Hs * (double)a.Ws);
  if constexpr (S == 1) {
    for (int it = threadIdx.x; it < nv * H1; it += blockDim.x) {
      const int v = it / H1, u1 = it - v * H1;
      double2 x[16];
      phi_split_r(tv, v, u1, x);
      ddft16_first(x);
      const int64_t vb = vbeg + v;
      // each group of four outputs is finished and stored before the next group's last DFT stage, so
      // the entries' fp64 temporaries are live for four outputs at a time (128 VGPRs, no spills)
#pragma unroll
      for (int k0 = 0; k0 < 4; ++k0) {
        ddft4(x[4 * k0], x[4 * k0 + 1], x[4 * k0 + 2], x[4 * k0 + 3]);
#pragma unroll
        for (int k1 = 0; k1 < 4; ++k1) {
          const double2 k = x[4 * k0 + k1];
          const int u = u1 + H1 * (k0 + 4 * k1);
          const double rD = drcp(k.x * k.x + k.y * k.y + lmb);
          if (op) {
            const int64_t o = (cp * a.Ws + vb) * Hs + u;
            a.kf[o] = make_float2((float)k.x, (float)k.y);
            a.phi[o] = make_float2((float)(k.x * rD * norm), (float)(-k.y * rD * norm));
          } else {
            const int64_t o = LAYOUT == kPhiFused256 ? fused256_phi_index(cp, (int)vb, u)
                              : LAYOUT == kPhiGeneric ? (cp * a.NCs + vb) * Hs + u
                                                      : phi_out_index(a, cp, vb, u);
            a.phi[o] = make_float2((float)((k.x + lmb) * rD * norm), (float)(-k.y * rD * norm));
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    constexpr int NM = 16 / S;  // alias classes per thread
    constexpr double inv_s2 = 1.0 / (double)(S * S);
    const int h = a.h;          // = NM H1
    // threads (b, v, u1), u1 fastest, then the chunk's column classes: a wave's stores cover runs of
    // consecutive columns of one member, as at S = 1, rather than S members Ws / S columns apart
    const int it = threadIdx.x;
    const bool act = it < nv * S * H1;
    const int b = it / (nv * H1), rem = it - b * nv * H1, v = rem / H1, u1 = rem - v * H1;
    const int e = v * S + b;
    double2 x[16];
    if (act) {
      phi_split_k(tv, e, u1, x);
      const double2 hv = tv.hW[e];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        double p2 = 0.0;
        double2 pk = make_double2(0.0, 0.0);
#pragma unroll
        for (int aa = 0; aa < S; ++aa) {
          const double2 k = x[m + NM * aa];
          p2 += k.x * k.x + k.y * k.y;
          if (!op) {
            const double2 t = dcmul(k, tv.hH[u1 + H1 * (m + NM * aa)]);
            pk.x += t.x;
            pk.y += t.y;
          }
        }
        pk = dcmul(pk, hv);
        double* pp = part + ((int64_t)(v * h + u1 + H1 * m) * S + b) * 3;
        pp[0] = p2;
        pp[1] = pk.x;
        pp[2] = pk.y;
      }
    }
    __syncthreads();
    if (act) {
      const int64_t vb = vbeg + v + (int64_t)b * a.w;
      const double2 hv = tv.hW[e];
      // module form: the host evaluates the column classes v0 <= w / 2 only.  Phi is Hermitian
      // (Phi(-u, -v) = conj Phi(u, v): real psf, and the hold sums satisfy h(-u) = conj h(u)), and the
      // class (-u0, -v0) holds the negated bins of this class's members, so a class other than v0 = 0
      // and v0 = w / 2 (which are their own mirror images) also writes its members past Ws / 2 as the
      // conjugate entries at the negated bins, which are bins <= Ws / 2 of the mirrored class.
      const int v0 = vbeg + v;
      const bool mirror = !op && v0 != 0 && 2 * v0 != a.w;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const double* pp = part + (int64_t)(v * h + u1 + H1 * m) * S * 3;
        double mk2 = 0.0;
        double2 mkh = make_double2(0.0, 0.0);
#pragma unroll
        for (int bb = 0; bb < S; ++bb) {
          mk2 += pp[3 * bb];
          mkh.x += pp[3 * bb + 1];
          mkh.y += pp[3 * bb + 2];
        }
        const double rD = drcp(mk2 * inv_s2 + lmb);
        const double2 g = make_double2((1.0 - mkh.x * inv_s2) * rD, -mkh.y * inv_s2 * rD);
        const double gop = rD * norm;
#pragma unroll
        for (int aa = 0; aa < S; ++aa) {
          const double2 k = x[m + NM * aa];
          const int u = u1 + H1 * (m + NM * aa);
          if (op) {
            const int64_t o = (cp * a.Ws + vb) * Hs + u;
            a.kf[o] = make_float2((float)k.x, (float)k.y);
            a.phi[o] = make_float2((float)(k.x * gop), (float)(-k.y * gop));
          } else if (vb <= a.Ws / 2 || mirror) {
            const double2 hn = dcmul(tv.hH[u], hv);
            const double2 t = dcmul(make_double2(k.x, -k.y), g);
            const float re = (float)((hn.x + t.x) * norm), im = (float)((hn.y + t.y) * norm);
            if (vb <= a.Ws / 2) {
              const int64_t o = LAYOUT == kPhiFused256 ? fused256_phi_index(cp, (int)vb, u)
                                : LAYOUT == kPhiGeneric ? (cp * a.NCs + vb) * Hs + u
                                                        : phi_out_index(a, cp, vb, u);
              a.phi[o] = make_float2(re, im);
            } else {  // the entry of the unevaluated class (-u0, -v0) at the negated bin
              const int un = u == 0 ? 0 : Hs - u;
              const int64_t vn = a.Ws - vb;
              const int64_t o = LAYOUT == kPhiFused256 ? fused256_phi_index(cp, (int)vn, un)
                                : LAYOUT == kPhiGeneric ? (cp * a.NCs + vn) * Hs + un
                                                        : phi_out_index(a, cp, vn, un);
              a.phi[o] = make_float2(re, -im);
            }
          }
        }
      }
    }
  }
}

// FAST: the split-DFT form (phi_rows16 holds; the host checks it), a separate instantiation so that
// the Horner form's registers (S^2 complex K values per item) do not set its occupancy: at S = 4,
// 127 instead of 220 VGPRs.  Its four-wave bound costs the S = 1 form a few spilled registers (144
// VGPRs unbounded) and measured 37.7 against 39.2 us per Converse-USRNet table.
template <int S, bool FAST>
__global__ void __launch_bounds__(256, FAST ? 4 : 1) k_phi_tile(PhiArgs a, int op, int vc, int nchunk) {
  extern __shared__ __align__(16) unsigned char phl[];
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t cp = blockIdx.x / nchunk;
  const int chunk = (int)(blockIdx.x - cp * nchunk);
  const int vbeg = chunk * vc;
  const int nv = min(vc, a.nv0 - vbeg);
  const int c = (int)(cp % a.C);
  const int Hs = a.Hs, Ws = a.Ws, h = a.h, kh = a.kh;
  const int kh4 = round4(kh);
  const double lmb = lambda_of(a, c);
  if constexpr (FAST) {
    const PhiTileView tv = phi_split_prep<S>(a, phl, cp, vbeg, nv, vc);
    static_assert(S != 3, "the split-DFT form serves scales 1, 2 and 4");
    double* part = (double*)(phl + phi_tile_lds(S, Hs, kh, a.kw, vc, true).part);
    // the host runs this form for the generic layout and for the fused 256 x 256 plan's slot order
    // only (the op form writes its own layout), so both are compile-time layouts here
    if (!op && a.layout == kPhiFused256)
      phi_tile_rows16<S, kPhiFused256>(a, op, tv, part, cp, vbeg, nv, lmb);
    else
      phi_tile_rows16<S, kPhiGeneric>(a, op, tv, part, cp, vbeg, nv, lmb);
    return;
  }
  const PhiTileView tv = phi_tile_prep<S>(a, phl, cp, vbeg, nv, vc);
  const double2 *zH = tv.zH, *phH = tv.phH, *hH = tv.hH, *hW = tv.hW, *P = tv.P;
  const double norm = 1.0 / ((double)Hs * (double)Ws);
  const double inv_s2 = 1.0 / (double)(S * S);
  const int items = nv * h;
  for (int it = tid; it < items; it += nth) {
    const int v = it / h, u0 = it - v * h;
    double2 K[S][S];  // [b][a]: member (u0 + a h, vbeg + v + b w)
    double2 mkh = make_double2(0.0, 0.0);
    double mk2 = 0.0;
#pragma unroll
    for (int b = 0; b < S; ++b) {
      const double2* Pvb = P + (v * S + b) * kh4;
      const double2 hv = hW[v * S + b];
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const int u = u0 + aa * h;
        K[b][aa] = dcmul(horner4(Pvb, kh4, zH[u]), phH[u]);
        mk2 += K[b][aa].x * K[b][aa].x + K[b][aa].y * K[b][aa].y;
        if (!op) {
          const double2 khn = S > 1 ? dcmul(K[b][aa], dcmul(hH[u], hv)) : K[b][aa];
          mkh.x += khn.x;
          mkh.y += khn.y;
        }
      }
    }
    const double rD = 1.0 / (mk2 * inv_s2 + lmb);
    const double2 g = make_double2((1.0 - mkh.x * inv_s2) * rD, -mkh.y * inv_s2 * rD);  // module
    const double gop = rD * norm;                                                       // op
#pragma unroll
    for (int b = 0; b < S; ++b) {
      const int64_t vb = vbeg + v + (int64_t)b * a.w;
      if (!op && vb > Ws / 2) continue;
      const double2 hv = hW[v * S + b];
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const int u = u0 + aa * h;
        const double2 k = K[b][aa];
        if (op) {
          const int64_t o = (cp * Ws + vb) * Hs + u;
          a.kf[o] = make_float2((float)k.x, (float)k.y);
          a.phi[o] = make_float2((float)(k.x * gop), (float)(-k.y * gop));
        } else {
          const double2 hn = S > 1 ? dcmul(hH[u], hv) : make_double2(1.0, 0.0);
          const double2 t = dcmul(make_double2(k.x, -k.y), g);
          a.phi[phi_out_index(a, cp, vb, u)] = make_float2((float)((hn.x + t.x) * norm), (float)((hn.y + t.y) * norm));
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Forward row pass: real rows of a (possibly padded) plane -> half spectrum S[plane][c][r]
// ------------------------------------------------------------------------------------------------
struct RowFwdArgs {
  const float* x;  // (P, Hin, Win)
  int Hin, Win, h, w, pad, mode;
  int NC;          // w / 2 + 1
  int rpb;         // rows per block (even)
  FftPlan plan;    // length w
  const char* tabs;  // the plan's tables (build_plan_tabs)
  int rad_off;     // byte offset of the plan's Rader tables in LDS
  float2* S;       // (P, NC, h)
};

// LC > 0: the row length a.w, fixed at compile time (fft_fixed_ct; constant index arithmetic).
template <int LC>
__global__ void __launch_bounds__(256) k_rows_fwd(RowFwdArgs a) {
  extern __shared__ float2 sm[];
  const int L = LC > 0 ? LC : a.w, ntr = a.rpb / 2, ld = L + 2;
  float2* tw = sm;
  float2* A = tw + L;
  float2* Bf = A + ntr * ld;
  const int64_t plane = blockIdx.y;
  const int r0 = blockIdx.x * a.rpb;
  const int tid = threadIdx.x, nth = blockDim.x;
  char* rad = (char*)sm + a.rad_off;
  if constexpr (LC > 0) {  // the twiddles only (no Rader stage at these lengths)
    const float2* gt = (const float2*)a.tabs;
    for (int m = tid; m < LC; m += nth) tw[m] = gt[m];
  } else {
    load_plan_tabs(a.plan, a.tabs, tw, rad, tid, nth);
  }
  const float* xp = a.x + plane * (int64_t)a.Hin * a.Win;
  const FastDiv fL = fast_div(L), frpb = fast_div(a.rpb);
  // Compile-time length with 16-byte aligned rows of a multiple of 4 samples: the interior of each
  // row as float4 loads (one row index map per item instead of three per sample), then the 2 pad
  // border columns per row from their padding sources
  const bool vec4 = LC > 0 && a.Win % 4 == 0 && ((uintptr_t)a.x & 15) == 0 && a.Win + 2 * a.pad == L;
  if (vec4) {
    const int W4 = a.Win >> 2, nI = ntr * W4, nb = 2 * a.pad;
    const FastDiv fW4 = fast_div(W4);
    for (int i0 = tid; i0 < nI; i0 += kBatch * nth) {
      float4 va[kBatch], vb[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int idx = i0 + k * nth;
        va[k] = vb[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (idx < nI) {
          const int t = idx / fW4, q = idx - t * W4;
          const int ra = r0 + 2 * t, rb = ra + 1;
          const int sa = ra < a.h ? pad_src(ra, a.Hin, a.pad, a.mode) : -1;
          const int sb = rb < a.h ? pad_src(rb, a.Hin, a.pad, a.mode) : -1;
          if (sa >= 0) va[k] = *(const float4*)(xp + (int64_t)sa * a.Win + 4 * q);
          if (sb >= 0) vb[k] = *(const float4*)(xp + (int64_t)sb * a.Win + 4 * q);
        }
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int idx = i0 + k * nth;
        if (idx < nI) {
          const int t = idx / fW4, q = idx - t * W4;
          float2* d = A + t * L + a.pad + 4 * q;
          d[0] = make_float2(va[k].x, vb[k].x);
          d[1] = make_float2(va[k].y, vb[k].y);
          d[2] = make_float2(va[k].z, vb[k].z);
          d[3] = make_float2(va[k].w, vb[k].w);
        }
      }
    }
    for (int idx = tid; idx < ntr * nb; idx += nth) {
      const int t = idx / nb, e = idx - t * nb;
      const int c = e < a.pad ? e : a.Win + e;  // border column of the padded row
      const int ra = r0 + 2 * t, rb = ra + 1;
      const int sc = pad_src(c, a.Win, a.pad, a.mode);
      const int sa = ra < a.h ? pad_src(ra, a.Hin, a.pad, a.mode) : -1;
      const int sb = rb < a.h ? pad_src(rb, a.Hin, a.pad, a.mode) : -1;
      float2 v = make_float2(0.f, 0.f);
      if (sc >= 0 && sa >= 0) v.x = xp[(int64_t)sa * a.Win + sc];
      if (sc >= 0 && sb >= 0) v.y = xp[(int64_t)sb * a.Win + sc];
      A[t * L + c] = v;
    }
  }
  for (int i0 = vec4 ? ntr * L : tid; i0 < ntr * L; i0 += kBatch * nth) {
    float2 v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      v[k] = make_float2(0.f, 0.f);
      if (idx < ntr * L) {
        const int t = idx / fL, c = idx - t * L;
        const int ra = r0 + 2 * t, rb = ra + 1;
        const int sc = pad_src(c, a.Win, a.pad, a.mode);
        if (sc >= 0) {
          if (ra < a.h) {
            const int sr = pad_src(ra, a.Hin, a.pad, a.mode);
            if (sr >= 0) v[k].x = xp[(int64_t)sr * a.Win + sc];
          }
          if (rb < a.h) {
            const int sr = pad_src(rb, a.Hin, a.pad, a.mode);
            if (sr >= 0) v[k].y = xp[(int64_t)sr * a.Win + sc];
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < ntr * L) A[idx] = v[k];  // A[t L + c] with idx = t L + c
    }
  }
  __syncthreads();
  const float2* Z;
  if constexpr (LC > 0) Z = fft_fixed_ct<LC, 0, false>(A, Bf, ntr, tw, tid, nth);
  else Z = fft_lds<false>(a.plan, A, Bf, ntr, tw, tid, nth, rad);
  // unpack two real rows: Ya = (Z[c] + conj Z[-c]) / 2, Yb = (Z[c] - conj Z[-c]) / (2i)
  float2* Sp = a.S + plane * (int64_t)a.NC * a.h;
  for (int idx = tid; idx < a.NC * a.rpb; idx += nth) {
    const int c = idx / frpb, rl = idx - c * a.rpb;
    const int r = r0 + rl;
    if (r >= a.h) continue;
    const int t = rl >> 1;
    const float2 z = Z[t * L + c];
    const float2 zm = Z[t * L + (c == 0 ? 0 : L - c)];
    float2 v;
    if ((rl & 1) == 0)
      v = make_float2(0.5f * (z.x + zm.x), 0.5f * (z.y - zm.y));
    else
      v = make_float2(0.5f * (z.y + zm.y), 0.5f * (zm.x - z.x));
    Sp[(int64_t)c * a.h + r] = v;
  }
}

// ------------------------------------------------------------------------------------------------
// Module column pass: per HR column v in [0, NCs): LR column FFT (h), tile to Hs, * Phi, inverse.
// ------------------------------------------------------------------------------------------------
struct ColModArgs {
  const float2* S;    // (P, NC, h)
  const float2* phi;  // (Cp, NCs, Hs)
  float2* SH;         // (P, NCs, Hs)   (may alias S when s == 1)
  int64_t C, psf_batch;
  int h, w, Hs, Ws, NC, NCs, cpb;
  FftPlan plan_h, plan_H;
  const char *tabs_h, *tabs_H;  // the plans' tables (build_plan_tabs)
  int rad_off;        // byte offset of plan_h's Rader tables in LDS (plan_H's follow)
};

__global__ void __launch_bounds__(256) k_cols_module(ColModArgs a) {
  extern __shared__ float2 sm[];
  const int tid = threadIdx.x, nth = blockDim.x;
  float2* twh = sm;
  float2* twH = twh + a.h;
  float2* A = twH + a.Hs;
  float2* Bf = A + a.cpb * a.Hs;
  const int64_t plane = blockIdx.y;
  const int v0 = blockIdx.x * a.cpb;
  const int ncol = min(a.cpb, a.NCs - v0);
  const int64_t cp = (a.psf_batch == 1) ? (plane % a.C) : plane;
  const float2* tH = (a.Hs != a.h) ? twH : twh;
  char* radh = (char*)sm + a.rad_off;
  char* radH = radh + rader_lds_bytes(a.plan_h);
  load_plan_tabs(a.plan_h, a.tabs_h, twh, radh, tid, nth);
  if (a.Hs != a.h) load_plan_tabs(a.plan_H, a.tabs_H, twH, radH, tid, nth);
  else radH = radh;
  const float2* Sp = a.S + plane * (int64_t)a.NC * a.h;
  const FastDiv fh = fast_div(a.h), fHs = fast_div(a.Hs);
  for (int i0 = tid; i0 < a.cpb * a.h; i0 += kBatch * nth) {
    float2 val[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      val[k] = make_float2(0.f, 0.f);
      if (idx < a.cpb * a.h) {
        const int cl = idx / fh, u = idx - cl * a.h;
        if (cl < ncol) {
          const int vv = (v0 + cl) % a.w;
          // row spectra of a real row are Hermitian in the column index (same row)
          val[k] = vv <= a.w / 2 ? Sp[(int64_t)vv * a.h + u] : cconj(Sp[(int64_t)(a.w - vv) * a.h + u]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < a.cpb * a.h) A[idx] = val[k];  // A[cl h + u] with idx = cl h + u
    }
  }
  __syncthreads();
  float2* Y = fft_lds<false>(a.plan_h, A, Bf, a.cpb, twh, tid, nth, radh);
  float2* X = (Y == A) ? Bf : A;
  const float2* ph = a.phi + cp * (int64_t)a.NCs * a.Hs;
  for (int i0 = tid; i0 < a.cpb * a.Hs; i0 += kBatch * nth) {
    float2 f[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      f[k] = make_float2(0.f, 0.f);
      if (idx < a.cpb * a.Hs) {
        const int cl = idx / fHs, u = idx - cl * a.Hs;
        if (cl < ncol) f[k] = ph[(int64_t)(v0 + cl) * a.Hs + u];
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < a.cpb * a.Hs) {
        const int cl = idx / fHs, u = idx - cl * a.Hs;
        X[idx] = cl < ncol ? cmul(Y[cl * a.h + (u - (u / fh) * a.h)], f[k]) : make_float2(0.f, 0.f);
      }
    }
  }
  __syncthreads();
  const float2* R = fft_lds<true>(a.plan_H, X, (X == A) ? Bf : A, a.cpb, tH, tid, nth, radH);
  float2* SHp = a.SH + plane * (int64_t)a.NCs * a.Hs;
  for (int idx = tid; idx < ncol * a.Hs; idx += nth) {
    const int cl = idx / fHs, u = idx - cl * a.Hs;
    SHp[(int64_t)(v0 + cl) * a.Hs + u] = R[cl * a.Hs + u];
  }
}

// ------------------------------------------------------------------------------------------------
// Op column pass: one block per (plane, LR column class v0 in [0, w)); members v0 + b w.
// ------------------------------------------------------------------------------------------------
struct ColOpArgs {
  const float2* S;    // (P, NC, h)      row spectra of y
  const float2* S0;   // (P, NCs, Hs)    row spectra of x0
  const float2* kf;   // (C, Ws, Hs)
  const float2* A;    // (C, Ws, Hs)     conj(K) / D / (Hs Ws)
  float2* SH;         // (P, NCs, Hs)
  int64_t C;
  int h, w, s, Hs, Ws, NC, NCs;
  FftPlan plan_h, plan_H;
  const char *tabs_h, *tabs_H;  // the plans' tables (build_plan_tabs)
  int rad_off;        // byte offset of plan_h's Rader tables in LDS (plan_H's follow)
};

__global__ void __launch_bounds__(256) k_cols_op(ColOpArgs a) {
  extern __shared__ float2 sm[];
  const int tid = threadIdx.x, nth = blockDim.x;
  float2* twh = sm;
  float2* twH = twh + a.h;
  float2* Ya = twH + a.Hs;             // h
  float2* Yb = Ya + a.h;               // h
  float2* Xa = Yb + a.h;               // s * Hs
  float2* Xb = Xa + a.s * a.Hs;        // s * Hs
  const int64_t plane = blockIdx.y;
  const int v0 = blockIdx.x;
  const int64_t c = plane % a.C;
  // any member with an output column?
  if (v0 > a.Ws / 2) return;  // member b = 0 is the smallest
  char* radh = (char*)sm + a.rad_off;
  char* radH = radh + rader_lds_bytes(a.plan_h);
  load_plan_tabs(a.plan_h, a.tabs_h, twh, radh, tid, nth);
  load_plan_tabs(a.plan_H, a.tabs_H, twH, radH, tid, nth);
  const float2* Sp = a.S + plane * (int64_t)a.NC * a.h;
  const float2* S0p = a.S0 + plane * (int64_t)a.NCs * a.Hs;
  for (int u = tid; u < a.h; u += nth) {
    Ya[u] = v0 <= a.w / 2 ? Sp[(int64_t)v0 * a.h + u] : cconj(Sp[(int64_t)(a.w - v0) * a.h + u]);
  }
  const FastDiv fHs = fast_div(a.Hs);
  for (int idx = tid; idx < a.s * a.Hs; idx += nth) {
    const int b = idx / fHs, u = idx - b * a.Hs;
    const int vb = v0 + b * a.w;
    Xa[b * a.Hs + u] = vb <= a.Ws / 2 ? S0p[(int64_t)vb * a.Hs + u]
                                      : cconj(S0p[(int64_t)(a.Ws - vb) * a.Hs + u]);
  }
  __syncthreads();
  const float2* Y = fft_lds<false>(a.plan_h, Ya, Yb, 1, twh, tid, nth, radh);
  float2* X0 = fft_lds<false>(a.plan_H, Xa, Xb, a.s, twH, tid, nth, radH);
  float2* Xo = (X0 == Xa) ? Xb : Xa;
  const float2* kf = a.kf + c * (int64_t)a.Ws * a.Hs;
  const float2* Am = a.A + c * (int64_t)a.Ws * a.Hs;
  const float inv_s2 = 1.0f / (float)(a.s * a.s);
  const float norm = 1.0f / ((float)a.Hs * (float)a.Ws);
  for (int u0 = tid; u0 < a.h; u0 += nth) {
    float2 m = make_float2(0.f, 0.f);
    for (int b = 0; b < a.s; ++b)
      for (int aa = 0; aa < a.s; ++aa) {
        const int ua = u0 + aa * a.h;
        const float2 t = cmul(kf[(int64_t)(v0 + b * a.w) * a.Hs + ua], X0[b * a.Hs + ua]);
        m.x += t.x;
        m.y += t.y;
      }
    const float2 d = make_float2(Y[u0].x - m.x * inv_s2, Y[u0].y - m.y * inv_s2);
    for (int b = 0; b < a.s; ++b)
      for (int aa = 0; aa < a.s; ++aa) {
        const int ua = u0 + aa * a.h;
        const float2 x0v = X0[b * a.Hs + ua];
        const float2 t = cmul(Am[(int64_t)(v0 + b * a.w) * a.Hs + ua], d);
        Xo[b * a.Hs + ua] = make_float2(fmaf(x0v.x, norm, t.x), fmaf(x0v.y, norm, t.y));
      }
  }
  __syncthreads();
  const float2* R = fft_lds<true>(a.plan_H, Xo, (Xo == Xa) ? Xb : Xa, a.s, twH, tid, nth, radH);
  float2* SHp = a.SH + plane * (int64_t)a.NCs * a.Hs;
  for (int idx = tid; idx < a.s * a.Hs; idx += nth) {
    const int b = idx / fHs, u = idx - b * a.Hs;
    const int vb = v0 + b * a.w;
    if (vb <= a.Ws / 2) SHp[(int64_t)vb * a.Hs + u] = R[b * a.Hs + u];
  }
}

// ------------------------------------------------------------------------------------------------
// Inverse row pass: half spectra SH[plane][v][u] -> real rows, crop + activation on store.
// ------------------------------------------------------------------------------------------------
struct RowInvArgs {
  const float2* SH;  // (P, NCs, Hs)
  float* out;        // (P, nrows, ncols)
  int Hs, Ws, NCs;
  int row0, nrows, col0, ncols;  // crop window
  int rpb, act;
  // Padding adjoint on the store (pad >= 0; crop window = the whole padded grid): row r of the
  // padded grid, its border columns folded into their padding sources, goes to out row r - pad
  // (interior rows, out is (P, nrows - 2 pad, ncols - 2 pad)) or to side row q (border row q,
  // side is (P, 2 pad, ncols - 2 pad)); k_pad_rows_fold then adds the side rows to their sources.
  int pad, pmode;
  float* side;
  int csrc_off;      // byte offset in LDS of the 2 pad column padding sources (pad >= 0)
  FftPlan plan;      // length Ws
  const char* tabs;  // the plan's tables (build_plan_tabs)
  int rad_off;       // byte offset of the plan's Rader tables in LDS
};

template <int LC>  // LC > 0: the row length a.Ws, fixed at compile time
__global__ void __launch_bounds__(256) k_rows_inv(RowInvArgs a) {
  extern __shared__ float2 sm[];
  const int tid = threadIdx.x, nth = blockDim.x;
  const int L = LC > 0 ? LC : a.Ws, ntr = a.rpb / 2, ld = L + 2;
  float2* tw = sm;
  float2* A = tw + L;
  float2* Bf = A + ntr * ld;
  const int64_t plane = blockIdx.y;
  const int r0 = blockIdx.x * a.rpb;  // local output row
  char* rad = (char*)sm + a.rad_off;
  if constexpr (LC > 0) {  // the twiddles only (no Rader stage at these lengths)
    const float2* gt = (const float2*)a.tabs;
    for (int m = tid; m < LC; m += nth) tw[m] = gt[m];
  } else {
    load_plan_tabs(a.plan, a.tabs, tw, rad, tid, nth);
  }
  int* csrc = (int*)((char*)sm + a.csrc_off);
  if (a.pad >= 0 && a.pmode != CVN_PAD_ZEROS)
    for (int q = tid; q < 2 * a.pad; q += nth)
      csrc[q] = pad_src(border_idx(q, a.ncols - 2 * a.pad, a.pad), a.ncols - 2 * a.pad, a.pad, a.pmode);
  const float2* SHp = a.SH + plane * (int64_t)a.NCs * a.Hs;
  const FastDiv fL = fast_div(L), frpb = fast_div(a.rpb), fnc = fast_div(a.ncols);
  // stage the half spectra: Bf[rl * NCs + v]
  for (int i0 = tid; i0 < a.NCs * a.rpb; i0 += kBatch * nth) {
    float2 val[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      val[k] = make_float2(0.f, 0.f);
      if (idx < a.NCs * a.rpb) {
        const int v = idx / frpb, rl = idx - v * a.rpb;
        if (r0 + rl < a.nrows) val[k] = SHp[(int64_t)v * a.Hs + a.row0 + r0 + rl];
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int idx = i0 + k * nth;
      if (idx < a.NCs * a.rpb) {
        const int v = idx / frpb, rl = idx - v * a.rpb;
        if (v == 0 || 2 * v == L) val[k].y = 0.f;
        Bf[rl * a.NCs + v] = val[k];
      }
    }
  }
  __syncthreads();
  for (int idx = tid; idx < ntr * L; idx += nth) {
    const int t = idx / fL, v = idx - t * L;
    const bool lo = v <= L / 2;
    const int vv = lo ? v : L - v;
    float2 ha = Bf[(2 * t) * a.NCs + vv], hb = Bf[(2 * t + 1) * a.NCs + vv];
    if (!lo) { ha.y = -ha.y; hb.y = -hb.y; }
    A[t * L + v] = make_float2(ha.x - hb.y, ha.y + hb.x);
  }
  __syncthreads();
  const float2* Z;
  if constexpr (LC > 0) Z = fft_fixed_ct<LC, 0, true>(A, Bf, ntr, tw, tid, nth);
  else Z = fft_lds<true>(a.plan, A, Bf, ntr, tw, tid, nth, rad);
  if (a.pad >= 0) {
    const int pad = a.pad, Hd = a.nrows - 2 * pad, Wd = a.ncols - 2 * pad;
    const int nb = (a.pmode == CVN_PAD_ZEROS) ? 0 : 2 * pad;
    // edge columns j <= pad or j >= Wd - 1 - pad are the only padding sources of border columns
    const bool all_edge = nb > 0 && Wd <= 2 * pad + 2;
    const int ne = nb == 0 ? 0 : (all_edge ? Wd : 2 * pad + 2);
    auto put = [&](int rl, int j, float v) {
      const int r = r0 + rl;
      if (r >= pad && r < pad + Hd)
        a.out[(plane * Hd + (r - pad)) * (int64_t)Wd + j] = v;
      else if (nb > 0)
        a.side[(plane * nb + (r < pad ? r : r - Hd)) * (int64_t)Wd + j] = v;
    };
    if (!all_edge) {
      // non-edge columns [j0, j1): with a compile-time length and 16-byte aligned rows, the aligned
      // middle [jb0, jb1) as float4 stores and the rest one sample at a time
      const int j0 = nb > 0 ? pad + 1 : 0, j1 = nb > 0 ? Wd - 1 - pad : Wd;
      int jb0 = j0, jb1 = j0;
      if (LC > 0 && Wd % 4 == 0 && ((uintptr_t)a.out & 15) == 0 && ((uintptr_t)a.side & 15) == 0) {
        jb0 = (j0 + 3) & ~3;
        jb1 = j1 & ~3;
        if (jb1 < jb0) jb1 = jb0;
      }
      const int nq = (jb1 - jb0) >> 2;
      if (nq > 0) {
        const FastDiv fq = fast_div(nq);
        for (int idx = tid; idx < a.rpb * nq; idx += nth) {
          const int rl = idx / fq, q = idx - rl * nq;
          const int r = r0 + rl;
          if (r >= a.nrows) continue;
          const int j = jb0 + 4 * q;
          const float2* zr = Z + (rl >> 1) * L + j + pad;
          const float4 v = (rl & 1) ? make_float4(zr[0].y, zr[1].y, zr[2].y, zr[3].y)
                                    : make_float4(zr[0].x, zr[1].x, zr[2].x, zr[3].x);
          float* dst = (r >= pad && r < pad + Hd) ? a.out + (plane * Hd + (r - pad)) * (int64_t)Wd + j
                       : (nb > 0 ? a.side + (plane * nb + (r < pad ? r : r - Hd)) * (int64_t)Wd + j : nullptr);
          if (dst) *(float4*)dst = v;
        }
      }
      const int nrest = (j1 - j0) - 4 * nq;  // columns [j0, jb0) and [jb1, j1)
      if (nrest > 0) {
        const FastDiv fr = fast_div(nrest);
        const int nh = jb0 - j0;
        for (int idx = tid; idx < a.rpb * nrest; idx += nth) {
          const int rl = idx / fr, e = idx - rl * nrest;
          if (r0 + rl >= a.nrows) continue;
          const int j = e < nh ? j0 + e : jb1 + (e - nh);
          const float2 z = Z[(rl >> 1) * L + j + pad];
          put(rl, j, (rl & 1) ? z.y : z.x);
        }
      }
    }
    for (int idx = tid; idx < a.rpb * ne; idx += nth) {
      const int rl = idx / ne, e = idx - rl * ne;
      if (r0 + rl >= a.nrows) continue;
      const int j = (all_edge || e <= pad) ? e : Wd - 1 - pad + (e - pad - 1);
      const float2* zr = Z + (rl >> 1) * L;
      const bool odd = rl & 1;
      float v = odd ? zr[j + pad].y : zr[j + pad].x;
      for (int qb = 0; qb < nb; ++qb)
        if (csrc[qb] == j) {
          const float2 z = zr[border_idx(qb, Wd, pad)];
          v += odd ? z.y : z.x;
        }
      put(rl, j, v);
    }
    return;
  }
  float* op = a.out + plane * (int64_t)a.nrows * a.ncols;
  for (int idx = tid; idx < a.rpb * a.ncols; idx += nth) {
    const int rl = idx / fnc, cc = idx - rl * a.ncols;
    const int r = r0 + rl;
    if (r >= a.nrows) continue;
    const float2 z = Z[(rl >> 1) * L + a.col0 + cc];
    float v = (rl & 1) ? z.y : z.x;
    if (a.act == CVN_ACT_GELU) v = gelu_exact(v);
    op[(int64_t)r * a.ncols + cc] = v;
  }
}

// ================================================================================================
// Backward of the module path.  With G = uncrop(grad_out) on the HR grid, dZ = F_{HsWs}(G):
//   dx      = pad^T(Re F*_{hw}(alias_sum(conj(Phi') dZ)))          (Phi' = Phi / (Hs Ws), the table)
//   dPhi    = sum over the samples sharing a psf of conj(tile Y) dZ / (Hs Ws),   Y = F_{hw}(pad x)
//   per alias class, with g = (1 - M(K Hn)) / D, D = M(|K|^2) + lambda, P = sum_m dPhi_m K_m and
//   rho = -Re(conj(P) g) / D:   dK_m = conj(dPhi_m) g - P conj(Hn_m) / (s^2 D) + 2 rho K_m / s^2,
//   dlambda = sum rho;   dpsf[i][j] = Re sum_{u,v} dK[u,v] exp(+2 pi i (u (i - ch) / Hs + v (j - cw) / Ws));
//   dbias = dlambda sigmoid'(bias - 9).
// The same chain as autograd through util_converse.py:142-192 (the reference registers its op as
// CompositeImplicitAutograd, converse2d.cpp:223-227).
// ================================================================================================

// Column pass: one block per (cpb consecutive LR column classes v0 in [0, NC), psf group); the block
// loops over the planes that share the group's psf (psf_batch 1: the B planes of channel c;
// otherwise one plane).  Per plane: forward HR column FFTs of the classes' members (dZ), forward LR
// column FFTs of pad(x) (Y, weight gradients only), dY = alias sum of conj(Phi') dZ, inverse LR
// column FFTs -> dS; dPhi accumulates in LDS over the planes.
struct ColBwdArgs {
  const float2* Sg;   // (P, NCs, Hs) row spectra of uncrop(grad_out)
  float2* Sx;         // (P, NC, h)   row spectra of pad(x) in (weight gradients), dS out (in place)
  const float2* phi;  // (Cp, NCs, Hs) module table Phi'
  float2* dphi;       // (Cp, Ws, Hs) or null: columns of the processed classes
  int64_t B, C, psf_batch;
  int h, w, s, Hs, Ws, NC, NCs, cpb;
  FftPlan plan_h, plan_H;
  const char *tabs_h, *tabs_H;
  int rad_off;
};

__host__ __device__ inline size_t cols_bwd_lds(int h, int Hs, int s, int cpb, bool wg) {
  return (size_t)(h + Hs + 3 * cpb * h + 2 * cpb * s * Hs + (wg ? cpb * s * Hs : 0)) * sizeof(float2);
}

constexpr int kColsBwdThreads = 512;  // 2 blocks of 8 waves per CU at the cfg3 LDS size
constexpr int kColRegs = 4;           // per-thread register slots of the scale-1 path
constexpr int kColLoad = 4;           // column elements per array loaded per thread and batch

// Asynchronous copy of nbytes (a multiple of 16) from global src to LDS dst, both contiguous, with
// global_load_lds_dwordx4: lane l of a wave's copy instruction writes its 16 bytes at dst + 16 l
// (the LDS base is wave-uniform), so no register holds the data.  The caller waits with
// s_waitcnt vmcnt(0) and a barrier before reading dst.
__device__ __forceinline__ void lds_copy_async(const float2* src, float2* dst, int nbytes, int tid, int nth) {
  const int lane = tid & 63, wave = tid >> 6, nwaves = nth >> 6;
  for (int off = wave * 1024; off < nbytes; off += nwaves * 1024)
    if (off + 16 * lane < nbytes)
      __builtin_amdgcn_global_load_lds((const void*)((const char*)src + off + 16 * lane),
                                       (__attribute__((address_space(3))) void*)((char*)dst + off), 16, 0, 0);
}

// The per-plane loop of k_cols_bwd at scale 1 on a compile-time column length, with conj(Phi') and
// the dPhi sums in registers (fr, ar: element idx = cl h + u of thread tid, k-th slot).  The block's
// columns of one plane are two contiguous runs (Sg and Sx columns vbase ..), copied into LDS by
// lds_copy_async; the next plane's copy is issued right after this plane's product, into the X and Y
// buffers that its forward transforms have freed, so its HBM round trip overlaps this plane's inverse
// transform and store.  Buffer roles rotate: xin / yin receive the copies, xfree / ytmp are the
// forward transforms' work buffers, yout the product, and the inverse transform works in yout and
// the buffer that held Y.
template <int HC>
__device__ __forceinline__ void cols_bwd_ct_planes(const ColBwdArgs& a, float2* Xa, float2* Xb, float2* Ya, float2* Yb,
                                                   float2* Yc, const float2* twh, const float2 (&fr)[kColRegs],
                                                   float2 (&ar)[kColRegs], int ncol, int vbase, int64_t grp,
                                                   int64_t nplanes, bool wg, float norm) {
  const int tid = threadIdx.x, nth = blockDim.x, cpb = a.cpb;
  // column slots past ncol are transformed but never stored: start them at zero
  for (int i = tid; i < cpb * HC; i += nth) {
    const float2 z = make_float2(0.f, 0.f);
    Xa[i] = z; Xb[i] = z; Ya[i] = z; Yb[i] = z; Yc[i] = z;
  }
  __syncthreads();
  const int nb = ncol * HC * (int)sizeof(float2);
  auto issue = [&](int64_t ib, float2* xd, float2* yd) {
    const int64_t plane = (a.psf_batch == 1) ? ib * a.C + grp : grp;
    lds_copy_async(a.Sg + plane * (int64_t)a.NCs * HC + (int64_t)vbase * HC, xd, nb, tid, nth);
    if (wg) lds_copy_async(a.Sx + plane * (int64_t)a.NC * HC + (int64_t)vbase * HC, yd, nb, tid, nth);
  };
  float2 *xin = Xa, *xfree = Xb, *yin = Ya, *ytmp = Yb, *yout = Yc;
  issue(0, xin, yin);
  for (int64_t ib = 0; ib < nplanes; ++ib) {
    const int64_t plane = (a.psf_batch == 1) ? ib * a.C + grp : grp;
    float2* Sxp = a.Sx + plane * (int64_t)a.NC * HC;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies (and earlier stores) done
    __syncthreads();                                  // every wave's copies; the previous plane's reads
    const float2* dZ = fft_fixed_ct<HC, 0, false>(xin, xfree, cpb, twh, tid, nth);
    const float2* Y = wg ? fft_fixed_ct<HC, 0, false>(yin, ytmp, cpb, twh, tid, nth) : nullptr;
#pragma unroll
    for (int k = 0; k < kColRegs; ++k) {
      const int idx = tid + k * nth;
      if (idx < cpb * HC) {
        const float2 z = dZ[idx];
        if (wg) {
          const float2 t = cmul(cconj(Y[idx]), z);
          ar[k].x = fmaf(t.x, norm, ar[k].x);
          ar[k].y = fmaf(t.y, norm, ar[k].y);
        }
        yout[idx] = cmul(fr[k], z);
      }
    }
    __syncthreads();
    // free now: the X buffer not holding dZ, the Y buffer not holding Y (both Y buffers without
    // weight gradients), and the one holding Y (read by the product only)
    float2* xnext = (dZ == xin) ? xfree : xin;
    float2* ynext = (wg && Y == yin) ? ytmp : yin;
    float2* yscr = (ynext == yin) ? ytmp : yin;
    if (ib + 1 < nplanes) issue(ib + 1, xnext, ynext);
    const float2* R = fft_fixed_ct<HC, 0, true>(yout, yscr, cpb, twh, tid, nth);
    for (int idx = tid; idx < ncol * HC; idx += nth) Sxp[(int64_t)vbase * HC + idx] = R[idx];
    xfree = (xnext == xin) ? xfree : xin;
    xin = xnext;
    ytmp = yscr;
    yin = ynext;
  }
}

// HC > 0: scale 1 with the column length h = Hs fixed at compile time (fft_fixed_ct).
// Four waves per SIMD (at most 128 VGPRs): two blocks per CU, which the LDS size allows at cfg3.
template <int HC>
__global__ void __launch_bounds__(kColsBwdThreads, 4) k_cols_bwd(ColBwdArgs a) {
  extern __shared__ float2 sm[];
  const int tid = threadIdx.x, nth = blockDim.x;
  const bool wg = a.dphi != nullptr;
  // scale, LR and HR column lengths (constants when HC > 0; the argument struct is left unmodified,
  // so that it is not copied to scratch)
  const int as = HC > 0 ? 1 : a.s, ah = HC > 0 ? HC : a.h, aHs = HC > 0 ? HC : a.Hs;
  const int cpb = a.cpb, sH = as * aHs;
  float2* twh = sm;
  float2* twH = twh + ah;
  float2* Ya = twH + aHs;           // cpb h: Y (LR column spectra of pad x)
  float2* Yb = Ya + cpb * ah;       // cpb h
  float2* Yc = Yb + cpb * ah;       // cpb h: dY
  float2* Xa = Yc + cpb * ah;       // cpb s Hs: dZ
  float2* Xb = Xa + cpb * sH;        // cpb s Hs
  float2* acc = Xb + cpb * sH;       // cpb s Hs: dPhi (weight gradients only)
  const int vbase = blockIdx.x * cpb;
  const int ncol = min(cpb, a.NC - vbase);
  const int64_t grp = blockIdx.y;    // psf plane: c (psf_batch 1) or the plane (psf_batch B)
  char* radh = nullptr;
  char* radH = nullptr;
  if constexpr (HC > 0) {  // the twiddles only (no Rader stage at these lengths)
    const float2* gt = (const float2*)a.tabs_h;
    for (int m = tid; m < HC; m += nth) twh[m] = gt[m];
  } else {
    radh = (char*)sm + a.rad_off;
    radH = radh + rader_lds_bytes(a.plan_h);
    load_plan_tabs(a.plan_h, a.tabs_h, twh, radh, tid, nth);
    if (aHs != ah) load_plan_tabs(a.plan_H, a.tabs_H, twH, radH, tid, nth);
    else radH = radh;
  }
  const float2* tH = (aHs != ah) ? twH : twh;
  const float2* ph = a.phi + grp * (int64_t)a.NCs * aHs;
  const FastDiv fHs = fast_div(aHs), fh = fast_div(ah), fsH = fast_div(sH);
  const float norm = 1.0f / ((float)aHs * (float)a.Ws);
  if (wg)
    for (int i = tid; i < cpb * sH; i += nth) acc[i] = make_float2(0.f, 0.f);
  // Scale 1 with at most kColRegs elements per thread: every class has one member column (vb =
  // vbase + cl <= Ws / 2) and one row per bin, so element idx = cl h + u of this thread is the same
  // in every plane; its conj(Phi') is read from HBM once and the dPhi sum stays in registers.
  const bool regs = as == 1 && cpb * ah <= kColRegs * nth;
  bool nplanes_done = false;
  float2 fr[kColRegs], ar[kColRegs];
  if (regs) {
#pragma unroll
    for (int k = 0; k < kColRegs; ++k) {
      const int idx = tid + k * nth;
      const int cl = idx / fh;
      fr[k] = (cl < ncol) ? cconj(ph[(int64_t)(vbase + cl) * aHs + (idx - cl * ah)]) : make_float2(0.f, 0.f);
      ar[k] = make_float2(0.f, 0.f);
    }
  }
  const int64_t nplanes = (a.psf_batch == 1) ? a.B : 1;
  if constexpr (HC > 0) {
    // (its 16-byte direct-to-LDS copies need 16-byte aligned spectra: every column offset is a
    // multiple of 16 bytes, so the bases decide; cvn_converse2d_bwd_f32 aligns them, and other bases
    // would take the loop below)
    if (regs && (((uintptr_t)a.Sg | (uintptr_t)a.Sx) & 15) == 0) {
      cols_bwd_ct_planes<HC>(a, Xa, Xb, Ya, Yb, Yc, twh, fr, ar, ncol, vbase, grp, nplanes, wg, norm);
      nplanes_done = true;
    }
  }
  for (int64_t ib = 0; ib < (nplanes_done ? 0 : nplanes); ++ib) {
    const int64_t plane = (a.psf_batch == 1) ? ib * a.C + grp : grp;
    const float2* Sgp = a.Sg + plane * (int64_t)a.NCs * aHs;
    float2* Sxp = a.Sx + plane * (int64_t)a.NC * ah;
    __syncthreads();  // the previous plane's LDS reads are done
    // member columns vb = v0 + b w of each class (row spectra of real rows are Hermitian in the
    // column); the Sg and Sx loads of a batch are all issued before the first LDS store, so a
    // plane waits for one HBM round trip, not two
    const int nG = cpb * sH, nX = wg ? cpb * ah : 0;
    for (int i0 = tid; i0 < max(nG, nX); i0 += kColLoad * nth) {
      float2 vg[kColLoad], vx[kColLoad];
#pragma unroll
      for (int k = 0; k < kColLoad; ++k) {
        const int idx = i0 + k * nth;
        vg[k] = make_float2(0.f, 0.f);
        vx[k] = make_float2(0.f, 0.f);
        if (idx < nG) {
          const int cl = idx / fsH, r = idx - cl * sH;
          const int b = r / fHs, u = r - b * aHs;
          if (cl < ncol) {
            const int vb = vbase + cl + b * a.w;
            vg[k] = vb <= a.Ws / 2 ? Sgp[(int64_t)vb * aHs + u] : cconj(Sgp[(int64_t)(a.Ws - vb) * aHs + u]);
          }
        }
        if (idx < nX && idx < ncol * ah) vx[k] = Sxp[(int64_t)vbase * ah + idx];  // columns vbase.. are contiguous
      }
#pragma unroll
      for (int k = 0; k < kColLoad; ++k) {
        const int idx = i0 + k * nth;
        if (idx < nG) Xa[idx] = vg[k];
        if (idx < nX) Ya[idx] = vx[k];
      }
    }
    __syncthreads();
    const float2 *dZ, *Y = nullptr;
    if constexpr (HC > 0) {
      dZ = fft_fixed_ct<HC, 0, false>(Xa, Xb, cpb, tH, tid, nth);
      if (wg) Y = fft_fixed_ct<HC, 0, false>(Ya, Yb, cpb, twh, tid, nth);
    } else {
      dZ = fft_lds<false>(a.plan_H, Xa, Xb, cpb * as, tH, tid, nth, radH);
      if (wg) Y = fft_lds<false>(a.plan_h, Ya, Yb, cpb, twh, tid, nth, radh);
    }
    if (regs) {
#pragma unroll
      for (int k = 0; k < kColRegs; ++k) {
        const int idx = tid + k * nth;
        if (idx < cpb * ah) {
          const float2 z = dZ[idx];
          if (wg) {
            const float2 t = cmul(cconj(Y[idx]), z);
            ar[k].x = fmaf(t.x, norm, ar[k].x);
            ar[k].y = fmaf(t.y, norm, ar[k].y);
          }
          Yc[idx] = cmul(fr[k], z);
        }
      }
    } else {
      if (wg) {
        for (int idx = tid; idx < cpb * sH; idx += nth) {
          const int cl = idx / fsH, r = idx - cl * sH;
          const int u = r - (r / fHs) * aHs;
          const float2 t = cmul(cconj(Y[cl * ah + u - (u / fh) * ah]), dZ[idx]);
          acc[idx].x = fmaf(t.x, norm, acc[idx].x);
          acc[idx].y = fmaf(t.y, norm, acc[idx].y);
        }
      }
      for (int idx = tid; idx < cpb * ah; idx += nth) {
        const int cl = idx / fh, u0 = idx - cl * ah;
        float2 m = make_float2(0.f, 0.f);
        if (cl < ncol) {
          for (int b = 0; b < as; ++b) {
            const int vb = vbase + cl + b * a.w;
            for (int aa = 0; aa < as; ++aa) {
              const int u = u0 + aa * ah;
              const float2 f = vb <= a.Ws / 2 ? ph[(int64_t)vb * aHs + u]
                                              : cconj(ph[(int64_t)(a.Ws - vb) * aHs + (u == 0 ? 0 : aHs - u)]);
              const float2 t = cmul(cconj(f), dZ[cl * sH + b * aHs + u]);
              m.x += t.x;
              m.y += t.y;
            }
          }
        }
        Yc[idx] = m;
      }
    }
    __syncthreads();
    const float2* R;
    if constexpr (HC > 0) R = fft_fixed_ct<HC, 0, true>(Yc, Ya, cpb, twh, tid, nth);
    else R = fft_lds<true>(a.plan_h, Yc, Ya, cpb, twh, tid, nth, radh);
    for (int idx = tid; idx < ncol * ah; idx += nth) Sxp[(int64_t)vbase * ah + idx] = R[idx];
  }
  if (wg && regs) {
    float2* dp = a.dphi + grp * (int64_t)a.Ws * aHs;
#pragma unroll
    for (int k = 0; k < kColRegs; ++k) {
      const int idx = tid + k * nth;
      if (idx < ncol * ah) {
        const int cl = idx / fh;
        dp[(int64_t)(vbase + cl) * aHs + (idx - cl * ah)] = ar[k];
      }
    }
  } else if (wg) {
    __syncthreads();
    float2* dp = a.dphi + grp * (int64_t)a.Ws * aHs;
    for (int idx = tid; idx < ncol * sH; idx += nth) {
      const int cl = idx / fsH, r = idx - cl * sH;
      const int b = r / fHs, u = r - b * aHs;
      dp[(int64_t)(vbase + cl + b * a.w) * aHs + u] = acc[idx];
    }
  }
}

// Second half of the padding adjoint (the first is k_rows_inv's store): border row q of every
// plane, already folded along its columns, is added to its padding source row.  Thread = (plane,
// column j); the 2 pad border rows are added in order by that one thread, so rows that share a
// source (replicate, wide reflect) need no atomics.
__global__ void __launch_bounds__(256) k_pad_rows_fold(const float* __restrict__ side, int H, int W, int pad, int mode,
                                                       float* __restrict__ dx) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= W) return;
  const int64_t plane = blockIdx.y;
  const int nb = 2 * pad;
  for (int q = 0; q < nb; ++q) {
    const int i = pad_src(border_idx(q, H, pad), H, pad, mode);
    dx[(plane * H + i) * (int64_t)W + j] += side[(plane * nb + q) * (int64_t)W + j];
  }
}

// Per-class gradient of the transfer function: block = (psf plane, chunk of vc column classes
// v0 in [0, w)), thread = alias class, same LDS tables as k_phi_tile.  Writes dK for every member
// (full width) and the block's sum of rho (the lambda gradient).
struct PhiGradArgs {
  const float2* dphi;  // (Cp, Ws, Hs): columns of classes v0 <= w / 2; the others by symmetry
  float2* dK;          // (Cp, Ws, Hs)
  double* part;        // (Cp, nchunk): per-block sums of rho
};

template <int S>
__global__ void __launch_bounds__(256) k_phi_grad(PhiArgs a, PhiGradArgs gr, int vc, int nchunk) {
  extern __shared__ __align__(16) unsigned char phl[];
  __shared__ double red[256];
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t cp = blockIdx.x / nchunk;
  const int chunk = (int)(blockIdx.x - cp * nchunk);
  const int vbeg = chunk * vc;
  const int nv = min(vc, a.nv0 - vbeg);
  const int c = (int)(cp % a.C);
  const int Hs = a.Hs, Ws = a.Ws, h = a.h, w = a.w, kh = a.kh;
  const int kh4 = round4(kh);
  const PhiTileView tv = phi_tile_prep<S>(a, phl, cp, vbeg, nv, vc);
  const double lmb = lambda_of(a, c);
  const double inv_s2 = 1.0 / (double)(S * S);
  const float2* dp = gr.dphi + cp * (int64_t)Ws * Hs;
  float2* dk = gr.dK + cp * (int64_t)Ws * Hs;
  double rsum = 0.0;
  const int items = nv * h;
  for (int it = tid; it < items; it += nth) {
    const int v = it / h, u0 = it - v * h;
    const bool direct = 2 * (vbeg + v) <= w;  // this class's columns were written by the column pass
    double2 K[S][S], G[S][S], Hn[S][S];
    double2 s1 = make_double2(0.0, 0.0);
    double k2 = 0.0;
#pragma unroll
    for (int b = 0; b < S; ++b) {
      const double2* Pvb = tv.P + (v * S + b) * kh4;
      const double2 hv = tv.hW[v * S + b];
      const int vb = vbeg + v + b * w;
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const int u = u0 + aa * h;
        K[b][aa] = dcmul(horner4(Pvb, kh4, tv.zH[u]), tv.phH[u]);
        Hn[b][aa] = S > 1 ? dcmul(tv.hH[u], hv) : make_double2(1.0, 0.0);
        const float2 d = direct ? dp[(int64_t)vb * Hs + u]
                                : cconj(dp[(int64_t)(Ws - vb) * Hs + (u == 0 ? 0 : Hs - u)]);
        G[b][aa] = make_double2((double)d.x, (double)d.y);
        const double2 kh_ = dcmul(K[b][aa], Hn[b][aa]);
        s1.x += kh_.x;
        s1.y += kh_.y;
        k2 += K[b][aa].x * K[b][aa].x + K[b][aa].y * K[b][aa].y;
      }
    }
    const double D = k2 * inv_s2 + lmb, rD = 1.0 / D;
    const double2 g = make_double2((1.0 - s1.x * inv_s2) * rD, -s1.y * inv_s2 * rD);
    double2 P = make_double2(0.0, 0.0);
#pragma unroll
    for (int b = 0; b < S; ++b)
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const double2 t = dcmul(G[b][aa], K[b][aa]);
        P.x += t.x;
        P.y += t.y;
      }
    const double rho = -(P.x * g.x + P.y * g.y) * rD;  // -Re(conj(P) g) / D
    rsum += rho;
    const double cP = inv_s2 * rD, cK = 2.0 * rho * inv_s2;
#pragma unroll
    for (int b = 0; b < S; ++b) {
      const int vb = vbeg + v + b * w;
#pragma unroll
      for (int aa = 0; aa < S; ++aa) {
        const int u = u0 + aa * h;
        const double2 t1 = dcmul(make_double2(G[b][aa].x, -G[b][aa].y), g);
        const double2 t2 = dcmul(P, make_double2(Hn[b][aa].x, -Hn[b][aa].y));
        const double2 r = make_double2(t1.x - cP * t2.x + cK * K[b][aa].x, t1.y - cP * t2.y + cK * K[b][aa].y);
        dk[(int64_t)vb * Hs + u] = make_float2((float)r.x, (float)r.y);
      }
    }
  }
  red[tid] = rsum;
  __syncthreads();
  for (int st = nth / 2; st > 0; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  if (tid == 0) gr.part[cp * nchunk + chunk] = red[0];
}

// Transposed DFT along the columns: T[cp][u][j] = sum_v dK[cp][v][u] exp(+2 pi i v (j - cw) / Ws),
// fp64 accumulation.  Block = (kGaU rows u, psf plane); its kGaV thread slices take the columns
// v = slice mod kGaV, kGaUnroll loads in flight per thread, and the slice sums are reduced in LDS.
constexpr int kJ = 8;          // taps j per accumulation round
constexpr int kGaU = 32;       // rows u per block (lanes of a slice)
constexpr int kGaV = 8;        // column slices per block (kGaU * kGaV = 256 threads)
constexpr int kGaUnroll = 4;   // column loads batched per thread
__global__ void __launch_bounds__(256) k_psf_grad_a(const float2* __restrict__ dK, int Hs, int Ws, int kw,
                                                    double2* __restrict__ T) {
  extern __shared__ double2 twW[];  // exp(+2 pi i m / Ws), then kGaV * kGaU * kJ slice sums
  double2* part = twW + Ws;
  const int tid = threadIdx.x;
  const int ul = tid % kGaU, vs = tid / kGaU;
  const int64_t cp = blockIdx.y;
  for (int m = tid; m < Ws; m += blockDim.x) {
    const double2 e = dexpi((double)m, (double)Ws);
    twW[m] = make_double2(e.x, -e.y);
  }
  const int u = blockIdx.x * kGaU + ul;
  const bool live = u < Hs;
  const float2* col = dK + cp * (int64_t)Ws * Hs + (live ? u : 0);
  const int cw = kw / 2;
  for (int j0 = 0; j0 < kw; j0 += kJ) {
    double2 acc[kJ];
    int idx[kJ], step[kJ];
#pragma unroll
    for (int q = 0; q < kJ; ++q) {
      acc[q] = make_double2(0.0, 0.0);
      int d = (j0 + q - cw) % Ws;
      d = d < 0 ? d + Ws : d;
      idx[q] = (int)(((int64_t)vs * d) % Ws);  // exponent index of column v = vs
      step[q] = (int)(((int64_t)kGaV * d) % Ws);
    }
    __syncthreads();  // twW written; the previous round's slice sums consumed
    for (int v0 = vs; v0 < Ws; v0 += kGaV * kGaUnroll) {
      float2 g[kGaUnroll];
#pragma unroll
      for (int r = 0; r < kGaUnroll; ++r) {
        const int v = v0 + r * kGaV;
        g[r] = (live && v < Ws) ? col[(int64_t)v * Hs] : make_float2(0.f, 0.f);
      }
#pragma unroll
      for (int r = 0; r < kGaUnroll; ++r) {
        const double2 gd = make_double2((double)g[r].x, (double)g[r].y);
#pragma unroll
        for (int q = 0; q < kJ; ++q) {
          const double2 e = twW[idx[q]];
          acc[q].x = fma(gd.x, e.x, fma(-gd.y, e.y, acc[q].x));
          acc[q].y = fma(gd.x, e.y, fma(gd.y, e.x, acc[q].y));
          idx[q] += step[q];
          if (idx[q] >= Ws) idx[q] -= Ws;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kJ; ++q) part[(vs * kGaU + ul) * kJ + q] = acc[q];
    __syncthreads();
    if (vs == 0 && live) {
#pragma unroll
      for (int q = 0; q < kJ; ++q) {
        if (j0 + q >= kw) break;
        double2 t = part[ul * kJ + q];
        for (int sl = 1; sl < kGaV; ++sl) {
          const double2 o = part[(sl * kGaU + ul) * kJ + q];
          t.x += o.x;
          t.y += o.y;
        }
        T[(cp * Hs + u) * kw + j0 + q] = t;
      }
    }
  }
}

// Second pass, one block per channel: dpsf[cp][i][j] = Re sum_u T[cp][u][j] exp(+2 pi i u (i - ch) / Hs)
// for every psf plane cp of channel c, and dbias[c] = sum of the lambda gradient x sigmoid'(bias - 9).
__global__ void __launch_bounds__(256) k_psf_grad_b(const double2* __restrict__ T, const double* __restrict__ part,
                                                    int nchunk, int64_t C, int64_t psf_batch, int Hs, int kh, int kw,
                                                    const float* __restrict__ bias, float* __restrict__ dpsf,
                                                    float* __restrict__ dbias) {
  extern __shared__ double2 twH[];  // exp(+2 pi i m / Hs)
  __shared__ double red[256];
  const int tid = threadIdx.x, nth = blockDim.x;
  const int64_t c = blockIdx.x;
  for (int m = tid; m < Hs; m += nth) {
    const double2 e = dexpi((double)m, (double)Hs);
    twH[m] = make_double2(e.x, -e.y);
  }
  __syncthreads();
  const int ch = kh / 2;
  double lsum = 0.0;
  for (int64_t pb = 0; pb < psf_batch; ++pb) {
    const int64_t cp = pb * C + c;
    if (dpsf && kh * kw <= nth) {
      // S threads per tap, each summing the rows u = slice mod S; slice sums reduced in LDS
      const int ne = kh * kw, S = nth / ne, e = tid % ne, sl = tid / ne;
      double acc = 0.0;
      if (sl < S) {
        const int i = e / kw, j = e - i * kw;
        int d = (i - ch) % Hs;
        if (d < 0) d += Hs;
        const int dS = (int)(((int64_t)d * S) % Hs);
        int idx = (int)(((int64_t)d * sl) % Hs);
        const double2* Tc = T + cp * (int64_t)Hs * kw + j;
        for (int u = sl; u < Hs; u += S) {
          const double2 t = Tc[(int64_t)u * kw], e2 = twH[idx];
          acc = fma(t.x, e2.x, fma(-t.y, e2.y, acc));
          idx += dS;
          if (idx >= Hs) idx -= Hs;
        }
      }
      red[tid] = acc;
      __syncthreads();
      if (tid < ne) {
        double t = 0.0;
        for (int k = 0; k < S; ++k) t += red[tid + k * ne];
        dpsf[cp * ne + tid] = (float)t;
      }
      __syncthreads();  // red is reused
    } else if (dpsf) {
      for (int e = tid; e < kh * kw; e += nth) {
        const int i = e / kw, j = e - i * kw;
        int d = (i - ch) % Hs;
        if (d < 0) d += Hs;
        int idx = 0;
        double acc = 0.0;
        const double2* Tc = T + cp * (int64_t)Hs * kw + j;
        for (int u = 0; u < Hs; ++u) {
          const double2 t = Tc[(int64_t)u * kw], e2 = twH[idx];
          acc = fma(t.x, e2.x, fma(-t.y, e2.y, acc));
          idx += d;
          if (idx >= Hs) idx -= Hs;
        }
        dpsf[cp * kh * kw + e] = (float)acc;
      }
    }
    for (int k = tid; k < nchunk; k += nth) lsum += part[cp * nchunk + k];
  }
  red[tid] = lsum;
  __syncthreads();
  for (int st = nth / 2; st > 0; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  if (tid == 0 && dbias) {
    const double sg = 1.0 / (1.0 + exp(-((double)bias[c] - 9.0)));
    dbias[c] = (float)(red[0] * sg * (1.0 - sg));
  }
}

// ================================================================================================
// host side
// ================================================================================================
namespace {

constexpr int kThreads = 256;
constexpr size_t kLdsLimit = 160 * 1024;

std::atomic<uint64_t> g_attr_done{0};
void set_lds_attrs() {
  once_per_device(g_attr_done, [] {
    for (const void* k : {(const void*)k_rows_fwd<0>, (const void*)k_rows_fwd<132>, (const void*)k_rows_fwd<256>,
                          (const void*)k_rows_fwd<260>, (const void*)k_rows_inv<0>, (const void*)k_rows_inv<132>,
                          (const void*)k_rows_inv<256>, (const void*)k_rows_inv<260>, (const void*)k_cols_bwd<0>,
                          (const void*)k_cols_bwd<132>, (const void*)k_cols_bwd<256>, (const void*)k_cols_bwd<260>})
      (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_cols_module, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_cols_op, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_phi_grad<1>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_phi_grad<2>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_phi_grad<3>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_phi_grad<4>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_psf_grad_a, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipFuncSetAttribute((const void*)k_psf_grad_b, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsLimit);
    (void)hipGetLastError();
  });
}

// rows per block (even) for a row pass of length L
int rows_per_block(int L, int nrows) {
  int ntr = std::max(1, std::min(8, 2048 / std::max(L, 1)));
  while (ntr > 1 && (size_t)(L + 2 * ntr * (L + 2)) * sizeof(float2) > 96 * 1024) --ntr;
  int rpb = 2 * ntr;
  while (rpb > 2 && rpb - 2 >= nrows) rpb -= 2;
  return rpb;
}
size_t rows_lds(int L, int rpb) { return (size_t)(L + 2 * (rpb / 2) * (L + 2)) * sizeof(float2); }

int cols_per_block(int h, int Hs) {
  int cpb = std::max(1, std::min(16, 2048 / std::max(Hs, 1)));
  while (cpb > 1 && (size_t)(h + Hs + 2 * cpb * Hs) * sizeof(float2) > 96 * 1024) --cpb;
  return cpb;
}
size_t cols_lds(int h, int Hs, int cpb) { return (size_t)(h + Hs + 2 * cpb * Hs) * sizeof(float2); }

struct Geo {
  int64_t B, C, P, Cp;
  int H, W, kh, kw, s, pad, h, w, Hs, Ws, NC, NCs;
};

int module_geo(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw,
               int scale, int pad, Geo* g) {
  if (B < 0 || C < 1 || H < 1 || W < 1) return fail(CVN_ERR_ARG, "bad input shape");
  if (kh < 1 || kw < 1) return fail(CVN_ERR_ARG, "bad psf shape");
  if (psf_batch != 1 && psf_batch != B) return fail(CVN_ERR_ARG, "psf batch must be 1 or B");
  if (scale < 1) return fail(CVN_ERR_ARG, "scale must be >= 1");
  if (pad < 0) return fail(CVN_ERR_ARG, "padding must be >= 0");
  g->B = B; g->C = C; g->P = B * C; g->Cp = psf_batch * C;
  g->H = (int)H; g->W = (int)W; g->kh = kh; g->kw = kw; g->s = scale; g->pad = pad;
  g->h = (int)H + 2 * pad; g->w = (int)W + 2 * pad;
  g->Hs = g->h * scale; g->Ws = g->w * scale;
  g->NC = g->w / 2 + 1; g->NCs = g->Ws / 2 + 1;
  if (g->Hs > kMaxFftLen || g->Ws > kMaxFftLen)
    return fail(CVN_ERR_UNSUPPORTED, "padded plane %dx%d exceeds %d", g->Hs, g->Ws, kMaxFftLen);
  if ((int64_t)scale * kh > 4096 || kh > 1024 || kw > 1024)
    return fail(CVN_ERR_UNSUPPORTED, "psf too large");
  return CVN_OK;
}

// FFT plan tables of the four transform lengths a call uses (w, h, Hs, Ws), one region each.
struct PlanTabs {
  FftPlan plan[4];
  size_t off[4], bytes;
};
enum { kTabW = 0, kTabH = 1, kTabHs = 2, kTabWs = 3 };
bool plan_tabs(const Geo& g, PlanTabs* t) {
  const int len[4] = {g.w, g.h, g.Hs, g.Ws};
  size_t o = 0;
  for (int i = 0; i < 4; ++i) {
    if (!make_plan(len[i], &t->plan[i])) return false;
    t->off[i] = o;
    o += align_up(plan_tab_bytes(t->plan[i]), 256);
  }
  t->bytes = o;
  return true;
}

struct PlanTabsArgs {
  FftPlan plan[4];
  char* dst[4];
};
__global__ void __launch_bounds__(256) k_plan_tabs(PlanTabsArgs a) {
  __shared__ double2 wd[kMaxRaderLen], bd[kMaxRaderLen];
  build_plan_tabs(a.plan[blockIdx.x], a.dst[blockIdx.x], wd, bd, threadIdx.x, blockDim.x);
}
int launch_plan_tabs(const PlanTabs& t, char* base, hipStream_t st) {
  PlanTabsArgs a;
  for (int i = 0; i < 4; ++i) {
    a.plan[i] = t.plan[i];
    a.dst[i] = base + t.off[i];
  }
  hipLaunchKernelGGL(k_plan_tabs, dim3(4), dim3(kThreads), 0, st, a);
  return check_launch("FFT plan tables");
}

struct ModWs {
  size_t phi, tabs, S, SH, total;
};
ModWs module_ws(const Geo& g, const PlanTabs& t) {
  ModWs w;
  w.phi = 0;
  size_t o = align_up((size_t)g.Cp * g.NCs * g.Hs * sizeof(float2));
  w.tabs = o;
  o += t.bytes;
  w.S = o;
  o += align_up((size_t)g.P * g.NC * g.h * sizeof(float2));
  if (g.s == 1) {
    w.SH = w.S;  // in-place column pass
  } else {
    w.SH = o;
    o += align_up((size_t)g.P * g.NCs * g.Hs * sizeof(float2));
  }
  w.total = o;
  return w;
}

// Transfer tables.  Returns CVN_ERR_UNSUPPORTED without launching anything when a layout other than
// the generic one is asked for and the tiled kernel does not apply (the caller then builds it otherwise).
int launch_phi(const float* psf, const float* bias, float eps, const Geo& g, bool op, float2* phi,
               float2* kf, hipStream_t st, int layout = kPhiGeneric) {
  PhiArgs a;
  a.psf = psf; a.bias = bias; a.Cp = g.Cp; a.C = (int)g.C; a.kh = g.kh; a.kw = g.kw; a.s = g.s;
  a.h = g.h; a.w = g.w; a.Hs = g.Hs; a.Ws = g.Ws; a.NCs = g.NCs; a.eps = (double)eps;
  a.phi = phi; a.kf = kf;
  a.layout = layout;
  const bool q268 = layout == kPhiPfa268;
  a.nv0 = (!op && g.s == 1) ? g.NC : g.w;
  // tiled kernel (scales 1..4): about 2048 blocks, chunk size bounded by an LDS budget of 64 KiB
  if (g.s <= 4) {
    constexpr int kTileLds = 64 * 1024;
    int nchunk = (int)std::min<int64_t>(a.nv0, std::max<int64_t>(1, (2048 + g.Cp - 1) / g.Cp));
    int vc = (a.nv0 + nchunk - 1) / nchunk;
    // split-DFT form (phi_tile_rows16): S Hs / 16 threads per LR column class, one round per block
    // (its set-up gives each thread one psf column and one row-twiddle column: kw and 16 NTh <= kThreads)
    const bool fast = phi_rows16(g.s, g.Hs, q268) && g.kw <= kThreads &&
                      16 * phi_tile_lds(g.s, g.Hs, g.kh, g.kw, 1, true).NTh <= kThreads &&
                      (op || layout == kPhiGeneric || (layout == kPhiFused256 && g.Hs == 256 && g.Ws == 256));
    // the split-DFT form's module tables at s > 1 evaluate the column classes v0 <= w / 2 and write the
    // others' entries by Hermitian symmetry (the kernels below, if this one does not apply, evaluate
    // every class: nv0 is restored for them)
    const int nv0_all = a.nv0;
    if (fast && !op && g.s > 1) a.nv0 = g.w / 2 + 1;
    if (fast) vc = std::max(1, std::min(a.nv0, 256 / (g.s * (g.Hs / 16))));
    while (vc > 1 && phi_tile_lds(g.s, g.Hs, g.kh, g.kw, vc, fast).total > kTileLds) --vc;
    const int lds = phi_tile_lds(g.s, g.Hs, g.kh, g.kw, vc, fast).total;
    nchunk = (a.nv0 + vc - 1) / vc;
    if (lds <= kTileLds && g.Cp * nchunk <= 0x7fffffff) {
      const dim3 grid((unsigned)(g.Cp * nchunk));
      const int o = op ? 1 : 0;
      auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), (size_t)lds, st, a, o, vc, nchunk); };
      switch (g.s) {
        case 1: fast ? go(k_phi_tile<1, true>) : go(k_phi_tile<1, false>); break;
        case 2: fast ? go(k_phi_tile<2, true>) : go(k_phi_tile<2, false>); break;
        case 3: go(k_phi_tile<3, false>); break;  // phi_rows16 needs s in {1, 2, 4}
        default: fast ? go(k_phi_tile<4, true>) : go(k_phi_tile<4, false>); break;
      }
      return check_launch("transfer table");
    }
    a.nv0 = nv0_all;
  }
  if (layout != kPhiGeneric) return fail(CVN_ERR_UNSUPPORTED, "this table layout needs the tiled kernel");
  const size_t lds = (size_t)g.s * g.kh * sizeof(double2);
  const int64_t blocks = g.Cp * a.nv0;
  if (blocks > 0x7fffffff) return fail(CVN_ERR_UNSUPPORTED, "too many transfer blocks");
  if (op)
    hipLaunchKernelGGL(k_phi_op, dim3((unsigned)blocks), dim3(kThreads), lds, st, a);
  else
    hipLaunchKernelGGL(k_phi_module, dim3((unsigned)blocks), dim3(kThreads), lds, st, a);
  return check_launch("transfer table");
}

int launch_rows_fwd(const float* x, int64_t P, int Hin, int Win, int pad, int mode, int h, int w,
                    const char* tabs, float2* S, hipStream_t st) {
  RowFwdArgs a;
  a.x = x; a.Hin = Hin; a.Win = Win; a.h = h; a.w = w; a.pad = pad; a.mode = mode;
  a.NC = w / 2 + 1;
  a.rpb = rows_per_block(w, h);
  if (!make_plan(w, &a.plan)) return fail(CVN_ERR_UNSUPPORTED, "no plan for length %d", w);
  a.rad_off = (int)align_up(rows_lds(w, a.rpb), 16);
  a.tabs = tabs;
  a.S = S;
  dim3 grid((h + a.rpb - 1) / a.rpb, (unsigned)P);
  const size_t lds = a.rad_off + rader_lds_bytes(a.plan);
  switch (w) {  // lengths with a compile-time plan
    case 132: hipLaunchKernelGGL(k_rows_fwd<132>, grid, dim3(kThreads), lds, st, a); break;
    case 256: hipLaunchKernelGGL(k_rows_fwd<256>, grid, dim3(kThreads), lds, st, a); break;
    case 260: hipLaunchKernelGGL(k_rows_fwd<260>, grid, dim3(kThreads), lds, st, a); break;
    default: hipLaunchKernelGGL(k_rows_fwd<0>, grid, dim3(kThreads), lds, st, a); break;
  }
  return check_launch("row forward pass");
}

int launch_rows_inv(const float2* SH, const Geo& g, int row0, int nrows, int col0, int ncols,
                    int act, const char* tabs, float* out, hipStream_t st, int pad = -1, int pmode = 0,
                    float* side = nullptr) {
  RowInvArgs a;
  a.SH = SH; a.out = out; a.Hs = g.Hs; a.Ws = g.Ws; a.NCs = g.NCs;
  a.row0 = row0; a.nrows = nrows; a.col0 = col0; a.ncols = ncols; a.act = act;
  a.pad = pad; a.pmode = pmode; a.side = side;
  a.rpb = rows_per_block(g.Ws, nrows);
  if (!make_plan(g.Ws, &a.plan)) return fail(CVN_ERR_UNSUPPORTED, "no plan for length %d", g.Ws);
  a.rad_off = (int)align_up(rows_lds(g.Ws, a.rpb), 16);
  a.csrc_off = (int)(a.rad_off + rader_lds_bytes(a.plan));
  a.tabs = tabs;
  dim3 grid((nrows + a.rpb - 1) / a.rpb, (unsigned)g.P);
  const size_t lds = a.csrc_off + sizeof(int) * 2 * std::max(pad, 0);
  switch (g.Ws) {  // lengths with a compile-time plan
    case 132: hipLaunchKernelGGL(k_rows_inv<132>, grid, dim3(kThreads), lds, st, a); break;
    case 256: hipLaunchKernelGGL(k_rows_inv<256>, grid, dim3(kThreads), lds, st, a); break;
    case 260: hipLaunchKernelGGL(k_rows_inv<260>, grid, dim3(kThreads), lds, st, a); break;
    default: hipLaunchKernelGGL(k_rows_inv<0>, grid, dim3(kThreads), lds, st, a); break;
  }
  return check_launch("row inverse pass");
}

}  // namespace
}  // namespace cvn

using namespace cvn;

bool cvn::fused_disabled() {
  const char* e = getenv("CVN_DISABLE_FUSED");
  return e && e[0] == '1';
}

namespace {

// Which kernels serve a module-level call (CVN_ROUTE_*), and the table / scratch sizes they need.
// The table holds the transfer function in the layout of the route's kernels; it depends only on the
// psf, bias, eps and geometry, so callers may cache it across calls with unchanged weights, keeping
// the route next to it.
struct Route {
  int id;
  size_t table_bytes, scratch_bytes;
};

int module_route(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw, int scale,
                 int pad, int want, Geo* g, Route* r) {
  int rc = module_geo(B, C, H, W, psf_batch, kh, kw, scale, pad, g);
  if (rc != CVN_OK) return rc;
  if (want < CVN_ROUTE_AUTO || want > CVN_ROUTE_GENERIC) return fail(CVN_ERR_ARG, "bad route %d", want);
  size_t fws = 0;
  const bool fused_ok = kh <= 64 && fused_query(g->H, g->W, g->pad, g->s, g->Cp, &fws);
  const bool pfa_ok = pfa268_applies(g->h, g->w, g->s);
  if (want == CVN_ROUTE_AUTO)
    want = fused_disabled() ? CVN_ROUTE_GENERIC
                            : fused_ok ? CVN_ROUTE_FUSED : pfa_ok ? CVN_ROUTE_PFA268 : CVN_ROUTE_GENERIC;
  if ((want == CVN_ROUTE_FUSED && !fused_ok) || (want == CVN_ROUTE_PFA268 && !pfa_ok))
    return fail(CVN_ERR_ARG, "route %d does not serve a %dx%d plane at scale %d", want, g->h, g->w, g->s);
  r->id = want;
  if (want == CVN_ROUTE_FUSED) {
    r->table_bytes = fws;
    r->scratch_bytes = fused_scratch(g->P, g->H, g->W, g->pad, g->s);
    return CVN_OK;
  }
  PlanTabs t;
  if (!plan_tabs(*g, &t)) return fail(CVN_ERR_UNSUPPORTED, "no FFT plan for this plane size");
  const ModWs w = module_ws(*g, t);
  r->table_bytes = w.S;
  r->scratch_bytes = want == CVN_ROUTE_PFA268 ? std::max(w.total - w.S, pfa268_scratch_bytes(g->P)) : w.total - w.S;
  return CVN_OK;
}

int check_mode_act(int64_t H, int64_t W, int pad, int pad_mode, int act) {
  if (pad_mode < CVN_PAD_ZEROS || pad_mode > CVN_PAD_CIRCULAR) return fail(CVN_ERR_ARG, "bad padding mode");
  if (pad_mode == CVN_PAD_REFLECT && (pad >= H || pad >= W))
    return fail(CVN_ERR_ARG, "reflect padding must be smaller than the input size");
  if (pad_mode == CVN_PAD_CIRCULAR && (pad > H || pad > W))
    return fail(CVN_ERR_ARG, "circular padding must not exceed the input size");
  if (act != CVN_ACT_NONE && act != CVN_ACT_GELU) return fail(CVN_ERR_ARG, "bad activation");
  return CVN_OK;
}

// ---- backward workspace: plan tables, module table, HR grad spectra (later dy), LR spectra / dS,
// and for weight gradients dPhi, dK, the column-transposed DFT T and the per-block lambda sums.
constexpr size_t kBwdWsAlign = 256;  // alignment of the backward's workspace regions
struct BwdWs {
  size_t tabs, phi, Sg, Sx, dphi, dK, T, part, total;
  int vc, nchunk, lds;
};
constexpr int kGradLds = 64 * 1024;
void bwd_layout(const Geo& g, const PlanTabs& t, BwdWs* w) {
  size_t o = 0;
  w->tabs = o; o += align_up(t.bytes);
  w->phi = o; o += align_up((size_t)g.Cp * g.NCs * g.Hs * sizeof(float2));
  // Sg: row spectra of the output gradient, then the padding adjoint's border rows (P 2 pad W floats)
  w->Sg = o; o += align_up((size_t)g.P * g.NCs * g.Hs * sizeof(float2));
  w->Sx = o; o += align_up((size_t)g.P * g.NC * g.h * sizeof(float2));
  // weight-gradient chunks over all w column classes, as in launch_phi
  w->nchunk = (int)std::min<int64_t>(g.w, std::max<int64_t>(1, (2048 + g.Cp - 1) / g.Cp));
  w->vc = (g.w + w->nchunk - 1) / w->nchunk;
  while (w->vc > 1 && phi_tile_lds(g.s, g.Hs, g.kh, g.kw, w->vc).total > kGradLds) --w->vc;
  w->lds = phi_tile_lds(g.s, g.Hs, g.kh, g.kw, w->vc).total;
  w->nchunk = (g.w + w->vc - 1) / w->vc;
  w->dphi = o; o += align_up((size_t)g.Cp * g.Ws * g.Hs * sizeof(float2));
  w->dK = o; o += align_up((size_t)g.Cp * g.Ws * g.Hs * sizeof(float2));
  w->T = o; o += align_up((size_t)g.Cp * g.Hs * g.kw * sizeof(double2));
  w->part = o; o += align_up((size_t)g.Cp * w->nchunk * sizeof(double));
  w->total = o;
}

// Every limit of the backward for this geometry: the workspace layout, the column pass's classes per
// block and LDS, or CVN_ERR_UNSUPPORTED with the reason.  wg: weight or bias gradients wanted.
int bwd_check(const Geo& g, bool wg, PlanTabs* t, BwdWs* ws, int* cpb, size_t* col_lds) {
  if (g.P > 65535) return fail(CVN_ERR_UNSUPPORTED, "B*C = %lld planes exceeds 65535", (long long)g.P);
  if (wg && g.s > 4) return fail(CVN_ERR_UNSUPPORTED, "weight gradients support scale <= 4");
  if (!plan_tabs(g, t)) return fail(CVN_ERR_UNSUPPORTED, "no FFT plan for this plane size");
  bwd_layout(g, *t, ws);
  if (wg && ws->lds > kGradLds) return fail(CVN_ERR_UNSUPPORTED, "plane too large for the weight gradient");
  // column pass: up to 8 classes per block, LDS within 80 KiB where possible (2 blocks per CU)
  const size_t rad = rader_lds_bytes(t->plan[kTabH]) + rader_lds_bytes(t->plan[kTabHs]);
  *cpb = std::max(1, std::min(8, g.NC));
  while (*cpb > 1 && align_up(cols_bwd_lds(g.h, g.Hs, g.s, *cpb, wg), 16) + rad > 80 * 1024) --*cpb;
  *col_lds = align_up(cols_bwd_lds(g.h, g.Hs, g.s, *cpb, wg), 16) + rad;
  if (*col_lds > kLdsLimit) return fail(CVN_ERR_UNSUPPORTED, "plane too large for the backward column pass");
  if (wg && g.Cp * ws->nchunk > 0x7fffffff) return fail(CVN_ERR_UNSUPPORTED, "too many gradient blocks");
  if (wg && g.Cp > 65535) return fail(CVN_ERR_UNSUPPORTED, "too many psf planes");
  return CVN_OK;
}

}  // namespace

extern "C" int cvn_converse2d_route(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw,
                                    int scale, int pad) {
  Geo g;
  Route r;
  const int rc = module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, CVN_ROUTE_AUTO, &g, &r);
  return rc != CVN_OK ? rc : r.id;
}

extern "C" size_t cvn_converse2d_table_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh,
                                             int kw, int scale, int pad, int route) {
  Geo g;
  Route r;
  if (module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, route, &g, &r) != CVN_OK) return 0;
  return r.table_bytes;
}

extern "C" size_t cvn_converse2d_scratch_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                               int kh, int kw, int scale, int pad, int route) {
  Geo g;
  Route r;
  if (module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, route, &g, &r) != CVN_OK) return 0;
  return r.scratch_bytes;
}

extern "C" size_t cvn_converse2d_fwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W,
                                               int64_t psf_batch, int kh, int kw, int scale,
                                               int pad) {
  Geo g;
  Route r;
  if (module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, CVN_ROUTE_AUTO, &g, &r) != CVN_OK) return 0;
  return align_up(r.table_bytes) + r.scratch_bytes;
}

extern "C" int cvn_converse2d_table_f32(const float* psf, int64_t psf_batch, int kh, int kw, const float* bias,
                                        float eps, int64_t B, int64_t C, int64_t H, int64_t W, int scale, int pad,
                                        int route, void* table, size_t table_bytes, cvn_stream_t stream) {
  Geo g;
  Route r;
  int rc = module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, route, &g, &r);
  if (rc != CVN_OK) return rc;
  if (!psf || !bias) return fail(CVN_ERR_ARG, "null pointer");
  if (!table || table_bytes < r.table_bytes)
    return fail(CVN_ERR_WORKSPACE, "table buffer too small: need %zu bytes", r.table_bytes);
  hipStream_t st = (hipStream_t)stream;
  if (r.id == CVN_ROUTE_FUSED) {
    // 256 x 256 HR planes (s = 1, or the up kernel at s = 4): the split-DFT table kernel writes the
    // fused plan's slot order directly (a per-sample 25 x 25 psf, Converse-USRNet's data steps, is
    // several times faster there than in k_phi_fused / k_phi_fused_up); the fused kernels' own table
    // kernels otherwise
    if (g.Hs == 256 && g.Ws == 256 &&
        launch_phi(psf, bias, eps, g, false, (float2*)table, nullptr, st, kPhiFused256) == CVN_OK)
      return CVN_OK;
    return fused_table(psf, bias, eps, g.C, g.Cp / g.C, kh, kw, g.H, g.W, g.pad, g.s, table, st);
  }
  PlanTabs t;
  if (!plan_tabs(g, &t)) return fail(CVN_ERR_UNSUPPORTED, "no FFT plan for this plane size");
  const ModWs ws = module_ws(g, t);
  if ((rc = launch_plan_tabs(t, (char*)table + ws.tabs, st)) != CVN_OK) return rc;
  return launch_phi(psf, bias, eps, g, false, (float2*)table, nullptr, st,
                    r.id == CVN_ROUTE_PFA268 ? kPhiPfa268 : kPhiGeneric);
}

extern "C" int cvn_converse2d_apply_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                                        int64_t psf_batch, int kh, int kw, int scale, int pad, int pad_mode,
                                        int act, int route, const void* table, size_t table_bytes, void* scratch,
                                        size_t scratch_bytes, float* out, cvn_stream_t stream) {
  Geo g;
  Route r;
  int rc = module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, route, &g, &r);
  if (rc != CVN_OK) return rc;
  if ((rc = check_mode_act(H, W, pad, pad_mode, act)) != CVN_OK) return rc;
  if (!x || !table || !out) return fail(CVN_ERR_ARG, "null pointer");
  if (table_bytes < r.table_bytes)
    return fail(CVN_ERR_ARG, "table of %zu bytes is smaller than route %d needs (%zu)", table_bytes, r.id,
                r.table_bytes);
  if (B == 0) return CVN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (r.id == CVN_ROUTE_FUSED) {
    if (((uintptr_t)x & 15) || ((uintptr_t)out & 15))
      return fail(CVN_ERR_ARG, "the fused kernel needs 16-byte aligned input and output");
    if (B * C > 0x7fffffff) return fail(CVN_ERR_UNSUPPORTED, "too many planes");
    // scratch is optional here: with it, a few planes run split over twice the workgroups
    if (scratch && scratch_bytes < r.scratch_bytes)
      return fail(CVN_ERR_WORKSPACE, "scratch too small: need %zu bytes", r.scratch_bytes);
    return fused_apply(x, B, C, g.H, g.W, g.Cp / g.C, pad, pad_mode, act, g.s, table,
                       r.scratch_bytes > 0 ? scratch : nullptr, out, st);
  }
  if (!scratch || scratch_bytes < r.scratch_bytes)
    return fail(CVN_ERR_WORKSPACE, "scratch too small: need %zu bytes", r.scratch_bytes);
  if (g.P > 65535) return fail(CVN_ERR_UNSUPPORTED, "B*C = %lld planes exceeds 65535", (long long)g.P);
  set_lds_attrs();
  PlanTabs t;
  if (!plan_tabs(g, &t)) return fail(CVN_ERR_UNSUPPORTED, "no FFT plan for this plane size");
  const ModWs ws = module_ws(g, t);
  char* base = (char*)scratch - ws.S;  // scratch holds the workspace regions after the table
  const float2* phi = (const float2*)table;
  const char* tabs = (const char*)table + ws.tabs;
  float2* S = (float2*)(base + ws.S);
  float2* SH = (float2*)(base + ws.SH);
  if (r.id == CVN_ROUTE_PFA268)
    return pfa268_forward(x, g.P, g.C, g.Cp / g.C, g.H, g.W, g.pad, pad_mode, act, phi, S, out, st);
  if (module_ct_supported(g.h, g.w, g.s, g.pad) && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0)
    return launch_module_ct(x, g.P, g.C, g.Cp / g.C, g.h, g.w, g.s, act, (const float2*)(tabs + t.off[kTabW]),
                            (const float2*)(tabs + t.off[kTabH]), (const float2*)(tabs + t.off[kTabHs]),
                            (const float2*)(tabs + t.off[kTabWs]), phi, S, SH, out, st);
  if ((rc = launch_rows_fwd(x, g.P, g.H, g.W, g.pad, pad_mode, g.h, g.w, tabs + t.off[kTabW], S, st)) != CVN_OK)
    return rc;
  ColModArgs ca;
  ca.S = S; ca.phi = phi; ca.SH = SH; ca.C = g.C; ca.psf_batch = g.Cp / g.C;
  ca.h = g.h; ca.w = g.w; ca.Hs = g.Hs; ca.Ws = g.Ws; ca.NC = g.NC; ca.NCs = g.NCs;
  ca.cpb = cols_per_block(g.h, g.Hs);
  if (!make_plan(g.h, &ca.plan_h) || !make_plan(g.Hs, &ca.plan_H))
    return fail(CVN_ERR_UNSUPPORTED, "no plan for column length");
  ca.tabs_h = tabs + t.off[kTabH];
  ca.tabs_H = tabs + t.off[kTabHs];
  ca.rad_off = (int)align_up(cols_lds(g.h, g.Hs, ca.cpb), 16);
  hipLaunchKernelGGL(k_cols_module, dim3((g.NCs + ca.cpb - 1) / ca.cpb, (unsigned)g.P), dim3(kThreads),
                     ca.rad_off + rader_lds_bytes(ca.plan_h) + rader_lds_bytes(ca.plan_H), st, ca);
  if ((rc = check_launch("column pass")) != CVN_OK) return rc;
  const int ps = g.pad * g.s;
  return launch_rows_inv(SH, g, ps, g.H * g.s, ps, g.W * g.s, act, tabs + t.off[kTabWs], out, st);
}

extern "C" int cvn_converse2d_fwd_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                                      const float* psf, int64_t psf_batch, int kh, int kw,
                                      const float* bias, float eps, int scale, int pad,
                                      int pad_mode, int act, float* out, void* workspace,
                                      size_t workspace_bytes, cvn_stream_t stream) {
  Geo g;
  Route r;
  int rc = module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, CVN_ROUTE_AUTO, &g, &r);
  if (rc != CVN_OK) return rc;
  if ((rc = check_mode_act(H, W, pad, pad_mode, act)) != CVN_OK) return rc;
  if (!x || !psf || !bias || !out) return fail(CVN_ERR_ARG, "null pointer");
  if (B == 0) return CVN_OK;
  const size_t tb = align_up(r.table_bytes);
  if (!workspace || workspace_bytes < tb + r.scratch_bytes)
    return fail(CVN_ERR_WORKSPACE, "workspace too small: need %zu bytes", tb + r.scratch_bytes);
  char* base = (char*)workspace;
  rc = cvn_converse2d_table_f32(psf, psf_batch, kh, kw, bias, eps, B, C, H, W, scale, pad, r.id, base, tb, stream);
  if (rc != CVN_OK) return rc;
  return cvn_converse2d_apply_f32(x, B, C, H, W, psf_batch, kh, kw, scale, pad, pad_mode, act, r.id, base, tb,
                                  base + tb, workspace_bytes - tb, out, stream);
}

// Op-level path: the table (FFT plan tables, the OTF K and the alias-class table A of the psf) depends
// on (psf, bias, eps, C, h, w, scale) only, like the reference's cached OTF (converse2d.cpp:52-102);
// the scratch holds the row spectra of x and x0 and the HR spectra between the passes.
namespace {
struct OpLayout {
  PlanTabs t;
  size_t kf, A, table;       // table regions
  size_t S, S0, SH, scratch;  // scratch regions
};
size_t op_col_lds(const Geo& g, const OpLayout& L) {
  return align_up((size_t)(3 * g.h + g.Hs + 2 * g.s * g.Hs) * sizeof(float2), 16) +
         rader_lds_bytes(L.t.plan[kTabH]) + rader_lds_bytes(L.t.plan[kTabHs]);
}
int op_layout(int64_t B, int64_t C, int64_t h, int64_t w, int kh, int kw, int scale, Geo* g, OpLayout* L) {
  int rc = module_geo(B, C, h, w, 1, kh, kw, scale, 0, g);
  if (rc != CVN_OK) return rc;
  if (!plan_tabs(*g, &L->t)) return fail(CVN_ERR_UNSUPPORTED, "no FFT plan for this plane size");
  size_t o = L->t.bytes;
  L->kf = o; o += align_up((size_t)g->C * g->Ws * g->Hs * sizeof(float2));
  L->A = o; o += align_up((size_t)g->C * g->Ws * g->Hs * sizeof(float2));
  L->table = o;
  o = 0;
  L->S = o; o += align_up((size_t)g->P * g->NC * g->h * sizeof(float2));
  L->S0 = o; o += align_up((size_t)g->P * g->NCs * g->Hs * sizeof(float2));
  L->SH = o; o += align_up((size_t)g->P * g->NCs * g->Hs * sizeof(float2));
  L->scratch = o;
  // the apply's launch limits, checked here so that every query (table, scratch, workspace) answers
  // 0 for a geometry the apply would reject
  if (g->P > 65535) return fail(CVN_ERR_UNSUPPORTED, "B*C exceeds 65535");
  if (op_col_lds(*g, *L) > kLdsLimit) return fail(CVN_ERR_UNSUPPORTED, "column class does not fit in LDS");
  return CVN_OK;
}
}  // namespace

extern "C" int cvn_converse2d_op_route(int64_t h, int64_t w, int scale) {
  if (h < 1 || w < 1 || h > kMaxFftLen || w > kMaxFftLen) return CVN_ROUTE_GENERIC;
  return op_ct_supported((int)h, (int)w, scale) ? CVN_ROUTE_OP_PLANNED : CVN_ROUTE_GENERIC;
}

extern "C" size_t cvn_converse2d_op_table_bytes(int64_t C, int64_t h, int64_t w, int kh, int kw, int scale) {
  Geo g;
  OpLayout L;
  if (op_layout(1, C, h, w, kh, kw, scale, &g, &L) != CVN_OK) return 0;
  return L.table;
}

extern "C" size_t cvn_converse2d_op_scratch_bytes(int64_t B, int64_t C, int64_t h, int64_t w, int scale) {
  Geo g;
  OpLayout L;
  if (op_layout(B, C, h, w, 1, 1, scale, &g, &L) != CVN_OK) return 0;
  return L.scratch;
}

extern "C" size_t cvn_converse2d_op_workspace(int64_t B, int64_t C, int64_t h, int64_t w, int kh,
                                              int kw, int scale) {
  Geo g;
  OpLayout L;
  if (op_layout(B, C, h, w, kh, kw, scale, &g, &L) != CVN_OK) return 0;
  return L.table + L.scratch;
}

extern "C" int cvn_converse2d_op_table_f32(const float* psf, int kh, int kw, const float* bias, float eps, int64_t C,
                                           int64_t h, int64_t w, int scale, void* table, size_t table_bytes,
                                           cvn_stream_t stream) {
  Geo g;
  OpLayout L;
  int rc = op_layout(1, C, h, w, kh, kw, scale, &g, &L);
  if (rc != CVN_OK) return rc;
  if (!psf || !bias) return fail(CVN_ERR_ARG, "null pointer");
  if (!table || table_bytes < L.table)
    return fail(CVN_ERR_WORKSPACE, "table buffer too small: need %zu bytes", L.table);
  hipStream_t st = (hipStream_t)stream;
  char* base = (char*)table;
  if ((rc = launch_plan_tabs(L.t, base, st)) != CVN_OK) return rc;
  return launch_phi(psf, bias, eps, g, true, (float2*)(base + L.A), (float2*)(base + L.kf), st);
}

extern "C" int cvn_converse2d_op_apply_f32(const float* x, const float* x0, int64_t B, int64_t C, int64_t h,
                                           int64_t w, int scale, const void* table, size_t table_bytes,
                                           void* scratch, size_t scratch_bytes, float* out, cvn_stream_t stream) {
  Geo g;
  OpLayout L;
  int rc = op_layout(B, C, h, w, 1, 1, scale, &g, &L);
  if (rc != CVN_OK) return rc;
  if (!x || !x0 || !table || !out) return fail(CVN_ERR_ARG, "null pointer");
  if (table_bytes < L.table) return fail(CVN_ERR_ARG, "op table of %zu bytes, need %zu", table_bytes, L.table);
  if (B == 0) return CVN_OK;
  if (!scratch || scratch_bytes < L.scratch)
    return fail(CVN_ERR_WORKSPACE, "scratch too small: need %zu bytes", L.scratch);
  const size_t lds = op_col_lds(g, L);  // within kLdsLimit (op_layout)
  set_lds_attrs();
  hipStream_t st = (hipStream_t)stream;
  const char* tabs = (const char*)table;
  const float2* kf = (const float2*)(tabs + L.kf);
  const float2* Am = (const float2*)(tabs + L.A);
  char* sc = (char*)scratch;
  float2* S = (float2*)(sc + L.S);
  float2* S0 = (float2*)(sc + L.S0);
  float2* SH = (float2*)(sc + L.SH);
  if (op_ct_supported(g.h, g.w, g.s) && (uintptr_t)x % 16 == 0 && (uintptr_t)x0 % 16 == 0 && (uintptr_t)out % 16 == 0)
    return launch_op_ct(x, x0, g.P, g.C, g.h, g.w, g.s, (const float2*)(tabs + L.t.off[kTabW]),
                        (const float2*)(tabs + L.t.off[kTabH]), (const float2*)(tabs + L.t.off[kTabHs]),
                        (const float2*)(tabs + L.t.off[kTabWs]), kf, Am, S, S0, SH, out, st);
  if ((rc = launch_rows_fwd(x, g.P, g.h, g.w, 0, CVN_PAD_ZEROS, g.h, g.w, tabs + L.t.off[kTabW], S, st)) != CVN_OK)
    return rc;
  if ((rc = launch_rows_fwd(x0, g.P, g.Hs, g.Ws, 0, CVN_PAD_ZEROS, g.Hs, g.Ws, tabs + L.t.off[kTabWs], S0, st)) !=
      CVN_OK)
    return rc;
  ColOpArgs ca;
  ca.S = S; ca.S0 = S0; ca.kf = kf; ca.A = Am; ca.SH = SH; ca.C = g.C;
  ca.h = g.h; ca.w = g.w; ca.s = g.s; ca.Hs = g.Hs; ca.Ws = g.Ws; ca.NC = g.NC; ca.NCs = g.NCs;
  ca.plan_h = L.t.plan[kTabH];
  ca.plan_H = L.t.plan[kTabHs];
  ca.tabs_h = tabs + L.t.off[kTabH];
  ca.tabs_H = tabs + L.t.off[kTabHs];
  ca.rad_off = (int)align_up((size_t)(3 * g.h + g.Hs + 2 * g.s * g.Hs) * sizeof(float2), 16);
  hipLaunchKernelGGL(k_cols_op, dim3(g.w, (unsigned)g.P), dim3(kThreads), lds, st, ca);
  if ((rc = check_launch("op column pass")) != CVN_OK) return rc;
  return launch_rows_inv(SH, g, 0, g.Hs, 0, g.Ws, CVN_ACT_NONE, tabs + L.t.off[kTabWs], out, st);
}

extern "C" int cvn_converse2d_op_f32(const float* x, const float* x0, int64_t B, int64_t C,
                                     int64_t h, int64_t w, const float* psf, int kh, int kw,
                                     const float* bias, float eps, int scale, float* out,
                                     void* workspace, size_t workspace_bytes,
                                     cvn_stream_t stream) {
  Geo g;
  OpLayout L;
  int rc = op_layout(B, C, h, w, kh, kw, scale, &g, &L);
  if (rc != CVN_OK) return rc;
  if (!x || !x0 || !psf || !bias || !out) return fail(CVN_ERR_ARG, "null pointer");
  if (B == 0) return CVN_OK;
  if (!workspace || workspace_bytes < L.table + L.scratch)
    return fail(CVN_ERR_WORKSPACE, "workspace too small: need %zu bytes", L.table + L.scratch);
  char* base = (char*)workspace;
  if ((rc = cvn_converse2d_op_table_f32(psf, kh, kw, bias, eps, C, h, w, scale, base, L.table, stream)) != CVN_OK)
    return rc;
  return cvn_converse2d_op_apply_f32(x, x0, B, C, h, w, scale, base, L.table, base + L.table,
                                     workspace_bytes - L.table, out, stream);
}

// ------------------------------------------------------------------------------------------------
// Backward of the module path (Converse2D.forward, util_converse.py:142-192, differentiated as the
// reference's CompositeImplicitAutograd registration does, converse2d.cpp:223-227).
// ------------------------------------------------------------------------------------------------
extern "C" size_t cvn_converse2d_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                               int kh, int kw, int scale, int pad) {
  Geo g;
  if (module_geo(B, C, H, W, psf_batch, kh, kw, scale, pad, &g) != CVN_OK) return 0;
  PlanTabs t;
  if (!plan_tabs(g, &t)) return 0;
  BwdWs w;
  bwd_layout(g, t, &w);
  return w.total + kBwdWsAlign;  // slack to align the caller's pointer (cvn_converse2d_bwd_f32)
}

extern "C" int cvn_converse2d_bwd_f32(const float* grad_out, const float* x, int64_t B, int64_t C, int64_t H,
                                      int64_t W, const float* psf, int64_t psf_batch, int kh, int kw,
                                      const float* bias, float eps, int scale, int pad, int pad_mode, float* grad_x,
                                      float* grad_psf, float* grad_bias, void* workspace, size_t workspace_bytes,
                                      cvn_stream_t stream) {
  Geo g;
  int rc = module_geo(B, C, H, W, psf_batch, kh, kw, scale, pad, &g);
  if (rc != CVN_OK) return rc;
  if ((rc = check_mode_act(H, W, pad, pad_mode, CVN_ACT_NONE)) != CVN_OK) return rc;
  const bool wg = grad_psf || grad_bias;
  if (!grad_out || !psf || !bias || (wg && !x)) return fail(CVN_ERR_ARG, "null pointer");
  if (!grad_x && !wg) return CVN_OK;
  if (B == 0) return CVN_OK;
  PlanTabs t;
  BwdWs ws;
  int cpb;
  size_t col_lds;
  if ((rc = bwd_check(g, wg, &t, &ws, &cpb, &col_lds)) != CVN_OK) return rc;
  // the regions are laid out from a 256-byte aligned base inside the caller's workspace, whatever the
  // pointer's alignment (the kernels read them with 16-byte loads and direct-to-LDS copies)
  const size_t skew = workspace ? (kBwdWsAlign - (uintptr_t)workspace % kBwdWsAlign) % kBwdWsAlign : 0;
  if (!workspace || workspace_bytes < ws.total + skew)
    return fail(CVN_ERR_WORKSPACE, "workspace too small: need %zu bytes", ws.total + kBwdWsAlign);
  hipStream_t st = (hipStream_t)stream;
  set_lds_attrs();
  char* base = (char*)workspace + skew;
  const char* tabs = base + ws.tabs;
  float2* phi = (float2*)(base + ws.phi);
  float2* Sg = (float2*)(base + ws.Sg);
  float2* Sx = (float2*)(base + ws.Sx);
  if ((rc = launch_plan_tabs(t, base + ws.tabs, st)) != CVN_OK) return rc;
  if ((rc = launch_phi(psf, bias, eps, g, false, phi, nullptr, st)) != CVN_OK) return rc;
  // row spectra of uncrop(grad_out) on the HR grid, and of pad(x) for the weight gradients
  if ((rc = launch_rows_fwd(grad_out, g.P, g.H * g.s, g.W * g.s, g.pad * g.s, CVN_PAD_ZEROS, g.Hs, g.Ws,
                            tabs + t.off[kTabWs], Sg, st)) != CVN_OK)
    return rc;
  if (wg && (rc = launch_rows_fwd(x, g.P, g.H, g.W, g.pad, pad_mode, g.h, g.w, tabs + t.off[kTabW], Sx, st)) !=
                CVN_OK)
    return rc;
  // column pass: dS (in place over Sx) and dPhi
  {
    ColBwdArgs a;
    a.Sg = Sg; a.Sx = Sx; a.phi = phi; a.dphi = wg ? (float2*)(base + ws.dphi) : nullptr;
    a.B = g.B; a.C = g.C; a.psf_batch = g.Cp / g.C;
    a.h = g.h; a.w = g.w; a.s = g.s; a.Hs = g.Hs; a.Ws = g.Ws; a.NC = g.NC; a.NCs = g.NCs;
    a.plan_h = t.plan[kTabH]; a.plan_H = t.plan[kTabHs];
    a.tabs_h = tabs + t.off[kTabH]; a.tabs_H = tabs + t.off[kTabHs];
    a.cpb = cpb;
    a.rad_off = (int)align_up(cols_bwd_lds(g.h, g.Hs, g.s, a.cpb, wg), 16);
    const size_t lds = col_lds;
    const dim3 grid((unsigned)((g.NC + a.cpb - 1) / a.cpb), (unsigned)(a.psf_batch == 1 ? g.C : g.P));
    const int hc = g.s == 1 ? g.h : 0;  // column lengths with a compile-time plan (scale 1)
    switch (hc) {
      case 132: hipLaunchKernelGGL(k_cols_bwd<132>, grid, dim3(kColsBwdThreads), lds, st, a); break;
      case 256: hipLaunchKernelGGL(k_cols_bwd<256>, grid, dim3(kColsBwdThreads), lds, st, a); break;
      case 260: hipLaunchKernelGGL(k_cols_bwd<260>, grid, dim3(kColsBwdThreads), lds, st, a); break;
      default: hipLaunchKernelGGL(k_cols_bwd<0>, grid, dim3(kColsBwdThreads), lds, st, a); break;
    }
    if ((rc = check_launch("backward column pass")) != CVN_OK) return rc;
  }
  // dx = pad^T(C2R rows of dS): interior rows and the column folds on the row pass's store, the
  // border rows (in the Sg scratch, free after the column pass) folded in afterwards
  if (grad_x) {
    Geo gl = g;
    gl.Hs = g.h; gl.Ws = g.w; gl.NCs = g.NC;
    float* side = (float*)(base + ws.Sg);
    if ((rc = launch_rows_inv(Sx, gl, 0, g.h, 0, g.w, CVN_ACT_NONE, tabs + t.off[kTabW], grad_x, st, g.pad, pad_mode,
                              side)) != CVN_OK)
      return rc;
    if (pad_mode != CVN_PAD_ZEROS && g.pad > 0) {
      hipLaunchKernelGGL(k_pad_rows_fold, dim3((unsigned)((g.W + 255) / 256), (unsigned)g.P), dim3(256), 0, st, side,
                         g.H, g.W, g.pad, pad_mode, grad_x);
      if ((rc = check_launch("padding adjoint")) != CVN_OK) return rc;
    }
  }
  if (!wg) return CVN_OK;
  {
    PhiArgs a;
    a.psf = psf; a.bias = bias; a.Cp = g.Cp; a.C = (int)g.C; a.kh = g.kh; a.kw = g.kw; a.s = g.s;
    a.h = g.h; a.w = g.w; a.Hs = g.Hs; a.Ws = g.Ws; a.NCs = g.NCs; a.eps = (double)eps;
    a.phi = nullptr; a.kf = nullptr;
    a.nv0 = g.w;
    PhiGradArgs gr;
    gr.dphi = (const float2*)(base + ws.dphi);
    gr.dK = (float2*)(base + ws.dK);
    gr.part = (double*)(base + ws.part);
    const dim3 grid((unsigned)(g.Cp * ws.nchunk));
    switch (g.s) {
      case 1: hipLaunchKernelGGL(k_phi_grad<1>, grid, dim3(kThreads), (size_t)ws.lds, st, a, gr, ws.vc, ws.nchunk); break;
      case 2: hipLaunchKernelGGL(k_phi_grad<2>, grid, dim3(kThreads), (size_t)ws.lds, st, a, gr, ws.vc, ws.nchunk); break;
      case 3: hipLaunchKernelGGL(k_phi_grad<3>, grid, dim3(kThreads), (size_t)ws.lds, st, a, gr, ws.vc, ws.nchunk); break;
      default: hipLaunchKernelGGL(k_phi_grad<4>, grid, dim3(kThreads), (size_t)ws.lds, st, a, gr, ws.vc, ws.nchunk); break;
    }
    if ((rc = check_launch("transfer-function gradient")) != CVN_OK) return rc;
  }
  double2* T = (double2*)(base + ws.T);
  if (grad_psf) {
    const dim3 grid((unsigned)((g.Hs + kGaU - 1) / kGaU), (unsigned)g.Cp);
    hipLaunchKernelGGL(k_psf_grad_a, grid, dim3(kGaU * kGaV), ((size_t)g.Ws + kGaU * kGaV * kJ) * sizeof(double2), st,
                       (const float2*)(base + ws.dK), g.Hs, g.Ws, g.kw, T);
    if ((rc = check_launch("psf gradient (columns)")) != CVN_OK) return rc;
  }
  hipLaunchKernelGGL(k_psf_grad_b, dim3((unsigned)g.C), dim3(256), (size_t)g.Hs * sizeof(double2), st, T,
                     (const double*)(base + ws.part), ws.nchunk, g.C, g.Cp / g.C, g.Hs, g.kh, g.kw, bias, grad_psf,
                     grad_bias);
  return check_launch("psf / bias gradient");
}

extern "C" int cvn_converse2d_supported(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw,
                                        int scale, int pad, int grad_x, int grad_weight) {
  Geo g;
  Route r;
  int rc = module_route(B, C, H, W, psf_batch, kh, kw, scale, pad, CVN_ROUTE_AUTO, &g, &r);
  if (rc != CVN_OK) return rc;
  if (r.id == CVN_ROUTE_FUSED ? B * C > 0x7fffffff : g.P > 65535)
    return fail(CVN_ERR_UNSUPPORTED, "B*C = %lld planes exceeds the forward's grid", (long long)g.P);
  if (!grad_x && !grad_weight) return CVN_OK;
  PlanTabs t;
  BwdWs ws;
  int cpb;
  size_t col_lds;
  return bwd_check(g, grad_weight != 0, &t, &ws, &cpb, &col_lds);
}
