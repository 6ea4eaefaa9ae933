// Device template library of the FUSED path: the building blocks that
// per-plan generated kernels call with every width a compile-time constant.
// It is compiled at run time by hipRTC together with the generated kernel
// (see fused.cpp), so the compiler sees a straight-line op sequence with
// exact tile counts and no runtime guards.
//
// fp32 register tile layout (one wave, NT*16 batch columns):
//   S<T,NT>::v[m][n][e] (lane l, g = l/16, c = l%16) <-> feature 16m + 4g + e,
//                                                      column  col0 + 16n + c,
// which is the D layout of v_mfma_f32_16x16x4f32, and -- contracting the
// feature set {16m + 4k + e : k = 0..3} -- also its B layout, so a dense
// layer feeds the next one straight from registers.  Dense weights arrive
// pre-packed in A-fragment order: 256 values per (output tile, input tile)
// pair, lane l holding elements e = 0..3 of W[16m + 4(l/16) + e][16mo + l%16]
// (fp64 tiles: output row 16mo + 4(r%4) + r/4 for r = l%16, because
// v_mfma_f64_16x16x4f64 returns the 4x4 row blocks transposed; the packing
// undoes it, so fp64 tiles have the same layout).
#pragma once

#include "pointwise.h"

namespace ponni_hip {
namespace fused {

// Element type of the tiles: float, or double where the including kernel
// defines PONNI_REAL as double (F64 plans, v_mfma_f64_16x16x4f64).
#ifndef PONNI_REAL
#define PONNI_REAL float
#endif
typedef PONNI_REAL real;
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef double doublex4 __attribute__((ext_vector_type(4)));
typedef real realx4 __attribute__((ext_vector_type(4)));

// One 16x16x4 MFMA step; fp32 and fp64 share the operand and result layout.
__device__ inline floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ inline doublex4 mfma4(double a, double b, doublex4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}
__device__ inline float d_max(float a, float b) { return fmaxf(a, b); }
__device__ inline double d_max(double a, double b) { return fmax(a, b); }
__device__ inline float d_min(float a, float b) { return fminf(a, b); }
__device__ inline double d_min(double a, double b) { return fmin(a, b); }

// 16-column tiles per wave: 2, or 1 for plans wider than 256 features (the
// generated source then defines PONNI_NT before including this header).
#ifndef PONNI_NT
#define PONNI_NT 2
#endif
constexpr int kNT = PONNI_NT;  // default column tiles of the tile routines

template <int T, int NT = kNT>
struct S {
  realx4 v[T > 0 ? T : 1][NT];
};

struct Lane {
  int lane, g, c;
  int64_t col0, batch;
};

// Cross-lane-group reductions: op(v, lane ^ 16) then op(v, lane ^ 32).  In
// fp32 each step is one v_permlane{16,32}_swap of v with a copy of itself,
// which leaves v's and its partner's values in the two results of every
// lane, combined by op (commutative); fp64 uses the LDS crossbar.
template <class Op>
__device__ inline float xreduce(float v, Op op) {
  auto const a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto const b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
template <class Op>
__device__ inline double xreduce(double v, Op op) {
  v = op(v, __shfl_xor(v, 16));
  return op(v, __shfl_xor(v, 32));
}
__device__ inline real xsum(real v) {
  return xreduce(v, [](real a, real b) { return a + b; });
}
__device__ inline real xmax(real v) {
  return xreduce(v, [](real a, real b) { return d_max(a, b); });
}
__device__ inline real xmin(real v) {
  return xreduce(v, [](real a, real b) { return d_min(a, b); });
}

__device__ inline realx4 ld4(real const* p) { return *reinterpret_cast<realx4 const*>(p); }

// Wave index within the workgroup as a uniform (scalar) value.
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// p plus an opaque zero: loads through the result cannot be hoisted out of
// the loop it is taken in, while p's address space (LDS or global) is kept.
template <class P>
__device__ inline P const* pin(P const* p) {
  int z = 0;
  asm volatile("" : "+s"(z));
  return p + z;
}

// A lane value made opaque at this point: what is derived from it is
// computed here, inside the caller's loop, instead of being hoisted out of
// the tile loop and held in registers (or spilled) for the whole kernel.
__device__ inline int fresh(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Offset of lane (g, c) in a [rows, ld] array: row 4g, column c.
__device__ inline int64_t lane_offset(Lane const& L, int64_t ld) {
  return int64_t(fresh(4 * L.g)) * ld + fresh(L.c);
}

// x [N, batch] (row stride ld) -> tile; rows >= N and columns >= batch read 0.
template <int N, int NT = kNT>
__device__ inline S<(N + 15) / 16, NT> load_rows(real const* __restrict__ x, int64_t ld, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  S<T, NT> s;
  // Row 16m + e of the lane's row group 4g: a uniform offset from one per-lane pointer.
  real const* __restrict__ xl = x + lane_offset(L, ld) + L.col0;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        s.v[m][n][e] = (f < N && col_ok) ? xl[int64_t(16 * m + e) * ld + 16 * n] : 0.0f;
      }
    }
  return s;
}

// The same in contraction order (input states read only by dense
// contractions, plan.cpp input_contractions): lane group g, element e of
// tile m holds feature 4(4m + e) + g, so the padding rows fill whole
// contraction steps at the end.
template <int N, int NT = kNT>
__device__ inline S<(N + 15) / 16, NT> load_rows_k(real const* __restrict__ x, int64_t ld, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  S<T, NT> s;
  // Row 16m + 4e of the lane's row g: a uniform offset from one per-lane pointer.
  real const* __restrict__ xl = x + int64_t(fresh(L.g)) * ld + fresh(L.c) + L.col0;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 4 * (4 * m + e) + L.g;
        s.v[m][n][e] = (f < N && col_ok) ? xl[int64_t(16 * m + 4 * e) * ld + 16 * n] : 0.0f;
      }
    }
  return s;
}

template <int N, int T, int NT>
__device__ inline void store_rows(S<T, NT> const& s, real* __restrict__ y, int64_t ld, Lane const& L) {
  real* __restrict__ yl = y + lane_offset(L, ld) + L.col0;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        if (f < N && col_ok) yl[int64_t(16 * m + e) * ld + 16 * n] = s.v[m][n][e];
      }
    }
}

template <int T, int NT = kNT>
__device__ inline S<T, NT> zeros() {
  S<T, NT> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = realx4{0.0f, 0.0f, 0.0f, 0.0f};
  return s;
}

// out = C + W^T in over TI input tiles and TO output tiles, with the
// epilogue of output tile mo-1 issued after the MFMAs of tile mo (so its VALU
// work overlaps the matrix pipe) and the A fragments streamed through an
// R-deep register ring: fragment i + R is requested while fragment i is
// consumed.  epi(mo, tile) finishes one output tile in place.  IL > 0 pins
// each epilogue among the next tile's MFMAs, IL VALU (and as many
// transcendentals) per input tile of MFMAs.  Contraction step 4m + e runs
// for 4m + e < KS only (an input state in contraction order, load_rows_k,
// ends in all-padding steps).
template <int IL, int TI, int TO, int KS = 4 * TI, int NT, class Epi, int D = 4>
__device__ inline S<TO, NT> dense_ep_il(S<TI, NT> const& in, real const* __restrict__ w, S<TO, NT> acc,
                                        Lane const& L, Epi epi) {
  static_assert(KS > 4 * (TI - 1) && KS <= 4 * TI, "every input tile holds a step");
  constexpr int NF = TI * TO;
  constexpr int R = D < NF ? D : NF;
  realx4 ring[R];
#pragma unroll
  for (int i = 0; i < R; i++) ring[i] = ld4(w + i * 256 + L.lane * 4);
#pragma unroll
  for (int mo = 0; mo < TO; mo++) {
    // (interleaving: one scheduling region per output tile)
    if (IL > 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < TI; m++) {
      int const i = mo * TI + m;
      realx4 const a = ring[i % R];
      if (i + R < NF) ring[i % R] = ld4(w + (i + R) * 256 + L.lane * 4);
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (4 * m + e < KS)
#pragma unroll
          for (int n = 0; n < NT; n++)
            acc.v[mo][n] = mfma4(a[e], in.v[m][n][e], acc.v[mo][n]);
    }
    if (mo > 0) {
      epi(mo - 1, acc.v[mo - 1]);
      // (pure arithmetic floats to its uses unless something ordered reads it)
      if (IL > 0)
#pragma unroll
        for (int n = 0; n < NT; n++) asm volatile("" : "+v"(acc.v[mo - 1][n]));
      // Keep that epilogue between this tile's MFMAs: left alone, its pure
      // arithmetic floats down to its first use (the next layer), so every
      // tile's epilogue runs after the layer's last MFMA.  The empty asm
      // above orders the results within this tile's scheduling region (a
      // sched_barrier at the top of each tile); per input tile (4 NT MFMAs)
      // up to IL VALU and as many transcendentals follow.
      if (IL > 0) {
#pragma unroll
        for (int k = 0; k + 1 < TI; k++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 4 * NT, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, IL, 0);
          __builtin_amdgcn_sched_group_barrier(0x400, IL, 0);
        }
        // (the last input tile holds KS - 4 (TI - 1) steps)
        __builtin_amdgcn_sched_group_barrier(0x008, (KS - 4 * (TI - 1)) * NT, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, IL, 0);
        __builtin_amdgcn_sched_group_barrier(0x400, IL, 0);
      }
    }
  }
  epi(TO - 1, acc.v[TO - 1]);
  return acc;
}

template <int TI, int TO, int KS = 4 * TI, int NT, class Epi, int D = 4>
__device__ inline S<TO, NT> dense_ep(S<TI, NT> const& in, real const* __restrict__ w, S<TO, NT> acc,
                                     Lane const& L, Epi epi) {
  return dense_ep_il<0, TI, TO, KS, NT, Epi, D>(in, w, acc, L, epi);
}

// Per-tile epilogue helpers (tile = one 16-feature row block, NT columns).
template <int NT>
__device__ inline void tile_add_rows(realx4 (&t)[NT], real const* __restrict__ b, int mo, Lane const& L) {
  realx4 const bb = ld4(b + 16 * mo + 4 * L.g);
#pragma unroll
  for (int n = 0; n < NT; n++) t[n] += bb;
}

template <int NT, class F>
__device__ inline void tile_map(realx4 (&t)[NT], F f) {
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int e = 0; e < 4; e++) t[n][e] = f(t[n][e]);
}

template <int N, int NT>
__device__ inline void tile_zero_pad(realx4 (&t)[NT], int mo, Lane const& L) {
#pragma unroll
  for (int e = 0; e < 4; e++)
    if (16 * mo + 4 * L.g + e >= N)
#pragma unroll
      for (int n = 0; n < NT; n++) t[n][e] = 0.0f;
}

// Per-feature vector (bias, gamma, beta) padded to 16*T.
template <int T, int NT>
__device__ inline void add_rows(S<T, NT>& s, real const* __restrict__ b, Lane const& L) {
#pragma unroll
  for (int m = 0; m < T; m++) {
    realx4 const bb = ld4(b + 16 * m + 4 * L.g);
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] += bb;
  }
}

template <int T, int NT, class F>
__device__ inline void map(S<T, NT>& s, F f) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = f(s.v[m][n][e]);
}

// Rows >= N return to exactly zero (they are K padding of the next layer).
template <int N, int T, int NT>
__device__ inline void zero_pad(S<T, NT>& s, Lane const& L) {
  if constexpr (N < 16 * T) {
#pragma unroll
    for (int m = N / 16; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (16 * m + 4 * L.g + e >= N)
#pragma unroll
          for (int n = 0; n < NT; n++) s.v[m][n][e] = 0.0f;
  }
}

template <int T, int NT>
__device__ inline void add(S<T, NT>& s, S<T, NT> const& o) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] += o.v[m][n];
}

// Output tile mo of a contraction plus tile mo of state s (an element-wise
// Add fused into the contraction's epilogue; mo is unrolled there).
template <int T, int NT>
__device__ inline void tile_add_state(realx4 (&t)[NT], S<T, NT> const& s, int mo) {
#pragma unroll
  for (int n = 0; n < NT; n++) t[n] += s.v[mo][n];
}

// Two-pass LayerNorm over N features, ponni_LayerNorm.h:82-98.
template <int N, int T, int NT>
__device__ inline void layer_norm(S<T, NT>& s, real const* __restrict__ gamma, real const* __restrict__ beta,
                                  real eps, Lane const& L) {
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real sum = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) sum += s.v[m][n][e];
    real const mean = xsum(sum) * (1.0f / real(N));
    real q = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) {
          real const d = s.v[m][n][e] - mean;
          q += d * d;
        }
    real const inv_std = 1.0f / d_sqrt(xsum(q) / real(N) + eps);
#pragma unroll
    for (int m = 0; m < T; m++) {
      realx4 const gm = ld4(gamma + 16 * m + 4 * L.g);
      realx4 const bt = ld4(beta + 16 * m + 4 * L.g);
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = gm[e] * ((s.v[m][n][e] - mean) * inv_std) + bt[e];
    }
  }
}

// Softmax / LogSoftmax over N features, ponni_Softmax.h:45-56, ponni_LogSoftmax.h:45-57.
// Softmax's exponentials (arguments <= 0 once the maximum is subtracted)
// and its division on the hardware transcendentals in fp32 -- exp(v) as
// 2^(v log2 e), the quotient as a product with 1 / sum (a sum >= 1) -- each
// within a few ulps of the libm forms; fp64 keeps the libm forms.
__device__ inline float softmax_exp(float v) { return __builtin_amdgcn_exp2f(v * 1.4426950408889634f); }
__device__ inline double softmax_exp(double v) { return exp(v); }
__device__ inline float softmax_recip(float v) { return __builtin_amdgcn_rcpf(v); }
__device__ inline double softmax_recip(double v) { return 1.0 / v; }

template <int N, bool LOG, int T, int NT>
__device__ inline void softmax(S<T, NT>& s, Lane const& L) {
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real mx = -real(__builtin_huge_val());
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) mx = d_max(mx, s.v[m][n][e]);
    mx = xmax(mx);
    real sum = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        real const ex = LOG ? d_exp(s.v[m][n][e] - mx) : softmax_exp(s.v[m][n][e] - mx);
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) sum += ex;
        if (!LOG) s.v[m][n][e] = ex;
      }
    sum = xsum(sum);
    if (LOG) {
      real const lse = d_log(sum) + mx;
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) s.v[m][n][e] -= lse;
    } else {
      real const inv = softmax_recip(sum);
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) s.v[m][n][e] = s.v[m][n][e] * inv;
    }
  }
}

// The reference's running minimum / maximum (MinMaxNorm, ReduceMax,
// ReduceMin, ReduceLogSumExp) starts from feature 0 and replaces it only on
// a strict comparison, so a NaN in feature 0 makes the result NaN and a NaN
// in any other feature is passed over.  The tile reductions use fmin / fmax,
// which pass over every NaN; this supplies feature 0's part: true in every
// lane of column tile n whose feature 0 (lane group 0, element 0 of tile 0)
// is NaN.
template <int T, int NT>
__device__ inline bool first_feature_nan(S<T, NT> const& s, int n, Lane const& L) {
  real const x0 = s.v[0][n][0];
  return xmax(L.g == 0 && x0 != x0 ? real(1) : real(0)) != real(0);
}

// MinMaxNorm over N features, ponni_MinMaxNorm.h:67-84.
template <int N, int T, int NT>
__device__ inline void min_max(S<T, NT>& s, real out_min, real out_max, real eps, Lane const& L) {
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real lo = real(__builtin_huge_val()), hi = -real(__builtin_huge_val());
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) {
          lo = d_min(lo, s.v[m][n][e]);
          hi = d_max(hi, s.v[m][n][e]);
        }
    lo = xmin(lo);
    hi = xmax(hi);
    if (first_feature_nan(s, n, L)) lo = hi = real(__builtin_nanf(""));
    real const scale = (out_max - out_min) / ((hi - lo) + eps);
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = out_min + (s.v[m][n][e] - lo) * scale;
  }
}

// [a; b] for tile-aligned operands.
template <int TA, int TB, int NT>
__device__ inline S<TA + TB, NT> concat(S<TA, NT> const& a, S<TB, NT> const& b) {
  S<TA + TB, NT> s;
#pragma unroll
  for (int m = 0; m < TA; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = a.v[m][n];
#pragma unroll
  for (int m = 0; m < TB; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[TA + m][n] = b.v[m][n];
  return s;
}

// [a; b] when a's N1 features do not fill whole tiles (N1 % 16 != 0): b's
// feature j moves to output feature N1 + j.  Output element e of tile m in
// lane group g holds feature f = 16 m + 4 g + e; with N1 = 16 Q + R and
// e - R = 4 dq + je (0 <= je < 4), the b feature f - N1 sits in element je of
// lane group (g + dq) mod 4, column c, of tile m - Q (or m - Q - 1 when
// g + dq < 0), so every output element is one of two shuffles from the same
// source lane.  Rows >= N1 + N2 stay zero.
template <int N1, int N2, int TA, int TB, int NT>
__device__ inline S<(N1 + N2 + 15) / 16, NT> concat_any(S<TA, NT> const& a, S<TB, NT> const& b, Lane const& L) {
  constexpr int T = (N1 + N2 + 15) / 16;
  constexpr int Q = N1 / 16, R = N1 % 16;
  S<T, NT> out;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      int const d = e - R;
      int const dq = d >= 0 ? 0 : -((3 - d) / 4);
      int const je = d - 4 * dq;
      int const G = L.g + dq;
      int const src = ((G & 3) << 4) | L.c;
      int const f = 16 * m + 4 * L.g + e;
      int const mb = m - Q;
#pragma unroll
      for (int n = 0; n < NT; n++) {
        real const va = m < TA ? a.v[m < TA ? m : 0][n][e] : real(0);
        if (16 * m + 16 <= N1) {  // the whole tile from a
          out.v[m][n][e] = va;
          continue;
        }
        real const v0 = (mb >= 0 && mb < TB) ? __shfl(b.v[(mb >= 0 && mb < TB) ? mb : 0][n][je], src) : real(0);
        real const v1 =
            (mb - 1 >= 0 && mb - 1 < TB) ? __shfl(b.v[(mb - 1 >= 0 && mb - 1 < TB) ? mb - 1 : 0][n][je], src) : real(0);
        real const vb = G < 0 ? v1 : v0;
        out.v[m][n][e] = f < N1 ? va : (f < N1 + N2 ? vb : real(0));
      }
    }
  return out;
}

// Saved residual states may live in LDS instead of registers (one region per
// wave, lane-contiguous 16-byte chunks, so accesses are bank-conflict free).
template <int T, int NT>
__device__ inline void save_lds(S<T, NT> const& s, realx4* __restrict__ slot, Lane const& L) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) slot[(m * NT + n) * 64 + L.lane] = s.v[m][n];
}

template <int T, int NT = kNT>
__device__ inline S<T, NT> load_lds(realx4 const* __restrict__ slot, Lane const& L) {
  S<T, NT> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = slot[(m * NT + n) * 64 + L.lane];
  return s;
}

template <int T, int NT>
__device__ inline void add_lds(S<T, NT>& s, realx4 const* __restrict__ slot, Lane const& L) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] += slot[(m * NT + n) * 64 + L.lane];
}

// ---- generated-graph operations (kokkos_nn/emitter.py) -------------------

// Per-feature vector b broadcast over the tile's columns (a Dense bias that
// seeds the accumulator: sum = bias; sum += W x, emitter.py:701-710).
template <int T, int NT = kNT>
__device__ inline S<T, NT> bias_rows(real const* __restrict__ b, Lane const& L) {
  S<T, NT> s;
#pragma unroll
  for (int m = 0; m < T; m++) {
    realx4 const bb = ld4(b + 16 * m + 4 * L.g);
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = bb;
  }
  return s;
}

// Element-wise op with a constant vector c (padded to 16 T): f(v, c).
template <int NT, class F>
__device__ inline void tile_const(realx4 (&t)[NT], real const* __restrict__ c, int mo, Lane const& L, F f) {
  realx4 const cc = ld4(c + 16 * mo + 4 * L.g);
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int e = 0; e < 4; e++) t[n][e] = f(t[n][e], cc[e]);
}

template <int T, int NT, class F>
__device__ inline void map_const(S<T, NT>& s, real const* __restrict__ c, Lane const& L, F f) {
#pragma unroll
  for (int m = 0; m < T; m++) tile_const(s.v[m], c, m, L, f);
}

// Feature 0 of every column of the wave's tile, in each lane's own column:
// feature 0 sits in lane c (group 0), element 0.
template <int T, int NT>
__device__ inline real feature0(S<T, NT> const& s, int n, Lane const& L) {
  return __shfl(s.v[0][n][0], L.c);
}

// out = f(a, b) over N output features; an operand with one feature (TA or
// TB == 1 with SA / SB set) is broadcast (emitter.py:735-741).
template <int N, bool SA, bool SB, int TA, int TB, int NT, class F>
__device__ inline S<(N + 15) / 16, NT> binary(S<TA, NT> const& a, S<TB, NT> const& b, Lane const& L, F f) {
  constexpr int T = (N + 15) / 16;
  S<T, NT> out;
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real const a0 = SA ? feature0(a, n, L) : 0.0f;
    real const b0 = SB ? feature0(b, n, L) : 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        real const x = SA ? a0 : a.v[SA ? 0 : m][n][e];
        real const y = SB ? b0 : b.v[SB ? 0 : m][n][e];
        out.v[m][n][e] = f(x, y);
      }
  }
  zero_pad<N, T, NT>(out, L);
  return out;
}

// out = cond != 0 ? a : b over N features (interpreter.py Where /
// CompareSelect); an operand with one feature (SC / SA / SB) is broadcast.
template <int N, bool SC, bool SA, bool SB, int TC, int TA, int TB, int NT>
__device__ inline S<(N + 15) / 16, NT> select3(S<TC, NT> const& c, S<TA, NT> const& a, S<TB, NT> const& b,
                                               Lane const& L) {
  constexpr int T = (N + 15) / 16;
  S<T, NT> out;
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real const c0 = SC ? feature0(c, n, L) : real(0);
    real const a0 = SA ? feature0(a, n, L) : real(0);
    real const b0 = SB ? feature0(b, n, L) : real(0);
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        real const x = SC ? c0 : c.v[SC ? 0 : m][n][e];
        real const y = SA ? a0 : a.v[SA ? 0 : m][n][e];
        real const z = SB ? b0 : b.v[SB ? 0 : m][n][e];
        out.v[m][n][e] = apply_select<real>(x, y, z);
      }
  }
  zero_pad<N, T, NT>(out, L);
  return out;
}

__device__ inline real xprod(real v) {
  v *= __shfl_xor(v, 16);
  return v * __shfl_xor(v, 32);
}

// Feature reduction to one feature, emitter.py:475-547; OP is a
// ponni_reduce_op value.  The result is feature 0; padding rows are 0.
// H2 (16-bit plans) follows the generated half2 path's running maximum /
// minimum, TwoHalf::maximum(reduction, value) = reduction > value ?
// reduction : value (emitter.py:578-592, ponni_TwoHalf.h:243-251): every NaN
// is handed on to the next feature, so the result is NaN when the last
// feature is, and otherwise the maximum of the features after the last NaN.
template <int OP, int N, bool H2, int T, int NT>
__device__ inline S<1, NT> reduce(S<T, NT> const& s, Lane const& L) {
  S<1, NT> out;
#pragma unroll
  for (int n = 0; n < NT; n++) {
    real r;
    if constexpr (OP == 2 || OP == 3 || OP == 8) {  // MAX, MIN, LOG_SUM_EXP
      real last = real(-1);  // H2: the last NaN feature (features ascend with m, e)
      if constexpr (H2) {
#pragma unroll
        for (int m = 0; m < T; m++)
#pragma unroll
          for (int e = 0; e < 4; e++)
            if ((N % 16 == 0 || 16 * m + 4 * L.g + e < N) && s.v[m][n][e] != s.v[m][n][e])
              last = real(16 * m + 4 * L.g + e);
        last = xmax(last);
      }
      real mx = OP == 3 ? real(__builtin_huge_val()) : -real(__builtin_huge_val());
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          int const f = 16 * m + 4 * L.g + e;
          if ((N % 16 == 0 || f < N) && (!H2 || real(f) > last))
            mx = OP == 3 ? d_min(mx, s.v[m][n][e]) : d_max(mx, s.v[m][n][e]);
        }
      mx = OP == 3 ? xmin(mx) : xmax(mx);
      if (H2 ? last == real(N - 1) : first_feature_nan(s, n, L)) mx = real(__builtin_nanf(""));
      r = mx;
      if constexpr (OP == 8) {
        real sum = 0.0f;
#pragma unroll
        for (int m = 0; m < T; m++)
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) sum += d_exp(s.v[m][n][e] - mx);
        sum = xsum(sum);
        r = __builtin_isinf(mx) ? mx : mx + d_log(sum);
      }
    } else {
      real acc = OP == 9 ? 1.0f : 0.0f;
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) {
            real const v = s.v[m][n][e];
            if constexpr (OP == 4) acc += d_abs(v);
            else if constexpr (OP == 5 || OP == 6) acc += v * v;
            else if constexpr (OP == 9) acc *= v;
            else acc += v;
          }
      acc = OP == 9 ? xprod(acc) : xsum(acc);
      if constexpr (OP == 1) acc = acc / real(N);
      else if constexpr (OP == 5) acc = d_sqrt(acc);
      else if constexpr (OP == 7) acc = d_log(acc);
      r = acc;
    }
    out.v[0][n] = realx4{L.g == 0 ? r : 0.0f, 0.0f, 0.0f, 0.0f};
  }
  return out;
}

// Copy n4 float4s of one per-feature vector into LDS (no barrier).
__device__ inline void stage_vec(realx4* __restrict__ lds, real const* __restrict__ src, int n4) {
  realx4 const* s4 = reinterpret_cast<realx4 const*>(src);
  for (int i = threadIdx.x; i < n4; i += blockDim.x) lds[i] = s4[i];
}

// Stage `count` values (a multiple of 4) of packed parameters into LDS.
__device__ inline void stage(realx4* __restrict__ lds, real const* __restrict__ src, int count) {
  realx4 const* s4 = reinterpret_cast<realx4 const*>(src);
  for (int i = threadIdx.x; i < count / 4; i += blockDim.x) lds[i] = s4[i];
  __syncthreads();
}

}  // namespace fused
}  // namespace ponni_hip
