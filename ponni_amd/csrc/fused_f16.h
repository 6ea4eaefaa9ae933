// FUSED path, fp16 / bf16 operands with fp32 accumulation.
//
// Register tile H<T,NT,E>::v[m][n] (4 elements of type E per lane) holds the
// same features as the fp32 tile -- lane l, element e <-> feature 16m + 4g + e,
// column col0 + 16n + c -- rounded to E.  A dense layer runs on
// v_mfma_f32_16x16x32_{f16,bf16}: step t contracts 32 features, lane group g,
// element j <-> feature phi(t, g, j) = 16(2t + j/4) + 4g + j%4, which is just
// the concatenation of the lane's own elements of tiles 2t and 2t+1, so the
// B operand needs no data movement.  The host packs A in the same order:
// 1 KB per (output tile, step), lane l holding W[phi(t, l/16, j)][16mo + l%16]
// for j = 0..7.  The fp32 accumulator of each output tile gets its epilogue
// (bias, activation) in fp32 and is rounded to E once, which is where the
// reference model materializes the state.
#pragma once

#include "fused_f32.h"

namespace ponni_hip {
namespace fused {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <class E> struct Vec;
template <> struct Vec<_Float16> {
  using x4 = f16x4;
  using x8 = f16x8;
  __device__ static floatx4 mfma(x8 a, x8 b, floatx4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};
template <> struct Vec<__bf16> {
  using x4 = bf16x4;
  using x8 = bf16x8;
  __device__ static floatx4 mfma(x8 a, x8 b, floatx4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};

template <int T, int NT, class E>
struct H {
  typename Vec<E>::x4 v[T > 0 ? T : 1][NT];
};

// Bias and tanh of one output tile in a single pass:
// tanh(v + b) = 1 - 2 / (1 + 2^(k v + k b)), k = 2 log2(e); five VALU ops per
// element, two of them transcendental.
template <int NT>
__device__ inline void tile_bias_tanh(floatx4 (&t)[NT], float const* __restrict__ b, int mo, Lane const& L) {
  constexpr float k = 2.8853900817779268f;
  floatx4 const kb = ld4(b + 16 * mo + 4 * L.g) * k;
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float const ex = __builtin_amdgcn_exp2f(fmaf(t[n][e], k, kb[e]));
      t[n][e] = fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + ex), 1.0f);
    }
}

#ifndef PONNI_RING_DEPTH
#define PONNI_RING_DEPTH 4
#endif

template <int N, int NT, class E>
__device__ inline H<(N + 15) / 16, NT, E> load_rows_h(E const* __restrict__ x, int64_t ld, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  H<T, NT, E> s;
  E const* __restrict__ xl = x + lane_offset(L, ld) + L.col0;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) {
      bool const col_ok = L.col0 + 16 * n + L.c < L.batch;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        s.v[m][n][e] = (f < N && col_ok) ? xl[int64_t(16 * m + e) * ld + 16 * n] : E(0.0f);
      }
    }
  return s;
}

template <int N, int T, int NT, class E>
__device__ inline void store_rows_h(H<T, NT, E> const& s, E* __restrict__ y, int64_t ld, Lane const& L) {
  E* __restrict__ yl = y + lane_offset(L, ld) + L.col0;
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

template <class E>
__device__ inline typename Vec<E>::x4 round4(floatx4 v) {
  return __builtin_convertvector(v, typename Vec<E>::x4);
}

template <class E>
__device__ inline floatx4 widen4(typename Vec<E>::x4 v) {
  return __builtin_convertvector(v, floatx4);
}

template <int T, int NT, class E>
__device__ inline S<T, NT> to_f32(H<T, NT, E> const& h) {
  S<T, NT> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) s.v[m][n] = widen4<E>(h.v[m][n]);
  return s;
}

template <class E, int T, int NT>
__device__ inline H<T, NT, E> to_h(S<T, NT> const& s) {
  H<T, NT, E> h;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < NT; n++) h.v[m][n] = round4<E>(s.v[m][n]);
  return h;
}

// Dense layer on fp16/bf16 MFMA; returns the rounded output tile.  The
// epilogue of output tile mo-1 runs after the MFMAs of tile mo; A fragments
// stream through an R-deep ring (1 KB per fragment: 16 B per lane).
// If `acc0` is given (projection add) it seeds every output tile's accumulator.
template <int TI, int TO, int NT, class E, class Epi, int D = PONNI_RING_DEPTH>
__device__ inline H<TO, NT, E> dense_h(H<TI, NT, E> const& in, E const* __restrict__ w, Lane const& L, Epi epi) {
  using V8 = typename Vec<E>::x8;
  using V4 = typename Vec<E>::x4;
  constexpr int TS = (TI + 1) / 2;
  constexpr int NF = TS * TO;
  constexpr int R = D < NF ? D : NF;
  H<TO, NT, E> out;
  V8 ring[R];
#pragma unroll
  for (int i = 0; i < R; i++) ring[i] = *reinterpret_cast<V8 const*>(w + i * 512 + L.lane * 8);
  floatx4 prev[NT];
#pragma unroll
  for (int mo = 0; mo < TO; mo++) {
#ifdef PONNI_TILE_BARRIER
    // Keep the workgroup's waves on the same output tile so their identical
    // A-fragment reads hit in L1 after the first wave's miss.
    __syncthreads();
#endif
    floatx4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < TS; t++) {
      int const i = mo * TS + t;
      V8 const a = ring[i % R];
      if (i + R < NF) ring[i % R] = *reinterpret_cast<V8 const*>(w + (i + R) * 512 + L.lane * 8);
#pragma unroll
      for (int n = 0; n < NT; n++) {
        V4 const lo = in.v[2 * t][n];
        V4 const hi = (2 * t + 1 < TI) ? in.v[(2 * t + 1 < TI) ? 2 * t + 1 : 2 * t][n] : V4{E(0.0f), E(0.0f), E(0.0f), E(0.0f)};
        V8 const b = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[n] = Vec<E>::mfma(a, b, acc[n]);
      }
    }
    if (mo > 0) {
      epi(mo - 1, prev);
#pragma unroll
      for (int n = 0; n < NT; n++) out.v[mo - 1][n] = round4<E>(prev[n]);
    }
#pragma unroll
    for (int n = 0; n < NT; n++) prev[n] = acc[n];
  }
  epi(TO - 1, prev);
#pragma unroll
  for (int n = 0; n < NT; n++) out.v[TO - 1][n] = round4<E>(prev[n]);
  return out;
}

// Projection add: out = in + round(b + W^T saved) computed in fp32, rounded once.
template <int TK, int TO, int NT, class E>
__device__ inline void proj_add_h(H<TO, NT, E>& cur, H<TK, NT, E> const& sv, E const* __restrict__ w,
                                  float const* __restrict__ bias, Lane const& L) {
  using V8 = typename Vec<E>::x8;
  using V4 = typename Vec<E>::x4;
  constexpr int TS = (TK + 1) / 2;
#pragma unroll
  for (int mo = 0; mo < TO; mo++) {
    floatx4 const bb = ld4(bias + 16 * mo + 4 * L.g);
    floatx4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) acc[n] = bb;
#pragma unroll
    for (int t = 0; t < TS; t++) {
      V8 const a = *reinterpret_cast<V8 const*>(w + (mo * TS + t) * 512 + L.lane * 8);
#pragma unroll
      for (int n = 0; n < NT; n++) {
        V4 const lo = sv.v[2 * t][n];
        V4 const hi = (2 * t + 1 < TK) ? sv.v[(2 * t + 1 < TK) ? 2 * t + 1 : 2 * t][n] : V4{E(0.0f), E(0.0f), E(0.0f), E(0.0f)};
        acc[n] = Vec<E>::mfma(a, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), acc[n]);
      }
    }
#pragma unroll
    for (int n = 0; n < NT; n++) cur.v[mo][n] = round4<E>(widen4<E>(cur.v[mo][n]) + acc[n]);
  }
}

template <int TA, int TB, int NT, class E>
__device__ inline H<TA + TB, NT, E> concat_h(H<TA, NT, E> const& a, H<TB, NT, E> const& b) {
  H<TA + TB, NT, E> s;
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

}  // namespace fused
}  // namespace ponni_hip
