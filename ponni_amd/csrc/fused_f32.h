// Device template library of the FUSED path (fp32): the building blocks that
// per-plan generated kernels call with every width a compile-time constant.
// It is compiled at run time by hipRTC together with the generated kernel
// (see codegen.cpp), so the compiler sees a straight-line op sequence with
// exact tile counts and no runtime guards.
//
// Register tile layout (one wave, kNT*16 batch columns):
//   S<T>::v[m][n][e] (lane l, g = l/16, c = l%16) <-> feature 16m + 4g + e,
//                                                   column  col0 + 16n + c,
// which is the D layout of v_mfma_f32_16x16x4f32, and -- contracting the
// feature set {16m + 4k + e : k = 0..3} -- also its B layout, so a dense
// layer feeds the next one straight from registers.  Dense weights arrive
// pre-packed in A-fragment order: 256 floats per (output tile, input tile)
// pair, lane l holding elements e = 0..3 of W[16m + 4(l/16) + e][16mo + l%16].
#pragma once

#include "pointwise.h"

namespace ponni_hip {
namespace fused {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kNT = 2;  // 16-column tiles per wave

template <int T>
struct S {
  floatx4 v[T > 0 ? T : 1][kNT];
};

struct Lane {
  int lane, g, c;
  int64_t col0, batch;
};

__device__ inline float xsum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}
__device__ inline float xmax(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}
__device__ inline float xmin(float v) {
  v = fminf(v, __shfl_xor(v, 16));
  return fminf(v, __shfl_xor(v, 32));
}

__device__ inline floatx4 ld4(float const* p) { return *reinterpret_cast<floatx4 const*>(p); }

// An opaque copy of a pointer: loads through it cannot be hoisted out of the
// loop it is taken in.
__device__ inline float const* pin(float const* p) {
  asm volatile("" : "+s"(p));
  return p;
}

// x [N, batch] (row stride ld) -> tile; rows >= N and columns >= batch read 0.
template <int N>
__device__ inline S<(N + 15) / 16> load_rows(float const* __restrict__ x, int64_t ld, Lane const& L) {
  constexpr int T = (N + 15) / 16;
  S<T> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) {
      int64_t const b = L.col0 + 16 * n + L.c;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        s.v[m][n][e] = (f < N && b < L.batch) ? x[int64_t(f) * ld + b] : 0.0f;
      }
    }
  return s;
}

template <int N, int T>
__device__ inline void store_rows(S<T> const& s, float* __restrict__ y, int64_t ld, Lane const& L) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) {
      int64_t const b = L.col0 + 16 * n + L.c;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int const f = 16 * m + 4 * L.g + e;
        if (f < N && b < L.batch) y[int64_t(f) * ld + b] = s.v[m][n][e];
      }
    }
}

// out = C + W^T in over TI input tiles and TO output tiles.
template <int TI, int TO>
__device__ inline S<TO> dense(S<TI> const& in, float const* __restrict__ w, S<TO> acc, Lane const& L) {
#pragma unroll
  for (int mo = 0; mo < TO; mo++) {
    floatx4 a[TI];
#pragma unroll
    for (int m = 0; m < TI; m++) a[m] = ld4(w + ((mo * TI + m) * 64 + L.lane) * 4);
#pragma unroll
    for (int m = 0; m < TI; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int n = 0; n < kNT; n++)
          acc.v[mo][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m][e], in.v[m][n][e], acc.v[mo][n], 0, 0, 0);
  }
  return acc;
}

template <int T>
__device__ inline S<T> zeros() {
  S<T> s;
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) s.v[m][n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  return s;
}

// Per-feature vector (bias, gamma, beta) padded to 16*T, as a tile-shaped constant.
template <int T>
__device__ inline void add_rows(S<T>& s, float const* __restrict__ b, Lane const& L) {
#pragma unroll
  for (int m = 0; m < T; m++) {
    floatx4 const bb = ld4(b + 16 * m + 4 * L.g);
#pragma unroll
    for (int n = 0; n < kNT; n++) s.v[m][n] += bb;
  }
}

template <int T, class F>
__device__ inline void map(S<T>& s, F f) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = f(s.v[m][n][e]);
}

// Rows >= N return to exactly zero (they are K padding of the next layer).
template <int N, int T>
__device__ inline void zero_pad(S<T>& s, Lane const& L) {
  if constexpr (N < 16 * T) {
#pragma unroll
    for (int m = N / 16; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (16 * m + 4 * L.g + e >= N)
#pragma unroll
          for (int n = 0; n < kNT; n++) s.v[m][n][e] = 0.0f;
  }
}

template <int T>
__device__ inline void add(S<T>& s, S<T> const& o) {
#pragma unroll
  for (int m = 0; m < T; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) s.v[m][n] += o.v[m][n];
}

// Two-pass LayerNorm over N features, ponni_LayerNorm.h:82-98.
template <int N, int T>
__device__ inline void layer_norm(S<T>& s, float const* __restrict__ gamma, float const* __restrict__ beta, float eps,
                                  Lane const& L) {
#pragma unroll
  for (int n = 0; n < kNT; n++) {
    float sum = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) sum += s.v[m][n][e];
    float const mean = xsum(sum) * (1.0f / float(N));
    float q = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) {
          float const d = s.v[m][n][e] - mean;
          q += d * d;
        }
    float const inv_std = 1.0f / sqrtf(xsum(q) / float(N) + eps);
#pragma unroll
    for (int m = 0; m < T; m++) {
      floatx4 const gm = ld4(gamma + 16 * m + 4 * L.g);
      floatx4 const bt = ld4(beta + 16 * m + 4 * L.g);
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = gm[e] * ((s.v[m][n][e] - mean) * inv_std) + bt[e];
    }
  }
}

// Softmax / LogSoftmax over N features, ponni_Softmax.h:45-56, ponni_LogSoftmax.h:45-57.
template <int N, int T, bool LOG>
__device__ inline void softmax(S<T>& s, Lane const& L) {
#pragma unroll
  for (int n = 0; n < kNT; n++) {
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) mx = fmaxf(mx, s.v[m][n][e]);
    mx = xmax(mx);
    float sum = 0.0f;
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float const ex = expf(s.v[m][n][e] - mx);
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) sum += ex;
        if (!LOG) s.v[m][n][e] = ex;
      }
    sum = xsum(sum);
    if (LOG) {
      float const lse = logf(sum) + mx;
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) s.v[m][n][e] -= lse;
    } else {
#pragma unroll
      for (int m = 0; m < T; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) s.v[m][n][e] = s.v[m][n][e] / sum;
    }
  }
}

// MinMaxNorm over N features, ponni_MinMaxNorm.h:67-84.
template <int N, int T>
__device__ inline void min_max(S<T>& s, float out_min, float out_max, float eps, Lane const& L) {
#pragma unroll
  for (int n = 0; n < kNT; n++) {
    float lo = __builtin_huge_valf(), hi = -__builtin_huge_valf();
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (N % 16 == 0 || 16 * m + 4 * L.g + e < N) {
          lo = fminf(lo, s.v[m][n][e]);
          hi = fmaxf(hi, s.v[m][n][e]);
        }
    lo = xmin(lo);
    hi = xmax(hi);
    float const scale = (out_max - out_min) / ((hi - lo) + eps);
#pragma unroll
    for (int m = 0; m < T; m++)
#pragma unroll
      for (int e = 0; e < 4; e++) s.v[m][n][e] = out_min + (s.v[m][n][e] - lo) * scale;
  }
}

// [a; b] for tile-aligned operands.
template <int TA, int TB>
__device__ inline S<TA + TB> concat(S<TA> const& a, S<TB> const& b) {
  S<TA + TB> s;
#pragma unroll
  for (int m = 0; m < TA; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) s.v[m][n] = a.v[m][n];
#pragma unroll
  for (int m = 0; m < TB; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) s.v[TA + m][n] = b.v[m][n];
  return s;
}

// Resize a tile to T2 tiles (extra tiles are zero).
template <int T2, int T>
__device__ inline S<T2> widen(S<T> const& s) {
  S<T2> o = zeros<T2>();
#pragma unroll
  for (int m = 0; m < (T < T2 ? T : T2); m++)
#pragma unroll
    for (int n = 0; n < kNT; n++) o.v[m][n] = s.v[m][n];
  return o;
}

// Stage `count` floats (a multiple of 4) of packed parameters into LDS.
__device__ inline void stage(floatx4* __restrict__ lds, float const* __restrict__ src, int count) {
  floatx4 const* s4 = reinterpret_cast<floatx4 const*>(src);
  for (int i = threadIdx.x; i < count / 4; i += blockDim.x) lds[i] = s4[i];
  __syncthreads();
}

}  // namespace fused
}  // namespace ponni_hip
