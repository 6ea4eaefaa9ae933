// NARROW path, generated form: building blocks for per-plan kernels of
// narrow chains (every width <= 16), compiled at run time by hipRTC with all
// widths and parameter offsets constant (see fused.cpp, narrow_source).
//
// One lane owns V consecutive samples; the state is C s[W][V] (W the plan's
// padded width class, C the compute type: float, or double for F64 plans),
// rows >= the current width held at exactly 0.  Inputs and outputs move as
// V-element vectors (16 B per row) when the views allow it, so each feature
// row is streamed with full-width coalesced accesses.  Parameters are in the
// NARROW packing (plan.cpp pack_params): dense weights W x W, [k * W + j] =
// W(k, j) of the reference's [in, out] Matvec layout, vectors padded to W;
// uniform addresses, so the compiler reads them with scalar loads.  The
// arithmetic mirrors the reference's per-sample executor
// (ponni_Inference.h:412-555) and the interpreted NARROW kernel
// (kernels_narrow.hip) operation for operation; graph operations follow the
// generator's emitted code (kokkos_nn/emitter.py, lines on each function).
#pragma once

#include "pointwise.h"

namespace ponni_hip {
namespace narrowj {

template <class S, int V>
struct VecOf {
  typedef S type __attribute__((ext_vector_type(V)));
};

template <class A, class B>
struct same_type {
  static constexpr bool value = false;
};
template <class A>
struct same_type<A, A> {
  static constexpr bool value = true;
};

// Rounding of a materialized state to the storage precision S.
template <class S, class C>
__device__ inline C round_state(C v) {
  if constexpr (same_type<S, C>::value) return v;
  else return static_cast<C>(static_cast<S>(v));
}

// Can rows of this view be moved as aligned V-element vectors?
template <class S, int V>
__device__ inline bool vec_ok(void const* p, int64_t ld) {
  return (reinterpret_cast<unsigned long long>(p) % (sizeof(S) * V)) == 0 && ld % V == 0;
}

// s[f][v] = x(f, b0 + v) for f < N; rows >= N and samples >= batch are 0.
template <class S, int V, int N, int W, class C>
__device__ inline void load(C (&s)[W][V], S const* __restrict__ x, int64_t ld, int64_t b0, int64_t batch, bool vec) {
  typedef typename VecOf<S, V>::type SV;
#pragma unroll
  for (int f = 0; f < W; f++)
#pragma unroll
    for (int v = 0; v < V; v++) s[f][v] = C(0);
  if (vec) {
#pragma unroll
    for (int f = 0; f < N; f++) {
      SV const r = *reinterpret_cast<SV const*>(x + int64_t(f) * ld + b0);
#pragma unroll
      for (int v = 0; v < V; v++) s[f][v] = static_cast<C>(r[v]);
    }
  } else {
#pragma unroll
    for (int f = 0; f < N; f++)
#pragma unroll
      for (int v = 0; v < V; v++)
        if (b0 + v < batch) s[f][v] = static_cast<C>(x[int64_t(f) * ld + b0 + v]);
  }
}

template <class S, int V, int N, int W, class C>
__device__ inline void store(C const (&s)[W][V], S* __restrict__ y, int64_t ld, int64_t b0, int64_t batch, bool vec) {
  typedef typename VecOf<S, V>::type SV;
  if (vec) {
#pragma unroll
    for (int f = 0; f < N; f++) {
      SV r;
#pragma unroll
      for (int v = 0; v < V; v++) r[v] = static_cast<S>(s[f][v]);
      *reinterpret_cast<SV*>(y + int64_t(f) * ld + b0) = r;
    }
  } else {
#pragma unroll
    for (int f = 0; f < N; f++)
#pragma unroll
      for (int v = 0; v < V; v++)
        if (b0 + v < batch) y[int64_t(f) * ld + b0 + v] = static_cast<S>(s[f][v]);
  }
}

// a[j] = sum_k W(k, j) s[k], ascending k (ponni_Matvec.h:70-79); rows >= N are 0.
template <int V, int K, int N, int W, class C>
__device__ inline void dense(C (&a)[W][V], C const (&s)[W][V], C const* __restrict__ w) {
#pragma unroll
  for (int j = 0; j < W; j++) {
#pragma unroll
    for (int v = 0; v < V; v++) a[j][v] = C(0);
    if (j < N) {
#pragma unroll
      for (int k = 0; k < K; k++) {
        C const wk = w[k * W + j];
#pragma unroll
        for (int v = 0; v < V; v++) a[j][v] += wk * s[k][v];
      }
    }
  }
}

// Generated Dense: a[j] = c[j] + sum_k W(k, j) s[k], the bias seeding the
// sum and k ascending (emitter.py:701-710); rows >= N are 0.
template <int V, int K, int N, int W, class C>
__device__ inline void dense_bias(C (&a)[W][V], C const (&s)[W][V], C const* __restrict__ w, C const* __restrict__ c) {
#pragma unroll
  for (int j = 0; j < W; j++) {
#pragma unroll
    for (int v = 0; v < V; v++) a[j][v] = C(0);
    if (j < N) {
      C const cj = c[j];
#pragma unroll
      for (int v = 0; v < V; v++) a[j][v] = cj;
#pragma unroll
      for (int k = 0; k < K; k++) {
        C const wk = w[k * W + j];
#pragma unroll
        for (int v = 0; v < V; v++) a[j][v] += wk * s[k][v];
      }
    }
  }
}

// a[j] += c[j] for j < N (ponni_Bias.h:66-68), or f(a[j], c[j]).
template <int V, int N, int W, class C, class F>
__device__ inline void with_vec(C (&a)[W][V], C const* __restrict__ c, F f) {
#pragma unroll
  for (int j = 0; j < N; j++) {
    C const cj = c[j];
#pragma unroll
    for (int v = 0; v < V; v++) a[j][v] = f(a[j][v], cj);
  }
}

template <int V, int N, int W, class C, class F>
__device__ inline void map(C (&a)[W][V], F f) {
#pragma unroll
  for (int j = 0; j < N; j++)
#pragma unroll
    for (int v = 0; v < V; v++) a[j][v] = f(a[j][v]);
}

// End of every operation: the state rounded to the storage precision with
// rows >= N at zero, as every materialization of the reference executor.
template <class S, int V, int N, int W, class C>
__device__ inline void finish(C (&s)[W][V], C const (&a)[W][V]) {
#pragma unroll
  for (int f = 0; f < W; f++)
#pragma unroll
    for (int v = 0; v < V; v++) s[f][v] = f < N ? round_state<S>(a[f][v]) : C(0);
}

template <int V, int W, class C>
__device__ inline void copy(C (&d)[W][V], C const (&s)[W][V]) {
#pragma unroll
  for (int f = 0; f < W; f++)
#pragma unroll
    for (int v = 0; v < V; v++) d[f][v] = s[f][v];
}

// Two-pass LayerNorm, ponni_LayerNorm.h:82-98.
template <int V, int N, int W, class C>
__device__ inline void layer_norm(C (&s)[W][V], C const* __restrict__ gamma, C const* __restrict__ beta, C eps) {
#pragma unroll
  for (int v = 0; v < V; v++) {
    C mean = C(0);
#pragma unroll
    for (int f = 0; f < N; f++) mean += s[f][v];
    mean /= C(N);
    C var = C(0);
#pragma unroll
    for (int f = 0; f < N; f++) {
      C const d = s[f][v] - mean;
      var += d * d;
    }
    var /= C(N);
    C const inv_std = C(1) / d_sqrt(var + eps);
#pragma unroll
    for (int f = 0; f < N; f++) s[f][v] = gamma[f] * ((s[f][v] - mean) * inv_std) + beta[f];
  }
}

// Softmax / LogSoftmax, ponni_Softmax.h:45-56, ponni_LogSoftmax.h:46-57.
template <int V, int N, int W, bool LOG, class C>
__device__ inline void softmax(C (&s)[W][V]) {
#pragma unroll
  for (int v = 0; v < V; v++) {
    C mx = s[0][v];
#pragma unroll
    for (int f = 1; f < N; f++) mx = s[f][v] > mx ? s[f][v] : mx;
    C sum = C(0);
#pragma unroll
    for (int f = 0; f < N; f++) sum += d_exp(s[f][v] - mx);
    if (!LOG) {
#pragma unroll
      for (int f = 0; f < N; f++) s[f][v] = d_exp(s[f][v] - mx) / sum;
    } else {
      C const lse = d_log(sum) + mx;
#pragma unroll
      for (int f = 0; f < N; f++) s[f][v] = s[f][v] - lse;
    }
  }
}

// MinMaxNorm, ponni_MinMaxNorm.h:68-84.
template <int V, int N, int W, class C>
__device__ inline void min_max(C (&s)[W][V], C out_min, C out_max, C eps) {
#pragma unroll
  for (int v = 0; v < V; v++) {
    C lo = s[0][v], hi = s[0][v];
#pragma unroll
    for (int f = 1; f < N; f++) {
      if (s[f][v] < lo) lo = s[f][v];
      if (s[f][v] > hi) hi = s[f][v];
    }
    C const scale = (out_max - out_min) / ((hi - lo) + eps);
#pragma unroll
    for (int f = 0; f < N; f++) s[f][v] = out_min + (s[f][v] - lo) * scale;
  }
}

// [lead; trail] with the leading operand's FIRST rows, ponni_Binop_Concatenate.h:63-86.
template <int V, int FIRST, int NOUT, int W, class C>
__device__ inline void concat(C (&s)[W][V], C const (&lead)[W][V], C const (&trail)[W][V]) {
  C o[W][V];
#pragma unroll
  for (int f = 0; f < W; f++)
#pragma unroll
    for (int v = 0; v < V; v++) o[f][v] = f < FIRST ? lead[f][v] : f < NOUT ? trail[f - FIRST][v] : C(0);
  copy<V, W>(s, o);
}

// s[i] += b[i] + sum_k W(k, i) saved[k] (bias first), ponni_Binop_Projection_Add.h:81-95.
template <int V, int NIN, int NSAVE, int W, class C>
__device__ inline void proj_add(C (&s)[W][V], C const (&sv)[W][V], C const* __restrict__ w, C const* __restrict__ b) {
#pragma unroll
  for (int i = 0; i < NIN; i++) {
    C proj[V];
#pragma unroll
    for (int v = 0; v < V; v++) proj[v] = b[i];
#pragma unroll
    for (int k = 0; k < NSAVE; k++) {
      C const wk = w[k * W + i];
#pragma unroll
      for (int v = 0; v < V; v++) proj[v] += wk * sv[k][v];
    }
#pragma unroll
    for (int v = 0; v < V; v++) s[i][v] = s[i][v] + proj[v];
  }
}

// Tensor-tensor operation of the state with saved state `sv` (emitter.py:735-741):
// operands of one feature broadcast (BinaryAux flags in AUX), the saved one
// on the left when BIN_SAVED_LEFT.
template <int V, int NOUT, int W, int AUX, class C>
__device__ inline void binary(C (&s)[W][V], C const (&sv)[W][V]) {
  constexpr int bop = AUX & 0xff;
#pragma unroll
  for (int v = 0; v < V; v++) {
    C const s0 = s[0][v], v0 = sv[0][v];
#pragma unroll
    for (int f = 0; f < NOUT; f++) {
      C const a = (AUX & BIN_STATE_SCALAR) ? s0 : s[f][v];
      C const c = (AUX & BIN_SAVED_SCALAR) ? v0 : sv[f][v];
      s[f][v] = (AUX & BIN_SAVED_LEFT) ? apply_binary<C>(bop, c, a) : apply_binary<C>(bop, a, c);
    }
  }
}

// state = cond != 0 ? a : b (interpreter.py:178-183 Where / CompareSelect).  AUX
// holds the operand sources of cond, a, b (2 bits each: 0 the state, 1 sv1,
// 2 sv2, 3 a constant vector, c1 for the first constant operand and c2 for
// a second) and the one-feature (broadcast) flags of program.h SelectAux.
template <int V, int NOUT, int W, int AUX, class C>
__device__ inline void select3(C (&s)[W][V], C const (&sv1)[W][V], C const (&sv2)[W][V], C const* __restrict__ c1,
                               C const* __restrict__ c2) {
  // The condition is never a constant, so b is the second constant exactly
  // when a is a constant too.
  auto operand = [&](int k, int f, int v) -> C {
    int const code = sel_src(AUX, k);
    bool const second_const = k == 2 && sel_src(AUX, 1) == 3;
    return code == 0 ? s[f][v] : code == 1 ? sv1[f][v] : code == 2 ? sv2[f][v] : second_const ? c2[f] : c1[f];
  };
#pragma unroll
  for (int v = 0; v < V; v++) {
    C const k0 = operand(0, 0, v), k1 = operand(1, 0, v), k2 = operand(2, 0, v);
#pragma unroll
    for (int f = 0; f < NOUT; f++) {
      C const c = (AUX & SEL_COND_SCALAR) ? k0 : operand(0, f, v);
      C const a = (AUX & SEL_A_SCALAR) ? k1 : operand(1, f, v);
      C const b = (AUX & SEL_B_SCALAR) ? k2 : operand(2, f, v);
      s[f][v] = apply_select<C>(c, a, b);
    }
  }
}

// Reduction over the N features into feature 0 (emitter.py:475-547); OP is
// a ponni_reduce_op value: 0 sum, 1 mean, 2 max, 3 min, 4 L1, 5 L2,
// 6 sum of squares, 7 log-sum, 8 log-sum-exp, 9 product.  H2 (16-bit plans)
// keeps the running maximum / minimum only if it compares past the next
// value, the generated half2 path's TwoHalf::maximum(reduction, value)
// (emitter.py:578-592); the float path replaces it when the next value
// compares past it.  The two differ only in where a NaN ends up.
template <int V, int N, int W, int OP, bool H2, class C>
__device__ inline void reduce(C (&s)[W][V]) {
#pragma unroll
  for (int v = 0; v < V; v++) {
    C r;
    if (OP == 2 || OP == 3 || OP == 8) {
      r = s[0][v];
#pragma unroll
      for (int f = 1; f < N; f++) {
        C const x = s[f][v];
        if (H2) r = OP == 3 ? (r < x ? r : x) : (r > x ? r : x);
        else r = OP == 3 ? (x < r ? x : r) : (x > r ? x : r);
      }
      if (OP == 8) {
        C sum = C(0);
#pragma unroll
        for (int f = 0; f < N; f++) sum += d_exp(s[f][v] - r);
        r = __builtin_isinf(r) ? r : r + d_log(sum);
      }
    } else {
      r = OP == 9 ? C(1) : C(0);
#pragma unroll
      for (int f = 0; f < N; f++) {
        C const x = s[f][v];
        if (OP == 4) r += d_abs(x);
        else if (OP == 5 || OP == 6) r += x * x;
        else if (OP == 9) r *= x;
        else r += x;
      }
      if (OP == 1) r /= C(N);
      else if (OP == 5) r = d_sqrt(r);
      else if (OP == 7) r = d_log(r);
    }
    s[0][v] = r;
  }
}

}  // namespace narrowj
}  // namespace ponni_hip
