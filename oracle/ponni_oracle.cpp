// TEST INFRASTRUCTURE ONLY -- never linked into or called by the product.
//
// CPU oracle and CPU baseline: a plain C++ restatement of the reference's
// batched forward pass, run with OpenMP over samples the way Kokkos'
// OpenMP RangePolicy runs it.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load this library, and only as the checker.
//
// What it restates (reference paths relative to the reference root):
//   traversal / buffers   src/ponni_Inference.h:453-555 (per-sample compile-time
//                         executor: dense blocks with pointwise epilogues,
//                         barriers materialized in tmp1 / tmp2 / saved slots,
//                         each a [features, batch] LayoutRight array)
//   dense                 src/layers/ponni_Matvec.h:70-79 (v = 0; ascending k)
//   fused epilogue        src/ponni_Inference.h:412-444, src/ponni_LayerTraits.h:51-61
//   layers                src/layers/*.h compute_all_outputs / apply (cited below)
//   fp16 chain            template half model: every operation rounds to half
//                         (ponni_create_model.h:86-92, Kokkos half_t)
//   generated-graph ops   the emitted per-sample code of kokkos_nn/emitter.py:
//                         Dense :693-734 (sum = bias first), unary :218-258,
//                         binary :261-275 with scalar broadcast :735-741,
//                         reductions :475-547; a graph reaches the oracle as
//                         the same linearized chain the product receives
//
// Modes: 0 fp32, 1 fp64, 2 fp16 operands with fp32 arithmetic (state rounded
// to fp16 at every materialization), 3 the same for bf16, 4 fp16 chain of the
// template half model (half_t: v += W * x rounds the product and the sum),
// 5 fp16 chain of the generated half2 model (each dot-product step one
// rounded fma, ponni_TwoHalf.h:97-105; activations in fp32 of the half value,
// rounded, :138-153), 6 / 7 as 2 / 3 with every dense dot product summed in
// 32-feature blocks (each block's products summed exactly, then added to the
// fp32 running sum with one rounding: the k-blocking of a 32-deep matrix
// instruction).  Modes 6 and 7 are not a restatement of the reference: they
// are a second legitimate fp32 order, which tests use to measure how far a
// chain's result moves under a change of summation order.
//
// Pinning: tests/test_oracle.py checks every function here against the
// reference's known-answer tests (unit/core/*.cpp, unit/performance_benchmark)
// and against brute-force float64 numpy evaluations of random chains.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../include/ponni_hip.h"

namespace {

// ---- binary16 / bfloat16 rounding (IEEE round-to-nearest-even) -------------
// One rounding of a double to binary16 (the result is exact in float).
float round_half_d(double v) {
  if (std::isnan(v) || std::isinf(v)) return static_cast<float>(v);
  double const a = std::fabs(v);
  if (a >= 65520.0) return std::copysign(INFINITY, static_cast<float>(v));  // rounds past max half (65504)
  double q;
  if (a < std::ldexp(1.0, -14)) {
    q = std::ldexp(1.0, -24);  // subnormal range: quantum 2^-24
  } else {
    int e = 0;
    std::frexp(a, &e);        // a = m * 2^e, m in [0.5, 1)
    q = std::ldexp(1.0, e - 11);  // 10 explicit mantissa bits
  }
  return static_cast<float>(std::copysign(std::nearbyint(a / q) * q, v));
}

float round_half(float v) { return round_half_d(v); }

float round_bf16(float v) {
  if (std::isnan(v) || std::isinf(v)) return v;
  uint32_t x;
  std::memcpy(&x, &v, 4);
  uint32_t const lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  x &= 0xffff0000u;
  float out;
  std::memcpy(&out, &x, 4);
  return out;
}

// ---- arithmetic types -------------------------------------------------------
// H16: every operation on it rounds its exact (double) result to binary16
// once, as half_t arithmetic and the packed-half operations of
// ponni_TwoHalf.h:97-135 (__hadd2 / __hmul2 / __hfma2) do.
struct H16 {
  float v = 0.0f;
  H16() = default;
  H16(double x) : v(round_half_d(x)) {}
  explicit operator double() const { return v; }
  explicit operator float() const { return v; }
};
inline H16 operator+(H16 a, H16 b) { return H16(double(a.v) + double(b.v)); }
inline H16 operator-(H16 a, H16 b) { return H16(double(a.v) - double(b.v)); }
inline H16 operator-(H16 a) { return H16(-double(a.v)); }
inline H16 operator*(H16 a, H16 b) { return H16(double(a.v) * double(b.v)); }
inline H16 operator/(H16 a, H16 b) { return H16(double(a.v) / double(b.v)); }
// TwoHalf::fma (ponni_TwoHalf.h:97-105, __hfma2 on the device): a * b + c
// rounded once (a * b of two halves is exact in double).
inline H16 fma_half(H16 a, H16 b, H16 c) { return H16(double(a.v) * double(b.v) + double(c.v)); }
inline H16& operator+=(H16& a, H16 b) { return a = a + b; }
inline H16& operator/=(H16& a, H16 b) { return a = a / b; }
inline bool operator>(H16 a, H16 b) { return a.v > b.v; }
inline bool operator<(H16 a, H16 b) { return a.v < b.v; }
inline bool operator>=(H16 a, H16 b) { return a.v >= b.v; }
inline bool operator<=(H16 a, H16 b) { return a.v <= b.v; }
inline bool operator==(H16 a, H16 b) { return a.v == b.v; }
inline bool operator!=(H16 a, H16 b) { return a.v != b.v; }
inline H16 o_exp(H16 x) { return H16(std::exp(x.v)); }
inline H16 o_log(H16 x) { return H16(std::log(x.v)); }
inline H16 o_tanh(H16 x) { return H16(std::tanh(x.v)); }
inline H16 o_erf(H16 x) { return H16(std::erf(x.v)); }
inline H16 o_sqrt(H16 x) { return H16(std::sqrt(x.v)); }
inline float o_exp(float x) { return std::exp(x); }
inline float o_log(float x) { return std::log(x); }
inline float o_tanh(float x) { return std::tanh(x); }
inline float o_erf(float x) { return std::erf(x); }
inline float o_sqrt(float x) { return std::sqrt(x); }
inline double o_exp(double x) { return std::exp(x); }
inline double o_log(double x) { return std::log(x); }
inline double o_tanh(double x) { return std::tanh(x); }
inline double o_erf(double x) { return std::erf(x); }
inline double o_sqrt(double x) { return std::sqrt(x); }
inline H16 o_abs(H16 x) { return H16(std::fabs(x.v)); }
inline H16 o_pow(H16 x, H16 y) { return H16(std::pow(x.v, y.v)); }
inline bool o_isinf(H16 x) { return std::isinf(x.v); }
inline float o_abs(float x) { return std::fabs(x); }
inline float o_pow(float x, float y) { return std::pow(x, y); }
inline bool o_isinf(float x) { return std::isinf(x); }
inline double o_abs(double x) { return std::fabs(x); }
inline double o_pow(double x, double y) { return std::pow(x, y); }
inline bool o_isinf(double x) { return std::isinf(x); }

// Unary math of generated graphs (emitter.py:218-258; interpreter.py:15-117)
// in the arithmetic of T: float overloads for fp32, double for fp64, and the
// fp32 value of a half rounded back to half (a half chain's activations,
// ponni_TwoHalf.h:138-153).  Round is ties-to-even (emitter.py:1659-1667).
double math_op(int op, double x) {
  switch (op) {
    case PONNI_UNARY_ACOS: return std::acos(x);
    case PONNI_UNARY_ACOSH: return std::acosh(x);
    case PONNI_UNARY_ASIN: return std::asin(x);
    case PONNI_UNARY_ASINH: return std::asinh(x);
    case PONNI_UNARY_ATAN: return std::atan(x);
    case PONNI_UNARY_ATANH: return std::atanh(x);
    case PONNI_UNARY_CEIL: return std::ceil(x);
    case PONNI_UNARY_COS: return std::cos(x);
    case PONNI_UNARY_COSH: return std::cosh(x);
    case PONNI_UNARY_FLOOR: return std::floor(x);
    case PONNI_UNARY_SIN: return std::sin(x);
    case PONNI_UNARY_SINH: return std::sinh(x);
    case PONNI_UNARY_TAN: return std::tan(x);
    default: return std::nearbyint(x);  // PONNI_UNARY_ROUND, default rounding mode: ties to even
  }
}
float math_op(int op, float x) {
  switch (op) {
    case PONNI_UNARY_ACOS: return std::acos(x);
    case PONNI_UNARY_ACOSH: return std::acosh(x);
    case PONNI_UNARY_ASIN: return std::asin(x);
    case PONNI_UNARY_ASINH: return std::asinh(x);
    case PONNI_UNARY_ATAN: return std::atan(x);
    case PONNI_UNARY_ATANH: return std::atanh(x);
    case PONNI_UNARY_CEIL: return std::ceil(x);
    case PONNI_UNARY_COS: return std::cos(x);
    case PONNI_UNARY_COSH: return std::cosh(x);
    case PONNI_UNARY_FLOOR: return std::floor(x);
    case PONNI_UNARY_SIN: return std::sin(x);
    case PONNI_UNARY_SINH: return std::sinh(x);
    case PONNI_UNARY_TAN: return std::tan(x);
    default: return std::nearbyint(x);
  }
}
H16 math_op(int op, H16 x) { return H16(math_op(op, x.v)); }
inline bool o_isnan(H16 x) { return std::isnan(x.v); }
inline bool o_isnan(float x) { return std::isnan(x); }
inline bool o_isnan(double x) { return std::isnan(x); }

// emitter.py:261-275; comparisons and logic (interpreter.py:132-162,
// emitter.py:397-424) give 1 / 0 and read any nonzero operand as true.
template <class T>
T binary_op(int op, T l, T r) {
  T const one = T(1), zero = T(0);
  switch (op) {
    case PONNI_BINARY_ADD: return l + r;
    case PONNI_BINARY_SUB: return l - r;
    case PONNI_BINARY_MUL: return l * r;
    case PONNI_BINARY_DIV: return l / r;
    case PONNI_BINARY_MIN: return l < r ? l : r;
    case PONNI_BINARY_MAX: return l > r ? l : r;
    case PONNI_BINARY_EQUAL: return l == r ? one : zero;
    case PONNI_BINARY_GREATER: return l > r ? one : zero;
    case PONNI_BINARY_GREATER_EQUAL: return l >= r ? one : zero;
    case PONNI_BINARY_LESS: return l < r ? one : zero;
    case PONNI_BINARY_LESS_EQUAL: return l <= r ? one : zero;
    case PONNI_BINARY_AND: return (l != zero && r != zero) ? one : zero;
    case PONNI_BINARY_OR: return (l != zero || r != zero) ? one : zero;
    case PONNI_BINARY_XOR: return ((l != zero) != (r != zero)) ? one : zero;
    case PONNI_BINARY_PRELU: return l >= zero ? l : l * r;  // interpreter.py:164-165
    default: return o_pow(l, r);
  }
}

// ---- pointwise layers (apply) ----------------------------------------------
template <class T>
T pointwise(ponni_layer_desc const& d, double const* p, T x, int f) {
  switch (d.kind) {
    case PONNI_LAYER_BIAS:  // ponni_Bias.h:66-68
      return x + T(p[f]);
    case PONNI_LAYER_RELU:  // ponni_Relu.h:49-51
      return x > T(0) ? x : T(0);
    case PONNI_LAYER_LEAKY_RELU:  // ponni_LeakyRelu.h:53-55
      return x > T(0) ? x : T(d.attr[0]) * x;
    case PONNI_LAYER_ELU:  // ponni_Elu.h:48-50
      return x > T(0) ? x : T(d.attr[0]) * (o_exp(x) - T(1));
    case PONNI_LAYER_SELU: {  // ponni_Selu.h:45-49
      T const alpha = T(1.6732632423543772848);
      T const scale = T(1.0507009873554804934);
      return x > T(0) ? scale * x : scale * alpha * (o_exp(x) - T(1));
    }
    case PONNI_LAYER_GELU:
      if (d.flags & PONNI_FLAG_GELU_APPROXIMATE) {  // ponni_Gelu.h:48-53
        T const x3 = x * x * x;
        return T(0.5) * x * (T(1) + o_tanh(T(0.79788456080286535588) * (x + T(0.044715) * x3)));
      }
      return T(0.5) * x * (T(1) + o_erf(x / T(1.4142135623730950488)));  // ponni_Gelu.h:55-56
    case PONNI_LAYER_SILU:  // ponni_Silu.h:45-49
      if (x >= T(0)) return x / (T(1) + o_exp(-x));
      return x * o_exp(x) / (T(1) + o_exp(x));
    case PONNI_LAYER_SIGMOID:  // ponni_Sigmoid.h:45-49
      if (x >= T(0)) return T(1) / (T(1) + o_exp(-x));
      return o_exp(x) / (T(1) + o_exp(x));
    case PONNI_LAYER_TANH:  // ponni_Tanh.h:44
      return o_tanh(x);
    case PONNI_LAYER_SOFTPLUS: {  // ponni_Softplus.h:44-50
      T const beta = T(d.attr[0]);
      T const s = beta * x;
      if (s > T(0)) return (s + o_log(T(1) + o_exp(-s))) / beta;
      return o_log(T(1) + o_exp(s)) / beta;
    }
    case PONNI_LAYER_HARD_SIGMOID: {  // ponni_HardSigmoid.h:52-56
      T v = T(d.attr[0]) * x + T(d.attr[1]);
      v = v < T(0) ? T(0) : v;
      return v > T(1) ? T(1) : v;
    }
    case PONNI_LAYER_HARD_SWISH: {  // ponni_HardSwish.h:42-47
      T r = x + T(3);
      r = r < T(0) ? T(0) : r;
      r = r > T(6) ? T(6) : r;
      return x * r / T(6);
    }
    case PONNI_LAYER_MISH: {  // ponni_Mish.h:44-52
      T sp = x > T(0) ? x + o_log(T(1) + o_exp(-x)) : o_log(T(1) + o_exp(x));
      return x * o_tanh(sp);
    }
    case PONNI_LAYER_UNARY: {  // emitter.py:218-258
      T const alpha = T(d.attr[1]);
      switch (static_cast<int>(d.attr[0])) {
        case PONNI_UNARY_ABS: return o_abs(x);
        case PONNI_UNARY_NEG: return -x;
        case PONNI_UNARY_EXP: return o_exp(x);
        case PONNI_UNARY_LOG: return o_log(x);
        case PONNI_UNARY_SQRT: return o_sqrt(x);
        case PONNI_UNARY_RECIPROCAL: return T(1) / x;
        case PONNI_UNARY_SOFTSIGN: return x / (T(1) + o_abs(x));
        case PONNI_UNARY_CELU: return x > T(0) ? x : alpha * (o_exp(x / alpha) - T(1));
        case PONNI_UNARY_THRESHOLDED_RELU: return x > alpha ? x : T(0);
        case PONNI_UNARY_SELU: return T(d.attr[2]) * (x > T(0) ? x : alpha * (o_exp(x) - T(1)));
        case PONNI_UNARY_ERF: return o_erf(x);
        case PONNI_UNARY_SIGN:  // emitter.py:1669-1674
          return o_isnan(x) ? x : x > T(0) ? T(1) : x < T(0) ? T(-1) : T(0);
        case PONNI_UNARY_IS_NAN: return o_isnan(x) ? T(1) : T(0);
        case PONNI_UNARY_IS_INF: {  // interpreter.py:171-177
          bool const neg = o_isinf(x) && x < T(0) && d.attr[1] != 0.0;
          bool const pos = o_isinf(x) && x > T(0) && d.attr[2] != 0.0;
          return neg || pos ? T(1) : T(0);
        }
        case PONNI_UNARY_NOT: return x == T(0) ? T(1) : T(0);
        case PONNI_UNARY_NONZERO: return x != T(0) ? T(1) : T(0);
        default: return math_op(static_cast<int>(d.attr[0]), x);
      }
    }
    case PONNI_LAYER_CONST_BINARY: {  // binary op with a constant operand
      int const op = static_cast<int>(d.attr[0]);
      return (d.flags & PONNI_FLAG_CONST_LEFT) ? binary_op<T>(op, T(p[f]), x) : binary_op<T>(op, x, T(p[f]));
    }
    default:
      return x;
  }
}

bool is_pointwise(int k) {
  return k == PONNI_LAYER_BIAS || (k >= PONNI_LAYER_RELU && k <= PONNI_LAYER_MISH) || k == PONNI_LAYER_UNARY ||
         k == PONNI_LAYER_CONST_BINARY;
}

bool is_dense(int k) { return k == PONNI_LAYER_MATVEC || k == PONNI_LAYER_DENSE; }

bool reads_slot(int k) {
  return k == PONNI_LAYER_BINOP_ADD || k == PONNI_LAYER_BINOP_CONCATENATE || k == PONNI_LAYER_BINOP_PROJECTION_ADD ||
         k == PONNI_LAYER_LOAD_STATE || k == PONNI_LAYER_BINARY || k == PONNI_LAYER_SELECT;
}

// Constant operands of a Select layer (the operands whose 2-bit source field
// in flags is PONNI_SELECT_CONST).
int select_constants(ponni_layer_desc const& d) {
  int n = 0;
  for (int k = 0; k < 3; k++) n += ((d.flags >> (2 * k)) & 3) == PONNI_SELECT_CONST;
  return n;
}

// ---- buffers ------------------------------------------------------------------
// A [features, batch] LayoutRight array of T with row stride ld.  `store`
// applies the storage rounding of the mode (fp16 / bf16 operands).
template <class T>
struct Buf {
  T* p = nullptr;
  int64_t ld = 0;
  T& operator()(int f, int64_t b) const { return p[int64_t(f) * ld + b]; }
};

template <class T>
struct Ctx {
  std::vector<ponni_layer_desc> layers;
  std::vector<double const*> params;
  int mode = 0;
  T store(T v) const {
    if constexpr (std::is_same_v<T, float>) {
      if (mode == 2 || mode == 6) return round_half(v);
      if (mode == 3 || mode == 7) return round_bf16(v);
    }
    return v;
  }
};

// Barrier layer compute_all_outputs(in[, saved], out) for one sample.
template <class T>
void barrier(Ctx<T> const& c, int i, Buf<T> in, Buf<T> saved, Buf<T> out, int64_t b, Buf<T> const* slots) {
  ponni_layer_desc const& d = c.layers[i];
  double const* p = c.params[i];
  int const n = d.n_in;
  switch (d.kind) {
    case PONNI_LAYER_LAYER_NORM: {  // ponni_LayerNorm.h:76-99
      T mean = T(0);
      for (int f = 0; f < n; f++) mean += in(f, b);
      mean /= T(n);
      T var = T(0);
      for (int f = 0; f < n; f++) {
        T const dlt = in(f, b) - mean;
        var += dlt * dlt;
      }
      var /= T(n);
      T const inv_std = T(1) / o_sqrt(var + T(d.attr[0]));
      for (int f = 0; f < n; f++) {
        T const xhat = (in(f, b) - mean) * inv_std;
        out(f, b) = c.store(T(p[f]) * xhat + T(p[n + f]));
      }
      return;
    }
    case PONNI_LAYER_SOFTMAX: {  // ponni_Softmax.h:45-56
      T mx = in(0, b);
      for (int f = 1; f < n; f++) mx = in(f, b) > mx ? in(f, b) : mx;
      T sum = T(0);
      for (int f = 0; f < n; f++) sum += o_exp(in(f, b) - mx);
      for (int f = 0; f < n; f++) out(f, b) = c.store(o_exp(in(f, b) - mx) / sum);
      return;
    }
    case PONNI_LAYER_LOG_SOFTMAX: {  // ponni_LogSoftmax.h:45-57
      T mx = in(0, b);
      for (int f = 1; f < n; f++) mx = in(f, b) > mx ? in(f, b) : mx;
      T sum = T(0);
      for (int f = 0; f < n; f++) sum += o_exp(in(f, b) - mx);
      T const lse = o_log(sum) + mx;
      for (int f = 0; f < n; f++) out(f, b) = c.store(in(f, b) - lse);
      return;
    }
    case PONNI_LAYER_MIN_MAX_NORM: {  // ponni_MinMaxNorm.h:67-84
      T lo = in(0, b), hi = in(0, b);
      for (int f = 1; f < n; f++) {
        if (in(f, b) < lo) lo = in(f, b);
        if (in(f, b) > hi) hi = in(f, b);
      }
      T const scale = (T(d.attr[1]) - T(d.attr[0])) / ((hi - lo) + T(d.attr[2]));
      for (int f = 0; f < n; f++) out(f, b) = c.store(T(d.attr[0]) + (in(f, b) - lo) * scale);
      return;
    }
    case PONNI_LAYER_SAVE_STATE:  // ponni_Save_State.h:57-67
      for (int f = 0; f < d.n_out; f++) out(f, b) = in(f, b);
      return;
    case PONNI_LAYER_BINOP_ADD:  // ponni_Binop_Add.h:57-68
      for (int f = 0; f < d.n_out; f++) out(f, b) = c.store(in(f, b) + saved(f, b));
      return;
    case PONNI_LAYER_BINOP_CONCATENATE: {  // ponni_Binop_Concatenate.h:63-86
      // Read the current rows before writing: the reference writes in place
      // and, for after == false, would overwrite rows it still has to read.
      std::vector<T> cur(n);
      for (int f = 0; f < n; f++) cur[f] = in(f, b);
      int const n_out = d.n_out;
      if (d.flags & PONNI_FLAG_CONCAT_AFTER) {
        for (int f = 0; f < n_out; f++) out(f, b) = f < n ? cur[f] : saved(f - n, b);
      } else {
        int const n2 = n_out - n;
        for (int f = 0; f < n_out; f++) out(f, b) = f < n2 ? saved(f, b) : cur[f - n2];
      }
      return;
    }
    case PONNI_LAYER_BINOP_PROJECTION_ADD: {  // ponni_Binop_Projection_Add.h:81-95
      int const nsave = d.n_aux;
      for (int i2 = 0; i2 < n; i2++) {
        T proj = T(p[int64_t(nsave) * n + i2]);
        for (int k = 0; k < nsave; k++) proj += T(p[int64_t(k) * n + i2]) * saved(k, b);
        out(i2, b) = c.store(in(i2, b) + proj);
      }
      return;
    }
    case PONNI_LAYER_LOAD_STATE:  // the state becomes saved[slot]
      for (int f = 0; f < d.n_out; f++) out(f, b) = saved(f, b);
      return;
    case PONNI_LAYER_BINARY: {  // emitter.py:735-741, operands of 1 or n_out features
      int const op = static_cast<int>(d.attr[0]);
      bool const saved_left = d.flags & PONNI_FLAG_SAVED_LEFT;
      std::vector<T> cur(n), sv(d.n_aux);
      for (int f = 0; f < n; f++) cur[f] = in(f, b);
      for (int f = 0; f < d.n_aux; f++) sv[f] = saved(f, b);
      for (int f = 0; f < d.n_out; f++) {
        T const a = cur[n == 1 ? 0 : f];
        T const s2 = sv[d.n_aux == 1 ? 0 : f];
        out(f, b) = c.store(saved_left ? binary_op<T>(op, s2, a) : binary_op<T>(op, a, s2));
      }
      return;
    }
    case PONNI_LAYER_SELECT: {  // interpreter.py:178-183 Where / CompareSelect
      // Operand k (cond, a, b) is the state, a saved slot (the first saved
      // operand reads d.slot, the second attr[1]) or a constant vector (the
      // constants' values follow one another in p); a one-feature operand
      // broadcasts.  All are read before the first write.
      std::vector<T> v[3];
      int slots_used = 0, consts_used = 0;
      for (int k = 0; k < 3; k++) {
        int const src = (d.flags >> (2 * k)) & 3;
        if (src == PONNI_SELECT_STATE) {
          for (int f = 0; f < d.n_in; f++) v[k].push_back(in(f, b));
        } else if (src == PONNI_SELECT_SLOT) {
          int const s = slots_used++ == 0 ? d.slot : static_cast<int>(d.attr[1]);
          int const width = (d.flags & (PONNI_SELECT_COND_SCALAR << k)) ? 1 : d.n_out;
          for (int f = 0; f < width; f++) v[k].push_back(slots[s](f, b));
        } else {
          double const* cv = p + int64_t(consts_used++) * d.n_out;
          for (int f = 0; f < d.n_out; f++) v[k].push_back(T(cv[f]));
        }
      }
      for (int f = 0; f < d.n_out; f++) {
        T const cond = v[0][v[0].size() == 1 ? 0 : f];
        T const a = v[1][v[1].size() == 1 ? 0 : f];
        T const bb = v[2][v[2].size() == 1 ? 0 : f];
        out(f, b) = c.store(cond != T(0) ? a : bb);
      }
      return;
    }
    case PONNI_LAYER_REDUCE: {  // emitter.py:475-547
      int const op = static_cast<int>(d.attr[0]);
      T r;
      if (op == PONNI_REDUCE_MAX || op == PONNI_REDUCE_MIN || op == PONNI_REDUCE_LOG_SUM_EXP) {
        // The float path keeps the running value unless the next one compares
        // past it (emitter.py:506-511); the half2 path (16-bit modes) keeps it
        // only if it compares past the next one, TwoHalf::maximum(reduction,
        // value) (emitter.py:578-592, ponni_TwoHalf.h:243-251).  They differ
        // only for NaN: the float order keeps a NaN in feature 0 and passes
        // over later ones, the half2 order hands every NaN on to the next
        // feature.
        bool const h2 = c.mode == 2 || c.mode == 3 || c.mode == 6 || c.mode == 7;
        bool const mn = op == PONNI_REDUCE_MIN;
        r = in(0, b);
        for (int f = 1; f < n; f++) {
          T const v = in(f, b);
          if (h2) r = mn ? (r < v ? r : v) : (r > v ? r : v);
          else r = mn ? (v < r ? v : r) : (v > r ? v : r);
        }
        if (op == PONNI_REDUCE_LOG_SUM_EXP) {
          T sum = T(0);
          for (int f = 0; f < n; f++) sum += o_exp(in(f, b) - r);
          r = o_isinf(r) ? r : r + o_log(sum);
        }
      } else {
        r = op == PONNI_REDUCE_PROD ? T(1) : T(0);
        for (int f = 0; f < n; f++) {
          T const v = in(f, b);
          if (op == PONNI_REDUCE_L1) r += o_abs(v);
          else if (op == PONNI_REDUCE_L2 || op == PONNI_REDUCE_SUM_SQUARE) r += v * v;
          else if (op == PONNI_REDUCE_PROD) r = r * v;
          else r += v;
        }
        if (op == PONNI_REDUCE_MEAN) r /= T(n);
        else if (op == PONNI_REDUCE_L2) r = o_sqrt(r);
        else if (op == PONNI_REDUCE_LOG_SUM) r = o_log(r);
      }
      out(0, b) = c.store(r);
      return;
    }
    default:  // a lone pointwise layer
      for (int f = 0; f < n; f++) out(f, b) = c.store(pointwise<T>(d, p, in(f, b), f));
      return;
  }
}

// One step of a dense dot product, v + w * x.  Mode 5 (the generated half2
// chain, emitter.py:978-999: sum = TwoHalf::fma(w_splat, x, sum)) rounds it
// once; every other mode evaluates the reference's `v += W * x`
// (ponni_Matvec.h:74-78) in its arithmetic type (two roundings in mode 4,
// half_t).
template <class T>
T dense_step(Ctx<T> const& c, T v, T w, T x) {
  if constexpr (std::is_same_v<T, H16>) {
    if (c.mode == 5) return fma_half(w, x, v);
  }
  return v + w * x;
}

// traverse_mixed_batch_parallel (ponni_Inference.h:453-555) for one sample.
template <class T>
void run_sample(Ctx<T> const& c, Buf<T> x, Buf<T> y, Buf<T> tmp1, Buf<T> tmp2, Buf<T> const* saved, int64_t b) {
  int const L = static_cast<int>(c.layers.size());
  bool in_tmp1 = false;
  int i = 0;
  while (i < L) {
    ponni_layer_desc const& d = c.layers[i];
    if (is_dense(d.kind)) {
      int end = i + 1;
      while (end < L && is_pointwise(c.layers[end].kind)) end++;
      Buf<T> in = i == 0 ? x : (in_tmp1 ? tmp1 : tmp2);
      Buf<T> out;
      if (end == L) {
        out = y;
      } else {
        bool const out_tmp1 = i == 0 ? true : !in_tmp1;
        out = out_tmp1 ? tmp1 : tmp2;
        in_tmp1 = out_tmp1;
      }
      double const* w = c.params[i];
      bool const generated = d.kind == PONNI_LAYER_DENSE;
      bool const bias = generated && (d.flags & PONNI_FLAG_DENSE_BIAS);
      for (int f = 0; f < d.n_out; f++) {  // compute_fused_dense_block, ponni_Inference.h:431-444
        T v = T(0);
        if (generated && bias) v = T(w[int64_t(d.n_out) * d.n_in + f]);  // emitter.py:701-710: sum = bias
        auto weight = [&](int k) {  // W[f][k] of a generated Dense, W(k, f) of a Matvec
          return T(generated ? w[int64_t(f) * d.n_in + k] : w[int64_t(k) * d.n_out + f]);
        };
        if (c.mode == 6 || c.mode == 7) {
          for (int k0 = 0; k0 < d.n_in; k0 += 32) {
            double blk = 0.0;
            for (int k = k0; k < std::min(k0 + 32, d.n_in); k++) blk += double(weight(k)) * double(in(k, b));
            v = T(double(v) + blk);
          }
        } else {
          for (int k = 0; k < d.n_in; k++) v = dense_step(c, v, weight(k), in(k, b));
        }
        for (int e = i + 1; e < end; e++) v = pointwise<T>(c.layers[e], c.params[e], v, f);
        out(f, b) = c.store(v);
      }
      i = end;
      continue;
    }
    Buf<T> const sv = reads_slot(d.kind) ? saved[d.slot] : Buf<T>{};
    if (i == 0 && L == 1) {
      barrier(c, i, x, sv, y, b, saved);
    } else if (i == 0) {
      if (d.kind == PONNI_LAYER_SAVE_STATE) barrier(c, i, x, sv, saved[d.slot], b, saved);
      barrier(c, i, x, sv, tmp1, b, saved);
      in_tmp1 = true;
    } else if (i < L - 1) {
      Buf<T> const in = in_tmp1 ? tmp1 : tmp2;
      Buf<T> const out = d.kind == PONNI_LAYER_SAVE_STATE ? saved[d.slot] : in;
      barrier(c, i, in, sv, out, b, saved);
    } else {
      barrier(c, i, in_tmp1 ? tmp1 : tmp2, sv, y, b, saved);
    }
    i++;
  }
}

// Scratch widths, get_planned_temporary_size<0/1>() and get_saved_state_size<s>().
// saved gets one entry per slot up to the highest Save_State index.
void plan_widths(std::vector<ponni_layer_desc> const& layers, int* tmp, std::vector<int>& saved) {
  int const L = static_cast<int>(layers.size());
  tmp[0] = tmp[1] = 0;
  saved.clear();
  bool in_tmp1 = false;
  int i = 0;
  while (i < L) {
    ponni_layer_desc const& d = layers[i];
    if (d.kind == PONNI_LAYER_SAVE_STATE && d.slot >= 0) {
      if (static_cast<int>(saved.size()) <= d.slot) saved.resize(d.slot + 1, 0);
      saved[d.slot] = std::max(saved[d.slot], d.n_out);
    }
    if (is_dense(d.kind)) {
      int end = i + 1;
      while (end < L && is_pointwise(layers[end].kind)) end++;
      if (end != L) {
        bool const out_tmp1 = i == 0 ? true : !in_tmp1;
        tmp[out_tmp1 ? 0 : 1] = std::max(tmp[out_tmp1 ? 0 : 1], d.n_out);
        in_tmp1 = out_tmp1;
      }
      i = end;
      continue;
    }
    if (i != L - 1) {
      bool const out_tmp1 = i == 0 ? true : in_tmp1;
      tmp[out_tmp1 ? 0 : 1] = std::max(tmp[out_tmp1 ? 0 : 1], d.n_out);
      in_tmp1 = out_tmp1;
    }
    i++;
  }
}

template <class T, class IO>
int forward(std::vector<ponni_layer_desc> const& layers, std::vector<double const*> const& params, int mode,
            IO const* x_io, int64_t ld_x, IO* y_io, int64_t ld_y, int64_t batch, int threads) {
  Ctx<T> c;
  c.layers = layers;
  c.params = params;
  c.mode = mode;
  int tmpw[2];
  std::vector<int> savedw;
  plan_widths(layers, tmpw, savedw);
  int const num_slots = std::max<int>(static_cast<int>(savedw.size()), 1);
  savedw.resize(num_slots, 0);
  int const n_in = layers.front().n_in;
  int const n_out = layers.back().n_out;
  // Inputs and outputs are converted to T at the boundary; scratch is T.
  std::vector<T> xs(size_t(n_in) * size_t(batch)), ys(size_t(n_out) * size_t(batch));
  std::vector<T> t1(size_t(tmpw[0]) * size_t(batch)), t2(size_t(tmpw[1]) * size_t(batch));
  std::vector<std::vector<T>> sv(num_slots);
  std::vector<Buf<T>> saved_v(num_slots);
  Buf<T>* saved = saved_v.data();
  for (int s = 0; s < num_slots; s++) {
    sv[s].resize(size_t(savedw[s]) * size_t(batch));
    saved[s] = Buf<T>{sv[s].data(), batch};
  }
  Buf<T> const x{xs.data(), batch}, y{ys.data(), batch}, tmp1{t1.data(), batch}, tmp2{t2.data(), batch};
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < batch; b++)
    for (int f = 0; f < n_in; f++) x(f, b) = c.store(T(x_io[int64_t(f) * ld_x + b]));
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < batch; b++) run_sample<T>(c, x, y, tmp1, tmp2, saved, b);
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < batch; b++)
    for (int f = 0; f < n_out; f++) y_io[int64_t(f) * ld_y + b] = static_cast<IO>(static_cast<double>(y(f, b)));
  return 0;
}

}  // namespace

extern "C" {

// Per-layer parameters are concatenated in layer order, each in the layer's
// own layout (Matvec W [n_in, n_out]; LayerNorm gamma, beta; Projection_Add
// W [NSAVE, n_in], bias; Dense W [n_out, n_in], bias; Const_Binary c [n_in];
// Select: its constant operands, n_out values each).  x / y are float for modes 0, 2, 3, 4, 5
// and double for mode 1.  Returns 0 on success.
int oracle_forward(ponni_layer_desc const* layers, int32_t num_layers, double const* params, int32_t mode,
                   void const* x, int64_t ld_x, void* y, int64_t ld_y, int64_t batch, int32_t threads) {
  if (!layers || num_layers <= 0 || batch <= 0) return 1;
  std::vector<ponni_layer_desc> ls(layers, layers + num_layers);
  std::vector<double const*> ps(num_layers);
  int64_t off = 0;
  for (int i = 0; i < num_layers; i++) {
    ps[i] = params + off;
    auto const& d = ls[i];
    switch (d.kind) {
      case PONNI_LAYER_MATVEC: off += int64_t(d.n_in) * d.n_out; break;
      case PONNI_LAYER_BIAS: off += d.n_in; break;
      case PONNI_LAYER_LAYER_NORM: off += 2 * int64_t(d.n_in); break;
      case PONNI_LAYER_BINOP_PROJECTION_ADD: off += int64_t(d.n_aux) * d.n_in + d.n_in; break;
      case PONNI_LAYER_DENSE:
        off += int64_t(d.n_out) * d.n_in + ((d.flags & PONNI_FLAG_DENSE_BIAS) ? d.n_out : 0);
        break;
      case PONNI_LAYER_CONST_BINARY: off += d.n_in; break;
      case PONNI_LAYER_SELECT: off += int64_t(select_constants(d)) * d.n_out; break;
      default: break;
    }
  }
  // fp16 / bf16 operand modes see every parameter at the operand precision.
  std::vector<double> rounded;
  if (mode == 2 || mode == 3 || mode == 6 || mode == 7) {
    rounded.assign(params, params + off);
    for (double& v : rounded) v = (mode == 2 || mode == 6) ? round_half(float(v)) : round_bf16(float(v));
    for (int i = 0; i < num_layers; i++) ps[i] = rounded.data() + (ps[i] - params);
  }
  switch (mode) {
    case 0:
    case 2:
    case 3:
    case 6:
    case 7:
      return forward<float, float>(ls, ps, mode, static_cast<float const*>(x), ld_x, static_cast<float*>(y), ld_y,
                                   batch, threads);
    case 1:
      return forward<double, double>(ls, ps, mode, static_cast<double const*>(x), ld_x, static_cast<double*>(y),
                                     ld_y, batch, threads);
    case 4:
    case 5:
      return forward<H16, float>(ls, ps, mode, static_cast<float const*>(x), ld_x, static_cast<float*>(y), ld_y,
                                 batch, threads);
    default:
      return 2;
  }
}

// Scratch planning of the reference: tmp1, tmp2, saved slot widths (the
// first max_saved slots); returns get_num_saved_states().
int32_t oracle_plan_widths(ponni_layer_desc const* layers, int32_t num_layers, int32_t* tmp, int32_t* saved,
                           int32_t max_saved) {
  std::vector<ponni_layer_desc> ls(layers, layers + num_layers);
  int t[2];
  std::vector<int> s;
  plan_widths(ls, t, s);
  tmp[0] = t[0];
  tmp[1] = t[1];
  for (int i = 0; i < max_saved; i++) saved[i] = i < static_cast<int>(s.size()) ? s[i] : 0;
  return static_cast<int32_t>(s.size());
}

float oracle_round_half(float v) { return round_half(v); }
float oracle_fma_half(float a, float b, float c) { return fma_half(H16(a), H16(b), H16(c)).v; }
float oracle_add_half(float a, float b) { return (H16(a) + H16(b)).v; }
float oracle_round_bf16(float v) { return round_bf16(v); }

}  // extern "C"
