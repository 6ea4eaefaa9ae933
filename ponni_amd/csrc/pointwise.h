// Pointwise layer math shared by every kernel family.  Each formula follows the
// reference layer's apply() (file:line on each function) term for term,
// including its branch structure, so results agree with the reference to
// rounding.
#pragma once
#define PONNI_POINTWISE_H 1

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

#include "program.h"

namespace ponni_hip {

__host__ __device__ inline float d_exp(float x) { return expf(x); }
__host__ __device__ inline double d_exp(double x) { return exp(x); }
__host__ __device__ inline float d_log(float x) { return logf(x); }
__host__ __device__ inline double d_log(double x) { return log(x); }
__host__ __device__ inline float d_tanh(float x) { return tanhf(x); }
__host__ __device__ inline double d_tanh(double x) { return tanh(x); }
__host__ __device__ inline float d_erf(float x) { return erff(x); }
__host__ __device__ inline double d_erf(double x) { return erf(x); }
__host__ __device__ inline float d_sqrt(float x) { return sqrtf(x); }
__host__ __device__ inline double d_sqrt(double x) { return sqrt(x); }
__host__ __device__ inline float d_pow(float x, float y) { return powf(x, y); }
__host__ __device__ inline double d_pow(double x, double y) { return pow(x, y); }
__host__ __device__ inline float d_abs(float x) { return fabsf(x); }
__host__ __device__ inline double d_abs(double x) { return fabs(x); }

// ponni_Relu.h:49-51
template <class T> __host__ __device__ inline T act_relu(T x) { return x > T(0) ? x : T(0); }
// ponni_LeakyRelu.h:53-55
template <class T> __host__ __device__ inline T act_leaky_relu(T x, T slope) { return x > T(0) ? x : slope * x; }
// ponni_Elu.h:48-50
template <class T> __host__ __device__ inline T act_elu(T x, T alpha) { return x > T(0) ? x : alpha * (d_exp(x) - T(1)); }
// ponni_Selu.h:45-49
template <class T> __host__ __device__ inline T act_selu(T x) {
  T const alpha = T(1.6732632423543772848);
  T const scale = T(1.0507009873554804934);
  return x > T(0) ? scale * x : scale * alpha * (d_exp(x) - T(1));
}
// ponni_Gelu.h:55-56
template <class T> __host__ __device__ inline T act_gelu_erf(T x) {
  return T(0.5) * x * (T(1) + d_erf(x / T(1.4142135623730950488)));
}
// ponni_Gelu.h:48-53
template <class T> __host__ __device__ inline T act_gelu_tanh(T x) {
  T const x3 = x * x * x;
  return T(0.5) * x * (T(1) + d_tanh(T(0.79788456080286535588) * (x + T(0.044715) * x3)));
}
// ponni_Silu.h:45-49
template <class T> __host__ __device__ inline T act_silu(T x) {
  if (x >= T(0)) return x / (T(1) + d_exp(-x));
  T const e = d_exp(x);
  return x * e / (T(1) + e);
}
// ponni_Sigmoid.h:45-49
template <class T> __host__ __device__ inline T act_sigmoid(T x) {
  if (x >= T(0)) return T(1) / (T(1) + d_exp(-x));
  T const e = d_exp(x);
  return e / (T(1) + e);
}
// ponni_Tanh.h:44
template <class T> __host__ __device__ inline T act_tanh(T x) { return d_tanh(x); }
// ponni_Softplus.h:44-50
template <class T> __host__ __device__ inline T act_softplus(T x, T beta) {
  T const s = beta * x;
  if (s > T(0)) return (s + d_log(T(1) + d_exp(-s))) / beta;
  return d_log(T(1) + d_exp(s)) / beta;
}
// ponni_HardSigmoid.h:52-56
template <class T> __host__ __device__ inline T act_hard_sigmoid(T x, T alpha, T beta) {
  T v = alpha * x + beta;
  v = v < T(0) ? T(0) : v;
  return v > T(1) ? T(1) : v;
}
// ponni_HardSwish.h:42-47
template <class T> __host__ __device__ inline T act_hard_swish(T x) {
  T r = x + T(3);
  r = r < T(0) ? T(0) : r;
  r = r > T(6) ? T(6) : r;
  return x * r / T(6);
}
// ponni_Mish.h:44-52
template <class T> __host__ __device__ inline T act_mish(T x) {
  T sp;
  if (x > T(0)) sp = x + d_log(T(1) + d_exp(-x));
  else sp = d_log(T(1) + d_exp(x));
  return x * d_tanh(sp);
}

// Unary operations of generated graphs, kokkos_nn/emitter.py:218-258.
template <class T> __host__ __device__ inline T act_softsign(T x) { return x / (T(1) + d_abs(x)); }
template <class T> __host__ __device__ inline T act_celu(T x, T alpha) {
  return x > T(0) ? x : alpha * (d_exp(x / alpha) - T(1));
}
template <class T> __host__ __device__ inline T act_thresholded_relu(T x, T alpha) { return x > alpha ? x : T(0); }
template <class T> __host__ __device__ inline T act_selu_ag(T x, T alpha, T gamma) {
  return gamma * (x > T(0) ? x : alpha * (d_exp(x) - T(1)));
}

// Unary math and predicates of generated graphs (interpreter.py:15-117,
// :171-181); a boolean is 1 / 0.
__host__ __device__ inline float d_acos(float x) { return acosf(x); }
__host__ __device__ inline double d_acos(double x) { return acos(x); }
__host__ __device__ inline float d_acosh(float x) { return acoshf(x); }
__host__ __device__ inline double d_acosh(double x) { return acosh(x); }
__host__ __device__ inline float d_asin(float x) { return asinf(x); }
__host__ __device__ inline double d_asin(double x) { return asin(x); }
__host__ __device__ inline float d_asinh(float x) { return asinhf(x); }
__host__ __device__ inline double d_asinh(double x) { return asinh(x); }
__host__ __device__ inline float d_atan(float x) { return atanf(x); }
__host__ __device__ inline double d_atan(double x) { return atan(x); }
__host__ __device__ inline float d_atanh(float x) { return atanhf(x); }
__host__ __device__ inline double d_atanh(double x) { return atanh(x); }
__host__ __device__ inline float d_ceil(float x) { return ceilf(x); }
__host__ __device__ inline double d_ceil(double x) { return ceil(x); }
__host__ __device__ inline float d_cos(float x) { return cosf(x); }
__host__ __device__ inline double d_cos(double x) { return cos(x); }
__host__ __device__ inline float d_cosh(float x) { return coshf(x); }
__host__ __device__ inline double d_cosh(double x) { return cosh(x); }
__host__ __device__ inline float d_floor(float x) { return floorf(x); }
__host__ __device__ inline double d_floor(double x) { return floor(x); }
__host__ __device__ inline float d_sin(float x) { return sinf(x); }
__host__ __device__ inline double d_sin(double x) { return sin(x); }
__host__ __device__ inline float d_sinh(float x) { return sinhf(x); }
__host__ __device__ inline double d_sinh(double x) { return sinh(x); }
__host__ __device__ inline float d_tan(float x) { return tanf(x); }
__host__ __device__ inline double d_tan(double x) { return tan(x); }
__host__ __device__ inline float d_round(float x) { return rintf(x); }  // ties to even, numpy round
__host__ __device__ inline double d_round(double x) { return rint(x); }
template <class T> __host__ __device__ inline T act_sign(T x) {
  return x > T(0) ? T(1) : x < T(0) ? T(-1) : x == T(0) ? T(0) : x;  // NaN stays NaN
}
template <class T> __host__ __device__ inline T act_is_nan(T x) { return x != x ? T(1) : T(0); }
template <class T> __host__ __device__ inline T act_is_inf(T x, T detect_negative, T detect_positive) {
  bool const neg = x == -__builtin_inff() && detect_negative != T(0);
  bool const pos = x == __builtin_inff() && detect_positive != T(0);
  return neg || pos ? T(1) : T(0);
}
template <class T> __host__ __device__ inline T act_not(T x) { return x == T(0) ? T(1) : T(0); }
template <class T> __host__ __device__ inline T act_nonzero(T x) { return x != T(0) ? T(1) : T(0); }

// Element-wise op of the state v with a constant c, emitter.py:261-275.
template <class T> __host__ __device__ inline T act_const(int act, T v, T c) {
  switch (act) {
    case ACT_BIAS: return v + c;
    case ACT_SUB_C: return v - c;
    case ACT_RSUB_C: return c - v;
    case ACT_MUL_C: return v * c;
    case ACT_DIV_C: return v / c;
    case ACT_RDIV_C: return c / v;
    case ACT_MIN_C: return v < c ? v : c;
    case ACT_RMIN_C: return c < v ? c : v;
    case ACT_MAX_C: return v > c ? v : c;
    case ACT_RMAX_C: return c > v ? c : v;
    case ACT_POW_C: return d_pow(v, c);
    case ACT_RPOW_C: return d_pow(c, v);
    default: return v;
  }
}

// Tensor-tensor binary operation of generated graphs (ponni_binary_op),
// emitter.py:261-275; comparisons and logic (interpreter.py:132-162) give 1 / 0.
template <class T> __host__ __device__ inline T apply_binary(int op, T l, T r) {
  switch (op) {
    case 0: return l + r;
    case 1: return l - r;
    case 2: return l * r;
    case 3: return l / r;
    case 4: return l < r ? l : r;
    case 5: return l > r ? l : r;
    case 7: return l == r ? T(1) : T(0);
    case 8: return l > r ? T(1) : T(0);
    case 9: return l >= r ? T(1) : T(0);
    case 10: return l < r ? T(1) : T(0);
    case 11: return l <= r ? T(1) : T(0);
    case 12: return (l != T(0)) && (r != T(0)) ? T(1) : T(0);
    case 13: return (l != T(0)) || (r != T(0)) ? T(1) : T(0);
    case 14: return (l != T(0)) != (r != T(0)) ? T(1) : T(0);
    case 15: return l >= T(0) ? l : l * r;  // PRelu
    default: return d_pow(l, r);
  }
}

// state = cond != 0 ? a : b
template <class T> __host__ __device__ inline T apply_select(T cond, T a, T b) { return cond != T(0) ? a : b; }

// Apply one parameter-free (or scalar-parameter) layer-template activation
// to every element visited by `each` (the NARROW and MFMA families, which run
// template chains only).  The switch sits outside the element loop so each case is
// one straight-line loop.  `each(f)` must call f(float&) on every element.
template <class T, class Each>
__host__ __device__ inline void map_activation(int act, T a, T b, Each&& each) {
  switch (act) {
    case ACT_RELU: each([](T& v) { v = act_relu(v); }); break;
    case ACT_LEAKY_RELU: each([a](T& v) { v = act_leaky_relu(v, a); }); break;
    case ACT_ELU: each([a](T& v) { v = act_elu(v, a); }); break;
    case ACT_SELU: each([](T& v) { v = act_selu(v); }); break;
    case ACT_GELU_ERF: each([](T& v) { v = act_gelu_erf(v); }); break;
    case ACT_GELU_TANH: each([](T& v) { v = act_gelu_tanh(v); }); break;
    case ACT_SILU: each([](T& v) { v = act_silu(v); }); break;
    case ACT_SIGMOID: each([](T& v) { v = act_sigmoid(v); }); break;
    case ACT_TANH: each([](T& v) { v = act_tanh(v); }); break;
    case ACT_SOFTPLUS: each([a](T& v) { v = act_softplus(v, a); }); break;
    case ACT_HARD_SIGMOID: each([a, b](T& v) { v = act_hard_sigmoid(v, a, b); }); break;
    case ACT_HARD_SWISH: each([](T& v) { v = act_hard_swish(v); }); break;
    case ACT_MISH: each([](T& v) { v = act_mish(v); }); break;
    default: break;
  }
}

// Scalar form for the per-sample generic kernel; `bias` is the step's
// parameter element (bias or constant operand) for the feature.
template <class T>
__host__ __device__ inline T apply_step(int act, T x, T bias, T a, T b) {
  switch (act) {
    case ACT_BIAS: return x + bias;  // ponni_Bias.h:66-68
    case ACT_ABS: return d_abs(x);
    case ACT_NEG: return -x;
    case ACT_EXP: return d_exp(x);
    case ACT_LOG: return d_log(x);
    case ACT_SQRT: return d_sqrt(x);
    case ACT_RECIPROCAL: return T(1) / x;
    case ACT_SOFTSIGN: return act_softsign(x);
    case ACT_CELU: return act_celu(x, a);
    case ACT_THRESHOLDED_RELU: return act_thresholded_relu(x, a);
    case ACT_ERF: return d_erf(x);
    case ACT_SELU_AG: return act_selu_ag(x, a, b);
    case ACT_ACOS: return d_acos(x);
    case ACT_ACOSH: return d_acosh(x);
    case ACT_ASIN: return d_asin(x);
    case ACT_ASINH: return d_asinh(x);
    case ACT_ATAN: return d_atan(x);
    case ACT_ATANH: return d_atanh(x);
    case ACT_CEIL: return d_ceil(x);
    case ACT_COS: return d_cos(x);
    case ACT_COSH: return d_cosh(x);
    case ACT_FLOOR: return d_floor(x);
    case ACT_SIN: return d_sin(x);
    case ACT_SINH: return d_sinh(x);
    case ACT_TAN: return d_tan(x);
    case ACT_ROUND: return d_round(x);
    case ACT_SIGN: return act_sign(x);
    case ACT_IS_NAN: return act_is_nan(x);
    case ACT_IS_INF: return act_is_inf(x, a, b);
    case ACT_NOT: return act_not(x);
    case ACT_NONZERO: return act_nonzero(x);
    case ACT_CBIN: return b != T(0) ? apply_binary<T>(static_cast<int>(a), bias, x)
                                    : apply_binary<T>(static_cast<int>(a), x, bias);
    case ACT_RELU: return act_relu(x);
    case ACT_LEAKY_RELU: return act_leaky_relu(x, a);
    case ACT_ELU: return act_elu(x, a);
    case ACT_SELU: return act_selu(x);
    case ACT_GELU_ERF: return act_gelu_erf(x);
    case ACT_GELU_TANH: return act_gelu_tanh(x);
    case ACT_SILU: return act_silu(x);
    case ACT_SIGMOID: return act_sigmoid(x);
    case ACT_TANH: return act_tanh(x);
    case ACT_SOFTPLUS: return act_softplus(x, a);
    case ACT_HARD_SIGMOID: return act_hard_sigmoid(x, a, b);
    case ACT_HARD_SWISH: return act_hard_swish(x);
    case ACT_MISH: return act_mish(x);
    default: return act_has_param(act) ? act_const(act, x, bias) : x;
  }
}

// ---- activations on the hardware transcendentals -------------------------
// The generated FUSED and NARROW kernels evaluate the logistic family through
// v_exp_f32 and v_rcp_f32 (2^x and 1/x, about 1 ulp each), branch-free.  Each is the same
// function as the reference formula it replaces, rewritten with
// sigmoid(t) = 1 / (1 + 2^(-t log2 e)); the results differ from the
// reference's libm-based evaluation by a few fp32 ulp relative to the
// quantities that are summed later (tanh near 0 carries ~1e-7 absolute,
// not relative, error, which is what 1 + tanh, the GELU and the next dense
// layer see).  Saturation comes out of 2^x -> inf / 0 and 1/inf = 0.
constexpr float kLog2e = 1.4426950408889634f;

__device__ inline float fast_sigmoid(float t) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * t));
}
// ponni_Sigmoid.h:45-49
__device__ inline float act_sigmoid_fast(float x) { return fast_sigmoid(x); }
// ponni_Silu.h:45-49: x * sigmoid(x)
__device__ inline float act_silu_fast(float x) { return x * fast_sigmoid(x); }
// ponni_Tanh.h:44: tanh(x) = 1 - 2 / (1 + 2^(2 x log2 e))
__device__ inline float act_tanh_fast(float x) {
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(2.0f * kLog2e * x)), 1.0f);
}
// ponni_Gelu.h:48-53: 0.5 x (1 + tanh(u)) = x sigmoid(2u),
// u = sqrt(2/pi) (x + 0.044715 x^3)
__device__ inline float act_gelu_tanh_fast(float x) {
  float const u = 0.79788456080286535588f * (x + 0.044715f * (x * x * x));
  return x * fast_sigmoid(2.0f * u);
}

}  // namespace ponni_hip
