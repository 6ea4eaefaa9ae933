// ponni::TwoHalf / ponni::TwoMask: two adjacent batch lanes of binary16
// values, and their predicates, as the reference's generated half2 models
// use them (src/utils/ponni_TwoHalf.h:15-371, ponni_TwoMask.h:11-49).  The
// names, argument meanings and lane results are the reference's; the
// implementation is this library's own:
//   - storage is a two-element _Float16 vector, so device code gets packed
//     v_pk_add / v_pk_mul / v_pk_fma_f16 for +, -, *, fma (one rounding per
//     lane, as __hadd2 / __hmul2 / __hfma2);
//   - division, reciprocal and every activation / math function evaluate
//     each lane in fp32 and round the result to binary16 once
//     (ponni_TwoHalf.h:134-371: fp32 per lane of the half value, rounded);
//   - host code computes +, -, *, / in fp32 and fma in fp64 before the one
//     rounding: both give the correctly rounded binary16 result (fp32 has
//     2 * 11 + 2 significand bits, so rounding through it is innocuous for
//     the four operations; fp64 holds the product exactly).
// Round is ties-to-even and Sign keeps NaN and returns +0 for -0
// (ponni_TwoHalf.h:31-48); comparisons and is_nan / is_inf give TwoMask.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>

namespace ponni {

class TwoMask {
  std::uint8_t bits_ = 0;
  __host__ __device__ explicit TwoMask(std::uint8_t bits) : bits_(bits) {}

 public:
  TwoMask() = default;
  __host__ __device__ static TwoMask from_bools(bool low, bool high) {
    return TwoMask(static_cast<std::uint8_t>((low ? 1u : 0u) | (high ? 2u : 0u)));
  }
  __host__ __device__ static TwoMask splat(bool value) { return from_bools(value, value); }
  __host__ __device__ bool low() const { return (bits_ & 1u) != 0; }
  __host__ __device__ bool high() const { return (bits_ & 2u) != 0; }
  __host__ __device__ static TwoMask logical_and(TwoMask a, TwoMask b) { return TwoMask(a.bits_ & b.bits_); }
  __host__ __device__ static TwoMask logical_or(TwoMask a, TwoMask b) { return TwoMask(a.bits_ | b.bits_); }
  __host__ __device__ static TwoMask logical_xor(TwoMask a, TwoMask b) { return TwoMask(a.bits_ ^ b.bits_); }
  __host__ __device__ static TwoMask logical_not(TwoMask a) { return TwoMask((~a.bits_) & 3u); }
  __host__ __device__ static TwoMask equal(TwoMask a, TwoMask b) {
    return from_bools(a.low() == b.low(), a.high() == b.high());
  }
};
static_assert(sizeof(TwoMask) == 1, "one byte of lane predicates");

class TwoHalf {
 public:
  using half_type = _Float16;
  typedef _Float16 lanes_type __attribute__((ext_vector_type(2)));

 private:
  lanes_type v_;
  __host__ __device__ explicit TwoHalf(lanes_type v) : v_(v) {}

  // One lane-wise fp32 function, each result rounded to binary16 once.
  template <class F>
  __host__ __device__ static TwoHalf map(TwoHalf x, F f) {
    return from_floats(f(x.low()), f(x.high()));
  }
  template <class F>
  __host__ __device__ static TwoHalf map2(TwoHalf x, TwoHalf y, F f) {
    return from_floats(f(x.low(), y.low()), f(x.high(), y.high()));
  }
  __host__ __device__ static bool nan_bits(float v) {
    std::uint32_t b;
    __builtin_memcpy(&b, &v, sizeof b);  // classification by bits survives fast-math flags
    return (b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu) != 0;
  }
  // Ties to even; a value that rounds to zero gives +0, a -0 input stays -0.
  __host__ __device__ static float round_even(float v) {
    if (!std::isfinite(v) || v == 0.0f) return v;
    float const r = std::nearbyint(v);
    return r == 0.0f ? 0.0f : r;
  }
  __host__ __device__ static float sign_of(float v) {
    return nan_bits(v) ? v : v > 0.0f ? 1.0f : v < 0.0f ? -1.0f : 0.0f;
  }

 public:
  TwoHalf() = default;
  __host__ __device__ explicit TwoHalf(__half2 h) { __builtin_memcpy(&v_, &h, sizeof v_); }
  __host__ __device__ __half2 value() const {
    __half2 h;
    __builtin_memcpy(&h, &v_, sizeof h);
    return h;
  }
  __host__ __device__ lanes_type lanes() const { return v_; }

  __host__ __device__ static TwoHalf from_floats(float low, float high) {
    lanes_type v;
    v[0] = static_cast<_Float16>(low);
    v[1] = static_cast<_Float16>(high);
    return TwoHalf(v);
  }
  __host__ __device__ static TwoHalf from_halves(half_type low, half_type high) {
    lanes_type v;
    v[0] = low;
    v[1] = high;
    return TwoHalf(v);
  }
  __host__ __device__ static TwoHalf splat(half_type value) { return from_halves(value, value); }
  __host__ __device__ static TwoHalf zero() { return from_floats(0.0f, 0.0f); }
  __host__ __device__ float low() const { return static_cast<float>(v_[0]); }
  __host__ __device__ float high() const { return static_cast<float>(v_[1]); }

  // a * b + c per lane, rounded once (TwoHalf::fma, ponni_TwoHalf.h:97-105).
  __host__ __device__ static TwoHalf fma(TwoHalf a, TwoHalf b, TwoHalf c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return TwoHalf(__builtin_elementwise_fma(a.v_, b.v_, c.v_));
#else
    return from_floats(static_cast<float>(std::fma(double(a.low()), double(b.low()), double(c.low()))),
                       static_cast<float>(std::fma(double(a.high()), double(b.high()), double(c.high()))));
#endif
  }
  __host__ __device__ friend TwoHalf operator+(TwoHalf a, TwoHalf b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return TwoHalf(a.v_ + b.v_);
#else
    return from_floats(a.low() + b.low(), a.high() + b.high());
#endif
  }
  __host__ __device__ friend TwoHalf operator-(TwoHalf a, TwoHalf b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return TwoHalf(a.v_ - b.v_);
#else
    return from_floats(a.low() - b.low(), a.high() - b.high());
#endif
  }
  __host__ __device__ friend TwoHalf operator*(TwoHalf a, TwoHalf b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return TwoHalf(a.v_ * b.v_);
#else
    return from_floats(a.low() * b.low(), a.high() * b.high());
#endif
  }
  __host__ __device__ friend TwoHalf operator/(TwoHalf a, TwoHalf b) {
    return map2(a, b, [](float x, float y) { return x / y; });
  }

  // Activations (ponni_TwoHalf.h:138-153, :278-371).
  __host__ __device__ static TwoHalf relu(TwoHalf x) {
    return map(x, [](float v) { return v > 0.0f ? v : 0.0f; });
  }
  __host__ __device__ static TwoHalf sigmoid(TwoHalf x) {
    return map(x, [](float v) { return 1.0f / (1.0f + std::exp(-v)); });
  }
  __host__ __device__ static TwoHalf tanh(TwoHalf x) {
    return map(x, [](float v) { return std::tanh(v); });
  }
  __host__ __device__ static TwoHalf leaky_relu(TwoHalf x, float alpha) {
    return map(x, [alpha](float v) { return v >= 0.0f ? v : alpha * v; });
  }
  __host__ __device__ static TwoHalf elu(TwoHalf x, float alpha) {
    return map(x, [alpha](float v) { return v >= 0.0f ? v : alpha * (std::exp(v) - 1.0f); });
  }
  __host__ __device__ static TwoHalf celu(TwoHalf x, float alpha) {
    return map(x, [alpha](float v) { return v > 0.0f ? v : alpha * (std::exp(v / alpha) - 1.0f); });
  }
  __host__ __device__ static TwoHalf selu(TwoHalf x, float alpha, float gamma) {
    return map(x, [alpha, gamma](float v) { return gamma * (v > 0.0f ? v : alpha * (std::exp(v) - 1.0f)); });
  }
  __host__ __device__ static TwoHalf softsign(TwoHalf x) {
    return map(x, [](float v) { return v / (1.0f + std::fabs(v)); });
  }
  __host__ __device__ static TwoHalf thresholded_relu(TwoHalf x, float alpha) {
    return map(x, [alpha](float v) { return v > alpha ? v : 0.0f; });
  }
  __host__ __device__ static TwoHalf prelu(TwoHalf x, TwoHalf slope) {
    return map2(x, slope, [](float v, float s) { return v >= 0.0f ? v : v * s; });
  }
  __host__ __device__ static TwoHalf gelu(TwoHalf x, bool approximate) {
    if (approximate)
      return map(x, [](float v) {
        return 0.5f * v * (1.0f + std::tanh(0.7978845608028654f * (v + 0.044715f * v * v * v)));
      });
    return map(x, [](float v) { return 0.5f * v * (1.0f + std::erf(v * 0.7071067811865475f)); });
  }
  __host__ __device__ static TwoHalf silu(TwoHalf x) { return x * sigmoid(x); }
  __host__ __device__ static TwoHalf softplus(TwoHalf x) {
    return map(x, [](float v) { return (v > 0.0f ? v : 0.0f) + std::log(1.0f + std::exp(-std::fabs(v))); });
  }
  __host__ __device__ static TwoHalf hard_sigmoid(TwoHalf x, float alpha, float beta) {
    return map(x, [alpha, beta](float v) {
      float const t = alpha * v + beta;
      return t < 0.0f ? 0.0f : (t > 1.0f ? 1.0f : t);
    });
  }
  __host__ __device__ static TwoHalf hard_swish(TwoHalf x) { return x * hard_sigmoid(x, 1.0f / 6.0f, 0.5f); }
  __host__ __device__ static TwoHalf mish(TwoHalf x) { return x * tanh(softplus(x)); }

  // Math (ponni_TwoHalf.h:155-241).
  __host__ __device__ static TwoHalf abs(TwoHalf x) { return map(x, [](float v) { return std::fabs(v); }); }
  __host__ __device__ static TwoHalf acos(TwoHalf x) { return map(x, [](float v) { return std::acos(v); }); }
  __host__ __device__ static TwoHalf acosh(TwoHalf x) { return map(x, [](float v) { return std::acosh(v); }); }
  __host__ __device__ static TwoHalf asin(TwoHalf x) { return map(x, [](float v) { return std::asin(v); }); }
  __host__ __device__ static TwoHalf asinh(TwoHalf x) { return map(x, [](float v) { return std::asinh(v); }); }
  __host__ __device__ static TwoHalf atan(TwoHalf x) { return map(x, [](float v) { return std::atan(v); }); }
  __host__ __device__ static TwoHalf atanh(TwoHalf x) { return map(x, [](float v) { return std::atanh(v); }); }
  __host__ __device__ static TwoHalf ceil(TwoHalf x) { return map(x, [](float v) { return std::ceil(v); }); }
  __host__ __device__ static TwoHalf cos(TwoHalf x) { return map(x, [](float v) { return std::cos(v); }); }
  __host__ __device__ static TwoHalf cosh(TwoHalf x) { return map(x, [](float v) { return std::cosh(v); }); }
  __host__ __device__ static TwoHalf erf(TwoHalf x) { return map(x, [](float v) { return std::erf(v); }); }
  __host__ __device__ static TwoHalf exp(TwoHalf x) { return map(x, [](float v) { return std::exp(v); }); }
  __host__ __device__ static TwoHalf floor(TwoHalf x) { return map(x, [](float v) { return std::floor(v); }); }
  __host__ __device__ static TwoHalf log(TwoHalf x) { return map(x, [](float v) { return std::log(v); }); }
  __host__ __device__ static TwoHalf sqrt(TwoHalf x) { return map(x, [](float v) { return std::sqrt(v); }); }
  __host__ __device__ static TwoHalf reciprocal(TwoHalf x) { return map(x, [](float v) { return 1.0f / v; }); }
  __host__ __device__ static TwoHalf round(TwoHalf x) { return map(x, [](float v) { return round_even(v); }); }
  __host__ __device__ static TwoHalf sign(TwoHalf x) { return map(x, [](float v) { return sign_of(v); }); }
  __host__ __device__ static TwoHalf sin(TwoHalf x) { return map(x, [](float v) { return std::sin(v); }); }
  __host__ __device__ static TwoHalf sinh(TwoHalf x) { return map(x, [](float v) { return std::sinh(v); }); }
  __host__ __device__ static TwoHalf tan(TwoHalf x) { return map(x, [](float v) { return std::tan(v); }); }
  __host__ __device__ static TwoHalf pow(TwoHalf base, TwoHalf e) {
    return map2(base, e, [](float b, float p) { return std::pow(b, p); });
  }
  __host__ __device__ static TwoHalf minimum(TwoHalf a, TwoHalf b) {
    return map2(a, b, [](float x, float y) { return x < y ? x : y; });
  }
  __host__ __device__ static TwoHalf maximum(TwoHalf a, TwoHalf b) {
    return map2(a, b, [](float x, float y) { return x > y ? x : y; });
  }

  // Predicates (ponni_TwoHalf.h:253-334).
  __host__ __device__ static TwoMask equal(TwoHalf a, TwoHalf b) {
    return TwoMask::from_bools(a.low() == b.low(), a.high() == b.high());
  }
  __host__ __device__ static TwoMask greater(TwoHalf a, TwoHalf b) {
    return TwoMask::from_bools(a.low() > b.low(), a.high() > b.high());
  }
  __host__ __device__ static TwoMask greater_or_equal(TwoHalf a, TwoHalf b) {
    return TwoMask::from_bools(a.low() >= b.low(), a.high() >= b.high());
  }
  __host__ __device__ static TwoMask less(TwoHalf a, TwoHalf b) {
    return TwoMask::from_bools(a.low() < b.low(), a.high() < b.high());
  }
  __host__ __device__ static TwoMask less_or_equal(TwoHalf a, TwoHalf b) {
    return TwoMask::from_bools(a.low() <= b.low(), a.high() <= b.high());
  }
  __host__ __device__ static TwoHalf select(TwoMask c, TwoHalf when_true, TwoHalf when_false) {
    return from_halves(c.low() ? when_true.v_[0] : when_false.v_[0], c.high() ? when_true.v_[1] : when_false.v_[1]);
  }
  __host__ __device__ static TwoMask is_nan(TwoHalf x) { return TwoMask::from_bools(nan_bits(x.low()), nan_bits(x.high())); }
  __host__ __device__ static TwoMask is_inf(TwoHalf x, bool detect_negative, bool detect_positive) {
    auto hit = [=](float v) { return std::isinf(v) && ((v < 0.0f && detect_negative) || (v > 0.0f && detect_positive)); };
    return TwoMask::from_bools(hit(x.low()), hit(x.high()));
  }
};
static_assert(sizeof(TwoHalf) == sizeof(__half2), "two binary16 lanes");

}  // namespace ponni
