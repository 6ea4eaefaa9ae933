// Host-side IEEE binary16 / bfloat16 conversions (round to nearest even),
// used to pre-round parameters of F16 / BF16 plans.
#pragma once

#include <cstdint>
#include <cstring>

namespace ponni_hip {

inline uint16_t float_to_half_bits(float value) {
  uint32_t x;
  std::memcpy(&x, &value, 4);
  uint32_t const sign = (x >> 16) & 0x8000u;
  uint32_t const exp = (x >> 23) & 0xffu;
  uint32_t mant = x & 0x7fffffu;
  if (exp == 0xffu) return static_cast<uint16_t>(sign | 0x7c00u | (mant ? 0x200u : 0u));
  int32_t e = static_cast<int32_t>(exp) - 127 + 15;
  if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);  // overflow -> inf
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);  // underflow -> signed zero
    mant |= 0x800000u;
    uint32_t const shift = static_cast<uint32_t>(14 - e);
    uint32_t half_mant = mant >> shift;
    uint32_t const rem = mant & ((1u << shift) - 1u);
    uint32_t const halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half_mant & 1u))) half_mant++;
    return static_cast<uint16_t>(sign | half_mant);
  }
  uint32_t half = sign | (static_cast<uint32_t>(e) << 10) | (mant >> 13);
  uint32_t const rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;  // may carry into exponent
  return static_cast<uint16_t>(half);
}

inline float half_bits_to_float(uint16_t h) {
  uint32_t const sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
  uint32_t const exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else {
      int e = -1;
      do {
        e++;
        mant <<= 1;
      } while ((mant & 0x400u) == 0);
      x = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (mant << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float out;
  std::memcpy(&out, &x, 4);
  return out;
}

inline uint16_t float_to_bf16_bits(float value) {
  uint32_t x;
  std::memcpy(&x, &value, 4);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return static_cast<uint16_t>((x >> 16) | 0x40u);
  uint32_t const lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return static_cast<uint16_t>(x >> 16);
}

inline float bf16_bits_to_float(uint16_t h) {
  uint32_t const x = static_cast<uint32_t>(h) << 16;
  float out;
  std::memcpy(&out, &x, 4);
  return out;
}

// Round a value to the precision of a plan dtype (identity for F32 / F64).
inline double round_to_dtype(double value, int dtype) {
  if (dtype == 3) return half_bits_to_float(float_to_half_bits(static_cast<float>(value)));
  if (dtype == 4) return bf16_bits_to_float(float_to_bf16_bits(static_cast<float>(value)));
  if (dtype == 1) return static_cast<float>(value);
  return value;
}

}  // namespace ponni_hip
