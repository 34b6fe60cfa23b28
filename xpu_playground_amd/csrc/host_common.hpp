// Host-side helpers of the product library: 16-bit codecs, the seeded
// counter-based generator, option parsing and statistics.
#pragma once

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace xpu {

// qwen3/model.cpp:497-502 (round to nearest even via +0x7fff+lsb).
inline uint16_t f32_to_bf16(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}

inline float bf16_to_f32(uint16_t v) {
  const uint32_t bits = static_cast<uint32_t>(v) << 16;
  float r;
  std::memcpy(&r, &bits, 4);
  return r;
}

// level_zero/peak_l0.cpp:740-761
inline uint16_t f32_to_fp16(float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int exponent = static_cast<int>((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return static_cast<uint16_t>(sign);
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return static_cast<uint16_t>(sign | ((mantissa + 0xfffu + ((mantissa >> 13) & 1u)) >> 13));
  }
  if (exponent >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
  mantissa += 0xfffu + ((mantissa >> 13) & 1u);
  if (mantissa & 0x800000u) {
    mantissa = 0;
    if (++exponent >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
  }
  return static_cast<uint16_t>(sign | (static_cast<uint32_t>(exponent) << 10) | (mantissa >> 13));
}

// level_zero/peak_l0.cpp:763-785
inline float fp16_to_f32(uint16_t v) {
  const uint32_t sign = static_cast<uint32_t>(v & 0x8000u) << 16;
  uint32_t exponent = (v >> 10) & 0x1fu;
  uint32_t mantissa = v & 0x3ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      int shift = 0;
      while ((mantissa & 0x400u) == 0) { mantissa <<= 1; ++shift; }
      mantissa &= 0x3ffu;
      bits = sign | (static_cast<uint32_t>(127 - 14 - shift) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float r;
  std::memcpy(&r, &bits, 4);
  return r;
}

inline uint16_t encode16(float v, int dtype) { return dtype ? f32_to_fp16(v) : f32_to_bf16(v); }
inline float decode16(uint16_t v, int dtype) { return dtype ? fp16_to_f32(v) : bf16_to_f32(v); }

// splitmix64 finaliser (Steele, Lea, Flood, OOPSLA 2014)
inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

inline uint64_t counter_hash(uint64_t seed, uint64_t index) {
  return mix64(mix64(seed) + (index + 1) * 0x9e3779b97f4a7c15ull);
}

// N(0,1) by Box-Muller (cosine branch) from the two 24-bit halves of a hash
inline double normal_from_hash(uint64_t h) {
  const double u1 = static_cast<double>((h >> 40) + 1) * 0x1p-24;
  const double u2 = static_cast<double>((h >> 16) & 0xffffffu) * 0x1p-24;
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// gemv.cpp:45-64 / main.cpp:31-41 style strict positive integer parsing
template <typename T> T parse_positive(std::string_view text, std::string_view option) {
  T value{};
  const auto parsed = std::from_chars(text.data(), text.data() + text.size(), value);
  if (parsed.ec != std::errc{} || parsed.ptr != text.data() + text.size() || !value)
    throw std::invalid_argument(std::string(option) + " requires a positive integer");
  return value;
}

template <typename T> T parse_unsigned(std::string_view text, std::string_view option) {
  T value{};
  const auto parsed = std::from_chars(text.data(), text.data() + text.size(), value);
  if (parsed.ec != std::errc{} || parsed.ptr != text.data() + text.size())
    throw std::invalid_argument(std::string(option) + " requires a non-negative integer");
  return value;
}

// median as in gemv.cpp:135-139 (mean of the two middle values when even)
inline double median_of(std::vector<double> v) {
  if (v.empty()) return 0.0;
  std::sort(v.begin(), v.end());
  const size_t mid = v.size() / 2;
  return (v.size() & 1) ? v[mid] : 0.5 * (v[mid - 1] + v[mid]);
}

inline double max_of(const std::vector<double> &v) {
  return v.empty() ? 0.0 : *std::max_element(v.begin(), v.end());
}

// unit in the last place of a bf16 value of magnitude |v| (2^(e-7))
inline double bf16_ulp(double v) {
  const double a = std::fabs(v);
  if (a < 0x1p-126) return 0x1p-133;
  return std::ldexp(1.0, std::ilogb(a) - 7);
}
inline double fp16_ulp(double v) {
  const double a = std::fabs(v);
  if (a < 0x1p-14) return 0x1p-24;
  return std::ldexp(1.0, std::ilogb(a) - 10);
}

}  // namespace xpu
