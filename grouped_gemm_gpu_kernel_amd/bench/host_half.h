// Host-side float -> IEEE binary16 conversion, round to nearest even: the
// value __float2half_rn gives for the reference benchmark's operands
// (bench/benchmark_grouped_gemm.cu:486-491).  Plain C++ so the benchmark
// harness needs no device compiler.
#pragma once

#include <cstdint>
#include <cstring>

inline uint16_t host_float_to_half_rn(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t mag = x & 0x7fffffffu;
  if (mag >= 0x7f800000u) return static_cast<uint16_t>(sign | (mag > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (mag >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // at or past 65520: infinity
  if (mag < 0x38800000u) {                                                  // below 2^-14: subnormal or zero
    if (mag <= 0x33000000u) return static_cast<uint16_t>(sign);           // at most half of 2^-24
    const uint32_t e = mag >> 23, m = (mag & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126 - e;  // value = m * 2^(e-150); the result counts units of 2^-24
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return static_cast<uint16_t>(sign | h);
  }
  uint32_t h = (mag - 0x38000000u) >> 13;  // rebias 127 -> 15, drop 13 mantissa bits
  const uint32_t rem = mag & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return static_cast<uint16_t>(sign | h);
}
