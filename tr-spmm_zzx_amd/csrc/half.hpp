// float32 -> IEEE binary16 bits, round to nearest even (c10::Half semantics: NaN -> 0x7e00 with the
// sign, overflow -> infinity, subnormals rounded exactly).  Integer arithmetic on the float's bits,
// so host code and device code (a constexpr function may run on either) produce the same bits.
#pragma once
#include <cstdint>

namespace trs {
constexpr uint16_t half_bits_of(uint32_t x) {
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    // subnormal result: round(|f| * 2^24) to nearest even, integer arithmetic on the mantissa
    if (ax < 0x33000000u) return (uint16_t)sign;   // below half of the smallest subnormal
    const uint32_t e = ax >> 23;                   // 102..112
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126 - e;                // |f| * 2^24 = m * 2^(e - 150 + 24)
    uint32_t q = m >> shift;
    const uint32_t rest = m & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rest > half || (rest == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = (((ax >> 23) - 112) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rest = ax & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}
}  // namespace trs
