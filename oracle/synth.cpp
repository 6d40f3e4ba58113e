// ORACLE — test infrastructure, not product code (see oracle.h).
//
// The seeded synthetic model, restated independently of the product's
// loader so that the two can be compared value for value. The reference
// reads real checkpoints (generator.cpp:364-434); its benchmark model here is
// the released dimensions with every matrix and embedding drawn from
// N(0, 0.02) and rounded to fp16, norms 1.0.
//
// Specification (shared with the product, written twice on purpose):
//   splitmix64(x)      Vigna's SplitMix64 finaliser of x + 0x9E3779B97F4A7C15
//   base               splitmix64(seed ^ splitmix64(tensor)) + 2 * element
//   u1                 ((splitmix64(base) >> 11) + 1) * 2^-53     in (0, 1]
//   u2                 (splitmix64(base + 1) >> 11) * 2^-53       in [0, 1)
//   normal             sqrt(-2 log u1) cos(2 pi u2)                (double)
//   matrix value       half(float(0.02 * normal))
//   norm value         1.0, or half(float(1 + jitter * normal))
// `element` is row * columns + column in the checkpoint tensor's own shape.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "oracle.h"

namespace {

std::uint64_t SplitMix64(std::uint64_t x) {
  std::uint64_t z = x + 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

// Round-to-nearest-even float -> binary16 -> float, subnormals included.
float RoundHalf(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, 4);
  const std::uint32_t sign = u & 0x80000000U;
  const std::uint32_t magnitude = u & 0x7FFFFFFFU;
  std::uint16_t h;
  if (magnitude >= 0x7F800000U) {  // inf or nan
    h = static_cast<std::uint16_t>((magnitude > 0x7F800000U) ? 0x7E00 : 0x7C00);
  } else if (magnitude >= 0x477FF000U) {  // rounds to >= 65520: overflow
    h = 0x7C00;
  } else if (magnitude >= 0x38800000U) {  // normal half (>= 2^-14)
    const std::uint32_t rest = magnitude & 0x1FFFU;
    std::uint32_t v = ((magnitude >> 13) - ((127 - 15) << 10));
    if (rest > 0x1000U || (rest == 0x1000U && (v & 1U)))
      v += 1;
    h = static_cast<std::uint16_t>(v);
  } else if (magnitude >= 0x33000000U) {  // subnormal half (>= 2^-25)
    const std::uint32_t exponent = magnitude >> 23;
    const std::uint32_t mantissa = (magnitude & 0x7FFFFFU) | 0x800000U;
    // value = mantissa * 2^(exponent - 150) = v * 2^-24 (the half
    // subnormal unit) with v = mantissa * 2^(exponent - 126).
    const std::uint32_t drop = 126 - exponent;  // 14 ... 24
    std::uint32_t v = mantissa >> drop;
    const std::uint32_t rest = mantissa & ((1U << drop) - 1U);
    const std::uint32_t halfway = 1U << (drop - 1);
    if (rest > halfway || (rest == halfway && (v & 1U)))
      v += 1;
    h = static_cast<std::uint16_t>(v);
  } else {
    h = 0;
  }
  // back to float
  const std::uint32_t he = (h >> 10) & 0x1FU;
  const std::uint32_t hm = h & 0x3FFU;
  float out;
  if (he == 0x1FU) {
    const std::uint32_t bits = sign | 0x7F800000U | (hm << 13);
    std::memcpy(&out, &bits, 4);
  } else if (he != 0) {
    const std::uint32_t bits = sign | ((he + 112U) << 23) | (hm << 13);
    std::memcpy(&out, &bits, 4);
  } else {
    out = static_cast<float>(hm) * 5.9604644775390625e-08F;  // 2^-24
    if (sign != 0U)
      out = -out;
  }
  return out;
}

}  // namespace

extern "C" {

double orc_synth_normal(uint64_t seed, uint64_t tensor, uint64_t element) {
  const std::uint64_t base = SplitMix64(seed ^ SplitMix64(tensor)) + 2 * element;
  const std::uint64_t h1 = SplitMix64(base);
  const std::uint64_t h2 = SplitMix64(base + 1);
  const double u1 = static_cast<double>((h1 >> 11) + 1) * 0x1.0p-53;
  const double u2 = static_cast<double>(h2 >> 11) * 0x1.0p-53;
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

float orc_round_half(float x) { return RoundHalf(x); }

void orc_synth_values(uint64_t seed, uint64_t tensor, uint64_t first,
                      int64_t count, int is_norm, float jitter, float* out) {
  for (int64_t i = 0; i < count; ++i) {
    const std::uint64_t e = first + static_cast<std::uint64_t>(i);
    if (is_norm) {
      out[i] = jitter == 0.0F
                   ? 1.0F
                   : RoundHalf(static_cast<float>(
                         1.0 + static_cast<double>(jitter) *
                                   orc_synth_normal(seed, tensor, e)));
    } else {
      out[i] = RoundHalf(
          static_cast<float>(0.02 * orc_synth_normal(seed, tensor, e)));
    }
  }
}

}  // extern "C"
