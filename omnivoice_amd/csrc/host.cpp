// Host-side decoding helpers and the seeded synthetic model.
#include "host.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <numeric>
#include <thread>

namespace ovg {

std::vector<std::size_t> UnmaskSchedule(std::size_t total, std::size_t steps,
                                        float t_shift) {
  // torch.linspace(0, 1, steps + 1) in float32 is evaluated from both ends:
  // the first half as step * i, the second half as 1 - step * (steps - i).
  std::vector<float> times(steps + 1);
  const float step = 1.0F / static_cast<float>(steps);
  const std::size_t middle = (steps + 1) / 2;
  for (std::size_t i = 0; i <= steps; ++i) {
    const float linear = i < middle
                             ? step * static_cast<float>(i)
                             : 1.0F - step * static_cast<float>(steps - i);
    times[i] = t_shift * linear / (1.0F + (t_shift - 1.0F) * linear);
  }
  std::vector<std::size_t> counts(steps, 0);
  std::size_t left = total;
  for (std::size_t i = 0; i < steps; ++i) {
    std::size_t count = left;
    if (i + 1 < steps) {
      const double width =
          static_cast<double>(times[i + 1]) - static_cast<double>(times[i]);
      count = std::min(left, static_cast<std::size_t>(std::ceil(
                                 static_cast<double>(total) * width)));
    }
    counts[i] = count;
    left -= count;
  }
  return counts;
}

std::vector<std::int32_t> BuildInput(const std::vector<std::uint32_t>& text,
                                     const std::vector<std::int32_t>& reference,
                                     std::size_t reference_frames,
                                     std::size_t target_frames,
                                     std::size_t codebooks,
                                     std::uint32_t mask_id) {
  const std::size_t length = text.size() + reference_frames + target_frames;
  std::vector<std::int32_t> ids(codebooks * length,
                                static_cast<std::int32_t>(mask_id));
  for (std::size_t c = 0; c < codebooks; ++c) {
    std::int32_t* row = ids.data() + c * length;
    std::transform(text.begin(), text.end(), row,
                   [](std::uint32_t t) { return static_cast<std::int32_t>(t); });
    if (reference_frames > 0)
      std::copy_n(reference.data() + c * reference_frames, reference_frames,
                  row + text.size());
  }
  return ids;
}

void GumbelNoise(std::mt19937_64* random, std::size_t count, float* out) {
  for (std::size_t i = 0; i < count; ++i) {
    // 24 random bits scaled into [0, 1), then -log(-log(u + 1e-10) + 1e-10)
    // in float, as the reference's _gumbel_sample restatement.
    const float uniform =
        static_cast<float>((*random)() >> 40) * 0x1.0p-24F;
    out[i] = -std::log(-std::log(uniform + 1e-10F) + 1e-10F);
  }
}

std::vector<std::size_t> SelectPositions(
    std::mt19937_64* random, float layer_penalty, float temperature,
    std::size_t count, std::size_t codebooks, std::size_t frames,
    const std::vector<std::int32_t>& prediction,
    const std::vector<float>& confidence, std::uint32_t mask_id,
    std::vector<std::int32_t>* codes) {
  const std::size_t total = codebooks * frames;
  std::vector<float> noise(temperature > 0.0F ? total : 0);
  if (temperature > 0.0F)
    GumbelNoise(random, total, noise.data());
  std::vector<float> scores(total);
  for (std::size_t i = 0; i < total; ++i) {
    const float penalty = static_cast<float>(i / frames) * layer_penalty;
    float score = confidence[i] - penalty;
    if (temperature > 0.0F)
      score = score / temperature + noise[i];
    if ((*codes)[i] != static_cast<std::int32_t>(mask_id))
      score = -std::numeric_limits<float>::infinity();
    scores[i] = score;
  }
  count = std::min(count, total);
  std::vector<std::size_t> order(total);
  std::iota(order.begin(), order.end(), std::size_t{0});
  std::nth_element(order.begin(), order.begin() + static_cast<std::ptrdiff_t>(count),
                   order.end(), [&](std::size_t a, std::size_t b) {
                     return scores[a] != scores[b] ? scores[a] > scores[b] : a < b;
                   });
  order.resize(count);
  std::sort(order.begin(), order.end(), [&](std::size_t a, std::size_t b) {
    return scores[a] != scores[b] ? scores[a] > scores[b] : a < b;
  });
  for (const std::size_t i : order)
    (*codes)[i] = prediction[i];
  return order;
}

namespace {

std::uint64_t Mix(std::uint64_t x) {
  // SplitMix64 (Vigna): golden-ratio increment, two xor-shift-multiplies.
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

}  // namespace

// float -> binary16 bits, round to nearest even, subnormals and overflow
// included. Written out so that the float rounding of half(float(x)) is
// never folded into a single double -> half rounding by the compiler.
std::uint16_t HalfBits(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, sizeof(u));
  const std::uint16_t sign = static_cast<std::uint16_t>((u >> 16) & 0x8000U);
  const std::uint32_t a = u & 0x7FFFFFFFU;
  if (a >= 0x7F800000U)  // inf, nan
    return sign | (a > 0x7F800000U ? 0x7E00 : 0x7C00);
  if (a >= 0x477FF000U)  // >= 65520 rounds to infinity
    return sign | 0x7C00;
  if (a >= 0x38800000U) {  // normal binary16
    std::uint32_t h = (a >> 13) - (112U << 10);
    const std::uint32_t dropped = a & 0x1FFFU;
    h += (dropped > 0x1000U || (dropped == 0x1000U && (h & 1U))) ? 1U : 0U;
    return sign | static_cast<std::uint16_t>(h);
  }
  if (a < 0x33000000U)  // below half the smallest subnormal
    return sign;
  // Subnormal: the value is m * 2^(e - 150) with the implicit bit in m;
  // in units of 2^-24 that is m >> (126 - e).
  const std::uint32_t e = a >> 23;
  const std::uint32_t m = (a & 0x7FFFFFU) | 0x800000U;
  const std::uint32_t shift = 126 - e;
  std::uint32_t h = m >> shift;
  const std::uint32_t dropped = m & ((1U << shift) - 1U);
  const std::uint32_t tie = 1U << (shift - 1);
  h += (dropped > tie || (dropped == tie && (h & 1U))) ? 1U : 0U;
  return sign | static_cast<std::uint16_t>(h);
}

_Float16 ToHalf(float x) {
  const std::uint16_t bits = HalfBits(x);
  _Float16 h;
  std::memcpy(&h, &bits, sizeof(h));
  return h;
}

double SynthNormal(std::uint64_t seed, std::uint64_t tensor,
                   std::uint64_t element) {
  const std::uint64_t counter = Mix(seed ^ Mix(tensor)) + 2 * element;
  const double u1 = static_cast<double>((Mix(counter) >> 11) + 1) * 0x1.0p-53;
  const double u2 = static_cast<double>(Mix(counter + 1) >> 11) * 0x1.0p-53;
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

void ParallelChunks(std::size_t count,
                    const std::function<void(std::size_t, std::size_t)>& body) {
  const std::size_t workers = std::clamp<std::size_t>(
      std::thread::hardware_concurrency(), 1, 32);
  const std::size_t chunk = std::max<std::size_t>(
      (count + workers - 1) / workers, 4096);
  std::vector<std::thread> threads;
  for (std::size_t begin = 0; begin < count; begin += chunk) {
    const std::size_t end = std::min(count, begin + chunk);
    threads.emplace_back([&body, begin, end] { body(begin, end); });
  }
  for (std::thread& t : threads)
    t.join();
}

void SynthFloat(std::uint64_t seed, std::uint64_t tensor, std::uint64_t first,
                std::size_t count, bool norm, float jitter, float* out) {
  ParallelChunks(count, [&](std::size_t begin, std::size_t end) {
    for (std::size_t i = begin; i < end; ++i) {
      const std::uint64_t e = first + i;
      if (norm) {
        out[i] = jitter == 0.0F
                     ? 1.0F
                     : static_cast<float>(ToHalf(static_cast<float>(
                           1.0 + static_cast<double>(jitter) *
                                     SynthNormal(seed, tensor, e))));
      } else {
        out[i] = static_cast<float>(
            ToHalf(static_cast<float>(0.02 * SynthNormal(seed, tensor, e))));
      }
    }
  });
}

void SynthHalf(std::uint64_t seed, std::uint64_t tensor, std::uint64_t first,
               std::size_t count, _Float16* out) {
  ParallelChunks(count, [&](std::size_t begin, std::size_t end) {
    for (std::size_t i = begin; i < end; ++i)
      out[i] = ToHalf(static_cast<float>(0.02 * SynthNormal(seed, tensor, first + i)));
  });
}

}  // namespace ovg
