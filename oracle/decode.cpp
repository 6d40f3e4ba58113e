// ORACLE — test infrastructure, not product code (see oracle.h).
//
// Host decoding and CFG scoring restated on the CPU:
//   UnmaskSchedule            decoding.cpp:12-40
//   ConditionalInput::Build   decoding.cpp:42-62
//   PositionSelector          decoding.cpp:64-107
//   kernels::Score            kernels/generator_kernels.hip:212-265
//
// Built with -ffp-contract=off: every fused multiply-add below is an
// explicit fmaf, so the arithmetic is the exact sequence the GPU score
// kernel executes. The score's reductions follow one 64-lane wavefront per
// (frame, codebook): lane l owns entries l, l+64, ... and sums them in
// that order, then lanes combine by xor butterfly over offsets 32..1.
// That order is the GPU kernel's design; the reference uses another order
// (256-thread blocks), which only changes the last bits of the sums.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <vector>

#include "oracle.h"

namespace {

inline std::uint32_t Bits(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, 4);
  return u;
}
inline float FromBits(std::uint32_t u) {
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

// exp by Cody-Waite range reduction, x = n ln2 + r with ln2 split into a
// 9-bit head (0.693359375 = 355/512, so n * head is exact) and its
// remainder, then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
// (truncation below 0.1 ulp) evaluated by Horner with fmaf.
constexpr float kLog2e = 1.44269504088896341F;
constexpr float kLn2Head = 0.693359375F;
constexpr float kLn2Tail = -2.12194440054690583e-4F;

float Exp(float x) {
  if (x != x)
    return x;
  if (x < -87.0F)
    return 0.0F;  // results stay normal floats
  if (x > 88.0F)
    return std::numeric_limits<float>::infinity();
  const float n = std::rint(x * kLog2e);
  float r = std::fmaf(n, -kLn2Head, x);
  r = std::fmaf(n, -kLn2Tail, r);
  float p = 1.0F / 5040.0F;
  p = std::fmaf(p, r, 1.0F / 720.0F);
  p = std::fmaf(p, r, 1.0F / 120.0F);
  p = std::fmaf(p, r, 1.0F / 24.0F);
  p = std::fmaf(p, r, 1.0F / 6.0F);
  p = std::fmaf(p, r, 0.5F);
  p = std::fmaf(p, r, 1.0F);
  p = std::fmaf(p, r, 1.0F);
  const int e = static_cast<int>(n);
  const float scale = FromBits(static_cast<std::uint32_t>(e + 127) << 23);
  return p * scale;
}

// log by exponent split x = 2^e m, m in (sqrt(1/2), sqrt(2)], and
// log m = 2 atanh(s) with s = (m - 1) / (m + 1), |s| <= 0.1716, summed
// through s^13 (the next term is below 1e-10 relative).
float Log(float x) {
  if (x != x)
    return x;
  if (x < 0.0F)
    return std::numeric_limits<float>::quiet_NaN();
  if (x == 0.0F)
    return -std::numeric_limits<float>::infinity();
  if (x == std::numeric_limits<float>::infinity())
    return x;
  int e = 0;
  std::uint32_t u = Bits(x);
  if (u < 0x00800000U) {  // subnormal: scale by 2^23
    x = x * 8388608.0F;
    u = Bits(x);
    e = -23;
  }
  e += static_cast<int>(u >> 23) - 127;
  float m = FromBits((u & 0x007FFFFFU) | 0x3F800000U);
  if (m > 1.41421356F) {
    m = m * 0.5F;
    e += 1;
  }
  const float f = m - 1.0F;
  const float s = f / (m + 1.0F);
  const float z = s * s;
  float p = std::fmaf(z, 2.0F / 13.0F, 2.0F / 11.0F);
  p = std::fmaf(p, z, 2.0F / 9.0F);
  p = std::fmaf(p, z, 2.0F / 7.0F);
  p = std::fmaf(p, z, 2.0F / 5.0F);
  p = std::fmaf(p, z, 2.0F / 3.0F);
  const float sz = s * z;
  const float lm = std::fmaf(sz, p, s + s);
  const float fe = static_cast<float>(e);
  return std::fmaf(fe, kLn2Head, std::fmaf(fe, kLn2Tail, lm));
}

constexpr int kLanes = 64;

// In-place xor-butterfly sum over 64 lanes, offsets 32, 16, ..., 1.
float ButterflySum(float lane[kLanes]) {
  for (int offset = kLanes / 2; offset > 0; offset /= 2) {
    float next[kLanes];
    for (int l = 0; l < kLanes; ++l)
      next[l] = lane[l] + lane[l ^ offset];
    std::memcpy(lane, next, sizeof(next));
  }
  return lane[0];
}

float ButterflyMax(const float lane[kLanes]) {
  float best = lane[0];
  for (int l = 1; l < kLanes; ++l)
    best = std::fmax(best, lane[l]);
  return best;
}

struct Selector {
  float layer_penalty;
  float temperature;
  std::mt19937_64 random;
};

}  // namespace

extern "C" {

float orc_exp(float x) { return Exp(x); }
float orc_log(float x) { return Log(x); }

// decoding.cpp:12-40: float32 linspace emulation (first half counts up from
// 0, second half down from 1), the shift t' = s t / (1 + (s - 1) t), and
// per-step counts ceil(total * (t'[i+1] - t'[i])) computed in double.
void orc_unmask_schedule(int64_t total, int64_t steps, float t_shift,
                         int64_t* schedule) {
  std::vector<float> t(static_cast<std::size_t>(steps) + 1);
  const float step = 1.0F / static_cast<float>(steps);
  const int64_t half = (steps + 1) / 2;
  for (int64_t i = 0; i <= steps; ++i) {
    float v = i < half ? step * static_cast<float>(i)
                       : 1.0F - step * static_cast<float>(steps - i);
    v = t_shift * v / (1.0F + (t_shift - 1.0F) * v);
    t[static_cast<std::size_t>(i)] = v;
  }
  int64_t left = total;
  for (int64_t i = 0; i < steps; ++i) {
    int64_t count = left;
    if (i + 1 < steps) {
      const double delta = static_cast<double>(t[i + 1]) -
                           static_cast<double>(t[i]);
      const auto want = static_cast<int64_t>(
          std::ceil(static_cast<double>(total) * delta));
      count = std::min(want, left);
    }
    schedule[i] = count;
    left -= count;
  }
}

// decoding.cpp:42-62.
int64_t orc_build_input(const uint32_t* text_ids, int64_t text_count,
                        const int32_t* reference_codes,
                        int64_t reference_frames, int64_t target_frames,
                        int64_t codebooks, uint32_t mask_id, int32_t* ids) {
  const int64_t length = text_count + reference_frames + target_frames;
  for (int64_t c = 0; c < codebooks; ++c) {
    int32_t* row = ids + c * length;
    for (int64_t p = 0; p < length; ++p)
      row[p] = static_cast<int32_t>(mask_id);
    for (int64_t t = 0; t < text_count; ++t)
      row[t] = static_cast<int32_t>(text_ids[t]);
    for (int64_t f = 0; f < reference_frames; ++f)
      row[text_count + f] = reference_codes[c * reference_frames + f];
  }
  return length;
}

// kernels/generator_kernels.hip:212-265: per (frame, codebook)
// c = x_c - lse(x_c), u = x_u - lse(x_u), g = c + w (c - u) (one fused
// multiply-add, as the reference kernel compiles), prediction = argmax of g
// over j != mask (lowest index on ties), confidence = g[pred] - lse(g).
void orc_score(const float* logits, int64_t frames, int64_t codebooks,
               int64_t vocab, uint32_t mask_id, float guidance,
               int32_t* prediction, float* confidence) {
  const int64_t width = codebooks * vocab;
  for (int64_t f = 0; f < frames; ++f) {
    for (int64_t c = 0; c < codebooks; ++c) {
      const float* cr = logits + f * width + c * vocab;
      const float* ur = logits + (frames + f) * width + c * vocab;
      float cm[kLanes], um[kLanes];
      for (int l = 0; l < kLanes; ++l) {
        cm[l] = -FLT_MAX;
        um[l] = -FLT_MAX;
        for (int64_t j = l; j < vocab; j += kLanes) {
          cm[l] = std::fmax(cm[l], cr[j]);
          um[l] = std::fmax(um[l], ur[j]);
        }
      }
      const float c_max = ButterflyMax(cm);
      const float u_max = ButterflyMax(um);
      float cs[kLanes], us[kLanes];
      for (int l = 0; l < kLanes; ++l) {
        cs[l] = 0.0F;
        us[l] = 0.0F;
        for (int64_t j = l; j < vocab; j += kLanes) {
          cs[l] = cs[l] + Exp(cr[j] - c_max);
          us[l] = us[l] + Exp(ur[j] - u_max);
        }
      }
      const float c_lse = c_max + Log(ButterflySum(cs));
      const float u_lse = u_max + Log(ButterflySum(us));
      auto guided = [&](int64_t j) {
        const float cv = cr[j] - c_lse;
        const float uv = ur[j] - u_lse;
        return std::fmaf(guidance, cv - uv, cv);
      };
      float gm[kLanes];
      for (int l = 0; l < kLanes; ++l) {
        gm[l] = -FLT_MAX;
        for (int64_t j = l; j < vocab; j += kLanes)
          gm[l] = std::fmax(gm[l], guided(j));
      }
      const float g_max = ButterflyMax(gm);
      float gs[kLanes];
      float best = -FLT_MAX;
      int64_t best_index = vocab;
      for (int l = 0; l < kLanes; ++l) {
        gs[l] = 0.0F;
        for (int64_t j = l; j < vocab; j += kLanes) {
          const float g = guided(j);
          gs[l] = gs[l] + Exp(g - g_max);
          if (j != static_cast<int64_t>(mask_id) &&
              (g > best || (g == best && j < best_index))) {
            best = g;
            best_index = j;
          }
        }
      }
      const float g_lse = g_max + Log(ButterflySum(gs));
      prediction[c * frames + f] = static_cast<int32_t>(best_index);
      confidence[c * frames + f] = best - g_lse;
    }
  }
}

void* orc_selector_create(float layer_penalty, float temperature,
                          uint64_t seed) {
  return new Selector{layer_penalty, temperature, std::mt19937_64(seed)};
}

void orc_selector_destroy(void* selector) {
  delete static_cast<Selector*>(selector);
}

// decoding.cpp:70-107.
int64_t orc_selector_fill(void* handle, int64_t count, int64_t codebooks,
                          int64_t frames, const int32_t* prediction,
                          const float* confidence, uint32_t mask_id,
                          int32_t* codes, int64_t* chosen) {
  Selector& s = *static_cast<Selector*>(handle);
  const int64_t total = codebooks * frames;
  std::vector<float> scores(static_cast<std::size_t>(total));
  for (int64_t c = 0; c < codebooks; ++c) {
    const float penalty = static_cast<float>(c) * s.layer_penalty;
    for (int64_t f = 0; f < frames; ++f) {
      const int64_t i = c * frames + f;
      float score = confidence[i] - penalty;
      if (s.temperature > 0.0F) {
        const float uniform =
            static_cast<float>(s.random() >> 40) * 0x1.0p-24F;
        const float gumbel =
            -std::log(-std::log(uniform + 1e-10F) + 1e-10F);
        score = score / s.temperature + gumbel;
      }
      if (codes[i] != static_cast<int32_t>(mask_id))
        score = -std::numeric_limits<float>::infinity();
      scores[static_cast<std::size_t>(i)] = score;
    }
  }
  count = std::min(count, total);
  std::vector<int64_t> order(static_cast<std::size_t>(total));
  std::iota(order.begin(), order.end(), int64_t{0});
  // A full sort by (score desc, index asc): its first `count` entries are
  // the partial_sort's.
  std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
    if (scores[a] != scores[b])
      return scores[a] > scores[b];
    return a < b;
  });
  for (int64_t r = 0; r < count; ++r) {
    const int64_t i = order[static_cast<std::size_t>(r)];
    codes[i] = prediction[i];
    if (chosen != nullptr)
      chosen[r] = i;
  }
  return count;
}

void orc_selector_noise(void* handle, int64_t total, float* noise) {
  Selector& s = *static_cast<Selector*>(handle);
  for (int64_t i = 0; i < total; ++i) {
    const float uniform = static_cast<float>(s.random() >> 40) * 0x1.0p-24F;
    noise[i] = -std::log(-std::log(uniform + 1e-10F) + 1e-10F);
  }
}

uint64_t orc_mt19937_64_nth(uint64_t seed, int64_t n) {
  std::mt19937_64 random(seed);
  uint64_t value = 0;
  for (int64_t i = 0; i < n; ++i)
    value = random();
  return value;
}

// generator.cpp:486-543 with the forward replaced by given logits.
int64_t orc_generate_from_logits(const float* logits_trace, int64_t executed,
                                 int64_t codebooks, int64_t frames,
                                 int64_t vocab, uint32_t mask_id,
                                 int64_t steps, float guidance, float t_shift,
                                 float layer_penalty, float temperature,
                                 uint64_t seed, int32_t* codes,
                                 int32_t* unmasked_at) {
  const int64_t total = codebooks * frames;
  std::vector<int64_t> schedule(static_cast<std::size_t>(steps));
  orc_unmask_schedule(total, steps, t_shift, schedule.data());
  for (int64_t i = 0; i < total; ++i) {
    codes[i] = static_cast<int32_t>(mask_id);
    unmasked_at[i] = -1;
  }
  Selector selector{layer_penalty, temperature, std::mt19937_64(seed)};
  std::vector<int32_t> prediction(static_cast<std::size_t>(total));
  std::vector<float> confidence(static_cast<std::size_t>(total));
  std::vector<int64_t> chosen(static_cast<std::size_t>(total));
  const int64_t step_logits = 2 * frames * codebooks * vocab;
  int64_t e = 0;
  for (int64_t step = 0; step < steps; ++step) {
    if (schedule[step] == 0)
      continue;
    if (e >= executed)
      return -1;
    orc_score(logits_trace + e * step_logits, frames, codebooks, vocab,
              mask_id, guidance, prediction.data(), confidence.data());
    const int64_t n = orc_selector_fill(
        &selector, schedule[step], codebooks, frames, prediction.data(),
        confidence.data(), mask_id, codes, chosen.data());
    for (int64_t r = 0; r < n; ++r)
      unmasked_at[chosen[r]] = static_cast<int32_t>(step);
    ++e;
  }
  return e;
}

}  // extern "C"
