// ORACLE — test infrastructure, not product code.
//
// extern "C" entry points over the reference's own decoding.cpp, compiled
// from /root/reference by oracle/Makefile into oracle/_ref/. The reference
// source is not copied: this file only calls UnmaskSchedule,
// ConditionalInput::Build and PositionSelector (decoding.hpp:23-77).
#include <cstdint>
#include <vector>

#include "decoding.hpp"

namespace ov = gufo::models::omnivoice;

extern "C" {

void ref_unmask_schedule(int64_t total, int64_t steps, float t_shift,
                         int64_t* out) {
  const std::vector<std::size_t> s = ov::UnmaskSchedule(
      static_cast<std::size_t>(total), static_cast<std::size_t>(steps),
      t_shift);
  for (std::size_t i = 0; i < s.size(); ++i)
    out[i] = static_cast<int64_t>(s[i]);
}

int64_t ref_build_input(const uint32_t* text_ids, int64_t text_count,
                        const int32_t* reference_codes,
                        int64_t reference_frames, int64_t target_frames,
                        int64_t codebooks, uint32_t mask_id, int32_t* ids) {
  std::vector<std::uint32_t> text(text_ids, text_ids + text_count);
  std::vector<std::int32_t> reference;
  if (reference_frames > 0)
    reference.assign(reference_codes,
                     reference_codes + codebooks * reference_frames);
  const ov::ConditionalInput input = ov::ConditionalInput::Build(
      text, reference, static_cast<std::size_t>(reference_frames),
      static_cast<std::size_t>(target_frames),
      static_cast<std::size_t>(codebooks), mask_id);
  for (std::size_t i = 0; i < input.ids.size(); ++i)
    ids[i] = input.ids[i];
  return static_cast<int64_t>(input.length);
}

void* ref_selector_create(float layer_penalty, float temperature,
                          uint64_t seed) {
  ov::DecodingConfig config;
  config.layer_penalty = layer_penalty;
  config.position_temperature = temperature;
  return new ov::PositionSelector(config, seed);
}

void ref_selector_destroy(void* selector) {
  delete static_cast<ov::PositionSelector*>(selector);
}

int64_t ref_selector_fill(void* selector, int64_t count, int64_t codebooks,
                          int64_t frames, const int32_t* prediction,
                          const float* confidence, uint32_t mask_id,
                          int32_t* codes, int64_t* chosen) {
  const std::size_t total = static_cast<std::size_t>(codebooks * frames);
  std::vector<std::int32_t> pred(prediction, prediction + total);
  std::vector<float> conf(confidence, confidence + total);
  std::vector<std::int32_t> current(codes, codes + total);
  const std::vector<std::size_t> order =
      static_cast<ov::PositionSelector*>(selector)->Fill(
          static_cast<std::size_t>(count), static_cast<std::size_t>(codebooks),
          static_cast<std::size_t>(frames), pred, conf, mask_id, &current);
  for (std::size_t i = 0; i < total; ++i)
    codes[i] = current[i];
  for (std::size_t r = 0; r < order.size(); ++r)
    chosen[r] = static_cast<int64_t>(order[r]);
  return static_cast<int64_t>(order.size());
}

}  // extern "C"
