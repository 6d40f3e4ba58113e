// Host side of the unmasking loop with the reference's interface
// (gufo-extensions/omnivoice decoding.hpp:12-88): the schedule, the
// conditional input layout and the host position selector. The generator
// itself schedules and selects on the GPU; these stay for the callers and
// tests that use them directly (reference decoding_test.cpp).
#ifndef GUFO_MODELS_OMNIVOICE_MI355X_DECODING_HPP_
#define GUFO_MODELS_OMNIVOICE_MI355X_DECODING_HPP_

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

namespace gufo::models::omnivoice {

/// Decoding parameters (reference decoding.hpp:14-21).
struct DecodingConfig {
  std::size_t steps = 32;
  float guidance = 2.0F;
  float t_shift = 0.1F;
  float layer_penalty = 5.0F;
  /// Temperature of the Gumbel-perturbed position choice (0 = greedy).
  float position_temperature = 5.0F;
};

/// Codes unmasked at each step (reference decoding.cpp:12-40).
[[nodiscard]] std::vector<std::size_t> UnmaskSchedule(std::size_t total,
                                                      std::size_t steps,
                                                      float t_shift);

/// [text tokens | reference frames | target frames] as `codebooks` rows of
/// `length` ids (reference decoding.hpp:32-47).
struct ConditionalInput {
  std::size_t codebooks = 0;
  std::size_t length = 0;
  std::size_t audio_start = 0;
  std::size_t target_frames = 0;
  /// Row-major ids, one row of `length` per codebook.
  std::vector<std::int32_t> ids;

  /// Lays out text ids, the reference codes (one row of `reference_frames`
  /// per codebook) and masked target frames (reference decoding.cpp:42-62).
  [[nodiscard]] static ConditionalInput Build(
      const std::vector<std::uint32_t>& text_ids,
      const std::vector<std::int32_t>& reference_codes,
      std::size_t reference_frames, std::size_t target_frames,
      std::size_t codebooks, std::uint32_t mask_id);
};

struct GenerationResult {
  /// Final codes, one row of target frames per codebook.
  std::vector<std::int32_t> codes;
  /// Per code, the index of the step at which it was chosen (same layout).
  std::vector<std::int32_t> unmasked_at;
};

/// Host position choice of one step (reference decoding.cpp:64-107).
class PositionSelector {
 public:
  PositionSelector(const DecodingConfig& config, std::uint64_t seed);

  /// Fills the `count` best masked entries of `codes` with their
  /// predictions (all three arrays hold one row of frames per codebook) and
  /// returns their flat indices in rank order.
  std::vector<std::size_t> Fill(std::size_t count, std::size_t codebooks,
                                std::size_t frames,
                                const std::vector<std::int32_t>& prediction,
                                const std::vector<float>& confidence,
                                std::uint32_t mask_id,
                                std::vector<std::int32_t>* codes);

 private:
  float layer_penalty_;
  float temperature_;
  std::mt19937_64 random_;
};

}  // namespace gufo::models::omnivoice

#endif  // GUFO_MODELS_OMNIVOICE_MI355X_DECODING_HPP_
