// The generator with the reference's interface (gufo-extensions/omnivoice
// generator.hpp:14-56), running the whole unmasking loop on one MI355X. A
// thin layer over the C ABI of omnivoice_mi355x.h, built into the same
// library. Not thread-safe; one instance per thread.
#ifndef GUFO_MODELS_OMNIVOICE_MI355X_GENERATOR_HPP_
#define GUFO_MODELS_OMNIVOICE_MI355X_GENERATOR_HPP_

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "config.hpp"
#include "decoding.hpp"

namespace gufo::models::omnivoice {

class Generator {
 public:
  /// Reference generator.hpp:22-24: reads model_root/model.safetensors (the
  /// checkpoint's float32 tensors). An empty `model_root` names
  /// model.safetensors in the working directory and fails, as the
  /// reference's Load does, when it is absent; synthetic weights come only
  /// from LoadSynthetic.
  [[nodiscard]] static std::unique_ptr<Generator> Load(
      const Config& config, const std::filesystem::path& model_root,
      std::string* error = nullptr);
  /// The synthetic model from a chosen weight seed (no reference
  /// counterpart: the stand-in for a checkpoint in tests and benchmarks).
  [[nodiscard]] static std::unique_ptr<Generator> LoadSynthetic(
      const Config& config, std::uint64_t weight_seed,
      std::string* error = nullptr);
  ~Generator();
  Generator(const Generator&) = delete;
  Generator& operator=(const Generator&) = delete;

  /// Reference generator.hpp:29-36: the unmasking loop from `input`'s
  /// masked target; `cancelled` (may be empty) is polled before every step.
  [[nodiscard]] bool Generate(const ConditionalInput& input,
                              const DecodingConfig& decoding,
                              std::uint64_t seed,
                              const std::function<bool()>& cancelled,
                              GenerationResult* result,
                              std::string* error = nullptr);

  /// Reference generator.hpp:38-43: logits [2 * frames][codebooks * vocab],
  /// conditional target rows then unconditional.
  [[nodiscard]] bool Forward(const ConditionalInput& input,
                             std::vector<float>* logits,
                             std::string* error = nullptr);

  /// Reference generator.hpp:45-50: per [codebook][frame] the guided argmax
  /// and its log-probability.
  [[nodiscard]] bool Score(const ConditionalInput& input, float guidance,
                           std::vector<std::int32_t>* prediction,
                           std::vector<float>* confidence,
                           std::string* error = nullptr);

 private:
  struct State;
  explicit Generator(std::unique_ptr<State> state);
  std::unique_ptr<State> state_;
};

}  // namespace gufo::models::omnivoice

#endif  // GUFO_MODELS_OMNIVOICE_MI355X_GENERATOR_HPP_
