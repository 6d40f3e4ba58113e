// The generator through the reference-shaped C++ interface on a small seeded
// synthetic model: shapes of Forward / Score, the contract of Generate (every
// code unmasked, per-step counts equal to the schedule, the same seed
// reproduces the same codes), cancellation reporting exactly "cancelled",
// and failures reported as false plus a prefixed message, never an
// exception (reference tests/generator_test.cpp and synthesis_test.cpp:
// 79, 126-129 check the same properties on the real model).
#include <cmath>
#include <cstdint>
#include <iostream>
#include <string>
#include <vector>

#include "omnivoice/generator.hpp"

namespace ov = gufo::models::omnivoice;

namespace {

int failures = 0;

void Expect(bool condition, const std::string& what) {
  if (!condition) {
    std::cout << "FAIL " << what << '\n';
    ++failures;
  }
}

ov::Config SmallConfig() {
  ov::Config c;
  c.backbone.vocab_size = 97;
  c.backbone.hidden_size = 256;
  c.backbone.intermediate_size = 384;
  c.backbone.layers = 2;
  c.backbone.heads = 4;
  c.backbone.kv_heads = 2;
  c.backbone.head_dim = 128;
  c.backbone.max_positions = 4096;
  c.backbone.rms_norm_eps = 1e-6F;
  c.backbone.rope_theta = 1e6F;
  c.audio_codebooks = 8;
  c.audio_vocab_size = 1025;
  c.audio_mask_id = 1024;
  return c;
}

}  // namespace

int main() {
  const ov::Config config = SmallConfig();
  std::string error;
  auto generator = ov::Generator::LoadSynthetic(config, 7, &error);
  if (!generator) {
    std::cout << "FAIL load: " << error << '\n';
    return 1;
  }
  std::vector<std::uint32_t> text;
  for (std::uint32_t i = 0; i < 12; ++i)
    text.push_back((i * 31 + 5) % 97);
  const std::size_t frames = 40;
  const auto input =
      ov::ConditionalInput::Build(text, {}, 0, frames, 8, 1024);

  std::vector<float> logits;
  Expect(generator->Forward(input, &logits, &error), "forward: " + error);
  Expect(logits.size() == 2 * frames * 8 * 1025, "forward shape");
  bool finite = true;
  for (const float v : logits)
    finite = finite && std::isfinite(v);
  Expect(finite, "forward logits finite");

  std::vector<std::int32_t> prediction;
  std::vector<float> confidence;
  Expect(generator->Score(input, 2.0F, &prediction, &confidence, &error),
         "score: " + error);
  Expect(prediction.size() == 8 * frames && confidence.size() == 8 * frames,
         "score shape");
  bool valid = true;
  for (std::size_t i = 0; i < prediction.size(); ++i)
    valid = valid && prediction[i] >= 0 && prediction[i] < 1024 &&
            confidence[i] <= 0.0F;
  Expect(valid, "score: predictions exclude the mask, confidences are log-probabilities");

  ov::DecodingConfig decoding;
  ov::GenerationResult first, second;
  Expect(generator->Generate(input, decoding, 42, {}, &first, &error),
         "generate: " + error);
  Expect(generator->Generate(input, decoding, 42, {}, &second, &error),
         "generate again: " + error);
  Expect(first.codes == second.codes && first.unmasked_at == second.unmasked_at,
         "same seed, same codes");
  const auto schedule = ov::UnmaskSchedule(8 * frames, decoding.steps,
                                           decoding.t_shift);
  std::vector<std::size_t> per_step(decoding.steps, 0);
  bool unmasked = first.codes.size() == 8 * frames;
  for (std::size_t i = 0; i < first.codes.size(); ++i) {
    unmasked = unmasked && first.codes[i] >= 0 && first.codes[i] < 1024;
    const std::int32_t step = first.unmasked_at[i];
    if (step >= 0 && static_cast<std::size_t>(step) < per_step.size())
      ++per_step[static_cast<std::size_t>(step)];
    else
      unmasked = false;
  }
  Expect(unmasked, "every code unmasked at a valid step");
  Expect(per_step == schedule, "per-step counts follow the schedule");

  int polls = 0;
  ov::GenerationResult cancelled_result;
  const bool ran = generator->Generate(
      input, decoding, 42, [&polls] { return ++polls > 3; }, &cancelled_result,
      &error);
  Expect(!ran && error == "cancelled", "cancellation reports \"cancelled\"");

  ov::ConditionalInput broken = input;
  broken.ids.pop_back();
  Expect(!generator->Generate(broken, decoding, 1, {}, &first, &error) &&
             error.rfind("OmniVoice generation: ", 0) == 0,
         "malformed input is an error with the generation prefix");
  Expect(!ov::Generator::Load(config, "/nonexistent/checkpoint", &error) &&
             error.rfind("OmniVoice generator: ", 0) == 0,
         "a missing checkpoint is an error with the generator prefix");
  Expect(!ov::Generator::Load(config, "", &error) &&
             error.rfind("OmniVoice generator: cannot open model.safetensors", 0) == 0,
         "an empty model root is an open error, not a synthetic model");

  std::cout << (failures == 0 ? "ok" : "FAIL") << " generator: " << failures
            << " failures\n";
  return failures == 0 ? 0 : 1;
}
