// The reference-shaped C++ surface (include/omnivoice/generator.hpp and
// decoding.hpp) over the C ABI: Generator forwards to ovg_* and turns their
// status codes into bool + message, the way the reference's methods report
// failures (generator.cpp:430, 450, 480, 539: no exception escapes).
#include <exception>
#include <string>
#include <utility>
#include <vector>

#include "../../include/omnivoice/generator.hpp"
#include "../../include/omnivoice_mi355x.h"
#include "host.hpp"

namespace gufo::models::omnivoice {
namespace {

constexpr std::size_t kMessage = 1024;

ovg_config ToC(const Config& c) {
  ovg_config out{};
  out.vocab_size = static_cast<std::int64_t>(c.backbone.vocab_size);
  out.hidden_size = static_cast<std::int64_t>(c.backbone.hidden_size);
  out.intermediate_size = static_cast<std::int64_t>(c.backbone.intermediate_size);
  out.layers = static_cast<std::int64_t>(c.backbone.layers);
  out.heads = static_cast<std::int64_t>(c.backbone.heads);
  out.kv_heads = static_cast<std::int64_t>(c.backbone.kv_heads);
  out.head_dim = static_cast<std::int64_t>(c.backbone.head_dim);
  out.max_positions = static_cast<std::int64_t>(c.backbone.max_positions);
  out.rms_norm_eps = c.backbone.rms_norm_eps;
  out.rope_theta = c.backbone.rope_theta;
  out.audio_codebooks = static_cast<std::int64_t>(c.audio_codebooks);
  out.audio_vocab_size = static_cast<std::int64_t>(c.audio_vocab_size);
  out.audio_mask_id = c.audio_mask_id;
  return out;
}

ovg_input ToC(const ConditionalInput& in) {
  ovg_input out{};
  out.codebooks = static_cast<std::int64_t>(in.codebooks);
  out.length = static_cast<std::int64_t>(in.length);
  out.audio_start = static_cast<std::int64_t>(in.audio_start);
  out.target_frames = static_cast<std::int64_t>(in.target_frames);
  out.ids = in.ids.data();
  return out;
}

// A malformed ConditionalInput is reported before any pointer reaches the
// library (its ids must hold codebooks x length entries).
bool CheckInput(const ConditionalInput& in, const char* prefix,
                std::string* error) {
  if (in.ids.size() == in.codebooks * in.length)
    return true;
  if (error != nullptr)
    *error = std::string(prefix) + "ids hold " + std::to_string(in.ids.size()) +
             " entries, not codebooks x length = " +
             std::to_string(in.codebooks * in.length);
  return false;
}

bool Report(int status, const char* message, std::string* error) {
  if (status == OVG_OK)
    return true;
  if (error != nullptr)
    *error = message;
  return false;
}

int PollCancelled(void* user) {
  const auto* cancelled = static_cast<const std::function<bool()>*>(user);
  return (*cancelled)() ? 1 : 0;
}

}  // namespace

struct Generator::State {
  ovg_handle* handle = nullptr;
  std::size_t codebooks = 0;
  std::size_t vocab = 0;
  ~State() { ovg_destroy(handle); }
};

Generator::Generator(std::unique_ptr<State> state) : state_(std::move(state)) {}
Generator::~Generator() = default;

std::unique_ptr<Generator> Generator::Load(const Config& config,
                                           const std::filesystem::path& model_root,
                                           std::string* error) {
  // model_root / "model.safetensors" (an empty root names the working
  // directory, as in the reference); synthetic weights only through
  // LoadSynthetic.
  const ovg_config c = ToC(config);
  char message[kMessage] = {};
  auto state = std::make_unique<State>();
  const std::string root = model_root.string();
  if (!Report(ovg_create(&c, root.c_str(), 0, &state->handle, message, kMessage),
              message, error))
    return nullptr;
  state->codebooks = config.audio_codebooks;
  state->vocab = config.audio_vocab_size;
  return std::unique_ptr<Generator>(new Generator(std::move(state)));
}

std::unique_ptr<Generator> Generator::LoadSynthetic(const Config& config,
                                                    std::uint64_t weight_seed,
                                                    std::string* error) {
  const ovg_config c = ToC(config);
  char message[kMessage] = {};
  auto state = std::make_unique<State>();
  if (!Report(ovg_create_synthetic(&c, weight_seed, 0.0F, &state->handle, message,
                                   kMessage),
              message, error))
    return nullptr;
  state->codebooks = config.audio_codebooks;
  state->vocab = config.audio_vocab_size;
  return std::unique_ptr<Generator>(new Generator(std::move(state)));
}

bool Generator::Generate(const ConditionalInput& input,
                         const DecodingConfig& decoding, std::uint64_t seed,
                         const std::function<bool()>& cancelled,
                         GenerationResult* result, std::string* error) {
  if (!CheckInput(input, "OmniVoice generation: ", error))
    return false;
  const std::size_t n = input.codebooks * input.target_frames;
  std::vector<std::int32_t> codes(n), unmasked_at(n);
  const ovg_input in = ToC(input);
  ovg_decoding d{};
  d.steps = static_cast<std::int64_t>(decoding.steps);
  d.guidance = decoding.guidance;
  d.t_shift = decoding.t_shift;
  d.layer_penalty = decoding.layer_penalty;
  d.position_temperature = decoding.position_temperature;
  char message[kMessage] = {};
  const bool poll = static_cast<bool>(cancelled);
  const int status = ovg_generate(
      state_->handle, &in, &d, seed, poll ? PollCancelled : nullptr,
      poll ? const_cast<std::function<bool()>*>(&cancelled) : nullptr,
      codes.data(), unmasked_at.data(), message, kMessage);
  if (!Report(status, message, error))
    return false;
  result->codes = std::move(codes);
  result->unmasked_at = std::move(unmasked_at);
  return true;
}

bool Generator::Forward(const ConditionalInput& input,
                        std::vector<float>* logits, std::string* error) {
  if (!CheckInput(input, "OmniVoice forward: ", error))
    return false;
  std::vector<float> out(2 * input.target_frames * state_->codebooks *
                         state_->vocab);
  const ovg_input in = ToC(input);
  char message[kMessage] = {};
  if (!Report(ovg_forward(state_->handle, &in, out.data(), message, kMessage),
              message, error))
    return false;
  *logits = std::move(out);
  return true;
}

bool Generator::Score(const ConditionalInput& input, float guidance,
                      std::vector<std::int32_t>* prediction,
                      std::vector<float>* confidence, std::string* error) {
  if (!CheckInput(input, "OmniVoice score: ", error))
    return false;
  const std::size_t n = input.codebooks * input.target_frames;
  std::vector<std::int32_t> pred(n);
  std::vector<float> conf(n);
  const ovg_input in = ToC(input);
  char message[kMessage] = {};
  if (!Report(ovg_score(state_->handle, &in, guidance, pred.data(), conf.data(),
                        message, kMessage),
              message, error))
    return false;
  *prediction = std::move(pred);
  *confidence = std::move(conf);
  return true;
}

std::vector<std::size_t> UnmaskSchedule(std::size_t total, std::size_t steps,
                                        float t_shift) {
  return ovg::UnmaskSchedule(total, steps, t_shift);
}

ConditionalInput ConditionalInput::Build(
    const std::vector<std::uint32_t>& text_ids,
    const std::vector<std::int32_t>& reference_codes,
    std::size_t reference_frames, std::size_t target_frames,
    std::size_t codebooks, std::uint32_t mask_id) {
  ConditionalInput input;
  input.codebooks = codebooks;
  input.audio_start = text_ids.size();
  input.target_frames = target_frames;
  input.length = text_ids.size() + reference_frames + target_frames;
  input.ids = ovg::BuildInput(text_ids, reference_codes, reference_frames,
                              target_frames, codebooks, mask_id);
  return input;
}

PositionSelector::PositionSelector(const DecodingConfig& config,
                                   std::uint64_t seed)
    : layer_penalty_(config.layer_penalty),
      temperature_(config.position_temperature),
      random_(seed) {}

std::vector<std::size_t> PositionSelector::Fill(
    std::size_t count, std::size_t codebooks, std::size_t frames,
    const std::vector<std::int32_t>& prediction,
    const std::vector<float>& confidence, std::uint32_t mask_id,
    std::vector<std::int32_t>* codes) {
  return ovg::SelectPositions(&random_, layer_penalty_, temperature_, count,
                              codebooks, frames, prediction, confidence,
                              mask_id, codes);
}

}  // namespace gufo::models::omnivoice
