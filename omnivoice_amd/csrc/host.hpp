// Host-side pieces of the generator: the unmasking schedule, the
// conditional-input layout, the Gumbel noise stream of the position
// selector, and the seeded synthetic model.
#ifndef OMNIVOICE_AMD_HOST_HPP_
#define OMNIVOICE_AMD_HOST_HPP_

#include <cstddef>
#include <cstdint>
#include <functional>
#include <random>
#include <vector>

namespace ovg {

// UnmaskSchedule (reference decoding.cpp:12-40).
std::vector<std::size_t> UnmaskSchedule(std::size_t total, std::size_t steps,
                                        float t_shift);

// ConditionalInput::Build (reference decoding.cpp:42-62): ids
// [codebooks][text + reference + target].
std::vector<std::int32_t> BuildInput(const std::vector<std::uint32_t>& text,
                                     const std::vector<std::int32_t>& reference,
                                     std::size_t reference_frames,
                                     std::size_t target_frames,
                                     std::size_t codebooks,
                                     std::uint32_t mask_id);

// The Gumbel term PositionSelector::Fill adds to each entry when the
// position temperature is positive (reference decoding.cpp:83-86): one
// std::mt19937_64 draw per entry, codebook-major, every executed step.
void GumbelNoise(std::mt19937_64* random, std::size_t count, float* out);

// PositionSelector::Fill on the host (reference decoding.cpp:70-107): kept
// for the decoding.hpp surface; the generator selects on the GPU.
std::vector<std::size_t> SelectPositions(
    std::mt19937_64* random, float layer_penalty, float temperature,
    std::size_t count, std::size_t codebooks, std::size_t frames,
    const std::vector<std::int32_t>& prediction,
    const std::vector<float>& confidence, std::uint32_t mask_id,
    std::vector<std::int32_t>* codes);

// Seeded synthetic model. Tensor ids: text embeddings 1, audio embeddings
// 2, audio heads 3, final norm 4, layer l tensor k (OVG_LAYER_* order)
// 100 + 16 l + k. Element e of a tensor is row * columns + column.
constexpr std::uint64_t kTextTensor = 1;
constexpr std::uint64_t kAudioEmbeddingTensor = 2;
constexpr std::uint64_t kAudioHeadTensor = 3;
constexpr std::uint64_t kFinalNormTensor = 4;
inline std::uint64_t LayerTensor(std::int64_t layer, int kind) {
  return 100 + 16 * static_cast<std::uint64_t>(layer) +
         static_cast<std::uint64_t>(kind);
}

// N(0, 1) of (seed, tensor, element): SplitMix64 counters, Box-Muller.
double SynthNormal(std::uint64_t seed, std::uint64_t tensor,
                   std::uint64_t element);

// Values of elements [first, first + count): matrices and embeddings
// half(float(0.02 * normal)); norms 1.0 or half(float(1 + jitter * normal)).
// Multi-threaded.
void SynthFloat(std::uint64_t seed, std::uint64_t tensor, std::uint64_t first,
                std::size_t count, bool norm, float jitter, float* out);
void SynthHalf(std::uint64_t seed, std::uint64_t tensor, std::uint64_t first,
               std::size_t count, _Float16* out);

// float -> fp16 with round-to-nearest-even (subnormals included).
std::uint16_t HalfBits(float x);
_Float16 ToHalf(float x);

// Parallel for over [0, count) in contiguous chunks.
void ParallelChunks(std::size_t count,
                    const std::function<void(std::size_t, std::size_t)>& body);

}  // namespace ovg

#endif  // OMNIVOICE_AMD_HOST_HPP_
