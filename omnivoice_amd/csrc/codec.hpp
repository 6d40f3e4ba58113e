// Launchers of the audio decoder's gfx950 kernels (codec_kernels.hip).
// Signals are float32, channel-major: [channels][samples].
#ifndef OMNIVOICE_AMD_CODEC_HPP_
#define OMNIVOICE_AMD_CODEC_HPP_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ovg {

constexpr int kConvMaxTaps = 7;
constexpr int kConvMaxPhases = 8;
// Largest spread between a convolution's first and last tap (kernel 7 at
// dilation 9 spans 54 samples).
constexpr int kConvMaxSpan = 64;

// Activations a convolution's epilogue applies.
enum ConvAct : int {
  kActNone = 0,
  kActGelu = 1,   // 0.5 v (1 + erf(v / sqrt 2)), pre-activation only
  kActSnake = 2,  // v + sin^2(alpha v) / (alpha + 1e-9), output activation only
  kActElu = 3,    // v > 0 ? v : exp(v) - 1, output activation only
};

// One convolution as an implicit GEMM on the fp32 matrix cores:
//   v[o][t] = pre(bias[o] + sum_{k, i} w[phase][k][i][o] * act_in(x[i][m + offsets[phase][k]]))
//   y[o][t] = v (or y += v), y_act[o][t] = out_act(y[o][t]),  t = m out_stride + phase
// for output positions m < positions, with x = 0 outside [0, len_in), and
// act_in the Snake activation of the channel's alpha (the identity when
// alpha_in is null). A Conv1d is one phase with taps at k dilation - pad; a
// ConvTranspose1d of stride s is s phases of two taps each (see the codec
// engine). Either output may be null (y not with accumulate); bias may be
// null (zero). `batches` independent convolutions of the same shape run in
// one launch, the pointers of batch b advanced by b times their batch
// strides (a grouped convolution, or attention heads).
struct ConvParams {
  const float* x;         // [cin][len_in]
  const float* alpha_in;  // [cin] or null
  const float* w;         // [phases][taps][cin][ldw], ldw >= cout (0: cout)
  const float* bias;      // [cout] or null
  float* y;               // [cout][len_out] or null
  float* y_act;           // [cout][len_out] or null
  const float* alpha_out; // [cout], with a Snake output activation
  int cin, len_in, cout, len_out;
  int taps, phases, positions, out_stride;
  int accumulate;  // y += v instead of y = v
  int ldw;
  int pre_act;     // kActNone or kActGelu
  int out_act;     // for y_act: kActSnake (default when 0) or kActElu
  int batches;     // 0 or 1: one convolution
  std::int64_t x_batch, w_batch, b_batch, y_batch;  // element strides per batch
  int offsets[kConvMaxPhases][kConvMaxTaps];
  // Optional split-K workspace (float32 elements): when the output tiles
  // alone leave CUs idle, the launcher may split the input channels over
  // several work-groups, which store partial sums here; a second kernel
  // adds them in a fixed order and applies the epilogue. Null: never split.
  float* partial;
  std::int64_t partial_capacity;
  // Set by the launcher.
  int splits, split_chunks;
};
void LaunchConv(const ConvParams& p, hipStream_t stream);

// The decoder's last layer, one output channel: y[t] = bias + sum_{k, i}
// w[k][i] act(x[i][t + k - pad]), pad = (taps - 1) / 2, act the Snake of
// `alpha` or the identity when it is null.
struct OutputConvParams {
  const float* x;      // [cin][length]
  const float* alpha;  // [cin] or null
  const float* w;      // [taps][cin]
  const float* bias;   // [1]
  float* y;            // [length]
  int cin, length, taps;
};
void LaunchOutputConv(const OutputConvParams& p, hipStream_t stream);

// RVQ decode folded with fc2: y[o][f] = bias[o] + sum_c
// table[c][codes[c][f]][o], i.e. the latent input of the decoder, channel
// major.
struct RvqParams {
  const float* table;  // [codebooks][entries][latent]
  const float* bias;   // [latent]
  const std::int32_t* codes;  // [codebooks][frames]
  float* y;            // [latent][frames]
  int codebooks, entries, latent, frames;
};
void LaunchRvq(const RvqParams& p, hipStream_t stream);

}  // namespace ovg

#endif  // OMNIVOICE_AMD_CODEC_HPP_
