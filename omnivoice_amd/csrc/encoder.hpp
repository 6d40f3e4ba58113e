// Launchers of the audio encoder's gfx950 kernels (encoder_kernels.hip).
// Signals are float32 and channel-major ([channels][positions]); every GEMM
// of the encoder runs through LaunchConv (codec.hpp).
#ifndef OMNIVOICE_AMD_ENCODER_HPP_
#define OMNIVOICE_AMD_ENCODER_HPP_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ovg {

// The polyphase resampler applied to device samples, written into a buffer
// with `pad` zeros on each side: y[pad + j] = sum_k bank[j % to][k]
// x[(j / to) from - width + k] over the taps inside the signal (summed in
// double), j < out_length; y has out_length + 2 pad elements.
struct ResampleParams {
  const float* x;     // [length]
  const float* bank;  // [to][taps]
  float* y;
  int length, from, to, width, taps, out_length, pad;
};
void LaunchResample(const ResampleParams& p, hipStream_t stream);

// Columns of a strided, dilated, padded convolution:
// y[c kernel + j][t] = act(x[c][t stride + j dilation - pad]), zero outside
// [0, len_in); act the identity or ELU (kActElu).
struct Im2colParams {
  const float* x;  // [channels][len_in]
  float* y;        // [channels * kernel][positions]
  int channels, len_in, kernel, stride, dilation, pad, positions, act;
};
void LaunchIm2col(const Im2colParams& p, hipStream_t stream);

// GroupNorm with one group per channel (statistics over the row), affine,
// then GELU, in place: x [channels][length].
void LaunchGroupNormGelu(float* x, const float* w, const float* b, int channels, int length,
                         float eps, hipStream_t stream);

// LayerNorm over the channels of every position: y[c][t] = (x[c][t] -
// mean_t) / sqrt(var_t + eps) w[c] + b[c] (y may be x). sum_mode 1 sets,
// 2 adds y into `sum` (double, the running sum of encoder states).
struct ColumnNormParams {
  const float* x;
  float* y;
  const float* w;
  const float* b;
  double* sum;
  int channels, positions, sum_mode;
  float eps;
};
void LaunchColumnNorm(const ColumnNormParams& p, hipStream_t stream);

// Softmax over the rows of every column of `batches` [rows][cols]
// matrices, of scale x, in place.
void LaunchColumnSoftmax(float* x, int batches, int rows, int cols, float scale,
                         hipStream_t stream);

// y[c][r] = x[r][c] for r < rows, c < cols; x rows `ldx` apart.
void LaunchTranspose(const float* x, int rows, int cols, int ldx, float* y,
                     hipStream_t stream);

// y[c][f] = sum[c][f stride] scale for c < channels, f < frames; sum rows
// `positions` long.
void LaunchPickFrames(const double* sum, int channels, int positions, int stride, int frames,
                      double scale, float* y, hipStream_t stream);

// One residual vector quantizer stage: for every frame f the entry e of the
// largest -((|p|^2 - 2 p.e) + |e|^2) (the nearest; the lowest index on
// ties, distances in double) of the projected residual p = proj[:, f];
// codes[f] = e and residual[:, f] -= table[e].
struct NearestParams {
  const float* proj;       // [dim][frames]
  const float* embed;      // [entries][dim]
  const double* norms;     // [entries], |e|^2
  const float* table;      // [entries][hidden]
  float* residual;         // [hidden][frames]
  std::int32_t* codes;     // [frames]
  int dim, entries, hidden, frames;
};
void LaunchNearest(const NearestParams& p, hipStream_t stream);

}  // namespace ovg

#endif  // OMNIVOICE_AMD_ENCODER_HPP_
