/*
 * C ABI of the MI355X audio decoder: RVQ codes to 24 kHz audio through the
 * Higgs Audio v2 tokenizer's DAC decoder, in float32 on the GPU.
 *
 * Replaces Codec::Load's decoder half (codec.cpp:92-148) and Codec::Decode
 * (codec.cpp:197-260) of gufo-extensions/omnivoice. Conventions as in
 * omnivoice_mi355x.h: int status (OVG_OK / OVG_ERROR), a caller-provided
 * message buffer, no exception crosses the boundary, and the library never
 * returns memory for the caller to free. A handle is not thread-safe.
 */
#ifndef OMNIVOICE_CODEC_MI355X_H_
#define OMNIVOICE_CODEC_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#include "omnivoice_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The decoder's dimensions: CodecConfig and AcousticConfig of the reference
 * (config.hpp:46-72). The released tokenizer: codebooks 8, codebook_size
 * 1024, codebook_dim 64, hidden 1024 (semantic 768 + acoustic 256), latent
 * 256, channels 1024, ratios 8 5 4 2 3 (960 samples per frame). */
typedef struct ovc_config {
  int64_t codebooks;
  int64_t codebook_size;
  int64_t codebook_dim;
  int64_t hidden;   /* RVQ output width: semantic hidden + latent */
  int64_t latent;   /* acoustic hidden_size: fc2 output channels */
  int64_t channels; /* decoder_hidden_size, halved by every block */
  int64_t blocks;   /* number of upsampling blocks, <= 8 */
  int64_t ratios[8];
} ovc_config;

typedef struct ovc_handle ovc_handle;

/* Loads model_root/audio_tokenizer/model.safetensors (float32 tensors under
 * the reference's names, codec.cpp:95-148); the path is joined as
 * std::filesystem joins it (NULL or "" names the working directory) and a
 * missing file is an error. `weight_seed` is unused. Errors carry the prefix
 * "OmniVoice audio tokenizer: ". Replaces Codec::Load (codec.cpp:92-148),
 * decoder half. */
int ovc_create(const ovc_config* config, const char* model_root,
               uint64_t weight_seed, ovc_handle** handle, char* error,
               size_t error_len);

/* The seeded synthetic decoder of `weight_seed` (no reference counterpart:
 * the benchmark's and the tests' random-init decoder). */
int ovc_create_synthetic(const ovc_config* config, uint64_t weight_seed,
                         ovc_handle** handle, char* error, size_t error_len);
void ovc_destroy(ovc_handle* handle);

/* Samples that `frames` frames decode to. */
int64_t ovc_samples(const ovc_handle* handle, int64_t frames);

/* codes [codebooks][frames] (host) to audio[ovc_samples(frames)] (host).
 * Codes outside [0, codebook_size) are an error, as is a zero frame count.
 * Errors carry the prefix "OmniVoice decode: ". Replaces Codec::Decode
 * (codec.cpp:197-260). */
int ovc_decode(ovc_handle* handle, const int32_t* codes, int64_t frames,
               float* audio, char* error, size_t error_len);

/* ovc_decode on device buffers, enqueued on `stream` (hipStream_t, NULL =
 * the handle's own stream) without synchronising: codes [codebooks][frames]
 * and audio [ovc_samples(frames)] in device memory. Codes are not checked
 * (out-of-range codes are clamped to the table). No reference counterpart:
 * for callers that keep the generator's codes on the device. */
int ovc_decode_device(ovc_handle* handle, const int32_t* codes, int64_t frames,
                      float* audio, void* stream, char* error,
                      size_t error_len);

/* Per-kernel durations of decoding `frames` frames of fixed codes, `repeats`
 * times (HIP events around every launch). A measurement hook with no
 * reference counterpart. */
int ovc_profile_decode(ovc_handle* handle, int64_t frames, int64_t repeats,
                       ovg_kernel_stat* stats, int64_t capacity,
                       int64_t* count, char* error, size_t error_len);

/* Values the synthetic decoder holds for elements [first, first + count) of
 * tensor `tensor` (ids and scales as in the codec engine's specification):
 * float(scale n) or, with exponential set, float(exp(scale n)), n the
 * seeded normal of ovg_synthetic_values. Host only. */
void ovc_synthetic_values(uint64_t weight_seed, uint64_t tensor, uint64_t first,
                          int64_t count, double scale, int exponential,
                          float* out);

/* One convolution layer for op-level tests: x [in][length], alpha [in] and
 * y [out][length] in device memory; w (PyTorch's layout [out][in][kernel])
 * and b [out] on the host. Padding (kernel - 1) dilation / 2; Snake on the
 * input when alpha is not NULL; y += result when accumulate is set.
 * Synchronises `stream`. */
int ovc_op_conv1d(const float* x, int64_t in, int64_t length, const float* alpha,
                  const float* w, const float* b, int64_t out, int64_t kernel,
                  int64_t dilation, int accumulate, float* y, void* stream,
                  char* error, size_t error_len);

/* The decoder's upsampling layer for op-level tests: x [in][length], alpha
 * and y [out][length * stride] in device memory; w [in][out][2 stride]
 * (PyTorch's ConvTranspose1d layout) and b [out] on the host. Padding
 * ceil(stride / 2), output_padding stride % 2; Snake on the input when
 * alpha is not NULL. Synchronises `stream`. */
int ovc_op_conv_transpose1d(const float* x, int64_t in, int64_t length,
                            const float* alpha, const float* w, const float* b,
                            int64_t out, int64_t stride, float* y, void* stream,
                            char* error, size_t error_len);

/* ------------------------------------------------------------ the encoder */

/* The encoder's dimensions: CodecConfig's frame_samples and
 * semantic_stride, SemanticEncoderConfig (HuBERT) and AcousticConfig's
 * encoder half (config.hpp:28-72). The released tokenizer: sample_rate
 * 24000, semantic_rate 16000, frame_samples 960, semantic_stride 2; 7
 * feature convolutions of 512 channels, kernels 10 3 3 3 3 2 2, strides
 * 5 2 2 2 2 2 2; width 768, intermediate 3072, 12 heads, 12 layers,
 * positional convolution of 128 taps in 16 groups, eps 1e-5; enc_channels
 * 64, latent 256, ratios 8 5 4 2 3; 8 codebooks of 1024 x 64. */
typedef struct ovc_encoder_config {
  int64_t sample_rate;     /* input audio, Hz */
  int64_t semantic_rate;   /* HuBERT input, Hz */
  int64_t frame_samples;   /* input samples per codec frame */
  int64_t semantic_stride; /* HuBERT frames per codec frame */
  int64_t feature_layers;  /* HuBERT feature convolutions, <= 8 */
  int64_t conv_dim[8];
  int64_t conv_kernel[8];
  int64_t conv_stride[8];
  int64_t width;           /* HuBERT hidden size */
  int64_t intermediate;
  int64_t heads;
  int64_t layers;
  int64_t pos_kernel;      /* positional convolution taps */
  int64_t pos_groups;
  double eps;              /* LayerNorm epsilon */
  int64_t enc_channels;    /* DAC encoder input channels, doubled per block */
  int64_t latent;          /* DAC encoder output channels */
  int64_t blocks;          /* DAC downsampling blocks, <= 8 */
  int64_t ratios[8];
  int64_t codebooks;
  int64_t codebook_size;
  int64_t codebook_dim;
} ovc_encoder_config;

typedef struct ovc_encoder ovc_encoder;

/* Loads the encoder half of model_root/audio_tokenizer/model.safetensors
 * (float32 tensors under the reference's names, codec_encoder.cpp:74-240);
 * the path is joined as std::filesystem joins it (NULL or "" names the
 * working directory) and a missing file is an error. `weight_seed` is
 * unused. Errors carry the prefix "OmniVoice audio tokenizer: ". Replaces
 * LoadEncoder (codec_encoder.cpp:74-240). */
int ovc_encoder_create(const ovc_encoder_config* config, const char* model_root,
                       uint64_t weight_seed, ovc_encoder** handle, char* error,
                       size_t error_len);

/* The seeded synthetic encoder of `weight_seed` (no reference counterpart:
 * the benchmark's and the tests' random-init encoder). */
int ovc_encoder_create_synthetic(const ovc_encoder_config* config,
                                 uint64_t weight_seed, ovc_encoder** handle,
                                 char* error, size_t error_len);
void ovc_encoder_destroy(ovc_encoder* handle);

/* Codec frames that `samples` input samples encode to. */
int64_t ovc_encoder_frames(const ovc_encoder* handle, int64_t samples);

/* 24 kHz mono samples (host, a whole number of frames) to codes
 * [codebooks][frames] (host). semantic [frames][width] (the averaged HuBERT
 * features), acoustic [frames][latent] (the DAC encoder output) and
 * embeddings [frames][codebooks' hidden] (fc's output, the quantizer's
 * input) are optional host outputs (NULL to skip). Errors carry the prefix
 * "OmniVoice encode: ". Replaces Codec::Encode (codec_encoder.cpp:249-492). */
int ovc_encode(ovc_encoder* handle, const float* samples, int64_t length,
               int32_t* codes, float* semantic, float* acoustic,
               float* embeddings, char* error, size_t error_len);

/* ovc_encode on device buffers, enqueued on `stream` (hipStream_t, NULL =
 * the default stream); does not synchronise. */
int ovc_encode_device(ovc_encoder* handle, const float* samples, int64_t length,
                      int32_t* codes, void* stream, char* error,
                      size_t error_len);

/* Per-kernel timings of `repeats` encodes of `length` samples of a
 * synthetic signal (HIP events around every launch), as
 * ovc_profile_decode. */
int ovc_profile_encode(ovc_encoder* handle, int64_t length, int64_t repeats,
                       ovg_kernel_stat* stats, int64_t capacity, int64_t* count,
                       char* error, size_t error_len);

#ifdef __cplusplus
}
#endif

#endif /* OMNIVOICE_CODEC_MI355X_H_ */
