/*
 * ORACLE — test infrastructure, not product code.
 *
 * A CPU restatement of the reference's unmasking generator (gufo-extensions/
 * omnivoice): decoding.cpp:12-107, generator.cpp:175-301,
 * kernels/generator_kernels.hip:62-265. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it, and only to check the product's
 * results or as the timed CPU baseline. The product (omnivoice_amd/) never links or calls it.
 *
 * Pinning (what fixes each function, besides the GPU comparison):
 *   orc_unmask_schedule  - the reference fixture's three 32-step schedules,
 *                          and oracle/_ref (the reference's decoding.cpp).
 *   orc_build_input      - the fixture's input_ids, and oracle/_ref.
 *   orc_selector_*       - the reference's greedy KAT (decoding_test.cpp:67-80),
 *                          oracle/_ref with Gumbel noise, brute-force sort,
 *                          and the std::mt19937_64 known answer.
 *   orc_exp / orc_log    - glibc expf/logf within 2 ulp over sweeps.
 *   orc_score            - float64 closed form per row; invariants.
 *   orc_forward pieces   - float64 textbook formulas at tiny shapes and the
 *                          installed transformers Qwen3 layer (fixtures);
 *                          orc_swiglu against float64; orc_attention's
 *                          rounded probabilities against float64 with fp16 P.
 *   orc_forward emulate  - bit for bit the composition of the pinned pieces
 *                          rounding (orc_round_half, pinned against numpy's
 *                          float16) at exactly the reference's seven fp16
 *                          points; dropping any one changes the bits.
 *   orc_synth_*          - numpy float16 rounding; closed-form moments.
 *   orc_model_from_host  - the synthetic model's tensors in the reference's
 *                          load layout give the synthetic model's logits bit
 *                          for bit; swapped gate/up or k/v do not.
 *   orc_generate         - the loop spelled out from the pinned forward,
 *                          score and oracle/_ref's PositionSelector, with the
 *                          write-back into the conditional target frames.
 *   orc_generate_from_logits
 *                        - score + the selector step by step.
 *   orc_conv1d, orc_conv_transpose1d, orc_snake
 *                        - torch.nn.functional.conv1d / conv_transpose1d
 *                          in float64 on the CPU, and the Snake closed form.
 *   orc_codec_decode     - the installed transformers' DAC decoder (with
 *                          HiggsAudioV2's output padding, no tanh) at a small
 *                          configuration (tests/golden/codec_tiny.json), and
 *                          the same composition of torch float64 layers;
 *                          the real-checkpoint decode
 *                          vectors of the reference fixture need the codec
 *                          weights, which are absent (parity unpinned there).
 */
#ifndef OMNIVOICE_ORACLE_H_
#define OMNIVOICE_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_config {
  int64_t vocab_size, hidden_size, intermediate_size, layers, heads, kv_heads,
      head_dim, max_positions;
  float rms_norm_eps, rope_theta;
  int64_t audio_codebooks, audio_vocab_size;
  uint32_t audio_mask_id;
} orc_config;

/* decode.cpp */
void orc_unmask_schedule(int64_t total, int64_t steps, float t_shift,
                         int64_t* schedule);
int64_t orc_build_input(const uint32_t* text_ids, int64_t text_count,
                        const int32_t* reference_codes,
                        int64_t reference_frames, int64_t target_frames,
                        int64_t codebooks, uint32_t mask_id, int32_t* ids);
float orc_exp(float x);
float orc_log(float x);
void orc_score(const float* logits, int64_t frames, int64_t codebooks,
               int64_t vocab, uint32_t mask_id, float guidance,
               int32_t* prediction, float* confidence);
void* orc_selector_create(float layer_penalty, float temperature,
                          uint64_t seed);
void orc_selector_destroy(void* selector);
int64_t orc_selector_fill(void* selector, int64_t count, int64_t codebooks,
                          int64_t frames, const int32_t* prediction,
                          const float* confidence, uint32_t mask_id,
                          int32_t* codes, int64_t* chosen);
/* Noise the selector would draw for one Fill of `total` entries. */
void orc_selector_noise(void* selector, int64_t total, float* noise);
uint64_t orc_mt19937_64_nth(uint64_t seed, int64_t n);
/* Unmasking driven by given per-step logits (teacher forcing): for each
 * executed step e, score logits_trace[e] and select. */
int64_t orc_generate_from_logits(const float* logits_trace, int64_t executed,
                                 int64_t codebooks, int64_t frames,
                                 int64_t vocab, uint32_t mask_id,
                                 int64_t steps, float guidance, float t_shift,
                                 float layer_penalty, float temperature,
                                 uint64_t seed, int32_t* codes,
                                 int32_t* unmasked_at);

/* synth.cpp */
double orc_synth_normal(uint64_t seed, uint64_t tensor, uint64_t element);
float orc_round_half(float x);
void orc_synth_values(uint64_t seed, uint64_t tensor, uint64_t first,
                      int64_t count, int is_norm, float jitter, float* out);

/* forward.cpp */
void* orc_model_synthetic(const orc_config* config, uint64_t seed,
                          float norm_jitter);
/* tensors[layer][11] in the OVG_LAYER_* order; the model copies them,
 * rounding matrices to fp16 values. */
void* orc_model_from_host(const orc_config* config, const float* text,
                          const float* audio_embeddings,
                          const float* audio_heads, const float* final_norm,
                          const float* const* layers);
void orc_model_destroy(void* model);
void orc_set_threads(int threads);
/* emulate: 0 = float32 activations, 1 = round to fp16 where the
 * reference's GPU path rounds. logits [2F][C*V]. */
void orc_forward(void* model, const int32_t* ids, int64_t length,
                 int64_t audio_start, int64_t target_frames, int emulate,
                 float* logits);
void orc_generate(void* model, const int32_t* ids, int64_t length,
                  int64_t audio_start, int64_t target_frames, int emulate,
                  int64_t steps, float guidance, float t_shift,
                  float layer_penalty, float temperature, uint64_t seed,
                  int32_t* codes, int32_t* unmasked_at);

/* kernel-level restatements (float32) */
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows,
                 int64_t width, float eps);
void orc_linear(const float* x, const float* w, float* y, int64_t rows,
                int64_t in, int64_t out, int accumulate);
void orc_qk_norm_rope(const float* qkv, const float* q_norm,
                      const float* k_norm, const int32_t* positions,
                      float* out, int64_t rows, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, float eps,
                      float theta);
void orc_attention(const float* qkv, float* out, int64_t rows, int64_t heads,
                   int64_t kv_heads, int64_t head_dim,
                   const int64_t* sequences, int64_t count, int round_p);
void orc_swiglu(const float* gate_up, float* out, int64_t rows, int64_t inter);

/* codec.cpp: the audio decoder (codec.cpp:197-260 of the reference) */
typedef struct orc_codec_config {
  int64_t codebooks, codebook_size, codebook_dim;
  int64_t hidden;    /* semantic hidden + latent: the RVQ output width */
  int64_t latent;    /* fc2 output channels */
  int64_t channels;  /* decoder channels before the first block */
  int64_t blocks;
  int64_t ratios[8]; /* upsampling ratio per block */
} orc_codec_config;
void orc_snake(const float* x, int64_t channels, int64_t length,
               const float* alpha, float* y);
/* w [out][in][kernel], padding (kernel - 1) dilation / 2 */
void orc_conv1d(const float* x, int64_t in, int64_t length, const float* w,
                const float* b, int64_t out, int64_t kernel, int64_t dilation,
                float* y);
/* w [in][out][2 stride], padding ceil(stride / 2), output_padding stride % 2 */
void orc_conv_transpose1d(const float* x, int64_t in, int64_t length,
                          const float* w, const float* b, int64_t out,
                          int64_t stride, float* y);
void orc_codec_values(uint64_t seed, uint64_t tensor, uint64_t first,
                      int64_t count, double scale, int exponential,
                      float* out);
void* orc_codec_synthetic(const orc_codec_config* config, uint64_t seed);
void orc_codec_destroy(void* codec);
/* codes [codebooks][frames]; audio receives the returned sample count */
int64_t orc_codec_decode(const void* codec, const int32_t* codes,
                         int64_t frames, float* audio);

/* codec_encoder.cpp: the audio encoder (codec_encoder.cpp:249-492) */
typedef struct orc_encoder_config {
  int64_t sample_rate, semantic_rate, frame_samples, semantic_stride;
  int64_t feat_layers, conv_dim[8], conv_kernel[8], conv_stride[8];
  int64_t width, intermediate, heads, layers, pos_kernel, pos_groups;
  float eps;
  int64_t enc_channels, latent, blocks, ratios[8];
  int64_t codebooks, codebook_size, codebook_dim;
} orc_encoder_config;
int64_t orc_resample(const float* samples, int64_t length, uint32_t from_rate,
                     uint32_t to_rate, float* output);
void* orc_encoder_synthetic(const orc_encoder_config* config, uint64_t seed);
void orc_encoder_destroy(void* encoder);
/* samples: a whole number of frames at sample_rate. codes [codebooks][count];
 * optional stage outputs, frame-major: semantic features [count][width],
 * acoustic [count][latent], embeddings (after fc) [count][width + latent].
 * Returns count, or < 0 (-1 not whole frames, -2 too short for the semantic
 * stride, -3 acoustic and semantic frame counts differ). */
int64_t orc_encoder_encode(const void* encoder, const float* samples, int64_t length,
                           int32_t* codes, float* semantic_out, float* acoustic_out,
                           float* embeddings_out);

#ifdef __cplusplus
}
#endif

#endif /* OMNIVOICE_ORACLE_H_ */
