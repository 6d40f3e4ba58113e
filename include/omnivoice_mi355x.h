/*
 * C ABI of the MI355X (gfx950) OmniVoice unmasking generator.
 *
 * Plain C types only: sizes are int64_t, tensors are plain pointers, errors are
 * an int status plus a caller-owned message buffer. The library never returns
 * memory that the caller must free. One handle per thread; a handle is not
 * thread-safe (generator.hpp:17-19 of the reference states the same for the
 * class this replaces).
 *
 * Status codes: OVG_OK on success, OVG_ERROR with `error` filled, and
 * OVG_CANCELLED with `error` set to exactly "cancelled"
 * (reference: generator.cpp:508-511).
 *
 * Every entry point is cited against the reference interface it replaces.
 * The C++ `gufo::models::omnivoice::Generator` in include/omnivoice/ is a thin
 * wrapper over these functions with the reference's exact signatures.
 */
#ifndef OMNIVOICE_MI355X_H_
#define OMNIVOICE_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OVG_OK 0
#define OVG_ERROR 1
#define OVG_CANCELLED 2

typedef struct ovg_handle ovg_handle;

/* BackboneConfig + Config fields the generator reads
 * (reference: config.hpp:15-26 and config.hpp:74-82). */
typedef struct ovg_config {
  int64_t vocab_size;        /* text vocabulary rows of llm.embed_tokens */
  int64_t hidden_size;       /* 1024 */
  int64_t intermediate_size; /* 3072 */
  int64_t layers;            /* 28 */
  int64_t heads;             /* 16 query heads */
  int64_t kv_heads;          /* 8 key/value heads */
  int64_t head_dim;          /* 128 (the only supported value, config.cpp:340-355) */
  int64_t max_positions;     /* rotary table length */
  float rms_norm_eps;        /* 1e-6 */
  float rope_theta;          /* 1e6 */
  int64_t audio_codebooks;   /* 8 */
  int64_t audio_vocab_size;  /* 1025 entries per codebook, mask included */
  uint32_t audio_mask_id;    /* 1024 */
} ovg_config;

/* ConditionalInput (reference: decoding.hpp:32-47). `ids` is
 * [codebooks][length]: text tokens repeated in every codebook row, then the
 * reference frames, then the target frames (initially the mask id). */
typedef struct ovg_input {
  int64_t codebooks;
  int64_t length;
  int64_t audio_start;
  int64_t target_frames;
  const int32_t* ids;
} ovg_input;

/* DecodingConfig (reference: decoding.hpp:14-21). */
typedef struct ovg_decoding {
  int64_t steps;              /* 32 */
  float guidance;             /* 2.0 */
  float t_shift;              /* 0.1 */
  float layer_penalty;        /* 5.0 */
  float position_temperature; /* 5.0; 0 selects positions greedily */
} ovg_decoding;

/* Host float32 tensors with the checkpoint's names and shapes
 * (reference: generator.cpp:364-425). `layers` points to `config.layers`
 * arrays of OVG_LAYER_TENSORS pointers in the order of the OVG_LAYER_* ids. */
enum {
  OVG_LAYER_Q_PROJ = 0,     /* self_attn.q_proj.weight [heads*head_dim][hidden] */
  OVG_LAYER_K_PROJ = 1,     /* self_attn.k_proj.weight [kv_heads*head_dim][hidden] */
  OVG_LAYER_V_PROJ = 2,     /* self_attn.v_proj.weight [kv_heads*head_dim][hidden] */
  OVG_LAYER_O_PROJ = 3,     /* self_attn.o_proj.weight [hidden][heads*head_dim] */
  OVG_LAYER_GATE_PROJ = 4,  /* mlp.gate_proj.weight [intermediate][hidden] */
  OVG_LAYER_UP_PROJ = 5,    /* mlp.up_proj.weight [intermediate][hidden] */
  OVG_LAYER_DOWN_PROJ = 6,  /* mlp.down_proj.weight [hidden][intermediate] */
  OVG_LAYER_INPUT_NORM = 7, /* input_layernorm.weight [hidden] */
  OVG_LAYER_POST_NORM = 8,  /* post_attention_layernorm.weight [hidden] */
  OVG_LAYER_Q_NORM = 9,     /* self_attn.q_norm.weight [head_dim] */
  OVG_LAYER_K_NORM = 10,    /* self_attn.k_norm.weight [head_dim] */
  OVG_LAYER_TENSORS = 11
};

typedef struct ovg_host_weights {
  const float* text_embeddings;  /* llm.embed_tokens.weight [vocab][hidden] */
  const float* audio_embeddings; /* audio_embeddings.weight [codebooks*vocab][hidden] */
  const float* audio_heads;      /* audio_heads.weight [codebooks*vocab][hidden] */
  const float* final_norm;       /* llm.norm.weight [hidden] */
  const float* const* layers;    /* [layers][OVG_LAYER_TENSORS] */
} ovg_host_weights;

/* Per-kernel timing of one eagerly launched forward + scoring step. */
typedef struct ovg_kernel_stat {
  char name[48];
  int64_t launches;
  double total_ms;     /* sum of launch durations, HIP events on the library stream */
  double flops;        /* algorithmic FLOPs summed over launches */
  double bytes;        /* algorithmic HBM bytes summed over launches */
} ovg_kernel_stat;

/* ---- Load (reference: Generator::Load, generator.hpp:22-24, generator.cpp:364-434) ----
 * Reads model_root/model.safetensors: the checkpoint's float32 tensors under
 * the names of ovg_host_weights (reference: generator.cpp:377-425). The path
 * is joined as std::filesystem joins it, so NULL or "" names
 * model.safetensors in the working directory, as the reference's Load does;
 * a missing file is an error ("OmniVoice generator: cannot open ..."). Every
 * tensor is found and checked against `config` before the GPU is touched,
 * and errors name the file or tensor at fault. `weight_seed` is unused;
 * synthetic weights come only from ovg_create_synthetic. */
int ovg_create(const ovg_config* config, const char* model_root,
               uint64_t weight_seed, ovg_handle** handle, char* error,
               size_t error_len);

/* The seeded synthetic model: every matrix and embedding drawn from
 * N(0, 0.02) (the counter-based values of ovg_synthetic_values) and rounded
 * to fp16; norm weights 1 + norm_jitter * N(0, 1) (rounded to fp16), 1.0 at
 * norm_jitter 0. No reference counterpart: the benchmark's and the tests'
 * random-init model. */
int ovg_create_synthetic(const ovg_config* config, uint64_t weight_seed,
                         float norm_jitter, ovg_handle** handle, char* error,
                         size_t error_len);

/* The model from host float32 tensors: matrices are rounded to fp16 and
 * fused (q|k|v, gate|up) on upload; norms and embeddings stay fp32
 * (reference: generator.cpp:393-425). */
int ovg_create_from_host(const ovg_config* config,
                         const ovg_host_weights* weights, ovg_handle** handle,
                         char* error, size_t error_len);

/* ~Generator (reference: generator.hpp:25). NULL is ignored. */
void ovg_destroy(ovg_handle* handle);

/* ---- Generator::Forward (reference: generator.hpp:41-43, generator.cpp:436-454) ----
 * `logits` receives [2 * target_frames][codebooks * audio_vocab_size]:
 * conditional target rows, then unconditional. */
int ovg_forward(ovg_handle* handle, const ovg_input* input, float* logits,
                char* error, size_t error_len);

/* ---- Generator::Score (reference: generator.hpp:47-50, generator.cpp:456-484) ----
 * `prediction` / `confidence` are [codebooks][target_frames]. */
int ovg_score(ovg_handle* handle, const ovg_input* input, float guidance,
              int32_t* prediction, float* confidence, char* error,
              size_t error_len);

/* ---- Generator::Generate (reference: generator.hpp:31-36, generator.cpp:486-543) ----
 * The whole unmasking loop runs on the GPU: forward, CFG scoring and top-k
 * position selection; only the final codes come back. `cancelled` (may be
 * NULL) is polled before every step. `codes` / `unmasked_at` are
 * [codebooks][target_frames]. */
int ovg_generate(ovg_handle* handle, const ovg_input* input,
                 const ovg_decoding* decoding, uint64_t seed,
                 int (*cancelled)(void* user), void* user, int32_t* codes,
                 int32_t* unmasked_at, char* error, size_t error_len);

/* Several independent inputs (e.g. chunks of a long text) generated in one
 * packed batch; item i uses seeds[i] and writes codes[i] / unmasked_at[i],
 * bit for bit what ovg_generate gives for the item alone (reference: the
 * sequential chunk loop at synthesizer.cpp:179-201 calls Generate once per
 * chunk): no kernel's order of summation depends on the other items. */
int ovg_generate_batch(ovg_handle* handle, int64_t count,
                       const ovg_input* inputs, const ovg_decoding* decoding,
                       const uint64_t* seeds, int (*cancelled)(void* user),
                       void* user, int32_t* const* codes,
                       int32_t* const* unmasked_at, char* error,
                       size_t error_len);

/* ---- The chunk loop of Synthesizer::Synthesize (reference: synthesizer.cpp:179-201) ----
 * Generates the `count` chunks of one long text with one seed, with the
 * results of the reference's loop, which calls Generate once per chunk
 * (synthesizer.cpp:70-71): chunk i's input is ConditionalInput::Build(
 * text_ids[i], reference, target_frames[i]) (decoding.cpp:42-62). With a
 * reference voice (reference_frames > 0, reference_codes [codebooks]
 * [reference_frames]) every chunk is conditioned on it and all chunks run as
 * one packed batch. Without one, chunk 0 runs alone and its codes become the
 * reference of chunks 1 .. count - 1 (synthesizer.cpp:195-200), which then
 * run as one batch. text_ids[i] (text_counts[i] ids) are chunk i's prompt
 * ids as the caller's prompt builder encodes them (EncodePromptText; for the
 * chunks after the first without a reference voice, with chunk 0's text as
 * the reference text). Batched items give bit for bit the codes of separate
 * ovg_generate calls. codes[i] / unmasked_at[i] are [codebooks]
 * [target_frames[i]]. Cancellation returns 2 with "cancelled". */
int ovg_generate_chunks(ovg_handle* handle, int64_t count,
                        const uint32_t* const* text_ids, const int64_t* text_counts,
                        const int32_t* reference_codes, int64_t reference_frames,
                        const int64_t* target_frames, const ovg_decoding* decoding,
                        uint64_t seed, int (*cancelled)(void* user), void* user,
                        int32_t* const* codes, int32_t* const* unmasked_at,
                        char* error, size_t error_len);

/* ovg_generate that also returns every executed step's logits, launched
 * eagerly instead of from the captured step graph. `logits_trace` receives
 * [executed steps][2 * target_frames][codebooks * audio_vocab_size] and
 * `executed` the number of executed (non-zero) steps. A test hook: the
 * reference has no counterpart. */
int ovg_generate_trace(ovg_handle* handle, const ovg_input* input,
                       const ovg_decoding* decoding, uint64_t seed,
                       int32_t* codes, int32_t* unmasked_at,
                       float* logits_trace, int64_t* executed, char* error,
                       size_t error_len);

/* ovg_generate_batch launched eagerly, returning item i's logits at every
 * step it executes: logits_traces[i] (may be NULL, as may logits_traces)
 * receives [executed[i]][2 * target_frames_i][codebooks * audio_vocab_size]
 * and executed[i] (may be NULL) the item's executed-step count. A test hook:
 * the reference has no counterpart. */
int ovg_generate_trace_batch(ovg_handle* handle, int64_t count,
                             const ovg_input* inputs, const ovg_decoding* decoding,
                             const uint64_t* seeds, int32_t* const* codes,
                             int32_t* const* unmasked_at, float* const* logits_traces,
                             int64_t* executed, char* error, size_t error_len);

/* Per-kernel durations of one eager forward + score + select of `input`
 * (HIP events around every launch). Writes up to `capacity` entries and
 * sets `count` to the number of distinct kernels. A measurement hook: the
 * reference has no counterpart. */
int ovg_profile_step(ovg_handle* handle, const ovg_input* input,
                     int64_t repeats, ovg_kernel_stat* stats,
                     int64_t capacity, int64_t* count, char* error,
                     size_t error_len);

/* ovg_profile_step over `items` inputs packed as one batch, as
 * ovg_generate_batch runs them. */
int ovg_profile_batch(ovg_handle* handle, int64_t items,
                      const ovg_input* inputs, int64_t repeats,
                      ovg_kernel_stat* stats, int64_t capacity, int64_t* count,
                      char* error, size_t error_len);

/* Values the synthetic model holds for elements [first, first + count) of
 * one tensor (ids: text embeddings 1, audio embeddings 2, audio heads 3,
 * final norm 4, layer l tensor k 100 + 16 l + k): matrices
 * half(float(0.02 * N(0, 1))), norms 1.0 or half(float(1 + jitter N(0, 1))).
 * Host only. It stands in for reading the checkpoint's float32 tensors
 * (reference: generator.cpp:309-352). */
void ovg_synthetic_values(uint64_t weight_seed, uint64_t tensor, uint64_t first,
                          int64_t count, int is_norm, float norm_jitter,
                          float* out);

/* Device bytes the handle holds (weights + workspace). */
int64_t ovg_device_bytes(const ovg_handle* handle);

/* ---- Host decoding helpers (reference: decoding.hpp:23-47, decoding.cpp:12-62) ---- */

/* UnmaskSchedule(total, steps, t_shift) into schedule[steps]. */
int ovg_unmask_schedule(int64_t total, int64_t steps, float t_shift,
                        int64_t* schedule);

/* ConditionalInput::Build: writes ids[codebooks][text + reference_frames +
 * target_frames]; `reference_codes` is [codebooks][reference_frames] (may be
 * NULL when reference_frames is 0). Returns the length. */
int64_t ovg_build_input(const uint32_t* text_ids, int64_t text_count,
                        const int32_t* reference_codes,
                        int64_t reference_frames, int64_t target_frames,
                        int64_t codebooks, uint32_t mask_id, int32_t* ids);

/* ---- Device operators on caller-owned device pointers ----
 * Each replaces one launcher of the reference's kernels namespace; `stream`
 * is a hipStream_t (NULL = the null stream). They validate their shapes and
 * return OVG_ERROR with a message instead of launching on a bad shape. */

/* kernels::Score (reference: generator_kernels.hpp:58-66). logits
 * [2*frames][codebooks*vocab] fp32 -> prediction int32 / confidence fp32
 * [codebooks][frames]. Bit-exact with the oracle's restatement. */
int ovg_op_score(const float* logits, int32_t* prediction, float* confidence,
                 int64_t frames, int64_t codebooks, int64_t vocab,
                 uint32_t mask_id, float guidance, void* stream, char* error,
                 size_t error_len);

/* PositionSelector::Fill on the device (reference: decoding.cpp:70-107) for
 * one item: scores = confidence - codebook * layer_penalty, then
 * score / temperature + noise when temperature > 0, masked codes only; the
 * `count` best by (score desc, index asc) take their prediction. `noise` is
 * [codebooks*frames] (ignored when temperature is 0). `codes` and
 * `unmasked_at` ([codebooks][frames]) are updated in place; chosen entries
 * get unmasked_at = step. */
int ovg_op_select(const int32_t* prediction, const float* confidence,
                  const float* noise, int32_t* codes, int32_t* unmasked_at,
                  int64_t codebooks, int64_t frames, int64_t count,
                  int32_t step, float layer_penalty, float temperature,
                  uint32_t mask_id, void* stream, char* error,
                  size_t error_len);

/* HalfGemm::Linear (reference: gemm.hpp:50-52, gemm.cpp:248-262):
 * y[rows][out] (+)= x[rows][in] * w[out][in]^T, fp16 operands, fp32
 * accumulation and output. `in` must be a multiple of 64. */
int ovg_op_linear(const void* x, const void* w, float* y, int64_t rows,
                  int64_t in, int64_t out, int accumulate, void* stream,
                  char* error, size_t error_len);

/* ovg_op_linear without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc). The split-K partials of
 * small-M shapes live in a static device array of
 * OVG_LINEAR_NOALLOC_SCRATCH_FLOATS floats (4 MiB per GPU, held until the
 * process ends), which every shape ovg_op_linear accepts fits; a plan that
 * did not would be rejected with an error. Same kernels and plan as
 * ovg_op_linear, so the same result bit for bit; enqueued on `stream`
 * without waiting for it. Calls that overlap on one GPU (two streams or two
 * threads) share the array and race: serialise them. The first call on each
 * GPU looks up that GPU's address of the array (hipGetSymbolAddress); make it
 * outside graph capture, after which calls may be captured and replayed. */
#define OVG_LINEAR_NOALLOC_SCRATCH_FLOATS 1048576
int ovg_op_linear_noalloc(const void* x, const void* w, float* y, int64_t rows,
                          int64_t in, int64_t out, int accumulate, void* stream,
                          char* error, size_t error_len);

/* HalfGemm::Linear as the generator runs it (reference: gemm.hpp:50-52,
 * gemm.cpp:248-262): ovg_op_linear's result through the packed-weight
 * kernel, w packed on the device first (row-major fp16 [out][in] in).
 * `tile_rows` and `tile_cols` 0 take the planned tile; 32, 64, 96 or 128
 * rows by 128, 64 or 32 columns, 128 by 256 or 256 by 256 force one (every tile
 * gives the same result bit for bit). */
int ovg_op_linear_packed(const void* x, const void* w, float* y, int64_t rows,
                         int64_t in, int64_t out, int accumulate, int64_t tile_rows,
                         int64_t tile_cols, void* stream, char* error, size_t error_len);

/* kernels::RmsNorm (reference: generator_kernels.hpp:25-28): output =
 * half(weight * x * rsqrt(mean(x^2) + eps)) per row. */
int ovg_op_rmsnorm(const float* input, const float* weight, void* output,
                   int64_t rows, int64_t width, float epsilon, void* stream,
                   char* error, size_t error_len);

/* Bidirectional GQA attention over packed sequences; replaces the two
 * State::Attention calls plus MergeHeads (reference: generator.cpp:122-172,
 * generator_kernels.hpp:44-47). qkv is fp16 [rows][(heads + 2*kv_heads) *
 * 128] after q/k norm and rotary; `sequences` holds `count` (first_row,
 * length) pairs (first_row a multiple of 16); output fp16 [rows][heads*128]. */
int ovg_op_attention(const void* qkv, void* output, int64_t rows,
                     int64_t heads, int64_t kv_heads,
                     const int64_t* sequences, int64_t count, void* stream,
                     char* error, size_t error_len);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* OMNIVOICE_MI355X_H_ */
