// ORACLE — test infrastructure, not product code (see oracle.h).
//
// The backbone forward over the packed CFG batch and the unmasking loop,
// restated on the CPU in float32:
//   State::Prepare / UploadIds   generator.cpp:175-258 (batch packing)
//   State::RunForward            generator.cpp:262-301 (layer order)
//   State::Attention             generator.cpp:122-172 (per sequence, per head)
//   kernels::Embed               kernels/generator_kernels.hip:62-83
//   kernels::RmsNorm             kernels/generator_kernels.hip:85-97
//   kernels::QkNormRope          kernels/generator_kernels.hip:102-159
//   kernels::Softmax             kernels/generator_kernels.hip:161-176
//   kernels::SwiGlu              kernels/generator_kernels.hip:191-200
//   kernels::GatherRows          kernels/generator_kernels.hip:202-209
//   Generator::Generate          generator.cpp:486-543
// With emulate = 1 the activations are rounded to fp16 at the points where
// the reference's GPU path stores float16 (normed rows, q/k/v, attention
// probabilities, merged heads, SwiGLU output); with emulate = 0 everything
// after the fp16-valued weights is float32 (the "fp32 reference").
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "oracle.h"

namespace {

constexpr std::uint64_t kTextTensor = 1;
constexpr std::uint64_t kAudioEmbeddingTensor = 2;
constexpr std::uint64_t kAudioHeadTensor = 3;
constexpr std::uint64_t kFinalNormTensor = 4;
constexpr int kLayerTensors = 11;
std::uint64_t LayerTensor(int64_t layer, int kind) {
  return 100 + 16 * static_cast<std::uint64_t>(layer) +
         static_cast<std::uint64_t>(kind);
}

typedef float v8 __attribute__((vector_size(32)));

inline v8 Load8(const float* p) {
  v8 v;
  std::memcpy(&v, p, sizeof(v));
  return v;
}

inline float Sum8(v8 v) {
  return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

inline float Dot(const float* a, const float* b, int64_t n) {
  v8 acc = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t k = 0;
  for (; k + 8 <= n; k += 8)
    acc += Load8(a + k) * Load8(b + k);
  float s = Sum8(acc);
  for (; k < n; ++k)
    s += a[k] * b[k];
  return s;
}

// y[m][n] (+)= sum_k x[m][k] w[n][k]: 4 x 4 register blocks vectorised over
// k, tasks of 64 output columns so a task's weight rows stay in cache.
void Gemm(const float* x, const float* w, float* y, int64_t rows, int64_t in,
          int64_t out, bool accumulate) {
  const int64_t tiles = (out + 63) / 64;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t tile = 0; tile < tiles; ++tile) {
    const int64_t n_end = std::min(out, tile * 64 + 64);
    for (int64_t m0 = 0; m0 < rows; m0 += 4) {
      const int64_t mc = std::min<int64_t>(4, rows - m0);
      for (int64_t n0 = tile * 64; n0 < n_end; n0 += 4) {
        const int64_t nc = std::min<int64_t>(4, n_end - n0);
        if (mc == 4 && nc == 4 && in % 8 == 0) {
          v8 acc[4][4];
          for (auto& r : acc)
            for (auto& c : r)
              c = v8{0, 0, 0, 0, 0, 0, 0, 0};
          const float* xr[4] = {x + m0 * in, x + (m0 + 1) * in,
                                x + (m0 + 2) * in, x + (m0 + 3) * in};
          const float* wr[4] = {w + n0 * in, w + (n0 + 1) * in,
                                w + (n0 + 2) * in, w + (n0 + 3) * in};
          for (int64_t k = 0; k < in; k += 8) {
            const v8 a0 = Load8(xr[0] + k), a1 = Load8(xr[1] + k),
                     a2 = Load8(xr[2] + k), a3 = Load8(xr[3] + k);
            for (int j = 0; j < 4; ++j) {
              const v8 b = Load8(wr[j] + k);
              acc[0][j] += a0 * b;
              acc[1][j] += a1 * b;
              acc[2][j] += a2 * b;
              acc[3][j] += a3 * b;
            }
          }
          for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j) {
              float* dst = y + (m0 + i) * out + n0 + j;
              const float v = Sum8(acc[i][j]);
              *dst = accumulate ? *dst + v : v;
            }
        } else {
          for (int64_t i = 0; i < mc; ++i)
            for (int64_t j = 0; j < nc; ++j) {
              float* dst = y + (m0 + i) * out + n0 + j;
              const float v = Dot(x + (m0 + i) * in, w + (n0 + j) * in, in);
              *dst = accumulate ? *dst + v : v;
            }
        }
      }
    }
  }
}

void RoundAll(float* data, int64_t count, bool emulate) {
  if (!emulate)
    return;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i)
    data[i] = orc_round_half(data[i]);
}

// kernels::RmsNorm: y = w * (x * rsqrt(mean(x^2) + eps)).
void RmsNormRows(const float* x, const float* w, float* y, int64_t rows,
                 int64_t width, float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * width;
    float squares = 0.0F;
    for (int64_t d = 0; d < width; ++d)
      squares += in[d] * in[d];
    const float scale =
        1.0F / std::sqrt(squares / static_cast<float>(width) + eps);
    float* o = y + r * width;
    for (int64_t d = 0; d < width; ++d)
      o[d] = w[d] * (in[d] * scale);
  }
}

// kernels::QkNormRope: per-head RMSNorm of q and k heads, Hugging Face's
// default rotary embedding (rotate-half, inv_freq = 1 / theta^(2i/d) in
// float32), v passed through. In and out are [rows][(h + 2 kv) * d].
void QkNormRopeRows(const float* qkv, const float* q_norm, const float* k_norm,
                    const int32_t* positions, float* out, int64_t rows,
                    int64_t heads, int64_t kv_heads, int64_t head_dim,
                    float eps, float theta) {
  const int64_t slots = heads + 2 * kv_heads;
  const int64_t width = slots * head_dim;
  const int64_t half = head_dim / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t s = 0; s < slots; ++s) {
      const float* in = qkv + r * width + s * head_dim;
      float* o = out + r * width + s * head_dim;
      if (s >= heads + kv_heads) {
        std::memcpy(o, in, static_cast<std::size_t>(head_dim) * sizeof(float));
        continue;
      }
      const float* weight = s < heads ? q_norm : k_norm;
      float squares = 0.0F;
      for (int64_t d = 0; d < head_dim; ++d)
        squares += in[d] * in[d];
      const float scale =
          1.0F / std::sqrt(squares / static_cast<float>(head_dim) + eps);
      for (int64_t i = 0; i < half; ++i) {
        const float a = weight[i] * (in[i] * scale);
        const float b = weight[i + half] * (in[i + half] * scale);
        const float inv_freq =
            1.0F / std::pow(theta, static_cast<float>(2 * i) /
                                       static_cast<float>(head_dim));
        const float angle = static_cast<float>(positions[r]) * inv_freq;
        const float c = std::cos(angle);
        const float sn = std::sin(angle);
        o[i] = a * c - b * sn;
        o[i + half] = b * c + a * sn;
      }
    }
  }
}

// State::Attention + Softmax + MergeHeads: per sequence (first, length) and
// query head h (kv head h / (heads / kv_heads)), softmax(q k^T / sqrt(d)) v,
// written row-major [rows][heads * d].
void AttentionRows(const float* qkv, float* out, int64_t rows, int64_t heads,
                   int64_t kv_heads, int64_t head_dim,
                   const int64_t* sequences, int64_t count, bool round_p) {
  (void)rows;
  const int64_t width = (heads + 2 * kv_heads) * head_dim;
  const int64_t group = heads / kv_heads;
  const float scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  for (int64_t s = 0; s < count; ++s) {
    const int64_t first = sequences[2 * s];
    const int64_t length = sequences[2 * s + 1];
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int64_t h = 0; h < heads; ++h) {
      for (int64_t i = 0; i < length; ++i) {
        const int64_t kv = h / group;
        const float* q = qkv + (first + i) * width + h * head_dim;
        std::vector<float> p(static_cast<std::size_t>(length));
        float maximum = -3.402823466e38F;
        for (int64_t j = 0; j < length; ++j) {
          const float* k =
              qkv + (first + j) * width + (heads + kv) * head_dim;
          p[j] = Dot(q, k, head_dim) * scale;
          maximum = std::max(maximum, p[j]);
        }
        float sum = 0.0F;
        for (int64_t j = 0; j < length; ++j) {
          p[j] = std::exp(p[j] - maximum);
          sum += p[j];
        }
        const float inverse = 1.0F / sum;
        for (int64_t j = 0; j < length; ++j) {
          p[j] = p[j] * inverse;
          if (round_p)
            p[j] = orc_round_half(p[j]);
        }
        float* o = out + (first + i) * heads * head_dim + h * head_dim;
        for (int64_t d = 0; d < head_dim; ++d)
          o[d] = 0.0F;
        for (int64_t j = 0; j < length; ++j) {
          const float* v = qkv + (first + j) * width +
                           (heads + kv_heads + kv) * head_dim;
          for (int64_t d = 0; d < head_dim; ++d)
            o[d] += p[j] * v[d];
        }
      }
    }
  }
}

// kernels::SwiGlu: silu(gate) * up, gate = columns [0, inter) and up =
// [inter, 2 inter) of each row (kernels/generator_kernels.hip:191-200).
void SwiGluRows(const float* gate_up, float* out, int64_t rows, int64_t inter) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < inter; ++i) {
      const float g = gate_up[r * 2 * inter + i];
      const float u = gate_up[r * 2 * inter + inter + i];
      out[r * inter + i] = g / (1.0F + std::exp(-g)) * u;
    }
}

struct Layer {
  std::vector<float> qkv;      // [q rows | k rows | v rows][hidden]
  std::vector<float> output;   // [hidden][heads * d]
  std::vector<float> gate_up;  // [gate rows | up rows][hidden]
  std::vector<float> down;     // [hidden][intermediate]
  std::vector<float> input_norm, post_norm, q_norm, k_norm;
};

struct Model {
  orc_config config{};
  bool synthetic = false;
  std::uint64_t seed = 0;
  float jitter = 0.0F;
  std::vector<float> text;  // host tensors only; synthetic rows on demand
  std::vector<float> audio_embeddings, audio_heads, final_norm;
  std::vector<Layer> layers;

  void TextRow(int64_t id, float* row) const {
    const int64_t h = config.hidden_size;
    if (synthetic)
      orc_synth_values(seed, kTextTensor, static_cast<std::uint64_t>(id * h),
                       h, 0, 0.0F, row);
    else
      std::memcpy(row, &text[static_cast<std::size_t>(id * h)],
                  static_cast<std::size_t>(h) * sizeof(float));
  }
};

void Synth(std::vector<float>* out, std::uint64_t seed, std::uint64_t tensor,
           std::uint64_t offset_elements, int64_t count, bool norm,
           float jitter, std::size_t at) {
  constexpr int64_t kChunk = 1 << 16;
  const int64_t chunks = (count + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t begin = c * kChunk;
    const int64_t n = std::min(kChunk, count - begin);
    orc_synth_values(seed, tensor, offset_elements + begin, n, norm ? 1 : 0,
                     jitter, out->data() + at + begin);
  }
}

void RoundMatrix(std::vector<float>* m) {
  RoundAll(m->data(), static_cast<int64_t>(m->size()), true);
}

}  // namespace

extern "C" {

void orc_set_threads(int threads) { omp_set_num_threads(threads); }

void* orc_model_synthetic(const orc_config* config, uint64_t seed,
                          float norm_jitter) {
  auto* m = new Model;
  m->config = *config;
  m->synthetic = true;
  m->seed = seed;
  m->jitter = norm_jitter;
  const orc_config& c = *config;
  const int64_t h = c.hidden_size, d = c.head_dim, in = c.intermediate_size;
  const int64_t q_rows = c.heads * d, kv_rows = c.kv_heads * d;
  const int64_t audio_rows = c.audio_codebooks * c.audio_vocab_size;
  m->audio_embeddings.resize(static_cast<std::size_t>(audio_rows * h));
  Synth(&m->audio_embeddings, seed, kAudioEmbeddingTensor, 0, audio_rows * h,
        false, 0.0F, 0);
  m->audio_heads.resize(static_cast<std::size_t>(audio_rows * h));
  Synth(&m->audio_heads, seed, kAudioHeadTensor, 0, audio_rows * h, false,
        0.0F, 0);
  m->final_norm.resize(static_cast<std::size_t>(h));
  Synth(&m->final_norm, seed, kFinalNormTensor, 0, h, true, norm_jitter, 0);
  m->layers.resize(static_cast<std::size_t>(c.layers));
  for (int64_t l = 0; l < c.layers; ++l) {
    Layer& L = m->layers[static_cast<std::size_t>(l)];
    L.qkv.resize(static_cast<std::size_t>((q_rows + 2 * kv_rows) * h));
    Synth(&L.qkv, seed, LayerTensor(l, 0), 0, q_rows * h, false, 0, 0);
    Synth(&L.qkv, seed, LayerTensor(l, 1), 0, kv_rows * h, false, 0,
          static_cast<std::size_t>(q_rows * h));
    Synth(&L.qkv, seed, LayerTensor(l, 2), 0, kv_rows * h, false, 0,
          static_cast<std::size_t>((q_rows + kv_rows) * h));
    L.output.resize(static_cast<std::size_t>(h * q_rows));
    Synth(&L.output, seed, LayerTensor(l, 3), 0, h * q_rows, false, 0, 0);
    L.gate_up.resize(static_cast<std::size_t>(2 * in * h));
    Synth(&L.gate_up, seed, LayerTensor(l, 4), 0, in * h, false, 0, 0);
    Synth(&L.gate_up, seed, LayerTensor(l, 5), 0, in * h, false, 0,
          static_cast<std::size_t>(in * h));
    L.down.resize(static_cast<std::size_t>(h * in));
    Synth(&L.down, seed, LayerTensor(l, 6), 0, h * in, false, 0, 0);
    L.input_norm.resize(static_cast<std::size_t>(h));
    Synth(&L.input_norm, seed, LayerTensor(l, 7), 0, h, true, norm_jitter, 0);
    L.post_norm.resize(static_cast<std::size_t>(h));
    Synth(&L.post_norm, seed, LayerTensor(l, 8), 0, h, true, norm_jitter, 0);
    L.q_norm.resize(static_cast<std::size_t>(d));
    Synth(&L.q_norm, seed, LayerTensor(l, 9), 0, d, true, norm_jitter, 0);
    L.k_norm.resize(static_cast<std::size_t>(d));
    Synth(&L.k_norm, seed, LayerTensor(l, 10), 0, d, true, norm_jitter, 0);
  }
  return m;
}

void* orc_model_from_host(const orc_config* config, const float* text,
                          const float* audio_embeddings,
                          const float* audio_heads, const float* final_norm,
                          const float* const* layers) {
  auto* m = new Model;
  m->config = *config;
  const orc_config& c = *config;
  const int64_t h = c.hidden_size, d = c.head_dim, in = c.intermediate_size;
  const int64_t q_rows = c.heads * d, kv_rows = c.kv_heads * d;
  const int64_t audio_rows = c.audio_codebooks * c.audio_vocab_size;
  auto copy = [](const float* src, int64_t n) {
    return std::vector<float>(src, src + n);
  };
  m->text = copy(text, c.vocab_size * h);
  m->audio_embeddings = copy(audio_embeddings, audio_rows * h);
  m->audio_heads = copy(audio_heads, audio_rows * h);
  RoundMatrix(&m->audio_heads);
  m->final_norm = copy(final_norm, h);
  m->layers.resize(static_cast<std::size_t>(c.layers));
  for (int64_t l = 0; l < c.layers; ++l) {
    const float* const* t = layers + l * kLayerTensors;
    Layer& L = m->layers[static_cast<std::size_t>(l)];
    L.qkv = copy(t[0], q_rows * h);
    L.qkv.insert(L.qkv.end(), t[1], t[1] + kv_rows * h);
    L.qkv.insert(L.qkv.end(), t[2], t[2] + kv_rows * h);
    RoundMatrix(&L.qkv);
    L.output = copy(t[3], h * q_rows);
    RoundMatrix(&L.output);
    L.gate_up = copy(t[4], in * h);
    L.gate_up.insert(L.gate_up.end(), t[5], t[5] + in * h);
    RoundMatrix(&L.gate_up);
    L.down = copy(t[6], h * in);
    RoundMatrix(&L.down);
    L.input_norm = copy(t[7], h);
    L.post_norm = copy(t[8], h);
    L.q_norm = copy(t[9], d);
    L.k_norm = copy(t[10], d);
  }
  return m;
}

void orc_model_destroy(void* model) { delete static_cast<Model*>(model); }

void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows,
                 int64_t width, float eps) {
  RmsNormRows(x, w, y, rows, width, eps);
}

void orc_linear(const float* x, const float* w, float* y, int64_t rows,
                int64_t in, int64_t out, int accumulate) {
  Gemm(x, w, y, rows, in, out, accumulate != 0);
}

void orc_qk_norm_rope(const float* qkv, const float* q_norm,
                      const float* k_norm, const int32_t* positions,
                      float* out, int64_t rows, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, float eps,
                      float theta) {
  QkNormRopeRows(qkv, q_norm, k_norm, positions, out, rows, heads, kv_heads,
                 head_dim, eps, theta);
}

void orc_attention(const float* qkv, float* out, int64_t rows, int64_t heads,
                   int64_t kv_heads, int64_t head_dim,
                   const int64_t* sequences, int64_t count, int round_p) {
  AttentionRows(qkv, out, rows, heads, kv_heads, head_dim, sequences, count,
                round_p != 0);
}

void orc_swiglu(const float* gate_up, float* out, int64_t rows, int64_t inter) {
  SwiGluRows(gate_up, out, rows, inter);
}

// Generator::Forward: the packed CFG batch of one ConditionalInput (cond
// rows [0, length), then its last target_frames again as the unconditional
// sequence), the layers, and the audio heads on the 2F target rows.
void orc_forward(void* handle, const int32_t* ids, int64_t length,
                 int64_t audio_start, int64_t target_frames, int emulate,
                 float* logits) {
  const Model& m = *static_cast<const Model*>(handle);
  const orc_config& c = m.config;
  const bool em = emulate != 0;
  const int64_t h = c.hidden_size, d = c.head_dim, in = c.intermediate_size;
  const int64_t frames = target_frames;
  const int64_t rows = length + frames;
  const int64_t codebooks = c.audio_codebooks, vocab = c.audio_vocab_size;
  const int64_t qkv_width = (c.heads + 2 * c.kv_heads) * d;
  // UploadIds: packed [codebook][row].
  std::vector<int32_t> packed(static_cast<std::size_t>(codebooks * rows));
  for (int64_t cb = 0; cb < codebooks; ++cb) {
    const int32_t* src = ids + cb * length;
    int32_t* dst = packed.data() + cb * rows;
    std::copy(src, src + length, dst);
    std::copy(src + length - frames, src + length, dst + length);
  }
  std::vector<int32_t> positions(static_cast<std::size_t>(rows));
  for (int64_t r = 0; r < length; ++r)
    positions[r] = static_cast<int32_t>(r);
  for (int64_t f = 0; f < frames; ++f)
    positions[length + f] = static_cast<int32_t>(f);
  // Embed.
  std::vector<float> hidden(static_cast<std::size_t>(rows * h));
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float* out = hidden.data() + r * h;
    if (r < audio_start) {
      m.TextRow(packed[r], out);
      continue;
    }
    for (int64_t k = 0; k < h; ++k) {
      float sum = 0.0F;
      for (int64_t cb = 0; cb < codebooks; ++cb) {
        const int64_t entry = cb * vocab + packed[cb * rows + r];
        sum += m.audio_embeddings[static_cast<std::size_t>(entry * h + k)];
      }
      out[k] = sum;
    }
  }
  std::vector<float> normed(static_cast<std::size_t>(rows * h));
  std::vector<float> qkv(static_cast<std::size_t>(rows * qkv_width));
  std::vector<float> roped(static_cast<std::size_t>(rows * qkv_width));
  std::vector<float> merged(static_cast<std::size_t>(rows * c.heads * d));
  std::vector<float> gate_up(static_cast<std::size_t>(rows * 2 * in));
  std::vector<float> activated(static_cast<std::size_t>(rows * in));
  const int64_t sequences[4] = {0, length, length, frames};
  for (const Layer& L : m.layers) {
    RmsNormRows(hidden.data(), L.input_norm.data(), normed.data(), rows, h,
                c.rms_norm_eps);
    RoundAll(normed.data(), rows * h, em);
    Gemm(normed.data(), L.qkv.data(), qkv.data(), rows, h, qkv_width, false);
    QkNormRopeRows(qkv.data(), L.q_norm.data(), L.k_norm.data(),
                   positions.data(), roped.data(), rows, c.heads, c.kv_heads,
                   d, c.rms_norm_eps, c.rope_theta);
    RoundAll(roped.data(), rows * qkv_width, em);
    AttentionRows(roped.data(), merged.data(), rows, c.heads, c.kv_heads, d,
                  sequences, 2, em);
    RoundAll(merged.data(), rows * c.heads * d, em);
    Gemm(merged.data(), L.output.data(), hidden.data(), rows, c.heads * d, h,
         true);
    RmsNormRows(hidden.data(), L.post_norm.data(), normed.data(), rows, h,
                c.rms_norm_eps);
    RoundAll(normed.data(), rows * h, em);
    Gemm(normed.data(), L.gate_up.data(), gate_up.data(), rows, h, 2 * in,
         false);
    SwiGluRows(gate_up.data(), activated.data(), rows, in);
    RoundAll(activated.data(), rows * in, em);
    Gemm(activated.data(), L.down.data(), hidden.data(), rows, in, h, true);
  }
  // GatherRows: conditional target rows, then the unconditional sequence.
  std::vector<float> final_rows(static_cast<std::size_t>(2 * frames * h));
  for (int64_t f = 0; f < frames; ++f) {
    std::memcpy(&final_rows[static_cast<std::size_t>(f * h)],
                &hidden[static_cast<std::size_t>((length - frames + f) * h)],
                static_cast<std::size_t>(h) * sizeof(float));
    std::memcpy(&final_rows[static_cast<std::size_t>((frames + f) * h)],
                &hidden[static_cast<std::size_t>((length + f) * h)],
                static_cast<std::size_t>(h) * sizeof(float));
  }
  std::vector<float> final_normed(final_rows.size());
  RmsNormRows(final_rows.data(), m.final_norm.data(), final_normed.data(),
              2 * frames, h, c.rms_norm_eps);
  RoundAll(final_normed.data(), 2 * frames * h, em);
  Gemm(final_normed.data(), m.audio_heads.data(), logits, 2 * frames, h,
       codebooks * vocab, false);
}

void orc_generate(void* handle, const int32_t* ids, int64_t length,
                  int64_t audio_start, int64_t target_frames, int emulate,
                  int64_t steps, float guidance, float t_shift,
                  float layer_penalty, float temperature, uint64_t seed,
                  int32_t* codes, int32_t* unmasked_at) {
  const Model& m = *static_cast<const Model*>(handle);
  const orc_config& c = m.config;
  const int64_t codebooks = c.audio_codebooks, vocab = c.audio_vocab_size;
  const int64_t frames = target_frames;
  const int64_t total = codebooks * frames;
  std::vector<int32_t> current(ids, ids + codebooks * length);
  std::vector<int64_t> schedule(static_cast<std::size_t>(steps));
  orc_unmask_schedule(total, steps, t_shift, schedule.data());
  for (int64_t i = 0; i < total; ++i) {
    codes[i] = static_cast<int32_t>(c.audio_mask_id);
    unmasked_at[i] = -1;
  }
  void* selector = orc_selector_create(layer_penalty, temperature, seed);
  std::vector<float> logits(static_cast<std::size_t>(2 * frames * codebooks * vocab));
  std::vector<int32_t> prediction(static_cast<std::size_t>(total));
  std::vector<float> confidence(static_cast<std::size_t>(total));
  std::vector<int64_t> chosen(static_cast<std::size_t>(total));
  for (int64_t step = 0; step < steps; ++step) {
    if (schedule[step] == 0)
      continue;
    orc_forward(handle, current.data(), length, audio_start, frames, emulate,
                logits.data());
    orc_score(logits.data(), frames, codebooks, vocab, c.audio_mask_id,
              guidance, prediction.data(), confidence.data());
    const int64_t n = orc_selector_fill(
        selector, schedule[step], codebooks, frames, prediction.data(),
        confidence.data(), c.audio_mask_id, codes, chosen.data());
    for (int64_t r = 0; r < n; ++r)
      unmasked_at[chosen[r]] = static_cast<int32_t>(step);
    for (int64_t cb = 0; cb < codebooks; ++cb)
      std::copy(codes + cb * frames, codes + cb * frames + frames,
                current.data() + cb * length + length - frames);
  }
  orc_selector_destroy(selector);
}

}  // extern "C"
