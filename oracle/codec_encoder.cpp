// ORACLE — test infrastructure, not product code (see oracle.h).
//
// CPU restatement of the reference's audio encoder, Codec::Encode
// (codec_encoder.cpp:249-492) with its weight loading (codec_encoder.cpp:
// 74-240) and kernels (kernels/encoder_kernels.hip): the 24 kHz -> 16 kHz
// resampler (audio.cpp:265-322), HuBERT features averaged over the encoder
// input and every layer output, every semantic_stride-th frame, the
// semantic encoder, the DAC encoder, fc, and residual vector quantization
// (nearest codebook entry, then the entry's decoded row subtracted). Float32
// signals between layers; sums in double.
//
// Synthetic weights: every tensor from orc_synth_normal under the ids and
// scales set in orc_encoder_synthetic below (value = offset + scale n, Snake alphas
// exp(0.1 n)); the codebooks and project_out are the decoder's
// (oracle/codec.cpp). The product states the same specification.
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <vector>

#include "oracle.h"

namespace {

constexpr double kPi = 3.14159265358979323846;
constexpr int64_t kDilations[3] = {1, 3, 9};

std::vector<float> Values(uint64_t seed, uint64_t id, std::size_t count, double scale,
                          double offset = 0.0) {
  std::vector<float> v(count);
  for (std::size_t e = 0; e < count; ++e)
    v[e] = static_cast<float>(offset + scale * orc_synth_normal(seed, id, e));
  return v;
}

std::vector<float> Alphas(uint64_t seed, uint64_t id, std::size_t count) {
  std::vector<float> v(count);
  for (std::size_t e = 0; e < count; ++e)
    v[e] = static_cast<float>(std::exp(0.1 * orc_synth_normal(seed, id, e)));
  return v;
}

// Conv1d over channel-major x [in][length]: weight [out][in / groups][kernel].
std::vector<float> Conv(const std::vector<float>& x, int64_t in, int64_t length,
                        const std::vector<float>& w, const float* bias, int64_t out,
                        int64_t kernel, int64_t stride, int64_t dilation, int64_t pad,
                        int64_t groups, int64_t* length_out) {
  const int64_t lo = (length + 2 * pad - dilation * (kernel - 1) - 1) / stride + 1;
  *length_out = lo;
  const int64_t in_g = in / groups, out_g = out / groups;
  std::vector<float> y(static_cast<std::size_t>(out * lo));
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < out; ++o) {
    const int64_t g = o / out_g;
    std::vector<double> acc(static_cast<std::size_t>(lo), bias != nullptr ? bias[o] : 0.0);
    for (int64_t i = 0; i < in_g; ++i) {
      const float* row = &x[static_cast<std::size_t>((g * in_g + i) * length)];
      for (int64_t k = 0; k < kernel; ++k) {
        const double wv = w[static_cast<std::size_t>((o * in_g + i) * kernel + k)];
        for (int64_t t = 0; t < lo; ++t) {
          const int64_t s = t * stride + k * dilation - pad;
          if (s >= 0 && s < length)
            acc[t] += wv * row[s];
        }
      }
    }
    for (int64_t t = 0; t < lo; ++t)
      y[static_cast<std::size_t>(o * lo + t)] = static_cast<float>(acc[t]);
  }
  return y;
}

// y [rows][out] = x [rows][in] W^T + b.
std::vector<float> Linear(const std::vector<float>& x, int64_t rows, int64_t in,
                          const std::vector<float>& w, const std::vector<float>& b,
                          int64_t out) {
  std::vector<float> y(static_cast<std::size_t>(rows * out));
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t o = 0; o < out; ++o) {
      double acc = b[o];
      for (int64_t i = 0; i < in; ++i)
        acc += static_cast<double>(x[r * in + i]) * w[o * in + i];
      y[r * out + o] = static_cast<float>(acc);
    }
  return y;
}

void LayerNormRows(std::vector<float>* x, int64_t rows, int64_t width,
                   const std::vector<float>& w, const std::vector<float>& b, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    float* row = &(*x)[r * width];
    double mean = 0.0, var = 0.0;
    for (int64_t j = 0; j < width; ++j)
      mean += row[j];
    mean /= width;
    for (int64_t j = 0; j < width; ++j)
      var += (row[j] - mean) * (row[j] - mean);
    const double inv = 1.0 / std::sqrt(var / width + eps);
    for (int64_t j = 0; j < width; ++j)
      row[j] = static_cast<float>((row[j] - mean) * inv * w[j] + b[j]);
  }
}

float Gelu(float x) {
  return static_cast<float>(0.5 * x * (1.0 + std::erf(x / std::sqrt(2.0))));
}
float Elu(float x) { return x > 0.0F ? x : std::expm1(x); }
float Snake(float v, float a) {
  const float s = std::sin(a * v);
  return v + (1.0F / (a + 1e-9F)) * (s * s);
}

std::vector<float> Transpose(const std::vector<float>& x, int64_t rows, int64_t cols) {
  std::vector<float> y(x.size());
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      y[c * rows + r] = x[r * cols + c];
  return y;
}

struct Layer {
  std::vector<float> qkv_w, qkv_b, out_w, out_b, ln_w, ln_b, ff1_w, ff1_b, ff2_w, ff2_b,
      fln_w, fln_b;
};
struct ResUnit {
  std::vector<float> alpha1, c1_w, c1_b, alpha2, c2_w, c2_b;
};
struct AcousticBlock {
  ResUnit units[3];
  std::vector<float> alpha, down_w, down_b;
  int64_t channels = 0, stride = 1;
};

struct Encoder {
  orc_encoder_config c;
  std::vector<std::vector<float>> feat_w;
  std::vector<float> gn_w, gn_b, proj_ln_w, proj_ln_b, proj_w, proj_b, pos_w, pos_b,
      enc_ln_w, enc_ln_b;
  std::vector<Layer> layers;
  std::vector<float> sem_in_w;
  std::vector<float> sem_c1[2][2], sem_c2[2][2], sem_block_w[2], sem_block_b[2];
  std::vector<float> ac_in_w, ac_in_b, ac_alpha, ac_out_w, ac_out_b;
  std::vector<AcousticBlock> blocks;
  std::vector<float> fc_w, fc_b;
  std::vector<std::vector<float>> pin_w, pin_b, embed, table;  // table [E][H]
};

int64_t Hidden(const orc_encoder_config& c) { return c.width + c.latent; }

}  // namespace

extern "C" {

int64_t orc_resample(const float* samples, int64_t length, uint32_t from_rate,
                     uint32_t to_rate, float* output) {
  // audio.cpp:265-322: torchaudio's sinc_interp_hann kernel (6 zero
  // crossings, rolloff 0.99) built in float32 operation by operation, then
  // one strided correlation per output phase, summed in double.
  if (from_rate == to_rate) {
    std::copy(samples, samples + length, output);
    return length;
  }
  constexpr int kZero = 6;
  const uint32_t gcd = std::gcd(from_rate, to_rate);
  const int64_t from = from_rate / gcd, to = to_rate / gcd;
  const double base = static_cast<double>(std::min(from, to)) * 0.99;
  const auto width = static_cast<int64_t>(std::ceil(kZero * static_cast<double>(from) / base));
  const int64_t taps = 2 * width + from;
  std::vector<float> kernel(static_cast<std::size_t>(to * taps));
  const auto base_f = static_cast<float>(base);
  const auto pi_f = static_cast<float>(kPi);
  const auto scale_f = static_cast<float>(base / static_cast<double>(from));
  for (int64_t phase = 0; phase < to; ++phase)
    for (int64_t tap = 0; tap < taps; ++tap) {
      const float index = static_cast<float>(tap - width) / static_cast<float>(from);
      float t = static_cast<float>(-phase) / static_cast<float>(to) + index;
      t *= base_f;
      t = std::clamp(t, -static_cast<float>(kZero), static_cast<float>(kZero));
      const float cosine = std::cos(t * pi_f / static_cast<float>(kZero) / 2.0F);
      const float window = cosine * cosine;
      t *= pi_f;
      const float sinc = t == 0.0F ? 1.0F : std::sin(t) / t;
      kernel[phase * taps + tap] = sinc * (window * scale_f);
    }
  const auto out_length = static_cast<int64_t>(
      std::ceil(static_cast<double>(to) * static_cast<double>(length) / static_cast<double>(from)));
  for (int64_t out = 0; out < out_length; ++out) {
    const int64_t block = out / to, phase = out % to;
    const float* w = &kernel[phase * taps];
    const int64_t origin = block * from - width;
    double sum = 0.0;
    for (int64_t tap = std::max<int64_t>(0, -origin); tap < std::min(taps, length - origin); ++tap)
      sum += static_cast<double>(w[tap]) * samples[origin + tap];
    output[out] = static_cast<float>(sum);
  }
  return out_length;
}

void* orc_encoder_synthetic(const orc_encoder_config* config, uint64_t seed) {
  auto* e = new Encoder();
  const orc_encoder_config& c = *config;
  e->c = c;
  const int64_t W = c.width, I = c.intermediate, H = Hidden(c), D = c.codebook_dim,
                E = c.codebook_size;
  int64_t in = 1;
  for (int64_t i = 0; i < c.feat_layers; ++i) {
    e->feat_w.push_back(Values(seed, 2000 + i, c.conv_dim[i] * in * c.conv_kernel[i],
                               1.0 / std::sqrt(static_cast<double>(in * c.conv_kernel[i]))));
    in = c.conv_dim[i];
  }
  e->gn_w = Values(seed, 2010, c.conv_dim[0], 0.1, 1.0);
  e->gn_b = Values(seed, 2011, c.conv_dim[0], 0.1);
  e->proj_ln_w = Values(seed, 2012, in, 0.1, 1.0);
  e->proj_ln_b = Values(seed, 2013, in, 0.1);
  e->proj_w = Values(seed, 2014, W * in, 1.0 / std::sqrt(static_cast<double>(in)));
  e->proj_b = Values(seed, 2015, W, 0.01);
  {
    // Weight norm over (out, in) per tap folded: w = g v / |v|.
    const int64_t K = c.pos_kernel, Wg = W / c.pos_groups;
    const auto g = Values(seed, 2016, K, 0.1, 1.0);
    const auto v = Values(seed, 2017, W * Wg * K, 1.0);
    std::vector<double> norm(K, 0.0);
    for (int64_t o = 0; o < W; ++o)
      for (int64_t i = 0; i < Wg; ++i)
        for (int64_t k = 0; k < K; ++k)
          norm[k] += static_cast<double>(v[(o * Wg + i) * K + k]) * v[(o * Wg + i) * K + k];
    e->pos_w.resize(v.size());
    for (int64_t o = 0; o < W; ++o)
      for (int64_t i = 0; i < Wg; ++i)
        for (int64_t k = 0; k < K; ++k)
          e->pos_w[(o * Wg + i) * K + k] =
              static_cast<float>(g[k] * v[(o * Wg + i) * K + k] / std::sqrt(norm[k]));
    e->pos_b = Values(seed, 2018, W, 0.01);
  }
  e->enc_ln_w = Values(seed, 2019, W, 0.1, 1.0);
  e->enc_ln_b = Values(seed, 2020, W, 0.1);
  for (int64_t l = 0; l < c.layers; ++l) {
    const uint64_t id = 2100 + 16 * l;
    Layer L;
    const double sw = 1.0 / std::sqrt(static_cast<double>(W));
    // q, k, v projections stacked (codec_encoder.cpp:35-52).
    for (int p = 0; p < 3; ++p) {
      const auto w = Values(seed, id + 2 * p, W * W, sw);
      const auto b = Values(seed, id + 2 * p + 1, W, 0.01);
      L.qkv_w.insert(L.qkv_w.end(), w.begin(), w.end());
      L.qkv_b.insert(L.qkv_b.end(), b.begin(), b.end());
    }
    L.out_w = Values(seed, id + 6, W * W, sw);
    L.out_b = Values(seed, id + 7, W, 0.01);
    L.ln_w = Values(seed, id + 8, W, 0.1, 1.0);
    L.ln_b = Values(seed, id + 9, W, 0.1);
    L.ff1_w = Values(seed, id + 10, I * W, sw);
    L.ff1_b = Values(seed, id + 11, I, 0.01);
    L.ff2_w = Values(seed, id + 12, W * I, 0.5 / std::sqrt(static_cast<double>(I)));
    L.ff2_b = Values(seed, id + 13, W, 0.01);
    L.fln_w = Values(seed, id + 14, W, 0.1, 1.0);
    L.fln_b = Values(seed, id + 15, W, 0.1);
    e->layers.push_back(std::move(L));
  }
  const double s3 = 1.0 / std::sqrt(3.0 * W);
  e->sem_in_w = Values(seed, 2400, W * W * 3, s3);
  for (int b = 0; b < 2; ++b) {
    for (int u = 0; u < 2; ++u) {
      e->sem_c1[b][u] = Values(seed, 2410 + 10 * b + 2 * u, W * W * 3, s3);
      e->sem_c2[b][u] = Values(seed, 2411 + 10 * b + 2 * u, W * W,
                               0.3 / std::sqrt(static_cast<double>(W)));
    }
    e->sem_block_w[b] = Values(seed, 2450 + 2 * b, W * W * 3, s3);
    e->sem_block_b[b] = Values(seed, 2451 + 2 * b, W, 0.01);
  }
  e->ac_in_w = Values(seed, 2500, c.enc_channels * 7, 1.0 / std::sqrt(7.0));
  e->ac_in_b = Values(seed, 2501, c.enc_channels, 0.01);
  int64_t ch = c.enc_channels;
  for (int64_t i = 0; i < c.blocks; ++i) {
    const uint64_t id = 2600 + 32 * i;
    AcousticBlock blk;
    blk.channels = ch;
    blk.stride = c.ratios[i];
    for (int u = 0; u < 3; ++u) {
      const uint64_t uid = id + 4 + 6 * u;
      ResUnit& r = blk.units[u];
      r.alpha1 = Alphas(seed, uid, ch);
      r.c1_w = Values(seed, uid + 1, ch * ch * 7, 1.0 / std::sqrt(7.0 * ch));
      r.c1_b = Values(seed, uid + 2, ch, 0.01);
      r.alpha2 = Alphas(seed, uid + 3, ch);
      r.c2_w = Values(seed, uid + 4, ch * ch, 0.3 / std::sqrt(static_cast<double>(ch)));
      r.c2_b = Values(seed, uid + 5, ch, 0.01);
    }
    blk.alpha = Alphas(seed, id, ch);
    blk.down_w = Values(seed, id + 1, 2 * ch * ch * 2 * blk.stride,
                        1.0 / std::sqrt(2.0 * ch * blk.stride));
    blk.down_b = Values(seed, id + 2, 2 * ch, 0.01);
    e->blocks.push_back(std::move(blk));
    ch *= 2;
  }
  e->ac_alpha = Alphas(seed, 2800, ch);
  e->ac_out_w = Values(seed, 2801, c.latent * ch * 3, 1.0 / std::sqrt(3.0 * ch));
  e->ac_out_b = Values(seed, 2802, c.latent, 0.01);
  e->fc_w = Values(seed, 2810, H * H, 1.0 / std::sqrt(static_cast<double>(H)));
  e->fc_b = Values(seed, 2811, H, 0.01);
  for (int64_t q = 0; q < c.codebooks; ++q) {
    e->pin_w.push_back(Values(seed, 2900 + 2 * q, D * H, 1.0 / std::sqrt(static_cast<double>(H))));
    e->pin_b.push_back(Values(seed, 2901 + 2 * q, D, 0.01));
    // The decoder's codebook and project_out (oracle/codec.cpp).
    e->embed.push_back(Values(seed, 1000 + 4 * q, E * D, 0.35));
    const auto pw = Values(seed, 1001 + 4 * q, H * D, 1.0 / std::sqrt(static_cast<double>(D)));
    const auto pb = Values(seed, 1002 + 4 * q, H, 0.01);
    std::vector<float> table(static_cast<std::size_t>(E * H));
    for (int64_t en = 0; en < E; ++en)
      for (int64_t h = 0; h < H; ++h) {
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d)
          acc += static_cast<double>(e->embed.back()[en * D + d]) * pw[h * D + d];
        table[en * H + h] = static_cast<float>(acc) + pb[h];
      }
    e->table.push_back(std::move(table));
  }
  return e;
}

void orc_encoder_destroy(void* encoder) { delete static_cast<Encoder*>(encoder); }

int64_t orc_encoder_encode(const void* handle, const float* samples, int64_t length,
                           int32_t* codes, float* semantic_out, float* acoustic_out,
                           float* embeddings_out) {
  const Encoder& e = *static_cast<const Encoder*>(handle);
  const orc_encoder_config& c = e.c;
  const int64_t W = c.width, H = Hidden(c), D = c.codebook_dim, E = c.codebook_size;
  if (length <= 0 || length % c.frame_samples != 0)
    return -1;
  const int64_t count = length / c.frame_samples;
  // ---- HuBERT at the semantic rate, 160 samples of padding each side.
  std::vector<float> x(static_cast<std::size_t>(
      std::ceil(static_cast<double>(c.semantic_rate) * length / c.sample_rate)));
  x.resize(orc_resample(samples, length, c.sample_rate, c.semantic_rate, x.data()));
  x.insert(x.begin(), 160, 0.0F);
  x.insert(x.end(), 160, 0.0F);
  int64_t len = static_cast<int64_t>(x.size()), in = 1;
  for (int64_t i = 0; i < c.feat_layers; ++i) {
    int64_t lo = 0;
    x = Conv(x, in, len, e.feat_w[i], nullptr, c.conv_dim[i], c.conv_kernel[i],
             c.conv_stride[i], 1, 0, 1, &lo);
    len = lo;
    in = c.conv_dim[i];
    if (i == 0) {
      // GroupNorm with one group per channel, eps 1e-5, then GELU.
      for (int64_t ch = 0; ch < in; ++ch) {
        float* row = &x[ch * len];
        double mean = 0.0, var = 0.0;
        for (int64_t t = 0; t < len; ++t)
          mean += row[t];
        mean /= len;
        for (int64_t t = 0; t < len; ++t)
          var += (row[t] - mean) * (row[t] - mean);
        const double inv = 1.0 / std::sqrt(var / len + 1e-5);
        for (int64_t t = 0; t < len; ++t)
          row[t] = Gelu(static_cast<float>((row[t] - mean) * inv * e.gn_w[ch] + e.gn_b[ch]));
      }
    } else {
      for (float& v : x)
        v = Gelu(v);
    }
  }
  const int64_t steps = len;
  std::vector<float> rows = Transpose(x, in, steps);  // [steps][features]
  LayerNormRows(&rows, steps, in, e.proj_ln_w, e.proj_ln_b, c.eps);
  std::vector<float> state = Linear(rows, steps, in, e.proj_w, e.proj_b, W);  // [steps][W]
  {
    // Grouped positional convolution (padding K / 2, the extra output of an
    // even kernel dropped), GELU, added to the states, then LayerNorm.
    const std::vector<float> cm = Transpose(state, steps, W);
    int64_t lo = 0;
    std::vector<float> pos = Conv(cm, W, steps, e.pos_w, e.pos_b.data(), W, c.pos_kernel, 1, 1,
                                  c.pos_kernel / 2, c.pos_groups, &lo);
    for (int64_t ch = 0; ch < W; ++ch)
      for (int64_t t = 0; t < steps; ++t)
        state[t * W + ch] += Gelu(pos[ch * lo + t]);
    LayerNormRows(&state, steps, W, e.enc_ln_w, e.enc_ln_b, c.eps);
  }
  std::vector<double> mean(state.begin(), state.end());
  const int64_t hd = W / c.heads;
  const double scale = 1.0 / std::sqrt(static_cast<double>(hd));
  for (const Layer& L : e.layers) {
    const std::vector<float> qkv = Linear(state, steps, W, L.qkv_w, L.qkv_b, 3 * W);
    std::vector<float> att(static_cast<std::size_t>(steps * W));
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t h = 0; h < c.heads; ++h)
      for (int64_t q = 0; q < steps; ++q) {
        std::vector<double> s(static_cast<std::size_t>(steps));
        double m = -1e300;
        for (int64_t k = 0; k < steps; ++k) {
          double acc = 0.0;
          for (int64_t d = 0; d < hd; ++d)
            acc += static_cast<double>(qkv[q * 3 * W + h * hd + d]) *
                   qkv[k * 3 * W + W + h * hd + d];
          s[k] = acc * scale;
          m = std::max(m, s[k]);
        }
        double sum = 0.0;
        for (int64_t k = 0; k < steps; ++k) {
          s[k] = std::exp(s[k] - m);
          sum += s[k];
        }
        for (int64_t d = 0; d < hd; ++d) {
          double acc = 0.0;
          for (int64_t k = 0; k < steps; ++k)
            acc += s[k] * qkv[k * 3 * W + 2 * W + h * hd + d];
          att[q * W + h * hd + d] = static_cast<float>(acc / sum);
        }
      }
    const std::vector<float> o = Linear(att, steps, W, L.out_w, L.out_b, W);
    for (std::size_t i = 0; i < state.size(); ++i)
      state[i] += o[i];
    LayerNormRows(&state, steps, W, L.ln_w, L.ln_b, c.eps);
    std::vector<float> ff = Linear(state, steps, W, L.ff1_w, L.ff1_b, c.intermediate);
    for (float& v : ff)
      v = Gelu(v);
    const std::vector<float> f2 = Linear(ff, steps, c.intermediate, L.ff2_w, L.ff2_b, W);
    for (std::size_t i = 0; i < state.size(); ++i)
      state[i] += f2[i];
    LayerNormRows(&state, steps, W, L.fln_w, L.fln_b, c.eps);
    for (std::size_t i = 0; i < state.size(); ++i)
      mean[i] += state[i];
  }
  if (steps < count * c.semantic_stride)
    return -2;
  // Every semantic_stride-th frame of the average, channel-major [W][count].
  std::vector<float> sem(static_cast<std::size_t>(W * count));
  for (int64_t f = 0; f < count; ++f)
    for (int64_t ch = 0; ch < W; ++ch) {
      const float v = static_cast<float>(mean[f * c.semantic_stride * W + ch] /
                                         static_cast<double>(c.layers + 1));
      sem[ch * count + f] = v;
      if (semantic_out != nullptr)
        semantic_out[f * W + ch] = v;
    }
  // ---- Semantic encoder (codec_encoder.cpp:400-416).
  int64_t lo = 0;
  std::vector<float> s = Conv(sem, W, count, e.sem_in_w, nullptr, W, 3, 1, 1, 1, 1, &lo);
  for (int b = 0; b < 2; ++b) {
    for (int u = 0; u < 2; ++u) {
      std::vector<float> a(s.size());
      for (std::size_t i = 0; i < s.size(); ++i)
        a[i] = Elu(s[i]);
      std::vector<float> y = Conv(a, W, count, e.sem_c1[b][u], nullptr, W, 3, 1, 1, 1, 1, &lo);
      for (float& v : y)
        v = Elu(v);
      const std::vector<float> z = Conv(y, W, count, e.sem_c2[b][u], nullptr, W, 1, 1, 1, 0, 1, &lo);
      for (std::size_t i = 0; i < s.size(); ++i)
        s[i] += z[i];
    }
    s = Conv(s, W, count, e.sem_block_w[b], e.sem_block_b[b].data(), W, 3, 1, 1, 1, 1, &lo);
  }
  // ---- DAC encoder on the 24 kHz samples.
  std::vector<float> a(samples, samples + length);
  a = Conv(a, 1, length, e.ac_in_w, e.ac_in_b.data(), c.enc_channels, 7, 1, 1, 3, 1, &lo);
  int64_t cur = length;
  for (const AcousticBlock& blk : e.blocks) {
    const int64_t ch = blk.channels;
    for (int u = 0; u < 3; ++u) {
      const ResUnit& r = blk.units[u];
      std::vector<float> t(a.size());
      for (int64_t i = 0; i < ch; ++i)
        for (int64_t j = 0; j < cur; ++j)
          t[i * cur + j] = Snake(a[i * cur + j], r.alpha1[i]);
      std::vector<float> y = Conv(t, ch, cur, r.c1_w, r.c1_b.data(), ch, 7, 1, kDilations[u],
                                  3 * kDilations[u], 1, &lo);
      for (int64_t i = 0; i < ch; ++i)
        for (int64_t j = 0; j < cur; ++j)
          y[i * cur + j] = Snake(y[i * cur + j], r.alpha2[i]);
      const std::vector<float> z = Conv(y, ch, cur, r.c2_w, r.c2_b.data(), ch, 1, 1, 1, 0, 1, &lo);
      for (std::size_t i = 0; i < a.size(); ++i)
        a[i] += z[i];
    }
    for (int64_t i = 0; i < ch; ++i)
      for (int64_t j = 0; j < cur; ++j)
        a[i * cur + j] = Snake(a[i * cur + j], blk.alpha[i]);
    a = Conv(a, ch, cur, blk.down_w, blk.down_b.data(), 2 * ch, 2 * blk.stride, blk.stride, 1,
             (blk.stride + 1) / 2, 1, &lo);
    cur = lo;
  }
  const int64_t chf = c.enc_channels << c.blocks;
  for (int64_t i = 0; i < chf; ++i)
    for (int64_t j = 0; j < cur; ++j)
      a[i * cur + j] = Snake(a[i * cur + j], e.ac_alpha[i]);
  if (cur != count)
    return -3;
  a = Conv(a, chf, cur, e.ac_out_w, e.ac_out_b.data(), c.latent, 3, 1, 1, 1, 1, &lo);
  if (acoustic_out != nullptr)
    for (int64_t f = 0; f < count; ++f)
      for (int64_t i = 0; i < c.latent; ++i)
        acoustic_out[f * c.latent + i] = a[i * count + f];
  // ---- Joint [acoustic; semantic] per frame, fc, then the RVQ.
  std::vector<float> joint(static_cast<std::size_t>(count * H));
  for (int64_t f = 0; f < count; ++f) {
    for (int64_t i = 0; i < c.latent; ++i)
      joint[f * H + i] = a[i * count + f];
    for (int64_t i = 0; i < W; ++i)
      joint[f * H + c.latent + i] = s[i * count + f];
  }
  std::vector<float> residual = Linear(joint, count, H, e.fc_w, e.fc_b, H);
  if (embeddings_out != nullptr)
    std::copy(residual.begin(), residual.end(), embeddings_out);
  for (int64_t q = 0; q < c.codebooks; ++q) {
    const std::vector<float> p = Linear(residual, count, H, e.pin_w[q], e.pin_b[q], D);
    for (int64_t f = 0; f < count; ++f) {
      double pp = 0.0;
      for (int64_t d = 0; d < D; ++d)
        pp += static_cast<double>(p[f * D + d]) * p[f * D + d];
      double best = -1e300;
      int32_t best_e = 0;
      for (int64_t en = 0; en < E; ++en) {
        double dot = 0.0, ee = 0.0;
        for (int64_t d = 0; d < D; ++d) {
          dot += static_cast<double>(p[f * D + d]) * e.embed[q][en * D + d];
          ee += static_cast<double>(e.embed[q][en * D + d]) * e.embed[q][en * D + d];
        }
        const double dist = -((pp - 2.0 * dot) + ee);
        if (dist > best) {
          best = dist;
          best_e = static_cast<int32_t>(en);
        }
      }
      codes[q * count + f] = best_e;
      for (int64_t h = 0; h < H; ++h)
        residual[f * H + h] -= e.table[q][best_e * H + h];
    }
  }
  return count;
}

}  // extern "C"
