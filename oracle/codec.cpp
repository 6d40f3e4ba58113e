// ORACLE — test infrastructure, not product code (see oracle.h).
//
// CPU restatement of the reference's audio decoder (the DAC decoder of the
// Higgs Audio v2 tokenizer): Codec::Decode (codec.cpp:197-260), the
// convolution helpers of Codec::State (codec_state.hpp:232-300) and the
// element-wise kernels (kernels/codec_kernels.hip:11-84). Channel-major
// float32 signals between layers, as the reference stores them; every
// convolution sums in double, so the oracle sits closer to the exact result
// than either float32 implementation.
//
// Synthetic weights (the reference reads audio_tokenizer/model.safetensors,
// codec.cpp:95-148): every tensor is drawn from the same SplitMix64 normal
// as the generator's synthetic model (orc_synth_normal), under the tensor ids
// and scales of CodecTensorSpec below, and rounded to float. The product
// states the same specification in its own code.
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "oracle.h"

namespace {

constexpr int64_t kResidualKernel = 7;
constexpr int64_t kDilations[3] = {1, 3, 9};

// Value of element e of a synthetic codec tensor: float(scale * n), or
// float(exp(scale * n)) for the Snake alphas.
void Fill(uint64_t seed, uint64_t id, double scale, bool exponential,
          std::vector<float>* out, std::size_t count) {
  out->resize(count);
  for (std::size_t e = 0; e < count; ++e) {
    const double n = orc_synth_normal(seed, id, e);
    (*out)[e] = static_cast<float>(exponential ? std::exp(scale * n) : scale * n);
  }
}

struct Conv {  // PyTorch layout [out][in][kernel]
  std::vector<float> weight, bias;
  int64_t in = 0, out = 0, kernel = 1, dilation = 1;
};

struct Unit {
  std::vector<float> alpha1, alpha2;
  Conv conv1, conv2;
};

struct Block {
  std::vector<float> alpha;
  std::vector<float> up_weight, up_bias;  // [in][out][2 stride]
  int64_t in = 0, out = 0, stride = 0;
  Unit units[3];
};

struct Codec {
  orc_codec_config cfg;
  std::vector<float> tables;  // [codebooks][entries][hidden]
  std::vector<float> fc2_weight, fc2_bias;
  Conv input;
  std::vector<Block> blocks;
  std::vector<float> final_alpha;
  Conv output;
};

Conv MakeConv(uint64_t seed, uint64_t id, int64_t in, int64_t out,
              int64_t kernel, int64_t dilation, double gain) {
  Conv c;
  c.in = in;
  c.out = out;
  c.kernel = kernel;
  c.dilation = dilation;
  Fill(seed, id, gain / std::sqrt(static_cast<double>(in * kernel)), false,
       &c.weight, static_cast<std::size_t>(out * in * kernel));
  Fill(seed, id + 1, 0.01, false, &c.bias, static_cast<std::size_t>(out));
  return c;
}

void Convolve(const Conv& c, const float* x, int64_t length, float* y) {
  orc_conv1d(x, c.in, length, c.weight.data(), c.bias.data(), c.out, c.kernel,
             c.dilation, y);
}

}  // namespace

extern "C" {

void orc_snake(const float* x, int64_t channels, int64_t length,
               const float* alpha, float* y) {
  // kernels/codec_kernels.hip:11-25 (float32, as there).
  for (int64_t c = 0; c < channels; ++c) {
    const float a = alpha[c];
    for (int64_t t = 0; t < length; ++t) {
      const float v = x[c * length + t];
      const float s = std::sin(a * v);
      y[c * length + t] = v + (1.0F / (a + 1e-9F)) * (s * s);
    }
  }
}

void orc_conv1d(const float* x, int64_t in, int64_t length, const float* w,
                const float* b, int64_t out, int64_t kernel, int64_t dilation,
                float* y) {
  // nn.Conv1d with padding (kernel - 1) dilation / 2, stride 1: the
  // reference's Conv::Pad and State::Apply (codec_state.hpp:35, 232-250).
  const int64_t pad = (kernel - 1) * dilation / 2;
#pragma omp parallel
  {
    std::vector<double> acc(static_cast<std::size_t>(length));
#pragma omp for schedule(static)
    for (int64_t o = 0; o < out; ++o) {
      for (int64_t t = 0; t < length; ++t)
        acc[t] = b[o];
      for (int64_t i = 0; i < in; ++i) {
        const float* row = x + i * length;
        for (int64_t k = 0; k < kernel; ++k) {
          const double wv = w[(o * in + i) * kernel + k];
          const int64_t shift = k * dilation - pad;
          const int64_t lo = shift < 0 ? -shift : 0;
          const int64_t hi = length - (shift > 0 ? shift : 0);
          for (int64_t t = lo; t < hi; ++t)
            acc[t] += wv * row[t + shift];
        }
      }
      for (int64_t t = 0; t < length; ++t)
        y[o * length + t] = static_cast<float>(acc[t]);
    }
  }
}

void orc_conv_transpose1d(const float* x, int64_t in, int64_t length,
                          const float* w, const float* b, int64_t out,
                          int64_t stride, float* y) {
  // nn.ConvTranspose1d with kernel 2 stride, padding ceil(stride / 2) and
  // output_padding stride % 2, so the output has length * stride samples
  // (codec_state.hpp:272-285, the scatter definition: input j, tap k land
  // on output j stride + k - padding).
  const int64_t kernel = 2 * stride;
  const int64_t pad = (stride + 1) / 2;
  const int64_t length_out = length * stride;
#pragma omp parallel
  {
    std::vector<double> acc(static_cast<std::size_t>(length_out));
#pragma omp for schedule(static)
    for (int64_t o = 0; o < out; ++o) {
      for (int64_t t = 0; t < length_out; ++t)
        acc[t] = b[o];
      for (int64_t i = 0; i < in; ++i) {
        const float* row = x + i * length;
        for (int64_t k = 0; k < kernel; ++k) {
          const double wv = w[(i * out + o) * kernel + k];
          for (int64_t j = 0; j < length; ++j) {
            const int64_t t = j * stride + k - pad;
            if (t >= 0 && t < length_out)
              acc[t] += wv * row[j];
          }
        }
      }
      for (int64_t t = 0; t < length_out; ++t)
        y[o * length_out + t] = static_cast<float>(acc[t]);
    }
  }
}

void orc_codec_values(uint64_t seed, uint64_t tensor, uint64_t first,
                      int64_t count, double scale, int exponential,
                      float* out) {
  for (int64_t i = 0; i < count; ++i) {
    const double n = orc_synth_normal(seed, tensor, first + i);
    out[i] = static_cast<float>(exponential ? std::exp(scale * n) : scale * n);
  }
}

void* orc_codec_synthetic(const orc_codec_config* cfg, uint64_t seed) {
  auto* codec = new Codec();
  codec->cfg = *cfg;
  const int64_t C = cfg->codebooks, E = cfg->codebook_size,
                D = cfg->codebook_dim, H = cfg->hidden, Lat = cfg->latent;
  // RVQ decode tables: each codebook entry through its project_out
  // (codec.cpp:112-140): table = embed project_out^T, then + bias.
  codec->tables.resize(static_cast<std::size_t>(C * E * H));
  for (int64_t c = 0; c < C; ++c) {
    std::vector<float> embed, project, bias;
    Fill(seed, 1000 + 4 * c, 0.35, false, &embed, E * D);
    Fill(seed, 1001 + 4 * c, 1.0 / std::sqrt(static_cast<double>(D)), false,
         &project, H * D);
    Fill(seed, 1002 + 4 * c, 0.01, false, &bias, H);
    float* table = codec->tables.data() + c * E * H;
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < E; ++e)
      for (int64_t h = 0; h < H; ++h) {
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d)
          acc += static_cast<double>(embed[e * D + d]) * project[h * D + d];
        table[e * H + h] = static_cast<float>(acc) + bias[h];
      }
  }
  Fill(seed, 1100, 1.0 / std::sqrt(static_cast<double>(H)), false,
       &codec->fc2_weight, Lat * H);
  Fill(seed, 1101, 0.01, false, &codec->fc2_bias, Lat);
  int64_t channels = cfg->channels;
  codec->input = MakeConv(seed, 1102, Lat, channels, kResidualKernel, 1, 1.0);
  for (int64_t i = 0; i < cfg->blocks; ++i) {
    Block blk;
    const uint64_t id = 1200 + 32 * i;
    blk.in = channels;
    blk.out = channels / 2;
    blk.stride = cfg->ratios[i];
    Fill(seed, id, 0.1, true, &blk.alpha, channels);
    Fill(seed, id + 1, 1.0 / std::sqrt(static_cast<double>(2 * channels)),
         false, &blk.up_weight, channels * blk.out * 2 * blk.stride);
    Fill(seed, id + 2, 0.01, false, &blk.up_bias, blk.out);
    for (int u = 0; u < 3; ++u) {
      Unit& unit = blk.units[u];
      const uint64_t uid = id + 4 + 6 * u;
      Fill(seed, uid, 0.1, true, &unit.alpha1, blk.out);
      unit.conv1 = MakeConv(seed, uid + 1, blk.out, blk.out, kResidualKernel,
                            kDilations[u], 1.0);
      Fill(seed, uid + 3, 0.1, true, &unit.alpha2, blk.out);
      unit.conv2 = MakeConv(seed, uid + 4, blk.out, blk.out, 1, 1, 0.3);
    }
    codec->blocks.push_back(std::move(blk));
    channels /= 2;
  }
  Fill(seed, 1400, 0.1, true, &codec->final_alpha, channels);
  codec->output = MakeConv(seed, 1401, channels, 1, kResidualKernel, 1, 0.1);
  return codec;
}

void orc_codec_destroy(void* codec) { delete static_cast<Codec*>(codec); }

int64_t orc_codec_decode(const void* handle, const int32_t* codes,
                         int64_t frames, float* audio) {
  const Codec& s = *static_cast<const Codec*>(handle);
  const orc_codec_config& cfg = s.cfg;
  const int64_t H = cfg.hidden, Lat = cfg.latent, E = cfg.codebook_size;
  // Codebook sum (codec_kernels.hip:69-82): float, codebook order.
  std::vector<float> quantized(static_cast<std::size_t>(frames * H));
  for (int64_t f = 0; f < frames; ++f)
    for (int64_t h = 0; h < H; ++h) {
      float sum = 0.0F;
      for (int64_t c = 0; c < cfg.codebooks; ++c)
        sum += s.tables[(c * E + codes[c * frames + f]) * H + h];
      quantized[f * H + h] = sum;
    }
  // fc2 into channel-major [latent][frames], then its bias (codec.cpp:218-232).
  std::vector<float> x(static_cast<std::size_t>(Lat * frames));
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < Lat; ++o)
    for (int64_t f = 0; f < frames; ++f) {
      double acc = 0.0;
      for (int64_t h = 0; h < H; ++h)
        acc += static_cast<double>(s.fc2_weight[o * H + h]) * quantized[f * H + h];
      x[o * frames + f] = static_cast<float>(acc) + s.fc2_bias[o];
    }
  std::vector<float> a(static_cast<std::size_t>(s.input.out * frames));
  Convolve(s.input, x.data(), frames, a.data());
  int64_t length = frames;
  std::vector<float> snaked, up, y, z;
  for (const Block& blk : s.blocks) {
    // Snake, transposed convolution, three residual units
    // (codec_state.hpp:252-290).
    snaked.resize(a.size());
    orc_snake(a.data(), blk.in, length, blk.alpha.data(), snaked.data());
    up.resize(static_cast<std::size_t>(blk.out * length * blk.stride));
    orc_conv_transpose1d(snaked.data(), blk.in, length, blk.up_weight.data(),
                         blk.up_bias.data(), blk.out, blk.stride, up.data());
    length *= blk.stride;
    for (const Unit& unit : blk.units) {
      snaked.resize(up.size());
      y.resize(up.size());
      z.resize(up.size());
      orc_snake(up.data(), blk.out, length, unit.alpha1.data(), snaked.data());
      Convolve(unit.conv1, snaked.data(), length, y.data());
      orc_snake(y.data(), blk.out, length, unit.alpha2.data(), snaked.data());
      Convolve(unit.conv2, snaked.data(), length, z.data());
      for (std::size_t i = 0; i < up.size(); ++i)
        up[i] += z[i];
    }
    a.swap(up);
  }
  // Final Snake and output convolution; no tanh (codec.cpp:244-251).
  const int64_t channels = s.output.in;
  snaked.resize(a.size());
  orc_snake(a.data(), channels, length, s.final_alpha.data(), snaked.data());
  Convolve(s.output, snaked.data(), length, audio);
  return length;
}

}  // extern "C"
