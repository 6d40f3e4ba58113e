// The audio encoder engine and its C ABI (include/omnivoice_codec_mi355x.h):
// 24 kHz reference audio to RVQ codes through the Higgs Audio v2
// tokenizer's encoder, float32 on the GPU.
//
// Reference counterparts: LoadEncoder (codec_encoder.cpp:74-240) and
// Codec::Encode (codec_encoder.cpp:249-492), with the resampler of
// audio.cpp:265-322.
//
// Layout: every signal is channel-major ([channels][positions]), HuBERT's
// hidden states included ([width][steps]), so that every GEMM-shaped layer
// is a convolution on the fp32 matrix cores (codec_kernels.hip):
//  * a linear layer is a one-tap convolution;
//  * a strided, long or grouped convolution runs over im2col columns;
//  * attention runs per head as two batched one-tap convolutions: the
//    transposed scores S^T[key][query] = K_h^T Q_h (K_h as the weights), a
//    softmax down each column, and the context O_h = V_h P^T (V^T as the
//    weights, P^T as the input);
//  * GELU, ELU and Snake are applied by the epilogue of the producing
//    convolution, residual additions by its accumulation.
// The mean of HuBERT's states is summed in double by the LayerNorm that
// produces each state. The nearest-entry search compares distances in
// double.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "../../include/omnivoice_codec_mi355x.h"
#include "checkpoint.hpp"
#include "codec.hpp"
#include "codec_common.hpp"
#include "device.hpp"
#include "encoder.hpp"
#include "host.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kDilations[3] = {1, 3, 9};
constexpr int kWavePad = 160;  // zeros each side of HuBERT's input
constexpr double kPi = 3.14159265358979323846;
constexpr std::int64_t kPartialFloats = std::int64_t{8} << 20;  // 32 MiB

// Synthetic encoder specification (tensor id, scale, offset), as for the
// decoder (codec.cpp): value float(offset + scale n), alphas float(exp(0.1 n)),
// n = SynthNormal(seed, id, element in the checkpoint tensor's shape).
//   semantic_model.feature_extractor.conv_layers.i.conv.weight  2000 + i  1/sqrt(in k)
//   ....conv_layers.0.layer_norm.weight, .bias        2010, 2011  0.1 (+1), 0.1
//   semantic_model.feature_projection.layer_norm      2012, 2013  0.1 (+1), 0.1
//   semantic_model.feature_projection.projection      2014, 2015  1/sqrt(in), 0.01
//   ....pos_conv_embed.conv original0, original1, bias 2016, 2017, 2018  0.1 (+1), 1, 0.01
//   semantic_model.encoder.layer_norm                 2019, 2020  0.1 (+1), 0.1
//   ....encoder.layers.l. (base 2100 + 16 l): q, k, v _proj +0..+5 (1/sqrt(W), 0.01),
//     out_proj +6, +7 (1/sqrt(W), 0.01), layer_norm +8, +9, intermediate_dense
//     +10, +11 (1/sqrt(W), 0.01), output_dense +12, +13 (0.5/sqrt(I), 0.01),
//     final_layer_norm +14, +15
//   encoder_semantic.conv.weight                      2400        1/sqrt(3W)
//   ....conv_blocks.b.res_units.u.conv1, conv2        2410 + 10b + 2u, +1  1/sqrt(3W), 0.3/sqrt(W)
//   ....conv_blocks.b.conv.weight, .bias              2450 + 2b, +1  1/sqrt(3W), 0.01
//   acoustic_encoder.conv1.weight, .bias              2500, 2501  1/sqrt(7), 0.01
//   acoustic_encoder.block.i (base 2600 + 32i): snake1.alpha +0, conv1 +1, +2
//     (1/sqrt(2 C s), 0.01), res_unit(u+1) at +4 + 6u: snake1.alpha +0, conv1
//     +1, +2 (1/sqrt(7C), 0.01), snake2.alpha +3, conv2 +4, +5 (0.3/sqrt(C), 0.01)
//   acoustic_encoder.snake1.alpha, conv2              2800, 2801, 2802  1/sqrt(3C), 0.01
//   fc.weight, .bias                                  2810, 2811  1/sqrt(H), 0.01
//   quantizer.quantizers.q.project_in                 2900 + 2q, +1  1/sqrt(H), 0.01
//   quantizer.quantizers.q.codebook.embed, project_out: the decoder's ids
// (LayerNorm weights carry the offset 1).

// A linear map on the matrix cores: w [in][out] (the im2col layout for a
// convolution), bias [out] or none.
struct Dense {
  DeviceBuffer<float> w, b;
  int in = 0, out = 0;
  bool bias = false;
};

void MakeDense(const std::vector<float>& w, const std::vector<float>* b, int out, int in,
               int kernel, Dense* d) {
  Upload(d->w, ConvLayout(w, out, in * kernel, 1));
  d->bias = b != nullptr;
  if (b != nullptr)
    Upload(d->b, *b);
  d->in = in * kernel;
  d->out = out;
}

struct Layer {
  Dense qkv, out, ff1, ff2;
  DeviceBuffer<float> ln_w, ln_b, fln_w, fln_b;
};
struct Conv7 {
  DeviceBuffer<float> w, b;  // [7][in][out], [out]
  int in = 0, out = 0, dilation = 1;
};
struct Unit {
  DeviceBuffer<float> alpha1, alpha2;
  Conv7 conv1;
  Dense conv2;
};
struct Block {
  Unit units[3];
  DeviceBuffer<float> alpha;
  Dense down;
  int channels = 0, stride = 1;
};
struct Stage {
  Dense project;
  DeviceBuffer<float> embed, table;  // [entries][dim], [entries][hidden]
  DeviceBuffer<double> norms;        // [entries]
};

// Shapes of one encode of `length` samples.
struct Plan {
  int64_t length = 0, frames = 0;
  int64_t resampled = 0;           // samples at the semantic rate
  std::vector<int64_t> features;   // HuBERT feature lengths after each conv
  int64_t steps = 0;               // HuBERT frames
  std::vector<int64_t> acoustic;   // DAC lengths after each block
};

}  // namespace

class EncoderEngine {
 public:
  EncoderEngine(const ovc_encoder_config& cfg, std::uint64_t seed, const SafetensorsFile* file);
  ~EncoderEngine() {
    if (stream_ != nullptr)
      (void)hipStreamDestroy(stream_);
  }
  int64_t Frames(int64_t length) const { return length / cfg_.frame_samples; }
  void Encode(const float* samples, int64_t length, std::int32_t* codes, float* semantic,
              float* acoustic, float* embeddings);
  void EncodeDevice(const float* samples, int64_t length, std::int32_t* codes,
                    hipStream_t stream);
  void Profile(int64_t length, int64_t repeats, std::map<std::string, KernelStat>* stats);

 private:
  Plan MakePlan(int64_t length) const;
  void Reserve(const Plan& plan);
  void Enqueue(const float* samples, const Plan& plan, std::int32_t* codes, hipStream_t stream,
               Profiler* prof);
  // y = pre(W x + b) (or y += ...), y_act = out_act(...), over `positions`
  // columns; `batches` independent maps with the given strides.
  struct Gemm {
    const Dense* d = nullptr;
    const float* x = nullptr;
    float* y = nullptr;
    float* y_act = nullptr;
    const float* alpha_out = nullptr;
    int positions = 0, pre_act = kActNone, out_act = kActNone;
    bool accumulate = false;
  };
  void RunGemm(const Gemm& g, hipStream_t stream, Profiler* prof, const char* name);
  void RunIm2col(const float* x, int channels, int len_in, int kernel, int stride, int pad,
                 int positions, int act, hipStream_t stream, Profiler* prof, const char* name);
  void RunConv7(const Conv7& c, const float* x, int length, float* y, float* y_act,
                const float* alpha_out, bool accumulate, hipStream_t stream, Profiler* prof,
                const char* name);

  ovc_encoder_config cfg_;
  int W_ = 0, H_ = 0;
  hipStream_t stream_ = nullptr;
  // resampler bank
  int from_ = 1, to_ = 1, width_ = 0, taps_ = 0;
  DeviceBuffer<float> bank_;
  // HuBERT
  std::vector<std::unique_ptr<Dense>> features_;
  DeviceBuffer<float> gn_w_, gn_b_, proj_ln_w_, proj_ln_b_, enc_ln_w_, enc_ln_b_;
  Dense projection_, position_;  // position_: [groups][in_g K][out_g]
  std::vector<std::unique_ptr<Layer>> layers_;
  // semantic encoder
  Dense sem_in_, sem_c1_[2][2], sem_c2_[2][2], sem_block_[2];
  // DAC encoder
  Conv7 ac_in_;
  std::vector<std::unique_ptr<Block>> blocks_;
  DeviceBuffer<float> ac_alpha_;
  Dense ac_out_, fc_;
  std::vector<std::unique_ptr<Stage>> stages_;
  // work buffers
  DeviceBuffer<float> samples_, wave_, fa_, fb_, cols_, tmp_, h_, qkv_, scores_, vt_, ctx_, ff_;
  DeviceBuffer<double> sum_;
  // Split-K workspace of the thin GEMMs (HuBERT at short lengths, the
  // semantic encoder, the quantizer's projections).
  DeviceBuffer<float> partial_;
  DeviceBuffer<float> sem_, st_, t1_, x_, xa_, ya_, joint_, emb_, resid_, proj_;
  DeviceBuffer<std::int32_t> codes_;
};

EncoderEngine::EncoderEngine(const ovc_encoder_config& cfg, std::uint64_t seed,
                             const SafetensorsFile* file)
    : cfg_(cfg) {
  const int W = static_cast<int>(cfg.width), I = static_cast<int>(cfg.intermediate);
  const int lat = static_cast<int>(cfg.latent), H = W + lat;
  const int D = static_cast<int>(cfg.codebook_dim), E = static_cast<int>(cfg.codebook_size);
  W_ = W;
  H_ = H;
  Check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  const Source src(seed, file);

  // ---- resampler bank (audio.cpp:265-322): torchaudio's sinc_interp_hann
  // kernel, 6 zero crossings, rolloff 0.99, evaluated in float32 in the same
  // order of operations so the bank matches the reference's bit for bit.
  if (cfg.sample_rate == cfg.semantic_rate) {
    // no resampling: one tap of weight 1
    Upload(bank_, std::vector<float>{1.0F});
    taps_ = 1;
  } else {
    const auto gcd = std::gcd(cfg.sample_rate, cfg.semantic_rate);
    from_ = static_cast<int>(cfg.sample_rate / gcd);
    to_ = static_cast<int>(cfg.semantic_rate / gcd);
    constexpr int kZeros = 6;
    const double base = static_cast<double>(std::min(from_, to_)) * 0.99;
    width_ = static_cast<int>(std::ceil(kZeros * static_cast<double>(from_) / base));
    taps_ = 2 * width_ + from_;
    std::vector<float> bank(static_cast<std::size_t>(to_) * taps_);
    const auto base_f = static_cast<float>(base);
    const auto pi_f = static_cast<float>(kPi);
    const auto scale_f = static_cast<float>(base / from_);
    for (int ph = 0; ph < to_; ++ph)
      for (int k = 0; k < taps_; ++k) {
        float t = static_cast<float>(-ph) / static_cast<float>(to_) +
                  static_cast<float>(k - width_) / static_cast<float>(from_);
        t = std::clamp(t * base_f, -static_cast<float>(kZeros), static_cast<float>(kZeros));
        const float c = std::cos(t * pi_f / static_cast<float>(kZeros) / 2.0F);
        t *= pi_f;
        bank[static_cast<std::size_t>(ph) * taps_ + k] =
            (t == 0.0F ? 1.0F : std::sin(t) / t) * ((c * c) * scale_f);
      }
    Upload(bank_, bank);
  }

  // ---- HuBERT (codec_encoder.cpp:74-165)
  int in = 1;
  for (int i = 0; i < cfg.feature_layers; ++i) {
    const int out = static_cast<int>(cfg.conv_dim[i]), k = static_cast<int>(cfg.conv_kernel[i]);
    const auto w = src.Get("semantic_model.feature_extractor.conv_layers." + std::to_string(i) +
                               ".conv.weight",
                           {out, in, k}, 2000 + i, 1.0 / std::sqrt(double(in) * k));
    features_.push_back(std::make_unique<Dense>());
    MakeDense(w, nullptr, out, in, k, features_.back().get());
    in = out;
  }
  const int c0 = static_cast<int>(cfg.conv_dim[0]);
  Upload(gn_w_, src.Get("semantic_model.feature_extractor.conv_layers.0.layer_norm.weight",
                        {c0}, 2010, 0.1, false, 1.0));
  Upload(gn_b_, src.Get("semantic_model.feature_extractor.conv_layers.0.layer_norm.bias", {c0},
                        2011, 0.1));
  Upload(proj_ln_w_, src.Get("semantic_model.feature_projection.layer_norm.weight", {in}, 2012,
                             0.1, false, 1.0));
  Upload(proj_ln_b_, src.Get("semantic_model.feature_projection.layer_norm.bias", {in}, 2013,
                             0.1));
  {
    const auto w = src.Get("semantic_model.feature_projection.projection.weight", {W, in}, 2014,
                           1.0 / std::sqrt(double(in)));
    const auto b = src.Get("semantic_model.feature_projection.projection.bias", {W}, 2015, 0.01);
    MakeDense(w, &b, W, in, 1, &projection_);
  }
  {
    // Weight norm over (out, in) for every tap, folded at load (in double):
    // w = g v / |v|.
    const int K = static_cast<int>(cfg.pos_kernel), G = static_cast<int>(cfg.pos_groups);
    const int Wg = W / G;
    const std::string p = "semantic_model.encoder.pos_conv_embed.conv.";
    const auto g = src.Get(p + "parametrizations.weight.original0", {1, 1, K}, 2016, 0.1, false,
                           1.0);
    const auto v = src.Get(p + "parametrizations.weight.original1", {W, Wg, K}, 2017, 1.0);
    std::vector<double> norm(K, 0.0);
    for (std::size_t e = 0; e < v.size(); ++e)
      norm[e % K] += static_cast<double>(v[e]) * v[e];
    // per group: [Wg in x K taps][Wg out]
    std::vector<float> w(v.size());
    for (int o = 0; o < W; ++o)
      for (int i = 0; i < Wg; ++i)
        for (int k = 0; k < K; ++k) {
          const int grp = o / Wg, oo = o % Wg;
          const std::size_t src_at = (static_cast<std::size_t>(o) * Wg + i) * K + k;
          w[(static_cast<std::size_t>(grp) * Wg * K + static_cast<std::size_t>(i) * K + k) * Wg +
            oo] = static_cast<float>(g[k] * v[src_at] / std::sqrt(norm[k]));
        }
    Upload(position_.w, w);
    Upload(position_.b, src.Get(p + "bias", {W}, 2018, 0.01));
    position_.bias = true;
    position_.in = Wg * K;
    position_.out = Wg;
  }
  Upload(enc_ln_w_, src.Get("semantic_model.encoder.layer_norm.weight", {W}, 2019, 0.1, false,
                            1.0));
  Upload(enc_ln_b_, src.Get("semantic_model.encoder.layer_norm.bias", {W}, 2020, 0.1));
  const double sw = 1.0 / std::sqrt(double(W));
  for (int l = 0; l < cfg.layers; ++l) {
    const std::string p = "semantic_model.encoder.layers." + std::to_string(l) + ".";
    const std::uint64_t id = 2100 + 16 * static_cast<std::uint64_t>(l);
    layers_.push_back(std::make_unique<Layer>());
    Layer& L = *layers_.back();
    std::vector<float> qkv_w, qkv_b;
    const char* names[3] = {"q_proj", "k_proj", "v_proj"};
    for (int j = 0; j < 3; ++j) {
      const auto w = src.Get(p + "attention." + names[j] + ".weight", {W, W}, id + 2 * j, sw);
      const auto b = src.Get(p + "attention." + names[j] + ".bias", {W}, id + 2 * j + 1, 0.01);
      qkv_w.insert(qkv_w.end(), w.begin(), w.end());
      qkv_b.insert(qkv_b.end(), b.begin(), b.end());
    }
    MakeDense(qkv_w, &qkv_b, 3 * W, W, 1, &L.qkv);
    auto dense = [&](const std::string& name, int out, int inn, std::uint64_t wid, double scale,
                     Dense* d) {
      const auto w = src.Get(p + name + ".weight", {out, inn}, wid, scale);
      const auto b = src.Get(p + name + ".bias", {out}, wid + 1, 0.01);
      MakeDense(w, &b, out, inn, 1, d);
    };
    dense("attention.out_proj", W, W, id + 6, sw, &L.out);
    Upload(L.ln_w, src.Get(p + "layer_norm.weight", {W}, id + 8, 0.1, false, 1.0));
    Upload(L.ln_b, src.Get(p + "layer_norm.bias", {W}, id + 9, 0.1));
    dense("feed_forward.intermediate_dense", I, W, id + 10, sw, &L.ff1);
    dense("feed_forward.output_dense", W, I, id + 12, 0.5 / std::sqrt(double(I)), &L.ff2);
    Upload(L.fln_w, src.Get(p + "final_layer_norm.weight", {W}, id + 14, 0.1, false, 1.0));
    Upload(L.fln_b, src.Get(p + "final_layer_norm.bias", {W}, id + 15, 0.1));
  }

  // ---- semantic encoder (codec_encoder.cpp:166-187)
  const double s3 = 1.0 / std::sqrt(3.0 * W);
  MakeDense(src.Get("encoder_semantic.conv.weight", {W, W, 3}, 2400, s3), nullptr, W, W, 3,
            &sem_in_);
  for (int b = 0; b < 2; ++b) {
    const std::string p = "encoder_semantic.conv_blocks." + std::to_string(b);
    for (int u = 0; u < 2; ++u) {
      const std::string q = p + ".res_units." + std::to_string(u);
      const std::uint64_t id = 2410 + 10 * b + 2 * u;
      MakeDense(src.Get(q + ".conv1.weight", {W, W, 3}, id, s3), nullptr, W, W, 3,
                &sem_c1_[b][u]);
      MakeDense(src.Get(q + ".conv2.weight", {W, W, 1}, id + 1, 0.3 / std::sqrt(double(W))),
                nullptr, W, W, 1, &sem_c2_[b][u]);
    }
    const auto bias = src.Get(p + ".conv.bias", {W}, 2451 + 2 * b, 0.01);
    MakeDense(src.Get(p + ".conv.weight", {W, W, 3}, 2450 + 2 * b, s3), &bias, W, W, 3,
              &sem_block_[b]);
  }

  // ---- DAC encoder (codec_encoder.cpp:188-223)
  const int ce = static_cast<int>(cfg.enc_channels);
  {
    const auto w = src.Get("acoustic_encoder.conv1.weight", {ce, 1, 7}, 2500, 1.0 / std::sqrt(7.0));
    Upload(ac_in_.w, ConvLayout(w, ce, 1, 7));
    Upload(ac_in_.b, src.Get("acoustic_encoder.conv1.bias", {ce}, 2501, 0.01));
    ac_in_.in = 1;
    ac_in_.out = ce;
  }
  int ch = ce;
  for (int i = 0; i < cfg.blocks; ++i) {
    auto blk = std::make_unique<Block>();
    const std::string p = "acoustic_encoder.block." + std::to_string(i);
    const std::uint64_t id = 2600 + 32 * static_cast<std::uint64_t>(i);
    const int s = static_cast<int>(cfg.ratios[i]);
    blk->channels = ch;
    blk->stride = s;
    for (int u = 0; u < 3; ++u) {
      const std::string name = p + ".res_unit" + std::to_string(u + 1);
      const std::uint64_t uid = id + 4 + 6 * static_cast<std::uint64_t>(u);
      Unit& unit = blk->units[u];
      Upload(unit.alpha1, src.Get(name + ".snake1.alpha", {1, ch, 1}, uid, 0.1, true));
      const auto w1 = src.Get(name + ".conv1.weight", {ch, ch, 7}, uid + 1,
                              1.0 / std::sqrt(7.0 * ch));
      Upload(unit.conv1.w, ConvLayout(w1, ch, ch, 7));
      Upload(unit.conv1.b, src.Get(name + ".conv1.bias", {ch}, uid + 2, 0.01));
      unit.conv1.in = unit.conv1.out = ch;
      unit.conv1.dilation = kDilations[u];
      Upload(unit.alpha2, src.Get(name + ".snake2.alpha", {1, ch, 1}, uid + 3, 0.1, true));
      const auto b2 = src.Get(name + ".conv2.bias", {ch}, uid + 5, 0.01);
      MakeDense(src.Get(name + ".conv2.weight", {ch, ch, 1}, uid + 4, 0.3 / std::sqrt(double(ch))),
                &b2, ch, ch, 1, &unit.conv2);
    }
    Upload(blk->alpha, src.Get(p + ".snake1.alpha", {1, ch, 1}, id, 0.1, true));
    const auto bd = src.Get(p + ".conv1.bias", {2 * ch}, id + 2, 0.01);
    MakeDense(src.Get(p + ".conv1.weight", {2 * ch, ch, 2 * s}, id + 1,
                      1.0 / std::sqrt(2.0 * ch * s)),
              &bd, 2 * ch, ch, 2 * s, &blk->down);
    blocks_.push_back(std::move(blk));
    ch *= 2;
  }
  Upload(ac_alpha_, src.Get("acoustic_encoder.snake1.alpha", {1, ch, 1}, 2800, 0.1, true));
  {
    const auto b = src.Get("acoustic_encoder.conv2.bias", {lat}, 2802, 0.01);
    MakeDense(src.Get("acoustic_encoder.conv2.weight", {lat, ch, 3}, 2801,
                      1.0 / std::sqrt(3.0 * ch)),
              &b, lat, ch, 3, &ac_out_);
  }
  {
    const auto b = src.Get("fc.bias", {H}, 2811, 0.01);
    MakeDense(src.Get("fc.weight", {H, H}, 2810, 1.0 / std::sqrt(double(H))), &b, H, H, 1, &fc_);
  }

  // ---- quantizer (codec_encoder.cpp:224-240): project_in, the codebook,
  // its squared norms (double) and the decoded rows embed project_out^T +
  // bias (double sums, rounded once).
  std::vector<std::thread> workers;
  stages_.resize(static_cast<std::size_t>(cfg.codebooks));
  std::vector<std::vector<float>> pw(cfg.codebooks), pb(cfg.codebooks), emb(cfg.codebooks),
      qw(cfg.codebooks), qb(cfg.codebooks);
  for (int q = 0; q < cfg.codebooks; ++q) {
    const std::string p = "quantizer.quantizers." + std::to_string(q);
    pw[q] = src.Get(p + ".project_in.weight", {D, H}, 2900 + 2 * q, 1.0 / std::sqrt(double(H)));
    pb[q] = src.Get(p + ".project_in.bias", {D}, 2901 + 2 * q, 0.01);
    emb[q] = src.Get(p + ".codebook.embed", {E, D}, 1000 + 4 * q, 0.35);
    qw[q] = src.Get(p + ".project_out.weight", {H, D}, 1001 + 4 * q, 1.0 / std::sqrt(double(D)));
    qb[q] = src.Get(p + ".project_out.bias", {H}, 1002 + 4 * q, 0.01);
  }
  std::vector<std::vector<float>> tables(cfg.codebooks);
  std::vector<std::vector<double>> norms(cfg.codebooks);
  for (int q = 0; q < cfg.codebooks; ++q)
    workers.emplace_back([&, q] {
      tables[q].resize(static_cast<std::size_t>(E) * H);
      norms[q].assign(E, 0.0);
      for (int e = 0; e < E; ++e) {
        const float* row = &emb[q][static_cast<std::size_t>(e) * D];
        for (int d = 0; d < D; ++d)
          norms[q][e] += static_cast<double>(row[d]) * row[d];
        for (int h = 0; h < H; ++h) {
          double acc = 0.0;
          for (int d = 0; d < D; ++d)
            acc += static_cast<double>(row[d]) * qw[q][static_cast<std::size_t>(h) * D + d];
          tables[q][static_cast<std::size_t>(e) * H + h] = static_cast<float>(acc) + qb[q][h];
        }
      }
    });
  for (auto& w : workers)
    w.join();
  for (int q = 0; q < cfg.codebooks; ++q) {
    auto st = std::make_unique<Stage>();
    MakeDense(pw[q], &pb[q], D, H, 1, &st->project);
    Upload(st->embed, emb[q]);
    Upload(st->table, tables[q]);
    Upload(st->norms, norms[q]);
    stages_[q] = std::move(st);
  }
  partial_.Reserve(kPartialFloats);
  Check(hipDeviceSynchronize(), "encoder upload");
}

Plan EncoderEngine::MakePlan(int64_t length) const {
  Require(length > 0 && length % cfg_.frame_samples == 0,
          "reference audio must be a whole number of frames");
  Plan p;
  p.length = length;
  p.frames = length / cfg_.frame_samples;
  p.resampled = cfg_.sample_rate == cfg_.semantic_rate ? length
                                                       : (to_ * length + from_ - 1) / from_;
  int64_t len = p.resampled + 2 * kWavePad;
  for (int i = 0; i < cfg_.feature_layers; ++i) {
    len = len < cfg_.conv_kernel[i] ? 0 : (len - cfg_.conv_kernel[i]) / cfg_.conv_stride[i] + 1;
    Require(len >= 1, "reference audio is too short for the semantic encoder");
    p.features.push_back(len);
  }
  p.steps = len;
  Require(p.steps >= p.frames * cfg_.semantic_stride,
          "reference audio is too short for the semantic encoder");
  int64_t cur = length;
  for (int i = 0; i < cfg_.blocks; ++i) {
    const int64_t s = cfg_.ratios[i], pad = (s + 1) / 2;
    cur = (cur + 2 * pad - 2 * s) / s + 1;
    p.acoustic.push_back(cur);
  }
  Require(cur == p.frames, "acoustic and semantic frame counts differ");
  return p;
}

void EncoderEngine::Reserve(const Plan& p) {
  const int64_t W = W_, T = p.steps, F = p.frames;
  int64_t feat = 0, cols = 0;
  int64_t in = 1, len = p.resampled + 2 * kWavePad;
  for (int i = 0; i < cfg_.feature_layers; ++i) {
    cols = std::max(cols, in * cfg_.conv_kernel[i] * p.features[i]);
    in = cfg_.conv_dim[i];
    len = p.features[i];
    feat = std::max(feat, in * len);
  }
  cols = std::max(cols, W * cfg_.pos_kernel * T);
  cols = std::max(cols, 3 * W * F);
  int64_t ch = cfg_.enc_channels, cur = p.length, dac = ch * cur;
  for (int i = 0; i < cfg_.blocks; ++i) {
    const int64_t s = cfg_.ratios[i];
    cols = std::max(cols, ch * 2 * s * p.acoustic[i]);
    ch *= 2;
    cur = p.acoustic[i];
    dac = std::max(dac, ch * cur);
  }
  cols = std::max(cols, 3 * ch * F);
  const int64_t scores = cfg_.heads * T * T;
  const int64_t hid = std::max<int64_t>(in, W) * T;
  const int64_t limit = int64_t{1} << 31;
  for (const int64_t n : {feat, cols, dac, scores, hid, cfg_.intermediate * T, 3 * W * T,
                          p.resampled + 2 * kWavePad})
    Require(n < limit, "reference audio too long: a buffer passes 2^31 elements");
  auto grow = [](auto& buffer, int64_t n) {
    if (buffer.size() < static_cast<std::size_t>(n))
      buffer.Reserve(static_cast<std::size_t>(n));
  };
  grow(samples_, p.length);
  grow(wave_, p.resampled + 2 * kWavePad);
  grow(fa_, feat);
  grow(fb_, feat);
  grow(cols_, cols);
  grow(tmp_, hid);
  grow(h_, W * T);
  grow(qkv_, 3 * W * T);
  grow(scores_, scores);
  grow(vt_, W * T);
  grow(ctx_, W * T);
  grow(ff_, cfg_.intermediate * T);
  grow(sum_, W * T);
  grow(sem_, W * F);
  grow(st_, W * F);
  grow(t1_, W * F);
  grow(x_, dac);
  grow(xa_, dac);
  grow(ya_, dac);
  grow(joint_, H_ * F);
  grow(emb_, H_ * F);
  grow(resid_, H_ * F);
  grow(proj_, cfg_.codebook_dim * F);
  grow(codes_, cfg_.codebooks * F);
}

void EncoderEngine::RunGemm(const Gemm& g, hipStream_t stream, Profiler* prof,
                            const char* name) {
  ConvParams p{};
  p.x = g.x;
  p.w = g.d->w.get();
  p.bias = g.d->bias ? g.d->b.get() : nullptr;
  p.y = g.y;
  p.y_act = g.y_act;
  p.alpha_out = g.alpha_out;
  p.cin = g.d->in;
  p.len_in = g.positions;
  p.cout = g.d->out;
  p.len_out = g.positions;
  p.taps = 1;
  p.phases = 1;
  p.positions = g.positions;
  p.out_stride = 1;
  p.accumulate = g.accumulate ? 1 : 0;
  p.pre_act = g.pre_act;
  p.out_act = g.out_act;
  p.partial = partial_.get();
  p.partial_capacity = kPartialFloats;
  const double flops = 2.0 * p.cin * p.cout * static_cast<double>(p.positions);
  const double outs = (g.y != nullptr) + (g.y_act != nullptr) + (g.accumulate ? 1 : 0);
  const double bytes =
      4.0 * (static_cast<double>(p.cin) * p.positions + outs * p.cout * p.positions +
             static_cast<double>(p.cin) * p.cout);
  auto launch = [&] { LaunchConv(p, stream); };
  if (prof != nullptr)
    prof->Run(name, flops, bytes, launch);
  else
    launch();
}

void EncoderEngine::RunIm2col(const float* x, int channels, int len_in, int kernel, int stride,
                              int pad, int positions, int act, hipStream_t stream,
                              Profiler* prof, const char* name) {
  Im2colParams p{x, cols_.get(), channels, len_in, kernel, stride, 1, pad, positions, act};
  const double bytes = 8.0 * channels * static_cast<double>(kernel) * positions;
  auto launch = [&] { LaunchIm2col(p, stream); };
  if (prof != nullptr)
    prof->Run(name, 0.0, bytes, launch);
  else
    launch();
}

void EncoderEngine::RunConv7(const Conv7& c, const float* x, int length, float* y, float* y_act,
                             const float* alpha_out, bool accumulate, hipStream_t stream,
                             Profiler* prof, const char* name) {
  ConvParams p{};
  p.x = x;
  p.w = c.w.get();
  p.bias = c.b.get();
  p.y = y;
  p.y_act = y_act;
  p.alpha_out = alpha_out;
  p.cin = c.in;
  p.len_in = length;
  p.cout = c.out;
  p.len_out = length;
  p.taps = 7;
  p.phases = 1;
  p.positions = length;
  p.out_stride = 1;
  p.accumulate = accumulate ? 1 : 0;
  p.partial = partial_.get();
  p.partial_capacity = kPartialFloats;
  for (int k = 0; k < 7; ++k)
    p.offsets[0][k] = (k - 3) * c.dilation;
  const double flops = 2.0 * c.out * static_cast<double>(length) * c.in * 7;
  const double outs = (y != nullptr) + (y_act != nullptr) + (accumulate ? 1 : 0);
  const double bytes = 4.0 * length * (c.in + c.out * outs) + 28.0 * c.in * c.out;
  auto launch = [&] { LaunchConv(p, stream); };
  if (prof != nullptr)
    prof->Run(name, flops, bytes, launch);
  else
    launch();
}

void EncoderEngine::Enqueue(const float* samples, const Plan& plan, std::int32_t* codes,
                            hipStream_t stream, Profiler* prof) {
  auto run = [&](const char* name, double flops, double bytes, auto&& launch) {
    if (prof != nullptr)
      prof->Run(name, flops, bytes, launch);
    else
      launch();
  };
  const int W = W_, H = H_, T = static_cast<int>(plan.steps), F = static_cast<int>(plan.frames);
  const int heads = static_cast<int>(cfg_.heads), hd = W / heads;
  const int L = static_cast<int>(plan.length);

  // ---- HuBERT features at the semantic rate (codec_encoder.cpp:265-330)
  ResampleParams rp{samples, bank_.get(), wave_.get(), L, from_, to_, width_, taps_,
                    static_cast<int>(plan.resampled), kWavePad};
  run("enc_resample", 2.0 * taps_ * plan.resampled, 4.0 * (L + plan.resampled + 2 * kWavePad),
      [&] { LaunchResample(rp, stream); });
  const float* x = wave_.get();
  int in = 1, len = static_cast<int>(plan.resampled + 2 * kWavePad);
  float* a = fa_.get();
  float* b = fb_.get();
  for (int i = 0; i < cfg_.feature_layers; ++i) {
    const int k = static_cast<int>(cfg_.conv_kernel[i]), s = static_cast<int>(cfg_.conv_stride[i]);
    const int out_len = static_cast<int>(plan.features[i]);
    RunIm2col(x, in, len, k, s, 0, out_len, kActNone, stream, prof, "enc_feature_im2col");
    Gemm g;
    g.d = features_[i].get();
    g.x = cols_.get();
    g.y = b;
    g.positions = out_len;
    g.pre_act = i == 0 ? kActNone : kActGelu;
    RunGemm(g, stream, prof, "enc_feature_conv");
    in = features_[i]->out;
    len = out_len;
    if (i == 0)
      run("enc_group_norm", 0.0, 12.0 * in * len, [&] {
        LaunchGroupNormGelu(b, gn_w_.get(), gn_b_.get(), in, len, 1e-5F, stream);
      });
    std::swap(a, b);
    x = a;
  }
  const float eps = static_cast<float>(cfg_.eps);
  auto norm = [&](const float* src, float* dst, const DeviceBuffer<float>& w,
                  const DeviceBuffer<float>& bb, int channels, int sum_mode) {
    ColumnNormParams np{src, dst, w.get(), bb.get(), sum_.get(), channels, T, sum_mode, eps};
    run("enc_layer_norm", 0.0, (12.0 + 8.0 * (sum_mode != 0)) * channels * T,
        [&] { LaunchColumnNorm(np, stream); });
  };
  norm(x, tmp_.get(), proj_ln_w_, proj_ln_b_, in, 0);
  {
    Gemm g;
    g.d = &projection_;
    g.x = tmp_.get();
    g.y = h_.get();
    g.positions = T;
    RunGemm(g, stream, prof, "enc_projection");
  }
  {
    // Grouped positional convolution: padding K / 2, the first T outputs,
    // GELU, added to the states.
    const int K = static_cast<int>(cfg_.pos_kernel), G = static_cast<int>(cfg_.pos_groups);
    const int Wg = W / G;
    RunIm2col(h_.get(), W, T, K, 1, K / 2, T, kActNone, stream, prof, "enc_pos_im2col");
    ConvParams p{};
    p.x = cols_.get();
    p.w = position_.w.get();
    p.bias = position_.b.get();
    p.y = h_.get();
    p.cin = Wg * K;
    p.len_in = T;
    p.cout = Wg;
    p.len_out = T;
    p.taps = 1;
    p.phases = 1;
    p.positions = T;
    p.out_stride = 1;
    p.accumulate = 1;
    p.pre_act = kActGelu;
    p.batches = G;
    p.partial = partial_.get();
    p.partial_capacity = kPartialFloats;
    p.x_batch = static_cast<int64_t>(Wg) * K * T;
    p.w_batch = static_cast<int64_t>(Wg) * K * Wg;
    p.b_batch = Wg;
    p.y_batch = static_cast<int64_t>(Wg) * T;
    run("enc_pos_conv", 2.0 * W * Wg * K * static_cast<double>(T),
        4.0 * (static_cast<double>(W) * K * T + 2.0 * W * T + static_cast<double>(W) * Wg * K),
        [&] { LaunchConv(p, stream); });
  }
  norm(h_.get(), h_.get(), enc_ln_w_, enc_ln_b_, W, 1);
  for (const auto& layer : layers_) {
    const Layer& ly = *layer;
    Gemm g;
    g.d = &ly.qkv;
    g.x = h_.get();
    g.y = qkv_.get();
    g.positions = T;
    RunGemm(g, stream, prof, "enc_qkv");
    {
      // S^T[key][query] = sum_d K[d][key] Q[d][query], per head.
      ConvParams p{};
      p.x = qkv_.get();
      p.w = qkv_.get() + static_cast<std::size_t>(W) * T;
      p.y = scores_.get();
      p.cin = hd;
      p.len_in = T;
      p.cout = T;
      p.len_out = T;
      p.ldw = T;
      p.taps = 1;
      p.phases = 1;
      p.positions = T;
      p.out_stride = 1;
      p.batches = heads;
      p.partial = partial_.get();
      p.partial_capacity = kPartialFloats;
      p.x_batch = static_cast<int64_t>(hd) * T;
      p.w_batch = static_cast<int64_t>(hd) * T;
      p.y_batch = static_cast<int64_t>(T) * T;
      run("enc_scores", 2.0 * heads * hd * static_cast<double>(T) * T,
          4.0 * (2.0 * W * T + static_cast<double>(heads) * T * T),
          [&] { LaunchConv(p, stream); });
    }
    run("enc_softmax", 0.0, 8.0 * heads * static_cast<double>(T) * T, [&] {
      LaunchColumnSoftmax(scores_.get(), heads, T, T,
                          static_cast<float>(1.0 / std::sqrt(static_cast<double>(hd))), stream);
    });
    run("enc_transpose", 0.0, 8.0 * W * static_cast<double>(T), [&] {
      LaunchTranspose(qkv_.get() + 2 * static_cast<std::size_t>(W) * T, W, T, T, vt_.get(),
                      stream);
    });
    {
      // O[d][query] = sum_key V[d][key] P[query][key], per head.
      ConvParams p{};
      p.x = scores_.get();
      p.w = vt_.get();
      p.y = ctx_.get();
      p.cin = T;
      p.len_in = T;
      p.cout = hd;
      p.len_out = T;
      p.ldw = W;
      p.taps = 1;
      p.phases = 1;
      p.positions = T;
      p.out_stride = 1;
      p.batches = heads;
      p.partial = partial_.get();
      p.partial_capacity = kPartialFloats;
      p.x_batch = static_cast<int64_t>(T) * T;
      p.w_batch = hd;
      p.y_batch = static_cast<int64_t>(hd) * T;
      run("enc_context", 2.0 * heads * hd * static_cast<double>(T) * T,
          4.0 * (static_cast<double>(heads) * T * T + 2.0 * W * T),
          [&] { LaunchConv(p, stream); });
    }
    g = Gemm();
    g.d = &ly.out;
    g.x = ctx_.get();
    g.y = h_.get();
    g.positions = T;
    g.accumulate = true;
    RunGemm(g, stream, prof, "enc_out_proj");
    norm(h_.get(), h_.get(), ly.ln_w, ly.ln_b, W, 0);
    g = Gemm();
    g.d = &ly.ff1;
    g.x = h_.get();
    g.y = ff_.get();
    g.positions = T;
    g.pre_act = kActGelu;
    RunGemm(g, stream, prof, "enc_ff1");
    g = Gemm();
    g.d = &ly.ff2;
    g.x = ff_.get();
    g.y = h_.get();
    g.positions = T;
    g.accumulate = true;
    RunGemm(g, stream, prof, "enc_ff2");
    norm(h_.get(), h_.get(), ly.fln_w, ly.fln_b, W, 2);
  }
  const int stride = static_cast<int>(cfg_.semantic_stride);
  run("enc_pick", 0.0, 12.0 * W * F, [&] {
    LaunchPickFrames(sum_.get(), W, T, stride, F, 1.0 / static_cast<double>(cfg_.layers + 1),
                     sem_.get(), stream);
  });

  // ---- semantic encoder (codec_encoder.cpp:400-416)
  const int lat = static_cast<int>(cfg_.latent);
  float* semantic_rows = joint_.get() + static_cast<std::size_t>(lat) * F;
  RunIm2col(sem_.get(), W, F, 3, 1, 1, F, kActNone, stream, prof, "enc_sem_im2col");
  {
    Gemm g;
    g.d = &sem_in_;
    g.x = cols_.get();
    g.y = st_.get();
    g.positions = F;
    RunGemm(g, stream, prof, "enc_sem_conv");
  }
  for (int bl = 0; bl < 2; ++bl) {
    for (int u = 0; u < 2; ++u) {
      RunIm2col(st_.get(), W, F, 3, 1, 1, F, kActElu, stream, prof, "enc_sem_im2col");
      Gemm g;
      g.d = &sem_c1_[bl][u];
      g.x = cols_.get();
      g.y_act = t1_.get();
      g.out_act = kActElu;
      g.positions = F;
      RunGemm(g, stream, prof, "enc_sem_conv");
      g = Gemm();
      g.d = &sem_c2_[bl][u];
      g.x = t1_.get();
      g.y = st_.get();
      g.positions = F;
      g.accumulate = true;
      RunGemm(g, stream, prof, "enc_sem_conv");
    }
    RunIm2col(st_.get(), W, F, 3, 1, 1, F, kActNone, stream, prof, "enc_sem_im2col");
    Gemm g;
    g.d = &sem_block_[bl];
    g.x = cols_.get();
    g.y = bl == 1 ? semantic_rows : st_.get();
    g.positions = F;
    RunGemm(g, stream, prof, "enc_sem_conv");
  }

  // ---- DAC encoder on the 24 kHz samples (codec_encoder.cpp:417-452).
  // xa holds snake(x) with the alpha of whatever reads it next, ya the
  // residual branch's snake(conv1(...)).
  auto first_alpha = [&](std::size_t bi) {
    return bi < blocks_.size() ? blocks_[bi]->units[0].alpha1.get() : ac_alpha_.get();
  };
  RunConv7(ac_in_, samples, L, x_.get(), xa_.get(), first_alpha(0), false, stream, prof,
           "enc_dac_conv_in");
  int cur = L;
  for (std::size_t bi = 0; bi < blocks_.size(); ++bi) {
    const Block& blk = *blocks_[bi];
    for (int u = 0; u < 3; ++u) {
      const Unit& unit = blk.units[u];
      RunConv7(unit.conv1, xa_.get(), cur, nullptr, ya_.get(), unit.alpha2.get(), false, stream,
               prof, "enc_dac_res_conv7");
      Gemm g;
      g.d = &unit.conv2;
      g.x = ya_.get();
      g.y = x_.get();
      g.y_act = xa_.get();
      g.out_act = kActSnake;
      g.alpha_out = u < 2 ? blk.units[u + 1].alpha1.get() : blk.alpha.get();
      g.positions = cur;
      g.accumulate = true;
      RunGemm(g, stream, prof, "enc_dac_res_conv1");
    }
    const int s = blk.stride, out_len = static_cast<int>(plan.acoustic[bi]);
    RunIm2col(xa_.get(), blk.channels, cur, 2 * s, s, (s + 1) / 2, out_len, kActNone, stream,
              prof, "enc_dac_im2col");
    Gemm g;
    g.d = &blk.down;
    g.x = cols_.get();
    g.y = x_.get();
    g.y_act = xa_.get();
    g.out_act = kActSnake;
    g.alpha_out = first_alpha(bi + 1);
    g.positions = out_len;
    RunGemm(g, stream, prof, "enc_dac_down");
    cur = out_len;
  }
  const int chf = static_cast<int>(cfg_.enc_channels << cfg_.blocks);
  RunIm2col(xa_.get(), chf, cur, 3, 1, 1, F, kActNone, stream, prof, "enc_dac_im2col");
  {
    Gemm g;
    g.d = &ac_out_;
    g.x = cols_.get();
    g.y = joint_.get();
    g.positions = F;
    RunGemm(g, stream, prof, "enc_dac_out");
  }

  // ---- fc, then the residual vector quantizer (codec_encoder.cpp:453-488)
  {
    Gemm g;
    g.d = &fc_;
    g.x = joint_.get();
    g.y = emb_.get();
    g.positions = F;
    RunGemm(g, stream, prof, "enc_fc");
  }
  // (a copy, not a kernel: the profiler times kernels only)
  Check(hipMemcpyAsync(resid_.get(), emb_.get(), sizeof(float) * H * F, hipMemcpyDeviceToDevice,
                       stream),
        "copy embeddings");
  const int D = static_cast<int>(cfg_.codebook_dim), E = static_cast<int>(cfg_.codebook_size);
  for (std::size_t q = 0; q < stages_.size(); ++q) {
    const Stage& st = *stages_[q];
    Gemm g;
    g.d = &st.project;
    g.x = resid_.get();
    g.y = proj_.get();
    g.positions = F;
    RunGemm(g, stream, prof, "enc_rvq_project");
    NearestParams np{proj_.get(), st.embed.get(), st.norms.get(), st.table.get(), resid_.get(),
                     codes + q * F, D, E, H, F};
    run("enc_rvq_nearest", 2.0 * D * static_cast<double>(E) * F,
        4.0 * (static_cast<double>(E) * D * F + 2.0 * H * F), [&] { LaunchNearest(np, stream); });
  }
}

void EncoderEngine::Encode(const float* samples, int64_t length, std::int32_t* codes,
                           float* semantic, float* acoustic, float* embeddings) {
  Require(samples != nullptr && codes != nullptr, "null argument");
  const Plan plan = MakePlan(length);
  Reserve(plan);
  Check(hipMemcpyAsync(samples_.get(), samples, sizeof(float) * length, hipMemcpyHostToDevice,
                       stream_),
        "upload audio");
  Enqueue(samples_.get(), plan, codes_.get(), stream_, nullptr);
  const int64_t F = plan.frames, W = W_, H = H_, lat = cfg_.latent;
  Check(hipMemcpyAsync(codes, codes_.get(), sizeof(std::int32_t) * cfg_.codebooks * F,
                       hipMemcpyDeviceToHost, stream_),
        "download codes");
  // Optional intermediate outputs, frame-major: [frames][channels].
  auto download = [&](const float* dev, int64_t rows, float* out) {
    if (out == nullptr)
      return;
    std::vector<float> host(static_cast<std::size_t>(rows * F));
    Check(hipMemcpyAsync(host.data(), dev, sizeof(float) * rows * F, hipMemcpyDeviceToHost,
                         stream_),
          "download");
    Check(hipStreamSynchronize(stream_), "encode");
    for (int64_t r = 0; r < rows; ++r)
      for (int64_t f = 0; f < F; ++f)
        out[f * rows + r] = host[static_cast<std::size_t>(r * F + f)];
  };
  download(sem_.get(), W, semantic);
  download(joint_.get(), lat, acoustic);
  download(emb_.get(), H, embeddings);
  Check(hipStreamSynchronize(stream_), "encode");
}

void EncoderEngine::EncodeDevice(const float* samples, int64_t length, std::int32_t* codes,
                                 hipStream_t stream) {
  Require(samples != nullptr && codes != nullptr, "null argument");
  const Plan plan = MakePlan(length);
  Reserve(plan);
  Enqueue(samples, plan, codes, stream, nullptr);
  Check(hipGetLastError(), "encode launch");
}

void EncoderEngine::Profile(int64_t length, int64_t repeats,
                            std::map<std::string, KernelStat>* stats) {
  Require(repeats >= 1, "repeats must be positive");
  const Plan plan = MakePlan(length);
  Reserve(plan);
  std::vector<float> audio(static_cast<std::size_t>(length));
  for (int64_t i = 0; i < length; ++i)
    audio[i] = 0.2F * std::sin(0.05F * static_cast<float>(i)) *
               (0.5F + 0.5F * std::sin(static_cast<float>(i) / 700.0F));
  Check(hipMemcpyAsync(samples_.get(), audio.data(), sizeof(float) * length,
                       hipMemcpyHostToDevice, stream_),
        "upload audio");
  Check(hipStreamSynchronize(stream_), "upload audio");
  Enqueue(samples_.get(), plan, codes_.get(), stream_, nullptr);  // warm-up
  Profiler prof(stream_);
  for (int64_t r = 0; r < repeats; ++r)
    Enqueue(samples_.get(), plan, codes_.get(), stream_, &prof);
  prof.Collect(stats);
}

}  // namespace ovg

namespace {

void CheckEncoderConfig(const ovc_encoder_config& c) {
  using ovg::Require;
  Require(c.sample_rate >= 1 && c.semantic_rate >= 1 && c.frame_samples >= 1 &&
              c.semantic_stride >= 1,
          "bad rates");
  Require(c.feature_layers >= 1 && c.feature_layers <= 8, "1 to 8 feature convolutions");
  for (int i = 0; i < c.feature_layers; ++i)
    Require(c.conv_dim[i] >= 1 && c.conv_kernel[i] >= 1 && c.conv_stride[i] >= 1,
            "bad feature convolution");
  Require(c.width >= 1 && c.intermediate >= 1 && c.heads >= 1 && c.width % c.heads == 0,
          "width must split into heads");
  Require(c.width <= 1024 && c.conv_dim[c.feature_layers - 1] <= 1024,
          "HuBERT widths above 1024 are not supported");
  Require(c.layers >= 0 && c.layers <= 64, "0 to 64 layers");
  Require(c.pos_kernel >= 1 && c.pos_groups >= 1 && c.width % c.pos_groups == 0,
          "width must split into positional groups");
  Require(c.eps > 0.0, "eps must be positive");
  Require(c.enc_channels >= 1 && c.latent >= 1 && c.blocks >= 1 && c.blocks <= 8,
          "bad acoustic encoder");
  int64_t hop = 1;
  for (int i = 0; i < c.blocks; ++i) {
    Require(c.ratios[i] >= 1 && c.ratios[i] <= 16, "ratios must be 1 to 16");
    hop *= c.ratios[i];
  }
  Require(hop == c.frame_samples, "ratios must multiply to frame_samples");
  Require(c.codebooks >= 1 && c.codebook_size >= 1 && c.codebook_dim >= 1 &&
              c.codebook_dim <= 1024,
          "bad quantizer");
}

}  // namespace

struct ovc_encoder {
  std::unique_ptr<ovg::EncoderEngine> engine;
};

extern "C" {

int ovc_encoder_create(const ovc_encoder_config* config, const char* model_root,
                       uint64_t weight_seed, ovc_encoder** handle, char* error,
                       size_t error_len) {
  return ovg::CodecGuard("OmniVoice audio tokenizer: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    CheckEncoderConfig(*config);
    // model_root / "audio_tokenizer/model.safetensors", as std::filesystem
    // joins it (an empty root names the working directory); synthetic
    // weights come only from the *_create_synthetic entry point.
    std::unique_ptr<ovg::SafetensorsFile> file = ovg::SafetensorsFile::Open(ovg::JoinPath(
        model_root == nullptr ? "" : model_root, "audio_tokenizer/model.safetensors"));
    auto h = std::make_unique<ovc_encoder>();
    h->engine = std::make_unique<ovg::EncoderEngine>(*config, weight_seed, file.get());
    *handle = h.release();
    return OVG_OK;
  });
}

int ovc_encoder_create_synthetic(const ovc_encoder_config* config, uint64_t weight_seed,
                                 ovc_encoder** handle, char* error, size_t error_len) {
  return ovg::CodecGuard("OmniVoice audio tokenizer: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    CheckEncoderConfig(*config);
    auto h = std::make_unique<ovc_encoder>();
    h->engine = std::make_unique<ovg::EncoderEngine>(*config, weight_seed, nullptr);
    *handle = h.release();
    return OVG_OK;
  });
}

void ovc_encoder_destroy(ovc_encoder* handle) { delete handle; }

int64_t ovc_encoder_frames(const ovc_encoder* handle, int64_t samples) {
  return handle == nullptr || samples < 0 ? 0 : handle->engine->Frames(samples);
}

int ovc_encode(ovc_encoder* handle, const float* samples, int64_t length, int32_t* codes,
               float* semantic, float* acoustic, float* embeddings, char* error,
               size_t error_len) {
  return ovg::CodecGuard("OmniVoice encode: ", error, error_len, [&] {
    ovg::Require(handle != nullptr, "null argument");
    handle->engine->Encode(samples, length, codes, semantic, acoustic, embeddings);
    return OVG_OK;
  });
}

int ovc_encode_device(ovc_encoder* handle, const float* samples, int64_t length,
                      int32_t* codes, void* stream, char* error, size_t error_len) {
  return ovg::CodecGuard("OmniVoice encode: ", error, error_len, [&] {
    ovg::Require(handle != nullptr, "null argument");
    handle->engine->EncodeDevice(samples, length, codes, static_cast<hipStream_t>(stream));
    return OVG_OK;
  });
}

int ovc_profile_encode(ovc_encoder* handle, int64_t length, int64_t repeats,
                       ovg_kernel_stat* stats, int64_t capacity, int64_t* count, char* error,
                       size_t error_len) {
  return ovg::CodecGuard("OmniVoice profile: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && count != nullptr, "null argument");
    std::map<std::string, ovg::KernelStat> table;
    handle->engine->Profile(length, repeats, &table);
    int64_t n = 0;
    for (const auto& [name, s] : table) {
      if (n < capacity && stats != nullptr) {
        ovg_kernel_stat& out = stats[n];
        std::memset(&out, 0, sizeof(out));
        std::snprintf(out.name, sizeof(out.name), "%s", name.c_str());
        out.launches = s.launches;
        out.total_ms = s.ms;
        out.flops = s.flops;
        out.bytes = s.bytes;
      }
      ++n;
    }
    *count = n;
    return OVG_OK;
  });
}

}  // extern "C"
