// The audio decoder engine and its C ABI (include/omnivoice_codec_mi355x.h):
// RVQ codes to audio through the Higgs Audio v2 tokenizer's DAC decoder.
//
// Reference counterparts: Codec::Load, decoder half (codec.cpp:92-148),
// Codec::Decode (codec.cpp:197-260) and Codec::State's convolution helpers
// (codec_state.hpp:184-300).
//
// Differences of design, not of results:
//  * fc2 is folded into the RVQ tables at load (in double on the host):
//    table[c][e][o] = sum_h fc2[o][h] (embed_c project_c^T + bias_c)[e][h],
//    so decoding starts with one gather-sum of codebook rows per frame
//    instead of a table gather and a GEMM.
//  * Every convolution is one kernel: the Snake activation of its input is
//    applied while the input is staged, bias and residual addition in the
//    epilogue. A transposed convolution of stride s runs as s output phases
//    of a two-tap convolution instead of a GEMM into columns plus col2im.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/omnivoice_codec_mi355x.h"
#include "checkpoint.hpp"
#include "codec.hpp"
#include "codec_common.hpp"
#include "device.hpp"
#include "host.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kResidualKernel = 7;
constexpr std::int64_t kPartialFloats = std::int64_t{8} << 20;  // 32 MiB
constexpr int kDilations[3] = {1, 3, 9};

// Synthetic decoder specification (tensor id, scale); element = flat index
// in the checkpoint tensor's own shape; value float(scale n), the Snake
// alphas float(exp(0.1 n)), n = SynthNormal(seed, id, element):
//   quantizer.quantizers.c.codebook.embed       1000 + 4c   0.35
//   quantizer.quantizers.c.project_out.weight   1001 + 4c   1 / sqrt(dim)
//   quantizer.quantizers.c.project_out.bias     1002 + 4c   0.01
//   fc2.weight, fc2.bias                        1100, 1101  1 / sqrt(hidden), 0.01
//   acoustic_decoder.conv1.weight, .bias        1102, 1103  1 / sqrt(7 latent), 0.01
//   acoustic_decoder.block.i.snake1.alpha       1200 + 32i  exp
//   ....block.i.conv_t1.weight, .bias           + 1, + 2    1 / sqrt(2 in), 0.01
//   ....block.i.res_unit(u+1).snake1.alpha      + 4 + 6u    exp
//   ....res_unit(u+1).conv1.weight, .bias       + 5, + 6    1 / sqrt(7 ch), 0.01
//   ....res_unit(u+1).snake2.alpha              + 7         exp
//   ....res_unit(u+1).conv2.weight, .bias       + 8, + 9    0.3 / sqrt(ch), 0.01
//   acoustic_decoder.snake1.alpha               1400        exp
//   acoustic_decoder.conv2.weight, .bias        1401, 1402  0.1 / sqrt(7 ch), 0.01
// ConvTranspose1d (kernel 2s, padding ceil(s / 2)) as s phases of two taps:
// output m s + p = sum_i w[i][o][ka] x[i][m + c] + w[i][o][ka + s] x[i][m + c - 1]
// with ka = (p + pad) % s and c = (p + pad) / s. Tap 0 is the one at offset
// c - 1. Weights [in][out][2s] -> [phase][tap][in][out].
struct UpsampleTaps {
  int offsets[kConvMaxPhases][2];
  int kernel_index[kConvMaxPhases][2];
};
UpsampleTaps Phases(int stride) {
  UpsampleTaps u{};
  const int pad = (stride + 1) / 2;
  for (int p = 0; p < stride; ++p) {
    const int ka = (p + pad) % stride;
    const int c = (p + pad) / stride;
    u.offsets[p][0] = c - 1;
    u.kernel_index[p][0] = ka + stride;
    u.offsets[p][1] = c;
    u.kernel_index[p][1] = ka;
  }
  return u;
}
std::vector<float> UpsampleLayout(const std::vector<float>& w, int in, int out, int stride) {
  const UpsampleTaps u = Phases(stride);
  std::vector<float> r(static_cast<std::size_t>(stride) * 2 * in * out);
  for (int p = 0; p < stride; ++p)
    for (int tap = 0; tap < 2; ++tap)
      for (int i = 0; i < in; ++i)
        for (int o = 0; o < out; ++o)
          r[((static_cast<std::size_t>(p) * 2 + tap) * in + i) * out + o] =
              w[(static_cast<std::size_t>(i) * out + o) * 2 * stride + u.kernel_index[p][tap]];
  return r;
}

struct Conv {
  DeviceBuffer<float> w, b;  // [taps][in][out], [out]
  int in = 0, out = 0, taps = 1, dilation = 1;
};
struct Unit {
  DeviceBuffer<float> alpha1, alpha2;
  Conv conv1, conv2;
};
struct Block {
  DeviceBuffer<float> alpha, w, b;  // w [stride][2][in][out]
  int in = 0, out = 0, stride = 1;
  Unit units[3];
};

void LoadConv(const Source& src, const std::string& prefix, std::uint64_t id, int in,
              int out, int kernel, int dilation, double gain, Conv* conv) {
  const auto w = src.Get(prefix + ".weight", {out, in, kernel}, id,
                         gain / std::sqrt(static_cast<double>(in) * kernel));
  const auto b = src.Get(prefix + ".bias", {out}, id + 1, 0.01);
  Upload(conv->w, ConvLayout(w, out, in, kernel));
  Upload(conv->b, b);
  conv->in = in;
  conv->out = out;
  conv->taps = kernel;
  conv->dilation = dilation;
}

}  // namespace

class CodecEngine {
 public:
  CodecEngine(const ovc_config& cfg, std::uint64_t seed, const SafetensorsFile* file);
  ~CodecEngine() {
    if (stream_ != nullptr)
      (void)hipStreamDestroy(stream_);
  }
  std::int64_t Samples(std::int64_t frames) const { return frames * hop_; }
  void Decode(const std::int32_t* codes, std::int64_t frames, float* audio);
  void DecodeDevice(const std::int32_t* codes, std::int64_t frames, float* audio,
                    hipStream_t stream);
  void Profile(std::int64_t frames, std::int64_t repeats,
               std::map<std::string, KernelStat>* stats);

 private:
  void Reserve(std::int64_t frames);
  void Enqueue(const std::int32_t* codes, std::int64_t frames, float* audio,
               hipStream_t stream, Profiler* prof);
  void RunConv(const Conv& c, const float* x, int length, float* y, float* y_act,
               const float* alpha_out, bool accumulate, hipStream_t stream, Profiler* prof,
               const char* name);

  ovc_config cfg_;
  std::int64_t hop_ = 1;
  hipStream_t stream_ = nullptr;
  DeviceBuffer<float> table_, fc2_bias_, final_alpha_, out_w_, out_b_;
  Conv input_;
  std::vector<std::unique_ptr<Block>> blocks_;
  // Work buffers: the latent input, the signal, its Snake-activated copies
  // (the next convolution's input; two, so that an upsampling layer reads
  // one and writes the other) and the residual branch's activated output.
  DeviceBuffer<float> latent_, x_, xa_[2], ya_, audio_;
  // Split-K workspace of the convolutions whose output tiles leave CUs idle
  // (the input convolution at short lengths).
  DeviceBuffer<float> partial_;
  DeviceBuffer<std::int32_t> codes_;
  std::int64_t reserved_ = 0;
};

CodecEngine::CodecEngine(const ovc_config& cfg, std::uint64_t seed,
                         const SafetensorsFile* file)
    : cfg_(cfg) {
  const int C = static_cast<int>(cfg.codebooks), E = static_cast<int>(cfg.codebook_size),
            D = static_cast<int>(cfg.codebook_dim), H = static_cast<int>(cfg.hidden),
            Lat = static_cast<int>(cfg.latent);
  for (int i = 0; i < cfg.blocks; ++i)
    hop_ *= cfg.ratios[i];
  Check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  const Source src(seed, file);

  // RVQ tables through project_out (codec.cpp:112-140), folded with fc2.
  const auto fc2 = src.Get("fc2.weight", {Lat, H}, 1100, 1.0 / std::sqrt(double(H)));
  const auto fc2_bias = src.Get("fc2.bias", {Lat}, 1101, 0.01);
  std::vector<float> table(static_cast<std::size_t>(C) * E * Lat);
  std::vector<std::vector<float>> embed(C), project(C), pbias(C);
  for (int c = 0; c < C; ++c) {
    const std::string prefix = "quantizer.quantizers." + std::to_string(c);
    embed[c] = src.Get(prefix + ".codebook.embed", {E, D}, 1000 + 4 * c, 0.35);
    project[c] = src.Get(prefix + ".project_out.weight", {H, D}, 1001 + 4 * c,
                         1.0 / std::sqrt(double(D)));
    pbias[c] = src.Get(prefix + ".project_out.bias", {H}, 1002 + 4 * c, 0.01);
  }
  std::vector<std::thread> workers;
  for (int c = 0; c < C; ++c)
    workers.emplace_back([&, c] {
      // P[o][d] = sum_h fc2[o][h] project[h][d], q[o] = sum_h fc2[o][h] bias[h]
      std::vector<double> P(static_cast<std::size_t>(Lat) * D, 0.0), q(Lat, 0.0);
      for (int o = 0; o < Lat; ++o)
        for (int h = 0; h < H; ++h) {
          const double f = fc2[static_cast<std::size_t>(o) * H + h];
          const float* row = &project[c][static_cast<std::size_t>(h) * D];
          for (int d = 0; d < D; ++d)
            P[static_cast<std::size_t>(o) * D + d] += f * row[d];
          q[o] += f * pbias[c][h];
        }
      for (int e = 0; e < E; ++e)
        for (int o = 0; o < Lat; ++o) {
          double acc = q[o];
          for (int d = 0; d < D; ++d)
            acc += static_cast<double>(embed[c][static_cast<std::size_t>(e) * D + d]) *
                   P[static_cast<std::size_t>(o) * D + d];
          table[(static_cast<std::size_t>(c) * E + e) * Lat + o] = static_cast<float>(acc);
        }
    });
  for (auto& w : workers)
    w.join();
  Upload(table_, table);
  Upload(fc2_bias_, fc2_bias);

  int channels = static_cast<int>(cfg.channels);
  LoadConv(src, "acoustic_decoder.conv1", 1102, Lat, channels, kResidualKernel, 1, 1.0,
           &input_);
  for (int i = 0; i < cfg.blocks; ++i) {
    auto blk = std::make_unique<Block>();
    const std::string prefix = "acoustic_decoder.block." + std::to_string(i);
    const std::uint64_t id = 1200 + 32 * static_cast<std::uint64_t>(i);
    const int out = channels / 2, stride = static_cast<int>(cfg.ratios[i]);
    blk->in = channels;
    blk->out = out;
    blk->stride = stride;
    Upload(blk->alpha, src.Get(prefix + ".snake1.alpha", {1, channels, 1}, id, 0.1, true));
    const auto w = src.Get(prefix + ".conv_t1.weight", {channels, out, 2 * stride}, id + 1,
                           1.0 / std::sqrt(2.0 * channels));
    Upload(blk->w, UpsampleLayout(w, channels, out, stride));
    Upload(blk->b, src.Get(prefix + ".conv_t1.bias", {out}, id + 2, 0.01));
    for (int u = 0; u < 3; ++u) {
      const std::string name = prefix + ".res_unit" + std::to_string(u + 1);
      const std::uint64_t uid = id + 4 + 6 * static_cast<std::uint64_t>(u);
      Unit& unit = blk->units[u];
      Upload(unit.alpha1, src.Get(name + ".snake1.alpha", {1, out, 1}, uid, 0.1, true));
      LoadConv(src, name + ".conv1", uid + 1, out, out, kResidualKernel, kDilations[u], 1.0,
               &unit.conv1);
      Upload(unit.alpha2, src.Get(name + ".snake2.alpha", {1, out, 1}, uid + 3, 0.1, true));
      LoadConv(src, name + ".conv2", uid + 4, out, out, 1, 1, 0.3, &unit.conv2);
    }
    blocks_.push_back(std::move(blk));
    channels = out;
  }
  Upload(final_alpha_, src.Get("acoustic_decoder.snake1.alpha", {1, channels, 1}, 1400, 0.1,
                               true));
  const auto ow = src.Get("acoustic_decoder.conv2.weight", {1, channels, kResidualKernel},
                          1401, 0.1 / std::sqrt(7.0 * channels));
  Upload(out_w_, ConvLayout(ow, 1, channels, kResidualKernel));
  Upload(out_b_, src.Get("acoustic_decoder.conv2.bias", {1}, 1402, 0.01));
  partial_.Reserve(kPartialFloats);
  Check(hipDeviceSynchronize(), "codec upload");
}

void CodecEngine::Reserve(std::int64_t frames) {
  if (frames <= reserved_)
    return;
  std::int64_t length = frames, largest = cfg_.channels * frames, channels = cfg_.channels;
  for (const auto& blk : blocks_) {
    length *= blk->stride;
    channels = blk->out;
    largest = std::max(largest, channels * length);
  }
  // Kernel indices are 32-bit per dimension: every signal must stay below
  // 2^31 samples per channel and elements in all.
  Require(largest < (std::int64_t{1} << 31), "too many frames");
  latent_.Reserve(static_cast<std::size_t>(cfg_.latent * frames));
  x_.Reserve(static_cast<std::size_t>(largest));
  xa_[0].Reserve(static_cast<std::size_t>(largest));
  xa_[1].Reserve(static_cast<std::size_t>(largest));
  ya_.Reserve(static_cast<std::size_t>(largest));
  audio_.Reserve(static_cast<std::size_t>(length));
  codes_.Reserve(static_cast<std::size_t>(cfg_.codebooks * frames));
  reserved_ = frames;
}

void CodecEngine::RunConv(const Conv& c, const float* x, int length, float* y, float* y_act,
                          const float* alpha_out, bool accumulate, hipStream_t stream,
                          Profiler* prof, const char* name) {
  ConvParams p{};
  p.x = x;
  p.w = c.w.get();
  p.bias = c.b.get();
  p.partial = partial_.get();
  p.partial_capacity = kPartialFloats;
  p.y = y;
  p.y_act = y_act;
  p.alpha_out = alpha_out;
  p.cin = c.in;
  p.len_in = length;
  p.cout = c.out;
  p.len_out = length;
  p.taps = c.taps;
  p.phases = 1;
  p.positions = length;
  p.out_stride = 1;
  p.accumulate = accumulate ? 1 : 0;
  const int pad = (c.taps - 1) * c.dilation / 2;
  for (int k = 0; k < c.taps; ++k)
    p.offsets[0][k] = k * c.dilation - pad;
  const double flops = 2.0 * c.out * static_cast<double>(length) * c.in * c.taps;
  const double outputs = (y != nullptr ? 1.0 : 0.0) + (y_act != nullptr ? 1.0 : 0.0) +
                         (accumulate ? 1.0 : 0.0);
  const double bytes = 4.0 * length * (c.in + c.out * outputs) + 4.0 * c.taps * c.in * c.out;
  auto launch = [&] { LaunchConv(p, stream); };
  if (prof != nullptr)
    prof->Run(name, flops, bytes, launch);
  else
    launch();
}

void CodecEngine::Enqueue(const std::int32_t* codes, std::int64_t frames, float* audio,
                          hipStream_t stream, Profiler* prof) {
  Require(frames >= 1, "no frames");
  Reserve(frames);
  const int F = static_cast<int>(frames);
  auto run = [&](const char* name, double flops, double bytes, auto&& launch) {
    if (prof != nullptr)
      prof->Run(name, flops, bytes, launch);
    else
      launch();
  };
  RvqParams r{};
  r.table = table_.get();
  r.bias = fc2_bias_.get();
  r.codes = codes;
  r.y = latent_.get();
  r.codebooks = static_cast<int>(cfg_.codebooks);
  r.entries = static_cast<int>(cfg_.codebook_size);
  r.latent = static_cast<int>(cfg_.latent);
  r.frames = F;
  run("codec_rvq", 0.0, 4.0 * cfg_.codebooks * cfg_.latent * F * 2.0,
      [&] { LaunchRvq(r, stream); });
  // Every Snake is computed once, by the epilogue of the convolution that
  // produces its input: xa holds snake(x) with the alpha of whatever reads
  // it next, ya the residual branch's snake(conv1(...)).
  const float* first_alpha =
      blocks_.empty() ? final_alpha_.get() : blocks_.front()->alpha.get();
  int cur = 0;
  RunConv(input_, latent_.get(), F, nullptr, xa_[cur].get(), first_alpha, false, stream, prof,
          "codec_conv_in");
  int length = F;
  for (std::size_t bi = 0; bi < blocks_.size(); ++bi) {
    const Block& blk = *blocks_[bi];
    // Transposed convolution (codec_state.hpp:272-288) of snake(x): the raw
    // output is the new signal, its Snake feeds the first residual unit.
    ConvParams p{};
    p.x = xa_[cur].get();
    p.w = blk.w.get();
    p.bias = blk.b.get();
    p.partial = partial_.get();
    p.partial_capacity = kPartialFloats;
    p.y = x_.get();
    p.y_act = xa_[1 - cur].get();
    p.alpha_out = blk.units[0].alpha1.get();
    p.cin = blk.in;
    p.len_in = length;
    p.cout = blk.out;
    p.len_out = length * blk.stride;
    p.taps = 2;
    p.phases = blk.stride;
    p.positions = length;
    p.out_stride = blk.stride;
    const UpsampleTaps u = Phases(blk.stride);
    for (int ph = 0; ph < blk.stride; ++ph)
      for (int k = 0; k < 2; ++k)
        p.offsets[ph][k] = u.offsets[ph][k];
    run("codec_upsample", 2.0 * blk.out * double(length) * blk.stride * blk.in * 2,
        4.0 * length * (blk.in + 2.0 * blk.out * blk.stride) +
            4.0 * 2 * blk.stride * blk.in * blk.out,
        [&] { LaunchConv(p, stream); });
    cur = 1 - cur;
    length *= blk.stride;
    // Residual units (codec_state.hpp:252-270): x += conv2(snake(conv1(snake(x)))).
    for (int ui = 0; ui < 3; ++ui) {
      const Unit& unit = blk.units[ui];
      const float* next_alpha = ui < 2 ? blk.units[ui + 1].alpha1.get()
                                : bi + 1 < blocks_.size() ? blocks_[bi + 1]->alpha.get()
                                                          : final_alpha_.get();
      RunConv(unit.conv1, xa_[cur].get(), length, nullptr, ya_.get(), unit.alpha2.get(), false,
              stream, prof, "codec_res_conv7");
      RunConv(unit.conv2, ya_.get(), length, x_.get(), xa_[cur].get(), next_alpha, true, stream,
              prof, "codec_res_conv1");
    }
  }
  // Output convolution of snake(x), no tanh (codec.cpp:244-251).
  OutputConvParams o{};
  o.x = xa_[cur].get();
  o.alpha = nullptr;
  o.w = out_w_.get();
  o.bias = out_b_.get();
  o.y = audio;
  o.cin = blocks_.empty() ? input_.out : blocks_.back()->out;
  o.length = length;
  o.taps = kResidualKernel;
  run("codec_conv_out", 2.0 * o.cin * double(length) * o.taps, 4.0 * length * (o.cin + 1.0),
      [&] { LaunchOutputConv(o, stream); });
}

void CodecEngine::Decode(const std::int32_t* codes, std::int64_t frames, float* audio) {
  Require(codes != nullptr && audio != nullptr, "null argument");
  Require(frames >= 1, "no frames");
  const std::int64_t count = cfg_.codebooks * frames;
  for (std::int64_t i = 0; i < count; ++i)
    Require(codes[i] >= 0 && codes[i] < cfg_.codebook_size, "code outside the codebook");
  Reserve(frames);
  Check(hipMemcpyAsync(codes_.get(), codes, count * sizeof(std::int32_t),
                       hipMemcpyHostToDevice, stream_),
        "upload codes");
  Enqueue(codes_.get(), frames, audio_.get(), stream_, nullptr);
  Check(hipMemcpyAsync(audio, audio_.get(), Samples(frames) * sizeof(float),
                       hipMemcpyDeviceToHost, stream_),
        "download audio");
  Check(hipStreamSynchronize(stream_), "decode");
}

void CodecEngine::DecodeDevice(const std::int32_t* codes, std::int64_t frames, float* audio,
                               hipStream_t stream) {
  Require(codes != nullptr && audio != nullptr, "null argument");
  Enqueue(codes, frames, audio, stream != nullptr ? stream : stream_, nullptr);
  Check(hipGetLastError(), "decode launch");
}

void CodecEngine::Profile(std::int64_t frames, std::int64_t repeats,
                          std::map<std::string, KernelStat>* stats) {
  Reserve(frames);
  std::vector<std::int32_t> codes(static_cast<std::size_t>(cfg_.codebooks * frames));
  for (std::size_t i = 0; i < codes.size(); ++i)
    codes[i] = static_cast<std::int32_t>((i * 2654435761U) % cfg_.codebook_size);
  Check(hipMemcpyAsync(codes_.get(), codes.data(), codes.size() * sizeof(std::int32_t),
                       hipMemcpyHostToDevice, stream_),
        "upload codes");
  Check(hipStreamSynchronize(stream_), "upload codes");
  for (std::int64_t r = 0; r < std::max<std::int64_t>(repeats, 1); ++r) {
    Profiler prof(stream_);
    Enqueue(codes_.get(), frames, audio_.get(), stream_, &prof);
    prof.Collect(stats);
  }
}

}  // namespace ovg

// ====================================================================== C ABI

struct ovc_handle {
  std::unique_ptr<ovg::CodecEngine> engine;
};

namespace {

using ovg::CodecGuard;

void CheckConfig(const ovc_config& c) {
  ovg::Require(c.codebooks >= 1 && c.codebook_size >= 1 && c.codebook_dim >= 1 &&
                   c.hidden >= 1 && c.latent >= 1 && c.channels >= 1,
               "config: empty dimension");
  ovg::Require(c.blocks >= 1 && c.blocks <= 8, "config: 1 to 8 upsampling blocks");
  ovg::Require(c.channels % (std::int64_t{1} << c.blocks) == 0,
               "config: decoder channels can't be halved once per upsampling block");
  for (int i = 0; i < c.blocks; ++i)
    ovg::Require(c.ratios[i] >= 1 && c.ratios[i] <= ovg::kConvMaxPhases,
                 "config: upsampling ratios must be 1 to 8");
  ovg::Require(c.codebooks * c.codebook_size * c.latent < (std::int64_t{1} << 31) &&
                   c.channels * c.latent * 7 < (std::int64_t{1} << 31),
               "config: tables too large");
}

}  // namespace

extern "C" {

int ovc_create(const ovc_config* config, const char* model_root, uint64_t weight_seed,
               ovc_handle** handle, char* error, size_t error_len) {
  // weight_seed is unused: the weights come from the file.
  return CodecGuard("OmniVoice audio tokenizer: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    CheckConfig(*config);
    // model_root / "audio_tokenizer/model.safetensors", as std::filesystem
    // joins it (an empty root names the working directory); synthetic
    // weights come only from the *_create_synthetic entry point.
    std::unique_ptr<ovg::SafetensorsFile> file = ovg::SafetensorsFile::Open(ovg::JoinPath(
        model_root == nullptr ? "" : model_root, "audio_tokenizer/model.safetensors"));
    auto h = std::make_unique<ovc_handle>();
    h->engine = std::make_unique<ovg::CodecEngine>(*config, weight_seed, file.get());
    *handle = h.release();
    return OVG_OK;
  });
}

int ovc_create_synthetic(const ovc_config* config, uint64_t weight_seed, ovc_handle** handle,
                         char* error, size_t error_len) {
  return CodecGuard("OmniVoice audio tokenizer: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    CheckConfig(*config);
    auto h = std::make_unique<ovc_handle>();
    h->engine = std::make_unique<ovg::CodecEngine>(*config, weight_seed, nullptr);
    *handle = h.release();
    return OVG_OK;
  });
}

void ovc_destroy(ovc_handle* handle) { delete handle; }

int64_t ovc_samples(const ovc_handle* handle, int64_t frames) {
  return handle == nullptr ? 0 : handle->engine->Samples(frames);
}

int ovc_decode(ovc_handle* handle, const int32_t* codes, int64_t frames, float* audio,
               char* error, size_t error_len) {
  return CodecGuard("OmniVoice decode: ", error, error_len, [&] {
    ovg::Require(handle != nullptr, "null argument");
    handle->engine->Decode(codes, frames, audio);
    return OVG_OK;
  });
}

int ovc_decode_device(ovc_handle* handle, const int32_t* codes, int64_t frames, float* audio,
                      void* stream, char* error, size_t error_len) {
  return CodecGuard("OmniVoice decode: ", error, error_len, [&] {
    ovg::Require(handle != nullptr, "null argument");
    handle->engine->DecodeDevice(codes, frames, audio, static_cast<hipStream_t>(stream));
    return OVG_OK;
  });
}

int ovc_profile_decode(ovc_handle* handle, int64_t frames, int64_t repeats,
                       ovg_kernel_stat* stats, int64_t capacity, int64_t* count, char* error,
                       size_t error_len) {
  return CodecGuard("OmniVoice profile: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && count != nullptr, "null argument");
    std::map<std::string, ovg::KernelStat> table;
    handle->engine->Profile(frames, repeats, &table);
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

void ovc_synthetic_values(uint64_t weight_seed, uint64_t tensor, uint64_t first,
                          int64_t count, double scale, int exponential, float* out) {
  if (count <= 0 || out == nullptr)
    return;
  ovg::SynthCodec(weight_seed, tensor, scale, exponential != 0, first,
                  static_cast<std::size_t>(count), out);
}

int ovc_op_conv1d(const float* x, int64_t in, int64_t length, const float* alpha,
                  const float* w, const float* b, int64_t out, int64_t kernel,
                  int64_t dilation, int accumulate, float* y, void* stream, char* error,
                  size_t error_len) {
  return CodecGuard("conv1d: ", error, error_len, [&] {
    ovg::Require(x && w && b && y, "null pointer");
    ovg::Require(in >= 1 && out >= 1 && length >= 1 && kernel >= 1 && dilation >= 1 &&
                     in * out * kernel < (int64_t{1} << 31) && length < (int64_t{1} << 31),
                 "bad shape");
    const int I = static_cast<int>(in), O = static_cast<int>(out), K = static_cast<int>(kernel);
    const std::vector<float> host(w, w + static_cast<std::size_t>(O) * I * K);
    ovg::DeviceBuffer<float> wd, bd;
    ovg::Upload(wd, ovg::ConvLayout(host, O, I, K));
    ovg::Upload(bd, std::vector<float>(b, b + O));
    ovg::ConvParams p{};
    p.x = x;
    p.alpha_in = alpha;
    p.w = wd.get();
    p.bias = bd.get();
    p.y = y;
    p.cin = I;
    p.len_in = static_cast<int>(length);
    p.cout = O;
    p.len_out = static_cast<int>(length);
    p.taps = K;
    p.phases = 1;
    p.positions = static_cast<int>(length);
    p.out_stride = 1;
    p.accumulate = accumulate ? 1 : 0;
    const int pad = (K - 1) * static_cast<int>(dilation) / 2;
    ovg::Require(K <= ovg::kConvMaxTaps, "1 to 7 taps");
    for (int k = 0; k < K; ++k)
      p.offsets[0][k] = k * static_cast<int>(dilation) - pad;
    auto s = static_cast<hipStream_t>(stream);
    ovg::LaunchConv(p, s);
    ovg::Check(hipStreamSynchronize(s), "conv1d");
    return OVG_OK;
  });
}

int ovc_op_conv_transpose1d(const float* x, int64_t in, int64_t length, const float* alpha,
                            const float* w, const float* b, int64_t out, int64_t stride,
                            float* y, void* stream, char* error, size_t error_len) {
  return CodecGuard("conv_transpose1d: ", error, error_len, [&] {
    ovg::Require(x && w && b && y, "null pointer");
    ovg::Require(in >= 1 && out >= 1 && length >= 1 && stride >= 1 &&
                     stride <= ovg::kConvMaxPhases &&
                     in * out * 2 * stride < (int64_t{1} << 31) &&
                     length * stride < (int64_t{1} << 31),
                 "bad shape");
    const int I = static_cast<int>(in), O = static_cast<int>(out), S = static_cast<int>(stride);
    const std::vector<float> host(w, w + static_cast<std::size_t>(I) * O * 2 * S);
    ovg::DeviceBuffer<float> wd, bd;
    ovg::Upload(wd, ovg::UpsampleLayout(host, I, O, S));
    ovg::Upload(bd, std::vector<float>(b, b + O));
    ovg::ConvParams p{};
    p.x = x;
    p.alpha_in = alpha;
    p.w = wd.get();
    p.bias = bd.get();
    p.y = y;
    p.cin = I;
    p.len_in = static_cast<int>(length);
    p.cout = O;
    p.len_out = static_cast<int>(length) * S;
    p.taps = 2;
    p.phases = S;
    p.positions = static_cast<int>(length);
    p.out_stride = S;
    const ovg::UpsampleTaps u = ovg::Phases(S);
    for (int ph = 0; ph < S; ++ph)
      for (int k = 0; k < 2; ++k)
        p.offsets[ph][k] = u.offsets[ph][k];
    auto s = static_cast<hipStream_t>(stream);
    ovg::LaunchConv(p, s);
    ovg::Check(hipStreamSynchronize(s), "conv_transpose1d");
    return OVG_OK;
  });
}

}  // extern "C"
