// The generator engine: weights in HBM, the packed CFG batch, the per-step
// launch sequence, the captured step graph and the C ABI
// (include/omnivoice_mi355x.h).
//
// Reference counterparts: Generator::State and its methods
// (generator.cpp:87-304), Generator::Load/Forward/Score/Generate
// (generator.cpp:364-543).
//
// Differences of design, not of results:
//  * The whole unmasking step runs on the device (forward, CFG score, top-k
//    select and the write-back of the chosen codes into both sequences), so
//    steps are queued back to back; the reference downloads predictions and
//    confidences and selects on the host every step (generator.cpp:517-535).
//  * One step is captured once as a HIP graph per batch layout and replayed;
//    the select kernel reads its step's (step, count, noise offset) from a
//    device table through a counter the embedding kernel advances.
//  * The Gumbel noise stream (std::mt19937_64, decoding.cpp:83-86) is drawn
//    on the host for every executed step up front and uploaded once.
//  * Several inputs can share one packed batch (sequences aligned to 16 rows).
//  * The text embedding table lives in HBM (the reference keeps it mmapped on
//    the host and gathers rows per request, generator.cpp:206-217).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/omnivoice_mi355x.h"
#include "checkpoint.hpp"
#include "device.hpp"
#include "host.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

void SetPrefetch(WeightPrefetch& w, std::initializer_list<const DeviceBuffer<half_t>*> ranges,
                 int groups) {
  Require(ranges.size() <= WeightPrefetch::kMaxRanges, "prefetch: too many ranges");
  w = WeightPrefetch{};
  int r = 0;
  for (const DeviceBuffer<half_t>* b : ranges) {
    w.range[r] = reinterpret_cast<const unsigned char*>(b->get());
    w.bytes[r] = b->bytes();
    ++r;
  }
  w.groups = groups;
}

struct Layer {
  DeviceBuffer<half_t> qkv;      // [(heads + 2 kv) * 128][hidden]
  DeviceBuffer<half_t> output;   // [hidden][heads * 128]
  DeviceBuffer<half_t> gate_up;  // packed blocks of 16 gate + 16 up rows (PackMap::kSwiGlu)
  DeviceBuffer<half_t> down;     // [hidden][intermediate]
  DeviceBuffer<float> input_norm, post_norm, q_norm, k_norm;
};

struct ItemLayout {
  std::int64_t length = 0, audio_start = 0, frames = 0;
  int cond_row = 0, uncond_row = 0;  // first packed row of each sequence
  int logit_row = 0;                 // cond target logits rows, then uncond
  int out_base = 0;                  // offset of its [codebooks][frames]
};

struct Layout {
  std::vector<ItemLayout> items;
  int rows = 0;        // packed rows, alignment padding included
  int real_rows = 0;   // rows without padding (algorithmic work)
  int rows_alloc = 0;  // rows + one key tile of slack
  int targets = 0;     // 2 * sum of frames
  int outputs = 0;     // codebooks * sum of frames
  int max_frames = 0;
  int max_total = 0;
  std::vector<int> ids;        // [codebooks][rows_alloc]
  std::vector<int> row_kind;   // [rows_alloc]
  std::vector<int> positions;  // [rows_alloc]
  std::vector<int> gather;     // [targets]
  std::vector<AttentionWork> work;
  int exact_work = 0;    // work[0, exact_work): the exact attention kernel
  int exact_rounds = 0;  // their largest number of key rounds
  std::vector<ScoreItem> score_items;
  std::vector<SelectItem> select_items;
  std::string signature;
};

struct Input {
  std::int64_t codebooks, length, audio_start, frames;
  const std::int32_t* ids;
};

}  // namespace

class Engine {
 public:
  explicit Engine(const ovg_config& c) : cfg_(c) {
    Require(c.head_dim == 128, "head_dim must be 128");
    Require(c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0,
            "heads must be a positive multiple of kv_heads");
    const std::int64_t group = c.heads / c.kv_heads;
    Require(group == 1 || group == 2,
            "query heads per kv head must be 1 or 2");
    Require(c.hidden_size % 64 == 0 && c.hidden_size <= 4096,
            "hidden_size must be a multiple of 64 and at most 4096");
    Require(c.intermediate_size % 64 == 0,
            "intermediate_size must be a multiple of 64");
    Require((c.heads * 128) % 64 == 0, "bad head count");
    Require(c.audio_codebooks >= 1 && c.audio_vocab_size >= 2 &&
                c.audio_vocab_size <= 1088,
            "audio vocabulary must hold 2 to 1088 entries");
    Require(c.audio_mask_id < c.audio_vocab_size, "mask id outside the vocabulary");
    Require(c.layers >= 1 && c.vocab_size >= 1 && c.max_positions >= 1,
            "empty model");
    Check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking),
          "hipStreamCreate");
  }
  ~Engine() {
    graphs_.clear();
    if (stream_ != nullptr)
      (void)hipStreamDestroy(stream_);
    if (noise_host_ != nullptr)
      (void)hipHostFree(noise_host_);
  }

  const ovg_config& config() const { return cfg_; }

  // ----------------------------------------------------------- weights
  void LoadSynthetic(std::uint64_t seed, float jitter);
  void UploadPacked(DeviceBuffer<half_t>& dst, const std::vector<half_t>& host, int rows,
                    int k, PackMap map);
  // Float32 host pieces, concatenated on the device in the given order,
  // rounded to fp16 and packed there.
  struct HostPiece {
    const float* data;
    std::size_t count;
  };
  void UploadPackedFloat(DeviceBuffer<half_t>& dst, const std::vector<HostPiece>& pieces,
                         int rows, int k, PackMap map);
  void LoadHost(const ovg_host_weights& w);
  std::int64_t DeviceBytes() const;

  // ----------------------------------------------------------- entry points
  void Forward(const Input& in, float* logits);
  void Score(const Input& in, float guidance, std::int32_t* pred, float* conf);
  int Generate(const std::vector<Input>& inputs, const ovg_decoding& d,
               const std::vector<std::uint64_t>& seeds,
               int (*cancelled)(void*), void* user,
               const std::vector<std::int32_t*>& codes,
               const std::vector<std::int32_t*>& unmasked_at);
  void GenerateTrace(const std::vector<Input>& inputs, const ovg_decoding& d,
                     const std::vector<std::uint64_t>& seeds,
                     const std::vector<std::int32_t*>& codes,
                     const std::vector<std::int32_t*>& unmasked_at,
                     const std::vector<float*>& traces,
                     std::vector<std::int64_t>* executed);
  void Profile(const std::vector<Input>& items, std::int64_t repeats,
               std::map<std::string, KernelStat>* stats);

 private:
  struct GraphEntry {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    ~GraphEntry() {
      if (exec != nullptr)
        (void)hipGraphExecDestroy(exec);
      if (graph != nullptr)
        (void)hipGraphDestroy(graph);
    }
  };

  Layout Plan(const std::vector<Input>& inputs) const;
  void Prepare(const Layout& L);
  void EnqueueForward(const Layout& L, Profiler* prof);
  void EnqueueScore(const Layout& L, float guidance, Profiler* prof);
  void EnqueueSelect(const Layout& L, const ovg_decoding& d, bool from_plan,
                     const SelectStep& single, Profiler* prof);
  void UploadRope();
  void UploadDecodingPlan(const Layout& L, const ovg_decoding& d,
                          const std::vector<std::uint64_t>& seeds,
                          std::vector<int>* launch_steps);
  // Draws the Gumbel noise of executed step k (every item's positions, in
  // the item's own mt19937_64 stream) into pinned host memory and enqueues
  // its copy to the device ahead of that step's kernels, so that the host
  // draws step k + 1's noise while the GPU runs step k.
  void EnqueueNoise(std::size_t k);
  GraphEntry* StepGraph(const Layout& L, const ovg_decoding& d);

  template <typename T>
  void Grow(DeviceBuffer<T>& b, std::size_t count) {
    if (b.Reserve(count))
      graphs_.clear();  // captured graphs hold the old addresses
  }
  template <typename F>
  void Run(Profiler* prof, const char* name, double flops, double bytes,
           F&& launch) {
    if (prof != nullptr)
      prof->Run(name, flops, bytes, launch);
    else
      launch();
  }

  ovg_config cfg_;
  hipStream_t stream_ = nullptr;

  DeviceBuffer<float> text_, audio_, final_norm_;
  DeviceBuffer<half_t> heads_;  // rows padded to a multiple of 128
  DeviceBuffer<float2> rope_;       // [max_positions][64]
  DeviceBuffer<float2> rope_rows_;  // [rows_alloc][64], per packed row
  std::vector<Layer> layers_;

  // Workspace of the packed batch.
  DeviceBuffer<int> ids_, row_kind_, positions_, gather_, epoch_;
  DeviceBuffer<AttentionWork> work_;
  DeviceBuffer<ScoreItem> score_items_;
  DeviceBuffer<SelectItem> select_items_;
  DeviceBuffer<float> hidden_, logits_, conf_, noise_, part_;
  DeviceBuffer<half_t> normed_, qk_, vt_, attn_, act_, final_normed_;
  DeviceBuffer<int> pred_, codes_, unmasked_at_;
  DeviceBuffer<SelectStep> plan_;

  std::map<std::string, std::unique_ptr<GraphEntry>> graphs_;

  // The decoding plan of the current call and its noise streams: executed
  // step k's noise is [noise_begin_[k], noise_begin_[k + 1]) of noise_ (and
  // of the pinned staging noise_host_), items in order.
  std::vector<SelectStep> plan_host_;
  std::vector<std::mt19937_64> noise_random_;
  std::vector<std::size_t> noise_total_, noise_begin_;
  float* noise_host_ = nullptr;
  std::size_t noise_host_count_ = 0;
};

// ------------------------------------------------------------------ weights

void Engine::UploadRope() {
  // Hugging Face's default rotary embedding in float32: inv_freq_i =
  // 1 / theta^(2i / d), angle = position * inv_freq_i, then cos / sin.
  const std::int64_t positions = cfg_.max_positions;
  std::vector<float2> table(static_cast<std::size_t>(positions) * 64);
  float inv_freq[64];
  for (int i = 0; i < 64; ++i)
    inv_freq[i] = 1.0F / std::pow(cfg_.rope_theta, static_cast<float>(2 * i) /
                                                       128.0F);
  ParallelChunks(static_cast<std::size_t>(positions),
                 [&](std::size_t begin, std::size_t end) {
                   for (std::size_t pos = begin; pos < end; ++pos)
                     for (int i = 0; i < 64; ++i) {
                       const float angle = static_cast<float>(pos) * inv_freq[i];
                       table[pos * 64 + i] = make_float2(
                           static_cast<float>(std::cos(static_cast<double>(angle))),
                           static_cast<float>(std::sin(static_cast<double>(angle))));
                     }
                 });
  rope_.Reserve(table.size());
  Check(hipMemcpy(rope_.get(), table.data(), table.size() * sizeof(float2),
                  hipMemcpyHostToDevice),
        "upload rotary table");
}

// Uploads a row-major fp16 matrix and packs it on the device into the
// matrix-core fragment order of the packed GEMM (for kSwiGlu, `host` holds
// the gate rows, then the up rows, `rows` each).
void Engine::UploadPacked(DeviceBuffer<half_t>& dst, const std::vector<half_t>& host,
                          int rows, int k, PackMap map) {
  // The copy goes on the engine's stream, ahead of the packing kernel: a
  // synchronous copy from pageable memory may return before its data has
  // landed, and the non-blocking stream would not wait for it.
  DeviceBuffer<half_t> staging;
  staging.Reserve(host.size());
  Check(hipMemcpyAsync(staging.get(), host.data(), host.size() * sizeof(half_t),
                       hipMemcpyHostToDevice, stream_),
        "upload weights");
  const int out_rows = map == PackMap::kSwiGlu ? 2 * rows : rows;
  dst.Reserve(PackedWeightHalves(out_rows, k));
  PackWeights(staging.get(),
              map == PackMap::kSwiGlu ? staging.get() + static_cast<std::size_t>(rows) * k
                                      : nullptr,
              rows, k, map, static_cast<int>(cfg_.heads / cfg_.kv_heads), dst.get(), stream_);
  Check(hipStreamSynchronize(stream_), "pack weights");
}

void Engine::UploadPackedFloat(DeviceBuffer<half_t>& dst, const std::vector<HostPiece>& pieces,
                               int rows, int k, PackMap map) {
  std::size_t total = 0;
  for (const HostPiece& piece : pieces) {
    Require(piece.data != nullptr, "missing host tensor");
    total += piece.count;
  }
  const int out_rows = map == PackMap::kSwiGlu ? 2 * rows : rows;
  Require(total == static_cast<std::size_t>(out_rows) * k, "host tensor sizes");
  DeviceBuffer<float> staging;
  staging.Reserve(total);
  std::size_t offset = 0;
  for (const HostPiece& piece : pieces) {
    Check(hipMemcpyAsync(staging.get() + offset, piece.data, piece.count * sizeof(float),
                         hipMemcpyHostToDevice, stream_),
          "upload weights");
    offset += piece.count;
  }
  dst.Reserve(PackedWeightHalves(out_rows, k));
  PackWeights(staging.get(),
              map == PackMap::kSwiGlu ? staging.get() + static_cast<std::size_t>(rows) * k
                                      : nullptr,
              rows, k, map, static_cast<int>(cfg_.heads / cfg_.kv_heads), dst.get(), stream_);
  Check(hipStreamSynchronize(stream_), "pack weights");
}

void Engine::LoadSynthetic(std::uint64_t seed, float jitter) {
  const std::size_t h = static_cast<std::size_t>(cfg_.hidden_size);
  const std::size_t inter = static_cast<std::size_t>(cfg_.intermediate_size);
  const std::size_t q_rows = static_cast<std::size_t>(cfg_.heads) * 128;
  const std::size_t kv_rows = static_cast<std::size_t>(cfg_.kv_heads) * 128;
  const std::size_t audio_rows =
      static_cast<std::size_t>(cfg_.audio_codebooks * cfg_.audio_vocab_size);
  UploadRope();

  // Embedding tables (fp32 holding fp16-rounded values), in slabs.
  {
    const std::size_t count = static_cast<std::size_t>(cfg_.vocab_size) * h;
    text_.Reserve(count);
    constexpr std::size_t kSlab = std::size_t{1} << 24;
    std::vector<float> slab(std::min(count, kSlab));
    for (std::size_t first = 0; first < count; first += kSlab) {
      const std::size_t n = std::min(kSlab, count - first);
      SynthFloat(seed, kTextTensor, first, n, false, 0.0F, slab.data());
      Check(hipMemcpy(text_.get() + first, slab.data(), n * sizeof(float),
                      hipMemcpyHostToDevice),
            "upload text embeddings");
    }
  }
  {
    std::vector<float> host(audio_rows * h);
    SynthFloat(seed, kAudioEmbeddingTensor, 0, host.size(), false, 0.0F,
               host.data());
    audio_.Reserve(host.size());
    Check(hipMemcpy(audio_.get(), host.data(), host.size() * sizeof(float),
                    hipMemcpyHostToDevice),
          "upload audio embeddings");
  }
  {
    std::vector<half_t> host(audio_rows * h, static_cast<half_t>(0.0F));
    SynthHalf(seed, kAudioHeadTensor, 0, audio_rows * h, host.data());
    UploadPacked(heads_, host, static_cast<int>(audio_rows), static_cast<int>(h),
                 PackMap::kIdentity);
  }
  {
    std::vector<float> host(h);
    SynthFloat(seed, kFinalNormTensor, 0, h, true, jitter, host.data());
    final_norm_.Reserve(h);
    Check(hipMemcpy(final_norm_.get(), host.data(), h * sizeof(float),
                    hipMemcpyHostToDevice),
          "upload final norm");
  }
  layers_ = std::vector<Layer>(static_cast<std::size_t>(cfg_.layers));
  std::vector<half_t> matrix;
  auto upload_norm = [&](DeviceBuffer<float>& b, std::uint64_t tensor,
                         std::size_t n) {
    std::vector<float> v(n);
    SynthFloat(seed, tensor, 0, n, true, jitter, v.data());
    b.Reserve(n);
    Check(hipMemcpy(b.get(), v.data(), n * sizeof(float),
                    hipMemcpyHostToDevice),
          "upload norm");
  };
  for (std::int64_t l = 0; l < cfg_.layers; ++l) {
    Layer& L = layers_[static_cast<std::size_t>(l)];
    matrix.assign((q_rows + 2 * kv_rows) * h, static_cast<half_t>(0.0F));
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_Q_PROJ), 0, q_rows * h,
              matrix.data());
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_K_PROJ), 0, kv_rows * h,
              matrix.data() + q_rows * h);
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_V_PROJ), 0, kv_rows * h,
              matrix.data() + (q_rows + kv_rows) * h);
    UploadPacked(L.qkv, matrix, static_cast<int>(q_rows + 2 * kv_rows), static_cast<int>(h),
                 PackMap::kRope);
    matrix.assign(h * q_rows, static_cast<half_t>(0.0F));
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_O_PROJ), 0, h * q_rows,
              matrix.data());
    UploadPacked(L.output, matrix, static_cast<int>(h), static_cast<int>(q_rows),
                 PackMap::kIdentity);
    // gate rows, then up rows.
    matrix.assign(2 * inter * h, static_cast<half_t>(0.0F));
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_GATE_PROJ), 0, inter * h, matrix.data());
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_UP_PROJ), 0, inter * h,
              matrix.data() + inter * h);
    UploadPacked(L.gate_up, matrix, static_cast<int>(inter), static_cast<int>(h),
                 PackMap::kSwiGlu);
    matrix.assign(h * inter, static_cast<half_t>(0.0F));
    SynthHalf(seed, LayerTensor(l, OVG_LAYER_DOWN_PROJ), 0, h * inter,
              matrix.data());
    UploadPacked(L.down, matrix, static_cast<int>(h), static_cast<int>(inter),
                 PackMap::kIdentity);
    upload_norm(L.input_norm, LayerTensor(l, OVG_LAYER_INPUT_NORM), h);
    upload_norm(L.post_norm, LayerTensor(l, OVG_LAYER_POST_NORM), h);
    upload_norm(L.q_norm, LayerTensor(l, OVG_LAYER_Q_NORM), 128);
    upload_norm(L.k_norm, LayerTensor(l, OVG_LAYER_K_NORM), 128);
  }
  Check(hipDeviceSynchronize(), "weight upload");
}

void Engine::LoadHost(const ovg_host_weights& w) {
  Require(w.text_embeddings && w.audio_embeddings && w.audio_heads &&
              w.final_norm && w.layers,
          "missing host tensor");
  const std::size_t h = static_cast<std::size_t>(cfg_.hidden_size);
  const std::size_t inter = static_cast<std::size_t>(cfg_.intermediate_size);
  const std::size_t q_rows = static_cast<std::size_t>(cfg_.heads) * 128;
  const std::size_t kv_rows = static_cast<std::size_t>(cfg_.kv_heads) * 128;
  const std::size_t audio_rows =
      static_cast<std::size_t>(cfg_.audio_codebooks * cfg_.audio_vocab_size);
  UploadRope();
  auto upload_float = [](DeviceBuffer<float>& b, const float* src,
                         std::size_t n) {
    Require(src != nullptr, "missing host tensor");
    b.Reserve(n);
    Check(hipMemcpy(b.get(), src, n * sizeof(float), hipMemcpyHostToDevice),
          "upload weights");
  };
  // The matrices go to the device as float32 and are rounded to fp16 there,
  // while being packed (the reference converts on the host,
  // generator.cpp:31-49, with the same rounding).
  upload_float(text_, w.text_embeddings,
               static_cast<std::size_t>(cfg_.vocab_size) * h);
  upload_float(audio_, w.audio_embeddings, audio_rows * h);
  upload_float(final_norm_, w.final_norm, h);
  UploadPackedFloat(heads_, {{w.audio_heads, audio_rows * h}}, static_cast<int>(audio_rows),
                    static_cast<int>(h), PackMap::kIdentity);
  layers_ = std::vector<Layer>(static_cast<std::size_t>(cfg_.layers));
  for (std::int64_t l = 0; l < cfg_.layers; ++l) {
    const float* const* t = w.layers + l * OVG_LAYER_TENSORS;
    Layer& L = layers_[static_cast<std::size_t>(l)];
    UploadPackedFloat(L.qkv,
                      {{t[OVG_LAYER_Q_PROJ], q_rows * h},
                       {t[OVG_LAYER_K_PROJ], kv_rows * h},
                       {t[OVG_LAYER_V_PROJ], kv_rows * h}},
                      static_cast<int>(q_rows + 2 * kv_rows), static_cast<int>(h), PackMap::kRope);
    UploadPackedFloat(L.output, {{t[OVG_LAYER_O_PROJ], h * q_rows}}, static_cast<int>(h),
                      static_cast<int>(q_rows), PackMap::kIdentity);
    UploadPackedFloat(L.gate_up,
                      {{t[OVG_LAYER_GATE_PROJ], inter * h}, {t[OVG_LAYER_UP_PROJ], inter * h}},
                      static_cast<int>(inter), static_cast<int>(h), PackMap::kSwiGlu);
    UploadPackedFloat(L.down, {{t[OVG_LAYER_DOWN_PROJ], h * inter}}, static_cast<int>(h),
                      static_cast<int>(inter), PackMap::kIdentity);
    upload_float(L.input_norm, t[OVG_LAYER_INPUT_NORM], h);
    upload_float(L.post_norm, t[OVG_LAYER_POST_NORM], h);
    upload_float(L.q_norm, t[OVG_LAYER_Q_NORM], 128);
    upload_float(L.k_norm, t[OVG_LAYER_K_NORM], 128);
  }
  Check(hipDeviceSynchronize(), "weight upload");
}

std::int64_t Engine::DeviceBytes() const {
  std::size_t total = text_.bytes() + audio_.bytes() + final_norm_.bytes() +
                      heads_.bytes() + rope_.bytes() + rope_rows_.bytes();
  for (const Layer& L : layers_)
    total += L.qkv.bytes() + L.output.bytes() + L.gate_up.bytes() +
             L.down.bytes() + L.input_norm.bytes() + L.post_norm.bytes() +
             L.q_norm.bytes() + L.k_norm.bytes();
  total += ids_.bytes() + row_kind_.bytes() + positions_.bytes() +
           gather_.bytes() + epoch_.bytes() + work_.bytes() +
           score_items_.bytes() + select_items_.bytes() + hidden_.bytes() +
           logits_.bytes() + conf_.bytes() + noise_.bytes() +
           part_.bytes() + normed_.bytes() + qk_.bytes() +
           vt_.bytes() +
           attn_.bytes() + act_.bytes() + final_normed_.bytes() +
           pred_.bytes() + codes_.bytes() + unmasked_at_.bytes() +
           plan_.bytes();
  return static_cast<std::int64_t>(total);
}

// ------------------------------------------------------------------ layout

// State::Prepare + UploadIds (reference generator.cpp:175-258) for one or
// more inputs: per item the conditional sequence (text, reference frames,
// target frames; positions 0 .. length - 1) and the unconditional sequence
// (its target frames only; positions 0 .. frames - 1), each starting on a
// multiple of 16 rows.
Layout Engine::Plan(const std::vector<Input>& inputs) const {
  Require(!inputs.empty(), "no input");
  const std::int64_t C = cfg_.audio_codebooks;
  const std::int64_t V = cfg_.audio_vocab_size;
  Layout L;
  auto align = [](int r) {
    return (r + kSequenceAlign - 1) / kSequenceAlign * kSequenceAlign;
  };
  int row = 0, logit_row = 0, out_base = 0;
  for (const Input& in : inputs) {
    Require(in.codebooks == C, "input codebooks differ from the model's");
    Require(in.frames >= 1, "no target frames");
    Require(in.audio_start >= 0 && in.audio_start + in.frames <= in.length,
            "inconsistent input layout");
    Require(in.length <= cfg_.max_positions,
            "input longer than the rotary table");
    Require(in.ids != nullptr, "missing input ids");
    ItemLayout it;
    it.length = in.length;
    it.audio_start = in.audio_start;
    it.frames = in.frames;
    it.cond_row = row;
    row = align(row + static_cast<int>(in.length));
    it.uncond_row = row;
    row = align(row + static_cast<int>(in.frames));
    it.logit_row = logit_row;
    logit_row += 2 * static_cast<int>(in.frames);
    it.out_base = out_base;
    out_base += static_cast<int>(C * in.frames);
    L.items.push_back(it);
    L.real_rows += static_cast<int>(in.length + in.frames);
    L.max_frames = std::max(L.max_frames, static_cast<int>(in.frames));
    L.max_total = std::max(L.max_total, static_cast<int>(C * in.frames));
  }
  L.rows = row;
  // One 32-row key tile of slack past the last sequence: attention reads
  // whole key tiles. GEMM operand loads clamp their rows to M - 1, so they
  // need no slack.
  L.rows_alloc = row + 32;
  L.targets = logit_row;
  L.outputs = out_base;
  L.ids.assign(static_cast<std::size_t>(C * L.rows_alloc),
               static_cast<int>(cfg_.audio_mask_id));
  L.row_kind.assign(static_cast<std::size_t>(L.rows_alloc), 2);
  L.positions.assign(static_cast<std::size_t>(L.rows_alloc), 0);
  L.gather.resize(static_cast<std::size_t>(L.targets));
  L.signature = std::to_string(C);
  for (std::size_t i = 0; i < inputs.size(); ++i) {
    const Input& in = inputs[i];
    const ItemLayout& it = L.items[i];
    for (std::int64_t c = 0; c < C; ++c) {
      const std::int32_t* src = in.ids + c * in.length;
      int* dst = L.ids.data() + c * L.rows_alloc;
      for (std::int64_t p = 0; p < in.length; ++p) {
        const std::int32_t id = src[p];
        if (p < in.audio_start) {
          if (c == 0 && (id < 0 || id >= cfg_.vocab_size))
            throw Error("text token outside the vocabulary");
        } else if (id < 0 || id >= V) {
          throw Error("audio code outside the codebook");
        }
        dst[it.cond_row + p] = id;
      }
      for (std::int64_t f = 0; f < in.frames; ++f)
        dst[it.uncond_row + f] = src[in.length - in.frames + f];
    }
    for (std::int64_t p = 0; p < in.length; ++p) {
      L.row_kind[static_cast<std::size_t>(it.cond_row + p)] =
          p < in.audio_start ? 0 : 1;
      L.positions[static_cast<std::size_t>(it.cond_row + p)] =
          static_cast<int>(p);
    }
    for (std::int64_t f = 0; f < in.frames; ++f) {
      L.row_kind[static_cast<std::size_t>(it.uncond_row + f)] = 1;
      L.positions[static_cast<std::size_t>(it.uncond_row + f)] =
          static_cast<int>(f);
      L.gather[static_cast<std::size_t>(it.logit_row + f)] =
          it.cond_row + static_cast<int>(in.length - in.frames + f);
      L.gather[static_cast<std::size_t>(it.logit_row + in.frames + f)] =
          it.uncond_row + static_cast<int>(f);
    }
    for (const auto& [first, length] :
         {std::pair<int, int>{it.cond_row, static_cast<int>(in.length)},
          std::pair<int, int>{it.uncond_row, static_cast<int>(in.frames)}}) {
      for (int q = 0; q < length; q += 32)
        L.work.push_back({first + q, std::min(32, length - q), first, length});
    }
    L.score_items.push_back(
        {it.logit_row, static_cast<int>(in.frames), it.out_base, 0});
    L.select_items.push_back(
        {static_cast<int>(in.frames), it.out_base,
         it.cond_row + static_cast<int>(in.length - in.frames), it.uncond_row});
    L.signature += ":" + std::to_string(in.length) + "/" +
                   std::to_string(in.audio_start) + "/" +
                   std::to_string(in.frames);
  }
  PlanAttentionWork(L.work, &L.exact_work, &L.exact_rounds);
  return L;
}

void Engine::Prepare(const Layout& L) {
  const std::size_t C = static_cast<std::size_t>(cfg_.audio_codebooks);
  const std::size_t ra = static_cast<std::size_t>(L.rows_alloc);
  const std::size_t h = static_cast<std::size_t>(cfg_.hidden_size);
  const std::size_t qk_heads = static_cast<std::size_t>(cfg_.heads + cfg_.kv_heads);
  const std::size_t width =
      static_cast<std::size_t>(cfg_.audio_codebooks * cfg_.audio_vocab_size);
  const int ldvt = (L.rows_alloc + 15) / 16 * 16;
  // q and k: ldvt rows per head in the attention's fragment order
  // (QkIndex), so that a 32-row tile of one head is 8 KB of consecutive
  // bytes.
  const std::size_t ldq = static_cast<std::size_t>(ldvt) * 128;
  Grow(ids_, C * ra);
  Grow(row_kind_, ra);
  Grow(positions_, ra);
  Grow(rope_rows_, ra * 64);
  Grow(gather_, static_cast<std::size_t>(L.targets));
  Grow(epoch_, 1);
  Grow(work_, L.work.size());
  Grow(score_items_, L.score_items.size());
  Grow(select_items_, L.select_items.size());
  Grow(hidden_, ra * h);
  Grow(normed_, ra * h);
  Grow(qk_, qk_heads * ldq);
  Grow(vt_, static_cast<std::size_t>(cfg_.kv_heads) * 128 * ldvt);
  Grow(attn_, ra * static_cast<std::size_t>(cfg_.heads) * 128);
  Grow(act_, ra * static_cast<std::size_t>(cfg_.intermediate_size));
  Grow(final_normed_, static_cast<std::size_t>(L.targets) * h);
  Grow(logits_, static_cast<std::size_t>(L.targets) * width);
  Grow(pred_, static_cast<std::size_t>(L.outputs));
  Grow(conf_, static_cast<std::size_t>(L.outputs));
  Grow(codes_, static_cast<std::size_t>(L.outputs));
  Grow(unmasked_at_, static_cast<std::size_t>(L.outputs));
  const int M = L.rows;
  const int K = static_cast<int>(cfg_.hidden_size);
  const int slices = std::max(
      PlanPacked(M, K, static_cast<int>(cfg_.heads * 128), Epilogue::kPartial).splits,
      PlanPacked(M, K, static_cast<int>(cfg_.intermediate_size), Epilogue::kPartial).splits);
  Grow(part_, static_cast<std::size_t>(slices) * ra * h);
  // The last 32-row tile of the last sequence reads up to 32 rows past the
  // packed rows, which no kernel writes: keep those q/k rows and V^T rows
  // zero, since a masked key's probability 0 times a non-finite stale value
  // would still be NaN (and a query row past the sequence, whose results are
  // dropped, stays finite). Rows inside the packed range, alignment padding
  // included, are written by the q/k/v GEMM every layer. Both layouts store
  // rows interleaved in 16-row blocks (QkIndex, VtIndex), so the clear
  // starts at the block that holds the last packed row (the GEMM rewrites
  // that block's own rows) and is one run of whole blocks per head.
  const int slack = L.rows & ~15;
  Check(hipMemset2DAsync(qk_.get() + QkIndex(0, slack, 0, ldq), ldq * sizeof(half_t), 0,
                         static_cast<std::size_t>(ldvt - slack) * 128 * sizeof(half_t),
                         qk_heads, stream_),
        "clear q/k slack");
  Check(hipMemset2DAsync(vt_.get() + VtIndex(0, 0, slack, ldvt),
                         static_cast<std::size_t>(ldvt) * 128 * sizeof(half_t), 0,
                         static_cast<std::size_t>(ldvt - slack) * 128 * sizeof(half_t),
                         static_cast<std::size_t>(cfg_.kv_heads), stream_),
        "clear value slack");
  auto up = [&](void* dst, const void* src, std::size_t bytes) {
    Check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_),
          "upload batch");
  };
  up(ids_.get(), L.ids.data(), L.ids.size() * sizeof(int));
  up(row_kind_.get(), L.row_kind.data(), L.row_kind.size() * sizeof(int));
  up(positions_.get(), L.positions.data(), L.positions.size() * sizeof(int));
  LaunchRopeRows(rope_.get(), positions_.get(), L.rows_alloc, rope_rows_.get(),
                 stream_);
  up(gather_.get(), L.gather.data(), L.gather.size() * sizeof(int));
  up(work_.get(), L.work.data(), L.work.size() * sizeof(AttentionWork));
  up(score_items_.get(), L.score_items.data(),
     L.score_items.size() * sizeof(ScoreItem));
  up(select_items_.get(), L.select_items.data(),
     L.select_items.size() * sizeof(SelectItem));
  // The host vectors belong to the caller's Layout, which outlives this
  // call, but synchronise anyway so that no copy reads freed memory.
  Check(hipStreamSynchronize(stream_), "upload batch");
}

// ------------------------------------------------------------------ launches

// State::RunForward (reference generator.cpp:262-301).
void Engine::EnqueueForward(const Layout& L, Profiler* prof) {
  const int M = L.rows;
  const int H = static_cast<int>(cfg_.hidden_size);
  const int I = static_cast<int>(cfg_.intermediate_size);
  const int qk_width = static_cast<int>(cfg_.heads + cfg_.kv_heads) * 128;
  const int qkv_n = qk_width + static_cast<int>(cfg_.kv_heads) * 128;
  const int heads_width = static_cast<int>(cfg_.heads) * 128;
  const int ldvt = (L.rows_alloc + 15) / 16 * 16;
  const int ldq = ldvt * 128;  // q/k head stride (head-major)
  const double R = L.real_rows;
  const int C = static_cast<int>(cfg_.audio_codebooks);
  const int Vw = static_cast<int>(cfg_.audio_codebooks * cfg_.audio_vocab_size);

  EmbedParams e{};
  e.ids = ids_.get();
  e.ld_ids = L.rows_alloc;
  e.row_kind = row_kind_.get();
  e.text = text_.get();
  e.audio = audio_.get();
  e.norm = layers_[0].input_norm.get();
  e.hidden = hidden_.get();
  e.normed = normed_.get();
  e.rows = M;
  e.hidden_size = H;
  e.codebooks = C;
  e.vocab = static_cast<int>(cfg_.audio_vocab_size);
  e.eps = cfg_.rms_norm_eps;
  e.epoch = epoch_.get();
  Run(prof, "embed_norm", 0.0, R * H * (4.0 * 2 + 2) + R * C * H * 4.0,
      [&] { LaunchEmbed(e, stream_); });

  auto gemm = [&](const char* name, Epilogue epi, const half_t* x, int lda,
                  const half_t* w, int m, int n, int k, double real_m,
                  double out_bytes, const std::function<void(GemmParams&)>& set) {
    const PackedPlan plan = PlanPacked(m, n, k, epi);
    GemmParams p{};
    p.x = x;
    p.w = w;
    p.lda = lda;
    p.ldb = k;
    p.m = m;
    p.n = n;
    p.k = k;
    p.splits = plan.splits;
    set(p);
    const double flops = 2.0 * real_m * n * k;
    const double bytes = 2.0 * n * k + 2.0 * real_m * k + out_bytes;
    Run(prof, name, flops, bytes, [&] { LaunchPacked(p, plan, epi, stream_); });
  };

  AttentionParams ap{};
  ap.qk = qk_.get();
  ap.vt = vt_.get();
  ap.out = attn_.get();
  ap.work = work_.get();
  ap.work_count = static_cast<int>(L.work.size());
  ap.exact_count = L.exact_work;
  ap.exact_rounds = L.exact_rounds;
  ap.ld_qk = ldq;
  ap.ldvt = ldvt;
  ap.heads = static_cast<int>(cfg_.heads);
  ap.kv_heads = static_cast<int>(cfg_.kv_heads);
  ap.scale_log2 = 1.44269504088896341F / std::sqrt(128.0F);
  double attention_flops = 0.0;
  for (const ItemLayout& it : L.items)
    attention_flops += 4.0 * cfg_.heads * 128.0 *
                       (static_cast<double>(it.length) * it.length +
                        static_cast<double>(it.frames) * it.frames);

  // The o and down projections leave their K-split slices in part_; the
  // next row kernel adds them to the residual stream and applies the
  // following RMSNorm (post-attention, the next layer's input norm, or the
  // final norm on the target rows only).
  const std::size_t part_stride = static_cast<std::size_t>(L.rows_alloc) * H;
  auto add_norm = [&](const char* name, int splits, const float* norm,
                      half_t* out, const int* gather, int rows) {
    AddNormParams a{};
    a.hidden = hidden_.get();
    a.partials = part_.get();
    a.split_stride = part_stride;
    a.splits = splits;
    a.norm = norm;
    a.out = out;
    a.gather = gather;
    a.rows = rows;
    a.width = H;
    a.eps = cfg_.rms_norm_eps;
    Run(prof, name, 0.0, static_cast<double>(rows) * H * (4.0 * (splits + 2) + 2.0),
        [&] { LaunchAddNorm(a, stream_); });
  };
  // How much weight the attention launch prefetches depends on how many
  // CUs it leaves idle. At most 96 busy work-groups (the 2 s shape: 40): the
  // four GEMMs that follow, 31.5 MB. At most 160 (the 10 s shape: 152): only
  // this layer's o, gate/up and down, 22 MB, which the idle CUs read within
  // about the attention's own time (all four: 535 vs 544 unmask steps/s
  // without; these three: 555 vs 546, o and gate/up alone 552, same boxes).
  // With more (clone, chunks) the reads outlast the attention and delay
  // everything after it: none.
  const int attention_busy = static_cast<int>(L.work.size()) * static_cast<int>(cfg_.kv_heads);
  const bool prefetch = attention_busy <= 96;
  const bool prefetch_near = !prefetch && attention_busy <= 160;
  const int o_splits = PlanPacked(M, H, heads_width, Epilogue::kPartial).splits;
  const int down_splits = PlanPacked(M, H, I, Epilogue::kPartial).splits;
  for (std::size_t l = 0; l < layers_.size(); ++l) {
    const Layer& W = layers_[l];
    gemm("gemm_qkv_rope", Epilogue::kQkvRope, normed_.get(), H, W.qkv.get(),
         M, qkv_n, H, R, R * qkv_n * 2.0, [&](GemmParams& p) {
           p.qk = qk_.get();
           p.ldq = ldq;
           p.vt = vt_.get();
           p.ldvt = ldvt;
           p.q_norm = W.q_norm.get();
           p.k_norm = W.k_norm.get();
           p.rope = rope_rows_.get();
           p.heads = static_cast<int>(cfg_.heads);
           p.kv_heads = static_cast<int>(cfg_.kv_heads);
           p.eps = cfg_.rms_norm_eps;
         });
    // The attention leaves CUs idle at short utterances (one work-group per
    // query tile and kv head): there, extra work-groups pull this layer's o,
    // gate/up and down weights, and at the shortest also the next layer's
    // q/k/v (after the last layer: the audio heads and layer 0's q/k/v),
    // into the memory-side cache, from which the GEMMs then stream them.
    // (Prefetch work-groups in the GEMM launches instead, on the CUs their
    // tiles leave free, slowed those GEMMs: 10 s 515 vs 545 unmask steps/s,
    // same box. Moving the down and
    // q/k/v parts into the add + norm launches, which leave CUs idle there
    // too, shortened the attention but made each add + norm wait for its
    // prefetch: 857 vs 870 unmask steps/s at 2 s, same box.)
    const Layer& next = layers_[(l + 1) % layers_.size()];
    const bool last_layer = l + 1 == layers_.size();
    ap.prefetch = WeightPrefetch{};
    if (prefetch_near) {
      SetPrefetch(ap.prefetch, {&W.output, &W.gate_up, &W.down}, kCus - attention_busy);
    } else if (prefetch) {
      if (last_layer)
        SetPrefetch(ap.prefetch, {&W.output, &W.gate_up, &W.down, &heads_, &next.qkv},
                    kCus - attention_busy);
      else
        SetPrefetch(ap.prefetch, {&W.output, &W.gate_up, &W.down, &next.qkv},
                    kCus - attention_busy);
    }
    Run(prof, "attention", attention_flops, R * (qkv_n + heads_width) * 2.0,
        [&] { LaunchAttention(ap, stream_); });
    gemm("gemm_o_partial", Epilogue::kPartial, attn_.get(), heads_width,
         W.output.get(), M, H, heads_width, R, R * H * 4.0 * o_splits,
         [&](GemmParams& p) {
           p.y = part_.get();
           p.ldc = H;
           p.split_stride = part_stride;
         });
    add_norm("add_norm", o_splits, W.post_norm.get(), normed_.get(), nullptr, M);
    gemm("gemm_gate_up_swiglu", Epilogue::kSwiGlu, normed_.get(), H,
         W.gate_up.get(), M, 2 * I, H, R, R * I * 2.0, [&](GemmParams& p) {
           p.act = act_.get();
           p.ldh = I;
         });
    gemm("gemm_down_partial", Epilogue::kPartial, act_.get(), I, W.down.get(),
         M, H, I, R, R * H * 4.0 * down_splits, [&](GemmParams& p) {
           p.y = part_.get();
           p.ldc = H;
           p.split_stride = part_stride;
         });
    if (!last_layer)
      add_norm("add_norm", down_splits, next.input_norm.get(), normed_.get(), nullptr, M);
    else  // GatherRows + final RmsNorm (generator.cpp:295-298)
      add_norm("add_norm_final", down_splits, final_norm_.get(),
               final_normed_.get(), gather_.get(), L.targets);
  }
  gemm("gemm_audio_heads", Epilogue::kStore, final_normed_.get(), H,
       heads_.get(), L.targets, Vw, H, L.targets,
       static_cast<double>(L.targets) * Vw * 4.0, [&](GemmParams& p) {
         p.y = logits_.get();
         p.ldc = Vw;
       });
}

void Engine::EnqueueScore(const Layout& L, float guidance, Profiler* prof) {
  ScoreParams s{};
  s.logits = logits_.get();
  s.items = score_items_.get();
  s.item_count = static_cast<int>(L.items.size());
  s.max_frames = L.max_frames;
  s.codebooks = static_cast<int>(cfg_.audio_codebooks);
  s.vocab = static_cast<int>(cfg_.audio_vocab_size);
  s.width = s.codebooks * s.vocab;
  s.mask_id = cfg_.audio_mask_id;
  s.guidance = guidance;
  s.prediction = pred_.get();
  s.confidence = conf_.get();
  Run(prof, "score", 0.0, static_cast<double>(L.targets) * s.width * 4.0,
      [&] { LaunchScore(s, stream_); });
}

void Engine::EnqueueSelect(const Layout& L, const ovg_decoding& d,
                           bool from_plan, const SelectStep& single,
                           Profiler* prof) {
  SelectParams s{};
  s.prediction = pred_.get();
  s.confidence = conf_.get();
  s.noise = noise_.get();
  s.codes = codes_.get();
  s.unmasked_at = unmasked_at_.get();
  s.ids = ids_.get();
  s.ld_ids = L.rows_alloc;
  s.items = select_items_.get();
  s.item_count = static_cast<int>(L.items.size());
  s.codebooks = static_cast<int>(cfg_.audio_codebooks);
  s.layer_penalty = d.layer_penalty;
  s.temperature = d.position_temperature;
  s.mask_id = cfg_.audio_mask_id;
  s.plan = from_plan ? plan_.get() : nullptr;
  s.epoch = from_plan ? epoch_.get() : nullptr;
  s.single = single;
  Run(prof, "select", 0.0, static_cast<double>(L.outputs) * 16.0,
      [&] { LaunchSelect(s, L.max_total, stream_); });
}

// The executed steps of every item and their Gumbel noise
// (PositionSelector::Fill draws C * F values per executed step when the
// position temperature is positive, decoding.cpp:77-86).
void Engine::UploadDecodingPlan(const Layout& L, const ovg_decoding& d,
                                const std::vector<std::uint64_t>& seeds,
                                std::vector<int>* launch_steps) {
  Require(d.steps >= 1, "steps must be positive");
  const std::size_t items = L.items.size();
  const std::size_t C = static_cast<std::size_t>(cfg_.audio_codebooks);
  std::vector<std::vector<std::size_t>> schedules(items);
  for (std::size_t i = 0; i < items; ++i)
    schedules[i] = UnmaskSchedule(C * static_cast<std::size_t>(L.items[i].frames),
                                  static_cast<std::size_t>(d.steps),
                                  d.t_shift);
  launch_steps->clear();
  for (std::int64_t s = 0; s < d.steps; ++s) {
    bool any = false;
    for (std::size_t i = 0; i < items; ++i)
      any = any || schedules[i][static_cast<std::size_t>(s)] > 0;
    if (any)
      launch_steps->push_back(static_cast<int>(s));
  }
  // Step-major noise offsets: executed step k's noise, all items, is one
  // contiguous range, drawn and uploaded just before step k (EnqueueNoise).
  const bool noisy = d.position_temperature > 0.0F;
  const std::size_t executed = launch_steps->size();
  plan_host_.assign(executed * items, SelectStep{});
  noise_total_.assign(items, 0);
  noise_begin_.assign(executed + 1, 0);
  std::size_t running = 0;
  for (std::size_t k = 0; k < executed; ++k) {
    noise_begin_[k] = running;
    const int step = (*launch_steps)[k];
    for (std::size_t i = 0; i < items; ++i) {
      const std::size_t total = C * static_cast<std::size_t>(L.items[i].frames);
      noise_total_[i] = total;
      SelectStep& st = plan_host_[k * items + i];
      st.step = step;
      st.count = static_cast<int>(schedules[i][static_cast<std::size_t>(step)]);
      st.noise_offset = 0;
      if (noisy && st.count > 0) {
        st.noise_offset = static_cast<int>(running);
        running += total;
      }
    }
  }
  noise_begin_[executed] = running;
  Require(running < (std::size_t{1} << 31), "noise plan too large");
  noise_random_.clear();
  for (std::size_t i = 0; i < items; ++i)
    noise_random_.emplace_back(seeds[i]);
  // Every entry point waits for its stream before it returns, so no copy
  // from the previous staging buffer is pending here.
  if (running > noise_host_count_) {
    if (noise_host_ != nullptr)
      Check(hipHostFree(noise_host_), "hipHostFree");
    noise_host_ = nullptr;
    noise_host_count_ = 0;
    Check(hipHostMalloc(reinterpret_cast<void**>(&noise_host_), running * sizeof(float),
                        hipHostMallocDefault),
          "hipHostMalloc");
    noise_host_count_ = running;
  }
  Grow(plan_, std::max<std::size_t>(plan_host_.size(), 1));
  Grow(noise_, std::max<std::size_t>(running, 1));
  if (!plan_host_.empty())
    Check(hipMemcpyAsync(plan_.get(), plan_host_.data(),
                         plan_host_.size() * sizeof(SelectStep),
                         hipMemcpyHostToDevice, stream_),
          "upload step plan");
}

void Engine::EnqueueNoise(std::size_t k) {
  Require(k + 1 < noise_begin_.size(), "noise step outside the plan");
  const std::size_t begin = noise_begin_[k], end = noise_begin_[k + 1];
  if (end == begin)
    return;
  const std::size_t items = noise_random_.size();
  for (std::size_t i = 0; i < items; ++i) {
    const SelectStep& st = plan_host_[k * items + i];
    if (st.count > 0)
      GumbelNoise(&noise_random_[i], noise_total_[i],
                  noise_host_ + static_cast<std::size_t>(st.noise_offset));
  }
  Check(hipMemcpyAsync(noise_.get() + begin, noise_host_ + begin, (end - begin) * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "upload noise");
}

Engine::GraphEntry* Engine::StepGraph(const Layout& L, const ovg_decoding& d) {
  char key_extra[96];
  std::snprintf(key_extra, sizeof(key_extra), "|%a|%a|%a", d.guidance,
                d.layer_penalty, d.position_temperature);
  const std::string key = L.signature + key_extra;
  if (auto found = graphs_.find(key); found != graphs_.end())
    return found->second.get();
  if (graphs_.size() >= 16)
    graphs_.clear();
  auto entry = std::make_unique<GraphEntry>();
  Check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal),
        "hipStreamBeginCapture");
  try {
    EnqueueForward(L, nullptr);
    EnqueueScore(L, d.guidance, nullptr);
    EnqueueSelect(L, d, true, SelectStep{}, nullptr);
  } catch (...) {
    hipGraph_t broken = nullptr;
    (void)hipStreamEndCapture(stream_, &broken);
    if (broken != nullptr)
      (void)hipGraphDestroy(broken);
    throw;
  }
  Check(hipStreamEndCapture(stream_, &entry->graph), "hipStreamEndCapture");
  Check(hipGraphInstantiate(&entry->exec, entry->graph, nullptr, nullptr, 0),
        "hipGraphInstantiate");
  GraphEntry* raw = entry.get();
  graphs_[key] = std::move(entry);
  return raw;
}

// ------------------------------------------------------------------ entry points

void Engine::Forward(const Input& in, float* logits) {
  const Layout L = Plan({in});
  Prepare(L);
  EnqueueForward(L, nullptr);
  const std::size_t n = static_cast<std::size_t>(L.targets) *
                        static_cast<std::size_t>(cfg_.audio_codebooks *
                                                 cfg_.audio_vocab_size);
  Check(hipMemcpyAsync(logits, logits_.get(), n * sizeof(float),
                       hipMemcpyDeviceToHost, stream_),
        "download logits");
  Check(hipStreamSynchronize(stream_), "forward");
}

void Engine::Score(const Input& in, float guidance, std::int32_t* pred,
                   float* conf) {
  const Layout L = Plan({in});
  Prepare(L);
  EnqueueForward(L, nullptr);
  EnqueueScore(L, guidance, nullptr);
  const std::size_t n = static_cast<std::size_t>(L.outputs);
  Check(hipMemcpyAsync(pred, pred_.get(), n * sizeof(std::int32_t),
                       hipMemcpyDeviceToHost, stream_),
        "download predictions");
  Check(hipMemcpyAsync(conf, conf_.get(), n * sizeof(float),
                       hipMemcpyDeviceToHost, stream_),
        "download confidences");
  Check(hipStreamSynchronize(stream_), "score");
}

int Engine::Generate(const std::vector<Input>& inputs, const ovg_decoding& d,
                     const std::vector<std::uint64_t>& seeds,
                     int (*cancelled)(void*), void* user,
                     const std::vector<std::int32_t*>& codes,
                     const std::vector<std::int32_t*>& unmasked_at) {
  const Layout L = Plan(inputs);
  Require(L.max_total <= kSelectThreads * kSelectPerThread,
          "codebooks * target frames above 16384");
  Prepare(L);
  std::vector<int> launch_steps;
  UploadDecodingPlan(L, d, seeds, &launch_steps);
  LaunchFill(codes_.get(), static_cast<int>(cfg_.audio_mask_id), L.outputs,
             stream_);
  LaunchFill(unmasked_at_.get(), -1, L.outputs, stream_);
  LaunchFill(epoch_.get(), 0, 1, stream_);
  GraphEntry* graph = StepGraph(L, d);
  // At most two steps in flight, so that `cancelled` is polled close to when
  // each step starts while the queue never runs dry.
  hipEvent_t done[2] = {nullptr, nullptr};
  Check(hipEventCreateWithFlags(&done[0], hipEventDisableTiming), "hipEventCreate");
  Check(hipEventCreateWithFlags(&done[1], hipEventDisableTiming), "hipEventCreate");
  int status = OVG_OK;
  try {
    for (std::size_t k = 0; k < launch_steps.size(); ++k) {
      if (k >= 2)
        Check(hipEventSynchronize(done[k % 2]), "step");
      if (cancelled != nullptr && cancelled(user) != 0) {
        status = OVG_CANCELLED;
        break;
      }
      EnqueueNoise(k);
      Check(hipGraphLaunch(graph->exec, stream_), "hipGraphLaunch");
      Check(hipEventRecord(done[k % 2], stream_), "hipEventRecord");
    }
    if (status == OVG_OK) {
      std::vector<std::int32_t> host_codes(static_cast<std::size_t>(L.outputs));
      std::vector<std::int32_t> host_at(static_cast<std::size_t>(L.outputs));
      Check(hipMemcpyAsync(host_codes.data(), codes_.get(),
                           host_codes.size() * sizeof(std::int32_t),
                           hipMemcpyDeviceToHost, stream_),
            "download codes");
      Check(hipMemcpyAsync(host_at.data(), unmasked_at_.get(),
                           host_at.size() * sizeof(std::int32_t),
                           hipMemcpyDeviceToHost, stream_),
            "download unmask steps");
      Check(hipStreamSynchronize(stream_), "generation");
      const std::size_t C = static_cast<std::size_t>(cfg_.audio_codebooks);
      for (std::size_t i = 0; i < L.items.size(); ++i) {
        const std::size_t n = C * static_cast<std::size_t>(L.items[i].frames);
        std::memcpy(codes[i], host_codes.data() + L.items[i].out_base,
                    n * sizeof(std::int32_t));
        std::memcpy(unmasked_at[i], host_at.data() + L.items[i].out_base,
                    n * sizeof(std::int32_t));
      }
    } else {
      Check(hipStreamSynchronize(stream_), "generation");
    }
  } catch (...) {
    (void)hipStreamSynchronize(stream_);
    (void)hipEventDestroy(done[0]);
    (void)hipEventDestroy(done[1]);
    throw;
  }
  (void)hipEventDestroy(done[0]);
  (void)hipEventDestroy(done[1]);
  return status;
}

// Generate launched eagerly, downloading every item's logits at each step
// the item executes (its schedule's count is positive there).
void Engine::GenerateTrace(const std::vector<Input>& inputs, const ovg_decoding& d,
                           const std::vector<std::uint64_t>& seeds,
                           const std::vector<std::int32_t*>& codes,
                           const std::vector<std::int32_t*>& unmasked_at,
                           const std::vector<float*>& traces,
                           std::vector<std::int64_t>* executed) {
  const Layout L = Plan(inputs);
  Require(L.max_total <= kSelectThreads * kSelectPerThread,
          "codebooks * target frames above 16384");
  Prepare(L);
  std::vector<int> launch_steps;
  UploadDecodingPlan(L, d, seeds, &launch_steps);
  LaunchFill(codes_.get(), static_cast<int>(cfg_.audio_mask_id), L.outputs,
             stream_);
  LaunchFill(unmasked_at_.get(), -1, L.outputs, stream_);
  LaunchFill(epoch_.get(), 0, 1, stream_);
  const std::size_t C = static_cast<std::size_t>(cfg_.audio_codebooks);
  const std::size_t width = C * static_cast<std::size_t>(cfg_.audio_vocab_size);
  std::vector<std::vector<std::size_t>> schedules;
  for (const ItemLayout& it : L.items)
    schedules.push_back(UnmaskSchedule(C * static_cast<std::size_t>(it.frames),
                                       static_cast<std::size_t>(d.steps), d.t_shift));
  executed->assign(L.items.size(), 0);
  for (std::size_t k = 0; k < launch_steps.size(); ++k) {
    const int step = launch_steps[k];
    EnqueueNoise(k);
    EnqueueForward(L, nullptr);
    EnqueueScore(L, d.guidance, nullptr);
    for (std::size_t i = 0; i < L.items.size(); ++i) {
      if (schedules[i][static_cast<std::size_t>(step)] == 0)
        continue;
      const ItemLayout& it = L.items[i];
      const std::size_t rows = 2 * static_cast<std::size_t>(it.frames);
      if (traces[i] != nullptr)
        Check(hipMemcpyAsync(traces[i] + static_cast<std::size_t>((*executed)[i]) * rows * width,
                             logits_.get() + static_cast<std::size_t>(it.logit_row) * width,
                             rows * width * sizeof(float), hipMemcpyDeviceToHost, stream_),
              "download logits");
      ++(*executed)[i];
    }
    EnqueueSelect(L, d, true, SelectStep{}, nullptr);
  }
  std::vector<std::int32_t> host_codes(static_cast<std::size_t>(L.outputs));
  std::vector<std::int32_t> host_at(static_cast<std::size_t>(L.outputs));
  Check(hipMemcpyAsync(host_codes.data(), codes_.get(),
                       host_codes.size() * sizeof(std::int32_t),
                       hipMemcpyDeviceToHost, stream_),
        "download codes");
  Check(hipMemcpyAsync(host_at.data(), unmasked_at_.get(),
                       host_at.size() * sizeof(std::int32_t), hipMemcpyDeviceToHost,
                       stream_),
        "download unmask steps");
  Check(hipStreamSynchronize(stream_), "generation");
  for (std::size_t i = 0; i < L.items.size(); ++i) {
    const std::size_t n = C * static_cast<std::size_t>(L.items[i].frames);
    std::memcpy(codes[i], host_codes.data() + L.items[i].out_base, n * sizeof(std::int32_t));
    std::memcpy(unmasked_at[i], host_at.data() + L.items[i].out_base,
                n * sizeof(std::int32_t));
  }
}

void Engine::Profile(const std::vector<Input>& items, std::int64_t repeats,
                     std::map<std::string, KernelStat>* stats) {
  const Layout L = Plan(items);
  Prepare(L);
  ovg_decoding d{32, 2.0F, 0.1F, 5.0F, 0.0F};
  std::vector<int> launch_steps;
  UploadDecodingPlan(L, d, std::vector<std::uint64_t>(items.size(), 0), &launch_steps);
  for (std::int64_t r = 0; r < std::max<std::int64_t>(repeats, 1); ++r) {
    LaunchFill(codes_.get(), static_cast<int>(cfg_.audio_mask_id), L.outputs,
               stream_);
    LaunchFill(epoch_.get(), 0, 1, stream_);
    Profiler prof(stream_);
    EnqueueForward(L, &prof);
    EnqueueScore(L, d.guidance, &prof);
    EnqueueSelect(L, d, true, SelectStep{}, &prof);
    prof.Collect(stats);
  }
}

}  // namespace ovg

// ====================================================================== C ABI

struct ovg_handle {
  std::unique_ptr<ovg::Engine> engine;
};

namespace {

void SetError(char* error, std::size_t len, const std::string& message) {
  if (error == nullptr || len == 0)
    return;
  const std::size_t n = std::min(len - 1, message.size());
  std::memcpy(error, message.data(), n);
  error[n] = '\0';
}

ovg::Input ToInput(const ovg_input* in) {
  ovg::Require(in != nullptr, "missing input");
  ovg::Require(in->codebooks > 0 && in->length > 0 && in->target_frames > 0,
               "empty input");
  return {in->codebooks, in->length, in->audio_start, in->target_frames,
          in->ids};
}

template <typename F>
int Guard(const char* prefix, char* error, std::size_t len, F&& body) {
  try {
    return body();
  } catch (const std::exception& failure) {
    SetError(error, len, std::string(prefix) + failure.what());
    return OVG_ERROR;
  }
}

}  // namespace

extern "C" {

int ovg_create(const ovg_config* config, const char* model_root,
               uint64_t /*weight_seed*/, ovg_handle** handle, char* error,
               size_t error_len) {
  return Guard("OmniVoice generator: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    // Every tensor is located and checked against the config before the GPU
    // is touched (reference: generator.cpp:364-434 reads the same names).
    // The file is model_root / "model.safetensors" as std::filesystem joins
    // it: an empty root names model.safetensors in the working directory,
    // which the reference's Load tries too and fails on when it is absent.
    const auto file = ovg::SafetensorsFile::Open(
        ovg::JoinPath(model_root == nullptr ? "" : model_root, "model.safetensors"));
    const ovg_config& c = *config;
    const std::int64_t h = c.hidden_size, q_rows = c.heads * c.head_dim,
                       kv_rows = c.kv_heads * c.head_dim,
                       audio_rows = c.audio_codebooks * c.audio_vocab_size;
    ovg::Require(c.layers >= 1, "empty model");
    std::vector<const float*> layers(
        static_cast<std::size_t>(c.layers) * OVG_LAYER_TENSORS);
    for (std::int64_t l = 0; l < c.layers; ++l) {
      const std::string prefix = "llm.layers." + std::to_string(l) + ".";
      const float** t = layers.data() + l * OVG_LAYER_TENSORS;
      t[OVG_LAYER_Q_PROJ] = file->F32(prefix + "self_attn.q_proj.weight", {q_rows, h});
      t[OVG_LAYER_K_PROJ] = file->F32(prefix + "self_attn.k_proj.weight", {kv_rows, h});
      t[OVG_LAYER_V_PROJ] = file->F32(prefix + "self_attn.v_proj.weight", {kv_rows, h});
      t[OVG_LAYER_O_PROJ] = file->F32(prefix + "self_attn.o_proj.weight", {h, q_rows});
      t[OVG_LAYER_GATE_PROJ] =
          file->F32(prefix + "mlp.gate_proj.weight", {c.intermediate_size, h});
      t[OVG_LAYER_UP_PROJ] =
          file->F32(prefix + "mlp.up_proj.weight", {c.intermediate_size, h});
      t[OVG_LAYER_DOWN_PROJ] =
          file->F32(prefix + "mlp.down_proj.weight", {h, c.intermediate_size});
      t[OVG_LAYER_INPUT_NORM] = file->F32(prefix + "input_layernorm.weight", {h});
      t[OVG_LAYER_POST_NORM] =
          file->F32(prefix + "post_attention_layernorm.weight", {h});
      t[OVG_LAYER_Q_NORM] = file->F32(prefix + "self_attn.q_norm.weight", {c.head_dim});
      t[OVG_LAYER_K_NORM] = file->F32(prefix + "self_attn.k_norm.weight", {c.head_dim});
    }
    ovg_host_weights w{};
    w.text_embeddings = file->F32("llm.embed_tokens.weight", {c.vocab_size, h});
    w.audio_embeddings = file->F32("audio_embeddings.weight", {audio_rows, h});
    w.audio_heads = file->F32("audio_heads.weight", {audio_rows, h});
    w.final_norm = file->F32("llm.norm.weight", {h});
    w.layers = layers.data();
    auto created = std::make_unique<ovg_handle>();
    created->engine = std::make_unique<ovg::Engine>(c);
    created->engine->LoadHost(w);
    *handle = created.release();
    return OVG_OK;
  });
}

int ovg_create_synthetic(const ovg_config* config, uint64_t weight_seed,
                         float norm_jitter, ovg_handle** handle, char* error,
                         size_t error_len) {
  return Guard("OmniVoice generator: ", error, error_len, [&] {
    ovg::Require(config != nullptr && handle != nullptr, "null argument");
    auto h = std::make_unique<ovg_handle>();
    h->engine = std::make_unique<ovg::Engine>(*config);
    h->engine->LoadSynthetic(weight_seed, norm_jitter);
    *handle = h.release();
    return OVG_OK;
  });
}

int ovg_create_from_host(const ovg_config* config,
                         const ovg_host_weights* weights, ovg_handle** handle,
                         char* error, size_t error_len) {
  return Guard("OmniVoice generator: ", error, error_len, [&] {
    ovg::Require(config != nullptr && weights != nullptr && handle != nullptr,
                 "null argument");
    auto h = std::make_unique<ovg_handle>();
    h->engine = std::make_unique<ovg::Engine>(*config);
    h->engine->LoadHost(*weights);
    *handle = h.release();
    return OVG_OK;
  });
}

void ovg_destroy(ovg_handle* handle) { delete handle; }

int ovg_forward(ovg_handle* handle, const ovg_input* input, float* logits,
                char* error, size_t error_len) {
  return Guard("OmniVoice forward: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && logits != nullptr, "null argument");
    handle->engine->Forward(ToInput(input), logits);
    return OVG_OK;
  });
}

int ovg_score(ovg_handle* handle, const ovg_input* input, float guidance,
              int32_t* prediction, float* confidence, char* error,
              size_t error_len) {
  return Guard("OmniVoice score: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && prediction != nullptr &&
                     confidence != nullptr,
                 "null argument");
    handle->engine->Score(ToInput(input), guidance, prediction, confidence);
    return OVG_OK;
  });
}

int ovg_generate(ovg_handle* handle, const ovg_input* input,
                 const ovg_decoding* decoding, uint64_t seed,
                 int (*cancelled)(void* user), void* user, int32_t* codes,
                 int32_t* unmasked_at, char* error, size_t error_len) {
  return ovg_generate_batch(handle, 1, input, decoding, &seed, cancelled,
                            user, &codes, &unmasked_at, error, error_len);
}

int ovg_generate_batch(ovg_handle* handle, int64_t count,
                       const ovg_input* inputs, const ovg_decoding* decoding,
                       const uint64_t* seeds, int (*cancelled)(void* user),
                       void* user, int32_t* const* codes,
                       int32_t* const* unmasked_at, char* error,
                       size_t error_len) {
  const int status = Guard("OmniVoice generation: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && inputs != nullptr &&
                     decoding != nullptr && seeds != nullptr &&
                     codes != nullptr && unmasked_at != nullptr && count > 0,
                 "null argument");
    std::vector<ovg::Input> list;
    std::vector<std::uint64_t> seed_list;
    std::vector<std::int32_t*> code_list, at_list;
    for (int64_t i = 0; i < count; ++i) {
      list.push_back(ToInput(&inputs[i]));
      seed_list.push_back(seeds[i]);
      ovg::Require(codes[i] != nullptr && unmasked_at[i] != nullptr,
                   "null output");
      code_list.push_back(codes[i]);
      at_list.push_back(unmasked_at[i]);
    }
    return handle->engine->Generate(list, *decoding, seed_list, cancelled,
                                    user, code_list, at_list);
  });
  if (status == OVG_CANCELLED)
    SetError(error, error_len, "cancelled");
  return status;
}

int ovg_generate_chunks(ovg_handle* handle, int64_t count,
                        const uint32_t* const* text_ids, const int64_t* text_counts,
                        const int32_t* reference_codes, int64_t reference_frames,
                        const int64_t* target_frames, const ovg_decoding* decoding,
                        uint64_t seed, int (*cancelled)(void* user), void* user,
                        int32_t* const* codes, int32_t* const* unmasked_at, char* error,
                        size_t error_len) {
  const int status = Guard("OmniVoice generation: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && text_ids != nullptr && text_counts != nullptr &&
                     target_frames != nullptr && decoding != nullptr && codes != nullptr &&
                     unmasked_at != nullptr && count > 0,
                 "null argument");
    ovg::Require(reference_frames >= 0 && (reference_frames == 0 || reference_codes != nullptr),
                 "missing reference codes");
    const ovg_config& c = handle->engine->config();
    const std::size_t C = static_cast<std::size_t>(c.audio_codebooks);
    for (int64_t i = 0; i < count; ++i)
      ovg::Require(text_counts[i] >= 0 && (text_counts[i] == 0 || text_ids[i] != nullptr) &&
                       target_frames[i] >= 1 && codes[i] != nullptr &&
                       unmasked_at[i] != nullptr,
                   "bad chunk");
    // ConditionalInput::Build (decoding.cpp:42-62) of chunk i against a
    // reference.
    auto build = [&](int64_t i, const std::vector<std::int32_t>& ref, std::size_t ref_frames) {
      const std::vector<std::uint32_t> text(text_ids[i], text_ids[i] + text_counts[i]);
      return ovg::BuildInput(text, ref, ref_frames, static_cast<std::size_t>(target_frames[i]),
                             C, c.audio_mask_id);
    };
    auto input = [&](int64_t i, const std::vector<std::int32_t>& ids, std::size_t ref_frames) {
      return ovg::Input{c.audio_codebooks,
                        text_counts[i] + static_cast<std::int64_t>(ref_frames) + target_frames[i],
                        text_counts[i], target_frames[i], ids.data()};
    };
    std::vector<std::int32_t> reference;
    if (reference_frames > 0)
      reference.assign(reference_codes, reference_codes + C * reference_frames);
    std::size_t ref_frames = static_cast<std::size_t>(reference_frames);
    int64_t first = 0;
    if (reference_frames == 0 && count > 1) {
      // Without a reference voice, chunk 0 runs alone and its codes carry
      // the voice into the others (synthesizer.cpp:195-200).
      const auto ids = build(0, {}, 0);
      const int done = handle->engine->Generate({input(0, ids, 0)}, *decoding, {seed}, cancelled,
                                                user, {codes[0]}, {unmasked_at[0]});
      if (done != OVG_OK)
        return done;
      reference.assign(codes[0], codes[0] + C * target_frames[0]);
      ref_frames = static_cast<std::size_t>(target_frames[0]);
      first = 1;
    }
    std::vector<std::vector<std::int32_t>> ids;
    for (int64_t i = first; i < count; ++i)
      ids.push_back(build(i, reference, ref_frames));
    std::vector<ovg::Input> list;
    std::vector<std::int32_t*> code_list, at_list;
    for (int64_t i = first; i < count; ++i) {
      list.push_back(input(i, ids[static_cast<std::size_t>(i - first)], ref_frames));
      code_list.push_back(codes[i]);
      at_list.push_back(unmasked_at[i]);
    }
    // Every chunk takes the request's seed, as each of the reference's
    // Generate calls does (synthesizer.cpp:70-71).
    return handle->engine->Generate(list, *decoding,
                                    std::vector<std::uint64_t>(list.size(), seed), cancelled,
                                    user, code_list, at_list);
  });
  if (status == OVG_CANCELLED)
    SetError(error, error_len, "cancelled");
  return status;
}

int ovg_generate_trace(ovg_handle* handle, const ovg_input* input,
                       const ovg_decoding* decoding, uint64_t seed,
                       int32_t* codes, int32_t* unmasked_at,
                       float* logits_trace, int64_t* executed, char* error,
                       size_t error_len) {
  return ovg_generate_trace_batch(handle, 1, input, decoding, &seed, &codes, &unmasked_at,
                                  &logits_trace, executed, error, error_len);
}

int ovg_generate_trace_batch(ovg_handle* handle, int64_t count, const ovg_input* inputs,
                             const ovg_decoding* decoding, const uint64_t* seeds,
                             int32_t* const* codes, int32_t* const* unmasked_at,
                             float* const* logits_traces, int64_t* executed,
                             char* error, size_t error_len) {
  return Guard("OmniVoice generation: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && inputs != nullptr && decoding != nullptr &&
                     seeds != nullptr && codes != nullptr && unmasked_at != nullptr &&
                     count > 0,
                 "null argument");
    std::vector<ovg::Input> list;
    std::vector<std::uint64_t> seed_list;
    std::vector<std::int32_t*> code_list, at_list;
    std::vector<float*> trace_list;
    for (int64_t i = 0; i < count; ++i) {
      list.push_back(ToInput(&inputs[i]));
      seed_list.push_back(seeds[i]);
      ovg::Require(codes[i] != nullptr && unmasked_at[i] != nullptr, "null output");
      code_list.push_back(codes[i]);
      at_list.push_back(unmasked_at[i]);
      trace_list.push_back(logits_traces == nullptr ? nullptr : logits_traces[i]);
    }
    std::vector<std::int64_t> steps;
    handle->engine->GenerateTrace(list, *decoding, seed_list, code_list, at_list, trace_list,
                                  &steps);
    if (executed != nullptr)
      for (int64_t i = 0; i < count; ++i)
        executed[i] = steps[static_cast<std::size_t>(i)];
    return OVG_OK;
  });
}

int ovg_profile_batch(ovg_handle* handle, int64_t items,
                      const ovg_input* inputs, int64_t repeats,
                      ovg_kernel_stat* stats, int64_t capacity, int64_t* count,
                      char* error, size_t error_len) {
  return Guard("OmniVoice profile: ", error, error_len, [&] {
    ovg::Require(handle != nullptr && count != nullptr && inputs != nullptr &&
                     items > 0,
                 "null argument");
    std::vector<ovg::Input> list;
    for (int64_t i = 0; i < items; ++i)
      list.push_back(ToInput(&inputs[i]));
    std::map<std::string, ovg::KernelStat> table;
    handle->engine->Profile(list, repeats, &table);
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

int ovg_profile_step(ovg_handle* handle, const ovg_input* input,
                     int64_t repeats, ovg_kernel_stat* stats,
                     int64_t capacity, int64_t* count, char* error,
                     size_t error_len) {
  return ovg_profile_batch(handle, 1, input, repeats, stats, capacity, count,
                           error, error_len);
}

void ovg_synthetic_values(uint64_t weight_seed, uint64_t tensor, uint64_t first,
                          int64_t count, int is_norm, float norm_jitter,
                          float* out) {
  if (count <= 0 || out == nullptr)
    return;
  ovg::SynthFloat(weight_seed, tensor, first, static_cast<std::size_t>(count),
                  is_norm != 0, norm_jitter, out);
}

int64_t ovg_device_bytes(const ovg_handle* handle) {
  return handle == nullptr ? 0 : handle->engine->DeviceBytes();
}

int ovg_unmask_schedule(int64_t total, int64_t steps, float t_shift,
                        int64_t* schedule) {
  if (total < 0 || steps <= 0 || schedule == nullptr)
    return OVG_ERROR;
  const auto s = ovg::UnmaskSchedule(static_cast<std::size_t>(total),
                                     static_cast<std::size_t>(steps), t_shift);
  for (std::size_t i = 0; i < s.size(); ++i)
    schedule[i] = static_cast<int64_t>(s[i]);
  return OVG_OK;
}

int64_t ovg_build_input(const uint32_t* text_ids, int64_t text_count,
                        const int32_t* reference_codes,
                        int64_t reference_frames, int64_t target_frames,
                        int64_t codebooks, uint32_t mask_id, int32_t* ids) {
  if (text_count < 0 || reference_frames < 0 || target_frames < 0 ||
      codebooks <= 0 || ids == nullptr ||
      (reference_frames > 0 && reference_codes == nullptr) ||
      (text_count > 0 && text_ids == nullptr))
    return -1;
  const std::vector<std::uint32_t> text(text_ids, text_ids + text_count);
  std::vector<std::int32_t> reference;
  if (reference_frames > 0)
    reference.assign(reference_codes,
                     reference_codes + codebooks * reference_frames);
  const auto built = ovg::BuildInput(
      text, reference, static_cast<std::size_t>(reference_frames),
      static_cast<std::size_t>(target_frames),
      static_cast<std::size_t>(codebooks), mask_id);
  std::memcpy(ids, built.data(), built.size() * sizeof(std::int32_t));
  return text_count + reference_frames + target_frames;
}

}  // extern "C"
