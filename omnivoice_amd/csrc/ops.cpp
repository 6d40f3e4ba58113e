// Device operators on caller-owned device pointers (include/omnivoice_mi355x.h,
// "Device operators"): each is one launcher of the generator's kernels
// behind the C ABI, for integration and for per-kernel parity tests.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>

#include "../../include/omnivoice_mi355x.h"
#include "kernels.hpp"

namespace {

void SetError(char* error, std::size_t len, const std::string& message) {
  if (error == nullptr || len == 0)
    return;
  const std::size_t n = std::min(len - 1, message.size());
  std::memcpy(error, message.data(), n);
  error[n] = '\0';
}

template <typename F>
int Guard(const char* prefix, char* error, std::size_t len, F&& body) {
  try {
    body();
    return OVG_OK;
  } catch (const std::exception& failure) {
    SetError(error, len, std::string(prefix) + failure.what());
    return OVG_ERROR;
  }
}

bool FitsInt(int64_t v) { return v >= 0 && v <= (int64_t{1} << 30); }

// A device allocation that lives for one operator call.
template <typename T>
struct Scratch {
  T* data = nullptr;
  explicit Scratch(std::size_t count) {
    ovg::Check(hipMalloc(reinterpret_cast<void**>(&data),
                         std::max<std::size_t>(count, 1) * sizeof(T)),
               "hipMalloc");
  }
  ~Scratch() {
    if (data != nullptr)
      (void)hipFree(data);
  }
};

}  // namespace

extern "C" {

int ovg_op_score(const float* logits, int32_t* prediction, float* confidence,
                 int64_t frames, int64_t codebooks, int64_t vocab,
                 uint32_t mask_id, float guidance, void* stream, char* error,
                 size_t error_len) {
  return Guard("score: ", error, error_len, [&] {
    ovg::Require(logits && prediction && confidence, "null pointer");
    ovg::Require(frames >= 1 && FitsInt(frames) && codebooks >= 1 &&
                     codebooks <= 64 && vocab >= 1 && vocab <= 1088,
                 "shape outside the kernel's range");
    auto s = static_cast<hipStream_t>(stream);
    Scratch<ovg::ScoreItem> item(1);
    const ovg::ScoreItem host{0, static_cast<int>(frames), 0, 0};
    ovg::Check(hipMemcpyAsync(item.data, &host, sizeof(host),
                              hipMemcpyHostToDevice, s),
               "upload");
    ovg::ScoreParams p{};
    p.logits = logits;
    p.items = item.data;
    p.item_count = 1;
    p.max_frames = static_cast<int>(frames);
    p.codebooks = static_cast<int>(codebooks);
    p.vocab = static_cast<int>(vocab);
    p.width = p.codebooks * p.vocab;
    p.mask_id = mask_id;
    p.guidance = guidance;
    p.prediction = prediction;
    p.confidence = confidence;
    ovg::LaunchScore(p, s);
    ovg::Check(hipStreamSynchronize(s), "score");
  });
}

int ovg_op_select(const int32_t* prediction, const float* confidence,
                  const float* noise, int32_t* codes, int32_t* unmasked_at,
                  int64_t codebooks, int64_t frames, int64_t count,
                  int32_t step, float layer_penalty, float temperature,
                  uint32_t mask_id, void* stream, char* error,
                  size_t error_len) {
  return Guard("select: ", error, error_len, [&] {
    ovg::Require(prediction && confidence && codes && unmasked_at,
                 "null pointer");
    ovg::Require(temperature <= 0.0F || noise != nullptr,
                 "noise required when the temperature is positive");
    ovg::Require(codebooks >= 1 && frames >= 1 &&
                     codebooks * frames <=
                         ovg::kSelectThreads * ovg::kSelectPerThread,
                 "codebooks * frames outside [1, 16384]");
    ovg::Require(count >= 0, "negative count");
    auto s = static_cast<hipStream_t>(stream);
    Scratch<ovg::SelectItem> item(1);
    const ovg::SelectItem host{static_cast<int>(frames), 0, 0, 0};
    ovg::Check(hipMemcpyAsync(item.data, &host, sizeof(host),
                              hipMemcpyHostToDevice, s),
               "upload");
    ovg::SelectParams p{};
    p.prediction = prediction;
    p.confidence = confidence;
    p.noise = noise;
    p.codes = codes;
    p.unmasked_at = unmasked_at;
    p.ids = nullptr;
    p.items = item.data;
    p.item_count = 1;
    p.codebooks = static_cast<int>(codebooks);
    p.layer_penalty = layer_penalty;
    p.temperature = temperature;
    p.mask_id = mask_id;
    p.plan = nullptr;
    p.epoch = nullptr;
    p.single = {step, static_cast<int>(std::min<int64_t>(count, 1 << 30)), 0, 0};
    ovg::LaunchSelect(p, static_cast<int>(codebooks * frames), s);
    ovg::Check(hipStreamSynchronize(s), "select");
  });
}

int ovg_op_linear(const void* x, const void* w, float* y, int64_t rows,
                  int64_t in, int64_t out, int accumulate, void* stream,
                  char* error, size_t error_len) {
  return Guard("linear: ", error, error_len, [&] {
    ovg::Require(x && w && y, "null pointer");
    ovg::Require(rows >= 1 && in >= 64 && out >= 1 && FitsInt(rows) &&
                     FitsInt(in) && FitsInt(out),
                 "empty or oversized shape");
    auto s = static_cast<hipStream_t>(stream);
    const auto epi =
        accumulate ? ovg::Epilogue::kAccumulate : ovg::Epilogue::kStore;
    const ovg::GemmPlan plan = ovg::PlanGemm(
        static_cast<int>(rows), static_cast<int>(out), static_cast<int>(in), epi, true);
    Scratch<float> partials(plan.partial_floats);
    ovg::GemmParams p{};
    p.x = static_cast<const ovg::half_t*>(x);
    p.w = static_cast<const ovg::half_t*>(w);
    p.lda = static_cast<int>(in);
    p.ldb = static_cast<int>(in);
    p.m = static_cast<int>(rows);
    p.n = static_cast<int>(out);
    p.k = static_cast<int>(in);
    p.splits = plan.splits;
    p.partials = partials.data;
    p.y = y;
    p.ldc = static_cast<int>(out);
    ovg::LaunchGemm(p, plan, epi, s);
    ovg::Check(hipStreamSynchronize(s), "linear");
  });
}

int ovg_op_linear_packed(const void* x, const void* w, float* y, int64_t rows,
                         int64_t in, int64_t out, int accumulate, int64_t tile_rows,
                         int64_t tile_cols, void* stream, char* error, size_t error_len) {
  return Guard("linear: ", error, error_len, [&] {
    ovg::Require(x && w && y, "null pointer");
    ovg::Require(rows >= 1 && in >= 64 && out >= 1 && FitsInt(rows) &&
                     FitsInt(in) && FitsInt(out),
                 "empty or oversized shape");
    const bool rows_ok = tile_rows == 32 || tile_rows == 64 || tile_rows == 96 || tile_rows == 128;
    const bool narrow = (tile_cols == 128 || tile_cols == 64 || tile_cols == 32) && rows_ok;
    const bool wide = tile_cols == 256 && (tile_rows == 128 || tile_rows == 256);
    ovg::Require((tile_rows == 0 && tile_cols == 0) || narrow || wide,
                 "tile must be 0 x 0 (planned), 32/64/96/128 x 128, 64 or 32, 128 x 256 or "
                 "256 x 256");
    auto s = static_cast<hipStream_t>(stream);
    const auto epi =
        accumulate ? ovg::Epilogue::kAccumulate : ovg::Epilogue::kStore;
    Scratch<ovg::half_t> packed(ovg::PackedWeightHalves(static_cast<int>(out),
                                                        static_cast<int>(in)));
    ovg::PackWeights(static_cast<const ovg::half_t*>(w), nullptr, static_cast<int>(out),
                     static_cast<int>(in), ovg::PackMap::kIdentity, 0, packed.data, s);
    ovg::PackedPlan plan = ovg::PlanPacked(static_cast<int>(rows), static_cast<int>(out),
                                           static_cast<int>(in), epi);
    if (tile_rows != 0) {
      plan.n_main = 0;  // one launch of the forced tile
      plan.xb = static_cast<int>(tile_rows / 32);
      plan.wb = tile_cols == 256 ? 2 : 1;
      plan.nw = tile_cols == 64 ? 2 : tile_cols == 32 ? 1 : 4;
      plan.tiles = (static_cast<int>(rows) + static_cast<int>(tile_rows) - 1) /
                   static_cast<int>(tile_rows) *
                   ((static_cast<int>(out) + static_cast<int>(tile_cols) - 1) /
                    static_cast<int>(tile_cols));
    }
    ovg::GemmParams p{};
    p.x = static_cast<const ovg::half_t*>(x);
    p.w = packed.data;
    p.lda = static_cast<int>(in);
    p.ldb = static_cast<int>(in);
    p.m = static_cast<int>(rows);
    p.n = static_cast<int>(out);
    p.k = static_cast<int>(in);
    p.splits = plan.splits;
    p.y = y;
    p.ldc = static_cast<int>(out);
    ovg::LaunchPacked(p, plan, epi, s);
    ovg::Check(hipStreamSynchronize(s), "linear");
  });
}

int ovg_op_rmsnorm(const float* input, const float* weight, void* output,
                   int64_t rows, int64_t width, float epsilon, void* stream,
                   char* error, size_t error_len) {
  return Guard("rmsnorm: ", error, error_len, [&] {
    ovg::Require(input && weight && output, "null pointer");
    ovg::Require(rows >= 1 && FitsInt(rows), "bad rows");
    auto s = static_cast<hipStream_t>(stream);
    ovg::LaunchRmsNorm(input, nullptr, weight,
                       static_cast<ovg::half_t*>(output), static_cast<int>(rows),
                       static_cast<int>(width), epsilon, s);
    ovg::Check(hipStreamSynchronize(s), "rmsnorm");
  });
}

int ovg_op_attention(const void* qkv, void* output, int64_t rows,
                     int64_t heads, int64_t kv_heads,
                     const int64_t* sequences, int64_t count, void* stream,
                     char* error, size_t error_len) {
  return Guard("attention: ", error, error_len, [&] {
    ovg::Require(qkv && output && sequences, "null pointer");
    ovg::Require(rows >= 1 && FitsInt(rows) && heads >= 1 && kv_heads >= 1 &&
                     heads <= 64 && count >= 1,
                 "bad shape");
    const int ld_qkv = static_cast<int>((heads + 2 * kv_heads) * 128);
    std::vector<ovg::AttentionWork> work;
    int64_t end = 0;
    for (int64_t i = 0; i < count; ++i) {
      const int64_t first = sequences[2 * i], length = sequences[2 * i + 1];
      ovg::Require(first >= 0 && length >= 1 && first + length <= rows,
                   "sequence outside the rows");
      ovg::Require(first % ovg::kSequenceAlign == 0,
                   "sequence start must be a multiple of 16");
      end = std::max(end, first + (length + 31) / 32 * 32);
      for (int64_t q = 0; q < length; q += 32)
        work.push_back({static_cast<int>(first + q),
                        static_cast<int>(std::min<int64_t>(32, length - q)),
                        static_cast<int>(first), static_cast<int>(length)});
    }
    int exact_count = 0, exact_rounds = 0;
    ovg::PlanAttentionWork(work, &exact_count, &exact_rounds);
    auto s = static_cast<hipStream_t>(stream);
    // Keys are read in whole 32-row tiles: q and k go head-major into a
    // buffer padded past the last tile, V into V^T blocks.
    const int padded = static_cast<int>(std::max(end, rows));
    const int ldvt = (padded + 15) / 16 * 16;
    const int ldq = ldvt * 128;
    Scratch<ovg::half_t> qk(static_cast<std::size_t>(heads + kv_heads) * ldq);
    Scratch<ovg::half_t> vt(static_cast<std::size_t>(kv_heads) * 128 * ldvt);
    Scratch<ovg::AttentionWork> dwork(work.size());
    ovg::Check(hipMemsetAsync(qk.data, 0,
                              static_cast<std::size_t>(heads + kv_heads) * ldq * 2, s),
               "clear");
    ovg::Check(hipMemsetAsync(vt.data, 0,
                              static_cast<std::size_t>(kv_heads) * 128 * ldvt * 2, s),
               "clear");
    ovg::Check(hipMemcpyAsync(dwork.data, work.data(),
                              work.size() * sizeof(ovg::AttentionWork),
                              hipMemcpyHostToDevice, s),
               "upload");
    ovg::LaunchAttentionLayout(static_cast<const ovg::half_t*>(qkv), ld_qkv, qk.data, ldq,
                               vt.data, ldvt, static_cast<int>(rows),
                               static_cast<int>(heads), static_cast<int>(kv_heads), s);
    ovg::AttentionParams p{};
    p.qk = qk.data;
    p.vt = vt.data;
    p.out = static_cast<ovg::half_t*>(output);
    p.work = dwork.data;
    p.work_count = static_cast<int>(work.size());
    p.exact_count = exact_count;
    p.exact_rounds = exact_rounds;
    p.ld_qk = ldq;
    p.ldvt = ldvt;
    p.heads = static_cast<int>(heads);
    p.kv_heads = static_cast<int>(kv_heads);
    p.scale_log2 = 1.44269504088896341F / 11.313708498984761F;
    ovg::LaunchAttention(p, s);
    ovg::Check(hipStreamSynchronize(s), "attention");
  });
}

}  // extern "C"
