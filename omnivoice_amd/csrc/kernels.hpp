// Launchers of the gfx950 generator kernels. Every launcher validates the
// shapes its kernel assumes and throws ovg::Error instead of launching on a
// shape the kernel cannot cover.
#ifndef OMNIVOICE_AMD_KERNELS_HPP_
#define OMNIVOICE_AMD_KERNELS_HPP_

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.hpp"

namespace ovg {

class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

inline void Check(hipError_t status, const char* what) {
  if (status != hipSuccess)
    throw Error(std::string(what) + ": " + hipGetErrorString(status));
}

inline void Require(bool condition, const std::string& what) {
  if (!condition)
    throw Error(what);
}

// Kernel-accurate timing for the profiler: while set on the launching
// thread, a launcher dispatches its first kernel with `start` and its last
// with `stop` (hipExtLaunchKernel), so the events bracket the kernels
// themselves rather than the gaps between dispatches. Null otherwise.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
inline LaunchTiming& CurrentTiming() {
  static thread_local LaunchTiming timing;
  return timing;
}

template <typename... Params, typename... Args>
void Dispatch(void (*kernel)(Params...), dim3 grid, dim3 block,
              std::uint32_t lds_bytes, hipStream_t stream, bool first,
              bool last, Args... args) {
  const LaunchTiming& t = CurrentTiming();
  hipEvent_t start = first ? t.start : nullptr;
  hipEvent_t stop = last ? t.stop : nullptr;
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, start, stop,
                          0, static_cast<Params>(args)...);
  else
    kernel<<<grid, block, lds_bytes, stream>>>(static_cast<Params>(args)...);
}

// ---------------------------------------------------------------- GEMM
// Y = X W^T: X fp16 [M][K] (row stride lda), W fp16 [N][K] (ldb), fp32
// accumulation; the epilogue decides what is written.
enum class Epilogue : int {
  kStore = 0,       // y fp32 [M][ldc] = acc
  kAccumulate = 1,  // y fp32 [M][ldc] += acc (the residual stream)
  kQkvRope = 2,     // per-head RMSNorm + rotary for q/k heads -> fp16
                    // qk at QkIndex(head, row, d, ldq); v heads ->
                    // fp16 V^T at VtIndex (ldvt % 16 == 0)
  kSwiGlu = 3,      // act fp16 [M][ldh] = silu(gate) * up; the W rows pair
                    // gate and up rows: per 128-row tile 64 gate rows then
                    // the matching 64 up rows (GemmKernel), or per packed
                    // 32-row block 16 and 16 (PackMap::kSwiGlu)
  kPartial = 4,     // split s stores its fp32 tile to y + s * split_stride
                    // ([M][ldc] per split); a row kernel sums the splits
};

struct GemmParams {
  const half_t* x;
  const half_t* w;
  int lda, ldb;
  int m, n, k;
  int splits;        // K split into `splits` equal ranges (1 = none)
  float* partials;   // [tiles * splits][tile floats] when splits > 1
  std::size_t split_stride;  // kPartial: floats between split slices of y
  // kStore / kAccumulate
  float* y;
  int ldc;
  // kQkvRope
  half_t* qk;
  int ldq;
  half_t* vt;
  int ldvt;
  const float* q_norm;
  const float* k_norm;
  const float2* rope;      // [M][head_dim / 2]: (cos, sin) of each row's
                           // position (LaunchRopeRows)
  int heads, kv_heads;
  float eps;
  // kSwiGlu
  half_t* act;
  int ldh;
};

// Picks the tile shape and split count for (m, n, k) and the number of
// floats of `partials` the launch needs.
struct GemmPlan {
  int stages = 3;  // LDS ring depth
  int fm = 1;      // strip height in 32-row blocks
  int strips = 4;  // strips per K group: tiles of 32 fm strips rows
  int splits = 1;
  int tiles = 0;
  // Row tiles per band of the tile order: each XCD takes a run of tiles
  // that covers `band` row tiles across columns, so its rows of X stay in
  // its L2 (0 or all row tiles: plain M-fastest order; always so with
  // split-K).
  int band = 0;
  std::size_t partial_floats = 0;
};
// The tile shape and split count of one GEMM. The split count of the
// partial-slice epilogue depends on K only, and no other epilogue is split
// unless `split_small` asks for it (stand-alone calls), so the generator's
// per-row results do not depend on the packed row count M.
GemmPlan PlanGemm(int m, int n, int k, Epilogue epilogue, bool split_small = false);
void LaunchGemm(const GemmParams& p, const GemmPlan& plan, Epilogue epilogue,
                hipStream_t stream);
// Split count of the partial-slice epilogue: a function of K steps alone.
int PartialSplits(int k_steps);

// ---------------------------------------------------------------- packed GEMM
// The generator's projections with W packed at load into matrix-core
// fragment order (packed_gemm.hip). GemmParams::w is then the packed matrix
// and ldb is unused.
enum class PackMap : int {
  kIdentity = 0,  // block column i = output column i
  kRope = 1,      // q/k/v: 128-column heads in kv-group order (each kv
                  // head's `group` query heads, then its k and v heads);
                  // block w of a head holds head columns 16 w .. +15 and
                  // 64 + 16 w .. +15 (rotate-half pairs in one lane)
  kSwiGlu = 2,    // block b holds gate rows 16 b .. +15 then up rows 16 b .. +15
};
// Halves a packed copy of a [rows][k] matrix takes (rows padded to 256).
std::size_t PackedWeightHalves(int rows, int k);
// Packs row-major fp16 w [rows][k] (for kSwiGlu: gate w and up w2, [rows][k]
// each, packed as 2 rows outputs; for kRope: [q; k; v] heads, `group` query
// heads per kv head) on the device.
void PackWeights(const half_t* w, const half_t* w2, int rows, int k, PackMap map, int group,
                 half_t* out, hipStream_t stream);
// The same from a float32 source, rounded to fp16 on the device.
void PackWeights(const float* w, const float* w2, int rows, int k, PackMap map, int group,
                 half_t* out, hipStream_t stream);
struct PackedPlan {
  int xb = 4;      // tile height in 32-row blocks (1-4, or 8 with wb 2)
  int wb = 1;      // tile width in 128-column units (2: 128 x 256 or 256 x 256)
  int splits = 1;  // K split (partial-slice epilogue only)
  int tiles = 0;   // row tiles x column tiles
  int nw = 4;      // waves (32-column blocks) of a 32 XB-row tile: 4, 2 or 1
  // Column split (256 x 256 tiles only): the tile above covers columns
  // [0, n_main) in whole rounds of work-groups, and a second launch covers
  // [n_main, N) with the tail tile; 0 = one launch for every column.
  int n_main = 0;
  int tail_xb = 0, tail_wb = 0, tail_nw = 0, tail_tiles = 0;
};
PackedPlan PlanPacked(int m, int n, int k, Epilogue epilogue);
void LaunchPacked(const GemmParams& p, const PackedPlan& plan, Epilogue epilogue,
                  hipStream_t stream);

// ---------------------------------------------------------------- rows
struct EmbedParams {
  const int* ids;          // [codebooks][ld_ids]
  int ld_ids;
  const int* row_kind;     // [rows]: 0 text, 1 audio, 2 padding
  const float* text;       // [vocab][hidden]
  const float* audio;      // [codebooks * vocab][hidden]
  const float* norm;       // first layer's input norm [hidden]
  float* hidden;           // [rows][hidden]
  half_t* normed;          // [rows][hidden]
  int rows, hidden_size, codebooks, vocab;
  float eps;
  int* epoch;              // incremented once per launch (may be null)
};
void LaunchEmbed(const EmbedParams& p, hipStream_t stream);

// normed[r] = half(w * x[r] * rsqrt(mean(x[r]^2) + eps)), r < rows; with
// `gather` non-null the source row is gather[r].
void LaunchRmsNorm(const float* x, const int* gather, const float* w,
                   half_t* out, int rows, int width, float eps,
                   hipStream_t stream);

// Weight prefetch: `groups` extra work-groups after the attention's own
// read these byte ranges (the weights of the GEMMs that follow), so that
// those GEMMs find them in the memory-side cache instead of HBM. Nothing is
// stored.
struct WeightPrefetch {
  static constexpr int kMaxRanges = 5;
  const unsigned char* range[kMaxRanges];
  unsigned long long bytes[kMaxRanges];
  int groups;
};

// The prefetch work-group `group` (0 .. w.groups - 1): each thread issues
// its 16-byte loads in batches of eight (clamped in bounds, no load under a
// condition) and folds each batch into a value that only an empty asm
// statement consumes, so only the cache fill remains. The next batch is
// issued before the previous one is folded, so that eight to sixteen loads
// stay in flight instead of the pipeline draining after every batch (2 s:
// the attention launch carrying the 31.5 MB 8.06 -> 7.4-7.7 us, +0.5-0.8 %
// unmask steps/s; batches of four or twelve no better).
__device__ __forceinline__ void PrefetchWeights(const WeightPrefetch& w, int group) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kInFlight = 8;
  const unsigned long long stride = static_cast<unsigned long long>(w.groups) * blockDim.x;
  unsigned int fold = 0;
  for (int r = 0; r < WeightPrefetch::kMaxRanges; ++r) {
    const unsigned long long chunks = w.bytes[r] / 16;
    if (chunks == 0)
      continue;
    const u32x4* src = reinterpret_cast<const u32x4*>(w.range[r]);
    unsigned long long c = static_cast<unsigned long long>(group) * blockDim.x + threadIdx.x;
    if (c >= chunks)
      continue;
    u32x4 v[kInFlight];
#pragma unroll
    for (int k = 0; k < kInFlight; ++k)
      v[k] = src[min(c + k * stride, chunks - 1)];
    for (c += kInFlight * stride; c < chunks; c += kInFlight * stride) {
      u32x4 next[kInFlight];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        next[k] = src[min(c + k * stride, chunks - 1)];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        fold ^= v[k].x;
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        v[k] = next[k];
    }
#pragma unroll
    for (int k = 0; k < kInFlight; ++k)
      fold ^= v[k].x;
  }
  asm volatile("" : : "v"(fold));
}

// The residual update and the next RMSNorm in one pass over rows:
//   h = hidden[src] + partial[0][src] + partial[1][src] + ... (that order)
//   out[r] = half(norm * h * rsqrt(mean(h^2) + eps))
// With `gather` null, src = r and h is written back to hidden[r]; with
// `gather` set, src = gather[r] and hidden is left untouched (the final
// norm of the target rows).
struct AddNormParams {
  float* hidden;             // [rows][width]
  const float* partials;     // splits slices of [rows][width]
  std::size_t split_stride;  // floats between slices
  int splits;
  const float* norm;         // [width]
  half_t* out;               // [rows][width]
  const int* gather;
  int rows, width;
  float eps;
};
void LaunchAddNorm(const AddNormParams& p, hipStream_t stream);

// The attention's operand layouts from row-major q|k|v rows (r < rows):
// qk[QkIndex(h, r, d, ldq)] = qkv[r][h * 128 + d] for the q and k heads,
// vt[VtIndex(g, d, r, ldvt)] = qkv[r][(heads + kv_heads + g) * 128 + d].
void LaunchAttentionLayout(const half_t* qkv, int ld_qkv, half_t* qk, int ldq,
                           half_t* vt, int ldvt, int rows, int heads, int kv_heads,
                           hipStream_t stream);

void LaunchFill(int* data, int value, int count, hipStream_t stream);

// rows_table[r][i] = table[positions[r]][i], i < 64, r < rows: the rotary
// (cos, sin) pairs of every packed row, gathered once per batch layout.
void LaunchRopeRows(const float2* table, const int* positions, int rows,
                    float2* rows_table, hipStream_t stream);

// ---------------------------------------------------------------- attention
struct AttentionWork {
  int q_begin, q_count, seq_begin, seq_length;
};
struct AttentionParams {
  const half_t* qk;        // q heads then k heads at QkIndex(head, row, d, ld_qk)
  const half_t* vt;        // V^T at VtIndex(g, d, row, ldvt)
  half_t* out;             // [rows][heads * 128]
  const AttentionWork* work;
  int work_count;
  int ld_qk, ldvt, heads, kv_heads;
  float scale_log2;        // log2(e) / sqrt(128)
  WeightPrefetch prefetch;
  // work[0, exact_count): sequences of at most kExactAttentionKeys keys,
  // whose scores fit in registers (two-pass softmax, at most exact_rounds
  // rounds of four 32-key tiles); the rest take the online-softmax kernel.
  int exact_count;
  int exact_rounds;
};
constexpr int kExactAttentionKeys = 768;
// Orders `work` so that the items of sequences of at most
// kExactAttentionKeys keys come first (each group in its given order) and
// sets AttentionParams::exact_count / exact_rounds for it. Which kernel a
// query takes depends on its own sequence's length only.
void PlanAttentionWork(std::vector<AttentionWork>& work, int* exact_count, int* exact_rounds);
void LaunchAttention(const AttentionParams& p, hipStream_t stream);

// ---------------------------------------------------------------- decoding
// Per item: logits rows [logit_row, logit_row + frames) conditional,
// [logit_row + frames, logit_row + 2 frames) unconditional; outputs
// [codebook][frame] at out_base.
struct ScoreItem {
  int logit_row, frames, out_base, pad;
};
struct ScoreParams {
  const float* logits;
  const ScoreItem* items;
  int item_count, max_frames;
  int codebooks, vocab, width;
  unsigned mask_id;
  float guidance;
  int* prediction;
  float* confidence;
};
void LaunchScore(const ScoreParams& p, hipStream_t stream);

// One work-group per item. The step's (step, count, noise offset) come from
// `plan[(epoch - 1) * items + item]` when `epoch` is non-null, else from
// the by-value fields.
struct SelectItem {
  int frames, out_base;      // pred/conf/codes/unmasked_at offset
  int cond_row, uncond_row;  // first packed row of the target frames
};
struct SelectStep {
  int step, count, noise_offset, pad;
};
struct SelectParams {
  const int* prediction;
  const float* confidence;
  const float* noise;
  int* codes;
  int* unmasked_at;
  int* ids;                  // packed [codebooks][ld_ids] or null
  int ld_ids;
  const SelectItem* items;
  int item_count;
  int codebooks;
  float layer_penalty, temperature;
  unsigned mask_id;
  const SelectStep* plan;
  const int* epoch;
  SelectStep single;
};
constexpr int kSelectThreads = 1024;
constexpr int kSelectPerThread = 16;
void LaunchSelect(const SelectParams& p, int max_total, hipStream_t stream);

}  // namespace ovg

#endif  // OMNIVOICE_AMD_KERNELS_HPP_
