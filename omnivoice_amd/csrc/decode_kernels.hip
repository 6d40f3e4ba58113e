// CFG scoring and unmask-position selection on the GPU, so that a whole
// unmasking step stays on the device.
//
// Score (reference kernels/generator_kernels.hip:212-265): one 64-lane
// wavefront per (item, codebook, frame). Lane l holds logits l, l + 64, ...
// of the conditional and unconditional rows in registers; each statistic is
// a per-lane sequential pass followed by an xor butterfly over offsets
// 32..1. exp and log are this file's own (Cody-Waite + Taylor, atanh
// series) so that the result is bit-identical to the CPU restatement of the
// same sequence of operations.
//
// Select (reference decoding.cpp:70-107): one 1024-thread work-group per
// item. Scores become 48-bit keys (order-preserving float bits, then
// 0xFFFF - index, so that larger keys are higher scores and lower indices on
// ties); a most-significant-digit radix select over six 8-bit digits finds
// the count-th largest key, and every entry at or above it takes its
// prediction. The chosen set is exactly the reference's partial_sort prefix.
//
// No FP contraction in this file: the only fused multiply-adds are the
// explicit fmaf calls, which the CPU restatement performs too.
#pragma clang fp contract(off)

#include "kernels.hpp"

namespace ovg {
namespace {

constexpr float kLog2e = 1.44269504088896341F;
constexpr float kLn2Head = 0.693359375F;
constexpr float kLn2Tail = -2.12194440054690583e-4F;

// Branch-free: the polynomial runs on x clamped to [-87, 88] (which leaves
// every in-range x untouched), then selects give 0 below the range, +inf
// above it and NaN for NaN, the values of the early returns of the CPU
// restatement.
__device__ __forceinline__ float ExpExact(float x) {
  const float xc = fminf(fmaxf(x, -87.0F), 88.0F);
  const float n = __builtin_rintf(xc * kLog2e);
  float r = __builtin_fmaf(n, -kLn2Head, xc);
  r = __builtin_fmaf(n, -kLn2Tail, r);
  float p = 1.0F / 5040.0F;
  p = __builtin_fmaf(p, r, 1.0F / 720.0F);
  p = __builtin_fmaf(p, r, 1.0F / 120.0F);
  p = __builtin_fmaf(p, r, 1.0F / 24.0F);
  p = __builtin_fmaf(p, r, 1.0F / 6.0F);
  p = __builtin_fmaf(p, r, 0.5F);
  p = __builtin_fmaf(p, r, 1.0F);
  p = __builtin_fmaf(p, r, 1.0F);
  const int e = static_cast<int>(n);
  const float scale = __uint_as_float(static_cast<unsigned>(e + 127) << 23);
  float y = p * scale;
  y = x < -87.0F ? 0.0F : y;
  y = x > 88.0F ? __builtin_inff() : y;
  return x != x ? x : y;
}

__device__ __forceinline__ float LogExact(float x) {
  if (x != x)
    return x;
  if (x < 0.0F)
    return __builtin_nanf("");
  if (x == 0.0F)
    return -__builtin_inff();
  if (x == __builtin_inff())
    return x;
  int e = 0;
  unsigned u = __float_as_uint(x);
  if (u < 0x00800000U) {
    x = x * 8388608.0F;
    u = __float_as_uint(x);
    e = -23;
  }
  e += static_cast<int>(u >> 23) - 127;
  float m = __uint_as_float((u & 0x007FFFFFU) | 0x3F800000U);
  if (m > 1.41421356F) {
    m = m * 0.5F;
    e += 1;
  }
  const float f = m - 1.0F;
  const float s = f / (m + 1.0F);
  const float z = s * s;
  float p = __builtin_fmaf(z, 2.0F / 13.0F, 2.0F / 11.0F);
  p = __builtin_fmaf(p, z, 2.0F / 9.0F);
  p = __builtin_fmaf(p, z, 2.0F / 7.0F);
  p = __builtin_fmaf(p, z, 2.0F / 5.0F);
  p = __builtin_fmaf(p, z, 2.0F / 3.0F);
  const float sz = s * z;
  const float lm = __builtin_fmaf(sz, p, s + s);
  const float fe = static_cast<float>(e);
  return __builtin_fmaf(fe, kLn2Head, __builtin_fmaf(fe, kLn2Tail, lm));
}

constexpr int kScorePerLane = 17;  // vocab <= 64 * 17 = 1088
constexpr int kScoreWaves = 4;

__global__ __launch_bounds__(kScoreWaves * kWave) void ScoreKernel(
    ScoreParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * kScoreWaves + (threadIdx.x >> 6);
  const ScoreItem item = p.items[blockIdx.y];
  if (wave >= item.frames * p.codebooks)
    return;
  const int codebook = wave / item.frames;
  const int frame = wave % item.frames;
  const float* cr = p.logits +
                    static_cast<size_t>(item.logit_row + frame) * p.width +
                    codebook * p.vocab;
  const float* ur = cr + static_cast<size_t>(item.frames) * p.width;
  // Entries past the vocabulary hold -inf: they leave every max unchanged
  // and add exp(-inf) = +0 to every per-lane sum, which is exactly the sum
  // without them, so the arithmetic needs no per-entry branches.
  float cv[kScorePerLane], uv[kScorePerLane];
  float cm = -3.402823466e38F, um = -3.402823466e38F;
#pragma unroll
  for (int t = 0; t < kScorePerLane; ++t) {
    const int j = lane + t * kWave;
    cv[t] = j < p.vocab ? cr[j] : -__builtin_inff();
    uv[t] = j < p.vocab ? ur[j] : -__builtin_inff();
    cm = fmaxf(cm, cv[t]);
    um = fmaxf(um, uv[t]);
  }
  cm = WaveMax(cm);
  um = WaveMax(um);
  float cs = 0.0F, us = 0.0F;
#pragma unroll
  for (int t = 0; t < kScorePerLane; ++t) {
    cs = cs + ExpExact(cv[t] - cm);
    us = us + ExpExact(uv[t] - um);
  }
  const float c_lse = cm + LogExact(WaveSum(cs));
  const float u_lse = um + LogExact(WaveSum(us));
  float gv[kScorePerLane];
  float gm = -3.402823466e38F;
#pragma unroll
  for (int t = 0; t < kScorePerLane; ++t) {
    const float c = cv[t] - c_lse;
    const float u = uv[t] - u_lse;
    gv[t] = lane + t * kWave < p.vocab ? __builtin_fmaf(p.guidance, c - u, c)
                                       : -__builtin_inff();
    gm = fmaxf(gm, gv[t]);
  }
  gm = WaveMax(gm);
  float gs = 0.0F;
  float best = -3.402823466e38F;
  int best_index = p.vocab;
#pragma unroll
  for (int t = 0; t < kScorePerLane; ++t) {
    const int j = lane + t * kWave;
    gs = gs + ExpExact(gv[t] - gm);
    // -inf (past the vocabulary) never beats the initial best.
    const bool better = j != static_cast<int>(p.mask_id) && gv[t] > best;
    best = better ? gv[t] : best;
    best_index = better ? j : best_index;
  }
  const float g_lse = gm + LogExact(WaveSum(gs));
  for (int offset = kWave / 2; offset > 0; offset /= 2) {
    const float other = __shfl_xor(best, offset);
    const int other_index = __shfl_xor(best_index, offset);
    if (other > best || (other == best && other_index < best_index)) {
      best = other;
      best_index = other_index;
    }
  }
  if (lane == 0) {
    const int out = item.out_base + codebook * item.frames + frame;
    p.prediction[out] = best_index;
    p.confidence[out] = best - g_lse;
  }
}

// Order-preserving map of float bits: a > b  <=>  Key(a) > Key(b) for
// non-NaN floats (-0 is folded into +0 first).
__device__ __forceinline__ unsigned OrderedBits(float s) {
  if (s == 0.0F)
    s = 0.0F;
  const unsigned u = __float_as_uint(s);
  return (u & 0x80000000U) ? ~u : (u | 0x80000000U);
}

// SLOTS: keys per thread the launch allows (4 covers items of up to 4096
// positions in registers; 16 the API's maximum of 16384).
template <int SLOTS>
__global__ __launch_bounds__(kSelectThreads) void SelectKernel(
    SelectParams p) {
  __shared__ unsigned histogram[256];
  __shared__ int chosen_digit;
  __shared__ int remaining;
  const SelectItem item = p.items[blockIdx.x];
  const int total = p.codebooks * item.frames;
  const int tid = threadIdx.x;
  // Key slots in use (the same for every thread): each loop below is
  // unrolled, so the keys stay in registers, and leaves after `slots`
  // iterations, so a 2000-key item costs 2 slots' work, not 16.
  const int slots = (total + kSelectThreads - 1) / kSelectThreads;
  // Every load that does not depend on the step (confidence, codes and
  // predictions, unconditionally at clamped indices) is issued together
  // with the step's plan entry, then the noise: three memory round trips in
  // all instead of one per load.
  float conf[SLOTS], noise[SLOTS];
  int code[SLOTS], pred[SLOTS];
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    if (r >= slots)
      break;
    const int i = min(tid + r * kSelectThreads, total - 1);
    conf[r] = p.confidence[item.out_base + i];
    code[r] = p.codes[item.out_base + i];
    pred[r] = p.prediction[item.out_base + i];
  }
  SelectStep s = p.single;
  if (p.epoch != nullptr)
    s = p.plan[(*p.epoch - 1) * p.item_count + blockIdx.x];
  if (s.count <= 0)
    return;
  if (p.temperature > 0.0F) {
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      if (r >= slots)
        break;
      noise[r] = p.noise[s.noise_offset + min(tid + r * kSelectThreads, total - 1)];
    }
  }
  uint64_t key[SLOTS];
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    if (r >= slots)
      break;
    const int i = tid + r * kSelectThreads;
    key[r] = 0;
    if (i < total) {
      const int c = i / item.frames;
      const float penalty = static_cast<float>(c) * p.layer_penalty;
      float score = conf[r] - penalty;
      if (p.temperature > 0.0F)
        score = score / p.temperature + noise[r];
      if (code[r] != static_cast<int>(p.mask_id))
        score = -__builtin_inff();
      key[r] = (static_cast<uint64_t>(OrderedBits(score)) << 16) |
               static_cast<uint64_t>(0xFFFF - i);
    }
  }
  // The count-th largest key, one 8-bit digit at a time from bit 47.
  const int count = s.count < total ? s.count : total;
  uint64_t prefix = 0;
  if (tid == 0)
    remaining = count;
  for (int shift = 40; shift >= 0; shift -= 8) {
    if (tid < 256)
      histogram[tid] = 0;
    __syncthreads();
    const uint64_t high = prefix >> (shift + 8);
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      if (r >= slots)
        break;
      const int i = tid + r * kSelectThreads;
      if (i < total && (key[r] >> (shift + 8)) == high)
        atomicAdd(&histogram[(key[r] >> shift) & 0xFF], 1U);
    }
    __syncthreads();
    if (tid < kWave) {
      // Suffix sums of the 256 bins: lane l owns bins 4l .. 4l + 3.
      const unsigned h0 = histogram[4 * tid], h1 = histogram[4 * tid + 1];
      const unsigned h2 = histogram[4 * tid + 2], h3 = histogram[4 * tid + 3];
      const unsigned s3 = h3, s2 = h2 + s3, s1 = h1 + s2, s0 = h0 + s1;
      unsigned above = s0;  // becomes the inclusive suffix over lanes >= tid
      for (int offset = 1; offset < kWave; offset *= 2) {
        const unsigned other = __shfl_down(above, offset);
        if (tid + offset < kWave)
          above += other;
      }
      above -= s0;  // bins of lanes > tid
      const unsigned want = static_cast<unsigned>(remaining);
      const unsigned suffix[5] = {s0 + above, s1 + above, s2 + above,
                                  s3 + above, above};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (suffix[b] >= want && suffix[b + 1] < want) {
          chosen_digit = 4 * tid + b;
          remaining = static_cast<int>(want - suffix[b + 1]);
        }
      }
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(chosen_digit) << shift;
    __syncthreads();
  }
  // prefix is now the count-th largest key: everything >= it is chosen.
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    if (r >= slots)
      break;
    const int i = tid + r * kSelectThreads;
    if (i < total && key[r] >= prefix) {
      const int value = pred[r];
      p.codes[item.out_base + i] = value;
      p.unmasked_at[item.out_base + i] = s.step;
      if (p.ids != nullptr) {
        const int c = i / item.frames;
        const int f = i % item.frames;
        int* row = p.ids + static_cast<size_t>(c) * p.ld_ids;
        row[item.cond_row + f] = value;
        row[item.uncond_row + f] = value;
      }
    }
  }
}

}  // namespace

void LaunchScore(const ScoreParams& p, hipStream_t stream) {
  Require(p.vocab >= 1 && p.vocab <= kScorePerLane * kWave,
          "score: vocab outside [1, 1088]");
  Require(p.item_count >= 1 && p.max_frames >= 1, "score: no frames");
  const int waves = p.max_frames * p.codebooks;
  const dim3 grid((waves + kScoreWaves - 1) / kScoreWaves, p.item_count);
  Dispatch(ScoreKernel, grid, dim3(kScoreWaves * kWave), 0, stream, true, true,
           p);
  Check(hipGetLastError(), "score launch");
}

void LaunchSelect(const SelectParams& p, int max_total, hipStream_t stream) {
  Require(max_total >= 1 && max_total <= kSelectThreads * kSelectPerThread,
          "select: codebooks * frames outside [1, 16384]");
  Require(p.item_count >= 1, "select: no items");
  if (max_total <= 4 * kSelectThreads)
    Dispatch(SelectKernel<4>, dim3(p.item_count), dim3(kSelectThreads), 0,
             stream, true, true, p);
  else
    Dispatch(SelectKernel<kSelectPerThread>, dim3(p.item_count),
             dim3(kSelectThreads), 0, stream, true, true, p);
  Check(hipGetLastError(), "select launch");
}

}  // namespace ovg
