// The audio decoder's kernels on gfx950 (replacing the reference's
// hipblasSgemm calls and element-wise kernels of the DAC decoder:
// codec_state.hpp:232-300, kernels/codec_kernels.hip:11-84).
//
// Every convolution is one implicit GEMM on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32): output channels x output positions, summed over
// input channels x taps. A work-group of four waves owns a BM x BN tile
// (32 x 128 or 64 x 64), one 32 x 32 accumulator block per wave. The K loop
// runs over chunks of 16 input channels: the chunk's input window (the tile's
// positions plus the taps' spread) is staged once in LDS with the Snake
// activation applied on the way and zeros outside the signal, the chunk's
// weights [tap][channel][output] beside it, and every tap then reads its
// shifted window from LDS. Bias and the residual addition are applied in
// the epilogue, straight from the accumulators. Nothing is rounded below
// float32, so the results match the reference's float32 GEMMs to rounding.
#include "codec.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kThreads = 256;
constexpr int kOutTile = 256;  // samples per work-group of the output conv
constexpr int kOutChunk = 32;  // input channels per chunk of the output conv

// kernels/codec_kernels.hip:20-22 of the reference: x + sin^2(a x) / (a + 1e-9).
__device__ __forceinline__ float Snake(float v, float a) {
  const float s = sinf(a * v);
  return v + (1.0F / (a + 1e-9F)) * (s * s);
}
__device__ __forceinline__ float Gelu(float v) {
  return 0.5F * v * (1.0F + erff(v * 0.70710678118654752F));
}
__device__ __forceinline__ float Elu(float v) { return v > 0.0F ? v : expm1f(v); }

// Channels staged per K chunk, by tap count: every chunk feeds
// TAPS x CHUNK / 2 MFMAs per wave between two barriers.
template <int TAPS>
constexpr int ChunkFor() {
  return TAPS == 1 ? 64 : TAPS == 2 ? 32 : 16;
}
// Largest spread of the taps' offsets the input window allows.
template <int TAPS>
constexpr int SpanFor() {
  return TAPS == 1 ? 0 : TAPS == 2 ? 1 : kConvMaxSpan;
}
constexpr int Pow2AtLeast(int n) {
  int p = 1;
  while (p < n)
    p *= 2;
  return p;
}

// The epilogue of one output: bias, pre-activation, residual accumulation,
// the stores.
__device__ __forceinline__ void Finish(const ConvParams& p, const float* bias, float* y,
                                       float* y_act, int co, size_t at, float v) {
  if (bias != nullptr)
    v += bias[co];
  if (p.pre_act == kActGelu)
    v = Gelu(v);
  if (p.accumulate)
    v += y[at];
  if (y != nullptr)
    y[at] = v;
  if (y_act != nullptr)
    y_act[at] = p.out_act == kActElu ? Elu(v) : Snake(v, p.alpha_out[co]);
}

template <int BM, int BN, int WAVES, int TAPS>
__global__ __launch_bounds__(64 * WAVES) void ConvKernel(ConvParams p) {
  static_assert(BM * BN == WAVES * 32 * 32, "one 32 x 32 block per wave");
  constexpr int kT = 64 * WAVES;
  constexpr int kC = ChunkFor<TAPS>();
  constexpr int kWavesN = BN / 32;
  constexpr int kWidth = BN + SpanFor<TAPS>();
  // Staging map: thread -> column j = tid % kCols (+ kCols per extra column
  // slot) and channels g, g + kGroups, ... with g = tid / kCols.
  constexpr int kCols = Pow2AtLeast(kWidth) < kT ? Pow2AtLeast(kWidth) : kT;
  constexpr int kColSlots = (kWidth + kCols - 1) / kCols;
  constexpr int kGroups = kT / kCols;
  constexpr int kPerGroup = kC / kGroups;  // channels per thread and column
  static_assert(kC % kGroups == 0, "staging map");
  constexpr int kWSlots = TAPS * kC * BM / kT;  // weights per thread
  static_assert(TAPS * kC * BM % kT == 0, "weight slots");
  constexpr int kSubs = kC / 16;        // 16-channel groups per tap
  constexpr int kSteps = TAPS * kSubs;  // groups of 8 MFMAs per chunk
  __shared__ float xs[kC][kWidth];
  __shared__ float ws[TAPS][kC][BM];

  const int split = blockIdx.z % p.splits;
  const int rest = blockIdx.z / p.splits;  // batch x phases + phase
  const int phase = rest % p.phases;
  const int batch = rest / p.phases;
  const int c_begin = split * p.split_chunks * kC;
  const int c_end = min(p.cin, c_begin + p.split_chunks * kC);
  const float* x = p.x + batch * p.x_batch;
  const float* bias = p.bias != nullptr ? p.bias + batch * p.b_batch : nullptr;
  float* y = p.y != nullptr ? p.y + batch * p.y_batch : nullptr;
  float* y_act = p.y_act != nullptr ? p.y_act + batch * p.y_batch : nullptr;
  const int m0 = blockIdx.x * BN;
  const int co0 = blockIdx.y * BM;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = (wave / kWavesN) * 32;  // first output channel of the wave
  const int col = (wave % kWavesN) * 32;  // first position of the wave
  const int half = lane >> 5;             // K index of the lane's operands
  const int l32 = lane & 31;
  int shift[TAPS];
  int lo = p.offsets[phase][0];
#pragma unroll
  for (int k = 0; k < TAPS; ++k) {
    shift[k] = p.offsets[phase][k];
    lo = min(lo, shift[k]);
  }
#pragma unroll
  for (int k = 0; k < TAPS; ++k)
    shift[k] -= lo;  // window column of position 0 for tap k (<= kWidth - BN)
  const float* w = p.w + batch * p.w_batch + static_cast<size_t>(phase) * TAPS * p.cin * p.ldw;
  const int jcol = tid % kCols;
  const int group = tid / kCols;

  // A chunk's operands pass through registers: fetch() issues the global
  // loads of chunk c0 (unconditional, clamped addresses), stash() writes
  // them to LDS with the input activation and the zero padding applied.
  // The next chunk is fetched before the current chunk's MFMAs, so its
  // loads are in flight while they run.
  float xr[kColSlots][kPerGroup];
  float wr[kWSlots];
  auto fetch = [&](int c0) {
#pragma unroll
    for (int q = 0; q < kColSlots; ++q) {
      const int t = min(max(m0 + lo + jcol + q * kCols, 0), p.len_in - 1);
#pragma unroll
      for (int i = 0; i < kPerGroup; ++i) {
        const int c = min(c0 + group + i * kGroups, p.cin - 1);
        xr[q][i] = x[static_cast<size_t>(c) * p.len_in + t];
      }
    }
#pragma unroll
    for (int q = 0; q < kWSlots; ++q) {
      const int e = tid + q * kT;
      const int o = e % BM;
      const int c = (e / BM) % kC;
      const int k = e / (BM * kC);
      wr[q] = w[(static_cast<size_t>(k) * p.cin + min(c0 + c, p.cin - 1)) * p.ldw +
                min(co0 + o, p.cout - 1)];
    }
  };
  auto stash = [&](int c0) {
#pragma unroll
    for (int q = 0; q < kColSlots; ++q) {
      const int j = jcol + q * kCols;
      if (j < kWidth) {
        const int t = m0 + lo + j;
        const bool inside = t >= 0 && t < p.len_in;
#pragma unroll
        for (int i = 0; i < kPerGroup; ++i) {
          const int c = group + i * kGroups;
          float v = xr[q][i];
          if (p.alpha_in != nullptr)
            v = Snake(v, p.alpha_in[min(c0 + c, p.cin - 1)]);
          xs[c][j] = inside && c0 + c < p.cin ? v : 0.0F;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kWSlots; ++q) {
      const int e = tid + q * kT;
      const int o = e % BM;
      const int c = (e / BM) % kC;
      const int k = e / (BM * kC);
      ws[k][c][o] = c0 + c < p.cin && co0 + o < p.cout ? wr[q] : 0.0F;
    }
  };

  // Operands of one group of 8 MFMAs (16 channels of one tap). Groups are
  // double-buffered in registers: group g + 1's LDS reads are issued before
  // group g's MFMAs. Two accumulator chains (alternate channel pairs).
  struct Operands {
    float a[8], b[8];
  };
  auto read = [&](int g) {
    const int k = g / kSubs;
    const int c = (g % kSubs) * 16;
    Operands op;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      op.a[s] = ws[k][c + 2 * s + half][row + l32];
      op.b[s] = xs[c + 2 * s + half][col + l32 + shift[k]];
    }
    return op;
  };
  floatx16 acc[2] = {};
  fetch(c_begin);
  for (int c0 = c_begin; c0 < c_end; c0 += kC) {
    stash(c0);
    __syncthreads();
    if (c0 + kC < c_end)
      fetch(c0 + kC);
    Operands cur = read(0);
#pragma unroll
    for (int g = 0; g < kSteps; ++g) {
      Operands next;
      if (g + 1 < kSteps)
        next = read(g + 1);
      // Keeps the scheduler from sinking the next group's reads down to
      // their uses, where every MFMA would wait for its own operands.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 8; ++s)
        acc[s & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[s], cur.b[s], acc[s & 1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (g + 1 < kSteps)
        cur = next;
    }
    __syncthreads();
  }

  // Element r of the accumulators: output channel row + 8 (r / 4) +
  // 4 half + r % 4, position col + l32.
  const int m = m0 + col + l32;
  if (m >= p.positions)
    return;
  if (p.splits > 1) {
    // partial[rest][split][co][m]
    float* part = p.partial + (static_cast<size_t>(rest) * p.splits + split) * p.cout * p.positions;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int co = co0 + row + 8 * (r >> 2) + 4 * half + (r & 3);
      if (co < p.cout)
        part[static_cast<size_t>(co) * p.positions + m] = acc[0][r] + acc[1][r];
    }
    return;
  }
  const size_t t = static_cast<size_t>(m) * p.out_stride + phase;
  // Every load of the epilogue (bias, the residual, the Snake alphas) is
  // issued before its first store: the stores may alias them as far as the
  // compiler knows, so loads left between them would each wait out a
  // memory round trip.
  float b[16], prior[16], a[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int co = min(co0 + row + 8 * (r >> 2) + 4 * half + (r & 3), p.cout - 1);
    b[r] = bias != nullptr ? bias[co] : 0.0F;
    prior[r] = p.accumulate ? y[static_cast<size_t>(co) * p.len_out + t] : 0.0F;
    a[r] = y_act != nullptr && p.out_act == kActSnake ? p.alpha_out[co] : 0.0F;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int co = co0 + row + 8 * (r >> 2) + 4 * half + (r & 3);
    if (co < p.cout) {
      const size_t at = static_cast<size_t>(co) * p.len_out + t;
      float v = (acc[0][r] + acc[1][r]) + b[r];
      if (p.pre_act == kActGelu)
        v = Gelu(v);
      v += prior[r];
      if (y != nullptr)
        y[at] = v;
      if (y_act != nullptr)
        y_act[at] = p.out_act == kActElu ? Elu(v) : Snake(v, a[r]);
    }
  }
}

// Sums the split-K partials of every output in split order, then the
// convolution's epilogue.
__global__ __launch_bounds__(kThreads) void SplitReduceKernel(ConvParams p) {
  const size_t per = static_cast<size_t>(p.cout) * p.positions;
  const size_t total = per * p.batches * p.phases;
  for (size_t e = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; e < total;
       e += static_cast<size_t>(gridDim.x) * kThreads) {
    const int rest = static_cast<int>(e / per);
    const size_t within = e % per;
    const int co = static_cast<int>(within / p.positions);
    const int m = static_cast<int>(within % p.positions);
    const float* part = p.partial + static_cast<size_t>(rest) * p.splits * per + within;
    float v = 0.0F;
    for (int s = 0; s < p.splits; ++s)
      v += part[static_cast<size_t>(s) * per];
    const int phase = rest % p.phases, batch = rest / p.phases;
    const float* bias = p.bias != nullptr ? p.bias + batch * p.b_batch : nullptr;
    float* y = p.y != nullptr ? p.y + batch * p.y_batch : nullptr;
    float* y_act = p.y_act != nullptr ? p.y_act + batch * p.y_batch : nullptr;
    const size_t t = static_cast<size_t>(m) * p.out_stride + phase;
    Finish(p, bias, y, y_act, co, static_cast<size_t>(co) * p.len_out + t, v);
  }
}

__global__ __launch_bounds__(kThreads) void OutputConvKernel(OutputConvParams p) {
  __shared__ float xs[kOutChunk][kOutTile + kConvMaxTaps - 1];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kOutTile;
  const int pad = (p.taps - 1) / 2;
  const int width = kOutTile + p.taps - 1;
  float acc = 0.0F;
  for (int c0 = 0; c0 < p.cin; c0 += kOutChunk) {
    for (int j = tid; j < width; j += kThreads) {
      const int t = t0 - pad + j;
      const bool inside = t >= 0 && t < p.length;
      const int tc = min(max(t, 0), p.length - 1);
      float v[kOutChunk];
#pragma unroll
      for (int c = 0; c < kOutChunk; ++c)
        v[c] = p.x[static_cast<size_t>(min(c0 + c, p.cin - 1)) * p.length + tc];
#pragma unroll
      for (int c = 0; c < kOutChunk; ++c)
        xs[c][j] = inside && c0 + c < p.cin
                       ? (p.alpha != nullptr ? Snake(v[c], p.alpha[min(c0 + c, p.cin - 1)]) : v[c])
                       : 0.0F;
    }
    __syncthreads();
    const int channels = min(kOutChunk, p.cin - c0);
    for (int c = 0; c < channels; ++c)
      for (int k = 0; k < p.taps; ++k)
        acc += p.w[k * p.cin + c0 + c] * xs[c][tid + k];
    __syncthreads();
  }
  const int t = t0 + tid;
  if (t < p.length)
    p.y[t] = acc + p.bias[0];
}

__global__ __launch_bounds__(kThreads) void RvqKernel(RvqParams p) {
  const int f = blockIdx.x;
  for (int o = threadIdx.x; o < p.latent; o += kThreads) {
    float v = 0.0F;
    for (int c = 0; c < p.codebooks; ++c) {
      // Codes were range-checked by the host; the clamp keeps a bad device
      // input inside the table.
      const int code = min(max(p.codes[static_cast<size_t>(c) * p.frames + f], 0),
                           p.entries - 1);
      v += p.table[(static_cast<size_t>(c) * p.entries + code) * p.latent + o];
    }
    p.y[static_cast<size_t>(o) * p.frames + f] = v + p.bias[o];
  }
}

template <int BM, int BN, int WAVES, int TAPS>
void DispatchConv(const ConvParams& p, hipStream_t stream, bool last = true) {
  const dim3 grid((p.positions + BN - 1) / BN, (p.cout + BM - 1) / BM,
                  p.phases * p.batches * p.splits);
  Dispatch(ConvKernel<BM, BN, WAVES, TAPS>, grid, dim3(64 * WAVES), 0, stream, true, last, p);
}

// Four-wave tiles when they give at least one work-group per CU, else
// one-wave 32 x 32 tiles (four times the work-groups).
//
// With a split-K workspace, a convolution whose four-wave tiles number
// under 256 instead splits its input channels (at least two chunks per
// split) until about 512 work-groups run, and a reduction kernel finishes
// it.
template <int TAPS>
void DispatchTaps(const ConvParams& params, hipStream_t stream) {
  ConvParams p = params;
  const auto groups = [&](int bm, int bn) {
    return static_cast<int64_t>((p.positions + bn - 1) / bn) * ((p.cout + bm - 1) / bm) *
           p.phases * p.batches;
  };
  constexpr int kC = ChunkFor<TAPS>();
  const int chunks = (p.cin + kC - 1) / kC;
  p.splits = 1;
  p.split_chunks = chunks;
  const bool small_m = p.cout <= 32;
  const int64_t tiles = small_m ? groups(32, 128) : groups(64, 64);
  if (p.partial != nullptr && tiles < 256 && chunks >= 4) {
    int64_t want = std::min<int64_t>((512 + tiles - 1) / tiles, chunks / 2);
    const int64_t outputs = static_cast<int64_t>(p.cout) * p.positions * p.phases * p.batches;
    want = std::min<int64_t>(want, p.partial_capacity / std::max<int64_t>(outputs, 1));
    want = std::min<int64_t>(want, 65535 / (static_cast<int64_t>(p.phases) * p.batches));
    if (want >= 2) {
      p.split_chunks = static_cast<int>((chunks + want - 1) / want);
      p.splits = (chunks + p.split_chunks - 1) / p.split_chunks;
    }
  }
  if (p.splits > 1) {
    if (small_m)
      DispatchConv<32, 128, 4, TAPS>(p, stream, false);
    else
      DispatchConv<64, 64, 4, TAPS>(p, stream, false);
    const size_t total = static_cast<size_t>(p.cout) * p.positions * p.phases * p.batches;
    const int blocks = static_cast<int>(std::min<size_t>((total + kThreads - 1) / kThreads, 16384));
    Dispatch(SplitReduceKernel, dim3(blocks), dim3(kThreads), 0, stream, false, true, p);
    return;
  }
  if (small_m && tiles >= 256)
    DispatchConv<32, 128, 4, TAPS>(p, stream);
  else if (!small_m && tiles >= 256)
    DispatchConv<64, 64, 4, TAPS>(p, stream);
  else
    DispatchConv<32, 32, 1, TAPS>(p, stream);
}

}  // namespace

void LaunchConv(const ConvParams& params, hipStream_t stream) {
  ConvParams p = params;
  if (p.ldw == 0)
    p.ldw = p.cout;
  if (p.batches == 0)
    p.batches = 1;
  if (p.out_act == kActNone)
    p.out_act = kActSnake;
  Require(p.x && p.w, "conv: null pointer");
  Require(p.y != nullptr || p.y_act != nullptr, "conv: no output");
  Require(!p.accumulate || p.y != nullptr, "conv: accumulation needs y");
  Require(p.y_act == nullptr || p.out_act != kActSnake || p.alpha_out != nullptr,
          "conv: activated output needs alpha");
  Require(p.pre_act == kActNone || p.pre_act == kActGelu, "conv: bad pre-activation");
  Require(p.out_act == kActSnake || p.out_act == kActElu, "conv: bad output activation");
  Require(p.ldw >= p.cout, "conv: weight rows shorter than cout");
  Require(p.batches >= 1 && static_cast<int64_t>(p.batches) * p.phases <= 65535,
          "conv: 1 to 65535 batches x phases");
  Require(p.batches == 1 || (p.x_batch >= 0 && p.w_batch >= 0 && p.b_batch >= 0 &&
                             p.y_batch >= 0),
          "conv: negative batch stride");
  Require(p.cin >= 1 && p.cout >= 1 && p.len_in >= 1 && p.positions >= 1,
          "conv: empty shape");
  Require(p.taps == 1 || p.taps == 2 || p.taps == 7, "conv: 1, 2 or 7 taps");
  Require(p.phases >= 1 && p.phases <= kConvMaxPhases, "conv: 1 to 8 phases");
  Require(p.out_stride >= p.phases, "conv: phases overlap in the output");
  Require(static_cast<int64_t>(p.positions - 1) * p.out_stride + p.phases - 1 < p.len_out,
          "conv: output positions past the output length");
  for (int ph = 0; ph < p.phases; ++ph) {
    int lo = p.offsets[ph][0], hi = lo;
    for (int k = 1; k < p.taps; ++k) {
      lo = std::min(lo, p.offsets[ph][k]);
      hi = std::max(hi, p.offsets[ph][k]);
    }
    Require(hi - lo <= (p.taps == 1 ? 0 : p.taps == 2 ? 1 : kConvMaxSpan),
            "conv: taps spread too far for their count");
  }
  if (p.taps == 1) {
    DispatchTaps<1>(p, stream);
  } else if (p.taps == 2) {
    DispatchTaps<2>(p, stream);
  } else {
    DispatchTaps<7>(p, stream);
  }
}

void LaunchOutputConv(const OutputConvParams& p, hipStream_t stream) {
  Require(p.x && p.w && p.bias && p.y, "output conv: null pointer");
  Require(p.cin >= 1 && p.length >= 1, "output conv: empty shape");
  Require(p.taps >= 1 && p.taps <= kConvMaxTaps && p.taps % 2 == 1,
          "output conv: 1, 3, 5 or 7 taps");
  Dispatch(OutputConvKernel, dim3((p.length + kOutTile - 1) / kOutTile), dim3(kThreads), 0,
           stream, true, true, p);
}

void LaunchRvq(const RvqParams& p, hipStream_t stream) {
  Require(p.table && p.bias && p.codes && p.y, "rvq: null pointer");
  Require(p.codebooks >= 1 && p.entries >= 1 && p.latent >= 1 && p.frames >= 1,
          "rvq: empty shape");
  Dispatch(RvqKernel, dim3(p.frames), dim3(kThreads), 0, stream, true, true, p);
}

}  // namespace ovg
