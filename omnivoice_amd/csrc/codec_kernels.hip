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
constexpr int kChunk = 16;     // input channels per K chunk
constexpr int kOutTile = 256;  // samples per work-group of the output conv
constexpr int kOutChunk = 32;  // input channels per chunk of the output conv

// kernels/codec_kernels.hip:20-22 of the reference: x + sin^2(a x) / (a + 1e-9).
__device__ __forceinline__ float Snake(float v, float a) {
  const float s = sinf(a * v);
  return v + (1.0F / (a + 1e-9F)) * (s * s);
}

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void ConvKernel(ConvParams p) {
  static_assert(BM * BN == 4 * 32 * 32, "four 32 x 32 wave blocks");
  constexpr int kWavesN = BN / 32;
  constexpr int kWidth = BN + kConvMaxSpan;
  __shared__ float xs[kChunk][kWidth];
  __shared__ float ws[kConvMaxTaps][kChunk][BM];

  const int phase = blockIdx.z;
  const int m0 = blockIdx.x * BN;
  const int co0 = blockIdx.y * BM;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = (wave / kWavesN) * 32;  // first output channel of the wave
  const int col = (wave % kWavesN) * 32;  // first position of the wave
  const int half = lane >> 5;             // K index of the lane's operands
  const int l32 = lane & 31;
  const int taps = p.taps;
  const int* offsets = p.offsets[phase];
  int lo = offsets[0], hi = offsets[0];
  for (int k = 1; k < taps; ++k) {
    lo = min(lo, offsets[k]);
    hi = max(hi, offsets[k]);
  }
  const int width = BN + hi - lo;  // <= kWidth (checked by the launcher)
  const float* w = p.w + static_cast<size_t>(phase) * taps * p.cin * p.cout;

  floatx16 acc = {};
  for (int c0 = 0; c0 < p.cin; c0 += kChunk) {
    // The input window: xs[c][j] = act(x[c0 + c][m0 + lo + j]). Each thread
    // takes whole columns, so a column's 16 loads leave together.
    // Loads are unconditional (clamped addresses, then a select), so that
    // all of them leave before the first returns.
    for (int j = tid; j < width; j += kThreads) {
      const int t = m0 + lo + j;
      const bool inside = t >= 0 && t < p.len_in;
      const int tc = min(max(t, 0), p.len_in - 1);
      float v[kChunk];
#pragma unroll
      for (int c = 0; c < kChunk; ++c)
        v[c] = p.x[static_cast<size_t>(min(c0 + c, p.cin - 1)) * p.len_in + tc];
      if (p.alpha != nullptr) {
#pragma unroll
        for (int c = 0; c < kChunk; ++c)
          v[c] = Snake(v[c], p.alpha[min(c0 + c, p.cin - 1)]);
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c)
        xs[c][j] = inside && c0 + c < p.cin ? v[c] : 0.0F;
    }
    for (int i = tid; i < taps * kChunk * BM; i += kThreads) {
      const int o = i % BM;
      const int c = (i / BM) % kChunk;
      const int k = i / (BM * kChunk);
      const int ci = c0 + c;
      const int co = co0 + o;
      const float v = w[(static_cast<size_t>(k) * p.cin + min(ci, p.cin - 1)) * p.cout +
                        min(co, p.cout - 1)];
      ws[k][c][o] = ci < p.cin && co < p.cout ? v : 0.0F;
    }
    __syncthreads();
    for (int k = 0; k < taps; ++k) {
      const int shift = offsets[k] - lo;
#pragma unroll
      for (int s = 0; s < kChunk / 2; ++s) {
        const float a = ws[k][2 * s + half][row + l32];
        const float b = xs[2 * s + half][col + l32 + shift];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // Element r of the accumulator: output channel row + 8 (r / 4) +
  // 4 half + r % 4, position col + l32.
  const int m = m0 + col + l32;
  if (m >= p.positions)
    return;
  float* out = p.y + static_cast<size_t>(m) * p.out_stride + phase;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int co = co0 + row + 8 * (r >> 2) + 4 * half + (r & 3);
    if (co < p.cout) {
      float* dst = out + static_cast<size_t>(co) * p.len_out;
      const float v = acc[r] + p.bias[co];
      *dst = p.accumulate ? *dst + v : v;
    }
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
        xs[c][j] = inside && c0 + c < p.cin ? Snake(v[c], p.alpha[min(c0 + c, p.cin - 1)])
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

template <int BM, int BN>
void DispatchConv(const ConvParams& p, hipStream_t stream) {
  const dim3 grid((p.positions + BN - 1) / BN, (p.cout + BM - 1) / BM, p.phases);
  Dispatch(ConvKernel<BM, BN>, grid, dim3(kThreads), 0, stream, true, true, p);
}

}  // namespace

void LaunchConv(const ConvParams& p, hipStream_t stream) {
  Require(p.x && p.w && p.bias && p.y, "conv: null pointer");
  Require(p.cin >= 1 && p.cout >= 1 && p.len_in >= 1 && p.positions >= 1,
          "conv: empty shape");
  Require(p.taps >= 1 && p.taps <= kConvMaxTaps, "conv: 1 to 7 taps");
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
    Require(hi - lo <= kConvMaxSpan, "conv: taps spread over more than 64 samples");
  }
  if (p.cout <= 32)
    DispatchConv<32, 128>(p, stream);
  else
    DispatchConv<64, 64>(p, stream);
}

void LaunchOutputConv(const OutputConvParams& p, hipStream_t stream) {
  Require(p.x && p.alpha && p.w && p.bias && p.y, "output conv: null pointer");
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
