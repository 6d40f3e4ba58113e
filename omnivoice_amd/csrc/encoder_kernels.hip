// The audio encoder's element-wise, normalisation and selection kernels on
// gfx950 (the reference's kernels/encoder_kernels.hip counterparts: the
// resampler that audio.cpp:265-322 runs on the host, GroupNorm + GELU,
// LayerNorm, softmax, the frame pick and the RVQ nearest-entry search).
// Every GEMM-shaped layer of the encoder runs on the fp32 matrix cores
// through the convolution kernel; these kernels move each element once or
// twice and are bound by HBM or, at the encoder's small sizes, by launch.
//
// The column kernels (LayerNorm over channels, softmax over keys) read a
// channel-major matrix along its slow dimension: a work-group owns 8
// adjacent columns, each column 32 lanes that hold every 32nd row in
// registers, so each element is read once, all of a thread's loads are in
// flight together, and the partial sums meet in LDS.
#include <algorithm>
#include <cfloat>
#include <type_traits>

#include "codec.hpp"
#include "common.hpp"
#include "encoder.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float Gelu(float v) {
  return 0.5F * v * (1.0F + erff(v * 0.70710678118654752F));
}
__device__ __forceinline__ float Elu(float v) { return v > 0.0F ? v : expm1f(v); }

__global__ __launch_bounds__(kThreads) void ResampleKernel(ResampleParams p) {
  const int total = p.out_length + 2 * p.pad;
  for (int i = blockIdx.x * kThreads + threadIdx.x; i < total; i += gridDim.x * kThreads) {
    const int j = i - p.pad;
    float out = 0.0F;
    if (j >= 0 && j < p.out_length) {
      const int phase = j % p.to;
      const int origin = (j / p.to) * p.from - p.width;
      const float* w = p.bank + static_cast<size_t>(phase) * p.taps;
      const int lo = max(0, -origin), hi = min(p.taps, p.length - origin);
      double sum = 0.0;
      for (int k = lo; k < hi; ++k)
        sum += static_cast<double>(w[k]) * p.x[origin + k];
      out = static_cast<float>(sum);
    }
    p.y[i] = out;
  }
}

__global__ __launch_bounds__(kThreads) void Im2colKernel(Im2colParams p) {
  const size_t total = static_cast<size_t>(p.channels) * p.kernel * p.positions;
  for (size_t e = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; e < total;
       e += static_cast<size_t>(gridDim.x) * kThreads) {
    const int t = static_cast<int>(e % p.positions);
    const int r = static_cast<int>(e / p.positions);
    const int j = r % p.kernel;
    const int c = r / p.kernel;
    const int s = t * p.stride + j * p.dilation - p.pad;
    float v = 0.0F;
    if (s >= 0 && s < p.len_in) {
      v = p.x[static_cast<size_t>(c) * p.len_in + s];
      if (p.act == kActElu)
        v = Elu(v);
    }
    p.y[e] = v;
  }
}

// Sum of one double per thread over the work-group (every thread gets it).
__device__ double BlockSum(double v, double* scratch) {
  for (int o = 32; o > 0; o >>= 1)
    v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    scratch[wave] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kThreads / 64; ++i)
    s += scratch[i];
  return s;
}

__global__ __launch_bounds__(kThreads) void GroupNormGeluKernel(float* x, const float* w,
                                                                const float* b, int length,
                                                                float eps) {
  __shared__ double scratch[kThreads / 64];
  float* row = x + static_cast<size_t>(blockIdx.x) * length;
  // One pass for the sum and the sum of squares (double), unrolled so that
  // eight loads are in flight per thread.
  double s = 0.0, q = 0.0;
#pragma unroll 8
  for (int t = threadIdx.x; t < length; t += kThreads) {
    const double v = row[t];
    s += v;
    q += v * v;
  }
  const double mean = BlockSum(s, scratch) / length;
  const double var = fmax(BlockSum(q, scratch) / length - mean * mean, 0.0);
  const double inv = 1.0 / sqrt(var + eps);
  const double wc = w[blockIdx.x], bc = b[blockIdx.x];
#pragma unroll 8
  for (int t = threadIdx.x; t < length; t += kThreads)
    row[t] = Gelu(static_cast<float>((row[t] - mean) * inv * wc + bc));
}

// The column kernels: a work-group of kCols adjacent columns x kLanes lanes;
// lane l of a column holds rows l, l + kLanes, ... (up to kPer of them) in
// registers, so every element is read once with all its loads in flight.
constexpr int kCols = 8;
constexpr int kLanes = kThreads / kCols;

// Sum over the lanes of a column.
__device__ double LaneSum(double v, double (*scratch)[kCols]) {
  const int col = threadIdx.x % kCols, lane = threadIdx.x / kCols;
  __syncthreads();
  scratch[lane][col] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kLanes; ++i)
    s += scratch[i][col];
  return s;
}

template <int kPer>
__global__ __launch_bounds__(kThreads) void ColumnNormKernel(ColumnNormParams p) {
  __shared__ double scratch[kLanes][kCols];
  const int t = blockIdx.x * kCols + threadIdx.x % kCols;
  const int lane = threadIdx.x / kCols;
  const int tc = min(t, p.positions - 1);
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = min(lane + i * kLanes, p.channels - 1);
    v[i] = p.x[static_cast<size_t>(c) * p.positions + tc];
  }
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (lane + i * kLanes < p.channels)
      s += v[i];
  const double mean = LaneSum(s, scratch) / p.channels;
  double q = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (lane + i * kLanes < p.channels) {
      const double d = v[i] - mean;
      q += d * d;
    }
  const double inv = 1.0 / sqrt(LaneSum(q, scratch) / p.channels + p.eps);
  if (t >= p.positions)
    return;
  // Every load of the store loop first, all in flight together: y may alias
  // them as far as the compiler knows, so loads left inside the loop would
  // each wait out a memory round trip behind the previous store.
  float w[kPer], b[kPer];
  double prior[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = min(lane + i * kLanes, p.channels - 1);
    w[i] = p.w[c];
    b[i] = p.b[c];
    prior[i] = p.sum_mode == 2 ? p.sum[static_cast<size_t>(c) * p.positions + t] : 0.0;
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = lane + i * kLanes;
    if (c < p.channels) {
      const size_t at = static_cast<size_t>(c) * p.positions + t;
      const float o = static_cast<float>((v[i] - mean) * inv * w[i] + b[i]);
      p.y[at] = o;
      if (p.sum_mode != 0)
        p.sum[at] = prior[i] + o;
    }
  }
}

// Softmax down columns longer than the registers hold: three passes over
// the rows, eight loads in flight per lane.
__global__ __launch_bounds__(kThreads) void ColumnSoftmaxLongKernel(float* x, int rows, int cols,
                                                                    float scale) {
  __shared__ double scratch[kLanes][kCols];
  __shared__ float peak[kLanes][kCols];
  float* m = x + static_cast<size_t>(blockIdx.y) * rows * cols;
  const int col = threadIdx.x % kCols, lane = threadIdx.x / kCols;
  const int t = blockIdx.x * kCols + col;
  const int tc = min(t, cols - 1);
  float hi = -FLT_MAX;
#pragma unroll 8
  for (int r = lane; r < rows; r += kLanes)
    hi = fmaxf(hi, m[static_cast<size_t>(r) * cols + tc]);
  peak[lane][col] = hi;
  __syncthreads();
  for (int i = 0; i < kLanes; ++i)
    hi = fmaxf(hi, peak[i][col]);
  double s = 0.0;
#pragma unroll 8
  for (int r = lane; r < rows; r += kLanes)
    s += expf((m[static_cast<size_t>(r) * cols + tc] - hi) * scale);
  const float inv = static_cast<float>(1.0 / LaneSum(s, scratch));
  if (t >= cols)
    return;
#pragma unroll 8
  for (int r = lane; r < rows; r += kLanes) {
    const size_t at = static_cast<size_t>(r) * cols + t;
    m[at] = expf((m[at] - hi) * scale) * inv;
  }
}

template <int kPer>
__global__ __launch_bounds__(kThreads) void ColumnSoftmaxKernel(float* x, int rows, int cols,
                                                                float scale) {
  __shared__ double scratch[kLanes][kCols];
  __shared__ float peak[kLanes][kCols];
  float* m = x + static_cast<size_t>(blockIdx.y) * rows * cols;
  const int col = threadIdx.x % kCols, lane = threadIdx.x / kCols;
  const int t = blockIdx.x * kCols + col;
  const int tc = min(t, cols - 1);
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    v[i] = m[static_cast<size_t>(min(lane + i * kLanes, rows - 1)) * cols + tc];
  float hi = -FLT_MAX;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (lane + i * kLanes < rows)
      hi = fmaxf(hi, v[i]);
  peak[lane][col] = hi;
  __syncthreads();
  for (int i = 0; i < kLanes; ++i)
    hi = fmaxf(hi, peak[i][col]);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = expf((v[i] - hi) * scale);
    if (lane + i * kLanes < rows)
      s += v[i];
  }
  const float inv = static_cast<float>(1.0 / LaneSum(s, scratch));
  if (t >= cols)
    return;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = lane + i * kLanes;
    if (r < rows)
      m[static_cast<size_t>(r) * cols + t] = v[i] * inv;
  }
}

__global__ __launch_bounds__(kThreads) void TransposeKernel(const float* x, int rows, int cols,
                                                            int ldx, float* y) {
  __shared__ float tile[32][33];
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 8 rows per pass
  for (int i = ty; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + tx;
    if (r < rows && c < cols)
      tile[i][tx] = x[static_cast<size_t>(r) * ldx + c];
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + tx;
    if (r < rows && c < cols)
      y[static_cast<size_t>(c) * rows + r] = tile[tx][i];
  }
}

__global__ __launch_bounds__(kThreads) void PickFramesKernel(const double* sum, int channels,
                                                             int positions, int stride,
                                                             int frames, double scale,
                                                             float* y) {
  const int total = channels * frames;
  for (int e = blockIdx.x * kThreads + threadIdx.x; e < total; e += gridDim.x * kThreads) {
    const int c = e / frames, f = e % frames;
    y[e] = static_cast<float>(sum[static_cast<size_t>(c) * positions +
                                  static_cast<size_t>(f) * stride] * scale);
  }
}

constexpr int kMaxDim = 1024;

__global__ __launch_bounds__(kThreads) void NearestKernel(NearestParams p) {
  __shared__ double v[kMaxDim];
  __shared__ double scratch[kThreads / 64];
  __shared__ double best_d[kThreads];
  __shared__ int best_e[kThreads];
  const int f = blockIdx.x;
  double pp = 0.0;
  for (int d = threadIdx.x; d < p.dim; d += kThreads) {
    const double x = p.proj[static_cast<size_t>(d) * p.frames + f];
    v[d] = x;
    pp += x * x;
  }
  // |p|^2 summed in a fixed order: lane partials, then the waves in turn.
  pp = BlockSum(pp, scratch);
  double best = -DBL_MAX;
  int arg = 0;
  for (int e = threadIdx.x; e < p.entries; e += kThreads) {
    const float* row = p.embed + static_cast<size_t>(e) * p.dim;
    double dot = 0.0;
    for (int d = 0; d < p.dim; ++d)
      dot += v[d] * row[d];
    const double dist = -((pp - 2.0 * dot) + p.norms[e]);
    if (dist > best) {  // entries ascend per thread: ties keep the lower
      best = dist;
      arg = e;
    }
  }
  best_d[threadIdx.x] = best;
  best_e[threadIdx.x] = arg;
  __syncthreads();
  for (int half = kThreads / 2; half > 0; half >>= 1) {
    if (threadIdx.x < half) {
      const double od = best_d[threadIdx.x + half];
      const int oe = best_e[threadIdx.x + half];
      if (od > best_d[threadIdx.x] || (od == best_d[threadIdx.x] && oe < best_e[threadIdx.x])) {
        best_d[threadIdx.x] = od;
        best_e[threadIdx.x] = oe;
      }
    }
    __syncthreads();
  }
  const int code = best_e[0];
  if (threadIdx.x == 0)
    p.codes[f] = code;
  const float* row = p.table + static_cast<size_t>(code) * p.hidden;
  for (int h = threadIdx.x; h < p.hidden; h += kThreads)
    p.residual[static_cast<size_t>(h) * p.frames + f] -= row[h];
}

// Register-cached column kernels hold up to 64 rows per lane: 2048 rows
// (LayerNorm, which also holds its weights and running sums: 1024).
constexpr int kMaxColumnRows = 64 * kLanes;
constexpr int kMaxNormChannels = 32 * kLanes;

template <typename K>
void ColumnDispatch(int rows, K&& launch) {
  if (rows <= 8 * kLanes)
    launch(std::integral_constant<int, 8>());
  else if (rows <= 16 * kLanes)
    launch(std::integral_constant<int, 16>());
  else if (rows <= 32 * kLanes)
    launch(std::integral_constant<int, 32>());
  else
    launch(std::integral_constant<int, 64>());
}

int Blocks(size_t work) {
  return static_cast<int>(std::min<size_t>((work + kThreads - 1) / kThreads, 256 * 64));
}

}  // namespace

void LaunchResample(const ResampleParams& p, hipStream_t stream) {
  Require(p.x && p.bank && p.y, "resample: null pointer");
  Require(p.length >= 1 && p.from >= 1 && p.to >= 1 && p.taps >= 1 && p.width >= 0 &&
              p.out_length >= 1 && p.pad >= 0,
          "resample: bad shape");
  Dispatch(ResampleKernel, dim3(Blocks(static_cast<size_t>(p.out_length) + 2 * p.pad)),
           dim3(kThreads), 0, stream, true, true, p);
}

void LaunchIm2col(const Im2colParams& p, hipStream_t stream) {
  Require(p.x && p.y, "im2col: null pointer");
  Require(p.channels >= 1 && p.len_in >= 1 && p.kernel >= 1 && p.stride >= 1 &&
              p.dilation >= 1 && p.pad >= 0 && p.positions >= 1,
          "im2col: bad shape");
  Require(p.act == kActNone || p.act == kActElu, "im2col: bad activation");
  const size_t total = static_cast<size_t>(p.channels) * p.kernel * p.positions;
  Dispatch(Im2colKernel, dim3(Blocks(total)), dim3(kThreads), 0, stream, true, true, p);
}

void LaunchGroupNormGelu(float* x, const float* w, const float* b, int channels, int length,
                         float eps, hipStream_t stream) {
  Require(x && w && b, "group norm: null pointer");
  Require(channels >= 1 && length >= 1, "group norm: empty shape");
  Dispatch(GroupNormGeluKernel, dim3(channels), dim3(kThreads), 0, stream, true, true, x, w, b,
           length, eps);
}

void LaunchColumnNorm(const ColumnNormParams& p, hipStream_t stream) {
  Require(p.x && p.y && p.w && p.b, "layer norm: null pointer");
  Require(p.sum_mode == 0 || p.sum != nullptr, "layer norm: no sum buffer");
  Require(p.channels >= 1 && p.channels <= kMaxNormChannels && p.positions >= 1,
          "layer norm: 1 to 1024 channels");
  ColumnDispatch(p.channels, [&](auto per) {
    if constexpr (decltype(per)::value <= kMaxNormChannels / kLanes)
      Dispatch(ColumnNormKernel<decltype(per)::value>, dim3((p.positions + kCols - 1) / kCols),
               dim3(kThreads), 0, stream, true, true, p);
  });
}

void LaunchColumnSoftmax(float* x, int batches, int rows, int cols, float scale,
                         hipStream_t stream) {
  Require(x != nullptr, "softmax: null pointer");
  Require(batches >= 1 && batches <= 65535 && rows >= 1 && cols >= 1, "softmax: bad shape");
  if (rows > kMaxColumnRows) {
    Dispatch(ColumnSoftmaxLongKernel, dim3((cols + kCols - 1) / kCols, batches), dim3(kThreads),
             0, stream, true, true, x, rows, cols, scale);
    return;
  }
  ColumnDispatch(rows, [&](auto per) {
    Dispatch(ColumnSoftmaxKernel<decltype(per)::value>,
             dim3((cols + kCols - 1) / kCols, batches), dim3(kThreads), 0, stream, true, true, x,
             rows, cols, scale);
  });
}

void LaunchTranspose(const float* x, int rows, int cols, int ldx, float* y,
                     hipStream_t stream) {
  Require(x && y, "transpose: null pointer");
  Require(rows >= 1 && cols >= 1 && ldx >= cols && (rows + 31) / 32 <= 65535,
          "transpose: bad shape");
  Dispatch(TransposeKernel, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(kThreads), 0, stream,
           true, true, x, rows, cols, ldx, y);
}

void LaunchPickFrames(const double* sum, int channels, int positions, int stride, int frames,
                      double scale, float* y, hipStream_t stream) {
  Require(sum && y, "pick frames: null pointer");
  Require(channels >= 1 && frames >= 1 && stride >= 1 &&
              static_cast<int64_t>(frames - 1) * stride < positions,
          "pick frames: frames past the states");
  Dispatch(PickFramesKernel, dim3(Blocks(static_cast<size_t>(channels) * frames)),
           dim3(kThreads), 0, stream, true, true, sum, channels, positions, stride, frames,
           scale, y);
}

void LaunchNearest(const NearestParams& p, hipStream_t stream) {
  Require(p.proj && p.embed && p.norms && p.table && p.residual && p.codes,
          "nearest: null pointer");
  Require(p.dim >= 1 && p.dim <= kMaxDim && p.entries >= 1 && p.hidden >= 1 && p.frames >= 1,
          "nearest: bad shape");
  Dispatch(NearestKernel, dim3(p.frames), dim3(kThreads), 0, stream, true, true, p);
}

}  // namespace ovg
