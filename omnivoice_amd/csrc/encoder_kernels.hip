// The audio encoder's element-wise, normalisation and selection kernels on
// gfx950 (the reference's kernels/encoder_kernels.hip counterparts: the
// resampler that audio.cpp:265-322 runs on the host, GroupNorm + GELU,
// LayerNorm, softmax, the frame pick and the RVQ nearest-entry search).
// Every GEMM-shaped layer of the encoder runs on the fp32 matrix cores
// through the convolution kernel; these kernels move each element once or
// twice and are bound by HBM or, at the encoder's small sizes, by launch.
//
// The column kernels (LayerNorm over channels, softmax over keys) read a
// channel-major matrix along its slow dimension: a work-group owns 16
// adjacent columns, 16 lanes of 16 threads each walk every 16th row, so
// each row read is 64 contiguous bytes, and the partial sums meet in LDS.
#include <algorithm>
#include <cfloat>

#include "codec.hpp"
#include "common.hpp"
#include "encoder.hpp"
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kThreads = 256;
constexpr int kColumns = 16;  // columns per work-group of a column kernel
constexpr int kSlices = kThreads / kColumns;

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
  double s = 0.0;
  for (int t = threadIdx.x; t < length; t += kThreads)
    s += row[t];
  const double mean = BlockSum(s, scratch) / length;
  double q = 0.0;
  for (int t = threadIdx.x; t < length; t += kThreads) {
    const double d = row[t] - mean;
    q += d * d;
  }
  const double inv = 1.0 / sqrt(BlockSum(q, scratch) / length + eps);
  const double wc = w[blockIdx.x], bc = b[blockIdx.x];
  for (int t = threadIdx.x; t < length; t += kThreads)
    row[t] = Gelu(static_cast<float>((row[t] - mean) * inv * wc + bc));
}

// Sum over the kSlices lanes of a column (threads col, col + 16, ...).
__device__ double ColumnSum(double v, double (*scratch)[kColumns]) {
  const int col = threadIdx.x % kColumns, slice = threadIdx.x / kColumns;
  __syncthreads();
  scratch[slice][col] = v;
  __syncthreads();
  double s = 0.0;
  for (int i = 0; i < kSlices; ++i)
    s += scratch[i][col];
  return s;
}

__global__ __launch_bounds__(kThreads) void ColumnNormKernel(ColumnNormParams p) {
  __shared__ double scratch[kSlices][kColumns];
  const int t = blockIdx.x * kColumns + threadIdx.x % kColumns;
  const int slice = threadIdx.x / kColumns;
  const bool live = t < p.positions;
  const int tc = min(t, p.positions - 1);
  double s = 0.0;
  for (int c = slice; c < p.channels; c += kSlices)
    s += p.x[static_cast<size_t>(c) * p.positions + tc];
  const double mean = ColumnSum(s, scratch) / p.channels;
  double q = 0.0;
  for (int c = slice; c < p.channels; c += kSlices) {
    const double d = p.x[static_cast<size_t>(c) * p.positions + tc] - mean;
    q += d * d;
  }
  const double inv = 1.0 / sqrt(ColumnSum(q, scratch) / p.channels + p.eps);
  if (!live)
    return;
  for (int c = slice; c < p.channels; c += kSlices) {
    const size_t at = static_cast<size_t>(c) * p.positions + t;
    const float v = static_cast<float>((p.x[at] - mean) * inv * p.w[c] + p.b[c]);
    p.y[at] = v;
    if (p.sum_mode == 1)
      p.sum[at] = v;
    else if (p.sum_mode == 2)
      p.sum[at] += v;
  }
}

__global__ __launch_bounds__(kThreads) void ColumnSoftmaxKernel(float* x, int rows, int cols,
                                                                float scale) {
  __shared__ double scratch[kSlices][kColumns];
  __shared__ float peak[kSlices][kColumns];
  float* m = x + static_cast<size_t>(blockIdx.y) * rows * cols;
  const int col = threadIdx.x % kColumns, slice = threadIdx.x / kColumns;
  const int t = blockIdx.x * kColumns + col;
  const int tc = min(t, cols - 1);
  float hi = -FLT_MAX;
  for (int r = slice; r < rows; r += kSlices)
    hi = fmaxf(hi, m[static_cast<size_t>(r) * cols + tc]);
  peak[slice][col] = hi;
  __syncthreads();
  for (int i = 0; i < kSlices; ++i)
    hi = fmaxf(hi, peak[i][col]);
  double s = 0.0;
  for (int r = slice; r < rows; r += kSlices)
    s += expf((m[static_cast<size_t>(r) * cols + tc] - hi) * scale);
  const float inv = static_cast<float>(1.0 / ColumnSum(s, scratch));
  if (t >= cols)
    return;
  for (int r = slice; r < rows; r += kSlices) {
    const size_t at = static_cast<size_t>(r) * cols + t;
    m[at] = expf((m[at] - hi) * scale) * inv;
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
  Require(p.channels >= 1 && p.positions >= 1, "layer norm: empty shape");
  Dispatch(ColumnNormKernel, dim3((p.positions + kColumns - 1) / kColumns), dim3(kThreads), 0,
           stream, true, true, p);
}

void LaunchColumnSoftmax(float* x, int batches, int rows, int cols, float scale,
                         hipStream_t stream) {
  Require(x != nullptr, "softmax: null pointer");
  Require(batches >= 1 && batches <= 65535 && rows >= 1 && cols >= 1, "softmax: bad shape");
  Dispatch(ColumnSoftmaxKernel, dim3((cols + kColumns - 1) / kColumns, batches), dim3(kThreads),
           0, stream, true, true, x, rows, cols, scale);
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
