// Row-wise kernels of the generator: the embedding gather-sum fused with the
// first layer's input RMSNorm, RMSNorm (optionally gathering rows), the V
// transpose used by the attention operator, and an int fill (used instead of
// hipMemsetAsync so that captured graphs hold kernel nodes only).
//
// One 256-thread work-group per row; each thread owns float4 columns, so a
// 1024-wide row is one float4 per thread and the sum of squares is a wave
// butterfly plus a fixed-order sum of the four wave totals.
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kRowThreads = 256;

__device__ __forceinline__ float BlockSum(float v, float* scratch) {
  v = WaveSumFast(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0)
    scratch[wave] = v;
  __syncthreads();
  const float total = (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
  __syncthreads();
  return total;
}

// kernels::Embed (reference kernels/generator_kernels.hip:62-83): text rows
// copy their token's float32 row, audio rows sum the 8 codebooks'
// embeddings of their codes (a masked frame sums the 8 mask rows),
// padding rows are zero. Then RMSNorm with the first layer's input norm
// (kernels/generator_kernels.hip:85-97).
__global__ __launch_bounds__(kRowThreads) void EmbedKernel(EmbedParams p) {
  __shared__ float scratch[4];
  const int row = blockIdx.x;
  if (p.epoch != nullptr && row == 0 && threadIdx.x == 0)
    *p.epoch += 1;
  const int kind = p.row_kind[row];
  float* out = p.hidden + static_cast<size_t>(row) * p.hidden_size;
  half_t* normed = p.normed + static_cast<size_t>(row) * p.hidden_size;
  float squares = 0.0F;
  constexpr int kMaxChunks = 4;  // hidden <= 4096
  constexpr int kMaxCodebooks = 16;
  // The row's ids, then every embedding row and the norm weights, are
  // loaded before any arithmetic: two dependent memory round trips in all.
  int entry[kMaxCodebooks];
  const int codebooks = kind == 1 ? p.codebooks : (kind == 0 ? 1 : 0);
#pragma unroll
  for (int c = 0; c < kMaxCodebooks; ++c)
    entry[c] = c >= codebooks ? 0
               : kind == 0    ? p.ids[row]
                              : c * p.vocab + p.ids[static_cast<size_t>(c) * p.ld_ids + row];
  const float* table = kind == 0 ? p.text : p.audio;
  floatx4 v[kMaxChunks], w[kMaxChunks];
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int d = (threadIdx.x + i * kRowThreads) * 4;
    v[i] = floatx4{0, 0, 0, 0};
    w[i] = floatx4{0, 0, 0, 0};
    if (d >= p.hidden_size)
      continue;
    w[i] = *reinterpret_cast<const floatx4*>(p.norm + d);
#pragma unroll
    for (int c = 0; c < kMaxCodebooks; ++c)
      if (c < codebooks)
        v[i] += *reinterpret_cast<const floatx4*>(
            table + static_cast<size_t>(entry[c]) * p.hidden_size + d);
  }
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int d = (threadIdx.x + i * kRowThreads) * 4;
    if (d >= p.hidden_size)
      continue;
    *reinterpret_cast<floatx4*>(out + d) = v[i];
    squares += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] +
               v[i][3] * v[i][3];
  }
  const float total = BlockSum(squares, scratch);
  const float scale =
      rsqrtf(total / static_cast<float>(p.hidden_size) + p.eps);
#pragma unroll
  for (int i = 0; i < kMaxChunks; ++i) {
    const int d = (threadIdx.x + i * kRowThreads) * 4;
    if (d >= p.hidden_size)
      continue;
    const half4 h = {static_cast<half_t>(w[i][0] * (v[i][0] * scale)),
                     static_cast<half_t>(w[i][1] * (v[i][1] * scale)),
                     static_cast<half_t>(w[i][2] * (v[i][2] * scale)),
                     static_cast<half_t>(w[i][3] * (v[i][3] * scale))};
    *reinterpret_cast<half4*>(normed + d) = h;
  }
}

// The same for the released shape (8 codebooks, hidden 1024: one float4 per
// thread), with no branch before the arithmetic: every id, then every
// embedding row, is loaded unconditionally (unused codebooks of text and
// padding rows re-read the row's first entry, a cache hit), and the sum
// selects the rows in use. A row then costs two memory round trips instead
// of one per conditionally loaded row. The sum runs in codebook order from
// +0, as in EmbedKernel (adding +0 for an unused codebook leaves it
// unchanged).
__global__ __launch_bounds__(kRowThreads) void Embed8Kernel(EmbedParams p) {
  constexpr int kCodebooks = 8;
  __shared__ float scratch[4];
  const int row = blockIdx.x;
  if (p.epoch != nullptr && row == 0 && threadIdx.x == 0)
    *p.epoch += 1;
  const int kind = p.row_kind[row];
  const int count = kind == 1 ? kCodebooks : (kind == 0 ? 1 : 0);
  int id[kCodebooks];
#pragma unroll
  for (int c = 0; c < kCodebooks; ++c)
    id[c] = p.ids[static_cast<size_t>(c) * p.ld_ids + row];
  const float* table = kind == 0 ? p.text : p.audio;
  const int d = threadIdx.x * 4;
  const floatx4 w = *reinterpret_cast<const floatx4*>(p.norm + d);
  floatx4 e[kCodebooks];
#pragma unroll
  for (int c = 0; c < kCodebooks; ++c) {
    const int entry = kind == 0 ? id[0] : c * p.vocab + id[c];
    e[c] = *reinterpret_cast<const floatx4*>(
        table + static_cast<size_t>(entry) * p.hidden_size + d);
  }
  floatx4 v = {0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < kCodebooks; ++c)
    v += c < count ? e[c] : floatx4{0, 0, 0, 0};
  float* out = p.hidden + static_cast<size_t>(row) * p.hidden_size;
  *reinterpret_cast<floatx4*>(out + d) = v;
  const float squares =
      v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  const float total = BlockSum(squares, scratch);
  const float scale =
      rsqrtf(total / static_cast<float>(p.hidden_size) + p.eps);
  half_t* normed = p.normed + static_cast<size_t>(row) * p.hidden_size;
  *reinterpret_cast<half4*>(normed + d) =
      half4{static_cast<half_t>(w[0] * (v[0] * scale)),
            static_cast<half_t>(w[1] * (v[1] * scale)),
            static_cast<half_t>(w[2] * (v[2] * scale)),
            static_cast<half_t>(w[3] * (v[3] * scale))};
}

// One wave per row, four rows per work-group: lane l owns the float4
// columns 4 (l + 64 i), so every load is a contiguous 1 KB per wave and the
// row sum of squares is one wave butterfly (no barriers). CHUNKS float4 per
// lane cover widths up to 256 CHUNKS.
template <int CHUNKS>
__global__ __launch_bounds__(kRowThreads) void RmsNormKernel(
    const float* x, const int* gather, const float* w, half_t* out, int rows,
    int width, float eps) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (r >= rows)
    return;
  const int src = gather != nullptr ? gather[r] : r;
  const float* in = x + static_cast<size_t>(src) * width;
  floatx4 v[CHUNKS], wv[CHUNKS];
  float squares = 0.0F;
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i) {
    const int d = (lane + 64 * i) * 4;
    v[i] = d < width ? *reinterpret_cast<const floatx4*>(in + d)
                     : floatx4{0, 0, 0, 0};
    wv[i] = d < width ? *reinterpret_cast<const floatx4*>(w + d)
                      : floatx4{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i)
    squares += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] +
               v[i][3] * v[i][3];
  const float scale = rsqrtf(WaveSumFast(squares) / static_cast<float>(width) + eps);
  half_t* o = out + static_cast<size_t>(r) * width;
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i) {
    const int d = (lane + 64 * i) * 4;
    if (d >= width)
      break;
    *reinterpret_cast<half4*>(o + d) =
        half4{static_cast<half_t>(wv[i][0] * (v[i][0] * scale)),
              static_cast<half_t>(wv[i][1] * (v[i][1] * scale)),
              static_cast<half_t>(wv[i][2] * (v[i][2] * scale)),
              static_cast<half_t>(wv[i][3] * (v[i][3] * scale))};
  }
}

// Residual update + RMSNorm (see AddNormParams), one single-wave work-group
// per row, so that the row's reads (up to 9 rows of 4 KB) spread over as
// many CUs as there are rows. All of a row's loads (hidden and every split
// slice) are issued before the sum, which then runs in the fixed order
// hidden + slice 0 + slice 1 + ...
template <int CHUNKS, int MAX_SPLITS>
__global__ __launch_bounds__(64) void AddNormKernel(AddNormParams p) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x;
  if (r >= p.rows)
    return;
  const int src = p.gather != nullptr ? p.gather[r] : r;
  float* h = p.hidden + static_cast<size_t>(src) * p.width;
  const float* part = p.partials + static_cast<size_t>(src) * p.width;
  floatx4 v[CHUNKS], wv[CHUNKS];
  floatx4 parts[MAX_SPLITS][CHUNKS];
  // Every load (norm weights included) is issued before any arithmetic, so
  // the row costs one memory round trip.
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i) {
    const int d = (lane + 64 * i) * 4;
    const bool ok = d < p.width;
    v[i] = ok ? *reinterpret_cast<const floatx4*>(h + d) : floatx4{0, 0, 0, 0};
    wv[i] = ok ? *reinterpret_cast<const floatx4*>(p.norm + d) : floatx4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; ++s)
      parts[s][i] = ok && s < p.splits
                        ? *reinterpret_cast<const floatx4*>(part + s * p.split_stride + d)
                        : floatx4{0, 0, 0, 0};
  }
  float squares = 0.0F;
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i) {
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; ++s)
      if (s < p.splits)
        v[i] += parts[s][i];
    squares += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] +
               v[i][3] * v[i][3];
  }
  if (p.gather == nullptr) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int d = (lane + 64 * i) * 4;
      if (d < p.width)
        *reinterpret_cast<floatx4*>(h + d) = v[i];
    }
  }
  const float scale =
      rsqrtf(WaveSumFast(squares) / static_cast<float>(p.width) + p.eps);
  half_t* o = p.out + static_cast<size_t>(r) * p.width;
#pragma unroll
  for (int i = 0; i < CHUNKS; ++i) {
    const int d = (lane + 64 * i) * 4;
    if (d >= p.width)
      break;
    *reinterpret_cast<half4*>(o + d) =
        half4{static_cast<half_t>(wv[i][0] * (v[i][0] * scale)),
              static_cast<half_t>(wv[i][1] * (v[i][1] * scale)),
              static_cast<half_t>(wv[i][2] * (v[i][2] * scale)),
              static_cast<half_t>(wv[i][3] * (v[i][3] * scale))};
  }
}

// The same for rows of 1024 (lane l owns float4 columns 4 (l + 64 i),
// i < 4) with the slice count fixed at compile time: no load is
// conditional, so all of a row's loads leave before the first returns (the
// guarded loads of AddNormKernel let the compiler wait between them). The
// arithmetic is AddNormKernel's, in the same order.
template <int SPLITS>
__global__ __launch_bounds__(64) void AddNorm1024Kernel(AddNormParams p) {
  constexpr int kChunks = 4;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x;
  const int src = p.gather != nullptr ? p.gather[r] : r;
  float* h = p.hidden + static_cast<size_t>(src) * 1024;
  const float* part = p.partials + static_cast<size_t>(src) * 1024;
  floatx4 v[kChunks], wv[kChunks], parts[SPLITS][kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int d = (lane + 64 * i) * 4;
    v[i] = *reinterpret_cast<const floatx4*>(h + d);
    wv[i] = *reinterpret_cast<const floatx4*>(p.norm + d);
#pragma unroll
    for (int s = 0; s < SPLITS; ++s)
      parts[s][i] = *reinterpret_cast<const floatx4*>(part + s * p.split_stride + d);
  }
  float squares = 0.0F;
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
#pragma unroll
    for (int s = 0; s < SPLITS; ++s)
      v[i] += parts[s][i];
    squares += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] +
               v[i][3] * v[i][3];
  }
  if (p.gather == nullptr) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
      *reinterpret_cast<floatx4*>(h + (lane + 64 * i) * 4) = v[i];
  }
  const float scale = rsqrtf(WaveSumFast(squares) / 1024.0F + p.eps);
  half_t* o = p.out + static_cast<size_t>(r) * 1024;
#pragma unroll
  for (int i = 0; i < kChunks; ++i)
    *reinterpret_cast<half4*>(o + (lane + 64 * i) * 4) =
        half4{static_cast<half_t>(wv[i][0] * (v[i][0] * scale)),
              static_cast<half_t>(wv[i][1] * (v[i][1] * scale)),
              static_cast<half_t>(wv[i][2] * (v[i][2] * scale)),
              static_cast<half_t>(wv[i][3] * (v[i][3] * scale))};
}

// One thread per (head slot, dim, row): slots below heads + kv_heads are q
// and k heads (QkIndex), the rest value heads (VtIndex).
__global__ void AttentionLayoutKernel(const half_t* qkv, int ld_qkv, half_t* qk, int ldq,
                                      half_t* vt, int ldvt, int rows, int heads,
                                      int kv_heads) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  const int d = blockIdx.y;
  const int slot = blockIdx.z;
  if (row >= rows)
    return;
  const half_t x = qkv[static_cast<size_t>(row) * ld_qkv + slot * 128 + d];
  if (slot < heads + kv_heads)
    qk[QkIndex(slot, row, d, ldq)] = x;
  else
    vt[VtIndex(slot - heads - kv_heads, d, row, ldvt)] = x;
}

__global__ void RopeRowsKernel(const float2* table, const int* positions,
                               int rows, float2* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows * 64)
    out[i] = table[static_cast<size_t>(positions[i / 64]) * 64 + i % 64];
}

__global__ void FillKernel(int* data, int value, int count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count)
    data[i] = value;
}

}  // namespace

void LaunchEmbed(const EmbedParams& p, hipStream_t stream) {
  Require(p.rows > 0, "embed: no rows");
  Require(p.hidden_size % 4 == 0 && p.hidden_size <= 4 * 4 * kRowThreads,
          "embed: hidden size must be a multiple of 4 and at most 4096");
  Require(p.codebooks >= 1 && p.codebooks <= 16, "embed: 1 to 16 codebooks");
  if (p.codebooks == 8 && p.hidden_size == 4 * kRowThreads)
    Dispatch(Embed8Kernel, dim3(p.rows), dim3(kRowThreads), 0, stream, true,
             true, p);
  else
    Dispatch(EmbedKernel, dim3(p.rows), dim3(kRowThreads), 0, stream, true,
             true, p);
  Check(hipGetLastError(), "embed launch");
}

void LaunchRmsNorm(const float* x, const int* gather, const float* w,
                   half_t* out, int rows, int width, float eps,
                   hipStream_t stream) {
  Require(rows > 0, "rmsnorm: no rows");
  Require(width % 4 == 0 && width <= 4096,
          "rmsnorm: width must be a multiple of 4 and at most 4096");
  const dim3 grid((rows + kRowThreads / 64 - 1) / (kRowThreads / 64));
  if (width <= 1024)
    Dispatch(RmsNormKernel<4>, grid, dim3(kRowThreads), 0, stream, true, true,
             x, gather, w, out, rows, width, eps);
  else
    Dispatch(RmsNormKernel<16>, grid, dim3(kRowThreads), 0, stream, true,
             true, x, gather, w, out, rows, width, eps);
  Check(hipGetLastError(), "rmsnorm launch");
}

void LaunchAddNorm(const AddNormParams& p, hipStream_t stream) {
  Require(p.rows > 0, "addnorm: no rows");
  Require(p.width % 4 == 0 && p.width <= 1024,
          "addnorm: width must be a multiple of 4 and at most 1024");
  Require(p.splits >= 1 && p.splits <= 8, "addnorm: 1 to 8 partial slices");
  const dim3 grid(p.rows);
  if (p.width == 1024) {
    switch (p.splits) {
      case 1: Dispatch(AddNorm1024Kernel<1>, grid, dim3(64), 0, stream, true, true, p); break;
      case 2: Dispatch(AddNorm1024Kernel<2>, grid, dim3(64), 0, stream, true, true, p); break;
      case 3: Dispatch(AddNorm1024Kernel<3>, grid, dim3(64), 0, stream, true, true, p); break;
      case 4: Dispatch(AddNorm1024Kernel<4>, grid, dim3(64), 0, stream, true, true, p); break;
      case 5: Dispatch(AddNorm1024Kernel<5>, grid, dim3(64), 0, stream, true, true, p); break;
      case 6: Dispatch(AddNorm1024Kernel<6>, grid, dim3(64), 0, stream, true, true, p); break;
      case 7: Dispatch(AddNorm1024Kernel<7>, grid, dim3(64), 0, stream, true, true, p); break;
      default: Dispatch(AddNorm1024Kernel<8>, grid, dim3(64), 0, stream, true, true, p); break;
    }
  } else if (p.splits <= 4)
    Dispatch(AddNormKernel<4, 4>, grid, dim3(64), 0, stream, true, true, p);
  else
    Dispatch(AddNormKernel<4, 8>, grid, dim3(64), 0, stream, true, true, p);
  Check(hipGetLastError(), "addnorm launch");
}

void LaunchAttentionLayout(const half_t* qkv, int ld_qkv, half_t* qk, int ldq,
                           half_t* vt, int ldvt, int rows, int heads, int kv_heads,
                           hipStream_t stream) {
  Require(rows > 0 && ldvt >= rows && ldvt % 16 == 0 &&
              static_cast<int64_t>(ldq) >= static_cast<int64_t>(rows) * 128,
          "attention layout: bad rows");
  Require(ld_qkv >= (heads + 2 * kv_heads) * 128, "attention layout: rows too narrow");
  const dim3 grid((rows + 255) / 256, 128, heads + 2 * kv_heads);
  Dispatch(AttentionLayoutKernel, grid, dim3(256), 0, stream, true, true, qkv,
           ld_qkv, qk, ldq, vt, ldvt, rows, heads, kv_heads);
  Check(hipGetLastError(), "attention layout launch");
}

void LaunchRopeRows(const float2* table, const int* positions, int rows,
                    float2* rows_table, hipStream_t stream) {
  Require(rows > 0, "rotary rows: no rows");
  Dispatch(RopeRowsKernel, dim3((rows * 64 + 255) / 256), dim3(256), 0, stream,
           true, true, table, positions, rows, rows_table);
  Check(hipGetLastError(), "rotary rows launch");
}

void LaunchFill(int* data, int value, int count, hipStream_t stream) {
  if (count <= 0)
    return;
  Dispatch(FillKernel, dim3((count + 255) / 256), dim3(256), 0, stream, true,
           true, data, value, count);
  Check(hipGetLastError(), "fill launch");
}

}  // namespace ovg
