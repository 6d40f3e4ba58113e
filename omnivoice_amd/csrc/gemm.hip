// fp16 x fp16 -> fp32 GEMM on gfx950 matrix cores with the generator's
// epilogues fused (replaces the hipBLASLt calls of the reference's
// HalfGemm::Linear, gemm.cpp:248-262, and the QkNormRope / SwiGlu kernels
// that followed them, kernels/generator_kernels.hip:102-159, 191-200).
//
// Y[m][n] = sum_k X[m][k] W[n][k]: both operands are K-contiguous, so a
// lane's eight consecutive k values are one 16-byte load, exactly the
// operand a v_mfma_f32_32x32x16_f16 lane supplies.
//
// Tile: BM = 128 * FM rows x BN = 128 columns x BK = 64, 256 threads as 4
// waves stacked along M; each wave owns FM x 4 accumulators of 32 x 32, so a
// wave holds complete 128-column rows. That is what lets the epilogues work
// in registers: a Qwen3 head is one 128-column tile (per-head RMSNorm is a
// 32-lane butterfly, and rotate-half pairs i, i + 64 sit in the same lane in
// accumulators fn and fn + 2), and the SwiGLU gate/up pair of a column sits
// in accumulators fn and fn + 2 of the interleaved weight tile.
//
// Operands are staged global -> registers -> LDS (row pitch BK + 8 halves,
// so the 16-byte fragment reads of 32 consecutive rows hit distinct banks),
// double-buffered with one barrier per K step.
//
// Split-K: when the output tiles alone cannot fill the 256 CUs, the K range
// is split; each work-group stores its partial tile in accumulator order and
// bumps the tile's counter, and the last one to arrive adds the partials in
// split order 0, 1, ... (a fixed order, whichever group arrives last), runs
// the epilogue and resets the counter to zero for the next launch.
//
// Work-groups are dispatched round-robin over the 8 XCDs; the block index is
// remapped so that each XCD receives a contiguous run of tiles, and tiles
// are ordered M-fastest, so the groups sharing a weight tile share an L2.
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // halves per LDS row
constexpr int kThreads = 256;
constexpr int kXcds = 8;

template <int FM>
struct Tile {
  static constexpr int kBM = 128 * FM;
  static constexpr int kAChunks = kBM * kBK / 8 / kThreads;  // 16-B chunks
  static constexpr int kBChunks = kBN * kBK / 8 / kThreads;
  static constexpr int kStageHalves = (kBM + kBN) * kPitch;
  static constexpr int kLdsBytes = 2 * kStageHalves * 2;
  static constexpr int kTileFloats = kBM * kBN;
};

__device__ __forceinline__ half8 LoadChunk(const half_t* p, bool valid) {
  if (!valid)
    return half8{0, 0, 0, 0, 0, 0, 0, 0};
  return *reinterpret_cast<const half8*>(p);
}

template <int FM>
__device__ __forceinline__ void Epilogue32(const GemmParams& p,
                                           floatx16 (&acc)[FM][4], int m0,
                                           int n0, bool accumulate) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wave * FM * 32 + fm * 32 + 8 * (r / 4) +
                    4 * (lane >> 5) + (r & 3);
      if (m >= p.m)
        continue;
      float* row = p.y + static_cast<size_t>(m) * p.ldc;
#pragma unroll
      for (int fn = 0; fn < 4; ++fn) {
        const int n = n0 + fn * 32 + (lane & 31);
        if (n < p.n) {
          if (accumulate)
            row[n] += acc[fm][fn][r];
          else
            row[n] = acc[fm][fn][r];
        }
      }
    }
  }
}

template <int FM>
__device__ __forceinline__ void EpilogueQkv(const GemmParams& p,
                                            floatx16 (&acc)[FM][4], int m0,
                                            int slot) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 31;
  if (slot < p.heads + p.kv_heads) {
    const float* weight = slot < p.heads ? p.q_norm : p.k_norm;
    const float w0 = weight[col], w1 = weight[col + 32];
    const float w2 = weight[col + 64], w3 = weight[col + 96];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v0 = acc[fm][0][r], v1 = acc[fm][1][r];
        const float v2 = acc[fm][2][r], v3 = acc[fm][3][r];
        float squares = v0 * v0 + v1 * v1 + v2 * v2 + v3 * v3;
#pragma unroll
        for (int offset = 16; offset > 0; offset /= 2)
          squares += __shfl_xor(squares, offset);
        const int m = m0 + wave * FM * 32 + fm * 32 + 8 * (r / 4) +
                      4 * (lane >> 5) + (r & 3);
        if (m >= p.m)
          continue;
        const float scale = rsqrtf(squares * (1.0F / 128.0F) + p.eps);
        const float2* rope = p.rope + static_cast<size_t>(p.positions[m]) * 64;
        const float2 cs0 = rope[col], cs1 = rope[col + 32];
        const float a0 = w0 * (v0 * scale), b0 = w2 * (v2 * scale);
        const float a1 = w1 * (v1 * scale), b1 = w3 * (v3 * scale);
        half_t* out = p.qk + static_cast<size_t>(m) * p.ldq + slot * 128;
        out[col] = static_cast<half_t>(a0 * cs0.x - b0 * cs0.y);
        out[col + 64] = static_cast<half_t>(b0 * cs0.x + a0 * cs0.y);
        out[col + 32] = static_cast<half_t>(a1 * cs1.x - b1 * cs1.y);
        out[col + 96] = static_cast<half_t>(b1 * cs1.x + a1 * cs1.y);
      }
    }
    return;
  }
  // Value heads: V^T[g][d][row], four consecutive rows per 8-byte store.
  const int g = slot - p.heads - p.kv_heads;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = m0 + wave * FM * 32 + fm * 32 + 8 * q + 4 * (lane >> 5);
      if (m >= p.m)
        continue;
#pragma unroll
      for (int fn = 0; fn < 4; ++fn) {
        const int d = fn * 32 + col;
        half_t* out = p.vt + static_cast<size_t>(g * 128 + d) * p.ldvt + m;
        const half4 v = {static_cast<half_t>(acc[fm][fn][4 * q]),
                         static_cast<half_t>(acc[fm][fn][4 * q + 1]),
                         static_cast<half_t>(acc[fm][fn][4 * q + 2]),
                         static_cast<half_t>(acc[fm][fn][4 * q + 3])};
        if (m + 3 < p.m) {
          *reinterpret_cast<half4*>(out) = v;
        } else {
          for (int e = 0; e < 4 && m + e < p.m; ++e)
            out[e] = v[e];
        }
      }
    }
  }
}

template <int FM>
__device__ __forceinline__ void EpilogueSwiGlu(const GemmParams& p,
                                               floatx16 (&acc)[FM][4], int m0,
                                               int tile_n) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 31;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wave * FM * 32 + fm * 32 + 8 * (r / 4) +
                    4 * (lane >> 5) + (r & 3);
      if (m >= p.m)
        continue;
      half_t* out = p.act + static_cast<size_t>(m) * p.ldh + tile_n * 64;
#pragma unroll
      for (int fn = 0; fn < 2; ++fn) {
        const float g = acc[fm][fn][r];
        const float u = acc[fm][fn + 2][r];
        out[fn * 32 + col] = static_cast<half_t>(g / (1.0F + __expf(-g)) * u);
      }
    }
  }
}

template <int FM, Epilogue EPI>
__global__ __launch_bounds__(kThreads) void GemmKernel(GemmParams p,
                                                       int tiles_m) {
  using T = Tile<FM>;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  half_t* lds = reinterpret_cast<half_t*>(lds_raw);
  __shared__ int last_flag;

  // XCD-aware remap of the dispatch order, then M-fastest tile order.
  const int groups = gridDim.x;
  const int pid = blockIdx.x;
  const int xcd = pid % kXcds;
  const int per = groups / kXcds;
  const int extra = groups % kXcds;
  const int logical = xcd * per + min(xcd, extra) + pid / kXcds;
  const int tile_m = logical % tiles_m;
  const int rest = logical / tiles_m;
  const int split = rest % p.splits;
  const int tile_n = rest / p.splits;
  const int tile = tile_n * tiles_m + tile_m;

  const int m0 = tile_m * T::kBM;
  const int n0 = tile_n * kBN;
  const int k_per = p.k / p.splits;
  const int k_begin = split * k_per;
  const int steps = k_per / kBK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  half8 ra[T::kAChunks], rb[T::kBChunks];
  auto load = [&](int kt) {
    const int kk = k_begin + kt * kBK;
#pragma unroll
    for (int i = 0; i < T::kAChunks; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3, c8 = (c & 7) * 8;
      ra[i] = LoadChunk(p.x + static_cast<size_t>(m0 + row) * p.lda + kk + c8,
                        m0 + row < p.m);
    }
#pragma unroll
    for (int i = 0; i < T::kBChunks; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3, c8 = (c & 7) * 8;
      rb[i] = LoadChunk(p.w + static_cast<size_t>(n0 + row) * p.ldb + kk + c8,
                        n0 + row < p.n);
    }
  };
  auto store = [&](int buffer) {
    half_t* as = lds + buffer * T::kStageHalves;
    half_t* bs = as + T::kBM * kPitch;
#pragma unroll
    for (int i = 0; i < T::kAChunks; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<half8*>(as + (c >> 3) * kPitch + (c & 7) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < T::kBChunks; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<half8*>(bs + (c >> 3) * kPitch + (c & 7) * 8) = rb[i];
    }
  };

  floatx16 acc[FM][4];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn)
      acc[fm][fn] = floatx16{};

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < steps; ++kt) {
    const int buffer = kt & 1;
    if (kt + 1 < steps)
      load(kt + 1);
    const half_t* as = lds + buffer * T::kStageHalves;
    const half_t* bs = as + T::kBM * kPitch;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int k_off = ks * 16 + (lane >> 5) * 8;
      half8 a[FM], b[4];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        a[fm] = *reinterpret_cast<const half8*>(
            as + (wave * FM * 32 + fm * 32 + (lane & 31)) * kPitch + k_off);
#pragma unroll
      for (int fn = 0; fn < 4; ++fn)
        b[fn] = *reinterpret_cast<const half8*>(
            bs + (fn * 32 + (lane & 31)) * kPitch + k_off);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < 4; ++fn)
          acc[fm][fn] = Mfma32(a[fm], b[fn], acc[fm][fn]);
    }
    if (kt + 1 < steps)
      store(buffer ^ 1);
    __syncthreads();
  }

  if (p.splits > 1) {
    // Partial tile in accumulator order: float4 q of accumulator (fm, fn)
    // of lane l at ((((wave * FM + fm) * 4 + fn) * 4 + q) * 64 + l) * 4.
    float* mine = p.partials + (static_cast<size_t>(tile) * p.splits + split) *
                                   T::kTileFloats;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < 4; ++fn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const floatx4 v = {acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1],
                             acc[fm][fn][4 * q + 2], acc[fm][fn][4 * q + 3]};
          *reinterpret_cast<floatx4*>(
              mine + ((((wave * FM + fm) * 4 + fn) * 4 + q) * 64 + lane) * 4) = v;
        }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const int arrived = atomicAdd(p.counters + tile, 1);
      last_flag = arrived == p.splits - 1;
    }
    __syncthreads();
    if (!last_flag)
      return;
    __threadfence();
    const float* base =
        p.partials + static_cast<size_t>(tile) * p.splits * T::kTileFloats;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < 4; ++fn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const size_t off =
              ((((wave * FM + fm) * 4 + fn) * 4 + q) * 64 + lane) * 4;
          floatx4 sum = {acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1],
                         acc[fm][fn][4 * q + 2], acc[fm][fn][4 * q + 3]};
          if (split != 0)
            sum = *reinterpret_cast<const floatx4*>(base + off);
          for (int s = 1; s < p.splits; ++s) {
            floatx4 v;
            if (s == split)
              v = floatx4{acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1],
                          acc[fm][fn][4 * q + 2], acc[fm][fn][4 * q + 3]};
            else
              v = *reinterpret_cast<const floatx4*>(
                  base + static_cast<size_t>(s) * T::kTileFloats + off);
            sum += v;
          }
          acc[fm][fn][4 * q] = sum[0];
          acc[fm][fn][4 * q + 1] = sum[1];
          acc[fm][fn][4 * q + 2] = sum[2];
          acc[fm][fn][4 * q + 3] = sum[3];
        }
    if (tid == 0)
      p.counters[tile] = 0;
  }

  if constexpr (EPI == Epilogue::kStore)
    Epilogue32<FM>(p, acc, m0, n0, false);
  else if constexpr (EPI == Epilogue::kAccumulate)
    Epilogue32<FM>(p, acc, m0, n0, true);
  else if constexpr (EPI == Epilogue::kQkvRope)
    EpilogueQkv<FM>(p, acc, m0, tile_n);
  else
    EpilogueSwiGlu<FM>(p, acc, m0, tile_n);
}

template <int FM, Epilogue EPI>
void Launch(const GemmParams& p, int tiles_m, int groups,
            hipStream_t stream) {
  hipLaunchKernelGGL((GemmKernel<FM, EPI>), dim3(groups), dim3(kThreads),
                     Tile<FM>::kLdsBytes, stream, p, tiles_m);
}

template <Epilogue EPI>
void LaunchEpi(const GemmParams& p, const GemmPlan& plan, hipStream_t stream) {
  const int tiles_m = (p.m + plan.block_m - 1) / plan.block_m;
  const int groups = plan.tiles * plan.splits;
  if (plan.block_m == 256)
    Launch<2, EPI>(p, tiles_m, groups, stream);
  else
    Launch<1, EPI>(p, tiles_m, groups, stream);
}

}  // namespace

GemmPlan PlanGemm(int m, int n, int k, Epilogue epilogue) {
  (void)epilogue;
  GemmPlan plan;
  plan.block_m = 128;
  const int tiles_m = (m + plan.block_m - 1) / plan.block_m;
  const int tiles_n = (n + kBN - 1) / kBN;
  plan.tiles = tiles_m * tiles_n;
  const int k_steps = k / kBK;
  // Split K until the grid covers the 256 CUs, keeping >= 2 K steps per
  // split so the double buffer has something to overlap.
  int splits = 1;
  for (const int s : {2, 3, 4, 6, 8, 12, 16}) {
    if (plan.tiles * splits >= 256)
      break;
    if (k_steps % s == 0 && k_steps / s >= 2)
      splits = s;
  }
  plan.splits = splits;
  plan.partial_floats =
      splits > 1 ? static_cast<std::size_t>(plan.tiles) * splits *
                       plan.block_m * kBN
                 : 0;
  return plan;
}

void LaunchGemm(const GemmParams& p, const GemmPlan& plan, Epilogue epilogue,
                hipStream_t stream) {
  Require(p.m > 0 && p.n > 0 && p.k > 0, "gemm: empty shape");
  Require(p.k % kBK == 0, "gemm: K must be a multiple of 64");
  Require(plan.splits >= 1 && (p.k / kBK) % plan.splits == 0,
          "gemm: K steps not divisible by the split count");
  Require(p.lda % 8 == 0 && p.ldb % 8 == 0, "gemm: leading dimensions must be multiples of 8");
  Require(plan.splits == 1 || (p.partials != nullptr && p.counters != nullptr),
          "gemm: split-K needs partials and counters");
  Require(p.splits == plan.splits, "gemm: params and plan disagree on splits");
  switch (epilogue) {
    case Epilogue::kStore:
      LaunchEpi<Epilogue::kStore>(p, plan, stream);
      break;
    case Epilogue::kAccumulate:
      LaunchEpi<Epilogue::kAccumulate>(p, plan, stream);
      break;
    case Epilogue::kQkvRope:
      Require(p.n == (p.heads + 2 * p.kv_heads) * 128,
              "gemm: q/k/v epilogue needs N = (heads + 2 kv_heads) * 128");
      LaunchEpi<Epilogue::kQkvRope>(p, plan, stream);
      break;
    case Epilogue::kSwiGlu:
      Require(p.n % 128 == 0, "gemm: SwiGLU epilogue needs N % 128 == 0");
      LaunchEpi<Epilogue::kSwiGlu>(p, plan, stream);
      break;
  }
  Check(hipGetLastError(), "gemm launch");
}

}  // namespace ovg
