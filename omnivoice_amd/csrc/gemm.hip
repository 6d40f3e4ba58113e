// fp16 x fp16 -> fp32 GEMM on gfx950 matrix cores with the generator's
// epilogues fused (replaces the hipBLASLt calls of the reference's
// HalfGemm::Linear, gemm.cpp:248-262, and the QkNormRope / SwiGlu kernels
// that followed them, kernels/generator_kernels.hip:102-159, 191-200).
//
// Y[m][n] = sum_k X[m][k] W[n][k]: both operands are K-contiguous, so a
// lane's eight consecutive k values are one 16-byte fragment of a
// v_mfma_f32_32x32x16_f16.
//
// One work-group computes a 128 x 128 output tile with 8 waves: two groups
// of four split each 64-wide K step between them (substeps 0-1 and 2-3), and
// inside a group the waves form a 2 x 2 grid of 64 x 64 sub-tiles. Two waves
// per SIMD hide each other's LDS latency, and 64 x 64 wave tiles read 4 KB
// of LDS per 4 MFMAs; gfx950's LDS delivers ~180 B/clk/CU with 8 waves but
// only ~100 with 4, which is what bounded a 4-wave tile.
//
// Operands go global -> LDS by DMA (global_load_lds_dwordx4) through a
// 2- to 4-stage ring of 32 KB stages, no registers involved; LDS rows are
// 128 bytes with an XOR swizzle of the 16-byte chunks.
//
// Epilogue: the two groups' accumulators are summed into an fp32 tile in
// LDS (group 0 + group 1, a fixed order), then all 8 waves walk the tile by
// rows: plain or residual-accumulating fp32 stores; the q/k/v epilogue (a
// Qwen3 head is one 128-column tile: per-head RMSNorm is one wave
// reduction, rotate-half pairs are columns l and l + 64 of lane l, value
// heads are written transposed); or SwiGLU over the interleaved gate/up
// weight tile (columns l and l + 64 are the gate and up of one output).
//
// Split-K (for small M only): work-groups store their reduced tile as a
// partial and a second launch sums the partials in split order 0, 1, ...
// and runs the same epilogue; the kernel boundary publishes the partials to
// every XCD.
//
// Work-groups are dispatched round-robin over the 8 XCDs; the block index is
// remapped so that each XCD receives a contiguous run of tiles, ordered
// M-fastest, so the groups sharing a weight tile share an L2.
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kThreads = 512;
constexpr int kXcds = 8;
constexpr int kABytes = kBM * kBK * 2;  // one stage of A: 16 KB
constexpr int kBBytes = kBN * kBK * 2;
constexpr int kStageBytes = kABytes + kBBytes;
constexpr int kAInstr = kABytes / 1024 / 8;  // 1 KB DMA blocks per wave
constexpr int kBInstr = kBBytes / 1024 / 8;
constexpr int kLoads = kAInstr + kBInstr;  // DMA instructions per stage
constexpr int kPitch = kBN + 4;            // floats per row of the fp32 tile
constexpr int kTileFloats = kBM * kBN;
constexpr int kEpilogueBytes = kBM * kPitch * 4;

template <int STAGES>
constexpr int LdsBytes() {
  return STAGES * kStageBytes > kEpilogueBytes ? STAGES * kStageBytes
                                               : kEpilogueBytes;
}

// LDS address (byte offset in the work-group's LDS) of a __shared__ pointer.
__device__ __forceinline__ uint32_t LdsAddress(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) unsigned char*)(p)));
}

// Operand stages are [rows][64 halves]: 128-byte rows, no padding. The
// 16-byte chunk c of row r sits at position c ^ (r & 7) ^ ((r >> 3) & 1):
// the 32 rows a fragment read touches then fall on distinct banks in both
// 8-lane (128-byte) and 16-lane (256-byte) LDS phases. Its own inverse.
__device__ __forceinline__ int Swizzle(int row, int chunk) {
  return chunk ^ (row & 7) ^ ((row >> 3) & 1);
}

// One wave-wide DMA of 64 x 16 bytes from global memory straight into LDS:
// lane l's 16 bytes land at lds_addr + 16 l. Inline assembly because the
// compiler's wait-count pass cannot tell which stage buffer such a load
// writes and would wait for every load in flight before any LDS read, which
// serialises the ring; the kernel waits explicitly instead.
__device__ __forceinline__ void DmaToLds(const void* src, uint32_t lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off"
      :
      : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(src)
      : "memory", "m0");
}

// Waits until at most N of this wave's vector memory loads are in flight.
template <int N>
__device__ __forceinline__ void WaitLoads() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Barrier without the memory fence __syncthreads() carries (that fence
// would wait for every DMA in flight); the empty asm statements keep the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void StageBarrier() {
  asm volatile("" : : : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" : : : "memory");
}

// ------------------------------------------------------------- epilogues
// All read the summed fp32 tile from LDS ([kBM][kPitch]) with 512 threads.

__device__ __forceinline__ void StoreRows(const GemmParams& p,
                                          const float* tile, int m0, int n0,
                                          bool accumulate) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int r = wave; r < kBM; r += kThreads / 64) {
    const int m = m0 + r;
    if (m >= p.m)
      break;
    const int n = n0 + 2 * lane;
    const float2 v = *reinterpret_cast<const float2*>(tile + r * kPitch + 2 * lane);
    float* dst = p.y + static_cast<size_t>(m) * p.ldc + n;
    if (n + 1 < p.n && (p.ldc & 1) == 0) {
      float2* d2 = reinterpret_cast<float2*>(dst);
      if (accumulate) {
        float2 o = *d2;
        o.x += v.x;
        o.y += v.y;
        *d2 = o;
      } else {
        *d2 = v;
      }
    } else {
      if (n < p.n)
        dst[0] = accumulate ? dst[0] + v.x : v.x;
      if (n + 1 < p.n)
        dst[1] = accumulate ? dst[1] + v.y : v.y;
    }
  }
}

__device__ __forceinline__ void QkvRows(const GemmParams& p, const float* tile,
                                        int m0, int slot) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (slot < p.heads + p.kv_heads) {
    const float* weight = slot < p.heads ? p.q_norm : p.k_norm;
    const float w0 = weight[lane], w1 = weight[lane + 64];
    // The wave's rows are wave + 8 i; fetch their positions (lane i holds
    // row i's) and all rotary entries before the row loop, so the loads'
    // latency is paid once rather than per row.
    constexpr int kRows = kBM / (kThreads / 64);
    const int my_row = min(m0 + wave + 8 * (lane & (kRows - 1)), p.m - 1);
    const int positions = p.positions[my_row];
    float2 cs[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i)
      cs[i] = p.rope[static_cast<size_t>(__shfl(positions, i)) * 64 + lane];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int r = wave + 8 * i;
      const int m = m0 + r;
      if (m >= p.m)
        break;
      const float v0 = tile[r * kPitch + lane];
      const float v1 = tile[r * kPitch + lane + 64];
      const float squares = WaveSumFast(v0 * v0 + v1 * v1);
      const float scale = rsqrtf(squares * (1.0F / 128.0F) + p.eps);
      const float a = w0 * (v0 * scale);
      const float b = w1 * (v1 * scale);
      half_t* out = p.qk + static_cast<size_t>(m) * p.ldq + slot * 128;
      out[lane] = static_cast<half_t>(a * cs[i].x - b * cs[i].y);
      out[lane + 64] = static_cast<half_t>(b * cs[i].x + a * cs[i].y);
    }
    return;
  }
  // Value heads: V^T[g][d][row], four consecutive rows per 8-byte store.
  const int g = slot - p.heads - p.kv_heads;
  const int d = threadIdx.x & 127;
  half_t* out = p.vt + static_cast<size_t>(g * 128 + d) * p.ldvt;
  for (int q = threadIdx.x >> 7; q < kBM / 4; q += kThreads / 128) {
    const int m = m0 + 4 * q;
    if (m >= p.m)
      break;
    const half4 v = {static_cast<half_t>(tile[(4 * q) * kPitch + d]),
                     static_cast<half_t>(tile[(4 * q + 1) * kPitch + d]),
                     static_cast<half_t>(tile[(4 * q + 2) * kPitch + d]),
                     static_cast<half_t>(tile[(4 * q + 3) * kPitch + d])};
    if (m + 3 < p.m) {
      *reinterpret_cast<half4*>(out + m) = v;
    } else {
      for (int e = 0; e < 4 && m + e < p.m; ++e)
        out[m + e] = v[e];
    }
  }
}

__device__ __forceinline__ void SwiGluRows(const GemmParams& p,
                                           const float* tile, int m0,
                                           int tile_n) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int r = wave; r < kBM; r += kThreads / 64) {
    const int m = m0 + r;
    if (m >= p.m)
      break;
    const float g = tile[r * kPitch + lane];
    const float u = tile[r * kPitch + lane + 64];
    p.act[static_cast<size_t>(m) * p.ldh + tile_n * 64 + lane] =
        static_cast<half_t>(g / (1.0F + __expf(-g)) * u);
  }
}

template <Epilogue EPI>
__device__ __forceinline__ void TileEpilogue(const GemmParams& p,
                                             const float* tile, int tile_m,
                                             int tile_n) {
  const int m0 = tile_m * kBM;
  if constexpr (EPI == Epilogue::kStore || EPI == Epilogue::kPartial)
    StoreRows(p, tile, m0, tile_n * kBN, false);
  else if constexpr (EPI == Epilogue::kAccumulate)
    StoreRows(p, tile, m0, tile_n * kBN, true);
  else if constexpr (EPI == Epilogue::kQkvRope)
    QkvRows(p, tile, m0, tile_n);
  else
    SwiGluRows(p, tile, m0, tile_n);
}

// ------------------------------------------------------------- main kernel

template <int STAGES, Epilogue EPI>
__global__ __launch_bounds__(kThreads) void GemmKernel(GemmParams p,
                                                       int tiles_m) {
  extern __shared__ __align__(16) unsigned char lds[];

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

  const int m0 = tile_m * kBM;
  const int n0 = tile_n * kBN;
  const int k_per = p.k / p.splits;
  const int k_begin = split * k_per;
  const int steps = k_per / kBK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int group = wave >> 2;         // K substeps 2 group, 2 group + 1
  const int wave_m = (wave >> 1) & 1;  // 64-row half of the tile
  const int wave_n = wave & 1;         // 64-column half

  // DMA sources: wave w fills 1 KB blocks w * kAInstr + i of A (8 rows each)
  // and of B; lane l brings row 8 b + l / 8 at LDS position l % 8, i.e.
  // chunk Swizzle(row, l % 8). Rows past M or N read the last valid row
  // (their results are never stored).
  const half_t* a_src[kAInstr];
  const half_t* b_src[kBInstr];
#pragma unroll
  for (int i = 0; i < kAInstr; ++i) {
    const int row = (wave * kAInstr + i) * 8 + (lane >> 3);
    a_src[i] = p.x + static_cast<size_t>(min(m0 + row, p.m - 1)) * p.lda +
               k_begin + Swizzle(row, lane & 7) * 8;
  }
#pragma unroll
  for (int i = 0; i < kBInstr; ++i) {
    const int row = (wave * kBInstr + i) * 8 + (lane >> 3);
    b_src[i] = p.w + static_cast<size_t>(min(n0 + row, p.n - 1)) * p.ldb +
               k_begin + Swizzle(row, lane & 7) * 8;
  }
  const uint32_t lds_base = LdsAddress(lds);
  auto issue = [&](int stage, int kt) {
    const uint32_t base = lds_base + stage * kStageBytes;
    const int kk = kt * kBK;
#pragma unroll
    for (int i = 0; i < kAInstr; ++i)
      DmaToLds(a_src[i] + kk, base + (wave * kAInstr + i) * 1024);
#pragma unroll
    for (int i = 0; i < kBInstr; ++i)
      DmaToLds(b_src[i] + kk, base + kABytes + (wave * kBInstr + i) * 1024);
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int fm = 0; fm < 2; ++fm)
#pragma unroll
    for (int fn = 0; fn < 2; ++fn)
      acc[fm][fn] = floatx16{};

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < steps)
      issue(s, s);
  for (int kt = 0; kt < steps; ++kt) {
    // Stage kt has landed once at most `ahead` later stages are in flight.
    const int ahead = min(STAGES - 2, steps - 1 - kt);
    if (ahead >= 2)
      WaitLoads<2 * kLoads>();
    else if (ahead == 1)
      WaitLoads<kLoads>();
    else
      WaitLoads<0>();
    StageBarrier();
    // Every wave is past its reads of stage kt - 1: refill that buffer.
    if (kt + STAGES - 1 < steps)
      issue((kt + STAGES - 1) % STAGES, kt + STAGES - 1);
    const unsigned char* as = lds + (kt % STAGES) * kStageBytes;
    const unsigned char* bs = as + kABytes;
    half8 a[2][2], b[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int chunk = 2 * (2 * group + j) + (lane >> 5);
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int ra = wave_m * 64 + f * 32 + (lane & 31);
        a[j][f] = *reinterpret_cast<const half8*>(as + ra * 128 +
                                                  Swizzle(ra, chunk) * 16);
        const int rb = wave_n * 64 + f * 32 + (lane & 31);
        b[j][f] = *reinterpret_cast<const half8*>(bs + rb * 128 +
                                                  Swizzle(rb, chunk) * 16);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int fm = 0; fm < 2; ++fm)
#pragma unroll
        for (int fn = 0; fn < 2; ++fn)
          acc[fm][fn] = Mfma32(a[j][fm], b[j][fn], acc[fm][fn]);
  }

  // Sum the groups into the fp32 tile: group 1 stores, group 0 adds its own
  // accumulators to what group 1 left (group 0 + group 1).
  __syncthreads();
  float* tile_lds = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int phase = 1; phase >= 0; --phase) {
    if (group == phase) {
#pragma unroll
      for (int fm = 0; fm < 2; ++fm)
#pragma unroll
        for (int fn = 0; fn < 2; ++fn)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = wave_m * 64 + fm * 32 + 8 * (r / 4) +
                            4 * (lane >> 5) + (r & 3);
            const int col = wave_n * 64 + fn * 32 + (lane & 31);
            float* cell = tile_lds + row * kPitch + col;
            *cell = phase == 1 ? acc[fm][fn][r] : acc[fm][fn][r] + *cell;
          }
    }
    __syncthreads();
  }

  if constexpr (EPI == Epilogue::kPartial) {
    // Each split owns a full [M][ldc] slice; the row kernel that consumes
    // the GEMM adds the slices.
    GemmParams q = p;
    q.y = p.y + static_cast<size_t>(split) * p.split_stride;
    TileEpilogue<EPI>(q, tile_lds, tile_m, tile_n);
    return;
  }
  if (p.splits > 1) {
    float* mine = p.partials +
                  (static_cast<size_t>(tile) * p.splits + split) * kTileFloats;
    for (int f = tid; f < kTileFloats / 4; f += kThreads) {
      const int row = f >> 5, c4 = (f & 31) * 4;
      *reinterpret_cast<floatx4*>(mine + row * kBN + c4) =
          *reinterpret_cast<const floatx4*>(tile_lds + row * kPitch + c4);
    }
    return;
  }
  TileEpilogue<EPI>(p, tile_lds, tile_m, tile_n);
}

// Sums a tile's split-K partials in split order 0, 1, ... (a fixed order,
// reproducible bit for bit) into the LDS tile and applies the epilogue.
template <Epilogue EPI>
__global__ __launch_bounds__(kThreads) void SplitReduceKernel(GemmParams p,
                                                              int tiles_m) {
  extern __shared__ __align__(16) unsigned char lds[];
  float* tile_lds = reinterpret_cast<float*>(lds);
  const int tile = blockIdx.x;
  const float* base =
      p.partials + static_cast<size_t>(tile) * p.splits * kTileFloats;
  for (int f = threadIdx.x; f < kTileFloats / 4; f += kThreads) {
    const int row = f >> 5, c4 = (f & 31) * 4;
    floatx4 sum = *reinterpret_cast<const floatx4*>(base + row * kBN + c4);
    for (int s = 1; s < p.splits; ++s)
      sum += *reinterpret_cast<const floatx4*>(
          base + static_cast<size_t>(s) * kTileFloats + row * kBN + c4);
    *reinterpret_cast<floatx4*>(tile_lds + row * kPitch + c4) = sum;
  }
  __syncthreads();
  TileEpilogue<EPI>(p, tile_lds, tile % tiles_m, tile / tiles_m);
}

template <int STAGES, Epilogue EPI>
void Launch(const GemmParams& p, int tiles_m, int groups, hipStream_t stream) {
  GemmKernel<STAGES, EPI>
      <<<dim3(groups), dim3(kThreads), LdsBytes<STAGES>(), stream>>>(p, tiles_m);
  if (p.splits > 1 && EPI != Epilogue::kPartial)
    SplitReduceKernel<EPI><<<dim3(groups / p.splits), dim3(kThreads),
                             kEpilogueBytes, stream>>>(p, tiles_m);
}

template <Epilogue EPI>
void LaunchEpi(const GemmParams& p, const GemmPlan& plan, hipStream_t stream) {
  const int tiles_m = (p.m + kBM - 1) / kBM;
  const int groups = plan.tiles * plan.splits;
  if (plan.stages == 2)
    Launch<2, EPI>(p, tiles_m, groups, stream);
  else if (plan.stages == 4)
    Launch<4, EPI>(p, tiles_m, groups, stream);
  else
    Launch<3, EPI>(p, tiles_m, groups, stream);
}

}  // namespace

GemmPlan PlanGemm(int m, int n, int k, Epilogue epilogue) {
  GemmPlan plan;
  const int tiles_m = (m + kBM - 1) / kBM;
  const int tiles_n = (n + kBN - 1) / kBN;
  plan.tiles = tiles_m * tiles_n;
  plan.stages = 3;
  const int k_steps = k / kBK;
  int splits = 1;
  if (epilogue == Epilogue::kPartial) {
    // Split slices are summed by the row kernel that reads the output
    // anyway: split until the grid covers most CUs, keeping >= 8 K steps
    // per split for the DMA ring to overlap.
    for (const int s : {2, 3, 4, 6, 8}) {
      if (plan.tiles * splits >= 160)
        break;
      if (k_steps % s == 0 && k_steps / s >= 8)
        splits = s;
    }
    plan.splits = splits;
    plan.partial_floats = 0;
    return plan;
  }
  // Otherwise split K only when the tiles leave most CUs idle; partials
  // cost a round trip through memory and a second launch.
  if (plan.tiles < 64) {
    for (const int s : {2, 3, 4, 6, 8}) {
      if (plan.tiles * splits >= 128)
        break;
      if (k_steps % s == 0 && k_steps / s >= 4)
        splits = s;
    }
  }
  plan.splits = splits;
  plan.partial_floats =
      splits > 1 ? static_cast<std::size_t>(plan.tiles) * splits * kTileFloats
                 : 0;
  return plan;
}

void LaunchGemm(const GemmParams& p, const GemmPlan& plan, Epilogue epilogue,
                hipStream_t stream) {
  Require(p.m > 0 && p.n > 0 && p.k > 0, "gemm: empty shape");
  Require(p.k % kBK == 0, "gemm: K must be a multiple of 64");
  Require(plan.splits >= 1 && (p.k / kBK) % plan.splits == 0,
          "gemm: K steps not divisible by the split count");
  Require(plan.stages >= 2 && plan.stages <= 4, "gemm: 2 to 4 stages");
  Require(plan.tiles == ((p.m + kBM - 1) / kBM) * ((p.n + kBN - 1) / kBN),
          "gemm: plan does not match the shape");
  Require(p.lda % 8 == 0 && p.ldb % 8 == 0,
          "gemm: leading dimensions must be multiples of 8");
  Require(plan.splits == 1 || epilogue == Epilogue::kPartial ||
              p.partials != nullptr,
          "gemm: split-K needs a partials buffer");
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
      Require(p.ldvt % 4 == 0, "gemm: V^T rows must be 8-byte aligned");
      LaunchEpi<Epilogue::kQkvRope>(p, plan, stream);
      break;
    case Epilogue::kSwiGlu:
      Require(p.n % 128 == 0, "gemm: SwiGLU epilogue needs N % 128 == 0");
      LaunchEpi<Epilogue::kSwiGlu>(p, plan, stream);
      break;
    case Epilogue::kPartial:
      Require(p.y != nullptr &&
                  p.split_stride >= static_cast<std::size_t>(p.m) * p.ldc,
              "gemm: partial slices overlap");
      LaunchEpi<Epilogue::kPartial>(p, plan, stream);
      break;
  }
  Check(hipGetLastError(), "gemm launch");
}

}  // namespace ovg
