// fp16 x fp16 -> fp32 GEMM on gfx950 matrix cores over unpacked row-major
// weights: the stand-alone linear operator (ovg_op_linear and its
// allocation-free variant), the reference's HalfGemm::Linear (gemm.cpp:
// 248-262). The generator's own projections, with their fused q/k/v and
// SwiGLU epilogues, run on weights packed at load (packed_gemm.hip).
//
// Y[m][n] = sum_k X[m][k] W[n][k]: both operands are K-contiguous, so a
// lane's eight consecutive k values are one 16-byte fragment of a
// v_mfma_f32_32x32x16_f16.
//
// One work-group computes a 128 x 128 output tile with 8 waves: two groups
// of four split each 64-wide K step between them (substeps 0-1 and 2-3), and
// inside a group wave w owns the 32 x 128 strip of rows 32 w .. 32 w + 31.
// A strip spans a whole 128-column tile, so one Qwen3 head (or one gate/up
// block) lives in one wave and every epilogue works from registers. Two
// waves per SIMD hide each other's LDS latency.
//
// Operands go global -> LDS by DMA (global_load_lds_dwordx4) through a
// 2- to 4-stage ring of 32 KB stages, no registers involved; LDS rows are
// 128 bytes with an XOR swizzle of the 16-byte chunks. Fragments of step
// k + 1 are read from LDS while step k's MFMAs run.
//
// Epilogue: the two groups swap halves of their accumulators through LDS
// (16-byte per lane, conflict-free) so that each wave ends up owning 16 rows
// x 128 columns of the summed tile (group 0 + group 1; fp32 addition of two
// terms is commutative, so both owners round identically), and writes them
// straight from registers: plain or residual-accumulating fp32 stores.
//
// Split-K: with the kPartial epilogue every split stores its own fp32 slice
// and the row kernel that consumes the output sums the slices; the split
// count depends on K only. Otherwise (stand-alone calls at small M only)
// each split stores its owned values as a partial and a second launch sums
// the partials in split order 0, 1, ... and runs the same epilogue; the
// kernel boundary publishes the partials to every XCD.
//
// Work-groups are dispatched round-robin over the 8 XCDs; the block index is
// remapped so that each XCD receives a contiguous run of tiles, ordered
// M-fastest, so the groups sharing a weight tile share an L2.
#include "kernels.hpp"

// No floating-point contraction in this file: every fused multiply-add in
// the epilogues is written out, so that each tile shape (each template
// instantiation) rounds a row's values identically and a row's result does
// not depend on the tile height the packed row count selects.
#pragma clang fp contract(off)

namespace ovg {
namespace {

constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kBBytes = kBN * kBK * 2;  // one stage of B: 16 KB

// FM = 32-row MFMA blocks per wave strip. Eight waves in two K groups of
// four strips: 128 x 128 tiles of 32-row strips (FM 1), or 256 x 128 tiles
// of 64-row strips (FM 2: a wave's A fragment serves twice the MFMAs, so
// the tile needs 36 % less LDS traffic and 25 % less fill per MFMA; for
// row counts that still give every CU a tile).
//
// STRIPS = strips per K group: four (eight waves), or one (two waves:
// 32 x 128 tiles, for row counts whose 128-row tiles leave most CUs idle).
template <int FM, int STRIPS = 4>
struct Shape {
  static constexpr int kBM = 32 * FM * STRIPS;
  static constexpr int kWaves = 2 * STRIPS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kStrips = STRIPS;
  static constexpr int kOwned = 8 * FM;  // owned elements per column block
  static constexpr int kABytes = kBM * kBK * 2;
  static constexpr int kStageBytes = kABytes + kBBytes;
  // DMA instructions (1 KB each) per wave per stage, for A and for B.
  static constexpr int kAInstr = kABytes / 1024 / kWaves;
  static constexpr int kBInstr = kBBytes / 1024 / kWaves;
  static constexpr int kLoads = kAInstr + kBInstr;
  // The accumulator swap: every wave hands over kOwned / 4 x 4 float4 per
  // lane.
  static constexpr int kSwapBytes = kThreads * kOwned * 4 * 4;
  static constexpr int kTileFloats = kBM * kBN;
};

template <int STAGES, int FM, int STRIPS = 4>
constexpr int LdsBytes() {
  using S = Shape<FM, STRIPS>;
  return STAGES * S::kStageBytes > S::kSwapBytes ? STAGES * S::kStageBytes : S::kSwapBytes;
}
static_assert(LdsBytes<3, 2>() <= 160 * 1024, "LDS budget");

// Operand stages are [rows][64 halves]: 128-byte rows, no padding. The
// 16-byte chunk c of row r sits at position c ^ (r & 7) ^ ((r >> 3) & 1):
// the 32 rows a fragment read touches then fall on distinct banks in both
// 8-lane (128-byte) and 16-lane (256-byte) LDS phases. Its own inverse.
__device__ __forceinline__ int Swizzle(int row, int chunk) {
  return chunk ^ (row & 7) ^ ((row >> 3) & 1);
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
// A wave's owned values: v[c][e] is column 32 c + (lane & 31) of row
// row0 + RowOf(e), e < 8 FM, where row0 = m0 + 32 FM strip + 16 FM group.
template <int FM>
struct Owned {
  float v[4][8 * FM];
};

__device__ __forceinline__ int RowOf(int e, int lane) {
  return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}

// Partial slices are stored write-through (their lines would otherwise keep
// the kernel alive at its end while L2 writes them back; the row kernel that
// sums them reads them from memory either way). Final outputs are stored
// plainly: write-through made their consumers slower than it made the
// producer faster.
template <int FM, bool THROUGH>
__device__ __forceinline__ void StoreOwned(const GemmParams& p,
                                           const Owned<FM>& o, float* y,
                                           int row0, int n0, bool accumulate) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int n = n0 + 32 * c + (lane & 31);
    if (n >= p.n)
      continue;
#pragma unroll
    for (int e = 0; e < 8 * FM; ++e) {
      const int m = row0 + RowOf(e, lane);
      if (m < p.m) {
        float* dst = y + static_cast<size_t>(m) * p.ldc + n;
        const float v = accumulate ? *dst + o.v[c][e] : o.v[c][e];
        if constexpr (THROUGH)
          StoreThrough(dst, v);
        else
          *dst = v;
      }
    }
  }
}

template <Epilogue EPI, int FM>
__device__ __forceinline__ void OwnedEpilogue(const GemmParams& p,
                                              const Owned<FM>& o, int row0,
                                              int tile_n) {
  if constexpr (EPI == Epilogue::kStore)
    StoreOwned<FM, false>(p, o, p.y, row0, tile_n * kBN, false);
  else if constexpr (EPI == Epilogue::kAccumulate)
    StoreOwned<FM, false>(p, o, p.y, row0, tile_n * kBN, true);
}

// ------------------------------------------------------------- main kernel

template <int STAGES, Epilogue EPI, int FM, int STRIPS>
__global__ __launch_bounds__(128 * STRIPS) void GemmKernel(
    GemmParams p, int tiles_m, int band) {
  using S = Shape<FM, STRIPS>;
  extern __shared__ __align__(16) unsigned char lds[];

  // XCD-aware remap of the dispatch order, then M-fastest tile order.
  const int groups = gridDim.x;
  const int pid = blockIdx.x;
  const int xcd = pid % kXcds;
  const int per = groups / kXcds;
  const int extra = groups % kXcds;
  const int logical = xcd * per + min(xcd, extra) + pid / kXcds;
  int tile_m, tile_n, split;
  if (band <= 0 || band >= tiles_m || p.splits > 1) {
    tile_m = logical % tiles_m;
    const int rest = logical / tiles_m;
    split = rest % p.splits;
    tile_n = rest / p.splits;
  } else {
    // Bands of `band` row tiles (the last one shorter), column by column
    // inside a band, rows fastest (no split-K here).
    const int tiles_n = groups / tiles_m;
    const int full = tiles_m / band;
    const int head = full * band * tiles_n;
    split = 0;
    if (logical < head) {
      const int within = logical % (band * tiles_n);
      tile_n = within / band;
      tile_m = logical / (band * tiles_n) * band + within % band;
    } else {
      const int rows = tiles_m - full * band;
      const int within = logical - head;
      tile_n = within / rows;
      tile_m = full * band + within % rows;
    }
  }
  const int tile = tile_n * tiles_m + tile_m;

  const int m0 = tile_m * S::kBM;
  const int n0 = tile_n * kBN;
  const int k_per = p.k / p.splits;
  const int k_begin = split * k_per;
  const int steps = k_per / kBK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform, so that everything derived from it stays scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave / S::kStrips;  // K substeps 2 group, 2 group + 1
  const int strip = wave % S::kStrips;  // rows 32 FM strip .. + 32 FM - 1

  // DMA sources: wave w fills 1 KB blocks w * kAInstr + i of A (8 rows each)
  // and of B; lane l brings row 8 b + l / 8 at LDS position l % 8, i.e.
  // chunk Swizzle(row, l % 8). Rows past M or N read the last valid row
  // (their results are never stored).
  uint32_t a_src[S::kAInstr], b_src[S::kBInstr];  // byte offsets from bases
#pragma unroll
  for (int i = 0; i < S::kAInstr; ++i) {
    const int row = (wave * S::kAInstr + i) * 8 + (lane >> 3);
    a_src[i] = static_cast<uint32_t>(min(m0 + row, p.m - 1)) * p.lda * 2 +
               Swizzle(row, lane & 7) * 16;
  }
#pragma unroll
  for (int i = 0; i < S::kBInstr; ++i) {
    const int row = (wave * S::kBInstr + i) * 8 + (lane >> 3);
    b_src[i] = static_cast<uint32_t>(min(n0 + row, p.n - 1)) * p.ldb * 2 +
               Swizzle(row, lane & 7) * 16;
  }
  const unsigned char* a_base =
      reinterpret_cast<const unsigned char*>(p.x) + k_begin * 2;
  const unsigned char* b_base =
      reinterpret_cast<const unsigned char*>(p.w) + k_begin * 2;
  const uint32_t lds_base = LdsAddress(lds);
  auto issue = [&](int stage, int kt) {
    const uint32_t base = lds_base + stage * S::kStageBytes;
    const int kk = kt * kBK * 2;
#pragma unroll
    for (int i = 0; i < S::kAInstr; ++i)
      DmaToLds(a_base + kk, a_src[i], base + (wave * S::kAInstr + i) * 1024);
#pragma unroll
    for (int i = 0; i < S::kBInstr; ++i)
      DmaToLds(b_base + kk, b_src[i],
               base + S::kABytes + (wave * S::kBInstr + i) * 1024);
  };

  floatx16 acc[FM][4];
#pragma unroll
  for (int f = 0; f < FM; ++f)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      acc[f][c] = floatx16{};

  // Byte offsets of this lane's fragments inside a stage (stage-invariant):
  // A rows of the wave's strip, B rows 32 c + (lane & 31) for column block c.
  int a_off[2][FM], b_off[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int chunk = 2 * (2 * group + j) + (lane >> 5);
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      const int ra = (strip * FM + f) * 32 + (lane & 31);
      a_off[j][f] = ra * 128 + Swizzle(ra, chunk) * 16;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int rb = c * 32 + (lane & 31);
      b_off[j][c] = S::kABytes + rb * 128 + Swizzle(rb, chunk) * 16;
    }
  }
  struct Fragments {
    half8 a[2][FM], b[2][4];
  };
  auto read = [&](int kt) {
    const unsigned char* s = lds + (kt % STAGES) * S::kStageBytes;
    Fragments fr;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int f = 0; f < FM; ++f)
        fr.a[j][f] = *reinterpret_cast<const half8*>(s + a_off[j][f]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        fr.b[j][c] = *reinterpret_cast<const half8*>(s + b_off[j][c]);
    }
    return fr;
  };

  // The ring: stage kt lives in buffer kt % STAGES. All buffers are filled
  // up front; in step kt, once stage kt + 1 has landed and every wave has
  // finished reading stage kt (its fragments are in registers), stage
  // kt + STAGES is loaded into kt's buffer, and stage kt + 1's fragments are
  // read while stage kt's MFMAs run.
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    if (s < steps)
      issue(s, s);
  {
    const int ahead = min(STAGES, steps) - 1;  // stages after 0 in flight
    if (ahead >= 3)
      WaitLoads<3 * S::kLoads>();
    else if (ahead == 2)
      WaitLoads<2 * S::kLoads>();
    else if (ahead == 1)
      WaitLoads<S::kLoads>();
    else
      WaitLoads<0>();
  }
  StageBarrier();
  // Makes stage kt + 1 readable and refills kt's buffer: stages up to
  // min(kt + STAGES - 1, steps - 1) are issued, so stage kt + 1 has landed
  // once at most `ahead` later ones are in flight; the barrier also tells
  // that every wave's fragment reads of stage kt have completed.
  auto advance = [&](int kt) {
    const int ahead = min(STAGES - 2, steps - 2 - kt);
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (ahead >= 2)
      WaitLoads<2 * S::kLoads>();
    else if (ahead == 1)
      WaitLoads<S::kLoads>();
    else
      WaitLoads<0>();
    StageBarrier();
    if (kt + STAGES < steps)
      issue(kt % STAGES, kt + STAGES);
  };
  // The scheduling barrier keeps the compiler from hoisting the next
  // advance's wait above these MFMAs, which would stall them behind the
  // reads they are meant to overlap.
  auto mma = [&](const Fragments& fr) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[f][c] = Mfma32(fr.a[j][f], fr.b[j][c], acc[f][c]);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Two fragment sets in ping-pong, so that a step's MFMAs never wait for
  // the next step's LDS reads, which are issued just before them.
  // The loop body has no branch around reads: a read on only one path makes
  // the compiler wait for it on both.
  if constexpr (FM == 1) {
    Fragments even = read(0), odd;
    int kt = 0;
    for (; kt + 2 < steps; kt += 2) {
      advance(kt);
      odd = read(kt + 1);
      mma(even);
      advance(kt + 1);
      even = read(kt + 2);
      mma(odd);
    }
    if (kt + 1 < steps) {
      advance(kt);
      odd = read(kt + 1);
      mma(even);
      mma(odd);
    } else {
      mma(even);
    }
  } else {
    // 64-row strips hold twice the accumulators, so fragments are
    // double-buffered per 16-wide substep instead of per K step: substep
    // u + 1 is read while substep u's MFMAs run.
    struct Half {
      half8 a[FM], b[4];
    };
    auto read_half = [&](int kt, int j) {
      const unsigned char* st = lds + (kt % STAGES) * S::kStageBytes;
      Half h;
#pragma unroll
      for (int f = 0; f < FM; ++f)
        h.a[f] = *reinterpret_cast<const half8*>(st + a_off[j][f]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        h.b[c] = *reinterpret_cast<const half8*>(st + b_off[j][c]);
      return h;
    };
    auto mma_half = [&](const Half& h) {
#pragma unroll
      for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[f][c] = Mfma32(h.a[f], h.b[c], acc[f][c]);
      __builtin_amdgcn_sched_barrier(0);
    };
    Half h0 = read_half(0, 0), h1;
    for (int kt = 0; kt + 1 < steps; ++kt) {
      h1 = read_half(kt, 1);
      mma_half(h0);
      advance(kt);
      h0 = read_half(kt + 1, 0);
      mma_half(h1);
    }
    h1 = read_half(steps - 1, 1);
    mma_half(h0);
    mma_half(h1);
  }

  // Swap accumulator halves. Flattening a column block's accumulators as
  // e = 16 f + r, group g keeps e in [8 FM g, 8 FM (g + 1)) (rows
  // 16 FM g .. 16 FM g + 16 FM - 1 of the strip) and hands the rest to its
  // partner wave (same strip, other group) as float4 number q = 2 FM c + h
  // at float4 index (wave * 8 FM + q) * 64 + lane.
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  StageBarrier();
  // Element e of column block c: accumulator e / 16, register e % 16. The
  // indices below are compile-time after unrolling; the group only selects
  // between two of them, so the accumulators stay in registers.
#define OVG_ACC(c, e) acc[(e) >> 4][c][(e) & 15]
  constexpr int kQuads = 2 * FM;  // float4 per column block
  constexpr int kHalf = 8 * FM;   // elements per group and column block
  const bool upper = group == 1;
  {
    floatx4* mine = reinterpret_cast<floatx4*>(lds) + wave * 4 * kQuads * 64 + lane;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int h = 0; h < kQuads; ++h) {
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = upper ? OVG_ACC(c, 4 * h + i) : OVG_ACC(c, kHalf + 4 * h + i);
        mine[(kQuads * c + h) * 64] = v;
      }
  }
  __syncthreads();
  Owned<FM> own;
  {
    const int partner = (1 - group) * S::kStrips + strip;
    const floatx4* theirs =
        reinterpret_cast<const floatx4*>(lds) + partner * 4 * kQuads * 64 + lane;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int h = 0; h < kQuads; ++h) {
        const floatx4 t = theirs[(kQuads * c + h) * 64];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          own.v[c][4 * h + i] =
              (upper ? OVG_ACC(c, kHalf + 4 * h + i) : OVG_ACC(c, 4 * h + i)) + t[i];
      }
  }
#undef OVG_ACC
  const int row0 = m0 + 32 * FM * strip + 16 * FM * group;

  if constexpr (EPI == Epilogue::kPartial) {
    // Each split owns a full [M][ldc] slice; the row kernel that consumes
    // the GEMM adds the slices.
    StoreOwned<FM, true>(p, own, p.y + static_cast<size_t>(split) * p.split_stride,
                         row0, n0, false);
    return;
  }
  if (p.splits > 1) {
    floatx4* mine = reinterpret_cast<floatx4*>(p.partials) +
                    ((static_cast<size_t>(tile) * p.splits + split) * S::kWaves + wave) *
                        4 * kQuads * 64 +
                    lane;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int h = 0; h < kQuads; ++h)
        StoreThrough(mine + (kQuads * c + h) * 64,
                     floatx4{own.v[c][4 * h], own.v[c][4 * h + 1],
                             own.v[c][4 * h + 2], own.v[c][4 * h + 3]});
    return;
  }
  OwnedEpilogue<EPI, FM>(p, own, row0, tile_n);
}

// Sums a tile's split-K partials in split order 0, 1, ... (a fixed order,
// reproducible bit for bit) in the same per-wave layout the GEMM kernel
// stored them in, and applies the epilogue. One single-wave work-group per
// (tile, GEMM wave): each wave's epilogue stands alone, and spreading the
// partials over that many CUs keeps every CU's share of the reads small.
template <Epilogue EPI, int FM, int STRIPS>
__global__ __launch_bounds__(64) void SplitReduceKernel(GemmParams p,
                                                       int tiles_m) {
  using S = Shape<FM, STRIPS>;
  constexpr int kQuads = 2 * FM;
  const int tile = blockIdx.x / S::kWaves;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x % S::kWaves;
  const size_t split_stride = static_cast<size_t>(S::kWaves) * 4 * kQuads * 64;
  const floatx4* base = reinterpret_cast<const floatx4*>(p.partials) +
                        static_cast<size_t>(tile) * p.splits * split_stride +
                        wave * 4 * kQuads * 64 + lane;
  // Split by split, each split's loads issued together (one memory round
  // trip per split), summing in split order 0, 1, ...
  floatx4 sum[4 * kQuads];
#pragma unroll
  for (int q = 0; q < 4 * kQuads; ++q)
    sum[q] = base[q * 64];
  for (int s = 1; s < p.splits; ++s) {
    floatx4 next[4 * kQuads];
#pragma unroll
    for (int q = 0; q < 4 * kQuads; ++q)
      next[q] = base[s * split_stride + q * 64];
#pragma unroll
    for (int q = 0; q < 4 * kQuads; ++q)
      sum[q] += next[q];
  }
  Owned<FM> own;
#pragma unroll
  for (int q = 0; q < 4 * kQuads; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      own.v[q / kQuads][4 * (q % kQuads) + i] = sum[q][i];
  const int tile_m = tile % tiles_m;
  const int row0 = tile_m * S::kBM + 32 * FM * (wave % S::kStrips) +
                   16 * FM * (wave / S::kStrips);
  OwnedEpilogue<EPI, FM>(p, own, row0, tile / tiles_m);
}

template <int STAGES, Epilogue EPI, int FM, int STRIPS>
void Launch(const GemmParams& p, int tiles_m, int band, int groups, hipStream_t stream) {
  const bool reduce = p.splits > 1 && EPI != Epilogue::kPartial;
  using S = Shape<FM, STRIPS>;
  Dispatch(GemmKernel<STAGES, EPI, FM, STRIPS>, dim3(groups), dim3(S::kThreads),
           LdsBytes<STAGES, FM, STRIPS>(), stream, true, !reduce, p, tiles_m, band);
  if (reduce)
    Dispatch(SplitReduceKernel<EPI, FM, STRIPS>, dim3(groups / p.splits * S::kWaves),
             dim3(64), 0, stream, false, true, p, tiles_m);
}

template <Epilogue EPI>
void LaunchEpi(const GemmParams& p, const GemmPlan& plan, hipStream_t stream) {
  const int groups = plan.tiles * plan.splits;
  if (plan.fm == 2)
    Launch<3, EPI, 2, 4>(p, (p.m + Shape<2>::kBM - 1) / Shape<2>::kBM, plan.band, groups, stream);
  else if (plan.strips == 1)
    Launch<3, EPI, 1, 1>(p, (p.m + Shape<1, 1>::kBM - 1) / Shape<1, 1>::kBM, plan.band, groups,
                         stream);
  else
    Launch<3, EPI, 1, 4>(p, (p.m + Shape<1>::kBM - 1) / Shape<1>::kBM, plan.band, groups, stream);
}

}  // namespace

// X bytes per band of row tiles (see GemmPlan::band).
constexpr std::int64_t kBandBytes = std::int64_t{2} << 20;

// Banded tile order once all rows of X outgrow what an XCD's L2 keeps
// beside the weight tiles: bands of at most kBandBytes of X. Split-K
// launches keep the plain order.
int BandFor(int m, int k, int bm, int splits) {
  const int tiles_m = (m + bm - 1) / bm;
  if (splits > 1)
    return tiles_m;
  const std::int64_t row_tile_bytes = static_cast<std::int64_t>(bm) * k * 2;
  return static_cast<int>(std::max<std::int64_t>(
      1, std::min<std::int64_t>(tiles_m, kBandBytes / row_tile_bytes)));
}

// Split count of the partial-slice GEMMs (o and down): a function of K
// alone, so that a row's slices, and the order in which the row kernel sums
// them, are the same whatever else is packed in the batch. Two splits where
// each keeps at least two K steps (the released o and down: 16 and 24 K
// steps each), else one. Four halved the K loop of each work-group but
// doubled the fp32 slices the next add + norm reads back; with two, 10 s
// 555 -> 570, clone 332 -> 367 and four batched chunks 608 -> 649 unmask
// steps/s (same box). Three for down (16 K steps each) help the short
// utterances and cost the long ones, re-measured on the current kernels:
// 10 s 578-585 -> 587-595, 2 s 893 -> 915-917, clone 387 -> 377, four
// chunks 689 -> 658 (its down 28.7 -> 35.8 us as 256 x 256 tiles, 43.5 as
// 128 x 256 in 1.3 rounds; same boxes). The count cannot follow M without
// making a row's sum depend on the batch, so two stay. Small M keeps its
// parallelism with two-wave tiles (PlanPacked).
int PartialSplits(int k_steps) {
  return k_steps % 2 == 0 && k_steps / 2 >= 2 ? 2 : 1;
}

GemmPlan PlanGemm(int m, int n, int k, Epilogue epilogue, bool split_small) {
  GemmPlan plan;
  const int tiles_n = (n + kBN - 1) / kBN;
  const int k_steps = k / kBK;
  const bool partial = epilogue == Epilogue::kPartial;
  const int splits = partial ? PartialSplits(k_steps) : 1;
  // Tile height from the work-group counts (tiles x splits). 256-row tiles
  // when they take fewer rounds of work-groups over the CUs, counting a
  // 256-row tile as 1.5 128-row tiles (twice the MFMAs at a quarter less LDS
  // traffic and fill per MFMA, the same fixed costs): large M, and shapes
  // whose 128-row tiles spill a few work-groups into a second round (the
  // audio heads at 500 rows: 260 tiles).
  const int wide = (m + Shape<1>::kBM - 1) / Shape<1>::kBM * tiles_n * splits;
  const int tall = (m + Shape<2>::kBM - 1) / Shape<2>::kBM * tiles_n * splits;
  const int rounds_wide = (wide + kCus - 1) / kCus;
  const int rounds_tall = (tall + kCus - 1) / kCus;
  plan.fm = 3 * rounds_tall < 2 * rounds_wide ? 2 : 1;
  // 32-row tiles (one strip per K group) when 128-row tiles would keep
  // under half the CUs busy and 32-row tiles still fit one round (2 s: the
  // packed 144 rows give q/k/v 64 tiles of 128 rows, the second holding 16
  // real rows).
  const int narrow = (m + Shape<1, 1>::kBM - 1) / Shape<1, 1>::kBM * tiles_n * splits;
  if (plan.fm == 1 && 2 * wide < kCus && narrow <= kCus)
    plan.strips = 1;
  const int bm = plan.fm == 2 ? Shape<2>::kBM : plan.strips == 1 ? Shape<1, 1>::kBM
                                                                 : Shape<1>::kBM;
  plan.tiles = (m + bm - 1) / bm * tiles_n;
  plan.stages = 3;
  plan.splits = splits;
  plan.partial_floats = 0;
  // The generator never splits the other GEMMs: a split chosen from M would
  // make a row's sums depend on the batch. Stand-alone callers may split K
  // when the tiles leave most CUs idle (partials cost a round trip through
  // memory and a second launch that sums them in split order).
  if (!partial && split_small && plan.tiles < 64) {
    int s_best = 1;
    for (const int s : {2, 3, 4, 6, 8}) {
      if (plan.tiles * s_best >= 128)
        break;
      if (k_steps % s == 0 && k_steps / s >= 4)
        s_best = s;
    }
    plan.splits = s_best;
    plan.partial_floats =
        s_best > 1 ? static_cast<std::size_t>(plan.tiles) * s_best * bm * kBN : 0;
  }
  plan.band = BandFor(m, k, bm, plan.splits);
  return plan;
}

void LaunchGemm(const GemmParams& p, const GemmPlan& plan, Epilogue epilogue,
                hipStream_t stream) {
  Require(p.m > 0 && p.n > 0 && p.k > 0, "gemm: empty shape");
  Require(p.k % kBK == 0, "gemm: K must be a multiple of 64");
  Require(plan.splits >= 1 && (p.k / kBK) % plan.splits == 0,
          "gemm: K steps not divisible by the split count");
  Require(plan.stages == 3, "gemm: a 3-stage ring");
  Require((plan.fm == 1 && (plan.strips == 4 || plan.strips == 1)) ||
              (plan.fm == 2 && plan.strips == 4),
          "gemm: 32-row strips by 4 or 1, or 64-row strips by 4");
  const int bm = 32 * plan.fm * plan.strips;
  Require(plan.tiles == ((p.m + bm - 1) / bm) * ((p.n + kBN - 1) / kBN),
          "gemm: plan does not match the shape");
  Require(p.lda % 8 == 0 && p.ldb % 8 == 0,
          "gemm: leading dimensions must be multiples of 8");
  // DMA sources are 32-bit byte offsets from the operand bases.
  Require(static_cast<uint64_t>(p.m) * p.lda * 2 < (uint64_t{1} << 32) &&
              static_cast<uint64_t>(p.n) * p.ldb * 2 < (uint64_t{1} << 32),
          "gemm: operands must be under 4 GiB");
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
    case Epilogue::kSwiGlu:
      throw Error("gemm: the q/k/v and SwiGLU epilogues run on packed weights (LaunchPacked)");
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
