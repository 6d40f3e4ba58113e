// fp16 x fp16 -> fp32 GEMM of the generator's projections on gfx950 matrix
// cores, with the weights packed at load into matrix-core fragment order
// (replaces the hipBLASLt calls of the reference's HalfGemm::Linear,
// gemm.cpp:248-262, and the QkNormRope / SwiGlu kernels that followed them,
// kernels/generator_kernels.hip:102-159, 191-200).
//
// Y[m][n] = sum_k X[m][k] W[n][k]. A work-group of four waves computes a
// (32 XB) x 128 output tile; wave w owns the 32 output columns
// 32 w .. 32 w + 31 of the tile over the whole K range, so its accumulators
// are final when the K loop ends (no exchange between waves).
//
// Operands:
//  * W (static) is packed at load (PackWeights) so that the fragment a wave
//    needs for one 16-wide K substep of one 32-column block is 1 KB of
//    consecutive bytes, lane l's 16 bytes at 16 l. Each wave streams its own
//    columns global -> registers, several K steps ahead; weights never pass
//    through LDS.
//  * X (the activations, shared by the four waves) goes global -> registers
//    -> LDS (a ring of four K steps, written two steps ahead, with an XOR
//    swizzle of the 16-byte chunks so that the fragment reads are
//    conflict-free) -> registers one step ahead, so a step's MFMAs never
//    wait for LDS.
// Every load is an ordinary load, so the compiler's wait counts are exact.
//
// The matrix-core instruction is v_mfma_f32_32x32x16_f16 (lane l receives
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] in element r). For the q/k/v and
// SwiGLU epilogues W is its first operand: a lane holds one output row
// (m = l % 32 of the 32-row block) and 16 of the block's 32 columns, four
// consecutive ones per group r / 4, so column pairs meet in one lane and
// the fp16 stores are 8-byte vectors. For the fp32 outputs X is the first
// operand: a lane holds one column and 16 rows, and the 32 lanes of a store
// write 128 consecutive bytes of a row (whole lines, which the write-through
// slices need). Inside a K step, lane half h supplies K elements
// 32 h + 8 j .. + 7 in substep j, for both operands.
//
// Column order inside a packed 32-column block (PackMap):
//  * identity: block column i is output column i (o, down, audio heads);
//  * rope: block w of a 128-column head holds head columns 16 w .. 16 w + 15
//    and 64 + 16 w .. 64 + 16 w + 15, so both halves of a rotate-half pair
//    are in one lane (elements r and r + 8);
//  * swiglu: block b holds gate rows 16 b .. 16 b + 15, then the matching up
//    rows, so gate and up of one output are in one lane (elements r, r + 8).
//
// Epilogues (the same Epilogue values as gemm.hip):
//  * kStore / kAccumulate / kPartial: fp32 stores, a row's 32 columns per
//    instruction (kPartial: write-through, each split its own slice, summed
//    by the next row kernel);
//  * kQkvRope: per-head RMSNorm (the squares of the wave's 32 columns, then
//    the four waves' sums through LDS in the fixed order (0 + 1) + (2 + 3)),
//    rotary in registers, fp16 q/k; value heads as V^T columns;
//  * kSwiGlu: silu(gate) * up in registers, fp16.
//
// No floating-point contraction in this file: every fused multiply-add is
// written out, so that the tile heights (template instantiations) round a
// row's values identically.

#include <algorithm>

#include "kernels.hpp"

#pragma clang fp contract(off)

namespace ovg {
namespace {


template <int XB>
struct Packed {
  static constexpr int kBM = 32 * XB;            // tile rows
  static constexpr int kStageBytes = kBM * 128;  // kBM rows x 64 halves
  static constexpr int kLds = 4 * kStageBytes;   // ring of four K steps
};

// q/k epilogue staging of one head: 32 XB rows of 256 bytes.
template <int XB>
constexpr int kHeadStage = 32 * XB * 256;
// The 128 x 256 tile's LDS: its ring, or the epilogue's sums ([4][128]
// floats) and two heads' staging after them.
constexpr int kWideSums = 4 * 128 * 4;
constexpr int kWideLds = Packed<4>::kLds > kWideSums + 2 * kHeadStage<4>
                             ? Packed<4>::kLds
                             : kWideSums + 2 * kHeadStage<4>;
static_assert(512 * 4 + kHeadStage<4> <= Packed<4>::kLds, "narrow q/k staging");

// The narrow tile's q/k/v instances stage the tile's rotary rows in LDS
// after the ring: 32 XB rows of 64 (cos, sin) pairs (512 bytes), 16-byte
// chunk c of row r at position c ^ (r % 32), so that the epilogue's reads
// (32 lanes, 32 rows, one chunk each) are free of bank conflicts.
constexpr int kRopeRowBytes = 64 * 8;
template <int XB, Epilogue EPI>
constexpr int NarrowLds() {
  return Packed<XB>::kLds + (EPI == Epilogue::kQkvRope ? 32 * XB * kRopeRowBytes : 0);
}

// 16-byte chunk c of LDS row r sits at position c ^ (r & 7) ^ ((r >> 3) & 1);
// its own inverse.
__device__ __forceinline__ int Swizzle(int row, int chunk) {
  return chunk ^ (row & 7) ^ ((row >> 3) & 1);
}

// Work-group barrier that first waits for this wave's LDS accesses only:
// the W and X prefetches stay in flight across it (a fence, or the
// compiler's barrier, would wait for every load).
__device__ __forceinline__ void Barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

// Lanes l and l + 32 hold the two 8-byte halves of two 16-byte chunks, a
// (their group 0) and b (group 1): lane l returns chunk a (a of lane l,
// then a of lane l + 32), lane l + 32 chunk b (b of lane l, then b of lane
// l + 32), by one v_permlane32_swap per dword.
__device__ __forceinline__ half8 SwapHalves(half4 a, half4 b) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 ua = __builtin_bit_cast(u32x2, a);
  const u32x2 ub = __builtin_bit_cast(u32x2, b);
  const auto s0 = __builtin_amdgcn_permlane32_swap(ua[0], ub[0], false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(ua[1], ub[1], false, false);
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 out = {s0[0], s1[0], s0[1], s1[1]};
  return __builtin_bit_cast(half8, out);
}

// Keeps the compiler from moving memory operations across this point.
__device__ __forceinline__ void AsmFence() { asm volatile("" : : : "memory"); }

// Packed q/k/v column tile (128-column head) `slot` in kv-group order: the
// `group` query heads of kv head g, then its key head, then its value head,
// for g = 0, 1, ... Returns the head's index in the reference's row order
// [q heads; k heads; v heads] (-1 past the last of `total` heads). With the
// tiles in this order the GEMM's XCD-contiguous tile runs write one kv
// group's q, k and v on one XCD, the XCD whose attention work-groups read
// them.
__host__ __device__ __forceinline__ int QkvHead(int slot, int total, int group) {
  if (slot >= total)
    return -1;
  const int kv = total / (group + 2);
  const int g = slot / (group + 2), j = slot % (group + 2);
  return j < group ? g * group + j : j == group ? kv * group + g : kv * (group + 1) + g;
}

// Epilogue of one wave: its WB packed 32-column blocks block0 .. block0 +
// WB - 1 (consecutive, inside one tile), accumulators acc[wb][b] for the
// 32-row blocks b of rows m0 ... Every result is rounded the same way
// whatever XB and WB are, so a row's outputs do not depend on the tile
// shape. `stage`: LDS offset of the q/k staging rows of this wave's head
// (32 XB rows of 256 bytes, shared by the 4 / WB waves of the head, clear of
// the LDS sums below).
template <int XB, int WB, Epilogue EPI>
__device__ __forceinline__ void WaveEpilogue(const GemmParams& p, floatx16 (&acc)[WB][XB],
                                             int m0, int split, int block0, int wave,
                                             int lane, unsigned char* lds, int stage,
                                             int rope_stage = -1) {
  constexpr int kBM = 32 * XB;
  const int h = lane >> 5;
  const int col = lane & 31;
  // Waves of a wide tile past the last column have nothing to store.
  const bool live = block0 * 32 < p.n;
  if constexpr (EPI == Epilogue::kStore || EPI == Epilogue::kAccumulate ||
                EPI == Epilogue::kPartial) {
    // Lane = column 32 block + lane % 32; element r of X block b is row
    // 32 b + 8 (r / 4) + 4 (lane / 32) + r % 4.
    float* y = p.y + (EPI == Epilogue::kPartial ? static_cast<size_t>(split) * p.split_stride : 0);
#pragma unroll
    for (int wb = 0; wb < WB; ++wb) {
      const int n = (block0 + wb) * 32 + col;
      if (n >= p.n)
        continue;
#pragma unroll
      for (int b = 0; b < XB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
          if (m >= p.m)
            continue;
          float* dst = y + static_cast<size_t>(m) * p.ldc + n;
          if constexpr (EPI == Epilogue::kAccumulate)
            *dst = *dst + acc[wb][b][r];
          else if constexpr (EPI == Epilogue::kPartial)
            StoreThrough(dst, acc[wb][b][r]);
          else
            *dst = acc[wb][b][r];
        }
    }
  } else if constexpr (EPI == Epilogue::kSwiGlu) {
    // Block `block` holds gate and up of outputs 16 block .. 16 block + 15.
    if (!live)
      return;
#pragma unroll
    for (int wb = 0; wb < WB; ++wb) {
      const int a_base = 16 * (block0 + wb) + 4 * h;
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        const int m = m0 + 32 * b + col;
        if (m >= p.m)
          continue;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          half4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float gate = acc[wb][b][4 * g + i];
            const float up = acc[wb][b][4 * g + 8 + i];
            v[i] = static_cast<half_t>(gate / (1.0F + __expf(-gate)) * up);
          }
          *reinterpret_cast<half4*>(p.act + static_cast<size_t>(m) * p.ldh + a_base + 8 * g) = v;
        }
      }
    }
  } else if constexpr (EPI == Epilogue::kQkvRope) {
    // Block `block` is block % 4 of packed head block / 4 (kv-group order,
    // QkvHead); a head's four blocks belong to 4 / WB waves of the tile.
    const int total = p.heads + 2 * p.kv_heads;
    const int slot = QkvHead(block0 / 4, total, p.heads / p.kv_heads);
    const bool qk = live && slot >= 0 && slot < p.heads + p.kv_heads;
    const float* weight = slot < p.heads ? p.q_norm : p.k_norm;
    // The rotary rows and norm weights of block wb (this lane's rotary
    // indices c = 16 (block % 4) + 8 g + 4 h + i, g < 2, i < 4), loaded a
    // block ahead into one of two register sets; the first block's before
    // the sums, so that their latency overlaps the sums and the barrier
    // rather than stalling once per block. Rows past M read row M - 1.
    // With `rope_stage` >= 0 the tile's rotary rows are already in LDS
    // there (one block per wave): they are read after the barrier.
    const bool staged = rope_stage >= 0;
    float2 rot[2][XB][8];
    float wt[2][16];  // w_lo[g][i] at 4 g + i, w_hi at 8 + 4 g + i
    auto load_weights = [&](int buf, int wb) {
      const int c_base = 16 * ((block0 + wb) & 3) + 4 * h;
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wt[buf][4 * g + i] = weight[c_base + 8 * g + i];
          wt[buf][8 + 4 * g + i] = weight[64 + c_base + 8 * g + i];
        }
    };
    auto load_rot = [&](int buf, int wb) {
      const int c_base = 16 * ((block0 + wb) & 3) + 4 * h;
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        if (staged) {
          // Pairs c_base + 8 g .. + 3 are chunks (c_base + 8 g) / 2 and + 1.
          const unsigned char* row = lds + rope_stage + (32 * b + col) * kRopeRowBytes;
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const int chunk = (c_base + 8 * g) / 2 + k;
              const float4 v = *reinterpret_cast<const float4*>(row + ((chunk ^ col) << 4));
              rot[buf][b][4 * g + 2 * k] = make_float2(v.x, v.y);
              rot[buf][b][4 * g + 2 * k + 1] = make_float2(v.z, v.w);
            }
        } else {
          const int m = min(m0 + 32 * b + col, p.m - 1);
          const float2* cs = p.rope + static_cast<size_t>(m) * 64 + c_base;
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              rot[buf][b][4 * g + i] = cs[8 * g + i];
        }
      }
    };
    auto load_rope = [&](int buf, int wb) {
      load_weights(buf, wb);
      load_rot(buf, wb);
    };
    if (qk) {
      load_weights(0, 0);
      if (!staged)
        load_rot(0, 0);
    }
    // Sum of squares of each block's 32 columns of a row, then over the
    // head's four blocks in the fixed order (0 + 1) + (2 + 3): a wave adds
    // its own pair when it holds two blocks, or all four when it holds the
    // head, and otherwise the waves' sums meet in LDS (the K loop's last
    // barrier separates the LDS reads of X from these writes).
    float* sums = reinterpret_cast<float*>(lds);  // [4][kBM]
    float part[WB][XB];
    if (qk) {
#pragma unroll
      for (int wb = 0; wb < WB; ++wb)
#pragma unroll
        for (int b = 0; b < XB; ++b) {
          float s = acc[wb][b][0] * acc[wb][b][0];
#pragma unroll
          for (int r = 1; r < 16; ++r)
            s = __builtin_fmaf(acc[wb][b][r], acc[wb][b][r], s);
          part[wb][b] = s + __shfl_xor(s, 32);
        }
      if (WB < 4 && h == 0) {
#pragma unroll
        for (int b = 0; b < XB; ++b)
          sums[wave * kBM + 32 * b + col] = WB == 2 ? part[0][b] + part[WB - 1][b] : part[0][b];
      }
    }
    if (staged)
      WaitLoads<0>();  // this wave's share of the staged rotary rows
    Barrier();  // LDS only: the rotary loads stay in flight
    if (qk && staged)
      load_rot(0, 0);
    // q/k heads: lanes l and l + 32 hold the two 8-byte halves of each of
    // two 16-byte chunks of a row (group g of lane half h: dims c_base + 8 g
    // .. + 3 of the block, c_base = 16 (block % 4) + 4 h), so one swap of
    // the upper and lower 32 lanes (v_permlane32_swap) gives lane half h the
    // whole chunk of dims 16 (block % 4) + 8 h .. + 7, which it stores in the
    // attention's operand order (QkIndex): a store covers 32 rows of 16
    // bytes, two 256-byte runs per lane half. (Staged through LDS instead,
    // to store 256-byte runs of 16 rows, it cost a second barrier and the
    // LDS round trip.)
    if (qk) {
      const int first = WB == 2 ? (wave & ~1) : 0;  // the first wave of this head
      float scale[XB];
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        const int r_local = 32 * b + col;
        float total;
        if constexpr (WB == 4)
          total = (part[0][b] + part[1][b]) + (part[2][b] + part[3][b]);
        else if constexpr (WB == 2)
          total = sums[first * kBM + r_local] + sums[(first + 1) * kBM + r_local];
        else
          total = (sums[r_local] + sums[kBM + r_local]) +
                  (sums[2 * kBM + r_local] + sums[3 * kBM + r_local]);
        scale[b] = rsqrtf(__builtin_fmaf(total, 1.0F / 128.0F, p.eps));
      }
#pragma unroll
      for (int wb = 0; wb < WB; ++wb) {
        if (wb + 1 < WB)
          load_rope((wb + 1) & 1, wb + 1);
        const int f = wb & 1;
        const int d0 = 16 * ((block0 + wb) & 3) + 8 * h;  // this lane's chunk after the swap
#pragma unroll
        for (int b = 0; b < XB; ++b) {
          half4 lo[2], hi[2];
#pragma unroll
          for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float2 cs = rot[f][b][4 * g + i];
              const float a = wt[f][4 * g + i] * (acc[wb][b][4 * g + i] * scale[b]);
              const float bb = wt[f][8 + 4 * g + i] * (acc[wb][b][4 * g + 8 + i] * scale[b]);
              lo[g][i] = static_cast<half_t>(__builtin_fmaf(a, cs.x, -(bb * cs.y)));
              hi[g][i] = static_cast<half_t>(__builtin_fmaf(bb, cs.x, a * cs.y));
            }
          const half8 lo_chunk = SwapHalves(lo[0], lo[1]);
          const half8 hi_chunk = SwapHalves(hi[0], hi[1]);
          const int m = m0 + 32 * b + col;
          if (live && m < p.m) {
            *reinterpret_cast<half8*>(p.qk + QkIndex(slot, m, d0, p.ldq)) = lo_chunk;
            *reinterpret_cast<half8*>(p.qk + QkIndex(slot, m, 64 + d0, p.ldq)) = hi_chunk;
          }
        }
      }
    } else if (live && slot >= 0) {
      // Value head: the head's staging area holds it as [dim 128][row 32 XB]
      // fp16, rows in VtColumn order inside each 16-row block, so that the
      // 8 keys of one V^T chunk are 16 consecutive bytes; d is the head
      // column of the element (rope order inside the block).
#pragma unroll
      for (int wb = 0; wb < WB; ++wb) {
        const int c_base = 16 * ((block0 + wb) & 3) + 4 * h;
#pragma unroll
        for (int b = 0; b < XB; ++b) {
          const int r_local = VtColumn(32 * b + col);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = c_base + 8 * ((r >> 2) & 1) + (r & 3) + 64 * (r >> 3);
            *reinterpret_cast<half_t*>(lds + stage + (d * kBM + r_local) * 2) =
                static_cast<half_t>(acc[wb][b][r]);
          }
        }
      }
    }
    // The value heads' staged V^T is read by the other waves of the head.
    // Where one head fills the work-group (four waves per head), a q/k
    // work-group has nothing staged and skips the barrier.
    if (WB != 1 || !qk)
      Barrier();
    if (!qk && live && slot >= 0) {
      // The 4 / WB waves of this value head copy its staged V^T out in
      // 16-byte chunks (VtIndex): chunk (16-row block, dim group, half,
      // dim 32) holds 8 keys of one dim; 32 lanes store 512 consecutive
      // bytes. Blocks past the last row are not written (a partial last
      // block is, with finite values from the clamped operand rows).
      const int gv = slot - p.heads - p.kv_heads;
      constexpr int kLanes = 64 * (4 / WB);
      const int t = (wave % (4 / WB)) * 64 + lane;
#pragma unroll
      for (int pass = 0; pass < 2 * XB * 256 / kLanes; ++pass) {
        const int e = pass * kLanes + t;
        const int d32 = e & 31, half = (e >> 5) & 1, dt = (e >> 6) & 3, b16 = e >> 8;
        const int d = 32 * dt + d32;
        const half8 v = *reinterpret_cast<const half8*>(
            lds + stage + (d * kBM + 16 * b16 + 8 * half) * 2);
        if (m0 + 16 * b16 < p.m)
          *reinterpret_cast<half8*>(p.vt + VtIndex(gv, d, m0 + 16 * b16 + (half ? 4 : 0),
                                                   p.ldvt)) = v;
      }
    }
  }
}

// NW waves, each owning one packed 32-column block: a (32 XB) x 128 tile
// with four, (32 XB) x 64 with two, (32 XB) x 32 with one (for small M,
// where the split-K slices alone leave too few tiles; not for the q/k/v
// epilogue, which needs a whole 128-column head in one work-group).
template <int XB, Epilogue EPI, int NW = 4, bool ANY_K = false>
__global__ __launch_bounds__(64 * NW) void PackedGemmKernel(GemmParams p, int tiles_m,
                                                            int k_steps) {
  static_assert(NW == 4 || ((NW == 2 || NW == 1) && EPI != Epilogue::kQkvRope),
                "the q/k/v epilogue needs four waves per 128-column head");
  using S = Packed<XB>;
  constexpr int XL = 4 * XB / NW;  // X loads (8 rows each) per wave and K step
  extern __shared__ __align__(16) unsigned char lds[];
  // Lane = output row (W as the first MFMA operand) for the epilogues that
  // pair columns inside a lane; lane = output column otherwise, so that the
  // 32 lanes of a fp32 store write 128 consecutive bytes of one row.
  constexpr bool kRowLanes = EPI == Epilogue::kQkvRope || EPI == Epilogue::kSwiGlu;

  // XCD-aware order: each XCD receives a contiguous run of tiles, rows
  // fastest, so the row tiles that share a column block of W share an L2.
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
  // The grid is tiles_m x tiles_n x splits work-groups; nothing past it.
  if (tile_n * 32 * NW >= p.n)
    return;
  const int m0 = tile_m * S::kBM;
  const int steps = k_steps / p.splits;  // K steps of this split
  const int t0 = split * steps;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int block = tile_n * NW + wave;  // this wave's packed 32-column block

  // X: wave w brings rows 8 (XL w + i) + lane / 8 of every K step (8 lanes
  // per 128-byte row), chunk lane % 8, to LDS position Swizzle(row, lane % 8).
  // Rows past M read row M - 1 (their results are never stored).
  const half8* x_src[XL];
  int x_dst[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int row = 8 * (XL * wave + i) + (lane >> 3);
    x_src[i] = reinterpret_cast<const half8*>(
        p.x + static_cast<size_t>(min(m0 + row, p.m - 1)) * p.lda + t0 * 64) + (lane & 7);
    x_dst[i] = row * 128 + Swizzle(row, lane & 7) * 16;
  }
  // W: fragment (t, j) of this block is 64 half8 at ((block k_steps + t) 4 + j) 64.
  const half8* w_src =
      reinterpret_cast<const half8*>(p.w) + (static_cast<size_t>(block) * k_steps + t0) * 256 + lane;
  // Fragment reads of X: row 32 b + lane % 32, chunk 4 (lane / 32) + j.
  int x_read[XB][4];
#pragma unroll
  for (int b = 0; b < XB; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 32 * b + (lane & 31);
      x_read[b][j] = row * 128 + Swizzle(row, 4 * (lane >> 5) + j) * 16;
    }

  floatx16 acc[1][XB];
#pragma unroll
  for (int b = 0; b < XB; ++b)
    acc[0][b] = floatx16{};

  half8 wf[4][4];       // W of steps t .. t + 3, slot t % 4
  half8 xs[2][XL];      // X of steps t + 2 and t + 3, slot t % 2
  half8 fr[2][4][XB];   // fragments of X(t) (slot t % 2) and X(t + 1)
  auto load_x = [&](half8 (&dst)[XL], int t) {
#pragma unroll
    for (int i = 0; i < XL; ++i)
      dst[i] = x_src[i][t * 8];  // 64 halves = 8 half8 per K step
  };
  auto store_x = [&](const half8 (&src)[XL], int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i)
      *reinterpret_cast<half8*>(lds + buf * S::kStageBytes + x_dst[i]) = src[i];
  };
  auto read_frag = [&](half8 (&dst)[XB], int buf, int j) {
#pragma unroll
    for (int b = 0; b < XB; ++b)
      dst[b] = *reinterpret_cast<const half8*>(lds + buf * S::kStageBytes + x_read[b][j]);
  };

  // Prologue: W of steps 0 .. 3 and X of steps 0 .. 3 are loaded; X(0) and
  // X(1) go to LDS buffers 0 and 1, X(0)'s fragments to registers. Step
  // indices past the last are clamped to it (in-bounds reloads whose values
  // are never used), so that no load sits under a condition: a conditional
  // load makes the compiler's wait counts assume it was skipped and wait for
  // the loads before it.
  //
  // The loads are issued in the loop's own order (W of a step's first three
  // substeps, X of the step, W of its last substep), so that at the loop's
  // first step the loads in flight are those of its steady state: the
  // compiler's wait counts at the loop head are the smaller of what the
  // first iteration and the later ones need, and a prologue in another order
  // made two steps in four wait for loads issued one step earlier instead of
  // two.
  const int last = steps - 1;
  // q/k tiles stage their 32 XB rotary rows (512 bytes each) in LDS after
  // the ring: XB 1 KB DMAs per wave in each of the last four K steps, which
  // issue no operand loads (nothing in the loop waits for them, and they
  // take none of the operand stream's bandwidth: issued in the earlier
  // steps they slowed the loop by as much as they saved), so that the
  // epilogue reads LDS instead of a row-strided table (issuing those loads
  // after the loop took ~1.5 K clocks at 580 rows). Only where the grid is
  // one round of work-groups: the 48 KB more LDS per work-group would keep
  // a second one off a CU (1055 rows: q/k/v 19.2 -> 21.2 us).
  // Block i of wave w holds tile rows 2 (4 XB w + i) and + 1; lane l writes
  // chunk (l % 32) ^ (row % 32) of row + l / 32. Rows past M read row M - 1.
  bool stage_rope = false;
  if constexpr (EPI == Epilogue::kQkvRope && !ANY_K) {
    const int slot = QkvHead(tile_n, p.heads + 2 * p.kv_heads, p.heads / p.kv_heads);
    stage_rope = groups <= kCus && slot >= 0 && slot < p.heads + p.kv_heads;
  }
  const unsigned char* rope_base =
      reinterpret_cast<const unsigned char*>(p.rope + static_cast<size_t>(m0) * 64);
  const uint32_t rope_lds = LdsAddress(lds) + S::kLds + wave * 4 * XB * 1024;
  auto stage_rope_block = [&](int i) {
    const int row = 2 * (4 * XB * wave + i) + (lane >> 5);
    const int chunk = (lane & 31) ^ (row & 31);
    const uint32_t off = static_cast<uint32_t>((min(m0 + row, p.m - 1) - m0) * kRopeRowBytes +
                                               chunk * 16);
    DmaToLds(rope_base, off, rope_lds + i * 1024);
  };
  {
    half8 x0[XL], x1[XL];
    auto load_step = [&](int s, half8 (&x)[XL]) {
      const int t = min(s, last);
#pragma unroll
      for (int j = 0; j < 3; ++j)
        wf[s][j] = w_src[(t * 4 + j) * 64];
      load_x(x, t);
      wf[s][3] = w_src[(t * 4 + 3) * 64];
    };
    load_step(0, x0);
    load_step(1, x1);
    load_step(2, xs[0]);
    load_step(3, xs[1]);
    store_x(x0, 0);
    store_x(x1, 1);
  }
  Barrier();
#pragma unroll
  for (int j = 0; j < 4; ++j)
    read_frag(fr[0][j], 0, j);

  // Step t (LDS buffers by t % 4, register slots by t % 4 and t % 2): the
  // 4 XB MFMAs of step t from fragments already in registers, each followed
  // by memory work of the step, so that it issues in the MFMA's shadow (with
  // one wave per SIMD an MFMA holds up the wave's next instruction for its 32
  // clocks): after every MFMA one read of X(t + 1)'s fragments from buffer
  // (t + 1) % 4 (written in step t - 1, before the barrier that ended it), so
  // no MFMA waits for LDS; after a substep's last MFMA the reload of its W
  // slot with W(t + 4); after the step's last XL MFMAs (the last substep
  // with four waves, the last two with two), one each, the write of part of
  // X(t + 2) into buffer (t + 2) % 4 (its previous content, X(t - 2), was
  // last read in step t - 3) and the reload of those registers with X(t + 4).
  // The step ends at a barrier that first waits for all of its LDS
  // operations, after which X(t + 2) is readable. (Writing X(t + 2) in the
  // first substep instead measured 1-3 % slower at 580 rows; letting the
  // fragment reads run on across the barrier measured no faster.)
  //
  // RELOAD, WRITE and READ (compile-time) switch off the step's global
  // reloads, its write of X(t + 2) and its reads of X(t + 1)'s fragments
  // where those steps are past the last: the last four steps of a K range
  // that is a multiple of four steps issue no loads, so that the epilogue's
  // loads and stores do not queue behind 28 KB per wave of clamped reloads
  // that nothing uses (at 580 x 4096 x 1024 they took ~2 K clocks to drain
  // before the q/k/v epilogue's first loads could issue).
  auto step = [&](int t, auto slot, auto reload, auto write, auto read) {
    constexpr int ws = decltype(slot)::value;  // t % 4
    constexpr int xo = ws & 1;                 // t % 2
    constexpr bool kReload = decltype(reload)::value;
    constexpr bool kWrite = decltype(write)::value;
    constexpr bool kRead = decltype(read)::value;
    const int ahead = min(t + 4, last);
#pragma unroll
    for (int i = 0; i < 4 * XB; ++i) {
      const int j = i / XB, b = i % XB;
      acc[0][b] = kRowLanes ? Mfma32(wf[ws][j], fr[xo][j][b], acc[0][b])
                            : Mfma32(fr[xo][j][b], wf[ws][j], acc[0][b]);
      __builtin_amdgcn_sched_barrier(0);
      if (i >= 4 * XB - XL) {
        const int xi = i - (4 * XB - XL);
        if constexpr (kWrite) {
          *reinterpret_cast<half8*>(lds + ((ws + 2) & 3) * S::kStageBytes + x_dst[xi]) =
              xs[xo][xi];
          AsmFence();
        }
        if constexpr (kReload)
          xs[xo][xi] = x_src[xi][ahead * 8];
      }
      if constexpr (kRead)
        fr[1 - xo][i / XB][i % XB] = *reinterpret_cast<const half8*>(
            lds + ((ws + 1) & 3) * S::kStageBytes + x_read[i % XB][i / XB]);
      if constexpr (kReload)
        if (b == XB - 1)
          wf[ws][j] = w_src[(ahead * 4 + j) * 64];
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EPI == Epilogue::kQkvRope && !kReload) {
      // The last four steps (slot = step - (steps - 4)): XB blocks each.
      if (stage_rope)
#pragma unroll
        for (int i = 0; i < XB; ++i)
          stage_rope_block(ws * XB + i);
    }
    Barrier();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using On = std::true_type;
  using Off = std::false_type;
  if constexpr (!ANY_K) {
    // K range per split a multiple of four steps (every shape of the model).
    const int body = steps - 4;
    for (int t = 0; t < body; t += 4) {
      step(t, I0{}, On{}, On{}, On{});
      step(t + 1, I1{}, On{}, On{}, On{});
      step(t + 2, I2{}, On{}, On{}, On{});
      step(t + 3, I3{}, On{}, On{}, On{});
    }
    step(body, I0{}, Off{}, On{}, On{});
    step(body + 1, I1{}, Off{}, On{}, On{});
    step(body + 2, I2{}, Off{}, Off{}, On{});
    step(body + 3, I3{}, Off{}, Off{}, Off{});
  } else {
    // Any K range (a separate instance, so that the loop above keeps its
    // registers): every step reloads, clamped to the last step, and the
    // last steps % 4 run after the groups of four.
    const int whole = steps & ~3;
    for (int t = 0; t < whole; t += 4) {
      step(t, I0{}, On{}, On{}, On{});
      step(t + 1, I1{}, On{}, On{}, On{});
      step(t + 2, I2{}, On{}, On{}, On{});
      step(t + 3, I3{}, On{}, On{}, On{});
    }
    if (whole < steps)
      step(whole, I0{}, On{}, On{}, On{});
    if (whole + 1 < steps)
      step(whole + 1, I1{}, On{}, On{}, On{});
    if (whole + 2 < steps)
      step(whole + 2, I2{}, On{}, On{}, On{});
  }

  // q/k staging after the LDS sums ([4][32 XB] floats).
  WaveEpilogue<XB, 1, EPI>(p, acc, m0, split, block, wave, lane, lds, 512 * XB,
                           stage_rope ? S::kLds : -1);
}

// The wide tile for large M: 128 x 256, each wave owning two packed blocks
// (64 columns), so every X fragment read from LDS feeds two MFMAs (half the
// LDS reads per MFMA of the 128 x 128 tile, which at large M is bound by
// them). Registers: W two K steps ahead (a ring of two) and X fragments one
// 16-wide substep ahead, with the eight MFMAs of a substep covering the
// fragment reads' latency.
template <Epilogue EPI>
__global__ __launch_bounds__(256) void PackedWideKernel(GemmParams p, int tiles_m, int k_steps) {
  constexpr int XB = 4;
  constexpr int WB = 2;
  using S = Packed<XB>;
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr bool kRowLanes = EPI == Epilogue::kQkvRope || EPI == Epilogue::kSwiGlu;

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
  if (tile_n * 256 >= p.n)
    return;
  const int m0 = tile_m * S::kBM;
  const int steps = k_steps / p.splits;
  const int t0 = split * steps;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int block0 = tile_n * 8 + 2 * wave;  // this wave's two packed blocks

  const half8* x_src[XB];
  int x_dst[XB];
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int row = 8 * (XB * wave + i) + (lane >> 3);
    x_src[i] = reinterpret_cast<const half8*>(
        p.x + static_cast<size_t>(min(m0 + row, p.m - 1)) * p.lda + t0 * 64) + (lane & 7);
    x_dst[i] = row * 128 + Swizzle(row, lane & 7) * 16;
  }
  // Block block0 + 1 follows block0 at k_steps * 256 half8.
  const half8* w_src =
      reinterpret_cast<const half8*>(p.w) + (static_cast<size_t>(block0) * k_steps + t0) * 256 + lane;
  const size_t w_next = static_cast<size_t>(k_steps) * 256;
  int x_read[XB][4];
#pragma unroll
  for (int b = 0; b < XB; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 32 * b + (lane & 31);
      x_read[b][j] = row * 128 + Swizzle(row, 4 * (lane >> 5) + j) * 16;
    }

  floatx16 acc[WB][XB];
#pragma unroll
  for (int wb = 0; wb < WB; ++wb)
#pragma unroll
    for (int b = 0; b < XB; ++b)
      acc[wb][b] = floatx16{};

  half8 wf[2][WB][4];  // W of steps t, t + 1, slot t % 2
  half8 xs[2][XB];     // X of steps t + 2 and t + 3, slot t % 2
  half8 fr[2][XB];     // X fragments of the current and the next substep
  auto load_x = [&](half8 (&dst)[XB], int t) {
#pragma unroll
    for (int i = 0; i < XB; ++i)
      dst[i] = x_src[i][t * 8];
  };
  auto store_x = [&](const half8 (&src)[XB], int buf) {
#pragma unroll
    for (int i = 0; i < XB; ++i)
      *reinterpret_cast<half8*>(lds + buf * S::kStageBytes + x_dst[i]) = src[i];
  };
  auto read_frag = [&](half8 (&dst)[XB], int buf, int j) {
#pragma unroll
    for (int b = 0; b < XB; ++b)
      dst[b] = *reinterpret_cast<const half8*>(lds + buf * S::kStageBytes + x_read[b][j]);
  };

  // Prologue: W of steps 0 and 1, X of steps 0 .. 3 (X(0), X(1) to LDS
  // buffers 0 and 1), then the fragments of step 0's first substep. Step
  // indices past the last are clamped (in-bounds reloads never used).
  // Loads in the loop's own order (W of step t + 2's first three substeps,
  // X of step t + 4, W of step t + 2's last substep), so that the
  // compiler's wait counts at the loop head are those of the steady state.
  const int last = steps - 1;
  {
    half8 x0[XB], x1[XB];
    load_x(x0, 0);
    load_x(x1, min(1, last));
    auto load_step = [&](int s, half8 (&x)[XB]) {
      const int t = min(s, last);
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int wb = 0; wb < WB; ++wb)
          wf[s][wb][j] = w_src[wb * w_next + (t * 4 + j) * 64];
      load_x(x, min(s + 2, last));
#pragma unroll
      for (int wb = 0; wb < WB; ++wb)
        wf[s][wb][3] = w_src[wb * w_next + (t * 4 + 3) * 64];
    };
    load_step(0, xs[0]);
    load_step(1, xs[1]);
    store_x(x0, 0);
    store_x(x1, 1);
  }
  Barrier();
  read_frag(fr[0], 0, 0);

  // Step t: for each substep j its eight MFMAs from fragments in
  // registers, each followed by memory work of the step, so that it issues
  // in the MFMA's shadow (with one wave per SIMD an MFMA holds up the wave's
  // next instruction for its 32 clocks): after every other MFMA one read of
  // the next substep's fragments (substep j + 1 of buffer t % 4, or the
  // first substep of step t + 1 from buffer (t + 1) % 4, written in step
  // t - 1); in substep 3, after the others, the write of X(t + 2) into LDS
  // buffer (t + 2) % 4 and the reload of those registers with X(t + 4);
  // after the last MFMA of a W fragment its reload with W(t + 2). The step
  // ends at a barrier that waits for all of its LDS operations. A buffer is
  // rewritten two barriers after its last read.
  auto step = [&](int t, auto slot) {
    constexpr int ws = decltype(slot)::value;  // t % 4
    constexpr int xo = ws & 1;                 // t % 2
    const int ahead_x = min(t + 4, last);
    const int ahead_w = min(t + 2, last);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < WB * XB; ++i) {
        const int wb = i / XB, b = i % XB;
        acc[wb][b] = kRowLanes ? Mfma32(wf[xo][wb][j], fr[j & 1][b], acc[wb][b])
                               : Mfma32(fr[j & 1][b], wf[xo][wb][j], acc[wb][b]);
        __builtin_amdgcn_sched_barrier(0);
        if (i % 2 == 0) {
          const int rb = i / 2;
          const int buf = j < 3 ? ws : (ws + 1) & 3;
          fr[(j + 1) & 1][rb] = *reinterpret_cast<const half8*>(
              lds + buf * S::kStageBytes + x_read[rb][j < 3 ? j + 1 : 0]);
        } else if (j == 3) {
          const int xi = i / 2;
          *reinterpret_cast<half8*>(lds + ((ws + 2) & 3) * S::kStageBytes + x_dst[xi]) =
              xs[xo][xi];
          AsmFence();
          xs[xo][xi] = x_src[xi][ahead_x * 8];
        }
        if (b == XB - 1)
          wf[xo][wb][j] = w_src[wb * w_next + (ahead_w * 4 + j) * 64];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    Barrier();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  const int whole = steps & ~3;
  for (int t = 0; t < whole; t += 4) {
    step(t, I0{});
    step(t + 1, I1{});
    step(t + 2, I2{});
    step(t + 3, I3{});
  }
  if (whole < steps)
    step(whole, I0{});
  if (whole + 1 < steps)
    step(whole + 1, I1{});
  if (whole + 2 < steps)
    step(whole + 2, I2{});

  // Two heads' q/k staging (waves 0-1, 2-3) after the LDS sums.
  WaveEpilogue<XB, WB, EPI>(p, acc, m0, split, block0, wave, lane, lds,
                            kWideSums + (wave >> 1) * kHeadStage<XB>);
}

// The large tile for large M: 256 x 256, four waves in a 2 x 2 arrangement,
// wave w owning rows 128 (w / 2) .. + 127 and the four packed blocks
// 4 (w % 2) .. + 3, 16 accumulators. Every fragment read from LDS feeds four
// MFMAs, and the operands a work-group pulls from L2 per K step serve twice
// the MFMAs of the 128 x 256 tile. X and W both go global -> LDS by DMA
// (no registers, so a deep prefetch costs nothing but LDS) through a ring of
// four half-steps (32 K values, 32 KB: X then W); a half-step's DMAs are
// issued four half-steps before its MFMAs.
//
// Half-step s holds K substeps 2 (s % 2) and 2 (s % 2) + 1 of K step s / 2,
// i.e. the 16-byte chunks {0, 1, 4, 5} or {2, 3, 6, 7} of every 128-byte
// X row segment (lane half h supplies chunk 4 h + j in substep j, as in the
// packed W): LDS X row r (64 bytes) holds those four chunks as positions
// q = 2 h + (j % 2), at Swizzle32(r, q). The packed W of half-step s is 2 KB
// of each block's 4 KB K step, copied verbatim.
constexpr int kBigHalf = 32768;         // one half-step: X 16 KB, then W 16 KB
constexpr int kBigLds = 4 * kBigHalf;   // ring of four half-steps
constexpr int kBigDmas = 8;             // DMAs per wave per half-step
static_assert(4 * kHeadStage<4> <= kBigLds, "q/k staging of four heads in the ring");

// Position of chunk q of 64-byte LDS row r: distinct banks for the rows of
// a fragment read in both 8-lane (128-byte) and 16-lane (256-byte) phases.
// Its own inverse.
__device__ __forceinline__ int Swizzle32(int row, int q) {
  return q ^ ((row >> 1) & 3) ^ ((row >> 3) & 1);
}

// The q/k/v epilogue of the 256 x 256 tile, where a wave holds one whole
// head (its four packed blocks) for 128 rows. The rotary rows of its 128
// rows are 64 KB, which the general epilogue loads block by block from the
// row-strided table (16 loads per lane and block, each touching 32 rows
// 512 bytes apart): at 3440 rows that took ~15 K of a launch's ~65 K clocks
// (41.6 against 37.5 us with constants in their place). Here the four waves
// copy the tile's 256 rotary rows (128 KB) into LDS by DMA once the K loop
// has freed the ring (chunk c of row r at position c ^ (r % 32), so the
// reads are conflict-free), and each wave stages and stores its head one
// 32-column block at a time (8 KB of LDS per wave instead of 32 KB, which
// leaves the room). Every value is computed and rounded as in WaveEpilogue.
constexpr int kBigStage = 8192;                    // per wave, one block
constexpr int kBigRope = 4 * kBigStage;            // 256 rows x 512 bytes after it
constexpr int kBigQkvLds = kBigRope + 256 * kRopeRowBytes;
static_assert(kBigQkvLds >= kBigLds && kBigQkvLds <= 160 * 1024, "q/k/v tile LDS");

__device__ __forceinline__ void BigQkvEpilogue(const GemmParams& p, floatx16 (&acc)[4][4],
                                               int tile_m0, int wr, int block0, int wave,
                                               int lane, unsigned char* lds) {
  constexpr int XB = 4, WB = 4, kBM = 128;
  const int h = lane >> 5;
  const int col = lane & 31;
  const int m0 = tile_m0 + 128 * wr;
  const int total = p.heads + 2 * p.kv_heads;
  const int slot = QkvHead(block0 / 4, total, p.heads / p.kv_heads);
  const bool live = block0 * 32 < p.n && slot >= 0;
  const bool qk = live && slot < p.heads + p.kv_heads;
  const float* weight = slot < p.heads ? p.q_norm : p.k_norm;
  // Rotary rows of the tile in four pieces, piece k the pairs 16 k .. + 15
  // (16-byte chunks 8 k .. + 7) of all 256 rows, 32 KB at kBigRope + 32 KB
  // k: row r's 128 bytes at 128 r, chunk c at position c ^ ((r / 2) % 8)
  // (conflict-free reads). DMA block i of a piece covers rows 8 i .. + 7,
  // wave w taking blocks 8 w .. 8 w + 7 of every piece, pieces in order, so
  // that piece k has landed everywhere once each wave has waited for its
  // own DMAs of pieces 0 .. k and the work-group has met. Rows past M read
  // row M - 1.
  const unsigned char* rope_base =
      reinterpret_cast<const unsigned char*>(p.rope + static_cast<size_t>(tile_m0) * 64);
  const uint32_t rope_dst = LdsAddress(lds) + kBigRope + wave * 8 * 1024;
  auto dma_piece = [&](int k) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 8 * (8 * wave + i) + (lane >> 3);
      const int chunk = (lane & 7) ^ ((row >> 1) & 7);
      const uint32_t off = static_cast<uint32_t>(
          (min(tile_m0 + row, p.m - 1) - tile_m0) * kRopeRowBytes + (8 * k + chunk) * 16);
      DmaToLds(rope_base, off, rope_dst + k * 32768 + i * 1024);
    }
  };
  // Piece 0, then the norm weights of all four blocks, which are waited for
  // (with piece 0, needed first anyway) before pieces 1 .. 3 are issued: the
  // compiler's wait for a load of its own would otherwise also wait for the
  // DMAs issued after it.
  dma_piece(0);
  float wt[WB][16];  // w_lo[g][i] at 4 g + i, w_hi at 8 + 4 g + i
  if (qk) {
#pragma unroll
    for (int wb = 0; wb < WB; ++wb) {
      const int c_base = 16 * ((block0 + wb) & 3) + 4 * h;
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wt[wb][4 * g + i] = weight[c_base + 8 * g + i];
          wt[wb][8 + 4 * g + i] = weight[64 + c_base + 8 * g + i];
        }
    }
  }
  float scale[XB];
  if (qk) {
    // The head's sum of squares per row: each block's 32 columns, then the
    // four blocks as (0 + 1) + (2 + 3).
    float part[WB][XB];
#pragma unroll
    for (int wb = 0; wb < WB; ++wb)
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        float s = acc[wb][b][0] * acc[wb][b][0];
#pragma unroll
        for (int r = 1; r < 16; ++r)
          s = __builtin_fmaf(acc[wb][b][r], acc[wb][b][r], s);
        part[wb][b] = s + __shfl_xor(s, 32);
      }
#pragma unroll
    for (int b = 0; b < XB; ++b) {
      const float t = (part[0][b] + part[1][b]) + (part[2][b] + part[3][b]);
      scale[b] = rsqrtf(__builtin_fmaf(t, 1.0F / 128.0F, p.eps));
    }
#pragma unroll
    for (int wb = 0; wb < WB; ++wb)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        asm volatile("" : : "v"(wt[wb][i]));
  }
  WaitLoads<0>();
  dma_piece(1);
  dma_piece(2);
  dma_piece(3);
  // Waits until piece k has landed in the whole work-group (piece 0: at
  // the wait above). The count assumes no later memory instruction; the
  // blocks' stores, issued after the DMAs, count too, so the wait can only
  // be longer than needed, never shorter.
  auto piece_ready = [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    WaitLoads<8 * (3 - k)>();
    __builtin_amdgcn_s_barrier();
    AsmFence();
  };
  unsigned char* stage = lds + wave * kBigStage;
  // Block wb uses piece (block0 + wb) % 4 = wb (block0 is a multiple of 4);
  // every wave meets at all four points, whatever its head.
  if (qk) {
#pragma unroll
    for (int wb = 0; wb < WB; ++wb) {
      if (wb == 0) piece_ready(std::integral_constant<int, 0>{});
      if (wb == 1) piece_ready(std::integral_constant<int, 1>{});
      if (wb == 2) piece_ready(std::integral_constant<int, 2>{});
      if (wb == 3) piece_ready(std::integral_constant<int, 3>{});
      const int c_base = 16 * ((block0 + wb) & 3) + 4 * h;
      const int chunk0 = 2 * ((block0 + wb) & 3);
      // Rotated, normalised q/k of this block: row r_local = 32 b + col,
      // position g (lo, chunk chunk0 + g) or 2 + g (hi, chunk chunk0 + 8 + g)
      // of its 64-byte staging row, swizzled by (r / 4) % 4, half h.
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        const int rr = 128 * wr + 32 * b + col;  // tile row
        const unsigned char* rope_row = lds + kBigRope + wb * 32768 + rr * 128;
        float2 rot[8];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int chunk = (c_base + 8 * g) / 2 + k - 8 * wb;  // within the piece
            const float4 v =
                *reinterpret_cast<const float4*>(rope_row + ((chunk ^ ((rr >> 1) & 7)) << 4));
            rot[4 * g + 2 * k] = make_float2(v.x, v.y);
            rot[4 * g + 2 * k + 1] = make_float2(v.z, v.w);
          }
        const int r_local = 32 * b + col;
        unsigned char* row = stage + r_local * 64 + 8 * h;
        const int swz = (r_local >> 2) & 3;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          half4 lo, hi;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float2 cs = rot[4 * g + i];
            const float a = wt[wb][4 * g + i] * (acc[wb][b][4 * g + i] * scale[b]);
            const float bb = wt[wb][8 + 4 * g + i] * (acc[wb][b][4 * g + 8 + i] * scale[b]);
            lo[i] = static_cast<half_t>(__builtin_fmaf(a, cs.x, -(bb * cs.y)));
            hi[i] = static_cast<half_t>(__builtin_fmaf(bb, cs.x, a * cs.y));
          }
          *reinterpret_cast<half4*>(row + ((g ^ swz) << 4)) = lo;
          *reinterpret_cast<half4*>(row + (((2 + g) ^ swz) << 4)) = hi;
        }
      }
      AsmFence();
      // Copy-out in the attention's fragment order (QkIndex): 16 lanes store
      // one chunk of 16 consecutive rows, a 256-byte run.
#pragma unroll
      for (int pass = 0; pass < 8; ++pass) {
        const int e = pass * 64 + lane;
        const int r = (e & 15) + 16 * (e >> 6);
        const int pos = (e >> 4) & 3;
        const int q = pos < 2 ? chunk0 + pos : chunk0 + 8 + (pos - 2);
        const half8 v = *reinterpret_cast<const half8*>(
            stage + r * 64 + ((pos ^ ((r >> 2) & 3)) << 4));
        if (m0 + r < p.m)
          *reinterpret_cast<half8*>(p.qk + QkIndex(slot, m0 + r, 8 * q, p.ldq)) = v;
      }
      AsmFence();
    }
  } else if (live) {
    // Value head: per block, V^T of its 32 dims (d_local = d % 16 + 16 (d /
    // 64)) x 128 rows in VtColumn order, then 16-byte chunks of 8 keys
    // (VtIndex).
    const int gv = slot - p.heads - p.kv_heads;
#pragma unroll
    for (int wb = 0; wb < WB; ++wb) {
      if (wb == 0) piece_ready(std::integral_constant<int, 0>{});
      if (wb == 1) piece_ready(std::integral_constant<int, 1>{});
      if (wb == 2) piece_ready(std::integral_constant<int, 2>{});
      if (wb == 3) piece_ready(std::integral_constant<int, 3>{});
      const int blk = (block0 + wb) & 3;
      const int c_base = 16 * blk + 4 * h;
#pragma unroll
      for (int b = 0; b < XB; ++b) {
        const int r_local = VtColumn(32 * b + col);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = c_base + 8 * ((r >> 2) & 1) + (r & 3) + 64 * (r >> 3);
          const int d_local = (d & 15) + 16 * (d >> 6);
          *reinterpret_cast<half_t*>(stage + (d_local * kBM + r_local) * 2) =
              static_cast<half_t>(acc[wb][b][r]);
        }
      }
      AsmFence();
#pragma unroll
      for (int pass = 0; pass < 8; ++pass) {
        const int e = pass * 64 + lane;
        const int d_local = e & 31, half = (e >> 5) & 1, b16 = e >> 6;
        const int d = (d_local & 15) + 16 * blk + 64 * (d_local >> 4);
        const half8 v = *reinterpret_cast<const half8*>(
            stage + (d_local * kBM + 16 * b16 + 8 * half) * 2);
        if (m0 + 16 * b16 < p.m)
          *reinterpret_cast<half8*>(p.vt + VtIndex(gv, d, m0 + 16 * b16 + (half ? 4 : 0),
                                                   p.ldvt)) = v;
      }
      AsmFence();
    }
  } else {
    // Past the last column: nothing to store, but the meetings are the
    // work-group's.
    piece_ready(std::integral_constant<int, 0>{});
    piece_ready(std::integral_constant<int, 1>{});
    piece_ready(std::integral_constant<int, 2>{});
    piece_ready(std::integral_constant<int, 3>{});
  }
}

template <Epilogue EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void PackedBigKernel(GemmParams p, int tiles_m, int k_steps) {
  constexpr int XB = 4;
  constexpr int WB = 4;
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr bool kRowLanes = EPI == Epilogue::kQkvRope || EPI == Epilogue::kSwiGlu;

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
  if (tile_n * 256 >= p.n)
    return;
  const int m0 = tile_m * 256;
  const int steps = k_steps / p.splits;  // K steps of this split
  const int t0 = split * steps;
  const int halves = 2 * steps;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave >> 1;
  const int wc = wave & 1;
  const uint32_t lds0 = LdsAddress(lds);

  // DMA sources. X: this wave brings LDS rows 64 w + 16 d + l / 4 (d < 4),
  // lane l filling position l % 4 with the chunk that belongs there; rows
  // past M read row M - 1 (never stored). W: blocks 2 w and 2 w + 1 of the
  // tile, 2 KB each (two DMAs). Half-step s adds (s / 2) 128 + (s % 2) 32
  // bytes to the X base and (s / 2) 4096 + (s % 2) 2048 to the W base.
  const unsigned char* x_base =
      reinterpret_cast<const unsigned char*>(p.x) + static_cast<size_t>(t0) * 128;
  uint32_t x_off[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int row = 64 * wave + 16 * d + (lane >> 2);
    const int q = Swizzle32(row, lane & 3);
    const int chunk = (q & 1) + 4 * (q >> 1);
    x_off[d] = static_cast<uint32_t>(
        (static_cast<size_t>(min(m0 + row, p.m - 1)) * p.lda + 8 * chunk) * 2);
  }
  const unsigned char* w_base =
      reinterpret_cast<const unsigned char*>(p.w) +
      (static_cast<size_t>(tile_n * 8 + 2 * wave) * k_steps + t0) * 4096;
  const uint32_t w_off0 = static_cast<uint32_t>(lane * 16);
  const uint32_t w_off1 = w_off0 + static_cast<uint32_t>(k_steps) * 4096;

  // DMA i (< 8) of half-step s into ring slot `slot`: X rows 16 i .. of this
  // wave's 64 (i < 4), or 1 KB of W blocks 2 w + (i - 4) / 2.
  auto dma_one = [&](int slot, int s, int i) {
    const uint32_t stage = lds0 + slot * kBigHalf;
    if (i < 4) {
      DmaToLds(x_base + (s >> 1) * 128 + (s & 1) * 32, x_off[i], stage + wave * 4096 + i * 1024);
    } else {
      const unsigned char* ws = w_base + (s >> 1) * 4096 + (s & 1) * 2048 + (i & 1) * 1024;
      DmaToLds(ws, i < 6 ? w_off0 : w_off1, stage + 16384 + wave * 4096 + (i - 4) * 1024);
    }
  };
  auto dma = [&](int slot, int s) {
#pragma unroll
    for (int i = 0; i < kBigDmas; ++i)
      dma_one(slot, s, i);
  };

  // Fragment reads: X row 128 wr + 32 b + lane % 32, position 2 h + jj;
  // W block 4 wc + wb, substep jj, lane's 16 bytes.
  int x_read[XB][2];
#pragma unroll
  for (int b = 0; b < XB; ++b)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int row = 128 * wr + 32 * b + (lane & 31);
      x_read[b][jj] = row * 64 + Swizzle32(row, 2 * (lane >> 5) + jj) * 16;
    }
  const int w_read = 16384 + wc * 8192 + lane * 16;

  floatx16 acc[WB][XB];
#pragma unroll
  for (int wb = 0; wb < WB; ++wb)
#pragma unroll
    for (int b = 0; b < XB; ++b)
      acc[wb][b] = floatx16{};

  half8 fx[2][XB];  // X fragments of the current and the next substep
  half8 fw[2][WB];  // W fragments likewise
  // Fragment read r (< 8) into set f: X fragment r (r < 4) or W fragment
  // r - 4, of substep jj of ring slot `slot`.
  auto read_one = [&](int f, int slot, int jj, int r) {
    const unsigned char* stage = lds + slot * kBigHalf;
    if (r < 4)
      fx[f][r] = *reinterpret_cast<const half8*>(stage + x_read[r][jj]);
    else
      fw[f][r - 4] = *reinterpret_cast<const half8*>(stage + w_read + (r - 4) * 2048 + jj * 1024);
  };
  auto read_frag = [&](int f, int slot, int jj) {
#pragma unroll
    for (int r = 0; r < 8; ++r)
      read_one(f, slot, jj, r);
  };
  // MFMA i (< 16) of fragment set f: W block i / 4, X block i % 4.
  auto mfma_one = [&](int f, int i) {
    const int wb = i >> 2, b = i & 3;
    acc[wb][b] = kRowLanes ? Mfma32(fw[f][wb], fx[f][b], acc[wb][b])
                           : Mfma32(fx[f][b], fw[f][wb], acc[wb][b]);
  };

  // Prologue: DMAs of half-steps 0 .. 3 (indices past the last clamped:
  // in-bounds reloads never read, so every half-step issues the same DMA
  // count and the wait counts below are fixed), then half-step 0's first
  // fragments once its DMAs have landed everywhere.
  const int last = halves - 1;
  dma(0, 0);
  dma(1, min(1, last));
  dma(2, min(2, last));
  dma(3, min(3, last));
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(3 * kBigDmas) : "memory");
  read_frag(0, 0, 0);

  // Half-step s, ring slot s % 4: the 16 MFMAs of its first substep
  // (fragments in registers), each followed by one of the reads of its
  // second substep; then a barrier that waits for this wave's DMAs of
  // half-step s + 1 and its LDS reads, after which half-step s + 1 is
  // readable everywhere and slot s % 4 is read by no one; then the 16 MFMAs
  // of the second substep, each followed by one of the DMAs of half-step
  // s + 4 into slot s % 4 or one of the reads of half-step s + 1's first
  // substep. With one wave per SIMD an MFMA holds up the wave's next
  // instruction for its 32 clocks, so a memory instruction slotted between
  // two MFMAs issues in that shadow; issued in a burst, the DMAs would stall
  // the wave on a full memory queue while the matrix core idles.
  auto half_step = [&](int s, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mfma_one(0, i);
      __builtin_amdgcn_sched_barrier(0);
      if (i % 2 == 0)
        read_one(1, slot, 1, i / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(2 * kBigDmas) : "memory");
    const int next = min(s + 4, last);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      mfma_one(1, i);
      __builtin_amdgcn_sched_barrier(0);
      if (i % 2 == 0)
        dma_one(slot, next, i / 2);
      else
        read_one(0, (slot + 1) & 3, 0, i / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  int s = 0;
  for (; s + 4 <= halves; s += 4) {
    half_step(s, I0{});
    half_step(s + 1, I1{});
    half_step(s + 2, I2{});
    half_step(s + 3, I3{});
  }
  if (s < halves) {  // halves is even: two more
    half_step(s, I0{});
    half_step(s + 1, I1{});
  }
  // No DMA may land in LDS once the epilogue uses it.
  WaitLoads<0>();
  __syncthreads();

  if constexpr (EPI == Epilogue::kQkvRope) {
    BigQkvEpilogue(p, acc, m0, wr, tile_n * 8 + 4 * wc, wave, lane, lds);
  } else {
    // Each wave's head staged in its own quarter of the ring.
    WaveEpilogue<XB, WB, EPI>(p, acc, m0 + 128 * wr, split, tile_n * 8 + 4 * wc, wave, lane, lds,
                              wave * kHeadStage<XB>);
  }
}

// Packs row-major W [rows][K] into the fragment order above: half8
// number ((block K/64 + t) 4 + j) 64 + l holds W[row(block, l % 32)][64 t +
// 32 (l / 32) + 8 j .. + 7]; rows past `rows` are zero. One thread per half8.
// A float32 source is rounded to fp16 here (round to nearest even, as the
// reference's ConvertToHalf does on the host, generator.cpp:31-49).
template <typename T>
__global__ void PackWeightsKernel(const T* w, const T* w2, int rows, int k,
                                  int blocks, PackMap map, int group, half8* out) {
  const size_t total = static_cast<size_t>(blocks) * (k / 64) * 256;
  const size_t o = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (o >= total)
    return;
  const int lane = static_cast<int>(o & 63);
  const int j = static_cast<int>((o >> 6) & 3);
  const size_t bt = o >> 8;  // block * (k / 64) + t
  const int t = static_cast<int>(bt % (k / 64));
  const int block = static_cast<int>(bt / (k / 64));
  const int i = lane & 31;
  const T* src = w;
  int row = 32 * block + i;
  if (map == PackMap::kRope) {
    const int wv = block % 4;
    const int head = QkvHead(block / 4, rows / 128, group);
    row = head < 0 ? rows
                   : 128 * head + (i < 16 ? 16 * wv + i : 64 + 16 * wv + (i - 16));
  } else if (map == PackMap::kSwiGlu) {
    row = 16 * block + (i & 15);
    src = i < 16 ? w : w2;
  }
  half8 v = {};
  if (row < rows) {
    const T* p = src + static_cast<size_t>(row) * k + 64 * t + 32 * (lane >> 5) + 8 * j;
    if constexpr (sizeof(T) == 2) {
      v = *reinterpret_cast<const half8*>(p);
    } else {
      const floatx4 lo = *reinterpret_cast<const floatx4*>(p);
      const floatx4 hi = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = static_cast<half_t>(lo[e]);
        v[4 + e] = static_cast<half_t>(hi[e]);
      }
    }
  }
  out[o] = v;
}

template <int XB, Epilogue EPI, int NW>
void LaunchPackedXB(const GemmParams& p, const PackedPlan& plan, hipStream_t stream, bool first,
                    bool last) {
  const int tiles_m = (p.m + Packed<XB>::kBM - 1) / Packed<XB>::kBM;
  const int tiles_n = (p.n + 32 * NW - 1) / (32 * NW);
  const int groups = tiles_m * tiles_n * p.splits;
  Require(groups == plan.tiles * plan.splits, "gemm: grid does not match the plan");
  if ((p.k / 64 / p.splits) % 4 == 0) {
    // The q/k/v tile stages its rotary rows when the grid is one round
    // (the kernel makes the same test on its grid size).
    const int lds = groups <= kCus ? NarrowLds<XB, EPI>() : Packed<XB>::kLds;
    Dispatch(PackedGemmKernel<XB, EPI, NW>, dim3(groups), dim3(64 * NW), lds, stream, first,
             last, p, tiles_m, p.k / 64);
    return;
  }
  // K ranges that are not a multiple of 256 per split (small models).
  Dispatch(PackedGemmKernel<XB, EPI, NW, true>, dim3(groups), dim3(64 * NW), Packed<XB>::kLds,
           stream, first, last, p, tiles_m, p.k / 64);
}

template <int XB, Epilogue EPI>
void LaunchPackedNarrow(const GemmParams& p, const PackedPlan& plan, hipStream_t stream,
                        bool first, bool last) {
  if constexpr (EPI != Epilogue::kQkvRope) {
    if (plan.nw == 2) {
      LaunchPackedXB<XB, EPI, 2>(p, plan, stream, first, last);
      return;
    }
    if (plan.nw == 1) {
      LaunchPackedXB<XB, EPI, 1>(p, plan, stream, first, last);
      return;
    }
  }
  LaunchPackedXB<XB, EPI, 4>(p, plan, stream, first, last);
}

template <Epilogue EPI>
void LaunchPackedWide(const GemmParams& p, const PackedPlan& plan, hipStream_t stream, bool first,
                      bool last) {
  const int tiles_m = (p.m + 127) / 128;
  const int tiles_n = (p.n + 255) / 256;
  const int groups = tiles_m * tiles_n * p.splits;
  Require(groups == plan.tiles * plan.splits, "gemm: grid does not match the plan");
  Dispatch(PackedWideKernel<EPI>, dim3(groups), dim3(256), kWideLds, stream, first, last, p,
           tiles_m, p.k / 64);
}

template <Epilogue EPI>
void LaunchPackedBig(const GemmParams& p, const PackedPlan& plan, hipStream_t stream, bool first,
                     bool last) {
  const int tiles_m = (p.m + 255) / 256;
  const int tiles_n = (p.n + 255) / 256;
  const int groups = tiles_m * tiles_n * p.splits;
  Require(groups == plan.tiles * plan.splits, "gemm: grid does not match the plan");
  // The DMA offsets are 32-bit.
  Require((static_cast<size_t>(p.m) * p.lda + p.k) * 2 < (size_t{1} << 31) &&
              static_cast<size_t>(p.k / 64) * 2 * 4096 < (size_t{1} << 31),
          "gemm: operands too large for the 256 x 256 tile");
  Dispatch(PackedBigKernel<EPI>, dim3(groups), dim3(256),
           EPI == Epilogue::kQkvRope ? kBigQkvLds : kBigLds, stream, first, last, p, tiles_m,
           p.k / 64);
}

template <Epilogue EPI>
void LaunchPackedShape(const GemmParams& p, const PackedPlan& plan, hipStream_t stream,
                       bool first, bool last) {
  if (plan.xb == 8) {
    LaunchPackedBig<EPI>(p, plan, stream, first, last);
    return;
  }
  if (plan.wb == 2) {
    LaunchPackedWide<EPI>(p, plan, stream, first, last);
    return;
  }
  switch (plan.xb) {
    case 1: LaunchPackedNarrow<1, EPI>(p, plan, stream, first, last); break;
    case 2: LaunchPackedNarrow<2, EPI>(p, plan, stream, first, last); break;
    case 3: LaunchPackedNarrow<3, EPI>(p, plan, stream, first, last); break;
    default: LaunchPackedNarrow<4, EPI>(p, plan, stream, first, last); break;
  }
}

// One launch, or with a column split (PackedPlan::n_main) the main tile's
// launch on columns [0, n_main) and the tail tile's on the rest: W from
// packed block n_main / 32 on, outputs from column n_main (SwiGLU: act
// column n_main / 2). Every tile sums the whole K range in the same order,
// so a value does not depend on which launch computed it.
template <Epilogue EPI>
void LaunchPackedEpi(const GemmParams& p, const PackedPlan& plan, hipStream_t stream) {
  if (plan.n_main == 0) {
    LaunchPackedShape<EPI>(p, plan, stream, true, true);
    return;
  }
  Require(plan.splits == 1 && EPI != Epilogue::kQkvRope && EPI != Epilogue::kPartial &&
              plan.n_main % 256 == 0 && plan.n_main < p.n,
          "gemm: column split only for unsplit store, accumulate and SwiGLU epilogues");
  GemmParams head = p;
  head.n = plan.n_main;
  LaunchPackedShape<EPI>(head, plan, stream, true, false);
  GemmParams tail = p;
  tail.n = p.n - plan.n_main;
  tail.w = p.w + static_cast<std::size_t>(plan.n_main) * p.k;
  if constexpr (EPI == Epilogue::kSwiGlu)
    tail.act = p.act + plan.n_main / 2;
  else
    tail.y = p.y + plan.n_main;
  PackedPlan t;
  t.xb = plan.tail_xb;
  t.wb = plan.tail_wb;
  t.nw = plan.tail_nw;
  t.tiles = plan.tail_tiles;
  LaunchPackedShape<EPI>(tail, t, stream, false, true);
}

}  // namespace

std::size_t PackedWeightHalves(int rows, int k) {
  return static_cast<std::size_t>((rows + 255) / 256 * 256) * k;
}

template <typename T>
void PackWeightsAny(const T* w, const T* w2, int rows, int k, PackMap map, int group,
                    half_t* out, hipStream_t stream) {
  Require(k % 64 == 0 && rows > 0, "pack: K must be a positive multiple of 64");
  Require(map != PackMap::kRope || (group > 0 && rows % 128 == 0 && (rows / 128) % (group + 2) == 0),
          "pack: q/k/v packing needs (group + 2) kv groups of 128-row heads");
  Require(map != PackMap::kSwiGlu || w2 != nullptr, "pack: SwiGLU packing needs gate and up");
  // Blocks of 32 columns, padded to whole 256-column tiles.
  const int out_rows = map == PackMap::kSwiGlu ? 2 * rows : rows;
  const int blocks = (out_rows + 255) / 256 * 8;
  const size_t total = static_cast<size_t>(blocks) * (k / 64) * 256;
  const int threads = 256;
  PackWeightsKernel<T><<<static_cast<unsigned>((total + threads - 1) / threads), threads, 0,
                         stream>>>(w, w2, rows, k, blocks, map, group,
                                   reinterpret_cast<half8*>(out));
  Check(hipGetLastError(), "pack launch");
}

void PackWeights(const half_t* w, const half_t* w2, int rows, int k, PackMap map, int group,
                 half_t* out, hipStream_t stream) {
  PackWeightsAny(w, w2, rows, k, map, group, out, stream);
}

void PackWeights(const float* w, const float* w2, int rows, int k, PackMap map, int group,
                 half_t* out, hipStream_t stream) {
  PackWeightsAny(w, w2, rows, k, map, group, out, stream);
}

PackedPlan PlanPacked(int m, int n, int k, Epilogue epilogue) {
  PackedPlan plan;
  const int k_steps = k / 64;
  plan.splits = epilogue == Epilogue::kPartial ? PartialSplits(k_steps) : 1;
  const int steps = k_steps / plan.splits;
  // Cycles per K step of one work-group, the largest of: the operands it
  // pulls from L2 (32 XB rows of X and 128 WB columns of W, 128 bytes each,
  // at 64 bytes per clock), its LDS traffic (X written once and read by
  // four waves, at 128 bytes per clock) and its MFMAs (XB WB 4 per SIMD, 32
  // clocks each); plus about 3200 clocks a tile (first loads, epilogue).
  // Estimated time: rounds of work-groups over the CUs times that, where a
  // last, partial round counts by its share of the CUs but at least half a
  // round (fewer work-groups at once run faster each, but a few stragglers
  // still cost most of a round: the 10 s audio heads run 20.4 us as 390
  // 96-row tiles, 1.5 rounds, against 23.1 us as 132 wide tiles).
  // The 256 x 256 tile (xb 8, wb 2) is priced by measurement instead: with
  // every CU busy a K step takes it 1.45 times as long as the 128 x 256
  // tile's (q/k/v at 3440 rows: 26.5 us of K loop in one round against
  // 36.6 us in 1.7 rounds of the 128 x 256 tile), i.e. 1500 of these clocks.
  // Two- and one-wave tiles ((32 XB) x 64 or x 32, nw 2 or 1) are priced
  // the same way: 64 or 32 columns of W per K step, X read by two waves or
  // one. They come after the four-wave tiles, which win ties.
  struct Shape {
    int xb, wb, nw;
  };
  // The cheapest shape for n columns (the 256 x 256 tile only if `big`).
  auto search = [&](int cols_n, bool big, PackedPlan* out) {
    double best = 0.0;
    for (const Shape sh :
         {Shape{8, 2, 4}, Shape{4, 2, 4}, Shape{4, 1, 4}, Shape{3, 1, 4}, Shape{2, 1, 4},
          Shape{1, 1, 4}, Shape{4, 1, 2}, Shape{3, 1, 2}, Shape{2, 1, 2}, Shape{1, 1, 2},
          Shape{2, 1, 1}, Shape{1, 1, 1}}) {
      // The 256 x 256 tile's DMA offsets are 32-bit (X of the generator's
      // GEMMs is [m][k]).
      if (sh.xb == 8 && (!big || static_cast<size_t>(m) * k * 2 >= (size_t{1} << 31)))
        continue;
      if (sh.nw < 4 && epilogue == Epilogue::kQkvRope)
        continue;
      const int cols = 32 * sh.nw * sh.wb;
      const int tiles =
          (m + 32 * sh.xb - 1) / (32 * sh.xb) * ((cols_n + cols - 1) / cols) * plan.splits;
      const int full = tiles / kCus, rest = tiles % kCus;
      const double rounds =
          full == 0 ? 1.0
                    : full + (rest == 0 ? 0.0 : std::max(0.5, static_cast<double>(rest) / kCus));
      const double l2 = (32.0 * sh.xb + cols) * 128.0 / 64.0;
      const double lds = (1.0 + sh.nw) * 32.0 * sh.xb * 128.0 / 128.0;
      const double mfma = 4.0 * sh.xb * sh.wb * 32.0;
      const double step = sh.xb == 8 ? 1500.0 : std::max(l2, std::max(lds, mfma));
      const double cost = rounds * (static_cast<double>(steps) * step + 3200.0);
      if (best == 0.0 || cost < best) {
        best = cost;
        out->xb = sh.xb;
        out->wb = sh.wb;
        out->nw = sh.nw;
        out->tiles = tiles / plan.splits;
      }
    }
  };
  search(n, true, &plan);
  // A 256 x 256 grid of between one and two rounds whose second round is
  // at most half full runs those few work-groups at nearly a whole tile's
  // time while the other CUs idle (gate/up at 3440 rows: 336 work-groups,
  // 54 us against 37 for the one-round q/k/v of the same K). Where the
  // epilogue allows a column offset, the tile then covers one round of
  // column tiles and a second launch the remaining columns with the
  // cheapest smaller tile (gate/up 54.0 -> 51.1 us; a 128 x 256 tail 52.1).
  // With a fuller second round the second launch costs more than it saves
  // (the audio heads at 3000 x 8200, 396 work-groups: 77 -> 84.5 us). The
  // smaller tiles fit two work-groups per CU, so their grids of up to two
  // rounds run at once (q/k/v at 1072 rows, 384 work-groups of 96 x 128:
  // 19.1 us, against 24.3 split as 252 + 187 work-groups).
  if (plan.xb == 8 && plan.splits == 1 &&
      (epilogue == Epilogue::kStore || epilogue == Epilogue::kAccumulate ||
       epilogue == Epilogue::kSwiGlu)) {
    const int tiles_m = (m + 255) / 256;
    const int tiles_n = (n + 255) / 256;
    const int full = plan.tiles / kCus;
    const int main_n = full * kCus / tiles_m;
    const int rest = plan.tiles % kCus;
    if (full == 1 && rest != 0 && 2 * rest <= kCus && main_n >= 1 && main_n < tiles_n) {
      PackedPlan tail;
      search(n - 256 * main_n, false, &tail);
      plan.n_main = 256 * main_n;
      plan.tiles = tiles_m * main_n;
      plan.tail_xb = tail.xb;
      plan.tail_wb = tail.wb;
      plan.tail_nw = tail.nw;
      plan.tail_tiles = tail.tiles;
    }
  }
  return plan;
}

void LaunchPacked(const GemmParams& p, const PackedPlan& plan, Epilogue epilogue,
                  hipStream_t stream) {
  Require(p.m > 0 && p.n > 0 && p.k > 0, "gemm: empty shape");
  Require(p.k % 64 == 0, "gemm: K must be a multiple of 64");
  Require(p.splits == plan.splits && (p.k / 64) % p.splits == 0,
          "gemm: K steps not divisible by the split count");
  Require(p.lda % 8 == 0, "gemm: the row stride of X must be a multiple of 8");
  Require((plan.xb >= 1 && plan.xb <= 4 && (plan.wb == 1 || (plan.wb == 2 && plan.xb == 4))) ||
              (plan.xb == 8 && plan.wb == 2),
          "gemm: tile of 32 to 128 rows x 128 columns, 128 x 256 or 256 x 256");
  Require(plan.nw == 4 || ((plan.nw == 2 || plan.nw == 1) && plan.wb == 1 && plan.xb <= 4 &&
                           epilogue != Epilogue::kQkvRope),
          "gemm: two- and one-wave tiles are 32 to 128 rows x 64 or 32 columns, not for q/k/v");
  switch (epilogue) {
    case Epilogue::kStore:
    case Epilogue::kAccumulate:
    case Epilogue::kPartial:
      Require(epilogue != Epilogue::kPartial ||
                  (p.y != nullptr && p.split_stride >= static_cast<std::size_t>(p.m) * p.ldc),
              "gemm: partial slices overlap");
      if (epilogue == Epilogue::kStore)
        LaunchPackedEpi<Epilogue::kStore>(p, plan, stream);
      else if (epilogue == Epilogue::kAccumulate)
        LaunchPackedEpi<Epilogue::kAccumulate>(p, plan, stream);
      else
        LaunchPackedEpi<Epilogue::kPartial>(p, plan, stream);
      break;
    case Epilogue::kQkvRope:
      Require(p.n == (p.heads + 2 * p.kv_heads) * 128,
              "gemm: q/k/v epilogue needs N = (heads + 2 kv_heads) * 128");
      Require(p.ldvt % 16 == 0 && p.ldq % 128 == 0 &&
                  static_cast<int64_t>(p.ldq) >= static_cast<int64_t>(p.m) * 128,
              "gemm: q/k/v output strides");
      LaunchPackedEpi<Epilogue::kQkvRope>(p, plan, stream);
      break;
    case Epilogue::kSwiGlu:
      Require(p.n % 128 == 0 && p.ldh % 4 == 0, "gemm: SwiGLU epilogue needs N % 128 == 0");
      LaunchPackedEpi<Epilogue::kSwiGlu>(p, plan, stream);
      break;
  }
  Check(hipGetLastError(), "gemm launch");
}

}  // namespace ovg
