// Bidirectional grouped-query attention over packed sequences on gfx950
// matrix cores: replaces State::Attention's two batched GEMMs, the
// materialised [heads][L][L] scores, SoftmaxKernel and MergeHeadsKernel of
// the reference (generator.cpp:122-172, kernels/generator_kernels.hip:
// 161-189). Scores never leave registers.
//
// A work-group takes one tile of 32 queries of one sequence and one key/value
// head g. Its 2 x GROUP waves are the GROUP query heads of g times two key
// halves: keys are staged in LDS as pairs of 32-key tiles (K [32][128] and
// V^T [128][32] each), the first tile of a pair for key-half 0, the second
// for key-half 1, so each K/V tile is read from memory once for the whole
// head group (no GQA repeat). The next pair is prefetched into registers
// while the current one is used (double-buffered LDS, one barrier per pair).
// At the end the two key halves' online-softmax states merge through LDS.
//
// Scores are formed transposed, S^T = K Q^T (keys as MFMA rows, queries as
// columns), so that every lane owns one query column: the running max and
// sum are per-lane values combined with the partner lane l ^ 32 only. The
// value product is likewise transposed, O^T = V^T P^T: P^T is the score
// accumulator itself converted to fp16 (the MFMA's k order is permuted to
// the accumulator's row order, and V^T is read from LDS in the same order),
// so probabilities never move between lanes. V^T comes pre-transposed from
// the q/k/v GEMM's epilogue ([kv head][dim][row]).
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kKTile = 32;
constexpr int kHeadDim = 128;
constexpr int kKPitch = kHeadDim + 8;  // halves per key row in LDS
constexpr int kVPitch = kKTile + 8;    // halves per dim row of V^T in LDS
constexpr int kKHalves = kKTile * kKPitch;
constexpr int kVHalves = kHeadDim * kVPitch;
constexpr int kTileHalves = kKHalves + kVHalves;  // one staged key tile
constexpr int kChunksPerTile = 2 * kKTile * kHeadDim / 8;  // K + V^T, 16 B

template <int GROUP>
__global__ __launch_bounds__(GROUP * 128) void AttentionKernel(
    AttentionParams p) {
  constexpr int kThreads = GROUP * 128;
  constexpr int kChunks = 2 * kChunksPerTile / kThreads;  // per thread per pair
  // Two buffers of a tile pair; the merge area reuses them.
  __shared__ __align__(16) half_t lds[2 * 2 * kTileHalves];
  const AttentionWork work = p.work[blockIdx.x];
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int head_local = wave % GROUP;
  const int key_half = wave / GROUP;
  const int head = g * GROUP + head_local;
  const int half_id = lane >> 5;
  const int col = lane & 31;

  // Q^T operand: lane supplies dims 16 kk + 8 half_id .. +7 of query col.
  half8 qf[8];
  {
    const bool valid = col < work.q_count;
    const half_t* q = p.qk + static_cast<size_t>(work.q_begin + col) * p.ld_qk +
                      head * kHeadDim + half_id * 8;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = valid ? *reinterpret_cast<const half8*>(q + kk * 16)
                     : half8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  floatx16 ot[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    ot[dt] = floatx16{};
  float run_max = -__builtin_inff();
  float run_sum = 0.0F;

  const half_t* kbase = p.qk + (p.heads + g) * kHeadDim;
  const half_t* vbase = p.vt + static_cast<size_t>(g) * kHeadDim * p.ldvt;
  const int tiles = (work.seq_length + kKTile - 1) / kKTile;
  const int pairs = (tiles + 1) / 2;

  // Chunk c of a pair: tile c / kChunksPerTile; within a tile the first 512
  // chunks are K rows (16 per key), the rest V^T rows (4 per dim).
  half8 staged[kChunks];
  auto load = [&](int pair) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * kThreads;
      const int t = 2 * pair + c / kChunksPerTile;
      const int ci = c % kChunksPerTile;
      const int key0 = work.seq_begin + t * kKTile;
      if (t >= tiles)
        continue;
      if (ci < kChunksPerTile / 2) {
        staged[j] = *reinterpret_cast<const half8*>(
            kbase + static_cast<size_t>(key0 + (ci >> 4)) * p.ld_qk + (ci & 15) * 8);
      } else {
        const int cv = ci - kChunksPerTile / 2;
        staged[j] = *reinterpret_cast<const half8*>(
            vbase + static_cast<size_t>(cv >> 2) * p.ldvt + key0 + (cv & 3) * 8);
      }
    }
  };
  auto store = [&](int pair, int buffer) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int c = tid + j * kThreads;
      const int slot = c / kChunksPerTile;
      const int ci = c % kChunksPerTile;
      if (2 * pair + slot >= tiles)
        continue;
      half_t* tile_lds = lds + (buffer * 2 + slot) * kTileHalves;
      if (ci < kChunksPerTile / 2) {
        *reinterpret_cast<half8*>(tile_lds + (ci >> 4) * kKPitch + (ci & 15) * 8) =
            staged[j];
      } else {
        const int cv = ci - kChunksPerTile / 2;
        *reinterpret_cast<half8*>(tile_lds + kKHalves + (cv >> 2) * kVPitch +
                                  (cv & 3) * 8) = staged[j];
      }
    }
  };

  load(0);
  store(0, 0);
  __syncthreads();
  for (int pair = 0; pair < pairs; ++pair) {
    if (pair + 1 < pairs)
      load(pair + 1);
    const int t = 2 * pair + key_half;
    if (t < tiles) {
      const half_t* ks = lds + ((pair & 1) * 2 + key_half) * kTileHalves;
      const half_t* vs = ks + kKHalves;
      floatx16 s = floatx16{};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const half8 kf = *reinterpret_cast<const half8*>(
            ks + col * kKPitch + kk * 16 + half_id * 8);
        s = Mfma32(kf, qf[kk], s);
      }
      // Lane holds keys 8 (r / 4) + 4 half_id + r % 4 of its query column.
      const int valid_keys = work.seq_length - t * kKTile;
      float tile_max = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r / 4) + 4 * half_id + (r & 3);
        s[r] = key < valid_keys ? s[r] * p.scale_log2 : -__builtin_inff();
        tile_max = fmaxf(tile_max, s[r]);
      }
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
      const float new_max = fmaxf(run_max, tile_max);
      const float alpha = __builtin_amdgcn_exp2f(run_max - new_max);
      run_max = new_max;
      float psum = 0.0F;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - new_max);
        psum += s[r];
      }
      run_sum = run_sum * alpha + psum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        ot[dt] *= alpha;
      // P^T operand for keys 16 j2 .. 16 j2 + 15: slot e <-> accumulator
      // element 8 j2 + e, i.e. key 16 j2 + (e < 4 ? 4 h + e : 8 + 4 h + e - 4).
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        half8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pb[e] = static_cast<half_t>(s[8 * j2 + e]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const half_t* vrow = vs + (dt * 32 + col) * kVPitch + 16 * j2 + 4 * half_id;
          const half4 lo = *reinterpret_cast<const half4*>(vrow);
          const half4 hi = *reinterpret_cast<const half4*>(vrow + 8);
          const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          ot[dt] = Mfma32(va, pb, ot[dt]);
        }
      }
    }
    if (pair + 1 < pairs)
      store(pair + 1, (pair + 1) & 1);
    __syncthreads();
  }

  // Merge the key halves: half 1 leaves (max, sum, O) per lane in LDS.
  float* merge = reinterpret_cast<float*>(lds);
  float* mine = merge + (head_local * 64 + lane) * 66;
  if (key_half == 1) {
    mine[0] = run_max;
    mine[1] = run_sum;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        mine[2 + dt * 16 + r] = ot[dt][r];
  }
  __syncthreads();
  if (key_half == 1)
    return;
  const float other_max = mine[0];
  const float new_max = fmaxf(run_max, other_max);
  const float a0 = __builtin_amdgcn_exp2f(run_max - new_max);
  const float a1 = __builtin_amdgcn_exp2f(other_max - new_max);
  const float sum = run_sum * a0 + mine[1] * a1;
  const float total = sum + __shfl_xor(sum, 32);
  const float inverse = 1.0F / total;
  if (col >= work.q_count)
    return;
  half_t* out = p.out + static_cast<size_t>(work.q_begin + col) * p.heads * kHeadDim +
                head * kHeadDim;
  // O^T accumulator dt: lane holds dims dt*32 + 8 (r / 4) + 4 half_id + r % 4.
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      half4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * q + e;
        v[e] = static_cast<half_t>(
            (ot[dt][r] * a0 + mine[2 + dt * 16 + r] * a1) * inverse);
      }
      *reinterpret_cast<half4*>(out + dt * 32 + 8 * q + 4 * half_id) = v;
    }
}

}  // namespace

void LaunchAttention(const AttentionParams& p, hipStream_t stream) {
  Require(p.work_count > 0, "attention: no work");
  Require(p.kv_heads > 0 && p.heads % p.kv_heads == 0,
          "attention: heads must be a multiple of kv_heads");
  Require(p.ld_qk % 8 == 0 && p.ldvt % 8 == 0,
          "attention: leading dimensions must be multiples of 8");
  const int group = p.heads / p.kv_heads;
  const dim3 grid(p.work_count, p.kv_heads);
  switch (group) {
    case 1:
      AttentionKernel<1><<<grid, dim3(128), 0, stream>>>(p);
      break;
    case 2:
      AttentionKernel<2><<<grid, dim3(256), 0, stream>>>(p);
      break;
    case 4:
      AttentionKernel<4><<<grid, dim3(512), 0, stream>>>(p);
      break;
    default:
      throw Error("attention: query heads per kv head must be 1, 2 or 4");
  }
  Check(hipGetLastError(), "attention launch");
}

}  // namespace ovg
