// Bidirectional grouped-query attention over packed sequences on gfx950
// matrix cores: replaces State::Attention's two batched GEMMs, the
// materialised [heads][L][L] scores, SoftmaxKernel and MergeHeadsKernel of
// the reference (generator.cpp:122-172, kernels/generator_kernels.hip:
// 161-189). Scores never leave registers.
//
// A work-group takes one tile of 32 queries of one sequence and one key/value
// head g, with 4 x GROUP waves (the GROUP query heads of g times four key
// quarters). Keys come in 32-key tiles (K [32][128] and V^T 2 x [128][16],
// 16 KB), fetched global -> LDS by DMA into an 8-slot ring, four tiles (a
// round) at a time, quarter q taking tile 4 r + q of round r. The queries
// and rounds 0 and 1 (both ring halves are free at the start) are fetched
// by all compute waves, an equal share each: the 144 one-KB DMAs would
// stall a single wave, whose wait counter tracks at most 63 loads. Later
// rounds come from one extra producer wave, so that no compute wave blocks
// on a full memory queue between rounds: round r + 2 as soon as barrier
// r + 1 frees round r's half of the ring. Each tile is read from memory once
// for the whole head group (no GQA repeat), and the group's query tiles come
// into LDS the same way, once. At
// the end every wave leaves its online-softmax state in LDS and wave
// (head, quarter q) merges the four quarters' states for dims 32 q .. 32 q +
// 31 of its head in a fixed order, ((0 + 1) + (2 + 3)), and stores them.
//
// Scores are formed transposed, S^T = K Q^T (keys as MFMA rows, queries as
// columns), so that every lane owns one query column: the running max and
// sum are per-lane values combined with the partner lane l ^ 32 only. The
// value product is likewise transposed, O^T = V^T P^T: P^T is the score
// accumulator itself converted to fp16, so probabilities never move between
// lanes. Lane half h holds keys {4h..4h+3, 8+4h..8+4h+3} of each 16-key
// block; V^T arrives from the q/k/v epilogue with the keys of every 16-row
// block stored in the order 0-3, 8-11, 4-7, 12-15 (VtColumn), which makes
// those eight keys one 16-byte run.
//
// A V^T tile is two 16-key blocks of [128 dims][16 keys] (VtIndex), 8 KB of
// consecutive bytes in memory, copied verbatim into LDS; a lane's 16-byte
// operand is half of one dim's row of a block, and the 64 lanes of one read
// cover 1 KB of consecutive LDS. K rows are XOR-swizzled in 16-byte chunks
// (chunk ^ (key & 15)), so both operand reads are conflict-free.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "kernels.hpp"

// No floating-point contraction in this file: every fused multiply-add is
// written out, so that the kernel's instantiations (the number of key rounds
// held in registers) round a query's values identically.
#pragma clang fp contract(off)

namespace ovg {
namespace {

constexpr int kKTile = 32;
constexpr int kHeadDim = 128;
constexpr int kTileBytes = 16384;  // K (8 KB) then V^T (8 KB)
constexpr int kSlots = 8;          // ring of 32-key tiles
constexpr int kRound = 4;          // tiles per round = key quarters
constexpr int kRingBytes = kSlots * kTileBytes;
constexpr int kQBytes = 8192;      // one head's 32 x 128 query tile

// Ring, then the group's query tiles; the merge reuses the space for every
// wave's (max, sum) pairs and O^T accumulators (16 float4 per lane).
template <int GROUP>
constexpr int AttentionLds() {
  const int ring = kRingBytes + GROUP * kQBytes;
  const int merge = 4 * GROUP * 64 * (8 + 16 * 16);
  return ring > merge ? ring : merge;
}

// Barrier without the fence of __syncthreads(), which would wait for every
// DMA in flight.
__device__ __forceinline__ void RingBarrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" : : : "memory");
}

struct State {
  float max, sum;
  floatx16 o[4];  // O^T: lane holds dims 32 dt + 8 (r / 4) + 4 h + r % 4
};

// One quarter's state restricted to a 32-dim slice.
struct Slice {
  float max, sum;
  floatx16 o;
};

// a then b: a state with max -inf is empty and weighs zero.
__device__ __forceinline__ Slice Merge(const Slice& a, const Slice& b) {
  const float m = fmaxf(a.max, b.max);
  const float wa = a.max == -__builtin_inff() ? 0.0F : __builtin_amdgcn_exp2f(a.max - m);
  const float wb = b.max == -__builtin_inff() ? 0.0F : __builtin_amdgcn_exp2f(b.max - m);
  Slice c;
  c.max = m;
  c.sum = a.sum * wa + b.sum * wb;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    c.o[r] = a.o[r] * wa + b.o[r] * wb;
  return c;
}

// The prefetch work-groups: each thread keeps eight 16-byte loads in
// flight (clamped in bounds, no load under a condition) and folds them into
// a value that is never stored, so only the cache fill remains.
__device__ __forceinline__ void PrefetchRanges(const AttentionParams& p, int group) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kInFlight = 8;
  const unsigned long long stride = static_cast<unsigned long long>(p.prefetch_groups) * blockDim.x;
  unsigned int fold = 0;
  for (int r = 0; r < AttentionParams::kMaxPrefetch; ++r) {
    const unsigned long long chunks = p.prefetch_bytes[r] / 16;
    if (chunks == 0)
      continue;
    const u32x4* src = reinterpret_cast<const u32x4*>(p.prefetch[r]);
    for (unsigned long long c = static_cast<unsigned long long>(group) * blockDim.x + threadIdx.x;
         c < chunks; c += kInFlight * stride) {
      u32x4 v[kInFlight];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        v[k] = src[min(c + k * stride, chunks - 1)];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        fold ^= v[k].x;
    }
  }
  // Never true (prefetch_groups > 0 here); keeps the loads alive.
  if (fold == 0x9e3779b9u && p.prefetch_groups < 0)
    p.out[0] = static_cast<half_t>(0.0F);
}

template <int GROUP>
__global__ __launch_bounds__((4 * GROUP + 1) * 64) void AttentionKernel(
    AttentionParams p) {
  if (static_cast<int>(blockIdx.x) >= p.work_count * p.kv_heads) {
    PrefetchRanges(p, static_cast<int>(blockIdx.x) - p.work_count * p.kv_heads);
    return;
  }
  constexpr int kWaves = 4 * GROUP;  // compute waves; wave kWaves: producer
  constexpr int kShare = 64 / kWaves;       // DMAs per wave and round
  constexpr int kQShare = 8 * GROUP / kWaves;  // query DMAs per wave
  static_assert(kShare % 8 == 0, "a share covers whole 8 KB halves of a tile");
  extern __shared__ __align__(16) unsigned char lds[];
  // Work-groups go round-robin over the 8 XCDs: block b takes kv head
  // b % kv_heads, so with 8 kv heads each XCD's L2 holds one head's keys,
  // values and queries only.
  const int g = blockIdx.x % p.kv_heads;
  const AttentionWork work = p.work[blockIdx.x / p.kv_heads];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head_local = wave % GROUP;
  const int quarter = wave / GROUP;
  const int head = g * GROUP + head_local;
  const int half_id = lane >> 5;
  const int col = lane & 31;
  const int tiles = (work.seq_length + kKTile - 1) / kKTile;
  const int rounds = (tiles + kRound - 1) / kRound;

  // DMA plan: instruction i of a round (64 of them) loads 1 KB of tile
  // 4 r + i / 16; part (i / 8) % 2 is K or V^T, sub = i % 8 its 1 KB block.
  // Rounds 0 and 1: compute wave w issues instructions kShare w ..
  // kShare (w + 1) - 1; later rounds: the producer issues all 64. Tiles past
  // the sequence reload its last tile.
  const unsigned char* k_base = reinterpret_cast<const unsigned char*>(
      p.qk + static_cast<size_t>(p.heads + g) * p.ld_qk);
  const unsigned char* v_base = reinterpret_cast<const unsigned char*>(
      p.vt + static_cast<size_t>(g) * kHeadDim * p.ldvt);
  // Lane offsets: K row 4 sub + lane / 16 at swizzled chunk; V^T bytes
  // 16 lane of the tile's 1 KB block sub.
  uint32_t k_lane[8];
#pragma unroll
  for (int sub = 0; sub < 8; ++sub) {
    const int key = 4 * sub + (lane >> 4);
    const int chunk = (lane & 15) ^ (key & 15);
    k_lane[sub] = static_cast<uint32_t>((lane >> 4) * kHeadDim + 8 * chunk) * 2;
  }
  const uint32_t v_lane = static_cast<uint32_t>(lane) * 16;
  const uint32_t lds_base = LdsAddress(lds);
  // The r-th round processed is key round (r + shift) % rounds: the query
  // tiles of a sequence start on different rounds, so they do not all pull
  // the same L2 lines at once. Its tiles go to ring half r % 2. The shift
  // is the query tile's index inside its own sequence, so a query's order of
  // accumulation does not depend on what else is packed in the batch.
  const int shift = ((work.q_begin - work.seq_begin) / kKTile) % rounds;
  auto round_of = [&](int r) {
    const int k = r + shift;
    return k >= rounds ? k - rounds : k;
  };
  auto issue = [&](int r, int first, auto count) {
    const int round = round_of(r);
#pragma unroll
    for (int j = 0; j < decltype(count)::value; ++j) {
      const int i = first + j;
      const int slot_in_round = i / 16;
      const int part = (i / 8) & 1;
      const int sub = j & 7;  // = i & 7: first is a multiple of 8
      const int t = min(round * kRound + slot_in_round, tiles - 1);
      const int key0 = work.seq_begin + t * kKTile;
      const uint32_t dst = lds_base + ((r & 1) * kRound + slot_in_round) * kTileBytes +
                           part * 8192 + sub * 1024;
      if (part == 0) {
        DmaToLds(k_base + static_cast<size_t>(key0 + 4 * sub) * kHeadDim * 2,
                 k_lane[sub], dst);
      } else {
        DmaToLds(v_base + static_cast<size_t>(key0 >> 4) * 4096 + sub * 1024, v_lane, dst);
      }
    }
  };

  using Share = std::integral_constant<int, kShare>;
  using Round = std::integral_constant<int, 64>;
  if (wave == kWaves) {
    // The producer: round r + 2 once barrier r + 1 has freed its ring half,
    // and waits for it before barrier r + 2. Its barriers pair one to one
    // with the compute waves'.
    RingBarrier();
    for (int r = 0; r < rounds; ++r) {
      if (r + 1 >= 2 && r + 1 < rounds)
        WaitLoads<0>();
      RingBarrier();
      if (r + 2 < rounds)
        issue(r + 2, 0, Round{});
    }
    __syncthreads();
    __syncthreads();
    return;
  }
  // The group's query tiles (laid out like a K tile; query rows past the
  // tile's count repeat its last row, whose results are never stored), then
  // rounds 0 and 1.
#pragma unroll
  for (int j = 0; j < kQShare; ++j) {
    const int i = wave * kQShare + j;
    const int h = i >> 3, sub = i & 7;
    const int row = min(4 * sub + (lane >> 4), work.q_count - 1);
    const int chunk = (lane & 15) ^ ((4 * sub + (lane >> 4)) & 15);
    DmaToLds(reinterpret_cast<const unsigned char*>(
                 p.qk + static_cast<size_t>(g * GROUP + h) * p.ld_qk +
                 static_cast<size_t>(work.q_begin) * kHeadDim),
             static_cast<uint32_t>(row * kHeadDim + 8 * chunk) * 2,
             lds_base + kRingBytes + h * kQBytes + sub * 1024);
  }
  issue(0, wave * kShare, Share{});
  if (rounds > 1) {
    issue(1, wave * kShare, Share{});
    WaitLoads<kShare>();  // this wave's queries and round 0 landed
  } else {
    WaitLoads<0>();
  }
  State st;
  st.max = -__builtin_inff();
  st.sum = 0.0F;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    st.o[dt] = floatx16{};

  // Stage-invariant LDS read offsets.
  int k_read[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    k_read[kk] = col * 256 + (((2 * kk + half_id) ^ (col & 15)) * 16);
  int v_read[4][2];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j2 = 0; j2 < 2; ++j2)
      v_read[dt][j2] = 8192 + j2 * 4096 + (32 * dt + col) * 32 + half_id * 16;

  // Barrier r: round r has landed (every wave waited for its share) and
  // every wave is done with round r - 1, whose ring half then takes round
  // r + 1.
  RingBarrier();
  // Q^T operand: lane supplies dims 16 kk + 8 half_id .. +7 of query col.
  half8 qf[8];
  {
    const unsigned char* qs = lds + kRingBytes + head_local * kQBytes;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[kk] = *reinterpret_cast<const half8*>(qs + k_read[kk]);
  }
  for (int r = 0; r < rounds; ++r) {
    const int t = round_of(r) * kRound + quarter;
    if (t < tiles) {
      const unsigned char* tile = lds + ((r & 1) * kRound + quarter) * kTileBytes;
      floatx16 s = floatx16{};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        s = Mfma32(*reinterpret_cast<const half8*>(tile + k_read[kk]), qf[kk], s);
      // Lane holds keys 8 (r / 4) + 4 half_id + r % 4 of its query column.
      const int valid_keys = work.seq_length - t * kKTile;
      float tile_max = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = 8 * (e / 4) + 4 * half_id + (e & 3);
        s[e] = key < valid_keys ? s[e] * p.scale_log2 : -__builtin_inff();
        tile_max = fmaxf(tile_max, s[e]);
      }
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
      const float new_max = fmaxf(st.max, tile_max);
      const float alpha = __builtin_amdgcn_exp2f(st.max - new_max);
      st.max = new_max;
      float psum = 0.0F;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[e] = __builtin_amdgcn_exp2f(s[e] - new_max);
        psum += s[e];
      }
      st.sum = st.sum * alpha + psum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        st.o[dt] *= alpha;
      // P^T operand for keys 16 j2 .. 16 j2 + 15: slot e is accumulator
      // element 8 j2 + e; V^T's permuted block order puts the same keys in
      // the 16 bytes at position 8 half_id of the block.
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        half8 pb;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pb[e] = static_cast<half_t>(s[8 * j2 + e]);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          st.o[dt] = Mfma32(*reinterpret_cast<const half8*>(tile + v_read[dt][j2]),
                            pb, st.o[dt]);
      }
    }
    if (r == 0 && rounds > 1)
      WaitLoads<0>();  // this wave's share of round 1
    RingBarrier();     // barrier r + 1
  }

  // Every wave leaves (max, sum) as a float2 and the three dim slices of
  // O^T that other waves merge (4 float4 per lane each); wave (head,
  // quarter) then merges dims 32 quarter .. +31 of its head, its own
  // quarter's part straight from registers.
  float2* pairs = reinterpret_cast<float2*>(lds);
  floatx4* accs = reinterpret_cast<floatx4*>(lds + kWaves * 64 * 8);
  __syncthreads();
  pairs[wave * 64 + lane] = float2{st.max, st.sum};
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    if (dt == quarter)
      continue;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      accs[(wave * 16 + dt * 4 + k) * 64 + lane] =
          floatx4{st.o[dt][4 * k], st.o[dt][4 * k + 1], st.o[dt][4 * k + 2],
                  st.o[dt][4 * k + 3]};
  }
  __syncthreads();
  const int dt = quarter;
  // This wave's own slice, selected without indexing the register array by
  // a runtime value.
  const floatx16 own = dt == 0 ? st.o[0] : dt == 1 ? st.o[1] : dt == 2 ? st.o[2] : st.o[3];
  auto load = [&](int q) {
    const int w = q * GROUP + head_local;
    const float2 ms = pairs[w * 64 + lane];
    Slice sl;
    sl.max = ms.x;
    sl.sum = ms.y;
    if (q == quarter) {
      sl.o = own;
      return sl;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const floatx4 v = accs[(w * 16 + dt * 4 + k) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sl.o[4 * k + i] = v[i];
    }
    return sl;
  };
  const Slice final_state = Merge(Merge(load(0), load(1)), Merge(load(2), load(3)));
  const float total = final_state.sum + __shfl_xor(final_state.sum, 32);
  const float inverse = 1.0F / total;
  if (col >= work.q_count)
    return;
  half_t* out = p.out + static_cast<size_t>(work.q_begin + col) * p.heads * kHeadDim +
                head * kHeadDim + dt * 32;
  // Lane holds dims 8 (r / 4) + 4 half_id + r % 4 of the slice.
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    half4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = static_cast<half_t>(final_state.o[4 * q + e] * inverse);
    *reinterpret_cast<half4*>(out + 8 * q + 4 * half_id) = v;
  }
}

// ------------------------------------------------------------ exact kernel
// Sequences of at most kExactKeys keys take a two-pass softmax with every
// score in registers, which is the reference's own order of operations
// (SoftmaxKernel, kernels/generator_kernels.hip:161-176): the exact row
// maximum and sum over all keys first, then the probabilities normalised
// and rounded to fp16, then O = P V with fp32 accumulation. Nothing is
// rescaled while keys stream, and the key quarters' partial outputs merge
// as a plain sum.
//
// One work-group per (32-query tile, kv head): 4 x GROUP compute waves,
// wave (head h, quarter q) taking key tiles q, q + 4, q + 8, ..., and one
// producer wave. A key round is four K tiles (one per quarter), a value
// round the four matching V^T tiles: R = ceil(tiles / 4) key rounds, then
// R value rounds, through one ring of four rounds (4 x 4 x 8 KB). Only
// tiles inside the sequence are fetched. The compute waves fetch the
// queries and the first four rounds, an equal share each (a share is one
// tile's 1 KB blocks); the producer fetches every later round, round j + 3
// right after barrier j, which is where every wave has finished round
// j - 1 in that ring quarter. Compute waves then never wait on a full
// memory queue between rounds; the producer's issue is paced by its wait
// counter (at most 63 loads in flight).
//
// Between the two phases each wave reduces its scores to a per-query
// maximum and, after the exchange, a sum, through 1 KB of LDS each; the
// probabilities are then formed in place and kept as the fp16 MFMA
// operand. Scores of up to MAXR key rounds live in registers (16 floats per
// lane and round), so MAXR = 6 covers 768 keys (a 32 x 768 score block per
// head), the most that fits beside the producer wave without spilling.
constexpr int kExactKeys = 768;
constexpr int kExactRing = 4;                 // rounds held by the ring
constexpr int kSlot = 8192;                   // one 32-key K or V^T tile
constexpr int kRoundBytes = kRound * kSlot;   // one round: four tiles
constexpr int kExactRingBytes = kExactRing * kRoundBytes;

template <int GROUP>
constexpr int ExactLds() {
  const int ring = kExactRingBytes + GROUP * kQBytes + 2 * GROUP * kRound * 32 * 4;
  const int merge = 4 * GROUP * 3 * 4 * 64 * 16;  // three O^T slices per wave
  return ring > merge ? ring : merge;
}

template <int GROUP, int MAXR>
__global__ __launch_bounds__((4 * GROUP + 1) * 64) void ExactAttentionKernel(AttentionParams p) {
  if (static_cast<int>(blockIdx.x) >= p.work_count * p.kv_heads) {
    PrefetchRanges(p, static_cast<int>(blockIdx.x) - p.work_count * p.kv_heads);
    return;
  }
  constexpr int kWaves = 4 * GROUP;           // compute waves; wave kWaves: producer
  constexpr int kPieces = 32 / kWaves;        // a compute wave's 1 KB DMAs per early round
  constexpr int kQPieces = 8 * GROUP / kWaves;
  static_assert(kPieces == 4 || kPieces == 8, "a wave's share is half or all of one tile");
  extern __shared__ __align__(16) unsigned char lds[];
  const int g = blockIdx.x % p.kv_heads;
  const AttentionWork work = p.work[blockIdx.x / p.kv_heads];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles = (work.seq_length + kKTile - 1) / kKTile;
  const int rounds = (tiles + kRound - 1) / kRound;
  const int total = 2 * rounds;
  const int early = min(kExactRing, total);   // rounds the compute waves fetch

  const unsigned char* k_base = reinterpret_cast<const unsigned char*>(
      p.qk + static_cast<size_t>(p.heads + g) * p.ld_qk);
  const unsigned char* v_base = reinterpret_cast<const unsigned char*>(
      p.vt + static_cast<size_t>(g) * kHeadDim * p.ldvt);
  // K block `sub` (keys 4 sub .. + 3): lane's key 4 sub + lane / 16 at its
  // swizzled chunk; the offset depends on sub % 4 only.
  uint32_t k_lane[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 4 * i + (lane >> 4);
    k_lane[i] = static_cast<uint32_t>((lane >> 4) * kHeadDim + 8 * ((lane & 15) ^ key)) * 2;
  }
  const uint32_t lds_base = LdsAddress(lds);
  // Tiles of round j inside the sequence (round j: key round j, or value
  // round j - rounds).
  auto round_tiles = [&](int j) {
    const int r = j < rounds ? j : j - rounds;
    return min(kRound, tiles - kRound * r);
  };
  // 1 KB block `sub` of tile s of round j: keys 4 sub .. 4 sub + 3 of a K
  // tile, or bytes 1024 sub .. of a V^T tile (8 KB of consecutive bytes).
  auto dma = [&](int j, int s, int sub, uint32_t k_offset) {
    const bool keys = j < rounds;
    const int t = kRound * (keys ? j : j - rounds) + s;
    const int key0 = work.seq_begin + t * kKTile;
    const uint32_t dst = lds_base + (j % kExactRing) * kRoundBytes + s * kSlot + sub * 1024;
    if (keys)
      DmaToLds(k_base + static_cast<size_t>(key0 + 4 * sub) * kHeadDim * 2, k_offset, dst);
    else
      DmaToLds(v_base + static_cast<size_t>(key0 >> 4) * 4096 + sub * 1024,
               static_cast<uint32_t>(lane) * 16, dst);
  };

  if (wave == kWaves) {
    // The producer: rounds early .. total - 1, round j + 3 after barrier j;
    // before barrier j it waits for its blocks of round j (rounds up to
    // j + 2 are in flight then). Its barriers pair one to one with the
    // compute waves': one per round, two for the softmax exchanges after
    // the last key round, two for the merge.
    for (int j = 0; j < total; ++j) {
      if (j >= early) {
        int later = 0;
        for (int i = j + 1; i <= min(j + 2, total - 1); ++i)
          later += round_tiles(i);
        switch (later) {
          case 0: WaitLoads<0>(); break;
          case 1: WaitLoads<8>(); break;
          case 2: WaitLoads<16>(); break;
          case 3: WaitLoads<24>(); break;
          case 4: WaitLoads<32>(); break;
          case 5: WaitLoads<40>(); break;
          case 6: WaitLoads<48>(); break;
          case 7: WaitLoads<56>(); break;
          default: WaitLoads<63>(); break;
        }
      }
      RingBarrier();
      const int next = j + kExactRing - 1;
      if (j >= 1 && next < total) {
        const int count = round_tiles(next);
        for (int s = 0; s < count; ++s)
#pragma unroll
          for (int sub = 0; sub < 8; ++sub)
            dma(next, s, sub, k_lane[sub & 3]);
      }
      if (j == rounds - 1) {
        RingBarrier();
        RingBarrier();
      }
    }
    RingBarrier();
    RingBarrier();
    return;
  }

  const int head_local = wave % GROUP;
  const int quarter = wave / GROUP;
  const int head = g * GROUP + head_local;
  const int half_id = lane >> 5;
  const int col = lane & 31;
  // This wave's share of an early round: blocks sub0 .. sub0 + kPieces - 1
  // (sub0 is 0 or 4) of the round's tile `slot`.
  const int slot = wave * kPieces / 8;
  const int sub0 = wave * kPieces % 8;
  auto fills = [&](int j) { return slot < round_tiles(j); };

  // The group's query tiles (rows past the tile's count repeat its last
  // row, whose results are never stored), then the early rounds.
#pragma unroll
  for (int i = 0; i < kQPieces; ++i) {
    const int piece = wave * kQPieces + i;
    const int h = piece >> 3, sub = piece & 7;
    const int row = min(4 * sub + (lane >> 4), work.q_count - 1);
    const int chunk = (lane & 15) ^ ((4 * sub + (lane >> 4)) & 15);
    DmaToLds(reinterpret_cast<const unsigned char*>(
                 p.qk + static_cast<size_t>(g * GROUP + h) * p.ld_qk +
                 static_cast<size_t>(work.q_begin) * kHeadDim),
             static_cast<uint32_t>(row * kHeadDim + 8 * chunk) * 2,
             lds_base + kExactRingBytes + h * kQBytes + sub * 1024);
  }
  for (int j = 0; j < early; ++j)
    if (fills(j))
#pragma unroll
      for (int i = 0; i < kPieces; ++i)
        dma(j, slot, sub0 + i, k_lane[i & 3]);
  // Barrier j: round j has landed and every wave is done with round j - 1.
  // A compute wave waits only for its own early blocks.
  auto begin_round = [&](int j) {
    if (j < early) {
      int later = 0;
      for (int i = j + 1; i < early; ++i)
        later += fills(i) ? 1 : 0;
      switch (later) {
        case 0: WaitLoads<0>(); break;
        case 1: WaitLoads<kPieces>(); break;
        case 2: WaitLoads<2 * kPieces>(); break;
        default: WaitLoads<3 * kPieces>(); break;
      }
    }
    RingBarrier();
  };

  // LDS read offsets: K (and the query tile, laid out alike) row col,
  // chunk 2 kk + half_id; V^T dim 32 dt + col of 16-key block j2, the
  // 16 bytes at 16 half_id.
  int k_read[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    k_read[kk] = col * 256 + (((2 * kk + half_id) ^ (col & 15)) * 16);
  int v_read[4][2];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j2 = 0; j2 < 2; ++j2)
      v_read[dt][j2] = j2 * 4096 + (32 * dt + col) * 32 + half_id * 16;

  // Key phase: S^T = K Q^T per tile; lane holds keys 8 (e / 4) + 4 half_id
  // + e % 4 of its query column, scaled by log2(e) / sqrt(128); keys past
  // the sequence are -inf. Up to four rounds the query fragments stay in
  // registers; with six they are re-read from LDS every round (registers).
  constexpr bool kHoldQ = MAXR <= 4;
  const unsigned char* qs = lds + kExactRingBytes + head_local * kQBytes;
  half8 qf[kHoldQ ? 8 : 1];
  floatx16 s[MAXR];
#pragma unroll
  for (int j = 0; j < MAXR; ++j) {
    if (j < rounds) {
      begin_round(j);
      if constexpr (kHoldQ) {
        if (j == 0)
#pragma unroll
          for (int kk = 0; kk < 8; ++kk)
            qf[kk] = *reinterpret_cast<const half8*>(qs + k_read[kk]);
      }
      const int t = kRound * j + quarter;
      if (t < tiles) {
        const unsigned char* tile = lds + (j % kExactRing) * kRoundBytes + quarter * kSlot;
        floatx16 acc = floatx16{};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          half8 q;
          if constexpr (kHoldQ)
            q = qf[kk];
          else
            q = *reinterpret_cast<const half8*>(qs + k_read[kk]);
          acc = Mfma32(*reinterpret_cast<const half8*>(tile + k_read[kk]), q, acc);
        }
        const int valid_keys = work.seq_length - t * kKTile;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = 8 * (e / 4) + 4 * half_id + (e & 3);
          s[j][e] = key < valid_keys ? acc[e] * p.scale_log2 : -__builtin_inff();
        }
      }
    }
  }

  // Exact softmax over all keys: per-query maximum of the four quarters,
  // then the sum of exp2(s - max), then p = fp16(exp2(s - max) / sum).
  float* smax = reinterpret_cast<float*>(lds + kExactRingBytes + GROUP * kQBytes);
  float* ssum = smax + GROUP * kRound * 32;
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < MAXR; ++j)
    if (j < rounds && kRound * j + quarter < tiles)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        m = fmaxf(m, s[j][e]);
  m = fmaxf(m, __shfl_xor(m, 32));
  const int stat = (head_local * kRound + quarter) * 32 + col;
  if (half_id == 0)
    smax[stat] = m;
  RingBarrier();
  const float* hmax = smax + head_local * kRound * 32 + col;
  const float row_max = fmaxf(fmaxf(hmax[0], hmax[32]), fmaxf(hmax[64], hmax[96]));
  float sum = 0.0F;
#pragma unroll
  for (int j = 0; j < MAXR; ++j)
    if (j < rounds && kRound * j + quarter < tiles)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[j][e] = __builtin_amdgcn_exp2f(s[j][e] - row_max);
        sum += s[j][e];
      }
  sum += __shfl_xor(sum, 32);
  if (half_id == 0)
    ssum[stat] = sum;
  RingBarrier();
  const float* hsum = ssum + head_local * kRound * 32 + col;
  const float inverse = 1.0F / ((hsum[0] + hsum[32]) + (hsum[64] + hsum[96]));
  // P^T operand for keys 16 j2 .. 16 j2 + 15 of a tile: slot e is
  // accumulator element 8 j2 + e; V^T's permuted block order puts the same
  // keys in the 16 bytes at position 8 half_id of the block.
  half8 pf[MAXR][2];
#pragma unroll
  for (int j = 0; j < MAXR; ++j)
    if (j < rounds && kRound * j + quarter < tiles)
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pf[j][j2][e] = static_cast<half_t>(s[j][8 * j2 + e] * inverse);

  // Value phase: O^T = V^T P^T over this quarter's tiles.
  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
    o[dt] = floatx16{};
#pragma unroll
  for (int j = 0; j < MAXR; ++j) {
    if (j < rounds) {
      begin_round(rounds + j);
      if (kRound * j + quarter < tiles) {
        const unsigned char* tile =
            lds + ((rounds + j) % kExactRing) * kRoundBytes + quarter * kSlot;
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2)
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
            o[dt] = Mfma32(*reinterpret_cast<const half8*>(tile + v_read[dt][j2]),
                           pf[j][j2], o[dt]);
      }
    }
  }

  // The four quarters' outputs are summed as ((0 + 1) + (2 + 3)); wave
  // (head, quarter) finishes dims 32 quarter .. + 31 of its head, its own
  // part straight from registers. Every DMA has landed (each wave waited
  // for its last one before the last round's barrier), so the ring is free
  // once every wave is past that round.
  floatx4* accs = reinterpret_cast<floatx4*>(lds);
  RingBarrier();
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    if (dt == quarter)
      continue;
    const int part = dt < quarter ? dt : dt - 1;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      accs[((wave * 3 + part) * 4 + k) * 64 + lane] =
          floatx4{o[dt][4 * k], o[dt][4 * k + 1], o[dt][4 * k + 2], o[dt][4 * k + 3]};
  }
  RingBarrier();
  const floatx16 own = quarter == 0 ? o[0] : quarter == 1 ? o[1] : quarter == 2 ? o[2] : o[3];
  auto load = [&](int q) {
    if (q == quarter)
      return own;
    const int w = q * GROUP + head_local;
    const int part = quarter < q ? quarter : quarter - 1;
    floatx16 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const floatx4 x = accs[((w * 3 + part) * 4 + k) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[4 * k + i] = x[i];
    }
    return v;
  };
  const floatx16 result = (load(0) + load(1)) + (load(2) + load(3));
  if (col >= work.q_count)
    return;
  half_t* out = p.out + static_cast<size_t>(work.q_begin + col) * p.heads * kHeadDim +
                head * kHeadDim + quarter * 32;
  // Lane holds dims 8 (e / 4) + 4 half_id + e % 4 of the slice.
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    half4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = static_cast<half_t>(result[4 * q + e]);
    *reinterpret_cast<half4*>(out + 8 * q + 4 * half_id) = v;
  }
}

}  // namespace

void PlanAttentionWork(std::vector<AttentionWork>& work, int* exact_count,
                       int* exact_rounds) {
  std::stable_partition(work.begin(), work.end(), [](const AttentionWork& w) {
    return w.seq_length <= kExactAttentionKeys;
  });
  int count = 0, rounds = 0;
  for (const AttentionWork& w : work) {
    if (w.seq_length > kExactAttentionKeys)
      break;
    ++count;
    rounds = std::max(rounds, ((w.seq_length + kKTile - 1) / kKTile + kRound - 1) / kRound);
  }
  *exact_count = count;
  *exact_rounds = rounds;
}

void LaunchAttention(const AttentionParams& p, hipStream_t stream) {
  Require(p.work_count > 0, "attention: no work");
  Require(p.kv_heads > 0 && p.heads % p.kv_heads == 0,
          "attention: heads must be a multiple of kv_heads");
  Require(p.ld_qk % kHeadDim == 0 && p.ld_qk >= p.ldvt * kHeadDim && p.ldvt % 16 == 0,
          "attention: the q/k head stride must hold ldvt rows of 128, and ldvt be a "
          "multiple of 16");
  const int group = p.heads / p.kv_heads;
  Require(group == 1 || group == 2, "attention: query heads per kv head must be 1 or 2");
  Require(p.prefetch_groups >= 0, "attention: negative prefetch group count");
  Require(p.exact_count >= 0 && p.exact_count <= p.work_count,
          "attention: exact work count outside the work list");
  Require(p.exact_count == 0 ||
              (p.exact_rounds >= 1 && p.exact_rounds * kRound * kKTile <= kExactAttentionKeys),
          "attention: exact key rounds outside 1 .. 6");
  static_assert(kExactAttentionKeys == kExactKeys, "exact kernel key limit");
  const bool online = p.exact_count < p.work_count;
  if (p.exact_count > 0) {
    AttentionParams e = p;
    e.work_count = p.exact_count;
    const dim3 grid(e.work_count * e.kv_heads + e.prefetch_groups);
    const int r = p.exact_rounds;
    auto launch = [&](auto kernel, int waves, int lds_bytes) {
      Dispatch(kernel, grid, dim3(waves * 64), lds_bytes, stream, true, !online, e);
    };
    if (group == 1) {
      if (r <= 1) launch(ExactAttentionKernel<1, 1>, 5, ExactLds<1>());
      else if (r <= 2) launch(ExactAttentionKernel<1, 2>, 5, ExactLds<1>());
      else if (r <= 4) launch(ExactAttentionKernel<1, 4>, 5, ExactLds<1>());
      else launch(ExactAttentionKernel<1, 6>, 5, ExactLds<1>());
    } else {
      if (r <= 1) launch(ExactAttentionKernel<2, 1>, 9, ExactLds<2>());
      else if (r <= 2) launch(ExactAttentionKernel<2, 2>, 9, ExactLds<2>());
      else if (r <= 4) launch(ExactAttentionKernel<2, 4>, 9, ExactLds<2>());
      else launch(ExactAttentionKernel<2, 6>, 9, ExactLds<2>());
    }
  }
  if (online) {
    AttentionParams l = p;
    l.work = p.work + p.exact_count;
    l.work_count = p.work_count - p.exact_count;
    l.prefetch_groups = p.exact_count > 0 ? 0 : p.prefetch_groups;
    const dim3 grid(l.work_count * l.kv_heads + l.prefetch_groups);
    if (group == 1)
      Dispatch(AttentionKernel<1>, grid, dim3(5 * 64), AttentionLds<1>(), stream,
               p.exact_count == 0, true, l);
    else
      Dispatch(AttentionKernel<2>, grid, dim3(9 * 64), AttentionLds<2>(), stream,
               p.exact_count == 0, true, l);
  }
  Check(hipGetLastError(), "attention launch");
}

}  // namespace ovg
