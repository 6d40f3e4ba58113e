// Bidirectional grouped-query attention over packed sequences on gfx950
// matrix cores: replaces State::Attention's two batched GEMMs, the
// materialised [heads][L][L] scores, SoftmaxKernel and MergeHeadsKernel of
// the reference (generator.cpp:122-172, kernels/generator_kernels.hip:
// 161-189). Scores never leave registers. Which kernel a query takes
// depends on its own sequence's length only (PlanAttentionWork):
//  * sequences of at most 768 keys (every shape of the generator's
//    workloads): the reference's exact softmax, in SharedKeyAttentionKernel
//    (two query heads per kv head; queries and keys shared through LDS) or
//    ExactAttentionKernel (one; operands straight from memory into
//    registers), both described below;
//  * AttentionKernel, longer sequences: online softmax over LDS-staged
//    tiles, described next.
//
// AttentionKernel: a work-group takes one tile of 32 queries of one
// sequence and one key/value head g, with 4 x GROUP waves (the GROUP query heads of g times four key
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
// The q/k/v GEMM stores queries, keys and V^T in matrix-core operand order
// (QkIndex, VtIndex): every 32-row tile of a head is 8 KB of consecutive
// bytes whose 1 KB blocks are the operands of one MFMA, in lane order. This
// kernel copies tiles verbatim into LDS; eight lanes of an operand read
// cover 128 consecutive bytes, so no read has bank conflicts.
#include <algorithm>
#include <type_traits>
#include <utility>
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

template <int GROUP>
__global__ __launch_bounds__((4 * GROUP + 1) * 64) void AttentionKernel(
    AttentionParams p) {
  if (static_cast<int>(blockIdx.x) >= p.work_count * p.kv_heads) {
    PrefetchWeights(p.prefetch, static_cast<int>(blockIdx.x) - p.work_count * p.kv_heads);
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
  // A K, V^T or query tile is 8 KB of consecutive bytes already in operand
  // order (QkIndex, VtIndex), copied verbatim: lane l's 16 bytes of 1 KB
  // block sub at 1024 sub + 16 l.
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
      DmaToLds((part == 0 ? k_base : v_base) + static_cast<size_t>(key0 >> 4) * 4096 +
                   sub * 1024,
               v_lane, dst);
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
  // tile's count are the rows that follow, whose results are never stored),
  // then rounds 0 and 1.
#pragma unroll
  for (int j = 0; j < kQShare; ++j) {
    const int i = wave * kQShare + j;
    const int h = i >> 3, sub = i & 7;
    DmaToLds(reinterpret_cast<const unsigned char*>(
                 p.qk + static_cast<size_t>(g * GROUP + h) * p.ld_qk +
                 static_cast<size_t>(work.q_begin >> 4) * 2048) +
                 sub * 1024,
             v_lane, lds_base + kRingBytes + h * kQBytes + sub * 1024);
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

  // Stage-invariant LDS read offsets: K step kk of a key or query tile
  // (QkIndex order), and the value-product operand (dims 32 dt .., keys of
  // block j2; VtIndex order). Eight lanes read 128 consecutive bytes, so
  // neither read has bank conflicts.
  int k_read[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    k_read[kk] = (col >> 4) * 4096 + kk * 512 + half_id * 256 + (col & 15) * 16;
  int v_read[4][2];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j2 = 0; j2 < 2; ++j2)
      v_read[dt][j2] = 8192 + j2 * 4096 + dt * 1024 + lane * 16;

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
// Two instances of it. ExactAttentionKernel (one query head per kv head,
// GROUP = HPW = 1): one work-group per (32-query tile, kv head) with four
// waves, wave w taking key tiles q, q + 4, q + 8, ... (q = w % 4). Every K
// and V^T operand goes from memory straight into registers (QkIndex and
// VtIndex store each 32-row tile's operands as whole 256-byte runs), as do
// the query operands: the LDS holds only the softmax statistics and the
// final merge. (Written for HPW of GROUP heads per wave; two query heads
// per kv head take the shared-key kernel below.) A wave's tiles stream through a ring of
// operand buffers, one or two tiles ahead: its key tiles, then its value
// tiles, so the first value tiles load while the softmax runs. Every load
// is unconditional (a slot past the wave's last tile re-reads a tile of the
// sequence and is not used), so the compiler's wait counts stay exact.
//
// Between the two phases each wave reduces its scores to a per-query
// maximum and, after the exchange, a sum, through LDS; the probabilities
// are then formed in place and kept as the fp16 MFMA operand. Scores of up
// to MAXR tiles per wave live in registers (16 floats per lane, tile and
// head), so MAXR = 6 covers 768 keys.
constexpr int kExactKeys = 768;
constexpr int kExactMaxTiles = 6;   // per wave: 4 x 6 x 32 = 768 keys

// Calls f(integral_constant<int, J>) for J = 0, 1, ...: a loop whose index
// is a compile-time constant in every iteration.
template <typename F, int... J>
__device__ __forceinline__ void UnrollEach(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}

// LDS of the exact kernels: the merge's O^T slices (three per wave) and the
// softmax statistics, maxima then sums (in the register-fed kernel they
// share the space: the statistics are dead once every wave is past the
// barrier before the merge).
template <int GROUP>
constexpr int kExactMerge = 4 * 3 * GROUP * 16 * 64 * 4;
template <int GROUP>
constexpr int kExactStats = 2 * GROUP * kRound * 32 * 4;
constexpr int kMeetings = 3;  // maxima, sums, merge
template <int GROUP>
constexpr int ExactLds() {
  return kExactStats<GROUP> > kExactMerge<GROUP> ? kExactStats<GROUP> : kExactMerge<GROUP>;
}

// The four waves of one head meet at an LDS arrival counter (zeroed at the
// start of the work-group): each waits for its own LDS writes, adds one and
// waits until all four have. The other head's waves run on, so that one
// head's softmax and products overlap the other's loads. The wait is
// bounded: every wave of the work-group reaches every meeting point, so the
// bound is never reached in a correct run, and it guarantees that no wave
// can spin forever.
constexpr int kMeetSpinLimit = 1 << 22;
__device__ __forceinline__ void HeadSync(unsigned int* counter) {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(counter, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int i = 0; i < kMeetSpinLimit; ++i) {
    const unsigned int arrived =
        __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(arrived) >= static_cast<unsigned int>(kRound))
      break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" : : : "memory");
}

template <int GROUP, int MAXR, int HPW>
__global__ __launch_bounds__(256 * GROUP / HPW) void ExactAttentionKernel(AttentionParams p) {
  if (static_cast<int>(blockIdx.x) >= p.work_count * p.kv_heads) {
    PrefetchWeights(p.prefetch, static_cast<int>(blockIdx.x) - p.work_count * p.kv_heads);
    return;
  }
  extern __shared__ __align__(16) unsigned char lds[];
  const int g = blockIdx.x % p.kv_heads;
  const AttentionWork work = p.work[blockIdx.x / p.kv_heads];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quarter = wave % kRound;
  const int head0 = (wave / kRound) * HPW;  // this wave's first head of the group
  const int half_id = lane >> 5;
  const int col = lane & 31;
  const int tiles = (work.seq_length + kKTile - 1) / kKTile;
  const int mine = (tiles - quarter + kRound - 1) / kRound;  // tiles 4 j + quarter < tiles
  const int block0 = work.seq_begin >> 4;

  // Operand offsets (halves) inside a 32-row tile: K step kk of the key
  // operand; value-product operand f = 2 dt + j2 (dims 32 dt .., keys of
  // block j2).
  int k_off[8], v_off[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    k_off[kk] = (col >> 4) * 2048 + kk * 256 + half_id * 128 + (col & 15) * 8;
#pragma unroll
  for (int f = 0; f < 8; ++f)
    v_off[f] = (f & 1) * 2048 + (f >> 1) * 512 + lane * 8;
  const half_t* k_head = p.qk + static_cast<size_t>(p.heads + g) * p.ld_qk;
  const half_t* v_head = p.vt + static_cast<size_t>(g) * kHeadDim * p.ldvt;
  // Stream slot s: key tile s (s < MAXR), else value tile s - MAXR, of this
  // wave; slots past its last tile re-read the sequence's last tile. A ring
  // of kDepth operand buffers, loads kDepth - 1 slots ahead (two buffers at
  // six tiles, where a third would not fit in registers).
  constexpr int kDepth = MAXR >= 6 ? 2 : 3;
  half8 buf[kDepth][8];
  auto load_slot = [&](auto slot) {
    constexpr int s = decltype(slot)::value;
    constexpr int j = s < MAXR ? s : s - MAXR;
    const int t = min(kRound * j + quarter, tiles - 1);
    const half_t* base = (s < MAXR ? k_head : v_head) + static_cast<size_t>(block0 + 2 * t) * 2048;
#pragma unroll
    for (int f = 0; f < 8; ++f)
      buf[s % kDepth][f] = *reinterpret_cast<const half8*>(base + (s < MAXR ? k_off[f] : v_off[f]));
    // Slots issue in stream order: a key tile's operands never queue behind
    // a later value tile's.
    __builtin_amdgcn_sched_barrier(0);
  };
  // The query tiles' operands straight into registers (rows past the
  // tile's count belong to the next rows; their results are never stored),
  // then the first operand slots.
  half8 qf[HPW][8];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    const half_t* q_tile = p.qk + static_cast<size_t>(g * GROUP + head0 + h) * p.ld_qk +
                           static_cast<size_t>(work.q_begin >> 4) * 2048;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[h][kk] = *reinterpret_cast<const half8*>(q_tile + k_off[kk]);
  }
  __builtin_amdgcn_sched_barrier(0);
  load_slot(std::integral_constant<int, 0>{});
  if constexpr (kDepth == 3)
    load_slot(std::integral_constant<int, 1>{});

  // Key phase: S^T = K Q^T per tile and head, unscaled; lane holds keys
  // 8 (e / 4) + 4 half_id + e % 4 of its query column. Keys past the
  // sequence (only in its last, partial tile) are -inf.
  floatx16 s[HPW][MAXR];
  auto key_tile = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j + kDepth - 1 < 2 * MAXR)
      load_slot(std::integral_constant<int, j + kDepth - 1>{});
    if (j < mine) {
      const int valid_keys = work.seq_length - (kRound * j + quarter) * kKTile;
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        floatx16 acc = floatx16{};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
          acc = Mfma32(buf[j % kDepth][kk], qf[h][kk], acc);
        s[h][j] = acc;
        if (valid_keys < kKTile)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = 8 * (e / 4) + 4 * half_id + (e & 3);
            s[h][j][e] = key < valid_keys ? s[h][j][e] : -__builtin_inff();
          }
      }
    }
  };
  UnrollEach(key_tile, std::make_integer_sequence<int, MAXR>{});

  // Exact softmax over all keys: per-query maximum of the four quarters,
  // then the sum of e = exp2(c s - c max), c = log2(e) / sqrt(128) (c > 0,
  // so the maximum of the unscaled scores serves), then p = fp16(e / sum).
  float* smax = reinterpret_cast<float*>(lds);
  float* ssum = smax + GROUP * kRound * 32;
  float inverse[HPW];
  {
    float m[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      m[h] = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < MAXR; ++j)
        if (j < mine)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            m[h] = fmaxf(m[h], s[h][j][e]);
      m[h] = fmaxf(m[h], __shfl_xor(m[h], 32));
      if (half_id == 0)
        smax[((head0 + h) * kRound + quarter) * 32 + col] = m[h];
    }
    RingBarrier();
    float sum[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const float* hm = smax + (head0 + h) * kRound * 32 + col;
      const float shift = -(fmaxf(fmaxf(hm[0], hm[32]), fmaxf(hm[64], hm[96])) * p.scale_log2);
      sum[h] = 0.0F;
#pragma unroll
      for (int j = 0; j < MAXR; ++j)
        if (j < mine)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            s[h][j][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[h][j][e], p.scale_log2, shift));
            sum[h] += s[h][j][e];
          }
      sum[h] += __shfl_xor(sum[h], 32);
      if (half_id == 0)
        ssum[((head0 + h) * kRound + quarter) * 32 + col] = sum[h];
    }
    RingBarrier();
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const float* hs = ssum + (head0 + h) * kRound * 32 + col;
      inverse[h] = 1.0F / ((hs[0] + hs[32]) + (hs[64] + hs[96]));
    }
  }
  // P^T operand for keys 16 j2 .. 16 j2 + 15 of a tile: slot e is
  // accumulator element 8 j2 + e; VtIndex puts the same keys in the chunk
  // of lane half half_id.
  half8 pf[HPW][MAXR][2];
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int j = 0; j < MAXR; ++j)
      if (j < mine)
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pf[h][j][j2][e] = static_cast<half_t>(s[h][j][8 * j2 + e] * inverse[h]);

  // Value phase: O^T = V^T P^T over this quarter's tiles, every head.
  floatx16 o[HPW][4];
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      o[h][dt] = floatx16{};
  auto value_tile = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    constexpr int slot = MAXR + j;
    if constexpr (slot + kDepth - 1 < 2 * MAXR)
      load_slot(std::integral_constant<int, slot + kDepth - 1>{});
    if (j < mine) {
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int h = 0; h < HPW; ++h)
            o[h][dt] = Mfma32(buf[slot % kDepth][2 * dt + j2], pf[h][j][j2], o[h][dt]);
    }
  };
  UnrollEach(value_tile, std::make_integer_sequence<int, MAXR>{});

  // The four quarters' outputs are summed as ((0 + 1) + (2 + 3)); wave q
  // finishes dims 32 q .. + 31 of every head, its own part straight from
  // registers. The statistics are dead once every wave is past the
  // barrier, so the merge reuses their space.
  floatx4* accs = reinterpret_cast<floatx4*>(lds);
  RingBarrier();
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      if (dt == quarter)
        continue;
      const int part = dt < quarter ? dt : dt - 1;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        accs[(((quarter * 3 + part) * GROUP + head0 + h) * 4 + k) * 64 + lane] =
            floatx4{o[h][dt][4 * k], o[h][dt][4 * k + 1], o[h][dt][4 * k + 2],
                    o[h][dt][4 * k + 3]};
    }
  RingBarrier();
  if (col >= work.q_count)
    return;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    const floatx16 own = quarter == 0   ? o[h][0]
                         : quarter == 1 ? o[h][1]
                         : quarter == 2 ? o[h][2]
                                        : o[h][3];
    auto load = [&](int q) {
      if (q == quarter)
        return own;
      const int part = quarter < q ? quarter : quarter - 1;
      floatx16 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const floatx4 x = accs[(((q * 3 + part) * GROUP + head0 + h) * 4 + k) * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[4 * k + i] = x[i];
      }
      return v;
    };
    const floatx16 result = (load(0) + load(1)) + (load(2) + load(3));
    half_t* out = p.out + static_cast<size_t>(work.q_begin + col) * p.heads * kHeadDim +
                  (g * GROUP + head0 + h) * kHeadDim + quarter * 32;
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
}


// --------------------------------------------------- shared-key kernel
// The exact kernel for two query heads per kv head and at most 512 keys
// (MAXR <= 4), with the queries and keys fetched once per work-group. The
// two heads' waves of a quarter use the same key tiles, and every wave of a
// head the same query tile: loaded straight into registers they cross the
// CU's load-return path (64 bytes per clock) twice and four times, and at
// 330 + 250 keys the operand loads (448 KB per CU) take about half of a
// work-group's time. Here the eight waves copy the two query tiles and every
// key tile of the sequence into LDS by DMA (a share each, 104 KB at 330
// keys), meet once, and read their operands from LDS, which returns about
// four times as many bytes per clock; the value tiles still stream into
// registers per wave, as in the kernel above. The products, the softmax,
// the merge and every rounding are the exact kernel's, in the same order,
// so the two kernels give the same bits.
//
// LDS: key tiles [tile][8 KB] and after them the two query tiles, verbatim
// copies of the operand-order layout; the merge's O^T slices reuse that
// space once all eight waves are past their key phase (an arrival counter);
// the statistics and the counters sit after both.
//
// The DMAs of a key round (4 tiles, 32 KB) are spread over the eight waves,
// and a work-group barrier after each round makes its tiles readable to
// all. With five or six tiles per wave the key rounds pass through a ring
// of three slots (96 KB), round r + 2 landing in round r - 1's slot once
// every wave is past round r's barrier.
//
// The phases are bound by different units of the CU: the operand loads by
// its 64 bytes per clock of load return, the softmax by the quarter-rate
// exp2, the products by the matrix cores, the merge by LDS. The two heads'
// waves share a SIMD pairwise and exchange nothing after the key phase, so
// from the softmax on they meet per head (HeadSync) rather than at
// work-group barriers: one head's softmax and products overlap the other's
// (in the register-fed form of this kernel, 330 + 250 keys: 8.90 -> 8.42
// us).
template <int MAXR>
constexpr int kKeySlots = MAXR <= 4 ? MAXR : 3;  // key rounds resident in LDS
template <int MAXR>
constexpr int kSharedKeyBytes = kRound * kKeySlots<MAXR> * kQBytes;
template <int MAXR>
constexpr int kSharedFront = kSharedKeyBytes<MAXR> + 2 * kQBytes > kExactMerge<2>
                                 ? kSharedKeyBytes<MAXR> + 2 * kQBytes
                                 : kExactMerge<2>;
constexpr int kSharedCounters = 2 * kMeetings + 1;  // per head and meeting, keys done
template <int MAXR>
constexpr int SharedKeyLds() {
  return kSharedFront<MAXR> + kExactStats<2> + kSharedCounters * 4;
}

template <int MAXR>
__global__ __launch_bounds__(512) void SharedKeyAttentionKernel(AttentionParams p) {
  constexpr int GROUP = 2;
  static_assert(MAXR >= 1 && MAXR <= 6, "shared-key kernel: 1 to 6 key tiles per wave");
  constexpr int kRing = kKeySlots<MAXR>;
  if (static_cast<int>(blockIdx.x) >= p.work_count * p.kv_heads) {
    PrefetchWeights(p.prefetch, static_cast<int>(blockIdx.x) - p.work_count * p.kv_heads);
    return;
  }
  extern __shared__ __align__(16) unsigned char lds[];
  const int g = blockIdx.x % p.kv_heads;
  const AttentionWork work = p.work[blockIdx.x / p.kv_heads];
  const int q_begin = __builtin_amdgcn_readfirstlane(work.q_begin);
  const int seq_begin = __builtin_amdgcn_readfirstlane(work.seq_begin);
  const int seq_length = __builtin_amdgcn_readfirstlane(work.seq_length);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quarter = wave % kRound;
  const int head = wave / kRound;  // this wave's query head of the group
  const int half_id = lane >> 5;
  const int col = lane & 31;
  const int tiles = (seq_length + kKTile - 1) / kKTile;
  const int mine = (tiles - quarter + kRound - 1) / kRound;  // tiles 4 j + quarter < tiles
  const int block0 = seq_begin >> 4;

  unsigned int* counters =
      reinterpret_cast<unsigned int*>(lds + kSharedFront<MAXR> + kExactStats<GROUP>);
  unsigned int* meet = counters + head * kMeetings;
  unsigned int* keys_done = counters + GROUP * kMeetings;

  // Queries and keys into LDS by wave-wide DMAs of 1 KB, in key rounds:
  // wave w brings query blocks 2 w and 2 w + 1 (query tile b / 8 of the
  // group's heads), then in every round r blocks 4 (w % 2) .. + 3 of key
  // tile 4 r + w / 2 (a tile past the sequence in its last round reloads
  // its last tile into a slot that is never read), so every wave issues the
  // same DMAs, four per round, and a wait names the number of rounds still
  // in flight. Rounds past the sequence's last (a shorter sequence in a
  // launch sized for a longer one) are not loaded. The queries and round 0
  // land before the first barrier; the later rounds are issued after it
  // (issued together with round 0 they delay it: 8.4 against 8.26 us at
  // 330 + 250 keys) and land while the waves compute on the earlier ones.
  const uint32_t lds0 = LdsAddress(lds);
  {
    const unsigned char* q_base = reinterpret_cast<const unsigned char*>(
        p.qk + static_cast<size_t>(g * GROUP) * p.ld_qk + static_cast<size_t>(q_begin >> 4) * 2048);
    const size_t q_head_bytes = static_cast<size_t>(p.ld_qk) * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int b = 2 * wave + i;
      DmaToLds(q_base + (b >> 3) * q_head_bytes + (b & 7) * 1024, lane * 16,
               lds0 + kSharedKeyBytes<MAXR> + b * 1024);
    }
  }
  const unsigned char* k_base = reinterpret_cast<const unsigned char*>(
      p.qk + static_cast<size_t>(p.heads + g) * p.ld_qk + static_cast<size_t>(block0) * 2048);
  auto dma_round = [&](int r) {
    const int slot = kRound * (r % kRing) + (wave >> 1);
    const int t = min(kRound * r + (wave >> 1), tiles - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int blk = 4 * (wave & 1) + i;
      DmaToLds(k_base + static_cast<size_t>(t) * kQBytes + blk * 1024, lane * 16,
               lds0 + slot * kQBytes + blk * 1024);
    }
  };
  // Rounds that hold keys of this sequence (the same for every wave); the
  // instance's later rounds are neither loaded nor waited for here.
  const int rounds = (tiles + kRound - 1) / kRound;
  dma_round(0);
  if (threadIdx.x < kSharedCounters)
    counters[threadIdx.x] = 0;
  WaitLoads<0>();
  RingBarrier();
#pragma unroll
  for (int r = 1; r < kRing; ++r)
    if (r < rounds)
      dma_round(r);

  // Operand offsets (bytes) inside a 32-row tile: K step kk of the key and
  // query operands; value-product operand f = 2 dt + j2 (halves, as above).
  int k_off[8], v_off[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    k_off[kk] = ((col >> 4) * 2048 + kk * 256 + half_id * 128 + (col & 15) * 8) * 2;
#pragma unroll
  for (int f = 0; f < 8; ++f)
    v_off[f] = (f & 1) * 2048 + (f >> 1) * 512 + lane * 8;
  const half_t* v_head = p.vt + static_cast<size_t>(g) * kHeadDim * p.ldvt;
  // Value tile j of this wave into ring slot j % 3, two tiles ahead; tiles
  // past its last re-read the sequence's last tile and are not used.
  constexpr int kDepth = 3;
  half8 buf[kDepth][8];
  auto load_value = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int t = min(kRound * j + quarter, tiles - 1);
    const half_t* base = v_head + static_cast<size_t>(block0 + 2 * t) * 2048;
#pragma unroll
    for (int f = 0; f < 8; ++f)
      buf[j % kDepth][f] = *reinterpret_cast<const half8*>(base + v_off[f]);
    __builtin_amdgcn_sched_barrier(0);
  };
  half8 qf[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk)
    qf[kk] = *reinterpret_cast<const half8*>(lds + kSharedKeyBytes<MAXR> + head * kQBytes + k_off[kk]);

  // Key phase from LDS: S^T = K Q^T per tile, unscaled, keys past the
  // sequence -inf (the exact kernel's key phase).
  floatx16 s[MAXR];
  auto key_tile = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j > 0) {
      if (j < rounds) {
        // Round j has landed once every wave's own DMAs of it have: only
        // the later rounds' DMAs may still be in flight, rounds j + 1 ..
        // min(j + kRing - 2, rounds - 1), four per wave each.
        constexpr int later = MAXR - 1 - j < kRing - 2 ? MAXR - 1 - j : kRing - 2;
        const int pending = min(later, rounds - 1 - j);
        if (later >= 2 && pending >= 2)
          WaitLoads<8>();
        else if (later >= 1 && pending >= 1)
          WaitLoads<4>();
        else
          WaitLoads<0>();
        RingBarrier();
        // Past the barrier no wave reads round j - 1 any more: its slot
        // takes round j + kRing - 1 (five or six tiles per wave, three
        // slots).
        if constexpr (j + kRing - 1 < MAXR && j + kRing - 1 >= kRing)
          if (j + kRing - 1 < rounds)
            dma_round(j + kRing - 1);
      }
    }
    if constexpr (j == MAXR - 1) {
      // The first value tiles once every key tile has landed, so that they
      // do not queue ahead of the last key round; they have the softmax to
      // arrive.
      load_value(std::integral_constant<int, 0>{});
      if constexpr (MAXR > 1)
        load_value(std::integral_constant<int, 1>{});
    }
    if (j < mine) {
      const unsigned char* tile = lds + (kRound * (j % kRing) + quarter) * kQBytes;
      half8 kf[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        kf[kk] = *reinterpret_cast<const half8*>(tile + k_off[kk]);
      const int valid_keys = seq_length - (kRound * j + quarter) * kKTile;
      floatx16 acc = floatx16{};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        acc = Mfma32(kf[kk], qf[kk], acc);
      s[j] = acc;
      if (valid_keys < kKTile)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = 8 * (e / 4) + 4 * half_id + (e & 3);
          s[j][e] = key < valid_keys ? s[j][e] : -__builtin_inff();
        }
    }
  };
  UnrollEach(key_tile, std::make_integer_sequence<int, MAXR>{});
  // This wave's last reads of the query and key tiles are done.
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  if (lane == 0)
    __hip_atomic_fetch_add(keys_done, 1U, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

  // Exact softmax (the exact kernel's, per head).
  float* smax = reinterpret_cast<float*>(lds + kSharedFront<MAXR>);
  float* ssum = smax + GROUP * kRound * 32;
  float inverse;
  {
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < MAXR; ++j)
      if (j < mine)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          m = fmaxf(m, s[j][e]);
    m = fmaxf(m, __shfl_xor(m, 32));
    if (half_id == 0)
      smax[(head * kRound + quarter) * 32 + col] = m;
    HeadSync(meet + 0);
    const float* hm = smax + head * kRound * 32 + col;
    const float shift = -(fmaxf(fmaxf(hm[0], hm[32]), fmaxf(hm[64], hm[96])) * p.scale_log2);
    float sum = 0.0F;
#pragma unroll
    for (int j = 0; j < MAXR; ++j)
      if (j < mine)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          s[j][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][e], p.scale_log2, shift));
          sum += s[j][e];
        }
    sum += __shfl_xor(sum, 32);
    if (half_id == 0)
      ssum[(head * kRound + quarter) * 32 + col] = sum;
    HeadSync(meet + 1);
    const float* hs = ssum + head * kRound * 32 + col;
    inverse = 1.0F / ((hs[0] + hs[32]) + (hs[64] + hs[96]));
  }
  half8 pf[MAXR][2];
#pragma unroll
  for (int j = 0; j < MAXR; ++j)
    if (j < mine)
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
  auto value_tile = [&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j + kDepth - 1 < MAXR)
      load_value(std::integral_constant<int, j + kDepth - 1>{});
    if (j < mine) {
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          o[dt] = Mfma32(buf[j % kDepth][2 * dt + j2], pf[j][j2], o[dt]);
    }
  };
  UnrollEach(value_tile, std::make_integer_sequence<int, MAXR>{});

  // Merge (the exact kernel's), once no wave reads the key tiles any more.
  for (int i = 0; i < kMeetSpinLimit; ++i) {
    const unsigned int done =
        __hip_atomic_load(keys_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(done) >= static_cast<unsigned int>(GROUP * kRound))
      break;
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" : : : "memory");
  floatx4* accs = reinterpret_cast<floatx4*>(lds);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    if (dt == quarter)
      continue;
    const int part = dt < quarter ? dt : dt - 1;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      accs[(((quarter * 3 + part) * GROUP + head) * 4 + k) * 64 + lane] =
          floatx4{o[dt][4 * k], o[dt][4 * k + 1], o[dt][4 * k + 2], o[dt][4 * k + 3]};
  }
  HeadSync(meet + 2);
  if (col >= work.q_count)
    return;
  const floatx16 own = quarter == 0 ? o[0] : quarter == 1 ? o[1] : quarter == 2 ? o[2] : o[3];
  auto load = [&](int q) {
    if (q == quarter)
      return own;
    const int part = quarter < q ? quarter : quarter - 1;
    floatx16 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const floatx4 x = accs[(((q * 3 + part) * GROUP + head) * 4 + k) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[4 * k + i] = x[i];
    }
    return v;
  };
  const floatx16 result = (load(0) + load(1)) + (load(2) + load(3));
  half_t* out = p.out + static_cast<size_t>(q_begin + col) * p.heads * kHeadDim +
                (g * GROUP + head) * kHeadDim + quarter * 32;
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
  Require(p.prefetch.groups >= 0, "attention: negative prefetch group count");
  Require(p.exact_count >= 0 && p.exact_count <= p.work_count,
          "attention: exact work count outside the work list");
  Require(p.exact_count == 0 ||
              (p.exact_rounds >= 1 && p.exact_rounds * kRound * kKTile <= kExactAttentionKeys),
          "attention: exact key rounds outside 1 .. 6");
  static_assert(kExactAttentionKeys == kExactKeys &&
                    kExactKeys == kExactMaxTiles * kRound * kKTile,
                "exact kernel key limit");
  const bool online = p.exact_count < p.work_count;
  if (p.exact_count > 0) {
    AttentionParams e = p;
    e.work_count = p.exact_count;
    const dim3 grid(e.work_count * e.kv_heads + e.prefetch.groups);
    // Two query heads per kv head: the shared-key kernel (eight waves);
    // one: the register-fed kernel (four waves). A query's arithmetic is
    // the same either way.
    auto launch = [&](auto kernel, int waves, int lds_bytes) {
      Dispatch(kernel, grid, dim3(64 * waves), lds_bytes, stream, true, !online, e);
    };
    // The kernel instance holds exactly the largest per-wave tile count.
    if (group == 2) {
      switch (p.exact_rounds) {
        case 1: launch(SharedKeyAttentionKernel<1>, 8, SharedKeyLds<1>()); break;
        case 2: launch(SharedKeyAttentionKernel<2>, 8, SharedKeyLds<2>()); break;
        case 3: launch(SharedKeyAttentionKernel<3>, 8, SharedKeyLds<3>()); break;
        case 4: launch(SharedKeyAttentionKernel<4>, 8, SharedKeyLds<4>()); break;
        case 5: launch(SharedKeyAttentionKernel<5>, 8, SharedKeyLds<5>()); break;
        default: launch(SharedKeyAttentionKernel<6>, 8, SharedKeyLds<6>()); break;
      }
    } else {
      switch (p.exact_rounds) {
        case 1: launch(ExactAttentionKernel<1, 1, 1>, 4, ExactLds<1>()); break;
        case 2: launch(ExactAttentionKernel<1, 2, 1>, 4, ExactLds<1>()); break;
        case 3: launch(ExactAttentionKernel<1, 3, 1>, 4, ExactLds<1>()); break;
        case 4: launch(ExactAttentionKernel<1, 4, 1>, 4, ExactLds<1>()); break;
        case 5: launch(ExactAttentionKernel<1, 5, 1>, 4, ExactLds<1>()); break;
        default: launch(ExactAttentionKernel<1, 6, 1>, 4, ExactLds<1>()); break;
      }
    }
  }
  if (online) {
    AttentionParams l = p;
    l.work = p.work + p.exact_count;
    l.work_count = p.work_count - p.exact_count;
    l.prefetch.groups = p.exact_count > 0 ? 0 : p.prefetch.groups;
    const dim3 grid(l.work_count * l.kv_heads + l.prefetch.groups);
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
