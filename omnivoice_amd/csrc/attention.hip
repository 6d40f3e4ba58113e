// Bidirectional grouped-query attention over packed sequences on gfx950
// matrix cores: replaces State::Attention's two batched GEMMs, the
// materialised [heads][L][L] scores, SoftmaxKernel and MergeHeadsKernel of
// the reference (generator.cpp:122-172, kernels/generator_kernels.hip:
// 161-189). Scores never leave registers.
//
// A work-group takes one tile of 32 queries of one sequence and one key/value
// head g; its waves are the query heads of g's group (2 for 16 q / 8 kv), so
// each K/V tile is staged in LDS once for the whole group (no GQA repeat).
//
// Scores are formed transposed, S^T = K Q^T (keys as MFMA rows, queries as
// columns), so that every lane owns one query column: the running max and
// sum of the online softmax are per-lane values combined with the partner
// lane l ^ 32 only. The value product is likewise transposed,
// O^T = V^T P^T: P^T is the score accumulator itself converted to fp16 (the
// k index order of the MFMA is permuted to the accumulator's row order, and
// V^T is read from LDS in the same permuted order), so probabilities never
// move between lanes. V^T comes pre-transposed from the q/k/v GEMM's
// epilogue ([kv head][dim][row]).
#include "kernels.hpp"

namespace ovg {
namespace {

constexpr int kKTile = 32;
constexpr int kHeadDim = 128;
constexpr int kKPitch = kHeadDim + 8;  // halves per key row in LDS
constexpr int kVPitch = kKTile + 8;    // halves per dim row of V^T in LDS

template <int GROUP>
__global__ __launch_bounds__(GROUP * 64) void AttentionKernel(
    AttentionParams p) {
  __shared__ __align__(16) half_t ks[kKTile * kKPitch];
  __shared__ __align__(16) half_t vs[kHeadDim * kVPitch];
  const AttentionWork work = p.work[blockIdx.x];
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int head = g * GROUP + wave;
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
  for (int t = 0; t < tiles; ++t) {
    const int key0 = work.seq_begin + t * kKTile;
    // Stage K [32 keys][128] and V^T [128 dims][32 keys] (512 chunks each).
    for (int c = tid; c < kKTile * kHeadDim / 8; c += GROUP * 64) {
      const int row = c >> 4, c8 = (c & 15) * 8;
      *reinterpret_cast<half8*>(ks + row * kKPitch + c8) =
          *reinterpret_cast<const half8*>(
              kbase + static_cast<size_t>(key0 + row) * p.ld_qk + c8);
      const int d = c >> 2, k8 = (c & 3) * 8;
      *reinterpret_cast<half8*>(vs + d * kVPitch + k8) =
          *reinterpret_cast<const half8*>(
              vbase + static_cast<size_t>(d) * p.ldvt + key0 + k8);
    }
    __syncthreads();

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
    __syncthreads();
  }

  const float total = run_sum + __shfl_xor(run_sum, 32);
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
      const half4 v = {static_cast<half_t>(ot[dt][4 * q] * inverse),
                       static_cast<half_t>(ot[dt][4 * q + 1] * inverse),
                       static_cast<half_t>(ot[dt][4 * q + 2] * inverse),
                       static_cast<half_t>(ot[dt][4 * q + 3] * inverse)};
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
      hipLaunchKernelGGL(AttentionKernel<1>, grid, dim3(64), 0, stream, p);
      break;
    case 2:
      hipLaunchKernelGGL(AttentionKernel<2>, grid, dim3(128), 0, stream, p);
      break;
    case 4:
      hipLaunchKernelGGL(AttentionKernel<4>, grid, dim3(256), 0, stream, p);
      break;
    default:
      throw Error("attention: query heads per kv head must be 1, 2 or 4");
  }
  Check(hipGetLastError(), "attention launch");
}

}  // namespace ovg
