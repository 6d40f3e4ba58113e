// Shared device-side definitions of the gfx950 generator kernels.
#ifndef OMNIVOICE_AMD_COMMON_HPP_
#define OMNIVOICE_AMD_COMMON_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ovg {

using half_t = _Float16;
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// MI355X: 8 XCDs of 32 compute units; a launch's work-groups are dealt to
// the XCDs in turn (work-group i to XCD i % 8).
constexpr int kXcds = 8;
constexpr int kCus = 256;

// Each packed sequence starts at a multiple of this many rows, so that its
// 32-row tiles are two whole 16-row blocks of the attention's operand
// layouts (QkIndex, VtIndex).
constexpr int kSequenceAlign = 16;

// Column of packed row `row` in V^T: within every 16-row block the rows are
// stored in the order 0-3, 8-11, 4-7, 12-15, the key order of the attention
// kernel's probability operand.
__host__ __device__ constexpr int VtColumn(int row) {
  return (row & ~15) | (((row >> 2) & 1) << 3) | (((row >> 3) & 1) << 2) |
         (row & 3);
}

// The attention's operands are stored in matrix-core fragment order, in
// blocks of 16 packed rows (4 KB per head and block), so that the operand of
// one v_mfma_f32_32x32x16_f16 for a 32-row tile is whole 256-byte runs that
// a wave loads straight into registers.
//
// q and k heads: head h's rows at h * ldq; block b (rows 16 b .. + 15) is
// [K step kk 8][half 2][row 16] of 16-byte chunks, chunk (kk, half, r)
// holding dims 16 kk + 8 half .. + 7 of row 16 b + r. The A (keys) or B
// (queries) operand of K step kk for the tile at block b is lane l: chunk
// (kk, l / 32, l % 16) of block b + (l % 32) / 16.
__host__ __device__ constexpr std::size_t QkIndex(int head, int row, int dim, std::size_t ldq) {
  return static_cast<std::size_t>(head) * ldq + static_cast<std::size_t>(row >> 4) * 2048 +
         (dim >> 4) * 256 + ((dim >> 3) & 1) * 128 + (row & 15) * 8 + (dim & 7);
}

// V^T of kv head g: `ldvt` rows (a multiple of 16) at g * 128 * ldvt; block
// b is [dim group dt 4][half 2][dim 32] of 16-byte chunks, chunk (dt, half,
// d) holding dim 32 dt + d of the 8 rows at VtColumn positions 8 half .. + 7
// of the block. The A operand (32 dims x 16 keys) of the value product for
// dims 32 dt .. + 31 and the keys of block b is lane l: chunk (dt, l / 32,
// l % 32) of block b, 1 KB of consecutive bytes.
__host__ __device__ constexpr std::size_t VtIndex(int g, int d, int row, int ldvt) {
  return static_cast<std::size_t>(g) * 128 * ldvt + static_cast<std::size_t>(row >> 4) * 2048 +
         (d >> 5) * 512 + ((VtColumn(row) >> 3) & 1) * 256 + (d & 31) * 8 + (VtColumn(row) & 7);
}

// Output stores that write through to memory: relaxed device-scope atomic
// stores, i.e. ordinary global stores carrying the sc1 coherence bit. The
// lines then do not sit dirty in this XCD's L2 until the write-back at the
// end of the kernel, which otherwise keeps the kernel alive for about 1.5 us
// after its last work-group finished. Nothing else changes: the next kernel
// reads the data after the kernel boundary, as before.
__device__ __forceinline__ void StoreThrough(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<unsigned*>(p),
                     __builtin_bit_cast(unsigned, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void StoreThrough(half_t* p, half_t v) {
  __hip_atomic_store(reinterpret_cast<unsigned short*>(p),
                     __builtin_bit_cast(unsigned short, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void StoreThrough(half4* p, half4 v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p),
                     __builtin_bit_cast(unsigned long long, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void StoreThrough(floatx4* p, floatx4 v) {
  typedef float floatx2 __attribute__((ext_vector_type(2)));
  auto* q = reinterpret_cast<unsigned long long*>(p);
  const floatx2 lo = {v[0], v[1]}, hi = {v[2], v[3]};
  __hip_atomic_store(q, __builtin_bit_cast(unsigned long long, lo),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, __builtin_bit_cast(unsigned long long, hi),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float WaveSum(float v) {
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    v = v + __shfl_xor(v, offset);
  return v;
}

// Wave sum without LDS traffic: DPP within 16-lane rows (swap neighbours,
// swap pairs, half-row mirror, row mirror), then the four row sums read with
// v_readlane and added as (row 0 + row 1) + (row 2 + row 3). Every lane gets
// the total. Its summation tree differs from WaveSum's, so the bit-exact
// score uses WaveSum.
template <int CTRL>
__device__ __forceinline__ float DppAdd(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                CTRL, 0xF, 0xF, false);
  return v + __builtin_bit_cast(float, moved);
}

__device__ __forceinline__ float WaveSumFast(float v) {
  v = DppAdd<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v = DppAdd<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v = DppAdd<0x141>(v);  // row_half_mirror
  v = DppAdd<0x140>(v);  // row_mirror
  const int bits = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float WaveMax(float v) {
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    v = fmaxf(v, __shfl_xor(v, offset));
  return v;
}

// LDS address (byte offset in the work-group's LDS) of a __shared__ pointer.
__device__ __forceinline__ uint32_t LdsAddress(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) unsigned char*)(p)));
}

// One wave-wide DMA of 64 x 16 bytes from global memory straight into LDS:
// lane l's 16 bytes land at lds_addr + 16 l. Inline assembly because the
// compiler's wait-count pass cannot tell which stage buffer such a load
// writes and would wait for every load in flight before any LDS read, which
// serialises a ring; the kernels wait explicitly instead (WaitLoads).
// The source is a wave-uniform base (scalar registers) plus a per-lane
// 32-bit byte offset, so that advancing a K step is one scalar add and the
// LDS address is scalar too: no vector work per DMA.
__device__ __forceinline__ void DmaToLds(const unsigned char* base, uint32_t offset,
                                         uint32_t lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(lds_addr), "v"(offset), "s"(base)
      : "memory", "m0");
}

// Waits until at most N of this wave's vector memory loads are in flight.
template <int N>
__device__ __forceinline__ void WaitLoads() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// 32x32x16 fp16 MFMA (gfx950): D = A B + C. Lane l supplies
// A[l % 32][8 (l / 32) .. +7] and B[8 (l / 32) .. +7][l % 32]; it receives
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] in element r.
__device__ __forceinline__ floatx16 Mfma32(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

}  // namespace ovg

#endif  // OMNIVOICE_AMD_COMMON_HPP_
