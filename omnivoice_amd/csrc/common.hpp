// Shared device-side definitions of the gfx950 generator kernels.
#ifndef OMNIVOICE_AMD_COMMON_HPP_
#define OMNIVOICE_AMD_COMMON_HPP_

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ovg {

using half_t = _Float16;
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Rows of every activation buffer are padded to this multiple (plus one
// 32-row key tile of slack) so tile loads never leave the allocation.
constexpr int kRowAlign = 256;
// Each packed sequence starts at a multiple of this many rows, so that a
// 32-key tile of V^T starts on a 16-byte boundary.
constexpr int kSequenceAlign = 8;

__device__ __forceinline__ float WaveSum(float v) {
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    v = v + __shfl_xor(v, offset);
  return v;
}

__device__ __forceinline__ float WaveMax(float v) {
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    v = fmaxf(v, __shfl_xor(v, offset));
  return v;
}

// 32x32x16 fp16 MFMA (gfx950): D = A B + C. Lane l supplies
// A[l % 32][8 (l / 32) .. +7] and B[8 (l / 32) .. +7][l % 32]; it receives
// D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] in element r.
__device__ __forceinline__ floatx16 Mfma32(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

}  // namespace ovg

#endif  // OMNIVOICE_AMD_COMMON_HPP_
