// CDNA4 matrix-core helpers: 16x16 output tiles, K staged in LDS chunks of 32.
//
// Instruction shapes (gfx950):
//   16-bit inputs: v_mfma_f32_16x16x32_{bf16,f16} -- one instruction per 32-wide chunk
//   fp32 inputs:   v_mfma_f32_16x16x4_f32        -- eight instructions per chunk
// Operand fragments: lane l supplies row (l % 16) of A and column (l % 16) of
// B, and a K slice selected by (l / 16); A and B use the same K slice
// mapping, so the product is correct for any slice order.  Result: lane l
// holds D[4 * (l / 16) + r][l % 16] for r = 0..3.
//
// LDS tiles are [rows][kLdk<T>] with K contiguous; the row pitch is padded so
// the 16 rows read by one 16-lane group hit distinct banks.
#pragma once

#include "common.h"

namespace pmsst {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunkK = 32;

template <typename T>
struct LdsPitch {
  static constexpr int value = sizeof(T) == 2 ? kChunkK + 8 : kChunkK + 1;
};

// acc += A_row-block(16 x 32) * B_col-block(32 x 16) for one K chunk.
// `a_row` / `b_row` point at the LDS row (l % 16) of the lane's A / B tile.
template <typename T>
__device__ __forceinline__ f32x4_t mfma_chunk(const T* a_row, const T* b_row, f32x4_t acc, int lane);

template <>
__device__ __forceinline__ f32x4_t mfma_chunk<bf16>(const bf16* a_row, const bf16* b_row, f32x4_t acc, int lane) {
  const int k = (lane >> 4) * 8;
  const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(a_row + k);
  const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(b_row + k);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4_t mfma_chunk<f16>(const f16* a_row, const f16* b_row, f32x4_t acc, int lane) {
  const int k = (lane >> 4) * 8;
  const f16x8_t a = *reinterpret_cast<const f16x8_t*>(a_row + k);
  const f16x8_t b = *reinterpret_cast<const f16x8_t*>(b_row + k);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4_t mfma_chunk<float>(const float* a_row, const float* b_row, f32x4_t acc, int lane) {
  const int k = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < kChunkK; kk += 4) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a_row[kk + k], b_row[kk + k], acc, 0, 0, 0);
  }
  return acc;
}

}  // namespace pmsst
