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
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

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

// Raw 16-bit pattern of a storage value (for register transposes).
__device__ __forceinline__ uint32_t bits16(bf16 v) { return __builtin_bit_cast(uint16_t, v); }
__device__ __forceinline__ uint32_t bits16(f16 v) { return __builtin_bit_cast(uint16_t, v); }

// Stage a K-contiguous source into lds[ROWS][pitch]: element (r, k) of the
// chunk is src[r * stride + k0 + k]; rows >= rows_valid and k >= k_valid are zero.
// Each thread moves 4-element groups; `vec4` selects 4-wide loads (the caller
// guarantees 4-element alignment of every row start and of k0).
template <typename T, int ROWS, int THREADS>
__device__ __forceinline__ void stage_kcontig(T* __restrict__ lds, const T* __restrict__ src, int64_t stride,
                                              int rows_valid, int k0, int k_valid, bool vec4, int tid) {
  constexpr int P = LdsPitch<T>::value;
  for (int q = tid; q < ROWS * (kChunkK / 4); q += THREADS) {
    const int r = q / (kChunkK / 4);
    const int kq = (q % (kChunkK / 4)) * 4;
    const int k = k0 + kq;
    float v[4];
    if (r < rows_valid && vec4 && k + 4 <= k_valid) {
      load_pack<T, 4>(src + r * stride + k, v);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (r < rows_valid && k + j < k_valid) ? to_f32(src[r * stride + k + j]) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) lds[r * P + kq + j] = from_f32<T>(v[j]);
  }
}

}  // namespace pmsst
