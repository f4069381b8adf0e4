// Shared device/host helpers for the pymsst_amd gfx950 kernels.
//
// Storage types: float, _Float16 and __bf16.  All arithmetic is fp32.
// Every kernel is written for 64-lane wavefronts (CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "pymsst_amd.h"

namespace pmsst {

using bf16 = __bf16;
using f16 = _Float16;

constexpr int kWave = 64;

// 16 raw bytes in one vector register quad (a whole-register load / store that the compiler
// does not slice).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ errors

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* kernel);
int num_cus();

#define PMSST_REQUIRE(cond, ...)                           \
  do {                                                     \
    if (!(cond)) return ::pmsst::fail(PMSST_EINVAL, __VA_ARGS__); \
  } while (0)

// ------------------------------------------------------------------ conversions

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }

// Packed element group, aligned to its own size so one access is one
// global_load/store of 4, 8 or 16 bytes.
template <typename T, int N>
struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ void load_pack(const T* __restrict__ p, float (&o)[N]) {
  const Pack<T, N> pk = *reinterpret_cast<const Pack<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = to_f32(pk.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_pack(T* __restrict__ p, const float (&o)[N]) {
  Pack<T, N> pk;
#pragma unroll
  for (int i = 0; i < N; ++i) pk.v[i] = from_f32<T>(o[i]);
  *reinterpret_cast<Pack<T, N>*>(p) = pk;
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over each aligned group of 16 lanes (one DPP row) with four DPP moves and no LDS traffic:
// quad permutes [1,0,3,2] and [2,3,0,1] (xor 1, xor 2), then the mirror within 8 lanes and within
// the row.  Each step adds two partial sums that every lane of the pair holds, so all 16 lanes end
// with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// Sum over the lanes that share (lane % width): offsets width, 2*width, ..., 32.
__device__ __forceinline__ float cross_group_sum(float v, int width) {
  for (int off = width; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Division of 32-bit unsigned values by a launch-invariant divisor with a
// multiply-high and shift (Granlund & Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994, round-up variant).
// With l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1:
//   t = mulhi(m, n);  q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
struct FastDiv {
  uint32_t d;
  uint32_t mul;
  uint32_t sh1;
  uint32_t sh2;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t divisor) : d(divisor) {
    uint32_t l = 0;
    while ((uint64_t{1} << l) < divisor) ++l;
    mul = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - divisor)) / divisor + 1);
    sh1 = l < 1 ? l : 1;
    sh2 = l > 0 ? l - 1 : 0;
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t t = __umulhi(n, mul);
#else
    const uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(n) * mul) >> 32);
#endif
    return (t + ((n - t) >> sh1)) >> sh2;
  }
  __host__ __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};

template <typename T>
constexpr int dtype_code();
template <>
constexpr int dtype_code<float>() { return PMSST_F32; }
template <>
constexpr int dtype_code<f16>() { return PMSST_F16; }
template <>
constexpr int dtype_code<bf16>() { return PMSST_BF16; }

// Host-side validation helpers.
inline bool dtype_ok(int dt) { return dt == PMSST_F32 || dt == PMSST_F16 || dt == PMSST_BF16; }
inline size_t dtype_size(int dt) { return dt == PMSST_F32 ? 4 : 2; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace pmsst
