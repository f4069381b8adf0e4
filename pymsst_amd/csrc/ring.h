// Helpers of the register-accumulating DMA-ring kernels (grouped_dx.hip, mask_dz.hip): LDS
// fragment reads the compiler waits for itself, an M0-preserving asm DMA, a runtime vmcnt wait.
#pragma once

#include "common.h"
#include "dma_gemm.h"

namespace pmsst {

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// Transposed fragment (two ds_read_b64_tr_b16 through the compiler's builtin, which it waits for)
__device__ __forceinline__ u32x4_t tr_frag(const char* p, int step) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + step));
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return u32x4_t{a.x, a.y, b.x, b.y};
}

// One 16-byte-per-lane global -> LDS DMA (lane l writes LDS byte lds + 16 l; lds wave-uniform),
// from inline asm that saves and restores M0 itself.  The compiler then sees no LDS write and no
// memory operation here: it neither waits for these DMAs before its own LDS reads (it cannot tell
// the ring's stages apart and would wait for the one just issued) nor counts them; the ring's
// ordering is explicit (vmcnt wait, then barrier).  One wait state separates the M0 write from the
// DMA that reads it.
__device__ __forceinline__ void dma16_m0(const void* g, uint32_t lds) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(g), "s"(lds)
      : "memory");
}

template <int N>
__device__ __forceinline__ void ring_vm_wait(int n) {
  // s_waitcnt vmcnt(n) for a wave-uniform n <= N
  if constexpr (N > 0) {
    if (n >= N) {
      vm_wait<N>();
      return;
    }
    ring_vm_wait<N - 1>(n);
  } else {
    vm_wait<0>();
  }
}

}  // namespace pmsst
