// Pipelined MFMA main loop for the ragged per-band GEMMs.
//
// A block computes C[BR x BC] += A[BR x K] * B[BC x K]^T with both operands
// staged in LDS as [rows][pitch] (K contiguous) in chunks of 32.  Two LDS
// buffers and a register copy of the next chunk overlap the global loads of
// chunk k+1 with the MFMAs of chunk k; one barrier per chunk.
//
// LDS layout (16-bit types): row r, element k of a chunk lives at
//   r * pitch + 8 * ((k / 8) ^ ((r / 16) % 4)) + k % 8,
// i.e. the four 16-byte k-units of a row are XOR-swizzled by the row's 16-row
// group.  MFMA fragment reads (16 consecutive rows, one unit) stay 16-byte
// aligned and conflict-free, and the transposed stores of MNLoader (8 bytes to
// rows 4q..4q+3) spread over all banks.  fp32 tiles use a plain odd pitch.
//
// Waves are laid out WR x WC over the tile; wave (wr, wc) owns rows
// [wr * BR/WR, ...) and columns [wc * BC/WC, ...) as TR x TC 16x16 tiles.
// Result layout (mfma.h): lane l of tile (i, j) holds
//   C[row0 + 16 i + 4 (l / 16) + r][col0 + 16 j + (l % 16)],  r = 0..3.
//
// Loaders move one 32-wide K chunk:  fetch(k0, regs) global -> registers,
// commit(regs, lds) registers -> LDS.  Out-of-range rows and k read as zero.
#pragma once

#include "mfma.h"

namespace pmsst {

constexpr int kGemmThreads = 256;

template <typename T>
__device__ __forceinline__ int lds_index(int r, int k) {
  constexpr int P = LdsPitch<T>::value;
  if constexpr (sizeof(T) == 2) {
    return r * P + ((((k >> 3) ^ ((r >> 4) & 3)) << 3) | (k & 7));
  } else {
    return r * P + k;
  }
}

// acc += A rows (ra..) x B rows (rb..) over one 32-wide chunk; `ra` / `rb` are the
// lane's row indices inside the A / B tiles.
template <typename T>
__device__ __forceinline__ f32x4_t mfma_tile(const T* __restrict__ a, int ra, const T* __restrict__ b, int rb,
                                             f32x4_t acc, int lane) {
  if constexpr (sizeof(T) == 2) {
    const int k = (lane >> 4) * 8;
    return mfma_chunk<T>(a + lds_index<T>(ra, k) - k, b + lds_index<T>(rb, k) - k, acc, lane);
  } else {
    return mfma_chunk<T>(a + ra * LdsPitch<T>::value, b + rb * LdsPitch<T>::value, acc, lane);
  }
}

// K-contiguous rows: element (r, k) = base[r * stride + k].  4-element groups
// (8 bytes for 16-bit types) when `vec4` (row starts and k0 4-aligned).
template <typename T, int ROWS>
struct KRowLoader {
  static constexpr int kQuads = ROWS * (kChunkK / 4) / kGemmThreads;
  static_assert(kQuads >= 1 && ROWS * (kChunkK / 4) % kGemmThreads == 0, "tile too small");
  struct Regs {
    Pack<T, 4> q[kQuads];
  };
  const T* base;
  int64_t stride;
  int rows_valid;
  int k_valid;
  bool vec4;

  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      const int idx = threadIdx.x + i * kGemmThreads;
      const int r = idx / (kChunkK / 4);
      const int k = k0 + (idx % (kChunkK / 4)) * 4;
      const T* p = base + r * stride + k;
      if (r < rows_valid && vec4 && k + 4 <= k_valid) {
        g.q[i] = *reinterpret_cast<const Pack<T, 4>*>(p);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) g.q[i].v[j] = (r < rows_valid && k + j < k_valid) ? p[j] : from_f32<T>(0.f);
      }
    }
  }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      const int idx = threadIdx.x + i * kGemmThreads;
      const int r = idx / (kChunkK / 4);
      const int kq = (idx % (kChunkK / 4)) * 4;
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<Pack<T, 4>*>(lds + lds_index<T>(r, kq)) = g.q[i];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[lds_index<T>(r, kq + j)] = g.q[i].v[j];
      }
    }
  }
};

// MN-contiguous source: element (k, mn) = base[k * kstride + mn], staged
// transposed into lds[mn][k].  A thread owns a block of KB consecutive k rows x 4
// consecutive mn (consecutive threads take consecutive mn quads, so each global
// load is coalesced along mn), transposes it in registers and stores KB
// consecutive k values per mn row.  KB = ROWS / 32 so one block per thread
// covers the chunk.  Optional scales: per-mn `cs[mn]`, per-k
// `rs[k * rs_stride] * rs_mul` (both global and cache-resident).
template <typename T, int ROWS>
struct MNLoader {
  static constexpr int kQuadsPerK = ROWS / 4;
  static constexpr int KB = ROWS / 32;
  static_assert(KB >= 1 && KB * kQuadsPerK * (kChunkK / KB) == ROWS * kChunkK / 4, "tile shape");
  static_assert(kQuadsPerK * (kChunkK / KB) == kGemmThreads, "one block per thread");
  struct Regs {
    float v[KB][4];
  };
  const T* base;
  int64_t kstride;
  int mn_valid;
  int k_valid;
  bool vec4;
  const T* cs = nullptr;        // per-mn scale, or null
  const float* rs = nullptr;    // per-k scale, or null
  int64_t rs_stride = 1;
  float rs_mul = 1.f;

  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    const int mn = (threadIdx.x % kQuadsPerK) * 4;
    const int kb = (threadIdx.x / kQuadsPerK) * KB;
    float c[4] = {1.f, 1.f, 1.f, 1.f};
    if (cs != nullptr) {
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = mn + j < mn_valid ? to_f32(cs[mn + j]) : 0.f;
    }
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int k = k0 + kb + t;
      float e[4] = {0.f, 0.f, 0.f, 0.f};
      if (k < k_valid) {
        const T* p = base + static_cast<int64_t>(k) * kstride + mn;
        if (vec4 && mn + 4 <= mn_valid) {
          load_pack<T, 4>(p, e);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) e[j] = mn + j < mn_valid ? to_f32(p[j]) : 0.f;
        }
        const float s = rs != nullptr ? rs[static_cast<int64_t>(k) * rs_stride] * rs_mul : 1.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] *= s * c[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) g.v[t][j] = e[j];
    }
  }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
    const int mn = (threadIdx.x % kQuadsPerK) * 4;
    const int kb = (threadIdx.x / kQuadsPerK) * KB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(T) == 2) {
        float col[KB];
#pragma unroll
        for (int t = 0; t < KB; ++t) col[t] = g.v[t][j];
        store_pack<T, KB>(lds + lds_index<T>(mn + j, kb), col);
      } else {
#pragma unroll
        for (int t = 0; t < KB; ++t) lds[lds_index<T>(mn + j, kb + t)] = g.v[t][j];
      }
    }
  }
};

template <int BR, int BC, int WR, int WC>
struct TileShape {
  static constexpr int kTR = BR / WR / 16;
  static constexpr int kTC = BC / WC / 16;
  static_assert(WR * WC == kGemmThreads / kWave, "4 waves per block");
  static_assert(kTR >= 1 && kTC >= 1 && BR % (WR * 16) == 0 && BC % (WC * 16) == 0, "bad tile");
};

// LDS elements the main loop needs for a BR x BC tile (two buffers).
template <typename T, int BR, int BC>
constexpr int gemm_lds_elems() {
  return 2 * (BR + BC) * LdsPitch<T>::value;
}

// Runs the K loop; `acc` is accumulated (callers zero it).
template <typename T, int BR, int BC, int WR, int WC, class LA, class LB>
__device__ __forceinline__ void gemm_mainloop(const LA& la, const LB& lb, int K, T* lds,
                                              f32x4_t (&acc)[TileShape<BR, BC, WR, WC>::kTR]
                                                            [TileShape<BR, BC, WR, WC>::kTC]) {
  using S = TileShape<BR, BC, WR, WC>;
  constexpr int P = LdsPitch<T>::value;
  T* abuf[2] = {lds, lds + (BR + BC) * P};
  T* bbuf[2] = {lds + BR * P, lds + (BR + BC) * P + BR * P};
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r0 = (wave / WC) * (BR / WR);
  const int c0 = (wave % WC) * (BC / WC);
  const int nk = (K + kChunkK - 1) / kChunkK;
  if (nk == 0) return;
  typename LA::Regs ra;
  typename LB::Regs rb;
  la.fetch(0, ra);
  lb.fetch(0, rb);
  la.commit(ra, abuf[0]);
  lb.commit(rb, bbuf[0]);
  __syncthreads();
  for (int kc = 0; kc < nk; ++kc) {
    const int cur = kc & 1;
    const bool more = kc + 1 < nk;
    if (more) {
      la.fetch((kc + 1) * kChunkK, ra);
      lb.fetch((kc + 1) * kChunkK, rb);
    }
#pragma unroll
    for (int i = 0; i < S::kTR; ++i) {
#pragma unroll
      for (int j = 0; j < S::kTC; ++j) {
        acc[i][j] = mfma_tile<T>(abuf[cur], r0 + i * 16 + (lane & 15), bbuf[cur], c0 + j * 16 + (lane & 15),
                                 acc[i][j], lane);
      }
    }
    if (more) {
      la.commit(ra, abuf[cur ^ 1]);
      lb.commit(rb, bbuf[cur ^ 1]);
    }
    __syncthreads();
  }
}

}  // namespace pmsst
