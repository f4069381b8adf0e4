// Row-per-lane-group geometry shared by the RMSNorm and fused q/k norm kernels,
// plus the deterministic column reduction used for dgamma.
#pragma once

#include "common.h"

namespace pmsst {

#ifndef PMSST_ROW_BWD_THREADS
#define PMSST_ROW_BWD_THREADS 512
#endif
constexpr int kRowBwdThreads = PMSST_ROW_BWD_THREADS;
// Upper bound on backward blocks; the dgamma workspace is kRowBwdMaxParts * dim fp32.
#ifndef PMSST_ROW_BWD_MAX_PARTS
#define PMSST_ROW_BWD_MAX_PARTS 1024
#endif
constexpr int kRowBwdMaxParts = PMSST_ROW_BWD_MAX_PARTS;

struct RowGeom {
  int vec;       // elements per pack (1 = scalar path with column guards)
  int nv;        // packs per lane
  int tpr_log2;  // log2(lanes per row)
  bool ok;
};

// Fast path: dim % vec == 0, every non-null pointer aligned to one pack and at
// most 4 packs per lane.  Otherwise the guarded scalar path (dim <= 512).
inline RowGeom pick_row_geom(int64_t dim, int vec, const void* const* ptrs, const size_t* elem_sizes, int n) {
  bool aligned = dim % vec == 0;
  for (int i = 0; i < n && aligned; ++i) {
    if (ptrs[i] != nullptr && reinterpret_cast<uintptr_t>(ptrs[i]) % (elem_sizes[i] * vec) != 0) aligned = false;
  }
  if (aligned) {
    const int64_t nvec = dim / vec;
    int tpr_log2 = 0;
    while (tpr_log2 < 6 && nvec % (int64_t{2} << tpr_log2) == 0) ++tpr_log2;
    const int64_t nv = nvec >> tpr_log2;
    if (nv >= 1 && nv <= 4) return RowGeom{vec, static_cast<int>(nv), tpr_log2, true};
  }
  if (dim <= 512) {
    const int64_t need = (dim + kWave - 1) / kWave;
    const int nv = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
    return RowGeom{1, nv, 6, true};
  }
  return RowGeom{0, 0, 0, false};
}

inline int row_bwd_parts(int64_t rows, int tpr_log2) {
  const int64_t rpb = static_cast<int64_t>(kWave >> tpr_log2) * (kRowBwdThreads / kWave);
  const int64_t blocks = (rows + rpb - 1) / rpb;
  return static_cast<int>(blocks < kRowBwdMaxParts ? blocks : kRowBwdMaxParts);
}

inline size_t row_bwd_workspace(int64_t dim) {
  return static_cast<size_t>(kRowBwdMaxParts) * static_cast<size_t>(dim) * sizeof(float);
}

// out[c] = sum_{p < parts} partial[p * dim + c], fixed order, stored in `out_dtype`.
// parts == 0 writes zeros.
int launch_col_sum(const float* partial, int parts, int dim, void* out, int out_dtype, hipStream_t stream);

constexpr int kColSumCols = 16;     // columns per 256-thread tile
constexpr int kColSumGroups = 64;   // row groups per column
constexpr int kColSumLds = kColSumGroups * (kColSumCols + 1) * 4;  // bytes of LDS a tile uses

// Columns [16 blk, 16 blk + 16) of out[c] = sum_p partial[p * dim + c] by one block of NT threads
// (256 or 1024: col_sum_kernel, and tail blocks of kernels that run after the partials are
// complete).  Row group g < 64 sums rows g, g + 64, ... with 8 loads in flight per trip; thread t
// works groups t / 16 + (NT / 16) v of column t % 16; the groups are then added in a fixed tree.
// The order of every addition depends on parts and dim only, not on NT.  `red` is kColSumLds
// bytes of LDS.
template <typename TO, int NT>
__device__ __forceinline__ void col_sum_tile(const float* __restrict__ partial, int parts, int dim,
                                             TO* __restrict__ out, int blk, float* red) {
  constexpr int G = kColSumGroups, P = kColSumCols + 1, TG = NT / kColSumCols;
  static_assert(NT == 256 || NT == 1024, "threads");
  const int cl = threadIdx.x % kColSumCols;
  const int tg = threadIdx.x / kColSumCols;
  const int c = blk * kColSumCols + cl;
#pragma unroll
  for (int v = 0; v < G / TG; ++v) {
    const int grp = tg + TG * v;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (c < dim) {
      int p = grp;
      for (; p + 7 * G < parts; p += 8 * G) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = partial[static_cast<int64_t>(p + u * G) * dim + c];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] += x[u];
      }
      for (; p < parts; p += G) acc[0] += partial[static_cast<int64_t>(p) * dim + c];
    }
    red[grp * P + cl] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  }
  __syncthreads();
  for (int stride = G / 2; stride > 0; stride >>= 1) {
    for (int grp = tg; grp < stride; grp += TG) red[grp * P + cl] += red[(grp + stride) * P + cl];
    __syncthreads();
  }
  if (tg == 0 && c < dim) out[c] = from_f32<TO>(red[cl]);
}

}  // namespace pmsst
