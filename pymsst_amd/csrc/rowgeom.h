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

}  // namespace pmsst
