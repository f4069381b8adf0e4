// Grouped linear backward on the register-accumulating input-gradient kernel (grouped_dx.hip) and
// on the DMA-ring weight-gradient kernel of the mask-estimator backward (mask_estimator.hip).
#pragma once

#include "common.h"

namespace pmsst {

// Whether launch_grouped_dx takes this shape (16-bit, in_features in {64, 128, 192, 256},
// out_features a multiple of 32, aligned pointers).
bool grouped_dx_supported(int64_t groups, int64_t in_features, int64_t out_features, int64_t rows, size_t elem,
                          const void* dy, const void* w, const void* dx);

// dx[m, g, :] = dy[m, g, :] W_g for dy[rows, groups, out_features], W[groups, out_features, in_features].
template <typename T>
int launch_grouped_dx(const void* dy, const void* w, void* dx, int64_t groups, int64_t in_features,
                      int64_t out_features, int64_t rows, hipStream_t stream);

// Whether launch_uniform_dw takes this shape (16-bit, rows >= 32, in_features % 64 == 0,
// out_features % 8 == 0, 16-byte aligned pointers).
bool uniform_dw_supported(int64_t groups, int64_t in_features, int64_t out_features, int64_t rows, size_t elem,
                          const void* dy, const void* x, const void* dw);

// dW[g][o][i] = sum_m dy[m, g, o] x[m, g, i] and db[g][o] = sum_m dy[m, g, o] (db may be null).
template <typename T>
int launch_uniform_dw(const void* dy, const void* x, void* dw, void* db, int64_t groups, int64_t in_features,
                      int64_t out_features, int64_t rows, hipStream_t stream);

}  // namespace pmsst
