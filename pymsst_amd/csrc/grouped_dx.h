// Band GEMMs of the backward on register-accumulating DMA-ring kernels: the grouped linear input
// gradient (grouped_dx.hip), its weight gradient on the mask-estimator DMA dW kernel
// (mask_estimator.hip), and the mask-estimator final layer input gradient (mask_dz.hip).
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

// Whether launch_mask_dz takes this shape (16-bit, H a multiple of 128 or 192, aligned pointers).
bool mask_dz_supported(int64_t H, int64_t rows, size_t elem, const void* dpre, const void* w, const void* x,
                       const void* dx, int64_t total);

// Mask-estimator final layer input gradient dx[m, b, :] = dpre[m, band b] W_b ([2 I_b, H] packed), with
// dz = round(dx) (1 - x^2) when tanh_in (mask_dz.hip).
template <typename T>
int launch_mask_dz(const void* dpre, const void* w, const void* x, void* dx, const int64_t* offsets,
                   const int64_t* dim_inputs, int NB, int64_t M, int64_t H, int F, bool tanh_in, hipStream_t stream);

}  // namespace pmsst
