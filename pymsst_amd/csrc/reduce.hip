// Deterministic column sums of [parts, dim] fp32 partials (second stage of
// every dgamma / dbias reduction).
#include "rowgeom.h"

namespace pmsst {
namespace {

// One 16-column tile per block of 1024 threads (col_sum_tile): one row group per thread.
template <typename TO>
__global__ __launch_bounds__(1024) void col_sum_kernel(const float* __restrict__ partial, int parts, int dim,
                                                       TO* __restrict__ out) {
  __shared__ float red[kColSumLds / 4];
  col_sum_tile<TO, 1024>(partial, parts, dim, out, blockIdx.x, red);
}

}  // namespace

int launch_col_sum(const float* partial, int parts, int dim, void* out, int out_dtype, hipStream_t stream) {
  const int blocks = (dim + kColSumCols - 1) / kColSumCols;
  const dim3 grid(blocks), block(1024);
  switch (out_dtype) {
    case PMSST_F32:
      hipLaunchKernelGGL(col_sum_kernel<float>, grid, block, 0, stream, partial, parts, dim,
                         static_cast<float*>(out));
      break;
    case PMSST_F16:
      hipLaunchKernelGGL(col_sum_kernel<f16>, grid, block, 0, stream, partial, parts, dim, static_cast<f16*>(out));
      break;
    case PMSST_BF16:
      hipLaunchKernelGGL(col_sum_kernel<bf16>, grid, block, 0, stream, partial, parts, dim,
                         static_cast<bf16*>(out));
      break;
    default:
      return fail(PMSST_EDTYPE, "col_sum: unsupported dtype %d", out_dtype);
  }
  return check_launch("col_sum_kernel");
}

}  // namespace pmsst
