// Deterministic column sums of [parts, dim] fp32 partials (second stage of
// every dgamma / dbias reduction).
#include "rowgeom.h"

namespace pmsst {
namespace {

constexpr int kColsPerBlock = 16;
constexpr int kGroups = 64;  // 16 x 64 = 1024 threads

template <typename TO>
__global__ __launch_bounds__(kColsPerBlock* kGroups) void col_sum_kernel(const float* __restrict__ partial,
                                                                         int parts, int dim, TO* __restrict__ out) {
  __shared__ float red[kGroups][kColsPerBlock + 1];
  const int cl = threadIdx.x % kColsPerBlock;
  const int grp = threadIdx.x / kColsPerBlock;
  const int c = blockIdx.x * kColsPerBlock + cl;
  float s0 = 0.f, s1 = 0.f;
  if (c < dim) {
    int p = grp;
    for (; p + kGroups < parts; p += 2 * kGroups) {
      s0 += partial[static_cast<int64_t>(p) * dim + c];
      s1 += partial[static_cast<int64_t>(p + kGroups) * dim + c];
    }
    if (p < parts) s0 += partial[static_cast<int64_t>(p) * dim + c];
  }
  red[grp][cl] = s0 + s1;
  __syncthreads();
  for (int stride = kGroups / 2; stride > 0; stride >>= 1) {
    if (grp < stride) red[grp][cl] += red[grp + stride][cl];
    __syncthreads();
  }
  if (grp == 0 && c < dim) out[c] = from_f32<TO>(red[0][cl]);
}

}  // namespace

int launch_col_sum(const float* partial, int parts, int dim, void* out, int out_dtype, hipStream_t stream) {
  const int blocks = (dim + kColsPerBlock - 1) / kColsPerBlock;
  const dim3 grid(blocks), block(kColsPerBlock * kGroups);
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
