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
  // 8 independent loads in flight per trip (a serial chain of round trips otherwise sets the time)
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < dim) {
    int p = grp;
    for (; p + 7 * kGroups < parts; p += 8 * kGroups) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = partial[static_cast<int64_t>(p + u * kGroups) * dim + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += v[u];
    }
    for (; p < parts; p += kGroups) acc[0] += partial[static_cast<int64_t>(p) * dim + c];
  }
  red[grp][cl] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
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
