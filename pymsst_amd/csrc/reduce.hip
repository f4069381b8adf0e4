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

// partial[pb][c] = sum of src[r][c] over row block pb (kColsumRowBlock rows, ascending), for
// row blocks pb = blockIdx.y, blockIdx.y + gridDim.y, ...; 4 columns per thread.  A whole row
// block issues all its loads before the first add.
template <typename T>
__global__ __launch_bounds__(256) void colsum_rows_kernel(const T* __restrict__ src, int64_t rows, int64_t cols,
                                                          bool vec4, float* __restrict__ partial) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (c >= cols) return;
  const int64_t parts = (rows + kColsumRowBlock - 1) / kColsumRowBlock;
  for (int64_t pb = blockIdx.y; pb < parts; pb += gridDim.y) {
    const int64_t r0 = pb * kColsumRowBlock;
    const int64_t r1 = r0 + kColsumRowBlock < rows ? r0 + kColsumRowBlock : rows;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (vec4 && c + 4 <= cols && r1 - r0 == kColsumRowBlock) {
      float v[kColsumRowBlock][4];
#pragma unroll
      for (int r = 0; r < kColsumRowBlock; ++r) load_pack<T, 4>(src + (r0 + r) * cols + c, v[r]);
#pragma unroll
      for (int r = 0; r < kColsumRowBlock; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += v[r][j];
    } else if (vec4 && c + 4 <= cols) {
      for (int64_t r = r0; r < r1; ++r) {
        float v[4];
        load_pack<T, 4>(src + r * cols + c, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += v[j];
      }
    } else {
      for (int64_t r = r0; r < r1; ++r)
        for (int j = 0; j < 4 && c + j < cols; ++j) s[j] += to_f32(src[r * cols + c + j]);
    }
    float* dst = partial + pb * cols + c;
    for (int j = 0; j < 4 && c + j < cols; ++j) dst[j] = s[j];
  }
}

}  // namespace

int launch_colsum_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, float* partial, void* out,
                       int out_dtype, hipStream_t stream) {
  PMSST_REQUIRE(cols > 0 && cols < (int64_t{1} << 31) && rows >= 0, "colsum_rows: bad shape");
  const int64_t parts = (rows + kColsumRowBlock - 1) / kColsumRowBlock;
  PMSST_REQUIRE(parts < (int64_t{1} << 31), "colsum_rows: too many rows");
  if (parts > 0) {
    const size_t esz = src_dtype == PMSST_F32 ? 4 : 2;
    const bool vec4 = cols % 4 == 0 && reinterpret_cast<uintptr_t>(src) % (4 * esz) == 0;
    const dim3 grid(static_cast<unsigned>((cols + 1023) / 1024), static_cast<unsigned>(parts < 65535 ? parts : 65535));
    switch (src_dtype) {
      case PMSST_F32:
        hipLaunchKernelGGL(colsum_rows_kernel<float>, grid, dim3(256), 0, stream, static_cast<const float*>(src),
                           rows, cols, vec4, partial);
        break;
      case PMSST_F16:
        hipLaunchKernelGGL(colsum_rows_kernel<f16>, grid, dim3(256), 0, stream, static_cast<const f16*>(src), rows,
                           cols, vec4, partial);
        break;
      case PMSST_BF16:
        hipLaunchKernelGGL(colsum_rows_kernel<bf16>, grid, dim3(256), 0, stream, static_cast<const bf16*>(src),
                           rows, cols, vec4, partial);
        break;
      default:
        return fail(PMSST_EDTYPE, "colsum_rows: unsupported dtype %d", src_dtype);
    }
    const int rc = check_launch("colsum_rows_kernel");
    if (rc != PMSST_OK) return rc;
  }
  return launch_col_sum(partial, static_cast<int>(parts), static_cast<int>(cols), out, out_dtype, stream);
}

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
