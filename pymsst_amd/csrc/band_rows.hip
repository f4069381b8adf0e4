// Band gather and overlap-averaged mask scatter of the Mel-band RoFormer front and back end.
//
// The spectrum is packed [batch, R, T, 2] (R = frequency x channel rows, T frames, re/im) and a
// band layout selects J rows (rows[j], bands in order, a row possibly selected by two bands).
//
//   gather:  out[b, t, j, :] = in[b, rows[j], t, :] / divisor[j]          (divisor optional)
//   scatter: out[b, r, t, :] = (sum_{j : rows[j] = r} in[b, t, j, :]) / count(r)   (or no division)
//
// The gather builds the band-split input (and, with divisor = count(rows[j]), the backward of
// the averaged scatter); the scatter averages the per-band masks onto the spectrum (and, without
// the division, is the gather's backward).  Sums run in ascending j and divide by the count
// like the stock scatter_add + division, so a bin covered once or twice matches it exactly.
// The scatter runs in gather form over a row -> selections table (row_start / sources, a CSR
// of the selection list), so every output is written once by one thread in a fixed order: no
// atomics, bitwise reproducible.
//
// Threads walk frames fastest, so the [.., T, 2] side of each kernel is read or written as
// contiguous 8- to 16-byte pairs per lane; the [.., J, 2] side is strided by J pairs.
#include "common.h"

namespace pmsst {
namespace {

constexpr int kRowsThreads = 256;

template <typename TI, typename TO>
__global__ __launch_bounds__(kRowsThreads) void band_gather_kernel(const TI* __restrict__ in,
                                                                   const int64_t* __restrict__ rows,
                                                                   const float* __restrict__ divisor,
                                                                   TO* __restrict__ out, int64_t batch,
                                                                   int64_t R, int64_t T, int64_t J) {
  const int64_t total = batch * J * T;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kRowsThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kRowsThreads) {
    const int64_t t = i % T;
    const int64_t bj = i / T;
    const int64_t j = bj % J;
    const int64_t b = bj / J;
    const int64_t r = rows[j];
    const TI* src = in + ((b * R + r) * T + t) * 2;
    float re = to_f32(src[0]), im = to_f32(src[1]);
    if (divisor != nullptr) {
      re /= divisor[j];
      im /= divisor[j];
    }
    TO* dst = out + ((b * T + t) * J + j) * 2;
    dst[0] = from_f32<TO>(re);
    dst[1] = from_f32<TO>(im);
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kRowsThreads) void band_scatter_kernel(const TI* __restrict__ in,
                                                                    const int64_t* __restrict__ row_start,
                                                                    const int64_t* __restrict__ sources,
                                                                    bool mean, TO* __restrict__ out,
                                                                    int64_t batch, int64_t R, int64_t T,
                                                                    int64_t J) {
  const int64_t total = batch * R * T;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kRowsThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kRowsThreads) {
    const int64_t t = i % T;
    const int64_t br = i / T;
    const int64_t r = br % R;
    const int64_t b = br / R;
    const int64_t k0 = row_start[r], k1 = row_start[r + 1];
    float re = 0.f, im = 0.f;
    for (int64_t k = k0; k < k1; ++k) {
      const TI* src = in + ((b * T + t) * J + sources[k]) * 2;
      re += to_f32(src[0]);
      im += to_f32(src[1]);
    }
    if (mean && k1 > k0) {
      const float c = static_cast<float>(k1 - k0);
      re /= c;
      im /= c;
    }
    TO* dst = out + (b * R + r) * T * 2 + t * 2;
    dst[0] = from_f32<TO>(re);
    dst[1] = from_f32<TO>(im);
  }
}

inline int rows_blocks(int64_t total) {
  const int64_t b = (total + kRowsThreads - 1) / kRowsThreads;
  return static_cast<int>(b < 65536 ? b : 65536);
}

template <typename F>
int rows_dtype2(int in_dtype, int out_dtype, const char* op, F&& f) {
  auto outer = [&](auto ti) -> int {
    switch (out_dtype) {
      case PMSST_F32: return f(ti, float{});
      case PMSST_F16: return f(ti, f16{});
      case PMSST_BF16: return f(ti, bf16{});
      default: return fail(PMSST_EDTYPE, "%s: unsupported output dtype code %d", op, out_dtype);
    }
  };
  switch (in_dtype) {
    case PMSST_F32: return outer(float{});
    case PMSST_F16: return outer(f16{});
    case PMSST_BF16: return outer(bf16{});
    default: return fail(PMSST_EDTYPE, "%s: unsupported input dtype code %d", op, in_dtype);
  }
}

}  // namespace
}  // namespace pmsst

using namespace pmsst;

extern "C" {

int pmsst_band_rows_gather(const void* in, int in_dtype, const int64_t* rows, const float* divisor, void* out,
                           int out_dtype, int64_t batch, int64_t num_rows, int64_t frames, int64_t num_sel,
                           void* stream) {
  const char* op = "band_rows_gather";
  PMSST_REQUIRE(batch >= 0 && num_rows > 0 && frames >= 0 && num_sel >= 0, "%s: bad shape", op);
  const int64_t total = batch * num_sel * frames;
  if (total == 0) return PMSST_OK;
  PMSST_REQUIRE(in && rows && out, "%s: null pointer", op);
  return rows_dtype2(in_dtype, out_dtype, op, [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    hipLaunchKernelGGL((band_gather_kernel<TI, TO>), dim3(rows_blocks(total)), dim3(kRowsThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const TI*>(in), rows, divisor,
                       static_cast<TO*>(out), batch, num_rows, frames, num_sel);
    return check_launch("band_gather_kernel");
  });
}

int pmsst_band_rows_scatter(const void* in, int in_dtype, const int64_t* row_start, const int64_t* sources, int mean,
                            void* out, int out_dtype, int64_t batch, int64_t num_rows, int64_t frames,
                            int64_t num_sel, void* stream) {
  const char* op = "band_rows_scatter";
  PMSST_REQUIRE(batch >= 0 && num_rows > 0 && frames >= 0 && num_sel >= 0, "%s: bad shape", op);
  const int64_t total = batch * num_rows * frames;
  if (total == 0) return PMSST_OK;
  PMSST_REQUIRE(in || num_sel == 0, "%s: null input", op);
  PMSST_REQUIRE(row_start && out && (sources || num_sel == 0), "%s: null pointer", op);
  return rows_dtype2(in_dtype, out_dtype, op, [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    hipLaunchKernelGGL((band_scatter_kernel<TI, TO>), dim3(rows_blocks(total)), dim3(kRowsThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const TI*>(in), row_start, sources,
                       mean != 0, static_cast<TO*>(out), batch, num_rows, frames, num_sel);
    return check_launch("band_scatter_kernel");
  });
}

}  // extern "C"
