// RMSNorm forward/backward over the last axis, all reference dtype modes.
//
// Layout: x[rows, dim] row-major.  A row is owned by a group of `tpr`
// consecutive lanes of one wavefront (tpr = largest power of two <= 64 that
// divides dim / VEC); each lane holds NV packs of VEC elements at columns
// (v * tpr + t) * VEC, so every pack access is one 16-byte global load and the
// tpr lanes of a row cover it contiguously.  Row sums are butterfly shuffles
// inside the lane group; a wavefront covers 64 / tpr rows per step.
//
// dgamma: each lane keeps fp32 partial sums for its own fixed columns over the
// rows it visits, the block folds them into one row of a [parts, dim] fp32
// workspace, and col_sum_kernel adds the parts in a fixed order.  No atomics,
// so results are bit-reproducible for a given (rows, dim).
#include <mutex>

#include "common.h"
#include "rowgeom.h"

namespace pmsst {
namespace {

constexpr int kFwdThreads = 256;

template <typename TX, typename TG, typename TO, int VEC, int NV, bool GUARD>
__global__ __launch_bounds__(kFwdThreads) void rms_fwd_kernel(const TX* __restrict__ x, const TG* __restrict__ gamma,
                                                              TO* __restrict__ out, TO* __restrict__ normed,
                                                              float* __restrict__ inv_norm, int64_t rows, int dim,
                                                              int tpr_log2, float scale) {
  const int tpr = 1 << tpr_log2;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t = lane & (tpr - 1);
  const int slot = lane >> tpr_log2;
  const int rows_per_wave = kWave >> tpr_log2;
  const int rows_per_block = rows_per_wave * (kFwdThreads / kWave);

  float g[NV][VEC];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int col = (v * tpr + t) * VEC;
    if (!GUARD || col < dim) {
      load_pack<TG, VEC>(gamma + col, g[v]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) g[v][i] = 0.f;
    }
  }

  for (int64_t base = static_cast<int64_t>(blockIdx.x) * rows_per_block; base < rows;
       base += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t row = base + wave * rows_per_wave + slot;
    const bool valid = row < rows;
    // unguarded packs load from a clamped row without a branch (a load inside a branch is
    // waited for at the join, which would serialize the packs of a lane)
    const int64_t rl = valid ? row : rows - 1;
    float xv[NV][VEC];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int col = (v * tpr + t) * VEC;
      if (!GUARD) {
        load_pack<TX, VEC>(x + rl * dim + col, xv[v]);
      } else if (valid && col < dim) {
        load_pack<TX, VEC>(x + row * dim + col, xv[v]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[v][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += xv[v][i] * xv[v][i];
    }
    ss = group_sum(ss, tpr);
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1.0e-12f);
    if (valid) {
      const float s = inv * scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        if (GUARD && col >= dim) continue;
        float nv[VEC], ov[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          nv[i] = xv[v][i] * s;
          ov[i] = nv[i] * g[v][i];
        }
        if (normed != nullptr) store_pack<TO, VEC>(normed + row * dim + col, nv);
        store_pack<TO, VEC>(out + row * dim + col, ov);
      }
      if (t == 0) inv_norm[row] = inv;
    }
  }
}

#ifndef PMSST_RMS_BWD_HALFVEC
#define PMSST_RMS_BWD_HALFVEC 1
#endif

// FROM_X: `nsrc` is the forward input x and n = x * inv * scale is recomputed;
// otherwise `nsrc` is the saved normalised tensor.
template <typename TDY, typename TN, typename TG, typename TDX, int VEC, int NV, bool GUARD, bool FROM_X>
__global__ __launch_bounds__(kRowBwdThreads) void rms_bwd_kernel(const TDY* __restrict__ dy,
                                                                 const TN* __restrict__ nsrc,
                                                                 const float* __restrict__ inv_norm,
                                                                 const TG* __restrict__ gamma, TDX* __restrict__ dx,
                                                                 float* __restrict__ partial, int64_t rows, int dim,
                                                                 int tpr_log2, float scale) {
  extern __shared__ float red[];  // [waves][dim]
  const int tpr = 1 << tpr_log2;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t = lane & (tpr - 1);
  const int slot = lane >> tpr_log2;
  const int rows_per_wave = kWave >> tpr_log2;
  const int rows_per_block = rows_per_wave * (kRowBwdThreads / kWave);

  float g[NV][VEC];
  float acc[NV][VEC];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int col = (v * tpr + t) * VEC;
    if (!GUARD || col < dim) {
      load_pack<TG, VEC>(gamma + col, g[v]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) g[v][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[v][i] = 0.f;
  }

  const float inv_scale = 1.0f / scale;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * rows_per_block; base < rows;
       base += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t row = base + wave * rows_per_wave + slot;
    const bool valid = row < rows;
    // unguarded packs load from a clamped row without a branch, so all packs of the lane are in
    // flight together; a row past the end only reduces within its own lanes and stores nothing
    const int64_t rl = valid ? row : rows - 1;
    float d[NV][VEC], n[NV][VEC];
    const float inv = inv_norm[rl];
    const float nscale = FROM_X ? inv * scale : 1.0f;
    float dot = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int col = (v * tpr + t) * VEC;
      if (!GUARD) {
        load_pack<TDY, VEC>(dy + rl * dim + col, d[v]);
        load_pack<TN, VEC>(nsrc + rl * dim + col, n[v]);
      } else if (valid && col < dim) {
        load_pack<TDY, VEC>(dy + row * dim + col, d[v]);
        load_pack<TN, VEC>(nsrc + row * dim + col, n[v]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) d[v][i] = n[v][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        if (FROM_X) n[v][i] *= nscale;
        dot += d[v][i] * g[v][i] * n[v][i];
      }
    }
    dot = group_sum(dot, tpr);
    if (valid) {
      const float dot_s = dot * inv_scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        if (GUARD && col >= dim) continue;
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          o[i] = inv * (d[v][i] * g[v][i] * scale - n[v][i] * dot_s);
          acc[v][i] += d[v][i] * n[v][i];
        }
        store_pack<TDX, VEC>(dx + row * dim + col, o);
      }
    }
  }

  // Fold the per-lane column partials: across row slots of the wave, then across waves.
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[v][i] = cross_group_sum(acc[v][i], tpr);
  }
  if (slot == 0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int col = (v * tpr + t) * VEC;
      if (GUARD && col >= dim) continue;
#pragma unroll
      for (int i = 0; i < VEC; ++i) red[wave * dim + col + i] = acc[v][i];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < dim; c += kRowBwdThreads) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kRowBwdThreads / kWave; ++w) s += red[w * dim + c];
    partial[static_cast<int64_t>(blockIdx.x) * dim + c] = s;
  }
}

// ------------------------------------------------------------------ dispatch

template <typename TX, typename TG, typename TO>
int launch_fwd(const void* x, const void* gamma, void* out, void* normed, float* inv_norm, int64_t rows,
               int64_t dim, hipStream_t stream) {
  PMSST_REQUIRE(rows >= 0 && dim > 0 && dim <= (1 << 20), "rms_norm_forward: bad shape rows=%lld dim=%lld",
                (long long)rows, (long long)dim);
  if (rows == 0) return PMSST_OK;
  PMSST_REQUIRE(x && gamma && out && inv_norm, "rms_norm_forward: null pointer");
  constexpr int kVec = 16 / sizeof(TX);
  const void* ptrs[] = {x, gamma, out, normed};
  const size_t sizes[] = {sizeof(TX), sizeof(TG), sizeof(TO), sizeof(TO)};
  RowGeom geo = pick_row_geom(dim, kVec, ptrs, sizes, 4);
  PMSST_REQUIRE(geo.ok, "rms_norm_forward: dim=%lld is not supported (needs dim %% %d == 0 or dim <= 512)",
                (long long)dim, kVec);
  const float scale = sqrtf(static_cast<float>(dim));
  const int rows_per_block = (kWave >> geo.tpr_log2) * (kFwdThreads / kWave);
  const int64_t blocks64 = (rows + rows_per_block - 1) / rows_per_block;
  const int blocks = static_cast<int>(blocks64 < 65536 ? blocks64 : 65536);
  const TX* px = static_cast<const TX*>(x);
  const TG* pg = static_cast<const TG*>(gamma);
  TO* po = static_cast<TO*>(out);
  TO* pn = static_cast<TO*>(normed);
#define PMSST_FWD(VEC, NV, GUARD)                                                                             \
  hipLaunchKernelGGL((rms_fwd_kernel<TX, TG, TO, VEC, NV, GUARD>), dim3(blocks), dim3(kFwdThreads), 0, stream, px, \
                     pg, po, pn, inv_norm, rows, static_cast<int>(dim), geo.tpr_log2, scale)
  if (geo.vec == kVec) {
    switch (geo.nv) {
      case 1: PMSST_FWD(kVec, 1, false); break;
      case 2: PMSST_FWD(kVec, 2, false); break;
      case 3: PMSST_FWD(kVec, 3, false); break;
      case 4: PMSST_FWD(kVec, 4, false); break;
      default: return fail(PMSST_EINVAL, "rms_norm_forward: internal geometry error");
    }
  } else {
    switch (geo.nv) {
      case 1: PMSST_FWD(1, 1, true); break;
      case 2: PMSST_FWD(1, 2, true); break;
      case 4: PMSST_FWD(1, 4, true); break;
      case 8: PMSST_FWD(1, 8, true); break;
      default: return fail(PMSST_EINVAL, "rms_norm_forward: internal geometry error");
    }
  }
#undef PMSST_FWD
  return check_launch("rms_fwd_kernel");
}

template <typename TDY, typename TN, typename TG, typename TDX, bool FROM_X>
int launch_bwd(const void* dy, const void* nsrc, const float* inv_norm, const void* gamma, void* dx,
               void* grad_gamma, int gamma_out_dtype, int64_t rows, int64_t dim, void* workspace,
               size_t workspace_bytes, hipStream_t stream) {
  PMSST_REQUIRE(rows >= 0 && dim > 0 && dim <= (1 << 20), "rms_norm_backward: bad shape rows=%lld dim=%lld",
                (long long)rows, (long long)dim);
  PMSST_REQUIRE(grad_gamma && (rows == 0 || (dy && nsrc && inv_norm && gamma && dx)),
                "rms_norm_backward: null pointer");
  constexpr int kVec = sizeof(TDY) >= sizeof(TDX) ? 16 / sizeof(TDY) : 16 / sizeof(TDX);
  const void* ptrs[] = {dy, nsrc, gamma, dx};
  const size_t sizes[] = {sizeof(TDY), sizeof(TN), sizeof(TG), sizeof(TDX)};
  RowGeom geo = pick_row_geom(dim, kVec, ptrs, sizes, 4);
  PMSST_REQUIRE(geo.ok, "rms_norm_backward: dim=%lld is not supported (needs dim %% %d == 0 or dim <= 512)",
                (long long)dim, kVec);
#if PMSST_RMS_BWD_HALFVEC
  // Three packs per lane (dim = 3 * 2^k) keep 4 x 3 x kVec fp32 values live per lane, which
  // caps occupancy at 3 waves per SIMD: half-width packs on twice the lanes halve that.
  bool half = false;
  if (geo.vec == kVec && geo.nv == 3 && kVec >= 4) {
    const RowGeom h = pick_row_geom(dim, kVec / 2, ptrs, sizes, 4);
    if (h.ok && h.vec == kVec / 2 && h.nv == 3 && h.tpr_log2 == geo.tpr_log2 + 1) {
      geo = h;
      half = true;
    }
  }
#else
  const bool half = false;
#endif
  const int parts = row_bwd_parts(rows, geo.tpr_log2);
  const size_t need = row_bwd_workspace(dim);
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(PMSST_EWORKSPACE, "rms_norm_backward: workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t{0} : workspace_bytes);
  }
  float* partial = static_cast<float*>(workspace);
  const float scale = sqrtf(static_cast<float>(dim));
  const size_t shmem = sizeof(float) * (kRowBwdThreads / kWave) * static_cast<size_t>(dim);
  PMSST_REQUIRE(shmem <= 64 * 1024, "rms_norm_backward: dim=%lld too large", (long long)dim);
  const TDY* pdy = static_cast<const TDY*>(dy);
  const TN* pn = static_cast<const TN*>(nsrc);
  const TG* pg = static_cast<const TG*>(gamma);
  TDX* pdx = static_cast<TDX*>(dx);
  if (parts > 0) {
#define PMSST_BWD(VEC, NV, GUARD)                                                                        \
  hipLaunchKernelGGL((rms_bwd_kernel<TDY, TN, TG, TDX, VEC, NV, GUARD, FROM_X>), dim3(parts),             \
                     dim3(kRowBwdThreads), shmem, stream, pdy, pn, inv_norm, pg, pdx, partial, rows,        \
                     static_cast<int>(dim), geo.tpr_log2, scale)
    if (half) {
      PMSST_BWD(kVec / 2, 3, false);
    } else if (geo.vec == kVec) {
      switch (geo.nv) {
        case 1: PMSST_BWD(kVec, 1, false); break;
        case 2: PMSST_BWD(kVec, 2, false); break;
        case 3: PMSST_BWD(kVec, 3, false); break;
        case 4: PMSST_BWD(kVec, 4, false); break;
        default: return fail(PMSST_EINVAL, "rms_norm_backward: internal geometry error");
      }
    } else {
      switch (geo.nv) {
        case 1: PMSST_BWD(1, 1, true); break;
        case 2: PMSST_BWD(1, 2, true); break;
        case 4: PMSST_BWD(1, 4, true); break;
        case 8: PMSST_BWD(1, 8, true); break;
        default: return fail(PMSST_EINVAL, "rms_norm_backward: internal geometry error");
      }
    }
#undef PMSST_BWD
    int rc = check_launch("rms_bwd_kernel");
    if (rc != PMSST_OK) return rc;
  }
  return launch_col_sum(partial, parts, static_cast<int>(dim), grad_gamma, gamma_out_dtype, stream);
}

template <typename F>
int with_dtype(int dtype, const char* op, F&& f) {
  switch (dtype) {
    case PMSST_F32: return f(float{});
    case PMSST_F16: return f(f16{});
    case PMSST_BF16: return f(bf16{});
    default: return fail(PMSST_EDTYPE, "%s: unsupported dtype code %d", op, dtype);
  }
}

// ------------------------------------------------------------------ allocation-free backward
//
// The dgamma partials of the saved-input backward live in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate.  It holds kRowBwdMaxParts partial rows of up
// to kNoAllocMaxDim columns (4 MiB per GPU, for the life of the process).  Every call on one GPU
// uses that GPU's array: calls that overlap on one GPU (other streams, other host threads) race.
// Nothing needs clearing: each call writes every partial row it reads.
constexpr int kNoAllocMaxDim = 1024;
constexpr size_t kScratchBytes = static_cast<size_t>(kRowBwdMaxParts) * kNoAllocMaxDim * sizeof(float);

__device__ __align__(256) char scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per device.  The array's
// host-side name is only a handle: kernels must be given this address.
int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    return fail(PMSST_ELAUNCH, "rms_norm_backward_from_input_noalloc: no current device");
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      return fail(PMSST_ELAUNCH, "rms_norm_backward_from_input_noalloc: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(err));
    }
    addr[dev] = p;
  }
  *out = addr[dev];
  return PMSST_OK;
}

}  // namespace
}  // namespace pmsst

using namespace pmsst;

extern "C" {

int pmsst_rms_norm_forward(const void* x, const void* gamma, void* out, void* normed, float* inv_norm, int64_t rows,
                           int64_t dim, int dtype, void* stream) {
  return with_dtype(dtype, "rms_norm_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T, T, T>(x, gamma, out, normed, inv_norm, rows, dim, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_forward_fp32_gamma(const void* x, const float* gamma, void* out, void* normed, float* inv_norm,
                                      int64_t rows, int64_t dim, int dtype, void* stream) {
  return with_dtype(dtype, "rms_norm_forward_fp32_gamma", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T, float, T>(x, gamma, out, normed, inv_norm, rows, dim, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_forward_mixed(const void* x, const float* gamma, float* out, float* normed, float* inv_norm,
                                 int64_t rows, int64_t dim, int dtype, void* stream) {
  return with_dtype(dtype, "rms_norm_forward_mixed", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T, float, float>(x, gamma, out, normed, inv_norm, rows, dim,
                                       static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_rms_norm_backward_workspace_size(int64_t rows, int64_t dim) {
  (void)rows;
  return dim > 0 ? row_bwd_workspace(dim) : 0;
}

int pmsst_rms_norm_backward(const void* grad_out, const void* normed, const float* inv_norm, const void* gamma,
                            void* grad_x, void* grad_gamma, int64_t rows, int64_t dim, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  return with_dtype(dtype, "rms_norm_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_bwd<T, T, T, T, false>(grad_out, normed, inv_norm, gamma, grad_x, grad_gamma, dtype, rows, dim,
                                         workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_backward_fp32_gamma(const void* grad_out, const void* normed, const float* inv_norm,
                                       const float* gamma, void* grad_x, float* grad_gamma, int64_t rows,
                                       int64_t dim, int dtype, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  return with_dtype(dtype, "rms_norm_backward_fp32_gamma", [&](auto tag) {
    using T = decltype(tag);
    return launch_bwd<T, T, float, T, false>(grad_out, normed, inv_norm, gamma, grad_x, grad_gamma, PMSST_F32, rows,
                                             dim, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_backward_mixed(const float* grad_out, const float* normed, const float* inv_norm,
                                  const float* gamma, void* grad_x, float* grad_gamma, int64_t rows, int64_t dim,
                                  int x_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return with_dtype(x_dtype, "rms_norm_backward_mixed", [&](auto tag) {
    using T = decltype(tag);
    return launch_bwd<float, float, float, T, false>(grad_out, normed, inv_norm, gamma, grad_x, grad_gamma,
                                                     PMSST_F32, rows, dim, workspace, workspace_bytes,
                                                     static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_backward_from_input(const void* grad_out, const void* x, const float* inv_norm,
                                       const void* gamma, void* grad_x, void* grad_gamma, int64_t rows,
                                       int64_t dim, int dtype, int gamma_dtype, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  if (gamma_dtype != dtype && gamma_dtype != PMSST_F32) {
    return fail(PMSST_EDTYPE, "rms_norm_backward_from_input: gamma dtype must equal x dtype or be fp32");
  }
  return with_dtype(dtype, "rms_norm_backward_from_input", [&](auto tag) {
    using T = decltype(tag);
    if (gamma_dtype == PMSST_F32) {
      return launch_bwd<T, T, float, T, true>(grad_out, x, inv_norm, gamma, grad_x, grad_gamma, PMSST_F32, rows,
                                              dim, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    }
    return launch_bwd<T, T, T, T, true>(grad_out, x, inv_norm, gamma, grad_x, grad_gamma, dtype, rows, dim,
                                        workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_backward_from_input_noalloc(const void* grad_out, const void* x, const float* inv_norm,
                                               const void* gamma, void* grad_x, void* grad_gamma, int64_t rows,
                                               int64_t dim, int dtype, int gamma_dtype, void* stream) {
  if (dim <= 0 || dim > kNoAllocMaxDim) {
    return fail(PMSST_EINVAL, "rms_norm_backward_from_input_noalloc: dim=%lld outside [1, %d] (the static scratch "
                "holds %d partial rows of %d columns)", (long long)dim, kNoAllocMaxDim, kRowBwdMaxParts,
                kNoAllocMaxDim);
  }
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != PMSST_OK) return rc;
  return pmsst_rms_norm_backward_from_input(grad_out, x, inv_norm, gamma, grad_x, grad_gamma, rows, dim, dtype,
                                            gamma_dtype, ws, kScratchBytes, stream);
}

}  // extern "C"
