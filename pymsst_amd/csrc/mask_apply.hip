// Complex mask application at the STFT / iSTFT boundary, forward and backward.
//
//   est[b, s, c, f, t] = spec[b, f C + c, t] * m_s[b, t, f C + c]            (complex product)
//
// spec  [B, F*C, T] complex64 (re, im interleaved fp32) - the packed mixture spectrum;
// mask  element (b, s, t, 2 (f C + c) + ri) at b * mask_bs + s * mask_ss + t * 2FC + 2(fC+c) + ri,
//       fp32 / fp16 / bf16 - the mask estimators' GLU output, (re, im) pairs per (frequency, channel);
// est   [B, S, C, F, T] complex64 = the iSTFT input [B*S*C, F, T].
// zero_dc writes 0 at f = 0 (the cached-zero iSTFT's index_fill, cuda_graph.py:140-158).
//
// Backward (PyTorch's complex convention: for est = spec * m, grad_m = g conj(spec)):
//   grad_m_s[b, t, fC + c] = g[b, s, c, f, t] conj(spec[b, fC + c, t])  stored as (re, im) in the
//                            mask dtype, mask layout (contiguous [B, S, T, 2FC]);
//   grad_spec[b, fC + c, t] = sum_s g[b, s, c, f, t] conj(m_s[b, t, fC + c])   (optional, fp32).
// With zero_dc both gradients are 0 at f = 0.
//
// A block owns a tile of 32 (frequency, channel) rows x 64 frames of one batch item and loops over
// the stems, so the spectrum tile is read once.  The mask side is [.., T, 2FC] (frames outer) and
// the spectrum / estimate side [.., FC, T] (frames inner): mask tiles pass through LDS ([64 t][65]
// floats, so reading a column is bank-conflict free) and every global access is row-contiguous.
#include "common.h"

namespace pmsst {
namespace {

constexpr int kMaT = 64;         // frames per tile
constexpr int kMaR = 32;         // (frequency, channel) rows per tile
constexpr int kMaP = 2 * kMaR + 1;  // LDS row pitch (floats) of a mask tile
constexpr int kMaThreads = 256;
constexpr int kMaItems = kMaT * kMaR / kMaThreads;  // (row, frame) items per thread

struct MaskApplyArgs {
  int64_t B, S, C, F, T;
  int64_t mask_bs, mask_ss;  // element strides of the mask between batch items and stems
  bool zero_dc;
};

template <typename TM>
__device__ __forceinline__ float2 mask_pair(const TM* p) {
  if constexpr (sizeof(TM) == 4) {
    return *reinterpret_cast<const float2*>(p);
  } else {
    const uint32_t raw = *reinterpret_cast<const uint32_t*>(p);
    typedef TM v2 __attribute__((ext_vector_type(2)));
    const v2 v = __builtin_bit_cast(v2, raw);
    return make_float2(static_cast<float>(v[0]), static_cast<float>(v[1]));
  }
}

template <typename TM>
__device__ __forceinline__ void store_mask_pair(TM* p, float re, float im) {
  if constexpr (sizeof(TM) == 4) {
    *reinterpret_cast<float2*>(p) = make_float2(re, im);
  } else {
    typedef TM v2 __attribute__((ext_vector_type(2)));
    const v2 v{static_cast<TM>(re), static_cast<TM>(im)};
    *reinterpret_cast<uint32_t*>(p) = __builtin_bit_cast(uint32_t, v);
  }
}

// Mask tile of stem s into sm[t][2 r + ri]: thread item i covers frame row tid / 32 + 8 i and
// (frequency, channel) row tid % 32, so a wave reads 2 frames x 32 pairs (contiguous per frame).
// Rows and frames past the end are clamped reads (their products are never stored).
template <typename TM>
__device__ __forceinline__ void load_mask_tile(const TM* __restrict__ mask, const MaskApplyArgs& a, int64_t b,
                                               int64_t s, int64_t t0, int64_t r0, float* sm) {
  const int64_t FC = a.F * a.C;
  const int rl = threadIdx.x % kMaR;
  const int64_t r = r0 + rl < FC ? r0 + rl : FC - 1;
  const TM* base = mask + b * a.mask_bs + s * a.mask_ss + 2 * r;
  float2 v[kMaItems];
#pragma unroll
  for (int i = 0; i < kMaItems; ++i) {
    const int tl = static_cast<int>(threadIdx.x / kMaR) + 8 * i;
    const int64_t t = t0 + tl < a.T ? t0 + tl : a.T - 1;
    v[i] = mask_pair(base + t * 2 * FC);
  }
#pragma unroll
  for (int i = 0; i < kMaItems; ++i) {
    const int tl = static_cast<int>(threadIdx.x / kMaR) + 8 * i;
    sm[tl * kMaP + 2 * rl] = v[i].x;
    sm[tl * kMaP + 2 * rl + 1] = v[i].y;
  }
}

// Spectrum-side item i of this thread: row r0 + idx / 64, frame t0 + idx % 64, idx = tid + 256 i.
__device__ __forceinline__ void item_pos(int i, int& rl, int& tl) {
  const int idx = static_cast<int>(threadIdx.x) + kMaThreads * i;
  rl = idx / kMaT;
  tl = idx % kMaT;
}

template <typename TM>
__global__ __launch_bounds__(kMaThreads) void mask_apply_fwd_kernel(const float2* __restrict__ spec,
                                                                    const TM* __restrict__ mask,
                                                                    float2* __restrict__ est, MaskApplyArgs a) {
  __shared__ float sm[kMaT * kMaP];
  const int64_t FC = a.F * a.C;
  const int64_t t_tiles = (a.T + kMaT - 1) / kMaT;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x % t_tiles) * kMaT;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x / t_tiles) * kMaR;
  const int64_t b = blockIdx.y;
  float2 sv[kMaItems];
#pragma unroll
  for (int i = 0; i < kMaItems; ++i) {
    int rl, tl;
    item_pos(i, rl, tl);
    const int64_t r = r0 + rl < FC ? r0 + rl : FC - 1;
    const int64_t t = t0 + tl < a.T ? t0 + tl : a.T - 1;
    sv[i] = spec[(b * FC + r) * a.T + t];
  }
  for (int64_t s = 0; s < a.S; ++s) {
    __syncthreads();  // the previous stem's tile has been read
    load_mask_tile(mask, a, b, s, t0, r0, sm);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMaItems; ++i) {
      int rl, tl;
      item_pos(i, rl, tl);
      const int64_t r = r0 + rl, t = t0 + tl;
      if (r >= FC || t >= a.T) continue;
      const float mr = sm[tl * kMaP + 2 * rl], mi = sm[tl * kMaP + 2 * rl + 1];
      const int64_t f = r / a.C, c = r % a.C;
      float2 e = make_float2(sv[i].x * mr - sv[i].y * mi, sv[i].x * mi + sv[i].y * mr);
      if (a.zero_dc && f == 0) e = make_float2(0.f, 0.f);
      est[(((b * a.S + s) * a.C + c) * a.F + f) * a.T + t] = e;
    }
  }
}

template <typename TM>
__global__ __launch_bounds__(kMaThreads) void mask_apply_bwd_kernel(const float2* __restrict__ grad_est,
                                                                    const float2* __restrict__ spec,
                                                                    const TM* __restrict__ mask,
                                                                    TM* __restrict__ grad_mask,
                                                                    float2* __restrict__ grad_spec,
                                                                    MaskApplyArgs a) {
  __shared__ float sm[kMaT * kMaP];  // mask tile (grad_spec) / grad_m tile
  const int64_t FC = a.F * a.C;
  const int64_t t_tiles = (a.T + kMaT - 1) / kMaT;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x % t_tiles) * kMaT;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x / t_tiles) * kMaR;
  const int64_t b = blockIdx.y;
  float2 sv[kMaItems], gs[kMaItems];
  int64_t gofs[kMaItems];  // grad_est / est offset of each item (stem 0), clamped
  bool dc[kMaItems];
#pragma unroll
  for (int i = 0; i < kMaItems; ++i) {
    int rl, tl;
    item_pos(i, rl, tl);
    const int64_t r = r0 + rl < FC ? r0 + rl : FC - 1;
    const int64_t t = t0 + tl < a.T ? t0 + tl : a.T - 1;
    sv[i] = spec[(b * FC + r) * a.T + t];
    const int64_t f = r / a.C, c = r % a.C;
    gofs[i] = ((b * a.S * a.C + c) * a.F + f) * a.T + t;
    dc[i] = a.zero_dc && f == 0;
    gs[i] = make_float2(0.f, 0.f);
  }
  const int64_t stem_step = a.C * a.F * a.T;
  for (int64_t s = 0; s < a.S; ++s) {
    float2 g[kMaItems];
#pragma unroll
    for (int i = 0; i < kMaItems; ++i) g[i] = grad_est[gofs[i] + s * stem_step];
    __syncthreads();  // the previous stem's tile has been read
    if (grad_spec != nullptr) {
      load_mask_tile(mask, a, b, s, t0, r0, sm);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kMaItems; ++i) {
        int rl, tl;
        item_pos(i, rl, tl);
        const float mr = sm[tl * kMaP + 2 * rl], mi = sm[tl * kMaP + 2 * rl + 1];
        if (!dc[i]) {  // g conj(m)
          gs[i].x += g[i].x * mr + g[i].y * mi;
          gs[i].y += g[i].y * mr - g[i].x * mi;
        }
      }
      __syncthreads();
    }
    // grad_m = g conj(spec) staged as [t][2 r + ri], then written in mask layout
#pragma unroll
    for (int i = 0; i < kMaItems; ++i) {
      int rl, tl;
      item_pos(i, rl, tl);
      float gr = g[i].x * sv[i].x + g[i].y * sv[i].y;
      float gi = g[i].y * sv[i].x - g[i].x * sv[i].y;
      if (dc[i]) gr = gi = 0.f;
      sm[tl * kMaP + 2 * rl] = gr;
      sm[tl * kMaP + 2 * rl + 1] = gi;
    }
    __syncthreads();
    const int rl = threadIdx.x % kMaR;
    if (r0 + rl < FC) {
      TM* base = grad_mask + (b * a.S + s) * a.T * 2 * FC + 2 * (r0 + rl);
#pragma unroll
      for (int i = 0; i < kMaItems; ++i) {
        const int tl = static_cast<int>(threadIdx.x / kMaR) + 8 * i;
        if (t0 + tl < a.T) store_mask_pair(base + (t0 + tl) * 2 * FC, sm[tl * kMaP + 2 * rl], sm[tl * kMaP + 2 * rl + 1]);
      }
    }
  }
  if (grad_spec != nullptr) {
#pragma unroll
    for (int i = 0; i < kMaItems; ++i) {
      int rl, tl;
      item_pos(i, rl, tl);
      const int64_t r = r0 + rl, t = t0 + tl;
      if (r < FC && t < a.T) grad_spec[(b * FC + r) * a.T + t] = gs[i];
    }
  }
}

int check_mask_apply(const char* op, const MaskApplyArgs& a, const void* spec, const void* mask, int mask_dtype) {
  PMSST_REQUIRE(a.B >= 0 && a.S >= 1 && a.C >= 1 && a.F >= 1 && a.T >= 1, "%s: bad shape", op);
  PMSST_REQUIRE(a.B < 65536, "%s: batch must be < 65536", op);
  PMSST_REQUIRE(mask_dtype == PMSST_F32 || mask_dtype == PMSST_F16 || mask_dtype == PMSST_BF16,
                "%s: unsupported mask dtype %d", op, mask_dtype);
  const int64_t FC = a.F * a.C;
  const int64_t blocks = (a.T + kMaT - 1) / kMaT * ((FC + kMaR - 1) / kMaR);
  PMSST_REQUIRE(blocks < (int64_t{1} << 31), "%s: too many tiles", op);
  PMSST_REQUIRE(a.mask_bs >= 0 && a.mask_ss >= 0, "%s: bad mask strides", op);
  const size_t esz = mask_dtype == PMSST_F32 ? 4 : 2;
  PMSST_REQUIRE(reinterpret_cast<uintptr_t>(spec) % 8 == 0 && reinterpret_cast<uintptr_t>(mask) % (2 * esz) == 0 &&
                    a.mask_bs % 2 == 0 && a.mask_ss % 2 == 0,
                "%s: spec must be 8-byte aligned and mask (re, im) pairs aligned", op);
  return PMSST_OK;
}

}  // namespace
}  // namespace pmsst

using namespace pmsst;

extern "C" {

int pmsst_mask_apply_forward(const void* spec, const void* mask, int64_t mask_batch_stride, int64_t mask_stem_stride,
                             int64_t batch, int64_t stems, int64_t channels, int64_t freqs, int64_t frames,
                             int zero_dc, void* est, int mask_dtype, void* stream) {
  const char* op = "mask_apply_forward";
  const MaskApplyArgs a{batch, stems, channels, freqs, frames, mask_batch_stride, mask_stem_stride, zero_dc != 0};
  if (batch == 0) return PMSST_OK;
  PMSST_REQUIRE(spec && mask && est, "%s: null pointer", op);
  int rc = check_mask_apply(op, a, spec, mask, mask_dtype);
  if (rc != PMSST_OK) return rc;
  PMSST_REQUIRE(reinterpret_cast<uintptr_t>(est) % 8 == 0, "%s: est must be 8-byte aligned", op);
  const int64_t FC = freqs * channels;
  const dim3 grid(static_cast<unsigned>((frames + kMaT - 1) / kMaT * ((FC + kMaR - 1) / kMaR)),
                  static_cast<unsigned>(batch));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float2* sp = static_cast<const float2*>(spec);
  float2* ep = static_cast<float2*>(est);
  switch (mask_dtype) {
    case PMSST_F32:
      hipLaunchKernelGGL(mask_apply_fwd_kernel<float>, grid, dim3(kMaThreads), 0, st, sp,
                         static_cast<const float*>(mask), ep, a);
      break;
    case PMSST_F16:
      hipLaunchKernelGGL(mask_apply_fwd_kernel<f16>, grid, dim3(kMaThreads), 0, st, sp, static_cast<const f16*>(mask),
                         ep, a);
      break;
    default:
      hipLaunchKernelGGL(mask_apply_fwd_kernel<bf16>, grid, dim3(kMaThreads), 0, st, sp,
                         static_cast<const bf16*>(mask), ep, a);
      break;
  }
  return check_launch("mask_apply_fwd_kernel");
}

int pmsst_mask_apply_backward(const void* grad_est, const void* spec, const void* mask, int64_t mask_batch_stride,
                              int64_t mask_stem_stride, int64_t batch, int64_t stems, int64_t channels, int64_t freqs,
                              int64_t frames, int zero_dc, void* grad_mask, void* grad_spec, int mask_dtype,
                              void* stream) {
  const char* op = "mask_apply_backward";
  const MaskApplyArgs a{batch, stems, channels, freqs, frames, mask_batch_stride, mask_stem_stride, zero_dc != 0};
  if (batch == 0) return PMSST_OK;
  PMSST_REQUIRE(grad_est && spec && mask && grad_mask, "%s: null pointer", op);
  int rc = check_mask_apply(op, a, spec, mask, mask_dtype);
  if (rc != PMSST_OK) return rc;
  const size_t esz = mask_dtype == PMSST_F32 ? 4 : 2;
  PMSST_REQUIRE(reinterpret_cast<uintptr_t>(grad_est) % 8 == 0 && reinterpret_cast<uintptr_t>(grad_mask) % (2 * esz) == 0 &&
                    reinterpret_cast<uintptr_t>(grad_spec) % 8 == 0,
                "%s: misaligned gradient", op);
  const int64_t FC = freqs * channels;
  const dim3 grid(static_cast<unsigned>((frames + kMaT - 1) / kMaT * ((FC + kMaR - 1) / kMaR)),
                  static_cast<unsigned>(batch));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float2* gp = static_cast<const float2*>(grad_est);
  const float2* sp = static_cast<const float2*>(spec);
  float2* gsp = static_cast<float2*>(grad_spec);
  switch (mask_dtype) {
    case PMSST_F32:
      hipLaunchKernelGGL(mask_apply_bwd_kernel<float>, grid, dim3(kMaThreads), 0, st, gp, sp,
                         static_cast<const float*>(mask), static_cast<float*>(grad_mask), gsp, a);
      break;
    case PMSST_F16:
      hipLaunchKernelGGL(mask_apply_bwd_kernel<f16>, grid, dim3(kMaThreads), 0, st, gp, sp,
                         static_cast<const f16*>(mask), static_cast<f16*>(grad_mask), gsp, a);
      break;
    default:
      hipLaunchKernelGGL(mask_apply_bwd_kernel<bf16>, grid, dim3(kMaThreads), 0, st, gp, sp,
                         static_cast<const bf16*>(mask), static_cast<bf16*>(grad_mask), gsp, a);
      break;
  }
  return check_launch("mask_apply_bwd_kernel");
}

}  // extern "C"
