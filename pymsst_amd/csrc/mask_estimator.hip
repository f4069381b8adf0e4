// Mask estimator final layer: per-band Linear H -> 2*I_b, bias, GLU; forward and
// backward on CDNA4 matrix cores.
//
// Layout (row-major):
//   x      [M, NB, H]
//   weight band-major concatenation of the per-band [2*I_b, H] weights (left rows first)
//   bias   [2F]    band b at [2*off_b, 2*off_b + 2*I_b)
//   pre    [M, 2F] x W^T + bias (saved for the backward)
//   out    [M, F]  left * sigmoid(gate)
// F = sum_b I_b.
//
// Forward block (m-tile of 64, band b, chunk of 64 GLU outputs l): each wave owns
// 16 outputs and computes both their left rows (l) and gate rows (I_b + l), so
// the GLU is applied to two accumulators held by the same lane.
//
// Backward: dpre = (g * s, g * L * s * (1 - s)) is recomputed from pre and
// grad_out while staging MFMA operands; it is never written to HBM.
//   dx block (m-tile, band, 256 hidden): dx^T[h][m] = W_b^T dpre^T, K = 2*I_b.
//   dW block (band, 64 j x 64 h): dW[j][h] = sum_m dpre[m][j] x[m][b][h], K = M;
//   blocks of the first h tile also reduce dbias.  No atomics.
#include "common.h"
#include "mfma.h"

namespace pmsst {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 64;

struct MaskArgs {
  const int64_t* offsets;  // device [NB + 1] (prefix sums of I_b)
  int64_t M;
  int NB;
  int H;
  int F;
  bool vec4;  // every I_b and H a multiple of 4 and all tensors 4-element aligned
};

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + __expf(-z)); }

// ------------------------------------------------------------------ forward

template <typename T>
__global__ __launch_bounds__(kThreads) void me_fwd_kernel(const T* __restrict__ x, const T* __restrict__ weight,
                                                          const T* __restrict__ bias, T* __restrict__ pre,
                                                          T* __restrict__ out, int max_lchunks, MaskArgs a) {
  constexpr int P = LdsPitch<T>::value;
  __shared__ T wl[64 * P];
  __shared__ T wg[64 * P];
  __shared__ T xs[kBM * P];

  const int band = blockIdx.y / max_lchunks;
  const int l0 = (blockIdx.y % max_lchunks) * 64;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  if (l0 >= I) return;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const int H = a.H;
  const T* wb = weight + static_cast<int64_t>(2) * off * H;  // [2I][H]
  const T* xb = x + (m0 * a.NB + band) * H;                   // row m at + m * NB * H

  f32x4_t accl[4], accg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) accl[j] = accg[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < H; k0 += kChunkK) {
    // 3 tiles of 64 rows x 32: left weights, gate weights, x  (768 quads per tile set, 3 per thread)
    stage_kcontig<T, 64, kThreads>(wl, wb + static_cast<int64_t>(l0) * H, H, I - l0, k0, H, a.vec4, tid);
    stage_kcontig<T, 64, kThreads>(wg, wb + static_cast<int64_t>(I + l0) * H, H, I - l0, k0, H, a.vec4, tid);
    stage_kcontig<T, kBM, kThreads>(xs, xb, static_cast<int64_t>(a.NB) * H, rows_valid, k0, H, a.vec4, tid);
    __syncthreads();
    const T* lrow = wl + (wave * 16 + (lane & 15)) * P;
    const T* grow = wg + (wave * 16 + (lane & 15)) * P;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const T* brow = xs + (j * 16 + (lane & 15)) * P;
      accl[j] = mfma_chunk<T>(lrow, brow, accl[j], lane);
      accg[j] = mfma_chunk<T>(grow, brow, accg[j], lane);
    }
    __syncthreads();
  }

  const int l = l0 + wave * 16 + 4 * (lane >> 4);
  if (l >= I) return;
  float bl[4], bg[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bl[r] = l + r < I ? to_f32(bias[2 * off + l + r]) : 0.f;
    bg[r] = l + r < I ? to_f32(bias[2 * off + I + l + r]) : 0.f;
  }
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = j * 16 + (lane & 15);
    if (m >= rows_valid) continue;
    float vl[4], vg[4], vo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vl[r] = accl[j][r] + bl[r];
      vg[r] = accg[j][r] + bg[r];
      vo[r] = vl[r] * sigmoidf_(vg[r]);
    }
    T* pl = pre + (m0 + m) * pitch2 + 2 * off + l;
    T* pg = pl + I;
    T* po = out + (m0 + m) * a.F + off + l;
    if (a.vec4) {
      store_pack<T, 4>(pl, vl);
      store_pack<T, 4>(pg, vg);
      store_pack<T, 4>(po, vo);
    } else {
      for (int r = 0; r < 4 && l + r < I; ++r) {
        pl[r] = from_f32<T>(vl[r]);
        pg[r] = from_f32<T>(vg[r]);
        po[r] = from_f32<T>(vo[r]);
      }
    }
  }
}

// ------------------------------------------------------------------ backward

// dpre for column j of band (width I) in one row: pre_row = pre + m * 2F + 2 * off,
// g_row = grad_out + m * F + off.
template <typename T>
__device__ __forceinline__ float dpre_at(const T* __restrict__ pre_row, const T* __restrict__ g_row, int I, int j) {
  const int l = j < I ? j : j - I;
  const float left = to_f32(pre_row[l]);
  const float gate = to_f32(pre_row[I + l]);
  const float s = sigmoidf_(gate);
  const float g = to_f32(g_row[l]);
  return j < I ? g * s : g * left * s * (1.0f - s);
}

// B tile for the dx GEMM: lds[m][k] = dpre[m0 + m][k0 + k], K-contiguous rows.
template <typename T>
__device__ __forceinline__ void stage_dpre_rows(T* __restrict__ lds, const T* __restrict__ pre,
                                                const T* __restrict__ gout, int64_t m0, int rows_valid, int off,
                                                int I, int F, int k0, int tid) {
  constexpr int P = LdsPitch<T>::value;
  const int K = 2 * I;
  for (int q = tid; q < kBM * (kChunkK / 4); q += kThreads) {
    const int r = q / (kChunkK / 4);
    const int kq = (q % (kChunkK / 4)) * 4;
    const T* prow = pre + (m0 + r) * 2 * static_cast<int64_t>(F) + 2 * off;
    const T* grow = gout + (m0 + r) * static_cast<int64_t>(F) + off;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + kq + j;
      const float v = (r < rows_valid && k < K) ? dpre_at(prow, grow, I, k) : 0.f;
      lds[r * P + kq + j] = from_f32<T>(v);
    }
  }
}

// A tile of the dx GEMM: lds[h][k] = W_b[k0 + k][h0 + h] (transposed: W_b rows are contiguous in h).
template <typename T, int ROWS>
__device__ __forceinline__ void stage_wT(T* __restrict__ lds, const T* __restrict__ wb, int H, int h0, int K, int k0,
                                         bool vec4, int tid) {
  constexpr int P = LdsPitch<T>::value;
  for (int q = tid; q < (ROWS / 4) * kChunkK; q += kThreads) {
    const int hq = (q % (ROWS / 4)) * 4;  // consecutive threads -> consecutive h quads (coalesced)
    const int k = q / (ROWS / 4);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (k0 + k < K) {
      const T* src = wb + static_cast<int64_t>(k0 + k) * H + h0 + hq;
      if (vec4 && h0 + hq + 4 <= H) {
        load_pack<T, 4>(src, v);
      } else {
        for (int j = 0; j < 4 && h0 + hq + j < H; ++j) v[j] = to_f32(src[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) lds[(hq + j) * P + k] = from_f32<T>(v[j]);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void me_bwd_dx_kernel(const T* __restrict__ gout, const T* __restrict__ pre,
                                                             const T* __restrict__ weight, T* __restrict__ dx,
                                                             int hchunks, MaskArgs a) {
  constexpr int P = LdsPitch<T>::value;
  constexpr int kBH = 256;  // hidden rows per block: 4 waves x 4 tiles x 16
  __shared__ T ws[kBH * P];
  __shared__ T ds[kBM * P];

  const int band = blockIdx.y;
  const int h0 = blockIdx.z * kBH;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int K = 2 * I;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const int H = a.H;
  const T* wb = weight + static_cast<int64_t>(2) * off * H;
  (void)hchunks;

  f32x4_t acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += kChunkK) {
    stage_wT<T, kBH>(ws, wb, H, h0, K, k0, a.vec4, tid);
    stage_dpre_rows<T>(ds, pre, gout, m0, rows_valid, off, I, a.F, k0, tid);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const T* arow = ws + (wave * 64 + t * 16 + (lane & 15)) * P;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = mfma_chunk<T>(arow, ds + (j * 16 + (lane & 15)) * P, acc[t][j], lane);
    }
    __syncthreads();
  }

#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int h = h0 + wave * 64 + t * 16 + 4 * (lane >> 4);
    if (h >= H) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = j * 16 + (lane & 15);
      if (m >= rows_valid) continue;
      T* dst = dx + ((m0 + m) * a.NB + band) * H + h;
      float v[4] = {acc[t][j][0], acc[t][j][1], acc[t][j][2], acc[t][j][3]};
      if (a.vec4) {
        store_pack<T, 4>(dst, v);
      } else {
        for (int r = 0; r < 4 && h + r < H; ++r) dst[r] = from_f32<T>(v[r]);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void me_bwd_dw_kernel(const T* __restrict__ gout, const T* __restrict__ pre,
                                                             const T* __restrict__ x, T* __restrict__ dw,
                                                             T* __restrict__ dbias, int max_jchunks, MaskArgs a) {
  constexpr int P = LdsPitch<T>::value;
  __shared__ T as[64 * P];  // [j][m]
  __shared__ T bs[64 * P];  // [h][m]
  __shared__ float sdb[4][64];

  const int h0 = blockIdx.x * 64;
  const int band = blockIdx.y / max_jchunks;
  const int j0 = (blockIdx.y % max_jchunks) * 64;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int K2 = 2 * I;
  if (j0 >= K2) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wj = (wave >> 1) * 32, wh = (wave & 1) * 32;
  const int H = a.H;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);

  f32x4_t acc[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v) acc[u][v] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float dbp0 = 0.f, dbp1 = 0.f;

  for (int64_t mb = 0; mb < a.M; mb += kChunkK) {
    const int k_valid = static_cast<int>(a.M - mb < kChunkK ? a.M - mb : kChunkK);
    if (tid < 128) {
      // A: lds[j][m] = dpre[mb + m][j0 + j]; thread -> j pair 2*(tid%32), m octet tid/32
      const int jj = 2 * (tid % 32);
      const int kb = (tid / 32) * 8;
      float v0[8], v1[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int m = kb + q;
        float e0 = 0.f, e1 = 0.f;
        if (m < k_valid) {
          const T* prow = pre + (mb + m) * pitch2 + 2 * off;
          const T* grow = gout + (mb + m) * static_cast<int64_t>(a.F) + off;
          if (j0 + jj < K2) e0 = dpre_at(prow, grow, I, j0 + jj);
          if (j0 + jj + 1 < K2) e1 = dpre_at(prow, grow, I, j0 + jj + 1);
        }
        v0[q] = e0;
        v1[q] = e1;
        dbp0 += e0;
        dbp1 += e1;
      }
      if constexpr (sizeof(T) == 2) {
        store_pack<T, 8>(as + jj * P + kb, v0);
        store_pack<T, 8>(as + (jj + 1) * P + kb, v1);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          as[jj * P + kb + q] = v0[q];
          as[(jj + 1) * P + kb + q] = v1[q];
        }
      }
    } else {
      // B: lds[h][m] = x[mb + m][band][h0 + h]; thread -> h pair, m octet
      const int t = tid - 128;
      const int hh = 2 * (t % 32);
      const int kb = (t / 32) * 8;
      float v0[8], v1[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int m = kb + q;
        float e0 = 0.f, e1 = 0.f;
        if (m < k_valid) {
          const T* src = x + ((mb + m) * a.NB + band) * static_cast<int64_t>(H) + h0 + hh;
          if (h0 + hh + 2 <= H && (H % 2 == 0)) {
            float e[2];
            load_pack<T, 2>(src, e);
            e0 = e[0];
            e1 = e[1];
          } else {
            if (h0 + hh < H) e0 = to_f32(src[0]);
            if (h0 + hh + 1 < H) e1 = to_f32(src[1]);
          }
        }
        v0[q] = e0;
        v1[q] = e1;
      }
      if constexpr (sizeof(T) == 2) {
        store_pack<T, 8>(bs + hh * P + kb, v0);
        store_pack<T, 8>(bs + (hh + 1) * P + kb, v1);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          bs[hh * P + kb + q] = v0[q];
          bs[(hh + 1) * P + kb + q] = v1[q];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const T* arow = as + (wj + u * 16 + (lane & 15)) * P;
#pragma unroll
      for (int v = 0; v < 2; ++v) acc[u][v] = mfma_chunk<T>(arow, bs + (wh + v * 16 + (lane & 15)) * P, acc[u][v], lane);
    }
    __syncthreads();
  }

  T* dwb = dw + static_cast<int64_t>(2) * off * H;  // [2I][H]
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int h = h0 + wh + v * 16 + (lane & 15);
      if (h >= H) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + wj + u * 16 + 4 * (lane >> 4) + r;
        if (j < K2) dwb[static_cast<int64_t>(j) * H + h] = from_f32<T>(acc[u][v][r]);
      }
    }
  }

  if (blockIdx.x == 0) {
    if (tid < 128) {
      sdb[tid / 32][2 * (tid % 32)] = dbp0;
      sdb[tid / 32][2 * (tid % 32) + 1] = dbp1;
    }
    __syncthreads();
    if (tid < 64 && j0 + tid < K2) {
      dbias[2 * off + j0 + tid] = from_f32<T>(sdb[0][tid] + sdb[1][tid] + sdb[2][tid] + sdb[3][tid]);
    }
  }
}

// ------------------------------------------------------------------ host side

struct HostMask {
  int NB, F, max_width;
  bool vec4;
};

int check_mask(const char* op, const int64_t* dim_inputs, int64_t band_count, int64_t H, HostMask* hm) {
  PMSST_REQUIRE(dim_inputs != nullptr && band_count > 0 && band_count < (1 << 16), "%s: bad band count", op);
  PMSST_REQUIRE(H > 0 && H < (1 << 20), "%s: bad hidden size %lld", op, (long long)H);
  int64_t total = 0, maxw = 0;
  bool vec4 = H % 4 == 0;
  for (int64_t b = 0; b < band_count; ++b) {
    PMSST_REQUIRE(dim_inputs[b] > 0, "%s: dim_inputs must be positive", op);
    if (dim_inputs[b] % 4 != 0) vec4 = false;
    total += dim_inputs[b];
    maxw = dim_inputs[b] > maxw ? dim_inputs[b] : maxw;
  }
  PMSST_REQUIRE(total < (int64_t{1} << 29), "%s: too many features", op);
  hm->NB = static_cast<int>(band_count);
  hm->F = static_cast<int>(total);
  hm->max_width = static_cast<int>(maxw);
  hm->vec4 = vec4;
  return PMSST_OK;
}

bool al(const void* p, size_t b) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % b == 0; }

template <typename T>
int launch_me_fwd(const void* x, const void* weight, const void* bias, const int64_t* offsets, const HostMask& hm,
                  int64_t M, int64_t H, void* pre, void* out, hipStream_t stream) {
  const char* op = "mask_estimator_final_forward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  if (M == 0) return PMSST_OK;
  PMSST_REQUIRE(x && weight && bias && offsets && pre && out, "%s: null pointer", op);
  MaskArgs a{offsets, M, hm.NB, static_cast<int>(H), hm.F, false};
  a.vec4 = hm.vec4 && al(x, 4 * sizeof(T)) && al(weight, 4 * sizeof(T)) && al(pre, 4 * sizeof(T)) &&
           al(out, 4 * sizeof(T));
  const int max_lchunks = (hm.max_width + 63) / 64;
  const dim3 grid(static_cast<unsigned>((M + kBM - 1) / kBM), static_cast<unsigned>(hm.NB * max_lchunks));
  hipLaunchKernelGGL((me_fwd_kernel<T>), grid, dim3(kThreads), 0, stream, static_cast<const T*>(x),
                     static_cast<const T*>(weight), static_cast<const T*>(bias), static_cast<T*>(pre),
                     static_cast<T*>(out), max_lchunks, a);
  return check_launch("me_fwd_kernel");
}

template <typename T>
int launch_me_bwd(const void* gout, const void* x, const void* pre, const void* weight, const int64_t* offsets,
                  const HostMask& hm, int64_t M, int64_t H, void* dx, void* dbias, void* dw, hipStream_t stream) {
  const char* op = "mask_estimator_final_backward";
  PMSST_REQUIRE(weight && offsets && dbias && dw && (M == 0 || (gout && x && pre && dx)), "%s: null pointer", op);
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  MaskArgs a{offsets, M, hm.NB, static_cast<int>(H), hm.F, false};
  a.vec4 = hm.vec4 && al(x, 4 * sizeof(T)) && al(weight, 4 * sizeof(T)) && al(pre, 4 * sizeof(T)) &&
           al(dx, 4 * sizeof(T));
  const T* pg = static_cast<const T*>(gout);
  const T* pp = static_cast<const T*>(pre);
  if (M > 0) {
    const int hchunks = static_cast<int>((H + 255) / 256);
    const dim3 grid(static_cast<unsigned>((M + kBM - 1) / kBM), static_cast<unsigned>(hm.NB),
                    static_cast<unsigned>(hchunks));
    hipLaunchKernelGGL((me_bwd_dx_kernel<T>), grid, dim3(kThreads), 0, stream, pg, pp, static_cast<const T*>(weight),
                       static_cast<T*>(dx), hchunks, a);
    int rc = check_launch("me_bwd_dx_kernel");
    if (rc != PMSST_OK) return rc;
  }
  const int max_jchunks = (2 * hm.max_width + 63) / 64;
  const dim3 grid(static_cast<unsigned>((H + 63) / 64), static_cast<unsigned>(hm.NB * max_jchunks));
  hipLaunchKernelGGL((me_bwd_dw_kernel<T>), grid, dim3(kThreads), 0, stream, pg, pp, static_cast<const T*>(x),
                     static_cast<T*>(dw), static_cast<T*>(dbias), max_jchunks, a);
  return check_launch("me_bwd_dw_kernel");
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

}  // namespace
}  // namespace pmsst

using namespace pmsst;

extern "C" {

int pmsst_mask_estimator_final_forward(const void* x, const void* weight, const void* bias,
                                       const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                       int64_t rows, int64_t hidden, void* pre, void* out, int dtype, void* stream) {
  HostMask hm;
  int rc = check_mask("mask_estimator_final_forward", dim_inputs, band_count, hidden, &hm);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "mask_estimator_final_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_me_fwd<T>(x, weight, bias, dim_offsets, hm, rows, hidden, pre, out,
                            static_cast<hipStream_t>(stream));
  });
}

int pmsst_mask_estimator_final_backward(const void* grad_out, const void* x, const void* pre, const void* weight,
                                        const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                        int64_t rows, int64_t hidden, void* grad_x, void* grad_bias,
                                        void* grad_weight, int dtype, void* stream) {
  HostMask hm;
  int rc = check_mask("mask_estimator_final_backward", dim_inputs, band_count, hidden, &hm);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "mask_estimator_final_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_me_bwd<T>(grad_out, x, pre, weight, dim_offsets, hm, rows, hidden, grad_x, grad_bias, grad_weight,
                            static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
