// Band split front end: per-band RMSNorm + per-band Linear over the ragged
// feature axis, forward and backward, on CDNA4 matrix cores.
//
// Data layout in HBM (all row-major):
//   x        [M, x_stride]   band b occupies columns [off_b, off_b + I_b)
//   gamma    [F]             band-major concatenation of the per-band gammas
//   weight   sum_b O*I_b     band-major concatenation of the per-band [O, I_b] weights
//   bias     [NB, O]         (optional)
//   out      [M, NB, O]
//   normed   [M, F]          x * inv * sqrt(I_b) (optional output)
//   inv_norm [M, NB] fp32
// F = sum_b I_b, 1 <= O <= 512 (tiles hold 64 * TO outputs; rows o >= O are zero).
//
// Forward block (m-tile of 64 rows, band b): out^T[o][m] = W_b (x*gamma)^T with
// K = I_b streamed through LDS in chunks of 32; the row sum of squares is
// accumulated while x is staged, and the epilogue applies inv*sqrt(I_b) and the
// bias.  Each lane stores 4 consecutive outputs of one row.
//
// Backward dx block (m-tile, band): gs^T[i][m] = W_b^T dy^T in 64-wide i chunks,
// two passes (pass 1 forms the per-row dot(gs*gamma, n) and the dgamma
// partials, pass 2 recomputes gs and writes dx).  dgamma partials go to a
// [m_tiles, F] fp32 workspace reduced by col_sum_kernel.
//
// Backward dW block (band, 64 o x 64 i tile): dW[o][i] = sum_m dy[m,o] n[m,i] gamma_i
// over all M, both operands staged transposed (row-major in m); blocks of the
// first i tile also reduce dbias.  No atomics anywhere.
#include "common.h"
#include "mfma.h"
#include "rowgeom.h"

#include <vector>

namespace pmsst {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 64;

struct BandArgs {
  const int64_t* offsets;  // device [NB + 1]
  int64_t M;
  int NB;
  int F;              // total input features (row pitch of normed / dx / saved input)
  int64_t x_stride;   // row pitch of x in the forward
  int O;              // out_features (<= the kernel's tile capacity 64 * TO)
  bool vec4;          // all offsets, pitches and widths are multiples of 4 elements
  bool ovec4;         // O % 4 == 0 and out / bias / grad_out are 4-element aligned
};

// ------------------------------------------------------------------ forward

template <typename T, int TO, bool WRITE_NORMED, bool NORM>
__global__ __launch_bounds__(kThreads) void bs_fwd_kernel(const T* __restrict__ x, const T* __restrict__ gamma,
                                                          const T* __restrict__ weight, const T* __restrict__ bias,
                                                          T* __restrict__ out, T* __restrict__ normed,
                                                          float* __restrict__ inv_norm, BandArgs a) {
  constexpr int OT = 64 * TO;
  constexpr int P = LdsPitch<T>::value;
  __shared__ T ws[OT * P];
  __shared__ T xs[kBM * P];
  __shared__ float sscale[kBM];

  const int O = a.O;
  const int band = blockIdx.y;
  const int oc = blockIdx.z * OT;  // first output of this block's chunk
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const T* xb = x + m0 * a.x_stride + off;
  const T* wb = weight + static_cast<int64_t>(O) * off + static_cast<int64_t>(oc) * I;

  f32x4_t acc[TO][4];
#pragma unroll
  for (int t = 0; t < TO; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[t][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // x staging: thread -> rows (tid/8) and (tid/8 + 32), k quad (tid%8)*4, fixed for all chunks.
  const int xr = tid >> 3, xq = (tid & 7) * 4;
  float ss0 = 0.f, ss1 = 0.f;

  for (int k0 = 0; k0 < I; k0 += kChunkK) {
    const int k = k0 + xq;
    float g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = (k + j < I) ? (NORM ? to_f32(gamma[off + k + j]) : 1.f) : 0.f;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = xr + 32 * p;
      float v[4];
      if (r < rows_valid && a.vec4 && k + 4 <= I) {
        load_pack<T, 4>(xb + r * a.x_stride + k, v);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (r < rows_valid && k + j < I) ? to_f32(xb[r * a.x_stride + k + j]) : 0.f;
      }
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s += v[j] * v[j];
        xs[r * P + xq + j] = from_f32<T>(v[j] * g[j]);
      }
      if (p == 0) ss0 += s; else ss1 += s;
    }
    stage_kcontig<T, OT, kThreads>(ws, wb, I, O - oc, k0, I, a.vec4, tid);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TO; ++t) {
      const T* arow = ws + (wave * 16 * TO + t * 16 + (lane & 15)) * P;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][j] = mfma_chunk<T>(arow, xs + (j * 16 + (lane & 15)) * P, acc[t][j], lane);
    }
    __syncthreads();
  }

  const float root = sqrtf(static_cast<float>(I));
  ss0 = group_sum(ss0, 8);
  ss1 = group_sum(ss1, 8);
  if ((tid & 7) == 0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = xr + 32 * p;
      const float inv = 1.0f / fmaxf(sqrtf(p == 0 ? ss0 : ss1), 1.0e-12f);
      sscale[r] = NORM ? inv * root : 1.0f;
      if (NORM && blockIdx.z == 0 && r < rows_valid) inv_norm[(m0 + r) * a.NB + band] = inv;
    }
  }
  __syncthreads();

#pragma unroll
  for (int t = 0; t < TO; ++t) {
    const int o = oc + wave * 16 * TO + t * 16 + 4 * (lane >> 4);
    if (o >= O) continue;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr) {
      if (a.ovec4) {
        load_pack<T, 4>(bias + static_cast<int64_t>(band) * O + o, bv);
      } else {
        for (int r = 0; r < 4 && o + r < O; ++r) bv[r] = to_f32(bias[static_cast<int64_t>(band) * O + o + r]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = j * 16 + (lane & 15);
      if (m < rows_valid) {
        const float s = sscale[m];
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = acc[t][j][r] * s + bv[r];
        T* dst = out + ((m0 + m) * a.NB + band) * O + o;
        if (a.ovec4) {
          store_pack<T, 4>(dst, v);
        } else {
          for (int r = 0; r < 4 && o + r < O; ++r) dst[r] = from_f32<T>(v[r]);
        }
      }
    }
  }

  if (WRITE_NORMED && blockIdx.z == 0) {
    for (int q = tid; q < kBM * ((I + 3) / 4); q += kThreads) {
      const int r = q / ((I + 3) / 4);
      const int k = (q % ((I + 3) / 4)) * 4;
      if (r >= rows_valid) continue;
      const float s = sscale[r];
      T* dst = normed + (m0 + r) * a.F + off + k;
      const T* srcp = xb + r * a.x_stride + k;
      if (a.vec4 && k + 4 <= I) {
        float v[4];
        load_pack<T, 4>(srcp, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] *= s;
        store_pack<T, 4>(dst, v);
      } else {
        for (int j = 0; j < 4 && k + j < I; ++j) dst[j] = from_f32<T>(to_f32(srcp[j]) * s);
      }
    }
  }
}

// ------------------------------------------------------------------ transposed staging

// Stage lds[mn][k] = src[(k0 + k) * kstride + mn0 + mn] * rs[k] * cs[mn0 + mn] for
// mn < ROWS, k < 32 (zero outside mn_valid / k_valid).  `rs` (LDS, chunk-relative)
// and `cs` (global) are optional.  `group_tid` runs over [0, GROUP).
template <typename T, int ROWS, int GROUP>
__device__ __forceinline__ void stage_mncontig(T* __restrict__ lds, const T* __restrict__ src, int64_t kstride,
                                               int mn_valid, int k0, int k_valid, bool vec2, int group_tid,
                                               const float* __restrict__ rs, const T* __restrict__ cs) {
  constexpr int P = LdsPitch<T>::value;
  constexpr int kPairs = ROWS / 2;
  for (int w = group_tid; w < kPairs * (kChunkK / 8); w += GROUP) {
    const int mn = 2 * (w % kPairs);
    const int kb = (w / kPairs) * 8;
    const float c0 = (cs != nullptr && mn < mn_valid) ? to_f32(cs[mn]) : 1.f;
    const float c1 = (cs != nullptr && mn + 1 < mn_valid) ? to_f32(cs[mn + 1]) : 1.f;
    float v0[8], v1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + kb + j;
      float e0 = 0.f, e1 = 0.f;
      if (k < k_valid) {
        const T* p = src + static_cast<int64_t>(k) * kstride + mn;
        if (vec2 && mn + 2 <= mn_valid) {
          float e[2];
          load_pack<T, 2>(p, e);
          e0 = e[0];
          e1 = e[1];
        } else {
          if (mn < mn_valid) e0 = to_f32(p[0]);
          if (mn + 1 < mn_valid) e1 = to_f32(p[1]);
        }
        const float r = rs != nullptr ? rs[kb + j] : 1.f;
        e0 *= r;
        e1 *= r;
      }
      v0[j] = e0 * c0;
      v1[j] = e1 * c1;
    }
    if constexpr (sizeof(T) == 2) {
      store_pack<T, 8>(lds + mn * P + kb, v0);
      store_pack<T, 8>(lds + (mn + 1) * P + kb, v1);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        lds[mn * P + kb + j] = v0[j];
        lds[(mn + 1) * P + kb + j] = v1[j];
      }
    }
  }
}

// ------------------------------------------------------------------ backward: dx + dgamma partials

template <typename T, bool FROM_X>
__global__ __launch_bounds__(kThreads) void bs_bwd_dx_kernel(const T* __restrict__ dy, const T* __restrict__ nsrc,
                                                             const float* __restrict__ inv_norm,
                                                             const T* __restrict__ gamma, const T* __restrict__ weight,
                                                             T* __restrict__ dx, float* __restrict__ dg_partial,
                                                             BandArgs a) {
  constexpr int P = LdsPitch<T>::value;
  constexpr int kBI = 64;  // i rows per chunk (4 waves x 16)
  const int O = a.O;
  __shared__ T ws[kBI * P];
  __shared__ T ys[kBM * P];
  __shared__ float sinv[kBM];
  __shared__ float sdot[4][kBM];

  const int band = blockIdx.y;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const T* wb = weight + static_cast<int64_t>(O) * off;       // [O][I]
  const T* dyb = dy + (m0 * a.NB + band) * O;                   // row m at + m * NB * O
  const float root = sqrtf(static_cast<float>(I));

  if (tid < kBM) sinv[tid] = tid < rows_valid ? inv_norm[(m0 + tid) * a.NB + band] : 0.f;
  __syncthreads();

  float dotp[4] = {0.f, 0.f, 0.f, 0.f};  // per m-tile j, for m = j*16 + (lane & 15)

  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      // fold the row dots: lanes sharing (lane & 15), then waves
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = dotp[j];
        v += __shfl_xor(v, 16, kWave);
        v += __shfl_xor(v, 32, kWave);
        if (lane < 16) sdot[wave][j * 16 + lane] = v;
      }
      __syncthreads();
      if (tid < kBM) sdot[0][tid] = sdot[0][tid] + sdot[1][tid] + sdot[2][tid] + sdot[3][tid];
      __syncthreads();
    }
    for (int i0 = 0; i0 < I; i0 += kBI) {
      f32x4_t acc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int k0 = 0; k0 < O; k0 += kChunkK) {
        // A[i][o] = W_b[o][i0 + i]  (transposed staging, 128 threads)  |  B[m][o] = dy[m][o]
        if (tid < 128) {
          stage_mncontig<T, kBI, 128>(ws, wb + i0, I, I - i0, k0, O, a.vec4, tid, nullptr, nullptr);
        } else {
          stage_kcontig<T, kBM, 128>(ys, dyb, static_cast<int64_t>(a.NB) * O, rows_valid, k0, O, a.ovec4,
                                     tid - 128);
        }
        __syncthreads();
        const T* arow = ws + (wave * 16 + (lane & 15)) * P;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = mfma_chunk<T>(arow, ys + (j * 16 + (lane & 15)) * P, acc[j], lane);
        __syncthreads();
      }
      // lane holds gs[m = j*16 + (lane&15)][i = i0 + wave*16 + 4*(lane>>4) + r]
      const int il = i0 + wave * 16 + 4 * (lane >> 4);
      float g[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) g[r] = il + r < I ? to_f32(gamma[off + il + r]) : 0.f;
      float dgp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = j * 16 + (lane & 15);
        if (m >= rows_valid || il >= I) continue;
        const T* np = nsrc + (m0 + m) * a.F + off + il;
        float n[4];
        if (a.vec4) {
          load_pack<T, 4>(np, n);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) n[r] = il + r < I ? to_f32(np[r]) : 0.f;
        }
        if (FROM_X) {
          const float s = sinv[m] * root;
#pragma unroll
          for (int r = 0; r < 4; ++r) n[r] *= s;
        }
        if (pass == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dotp[j] += acc[j][r] * g[r] * n[r];
            dgp[r] += acc[j][r] * n[r];
          }
        } else {
          const float inv = sinv[m];
          const float dots = sdot[0][m] / root;
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = inv * (acc[j][r] * g[r] * root - n[r] * dots);
          T* dp = dx + (m0 + m) * a.F + off + il;
          if (a.vec4) {
            store_pack<T, 4>(dp, o);
          } else {
            for (int r = 0; r < 4 && il + r < I; ++r) dp[r] = from_f32<T>(o[r]);
          }
        }
      }
      if (pass == 0) {
        // dgamma partial for this m-tile: sum over the 16 lanes sharing (lane >> 4)
#pragma unroll
        for (int r = 0; r < 4; ++r) dgp[r] = group_sum(dgp[r], 16);
        if ((lane & 15) == 0) {
          float* dst = dg_partial + static_cast<int64_t>(blockIdx.x) * a.F + off;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (il + r < I) dst[il + r] = dgp[r];
        }
      }
    }
  }
}

// ------------------------------------------------------------------ backward: dW, dbias

template <typename T, bool FROM_X>
__global__ __launch_bounds__(kThreads) void bs_bwd_dw_kernel(const T* __restrict__ dy, const T* __restrict__ nsrc,
                                                             const float* __restrict__ inv_norm,
                                                             const T* __restrict__ gamma, T* __restrict__ dw,
                                                             T* __restrict__ db, int O, int max_itiles, BandArgs a) {
  constexpr int P = LdsPitch<T>::value;
  __shared__ T as[64 * P];  // [o][m]
  __shared__ T bs[64 * P];  // [i][m]
  __shared__ float srs[kChunkK];
  __shared__ float sdb[4][64];

  const int o0 = blockIdx.x * 64;
  const int band = blockIdx.y / max_itiles;
  const int it = blockIdx.y % max_itiles;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int i0 = it * 64;
  if (i0 >= I) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wo = (wave >> 1) * 32, wi = (wave & 1) * 32;  // 2x2 waves, 32x32 each
  const float root = sqrtf(static_cast<float>(I));
  const T* dyb = dy + static_cast<int64_t>(band) * O + o0;  // element (m, o) at + m * NB * O + o
  const T* nb = nsrc + off + i0;                              // element (m, i) at + m * F + i

  f32x4_t acc[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < 2; ++v) acc[u][v] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float dbp0 = 0.f, dbp1 = 0.f;

  for (int64_t mb = 0; mb < a.M; mb += kChunkK) {
    const int k_valid = static_cast<int>(a.M - mb < kChunkK ? a.M - mb : kChunkK);
    if (FROM_X && tid < kChunkK) {
      srs[tid] = tid < k_valid ? inv_norm[(mb + tid) * a.NB + band] * root : 0.f;
    }
    if (FROM_X) __syncthreads();
    if (tid < 128) {
      stage_mncontig<T, 64, 128>(as, dyb + mb * a.NB * O, static_cast<int64_t>(a.NB) * O, O - o0, 0, k_valid,
                                 O % 2 == 0, tid, nullptr, nullptr);
      if (it == 0) {
        // dbias partials: this thread staged o pair (2*(tid%32)) for m octet (tid/32)
        const int mn = 2 * (tid % 32);
        const int kb = (tid / 32) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          dbp0 += to_f32(as[mn * P + kb + j]);
          dbp1 += to_f32(as[(mn + 1) * P + kb + j]);
        }
      }
    } else {
      stage_mncontig<T, 64, 128>(bs, nb + mb * a.F, a.F, I - i0, 0, k_valid, a.vec4, tid - 128,
                                 FROM_X ? srs : nullptr, gamma + off + i0);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const T* arow = as + (wo + u * 16 + (lane & 15)) * P;
#pragma unroll
      for (int v = 0; v < 2; ++v) acc[u][v] = mfma_chunk<T>(arow, bs + (wi + v * 16 + (lane & 15)) * P, acc[u][v], lane);
    }
    __syncthreads();
  }

  T* dwb = dw + static_cast<int64_t>(O) * off;  // [O][I]
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int i = i0 + wi + v * 16 + (lane & 15);
      if (i >= I) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = o0 + wo + u * 16 + 4 * (lane >> 4) + r;
        if (o < O) dwb[static_cast<int64_t>(o) * I + i] = from_f32<T>(acc[u][v][r]);
      }
    }
  }

  if (it == 0 && db != nullptr) {
    // threads 0..127: o pair 2*(tid%32), m octet tid/32 -> sum the 4 octets
    if (tid < 128) {
      sdb[tid / 32][2 * (tid % 32)] = dbp0;
      sdb[tid / 32][2 * (tid % 32) + 1] = dbp1;
    }
    __syncthreads();
    if (tid < 64 && o0 + tid < O) {
      const float s = sdb[0][tid] + sdb[1][tid] + sdb[2][tid] + sdb[3][tid];
      db[static_cast<int64_t>(band) * O + o0 + tid] = from_f32<T>(s);
    }
  }
}

// ------------------------------------------------------------------ host side

struct HostBands {
  int NB;
  int F;
  int max_width;
  bool vec4;
};

int check_bands(const char* op, const int64_t* dim_inputs, int64_t band_count, HostBands* hb) {
  PMSST_REQUIRE(dim_inputs != nullptr && band_count > 0 && band_count < (1 << 16), "%s: bad band count %lld", op,
                (long long)band_count);
  int64_t total = 0, maxw = 0;
  bool vec4 = true;
  for (int64_t b = 0; b < band_count; ++b) {
    PMSST_REQUIRE(dim_inputs[b] > 0, "%s: dim_inputs must be positive", op);
    if (total % 4 != 0 || dim_inputs[b] % 4 != 0) vec4 = false;
    total += dim_inputs[b];
    maxw = dim_inputs[b] > maxw ? dim_inputs[b] : maxw;
  }
  PMSST_REQUIRE(total < (int64_t{1} << 30), "%s: too many features", op);
  hb->NB = static_cast<int>(band_count);
  hb->F = static_cast<int>(total);
  hb->max_width = static_cast<int>(maxw);
  hb->vec4 = vec4;
  return PMSST_OK;
}

// 64-wide output tiles needed for O outputs, rounded up to an instantiated capacity.
int tile_capacity(int64_t O) {
  const int64_t t = (O + 63) / 64;
  return t <= 4 ? static_cast<int>(t) : 8;
}

bool aligned_to(const void* p, size_t bytes) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % bytes == 0; }

// norm = false runs the same kernel as a plain grouped linear (gamma, normed and inv_norm unused).
template <typename T>
int launch_fwd(const void* x, int64_t x_stride, const void* gamma, const void* weight, const void* bias,
               const int64_t* offsets, const HostBands& hb, int64_t M, int64_t O, void* out, void* normed,
               float* inv_norm, bool norm, hipStream_t stream) {
  const char* op = norm ? "band_split_ragged_forward" : "grouped_linear_forward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && (O <= 512 || !norm) && O < (1 << 20), "%s: bad out_features %lld", op, (long long)O);
  if (M == 0) return PMSST_OK;
  PMSST_REQUIRE(x && weight && offsets && out && (!norm || (gamma && inv_norm)), "%s: null pointer", op);
  PMSST_REQUIRE(x_stride >= hb.F, "%s: x row stride %lld < total features %d", op, (long long)x_stride, hb.F);
  BandArgs a{offsets, M, hb.NB, hb.F, x_stride, static_cast<int>(O), false, false};
  a.vec4 = hb.vec4 && x_stride % 4 == 0 && aligned_to(x, 4 * sizeof(T)) && aligned_to(normed, 4 * sizeof(T)) &&
           aligned_to(weight, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(out, 4 * sizeof(T)) && aligned_to(bias, 4 * sizeof(T));
  const int cap = 64 * tile_capacity(O);
  const dim3 grid(static_cast<unsigned>((M + kBM - 1) / kBM), static_cast<unsigned>(hb.NB),
                  static_cast<unsigned>((O + cap - 1) / cap));
  const T* px = static_cast<const T*>(x);
  const T* pg = static_cast<const T*>(gamma);
  const T* pw = static_cast<const T*>(weight);
  const T* pb = static_cast<const T*>(bias);
  T* po = static_cast<T*>(out);
  T* pn = static_cast<T*>(normed);
#define PMSST_BSF(TO)                                                                                            \
  do {                                                                                                           \
    if (!norm)                                                                                                   \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, false, false>), grid, dim3(kThreads), 0, stream, px, pg, pw, pb,  \
                         po, pn, inv_norm, a);                                                                   \
    else if (pn != nullptr)                                                                                      \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, true, true>), grid, dim3(kThreads), 0, stream, px, pg, pw, pb,    \
                         po, pn, inv_norm, a);                                                                   \
    else                                                                                                         \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, false, true>), grid, dim3(kThreads), 0, stream, px, pg, pw, pb,   \
                         po, pn, inv_norm, a);                                                                   \
  } while (0)
  switch (tile_capacity(O)) {
    case 1: PMSST_BSF(1); break;
    case 2: PMSST_BSF(2); break;
    case 3: PMSST_BSF(3); break;
    case 4: PMSST_BSF(4); break;
    default: PMSST_BSF(8); break;
  }
#undef PMSST_BSF
  return check_launch("bs_fwd_kernel");
}

size_t bwd_workspace(int64_t M, int F) {
  return static_cast<size_t>((M + kBM - 1) / kBM) * static_cast<size_t>(F) * sizeof(float);
}

template <typename T>
int launch_bwd(const void* dy, const void* nsrc, bool from_x, const float* inv_norm, const void* gamma,
               const void* weight, const int64_t* offsets, const HostBands& hb, int64_t M, int64_t O, void* dx,
               void* dgamma, void* dw, void* db, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* op = "band_split_ragged_backward";
  PMSST_REQUIRE(gamma && weight && offsets && dgamma && dw && (M == 0 || (dy && nsrc && inv_norm && dx)),
                "%s: null pointer", op);
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && O <= 512, "%s: out_features must be in [1, 512] (got %lld)", op, (long long)O);
  const size_t need = bwd_workspace(M, hb.F);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(PMSST_EWORKSPACE, "%s: workspace of %zu bytes needed", op, need);
  }
  BandArgs a{offsets, M, hb.NB, hb.F, hb.F, static_cast<int>(O), false, false};
  a.vec4 = hb.vec4 && aligned_to(nsrc, 4 * sizeof(T)) && aligned_to(dx, 4 * sizeof(T)) &&
           aligned_to(weight, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(dy, 4 * sizeof(T));
  const T* pdy = static_cast<const T*>(dy);
  const T* pn = static_cast<const T*>(nsrc);
  const T* pg = static_cast<const T*>(gamma);
  const T* pw = static_cast<const T*>(weight);
  float* partial = static_cast<float*>(workspace);
  const int m_tiles = static_cast<int>((M + kBM - 1) / kBM);
  if (M > 0) {
    const dim3 grid(static_cast<unsigned>(m_tiles), static_cast<unsigned>(hb.NB));
    if (from_x)
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, true>), grid, dim3(kThreads), 0, stream, pdy, pn, inv_norm, pg, pw,
                         static_cast<T*>(dx), partial, a);
    else
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, false>), grid, dim3(kThreads), 0, stream, pdy, pn, inv_norm, pg, pw,
                         static_cast<T*>(dx), partial, a);
    int rc = check_launch("bs_bwd_dx_kernel");
    if (rc != PMSST_OK) return rc;
  }
  {
    const int max_itiles = (hb.max_width + 63) / 64;
    const dim3 grid(static_cast<unsigned>((O + 63) / 64), static_cast<unsigned>(hb.NB * max_itiles));
    if (from_x)
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, true>), grid, dim3(kThreads), 0, stream, pdy, pn, inv_norm, pg,
                         static_cast<T*>(dw), static_cast<T*>(db), static_cast<int>(O), max_itiles, a);
    else
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, false>), grid, dim3(kThreads), 0, stream, pdy, pn, inv_norm, pg,
                         static_cast<T*>(dw), static_cast<T*>(db), static_cast<int>(O), max_itiles, a);
    int rc = check_launch("bs_bwd_dw_kernel");
    if (rc != PMSST_OK) return rc;
  }
  return launch_col_sum(partial, m_tiles, hb.F, dgamma, dtype_code<T>(), stream);
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

int pmsst_band_split_ragged_forward(const void* x, int64_t x_row_stride, const void* gamma, const void* weight,
                                    const void* bias, const int64_t* dim_offsets, const int64_t* dim_inputs,
                                    int64_t band_count, int64_t rows, int64_t out_features, void* out, void* normed,
                                    float* inv_norm, int dtype, void* stream) {
  HostBands hb;
  int rc = check_bands("band_split_ragged_forward", dim_inputs, band_count, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "band_split_ragged_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T>(x, x_row_stride, gamma, weight, bias, dim_offsets, hb, rows, out_features, out, normed,
                         inv_norm, true, static_cast<hipStream_t>(stream));
  });
}

int pmsst_grouped_linear_forward(const void* x, int64_t x_row_stride, const void* weight, const void* bias,
                                 const int64_t* group_offsets, int64_t groups, int64_t in_features, int64_t rows,
                                 int64_t out_features, void* out, int dtype, void* stream) {
  PMSST_REQUIRE(groups > 0 && groups < (1 << 16) && in_features > 0, "grouped_linear_forward: bad shape");
  std::vector<int64_t> dims(static_cast<size_t>(groups), in_features);
  HostBands hb;
  int rc = check_bands("grouped_linear_forward", dims.data(), groups, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "grouped_linear_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T>(x, x_row_stride, nullptr, weight, bias, group_offsets, hb, rows, out_features, out, nullptr,
                         nullptr, false, static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_band_split_ragged_backward_workspace_size(int64_t rows, int64_t total_in) {
  if (rows <= 0 || total_in <= 0) return 0;
  return bwd_workspace(rows, static_cast<int>(total_in));
}

int pmsst_band_split_ragged_backward(const void* grad_out, const void* saved, int saved_is_input,
                                     const float* inv_norm, const void* gamma, const void* weight,
                                     const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                     int64_t rows, int64_t out_features, void* grad_x, void* grad_gamma,
                                     void* grad_weight, void* grad_bias, int dtype, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  HostBands hb;
  int rc = check_bands("band_split_ragged_backward", dim_inputs, band_count, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "band_split_ragged_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_bwd<T>(grad_out, saved, saved_is_input != 0, inv_norm, gamma, weight, dim_offsets, hb, rows,
                         out_features, grad_x, grad_gamma, grad_weight, grad_bias, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
