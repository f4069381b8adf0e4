// Band split front end: per-band RMSNorm + per-band Linear over the ragged
// feature axis, forward and backward, on CDNA4 matrix cores (gemm.h main loop).
//
// Data layout in HBM (all row-major):
//   x        [M, x_stride]   band b occupies columns [off_b, off_b + I_b)
//   gamma    [F]             band-major concatenation of the per-band gammas
//   weight   sum_b O*I_b     band-major concatenation of the per-band [O, I_b] weights
//   bias     [NB, O]         (optional)
//   out      [M, NB, O]
//   normed   [M, F]          x * inv * sqrt(I_b) (optional output)
//   inv_norm [M, NB] fp32
// F = sum_b I_b, 1 <= O <= 512.
//
// Forward block (64 rows, band b, <= 256 outputs): out^T[o][m] = W_b (x*gamma)^T,
// K = I_b.  The x loader multiplies by gamma on the way into LDS and sums x^2
// for its rows, so the epilogue applies inv*sqrt(I_b) and the bias; each lane
// stores 4 consecutive outputs of one row.  With norm off the same kernel is
// the grouped linear of the mask-MLP hidden layer.
//
// Backward dx block (64 rows, band b, 64-wide input chunk): gs^T[i][m] = W_b^T dy^T
// (K = O) on MFMA; the block writes t = gs * gamma (fp32), its chunk's part of the
// per-row dot(gs * gamma, n) and the dgamma partials ([m_tiles, F], reduced by
// col_sum_kernel).  A finish pass over the same blocks adds the dot partials of the
// band's chunks and writes dx = inv (t sqrt(I) - n dot / sqrt(I)).  dW block
// (band, 64 i x 64 o): dW^T[i][o] = sum_m n[m][i] gamma_i dy[m][o], K = M.  dbias =
// column sums of dy.  No atomics anywhere.
#include "common.h"
#include "dma_gemm.h"
#include "gemm.h"
#include "grouped_dx.h"
#include "rowgeom.h"

#include <vector>

// K-loop prefetch depth (chunks in registers ahead of the one in use) of each kernel
#ifndef PMSST_BS_FWD_DEPTH
#define PMSST_BS_FWD_DEPTH 2
#endif
#ifndef PMSST_BS_DX_DEPTH
#define PMSST_BS_DX_DEPTH 1
#endif
#ifndef PMSST_BS_DW_DEPTH
#define PMSST_BS_DW_DEPTH 1
#endif

namespace pmsst {
namespace {

constexpr int kBM = 64;

struct BandArgs {
  const int64_t* offsets;  // device [NB + 1]
  int64_t M;
  int NB;
  int F;              // total input features (row pitch of normed / dx / saved input)
  int64_t x_stride;   // row pitch of x in the forward
  int O;              // out_features
  bool vec4;          // all offsets, pitches and widths are multiples of 4 elements
  bool ovec4;         // O % 4 == 0 and out / bias / grad_out are 4-element aligned
  bool ovec8;         // 16-bit, O % 8 == 0, out 16-byte aligned and bias 4-element aligned:
                      // the forward stages its output tile through LDS
};

// B operand of the forward: rows m of x (K = band features) scaled by gamma;
// keeps the running sum of squares of the raw values of its two rows
// (rows tid/8 and tid/8 + 32, k quad (tid%8)*4 of every chunk).  gamma for the
// thread's k quad is fetched with the chunk.  Rows past rows_valid are clamped to the
// last valid row in interior chunks (their outputs and sums are discarded).
template <typename T, bool NORM, bool V4>
struct XGammaLoader {
  static constexpr int kQuads = kBM * (kChunkK / 4) / kGemmThreads;
  static_assert(kQuads == 2, "two rows per thread");
  struct Regs {
    quad_t<T> q[kQuads];
    quad_t<T> g;
    uint32_t ok;
  };
  const T* base;
  int64_t stride;
  const T* gamma;  // band gamma (k indexed)
  int rows_valid;
  int k_valid;
  mutable float ss[kQuads] = {0.f, 0.f};
  int64_t src_row[kQuads] = {};
  uint32_t off[kQuads] = {};

  static __device__ __forceinline__ int tile_row(int i) {
    return (static_cast<int>(threadIdx.x) + i * kGemmThreads) / (kChunkK / 4);
  }
  static __device__ __forceinline__ int lane_k() { return (threadIdx.x % (kChunkK / 4)) * 4; }

  __device__ __forceinline__ void prepare() {
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      const int r = tile_row(i);
      src_row[i] = r < rows_valid ? r : rows_valid - 1;
      off[i] = static_cast<uint32_t>((src_row[i] * stride + lane_k()) * static_cast<int64_t>(sizeof(T)));
    }
  }
  __device__ __forceinline__ void fetch_edge(int k0, Regs& g) const {
    const int k = k0 + lane_k();
    g.ok = 0;
#pragma unroll
    for (int i = 0; i < kQuads; ++i)
      g.q[i] = fetch_quad_k<T, V4>(base + src_row[i] * stride + k, base, tile_row(i) < rows_valid, k, k_valid, g.ok, i);
    if (NORM) g.g = fetch_quad_k<T, V4>(gamma + k, gamma, true, k, k_valid, g.ok, kQuads);
  }
  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    if constexpr (V4) {
#pragma unroll
      for (int i = 0; i < kQuads; ++i) g.q[i] = quad_at<T>(base + k0, off[i]);
      if (NORM) g.g = quad_at<T>(gamma + k0, static_cast<uint32_t>(lane_k() * sizeof(T)));
    } else {
      fetch_edge(k0, g);
    }
  }
  __device__ __forceinline__ void commit_impl(const Regs& g, T* lds, bool masked) const {
    const int kq = lane_k();
    if constexpr (!NORM) {
      // plain grouped linear: no gamma, no sums of squares
#pragma unroll
      for (int i = 0; i < kQuads; ++i)
        commit_quad<T>(lds, tile_row(i), kq, masked ? mask_quad<T>(g.q[i], (g.ok >> i) & 1) : g.q[i]);
      return;
    }
    float gm[4];
    quad_to_f32<T>(masked ? mask_quad<T>(g.g, (g.ok >> kQuads) & 1) : g.g, gm);
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      float v[4];
      quad_to_f32<T>(masked ? mask_quad<T>(g.q[i], (g.ok >> i) & 1) : g.q[i], v);
      Pack<T, 4> pk;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ss[i] += v[j] * v[j];
        pk.v[j] = from_f32<T>(v[j] * gm[j]);
      }
      commit_quad<T>(lds, tile_row(i), kq, __builtin_bit_cast(quad_t<T>, pk));
    }
  }
  __device__ __forceinline__ void commit_edge(const Regs& g, T* lds) const { commit_impl(g, lds, true); }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const { commit_impl(g, lds, !V4); }
};

template <typename T, int TO, bool WRITE_NORMED, bool NORM, int ACT, bool V4>
__global__ __launch_bounds__(kGemmThreads) void bs_fwd_kernel(const T* __restrict__ x, const T* __restrict__ gamma,
                                                              const T* __restrict__ weight,
                                                              const T* __restrict__ bias, T* __restrict__ out,
                                                              T* __restrict__ normed, float* __restrict__ inv_norm,
                                                              BandArgs a) {
  constexpr int OT = 64 * TO;
  __shared__ T lds[gemm_lds_elems<T, OT, kBM>()];
  __shared__ float sscale[kBM];
  using S = TileShape<OT, kBM, 4, 1>;  // TR = TO, TC = 4

  const int O = a.O;
  // widest bands (highest index in the usual layouts) first: their long K loops start at once
  // instead of forming the tail
  const int band = a.NB - 1 - static_cast<int>(blockIdx.y);
  const int oc = blockIdx.z * OT;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const T* xb = x + m0 * a.x_stride + off;

  KRowLoader<T, OT, V4> la{weight + static_cast<int64_t>(O) * off + static_cast<int64_t>(oc) * I, I, O - oc, I};
  XGammaLoader<T, NORM, V4> lb{xb, a.x_stride, gamma + off, rows_valid, I};
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int i = 0; i < S::kTR; ++i)
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, OT, kBM, 4, 1, PMSST_BS_FWD_DEPTH>(la, lb, I, lds, acc);

  const float root = sqrtf(static_cast<float>(I));
  const float ss0 = group_sum(lb.ss[0], 8);
  const float ss1 = group_sum(lb.ss[1], 8);
  if ((tid & 7) == 0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = (tid >> 3) + 32 * p;
      const float inv = 1.0f / fmaxf(sqrtf(p == 0 ? ss0 : ss1), 1.0e-12f);
      sscale[r] = NORM ? inv * root : 1.0f;
      if (NORM && blockIdx.z == 0 && r < rows_valid) inv_norm[(m0 + r) * a.NB + band] = inv;
    }
  }
  __syncthreads();

  if (a.ovec8) {
    // epilogue through LDS: lane holds 4 consecutive outputs of one row (8-byte runs of 16 rows
    // per instruction); the tile is staged as [64 m][OT o] (row pitch OT + 8 elements) and
    // written back as 16-byte pieces, 2 OT contiguous bytes per row, so HBM sees whole lines
    constexpr int kOP = OT + 8;
    T* ot = lds;  // the main loop's buffers are free after its last barrier
#pragma unroll
    for (int t = 0; t < S::kTR; ++t) {
      const int ol = wave * 16 * TO + t * 16 + 4 * (lane >> 4);
      const int o = oc + ol;
      if (o >= O) continue;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias != nullptr) load_pack<T, 4>(bias + static_cast<int64_t>(band) * O + o, bv);
#pragma unroll
      for (int j = 0; j < S::kTC; ++j) {
        const int m = j * 16 + (lane & 15);
        const float s = sscale[m];
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = acc[t][j][r] * s + bv[r];
          // the reference rounds the linear output to the tensor dtype before tanh (fr.py:338-340)
          if (ACT == PMSST_ACT_TANH) v[r] = tanhf(to_f32(from_f32<T>(v[r])));
        }
        store_pack<T, 4>(ot + m * kOP + ol, v);
      }
    }
    __syncthreads();
    const int ov = O - oc < OT ? O - oc : OT;  // valid outputs of this tile (a multiple of 8)
    const int pieces = kBM * (ov / 8);
    for (int q = tid; q < pieces; q += kGemmThreads) {
      const int m = q / (ov / 8);
      const int c = (q - m * (ov / 8)) * 8;
      if (m < rows_valid)
        *reinterpret_cast<u32x4_t*>(out + ((m0 + m) * a.NB + band) * O + oc + c) =
            *reinterpret_cast<const u32x4_t*>(ot + m * kOP + c);
    }
  } else {
#pragma unroll
    for (int t = 0; t < S::kTR; ++t) {
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
      for (int j = 0; j < S::kTC; ++j) {
        const int m = j * 16 + (lane & 15);
        if (m >= rows_valid) continue;
        const float s = sscale[m];
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = acc[t][j][r] * s + bv[r];
          // the reference rounds the linear output to the tensor dtype before tanh (fr.py:338-340)
          if (ACT == PMSST_ACT_TANH) v[r] = tanhf(to_f32(from_f32<T>(v[r])));
        }
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
    const int nq = (I + 3) / 4;
    for (int q = tid; q < kBM * nq; q += kGemmThreads) {
      const int r = q / nq;
      const int k = (q - r * nq) * 4;
      if (r >= rows_valid) continue;
      const float s = sscale[r];
      T* dst = normed + (m0 + r) * a.F + off + k;
      const T* srcp = xb + r * a.x_stride + k;
      if (a.vec4) {
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

// ------------------------------------------------------------------ backward: dx + dgamma partials

// One (64-row tile, band, 64-wide input chunk) block: gs^T[i][m] = W_b^T dy^T for the chunk
// (K = O), then
//   NORM:  t = gs * gamma (fp32, [M, F]), the chunk's part of dot[m] = sum_i t n (fp32, row m
//          of a [M, pitch] array, column off_b / 64 + b + chunk) and the dgamma partials
//          sum_m gs n ([m_tiles, F]);
//          bs_dx_finish_kernel turns them into dx;
//   !NORM: dx = gs (plain grouped linear; nsrc, inv_norm, gamma and the partials unused).
// The blocks form a 1-D XCD-ordered grid: group = (band, input chunk), member = row tile,
// so the row tiles sharing a weight chunk run on one XCD and share its L2.
// Block -> (band, row tile, 64-wide input chunk) of the dx and finish grids: with a schedule
// (sc.m_tiles != 0) only the chunks that exist get a block, XCD x running a contiguous range
// (a row tile's chunks and a band's row tiles share its L2); without one (more bands than the
// schedule holds) the XcdGrid of NB * max_ichunks groups, whose blocks past a band's width exit.
__device__ __forceinline__ bool bs_dx_block(const BandSched& sc, const XcdGrid& xg, int max_ichunks, int nb,
                                            uint32_t blk, int& band, int& ichunk, uint32_t& mt) {
  if (sc.m_tiles != 0) {
    uint32_t sub, per_unit;
    if (!sched_block_at<true>(sc, blk, band, mt, sub, per_unit)) return false;
    ichunk = static_cast<int>(sub);
    return true;
  }
  uint32_t grp;
  if (!xcd_block(xg, grp, mt)) return false;
  band = nb - 1 - static_cast<int>(grp) / max_ichunks;  // widest bands first
  ichunk = static_cast<int>(grp) % max_ichunks;
  return true;
}

template <typename T, bool FROM_X, bool NORM, bool V4>
__global__ __launch_bounds__(kGemmThreads) void bs_bwd_dx_kernel(const T* __restrict__ dy,
                                                                 const T* __restrict__ nsrc,
                                                                 const float* __restrict__ inv_norm,
                                                                 const T* __restrict__ gamma,
                                                                 const T* __restrict__ weight, T* __restrict__ dx,
                                                                 float* __restrict__ tbuf,
                                                                 float* __restrict__ dg_partial,
                                                                 float* __restrict__ pdot, int pitch,
                                                                 int max_ichunks, XcdGrid xg, BandSched sc,
                                                                 BandArgs a) {
  constexpr int kBI = 64;
  __shared__ T lds[gemm_lds_elems<T, kBI, kBM>()];
  __shared__ float sinv[kBM];
  __shared__ float sdot[4][kBM];
  using S = TileShape<kBI, kBM, 4, 1>;  // TR = 1, TC = 4

  const int O = a.O;
  int band, ichunk;
  uint32_t mt;
  if (!bs_dx_block(sc, xg, max_ichunks, a.NB, blockIdx.x, band, ichunk, mt)) return;
  const int64_t mtile = mt;
  const int64_t m0 = mtile * kBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int i0 = ichunk * kBI;
  if (i0 >= I) return;  // uniform over the block
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const T* wb = weight + static_cast<int64_t>(O) * off;  // [O][I]
  const T* dyb = dy + (m0 * a.NB + band) * O;
  const float root = sqrtf(static_cast<float>(I));

  if (NORM) {
    if (tid < kBM) sinv[tid] = tid < rows_valid ? inv_norm[(m0 + tid) * a.NB + band] : 0.f;
    __syncthreads();
  }

  // A[i][o] = W_b[o][i0 + i] (MN-contiguous in i);  B[m][o] = dy[m0 + m][band][o]
  MNLoader<T, kBI, V4> la{wb + i0, I, I - i0, O};
  KRowLoader<T, kBM, V4> lb{dyb, static_cast<int64_t>(a.NB) * O, rows_valid, O};
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[0][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, kBI, kBM, 4, 1, PMSST_BS_DX_DEPTH>(la, lb, O, lds, acc);

  // lane holds gs[m = 16 j + (lane & 15)][i = i0 + 16 wave + 4 (lane >> 4) + r]
  const int il = i0 + wave * 16 + 4 * (lane >> 4);
  if (!NORM) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = j * 16 + (lane & 15);
      if (m >= rows_valid || il >= I) continue;
      float o[4] = {acc[0][j][0], acc[0][j][1], acc[0][j][2], acc[0][j][3]};
      T* dp = dx + (m0 + m) * a.F + off + il;
      if (a.vec4) {
        store_pack<T, 4>(dp, o);
      } else {
        for (int r = 0; r < 4 && il + r < I; ++r) dp[r] = from_f32<T>(o[r]);
      }
    }
    return;
  }
  float g[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) g[r] = il + r < I ? to_f32(gamma[off + il + r]) : 0.f;
  float dgp[4] = {0.f, 0.f, 0.f, 0.f};
  float dotp[4] = {0.f, 0.f, 0.f, 0.f};  // per m-tile j
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
      const float sc = sinv[m] * root;
#pragma unroll
      for (int r = 0; r < 4; ++r) n[r] *= sc;
    }
    float t[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      t[r] = acc[0][j][r] * g[r];
      dotp[j] += t[r] * n[r];
      dgp[r] += acc[0][j][r] * n[r];
    }
    float* tp = tbuf + (m0 + m) * a.F + off + il;
    if (a.vec4) {
      *reinterpret_cast<float4*>(tp) = make_float4(t[0], t[1], t[2], t[3]);
    } else {
      for (int r = 0; r < 4 && il + r < I; ++r) tp[r] = t[r];
    }
  }
  // dot partial of the chunk: the 4 lane groups of a wave, then the 4 waves (16 i each)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = dotp[j];
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    if (lane < 16) sdot[wave][j * 16 + lane] = v;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) dgp[r] = row16_sum(dgp[r]);
  if ((lane & 15) == 0) {
    float* dst = dg_partial + mtile * a.F + off;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (il + r < I) dst[il + r] = dgp[r];
  }
  __syncthreads();
  if (tid < rows_valid)
    pdot[(m0 + tid) * pitch + off / 64 + band + ichunk] = (sdot[0][tid] + sdot[1][tid]) + (sdot[2][tid] + sdot[3][tid]);
}

// dx of one (64-row tile, band, 64-wide input chunk), the blocks of the dx kernel's grid:
// dot[m] = the band's chunk partials added in a fixed order (4 threads per row, then a fixed
// butterfly), dx = inv (t sqrt(I) - n dot / sqrt(I)) with n = x inv sqrt(I) (FROM_X) or the saved
// normed.  Thread t covers the 4-element quad t % 16 of the chunk on rows t / 16 + 16 j, j < 4:
// every load of the thread is issued before the first store.
// The finish of block `blk` of the grid (256 threads; sinv and sdot are kBM floats of LDS each):
// bs_dx_finish_kernel, or tail blocks of the DMA dW kernel, which runs after the dx kernel.
template <typename T, bool FROM_X, bool V4>
__device__ __forceinline__ void bs_dx_finish_body(const float* __restrict__ tbuf, const T* __restrict__ nsrc,
                                                  const float* __restrict__ inv_norm, const float* __restrict__ pdot,
                                                  T* __restrict__ dx, int pitch, int max_ichunks, const XcdGrid& xg,
                                                  const BandSched& sc, const BandArgs& a, uint32_t blk, float* sinv,
                                                  float* sdot) {
  int band, ichunk;
  uint32_t mt;
  if (!bs_dx_block(sc, xg, max_ichunks, a.NB, blk, band, ichunk, mt)) return;
  const int i0 = ichunk * 64;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  if (i0 >= I) return;  // uniform over the block
  const int64_t m0 = static_cast<int64_t>(mt) * kBM;
  const int rows_valid = static_cast<int>(a.M - m0 < kBM ? a.M - m0 : kBM);
  const int tid = threadIdx.x;
  const float root = sqrtf(static_cast<float>(I));
  {
    const int r = tid >> 2, part = tid & 3;
    const int nch = (I + 63) / 64;
    float d = 0.f;
    if (r < rows_valid) {
      const float* pd = pdot + (m0 + r) * pitch + off / 64 + band;
      for (int c = part; c < nch; c += 4) d += pd[c];
    }
    d += __shfl_xor(d, 1, kWave);
    d += __shfl_xor(d, 2, kWave);
    if (part == 0 && r < rows_valid) {
      sinv[r] = inv_norm[(m0 + r) * a.NB + band];
      sdot[r] = d / root;
    }
  }
  __syncthreads();
  const int k = i0 + 4 * (tid & 15);
  if (k >= I) return;
  constexpr int kJ = kBM / 16;
  if (V4) {
    float4 t[kJ];
    float n[kJ][4];
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int r = (tid >> 4) + 16 * j;
      const int rc = r < rows_valid ? r : rows_valid - 1;  // clamped loads, no branch before the math
      const int64_t e = (m0 + rc) * a.F + off + k;
      t[j] = *reinterpret_cast<const float4*>(tbuf + e);
      load_pack<T, 4>(nsrc + e, n[j]);
    }
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int r = (tid >> 4) + 16 * j;
      if (r >= rows_valid) continue;
      const float inv = sinv[r], c = sdot[r] * (FROM_X ? inv * root : 1.f);
      const float o[4] = {inv * (t[j].x * root - n[j][0] * c), inv * (t[j].y * root - n[j][1] * c),
                          inv * (t[j].z * root - n[j][2] * c), inv * (t[j].w * root - n[j][3] * c)};
      store_pack<T, 4>(dx + (m0 + r) * a.F + off + k, o);
    }
  } else {
    for (int j = 0; j < kJ; ++j) {
      const int r = (tid >> 4) + 16 * j;
      if (r >= rows_valid) continue;
      const float inv = sinv[r], c = sdot[r] * (FROM_X ? inv * root : 1.f);
      const int64_t e = (m0 + r) * a.F + off + k;
      for (int q = 0; q < 4 && k + q < I; ++q)
        dx[e + q] = from_f32<T>(inv * (tbuf[e + q] * root - to_f32(nsrc[e + q]) * c));
    }
  }
}

template <typename T, bool FROM_X, bool V4>
__global__ __launch_bounds__(256) void bs_dx_finish_kernel(const float* __restrict__ tbuf, const T* __restrict__ nsrc,
                                                           const float* __restrict__ inv_norm,
                                                           const float* __restrict__ pdot, T* __restrict__ dx,
                                                           int pitch, int max_ichunks, XcdGrid xg, BandSched sc,
                                                           BandArgs a) {
  __shared__ float sinv[kBM];
  __shared__ float sdot[kBM];
  bs_dx_finish_body<T, FROM_X, V4>(tbuf, nsrc, inv_norm, pdot, dx, pitch, max_ichunks, xg, sc, a, blockIdx.x, sinv,
                                   sdot);
}

// ------------------------------------------------------------------ backward: dW

constexpr int kDwBI = 64;
constexpr int kDwBO = 64;

// NORM = false: plain grouped linear, dW_b^T = x_b^T dy_b (no gamma / inv_norm scaling).
template <typename T, bool FROM_X, bool NORM, bool V4>
__global__ __launch_bounds__(kGemmThreads) void bs_bwd_dw_kernel(const T* __restrict__ dy,
                                                                 const T* __restrict__ nsrc,
                                                                 const float* __restrict__ inv_norm,
                                                                 const T* __restrict__ gamma, T* __restrict__ dw,
                                                                 T* __restrict__ db, int max_itiles, XcdGrid xg,
                                                                 BandSched sc, BandArgs a) {
  __shared__ T lds[gemm_lds_elems<T, kDwBI, kDwBO>()];
  using S = TileShape<kDwBI, kDwBO, 2, 2>;
  const int O = a.O;
  int band, i0, o0;
  if (sc.m_tiles != 0) {
    // one block per existing (band, input tile, output tile), evenly split over the XCDs; the
    // output tiles of one input slab are neighbours
    const uint32_t otiles = (O + kDwBO - 1) / kDwBO;
    uint32_t mt, sub, per_unit;
    if (!sched_block(sc, band, mt, sub, per_unit)) return;
    i0 = static_cast<int>(sub / otiles) * kDwBI;
    o0 = static_cast<int>(sub % otiles) * kDwBO;
  } else {
    uint32_t grp, ot;  // group = (band, input tile), member = output tile: the input slab shared in L2
    if (!xcd_block(xg, grp, ot)) return;
    o0 = static_cast<int>(ot) * kDwBO;
    band = static_cast<int>(grp) / max_itiles;
    i0 = (static_cast<int>(grp) % max_itiles) * kDwBI;
  }
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  if (i0 >= I) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // A[i][m] = n[m][off + i0 + i] * gamma (MN-contiguous in i; n = x * inv * sqrt(I) when FROM_X)
  // B[o][m] = dy[m][band][o0 + o]       (MN-contiguous in o)
  MNLoader<T, kDwBI, V4> la{nsrc + off + i0, a.F, I - i0, static_cast<int>(a.M)};
  if (NORM) la.cs = gamma + off + i0;
  if (NORM && FROM_X) {
    la.rs = inv_norm + band;
    la.rs_stride = a.NB;
    la.rs_mul = sqrtf(static_cast<float>(I));
  }
  MNLoader<T, kDwBO, V4> lb{dy + static_cast<int64_t>(band) * O + o0, static_cast<int64_t>(a.NB) * O, O - o0,
                            static_cast<int>(a.M)};
  // the first input tile of each (band, output tile) also sums dy over the rows: dbias
  lb.colsum = db != nullptr && i0 == 0;
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int i = 0; i < S::kTR; ++i)
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, kDwBI, kDwBO, 2, 2, PMSST_BS_DW_DEPTH>(la, lb, static_cast<int>(a.M), lds, acc);
  if (lb.colsum) reduce_colsum<T, kDwBO, V4>(lb, lds, db + static_cast<int64_t>(band) * O + o0);

  T* dwb = dw + static_cast<int64_t>(O) * off;  // [O][I]
  const int ir = (wave >> 1) * (kDwBI / 2), oc = (wave & 1) * (kDwBO / 2);
#pragma unroll
  for (int u = 0; u < S::kTR; ++u) {
    const int i = i0 + ir + u * 16 + 4 * (lane >> 4);
    if (i >= I) continue;
#pragma unroll
    for (int v = 0; v < S::kTC; ++v) {
      const int o = o0 + oc + v * 16 + (lane & 15);
      if (o >= O) continue;
      T* dst = dwb + static_cast<int64_t>(o) * I + i;
      float e[4] = {acc[u][v][0], acc[u][v][1], acc[u][v][2], acc[u][v][3]};
      if (a.vec4) {
        store_pack<T, 4>(dst, e);
      } else {
        for (int r = 0; r < 4 && i + r < I; ++r) dst[r] = from_f32<T>(e[r]);
      }
    }
  }
}

// ------------------------------------------------------------------ backward: dW on the DMA ring
// 16-bit, 4-aligned widths, O % 8 == 0:
//   dW_b^T[i][o] = gamma_i s_b sum_m n'[m][i] dy[m][b][o],
// n' = x * inv with s_b = sqrt(I_b) from the saved input (FROM_X), n' = normed with s_b = 1.
// Block = (band, 64-wide input tile, 64-wide output tile); K = the rows, walked in steps of
// KR = 32 KS rows.  Both operands move as stored (KR rows x 64 columns each
// per step) into a ring of S LDS stages: x by 4-byte DMA (its rows are only 8-byte aligned), dy
// by 16-byte DMA; both are read as transposed fragments (ds_read_b64_tr_b16, swz_mn swizzle).
// Wave w moves rows KR/4 w .. + KR/4 - 1 of both tiles.  From the saved input each landed x tile
// is scaled by inv in LDS (KS 16-byte units per thread, of its own wave's rows; inv of the
// block's rows sits in LDS in windows of kBdWinRows rows).  Columns past the band or past O are
// clamped reads whose products land in discarded outputs; step 0's rows before the range start
// are read from its first row and zeroed.  dbias: the two top waves of input tile 0 also
// multiply their dy fragments by an all-ones A fragment (every row of that product is the
// column sum).  The tile leaves through LDS as rows o of dW_b.
constexpr int kBdT = 64;
// 1024 rows (4 KB) keep the kernel at 52 KB of LDS, three blocks per CU, so the dx finish and
// dgamma tail blocks run beside the dW blocks' row loops (2048 rows: 56 KB, two per CU)
constexpr int kBdWinRows = 1024;
#ifndef PMSST_BS_DW_DMA
#define PMSST_BS_DW_DMA 1
#endif
#ifndef PMSST_BS_DWD_STAGES
#define PMSST_BS_DWD_STAGES 3
#endif
#ifndef PMSST_BS_DWD_KS
#define PMSST_BS_DWD_KS 2
#endif

template <typename T>
__device__ __forceinline__ u32x4_t scale8(const u32x4_t& v, float sc) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  const v8 e = __builtin_bit_cast(v8, v);
  v8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = static_cast<T>(static_cast<float>(e[j]) * sc);
  return __builtin_bit_cast(u32x4_t, r);
}

template <int N>
__device__ __forceinline__ void vm_wait_steps(int nd) {  // at most N nd DMAs outstanding, nd <= 6
  switch (nd) {
    case 0: vm_wait<0>(); break;
    case 1: vm_wait<N>(); break;
    case 2: vm_wait<2 * N>(); break;
    case 3: vm_wait<3 * N>(); break;
    case 4: vm_wait<4 * N>(); break;
    case 5: vm_wait<5 * N>(); break;
    default: vm_wait<6 * N>(); break;
  }
}

template <typename T, bool FROM_X>
__global__ __launch_bounds__(kGemmThreads) void bs_bwd_dw_dma_kernel(
    const T* __restrict__ dy, const T* __restrict__ nsrc, const float* __restrict__ inv_norm,
    const T* __restrict__ gamma, T* __restrict__ dw, T* __restrict__ db, BandSched sc, BandArgs a, int otiles,
    const float* __restrict__ dg_partial, int dg_parts, T* __restrict__ dgamma, uint32_t main_blocks,
    const float* __restrict__ tbuf, const float* __restrict__ pdot, T* __restrict__ dx, int pitch, BandSched fsc,
    uint32_t fin_blocks) {
  constexpr int S = PMSST_BS_DWD_STAGES;
  constexpr int KS = PMSST_BS_DWD_KS;
  constexpr int KR = KS * kChunkK;             // rows per step
  constexpr int kTile = KR * 2 * kBdT;          // bytes of one operand tile
  constexpr int kStage = 2 * kTile;
  constexpr int kWR = KR / 4;                   // rows per wave
  constexpr int kXI = kWR / 2;                  // 4-byte x DMAs per wave and step
  constexpr int kDI = kWR / 8;                  // 16-byte dy DMAs per wave and step
  constexpr int kWinSteps = kBdWinRows / KR;
  static_assert(KS == 1 || KS == 2 || KS == 4, "rows per step");
  static_assert(S >= 3 && (S - 2) <= 6 && (S - 2) * (kXI + kDI) <= 63, "stages (wait table)");
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];
  __shared__ float sinv[FROM_X ? kBdWinRows : 1];
  static_assert(S * kStage >= kColSumLds, "column-sum tile LDS");
  // Tail blocks, after the scheduled ones, for work that needs only the dx kernel's results: first
  // fin_blocks blocks of the dx finish (on the dx kernel's schedule fsc; main_blocks is a multiple
  // of kXcds, so each keeps its XCD), then dgamma = the column sums of the dx kernel's partials in
  // col_sum_kernel's order.  Neither gets a launch of its own.
  if (blockIdx.x >= main_blocks + fin_blocks) {
    col_sum_tile<T, kGemmThreads>(dg_partial, dg_parts, a.F, dgamma,
                                  static_cast<int>(blockIdx.x - main_blocks - fin_blocks),
                                  reinterpret_cast<float*>(lds));
    return;
  }
  if (blockIdx.x >= main_blocks) {
    const XcdGrid nogrid{0, 1};  // unused: fsc is a schedule
    float* fl = reinterpret_cast<float*>(lds);
    bs_dx_finish_body<T, FROM_X, true>(tbuf, nsrc, inv_norm, pdot, dx, pitch, 1, nogrid, fsc, a,
                                       blockIdx.x - main_blocks, fl, fl + kBM);
    return;
  }
  int band;
  uint32_t mt, sub, per_unit;
  if (!sched_block(sc, band, mt, sub, per_unit)) return;
  const int i0 = static_cast<int>(sub) / otiles * kBdT;
  const int o0 = static_cast<int>(sub) % otiles * kBdT;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int O = a.O;
  const int NB = a.NB;
  const int K = static_cast<int>(a.M);
  const int nk = (K + KR - 1) / KR;
  const int kbeg = K - nk * KR;  // step c covers rows kbeg + KR c .. + KR - 1
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t dstride = static_cast<int64_t>(NB) * O;  // elements between rows of dy
  const int64_t xstride = a.F;

  // DMA pieces.  dy instruction t: row kWR wave + 8 t + lane / 8, LDS unit lane % 8 <- unit
  // (lane % 8) ^ swz_mn(row).  x instruction t: row kWR wave + 2 t + lane / 32, 4-byte word
  // lane % 32 of the row: LDS unit (lane % 32) / 4 <- unit ((lane % 32) / 4) ^ swz_mn(row).
  uint32_t doff[kDI], doff0[kDI], xoff[kXI], xoff0[kXI];
#pragma unroll
  for (int t = 0; t < kDI; ++t) {
    const int r = kWR * wave + 8 * t + (lane >> 3);
    int col = o0 + 8 * ((lane & 7) ^ swz_mn(r));
    col = col <= O - 8 ? col : O - 8;
    doff[t] = static_cast<uint32_t>((r * dstride + col) * 2);
    doff0[t] = kbeg + r >= 0 ? doff[t] : static_cast<uint32_t>((-kbeg * dstride + col) * 2);
  }
#pragma unroll
  for (int t = 0; t < kXI; ++t) {
    const int r = kWR * wave + 2 * t + (lane >> 5);
    int i = i0 + 8 * (((lane & 31) >> 2) ^ swz_mn(r)) + 2 * (lane & 3);
    i = i <= I - 2 ? i : I - 2;
    xoff[t] = static_cast<uint32_t>((r * xstride + i) * 2);
    xoff0[t] = kbeg + r >= 0 ? xoff[t] : static_cast<uint32_t>((-kbeg * xstride + i) * 2);
  }
  const char* xsrc0 = reinterpret_cast<const char*>(nsrc + static_cast<int64_t>(kbeg) * xstride + off);
  const char* dsrc0 = reinterpret_cast<const char*>(dy + (static_cast<int64_t>(kbeg) * NB + band) * O);
  const uint32_t lds0 = lds_addr(lds);

  auto dma = [&](int c, int stage) {  // step c into `stage`
    const char* xs = xsrc0 + static_cast<int64_t>(c) * KR * xstride * 2;
    const char* ds = dsrc0 + static_cast<int64_t>(c) * KR * dstride * 2;
    char* st = lds + stage * kStage;
#pragma unroll
    for (int t = 0; t < kXI; ++t)
      __builtin_amdgcn_global_load_lds(xs + (c == 0 ? xoff0[t] : xoff[t]), st + 128 * (kWR * wave + 2 * t), 4, 0,
                                       0);
#pragma unroll
    for (int t = 0; t < kDI; ++t)
      __builtin_amdgcn_global_load_lds(ds + (c == 0 ? doff0[t] : doff[t]), st + kTile + 128 * (kWR * wave + 8 * t),
                                       16, 0, 0);
  };
  // inv of the rows of steps c0 .. c0 + kWinSteps - 1 (0 before row 0)
  auto load_inv = [&](int c0) {
    const int64_t r0 = kbeg + static_cast<int64_t>(c0) * KR;
    const int64_t rows = static_cast<int64_t>(nk - c0) * KR;
    const int n = static_cast<int>(rows < kBdWinRows ? rows : kBdWinRows);
    for (int j = threadIdx.x; j < n; j += kGemmThreads) {
      const int64_t rr = r0 + j;
      sinv[j] = rr >= 0 ? inv_norm[rr * NB + band] : 0.f;
    }
  };
  if constexpr (FROM_X) {
    load_inv(0);
    __syncthreads();
  }
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) dma(s, s);

  uint32_t fa[2], fb[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    fa[f] = frag_mn_addr(0, 32 * wr + 16 * f, 2 * kBdT, lane);
    fb[f] = frag_mn_addr(kTile, 32 * wc + 16 * f, 2 * kBdT, lane);
  }
  f32x4_t acc[2][2], accb[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    accb[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 2; ++g) acc[f][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const bool do_bias = db != nullptr && i0 == 0 && wr == 0;
  const uint32_t one2 = std::is_same<T, bf16>::value ? 0x3F803F80u : 0x3C003C00u;
  const u32x4_t ones{one2, one2, one2, one2};
  // this thread's units of a tile (rows of its own wave): row kWR wave + 8 j + lane / 8, unit lane % 8
  const int urow = kWR * wave + (lane >> 3);
  const uint32_t uoff = static_cast<uint32_t>(urow * 2 * kBdT + 16 * (lane & 7));
  const uint32_t sinv0 = lds_addr(sinv);

  for (int s = 0; s < nk; ++s) {
    // step s landed once at most (kXI + kDI) nd DMAs of this wave are outstanding
    const int nd = nk - 1 - s < S - 2 ? nk - 1 - s : S - 2;
    vm_wait_steps<kXI + kDI>(nd);
    if (s == 0 && kbeg < 0) {
      const u32x4_t z{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < KS; ++j)
        if (kbeg + urow + 8 * j < 0) {
          lds_write_b128(lds0 + uoff + 8 * j * 128, z);
          lds_write_b128(lds0 + kTile + uoff + 8 * j * 128, z);
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (FROM_X) {
      if (s > 0 && s % kWinSteps == 0) {  // next window of inv (every DMA in flight drains)
        vm_wait<0>();
        load_inv(s);
        __syncthreads();
      }
    }
    if (s + S - 1 < nk) dma(s + S - 1, (s + S - 1) % S);  // into the stage step s - 1 used
    const uint32_t so = lds0 + static_cast<uint32_t>((s % S) * kStage);
    if constexpr (FROM_X) {
      u32x4_t v[KS];
      float scl[KS];
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        v[j] = lds_read_b128(so + uoff + 8 * j * 128);
        scl[j] = lds_read_f32(sinv0 + 4u * static_cast<uint32_t>((s % kWinSteps) * KR + urow + 8 * j));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        asm volatile("" : "+v"(v[j]), "+v"(scl[j]));
        lds_write_b128(so + uoff + 8 * j * 128, scale8<T>(v[j], scl[j]));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      u32x4_t af[2], bfr[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        af[f] = lds_read_tr_pair(so + fa[f] + kk * 32 * 128, 4 * 2 * kBdT);
        bfr[f] = lds_read_tr_pair(so + fb[f] + kk * 32 * 128, 4 * 2 * kBdT);
      }
      lds_wait(af, bfr);
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int g = 0; g < 2; ++g) acc[f][g] = mfma_raw<T>(af[f], bfr[g], acc[f][g]);
      if (do_bias) {
#pragma unroll
        for (int g = 0; g < 2; ++g) accb[g] = mfma_raw<T>(ones, bfr[g], accb[g]);
      }
    }
  }

  // lane holds i = 32 wr + 16 f + 4 (lane / 16) + r, o = 32 wc + 16 g + lane % 16 of the tile
  const float sb = FROM_X ? sqrtf(static_cast<float>(I)) : 1.f;
  float gsc[2][4];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int i = i0 + 32 * wr + 16 * f + 4 * (lane >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // clamped loads outside any branch: issued together
      const float gv = to_f32(gamma[off + (i + r < I ? i + r : I - 1)]);
      gsc[f][r] = i + r < I ? gv * sb : 0.f;
    }
  }
  if (do_bias && lane < 16) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int o = o0 + 32 * wc + 16 * g + lane;
      if (o < O) db[static_cast<int64_t>(band) * O + o] = from_f32<T>(accb[g][0]);
    }
  }
  const int64_t wbase = static_cast<int64_t>(O) * off;  // dW_b is [O][I]
  // staged as [64 o][64 i] (row pitch 144 bytes), then rows o of dW_b, 8 bytes per lane
  __syncthreads();  // every wave is done with the ring (its last wait was vmcnt(0))
  constexpr int kOP = kBdT + 8;
  static_assert(kBdT * kOP * 2 <= S * kStage, "staging tile");
  T* ot = reinterpret_cast<T*>(lds);
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[f][g][r] * gsc[f][r];
      store_pack<T, 4>(ot + (32 * wc + 16 * g + (lane & 15)) * kOP + 32 * wr + 16 * f + 4 * (lane >> 4), v);
    }
  __syncthreads();
  const int iv = I - i0 < kBdT ? I - i0 : kBdT;
  const int q = static_cast<int>(threadIdx.x & 15);
#pragma unroll
  for (int p = 0; p < kBdT / 16; ++p) {
    const int ol = static_cast<int>(threadIdx.x >> 4) + 16 * p;
    if (o0 + ol < O && 4 * q < iv)
      *reinterpret_cast<u32x2_t*>(dw + wbase + static_cast<int64_t>(o0 + ol) * I + i0 + 4 * q) =
          *reinterpret_cast<const u32x2_t*>(ot + ol * kOP + 4 * q);
  }
}

// ------------------------------------------------------------------ fp32 input, 16-bit projection
// The band split under autocast: the input is the fp32 STFT, the norm runs in fp32 and only the
// projection's operands are 16-bit, at the point where the stock module rounds them (its RMSNorm
// in fp32, then nn.Linear casts its input and weight to the autocast dtype):
//   forward:  inv = 1 / max(|x_b|, 1e-12) (fp32), u = T(x inv sqrt(I_b) gamma), out = T(u W_b^T + bias)
//   backward: g = T(dy W_b) (the Linear's input gradient in the autocast dtype), then the fp32
//             RMSNorm backward dx = inv (sqrt(I) g gamma - n inv sum_i(g gamma x)), n = x inv sqrt(I),
//             dgamma = sum_m g n (fp32); dW = T(dy^T u), dbias = T(sum_m dy).
// The GEMMs are the norm-free band kernels above; the two kernels below are the fp32 row
// reductions and the column-wise elementwise passes around them.

// One wave per (64-row tile, band), one lane per row: lane m sums over its row's band
//   MODE 0: x^2                     -> out[m, b] = inv = 1 / max(sqrt(sum), 1e-12)
//   MODE 1: g * gamma * x (g in T)  -> out[m, b] = sum
// The waves of a block are four row tiles of one band (equal trip counts); the widest bands come
// first.  Rows past M are clamped to the last row and not stored.
template <int MODE, typename T, bool V4>
__global__ __launch_bounds__(256) void band_rowsum_kernel(const float* __restrict__ x, int64_t x_stride,
                                                          const T* __restrict__ g, const float* __restrict__ gamma,
                                                          const int64_t* __restrict__ offsets, int NB, int F,
                                                          int64_t M, int m_tiles, float* __restrict__ out) {
  const int wave = static_cast<int>(threadIdx.x >> 6), lane = static_cast<int>(threadIdx.x & 63);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const int band = NB - 1 - static_cast<int>(w / m_tiles);
  if (band < 0) return;
  const int64_t m = (w % m_tiles) * kWave + lane;
  const int64_t mr = m < M ? m : M - 1;
  const int off = static_cast<int>(offsets[band]);
  const int I = static_cast<int>(offsets[band + 1]) - off;
  const float* xr = x + mr * x_stride + off;
  const T* gr = MODE == 1 ? g + mr * F + off : nullptr;
  const float* gm = gamma + off;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (V4) {
    for (int i = 0; i < I; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(xr + i);
      if constexpr (MODE == 0) {
        acc[0] += v.x * v.x;
        acc[1] += v.y * v.y;
        acc[2] += v.z * v.z;
        acc[3] += v.w * v.w;
      } else {
        float gv[4];
        load_pack<T, 4>(gr + i, gv);
        const float4 c = *reinterpret_cast<const float4*>(gm + i);
        acc[0] += gv[0] * c.x * v.x;
        acc[1] += gv[1] * c.y * v.y;
        acc[2] += gv[2] * c.z * v.z;
        acc[3] += gv[3] * c.w * v.w;
      }
    }
  } else {
    for (int i = 0; i < I; ++i) {
      const float v = xr[i];
      acc[i & 3] += MODE == 0 ? v * v : to_f32(gr[i]) * gm[i] * v;
    }
  }
  const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  if (m < M) out[m * NB + band] = MODE == 0 ? 1.0f / fmaxf(sqrtf(sum), 1.0e-12f) : sum;
}

// The same row sums with coalesced loads, one block per row (4-aligned widths, F <= kRowSumMaxF):
// thread t forms the sums of the row's 4-column quads t, t + 256, ... into LDS; thread p then adds
// the (at most 16) quads of piece p, the c-th 64-column stretch of band b at p = off_b / 64 + b + c
// (injective over (b, c < ceil(I_b / 64))), and thread b adds its band's pieces in order.  Every
// sum runs in a fixed order.
constexpr int kRowSumMaxF = 16384;

template <int MODE, typename T>
__global__ __launch_bounds__(256) void band_rowsum_row_kernel(const float* __restrict__ x, int64_t x_stride,
                                                              const T* __restrict__ g, const float* __restrict__ gamma,
                                                              const int64_t* __restrict__ offsets, int NB, int F,
                                                              float* __restrict__ out) {
  __shared__ float qsum[kRowSumMaxF / 4];
  __shared__ float psum[kRowSumMaxF / 64 + kSchedMaxBands + 1];
  __shared__ int soff[kSchedMaxBands + 1];
  const int64_t m = blockIdx.x;
  for (int b = threadIdx.x; b <= NB; b += 256) soff[b] = static_cast<int>(offsets[b]);
  const float* xr = x + m * x_stride;
  const int nq = F >> 2;
  for (int q = threadIdx.x; q < nq; q += 256) {
    const float4 v = *reinterpret_cast<const float4*>(xr + 4 * q);
    if constexpr (MODE == 0) {
      qsum[q] = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    } else {
      float gv[4];
      load_pack<T, 4>(g + m * F + 4 * q, gv);
      const float4 c = *reinterpret_cast<const float4*>(gamma + 4 * q);
      qsum[q] = (gv[0] * c.x * v.x + gv[1] * c.y * v.y) + (gv[2] * c.z * v.z + gv[3] * c.w * v.w);
    }
  }
  __syncthreads();
  const int npieces = F / 64 + NB + 1;
  for (int p = threadIdx.x; p < npieces; p += 256) {
    int lo = 0, hi = NB - 1;  // the largest b with off_b / 64 + b <= p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (soff[mid] / 64 + mid <= p) lo = mid; else hi = mid - 1;
    }
    const int q0 = soff[lo] / 4 + 16 * (p - soff[lo] / 64 - lo);
    const int q1 = q0 + 16 < soff[lo + 1] / 4 ? q0 + 16 : soff[lo + 1] / 4;  // none past the band's end
    float s = 0.f;
    for (int q = q0; q < q1; ++q) s += qsum[q];
    psum[p] = s;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < NB; b += 256) {
    const int p0 = soff[b] / 64 + b;
    const int pieces = (soff[b + 1] - soff[b] + 63) / 64;
    float s = 0.f;
    for (int c = 0; c < pieces; ++c) s += psum[p0 + c];
    out[m * NB + b] = MODE == 0 ? 1.0f / fmaxf(sqrtf(s), 1.0e-12f) : s;
  }
}

// Band of column i: the largest b with offsets[b] <= i (binary search over the device offsets).
__device__ __forceinline__ int band_of_column(const int64_t* __restrict__ offsets, int NB, int i) {
  int lo = 0, hi = NB - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return lo;
}

constexpr int kColRows = 16;  // rows per block of the column passes

// Column-wise pass over a (kColRows-row, 1024-column) tile, 4 consecutive columns per thread (one
// band: with V4 every band offset is a multiple of 4; else one column per thread):
//   MODE 0: u[m, i] = T(x inv[m, b] sqrt(I_b) gamma_i)
//   MODE 1: dx[m, i] = inv (sqrt(I) g gamma_i - n inv dot[m, b]), n = x inv sqrt(I) (fp32), and the
//           dgamma partial sum_{rows of the tile} g n to partial[row tile, i]
template <int MODE, typename T, bool V4>
__global__ __launch_bounds__(256) void band_colpass_kernel(const float* __restrict__ x, int64_t x_stride,
                                                           const T* __restrict__ g, const float* __restrict__ gamma,
                                                           const float* __restrict__ inv, const float* __restrict__ dot,
                                                           const int64_t* __restrict__ offsets, int NB, int F,
                                                           int64_t M, T* __restrict__ u, float* __restrict__ dx,
                                                           float* __restrict__ partial) {
  constexpr int C = V4 ? 4 : 1;
  const int i = (static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x)) * C;
  if (i >= F) return;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kColRows;
  const int band = band_of_column(offsets, NB, i);
  const int I = static_cast<int>(offsets[band + 1] - offsets[band]);
  const float root = sqrtf(static_cast<float>(I));
  float gm[C];
#pragma unroll
  for (int c = 0; c < C; ++c) gm[c] = gamma[i + c];
  float dg[C];
#pragma unroll
  for (int c = 0; c < C; ++c) dg[c] = 0.f;
  const int rows = static_cast<int>(M - m0 < kColRows ? M - m0 : kColRows);
  for (int r = 0; r < rows; ++r) {
    const int64_t m = m0 + r;
    float xv[C];
    if constexpr (V4) {
      const float4 v = *reinterpret_cast<const float4*>(x + m * x_stride + i);
      xv[0] = v.x; xv[1] = v.y; xv[2] = v.z; xv[3] = v.w;
    } else {
      xv[0] = x[m * x_stride + i];
    }
    const float iv = inv[m * NB + band];
    if constexpr (MODE == 0) {
      float o[C];
#pragma unroll
      for (int c = 0; c < C; ++c) o[c] = xv[c] * iv * root * gm[c];
      if constexpr (V4) {
        store_pack<T, 4>(u + m * F + i, o);
      } else {
        u[m * F + i] = from_f32<T>(o[0]);
      }
    } else {
      float gv[C];
      if constexpr (V4) {
        load_pack<T, 4>(g + m * F + i, gv);
      } else {
        gv[0] = to_f32(g[m * F + i]);
      }
      const float c1 = iv * dot[m * NB + band];
      float o[C];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const float n = xv[c] * iv * root;
        o[c] = iv * (root * gv[c] * gm[c] - n * c1);
        dg[c] += gv[c] * n;
      }
      if constexpr (V4) {
        *reinterpret_cast<float4*>(dx + m * F + i) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
        dx[m * F + i] = o[0];
      }
    }
  }
  if constexpr (MODE == 1) {
    float* pp = partial + static_cast<int64_t>(blockIdx.y) * F + i;
    if constexpr (V4) {
      *reinterpret_cast<float4*>(pp) = make_float4(dg[0], dg[1], dg[2], dg[3]);
    } else {
      pp[0] = dg[0];
    }
  }
}

// ------------------------------------------------------------------ host side

struct HostBands {
  int NB;
  int F;
  int max_width;
  bool vec4;
  const int64_t* widths;  // host [NB], the caller's array (valid for the call)
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
  hb->widths = dim_inputs;
  return PMSST_OK;
}

// Grid of bs_bwd_dw_kernel: one block per existing (band, 64-wide input tile, 64-wide output tile)
// on an even XCD schedule; past the schedule's band count sc->m_tiles = 0 and the XcdGrid.
uint32_t dw_grid(const HostBands& hb, int64_t O, const XcdGrid& xg, BandSched* sc) {
  const int64_t otiles = (O + kDwBO - 1) / kDwBO;
  uint32_t per_xcd = 0;
  if (build_even_sched(hb.NB, 1, [&](int b) { return (hb.widths[b] + kDwBI - 1) / kDwBI * otiles; }, sc, &per_xcd))
    return per_xcd * kXcds;
  return xg.blocks();
}

// 64-wide output tiles per forward block (capacity 64 * TO >= min(O, 256)).
int tile_capacity(int64_t O) {
  const int64_t t = (O + 63) / 64;
  return t <= 4 ? static_cast<int>(t) : 4;
}

bool aligned_to(const void* p, size_t bytes) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % bytes == 0; }

// norm = false runs the same kernel as a plain grouped linear (gamma, normed and inv_norm unused).
template <typename T>
int launch_fwd(const void* x, int64_t x_stride, const void* gamma, const void* weight, const void* bias,
               const int64_t* offsets, const HostBands& hb, int64_t M, int64_t O, void* out, void* normed,
               float* inv_norm, bool norm, int act, hipStream_t stream) {
  const char* op = norm ? "band_split_ragged_forward" : "grouped_linear_forward";
  PMSST_REQUIRE(act == PMSST_ACT_NONE || (act == PMSST_ACT_TANH && !norm), "%s: bad activation %d", op, act);
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && (O <= 512 || !norm) && O < (1 << 20), "%s: bad out_features %lld", op, (long long)O);
  if (M == 0) return PMSST_OK;
  PMSST_REQUIRE(x && weight && offsets && out && (!norm || (gamma && inv_norm)), "%s: null pointer", op);
  PMSST_REQUIRE(x_stride >= hb.F, "%s: x row stride %lld < total features %d", op, (long long)x_stride, hb.F);
  PMSST_REQUIRE(gemm_stride_ok(x_stride, sizeof(T)) && gemm_stride_ok(int64_t{hb.NB} * O, sizeof(T)),
                "%s: rows too long for 32-bit tile offsets", op);
  BandArgs a{offsets, M, hb.NB, hb.F, x_stride, static_cast<int>(O), false, false, false};
  a.vec4 = hb.vec4 && x_stride % 4 == 0 && aligned_to(x, 4 * sizeof(T)) && aligned_to(normed, 4 * sizeof(T)) &&
           aligned_to(weight, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(out, 4 * sizeof(T)) && aligned_to(bias, 4 * sizeof(T));
  a.ovec8 = sizeof(T) == 2 && a.ovec4 && O % 8 == 0 && aligned_to(out, 16);
  const int cap = 64 * tile_capacity(O);
  const dim3 grid(static_cast<unsigned>((M + kBM - 1) / kBM), static_cast<unsigned>(hb.NB),
                  static_cast<unsigned>((O + cap - 1) / cap));
  const T* px = static_cast<const T*>(x);
  const T* pg = static_cast<const T*>(gamma);
  const T* pw = static_cast<const T*>(weight);
  const T* pb = static_cast<const T*>(bias);
  T* po = static_cast<T*>(out);
  T* pn = static_cast<T*>(normed);
#define PMSST_BSF(TO, V4)                                                                                           \
  do {                                                                                                              \
    if (!norm && act == PMSST_ACT_TANH)                                                                             \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, false, false, PMSST_ACT_TANH, V4>), grid, dim3(kGemmThreads), 0,      \
                         stream, px, pg, pw, pb, po, pn, inv_norm, a);                                              \
    else if (!norm)                                                                                                 \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, false, false, PMSST_ACT_NONE, V4>), grid, dim3(kGemmThreads), 0,      \
                         stream, px, pg, pw, pb, po, pn, inv_norm, a);                                              \
    else if (pn != nullptr)                                                                                         \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, true, true, PMSST_ACT_NONE, V4>), grid, dim3(kGemmThreads), 0, stream, \
                         px, pg, pw, pb, po, pn, inv_norm, a);                                                      \
    else                                                                                                            \
      hipLaunchKernelGGL((bs_fwd_kernel<T, TO, false, true, PMSST_ACT_NONE, V4>), grid, dim3(kGemmThreads), 0,       \
                         stream, px, pg, pw, pb, po, pn, inv_norm, a);                                              \
  } while (0)
  // Unaligned shapes (odd band widths) take one scalar-load variant with the widest tile.
  if (!a.vec4) {
    PMSST_BSF(4, false);
  } else {
    switch (tile_capacity(O)) {
      case 1: PMSST_BSF(1, true); break;
      case 2: PMSST_BSF(2, true); break;
      case 3: PMSST_BSF(3, true); break;
      default: PMSST_BSF(4, true); break;
    }
  }
#undef PMSST_BSF
  return check_launch("bs_fwd_kernel");
}

size_t dg_partial_bytes(int64_t M, int F) {
  return align_up(static_cast<size_t>((M + kBM - 1) / kBM) * static_cast<size_t>(F) * sizeof(float), 256);
}

// Row pitch of the dot partials: chunk c of band b sits at column off_b / 64 + b + c, which is
// injective over (b, c < ceil(I_b / 64)) and below F / 64 + NB + 1.
int pdot_pitch(int F, int NB) { return F / 64 + NB + 1; }

size_t pdot_bytes(int64_t M, int F, int NB) {
  return align_up(static_cast<size_t>(M) * static_cast<size_t>(pdot_pitch(F, NB)) * sizeof(float), 256);
}

size_t tbuf_bytes(int64_t M, int F) { return align_up(static_cast<size_t>(M) * F * sizeof(float), 256); }

// [dgamma partials | dot partials | t = gs * gamma (fp32)]
size_t bwd_workspace(int64_t M, int F, int NB) {
  return M == 0 ? 0 : dg_partial_bytes(M, F) + pdot_bytes(M, F, NB) + tbuf_bytes(M, F);
}

template <typename T>
int launch_bwd(const void* dy, const void* nsrc, bool from_x, const float* inv_norm, const void* gamma,
               const void* weight, const int64_t* offsets, const int64_t* dim_inputs, const HostBands& hb,
               int64_t M, int64_t O, void* dx, void* dgamma, void* dw, void* db, void* workspace,
               size_t workspace_bytes, hipStream_t stream) {
  const char* op = "band_split_ragged_backward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && O <= 512, "%s: out_features must be in [1, 512] (got %lld)", op, (long long)O);
  PMSST_REQUIRE(gamma && weight && offsets && dgamma && dw && (M == 0 || (dy && nsrc && inv_norm && dx)),
                "%s: null pointer", op);
  PMSST_REQUIRE(gemm_stride_ok(hb.F, sizeof(T)) && gemm_stride_ok(int64_t{hb.NB} * O, sizeof(T)),
                "%s: rows too long for 32-bit tile offsets", op);
  const size_t need = bwd_workspace(M, hb.F, hb.NB);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(PMSST_EWORKSPACE, "%s: workspace of %zu bytes needed", op, need);
  }
  BandArgs a{offsets, M, hb.NB, hb.F, hb.F, static_cast<int>(O), false, false, false};
  a.vec4 = hb.vec4 && aligned_to(nsrc, 4 * sizeof(T)) && aligned_to(dx, 4 * sizeof(T)) &&
           aligned_to(weight, 4 * sizeof(T)) && aligned_to(dw, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(dy, 4 * sizeof(T));
  const T* pdy = static_cast<const T*>(dy);
  const T* pn = static_cast<const T*>(nsrc);
  const T* pg = static_cast<const T*>(gamma);
  const T* pw = static_cast<const T*>(weight);
  char* ws = static_cast<char*>(workspace);
  float* partial = reinterpret_cast<float*>(ws);
  float* pdot = reinterpret_cast<float*>(ws + dg_partial_bytes(M, hb.F));
  float* tbuf = reinterpret_cast<float*>(ws + dg_partial_bytes(M, hb.F) + pdot_bytes(M, hb.F, hb.NB));
  const int pitch = pdot_pitch(hb.F, hb.NB);
  const int m_tiles = static_cast<int>((M + kBM - 1) / kBM);
  // DMA-ring dW: 16-bit, 4-aligned widths and pointers, O % 8 == 0 with 16-byte aligned dy rows
  constexpr int KR = PMSST_BS_DWD_KS * kChunkK;
  const int otiles = static_cast<int>((O + kBdT - 1) / kBdT);
  BandSched wsc;
  uint32_t w_per_xcd = 0;
  const bool dma_dw = sizeof(T) == 2 && PMSST_BS_DW_DMA && M >= KR && a.vec4 && O % 8 == 0 && aligned_to(dy, 16) &&
                      (static_cast<int64_t>(KR) * hb.F + hb.F) * 2 < (int64_t{1} << 31) &&
                      (static_cast<int64_t>(KR) * hb.NB * O + O) * 2 < (int64_t{1} << 31) &&
                      build_band_sched(hb.NB, 1, [&](int b) { return (dim_inputs[b] + kBdT - 1) / kBdT * otiles; },
                                       &wsc, &w_per_xcd);
  BandSched sc;  // dx and finish: one block per existing (band, row tile, chunk); sc.m_tiles = 0 without
  uint32_t per_xcd = 0;
  const bool dx_sched =
      M > 0 && build_even_sched(hb.NB, m_tiles, [&](int b) { return (dim_inputs[b] + 63) / 64; }, &sc, &per_xcd);
  // the finish runs in the DMA dW kernel's tail blocks when both have their schedules
  const bool fold_finish = dma_dw && dx_sched;
  if (M > 0) {
    const bool v4 = a.vec4 && a.ovec4;
    const int max_ichunks = (hb.max_width + 63) / 64;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_ichunks), static_cast<uint32_t>(m_tiles)};
    const dim3 grid(dx_sched ? per_xcd * kXcds : xg.blocks());
#define PMSST_BDX(FX, V4)                                                                                          \
  hipLaunchKernelGGL((bs_bwd_dx_kernel<T, FX, true, V4>), grid, dim3(kGemmThreads), 0, stream, pdy, pn, inv_norm, pg, \
                     pw, static_cast<T*>(dx), tbuf, partial, pdot, pitch, max_ichunks, xg, sc, a)
    if (from_x) {
      if (v4) PMSST_BDX(true, true); else PMSST_BDX(true, false);
    } else {
      if (v4) PMSST_BDX(false, true); else PMSST_BDX(false, false);
    }
#undef PMSST_BDX
    int rc = check_launch("bs_bwd_dx_kernel");
    if (rc != PMSST_OK) return rc;
    if (!fold_finish) {  // else the DMA dW kernel's tail blocks finish dx
      const bool fv4 = a.vec4;
#define PMSST_FIN(FX, V4)                                                                                        \
  hipLaunchKernelGGL((bs_dx_finish_kernel<T, FX, V4>), grid, dim3(256), 0, stream, tbuf, pn, inv_norm, pdot, \
                     static_cast<T*>(dx), pitch, max_ichunks, xg, sc, a)
      if (from_x) {
        if (fv4) PMSST_FIN(true, true); else PMSST_FIN(true, false);
      } else {
        if (fv4) PMSST_FIN(false, true); else PMSST_FIN(false, false);
      }
#undef PMSST_FIN
      rc = check_launch("bs_dx_finish_kernel");
      if (rc != PMSST_OK) return rc;
    }
  }
  bool dw_done = false;
  if constexpr (sizeof(T) == 2) {
    if (dma_dw) {
      // + the finish's blocks (when folded) and one block per 16 columns of dgamma
      const uint32_t main_blocks = w_per_xcd * kXcds;
      const uint32_t fin_blocks = fold_finish ? per_xcd * kXcds : 0;
      const BandSched& fsc = fold_finish ? sc : wsc;  // unused without fin_blocks
      const dim3 grid(main_blocks + fin_blocks + static_cast<uint32_t>((hb.F + kColSumCols - 1) / kColSumCols));
      T* pdg = static_cast<T*>(dgamma);
      T* pdx = static_cast<T*>(dx);
      if (from_x)
        hipLaunchKernelGGL((bs_bwd_dw_dma_kernel<T, true>), grid, dim3(kGemmThreads), 0, stream, pdy, pn, inv_norm,
                           pg, static_cast<T*>(dw), static_cast<T*>(db), wsc, a, otiles, partial, m_tiles, pdg,
                           main_blocks, tbuf, pdot, pdx, pitch, fsc, fin_blocks);
      else
        hipLaunchKernelGGL((bs_bwd_dw_dma_kernel<T, false>), grid, dim3(kGemmThreads), 0, stream, pdy, pn,
                           inv_norm, pg, static_cast<T*>(dw), static_cast<T*>(db), wsc, a, otiles, partial, m_tiles,
                           pdg, main_blocks, tbuf, pdot, pdx, pitch, fsc, fin_blocks);
      const int rc = check_launch("bs_bwd_dw_dma_kernel");
      if (rc != PMSST_OK) return rc;
      dw_done = true;
    }
  }
  if (!dw_done) {
    BandSched wsc;
    const int max_itiles = (hb.max_width + kDwBI - 1) / kDwBI;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_itiles), static_cast<uint32_t>((O + kDwBO - 1) / kDwBO)};
    const dim3 grid(dw_grid(hb, O, xg, &wsc));
    const bool v4 = a.vec4 && a.ovec4;
#define PMSST_BDW(FX, V4)                                                                                   \
  hipLaunchKernelGGL((bs_bwd_dw_kernel<T, FX, true, V4>), grid, dim3(kGemmThreads), 0, stream, pdy, pn, inv_norm, \
                     pg, static_cast<T*>(dw), static_cast<T*>(db), max_itiles, xg, wsc, a)
    if (from_x) {
      if (v4) PMSST_BDW(true, true); else PMSST_BDW(true, false);
    } else {
      if (v4) PMSST_BDW(false, true); else PMSST_BDW(false, false);
    }
#undef PMSST_BDW
    int rc = check_launch("bs_bwd_dw_kernel");
    if (rc != PMSST_OK) return rc;
  }
  // dbias was summed by the dW kernel (the fallback one also runs for M == 0 and then writes zeros);
  // the DMA dW kernel's tail blocks summed dgamma
  if (dw_done) return PMSST_OK;
  return launch_col_sum(partial, m_tiles, hb.F, dgamma, dtype_code<T>(), stream);
}

// Grouped linear backward: the norm-free dx / dW kernels plus the bias column sums.
template <typename T>
int launch_grouped_bwd(const void* dy, const void* x, const void* weight, const int64_t* offsets,
                       const HostBands& hb, int64_t M, int64_t O, void* dx, void* dw, void* db, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  const char* op = "grouped_linear_backward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && O < (1 << 20), "%s: bad out_features %lld", op, (long long)O);
  PMSST_REQUIRE(weight && offsets && dw && (M == 0 || (dy && x && dx)), "%s: null pointer", op);
  PMSST_REQUIRE(gemm_stride_ok(hb.F, sizeof(T)) && gemm_stride_ok(int64_t{hb.NB} * O, sizeof(T)),
                "%s: rows too long for 32-bit tile offsets", op);
  BandArgs a{offsets, M, hb.NB, hb.F, hb.F, static_cast<int>(O), false, false, false};
  a.vec4 = hb.vec4 && aligned_to(x, 4 * sizeof(T)) && aligned_to(dx, 4 * sizeof(T)) &&
           aligned_to(weight, 4 * sizeof(T)) && aligned_to(dw, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(dy, 4 * sizeof(T));
  const T* pdy = static_cast<const T*>(dy);
  const T* px = static_cast<const T*>(x);
  const T* pw = static_cast<const T*>(weight);
  if (M > 0 && grouped_dx_supported(hb.NB, hb.max_width, O, M, sizeof(T), dy, weight, dx)) {
    if constexpr (sizeof(T) == 2) {
      const int rc = launch_grouped_dx<T>(dy, weight, dx, hb.NB, hb.max_width, O, M, stream);
      if (rc != PMSST_OK) return rc;
    }
  } else if (M > 0) {
    const int max_ichunks = (hb.max_width + 63) / 64;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_ichunks), static_cast<uint32_t>((M + kBM - 1) / kBM)};
    const dim3 grid(xg.blocks());
    const BandSched nosc{};  // groups of one width: every XcdGrid block has a chunk
    if (a.vec4 && a.ovec4)
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, false, false, true>), grid, dim3(kGemmThreads), 0, stream, pdy, px,
                         nullptr, nullptr, pw, static_cast<T*>(dx), nullptr, nullptr, nullptr, 0, max_ichunks, xg, nosc,
                         a);
    else
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, false, false, false>), grid, dim3(kGemmThreads), 0, stream, pdy, px,
                         nullptr, nullptr, pw, static_cast<T*>(dx), nullptr, nullptr, nullptr, 0, max_ichunks, xg, nosc,
                         a);
    int rc = check_launch("bs_bwd_dx_kernel");
    if (rc != PMSST_OK) return rc;
  }
  if (uniform_dw_supported(hb.NB, hb.max_width, O, M, sizeof(T), dy, x, dw)) {
    if constexpr (sizeof(T) == 2) {
      const int rc = launch_uniform_dw<T>(dy, x, dw, db, hb.NB, hb.max_width, O, M, stream);
      if (rc != PMSST_OK) return rc;
    }
  } else {
    const int max_itiles = (hb.max_width + kDwBI - 1) / kDwBI;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_itiles), static_cast<uint32_t>((O + kDwBO - 1) / kDwBO)};
    BandSched wsc;
    const dim3 grid(dw_grid(hb, O, xg, &wsc));
    if (a.vec4 && a.ovec4)
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, false, false, true>), grid, dim3(kGemmThreads), 0, stream, pdy, px,
                         nullptr, nullptr, static_cast<T*>(dw), static_cast<T*>(db), max_itiles, xg, wsc, a);
    else
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, false, false, false>), grid, dim3(kGemmThreads), 0, stream, pdy, px,
                         nullptr, nullptr, static_cast<T*>(dw), static_cast<T*>(db), max_itiles, xg, wsc, a);
    int rc = check_launch("bs_bwd_dw_kernel");
    if (rc != PMSST_OK) return rc;
  }
  // dbias was summed by the dW kernel (which also runs for M == 0 and then writes zeros)
  (void)workspace;
  (void)workspace_bytes;
  return PMSST_OK;
}

// ------------------------------------------------------------------ fp32 input, 16-bit projection

bool mixed_vec4(const HostBands& hb, int64_t x_stride, const void* x) {
  return hb.vec4 && x_stride % 4 == 0 && aligned_to(x, 16);
}

// Row sums of band_rowsum_row_kernel<MODE> (band_rowsum_kernel<MODE> past its shapes) into out[M, NB].
template <int MODE, typename T>
int launch_rowsum(const float* x, int64_t x_stride, const T* g, const float* gamma, const int64_t* offsets,
                  const HostBands& hb, int64_t M, bool v4, float* out, hipStream_t stream) {
  if (v4 && hb.F <= kRowSumMaxF && hb.NB <= kSchedMaxBands && M < (int64_t{1} << 31)) {
    hipLaunchKernelGGL((band_rowsum_row_kernel<MODE, T>), dim3(static_cast<unsigned>(M)), dim3(256), 0, stream, x,
                       x_stride, g, gamma, offsets, hb.NB, hb.F, out);
    return check_launch("band_rowsum_row_kernel");
  }
  const int m_tiles = static_cast<int>((M + kWave - 1) / kWave);
  const int64_t waves = static_cast<int64_t>(m_tiles) * hb.NB;
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
  if (v4)
    hipLaunchKernelGGL((band_rowsum_kernel<MODE, T, true>), grid, dim3(256), 0, stream, x, x_stride, g, gamma, offsets,
                       hb.NB, hb.F, M, m_tiles, out);
  else
    hipLaunchKernelGGL((band_rowsum_kernel<MODE, T, false>), grid, dim3(256), 0, stream, x, x_stride, g, gamma,
                       offsets, hb.NB, hb.F, M, m_tiles, out);
  return check_launch("band_rowsum_kernel");
}

template <int MODE, typename T>
int launch_colpass(const float* x, int64_t x_stride, const T* g, const float* gamma, const float* inv,
                   const float* dot, const int64_t* offsets, const HostBands& hb, int64_t M, bool v4, T* u, float* dx,
                   float* partial, hipStream_t stream) {
  const int per_block = 256 * (v4 ? 4 : 1);
  const dim3 grid(static_cast<unsigned>((hb.F + per_block - 1) / per_block),
                  static_cast<unsigned>((M + kColRows - 1) / kColRows));
  if (v4)
    hipLaunchKernelGGL((band_colpass_kernel<MODE, T, true>), grid, dim3(256), 0, stream, x, x_stride, g, gamma, inv,
                       dot, offsets, hb.NB, hb.F, M, u, dx, partial);
  else
    hipLaunchKernelGGL((band_colpass_kernel<MODE, T, false>), grid, dim3(256), 0, stream, x, x_stride, g, gamma, inv,
                       dot, offsets, hb.NB, hb.F, M, u, dx, partial);
  return check_launch("band_colpass_kernel");
}

template <typename T>
int launch_mixed_fwd(const float* x, int64_t x_stride, const float* gamma, const void* weight, const void* bias,
                     const int64_t* offsets, const HostBands& hb, int64_t M, int64_t O, void* features, void* out,
                     float* inv_norm, hipStream_t stream) {
  const char* op = "band_split_mixed_forward";
  PMSST_REQUIRE(sizeof(T) == 2, "%s: the projection dtype must be float16 or bfloat16", op);
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && O <= 512, "%s: out_features must be in [1, 512] (got %lld)", op, (long long)O);
  if (M == 0) return PMSST_OK;
  PMSST_REQUIRE(x && gamma && weight && offsets && features && out && inv_norm, "%s: null pointer", op);
  PMSST_REQUIRE(x_stride >= hb.F, "%s: x row stride %lld < total features %d", op, (long long)x_stride, hb.F);
  PMSST_REQUIRE(gemm_stride_ok(x_stride, sizeof(float)), "%s: rows too long for 32-bit offsets", op);
  const bool v4 = mixed_vec4(hb, x_stride, x) && aligned_to(gamma, 16) && aligned_to(features, 8);
  int rc = launch_rowsum<0, T>(x, x_stride, nullptr, gamma, offsets, hb, M, v4, inv_norm, stream);
  if (rc != PMSST_OK) return rc;
  rc = launch_colpass<0, T>(x, x_stride, nullptr, gamma, inv_norm, nullptr, offsets, hb, M, v4,
                            static_cast<T*>(features), nullptr, nullptr, stream);
  if (rc != PMSST_OK) return rc;
  return launch_fwd<T>(features, hb.F, nullptr, weight, bias, offsets, hb, M, O, out, nullptr, nullptr, false,
                       PMSST_ACT_NONE, stream);
}

size_t mixed_g_bytes(int64_t M, int F) { return align_up(static_cast<size_t>(M) * F * 2, 256); }
size_t mixed_dot_bytes(int64_t M, int NB) { return align_up(static_cast<size_t>(M) * NB * sizeof(float), 256); }
size_t mixed_partial_bytes(int64_t M, int F) {
  return align_up(static_cast<size_t>((M + kColRows - 1) / kColRows) * F * sizeof(float), 256);
}
// [g = T(dy W) (16-bit, [M, F]) | dot [M, NB] | dgamma partials [ceil(M / 16), F]]
size_t mixed_bwd_workspace(int64_t M, int F, int NB) {
  return M == 0 ? 0 : mixed_g_bytes(M, F) + mixed_dot_bytes(M, NB) + mixed_partial_bytes(M, F);
}

template <typename T>
int launch_mixed_bwd(const void* dy, const float* x, int64_t x_stride, const void* features, const float* inv_norm,
                     const float* gamma, const void* weight, const int64_t* offsets, const HostBands& hb, int64_t M,
                     int64_t O, float* dx, float* dgamma, void* dw, void* db, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  const char* op = "band_split_mixed_backward";
  PMSST_REQUIRE(sizeof(T) == 2, "%s: the projection dtype must be float16 or bfloat16", op);
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(O >= 1 && O <= 512, "%s: out_features must be in [1, 512] (got %lld)", op, (long long)O);
  PMSST_REQUIRE(gamma && weight && offsets && dgamma && dw && (M == 0 || (dy && x && features && inv_norm && dx)),
                "%s: null pointer", op);
  PMSST_REQUIRE(M == 0 || x_stride >= hb.F, "%s: x row stride %lld < total features %d", op, (long long)x_stride, hb.F);
  PMSST_REQUIRE(gemm_stride_ok(hb.F, sizeof(float)) && gemm_stride_ok(x_stride, sizeof(float)) &&
                    gemm_stride_ok(int64_t{hb.NB} * O, sizeof(T)),
                "%s: rows too long for 32-bit tile offsets", op);
  const size_t need = mixed_bwd_workspace(M, hb.F, hb.NB);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(PMSST_EWORKSPACE, "%s: workspace of %zu bytes needed", op, need);
  BandArgs a{offsets, M, hb.NB, hb.F, hb.F, static_cast<int>(O), false, false, false};
  a.vec4 = hb.vec4 && aligned_to(features, 4 * sizeof(T)) && aligned_to(weight, 4 * sizeof(T)) &&
           aligned_to(dw, 4 * sizeof(T));
  a.ovec4 = O % 4 == 0 && aligned_to(dy, 4 * sizeof(T));
  const T* pdy = static_cast<const T*>(dy);
  const T* pu = static_cast<const T*>(features);
  const T* pw = static_cast<const T*>(weight);
  char* ws = static_cast<char*>(workspace);
  T* g = reinterpret_cast<T*>(ws);
  float* dot = reinterpret_cast<float*>(ws + mixed_g_bytes(M, hb.F));
  float* partial = reinterpret_cast<float*>(ws + mixed_g_bytes(M, hb.F) + mixed_dot_bytes(M, hb.NB));
  if (M > 0) {
    // g = T(dy W_b): the norm-free dx kernel, one block per existing (band, row tile, 64-wide chunk)
    const int m_tiles = static_cast<int>((M + kBM - 1) / kBM);
    const int max_ichunks = (hb.max_width + 63) / 64;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_ichunks), static_cast<uint32_t>(m_tiles)};
    BandSched sc;
    uint32_t per_xcd = 0;
    const bool sched =
        build_even_sched(hb.NB, m_tiles, [&](int b) { return (hb.widths[b] + 63) / 64; }, &sc, &per_xcd);
    const dim3 grid(sched ? per_xcd * kXcds : xg.blocks());
    const bool gv4 = a.vec4 && a.ovec4;
    if (gv4)
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, false, false, true>), grid, dim3(kGemmThreads), 0, stream, pdy, pu,
                         nullptr, nullptr, pw, g, nullptr, nullptr, nullptr, 0, max_ichunks, xg, sc, a);
    else
      hipLaunchKernelGGL((bs_bwd_dx_kernel<T, false, false, false>), grid, dim3(kGemmThreads), 0, stream, pdy, pu,
                         nullptr, nullptr, pw, g, nullptr, nullptr, nullptr, 0, max_ichunks, xg, sc, a);
    int rc = check_launch("bs_bwd_dx_kernel");
    if (rc != PMSST_OK) return rc;
    // fp32 RMSNorm backward: dot = sum g gamma x per (row, band), then dx and the dgamma partials
    const bool v4 = mixed_vec4(hb, x_stride, x) && aligned_to(gamma, 16) && aligned_to(dx, 16) &&
                    aligned_to(g, 8);
    rc = launch_rowsum<1, T>(x, x_stride, g, gamma, offsets, hb, M, v4, dot, stream);
    if (rc != PMSST_OK) return rc;
    rc = launch_colpass<1, T>(x, x_stride, g, gamma, inv_norm, dot, offsets, hb, M, v4, nullptr, dx, partial,
                              stream);
    if (rc != PMSST_OK) return rc;
  }
  // dW_b = T(dy_b^T u_b), dbias = T(sum_m dy_b): the norm-free register-staged dW kernel (it also
  // runs for M == 0 and then writes zeros)
  {
    const int max_itiles = (hb.max_width + kDwBI - 1) / kDwBI;
    const XcdGrid xg{static_cast<uint32_t>(hb.NB * max_itiles), static_cast<uint32_t>((O + kDwBO - 1) / kDwBO)};
    BandSched wsc;
    const dim3 grid(dw_grid(hb, O, xg, &wsc));
    if (a.vec4 && a.ovec4)
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, false, false, true>), grid, dim3(kGemmThreads), 0, stream, pdy, pu,
                         nullptr, nullptr, static_cast<T*>(dw), static_cast<T*>(db), max_itiles, xg, wsc, a);
    else
      hipLaunchKernelGGL((bs_bwd_dw_kernel<T, false, false, false>), grid, dim3(kGemmThreads), 0, stream, pdy, pu,
                         nullptr, nullptr, static_cast<T*>(dw), static_cast<T*>(db), max_itiles, xg, wsc, a);
    const int rc = check_launch("bs_bwd_dw_kernel");
    if (rc != PMSST_OK) return rc;
  }
  // dgamma = the column sums of the partials (parts == 0 writes zeros)
  const int parts = static_cast<int>((M + kColRows - 1) / kColRows);
  return launch_col_sum(partial, parts, hb.F, dgamma, PMSST_F32, stream);
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
                         inv_norm, true, PMSST_ACT_NONE, static_cast<hipStream_t>(stream));
  });
}

int pmsst_grouped_linear_forward(const void* x, int64_t x_row_stride, const void* weight, const void* bias,
                                 const int64_t* group_offsets, int64_t groups, int64_t in_features, int64_t rows,
                                 int64_t out_features, void* out, int activation, int dtype, void* stream) {
  PMSST_REQUIRE(groups > 0 && groups < (1 << 16) && in_features > 0, "grouped_linear_forward: bad shape");
  std::vector<int64_t> dims(static_cast<size_t>(groups), in_features);
  HostBands hb;
  int rc = check_bands("grouped_linear_forward", dims.data(), groups, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "grouped_linear_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_fwd<T>(x, x_row_stride, nullptr, weight, bias, group_offsets, hb, rows, out_features, out, nullptr,
                         nullptr, false, activation, static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_grouped_linear_backward_workspace_size(int64_t rows, int64_t groups, int64_t out_features) {
  (void)rows;
  (void)groups;
  (void)out_features;
  return 0;  // dbias is the column sum the dW kernel's dy loader gathers
}

int pmsst_grouped_linear_backward(const void* grad_out, const void* x, const void* weight,
                                  const int64_t* group_offsets, int64_t groups, int64_t in_features, int64_t rows,
                                  int64_t out_features, void* grad_x, void* grad_weight, void* grad_bias, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  PMSST_REQUIRE(groups > 0 && groups < (1 << 16) && in_features > 0, "grouped_linear_backward: bad shape");
  std::vector<int64_t> dims(static_cast<size_t>(groups), in_features);
  HostBands hb;
  int rc = check_bands("grouped_linear_backward", dims.data(), groups, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "grouped_linear_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_grouped_bwd<T>(grad_out, x, weight, group_offsets, hb, rows, out_features, grad_x, grad_weight,
                                 grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_band_split_ragged_backward_workspace_size(int64_t rows, int64_t total_in, int64_t band_count,
                                                       int64_t out_features) {
  if (rows < 0 || total_in <= 0 || band_count <= 0 || out_features <= 0) return 0;
  return bwd_workspace(rows, static_cast<int>(total_in), static_cast<int>(band_count));
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
    return launch_bwd<T>(grad_out, saved, saved_is_input != 0, inv_norm, gamma, weight, dim_offsets, dim_inputs, hb,
                         rows, out_features, grad_x, grad_gamma, grad_weight, grad_bias, workspace, workspace_bytes,
                         static_cast<hipStream_t>(stream));
  });
}

int pmsst_band_split_mixed_forward(const float* x, int64_t x_row_stride, const float* gamma, const void* weight,
                                   const void* bias, const int64_t* dim_offsets, const int64_t* dim_inputs,
                                   int64_t band_count, int64_t rows, int64_t out_features, void* features, void* out,
                                   float* inv_norm, int dtype, void* stream) {
  HostBands hb;
  int rc = check_bands("band_split_mixed_forward", dim_inputs, band_count, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "band_split_mixed_forward", [&](auto tag) {
    using T = decltype(tag);
    if constexpr (sizeof(T) != 2) {
      return fail(PMSST_EDTYPE, "band_split_mixed_forward: the projection dtype must be float16 or bfloat16");
    } else {
      return launch_mixed_fwd<T>(x, x_row_stride, gamma, weight, bias, dim_offsets, hb, rows, out_features, features,
                                 out, inv_norm, static_cast<hipStream_t>(stream));
    }
  });
}

size_t pmsst_band_split_mixed_backward_workspace_size(int64_t rows, int64_t total_in, int64_t band_count) {
  if (rows < 0 || total_in <= 0 || band_count <= 0) return 0;
  return mixed_bwd_workspace(rows, static_cast<int>(total_in), static_cast<int>(band_count));
}

int pmsst_band_split_mixed_backward(const void* grad_out, const float* x, int64_t x_row_stride, const void* features,
                                    const float* inv_norm, const float* gamma, const void* weight,
                                    const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                    int64_t rows, int64_t out_features, float* grad_x, float* grad_gamma,
                                    void* grad_weight, void* grad_bias, int dtype, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  HostBands hb;
  int rc = check_bands("band_split_mixed_backward", dim_inputs, band_count, &hb);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "band_split_mixed_backward", [&](auto tag) {
    using T = decltype(tag);
    if constexpr (sizeof(T) != 2) {
      return fail(PMSST_EDTYPE, "band_split_mixed_backward: the projection dtype must be float16 or bfloat16");
    } else {
      return launch_mixed_bwd<T>(grad_out, x, x_row_stride, features, inv_norm, gamma, weight, dim_offsets, hb, rows,
                                 out_features, grad_x, grad_gamma, grad_weight, grad_bias, workspace,
                                 workspace_bytes, static_cast<hipStream_t>(stream));
    }
  });
}

}  // extern "C"
