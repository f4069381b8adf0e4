// Mask-estimator final layer backward, gradient of the layer input (16-bit storage):
//   dx[m, b, h] = sum_j dpre[m, 2 off_b + j] W_b[j][h]      (K = 2 I_b, ragged per band)
// and, for the mask MLP's hidden layer (TANH), dz = round(dx) * (1 - x^2) with x the saved tanh
// output, the gradient of the hidden pre-activation.
//
// Data layout: dpre [M, 2F] (band b at columns 2 off_b .. 2 off_b + 2 I_b), W packed band-major as
// [2 I_b, H] matrices, x and dx [M, NB, H].
//
// Block = (band b, row tile, hidden tile of HT = 16 DT columns): 4 waves x 16 NT rows.  Per 32-wide K
// chunk a ring stage receives by global -> LDS DMA the weight slab W_b[32 c .. + 31][h0 .. h0 + HT)
// (read as transposed A fragments) and each wave's dpre rows [32 c .. + 31] (K-contiguous B
// fragments); K values past 2 I_b are zeroed in the B fragments (I_b is a multiple of 4, so whole
// 8-value units are in or out), the weight rows past it are clamped reads multiplied by those
// zeros.  The accumulators stay in registers over the whole K; the epilogue stages the tile in LDS
// and streams x in and dz out along whole rows.  Blocks of wide bands (long K) are dispatched first.
#include "common.h"
#include "dma_gemm.h"
#include "grouped_dx.h"
#include "ring.h"

namespace pmsst {
namespace {

constexpr int kDzStages = 4;

struct DzArgs {
  const int64_t* offsets;  // device [NB + 1] prefix sums of I_b
  int64_t M;
  int NB, H, F;
};

template <typename T, int DT, int NT, bool TANH>
__global__ __launch_bounds__(256) void me_dz_kernel(const T* __restrict__ dpre, const T* __restrict__ w,
                                                    const T* __restrict__ xin, T* __restrict__ dz, DzArgs a,
                                                    BandSched sc) {
  constexpr int S = kDzStages;
  constexpr int HT = 16 * DT;            // hidden columns of the block
  constexpr int kUnits = HT / 8;         // 16-byte units per slab row
  constexpr int kSlab = 32 * 2 * HT;
  constexpr int kInstr = kSlab / 1024;   // = DT
  constexpr int kMaxPW = (kInstr + 3) / 4;
  constexpr int kWaveRows = 16 * NT;
  constexpr int kStage = kSlab + 4 * kWaveRows * 64;
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];

  int band;
  uint32_t mt, sub, per;
  if (!sched_block<true>(sc, band, mt, sub, per)) return;
  const int H = a.H;
  const int h0 = static_cast<int>(sub) * HT;
  const int off = static_cast<int>(a.offsets[band]);
  const int K = 2 * (static_cast<int>(a.offsets[band + 1]) - off);
  const int nc = (K + 31) / 32;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  const int lane = threadIdx.x & 63, gq = lane >> 4, rr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t wrow0 = static_cast<int64_t>(mt) * (4 * kWaveRows) + wave * kWaveRows;
  const int64_t left = a.M - wrow0;
  const int nvt = left <= 0 ? 0 : (left >= kWaveRows ? NT : static_cast<int>((left + 15) / 16));

  // weight DMA: instruction t (wave t % 4) moves flattened units 64 t + lane of the slab: row
  // kr = P / kUnits (weight row 32 c + kr, clamped to the band), physical unit P % kUnits <-
  // logical unit (P % kUnits) ^ swz_mn(kr)
  const int npw = (kInstr - wave + 3) / 4;
  int wrow[kMaxPW], wcol[kMaxPW];
#pragma unroll
  for (int q = 0; q < kMaxPW; ++q) {
    const int t = wave + 4 * q;
    const int P = 64 * t + lane;
    const int kr = P / kUnits, pu = P % kUnits;
    wrow[q] = kr;
    wcol[q] = h0 + 8 * (pu ^ swz_mn(kr));
  }
  const T* wb = w + static_cast<int64_t>(2) * off * H;
  // dpre DMA: instruction n moves rows wrow0 + 16 n + lane / 4 (clamped), physical unit lane % 4 <-
  // logical unit (lane % 4) ^ swz_k(lane / 4), columns past the band clamped to its last unit
  const int du = (lane & 3) ^ swz_k(lane >> 2);
  const T* dr[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    int64_t m = wrow0 + 16 * n + (lane >> 2);
    m = m < a.M ? m : a.M - 1;
    dr[n] = dpre + m * pitch2 + 2 * off;
  }
  const uint32_t lds0 = lds_addr(lds);
  auto dma = [&](int c, int stage) {
    const uint32_t st = lds0 + static_cast<uint32_t>(stage * kStage);
#pragma unroll
    for (int q = 0; q < kMaxPW; ++q) {
      if (q < npw) {
        const int j = 32 * c + wrow[q] < K ? 32 * c + wrow[q] : K - 1;
        dma16_m0(wb + static_cast<int64_t>(j) * H + wcol[q], __builtin_amdgcn_readfirstlane(st + (wave + 4 * q) * 1024));
      }
    }
    const int col = 32 * c + 8 * du < K ? 32 * c + 8 * du : K - 8;
#pragma unroll
    for (int n = 0; n < NT; ++n)
      if (n < nvt) dma16_m0(dr[n] + col, __builtin_amdgcn_readfirstlane(st + kSlab + (wave * NT + n) * 1024));
  };

#pragma unroll
  for (int c = 0; c < S - 1; ++c)
    if (c < nc) dma(c, c);

  f32x4_t acc[DT][NT];
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[d][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int jq = lane & 15;
  const int kr0 = 8 * gq + (jq >> 2);
  uint32_t aoff[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const int col = 16 * d + 4 * (jq & 3);
    aoff[d] = static_cast<uint32_t>(kr0 * 2 * HT + 16 * ((col >> 3) ^ swz_mn(kr0)) + 2 * (col & 7));
  }
  const uint32_t boff = static_cast<uint32_t>(kSlab + wave * NT * 1024 + rr * 64 + 16 * (gq ^ swz_k(rr)));

  const int per_chunk = npw + nvt;
  // chunk c landed once at most (chunks issued after it) x per_chunk DMAs are outstanding; only
  // chunks < nc are moved (short bands have fewer than S - 1)
  auto ring_step = [&](int c) {
    const int after = nc - 1 - c < S - 2 ? nc - 1 - c : S - 2;
    ring_vm_wait<(S - 2) * (kMaxPW + NT)>(after * per_chunk);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + S - 1 < nc) dma(c + S - 1, (c + S - 1) % S);
  };
  if (nvt > 0) {
    for (int c = 0; c < nc; ++c) {
      ring_step(c);
      const char* sb = lds + (c % S) * kStage;
      const bool kin = 32 * c + 8 * gq < K;  // this lane's 8 K values lie in the band
      u32x4_t b[NT];
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        b[n] = *reinterpret_cast<const u32x4_t*>(sb + boff + n * 1024);
        if (!kin) b[n] = u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const u32x4_t af = tr_frag(sb + aoff[d], 4 * 2 * HT);
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[d][n] = mfma_raw<T>(af, b[n], acc[d][n]);
      }
    }
  } else {  // a wave without rows only moves its part of the weight slabs
    for (int c = 0; c < nc; ++c) ring_step(c);
  }
  vm_wait<0>();  // no DMA may still be writing this block's LDS
  __syncthreads();

  // epilogue through LDS: the tile dx[rows][h0 .. h0 + HT) rounded to the storage dtype is staged
  // row-major (pitch HT + 8 elements), then written out 16 bytes per lane along whole rows; with a
  // tanh input each unit is multiplied by 1 - x^2 of the same 8 elements, read the same way.
  constexpr int kOP = HT + 8;
  static_assert(4 * kWaveRows * kOP * 2 <= S * kStage, "staging tile");
  T* ot = reinterpret_cast<T*>(lds);
  if (nvt > 0) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int r = wave * kWaveRows + 16 * n + rr;
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const float v[4] = {acc[d][n][0], acc[d][n][1], acc[d][n][2], acc[d][n][3]};
        store_pack<T, 4>(ot + r * kOP + 16 * d + 4 * gq, v);
      }
    }
  }
  __syncthreads();
  const int64_t m0 = static_cast<int64_t>(mt) * (4 * kWaveRows);
  constexpr int kRowUnits = HT / 8;
  constexpr int kUnitsPerThread = 4 * kWaveRows * kRowUnits / 256;
  static_assert(4 * kWaveRows * kRowUnits % 256 == 0, "units per thread");
  const int tid = threadIdx.x;
  uint4 xin_u[kUnitsPerThread];
  if constexpr (TANH) {
#pragma unroll
    for (int k = 0; k < kUnitsPerThread; ++k) {
      const int q = tid + 256 * k;
      const int r = q / kRowUnits, u = q % kRowUnits;
      int64_t m = m0 + r;
      m = m < a.M ? m : a.M - 1;
      xin_u[k] = *reinterpret_cast<const uint4*>(xin + (m * a.NB + band) * H + h0 + 8 * u);
    }
  }
#pragma unroll
  for (int k = 0; k < kUnitsPerThread; ++k) {
    const int q = tid + 256 * k;
    const int r = q / kRowUnits, u = q % kRowUnits;
    if (m0 + r >= a.M) continue;
    uint4 v = *reinterpret_cast<const uint4*>(ot + r * kOP + 8 * u);
    if constexpr (TANH) {
      const T* dv = reinterpret_cast<const T*>(&v);
      const T* xv = reinterpret_cast<const T*>(&xin_u[k]);
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = to_f32(xv[e]);
        o[e] = to_f32(dv[e]) * (1.0f - t * t);
      }
      Pack<T, 8> pk;
#pragma unroll
      for (int e = 0; e < 8; ++e) pk.v[e] = from_f32<T>(o[e]);
      v = __builtin_bit_cast(uint4, pk);
    }
    // non-temporal: dz (M x NB x H, far larger than the L2s) would otherwise displace the weight slabs,
    // dpre rows and x lines this kernel is still reading; the stores are whole 16-byte units along rows
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v),
                                reinterpret_cast<u32x4_t*>(dz + ((m0 + r) * a.NB + band) * H + h0 + 8 * u));
  }
}

template <typename T, int DT, int NT>
int launch(const void* dpre, const void* w, const void* x, void* dz, const DzArgs& a, const int64_t* dim_inputs,
           bool tanh_in, hipStream_t stream) {
  constexpr int HT = 16 * DT;
  BandSched sc;
  uint32_t per_xcd = 0;
  const int64_t rows = 64 * NT;
  if (!build_band_sched(
          a.NB, (a.M + rows - 1) / rows, [&](int) { return static_cast<int64_t>(a.H / HT); },
          // cost of a block: its K chunks plus 5 for the prologue and the epilogue (its x read and dz
          // write); measured at configs[1], a 1-chunk block takes ~5.8 us against ~1.2 us per chunk of
          // a 33-chunk one.  With +2 the XCDs holding the 8- and 16-wide bands ran 9 rounds of them and
          // finished last (73 -> 59 us)
          [&](int b) { return (2 * dim_inputs[b] + 31) / 32 + 5; },
          &sc, &per_xcd))
    return fail(PMSST_EINVAL, "mask_estimator_final_backward: too many bands or rows for the dz schedule");
  const dim3 grid(per_xcd * kXcds);
  const T* dp = static_cast<const T*>(dpre);
  const T* wp = static_cast<const T*>(w);
  const T* xp = static_cast<const T*>(x);
  if (tanh_in)
    hipLaunchKernelGGL((me_dz_kernel<T, DT, NT, true>), grid, dim3(256), 0, stream, dp, wp, xp, static_cast<T*>(dz),
                       a, sc);
  else
    hipLaunchKernelGGL((me_dz_kernel<T, DT, NT, false>), grid, dim3(256), 0, stream, dp, wp, xp,
                       static_cast<T*>(dz), a, sc);
  return check_launch("me_dz_kernel");
}

}  // namespace

bool mask_dz_supported(int64_t H, int64_t rows, size_t elem, const void* dpre, const void* w, const void* x,
                       const void* dx, int64_t total) {
  const bool al = reinterpret_cast<uintptr_t>(dpre) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(x) % 8 == 0 && reinterpret_cast<uintptr_t>(dx) % 8 == 0;
  return elem == 2 && al && rows > 0 && (H % 192 == 0 || H % 128 == 0) && H <= 8192 &&
         2 * total * H * 2 < (int64_t{1} << 40);
}

template <typename T>
int launch_mask_dz(const void* dpre, const void* w, const void* x, void* dx, const int64_t* offsets,
                   const int64_t* dim_inputs, int NB, int64_t M, int64_t H, int F, bool tanh_in, hipStream_t stream) {
  const DzArgs a{offsets, M, NB, static_cast<int>(H), F};
  if (H % 192 == 0) return launch<T, 12, 2>(dpre, w, x, dx, a, dim_inputs, tanh_in, stream);
  return launch<T, 8, 2>(dpre, w, x, dx, a, dim_inputs, tanh_in, stream);
}

template int launch_mask_dz<bf16>(const void*, const void*, const void*, void*, const int64_t*, const int64_t*, int,
                                  int64_t, int64_t, int, bool, hipStream_t);
template int launch_mask_dz<f16>(const void*, const void*, const void*, void*, const int64_t*, const int64_t*, int,
                                 int64_t, int64_t, int, bool, hipStream_t);

}  // namespace pmsst
