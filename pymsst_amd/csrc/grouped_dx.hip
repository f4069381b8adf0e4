// Grouped linear backward, input gradient, 16-bit storage:
//   dx[m, g, :] = dy[m, g, :] W_g          (K = out_features = O, the mask MLP's hidden size)
// dy[M, G, O], W[G, O, I] (group g's [O, I] weight), dx[M, G, I].
//
// Block = (group g, row tile): 4 waves x 16 NT rows (NT 2 or 3 at I = 192, picked per shape); a row
// tile may be shorter than the block's 64 NT rows (a multiple of 16: the waves past its end only move
// weight slabs, see gdx_row_tile).  Each
// wave accumulates dx^T[I x 16 NT] for its rows over the whole K = O in registers.  Per 32-wide K
// chunk c a ring stage receives, by global -> LDS DMA, the weight slab W_g[32 c .. 32 c + 31][0 .. I)
// (shared by the 4 waves; read as transposed A fragments, ds_read_b64_tr_b16) and the block's dy tile
// dy[rows][g][32 c .. + 31] (each wave moves and reads its own rows; K-contiguous B fragments).
// S stages keep S - 1 chunks of both in flight (S = 4, or 3 for 48-row waves to stay at two blocks
// per CU), which the short per-chunk MFMA work needs to cover HBM latency.  dy is read once and dx
// written once; the weight comes from L2.  No atomics.
#include "common.h"
#include "dma_gemm.h"
#include "grouped_dx.h"
#include "ring.h"

namespace pmsst {
namespace {

struct GdxArgs {
  int64_t M;
  int G, O, I;
  int rb;  // rows of a block's row tile (a multiple of 16, at most 64 NT)
};

template <typename T, int DT, int NT, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void glin_dx_kernel(const T* __restrict__ dy, const T* __restrict__ w,
                                                      T* __restrict__ dx, GdxArgs a, BandSched sc) {
  constexpr int I = 16 * DT;               // input features
  constexpr int kUnits = I / 8;            // 16-byte units per weight row
  constexpr int kSlab = 32 * 2 * I;        // weight slab bytes
  constexpr int kInstr = kSlab / 1024;     // its DMA instructions (= DT)
  constexpr int kMaxPW = (kInstr + 3) / 4;
  constexpr int kWaveRows = 16 * NT;
  constexpr int kStage = kSlab + 4 * kWaveRows * 64;  // + the dy tile: 64 bytes per row
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];

  int g;
  uint32_t mt, sub, per;
  if (!sched_block<true>(sc, g, mt, sub, per)) return;
  const int O = a.O;
  const int lane = threadIdx.x & 63, gq = lane >> 4, rr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t wrow0 = static_cast<int64_t>(mt) * a.rb + wave * kWaveRows;
  const int64_t tile_end = static_cast<int64_t>(mt + 1) * a.rb < a.M ? static_cast<int64_t>(mt + 1) * a.rb : a.M;
  const int64_t left = tile_end - wrow0;
  const int nvt = left <= 0 ? 0 : (left >= kWaveRows ? NT : static_cast<int>((left + 15) / 16));
  const int nc = O / 32;

  // weight DMA: instruction t (wave t % 4) moves flattened units 64 t + lane of the slab: row
  // P / kUnits, physical unit P % kUnits <- logical unit (P % kUnits) ^ swz_mn(row) (a permutation
  // inside aligned groups of 8 units, so it stays inside the row)
  const int npw = (kInstr - wave + 3) / 4;
  uint32_t gsrc[kMaxPW];
#pragma unroll
  for (int q = 0; q < kMaxPW; ++q) {
    const int t = wave + 4 * q;
    const int P = 64 * t + lane;
    const int kr = P / kUnits, pu = P % kUnits;
    const int u = pu ^ swz_mn(kr);
    gsrc[q] = static_cast<uint32_t>((kr * I + 8 * u) * 2);
  }
  const char* wg = reinterpret_cast<const char*>(w + static_cast<int64_t>(g) * O * I);
  // dy DMA: instruction n of this wave moves rows wrow0 + 16 n + lane / 4 (clamped), physical unit
  // lane % 4 <- logical unit (lane % 4) ^ swz_k(lane / 4)
  const char* dyr[NT];
  {
    const int u = (lane & 3) ^ swz_k(lane >> 2);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      int64_t m = wrow0 + 16 * n + (lane >> 2);
      m = m < a.M ? m : a.M - 1;
      dyr[n] = reinterpret_cast<const char*>(dy + (m * a.G + g) * O + 8 * u);
    }
  }
  const int ndy = nvt;  // dy DMAs of this wave per chunk (row groups with a valid row)
  const uint32_t lds0 = lds_addr(lds);
  auto dma = [&](int c, int stage) {
    const uint32_t st = lds0 + static_cast<uint32_t>(stage * kStage);
#pragma unroll
    for (int q = 0; q < kMaxPW; ++q)
      if (q < npw)
        dma16_m0(wg + gsrc[q] + static_cast<uint32_t>(c) * (64u * I),
                 __builtin_amdgcn_readfirstlane(st + (wave + 4 * q) * 1024));
#pragma unroll
    for (int n = 0; n < NT; ++n)
      if (n < ndy)
        dma16_m0(dyr[n] + static_cast<uint32_t>(c) * 64u,
                 __builtin_amdgcn_readfirstlane(st + kSlab + (wave * NT + n) * 1024));
  };

#pragma unroll
  for (int c = 0; c < S - 1; ++c) dma(c < nc ? c : nc - 1, c);

  f32x4_t acc[DT][NT];
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[d][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // transposed-fragment offsets of d-tile d inside a slab (columns 16 d .. + 15, K rows 8 gq ..)
  const int jq = lane & 15;
  const int kr0 = 8 * gq + (jq >> 2);
  const int col0 = 4 * (jq & 3);
  uint32_t aoff[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const int col = 16 * d + col0;
    aoff[d] = static_cast<uint32_t>(kr0 * 2 * I + 16 * ((col >> 3) ^ swz_mn(kr0)) + 2 * (col & 7));
  }
  // B fragment of row tile n: row 16 n + rr of this wave's tile, logical unit gq
  const uint32_t boff = static_cast<uint32_t>(kSlab + wave * NT * 1024 + rr * 64 + 16 * (gq ^ swz_k(rr)));

  const int per_chunk = npw + ndy;
  // chunk c: this wave's DMAs of chunk c have landed (chunks c + 1 .. c + S - 2 may be in flight),
  // its LDS reads of chunk c - 1 are done, then every wave's (barrier): the stage of chunk c - 1 is
  // free for chunk c + S - 1
  auto ring_step = [&](int c) {
    ring_vm_wait<(S - 2) * (kMaxPW + NT)>((S - 2) * per_chunk);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    dma(c + S - 1 < nc ? c + S - 1 : nc - 1, (c + S - 1) % S);
  };
  if (nvt == 0) {  // a wave without rows only moves its part of the weight slabs
    for (int c = 0; c < nc; ++c) ring_step(c);
    vm_wait<0>();
    return;
  }
  for (int c = 0; c < nc; ++c) {
    ring_step(c);
    const char* sb = lds + (c % S) * kStage;
    u32x4_t b[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) b[n] = *reinterpret_cast<const u32x4_t*>(sb + boff + n * 1024);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const u32x4_t af = tr_frag(sb + aoff[d], 4 * 2 * I);
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[d][n] = mfma_raw<T>(af, b[n], acc[d][n]);
    }
  }
  vm_wait<0>();  // no DMA may still be writing this block's LDS when its waves end

  // lane holds dx^T[16 d + 4 gq + r][16 n + rr]: 4 consecutive inputs of one row
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int64_t m = wrow0 + 16 * n + rr;
    if (n >= nvt || m >= a.M) continue;
    T* row = dx + (m * a.G + g) * I + 4 * gq;
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const float v[4] = {acc[d][n][0], acc[d][n][1], acc[d][n][2], acc[d][n][3]};
      store_pack<T, 4>(row + 16 * d, v);
    }
  }
}

// Row tile of the 48-row-wave form: the smallest multiple of 16 rows that keeps the grid in the block
// rounds the full tile (192 rows) needs.  Every block costs the same K loop, and a round lasts as
// long as its longest blocks, so shorter tiles on the same rounds shorten the kernel (configs[1],
// M = 1032, 62 groups: 8 tiles of 144 rows instead of 6 of 192 (5 x 192 + 72), 496 blocks against
// 372 in one round of two per CU: 50.2-50.5 -> 43.1 us on two boxes; 160 rows 45.6-46.1 us).
int64_t gdx_row_tile(int64_t M, int64_t groups, int64_t full, int64_t slots) {
  const int64_t rounds = (groups * ((M + full - 1) / full) + slots - 1) / slots;
  const int64_t tiles = rounds * slots / groups;  // row tiles that fit in those rounds
  if (tiles <= 0) return full;
  const int64_t rb = ((M + tiles - 1) / tiles + 15) / 16 * 16;
  return rb < full ? rb : full;
}

template <typename T, int DT, int NT, int S>
int launch(const void* dy, const void* w, void* dx, const GdxArgs& a, int64_t rows, hipStream_t stream) {
  BandSched sc;
  uint32_t per_xcd = 0;
  if (rows <= 0 || rows > 64 * NT || rows % 16 != 0)
    return fail(PMSST_EINVAL, "grouped_linear_backward: row tile %lld outside the block", (long long)rows);
  GdxArgs ar = a;
  ar.rb = static_cast<int>(rows);
  if (!build_even_sched(a.G, (a.M + rows - 1) / rows, [](int) { return int64_t{1}; }, &sc, &per_xcd))
    return fail(PMSST_EINVAL, "grouped_linear_backward: too many groups or rows for the block schedule");
  hipLaunchKernelGGL((glin_dx_kernel<T, DT, NT, S>), dim3(per_xcd * kXcds), dim3(256), 0, stream,
                     static_cast<const T*>(dy), static_cast<const T*>(w), static_cast<T*>(dx), ar, sc);
  return check_launch("glin_dx_kernel");
}

}  // namespace

bool grouped_dx_supported(int64_t groups, int64_t in_features, int64_t out_features, int64_t rows, size_t elem,
                          const void* dy, const void* w, const void* dx) {
  const bool al = reinterpret_cast<uintptr_t>(dy) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(dx) % 8 == 0;
  const bool in_ok = in_features == 64 || in_features == 128 || in_features == 192 || in_features == 256;
  return elem == 2 && al && in_ok && out_features >= 64 && out_features % 32 == 0 && rows > 0 &&
         groups <= kSchedMaxBands && out_features * in_features * 2 < (int64_t{1} << 31);
}

template <typename T>
int launch_grouped_dx(const void* dy, const void* w, void* dx, int64_t groups, int64_t in_features,
                      int64_t out_features, int64_t rows, hipStream_t stream) {
  const GdxArgs a{rows, static_cast<int>(groups), static_cast<int>(out_features), static_cast<int>(in_features)};
  switch (in_features) {
    case 64: return launch<T, 4, 4, 4>(dy, w, dx, a, 256, stream);
    case 128: return launch<T, 8, 4, 4>(dy, w, dx, a, 256, stream);
    case 192: {
      // 4 waves of 32 rows (4 ring stages) or of 48 rows (3 stages), both two blocks per CU: the form
      // with fewer block rounds x rows per wave (48 on a tie).  A grid a few blocks past the CUs' slots
      // pays a whole block time for its last round (configs[1], M = 1032: 558 blocks of 32-row waves
      // took 43.4 us, 372 of 48-row waves 39.2 us; M = 1024: 496 blocks, 32.0 against 39.2 us).
      const int64_t slots = 2 * static_cast<int64_t>(num_cus());
      auto rounds = [&](int64_t block_rows) {
        const int64_t blocks = groups * ((rows + block_rows - 1) / block_rows);
        return (blocks + slots - 1) / slots;
      };
      if (rounds(192) * 3 <= rounds(128) * 2)
        return launch<T, 12, 3, 3>(dy, w, dx, a, gdx_row_tile(rows, groups, 192, slots), stream);
      return launch<T, 12, 2, 4>(dy, w, dx, a, 128, stream);
    }
    case 256: return launch<T, 16, 2, 4>(dy, w, dx, a, 128, stream);
    default: return fail(PMSST_EINVAL, "grouped_linear_backward: in_features %lld not supported by glin_dx_kernel",
                         static_cast<long long>(in_features));
  }
}

template int launch_grouped_dx<bf16>(const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                                     hipStream_t);
template int launch_grouped_dx<f16>(const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                                    hipStream_t);

}  // namespace pmsst
