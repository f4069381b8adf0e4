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
// Forward block (128 rows of M, band b, 64 GLU outputs l): A = the 64 left rows
// and the 64 gate rows of W_b for those outputs, B = x rows; each lane holds a
// left accumulator and the gate accumulator of the same output, and the GLU is
// applied in registers.  16-bit inputs with 4-aligned widths run me_fwd_dma_kernel
// (global -> LDS DMA ring, XCD-grouped block schedule); other cases run
// me_fwd_kernel (register-staged main loop of gemm.h).
//
// Backward:
//   1. me_dpre_kernel writes dpre = (g * s, g * L * s * (1 - s)), s = sigmoid(G),
//      to a [M, 2F] workspace (one pass over pre and grad_out);
//   2. dbias = column sums of dpre (colsum_rows_kernel + col_sum_kernel);
//   3. dx^T[h][m] = W_b^T dpre_b^T  (K = 2*I_b), tiles 128 h x 64 m; with a tanh
//      input (mask-MLP hidden layer) the epilogue writes dz = dx * (1 - x^2);
//   4. dW^T[h][j] = x_b^T dpre_b    (K = M),     tiles 128 h x 64 j.
// All reductions have a fixed order; no atomics.
#include "common.h"
#include "dma_gemm.h"
#include "gemm.h"
#include "rowgeom.h"
#include "grouped_dx.h"
#include "ring.h"

namespace pmsst {
namespace {

struct MaskArgs {
  const int64_t* offsets;  // device [NB + 1] (prefix sums of I_b)
  int64_t M;
  int NB;
  int H;
  int F;
  bool vec4;  // every I_b and H a multiple of 4 and all tensors 4-element aligned
  int uniform_I = 0;  // > 0: every band has I_b = uniform_I (offsets unused; the dW kernel only)
};

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + __expf(-z)); }

// ------------------------------------------------------------------ forward

// A operand of the forward: rows [0, 64) are left rows l0 + r of W_b, rows
// [64, 128) the gate rows I + l0 + (r - 64); K = H contiguous.  Outputs l >= I are
// clamped to l = I - 1 in interior chunks (discarded by the epilogue).
template <typename T, bool V4>
struct LeftGateLoader : KRowLoader<T, 128, V4> {
  using Base = KRowLoader<T, 128, V4>;
  int I, l0;
  __device__ __forceinline__ LeftGateLoader(const T* wb, int H, int I_, int l0_) : Base{wb, H, 128, H}, I(I_), l0(l0_) {}
  __device__ __forceinline__ void prepare() {
    this->rowok = 0;
#pragma unroll
    for (int i = 0; i < Base::kQuads; ++i) {
      const int r = Base::tile_row(i);
      const int l = l0 + (r & 63);
      const int lc = l < I ? l : I - 1;
      this->src_row[i] = r < 64 ? lc : I + lc;
      this->rowok |= static_cast<uint32_t>(l < I) << i;
    }
    this->finish_prepare();
  }
};

// Forward tile: 128 rows of M x (64 left + 64 gate outputs).  One chunk of prefetch in
// registers and a register budget of 3 waves per SIMD (the compiler fits 4) measured faster
// than two chunks in flight at 2 waves per SIMD: 52 vs 60 us at configs[1] shapes.
#ifndef PMSST_ME_FWD_DEPTH
#define PMSST_ME_FWD_DEPTH 1
#endif
#ifndef PMSST_ME_FWD_WAVES
#define PMSST_ME_FWD_WAVES 3
#endif
constexpr int kFwdBM = 128;

template <typename T, bool V4>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(PMSST_ME_FWD_WAVES))) void me_fwd_kernel(const T* __restrict__ x, const T* __restrict__ weight,
                                                              const T* __restrict__ bias, T* __restrict__ pre,
                                                              T* __restrict__ out, int max_lchunks, XcdGrid xg,
                                                              MaskArgs a, BandSched sc) {
  __shared__ T lds[gemm_lds_elems<T, 128, kFwdBM>()];
  using S = TileShape<128, kFwdBM, 1, 4>;  // TR = 8 (4 left + 4 gate), TC = 2
  int band, l0;
  uint32_t mt;
  if (sc.m_tiles != 0) {
    // one block per existing (band, row tile, 64-output chunk), evenly split over the XCDs
    uint32_t chunk, nch;
    if (!sched_block(sc, band, mt, chunk, nch)) return;
    l0 = static_cast<int>(chunk) * 64;
  } else {
    uint32_t grp;  // group = (band, 64-output chunk), member = row tile: weight chunk shared in L2
    if (!xcd_block(xg, grp, mt)) return;
    band = static_cast<int>(grp) / max_lchunks;
    l0 = (static_cast<int>(grp) % max_lchunks) * 64;
  }
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  if (l0 >= I) return;
  const int64_t m0 = static_cast<int64_t>(mt) * kFwdBM;
  const int rows_valid = static_cast<int>(a.M - m0 < kFwdBM ? a.M - m0 : kFwdBM);
  const int H = a.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  LeftGateLoader<T, V4> la(weight + static_cast<int64_t>(2) * off * H, H, I, l0);
  KRowLoader<T, kFwdBM, V4> lb{x + (m0 * a.NB + band) * H, static_cast<int64_t>(a.NB) * H, rows_valid, H};
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int i = 0; i < S::kTR; ++i)
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, 128, kFwdBM, 1, 4, PMSST_ME_FWD_DEPTH>(la, lb, H, lds, acc);

  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int l = l0 + i * 16 + 4 * (lane >> 4);
    if (l >= I) continue;
    float bl[4], bg[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bl[r] = l + r < I ? to_f32(bias[2 * off + l + r]) : 0.f;
      bg[r] = l + r < I ? to_f32(bias[2 * off + I + l + r]) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) {
      const int m = wave * (kFwdBM / 4) + j * 16 + (lane & 15);
      if (m >= rows_valid) continue;
      float vl[4], vg[4], vo[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vl[r] = acc[i][j][r] + bl[r];
        vg[r] = acc[i + 4][j][r] + bg[r];
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
}

// ------------------------------------------------------------------ forward, DMA pipeline
//
// The register-staged main loop keeps one 16 KB chunk per block in flight, and at three
// blocks per CU the forward is bound by load latency, not by HBM, LDS or MFMA throughput.
// This kernel moves the chunks with global -> LDS DMA (global_load_lds_dwordx4: 16 bytes per
// lane into LDS at M0 + 16 * lane, no registers involved), so S - 1 chunks of both operands are
// in flight per block (a ring of S LDS stages of 16 KB), with one barrier per chunk.
//
// Tile: 128 rows of M x 64 GLU outputs of one band.  A stage holds 128 weight rows then 128 x
// rows, 64 bytes (one 32-wide K chunk) per row.  Weight rows are ordered in 16-row blocks left,
// gate, left, gate, ...: tile row R is output l0 + 16 (R / 32) + R % 16, gate when (R / 16) is
// odd.  The four 16-byte units of a row are stored XOR-swizzled (swz_k) so MFMA fragment
// reads are free of bank conflicts.
//
// Waves are 2 x 2: wave (wr, wc) multiplies weight rows 64 wr .. + 64 (4 fragments = 32
// outputs, left and gate of each) by x rows 64 wc .. + 64 (4 fragments), so each lane ends
// with 4 consecutive outputs and their gates (in-register GLU).  A wave whose 32 outputs lie
// past the band skips its reads and MFMAs.  DMA: wave w moves tile rows 64 w .. + 64 (waves
// 0-1 weight rows, 2-3 x rows), one dwordx4 per lane per 16 rows.
//
// The LDS reads are inline ds_read_b128 followed by an explicit lgkmcnt wait that the MFMA
// operands depend on; the DMA completion wait (vmcnt) and the barrier are explicit too.  This
// keeps the compiler from waiting for every DMA in flight before each LDS read (it cannot tell
// the ring's stages apart).  Chunk 0 (the only partial one: K is walked in chunks that end at
// H) is loaded through registers with the out-of-range units zeroed.
#ifndef PMSST_MEF_STAGES
#define PMSST_MEF_STAGES 4
#endif
#ifndef PMSST_MEF_BAND_DMA
#define PMSST_MEF_BAND_DMA 1
#endif
constexpr int kMefStage = 16384;  // bytes of one LDS stage


template <typename T>
__global__ __launch_bounds__(kGemmThreads) void me_fwd_dma_kernel(const T* __restrict__ x,
                                                                  const T* __restrict__ weight,
                                                                  const T* __restrict__ bias, T* __restrict__ pre,
                                                                  T* __restrict__ out, int max_lchunks, XcdGrid xg,
                                                                  MaskArgs a, BandSched sc) {
  constexpr int S = PMSST_MEF_STAGES;
  static_assert(S >= 2 && S <= 8, "stages");
  __shared__ __attribute__((aligned(1024))) char lds[S * kMefStage];
  int band, l0;
  uint32_t mt;
  if (sc.m_tiles != 0) {
    uint32_t chunk, nch;
    if (!sched_block(sc, band, mt, chunk, nch)) return;
    l0 = static_cast<int>(chunk) * 64;
  } else {
    uint32_t grp;  // group = (band, 64-output chunk), member = row tile: weight chunk shared in L2
    if (!xcd_block(xg, grp, mt)) return;
    band = static_cast<int>(grp) / max_lchunks;
    l0 = (static_cast<int>(grp) % max_lchunks) * 64;
  }
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  if (l0 >= I) return;
  const int64_t m0 = static_cast<int64_t>(mt) * kFwdBM;
  const int rows_valid = static_cast<int>(a.M - m0 < kFwdBM ? a.M - m0 : kFwdBM);
  const int H = a.H;
  const int lane = threadIdx.x & 63, g = lane >> 4, rr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wr = wave >> 1, wc = wave & 1;
  const bool active = l0 + 32 * wr < I;  // wave-uniform

  // DMA pieces of this lane: instruction t moves tile row R = 64 wave + 16 t + lane / 4
  // (R % 16 = lane / 4), physical unit lane % 4, i.e. logical K unit u = (lane % 4) ^ swz(lane / 4)
  const uint32_t u = static_cast<uint32_t>((lane & 3) ^ swz_k(lane >> 2));
  const int rsub = lane >> 2;
  uint32_t soff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int R = 64 * wave + 16 * t + rsub;
    if (wave < 2) {
      const int l = l0 + 16 * (R >> 5) + (R & 15);
      const int lc = l < I ? l : I - 1;
      soff[t] = static_cast<uint32_t>(((R >> 4) & 1) ? I + lc : lc) * static_cast<uint32_t>(H) * 2u + 16u * u;
    } else {
      const int m = R - 128 < rows_valid ? R - 128 : rows_valid - 1;
      soff[t] = static_cast<uint32_t>(m) * static_cast<uint32_t>(a.NB) * static_cast<uint32_t>(H) * 2u + 16u * u;
    }
  }
  const char* gbase = wave < 2 ? reinterpret_cast<const char*>(weight + static_cast<int64_t>(2) * off * H)
                               : reinterpret_cast<const char*>(x + (m0 * a.NB + band) * static_cast<int64_t>(H));
  const int nk = (H + kChunkK - 1) / kChunkK;  // >= 2 (host check)
  const int kbeg = H - nk * kChunkK;           // chunk c covers k in [kbeg + 32 c, +32)
  char* my_lds = lds + (4 * wave) * 1024;      // this wave's 4 KB of a stage

  // Weight waves move only the 16-output groups inside the band (instruction t of wave w holds
  // outputs l0 + 32 w + 16 (t / 2) ..; the groups past the band would re-read its clamped last row
  // and only feed outputs that are never stored): nv = 4, 2 or 0 DMAs per chunk, wave-uniform.
#if PMSST_MEF_BAND_DMA
  const int nv = wave >= 2 ? 4 : (l0 + 32 * wave + 16 < I ? 4 : (l0 + 32 * wave < I ? 2 : 0));
#else
  const int nv = 4;
#endif
  auto dma = [&](int c, int stage) {  // chunk c >= 1 into `stage`
    const char* src = gbase + 2 * (kbeg + kChunkK * c);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t < nv)
        __builtin_amdgcn_global_load_lds(src + soff[t], my_lds + stage * kMefStage + t * 1024, 16, 0, 0);
  };

  // chunk 0 through registers: units with k < 0 are zero (they load k = 0 of the row)
  {
    const bool ok = kbeg + 8 * static_cast<int>(u) >= 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t o = ok ? soff[t] + static_cast<uint32_t>(2 * kbeg) : soff[t] - 16u * u;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(gbase + o);
      *reinterpret_cast<u32x4_t*>(my_lds + t * 1024 + lane * 16) = ok ? v : u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int c = 1; c < S - 1; ++c) dma(c < nk ? c : nk - 1, c);

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // fragment read addresses inside a stage: row R, logical unit g -> R * 64 + 16 (g ^ swz(R % 16))
  const uint32_t sw = 16u * static_cast<uint32_t>(g ^ swz_k(rr));
  const uint32_t abase = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)) +
                         static_cast<uint32_t>((64 * wr + rr) * 64) + sw;
  const uint32_t bbase = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)) + 8192u +
                         static_cast<uint32_t>((64 * wc + rr) * 64) + sw;

  for (int c = 0; c < nk; ++c) {
    // chunk c landed: the DMAs issued after it are chunks c + 1 .. c + S - 2 (nv per chunk)
    if (c > 0) {
      if (nv == 4) vm_wait<4 * (S - 2)>();
      else if (nv == 2) vm_wait<2 * (S - 2)>();
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // refill the stage chunk c - 1 used (every wave is past its reads); clamped at the end
    dma(c + S - 1 < nk ? c + S - 1 : nk - 1, (c + S - 1) % S);
    if (active) {
      const uint32_t st = static_cast<uint32_t>((c % S) * kMefStage);
      u32x4_t af[4], bf[4];
      const uint32_t pa = abase + st, pb = bbase + st;
      asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(af[0]) : "v"(pa));
      asm volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(af[1]) : "v"(pa));
      asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(af[2]) : "v"(pa));
      asm volatile("ds_read_b128 %0, %1 offset:3072" : "=v"(af[3]) : "v"(pa));
      asm volatile("ds_read_b128 %0, %1 offset:0" : "=v"(bf[0]) : "v"(pb));
      asm volatile("ds_read_b128 %0, %1 offset:1024" : "=v"(bf[1]) : "v"(pb));
      asm volatile("ds_read_b128 %0, %1 offset:2048" : "=v"(bf[2]) : "v"(pb));
      asm volatile("ds_read_b128 %0, %1 offset:3072" : "=v"(bf[3]) : "v"(pb));
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(af[0]), "+v"(af[1]), "+v"(af[2]), "+v"(af[3]), "+v"(bf[0]), "+v"(bf[1]), "+v"(bf[2]),
                     "+v"(bf[3]));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_raw<T>(af[i], bf[j], acc[i][j]);
    }
  }
  // no DMA may still be writing this block's LDS when its waves end or the epilogue reuses it
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // epilogue through LDS: fragment pair (2h, 2h + 1) = (left, gate) of outputs
  // l0 + 32 wr + 16 h + 4 g + r of rows m = 64 wc + 16 j + rr (8-byte runs of 16 rows per
  // instruction).  The three result tiles (pre left, pre gate, out) are staged as [128 m][64 l]
  // (row pitch 144 bytes) and written back row by row, 16 lanes x 8 bytes = 128 contiguous
  // bytes per row, so HBM sees whole lines.
  __syncthreads();  // every wave is done with the ring
  constexpr int kOP = 72;  // staged row pitch in elements
  T* ol = reinterpret_cast<T*>(lds);
  T* og = ol + kFwdBM * kOP;
  T* oo = og + kFwdBM * kOP;
  if (active) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int lt = 32 * wr + 16 * h + 4 * g;  // tile column
      const int l = l0 + lt;
      float bl[4] = {0.f, 0.f, 0.f, 0.f}, bgt[4] = {0.f, 0.f, 0.f, 0.f};
      if (l < I) {  // I_b is a multiple of 4 on this path: the 4 outputs are all valid or none
        load_pack<T, 4>(bias + 2 * off + l, bl);
        load_pack<T, 4>(bias + 2 * off + I + l, bgt);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = 64 * wc + 16 * j + rr;
        float vl[4], vg[4], vo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          vl[r] = acc[2 * h][j][r] + bl[r];
          vg[r] = acc[2 * h + 1][j][r] + bgt[r];
          vo[r] = vl[r] * sigmoidf_(vg[r]);
        }
        store_pack<T, 4>(ol + m * kOP + lt, vl);
        store_pack<T, 4>(og + m * kOP + lt, vg);
        store_pack<T, 4>(oo + m * kOP + lt, vo);
      }
    }
  }
  __syncthreads();
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  const int c4 = (static_cast<int>(threadIdx.x) & 15) * 4;  // tile column of this thread's piece
  if (l0 + c4 < I) {
#pragma unroll
    for (int p = 0; p < kFwdBM / 16; ++p) {
      const int m = static_cast<int>(threadIdx.x >> 4) + 16 * p;
      if (m >= rows_valid) break;
      T* pl = pre + (m0 + m) * pitch2 + 2 * off + l0 + c4;
      *reinterpret_cast<u32x2_t*>(pl) = *reinterpret_cast<const u32x2_t*>(ol + m * kOP + c4);
      *reinterpret_cast<u32x2_t*>(pl + I) = *reinterpret_cast<const u32x2_t*>(og + m * kOP + c4);
      *reinterpret_cast<u32x2_t*>(out + (m0 + m) * a.F + off + l0 + c4) =
          *reinterpret_cast<const u32x2_t*>(oo + m * kOP + c4);
    }
  }
}

// ------------------------------------------------------------------ backward

constexpr int kDpreRows = 64;
constexpr int kDpreFlatRows = 4;  // 4 rows: 10.9 us at configs[1] against 12.5 us with 8
constexpr int kDpreFlatMaxBands = 4096;  // band offsets in LDS, 16 KB

// dpre over whole rows (aligned case): thread t takes column quad t % (F / 4) of the kDpreFlatRows
// rows of row group t / (F / 4), so consecutive threads read consecutive quads of the same rows
// whatever the band widths (band offsets are multiples of 4, so a quad lies in one band, found by
// binary search over the offsets staged in LDS).  The thread index fits 32 bits (host check), so the
// row group and quad come from one 32-bit division (a 64-bit one took 0.3 us more at configs[1]).  The
// rows past M are clamped reads (issued with the others, no branch before the arithmetic) whose
// results are not stored.
template <typename T>
__global__ __launch_bounds__(256) void me_dpre_flat_kernel(const T* __restrict__ gout, const T* __restrict__ pre,
                                                           T* __restrict__ dpre, MaskArgs a) {
  __shared__ int soff[kDpreFlatMaxBands + 1];
  for (int b = threadIdx.x; b <= a.NB; b += 256) soff[b] = static_cast<int>(a.offsets[b]);
  __syncthreads();
  constexpr int V = 4;
  const uint32_t nq = static_cast<uint32_t>(a.F / V);
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const int64_t m0 = static_cast<int64_t>(t / nq) * kDpreFlatRows;
  if (m0 >= a.M) return;
  const int c0 = V * static_cast<int>(t % nq);
  int lo = 0, hi = a.NB - 1;  // last band with soff[b] <= c0
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (soff[mid] <= c0) lo = mid; else hi = mid - 1;
  }
  const int off = soff[lo];
  const int I = soff[lo + 1] - off;
  const int l = c0 - off;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  float g[kDpreFlatRows][V], L[kDpreFlatRows][V], G[kDpreFlatRows][V];
#pragma unroll
  for (int r = 0; r < kDpreFlatRows; ++r) {
    const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;
    load_pack<T, V>(gout + m * a.F + c0, g[r]);
    load_pack<T, V>(pre + m * pitch2 + 2 * off + l, L[r]);
    load_pack<T, V>(pre + m * pitch2 + 2 * off + l + I, G[r]);
  }
#pragma unroll
  for (int r = 0; r < kDpreFlatRows; ++r) {
    float ol[V], og[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float sg = sigmoidf_(G[r][j]);
      ol[j] = g[r][j] * sg;
      og[j] = g[r][j] * L[r][j] * sg * (1.0f - sg);
    }
    if (m0 + r < a.M) {
      T* dl = dpre + (m0 + r) * pitch2 + 2 * off + l;
      store_pack<T, V>(dl, ol);
      store_pack<T, V>(dl + I, og);
    }
  }
}

// dpre for rows [blockIdx.x * 64, +64) of band blockIdx.y, 4 outputs per item.
template <typename T>
__global__ __launch_bounds__(256) void me_dpre_kernel(const T* __restrict__ gout, const T* __restrict__ pre,
                                                      T* __restrict__ dpre, MaskArgs a) {
  const int band = blockIdx.y;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kDpreRows;
  const int rows = static_cast<int>(a.M - m0 < kDpreRows ? a.M - m0 : kDpreRows);
  const int nq = (I + 3) / 4;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  for (int idx = threadIdx.x; idx < rows * nq; idx += 256) {
    const int r = idx / nq;
    const int l = (idx - r * nq) * 4;
    const int64_t m = m0 + r;
    const T* gp = gout + m * a.F + off + l;
    const T* pl = pre + m * pitch2 + 2 * off + l;
    const T* pg = pl + I;
    T* dl = dpre + m * pitch2 + 2 * off + l;
    T* dg = dl + I;
    float g[4], L[4], G[4], ol[4], og[4];
    if (a.vec4) {
      load_pack<T, 4>(gp, g);
      load_pack<T, 4>(pl, L);
      load_pack<T, 4>(pg, G);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = l + j < I;
        g[j] = ok ? to_f32(gp[j]) : 0.f;
        L[j] = ok ? to_f32(pl[j]) : 0.f;
        G[j] = ok ? to_f32(pg[j]) : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = sigmoidf_(G[j]);
      ol[j] = g[j] * s;
      og[j] = g[j] * L[j] * s * (1.0f - s);
    }
    if (a.vec4) {
      store_pack<T, 4>(dl, ol);
      store_pack<T, 4>(dg, og);
    } else {
      for (int j = 0; j < 4 && l + j < I; ++j) {
        dl[j] = from_f32<T>(ol[j]);
        dg[j] = from_f32<T>(og[j]);
      }
    }
  }
}

constexpr int kDxBH = 128;
constexpr int kDxBM = 64;

// TANH_IN: the layer input x is tanh(z) of the previous layer, and the kernel writes
// dz = (dpre W_b) * (1 - x^2) instead of dx (the hidden activation's backward, fused).
template <typename T, bool TANH_IN, bool V4>
__global__ __launch_bounds__(kGemmThreads) void me_bwd_dx_kernel(const T* __restrict__ dpre,
                                                                 const T* __restrict__ weight,
                                                                 const T* __restrict__ x, T* __restrict__ dx,
                                                                 int hchunks, XcdGrid xg, MaskArgs a) {
  __shared__ T lds[gemm_lds_elems<T, kDxBH, kDxBM>()];
  using S = TileShape<kDxBH, kDxBM, 2, 2>;
  uint32_t grp, mt;  // group = (band, hidden chunk), member = row tile: weight chunk shared in L2
  if (!xcd_block(xg, grp, mt)) return;
  const int band = static_cast<int>(grp) / hchunks;
  const int h0 = (static_cast<int>(grp) % hchunks) * kDxBH;
  const int64_t m0 = static_cast<int64_t>(mt) * kDxBM;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int H = a.H;
  const int rows_valid = static_cast<int>(a.M - m0 < kDxBM ? a.M - m0 : kDxBM);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);

  // A[h][j] = W_b[j][h0 + h]  (MN-contiguous in h);  B[m][j] = dpre[m0 + m][2 off + j]
  MNLoader<T, kDxBH, V4> la{weight + static_cast<int64_t>(2) * off * H + h0, H, H - h0, 2 * I};
  KRowLoader<T, kDxBM, V4> lb{dpre + m0 * pitch2 + 2 * off, pitch2, rows_valid, 2 * I};
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int i = 0; i < S::kTR; ++i)
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, kDxBH, kDxBM, 2, 2>(la, lb, 2 * I, lds, acc);

  const int hr = (wave >> 1) * (kDxBH / 2), mc = (wave & 1) * (kDxBM / 2);
#pragma unroll
  for (int i = 0; i < S::kTR; ++i) {
    const int h = h0 + hr + i * 16 + 4 * (lane >> 4);
    if (h >= H) continue;
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) {
      const int m = mc + j * 16 + (lane & 15);
      if (m >= rows_valid) continue;
      const int64_t idx = ((m0 + m) * a.NB + band) * H + h;
      T* dst = dx + idx;
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      if (TANH_IN) {
        float t[4] = {0.f, 0.f, 0.f, 0.f};
        if (a.vec4) {
          load_pack<T, 4>(x + idx, t);
        } else {
          for (int r = 0; r < 4 && h + r < H; ++r) t[r] = to_f32(x[idx + r]);
        }
#pragma unroll
        // dh is rounded to the tensor dtype before the tanh factor, as the reference's autograd
        // rounds the final layer's input gradient before tanh's backward
        for (int r = 0; r < 4; ++r) v[r] = to_f32(from_f32<T>(v[r])) * (1.0f - t[r] * t[r]);
      }
      if (a.vec4) {
        store_pack<T, 4>(dst, v);
      } else {
        for (int r = 0; r < 4 && h + r < H; ++r) dst[r] = from_f32<T>(v[r]);
      }
    }
  }
}

// dx on the DMA ring (16-bit, 4-aligned widths, H % 128 == 0).  Tile 128 h x 128 m: per K
// chunk, A = W_b^T as stored (32 K-rows j x 128 h, 8 KB, transpose-read fragments) and
// B = dpre rows (128 m x 32 j, 8 KB).  The bound is the L2 -> CU traffic of the re-read
// operand tiles, so the tile is as large as one block's registers allow (every weight chunk
// is read once per 128 rows).  Chunk 0 of K is the partial one (K chunks end at 2 I_b);
// its pieces with j < 0 are read from row / column 0 and zeroed in LDS once the DMA has
// landed.  DMA: 16 dwordx4 per stage, wave w moves weight K-rows 4w .. 4w + 3 and
// 16 + 4w .. 16 + 4w + 3 and dpre rows 16w .. 16w + 15 and 64 + 16w .. 64 + 16w + 15.
// The block schedule balances the XCDs by K steps and starts the long (wide-band) blocks
// first.
#ifndef PMSST_ME_DX_DMA
#define PMSST_ME_DX_DMA 1
#endif
#ifndef PMSST_ME_DX_STAGES
#define PMSST_ME_DX_STAGES 4
#endif
#ifndef PMSST_ME_DX256_STAGES
#define PMSST_ME_DX256_STAGES 3
#endif
// Hidden columns per block: 256 (8 waves) when the hidden size allows, else 128 (4 waves).
#ifndef PMSST_ME_DX_HC
#define PMSST_ME_DX_HC 256
#endif
constexpr int kDxBMd = 128;  // rows per block

template <typename T, bool TANH_IN, int HC>
__global__ __launch_bounds__(512) void me_bwd_dx_dma_kernel(const T* __restrict__ dpre,
                                                              const T* __restrict__ weight,
                                                              const T* __restrict__ x, T* __restrict__ dx,
                                                              BandSched sc, MaskArgs a) {
  constexpr int S = HC == 128 ? PMSST_ME_DX_STAGES : PMSST_ME_DX256_STAGES;
  static_assert(S >= 3 && S <= 8, "stages");
  constexpr int NW = HC / 32;              // waves: (HC / 64) x 2
  constexpr int kU = HC / 8;               // 16-byte units per weight K-row
  constexpr int kWTile = kChunkK * HC * 2;  // weight tile bytes; the dpre tile (8 KB) follows
  constexpr int kStage = kWTile + 8192;
  constexpr int kDI = 8 / NW;               // dpre DMAs per wave and stage (2 weight DMAs each)
  static_assert(HC == 128 || HC == 256, "hidden columns per block");
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];
  int band;
  uint32_t mt, hc, nhc_u;
  if (!sched_block<true>(sc, band, mt, hc, nhc_u)) return;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int H = a.H, K = 2 * I;
  const int64_t m0 = static_cast<int64_t>(mt) * kDxBMd;
  const int rows_valid = static_cast<int>(a.M - m0 < kDxBMd ? a.M - m0 : kDxBMd);
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wr = wave >> 1, wc = wave & 1;  // hidden columns 64 wr .., rows 64 wc ..
  const int nk = (K + kChunkK - 1) / kChunkK;
  const int kbeg = K - nk * kChunkK;  // multiple of 8 (I % 4 == 0)

  // DMA pieces of this lane.  Weight instruction t (of 2) of wave w is q = w + NW t: K-rows
  // (64 / kU) q + lane / kU, unit lane % kU of the row (logical unit ^ swz_mn).  dpre instruction
  // t (of kDI) is q = w + NW t: rows 16 q + lane / 4, unit (lane % 4) ^ swz_k.
  uint32_t aoff[2], aoff0[2], boff[kDI], boff0[kDI];  // byte offsets from the chunk's bases (full / chunk 0)
  bool aok0[2], bok0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int kr = (64 / kU) * (wave + NW * t) + lane / kU;
    const int ua = (lane % kU) ^ swz_mn_p<2 * HC>(kr);
    aoff[t] = static_cast<uint32_t>((kr * H + 8 * ua) * 2);
    aok0[t] = kbeg + kr >= 0;
    aoff0[t] = aok0[t] ? aoff[t] : static_cast<uint32_t>((-kbeg * H + 8 * ua) * 2);  // row j = 0
  }
  {
    const int ub = (lane & 3) ^ swz_k((lane >> 2) & 15);  // rows 16 q + lane / 4: same swizzle
    bok0 = kbeg + 8 * ub >= 0;
#pragma unroll
    for (int t = 0; t < kDI; ++t) {
      const int mr = 16 * (wave + NW * t) + (lane >> 2);
      const int mrc = mr < rows_valid ? mr : rows_valid - 1;
      boff[t] = static_cast<uint32_t>((mrc * pitch2 + 8 * ub) * 2);
      boff0[t] = bok0 ? boff[t] : static_cast<uint32_t>((mrc * pitch2 - kbeg) * 2);  // column j = 0
    }
  }
  const char* wsrc0 = reinterpret_cast<const char*>(weight + static_cast<int64_t>(2) * off * H +
                                                    static_cast<int64_t>(kbeg) * H + hc * HC);
  const char* dsrc0 = reinterpret_cast<const char*>(dpre + m0 * pitch2 + 2 * off + kbeg);
  const uint32_t lds0 = lds_addr(lds);

  auto dma = [&](int kc, int stage) {  // K chunk kc into `stage`
    const char* wsrc = wsrc0 + static_cast<int64_t>(kc) * kChunkK * H * 2;
    const char* dsrc = dsrc0 + kc * kChunkK * 2;
    char* st = lds + stage * kStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) dma_lds16(wsrc + (kc == 0 ? aoff0[t] : aoff[t]), st + (wave + NW * t) * 1024);
#pragma unroll
    for (int t = 0; t < kDI; ++t)
      dma_lds16(dsrc + (kc == 0 ? boff0[t] : boff[t]), st + kWTile + (wave + NW * t) * 1024);
  };
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) dma(s, s);

  uint32_t fa[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) fa[i] = frag_mn_addr_p<2 * HC>(lds0, 64 * wr + 16 * i, lane);
  const uint32_t fb = frag_k_addr(lds0 + kWTile, 64 * wc, lane);
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < nk; ++s) {
    // chunk s landed once at most (2 + kDI) nd DMAs are outstanding, nd = chunks issued after it
    // (s + 1 .. s + S - 2 that exist); the loop issues no other memory operation
    const int nd = nk - 1 - s < S - 2 ? nk - 1 - s : S - 2;
    static_assert(S - 2 <= 6, "wait table");
    switch (nd) {
      case 0: vm_wait<0>(); break;
      case 1: vm_wait<2 + kDI>(); break;
      case 2: vm_wait<2 * (2 + kDI)>(); break;
      case 3: vm_wait<3 * (2 + kDI)>(); break;
      case 4: vm_wait<4 * (2 + kDI)>(); break;
      case 5: vm_wait<5 * (2 + kDI)>(); break;
      default: vm_wait<6 * (2 + kDI)>(); break;
    }
    if (s == 0 && kbeg < 0) {
      // zero this lane's pieces of chunk 0 that lie below j = 0
      const u32x4_t z{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < 2; ++t)
        if (!aok0[t]) *reinterpret_cast<u32x4_t*>(lds + (wave + NW * t) * 1024 + lane * 16) = z;
#pragma unroll
      for (int t = 0; t < kDI; ++t)
        if (!bok0) *reinterpret_cast<u32x4_t*>(lds + kWTile + (wave + NW * t) * 1024 + lane * 16) = z;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s + S - 1 < nk) dma(s + S - 1, (s + S - 1) % S);  // into the stage chunk s - 1 used
    const uint32_t so = static_cast<uint32_t>((s % S) * kStage);
    u32x4_t af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = lds_read_tr_pair(fa[i] + so, 4 * 2 * HC);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[j] = lds_read_b128(fb + so + 1024 * j);
    lds_wait(af, bfr);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma_raw<T>(af[i], bfr[j], acc[i][j]);
  }

  // epilogue through LDS: lane holds h = 64 wr + 16 i + 4 (lane / 16) + r of rows
  // m = 64 wc + 16 j + lane % 16 (8-byte runs of 16 rows per instruction); the tile is staged as
  // [128 m][HC h] (row pitch 2 HC + 16 bytes) and written back as 16-byte pieces, 2 HC contiguous
  // bytes per row, so HBM sees whole lines.  With a tanh input the factor 1 - x^2 is applied
  // before staging (x read at the lane's own positions) to dpre W rounded to the tensor dtype, the
// reference's rounding point of the hidden activation's input gradient.
  __syncthreads();  // every wave is done with the ring (its last wait was vmcnt(0))
  constexpr int kOP = HC + 8;  // staged row pitch in elements
  static_assert(kDxBMd * kOP * 2 <= S * kStage, "staging tile");
  T* ot = reinterpret_cast<T*>(lds);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = 64 * wc + 16 * j + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 64 * wr + 16 * i + 4 * (lane >> 4);
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      if (TANH_IN) {
        const int mc = m < rows_valid ? m : rows_valid - 1;
        float tx[4];
        load_pack<T, 4>(x + ((m0 + mc) * a.NB + band) * H + hc * HC + h, tx);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = to_f32(from_f32<T>(v[r])) * (1.0f - tx[r] * tx[r]);
      }
      store_pack<T, 4>(ot + m * kOP + h, v);
    }
  }
  __syncthreads();
  const int c8 = static_cast<int>(threadIdx.x % kU) * 8;
#pragma unroll
  for (int p = 0; p < kDxBMd / 16; ++p) {
    const int row = static_cast<int>(threadIdx.x / kU) + 16 * p;
    if (row < rows_valid)
      *reinterpret_cast<u32x4_t*>(dx + ((m0 + row) * a.NB + band) * H + hc * HC + c8) =
          *reinterpret_cast<const u32x4_t*>(ot + row * kOP + c8);
  }
}

constexpr int kDwBH = 128;
constexpr int kDwBJ = 64;

template <typename T, bool V4>
__global__ __launch_bounds__(kGemmThreads) void me_bwd_dw_kernel(const T* __restrict__ dpre, const T* __restrict__ x,
                                                                 T* __restrict__ dw, T* __restrict__ dbias,
                                                                 int htiles, XcdGrid xg, MaskArgs a, BandSched sc) {
  __shared__ T lds[gemm_lds_elems<T, kDwBH, kDwBJ>()];
  using S = TileShape<kDwBH, kDwBJ, 2, 2>;
  int band, h0, j0, off, I;
  if (sc.m_tiles != 0) {
    // one block per existing (band, hidden tile, j chunk), evenly split over the XCDs; a band's
    // blocks run hidden tile by hidden tile, so the blocks of one x slab are neighbours
    uint32_t mt, sub, per_unit;
    if (!sched_block(sc, band, mt, sub, per_unit)) return;
    off = static_cast<int>(a.offsets[band]);
    I = static_cast<int>(a.offsets[band + 1]) - off;
    const uint32_t nj = (2 * I + kDwBJ - 1) / kDwBJ;
    h0 = static_cast<int>(sub / nj) * kDwBH;
    j0 = static_cast<int>(sub % nj) * kDwBJ;
  } else {
    uint32_t grp, jchunk;  // group = (band, hidden tile), member = j chunk: the x slab shared in L2
    if (!xcd_block(xg, grp, jchunk)) return;
    band = static_cast<int>(grp) / htiles;
    h0 = (static_cast<int>(grp) % htiles) * kDwBH;
    j0 = static_cast<int>(jchunk) * kDwBJ;
    off = static_cast<int>(a.offsets[band]);
    I = static_cast<int>(a.offsets[band + 1]) - off;
  }
  const int K2 = 2 * I;
  if (j0 >= K2) return;
  const int H = a.H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);

  // A[h][m] = x[m][band][h0 + h];  B[j][m] = dpre[m][2 off + j0 + j]   (both MN-contiguous, K = M)
  MNLoader<T, kDwBH, V4> la{x + static_cast<int64_t>(band) * H + h0, static_cast<int64_t>(a.NB) * H, H - h0,
                            static_cast<int>(a.M)};
  MNLoader<T, kDwBJ, V4> lb{dpre + 2 * off + j0, pitch2, K2 - j0, static_cast<int>(a.M)};
  // the first hidden tile of each (band, j chunk) also sums dpre over the rows: dbias
  lb.colsum = h0 == 0;
  f32x4_t acc[S::kTR][S::kTC];
#pragma unroll
  for (int i = 0; i < S::kTR; ++i)
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  gemm_mainloop<T, kDwBH, kDwBJ, 2, 2>(la, lb, static_cast<int>(a.M), lds, acc);
  if (lb.colsum) reduce_colsum<T, kDwBJ, V4>(lb, lds, dbias + 2 * off + j0);

  T* dwb = dw + static_cast<int64_t>(2) * off * H;  // [2I][H]
  const int hr = (wave >> 1) * (kDwBH / 2), jc = (wave & 1) * (kDwBJ / 2);
#pragma unroll
  for (int i = 0; i < S::kTR; ++i) {
    const int h = h0 + hr + i * 16 + 4 * (lane >> 4);
    if (h >= H) continue;
#pragma unroll
    for (int j = 0; j < S::kTC; ++j) {
      const int jj = j0 + jc + j * 16 + (lane & 15);
      if (jj >= K2) continue;
      T* dst = dwb + static_cast<int64_t>(jj) * H + h;
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      if (a.vec4) {
        store_pack<T, 4>(dst, v);
      } else {
        for (int r = 0; r < 4 && h + r < H; ++r) dst[r] = from_f32<T>(v[r]);
      }
    }
  }
}

// dW on the DMA ring (16-bit, 4-aligned widths, H % HT == 0): dW_b^T[h][j] =
// sum_m x[m][b][h] dpre[m][2 off + j], K = M.  Tile HT h x 128 j per block (band, hidden tile,
// j chunk), HT = 128 on 4 waves (2 x 2 of 64 x 64; 256 on 8 waves is built too: at configs[1] it
// measured 102 us of mask backward against 94.5 us with 128, whose 48 KB ring keeps three blocks
// per CU); both
// operands are moved as stored (32 K-rows m x HT or 128 columns) and read as transposed
// fragments, so each x row slab is re-read once per 128 columns of dpre and each dpre slab once
// per HT hidden columns.  K chunks end at M; chunk 0's rows m < 0 are read from row 0 and zeroed
// in LDS once the DMA has landed.  DMA per wave and stage: 2 x pieces and 8 / waves dpre pieces.
// dbias[j] = sum_m dpre[m][j] comes from the blocks of hidden tile 0: their two waves of hidden
// columns 0 .. 63 add 4 MFMAs per chunk with an all-ones A fragment.  The tile leaves through
// LDS as rows j of dW_b, 2 HT contiguous bytes each.  Three stages (48 or 72 KB) keep two or three
// blocks per CU.
#ifndef PMSST_ME_DW_DMA
#define PMSST_ME_DW_DMA 1
#endif
#ifndef PMSST_ME_DW_STAGES
#define PMSST_ME_DW_STAGES 3
#endif
#ifndef PMSST_ME_DW256_STAGES
#define PMSST_ME_DW256_STAGES 3
#endif
// Hidden columns per block: 128 (4 waves), or 256 (8 waves) when the hidden size allows.
#ifndef PMSST_ME_DW_HT
#define PMSST_ME_DW_HT 128
#endif
constexpr int kDwT = 128;  // j columns per block (the final layer's dW; the grouped dW may take 192)
constexpr int64_t kLdsBytes = 160 * 1024;  // LDS per CU (gfx950)

template <typename T, int HT, int JT = kDwT>
__global__ __launch_bounds__(512) void me_bwd_dw_dma_kernel(const T* __restrict__ dpre, const T* __restrict__ x,
                                                           T* __restrict__ dw, T* __restrict__ dbias, BandSched sc,
                                                           MaskArgs a) {
  constexpr int S = HT == 128 ? PMSST_ME_DW_STAGES : PMSST_ME_DW256_STAGES;
  static_assert(S >= 3 && S <= 8, "stages");
  static_assert(HT == 64 || HT == 128 || HT == 256, "hidden columns per block");
  static_assert(JT == 128 || JT == 192, "j columns per block");
  constexpr int WJ = JT / 64;               // wave columns (64 j each)
  constexpr int NW = HT / 64 * WJ;          // waves: (HT / 64) x WJ tiles of 64 x 64
  constexpr int kU = HT / 8;                // 16-byte units per x K-row
  constexpr int kJU = JT / 8;               // 16-byte units per dpre K-row
  constexpr int kXTile = kChunkK * HT * 2;  // x tile bytes; the dpre tile (32 K-rows x JT j) follows
  constexpr int kStage = kXTile + kChunkK * JT * 2;
  constexpr int kPX = kXTile / 1024;        // 1 KB DMA pieces of the x tile, then of the dpre tile
  constexpr int kPT = kPX + kChunkK * JT * 2 / 1024;
  constexpr int kMaxPW = (kPT + NW - 1) / NW;  // pieces per wave and stage, at most
  // both tiles' pieces split evenly over the waves: each wave's first kPX / NW pieces are x pieces
  // and its count is kMaxPW, both known at compile time
  constexpr bool kEven = kPX % NW == 0 && (kPT - kPX) % NW == 0;
  __shared__ __attribute__((aligned(1024))) char lds[S * kStage];
  int band;
  uint32_t mt0, sub, per_unit;
  if (!sched_block(sc, band, mt0, sub, per_unit)) return;
  const int H = a.H;
  const int htiles = H / HT;
  const int h0 = static_cast<int>(sub % htiles) * HT;
  const int j0 = static_cast<int>(sub / htiles) * JT;
  const int off = a.uniform_I > 0 ? band * a.uniform_I : static_cast<int>(a.offsets[band]);
  const int I = a.uniform_I > 0 ? a.uniform_I : static_cast<int>(a.offsets[band + 1]) - off;
  const int K2 = 2 * I;
  const int M = static_cast<int>(a.M);
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  const int64_t xstride = static_cast<int64_t>(a.NB) * H;  // elements between rows m of x
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wr = wave / WJ, wc = wave % WJ;  // hidden columns 64 wr .., j columns 64 wc ..
  const int nk = (M + kChunkK - 1) / kChunkK;
  const int kbeg = M - nk * kChunkK;

  // DMA pieces: piece k < kPX moves flattened units 64 k + lane of the x tile (K-row U / kU,
  // physical unit U % kU <- logical unit (U % kU) ^ swz_mn(K-row)); piece k >= kPX the same of the
  // dpre tile with kJU units per K-row (columns past 2 I clamped to the band's last 8).  Wave w
  // issues pieces w, w + NW, ... < kPT.
  const int npw = kEven ? kMaxPW : (kPT - wave + NW - 1) / NW;
  uint32_t goff[kMaxPW], goff0[kMaxPW];
  bool ok0[kMaxPW], isx[kMaxPW];
#pragma unroll
  for (int t = 0; t < kMaxPW; ++t) {
    const int k = wave + NW * t;
    isx[t] = kEven ? t < kPX / NW : k < kPX;
    const int units = isx[t] ? kU : kJU;
    const int U = 64 * (isx[t] ? k : k - kPX) + lane;
    const int kr = U / units;
    const int u = (U % units) ^ swz_mn(kr);
    ok0[t] = kbeg + kr >= 0;
    if (isx[t]) {
      goff[t] = static_cast<uint32_t>((kr * xstride + 8 * u) * 2);
      goff0[t] = ok0[t] ? goff[t] : static_cast<uint32_t>((-kbeg * xstride + 8 * u) * 2);  // row m = 0
    } else {
      const int jc = j0 + 8 * u < K2 ? j0 + 8 * u : K2 - 8;
      goff[t] = static_cast<uint32_t>((kr * pitch2 + jc) * 2);
      goff0[t] = ok0[t] ? goff[t] : static_cast<uint32_t>((-kbeg * pitch2 + jc) * 2);
    }
  }
  const char* xsrc0 = reinterpret_cast<const char*>(x + (static_cast<int64_t>(kbeg) * a.NB + band) * H + h0);
  const char* dsrc0 = reinterpret_cast<const char*>(dpre + static_cast<int64_t>(kbeg) * pitch2 + 2 * off);
  const uint32_t lds0 = lds_addr(lds);

  auto dma = [&](int kc, int stage) {  // K chunk kc into `stage`
    const char* xs = xsrc0 + static_cast<int64_t>(kc) * kChunkK * xstride * 2;
    const char* ds = dsrc0 + static_cast<int64_t>(kc) * kChunkK * pitch2 * 2;
    char* st = lds + stage * kStage;
#pragma unroll
    for (int t = 0; t < kMaxPW; ++t)
      if (t < npw) dma_lds16((isx[t] ? xs : ds) + (kc == 0 ? goff0[t] : goff[t]), st + (wave + NW * t) * 1024);
  };
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) dma(s, s);

  uint32_t fa[4], fb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fa[i] = frag_mn_addr(lds0, 64 * wr + 16 * i, 2 * HT, lane);
    fb[i] = frag_mn_addr(lds0 + kXTile, 64 * wc + 16 * i, 2 * JT, lane);
  }
  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // dbias = ones^T dpre: the waves of the first hidden tile's first 64 columns also multiply
  // their dpre fragments by an all-ones A fragment (every row of the product is the column sum)
  const bool do_bias = h0 == 0 && wr == 0 && dbias != nullptr;
  const uint32_t one2 = std::is_same<T, bf16>::value ? 0x3F803F80u : 0x3C003C00u;
  const u32x4_t ones{one2, one2, one2, one2};
  f32x4_t accb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) accb[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < nk; ++s) {
    // chunk s landed once at most npw nd DMAs are outstanding, nd = chunks issued after it
    const int nd = nk - 1 - s < S - 2 ? nk - 1 - s : S - 2;
    if constexpr (kEven) {
      static_assert(S - 2 <= 6, "wait table");
      switch (nd) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<kMaxPW>(); break;
        case 2: vm_wait<2 * kMaxPW>(); break;
        case 3: vm_wait<3 * kMaxPW>(); break;
        case 4: vm_wait<4 * kMaxPW>(); break;
        case 5: vm_wait<5 * kMaxPW>(); break;
        default: vm_wait<6 * kMaxPW>(); break;
      }
    } else {
      ring_vm_wait<(S - 2) * kMaxPW>(nd * npw);
    }
    if (s == 0 && kbeg < 0) {  // zero this wave's own pieces of chunk 0 that lie before row 0
      const u32x4_t z{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < kMaxPW; ++t)
        if (t < npw && !ok0[t]) *reinterpret_cast<u32x4_t*>(lds + (wave + NW * t) * 1024 + lane * 16) = z;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (s + S - 1 < nk) dma(s + S - 1, (s + S - 1) % S);  // into the stage chunk s - 1 used
    const uint32_t so = static_cast<uint32_t>((s % S) * kStage);
    u32x4_t af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = lds_read_tr_pair(fa[i] + so, 4 * 2 * HT);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[j] = lds_read_tr_pair(fb[j] + so, 4 * 2 * JT);
    lds_wait(af, bfr);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma_raw<T>(af[i], bfr[j], acc[i][j]);
    if (do_bias) {
#pragma unroll
      for (int j = 0; j < 4; ++j) accb[j] = mfma_raw<T>(ones, bfr[j], accb[j]);
    }
  }

  const int jv = K2 - j0 < JT ? K2 - j0 : JT;
  if (do_bias && lane < 16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int jj = 64 * wc + 16 * j + lane;
      if (jj < jv) dbias[2 * off + j0 + jj] = from_f32<T>(accb[j][0]);
    }
  }

  // epilogue through LDS: lane holds h = 64 wr + 16 i + 4 (lane / 16) + r of columns
  // j = 64 wc + 16 jj + lane % 16; staged as [JT j][HT h] (row pitch 2 HT + 16 bytes)
  __syncthreads();  // every wave is done with the ring (its last wait was vmcnt(0))
  constexpr int kOP = HT + 8;
  static_assert(JT * kOP * 2 <= S * kStage, "staging tile");
  T* ot = reinterpret_cast<T*>(lds);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int jj = 64 * wc + 16 * j + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      store_pack<T, 4>(ot + jj * kOP + 64 * wr + 16 * i + 4 * (lane >> 4), v);
    }
  }
  __syncthreads();
  T* dwb = dw + (static_cast<int64_t>(2) * off + j0) * H + h0;  // rows j of dW_b
  constexpr int kRowsPerPass = 64 * NW / kU;  // rows j written per pass, kU threads each
  static_assert(64 * NW % kU == 0 && JT % kRowsPerPass == 0, "write-out passes");
  const int c8 = static_cast<int>(threadIdx.x % kU) * 8;
#pragma unroll
  for (int p = 0; p < JT / kRowsPerPass; ++p) {
    const int jj = static_cast<int>(threadIdx.x / kU) + kRowsPerPass * p;
    if (jj < jv)
      *reinterpret_cast<u32x4_t*>(dwb + static_cast<int64_t>(jj) * H + c8) =
          *reinterpret_cast<const u32x4_t*>(ot + jj * kOP + c8);
  }
}

// ------------------------------------------------------------------ host side

struct HostMask {
  int NB, F, max_width;
  bool vec4;
};

#ifndef PMSST_ME_FWD_DMA
#define PMSST_ME_FWD_DMA 1
#endif
#ifndef PMSST_ME_FWD_SCHED
#define PMSST_ME_FWD_SCHED 1
#endif


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
  PMSST_REQUIRE(gemm_stride_ok(band_count * H, 4) && gemm_stride_ok(2 * total, 4),
                "%s: rows too long for 32-bit tile offsets", op);
  hm->NB = static_cast<int>(band_count);
  hm->F = static_cast<int>(total);
  hm->max_width = static_cast<int>(maxw);
  hm->vec4 = vec4;
  return PMSST_OK;
}

bool al(const void* p, size_t b) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % b == 0; }

template <typename T>
int launch_me_fwd(const void* x, const void* weight, const void* bias, const int64_t* offsets,
                  const int64_t* dim_inputs, const HostMask& hm, int64_t M, int64_t H, void* pre, void* out,
                  hipStream_t stream) {
  const char* op = "mask_estimator_final_forward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  if (M == 0) return PMSST_OK;
  PMSST_REQUIRE(x && weight && bias && offsets && pre && out, "%s: null pointer", op);
  MaskArgs a{offsets, M, hm.NB, static_cast<int>(H), hm.F, false};
  a.vec4 = hm.vec4 && al(x, 4 * sizeof(T)) && al(weight, 4 * sizeof(T)) && al(pre, 4 * sizeof(T)) &&
           al(out, 4 * sizeof(T));
  const int max_lchunks = (hm.max_width + 63) / 64;
  const XcdGrid xg{static_cast<uint32_t>(hm.NB * max_lchunks), static_cast<uint32_t>((M + kFwdBM - 1) / kFwdBM)};
  const dim3 grid(xg.blocks());
  // 16-bit, 4-aligned widths and bias, hidden a multiple of 8 (whole 16-byte K units), at least
  // two K chunks, 16-byte aligned rows: the DMA-pipelined kernel
  if constexpr (sizeof(T) == 2) {
    if (PMSST_ME_FWD_DMA && a.vec4 && H % 8 == 0 && H > kChunkK && al(x, 16) && al(weight, 16) &&
        al(bias, 4 * sizeof(T)) && (2 * static_cast<int64_t>(hm.max_width) + 1) * H * 2 < (int64_t{1} << 31) &&
        (static_cast<int64_t>(kFwdBM) * hm.NB + 1) * H * 2 < (int64_t{1} << 31)) {
      BandSched sc;
      uint32_t per_xcd = 0;
      const bool sched =
          PMSST_ME_FWD_SCHED && build_band_sched(
                                    hm.NB, (M + kFwdBM - 1) / kFwdBM,
                                    [&](int b) { return (dim_inputs[b] + 63) / 64; }, &sc, &per_xcd);
      const dim3 g(sched ? per_xcd * kXcds : grid.x);
      hipLaunchKernelGGL((me_fwd_dma_kernel<T>), g, dim3(kGemmThreads), 0, stream, static_cast<const T*>(x),
                         static_cast<const T*>(weight), static_cast<const T*>(bias), static_cast<T*>(pre),
                         static_cast<T*>(out), max_lchunks, xg, a, sc);
      return check_launch("me_fwd_dma_kernel");
    }
  }
  BandSched sc;  // sc.m_tiles = 0 (the XcdGrid, whose blocks past a band's width exit) past 256 bands
  uint32_t per_xcd = 0;
  const dim3 g(build_even_sched(hm.NB, (M + kFwdBM - 1) / kFwdBM, [&](int b) { return (dim_inputs[b] + 63) / 64; },
                                &sc, &per_xcd)
                   ? per_xcd * kXcds
                   : grid.x);
  if (a.vec4)
    hipLaunchKernelGGL((me_fwd_kernel<T, true>), g, dim3(kGemmThreads), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(weight), static_cast<const T*>(bias), static_cast<T*>(pre),
                       static_cast<T*>(out), max_lchunks, xg, a, sc);
  else
    hipLaunchKernelGGL((me_fwd_kernel<T, false>), g, dim3(kGemmThreads), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(weight), static_cast<const T*>(bias), static_cast<T*>(pre),
                       static_cast<T*>(out), max_lchunks, xg, a, sc);
  return check_launch("me_fwd_kernel");
}

size_t me_bwd_workspace(int64_t M, int F, size_t elem) {
  const size_t dpre = align_up(static_cast<size_t>(M) * 2 * static_cast<size_t>(F) * elem, 256);
  return dpre;
}

template <typename T>
int launch_me_bwd(const void* gout, const void* x, const void* pre, const void* weight, const int64_t* offsets,
                  const int64_t* dim_inputs, const HostMask& hm, int64_t M, int64_t H, void* dx, void* dbias,
                  void* dw, int input_act, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* op = "mask_estimator_final_backward";
  PMSST_REQUIRE(M >= 0 && M < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(input_act == PMSST_ACT_NONE || input_act == PMSST_ACT_TANH, "%s: bad input_activation %d", op,
                input_act);
  PMSST_REQUIRE(weight && offsets && dbias && dw && (M == 0 || (gout && x && pre && dx)), "%s: null pointer", op);
  const size_t need = me_bwd_workspace(M, hm.F, sizeof(T));
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(PMSST_EWORKSPACE, "%s: workspace of %zu bytes needed, got %zu", op, need,
                workspace == nullptr ? size_t{0} : workspace_bytes);
  }
  MaskArgs a{offsets, M, hm.NB, static_cast<int>(H), hm.F, false};
  a.vec4 = hm.vec4 && al(x, 4 * sizeof(T)) && al(weight, 4 * sizeof(T)) && al(pre, 4 * sizeof(T)) &&
           al(dx, 4 * sizeof(T)) && al(gout, 4 * sizeof(T)) && al(dw, 4 * sizeof(T));
  T* dpre = static_cast<T*>(workspace);
  if (M > 0) {
    const dim3 g1(static_cast<unsigned>((M + kDpreRows - 1) / kDpreRows), static_cast<unsigned>(hm.NB));
    const int64_t flat_threads = (M + kDpreFlatRows - 1) / kDpreFlatRows * (hm.F / 4);
    if (a.vec4 && hm.NB <= kDpreFlatMaxBands && flat_threads + 255 < (int64_t{1} << 31)) {
      hipLaunchKernelGGL((me_dpre_flat_kernel<T>), dim3(static_cast<unsigned>((flat_threads + 255) / 256)), dim3(256),
                         0, stream, static_cast<const T*>(gout), static_cast<const T*>(pre), dpre, a);
    } else
    hipLaunchKernelGGL((me_dpre_kernel<T>), g1, dim3(256), 0, stream, static_cast<const T*>(gout),
                       static_cast<const T*>(pre), dpre, a);
    int rc = check_launch("me_dpre_kernel");
    if (rc != PMSST_OK) return rc;
    bool dx_done = false;
    if constexpr (sizeof(T) == 2) {
      if (mask_dz_supported(H, M, sizeof(T), dpre, weight, x, dx, hm.F)) {
        rc = launch_mask_dz<T>(dpre, weight, x, dx, offsets, dim_inputs, hm.NB, M, H, hm.F,
                               input_act == PMSST_ACT_TANH, stream);
        if (rc != PMSST_OK) return rc;
        dx_done = true;
      }
    }
    BandSched dsc;
    uint32_t dx_per_xcd = 0;
    const int dx_hc = PMSST_ME_DX_HC == 256 && H % 256 == 0 ? 256 : 128;
    const int nhc = static_cast<int>(H / dx_hc);
    const bool dx_dma = !dx_done && sizeof(T) == 2 && PMSST_ME_DX_DMA && a.vec4 && H % dx_hc == 0 && al(weight, 16) &&
                        al(dx, 16) &&
                        (static_cast<int64_t>(kChunkK) * H + H) * 2 < (int64_t{1} << 31) &&
                        (kDxBMd * 2 * static_cast<int64_t>(hm.F) + 64) * 2 < (int64_t{1} << 31) &&
                        build_band_sched(
                            hm.NB, (M + kDxBMd - 1) / kDxBMd,
                            [&](int) { return static_cast<int64_t>(nhc); },  // hidden chunks
                            [&](int b) {  // K steps per block (+2 for its prologue and epilogue)
                              return (2 * dim_inputs[b] + kChunkK - 1) / kChunkK + 2;
                            },
                            &dsc, &dx_per_xcd);
    if constexpr (sizeof(T) == 2) {
      if (dx_dma) {
        const dim3 gd(dx_per_xcd * kXcds);
        const T* wp = static_cast<const T*>(weight);
        const T* xp = static_cast<const T*>(x);
        T* dxp = static_cast<T*>(dx);
        const bool tanh_in = input_act == PMSST_ACT_TANH;
        if (dx_hc == 256 && tanh_in)
          me_bwd_dx_dma_kernel<T, true, 256><<<gd, dim3(512), 0, stream>>>(dpre, wp, xp, dxp, dsc, a);
        else if (dx_hc == 256)
          me_bwd_dx_dma_kernel<T, false, 256><<<gd, dim3(512), 0, stream>>>(dpre, wp, xp, dxp, dsc, a);
        else if (tanh_in)
          me_bwd_dx_dma_kernel<T, true, 128><<<gd, dim3(256), 0, stream>>>(dpre, wp, xp, dxp, dsc, a);
        else
          me_bwd_dx_dma_kernel<T, false, 128><<<gd, dim3(256), 0, stream>>>(dpre, wp, xp, dxp, dsc, a);
        rc = check_launch("me_bwd_dx_dma_kernel");
        if (rc != PMSST_OK) return rc;
      }
    }
    if (!dx_dma && !dx_done) {
      const int hchunks = static_cast<int>((H + kDxBH - 1) / kDxBH);
      const XcdGrid xg2{static_cast<uint32_t>(hm.NB * hchunks), static_cast<uint32_t>((M + kDxBM - 1) / kDxBM)};
      const dim3 g2(xg2.blocks());
#define PMSST_MDX(TANH, V4)                                                                                    \
  hipLaunchKernelGGL((me_bwd_dx_kernel<T, TANH, V4>), g2, dim3(kGemmThreads), 0, stream, dpre,                   \
                     static_cast<const T*>(weight), static_cast<const T*>(x), static_cast<T*>(dx), hchunks, xg2, a)
      if (input_act == PMSST_ACT_TANH) {
        if (a.vec4) PMSST_MDX(true, true); else PMSST_MDX(true, false);
      } else {
        if (a.vec4) PMSST_MDX(false, true); else PMSST_MDX(false, false);
      }
#undef PMSST_MDX
      rc = check_launch("me_bwd_dx_kernel");
      if (rc != PMSST_OK) return rc;
    }
  }
  if constexpr (sizeof(T) == 2) {
    BandSched wsc;
    uint32_t dw_per_xcd = 0;
    const int dw_ht = PMSST_ME_DW_HT == 256 && H % 256 == 0 ? 256 : 128;
    const int htl = static_cast<int>(H / dw_ht);
    if (PMSST_ME_DW_DMA && M >= kChunkK && a.vec4 && H % dw_ht == 0 && al(x, 16) && al(dw, 16) &&
        (static_cast<int64_t>(kChunkK) * hm.NB * H + H) * 2 < (int64_t{1} << 31) &&
        (static_cast<int64_t>(kChunkK) * 2 * hm.F + 2 * hm.F) * 2 < (int64_t{1} << 31) &&
        build_band_sched(hm.NB, 1,
                         [&](int b) { return static_cast<int64_t>(htl) * ((2 * dim_inputs[b] + kDwT - 1) / kDwT); },
                         &wsc, &dw_per_xcd)) {
      if (dw_ht == 256)
        hipLaunchKernelGGL((me_bwd_dw_dma_kernel<T, 256>), dim3(dw_per_xcd * kXcds), dim3(512), 0, stream, dpre,
                           static_cast<const T*>(x), static_cast<T*>(dw), static_cast<T*>(dbias), wsc, a);
      else
        hipLaunchKernelGGL((me_bwd_dw_dma_kernel<T, 128>), dim3(dw_per_xcd * kXcds), dim3(256), 0, stream, dpre,
                           static_cast<const T*>(x), static_cast<T*>(dw), static_cast<T*>(dbias), wsc, a);
      return check_launch("me_bwd_dw_dma_kernel");  // dbias summed by the kernel
    }
  }
  const int max_jchunks = (2 * hm.max_width + kDwBJ - 1) / kDwBJ;
  const int htiles = static_cast<int>((H + kDwBH - 1) / kDwBH);
  const XcdGrid xg3{static_cast<uint32_t>(hm.NB * htiles), static_cast<uint32_t>(max_jchunks)};
  BandSched wsc3;  // wsc3.m_tiles = 0 (the XcdGrid, whose blocks past a band's width exit) past 256 bands
  uint32_t w3_per_xcd = 0;
  const dim3 g3(build_even_sched(
                    hm.NB, 1, [&](int b) { return htiles * ((2 * dim_inputs[b] + kDwBJ - 1) / kDwBJ); }, &wsc3,
                    &w3_per_xcd)
                    ? w3_per_xcd * kXcds
                    : xg3.blocks());
  if (a.vec4)
    hipLaunchKernelGGL((me_bwd_dw_kernel<T, true>), g3, dim3(kGemmThreads), 0, stream, dpre, static_cast<const T*>(x),
                       static_cast<T*>(dw), static_cast<T*>(dbias), htiles, xg3, a, wsc3);
  else
    hipLaunchKernelGGL((me_bwd_dw_kernel<T, false>), g3, dim3(kGemmThreads), 0, stream, dpre,
                       static_cast<const T*>(x), static_cast<T*>(dw), static_cast<T*>(dbias), htiles, xg3, a, wsc3);
  int rc = check_launch("me_bwd_dw_kernel");
  if (rc != PMSST_OK) return rc;
  // dbias was summed by the dW kernel (which also runs for M == 0 and then writes zeros)
  return PMSST_OK;
}

template <typename T>
int launch_uniform_dw_impl(const void* dy, const void* x, void* dw, void* db, int64_t groups, int64_t in_features,
                           int64_t out_features, int64_t rows, hipStream_t stream) {
  // dW_g[o][i] = sum_m dy[m][g][o] x[m][g][i] on me_bwd_dw_dma_kernel: dy plays dpre (bands of
  // uniform width 2 I_b = out_features), x plays the hidden activations (H = in_features)
  const int I = static_cast<int>(out_features / 2);
  MaskArgs a{nullptr, rows, static_cast<int>(groups), static_cast<int>(in_features), static_cast<int>(groups) * I,
             true, I};
  BandSched wsc;
  uint32_t per_xcd = 0;
  const int64_t htl = in_features / 64;
  // j tile: 192 columns (3 waves, 48 KB of ring: three blocks per CU) when that takes fewer rounds
  // of resident blocks than 128 (2 waves, 36 KB: four per CU); each x tile is then re-read for 4
  // instead of 6 column tiles at out_features 768
  auto rounds = [&](int64_t jt, int64_t ring_bytes) {
    const int64_t blocks = groups * htl * ((out_features + jt - 1) / jt);
    const int64_t slots = static_cast<int64_t>(num_cus()) * (kLdsBytes / ring_bytes);
    return (blocks + slots - 1) / slots;
  };
  const int64_t ring128 = 3 * kChunkK * 2 * (64 + 128), ring192 = 3 * kChunkK * 2 * (64 + 192);
  const int jt = rounds(192, ring192) < rounds(128, ring128) ? 192 : 128;
  if (!build_band_sched(static_cast<int>(groups), 1,
                        [&](int) { return htl * ((out_features + jt - 1) / jt); }, &wsc, &per_xcd))
    return fail(PMSST_EINVAL, "grouped_linear_backward: too many groups for the dW schedule");
  if (jt == 192)
    hipLaunchKernelGGL((me_bwd_dw_dma_kernel<T, 64, 192>), dim3(per_xcd * kXcds), dim3(192), 0, stream,
                       static_cast<const T*>(dy), static_cast<const T*>(x), static_cast<T*>(dw), static_cast<T*>(db),
                       wsc, a);
  else
    hipLaunchKernelGGL((me_bwd_dw_dma_kernel<T, 64>), dim3(per_xcd * kXcds), dim3(128), 0, stream,
                       static_cast<const T*>(dy), static_cast<const T*>(x), static_cast<T*>(dw), static_cast<T*>(db),
                       wsc, a);
  return check_launch("me_bwd_dw_dma_kernel");
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

bool uniform_dw_supported(int64_t groups, int64_t in_features, int64_t out_features, int64_t rows, size_t elem,
                          const void* dy, const void* x, const void* dw) {
  return elem == 2 && rows >= kChunkK && in_features % 64 == 0 && in_features > 0 && out_features % 8 == 0 &&
         out_features >= 8 && groups > 0 && groups <= kSchedMaxBands && al(dy, 16) && al(x, 16) && al(dw, 16) &&
         (static_cast<int64_t>(kChunkK) * groups * in_features + in_features) * 2 < (int64_t{1} << 31) &&
         (static_cast<int64_t>(kChunkK) * groups * out_features + groups * out_features) * 2 < (int64_t{1} << 31);
}

template <typename T>
int launch_uniform_dw(const void* dy, const void* x, void* dw, void* db, int64_t groups, int64_t in_features,
                      int64_t out_features, int64_t rows, hipStream_t stream) {
  return launch_uniform_dw_impl<T>(dy, x, dw, db, groups, in_features, out_features, rows, stream);
}
template int launch_uniform_dw<bf16>(const void*, const void*, void*, void*, int64_t, int64_t, int64_t, int64_t,
                                     hipStream_t);
template int launch_uniform_dw<f16>(const void*, const void*, void*, void*, int64_t, int64_t, int64_t, int64_t,
                                    hipStream_t);

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
    return launch_me_fwd<T>(x, weight, bias, dim_offsets, dim_inputs, hm, rows, hidden, pre, out,
                            static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_mask_estimator_final_backward_workspace_size(int64_t rows, int64_t total, int dtype) {
  if (rows < 0 || total <= 0 || !dtype_ok(dtype)) return 0;
  return me_bwd_workspace(rows, static_cast<int>(total), dtype_size(dtype));
}

int pmsst_mask_estimator_final_backward(const void* grad_out, const void* x, const void* pre, const void* weight,
                                        const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                        int64_t rows, int64_t hidden, void* grad_x, void* grad_bias,
                                        void* grad_weight, int input_activation, int dtype, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  HostMask hm;
  int rc = check_mask("mask_estimator_final_backward", dim_inputs, band_count, hidden, &hm);
  if (rc != PMSST_OK) return rc;
  return with_dtype(dtype, "mask_estimator_final_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_me_bwd<T>(grad_out, x, pre, weight, dim_offsets, dim_inputs, hm, rows, hidden, grad_x, grad_bias,
                            grad_weight,
                            input_activation, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
