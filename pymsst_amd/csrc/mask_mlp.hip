// Whole per-band mask MLP forward in one pass (16-bit storage):
//   z = x_b W1_b^T + b1_b  (stored dtype),  h = tanh(z)  (stored dtype),
//   pre = h W2_b^T + b2_b, out = left * sigmoid(gate)
// for every band b, without writing the hidden layer to HBM (it is written only when the caller
// asks for it, e.g. to keep it for the backward).
//
// Data layout in HBM (row-major):
//   x   [M, NB, D]      w1 [NB, H, D]       b1 [NB, H]
//   w2  sum_b 2 I_b H   (band b's [2 I_b, H] at 2 off_b H)      b2 [2F] (band b at 2 off_b)
//   pre [M, 2F]         out [M, F]          hidden (optional) [M, NB, H]
//
// Block = (band b, pass p, row tile): WV waves x 16 NT rows (4 x 64 or, at dim 192, 8 x 32), GLU
// outputs j in [64 p, 64 p + 64).
// Each wave keeps its rows of x_b in registers as MFMA B fragments (NT tiles x D / 32 K steps)
// and walks the hidden axis in chunks of 32:
//   GEMM1  h^T[32 x 16 NT] = W1_b[chunk] x_b^T     (A = W1 rows from LDS, B = x registers)
//   tanh   in registers; GEMM1's tile rows are ordered so that lane l's accumulators of the
//          two 16-row tiles hold hidden 8 (l / 16) .. + 7 of the chunk, which is exactly the K
//          slice of a GEMM2 B fragment: the hidden tile never leaves the registers
//   GEMM2  pre^T[128 x 16 NT] += W2_b[64 left + 64 gate rows, chunk] h^T
// The W1 chunk (32 x D) and the W2 chunk (128 x 32) of the block's band move from HBM/L2 into a
// ring of LDS stages by global -> LDS DMA, shared by the waves.  Epilogue: bias, GLU, stores.
// Bands wider than 64 take several passes, each recomputing GEMM1 (the price of keeping every
// accumulator in registers).  A pass whose band part has 1 or 2 groups of 16 GLU outputs per half
// runs an instance of the block with 2 or 4 GEMM2 tiles instead of 8.
//
// tanh: z is rounded to the storage dtype before the tanh (the reference's grouped Linear output),
// so tanh is a function of 16 bits.  A 64 KB table of the correctly rounded tanh of every
// non-negative 16-bit pattern (NaN and inf included; built on the host in double precision) sits in
// LDS; a packed pair of z costs two masked indices, two 16-bit LDS reads and one sign merge, and
// the pair is already half of a GEMM2 B fragment.
#include <cmath>
#include <cstring>
#include <mutex>

#include "common.h"
#include "dma_gemm.h"
#include "ring.h"


namespace pmsst {
namespace {

constexpr int kMlpMaxH = 2048;
constexpr int kMlpJ = 64;                  // GLU outputs per pass
constexpr int kMlpW2Bytes = 2 * kMlpJ * 64;  // 128 W2 rows x 32 hidden x 2 bytes
constexpr int kTanhEntries = 1 << 15;      // non-negative 16-bit patterns
constexpr int kTanhBytes = kTanhEntries * 2;

// tanh tables: [bf16 patterns | fp16 patterns], filled once per device from the host
__device__ __align__(256) uint16_t g_tanh_tables[2 * kTanhEntries];

// Mask application in the epilogue (stem s of S): est[b, s, c, f, t] = spec[b, f C + c, t] x the
// complex mask (out[m, 2 r], out[m, 2 r + 1]) of row m = b T + t, complex row r = f C + c, in the
// iSTFT layout [B * S * C, Fbins, T] (complex64); bin 0 zero when zero_dc.  The mask values are
// rounded to the storage dtype first, as the stored mask the stock product multiplies is.
struct MlpApply {
  const float2* spec;  // complex64 [B, Fbins * C, T]
  float2* est;         // complex64 [B * S * C, Fbins, T]
  FastDiv frames;      // T
  int C, Fbins, S, s, zero_dc;
};

struct MlpArgs {
  const int64_t* offsets;  // device [NB + 1] prefix sums of I_b
  const uint16_t* tanh;    // this dtype's table in device memory
  int64_t M;
  int NB, H, F;
  MlpApply ap;             // used by the APPLY kernels only
  int rb;                  // rows of a block's row tile (a multiple of 16, at most 16 NT WV)
};

template <int DK>
constexpr int mlp_stage_bytes() {
  return DK * 2048 + kMlpW2Bytes;
}

// Ring depth: three stages where LDS allows (the 64 KB table takes the rest), two for dim 384 / 512.
template <int DK>
constexpr int mlp_stages() {
  return DK >= 12 ? 2 : 3;
}

// Hidden row (inside the chunk) of row r of GEMM1 tile t: tile 0 takes 8 (r / 4) + r % 4, tile 1
// the same + 4.  Lane l holds rows 4 (l / 16) + i of each tile, i.e. hidden 8 (l / 16) + i and
// 8 (l / 16) + 4 + i: together the 8 consecutive K values of its GEMM2 B fragment.
__device__ __forceinline__ int mlp_hid_row(int t, int r) { return 8 * (r >> 2) + 4 * t + (r & 3); }

__device__ __forceinline__ float mlp_sigmoid(float z) { return 1.0f / (1.0f + __expf(-z)); }

// z pair (lo, hi) rounded to the storage dtype (round to nearest even), as packed 16-bit patterns
template <typename T>
__device__ __forceinline__ uint32_t round_pair(float lo, float hi) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, t2));
}

// LDS fragment read the compiler schedules and waits for itself (no inline asm: a value of an asm
// read is not known to be in flight, so the compiler may copy its register before the explicit wait).
__device__ __forceinline__ u32x4_t lds_frag(const char* lds, uint32_t off) {
  return *reinterpret_cast<const u32x4_t*>(lds + off);
}

// One block of the kernel below, for a pass whose band has NV (1, 2 or 4) 16-row groups of GLU
// outputs in each half: GEMM2 runs 2 NV tiles (left 0 .. NV - 1, gate NV .. 2 NV - 1 of acc2).
template <typename T, int DK, int NT, int WV, bool WRITE_H, bool APPLY, int NV>
__device__ __forceinline__ void mlp_fwd_block(const T* __restrict__ x, const T* __restrict__ w1,
                                              const T* __restrict__ b1, const T* __restrict__ w2,
                                              const T* __restrict__ b2, T* __restrict__ pre, T* __restrict__ out,
                                              T* __restrict__ hid, const MlpArgs& a, char* lds, uint16_t* stab,
                                              float* sb1, int band, uint32_t mt, uint32_t pass, int off, int I) {
  constexpr int S = mlp_stages<DK>();
  constexpr int kStage = mlp_stage_bytes<DK>();
  constexpr int D = 32 * DK;
  constexpr int kWaveRows = 16 * NT;
  constexpr int kMaxPW = (2 * DK + 2 * NV + WV - 1) / WV;  // DMA instructions per wave and chunk, at most
  // kLean: DMAs through dma16_m0 (the compiler does not track them, so its waits for its own LDS
  // reads stay exact; a tracked LDS DMA makes it drain every LDS read before each use) and every
  // wave issues kMaxPW of them per chunk (padded), so the ring waits on a compile-time count.  Dim
  // 256 (4 waves of 64 rows) has no registers left for either and keeps the builtin DMA and its own
  // count.
  constexpr bool kLean = DK != 8;
  static_assert(WV <= 2 * DK, "a wave's padding DMA repeats its first piece, which must be a W1 piece");
  const int j0 = static_cast<int>(pass) * kMlpJ;
  const int H = a.H;
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, rr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t wrow0 = static_cast<int64_t>(mt) * a.rb + wave * kWaveRows;
  const int64_t tile_end = static_cast<int64_t>(mt + 1) * a.rb < a.M ? static_cast<int64_t>(mt + 1) * a.rb : a.M;
  const int64_t rows_left = tile_end - wrow0;
  const int nvt = rows_left <= 0 ? 0 : (rows_left >= kWaveRows ? NT : static_cast<int>((rows_left + 15) / 16));

  for (int i = tid; i < H; i += 64 * WV) sb1[i] = to_f32(b1[static_cast<int64_t>(band) * H + i]);
  __syncthreads();

  // ---- DMA plan.  Instruction k of a chunk: k < 2 DK moves rows 16 (k % 2) .. + 15 of W1 K slice
  // k / 2 (1 KB); the next 2 nv2 move 16-row groups of the W2 chunk (left rows j0 + 16 q + r, then
  // gate rows I + j0 + 16 q + r; rows past the band clamped to its last row).  Groups wholly past
  // the band are not moved (their products are never stored).  Wave w issues k = w, w + WV, ...
  // and, with kLean, pads its share to kMaxPW with piece k = w again (same source, same LDS bytes).
  const int nv2 = (I - j0 + 15) / 16 < NV ? (I - j0 + 15) / 16 : NV;
  const int ntot = 2 * DK + 2 * nv2;
  const int npw = kLean ? kMaxPW : (ntot - wave + WV - 1) / WV;
  const int u = (lane & 3) ^ swz_k(lane >> 2);  // logical 16-byte unit this lane moves
  const char* w1b = reinterpret_cast<const char*>(w1 + static_cast<int64_t>(band) * H * D);
  const char* w2b = reinterpret_cast<const char*>(w2 + static_cast<int64_t>(2) * off * H);
  uint32_t gsrc[kMaxPW];
  uint32_t ldst[kMaxPW];
  bool w1k[kMaxPW];
#pragma unroll
  for (int q = 0; q < kMaxPW; ++q) {
    const int k = wave + WV * q;
    w1k[q] = k < 2 * DK || k >= ntot;
    if (kLean && k >= ntot) {  // padding: piece k = wave (wave < WV <= 2 DK, a W1 piece)
      const int r = 16 * (wave & 1) + (lane >> 2);
      gsrc[q] = static_cast<uint32_t>((r * D + 32 * (wave >> 1) + 8 * u) * 2);
      ldst[q] = static_cast<uint32_t>((wave >> 1) * 2048 + (wave & 1) * 1024);
    } else if (k < 2 * DK) {
      const int r = 16 * (k & 1) + (lane >> 2);
      gsrc[q] = static_cast<uint32_t>((r * D + 32 * (k >> 1) + 8 * u) * 2);
      ldst[q] = static_cast<uint32_t>((k >> 1) * 2048 + (k & 1) * 1024);
    } else {
      const int k2 = k - 2 * DK;
      const int half = k2 / (nv2 > 0 ? nv2 : 1), grp = k2 - half * nv2;
      const int jr = j0 + 16 * grp + (lane >> 2);
      const int jc = jr < I ? jr : I - 1;
      const int prow = half ? I + jc : jc;
      gsrc[q] = static_cast<uint32_t>((static_cast<int64_t>(prow) * H + 8 * u) * 2);
      ldst[q] = static_cast<uint32_t>(DK * 2048 + (4 * half + grp) * 1024);
    }
  }
  const int nc = H / 32;
  const uint32_t lds0 = lds_addr(lds);
  auto dma = [&](int c, int stage) {
#pragma unroll
    for (int q = 0; q < kMaxPW; ++q) {
      if (kLean || q < npw) {
        const char* src = w1k[q] ? w1b + gsrc[q] + static_cast<uint32_t>(c) * (64u * D)
                                 : w2b + gsrc[q] + static_cast<uint32_t>(c) * 64u;
        if constexpr (kLean)
          dma16_m0(src, __builtin_amdgcn_readfirstlane(lds0 + static_cast<uint32_t>(stage * kStage) + ldst[q]));
        else
          dma_lds16(src, lds + stage * kStage + ldst[q]);
      }
    }
  };

  // ---- x rows of this wave as B fragments: row wrow0 + 16 n + rr, K values 32 s + 8 g .. + 7
  u32x4_t xf[NT][DK];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    int64_t m = wrow0 + 16 * n + rr;
    m = m < a.M ? m : a.M - 1;
    const T* xr = x + (m * a.NB + band) * D + 8 * g;
#pragma unroll
    for (int s = 0; s < DK; ++s) xf[n][s] = *reinterpret_cast<const u32x4_t*>(xr + 32 * s);
  }

  // the tanh table: 64 DMAs of 1 KB, wave w moves pieces w, w + WV, ...; issued before
  // the ring's first chunks, so the first ring wait covers them (loads complete in order)
#pragma unroll
  for (int q = 0; q < kTanhBytes / 1024 / WV; ++q) {
    const int k = wave + WV * q;
    if constexpr (kLean)
      dma16_m0(reinterpret_cast<const char*>(a.tanh) + k * 1024 + lane * 16,
               __builtin_amdgcn_readfirstlane(lds_addr(stab) + static_cast<uint32_t>(k) * 1024u));
    else
      dma_lds16(reinterpret_cast<const char*>(a.tanh) + k * 1024 + lane * 16, reinterpret_cast<char*>(stab) + k * 1024);
  }
#pragma unroll
  for (int c = 0; c < S - 1; ++c) dma(c < nc ? c : nc - 1, c);

  f32x4_t acc2[2 * NV][NT];
#pragma unroll
  for (int t = 0; t < 2 * NV; ++t)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc2[t][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // fragment offsets inside a stage
  uint32_t a1off[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = mlp_hid_row(t, rr);
    a1off[t] = static_cast<uint32_t>(r * 64 + 16 * (g ^ swz_k(r & 15)));
  }
  const uint32_t a2off = static_cast<uint32_t>(DK * 2048 + rr * 64 + 16 * (g ^ swz_k(rr)));
  // GEMM2 row tiles: left 0 .. NV - 1 and gate NV .. 2 NV - 1 (acc2 index), the stage's W2 groups
  // t and 4 + t; tiles t >= nv2 (NV = 4 with 3 groups) hold stale LDS data and feed accumulators
  // that are never stored
  const int nt2 = nv2;

  // ---- per-chunk pieces
  // ring step of chunk c: this wave's DMAs of chunk c have landed (only chunks c + 1 .. c + S - 2
  // may still be in flight; loads complete in order) and its LDS reads are done, then every wave's
  // are (barrier), so the stage chunk c - 1 used is free for chunk c + S - 1
  auto ring_step = [&](int c) {
    if constexpr (kLean) vm_wait<(S - 2) * kMaxPW>();
    else ring_vm_wait<(S - 2) * kMaxPW>((S - 2) * npw);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    dma(c + S - 1 < nc ? c + S - 1 : nc - 1, (c + S - 1) % S);
  };
  // GEMM1 of chunk c: acc starts at b1 (lane: hidden 8 g + 4 t + i of the chunk in tile t), K = D
  auto gemm1 = [&](int c, f32x4_t (&acc)[2][NT]) {
    const char* sb = lds + (c % S) * kStage;
    const float4 bl = *reinterpret_cast<const float4*>(sb1 + 32 * c + 8 * g);
    const float4 bh = *reinterpret_cast<const float4*>(sb1 + 32 * c + 8 * g + 4);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      acc[0][n] = f32x4_t{bl.x, bl.y, bl.z, bl.w};
      acc[1][n] = f32x4_t{bh.x, bh.y, bh.z, bh.w};
    }
#pragma unroll
    for (int s = 0; s < DK; ++s) {
      const u32x4_t f0 = lds_frag(sb, a1off[0] + 2048u * s);
      const u32x4_t f1 = lds_frag(sb, a1off[1] + 2048u * s);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        acc[0][n] = mfma_raw<T>(f0, xf[n][s], acc[0][n]);
        acc[1][n] = mfma_raw<T>(f1, xf[n][s], acc[1][n]);
      }
    }
  };
  // GEMM2 A fragments of chunk c (the 2 NV tiles; skipping tiles per block at run time costs
  // registers (spills), hence the NV instances)
  auto read_fb = [&](int c, u32x4_t (&fb)[2 * NV]) {
    const char* sb = lds + (c % S) * kStage;
#pragma unroll
    for (int t = 0; t < 2 * NV; ++t) fb[t] = lds_frag(sb, a2off + 1024u * (t < NV ? t : 4 + t - NV));
  };
  // z pairs in the stored dtype (word k of tile n: hidden 8 g + 2 k, + 1) and their table reads
  auto tanh_issue = [&](const f32x4_t (&acc)[2][NT], uint32_t (&zp)[NT][4], uint32_t (&th)[NT][8]) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      zp[n][0] = round_pair<T>(acc[0][n][0], acc[0][n][1]);
      zp[n][1] = round_pair<T>(acc[0][n][2], acc[0][n][3]);
      zp[n][2] = round_pair<T>(acc[1][n][0], acc[1][n][1]);
      zp[n][3] = round_pair<T>(acc[1][n][2], acc[1][n][3]);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        th[n][2 * k] = stab[zp[n][k] & 0x7fffu];
        th[n][2 * k + 1] = stab[(zp[n][k] >> 16) & 0x7fffu];
      }
  };
  // h = tanh(z) in the stored dtype, packed as B fragments; stored when asked
  auto tanh_finish = [&](int c, const uint32_t (&zp)[NT][4], const uint32_t (&th)[NT][8], u32x4_t (&hb)[NT]) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = (th[n][2 * k] | (th[n][2 * k + 1] << 16)) | (zp[n][k] & 0x80008000u);
      hb[n] = u32x4_t{w[0], w[1], w[2], w[3]};
      if constexpr (WRITE_H) {
        const int64_t m = wrow0 + 16 * n + rr;
        if (n < nvt && m < a.M)
          *reinterpret_cast<u32x4_t*>(hid + (m * a.NB + band) * H + 32 * c + 8 * g) = hb[n];
      }
    }
  };
  auto gemm2 = [&](const u32x4_t (&fb)[2 * NV], const u32x4_t (&hb)[NT]) {
#pragma unroll
    for (int t = 0; t < 2 * NV; ++t)
#pragma unroll
      for (int n = 0; n < NT; ++n) acc2[t][n] = mfma_raw<T>(fb[t], hb[n], acc2[t][n]);
  };

  // ---- software pipeline over the chunks: iteration c runs GEMM1(c) while the table reads of chunk
  // c - 1 are in flight, then GEMM2(c - 1) with the fragments read in iteration c - 1
  f32x4_t accA[2][NT], accB[2][NT];
  u32x4_t fbp[2 * NV], hbp[NT];
  uint32_t zp[NT][4], th[NT][8];
  ring_step(0);
  if (nvt > 0) {
    gemm1(0, accA);
    read_fb(0, fbp);
  }
  for (int c = 1; c < nc; c += 2) {
    ring_step(c);
    if (nvt > 0) {
      tanh_issue(accA, zp, th);
      gemm1(c, accB);
      tanh_finish(c - 1, zp, th, hbp);
      gemm2(fbp, hbp);
      read_fb(c, fbp);
    }
    if (c + 1 < nc) {
      ring_step(c + 1);
      if (nvt > 0) {
        tanh_issue(accB, zp, th);
        gemm1(c + 1, accA);
        tanh_finish(c, zp, th, hbp);
        gemm2(fbp, hbp);
        read_fb(c + 1, fbp);
      }
    }
  }
  // the last chunk: nc - 1 (accA when nc is odd, accB when even)
  if (nvt > 0) {
    if (nc & 1) tanh_issue(accA, zp, th);
    else tanh_issue(accB, zp, th);
    tanh_finish(nc - 1, zp, th, hbp);
    gemm2(fbp, hbp);
  }
  // no DMA may still be writing this block's LDS when its waves end
  vm_wait<0>();
  if (nvt == 0) return;

  // ---- epilogue: lane holds pre columns j0 + 16 t + 4 g + i (left, tile t) and the same + I
  // (gate, tile NV + t) of rows wrow0 + 16 n + rr.  I is a multiple of 4 (host check): the 4
  // outputs of a lane are all inside the band or all outside.  Every load of the epilogue (b2, and
  // the spectrum with APPLY) is issued first, from addresses clamped into the band and the rows, so
  // the block waits for one memory latency instead of one per tile.
  const int64_t pitch2 = 2 * static_cast<int64_t>(a.F);
  // the lane's row and column indices pass an empty asm here, so the compiler cannot compute the
  // epilogue's addresses before the main loop (where they would take registers from it)
  int ge = g, rre = rr;
  asm volatile("" : "+v"(ge), "+v"(rre));
  float bl[NV][4], bg[NV][4];
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const int jt = j0 + 16 * t + 4 * ge;
    const int jc = t < nt2 && jt < I ? jt : I - 4;
    load_pack<T, 4>(b2 + 2 * off + jc, bl[t]);
    load_pack<T, 4>(b2 + 2 * off + I + jc, bg[t]);
  }
  // APPLY: the lane's 4 outputs of tile t are the (re, im) pairs of complex rows r0 and r0 + 1
  // (off + j is a multiple of 4); lanes rr = 0..15 hold consecutive rows m, i.e. consecutive frames
  [[maybe_unused]] float2 spv[NV][NT][2];
  [[maybe_unused]] uint32_t bbn[NT], ttn[NT];
  if constexpr (APPLY) {
    const MlpApply& ap = a.ap;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int64_t m = wrow0 + 16 * n + rre;
      const uint32_t um = static_cast<uint32_t>(m < a.M ? m : a.M - 1);
      bbn[n] = ap.frames.div(um);
      ttn[n] = um - bbn[n] * ap.frames.d;
    }
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int jt = j0 + 16 * t + 4 * ge;
      const int r0 = (off + (t < nt2 && jt < I ? jt : I - 4)) >> 1;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          spv[t][n][q] = ap.spec[(static_cast<int64_t>(bbn[n]) * ap.Fbins * ap.C + r0 + q) * ap.frames.d + ttn[n]];
    }
  }
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const int j = j0 + 16 * t + 4 * ge;
    if (t >= nt2 || j >= I) continue;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int64_t m = wrow0 + 16 * n + rre;
      if (n >= nvt || m >= a.M) continue;
      float vl[4], vg[4], vo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vl[i] = acc2[t][n][i] + bl[t][i];
        vg[i] = acc2[NV + t][n][i] + bg[t][i];
        vo[i] = vl[i] * mlp_sigmoid(vg[i]);
        // the GLU output rounded to fp32 before its 16-bit conversion, as torch and the reference
        // round it: the empty asm keeps the product in a register, or the compiler may fuse product
        // and fp16 conversion into a v_fma_mixlo_f16 that rounds once (one fp16 ulp away at times)
        asm volatile("" : "+v"(vo[i]));
      }
      T* pl = pre + m * pitch2 + 2 * off + j;
      store_pack<T, 4>(pl, vl);
      store_pack<T, 4>(pl + I, vg);
      if constexpr (APPLY) {
        const MlpApply& ap = a.ap;
        const int r0 = (off + j) >> 1;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int r = r0 + q;
          const int f = r / ap.C, c = r - f * ap.C;
          // the mask rounded to the storage dtype, as the stored mask is
          const float mr = to_f32(from_f32<T>(vo[2 * q])), mi = to_f32(from_f32<T>(vo[2 * q + 1]));
          const float2 sv = spv[t][n][q];
          float2 e = make_float2(sv.x * mr - sv.y * mi, sv.x * mi + sv.y * mr);
          if (ap.zero_dc && f == 0) e = make_float2(0.f, 0.f);
          ap.est[((static_cast<int64_t>(bbn[n]) * ap.S + ap.s) * ap.C + c) * static_cast<int64_t>(ap.Fbins) *
                     ap.frames.d +
                 static_cast<int64_t>(f) * ap.frames.d + ttn[n]] = e;
        }
      } else {
        store_pack<T, 4>(out + m * a.F + off + j, vo);
      }
    }
  }
}

template <typename T, int DK, int NT, int WV, bool WRITE_H, bool APPLY>
__global__ __launch_bounds__(64 * WV) void mlp_fwd_kernel(const T* __restrict__ x, const T* __restrict__ w1,
                                                      const T* __restrict__ b1, const T* __restrict__ w2,
                                                      const T* __restrict__ b2, T* __restrict__ pre,
                                                      T* __restrict__ out, T* __restrict__ hid, MlpArgs a,
                                                      BandSched sc) {
  __shared__ __attribute__((aligned(1024))) char lds[mlp_stages<DK>() * mlp_stage_bytes<DK>()];
  __shared__ __attribute__((aligned(1024))) uint16_t stab[kTanhEntries];
  __shared__ float sb1[kMlpMaxH];

  int band;
  uint32_t mt, pass, npass;
  if (!sched_block<true>(sc, band, mt, pass, npass)) return;
  const int off = static_cast<int>(a.offsets[band]);
  const int I = static_cast<int>(a.offsets[band + 1]) - off;
  const int groups = (I - static_cast<int>(pass) * kMlpJ + 15) / 16;  // 16-row groups of this pass, 1 .. 4+
  // the widest instance first: in this order none of the three spills registers
  if (groups >= 3)
    mlp_fwd_block<T, DK, NT, WV, WRITE_H, APPLY, 4>(x, w1, b1, w2, b2, pre, out, hid, a, lds, stab, sb1, band, mt,
                                                    pass, off, I);
  else if (groups == 2)
    mlp_fwd_block<T, DK, NT, WV, WRITE_H, APPLY, 2>(x, w1, b1, w2, b2, pre, out, hid, a, lds, stab, sb1, band, mt,
                                                    pass, off, I);
  else
    mlp_fwd_block<T, DK, NT, WV, WRITE_H, APPLY, 1>(x, w1, b1, w2, b2, pre, out, hid, a, lds, stab, sb1, band, mt,
                                                    pass, off, I);
}

// ------------------------------------------------------------------ host side

// Correctly rounded tanh of every non-negative 16-bit pattern of bf16 (bf = true) or fp16: the
// double tanh rounded once to the format's grid (round to nearest even), NaN to the quiet NaN.
double decode16(uint16_t bits, bool bf) {
  if (bf) {
    const uint32_t u = static_cast<uint32_t>(bits) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  }
  _Float16 h;
  std::memcpy(&h, &bits, 2);
  return static_cast<double>(h);
}

uint16_t encode_rne(double t, bool bf) {
  if (std::isnan(t)) return bf ? 0x7fc0 : 0x7e00;
  if (t == 0.0) return 0;
  const int prec = bf ? 8 : 11;     // significant bits
  const int emin = bf ? -126 : -14; // exponent of the smallest normal number
  int e;
  std::frexp(t, &e);  // t = m 2^e, m in [0.5, 1): leading bit 2^(e - 1)
  const int lead = e - 1 > emin ? e - 1 : emin;
  const double q = std::ldexp(1.0, lead - (prec - 1));  // grid spacing at t
  const double r = std::nearbyint(t / q) * q;           // default rounding: to nearest even
  if (bf) {
    const float f = static_cast<float>(r);  // exact: r has at most 8 significant bits
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return static_cast<uint16_t>(u >> 16);
  }
  const _Float16 h = static_cast<_Float16>(r);  // exact
  uint16_t out;
  std::memcpy(&out, &h, 2);
  return out;
}

uint16_t g_tanh_host[2 * kTanhEntries];
std::once_flag g_tanh_built;
std::mutex g_tanh_mu;
const uint16_t* g_tanh_dev[256];

void build_tanh_host() {
  for (int f = 0; f < 2; ++f)
    for (int b = 0; b < kTanhEntries; ++b)
      g_tanh_host[f * kTanhEntries + b] = encode_rne(std::tanh(decode16(static_cast<uint16_t>(b), f == 0)), f == 0);
}

// Device copy of the tables for the current device, uploaded on its first use with a synchronous
// copy (visible to every stream once it returns).  A first use under stream capture is refused.
int tanh_tables(hipStream_t stream, const uint16_t** out) {
  std::call_once(g_tanh_built, build_tanh_host);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256)
    return fail(PMSST_EINVAL, "mask_mlp_forward: no current device");
  std::lock_guard<std::mutex> lock(g_tanh_mu);
  if (g_tanh_dev[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(PMSST_EINVAL, "mask_mlp_forward: first call on a device must not be under stream capture");
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_tanh_tables)) != hipSuccess)
      return fail(PMSST_EINVAL, "mask_mlp_forward: tanh table symbol not found");
    if (hipMemcpy(p, g_tanh_host, sizeof(g_tanh_host), hipMemcpyHostToDevice) != hipSuccess)
      return fail(PMSST_EINVAL, "mask_mlp_forward: tanh table upload failed");
    g_tanh_dev[dev] = static_cast<const uint16_t*>(p);
  }
  *out = g_tanh_dev[dev];
  return PMSST_OK;
}

// Rows of a block's row tile.  The blocks run in rounds of one per CU, so a last row tile of a few
// rows costs a dispatch slot for little work: where the full tile leaves at most an eighth of itself
// in the last tile and one wave's rows less (full - 32) needs no extra tile, the tiles take full - 32
// rows (configs[1]: M = 1032 in 4 x 224 + 136 rows instead of 4 x 256 + 8: 1 to 3 us less per launch
// on each of three boxes, 96-98 -> 93-96 us; 208 and 240 rows were no faster than 256).
int64_t mlp_row_tile(int64_t M, int64_t full) {
  const int64_t tiles = (M + full - 1) / full, tail = M - (tiles - 1) * full;
  const int64_t alt = full - 32;
  if (M > full && tail <= full / 8 && (M + alt - 1) / alt == tiles) return alt;
  return full;
}

template <typename T, int DK, int NT, int WV = 4>
int launch_dk(const void* x, const void* w1, const void* b1, const void* w2, const void* b2, void* pre, void* out,
              void* hid, const MlpArgs& a, const int64_t* dim_inputs, hipStream_t stream) {
  BandSched sc;
  uint32_t per_xcd = 0;
  const int64_t rows_per_block = mlp_row_tile(a.M, 16 * NT * WV);
  MlpArgs ar = a;
  ar.rb = static_cast<int>(rows_per_block);
  // an even split of the blocks over the XCDs (units of one band stay contiguous, so its weight chunks
  // are shared in one L2 but at the seams).  Narrow passes (NV 1 or 2) run fewer GEMM2 tiles, but
  // measured they take nearly the time of full ones (a split weighted by MFMA count was slower).
  if (!build_even_sched(a.NB, (a.M + rows_per_block - 1) / rows_per_block,
                        [&](int b) { return (dim_inputs[b] + kMlpJ - 1) / kMlpJ; }, &sc, &per_xcd))
    return fail(PMSST_EINVAL, "mask_mlp_forward: too many bands or rows for the block schedule");
  const dim3 grid(per_xcd * kXcds);
  const T* xp = static_cast<const T*>(x);
  const T* w1p = static_cast<const T*>(w1);
  const T* b1p = static_cast<const T*>(b1);
  const T* w2p = static_cast<const T*>(w2);
  const T* b2p = static_cast<const T*>(b2);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(64 * WV), 0, stream, xp, w1p, b1p, w2p, b2p, static_cast<T*>(pre),
                       static_cast<T*>(out), static_cast<T*>(hid), ar, sc);
  };
  if (a.ap.est != nullptr) {
    if (hid != nullptr) go(mlp_fwd_kernel<T, DK, NT, WV, true, true>);
    else go(mlp_fwd_kernel<T, DK, NT, WV, false, true>);
  } else {
    if (hid != nullptr) go(mlp_fwd_kernel<T, DK, NT, WV, true, false>);
    else go(mlp_fwd_kernel<T, DK, NT, WV, false, false>);
  }
  return check_launch("mlp_fwd_kernel");
}

template <typename T>
int launch_mlp_fwd(const void* x, const void* w1, const void* b1, const void* w2, const void* b2, void* pre,
                   void* out, void* hid, const MlpArgs& a, int64_t D, const int64_t* dim_inputs, hipStream_t stream) {
  switch (D) {
    case 64: return launch_dk<T, 2, 4>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    case 128: return launch_dk<T, 4, 4>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    // 8 waves of 32 rows: 254 VGPRs, two waves per SIMD (one block per CU, for its LDS), so one wave's
    // table lookups overlap the other's MFMAs (4 waves of 64 rows: 111 -> 97 us at configs[1])
    case 192: return launch_dk<T, 6, 2, 8>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    case 256: return launch_dk<T, 8, 4>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    case 384: return launch_dk<T, 12, 2>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    case 512: return launch_dk<T, 16, 2>(x, w1, b1, w2, b2, pre, out, hid, a, dim_inputs, stream);
    default: return fail(PMSST_EINVAL, "mask_mlp_forward: dim %lld not supported", static_cast<long long>(D));
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace pmsst

using namespace pmsst;

namespace pmsst {

int mask_mlp_forward_impl(const char* op, const void* x, const void* w1, const void* b1, const void* w2,
                          const void* b2, const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                          int64_t rows, int64_t dim, int64_t hidden, void* pre, void* out, void* hidden_out,
                          const MlpApply& ap, int dtype, void* stream) {
  PMSST_REQUIRE(pmsst_mask_mlp_supported(dim, hidden, dim_inputs, band_count, dtype) == 1,
                "%s: unsupported shape or dtype (dim %lld, hidden %lld, dtype %d)", op, (long long)dim,
                (long long)hidden, dtype);
  PMSST_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), "%s: bad row count", op);
  PMSST_REQUIRE(dim_offsets != nullptr, "%s: dim_offsets is null", op);
  if (rows == 0) return PMSST_OK;
  PMSST_REQUIRE(x && w1 && b1 && w2 && b2 && pre, "%s: null tensor", op);
  PMSST_REQUIRE(aligned16(x) && aligned16(w1) && aligned16(w2) && aligned16(hidden_out),
                "%s: x, w1, w2 and hidden must be 16-byte aligned", op);
  PMSST_REQUIRE(reinterpret_cast<uintptr_t>(b2) % 8 == 0 && reinterpret_cast<uintptr_t>(pre) % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(out) % 8 == 0,
                "%s: b2, pre and out must be 8-byte aligned", op);
  int64_t total = 0;
  for (int64_t b = 0; b < band_count; ++b) total += dim_inputs[b];
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* tabs = nullptr;
  const int rc = tanh_tables(s, &tabs);
  if (rc != PMSST_OK) return rc;
  MlpArgs a{dim_offsets, tabs + (dtype == PMSST_BF16 ? 0 : kTanhEntries), rows, static_cast<int>(band_count),
            static_cast<int>(hidden), static_cast<int>(total), ap};
  if (dtype == PMSST_BF16) return launch_mlp_fwd<bf16>(x, w1, b1, w2, b2, pre, out, hidden_out, a, dim, dim_inputs, s);
  return launch_mlp_fwd<f16>(x, w1, b1, w2, b2, pre, out, hidden_out, a, dim, dim_inputs, s);
}

}  // namespace pmsst

extern "C" {

int pmsst_mask_mlp_supported(int64_t dim, int64_t hidden, const int64_t* dim_inputs, int64_t band_count,
                             int dtype) {
  if (dtype != PMSST_BF16 && dtype != PMSST_F16) return 0;
  if (dim != 64 && dim != 128 && dim != 192 && dim != 256 && dim != 384 && dim != 512) return 0;
  if (hidden < 64 || hidden > kMlpMaxH || hidden % 32 != 0) return 0;
  if (dim_inputs == nullptr || band_count <= 0 || band_count > kSchedMaxBands) return 0;
  int64_t total = 0;
  for (int64_t b = 0; b < band_count; ++b) {
    if (dim_inputs[b] <= 0 || dim_inputs[b] % 4 != 0) return 0;
    total += dim_inputs[b];
    // W2 byte offsets of a band are 32-bit
    if (2 * dim_inputs[b] * hidden * 2 >= (int64_t{1} << 31)) return 0;
  }
  return total < (int64_t{1} << 29) ? 1 : 0;
}

int pmsst_mask_mlp_tanh_table(int dtype, uint16_t* out, int64_t entries) {
  if ((dtype != PMSST_BF16 && dtype != PMSST_F16) || out == nullptr || entries != kTanhEntries)
    return fail(PMSST_EINVAL, "mask_mlp_tanh_table: dtype must be bf16 or fp16 and entries %d", kTanhEntries);
  std::call_once(g_tanh_built, build_tanh_host);
  std::memcpy(out, g_tanh_host + (dtype == PMSST_BF16 ? 0 : kTanhEntries), sizeof(uint16_t) * kTanhEntries);
  return PMSST_OK;
}

int pmsst_mask_mlp_forward(const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                           const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count, int64_t rows,
                           int64_t dim, int64_t hidden, void* pre, void* out, void* hidden_out, int dtype,
                           void* stream) {
  PMSST_REQUIRE(out != nullptr || rows == 0, "mask_mlp_forward: null tensor");
  return pmsst::mask_mlp_forward_impl("mask_mlp_forward", x, w1, b1, w2, b2, dim_offsets, dim_inputs, band_count, rows,
                                      dim, hidden, pre, out, hidden_out, pmsst::MlpApply{}, dtype, stream);
}

int pmsst_mask_mlp_forward_apply(const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                                 const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                 int64_t rows, int64_t dim, int64_t hidden, void* pre, void* hidden_out,
                                 const void* spec, void* est, int64_t frames, int64_t channels, int64_t stems,
                                 int64_t stem, int zero_dc, int dtype, void* stream) {
  const char* op = "mask_mlp_forward_apply";
  PMSST_REQUIRE(frames > 0 && frames < (int64_t{1} << 31) && rows % frames == 0, "%s: rows must be batch * frames",
                op);
  PMSST_REQUIRE(channels > 0 && channels < 64 && stems > 0 && stem >= 0 && stem < stems && stems < (1 << 16),
                "%s: bad channels / stems / stem", op);
  PMSST_REQUIRE(dim_inputs != nullptr && band_count > 0, "%s: no bands", op);
  int64_t total = 0;
  for (int64_t b = 0; b < band_count; ++b) total += dim_inputs[b];
  PMSST_REQUIRE(total % (2 * channels) == 0, "%s: features must be 2 * channels * bins", op);
  const int64_t fbins = total / (2 * channels);
  PMSST_REQUIRE(rows == 0 || (spec && est), "%s: null spectrum or estimate", op);
  PMSST_REQUIRE(reinterpret_cast<uintptr_t>(spec) % 8 == 0 && reinterpret_cast<uintptr_t>(est) % 8 == 0,
                "%s: spectrum and estimate must be 8-byte aligned", op);
  PMSST_REQUIRE((rows / frames) * stems * channels * fbins * frames < (int64_t{1} << 40), "%s: estimate too large", op);
  const pmsst::MlpApply ap{static_cast<const float2*>(spec), static_cast<float2*>(est),
                           pmsst::FastDiv(static_cast<uint32_t>(frames)), static_cast<int>(channels),
                           static_cast<int>(fbins), static_cast<int>(stems), static_cast<int>(stem), zero_dc != 0};
  return pmsst::mask_mlp_forward_impl(op, x, w1, b1, w2, b2, dim_offsets, dim_inputs, band_count, rows, dim, hidden,
                                      pre, nullptr, hidden_out, ap, dtype, stream);
}

}  // extern "C"
