// Building blocks of the DMA-pipelined MFMA kernels (global -> LDS DMA ring).
//
// A block keeps S - 1 K chunks of both operands in flight by moving them with
// global_load_lds_dwordx4 (16 bytes per lane straight into LDS at M0 + 16 * lane, no
// staging registers) into a ring of S LDS stages, one barrier per chunk.  The LDS reads
// are inline ds_read instructions followed by an explicit lgkmcnt wait that the MFMA
// operands depend on, and the DMA completion wait (vmcnt) is explicit too: the compiler
// cannot tell the ring's stages apart and would otherwise wait for every DMA in flight
// before each LDS read.
//
// Operand tiles in a stage (one 32-wide K chunk, 16-bit elements):
//  * K-contiguous ("row") tile: ROWS rows x 32 K, 64 bytes per row.  The four 16-byte
//    units of row r sit XOR-swizzled by swz_k(r % 16); an MFMA fragment (16 rows x one
//    unit) is one ds_read_b128 per lane.
//  * MN-contiguous ("k-major") tile: 32 K-rows x COLS, 2 COLS bytes per K-row as in HBM.
//    Units of K-row k sit XOR-swizzled by swz_mn(k); a fragment is two
//    ds_read_b64_tr_b16 (gfx950 transpose read: in each 16-lane group, lane i receives
//    element i % 4 of the 4 elements lane 4 k + i / 4 addressed, k = 0..3), which hand
//    lane i of the group the 4 K values of column c0 + i.
// On gfx950 the swizzled fragment reads of K-contiguous tiles still take 4 LDS bank-conflict
// cycles per ds_read_b128 (SQ_LDS_BANK_CONFLICT on a probe kernel; contiguous 16-byte reads take
// none); the transpose reads at a 512-byte pitch take 2 with swz_mn.
#pragma once

#include <type_traits>

#include "gemm.h"

namespace pmsst {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int swz_k(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
__device__ __forceinline__ int swz_mn(int k) { return 2 * (k & 3); }
// swz_mn for a 512-byte K-row pitch: a transpose read covers K-rows 8 g + 0..3 (g = 0..3), which
// start on the same bank at this pitch; spreading them over 16 unit pairs makes the read
// conflict-free (0 conflict cycles against 2 for swz_mn, measured on a probe kernel).  Rows k
// and k + 4 keep the same swizzle, as the second read of a fragment needs.
template <int PITCH>
__device__ __forceinline__ int swz_mn_p(int k) {
  if constexpr (PITCH == 512) return 2 * ((k & 3) | (((k >> 3) & 3) << 2));
  else return swz_mn(k);
}

template <typename T>
__device__ __forceinline__ f32x4_t mfma_raw(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (std::is_same<T, bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// LDS byte address (inside the block's allocation) of __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Fragment of a K-contiguous tile: rows r0 .. r0 + 15 (r0 % 16 == 0), this lane's K unit.
__device__ __forceinline__ uint32_t frag_k_addr(uint32_t region, int r0, int lane) {
  const int rr = lane & 15, g = lane >> 4;
  return region + static_cast<uint32_t>((r0 + rr) * 64 + 16 * (g ^ swz_k(rr)));
}

// First of the two transpose reads of an MN-contiguous fragment (columns c0 .. c0 + 15,
// c0 % 16 == 0, row pitch `pitch` bytes); the second is at + 4 * pitch.
__device__ __forceinline__ uint32_t frag_mn_addr(uint32_t region, int c0, int pitch, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const int k = 8 * g + (j >> 2);                // K-row of this lane's 4 elements
  const int col = c0 + 4 * (j & 3);
  const int unit = col >> 3;
  return region + static_cast<uint32_t>(k * pitch + 16 * (unit ^ swz_mn(k)) + 2 * (col & 7));
}

template <int PITCH>
__device__ __forceinline__ uint32_t frag_mn_addr_p(uint32_t region, int c0, int lane) {
  const int j = lane & 15, g = lane >> 4;
  const int k = 8 * g + (j >> 2);
  const int col = c0 + 4 * (j & 3);
  const int unit = col >> 3;
  return region + static_cast<uint32_t>(k * PITCH + 16 * (unit ^ swz_mn_p<PITCH>(k)) + 2 * (col & 7));
}

__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t addr) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

__device__ __forceinline__ void lds_write_b128(uint32_t addr, const u32x4_t& v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

__device__ __forceinline__ float lds_read_f32(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// ds_read_b64_tr_b16 at addr and addr + step (the two K halves of an MN fragment).
__device__ __forceinline__ u32x4_t lds_read_tr_pair(uint32_t addr, uint32_t step) {
  u32x2_t lo, hi;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(lo) : "v"(addr));
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(hi) : "v"(addr + step));
  return u32x4_t{lo.x, lo.y, hi.x, hi.y};
}

// Waits for this wave's LDS reads; the fragments are tied to the wait so no use of them
// is scheduled above it.
template <int NA, int NB>
__device__ __forceinline__ void lds_wait(u32x4_t (&a)[NA], u32x4_t (&b)[NB]) {
  static_assert(NA + NB <= 12, "operand count");
  if constexpr (NA == 4 && NB == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]));
  else if constexpr (NA == 4 && NB == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
  else if constexpr (NA == 2 && NB == 4)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
  else if constexpr (NA == 2 && NB == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]));
  else
    static_assert(NA < 0, "add the operand list for this shape");
}

// One 16-byte-per-lane global -> LDS DMA (to lds + 16 * lane).  Kernel templates with a non-type
// parameter call it instead of the builtin: hipcc (ROCm 7.2) drops the host launch stub of such a
// kernel template when its body calls __builtin_amdgcn_global_load_lds directly.
__device__ __forceinline__ void dma_lds16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---------------------------------------------------------------- block schedule
// Blocks in canonical order (band, row tile, unit-local index) cut into kXcds contiguous
// ranges of whole (band, row tile) units, balanced by cost; range x runs on XCD x
// (the hardware places block i on XCD i % 8).  Blocks that read the same rows or the same
// weights then share one L2.
constexpr int kSchedMaxBands = 256;
struct BandSched {
  uint32_t gs[kXcds + 1];             // canonical block range [gs[x], gs[x+1]) of XCD x
  uint32_t cumb[kSchedMaxBands + 1];  // canonical index of each band's first block
  uint32_t bstart[kXcds];             // band of XCD x's first block
  uint32_t m_tiles;                   // row tiles; 0: no schedule
};

// Decodes this block: band, row tile, and index inside the (band, row tile) unit.  With
// LAST_FIRST an XCD dispatches its range from the end (in canonical order the costly wide
// bands come last, and starting them first keeps them out of the tail).
// sched_block_at decodes block `blk` of the schedule: a kernel whose scheduled blocks start at a
// multiple of kXcds past its own first block passes blockIdx.x minus that offset (the XCD stays
// blk % kXcds).
template <bool LAST_FIRST = false>
__device__ __forceinline__ bool sched_block_at(const BandSched& sc, uint32_t blk, int& band, uint32_t& mt,
                                               uint32_t& sub, uint32_t& per_unit) {
  const uint32_t xcd = blk % kXcds;
  const uint32_t local = blk / kXcds;
  if (sc.gs[xcd] + local >= sc.gs[xcd + 1]) return false;
  const uint32_t gb = LAST_FIRST ? sc.gs[xcd + 1] - 1 - local : sc.gs[xcd] + local;
  uint32_t b = sc.bstart[xcd];
  while (gb >= sc.cumb[b + 1]) ++b;
  per_unit = (sc.cumb[b + 1] - sc.cumb[b]) / sc.m_tiles;
  const uint32_t within = gb - sc.cumb[b];
  band = static_cast<int>(b);
  mt = within / per_unit;
  sub = within % per_unit;
  return true;
}

template <bool LAST_FIRST = false>
__device__ __forceinline__ bool sched_block(const BandSched& sc, int& band, uint32_t& mt, uint32_t& sub,
                                            uint32_t& per_unit) {
  return sched_block_at<LAST_FIRST>(sc, blockIdx.x, band, mt, sub, per_unit);
}

// Host: schedule for per-band unit sizes units(b) (blocks per (band, row tile)) and per-block
// costs cost(b) (e.g. K steps); the XCD ranges are balanced by total cost.  Returns false
// (and leaves m_tiles = 0) when the band count exceeds the table.
template <class UnitsOf, class CostOf>
inline bool build_band_sched(int NB, int64_t m_tiles, UnitsOf units, CostOf cost, BandSched* sc,
                             uint32_t* per_xcd) {
  sc->m_tiles = 0;
  if (NB > kSchedMaxBands || m_tiles <= 0) return false;
  int64_t total = 0, total_cost = 0, unit_cost_max = 0;
  sc->cumb[0] = 0;
  for (int b = 0; b < NB; ++b) {
    const int64_t u = units(b), uc = u * cost(b);
    unit_cost_max = uc > unit_cost_max ? uc : unit_cost_max;
    total += u * m_tiles;
    total_cost += uc * m_tiles;
    if (total >= (int64_t{1} << 31)) return false;
    sc->cumb[b + 1] = static_cast<uint32_t>(total);
  }
  // greedy fill of whole (band, row tile) units up to a cost cap; the smallest cap that needs
  // at most kXcds ranges is found by bisection
  auto ranges = [&](int64_t cap, bool fill) {
    int x = 0;
    int64_t acc = 0, g = 0;
    if (fill) {
      sc->gs[0] = 0;
      sc->bstart[0] = 0;
    }
    for (int b = 0; b < NB; ++b) {
      const int64_t ch = (sc->cumb[b + 1] - sc->cumb[b]) / m_tiles;
      const int64_t uc = ch * cost(b);
      for (int64_t t = 0; t < m_tiles; ++t, g += ch) {
        if (acc + uc > cap) {
          ++x;
          acc = 0;
          if (fill && x < static_cast<int>(kXcds)) {
            sc->gs[x] = static_cast<uint32_t>(g);
            sc->bstart[x] = static_cast<uint32_t>(b);
          }
        }
        acc += uc;
      }
    }
    if (fill)
      for (int y = x + 1; y <= static_cast<int>(kXcds); ++y) {
        sc->gs[y] = static_cast<uint32_t>(total);
        if (y < static_cast<int>(kXcds)) sc->bstart[y] = static_cast<uint32_t>(NB - 1);
      }
    return x + 1;
  };
  int64_t lo = unit_cost_max, hi = total_cost > unit_cost_max ? total_cost : unit_cost_max;
  while (lo < hi) {
    const int64_t mid = (lo + hi) / 2;
    if (ranges(mid, false) <= static_cast<int>(kXcds)) hi = mid;
    else lo = mid + 1;
  }
  ranges(lo, true);
  uint32_t mx = 0;
  for (uint32_t y = 0; y < kXcds; ++y) mx = sc->gs[y + 1] - sc->gs[y] > mx ? sc->gs[y + 1] - sc->gs[y] : mx;
  sc->m_tiles = static_cast<uint32_t>(m_tiles);
  *per_xcd = mx;
  return true;
}

// Equal-cost blocks split evenly: XCD x takes canonical blocks [x total / 8, (x + 1) total / 8), so a
// (band, row tile) unit may straddle two XCDs.  For kernels whose blocks all cost about the same,
// where whole-unit ranges would leave some XCDs with a round of blocks more than others.
template <class UnitsOf>
inline bool build_even_sched(int NB, int64_t m_tiles, UnitsOf units, BandSched* sc, uint32_t* per_xcd) {
  sc->m_tiles = 0;
  if (NB > kSchedMaxBands || m_tiles <= 0) return false;
  int64_t total = 0;
  sc->cumb[0] = 0;
  for (int b = 0; b < NB; ++b) {
    total += units(b) * m_tiles;
    if (total >= (int64_t{1} << 31)) return false;
    sc->cumb[b + 1] = static_cast<uint32_t>(total);
  }
  uint32_t mx = 0;
  int b = 0;
  for (uint32_t x = 0; x <= kXcds; ++x) {
    sc->gs[x] = static_cast<uint32_t>(total * x / kXcds);
    if (x < kXcds) {
      while (b < NB - 1 && sc->cumb[b + 1] <= sc->gs[x]) ++b;
      sc->bstart[x] = static_cast<uint32_t>(b);
    }
    if (x > 0) mx = sc->gs[x] - sc->gs[x - 1] > mx ? sc->gs[x] - sc->gs[x - 1] : mx;
  }
  sc->m_tiles = static_cast<uint32_t>(m_tiles);
  *per_xcd = mx;
  return true;
}

// Equal-cost blocks.
template <class UnitsOf>
inline bool build_band_sched(int NB, int64_t m_tiles, UnitsOf units, BandSched* sc, uint32_t* per_xcd) {
  return build_band_sched(NB, m_tiles, units, [](int) { return int64_t{1}; }, sc, per_xcd);
}

}  // namespace pmsst
