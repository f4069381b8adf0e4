// Pipelined MFMA main loop for the ragged per-band GEMMs.
//
// A block computes C[BR x BC] += A[BR x K] * B[BC x K]^T with both operands
// staged in LDS as [rows][pitch] (K contiguous) in chunks of 32.  Two LDS
// buffers and one or two register copies keep the global loads of the next one
// or two chunks in flight during the MFMAs of chunk k; one barrier per chunk.
//
// LDS layout (16-bit types): row r, element k of a chunk lives at
//   r * pitch + 8 * ((k / 8) ^ ((r / 16) % 4)) + k % 8,
// i.e. the four 16-byte k-units of a row are XOR-swizzled by the row's 16-row
// group.  MFMA fragment reads (16 consecutive rows, one unit) stay 16-byte
// aligned and conflict-free, and the transposed stores of MNLoader (8 bytes to
// rows 4q..4q+3) spread over all banks.  fp32 tiles use a plain odd pitch.
//
// Waves are laid out WR x WC over the tile; wave (wr, wc) owns rows
// [wr * BR/WR, ...) and columns [wc * BC/WC, ...) as TR x TC 16x16 tiles.
// Result layout (mfma.h): lane l of tile (i, j) holds
//   C[row0 + 16 i + 4 (l / 16) + r][col0 + 16 j + (l % 16)],  r = 0..3.
//
// Loaders move one 32-wide K chunk:  fetch(k0, regs) global -> registers,
// commit(regs, lds) registers -> LDS.  Out-of-range rows and k read as zero.
#pragma once

#include <type_traits>

#include "mfma.h"

namespace pmsst {

constexpr int kGemmThreads = 256;

template <typename T>
__device__ __forceinline__ int lds_index(int r, int k) {
  constexpr int P = LdsPitch<T>::value;
  if constexpr (sizeof(T) == 2) {
    return r * P + ((((k >> 3) ^ ((r >> 4) & 3)) << 3) | (k & 7));
  } else {
    return r * P + k;
  }
}

// acc += A rows (ra..) x B rows (rb..) over one 32-wide chunk; `ra` / `rb` are the
// lane's row indices inside the A / B tiles.
template <typename T>
__device__ __forceinline__ f32x4_t mfma_tile(const T* __restrict__ a, int ra, const T* __restrict__ b, int rb,
                                             f32x4_t acc, int lane) {
  if constexpr (sizeof(T) == 2) {
    const int k = (lane >> 4) * 8;
    return mfma_chunk<T>(a + lds_index<T>(ra, k) - k, b + lds_index<T>(rb, k) - k, acc, lane);
  } else {
    return mfma_chunk<T>(a + ra * LdsPitch<T>::value, b + rb * LdsPitch<T>::value, acc, lane);
  }
}

// ---------------------------------------------------------------- guarded loads
// Loads never branch on bounds, and nothing consumes a loaded value until commit():
// an out-of-range lane reads the tile origin (always a valid element) and records a
// validity bit; commit() masks the value to zero.  fetch() therefore issues all of
// its loads back to back and the MFMAs of the current chunk run while they are in
// flight.  When a loader's `vec4` flag is set, every k / mn extent it is given is a
// multiple of 4 (the launchers only set it then), so a quad is either fully in
// range or fully out; without it (unaligned shapes) the loader falls back to
// per-element loads that are masked at once.

template <typename T>
using raw_t = typename std::conditional<sizeof(T) == 2, uint16_t, uint32_t>::type;
// 4 consecutive elements as raw bits: 8 bytes for 16-bit types, 16 for fp32.
template <typename T>
using quad_t = typename std::conditional<sizeof(T) == 2, uint2, uint4>::type;

template <typename T>
__device__ __forceinline__ quad_t<T> raw_quad(const T* p) {
  return *reinterpret_cast<const quad_t<T>*>(p);
}

template <typename T>
__device__ __forceinline__ quad_t<T> mask_quad(quad_t<T> q, bool ok) {
  q.x = ok ? q.x : 0u;
  q.y = ok ? q.y : 0u;
  if constexpr (sizeof(T) == 4) {
    q.z = ok ? q.z : 0u;
    q.w = ok ? q.w : 0u;
  }
  return q;
}

// Unaligned fallback: element j is loaded when `ok && j < valid`, masked at once.
template <typename T>
__device__ __forceinline__ quad_t<T> load_quad_scalar(const T* p, const T* safe, bool ok, int valid) {
  uint32_t e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = ok && j < valid;
    const raw_t<T> v = *reinterpret_cast<const raw_t<T>*>(in ? p + j : safe);
    e[j] = in ? static_cast<uint32_t>(v) : 0u;
  }
  quad_t<T> q;
  if constexpr (sizeof(T) == 2) {
    q.x = e[0] | (e[1] << 16);
    q.y = e[2] | (e[3] << 16);
  } else {
    q.x = e[0];
    q.y = e[1];
    q.z = e[2];
    q.w = e[3];
  }
  return q;
}

// One quad: raw load (vec4) recording validity, or the masked scalar fallback.
template <typename T>
__device__ __forceinline__ quad_t<T> fetch_quad(const T* p, const T* safe, bool vec4, bool row_ok, int k_left,
                                                uint32_t& okbits, int bit) {
  if (vec4) {
    const bool ok = row_ok && k_left > 0;
    okbits |= static_cast<uint32_t>(ok) << bit;
    return raw_quad<T>(ok ? p : safe);
  }
  okbits |= 1u << bit;
  return load_quad_scalar<T>(p, safe, row_ok, k_left);
}

template <typename T>
__device__ __forceinline__ void quad_to_f32(const quad_t<T>& q, float (&o)[4]) {
  if constexpr (sizeof(T) == 2) {
    const Pack<T, 4> pk = __builtin_bit_cast(Pack<T, 4>, q);
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = to_f32(pk.v[j]);
  } else {
    o[0] = __uint_as_float(q.x);
    o[1] = __uint_as_float(q.y);
    o[2] = __uint_as_float(q.z);
    o[3] = __uint_as_float(q.w);
  }
}

// Stores a quad of consecutive k (kq % 4 == 0) of LDS row r.
template <typename T>
__device__ __forceinline__ void commit_quad(T* lds, int r, int kq, const quad_t<T>& q) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint2*>(lds + lds_index<T>(r, kq)) = q;
  } else {
    uint32_t* row = reinterpret_cast<uint32_t*>(lds);
    row[lds_index<T>(r, kq + 0)] = q.x;
    row[lds_index<T>(r, kq + 1)] = q.y;
    row[lds_index<T>(r, kq + 2)] = q.z;
    row[lds_index<T>(r, kq + 3)] = q.w;
  }
}

// K-contiguous rows: element (r, k) = base[r * stride + k].  Thread t moves the quad
// (r, k) = (t / 8 + 32 i, 4 (t % 8)) of every chunk, i < ROWS / 32.
template <typename T, int ROWS>
struct KRowLoader {
  static constexpr int kQuads = ROWS * (kChunkK / 4) / kGemmThreads;
  static_assert(kQuads >= 1 && ROWS * (kChunkK / 4) % kGemmThreads == 0, "tile too small");
  struct Regs {
    quad_t<T> q[kQuads];
    uint32_t ok;
  };
  const T* base;
  int64_t stride;
  int rows_valid;
  int k_valid;
  bool vec4;

  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    const int k = k0 + (threadIdx.x % (kChunkK / 4)) * 4;
    g.ok = 0;
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      const int r = (threadIdx.x + i * kGemmThreads) / (kChunkK / 4);
      g.q[i] = fetch_quad<T>(base + r * stride + k, base, vec4, r < rows_valid, k_valid - k, g.ok, i);
    }
  }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
    const int kq = (threadIdx.x % (kChunkK / 4)) * 4;
#pragma unroll
    for (int i = 0; i < kQuads; ++i)
      commit_quad<T>(lds, (threadIdx.x + i * kGemmThreads) / (kChunkK / 4), kq, mask_quad<T>(g.q[i], (g.ok >> i) & 1));
  }
};

// MN-contiguous source: element (k, mn) = base[k * kstride + mn], staged
// transposed into lds[mn][k].  A thread owns a block of KB consecutive k rows x 4
// consecutive mn (consecutive threads take consecutive mn quads, so each global
// load is coalesced along mn), transposes it in registers and stores KB
// consecutive k values per mn row.  KB = ROWS / 32 so one block per thread
// covers the chunk.  Optional scales: per-mn `cs[mn]`, per-k
// `rs[k * rs_stride] * rs_mul` (both global and cache-resident).
template <typename T, int ROWS>
struct MNLoader {
  static constexpr int kQuadsPerK = ROWS / 4;
  static constexpr int KB = ROWS / 32;
  static_assert(KB >= 1 && KB * kQuadsPerK * (kChunkK / KB) == ROWS * kChunkK / 4, "tile shape");
  static_assert(kQuadsPerK * (kChunkK / KB) == kGemmThreads, "one block per thread");
  struct Regs {
    quad_t<T> q[KB];
    float s[KB];
    uint32_t ok;
  };
  const T* base;
  int64_t kstride;
  int mn_valid;
  int k_valid;
  bool vec4;
  const T* cs = nullptr;        // per-mn scale, or null
  const float* rs = nullptr;    // per-k scale, or null
  int64_t rs_stride = 1;
  float rs_mul = 1.f;
  // per-mn scale of this thread's quad (loaded once; cs does not depend on k)
  float c[4] = {1.f, 1.f, 1.f, 1.f};
  // with `colsum` set, commit() also accumulates the unscaled values of the thread's mn
  // quad over its k rows (column sums over K, e.g. a bias gradient); see reduce_colsum()
  bool colsum = false;
  mutable float csum[4] = {0.f, 0.f, 0.f, 0.f};

  __device__ __forceinline__ void init() {
    if (cs != nullptr) {
      const int mn = (threadIdx.x % kQuadsPerK) * 4;
      quad_to_f32<T>(load_quad_scalar<T>(cs + mn, cs, true, mn_valid - mn), c);
    }
  }
  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    const int mn = (threadIdx.x % kQuadsPerK) * 4;
    const int kb = (threadIdx.x / kQuadsPerK) * KB;
    g.ok = 0;
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int k = k0 + kb + t;
      g.q[t] = fetch_quad<T>(base + static_cast<int64_t>(k) * kstride + mn, base, vec4, k < k_valid, mn_valid - mn,
                             g.ok, t);
      g.s[t] = rs != nullptr ? rs[static_cast<int64_t>(k < k_valid ? k : 0) * rs_stride] : 1.f;
    }
  }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
    const int mn = (threadIdx.x % kQuadsPerK) * 4;
    const int kb = (threadIdx.x / kQuadsPerK) * KB;
    float v[KB][4];
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      quad_to_f32<T>(mask_quad<T>(g.q[t], (g.ok >> t) & 1), v[t]);
      if (colsum) {
#pragma unroll
        for (int j = 0; j < 4; ++j) csum[j] += v[t][j];
      }
      const float st = rs != nullptr ? g.s[t] * rs_mul : 1.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[t][j] *= st * c[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(T) == 2) {
        float col[KB];
#pragma unroll
        for (int t = 0; t < KB; ++t) col[t] = v[t][j];
        store_pack<T, KB>(lds + lds_index<T>(mn + j, kb), col);
      } else {
#pragma unroll
        for (int t = 0; t < KB; ++t) lds[lds_index<T>(mn + j, kb + t)] = v[t][j];
      }
    }
  }
};

// Column sums gathered by a `colsum` MNLoader: the 256 threads hold partial sums of
// 4 consecutive mn each (thread t: mn = 4 (t % ROWS/4)); they are combined in a fixed
// order through LDS and written as dst[mn] for mn < mn_valid.  Call after the main loop
// (which ends with a barrier), with every thread of the block.
template <typename T, int ROWS>
__device__ __forceinline__ void reduce_colsum(const MNLoader<T, ROWS>& ld, T* lds, T* __restrict__ dst) {
  constexpr int kQ = ROWS / 4;                  // mn quads
  constexpr int kGroups = kGemmThreads / kQ;    // threads per quad
  float* red = reinterpret_cast<float*>(lds);   // [kGroups][ROWS]
  const int q = threadIdx.x % kQ, grp = threadIdx.x / kQ;
#pragma unroll
  for (int j = 0; j < 4; ++j) red[grp * ROWS + 4 * q + j] = ld.csum[j];
  __syncthreads();
  if (threadIdx.x < ROWS && static_cast<int>(threadIdx.x) < ld.mn_valid) {
    float s = 0.f;
#pragma unroll 4
    for (int g2 = 0; g2 < kGroups; ++g2) s += red[g2 * ROWS + threadIdx.x];
    dst[threadIdx.x] = from_f32<T>(s);
  }
}

// ---------------------------------------------------------------- XCD-aware block order
// MI355X has 8 XCDs (32 CUs and one L2 each); the hardware dispatches 1-D block b to
// XCD b % 8.  Kernels whose blocks fall into groups that read the same operand tile
// (e.g. the m-tiles of one band's weight chunk) number their blocks so that all
// `members` blocks of a group land on one XCD and are dispatched close together:
//   block b -> group (b / 8 / members) * 8 + b % 8, member (b / 8) % members.
// The grid is padded to whole groups of 8; padding blocks exit at once.
constexpr uint32_t kXcds = 8;

struct XcdGrid {
  uint32_t groups;
  uint32_t members;
  uint32_t blocks() const { return ((groups + kXcds - 1) / kXcds) * kXcds * members; }
};

__device__ __forceinline__ bool xcd_block(const XcdGrid& xg, uint32_t& group, uint32_t& member) {
  const uint32_t b = blockIdx.x;
  const uint32_t r = b / kXcds;
  member = r % xg.members;
  group = (r / xg.members) * kXcds + b % kXcds;
  return group < xg.groups;
}

template <int BR, int BC, int WR, int WC>
struct TileShape {
  static constexpr int kTR = BR / WR / 16;
  static constexpr int kTC = BC / WC / 16;
  static_assert(WR * WC == kGemmThreads / kWave, "4 waves per block");
  static_assert(kTR >= 1 && kTC >= 1 && BR % (WR * 16) == 0 && BC % (WC * 16) == 0, "bad tile");
};

// LDS elements the main loop needs for a BR x BC tile (two buffers).
template <typename T, int BR, int BC>
constexpr int gemm_lds_elems() {
  return 2 * (BR + BC) * LdsPitch<T>::value;
}

// Runs the K loop; `acc` is accumulated (callers zero it).
//
// DEPTH = 1: chunk c + 1 is fetched into registers while chunk c is multiplied and
// committed to the other LDS buffer afterwards.  DEPTH = 2: chunk c is fetched into
// register set R[c % 2] two iterations ahead, so two chunks of global loads are in
// flight during the MFMAs of a third, at the cost of a second register set (the
// loop is unrolled by two so the sets stay fixed registers).  Buffer offsets are
// computed from the __shared__ base (no pointer tables), so every LDS access stays
// a ds_* instruction and waits only on the LDS counter.
template <typename T, int BR, int BC, int WR, int WC, int DEPTH = 1, class LA, class LB>
__device__ __forceinline__ void gemm_mainloop(const LA& la, const LB& lb, int K, T* lds,
                                              f32x4_t (&acc)[TileShape<BR, BC, WR, WC>::kTR]
                                                            [TileShape<BR, BC, WR, WC>::kTC]) {
  static_assert(DEPTH == 1 || DEPTH == 2, "prefetch depth 1 or 2");
  using S = TileShape<BR, BC, WR, WC>;
  constexpr int P = LdsPitch<T>::value;
  constexpr int kBuf = (BR + BC) * P;  // elements of one (A, B) buffer pair
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r0 = (wave / WC) * (BR / WR);
  const int c0 = (wave % WC) * (BC / WC);
  const int nk = (K + kChunkK - 1) / kChunkK;
  if (nk == 0) return;

  // The scheduler would otherwise hoist the LDS commit of the next chunk (independent
  // addresses) above the MFMAs, making them wait for the in-flight loads it commits.
  auto mma = [&](int cur) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < S::kTR; ++i) {
#pragma unroll
      for (int j = 0; j < S::kTC; ++j) {
        acc[i][j] = mfma_tile<T>(lds + cur, r0 + i * 16 + (lane & 15), lds + cur + BR * P, c0 + j * 16 + (lane & 15),
                                 acc[i][j], lane);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  typename LA::Regs ra0;
  typename LB::Regs rb0;
  la.fetch(0, ra0);
  lb.fetch(0, rb0);
  // The steady-state loops below fetch unconditionally: with every trip issuing the
  // same loads into the same registers, the wait-count analysis can see that a
  // register set's previous loads retired before it is refilled, and no conditional
  // path splits the accumulators' live ranges.
  if constexpr (DEPTH == 1) {
    la.commit(ra0, lds);
    lb.commit(rb0, lds + BR * P);
    __syncthreads();
    int kc = 0;
    for (; kc + 1 < nk; ++kc) {
      const int cur = (kc & 1) * kBuf;
      la.fetch((kc + 1) * kChunkK, ra0);
      lb.fetch((kc + 1) * kChunkK, rb0);
      mma(cur);
      la.commit(ra0, lds + kBuf - cur);
      lb.commit(rb0, lds + kBuf - cur + BR * P);
      __syncthreads();
    }
    mma((kc & 1) * kBuf);
    __syncthreads();
  } else {
    typename LA::Regs ra1;
    typename LB::Regs rb1;
    if (nk > 1) {
      la.fetch(kChunkK, ra1);
      lb.fetch(kChunkK, rb1);
    }
    la.commit(ra0, lds);
    lb.commit(rb0, lds + BR * P);
    __syncthreads();
    // Entering each trip: chunk kc is in LDS buffer (kc & 1) and its registers (set 0)
    // are free; chunk kc + 1 is in flight into set 1.
    int kc = 0;
    for (; kc + 3 < nk; kc += 2) {
      const int cur = (kc & 1) * kBuf;
      la.fetch((kc + 2) * kChunkK, ra0);
      lb.fetch((kc + 2) * kChunkK, rb0);
      mma(cur);
      la.commit(ra1, lds + kBuf - cur);
      lb.commit(rb1, lds + kBuf - cur + BR * P);
      __syncthreads();
      la.fetch((kc + 3) * kChunkK, ra1);
      lb.fetch((kc + 3) * kChunkK, rb1);
      mma(kBuf - cur);
      la.commit(ra0, lds + cur);
      lb.commit(rb0, lds + cur + BR * P);
      __syncthreads();
    }
    // 1 to 3 chunks left: kc (in LDS), kc + 1 (set 1, in flight), kc + 2 (not fetched)
    const int cur = (kc & 1) * kBuf;
    if (kc + 2 < nk) {
      la.fetch((kc + 2) * kChunkK, ra0);
      lb.fetch((kc + 2) * kChunkK, rb0);
      mma(cur);
      la.commit(ra1, lds + kBuf - cur);
      lb.commit(rb1, lds + kBuf - cur + BR * P);
      __syncthreads();
      mma(kBuf - cur);
      la.commit(ra0, lds + cur);
      lb.commit(rb0, lds + cur + BR * P);
      __syncthreads();
      mma(cur);
    } else if (kc + 1 < nk) {
      mma(cur);
      la.commit(ra1, lds + kBuf - cur);
      lb.commit(rb1, lds + kBuf - cur + BR * P);
      __syncthreads();
      mma(kBuf - cur);
    } else {
      mma(cur);
    }
    __syncthreads();
  }
}

}  // namespace pmsst
