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
// commit(regs, lds) registers -> LDS (fetch_edge / commit_edge for a partial chunk);
// prepare() runs once before the first chunk.
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

// ---------------------------------------------------------------- loads
// K is walked in chunks of 32 that END at K: chunk c covers k in [kbeg + 32 c, kbeg + 32 c + 32)
// with kbeg = K - 32 ceil(K / 32) <= 0, so only chunk 0 can be partial (k < 0 masked).
// Loaders therefore have two paths:
//  * interior chunks (fetch / commit): rows / columns outside the tile's valid range are
//    CLAMPED to a valid one when the loader is prepared (their products only reach outputs
//    the epilogue discards), every k is in range, and each load is a uniform chunk base plus a
//    per-lane 32-bit byte offset computed once -- no per-chunk address arithmetic or masking;
//  * the partial chunk 0 (fetch_edge / commit_edge): loads never branch on bounds (an
//    out-of-range lane reads a valid element and records a bit) and commit_edge zeroes them.
// With V4 false (widths or strides not multiples of 4 elements) every chunk takes the
// element-wise guarded path.

template <typename T>
using raw_t = typename std::conditional<sizeof(T) == 2, uint16_t, uint32_t>::type;
// 4 consecutive elements as raw bits: 8 bytes for 16-bit types, 16 for fp32.
template <typename T>
using quad_t = typename std::conditional<sizeof(T) == 2, uint2, uint4>::type;

template <typename T>
__device__ __forceinline__ quad_t<T> raw_quad(const T* p) {
  return *reinterpret_cast<const quad_t<T>*>(p);
}

// Quad at a uniform base plus a per-lane byte offset (global_load with an SGPR base).
template <typename T>
__device__ __forceinline__ quad_t<T> quad_at(const T* base, uint32_t byte_off) {
  return *reinterpret_cast<const quad_t<T>*>(reinterpret_cast<const char*>(base) + byte_off);
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

// Element-wise guarded quad: element j is loaded when `ok` and lo <= j < hi, else zero.
template <typename T>
__device__ __forceinline__ quad_t<T> load_quad_scalar(const T* p, const T* safe, bool ok, int lo, int hi) {
  uint32_t e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = ok && j >= lo && j < hi;
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

// Edge-path quad of elements k .. k+3 of a row (valid range [0, k_valid)): with V4 the quad is
// wholly in or out (raw load recording a validity bit, masked at commit); otherwise element-wise.
template <typename T, bool V4>
__device__ __forceinline__ quad_t<T> fetch_quad_k(const T* p, const T* safe, bool row_ok, int k, int k_valid,
                                                  uint32_t& okbits, int bit) {
  if constexpr (V4) {
    const bool ok = row_ok && k >= 0 && k < k_valid;
    okbits |= static_cast<uint32_t>(ok) << bit;
    return raw_quad<T>(ok ? p : safe);
  } else {
    okbits |= 1u << bit;
    return load_quad_scalar<T>(p, safe, row_ok, -k, k_valid - k);
  }
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

// K-contiguous rows: element (r, k) = base[row(r) * stride + k].  Thread t moves the quad
// (r, k) = (t / 8 + 32 i, 4 (t % 8)) of every chunk, i < ROWS / 32.  By default row(r) = r for
// r < rows_valid; prepare_rows() lets a kernel map tile rows to other source rows.
template <typename T, int ROWS, bool V4>
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
  int64_t src_row[kQuads] = {};  // source row of each of the thread's tile rows (clamped)
  uint32_t off[kQuads] = {};     // byte offset of (src_row, k = 4 (t % 8)) from base
  uint32_t rowok = 0;            // bit i: tile row i of this thread is a real row

  static __device__ __forceinline__ int tile_row(int i) {
    return (static_cast<int>(threadIdx.x) + i * kGemmThreads) / (kChunkK / 4);
  }
  static __device__ __forceinline__ int lane_k() { return (threadIdx.x % (kChunkK / 4)) * 4; }

  __device__ __forceinline__ void prepare() {
    rowok = 0;
#pragma unroll
    for (int i = 0; i < kQuads; ++i) {
      const int r = tile_row(i);
      src_row[i] = r < rows_valid ? r : rows_valid - 1;
      rowok |= static_cast<uint32_t>(r < rows_valid) << i;
    }
    finish_prepare();
  }
  // Call after filling src_row and rowok (custom row maps).
  __device__ __forceinline__ void finish_prepare() {
#pragma unroll
    for (int i = 0; i < kQuads; ++i)
      off[i] = static_cast<uint32_t>((src_row[i] * stride + lane_k()) * static_cast<int64_t>(sizeof(T)));
  }
  __device__ __forceinline__ bool row_ok(int i) const { return (rowok >> i) & 1; }

  __device__ __forceinline__ void fetch_edge(int k0, Regs& g) const {
    const int k = k0 + lane_k();
    g.ok = 0;
#pragma unroll
    for (int i = 0; i < kQuads; ++i)
      g.q[i] = fetch_quad_k<T, V4>(base + src_row[i] * stride + k, base, row_ok(i), k, k_valid, g.ok, i);
  }
  __device__ __forceinline__ void commit_edge(const Regs& g, T* lds) const {
#pragma unroll
    for (int i = 0; i < kQuads; ++i) commit_quad<T>(lds, tile_row(i), lane_k(), mask_quad<T>(g.q[i], (g.ok >> i) & 1));
  }
  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    if constexpr (V4) {
#pragma unroll
      for (int i = 0; i < kQuads; ++i) g.q[i] = quad_at<T>(base + k0, off[i]);
    } else {
      fetch_edge(k0, g);
    }
  }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
    if constexpr (V4) {
#pragma unroll
      for (int i = 0; i < kQuads; ++i) commit_quad<T>(lds, tile_row(i), lane_k(), g.q[i]);
    } else {
      commit_edge(g, lds);
    }
  }
};

// MN-contiguous source: element (k, mn) = base[k * kstride + mn], staged transposed into
// lds[mn][k].  A thread owns a block of KB consecutive k rows x 4 consecutive mn
// (consecutive threads take consecutive mn quads, so each global load is coalesced along mn),
// transposes it in registers and stores KB consecutive k values per mn row.  KB = ROWS / 32 so
// one block per thread covers the chunk.  Optional scales: per-mn `cs[mn]`, per-k
// `rs[k * rs_stride] * rs_mul`; `colsum` also sums the unscaled values of the thread's mn quad
// over its k rows (e.g. a bias gradient, see reduce_colsum).  Unscaled 16-bit interior chunks
// are transposed as raw bits (byte permutes, no conversions).
template <typename T, int ROWS, bool V4>
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
  const T* cs = nullptr;        // per-mn scale, or null
  const float* rs = nullptr;    // per-k scale, or null
  int64_t rs_stride = 1;
  float rs_mul = 1.f;
  bool colsum = false;
  float c[4] = {1.f, 1.f, 1.f, 1.f};       // per-mn scale of this thread's quad
  mutable float csum[4] = {0.f, 0.f, 0.f, 0.f};
  int mn_src = 0;                          // this thread's (clamped) mn quad start
  uint32_t off[KB] = {};                   // byte offset of (kb + t, mn_src) from a chunk base

  static __device__ __forceinline__ int lane_mn() { return (threadIdx.x % kQuadsPerK) * 4; }
  static __device__ __forceinline__ int lane_kb() { return (threadIdx.x / kQuadsPerK) * KB; }

  __device__ __forceinline__ void prepare() {
    const int mn = lane_mn();
    mn_src = (V4 && mn >= mn_valid) ? mn_valid - 4 : mn;
#pragma unroll
    for (int t = 0; t < KB; ++t)
      off[t] = static_cast<uint32_t>(((lane_kb() + t) * kstride + mn_src) * static_cast<int64_t>(sizeof(T)));
    if (cs != nullptr) quad_to_f32<T>(load_quad_scalar<T>(cs + mn, cs, true, 0, mn_valid - mn), c);
  }

  __device__ __forceinline__ void fetch_edge(int k0, Regs& g) const {
    const int mn = lane_mn();
    g.ok = 0;
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int k = k0 + lane_kb() + t;
      const bool kok = k >= 0 && k < k_valid;
      const int kc = kok ? k : 0;
      if constexpr (V4) {
        g.ok |= static_cast<uint32_t>(kok) << t;
        g.q[t] = raw_quad<T>(kok ? base + static_cast<int64_t>(k) * kstride + mn_src : base);
      } else {
        g.ok |= 1u << t;
        g.q[t] = load_quad_scalar<T>(base + static_cast<int64_t>(kc) * kstride + mn, base, kok, 0, mn_valid - mn);
      }
      g.s[t] = rs != nullptr ? rs[static_cast<int64_t>(kc) * rs_stride] : 1.f;
    }
  }
  __device__ __forceinline__ void fetch(int k0, Regs& g) const {
    if constexpr (V4) {
      const T* kb = base + static_cast<int64_t>(k0) * kstride;
#pragma unroll
      for (int t = 0; t < KB; ++t) {
        g.q[t] = quad_at<T>(kb, off[t]);
        g.s[t] = rs != nullptr ? rs[static_cast<int64_t>(k0 + lane_kb() + t) * rs_stride] : 1.f;
      }
    } else {
      fetch_edge(k0, g);
    }
  }

  // Float path: optional masking of k rows (edge), column sums, scales.
  __device__ __forceinline__ void commit_f32(const Regs& g, T* lds, bool masked) const {
    const int mn = lane_mn();
    const int kb = lane_kb();
    float v[KB][4];
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      quad_to_f32<T>(masked ? mask_quad<T>(g.q[t], (g.ok >> t) & 1) : g.q[t], v[t]);
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
  // Raw transpose of 16-bit values: element j of quad t is the 16-bit half (j & 1) of word
  // (j >> 1); pairs of k rows are merged into one 32-bit word per mn with a byte permute.
  __device__ __forceinline__ void commit_raw16(const Regs& g, T* lds) const {
    const int mn = lane_mn();
    const int kb = lane_kb();
    constexpr uint32_t kLo = 0x05040100u, kHi = 0x07060302u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w[(KB + 1) / 2];
#pragma unroll
      for (int t = 0; t + 1 < KB; t += 2) {
        const uint32_t a = (j >> 1) ? g.q[t].y : g.q[t].x;
        const uint32_t b = (j >> 1) ? g.q[t + 1].y : g.q[t + 1].x;
        w[t / 2] = __builtin_amdgcn_perm(b, a, (j & 1) ? kHi : kLo);
      }
      if constexpr (KB == 1) {
        const uint32_t a = (j >> 1) ? g.q[0].y : g.q[0].x;
        *reinterpret_cast<uint16_t*>(lds + lds_index<T>(mn + j, kb)) = static_cast<uint16_t>((j & 1) ? a >> 16 : a);
      } else if constexpr (KB == 2) {
        *reinterpret_cast<uint32_t*>(lds + lds_index<T>(mn + j, kb)) = w[0];
      } else {
        static_assert(KB == 4, "KB in {1, 2, 4}");
        *reinterpret_cast<uint2*>(lds + lds_index<T>(mn + j, kb)) = make_uint2(w[0], w[1]);
      }
    }
  }
  __device__ __forceinline__ void commit_edge(const Regs& g, T* lds) const { commit_f32(g, lds, true); }
  __device__ __forceinline__ void commit(const Regs& g, T* lds) const {
    if constexpr (!V4) {
      commit_f32(g, lds, true);
    } else if constexpr (sizeof(T) == 2) {
      if (cs == nullptr && rs == nullptr && !colsum) {
        commit_raw16(g, lds);
      } else {
        commit_f32(g, lds, false);
      }
    } else {
      commit_f32(g, lds, false);
    }
  }
};

// Column sums gathered by a `colsum` MNLoader: the 256 threads hold partial sums of
// 4 consecutive mn each (thread t: mn = 4 (t % ROWS/4)); they are combined in a fixed
// order through LDS and written as dst[mn] for mn < mn_valid.  Call after the main loop
// (which ends with a barrier), with every thread of the block.
template <typename T, int ROWS, bool V4>
__device__ __forceinline__ void reduce_colsum(const MNLoader<T, ROWS, V4>& ld, T* lds, T* __restrict__ dst) {
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

// Host check: loaders address a tile as a uniform base plus 32-bit per-lane byte offsets that
// span at most 256 rows of `stride` elements.
inline bool gemm_stride_ok(int64_t stride, size_t esz) {
  return stride >= 0 && (stride + 1) * 256 * static_cast<int64_t>(esz) < (int64_t{1} << 31);
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
__device__ __forceinline__ void gemm_mainloop(LA& la, LB& lb, int K, T* lds,
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

  // chunk c covers k in [kbeg + 32 c, kbeg + 32 c + 32); only chunk 0 can be partial
  const int kbeg = K - nk * kChunkK;
  const bool edge0 = kbeg < 0;
  la.prepare();
  lb.prepare();
  typename LA::Regs ra0;
  typename LB::Regs rb0;
  if (edge0) {
    la.fetch_edge(kbeg, ra0);
    lb.fetch_edge(kbeg, rb0);
  } else {
    la.fetch(kbeg, ra0);
    lb.fetch(kbeg, rb0);
  }
  auto commit0 = [&]() {
    if (edge0) {
      la.commit_edge(ra0, lds);
      lb.commit_edge(rb0, lds + BR * P);
    } else {
      la.commit(ra0, lds);
      lb.commit(rb0, lds + BR * P);
    }
  };
  // The steady-state loops below fetch unconditionally: with every trip issuing the
  // same loads into the same registers, the wait-count analysis can see that a
  // register set's previous loads retired before it is refilled, and no conditional
  // path splits the accumulators' live ranges.
  if constexpr (DEPTH == 1) {
    commit0();
    __syncthreads();
    int kc = 0;
    for (; kc + 1 < nk; ++kc) {
      const int cur = (kc & 1) * kBuf;
      la.fetch(kbeg + (kc + 1) * kChunkK, ra0);
      lb.fetch(kbeg + (kc + 1) * kChunkK, rb0);
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
      la.fetch(kbeg + kChunkK, ra1);
      lb.fetch(kbeg + kChunkK, rb1);
    }
    commit0();
    __syncthreads();
    // Entering each trip: chunk kc is in LDS buffer (kc & 1) and its registers (set 0)
    // are free; chunk kc + 1 is in flight into set 1.
    int kc = 0;
    for (; kc + 3 < nk; kc += 2) {
      const int cur = (kc & 1) * kBuf;
      la.fetch(kbeg + (kc + 2) * kChunkK, ra0);
      lb.fetch(kbeg + (kc + 2) * kChunkK, rb0);
      mma(cur);
      la.commit(ra1, lds + kBuf - cur);
      lb.commit(rb1, lds + kBuf - cur + BR * P);
      __syncthreads();
      la.fetch(kbeg + (kc + 3) * kChunkK, ra1);
      lb.fetch(kbeg + (kc + 3) * kChunkK, rb1);
      mma(kBuf - cur);
      la.commit(ra0, lds + cur);
      lb.commit(rb0, lds + cur + BR * P);
      __syncthreads();
    }
    // 1 to 3 chunks left: kc (in LDS), kc + 1 (set 1, in flight), kc + 2 (not fetched)
    const int cur = (kc & 1) * kBuf;
    if (kc + 2 < nk) {
      la.fetch(kbeg + (kc + 2) * kChunkK, ra0);
      lb.fetch(kbeg + (kc + 2) * kChunkK, rb0);
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
