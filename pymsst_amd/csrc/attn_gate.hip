// Attention output gate, forward and backward.
//
//   gate[m, h] = sigmoid(x[m, :] . W[h, :] + b[h])          (stored in the tensor dtype)
//   out[m, h*Dh + d] = attn[m, h, d] * gate[m, h]
//   grad_attn = g * gate;  gpre[m, h] = (sum_d g * attn) * gate * (1 - gate)  (stored)
//   grad_x = gpre W;  grad_W = gpre^T x;  grad_b = sum_m gpre
//
// Semantics follow the reference's attention-gate kernels (fused_band_split.cu:1777-2036):
// the stored (rounded) gate scales attn, and the stored gpre feeds the three products.
//
// Layout: m = b * seq + n is a token; attn is [B, N, H, Dh] with any (b, n, h) strides and a
// contiguous head vector, so the SDPA output can be read through its transposed view and the
// attn gradient written in the [B, H, N, Dh] layout SDPA's backward consumes.  x, out, gate and
// grad_out are dense.
//
// Fast path (H in {2,4,8,16}, H*Dh = 64*E with E in {2,4,8}): one wave per token.  Lane l holds
// E consecutive elements of the token's H*Dh attention row, all inside head l / (64/H).  The H
// gate dots are computed by every lane over its strided slice of x (W transposed in LDS as
// [D][H] fp32), then one reduce-scatter butterfly (H - 1 exchanges) leaves each 64/H-lane group
// with its own head's partial, and log2(64/H) more exchanges finish the sum.  The backward row
// kernel mirrors it, hands the per-head gpre to every lane with readlane for grad_x, and keeps
// each lane's [D/64][H] slice of grad_W in registers; blocks fold their waves in order and the
// deterministic column sum over blocks finishes grad_W / grad_b.  Each wave takes two tokens per
// loop trip, software-pipelined: the next trip's loads (raw 16-byte packs) are issued before this
// trip's stores, so waiting for them never waits for the stores (vmcnt counts loads and stores in
// issue order).  The grids hold as many blocks as fit on the device at once, so a block's staging of
// W is spread over as many tokens as possible.
//
// Any other shape runs the generic kernels (one wave per token, one head at a time).
#include <algorithm>

#include "common.h"
#include "rowgeom.h"

namespace pmsst {
namespace {

constexpr int kGateThreads = 256;
constexpr int kGateWaves = kGateThreads / kWave;
constexpr int kGateMaxBlocks = 4096;
constexpr int kGateDwRows = 64;       // rows per dW chunk
constexpr int kGateDwMaxChunks = 2048;

struct GateRows {
  int64_t sb, sn, sh;  // attn strides (elements) of batch, position, head
  FastDiv seq;
};

__device__ __forceinline__ float sigmoidf(float v) { return 1.0f / (1.0f + expf(-v)); }

template <typename T>
__device__ __forceinline__ const T* token_base(const T* p, const GateRows& g, uint32_t m) {
  const uint32_t b = g.seq.div(m);
  const uint32_t n = m - b * g.seq.d;
  return p + static_cast<int64_t>(b) * g.sb + static_cast<int64_t>(n) * g.sn;
}

template <typename T>
__device__ __forceinline__ T* token_base(T* p, const GateRows& g, uint32_t m) {
  const uint32_t b = g.seq.div(m);
  const uint32_t n = m - b * g.seq.d;
  return p + static_cast<int64_t>(b) * g.sb + static_cast<int64_t>(n) * g.sn;
}

// W[H, D] (storage T) -> LDS wl[i * H + h] (fp32).
template <typename T, int H>
__device__ __forceinline__ void stage_weight(const T* __restrict__ w, float* wl, int dim) {
  for (int k = threadIdx.x; k < H * dim; k += kGateThreads) {
    const int h = k / dim;
    const int i = k - h * dim;
    wl[i * H + h] = to_f32(w[k]);
  }
  __syncthreads();
}

// p[h] holds this lane's partial for head h.  Returns the full 64-lane sum for head
// lane >> (6 - LOGH), in every lane of that head's group.
template <int LOGH>
__device__ __forceinline__ float head_sums(float (&p)[1 << LOGH], int lane) {
  constexpr int H = 1 << LOGH;
  int cnt = H;
#pragma unroll
  for (int lvl = 0; lvl < LOGH; ++lvl) {
    const int off = 32 >> lvl;
    const bool upper = (lane & off) != 0;
    const int half = cnt >> 1;
#pragma unroll
    for (int j = 0; j < H / 2; ++j) {
      if (j < half) {
        const float lo = p[j];
        const float hi = p[half + j];
        const float keep = upper ? hi : lo;
        const float send = upper ? lo : hi;
        p[j] = keep + __shfl_xor(send, off, kWave);
      }
    }
    cnt = half;
  }
  float s = p[0];
#pragma unroll
  for (int off = (kWave >> LOGH) >> 1; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
  return s;
}

// ------------------------------------------------------------------ fast forward

// Rows per wave per loop trip: the loads of both rows (attention packs and x slices) are
// issued a trip ahead, so no global-memory latency sits inside the dot loop.
constexpr int kGateRows = 2;

template <typename T, int E, int LOGH, int JX>
__global__ __launch_bounds__(kGateThreads) void gate_fwd_kernel(const T* __restrict__ attn, GateRows ar,
                                                                const T* __restrict__ x,
                                                                const T* __restrict__ w,
                                                                const T* __restrict__ bias, T* __restrict__ out,
                                                                T* __restrict__ gate, int64_t rows, int dim) {
  constexpr int H = 1 << LOGH;
  constexpr int LPH = kWave >> LOGH;
  constexpr int R = kGateRows;
  extern __shared__ float wl[];
  stage_weight<T, H>(w, wl, dim);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int head = lane / LPH;
  const int sub = lane - head * LPH;
  const float bh = to_f32(bias[head]);
  const int64_t step = static_cast<int64_t>(gridDim.x) * kGateWaves * R;
  int64_t m0 = (static_cast<int64_t>(blockIdx.x) * kGateWaves + wave) * R;
  // rows past the end load the last row (their results are not stored)
  Pack<T, E> ap[R];
  T xr[R][JX];
  auto load = [&](int64_t mb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t m = mb + r < rows ? mb + r : rows - 1;
      ap[r] = *reinterpret_cast<const Pack<T, E>*>(token_base(attn, ar, static_cast<uint32_t>(m)) + head * ar.sh +
                                                   sub * E);
#pragma unroll
      for (int j = 0; j < JX; ++j) {
        const int i = lane + j * kWave;
        xr[r][j] = x[m * dim + (i < dim ? i : 0)];
      }
    }
  };
  if (m0 < rows) load(m0);
  for (; m0 < rows; m0 += step) {
    float a[R][E], xv[R][JX];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int e = 0; e < E; ++e) a[r][e] = to_f32(ap[r].v[e]);
#pragma unroll
      for (int j = 0; j < JX; ++j) xv[r][j] = lane + j * kWave < dim ? to_f32(xr[r][j]) : 0.f;
    }
    if (m0 + step < rows) load(m0 + step);
    float p[R][H];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int h = 0; h < H; ++h) p[r][h] = 0.f;
#pragma unroll
    for (int j = 0; j < JX; ++j) {
      const int i = lane + j * kWave;
      if (i < dim) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const float wv = wl[i * H + h];
#pragma unroll
          for (int r = 0; r < R; ++r) p[r][h] += xv[r][j] * wv;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t m = m0 + r;
      if (m < rows) {  // uniform across the wave
        float q[H];
#pragma unroll
        for (int h = 0; h < H; ++h) q[h] = p[r][h];
        const float s = head_sums<LOGH>(q, lane);
        const T gt = from_f32<T>(sigmoidf(s + bh));
        const float gf = to_f32(gt);
        if (sub == 0) gate[m * H + head] = gt;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = a[r][e] * gf;
        store_pack<T, E>(out + m * (H * LPH * E) + lane * E, o);
      }
    }
  }
}

// ------------------------------------------------------------------ fast backward

// Rows and grad_W / grad_b in one pass: each lane keeps the [JX][H] grad_W columns
// i = lane + 64 j of every head for the rows its wave visits; the block folds its waves in
// wave order through LDS and writes one partial row pw[block][h * dim + i], pb[block][h].
template <typename T, int E, int LOGH, int JX>
__global__ __launch_bounds__(kGateThreads) void gate_bwd_kernel(
    const T* __restrict__ grad_out, const T* __restrict__ attn, GateRows ar, const T* __restrict__ x,
    const T* __restrict__ w, const T* __restrict__ gate, T* __restrict__ grad_attn, GateRows gr,
    T* __restrict__ grad_x, float* __restrict__ pw, float* __restrict__ pb, int64_t rows, int dim) {
  constexpr int H = 1 << LOGH;
  constexpr int LPH = kWave >> LOGH;
  constexpr int R = kGateRows;
  extern __shared__ float sm[];
  float* wl = sm;
  float* red = sm + H * dim;  // [H * dim] grad_W, then [H] grad_b
  stage_weight<T, H>(w, wl, dim);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int head = lane / LPH;
  const int sub = lane - head * LPH;
  float acc[JX][H], accb = 0.f;
#pragma unroll
  for (int j = 0; j < JX; ++j)
#pragma unroll
    for (int h = 0; h < H; ++h) acc[j][h] = 0.f;

  const int64_t step = static_cast<int64_t>(gridDim.x) * kGateWaves * R;
  int64_t m0 = (static_cast<int64_t>(blockIdx.x) * kGateWaves + wave) * R;
  // rows past the end load the last row (their results are not stored)
  Pack<T, E> gp[R], ap[R];
  T gtr[R], xr[R][JX];
  auto load = [&](int64_t mb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t m = mb + r < rows ? mb + r : rows - 1;
      gp[r] = *reinterpret_cast<const Pack<T, E>*>(grad_out + m * (H * LPH * E) + lane * E);
      ap[r] = *reinterpret_cast<const Pack<T, E>*>(token_base(attn, ar, static_cast<uint32_t>(m)) + head * ar.sh +
                                                   sub * E);
      gtr[r] = gate[m * H + head];
#pragma unroll
      for (int j = 0; j < JX; ++j) {
        const int i = lane + j * kWave;
        xr[r][j] = x[m * dim + (i < dim ? i : 0)];
      }
    }
  };
  if (m0 < rows) load(m0);
  for (; m0 < rows; m0 += step) {
    float g[R][E], a[R][E], gf[R], xv[R][JX];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        g[r][e] = to_f32(gp[r].v[e]);
        a[r][e] = to_f32(ap[r].v[e]);
      }
      gf[r] = to_f32(gtr[r]);
#pragma unroll
      for (int j = 0; j < JX; ++j) xv[r][j] = lane + j * kWave < dim ? to_f32(xr[r][j]) : 0.f;
    }
    if (m0 + step < rows) load(m0 + step);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t m = m0 + r;
      if (m >= rows) continue;  // uniform across the wave
      float s = 0.f, o[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        s += g[r][e] * a[r][e];
        o[e] = g[r][e] * gf[r];
      }
      store_pack<T, E>(token_base(grad_attn, gr, static_cast<uint32_t>(m)) + head * gr.sh + sub * E, o);
#pragma unroll
      for (int off = LPH >> 1; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
      const float gpf = to_f32(from_f32<T>(s * gf[r] * (1.0f - gf[r])));
      accb += gpf;
      float gh[H];
#pragma unroll
      for (int h = 0; h < H; ++h) {
        gh[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gpf), h * LPH));
      }
#pragma unroll
      for (int j = 0; j < JX; ++j) {
        const int i = lane + j * kWave;
        float gx = 0.f;
#pragma unroll
        for (int h = 0; h < H; ++h) {
          acc[j][h] += gh[h] * xv[r][j];
          if (i < dim) gx += gh[h] * wl[i * H + h];
        }
        if (i < dim) grad_x[m * dim + i] = from_f32<T>(gx);
      }
    }
  }

  // fold the waves in order (deterministic), then one partial row per block
  for (int wv = 0; wv < kGateWaves; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int j = 0; j < JX; ++j) {
        const int i = lane + j * kWave;
        if (i < dim) {
#pragma unroll
          for (int h = 0; h < H; ++h) red[h * dim + i] = (wv == 0 ? 0.f : red[h * dim + i]) + acc[j][h];
        }
      }
      if (sub == 0) red[H * dim + head] = (wv == 0 ? 0.f : red[H * dim + head]) + accb;
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < H * dim; c += kGateThreads) pw[static_cast<int64_t>(blockIdx.x) * H * dim + c] = red[c];
  if (threadIdx.x < H) pb[static_cast<int64_t>(blockIdx.x) * H + threadIdx.x] = red[H * dim + threadIdx.x];
}

// ------------------------------------------------------------------ generic kernels (any shape)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <typename T>
__global__ __launch_bounds__(kGateThreads) void gate_fwd_generic_kernel(const T* __restrict__ attn, GateRows ar,
                                                                        const T* __restrict__ x,
                                                                        const T* __restrict__ w,
                                                                        const T* __restrict__ bias,
                                                                        T* __restrict__ out, T* __restrict__ gate,
                                                                        int64_t rows, int heads, int dh, int dim) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  for (int64_t m = static_cast<int64_t>(blockIdx.x) * kGateWaves + wave; m < rows;
       m += static_cast<int64_t>(gridDim.x) * kGateWaves) {
    const T* ab = token_base(attn, ar, static_cast<uint32_t>(m));
    const T* xr = x + m * dim;
    for (int h = 0; h < heads; ++h) {
      float p = 0.f;
      for (int i = lane; i < dim; i += kWave) p += to_f32(xr[i]) * to_f32(w[static_cast<int64_t>(h) * dim + i]);
      p = wave_sum(p);
      const T gt = from_f32<T>(sigmoidf(p + to_f32(bias[h])));
      const float gf = to_f32(gt);
      if (lane == 0) gate[m * heads + h] = gt;
      for (int d = lane; d < dh; d += kWave) {
        out[m * heads * dh + static_cast<int64_t>(h) * dh + d] = from_f32<T>(to_f32(ab[h * ar.sh + d]) * gf);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kGateThreads) void gate_bwd_rows_generic_kernel(
    const T* __restrict__ grad_out, const T* __restrict__ attn, GateRows ar, const T* __restrict__ gate,
    T* __restrict__ grad_attn, GateRows gr, T* __restrict__ gpre, int64_t rows, int heads, int dh) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  for (int64_t m = static_cast<int64_t>(blockIdx.x) * kGateWaves + wave; m < rows;
       m += static_cast<int64_t>(gridDim.x) * kGateWaves) {
    const T* ab = token_base(attn, ar, static_cast<uint32_t>(m));
    T* gb = token_base(grad_attn, gr, static_cast<uint32_t>(m));
    for (int h = 0; h < heads; ++h) {
      const float gf = to_f32(gate[m * heads + h]);
      float s = 0.f;
      for (int d = lane; d < dh; d += kWave) {
        const float g = to_f32(grad_out[m * heads * dh + static_cast<int64_t>(h) * dh + d]);
        s += g * to_f32(ab[h * ar.sh + d]);
        gb[h * gr.sh + d] = from_f32<T>(g * gf);
      }
      s = wave_sum(s);
      if (lane == 0) gpre[m * heads + h] = from_f32<T>(s * gf * (1.0f - gf));
    }
  }
}

// grad_x[m, i] = sum_h gpre[m, h] W[h, i]; one thread per element.
template <typename T>
__global__ __launch_bounds__(kGateThreads) void gate_bwd_x_generic_kernel(const T* __restrict__ gpre,
                                                                          const T* __restrict__ w,
                                                                          T* __restrict__ grad_x, int64_t rows,
                                                                          int heads, int dim) {
  const int64_t total = rows * dim;
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kGateThreads + threadIdx.x; k < total;
       k += static_cast<int64_t>(gridDim.x) * kGateThreads) {
    const int64_t m = k / dim;
    const int i = static_cast<int>(k - m * dim);
    float acc = 0.f;
    for (int h = 0; h < heads; ++h) acc += to_f32(gpre[m * heads + h]) * to_f32(w[static_cast<int64_t>(h) * dim + i]);
    grad_x[k] = from_f32<T>(acc);
  }
}

// Partials of grad_W (columns h * dim + i) and grad_b (columns H * dim + h) over one chunk of
// rows per block; the block's threads stride over the columns.
template <typename T>
__global__ __launch_bounds__(kGateThreads) void gate_dw_generic_kernel(const T* __restrict__ gpre,
                                                                       const T* __restrict__ x,
                                                                       float* __restrict__ pw,
                                                                       float* __restrict__ pb, int64_t rows,
                                                                       int heads, int dim, int rows_per_chunk) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_chunk;
  const int64_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
  const int64_t ncol = static_cast<int64_t>(heads) * dim + heads;
  for (int64_t c = threadIdx.x; c < ncol; c += kGateThreads) {
    const bool is_b = c >= static_cast<int64_t>(heads) * dim;
    const int h = is_b ? static_cast<int>(c - static_cast<int64_t>(heads) * dim) : static_cast<int>(c / dim);
    const int i = is_b ? 0 : static_cast<int>(c - static_cast<int64_t>(h) * dim);
    float acc = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
      const float gp = to_f32(gpre[r * heads + h]);
      acc += is_b ? gp : gp * to_f32(x[r * dim + i]);
    }
    if (is_b) {
      pb[static_cast<int64_t>(blockIdx.x) * heads + h] = acc;
    } else {
      pw[static_cast<int64_t>(blockIdx.x) * heads * dim + c] = acc;
    }
  }
}

// ------------------------------------------------------------------ host side

struct GateShape {
  int64_t batch, seq, heads, dh, dim;
  int64_t rows() const { return batch * seq; }
};

inline int gate_log2(int64_t h) {
  int l = 0;
  while ((int64_t{1} << l) < h) ++l;
  return (int64_t{1} << l) == h ? l : -1;
}

// x slices per lane: ceil(dim / 64) up to 4, else 8; 0 when dim > 512.
inline int gate_jx(int64_t dim) {
  const int64_t jx = (dim + kWave - 1) / kWave;
  return jx <= 4 ? static_cast<int>(jx < 1 ? 1 : jx) : jx <= 8 ? 8 : 0;
}

// Fast-path pack width E (elements per lane) or 0 when the generic kernels must run.
inline int gate_fast_e(const GateShape& s, size_t esz, const void* const* ptrs, int nptr, const int64_t* const* strides,
                       int nstr, bool bwd) {
  const int logh = gate_log2(s.heads);
  if (logh < 1 || logh > 4) return 0;
  if ((s.heads * s.dh) % kWave != 0) return 0;
  const int64_t e = s.heads * s.dh / kWave;
  if (e != 2 && e != 4 && e != 8) return 0;
  const int jx = gate_jx(s.dim);
  if (jx == 0) return 0;
  // backward: [jx][H] grad_W accumulators per lane and W + the block fold in LDS
  if (bwd && (s.heads * jx > 64 || static_cast<size_t>(2 * s.heads * s.dim + s.heads) * sizeof(float) > 48 * 1024)) {
    return 0;
  }
  for (int i = 0; i < nptr; ++i) {
    if (reinterpret_cast<uintptr_t>(ptrs[i]) % (e * esz) != 0) return 0;
  }
  for (int i = 0; i < nstr; ++i) {
    for (int k = 0; k < 3; ++k) {
      if (strides[i][k] % e != 0) return 0;
    }
  }
  return static_cast<int>(e);
}

inline int gate_blocks(int64_t rows, int rows_per_wave, int max_blocks) {
  const int64_t per_block = static_cast<int64_t>(kGateWaves) * rows_per_wave;
  const int64_t b = (rows + per_block - 1) / per_block;
  return static_cast<int>(b < max_blocks ? b : max_blocks);
}

// Blocks of a kGateThreads-thread kernel with `shmem` bytes of dynamic LDS that fit on the device at
// once (at least one per CU).
inline int gate_resident_blocks(const void* kernel, size_t shmem) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGateThreads, shmem) != hipSuccess || per_cu < 1)
    per_cu = 1;
  return per_cu * num_cus();
}

// Blocks of the fused backward = rows of its grad_W / grad_b partials.
constexpr int kGateBwdMaxBlocks = 1024;

inline int64_t gate_dw_chunk_rows(int64_t rows) {
  int64_t per = kGateDwRows;
  while ((rows + per - 1) / per > kGateDwMaxChunks) per *= 2;
  return per;
}

inline int64_t gate_dw_chunks(int64_t rows) {
  if (rows <= 0) return 0;
  const int64_t per = gate_dw_chunk_rows(rows);
  return (rows + per - 1) / per;
}

// Workspace of either backward path: [gpre (generic path)] [grad_W partials] [grad_b partials].
inline size_t gate_ws_bytes(int64_t rows, int64_t heads, int64_t dim) {
  int64_t parts = gate_dw_chunks(rows);
  if (parts < kGateBwdMaxBlocks) parts = kGateBwdMaxBlocks;
  return align_up(static_cast<size_t>(rows * heads) * 4, 256) + align_up(static_cast<size_t>(parts * heads * dim) * 4, 256) +
         align_up(static_cast<size_t>(parts * heads) * 4, 256);
}

inline int gate_check(const char* op, const GateShape& s) {
  PMSST_REQUIRE(s.batch >= 0 && s.seq >= 0 && s.heads > 0 && s.dh > 0 && s.dim > 0,
                "%s: bad shape batch=%lld seq=%lld heads=%lld dim_head=%lld dim=%lld", op, (long long)s.batch,
                (long long)s.seq, (long long)s.heads, (long long)s.dh, (long long)s.dim);
  PMSST_REQUIRE(s.rows() < (int64_t{1} << 31) && s.heads * s.dh < (int64_t{1} << 31) && s.dim < (int64_t{1} << 31),
                "%s: tensor too large", op);
  return PMSST_OK;
}

inline GateRows gate_rows(const int64_t* st, const GateShape& s) {
  const int64_t dense_n = s.heads * s.dh;
  GateRows g;
  g.sb = st ? st[0] : s.seq * dense_n;
  g.sn = st ? st[1] : dense_n;
  g.sh = st ? st[2] : s.dh;
  g.seq = FastDiv(static_cast<uint32_t>(s.seq > 0 ? s.seq : 1));
  return g;
}

template <typename T>
int launch_gate_fwd(const void* attn, const int64_t* attn_strides, const void* x, const void* weight,
                    const void* bias, void* out, void* gate, const GateShape& s, hipStream_t stream) {
  const char* op = "attention_gate_forward";
  int rc = gate_check(op, s);
  if (rc != PMSST_OK) return rc;
  const int64_t rows = s.rows();
  if (rows == 0) return PMSST_OK;
  PMSST_REQUIRE(attn && x && weight && bias && out && gate, "%s: null pointer", op);
  const GateRows ar = gate_rows(attn_strides, s);
  PMSST_REQUIRE(ar.sb >= 0 && ar.sn >= 0 && ar.sh >= 0, "%s: negative stride", op);
  const T* pa = static_cast<const T*>(attn);
  const T* px = static_cast<const T*>(x);
  const T* pw = static_cast<const T*>(weight);
  const T* pb = static_cast<const T*>(bias);
  T* po = static_cast<T*>(out);
  T* pg = static_cast<T*>(gate);
  const void* ptrs[] = {attn, out};
  const int64_t ast[3] = {ar.sb, ar.sn, ar.sh};
  const int64_t* strs[] = {ast};
  const int e = gate_fast_e(s, sizeof(T), ptrs, 2, strs, 1, false);
  const int dim = static_cast<int>(s.dim);
  if (e == 0) {
    hipLaunchKernelGGL(gate_fwd_generic_kernel<T>, dim3(gate_blocks(rows, 1, kGateMaxBlocks)), dim3(kGateThreads), 0,
                       stream, pa, ar, px, pw, pb, po, pg, rows, static_cast<int>(s.heads), static_cast<int>(s.dh),
                       dim);
    return check_launch("gate_fwd_generic_kernel");
  }
  const int blocks = gate_blocks(rows, kGateRows, kGateMaxBlocks);
  const int jx = gate_jx(s.dim);
  const size_t shmem = static_cast<size_t>(s.heads * s.dim) * sizeof(float);
#define PMSST_GF(E, LOGH, JX)                                                                                  \
  hipLaunchKernelGGL((gate_fwd_kernel<T, E, LOGH, JX>),                                                          \
                     dim3(std::min(blocks, gate_resident_blocks(reinterpret_cast<const void*>(                    \
                                                                   &gate_fwd_kernel<T, E, LOGH, JX>),             \
                                                               shmem))),                                          \
                     dim3(kGateThreads), shmem, stream, pa, ar, px, pw, pb, po, pg, rows, dim)
#define PMSST_GF_J(E, LOGH)                  \
  do {                                       \
    if (jx == 1) PMSST_GF(E, LOGH, 1);       \
    else if (jx == 2) PMSST_GF(E, LOGH, 2);  \
    else if (jx == 3) PMSST_GF(E, LOGH, 3);  \
    else if (jx == 4) PMSST_GF(E, LOGH, 4);  \
    else PMSST_GF(E, LOGH, 8);               \
  } while (0)
#define PMSST_GF_E(LOGH)                   \
  do {                                     \
    if (e == 2) PMSST_GF_J(2, LOGH);       \
    else if (e == 4) PMSST_GF_J(4, LOGH);  \
    else PMSST_GF_J(8, LOGH);              \
  } while (0)
  switch (gate_log2(s.heads)) {
    case 1: PMSST_GF_E(1); break;
    case 2: PMSST_GF_E(2); break;
    case 3: PMSST_GF_E(3); break;
    default: PMSST_GF_E(4); break;
  }
#undef PMSST_GF_E
#undef PMSST_GF_J
#undef PMSST_GF
  return check_launch("gate_fwd_kernel");
}

template <typename T>
int launch_gate_bwd(const void* grad_out, const void* attn, const int64_t* attn_strides, const void* x,
                    const void* weight, const void* gate, void* grad_attn, const int64_t* grad_attn_strides,
                    void* grad_x, void* grad_weight, void* grad_bias, const GateShape& s, int dtype,
                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const char* op = "attention_gate_backward";
  int rc = gate_check(op, s);
  if (rc != PMSST_OK) return rc;
  const int64_t rows = s.rows();
  PMSST_REQUIRE(grad_weight && grad_bias, "%s: null pointer", op);
  PMSST_REQUIRE(rows == 0 || (grad_out && attn && x && weight && gate && grad_attn && grad_x), "%s: null pointer",
                op);
  const size_t need = gate_ws_bytes(rows, s.heads, s.dim);
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(PMSST_EWORKSPACE, "%s: workspace of %zu bytes needed", op, need);
  }
  const int heads = static_cast<int>(s.heads);
  const int dim = static_cast<int>(s.dim);
  int64_t parts = gate_dw_chunks(rows);
  if (parts < kGateBwdMaxBlocks) parts = kGateBwdMaxBlocks;
  char* ws = static_cast<char*>(workspace);
  T* gpre = reinterpret_cast<T*>(ws);
  float* pw = reinterpret_cast<float*>(ws + align_up(static_cast<size_t>(rows * s.heads) * 4, 256));
  float* pbias =
      reinterpret_cast<float*>(reinterpret_cast<char*>(pw) + align_up(static_cast<size_t>(parts * s.heads * s.dim) * 4, 256));
  int nparts = 0;
  if (rows > 0) {
    const GateRows ar = gate_rows(attn_strides, s);
    const GateRows gr = gate_rows(grad_attn_strides, s);
    PMSST_REQUIRE(ar.sb >= 0 && ar.sn >= 0 && ar.sh >= 0 && gr.sb >= 0 && gr.sn >= 0 && gr.sh >= 0,
                  "%s: negative stride", op);
    const T* pgo = static_cast<const T*>(grad_out);
    const T* pa = static_cast<const T*>(attn);
    const T* px = static_cast<const T*>(x);
    const T* pw_ = static_cast<const T*>(weight);
    const T* pg = static_cast<const T*>(gate);
    T* pga = static_cast<T*>(grad_attn);
    T* pgx = static_cast<T*>(grad_x);
    const void* ptrs[] = {grad_out, attn, grad_attn};
    const int64_t ast[3] = {ar.sb, ar.sn, ar.sh};
    const int64_t gst[3] = {gr.sb, gr.sn, gr.sh};
    const int64_t* strs[] = {ast, gst};
    const int e = gate_fast_e(s, sizeof(T), ptrs, 3, strs, 2, true);
    if (e == 0) {
      const int blocks = gate_blocks(rows, 1, kGateMaxBlocks);
      hipLaunchKernelGGL(gate_bwd_rows_generic_kernel<T>, dim3(blocks), dim3(kGateThreads), 0, stream, pgo, pa, ar,
                         pg, pga, gr, gpre, rows, heads, static_cast<int>(s.dh));
      rc = check_launch("gate_bwd_rows_generic_kernel");
      if (rc != PMSST_OK) return rc;
      const int64_t xb64 = (rows * s.dim + kGateThreads - 1) / kGateThreads;
      const int xb = static_cast<int>(xb64 < 65536 ? xb64 : 65536);
      hipLaunchKernelGGL(gate_bwd_x_generic_kernel<T>, dim3(xb), dim3(kGateThreads), 0, stream, gpre, pw_, pgx, rows,
                         heads, dim);
      rc = check_launch("gate_bwd_x_generic_kernel");
      if (rc != PMSST_OK) return rc;
      nparts = static_cast<int>(gate_dw_chunks(rows));
      hipLaunchKernelGGL(gate_dw_generic_kernel<T>, dim3(static_cast<unsigned>(nparts)), dim3(kGateThreads), 0,
                         stream, gpre, px, pw, pbias, rows, heads, dim, static_cast<int>(gate_dw_chunk_rows(rows)));
      rc = check_launch("gate_dw_generic_kernel");
      if (rc != PMSST_OK) return rc;
    } else {
      nparts = gate_blocks(rows, kGateRows, kGateBwdMaxBlocks);
      const int jx = gate_jx(s.dim);
      const size_t shmem = static_cast<size_t>(2 * s.heads * s.dim + s.heads) * sizeof(float);
      // (as many blocks as fit on the device at once; nparts is also the partial rows' count)
#define PMSST_GB(E, LOGH, JX)                                                                                   \
  do {                                                                                                          \
    nparts = std::min(nparts, gate_resident_blocks(reinterpret_cast<const void*>(&gate_bwd_kernel<T, E, LOGH, JX>), \
                                                   shmem));                                                     \
    hipLaunchKernelGGL((gate_bwd_kernel<T, E, LOGH, JX>), dim3(nparts), dim3(kGateThreads), shmem, stream, pgo,  \
                       pa, ar, px, pw_, pg, pga, gr, pgx, pw, pbias, rows, dim);                                \
  } while (0)
#define PMSST_GB_J(E, LOGH)                  \
  do {                                       \
    if (jx == 1) PMSST_GB(E, LOGH, 1);       \
    else if (jx == 2) PMSST_GB(E, LOGH, 2);  \
    else if (jx == 3) PMSST_GB(E, LOGH, 3);  \
    else if (jx == 4) PMSST_GB(E, LOGH, 4);  \
    else PMSST_GB(E, LOGH, 8);               \
  } while (0)
#define PMSST_GB_E(LOGH)                   \
  do {                                     \
    if (e == 2) PMSST_GB_J(2, LOGH);       \
    else if (e == 4) PMSST_GB_J(4, LOGH);  \
    else PMSST_GB_J(8, LOGH);              \
  } while (0)
      switch (gate_log2(s.heads)) {
        case 1: PMSST_GB_E(1); break;
        case 2: PMSST_GB_E(2); break;
        case 3: PMSST_GB_E(3); break;
        default: PMSST_GB_E(4); break;
      }
#undef PMSST_GB_E
#undef PMSST_GB_J
#undef PMSST_GB
      rc = check_launch("gate_bwd_kernel");
      if (rc != PMSST_OK) return rc;
    }
  }
  rc = launch_col_sum(pw, nparts, heads * dim, grad_weight, dtype, stream);
  if (rc != PMSST_OK) return rc;
  return launch_col_sum(pbias, nparts, heads, grad_bias, dtype, stream);
}

template <typename F>
int gate_dtype(int dtype, const char* op, F&& f) {
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

int pmsst_attention_gate_forward(const void* attn, const int64_t* attn_strides, const void* x, const void* weight,
                                 const void* bias, void* out, void* gate, int64_t batch, int64_t seq, int64_t heads,
                                 int64_t dim_head, int64_t dim, int dtype, void* stream) {
  const GateShape s{batch, seq, heads, dim_head, dim};
  return gate_dtype(dtype, "attention_gate_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_gate_fwd<T>(attn, attn_strides, x, weight, bias, out, gate, s, static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_attention_gate_backward_workspace_size(int64_t rows, int64_t heads, int64_t dim) {
  if (rows < 0 || heads <= 0 || dim <= 0) return 0;
  return gate_ws_bytes(rows, heads, dim);
}

int pmsst_attention_gate_backward(const void* grad_out, const void* attn, const int64_t* attn_strides, const void* x,
                                  const void* weight, const void* gate, void* grad_attn,
                                  const int64_t* grad_attn_strides, void* grad_x, void* grad_weight, void* grad_bias,
                                  int64_t batch, int64_t seq, int64_t heads, int64_t dim_head, int64_t dim, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  const GateShape s{batch, seq, heads, dim_head, dim};
  return gate_dtype(dtype, "attention_gate_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_gate_bwd<T>(grad_out, attn, attn_strides, x, weight, gate, grad_attn, grad_attn_strides, grad_x,
                              grad_weight, grad_bias, s, dtype, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
