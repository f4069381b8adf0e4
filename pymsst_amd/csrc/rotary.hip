// Rotary embedding on bnhd q/k, and the fused q/k RMSNorm + rotary + cast.
//
// Rotary is a pure stream: each lane moves one 16-byte pack (VEC elements,
// VEC/2 adjacent pairs) per step.  One launch can carry q, k and v of a fused qkv
// projection (v copied): the split into the attention layout, and in the backward
// the stacking of the three gradients back into the qkv gradient, cost no extra pass.  The pack's (batch, position, head, element)
// come from multiply-shift divisions; cos/sin rows (seq x dim/2, a few KB) stay
// in L1/L2.  Input and output take independent (batch, seq, head) strides, so
// q/k are read straight out of the fused qkv projection and can be written in
// the [B, H, N, D] layout attention consumes (no copies on either side).
//
// The fused kernel uses the RMSNorm row geometry: one row = one head vector
// of `dim` elements; pairs never straddle a pack because VEC is even.
#include "common.h"
#include "rowgeom.h"

namespace pmsst {
namespace {

constexpr int kRotThreads = 256;
#ifndef PMSST_ROT_UNROLL
#define PMSST_ROT_UNROLL 2
#endif
constexpr int kRotUnroll = PMSST_ROT_UNROLL;  // packs per thread per trip
constexpr int kNormRotThreads = 256;

struct TableRef {
  int64_t stride_seq;
  int64_t stride_pair;
};

// Element strides of a [B, N, H, D] view whose last axis is contiguous.
struct BnhStrides {
  int64_t b, n, h;
};

// Table access modes: 1 = one value per pair, contiguous; 2 = the pair-repeated
// [.., D] table read through its [..., ::2] view (stride 2): one 16-byte load covers
// the pairs of a pack and the even elements are used; 0 = any strides, scalar loads.
enum { kTabAny = 0, kTabDense = 1, kTabRepeated = 2 };

// cos or sin of pairs p0 .. p0 + NP - 1 of one table row `r`.
template <typename T, int NP, int TS>
__device__ __forceinline__ void load_table(const T* __restrict__ r, int p0, int64_t stride_pair, float (&o)[NP]) {
  if constexpr (TS == kTabDense) {
    load_pack<T, NP>(r + p0, o);
  } else if constexpr (TS == kTabRepeated) {
    if constexpr (sizeof(T) == 2 && NP == 4) {
      // one 16-byte load; the even elements (low halves of the 4 words) are gathered with byte
      // permutes, which keeps the compiler from splitting the load into 4 two-byte loads
      const uint4 w = *reinterpret_cast<const uint4*>(r + 2 * p0);
      const uint2 ev{__builtin_amdgcn_perm(w.y, w.x, 0x05040100u), __builtin_amdgcn_perm(w.w, w.z, 0x05040100u)};
      const Pack<T, 4> pk = __builtin_bit_cast(Pack<T, 4>, ev);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = to_f32(pk.v[j]);
    } else {
      float tmp[2 * NP];
      load_pack<T, 2 * NP>(r + 2 * p0, tmp);
#pragma unroll
      for (int j = 0; j < NP; ++j) o[j] = tmp[2 * j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < NP; ++j) o[j] = to_f32(r[(p0 + j) * stride_pair]);
  }
}

// A raw 16-byte pack (VEC = 16 / sizeof(T) elements) as fp32, converted from the bits (a
// vector register keeps the compiler from slicing the load into pieces).
template <typename T>
__device__ __forceinline__ void raw_to_f32(const u32x4_t& w, float (&o)[16 / sizeof(T)]) {
  if constexpr (std::is_same<T, bf16>::value) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __uint_as_float(w[k] << 16);
      o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  } else if constexpr (std::is_same<T, f16>::value) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(w[k] & 0xffffu)));
      o[2 * k + 1] = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(w[k] >> 16)));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __uint_as_float(w[k]);
  }
}

// A table piece held as loaded until the arithmetic: the 16-byte repeated-table piece stays raw
// (converted by get() after every load of a trip has issued); other modes convert at load.
template <typename T, int NP, int TS>
struct TabPiece {
  static constexpr bool kRaw = TS == kTabRepeated && sizeof(T) == 2 && NP == 4;
  u32x4_t w;
  float f[NP];
  __device__ __forceinline__ void load(const T* __restrict__ r, int p0, int64_t stride_pair) {
    if constexpr (kRaw) w = *reinterpret_cast<const u32x4_t*>(r + 2 * p0);
    else load_table<T, NP, TS>(r, p0, stride_pair, f);
  }
  __device__ __forceinline__ void get(float (&o)[NP]) const {
    if constexpr (kRaw) {
      const uint2 ev{__builtin_amdgcn_perm(w.y, w.x, 0x05040100u), __builtin_amdgcn_perm(w.w, w.z, 0x05040100u)};
      const Pack<T, 4> pk = __builtin_bit_cast(Pack<T, 4>, ev);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = to_f32(pk.v[j]);
    } else {
#pragma unroll
      for (int j = 0; j < NP; ++j) o[j] = f[j];
    }
  }
};

// Fastest table mode the strides and alignment allow for packs of `vec` elements.
inline int table_mode(const void* cosv, const void* sinv, int64_t cs_seq, int64_t cs_pair, int vec, size_t elem) {
  auto al = [&](const void* p, int64_t n) { return reinterpret_cast<uintptr_t>(p) % (n * elem) == 0; };
  if (cs_pair == 2 && cs_seq % vec == 0 && al(cosv, vec) && al(sinv, vec)) return kTabRepeated;
  if (vec >= 4 && cs_pair == 1 && cs_seq % (vec / 2) == 0 && al(cosv, vec / 2) && al(sinv, vec / 2)) return kTabDense;
  return kTabAny;
}

// Up to three [B, N, H, D] tensors per launch, one per blockIdx.y: parts [0, rotated) are
// rotated, the others copied (v next to q and k when a fused qkv buffer is split).
template <typename T>
struct RotParts {
  const T* in[3];
  T* out[3];
  BnhStrides si[3];
  BnhStrides so[3];
  int rotated;
};

template <typename T, int VEC, bool INVERSE, int TS>
__global__ __launch_bounds__(kRotThreads) void rotary_kernel(RotParts<T> io, const T* __restrict__ cosv,
                                                             const T* __restrict__ sinv, uint32_t part_packs,
                                                             FastDiv packs_per_token, FastDiv seq, FastDiv dim,
                                                             TableRef tab) {
  const int part = blockIdx.y;
  const T* __restrict__ in = io.in[part];
  T* __restrict__ out = io.out[part];
  const BnhStrides si = io.si[part];
  const BnhStrides so = io.so[part];
  // kRotUnroll packs per thread per trip, all loads issued first; 16-byte packs are moved raw in
  // a vector register (the copied part is stored as loaded).  Packs past the end redo the last
  // pack.  The rotate / copy choice is made once per block, outside the loop: no load sits in a
  // branch (a load inside a branch, or used only inside one, is waited for at the join).
  constexpr bool kRaw = VEC * sizeof(T) == 16;
  const uint32_t stride = gridDim.x * kRotThreads;
  auto run = [&](auto rot_tag) {
    constexpr bool ROT = decltype(rot_tag)::value;
    for (uint32_t i0 = blockIdx.x * kRotThreads * kRotUnroll + threadIdx.x; i0 < part_packs;
         i0 += stride * kRotUnroll) {
      u32x4_t raw[kRotUnroll];
      float v[kRotUnroll][VEC];
      float cv[kRotUnroll][VEC / 2], sv[kRotUnroll][VEC / 2];
      int64_t oo[kRotUnroll];
#pragma unroll
      for (int u = 0; u < kRotUnroll; ++u) {
        const uint32_t iu = i0 + u * kRotThreads;
        const uint32_t i = iu < part_packs ? iu : part_packs - 1;
        const uint32_t tok = packs_per_token.div(i);
        const uint32_t e = (i - tok * packs_per_token.d) * VEC;  // element offset inside the token
        const uint32_t b = seq.div(tok);
        const uint32_t n = tok - b * seq.d;
        const uint32_t h = dim.div(e);
        const uint32_t d = e - h * dim.d;
        const T* src = in + b * si.b + n * si.n + h * si.h + d;
        if constexpr (kRaw) raw[u] = *reinterpret_cast<const u32x4_t*>(src);
        else load_pack<T, VEC>(src, v[u]);
        if constexpr (ROT) {
          load_table<T, VEC / 2, TS>(cosv + n * tab.stride_seq, d >> 1, tab.stride_pair, cv[u]);
          load_table<T, VEC / 2, TS>(sinv + n * tab.stride_seq, d >> 1, tab.stride_pair, sv[u]);
        }
        oo[u] = b * so.b + n * so.n + h * so.h + d;
      }
#pragma unroll
      for (int u = 0; u < kRotUnroll; ++u) {
        if constexpr (!(kRaw && !ROT)) {
          if constexpr (kRaw) raw_to_f32<T>(raw[u], v[u]);
          if constexpr (ROT) {
#pragma unroll
            for (int j = 0; j < VEC / 2; ++j) {
              const float c = cv[u][j];
              const float s = sv[u][j];
              const float ev = v[u][2 * j], ov = v[u][2 * j + 1];
              if (INVERSE) {
                v[u][2 * j] = ev * c + ov * s;
                v[u][2 * j + 1] = ov * c - ev * s;
              } else {
                v[u][2 * j] = ev * c - ov * s;
                v[u][2 * j + 1] = ov * c + ev * s;
              }
            }
          }
        }
      }
      // a pack past the end recomputes the last pack from the same input and position, so its
      // store writes the same bits the last pack's own store writes: no guard is needed
#pragma unroll
      for (int u = 0; u < kRotUnroll; ++u) {
        if constexpr (kRaw && !ROT) *reinterpret_cast<u32x4_t*>(out + oo[u]) = raw[u];
        else store_pack<T, VEC>(out + oo[u], v[u]);
      }
    }
  };
  if (part < io.rotated) run(std::true_type{});
  else run(std::false_type{});
}

// `nparts` tensors of one [batch, seq, heads, dim] shape; strides are {b, n, h} triples (NULL
// = dense bnhd); the first `rotated` parts are rotated, the rest copied.
template <typename T>
int launch_rotary_parts(const char* op, int nparts, int rotated, const void* const* in,
                        const int64_t* const* in_strides, const void* cosv, const void* sinv, void* const* out,
                        const int64_t* const* out_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                        int64_t cs_seq, int64_t cs_pair, bool inverse, hipStream_t stream) {
  PMSST_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0 && dim > 0 && dim % 2 == 0,
                "%s: bad shape [%lld, %lld, %lld, %lld]", op, (long long)batch, (long long)seq, (long long)heads,
                (long long)dim);
  const int64_t total = batch * seq * heads * dim;
  if (total == 0) return PMSST_OK;
  PMSST_REQUIRE(cosv && sinv, "%s: null pointer", op);
  RotParts<T> io{};
  io.rotated = rotated;
  const BnhStrides dense{seq * heads * dim, heads * dim, dim};
  for (int p = 0; p < nparts; ++p) {
    PMSST_REQUIRE(in[p] && out[p], "%s: null pointer", op);
    io.in[p] = static_cast<const T*>(in[p]);
    io.out[p] = static_cast<T*>(out[p]);
    io.si[p] = in_strides[p] ? BnhStrides{in_strides[p][0], in_strides[p][1], in_strides[p][2]} : dense;
    io.so[p] = out_strides[p] ? BnhStrides{out_strides[p][0], out_strides[p][1], out_strides[p][2]} : dense;
    PMSST_REQUIRE(io.si[p].b >= 0 && io.si[p].n >= 0 && io.si[p].h >= 0 && io.so[p].b >= 0 && io.so[p].n >= 0 &&
                      io.so[p].h >= 0,
                  "%s: negative stride", op);
  }
  int vec = 16 / sizeof(T);
  auto aligned = [&](int v) {
    bool ok = dim % v == 0;
    for (int p = 0; p < nparts; ++p) {
      ok = ok && reinterpret_cast<uintptr_t>(in[p]) % (v * sizeof(T)) == 0 &&
           reinterpret_cast<uintptr_t>(out[p]) % (v * sizeof(T)) == 0;
      for (int64_t st : {io.si[p].b, io.si[p].n, io.si[p].h, io.so[p].b, io.so[p].n, io.so[p].h}) ok = ok && st % v == 0;
    }
    return ok;
  };
  while (vec > 2 && !aligned(vec)) vec /= 2;
  PMSST_REQUIRE(aligned(vec), "%s: tensors must be 4-byte aligned", op);
  const int64_t packs = total / vec;
  PMSST_REQUIRE(packs < (int64_t{1} << 31) && seq * heads < (int64_t{1} << 31), "%s: tensor too large", op);
  const FastDiv ppt(static_cast<uint32_t>(heads * dim / vec));
  const FastDiv fseq(static_cast<uint32_t>(seq));
  const FastDiv fdim(static_cast<uint32_t>(dim));
  const TableRef tab{cs_seq, cs_pair};
  const int64_t blocks64 = (packs + kRotThreads * kRotUnroll - 1) / (kRotThreads * kRotUnroll);
  const dim3 grid(static_cast<unsigned>(blocks64 < 65536 ? blocks64 : 65536), static_cast<unsigned>(nparts));
  const uint32_t np = static_cast<uint32_t>(packs);
  const int ts = table_mode(cosv, sinv, cs_seq, cs_pair, vec, sizeof(T));
  const T* pc = static_cast<const T*>(cosv);
  const T* ps = static_cast<const T*>(sinv);
#define PMSST_ROT1(VEC, INV, TS) \
  hipLaunchKernelGGL((rotary_kernel<T, VEC, INV, TS>), grid, dim3(kRotThreads), 0, stream, io, pc, ps, np, ppt, fseq, fdim, tab)
#define PMSST_ROT(VEC, INV)                                     \
  do {                                                          \
    if (ts == kTabRepeated) PMSST_ROT1(VEC, INV, kTabRepeated); \
    else if (ts == kTabDense) PMSST_ROT1(VEC, INV, kTabDense);  \
    else PMSST_ROT1(VEC, INV, kTabAny);                         \
  } while (0)
  if (inverse) {
    if (vec == 16 / (int)sizeof(T)) PMSST_ROT(16 / sizeof(T), true);
    else if (vec == 8 / (int)sizeof(T)) PMSST_ROT(8 / sizeof(T), true);
    else PMSST_ROT(2, true);
  } else {
    if (vec == 16 / (int)sizeof(T)) PMSST_ROT(16 / sizeof(T), false);
    else if (vec == 8 / (int)sizeof(T)) PMSST_ROT(8 / sizeof(T), false);
    else PMSST_ROT(2, false);
  }
#undef PMSST_ROT
#undef PMSST_ROT1
  return check_launch("rotary_kernel");
}

template <typename T>
int launch_rotary(const void* in, const int64_t* in_strides, const void* cosv, const void* sinv, void* out,
                  const int64_t* out_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim, int64_t cs_seq,
                  int64_t cs_pair, bool inverse, hipStream_t stream) {
  const void* ins[] = {in};
  void* outs[] = {out};
  const int64_t* sis[] = {in_strides};
  const int64_t* sos[] = {out_strides};
  return launch_rotary_parts<T>(inverse ? "rotary_backward" : "rotary_forward", 1, 1, ins, sis, cosv, sinv, outs, sos,
                                batch, seq, heads, dim, cs_seq, cs_pair, inverse, stream);
}

// ------------------------------------------------------------------ fused q/k RMSNorm + rotary

// Rows per lane slot in flight: the loads of kRowsPerSlot rows are issued before any
// reduction, so each lane keeps several 16-byte packs outstanding.
#ifndef PMSST_NR_ROWS
#define PMSST_NR_ROWS 2
#endif
constexpr int kRowsPerSlot = PMSST_NR_ROWS;
// Forward grid: 0 = one trip per block; N = at most N blocks per CU, each looping over trips.
#ifndef PMSST_NR_GRID
#define PMSST_NR_GRID 0
#endif

// One or two tensors of one shape (q and k) in one launch: blocks [0, per_tensor) take tensor 0, the
// next per_tensor blocks tensor 1; each has its own input, gamma, output and inv_norm.
template <typename T, typename TG>
struct NormRotIO {
  const T* x[2];
  const TG* gamma[2];
  T* out[2];         // forward output / backward dx
  float* inv[2];     // inv_norm (the backward reads it)
  const T* dy[2];    // backward only
  int per_tensor;    // blocks per tensor
};

template <typename T, typename TG, int VEC, int NV, int TS>
__global__ __launch_bounds__(kNormRotThreads) void norm_rot_fwd_kernel(NormRotIO<T, TG> io, const T* __restrict__ cosv,
                                                                    const T* __restrict__ sinv, int64_t rows,
                                                                    int tpr_log2, float scale, FastDiv heads,
                                                                    FastDiv seq, TableRef tab) {
  const int tsel = static_cast<int>(blockIdx.x) >= io.per_tensor ? 1 : 0;
  const int blk = static_cast<int>(blockIdx.x) - tsel * io.per_tensor;
  const T* __restrict__ x = io.x[tsel];
  const TG* __restrict__ gamma = io.gamma[tsel];
  T* __restrict__ out = io.out[tsel];
  float* __restrict__ inv_norm = io.inv[tsel];
  const int tpr = 1 << tpr_log2;
  const int dim = VEC * NV * tpr;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t = lane & (tpr - 1);
  const int slot = lane >> tpr_log2;
  const int rows_per_wave = kWave >> tpr_log2;
  const int rows_per_block = rows_per_wave * (kNormRotThreads / kWave);

  float g[NV][VEC];
#pragma unroll
  for (int v = 0; v < NV; ++v) load_pack<TG, VEC>(gamma + (v * tpr + t) * VEC, g[v]);

  for (int64_t base = static_cast<int64_t>(blk) * rows_per_block * kRowsPerSlot; base < rows;
       base += static_cast<int64_t>(io.per_tensor) * rows_per_block * kRowsPerSlot) {
    // every load of the trip (x packs and the cos / sin of each row's position) is issued
    // before the first reduction; the packs stay raw until then
    u32x4_t xr[kRowsPerSlot][NV];
    TabPiece<T, VEC / 2, TS> ct[kRowsPerSlot][NV], st[kRowsPerSlot][NV];
#pragma unroll
    for (int u = 0; u < kRowsPerSlot; ++u) {
      // rows past the end load the last row (no branch around the loads: a load inside a
      // branch is waited for at the join, which would serialize the rows of the trip)
      const int64_t row = base + u * rows_per_block + wave * rows_per_wave + slot;
      const int64_t rl = row < rows ? row : rows - 1;
      const uint32_t n = seq.mod(heads.div(static_cast<uint32_t>(rl)));
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        xr[u][v] = *reinterpret_cast<const u32x4_t*>(x + rl * dim + col);
        ct[u][v].load(cosv + n * tab.stride_seq, col / 2, tab.stride_pair);
        st[u][v].load(sinv + n * tab.stride_seq, col / 2, tab.stride_pair);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads of the trip issue before the first wait
    // a row past the end recomputes the last row from the same data, so its stores write the
    // bits the last row's own stores write: the arithmetic and stores need no guard (a load
    // used only under a guard would be moved into it and waited for there)
#pragma unroll
    for (int u = 0; u < kRowsPerSlot; ++u) {
      const int64_t row = base + u * rows_per_block + wave * rows_per_wave + slot;
      const int64_t rl = row < rows ? row : rows - 1;
      float xv[NV][VEC];
      float ss = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        raw_to_f32<T>(xr[u][v], xv[v]);
#pragma unroll
        for (int i = 0; i < VEC; ++i) ss += xv[v][i] * xv[v][i];
      }
      ss = group_sum(ss, tpr);
      const float inv = 1.0f / fmaxf(sqrtf(ss), 1.0e-12f);
      const float s = inv * scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        float cv[VEC / 2], sv[VEC / 2], o[VEC];
        ct[u][v].get(cv);
        st[u][v].get(sv);
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          const float ev = xv[v][2 * j] * s * g[v][2 * j];
          const float ov = xv[v][2 * j + 1] * s * g[v][2 * j + 1];
          o[2 * j] = ev * cv[j] - ov * sv[j];
          o[2 * j + 1] = ov * cv[j] + ev * sv[j];
        }
        store_pack<T, VEC>(out + rl * dim + col, o);
      }
      if (t == 0) inv_norm[rl] = inv;
    }
  }
}

// dgamma partials: block b of tensor t writes row b, columns t * dim .. of partial[per_tensor, ntensors * dim]
template <typename T, typename TG, int VEC, int NV, int TS>
__global__ __launch_bounds__(kRowBwdThreads) void norm_rot_bwd_kernel(NormRotIO<T, TG> io, const T* __restrict__ cosv,
                                                                      const T* __restrict__ sinv,
                                                                      float* __restrict__ partial, int pitch,
                                                                      int64_t rows, int tpr_log2, float scale,
                                                                      FastDiv heads, FastDiv seq, TableRef tab) {
  extern __shared__ float red[];
  const int tsel = static_cast<int>(blockIdx.x) >= io.per_tensor ? 1 : 0;
  const int blk = static_cast<int>(blockIdx.x) - tsel * io.per_tensor;
  const T* __restrict__ dy = io.dy[tsel];
  const T* __restrict__ x = io.x[tsel];
  const float* __restrict__ inv_norm = io.inv[tsel];
  const TG* __restrict__ gamma = io.gamma[tsel];
  T* __restrict__ dx = io.out[tsel];
  const int tpr = 1 << tpr_log2;
  const int dim = VEC * NV * tpr;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t = lane & (tpr - 1);
  const int slot = lane >> tpr_log2;
  const int rows_per_wave = kWave >> tpr_log2;
  const int rows_per_block = rows_per_wave * (kRowBwdThreads / kWave);

  float g[NV][VEC], acc[NV][VEC];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    load_pack<TG, VEC>(gamma + (v * tpr + t) * VEC, g[v]);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[v][i] = 0.f;
  }
  const float inv_scale = 1.0f / scale;
  // rows per lane slot in flight: one for rows of 3 or 4 packs per lane (two would need more than
  // the 256 registers of a wave and spill)
  constexpr int RPS = NV >= 3 ? 1 : kRowsPerSlot;

  for (int64_t base = static_cast<int64_t>(blk) * rows_per_block * RPS; base < rows;
       base += static_cast<int64_t>(io.per_tensor) * rows_per_block * RPS) {
    // loads of all RPS rows first, held raw until every load of the trip has issued.
    // Rows past the end load the last row (no branch around the loads) and recompute it: their
    // dx stores write the bits the last row's own stores write, and only the dgamma
    // accumulation excludes them.
    u32x4_t dr[RPS][NV], xr[RPS][NV];
    TabPiece<T, VEC / 2, TS> ct[RPS][NV], st[RPS][NV];
    float inv[RPS];
#pragma unroll
    for (int u = 0; u < RPS; ++u) {
      const int64_t row = base + u * rows_per_block + wave * rows_per_wave + slot;
      const int64_t rl = row < rows ? row : rows - 1;
      inv[u] = inv_norm[rl];
      const uint32_t pos = seq.mod(heads.div(static_cast<uint32_t>(rl)));
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        dr[u][v] = *reinterpret_cast<const u32x4_t*>(dy + rl * dim + col);
        xr[u][v] = *reinterpret_cast<const u32x4_t*>(x + rl * dim + col);
        ct[u][v].load(cosv + pos * tab.stride_seq, col / 2, tab.stride_pair);
        st[u][v].load(sinv + pos * tab.stride_seq, col / 2, tab.stride_pair);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads of the trip issue before the first wait
#pragma unroll
    for (int u = 0; u < RPS; ++u) {
      const int64_t row = base + u * rows_per_block + wave * rows_per_wave + slot;
      const bool valid = row < rows;
      const int64_t rl = valid ? row : rows - 1;
      const float ns = inv[u] * scale;
      float gr[NV][VEC], n[NV][VEC];
      float dot = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float d[VEC], cv[VEC / 2], sv[VEC / 2];
        raw_to_f32<T>(dr[u][v], d);
        raw_to_f32<T>(xr[u][v], n[v]);
        ct[u][v].get(cv);
        st[u][v].get(sv);
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          gr[v][2 * j] = d[2 * j] * cv[j] + d[2 * j + 1] * sv[j];
          gr[v][2 * j + 1] = d[2 * j + 1] * cv[j] - d[2 * j] * sv[j];
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          n[v][i] *= ns;
          dot += gr[v][i] * g[v][i] * n[v][i];
        }
      }
      dot = group_sum(dot, tpr);
      const float dot_s = dot * inv_scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          o[i] = inv[u] * (gr[v][i] * g[v][i] * scale - n[v][i] * dot_s);
          acc[v][i] += valid ? gr[v][i] * n[v][i] : 0.f;
        }
        store_pack<T, VEC>(dx + rl * dim + (v * tpr + t) * VEC, o);
      }
    }
  }

#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[v][i] = cross_group_sum(acc[v][i], tpr);
  }
  if (slot == 0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) red[wave * dim + (v * tpr + t) * VEC + i] = acc[v][i];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < dim; c += kRowBwdThreads) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kRowBwdThreads / kWave; ++w) s += red[w * dim + c];
    partial[static_cast<int64_t>(blk) * pitch + tsel * dim + c] = s;
  }
}

struct NormRotArgs {
  int64_t batch, seq, heads, dim, cs_seq, cs_pair;
};

inline int norm_rot_check(const char* op, const NormRotArgs& a, int vec, const void* const* ptrs,
                          const size_t* sizes, int nptr, RowGeom* geo) {
  PMSST_REQUIRE(a.batch >= 0 && a.seq >= 0 && a.heads >= 0 && a.dim > 0 && a.dim % 2 == 0,
                "%s: bad shape [%lld, %lld, %lld, %lld]", op, (long long)a.batch, (long long)a.seq,
                (long long)a.heads, (long long)a.dim);
  PMSST_REQUIRE(a.batch * a.seq * a.heads < (int64_t{1} << 31), "%s: too many rows", op);
  *geo = pick_row_geom(a.dim, vec, ptrs, sizes, nptr);
  PMSST_REQUIRE(geo->ok && geo->vec == vec,
                "%s: head dim %lld must be a multiple of %d with 16-byte aligned tensors and at most %d elements",
                op, (long long)a.dim, vec, 4 * 64 * vec);
  return PMSST_OK;
}

// nt = 1 or 2 tensors of one shape (x[t], gamma[t], out[t], inv_norm[t]), one launch.
template <typename T, typename TG>
int launch_norm_rot_fwd(int nt, const void* const* x, const void* const* gamma, const void* cosv, const void* sinv,
                        void* const* out, float* const* inv_norm, const NormRotArgs& a, hipStream_t stream) {
  if (a.batch * a.seq * a.heads == 0 && a.dim > 0) return PMSST_OK;
  constexpr int kVec = 16 / sizeof(T);
  NormRotIO<T, TG> io{};
  RowGeom geo{};
  for (int t = 0; t < nt; ++t) {
    PMSST_REQUIRE(x[t] && gamma[t] && cosv && sinv && out[t] && inv_norm[t], "rms_norm_rotary_forward: null pointer");
    const void* ptrs[] = {x[t], gamma[t], out[t]};
    const size_t sizes[] = {sizeof(T), sizeof(TG), sizeof(T)};
    const int rc = norm_rot_check("rms_norm_rotary_forward", a, kVec, ptrs, sizes, 3, &geo);
    if (rc != PMSST_OK) return rc;
    io.x[t] = static_cast<const T*>(x[t]);
    io.gamma[t] = static_cast<const TG*>(gamma[t]);
    io.out[t] = static_cast<T*>(out[t]);
    io.inv[t] = inv_norm[t];
  }
  const int64_t rows = a.batch * a.seq * a.heads;
  if (rows == 0) return PMSST_OK;
  const int rpb = (kWave >> geo.tpr_log2) * (kNormRotThreads / kWave) * kRowsPerSlot;
  int64_t blocks64 = (rows + rpb - 1) / rpb;
  if (PMSST_NR_GRID > 0 && blocks64 > static_cast<int64_t>(PMSST_NR_GRID) * num_cus())
    blocks64 = static_cast<int64_t>(PMSST_NR_GRID) * num_cus();
  io.per_tensor = static_cast<int>(blocks64 < 32768 ? blocks64 : 32768);
  const int blocks = io.per_tensor * nt;
  const float scale = sqrtf(static_cast<float>(a.dim));
  const FastDiv fh(static_cast<uint32_t>(a.heads)), fs(static_cast<uint32_t>(a.seq));
  const TableRef tab{a.cs_seq, a.cs_pair};
  const int ts = table_mode(cosv, sinv, a.cs_seq, a.cs_pair, kVec, sizeof(T));
#define PMSST_NRF1(NV, TS)                                                                                        \
  hipLaunchKernelGGL((norm_rot_fwd_kernel<T, TG, kVec, NV, TS>), dim3(blocks), dim3(kNormRotThreads), 0, stream, \
                     io, static_cast<const T*>(cosv), static_cast<const T*>(sinv), rows, geo.tpr_log2, scale,    \
                     fh, fs, tab)
#define PMSST_NRF(NV)                                          \
  do {                                                         \
    if (ts == kTabRepeated) PMSST_NRF1(NV, kTabRepeated);      \
    else if (ts == kTabDense) PMSST_NRF1(NV, kTabDense);       \
    else PMSST_NRF1(NV, kTabAny);                              \
  } while (0)
  switch (geo.nv) {
    case 1: PMSST_NRF(1); break;
    case 2: PMSST_NRF(2); break;
    case 3: PMSST_NRF(3); break;
    case 4: PMSST_NRF(4); break;
    default: return fail(PMSST_EINVAL, "rms_norm_rotary_forward: internal geometry error");
  }
#undef PMSST_NRF
#undef PMSST_NRF1
  return check_launch("norm_rot_fwd_kernel");
}

// nt = 1 or 2 tensors of one shape; dgamma[nt * dim] holds tensor t's dgamma at t * dim.
template <typename T, typename TG>
int launch_norm_rot_bwd(int nt, const void* const* dy, const void* const* x, const float* const* inv_norm,
                        const void* const* gamma, const void* cosv, const void* sinv, void* const* dx, void* dgamma,
                        int gamma_dtype, const NormRotArgs& a, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  const bool empty = a.batch * a.seq * a.heads == 0;
  constexpr int kVec = 16 / sizeof(T);
  NormRotIO<T, TG> io{};
  RowGeom geo{};
  PMSST_REQUIRE(dgamma != nullptr, "rms_norm_rotary_backward: null pointer");
  for (int t = 0; t < nt; ++t) {
    PMSST_REQUIRE(gamma[t] && (empty || (dy[t] && x[t] && inv_norm[t] && cosv && sinv && dx[t])),
                  "rms_norm_rotary_backward: null pointer");
    const void* ptrs[] = {dy[t], x[t], gamma[t], dx[t]};
    const size_t sizes[] = {sizeof(T), sizeof(T), sizeof(TG), sizeof(T)};
    const int rc = norm_rot_check("rms_norm_rotary_backward", a, kVec, ptrs, sizes, 4, &geo);
    if (rc != PMSST_OK) return rc;
    io.dy[t] = static_cast<const T*>(dy[t]);
    io.x[t] = static_cast<const T*>(x[t]);
    io.inv[t] = const_cast<float*>(inv_norm[t]);
    io.gamma[t] = static_cast<const TG*>(gamma[t]);
    io.out[t] = static_cast<T*>(dx[t]);
  }
  int rc = PMSST_OK;
  const int64_t rows = a.batch * a.seq * a.heads;
  const size_t need = row_bwd_workspace(nt * a.dim);
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(PMSST_EWORKSPACE, "rms_norm_rotary_backward: workspace of %zu bytes needed", need);
  }
  float* partial = static_cast<float*>(workspace);
  const int parts = row_bwd_parts(rows, geo.tpr_log2);
  io.per_tensor = parts;
  const float scale = sqrtf(static_cast<float>(a.dim));
  const FastDiv fh(static_cast<uint32_t>(a.heads > 0 ? a.heads : 1)), fs(static_cast<uint32_t>(a.seq > 0 ? a.seq : 1));
  const TableRef tab{a.cs_seq, a.cs_pair};
  const size_t shmem = sizeof(float) * (kRowBwdThreads / kWave) * static_cast<size_t>(a.dim);
  if (parts > 0) {
    const int ts = table_mode(cosv, sinv, a.cs_seq, a.cs_pair, kVec, sizeof(T));
#define PMSST_NRB1(NV, TS)                                                                                           \
  hipLaunchKernelGGL((norm_rot_bwd_kernel<T, TG, kVec, NV, TS>), dim3(parts * nt), dim3(kRowBwdThreads), shmem,   \
                     stream, io, static_cast<const T*>(cosv), static_cast<const T*>(sinv), partial,                   \
                     static_cast<int>(nt * a.dim), rows, geo.tpr_log2, scale, fh, fs, tab)
#define PMSST_NRB(NV)                                          \
  do {                                                         \
    if (ts == kTabRepeated) PMSST_NRB1(NV, kTabRepeated);      \
    else if (ts == kTabDense) PMSST_NRB1(NV, kTabDense);       \
    else PMSST_NRB1(NV, kTabAny);                              \
  } while (0)
    switch (geo.nv) {
      case 1: PMSST_NRB(1); break;
      case 2: PMSST_NRB(2); break;
      case 3: PMSST_NRB(3); break;
      case 4: PMSST_NRB(4); break;
      default: return fail(PMSST_EINVAL, "rms_norm_rotary_backward: internal geometry error");
    }
#undef PMSST_NRB
#undef PMSST_NRB1
    rc = check_launch("norm_rot_bwd_kernel");
    if (rc != PMSST_OK) return rc;
  }
  return launch_col_sum(partial, parts, static_cast<int>(nt * a.dim), dgamma, gamma_dtype, stream);
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

int pmsst_rotary_forward(const void* t, const int64_t* t_strides, const void* cos, const void* sin, void* out,
                         const int64_t* out_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                         int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream) {
  return with_dtype(dtype, "rotary_forward", [&](auto tag) {
    using T = decltype(tag);
    return launch_rotary<T>(t, t_strides, cos, sin, out, out_strides, batch, seq, heads, dim, cs_stride_seq,
                            cs_stride_pair, false, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rotary_backward(const void* grad_out, const int64_t* grad_out_strides, const void* cos, const void* sin,
                          void* grad_t, const int64_t* grad_t_strides, int64_t batch, int64_t seq, int64_t heads,
                          int64_t dim, int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream) {
  return with_dtype(dtype, "rotary_backward", [&](auto tag) {
    using T = decltype(tag);
    return launch_rotary<T>(grad_out, grad_out_strides, cos, sin, grad_t, grad_t_strides, batch, seq, heads, dim,
                            cs_stride_seq, cs_stride_pair, true, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rotary_qkv_forward(const void* q, const void* k, const void* v, const int64_t* in_strides, const void* cos,
                             const void* sin, void* q_out, void* k_out, void* v_out, const int64_t* out_strides,
                             int64_t batch, int64_t seq, int64_t heads, int64_t dim, int64_t cs_stride_seq,
                             int64_t cs_stride_pair, int dtype, void* stream) {
  return with_dtype(dtype, "rotary_qkv_forward", [&](auto tag) {
    using T = decltype(tag);
    const void* ins[] = {q, k, v};
    void* outs[] = {q_out, k_out, v_out};
    const int64_t* sis[] = {in_strides ? in_strides : nullptr, in_strides ? in_strides + 3 : nullptr,
                            in_strides ? in_strides + 6 : nullptr};
    const int64_t* sos[] = {out_strides ? out_strides : nullptr, out_strides ? out_strides + 3 : nullptr,
                            out_strides ? out_strides + 6 : nullptr};
    return launch_rotary_parts<T>("rotary_qkv_forward", 3, 2, ins, sis, cos, sin, outs, sos, batch, seq, heads, dim,
                                  cs_stride_seq, cs_stride_pair, false, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rotary_qkv_backward(const void* grad_q, const void* grad_k, const void* grad_v, const int64_t* grad_strides,
                              const void* cos, const void* sin, void* grad_q_in, void* grad_k_in, void* grad_v_in,
                              const int64_t* grad_in_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                              int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream) {
  return with_dtype(dtype, "rotary_qkv_backward", [&](auto tag) {
    using T = decltype(tag);
    const void* ins[] = {grad_q, grad_k, grad_v};
    void* outs[] = {grad_q_in, grad_k_in, grad_v_in};
    const int64_t* sis[] = {grad_strides ? grad_strides : nullptr, grad_strides ? grad_strides + 3 : nullptr,
                            grad_strides ? grad_strides + 6 : nullptr};
    const int64_t* sos[] = {grad_in_strides ? grad_in_strides : nullptr, grad_in_strides ? grad_in_strides + 3 : nullptr,
                            grad_in_strides ? grad_in_strides + 6 : nullptr};
    return launch_rotary_parts<T>("rotary_qkv_backward", 3, 2, ins, sis, cos, sin, outs, sos, batch, seq, heads, dim,
                                  cs_stride_seq, cs_stride_pair, true, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_rotary_forward(const void* x, const void* gamma, const void* cos, const void* sin, void* out,
                                  float* inv_norm, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                                  int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, int gamma_dtype,
                                  void* stream) {
  if (gamma_dtype != dtype && gamma_dtype != PMSST_F32) {
    return fail(PMSST_EDTYPE, "rms_norm_rotary_forward: gamma dtype must equal x dtype or be fp32");
  }
  const NormRotArgs a{batch, seq, heads, dim, cs_stride_seq, cs_stride_pair};
  return with_dtype(dtype, "rms_norm_rotary_forward", [&](auto tag) {
    using T = decltype(tag);
    const void* xs[] = {x};
    const void* gs[] = {gamma};
    void* os[] = {out};
    float* is[] = {inv_norm};
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_fwd<T, float>(1, xs, gs, cos, sin, os, is, a, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_fwd<T, T>(1, xs, gs, cos, sin, os, is, a, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_rotary_pair_forward(const void* x0, const void* x1, const void* gamma0, const void* gamma1,
                                       const void* cos, const void* sin, void* out0, void* out1, float* inv_norm0,
                                       float* inv_norm1, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                                       int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, int gamma_dtype,
                                       void* stream) {
  if (gamma_dtype != dtype && gamma_dtype != PMSST_F32) {
    return fail(PMSST_EDTYPE, "rms_norm_rotary_forward: gamma dtype must equal x dtype or be fp32");
  }
  const NormRotArgs a{batch, seq, heads, dim, cs_stride_seq, cs_stride_pair};
  return with_dtype(dtype, "rms_norm_rotary_forward", [&](auto tag) {
    using T = decltype(tag);
    const void* xs[] = {x0, x1};
    const void* gs[] = {gamma0, gamma1};
    void* os[] = {out0, out1};
    float* is[] = {inv_norm0, inv_norm1};
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_fwd<T, float>(2, xs, gs, cos, sin, os, is, a, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_fwd<T, T>(2, xs, gs, cos, sin, os, is, a, static_cast<hipStream_t>(stream));
  });
}

size_t pmsst_rms_norm_rotary_backward_workspace_size(int64_t rows, int64_t dim) {
  (void)rows;
  return dim > 0 ? row_bwd_workspace(dim) : 0;
}

int pmsst_rms_norm_rotary_backward(const void* grad_out, const void* x, const float* inv_norm, const void* gamma,
                                   const void* cos, const void* sin, void* grad_x, void* grad_gamma, int64_t batch,
                                   int64_t seq, int64_t heads, int64_t dim, int64_t cs_stride_seq,
                                   int64_t cs_stride_pair, int dtype, int gamma_dtype, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (gamma_dtype != dtype && gamma_dtype != PMSST_F32) {
    return fail(PMSST_EDTYPE, "rms_norm_rotary_backward: gamma dtype must equal x dtype or be fp32");
  }
  const NormRotArgs a{batch, seq, heads, dim, cs_stride_seq, cs_stride_pair};
  return with_dtype(dtype, "rms_norm_rotary_backward", [&](auto tag) {
    using T = decltype(tag);
    const void* dys[] = {grad_out};
    const void* xs[] = {x};
    const float* is[] = {inv_norm};
    const void* gs[] = {gamma};
    void* dxs[] = {grad_x};
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_bwd<T, float>(1, dys, xs, is, gs, cos, sin, dxs, grad_gamma, PMSST_F32, a, workspace,
                                           workspace_bytes, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_bwd<T, T>(1, dys, xs, is, gs, cos, sin, dxs, grad_gamma, dtype, a, workspace,
                                     workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

int pmsst_rms_norm_rotary_pair_backward(const void* grad_out0, const void* grad_out1, const void* x0, const void* x1,
                                        const float* inv_norm0, const float* inv_norm1, const void* gamma0,
                                        const void* gamma1, const void* cos, const void* sin, void* grad_x0,
                                        void* grad_x1, void* grad_gamma, int64_t batch, int64_t seq, int64_t heads,
                                        int64_t dim, int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype,
                                        int gamma_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (gamma_dtype != dtype && gamma_dtype != PMSST_F32) {
    return fail(PMSST_EDTYPE, "rms_norm_rotary_backward: gamma dtype must equal x dtype or be fp32");
  }
  const NormRotArgs a{batch, seq, heads, dim, cs_stride_seq, cs_stride_pair};
  return with_dtype(dtype, "rms_norm_rotary_backward", [&](auto tag) {
    using T = decltype(tag);
    const void* dys[] = {grad_out0, grad_out1};
    const void* xs[] = {x0, x1};
    const float* is[] = {inv_norm0, inv_norm1};
    const void* gs[] = {gamma0, gamma1};
    void* dxs[] = {grad_x0, grad_x1};
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_bwd<T, float>(2, dys, xs, is, gs, cos, sin, dxs, grad_gamma, PMSST_F32, a, workspace,
                                           workspace_bytes, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_bwd<T, T>(2, dys, xs, is, gs, cos, sin, dxs, grad_gamma, dtype, a, workspace,
                                     workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
