// Rotary embedding on bnhd q/k, and the fused q/k RMSNorm + rotary + cast.
//
// Rotary is a pure stream: each lane moves one 16-byte pack (VEC elements,
// VEC/2 adjacent pairs) per step.  The pack's (batch, position, head, element)
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
constexpr int kNormRotThreads = 256;

struct TableRef {
  int64_t stride_seq;
  int64_t stride_pair;
};

// Element strides of a [B, N, H, D] view whose last axis is contiguous.
struct BnhStrides {
  int64_t b, n, h;
};

template <typename T, int VEC, bool INVERSE>
__global__ __launch_bounds__(kRotThreads) void rotary_kernel(const T* __restrict__ in, const T* __restrict__ cosv,
                                                             const T* __restrict__ sinv, T* __restrict__ out,
                                                             uint32_t total_packs, FastDiv packs_per_token,
                                                             FastDiv seq, FastDiv dim, TableRef tab, BnhStrides si,
                                                             BnhStrides so) {
  for (uint32_t i = blockIdx.x * kRotThreads + threadIdx.x; i < total_packs; i += gridDim.x * kRotThreads) {
    const uint32_t tok = packs_per_token.div(i);
    const uint32_t e = (i - tok * packs_per_token.d) * VEC;  // element offset inside the token
    const uint32_t b = seq.div(tok);
    const uint32_t n = tok - b * seq.d;
    const uint32_t h = dim.div(e);
    const uint32_t d = e - h * dim.d;
    const uint32_t p0 = d >> 1;
    float v[VEC];
    load_pack<T, VEC>(in + b * si.b + n * si.n + h * si.h + d, v);
    const T* cr = cosv + n * tab.stride_seq;
    const T* sr = sinv + n * tab.stride_seq;
#pragma unroll
    for (int j = 0; j < VEC / 2; ++j) {
      const float c = to_f32(cr[(p0 + j) * tab.stride_pair]);
      const float s = to_f32(sr[(p0 + j) * tab.stride_pair]);
      const float ev = v[2 * j], ov = v[2 * j + 1];
      if (INVERSE) {
        v[2 * j] = ev * c + ov * s;
        v[2 * j + 1] = ov * c - ev * s;
      } else {
        v[2 * j] = ev * c - ov * s;
        v[2 * j + 1] = ov * c + ev * s;
      }
    }
    store_pack<T, VEC>(out + b * so.b + n * so.n + h * so.h + d, v);
  }
}

template <typename T>
int launch_rotary(const void* in, const int64_t* in_strides, const void* cosv, const void* sinv, void* out,
                  const int64_t* out_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim, int64_t cs_seq,
                  int64_t cs_pair, bool inverse, hipStream_t stream) {
  const char* op = inverse ? "rotary_backward" : "rotary_forward";
  PMSST_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0 && dim > 0 && dim % 2 == 0,
                "%s: bad shape [%lld, %lld, %lld, %lld]", op, (long long)batch, (long long)seq, (long long)heads,
                (long long)dim);
  const int64_t total = batch * seq * heads * dim;
  if (total == 0) return PMSST_OK;
  PMSST_REQUIRE(in && cosv && sinv && out, "%s: null pointer", op);
  const BnhStrides dense{seq * heads * dim, heads * dim, dim};
  const BnhStrides si = in_strides ? BnhStrides{in_strides[0], in_strides[1], in_strides[2]} : dense;
  const BnhStrides so = out_strides ? BnhStrides{out_strides[0], out_strides[1], out_strides[2]} : dense;
  PMSST_REQUIRE(si.b >= 0 && si.n >= 0 && si.h >= 0 && so.b >= 0 && so.n >= 0 && so.h >= 0, "%s: negative stride",
                op);
  int vec = 16 / sizeof(T);
  auto aligned = [&](int v) {
    bool ok = dim % v == 0 && reinterpret_cast<uintptr_t>(in) % (v * sizeof(T)) == 0 &&
              reinterpret_cast<uintptr_t>(out) % (v * sizeof(T)) == 0;
    for (int64_t st : {si.b, si.n, si.h, so.b, so.n, so.h}) ok = ok && st % v == 0;
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
  const int64_t blocks64 = (packs + kRotThreads - 1) / kRotThreads;
  const int blocks = static_cast<int>(blocks64 < 65536 ? blocks64 : 65536);
  const T* pin = static_cast<const T*>(in);
  const T* pc = static_cast<const T*>(cosv);
  const T* ps = static_cast<const T*>(sinv);
  T* po = static_cast<T*>(out);
  const uint32_t np = static_cast<uint32_t>(packs);
#define PMSST_ROT(VEC, INV)                                                                                     \
  hipLaunchKernelGGL((rotary_kernel<T, VEC, INV>), dim3(blocks), dim3(kRotThreads), 0, stream, pin, pc, ps, po, \
                     np, ppt, fseq, fdim, tab, si, so)
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
  return check_launch("rotary_kernel");
}

// ------------------------------------------------------------------ fused q/k RMSNorm + rotary

template <typename T, typename TG, int VEC, int NV>
__global__ __launch_bounds__(kNormRotThreads) void norm_rot_fwd_kernel(
    const T* __restrict__ x, const TG* __restrict__ gamma, const T* __restrict__ cosv, const T* __restrict__ sinv,
    T* __restrict__ out, float* __restrict__ inv_norm, int64_t rows, int tpr_log2, float scale, FastDiv heads,
    FastDiv seq, TableRef tab) {
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

  for (int64_t base = static_cast<int64_t>(blockIdx.x) * rows_per_block; base < rows;
       base += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t row = base + wave * rows_per_wave + slot;
    const bool valid = row < rows;
    float xv[NV][VEC];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (valid) {
        load_pack<T, VEC>(x + row * dim + (v * tpr + t) * VEC, xv[v]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[v][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += xv[v][i] * xv[v][i];
    }
    ss = group_sum(ss, tpr);
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1.0e-12f);
    if (valid) {
      const uint32_t n = seq.mod(heads.div(static_cast<uint32_t>(row)));
      const T* cr = cosv + n * tab.stride_seq;
      const T* sr = sinv + n * tab.stride_seq;
      const float s = inv * scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int col = (v * tpr + t) * VEC;
        float o[VEC];
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          const int p = col / 2 + j;
          const float c = to_f32(cr[p * tab.stride_pair]);
          const float sn = to_f32(sr[p * tab.stride_pair]);
          const float ev = xv[v][2 * j] * s * g[v][2 * j];
          const float ov = xv[v][2 * j + 1] * s * g[v][2 * j + 1];
          o[2 * j] = ev * c - ov * sn;
          o[2 * j + 1] = ov * c + ev * sn;
        }
        store_pack<T, VEC>(out + row * dim + col, o);
      }
      if (t == 0) inv_norm[row] = inv;
    }
  }
}

template <typename T, typename TG, int VEC, int NV>
__global__ __launch_bounds__(kRowBwdThreads) void norm_rot_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ x, const float* __restrict__ inv_norm,
    const TG* __restrict__ gamma, const T* __restrict__ cosv, const T* __restrict__ sinv, T* __restrict__ dx,
    float* __restrict__ partial, int64_t rows, int tpr_log2, float scale, FastDiv heads, FastDiv seq,
    TableRef tab) {
  extern __shared__ float red[];
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

  for (int64_t base = static_cast<int64_t>(blockIdx.x) * rows_per_block; base < rows;
       base += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t row = base + wave * rows_per_wave + slot;
    const bool valid = row < rows;
    float gr[NV][VEC], n[NV][VEC];
    float dot = 0.f;
    const float inv = valid ? inv_norm[row] : 0.f;
    const float ns = inv * scale;
    const uint32_t pos = valid ? seq.mod(heads.div(static_cast<uint32_t>(row))) : 0u;
    const T* cr = cosv + pos * tab.stride_seq;
    const T* sr = sinv + pos * tab.stride_seq;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int col = (v * tpr + t) * VEC;
      if (valid) {
        float d[VEC];
        load_pack<T, VEC>(dy + row * dim + col, d);
        load_pack<T, VEC>(x + row * dim + col, n[v]);
#pragma unroll
        for (int j = 0; j < VEC / 2; ++j) {
          const int p = col / 2 + j;
          const float c = to_f32(cr[p * tab.stride_pair]);
          const float sn = to_f32(sr[p * tab.stride_pair]);
          gr[v][2 * j] = d[2 * j] * c + d[2 * j + 1] * sn;
          gr[v][2 * j + 1] = d[2 * j + 1] * c - d[2 * j] * sn;
        }
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) gr[v][i] = n[v][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        n[v][i] *= ns;
        dot += gr[v][i] * g[v][i] * n[v][i];
      }
    }
    dot = group_sum(dot, tpr);
    if (valid) {
      const float dot_s = dot * inv_scale;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          o[i] = inv * (gr[v][i] * g[v][i] * scale - n[v][i] * dot_s);
          acc[v][i] += gr[v][i] * n[v][i];
        }
        store_pack<T, VEC>(dx + row * dim + (v * tpr + t) * VEC, o);
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
    partial[static_cast<int64_t>(blockIdx.x) * dim + c] = s;
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

template <typename T, typename TG>
int launch_norm_rot_fwd(const void* x, const void* gamma, const void* cosv, const void* sinv, void* out,
                        float* inv_norm, const NormRotArgs& a, hipStream_t stream) {
  if (a.batch * a.seq * a.heads == 0 && a.dim > 0) return PMSST_OK;
  PMSST_REQUIRE(x && gamma && cosv && sinv && out && inv_norm, "rms_norm_rotary_forward: null pointer");
  constexpr int kVec = 16 / sizeof(T);
  const void* ptrs[] = {x, gamma, out};
  const size_t sizes[] = {sizeof(T), sizeof(TG), sizeof(T)};
  RowGeom geo;
  int rc = norm_rot_check("rms_norm_rotary_forward", a, kVec, ptrs, sizes, 3, &geo);
  if (rc != PMSST_OK) return rc;
  const int64_t rows = a.batch * a.seq * a.heads;
  if (rows == 0) return PMSST_OK;
  const int rpb = (kWave >> geo.tpr_log2) * (kNormRotThreads / kWave);
  const int64_t blocks64 = (rows + rpb - 1) / rpb;
  const int blocks = static_cast<int>(blocks64 < 65536 ? blocks64 : 65536);
  const float scale = sqrtf(static_cast<float>(a.dim));
  const FastDiv fh(static_cast<uint32_t>(a.heads)), fs(static_cast<uint32_t>(a.seq));
  const TableRef tab{a.cs_seq, a.cs_pair};
#define PMSST_NRF(NV)                                                                                        \
  hipLaunchKernelGGL((norm_rot_fwd_kernel<T, TG, kVec, NV>), dim3(blocks), dim3(kNormRotThreads), 0, stream, \
                     static_cast<const T*>(x), static_cast<const TG*>(gamma), static_cast<const T*>(cosv),    \
                     static_cast<const T*>(sinv), static_cast<T*>(out), inv_norm, rows, geo.tpr_log2, scale, \
                     fh, fs, tab)
  switch (geo.nv) {
    case 1: PMSST_NRF(1); break;
    case 2: PMSST_NRF(2); break;
    case 3: PMSST_NRF(3); break;
    case 4: PMSST_NRF(4); break;
    default: return fail(PMSST_EINVAL, "rms_norm_rotary_forward: internal geometry error");
  }
#undef PMSST_NRF
  return check_launch("norm_rot_fwd_kernel");
}

template <typename T, typename TG>
int launch_norm_rot_bwd(const void* dy, const void* x, const float* inv_norm, const void* gamma, const void* cosv,
                        const void* sinv, void* dx, void* dgamma, int gamma_dtype, const NormRotArgs& a,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const bool empty = a.batch * a.seq * a.heads == 0;
  PMSST_REQUIRE(dgamma && gamma && (empty || (dy && x && inv_norm && cosv && sinv && dx)),
                "rms_norm_rotary_backward: null pointer");
  constexpr int kVec = 16 / sizeof(T);
  const void* ptrs[] = {dy, x, gamma, dx};
  const size_t sizes[] = {sizeof(T), sizeof(T), sizeof(TG), sizeof(T)};
  RowGeom geo;
  int rc = norm_rot_check("rms_norm_rotary_backward", a, kVec, ptrs, sizes, 4, &geo);
  if (rc != PMSST_OK) return rc;
  const int64_t rows = a.batch * a.seq * a.heads;
  const size_t need = row_bwd_workspace(a.dim);
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(PMSST_EWORKSPACE, "rms_norm_rotary_backward: workspace of %zu bytes needed", need);
  }
  float* partial = static_cast<float*>(workspace);
  const int parts = row_bwd_parts(rows, geo.tpr_log2);
  const float scale = sqrtf(static_cast<float>(a.dim));
  const FastDiv fh(static_cast<uint32_t>(a.heads > 0 ? a.heads : 1)), fs(static_cast<uint32_t>(a.seq > 0 ? a.seq : 1));
  const TableRef tab{a.cs_seq, a.cs_pair};
  const size_t shmem = sizeof(float) * (kRowBwdThreads / kWave) * static_cast<size_t>(a.dim);
  if (parts > 0) {
#define PMSST_NRB(NV)                                                                                          \
  hipLaunchKernelGGL((norm_rot_bwd_kernel<T, TG, kVec, NV>), dim3(parts), dim3(kRowBwdThreads), shmem, stream, \
                     static_cast<const T*>(dy), static_cast<const T*>(x), inv_norm, static_cast<const TG*>(gamma), \
                     static_cast<const T*>(cosv), static_cast<const T*>(sinv), static_cast<T*>(dx), partial,     \
                     rows, geo.tpr_log2, scale, fh, fs, tab)
    switch (geo.nv) {
      case 1: PMSST_NRB(1); break;
      case 2: PMSST_NRB(2); break;
      case 3: PMSST_NRB(3); break;
      case 4: PMSST_NRB(4); break;
      default: return fail(PMSST_EINVAL, "rms_norm_rotary_backward: internal geometry error");
    }
#undef PMSST_NRB
    rc = check_launch("norm_rot_bwd_kernel");
    if (rc != PMSST_OK) return rc;
  }
  return launch_col_sum(partial, parts, static_cast<int>(a.dim), dgamma, gamma_dtype, stream);
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
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_fwd<T, float>(x, gamma, cos, sin, out, inv_norm, a, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_fwd<T, T>(x, gamma, cos, sin, out, inv_norm, a, static_cast<hipStream_t>(stream));
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
    if (gamma_dtype == PMSST_F32) {
      return launch_norm_rot_bwd<T, float>(grad_out, x, inv_norm, gamma, cos, sin, grad_x, grad_gamma, PMSST_F32, a,
                                           workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    }
    return launch_norm_rot_bwd<T, T>(grad_out, x, inv_norm, gamma, cos, sin, grad_x, grad_gamma, dtype, a, workspace,
                                     workspace_bytes, static_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
