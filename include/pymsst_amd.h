/*
 * pymsst_amd: C ABI of the MI355X (gfx950) fused RoFormer layer kernels.
 *
 * Each entry point replaces one op of the reference's pybind11 extension
 * (baicai-1145/pymsst src/pymsst/training/cuda/fused_band_split.cpp:731-753,
 * kernels in fused_band_split.cu).  The cited file:line is the reference
 * wrapper whose tensor contract the entry point implements.
 *
 * Conventions (all entry points):
 *  - Plain device pointers and sizes; every tensor is dense and row-major
 *    unless a stride argument says otherwise.  Storage dtype codes are
 *    PMSST_F32 / PMSST_F16 / PMSST_BF16; arithmetic is fp32.
 *  - Outputs are caller-allocated.  The library never allocates device
 *    memory: reductions use a caller-provided workspace whose size the
 *    matching *_workspace_size() reports for the current device.
 *  - Work is enqueued on `stream` (a hipStream_t) and never synchronised.
 *  - Returns PMSST_OK (0) or a negative code; pmsst_last_error() then holds
 *    a message for the calling thread.
 *  - Reductions over rows (dgamma, dW, dbias) are deterministic: fixed
 *    partition, fixed summation order, no floating-point atomics.
 */
#ifndef PYMSST_AMD_H
#define PYMSST_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { PMSST_F32 = 0, PMSST_F16 = 1, PMSST_BF16 = 2 };
/* Activation codes (mask-MLP hidden layer: Linear -> tanh, fr.py:340,538). */
enum { PMSST_ACT_NONE = 0, PMSST_ACT_TANH = 1 };
enum {
  PMSST_OK = 0,
  PMSST_EINVAL = -1,     /* bad shape, size, pointer or alignment */
  PMSST_EDTYPE = -2,     /* unsupported dtype combination */
  PMSST_ELAUNCH = -3,    /* HIP launch failure */
  PMSST_EWORKSPACE = -4  /* workspace missing or too small */
};

/* Message of the last failing call on this thread ("" if none). */
const char* pmsst_last_error(void);
/* ABI revision of this header; bumped on any signature change. */
int pmsst_abi_version(void);

/* ------------------------------------------------------------------ RMSNorm
 * y = x / max(||x||_2, 1e-12) * sqrt(dim) * gamma over the last axis of
 * x[rows, dim].  inv_norm[rows] (fp32) = 1 / max(||x||, 1e-12).
 * `normed` may be NULL: the normalised copy is then not written (the
 * saved-input backward below recomputes it).
 */

/* fused_band_split.cpp:434-444 rms_norm_forward (.cu:1210-1249): x, gamma, out, normed in `dtype`. */
int pmsst_rms_norm_forward(const void* x, const void* gamma, void* out, void* normed, float* inv_norm,
                           int64_t rows, int64_t dim, int dtype, void* stream);
/* fused_band_split.cpp:467-477 rms_norm_forward_fp32_gamma (.cu:1399-1438): gamma fp32, rest `dtype`. */
int pmsst_rms_norm_forward_fp32_gamma(const void* x, const float* gamma, void* out, void* normed,
                                      float* inv_norm, int64_t rows, int64_t dim, int dtype, void* stream);
/* fused_band_split.cpp:500-510 rms_norm_forward_mixed (.cu:1588-1627): x `dtype`, gamma/out/normed fp32. */
int pmsst_rms_norm_forward_mixed(const void* x, const float* gamma, float* out, float* normed, float* inv_norm,
                                 int64_t rows, int64_t dim, int dtype, void* stream);

/* Bytes of workspace every RMSNorm backward entry point needs for `dim`. */
size_t pmsst_rms_norm_backward_workspace_size(int64_t rows, int64_t dim);

/* fused_band_split.cpp:446-465 rms_norm_backward (.cu:1251-1397):
 * grad_out, normed, gamma, grad_x, grad_gamma in `dtype`. */
int pmsst_rms_norm_backward(const void* grad_out, const void* normed, const float* inv_norm, const void* gamma,
                            void* grad_x, void* grad_gamma, int64_t rows, int64_t dim, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream);
/* fused_band_split.cpp:479-498 rms_norm_backward_fp32_gamma (.cu:1440-1586): gamma/grad_gamma fp32. */
int pmsst_rms_norm_backward_fp32_gamma(const void* grad_out, const void* normed, const float* inv_norm,
                                       const float* gamma, void* grad_x, float* grad_gamma, int64_t rows,
                                       int64_t dim, int dtype, void* workspace, size_t workspace_bytes,
                                       void* stream);
/* fused_band_split.cpp:512-534 rms_norm_backward_mixed (.cu:1629-1775): grad_out/normed/gamma/grad_gamma
 * fp32, grad_x in `x_dtype` (the dtype of the forward input, the reference's x_meta). */
int pmsst_rms_norm_backward_mixed(const float* grad_out, const float* normed, const float* inv_norm,
                                  const float* gamma, void* grad_x, float* grad_gamma, int64_t rows, int64_t dim,
                                  int x_dtype, void* workspace, size_t workspace_bytes, void* stream);
/* Saved-input backward (no reference counterpart; same algebra as .cu:1251-1315 with
 * normed = x * inv_norm * sqrt(dim) recomputed): lets the forward skip writing `normed`.
 * grad_out, x, grad_x in `dtype`; gamma/grad_gamma in `gamma_dtype` (`dtype` or PMSST_F32). */
int pmsst_rms_norm_backward_from_input(const void* grad_out, const void* x, const float* inv_norm,
                                       const void* gamma, void* grad_x, void* grad_gamma, int64_t rows,
                                       int64_t dim, int dtype, int gamma_dtype, void* workspace,
                                       size_t workspace_bytes, void* stream);
/* No reference counterpart: pmsst_rms_norm_backward_from_input that allocates nothing and takes no
 * workspace, for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Its dgamma partials live in a static 4 MiB device
 * array per GPU, so dim <= 1024 (larger dims return PMSST_EINVAL); calls that overlap on one GPU
 * (concurrent streams or threads) race on that array. */
int pmsst_rms_norm_backward_from_input_noalloc(const void* grad_out, const void* x, const float* inv_norm,
                                               const void* gamma, void* grad_x, void* grad_gamma, int64_t rows,
                                               int64_t dim, int dtype, int gamma_dtype, void* stream);

/* ------------------------------------------------------------------ rotary
 * t[batch, seq, heads, dim] (bnhd shape); cos/sin[seq, dim/2] addressed as
 * cos[n * cs_stride_seq + p * cs_stride_pair] (the reference's [1,N,1,D/2]
 * table; strides let the caller pass the cos[..., ::2] view without a copy).
 * Pair p = (t[2p], t[2p+1]) is rotated by angle (n, p).
 * *_strides: host int64[3] element strides of the batch, seq and head axes of
 * that tensor (its last axis is contiguous), or NULL for the dense bnhd layout.
 * They let q/k be read straight from a fused qkv buffer and written in the
 * [B, H, N, D] layout attention consumes (the reference copies with .contiguous()).
 * With cs_stride_pair == 2 (the [..., ::2] view of a pair-repeated table) the
 * kernels read the table rows 16 bytes at a time, so every element
 * cos[n * cs_stride_seq + k], k < dim, must be readable (as it is for such a view).
 */

/* fused_band_split.cpp:390-410 rotary_forward (.cu:1076-1101,1130-1168). */
int pmsst_rotary_forward(const void* t, const int64_t* t_strides, const void* cos, const void* sin, void* out,
                         const int64_t* out_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                         int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream);
/* fused_band_split.cpp:412-432 rotary_backward (.cu:1103-1128,1170-1208): transpose rotation. */
int pmsst_rotary_backward(const void* grad_out, const int64_t* grad_out_strides, const void* cos, const void* sin,
                          void* grad_t, const int64_t* grad_t_strides, int64_t batch, int64_t seq, int64_t heads,
                          int64_t dim, int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream);

/* No reference counterpart: q, k and v of one fused qkv projection in one launch (the
 * reference's rotary patch, fr.py:710-732, rotates q and k in two calls and leaves the split
 * and the gradient stacking of qkv_to_bnhd to torch).  q and k are rotated, v is copied.
 * in_strides / out_strides: three {batch, seq, head} element-stride triples (q, k, v order;
 * NULL = dense bnhd).  The backward applies the transpose rotation to grad_q / grad_k and copies
 * grad_v, typically into the three slices of the qkv gradient. */
int pmsst_rotary_qkv_forward(const void* q, const void* k, const void* v, const int64_t* in_strides, const void* cos,
                             const void* sin, void* q_out, void* k_out, void* v_out, const int64_t* out_strides,
                             int64_t batch, int64_t seq, int64_t heads, int64_t dim, int64_t cs_stride_seq,
                             int64_t cs_stride_pair, int dtype, void* stream);
int pmsst_rotary_qkv_backward(const void* grad_q, const void* grad_k, const void* grad_v, const int64_t* grad_strides,
                              const void* cos, const void* sin, void* grad_q_in, void* grad_k_in, void* grad_v_in,
                              const int64_t* grad_in_strides, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                              int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, void* stream);

/* Fused q/k RMSNorm over the head dim + rotary + cast (no reference counterpart; composition of
 * .cu:1399-1438 and .cu:1076-1101 with no intermediate round trip).  x/out/cos/sin in `dtype`,
 * gamma[dim] in `gamma_dtype`; writes inv_norm[batch*seq*heads]. */
int pmsst_rms_norm_rotary_forward(const void* x, const void* gamma, const void* cos, const void* sin, void* out,
                                  float* inv_norm, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                                  int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, int gamma_dtype,
                                  void* stream);
/* Backward of the fused op from the saved input x and inv_norm. */
size_t pmsst_rms_norm_rotary_backward_workspace_size(int64_t rows, int64_t dim);
int pmsst_rms_norm_rotary_backward(const void* grad_out, const void* x, const float* inv_norm, const void* gamma,
                                   const void* cos, const void* sin, void* grad_x, void* grad_gamma, int64_t batch,
                                   int64_t seq, int64_t heads, int64_t dim, int64_t cs_stride_seq,
                                   int64_t cs_stride_pair, int dtype, int gamma_dtype, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* The two ops above on q and k together (two tensors of one shape, each with its own gamma and
 * inv_norm) in one launch each way: this build's addition, no reference counterpart (the reference
 * calls rotary_forward / rotary_backward once per tensor, fr.py:722-727).  grad_gamma[2 * dim] holds
 * q's dgamma, then k's; the workspace is pmsst_rms_norm_rotary_backward_workspace_size(rows, 2 * dim). */
int pmsst_rms_norm_rotary_pair_forward(const void* x0, const void* x1, const void* gamma0, const void* gamma1,
                                       const void* cos, const void* sin, void* out0, void* out1, float* inv_norm0,
                                       float* inv_norm1, int64_t batch, int64_t seq, int64_t heads, int64_t dim,
                                       int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype, int gamma_dtype,
                                       void* stream);
int pmsst_rms_norm_rotary_pair_backward(const void* grad_out0, const void* grad_out1, const void* x0, const void* x1,
                                        const float* inv_norm0, const float* inv_norm1, const void* gamma0,
                                        const void* gamma1, const void* cos, const void* sin, void* grad_x0,
                                        void* grad_x1, void* grad_gamma, int64_t batch, int64_t seq, int64_t heads,
                                        int64_t dim, int64_t cs_stride_seq, int64_t cs_stride_pair, int dtype,
                                        int gamma_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ band split
 * Ragged per-band RMSNorm + Linear (BS-RoFormer / MBR front end).  Band b spans
 * columns [off_b, off_b + I_b) of x with off = exclusive prefix sum of
 * dim_inputs; F = sum I_b.  gamma[F]; weight = band-major concatenation of the
 * per-band [O, I_b] Linear weights (sum_b O*I_b elements); bias[NB, O] or NULL;
 * out[rows, NB, O]; normed[rows, F] or NULL; inv_norm[rows, NB] fp32.
 * dim_offsets is the device copy of the NB+1 prefix sums, dim_inputs the host
 * copy of the NB widths.  1 <= O <= 512.
 */

/* fused_band_split.cpp:271-314 band_split_ragged_forward (.cu:589-739).  With equal widths it also
 * implements fused_band_split.cpp:141-170 band_split_forward (.cu:13-122): x_row_stride is then the
 * row pitch of the [M, G, I] group view. */
int pmsst_band_split_ragged_forward(const void* x, int64_t x_row_stride, const void* gamma, const void* weight,
                                    const void* bias, const int64_t* dim_offsets, const int64_t* dim_inputs,
                                    int64_t band_count, int64_t rows, int64_t out_features, void* out, void* normed,
                                    float* inv_norm, int dtype, void* stream);
/* Workspace bytes of the backward: per-row-tile dgamma partials, the per-(row, band, 64-wide
 * input chunk) dot partials and the fp32 gs * gamma of every input (0 when rows == 0; a zero-byte
 * workspace may be null). */
size_t pmsst_band_split_ragged_backward_workspace_size(int64_t rows, int64_t total_in, int64_t band_count,
                                                       int64_t out_features);
/* fused_band_split.cpp:316-363 band_split_ragged_backward (.cu:741-1003).  With equal widths it also
 * implements band_split_backward / _v2 / _v3 (fused_band_split.cpp:172-269, .cu:125-587).
 * `saved` is normed[rows, F] (saved_is_input = 0) or the forward input x[rows, F] (saved_is_input = 1,
 * normed recomputed as x * inv_norm * sqrt(I_b)).  Outputs: grad_x[rows, F], grad_gamma[F],
 * grad_weight (packed like weight), grad_bias[NB, O] or NULL.
 * Every 64-wide input chunk of every band is an independent block that computes gs = grad_out W_b
 * for its chunk in fp32 and its part of the per-row dot sum_i gs gamma n; a finish pass per
 * (rows, band) adds the parts in a fixed order and writes grad_x (the reference's form makes two
 * passes over each band instead, .cu:768-799). */
int pmsst_band_split_ragged_backward(const void* grad_out, const void* saved, int saved_is_input,
                                     const float* inv_norm, const void* gamma, const void* weight,
                                     const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                     int64_t rows, int64_t out_features, void* grad_x, void* grad_gamma,
                                     void* grad_weight, void* grad_bias, int dtype, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* The ragged band split with an fp32 input and a 16-bit projection: fused_band_split.cpp:271-363
 * band_split_ragged_forward / _backward (.cu:589-1003) called, as fr.py:827-857 does under autocast, with
 * the fp32 STFT input x (the norm, inv_norm and grad_gamma in fp32, as the reference computes them),
 * the projection's operands in `dtype` (F16 or BF16) where the stock module rounds them (RMSNorm in
 * fp32, then nn.Linear in the autocast dtype).  x[rows, x_row_stride] fp32, gamma[F] fp32, weight
 * and bias in `dtype` (packed as above); features[rows, F] (`dtype`) = x * inv_norm * sqrt(I_b) *
 * gamma, the projection's input, written for the backward; out[rows, NB, O] (`dtype`);
 * inv_norm[rows, NB] fp32. */
int pmsst_band_split_mixed_forward(const float* x, int64_t x_row_stride, const float* gamma, const void* weight,
                                   const void* bias, const int64_t* dim_offsets, const int64_t* dim_inputs,
                                   int64_t band_count, int64_t rows, int64_t out_features, void* features, void* out,
                                   float* inv_norm, int dtype, void* stream);
/* Workspace bytes of the backward below: the projection's input gradient g[rows, F] (`dtype`),
 * the per-(row, band) dots and the dgamma partials of every 16 rows (0 when rows == 0). */
size_t pmsst_band_split_mixed_backward_workspace_size(int64_t rows, int64_t total_in, int64_t band_count);
/* Backward of pmsst_band_split_mixed_forward: g = grad_out W_b rounded to `dtype` (the stock Linear's
 * input gradient), then the fp32 RMSNorm backward grad_x[rows, F] = inv (sqrt(I) g gamma - n inv
 * sum_i g gamma x) with n = x inv sqrt(I), grad_gamma[F] = sum_m g n (fp32); grad_weight = grad_out^T
 * features, grad_bias = sum_m grad_out (`dtype`; grad_bias may be NULL). */
int pmsst_band_split_mixed_backward(const void* grad_out, const float* x, int64_t x_row_stride, const void* features,
                                    const float* inv_norm, const float* gamma, const void* weight,
                                    const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                    int64_t rows, int64_t out_features, float* grad_x, float* grad_gamma,
                                    void* grad_weight, void* grad_bias, int dtype, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ grouped linear
 * fused_band_split.cpp:365-388 grouped_linear_forward (.cu:1005-1074):
 * out[m, g, :] = act(W_g x[m, g, :] + b_g) for x[rows, groups, in_features] with row pitch
 * x_row_stride (group g at column g * in_features), weight[groups, O, in_features],
 * bias[groups, O] or NULL, out[rows, groups, O].  group_offsets is the device copy of
 * the groups+1 prefix sums g * in_features.  Any O >= 1.  `activation` PMSST_ACT_TANH
 * fuses the mask-MLP hidden tanh (bands.inference_tanh, fr.py:340) into the epilogue;
 * PMSST_ACT_NONE is the reference op.
 */
int pmsst_grouped_linear_forward(const void* x, int64_t x_row_stride, const void* weight, const void* bias,
                                 const int64_t* group_offsets, int64_t groups, int64_t in_features, int64_t rows,
                                 int64_t out_features, void* out, int activation, int dtype, void* stream);
/* Workspace bytes of the grouped-linear backward: 0 (kept for the op's calling convention; the
 * workspace arguments of pmsst_grouped_linear_backward may be NULL / 0). */
size_t pmsst_grouped_linear_backward_workspace_size(int64_t rows, int64_t groups, int64_t out_features);
/* Backward of grouped_linear (the reference computes it with batched GEMMs in _FusedGroupedLinear,
 * fr.py:1042-1048): grad_out[rows, groups, O] (the gradient of the pre-activation output),
 * x[rows, groups * in_features] dense -> grad_x[rows, groups * in_features],
 * grad_weight[groups, O, in_features], grad_bias[groups, O] or NULL. */
int pmsst_grouped_linear_backward(const void* grad_out, const void* x, const void* weight,
                                  const int64_t* group_offsets, int64_t groups, int64_t in_features, int64_t rows,
                                  int64_t out_features, void* grad_x, void* grad_weight, void* grad_bias, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ mask estimator final layer
 * Per-band Linear hidden -> 2*I_b, bias, GLU.  x[rows, NB, hidden]; weight = band-major
 * concatenation of the per-band [2*I_b, hidden] weights; bias[2F] (band b at 2*off_b);
 * pre[rows, 2F] = x W^T + bias; out[rows, F] = left * sigmoid(gate).  dim_offsets is the
 * device copy of the NB+1 prefix sums of dim_inputs (host copy).
 */

/* fused_band_split.cpp:589-622 mask_estimator_final_forward and :660-693
 * mask_estimator_final_direct_forward (.cu:2283-2310, 2369-2552): both reference modes compute
 * these values; one kernel serves both. */
int pmsst_mask_estimator_final_forward(const void* x, const void* weight, const void* bias,
                                       const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                       int64_t rows, int64_t hidden, void* pre, void* out, int dtype, void* stream);
/* Workspace bytes of the backward: the [rows, 2*total] GLU derivative (0 when rows == 0; a
 * zero-byte workspace may be null). */
size_t pmsst_mask_estimator_final_backward_workspace_size(int64_t rows, int64_t total, int dtype);
/* fused_band_split.cpp:624-658 mask_estimator_final_backward and :695-729
 * mask_estimator_final_direct_backward (.cu:2312-2367, 2585-2851): grad_out[rows, F] ->
 * grad_x[rows, NB, hidden], grad_bias[2F], grad_weight (packed like weight).
 * input_activation PMSST_ACT_TANH: x is the tanh output of the mask-MLP hidden layer and
 * grad_x receives the gradient of its pre-activation, (dpre W) * (1 - x^2);
 * PMSST_ACT_NONE is the reference op. */
int pmsst_mask_estimator_final_backward(const void* grad_out, const void* x, const void* pre, const void* weight,
                                        const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                        int64_t rows, int64_t hidden, void* grad_x, void* grad_bias,
                                        void* grad_weight, int input_activation, int dtype, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ whole mask MLP (depth 2)
 * out = GLU(tanh(x_b W1_b^T + b1_b) W2_b^T + b2_b) for every band in one pass: x[rows, NB, dim],
 * w1[NB, hidden, dim], b1[NB, hidden], w2 / b2 packed as for pmsst_mask_estimator_final_forward;
 * writes pre[rows, 2F] and out[rows, F], and hidden_out[rows, NB, hidden] = tanh(...) only when
 * hidden_out is not NULL.  The pre-activation and the tanh are rounded to the storage dtype as
 * the reference's grouped Linear and inference_tanh do.  16-bit dtypes only.
 */

/* 1 when pmsst_mask_mlp_forward takes this shape: a 16-bit dtype, dim in {64, 128, 192, 256,
 * 384, 512}, hidden a multiple of 32 in [64, 2048], every I_b a positive multiple of 4. */
int pmsst_mask_mlp_supported(int64_t dim, int64_t hidden, const int64_t* dim_inputs, int64_t band_count, int dtype);
/* Host copy of the table the forward reads tanh from: entries = 32768, out[b] = the correctly rounded
 * tanh of the non-negative 16-bit pattern b of the dtype (bf16 or fp16).  No reference
 * counterpart; it lets tests check the table on the CPU. */
int pmsst_mask_mlp_tanh_table(int dtype, uint16_t* out, int64_t entries);
/* Replaces the hidden-layer loop of fr.py:332-369 (grouped Linear .cu:1005-1030 + inference_tanh)
 * followed by mask_estimator_final_forward (.cpp:589-622, .cu:2283-2310) for the depth-2 MLP. */
int pmsst_mask_mlp_forward(const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                           const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count, int64_t rows,
                           int64_t dim, int64_t hidden, void* pre, void* out, void* hidden_out, int dtype,
                           void* stream);
/* The same MLP for stem `stem` of `stems` with the mask application in its epilogue (the fusion that
 * cuda_graph.py:140-158's layout and the stock `spec * mask` product leave to two passes): instead
 * of out, writes est[b, stem, c, f, t] = spec[b, f*channels + c, t] * (out[m, 2r], out[m, 2r+1]) for
 * rows m = b*frames + t and complex rows r = f*channels + c, with the mask rounded to the storage
 * dtype first (est is 0 at f = 0 when zero_dc).  spec: complex64 [rows/frames, bins*channels, frames];
 * est: complex64 [rows/frames * stems * channels, bins, frames] (the iSTFT input), bins = sum of the
 * widths / (2 * channels).  pre and hidden_out as for pmsst_mask_mlp_forward. */
int pmsst_mask_mlp_forward_apply(const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                                 const int64_t* dim_offsets, const int64_t* dim_inputs, int64_t band_count,
                                 int64_t rows, int64_t dim, int64_t hidden, void* pre, void* hidden_out,
                                 const void* spec, void* est, int64_t frames, int64_t channels, int64_t stems,
                                 int64_t stem, int zero_dc, int dtype, void* stream);

/* ------------------------------------------------------------------ attention output gate
 * gate[m, h] = sigmoid(x[m] . W[h] + b[h]) stored in the tensor dtype; out[m, h*Dh + d] =
 * attn[m, h, d] * gate[m, h].  Rows m = b * seq + n.  attn is [batch, seq, heads, dim_head]
 * with element strides attn_strides = {batch, seq, head} (NULL = dense) and a contiguous last
 * axis: the SDPA output is read through its transposed view.  x[rows, dim], weight[heads, dim],
 * bias[heads], out[rows, heads * dim_head] and gate[rows, heads] are dense.
 */

/* fused_band_split.cpp:536-557 attention_gate_forward (.cu:1777-1826, 1922-1971). */
int pmsst_attention_gate_forward(const void* attn, const int64_t* attn_strides, const void* x, const void* weight,
                                 const void* bias, void* out, void* gate, int64_t batch, int64_t seq, int64_t heads,
                                 int64_t dim_head, int64_t dim, int dtype, void* stream);
/* Workspace bytes of the backward: the stored gate pre-activation gradient plus grad_weight /
 * grad_bias partials over row chunks. */
size_t pmsst_attention_gate_backward_workspace_size(int64_t rows, int64_t heads, int64_t dim);
/* fused_band_split.cpp:559-587 attention_gate_backward (.cu:1828-1920, 1973-2036):
 * grad_out[rows, heads * dim_head] dense -> grad_attn (strides grad_attn_strides like attn's,
 * NULL = dense), grad_x[rows, dim], grad_weight[heads, dim], grad_bias[heads]. */
int pmsst_attention_gate_backward(const void* grad_out, const void* attn, const int64_t* attn_strides, const void* x,
                                  const void* weight, const void* gate, void* grad_attn,
                                  const int64_t* grad_attn_strides, void* grad_x, void* grad_weight, void* grad_bias,
                                  int64_t batch, int64_t seq, int64_t heads, int64_t dim_head, int64_t dim, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------ Mel-band RoFormer band rows
 * No reference counterpart (the band gather and the overlap-averaged mask scatter live in
 * pymss-core, absent from the reference; the Mel-band model calls them around the band split and
 * the mask estimators).  The spectrum is packed [batch, num_rows, frames, 2] (frequency x channel
 * rows, re/im) and a band layout selects num_sel rows: rows[j] (device int64), bands in order.
 * row_start (device int64 [num_rows + 1]) and sources (device int64 [num_sel]) list, for every
 * row, the selections j that point at it (a CSR of rows[], ascending j); the caller builds and
 * validates both (0 <= rows[j] < num_rows).
 */

/* out[b, t, j, :] = in[b, rows[j], t, :] / divisor[j] (divisor: device fp32 [num_sel], NULL = no
 * division); out is [batch, frames, num_sel, 2].  in_dtype / out_dtype may differ. */
int pmsst_band_rows_gather(const void* in, int in_dtype, const int64_t* rows, const float* divisor, void* out,
                           int out_dtype, int64_t batch, int64_t num_rows, int64_t frames, int64_t num_sel,
                           void* stream);
/* out[b, r, t, :] = sum_{j in sources[row_start[r] .. row_start[r+1])} in[b, t, j, :], divided by the
 * count when mean is nonzero (rows no band selects get 0); in is [batch, frames, num_sel, 2], out
 * [batch, num_rows, frames, 2]. */
int pmsst_band_rows_scatter(const void* in, int in_dtype, const int64_t* row_start, const int64_t* sources, int mean,
                            void* out, int out_dtype, int64_t batch, int64_t num_rows, int64_t frames,
                            int64_t num_sel, void* stream);

/* ---------------------------------------------------------------- mask application / iSTFT layout
 * No kernel counterpart in the reference: the stock model multiplies the complex spectrum by the
 * masks (after a float cast and a transposed complex view) and permutes the product into the iSTFT
 * input, which the reference's cached-zero iSTFT then consumes (cuda_graph.py:140-158, including its
 * zero_dc index_fill of frequency bin 0).  One pass each way here:
 *   est[b, s, c, f, t] = spec[b, f*C + c, t] * mask_s[b, t, f*C + c]   (complex)
 * spec: complex64 [batch, freqs*channels, frames] (re, im fp32 pairs), 8-byte aligned.
 * mask: (re, im) pairs of dtype mask_dtype; element (b, s, t, k) at
 *       b * mask_batch_stride + s * mask_stem_stride + t * 2*freqs*channels + k (even strides).
 * est:  complex64 [batch, stems, channels, freqs, frames] = the iSTFT input [B*S*C, F, T].
 * zero_dc nonzero: est (and both gradients) are 0 at f = 0. */
int pmsst_mask_apply_forward(const void* spec, const void* mask, int64_t mask_batch_stride, int64_t mask_stem_stride,
                             int64_t batch, int64_t stems, int64_t channels, int64_t freqs, int64_t frames,
                             int zero_dc, void* est, int mask_dtype, void* stream);
/* grad_mask (mask_dtype, contiguous [batch, stems, frames, 2*freqs*channels]) = grad_est * conj(spec);
 * grad_spec (complex64 like spec, NULL to skip) = sum over stems of grad_est * conj(mask).  mask is read
 * only for grad_spec: with grad_spec NULL any buffer of its layout may be passed (e.g. grad_mask). */
int pmsst_mask_apply_backward(const void* grad_est, const void* spec, const void* mask, int64_t mask_batch_stride,
                              int64_t mask_stem_stride, int64_t batch, int64_t stems, int64_t channels, int64_t freqs,
                              int64_t frames, int zero_dc, void* grad_mask, void* grad_spec, int mask_dtype,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PYMSST_AMD_H */
