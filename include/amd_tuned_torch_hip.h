/*
 * amd_tuned_torch_hip.h -- C ABI of libamd_tuned_torch_hip.so, the gfx950 (MI355X)
 * kernel library behind the `amd_tuned_torch` Python package.
 *
 * The reference (WifiLast/rocm-kernel-select) reaches its kernels through pybind11
 * functions that take torch::Tensor and allocate their own outputs.  This library
 * replaces those entry points with plain C functions: raw device pointers, sizes,
 * a dtype code and an explicit hipStream_t.  The caller (the Python host, or any
 * other FFI) owns every buffer: inputs, outputs and the optional workspace.  The
 * library never allocates or frees device memory and keeps no per-shape state,
 * so every entry point is reentrant; calls that share one workspace buffer must
 * not run concurrently (they are ordered when issued on one stream).
 *
 * Return codes (every compute entry point):
 *   ATK_OK           (0) kernels were enqueued on `stream`;
 *   ATK_UNSUPPORTED  (1) this build has no kernel for the shape / dtype / variant:
 *                        nothing was enqueued and the output is untouched.  The
 *                        Python host turns this into a declining candidate, the
 *                        same contract as the reference's `launch_conv3d_fp32_winograd`
 *                        returning false (src/main_rocm.cpp:165-177);
 *   ATK_EINVAL       (2) inconsistent arguments (the reference's TORCH_CHECK
 *                        failures, src/main_rocm.cpp:556-599,669-715,798-854);
 *   ATK_ELAUNCH      (3) the HIP runtime rejected a launch.
 * atk_last_error() returns a thread-local, human-readable reason for the last
 * non-zero code.
 *
 * Layout: every tensor argument is dense and row-major ("contiguous" in torch
 * terms), 16-byte alignment of base pointers is not required (kernels take a
 * slower element-wise path when it is missing).
 */
#ifndef AMD_TUNED_TORCH_HIP_H
#define AMD_TUNED_TORCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* atk_stream_t; /* == hipStream_t; NULL = the null stream */

enum {
  ATK_OK = 0,
  ATK_UNSUPPORTED = 1,
  ATK_EINVAL = 2,
  ATK_ELAUNCH = 3
};

/* Element type codes. */
enum { ATK_F32 = 0, ATK_F16 = 1, ATK_BF16 = 2 };

/* Operation codes for the variant-table queries. */
enum { ATK_OP_DWCONV1D = 0, ATK_OP_GROUP_NORM = 1, ATK_OP_CONV = 2 };

/* Library ABI version (bumped on any signature change). */
int atk_abi_version(void);

/* Thread-local message for the last failing call on this thread ("" if none). */
const char* atk_last_error(void);

/* Variant tables: the tile / wave-count instances of each op this build carries.
 * Variant indices are stable within one ABI version.  The per-shape selector in
 * the Python host times these against stock PyTorch and caches the winner by
 * name.  Returns the count / a static string (NULL when out of range). */
int atk_num_variants(int op);
const char* atk_variant_name(int op, int variant);

/* ---------------------------------------------------------------------------
 * Depthwise conv1d forward (groups == channels, one input channel per group,
 * stride 1, dilation 1), BCL layout:
 *
 *   y[n,c,t] = bias[c] + sum_{j<K} w[c,j] * x[n,c,t - pad_left + j],   t in [0, L_out)
 *
 * with x taken as zero outside [0, L).  Covers both callers of the reference:
 *   - symmetric padding p (odd K): pad_left = p, L_out = L + 2p - K + 1
 *     (replaces `conv1d_forward(u, weight, bias, padding, is_bhl=True)`,
 *      amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/host.cpp:10,
 *      conv1d.h:56-83, conv1d_bhl.hip:102-142);
 *   - causal (Mamba) padding: pad_left = K - 1 with L_out = L + K - 1 (stock
 *     F.conv1d shape) or L_out = L (the truncated shape
 *     `causal_conv1d_fwd(x, w, bias, ..., silu)` returns,
 *     src/causal-conv1d-amd/csrc/causal_conv1d.cpp:131-238).
 * x: [N, C, L], y: [N, C, L_out] of `dtype`; w: [C, K] and bias: [C] (or NULL) of
 * w_dtype, which is `dtype` or fp32 (the causal interface keeps fp32 weights with
 * 16-bit activations, causal_conv1d.cpp:139-141; they are used unrounded).
 * Accumulation is fp32 for every dtype.  fuse_silu != 0 applies y*sigmoid(y)
 * before the store (the causal kernel's `silu_activation` flag).
 * K in [1, 64]; pad_left in [0, 64].  variant < 0 takes the first of xlane,
 * lds_opt32_nt, lds_opt16, direct that accepts the shape.
 * ------------------------------------------------------------------------- */
int atk_dwconv1d_fwd(const void* x, const void* w, const void* bias, void* y,
                     int64_t N, int64_t C, int64_t L, int K, int pad_left, int64_t L_out,
                     int dtype, int w_dtype, int fuse_silu, int variant, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Causal conv1d decode step (replaces `causal_conv1d_update(x, conv_state, weight,
 * bias?, silu_activation)`, src/causal-conv1d-amd/csrc/causal_conv1d.cpp:385-440 ->
 * causal_conv1d_update.cu:27-66):
 *   conv_state[b,d,:] <- (conv_state[b,d,1:], x[b,d]),
 *   y[b,d] = bias[d] + sum_j w[d,j] * conv_state[b,d,j]   (+ SiLU if fuse_silu).
 * x, y: [B, D] and conv_state: [B, D, W] (updated in place) of `dtype`; w: [D, W] and
 * bias: [D] (or NULL) of w_dtype, `dtype` or fp32 (causal_conv1d.cpp:437 dispatches the
 * weight type separately).  W in [1, 64] (the reference: [2, 4]).
 * ------------------------------------------------------------------------- */
int atk_causal_conv1d_update(const void* x, void* conv_state, const void* w, const void* bias, void* y,
                             int64_t B, int64_t D, int W, int dtype, int w_dtype, int fuse_silu,
                             atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Depthwise / causal conv1d backward, weight and bias gradients (replaces the
 * dweight / dbias half of `conv1d_backward(dout, u, weight, bias, padding, is_bhl)`,
 * amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/conv1d_bwd_hip_bhl.hip:
 * 78-116, and of `causal_conv1d_bwd(x, weight, bias, dout, ...)`,
 * src/causal-conv1d-amd/csrc/causal_conv1d.cpp:240-380):
 *   dw[c,k] = sum_{n,t} dy[n,c,t] * x[n,c,t-pad_left+k],  db[c] = sum_{n,t} dy[n,c,t].
 * x: [N, C, L], dy: [N, C, L_out], both of `dtype`; dw: [C, K] fp32, db: [C] fp32 or
 * NULL.  The input gradient is atk_dwconv1d_fwd run on dy with the weights reversed
 * along K and pad_left' = K-1-pad_left (output length L).  K in [1, 5].  The
 * workspace (atk_dwconv1d_bwd_weight_workspace_bytes) holds per-row partials; it
 * needs no initialisation.  Sums over n are taken in a fixed order (deterministic).
 * ------------------------------------------------------------------------- */
size_t atk_dwconv1d_bwd_weight_workspace_bytes(int64_t N, int64_t C, int K);
int atk_dwconv1d_bwd_weight(const void* x, const void* dy, float* dw, float* db,
                            int64_t N, int64_t C, int64_t L, int K, int pad_left, int64_t L_out,
                            int dtype, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Causal conv1d backward, fused, (B, C, L) layout (replaces the non-channel-last branch
 * of `causal_conv1d_bwd(x, weight, bias, dout, ..., silu)`,
 * src/causal-conv1d-amd/csrc/causal_conv1d.cpp:240-380 -> causal_conv1d_bwd.cu:100-235):
 * with z the recomputed fp32 pre-activation and g = dout * silu'(z) (dout without SiLU),
 *   dx[p] = sum_k w[k] g[p+K-1-k],  dw[c,k] = sum_{b,p} g[p] x[p-K+1+k],  db[c] = sum g.
 * x, dout, dx: [B, D, L] of `dtype`, contiguous, 16-byte aligned, L a multiple of 16 bytes;
 * w[c,k] at c*w_stride_c + k*w_stride_k in w_dtype (fp32 or `dtype`), bias [D] in w_dtype
 * or NULL; dw [D, K], db [D] fp32.  K in [2, 4].  The workspace (B*D*(K+1) floats) holds
 * per-row partials, summed over b in a fixed order.
 * ------------------------------------------------------------------------- */
int atk_causal_conv1d_bwd(const void* x, const void* dout, const void* w, const void* bias, void* dx, float* dw,
                          float* db, int64_t B, int64_t D, int64_t L, int K, int64_t w_stride_c, int64_t w_stride_k,
                          int dtype, int w_dtype, int silu, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Channels-last depthwise conv1d forward (replaces `conv1d_forward(u, weight, bias,
 * padding, is_bhl=false)`, amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/
 * conv1d.h:56-83 -> conv1d_blh.hip:54-220, and the channel-last branch of
 * `causal_conv1d_fwd(x, weight, bias, seq_idx, initial_states, final_states, silu)`,
 * src/causal-conv1d-amd/csrc/causal_conv1d.cpp:131-238 -> causal_conv1d_fwd.cu:194-365):
 *   y[b,t,c] = act(bias[c] + sum_{k<K} m * w[c,k] * x[b, t-pad_left+k, c]),  t < L_out.
 * Element (b, t, c) of x sits at b*x_stride_b + t*x_stride_l + c (channel stride 1),
 * of y at b*y_stride_b + t*y_stride_l + c; w[c,k] at c*w_stride_c + k*w_stride_k in
 * w_dtype (fp32 or `dtype`), bias [D] in w_dtype or NULL.  x = 0 outside [0, L), except
 * that positions -(K-1)..-1 read initial_states[b, p+K-1, c] (at b*is_stride_b +
 * j*is_stride_l + c) when given.  seq_idx: int32 [B, L] or NULL; seq_mode 1 drops taps
 * whose seq differs from the output position's (causal form, pad_left = K-1), 2 from
 * the first tap's (pad_left = 0: the input gradient on reversed weights); positions < 0
 * have seq -1.  final_states[b, j, c] (at b*fs_stride_b + j*fs_stride_l + c) receives
 * x[b, L-(K-1)+j, c].  States need the causal form (pad_left = K-1, L_out = L).
 * K <= 8 (seq_idx: K <= 4); D, every stride and pointer in 16-byte units.
 * ------------------------------------------------------------------------- */
int atk_dwconv1d_cl_fwd(const void* x, const void* w, const void* bias, void* y, const int* seq_idx,
                        const void* initial_states, void* final_states, int64_t B, int64_t D, int64_t L,
                        int K, int pad_left, int64_t L_out, int64_t x_stride_b, int64_t x_stride_l,
                        int64_t y_stride_b, int64_t y_stride_l, int64_t w_stride_c, int64_t w_stride_k,
                        int64_t is_stride_b, int64_t is_stride_l, int64_t fs_stride_b, int64_t fs_stride_l,
                        int dtype, int w_dtype, int fuse_silu, int seq_mode, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Channels-last depthwise conv1d weight / bias gradients (replaces the dweight /
 * dbias half of `conv1d_backward(..., is_bhl=false)`, amd_tuned_torch/_vendor/
 * flashfftconv_depthwise_conv1d/conv1d_bwd_hip_blh.hip:21-127):
 *   dw[c,k] = sum_{b,t} dy[b,t,c] * m * x[b, t-pad_left+k, c],  db[c] = sum_{b,t} dy[b,t,c],
 * x extended and masked as in atk_dwconv1d_cl_fwd (seq_mode 0 or 1).  dw [D, K] fp32,
 * db [D] fp32 or NULL.  K <= 5.  The workspace holds per-span partials, summed in a
 * fixed order (deterministic); it needs no initialisation.
 * ------------------------------------------------------------------------- */
size_t atk_dwconv1d_cl_bwd_weight_workspace_bytes(int64_t B, int64_t D, int64_t L_out, int K, int dtype);
int atk_dwconv1d_cl_bwd_weight(const void* x, const void* dy, const int* seq_idx, const void* initial_states,
                               float* dw, float* db, int64_t B, int64_t D, int64_t L, int K, int pad_left,
                               int64_t L_out, int64_t x_stride_b, int64_t x_stride_l, int64_t dy_stride_b,
                               int64_t dy_stride_l, int64_t is_stride_b, int64_t is_stride_l, int dtype,
                               int seq_mode, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Causal channel-last conv1d backward, fused (replaces the channel-last branch of
 * `causal_conv1d_bwd(x, weight, bias, dout, seq_idx, initial_states, dfinal_states, dx,
 * return_dinitial_states, silu)`, src/causal-conv1d-amd/csrc/causal_conv1d.cpp:240-380):
 * with z the recomputed fp32 pre-activation and g = dout * silu'(z) (dout without SiLU),
 *   dx[b,q,c] = sum_k w[c,k] * g[b, q+K-1-k, c] * [seq(q) == seq(q+K-1-k)],
 *   dw[c,k]   = sum_{b,t} g[b,t,c] * x[b, t-K+1+k, c] * [seq(t-K+1+k) == seq(t)],
 *   db[c]     = sum_{b,t} g[b,t,c].
 * Layouts and operands as in atk_dwconv1d_cl_fwd (x, dout, dx: channel stride 1).
 * initial_states feed x at negative positions; their gradient and dfinal_states are
 * the caller's (a few K-1-wide slices).  K in [2, 4].  dw [D, K], db [D] fp32.  The
 * workspace holds per-span partials (deterministic fixed-order sum).
 * ------------------------------------------------------------------------- */
size_t atk_causal_conv1d_cl_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K, int dtype);
int atk_causal_conv1d_cl_bwd(const void* x, const void* dout, const void* w, const void* bias, const int* seq_idx,
                             const void* initial_states, void* dx, float* dw, float* db, int64_t B, int64_t D,
                             int64_t L, int K, int64_t x_stride_b, int64_t x_stride_l, int64_t dout_stride_b,
                             int64_t dout_stride_l, int64_t dx_stride_b, int64_t dx_stride_l, int64_t w_stride_c,
                             int64_t w_stride_k, int64_t is_stride_b, int64_t is_stride_l, int dtype,
                             int w_dtype, int silu, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Channels-last depthwise conv1d backward in one pass (replaces `conv1d_backward(dout, u,
 * weight, bias, padding, is_bhl=false)`, amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/
 * conv1d_bwd_hip_blh.hip:21-127, behind amd_tuned_torch/depthwise_conv1d_ops.py's backward):
 * for y = atk_dwconv1d_cl_fwd(x, w, NULL, pad_left, L_out),
 *   dx[b,q,c] = sum_k w[c,k] * dy[b, q+pad_left-k, c]   (dy = 0 outside [0, L_out)),
 *   dw[c,k]   = sum_{b,t} dy[b,t,c] * x[b, t-pad_left+k, c],   db[c] = sum_{b,t} dy[b,t,c].
 * x, dx (B, L, D) and dy (B, L_out, D) views with channel stride 1 (layouts as in
 * atk_dwconv1d_cl_fwd); w read at (w_stride_c, w_stride_k) in w_dtype; dw [D, K], db [D]
 * fp32 (db may be NULL).  x and dy are each read once; the two-pass route (the forward
 * kernel on dy for dx, atk_dwconv1d_cl_bwd_weight for dw / db) reads dy twice.  K in [2, 4],
 * any pad_left >= 0 and L_out >= 1.  The workspace holds per-span partials (deterministic
 * fixed-order sum); it needs no initialisation.
 * ------------------------------------------------------------------------- */
size_t atk_dwconv1d_cl_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K, int pad_left, int64_t L_out,
                                           int dtype);
int atk_dwconv1d_cl_bwd(const void* x, const void* dy, const void* w, void* dx, float* dw, float* db, int64_t B,
                        int64_t D, int64_t L, int K, int pad_left, int64_t L_out, int64_t x_stride_b,
                        int64_t x_stride_l, int64_t dy_stride_b, int64_t dy_stride_l, int64_t dx_stride_b,
                        int64_t dx_stride_l, int64_t w_stride_c, int64_t w_stride_k, int dtype, int w_dtype,
                        void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Depthwise conv1d backward in one pass (replaces `conv1d_backward(dout, u, weight, bias,
 * padding, is_bhl=True)`, _vendor/flashfftconv_depthwise_conv1d/conv1d_bwd_hip_bhl.hip:39-116,
 * behind amd_tuned_torch/depthwise_conv1d_ops.py's backward, and the (B, C, L) backward of a
 * depthwise F.conv1d): for y = dwconv1d(x, w, bias, pad_left, L_out),
 *   dx[n,c,s] = sum_j w[c,j] * dy[n,c,s+pad_left-j],
 *   dw[c,j]   = sum_{n,t} dy[n,c,t] * x[n,c,t-pad_left+j],   db[c] = sum_{n,t} dy[n,c,t],
 * x, dx [N,C,L]; dy [N,C,L_out]; w [C,K] of `dtype`; dw [C,K], db [C] fp32.  x and dy are
 * read once (atk_dwconv1d_fwd on dy plus atk_dwconv1d_bwd_weight read dy twice).  dw / db
 * may be NULL (dx only; db needs dw), and then no workspace is needed; otherwise the
 * workspace is atk_dwconv1d_bwd_weight_workspace_bytes(N, C, K), no initialisation.
 * K in [1, 5], pad_left <= 64; dx rows must be 16-byte aligned (L * sizeof(dtype) a
 * multiple of 16 and an aligned dx), else ATK_UNSUPPORTED.  Sums over n in a fixed order.
 * ------------------------------------------------------------------------- */
int atk_dwconv1d_bwd(const void* x, const void* dy, const void* w, void* dx, float* dw, float* db,
                     int64_t N, int64_t C, int64_t L, int K, int pad_left, int64_t L_out, int dtype,
                     void* workspace, size_t workspace_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * GroupNorm forward, NC[spatial] layout (replaces `group_norm(input, num_groups,
 * weight?, bias?, eps)`, src/main_rocm.cpp:556-599 -> src/cuda/group_norm.cu:41-136,
 * and the fused GroupNorm+SiLU of amd_tuned_torch/conv_fusion_ops.py:192-275):
 *
 *   y[n,c,s] = act( (x[n,c,s] - mean[n,g]) * rsqrt(var[n,g] + eps) * gamma[c] + beta[c] )
 *
 * g = c / (C/G); mean/var are the population statistics of the C/G * S elements
 * of group (n, g), computed in fp32 from data held on chip (exact two-pass
 * statistics, no E[x^2]-E[x]^2 cancellation).  act = SiLU when fuse_silu != 0,
 * identity otherwise.  gamma/beta may be NULL (non-affine) and have their own
 * element type `param_dtype` (torch allows fp32 affine parameters under 16-bit
 * activations).  S = product of the spatial extents (1 for a [N, C] input).
 * Needs a workspace of atk_group_norm_workspace_bytes(...) bytes whose first
 * atk_group_norm_workspace_zero_bytes(...) bytes are zero before the FIRST call
 * that uses it (the kernels leave them zero again on exit, apart from the first
 * 4 bytes: a diagnostics word set to 1 when a workgroup stopped waiting for another's
 * partial statistics and computed them itself -- results are exact either way).
 * The zeroed region has a fixed size and layout for every shape, so one workspace
 * serves calls of any shape (ordered on one stream), including HIP graph replays.
 * ------------------------------------------------------------------------- */
size_t atk_group_norm_workspace_bytes(int64_t N, int64_t C, int64_t S, int G, int dtype,
                                      int variant);
size_t atk_group_norm_workspace_zero_bytes(int64_t N, int64_t C, int64_t S, int G,
                                           int dtype, int variant);
int atk_group_norm_fwd(const void* x, const void* gamma, const void* beta, void* y,
                       int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                       int dtype, int param_dtype, int variant, void* workspace,
                       size_t workspace_bytes, atk_stream_t stream);
/* Diagnostics, no counterpart in the reference (its group_norm.cu has no phase timing):
 * register a device buffer of n_words 64-bit words (NULL / 0 drops it); every later
 * register-resident launch (res_* variants of atk_group_norm_fwd, and the single-pass kernel
 * of atk_group_norm_cl_fwd) with at most n_words / 4 workgroups stores, per
 * workgroup w, four wall-clock stamps at words 4w..4w+3: entry, slice statistics done (all its
 * loads arrived), group statistics known (after the exchange between workgroups), stores issued.
 * Returns the wall-clock rate in kHz (0 on error).  Process-wide; not for concurrent use. */
int atk_group_norm_trace(void* device_words, int64_t n_words);

/* ---------------------------------------------------------------------------
 * GroupNorm forward that allocates nothing and takes no workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory or hand over scratch --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments (minus the workspace), kernels and results as atk_group_norm_fwd; the caller
 * still passes x and y.  The scratch is a static device array of 4 slices of
 * atk_group_norm_noalloc_scratch_bytes() bytes (about 2.1 MB each, 8.5 MB in all) that each
 * GPU the library runs on holds until the process ends; shapes needing more than a slice
 * (two-pass partials above 1 MiB) are rejected with ATK_EINVAL.  The first call from a stream
 * binds the next free slice of the current GPU to that stream handle for the rest of the
 * process: calls on one stream are ordered and calls on different streams use different
 * slices, so neither races.  A fifth stream on one GPU is refused with ATK_EINVAL.  A slice
 * follows the handle value, so a stream destroyed with calls still in flight must not have
 * its handle reused by a new stream before that work ends.  The first call on a device
 * resolves the array's address there (make it outside graph capture).
 * ------------------------------------------------------------------------- */
size_t atk_group_norm_noalloc_scratch_bytes(void);
int atk_group_norm_fwd_noalloc(const void* x, const void* gamma, const void* beta, void* y,
                               int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                               int dtype, int param_dtype, int variant, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * GroupNorm forward, channels-last layout (NHWC / NDHWC memory: x[n][s][c]), optional
 * fused SiLU.  The reference serves this layout with Composable Kernel's groupnorm
 * (amd_tuned_torch/ck_norm_ops.py:9-27,93-103, picked by the contest in
 * amd_tuned_torch/_dispatch.py:2140-2200); same arithmetic and parameters as
 * atk_group_norm_fwd.  Needs (C/G)*sizeof(dtype) % 16 == 0, C*sizeof(dtype)/16 dividing
 * 256 (C <= 2048 for 16-bit types), G <= 256 and 16-byte aligned x / y (else
 * ATK_UNSUPPORTED).  Deterministic.
 * Where 128 KB chunks cover every CU, one register-resident launch exchanges per-chunk
 * statistics between workgroups through the workspace (atk_group_norm_cl_workspace_bytes),
 * whose first bytes hold an epoch and counters that every launch leaves consistent: the
 * workspace must be zero-filled once when it is allocated and then passed unchanged to
 * later calls (its contents are the state), and calls sharing one workspace must be
 * ordered (one stream).  ATK_GN_CL_RESIDENT=0 in the environment keeps the three-kernel
 * path (8 or 16 forces the resident configuration with that many vectors per thread), and
 * ATK_GN_CL_LAYOUT=rows / blocks forces its chunk shape (whole positions, or 128-byte column
 * blocks of a position; by default blocks where the rows grid would need more than one
 * workgroup per CU).
 * ------------------------------------------------------------------------- */
size_t atk_group_norm_cl_workspace_bytes(int64_t N, int64_t C, int64_t S, int G);
int atk_group_norm_cl_fwd(const void* x, const void* gamma, const void* beta, void* y,
                          int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                          int dtype, int param_dtype, void* workspace, size_t workspace_bytes,
                          atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * GroupNorm backward, NC[spatial] layout (replaces the torch-op backward of
 * amd_tuned_torch/_dispatch.py:2212-2302 behind _GroupNormFn, 2305-2359):
 *   x_hat = (x - mu) * rstd,  g = gamma_c * dy,
 *   dx = rstd * (g - mean_group(g) - x_hat * mean_group(g * x_hat)),
 *   dgamma_c = sum_{n,s} dy * x_hat,  dbeta_c = sum_{n,s} dy.
 * x, dy, dx: [N, C, S] of `dtype`; gamma: [C] of `param_dtype` or NULL (ones);
 * dgamma / dbeta: [C] fp32.  Any of dx / dgamma / dbeta may be NULL.  The group
 * statistics are recomputed from x with the forward's eps.  Needs S * sizeof(dtype)
 * to be a multiple of 16 and 16-byte aligned x / dy / dx (else ATK_UNSUPPORTED).
 * The first 16 KiB of the workspace (atk_group_norm_bwd_workspace_bytes) must be zero
 * before the first call that uses it; every call leaves them zero (per-group counters).
 * Sums over n are taken in a fixed order (deterministic).  Groups of up to 8192 16-byte
 * vectors whose spatial size is a multiple of 64 vectors run register-resident (x and dy
 * read once) when a group has at most 512 channels; other shapes take two kernels that
 * read x and dy twice.
 * ------------------------------------------------------------------------- */
size_t atk_group_norm_bwd_workspace_bytes(int64_t N, int64_t C);
int atk_group_norm_bwd(const void* x, const void* dy, const void* gamma, void* dx, float* dgamma,
                       float* dbeta, int64_t N, int64_t C, int64_t S, int G, float eps, int dtype,
                       int param_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * GroupNorm backward, channels-last layout (x, dy, dx: [N][S][C], NHWC / NDHWC
 * memory).  Replaces the same torch-op backward (amd_tuned_torch/_dispatch.py:
 * 2212-2302) for the channels-last input the reference's CK forward serves
 * (amd_tuned_torch/ck_norm_ops.py:9-27, 93-103).  Same math and arguments as
 * atk_group_norm_bwd.  Needs (C/G) * sizeof(dtype) a multiple of 16,
 * C / (16 / sizeof(dtype)) dividing 256 (C <= 2048 for 16-bit types), 16-byte
 * aligned x / dy / dx and one sample under 2 GiB (else ATK_UNSUPPORTED).  All sums are
 * taken in a fixed order (deterministic).  The workspace
 * (atk_group_norm_cl_bwd_workspace_bytes, 16-byte aligned) follows the forward's rule: zero-
 * filled once when allocated, then passed unchanged to later calls on one stream (a register-
 * resident launch, taken where the grid is one workgroup per CU, keeps an epoch and counters
 * in its first bytes).
 * ------------------------------------------------------------------------- */
size_t atk_group_norm_cl_bwd_workspace_bytes(int64_t N, int64_t C, int64_t S, int G);
int atk_group_norm_cl_bwd(const void* x, const void* dy, const void* gamma, void* dx, float* dgamma,
                          float* dbeta, int64_t N, int64_t C, int64_t S, int G, float eps, int dtype,
                          int param_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Dense convolution forward, groups = 1, NCDHW layout, as an implicit GEMM on
 * MFMA (replaces `conv3d(input, weight, bias?, stride, padding, dilation)`,
 * src/main_rocm.cpp:798-854, and `conv2d(...)`, src/main_rocm.cpp:669-715):
 *
 *   y[n,o,z,y,x] = bias[o] + sum_{i,a,b,c} w[o,i,a,b,c] *
 *                  x[n, i, z*sd - pd + a*dd, y*sh - ph + b*dh, x*sw - pw + c*dw]
 *
 * x: [N, Ci, D, H, W], w: [Co, Ci, KD, KH, KW], bias: [Co] or NULL,
 * y: [N, Co, Do, Ho, Wo] with Do = (D + 2pd - dd(KD-1) - 1)/sd + 1 (likewise H, W),
 * the output-size formula of src/main_rocm.cpp:204-206.  conv2d is the D = KD = 1
 * case.  16-bit inputs use bf16/fp16 MFMA with fp32 accumulation; fp32 inputs use
 * fp32 MFMA.  Needs a workspace of atk_conv_workspace_bytes(...) bytes (repacked
 * weights and split-K partial sums).
 * ------------------------------------------------------------------------- */
size_t atk_conv_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W,
                                int64_t Co, int KD, int KH, int KW, int sd, int sh, int sw,
                                int pd, int ph, int pw, int dd, int dh, int dw, int dtype,
                                int variant);
int atk_conv_fwd(const void* x, const void* w, const void* bias, void* y, int64_t N,
                 int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH,
                 int KW, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh,
                 int dw, int dtype, int variant, void* workspace, size_t workspace_bytes,
                 atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * The same convolution in two steps, for weights that stay constant across calls (the
 * reference's native conv re-derives its weight layout inside every `conv3d` /
 * `conv2d` call, src/main_rocm.cpp:669-715,798-854; inference weights need it once):
 *   atk_conv_pack_weights   w -> packed (atk_conv_packed_weight_bytes bytes, the fragment
 *                           order MFMA variant `variant` reads; valid for that variant and
 *                           geometry only, and only while w is unchanged);
 *   atk_conv_fwd_prepacked  y from x and the packed weights; the workspace holds only the
 *                           split-K partial sums (atk_conv_prepacked_workspace_bytes bytes,
 *                           0 when the variant does not split this shape).
 * Same geometry arguments, arithmetic and results as atk_conv_fwd.  Variant 0 (the direct
 * kernel) has no packed form: ATK_UNSUPPORTED.  The size queries return 0 for shapes the
 * variant declines.
 * ------------------------------------------------------------------------- */
size_t atk_conv_packed_weight_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W,
                                    int64_t Co, int KD, int KH, int KW, int sd, int sh, int sw,
                                    int pd, int ph, int pw, int dd, int dh, int dw, int dtype,
                                    int variant);
size_t atk_conv_prepacked_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W,
                                          int64_t Co, int KD, int KH, int KW, int sd, int sh,
                                          int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                                          int dtype, int variant);
int atk_conv_pack_weights(const void* w, void* packed, size_t packed_bytes, int64_t N, int64_t Ci,
                          int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH, int KW,
                          int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                          int dtype, int variant, atk_stream_t stream);
int atk_conv_fwd_prepacked(const void* x, const void* packed, size_t packed_bytes,
                           const void* bias, void* y, int64_t N, int64_t Ci, int64_t D,
                           int64_t H, int64_t W, int64_t Co, int KD, int KH, int KW, int sd,
                           int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                           int dtype, int variant, void* workspace, size_t workspace_bytes,
                           atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * atk_conv_fwd_prepacked on channels-last tensors: x [N, D, H, W, Ci] and y [N, Do, Ho, Wo,
 * Co] in memory (NDHWC; conv2d NHWC with D = KD = 1), the same packed weights, geometry
 * arguments (logical sizes), arithmetic and workspace.  The reference serves channels-last
 * convs with CK or stock (amd_tuned_torch/_dispatch.py:1813,1947, contest key with the memory
 * format kernel_select.py:438-445); here the MFMA tiles stage channels-last patches straight
 * into LDS, with no layout conversion.  16-bit dtypes, a 3x3 or 7x7 (kh, kw) plane, Ci and Co
 * multiples of 8 and 16-byte aligned x and y; otherwise ATK_UNSUPPORTED.
 * ------------------------------------------------------------------------- */
int atk_conv_fwd_prepacked_cl(const void* x, const void* packed, size_t packed_bytes,
                              const void* bias, void* y, int64_t N, int64_t Ci, int64_t D,
                              int64_t H, int64_t W, int64_t Co, int KD, int KH, int KW, int sd,
                              int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                              int dtype, int variant, void* workspace, size_t workspace_bytes,
                              atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Conv epilogue fusion (the reference fuses GroupNorm+SiLU before a conv and names
 * "Conv -> +residual" as the epilogue to fuse, amd_tuned_torch/conv_fusion_ops.py:1-40,
 * 355-439): atk_conv_fwd_prepacked with, on an unsplit launch,
 *   residual   y = conv + bias + residual (residual: y's shape and layout, dtype), or NULL;
 *   gn_stats   GroupNorm statistics of the stored y for `gn_groups` groups: records
 *              (count, mean, M2, 0) as 4 floats, atk_conv_gn_records(...) per (n, g),
 *              laid out [N * gn_groups][records]; atk_conv_gn_stats_bytes(...) bytes (0
 *              when the variant splits this shape or Co/groups is not 4, 8, 16, 32 or a
 *              multiple of 32 -- then the call returns ATK_UNSUPPORTED), or NULL.
 * atk_group_norm_apply then normalises y with those records (no statistics pass over y):
 *   y_out = act((x - mean) * rsqrt(var + eps) * gamma + beta), x and y_out may be the same
 *   buffer; `variant` is a split GroupNorm variant (-1: split_nt256_v8).
 * ------------------------------------------------------------------------- */
size_t atk_conv_gn_stats_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co,
                               int KD, int KH, int KW, int sd, int sh, int sw, int pd, int ph, int pw,
                               int dd, int dh, int dw, int dtype, int variant, int gn_groups);
int atk_conv_gn_records(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD,
                        int KH, int KW, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh,
                        int dw, int dtype, int variant, int gn_groups);
int atk_conv_fwd_prepacked_ex(const void* x, const void* packed, size_t packed_bytes,
                              const void* bias, const void* residual, void* y, int64_t N,
                              int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD,
                              int KH, int KW, int sd, int sh, int sw, int pd, int ph, int pw,
                              int dd, int dh, int dw, int dtype, int variant, int gn_groups,
                              void* gn_stats, size_t gn_stats_bytes, void* workspace,
                              size_t workspace_bytes, atk_stream_t stream);
int atk_group_norm_apply(const void* x, const void* gamma, const void* beta, void* y, int64_t N,
                         int64_t C, int64_t S, int G, float eps, int fuse_silu, int dtype,
                         int param_dtype, const void* stats, int64_t records_per_group,
                         int variant, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Conv -> GroupNorm -> (SiLU) in one launch: the block the reference's fused module runs
 * (amd_tuned_torch/conv_fusion_ops.py:355-439, "Conv3d -> GroupNorm -> SiLU") as three
 * kernels.  The MFMA tile keeps its output in registers while the epilogue's GroupNorm
 * records are exchanged between workgroups (tagged slots in `workspace`), then stores
 *   y = act((conv + bias - mean) * rsqrt(var + eps) * gamma + beta)
 * once.  The statistics are of the conv output rounded to the dtype, as the three-kernel
 * block computes them.  16-bit NC[D]HW, groups with Co/groups in {4, 8, 16, 32} or a multiple
 * of 32, an unsplit variant whose records are summed in registers and a grid that is resident
 * at once: it is a cooperative launch.  atk_conv_gn_onepass_workspace_bytes(...) gives the
 * workspace (0: the variant cannot take the shape; the call then returns ATK_UNSUPPORTED); the
 * workspace is zeroed before its first use, kept between calls and private to one stream.
 * gamma / beta: C values of param_dtype, or NULL (1 / 0).  Word 0 of the workspace (int32) is
 * set if a wait for another workgroup ran out, which a resident grid never does.
 * ------------------------------------------------------------------------- */
size_t atk_conv_gn_onepass_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W,
                                           int64_t Co, int KD, int KH, int KW, int sd, int sh, int sw,
                                           int pd, int ph, int pw, int dd, int dh, int dw, int dtype,
                                           int variant, int groups);
int atk_conv_group_norm_fwd(const void* x, const void* packed, size_t packed_bytes, const void* bias,
                            const void* gamma, const void* beta, void* y, int64_t N, int64_t Ci,
                            int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH, int KW,
                            int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                            int dtype, int variant, int groups, float eps, int fuse_silu,
                            int param_dtype, void* workspace, size_t workspace_bytes,
                            atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Conv weight gradient (replaces the dweight part of `aten.convolution_backward` that the
 * reference's _Conv3dFn.backward calls, amd_tuned_torch/_dispatch.py:2064-2075), for
 * stride-1, dilation-1 convs with kernel (KD, 3, 3), KD in {1, 3}, and "same" padding
 * (KD/2, 1, 1):
 *   dw[co,ci,kz,ky,kx] = sum_{n,z,y,x} dy[n,co,z,y,x] * x[n,ci,z+kz-KD/2,y+ky-1,x+kx-1].
 * x: [N, Ci, D, H, W], dy: [N, Co, D, H, W], fp16 / bf16, contiguous; dw: [Co, Ci, KD, 3, 3]
 * fp32.  Ci % 32 == 0, Co % 128 == 0, W % 16 == 0, W <= 64.  conv2d is D = 1, KD = 1.  The
 * workspace holds per-chunk fp32 partials, summed in a fixed order (deterministic); it
 * needs no initialisation.
 * ------------------------------------------------------------------------- */
size_t atk_conv_wgrad_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD);
int atk_conv_wgrad(const void* x, const void* dy, float* dw, int64_t N, int64_t Ci, int64_t D, int64_t H,
                   int64_t W, int64_t Co, int KD, int dtype, void* workspace, size_t ws_bytes, atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Layout conversion between channels-last and channels-first memory (replaces the strided
 * `.contiguous(memory_format=...)` copies around the channels-last conv candidates; the
 * reference runs channels-last convs through CK or stock instead, amd_tuned_torch/
 * _dispatch.py:1840-1920, and has no counterpart kernel): a batched transpose of the last
 * two axes,
 *   out[b][c][r] = in[b][r][c],   in: [B, R, C], out: [B, C, R], both dense.
 * NDHWC [N][S][C] -> NCDHW [N][C][S] is (B, R, C) = (N, S, C); the reverse is (N, C, S).
 * Any element type of the dtype codes (2 or 4 bytes; the bytes are copied unchanged).
 * in and out must not overlap.  16-byte vectors when R and C are multiples of a vector and
 * both bases are 16-byte aligned, element-wise otherwise.  Needs no workspace.
 * ------------------------------------------------------------------------- */
int atk_transpose_last2(const void* in, void* out, int64_t B, int64_t R, int64_t C, int dtype,
                        atk_stream_t stream);

/* ---------------------------------------------------------------------------
 * Argument-block forms of the three forward entry points a framework calls once per op:
 * atk_dwconv1d_fwd, atk_group_norm_fwd and atk_conv_fwd_prepacked.  No counterpart in the
 * reference (its extension receives torch::Tensor arguments through pybind11).  Each takes
 * one pointer to a struct whose fields are that entry point's parameters, in order and of
 * the same types, and behaves exactly as that entry point (same checks, return codes and
 * launches).  They are for FFI callers that pay per scalar argument -- Python ctypes
 * converts each argument of a call (about 0.1 us apiece, 2.9 us for the 28 of
 * atk_conv_fwd_prepacked) -- and can keep one filled struct per shape, changing only the
 * pointers between calls.  The struct is read before the call returns and not kept.
 * ------------------------------------------------------------------------- */
typedef struct atk_dwconv1d_args {
  const void* x; const void* w; const void* bias; void* y;
  int64_t N; int64_t C; int64_t L; int K; int pad_left; int64_t L_out;
  int dtype; int w_dtype; int fuse_silu; int variant;
  atk_stream_t stream;
} atk_dwconv1d_args;
int atk_dwconv1d_fwd_args(const atk_dwconv1d_args* a);

typedef struct atk_group_norm_args {
  const void* x; const void* gamma; const void* beta; void* y;
  int64_t N; int64_t C; int64_t S; int G; float eps; int fuse_silu;
  int dtype; int param_dtype; int variant;
  void* workspace; size_t workspace_bytes;
  atk_stream_t stream;
} atk_group_norm_args;
int atk_group_norm_fwd_args(const atk_group_norm_args* a);

typedef struct atk_conv_prepacked_args {
  const void* x; const void* packed; size_t packed_bytes; const void* bias; void* y;
  int64_t N; int64_t Ci; int64_t D; int64_t H; int64_t W; int64_t Co;
  int KD; int KH; int KW; int sd; int sh; int sw; int pd; int ph; int pw; int dd; int dh; int dw;
  int dtype; int variant;
  void* workspace; size_t workspace_bytes;
  atk_stream_t stream;
} atk_conv_prepacked_args;
int atk_conv_fwd_prepacked_args(const atk_conv_prepacked_args* a);

#ifdef __cplusplus
}
#endif

#endif /* AMD_TUNED_TORCH_HIP_H */
