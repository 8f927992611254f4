// Shape descriptor shared by the conv entry points and kernels.
#pragma once
#include "atk_common.h"

namespace atk {

struct ConvShape {
  int N, Ci, D, H, W, Co;
  int KD, KH, KW;
  int sd, sh, sw, pd, ph, pw, dd, dh, dw;
  int Do, Ho, Wo;
  int dtype;
};

// MFMA implicit-GEMM kernels (conv_igemm.hip).  Variant indices here are local to the
// implicit-GEMM table; the C ABI offsets them by one (ABI variant 0 = direct kernel).
int conv_igemm_num_variants();
const char* conv_igemm_variant_name(int v);
size_t conv_igemm_workspace_bytes(const ConvShape& p, int v);
int conv_igemm_launch(const ConvShape& p, const void* x, const void* w, const void* bias, void* y,
                      int v, void* ws, size_t ws_bytes, hipStream_t s);
// The same in two steps: pack the weights once, then run on the packed weights.
size_t conv_igemm_packed_bytes(const ConvShape& p, int v);
size_t conv_igemm_prepacked_workspace_bytes(const ConvShape& p, int v);
int conv_igemm_pack(const ConvShape& p, const void* w, void* packed, size_t packed_bytes, int v, hipStream_t s);
// resid: y += resid (same layout), or null.  gn_stats: GroupNorm records of y for gn_G groups
// (conv_igemm_gn_stats_bytes bytes, conv_igemm_gn_records per (n, g)), or null.  Both need an
// unsplit launch.
int conv_igemm_run_prepacked(const ConvShape& p, const void* x, const void* packed, size_t packed_bytes,
                             const void* bias, void* y, int v, void* ws, size_t ws_bytes, hipStream_t s,
                             const void* resid = nullptr, void* gn_stats = nullptr, size_t gn_stats_bytes = 0,
                             int gn_G = 0, bool channels_last = false);
size_t conv_igemm_gn_stats_bytes(const ConvShape& p, int v, int G);
int conv_igemm_gn_records(const ConvShape& p, int v, int G);
// Conv + GroupNorm (+ SiLU) in one cooperative launch (16-bit NC[D]HW, unsplit, no residual):
// y is written once, normalised.  ws: conv_igemm_gn_onepass_bytes bytes, zeroed before its
// first use and private to one stream; 0 bytes = the variant cannot take the shape.
size_t conv_igemm_gn_onepass_bytes(const ConvShape& p, int v, int G);
int conv_igemm_run_gn_onepass(const ConvShape& p, const void* x, const void* packed, size_t packed_bytes,
                              const void* bias, const void* gamma, const void* beta, int param_dtype, float eps,
                              int silu, void* y, int v, int G, void* ws, size_t ws_bytes, hipStream_t s);

}  // namespace atk
