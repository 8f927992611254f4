// Dense conv2d/conv3d forward (groups = 1, NCDHW) for gfx950: host entry points, variant
// table and the direct (non-MFMA) kernel.  The MFMA implicit-GEMM kernels live in
// conv_igemm.hip and register through conv_igemm_launch().
//
//   y[n,o,z,y,x] = bias[o] + sum_{i,a,b,c} w[o,i,a,b,c] * x[n,i,z*sd-pd+a*dd, y*sh-ph+b*dh, x*sw-pw+c*dw]
//
// Output-size formula of the reference host (src/main_rocm.cpp:204-206).
#include "atk_common.h"
#include "conv_common.h"

namespace atk {

namespace {

constexpr int DC_NT = 256;
constexpr int DC_COT = 8;  // output channels per thread

// One thread: one output position x DC_COT output channels, fp32 accumulation.
template <typename T>
__global__ __launch_bounds__(DC_NT) void conv_direct_kernel(ConvShape p, const T* __restrict__ x,
                                                            const T* __restrict__ w,
                                                            const T* __restrict__ bias,
                                                            T* __restrict__ y) {
  const int64_t sp_out = (int64_t)p.Do * p.Ho * p.Wo;
  const int64_t m = (int64_t)blockIdx.x * DC_NT + threadIdx.x;  // (n, z, y, x) flat
  const int co0 = blockIdx.y * DC_COT;
  if (m >= (int64_t)p.N * sp_out) return;
  const int64_t n = m / sp_out;
  const int64_t sp = m - n * sp_out;  // output spatial offset
  const int oz = (int)(sp / ((int64_t)p.Ho * p.Wo));
  const int64_t r = sp - (int64_t)oz * p.Ho * p.Wo;
  const int oy = (int)(r / p.Wo);
  const int ox = (int)(r - (int64_t)oy * p.Wo);
  float acc[DC_COT];
#pragma unroll
  for (int j = 0; j < DC_COT; ++j) {
    const int co = co0 + j;
    acc[j] = (bias && co < p.Co) ? to_f32(bias[co]) : 0.f;
  }
  const int64_t in_sp = (int64_t)p.D * p.H * p.W;
  const int ktaps = p.KD * p.KH * p.KW;
  for (int ci = 0; ci < p.Ci; ++ci) {
    const T* xc = x + (n * p.Ci + ci) * in_sp;
    for (int a = 0; a < p.KD; ++a) {
      const int iz = oz * p.sd - p.pd + a * p.dd;
      if ((unsigned)iz >= (unsigned)p.D) continue;
      for (int b = 0; b < p.KH; ++b) {
        const int iy = oy * p.sh - p.ph + b * p.dh;
        if ((unsigned)iy >= (unsigned)p.H) continue;
        for (int c = 0; c < p.KW; ++c) {
          const int ix = ox * p.sw - p.pw + c * p.dw;
          if ((unsigned)ix >= (unsigned)p.W) continue;
          const float xv = to_f32(xc[((int64_t)iz * p.H + iy) * p.W + ix]);
          const int tap = (a * p.KH + b) * p.KW + c;
#pragma unroll
          for (int j = 0; j < DC_COT; ++j) {
            const int co = co0 + j;
            if (co < p.Co) acc[j] = fmaf(to_f32(w[((int64_t)co * p.Ci + ci) * ktaps + tap]), xv, acc[j]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DC_COT; ++j) {
    const int co = co0 + j;
    if (co < p.Co) y[(n * p.Co + co) * sp_out + sp] = from_f32<T>(acc[j]);
  }
}

template <typename T>
int launch_direct(const ConvShape& p, const void* x, const void* w, const void* b, void* y,
                  hipStream_t s) {
  const int64_t M = (int64_t)p.N * p.Do * p.Ho * p.Wo;
  const int64_t gx = (M + DC_NT - 1) / DC_NT;
  const int64_t gy = (p.Co + DC_COT - 1) / DC_COT;
  if (gx > 0x7fffffff || gy > 65535) return fail(ATK_UNSUPPORTED, "conv direct: grid too large");
  hipLaunchKernelGGL((conv_direct_kernel<T>), dim3((unsigned)gx, (unsigned)gy), dim3(DC_NT), 0, s, p,
                     static_cast<const T*>(x), static_cast<const T*>(w), static_cast<const T*>(b),
                     static_cast<T*>(y));
  return check_launch("conv_direct_kernel");
}

int conv_shape(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH,
               int KW, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
               int dtype, ConvShape& p) {
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "conv: unknown dtype code %d", dtype);
  if (N < 0 || Ci <= 0 || Co <= 0 || D <= 0 || H <= 0 || W <= 0 || KD <= 0 || KH <= 0 || KW <= 0)
    return fail(ATK_EINVAL, "conv: bad sizes");
  if (sd <= 0 || sh <= 0 || sw <= 0 || dd <= 0 || dh <= 0 || dw <= 0 || pd < 0 || ph < 0 || pw < 0)
    return fail(ATK_EINVAL, "conv: bad stride/padding/dilation");
  const int64_t Do = (D + 2 * pd - (int64_t)dd * (KD - 1) - 1) / sd + 1;
  const int64_t Ho = (H + 2 * ph - (int64_t)dh * (KH - 1) - 1) / sh + 1;
  const int64_t Wo = (W + 2 * pw - (int64_t)dw * (KW - 1) - 1) / sw + 1;
  if (Do <= 0 || Ho <= 0 || Wo <= 0) return fail(ATK_EINVAL, "conv: output size must be positive");
  const int64_t lim = 1ll << 30;
  if (D >= lim || H >= lim || W >= lim || Ci >= lim || Co >= lim || N >= lim ||
      N * Ci * D * H * W >= (1ll << 40) || N * Co * Do * Ho * Wo >= (1ll << 40))
    return fail(ATK_UNSUPPORTED, "conv: sizes too large");
  p.N = (int)N; p.Ci = (int)Ci; p.D = (int)D; p.H = (int)H; p.W = (int)W; p.Co = (int)Co;
  p.KD = KD; p.KH = KH; p.KW = KW; p.sd = sd; p.sh = sh; p.sw = sw;
  p.pd = pd; p.ph = ph; p.pw = pw; p.dd = dd; p.dh = dh; p.dw = dw;
  p.Do = (int)Do; p.Ho = (int)Ho; p.Wo = (int)Wo;
  p.dtype = dtype;
  return ATK_OK;
}

}  // namespace

int conv_num_variants() { return 1 + conv_igemm_num_variants(); }
const char* conv_variant_name(int v) {
  if (v == 0) return "direct";
  return conv_igemm_variant_name(v - 1);
}

}  // namespace atk

extern "C" size_t atk_conv_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W,
                                           int64_t Co, int KD, int KH, int KW, int sd, int sh,
                                           int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                                           int dtype, int variant) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(N, Ci, D, H, W, Co, KD, KH, KW, sd, sh, sw, pd, ph, pw, dd, dh, dw, dtype, p))
    return 0;
  if (variant <= 0) return 0;
  if (variant > conv_igemm_num_variants()) return 0;
  return conv_igemm_workspace_bytes(p, variant - 1);
}

extern "C" int atk_conv_fwd(const void* x, const void* w, const void* bias, void* y, int64_t N,
                            int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH,
                            int KW, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh,
                            int dw, int dtype, int variant, void* workspace,
                            size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(N, Ci, D, H, W, Co, KD, KH, KW, sd, sh, sw, pd, ph, pw, dd, dh, dw, dtype, p);
  if (rc) return rc;
  if (variant < 0) variant = 0;
  if (variant >= conv_num_variants()) return fail(ATK_EINVAL, "conv: variant %d out of range", variant);
  if (N == 0) return ATK_OK;
  if (!x || !w || !y) return fail(ATK_EINVAL, "conv: null pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (variant > 0)
    return conv_igemm_launch(p, x, w, bias, y, variant - 1, workspace, workspace_bytes, s);
  switch (dtype) {
    case ATK_F32: return launch_direct<float>(p, x, w, bias, y, s);
    case ATK_F16: return launch_direct<_Float16>(p, x, w, bias, y, s);
    default: return launch_direct<__bf16>(p, x, w, bias, y, s);
  }
}

// ---- packed-weight entry points (MFMA variants only) ------------------------------------
#define ATK_CONV_GEOM_ARGS                                                                          \
  int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int KD, int KH, int KW, int sd, \
      int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw, int dtype
#define ATK_CONV_GEOM N, Ci, D, H, W, Co, KD, KH, KW, sd, sh, sw, pd, ph, pw, dd, dh, dw, dtype

extern "C" size_t atk_conv_packed_weight_bytes(ATK_CONV_GEOM_ARGS, int variant) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(ATK_CONV_GEOM, p) || variant <= 0 || variant >= conv_num_variants()) return 0;
  return conv_igemm_packed_bytes(p, variant - 1);
}

extern "C" size_t atk_conv_prepacked_workspace_bytes(ATK_CONV_GEOM_ARGS, int variant) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(ATK_CONV_GEOM, p) || variant <= 0 || variant >= conv_num_variants()) return 0;
  return conv_igemm_prepacked_workspace_bytes(p, variant - 1);
}

extern "C" int atk_conv_pack_weights(const void* w, void* packed, size_t packed_bytes, ATK_CONV_GEOM_ARGS,
                                     int variant, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(ATK_CONV_GEOM, p);
  if (rc) return rc;
  if (variant <= 0 || variant >= conv_num_variants())
    return fail(variant == 0 ? ATK_UNSUPPORTED : ATK_EINVAL, "conv: variant %d has no packed weights", variant);
  if (!w) return fail(ATK_EINVAL, "conv: null weight pointer");
  return conv_igemm_pack(p, w, packed, packed_bytes, variant - 1, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int atk_conv_fwd_prepacked(const void* x, const void* packed, size_t packed_bytes, const void* bias,
                                      void* y, ATK_CONV_GEOM_ARGS, int variant, void* workspace,
                                      size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(ATK_CONV_GEOM, p);
  if (rc) return rc;
  if (variant <= 0 || variant >= conv_num_variants())
    return fail(variant == 0 ? ATK_UNSUPPORTED : ATK_EINVAL, "conv: variant %d has no packed weights", variant);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "conv: null pointer");
  return conv_igemm_run_prepacked(p, x, packed, packed_bytes, bias, y, variant - 1, workspace, workspace_bytes,
                                  reinterpret_cast<hipStream_t>(stream));
}

extern "C" int atk_conv_fwd_prepacked_cl(const void* x, const void* packed, size_t packed_bytes, const void* bias,
                                         void* y, ATK_CONV_GEOM_ARGS, int variant, void* workspace,
                                         size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(ATK_CONV_GEOM, p);
  if (rc) return rc;
  if (variant <= 0 || variant >= conv_num_variants())
    return fail(variant == 0 ? ATK_UNSUPPORTED : ATK_EINVAL, "conv: variant %d has no packed weights", variant);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "conv: null pointer");
  return conv_igemm_run_prepacked(p, x, packed, packed_bytes, bias, y, variant - 1, workspace, workspace_bytes,
                                  reinterpret_cast<hipStream_t>(stream), nullptr, nullptr, 0, 0, true);
}

extern "C" size_t atk_conv_gn_stats_bytes(ATK_CONV_GEOM_ARGS, int variant, int groups) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(ATK_CONV_GEOM, p) || variant <= 0 || variant >= conv_num_variants()) return 0;
  return conv_igemm_gn_stats_bytes(p, variant - 1, groups);
}

extern "C" int atk_conv_gn_records(ATK_CONV_GEOM_ARGS, int variant, int groups) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(ATK_CONV_GEOM, p) || variant <= 0 || variant >= conv_num_variants()) return 0;
  return conv_igemm_gn_records(p, variant - 1, groups);
}

extern "C" size_t atk_conv_gn_onepass_workspace_bytes(ATK_CONV_GEOM_ARGS, int variant, int groups) {
  using namespace atk;
  ConvShape p;
  if (conv_shape(ATK_CONV_GEOM, p) || variant <= 0 || variant >= conv_num_variants()) return 0;
  return conv_igemm_gn_onepass_bytes(p, variant - 1, groups);
}

extern "C" int atk_conv_group_norm_fwd(const void* x, const void* packed, size_t packed_bytes, const void* bias,
                                       const void* gamma, const void* beta, void* y, ATK_CONV_GEOM_ARGS,
                                       int variant, int groups, float eps, int silu, int param_dtype,
                                       void* workspace, size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(ATK_CONV_GEOM, p);
  if (rc) return rc;
  if (variant <= 0 || variant >= conv_num_variants())
    return fail(variant == 0 ? ATK_UNSUPPORTED : ATK_EINVAL, "conv: variant %d has no packed weights", variant);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "conv: null pointer");
  return conv_igemm_run_gn_onepass(p, x, packed, packed_bytes, bias, gamma, beta, param_dtype, eps, silu, y,
                                   variant - 1, groups, workspace, workspace_bytes,
                                   reinterpret_cast<hipStream_t>(stream));
}

extern "C" int atk_conv_fwd_prepacked_ex(const void* x, const void* packed, size_t packed_bytes, const void* bias,
                                         const void* residual, void* y, ATK_CONV_GEOM_ARGS, int variant,
                                         int gn_groups, void* gn_stats, size_t gn_stats_bytes, void* workspace,
                                         size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  ConvShape p;
  int rc = conv_shape(ATK_CONV_GEOM, p);
  if (rc) return rc;
  if (variant <= 0 || variant >= conv_num_variants())
    return fail(variant == 0 ? ATK_UNSUPPORTED : ATK_EINVAL, "conv: variant %d has no packed weights", variant);
  if (gn_stats && (gn_groups <= 0 || Co % gn_groups))
    return fail(ATK_EINVAL, "conv: %d GroupNorm groups do not divide %lld channels", gn_groups, (long long)Co);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "conv: null pointer");
  return conv_igemm_run_prepacked(p, x, packed, packed_bytes, bias, y, variant - 1, workspace, workspace_bytes,
                                  reinterpret_cast<hipStream_t>(stream), residual, gn_stats, gn_stats_bytes,
                                  gn_stats ? gn_groups : 0);
}

extern "C" int atk_conv_fwd_prepacked_args(const atk_conv_prepacked_args* a) {
  if (!a) return atk::fail(ATK_EINVAL, "conv: null argument block");
  return atk_conv_fwd_prepacked(a->x, a->packed, a->packed_bytes, a->bias, a->y, a->N, a->Ci, a->D, a->H, a->W, a->Co,
                                a->KD, a->KH, a->KW, a->sd, a->sh, a->sw, a->pd, a->ph, a->pw, a->dd, a->dh, a->dw,
                                a->dtype, a->variant, a->workspace, a->workspace_bytes, a->stream);
}
