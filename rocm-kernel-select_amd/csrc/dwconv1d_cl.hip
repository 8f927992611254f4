// Depthwise conv1d for gfx950, channels-last layout: element (b, t, c) of a sequence at
// b*sb + t*sl + c (channel stride 1).  Two reference layouts land here:
//   * FlashFFTConv's BLH depthwise conv1d, input (B, L, D), weight (K, D), symmetric
//     padding (amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/conv1d_blh.hip:54-220);
//   * causal-conv1d's channel-last kernel, x logically (B, D, L) with x.stride(1) == 1,
//     weight (D, K), pad = K-1, output length L, with seq_idx and initial / final states
//     (src/causal-conv1d-amd/csrc/causal_conv1d_fwd.cu:194-332, host checks
//     causal_conv1d.cpp:155-222).
//
//   y[b,t,c] = act(bias[c] + sum_{j<K} m(t,j) * w[c,j] * x[b, t - pad + j, c]),  t in [0, L_out)
//   x[b,p,c] = 0 for p >= L; for p < 0 it is initial_states[b, c, p + K - 1] when given, else 0;
//   m(t,j) = 1, or with seq_idx: seq(t - pad + j) == seq(t - pad + CUR) (seq(p < 0) = -1), where
//   the causal forward compares with the output position itself (CUR = K-1) and the input
//   gradient through the flipped conv (pad 0) compares with its own position (CUR = 0).
//   final_states[b, c, j] = x[b, L - (K-1) + j, c] (same extension for negative positions).
//
// Design (HBM-bound; no LDS): a thread owns VEC = 16 bytes of channels and a run of CL_RUN
// consecutive output positions.  It reads the CL_RUN + K - 1 input rows of its run as 16-byte
// buffer loads (rows outside [0, L) read zero through an out-of-range offset, no branches),
// keeps them in registers and slides the K-tap window over them; the K - 1 halo rows it
// shares with the previous run are L2 hits.  Threads are numbered channel-vector fastest, so
// a wave covers 64 adjacent 16-byte chunks of a row: every load and store is one coalesced
// 1 KiB segment.  Weights are read once per thread as fp32 (fp32 or 16-bit weights of any
// stride).  The weight gradient reduces per thread over a longer run into fp32 partials in a
// caller workspace, summed in a fixed order by a finalize kernel (deterministic).
#include <algorithm>
#include <utility>

#include "atk_common.h"

namespace atk {

namespace {

constexpr int CL_NT = 256;      // threads per block
constexpr int CL_RUN = 16;      // output positions per thread (forward)
constexpr int CL_KMAX = 8;      // widest kernel served
constexpr int CLW_STEP = 16;    // rows per unrolled step of the weight-gradient loop
constexpr int CLW_MAXRUN = 512; // longest per-thread run of the weight-gradient kernel

struct DwClArgs {
  const void* x;
  void* y;
  const void* w;
  const void* b;
  int wdt;                    // weight / bias dtype code
  int64_t wc, wk;             // weight strides (elements): channel, tap
  int wmode, bvec;            // weight / bias load forms (cl_params)
  const int* seq;             // [B, L] int32 or null
  const void* init;           // initial states or null
  int64_t ib, il;             // their batch / position strides (channel stride 1)
  void* fin;                  // final states or null
  int64_t fb, fl;
  int64_t xb, xl, yb, yl;     // element strides of x and y
  uint32_t B, D, L, Lout;
  int pad;
  uint32_t x_bytes, seq_bytes;  // buffer extents of this launch's x / seq
  uint32_t ncv, nrun;
  FastDiv div_ncv, div_nrun;
};

template <typename T>
__device__ __forceinline__ void unpack16(uint4 raw, float* f) {
  Vec16<T> v;
  v.raw = raw;
#pragma unroll
  for (int i = 0; i < Vec16<T>::N; ++i) f[i] = to_f32(v.e[i]);
}

// Weight / bias loads.  wmode 1: w is (D, K) contiguous, so a thread's VEC*K weights are one
// contiguous, 16-byte aligned block; wmode 2: w is tap-major (channel stride 1, tap stride a
// multiple of 16 bytes): one or two 16-byte loads per tap; wmode 0: element loads at any
// strides.  bvec: the bias is 16-byte aligned (vector load).  Weights and bias are fp32 or T.
template <typename T, int KT>
__device__ __forceinline__ void cl_params(const void* w, const void* bp, int wdt, int64_t wc, int64_t wk, int wmode,
                                          int bvec, uint32_t c0, float (&wv)[KT][16 / sizeof(T)],
                                          float (&bv)[16 / sizeof(T)]) {
  constexpr int VEC = 16 / sizeof(T);
  const bool f32 = wdt == ATK_F32;
  if (wmode == 1) {
    float f[VEC * KT];
    if (f32) {
      const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(w) + (size_t)c0 * KT);
#pragma unroll
      for (int i = 0; i < VEC * KT / 4; ++i) {
        const float4 u = q[i];
        f[4 * i] = u.x; f[4 * i + 1] = u.y; f[4 * i + 2] = u.z; f[4 * i + 3] = u.w;
      }
    } else {
      const uint4* q = reinterpret_cast<const uint4*>(static_cast<const T*>(w) + (size_t)c0 * KT);
#pragma unroll
      for (int i = 0; i < KT; ++i) unpack16<T>(q[i], f + i * VEC);
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v)
#pragma unroll
      for (int j = 0; j < KT; ++j) wv[j][v] = f[v * KT + j];
  } else if (wmode == 2) {
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      if (f32) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(w) + (size_t)j * wk + c0);
#pragma unroll
        for (int i = 0; i < VEC / 4; ++i) {
          const float4 u = q[i];
          wv[j][4 * i] = u.x; wv[j][4 * i + 1] = u.y; wv[j][4 * i + 2] = u.z; wv[j][4 * i + 3] = u.w;
        }
      } else {
        unpack16<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(w) + (size_t)j * wk + c0), wv[j]);
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
#pragma unroll
      for (int j = 0; j < KT; ++j) wv[j][v] = load_param(w, wdt, (int64_t)(c0 + v) * wc + (int64_t)j * wk);
  }
  if (!bp) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) bv[v] = 0.f;
  } else if (bvec) {
    if (f32) {
      const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(bp) + c0);
#pragma unroll
      for (int i = 0; i < VEC / 4; ++i) {
        const float4 u = q[i];
        bv[4 * i] = u.x; bv[4 * i + 1] = u.y; bv[4 * i + 2] = u.z; bv[4 * i + 3] = u.w;
      }
    } else {
      unpack16<T>(*reinterpret_cast<const uint4*>(static_cast<const T*>(bp) + c0), bv);
    }
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) bv[v] = load_param(bp, wdt, c0 + v);
  }
}

// SEQ: 0 = no seq_idx, 1 = compare with the last tap's row (causal forward, pad = K-1),
// 2 = compare with the first tap's row (flipped input-gradient conv, pad = 0).
template <typename T, int KT, bool SILU, int SEQ>
__global__ __launch_bounds__(CL_NT) void dwconv1d_cl_kernel(DwClArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int R = CL_RUN + KT - 1;
  const uint32_t g = blockIdx.x * CL_NT + threadIdx.x;
  const uint32_t rest = fdiv(g, a.div_ncv);
  const uint32_t cv = g - rest * a.ncv;
  const uint32_t b = fdiv(rest, a.div_nrun);
  const uint32_t r = rest - b * a.nrun;
  if (b >= a.B) return;
  const int t0 = (int)(r * CL_RUN);
  const int p0 = t0 - a.pad;
  const uint32_t c0 = cv * VEC;

  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, a.x_bytes);
  const uint32_t xbase = (uint32_t)(b * a.xb + c0) * (uint32_t)sizeof(T);
  const uint32_t xrow = (uint32_t)a.xl * (uint32_t)sizeof(T);
  uint4 raw[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int p = p0 + i;
    raw[i] = bload16(rs, (p >= 0 && p < (int)a.L) ? xbase + (uint32_t)p * xrow : kOOB, 0);
  }
  int s[SEQ ? R : 1];
  if constexpr (SEQ != 0) {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.seq, a.seq_bytes);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int p = p0 + i;
      const bool in = p >= 0 && p < (int)a.L;
      const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(rq, in ? (b * a.L + (uint32_t)p) * 4u : kOOB, 0, 0);
      s[i] = in ? v : -1;
    }
  }
  float wv[KT][VEC], bv[VEC];
  cl_params<T, KT>(a.w, a.b, a.wdt, a.wc, a.wk, a.wmode, a.bvec, c0, wv, bv);
  // rows before the sequence come from the initial states (causal form only: pad == K-1)
  if (a.init && p0 < 0) {
    const T* ip = static_cast<const T*>(a.init) + (int64_t)b * a.ib + c0;
#pragma unroll
    for (int i = 0; i < KT - 1; ++i)
      if (p0 + i < 0) raw[i] = ld16<false>(ip + (int64_t)(p0 + i + KT - 1) * a.il);
  }

  T* yp = static_cast<T*>(a.y) + (int64_t)b * a.yb + c0;
#pragma unroll
  for (int i = 0; i < CL_RUN; ++i) {
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = bv[v];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      float xf[VEC];
      unpack16<T>(raw[i + j], xf);
      bool m = true;
      if constexpr (SEQ == 1) m = s[i + j] == s[i + KT - 1];
      if constexpr (SEQ == 2) m = s[i + j] == s[i];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = __builtin_fmaf(wv[j][v], m ? xf[v] : 0.f, acc[v]);
    }
    if constexpr (SILU) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = silu_f32(acc[v]);
    }
    const int t = t0 + i;
    if (t < (int)a.Lout) st16<false>(yp + (int64_t)t * a.yl, pack16<T>(acc));
  }

  // final states: the thread whose run holds the last position writes the last K-1 rows
  if (a.fin && t0 <= (int)a.L - 1 && (int)a.L - 1 < t0 + CL_RUN) {
    const T* xp = static_cast<const T*>(a.x) + (int64_t)b * a.xb + c0;
    T* fp = static_cast<T*>(a.fin) + (int64_t)b * a.fb + c0;
#pragma unroll
    for (int j = 0; j < KT - 1; ++j) {
      const int p = (int)a.L - (KT - 1) + j;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (p >= 0) v = ld16<false>(xp + (int64_t)p * a.xl);
      else if (a.init) v = ld16<false>(static_cast<const T*>(a.init) + (int64_t)b * a.ib + c0 + (int64_t)(p + KT - 1) * a.il);
      st16<false>(fp + (int64_t)j * a.fl, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Weight / bias gradient:  dw[c,j] = sum_{b,t} dy[b,t,c] * m(t,j) * x[b, t - pad + j, c],
// db[c] = sum_{b,t} dy[b,t,c], over t in [0, L_out), with x extended as in the forward.
// ---------------------------------------------------------------------------
struct DwClBwArgs {
  const void* x;
  const void* dy;
  const int* seq;
  const void* init;
  int64_t ib, il;
  int64_t xb, xl, gb, gl;     // element strides of x and dy
  uint32_t B, D, L, Lout;
  int pad;
  uint32_t x_bytes, g_bytes, seq_bytes;
  uint32_t ncv, nrw, run;     // run: positions per thread (multiple of CLW_STEP)
  FastDiv div_ncv, div_nrw;
  float* part;                // [B * nrw][K + 1][D]
  float* dw;                  // [D, K] fp32
  float* db;                  // [D] fp32 or null
  uint32_t P;                 // partial rows = B * nrw
};

template <typename T, int KT, int SEQ>
__global__ __launch_bounds__(CL_NT) void dwconv1d_cl_bwd_w_kernel(DwClBwArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int H = KT - 1;  // rows carried between steps
  const uint32_t g = blockIdx.x * CL_NT + threadIdx.x;
  const uint32_t rest = fdiv(g, a.div_ncv);
  const uint32_t cv = g - rest * a.ncv;
  const uint32_t b = fdiv(rest, a.div_nrw);
  const uint32_t rw = rest - b * a.nrw;
  if (b >= a.B) return;
  const uint32_t c0 = cv * VEC;
  const int t0 = (int)(rw * a.run);
  const int t1 = min((int)(t0 + a.run), (int)a.Lout);

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.dy, a.g_bytes);
  const uint32_t xbase = (uint32_t)(b * a.xb + c0) * (uint32_t)sizeof(T);
  const uint32_t gbase = (uint32_t)(b * a.gb + c0) * (uint32_t)sizeof(T);
  const uint32_t xrow = (uint32_t)a.xl * (uint32_t)sizeof(T);
  const uint32_t grow = (uint32_t)a.gl * (uint32_t)sizeof(T);
  auto xoff = [&](int p) { return (p >= 0 && p < (int)a.L) ? xbase + (uint32_t)p * xrow : kOOB; };
  __amdgpu_buffer_rsrc_t rq;
  if constexpr (SEQ != 0) rq = make_rsrc(a.seq, a.seq_bytes);
  auto seq_at = [&](int p) {
    const bool in = p >= 0 && p < (int)a.L;
    const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(rq, in ? (b * a.L + (uint32_t)p) * 4u : kOOB, 0, 0);
    return in ? v : -1;
  };

  float acc[KT][VEC], accb[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    accb[v] = 0.f;
#pragma unroll
    for (int j = 0; j < KT; ++j) acc[j][v] = 0.f;
  }
  // carried window: the H input rows before the current step's first tap row
  float hx[H > 0 ? H : 1][VEC];
  int hs[H > 0 ? H : 1];
  const int q0 = t0 - a.pad;  // input row of tap 0 for output t0
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int p = q0 + i;
    uint4 rv = bload16(rx, xoff(p), 0);
    if (a.init && p < 0 && p >= -H)
      rv = ld16<false>(static_cast<const T*>(a.init) + (int64_t)b * a.ib + c0 + (int64_t)(p + H) * a.il);
    unpack16<T>(rv, hx[i]);
    if constexpr (SEQ != 0) hs[i] = seq_at(p);
  }
  for (int t = t0; t < t1; t += CLW_STEP) {
    uint4 gr[CLW_STEP], xr[CLW_STEP];
    int sr[SEQ ? CLW_STEP : 1];
#pragma unroll
    for (int i = 0; i < CLW_STEP; ++i) {
      const int tt = t + i;
      gr[i] = bload16(rg, tt < t1 ? gbase + (uint32_t)tt * grow : kOOB, 0);
      const int p = tt - a.pad + H;  // newest tap row of output tt
      xr[i] = bload16(rx, xoff(p), 0);
      if constexpr (SEQ != 0) sr[i] = seq_at(p);
    }
    // (with initial states pad == K-1, so the newest tap row t + i is never negative)
#pragma unroll
    for (int i = 0; i < CLW_STEP; ++i) {
      float gf[VEC], xn[VEC];
      unpack16<T>(gr[i], gf);
      unpack16<T>(xr[i], xn);
      const int cur = SEQ ? sr[i] : 0;  // seq of the output position itself (pad == K-1)
#pragma unroll
      for (int v = 0; v < VEC; ++v) accb[v] += gf[v];
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const float* xs = j < H ? hx[j] : xn;
        bool m = true;
        if constexpr (SEQ != 0) m = (j < H ? hs[j] : sr[i]) == cur;
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[j][v] = __builtin_fmaf(gf[v], m ? xs[v] : 0.f, acc[j][v]);
      }
      // slide the window by one row
#pragma unroll
      for (int j = 0; j + 1 < H; ++j) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) hx[j][v] = hx[j + 1][v];
        if constexpr (SEQ != 0) hs[j] = hs[j + 1];
      }
      if constexpr (H > 0) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) hx[H - 1][v] = xn[v];
        if constexpr (SEQ != 0) hs[H - 1] = sr[i];
      }
    }
  }
  // outputs past t1 inside the last step were loaded with dy = 0: they add nothing
  float* pp = a.part + (size_t)(b * a.nrw + rw) * (KT + 1) * a.D + c0;
#pragma unroll
  for (int j = 0; j < KT; ++j)
#pragma unroll
    for (int v = 0; v < VEC; v += 4)
      *reinterpret_cast<float4*>(pp + (size_t)j * a.D + v) = make_float4(acc[j][v], acc[j][v + 1], acc[j][v + 2], acc[j][v + 3]);
#pragma unroll
  for (int v = 0; v < VEC; v += 4)
    *reinterpret_cast<float4*>(pp + (size_t)KT * a.D + v) = make_float4(accb[v], accb[v + 1], accb[v + 2], accb[v + 3]);
}

// Sum the P partial rows of each (tap, channel) in a fixed order: a block covers CLF_COLS
// columns, CLF_SPLIT threads per column each sum every CLF_SPLIT-th row, and the CLF_SPLIT
// sums are added in order through LDS (deterministic for a given P).
constexpr int CLF_COLS = 32, CLF_SPLIT = 8;
__global__ __launch_bounds__(CLF_COLS * CLF_SPLIT) void dwconv1d_cl_bwd_finalize_kernel(DwClBwArgs a, int K) {
  __shared__ float red[CLF_SPLIT][CLF_COLS];
  const int tx = threadIdx.x % CLF_COLS, ty = threadIdx.x / CLF_COLS;
  const uint32_t ncol = (uint32_t)(K + 1) * a.D;
  const uint32_t i = blockIdx.x * CLF_COLS + tx;  // column: (tap or bias row) * D + channel
  float s0 = 0.f, s1 = 0.f;
  if (i < ncol) {
    const float* p = a.part + i;
    uint32_t q = ty;
    for (; q + CLF_SPLIT < a.P; q += 2 * CLF_SPLIT) {
      s0 += p[(size_t)q * ncol];
      s1 += p[(size_t)(q + CLF_SPLIT) * ncol];
    }
    if (q < a.P) s0 += p[(size_t)q * ncol];
  }
  red[ty][tx] = s0 + s1;
  __syncthreads();
  if (ty == 0 && i < ncol) {
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < CLF_SPLIT; ++t) s += red[t][tx];
    const uint32_t j = i / a.D, c = i - j * a.D;
    if (j < (uint32_t)K) a.dw[(size_t)c * K + j] = s;
    else if (a.db) a.db[c] = s;
  }
}

// ---------------------------------------------------------------------------
// Backward, fused (src/causal-conv1d-amd/csrc/causal_conv1d_bwd.cu channel-last path, and
// the (B, L, C) depthwise conv1d backward of conv1d_bwd_hip_bhl.hip): with H = K-1 and z[t]
// the pre-activation of the forward (recomputed here in fp32; causal form only),
//   g[t]  = dout[t] * silu'(z[t])   (or dout[t] without the activation),
//   dx[q] = sum_j w[j] * g[q + H - j] * [seq(q) == seq(q + H - j)],
//   dw[j] = sum_t g[t] * x[t - H + j] * [seq(t - H + j) == seq(t)],  db = sum_t g[t].
// Any left padding P and output length L_out reduce to that form by a shift sh = H - P: the
// kernel walks u over the union of [0, L_out) (dout rows) and [-sh, L - sh) (dx rows), reads
// x at u + sh (x~[u] = x[u + sh]) and stores dx[u + sh]; with x~ the sums above read
//   dx[u + sh] = sum_j w[j] g[u + H - j],   dw[j] = sum_t g[t] x~[t - H + j] = sum_t g[t] x[t - P + j],
// i.e. dx[q] = sum_j w[j] g[q + P - j], the depthwise conv's input gradient.  dout rows outside
// [0, L_out) read zero and so add nothing.  The causal form is sh = 0, L_out = L.
// A thread owns VEC channels and a span of positions, walked in steps of CLB_STEP rows.
// Each step loads the CLB_STEP new dout / x rows at positions [p + H, p + H + STEP) and keeps
// the 2H x rows and H gradient rows that the next step shares as carried registers, so dout
// and x are each read once.  dw / db leave as fp32 partials per span (finalize kernel above).
// ---------------------------------------------------------------------------
constexpr int CLB_STEP = 8;

struct DwClCbArgs {
  const void* x;
  const void* dy;
  void* dx;
  const void* w;
  const void* b;
  int wdt;
  int64_t wc, wk;
  int wmode, bvec;
  const int* seq;
  const void* init;
  int64_t ib, il;
  int64_t xb, xl, gb, gl, ob, ol;  // element strides of x, dout, dx
  uint32_t B, D, L;
  uint32_t Lout;                   // dout rows (L in the causal form)
  int sh, u0;                      // x / dx shift H - P; first loop position min(0, -sh)
  int u1;                          // loop end max(L_out, L - sh)
  uint32_t x_bytes, g_bytes, seq_bytes;
  uint32_t ncv, nspan, span;       // span: positions per thread, a multiple of CLB_STEP
  FastDiv div_ncv, div_nspan;
  float* part;                     // [B * nspan][K + 1][D]
};

__device__ __forceinline__ float dsilu_f32(float z) {
  const float s = __builtin_amdgcn_rcpf(1.0f + __expf(-z));
  return s * (1.0f + z * (1.0f - s));
}

template <typename T, int KT, bool SILU, bool SEQ>
__global__ __launch_bounds__(CL_NT) void dwconv1d_cl_causal_bwd_kernel(DwClCbArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int H = KT - 1;
  constexpr int S = CLB_STEP;
  constexpr int XC = 2 * H > 0 ? 2 * H : 1, GC = H > 0 ? H : 1;
  static_assert(S >= 2 * H, "carried rows come from one step");
  const uint32_t g = blockIdx.x * CL_NT + threadIdx.x;
  const uint32_t rest = fdiv(g, a.div_ncv);
  const uint32_t cv = g - rest * a.ncv;
  const uint32_t b = fdiv(rest, a.div_nspan);
  const uint32_t sp = rest - b * a.nspan;
  if (b >= a.B) return;
  const uint32_t c0 = cv * VEC;
  const int p_start = a.u0 + (int)(sp * a.span);
  const int p_end = min(p_start + (int)a.span, a.u1);

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.dy, a.g_bytes);
  const uint32_t xbase = (uint32_t)(b * a.xb + c0) * (uint32_t)sizeof(T);
  const uint32_t gbase = (uint32_t)(b * a.gb + c0) * (uint32_t)sizeof(T);
  const uint32_t xrow = (uint32_t)a.xl * (uint32_t)sizeof(T);
  const uint32_t grow = (uint32_t)a.gl * (uint32_t)sizeof(T);
  const int L = (int)a.L, Lout = (int)a.Lout, sh = a.sh;
  auto xld = [&](int p) {
    const int q = p + sh;
    return bload16(rx, (q >= 0 && q < L) ? xbase + (uint32_t)q * xrow : kOOB, 0);
  };
  auto gld = [&](int t) { return bload16(rg, (t >= 0 && t < Lout) ? gbase + (uint32_t)t * grow : kOOB, 0); };
  __amdgpu_buffer_rsrc_t rq;
  if constexpr (SEQ) rq = make_rsrc(a.seq, a.seq_bytes);
  auto seq_at = [&](int p) {
    const bool in = p >= 0 && p < L;
    const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(rq, in ? (b * a.L + (uint32_t)p) * 4u : kOOB, 0, 0);
    return in ? v : -1;
  };

  float wv[KT][VEC], bv[VEC];
  cl_params<T, KT>(a.w, SILU ? a.b : nullptr, a.wdt, a.wc, a.wk, a.wmode, a.bvec, c0, wv, bv);

  float xc[XC][VEC];  // x rows [p - H, p + H)
  int sc[XC];
  float gc[GC][VEC];  // gradient rows [p, p + H)
  {
    // prologue: x rows [p_start - 2H, p_start + H), dout rows [p_start, p_start + H)
    constexpr int PR = 3 * H > 0 ? 3 * H : 1;
    float xp[PR][VEC];
    int spv[PR];
#pragma unroll
    for (int k = 0; k < 3 * H; ++k) {
      const int pos = p_start - 2 * H + k;
      uint4 r = xld(pos);
      if (a.init && pos < 0 && pos >= -H)
        r = ld16<false>(static_cast<const T*>(a.init) + (int64_t)b * a.ib + c0 + (int64_t)(pos + H) * a.il);
      unpack16<T>(r, xp[k]);
      spv[k] = SEQ ? seq_at(pos) : 0;
    }
#pragma unroll
    for (int k = 0; k < H; ++k) {
      float gf[VEC];
      unpack16<T>(gld(p_start + k), gf);
      if constexpr (SILU) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          float z = bv[v];
#pragma unroll
          for (int j = 0; j < KT; ++j) {
            const bool m = !SEQ || spv[k + H + j] == spv[k + 2 * H];
            z = __builtin_fmaf(wv[j][v], m ? xp[k + H + j][v] : 0.f, z);
          }
          gf[v] *= dsilu_f32(z);
        }
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) gc[k][v] = gf[v];
    }
#pragma unroll
    for (int k = 0; k < 2 * H; ++k) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xc[k][v] = xp[H + k][v];
      sc[k] = spv[H + k];
    }
  }

  float acc[KT][VEC], accb[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    accb[v] = 0.f;
#pragma unroll
    for (int j = 0; j < KT; ++j) acc[j][v] = 0.f;
  }
  T* op = static_cast<T*>(a.dx) + (int64_t)b * a.ob + c0;

  for (int p = p_start; p < p_end; p += S) {
    uint4 xr[S], gr[S];
    int sr[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      xr[i] = xld(p + H + i);
      gr[i] = gld(p + H + i);
      sr[i] = SEQ ? seq_at(p + H + i) : 0;
    }
    // x rows [p - H, p + H + S): combined index k -> xc[k] (k < 2H) or new row k - 2H
    float xn[S][VEC];
#pragma unroll
    for (int i = 0; i < S; ++i) unpack16<T>(xr[i], xn[i]);
#define XAT(k, v) ((k) < 2 * H ? xc[(k) < 2 * H ? (k) : 0][v] : xn[(k) < 2 * H ? 0 : (k) - 2 * H][v])
#define SAT(k) ((k) < 2 * H ? sc[(k) < 2 * H ? (k) : 0] : sr[(k) < 2 * H ? 0 : (k) - 2 * H])
    // new gradient rows t = p + H + i
    float gn[S][VEC];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      unpack16<T>(gr[i], gn[i]);
      if constexpr (SILU) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          float z = bv[v];
#pragma unroll
          for (int j = 0; j < KT; ++j) {  // x rows t - H + j = combined index i + H + j
            const bool m = !SEQ || SAT(i + H + j) == SAT(i + 2 * H);
            z = __builtin_fmaf(wv[j][v], m ? XAT(i + H + j, v) : 0.f, z);
          }
          gn[i][v] *= dsilu_f32(z);
        }
      }
    }
    // gradient rows [p, p + H + S): combined index k -> gc[k] (k < H) or gn[k - H]
#define GAT(k, v) ((k) < H ? gc[(k) < H ? (k) : 0][v] : gn[(k) < H ? 0 : (k) - H][v])
#pragma unroll
    for (int i = 0; i < S; ++i) {
      // dx[q], q = p + i
      float d[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) d[v] = 0.f;
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const bool m = !SEQ || SAT(i + 2 * H - j) == SAT(i + H);
#pragma unroll
        for (int v = 0; v < VEC; ++v) d[v] = __builtin_fmaf(wv[j][v], m ? GAT(i + H - j, v) : 0.f, d[v]);
      }
      const int q = p + i + sh;
      if (q >= 0 && q < L) st16<false>(op + (int64_t)q * a.ol, pack16<T>(d));
      // dw / db for t = p + i (rows outside [0, L_out) carry a zero gradient)
#pragma unroll
      for (int v = 0; v < VEC; ++v) accb[v] += GAT(i, v);
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        const bool m = !SEQ || SAT(i + j) == SAT(i + H);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[j][v] = __builtin_fmaf(GAT(i, v), m ? XAT(i + j, v) : 0.f, acc[j][v]);
      }
    }
    // carry: gradient rows [p + S, p + S + H) and x rows [p + S - H, p + S + H)
#pragma unroll
    for (int k = 0; k < H; ++k)
#pragma unroll
      for (int v = 0; v < VEC; ++v) gc[k][v] = gn[S + k - H][v];
#pragma unroll
    for (int k = 0; k < 2 * H; ++k) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xc[k][v] = xn[S + k - 2 * H][v];
      sc[k] = sr[S + k - 2 * H];
    }
#undef XAT
#undef SAT
#undef GAT
  }
  float* pp = a.part + (size_t)(b * a.nspan + sp) * (KT + 1) * a.D + c0;
#pragma unroll
  for (int j = 0; j < KT; ++j)
#pragma unroll
    for (int v = 0; v < VEC; v += 4)
      *reinterpret_cast<float4*>(pp + (size_t)j * a.D + v) = make_float4(acc[j][v], acc[j][v + 1], acc[j][v + 2], acc[j][v + 3]);
#pragma unroll
  for (int v = 0; v < VEC; v += 4)
    *reinterpret_cast<float4*>(pp + (size_t)KT * a.D + v) = make_float4(accb[v], accb[v + 1], accb[v + 2], accb[v + 3]);
}

// --------------------------------------------------------------------------- launchers
template <typename T, int KT, bool SILU, int SEQ>
void launch_cl_k(const DwClArgs& a, uint32_t blocks, hipStream_t s) {
  hipLaunchKernelGGL((dwconv1d_cl_kernel<T, KT, SILU, SEQ>), dim3(blocks), dim3(CL_NT), 0, s, a);
}

template <typename T, int KT>
int launch_cl_kt(const DwClArgs& a, uint32_t blocks, int silu, int seq, hipStream_t s) {
  if (seq != 0 && KT > 4) return ATK_UNSUPPORTED;
  if (seq == 0) {
    if (silu) launch_cl_k<T, KT, true, 0>(a, blocks, s);
    else launch_cl_k<T, KT, false, 0>(a, blocks, s);
  } else if constexpr (KT <= 4) {
    if (seq == 1) {
      if (silu) launch_cl_k<T, KT, true, 1>(a, blocks, s);
      else launch_cl_k<T, KT, false, 1>(a, blocks, s);
    } else {
      if (silu) launch_cl_k<T, KT, true, 2>(a, blocks, s);
      else launch_cl_k<T, KT, false, 2>(a, blocks, s);
    }
  }
  return ATK_OK;
}

template <typename T>
int launch_cl(const DwClArgs& a, int K, uint32_t blocks, int silu, int seq, hipStream_t s) {
  switch (K) {
    case 1: return launch_cl_kt<T, 1>(a, blocks, silu, seq, s);
    case 2: return launch_cl_kt<T, 2>(a, blocks, silu, seq, s);
    case 3: return launch_cl_kt<T, 3>(a, blocks, silu, seq, s);
    case 4: return launch_cl_kt<T, 4>(a, blocks, silu, seq, s);
    case 5: return launch_cl_kt<T, 5>(a, blocks, silu, seq, s);
    case 6: return launch_cl_kt<T, 6>(a, blocks, silu, seq, s);
    case 7: return launch_cl_kt<T, 7>(a, blocks, silu, seq, s);
    case 8: return launch_cl_kt<T, 8>(a, blocks, silu, seq, s);
    default: return ATK_UNSUPPORTED;
  }
}

template <typename T, int KT>
void launch_clw_kt(const DwClBwArgs& a, uint32_t blocks, int seq, hipStream_t s) {
  if (seq == 0) hipLaunchKernelGGL((dwconv1d_cl_bwd_w_kernel<T, KT, 0>), dim3(blocks), dim3(CL_NT), 0, s, a);
  else hipLaunchKernelGGL((dwconv1d_cl_bwd_w_kernel<T, KT, 1>), dim3(blocks), dim3(CL_NT), 0, s, a);
}

template <typename T>
int launch_clw(const DwClBwArgs& a, int K, uint32_t blocks, int seq, hipStream_t s) {
  switch (K) {
    case 1: launch_clw_kt<T, 1>(a, blocks, seq, s); return ATK_OK;
    case 2: launch_clw_kt<T, 2>(a, blocks, seq, s); return ATK_OK;
    case 3: launch_clw_kt<T, 3>(a, blocks, seq, s); return ATK_OK;
    case 4: launch_clw_kt<T, 4>(a, blocks, seq, s); return ATK_OK;
    case 5: launch_clw_kt<T, 5>(a, blocks, seq, s); return ATK_OK;
    default: return ATK_UNSUPPORTED;
  }
}

template <typename T, int KT>
void launch_clb_kt(const DwClCbArgs& a, uint32_t blocks, int silu, bool seq, hipStream_t s) {
  if (silu) {
    if (seq) hipLaunchKernelGGL((dwconv1d_cl_causal_bwd_kernel<T, KT, true, true>), dim3(blocks), dim3(CL_NT), 0, s, a);
    else hipLaunchKernelGGL((dwconv1d_cl_causal_bwd_kernel<T, KT, true, false>), dim3(blocks), dim3(CL_NT), 0, s, a);
  } else {
    if (seq) hipLaunchKernelGGL((dwconv1d_cl_causal_bwd_kernel<T, KT, false, true>), dim3(blocks), dim3(CL_NT), 0, s, a);
    else hipLaunchKernelGGL((dwconv1d_cl_causal_bwd_kernel<T, KT, false, false>), dim3(blocks), dim3(CL_NT), 0, s, a);
  }
}

template <typename T>
int launch_clb(const DwClCbArgs& a, int K, uint32_t blocks, int silu, bool seq, hipStream_t s) {
  switch (K) {
    case 2: launch_clb_kt<T, 2>(a, blocks, silu, seq, s); return ATK_OK;
    case 3: launch_clb_kt<T, 3>(a, blocks, silu, seq, s); return ATK_OK;
    case 4: launch_clb_kt<T, 4>(a, blocks, silu, seq, s); return ATK_OK;
    default: return ATK_UNSUPPORTED;
  }
}

// Per-thread run of the weight-gradient kernel: long enough that the partials stay small,
// short enough that about 64K threads are in flight.
uint32_t clw_run(int64_t B, int64_t D, int64_t Lout, int vec) {
  const int64_t ncv = D / vec;
  int64_t run = CLW_STEP;
  while (run < CLW_MAXRUN && B * ncv * ((Lout + run - 1) / run) > 65536) run *= 2;
  return (uint32_t)run;
}

// Load forms of cl_params for a weight at (w_stride_c, w_stride_k) and a bias.
void cl_param_modes(const void* w, const void* bias, int w_dtype, int K, int64_t wc, int64_t wk, int vec, int* wmode,
                    int* bvec) {
  const int64_t wes = (int64_t)dtype_size(w_dtype);
  *wmode = 0;
  if (aligned16(w)) {
    if (wk == 1 && wc == K) *wmode = 1;  // c0 * K * wes is a multiple of 16 since c0 is of vec
    else if (wc == 1 && (wk * wes) % 16 == 0 && (vec * wes) % 16 == 0) *wmode = 2;
  }
  if (*wmode == 1 && (vec * K * wes) % 16 != 0) *wmode = 0;
  *bvec = bias && aligned16(bias) && (vec * wes) % 16 == 0;
}

// Checks shared by both entry points; returns the vector width or an error code (< 0).
int cl_check(const void* x, int64_t B, int64_t D, int64_t L, int K, int dtype, int64_t xb, int64_t xl) {
  if (!x || !dtype_ok(dtype)) return -ATK_EINVAL;
  if (B <= 0 || D <= 0 || L <= 0 || K < 1) return -ATK_EINVAL;
  const int vec = 16 / (int)dtype_size(dtype);
  if (K > CL_KMAX || D % vec || xb % vec || xl % vec || !aligned16(x)) return -ATK_UNSUPPORTED;
  if (xl < D || xb < 0 || L > (1 << 30)) return -ATK_UNSUPPORTED;
  return vec;
}

// Batches per launch so that every byte offset inside one launch's x fits the 31-bit range
// the buffer loads use.
int64_t cl_batches_per_launch(int64_t B, int64_t xb, int64_t span_elems, size_t es) {
  const int64_t limit = (int64_t)1 << 31;
  if ((int64_t)(span_elems * (int64_t)es) >= limit) return 0;
  if (xb <= 0) return B;
  return std::max<int64_t>(0, std::min<int64_t>(B, (limit - span_elems * (int64_t)es) / (xb * (int64_t)es) + 1));
}

}  // namespace
}  // namespace atk

extern "C" int atk_dwconv1d_cl_fwd(const void* x, const void* w, const void* bias, void* y, const int* seq_idx,
                                   const void* initial_states, void* final_states, int64_t B, int64_t D,
                                   int64_t L, int K, int pad_left, int64_t L_out, int64_t x_stride_b,
                                   int64_t x_stride_l, int64_t y_stride_b, int64_t y_stride_l, int64_t w_stride_c,
                                   int64_t w_stride_k, int64_t is_stride_b, int64_t is_stride_l,
                                   int64_t fs_stride_b, int64_t fs_stride_l, int dtype, int w_dtype,
                                   int fuse_silu, int seq_mode, atk_stream_t stream) {
  using namespace atk;
  const int vec = cl_check(x, B, D, L, K, dtype, x_stride_b, x_stride_l);
  if (vec < 0) return fail(-vec, "dwconv1d_cl_fwd: unsupported shape/layout (D and strides in 16-byte units, K <= 8)");
  if (!w || !y || !dtype_ok(w_dtype) || L_out <= 0 || pad_left < 0 || L_out > (1 << 30))
    return fail(ATK_EINVAL, "dwconv1d_cl_fwd: bad arguments");
  if (y_stride_b % vec || y_stride_l % vec || y_stride_l < D || !aligned16(y))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: output layout");
  const bool causal = pad_left == K - 1 && L_out == L;
  if ((initial_states || final_states) && !causal)
    return fail(ATK_EINVAL, "dwconv1d_cl_fwd: states need the causal form (pad K-1, L_out = L)");
  if (seq_mode < 0 || seq_mode > 2 || (seq_mode != 0) != (seq_idx != nullptr))
    return fail(ATK_EINVAL, "dwconv1d_cl_fwd: seq_mode must be 1 or 2 exactly when seq_idx is given");
  if ((seq_mode == 1 && pad_left != K - 1) || (seq_mode == 2 && pad_left != 0))
    return fail(ATK_EINVAL, "dwconv1d_cl_fwd: seq_idx needs pad K-1 (mode 1) or 0 (mode 2)");
  if (seq_mode && K > 4) return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: seq_idx for K <= 4");
  if (initial_states && (is_stride_b % vec || is_stride_l % vec || !aligned16(initial_states)))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: initial_states layout");
  if (final_states && (fs_stride_b % vec || fs_stride_l % vec || !aligned16(final_states)))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: final_states layout");
  if (seq_idx && (uint64_t)B * (uint64_t)L * 4u >= (1ull << 31))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: seq_idx larger than 2 GiB");
  const size_t es = dtype_size(dtype);
  const int64_t span = (L - 1) * x_stride_l + D;
  const int64_t per = cl_batches_per_launch(B, x_stride_b, span, es);
  if (per <= 0) return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: one sequence spans 2 GiB");
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int64_t b0 = 0; b0 < B; b0 += per) {
    const int64_t nb = std::min(per, B - b0);
    DwClArgs a{};
    a.x = static_cast<const char*>(x) + b0 * x_stride_b * (int64_t)es;
    a.y = static_cast<char*>(y) + b0 * y_stride_b * (int64_t)es;
    a.w = w; a.b = bias; a.wdt = w_dtype; a.wc = w_stride_c; a.wk = w_stride_k;
    cl_param_modes(w, bias, w_dtype, K, w_stride_c, w_stride_k, vec, &a.wmode, &a.bvec);
    a.seq = seq_idx ? seq_idx + b0 * L : nullptr;
    a.init = initial_states ? static_cast<const char*>(initial_states) + b0 * is_stride_b * (int64_t)es : nullptr;
    a.ib = is_stride_b; a.il = is_stride_l;
    a.fin = final_states ? static_cast<char*>(final_states) + b0 * fs_stride_b * (int64_t)es : nullptr;
    a.fb = fs_stride_b; a.fl = fs_stride_l;
    a.xb = x_stride_b; a.xl = x_stride_l; a.yb = y_stride_b; a.yl = y_stride_l;
    a.B = (uint32_t)nb; a.D = (uint32_t)D; a.L = (uint32_t)L; a.Lout = (uint32_t)L_out; a.pad = pad_left;
    a.x_bytes = (uint32_t)(((nb - 1) * x_stride_b + span) * (int64_t)es);
    a.seq_bytes = (uint32_t)(nb * L * 4);
    a.ncv = (uint32_t)(D / vec);
    a.nrun = (uint32_t)((L_out + CL_RUN - 1) / CL_RUN);
    a.div_ncv = make_fastdiv(a.ncv);
    a.div_nrun = make_fastdiv(a.nrun);
    const uint64_t threads = (uint64_t)nb * a.nrun * a.ncv;
    if (threads + CL_NT >= (1ull << 31)) return fail(ATK_UNSUPPORTED, "dwconv1d_cl_fwd: too many threads");
    const uint32_t blocks = (uint32_t)((threads + CL_NT - 1) / CL_NT);
    int rc;
    if (dtype == ATK_F32) rc = launch_cl<float>(a, K, blocks, fuse_silu, seq_mode, s);
    else if (dtype == ATK_F16) rc = launch_cl<_Float16>(a, K, blocks, fuse_silu, seq_mode, s);
    else rc = launch_cl<__bf16>(a, K, blocks, fuse_silu, seq_mode, s);
      if (rc != ATK_OK) return fail(rc, "dwconv1d_cl_fwd: kernel width not served");
    if (check_launch("dwconv1d_cl_fwd") != ATK_OK) return ATK_ELAUNCH;
  }
  return ATK_OK;
}

extern "C" size_t atk_dwconv1d_cl_bwd_weight_workspace_bytes(int64_t B, int64_t D, int64_t L_out, int K,
                                                             int dtype) {
  using namespace atk;
  if (B <= 0 || D <= 0 || L_out <= 0 || K < 1 || !dtype_ok(dtype)) return 0;
  const int vec = 16 / (int)dtype_size(dtype);
  const uint32_t run = clw_run(B, D, L_out, vec);
  const int64_t nrw = (L_out + run - 1) / run;
  return (size_t)B * (size_t)nrw * (size_t)(K + 1) * (size_t)D * sizeof(float);
}

extern "C" int atk_dwconv1d_cl_bwd_weight(const void* x, const void* dy, const int* seq_idx,
                                          const void* initial_states, float* dw, float* db, int64_t B,
                                          int64_t D, int64_t L, int K, int pad_left, int64_t L_out,
                                          int64_t x_stride_b, int64_t x_stride_l, int64_t dy_stride_b,
                                          int64_t dy_stride_l, int64_t is_stride_b, int64_t is_stride_l,
                                          int dtype, int seq_mode, void* workspace, size_t ws_bytes,
                                          atk_stream_t stream) {
  using namespace atk;
  const int vec = cl_check(x, B, D, L, K, dtype, x_stride_b, x_stride_l);
  if (vec < 0) return fail(-vec, "dwconv1d_cl_bwd_weight: unsupported shape/layout");
  if (K > 5) return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: K <= 5");
  if (!dy || !dw || L_out <= 0 || pad_left < 0 || L_out > (1 << 30))
    return fail(ATK_EINVAL, "dwconv1d_cl_bwd_weight: bad arguments");
  if (dy_stride_b % vec || dy_stride_l % vec || dy_stride_l < D || !aligned16(dy))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: dy layout");
  if (initial_states && (pad_left != K - 1 || is_stride_b % vec || is_stride_l % vec || !aligned16(initial_states)))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: initial_states layout / form");
  if (seq_mode < 0 || seq_mode > 1 || (seq_mode != 0) != (seq_idx != nullptr) ||
      (seq_mode == 1 && pad_left != K - 1))
    return fail(ATK_EINVAL, "dwconv1d_cl_bwd_weight: seq_idx needs seq_mode 1 and pad K-1");
  if (seq_idx && (uint64_t)B * (uint64_t)L * 4u >= (1ull << 31))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: seq_idx larger than 2 GiB");
  const size_t need = atk_dwconv1d_cl_bwd_weight_workspace_bytes(B, D, L_out, K, dtype);
  if (!workspace || ws_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(ATK_EINVAL, "dwconv1d_cl_bwd_weight: workspace too small or misaligned");
  const size_t es = dtype_size(dtype);
  const int64_t xspan = (L - 1) * x_stride_l + D, gspan = (L_out - 1) * dy_stride_l + D;
  if ((B - 1) * x_stride_b * (int64_t)es + xspan * (int64_t)es >= ((int64_t)1 << 31) ||
      (B - 1) * dy_stride_b * (int64_t)es + gspan * (int64_t)es >= ((int64_t)1 << 31))
    return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: tensors over 2 GiB");
  DwClBwArgs a{};
  a.x = x; a.dy = dy; a.seq = seq_idx; a.init = initial_states; a.ib = is_stride_b; a.il = is_stride_l;
  a.xb = x_stride_b; a.xl = x_stride_l; a.gb = dy_stride_b; a.gl = dy_stride_l;
  a.B = (uint32_t)B; a.D = (uint32_t)D; a.L = (uint32_t)L; a.Lout = (uint32_t)L_out; a.pad = pad_left;
  a.x_bytes = (uint32_t)(((B - 1) * x_stride_b + xspan) * (int64_t)es);
  a.g_bytes = (uint32_t)(((B - 1) * dy_stride_b + gspan) * (int64_t)es);
  a.seq_bytes = (uint32_t)(B * L * 4);
  a.ncv = (uint32_t)(D / vec);
  a.run = clw_run(B, D, L_out, vec);
  a.nrw = (uint32_t)((L_out + a.run - 1) / a.run);
  a.div_ncv = make_fastdiv(a.ncv);
  a.div_nrw = make_fastdiv(a.nrw);
  a.part = static_cast<float*>(workspace);
  a.dw = dw; a.db = db;
  a.P = (uint32_t)(B * a.nrw);
  const uint64_t threads = (uint64_t)B * a.nrw * a.ncv;
  if (threads + CL_NT >= (1ull << 31)) return fail(ATK_UNSUPPORTED, "dwconv1d_cl_bwd_weight: too many threads");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t blocks = (uint32_t)((threads + CL_NT - 1) / CL_NT);
  int rc;
  if (dtype == ATK_F32) rc = launch_clw<float>(a, K, blocks, seq_mode, s);
  else if (dtype == ATK_F16) rc = launch_clw<_Float16>(a, K, blocks, seq_mode, s);
  else rc = launch_clw<__bf16>(a, K, blocks, seq_mode, s);
  if (rc != ATK_OK) return fail(rc, "dwconv1d_cl_bwd_weight: kernel width not served");
  const uint32_t fblocks = (uint32_t)(((K + 1) * D + CLF_COLS - 1) / CLF_COLS);
  hipLaunchKernelGGL(dwconv1d_cl_bwd_finalize_kernel, dim3(fblocks), dim3(CLF_COLS * CLF_SPLIT), 0, s, a, K);
  return check_launch("dwconv1d_cl_bwd_weight");
}

namespace atk {
namespace {

// Loop span of the fused backward: positions u in [min(0, -sh), max(L_out, L - sh)), cut
// into per-thread runs (multiples of CLB_STEP, at least 64) such that the grid is about one
// workgroup per CU.  The wide kernels hold one wave per SIMD, so a grid slightly larger than
// the CUs runs its last workgroups in a second round: 272 workgroups took C2's K = 4 backward
// from 320 to 480 us, and 144 left half the CUs idle (0.50 of HBM); 256 ran every (K, pad) at
// 0.61-0.65.  Each run leaves (K + 1) x VEC fp32 partials per thread for the finalize kernel.
struct ClbSpan {
  int sh, u0, u1;
  uint32_t run, nrun;
};
ClbSpan clb_span(int64_t B, int64_t D, int64_t L, int K, int pad_left, int64_t L_out, int vec) {
  ClbSpan r;
  r.sh = (K - 1) - pad_left;
  r.u0 = std::min(0, -r.sh);
  r.u1 = (int)std::max<int64_t>(L_out, L - r.sh);
  const int64_t len = (int64_t)r.u1 - r.u0, lanes = B * (D / vec);
  const int64_t wg_per_run = (lanes + CL_NT - 1) / CL_NT;
  const int cus = device_cu_count();
  const int64_t runs = std::max<int64_t>(1, (cus > 0 ? cus : 256) / wg_per_run);
  int64_t run = (len + runs - 1) / runs;
  run = std::max<int64_t>(64, (run + CLB_STEP - 1) / CLB_STEP * CLB_STEP);
  r.run = (uint32_t)run;
  r.nrun = (uint32_t)((len + run - 1) / run);
  return r;
}
size_t clb_workspace_bytes(int64_t B, int64_t D, int K, const ClbSpan& sp) {
  return (size_t)B * sp.nrun * (size_t)(K + 1) * (size_t)D * sizeof(float);
}

// The fused backward behind atk_causal_conv1d_cl_bwd (pad K-1, L_out = L, SiLU / seq_idx /
// initial states) and atk_dwconv1d_cl_bwd (any left padding and output length, none of those).
int cl_bwd_fused(const char* what, const void* x, const void* dout, const void* w, const void* bias,
                 const int* seq_idx, const void* initial_states, void* dx, float* dw, float* db, int64_t B,
                 int64_t D, int64_t L, int K, int pad_left, int64_t L_out, int64_t x_stride_b, int64_t x_stride_l,
                 int64_t dout_stride_b, int64_t dout_stride_l, int64_t dx_stride_b, int64_t dx_stride_l,
                 int64_t w_stride_c, int64_t w_stride_k, int64_t is_stride_b, int64_t is_stride_l, int dtype,
                 int w_dtype, int silu, void* workspace, size_t ws_bytes, hipStream_t s) {
  const int vec = cl_check(x, B, D, L, K, dtype, x_stride_b, x_stride_l);
  if (vec < 0) return fail(-vec, "%s: unsupported shape/layout", what);
  if (K < 2 || K > 4) return fail(ATK_UNSUPPORTED, "%s: width 2..4", what);
  if (pad_left < 0 || L_out <= 0 || L_out > (1 << 30) || pad_left > (1 << 20))
    return fail(ATK_EINVAL, "%s: bad padding / output length", what);
  if (!dout || !dx || !w || !dw || !dtype_ok(w_dtype)) return fail(ATK_EINVAL, "%s: null pointer / dtype", what);
  for (const auto& st : {std::pair<int64_t, int64_t>{dout_stride_b, dout_stride_l}, {dx_stride_b, dx_stride_l}})
    if (st.first % vec || st.second % vec || st.second < D) return fail(ATK_UNSUPPORTED, "%s: dout / dx layout", what);
  if (!aligned16(dout) || !aligned16(dx)) return fail(ATK_UNSUPPORTED, "%s: dout / dx alignment", what);
  if (initial_states && (is_stride_b % vec || is_stride_l % vec || !aligned16(initial_states)))
    return fail(ATK_UNSUPPORTED, "%s: initial_states layout", what);
  if (seq_idx && (uint64_t)B * (uint64_t)L * 4u >= (1ull << 31))
    return fail(ATK_UNSUPPORTED, "%s: seq_idx larger than 2 GiB", what);
  const ClbSpan sp = clb_span(B, D, L, K, pad_left, L_out, vec);
  const size_t need = clb_workspace_bytes(B, D, K, sp);
  if (!workspace || ws_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(ATK_EINVAL, "%s: workspace too small or misaligned", what);
  const size_t es = dtype_size(dtype);
  const int64_t xspan = (L - 1) * x_stride_l + D, gspan = (L_out - 1) * dout_stride_l + D;
  if ((B - 1) * x_stride_b * (int64_t)es + xspan * (int64_t)es >= ((int64_t)1 << 31) ||
      (B - 1) * dout_stride_b * (int64_t)es + gspan * (int64_t)es >= ((int64_t)1 << 31))
    return fail(ATK_UNSUPPORTED, "%s: tensors over 2 GiB", what);
  DwClCbArgs a{};
  a.x = x; a.dy = dout; a.dx = dx; a.w = w; a.b = bias; a.wdt = w_dtype; a.wc = w_stride_c; a.wk = w_stride_k;
  cl_param_modes(w, bias, w_dtype, K, w_stride_c, w_stride_k, vec, &a.wmode, &a.bvec);
  a.seq = seq_idx; a.init = initial_states; a.ib = is_stride_b; a.il = is_stride_l;
  a.xb = x_stride_b; a.xl = x_stride_l; a.gb = dout_stride_b; a.gl = dout_stride_l;
  a.ob = dx_stride_b; a.ol = dx_stride_l;
  a.B = (uint32_t)B; a.D = (uint32_t)D; a.L = (uint32_t)L; a.Lout = (uint32_t)L_out;
  a.sh = sp.sh; a.u0 = sp.u0; a.u1 = sp.u1;
  a.x_bytes = (uint32_t)(((B - 1) * x_stride_b + xspan) * (int64_t)es);
  a.g_bytes = (uint32_t)(((B - 1) * dout_stride_b + gspan) * (int64_t)es);
  a.seq_bytes = (uint32_t)(B * L * 4);
  a.ncv = (uint32_t)(D / vec);
  a.span = sp.run;
  a.nspan = sp.nrun;
  a.div_ncv = make_fastdiv(a.ncv);
  a.div_nspan = make_fastdiv(a.nspan);
  a.part = static_cast<float*>(workspace);
  const uint64_t threads = (uint64_t)B * a.nspan * a.ncv;
  if (threads + CL_NT >= (1ull << 31)) return fail(ATK_UNSUPPORTED, "%s: too many threads", what);
  const uint32_t blocks = (uint32_t)((threads + CL_NT - 1) / CL_NT);
  int rc;
  if (dtype == ATK_F32) rc = launch_clb<float>(a, K, blocks, silu, seq_idx != nullptr, s);
  else if (dtype == ATK_F16) rc = launch_clb<_Float16>(a, K, blocks, silu, seq_idx != nullptr, s);
  else rc = launch_clb<__bf16>(a, K, blocks, silu, seq_idx != nullptr, s);
  if (rc != ATK_OK) return fail(rc, "%s: kernel width not served", what);
  DwClBwArgs f{};
  f.D = (uint32_t)D; f.part = a.part; f.dw = dw; f.db = db; f.P = (uint32_t)(B * a.nspan);
  const uint32_t fblocks = (uint32_t)(((K + 1) * D + CLF_COLS - 1) / CLF_COLS);
  hipLaunchKernelGGL(dwconv1d_cl_bwd_finalize_kernel, dim3(fblocks), dim3(CLF_COLS * CLF_SPLIT), 0, s, f, K);
  return check_launch(what);
}

}  // namespace
}  // namespace atk

extern "C" size_t atk_causal_conv1d_cl_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K, int dtype) {
  if (B <= 0 || D <= 0 || L <= 0 || K < 1 || !atk::dtype_ok(dtype)) return 0;
  const int vec = 16 / (int)atk::dtype_size(dtype);
  return atk::clb_workspace_bytes(B, D, K, atk::clb_span(B, D, L, K, K - 1, L, vec));
}

extern "C" int atk_causal_conv1d_cl_bwd(const void* x, const void* dout, const void* w, const void* bias,
                                        const int* seq_idx, const void* initial_states, void* dx, float* dw,
                                        float* db, int64_t B, int64_t D, int64_t L, int K, int64_t x_stride_b,
                                        int64_t x_stride_l, int64_t dout_stride_b, int64_t dout_stride_l,
                                        int64_t dx_stride_b, int64_t dx_stride_l, int64_t w_stride_c,
                                        int64_t w_stride_k, int64_t is_stride_b, int64_t is_stride_l, int dtype,
                                        int w_dtype, int silu, void* workspace, size_t ws_bytes,
                                        atk_stream_t stream) {
  return atk::cl_bwd_fused("causal_conv1d_cl_bwd", x, dout, w, bias, seq_idx, initial_states, dx, dw, db, B, D, L,
                           K, K - 1, L, x_stride_b, x_stride_l, dout_stride_b, dout_stride_l, dx_stride_b,
                           dx_stride_l, w_stride_c, w_stride_k, is_stride_b, is_stride_l, dtype, w_dtype, silu,
                           workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

extern "C" size_t atk_dwconv1d_cl_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K, int pad_left,
                                                      int64_t L_out, int dtype) {
  if (B <= 0 || D <= 0 || L <= 0 || K < 1 || pad_left < 0 || L_out <= 0 || pad_left > (1 << 20) ||
      !atk::dtype_ok(dtype))
    return 0;
  const int vec = 16 / (int)atk::dtype_size(dtype);
  return atk::clb_workspace_bytes(B, D, K, atk::clb_span(B, D, L, K, pad_left, L_out, vec));
}

extern "C" int atk_dwconv1d_cl_bwd(const void* x, const void* dy, const void* w, void* dx, float* dw, float* db,
                                   int64_t B, int64_t D, int64_t L, int K, int pad_left, int64_t L_out,
                                   int64_t x_stride_b, int64_t x_stride_l, int64_t dy_stride_b, int64_t dy_stride_l,
                                   int64_t dx_stride_b, int64_t dx_stride_l, int64_t w_stride_c, int64_t w_stride_k,
                                   int dtype, int w_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream) {
  return atk::cl_bwd_fused("dwconv1d_cl_bwd", x, dy, w, nullptr, nullptr, nullptr, dx, dw, db, B, D, L, K, pad_left,
                           L_out, x_stride_b, x_stride_l, dy_stride_b, dy_stride_l, dx_stride_b, dx_stride_l,
                           w_stride_c, w_stride_k, 0, 0, dtype, w_dtype, 0, workspace, ws_bytes,
                           static_cast<hipStream_t>(stream));
}
