// Depthwise conv1d forward for gfx950 (BCL layout, stride 1, dilation 1).
//
//   y[n,c,t] = bias[c] + sum_{j<K} w[c,j] * x[n,c,t - pad + j],  t in [0, L_out),
//   x == 0 outside [0, L).
//
// Math follows the reference's two kernels for this op
// (amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/conv1d_bhl.hip:25-100 for the
// symmetric case, src/causal-conv1d-amd/csrc/causal_conv1d_fwd.cu:39-130 for the causal
// one, whose output is the first L columns of the pad = K-1 result); unlike the first of
// those it accumulates in fp32 for 16-bit inputs.
//
// Design (HBM-bound streaming, 2 bytes in + 2 bytes out per element for 16-bit):
//   * The output tensor is treated as ONE flat array of N*C*L_out elements and cut into
//     tiles of 256 threads x OPT outputs.  Tile origins are chosen so that every thread's
//     outputs are a naturally aligned 16-byte vector in memory, whatever L_out is: the
//     stock-shaped causal output (L_out = L + K - 1, rows not 16-byte aligned) is stored
//     with full-width coalesced stores just like the symmetric case.
//   * The flat input range a tile depends on (its rows' windows, including the K-1 halo)
//     is staged once into LDS with aligned 16-byte loads; each thread then reads its
//     VEC + K - 1 window from LDS.  Zero padding is a mask on the row position, applied
//     only on the few windows that touch a row edge.
//   * Per-row weights and bias of the (few) rows a tile touches are staged to LDS as
//     fp32 and read as broadcasts.
// A "direct" variant (one output per thread, global loads, no LDS) covers shapes whose
// LDS window would not fit.
#include <cstring>

#include "atk_common.h"

namespace atk {

namespace {

constexpr int DW_NT = 256;        // threads per block
constexpr int DW_MAXR = 16;       // rows whose weights are staged in LDS
constexpr int DW_KMAX = 64;       // largest supported kernel width
constexpr int DW_PADMAX = 64;     // largest supported left padding

struct DwArgs {
  const void* x;
  const void* w;
  const void* b;
  void* y;
  int64_t total_in, total_out;
  uint32_t C, L, Lout;
  int K, pad;
  int x_off, y_off;        // misalignment of the x / y base pointers, in elements
  int silu;
  int w32;                 // w and b are fp32 (else the activations' type)
  FastDiv div_lout, div_c;
  int win_cap;             // LDS window capacity, elements
};

// Weight / bias element i, stored in the activations' type T or (w32) in fp32 -- the causal
// interface takes fp32 weights with 16-bit activations and computes with them unrounded
// (src/causal-conv1d-amd/csrc/causal_conv1d.cpp:139-141).  The dword holding the element is
// loaded either way (it lies inside the array's allocation) and decoded by the flag, so the
// load is issued before the value is needed with no branch around it.
template <typename T>
__device__ __forceinline__ uint32_t dw_pword(const void* p, bool w32, int64_t i) {
  const uintptr_t ad = reinterpret_cast<uintptr_t>(p) + (uintptr_t)i * ((sizeof(T) == 4 || w32) ? 4u : 2u);
  return *reinterpret_cast<const uint32_t*>(ad & ~(uintptr_t)3);
}
template <typename T>
__device__ __forceinline__ float dw_pdecode(uint32_t d, const void* p, bool w32, int64_t i) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(d);
  } else {
    if (w32) return __uint_as_float(d);
    const uintptr_t ad = reinterpret_cast<uintptr_t>(p) + (uintptr_t)i * 2u;
    return to_f32(__builtin_bit_cast(T, (unsigned short)((ad & 2u) ? (d >> 16) : (d & 0xffffu))));
  }
}
template <typename T>
__device__ __forceinline__ float dw_param(const void* p, bool w32, int64_t i) {
  return dw_pdecode<T>(dw_pword<T>(p, w32, i), p, w32, i);
}

template <typename T, int KT, int OPT, bool NTH, bool SILU>
__global__ __launch_bounds__(DW_NT) void dwconv1d_lds_kernel(DwArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int U = OPT / VEC;
  constexpr int TO = DW_NT * OPT;
  const int K = KT > 0 ? KT : a.K;
  const int pad = a.pad;
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ w = static_cast<const T*>(a.w);
  const T* __restrict__ bias = static_cast<const T*>(a.b);
  T* __restrict__ y = static_cast<T*>(a.y);

  extern __shared__ uint4 lds_raw[];
  T* win = reinterpret_cast<T*>(lds_raw);
  float* wl = reinterpret_cast<float*>(win + a.win_cap);  // [DW_MAXR][K + 1]

  const int tid = threadIdx.x;
  const int64_t F0 = (int64_t)blockIdx.x * TO - a.y_off;  // tile origin, 16B aligned in memory
  const int64_t Fs = F0 > 0 ? F0 : 0;
  const int64_t Fe = (F0 + TO) < a.total_out ? (F0 + TO) : a.total_out;
  if (Fs >= Fe) return;

  const uint32_t L = a.L, Lout = a.Lout;
  const int64_t ra = Fs / Lout;
  const uint32_t ta = (uint32_t)(Fs - ra * Lout);
  const int64_t rb = (Fe - 1) / Lout;
  const uint32_t tb = (uint32_t)((Fe - 1) - rb * Lout);

  // ---- stage the flat input window [I_lo, I_hi) -------------------------------------
  int64_t I_lo = ra * (int64_t)L + (((int)ta - pad) > 0 ? ((int)ta - pad) : 0);
  int64_t hi_t = (int64_t)tb - pad + K;
  if (hi_t > (int64_t)L) hi_t = L;
  const int64_t I_hi = rb * (int64_t)L + hi_t;
  // aligned-down start so that global vectors land on 16B boundaries
  int64_t t0 = I_lo + a.x_off;
  t0 = (t0 >= 0 ? t0 / VEC : -((-t0 + VEC - 1) / VEC)) * VEC;
  const int64_t I_base = t0 - a.x_off;
  const int nvec = I_hi > I_lo ? (int)((I_hi - I_base + VEC - 1) / VEC) : 0;
  // Every load of the window is issued before any is used: MAXV unrolled, branch-free
  // buffer loads from a resource based at the window start (offsets stay small for any
  // tensor size); vectors outside the window or not wholly inside the tensor take an
  // out-of-range offset (zero) and the few partial ones are patched element-wise after.
  // (The host guarantees nvec <= MAXV * DW_NT.)
  constexpr int MAXV = U + 2;
  {
    const int64_t rem = a.total_in - I_base;  // elements from the window start to the tensor end
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x + I_base, (uint32_t)((rem < (int64_t)MAXV * DW_NT * VEC ? rem : (int64_t)MAXV * DW_NT * VEC) *
                                         (int64_t)sizeof(T)));
    uint4 stage[MAXV];
#pragma unroll
    for (int m = 0; m < MAXV; ++m) {
      const int v = m * DW_NT + tid;
      const int64_t gi = I_base + (int64_t)v * VEC;
      const bool full = v < nvec && gi >= 0 && gi + VEC <= a.total_in;
      stage[m] = bload16<NTH ? 2 : 0>(rx, full ? (uint32_t)v * 16u : kOOB, 0);
    }
#pragma unroll
    for (int m = 0; m < MAXV; ++m) {
      const int v = m * DW_NT + tid;
      if (v >= nvec) break;
      const int64_t gi = I_base + (int64_t)v * VEC;
      if (!(gi >= 0 && gi + VEC <= a.total_in)) {  // partial vector at a tensor end (rare)
        Vec16<T> val;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int64_t idx = gi + e;
          val.e[e] = (idx >= 0 && idx < a.total_in) ? x[idx] : static_cast<T>(0.0f);
        }
        stage[m] = val.raw;
      }
      reinterpret_cast<uint4*>(win)[v] = stage[m];
    }
  }
  // ---- stage per-row weights + bias (fp32) --------------------------------------------
  const int nrows = (int)(rb - ra + 1);
  const bool rows_in_lds = nrows <= DW_MAXR;
  if (rows_in_lds) {
    const int per = K + 1;
    for (int i = tid; i < nrows * per; i += DW_NT) {
      const int rr = i / per, j = i - rr * per;
      const uint32_t c = fdiv((uint32_t)(ra + rr), a.div_c);
      const uint32_t ch = (uint32_t)(ra + rr) - c * a.C;
      float v;
      if (j < K) v = dw_param<T>(w, a.w32, (int64_t)ch * K + j);
      else v = bias ? dw_param<T>(bias, a.w32, ch) : 0.f;
      wl[i] = v;
    }
  }
  __syncthreads();

  const int per = K + 1;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int vi = u * DW_NT + tid;
    const int64_t f = F0 + (int64_t)vi * VEC;
    if (f + VEC <= Fs || f >= Fe) continue;
    const bool whole = (f >= Fs) && (f + VEC <= Fe);
    bool fast = whole;
    uint32_t r_rel = 0, t = 0;
    if (whole) {
      const uint32_t q = ta + (uint32_t)(f - Fs);
      r_rel = fdiv(q, a.div_lout);
      t = q - r_rel * Lout;
      fast = (t + VEC <= Lout);
    }
    if (whole && !fast && rows_in_lds && KT > 0) {
      // the vector crosses one row boundary (rows are not 16-byte aligned in memory when
      // Lout % VEC != 0, e.g. the stock-shaped causal output): elements e < eb finish row
      // r, the rest start row r+1; still one full 16-byte store
      const uint32_t eb = Lout - t;
      const int64_t r = ra + r_rel;
      Vec16<T> o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const bool second = (uint32_t)e >= eb;
        const float* wr = wl + (r_rel + (second ? 1u : 0u)) * per;
        const int te = second ? e - (int)eb : (int)t + e;
        const int s = te - pad;
        const int pb = (int)((r + (second ? 1 : 0)) * (int64_t)L + s - I_base);
        float acc = wr[K];
#pragma unroll
        for (int j = 0; j < (KT > 0 ? KT : 1); ++j) {
          const int pos = s + j;
          const float xv = ((unsigned)pos < L) ? to_f32(win[pb + j]) : 0.f;
          acc = fmaf(wr[j], xv, acc);
        }
        if constexpr (SILU) acc = silu_f32(acc);
        o.e[e] = from_f32<T>(acc);
      }
      st16<NTH>(y + f, o.raw);
    } else if (fast) {
      const int64_t r = ra + r_rel;
      float wk[KT > 0 ? KT : 1];
      float bv;
      const float* wrow = nullptr;
      int64_t wg = 0;  // element index of the row's first weight
      uint32_t ch = 0;
      if (rows_in_lds) {
        wrow = wl + r_rel * per;
        bv = wrow[K];
      } else {
        const uint32_t c = fdiv((uint32_t)r, a.div_c);
        ch = (uint32_t)r - c * a.C;
        wg = (int64_t)ch * K;
        bv = bias ? dw_param<T>(bias, a.w32, ch) : 0.f;
      }
      if (KT > 0) {
        if (rows_in_lds) {
#pragma unroll
          for (int j = 0; j < (KT > 0 ? KT : 1); ++j) wk[j] = wrow[j];
        } else {
#pragma unroll
          for (int j = 0; j < (KT > 0 ? KT : 1); ++j) wk[j] = dw_param<T>(w, a.w32, wg + j);
        }
      }
      const int s = (int)t - pad;  // input position of window element 0
      const int p0 = (int)(r * (int64_t)L + s - I_base);
      const bool interior = (s >= 0) && (s + VEC + K - 1 <= (int)L);
      float acc[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = bv;
      if (KT > 0) {
        constexpr int WN = VEC + (KT > 0 ? KT : 1) - 1;
        float wv[WN];
        if (interior) {
#pragma unroll
          for (int q = 0; q < WN; ++q) wv[q] = to_f32(win[p0 + q]);
        } else {
#pragma unroll
          for (int q = 0; q < WN; ++q) {
            const int pos = s + q;
            wv[q] = ((unsigned)pos < L) ? to_f32(win[p0 + q]) : 0.f;
          }
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e)
#pragma unroll
          for (int j = 0; j < (KT > 0 ? KT : 1); ++j) acc[e] = fmaf(wk[j], wv[e + j], acc[e]);
      } else {
        for (int j = 0; j < K; ++j) {
          float wj;
          if (rows_in_lds) wj = wrow[j];
          else wj = dw_param<T>(w, a.w32, wg + j);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const int pos = s + e + j;
            const float xv = (interior || (unsigned)pos < L) ? to_f32(win[p0 + e + j]) : 0.f;
            acc[e] = fmaf(wj, xv, acc[e]);
          }
        }
      }
      if constexpr (SILU) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = silu_f32(acc[e]);
      }
      st16<NTH>(y + f, pack16<T>(acc));
    } else {
      // row boundary inside the vector, or a partial vector at the tensor ends
#pragma unroll 1
      for (int e = 0; e < VEC; ++e) {
        const int64_t fe = f + e;
        if (fe < Fs || fe >= Fe) continue;
        const uint32_t q = ta + (uint32_t)(fe - Fs);
        const uint32_t rr = fdiv(q, a.div_lout);
        const uint32_t te = q - rr * Lout;
        const int64_t r = ra + rr;
        float acc, wj;
        const uint32_t c = fdiv((uint32_t)r, a.div_c);
        const uint32_t ch = (uint32_t)r - c * a.C;
        if (rows_in_lds) acc = wl[rr * per + K];
        else acc = bias ? dw_param<T>(bias, a.w32, ch) : 0.f;
        const int s = (int)te - pad;
        const int p0 = (int)(r * (int64_t)L + s - I_base);
        for (int j = 0; j < K; ++j) {
          const int pos = s + j;
          if ((unsigned)pos >= L) continue;
          wj = rows_in_lds ? wl[rr * per + j] : dw_param<T>(w, a.w32, (int64_t)ch * K + j);
          acc = fmaf(wj, to_f32(win[p0 + j]), acc);
        }
        if constexpr (SILU) acc = silu_f32(acc);
        y[fe] = from_f32<T>(acc);
      }
    }
  }
}

// One output per thread, straight from global memory.  Generic fallback.
template <typename T, bool SILU>
__global__ __launch_bounds__(DW_NT) void dwconv1d_direct_kernel(DwArgs a) {
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ w = static_cast<const T*>(a.w);
  const T* __restrict__ bias = static_cast<const T*>(a.b);
  T* __restrict__ y = static_cast<T*>(a.y);
  const int64_t f = (int64_t)blockIdx.x * DW_NT + threadIdx.x;
  if (f >= a.total_out) return;
  const int64_t r = f / a.Lout;
  const int64_t t = f - r * a.Lout;
  const int64_t ch = r % a.C;
  float acc = bias ? dw_param<T>(bias, a.w32, ch) : 0.f;
  const int64_t s = t - a.pad;
  for (int j = 0; j < a.K; ++j) {
    const int64_t pos = s + j;
    if (pos < 0 || pos >= (int64_t)a.L) continue;
    acc = fmaf(dw_param<T>(w, a.w32, ch * a.K + j), to_f32(x[r * (int64_t)a.L + pos]), acc);
  }
  if constexpr (SILU) acc = silu_f32(acc);
  y[f] = from_f32<T>(acc);
}

// Register-only kernel: one 16-byte output vector per thread, no LDS, no barrier -- the
// access pattern of a one-vector-per-thread streaming copy, which is what HBM serves best.
// The vector's input window (VEC + K - 1 elements, starting at an arbitrary element) is
// cut out of the NBLK aligned 16-byte blocks that cover it with a per-lane funnel shift;
// neighbouring lanes fetch overlapping blocks, which the L1 serves.  Positions outside
// the row read as zero (padding), which also masks anything fetched past the tensor ends
// (those bytes stay inside the 16-byte block that holds the first / last element).  A
// vector that crosses one row boundary (rows of a stock-shaped causal output are not
// 16-byte aligned) uses two such windows; only partial vectors at the tensor ends are
// computed element-wise.  Requires input and output below 2^31 elements (host check).
template <typename T, int KT>
struct DwWindow {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int WN = VEC + KT - 1;                     // window elements
  static constexpr int NBLK = (VEC - 1 + WN + VEC - 1) / VEC;  // blocks covering it at any start
  // fetch: the NBLK blocks holding elements g .. g + WN - 1 (g counted from the aligned
  // base of rx); active == false issues the loads with out-of-range offsets (zeros)
  __device__ __forceinline__ static void fetch(__amdgpu_buffer_rsrc_t rx, int g, bool active, uint32_t* D,
                                               int& m) {
    const int bA = g >= 0 ? g / VEC : -((-g + VEC - 1) / VEC);
    m = g - bA * VEC;  // 0 .. VEC-1
#pragma unroll
    for (int k = 0; k < NBLK; ++k) {
      const int b = bA + k;
      const uint4 q = bload16(rx, (active && b >= 0) ? (uint32_t)b * 16u : kOOB, 0);
      D[4 * k] = q.x; D[4 * k + 1] = q.y; D[4 * k + 2] = q.z; D[4 * k + 3] = q.w;
    }
  }
  // extract: xv[i] = element g + i, zero where the row position p0 + i is outside [0, L)
  __device__ __forceinline__ static void extract(const uint32_t* D, int m, int p0, uint32_t L, float* xv) {
    if constexpr (sizeof(T) == 2) {
      // dword shift by m/2 (select), then half-dword shift by m%2 (alignbyte)
      constexpr int NS = (WN + 1) / 2;
      const int qd = m >> 1;
      uint32_t Tq[NS + 1];
#pragma unroll
      for (int j = 0; j <= NS; ++j) {
        const uint32_t d0 = D[j], d1 = D[j + 1], d2 = D[j + 2], d3 = D[j + 3];
        Tq[j] = qd == 0 ? d0 : qd == 1 ? d1 : qd == 2 ? d2 : d3;
      }
      const bool odd = m & 1;
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const uint32_t sd = odd ? __builtin_amdgcn_alignbyte(Tq[j + 1], Tq[j], 2) : Tq[j];
        if (2 * j < WN) xv[2 * j] = to_f32(__builtin_bit_cast(T, (unsigned short)(sd & 0xffffu)));
        if (2 * j + 1 < WN) xv[2 * j + 1] = to_f32(__builtin_bit_cast(T, (unsigned short)(sd >> 16)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < WN; ++i) {
        const uint32_t d0 = D[i], d1 = D[i + 1], d2 = D[i + 2], d3 = D[i + 3];
        xv[i] = __uint_as_float(m == 0 ? d0 : m == 1 ? d1 : m == 2 ? d2 : d3);
      }
    }
    if (p0 < 0 || p0 + WN > (int)L) {
#pragma unroll
      for (int i = 0; i < WN; ++i)
        if ((unsigned)(p0 + i) >= L) xv[i] = 0.f;
    }
  }
};

// The output vector at flat element f (f counted from y, may be negative at the start).
template <typename T, int KT, bool NTH, bool SILU>
__device__ __forceinline__ void reg_vector(const DwArgs& a, int64_t f) {
  using Win = DwWindow<T, KT>;
  constexpr int VEC = Win::VEC, WN = Win::WN;
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ w = static_cast<const T*>(a.w);
  const T* __restrict__ bias = static_cast<const T*>(a.b);
  T* __restrict__ y = static_cast<T*>(a.y);
  const uint32_t L = a.L, Lout = a.Lout;
  const int pad = a.pad;

  if (f >= a.total_out || f + VEC <= 0) return;
  bool whole = f >= 0 && f + VEC <= a.total_out;
  uint32_t r = 0, t = 0, eb = VEC;
  if (whole) {
    r = fdiv((uint32_t)f, a.div_lout);
    t = (uint32_t)f - r * Lout;
    // elements e < eb are row r (positions t + e); the rest, if any, start row r + 1 --
    // which must hold them all (Lout < VEC can put a vector across several rows)
    eb = t + VEC <= Lout ? (uint32_t)VEC : Lout - t;
    whole = (uint32_t)VEC - eb <= Lout;
  }
  if (whole) {
    const __amdgpu_buffer_rsrc_t rx =
        make_rsrc(x - a.x_off, (uint32_t)(((int64_t)a.total_in + a.x_off + VEC - 1) / VEC * 16));
    // the window, weights and bias loads are all issued before any is used (the bias read
    // is branch-free: a load under a branch would be waited for inside it)
    uint32_t DA[4 * Win::NBLK];
    int mA;
    Win::fetch(rx, (int)(r * L + t) - pad + a.x_off, true, DA, mA);
    const uint32_t c = r - fdiv(r, a.div_c) * a.C;
    const void* bsrc = bias ? static_cast<const void*>(bias) : a.w;  // w has >= C elements
    const float bscale = bias ? 1.f : 0.f;
    const bool w32 = a.w32;
    uint32_t wr[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) wr[j] = dw_pword<T>(w, w32, (int64_t)c * KT + j);
    const uint32_t br = dw_pword<T>(bsrc, w32, c);
    float xv[WN], xw[WN], wk[KT], wk2[KT];
    Win::extract(DA, mA, (int)t - pad, L, xv);
#pragma unroll
    for (int j = 0; j < KT; ++j) wk[j] = dw_pdecode<T>(wr[j], w, w32, (int64_t)c * KT + j);
    const float bv = dw_pdecode<T>(br, bsrc, w32, c) * bscale;
    float bv2 = bv;
    // a vector crossing into row r + 1 (once per row for unaligned rows): its second window
    // and the next channel's weights are fetched here, off the common path
    const bool split = eb < (uint32_t)VEC;
    if (split) {
      uint32_t DB[4 * Win::NBLK];
      int mB;
      Win::fetch(rx, (int)((r + 1) * L) - (int)eb - pad + a.x_off, true, DB, mB);
      const uint32_t c2 = c + 1 == a.C ? 0u : c + 1;
#pragma unroll
      for (int j = 0; j < KT; ++j) wk2[j] = dw_param<T>(w, w32, (int64_t)c2 * KT + j);
      bv2 = dw_param<T>(bsrc, w32, c2) * bscale;
      Win::extract(DB, mB, -(int)eb - pad, L, xw);
    }
    Vec16<T> o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float acc;
      if (!split || (uint32_t)e < eb) {
        acc = bv;
#pragma unroll
        for (int j = 0; j < KT; ++j) acc = fmaf(wk[j], xv[e + j], acc);
      } else {
        acc = bv2;
#pragma unroll
        for (int j = 0; j < KT; ++j) acc = fmaf(wk2[j], xw[e + j], acc);
      }
      if constexpr (SILU) acc = silu_f32(acc);
      o.e[e] = from_f32<T>(acc);
    }
    st16<NTH>(y + f, o.raw);
  } else {
    // partial vector at a tensor end, or rows shorter than a vector
#pragma unroll 1
    for (int e = 0; e < VEC; ++e) {
      const int64_t fe = f + e;
      if (fe < 0 || fe >= a.total_out) continue;
      const uint32_t re = fdiv((uint32_t)fe, a.div_lout);
      const uint32_t te = (uint32_t)fe - re * Lout;
      const uint32_t ce = re - fdiv(re, a.div_c) * a.C;
      float acc = bias ? dw_param<T>(bias, a.w32, ce) : 0.f;
      const int se = (int)te - pad;
      for (int j = 0; j < KT; ++j) {
        const int pos = se + j;
        if ((unsigned)pos < L) acc = fmaf(dw_param<T>(w, a.w32, (int64_t)ce * KT + j), to_f32(x[(int64_t)re * L + pos]), acc);
      }
      if constexpr (SILU) acc = silu_f32(acc);
      y[fe] = from_f32<T>(acc);
    }
  }
}

template <typename T, int KT, bool NTH, bool SILU>
__global__ __launch_bounds__(DW_NT) void dwconv1d_reg_kernel(DwArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  reg_vector<T, KT, NTH, SILU>(a, ((int64_t)blockIdx.x * DW_NT + threadIdx.x) * VEC - a.y_off);
}

// Weights w[c, 0..KT) and bias[c] of one wave-uniform channel through scalar loads of the
// dwords that hold them: no vector-memory instruction, and every read stays inside a dword
// that holds an element of the array (w and b are element-aligned).
template <typename T, int KT>
__device__ __forceinline__ void uniform_params(const void* wp, const void* bp, uint32_t c, float* wk,
                                               float& bv, bool w32) {
  typedef const __attribute__((address_space(4))) uint32_t* cptr;
  auto fp32_params = [&]() {
    const cptr q = (cptr)((uintptr_t)wp + (uintptr_t)c * KT * 4u);
#pragma unroll
    for (int j = 0; j < KT; ++j) wk[j] = __uint_as_float(q[j]);
    bv = bp ? __uint_as_float(((cptr)((uintptr_t)bp + (uintptr_t)c * 4u))[0]) : 0.f;
  };
  if constexpr (sizeof(T) == 4) {
    fp32_params();
  } else if (w32) {
    fp32_params();
  } else {
    auto half = [](uint32_t d, uint32_t byte) {
      return to_f32(__builtin_bit_cast(T, (unsigned short)((byte & 2u) ? (d >> 16) : (d & 0xffffu))));
    };
    const uintptr_t a0 = (uintptr_t)wp + (uintptr_t)c * KT * 2u;
    const uintptr_t al = a0 & ~(uintptr_t)3;
    const uint32_t sh = (uint32_t)(a0 - al);  // 0 or 2
    constexpr int NDM = (2 + 2 * KT + 3) / 4;
    const int nd = (int)((sh + 2u * KT + 3u) / 4u);
    const cptr q = (cptr)al;
    uint32_t d[NDM];
#pragma unroll
    for (int i = 0; i < NDM; ++i) d[i] = q[i < nd ? i : nd - 1];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const uint32_t o = sh + 2u * j;
      wk[j] = half(d[o >> 2], o);
    }
    if (bp) {
      const uintptr_t ab = (uintptr_t)bp + (uintptr_t)c * 2u;
      bv = half(((cptr)(ab & ~(uintptr_t)3))[0], (uint32_t)ab);
    } else {
      bv = 0.f;
    }
  }
}

// Element e of a window held as packed dwords D (e is a compile-time index after unrolling).
template <typename T>
__device__ __forceinline__ float win_elem(const uint32_t* D, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(D[e]);
  } else {
    const uint32_t d = D[e >> 1];
    return to_f32(__builtin_bit_cast(T, (unsigned short)((e & 1) ? (d >> 16) : (d & 0xffffu))));
  }
}

// c + w.lo * x.lo + w.hi * x.hi for two packed 16-bit elements (v_dot2c_f32_{bf16,f16}): the
// products of 16-bit values are exact in fp32.
template <typename T>
__device__ __forceinline__ float dot2_acc(uint32_t w, uint32_t x, float c) {
  if constexpr (sizeof(T) == 2 && __is_same(T, __bf16)) {
    typedef __bf16 p2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(p2, w), __builtin_bit_cast(p2, x), c, false);
  } else {
    typedef _Float16 p2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(p2, w), __builtin_bit_cast(p2, x), c, false);
  }
}

// Tail of the cross-lane kernel for a wave-uniform window offset M (the window's first
// element is element M of block bA + lane).  Fixed per M: which neighbour blocks are
// exchanged and which register holds each window element, so the window costs only its
// conversions -- no per-lane selects or shifts.  The padding mask runs only in waves with
// a lane at a row edge.
// DOT (16-bit x with weights of its own dtype): the window stays packed, two taps per
// v_dot2c with the weight pair (w[j], w[j+1]) -- an element pair that starts at an odd
// element is cut from two dwords with one v_alignbit -- and an odd last tap is an FMA on the
// converted element: about half the VALU work of converting every element and four FMAs
// per output.
template <typename T, int KT, bool NTH, bool SILU, int M, bool DOT>
__device__ __forceinline__ void xlane_tail(const uint4& E, const uint4& X, int lane, bool edge, int p0,
                                           uint32_t L, const float* wk, const uint32_t* wp, float bv, T* dst) {
  using Win = DwWindow<T, KT>;
  constexpr int VEC = Win::VEC, WN = Win::WN;
  // lanes 0 and 1 stand in with the blocks past the wave, which lanes 62 and 63 need
  const uint4 Z1 = lane == 0 ? X : E;
  const int src1 = ((lane + 1) & 63) * 4;
  uint32_t D[12];
  D[0] = E.x; D[1] = E.y; D[2] = E.z; D[3] = E.w;
  D[4] = (uint32_t)__builtin_amdgcn_ds_bpermute(src1, (int)Z1.x);
  D[5] = (uint32_t)__builtin_amdgcn_ds_bpermute(src1, (int)Z1.y);
  D[6] = (uint32_t)__builtin_amdgcn_ds_bpermute(src1, (int)Z1.z);
  D[7] = (uint32_t)__builtin_amdgcn_ds_bpermute(src1, (int)Z1.w);
  if constexpr (M + WN > 2 * VEC) {
    const uint4 Z2 = lane < 2 ? X : E;
    const int src2 = ((lane + 2) & 63) * 4;
    D[8] = (uint32_t)__builtin_amdgcn_ds_bpermute(src2, (int)Z2.x);
    D[9] = (uint32_t)__builtin_amdgcn_ds_bpermute(src2, (int)Z2.y);
    D[10] = (uint32_t)__builtin_amdgcn_ds_bpermute(src2, (int)Z2.z);
    D[11] = (uint32_t)__builtin_amdgcn_ds_bpermute(src2, (int)Z2.w);
  } else {
    D[8] = D[9] = D[10] = D[11] = 0u;
  }
  float acc[VEC];
  if constexpr (DOT && sizeof(T) == 2) {
    if (edge) {  // zero the halves that hold elements past a row edge
#pragma unroll
      for (int i = 0; i < WN; ++i)
        if ((unsigned)(p0 + i) >= L) D[(M + i) >> 1] &= ((M + i) & 1) ? 0x0000ffffu : 0xffff0000u;
    }
    // elements s, s + 1 as one dword (s is a compile-time index here)
    auto pair = [&](int s) -> uint32_t {
      return (s & 1) ? __builtin_amdgcn_alignbit(D[(s >> 1) + 1], D[s >> 1], 16) : D[s >> 1];
    };
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float c = bv;
#pragma unroll
      for (int j = 0; j + 1 < KT; j += 2) c = dot2_acc<T>(wp[j >> 1], pair(M + e + j), c);
      if constexpr (KT & 1) c = fmaf(wk[KT - 1], win_elem<T>(D, M + e + KT - 1), c);
      if constexpr (SILU) c = silu_f32(c);
      acc[e] = c;
    }
  } else {
    float xv[WN];
#pragma unroll
    for (int i = 0; i < WN; ++i) xv[i] = win_elem<T>(D, M + i);
    if (edge) {
#pragma unroll
      for (int i = 0; i < WN; ++i)
        if ((unsigned)(p0 + i) >= L) xv[i] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      acc[e] = bv;
#pragma unroll
      for (int j = 0; j < KT; ++j) acc[e] = fmaf(wk[j], xv[e + j], acc[e]);
      if constexpr (SILU) acc[e] = silu_f32(acc[e]);
    }
  }
  // SiLU is a template parameter: as a runtime flag the compiler evaluates it for every
  // output (two quarter-rate transcendentals each) and selects
  uint4 o = pack16<T>(acc);
  // whole vector in registers first: otherwise the plain store may be split into pieces
  asm volatile("" : "+v"(o.x), "+v"(o.y), "+v"(o.z), "+v"(o.w));
  st16<NTH>(dst, o);
}

// Uniform dispatch of the window offset m to its xlane_tail (a scalar compare chain).
template <typename T, int KT, bool NTH, bool SILU, bool DOT, int M = 0>
__device__ __forceinline__ void xlane_dispatch(int m, const uint4& E, const uint4& X, int lane, bool edge,
                                               int p0, uint32_t L, const float* wk, const uint32_t* wp, float bv,
                                               T* dst) {
  if constexpr (M < (int)(16 / sizeof(T))) {
    if (m == M) xlane_tail<T, KT, NTH, SILU, M, DOT>(E, X, lane, edge, p0, L, wk, wp, bv, dst);
    else xlane_dispatch<T, KT, NTH, SILU, DOT, M + 1>(m, E, X, lane, edge, p0, L, wk, wp, bv, dst);
  }
}

// Cross-lane register kernel: the one-vector-per-thread kernel above with the window
// shared across the wave.  In a wave whose 64 vectors all lie in one row (all but the few
// waves that meet a row boundary or a tensor end), lane t's window starts VEC elements
// after lane t-1's, so it is cut from blocks bA+t, bA+t+1, bA+t+2 of the input: each lane
// loads only block bA+t, lanes 0 and 1 also load the two blocks past the wave, and the
// neighbours' blocks arrive through ds_bpermute.  The channel is uniform there, so weights
// and bias come through scalar loads.  Vector-memory instructions per output vector: about
// 1 load and 1 store, the access pattern of a streaming copy.  Other waves take the
// per-lane path of the register kernel.
template <typename T, int KT, bool NTH, bool SILU, int NV>
__global__ __launch_bounds__(DW_NT) void dwconv1d_xlane_kernel(DwArgs a) {
  using Win = DwWindow<T, KT>;
  constexpr int VEC = Win::VEC, WN = Win::WN;
  constexpr int SPAN = 64 * VEC;  // outputs of one 64-vector part of a wave
  static_assert(Win::NBLK <= 3, "window spans at most three blocks");
  const int lane = threadIdx.x & 63;
  // the wave's NV * 64 consecutive output vectors: part h holds vectors 64 h .. 64 h + 63
  const int64_t vw = ((int64_t)blockIdx.x * (DW_NT / 64) + (threadIdx.x >> 6)) * 64 * NV;
  const int64_t f = (vw + lane) * VEC - a.y_off;  // this lane's output in part 0
  uint32_t r = 0, t = 0;
  bool inrow = f >= 0 && f + (int64_t)SPAN * (NV - 1) + VEC <= a.total_out;
  if (inrow) {
    r = fdiv((uint32_t)f, a.div_lout);
    t = (uint32_t)f - r * a.Lout;
    inrow = t + SPAN * (NV - 1) + VEC <= a.Lout;
  }
  const uint32_t r0 = __builtin_amdgcn_readfirstlane(r);
  if (__builtin_amdgcn_ballot_w64(inrow && r == r0) != ~0ull) {
#pragma unroll
    for (int h = 0; h < NV; ++h) reg_vector<T, KT, NTH, SILU>(a, f + (int64_t)SPAN * h);
    return;
  }
  // every lane: row r0, position t = t0 + VEC * lane (+ SPAN * h in part h)
  const uint32_t t0 = __builtin_amdgcn_readfirstlane(t);
  const int g0 = (int)(r0 * a.L + t0) - a.pad + a.x_off;  // lane 0's window start, from x's aligned base
  const int bA = g0 >= 0 ? g0 / VEC : -((-g0 + VEC - 1) / VEC);
  const int m = g0 - bA * VEC;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      static_cast<const T*>(a.x) - a.x_off, (uint32_t)(((int64_t)a.total_in + a.x_off + VEC - 1) / VEC * 16));
  // part h's blocks; the two blocks past part h are part h + 1's first two (lanes 0 and 1
  // hold them), and past the last part two more blocks are loaded
  uint4 E[NV];
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int be = bA + 64 * h + lane;
    E[h] = bload16<NTH ? 2 : 0>(rx, be >= 0 ? (uint32_t)be * 16u : kOOB, 0);
  }
  const int bx = bA + 64 * NV + lane;
  const uint4 X = bload16(rx, lane < 2 && bx >= 0 ? (uint32_t)bx * 16u : kOOB, 0);
  float wk[KT], bv;
  uniform_params<T, KT>(a.w, a.b, r0 - fdiv(r0, a.div_c) * a.C, wk, bv, a.w32);
  T* dst = static_cast<T*>(a.y) + f;
  auto parts = [&](auto dot, const uint32_t* wp) {
#pragma unroll
    for (int h = 0; h < NV; ++h) {
      const int th = (int)t0 + SPAN * h;
      // lanes whose window reaches past a row edge need the zero-padding mask (uniform test)
      const bool edge = th - a.pad < 0 || th + VEC * 63 - a.pad + WN > (int)a.L;
      xlane_dispatch<T, KT, NTH, SILU, decltype(dot)::value>(m, E[h], h + 1 < NV ? E[h + 1 < NV ? h + 1 : h] : X, lane,
                                                             edge, (int)t - a.pad + SPAN * h, a.L, wk, wp, bv,
                                                             dst + SPAN * h);
    }
  };
  if constexpr (sizeof(T) == 2 && KT >= 2) {
    if (!a.w32) {
      // weight pairs (w[j], w[j+1]) packed back into 16-bit halves (exact: they were 16-bit)
      constexpr int NP = KT / 2;
      uint32_t wp[NP];
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef T t2 __attribute__((ext_vector_type(2)));
        const f2 pr = {wk[2 * j], wk[2 * j + 1]};
        wp[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pr, t2));
      }
      parts(std::true_type(), wp);
      return;
    }
  }
  parts(std::false_type(), nullptr);
}

struct DwVariant {
  const char* name;
  int opt;  // outputs per thread; 0 = direct kernel, -1 = register kernel (one vector),
            // -2 / -3 = cross-lane register kernel (64 / 128 vectors per wave)
  bool nt;  // nontemporal loads/stores
};

const DwVariant kDwVariants[] = {
    {"lds_opt16", 16, false},
    {"lds_opt8", 8, false},
    {"lds_opt32", 32, false},
    {"direct", 0, false},
    {"lds_opt16_nt", 16, true},
    {"lds_opt32_nt", 32, true},
    {"lds_opt64_nt", 64, true},
    {"reg_nt", -1, true},
    {"reg", -1, false},
    {"xlane_nt", -2, true},
    {"xlane", -2, false},
    {"xlane2_nt", -3, true},
};
constexpr int kNumDw = sizeof(kDwVariants) / sizeof(kDwVariants[0]);

template <typename T, int KT, int OPT, bool NTH>
int launch_lds_t(const DwArgs& a, size_t shmem, hipStream_t s) {
  constexpr int TO = DW_NT * OPT;
  const int64_t nblk = (a.total_out + a.y_off + TO - 1) / TO;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "dwconv1d: grid too large");
  if (a.silu)
    hipLaunchKernelGGL((dwconv1d_lds_kernel<T, KT, OPT, NTH, true>), dim3((unsigned)nblk), dim3(DW_NT), shmem, s, a);
  else
    hipLaunchKernelGGL((dwconv1d_lds_kernel<T, KT, OPT, NTH, false>), dim3((unsigned)nblk), dim3(DW_NT), shmem, s, a);
  return check_launch("dwconv1d_lds_kernel");
}

template <typename T, int OPT, bool NTH>
int launch_lds_k(const DwArgs& a, size_t shmem, hipStream_t s) {
  switch (a.K) {
    case 2: return launch_lds_t<T, 2, OPT, NTH>(a, shmem, s);
    case 3: return launch_lds_t<T, 3, OPT, NTH>(a, shmem, s);
    case 4: return launch_lds_t<T, 4, OPT, NTH>(a, shmem, s);
    case 5: return launch_lds_t<T, 5, OPT, NTH>(a, shmem, s);
    default: return launch_lds_t<T, 0, OPT, NTH>(a, shmem, s);
  }
}

template <typename T, int KT, bool NTH, int XL>
void launch_reg_k(dim3 grid, dim3 block, hipStream_t s, const DwArgs& a) {
  if constexpr (XL > 0) {
    if (a.silu) hipLaunchKernelGGL((dwconv1d_xlane_kernel<T, KT, NTH, true, XL>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dwconv1d_xlane_kernel<T, KT, NTH, false, XL>), grid, block, 0, s, a);
  } else {
    if (a.silu) hipLaunchKernelGGL((dwconv1d_reg_kernel<T, KT, NTH, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dwconv1d_reg_kernel<T, KT, NTH, false>), grid, block, 0, s, a);
  }
}

// XL: 0 = the one-vector register kernel, 1 / 2 = the cross-lane kernel with 1 / 2 vectors per lane
template <typename T, bool NTH, int XL>
int launch_reg(const DwArgs& a, hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int64_t PER_WG = (int64_t)DW_NT * VEC * (XL > 1 ? XL : 1);
  if (a.total_out + a.y_off >= (1ll << 31) - PER_WG || a.total_in + a.x_off >= (1ll << 31) / (int64_t)sizeof(T) - VEC)
    return fail(ATK_UNSUPPORTED, "dwconv1d: tensor too large for the register kernel");
  const int64_t nblk = (a.total_out + a.y_off + PER_WG - 1) / PER_WG;
  const dim3 grid((unsigned)nblk), block(DW_NT);
  switch (a.K) {
    case 2: launch_reg_k<T, 2, NTH, XL>(grid, block, s, a); break;
    case 3: launch_reg_k<T, 3, NTH, XL>(grid, block, s, a); break;
    case 4: launch_reg_k<T, 4, NTH, XL>(grid, block, s, a); break;
    case 5: launch_reg_k<T, 5, NTH, XL>(grid, block, s, a); break;
    default: return fail(ATK_UNSUPPORTED, "dwconv1d: register kernels serve K in [2, 5]");
  }
  return check_launch(XL > 0 ? "dwconv1d_xlane_kernel" : "dwconv1d_reg_kernel");
}

template <typename T>
int launch_dw(DwArgs a, int variant, hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  const int opt = kDwVariants[variant].opt;
  if (opt == -1) return kDwVariants[variant].nt ? launch_reg<T, true, 0>(a, s) : launch_reg<T, false, 0>(a, s);
  if (opt == -2) return kDwVariants[variant].nt ? launch_reg<T, true, 1>(a, s) : launch_reg<T, false, 1>(a, s);
  if (opt == -3) return kDwVariants[variant].nt ? launch_reg<T, true, 2>(a, s) : launch_reg<T, false, 2>(a, s);
  if (opt == 0 || opt < VEC) {
    const int64_t nblk = (a.total_out + DW_NT - 1) / DW_NT;
    if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "dwconv1d: grid too large");
    if (a.silu) hipLaunchKernelGGL((dwconv1d_direct_kernel<T, true>), dim3((unsigned)nblk), dim3(DW_NT), 0, s, a);
    else hipLaunchKernelGGL((dwconv1d_direct_kernel<T, false>), dim3((unsigned)nblk), dim3(DW_NT), 0, s, a);
    return check_launch("dwconv1d_direct_kernel");
  }
  // LDS window bound for one tile (see the kernel): TO outputs span at most
  // floor((TO-1)/Lout)+1 row boundaries, each adding (L - Lout) inputs when L > Lout.
  const int64_t TO = (int64_t)DW_NT * opt;
  const int64_t extra_rows = (TO - 1) / a.Lout + 1;
  int64_t need = TO + a.K + a.pad + 2 * VEC;
  if ((int64_t)a.L > (int64_t)a.Lout) need += extra_rows * ((int64_t)a.L - a.Lout);
  need = (need + VEC - 1) / VEC * VEC;
  const size_t shmem = (size_t)need * sizeof(T) + (size_t)DW_MAXR * (a.K + 1) * sizeof(float);
  if (shmem > 64 * 1024) return fail(ATK_UNSUPPORTED, "dwconv1d: LDS window too large for variant");
  if (need / VEC > (int64_t)(opt / VEC + 2) * DW_NT)  // the kernel stages at most MAXV vectors per thread
    return fail(ATK_UNSUPPORTED, "dwconv1d: LDS window needs more loads per thread than the variant issues");
  a.win_cap = (int)need;
  if (kDwVariants[variant].nt) {
    switch (opt) {
      case 16: return launch_lds_k<T, 16, true>(a, shmem, s);
      case 32: return launch_lds_k<T, 32, true>(a, shmem, s);
      case 64: return launch_lds_k<T, 64, true>(a, shmem, s);
      default: return fail(ATK_UNSUPPORTED, "dwconv1d: bad variant");
    }
  }
  switch (opt) {
    case 8: return launch_lds_k<T, 8, false>(a, shmem, s);
    case 16: return launch_lds_k<T, 16, false>(a, shmem, s);
    case 32: return launch_lds_k<T, 32, false>(a, shmem, s);
    default: return fail(ATK_UNSUPPORTED, "dwconv1d: bad variant");
  }
}

// ---------------------------------------------------------------------------------------
// Backward.  The input gradient needs no kernel of its own: dx[s] = sum_k w[k] dy[s+pad-k]
// is the forward kernel run on dy with w'[j] = w[K-1-j] and pad' = K-1-pad (the identity
// the reference's backward uses, _vendor/flashfftconv_depthwise_conv1d/
// conv1d_bwd_hip_bhl.hip:39-57).  The weight and bias gradients
//   dw[c,k] = sum_{n,t} dy[n,c,t] * x[n,c,t-pad+k],   db[c] = sum_{n,t} dy[n,c,t]
// are one streaming pass over x and dy: a workgroup per (n, c) row reduces its row into
// K+1 fp32 partials, a finalize kernel sums the partials over n in a fixed order.  Both
// windows (dy's VEC outputs, x's VEC+K-1 inputs) are cut from aligned 16-byte blocks as in
// the register kernel, so rows need not be 16-byte aligned (the stock-shaped causal dy).
// HBM traffic: one read of x and one of dy; the reference materialises dk[B,C,K,L] and
// multiplies it with dy (conv1d_bwd_hip_bhl.hip:62-116).
struct DwBwdArgs {
  const void* x;
  const void* dy;
  float* part;        // [N*C][K+1]
  uint32_t L, Lout;
  int pad;
  int x_off, dy_off;  // misalignment of the x / dy base pointers, in elements
  int64_t total_in, total_out;
};

template <typename T, int KT>
__global__ __launch_bounds__(DW_NT) void dwconv1d_bwd_w_kernel(DwBwdArgs a) {
  using Win = DwWindow<T, KT>;
  using Dyw = DwWindow<T, 1>;
  constexpr int VEC = Win::VEC, WN = Win::WN;
  // output vectors fetched per thread before any is used: config 2's 8195-output rows take 5
  // serial load rounds with 1, 3 with 2; 2 measured level with or up to 3% faster than 1 over
  // the whole backward, 4 (more registers, fewer resident workgroups) 8% slower
  constexpr int BWD_U = 2;
  __shared__ float red[(KT + 1) * (DW_NT / 64)];
  const uint32_t r = blockIdx.x;  // row n*C + c
  const uint32_t L = a.L, Lout = a.Lout;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      static_cast<const T*>(a.x) - a.x_off, (uint32_t)((a.total_in + a.x_off + VEC - 1) / VEC * 16));
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(
      static_cast<const T*>(a.dy) - a.dy_off, (uint32_t)((a.total_out + a.dy_off + VEC - 1) / VEC * 16));
  float acc[KT + 1];
#pragma unroll
  for (int k = 0; k <= KT; ++k) acc[k] = 0.f;
  // BWD_U output vectors per thread are fetched before any is used (positions past the row
  // issue out-of-range loads that read zero); the sums still run over t in order
  for (uint32_t t0 = threadIdx.x * VEC; t0 < Lout; t0 += BWD_U * DW_NT * VEC) {
    uint32_t DD[BWD_U][4 * Dyw::NBLK], DX[BWD_U][4 * Win::NBLK];
    int md[BWD_U], mx[BWD_U];
#pragma unroll
    for (int u = 0; u < BWD_U; ++u) {
      const uint32_t t = t0 + u * DW_NT * VEC;
      const bool act = t < Lout;
      const uint32_t tc = act ? t : 0u;
      Dyw::fetch(rd, (int)(r * Lout + tc) + a.dy_off, act, DD[u], md[u]);
      Win::fetch(rx, (int)(r * L + tc) - a.pad + a.x_off, act, DX[u], mx[u]);
    }
#pragma unroll
    for (int u = 0; u < BWD_U; ++u) {
      const uint32_t t = t0 + u * DW_NT * VEC;
      float dv[VEC], xv[WN];
      Dyw::extract(DD[u], md[u], (int)t, Lout, dv);       // zero past the row end
      Win::extract(DX[u], mx[u], (int)t - a.pad, L, xv);  // zero outside [0, L)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        acc[KT] += dv[e];
#pragma unroll
        for (int k = 0; k < KT; ++k) acc[k] = fmaf(dv[e], xv[e + k], acc[k]);
      }
    }
  }
  // only thread 0 writes the row's partials: one LDS exchange for all K+1 sums
#pragma unroll
  for (int k = 0; k <= KT; ++k) acc[k] = wave_sum(acc[k]);
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k <= KT; ++k) red[k * (DW_NT / 64) + (threadIdx.x >> 6)] = acc[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k <= KT; ++k) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < DW_NT / 64; ++w) v += red[k * (DW_NT / 64) + w];  // block_sum's order
      a.part[(int64_t)r * (KT + 1) + k] = v;
    }
  }
}

// dx, dw and db in one pass over each (n, c) row: x and dy are read once and dx written once
// (the two-kernel form -- the forward kernel on dy for dx, dwconv1d_bwd_w_kernel for dw / db --
// reads dy twice).  A thread walks x positions p0 = p_lo + (tid + m * DW_NT) * VEC over
// [p_lo, p_end); at each it cuts the dy window dy[p0 + pad - (K-1) ... + VEC + K - 2] and the x
// vector x[p0 ... p0 + VEC - 1] from aligned 16-byte blocks (so neither row needs alignment)
// and computes
//   dx[p0 + e] = sum_j w[j] * dy[p0 + e + pad - j]            (stored for p0 in [0, L)),
//   dw[j]     += sum_e x[p0 + e] * dy[p0 + e + pad - j],
//   db        += sum_e dy[p0 + pad - (K-1) + e].
// Positions outside [0, L) / [0, L_out) read as zero.  The host picks p_lo <= min(0, K-1-pad)
// (a multiple of VEC) and p_end >= max(L, L_out + K-1-pad), so every x position and every dy
// position is visited exactly once.  dx rows must be 16-byte aligned (L % VEC == 0, aligned
// base: host check).
struct DwBwdFusedArgs {
  const void* x;
  const void* dy;
  const void* w;      // [C][K], the dtype of x
  void* dx;
  float* part;        // [N*C][K+1], or null (dx only)
  uint32_t L, Lout, C;
  int pad;
  int x_off, dy_off;  // misalignment of the x / dy base pointers, in elements
  int64_t total_in, total_out;
  int p_lo, p_end;
};

template <typename T, int KT>
__global__ __launch_bounds__(DW_NT) void dwconv1d_bwd_fused_kernel(DwBwdFusedArgs a) {
  using Dyw = DwWindow<T, KT>;
  using Xw = DwWindow<T, 1>;
  constexpr int VEC = Dyw::VEC, WN = Dyw::WN;
  __shared__ float red[(KT + 1) * (DW_NT / 64)];
  const uint32_t r = blockIdx.x;  // row n*C + c
  const uint32_t c = r % a.C;
  float wv[KT];
#pragma unroll
  for (int j = 0; j < KT; ++j) wv[j] = to_f32(static_cast<const T*>(a.w)[c * KT + j]);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      static_cast<const T*>(a.x) - a.x_off, (uint32_t)((a.total_in + a.x_off + VEC - 1) / VEC * 16));
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(
      static_cast<const T*>(a.dy) - a.dy_off, (uint32_t)((a.total_out + a.dy_off + VEC - 1) / VEC * 16));
  T* __restrict__ dxr = static_cast<T*>(a.dx) + (int64_t)r * a.L;
  const int L = (int)a.L;
  float acc[KT + 1];
#pragma unroll
  for (int k = 0; k <= KT; ++k) acc[k] = 0.f;
  // two positions per trip, every load of both issued before either is used (a trip past
  // p_end loads zeros, which add nothing, and stores nothing)
  constexpr int STEP = DW_NT * VEC;
  for (int p0 = a.p_lo + (int)threadIdx.x * VEC; p0 < a.p_end; p0 += 2 * STEP) {
    uint32_t DD[2][4 * Dyw::NBLK], DX[2][4 * Xw::NBLK];
    int md[2], mx[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int pu = p0 + u * STEP;
      const int g = pu + a.pad - (KT - 1);  // row position of the window's first dy element
      Dyw::fetch(rd, (int)(r * a.Lout) + g + a.dy_off, pu < a.p_end, DD[u], md[u]);
      Xw::fetch(rx, (int)(r * a.L) + pu + a.x_off, pu < a.p_end, DX[u], mx[u]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int pu = p0 + u * STEP;
      const int g = pu + a.pad - (KT - 1);
      float dv[WN], xv[VEC];
      Dyw::extract(DD[u], md[u], g, a.Lout, dv);  // zero outside [0, L_out)
      Xw::extract(DX[u], mx[u], pu, a.L, xv);     // zero outside [0, L)
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float sx = 0.f;
#pragma unroll
        for (int j = 0; j < KT; ++j) sx = fmaf(wv[j], dv[e + KT - 1 - j], sx);
        o[e] = sx;
        acc[KT] += dv[e];
#pragma unroll
        for (int j = 0; j < KT; ++j) acc[j] = fmaf(xv[e], dv[e + KT - 1 - j], acc[j]);
      }
      if (pu < a.p_end && pu >= 0 && pu < L) st16<false>(dxr + pu, pack16<T>(o));
    }
  }
  if (!a.part) return;
  // thread 0 writes the row's K+1 partials: one LDS exchange
#pragma unroll
  for (int k = 0; k <= KT; ++k) acc[k] = wave_sum(acc[k]);
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k <= KT; ++k) red[k * (DW_NT / 64) + (threadIdx.x >> 6)] = acc[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k <= KT; ++k) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < DW_NT / 64; ++w) v += red[k * (DW_NT / 64) + w];
      a.part[(int64_t)r * (KT + 1) + k] = v;
    }
  }
}

template <typename T>
int launch_dw_bwd_fused(const DwBwdFusedArgs& a, int64_t rows, int K, hipStream_t s) {
  const dim3 grid((unsigned)rows), block(DW_NT);
  switch (K) {
    case 1: hipLaunchKernelGGL((dwconv1d_bwd_fused_kernel<T, 1>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((dwconv1d_bwd_fused_kernel<T, 2>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((dwconv1d_bwd_fused_kernel<T, 3>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((dwconv1d_bwd_fused_kernel<T, 4>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((dwconv1d_bwd_fused_kernel<T, 5>), grid, block, 0, s, a); break;
    default: return fail(ATK_UNSUPPORTED, "dwconv1d backward: K %d outside [1, 5]", K);
  }
  return check_launch("dwconv1d_bwd_fused_kernel");
}

// dw[c,k] (k < K) and db[c] (k == K) = sum over n of the row partials, n in order.
__global__ __launch_bounds__(256) void dwconv1d_bwd_finalize_kernel(const float* __restrict__ part, float* __restrict__ dw,
                                                                    float* __restrict__ db, int N, int C, int K) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // c * (K+1) + k
  if (i >= C * (K + 1)) return;
  const int c = i / (K + 1), k = i - c * (K + 1);
  float s = 0.f;
  for (int n = 0; n < N; ++n) s += part[((int64_t)n * C + c) * (K + 1) + k];
  if (k < K) dw[c * K + k] = s;
  else if (db) db[c] = s;
}

template <typename T>
int launch_dw_bwd_w(const DwBwdArgs& a, int64_t rows, int K, hipStream_t s) {
  const dim3 grid((unsigned)rows), block(DW_NT);
  switch (K) {
    case 1: hipLaunchKernelGGL((dwconv1d_bwd_w_kernel<T, 1>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((dwconv1d_bwd_w_kernel<T, 2>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((dwconv1d_bwd_w_kernel<T, 3>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((dwconv1d_bwd_w_kernel<T, 4>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((dwconv1d_bwd_w_kernel<T, 5>), grid, block, 0, s, a); break;
    default: return fail(ATK_UNSUPPORTED, "dwconv1d backward: K %d outside [1, 5]", K);
  }
  return check_launch("dwconv1d_bwd_w_kernel");
}

// ---------------------------------------------------------------------------------------
// Decode step of the causal conv (reference: src/causal-conv1d-amd/csrc/
// causal_conv1d_update.cu:27-66, interface causal_conv1d_interface.py:175-213):
//   state[b,d,:] <- (state[b,d,1:], x[b,d]),   y[b,d] = bias[d] + sum_j w[d,j] * state[b,d,j]
// (+ SiLU).  One thread per (b, d); the state row is shifted in place in order, so every
// element is read before it is overwritten.  Latency-bound: B*D*(W+2) elements per step.
template <typename T, bool SILU>
__global__ __launch_bounds__(256) void causal_conv1d_update_kernel(const T* __restrict__ x, T* __restrict__ state,
                                                                   const void* __restrict__ w,
                                                                   const void* __restrict__ bias, T* __restrict__ y,
                                                                   int64_t rows, uint32_t D, int W, bool w32) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // b * D + d
  if (i >= rows) return;
  const uint32_t d = (uint32_t)(i % D);
  T* st = state + i * W;
  const int64_t wd = (int64_t)d * W;
  float acc = bias ? dw_param<T>(bias, w32, d) : 0.f;
  for (int j = 0; j + 1 < W; ++j) {
    const T v = st[j + 1];
    st[j] = v;
    acc = fmaf(dw_param<T>(w, w32, wd + j), to_f32(v), acc);
  }
  const T v = x[i];
  st[W - 1] = v;
  acc = fmaf(dw_param<T>(w, w32, wd + W - 1), to_f32(v), acc);
  if constexpr (SILU) acc = silu_f32(acc);
  y[i] = from_f32<T>(acc);
}

template <typename T>
int launch_update(const void* x, void* state, const void* w, const void* bias, void* y, int64_t rows, int64_t D,
                  int W, int silu, bool w32, hipStream_t s) {
  const dim3 grid((unsigned)((rows + 255) / 256)), block(256);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, s, static_cast<const T*>(x), static_cast<T*>(state), w, bias,
                       static_cast<T*>(y), rows, (uint32_t)D, W, w32);
  };
  if (silu) args(causal_conv1d_update_kernel<T, true>);
  else args(causal_conv1d_update_kernel<T, false>);
  return check_launch("causal_conv1d_update_kernel");
}

// ---------------------------------------------------------------------------------------
// Causal conv1d backward, fused, (B, C, L) layout (src/causal-conv1d-amd/csrc/
// causal_conv1d_bwd.cu:100-235, the non-channel-last kernel): with H = K-1, z the forward's
// pre-activation (recomputed in fp32) and g = dout * silu'(z) (dout without the activation),
//   dx[p] = sum_j w[j] * g[p + H - j],  dw[j] = sum_p g[p] * x[p - H + j],  db = sum_p g[p].
// One workgroup per (b, c) row; a thread owns CB_T consecutive positions and loads, as aligned
// 16-byte buffer loads (positions < 0 or >= L read zero), the x window [p0 - PRE*VEC,
// p0 + CB_T + POST*VEC) and the dout window [p0, p0 + CB_T + POST*VEC): x and dout are read once
// (the halos are L1/L2 hits) and dx written once.  dw / db: per-thread sums, a fixed-order block
// reduction into per-row partials, and the per-channel finalize above (sum over b in order).
// ---------------------------------------------------------------------------------------
constexpr int CB_T = 32;  // positions per thread

struct CbArgs {
  const void* x;
  const void* dy;
  void* dx;
  const void* w;
  const void* b;
  int wdt;
  int64_t wc, wk;
  float* part;    // [B*D][K+1]
  uint32_t D, L;
  uint32_t row_bytes;
};

template <typename T, int KT, bool SILU>
__global__ __launch_bounds__(DW_NT) void causal_bwd_bcl_kernel(CbArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int H = KT - 1;
  constexpr int NV = CB_T / VEC;               // vectors of the thread's own positions
  constexpr int PRE = (2 * H + VEC - 1) / VEC;  // x vectors before p0 (SiLU recompute reaches p0 - 2H)
  constexpr int POST = (H + VEC - 1) / VEC;     // vectors after p0 + CB_T (g reaches p0 + CB_T + H - 1)
  constexpr int XV = PRE + NV + POST, GV = NV + POST;
  __shared__ float red[DW_NT / 64];
  const int64_t row = blockIdx.x;
  const uint32_t d = (uint32_t)(row % a.D);
  float wv[KT], bv = 0.f;
#pragma unroll
  for (int j = 0; j < KT; ++j) wv[j] = load_param(a.w, a.wdt, (int64_t)d * a.wc + (int64_t)j * a.wk);
  if (SILU && a.b) bv = load_param(a.b, a.wdt, d);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + row * a.L, a.row_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(static_cast<const T*>(a.dy) + row * a.L, a.row_bytes);
  T* dxr = static_cast<T*>(a.dx) + row * a.L;
  const int L = (int)a.L;
  float accw[KT], accb = 0.f;
#pragma unroll
  for (int j = 0; j < KT; ++j) accw[j] = 0.f;
  for (int base = 0; base < L; base += DW_NT * CB_T) {
    const int p0 = base + (int)threadIdx.x * CB_T;
    if (p0 >= L) break;
    Vec16<T> xr[XV], gr[GV];
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int p = p0 + (v - PRE) * VEC;
      xr[v].raw = bload16(rx, (p >= 0 && p < L) ? (uint32_t)p * (uint32_t)sizeof(T) : kOOB, 0);
    }
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int p = p0 + v * VEC;
      gr[v].raw = bload16(rg, p < L ? (uint32_t)p * (uint32_t)sizeof(T) : kOOB, 0);
    }
    // x element of position p0 + i:  xe(i) = xr[(PRE*VEC + i) / VEC].e[(PRE*VEC + i) % VEC]
#define XE(i) to_f32(xr[(PRE * VEC + (i)) / VEC].e[(PRE * VEC + (i)) % VEC])
    // g for positions p0 .. p0 + CB_T + H - 1
    float g[CB_T + H];
#pragma unroll
    for (int i = 0; i < CB_T + H; ++i) {
      float gi = to_f32(gr[i / VEC].e[i % VEC]);
      if constexpr (SILU) {
        float z = bv;
#pragma unroll
        for (int j = 0; j < KT; ++j) z = __builtin_fmaf(wv[j], XE(i - H + j), z);
        const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-z));
        gi *= sg * (1.0f + z * (1.0f - sg));
      }
      g[i] = gi;
    }
    // dx for the thread's positions, and the dw / db sums (g past L is zero: dout read zero)
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int i = v * VEC + e;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KT; ++j) acc = __builtin_fmaf(wv[j], g[i + H - j], acc);
        o[e] = acc;
        accb += g[i];
#pragma unroll
        for (int j = 0; j < KT; ++j) accw[j] = __builtin_fmaf(g[i], XE(i - H + j), accw[j]);
      }
      if (p0 + v * VEC < L) st16<false>(dxr + p0 + v * VEC, pack16<T>(o));
    }
#undef XE
  }
#pragma unroll
  for (int j = 0; j < KT; ++j) {
    const float sj = block_sum<DW_NT>(accw[j], red);
    if (threadIdx.x == 0) a.part[row * (KT + 1) + j] = sj;
  }
  const float sb = block_sum<DW_NT>(accb, red);
  if (threadIdx.x == 0) a.part[row * (KT + 1) + KT] = sb;
}

template <typename T, int KT>
void launch_cb_kt(const CbArgs& a, int64_t rows, int silu, hipStream_t s) {
  if (silu) hipLaunchKernelGGL((causal_bwd_bcl_kernel<T, KT, true>), dim3((unsigned)rows), dim3(DW_NT), 0, s, a);
  else hipLaunchKernelGGL((causal_bwd_bcl_kernel<T, KT, false>), dim3((unsigned)rows), dim3(DW_NT), 0, s, a);
}

template <typename T>
int launch_cb(const CbArgs& a, int64_t rows, int K, int silu, hipStream_t s) {
  switch (K) {
    case 2: launch_cb_kt<T, 2>(a, rows, silu, s); break;
    case 3: launch_cb_kt<T, 3>(a, rows, silu, s); break;
    case 4: launch_cb_kt<T, 4>(a, rows, silu, s); break;
    default: return fail(ATK_UNSUPPORTED, "causal_conv1d_bwd: width %d outside [2, 4]", K);
  }
  return check_launch("causal_bwd_bcl_kernel");
}

}  // namespace

int dwconv1d_num_variants() { return kNumDw; }
const char* dwconv1d_variant_name(int v) {
  return (v >= 0 && v < kNumDw) ? kDwVariants[v].name : nullptr;
}

}  // namespace atk

extern "C" int atk_dwconv1d_fwd(const void* x, const void* w, const void* bias, void* y,
                                int64_t N, int64_t C, int64_t L, int K, int pad_left,
                                int64_t L_out, int dtype, int w_dtype, int fuse_silu, int variant,
                                atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "dwconv1d: unknown dtype code %d", dtype);
  if (w_dtype != dtype && w_dtype != ATK_F32)
    return fail(ATK_EINVAL, "dwconv1d: weights must be in the input's dtype or fp32 (code %d)", w_dtype);
  if (w_dtype == ATK_F32 && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(bias)) & 3u))
    return fail(ATK_EINVAL, "dwconv1d: misaligned fp32 weight or bias pointer");
  if (N < 0 || C <= 0 || L < 0 || L_out < 0) return fail(ATK_EINVAL, "dwconv1d: bad sizes");
  if (K < 1 || K > DW_KMAX) return fail(ATK_UNSUPPORTED, "dwconv1d: kernel width %d outside [1, %d]", K, DW_KMAX);
  if (pad_left < 0 || pad_left > DW_PADMAX) return fail(ATK_UNSUPPORTED, "dwconv1d: padding %d outside [0, %d]", pad_left, DW_PADMAX);
  if (variant >= kNumDw) return fail(ATK_EINVAL, "dwconv1d: variant %d out of range", variant);
  const int64_t total_out = N * C * L_out;
  if (total_out == 0) return ATK_OK;
  if (!x || !w || !y) return fail(ATK_EINVAL, "dwconv1d: null pointer");
  const int64_t rows = N * C;
  if (rows >= (1ll << 31) || L >= (1ll << 30) || L_out >= (1ll << 30))
    return fail(ATK_UNSUPPORTED, "dwconv1d: sizes exceed 32-bit row/column indexing");
  const size_t es = dtype_size(dtype);
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), ya = reinterpret_cast<uintptr_t>(y);
  if ((xa % es) || (ya % es)) return fail(ATK_EINVAL, "dwconv1d: misaligned element pointer");
  DwArgs a;
  a.x = x; a.w = w; a.b = bias; a.y = y;
  a.total_in = rows * L;
  a.total_out = total_out;
  a.C = (uint32_t)C; a.L = (uint32_t)L; a.Lout = (uint32_t)L_out;
  a.K = K; a.pad = pad_left;
  a.x_off = (int)((xa & 15u) / es);
  a.y_off = (int)((ya & 15u) / es);
  a.silu = fuse_silu ? 1 : 0;
  a.w32 = w_dtype == ATK_F32 && dtype != ATK_F32;
  a.div_lout = make_fastdiv((uint32_t)L_out);
  a.div_c = make_fastdiv((uint32_t)C);
  a.win_cap = 0;
  // fdiv() needs numerators below 2^31: row-relative offsets stay below L_out + tile.
  if ((uint64_t)L_out + 65536 >= (1ull << 31)) return fail(ATK_UNSUPPORTED, "dwconv1d: L_out too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto run = [&](int v) {
    switch (dtype) {
      case ATK_F32: return launch_dw<float>(a, v, s);
      case ATK_F16: return launch_dw<_Float16>(a, v, s);
      default: return launch_dw<__bf16>(a, v, s);
    }
  };
  if (variant >= 0) return run(variant);
  // default: the first of these that takes the shape (a declining variant enqueues nothing)
  for (const char* name : {"xlane", "lds_opt32_nt", "lds_opt16", "direct"}) {
    int v = 0;
    while (v < kNumDw && std::strcmp(kDwVariants[v].name, name) != 0) ++v;
    const int rc = run(v);
    if (rc != ATK_UNSUPPORTED) return rc;
  }
  return fail(ATK_UNSUPPORTED, "dwconv1d: no variant takes the shape");
}

extern "C" size_t atk_dwconv1d_bwd_weight_workspace_bytes(int64_t N, int64_t C, int K) {
  if (N <= 0 || C <= 0 || K < 1) return 0;
  return (size_t)N * (size_t)C * (size_t)(K + 1) * sizeof(float);
}

extern "C" int atk_dwconv1d_bwd_weight(const void* x, const void* dy, float* dw, float* db, int64_t N,
                                       int64_t C, int64_t L, int K, int pad_left, int64_t L_out, int dtype,
                                       void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "dwconv1d backward: unknown dtype code %d", dtype);
  if (N <= 0 || C <= 0 || L < 0 || L_out < 0) return fail(ATK_EINVAL, "dwconv1d backward: bad sizes");
  if (K < 1 || K > 5) return fail(ATK_UNSUPPORTED, "dwconv1d backward: K %d outside [1, 5]", K);
  if (pad_left < 0 || pad_left > DW_PADMAX)
    return fail(ATK_UNSUPPORTED, "dwconv1d backward: padding %d outside [0, %d]", pad_left, DW_PADMAX);
  if (!x || !dy || !dw) return fail(ATK_EINVAL, "dwconv1d backward: null pointer");
  const size_t need = atk_dwconv1d_bwd_weight_workspace_bytes(N, C, K);
  if (!workspace || ws_bytes < need) return fail(ATK_EINVAL, "dwconv1d backward: workspace of %zu bytes needed", need);
  const size_t es = dtype_size(dtype);
  const int64_t rows = N * C;
  const int64_t vec = 16 / (int64_t)es;
  // windows are addressed with 32-bit element offsets and 32-bit buffer byte ranges
  if (rows >= (1ll << 31) || rows * L + vec >= (1ll << 31) / (int64_t)es ||
      rows * L_out + vec >= (1ll << 31) / (int64_t)es)
    return fail(ATK_UNSUPPORTED, "dwconv1d backward: tensor too large");
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), da = reinterpret_cast<uintptr_t>(dy);
  if ((xa % es) || (da % es)) return fail(ATK_EINVAL, "dwconv1d backward: misaligned element pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // (L_out == 0 needs no special case: every row reduces nothing and the gradients are 0)
  DwBwdArgs a;
  a.x = x; a.dy = dy;
  a.part = static_cast<float*>(workspace);
  a.L = (uint32_t)L; a.Lout = (uint32_t)L_out;
  a.pad = pad_left;
  a.x_off = (int)((xa & 15u) / es);
  a.dy_off = (int)((da & 15u) / es);
  a.total_in = rows * L;
  a.total_out = rows * L_out;
  int rc;
  switch (dtype) {
    case ATK_F32: rc = launch_dw_bwd_w<float>(a, rows, K, s); break;
    case ATK_F16: rc = launch_dw_bwd_w<_Float16>(a, rows, K, s); break;
    default: rc = launch_dw_bwd_w<__bf16>(a, rows, K, s); break;
  }
  if (rc) return rc;
  const int outs = (int)(C * (K + 1));
  hipLaunchKernelGGL(dwconv1d_bwd_finalize_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s,
                     a.part, dw, db, (int)N, (int)C, K);
  return check_launch("dwconv1d_bwd_finalize_kernel");
}

extern "C" int atk_dwconv1d_bwd(const void* x, const void* dy, const void* w, void* dx, float* dw, float* db,
                                int64_t N, int64_t C, int64_t L, int K, int pad_left, int64_t L_out, int dtype,
                                void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "dwconv1d backward: unknown dtype code %d", dtype);
  if (N <= 0 || C <= 0 || L <= 0 || L_out < 0) return fail(ATK_EINVAL, "dwconv1d backward: bad sizes");
  if (K < 1 || K > 5) return fail(ATK_UNSUPPORTED, "dwconv1d backward: K %d outside [1, 5]", K);
  if (pad_left < 0 || pad_left > DW_PADMAX)
    return fail(ATK_UNSUPPORTED, "dwconv1d backward: padding %d outside [0, %d]", pad_left, DW_PADMAX);
  if (!x || !dy || !w || !dx) return fail(ATK_EINVAL, "dwconv1d backward: null pointer");
  if (db && !dw) return fail(ATK_EINVAL, "dwconv1d backward: db needs dw");
  const bool with_w = dw != nullptr;
  const size_t need = with_w ? atk_dwconv1d_bwd_weight_workspace_bytes(N, C, K) : 0;
  if (with_w && (!workspace || ws_bytes < need))
    return fail(ATK_EINVAL, "dwconv1d backward: workspace of %zu bytes needed", need);
  const size_t es = dtype_size(dtype);
  const int64_t rows = N * C;
  const int64_t vec = 16 / (int64_t)es;
  if (rows >= (1ll << 31) || rows * L + vec >= (1ll << 31) / (int64_t)es ||
      rows * L_out + 2 * vec + K + DW_PADMAX >= (1ll << 31) / (int64_t)es)
    return fail(ATK_UNSUPPORTED, "dwconv1d backward: tensor too large");
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), da = reinterpret_cast<uintptr_t>(dy);
  if ((xa % es) || (da % es)) return fail(ATK_EINVAL, "dwconv1d backward: misaligned element pointer");
  if (L % vec || !aligned16(dx))
    return fail(ATK_UNSUPPORTED, "dwconv1d backward: the fused kernel needs 16-byte aligned dx rows");
  DwBwdFusedArgs a;
  a.x = x; a.dy = dy; a.w = w; a.dx = dx;
  a.part = with_w ? static_cast<float*>(workspace) : nullptr;
  a.L = (uint32_t)L; a.Lout = (uint32_t)L_out; a.C = (uint32_t)C;
  a.pad = pad_left;
  a.x_off = (int)((xa & 15u) / es);
  a.dy_off = (int)((da & 15u) / es);
  a.total_in = rows * L;
  a.total_out = rows * L_out;
  const int lo = std::min(0, K - 1 - pad_left);
  a.p_lo = lo >= 0 ? 0 : -(int)(((-lo) + vec - 1) / vec * vec);
  a.p_end = (int)std::max<int64_t>(L, L_out + K - 1 - pad_left);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc;
  switch (dtype) {
    case ATK_F32: rc = launch_dw_bwd_fused<float>(a, rows, K, s); break;
    case ATK_F16: rc = launch_dw_bwd_fused<_Float16>(a, rows, K, s); break;
    default: rc = launch_dw_bwd_fused<__bf16>(a, rows, K, s); break;
  }
  if (rc || !with_w) return rc;
  const int outs = (int)(C * (K + 1));
  hipLaunchKernelGGL(dwconv1d_bwd_finalize_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s,
                     a.part, dw, db, (int)N, (int)C, K);
  return check_launch("dwconv1d_bwd_finalize_kernel");
}

extern "C" int atk_causal_conv1d_update(const void* x, void* conv_state, const void* w, const void* bias, void* y,
                                        int64_t B, int64_t D, int W, int dtype, int w_dtype, int fuse_silu,
                                        atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "causal_conv1d_update: unknown dtype code %d", dtype);
  if (w_dtype != dtype && w_dtype != ATK_F32)
    return fail(ATK_EINVAL, "causal_conv1d_update: weights must be in the input's dtype or fp32 (code %d)", w_dtype);
  if (w_dtype == ATK_F32 && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(bias)) & 3u))
    return fail(ATK_EINVAL, "causal_conv1d_update: misaligned fp32 weight or bias pointer");
  const bool w32 = w_dtype == ATK_F32 && dtype != ATK_F32;
  if (B < 0 || D <= 0) return fail(ATK_EINVAL, "causal_conv1d_update: bad sizes");
  if (W < 1 || W > DW_KMAX) return fail(ATK_UNSUPPORTED, "causal_conv1d_update: width %d outside [1, %d]", W, DW_KMAX);
  const int64_t rows = B * D;
  if (rows == 0) return ATK_OK;
  if (!x || !conv_state || !w || !y) return fail(ATK_EINVAL, "causal_conv1d_update: null pointer");
  if (rows >= (1ll << 31) * 256ll) return fail(ATK_UNSUPPORTED, "causal_conv1d_update: too many rows");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case ATK_F32: return launch_update<float>(x, conv_state, w, bias, y, rows, D, W, fuse_silu, w32, s);
    case ATK_F16: return launch_update<_Float16>(x, conv_state, w, bias, y, rows, D, W, fuse_silu, w32, s);
    default: return launch_update<__bf16>(x, conv_state, w, bias, y, rows, D, W, fuse_silu, w32, s);
  }
}

extern "C" int atk_causal_conv1d_bwd(const void* x, const void* dout, const void* w, const void* bias, void* dx,
                                     float* dw, float* db, int64_t B, int64_t D, int64_t L, int K,
                                     int64_t w_stride_c, int64_t w_stride_k, int dtype, int w_dtype, int silu,
                                     void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype) || !dtype_ok(w_dtype)) return fail(ATK_EINVAL, "causal_conv1d_bwd: unknown dtype code");
  if (B <= 0 || D <= 0 || L <= 0) return fail(ATK_EINVAL, "causal_conv1d_bwd: bad sizes");
  if (!x || !dout || !dx || !w || !dw) return fail(ATK_EINVAL, "causal_conv1d_bwd: null pointer");
  if (K < 2 || K > 4) return fail(ATK_UNSUPPORTED, "causal_conv1d_bwd: width %d outside [2, 4]", K);
  const int64_t es = (int64_t)dtype_size(dtype), vec = 16 / es;
  if (L % vec || !aligned16(x) || !aligned16(dout) || !aligned16(dx))
    return fail(ATK_UNSUPPORTED, "causal_conv1d_bwd: needs L %% %lld == 0 and 16-byte aligned tensors",
                (long long)vec);
  const int64_t rows = B * D;
  if (rows >= (1ll << 31) || L * es >= (1ll << 31)) return fail(ATK_UNSUPPORTED, "causal_conv1d_bwd: too large");
  const size_t need = (size_t)rows * (size_t)(K + 1) * sizeof(float);
  if (!workspace || ws_bytes < need) return fail(ATK_EINVAL, "causal_conv1d_bwd: workspace of %zu bytes needed", need);
  CbArgs a;
  a.x = x; a.dy = dout; a.dx = dx; a.w = w; a.b = bias; a.wdt = w_dtype; a.wc = w_stride_c; a.wk = w_stride_k;
  a.part = static_cast<float*>(workspace);
  a.D = (uint32_t)D; a.L = (uint32_t)L;
  a.row_bytes = (uint32_t)(L * es);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc;
  switch (dtype) {
    case ATK_F32: rc = launch_cb<float>(a, rows, K, silu, s); break;
    case ATK_F16: rc = launch_cb<_Float16>(a, rows, K, silu, s); break;
    default: rc = launch_cb<__bf16>(a, rows, K, silu, s); break;
  }
  if (rc) return rc;
  const int outs = (int)(D * (K + 1));
  hipLaunchKernelGGL(dwconv1d_bwd_finalize_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s,
                     a.part, dw, db, (int)B, (int)D, K);
  return check_launch("dwconv1d_bwd_finalize_kernel");
}

extern "C" int atk_dwconv1d_fwd_args(const atk_dwconv1d_args* a) {
  if (!a) return atk::fail(ATK_EINVAL, "dwconv1d: null argument block");
  return atk_dwconv1d_fwd(a->x, a->w, a->bias, a->y, a->N, a->C, a->L, a->K, a->pad_left, a->L_out, a->dtype,
                          a->w_dtype, a->fuse_silu, a->variant, a->stream);
}
