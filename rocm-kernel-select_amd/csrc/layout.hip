// Layout conversion between channels-last and channels-first memory: a batched transpose of
// the last two axes, out[b][c][r] = in[b][r][c].
//
// An NDHWC tensor is [N][D*H*W][C] in memory and its NCDHW form is [N][C][D*H*W], so one
// batched transpose converts either way (weights: [Co][taps][Ci] <-> [Co][Ci][taps]).  The
// channels-last conv path needs these conversions around the NCDHW MFMA tiles; torch's strided
// copy ran them at a fraction of HBM bandwidth.
//
// A workgroup moves one 64 x 64 tile through LDS: the tile's rows are read as 16-byte vectors
// (coalesced along c), written to LDS with a padded pitch, and read back along r so that the
// output rows are again written as 16-byte vectors (coalesced along r).  When a row length is
// not a multiple of a vector, or a base pointer is not 16-byte aligned, the same tile walk runs
// element by element.  Pure data movement: every byte of the input is copied unchanged.
#include "atk_common.h"

namespace atk {
namespace {

constexpr int TP_T = 64;    // tile edge (elements)
constexpr int TP_NT = 256;  // threads per workgroup

// a 16-byte vector viewed as its elements
template <typename E>
union TpVec {
  uint4 v;
  E e[16 / sizeof(E)];
};

struct TpArgs {
  const void* in;
  void* out;
  int64_t B, R, C;
  int64_t tiles_c;  // tiles along c
};

template <typename E, bool VECOK>
__global__ __launch_bounds__(TP_NT) void transpose_tile_kernel(TpArgs a) {
  constexpr int VEC = 16 / sizeof(E);        // elements per 16-byte vector
  constexpr int PITCH = TP_T + 2;            // LDS row pitch: consecutive rows start on other banks
  constexpr int VPR = TP_T / VEC;            // vectors per tile row
  constexpr int NV = TP_T * VPR / TP_NT;     // vectors per thread (2 for 16-bit, 4 for fp32)
  __shared__ E tile[TP_T * PITCH];
  const int64_t t = blockIdx.x;
  const int64_t r0 = (t / a.tiles_c) * TP_T, c0 = (t % a.tiles_c) * TP_T;
  const int tid = threadIdx.x;
  for (int64_t b = blockIdx.y; b < a.B; b += gridDim.y) {
    const E* __restrict__ in = static_cast<const E*>(a.in) + b * a.R * a.C;
    E* __restrict__ out = static_cast<E*>(a.out) + b * a.R * a.C;
    if constexpr (VECOK) {
      // C % VEC == 0 and aligned bases: a vector is wholly inside or outside the row
      TpVec<E> v[NV];
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const int q = tid + u * TP_NT;
        const int64_t r = r0 + q / VPR, c = c0 + (q % VPR) * VEC;
        v[u].v = (r < a.R && c < a.C) ? *reinterpret_cast<const uint4*>(in + r * a.C + c) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const int q = tid + u * TP_NT;
        const int rl = q / VPR, cl = (q % VPR) * VEC;
#pragma unroll
        for (int k = 0; k < VEC; ++k) tile[rl * PITCH + cl + k] = v[u].e[k];
      }
    } else {
      for (int i = tid; i < TP_T * TP_T; i += TP_NT) {
        const int rl = i / TP_T, cl = i % TP_T;
        const int64_t r = r0 + rl, c = c0 + cl;
        tile[rl * PITCH + cl] = (r < a.R && c < a.C) ? in[r * a.C + c] : E(0);
      }
    }
    __syncthreads();
    if constexpr (VECOK) {
      // output rows (fixed c) hold R elements: vectors need R % VEC == 0 as well (host check)
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const int q = tid + u * TP_NT;
        const int cl = q / VPR, rl = (q % VPR) * VEC;
        const int64_t c = c0 + cl, r = r0 + rl;
        TpVec<E> o;
#pragma unroll
        for (int k = 0; k < VEC; ++k) o.e[k] = tile[(rl + k) * PITCH + cl];
        if (c < a.C && r < a.R) *reinterpret_cast<uint4*>(out + c * a.R + r) = o.v;
      }
    } else {
      for (int i = tid; i < TP_T * TP_T; i += TP_NT) {
        const int cl = i / TP_T, rl = i % TP_T;
        const int64_t c = c0 + cl, r = r0 + rl;
        if (c < a.C && r < a.R) out[c * a.R + r] = tile[rl * PITCH + cl];
      }
    }
    __syncthreads();  // the tile is rewritten for the next batch entry
  }
}

template <typename E>
int launch_transpose(const TpArgs& a, bool vec_ok, hipStream_t s) {
  const int64_t tiles = ((a.R + TP_T - 1) / TP_T) * a.tiles_c;
  const dim3 grid((unsigned)tiles, (unsigned)(a.B < 65535 ? a.B : 65535)), block(TP_NT);
  if (vec_ok) hipLaunchKernelGGL((transpose_tile_kernel<E, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((transpose_tile_kernel<E, false>), grid, block, 0, s, a);
  return check_launch("transpose_tile_kernel");
}

}  // namespace
}  // namespace atk

extern "C" int atk_transpose_last2(const void* in, void* out, int64_t B, int64_t R, int64_t C, int dtype,
                                   atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "transpose: unknown dtype code %d", dtype);
  if (B < 0 || R < 0 || C < 0) return fail(ATK_EINVAL, "transpose: negative size");
  if (B == 0 || R == 0 || C == 0) return ATK_OK;
  if (!in || !out) return fail(ATK_EINVAL, "transpose: null pointer");
  if (in == out) return fail(ATK_EINVAL, "transpose: input and output must not alias");
  const int64_t tiles_r = (R + TP_T - 1) / TP_T, tiles_c = (C + TP_T - 1) / TP_T;
  if (tiles_r * tiles_c > 0x7fffffff) return fail(ATK_UNSUPPORTED, "transpose: too many tiles");
  const int64_t es = (int64_t)dtype_size(dtype), vec = 16 / es;
  const bool vec_ok = C % vec == 0 && R % vec == 0 && aligned16(in) && aligned16(out);
  TpArgs a;
  a.in = in; a.out = out; a.B = B; a.R = R; a.C = C; a.tiles_c = tiles_c;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return es == 4 ? launch_transpose<uint32_t>(a, vec_ok, s) : launch_transpose<uint16_t>(a, vec_ok, s);
}
