// Weight gradient of a stride-1 "same" 3x3(x3) conv2d / conv3d on gfx950 MFMA.
//
//   dW[co, ci, kz, ky, kx] = sum_{n, z, y, x} dy[n, co, z, y, x] * x[n, ci, z+kz-pd, y+ky-1, x+kx-1]
//
// (x = 0 outside the input).  The reference computes this with aten.convolution_backward
// (amd_tuned_torch/_dispatch.py:2064-2075).  As a GEMM it is M = Co, N = Ci, K = output
// positions, once per tap:
//  * A operand (32 co x 16 positions): dy rows are contiguous along x, so a lane's fragment
//    (8 positions of one co) is one 16-byte global load, shared by all 9 in-plane taps.
//  * B operand (16 positions x 32 ci): for a workgroup's 32 input channels, TY+2 input rows
//    of the plane z+kz-pd are staged in LDS with 8 zero elements on either side of each row.
//    For 8 output positions a lane needs input elements [x0-1, x0+9) of a row (covering the
//    kx = 0, 1, 2 shifts): one b32 + one b128 + one b32 LDS read; the three shifted fragments
//    are byte-aligned from those six dwords (v_alignbyte).
//  * A workgroup = 4 waves = 128 output channels x 32 input channels x one kz; each wave
//    holds 3x3 accumulator tiles (144 fp32 registers) for its 32 output channels.
//  * The position range is split into chunks of (n, z) output planes across workgroups;
//    each writes its fp32 partials in the accumulator layout of its waves (one 1 KB run per
//    store instruction), summed in a fixed order by a reduce kernel (deterministic) that
//    turns them into the weight layout through LDS.  Partials written straight in the
//    weight layout cost more than all the MFMAs: each 128-byte line of that layout holds
//    the taps of all kz, so three workgroups (often on different XCDs, with separate L2s)
//    each write a few 4-byte pieces of it.
// The next stage's input rows are loaded into registers while the current stage computes.
#include <algorithm>

#include "conv_common.h"

namespace atk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int WG_NT = 256;   // 4 waves
constexpr int WG_CO = 128;   // output channels per workgroup (32 per wave)
constexpr int WG_CI = 32;    // input channels per workgroup
constexpr int WG_TY = 4;     // output rows per stage
constexpr int WG_R = WG_TY + 2;
constexpr int WG_PAD = 8;    // zero elements left / right of each staged row
constexpr int WG_MAXW = 64;  // staging map: 32 ci x 6 rows x W / 8 chunks over 256 threads x 6 loads
constexpr int WG_LD = 6;     // 16-byte staging loads per thread
constexpr int WG_PF = 4;     // dy fragments in flight per lane
constexpr int WG_UNIT = 9 * 16 * 64;  // partial floats of one wave: 9 taps x 16 registers x 64 lanes
constexpr int WG_RNT = 288;  // reduce workgroup: 9 taps x 32 input channels

struct WgArgs {
  const void* x;
  const void* dy;
  float* part;                 // [chunks][kz][Co/128][Ci/32][wave][tap 9][reg quad 4][lane 64][4]
  float* dw;                   // [Co][Ci][KD*9]
  int N, Ci, Co, D, H, W, KD, pd;
  int stages_per_chunk, chunks;  // a chunk is a run of (n, z, 4-row) stages
  int pitch;                   // staged row pitch in elements (W + 2*PAD)
  int slab;                    // elements per input channel in LDS (R * pitch, bank padded)
  int chunks16;                // 16-byte chunks per staged stage = WG_CI * R * W / 8
  uint32_t x_bytes, dy_bytes;
};

template <typename T>
__device__ __forceinline__ void mfma(f32x16& acc, const uint4& a, const uint4& b) {
  if constexpr (sizeof(T) == 2 && __is_same(T, __bf16))
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8*>(&a),
                                                  *reinterpret_cast<const bf16x8*>(&b), acc, 0, 0, 0);
  else
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const f16x8*>(&a),
                                                 *reinterpret_cast<const f16x8*>(&b), acc, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(WG_NT, 2) void conv_wgrad_kernel(WgArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* s_x = reinterpret_cast<T*>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int n_ci = a.Ci / WG_CI;
  // Consecutive workgroup ids are dispatched to the 8 XCDs in turn.  Each XCD gets a
  // contiguous run of logical tiles instead, so the input-channel blocks that read the same
  // dy rows (and the output-channel blocks that read the same input rows) share one L2.
  const int gx = gridDim.x, gy = gridDim.y;
  const int nwg = gx * gy * gridDim.z;
  int lid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  if ((nwg & 7) == 0) lid = (lid & 7) * (nwg >> 3) + (lid >> 3);
  const int bx = lid % gx, kz = (lid / gx) % gy, chunk = lid / (gx * gy);
  const int ci_base = (bx % n_ci) * WG_CI;
  const int co_base = (bx / n_ci) * WG_CO + wave * 32;
  const int HW = a.H * a.W;
  const int64_t plane_x = (int64_t)a.D * HW;  // elements per (n, channel) volume

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.dy, a.dy_bytes);

  // zero the row pads once (never overwritten by the staged data)
  for (int i = tid; i < WG_CI * WG_R * 2; i += WG_NT) {
    const int side = i & 1, row = (i >> 1) % WG_R, c = (i >> 1) / WG_R;
    *reinterpret_cast<uint4*>(s_x + c * a.slab + row * a.pitch + (side ? WG_PAD + a.W : 0)) = make_uint4(0, 0, 0, 0);
  }

  f32x16 acc[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // staging map: chunk q of 16 bytes -> (ci c, row r, x0)
  const int xq = a.W >> 3;  // 16-byte chunks per row
  auto stage_load = [&](int n, int zi, int y0, uint4 (&buf)[WG_LD]) {
#pragma unroll
    for (int k = 0; k < WG_LD; ++k) {
      const int q = tid + k * WG_NT;
      const int c = q / (WG_R * xq), rem = q - c * (WG_R * xq);
      const int r = rem / xq, x0 = (rem - r * xq) * 8;
      const int yi = y0 - 1 + r;
      const bool ok = q < a.chunks16 && zi >= 0 && zi < a.D && yi >= 0 && yi < a.H;
      const int64_t e = ((int64_t)n * a.Ci + ci_base + c) * plane_x + ((int64_t)zi * a.H + yi) * a.W + x0;
      buf[k] = bload16(rx, ok ? (uint32_t)(e * (int64_t)sizeof(T)) : kOOB, 0);
    }
  };
  auto stage_store = [&](const uint4 (&buf)[WG_LD]) {
#pragma unroll
    for (int k = 0; k < WG_LD; ++k) {
      const int q = tid + k * WG_NT;
      if (q < a.chunks16) {
        const int c = q / (WG_R * xq), rem = q - c * (WG_R * xq);
        const int r = rem / xq, x0 = (rem - r * xq) * 8;
        *reinterpret_cast<uint4*>(s_x + c * a.slab + r * a.pitch + WG_PAD + x0) = buf[k];
      }
    }
  };

  const int n_ystages = (a.H + WG_TY - 1) / WG_TY;
  const int ksteps_row = a.W >> 4;
  // LDS read base of this lane: input channel `col`, first 8 output positions of its half
  const T* s_lane = s_x + col * a.slab + half * 8;

  uint4 buf[WG_LD];
  int st = chunk * a.stages_per_chunk;
  const int st_end = min(st + a.stages_per_chunk, a.N * a.D * n_ystages);
  if (st < st_end) {
    const int pl = st / n_ystages, ys = st - (st / n_ystages) * n_ystages;
    stage_load(pl / a.D, pl % a.D + kz - a.pd, ys * WG_TY, buf);
  }
  for (; st < st_end; ++st) {
    const int pl = st / n_ystages, ys = st - pl * n_ystages;
    const int n = pl / a.D, z = pl - n * a.D;
    const int y0 = ys * WG_TY;
    __syncthreads();  // previous stage's reads done
    stage_store(buf);
    __syncthreads();
    const int zi = z + kz - a.pd;
    const bool live = zi >= 0 && zi < a.D;  // else this kz tap reads only zero padding (uniform)
    // a stage covers whole output rows, so k-step ks (16 positions) starts at position
    // y0*W + ks*16 of the plane: the dy offset is linear in ks
    const uint32_t g0 = (uint32_t)((((int64_t)n * a.Co + co_base + col) * plane_x + (int64_t)z * HW +
                                    (int64_t)y0 * a.W + half * 8) * (int64_t)sizeof(T));
    const int rows = min(WG_TY, a.H - y0);
    const int nk = live ? rows * ksteps_row : 0;
    uint4 ar[WG_PF];  // dy fragments stream through a ring, WG_PF k-steps ahead
#pragma unroll
    for (int u = 0; u < WG_PF; ++u) ar[u] = bload16(rg, u < nk ? g0 + (uint32_t)u * 32u : kOOB, 0);
    // the next stage's input rows are requested after this stage's first dy fragments: load
    // counters complete in issue order, so the first MFMAs do not wait for the input rows
    if (st + 1 < st_end) {
      const int pl2 = (st + 1) / n_ystages, ys2 = (st + 1) - pl2 * n_ystages;
      stage_load(pl2 / a.D, pl2 % a.D + kz - a.pd, ys2 * WG_TY, buf);
    }
    if (!live) continue;
    int xs = 0;                   // 16-position column block of the current k-step
    const T* prow = s_lane + WG_PAD;  // staged row ty (+ ky below) of the current k-step
    for (int ks0 = 0; ks0 < nk; ks0 += WG_PF) {
#pragma unroll
      for (int u = 0; u < WG_PF; ++u) {
        const int ks = ks0 + u;
        if (ks >= nk) break;
        const uint4 av = ar[u];
        ar[u] = bload16(rg, ks + WG_PF < nk ? g0 + (uint32_t)(ks + WG_PF) * 32u : kOOB, 0);
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
          // staged element index of input x' = x0 - 1 + e is PAD + x0 - 1 + e; read dwords
          // covering [PAD + x0 - 2, PAD + x0 + 10): D3 = b32 at PAD+x0-2, D4..7 = b128 at
          // PAD+x0, D8 = b32 at PAD+x0+8  (x0 = xs*16 + half*8, PAD = 8 keeps them aligned)
          const T* p = prow + ky * a.pitch + xs * 16;
          const uint32_t d3 = *reinterpret_cast<const uint32_t*>(p - 2);
          const uint4 d47 = *reinterpret_cast<const uint4*>(p);
          const uint32_t d8 = *reinterpret_cast<const uint32_t*>(p + 8);
          // kx = 0: elements start at x0 - 1 (odd): bytes 2.. of (d3, d4, ..., d7)
          uint4 f0, f2;
          f0.x = __builtin_amdgcn_alignbyte(d47.x, d3, 2);
          f0.y = __builtin_amdgcn_alignbyte(d47.y, d47.x, 2);
          f0.z = __builtin_amdgcn_alignbyte(d47.z, d47.y, 2);
          f0.w = __builtin_amdgcn_alignbyte(d47.w, d47.z, 2);
          // kx = 2: elements start at x0 + 1
          f2.x = __builtin_amdgcn_alignbyte(d47.y, d47.x, 2);
          f2.y = __builtin_amdgcn_alignbyte(d47.z, d47.y, 2);
          f2.z = __builtin_amdgcn_alignbyte(d47.w, d47.z, 2);
          f2.w = __builtin_amdgcn_alignbyte(d8, d47.w, 2);
          mfma<T>(acc[ky][0], av, f0);
          mfma<T>(acc[ky][1], av, d47);
          mfma<T>(acc[ky][2], av, f2);
        }
        if (++xs == ksteps_row) {
          xs = 0;
          prow += a.pitch;
        }
      }
    }
  }

  // partials in the accumulator layout: one float4 (4 consecutive accumulator registers)
  // per lane, so a store instruction writes 1 KB contiguous
  const int n_ci_blk = a.Ci / WG_CI;
  const int64_t unit = ((int64_t)kz * (a.Co / WG_CO) + bx / n_ci_blk) * n_ci_blk + bx % n_ci_blk;
  float* dst = a.part + (int64_t)chunk * a.Co * a.Ci * a.KD * 9 + (unit * 4 + wave) * WG_UNIT + lane * 4;
#pragma unroll
  for (int ky = 0; ky < 3; ++ky)
#pragma unroll
    for (int kx = 0; kx < 3; ++kx)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(dst + ((ky * 3 + kx) * 4 + q) * 256) =
            make_float4(acc[ky][kx][4 * q], acc[ky][kx][4 * q + 1], acc[ky][kx][4 * q + 2], acc[ky][kx][4 * q + 3]);
}

// Sums the chunks' partials in a fixed order and writes dW.  In a wave's accumulator,
// register r = 4 q + e of lane (half, col) holds output channel 8 q + 4 half + e and input
// channel col, so a (wave, q, half) slice is 4 consecutive output channels x 32 input
// channels: a workgroup takes one such slice over every kz and tap, sums it into LDS as
// [co 4][ci 32][kz][tap] -- 4 contiguous runs of dW -- and writes those with float4 stores.
template <int KD>
__global__ __launch_bounds__(WG_RNT) void conv_wgrad_reduce_kernel(WgArgs a) {
  __shared__ __align__(16) float s_w[4 * WG_CI * KD * 9];
  constexpr int ROW = WG_CI * KD * 9;  // floats of one output channel's run in dW
  const int t = threadIdx.x;
  const int n_ci_blk = a.Ci / WG_CI, n_co_blk = a.Co / WG_CO;
  const int half = blockIdx.x & 1, q = (blockIdx.x >> 1) & 3, wave = (blockIdx.x >> 3) & 3;
  const int tile = blockIdx.x >> 5;
  const int co_blk = tile / n_ci_blk, ci_blk = tile - co_blk * n_ci_blk;
  const int64_t total = (int64_t)a.Co * a.Ci * KD * 9;
  const int tap = t >> 5, col = t & 31;
  const int64_t lane_off = (((int64_t)tap * 4 + q) * 64 + half * 32 + col) * 4;
#pragma unroll
  for (int kz = 0; kz < KD; ++kz) {
    const int64_t unit = ((int64_t)kz * n_co_blk + co_blk) * n_ci_blk + ci_blk;
    const float* src = a.part + (unit * 4 + wave) * WG_UNIT + lane_off;
    float4 s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0;
    int c = 0;
    for (; c + 2 <= a.chunks; c += 2) {
      const float4 v0 = *reinterpret_cast<const float4*>(src + c * total);
      const float4 v1 = *reinterpret_cast<const float4*>(src + (c + 1) * total);
      s0.x += v0.x; s0.y += v0.y; s0.z += v0.z; s0.w += v0.w;
      s1.x += v1.x; s1.y += v1.y; s1.z += v1.z; s1.w += v1.w;
    }
    if (c < a.chunks) {
      const float4 v0 = *reinterpret_cast<const float4*>(src + c * total);
      s0.x += v0.x; s0.y += v0.y; s0.z += v0.z; s0.w += v0.w;
    }
    float* d = s_w + col * (KD * 9) + kz * 9 + tap;
    d[0] = s0.x + s1.x;
    d[ROW] = s0.y + s1.y;
    d[2 * ROW] = s0.z + s1.z;
    d[3 * ROW] = s0.w + s1.w;
  }
  __syncthreads();
  float* out = a.dw + ((int64_t)(co_blk * WG_CO + wave * 32 + q * 8 + half * 4) * a.Ci + ci_blk * WG_CI) * (KD * 9);
#pragma unroll
  for (int i = t; i < ROW; i += WG_RNT) {  // 4 rows of ROW / 4 float4s
    const int row = i / (ROW / 4), v = i - row * (ROW / 4);
    *reinterpret_cast<float4*>(out + (int64_t)row * a.Ci * (KD * 9) + v * 4) =
        *reinterpret_cast<const float4*>(s_w + row * ROW + v * 4);
  }
}

int wgrad_plan(int64_t N, int64_t Ci, int64_t Co, int64_t D, int64_t H, int64_t W, int KD, WgArgs* a) {
  a->N = (int)N; a->Ci = (int)Ci; a->Co = (int)Co; a->D = (int)D; a->H = (int)H; a->W = (int)W;
  a->KD = KD; a->pd = (KD - 1) / 2;
  a->pitch = (int)W + 2 * WG_PAD;
  int slab = WG_R * a->pitch;               // elements; keep the per-channel stride off a multiple
  while (((slab / 2) & 31) != 4) slab += 8;  // of the bank count (ds_read_b128 across 32 channels)
  a->slab = slab;
  a->chunks16 = (int)(WG_CI * WG_R * (W / 8));
  const int64_t groups = std::max<int64_t>(1, (Ci / WG_CI) * (Co / WG_CO) * KD);
  // as many chunks as keep the grid within one round of 512 resident workgroups (2 per CU):
  // a grid just over a multiple of 512 leaves most CUs idle for its last round.  A chunk
  // spans at least 4 stages, so a workgroup's partials (128 x 32 x 9 floats, 147 KB) stay
  // below half of what it reads (88 KB of input and dy rows per stage at W = 64).
  const int64_t stages = N * D * ((H + WG_TY - 1) / WG_TY);
  int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(512 / groups, stages / 4));
  a->stages_per_chunk = (int)((stages + chunks - 1) / chunks);
  a->chunks = (int)((stages + a->stages_per_chunk - 1) / a->stages_per_chunk);
  return ATK_OK;
}

}  // namespace
}  // namespace atk

extern "C" size_t atk_conv_wgrad_workspace_bytes(int64_t N, int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co,
                                                 int KD) {
  using namespace atk;
  if (N <= 0 || Ci <= 0 || Co <= 0 || D <= 0 || H <= 0 || W <= 0 || (KD != 1 && KD != 3)) return 0;
  if (Ci % WG_CI || Co % WG_CO || W % 16 || W > WG_MAXW) return 0;  // shapes the kernel declines
  WgArgs a{};
  wgrad_plan(N, Ci, Co, D, H, W, KD, &a);
  return (size_t)a.chunks * (size_t)Co * (size_t)Ci * (size_t)KD * 9 * sizeof(float);
}

extern "C" int atk_conv_wgrad(const void* x, const void* dy, float* dw, int64_t N, int64_t Ci, int64_t D, int64_t H,
                              int64_t W, int64_t Co, int KD, int dtype, void* workspace, size_t ws_bytes,
                              atk_stream_t stream) {
  using namespace atk;
  if (!x || !dy || !dw) return fail(ATK_EINVAL, "conv_wgrad: null pointer");
  if (dtype != ATK_F16 && dtype != ATK_BF16) return fail(ATK_UNSUPPORTED, "conv_wgrad: 16-bit types only");
  if (N <= 0 || Ci <= 0 || Co <= 0 || D <= 0 || H <= 0 || W <= 0) return fail(ATK_EINVAL, "conv_wgrad: bad sizes");
  if (KD != 1 && KD != 3) return fail(ATK_UNSUPPORTED, "conv_wgrad: kernel depth 1 or 3");
  if (Ci % WG_CI || Co % WG_CO || W % 16 || W > WG_MAXW)
    return fail(ATK_UNSUPPORTED, "conv_wgrad: needs Ci %% 32, Co %% 128, W %% 16 == 0 and W <= 64");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dw)) return fail(ATK_UNSUPPORTED, "conv_wgrad: 16-byte aligned tensors");
  const int64_t xe = N * Ci * D * H * W, ge = N * Co * D * H * W;
  if (xe * 2 >= ((int64_t)1 << 31) || ge * 2 >= ((int64_t)1 << 31))
    return fail(ATK_UNSUPPORTED, "conv_wgrad: tensors over 2 GiB");
  WgArgs a{};
  wgrad_plan(N, Ci, Co, D, H, W, KD, &a);
  if ((int64_t)WG_CI * WG_R * (W / 8) > (int64_t)WG_LD * WG_NT)
    return fail(ATK_UNSUPPORTED, "conv_wgrad: staging map too small for W");
  const size_t need = (size_t)a.chunks * Co * Ci * KD * 9 * sizeof(float);
  if (!workspace || ws_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(ATK_EINVAL, "conv_wgrad: workspace too small or misaligned");
  a.x = x; a.dy = dy; a.dw = dw; a.part = static_cast<float*>(workspace);
  a.x_bytes = (uint32_t)(xe * 2);
  a.dy_bytes = (uint32_t)(ge * 2);
  const size_t lds = (size_t)WG_CI * a.slab * 2;
  if (lds > 64 * 1024) return fail(ATK_UNSUPPORTED, "conv_wgrad: LDS stage too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)((Ci / WG_CI) * (Co / WG_CO)), (unsigned)KD, (unsigned)a.chunks);
  if (dtype == ATK_BF16) hipLaunchKernelGGL((conv_wgrad_kernel<__bf16>), grid, dim3(WG_NT), lds, s, a);
  else hipLaunchKernelGGL((conv_wgrad_kernel<_Float16>), grid, dim3(WG_NT), lds, s, a);
  int rc = check_launch("conv_wgrad_kernel");
  if (rc != ATK_OK) return rc;
  const dim3 rgrid((unsigned)((Co / WG_CO) * (Ci / WG_CI) * 32));
  if (KD == 3) hipLaunchKernelGGL(conv_wgrad_reduce_kernel<3>, rgrid, dim3(WG_RNT), 0, s, a);
  else hipLaunchKernelGGL(conv_wgrad_reduce_kernel<1>, rgrid, dim3(WG_RNT), 0, s, a);
  return check_launch("conv_wgrad_reduce_kernel");
}
