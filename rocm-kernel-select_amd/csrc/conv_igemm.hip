// Dense conv2d/conv3d forward as an implicit GEMM on gfx950 MFMA.
//
//   Y[co, m] = bias[co] + sum_k Wt[co, k] * X_im2col[k, m]
//   m = output position (n, z, y, x), k = (tap, ci), tap = (kd, kh, kw)
//
// The reference's kernel for this op (src/cuda/generated/conv3d_fp16_bm256_bn128_bk32_s2.cu:
// 84-324) is a rocWMMA implicit GEMM with M = positions, N = Co, K = Ci*taps, gathering im2col
// rows from global memory per K step.  This kernel is organised around CDNA4 instead:
//
//  * MFMA v_mfma_f32_32x32x16_{bf16,f16} (fp32 inputs: v_mfma_f32_32x32x2_f32 with four
//    steps per 8-channel block), fp32 accumulation.  Weights are the MFMA A operand (32
//    output channels per fragment) and im2col the B operand (32 positions per fragment), so
//    accumulator lanes hold 32 consecutive positions of one channel: stores are coalesced
//    along x in NCDHW.
//  * The K loop runs over "stages" = (input-channel chunk of CB, kd).  A stage stages the
//    input PATCH its tile needs -- (TY-1)*sh+(KH-1)*dh+1 rows x (TX-1)*sw+(KW-1)*dw+1 columns
//    of one input plane -- into LDS once, channels-last with a 16-byte pad per position
//    (conflict-free ds_read_b128), and every tap (kh, kw) of the stage reads its im2col
//    fragments from that patch: each input element is fetched from memory once per stage
//    instead of once per tap.
//  * Weights are pre-packed (a small kernel, into the workspace) into fragment order
//    [tap][ci-block][co-block32][32 co][KB ci]: a wave's A fragment is one contiguous 1 KB
//    global load, L2-resident across the workgroups that share the output-channel tile.
//  * Split-K over stages for shapes with too few output tiles to fill 256 CUs, with
//    per-split fp32 partials summed in a deterministic finalize kernel.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "conv_common.h"

namespace atk {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct IgArgs {
  const void* x;
  const void* wp;     // packed weights
  const void* bias;
  void* y;
  float* part;        // split-K partials [splits][N*Co*SPo], or null
  int N, Ci, D, H, W, Co, KD, KH, KW, sd, sh, sw, pd, ph, pw, dd, dh, dw, Do, Ho, Wo;
  int TX, TY, tiles_x, tiles_y;
  int PX, PY;
  int NCX;            // 16-byte chunks per patch row (aligned-down start)
  int PXS;            // patch row stride in positions: NCX * VEC, padded against bank conflicts
  int vec_rows;       // input rows are 16-byte aligned (W % VEC == 0, aligned base)
  int patch_elems;    // elements of one patch buffer (two are allocated)
  uint32_t x_sample_bytes;  // bytes of one input sample (buffer range of the patch loads)
  uint32_t wp_bytes;        // bytes of the packed weights
  int n_stages;       // n_cc * KD
  int stages_per_split;
  int n_kb;           // ci k-blocks in the packed weights = n_cc * CB / KB
  int co_blocks;      // 32-row co blocks in the packed weights (multiple of BN / 32)
  // epilogue extras (unsplit launches only)
  const void* resid;  // y += resid (same shape and layout as y), or null
  float4* gn_parts;   // GroupNorm partial records [N * G][gn_np] (count, mean, M2, -), or null
  int gn_cpg;         // channels per GroupNorm group: 4, 8, 16, 32 or a multiple of 32
  int gn_G;           // groups (Co = gn_G * gn_cpg)
  int gn_np;          // records per (n, g)
  int lds_epi;        // unsplit 16-bit output through the LDS-staged epilogue
  int epi_pitch;      // its staging row pitch in bytes (NC[D]HW: BM * 2 + 16; channels-last: BN * 2 + 8)
  // One-pass GroupNorm (+ SiLU) of the output inside the launch (cooperative launch: every
  // workgroup is resident): the records go to tagged slots, one workgroup per (n, g) merges
  // them and publishes (mean, rstd), and every tile is stored normalised from registers.
  int gn_onepass;
  int gn_silu;
  int gn_pdt;                      // dtype code of gamma / beta
  float gn_eps;
  const void* gn_gamma;            // or null (1)
  const void* gn_beta;             // or null (0)
  unsigned long long* gn_slots;    // [N * G][gn_np][3] record words, then [N * G][2] result words
  unsigned int* gn_hdr;            // diagnostics [0], epoch [16], launch counter [32], block counters [64 + 16 b]
  unsigned long long gn_wait_ticks;  // bound of every wait (wall-clock ticks): a hang guard only
};

template <typename T> struct MfmaTraits;
template <> struct MfmaTraits<__bf16> { static constexpr int KB = 16, VEC = 8; };
template <> struct MfmaTraits<_Float16> { static constexpr int KB = 16, VEC = 8; };
template <> struct MfmaTraits<float> { static constexpr int KB = 8, VEC = 4; };

__device__ __forceinline__ void mfma_block(f32x16& acc, const uint4& a, const uint4& b, __bf16*) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8*>(&a),
                                                *reinterpret_cast<const bf16x8*>(&b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma_block(f32x16& acc, const uint4& a, const uint4& b, _Float16*) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const f16x8*>(&a),
                                               *reinterpret_cast<const f16x8*>(&b), acc, 0, 0, 0);
}
// fp32: the lane's 4 consecutive channels feed 4 MFMA steps; step e pairs channels (e, 4+e)
// of the 8-channel block across the two lane halves, identically for A and B.
__device__ __forceinline__ void mfma_block(f32x16& acc, const uint4& a, const uint4& b, float*) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

// Patch staging.  The patch of a stage is CB channels x PY input rows x NCX 16-byte chunks,
// stored channels-last as patch[(py * PXS + px') * CBS + cl] with PXS >= NCX * VEC: position
// px' = chunk * VEC + e holds input column gx0 + px', gx0 being the tile's first needed
// column (ix0) rounded down to a 16-byte boundary, so every chunk is written whole with no
// per-element bounds test; readers add mis = ix0 - gx0.  Chunk c maps to (row-chunk
// rc = c / CB, channel cl = c % CB): consecutive lanes write consecutive channels of one
// patch position.
template <typename T, int CB, bool VR, int NTH = 256, int XC = 1>
struct PatchLoader {
  static constexpr int VEC = 16 / sizeof(T);
  // chunks per thread held for the next stage: CB/4 for 16-bit types, CB/2 for fp32, at 256
  // threads per workgroup (scaled by 256 / NTH for other workgroup sizes), times XC for tiles whose patch
  // has a wide halo (7x7 planes); the host plan rejects tiles whose patch needs more
  static constexpr int MAXC = (sizeof(T) == 2 ? CB / 4 : CB / 2) * XC * 256 / NTH;
  uint4 buf[MAXC];

  // rsrc covers sample n of the input; iz may be out of range (a padding plane)
  // valid == false issues the same loads with out-of-range offsets (they read zero): callers
  // prefetch unconditionally, because a load inside a branch makes the compiler wait for it
  // (and unpack it) inside that branch instead of where the data is used.
  __device__ __forceinline__ void load(const IgArgs& a, __amdgpu_buffer_rsrc_t rx, int cc, int iz, int iy0,
                                       int gx0, int total, int tid, int nt, bool valid = true) {
    const bool zin = valid && (unsigned)iz < (unsigned)a.D;
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
      const int c = tid + u * nt;
      const int cl = c % CB, rc = c / CB;
      const int py = rc / a.NCX, cx = rc - (rc / a.NCX) * a.NCX;
      const int ci = cc * CB + cl, iy = iy0 + py, gx = gx0 + cx * VEC;
      const bool rowok = c < total && zin && ci < a.Ci && (unsigned)iy < (unsigned)a.H;
      const uint32_t row = (uint32_t)((((uint32_t)ci * a.D + iz) * a.H + iy) * a.W);
      if (VR) {
        const bool ok = rowok && gx >= 0 && gx + VEC <= a.W;  // chunks are all-in or all-out
        buf[u] = bload16(rx, ok ? (row + gx) * (uint32_t)sizeof(T) : kOOB, 0);
      } else {
        Vec16<T> v;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int ix = gx + e;
          const bool ok = rowok && (unsigned)ix < (unsigned)a.W;
          v.e[e] = bload_elem<T>(rx, ok ? (row + ix) * (uint32_t)sizeof(T) : kOOB);
        }
        buf[u] = v.raw;
      }
    }
  }

  // Issue the load of chunk u only (same addressing as load()).
  __device__ __forceinline__ void load_one(const IgArgs& a, __amdgpu_buffer_rsrc_t rx, int u, int cc, int iz,
                                           int iy0, int gx0, int total, int tid, int nt, bool valid = true) {
    const bool zin = valid && (unsigned)iz < (unsigned)a.D;
    const int c = tid + u * nt;
    const int cl = c % CB, rc = c / CB;
    const int py = rc / a.NCX, cx = rc - (rc / a.NCX) * a.NCX;
    const int ci = cc * CB + cl, iy = iy0 + py, gx = gx0 + cx * VEC;
    const bool rowok = c < total && zin && ci < a.Ci && (unsigned)iy < (unsigned)a.H;
    const uint32_t row = (uint32_t)((((uint32_t)ci * a.D + iz) * a.H + iy) * a.W);
    if (VR) {
      const bool ok = rowok && gx >= 0 && gx + VEC <= a.W;
      buf[u] = bload16(rx, ok ? (row + gx) * (uint32_t)sizeof(T) : kOOB, 0);
    } else {
      Vec16<T> v;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int ix = gx + e;
        const bool ok = rowok && (unsigned)ix < (unsigned)a.W;
        v.e[e] = bload_elem<T>(rx, ok ? (row + ix) * (uint32_t)sizeof(T) : kOOB);
      }
      buf[u] = v.raw;
    }
  }

  // ---- precomputed quad path (VR only) --------------------------------------------------
  // A thread owns NQ "quads": 4 consecutive channels x one 16-byte row chunk (VEC positions),
  // chunks 4g..4g+3 of buf.  Quad q of the tile is (channel quad cq = q % (CB/4), patch row
  // py, chunk column cx) with py next-fastest after cq: the lanes of one LDS write cycle then
  // cover several patch rows at the same positions, and the host pads the row pitch (PXS) so
  // that those rows fall on disjoint banks.  A quad goes to LDS as one 64-bit (16-bit types)
  // or 128-bit (fp32) store per position -- 4x fewer LDS writes than one per element.  All
  // offsets are fixed for the tile, so a stage only adds a uniform term: no division is
  // left in the stage loop.
  static constexpr int NQ = MAXC / 4;
  uint32_t goff[MAXC];  // element offset in the sample without the stage term (cc*CB*DHW + iz*HW)
  int clim[MAXC];       // channel inside the CB block, or a huge value if outside patch/input
  uint32_t qoff[NQ];    // LDS element offset of the quad's first element

  __device__ __forceinline__ void init(const IgArgs& a, int iy0, int gx0, int total_quads, int tid, int nt) {
    constexpr int CBS = CB + VEC;
#pragma unroll
    for (int g = 0; g < NQ; ++g) {
      const int q = tid + g * nt;
      const int cq = q % (CB / 4), rr = q / (CB / 4);
      const int py = rr % a.PY, cx = rr / a.PY;
      const int iy = iy0 + py, gx = gx0 + cx * VEC;
      const bool ok = q < total_quads && (unsigned)iy < (unsigned)a.H && gx >= 0 && gx + VEC <= a.W;
      qoff[g] = (uint32_t)((py * a.PXS + cx * VEC) * CBS + cq * 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int cl = cq * 4 + k;
        goff[g * 4 + k] = (uint32_t)((cl * a.D * a.H + iy) * a.W + gx);
        clim[g * 4 + k] = ok ? cl : (1 << 30);
      }
    }
  }
  // Stage term and channel limit of stage (cc, iz); valid == false or a padding plane (iz
  // outside [0, D)) gives a limit no chunk passes, so every load reads zero.
  __device__ __forceinline__ static uint32_t stage_off(const IgArgs& a, int cc, int iz) {
    return (uint32_t)((cc * CB * a.D + iz) * a.H * a.W);
  }
  __device__ __forceinline__ static int stage_lim(const IgArgs& a, int cc, int iz, bool valid) {
    return (valid && (unsigned)iz < (unsigned)a.D) ? a.Ci - cc * CB : 0;
  }
  __device__ __forceinline__ void load_fast(__amdgpu_buffer_rsrc_t rx, int u, uint32_t soff_el, int lim) {
    buf[u] = bload16(rx, clim[u] < lim ? (goff[u] + soff_el) * (uint32_t)sizeof(T) : kOOB, 0);
  }
  __device__ __forceinline__ static uint32_t dw(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
  }
  __device__ __forceinline__ void store_quad(T* patch, int g, int total_quads, int tid, int nt) const {
    constexpr int CBS = CB + VEC;
    if (tid + g * nt >= total_quads) return;
    T* dst = patch + qoff[g];
    const uint4 &c0 = buf[4 * g], &c1 = buf[4 * g + 1], &c2 = buf[4 * g + 2], &c3 = buf[4 * g + 3];
    if constexpr (sizeof(T) == 2) {
      // position e of the 4 channels: halves e%2 of dword e/2 of each chunk
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(dw(c1, e >> 1), dw(c0, e >> 1), sel);
        const uint32_t hi = __builtin_amdgcn_perm(dw(c3, e >> 1), dw(c2, e >> 1), sel);
        *reinterpret_cast<uint2*>(dst + e * CBS) = make_uint2(lo, hi);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        *reinterpret_cast<uint4*>(dst + e * CBS) = make_uint4(dw(c0, e), dw(c1, e), dw(c2, e), dw(c3, e));
    }
  }

  __device__ __forceinline__ void store(const IgArgs& a, T* patch, int total, int tid, int nt) const {
    constexpr int CBS = CB + VEC;
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
      const int c = tid + u * nt;
      if (c >= total) break;
      const int cl = c % CB, rc = c / CB;
      const int py = rc / a.NCX, cx = rc - (rc / a.NCX) * a.NCX;
      Vec16<T> v;
      v.raw = buf[u];
      T* dst = patch + (py * a.PXS + cx * VEC) * CBS + cl;
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e * CBS] = v.e[e];
    }
  }
};

// Patch staging from a channels-last input (x[n][z][y][x][ci], NDHWC / NHWC).  A 16-byte
// chunk of memory is 8 consecutive channels of one position, which is exactly the patch's
// LDS layout (patch[(py * PXS + px) * CBS + cl]), so each chunk goes to LDS as one 16-byte
// store with no transposition.  Chunk c of a stage is (position p = c / (CB/8), channel
// octet c % (CB/8)), positions row-major over PY x PX from (iy0, ix0); chunks outside the
// input (padding) read zero.  Same interface as PatchLoader (MAXC chunks per thread, NQ
// groups of four written together), so the tap schedules drive either.  Needs Ci % 8 == 0
// and 16-byte aligned x (host check).  16-bit types only.
template <typename T, int CB, int NTH = 256, int XC = 1>
struct PatchLoaderCL {
  static_assert(sizeof(T) == 2, "channels-last staging is for 16-bit types");
  static constexpr int MAXC = CB / 4 * XC * 256 / NTH;
  static constexpr int NQ = MAXC / 4;
  static constexpr int CO8 = CB / 8;  // chunks per position
  uint4 buf[MAXC];
  uint32_t goff[MAXC];  // element offset in the sample without the stage term
  int clim[MAXC];       // the chunk's first channel inside the CB block, or a huge value
  uint32_t loff[MAXC];  // LDS element offset
  int total;            // chunks of a stage

  __device__ __forceinline__ void init(const IgArgs& a, int iy0, int ix0, int /*total_quads*/, int tid, int nt) {
    constexpr int CBS = CB + 8;
    const int PX = a.PX;
    total = a.PY * PX * CO8;
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
      const int c = tid + u * nt;
      const int p = c / CO8, o8 = c - (c / CO8) * CO8;
      const int py = p / PX, px = p - (p / PX) * PX;
      const int iy = iy0 + py, ix = ix0 + px;
      const bool ok = c < total && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
      goff[u] = ok ? (uint32_t)(((iy * a.W + ix) * a.Ci) + o8 * 8) : 0u;
      clim[u] = ok ? o8 * 8 : (1 << 30);
      loff[u] = (uint32_t)((py * a.PXS + px) * CBS + o8 * 8);
    }
  }
  __device__ __forceinline__ static uint32_t stage_off(const IgArgs& a, int cc, int iz) {
    return (uint32_t)(iz * a.H * a.W * a.Ci + cc * CB);
  }
  __device__ __forceinline__ static int stage_lim(const IgArgs& a, int cc, int iz, bool valid) {
    return (valid && (unsigned)iz < (unsigned)a.D) ? a.Ci - cc * CB : 0;
  }
  __device__ __forceinline__ void load_fast(__amdgpu_buffer_rsrc_t rx, int u, uint32_t soff_el, int lim) {
    buf[u] = bload16(rx, clim[u] < lim ? (goff[u] + soff_el) * (uint32_t)sizeof(T) : kOOB, 0);
  }
  __device__ __forceinline__ void store_quad(T* patch, int g, int /*total_quads*/, int tid, int nt) const {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = 4 * g + k;
      if (tid + u * nt < total) *reinterpret_cast<uint4*>(patch + loff[u]) = buf[u];
    }
  }
};

template <typename T, int CB, bool VR, int NTH, int XC, bool CL>
struct LoaderSel {
  using type = PatchLoader<T, CB, VR, NTH, XC>;
};
template <typename T, int CB, bool VR, int NTH, int XC>
struct LoaderSel<T, CB, VR, NTH, XC, true> {
  using type = PatchLoaderCL<T, CB, NTH, XC>;
};

// Bias of the workgroup's BN output channels as fp32 in LDS (zero without bias or when
// writing split-K partials), staged before the main loop: read per element in the epilogue
// from global memory, every element would wait for its own load.
template <typename T, int BN, int NT>
__device__ __forceinline__ void stage_bias(const IgArgs& a, int co_tile, float* s_bias) {
  const T* __restrict__ bias = static_cast<const T*>(a.bias);
  for (int i = threadIdx.x; i < BN; i += NT) {
    const int co = co_tile * BN + i;
    s_bias[i] = (bias && !a.part && co < a.Co) ? to_f32(bias[co]) : 0.f;
  }
}

// GroupNorm statistics of the values a wave stores (an unsplit launch): one (count, mean, M2)
// record per (wave tile, group) -- per 32-channel block and group for groups of up to 32
// channels, per block for wider groups -- so the merge in the apply kernel is exact.  A lane
// holds, for block i and position column j, the channels (r >> 2) * 8 + half * 4 + (r & 3),
// r = 0..15: its 4 channels of octet q = r >> 2 always lie in one group (cpg >= 8) or are the
// group (cpg == 4).  While the values are stored, each lane keeps per (block, octet) the sums
// of d = v - K and d^2 about K = its first value of that octet (n <= 16 values, so the shifted
// one-pass M2 = sum d^2 - (sum d)^2 / n is exact to rounding); nothing else stays live, so
// the epilogue adds little register pressure to the kernel.  The lanes are then merged per
// group: mean = sum n_l mean_l / n, M2 = sum (M2_l + n_l (mean_l - mean)^2).
template <int FCO>
struct GnLaneStats {
  float K[FCO][4], s1[FCO][4], s2[FCO][4];
};

template <int FCO, int FSP, int BN>
__device__ __forceinline__ void tile_gn_records(const IgArgs& a, const GnLaneStats<FCO>& st, float nl, int n,
                                                int co_tile, int sp_rec, int wco, int half) {
  const int cpg = a.gn_cpg;
  const int lane = threadIdx.x & 63;
  // values this wave stored: lanes 0-31 cover the columns once, nl of them each
  const float npos = wave_sum(lane < 32 ? nl : 0.f);
  const int per_blk = cpg >= 32 ? 1 : 32 / cpg;  // records (groups) per 32-channel block
  const int oct = cpg >= 32 ? 4 : (cpg >= 8 ? cpg / 8 : 1);
  const float cnt = npos * (float)(cpg >= 32 ? 32 : cpg);
  const float nq = 4.f * nl;  // values per (lane, octet)
  // sum over a group's lanes: 64 lanes, or one half (cpg == 4; xor offsets below 32 stay
  // within a half)
  auto group_sum = [&](float x) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) x += __shfl_xor(x, off, 64);
    if (cpg != 4) x += __shfl_xor(x, 32, 64);
    return x;
  };
#pragma unroll
  for (int i = 0; i < FCO; ++i) {
    const int cblk = co_tile * BN + (wco * FCO + i) * 32;  // first channel of the block
    if (cblk >= a.gn_G * cpg) continue;
    float mq[4], m2q[4];  // the lane's mean and M2 per octet
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float t = nq > 0.f ? st.s1[i][q] / nq : 0.f;
      mq[q] = st.K[i][q] + t;
      m2q[q] = fmaxf(fmaf(-st.s1[i][q], t, st.s2[i][q]), 0.f);
    }
    for (int k = 0; k < per_blk && k < 8; ++k) {  // group k of the block (cpg == 4: k = 2q + half)
      const int q0 = cpg == 4 ? k >> 1 : k * oct;
      const bool mine = cpg != 4 || (k & 1) == half;
      float sm = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sm += (mine && q >= q0 && q < q0 + oct) ? nq * mq[q] : 0.f;
      const float mean = cnt > 0.f ? group_sum(sm) / cnt : 0.f;
      float m2 = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float d = mq[q] - mean;
        m2 += (mine && q >= q0 && q < q0 + oct) ? m2q[q] + nq * d * d : 0.f;
      }
      m2 = group_sum(m2);
      const int g = (cblk + k * (cpg >= 32 ? 0 : cpg)) / cpg;
      const bool writer = cpg == 4 ? lane == ((k & 1) ? 32 : 0) : lane == 0;
      if (writer && g < a.gn_G) {
        const int part = cpg > 32 ? (cblk % cpg) / 32 : 0;
        const int rec = sp_rec * (cpg > 32 ? cpg / 32 : 1) + part;
        // every record the layout reserves is written -- a wave whose tile lies past the
        // output's edge writes a zero-count record, which the merge weighs by its count 0
        a.gn_parts[((int64_t)n * a.gn_G + g) * a.gn_np + rec] = make_float4(cnt, mean, m2, 0.f);
      }
    }
  }
}

// Epilogue: accumulator rows = output channels, columns = positions.  Writes y (bias and the
// optional residual added, converted) or, under split-K, this split's fp32 partial sums; on an
// unsplit launch with gn_parts set it also writes the GroupNorm records of the stored values.
template <typename T, int FCO, int FSP, int BN, bool EPI, bool CL = false>
__device__ __forceinline__ void store_tile(const IgArgs& a, f32x16 (&acc)[FCO][FSP], const float* s_bias,
                                           int n, int co_tile, int split, int oz, int oy0, int ox0, int wco,
                                           int wsp, int half, int col, int sp_rec) {
  const int64_t spo = (int64_t)a.Do * a.Ho * a.Wo;
  if constexpr (CL) {
    // channels-last output y[n][sp][co]: a lane's 4 consecutive channels (r & 3) of one
    // position go out as one 8-byte store (fp32 partials: one 16-byte store); Co % 8 == 0
#pragma unroll
    for (int j = 0; j < FSP; ++j) {
      const int m = (wsp * FSP + j) * 32 + col;
      const int ty = m / a.TX, tx = m - (m / a.TX) * a.TX;
      const int oy = oy0 + ty, ox = ox0 + tx;
      if (oy >= a.Ho || ox >= a.Wo) continue;
      const int64_t base = ((int64_t)n * spo + ((int64_t)oz * a.Ho + oy) * a.Wo + ox) * a.Co;
#pragma unroll
      for (int i = 0; i < FCO; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int cl = (wco * FCO + i) * 32 + q * 8 + half * 4;
          const int co = co_tile * BN + cl;
          if (co >= a.Co) continue;
          if (a.part) {
            *reinterpret_cast<float4*>(a.part + (int64_t)split * a.N * a.Co * spo + base + co) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          } else {
            float v[8] = {acc[i][j][4 * q] + s_bias[cl], acc[i][j][4 * q + 1] + s_bias[cl + 1],
                          acc[i][j][4 * q + 2] + s_bias[cl + 2], acc[i][j][4 * q + 3] + s_bias[cl + 3],
                          0.f, 0.f, 0.f, 0.f};
            const uint4 pk = pack16<T>(v);
            *reinterpret_cast<uint2*>(static_cast<T*>(a.y) + base + co) = make_uint2(pk.x, pk.y);
          }
        }
      }
    }
    return;
  }
  if constexpr (EPI) {
    // opaque copies of the lane coordinates: the address math below then cannot be hoisted
    // above the main loop, where its results would stay live (and cost registers) throughout
    int colx = col, halfx = half;
    asm volatile("" : "+v"(colx), "+v"(halfx));
    GnLaneStats<FCO> st;
    float nl = 0.f;  // positions this lane stores (per channel)
#pragma unroll
    for (int j = 0; j < FSP; ++j) {
      const int m = (wsp * FSP + j) * 32 + colx;
      const int ty = m / a.TX, tx = m - (m / a.TX) * a.TX;
      const int oy = oy0 + ty, ox = ox0 + tx;
      const bool okj = oy < a.Ho && ox < a.Wo;
      nl += okj ? 1.f : 0.f;
      const int64_t sp = okj ? ((int64_t)oz * a.Ho + oy) * a.Wo + ox : 0;
#pragma unroll
      for (int i = 0; i < FCO; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int cl = (wco * FCO + i) * 32 + (r >> 2) * 8 + halfx * 4 + (r & 3);
          const int co = co_tile * BN + cl;
          const bool in = okj && co < a.Co;
          const int64_t o = ((int64_t)n * a.Co + (in ? co : 0)) * spo + sp;
          float v = acc[i][j][r] + s_bias[cl];
          if (a.resid && in) v += to_f32(static_cast<const T*>(a.resid)[o]);
          const T t = from_f32<T>(v);
          if (in) static_cast<T*>(a.y)[o] = t;
          // running shifted sums of the stored value (shift: the octet's value at j = 0, r = 4q)
          const int q = r >> 2;
          const float sv = okj ? to_f32(t) : 0.f;
          if (j == 0 && (r & 3) == 0) {
            st.K[i][q] = sv;
            st.s1[i][q] = 0.f;
            st.s2[i][q] = 0.f;
          }
          const float d = okj ? sv - st.K[i][q] : 0.f;
          st.s1[i][q] += d;
          st.s2[i][q] = fmaf(d, d, st.s2[i][q]);
        }
      }
    }
    if (a.gn_parts) tile_gn_records<FCO, FSP, BN>(a, st, nl, n, co_tile, sp_rec, wco, halfx);
    return;
  }
#pragma unroll
  for (int j = 0; j < FSP; ++j) {
    const int m = (wsp * FSP + j) * 32 + col;
    const int ty = m / a.TX, tx = m - (m / a.TX) * a.TX;
    const int oy = oy0 + ty, ox = ox0 + tx;
    if (oy >= a.Ho || ox >= a.Wo) continue;
    const int64_t sp = ((int64_t)oz * a.Ho + oy) * a.Wo + ox;
#pragma unroll
    for (int i = 0; i < FCO; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int cl = (wco * FCO + i) * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
        const int co = co_tile * BN + cl;
        if (co >= a.Co) continue;
        const int64_t o = ((int64_t)n * a.Co + co) * spo + sp;
        if (a.part) {
          a.part[(int64_t)split * a.N * a.Co * spo + o] = acc[i][j][r];
        } else {
          static_cast<T*>(a.y)[o] = from_f32<T>(acc[i][j][r] + s_bias[cl]);
        }
      }
    }
  }
}

// Tagged words of the one-pass GroupNorm exchange: the launch's tag in the high half, a
// float's bits in the low half, each one 64-bit agent-scope store or load, so a word read with
// the current tag is whole and current without a fence.
__device__ __forceinline__ void gn_put(unsigned long long* p, uint32_t tag, float v) {
  __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool gn_get(unsigned long long* p, uint32_t tag, float& v) {
  const unsigned long long w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __uint_as_float((uint32_t)w);
  return (uint32_t)(w >> 32) == tag;
}

// One-pass GroupNorm (+SiLU), after this workgroup has published its records (every record
// slot (n, g, tile, wave share < span, part) of the launch is written by exactly one wave):
//  1. workgroup j (linear index) merges the records of (n, g) = j, j + nwg, ..., one group per
//     wave: records read once into registers, counted merge in record order with DPP wave sums
//     (mean = sum c_i m_i / n, M2 = sum (M2_i + c_i (m_i - mean)^2)), then (mean, rstd) published;
//  2. every workgroup polls the results of the groups its channel tile touches into LDS;
//  3. the runs, held in registers since the statistics were taken, are normalised (+SiLU) and
//     stored -- y is written once, normalised;
//  4. the last workgroup to finish advances the epoch in the header (a counter per 64
//     workgroups, then a launch counter, each reset by the workgroup that completes it), so no
//     slot is ever cleared and a replayed graph sees fresh tags.
// The host launches this cooperatively (every workgroup resident), so every record arrives.
// Each wait is still bounded by a.gn_wait_ticks -- a guard against a hang, not a fallback: a
// wait that runs out sets the header's diagnostics word and the launch's output is invalid.
template <typename T, int BN, int RPR, int NRUN, int NTHR, int WSP>
__device__ __forceinline__ void gn_onepass_finish(const IgArgs& a, const uint4 (&keep)[NRUN], int n, int co_tile,
                                                  int oz, int oy0, int ox0, int q0, int lane, int tid, int span,
                                                  uint32_t tag) {
  constexpr int NW = NTHR / 64, RC = 4;
  __shared__ float2 s_mr[BN / 4];  // (mean, rstd) of the groups of this channel tile
  const int cpg = a.gn_cpg, G = a.gn_G, np = a.gn_np;
  const int parts = cpg > 32 ? cpg / 32 : 1;
  const int64_t spo = (int64_t)a.Do * a.Ho * a.Wo;
  const int txs = __builtin_ctz((unsigned)a.TX);
  // this thread's runs and their affine parameters, loaded before any wait
  float gm[NRUN], bt[NRUN];
#pragma unroll
  for (int k = 0; k < NRUN; ++k) {
    const int co = min(co_tile * BN + (q0 + 64 * k + lane) / RPR, a.Co - 1);
    gm[k] = a.gn_gamma ? load_param(a.gn_gamma, a.gn_pdt, co) : 1.f;
    bt[k] = a.gn_beta ? load_param(a.gn_beta, a.gn_pdt, co) : 0.f;
  }
  const int nwg = gridDim.x * gridDim.y;  // (unsplit: gridDim.z == 1)
  const int wg = blockIdx.x + gridDim.x * blockIdx.y;
  const uint64_t deadline = wall_clock64() + a.gn_wait_ticks;
  bool late = false;
  unsigned long long* res = a.gn_slots + (int64_t)a.N * G * np * 3;  // result words
  // 1. merges
  for (int j = wg + nwg * (tid >> 6); j < a.N * G; j += nwg * NW) {
    unsigned long long* rs = a.gn_slots + (int64_t)j * np * 3;
    auto live = [&](int r) { return r < np && (r / parts) % WSP < span; };
    float c[RC], mu[RC], q2[RC];
    bool have[RC];
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      c[i] = mu[i] = q2[i] = 0.f;
      have[i] = !live(lane + 64 * i);
    }
    while (true) {
      bool all = true;
#pragma unroll
      for (int i = 0; i < RC; ++i) {
        if (have[i]) continue;
        unsigned long long* w = rs + (int64_t)(lane + 64 * i) * 3;
        float x0, x1, x2;
        const bool o0 = gn_get(w, tag, x0), o1 = gn_get(w + 1, tag, x1), o2 = gn_get(w + 2, tag, x2);
        if (o0 && o1 && o2) {
          have[i] = true;
          c[i] = x0;
          mu[i] = x1;
          q2[i] = x2;
        }
        all = all && have[i];
      }
      if (all) break;
      if (wall_clock64() > deadline) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    float sn = 0.f, sm = 0.f;
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      sn += c[i];
      sm = fmaf(c[i], mu[i], sm);
    }
    // records past 64 * RC (large grids): polled one at a time, read again below
    for (int r = lane + 64 * RC; r < np; r += 64) {
      if (!live(r)) continue;
      float x0 = 0.f, x1 = 0.f, x2;
      while (!(gn_get(rs + (int64_t)r * 3, tag, x0) && gn_get(rs + (int64_t)r * 3 + 1, tag, x1) &&
               gn_get(rs + (int64_t)r * 3 + 2, tag, x2))) {
        if (wall_clock64() > deadline) {
          late = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      sn += x0;
      sm = fmaf(x0, x1, sm);
    }
    const float cnt = wave_sum_rows(sn);
    const float mean = wave_sum_rows(sm) / cnt;
    float m2 = 0.f;
#pragma unroll
    for (int i = 0; i < RC; ++i) {
      const float d = mu[i] - mean;
      m2 += q2[i] + c[i] * d * d;
    }
    for (int r = lane + 64 * RC; r < np; r += 64) {
      if (!live(r)) continue;
      float x0, x1, x2;
      gn_get(rs + (int64_t)r * 3, tag, x0);
      gn_get(rs + (int64_t)r * 3 + 1, tag, x1);
      gn_get(rs + (int64_t)r * 3 + 2, tag, x2);
      const float d = x1 - mean;
      m2 += x2 + x0 * d * d;
    }
    const float var = wave_sum_rows(m2) / cnt;
    if (lane == 0) {
      gn_put(res + 2 * (int64_t)j, tag, mean);
      gn_put(res + 2 * (int64_t)j + 1, tag, 1.0f / sqrtf(var + a.gn_eps));
    }
  }
  // 2. the results this tile needs
  const int g0 = (co_tile * BN) / cpg;
  const int ng = min(G, ((co_tile + 1) * BN + cpg - 1) / cpg) - g0;
  for (int t = tid; t < ng; t += NTHR) {
    unsigned long long* w = res + 2 * ((int64_t)n * G + g0 + t);
    float mean = 0.f, rstd = 0.f;
    while (true) {
      const bool o0 = gn_get(w, tag, mean), o1 = gn_get(w + 1, tag, rstd);
      if (o0 && o1) break;
      if (wall_clock64() > deadline) {
        late = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    s_mr[t] = make_float2(mean, rstd);
  }
  if (late) __hip_atomic_store(a.gn_hdr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  // 3. normalise and store
  auto finish = [&](auto silu) {
#pragma unroll
    for (int k = 0; k < NRUN; ++k) {
      const int q = q0 + 64 * k + lane;
      const int cl = q / RPR, m = (q - (q / RPR) * RPR) * 8;
      const int oy = oy0 + (m >> txs), ox = ox0 + (m & (a.TX - 1));
      const int co = co_tile * BN + cl;
      const bool ok = oy < a.Ho && ox < a.Wo && co < a.Co;
      const float2 st = s_mr[ok ? co / cpg - g0 : 0];
      const float sc = st.y * gm[k], sh = bt[k] - st.x * sc;
      Vec16<T> iv;
      iv.raw = keep[k];
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        f[e] = fmaf(to_f32(iv.e[e]), sc, sh);
        if constexpr (decltype(silu)::value) f[e] = silu_f32(f[e]);
      }
      if (ok)
        *reinterpret_cast<uint4*>(static_cast<T*>(a.y) + ((int64_t)n * a.Co + co) * spo +
                                  ((int64_t)oz * a.Ho + oy) * a.Wo + ox) = pack16<T>(f);
    }
  };
  if (a.gn_silu) finish(std::true_type());
  else finish(std::false_type());
  // 4. epoch
  if (tid == 0) {
    const int nb = (nwg + 63) / 64, b = wg / 64, in_b = min(64, nwg - b * 64);
    unsigned int* bc = a.gn_hdr + 64 + 16 * b;
    if (__hip_atomic_fetch_add(bc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)in_b - 1) {
      __hip_atomic_store(bc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(a.gn_hdr + 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          (unsigned)nb - 1) {
        __hip_atomic_store(a.gn_hdr + 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.gn_hdr + 16, ((tag >> 1) + 1u) & 0x7fffffffu, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Channels-last output (y[n][position][co], bias added, 16-bit, unsplit) through LDS.  Stored
// straight from the accumulators, a lane's 4 consecutive channels of one position are one 8-byte
// store, and the 64 lanes of a store instruction hit 64 positions Co * 2 bytes apart: partial
// lines everywhere.  Here the tile goes to LDS as [position][channel] rows (pitch
// a.epi_pitch = BN * 2 + 8, so the 32 positions of a write land on distinct bank pairs), each
// lane's 4 channels as one 8-byte write; then consecutive threads store consecutive 16-byte runs
// of 8 channels of one position -- BN * 2 contiguous bytes per position.  Needs Co % 8 == 0 and a
// 16-byte aligned y (host check).  Every thread of the workgroup calls this after a barrier that
// ends the last read of the stage buffers (`active`: the K group holding the sums).
template <typename T, int FCO, int FSP, int BN, int BM, int WSP, int NTHR>
__device__ __forceinline__ void store_tile_lds_cl(const IgArgs& a, f32x16 (&acc)[FCO][FSP], const float* s_bias,
                                                  char* stg, int n, int co_tile, int oz, int oy0, int ox0, int wco,
                                                  int wsp, bool active, int tid) {
  static_assert(sizeof(T) == 2, "16-bit outputs");
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));  // keep the address math below the main loop
  const int half = lane >> 5, col = lane & 31;
  const int EP = a.epi_pitch;
  if (active) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < FCO; ++i)
#pragma unroll
      for (int j = 0; j < FSP; ++j) {
        const int m = (wsp * FSP + j) * 32 + col;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int cl = (wco * FCO + i) * 32 + q * 8 + half * 4;
          const f2 lo = {acc[i][j][4 * q] + s_bias[cl], acc[i][j][4 * q + 1] + s_bias[cl + 1]};
          const f2 hi = {acc[i][j][4 * q + 2] + s_bias[cl + 2], acc[i][j][4 * q + 3] + s_bias[cl + 3]};
          *reinterpret_cast<uint2*>(stg + m * EP + cl * 2) =
              make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, t2)),
                         __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, t2)));
        }
      }
  }
  __syncthreads();
  const int64_t spo = (int64_t)a.Do * a.Ho * a.Wo;
  const int txs = __builtin_ctz((unsigned)a.TX);  // (TX is a power of two)
  constexpr int RPP = BN / 8;  // 16-byte runs per position
  constexpr int NRUN = (BM * RPP + NTHR - 1) / NTHR, RB = NRUN < 8 ? NRUN : 8;
#pragma unroll
  for (int k0 = 0; k0 < NRUN; k0 += RB) {
    int64_t off[RB];
    bool ok[RB];
    uint4 v[RB];
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int q = tid + (k0 + k) * NTHR;
      const int m = q / RPP, c8 = q - (q / RPP) * RPP;
      const int oy = oy0 + (m >> txs), ox = ox0 + (m & (a.TX - 1));
      const int co = co_tile * BN + c8 * 8;
      ok[k] = k0 + k < NRUN && q < BM * RPP && oy < a.Ho && ox < a.Wo && co < a.Co;
      off[k] = ((int64_t)n * spo + ((int64_t)oz * a.Ho + (ok[k] ? oy : 0)) * a.Wo + (ok[k] ? ox : 0)) * a.Co +
               (ok[k] ? co : 0);
      // (rows are 8-byte aligned: two 8-byte reads)
      const char* sp = stg + (ok[k] ? m : 0) * EP + (ok[k] ? c8 : 0) * 16;
      const uint2 lo = *reinterpret_cast<const uint2*>(sp), hi = *reinterpret_cast<const uint2*>(sp + 8);
      v[k] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
#pragma unroll
    for (int k = 0; k < RB; ++k)
      if (ok[k]) *reinterpret_cast<uint4*>(static_cast<T*>(a.y) + off[k]) = v[k];
  }
}

// Output (bias added, 16-bit, NC[D]HW, unsplit) through LDS.  Stored straight from the
// accumulators, every value is its own 2-byte store (a lane holds one position of 16 channels
// per block), so a wave issues FCO * FSP * 16 store instructions, each moving 128 bytes; at the
// end of a launch whose workgroups all finish together those stores are what the chip waits
// for.  Here the tile goes to LDS as [channel][position] rows (pitch a.epi_pitch = BM * 2 + 16:
// the two lane halves' rows, 4 channels apart, fall on disjoint banks), then every thread of
// the workgroup stores 16-byte runs of 8 positions of one channel.  Needs TX % 8 == 0,
// Wo % 8 == 0 and 16-byte aligned y / residual (host check), so a run is whole inside or
// outside the output and aligned.  The caller has passed a barrier after the last read of the
// stage buffers; every thread of the workgroup calls this (the K groups of a split workgroup
// too: `active` is false for the ones whose accumulators were already handed over).
//
// With EPI, the residual is added to each run before its store (the staged value is the
// conv output rounded to T; residual added in fp32, rounded again -- the stock composition of
// a conv followed by an add), and GroupNorm records of the stored values are written: per
// 32-channel block and group (groups of up to 32 channels) or per block (wider groups), in the
// WSP per-tile slots that gn_records() counts (one record per wave holding a share of the
// unit, count-0 records in the rest); each a shifted one-pass mean / M2 of the unit's values
// inside the output, summed per lane as they are stored.
template <typename T, int FCO, int FSP, int BN, int BM, int WSP, bool EPI, int NTHR>
__device__ __forceinline__ void store_tile_lds(const IgArgs& a, f32x16 (&acc)[FCO][FSP], const float* s_bias,
                                               char* stg, int n, int co_tile, int oz, int oy0, int ox0, int wco,
                                               int wsp, bool active, int tid, int tile_rec, uint32_t gn_tag) {
  static_assert(sizeof(T) == 2, "16-bit outputs");
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));  // keep the address math below the main loop
  const int half = lane >> 5, col = lane & 31;
  const int EP = a.epi_pitch;
  if (active) {
#pragma unroll
    for (int i = 0; i < FCO; ++i)
#pragma unroll
      for (int j = 0; j < FSP; ++j) {
        const int m = (wsp * FSP + j) * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int cl = (wco * FCO + i) * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          *reinterpret_cast<T*>(stg + cl * EP + m * 2) = from_f32<T>(acc[i][j][r] + s_bias[cl]);
        }
      }
  }
  __syncthreads();
  const int64_t spo = (int64_t)a.Do * a.Ho * a.Wo;
  constexpr int RPR = BM / 8;  // 16-byte runs per channel row
  // (EXACT: every thread stores the same number of runs; otherwise -- workgroups of 3 K groups
  // -- run q of store k is tid + k * NTHR and the register statistics are off)
  constexpr bool EXACT = (BN * RPR) % NTHR == 0;
  constexpr int NRUN = (BN * RPR + NTHR - 1) / NTHR, RB = NRUN < 8 ? NRUN : 8;
  const bool resid = EPI && a.resid;
  // Wave w stores runs [w, w + 1) * NRUN * 64, store k of a lane being run q0 + 64 k + lane
  // (64 consecutive runs per instruction: whole channel rows or one part of a row), in batches
  // of RB: every residual load of a batch is issued, then every value is formed, then every
  // store is issued.  (On this ISA stores and loads share one counter: a store between two
  // waited-for loads would make each wait cover the store too, serialising the batch on store
  // latency.)
  const int q0 = (tid >> 6) * NRUN * 64;
  // GroupNorm records from registers.  A unit (a group inside a 32-channel block, or a
  // 32-channel part of a wider group) is uch channels, urun = uch * RPR runs.  When urun is a
  // multiple of 64 every store instruction lies inside one unit, so each lane keeps one pair of
  // shifted sums per instruction, about a wave-uniform K (the first staged value of the unit's
  // runs in this wave), and the wave reduces them per unit on the VALU.  A unit longer than a
  // wave's runs spans S <= WSP waves, each writing one of the tile's WSP record slots.  Other
  // layouts take the LDS pass at the end.
  // (With gn_onepass the values stay in registers until the group statistics are known, and
  // the host has checked that the records come from registers.)
  const int cpg = a.gn_cpg;
  const int uch = cpg >= 32 ? 32 : cpg;
  const int urun = uch * RPR;
  const bool onepass = EPI && a.gn_onepass;
  const bool gn = EPI && (a.gn_parts || onepass);
  const bool gn_reg = EXACT && gn && urun % 64 == 0 && (urun <= NRUN * 64 || urun / (NRUN * 64) <= WSP);
  const int txs = __builtin_ctz((unsigned)a.TX);  // (TX is a power of two)
  uint4 keep[NRUN];
  const int ush = gn_reg ? __builtin_ctz((unsigned)urun) : 0;
  float s1[NRUN], s2[NRUN], kk[NRUN];
#pragma unroll
  for (int k = 0; k < NRUN; ++k) {
    s1[k] = s2[k] = kk[k] = 0.f;
    if (gn_reg) {
      const int ps = max(((q0 + 64 * k) >> ush) << ush, q0);  // first run of the unit in this wave
      kk[k] = to_f32(*reinterpret_cast<const T*>(stg + (ps / RPR) * EP));
    }
  }
#pragma unroll
  for (int k0 = 0; k0 < NRUN; k0 += RB) {
    int64_t off[RB];
    bool ok[RB];
    uint4 v[RB];
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int q = EXACT ? q0 + 64 * (k0 + k) + lane : tid + (k0 + k) * NTHR;
      const int cl = q / RPR, m = (q - (q / RPR) * RPR) * 8;
      const int oy = oy0 + (m >> txs), ox = ox0 + (m & (a.TX - 1));
      const int co = co_tile * BN + cl;
      ok[k] = k0 + k < NRUN && q < BN * RPR && oy < a.Ho && ox < a.Wo && co < a.Co;
      off[k] = ((int64_t)n * a.Co + (ok[k] ? co : 0)) * spo + ((int64_t)oz * a.Ho + (ok[k] ? oy : 0)) * a.Wo +
               (ok[k] ? ox : 0);
      // (out-of-range runs load element 0 of their plane, which exists, and discard it)
      if (resid) v[k] = *reinterpret_cast<const uint4*>(static_cast<const T*>(a.resid) + off[k]);
    }
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int q = EXACT ? q0 + 64 * (k0 + k) + lane : tid + (k0 + k) * NTHR;
      const int cl = ok[k] ? q / RPR : 0, m = ok[k] ? (q - (q / RPR) * RPR) * 8 : 0;
      uint4* sp = reinterpret_cast<uint4*>(stg + cl * EP + m * 2);
      const uint4 c = *sp;
      if (resid) {
        Vec16<T> cv, r;
        cv.raw = c;
        r.raw = v[k];
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = to_f32(cv.e[e]) + to_f32(r.e[e]);
        v[k] = pack16<T>(f);
        // (the LDS statistics pass reads the stored values back from the staging rows)
        if (gn && !gn_reg && ok[k]) *sp = v[k];
      } else {
        v[k] = c;
      }
      if (gn_reg) {  // the statistics are of the stored values
        Vec16<T> sv;
        sv.raw = v[k];
        float t1 = 0.f, t2 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = to_f32(sv.e[e]) - kk[k0 + k];
          t1 += d;
          t2 = fmaf(d, d, t2);
        }
        s1[k0 + k] = ok[k] ? t1 : 0.f;
        s2[k0 + k] = ok[k] ? t2 : 0.f;
      }
      keep[k0 + k] = v[k];
    }
#pragma unroll
    for (int k = 0; k < RB; ++k)
      if (ok[k] && !onepass) *reinterpret_cast<uint4*>(static_cast<T*>(a.y) + off[k]) = v[k];
  }
  if (gn_reg) {
    // stores k of one unit: KPU = min(urun / 64, NRUN) consecutive ones, from a multiple of
    // KPU; pairwise sums in a fixed tree leave each unit's lane sums at its first store
    const int kpu = min(urun >> 6, NRUN);
#pragma unroll
    for (int w = 1; w < NRUN; w *= 2)
#pragma unroll
      for (int k = 0; k + w < NRUN; k += 2 * w) {
        const bool take = 2 * w <= kpu;
        s1[k] = take ? s1[k] + s1[k + w] : s1[k];
        s2[k] = take ? s2[k] + s2[k + w] : s2[k];
      }
    const int vy = min(BM / a.TX, a.Ho - oy0), vx = min(a.TX, a.Wo - ox0);
    const int parts = cpg > 32 ? cpg / 32 : 1;
    const int span = urun > NRUN * 64 ? urun / (NRUN * 64) : 1;  // waves per unit
#pragma unroll
    for (int k = 0; k < NRUN; ++k) {
      if (k % kpu) continue;  // (wave-uniform)
      const float w1 = wave_sum_rows(s1[k]), w2 = wave_sum_rows(s2[k]);
      const int qk = q0 + 64 * k;
      const int us = (qk >> ush) << ush, ps = max(us, q0);
      const int co0 = co_tile * BN + ps / RPR;
      const int nvch = min(min(urun, NRUN * 64) / RPR, a.Co - co0);
      if (nvch <= 0 || lane != 0) continue;
      const float cnt = (float)(vy * vx * nvch);
      const float t = w1 / cnt;
      const int g = co0 / cpg, part = cpg > 32 ? (co0 % cpg) / 32 : 0;
      const int pw = (ps - us) / (NRUN * 64);  // this wave's share of the unit
      const int64_t rec = ((int64_t)n * a.gn_G + g) * a.gn_np + (tile_rec * WSP + pw) * parts + part;
      const float mean = kk[k] + t, m2 = fmaxf(fmaf(-w1, t, w2), 0.f);
      if (onepass) {
        // (slots with pw >= span are never written and never read)
        gn_put(a.gn_slots + rec * 3, gn_tag, cnt);
        gn_put(a.gn_slots + rec * 3 + 1, gn_tag, mean);
        gn_put(a.gn_slots + rec * 3 + 2, gn_tag, m2);
        continue;
      }
      float4* recs = a.gn_parts + ((int64_t)n * a.gn_G + g) * a.gn_np;
      recs[(tile_rec * WSP + pw) * parts + part] = make_float4(cnt, mean, m2, 0.f);
      if (pw == 0)  // the slots no wave of this unit fills hold count 0
        for (int w = span; w < WSP; ++w) recs[(tile_rec * WSP + w) * parts + part] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (onepass)
      gn_onepass_finish<T, BN, RPR, NRUN, NTHR, WSP>(a, keep, n, co_tile, oz, oy0, ox0, q0, lane, tid, span, gn_tag);
    return;
  }
  if (!gn) return;
  if (resid) __syncthreads();
  // GroupNorm records: unit u = (32-channel block, group inside it) of this tile, one wave per
  // unit.  One pass over the staged values with sums shifted by the unit's first value K (the
  // tile's first position always lies inside the output): mean = K + s1 / n, M2 = s2 - s1^2 / n,
  // exact to rounding for values that spread over a few standard deviations.  A lane's runs
  // are all read before any is used; the count follows from the tile's extent inside the
  // output.  (TX is a power of two: positions split by shift and mask.)
  const int upb = cpg >= 32 ? 1 : 32 / cpg;  // units per block
  const int nunits = (BN / 32) * upb;
  constexpr int NW = NTHR / 64, MAXR = (32 * RPR + 63) / 64;  // runs per lane for a 32-channel unit
  const int wave = tid >> 6;
  const int txm = a.TX - 1;
  const int vy = min(BM / a.TX, a.Ho - oy0), vx = min(a.TX, a.Wo - ox0);
  const int nruns = uch * RPR, nri = (nruns + 63) / 64;  // runs of the unit, runs per lane
  for (int u = wave; u < nunits; u += NW) {
    const int c0 = (u / upb) * 32 + (u - (u / upb) * upb) * uch;  // first channel (tile-local)
    const int co0 = co_tile * BN + c0;
    const int nvch = min(uch, a.Co - co0);
    if (nvch <= 0) continue;
    const float cnt = (float)(vy * vx * nvch);
    const float K = to_f32(*reinterpret_cast<const T*>(stg + c0 * EP));
    Vec16<T> v[MAXR];
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      if (i < nri) {
        const int r = lane + 64 * i;
        const int rr = r < nruns ? r : 0;
        v[i].raw = *reinterpret_cast<const uint4*>(stg + (c0 + rr / RPR) * EP + (rr % RPR) * 16);
      }
    }
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      if (i < nri) {
        const int r = lane + 64 * i;
        const int m = (r % RPR) * 8;
        const bool ok = r < nruns && ((m >> txs) < vy) && ((m & txm) < vx) && (r / RPR) < nvch;
        if (ok) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float d = to_f32(v[i].e[e]) - K;
            s1 += d;
            s2 = fmaf(d, d, s2);
          }
        }
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float t = s1 / cnt;
    const float mean = K + t, m2 = fmaxf(fmaf(-s1, t, s2), 0.f);
    const int g = co0 / cpg;
    if (lane == 0 && co0 < a.gn_G * cpg) {
      const int parts = cpg > 32 ? cpg / 32 : 1;
      const int part = cpg > 32 ? (co0 % cpg) / 32 : 0;
      float4* recs = a.gn_parts + ((int64_t)n * a.gn_G + g) * a.gn_np;
      // slot (tile, wave-column 0, part); the tile's other WSP - 1 slots hold count 0
      recs[(tile_rec * WSP) * parts + part] = make_float4(cnt, mean, m2, 0.f);
      for (int w = 1; w < WSP; ++w) recs[(tile_rec * WSP + w) * parts + part] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// Tiles of 8 accumulator blocks (128 AGPRs) are asked to fit 2 waves per SIMD: with their
// LDS footprint two workgroups share a CU, and one wave per SIMD leaves no latency cover.
//
// KS > 1 splits K inside the workgroup: KS groups of WCO x WSP waves each take a contiguous
// share of the stages, with patch buffers of their own, and run in lockstep (same iteration
// count, shared barriers).  At the end groups 1..KS-1 hand their accumulators to group 0
// through LDS, which adds them in group order (deterministic) and stores the tile.  Shapes
// too small to fill the chip with one wave per SIMD (a few stages, one accumulator block per
// wave) then get KS waves per SIMD and a KS-times shorter chain of stage latencies, in one
// launch and with no partial sums in memory.
template <typename T, int WCO, int WSP, int FCO, int FSP, int CB, int XC, bool VR, int KHT, int KWT, bool EPI,
          int KS = 1, bool CL = false, bool LEPI = false>
__global__ __launch_bounds__(64 * WCO * WSP * KS)
__attribute__((amdgpu_waves_per_eu(KS > 1 ? KS : ((FCO * FSP >= 8 && CB == 16) || XC > 1 ? 2 : 1))))
void conv_igemm_kernel(IgArgs a) {
  static_assert(KS == 1 || KHT > 0, "the in-workgroup K split runs on the static tap schedule");
  static_assert(!CL || (KHT > 0 && VR && !EPI), "channels-last staging runs on the static tap schedule");
  using Loader = typename LoaderSel<T, CB, VR, 64 * WCO * WSP, XC, CL>::type;
  constexpr int NWG = WCO * WSP;          // waves per K group
  constexpr int NT = 64 * NWG;            // threads per K group (the tile's loaders)
  constexpr int KB = MfmaTraits<T>::KB, VEC = MfmaTraits<T>::VEC;
  constexpr int ES = sizeof(T);
  constexpr int CBS = CB + VEC;           // padded channel stride of a patch position
  constexpr int BN = WCO * FCO * 32;      // output channels per workgroup
  constexpr int NKB = CB / KB;            // k-blocks per tap
  constexpr uint32_t FRAG = 32 * KB * ES; // bytes of one packed weight fragment
  static_assert(CB % KB == 0, "chunk must hold whole k-blocks");
  extern __shared__ uint4 lds_raw[];
  char* lds_base = reinterpret_cast<char*>(lds_raw);

  const int lane = threadIdx.x & 63;
  const int kg = (threadIdx.x >> 6) / NWG;          // K group
  const int tid = threadIdx.x - kg * NT, wv = tid >> 6;
  const int wco = wv % WCO, wsp = wv / WCO;
  const int half = lane >> 5, col = lane & 31;
  // this K group's patch buffers
  char* lds_bytes = lds_base + (size_t)kg * 2 * (size_t)a.patch_elems * sizeof(T);

  // ---- tile coordinates ---------------------------------------------------------------
  int t = blockIdx.x;
  const int tx_t = t % a.tiles_x; t /= a.tiles_x;
  const int ty_t = t % a.tiles_y; t /= a.tiles_y;
  const int oz = t % a.Do;
  const int n = t / a.Do;
  const int co_tile = blockIdx.y;
  const int split = blockIdx.z;
  __shared__ float s_bias[BN];
  if (kg == 0) stage_bias<T, BN, NT>(a, co_tile, s_bias);  // visible after the prologue's barrier
  // one-pass GroupNorm: this launch's slot tag, from the epoch every workgroup reads first
  __shared__ uint32_t s_tag;
  if constexpr (EPI && LEPI) {
    if (a.gn_onepass && threadIdx.x == 0)
      s_tag = (__hip_atomic_load(a.gn_hdr + 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) << 1) | 1u;
  }
  // stages of this split, then this K group's share of them; every group runs n_it iterations
  const int sp_begin = split * a.stages_per_split;
  const int sp_end = min(a.n_stages, sp_begin + a.stages_per_split);
  const int n_it = KS == 1 ? sp_end - sp_begin : (sp_end - sp_begin + KS - 1) / KS;
  const int s_begin = sp_begin + kg * n_it;
  const int s_end = min(sp_end, s_begin + n_it);
  const int oy0 = ty_t * a.TY, ox0 = tx_t * a.TX;
  const int iy0 = oy0 * a.sh - a.ph, ix0 = ox0 * a.sw - a.pw;
  // aligned-down start of the patch rows (channels-last rows need no alignment along x)
  const int gx0 = CL ? ix0 : (ix0 >= 0 ? ix0 / VEC : -((-ix0 + VEC - 1) / VEC)) * VEC;
  const int mis = ix0 - gx0;
  const int total_chunks = CB * a.PY * a.NCX;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(
      static_cast<const T*>(a.x) + (int64_t)n * a.Ci * a.D * a.H * a.W, a.x_sample_bytes);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.wp, a.wp_bytes);

  // byte offset of this lane's first im2col element of column block j in a patch buffer
  uint32_t pb[FSP];
#pragma unroll
  for (int j = 0; j < FSP; ++j) {
    const int m = (wsp * FSP + j) * 32 + col;
    const int ty = m / a.TX, tx = m - (m / a.TX) * a.TX;
    pb[j] = (uint32_t)(((ty * a.sh) * a.PXS + tx * a.sw + mis) * CBS + half * VEC) * ES;
  }
  const uint32_t wlane = (uint32_t)(col * KB + half * VEC) * ES;
  const uint32_t patch_bytes = (uint32_t)a.patch_elems * ES;
  const uint32_t kh_step = (uint32_t)(a.dh * a.PXS * CBS) * ES;  // patch bytes per kernel row
  const uint32_t kw_step = (uint32_t)(a.dw * CBS) * ES;          // patch bytes per kernel column

  f32x16 acc[FCO][FSP];
#pragma unroll
  for (int i = 0; i < FCO; ++i)
#pragma unroll
    for (int j = 0; j < FSP; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int ntaps2d = a.KH * a.KW;
  const int co_blk0 = co_tile * (BN / 32) + wco * FCO;

  Loader ld;
  const int total_quads = total_chunks / 4;
  if constexpr (VR) ld.init(a, iy0, gx0, total_quads, tid, NT);
  // stage s = (channel chunk cc, kernel plane kd), walked incrementally
  int cc = s_begin / a.KD, kd = s_begin - (s_begin / a.KD) * a.KD;
  const int iz_base = oz * a.sd - a.pd;
  if (s_begin < s_end) {
    if constexpr (VR) {
      const int iz = iz_base + kd * a.dd;
      const uint32_t so = ld.stage_off(a, cc, iz);
      const int lim = ld.stage_lim(a, cc, iz, true);
#pragma unroll
      for (int u = 0; u < Loader::MAXC; ++u) ld.load_fast(rx, u, so, lim);
#pragma unroll
      for (int g = 0; g < Loader::NQ; ++g)
        ld.store_quad(reinterpret_cast<T*>(lds_bytes), g, total_quads, tid, NT);
    } else {
      ld.load(a, rx, cc, iz_base + kd * a.dd, iy0, gx0, total_chunks, tid, NT);
      ld.store(a, reinterpret_cast<T*>(lds_bytes), total_chunks, tid, NT);
    }
  }
  __syncthreads();

  const uint32_t tap_bytes = (uint32_t)a.n_kb * a.co_blocks * FRAG;
  const uint32_t kb_bytes = (uint32_t)a.co_blocks * FRAG;
  // byte offset of (stage (cc, kd), in-plane tap 0) in the packed weights for this wave
  // (readfirstlane: the value is wave-uniform; saying so keeps the compiler from wrapping each
  // buffer load that uses it as an SGPR offset in a waterfall loop)
  auto wbase = [&](int c, int k) -> uint32_t {
    return __builtin_amdgcn_readfirstlane((uint32_t)(k * ntaps2d) * tap_bytes + (uint32_t)(c * NKB) * kb_bytes +
                                          co_blk0 * FRAG);
  };

  if constexpr (KHT > 0) {
    // ---- static schedule for a KHT x KWT kernel plane -----------------------------------
    // Weights stream through NB rotating register buffers PF taps ahead, continuing across
    // stage boundaries.  The next stage's patch chunks are issued two per tap (taps 0-3) and
    // written to the idle LDS buffer a quad at a time at taps QS0 and QS1, where the wait for
    // that tap's weights (issued PF taps earlier, after those chunks) has already covered
    // them; the stage then ends with the barrier alone.  The tap loop is straight-line code,
    // so every wait is an exact vmcnt/lgkmcnt count.
    constexpr int NT2 = KHT * KWT;
    // NB rotating weight buffers (a divisor of NT2, so the rotation repeats every stage),
    // prefetching PF taps ahead; only PF + 1 of them are live at once.  Tiles of one or two
    // accumulator blocks (one output-channel block) run a tap's MFMAs in 32-64 cycles, far
    // less than an L2 round trip, so they keep a whole 3x3 stage of weights in registers and
    // prefetch 6 taps ahead.
    constexpr bool DEEPW = FCO == 1 && FSP <= 2 && NT2 == 9;
    constexpr int NB = DEEPW ? 9 : NT2 % 3 == 0 ? 3 : NT2 % 5 == 0 ? 5 : 7;
    constexpr int PF = DEEPW ? 6 : NB - 1 < 3 ? NB - 1 : 3;
    constexpr int MAXC = Loader::MAXC;
    constexpr int NQ = Loader::NQ;
    static_assert(NT2 % NB == 0, "buffer rotation must repeat every stage");
    static_assert(NQ >= 1 && NQ <= 4 && NT2 >= 9, "schedule below assumes <= 4 quads, 9+ taps");
    // chunks are issued LPT per tap over taps 0-3; quads [0, QH) are written at tap QS0 (their
    // chunks issued by tap 1), quads [QH, NQ) at tap QS1 (chunks issued by tap 3)
    constexpr int LPT = MAXC <= 8 ? 2 : MAXC / 4;
    constexpr int QH = (NQ + 1) / 2;
    // (deep-prefetch tiles write the quads as late as the stage allows: their loads then
    // have the longest time to arrive)
    constexpr int QS0 = DEEPW ? 7 : 5, QS1 = 8;
    uint4 wb[NB][NKB][FCO];
    auto load_w = [&](uint4 (&w)[NKB][FCO], uint32_t so) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < FCO; ++i) w[kb][i] = bload16(rw, wlane, so + kb * kb_bytes + i * FRAG);
    };
    if (s_begin < s_end) {
#pragma unroll
      for (int p = 0; p < PF; ++p) load_w(wb[p], wbase(cc, kd) + p * tap_bytes);
    }
    // im2col fragments are read from LDS one k-step ahead of the MFMAs that use them (two
    // register sets), so inside a stage a wave's MFMAs do not wait on its own LDS reads
    constexpr int NSTEP = NT2 * NKB;
    auto rd_b = [&](uint4 (&pf)[FSP], uint32_t pbuf, int step) {
      const int t2 = step / NKB, kb = step % NKB;
      const uint32_t toffb = (uint32_t)(t2 / KWT) * kh_step + (uint32_t)(t2 % KWT) * kw_step + kb * KB * ES;
#pragma unroll
      for (int j = 0; j < FSP; ++j) pf[j] = *reinterpret_cast<const uint4*>(lds_bytes + pbuf + pb[j] + toffb);
    };
    for (int s = s_begin; s < s_begin + n_it; ++s) {
      // (s >= s_end: a K group with fewer stages than n_it keeps the shared barriers)
      const int iz = iz_base + kd * a.dd;
      const bool zin = s < s_end && (unsigned)iz < (unsigned)a.D;
      const uint32_t pbuf = ((s - s_begin) & 1) ? patch_bytes : 0u;
      const bool has_next = s + 1 < s_end;
      int cc1 = cc, kd1 = kd + 1;
      if (kd1 == a.KD) {
        kd1 = 0;
        ++cc1;
      }
      const int iz1 = iz_base + kd1 * a.dd;
      const uint32_t so1 = __builtin_amdgcn_readfirstlane(ld.stage_off(a, cc1, iz1));
      const int lim1 = __builtin_amdgcn_readfirstlane(ld.stage_lim(a, cc1, iz1, has_next));
      const uint32_t wb_cur = wbase(cc, kd);
      const uint32_t wb_nxt = has_next ? wbase(cc1, kd1) : wb_cur;  // last stage: harmless reload
      uint4 pfb[2][FSP];
      if (zin) rd_b(pfb[0], pbuf, 0);
#pragma unroll
      for (int t2 = 0; t2 < NT2; ++t2) {
        const int tp = t2 + PF;
        load_w(wb[tp % NB], tp < NT2 ? wb_cur + tp * tap_bytes : wb_nxt + (tp - NT2) * tap_bytes);
        if (t2 < 4) {
#pragma unroll
          for (int l = 0; l < LPT; ++l)
            if (t2 * LPT + l < MAXC) ld.load_fast(rx, t2 * LPT + l, so1, lim1);
        }
        if (zin) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            const int step = t2 * NKB + kb;
            if (step + 1 < NSTEP) rd_b(pfb[(step + 1) & 1], pbuf, step + 1);
#pragma unroll
            for (int i = 0; i < FCO; ++i)
#pragma unroll
              for (int j = 0; j < FSP; ++j)
                mfma_block(acc[i][j], wb[t2 % NB][kb][i], pfb[step & 1][j], static_cast<T*>(nullptr));
          }
        }
        // the idle buffer was released by every wave at the previous stage's barrier
        if ((t2 == QS0 || t2 == QS1) && has_next) {
#pragma unroll
          for (int g = (t2 == QS0 ? 0 : QH); g < (t2 == QS0 ? QH : NQ); ++g)
            ld.store_quad(reinterpret_cast<T*>(lds_bytes + (pbuf ^ patch_bytes)), g, total_quads, tid, NT);
        }
      }
      __syncthreads();
      cc = cc1;
      kd = kd1;
    }
  } else
  for (int s = s_begin; s < s_end; ++s) {
    const int iz = iz_base + kd * a.dd;
    const uint32_t pbuf = ((s - s_begin) & 1) ? patch_bytes : 0u;
    const bool has_next = s + 1 < s_end;
    int cc1 = cc, kd1 = kd + 1;
    if (kd1 == a.KD) {
      kd1 = 0;
      ++cc1;
    }
    // prefetch the next stage's patch into registers while this stage computes
    if constexpr (VR) {
      const int iz1 = iz_base + kd1 * a.dd;
      const uint32_t so1 = __builtin_amdgcn_readfirstlane(ld.stage_off(a, cc1, iz1));
      const int lim1 = __builtin_amdgcn_readfirstlane(ld.stage_lim(a, cc1, iz1, has_next));
#pragma unroll
      for (int u = 0; u < Loader::MAXC; ++u) ld.load_fast(rx, u, so1, lim1);
    } else {
      ld.load(a, rx, cc1, iz_base + kd1 * a.dd, iy0, gx0, total_chunks, tid, NT, has_next);
    }
    if ((unsigned)iz < (unsigned)a.D) {
      const uint32_t wsoff = wbase(cc, kd);
      uint4 wA[NKB][FCO], wB[NKB][FCO];
      auto load_w = [&](uint4 (&w)[NKB][FCO], uint32_t so) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < FCO; ++i) w[kb][i] = bload16(rw, wlane, so + kb * kb_bytes + i * FRAG);
      };
      auto compute = [&](const uint4 (&w)[NKB][FCO], uint32_t toffb) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          uint4 pf[FSP];
#pragma unroll
          for (int j = 0; j < FSP; ++j)
            pf[j] = *reinterpret_cast<const uint4*>(lds_bytes + pbuf + pb[j] + toffb + kb * KB * ES);
#pragma unroll
          for (int i = 0; i < FCO; ++i)
#pragma unroll
            for (int j = 0; j < FSP; ++j) mfma_block(acc[i][j], w[kb][i], pf[j], static_cast<T*>(nullptr));
        }
      };
      load_w(wA, wsoff);
      int kh = 0, kw = 0;
      uint32_t toffb = 0;
      auto next_tap = [&]() {
        if (++kw == a.KW) {
          kw = 0;
          ++kh;
          toffb = kh * kh_step;
        } else {
          toffb += kw_step;
        }
      };
      for (int t2 = 0; t2 < ntaps2d; t2 += 2) {
        const bool two = t2 + 1 < ntaps2d;
        if (two) load_w(wB, wsoff + (t2 + 1) * tap_bytes);
        compute(wA, toffb);
        next_tap();
        if (t2 + 2 < ntaps2d) load_w(wA, wsoff + (t2 + 2) * tap_bytes);
        if (two) {
          compute(wB, toffb);
          next_tap();
        }
      }
    }
    if (has_next) {
      if constexpr (VR) {
#pragma unroll
        for (int g = 0; g < Loader::NQ; ++g)
          ld.store_quad(reinterpret_cast<T*>(lds_bytes + (pbuf ^ patch_bytes)), g, total_quads, tid, NT);
      } else {
        ld.store(a, reinterpret_cast<T*>(lds_bytes + (pbuf ^ patch_bytes)), total_chunks, tid, NT);
      }
    }
    __syncthreads();
    cc = cc1;
    kd = kd1;
  }

  // the LDS-staged epilogue (a runtime choice of the host: see store_tile_lds)
  constexpr bool LDS_EPI_OK = sizeof(T) == 2;
  const bool lds_epi = LDS_EPI_OK && a.lds_epi;
  if constexpr (KS > 1) {
    // pairwise rounds of stride st = 1, 2, ...: a group still holding a partial sum whose index
    // is an odd multiple of st parks it in LDS, and the group st below adds it -- a fixed order
    // ((g0 + g1) + (g2 + g3), ...) with at most KS / 2 groups parked at once (the patch
    // buffers are free: the last iteration ended with a barrier)
    float* red = reinterpret_cast<float*>(lds_base);
    auto slot = [&](int p, int i, int j, int r) {
      return ((((p * NWG + wv) * FCO + i) * FSP + j) * 16 + r) * 64 + lane;
    };
#pragma unroll
    for (int st = 1; st < KS; st *= 2) {
      const bool parks = kg % (2 * st) == st;
      const bool adds = kg % (2 * st) == 0 && kg + st < KS;
      const int p = kg / (2 * st);
      if (parks) {
#pragma unroll
        for (int i = 0; i < FCO; ++i)
#pragma unroll
          for (int j = 0; j < FSP; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[slot(p, i, j, r)] = acc[i][j][r];
      }
      __syncthreads();
      if (adds) {
#pragma unroll
        for (int i = 0; i < FCO; ++i)
#pragma unroll
          for (int j = 0; j < FSP; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] += red[slot(p, i, j, r)];
      }
      // (the next round, or the staged epilogue, reuses the area)
      if (st * 2 < KS || lds_epi) __syncthreads();
    }
    if (kg > 0 && !lds_epi) return;
  }
  if constexpr (LDS_EPI_OK) {
    if (lds_epi) {
      // (KS == 1: the last stage ended with a barrier, so the patch buffers are free)
      if constexpr (CL)
        store_tile_lds_cl<T, FCO, FSP, BN, WSP * FSP * 32, WSP, 64 * NWG * KS>(
            a, acc, s_bias, lds_base, n, co_tile, oz, oy0, ox0, wco, wsp, kg == 0, threadIdx.x);
      else
        store_tile_lds<T, FCO, FSP, BN, WSP * FSP * 32, WSP, EPI, 64 * NWG * KS>(
            a, acc, s_bias, lds_base, n, co_tile, oz, oy0, ox0, wco, wsp, kg == 0, threadIdx.x,
            (oz * a.tiles_y + ty_t) * a.tiles_x + tx_t, EPI && LEPI ? s_tag : 0u);
      return;
    }
  }
  // (LEPI: the instantiation that carries only the LDS-staged epilogue -- the host launches
  // it only with a.lds_epi set; without the per-value epilogue extras beside it, the epilogue
  // variant keeps the plain kernel's register budget)
  if constexpr (!LEPI) {
    // GroupNorm record index of this wave's spatial tile: (z, tile row, tile column), then wave
    const int sp_rec = ((oz * a.tiles_y + ty_t) * a.tiles_x + tx_t) * WSP + wsp;
    store_tile<T, FCO, FSP, BN, EPI, CL>(a, acc, s_bias, n, co_tile, split, oz, oy0, ox0, wco, wsp, half, col,
                                         sp_rec);
  }
}

// Packed weights Wp[tap][kb][co_block][32][KB] from w[Co][Ci][taps]; zero beyond Co / Ci.
template <typename T>
__global__ __launch_bounds__(256) void pack_weights_kernel(const T* __restrict__ w, T* __restrict__ wp,
                                                           int Co, int Ci, int taps, int n_kb,
                                                           int co_blocks, uint32_t chunks) {
  // one thread per 16-byte chunk of the packed layout [tap][kb][co_block][32][KB] (KB is a
  // multiple of the chunk's E elements, so a chunk never crosses a row).  Consecutive threads
  // take consecutive taps of one chunk position: tap is w's contiguous axis, so each of the E
  // loads of a wave reads a few contiguous runs instead of 64 rows Ci*taps apart; only the one
  // 16-byte store per thread is scattered.  32-bit index math (the host keeps the packed
  // weights under 2 GiB).
  constexpr int KB = MfmaTraits<T>::KB;
  constexpr int E = 16 / sizeof(T);
  constexpr uint32_t KPR = KB / E;  // chunks per packed row
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const uint32_t tap = c % (uint32_t)taps;
  uint32_t r = c / (uint32_t)taps;
  const uint32_t k8 = r % KPR;
  r /= KPR;
  const uint32_t row = r % 32;
  r /= 32;
  const uint32_t cb = r % (uint32_t)co_blocks;
  const uint32_t kb = r / (uint32_t)co_blocks;
  const int co = (int)(cb * 32 + row);
  const uint32_t dst = ((((tap * (uint32_t)n_kb + kb) * (uint32_t)co_blocks + cb) * 32 + row) * KPR + k8) * E;
  Vec16<T> v;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int ci = (int)(kb * KB + k8 * E) + e;
    v.e[e] = (co < Co && ci < Ci) ? w[((int64_t)co * Ci + ci) * taps + tap] : static_cast<T>(0.0f);
  }
  *reinterpret_cast<uint4*>(wp + dst) = v.raw;
}

// y = sum over splits of the fp32 partials + bias
// (cl: y and the partials channels-last, so element i is channel i % Co)
template <typename T>
__global__ __launch_bounds__(256) void splitk_finalize_kernel(const float* __restrict__ part, const T* __restrict__ bias,
                                                              T* __restrict__ y, int splits, int Co, int64_t spo,
                                                              int64_t total, int cl) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float v = 0.f;
  for (int s = 0; s < splits; ++s) v += part[(int64_t)s * total + i];
  if (bias) v += to_f32(bias[cl ? i % Co : (i / spo) % Co]);
  y[i] = from_f32<T>(v);
}

// The same sum, 4 consecutive outputs per thread (16-byte partial loads, one 8- or 16-byte
// store): for 4-aligned y / partials with the 4 outputs in one channel (NC[D]HW, spo % 4 == 0)
// or in 4 consecutive channels (channels-last, Co % 4 == 0).  Same order of additions as the
// scalar kernel, so the same bits.
template <typename T>
__global__ __launch_bounds__(256) void splitk_finalize4_kernel(const float4* __restrict__ part,
                                                               const T* __restrict__ bias, T* __restrict__ y,
                                                               int splits, int Co, int64_t spo4, int64_t total4,
                                                               int cl) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total4) return;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const float4 q = part[(int64_t)s * total4 + i];
    v[0] += q.x;
    v[1] += q.y;
    v[2] += q.z;
    v[3] += q.w;
  }
  if (bias) {
    if (cl) {
      const int c = (int)((i * 4) % Co);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] += to_f32(bias[c + k]);
    } else {
      const float b = to_f32(bias[(i / spo4) % Co]);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] += b;
    }
  }
  if constexpr (sizeof(T) == 4) {
    reinterpret_cast<float4*>(y)[i] = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    T o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = from_f32<T>(v[k]);
    reinterpret_cast<uint2*>(y)[i] = *reinterpret_cast<const uint2*>(o);
  }
}

struct IgVariant {
  const char* name;
  int dtype_class;  // 0 = 16-bit, 1 = fp32
  int wco, wsp, fco, fsp, cb;
  int xc;           // patch-loader capacity multiplier (PatchLoader XC)
  int max_splits;   // split-K limit (1: never split, so a call is one launch)
  int ks = 1;       // K groups inside the workgroup (conv_igemm_kernel KS)
};

const IgVariant kIg[] = {
    {"h_w22_f22_cb32", 0, 2, 2, 2, 2, 32, 1, 16},
    {"h_w22_f24_cb32", 0, 2, 2, 2, 4, 32, 1, 16},
    {"h_w14_f22_cb32", 0, 1, 4, 2, 2, 32, 1, 16},
    {"h_w22_f22_cb16", 0, 2, 2, 2, 2, 16, 1, 16},
    {"h_w41_f22_cb32", 0, 4, 1, 2, 2, 32, 1, 16},
    {"h_w21_f24_cb32", 0, 2, 1, 2, 4, 32, 1, 16},
    {"h_w22_f12_cb32", 0, 2, 2, 1, 2, 32, 1, 16},
    {"h_w21_f14_cb32", 0, 2, 1, 1, 4, 32, 1, 16},
    {"h_w22_f24_cb16", 0, 2, 2, 2, 4, 16, 1, 16},
    {"f32_w22_f22_cb16", 1, 2, 2, 2, 2, 16, 1, 16},
    {"f32_w14_f22_cb16", 1, 1, 4, 2, 2, 16, 1, 16},
    {"f32_w22_f12_cb16", 1, 2, 2, 1, 2, 16, 1, 16},
    {"f32_w21_f14_cb16", 1, 2, 1, 1, 4, 16, 1, 16},
    // 64 output channels with a 7x7 plane: the 32x32-position tile's 14-row patch needs twice
    // the default loader capacity
    {"h_w14_f22_cb16x2", 0, 1, 4, 2, 2, 16, 2, 16},
    // small tiles that never split K: for shapes too small to fill the chip (config 4's
    // 64-channel conv), one launch with no partial sums to write and add up
    {"h_w12_f21_cb32_ns", 0, 1, 2, 2, 1, 32, 1, 1},
    {"h_w22_f11_cb32_ns", 0, 2, 2, 1, 1, 32, 1, 1},
    {"h_w21_f12_cb32_ns", 0, 2, 1, 1, 2, 32, 1, 1},
    // the same small tiles with K split inside the workgroup (2-4 waves per SIMD on shapes
    // that give each SIMD one output tile)
    {"h_w22_f11_cb32_k2", 0, 2, 2, 1, 1, 32, 1, 1, 2},
    {"h_w22_f11_cb32_k3", 0, 2, 2, 1, 1, 32, 1, 1, 3},
    {"h_w22_f11_cb16_k4", 0, 2, 2, 1, 1, 16, 1, 1, 4},
    {"h_w12_f21_cb32_k2", 0, 1, 2, 2, 1, 32, 1, 1, 2},
    {"f32_w22_f11_cb16_k2", 1, 2, 2, 1, 1, 16, 1, 1, 2},
    {"f32_w22_f11_cb16_k3", 1, 2, 2, 1, 1, 16, 1, 1, 3},
    // the 7x7-plane tile with two K groups: half the split-K partials in memory
    {"h_w14_f22_cb16x2_k2", 0, 1, 4, 2, 2, 16, 2, 16, 2},
    // the large tiles with two K groups (two waves per SIMD from one workgroup per CU):
    // shapes with about one output tile per CU (config 5's 256-channel conv) then need no
    // split-K partials in memory and no finalize pass
    {"h_w22_f24_cb16_k2", 0, 2, 2, 2, 4, 16, 1, 16, 2},
    {"h_w41_f22_cb32_k2", 0, 4, 1, 2, 2, 32, 1, 16, 2},
    // 64 output channels on large grids: 2x4 register tiles (half the weight loads per MFMA of
    // the 2x2 ones) over a 512-position tile, two workgroups per CU
    {"h_w14_f24_cb16x2", 0, 1, 4, 2, 4, 16, 2, 16},
};
constexpr int kNumIg = sizeof(kIg) / sizeof(kIg[0]);

struct IgPlan {
  IgArgs a;
  bool cl = false;  // channels-last x and y (NDHWC / NHWC)
  int bn, bm, splits, nthreads;
  size_t lds, wp_bytes, part_bytes;
  int64_t tiles;
};

int plan_ig(const ConvShape& p, int v, IgPlan& pl, bool unsplit = false) {
  const IgVariant& vr = kIg[v];
  const bool f32 = p.dtype == ATK_F32;
  if ((vr.dtype_class == 1) != f32) return fail(ATK_UNSUPPORTED, "conv %s: dtype not served", vr.name);
  const int es = f32 ? 4 : 2;
  const int KB = f32 ? 8 : 16, VEC = f32 ? 4 : 8;
  pl.bn = vr.wco * vr.fco * 32;
  pl.bm = vr.wsp * vr.fsp * 32;
  const int ntg = 64 * vr.wco * vr.wsp;  // threads of one K group (the patch loaders)
  pl.nthreads = ntg * vr.ks;
  IgArgs& a = pl.a;
  a.N = p.N; a.Ci = p.Ci; a.D = p.D; a.H = p.H; a.W = p.W; a.Co = p.Co;
  a.KD = p.KD; a.KH = p.KH; a.KW = p.KW; a.sd = p.sd; a.sh = p.sh; a.sw = p.sw;
  a.pd = p.pd; a.ph = p.ph; a.pw = p.pw; a.dd = p.dd; a.dh = p.dh; a.dw = p.dw;
  a.Do = p.Do; a.Ho = p.Ho; a.Wo = p.Wo;
  int tx = 1;
  while (tx < p.Wo && tx < 64) tx <<= 1;
  if (tx > pl.bm) tx = pl.bm;
  a.TX = tx;
  a.TY = pl.bm / tx;
  a.tiles_x = (p.Wo + a.TX - 1) / a.TX;
  a.tiles_y = (p.Ho + a.TY - 1) / a.TY;
  a.PX = (a.TX - 1) * p.sw + (p.KW - 1) * p.dw + 1;
  const int n_cc = (p.Ci + vr.cb - 1) / vr.cb;
  a.n_kb = n_cc * (vr.cb / KB);
  a.co_blocks = (p.Co + pl.bn - 1) / pl.bn * (pl.bn / 32);
  a.NCX = (a.PX + VEC - 1) / VEC + 1;
  // Row pitch: padded (0-7 positions) so that consecutive patch rows start CB*es bytes apart
  // modulo 128 -- the quad writes of one LDS cycle, CB*es bytes per row, then tile 128 bytes
  // -- unless the padding would cost a resident workgroup per CU (decided below).
  int row_pad = 0;
  for (int pad = 0; pad < 8; ++pad) {
    if (((a.NCX * VEC + pad) * (vr.cb + VEC) * es) % 128 == (vr.cb * es) % 128) {
      row_pad = pad;
      break;
    }
  }
  // stage = (ci chunk, kd): the patch of all KH x KW taps of one input plane
  a.PY = (a.TY - 1) * p.sh + (p.KH - 1) * p.dh + 1;
  {
    constexpr size_t kLdsCu = 160 * 1024;
    const size_t plain = (size_t)2 * a.PY * a.NCX * VEC * (vr.cb + VEC) * es + 1024;
    const size_t padded = (size_t)2 * a.PY * (a.NCX * VEC + row_pad) * (vr.cb + VEC) * es + 1024;
    a.PXS = a.NCX * VEC + (kLdsCu / padded == kLdsCu / plain ? row_pad : 0);
  }
  a.patch_elems = a.PY * a.PXS * (vr.cb + VEC);
  // two patch buffers per K group; with K groups, the accumulator hand-over reuses them (at
  // most KS / 2 groups park at once)
  pl.lds = (size_t)2 * a.patch_elems * es * vr.ks;
  if (vr.ks > 1)
    pl.lds = std::max(pl.lds, (size_t)(vr.ks / 2) * vr.wco * vr.wsp * vr.fco * vr.fsp * 16 * 64 * 4);
  {
    const int maxc = (f32 ? vr.cb / 2 : vr.cb / 4) * vr.xc * 256 / ntg;  // PatchLoader::MAXC
    if (pl.lds > 150 * 1024 || vr.cb * a.PY * a.NCX > maxc * ntg)
      return fail(ATK_UNSUPPORTED, "conv %s: stage of %zu LDS bytes does not fit the variant", vr.name, pl.lds);
  }
  a.n_stages = n_cc * p.KD;
  pl.tiles = (int64_t)p.N * p.Do * a.tiles_y * a.tiles_x;
  const int co_tiles = (p.Co + pl.bn - 1) / pl.bn;
  if (pl.tiles > 0x7fffffff || co_tiles > 65535) return fail(ATK_UNSUPPORTED, "conv %s: grid too large", vr.name);
  // split K (stages) until the grid covers the chip about twice (a workgroup with K groups
  // counts as that many workgroups); `unsplit` (the one-pass GroupNorm) keeps one split
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const int64_t wgs = pl.tiles * co_tiles * vr.ks;
  int splits = 1;
  while (!unsplit && wgs * splits < 2 * cus && splits * 2 * vr.ks <= a.n_stages && splits * 2 <= vr.max_splits)
    splits *= 2;
  a.stages_per_split = (a.n_stages + splits - 1) / splits;
  splits = (a.n_stages + a.stages_per_split - 1) / a.stages_per_split;
  pl.splits = splits;
  const int taps = p.KD * p.KH * p.KW;
  pl.wp_bytes = (size_t)taps * a.n_kb * a.co_blocks * 32 * KB * es;
  // buffer loads address one input sample / the packed weights with 31-bit byte offsets
  if ((int64_t)p.Ci * p.D * p.H * p.W * es >= (1ll << 31) || pl.wp_bytes >= (1ull << 31))
    return fail(ATK_UNSUPPORTED, "conv %s: sample or weights exceed 2 GiB", vr.name);
  const int64_t ysz = (int64_t)p.N * p.Co * p.Do * p.Ho * p.Wo;
  pl.part_bytes = splits > 1 ? (size_t)splits * ysz * 4 : 0;
  return ATK_OK;
}

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// One kernel instantiation: the LDS opt-in is a per-kernel attribute, set once per kernel.
// Workgroups of kernel Kern resident per CU with `lds` bytes of dynamic LDS: the register /
// wave limit (queried once per kernel and device) and the 160 KB of LDS, whichever is lower.
template <void (*Kern)(IgArgs)>
int resident_per_cu(int nthreads, size_t lds) {
  static int by_regs[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (by_regs[dev] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(Kern), nthreads, 0) !=
        hipSuccess)
      return 0;
    by_regs[dev] = n;
  }
  return std::min<int>(by_regs[dev], (int)((160 * 1024) / std::max<size_t>(lds, 1)));
}

// Launches Kern.  With `lds_only` (an instantiation carrying only the LDS-staged epilogue)
// it returns kNeedPerValue instead of launching when that epilogue cannot be kept.  The
// one-pass GroupNorm launch is cooperative.
constexpr int kNeedPerValue = -1;
constexpr int kOnePassHdrBytes = 4096;  // diagnostics, epoch, launch counter, block counters
constexpr int kOnePassMaxWg = (kOnePassHdrBytes - 256) / 64 * 64;  // one 64-byte counter per 64 workgroups

template <void (*Kern)(IgArgs)>
int launch_ig_kern(const IgPlan& plan, int nthreads, hipStream_t s, bool lds_only = false) {
  IgPlan pl = plan;
  if (pl.a.lds_epi) {
    // the staging area of the LDS-staged epilogue: keep it only where it costs no resident
    // workgroup per CU
    const size_t stg = (size_t)(pl.cl ? pl.bm : pl.bn) * pl.a.epi_pitch;
    if (stg > pl.lds) {
      const int before = resident_per_cu<Kern>(nthreads, pl.lds);
      if (before > 0 && resident_per_cu<Kern>(nthreads, stg) == before) pl.lds = stg;
      else pl.a.lds_epi = 0;
    }
  }
  if (lds_only && !pl.a.lds_epi) return pl.a.gn_onepass ? fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm "
                                                                  "needs the LDS-staged epilogue") : kNeedPerValue;
  if (pl.lds > 64 * 1024) {
    // opt in to more than 64 KB of dynamic LDS (gfx950 has 160 KB per CU)
    static bool raised = false;
    if (!raised) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(Kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              150 * 1024) != hipSuccess)
        return fail(ATK_UNSUPPORTED, "conv: cannot raise the LDS limit");
      raised = true;
    }
  }
  dim3 grid((unsigned)pl.tiles, (unsigned)((pl.a.Co + pl.bn - 1) / pl.bn), (unsigned)pl.splits);
  if (pl.a.gn_onepass) {
    // every workgroup waits for records of others: the grid must be resident at once, which a
    // cooperative launch guarantees (or refuses)
    const int64_t nwg = (int64_t)grid.x * grid.y;
    if (nwg > (int64_t)resident_per_cu<Kern>(nthreads, pl.lds) * device_cu_count() || nwg > kOnePassMaxWg)
      return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm grid (%lld workgroups) is not resident at once",
                  (long long)nwg);
    void* args[] = {&pl.a};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(Kern), grid, dim3(nthreads), args,
                                                    (unsigned)pl.lds, s);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // (not sticky: clear it for the next launch's check)
      return fail(e == hipErrorCooperativeLaunchTooLarge ? ATK_UNSUPPORTED : ATK_ELAUNCH,
                  "conv (one-pass GroupNorm): cooperative launch refused: %s", hipGetErrorString(e));
    }
    return ATK_OK;
  }
  hipLaunchKernelGGL(Kern, grid, dim3(nthreads), pl.lds, s, pl.a);
  return check_launch("conv_igemm_kernel");
}

template <typename T, int WCO, int WSP, int FCO, int FSP, int CB, int XC, bool VR, int KHT, int KWT, int KS = 1>
int launch_ig_vr(const IgPlan& pl, hipStream_t s) {
  constexpr int nt = 64 * WCO * WSP * KS;
  if (pl.cl) {
    if constexpr (sizeof(T) == 2 && VR && KHT > 0)
      return launch_ig_kern<conv_igemm_kernel<T, WCO, WSP, FCO, FSP, CB, XC, VR, KHT, KWT, false, KS, true>>(pl, nt, s);
    else
      return fail(ATK_UNSUPPORTED, "conv (channels-last): 16-bit types with a 3x3 or 7x7 plane only");
  }
  // the residual / GroupNorm epilogue is its own instantiation, so the plain kernel is unchanged;
  // the LDS-staged form of it (16-bit types) another, tried first
  if (pl.a.resid || pl.a.gn_parts || pl.a.gn_onepass) {
    if constexpr (VR) {
      if constexpr (sizeof(T) == 2 && KHT > 0) {
        if (pl.a.lds_epi) {
          const int rc = launch_ig_kern<conv_igemm_kernel<T, WCO, WSP, FCO, FSP, CB, XC, VR, KHT, KWT, true, KS,
                                                          false, true>>(pl, nt, s, true);
          if (rc != kNeedPerValue) return rc;
        }
      }
      if (pl.a.gn_onepass) return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm needs the LDS-staged epilogue");
      IgPlan pv = pl;
      pv.a.lds_epi = 0;
      return launch_ig_kern<conv_igemm_kernel<T, WCO, WSP, FCO, FSP, CB, XC, VR, KHT, KWT, true, KS>>(pv, nt, s);
    } else {
      return fail(ATK_UNSUPPORTED, "conv: the residual / GroupNorm epilogue needs 16-byte aligned input rows");
    }
  }
  return launch_ig_kern<conv_igemm_kernel<T, WCO, WSP, FCO, FSP, CB, XC, VR, KHT, KWT, false, KS>>(pl, nt, s);
}

template <typename T, int WCO, int WSP, int FCO, int FSP, int CB, int XC = 1, int KS = 1>
int launch_ig_t(const IgPlan& pl, hipStream_t s) {
  if (pl.a.KH == 3 && pl.a.KW == 3 && pl.a.vec_rows)
    return launch_ig_vr<T, WCO, WSP, FCO, FSP, CB, XC, true, 3, 3, KS>(pl, s);
  if (pl.a.KH == 7 && pl.a.KW == 7 && pl.a.vec_rows)
    return launch_ig_vr<T, WCO, WSP, FCO, FSP, CB, XC, true, 7, 7, KS>(pl, s);
  if (pl.cl)
    return fail(ATK_UNSUPPORTED, "conv (channels-last): needs a 3x3 or 7x7 plane, Ci %% 8 == 0 and aligned tensors");
  if constexpr (KS > 1) {
    return fail(ATK_UNSUPPORTED, "conv: the in-workgroup K split needs a 3x3 or 7x7 plane and 16-byte aligned rows");
  } else if constexpr (XC > 1) {
    // the element-wise loader of unaligned rows spills at this capacity
    if (!pl.a.vec_rows) return fail(ATK_UNSUPPORTED, "conv: this tile needs 16-byte aligned input rows");
    return launch_ig_vr<T, WCO, WSP, FCO, FSP, CB, XC, true, 0, 0>(pl, s);
  } else {
    return pl.a.vec_rows ? launch_ig_vr<T, WCO, WSP, FCO, FSP, CB, XC, true, 0, 0>(pl, s)
                         : launch_ig_vr<T, WCO, WSP, FCO, FSP, CB, XC, false, 0, 0>(pl, s);
  }
}

// Pack w[Co][Ci][taps] into the fragment order variant v reads (plan_ig's layout) at wp.
template <typename T>
int pack_ig(const ConvShape& p, const IgPlan& pl, const void* w, void* wp, hipStream_t s) {
  const int taps = p.KD * p.KH * p.KW;
  const uint32_t chunks = (uint32_t)(pl.wp_bytes / 16);  // wp_bytes: a multiple of 32 rows x KB elements
  hipLaunchKernelGGL((pack_weights_kernel<T>), dim3((chunks + 255) / 256), dim3(256), 0, s,
                     static_cast<const T*>(w), static_cast<T*>(wp), p.Co, p.Ci, taps, pl.a.n_kb, pl.a.co_blocks,
                     chunks);
  return check_launch("pack_weights_kernel");
}

// The implicit GEMM on weights already packed at wp; `part` holds the split-K partials (or is
// null when the plan does not split).
// GroupNorm records per (n, g) that an unsplit launch of variant v writes (0: it cannot).
int gn_records(const ConvShape& p, const IgPlan& pl, int v, int G) {
  if (G <= 0 || p.Co % G || pl.splits != 1) return 0;
  const int cpg = p.Co / G;
  if (!((cpg % 4 == 0 && 32 % cpg == 0) || cpg % 32 == 0)) return 0;
  const int64_t np = (int64_t)p.Do * pl.a.tiles_y * pl.a.tiles_x * kIg[v].wsp * (cpg > 32 ? cpg / 32 : 1);
  return np < (1 << 30) ? (int)np : 0;
}

// Whether store_tile_lds sums a tile's GroupNorm records in registers for channels-per-group
// cpg (its gn_reg condition): equal run counts per thread, every store instruction inside one
// unit, and a unit spread over at most WSP waves.
bool gn_reg_layout(const IgPlan& pl, int v, int cpg) {
  const int rpr = pl.bm / 8, nthr = pl.nthreads;
  if (cpg <= 0 || (pl.bn * rpr) % nthr) return false;
  const int nrun = pl.bn * rpr / nthr;
  const int urun = (cpg >= 32 ? 32 : cpg) * rpr;
  return urun % 64 == 0 && (urun <= nrun * 64 || urun / (nrun * 64) <= kIg[v].wsp);
}

// The one-pass GroupNorm's parameters and its workspace (kOnePassHdrBytes of header, then
// 24 bytes per record slot and 16 per (n, g) result)
struct GnOnePass {
  const void* gamma;
  const void* beta;
  int pdt;
  float eps;
  int silu;
  void* ws;
};

size_t gn_onepass_bytes(const ConvShape& p, int np, int G) {
  return (size_t)kOnePassHdrBytes + (size_t)p.N * G * np * 24 + (size_t)p.N * G * 16;
}

template <typename T>
int run_ig(const ConvShape& p, IgPlan& pl, const void* x, const void* wp, const void* bias, void* y, int v,
           float* part, hipStream_t s, const void* resid = nullptr, float4* gn_parts = nullptr, int gn_G = 0,
           bool cl = false, const GnOnePass* op = nullptr) {
  int rc = ATK_OK;
  IgArgs& a = pl.a;
  pl.cl = cl;
  a.gn_onepass = 0;
  if (op) {
    if (sizeof(T) != 2 || cl || resid || gn_parts || pl.splits != 1)
      return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm takes unsplit 16-bit NC[D]HW convs without a residual");
    if (!gn_reg_layout(pl, v, gn_G > 0 ? p.Co / gn_G : 0))
      return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm needs this tile's records summed in registers");
    a.gn_onepass = 1;
    a.gn_silu = op->silu;
    a.gn_pdt = op->pdt;
    a.gn_eps = op->eps;
    a.gn_gamma = op->gamma;
    a.gn_beta = op->beta;
    a.gn_hdr = static_cast<unsigned int*>(op->ws);
    a.gn_slots = reinterpret_cast<unsigned long long*>(static_cast<char*>(op->ws) + kOnePassHdrBytes);
    const int khz = device_wall_clock_khz();
    a.gn_wait_ticks = (unsigned long long)(khz > 0 ? khz : 100000) * 200;  // 200 ms
  }
  if (cl && (sizeof(T) != 2 || resid || gn_parts || p.Ci % 8 || p.Co % 8))
    return fail(ATK_UNSUPPORTED, "conv (channels-last): 16-bit types, Ci and Co multiples of 8, no epilogue extras");
  a.x = x; a.bias = bias; a.y = y;
  a.resid = resid;
  a.gn_parts = gn_parts;
  a.gn_G = gn_G;
  a.gn_cpg = gn_G > 0 ? p.Co / gn_G : 0;
  a.gn_np = gn_parts || op ? gn_records(p, pl, v, gn_G) : 0;
  if ((resid || gn_parts) && pl.splits != 1)
    return fail(ATK_UNSUPPORTED, "conv: the residual / GroupNorm epilogue needs an unsplit launch");
  if ((gn_parts || op) && a.gn_np == 0)
    return fail(ATK_UNSUPPORTED, "conv: GroupNorm statistics need Co/G in {4, 8, 16, 32} or a multiple of 32");
  // 16-byte patch chunks: along x rows (NCDHW) or along channels (channels-last)
  a.vec_rows = cl ? (aligned16(x) && aligned16(y)) : (p.W % (16 / (int)sizeof(T)) == 0) && aligned16(x);
  a.x_sample_bytes = (uint32_t)((int64_t)p.Ci * p.D * p.H * p.W * sizeof(T));
  a.wp_bytes = (uint32_t)pl.wp_bytes;
  a.wp = wp;
  a.part = pl.splits > 1 ? part : nullptr;
  // LDS-staged epilogue for plain unsplit 16-bit NC[D]HW output (store_tile_lds) where the
  // shape allows it; launch_ig_kern keeps it only if its staging area costs no resident
  // workgroup per CU
  a.epi_pitch = cl ? pl.bn * 2 + 8 : pl.bm * 2 + 16;
  {
    // ATK_CONV_LDS_EPI=0 keeps the per-value stores (read per call: tests compare the two)
    const char* e = getenv("ATK_CONV_LDS_EPI");
    const bool off = e && e[0] == '0';
    if (cl)
      a.lds_epi = (!off && sizeof(T) == 2 && pl.splits == 1 && p.Co % 8 == 0 && aligned16(y) &&
                   (size_t)pl.bm * a.epi_pitch <= 150 * 1024) ? 1 : 0;
    else
      a.lds_epi = (!off && sizeof(T) == 2 && pl.splits == 1 && p.Wo % 8 == 0 && a.TX % 8 == 0 && aligned16(y) &&
                   (!resid || aligned16(resid)) && (size_t)pl.bn * a.epi_pitch <= 150 * 1024) ? 1 : 0;
  }
  // instantiate only the variants of this element type's class
  if constexpr (sizeof(T) == 2) {
    switch (v) {
      case 0: rc = launch_ig_t<T, 2, 2, 2, 2, 32>(pl, s); break;
      case 1: rc = launch_ig_t<T, 2, 2, 2, 4, 32>(pl, s); break;
      case 2: rc = launch_ig_t<T, 1, 4, 2, 2, 32>(pl, s); break;
      case 3: rc = launch_ig_t<T, 2, 2, 2, 2, 16>(pl, s); break;
      case 4: rc = launch_ig_t<T, 4, 1, 2, 2, 32>(pl, s); break;
      case 5: rc = launch_ig_t<T, 2, 1, 2, 4, 32>(pl, s); break;
      case 6: rc = launch_ig_t<T, 2, 2, 1, 2, 32>(pl, s); break;
      case 7: rc = launch_ig_t<T, 2, 1, 1, 4, 32>(pl, s); break;
      case 8: rc = launch_ig_t<T, 2, 2, 2, 4, 16>(pl, s); break;
      case 13: rc = launch_ig_t<T, 1, 4, 2, 2, 16, 2>(pl, s); break;
      case 14: rc = launch_ig_t<T, 1, 2, 2, 1, 32>(pl, s); break;
      case 15: rc = launch_ig_t<T, 2, 2, 1, 1, 32>(pl, s); break;
      case 16: rc = launch_ig_t<T, 2, 1, 1, 2, 32>(pl, s); break;
      case 17: rc = launch_ig_t<T, 2, 2, 1, 1, 32, 1, 2>(pl, s); break;
      case 18: rc = launch_ig_t<T, 2, 2, 1, 1, 32, 1, 3>(pl, s); break;
      case 19: rc = launch_ig_t<T, 2, 2, 1, 1, 16, 1, 4>(pl, s); break;
      case 20: rc = launch_ig_t<T, 1, 2, 2, 1, 32, 1, 2>(pl, s); break;
      case 23: rc = launch_ig_t<T, 1, 4, 2, 2, 16, 2, 2>(pl, s); break;
      case 24: rc = launch_ig_t<T, 2, 2, 2, 4, 16, 1, 2>(pl, s); break;
      case 25: rc = launch_ig_t<T, 4, 1, 2, 2, 32, 1, 2>(pl, s); break;
      case 26: rc = launch_ig_t<T, 1, 4, 2, 4, 16, 2>(pl, s); break;
      default: return fail(ATK_EINVAL, "conv: bad variant");
    }
  } else {
    switch (v) {
      case 9: rc = launch_ig_t<T, 2, 2, 2, 2, 16>(pl, s); break;
      case 10: rc = launch_ig_t<T, 1, 4, 2, 2, 16>(pl, s); break;
      case 11: rc = launch_ig_t<T, 2, 2, 1, 2, 16>(pl, s); break;
      case 12: rc = launch_ig_t<T, 2, 1, 1, 4, 16>(pl, s); break;
      case 21: rc = launch_ig_t<T, 2, 2, 1, 1, 16, 1, 2>(pl, s); break;
      case 22: rc = launch_ig_t<T, 2, 2, 1, 1, 16, 1, 3>(pl, s); break;
      default: return fail(ATK_EINVAL, "conv: bad variant");
    }
  }
  if (rc || pl.splits == 1) return rc;
  const int64_t ysz = (int64_t)p.N * p.Co * p.Do * p.Ho * p.Wo;
  const int64_t spo = (int64_t)p.Do * p.Ho * p.Wo;
  const bool by4 = (cl ? p.Co % 4 == 0 : spo % 4 == 0) && (reinterpret_cast<uintptr_t>(y) % (4 * sizeof(T))) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.part) % 16) == 0;
  if (by4) {
    const int64_t n4 = ysz / 4;
    hipLaunchKernelGGL((splitk_finalize4_kernel<T>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(a.part), static_cast<const T*>(bias), static_cast<T*>(y),
                       pl.splits, p.Co, spo / 4, n4, cl ? 1 : 0);
    return check_launch("splitk_finalize4_kernel");
  }
  hipLaunchKernelGGL((splitk_finalize_kernel<T>), dim3((unsigned)((ysz + 255) / 256)), dim3(256), 0, s,
                     a.part, static_cast<const T*>(bias), static_cast<T*>(y), pl.splits, p.Co, spo, ysz, cl ? 1 : 0);
  return check_launch("splitk_finalize_kernel");
}

// Pack, then run: the packed weights at the front of the workspace, the partials after them.
template <typename T>
int launch_ig(const ConvShape& p, const void* x, const void* w, const void* bias, void* y, int v,
              void* ws, size_t ws_bytes, hipStream_t s) {
  IgPlan pl;
  int rc = plan_ig(p, v, pl);
  if (rc) return rc;
  const size_t need = align256(pl.wp_bytes) + pl.part_bytes;
  if (!ws || ws_bytes < need) return fail(ATK_EINVAL, "conv: workspace of %zu bytes needed", need);
  rc = pack_ig<T>(p, pl, w, ws, s);
  if (rc) return rc;
  return run_ig<T>(p, pl, x, ws, bias, y, v,
                   reinterpret_cast<float*>(static_cast<char*>(ws) + align256(pl.wp_bytes)), s);
}

}  // namespace

int conv_igemm_num_variants() { return kNumIg; }
const char* conv_igemm_variant_name(int v) { return (v >= 0 && v < kNumIg) ? kIg[v].name : nullptr; }

size_t conv_igemm_workspace_bytes(const ConvShape& p, int v) {
  if (v < 0 || v >= kNumIg) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl)) return 0;
  return align256(pl.wp_bytes) + pl.part_bytes;
}

size_t conv_igemm_packed_bytes(const ConvShape& p, int v) {
  if (v < 0 || v >= kNumIg) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl)) return 0;
  return align256(pl.wp_bytes);
}

size_t conv_igemm_prepacked_workspace_bytes(const ConvShape& p, int v) {
  if (v < 0 || v >= kNumIg) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl)) return 0;
  return pl.part_bytes;
}

int conv_igemm_pack(const ConvShape& p, const void* w, void* packed, size_t packed_bytes, int v, hipStream_t s) {
  if (v < 0 || v >= kNumIg) return fail(ATK_EINVAL, "conv: variant out of range");
  IgPlan pl;
  int rc = plan_ig(p, v, pl);
  if (rc) return rc;
  if (!packed || packed_bytes < align256(pl.wp_bytes))
    return fail(ATK_EINVAL, "conv: packed weights need %zu bytes", align256(pl.wp_bytes));
  switch (p.dtype) {
    case ATK_F32: return pack_ig<float>(p, pl, w, packed, s);
    case ATK_F16: return pack_ig<_Float16>(p, pl, w, packed, s);
    default: return pack_ig<__bf16>(p, pl, w, packed, s);
  }
}

size_t conv_igemm_gn_stats_bytes(const ConvShape& p, int v, int G) {
  if (v < 0 || v >= kNumIg) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl)) return 0;
  const int np = gn_records(p, pl, v, G);
  return np ? (size_t)p.N * G * np * sizeof(float4) : 0;
}

int conv_igemm_gn_records(const ConvShape& p, int v, int G) {
  if (v < 0 || v >= kNumIg) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl)) return 0;
  return gn_records(p, pl, v, G);
}

size_t conv_igemm_gn_onepass_bytes(const ConvShape& p, int v, int G) {
  if (v < 0 || v >= kNumIg || p.dtype == ATK_F32) return 0;
  IgPlan pl;
  if (plan_ig(p, v, pl, true) || !gn_reg_layout(pl, v, G > 0 && p.Co % G == 0 ? p.Co / G : 0)) return 0;
  const int np = gn_records(p, pl, v, G);
  return np ? gn_onepass_bytes(p, np, G) : 0;
}

int conv_igemm_run_gn_onepass(const ConvShape& p, const void* x, const void* packed, size_t packed_bytes,
                              const void* bias, const void* gamma, const void* beta, int param_dtype, float eps,
                              int silu, void* y, int v, int G, void* ws, size_t ws_bytes, hipStream_t s) {
  if (v < 0 || v >= kNumIg) return fail(ATK_EINVAL, "conv: variant out of range");
  if (p.dtype == ATK_F32) return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm takes 16-bit types");
  if (G <= 0 || p.Co % G) return fail(ATK_EINVAL, "conv: %d GroupNorm groups do not divide %d channels", G, p.Co);
  if (!dtype_ok(param_dtype)) return fail(ATK_EINVAL, "conv: unknown GroupNorm parameter dtype code %d", param_dtype);
  IgPlan pl;
  int rc = plan_ig(p, v, pl, true);
  if (rc) return rc;
  if (!packed || packed_bytes < align256(pl.wp_bytes))
    return fail(ATK_EINVAL, "conv: packed weights of %zu bytes expected", align256(pl.wp_bytes));
  if (pl.splits != 1) return fail(ATK_UNSUPPORTED, "conv: the one-pass GroupNorm needs an unsplit launch");
  const int np = gn_records(p, pl, v, G);
  if (!np) return fail(ATK_UNSUPPORTED, "conv: GroupNorm statistics need Co/G in {4, 8, 16, 32} or a multiple of 32");
  const size_t need = gn_onepass_bytes(p, np, G);
  if (!ws || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 255))
    return fail(ATK_EINVAL, "conv: the one-pass GroupNorm needs a 256-byte aligned workspace of %zu bytes", need);
  const GnOnePass op{gamma, beta, param_dtype, eps, silu ? 1 : 0, ws};
  if (p.dtype == ATK_F16) return run_ig<_Float16>(p, pl, x, packed, bias, y, v, nullptr, s, nullptr, nullptr, G, false, &op);
  return run_ig<__bf16>(p, pl, x, packed, bias, y, v, nullptr, s, nullptr, nullptr, G, false, &op);
}

int conv_igemm_run_prepacked(const ConvShape& p, const void* x, const void* packed, size_t packed_bytes,
                             const void* bias, void* y, int v, void* ws, size_t ws_bytes, hipStream_t s,
                             const void* resid, void* gn_stats, size_t gn_stats_bytes, int gn_G, bool cl) {
  if (v < 0 || v >= kNumIg) return fail(ATK_EINVAL, "conv: variant out of range");
  const int64_t ysz = (int64_t)p.N * p.Co * p.Do * p.Ho * p.Wo;
  if (ysz >= (1ll << 31)) return fail(ATK_UNSUPPORTED, "conv: output too large for the split-K finalize");
  IgPlan pl;
  int rc = plan_ig(p, v, pl);
  if (rc) return rc;
  if (!packed || packed_bytes < align256(pl.wp_bytes))
    return fail(ATK_EINVAL, "conv: packed weights of %zu bytes expected", align256(pl.wp_bytes));
  if (pl.part_bytes && (!ws || ws_bytes < pl.part_bytes))
    return fail(ATK_EINVAL, "conv: workspace of %zu bytes needed", pl.part_bytes);
  float* part = static_cast<float*>(ws);
  float4* gp = nullptr;
  if (gn_stats) {
    const int np = gn_records(p, pl, v, gn_G);
    if (!np) return fail(ATK_UNSUPPORTED, "conv: this variant cannot write GroupNorm statistics for the shape");
    const size_t need = (size_t)p.N * gn_G * np * sizeof(float4);
    if (gn_stats_bytes < need) return fail(ATK_EINVAL, "conv: GroupNorm statistics need %zu bytes", need);
    gp = static_cast<float4*>(gn_stats);
  }
  switch (p.dtype) {
    case ATK_F32: return run_ig<float>(p, pl, x, packed, bias, y, v, part, s, resid, gp, gn_G, cl);
    case ATK_F16: return run_ig<_Float16>(p, pl, x, packed, bias, y, v, part, s, resid, gp, gn_G, cl);
    default: return run_ig<__bf16>(p, pl, x, packed, bias, y, v, part, s, resid, gp, gn_G, cl);
  }
}

int conv_igemm_launch(const ConvShape& p, const void* x, const void* w, const void* bias, void* y, int v,
                      void* ws, size_t ws_bytes, hipStream_t s) {
  if (v < 0 || v >= kNumIg) return fail(ATK_EINVAL, "conv: variant out of range");
  const int64_t ysz = (int64_t)p.N * p.Co * p.Do * p.Ho * p.Wo;
  if (ysz >= (1ll << 31)) return fail(ATK_UNSUPPORTED, "conv: output too large for the split-K finalize");
  switch (p.dtype) {
    case ATK_F32: return launch_ig<float>(p, x, w, bias, y, v, ws, ws_bytes, s);
    case ATK_F16: return launch_ig<_Float16>(p, x, w, bias, y, v, ws, ws_bytes, s);
    default: return launch_ig<__bf16>(p, x, w, bias, y, v, ws, ws_bytes, s);
  }
}

}  // namespace atk
