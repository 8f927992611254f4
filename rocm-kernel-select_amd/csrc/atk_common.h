// Shared device/host helpers for the gfx950 kernels of libamd_tuned_torch_hip.so.
//
// Element types: float, _Float16 and __bf16 (clang's native types; on gfx950 the
// f32->bf16 conversion lowers to the hardware round-to-nearest-even convert, which
// is the rounding PyTorch applies when it narrows an fp32 result).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/amd_tuned_torch_hip.h"

namespace atk {

// ---------------------------------------------------------------------------
// Host-side error reporting (thread-local message behind atk_last_error()).
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
int device_cu_count();
// Frequency of the device's constant wall clock (wall_clock64()) in kHz, 0 on error.
int device_wall_clock_khz();

inline size_t dtype_size(int dtype) { return dtype == ATK_F32 ? 4 : 2; }
inline bool dtype_ok(int dtype) { return dtype == ATK_F32 || dtype == ATK_F16 || dtype == ATK_BF16; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Element conversions.
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(T v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

// Runtime-typed scalar load (affine parameters, per-channel bias): cheap, used
// off the streaming path only.
__device__ __forceinline__ float load_param(const void* p, int dtype, int64_t i) {
  if (dtype == ATK_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == ATK_F16) return static_cast<float>(reinterpret_cast<const _Float16*>(p)[i]);
  return static_cast<float>(reinterpret_cast<const __bf16*>(p)[i]);
}

// 16-byte vector of elements, reinterpretable as raw dwords.
template <typename T> struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  union {
    uint4 raw;
    T e[N];
  };
};

// SiLU v * sigmoid(v) with the hardware exp2 and reciprocal (about 1 ulp each); exp(-v)
// overflowing to +inf gives v * 0 = -0 for very negative v, as the exact formula does.
__device__ __forceinline__ float silu_f32(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}

// 16-byte global accesses with an optional nontemporal (streaming) hint: data read or
// written exactly once should not displace reusable lines in L2 / MALL.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
  uint4 r;
  if (NT) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    r.x = v.x; r.y = v.y; r.z = v.z; r.w = v.w;
  } else {
    r = *reinterpret_cast<const uint4*>(p);
  }
  return r;
}
// 16 bytes of T from VEC = 16 / sizeof(T) fp32 values, round-to-nearest-even, converted in
// pairs (v_cvt_pk_bf16_f32 for bf16) rather than one element at a time.
template <typename T>
__device__ __forceinline__ uint4 pack16(const float* v) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
  } else {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f2 pr = {v[2 * i], v[2 * i + 1]};
      d[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pr, t2));
    }
    return make_uint4(d[0], d[1], d[2], d[3]);
  }
}

template <bool NT>
__device__ __forceinline__ void st16(void* p, uint4 r) {
  if (NT) {
    u32x4 v = {r.x, r.y, r.z, r.w};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = r;
  }
}

// ---------------------------------------------------------------------------
// Raw buffer access (gfx9 buffer resource, stride 0): a 32-bit lane offset plus a uniform
// SGPR offset, and offsets at or beyond `bytes` read as zero -- used both to keep address
// arithmetic off the VALU and to zero-fill masked loads without branches (a branch per
// masked load makes the compiler wait for each load inside its branch).
// ---------------------------------------------------------------------------
constexpr uint32_t kOOB = 0x80000000u;  // >= every num_records used: reads zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// AUX: cache-policy bits of the instruction (0 = default, 2 = nontemporal)
template <int AUX = 0>
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// (No buffer stores: 16-byte buffer stores with an SGPR offset produced sporadically wrong
// output values on gfx950 in workgroups of >= 512 threads; stores use global_store.)
template <typename T>
__device__ __forceinline__ T bload_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  if constexpr (sizeof(T) == 2) {
    const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, 0, 0);
    return __builtin_bit_cast(T, u);
  } else {
    const unsigned int u = __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, 0);
    return __builtin_bit_cast(T, u);
  }
}

// ---------------------------------------------------------------------------
// Wave64 / block reductions (fp32 sums).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the wave on the VALU: DPP swaps inside quads (xor 1, xor 2), then half-row and row
// mirrors give every lane its 16-lane row's sum; the four row sums are read out by lane reads
// and added in row order.  The result is wave-uniform and its order fixed.  Unlike wave_sum
// (LDS-pipe permutes, each waited for in turn) independent calls interleave freely.  Every lane
// of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_rows(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return ((r0 + r1) + r2) + r3;
}

// Sum over the block; every thread receives the total.  `red` must hold
// blockDim/64 floats of shared memory.  Contains two __syncthreads().
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  constexpr int NW = NT / 64;
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (NW == 1) return v;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];  // identical order in every thread
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------
// Division by a runtime-invariant divisor d (1 <= d < 2^31) for numerators
// n < 2^31:  q = (umulhi(n, m) + n) >> s   (round-up multiplier method,
// Granlund & Montgomery 1994, "Division by invariant integers using
// multiplication").
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;  // s = ceil(log2 d)
  f.s = s;
  f.m = (uint32_t)((((1ull << s) - d) << 32) / d + 1);
  if (d == 1) { f.m = 0; f.s = 0; }
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

}  // namespace atk
