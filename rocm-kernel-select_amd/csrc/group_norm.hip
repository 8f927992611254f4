// GroupNorm (+ optional fused SiLU) forward for gfx950.
//
//   y = act( (x - mean_g) * rsqrt(var_g + eps) * gamma_c + beta_c )
//
// Semantics of the reference's native kernel (src/cuda/group_norm.cu:41-104: one group =
// the C/G * S contiguous elements of (n, g), population variance, eps inside the rsqrt,
// optional affine) and of its fused GroupNorm+SiLU (amd_tuned_torch/conv_fusion_ops.py:
// 192-242).  The statistics differ deliberately: the reference computes E[x^2]-E[x]^2
// (group_norm.cu:93); here they are exact two-pass values, mean first and then the sum of
// squared deviations, merged across workgroups with Chan, Golub & LeVeque's pairwise
// formula  M2 = sum M2_i + sum n_i (mean_i - mean)^2.
//
// Variants
//   res_*    Register-resident single pass.  A group is cut into NS slices of
//            NT threads x EPV 16-byte vectors; each workgroup loads its slice ONCE into
//            registers, reduces it twice (sum, then squared deviations about the slice
//            mean) and, when NS > 1, publishes its (mean, M2) in a workspace slot.  One
//            wave then collects the group's slots, lanes polling different slots.  A slot
//            that has not appeared within a wall-clock bound is computed by the waiting
//            workgroup itself, from x, with arithmetic identical to the owner's, so no
//            workgroup ever depends on another being scheduled (no cooperative launch, no
//            deadlock when the grid exceeds what is resident) and every workgroup of a
//            group derives bit-identical statistics.  The last workgroup of a group to
//            finish reading (a per-group counter) clears the group's slots, so every
//            launch starts from empty slots -- also when replayed from a HIP graph.
//            HBM traffic: one read + one write of the tensor.
//   twopass  Streaming fallback for any size / alignment: a statistics kernel writes
//            per-slice (mean, M2) partials, an apply kernel merges them and normalises.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "atk_common.h"

namespace atk {

namespace {

constexpr int GN_MAX_NS = 4096;      // slices per group, two-pass
constexpr int GN_RES_MAX_NS = 1024;  // slices per group, register-resident (LDS slot table)
constexpr uint32_t GN_WAIT_US = 200; // wait for a slot before computing it locally
// Workspace layout is FIXED (independent of the shape) so that calls of different shapes
// sharing one workspace never see each other's state:
//   [0, 256)                    diagnostics word (set when a wait timed out)
//   [256, GN_SLOTS_OFF)         per-group "done reading" counters (register-resident)
//   [GN_SLOTS_OFF, GN_ZERO_BYTES) register-resident slots, 16 B each
//   [GN_PARTIALS_OFF, ...)      two-pass (mean, M2) partials
// Everything below GN_ZERO_BYTES is zeroed once, at allocation, and every launch leaves
// it zero again (apart from the diagnostics word).
constexpr int GN_MAX_SLOTTED = 4096;   // groups a multi-slice register-resident launch may have
constexpr int GN_MAX_SLOTS = 65536;    // groups x slices of such a launch
constexpr size_t GN_SLOTS_OFF = 256 + 8 * (size_t)GN_MAX_SLOTTED;
constexpr size_t GN_ZERO_BYTES = GN_SLOTS_OFF + 16 * (size_t)GN_MAX_SLOTS;
constexpr size_t GN_PARTIALS_OFF = GN_ZERO_BYTES;
constexpr int GN_TP_NT = 256;                 // two-pass kernels
constexpr int GN_BWD_U = 4;                   // backward: vectors of x and dy in flight per thread (most)
constexpr int GN_MAX_AFF = 512;               // channels per slice whose affine is staged in LDS

// One slot = two 64-bit words (tag << 32 | bits(mean)), (tag << 32 | bits(M2)), each
// stored and read with single-copy-atomic relaxed agent-scope accesses: a reader that sees
// this launch's tag in both words has both values, with no fence on either side
// (agent-scope acquire/release would write back / invalidate the XCD's L2 on every poll).
// The tag is a nonzero per-launch number chosen by the host, so a slot left over from any
// other launch (another shape, another tensor) never passes for this launch's; empty = 0.
struct GnSlot {
  unsigned long long w[2];
};

struct GnArgs {
  const void* x;
  const void* gamma;
  const void* beta;
  void* y;
  int64_t E;          // elements per group = cpg * S
  uint32_t S, cpg, G;
  int NS;             // slices per group
  int64_t slice;      // elements per slice (multiple of the vector width)
  float eps;
  int silu;
  int pdt;            // dtype of gamma/beta
  FastDiv div_s;
  uint64_t wait_ticks;// wall-clock ticks to wait for a slot
  uint32_t tag;       // this launch's slot marker (nonzero)
  uint32_t* diag;     // workspace: diagnostics word
  uint32_t* done;     // workspace: [ngroups] workgroups that finished reading the slots
  GnSlot* slots;      // workspace: [ngroups][NS] (register-resident)
  float* partials;    // workspace: [ngroups][NS][2] (mean, M2) (two-pass)
  float4* parts;      // split kernels: [ngroups][NP] records (count, mean, M2, -)
  int NP;             // records per group
  uint64_t* trace;    // resident kernel, diagnostics: [workgroup][4] wall-clock stamps, or null
};

// Phase trace of the register-resident kernel (atk_group_norm_trace): thread 0 of every
// workgroup stamps the wall clock at entry, when its slice statistics are done (all its loads
// have arrived), when the group statistics are known (after the exchange) and when its stores
// are issued.  A process-wide registration read at launch; null = off.
uint64_t* g_gn_trace = nullptr;
int64_t g_gn_trace_words = 0;
__device__ __forceinline__ void gn_stamp(const GnArgs& a, int k) {
  if (a.trace && threadIdx.x == 0) a.trace[(int64_t)blockIdx.x * 4 + k] = wall_clock64();
}

__device__ __forceinline__ int64_t slice_len(int i, int64_t slice, int64_t E) {
  return (int64_t)(i + 1) * slice <= E ? slice : E - (int64_t)i * slice;
}

// Merge NS (mean, M2) partials on one wave (call with all 64 lanes of wave 0):
//   mean = sum n_i mean_i / E,   M2 = sum (M2_i + n_i (mean_i - mean)^2).
// Lane l takes i = l, l+64, ... in order; the xor-butterfly then gives every lane the
// same, order-fixed total, so every workgroup of a group derives bit-identical values.
template <typename GetMean, typename GetM2>
__device__ __forceinline__ void wave_merge(int NS, int64_t slice, int64_t E, GetMean gm, GetM2 g2,
                                           float& mean, float& var) {
  const int lane = threadIdx.x & 63;
  float sm = 0.f;
  for (int i = lane; i < NS; i += 64) sm += (float)slice_len(i, slice, E) * gm(i);
  mean = wave_sum(sm) / (float)E;
  float m2 = 0.f;
  for (int i = lane; i < NS; i += 64) {
    const float d = gm(i) - mean;
    m2 += g2(i) + (float)slice_len(i, slice, E) * d * d;
  }
  var = wave_sum(m2) / (float)E;
}

// The dword holding element i of a gamma/beta array of n elements (dtype pdt; p may be
// null or 2-byte aligned), loaded through a resource that covers the array rounded out to
// whole dwords: unconditional, branch-free, and out-of-range (or null) reads return 0.
// `sel` says which half holds a 16-bit element.
__device__ __forceinline__ uint32_t param_word(const void* p, int pdt, int64_t i, int64_t n, uint32_t& sel) {
  const uint32_t es = pdt == ATK_F32 ? 4u : 2u;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uint32_t mis = (uint32_t)(addr & 3u);
  const uint32_t bytes = p ? (uint32_t)(((int64_t)mis + n * es + 3) & ~(int64_t)3) : 0u;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(reinterpret_cast<const void*>(addr - mis), bytes);
  const uint32_t off = mis + (uint32_t)i * es;
  sel = off & 2u;
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)(off & ~3u), 0, 0);
}

__device__ __forceinline__ float param_decode(uint32_t w, uint32_t sel, int pdt) {
  if (pdt == ATK_F32) return __uint_as_float(w);
  const unsigned short h = (unsigned short)(sel ? (w >> 16) : (w & 0xffffu));
  return pdt == ATK_F16 ? (float)__builtin_bit_cast(_Float16, h) : (float)__builtin_bit_cast(__bf16, h);
}

// scale/shift of absolute channel `c` given the group statistics
__device__ __forceinline__ void channel_affine(const GnArgs& a, int64_t c, float mean, float rstd,
                                               float& sc, float& sh) {
  const float gm = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
  const float bt = a.beta ? load_param(a.beta, a.pdt, c) : 0.f;
  sc = rstd * gm;
  sh = bt - mean * sc;
}

// SiLU is a template parameter: as a runtime flag the compiler evaluates it for every
// element (two quarter-rate transcendentals each) and selects.
template <typename T, bool SILU>
__device__ __forceinline__ uint4 normalize_vec(const Vec16<T>& in, float sc, float sh) {
  constexpr int VEC = 16 / sizeof(T);
  float v[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    v[k] = fmaf(to_f32(in.e[k]), sc, sh);
    if constexpr (SILU) v[k] = silu_f32(v[k]);
  }
  return pack16<T>(v);
}

// ---------------------------------------------------------------------------------------
// Register-resident single pass.  Requires S % VEC == 0 and 16B-aligned x / y (host check).
// ---------------------------------------------------------------------------------------
// Opaque to the optimiser: keeps it from holding all VEC*EPV elements converted to fp32
// across phases (that doubles the registers and spills); reconverting is a few VALU ops.
template <typename T, int EPV>
__device__ __forceinline__ void reg_fence(Vec16<T>* buf) {
#pragma unroll
  for (int i = 0; i < EPV; ++i)
    asm volatile("" : "+v"(buf[i].raw.x), "+v"(buf[i].raw.y), "+v"(buf[i].raw.z), "+v"(buf[i].raw.w));
}

// Statistics of one slice of a group, in one pass over the data as it arrives.  Each thread
// accumulates d = x - K, sum d and sum d^2, about K = its own first element, and turns them
// into its (n_t, mean_t, M2_t = sum d^2 - (sum d)^2 / n_t); K being one of its values bounds
// the cancellation (sum d^2 <= (n_t + 1) M2_t).  The block then merges the threads exactly:
// mean = sum n_t mean_t / n, M2 = sum M2_t + n_t (mean_t - mean)^2.  Element order is
// i = 0..EPV-1 (vector i of this thread = element s0 + (i*NT + tid)*VEC), k = 0..VEC-1, with
// plain adds and explicit fmas, then fixed-order block reductions.  The owner runs it on its
// registers (FROM_REG), a workgroup standing in for a late owner runs it on memory with
// rolled loops; the arithmetic, and so every bit, is the same.
template <typename T, int NT, int EPV, bool FROM_REG>
__device__ __forceinline__ void slice_stats(Vec16<T>* buf, const T* xg, int64_t s0, int64_t E,
                                            int64_t slice, float* red, float& mean_l, float& m2) {
  constexpr int VEC = 16 / sizeof(T);
  const int tid = threadIdx.x;
  const int64_t nv = (E - s0) / VEC;  // vectors from s0 to the group end (E % VEC == 0)
  auto valid = [&](int i) { return (int64_t)i * NT + tid < nv; };
  auto get = [&](int i) -> Vec16<T> {
    if constexpr (FROM_REG) {
      return buf[i];
    } else {
      Vec16<T> v;
      if (valid(i)) v.raw = *reinterpret_cast<const uint4*>(xg + s0 + ((int64_t)i * NT + tid) * VEC);
      else v.raw = make_uint4(0u, 0u, 0u, 0u);
      return v;
    }
  };
  // vector 0 is the thread's first; a thread without it has no element in the slice
  const float K = to_f32(get(0).e[0]);
  float s1 = 0.f, s2 = 0.f;
  int nvt = 0;
  // branch-free: a vector past the group end reads as zeros and is shifted by 0, so it adds
  // exactly nothing.  On registers, vector i is fenced together with the running sums: it
  // is converted only after vector i-1 is accumulated (left free, the compiler converts
  // every vector up front and spills the fp32 copies).
  auto acc = [&](int i) {
    const bool ok = valid(i);
    const float Ki = ok ? K : 0.f;
    if constexpr (FROM_REG)
      asm volatile("" : "+v"(buf[i].raw.x), "+v"(buf[i].raw.y), "+v"(buf[i].raw.z), "+v"(buf[i].raw.w),
                   "+v"(s1), "+v"(s2));
    const Vec16<T> v = get(i);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = to_f32(v.e[k]) - Ki;
      s1 += d;
      s2 = fmaf(d, d, s2);
    }
    nvt += ok ? 1 : 0;
  };
  if constexpr (FROM_REG) {
#pragma unroll
    for (int i = 0; i < EPV; ++i) acc(i);
  } else {
#pragma unroll 1
    for (int i = 0; i < EPV; ++i) acc(i);
  }
  const float nt = (float)(nvt * VEC);
  float mean_t = 0.f, m2_t = 0.f;
  if (nvt > 0) {
    const float q = s1 / nt;
    mean_t = K + q;
    m2_t = fmaxf(fmaf(-s1, q, s2), 0.f);
  }
  const int64_t n_l = (E - s0) < slice ? (E - s0) : slice;
  mean_l = block_sum<NT>(nt * mean_t, red) / (float)n_l;
  const float dm = mean_t - mean_l;
  m2 = block_sum<NT>(fmaf(nt * dm, dm, m2_t), red);
  if constexpr (FROM_REG) reg_fence<T, EPV>(buf);
}

// ---------------------------------------------------------------------------------------
// Register-resident single pass.  Requires S % VEC == 0 and 16B-aligned x / y (host check).
// ---------------------------------------------------------------------------------------
// Up to 16 vectors per thread fit 128 VGPRs: four waves per SIMD, so two 512-thread (or
// four 256-thread) workgroups share a CU -- left alone, the fp16 build of EPV = 16 takes
// 144 and halves the residency that a multi-slice launch relies on.
template <typename T, int NT, int EPV, bool SILU>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(EPV <= 16 ? 4 : 1)))
void gn_resident_kernel(GnArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float red[NT / 64];
  __shared__ float s_stat[2];
  __shared__ float aff[2 * GN_MAX_AFF];  // scale[ ], shift[ ] of the slice's channels
  __shared__ float sl_mean[GN_RES_MAX_NS], sl_m2[GN_RES_MAX_NS];
  __shared__ int s_missing[GN_RES_MAX_NS + 1];  // [0] = count, then slice indices

  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;
  T* __restrict__ yg = static_cast<T*>(a.y) + gi * E;
  gn_stamp(a, 0);

  // All EPV loads in flight at once, branch-free: one lane offset (tid*16 B) plus a
  // uniform SGPR offset per vector; lanes past the group take an out-of-range offset and
  // read 0 (and, below, store nothing).  Offsets are bytes from the group start (< 2^31).
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xg, (uint32_t)(E * (int64_t)sizeof(T)));
  const uint32_t lane_off = (uint32_t)tid * 16u;
  const uint32_t n_vec = (uint32_t)((E - s0 + VEC - 1) / VEC);  // vectors of this slice in the group
  auto voff = [&](int i) { return (uint32_t)(i * NT + tid) < n_vec ? lane_off : kOOB; };
  auto soff = [&](int i) { return (uint32_t)((s0 + (int64_t)i * NT * VEC) * (int64_t)sizeof(T)); };
  Vec16<T> buf[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) buf[i].raw = bload16<2>(rx, voff(i), soff(i));

  // gamma/beta of the channels this slice spans (group-local [c_lo, c_hi)): thread t fetches
  // channel t now, while x is in flight, with unconditional buffer loads that nothing waits
  // for until the statistics are done (a plain load here is waited for with vmcnt(0), which
  // also waits for every x load and keeps the sums from overlapping their arrival).
  const int64_t last = (s0 + a.slice < E ? s0 + a.slice : E) - 1;
  const uint32_t c_lo = fdiv((uint32_t)s0, a.div_s);
  const uint32_t c_hi = fdiv((uint32_t)last, a.div_s) + 1;
  const int nch = (int)(c_hi - c_lo);
  const int64_t cabs0 = (int64_t)(gi % a.G) * a.cpg + c_lo;  // absolute channel of c_lo
  const bool staged = nch <= GN_MAX_AFF;
  const int64_t nchan = (int64_t)a.G * a.cpg;
  const int64_t cme = cabs0 + (tid < nch ? tid : 0);
  uint32_t gsel, bsel;
  const uint32_t gword = param_word(a.gamma, a.pdt, cme, nchan, gsel);
  const uint32_t bword = param_word(a.beta, a.pdt, cme, nchan, bsel);

  float mean_l, m2;
  slice_stats<T, NT, EPV, true>(buf, xg, s0, E, a.slice, red, mean_l, m2);
  gn_stamp(a, 1);
  if (staged) {
    if (tid < nch) {
      aff[tid] = a.gamma ? param_decode(gword, gsel, a.pdt) : 1.f;
      aff[GN_MAX_AFF + tid] = a.beta ? param_decode(bword, bsel, a.pdt) : 0.f;
    }
    for (int i = tid + NT; i < nch; i += NT) {
      aff[i] = a.gamma ? load_param(a.gamma, a.pdt, cabs0 + i) : 1.f;
      aff[GN_MAX_AFF + i] = a.beta ? load_param(a.beta, a.pdt, cabs0 + i) : 0.f;
    }
  }

  float mean, var;
  if (a.NS == 1) {
    mean = mean_l;
    var = m2 / (float)((E - s0) < a.slice ? (E - s0) : a.slice);
  } else {
    GnSlot* slots = a.slots + gi * (int64_t)a.NS;
    const unsigned long long hi = (unsigned long long)a.tag << 32;
    if (tid == 0) {
      __hip_atomic_store(&slots[s].w[0], hi | __float_as_uint(mean_l), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&slots[s].w[1], hi | __float_as_uint(m2), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      // the publish completes before this workgroup counts itself done (below, after its
      // stores), so the last workgroup's clear can never be overtaken by a late publish, which
      // would leave a filled slot behind (the barrier that follows waits for it anyway)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      s_missing[0] = 0;
    }
    __syncthreads();
    if (tid < 64) {
      // collect the group's slots, one lane per slot; wait at most wait_ticks in total
      const uint64_t t0 = wall_clock64();
      for (int j = tid; j < a.NS; j += 64) {
        bool ok;
        if (j == s) {
          ok = true;
          sl_mean[j] = mean_l;
          sl_m2[j] = m2;
        } else {
          unsigned long long w0, w1;
          for (;;) {
            w0 = __hip_atomic_load(&slots[j].w[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            w1 = __hip_atomic_load(&slots[j].w[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = (w0 >> 32) == a.tag && (w1 >> 32) == a.tag;
            if (ok || wall_clock64() - t0 > a.wait_ticks) break;
            __builtin_amdgcn_s_sleep(1);
          }
          if (ok) {
            sl_mean[j] = __uint_as_float((uint32_t)w0);
            sl_m2[j] = __uint_as_float((uint32_t)w1);
          }
        }
        if (!ok) s_missing[1 + atomicAdd(&s_missing[0], 1)] = j;
      }
    }
    __syncthreads();
    const int nmiss = s_missing[0];
    if (nmiss > 0) {
      // stand in for late owners: the same statistics, computed from x
      if (tid == 0) __hip_atomic_store(a.diag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int m = 0; m < nmiss; ++m) {
        const int j = s_missing[1 + m];
        const int64_t j0 = (int64_t)j * a.slice;
        float mj, qj;
        slice_stats<T, NT, EPV, false>(nullptr, xg, j0, E, a.slice, red, mj, qj);
        if (tid == 0) {
          sl_mean[j] = mj;
          sl_m2[j] = qj;
        }
      }
      __syncthreads();
    }
    if (tid < 64) {
      wave_merge(a.NS, a.slice, E, [&](int i) { return sl_mean[i]; }, [&](int i) { return sl_m2[i]; },
                 mean, var);
      if (tid == 0) {
        s_stat[0] = mean;
        s_stat[1] = var;
      }
    }
    __syncthreads();
    mean = s_stat[0];
    var = s_stat[1];
  }
  const float rstd = 1.0f / sqrtf(var + a.eps);
  gn_stamp(a, 2);

  if (staged) {
    for (int i = tid; i < nch; i += NT) {  // the entries this thread fetched above
      const float sc = rstd * aff[i];
      aff[GN_MAX_AFF + i] = aff[GN_MAX_AFF + i] - mean * sc;
      aff[i] = sc;
    }
  }
  __syncthreads();

  if (staged) {
    // Offsets recomputed from an opaque copy of tid: reusing the load phase's per-vector
    // offsets would keep EPV more registers alive across the reductions.
    int tid_s = tid;
    asm volatile("" : "+v"(tid_s));
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      // vector i is unpacked only after store i-1 has issued: left free, the fp16 build
      // splits every packed pair up front and spills the halves
      reg_fence<T, 1>(&buf[i]);
      const bool ok = (uint32_t)(i * NT + tid_s) < n_vec;
      const int64_t e = ok ? s0 + ((int64_t)i * NT + tid_s) * VEC : s0;
      const int cl = (int)(fdiv((uint32_t)e, a.div_s) - c_lo);
      if (ok) st16<true>(yg + e, normalize_vec<T, SILU>(buf[i], aff[cl], aff[GN_MAX_AFF + cl]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      const int64_t e = s0 + ((int64_t)i * NT + tid) * VEC;
      if (e < E) {
        const int cl = (int)(fdiv((uint32_t)e, a.div_s) - c_lo);
        float sc, sh;
        channel_affine(a, cabs0 + cl, mean, rstd, sc, sh);
        st16<true>(yg + e, normalize_vec<T, SILU>(buf[i], sc, sh));
      }
    }
  }
  gn_stamp(a, 3);
  if (a.NS > 1 && tid < 64) {
    // This workgroup is done with the slots (every read of them returned before the barrier
    // above) and its publish completed: count it, after its stores are issued, so that the
    // atomic's round trip overlaps them rather than delaying them.  The last of the group's NS
    // workgroups to count itself -- every one has published and finished reading by then --
    // empties the slots for the next launch and resets the counter.
    GnSlot* slots = a.slots + gi * (int64_t)a.NS;
    uint32_t prev = 0;
    if (tid == 0) prev = __hip_atomic_fetch_add(a.done + gi, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (prev == (uint32_t)a.NS - 1) {
      for (int j = tid; j < a.NS; j += 64) {
        __hip_atomic_store(&slots[j].w[0], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&slots[j].w[1], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (tid == 0) __hip_atomic_store(a.done + gi, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Split GroupNorm: a statistics kernel and an apply kernel.  For groups too large for one
// workgroup's registers, the register-resident kernel exchanges slice statistics between
// workgroups inside one launch; here the launch boundary is the exchange.  The statistics
// kernel loads its slice with every 16-byte load in flight (cached: the apply kernel reads
// x again, from L2 / the Infinity Cache) and writes one record (count, mean, M2) per slice;
// the apply kernel issues its loads, merges the group's records on one wave meanwhile, and
// normalises from registers.  The records have explicit counts, so the apply kernel also
// takes statistics written by other producers (the conv epilogue).
// ---------------------------------------------------------------------------------------
// Merge NP (count, mean, M2) records on one wave (all 64 lanes of wave 0), in a fixed order:
//   n = sum n_i,  mean = sum n_i mean_i / n,  M2 = sum (M2_i + n_i (mean_i - mean)^2).
// Lane l takes records l, l+64, ...; up to 64 * RC of them are read once and kept in registers
// for the second sum.  The xor-butterfly sums give every lane (and every workgroup merging the
// same records) bit-identical statistics.
constexpr int GN_MERGE_RC = 8;  // records per lane held in registers by wave_merge_counted

// The first 64 * GN_MERGE_RC records of a group, lane l holding l, l+64, ...: loaded by the
// caller before anything else it waits for less urgently (vector-memory loads complete in
// issue order, so records loaded after x would wait for x).
template <typename GetRec>
__device__ __forceinline__ void load_records(int NP, GetRec rec, float4 (&r)[GN_MERGE_RC]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < GN_MERGE_RC; ++k)
    r[k] = lane + 64 * k < NP ? rec(lane + 64 * k) : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <typename GetRec>
__device__ __forceinline__ void wave_merge_counted(int NP, GetRec rec, const float4 (&r)[GN_MERGE_RC], float& mean,
                                                   float& var) {
  constexpr int RC = GN_MERGE_RC;
  const int lane = threadIdx.x & 63;
  float sn = 0.f, sm = 0.f;
#pragma unroll
  for (int k = 0; k < RC; ++k) {
    sn += r[k].x;
    sm = fmaf(r[k].x, r[k].y, sm);
  }
  for (int i = lane + 64 * RC; i < NP; i += 64) {
    const float4 x = rec(i);
    sn += x.x;
    sm = fmaf(x.x, x.y, sm);
  }
  const float n = wave_sum(sn);
  mean = wave_sum(sm) / n;
  float m2 = 0.f;
#pragma unroll
  for (int k = 0; k < RC; ++k) {
    const float d = r[k].y - mean;
    m2 += r[k].z + r[k].x * d * d;
  }
  for (int i = lane + 64 * RC; i < NP; i += 64) {
    const float4 x = rec(i);
    const float d = x.y - mean;
    m2 += x.z + x.x * d * d;
  }
  var = wave_sum(m2) / n;
}

template <typename T, int NT, int EPV>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(EPV <= 16 ? 4 : 1)))
void gn_split_stats_kernel(GnArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float red[NT / 64];
  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xg, (uint32_t)(E * (int64_t)sizeof(T)));
  const uint32_t lane_off = (uint32_t)tid * 16u;
  const uint32_t n_vec = (uint32_t)((E - s0 + VEC - 1) / VEC);
  Vec16<T> buf[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i)
    buf[i].raw = bload16(rx, (uint32_t)(i * NT + tid) < n_vec ? lane_off : kOOB,
                         (uint32_t)((s0 + (int64_t)i * NT * VEC) * (int64_t)sizeof(T)));
  float mean_l, m2;
  slice_stats<T, NT, EPV, true>(buf, xg, s0, E, a.slice, red, mean_l, m2);
  if (tid == 0) {
    const float n_l = (float)((E - s0) < a.slice ? (E - s0) : a.slice);
    a.parts[gi * a.NP + s] = make_float4(n_l, mean_l, m2, 0.f);
  }
}

template <typename T, int NT, int EPV, bool SILU>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(EPV <= 16 ? 4 : 1)))
void gn_split_apply_kernel(GnArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float s_stat[2];
  __shared__ float aff[2 * GN_MAX_AFF];
  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;
  T* __restrict__ yg = static_cast<T*>(a.y) + gi * E;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xg, (uint32_t)(E * (int64_t)sizeof(T)));
  const uint32_t lane_off = (uint32_t)tid * 16u;
  const uint32_t n_vec = (uint32_t)((E - s0 + VEC - 1) / VEC);
  // the group's records first: merged while x is still arriving
  const float4* rp = a.parts + gi * a.NP;
  float4 rec[GN_MERGE_RC];
  if (tid < 64) load_records(a.NP, [&](int i) { return rp[i]; }, rec);
  Vec16<T> buf[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i)  // last read of x: nontemporal
    buf[i].raw = bload16<2>(rx, (uint32_t)(i * NT + tid) < n_vec ? lane_off : kOOB,
                            (uint32_t)((s0 + (int64_t)i * NT * VEC) * (int64_t)sizeof(T)));
  // the slice's channels and their gamma / beta words (unconditional buffer loads that
  // nothing waits for until the merge is done)
  const int64_t last = (s0 + a.slice < E ? s0 + a.slice : E) - 1;
  const uint32_t c_lo = fdiv((uint32_t)s0, a.div_s);
  const uint32_t c_hi = fdiv((uint32_t)last, a.div_s) + 1;
  const int nch = (int)(c_hi - c_lo);
  const int64_t cabs0 = (int64_t)(gi % a.G) * a.cpg + c_lo;
  const bool staged = nch <= GN_MAX_AFF;
  const int64_t nchan = (int64_t)a.G * a.cpg;
  const int64_t cme = cabs0 + (tid < nch ? tid : 0);
  uint32_t gsel, bsel;
  const uint32_t gword = param_word(a.gamma, a.pdt, cme, nchan, gsel);
  const uint32_t bword = param_word(a.beta, a.pdt, cme, nchan, bsel);
  if (tid < 64) {
    float mean, var;
    wave_merge_counted(a.NP, [&](int i) { return rp[i]; }, rec, mean, var);
    if (tid == 0) {
      s_stat[0] = mean;
      s_stat[1] = 1.0f / sqrtf(var + a.eps);
    }
  }
  __syncthreads();
  const float mean = s_stat[0], rstd = s_stat[1];
  if (staged) {
    if (tid < nch) {
      const float sc = rstd * (a.gamma ? param_decode(gword, gsel, a.pdt) : 1.f);
      aff[tid] = sc;
      aff[GN_MAX_AFF + tid] = (a.beta ? param_decode(bword, bsel, a.pdt) : 0.f) - mean * sc;
    }
    for (int i = tid + NT; i < nch; i += NT) {
      float sc, sh;
      channel_affine(a, cabs0 + i, mean, rstd, sc, sh);
      aff[i] = sc;
      aff[GN_MAX_AFF + i] = sh;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    reg_fence<T, 1>(&buf[i]);
    const bool ok = (uint32_t)(i * NT + tid) < n_vec;
    const int64_t e = ok ? s0 + ((int64_t)i * NT + tid) * VEC : s0;
    const int cl = (int)(fdiv((uint32_t)e, a.div_s) - c_lo);
    float sc, sh;
    if (staged) {
      sc = aff[cl];
      sh = aff[GN_MAX_AFF + cl];
    } else {
      channel_affine(a, cabs0 + cl, mean, rstd, sc, sh);
    }
    if (ok) st16<true>(yg + e, normalize_vec<T, SILU>(buf[i], sc, sh));
  }
}

// ---------------------------------------------------------------------------------------
// Two-pass streaming fallback.  VECOK: S % VEC == 0 and 16B-aligned pointers.
// ---------------------------------------------------------------------------------------
template <typename T, bool VECOK>
__global__ __launch_bounds__(GN_TP_NT) void gn_stats_kernel(GnArgs a) {
  constexpr int VEC = VECOK ? 16 / sizeof(T) : 1;
  __shared__ float red[GN_TP_NT / 64];
  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const int64_t s1 = s0 + a.slice < E ? s0 + a.slice : E;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;

  // per-thread running (n, mean, M2), merged one vector at a time
  float tn = 0.f, tmean = 0.f, tm2 = 0.f;
  for (int64_t e = s0 + (int64_t)tid * VEC; e < s1; e += (int64_t)GN_TP_NT * VEC) {
    float v[VEC];
    if (VECOK) {
      Vec16<T> b;
      b.raw = *reinterpret_cast<const uint4*>(xg + e);
#pragma unroll
      for (int k = 0; k < VEC; ++k) v[k] = to_f32(b.e[k]);
    } else {
      v[0] = to_f32(xg[e]);
    }
    float vm = 0.f;
#pragma unroll
    for (int k = 0; k < VEC; ++k) vm += v[k];
    vm *= (1.0f / VEC);
    float vm2 = 0.f;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = v[k] - vm;
      vm2 = fmaf(d, d, vm2);
    }
    const float nn = tn + (float)VEC;
    const float d = vm - tmean;
    const float f = (float)VEC / nn;
    tmean = fmaf(d, f, tmean);
    tm2 += vm2 + d * d * tn * f;
    tn = nn;
  }
  // block merge: mean_b = sum(n_t mean_t)/n_b ; M2_b = sum(M2_t + n_t (mean_t - mean_b)^2)
  const float nb = (float)(s1 - s0);
  const float mean_b = block_sum<GN_TP_NT>(tn * tmean, red) / nb;
  const float dd = tmean - mean_b;
  const float m2_b = block_sum<GN_TP_NT>(tm2 + tn * dd * dd, red);
  if (tid == 0) {
    float* p = a.partials + (gi * a.NS + s) * 2;
    p[0] = mean_b;
    p[1] = m2_b;
  }
}

template <typename T, bool VECOK, bool SILU>
__global__ __launch_bounds__(GN_TP_NT) void gn_apply_kernel(GnArgs a) {
  constexpr int VEC = VECOK ? 16 / sizeof(T) : 1;
  __shared__ float s_stat[2];
  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const int64_t s1 = s0 + a.slice < E ? s0 + a.slice : E;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;
  T* __restrict__ yg = static_cast<T*>(a.y) + gi * E;
  if (tid < 64) {
    const float* p = a.partials + gi * (int64_t)a.NS * 2;
    float mean, var;
    wave_merge(a.NS, a.slice, E, [&](int i) { return p[2 * i]; }, [&](int i) { return p[2 * i + 1]; },
               mean, var);
    if (tid == 0) {
      s_stat[0] = mean;
      s_stat[1] = 1.0f / sqrtf(var + a.eps);
    }
  }
  __syncthreads();
  const float mean = s_stat[0], rstd = s_stat[1];
  const int64_t cbase = (int64_t)(gi % a.G) * a.cpg;
  int64_t cur_c = -1;
  float sc = 0.f, sh = 0.f;
  for (int64_t e = s0 + (int64_t)tid * VEC; e < s1; e += (int64_t)GN_TP_NT * VEC) {
    const int64_t c = cbase + fdiv((uint32_t)e, a.div_s);
    if (c != cur_c) {
      channel_affine(a, c, mean, rstd, sc, sh);
      cur_c = c;
    }
    if (VECOK) {
      Vec16<T> b;
      b.raw = *reinterpret_cast<const uint4*>(xg + e);
      st16<true>(yg + e, normalize_vec<T, SILU>(b, sc, sh));
    } else {
      float v = fmaf(to_f32(xg[e]), sc, sh);
      if constexpr (SILU) v = silu_f32(v);
      yg[e] = from_f32<T>(v);
    }
  }
}

enum GnKind { GN_RESIDENT = 0, GN_TWOPASS = 1, GN_SPLIT = 2 };

struct GnVariant {
  const char* name;
  int nt, epv;  // threads per workgroup, 16-byte vectors per thread (two-pass: unused)
  int kind;
};

const GnVariant kGnVariants[] = {
    {"res_nt1024_v8", 1024, 8, GN_RESIDENT},
    {"res_nt1024_v16", 1024, 16, GN_RESIDENT},
    {"res_nt1024_v4", 1024, 4, GN_RESIDENT},
    {"res_nt512_v8", 512, 8, GN_RESIDENT},
    {"res_nt256_v8", 256, 8, GN_RESIDENT},
    {"res_nt256_v16", 256, 16, GN_RESIDENT},
    {"twopass", GN_TP_NT, 0, GN_TWOPASS},
    {"res_nt256_v4", 256, 4, GN_RESIDENT},
    {"res_nt512_v4", 512, 4, GN_RESIDENT},
    {"res_nt512_v16", 512, 16, GN_RESIDENT},
    {"res_nt512_v32", 512, 32, GN_RESIDENT},
    {"res_nt256_v32", 256, 32, GN_RESIDENT},
    {"split_nt256_v8", 256, 8, GN_SPLIT},
    {"split_nt512_v8", 512, 8, GN_SPLIT},
    {"split_nt256_v4", 256, 4, GN_SPLIT},
    {"split_nt1024_v4", 1024, 4, GN_SPLIT},
};
constexpr int kNumGn = sizeof(kGnVariants) / sizeof(kGnVariants[0]);

struct GnPlan {
  int NS;
  int64_t slice;
  size_t ws_bytes, zero_bytes;
  bool vec_ok;
};

inline size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

// Per-launch slot marker: a process-wide counter, never 0 (0 marks an empty slot).  A HIP
// graph replays the tag it captured; its launches still start from empty slots, because
// the last workgroup of every group clears them.
std::atomic<uint32_t> g_slot_tag{0};
uint32_t next_slot_tag() {
  uint32_t t = g_slot_tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
  while (t == 0u) t = g_slot_tag.fetch_add(1u, std::memory_order_relaxed) + 1u;
  return t;
}

// Slicing and workspace size (layout: see GN_ZERO_BYTES / GN_PARTIALS_OFF)
bool plan_gn(int64_t N, int64_t C, int64_t S, int G, int dtype, int variant, GnPlan& p) {
  const int64_t cpg = C / G;
  const int64_t E = cpg * S;
  const int64_t ngroups = N * G;
  const int vec = (int)(16 / dtype_size(dtype));
  const GnVariant& v = kGnVariants[variant];
  if (v.kind != GN_TWOPASS) {
    p.slice = (int64_t)v.nt * v.epv * vec;
    p.NS = (int)((E + p.slice - 1) / p.slice);
    if (v.kind == GN_RESIDENT && p.NS > GN_RES_MAX_NS) return false;
    if (E * (int64_t)dtype_size(dtype) >= (int64_t)kOOB) return false;  // 32-bit buffer offsets
  } else {
    // aim for >= ~2048 workgroups, slices of at least 4K elements
    int64_t ns = (2048 + ngroups - 1) / (ngroups > 0 ? ngroups : 1);
    const int64_t max_ns = (E + 4095) / 4096;
    if (ns > max_ns) ns = max_ns;
    if (ns < 1) ns = 1;
    if (ns > GN_MAX_NS) ns = GN_MAX_NS;
    int64_t sl = (E + ns - 1) / ns;
    sl = (sl + vec - 1) / vec * vec;
    p.slice = sl;
    p.NS = (int)((E + sl - 1) / sl);
  }
  if (p.NS > GN_MAX_NS) return false;
  p.zero_bytes = GN_ZERO_BYTES;
  const size_t rec = v.kind == GN_TWOPASS ? 8 : v.kind == GN_SPLIT ? 16 : 0;
  p.ws_bytes = GN_PARTIALS_OFF + round256((size_t)ngroups * p.NS * rec);
  return true;
}

template <typename T, int NT, int EPV, bool SILU>
int launch_resident_s(GnArgs a, int64_t ngroups, hipStream_t s) {
  const int64_t nblk = ngroups * a.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm: grid too large");
  auto kern = gn_resident_kernel<T, NT, EPV, SILU>;
  if (a.NS > 1) {
    if (ngroups > GN_MAX_SLOTTED || nblk > GN_MAX_SLOTS)
      return fail(ATK_UNSUPPORTED, "group_norm: %lld groups x %d slices exceed the slot table",
                  (long long)ngroups, a.NS);
    // Correct at any grid size (late slices are computed by the waiting workgroups),
    // but only fast when every workgroup of the grid can be resident at once.
    static int per_cu_cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
      return fail(ATK_ELAUNCH, "group_norm: no current device");
    if (per_cu_cache[dev] == 0 &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_cache[dev], reinterpret_cast<const void*>(kern),
                                                     NT, 0) != hipSuccess)
      return fail(ATK_ELAUNCH, "group_norm: occupancy query failed");
    const int64_t cap = (int64_t)per_cu_cache[dev] * device_cu_count();
    if (nblk > cap)
      return fail(ATK_UNSUPPORTED, "group_norm: %lld workgroups exceed the %lld that can be resident",
                  (long long)nblk, (long long)cap);
  }
  a.trace = g_gn_trace && nblk * 4 <= g_gn_trace_words ? g_gn_trace : nullptr;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(NT), 0, s, a);
  return check_launch("gn_resident_kernel");
}

template <typename T, int NT, int EPV>
int launch_resident(GnArgs a, int64_t ngroups, hipStream_t s) {
  return a.silu ? launch_resident_s<T, NT, EPV, true>(a, ngroups, s)
                : launch_resident_s<T, NT, EPV, false>(a, ngroups, s);
}

template <typename T, bool VECOK>
int launch_twopass(const GnArgs& a, int64_t nblk, hipStream_t s) {
  hipLaunchKernelGGL((gn_stats_kernel<T, VECOK>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
  const int rc = check_launch("gn_stats_kernel");
  if (rc) return rc;
  if (a.silu) hipLaunchKernelGGL((gn_apply_kernel<T, VECOK, true>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
  else hipLaunchKernelGGL((gn_apply_kernel<T, VECOK, false>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
  return check_launch("gn_apply_kernel");
}

template <typename T, int NT, int EPV>
int launch_split(GnArgs a, int64_t ngroups, hipStream_t s) {
  const int64_t nblk = ngroups * a.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm: grid too large");
  a.NP = a.NS;
  hipLaunchKernelGGL((gn_split_stats_kernel<T, NT, EPV>), dim3((unsigned)nblk), dim3(NT), 0, s, a);
  const int rc = check_launch("gn_split_stats_kernel");
  if (rc) return rc;
  if (a.silu) hipLaunchKernelGGL((gn_split_apply_kernel<T, NT, EPV, true>), dim3((unsigned)nblk), dim3(NT), 0, s, a);
  else hipLaunchKernelGGL((gn_split_apply_kernel<T, NT, EPV, false>), dim3((unsigned)nblk), dim3(NT), 0, s, a);
  return check_launch("gn_split_apply_kernel");
}

template <typename T>
int launch_gn(GnArgs a, int64_t ngroups, int variant, bool vec_ok, hipStream_t s) {
  const GnVariant& v = kGnVariants[variant];
  if (v.kind == GN_SPLIT) {
    if (!vec_ok) return fail(ATK_UNSUPPORTED, "group_norm: %s needs S %% 16B == 0 and aligned pointers", v.name);
    switch (variant) {
      case 12: return launch_split<T, 256, 8>(a, ngroups, s);
      case 13: return launch_split<T, 512, 8>(a, ngroups, s);
      case 14: return launch_split<T, 256, 4>(a, ngroups, s);
      case 15: return launch_split<T, 1024, 4>(a, ngroups, s);
      default: return fail(ATK_EINVAL, "group_norm: bad variant");
    }
  }
  if (v.kind == GN_RESIDENT) {
    if (!vec_ok) return fail(ATK_UNSUPPORTED, "group_norm: %s needs S %% 16B == 0 and aligned pointers", v.name);
    switch (variant) {
      case 0: return launch_resident<T, 1024, 8>(a, ngroups, s);
      case 1: return launch_resident<T, 1024, 16>(a, ngroups, s);
      case 2: return launch_resident<T, 1024, 4>(a, ngroups, s);
      case 3: return launch_resident<T, 512, 8>(a, ngroups, s);
      case 4: return launch_resident<T, 256, 8>(a, ngroups, s);
      case 5: return launch_resident<T, 256, 16>(a, ngroups, s);
      case 7: return launch_resident<T, 256, 4>(a, ngroups, s);
      case 8: return launch_resident<T, 512, 4>(a, ngroups, s);
      case 9: return launch_resident<T, 512, 16>(a, ngroups, s);
      case 10: return launch_resident<T, 512, 32>(a, ngroups, s);
      case 11: return launch_resident<T, 256, 32>(a, ngroups, s);
      default: return fail(ATK_EINVAL, "group_norm: bad variant");
    }
  }
  const int64_t nblk = ngroups * a.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm: grid too large");
  return vec_ok ? launch_twopass<T, true>(a, nblk, s) : launch_twopass<T, false>(a, nblk, s);
}

int validate_gn(int64_t N, int64_t C, int64_t S, int G, int dtype, int variant) {
  if (!dtype_ok(dtype)) return fail(ATK_EINVAL, "group_norm: unknown dtype code %d", dtype);
  if (N < 0 || C <= 0 || S < 1 || G <= 0) return fail(ATK_EINVAL, "group_norm: bad sizes");
  if (C % G != 0) return fail(ATK_EINVAL, "group_norm: channels (%lld) must be divisible by groups (%d)", (long long)C, G);
  if (variant < 0 || variant >= kNumGn) return fail(ATK_EINVAL, "group_norm: variant %d out of range", variant);
  const int64_t E = (C / G) * S;
  if (E >= (1ll << 31) - 65536) return fail(ATK_UNSUPPORTED, "group_norm: group of %lld elements too large", (long long)E);
  return ATK_OK;
}

// ---------------------------------------------------------------------------------------
// Backward (reference: textbook torch ops, amd_tuned_torch/_dispatch.py:2212-2302):
//   g = gamma_c * dy,  x_hat = (x - mu) * rstd,
//   dx = rstd * (g - mean_group(g) - x_hat * mean_group(g * x_hat)),
//   dgamma_c = sum_{n,s} dy * x_hat,  dbeta_c = sum_{n,s} dy.
// Two kernels, 5 tensor-passes of HBM traffic (x and dy read twice, dx written once):
//   rows:     one workgroup per (n, c) row: x's mean / M2 about a row-wide shift K (the
//             row's first element), A = sum dy, B = sum dy * (x - K);
//   apply:    one workgroup per row: one wave merges the group's rows (Chan, fixed order, so
//             every row of a group derives the same statistics), then dx.  The workgroups
//             of n = 0 then also sum channel c's parameter gradients over n in a fixed
//             order, from the rows alone: dgamma_c = sum_n rstd_n * (B + (K - mu_n) * A),
//             dbeta_c = sum_n A.  They are dispatched first, so this tail hides behind
//             the later rows' work (a separate kernel cost a launch gap).
// Requires S % VEC == 0 and 16-byte aligned x / dy / dx (host check).
struct GnBwdArgs {
  const void* x;
  const void* dy;
  const void* gamma;
  void* dx;           // may be null (parameter gradients only)
  float* rows;        // [N*C][5]: mean, M2, A, B, K
  float* dgamma;      // [C] or null
  float* dbeta;       // [C] or null
  int64_t S;
  uint32_t C, cpg;
  int N;
  float eps;
  int pdt;
};

template <typename T, int U>
__global__ __launch_bounds__(GN_TP_NT) void gn_bwd_rows_kernel(GnBwdArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float red[4 * (GN_TP_NT / 64)];
  const int64_t r = blockIdx.x;
  const T* __restrict__ xr = static_cast<const T*>(a.x) + r * a.S;
  const T* __restrict__ gr = static_cast<const T*>(a.dy) + r * a.S;
  const float K = to_f32(xr[0]);
  float s1 = 0.f, s2 = 0.f, sa = 0.f, sb = 0.f;
  // U vectors of x and of dy in flight per thread (branch-free buffer loads; vectors
  // past the row read zero and are masked out of the sums)
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xr, (uint32_t)(a.S * (int64_t)sizeof(T)));
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(gr, (uint32_t)(a.S * (int64_t)sizeof(T)));
  for (int64_t e0 = (int64_t)threadIdx.x * VEC; e0 < a.S; e0 += (int64_t)GN_TP_NT * VEC * U) {
    Vec16<T> xv[U], gv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = e0 + (int64_t)u * GN_TP_NT * VEC;
      const uint32_t off = e < a.S ? (uint32_t)(e * (int64_t)sizeof(T)) : kOOB;
      xv[u].raw = bload16(rx, off, 0);  // cached: the apply kernel reads x and dy again
      gv[u].raw = bload16(rg, off, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float m = (e0 + (int64_t)u * GN_TP_NT * VEC < a.S) ? 1.f : 0.f;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float d = (to_f32(xv[u].e[k]) - K) * m;
        const float g = to_f32(gv[u].e[k]);
        s1 += d;
        s2 = fmaf(d, d, s2);
        sa += g;
        sb = fmaf(g, d, sb);
      }
    }
  }
  // only thread 0 needs the totals: the four wave sums go through LDS in one exchange
  // (four block_sum calls would cost eight barriers in a workgroup this short-lived)
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
  sa = wave_sum(sa);
  sb = wave_sum(sb);
  if ((threadIdx.x & 63) == 0) {
    const int w = threadIdx.x >> 6;
    red[w] = s1;
    red[GN_TP_NT / 64 + w] = s2;
    red[2 * (GN_TP_NT / 64) + w] = sa;
    red[3 * (GN_TP_NT / 64) + w] = sb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    s1 = s2 = sa = sb = 0.f;
#pragma unroll
    for (int w = 0; w < GN_TP_NT / 64; ++w) {  // the order block_sum uses
      s1 += red[w];
      s2 += red[GN_TP_NT / 64 + w];
      sa += red[2 * (GN_TP_NT / 64) + w];
      sb += red[3 * (GN_TP_NT / 64) + w];
    }
    const float q = s1 / (float)a.S;
    float* o = a.rows + r * 5;
    o[0] = K + q;
    o[1] = fmaxf(fmaf(-s1, q, s2), 0.f);
    o[2] = sa;
    o[3] = sb;
    o[4] = K;
  }
}

// mean and rstd of group (rows rg[0 .. cpg)) from its rows' (mean, M2): call with all 64
// lanes of a wave; every lane gets the same values (fixed-order butterfly sums)
__device__ __forceinline__ void gn_bwd_group_stats(const GnBwdArgs& a, const float* rg, int lane, float& mu,
                                                   float& rstd) {
  float sm = 0.f;
  for (uint32_t j = lane; j < a.cpg; j += 64) sm += rg[j * 5];
  mu = wave_sum(sm) / (float)a.cpg;  // equal row sizes
  float m2 = 0.f;
  for (uint32_t j = lane; j < a.cpg; j += 64) {
    const float dm = rg[j * 5] - mu;
    m2 += rg[j * 5 + 1] + (float)a.S * dm * dm;
  }
  m2 = wave_sum(m2);
  rstd = 1.0f / sqrtf(m2 / (float)((int64_t)a.cpg * a.S) + a.eps);
}

template <typename T, int U>
__global__ __launch_bounds__(GN_TP_NT) void gn_bwd_apply_kernel(GnBwdArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float st[5];  // mu, rstd, c1, c2, gamma_c
  const int64_t r = blockIdx.x;
  const uint32_t c = (uint32_t)(r % a.C);
  const int64_t n = r / a.C;
  const uint32_t g0 = c - c % a.cpg;          // first channel of the group
  const int64_t r0 = n * a.C + g0;            // its row
  const float E = (float)((int64_t)a.cpg * a.S);
  const T* __restrict__ xr = static_cast<const T*>(a.x) + r * a.S;
  const T* __restrict__ gr = static_cast<const T*>(a.dy) + r * a.S;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xr, (uint32_t)(a.S * (int64_t)sizeof(T)));
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(gr, (uint32_t)(a.S * (int64_t)sizeof(T)));
  Vec16<T> xv[U], gv[U];
  auto issue = [&](int64_t e0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = e0 + (int64_t)u * GN_TP_NT * VEC;
      const uint32_t off = e < a.S ? (uint32_t)(e * (int64_t)sizeof(T)) : kOOB;
      xv[u].raw = bload16<2>(rx, off, 0);  // last reads of x and dy
      gv[u].raw = bload16<2>(rg, off, 0);
    }
  };
  // the first batch of x and dy does not depend on the statistics: its loads are issued
  // before the group merge below, so their latency overlaps it (a C3-sized row is one batch)
  const int64_t e_first = (int64_t)threadIdx.x * VEC;
  issue(e_first);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const float* rows = a.rows + r0 * 5;
    float mu, rstd;
    gn_bwd_group_stats(a, rows, lane, mu, rstd);
    float sg = 0.f, sgx = 0.f;
    for (uint32_t j = lane; j < a.cpg; j += 64) {
      const float* o = rows + j * 5;
      const float gam = a.gamma ? load_param(a.gamma, a.pdt, g0 + j) : 1.f;
      sg = fmaf(gam, o[2], sg);
      sgx = fmaf(gam, o[3] + (o[4] - mu) * o[2], sgx);
    }
    sg = wave_sum(sg);
    sgx = wave_sum(sgx);
    if (lane == 0) {
      st[0] = mu;
      st[1] = rstd;
      st[2] = sg / E;
      st[3] = rstd * sgx / E;
      st[4] = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
    }
  }
  __syncthreads();
  if (a.dx) {
    const float mu = st[0], rstd = st[1], c1 = st[2], c2 = st[3], gam = st[4];
    T* __restrict__ dxr = static_cast<T*>(a.dx) + r * a.S;
    for (int64_t e0 = e_first; e0 < a.S; e0 += (int64_t)GN_TP_NT * VEC * U) {
      if (e0 != e_first) issue(e0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t e = e0 + (int64_t)u * GN_TP_NT * VEC;
        float o[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float xh = (to_f32(xv[u].e[k]) - mu) * rstd;
          o[k] = rstd * (fmaf(gam, to_f32(gv[u].e[k]), -c1) - xh * c2);
        }
        if (e < a.S) st16<true>(dxr + e, pack16<T>(o));
      }
    }
  }
  if (n != 0 || (!a.dgamma && !a.dbeta)) return;
  // parameter gradients of channel c: wave w takes samples w, w + 4, ... in order; the four
  // wave totals are added in wave order (deterministic)
  __shared__ float fin[2 * (GN_TP_NT / 64)];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float sgm = 0.f, sbt = 0.f;
  for (int m = w; m < a.N; m += GN_TP_NT / 64) {
    float mu, rstd;
    gn_bwd_group_stats(a, a.rows + ((int64_t)m * a.C + g0) * 5, lane, mu, rstd);
    const float* o = a.rows + ((int64_t)m * a.C + c) * 5;
    sgm += rstd * (o[3] + (o[4] - mu) * o[2]);
    sbt += o[2];
  }
  if (lane == 0) {
    fin[w] = sgm;
    fin[GN_TP_NT / 64 + w] = sbt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    sgm = sbt = 0.f;
#pragma unroll
    for (int v = 0; v < GN_TP_NT / 64; ++v) {
      sgm += fin[v];
      sbt += fin[GN_TP_NT / 64 + v];
    }
    if (a.dgamma) a.dgamma[c] = sgm;
    if (a.dbeta) a.dbeta[c] = sbt;
  }
}

template <typename T, int U>
void launch_gn_bwd_u(const GnBwdArgs& a, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL((gn_bwd_rows_kernel<T, U>), dim3((unsigned)rows), dim3(GN_TP_NT), 0, s, a);
  hipLaunchKernelGGL((gn_bwd_apply_kernel<T, U>), dim3((unsigned)rows), dim3(GN_TP_NT), 0, s, a);
}

// ---------------------------------------------------------------------------------------
// Register-resident backward: one workgroup per group (n, g) holds the group's x and dy in
// registers (up to NT * EPV 16-byte vectors of each), so x and dy are read once and dx
// written once -- 3 tensor passes instead of the rows / apply pair's 5.  In one pass over
// the registers after the statistics (mu, rstd of x, as the forward computes them):
//   A = sum gamma_c dy,  B = sum gamma_c dy (x - mu)   -> c1 = A / E,  c2 = B rstd / E,
//   dx = rstd (gamma_c dy - c1 - (x - mu) rstd c2).
// Parameter gradients: each wave's segment of 64 vectors lies in one channel (host check:
// S a multiple of 64 vectors), so per-channel sums of dy (x - mu) rstd and dy are wave sums,
// added per channel in (vector, wave) order into a row per (n, c), stored with agent-scope
// atomic stores by wave 0, which then counts the workgroup in on a per-group counter while
// the other waves write dx.  The last of the group's N workgroups adds the N rows of its
// channels in n order (deterministic) and resets the counter: no workgroup waits for
// another, and every launch leaves the counters zero (HIP-graph replay safe).  A second
// kernel for the sums over n cost more (a dependent launch's gap).
constexpr int GN_BWD_MAXG = 4096;                        // groups per launch (counters)
constexpr size_t GN_BWD_CNT_BYTES = 4 * (size_t)GN_BWD_MAXG;
constexpr int GN_BWD_RES_NT = 1024;

struct GnBwdResArgs {
  const void* x;
  const void* dy;
  const void* gamma;
  void* dx;            // may be null
  float* dgamma;       // [C] or null
  float* dbeta;        // [C] or null
  uint32_t* counter;   // [G], zero on entry and on exit
  float* part;         // [N][C][2]: sum dy (x - mu) rstd, sum dy of (n, c)
  int64_t E;           // cpg * S
  uint32_t S, cpg, C, G;
  int N;
  float eps;
  int pdt;
  FastDiv div_s;
};

template <typename T, int NT, int EPV>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4)))
void gn_bwd_resident_kernel(GnBwdResArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NW = NT / 64;
  __shared__ float red[NW];
  __shared__ float s_gam[GN_MAX_AFF];
  __shared__ float2 s_part[EPV][NW];
  __shared__ float2 s_rows[NT];
  __shared__ uint32_t s_prev;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t gi = blockIdx.x;
  const int n = (int)(gi / a.G), g = (int)(gi - (int64_t)n * a.G);
  const int cpg = (int)a.cpg;
  const int64_t E = a.E;
  const int64_t c0 = (int64_t)g * cpg;  // the group's first channel

  // gamma word first (loads complete in issue order: issued after x / dy it would wait for them)
  uint32_t gsel;
  const uint32_t gword = param_word(a.gamma, a.pdt, c0 + (tid < cpg ? tid : 0), (int64_t)a.C, gsel);
  const uint32_t bytes = (uint32_t)(E * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + gi * E, bytes);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(static_cast<const T*>(a.dy) + gi * E, bytes);
  const uint32_t lane_off = (uint32_t)tid * 16u;
  const uint32_t n_vec = (uint32_t)(E / VEC);
  auto voff = [&](int i) { return (uint32_t)(i * NT + tid) < n_vec ? lane_off : kOOB; };
  auto soff = [&](int i) { return (uint32_t)i * NT * 16u; };
  Vec16<T> xb[EPV], db[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) xb[i].raw = bload16<2>(rx, voff(i), soff(i));
#pragma unroll
  for (int i = 0; i < EPV; ++i) db[i].raw = bload16<2>(rd, voff(i), soff(i));
  if (tid < cpg) s_gam[tid] = a.gamma ? param_decode(gword, gsel, a.pdt) : 1.f;

  // statistics of x, bit-identical to the forward's single-slice arithmetic (the barriers
  // inside also publish s_gam)
  float mean, m2;
  slice_stats<T, NT, EPV, true>(xb, nullptr, 0, E, E, red, mean, m2);
  const float rstd = 1.0f / sqrtf(m2 / (float)E + a.eps);

  // per thread: A, B and, per vector, sum dy (x - mu) and sum dy.  Each vector pair is
  // fenced together with the running sums, so it is unpacked only after the previous one is
  // accumulated (left free, the compiler unpacks every vector up front and spills).
  float A = 0.f, B = 0.f;
  const bool params = a.dgamma || a.dbeta;
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    asm volatile("" : "+v"(xb[i].raw.x), "+v"(xb[i].raw.y), "+v"(xb[i].raw.z), "+v"(xb[i].raw.w),
                 "+v"(db[i].raw.x), "+v"(db[i].raw.y), "+v"(db[i].raw.z), "+v"(db[i].raw.w), "+v"(A), "+v"(B));
    const bool ok = (uint32_t)(i * NT + tid) < n_vec;
    const uint32_t e = ok ? (uint32_t)((i * NT + tid) * VEC) : 0u;
    const float gm = s_gam[fdiv(e, a.div_s)];
    float sg = 0.f, sb = 0.f;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = to_f32(db[i].e[k]);
      const float xc = to_f32(xb[i].e[k]) - mean;
      sb += d;
      sg = fmaf(d, xc, sg);
    }
    // out-of-range vectors read zeros: d = 0 adds nothing
    A = fmaf(gm, sb, A);
    B = fmaf(gm, sg, B);
    if (params) {  // the wave's segment sums, right away (nothing stays live for later)
      const float wg = wave_sum(sg), wb = wave_sum(sb);
      if (lane == 0) s_part[i][wv] = make_float2(wg, wb);
    }
  }
  reg_fence<T, EPV>(xb);
  reg_fence<T, EPV>(db);
  const float c1 = block_sum<NT>(A, red) / (float)E;
  const float c2 = block_sum<NT>(B, red) * rstd / (float)E;

  uint32_t prev = 0;  // thread 0: the group counter before this workgroup's count
  if (params && wv == 0) {
    // Wave 0 alone (lane l for channels l, l + 64, ...) writes the rows and counts the
    // workgroup in, so the wait for the row stores is the wave's own and the other waves go
    // on to write dx meanwhile.  s_part is complete: the block sums above contain barriers.
    // Segment q = i * NW + w covers elements [q, q + 1) * 64 * VEC, so channel c owns
    // segments [c, c + 1) * spc.
    const int spc = (int)(a.S / (64 * VEC));
    const float2* seg = &s_part[0][0];
    for (int c = lane; c < cpg; c += 64) {
      float sg = 0.f, sb = 0.f;
      for (int q = c * spc; q < (c + 1) * spc; ++q) {  // in order
        sg += seg[q].x;
        sb += seg[q].y;
      }
      uint32_t* row = reinterpret_cast<uint32_t*>(a.part + ((int64_t)n * a.C + c0 + c) * 2);
      __hip_atomic_store(row, __float_as_uint(sg * rstd), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(row + 1, __float_as_uint(sb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the wave's rows are complete before it counts the workgroup done (issued before this
    // wave's dx stores, so this waits for the row stores only)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid == 0) prev = __hip_atomic_fetch_add(a.counter + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (a.dx) {
    T* __restrict__ dxg = static_cast<T*>(a.dx) + gi * E;
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      // vector i is unpacked only after store i-1 has issued
      reg_fence<T, 1>(&xb[i]);
      reg_fence<T, 1>(&db[i]);
      const bool ok = (uint32_t)(i * NT + tid) < n_vec;
      const uint32_t e = ok ? (uint32_t)((i * NT + tid) * VEC) : 0u;
      const float gm = s_gam[fdiv(e, a.div_s)];
      float v[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float xh = (to_f32(xb[i].e[k]) - mean) * rstd;
        v[k] = rstd * (gm * to_f32(db[i].e[k]) - c1 - xh * c2);
      }
      if (ok) st16<true>(dxg + e, pack16<T>(v));
    }
  }

  if (params) {
    if (tid == 0) s_prev = prev;
    __syncthreads();
    if (s_prev == (uint32_t)a.N - 1) {
      // last of the group's N workgroups: every row of the group is written.  The N x cpg
      // rows are fetched NT at a time, one per thread with all loads in flight, staged in
      // LDS and added per channel in n order.
      const int per = NT / cpg;  // samples per round (cpg <= NT)
      float sg = 0.f, sb = 0.f;
      for (int m0 = 0; m0 < a.N; m0 += per) {
        const int m = m0 + tid / cpg, c = tid - (tid / cpg) * cpg;
        if (tid < per * cpg && m < a.N) {
          const uint32_t* row = reinterpret_cast<const uint32_t*>(a.part + ((int64_t)m * a.C + c0 + c) * 2);
          s_rows[tid] = make_float2(
              __uint_as_float(__hip_atomic_load(row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
              __uint_as_float(__hip_atomic_load(row + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
        }
        __syncthreads();
        if (tid < cpg) {
          const int mn = min(per, a.N - m0);
          for (int k = 0; k < mn; ++k) {
            sg += s_rows[k * cpg + tid].x;
            sb += s_rows[k * cpg + tid].y;
          }
        }
        __syncthreads();
      }
      if (tid < cpg) {
        if (a.dgamma) a.dgamma[c0 + tid] = sg;
        if (a.dbeta) a.dbeta[c0 + tid] = sb;
      }
      if (tid == 0) __hip_atomic_store(a.counter + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// vectors per thread the resident backward needs for (cpg, S), or 0 when it does not apply
inline int gn_bwd_resident_epv(int64_t N, int64_t C, int64_t S, int G, int dtype) {
  const int64_t vec = 16 / (int64_t)dtype_size(dtype);
  const int64_t cpg = C / G, E = cpg * S;
  if (S % (64 * vec) || cpg > GN_MAX_AFF || G > GN_BWD_MAXG || N * G >= (1ll << 31) || N * C >= (1ll << 30))
    return 0;
  const int64_t per = (int64_t)GN_BWD_RES_NT * vec;
  if (E > 8 * per) return 0;
  return E <= 2 * per ? 2 : E <= 4 * per ? 4 : 8;
}

template <typename T>
int launch_gn_bwd_resident(const GnBwdResArgs& a, int epv, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)a.N * a.G)), block(GN_BWD_RES_NT);
  if (epv == 2) hipLaunchKernelGGL((gn_bwd_resident_kernel<T, GN_BWD_RES_NT, 2>), grid, block, 0, s, a);
  else if (epv == 4) hipLaunchKernelGGL((gn_bwd_resident_kernel<T, GN_BWD_RES_NT, 4>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((gn_bwd_resident_kernel<T, GN_BWD_RES_NT, 8>), grid, block, 0, s, a);
  return check_launch("gn_bwd_resident_kernel");
}

template <typename T>
int launch_gn_bwd(const GnBwdArgs& a, int64_t rows, hipStream_t s) {
  // vectors per thread and batch: no more than a row holds (C3a's 4096-element rows are two
  // per thread; four would leave half the loads reading past the row)
  constexpr int VEC = 16 / sizeof(T);
  const int64_t vpt = (a.S + (int64_t)GN_TP_NT * VEC - 1) / ((int64_t)GN_TP_NT * VEC);
  if (vpt <= 1) launch_gn_bwd_u<T, 1>(a, rows, s);
  else if (vpt <= 2) launch_gn_bwd_u<T, 2>(a, rows, s);
  else launch_gn_bwd_u<T, GN_BWD_U>(a, rows, s);
  return check_launch("gn_bwd_rows_kernel / gn_bwd_apply_kernel");
}

// ---------------------------------------------------------------------------------------
// Channels-last GroupNorm forward (NHWC / NDHWC memory: x[n][s][c]).  The reference serves
// this layout with Composable Kernel's groupnorm (amd_tuned_torch/ck_norm_ops.py:9-27,
// 93-103); the arithmetic is the NC[S] kernel's: group (n, g) = channels [g*cpg, (g+1)*cpg)
// at every spatial position.  Two kernels, deterministic:
//   stats: a workgroup per (n, spatial chunk); thread t owns one 16-byte channel vector
//          (column t % CV, so one group: cpg % VEC == 0) on rows t / CV, t / CV + R, ... and
//          accumulates shifted sums; one thread per group then merges that group's
//          per-thread (n, mean, M2) with Chan's formula in a fixed order;
//   merge: one wave per (n, g) merges the group's chunk partials (the fixed-order butterfly
//          of the NC[S] kernels) into (mean, rstd);
//   apply: a workgroup per (n, chunk) stages per-channel scale / shift in LDS and
//          normalises its chunk (+ SiLU).
// Requires C / VEC to divide the workgroup size (C <= 2048 for 16-bit types), 16-byte
// aligned x / y and samples under 2 GiB (host check).  Traffic: x read twice (the second
// read mostly from the Infinity Cache), y written once.  Both streaming kernels keep
// GN_CL_U rows of loads in flight per thread.
constexpr int GN_CL_NT = 256;
constexpr int GN_CL_MAXC = 2048;
constexpr int GN_CL_MAXG = 256;
constexpr int GN_CL_U = 8;  // rows in flight per thread

struct GnClArgs {
  const void* x;
  const void* gamma;
  const void* beta;
  void* y;
  float* part;        // [N][NCH][G][2] (mean, M2) of each chunk's slice of each group
  float* stat;        // [N][G][2] (mean, rstd)
  int64_t S, SC;      // spatial positions, positions per chunk
  uint32_t sample_bytes;  // bytes of one sample (buffer-load range; host checks < 2 GiB)
  uint32_t C, G, cpg;
  int NCH;
  float eps;
  int pdt;
};

template <typename T>
__global__ __launch_bounds__(GN_CL_NT) void gn_cl_stats_kernel(GnClArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float sm[GN_CL_NT], sq[GN_CL_NT], sn[GN_CL_NT];
  const int n = blockIdx.y, ch = blockIdx.x;
  const int CV = (int)(a.C / VEC), R = GN_CL_NT / CV;
  const int v = threadIdx.x % CV, rr = threadIdx.x / CV;
  const int64_t s0 = (int64_t)ch * a.SC, s1 = min(a.S, s0 + a.SC);
  const T* __restrict__ xn = static_cast<const T*>(a.x) + (int64_t)n * a.S * a.C + v * VEC;
  // GN_CL_U rows per batch as branch-free buffer loads (rows past the chunk read zero and are
  // masked out of the sums), so a thread has GN_CL_U loads in flight instead of one
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + (int64_t)n * a.S * a.C, a.sample_bytes);
  const uint32_t vb = (uint32_t)(v * VEC * sizeof(T)), rowb = (uint32_t)(a.C * sizeof(T));
  float K = 0.f, t1 = 0.f, t2 = 0.f, cnt = 0.f;
  if (s0 + rr < s1) K = to_f32(xn[(s0 + rr) * a.C]);
  for (int64_t s = s0 + rr; s < s1; s += (int64_t)R * GN_CL_U) {
    Vec16<T> xv[GN_CL_U];
#pragma unroll
    for (int u = 0; u < GN_CL_U; ++u) {
      const int64_t sp = s + (int64_t)u * R;
      xv[u].raw = bload16(rx, sp < s1 ? (uint32_t)sp * rowb + vb : kOOB, 0);  // cached: x is read again
    }
#pragma unroll
    for (int u = 0; u < GN_CL_U; ++u) {
      const float m = (s + (int64_t)u * R < s1) ? 1.f : 0.f;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float d = (to_f32(xv[u].e[k]) - K) * m;
        t1 += d;
        t2 = fmaf(d, d, t2);
      }
      cnt += m * (float)VEC;
    }
  }
  float mean_t = 0.f, m2_t = 0.f;
  if (cnt > 0.f) {
    const float q = t1 / cnt;
    mean_t = K + q;
    m2_t = fmaxf(fmaf(-t1, q, t2), 0.f);
  }
  sm[threadIdx.x] = mean_t;
  sq[threadIdx.x] = m2_t;
  sn[threadIdx.x] = cnt;
  __syncthreads();
  const int cpv = (int)(a.cpg / VEC);  // vectors per group
  for (int g = threadIdx.x; g < (int)a.G; g += GN_CL_NT) {
    // entries of group g: rows rr' in [0, R), columns [g*cpv, (g+1)*cpv)
    float nt = 0.f, mt = 0.f;
    for (int r2 = 0; r2 < R; ++r2)
      for (int c2 = 0; c2 < cpv; ++c2) {
        const int e = r2 * CV + g * cpv + c2;
        nt += sn[e];
        mt = fmaf(sn[e], sm[e], mt);
      }
    const float mean = nt > 0.f ? mt / nt : 0.f;
    float m2 = 0.f;
    for (int r2 = 0; r2 < R; ++r2)
      for (int c2 = 0; c2 < cpv; ++c2) {
        const int e = r2 * CV + g * cpv + c2;
        const float d = sm[e] - mean;
        m2 += sq[e] + sn[e] * d * d;
      }
    float* o = a.part + (((int64_t)n * a.NCH + ch) * a.G + g) * 2;
    o[0] = mean;
    o[1] = m2;
  }
}

// One workgroup per (n, g): thread t takes chunks t, t + NT, ... (up to GN_CL_MERGE_U each),
// all of whose (mean, M2) loads are issued before any is used -- walked one dependent load
// at a time, the merge of C3b's 1024 chunks took longer than the stats kernel -- and two
// fixed-order block sums give mean = sum n_i mean_i / E, M2 = sum (M2_i + n_i (mean_i - mean)^2).
constexpr int GN_CL_MERGE_NT = 256;
constexpr int GN_CL_MERGE_U = 16;  // chunks per thread: NCH <= 4096 (host check)
__global__ __launch_bounds__(GN_CL_MERGE_NT) void gn_cl_merge_kernel(GnClArgs a) {
  __shared__ float red[GN_CL_MERGE_NT / 64];
  const int64_t ng = blockIdx.x;  // n * G + g
  const int64_t n = ng / a.G, g = ng - n * a.G;
  const int tid = threadIdx.x;
  // the partials of sample n: [NCH][G][2] floats; chunks past NCH read zero
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.part + n * a.NCH * a.G * 2, (uint32_t)a.NCH * a.G * 8u);
  float mv[GN_CL_MERGE_U], qv[GN_CL_MERGE_U];
#pragma unroll
  for (int u = 0; u < GN_CL_MERGE_U; ++u) {
    const int i = tid + u * GN_CL_MERGE_NT;
    const uint32_t off = i < a.NCH ? ((uint32_t)i * a.G + (uint32_t)g) * 8u : kOOB;
    mv[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, (int)off, 0, 0));
    qv[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, (int)(off + (i < a.NCH ? 4u : 0u)), 0, 0));
  }
  const int64_t slice = a.SC * a.cpg, E = a.S * a.cpg;
  float sm = 0.f;
#pragma unroll
  for (int u = 0; u < GN_CL_MERGE_U; ++u) {
    const int i = tid + u * GN_CL_MERGE_NT;
    const float len = i < a.NCH ? (float)slice_len(i, slice, E) : 0.f;
    sm = fmaf(len, mv[u], sm);
  }
  const float mean = block_sum<GN_CL_MERGE_NT>(sm, red) / (float)E;
  float m2 = 0.f;
#pragma unroll
  for (int u = 0; u < GN_CL_MERGE_U; ++u) {
    const int i = tid + u * GN_CL_MERGE_NT;
    const float len = i < a.NCH ? (float)slice_len(i, slice, E) : 0.f;
    const float d = mv[u] - mean;
    m2 += qv[u] + len * d * d;
  }
  const float var = block_sum<GN_CL_MERGE_NT>(m2, red) / (float)E;
  if (tid == 0) {
    a.stat[ng * 2] = mean;
    a.stat[ng * 2 + 1] = 1.0f / sqrtf(var + a.eps);
  }
}

template <typename T, bool SILU>
__global__ __launch_bounds__(GN_CL_NT) void gn_cl_apply_kernel(GnClArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float scs[GN_CL_MAXC], shs[GN_CL_MAXC];
  __shared__ float gmean[GN_CL_MAXG], grstd[GN_CL_MAXG];
  const int n = blockIdx.y, ch = blockIdx.x;
  const int CV = (int)(a.C / VEC), R = GN_CL_NT / CV;
  const int v = threadIdx.x % CV, rr = threadIdx.x / CV;
  const int64_t s0 = (int64_t)ch * a.SC, s1 = min(a.S, s0 + a.SC);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + (int64_t)n * a.S * a.C, a.sample_bytes);
  const uint32_t vb = (uint32_t)(v * VEC * sizeof(T)), rowb = (uint32_t)(a.C * sizeof(T));
  Vec16<T> xv[GN_CL_U];
  auto issue = [&](int64_t s) {
#pragma unroll
    for (int u = 0; u < GN_CL_U; ++u) {
      const int64_t sp = s + (int64_t)u * R;
      xv[u].raw = bload16<2>(rx, sp < s1 ? (uint32_t)sp * rowb + vb : kOOB, 0);  // last read of x
    }
  };
  // the first rows do not depend on the statistics: their loads overlap the prologue
  const int64_t s_first = s0 + rr;
  issue(s_first);
  for (int g = threadIdx.x; g < (int)a.G; g += GN_CL_NT) {
    gmean[g] = a.stat[((int64_t)n * a.G + g) * 2];
    grstd[g] = a.stat[((int64_t)n * a.G + g) * 2 + 1];
  }
  __syncthreads();
  for (uint32_t c = threadIdx.x; c < a.C; c += GN_CL_NT) {
    const uint32_t g = c / a.cpg;
    const float gm = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
    const float bt = a.beta ? load_param(a.beta, a.pdt, c) : 0.f;
    const float sc = grstd[g] * gm;
    scs[c] = sc;
    shs[c] = bt - gmean[g] * sc;
  }
  __syncthreads();
  T* __restrict__ yn = static_cast<T*>(a.y) + (int64_t)n * a.S * a.C + v * VEC;
  float sc[VEC], sh[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    sc[k] = scs[v * VEC + k];
    sh[k] = shs[v * VEC + k];
  }
  for (int64_t s = s_first; s < s1; s += (int64_t)R * GN_CL_U) {
    if (s != s_first) issue(s);
#pragma unroll
    for (int u = 0; u < GN_CL_U; ++u) {
      const int64_t sp = s + (int64_t)u * R;
      float o[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        o[k] = fmaf(to_f32(xv[u].e[k]), sc[k], sh[k]);
        if constexpr (SILU) o[k] = silu_f32(o[k]);
      }
      if (sp < s1) st16<true>(yn + sp * a.C, pack16<T>(o));
    }
  }
}

struct GnClPlan {
  int NCH;
  int64_t SC;
};

inline GnClPlan plan_gn_cl(int64_t N, int64_t S) {
  // about 2048 workgroups over the chip, at least 64 positions per chunk
  int64_t nch = (2048 + N - 1) / N;
  nch = std::max<int64_t>(1, std::min<int64_t>(nch, (S + 63) / 64));
  GnClPlan p;
  p.SC = (S + nch - 1) / nch;
  p.NCH = (int)((S + p.SC - 1) / p.SC);
  return p;
}

template <typename T>
int launch_gn_cl(const GnClArgs& a, int N, int silu, hipStream_t s) {
  const dim3 grid((unsigned)a.NCH, (unsigned)N), block(GN_CL_NT);
  hipLaunchKernelGGL((gn_cl_stats_kernel<T>), grid, block, 0, s, a);
  int rc = check_launch("gn_cl_stats_kernel");
  if (rc) return rc;
  if (a.NCH > GN_CL_MERGE_NT * GN_CL_MERGE_U) return fail(ATK_UNSUPPORTED, "group_norm (channels-last): too many chunks");
  hipLaunchKernelGGL(gn_cl_merge_kernel, dim3((unsigned)(N * a.G)), dim3(GN_CL_MERGE_NT), 0, s, a);
  rc = check_launch("gn_cl_merge_kernel");
  if (rc) return rc;
  if (silu) hipLaunchKernelGGL((gn_cl_apply_kernel<T, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((gn_cl_apply_kernel<T, false>), grid, block, 0, s, a);
  return check_launch("gn_cl_apply_kernel");
}

// ---------------------------------------------------------------------------------------
// Channels-last GroupNorm forward, register-resident single pass (same semantics as the
// kernels above; one read and one write of the tensor, one launch).  A workgroup owns a
// chunk of SC consecutive positions of sample n, all C channels: NT threads x EPV 16-byte
// vectors, vector i of thread t being element (i * NT + t) * VEC of the chunk, i.e. column
// v = t % CV (channels v*VEC .. v*VEC+VEC-1, inside one group) at position i * R + t / CV
// (CV = C / VEC, R = NT / CV).  It loads its chunk once, computes every group's (mean, M2)
// over the chunk, publishes them in slots, obtains every group's statistics over the sample
// and normalises from its registers.  Two ways to obtain them:
//   direct     every workgroup merges all G x NCH chunk records of its sample (G x NCH small);
//   two-level  workgroup g < G of a sample merges group g's NCH records and publishes the
//              group's (mean, var) in a second slot; every workgroup then reads the G results.
// Slots are tagged with an epoch held in the workspace header.  Every workgroup reads it at
// its start; the last workgroup of the launch to finish reading slots (counted per block of
// 64 workgroups, then per block) advances it and resets the counters.  A slot written by any
// earlier launch -- including an earlier replay of the same HIP graph -- never carries the
// current tag, so no slot ever needs clearing.  Every wait is bounded by wall-clock time: a chunk record that
// has not appeared is computed by the waiting workgroup from x with the owner's arithmetic
// (bit-identical), so the result never depends on which workgroups are resident; the host
// only launches grids that fit at once, since stand-ins are slow.
// ---------------------------------------------------------------------------------------
constexpr int GN_CLR_MAXNCH = 1024;              // chunks per sample
constexpr int GN_CLR_DIRECT = 1024;              // records merged by every workgroup (direct)
constexpr int64_t GN_CLR_MAX_SLOTS = 65536;      // N x G x NCH chunk records
constexpr int64_t GN_CLR_MAX_FINALS = 16384;     // N x G group results (two-level)
// workspace: diagnostics word [0], epoch [64], launch counter [128], block counters (one
// per 64 workgroups, 128 bytes apart) from [256]; slots; group results
constexpr int GN_CLR_BLOCK = 64;                 // workgroups per block counter
constexpr int GN_CLR_MAXBLK = 64;                // block counters: at most 4096 workgroups
constexpr size_t GN_CLR_SLOTS_OFF = 256 + 128 * (size_t)GN_CLR_MAXBLK;
constexpr size_t GN_CLR_FINALS_OFF = GN_CLR_SLOTS_OFF + 16 * (size_t)GN_CLR_MAX_SLOTS;
constexpr size_t GN_CLR_BYTES = GN_CLR_FINALS_OFF + 16 * (size_t)GN_CLR_MAX_FINALS;

struct GnClResArgs {
  const void* x;
  const void* gamma;
  const void* beta;
  void* y;
  uint32_t* hdr;        // workspace header (zero at allocation)
  GnSlot* slots;        // [N][G][NCH]
  GnSlot* finals;       // [N][G]
  int64_t S;            // positions per sample
  int SC, NCH;          // positions per chunk (EPV * R), chunks per sample
  int C, G, cpg;
  int CW, NB, GW;       // 16-byte columns per workgroup, channel blocks (C / VEC / CW), groups per block
  int two_level;
  int pdt;
  float eps;
  uint64_t wait_ticks;  // longest a workgroup waits, in total, for other workgroups' slots
  uint64_t* trace;      // diagnostics: [workgroup][4] wall-clock stamps, or null
};

__device__ __forceinline__ void gn_stamp(const GnClResArgs& a, int k) {
  if (a.trace && threadIdx.x == 0) a.trace[(int64_t)blockIdx.x * 4 + k] = wall_clock64();
}

__device__ __forceinline__ int cl_chunk_positions(const GnClResArgs& a, int c) {
  const int64_t left = a.S - (int64_t)c * a.SC;
  return left < a.SC ? (int)left : a.SC;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t cl_chunk_rsrc(const GnClResArgs& a, int n, int c, int es) {
  const char* base = static_cast<const char*>(a.x) + (((int64_t)n * a.S + (int64_t)c * a.SC) * a.C) * es;
  return make_rsrc(base, (uint32_t)((int64_t)cl_chunk_positions(a, c) * a.C * es));
}

// Byte offset, inside its chunk, of this thread's first vector (row tid / CW, column tid % CW
// of channel block b); vector i lies i * R rows further (R = NT / CW).
__device__ __forceinline__ uint32_t cl_lane_off(const GnClResArgs& a, int tid, int b, int es) {
  const int row = tid / a.CW, col = tid - row * a.CW;
  return (uint32_t)(row * a.C * es + (b * a.CW + col) * 16);
}

// Sum of v over the M consecutive threads of this thread's segment (M a power of two, segments
// aligned to M): an xor butterfly inside the wave, then, for segments spanning several waves,
// the waves' totals in order.  Every thread of a segment gets the same bits.  M is uniform
// over the workgroup (the barriers are reached by every thread or by none).
template <int NT>
__device__ __forceinline__ float seg_sum(float v, int M, float* red) {
  const int lim = M < 64 ? M : 64;
  for (int off = lim >> 1; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if (M <= 64) return v;
  const int w = threadIdx.x >> 6, wpg = M >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < wpg; ++i) t += red[(w / wpg) * wpg + i];
  return t;
}

// Per-group (mean, M2) of chunk `ch` into rm[g], rq[g] (g < G).  Thread t accumulates shifted
// sums over its vectors (about K = its first element; vectors past the chunk read zero and
// are shifted by zero, so they add nothing), leaves (n_t, mean_t, M2_t) in LDS, and thread g
// merges group g's threads in a fixed order -- rows, then the group's columns:
//   mean = sum n_e mean_e / n,  M2 = sum (M2_e + n_e (mean_e - mean)^2).
// The owner runs it on its registers (FROM_REG), a workgroup standing in for a late owner
// on memory, with the same operations in the same order: the results are bit-identical.
// Ends with the records visible to the whole workgroup.
template <typename T, int NT, int EPV, bool FROM_REG>
__device__ __forceinline__ void cl_chunk_stats(Vec16<T>* buf, __amdgpu_buffer_rsrc_t rx, int P, int b,
                                               const GnClResArgs& a, float* en, float* em, float* eq, float* red,
                                               float* rm, float* rq) {
  constexpr int VEC = 16 / sizeof(T);
  const int tid = threadIdx.x;
  const int CW = a.CW, R = NT / CW;
  const int row = tid / CW;
  auto get = [&](int i) -> Vec16<T> {
    if constexpr (FROM_REG) {
      return buf[i];
    } else {
      Vec16<T> v;
      v.raw = bload16(rx, cl_lane_off(a, tid, b, (int)sizeof(T)), (uint32_t)(i * R * a.C * (int)sizeof(T)));
      return v;
    }
  };
  const float K = to_f32(get(0).e[0]);
  float s1 = 0.f, s2 = 0.f;
  int nvt = 0;
  auto acc = [&](int i) {
    const bool ok = i * R + row < P;
    const float Ki = ok ? K : 0.f;
    if constexpr (FROM_REG)
      asm volatile("" : "+v"(buf[i].raw.x), "+v"(buf[i].raw.y), "+v"(buf[i].raw.z), "+v"(buf[i].raw.w),
                   "+v"(s1), "+v"(s2));
    const Vec16<T> v = get(i);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = to_f32(v.e[k]) - Ki;
      s1 += d;
      s2 = fmaf(d, d, s2);
    }
    nvt += ok ? 1 : 0;
  };
  if constexpr (FROM_REG) {
#pragma unroll
    for (int i = 0; i < EPV; ++i) acc(i);
  } else {
#pragma unroll 1
    for (int i = 0; i < EPV; ++i) acc(i);
  }
  const float nt = (float)(nvt * VEC);
  float mean_t = 0.f, m2_t = 0.f;
  if (nvt > 0) {
    const float q = s1 / nt;
    mean_t = K + q;
    m2_t = fmaxf(fmaf(-s1, q, s2), 0.f);
  }
  en[tid] = nt;
  em[tid] = mean_t;
  eq[tid] = m2_t;
  __syncthreads();
  // Thread t takes entry j = t % M of the workgroup's group g = t / M (M = NT / GW: GW groups
  // of cpv columns tile the CW columns, a power of two dividing NT), entry j being row j / cpv,
  // column g * cpv + j % cpv.
  const int cpv = a.cpg / VEC, M = NT / a.GW;
  const int g = tid / M, j = tid - (tid / M) * M;
  const int e = (j / cpv) * CW + g * cpv + (j - (j / cpv) * cpv);
  const float ne = en[e], me = em[e], qe = eq[e];
  const float n = seg_sum<NT>(ne, M, red);
  const float mean = seg_sum<NT>(ne * me, M, red) / n;
  const float d = me - mean;
  const float m2 = seg_sum<NT>(fmaf(ne * d, d, qe), M, red);
  if (j == 0) {
    rm[g] = mean;
    rq[g] = m2;
  }
  __syncthreads();
}

// (mean, var) of a group from its NCH chunk records tm[c], tq[c] (chunk c holding
// positions(c) * cpg elements), on one wave: lanes over chunks, then the xor butterfly, so
// every lane -- and every workgroup merging the same records -- gets the same bits.
__device__ __forceinline__ void cl_merge_group(const GnClResArgs& a, const float* tm, const float* tq, float& mean,
                                               float& var) {
  const int lane = threadIdx.x & 63;
  const float E = (float)(a.S * a.cpg);
  float sm = 0.f;
  for (int c = lane; c < a.NCH; c += 64) sm = fmaf((float)(cl_chunk_positions(a, c) * a.cpg), tm[c], sm);
  mean = wave_sum(sm) / E;
  float m2 = 0.f;
  for (int c = lane; c < a.NCH; c += 64) {
    const float d = tm[c] - mean;
    m2 += tq[c];
    m2 = fmaf((float)(cl_chunk_positions(a, c) * a.cpg) * d, d, m2);
  }
  var = wave_sum(m2) / E;
}

// Reads slot w (two tagged words) once; true with the values if both carry `tag`.
__device__ __forceinline__ bool read_slot(const GnSlot* sl, uint32_t tag, float& m, float& q) {
  const unsigned long long w0 = __hip_atomic_load(&sl->w[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long w1 = __hip_atomic_load(&sl->w[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  m = __uint_as_float((uint32_t)w0);
  q = __uint_as_float((uint32_t)w1);
  return (uint32_t)(w0 >> 32) == tag && (uint32_t)(w1 >> 32) == tag;
}

__device__ __forceinline__ void write_slot(GnSlot* sl, uint32_t tag, float m, float q) {
  const unsigned long long hi = (unsigned long long)tag << 32;
  __hip_atomic_store(&sl->w[0], hi | __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&sl->w[1], hi | __float_as_uint(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup-wide: chunk records r < nrec into tm[r], tq[r], record r being group gr(r) of
// chunk cr(r); this workgroup's own chunk comes from rm / rq.  Thread t polls records
// t, t + NT, ... (up to RPT), all outstanding loads issued together, until they carry the
// tag or the workgroup's deadline passes; a chunk with a record still missing is then
// computed from x by the whole workgroup (cl_chunk_stats on memory) and its records filled in.
template <typename T, int NT, int EPV, int RPT, typename GR, typename CR>
__device__ __forceinline__ void cl_collect(const GnClResArgs& a, int n, int b, int ch, uint32_t tag, uint64_t deadline,
                                           int nrec,
                                           GR gr, CR cr, float* tm, float* tq, const float* rm, const float* rq,
                                           float* en, float* em, float* eq, float* red, float* xm, float* xq, int* s_flag,
                                           int* s_list, int* s_cnt) {
  const int tid = threadIdx.x;
  bool need[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int r = tid + k * NT;
    need[k] = false;
    if (r < nrec) {
      if (cr(r) == ch) {
        tm[r] = rm[gr(r) - b * a.GW];
        tq[r] = rq[gr(r) - b * a.GW];
      } else {
        need[k] = true;
      }
    }
  }
  for (;;) {
    float m[RPT], q[RPT];
    bool ok[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      ok[k] = false;
      if (need[k]) {
        const int r = tid + k * NT;
        ok[k] = read_slot(&a.slots[((int64_t)n * a.G + gr(r)) * a.NCH + cr(r)], tag, m[k], q[k]);
      }
    }
    bool left = false;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      if (need[k] && ok[k]) {
        tm[tid + k * NT] = m[k];
        tq[tid + k * NT] = q[k];
        need[k] = false;
      }
      left = left || need[k];
    }
    if (!left || wall_clock64() > deadline) break;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k)
    if (need[k]) {
      const int c = cr(tid + k * NT);
      if (atomicExch(&s_flag[c], 1) == 0) s_list[atomicAdd(s_cnt, 1)] = c;
    }
  __syncthreads();
  const int nmiss = *s_cnt;
  if (nmiss > 0) {
    if (tid == 0) __hip_atomic_store(a.hdr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int m = 0; m < nmiss; ++m) {
      const int c = s_list[m];
      cl_chunk_stats<T, NT, EPV, false>(nullptr, cl_chunk_rsrc(a, n, c, (int)sizeof(T)), cl_chunk_positions(a, c), b,
                                        a, en, em, eq, red, xm, xq);
      for (int r = tid; r < nrec; r += NT)
        if (cr(r) == c) {
          tm[r] = xm[gr(r) - b * a.GW];
          tq[r] = xq[gr(r) - b * a.GW];
        }
      // Publish every group's record of the stand-in chunk (the owner, when it runs, writes
      // the same bits: same loads, same order of operations): a later collect for another
      // group then finds them in the slots instead of reading the chunk from x again.
      for (int g = tid; g < a.GW; g += NT)
        write_slot(&a.slots[((int64_t)n * a.G + b * a.GW + g) * a.NCH + c], tag, xm[g], xq[g]);
      __threadfence();
      __syncthreads();
    }
    for (int m = tid; m < nmiss; m += NT) s_flag[s_list[m]] = 0;
    __syncthreads();
    if (tid == 0) *s_cnt = 0;
    __syncthreads();
  }
}

// WPE: waves per SIMD the build is sized for.  At 4 (two workgroups per CU, for grids up to
// twice the CU count) the 16-vector build fits 128 VGPRs only by spilling two dwords to scratch;
// grids of at most one workgroup per CU take the 2-wave build, which holds everything in
// registers (no scratch traffic).
template <typename T, int NT, int EPV, bool SILU, int WPE = 4>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WPE)))
void gn_cl_resident_kernel(GnClResArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NW = NT / 64;
  constexpr int RPT = GN_CLR_DIRECT / NT;  // records per thread (direct: G x NCH; one group: NCH)
  static_assert(GN_CLR_MAXNCH <= GN_CLR_DIRECT, "one group's records fit the record table");
  __shared__ float en[NT], em[NT], eq[NT];
  __shared__ float s_red[NT / 64];
  __shared__ float rm[GN_CL_MAXG], rq[GN_CL_MAXG];  // this chunk's records
  __shared__ float xm[GN_CL_MAXG], xq[GN_CL_MAXG];  // a stand-in chunk's records
  __shared__ float gm[GN_CL_MAXG], gv[GN_CL_MAXG];  // the sample's group statistics
  __shared__ float gam[GN_CL_MAXC], bet[GN_CL_MAXC];
  __shared__ float big[2 * GN_CL_MAXC];             // records tm / tq, then scale / shift
  static_assert(GN_CLR_DIRECT <= GN_CL_MAXC, "the record table fits the scale / shift arrays");
  __shared__ int s_flag[GN_CLR_MAXNCH], s_list[GN_CLR_MAXNCH];
  __shared__ int s_cnt, s_gcnt;
  __shared__ int s_glist[GN_CL_MAXG + 1];
  float* tm = big;
  float* tq = big + GN_CLR_DIRECT;

  const int tid = threadIdx.x;
  // workgroup -> (sample n, channel block b, chunk ch), chunks fastest
  const int per_n = a.NB * a.NCH;
  const int n = blockIdx.x / per_n, rem = blockIdx.x - (blockIdx.x / per_n) * per_n;
  const int b = rem / a.NCH, ch = rem - (rem / a.NCH) * a.NCH;
  const int CW = a.CW, R = NT / CW;
  const int CB = CW * VEC;  // channels of the block, the first being c0
  const int c0 = b * CB, g0 = b * a.GW;
  const int P = cl_chunk_positions(a, ch);
  gn_stamp(a, 0);

  // Every x load of the chunk first, branch-free; then the epoch and gamma / beta, with
  // unconditional buffer loads that nothing waits for until the chunk's statistics are done
  // (loads complete in issue order: waiting for a parameter load issued before x would hold
  // back every x load behind its round trip).
  const __amdgpu_buffer_rsrc_t rx = cl_chunk_rsrc(a, n, ch, (int)sizeof(T));
  const uint32_t lane_off = cl_lane_off(a, tid, b, (int)sizeof(T));
  const uint32_t row_step = (uint32_t)(R * a.C * (int)sizeof(T));  // bytes between a thread's vectors
  Vec16<T> buf[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) buf[i].raw = bload16<2>(rx, lane_off, (uint32_t)i * row_step);
  const uint32_t epoch = __hip_atomic_load(a.hdr + 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  constexpr int PPT = (GN_CL_MAXC + NT - 1) / NT;  // parameters per thread, at most
  uint32_t gword[PPT], bword[PPT], gsel[PPT], bsel[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    gword[k] = bword[k] = gsel[k] = bsel[k] = 0;
    if (k == 0 || CB > k * NT) {  // uniform
      const int c = tid + k * NT;
      const int64_t ci = c0 + (c < CB ? c : 0);
      gword[k] = param_word(a.gamma, a.pdt, ci, a.C, gsel[k]);
      bword[k] = param_word(a.beta, a.pdt, ci, a.C, bsel[k]);
    }
  }
  if (tid == 0) {
    s_cnt = 0;
    // the record sets this workgroup merges: all groups (-1, direct) or its own group
    // (two-level, workgroup g < G); groups whose published result does not appear in time
    // are appended later
    s_gcnt = a.two_level ? (ch < a.G ? 1 : 0) : 1;
    s_glist[0] = a.two_level ? ch : -1;
  }
  for (int c = tid; c < GN_CLR_MAXNCH; c += NT) s_flag[c] = 0;

  cl_chunk_stats<T, NT, EPV, true>(buf, rx, P, b, a, en, em, eq, s_red, rm, rq);
  reg_fence<T, EPV>(buf);
  gn_stamp(a, 1);
  // (gam / bet are read only after the exchange's barriers)
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int c = tid + k * NT;
    if (c < CB) {
      gam[c] = a.gamma ? param_decode(gword[k], gsel[k], a.pdt) : 1.f;
      bet[c] = a.beta ? param_decode(bword[k], bsel[k], a.pdt) : 0.f;
    }
  }
  const uint32_t tag = (epoch << 1) | 1u;
  for (int g = tid; g < a.GW; g += NT)
    write_slot(&a.slots[((int64_t)n * a.G + g0 + g) * a.NCH + ch], tag, rm[g], rq[g]);
  const uint64_t deadline = wall_clock64() + a.wait_ticks;

  GnSlot* fin = a.finals + (int64_t)n * a.G;
  const int NCH = a.NCH;
  bool polled = !a.two_level;
  for (int k = 0;;) {
    if (k < s_gcnt) {  // uniform: LDS read after a barrier
      const int gf = s_glist[k++];
      cl_collect<T, NT, EPV, RPT>(a, n, b, ch, tag, deadline, gf < 0 ? a.GW * NCH : NCH,
                                  [&](int r) { return gf < 0 ? g0 + r / NCH : gf; },
                                  [&](int r) { return gf < 0 ? r - (r / NCH) * NCH : r; }, tm, tq, rm, rq, en, em,
                                  eq, s_red, xm, xq, s_flag, s_list, &s_cnt);
      __syncthreads();
      const int w = tid >> 6;
      // direct: the block's GW groups (local indices); two-level (one block, g0 = 0): group gf
      for (int g = gf < 0 ? w : (w == 0 ? gf : a.GW); g < (gf < 0 ? a.GW : gf + 1); g += NW) {
        float mean, var;
        cl_merge_group(a, gf < 0 ? tm + g * NCH : tm, gf < 0 ? tq + g * NCH : tq, mean, var);
        if ((tid & 63) == 0) {
          gm[g] = mean;
          gv[g] = var;
          if (gf == ch && a.two_level) write_slot(&fin[gf], tag, mean, var);
        }
      }
      __syncthreads();
      continue;
    }
    if (polled) break;
    polled = true;
    // two-level: the other groups' results, one thread per group
    for (int g = tid; g < a.G; g += NT) {
      if (g == ch) continue;
      float m, q;
      bool ok;
      for (;;) {
        ok = read_slot(&fin[g], tag, m, q);
        if (ok || wall_clock64() > deadline) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (ok) {
        gm[g] = m;
        gv[g] = q;
      } else {
        s_glist[atomicAdd(&s_gcnt, 1)] = g;
      }
    }
    __syncthreads();
  }
  gn_stamp(a, 2);
  // per-channel scale / shift of the block (over the record table, no longer needed)
  float* scs = big;
  float* shs = big + GN_CL_MAXC;
  for (int c = tid; c < CB; c += NT) {
    const int g = c / a.cpg;
    const float rstd = 1.0f / sqrtf(gv[g] + a.eps);
    const float sc = rstd * gam[c];
    scs[c] = sc;
    shs[c] = bet[c] - gm[g] * sc;
  }
  __syncthreads();
  const int v = tid % CW;
  float sc[VEC], sh[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    sc[k] = scs[v * VEC + k];
    sh[k] = shs[v * VEC + k];
  }
  T* __restrict__ yc = static_cast<T*>(a.y) + ((int64_t)n * a.S + (int64_t)ch * a.SC) * a.C;
  // (indices from an opaque copy of tid: the statistics phase's per-vector offsets would
  // otherwise be kept for the stores, and at four waves per SIMD those are the values that spill)
  int tid_s = tid;
  asm volatile("" : "+v"(tid_s));
  const int row_s = tid_s / CW;
  const int lane_e = row_s * a.C + c0 + (tid_s - row_s * CW) * VEC;  // element offset of vector 0
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    reg_fence<T, 1>(&buf[i]);
    if (i * R + row_s < P) {
      float o[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        o[k] = fmaf(to_f32(buf[i].e[k]), sc[k], sh[k]);
        if constexpr (SILU) o[k] = silu_f32(o[k]);
      }
      st16<true>(yc + lane_e + (int64_t)i * R * a.C, pack16<T>(o));
    }
  }
  gn_stamp(a, 3);
  // Done with the slots (every read above has returned): count this workgroup in its block
  // of GN_CLR_BLOCK; the block's last counts the block in the launch, and the launch's last
  // advances the epoch.  Each counter is reset by the workgroup that completes it.  Counting
  // after the stores keeps the atomics' round trips off the store phase, and the blocks keep
  // all workgroups from queueing on one address.
  if (tid == 0) {
    const uint32_t b = blockIdx.x / GN_CLR_BLOCK, nb = (gridDim.x + GN_CLR_BLOCK - 1) / GN_CLR_BLOCK;
    const uint32_t in_b = min((uint32_t)GN_CLR_BLOCK, gridDim.x - b * GN_CLR_BLOCK);
    uint32_t* bc = a.hdr + 64 + 32 * b;
    if (__hip_atomic_fetch_add(bc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == in_b - 1) {
      __hip_atomic_store(bc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(a.hdr + 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nb - 1) {
        __hip_atomic_store(a.hdr + 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.hdr + 16, (epoch + 1u) & 0x7fffffffu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

struct GnClResPlan {
  int nt, epv, NCH, SC, two_level;
  int CW, NB;  // 16-byte columns per workgroup, channel blocks per sample
};

// The register-resident configuration for a channels-last shape, or false.  Left to itself
// the library takes 16 vectors per thread (128 KB chunks in 16-bit types) when that grid
// covers every CU and fits at once: the exchange of statistics costs about 5 us (two rounds
// of agent-coherent stores and polls), which a 128 KB chunk per workgroup amortises against
// the three-kernel path's second read of x and two extra launches, and 64 KB chunks do not.
// `force_epv` (8 or 16) takes that configuration wherever it fits.  Two-level whenever there
// are at least as many chunks as groups (measured faster than every workgroup polling all
// G x NCH records), else direct if G x NCH <= GN_CLR_DIRECT.
//
// Chunk shape.  `rows`: a chunk is SC whole positions (all C channels), and its records cover
// every group, so a sample's statistics need the records of all its chunks (two-level or
// direct).  `blocks`: a chunk is 8 columns (128 bytes of each position, whole groups) of
// EPV * NT / 8 positions, so a workgroup merges only its block's groups over the sample's
// chunks of that block -- one exchange round instead of two, over a few records.  Blocks are
// taken where the groups tile 8 columns, C spans more than 8 and the rows grid would need more
// than one workgroup per CU (measured, bf16, graph replay: C3b NDHWC 31.4 -> 27.6 us, +SiLU
// 32.0 -> 30.2 us; on C3a NHWC, one rows workgroup per CU, blocks lose 17.8 -> 18.0 us and
// +SiLU 17.8 -> 19.1 us: their 128-byte runs 1 KB apart load slower than whole 128 KB chunks,
// which eats the saved round).  `layout` 1 / 2 forces rows / blocks (blocks only where they
// apply).
template <typename T>
bool plan_gn_cl_res(int64_t N, int64_t C, int64_t S, int G, int force_epv, int layout, GnClResPlan& out);

// Workgroups of the resident kernel that fit the GPU at once: the smaller of its two builds
// (with and without SiLU), since either may be launched on the plan this capacity admits.
template <typename T, int NT, int EPV>
int64_t gn_cl_res_capacity() {
  static int per_cu[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (per_cu[dev] == 0) {
    int with_silu = 0, without = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &with_silu, reinterpret_cast<const void*>(gn_cl_resident_kernel<T, NT, EPV, true>), NT, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &without, reinterpret_cast<const void*>(gn_cl_resident_kernel<T, NT, EPV, false>), NT, 0) != hipSuccess)
      return 0;
    per_cu[dev] = std::min(with_silu, without);
    if (per_cu[dev] == 0) return 0;
  }
  return (int64_t)per_cu[dev] * device_cu_count();
}

template <typename T>
bool plan_gn_cl_res(int64_t N, int64_t C, int64_t S, int G, int force_epv, int layout, GnClResPlan& out) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NT = 512;
  constexpr int BCOLS = 8;  // columns of a block: 128 bytes of a position
  const int64_t CV = C / VEC;
  if (C % VEC || (C / G) % VEC || C > GN_CL_MAXC || G > GN_CL_MAXG || NT % CV) return false;
  const int epv = force_epv ? force_epv : 16;
  const int64_t cpv = (C / G) / VEC;
  const int64_t rows_grid = N * ((S + (int64_t)epv * (NT / CV) - 1) / ((int64_t)epv * (NT / CV)));
  const bool blocks_fit = CV > BCOLS && CV % BCOLS == 0 && BCOLS % cpv == 0 &&
                          (layout == 2 || rows_grid > device_cu_count());
  GnClResPlan p{NT, epv, 0, 0, 0, (int)CV, 1};
  int64_t nch = 0;
  bool ok = false;
  if (blocks_fit && layout != 1) {
    const int64_t sc = (int64_t)epv * (NT / BCOLS);
    nch = (S + sc - 1) / sc;
    const int64_t gw = G / (CV / BCOLS);
    if (nch <= GN_CLR_MAXNCH && N * G * nch <= GN_CLR_MAX_SLOTS && gw * nch <= GN_CLR_DIRECT) {
      p.CW = BCOLS;
      p.NB = (int)(CV / BCOLS);
      p.SC = (int)sc;
      p.NCH = (int)nch;
      p.two_level = 0;
      ok = true;
    }
  }
  if (!ok) {
    const int64_t sc = (int64_t)epv * (NT / CV);
    nch = (S + sc - 1) / sc;
    if (nch > GN_CLR_MAXNCH || N * G * nch > GN_CLR_MAX_SLOTS || N * G > GN_CLR_MAX_FINALS) return false;
    p.SC = (int)sc;
    p.NCH = (int)nch;
    if (nch >= G) p.two_level = 1;
    else if (G * nch <= GN_CLR_DIRECT) p.two_level = 0;
    else return false;
  }
  const int64_t nblk = N * p.NB * nch;
  const int64_t cap = epv == 16 ? gn_cl_res_capacity<T, NT, 16>() : gn_cl_res_capacity<T, NT, 8>();
  if (nblk > cap || nblk > (int64_t)GN_CLR_BLOCK * GN_CLR_MAXBLK) return false;
  if (!force_epv && nblk < device_cu_count()) return false;
  out = p;
  return true;
}

// Whether both 2-wave builds fit one workgroup per CU (checked once per device): grids of at
// most one workgroup per CU are then resident at once with either build.
template <typename T>
bool gn_cl_res_two_wave_ok() {
  static int ok[64] = {0};  // 0 unknown, 1 yes, -1 no
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (ok[dev] == 0) {
    int a = 0, b = 0;
    const bool q =
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &a, reinterpret_cast<const void*>(gn_cl_resident_kernel<T, 512, 16, true, 2>), 512, 0) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void*>(gn_cl_resident_kernel<T, 512, 16, false, 2>), 512, 0) == hipSuccess;
    ok[dev] = (q && a >= 1 && b >= 1) ? 1 : -1;
  }
  return ok[dev] > 0;
}

template <typename T>
int launch_gn_cl_res(const GnClResArgs& a, const GnClResPlan& p, int64_t N, int silu, hipStream_t s) {
  const dim3 grid((unsigned)(N * p.NB * p.NCH)), block(p.nt);
  if (p.epv == 16 && (int64_t)grid.x <= device_cu_count() && gn_cl_res_two_wave_ok<T>()) {
    if (silu) hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 16, true, 2>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 16, false, 2>), grid, block, 0, s, a);
  } else if (p.epv == 16) {
    if (silu) hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 16, false>), grid, block, 0, s, a);
  } else {
    if (silu) hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 8, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gn_cl_resident_kernel<T, 512, 8, false>), grid, block, 0, s, a);
  }
  return check_launch("gn_cl_resident_kernel");
}

// ---------------------------------------------------------------------------------------
// Channels-last GroupNorm backward (x, dy, dx: [n][s][c]); the math of the NC[S] backward
// above, without the layout conversions.  Three kernels, 5 tensor passes (x and dy read
// twice, the second time mostly from the Infinity Cache; dx written once):
//   stats: a workgroup per (n, spatial chunk); thread t owns one channel vector on rows
//          t / CV, t / CV + R, ... and accumulates per channel x's sums about a shift K (its
//          first x of that channel), sum dy and sum dy * (x - K); the workgroup then merges
//          its rows per channel, in row order, into the chunk's record
//          (mean, M2, A = sum dy, B = sum dy * (x - mean));
//   merge: a workgroup per (n, g) merges the group's (chunk, channel) records into the
//          group's mean and rstd, c1 = sum gamma*dy / E and c2 = rstd * sum gamma*dy*(x - mean) / E,
//          and writes each channel's dx coefficients and its dgamma / dbeta term of sample n;
//   apply: a workgroup per (n, chunk) forms dx = rstd*gamma_c*dy - rstd*c1 - rstd^2*c2*(x - mean),
//          each thread loading its channels' coefficients next to its first rows of x and dy;
//          workgroup (0, 0) also sums the parameter-gradient terms over n, in order
//          (deterministic).
struct GnClBwdArgs {
  const void* x;
  const void* dy;
  const void* gamma;
  void* dx;           // may be null
  float* dgamma;      // [C] or null
  float* dbeta;       // [C] or null
  float4* part;       // [N][NCH][C] chunk records (mean, M2, A, B)
  float4* coef;       // [N][C] dx coefficients (rstd * gamma_c, mean, -rstd^2 * c2, -rstd * c1)
  float2* dpar;       // [N][C] (dgamma term, dbeta term)
  int64_t S, SC;      // spatial positions, positions per chunk
  uint32_t sample_bytes;
  uint32_t C, G, cpg;
  int N, NCH;
  float eps;
  int pdt;
};

// (count, mean, M2, A = sum dy, B = sum dy * (x - mean)) of a set of positions
struct GnBwdRec {
  float n, mean, m2, a, b;
};

__device__ __forceinline__ void bwd_rec_merge(GnBwdRec& r, const GnBwdRec& o) {
  if (o.n == 0.f) return;
  if (r.n == 0.f) {
    r = o;
    return;
  }
  const float n = r.n + o.n, d = o.mean - r.mean;
  const float mean = r.mean + d * (o.n / n);
  r.m2 = r.m2 + o.m2 + d * d * (r.n * o.n / n);
  r.b = (r.b + (r.mean - mean) * r.a) + (o.b + (o.mean - mean) * o.a);
  r.a = r.a + o.a;
  r.mean = mean;
  r.n = n;
}

constexpr int GN_CL_BWD_U = 4;  // rows of x and of dy in flight per thread

template <typename T>
__global__ __launch_bounds__(GN_CL_NT) void gn_cl_bwd_stats_kernel(GnClBwdArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float4 rec[GN_CL_NT * VEC];  // [row phase rr][channel]
  __shared__ float cnt_s[GN_CL_NT];
  const int n = blockIdx.y, ch = blockIdx.x;
  const int CV = (int)(a.C / VEC), R = GN_CL_NT / CV;
  const int v = threadIdx.x % CV, rr = threadIdx.x / CV;
  const int64_t s0 = (int64_t)ch * a.SC, s1 = min(a.S, s0 + a.SC);
  const int64_t base = (int64_t)n * a.S * a.C;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + base, a.sample_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(static_cast<const T*>(a.dy) + base, a.sample_bytes);
  const uint32_t vb = (uint32_t)(v * VEC * sizeof(T)), rowb = (uint32_t)(a.C * sizeof(T));
  float K[VEC], t1[VEC], t2[VEC], sa[VEC], sb[VEC];
  float cnt = 0.f;
  {
    Vec16<T> k0;
    k0.raw = bload16(rx, s0 + rr < s1 ? (uint32_t)(s0 + rr) * rowb + vb : kOOB, 0);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      K[k] = to_f32(k0.e[k]);
      t1[k] = t2[k] = sa[k] = sb[k] = 0.f;
    }
  }
  for (int64_t s = s0 + rr; s < s1; s += (int64_t)R * GN_CL_BWD_U) {
    Vec16<T> xv[GN_CL_BWD_U], gv[GN_CL_BWD_U];
#pragma unroll
    for (int u = 0; u < GN_CL_BWD_U; ++u) {
      const int64_t sp = s + (int64_t)u * R;
      const uint32_t off = sp < s1 ? (uint32_t)sp * rowb + vb : kOOB;
      xv[u].raw = bload16(rx, off, 0);  // cached: the apply kernel reads x and dy again
      gv[u].raw = bload16(rg, off, 0);
    }
#pragma unroll
    for (int u = 0; u < GN_CL_BWD_U; ++u) {
      const float m = (s + (int64_t)u * R < s1) ? 1.f : 0.f;
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float d = (to_f32(xv[u].e[k]) - K[k]) * m;
        const float g = to_f32(gv[u].e[k]);  // 0 past the chunk (out-of-range loads)
        t1[k] += d;
        t2[k] = fmaf(d, d, t2[k]);
        sa[k] += g;
        sb[k] = fmaf(g, d, sb[k]);
      }
      cnt += m;
    }
  }
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (cnt > 0.f) {
      const float q = t1[k] / cnt;
      o = make_float4(K[k] + q, fmaxf(fmaf(-t1[k], q, t2[k]), 0.f), sa[k], fmaf(-q, sa[k], sb[k]));
    }
    rec[rr * a.C + v * VEC + k] = o;
  }
  if (v == 0) cnt_s[rr] = cnt;
  __syncthreads();
  float4* out = a.part + ((int64_t)n * a.NCH + ch) * a.C;
  for (uint32_t c = threadIdx.x; c < a.C; c += GN_CL_NT) {
    GnBwdRec r{0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r2 = 0; r2 < R; ++r2) {
      const float4 e = rec[r2 * a.C + c];
      bwd_rec_merge(r, GnBwdRec{cnt_s[r2], e.x, e.y, e.z, e.w});
    }
    out[c] = make_float4(r.mean, r.m2, r.a, r.b);
  }
}

// Two flat passes over the group's (chunk, channel) records, no per-record division:
//   1. mean  = sum len * mean_r / E;
//   2. M2    = sum (M2_r + len * (mean_r - mean)^2), and per channel A_c = sum A_r and
//      B_c   = sum (B_r + (mean_r - mean) * A_r), i.e. sum dy * (x - mean) about the group mean.
// Thread t = p * cblk + j takes channel j's chunks p, p + tpc, ... (lanes run along the
// channels, so a wave's loads are contiguous runs of a chunk's records); a channel's tpc
// partial sums are added in p order, the group totals in thread order (deterministic).
constexpr int GN_CL_BWD_MNT = 1024;
__global__ __launch_bounds__(GN_CL_BWD_MNT) void gn_cl_bwd_merge_kernel(GnClBwdArgs a) {
  __shared__ float red[GN_CL_BWD_MNT / 64];
  __shared__ float2 part_s[GN_CL_BWD_MNT];
  const int64_t ng = blockIdx.x;  // n * G + g
  const int n = (int)(ng / a.G);
  const uint32_t g = (uint32_t)(ng - (int64_t)n * a.G);
  const int tid = threadIdx.x;
  const int cblk = (int)min(a.cpg, (uint32_t)GN_CL_BWD_MNT);  // channels taken at once
  const int tpc = GN_CL_BWD_MNT / cblk;                       // threads per channel
  const int jt = tid % cblk, p = tid / cblk;
  const float4* pn = a.part + (int64_t)n * a.NCH * a.C + (int64_t)g * a.cpg;
  const float E = (float)((int64_t)a.cpg * a.S);
  auto len_of = [&](int q) { return (float)(min(a.S, (int64_t)(q + 1) * a.SC) - (int64_t)q * a.SC); };
  // pass 1: the group mean
  float sm = 0.f;
  for (int j0 = 0; j0 < (int)a.cpg; j0 += cblk) {
    const int j = j0 + jt;
    if (p < tpc && j < (int)a.cpg) {
#pragma unroll 4
      for (int q = p; q < a.NCH; q += tpc) sm = fmaf(len_of(q), pn[(int64_t)q * a.C + j].x, sm);
    }
  }
  const float mu = block_sum<GN_CL_BWD_MNT>(sm, red) / E;
  // pass 2: M2 and the per-channel sums about mu
  float m2 = 0.f, sg = 0.f, sgx = 0.f;
  for (int j0 = 0; j0 < (int)a.cpg; j0 += cblk) {
    const int j = j0 + jt;
    float ca = 0.f, cb = 0.f;
    if (p < tpc && j < (int)a.cpg) {
#pragma unroll 4
      for (int q = p; q < a.NCH; q += tpc) {
        const float4 e = pn[(int64_t)q * a.C + j];
        const float dm = e.x - mu;
        m2 += e.y + len_of(q) * dm * dm;
        ca += e.z;
        cb += e.w + dm * e.z;
      }
    }
    part_s[tid] = make_float2(ca, cb);
    __syncthreads();
    if (tid < cblk && j0 + tid < (int)a.cpg) {
      float A = 0.f, B = 0.f;
      for (int q = 0; q < tpc; ++q) {
        A += part_s[q * cblk + tid].x;
        B += part_s[q * cblk + tid].y;
      }
      const uint32_t c = g * a.cpg + j0 + tid;
      const float gam = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
      sg = fmaf(gam, A, sg);
      sgx = fmaf(gam, B, sgx);
      a.dpar[(int64_t)n * a.C + c] = make_float2(B, A);  // B scaled by rstd below
    }
    __syncthreads();
  }
  m2 = block_sum<GN_CL_BWD_MNT>(m2, red);
  sg = block_sum<GN_CL_BWD_MNT>(sg, red);
  sgx = block_sum<GN_CL_BWD_MNT>(sgx, red);
  const float rstd = 1.0f / sqrtf(m2 / E + a.eps);
  const float c1 = sg / E, c2 = rstd * sgx / E;
  // per channel: the dx coefficients, and the dgamma term rstd * sum dy * (x - mean) (this
  // thread wrote the dpar entries it scales: same thread, program order)
  for (uint32_t j = tid; j < a.cpg; j += GN_CL_BWD_MNT) {
    const uint32_t c = g * a.cpg + j;
    const float gam = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
    a.coef[(int64_t)n * a.C + c] = make_float4(rstd * gam, mu, -rstd * rstd * c2, -rstd * c1);
  }
  for (int j0 = 0; j0 < (int)a.cpg; j0 += cblk)
    if (tid < cblk && j0 + tid < (int)a.cpg) {
      float2* d = a.dpar + (int64_t)n * a.C + g * a.cpg + j0 + tid;
      d->x *= rstd;
    }
}

template <typename T>
__global__ __launch_bounds__(GN_CL_NT) void gn_cl_bwd_apply_kernel(GnClBwdArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  const int n = blockIdx.y, ch = blockIdx.x;
  const int CV = (int)(a.C / VEC), R = GN_CL_NT / CV;
  const int v = threadIdx.x % CV, rr = threadIdx.x / CV;
  const int64_t s0 = (int64_t)ch * a.SC, s1 = min(a.S, s0 + a.SC);
  const int64_t base = (int64_t)n * a.S * a.C;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const T*>(a.x) + base, a.sample_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(static_cast<const T*>(a.dy) + base, a.sample_bytes);
  const uint32_t vb = (uint32_t)(v * VEC * sizeof(T)), rowb = (uint32_t)(a.C * sizeof(T));
  if (a.dx) {
    Vec16<T> xv[GN_CL_BWD_U], gv[GN_CL_BWD_U];
    auto issue = [&](int64_t s) {
#pragma unroll
      for (int u = 0; u < GN_CL_BWD_U; ++u) {
        const int64_t sp = s + (int64_t)u * R;
        const uint32_t off = sp < s1 ? (uint32_t)sp * rowb + vb : kOOB;
        xv[u].raw = bload16<2>(rx, off, 0);  // last reads of x and dy
        gv[u].raw = bload16<2>(rg, off, 0);
      }
    };
    // the first rows and this thread's channel coefficients are requested together
    const int64_t s_first = s0 + rr;
    issue(s_first);
    const float4* cf = a.coef + (int64_t)n * a.C + v * VEC;
    float P[VEC], M[VEC], Q[VEC], Rc[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float4 e = cf[k];
      P[k] = e.x;
      M[k] = e.y;
      Q[k] = e.z;
      Rc[k] = e.w;
    }
    T* __restrict__ dxn = static_cast<T*>(a.dx) + base + v * VEC;
    for (int64_t s = s_first; s < s1; s += (int64_t)R * GN_CL_BWD_U) {
      if (s != s_first) issue(s);
#pragma unroll
      for (int u = 0; u < GN_CL_BWD_U; ++u) {
        const int64_t sp = s + (int64_t)u * R;
        float o[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          o[k] = fmaf(P[k], to_f32(gv[u].e[k]), fmaf(Q[k], to_f32(xv[u].e[k]) - M[k], Rc[k]));
        if (sp < s1) st16<true>(dxn + sp * a.C, pack16<T>(o));
      }
    }
  }
  if (n != 0 || ch != 0 || (!a.dgamma && !a.dbeta)) return;
  for (uint32_t c = threadIdx.x; c < a.C; c += GN_CL_NT) {
    float sgm = 0.f, sbt = 0.f;
    for (int m = 0; m < a.N; ++m) {
      const float2 d = a.dpar[(int64_t)m * a.C + c];
      sgm += d.x;
      sbt += d.y;
    }
    if (a.dgamma) a.dgamma[c] = sgm;
    if (a.dbeta) a.dbeta[c] = sbt;
  }
}

// About 512 workgroups (two per CU; each keeps 32 KB of x and dy in flight), at least 64
// positions per chunk: fewer, larger chunks than the forward's, since every chunk leaves a
// 16-byte record per channel that the merge reads twice.
inline GnClPlan plan_gn_cl_bwd(int64_t N, int64_t S) {
  int64_t nch = (512 + N - 1) / N;
  nch = std::max<int64_t>(1, std::min<int64_t>(nch, (S + 63) / 64));
  GnClPlan p;
  p.SC = (S + nch - 1) / nch;
  p.NCH = (int)((S + p.SC - 1) / p.SC);
  return p;
}

template <typename T>
int launch_gn_cl_bwd(const GnClBwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)a.NCH, (unsigned)a.N), block(GN_CL_NT);
  hipLaunchKernelGGL((gn_cl_bwd_stats_kernel<T>), grid, block, 0, s, a);
  int rc = check_launch("gn_cl_bwd_stats_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(gn_cl_bwd_merge_kernel, dim3((unsigned)((int64_t)a.N * a.G)), dim3(GN_CL_BWD_MNT), 0, s, a);
  rc = check_launch("gn_cl_bwd_merge_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((gn_cl_bwd_apply_kernel<T>), grid, block, 0, s, a);
  return check_launch("gn_cl_bwd_apply_kernel");
}

// ---------------------------------------------------------------------------------------
// Channels-last GroupNorm backward, register-resident: one read of x and dy, one write of
// dx, in one launch plus a small finalize for the parameter gradients.  The chunking,
// slots, epoch tags, stand-ins and the direct / two-level merge are the forward's
// (gn_cl_resident_kernel); a chunk here holds EPV vectors of x and EPV of dy per thread.
// Per (chunk, group) the record is (mean, M2) of x and, with gamma_c per channel,
//   A = sum gamma_c dy,   B = sum gamma_c dy (x - mean_chunk),
// merged over chunks as  A = sum A_i,  B = sum (B_i + (mean_i - mu) A_i).  Then, as in the
// NC[S] backward, c1 = A / E, c2 = B rstd / E and  dx = rstd (gamma_c dy - c1 - (x - mu) rstd c2).
// Each workgroup also writes a row of per-channel sums over its chunk, (rstd sum dy (x - mu),
// sum dy); the finalize kernel adds the rows of every workgroup in a fixed order into
// dgamma / dbeta.  Records travel as two slots (mean, M2) and (A, B), results as (mu, var),
// (A, B).
// ---------------------------------------------------------------------------------------
struct GnClBwdResArgs {
  const void* x;
  const void* dy;
  const void* gamma;
  void* dx;             // may be null
  float* dgamma;        // [C] or null
  float* dbeta;         // [C] or null
  uint32_t* hdr;        // workspace header (zero at allocation)
  GnSlot* slots;        // [N][G][NCH][2]
  GnSlot* finals;       // [N][G][2]
  float2* rows;         // [N * NCH][C] (dgamma term, dbeta term) of each workgroup
  int64_t S;
  int SC, NCH;
  int C, G, cpg, N;
  int two_level;
  int pdt;
  float eps;
  uint64_t wait_ticks;
};

template <typename A>
__device__ __forceinline__ int clb_positions(const A& a, int c) {
  const int64_t left = a.S - (int64_t)c * a.SC;
  return left < a.SC ? (int)left : a.SC;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t clb_rsrc(const void* t, const GnClBwdResArgs& a, int n, int c,
                                                           int es) {
  const char* base = static_cast<const char*>(t) + (((int64_t)n * a.S + (int64_t)c * a.SC) * a.C) * es;
  return make_rsrc(base, (uint32_t)((int64_t)clb_positions(a, c) * a.C * es));
}

// Per-group records of chunk `ch` into r4[0..3][g] (mean, M2, A, B).  Thread t accumulates,
// about K = its first x element, sum (x - K), sum (x - K)^2, A_t = sum gamma dy and
// sum gamma dy (x - K); its (n, mean, M2, A, B about its own mean) go to LDS, and each group's
// threads are merged by segmented butterflies.  FROM_REG: the owner, on its registers, which
// also leaves per channel pdy[k] = sum dy and pdx[k] = sum dy (x - K) for the parameter
// gradients; otherwise a stand-in, on memory, with the same arithmetic for the records.
template <typename T, int NT, int EPV, bool FROM_REG>
__device__ __forceinline__ void clb_chunk_stats(Vec16<T>* xb, Vec16<T>* db, __amdgpu_buffer_rsrc_t rx,
                                                __amdgpu_buffer_rsrc_t rd, int P, const GnClBwdResArgs& a,
                                                const float* gam, float* e5, float* red, float* r4, float& Kout,
                                                float* pdy, float* pdx) {
  constexpr int VEC = 16 / sizeof(T);
  const int tid = threadIdx.x;
  const int CV = a.C / VEC;
  const int nv = P * CV;
  const int v = tid % CV;
  float gm[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) gm[k] = gam[v * VEC + k];
  auto getx = [&](int i) -> Vec16<T> {
    if constexpr (FROM_REG) {
      return xb[i];
    } else {
      Vec16<T> r;
      r.raw = bload16(rx, (uint32_t)tid * 16u, (uint32_t)(i * NT * 16));
      return r;
    }
  };
  auto getd = [&](int i) -> Vec16<T> {
    if constexpr (FROM_REG) {
      return db[i];
    } else {
      Vec16<T> r;
      r.raw = bload16(rd, (uint32_t)tid * 16u, (uint32_t)(i * NT * 16));
      return r;
    }
  };
  const float K = to_f32(getx(0).e[0]);
  float s1 = 0.f, s2 = 0.f, sa = 0.f, sb = 0.f;
  int nvt = 0;
  auto acc = [&](int i) {
    const bool ok = i * NT + tid < nv;
    const float Ki = ok ? K : 0.f;
    if constexpr (FROM_REG)
      asm volatile("" : "+v"(xb[i].raw.x), "+v"(xb[i].raw.y), "+v"(xb[i].raw.z), "+v"(xb[i].raw.w),
                   "+v"(db[i].raw.x), "+v"(db[i].raw.y), "+v"(db[i].raw.z), "+v"(db[i].raw.w), "+v"(s1), "+v"(s2),
                   "+v"(sa), "+v"(sb));
    const Vec16<T> xv = getx(i), dv = getd(i);
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float d = to_f32(xv.e[k]) - Ki;  // vectors past the chunk read zero: d = 0, dy = 0
      const float g = to_f32(dv.e[k]);
      s1 += d;
      s2 = fmaf(d, d, s2);
      const float gg = gm[k] * g;
      sa += gg;
      sb = fmaf(gg, d, sb);
      if constexpr (FROM_REG) {
        pdy[k] += g;
        pdx[k] = fmaf(g, d, pdx[k]);
      }
    }
    // the per-channel sums are needed only at the end: left free, the compiler defers them
    // there and keeps every vector's converted x and dy alive (and spills them)
    if constexpr (FROM_REG) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) asm volatile("" : "+v"(pdy[k]), "+v"(pdx[k]));
    }
    nvt += ok ? 1 : 0;
  };
  if constexpr (FROM_REG) {
#pragma unroll
    for (int i = 0; i < EPV; ++i) acc(i);
  } else {
#pragma unroll 1
    for (int i = 0; i < EPV; ++i) acc(i);
  }
  const float nt = (float)(nvt * VEC);
  float mean_t = 0.f, m2_t = 0.f, b_t = 0.f;
  if (nvt > 0) {
    const float q = s1 / nt;
    mean_t = K + q;
    m2_t = fmaxf(fmaf(-s1, q, s2), 0.f);
    b_t = fmaf(-q, sa, sb);  // sum gamma dy (x - mean_t) = sum gamma dy (x - K) - (mean_t - K) A_t
  }
  Kout = K;
  e5[tid] = nt;
  e5[NT + tid] = mean_t;
  e5[2 * NT + tid] = m2_t;
  e5[3 * NT + tid] = sa;
  e5[4 * NT + tid] = b_t;
  __syncthreads();
  const int cpv = a.cpg / VEC, M = NT / a.G;
  const int g = tid / M, j = tid - (tid / M) * M;
  const int e = (j / cpv) * CV + g * cpv + (j - (j / cpv) * cpv);
  const float ne = e5[e], me = e5[NT + e], qe = e5[2 * NT + e], ae = e5[3 * NT + e], be = e5[4 * NT + e];
  const float n = seg_sum<NT>(ne, M, red);
  const float mean = seg_sum<NT>(ne * me, M, red) / n;
  const float d = me - mean;
  const float m2 = seg_sum<NT>(fmaf(ne * d, d, qe), M, red);
  const float A = seg_sum<NT>(ae, M, red);
  const float B = seg_sum<NT>(fmaf(d, ae, be), M, red);
  if (j == 0) {
    r4[g] = mean;
    r4[GN_CL_MAXG + g] = m2;
    r4[2 * GN_CL_MAXG + g] = A;
    r4[3 * GN_CL_MAXG + g] = B;
  }
  __syncthreads();
}

// (mu, var, A, B) of a group from its NCH chunk records t4[0..3][c], on one wave (lanes over
// chunks, then the xor butterfly: every lane and every workgroup gets the same bits).
__device__ __forceinline__ void clb_merge_group(const GnClBwdResArgs& a, const float* t4, int stride, float out[4]) {
  const int lane = threadIdx.x & 63;
  const float E = (float)(a.S * a.cpg);
  float sm = 0.f, sa = 0.f;
  for (int c = lane; c < a.NCH; c += 64) {
    sm = fmaf((float)(clb_positions(a, c) * a.cpg), t4[c], sm);
    sa += t4[2 * stride + c];
  }
  const float mu = wave_sum(sm) / E;
  float m2 = 0.f, b = 0.f;
  for (int c = lane; c < a.NCH; c += 64) {
    const float d = t4[c] - mu;
    m2 += t4[stride + c];
    m2 = fmaf((float)(clb_positions(a, c) * a.cpg) * d, d, m2);
    b = fmaf(d, t4[2 * stride + c], b + t4[3 * stride + c]);
  }
  out[0] = mu;
  out[1] = wave_sum(m2) / E;
  out[2] = wave_sum(sa);
  out[3] = wave_sum(b);
}

// Workgroup-wide: records r < nrec (group gr(r) of chunk cr(r)) into t4[0..3][r] (stride
// GN_CLR_DIRECT); this workgroup's own chunk from r4.  Polls as the forward's cl_collect;
// chunks still missing at the deadline are computed from x and dy by the whole workgroup.
template <typename T, int NT, int EPV, int RPT, typename GR, typename CR>
__device__ __forceinline__ void clb_collect(const GnClBwdResArgs& a, int n, int ch, uint32_t tag, uint64_t deadline,
                                            int nrec, GR gr, CR cr, float* t4, const float* r4, const float* gam,
                                            float* e5, float* red, float* x4, int* s_flag, int* s_list, int* s_cnt) {
  constexpr int ST = GN_CLR_DIRECT;
  const int tid = threadIdx.x;
  bool need[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int r = tid + k * NT;
    need[k] = false;
    if (r < nrec) {
      if (cr(r) == ch) {
#pragma unroll
        for (int q = 0; q < 4; ++q) t4[q * ST + r] = r4[q * GN_CL_MAXG + gr(r)];
      } else {
        need[k] = true;
      }
    }
  }
  for (;;) {
    float v[RPT][4];
    bool ok[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      ok[k] = false;
      if (need[k]) {
        const int r = tid + k * NT;
        const GnSlot* sl = &a.slots[(((int64_t)n * a.G + gr(r)) * a.NCH + cr(r)) * 2];
        const bool o0 = read_slot(sl, tag, v[k][0], v[k][1]);
        const bool o1 = read_slot(sl + 1, tag, v[k][2], v[k][3]);
        ok[k] = o0 && o1;
      }
    }
    bool left = false;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      if (need[k] && ok[k]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) t4[q * ST + tid + k * NT] = v[k][q];
        need[k] = false;
      }
      left = left || need[k];
    }
    if (!left || wall_clock64() > deadline) break;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k)
    if (need[k]) {
      const int c = cr(tid + k * NT);
      if (atomicExch(&s_flag[c], 1) == 0) s_list[atomicAdd(s_cnt, 1)] = c;
    }
  __syncthreads();
  const int nmiss = *s_cnt;
  if (nmiss > 0) {
    if (tid == 0) __hip_atomic_store(a.hdr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int m = 0; m < nmiss; ++m) {
      const int c = s_list[m];
      float Kd;
      clb_chunk_stats<T, NT, EPV, false>(nullptr, nullptr, clb_rsrc(a.x, a, n, c, (int)sizeof(T)),
                                         clb_rsrc(a.dy, a, n, c, (int)sizeof(T)), clb_positions(a, c), a, gam, e5,
                                         red, x4, Kd, nullptr, nullptr);
      for (int r = tid; r < nrec; r += NT)
        if (cr(r) == c) {
#pragma unroll
          for (int q = 0; q < 4; ++q) t4[q * ST + r] = x4[q * GN_CL_MAXG + gr(r)];
        }
      // publish all of the stand-in chunk's records (as the forward's cl_collect does)
      for (int g = tid; g < a.G; g += NT) {
        GnSlot* sl = &a.slots[(((int64_t)n * a.G + g) * a.NCH + c) * 2];
        write_slot(sl, tag, x4[g], x4[GN_CL_MAXG + g]);
        write_slot(sl + 1, tag, x4[2 * GN_CL_MAXG + g], x4[3 * GN_CL_MAXG + g]);
      }
      __threadfence();
      __syncthreads();
    }
    for (int m = tid; m < nmiss; m += NT) s_flag[s_list[m]] = 0;
    __syncthreads();
    if (tid == 0) *s_cnt = 0;
    __syncthreads();
  }
}

// 512 threads x 16 vectors of x and of dy: 128 registers of data per thread, so two waves per
// SIMD (256 VGPRs) and one workgroup per CU; at 8 vectors and four waves per SIMD the
// per-channel sums and gamma spilled.
template <typename T, int NT, int EPV>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2)))
void gn_cl_bwd_resident_kernel(GnClBwdResArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NW = NT / 64;
  constexpr int RPT = GN_CLR_DIRECT / NT;
  constexpr int ST = GN_CLR_DIRECT;
  __shared__ float e5[5 * NT];
  __shared__ float s_red[NW];
  __shared__ float r4[4 * GN_CL_MAXG], x4[4 * GN_CL_MAXG];  // own chunk's / a stand-in's records
  __shared__ float g4[4 * GN_CL_MAXG];                      // the sample's (mu, var, A, B) per group
  __shared__ float gam[GN_CL_MAXC];
  __shared__ float big[2 * NT * 8];                          // record table, then per-channel sums
  __shared__ int s_flag[GN_CLR_MAXNCH], s_list[GN_CLR_MAXNCH];
  __shared__ int s_cnt, s_gcnt;
  __shared__ int s_glist[GN_CL_MAXG + 1];
  static_assert(4 * GN_CLR_DIRECT <= 2 * NT * 8, "the record table fits");

  const int tid = threadIdx.x;
  const int n = blockIdx.x / a.NCH, ch = blockIdx.x - (blockIdx.x / a.NCH) * a.NCH;
  const int CV = a.C / VEC;
  const int P = clb_positions(a, ch);
  const int nv = P * CV;
  const int v = tid % CV, row = tid / CV, R = NT / CV;

  const uint32_t epoch = __hip_atomic_load(a.hdr + 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int c = tid; c < a.C; c += NT) gam[c] = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
  const __amdgpu_buffer_rsrc_t rx = clb_rsrc(a.x, a, n, ch, (int)sizeof(T));
  const __amdgpu_buffer_rsrc_t rd = clb_rsrc(a.dy, a, n, ch, (int)sizeof(T));
  Vec16<T> xb[EPV], db[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) xb[i].raw = bload16<2>(rx, (uint32_t)tid * 16u, (uint32_t)(i * NT * 16));
#pragma unroll
  for (int i = 0; i < EPV; ++i) db[i].raw = bload16<2>(rd, (uint32_t)tid * 16u, (uint32_t)(i * NT * 16));
  if (tid == 0) {
    s_cnt = 0;
    s_gcnt = a.two_level ? (ch < a.G ? 1 : 0) : 1;
    s_glist[0] = a.two_level ? ch : -1;
  }
  for (int c = tid; c < GN_CLR_MAXNCH; c += NT) s_flag[c] = 0;
  __syncthreads();  // gam

  float pdy[VEC], pdx[VEC], K;
#pragma unroll
  for (int k = 0; k < VEC; ++k) pdy[k] = pdx[k] = 0.f;
  clb_chunk_stats<T, NT, EPV, true>(xb, db, rx, rd, P, a, gam, e5, s_red, r4, K, pdy, pdx);
  reg_fence<T, EPV>(xb);
  reg_fence<T, EPV>(db);
  const uint32_t tag = (epoch << 1) | 1u;
  for (int g = tid; g < a.G; g += NT) {
    GnSlot* sl = &a.slots[(((int64_t)n * a.G + g) * a.NCH + ch) * 2];
    write_slot(sl, tag, r4[g], r4[GN_CL_MAXG + g]);
    write_slot(sl + 1, tag, r4[2 * GN_CL_MAXG + g], r4[3 * GN_CL_MAXG + g]);
  }
  const uint64_t deadline = wall_clock64() + a.wait_ticks;

  GnSlot* fin = a.finals + (int64_t)n * a.G * 2;
  const int NCH = a.NCH;
  bool polled = !a.two_level;
  for (int k = 0;;) {
    if (k < s_gcnt) {
      const int gf = s_glist[k++];
      clb_collect<T, NT, EPV, RPT>(a, n, ch, tag, deadline, gf < 0 ? a.G * NCH : NCH,
                                   [&](int r) { return gf < 0 ? r / NCH : gf; },
                                   [&](int r) { return gf < 0 ? r - (r / NCH) * NCH : r; }, big, r4, gam, e5, s_red,
                                   x4, s_flag, s_list, &s_cnt);
      __syncthreads();
      const int w = tid >> 6;
      for (int g = gf < 0 ? w : (w == 0 ? gf : a.G); g < (gf < 0 ? a.G : gf + 1); g += NW) {
        float o[4];
        clb_merge_group(a, gf < 0 ? big + g * NCH : big, ST, o);
        if ((tid & 63) == 0) {
#pragma unroll
          for (int q = 0; q < 4; ++q) g4[q * GN_CL_MAXG + g] = o[q];
          if (gf == ch && a.two_level) {
            write_slot(&fin[2 * gf], tag, o[0], o[1]);
            write_slot(&fin[2 * gf + 1], tag, o[2], o[3]);
          }
        }
      }
      __syncthreads();
      continue;
    }
    if (polled) break;
    polled = true;
    for (int g = tid; g < a.G; g += NT) {
      if (g == ch) continue;
      float o[4];
      bool ok;
      for (;;) {
        ok = read_slot(&fin[2 * g], tag, o[0], o[1]) && read_slot(&fin[2 * g + 1], tag, o[2], o[3]);
        if (ok || wall_clock64() > deadline) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (ok) {
#pragma unroll
        for (int q = 0; q < 4; ++q) g4[q * GN_CL_MAXG + g] = o[q];
      } else {
        s_glist[atomicAdd(&s_gcnt, 1)] = g;
      }
    }
    __syncthreads();
  }

  // this thread's channels lie in one group
  const int g = (v * VEC) / a.cpg;
  const float mu = g4[g], rstd = 1.0f / sqrtf(g4[GN_CL_MAXG + g] + a.eps);
  const float E = (float)(a.S * a.cpg);
  const float c1 = g4[2 * GN_CL_MAXG + g] / E;
  const float c2 = g4[3 * GN_CL_MAXG + g] * rstd / E;
  float gm[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) gm[k] = gam[v * VEC + k];
  if (a.dx) {
    T* __restrict__ dxc = static_cast<T*>(a.dx) + ((int64_t)n * a.S + (int64_t)ch * a.SC) * a.C;
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      reg_fence<T, 1>(&xb[i]);
      reg_fence<T, 1>(&db[i]);
      const int e = i * NT + tid;
      float o[VEC];
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float xh = (to_f32(xb[i].e[k]) - mu) * rstd;
        o[k] = rstd * (gm[k] * to_f32(db[i].e[k]) - c1 - xh * c2);
      }
      if (e < nv) st16<true>(dxc + (int64_t)e * VEC, pack16<T>(o));
    }
  }
  if (a.dgamma || a.dbeta) {
    // per channel over the chunk: rstd sum dy (x - mu) = rstd (pdx + (K - mu) pdy), sum dy;
    // the R threads of a column are added in row order (threads past the chunk hold zeros)
    float* cs = big;  // [R][C][2]
    const float sh = K - mu;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      cs[((int64_t)row * a.C + v * VEC + k) * 2] = rstd * fmaf(sh, pdy[k], pdx[k]);
      cs[((int64_t)row * a.C + v * VEC + k) * 2 + 1] = pdy[k];
    }
    __syncthreads();
    float2* out = a.rows + (int64_t)blockIdx.x * a.C;
    for (int c = tid; c < a.C; c += NT) {
      float sg = 0.f, sb = 0.f;
      for (int r = 0; r < R; ++r) {
        sg += cs[((int64_t)r * a.C + c) * 2];
        sb += cs[((int64_t)r * a.C + c) * 2 + 1];
      }
      out[c] = make_float2(sg, sb);
    }
  }
  // done with the slots: count in blocks of GN_CLR_BLOCK; the last advances the epoch
  if (tid == 0) {
    const uint32_t b = blockIdx.x / GN_CLR_BLOCK, nb = (gridDim.x + GN_CLR_BLOCK - 1) / GN_CLR_BLOCK;
    const uint32_t in_b = min((uint32_t)GN_CLR_BLOCK, gridDim.x - b * GN_CLR_BLOCK);
    uint32_t* bc = a.hdr + 64 + 32 * b;
    if (__hip_atomic_fetch_add(bc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == in_b - 1) {
      __hip_atomic_store(bc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(a.hdr + 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nb - 1) {
        __hip_atomic_store(a.hdr + 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.hdr + 16, (epoch + 1u) & 0x7fffffffu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// dgamma / dbeta: column c of the rows [nrows][C] summed in row order.  Each column's rows
// are split over CLBF_SPLIT threads (contiguous ranges, loaded CLBF_U at a time so the loads
// overlap), whose partials are then added in order: deterministic.
constexpr int CLBF_COLS = 16, CLBF_SPLIT = 32, CLBF_U = 8;
__global__ __launch_bounds__(CLBF_COLS * CLBF_SPLIT) void gn_cl_bwd_rows_finalize_kernel(const float2* rows, int nrows,
                                                                                         int C, float* dgamma,
                                                                                         float* dbeta) {
  __shared__ float2 part[CLBF_SPLIT][CLBF_COLS];
  const int cl = threadIdx.x % CLBF_COLS, sp = threadIdx.x / CLBF_COLS;
  const int c = blockIdx.x * CLBF_COLS + cl;
  const int per = (nrows + CLBF_SPLIT - 1) / CLBF_SPLIT;
  const int r0 = sp * per, r1 = min(nrows, r0 + per);
  float sg = 0.f, sb = 0.f;
  if (c < C)
    for (int r = r0; r < r1; r += CLBF_U) {
      float2 q[CLBF_U];
#pragma unroll
      for (int u = 0; u < CLBF_U; ++u)
        q[u] = r + u < r1 ? rows[(int64_t)(r + u) * C + c] : make_float2(0.f, 0.f);
#pragma unroll
      for (int u = 0; u < CLBF_U; ++u) {
        sg += q[u].x;
        sb += q[u].y;
      }
    }
  part[sp][cl] = make_float2(sg, sb);
  __syncthreads();
  if (sp == 0 && c < C) {
    float tg = 0.f, tb = 0.f;
    for (int k = 0; k < CLBF_SPLIT; ++k) {
      tg += part[k][cl].x;
      tb += part[k][cl].y;
    }
    if (dgamma) dgamma[c] = tg;
    if (dbeta) dbeta[c] = tb;
  }
}

struct GnClBwdResPlan {
  int NCH, SC, two_level;
};

template <typename T>
int64_t gn_cl_bwd_res_capacity() {
  static int per_cu[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (per_cu[dev] == 0 &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu[dev], reinterpret_cast<const void*>(gn_cl_bwd_resident_kernel<T, 512, 16>), 512, 0) != hipSuccess)
    return 0;
  return (int64_t)per_cu[dev] * device_cu_count();
}

// Register-resident configuration (512 threads x 16 vectors of x and of dy) for a shape, or
// false.  Taken when the grid covers every CU and fits at once (`force` takes it wherever
// it fits); merge forms as the forward's.
template <typename T>
bool plan_gn_cl_bwd_res(int64_t N, int64_t C, int64_t S, int G, bool force, GnClBwdResPlan& out) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NT = 512, EPV = 16;
  const int64_t CV = C / VEC;
  if (C % VEC || (C / G) % VEC || C > GN_CL_MAXC || G > GN_CL_MAXG || NT % CV) return false;
  const int64_t sc = (int64_t)EPV * (NT / CV);
  const int64_t nch = (S + sc - 1) / sc;
  if (nch > GN_CLR_MAXNCH || 2 * N * G * nch > GN_CLR_MAX_SLOTS || 2 * N * G > GN_CLR_MAX_FINALS) return false;
  GnClBwdResPlan p{(int)nch, (int)sc, 0};
  if (nch >= G) p.two_level = 1;
  else if (G * nch <= GN_CLR_DIRECT) p.two_level = 0;
  else return false;
  const int64_t nblk = N * nch;
  if (nblk > gn_cl_bwd_res_capacity<T>() || nblk > (int64_t)GN_CLR_BLOCK * GN_CLR_MAXBLK) return false;
  if (!force && nblk < device_cu_count()) return false;
  out = p;
  return true;
}

template <typename T>
int launch_gn_cl_bwd_res(const GnClBwdResArgs& a, int64_t N, hipStream_t s) {
  hipLaunchKernelGGL((gn_cl_bwd_resident_kernel<T, 512, 16>), dim3((unsigned)(N * a.NCH)), dim3(512), 0, s, a);
  int rc = check_launch("gn_cl_bwd_resident_kernel");
  if (rc || !(a.dgamma || a.dbeta)) return rc;
  hipLaunchKernelGGL(gn_cl_bwd_rows_finalize_kernel, dim3((unsigned)((a.C + CLBF_COLS - 1) / CLBF_COLS)),
                     dim3(CLBF_COLS * CLBF_SPLIT), 0, s, a.rows, (int)(N * a.NCH), a.C, a.dgamma, a.dbeta);
  return check_launch("gn_cl_bwd_rows_finalize_kernel");
}

}  // namespace

int group_norm_num_variants() { return kNumGn; }
const char* group_norm_variant_name(int v) {
  return (v >= 0 && v < kNumGn) ? kGnVariants[v].name : nullptr;
}

}  // namespace atk

extern "C" size_t atk_group_norm_workspace_bytes(int64_t N, int64_t C, int64_t S, int G, int dtype,
                                                 int variant) {
  using namespace atk;
  if (variant < 0) variant = 0;
  if (validate_gn(N, C, S, G, dtype, variant)) return 0;
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p)) return 0;
  return p.ws_bytes;
}

extern "C" size_t atk_group_norm_workspace_zero_bytes(int64_t N, int64_t C, int64_t S, int G,
                                                      int dtype, int variant) {
  using namespace atk;
  if (variant < 0) variant = 0;
  if (validate_gn(N, C, S, G, dtype, variant)) return 0;
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p)) return 0;
  return p.zero_bytes;
}

namespace atk {
namespace {

// The forward behind both entry points: `ws` is the caller's workspace or the static scratch.
int gn_fwd(const void* x, const void* gamma, const void* beta, void* y, int64_t N, int64_t C, int64_t S,
           int G, float eps, int fuse_silu, int dtype, int param_dtype, int variant, void* workspace,
           size_t workspace_bytes, hipStream_t s, size_t* need_out) {
  if (variant < 0) variant = 0;
  int rc = validate_gn(N, C, S, G, dtype, variant);
  if (rc) return rc;
  if ((gamma || beta) && !dtype_ok(param_dtype))
    return fail(ATK_EINVAL, "group_norm: unknown param dtype code %d", param_dtype);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "group_norm: null pointer");
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p))
    return fail(ATK_UNSUPPORTED, "group_norm: %s does not take this shape (slices per group)",
                kGnVariants[variant].name);
  if (need_out) *need_out = p.ws_bytes;
  if (!workspace || workspace_bytes < p.ws_bytes)
    return fail(ATK_EINVAL, "group_norm: workspace of %zu bytes needed", p.ws_bytes);
  const size_t es = dtype_size(dtype);
  const int vec = (int)(16 / es);
  const bool vec_ok = (S % vec == 0) && aligned16(x) && aligned16(y);
  GnArgs a;
  a.trace = nullptr;
  a.x = x; a.gamma = gamma; a.beta = beta; a.y = y;
  a.E = (C / G) * S;
  a.S = (uint32_t)S;
  a.cpg = (uint32_t)(C / G);
  a.G = (uint32_t)G;
  a.NS = p.NS;
  a.slice = p.slice;
  a.eps = eps;
  a.silu = fuse_silu ? 1 : 0;
  a.pdt = param_dtype;
  a.div_s = make_fastdiv((uint32_t)S);
  char* ws = static_cast<char*>(workspace);
  a.diag = reinterpret_cast<uint32_t*>(ws);
  a.done = reinterpret_cast<uint32_t*>(ws + 256);
  a.slots = reinterpret_cast<GnSlot*>(ws + GN_SLOTS_OFF);
  a.partials = reinterpret_cast<float*>(ws + GN_PARTIALS_OFF);
  a.parts = reinterpret_cast<float4*>(ws + GN_PARTIALS_OFF);
  a.NP = p.NS;
  const int khz = device_wall_clock_khz();
  // ATK_GN_WAIT_US overrides the wait (tests set 0 to exercise the stand-in path)
  const char* wenv = getenv("ATK_GN_WAIT_US");
  const uint64_t wait_us = wenv ? strtoull(wenv, nullptr, 10) : GN_WAIT_US;
  a.wait_ticks = (uint64_t)(khz > 0 ? khz : 100000) * wait_us / 1000;
  a.tag = next_slot_tag();
  const int64_t ngroups = N * G;
  switch (dtype) {
    case ATK_F32: return launch_gn<float>(a, ngroups, variant, vec_ok, s);
    case ATK_F16: return launch_gn<_Float16>(a, ngroups, variant, vec_ok, s);
    default: return launch_gn<__bf16>(a, ngroups, variant, vec_ok, s);
  }
}

}  // namespace
}  // namespace atk

// Diagnostics: register (or, with NULL, drop) a device buffer of n_words 64-bit words that
// later register-resident launches fill with per-workgroup phase stamps; returns the wall-clock
// rate in kHz that converts them.
extern "C" int atk_group_norm_trace(void* device_words, int64_t n_words) {
  using namespace atk;
  g_gn_trace = device_words && n_words > 0 ? static_cast<uint64_t*>(device_words) : nullptr;
  g_gn_trace_words = g_gn_trace ? n_words : 0;
  return device_wall_clock_khz();
}

extern "C" int atk_group_norm_fwd(const void* x, const void* gamma, const void* beta, void* y,
                                  int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                                  int dtype, int param_dtype, int variant, void* workspace,
                                  size_t workspace_bytes, atk_stream_t stream) {
  return atk::gn_fwd(x, gamma, beta, y, N, C, S, G, eps, fuse_silu, dtype, param_dtype, variant, workspace,
                     workspace_bytes, reinterpret_cast<hipStream_t>(stream), nullptr);
}

// ---------------------------------------------------------------------------------------
// No-allocation GroupNorm forward.  The scratch that atk_group_norm_fwd takes from the caller
// (diagnostics word, per-group counters, slot table, two-pass partials) lives in a fixed
// device array instead.  Static device memory starts zeroed, and every launch leaves the
// counters and slots zero again, which is the state the kernels need.  Each GPU holds its own
// copy for the life of the process; its address is looked up once per device with
// hipGetSymbolAddress, and that address -- never the array's name, which in host code is only
// a stand-in -- is what the kernels get.
//
// The array holds GN_NOALLOC_SLICES slices of GN_NOALLOC_BYTES, one per stream: the first
// call from a stream binds the next free slice of the current device to that stream handle,
// and later calls from it reuse that slice.  Calls from one stream are ordered, so they never
// overlap on a slice; calls on different streams use different slices, so they may overlap.
// A further stream finds no slice and is refused (ATK_EINVAL) instead of sharing one.
// ---------------------------------------------------------------------------------------
namespace atk {
namespace {

constexpr size_t GN_NOALLOC_PARTIAL_BYTES = (size_t)1 << 20;  // 131072 (mean, M2) pairs
constexpr size_t GN_NOALLOC_BYTES = GN_PARTIALS_OFF + GN_NOALLOC_PARTIAL_BYTES;
constexpr int GN_NOALLOC_SLICES = 4;
constexpr int GN_NOALLOC_MAX_DEVICES = 64;
static_assert(GN_NOALLOC_BYTES % 256 == 0, "slices keep the array's 256-byte alignment");

static __device__ __align__(256) unsigned char scratch[GN_NOALLOC_SLICES * GN_NOALLOC_BYTES];

struct NoallocDevice {
  void* base = nullptr;                         // this device's copy of `scratch`
  hipStream_t owner[GN_NOALLOC_SLICES] = {};    // stream bound to each slice
  int used = 0;                                 // slices bound so far
};
std::mutex g_scratch_mu;
NoallocDevice g_noalloc[GN_NOALLOC_MAX_DEVICES];

// The slice of the current device's `scratch` bound to stream s (binding a free one on the
// stream's first call), resolving the array's address on the device's first call.
int current_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= GN_NOALLOC_MAX_DEVICES)
    return fail(ATK_ELAUNCH, "group_norm (no-alloc): no current device (or device index >= %d)",
                GN_NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  NoallocDevice& d = g_noalloc[dev];
  if (!d.base) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(ATK_ELAUNCH, "group_norm (no-alloc): hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(e));
    d.base = p;
  }
  int slice = -1;
  for (int i = 0; i < d.used; ++i)
    if (d.owner[i] == s) slice = i;
  if (slice < 0) {
    if (d.used == GN_NOALLOC_SLICES)
      return fail(ATK_EINVAL, "group_norm (no-alloc): the static scratch of device %d has %d stream slices and "
                  "all are bound to other streams; calls from a further stream would race on them (use "
                  "atk_group_norm_fwd with a workspace)", dev, GN_NOALLOC_SLICES);
    slice = d.used++;
    d.owner[slice] = s;
  }
  *out = static_cast<char*>(d.base) + (size_t)slice * GN_NOALLOC_BYTES;
  return ATK_OK;
}

}  // namespace
}  // namespace atk

extern "C" size_t atk_group_norm_noalloc_scratch_bytes(void) { return atk::GN_NOALLOC_BYTES; }

extern "C" int atk_group_norm_fwd_noalloc(const void* x, const void* gamma, const void* beta, void* y,
                                          int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                                          int dtype, int param_dtype, int variant, atk_stream_t stream) {
  using namespace atk;
  if (variant < 0) variant = 0;
  int rc = validate_gn(N, C, S, G, dtype, variant);
  if (rc) return rc;
  if (N == 0) return ATK_OK;
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p))
    return fail(ATK_UNSUPPORTED, "group_norm: %s does not take this shape (slices per group)",
                kGnVariants[variant].name);
  if (p.ws_bytes > GN_NOALLOC_BYTES)
    return fail(ATK_EINVAL, "group_norm (no-alloc): this shape and variant need %zu bytes of scratch; the "
                "static scratch holds %zu (use atk_group_norm_fwd with a workspace)", p.ws_bytes,
                GN_NOALLOC_BYTES);
  const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  rc = current_scratch(hs, &ws);
  if (rc) return rc;
  return gn_fwd(x, gamma, beta, y, N, C, S, G, eps, fuse_silu, dtype, param_dtype, variant, ws, GN_NOALLOC_BYTES,
                hs, nullptr);
}

extern "C" int atk_group_norm_apply(const void* x, const void* gamma, const void* beta, void* y, int64_t N,
                                    int64_t C, int64_t S, int G, float eps, int fuse_silu, int dtype,
                                    int param_dtype, const void* stats, int64_t records_per_group, int variant,
                                    atk_stream_t stream) {
  using namespace atk;
  if (variant < 0) {
    // default: the split variant with the largest slices whose grid still covers every CU (one
    // record merge per workgroup, so fewer, larger workgroups merge less), else the smallest
    // slices; split_nt1024_v4, split_nt512_v8, split_nt256_v8, split_nt256_v4 in that order
    static const int order[] = {15, 13, 12, 14};
    variant = 14;
    const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
    for (int v : order) {
      GnPlan q;
      if (validate_gn(N, C, S, G, dtype, v) == ATK_OK && plan_gn(N, C, S, G, dtype, v, q) && N * G * q.NS >= cus) {
        variant = v;
        break;
      }
    }
  }
  int rc = validate_gn(N, C, S, G, dtype, variant);
  if (rc) return rc;
  if (kGnVariants[variant].kind != GN_SPLIT)
    return fail(ATK_EINVAL, "group_norm apply: %s is not a split variant", kGnVariants[variant].name);
  if ((gamma || beta) && !dtype_ok(param_dtype))
    return fail(ATK_EINVAL, "group_norm apply: unknown param dtype code %d", param_dtype);
  if (N == 0) return ATK_OK;
  if (!x || !y || !stats || records_per_group <= 0 || records_per_group >= (1ll << 30))
    return fail(ATK_EINVAL, "group_norm apply: null pointer or bad record count");
  const int vec = (int)(16 / dtype_size(dtype));
  if (S % vec || !aligned16(x) || !aligned16(y) || !aligned16(stats))
    return fail(ATK_UNSUPPORTED, "group_norm apply: needs S %% %d == 0 and 16-byte aligned tensors", vec);
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p)) return fail(ATK_UNSUPPORTED, "group_norm apply: shape too large");
  GnArgs a = {};
  a.x = x; a.gamma = gamma; a.beta = beta; a.y = y;
  a.E = (C / G) * S;
  a.S = (uint32_t)S;
  a.cpg = (uint32_t)(C / G);
  a.G = (uint32_t)G;
  a.NS = p.NS;
  a.slice = p.slice;
  a.eps = eps;
  a.silu = fuse_silu ? 1 : 0;
  a.pdt = param_dtype;
  a.div_s = make_fastdiv((uint32_t)S);
  a.parts = static_cast<float4*>(const_cast<void*>(stats));
  a.NP = (int)records_per_group;
  const int64_t nblk = N * G * p.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm apply: grid too large");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const GnVariant& v = kGnVariants[variant];
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(v.nt), 0, s, a);
    return check_launch("gn_split_apply_kernel");
  };
#define ATK_GN_APPLY(T, NT_, EPV_)                                                                      \
  return a.silu ? go(gn_split_apply_kernel<T, NT_, EPV_, true>) : go(gn_split_apply_kernel<T, NT_, EPV_, false>)
#define ATK_GN_APPLY_T(T)                                        \
  switch (variant) {                                             \
    case 12: ATK_GN_APPLY(T, 256, 8);                            \
    case 13: ATK_GN_APPLY(T, 512, 8);                            \
    case 14: ATK_GN_APPLY(T, 256, 4);                            \
    default: ATK_GN_APPLY(T, 1024, 4);                           \
  }
  switch (dtype) {
    case ATK_F32: ATK_GN_APPLY_T(float);
    case ATK_F16: ATK_GN_APPLY_T(_Float16);
    default: ATK_GN_APPLY_T(__bf16);
  }
#undef ATK_GN_APPLY_T
#undef ATK_GN_APPLY
}

extern "C" size_t atk_group_norm_bwd_workspace_bytes(int64_t N, int64_t C) {
  if (N <= 0 || C <= 0) return 0;
  // per-group counters of the resident kernel (zero between launches), then per (n, c) row:
  // mean, M2, A, B, K (the rows / apply pair) or the resident kernel's two sums
  return atk::GN_BWD_CNT_BYTES + (size_t)N * (size_t)C * 5 * sizeof(float);
}

extern "C" int atk_group_norm_bwd(const void* x, const void* dy, const void* gamma, void* dx, float* dgamma,
                                  float* dbeta, int64_t N, int64_t C, int64_t S, int G, float eps, int dtype,
                                  int param_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype) || (gamma && !dtype_ok(param_dtype)))
    return fail(ATK_EINVAL, "group_norm backward: unknown dtype code");
  if (N <= 0 || C <= 0 || S <= 0 || G <= 0) return fail(ATK_EINVAL, "group_norm backward: bad sizes");
  if (C % G) return fail(ATK_EINVAL, "group_norm backward: channels (%lld) not divisible by groups (%d)",
                         (long long)C, G);
  if (!x || !dy) return fail(ATK_EINVAL, "group_norm backward: null pointer");
  const size_t need = atk_group_norm_bwd_workspace_bytes(N, C);
  if (!workspace || ws_bytes < need) return fail(ATK_EINVAL, "group_norm backward: workspace of %zu bytes needed", need);
  const int64_t es = (int64_t)dtype_size(dtype), vec = 16 / es;
  if (S % vec || !aligned16(x) || !aligned16(dy) || (dx && !aligned16(dx)))
    return fail(ATK_UNSUPPORTED, "group_norm backward: needs spatial size %% %lld == 0 and 16-byte aligned tensors",
                (long long)vec);
  const int64_t rows = N * C;
  if (rows >= (1ll << 31) || C >= (1ll << 31) || N >= (1ll << 31))
    return fail(ATK_UNSUPPORTED, "group_norm backward: too many rows");
  if (S * es >= (1ll << 31)) return fail(ATK_UNSUPPORTED, "group_norm backward: rows over 2 GiB (32-bit buffer offsets)");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int epv = gn_bwd_resident_epv(N, C, S, G, dtype);
  if (epv) {
    GnBwdResArgs r;
    r.x = x; r.dy = dy; r.gamma = gamma; r.dx = dx;
    r.dgamma = dgamma; r.dbeta = dbeta;
    r.counter = static_cast<uint32_t*>(workspace);
    r.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + GN_BWD_CNT_BYTES);
    r.E = (C / G) * S;
    r.S = (uint32_t)S; r.cpg = (uint32_t)(C / G); r.C = (uint32_t)C; r.G = (uint32_t)G;
    r.N = (int)N; r.eps = eps; r.pdt = param_dtype;
    r.div_s = make_fastdiv((uint32_t)S);
    switch (dtype) {
      case ATK_F32: return launch_gn_bwd_resident<float>(r, epv, s);
      case ATK_F16: return launch_gn_bwd_resident<_Float16>(r, epv, s);
      default: return launch_gn_bwd_resident<__bf16>(r, epv, s);
    }
  }
  GnBwdArgs a;
  a.x = x; a.dy = dy; a.gamma = gamma; a.dx = dx;
  a.rows = reinterpret_cast<float*>(static_cast<char*>(workspace) + GN_BWD_CNT_BYTES);
  a.dgamma = dgamma; a.dbeta = dbeta;
  a.S = S; a.C = (uint32_t)C; a.cpg = (uint32_t)(C / G); a.N = (int)N;
  a.eps = eps; a.pdt = param_dtype;
  switch (dtype) {
    case ATK_F32: return launch_gn_bwd<float>(a, rows, s);
    case ATK_F16: return launch_gn_bwd<_Float16>(a, rows, s);
    default: return launch_gn_bwd<__bf16>(a, rows, s);
  }
}

extern "C" size_t atk_group_norm_cl_workspace_bytes(int64_t N, int64_t C, int64_t S, int G) {
  if (N <= 0 || C <= 0 || S <= 0 || G <= 0) return 0;
  // the register-resident kernel's header and slots (fixed layout), then the three-kernel
  // path's chunk partials and group statistics
  const atk::GnClPlan p = atk::plan_gn_cl(N, S);
  return atk::GN_CLR_BYTES + ((size_t)N * (size_t)p.NCH + (size_t)N) * (size_t)G * 2 * sizeof(float);
}

extern "C" int atk_group_norm_cl_fwd(const void* x, const void* gamma, const void* beta, void* y, int64_t N,
                                     int64_t C, int64_t S, int G, float eps, int fuse_silu, int dtype,
                                     int param_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype) || ((gamma || beta) && !dtype_ok(param_dtype)))
    return fail(ATK_EINVAL, "group_norm (channels-last): unknown dtype code");
  if (N < 0 || C <= 0 || S < 0 || G <= 0) return fail(ATK_EINVAL, "group_norm (channels-last): bad sizes");
  if (C % G) return fail(ATK_EINVAL, "group_norm (channels-last): channels (%lld) not divisible by groups (%d)",
                         (long long)C, G);
  if (N == 0 || S == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "group_norm (channels-last): null pointer");
  const int64_t es = (int64_t)dtype_size(dtype), vec = 16 / es;
  const int64_t cpg = C / G;
  if (cpg % vec || C > GN_CL_MAXC || G > GN_CL_MAXG || GN_CL_NT % (C / vec) || !aligned16(x) || !aligned16(y))
    return fail(ATK_UNSUPPORTED, "group_norm (channels-last): needs C/G %% %lld == 0, C/%lld dividing %d and "
                "16-byte aligned tensors", (long long)vec, (long long)vec, GN_CL_NT);
  if (N >= 65536) return fail(ATK_UNSUPPORTED, "group_norm (channels-last): batch too large");
  if (S * C * es >= ((int64_t)1 << 31))
    return fail(ATK_UNSUPPORTED, "group_norm (channels-last): one sample over 2 GiB (32-bit buffer offsets)");
  const GnClPlan p = plan_gn_cl(N, S);
  const size_t need = atk_group_norm_cl_workspace_bytes(N, C, S, G);
  if (!workspace || ws_bytes < need)
    return fail(ATK_EINVAL, "group_norm (channels-last): workspace of %zu bytes needed", need);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Register-resident single pass where the library's rule takes it (plan_gn_cl_res);
  // ATK_GN_CL_RESIDENT=0 turns it off, =8 / =16 takes that many vectors per thread wherever
  // that configuration fits; ATK_GN_CL_LAYOUT=rows / blocks forces the chunk shape.
  const char* renv = getenv("ATK_GN_CL_RESIDENT");
  const int rmode = renv ? atoi(renv) : 1;
  if (rmode != 0) {
    const int force = (rmode == 8 || rmode == 16) ? rmode : 0;
    const char* lenv = getenv("ATK_GN_CL_LAYOUT");
    const int layout = !lenv ? 0 : !strcmp(lenv, "rows") ? 1 : !strcmp(lenv, "blocks") ? 2 : 0;
    GnClResPlan rp;
    const bool fits = dtype == ATK_F32   ? plan_gn_cl_res<float>(N, C, S, G, force, layout, rp)
                      : dtype == ATK_F16 ? plan_gn_cl_res<_Float16>(N, C, S, G, force, layout, rp)
                                         : plan_gn_cl_res<__bf16>(N, C, S, G, force, layout, rp);
    if (fits) {
      GnClResArgs r;
      r.x = x; r.gamma = gamma; r.beta = beta; r.y = y;
      char* ws = static_cast<char*>(workspace);
      r.hdr = reinterpret_cast<uint32_t*>(ws);
      r.slots = reinterpret_cast<GnSlot*>(ws + GN_CLR_SLOTS_OFF);
      r.finals = reinterpret_cast<GnSlot*>(ws + GN_CLR_FINALS_OFF);
      r.S = S; r.SC = rp.SC; r.NCH = rp.NCH;
      r.C = (int)C; r.G = G; r.cpg = (int)cpg;
      r.CW = rp.CW; r.NB = rp.NB; r.GW = G / rp.NB;
      r.trace = g_gn_trace && N * rp.NB * rp.NCH * 4 <= g_gn_trace_words ? g_gn_trace : nullptr;
      r.two_level = rp.two_level;
      r.pdt = param_dtype;
      r.eps = eps;
      const int khz = device_wall_clock_khz();
      const char* wenv = getenv("ATK_GN_WAIT_US");
      const uint64_t wait_us = wenv ? strtoull(wenv, nullptr, 10) : GN_WAIT_US;
      r.wait_ticks = (uint64_t)(khz > 0 ? khz : 100000) * wait_us / 1000;
      switch (dtype) {
        case ATK_F32: return launch_gn_cl_res<float>(r, rp, N, fuse_silu, s);
        case ATK_F16: return launch_gn_cl_res<_Float16>(r, rp, N, fuse_silu, s);
        default: return launch_gn_cl_res<__bf16>(r, rp, N, fuse_silu, s);
      }
    }
  }
  GnClArgs a;
  a.x = x; a.gamma = gamma; a.beta = beta; a.y = y;
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + GN_CLR_BYTES);
  a.stat = a.part + (size_t)N * p.NCH * G * 2;
  a.S = S; a.SC = p.SC; a.NCH = p.NCH;
  a.sample_bytes = (uint32_t)(S * C * es);
  a.C = (uint32_t)C; a.G = (uint32_t)G; a.cpg = (uint32_t)cpg;
  a.eps = eps; a.pdt = param_dtype;
  switch (dtype) {
    case ATK_F32: return launch_gn_cl<float>(a, (int)N, fuse_silu, s);
    case ATK_F16: return launch_gn_cl<_Float16>(a, (int)N, fuse_silu, s);
    default: return launch_gn_cl<__bf16>(a, (int)N, fuse_silu, s);
  }
}

extern "C" size_t atk_group_norm_cl_bwd_workspace_bytes(int64_t N, int64_t C, int64_t S, int G) {
  if (N <= 0 || C <= 0 || S <= 0 || G <= 0) return 0;
  // the register-resident kernel's header, slots and results (fixed layout), then either the
  // three-kernel path's records / dx coefficients / dpar or the resident kernel's per-workgroup
  // rows (chunks as small as fp32 makes them)
  const atk::GnClPlan p = atk::plan_gn_cl_bwd(N, S);
  const size_t three = (size_t)N * (size_t)C * ((size_t)p.NCH * 16 + 16 + 8);
  const int64_t sc32 = std::max<int64_t>(1, 16 * (512 / std::max<int64_t>(1, C / 4)));
  const size_t rows = (size_t)N * (size_t)((S + sc32 - 1) / sc32) * (size_t)C * 8;
  return atk::GN_CLR_BYTES + std::max(three, rows);
}

extern "C" int atk_group_norm_cl_bwd(const void* x, const void* dy, const void* gamma, void* dx, float* dgamma,
                                     float* dbeta, int64_t N, int64_t C, int64_t S, int G, float eps, int dtype,
                                     int param_dtype, void* workspace, size_t ws_bytes, atk_stream_t stream) {
  using namespace atk;
  if (!dtype_ok(dtype) || (gamma && !dtype_ok(param_dtype)))
    return fail(ATK_EINVAL, "group_norm backward (channels-last): unknown dtype code");
  if (N <= 0 || C <= 0 || S <= 0 || G <= 0) return fail(ATK_EINVAL, "group_norm backward (channels-last): bad sizes");
  if (C % G)
    return fail(ATK_EINVAL, "group_norm backward (channels-last): channels (%lld) not divisible by groups (%d)",
                (long long)C, G);
  if (!x || !dy) return fail(ATK_EINVAL, "group_norm backward (channels-last): null pointer");
  const int64_t es = (int64_t)dtype_size(dtype), vec = 16 / es;
  const int64_t cpg = C / G;
  if (cpg % vec || C > GN_CL_MAXC || GN_CL_NT % (C / vec) || !aligned16(x) || !aligned16(dy) || (dx && !aligned16(dx)))
    return fail(ATK_UNSUPPORTED, "group_norm backward (channels-last): needs C/G %% %lld == 0, C/%lld dividing %d "
                "and 16-byte aligned tensors", (long long)vec, (long long)vec, GN_CL_NT);
  if (N >= 65536) return fail(ATK_UNSUPPORTED, "group_norm backward (channels-last): batch too large");
  if (S * C * es >= ((int64_t)1 << 31))
    return fail(ATK_UNSUPPORTED, "group_norm backward (channels-last): one sample over 2 GiB (32-bit buffer offsets)");
  const size_t need = atk_group_norm_cl_bwd_workspace_bytes(N, C, S, G);
  if (!workspace || ws_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 15u))
    return fail(ATK_EINVAL, "group_norm backward (channels-last): workspace of %zu bytes (16-byte aligned) needed",
                need);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Register-resident single pass where the rule takes it (plan_gn_cl_bwd_res);
  // ATK_GN_CL_RESIDENT=0 turns it off, =8 / =16 takes it wherever it fits.
  const char* renv = getenv("ATK_GN_CL_RESIDENT");
  const int rmode = renv ? atoi(renv) : 1;
  if (rmode != 0) {
    const bool force = rmode == 8 || rmode == 16;
    GnClBwdResPlan rp;
    const bool fits = dtype == ATK_F32   ? plan_gn_cl_bwd_res<float>(N, C, S, G, force, rp)
                      : dtype == ATK_F16 ? plan_gn_cl_bwd_res<_Float16>(N, C, S, G, force, rp)
                                         : plan_gn_cl_bwd_res<__bf16>(N, C, S, G, force, rp);
    if (fits && GN_CLR_BYTES + (size_t)N * rp.NCH * (size_t)C * 8 <= ws_bytes) {
      GnClBwdResArgs r;
      r.x = x; r.dy = dy; r.gamma = gamma; r.dx = dx; r.dgamma = dgamma; r.dbeta = dbeta;
      char* ws = static_cast<char*>(workspace);
      r.hdr = reinterpret_cast<uint32_t*>(ws);
      r.slots = reinterpret_cast<GnSlot*>(ws + GN_CLR_SLOTS_OFF);
      r.finals = reinterpret_cast<GnSlot*>(ws + GN_CLR_FINALS_OFF);
      r.rows = reinterpret_cast<float2*>(ws + GN_CLR_BYTES);
      r.S = S; r.SC = rp.SC; r.NCH = rp.NCH;
      r.C = (int)C; r.G = G; r.cpg = (int)cpg; r.N = (int)N;
      r.two_level = rp.two_level;
      r.pdt = param_dtype;
      r.eps = eps;
      const int khz = device_wall_clock_khz();
      const char* wenv = getenv("ATK_GN_WAIT_US");
      const uint64_t wait_us = wenv ? strtoull(wenv, nullptr, 10) : GN_WAIT_US;
      r.wait_ticks = (uint64_t)(khz > 0 ? khz : 100000) * wait_us / 1000;
      switch (dtype) {
        case ATK_F32: return launch_gn_cl_bwd_res<float>(r, N, s);
        case ATK_F16: return launch_gn_cl_bwd_res<_Float16>(r, N, s);
        default: return launch_gn_cl_bwd_res<__bf16>(r, N, s);
      }
    }
  }
  const GnClPlan p = plan_gn_cl_bwd(N, S);
  GnClBwdArgs a;
  a.x = x; a.dy = dy; a.gamma = gamma; a.dx = dx; a.dgamma = dgamma; a.dbeta = dbeta;
  a.part = reinterpret_cast<float4*>(static_cast<char*>(workspace) + GN_CLR_BYTES);
  a.coef = a.part + (size_t)N * p.NCH * C;
  a.dpar = reinterpret_cast<float2*>(a.coef + (size_t)N * C);
  a.S = S; a.SC = p.SC; a.NCH = p.NCH; a.N = (int)N;
  a.sample_bytes = (uint32_t)(S * C * es);
  a.C = (uint32_t)C; a.G = (uint32_t)G; a.cpg = (uint32_t)cpg;
  a.eps = eps; a.pdt = param_dtype;
  switch (dtype) {
    case ATK_F32: return launch_gn_cl_bwd<float>(a, s);
    case ATK_F16: return launch_gn_cl_bwd<_Float16>(a, s);
    default: return launch_gn_cl_bwd<__bf16>(a, s);
  }
}

extern "C" int atk_group_norm_fwd_args(const atk_group_norm_args* a) {
  if (!a) return atk::fail(ATK_EINVAL, "group_norm: null argument block");
  return atk_group_norm_fwd(a->x, a->gamma, a->beta, a->y, a->N, a->C, a->S, a->G, a->eps, a->fuse_silu, a->dtype,
                            a->param_dtype, a->variant, a->workspace, a->workspace_bytes, a->stream);
}
