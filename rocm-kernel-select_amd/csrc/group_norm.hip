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
//            mean), and, when NS > 1, exchanges (mean, M2) with the other slices of its
//            group through a per-group generation barrier in the workspace.  All
//            workgroups must be co-resident, so NS > 1 launches cooperatively (the
//            runtime refuses the launch rather than oversubscribe) and the barrier spin
//            is bounded.  HBM traffic: one read + one write of the tensor.
//   twopass  Streaming fallback for any size / alignment: a statistics kernel writes
//            per-slice (mean, M2) partials, an apply kernel merges them and normalises.
#include "atk_common.h"

namespace atk {

namespace {

constexpr uint32_t GN_SPIN_LIMIT = 1u << 20;  // polls (s_sleep(2) apart): never reached when co-resident
constexpr int GN_MAX_NS = 4096;
// Workspace layout is FIXED so that calls of different shapes sharing one workspace can
// never write partials over another shape's barrier counters:
//   [0, 256)                      error flag
//   [256, 256 + 8*GN_MAX_COOP)    (arrivals, generation) per group, cooperative variants
//   [GN_PARTIALS_OFF, ...)        per-slice (mean, M2) partials
constexpr int GN_MAX_COOP = 4096;             // groups a cooperative launch may span
constexpr size_t GN_ZERO_BYTES = 256 + 8 * (size_t)GN_MAX_COOP;
constexpr size_t GN_PARTIALS_OFF = GN_ZERO_BYTES;
constexpr int GN_TP_NT = 256;                 // two-pass kernels
constexpr int GN_MAX_AFF = 512;               // channels per slice whose affine is staged in LDS

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
  uint32_t* err;      // workspace: error flag
  uint32_t* counters; // workspace: [ngroups][2] (arrivals, generation)
  float* partials;    // workspace: [ngroups][NS][2] (mean, M2)
};

__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-group barrier among NS workgroups; called by one thread per workgroup, after that
// thread stored its partial.  Generation counting leaves `cnt` at zero on exit, so the
// workspace needs zeroing only once.
__device__ void group_barrier(uint32_t* cnt, uint32_t* gen, int NS, uint32_t* err) {
  const uint32_t g0 = __hip_atomic_load(gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  if (arrived == (uint32_t)NS - 1) {
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    uint32_t it = 0;
    while (__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g0) {
      __builtin_amdgcn_s_sleep(2);
      if (++it > GN_SPIN_LIMIT) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
}

__device__ __forceinline__ int64_t slice_len(int i, int64_t slice, int64_t E) {
  return (int64_t)(i + 1) * slice <= E ? slice : E - (int64_t)i * slice;
}

// Merge the NS (mean, M2) partials of one group, in a fixed order so that every
// workgroup of the group derives bit-identical statistics.
__device__ __forceinline__ void merge_partials(const float* p, int NS, int64_t slice, int64_t E,
                                               float& mean, float& var) {
  float sm = 0.f;
  for (int i = 0; i < NS; ++i) sm += (float)slice_len(i, slice, E) * load_agent(p + 2 * i);
  mean = sm / (float)E;
  float m2 = 0.f;
  for (int i = 0; i < NS; ++i) {
    const float d = load_agent(p + 2 * i) - mean;
    m2 += load_agent(p + 2 * i + 1) + (float)slice_len(i, slice, E) * d * d;
  }
  var = m2 / (float)E;
}

// scale/shift of absolute channel `c` given the group statistics
__device__ __forceinline__ void channel_affine(const GnArgs& a, int64_t c, float mean, float rstd,
                                               float& sc, float& sh) {
  const float gm = a.gamma ? load_param(a.gamma, a.pdt, c) : 1.f;
  const float bt = a.beta ? load_param(a.beta, a.pdt, c) : 0.f;
  sc = rstd * gm;
  sh = bt - mean * sc;
}

template <typename T>
__device__ __forceinline__ uint4 normalize_vec(const Vec16<T>& in, float sc, float sh, int silu) {
  constexpr int VEC = 16 / sizeof(T);
  Vec16<T> o;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    float v = fmaf(to_f32(in.e[k]), sc, sh);
    if (silu) v = silu_f32(v);
    o.e[k] = from_f32<T>(v);
  }
  return o.raw;
}

// ---------------------------------------------------------------------------------------
// Register-resident single pass.  Requires S % VEC == 0 and 16B-aligned x / y (host check).
// ---------------------------------------------------------------------------------------
template <typename T, int NT, int EPV>
__global__ __launch_bounds__(NT) void gn_resident_kernel(GnArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float red[NT / 64];
  __shared__ float s_stat[2];
  __shared__ float aff[2 * GN_MAX_AFF];  // scale[ ], shift[ ] of the slice's channels

  const int tid = threadIdx.x;
  const int64_t gi = blockIdx.x / a.NS;
  const int s = (int)(blockIdx.x - gi * a.NS);
  const int64_t E = a.E;
  const int64_t s0 = (int64_t)s * a.slice;
  const T* __restrict__ xg = static_cast<const T*>(a.x) + gi * E;
  T* __restrict__ yg = static_cast<T*>(a.y) + gi * E;

  Vec16<T> buf[EPV];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const int64_t e = s0 + ((int64_t)i * NT + tid) * VEC;
    if (e < E) buf[i].raw = ld16<true>(xg + e);
    else buf[i].raw = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int k = 0; k < VEC; ++k) sum += to_f32(buf[i].e[k]);  // padding lanes hold +0
  }
  const int64_t n_l = (E - s0) < a.slice ? (E - s0) : a.slice;
  sum = block_sum<NT>(sum, red);
  const float mean_l = sum / (float)n_l;
  float m2 = 0.f;
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const int64_t e = s0 + ((int64_t)i * NT + tid) * VEC;
    if (e < E) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        const float d = to_f32(buf[i].e[k]) - mean_l;
        m2 = fmaf(d, d, m2);
      }
    }
  }
  m2 = block_sum<NT>(m2, red);

  float mean, var;
  if (a.NS == 1) {
    mean = mean_l;
    var = m2 / (float)n_l;
  } else {
    float* part = a.partials + gi * (int64_t)a.NS * 2;
    if (tid == 0) {
      __hip_atomic_store(part + 2 * s, mean_l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(part + 2 * s + 1, m2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      group_barrier(a.counters + 2 * gi, a.counters + 2 * gi + 1, a.NS, a.err);
      merge_partials(part, a.NS, a.slice, E, mean, var);
      s_stat[0] = mean;
      s_stat[1] = var;
    }
    __syncthreads();
    mean = s_stat[0];
    var = s_stat[1];
  }
  const float rstd = 1.0f / sqrtf(var + a.eps);

  // scale/shift of the channels this slice spans (group-local channel range [c_lo, c_hi))
  const int64_t last = (s0 + a.slice < E ? s0 + a.slice : E) - 1;
  const uint32_t c_lo = fdiv((uint32_t)s0, a.div_s);
  const uint32_t c_hi = fdiv((uint32_t)last, a.div_s) + 1;
  const int nch = (int)(c_hi - c_lo);
  const int64_t cabs0 = (int64_t)(gi % a.G) * a.cpg + c_lo;  // absolute channel of c_lo
  const bool staged = nch <= GN_MAX_AFF;
  if (staged) {
    for (int i = tid; i < nch; i += NT) {
      float sc, sh;
      channel_affine(a, cabs0 + i, mean, rstd, sc, sh);
      aff[i] = sc;
      aff[GN_MAX_AFF + i] = sh;
    }
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const int64_t e = s0 + ((int64_t)i * NT + tid) * VEC;
    if (e < E) {
      const int cl = (int)(fdiv((uint32_t)e, a.div_s) - c_lo);
      float sc, sh;
      if (staged) {
        sc = aff[cl];
        sh = aff[GN_MAX_AFF + cl];
      } else {
        channel_affine(a, cabs0 + cl, mean, rstd, sc, sh);
      }
      st16<true>(yg + e, normalize_vec<T>(buf[i], sc, sh, a.silu));
    }
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

template <typename T, bool VECOK>
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
  if (tid == 0) {
    float mean, var;
    merge_partials(a.partials + gi * (int64_t)a.NS * 2, a.NS, a.slice, E, mean, var);
    s_stat[0] = mean;
    s_stat[1] = 1.0f / sqrtf(var + a.eps);
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
      st16<true>(yg + e, normalize_vec<T>(b, sc, sh, a.silu));
    } else {
      float v = fmaf(to_f32(xg[e]), sc, sh);
      if (a.silu) v = silu_f32(v);
      yg[e] = from_f32<T>(v);
    }
  }
}

struct GnVariant {
  const char* name;
  int nt, epv;  // epv == 0: two-pass
};

const GnVariant kGnVariants[] = {
    {"res_nt1024_v8", 1024, 8},
    {"res_nt1024_v16", 1024, 16},
    {"res_nt1024_v4", 1024, 4},
    {"res_nt512_v8", 512, 8},
    {"res_nt256_v8", 256, 8},
    {"res_nt256_v16", 256, 16},
    {"twopass", GN_TP_NT, 0},
};
constexpr int kNumGn = sizeof(kGnVariants) / sizeof(kGnVariants[0]);

struct GnPlan {
  int NS;
  int64_t slice;
  size_t ws_bytes, zero_bytes;
  bool vec_ok;
};

inline size_t round256(size_t v) { return (v + 255) & ~(size_t)255; }

// Slicing and workspace size (layout: see GN_ZERO_BYTES / GN_PARTIALS_OFF)
bool plan_gn(int64_t N, int64_t C, int64_t S, int G, int dtype, int variant, GnPlan& p) {
  const int64_t cpg = C / G;
  const int64_t E = cpg * S;
  const int64_t ngroups = N * G;
  const int vec = (int)(16 / dtype_size(dtype));
  const GnVariant& v = kGnVariants[variant];
  if (v.epv > 0) {
    p.slice = (int64_t)v.nt * v.epv * vec;
    p.NS = (int)((E + p.slice - 1) / p.slice);
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
  p.ws_bytes = GN_PARTIALS_OFF + round256((size_t)ngroups * p.NS * 8);
  return true;
}

template <typename T, int NT, int EPV>
int launch_resident(GnArgs a, int64_t ngroups, hipStream_t s) {
  const int64_t nblk = ngroups * a.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm: grid too large");
  auto kern = gn_resident_kernel<T, NT, EPV>;
  if (a.NS == 1) {
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(NT), 0, s, a);
    return check_launch("gn_resident_kernel");
  }
  if (ngroups > GN_MAX_COOP)
    return fail(ATK_UNSUPPORTED, "group_norm: %lld groups exceed the cooperative barrier table",
                (long long)ngroups);
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern), NT, 0) != hipSuccess)
    return fail(ATK_ELAUNCH, "group_norm: occupancy query failed");
  const int64_t cap = (int64_t)per_cu * device_cu_count();
  if (nblk > cap)
    return fail(ATK_UNSUPPORTED, "group_norm: %lld workgroups cannot be co-resident (max %lld)",
                (long long)nblk, (long long)cap);
  void* args[] = {&a};
  hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3((unsigned)nblk),
                                            dim3(NT), args, 0, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (e == hipErrorCooperativeLaunchTooLarge)
      return fail(ATK_UNSUPPORTED, "group_norm: cooperative launch too large");
    return fail(ATK_ELAUNCH, "group_norm: cooperative launch: %s", hipGetErrorString(e));
  }
  return ATK_OK;
}

template <typename T>
int launch_gn(GnArgs a, int64_t ngroups, int variant, bool vec_ok, hipStream_t s) {
  const GnVariant& v = kGnVariants[variant];
  if (v.epv > 0) {
    if (!vec_ok) return fail(ATK_UNSUPPORTED, "group_norm: %s needs S %% 16B == 0 and aligned pointers", v.name);
    switch (variant) {
      case 0: return launch_resident<T, 1024, 8>(a, ngroups, s);
      case 1: return launch_resident<T, 1024, 16>(a, ngroups, s);
      case 2: return launch_resident<T, 1024, 4>(a, ngroups, s);
      case 3: return launch_resident<T, 512, 8>(a, ngroups, s);
      case 4: return launch_resident<T, 256, 8>(a, ngroups, s);
      case 5: return launch_resident<T, 256, 16>(a, ngroups, s);
      default: return fail(ATK_EINVAL, "group_norm: bad variant");
    }
  }
  const int64_t nblk = ngroups * a.NS;
  if (nblk > 0x7fffffff) return fail(ATK_UNSUPPORTED, "group_norm: grid too large");
  if (vec_ok) {
    hipLaunchKernelGGL((gn_stats_kernel<T, true>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
    int rc = check_launch("gn_stats_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL((gn_apply_kernel<T, true>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
    return check_launch("gn_apply_kernel");
  }
  hipLaunchKernelGGL((gn_stats_kernel<T, false>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
  int rc = check_launch("gn_stats_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((gn_apply_kernel<T, false>), dim3((unsigned)nblk), dim3(GN_TP_NT), 0, s, a);
  return check_launch("gn_apply_kernel");
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

extern "C" int atk_group_norm_fwd(const void* x, const void* gamma, const void* beta, void* y,
                                  int64_t N, int64_t C, int64_t S, int G, float eps, int fuse_silu,
                                  int dtype, int param_dtype, int variant, void* workspace,
                                  size_t workspace_bytes, atk_stream_t stream) {
  using namespace atk;
  if (variant < 0) variant = 0;
  int rc = validate_gn(N, C, S, G, dtype, variant);
  if (rc) return rc;
  if ((gamma || beta) && !dtype_ok(param_dtype))
    return fail(ATK_EINVAL, "group_norm: unknown param dtype code %d", param_dtype);
  if (N == 0) return ATK_OK;
  if (!x || !y) return fail(ATK_EINVAL, "group_norm: null pointer");
  GnPlan p;
  if (!plan_gn(N, C, S, G, dtype, variant, p))
    return fail(ATK_UNSUPPORTED, "group_norm: too many slices per group for %s", kGnVariants[variant].name);
  if (!workspace || workspace_bytes < p.ws_bytes)
    return fail(ATK_EINVAL, "group_norm: workspace of %zu bytes needed", p.ws_bytes);
  const size_t es = dtype_size(dtype);
  const int vec = (int)(16 / es);
  const bool vec_ok = (S % vec == 0) && aligned16(x) && aligned16(y);
  GnArgs a;
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
  a.err = reinterpret_cast<uint32_t*>(ws);
  a.counters = reinterpret_cast<uint32_t*>(ws + 256);
  a.partials = reinterpret_cast<float*>(ws + GN_PARTIALS_OFF);
  const int64_t ngroups = N * G;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case ATK_F32: return launch_gn<float>(a, ngroups, variant, vec_ok, s);
    case ATK_F16: return launch_gn<_Float16>(a, ngroups, variant, vec_ok, s);
    default: return launch_gn<__bf16>(a, ngroups, variant, vec_ok, s);
  }
}
