/*
 * atk_oracle.c -- CPU restatement (float64) of the hot-path operators, used ONLY as the
 * checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in
 * the product links or calls it.
 *
 * The parity target of the reference is stock torch.nn.functional (its selector verifies
 * every candidate against stock, amd_tuned_torch/kernel_select.py:68-82,615-651); these are
 * the textbook definitions of those stock operators, written as loops with float64
 * accumulation, in the form each reference kernel states them.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

/* Depthwise conv1d, BCL (amd_tuned_torch/_vendor/flashfftconv_depthwise_conv1d/
 * conv1d_bhl.hip:55-100; causal variant src/causal-conv1d-amd/csrc/causal_conv1d_fwd.cu:
 * 39-130 == pad_left = K-1 and the first L outputs):
 *   y[n,c,t] = b[c] + sum_j w[c,j] * x[n,c,t-pad_left+j],  t in [0, L_out), x = 0 outside [0, L).
 * silu != 0 applies y / (1 + exp(-y)) (causal_conv1d_fwd.cu silu_activation). */
void oracle_dwconv1d(const double* x, const double* w, const double* b, double* y, int64_t N,
                     int64_t C, int64_t L, int64_t K, int64_t pad_left, int64_t L_out, int silu) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c) {
      const double* xr = x + (n * C + c) * L;
      double* yr = y + (n * C + c) * L_out;
      for (int64_t t = 0; t < L_out; ++t) {
        double acc = b ? b[c] : 0.0;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t p = t - pad_left + j;
          if (p >= 0 && p < L) acc += w[c * K + j] * xr[p];
        }
        yr[t] = silu ? acc / (1.0 + exp(-acc)) : acc;
      }
    }
}

/* Gradients of oracle_dwconv1d (no SiLU) for an upstream gradient dy [N, C, L_out], in
 * the form of the reference's depthwise backward (amd_tuned_torch/_vendor/
 * flashfftconv_depthwise_conv1d/conv1d_bwd_hip_bhl.hip:39-57 correlates dout with the
 * reversed kernel for du; :62-116 builds dk and sums dk . dout over the batch for
 * dweight and dout over batch and length for dbias; the causal form is
 * src/causal-conv1d-amd/csrc/causal_conv1d_bwd.cu:100-235):
 *   dx[n,c,s] = sum_j w[c,j] * dy[n,c,s+pad_left-j]     (dy = 0 outside [0, L_out))
 *   dw[c,j]   = sum_{n,t} dy[n,c,t] * x[n,c,t-pad_left+j] (x = 0 outside [0, L))
 *   db[c]     = sum_{n,t} dy[n,c,t]
 * Any of dx / dw / db may be NULL. */
void oracle_dwconv1d_bwd(const double* x, const double* w, const double* dy, double* dx, double* dw,
                         double* db, int64_t N, int64_t C, int64_t L, int64_t K, int64_t pad_left,
                         int64_t L_out) {
  if (dw)
    for (int64_t i = 0; i < C * K; ++i) dw[i] = 0.0;
  if (db)
    for (int64_t c = 0; c < C; ++c) db[c] = 0.0;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t c = 0; c < C; ++c) {
      const double* xr = x + (n * C + c) * L;
      const double* gr = dy + (n * C + c) * L_out;
      if (dx) {
        double* dr = dx + (n * C + c) * L;
        for (int64_t s = 0; s < L; ++s) {
          double acc = 0.0;
          for (int64_t j = 0; j < K; ++j) {
            const int64_t t = s + pad_left - j;
            if (t >= 0 && t < L_out) acc += w[c * K + j] * gr[t];
          }
          dr[s] = acc;
        }
      }
      for (int64_t t = 0; t < L_out; ++t) {
        if (db) db[c] += gr[t];
        if (dw)
          for (int64_t j = 0; j < K; ++j) {
            const int64_t p = t - pad_left + j;
            if (p >= 0 && p < L) dw[c * K + j] += gr[t] * xr[p];
          }
      }
    }
}

/* Decode step of the causal conv (src/causal-conv1d-amd/csrc/causal_conv1d_update.cu:27-66;
 * causal_conv1d_interface.py:192-213): state [B, D, W] <- (state[..., 1:], x[b, d]),
 * y[b, d] = b[d] + sum_j w[d, j] * state[b, d, j]; silu != 0 applies y / (1 + exp(-y)).
 * The state is updated in place. */
void oracle_causal_conv1d_update(const double* x, double* state, const double* w, const double* b, double* y,
                                 int64_t B, int64_t D, int64_t W, int silu) {
  for (int64_t i = 0; i < B * D; ++i) {
    const int64_t d = i % D;
    double* st = state + i * W;
    for (int64_t j = 0; j + 1 < W; ++j) st[j] = st[j + 1];
    st[W - 1] = x[i];
    double acc = b ? b[d] : 0.0;
    for (int64_t j = 0; j < W; ++j) acc += w[d * W + j] * st[j];
    y[i] = silu ? acc / (1.0 + exp(-acc)) : acc;
  }
}

/* GroupNorm over NC[S] (src/cuda/group_norm.cu:41-104; fused SiLU of
 * amd_tuned_torch/conv_fusion_ops.py:192-242): group (n, g) = channels [g*C/G, (g+1)*C/G)
 * x all S positions; population variance (divide by the group size), eps inside the
 * square root, optional per-channel affine.  Statistics by two passes in float64.
 * mean_out / rstd_out ([N*G], may be NULL) receive the group statistics. */
void oracle_group_norm(const double* x, const double* gamma, const double* beta, double* y,
                       int64_t N, int64_t C, int64_t S, int64_t G, double eps, int silu,
                       double* mean_out, double* rstd_out) {
  const int64_t cpg = C / G, E = cpg * S;
  for (int64_t gi = 0; gi < N * G; ++gi) {
    const double* xg = x + gi * E;
    double* yg = y + gi * E;
    double s = 0.0;
    for (int64_t e = 0; e < E; ++e) s += xg[e];
    const double mean = s / (double)E;
    double m2 = 0.0;
    for (int64_t e = 0; e < E; ++e) {
      const double d = xg[e] - mean;
      m2 += d * d;
    }
    const double rstd = 1.0 / sqrt(m2 / (double)E + eps);
    if (mean_out) mean_out[gi] = mean;
    if (rstd_out) rstd_out[gi] = rstd;
    const int64_t g = gi % G;
    for (int64_t cl = 0; cl < cpg; ++cl) {
      const int64_t c = g * cpg + cl;
      const double gm = gamma ? gamma[c] : 1.0, bt = beta ? beta[c] : 0.0;
      for (int64_t sp = 0; sp < S; ++sp) {
        const int64_t e = cl * S + sp;
        double v = (xg[e] - mean) * rstd * gm + bt;
        if (silu) v = v / (1.0 + exp(-v));
        yg[e] = v;
      }
    }
  }
}

/* Gradients of oracle_group_norm (no SiLU) for an upstream gradient dy, in the form of the
 * reference's backward (amd_tuned_torch/_dispatch.py:2212-2302, torch ops over an (N, G,
 * M, S) view):  x_hat = (x - mu) * rstd,  g = gamma_c * dy,
 *   dx = rstd * (g - mean_group(g) - x_hat * mean_group(g * x_hat)),
 *   dgamma_c = sum_{n,s} dy * x_hat,  dbeta_c = sum_{n,s} dy.
 * gamma may be NULL (ones); any output may be NULL.  Statistics by two passes. */
void oracle_group_norm_bwd(const double* x, const double* gamma, const double* dy, double* dx,
                           double* dgamma, double* dbeta, int64_t N, int64_t C, int64_t S, int64_t G,
                           double eps) {
  const int64_t cpg = C / G, E = cpg * S;
  if (dgamma)
    for (int64_t c = 0; c < C; ++c) dgamma[c] = 0.0;
  if (dbeta)
    for (int64_t c = 0; c < C; ++c) dbeta[c] = 0.0;
  for (int64_t gi = 0; gi < N * G; ++gi) {
    const double* xg = x + gi * E;
    const double* dg = dy + gi * E;
    const int64_t c0 = (gi % G) * cpg;
    double s = 0.0;
    for (int64_t e = 0; e < E; ++e) s += xg[e];
    const double mu = s / (double)E;
    double q = 0.0;
    for (int64_t e = 0; e < E; ++e) q += (xg[e] - mu) * (xg[e] - mu);
    const double rstd = 1.0 / sqrt(q / (double)E + eps);
    double m1 = 0.0, m2 = 0.0;
    for (int64_t e = 0; e < E; ++e) {
      const double gam = gamma ? gamma[c0 + e / S] : 1.0;
      const double gg = gam * dg[e];
      m1 += gg;
      m2 += gg * (xg[e] - mu) * rstd;
    }
    m1 /= (double)E;
    m2 /= (double)E;
    for (int64_t e = 0; e < E; ++e) {
      const int64_t c = c0 + e / S;
      const double xh = (xg[e] - mu) * rstd;
      const double gam = gamma ? gamma[c] : 1.0;
      if (dx) dx[gi * E + e] = rstd * (gam * dg[e] - m1 - xh * m2);
      if (dgamma) dgamma[c] += dg[e] * xh;
      if (dbeta) dbeta[c] += dg[e];
    }
  }
}

/* Dense conv3d, groups = 1, NCDHW (the implicit GEMM of src/cuda/generated/
 * conv3d_fp16_bm256_bn128_bk32_s2.cu:84-324 and the direct kernel of src/cuda/conv3d_fp32.cu:
 * 33-149 both compute this):
 *   y[n,o,z,h,v] = b[o] + sum_{i,a,bb,c} w[o,i,a,bb,c] * x[n,i,z*sd-pd+a*dd, h*sh-ph+bb*dh, v*sw-pw+c*dw]
 * Output extents follow src/main_rocm.cpp:204-206.  Computes only the `npts` output
 * elements whose flat NCDHW indices are listed in `pts` (all of them when pts == NULL, in
 * which case npts must equal the output size), so large problems can be spot-checked. */
static int64_t out_extent(int64_t in, int64_t k, int64_t s, int64_t p, int64_t d) {
  return (in + 2 * p - d * (k - 1) - 1) / s + 1;
}

void oracle_conv3d(const double* x, const double* w, const double* b, double* y, int64_t N,
                   int64_t Ci, int64_t D, int64_t H, int64_t W, int64_t Co, int64_t KD,
                   int64_t KH, int64_t KW, int64_t sd, int64_t sh, int64_t sw, int64_t pd,
                   int64_t ph, int64_t pw, int64_t dd, int64_t dh, int64_t dw, const int64_t* pts,
                   int64_t npts) {
  (void)N; /* batch index comes from the flat output index */
  const int64_t Do = out_extent(D, KD, sd, pd, dd), Ho = out_extent(H, KH, sh, ph, dh),
                Wo = out_extent(W, KW, sw, pw, dw);
  const int64_t osp = Do * Ho * Wo, isp = D * H * W, taps = KD * KH * KW;
  for (int64_t q = 0; q < npts; ++q) {
    const int64_t f = pts ? pts[q] : q;
    const int64_t n = f / (Co * osp);
    int64_t r = f - n * Co * osp;
    const int64_t o = r / osp;
    r -= o * osp;
    const int64_t z = r / (Ho * Wo);
    r -= z * Ho * Wo;
    const int64_t h = r / Wo;
    const int64_t v = r - h * Wo;
    double acc = b ? b[o] : 0.0;
    for (int64_t i = 0; i < Ci; ++i) {
      const double* xc = x + (n * Ci + i) * isp;
      const double* wc = w + (o * Ci + i) * taps;
      for (int64_t a = 0; a < KD; ++a) {
        const int64_t iz = z * sd - pd + a * dd;
        if (iz < 0 || iz >= D) continue;
        for (int64_t bb = 0; bb < KH; ++bb) {
          const int64_t iy = h * sh - ph + bb * dh;
          if (iy < 0 || iy >= H) continue;
          for (int64_t c = 0; c < KW; ++c) {
            const int64_t ix = v * sw - pw + c * dw;
            if (ix < 0 || ix >= W) continue;
            acc += wc[(a * KH + bb) * KW + c] * xc[(iz * H + iy) * W + ix];
          }
        }
      }
    }
    y[q] = acc;
  }
}

/* Causal depthwise conv with seq_idx and initial / final states: the reference's channel-last
 * kernel (src/causal-conv1d-amd/csrc/causal_conv1d_fwd.cu:194-332) restated on plain arrays,
 * x [B, D, L], w [D, K], b [D] or NULL, seq [B, L] int32 or NULL, init [B, D, K-1] or NULL,
 * y [B, D, L], fin [B, D, K-1] or NULL.  With H = K-1:
 *   xv(p)  = x[p] for p >= 0, init[p + H] for p < 0 (0 without init);
 *   sq(p)  = seq[p] for p >= 0, -1 for p < 0 (fwd.cu:293-299);
 *   y[t]   = act(b + sum_j [sq(t-H+j) == sq(t)] * w[j] * xv(t-H+j))      (fwd.cu:302-315);
 *   fin[j] = xv(L - H + j)                                                (fwd.cu:259-266). */
static double xv_at(const double* xr, const double* ir, int64_t p, int64_t H) {
  if (p >= 0) return xr[p];
  return ir ? ir[p + H] : 0.0;
}

void oracle_causal_conv1d_states(const double* x, const double* w, const double* b, const int* seq,
                                 const double* init, double* y, double* fin, int64_t B, int64_t D,
                                 int64_t L, int64_t K, int silu) {
  const int64_t H = K - 1;
  for (int64_t n = 0; n < B; ++n)
    for (int64_t c = 0; c < D; ++c) {
      const double* xr = x + (n * D + c) * L;
      const double* ir = init ? init + (n * D + c) * H : 0;
      const int* sr = seq ? seq + n * L : 0;
      for (int64_t t = 0; t < L; ++t) {
        double acc = b ? b[c] : 0.0;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t p = t - H + j;
          if (sr && (p >= 0 ? sr[p] : -1) != sr[t]) continue;
          acc += w[c * K + j] * xv_at(xr, ir, p, H);
        }
        y[(n * D + c) * L + t] = silu ? acc / (1.0 + exp(-acc)) : acc;
      }
      if (fin)
        for (int64_t j = 0; j < H; ++j) fin[(n * D + c) * H + j] = xv_at(xr, ir, L - H + j, H);
    }
}

/* Gradients of oracle_causal_conv1d_states for dout [B, D, L] and dfinal [B, D, K-1] (or NULL),
 * the reference's causal_conv1d_bwd (causal_conv1d.cpp:240-380): with z the pre-activation and
 * g[t] = dout[t] * silu'(z[t]) (dout[t] without the activation), every term
 * w[j] * xv(p), p = t-H+j, kept by the mask adds g[t] * w[j] to dxv(p), g[t] * xv(p) to dw[j]
 * and g[t] to db; dfinal[j] adds to dxv(L - H + j).  dxv(p) is dx[p] for p >= 0 and
 * dinit[p + H] for p < 0.  Any of dx / dw / db / dinit may be NULL. */
void oracle_causal_conv1d_states_bwd(const double* x, const double* w, const double* b, const int* seq,
                                     const double* init, const double* dout, const double* dfinal,
                                     double* dx, double* dw, double* db, double* dinit, int64_t B,
                                     int64_t D, int64_t L, int64_t K, int silu) {
  const int64_t H = K - 1;
  if (dw) for (int64_t i = 0; i < D * K; ++i) dw[i] = 0.0;
  if (db) for (int64_t c = 0; c < D; ++c) db[c] = 0.0;
  if (dx) for (int64_t i = 0; i < B * D * L; ++i) dx[i] = 0.0;
  if (dinit) for (int64_t i = 0; i < B * D * H; ++i) dinit[i] = 0.0;
  for (int64_t n = 0; n < B; ++n)
    for (int64_t c = 0; c < D; ++c) {
      const double* xr = x + (n * D + c) * L;
      const double* ir = init ? init + (n * D + c) * H : 0;
      const int* sr = seq ? seq + n * L : 0;
      double* dxr = dx ? dx + (n * D + c) * L : 0;
      double* dir = dinit ? dinit + (n * D + c) * H : 0;
      for (int64_t t = 0; t < L; ++t) {
        double g = dout[(n * D + c) * L + t];
        if (silu) {
          double z = b ? b[c] : 0.0;
          for (int64_t j = 0; j < K; ++j) {
            const int64_t p = t - H + j;
            if (sr && (p >= 0 ? sr[p] : -1) != sr[t]) continue;
            z += w[c * K + j] * xv_at(xr, ir, p, H);
          }
          const double s = 1.0 / (1.0 + exp(-z));
          g *= s * (1.0 + z * (1.0 - s));
        }
        if (db) db[c] += g;
        for (int64_t j = 0; j < K; ++j) {
          const int64_t p = t - H + j;
          if (sr && (p >= 0 ? sr[p] : -1) != sr[t]) continue;
          if (dw) dw[c * K + j] += g * xv_at(xr, ir, p, H);
          if (p >= 0) { if (dxr) dxr[p] += g * w[c * K + j]; }
          else if (dir) dir[p + H] += g * w[c * K + j];
        }
      }
      if (dfinal)
        for (int64_t j = 0; j < H; ++j) {
          const int64_t p = L - H + j;
          const double v = dfinal[(n * D + c) * H + j];
          if (p >= 0) { if (dxr) dxr[p] += v; }
          else if (dir) dir[p + H] += v;
        }
    }
}
