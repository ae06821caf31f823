/*
 * CPU fp64 oracle for the fused SDPA / LayerNorm / RMSNorm path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * Every function restates, in double precision, the closed-form arithmetic of
 * the reference op it stands for (citations are to /root/reference):
 *
 *   oracle_layer_norm   src/jax_mlx/layer_norm.py:20-25   (population variance,
 *                       (x-mu)/sqrt(var+eps)*w+b); matcher form
 *                       src/jax_mlx_pjrt.cpp:2337-2339; custom_call
 *                       src/jax_mlx_pjrt.cpp:8207-8236.
 *   oracle_rms_norm     src/jax_mlx_pjrt.cpp:2166-2169 (x*rsqrt(mean(x^2)+eps),
 *                       optional weight), executed at :4422-4429.
 *   oracle_softmax      src/jax_mlx_pjrt.cpp:1857-2044 (exp(x-max)/sum).
 *   oracle_log_softmax  src/jax_mlx_pjrt.cpp:5624-5641 ((x-max) - log(sum(exp(x-max)))).
 *   oracle_sdpa         src/jax_mlx/sdpa.py:19-31 and src/jax_mlx_pjrt.cpp:
 *                       2491-2495 (softmax(scale*QK^T + M) V) in BHTD layout;
 *                       M is 0, causal (key j allowed iff j <= query i, top-left
 *                       aligned like jax.nn.dot_product_attention) or an
 *                       additive tensor broadcast through element strides.
 *                       GQA maps query head h to kv head h / (Hq/Hkv).
 *   oracle_layer_norm_bwd  src/jax_mlx/layer_norm.py:59-76.
 *   oracle_sdpa_bwd        src/jax_mlx/sdpa.py:65-87 (extended to masks/GQA:
 *                       dK/dV of a kv head sum over its query heads).
 *
 * Pins (tests/test_oracle.py): torch fp64 library routines through the
 * committed fixtures in tests/golden/, closed forms (constant rows, Tk=1,
 * identical keys, single allowed key), invariants (permutation of keys,
 * GQA == MHA with repeated K/V, convex hull), finite differences for the
 * backward functions.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

ORACLE_API int oracle_version(void) { return 1; }

/* y[r, :] = (x - mean) / sqrt(var + eps) * gamma + beta, var = mean((x-mean)^2). */
ORACLE_API void oracle_layer_norm(const double* x, const double* gamma,
                                  const double* beta, int64_t rows, int64_t n,
                                  double eps, double* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * n;
    double* yr = y + r * n;
    double mean = 0.0;
    for (int64_t i = 0; i < n; ++i) mean += xr[i];
    mean /= (double)n;
    double var = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      double d = xr[i] - mean;
      var += d * d;
    }
    var /= (double)n;
    double inv = 1.0 / sqrt(var + eps);
    for (int64_t i = 0; i < n; ++i) {
      double v = (xr[i] - mean) * inv;
      if (gamma) v *= gamma[i];
      if (beta) v += beta[i];
      yr[i] = v;
    }
  }
}

/* y[r, :] = x * (1/sqrt(mean(x^2) + eps)) * weight. */
ORACLE_API void oracle_rms_norm(const double* x, const double* weight,
                                int64_t rows, int64_t n, double eps, double* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * n;
    double* yr = y + r * n;
    double ms = 0.0;
    for (int64_t i = 0; i < n; ++i) ms += xr[i] * xr[i];
    ms /= (double)n;
    double inv = 1.0 / sqrt(ms + eps);
    for (int64_t i = 0; i < n; ++i) {
      double v = xr[i] * inv;
      if (weight) v *= weight[i];
      yr[i] = v;
    }
  }
}

/* Row log-softmax: shifted = x - max(x), y = shifted - log(sum(exp(shifted))).
 * An all -inf row yields NaN, as the shifted difference does. */
ORACLE_API void oracle_log_softmax(const double* x, int64_t rows, int64_t n,
                                   double* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * n;
    double* yr = y + r * n;
    double m = -INFINITY;
    for (int64_t i = 0; i < n; ++i) m = xr[i] > m ? xr[i] : m;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += exp(xr[i] - m);
    const double ls = log(s);
    for (int64_t i = 0; i < n; ++i) yr[i] = (xr[i] - m) - ls;
  }
}

/* Row softmax; an all -inf row yields NaN, as exp(x - max(x)) does in JAX. */
ORACLE_API void oracle_softmax(const double* x, int64_t rows, int64_t n,
                               double* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * n;
    double* yr = y + r * n;
    double m = -INFINITY;
    for (int64_t i = 0; i < n; ++i) m = xr[i] > m ? xr[i] : m;
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      yr[i] = exp(xr[i] - m);
      s += yr[i];
    }
    for (int64_t i = 0; i < n; ++i) yr[i] /= s;
  }
}

/* Scores row for (b, h, i): s[j] = scale * <q_i, k_j> + mask, -inf if causal
 * and j > i.  Returns the row's probabilities in p (length Tk). */
static void sdpa_row_probs(const double* q, const double* k, const double* mask,
                           const int64_t* ms, int64_t b, int64_t h, int64_t hk,
                           int64_t i, int64_t Hq, int64_t Hkv, int64_t Tq,
                           int64_t Tk, int64_t D, double scale, int causal,
                           double* p) {
  const double* qi = q + (((b * Hq) + h) * Tq + i) * D;
  double m = -INFINITY;
  for (int64_t j = 0; j < Tk; ++j) {
    const double* kj = k + (((b * Hkv) + hk) * Tk + j) * D;
    double s = 0.0;
    for (int64_t d = 0; d < D; ++d) s += qi[d] * kj[d];
    s *= scale;
    if (mask) s += mask[b * ms[0] + h * ms[1] + i * ms[2] + j * ms[3]];
    if (causal && j > i) s = -INFINITY;
    p[j] = s;
    if (s > m) m = s;
  }
  double l = 0.0;
  for (int64_t j = 0; j < Tk; ++j) {
    p[j] = exp(p[j] - m);
    l += p[j];
  }
  for (int64_t j = 0; j < Tk; ++j) p[j] /= l;
}

/*
 * out[b,h,i,:] = sum_j softmax_j(scale*q.k_j + M)[j] * v[b,h/(Hq/Hkv),j,:].
 * q [B,Hq,Tq,D], k [B,Hkv,Tk,D], v [B,Hkv,Tk,Dv], out [B,Hq,Tq,Dv], all
 * contiguous.  mask (nullable) is read at b*ms[0]+h*ms[1]+i*ms[2]+j*ms[3].
 * Returns 0, or -1 on an invalid head ratio.
 */
ORACLE_API int oracle_sdpa(const double* q, const double* k, const double* v,
                           const double* mask, const int64_t* mask_strides,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq,
                           int64_t Tk, int64_t D, int64_t Dv, double scale,
                           int causal, double* out) {
  if (Hkv <= 0 || Hq % Hkv != 0) return -1;
  int64_t group = Hq / Hkv;
  double* p = (double*)malloc(sizeof(double) * (size_t)(Tk > 0 ? Tk : 1));
  if (!p) return -2;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      int64_t hk = h / group;
      for (int64_t i = 0; i < Tq; ++i) {
        sdpa_row_probs(q, k, mask, mask_strides, b, h, hk, i, Hq, Hkv, Tq, Tk,
                       D, scale, causal, p);
        double* o = out + (((b * Hq) + h) * Tq + i) * Dv;
        for (int64_t d = 0; d < Dv; ++d) o[d] = 0.0;
        for (int64_t j = 0; j < Tk; ++j) {
          const double* vj = v + (((b * Hkv) + hk) * Tk + j) * Dv;
          for (int64_t d = 0; d < Dv; ++d) o[d] += p[j] * vj[d];
        }
      }
    }
  free(p);
  return 0;
}

/*
 * LayerNorm backward over the last axis (src/jax_mlx/layer_norm.py:59-76):
 *   xhat = (x-mu)/std, dxhat = g*w,
 *   dx = (dxhat - mean(dxhat) - xhat*mean(dxhat*xhat)) / std,
 *   dw = sum_rows(g*xhat), db = sum_rows(g).
 */
ORACLE_API void oracle_layer_norm_bwd(const double* x, const double* w,
                                      const double* g, int64_t rows, int64_t n,
                                      double eps, double* dx, double* dw,
                                      double* db) {
  for (int64_t i = 0; i < n; ++i) {
    dw[i] = 0.0;
    db[i] = 0.0;
  }
  for (int64_t r = 0; r < rows; ++r) {
    const double* xr = x + r * n;
    const double* gr = g + r * n;
    double mean = 0.0;
    for (int64_t i = 0; i < n; ++i) mean += xr[i];
    mean /= (double)n;
    double var = 0.0;
    for (int64_t i = 0; i < n; ++i) var += (xr[i] - mean) * (xr[i] - mean);
    var /= (double)n;
    double inv = 1.0 / sqrt(var + eps);
    double m1 = 0.0, m2 = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      double xh = (xr[i] - mean) * inv;
      double dxh = gr[i] * (w ? w[i] : 1.0);
      m1 += dxh;
      m2 += dxh * xh;
      dw[i] += gr[i] * xh;
      db[i] += gr[i];
    }
    m1 /= (double)n;
    m2 /= (double)n;
    for (int64_t i = 0; i < n; ++i) {
      double xh = (xr[i] - mean) * inv;
      double dxh = gr[i] * (w ? w[i] : 1.0);
      dx[r * n + i] = inv * (dxh - m1 - xh * m2);
    }
  }
}

/*
 * SDPA backward (src/jax_mlx/sdpa.py:65-87), BHTD layout as oracle_sdpa:
 *   dV = P^T dO, dP = dO V^T, dS = P*(dP - rowsum(dP*P)) * scale,
 *   dQ = dS K, dK = dS^T Q; kv-head gradients sum over their query heads.
 */
ORACLE_API int oracle_sdpa_bwd(const double* q, const double* k, const double* v,
                               const double* dout, const double* mask,
                               const int64_t* mask_strides, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t Tq, int64_t Tk,
                               int64_t D, int64_t Dv, double scale, int causal,
                               double* dq, double* dk, double* dv) {
  if (Hkv <= 0 || Hq % Hkv != 0) return -1;
  int64_t group = Hq / Hkv;
  size_t nk = (size_t)(Tk > 0 ? Tk : 1);
  double* p = (double*)malloc(sizeof(double) * nk);
  double* dp = (double*)malloc(sizeof(double) * nk);
  if (!p || !dp) {
    free(p);
    free(dp);
    return -2;
  }
  memset(dq, 0, sizeof(double) * (size_t)(B * Hq * Tq * D));
  memset(dk, 0, sizeof(double) * (size_t)(B * Hkv * Tk * D));
  memset(dv, 0, sizeof(double) * (size_t)(B * Hkv * Tk * Dv));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      int64_t hk = h / group;
      for (int64_t i = 0; i < Tq; ++i) {
        sdpa_row_probs(q, k, mask, mask_strides, b, h, hk, i, Hq, Hkv, Tq, Tk,
                       D, scale, causal, p);
        const double* go = dout + (((b * Hq) + h) * Tq + i) * Dv;
        const double* qi = q + (((b * Hq) + h) * Tq + i) * D;
        double* dqi = dq + (((b * Hq) + h) * Tq + i) * D;
        double rs = 0.0;
        for (int64_t j = 0; j < Tk; ++j) {
          const double* vj = v + (((b * Hkv) + hk) * Tk + j) * Dv;
          double s = 0.0;
          for (int64_t d = 0; d < Dv; ++d) s += go[d] * vj[d];
          dp[j] = s;
          rs += s * p[j];
          double* dvj = dv + (((b * Hkv) + hk) * Tk + j) * Dv;
          for (int64_t d = 0; d < Dv; ++d) dvj[d] += p[j] * go[d];
        }
        for (int64_t j = 0; j < Tk; ++j) {
          double ds = p[j] * (dp[j] - rs) * scale;
          if (ds == 0.0) continue;
          const double* kj = k + (((b * Hkv) + hk) * Tk + j) * D;
          double* dkj = dk + (((b * Hkv) + hk) * Tk + j) * D;
          for (int64_t d = 0; d < D; ++d) {
            dqi[d] += ds * kj[d];
            dkj[d] += ds * qi[d];
          }
        }
      }
    }
  free(p);
  free(dp);
  return 0;
}
