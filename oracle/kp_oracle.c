/*
 * kp_oracle.c -- CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker; the product path (kernelproblems_amd/) never calls it.
 *
 * Scalar C, one thread, no vector intrinsics, built with -ffp-contract=off.
 * Reductions are accumulated in double; the bf16 rounding points are the
 * ones the reference's torch ops have:
 *   - eager bf16 add.Tensor: fp32 add of the two widened operands, one
 *     round-to-nearest-even to bf16 (bf16_add below);
 *   - _fused_rms_norm: fp32 upcast, rstd = rsqrt(mean(x^2) + eps) kept as an
 *     fp32 tensor, out = x * rstd * w cast to bf16 once
 *     (torch/_decomp/decompositions.py:1760-1812);
 *   - _fused_rms_norm_backward: grad_x_hat = dy * w, x_hat = x * rstd,
 *     dx = (grad_x_hat - x_hat / N * sum(x_hat * grad_x_hat)) * rstd,
 *     dw = sum_rows dy * x_hat (decompositions.py:1815-1887);
 *   - embedding_dense_backward: grad rows of equal index summed in the
 *     computation dtype, padding_idx rows masked, optional division by the
 *     index count (decompositions.py:1245-1275);
 *   - RoPE: complex multiply (a + ib)(c + id) of the interleaved pairs
 *     (v8/c8c60d8f7015/problem.py:18-71) or rotate-half pairs with
 *     inv_freq_i = theta^(-2i/D) rounded to fp32 and angle = fp32(p * inv_freq_i).
 * Values computed in double and then rounded once to bf16 are the exactly
 * rounded results of the fp32 formulas given their fp32 inputs (rstd, cos/sin,
 * table entries), i.e. the limit the GPU's fp32 arithmetic approximates.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KPO_ROPE_HALF 0
#define KPO_ROPE_INTERLEAVED 1

/* ---------------------------------------------------------------- bf16 */
static float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16, round to nearest even; NaN stays a quiet NaN. */
static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* double -> bf16 with a single round-to-nearest-even: the double is first
 * narrowed to fp32 with round-to-odd (truncate, set the sticky bit if
 * inexact), which keeps the following fp32 -> bf16 rounding exact. */
static uint16_t d2bf(double d) {
  if (isnan(d)) return 0x7fc0u;
  float f = (float)d;
  if ((double)f != d && !isinf(f)) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (fabs((double)f) > fabs(d)) u -= 1u; /* step back toward zero */
    u |= 1u;
    memcpy(&f, &u, 4);
  } else if (isinf(f) && !isinf(d)) {
    uint32_t u = (d > 0 ? 0x7f7fffffu : 0xff7fffffu);
    memcpy(&f, &u, 4);
  }
  return f2bf(f);
}

/* eager bf16 + bf16 -> bf16 */
static float bf16_add(float a, float b) {
  volatile float s = a + b; /* fp32 add (no excess precision on x86-64 SSE) */
  return bf2f(f2bf(s));
}

static float term_sum(const uint16_t* const* t, const int64_t* st, int n, int64_t row, int64_t c) {
  float v = bf2f(t[0][row * st[0] + c]);
  for (int i = 1; i < n; ++i) v = bf16_add(v, bf2f(t[i][row * st[i] + c]));
  return v;
}

static double weight_at(const uint16_t* w, int64_t seg_len, int64_t seg_stride, int64_t c) {
  if (!w) return 1.0;
  return (double)bf2f(w[(c / seg_len) * seg_stride + c % seg_len]);
}

void kpo_bf16_from_f32(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = f2bf(src[i]);
}
void kpo_bf16_from_f64(const double* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = d2bf(src[i]);
}
void kpo_bf16_add(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f2bf(bf16_add(bf2f(a[i]), bf2f(b[i])));
}

static float rstd_of(double sumsq, int64_t N, float eps) {
  return (float)(1.0 / sqrt(sumsq / (double)N + (double)eps));
}

/* ------------------------------------------------------------ RMSNorm fwd */
int kpo_rmsnorm_fwd(const uint16_t* const* x, const int64_t* xs, int nx, const uint16_t* w, int64_t seg_len,
                    int64_t seg_stride, uint16_t* h, uint16_t* y, float* rstd, int64_t M, int64_t N, float eps) {
  if (nx < 1 || nx > 3 || N <= 0 || M < 0) return 1;
  float* row = (float*)malloc((size_t)N * sizeof(float));
  if (!row) return 2;
  for (int64_t r = 0; r < M; ++r) {
    double ss = 0.0;
    for (int64_t c = 0; c < N; ++c) {
      row[c] = term_sum(x, xs, nx, r, c);
      ss += (double)row[c] * (double)row[c];
    }
    const float rs = rstd_of(ss, N, eps);
    for (int64_t c = 0; c < N; ++c) {
      if (h) h[r * N + c] = f2bf(row[c]);
      y[r * N + c] = d2bf((double)row[c] * (double)rs * weight_at(w, seg_len, seg_stride, c));
    }
    if (rstd) rstd[r] = rs;
  }
  free(row);
  return 0;
}

/* ------------------------------------------------------------ RMSNorm bwd */
int kpo_rmsnorm_bwd(const uint16_t* const* dy, const int64_t* dys, int ndy, const uint16_t* const* x,
                    const int64_t* xs, int nx, const float* rstd_in, const uint16_t* w, int64_t seg_len,
                    int64_t seg_stride, const uint16_t* dxr, uint16_t* dx, double* dw, float* rstd_out,
                    int64_t M, int64_t N, float eps) {
  if (nx < 1 || nx > 3 || ndy < 1 || ndy > 3 || N <= 0 || M < 0) return 1;
  double* xr = (double*)malloc((size_t)N * sizeof(double));
  double* dr = (double*)malloc((size_t)N * sizeof(double));
  if (!xr || !dr) {
    free(xr);
    free(dr);
    return 2;
  }
  if (dw)
    for (int64_t c = 0; c < N; ++c) dw[c] = 0.0;
  for (int64_t r = 0; r < M; ++r) {
    double ss = 0.0;
    for (int64_t c = 0; c < N; ++c) {
      xr[c] = term_sum(x, xs, nx, r, c);
      dr[c] = term_sum(dy, dys, ndy, r, c);
      ss += xr[c] * xr[c];
    }
    const float rs = rstd_in ? rstd_in[r] : rstd_of(ss, N, eps);
    if (rstd_out) rstd_out[r] = rs;
    double s = 0.0;
    for (int64_t c = 0; c < N; ++c) s += (xr[c] * rs) * (dr[c] * weight_at(w, seg_len, seg_stride, c));
    for (int64_t c = 0; c < N; ++c) {
      const double xh = xr[c] * rs;
      const double g = dr[c] * weight_at(w, seg_len, seg_stride, c);
      const double d = (g - xh / (double)N * s) * rs;
      uint16_t o = d2bf(d);
      if (dxr) o = f2bf(bf16_add(bf2f(dxr[r * N + c]), bf2f(o)));
      dx[r * N + c] = o;
      if (dw) dw[c] += dr[c] * xh;
    }
  }
  free(xr);
  free(dr);
  return 0;
}

/* ------------------------------------------------------------ embedding */
/* Returns the number of out-of-range indices (their rows are zero-filled). */
int64_t kpo_embedding_fwd(const uint16_t* table, int64_t V, int64_t D, int64_t trs, const int64_t* idx, int64_t T,
                          uint16_t* out) {
  int64_t bad = 0;
  for (int64_t t = 0; t < T; ++t) {
    const int64_t id = idx[t];
    if (id < 0 || id >= V) {
      ++bad;
      memset(out + t * D, 0, (size_t)D * 2);
      continue;
    }
    memcpy(out + t * D, table + id * trs, (size_t)D * 2);
  }
  return bad;
}

typedef struct {
  int64_t id, t;
} kpo_pair;

static int cmp_pair(const void* a, const void* b) {
  const kpo_pair* x = (const kpo_pair*)a;
  const kpo_pair* y = (const kpo_pair*)b;
  if (x->id != y->id) return x->id < y->id ? -1 : 1;
  return (x->t > y->t) - (x->t < y->t);
}

/* Touched rows of the dense embedding gradient.  Writes, for each distinct
 * contributing id in ascending order, ids[k], the fp64 row sum rows[k*D + c]
 * and the fp64 sum of absolute contributions absrows[k*D + c] (for error
 * bounds); *n_rows receives the count.  Untouched rows are zero.  Returns the
 * number of out-of-range indices (skipped). */
int64_t kpo_embedding_bwd_rows(const uint16_t* grad, int64_t grs, const int64_t* idx, int64_t T, int64_t V,
                               int64_t D, int64_t padding_idx, int scale, int64_t* ids, double* rows,
                               double* absrows, int64_t* counts, int64_t* n_rows) {
  kpo_pair* p = (kpo_pair*)malloc((size_t)(T > 0 ? T : 1) * sizeof(kpo_pair));
  if (!p) return -1;
  int64_t n = 0, bad = 0;
  for (int64_t t = 0; t < T; ++t) {
    const int64_t id = idx[t];
    if (id < 0 || id >= V) {
      ++bad;
      continue;
    }
    if (id == padding_idx) continue;
    p[n].id = id;
    p[n].t = t;
    ++n;
  }
  qsort(p, (size_t)n, sizeof(kpo_pair), cmp_pair);
  int64_t k = -1;
  for (int64_t i = 0; i < n;) {
    int64_t j = i;
    while (j < n && p[j].id == p[i].id) ++j;
    ++k;
    ids[k] = p[i].id;
    if (counts) counts[k] = j - i;
    double* r = rows + k * D;
    double* ar = absrows ? absrows + k * D : NULL;
    for (int64_t c = 0; c < D; ++c) {
      r[c] = 0.0;
      if (ar) ar[c] = 0.0;
    }
    for (int64_t q = i; q < j; ++q) {
      const uint16_t* g = grad + p[q].t * grs;
      for (int64_t c = 0; c < D; ++c) {
        double v = (double)bf2f(g[c]);
        if (scale) v = (double)((float)v / (float)(j - i)); /* fp32 division, as grad / count */
        r[c] += v;
        if (ar) ar[c] += fabs(v);
      }
    }
    i = j;
  }
  *n_rows = k + 1;
  free(p);
  return bad;
}

/* Dense fp32 gradient [V, D]: touched rows are the fp64 sums rounded to fp32
 * (to bf16 and widened when round_bf16), all other rows zero. */
int64_t kpo_embedding_bwd_dense(const uint16_t* grad, int64_t grs, const int64_t* idx, int64_t T, int64_t V,
                                int64_t D, int64_t padding_idx, int scale, int round_bf16, float* out) {
  int64_t* ids = (int64_t*)malloc((size_t)(T > 0 ? T : 1) * sizeof(int64_t));
  double* rows = (double*)malloc((size_t)(T > 0 ? T : 1) * (size_t)D * sizeof(double));
  if (!ids || !rows) {
    free(ids);
    free(rows);
    return -1;
  }
  int64_t nr = 0;
  const int64_t bad = kpo_embedding_bwd_rows(grad, grs, idx, T, V, D, padding_idx, scale, ids, rows, NULL, NULL, &nr);
  memset(out, 0, (size_t)V * (size_t)D * sizeof(float));
  for (int64_t k = 0; k < nr; ++k)
    for (int64_t c = 0; c < D; ++c) {
      const double v = rows[k * D + c];
      out[ids[k] * D + c] = round_bf16 ? bf2f(d2bf(v)) : (float)v;
    }
  free(ids);
  free(rows);
  return bad;
}

/* ------------------------------------------------------------ RoPE */
/* x, out: bf16 [B, S, H, D] with element strides xs/os = {b, s, h} (D unit).
 * pos: NULL (p = s) or int64 at pos[b * psb + s * pss].
 * freqs: NULL (theta mode) or float pairs [frows, D/2] with row stride frs
 * complex elements.  Returns the number of (b, s) positions outside the
 * table (their output is zero). */
int64_t kpo_rope(const uint16_t* x, const int64_t* xs, uint16_t* out, const int64_t* os, int64_t B, int64_t S,
                 int64_t H, int64_t D, const int64_t* pos, int64_t psb, int64_t pss, int pairing, double theta,
                 const float* freqs, int64_t frows, int64_t frs, int conj) {
  const int64_t half = D / 2;
  float* inv = (float*)malloc((size_t)(half > 0 ? half : 1) * sizeof(float));
  double* cv = (double*)malloc((size_t)(half > 0 ? half : 1) * sizeof(double));
  double* sv = (double*)malloc((size_t)(half > 0 ? half : 1) * sizeof(double));
  if (!inv || !cv || !sv) {
    free(inv);
    free(cv);
    free(sv);
    return -1;
  }
  for (int64_t i = 0; i < half; ++i) inv[i] = (float)pow(theta, -(double)(2 * i) / (double)D);
  int64_t bad = 0;
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t s = 0; s < S; ++s) {
      const int64_t p = pos ? pos[b * psb + s * pss] : s;
      int ok = 1;
      for (int64_t i = 0; i < half; ++i) {
        if (freqs) {
          if (p < 0 || p >= frows) {
            ok = 0;
            cv[i] = sv[i] = 0.0;
            continue;
          }
          cv[i] = (double)freqs[2 * (p * frs + i)];
          sv[i] = (double)freqs[2 * (p * frs + i) + 1];
        } else {
          volatile float a = (float)p * inv[i]; /* fp32 angle */
          cv[i] = cos((double)a);
          sv[i] = sin((double)a);
        }
        if (conj) sv[i] = -sv[i];
      }
      if (!ok) ++bad;
      for (int64_t h = 0; h < H; ++h) {
        const uint16_t* xp = x + b * xs[0] + s * xs[1] + h * xs[2];
        uint16_t* op = out + b * os[0] + s * os[1] + h * os[2];
        for (int64_t i = 0; i < half; ++i) {
          const int64_t ia = pairing == KPO_ROPE_HALF ? i : 2 * i;
          const int64_t ib = pairing == KPO_ROPE_HALF ? i + half : 2 * i + 1;
          const double xa = bf2f(xp[ia]), xb = bf2f(xp[ib]);
          if (!ok) {
            op[ia] = op[ib] = 0;
            continue;
          }
          op[ia] = d2bf(xa * cv[i] - xb * sv[i]);
          op[ib] = d2bf(xb * cv[i] + xa * sv[i]);
        }
      }
    }
  }
  free(inv);
  free(cv);
  free(sv);
  return bad;
}

/* ---------------------------------------------------------------- SwiGLU
 * Forward (v8/c68dae22972b/problem.py:15-28): silu.default of the w1 output
 * a, materialised as bf16, then mul.Tensor with the w3 output b:
 *   out = bf16(bf16(silu(a)) * b),  silu(x) = x / (1 + e^-x).
 * Backward (v8/385e1beb9bb9/problem.py:17-33): db = mul.Tensor(g, s);
 * t = mul.Tensor(g, b); da = silu_backward(t, a) =
 *   t * sig * (1 + a * (1 - sig)),  sig = 1 / (1 + e^-a)
 * (the derivative of x * sig(x); aten silu_backward as decomposed at
 * torch/_decomp/decompositions.py:297-302).
 * silu and silu_backward are evaluated in double and rounded once to bf16,
 * the exactly rounded value of the fp32 formula's limit.  bf16 x bf16
 * products are exact in double, so db, t and the final multiply of the
 * forward carry exactly one rounding, as in fp32.  Contiguous arrays. */
static double silu_d(double x) { return x / (1.0 + exp(-x)); }

static double silu_bwd_d(double t, double x) {
  const double sig = 1.0 / (1.0 + exp(-x));
  return t * sig * (1.0 + x * (1.0 - sig));
}

void kpo_swiglu_fwd(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double s = (double)bf2f(d2bf(silu_d((double)bf2f(a[i]))));
    out[i] = d2bf(s * (double)bf2f(b[i]));
  }
}

void kpo_swiglu_bwd(const uint16_t* g, const uint16_t* s, const uint16_t* b, const uint16_t* a, uint16_t* db,
                    uint16_t* da, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const double gv = (double)bf2f(g[i]);
    db[i] = d2bf(gv * (double)bf2f(s[i]));
    const double t = (double)bf2f(d2bf(gv * (double)bf2f(b[i])));
    da[i] = d2bf(silu_bwd_d(t, (double)bf2f(a[i])));
  }
}

/* ---------------------------------------------------------------- cross-entropy
 * Forward (v8/71f1d2c9f38b/problem.py:15-40): _to_copy(f32) of the bf16
 * logits, _log_softmax over the vocabulary, nll_loss_forward with weight
 * None, reduction sum and ignore_index, div by a constant:
 *   lse_i = m_i + log(sum_j exp(x_ij - m_i)),  m_i = max_j x_ij
 *   loss  = scale * sum_{i: t_i != ignore} (lse_i - x_{i, t_i}),  total_weight = #{i: t_i != ignore}
 * (log_softmax(x)_ij = x_ij - lse_i, torch/_decomp/decompositions.py:1198-1221
 * (_log_softmax); nll picks -lsm[i, t_i] and counts the non-ignored rows,
 * :4099-4150 (_nll_loss_forward)), all in double.  Targets outside [0, V)
 * other than ignore_index are counted in the return value and treated as
 * ignored.
 * Backward (v8/622c35f5d1c6/problem.py:16-33): nll_loss_backward puts -g at
 * (i, t_i) of valid rows (decompositions.py:485-514, _nll_loss_backward);
 * _log_softmax_backward_data gives
 *   out_ij = grad_ij - exp(L_ij) * sum_j grad_ij
 * (decompositions.py:879-889), rounded once to bf16 from double. */
int64_t kpo_cross_entropy_fwd(const uint16_t* logits, int64_t M, int64_t V, const int64_t* targets, int64_t ignore,
                              double scale, double* loss, double* total_weight, double* lse_out) {
  double acc = 0.0, cnt = 0.0;
  int64_t bad = 0;
  for (int64_t i = 0; i < M; ++i) {
    const uint16_t* x = logits + i * V;
    double m = -INFINITY;
    for (int64_t j = 0; j < V; ++j) {
      const double v = (double)bf2f(x[j]);
      if (v > m || isnan(v)) m = v;
    }
    double lse;
    if (isinf(m) || isnan(m)) {
      lse = m; /* all -inf: -inf; any +inf or NaN: propagates */
      if (m > 0) lse = NAN;
    } else {
      double s = 0.0;
      for (int64_t j = 0; j < V; ++j) s += exp((double)bf2f(x[j]) - m);
      lse = m + log(s);
    }
    if (lse_out) lse_out[i] = lse;
    const int64_t t = targets[i];
    if (t == ignore) continue;
    if (t < 0 || t >= V) {
      ++bad;
      continue;
    }
    acc += lse - (double)bf2f(x[t]);
    cnt += 1.0;
  }
  *loss = acc * scale;
  *total_weight = cnt;
  return bad;
}

int64_t kpo_cross_entropy_bwd(const float* lsm, int64_t M, int64_t V, const int64_t* targets, int64_t ignore, double g,
                              uint16_t* out) {
  int64_t bad = 0;
  for (int64_t i = 0; i < M; ++i) {
    const int64_t t = targets[i];
    const int in_range = t >= 0 && t < V;
    if (t != ignore && !in_range) ++bad;
    const int valid = t != ignore && in_range;
    const double sum = valid ? -g : 0.0;
    for (int64_t j = 0; j < V; ++j) {
      const double grad = (valid && j == t) ? -g : 0.0;
      out[i * V + j] = d2bf(grad - exp((double)lsm[i * V + j]) * sum);
    }
  }
  return bad;
}

/* Forward and backward from the logits in one region
 * (v5/fb5b36393cbd/problem.py:16-59): the backward above applied to
 * L_ij = x_ij - lse_i, with lse_i computed as in kpo_cross_entropy_fwd, all in
 * double, one rounding to bf16:
 *   out_ij = grad_ij - exp(x_ij - lse_i) * sum_j grad_ij. */
int64_t kpo_cross_entropy_fwd_bwd(const uint16_t* logits, int64_t M, int64_t V, const int64_t* targets, int64_t ignore,
                                  double g, uint16_t* out) {
  int64_t bad = 0;
  for (int64_t i = 0; i < M; ++i) {
    const uint16_t* x = logits + i * V;
    double m = -INFINITY;
    for (int64_t j = 0; j < V; ++j) {
      const double v = (double)bf2f(x[j]);
      if (v > m || isnan(v)) m = v;
    }
    double s = 0.0;
    for (int64_t j = 0; j < V; ++j) s += exp((double)bf2f(x[j]) - m);
    const double lse = m + log(s);
    const int64_t t = targets[i];
    const int in_range = t >= 0 && t < V;
    if (t != ignore && !in_range) ++bad;
    const int valid = t != ignore && in_range;
    const double sum = valid ? -g : 0.0;
    for (int64_t j = 0; j < V; ++j) {
      const double grad = (valid && j == t) ? -g : 0.0;
      out[i * V + j] = d2bf(grad - exp((double)bf2f(x[j]) - lse) * sum);
    }
  }
  return bad;
}
