/*
 * fmxq_oracle.c -- CPU restatement of the quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see fmxq_oracle.h): imported by tests/, by
 * __graft_entry__.smoke() and by the cpu_baseline leg of bench.py, never by the
 * product library.
 *
 * The arithmetic lives in MLX/mlx-c, which the reference binds but does not
 * vendor (mlxgo/binding_cgo.go:19-23 links -lmlxc -lmlx; no third_party/ and
 * no version pin in go.mod:1-3).  The semantics restated here are the ones the
 * reference's call sites and stub documentation fix:
 *   - packing: 32/bits values per uint32, LSB first; [out, in*bits/32] words
 *     (compute/models/switch_glu_test.go:123-163, "8 int4 values per uint32")
 *   - dequantize: w = scale * q + bias per group along the input axis
 *     (mlxgo/binding_stub.go:312-318, compute/models/quant.go:117-142)
 *   - quantized_matmul with transpose=true: y = x . deq(W)^T
 *     (compute/models/quant.go:91-101, mlxgo/binding_cgo.go:636-643)
 *   - gather_qmm: per-row expert selection by rhs indices
 *     (compute/models/switch_glu.go:179-186, mlxgo/binding_cgo.go:645-673)
 *   - SwitchGLU: silu(gate) * up then down, silu = x * sigmoid(x)
 *     (compute/models/switch_glu.go:107-153, qwen3_forward.go:229-239)
 * Build with -ffp-contract=off so every a*b+c below rounds the way it reads.
 */
#include "fmxq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round to nearest, ties to even; NaN stays a quiet NaN. */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float r16(float f) { return oracle_bf16_to_f32(oracle_f32_to_bf16(f)); }

uint32_t oracle_unpack(const uint32_t *row_words, int64_t k, int bits) {
  const int per = 32 / bits;
  const uint32_t word = row_words[k / per];
  return (word >> ((k % per) * bits)) & ((1u << bits) - 1u);
}

static int supported(int group_size, int bits, int64_t K) {
  if (bits != 4 && bits != 8) return 0;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
  if (K <= 0 || K % group_size != 0) return 0;
  return 1;
}

/* One dequantized element as fp32 (exactly a bf16 value). */
static inline float deq_elem(uint32_t q, uint16_t s16, uint16_t b16, int mode) {
  const float s = oracle_bf16_to_f32(s16), b = oracle_bf16_to_f32(b16);
  if (mode == ORACLE_DEQ_MLX) {
    /* multiply(q, scales) -> bf16, then add(., biases) -> bf16 */
    return r16(r16((float)q * s) + b);
  }
  if (mode == ORACLE_DEQ_EXACT) return (float)q * s + b; /* q*s exact in fp32 */
  return r16((float)q * s + b);
}

static void deq_row(const uint32_t *wrow, const uint16_t *srow,
                    const uint16_t *brow, float *out, int64_t K, int group_size,
                    int bits, int mode) {
  for (int64_t k = 0; k < K; ++k) {
    const int64_t g = k / group_size;
    out[k] = deq_elem(oracle_unpack(wrow, k, bits), srow[g], brow[g], mode);
  }
}

int oracle_dequantize(const uint32_t *w, const uint16_t *scales,
                      const uint16_t *biases, uint16_t *out, int64_t rows,
                      int64_t K, int group_size, int bits, int mode) {
  if (!supported(group_size, bits, K) || rows < 0) return -1;
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < K; ++k) {
      const int64_t g = k / group_size;
      out[r * K + k] = oracle_f32_to_bf16(
          deq_elem(oracle_unpack(w + r * wpr, k, bits), scales[r * gpr + g],
                   biases[r * gpr + g], mode));
    }
  }
  return 0;
}

/* MLX affine quantization, the requantize step of absorbKVB
 * (compute/models/deepseekv3.go:662-669 through mlxgo.Quantize ->
 * mlx_quantize, mlxgo/binding_cgo.go:684-697; inverse of Dequantize per
 * binding_stub.go:320-326).  MLX is not vendored, so the per-group steps are
 * MLX's published affine algorithm, in fp32:
 *   delta = max((max - min) / (2^bits - 1), 1e-7)
 *   the end of larger magnitude is the edge: min with scale +delta, else max
 *   with scale -delta (so q = 0 sits at the edge and q grows inward)
 *   q0 = rint(edge / scale); if q0 != 0: scale = edge / q0, bias = edge
 *   (the edge is hit exactly and zero lands on the grid point -q0), else bias 0
 *   q = clamp(rint((w - bias) / scale), 0, 2^bits - 1)
 * scales and biases are stored as bf16 (the input's dtype), rounded to
 * nearest-even.  rint is round-half-to-even (MLX's round op). */
static void quantize_group(const uint16_t *src, int group_size, int bits, uint32_t *qout,
                           uint16_t *s_out, uint16_t *b_out) {
  const float n_bins = (float)((1 << bits) - 1);
  float mn = oracle_bf16_to_f32(src[0]), mx = mn;
  for (int i = 1; i < group_size; ++i) {
    const float v = oracle_bf16_to_f32(src[i]);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  float delta = (mx - mn) / n_bins;
  if (!(delta > 1e-7f)) delta = 1e-7f;
  const int side = fabsf(mn) > fabsf(mx);
  float scale = side ? delta : -delta;
  const float edge = side ? mn : mx;
  const float q0 = rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  for (int i = 0; i < group_size; ++i) {
    float q = rintf((oracle_bf16_to_f32(src[i]) - bias) / scale);
    q = q < 0.0f ? 0.0f : q > n_bins ? n_bins : q;
    qout[i] = (uint32_t)q;
  }
  *s_out = oracle_f32_to_bf16(scale);
  *b_out = oracle_f32_to_bf16(bias);
}

int oracle_quantize(const uint16_t *w, uint32_t *wq, uint16_t *scales, uint16_t *biases,
                    int64_t rows, int64_t K, int group_size, int bits) {
  if (!supported(group_size, bits, K) || rows < 0) return -1;
  const int per = 32 / bits;
  const int64_t wpr = K / per, gpr = K / group_size;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t q[128];
    for (int64_t g = 0; g < gpr; ++g) {
      quantize_group(w + r * K + g * group_size, group_size, bits, q, scales + r * gpr + g,
                     biases + r * gpr + g);
      for (int i = 0; i < group_size; i += per) {
        uint32_t word = 0;
        for (int j = 0; j < per; ++j) word |= q[i + j] << (j * bits);
        wq[r * wpr + (g * group_size + i) / per] = word;
      }
    }
  }
  return 0;
}

int oracle_qmm_f32(const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                   const uint16_t *biases, uint16_t *y, float *y_f32,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits,
                   int mode) {
  if (!supported(group_size, bits, K) || M < 0 || N < 0) return -1;
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
#pragma omp parallel
  {
    float *wf = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      deq_row(w + n * wpr, scales + n * gpr, biases + n * gpr, wf, K,
              group_size, bits, mode);
      for (int64_t m = 0; m < M; ++m) {
        const uint16_t *xr = x + m * K;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) acc += oracle_bf16_to_f32(xr[k]) * wf[k];
        if (y) y[m * N + n] = oracle_f32_to_bf16(acc);
        if (y_f32) y_f32[m * N + n] = acc;
      }
    }
    free(wf);
  }
  return 0;
}

int oracle_qmm_f64(const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                   const uint16_t *biases, double *y, int64_t M, int64_t N,
                   int64_t K, int group_size, int bits, int mode) {
  if (!supported(group_size, bits, K) || M < 0 || N < 0) return -1;
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
#pragma omp parallel
  {
    float *wf = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      deq_row(w + n * wpr, scales + n * gpr, biases + n * gpr, wf, K,
              group_size, bits, mode);
      for (int64_t m = 0; m < M; ++m) {
        const uint16_t *xr = x + m * K;
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k)
          acc += (double)oracle_bf16_to_f32(xr[k]) * (double)wf[k];
        y[m * N + n] = acc;
      }
    }
    free(wf);
  }
  return 0;
}

int oracle_gather_qmm(const uint16_t *x, const uint32_t *w,
                      const uint16_t *scales, const uint16_t *biases,
                      const int32_t *xrow, const int32_t *expert, uint16_t *y,
                      int64_t S, int64_t E, int64_t N, int64_t K,
                      int group_size, int bits, int mode) {
  if (!supported(group_size, bits, K) || S < 0 || N < 0) return -1;
  for (int64_t i = 0; i < S; ++i)
    if (expert[i] < 0 || expert[i] >= E) return -2;
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
#pragma omp parallel
  {
    float *wf = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < S * N; ++t) {
      const int64_t i = t / N, n = t % N;
      const int64_t e = expert[i];
      const int64_t row = e * N + n;
      deq_row(w + row * wpr, scales + row * gpr, biases + row * gpr, wf, K,
              group_size, bits, mode);
      const uint16_t *xr = x + (int64_t)xrow[i] * K;
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += oracle_bf16_to_f32(xr[k]) * wf[k];
      y[i * N + n] = oracle_f32_to_bf16(acc);
    }
    free(wf);
  }
  return 0;
}

/* One quantized GEMV row against expert e of a stacked projection.  sq
 * (optional) receives sqrt(sum_k (x_k w_k)^2), the scale of what one-ulp
 * changes of the x_k move the result by. */
static float gemv_row(const float *xv, const uint32_t *w, const uint16_t *s,
                      const uint16_t *b, int64_t e, int64_t N, int64_t n,
                      int64_t K, int group_size, int bits, int mode, float *wf,
                      double *sq) {
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
  const int64_t row = e * N + n;
  deq_row(w + row * wpr, s + row * gpr, b + row * gpr, wf, K, group_size, bits, mode);
  float acc = 0.0f;
  double ss = 0.0;
  for (int64_t k = 0; k < K; ++k) {
    acc += xv[k] * wf[k];
    if (sq) ss += ((double)xv[k] * wf[k]) * ((double)xv[k] * wf[k]);
  }
  if (sq) *sq = sqrt(ss);
  return acc;
}

int oracle_switch_glu(const uint16_t *x, const int32_t *inds,
                      const uint32_t *wg, const uint16_t *sg, const uint16_t *bg,
                      const uint32_t *wu, const uint16_t *su, const uint16_t *bu,
                      const uint32_t *wd, const uint16_t *sd, const uint16_t *bd,
                      uint16_t *out, int64_t T, int64_t topk, int64_t E,
                      int64_t D, int64_t I, int group_size, int bits,
                      const int32_t *token_sel, int64_t n_sel, int mode,
                      double *hscale) {
  if (!supported(group_size, bits, D) || !supported(group_size, bits, I)) return -1;
  const int64_t nt = token_sel ? n_sel : T;
  for (int64_t j = 0; j < nt; ++j) {
    const int64_t t = token_sel ? token_sel[j] : j;
    if (t < 0 || t >= T) return -2;
    for (int64_t q = 0; q < topk; ++q)
      if (inds[t * topk + q] < 0 || inds[t * topk + q] >= E) return -2;
  }
  const int64_t maxk = D > I ? D : I;
  for (int64_t j = 0; j < nt; ++j) {
    const int64_t t = token_sel ? token_sel[j] : j;
    float *xv = (float *)malloc(sizeof(float) * (size_t)D);
    float *hv = (float *)malloc(sizeof(float) * (size_t)I);
    for (int64_t k = 0; k < D; ++k) xv[k] = oracle_bf16_to_f32(x[t * D + k]);
    for (int64_t q = 0; q < topk; ++q) {
      const int64_t e = inds[t * topk + q];
#pragma omp parallel
      {
        float *wf = (float *)malloc(sizeof(float) * (size_t)maxk);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < I; ++n) {
          const float g = r16(gemv_row(xv, wg, sg, bg, e, I, n, D, group_size, bits, mode, wf, NULL));
          const float u = r16(gemv_row(xv, wu, su, bu, e, I, n, D, group_size, bits, mode, wf, NULL));
          const float sig = r16(1.0f / (1.0f + expf(-g)));
          const float silu = r16(g * sig);
          hv[n] = r16(silu * u);
        }
#pragma omp for schedule(static)
        for (int64_t n = 0; n < D; ++n) {
          double sq = 0.0;
          const float d = gemv_row(hv, wd, sd, bd, e, D, n, I, group_size, bits, mode, wf,
                                   hscale ? &sq : NULL);
          out[(j * topk + q) * D + n] = oracle_f32_to_bf16(d);
          if (hscale) hscale[(j * topk + q) * D + n] = sq;
        }
        free(wf);
      }
    }
    free(xv);
    free(hv);
  }
  return 0;
}

/* CPU baseline.  Per row n and group g the product is
 *   sum_k x_k (s q_k + b) = s * sum_k x_k q_k + b * sum_k x_k,
 * which is exact algebra; the fp32 sums round differently from the
 * element-wise form, well inside the parity tolerance.  x is converted to fp32
 * once and its per-group sums are computed once per row of x. */
int oracle_qmm_cpu_fast(const uint16_t *x, const uint32_t *w,
                        const uint16_t *scales, const uint16_t *biases,
                        uint16_t *y, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits) {
  if (!supported(group_size, bits, K) || M < 0 || N < 0) return -1;
  const int64_t wpr = K * bits / 32, gpr = K / group_size;
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
  float *xs = (float *)malloc(sizeof(float) * (size_t)(M * gpr));
  for (int64_t i = 0; i < M * K; ++i) xf[i] = oracle_bf16_to_f32(x[i]);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < gpr; ++g) {
      float a = 0.0f;
      for (int64_t k = 0; k < group_size; ++k) a += xf[m * K + g * group_size + k];
      xs[m * gpr + g] = a;
    }
#pragma omp parallel
  {
    float *qf = (float *)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t *wr = w + n * wpr;
      for (int64_t i = 0; i < wpr; ++i) {
        const uint32_t word = wr[i];
        for (int p = 0; p < per; ++p) qf[i * per + p] = (float)((word >> (p * bits)) & mask);
      }
      for (int64_t m = 0; m < M; ++m) {
        const float *xr = xf + m * K;
        float acc = 0.0f;
        for (int64_t g = 0; g < gpr; ++g) {
          const float *xq = xr + g * group_size;
          const float *qq = qf + g * group_size;
          float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int64_t k = 0; k < group_size; k += 8)
            for (int j = 0; j < 8; ++j) part[j] = fmaf(xq[k + j], qq[k + j], part[j]);
          const float dot = ((part[0] + part[1]) + (part[2] + part[3])) +
                            ((part[4] + part[5]) + (part[6] + part[7]));
          const float s = oracle_bf16_to_f32(scales[n * gpr + g]);
          const float b = oracle_bf16_to_f32(biases[n * gpr + g]);
          acc = fmaf(s, dot, fmaf(b, xs[m * gpr + g], acc));
        }
        y[m * N + n] = oracle_f32_to_bf16(acc);
      }
    }
    free(qf);
  }
  free(xf);
  free(xs);
  return 0;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}


/* ---- MoE routers ------------------------------------------------------- */

/* Indices 0..n-1 ordered by val descending; equal values keep index order (the
 * reference's sort.SliceStable on an ascending index list). */
static void stable_desc_order(const double *val, int64_t n, int64_t *order) {
  for (int64_t i = 0; i < n; ++i) order[i] = i;
  for (int64_t i = 1; i < n; ++i) { /* insertion sort: stable */
    const int64_t cur = order[i];
    int64_t j = i - 1;
    while (j >= 0 && val[order[j]] < val[cur]) {
      order[j + 1] = order[j];
      --j;
    }
    order[j + 1] = cur;
  }
}

/* GroupExpertSelect, compute/models/deepseekv3.go:305-384. */
int oracle_route_group_topk(const float *gates, const float *bias, int64_t T, int64_t E,
                            int top_k, int n_group, int topk_group, double scale, int norm,
                            int32_t *inds, double *scores) {
  if (T < 0 || E < 1 || top_k < 1 || n_group < 1 || E % n_group) return -1;
  if (top_k > E) top_k = (int)E; /* :354-356 */
  double *orig = malloc(sizeof(double) * E), *biased = malloc(sizeof(double) * E);
  double *gscore = malloc(sizeof(double) * n_group);
  int64_t *order = malloc(sizeof(int64_t) * E), *gorder = malloc(sizeof(int64_t) * n_group);
  char *keep = malloc(n_group);
  for (int64_t t = 0; t < T; ++t) {
    const float *g = gates + t * E;
    for (int64_t i = 0; i < E; ++i) { /* :307-316 */
      orig[i] = 1.0 / (1.0 + exp(-(double)g[i]));
      biased[i] = orig[i] + (bias ? (double)bias[i] : 0.0);
    }
    if (n_group > 1) { /* :318-346 */
      const int64_t per = E / n_group;
      for (int grp = 0; grp < n_group; ++grp) {
        /* the group's two best biased scores (one when the group has one expert) */
        double t1 = -INFINITY, t2 = -INFINITY;
        for (int64_t j = grp * per; j < (grp + 1) * per; ++j) {
          const double v = biased[j];
          if (v > t1) { t2 = t1; t1 = v; } else if (v > t2) { t2 = v; }
        }
        gscore[grp] = per > 1 ? t1 + t2 : t1;
      }
      stable_desc_order(gscore, n_group, gorder);
      for (int grp = 0; grp < n_group; ++grp) keep[grp] = 0;
      for (int i = 0; i < topk_group && i < n_group; ++i) keep[gorder[i]] = 1;
      for (int grp = 0; grp < n_group; ++grp)
        if (!keep[grp])
          for (int64_t j = grp * per; j < (grp + 1) * per; ++j) biased[j] = 0.0;
    }
    stable_desc_order(biased, E, order); /* :349-353 */
    double denom = 0.0;
    for (int j = 0; j < top_k; ++j) {
      inds[t * top_k + j] = (int32_t)order[j];
      scores[t * top_k + j] = orig[order[j]]; /* :359-362 */
      denom += scores[t * top_k + j];
    }
    if (top_k > 1 && norm && denom != 0.0) /* :363-372 */
      for (int j = 0; j < top_k; ++j) scores[t * top_k + j] /= denom;
    for (int j = 0; j < top_k; ++j) scores[t * top_k + j] *= scale; /* :373-375 */
  }
  free(orig); free(biased); free(gscore); free(order); free(gorder); free(keep);
  return 0;
}

/* qwen3NextMoE's router, compute/models/qwen3next_forward.go:513-518. */
int oracle_route_softmax_topk(const float *logits, int64_t T, int64_t E, int top_k, int norm,
                              int32_t *inds, double *weights) {
  if (T < 0 || E < 1 || top_k < 1 || top_k > E) return -1;
  double *p = malloc(sizeof(double) * E);
  int64_t *order = malloc(sizeof(int64_t) * E);
  for (int64_t t = 0; t < T; ++t) {
    const float *x = logits + t * E;
    double m = -INFINITY, s = 0.0;
    for (int64_t i = 0; i < E; ++i) m = x[i] > m ? x[i] : m;
    for (int64_t i = 0; i < E; ++i) { p[i] = exp((double)x[i] - m); s += p[i]; }
    for (int64_t i = 0; i < E; ++i) p[i] /= s; /* softmax, :514 */
    stable_desc_order(p, E, order);              /* argpartition top-k, :515 */
    double sel = 0.0;
    for (int j = 0; j < top_k; ++j) {
      inds[t * top_k + j] = (int32_t)order[j];
      weights[t * top_k + j] = p[order[j]]; /* takeAlongAxis, :516 */
      sel += p[order[j]];
    }
    if (norm) /* :517-518 */
      for (int j = 0; j < top_k; ++j) weights[t * top_k + j] /= sel;
  }
  free(p); free(order);
  return 0;
}
