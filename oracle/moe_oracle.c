/*
 * CPU restatement of mixlab's MoE feed-forward op (IR op 74).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for libmixmoe: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product never calls it.
 *
 * It follows moe_feed_forward, gpu/ir.cpp:1073-1164, step by step:
 *   (ii)   logits = x . router_w                     gpu/ir.cpp:1106
 *   (iii)  probs = softmax(logits, -1)               gpu/ir.cpp:1107
 *   (iv)   top_idx = argsort(-probs)[:, :K] (stable) gpu/ir.cpp:1108-1109
 *   (v)    top_norm = top_p / max(sum_k top_p, 1e-12) gpu/ir.cpp:1110-1111
 *   (vi)   for e in 0..E-1: out += FFN_e(x) * gate_e  gpu/ir.cpp:1118-1148
 *   (vii)  aux = E * sum_e mean(probs[:,e]) * mean(sel_e / K)  gpu/ir.cpp:1150-1159
 *   (viii) entropy = -mean_n sum_e p log max(p, 1e-12) gpu/ir.cpp:1161-1162
 * with the expert FFNs of gpu/ir.cpp:1126-1145 and activations of
 * gpu/ir.cpp:1053-1071.  `dense` runs every expert on every row, as the
 * reference does; otherwise only routed rows are computed, which gives the
 * same bits (unselected experts add y*0 = +-0 to `out`).
 *
 * Dtype flows.  fp32: every step in fp32.  bf16 (compute_dtype "bf16"): the
 * MLX dtype flow implied by gpu/ir.cpp under MLX's promotion rules -- logits
 * and probs bf16; the top-p sum is bf16, the renorm fp32 (the 1e-12 array is
 * fp32); projections bf16; sigmoid / products bf16 for swiglu, mlp-silu and
 * relu; gelu and leaky_relu_sq in fp32 (their float32 scalar arrays promote);
 * y bf16 exactly when the hidden is bf16; out fp32.  Callers pass inputs
 * already rounded to bf16 in the bf16 flow.
 *
 * Arithmetic contract (what MLX leaves unspecified, fixed here and in the
 * device code alike): the router logits split d into chunks of 64 from d = 0,
 * each chunk's partial an fmaf chain over its d in ascending order from +0,
 * and the logit is +0 plus the chunk partials added in ascending chunk order;
 * the expert FFN's dot products accumulate in fp32 by fmaf over the reduction
 * index in ascending order; exp is Cody-Waite reduction with a
 * degree-7 Taylor polynomial; the softmax denominator is summed lane-wise
 * (lane l holds experts l, l+64, ...) and then by an xor butterfly over 64
 * lanes; probabilities below 2^-126 flush to +0; bf16 rounding is
 * round-to-nearest-even.  The combine multiplies then adds (no fma).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* Planted mistakes.  tests/test_oracle_bf16.py compiles copies of this file
 * with one ORACLE_PLANT_<NAME> macro defined and checks that its pins reject
 * each; the default build (oracle/Makefile) defines none, and then every
 * PLANT(...) below is 0.  Each names one plausible slip in the bf16 dtype
 * flow: a rounding dropped, or a decision taken on unrounded values. */
#define PLANT(name) PLANT_##name
#ifdef ORACLE_PLANT_LOGITS_FP32
#define PLANT_LOGITS_FP32 1 /* logits not rounded to bf16 */
#else
#define PLANT_LOGITS_FP32 0
#endif
#ifdef ORACLE_PLANT_PROBS_FP32
#define PLANT_PROBS_FP32 1 /* probabilities not rounded to bf16 */
#else
#define PLANT_PROBS_FP32 0
#endif
#ifdef ORACLE_PLANT_TOPK_FP32
#define PLANT_TOPK_FP32 1 /* top-k ranked on the unrounded fp32 probabilities */
#else
#define PLANT_TOPK_FP32 0
#endif
#ifdef ORACLE_PLANT_TOPSUM_FP32
#define PLANT_TOPSUM_FP32 1 /* the top-p sum left in fp32 */
#else
#define PLANT_TOPSUM_FP32 0
#endif
#ifdef ORACLE_PLANT_AUX_MEAN_FP32
#define PLANT_AUX_MEAN_FP32 1 /* the per-expert mean probability left in fp32 */
#else
#define PLANT_AUX_MEAN_FP32 0
#endif
#ifdef ORACLE_PLANT_ENTROPY_FP32
#define PLANT_ENTROPY_FP32 1 /* entropy from the unrounded probabilities */
#else
#define PLANT_ENTROPY_FP32 0
#endif
#ifdef ORACLE_PLANT_PROJ_FP32
#define PLANT_PROJ_FP32 1 /* expert projections not rounded to bf16 */
#else
#define PLANT_PROJ_FP32 0
#endif
#ifdef ORACLE_PLANT_SWIGLU_SIG
#define PLANT_SWIGLU_SIG 1 /* swiglu: sigmoid(g) not rounded */
#else
#define PLANT_SWIGLU_SIG 0
#endif
#ifdef ORACLE_PLANT_SWIGLU_PROD
#define PLANT_SWIGLU_PROD 1 /* swiglu: sigmoid(g) * u not rounded */
#else
#define PLANT_SWIGLU_PROD 0
#endif
#ifdef ORACLE_PLANT_GEGLU_SQ
#define PLANT_GEGLU_SQ 1 /* geglu: square(g) not rounded */
#else
#define PLANT_GEGLU_SQ 0
#endif
#ifdef ORACLE_PLANT_SILU_SIG
#define PLANT_SILU_SIG 1 /* mlp silu: sigmoid(u) not rounded */
#else
#define PLANT_SILU_SIG 0
#endif
#ifdef ORACLE_PLANT_GELU_SQ
#define PLANT_GELU_SQ 1 /* mlp gelu: square(u) not rounded */
#else
#define PLANT_GELU_SQ 0
#endif
#ifdef ORACLE_PLANT_Y_FP32
#define PLANT_Y_FP32 1 /* expert output y of a bf16-hidden kind left in fp32 */
#else
#define PLANT_Y_FP32 0
#endif
#ifdef ORACLE_PLANT_Y_BF16
#define PLANT_Y_BF16 1 /* expert output y rounded to bf16 for every kind */
#else
#define PLANT_Y_BF16 0
#endif

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_round_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return u2f(((u >> 16) | 0x0040u) << 16);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u2f(u & 0xffff0000u);
}

static inline float ftz(float f) { return ((f2u(f) & 0x7f800000u) == 0u) ? 0.0f : f; }

/* e^x = 2^n e^r, n = rint(x log2 e), r = x - n ln2 (Cody & Waite split of
 * ln2 into 0.693145751953125 + 1.4286068203094172e-06), e^r by the Taylor
 * polynomial of degree 7 in Horner form. */
float oracle_exp(float x) {
  if (!(x == x)) return x;
  if (x > 88.0f) return INFINITY;
  if (x < -86.5f) return 0.0f;
  const float n = rintf(x * 1.4426950408889634f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.4286068203094172e-06f, r);
  float p = 1.9841269841269841e-04f;
  p = fmaf(p, r, 1.3888888888888889e-03f);
  p = fmaf(p, r, 8.3333333333333333e-03f);
  p = fmaf(p, r, 4.1666666666666667e-02f);
  p = fmaf(p, r, 1.6666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return p * u2f((uint32_t)((int)n + 127) << 23);
}

float oracle_sigmoid(float x) { return 1.0f / (1.0f + oracle_exp(-x)); }

float oracle_tanh(float x) {
  const float a = fabsf(x);
  const float t = oracle_exp(-2.0f * a);
  return copysignf((1.0f - t) / (1.0f + t), x);
}

/* gpu/ir.cpp:1054-1056, operation by operation; sq = square(v). */
float oracle_gelu_tanh(float v, float sq) {
  const float a = 0.044715f * v;
  const float b = a * sq;
  const float c = v + b;
  const float d = 0.7978845608f * c;
  const float t = oracle_tanh(d);
  const float e = 1.0f + t;
  const float f = 0.5f * v;
  return f * e;
}

/* d per chunk of the router logits' summation order */
#define ORACLE_LOGIT_CHUNK 64

enum { SWIGLU = 0, GEGLU = 1, MLP = 2 };
enum { SILU = 0, GELU = 1, RELU = 2, LEAKY_RELU_SQ = 3 };

static inline float R(int bf16, float v) { return bf16 ? oracle_round_bf16(v) : v; }

/* Hidden unit of one expert row (gpu/ir.cpp:1130-1145 and 1057-1068). */
float oracle_hidden(int bf16, int etype, int act, float slope, float g, float u) {
  if (etype == SWIGLU)
    return R(bf16 && !PLANT(SWIGLU_PROD), R(bf16 && !PLANT(SWIGLU_SIG), oracle_sigmoid(g)) * u);
  if (etype == GEGLU) return oracle_gelu_tanh(g, R(bf16 && !PLANT(GEGLU_SQ), g * g)) * u;
  switch (act) {
    case SILU:
      return R(bf16, u * R(bf16 && !PLANT(SILU_SIG), oracle_sigmoid(u)));
    case GELU:
      return oracle_gelu_tanh(u, R(bf16 && !PLANT(GELU_SQ), u * u));
    case RELU:
      return u > 0.0f ? u : 0.0f;
    default: {
      const float y = u > 0.0f ? u : u * slope;
      return y * y;
    }
  }
}

static int hidden_is_bf16(int etype, int act) {
  if (PLANT(Y_FP32)) return 0;
  if (PLANT(Y_BF16)) return 1;
  if (etype == SWIGLU) return 1;
  if (etype == GEGLU) return 0;
  return act == SILU || act == RELU;
}

/* out[r][c] = sum_k a[r][k] * b[k][c], fmaf in ascending k, for `nr` rows
 * of `a` given by row pointers. */
static void gemm_rows(const float* const* arows, int nr, const float* b, int inner, int cols,
                      float* out /* [nr][cols] */) {
  for (int i = 0; i < nr * cols; ++i) out[i] = 0.0f;
  for (int k = 0; k < inner; ++k) {
    const float* bk = b + (size_t)k * cols;
    for (int r = 0; r < nr; ++r) {
      const float av = arows[r][k];
      float* o = out + (size_t)r * cols;
      for (int c = 0; c < cols; ++c) o[c] = fmaf(av, bk[c], o[c]);
    }
  }
}

/* Router for rows [n0, n1): logits, probs, top-k, gates. */
static void route_rows(int n0, int n1, int D, int E, int K, int bf16, const float* x,
                       const float* wr, float* logits, float* probs, float* probs_raw,
                       int32_t* top_idx, float* gates) {
  float* acc = (float*)malloc(sizeof(float) * (size_t)E);
  float* part = (float*)malloc(sizeof(float) * (size_t)E);
  float* ex = (float*)malloc(sizeof(float) * (size_t)E);
  unsigned char* taken = (unsigned char*)malloc((size_t)E);
  for (int n = n0; n < n1; ++n) {
    /* logits: chunks of ORACLE_LOGIT_CHUNK d, each an fmaf chain from +0,
       the partials added to +0 in chunk order */
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    for (int d0 = 0; d0 < D; d0 += ORACLE_LOGIT_CHUNK) {
      const int d1 = (d0 + ORACLE_LOGIT_CHUNK < D) ? d0 + ORACLE_LOGIT_CHUNK : D;
      for (int e = 0; e < E; ++e) part[e] = 0.0f;
      for (int d = d0; d < d1; ++d) {
        const float xv = x[(size_t)n * D + d];
        const float* w = wr + (size_t)d * E;
        for (int e = 0; e < E; ++e) part[e] = fmaf(xv, w[e], part[e]);
      }
      for (int e = 0; e < E; ++e) acc[e] = acc[e] + part[e];
    }
    float* lg = logits + (size_t)n * E;
    float* p = probs + (size_t)n * E;
    float* praw = probs_raw + (size_t)n * E;
    float m = -INFINITY;
    for (int e = 0; e < E; ++e) {
      lg[e] = R(bf16 && !PLANT(LOGITS_FP32), acc[e]);
      m = fmaxf(m, lg[e]);
    }
    for (int e = 0; e < E; ++e) ex[e] = oracle_exp(lg[e] - m);
    float lane[64];
    for (int l = 0; l < 64; ++l) {
      float s = (l < E) ? ex[l] : 0.0f;
      for (int e = l + 64; e < E; e += 64) s = s + ex[e];
      lane[l] = s;
    }
    for (int off = 32; off >= 1; off >>= 1) {
      float nx[64];
      for (int l = 0; l < 64; ++l) nx[l] = lane[l] + lane[l ^ off];
      memcpy(lane, nx, sizeof lane);
    }
    const float sum = lane[0];
    for (int e = 0; e < E; ++e) {
      praw[e] = ftz(ex[e] / sum);
      p[e] = R(bf16 && !PLANT(PROBS_FP32), praw[e]);
    }
    /* stable argsort(-p): largest first, ties to the lower expert index */
    const float* rank = PLANT(TOPK_FP32) ? praw : p;
    memset(taken, 0, (size_t)E);
    float s_top = 0.0f;
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (!taken[e] && (best < 0 || rank[e] > rank[best])) best = e;
      taken[best] = 1;
      top_idx[(size_t)n * K + k] = best;
      s_top = (k == 0) ? p[best] : s_top + p[best];
    }
    const float den = fmaxf(R(bf16 && !PLANT(TOPSUM_FP32), s_top), 1e-12f);
    for (int k = 0; k < K; ++k) gates[(size_t)n * K + k] = p[top_idx[(size_t)n * K + k]] / den;
  }
  free(acc);
  free(part);
  free(ex);
  free(taken);
}

/*
 * Returns 0 on success, -1 on bad arguments.
 *   x [N, D], router_w [D, E], expert_w: per expert, in input order,
 *   (w_gate [D,F], w_up [D,F], w_down [F,D]) or (w_up [D,F], w_down [F,D]).
 *   rows/n_rows: optional subset of rows for which delta is computed (other
 *   rows of delta are left untouched); routing, aux and entropy always cover
 *   all N rows.
 *   Outputs (any may be NULL except delta when delta is wanted):
 *   delta [N, D], aux [1], entropy [1], top_idx [N, K], gates [N, K],
 *   probs [N, E], logits [N, E], counts [E], offsets [E+1], perm [N*K].
 */
int oracle_moe_forward(int N, int D, int E, int K, int etype, int F, int act, float slope,
                       int bf16, int dense, const float* x, const float* router_w,
                       const float* expert_w, const int32_t* rows, int n_rows, float* delta,
                       float* aux, float* entropy, int32_t* top_idx_out, float* gates_out,
                       float* probs_out, float* logits_out, int32_t* counts, int32_t* offsets,
                       int32_t* perm) {
  if (N <= 0 || D <= 0 || E <= 0 || K <= 0 || K > E || F <= 0) return -1;
  if (etype < SWIGLU || etype > MLP) return -1;
  const int wpe = (etype == MLP) ? 2 : 3;
  const size_t NE = (size_t)N * E, NK = (size_t)N * K;
  float* logits = logits_out ? logits_out : (float*)malloc(sizeof(float) * NE);
  float* probs = probs_out ? probs_out : (float*)malloc(sizeof(float) * NE);
  int32_t* top_idx = top_idx_out ? top_idx_out : (int32_t*)malloc(sizeof(int32_t) * NK);
  float* gates = gates_out ? gates_out : (float*)malloc(sizeof(float) * NK);
  float* probs_raw = (float*)malloc(sizeof(float) * NE); /* before the bf16 rounding */

#pragma omp parallel
  {
#ifdef _OPENMP
    const int nt = omp_get_num_threads(), it = omp_get_thread_num();
#else
    const int nt = 1, it = 0;
#endif
    const int chunk = (N + nt - 1) / nt;
    const int a = it * chunk, b = (a + chunk < N) ? a + chunk : N;
    if (a < b)
      route_rows(a, b, D, E, K, bf16, x, router_w, logits, probs, probs_raw, top_idx, gates);
  }

  /* aux and entropy (gpu/ir.cpp:1150-1162) */
  int32_t* cnt = (int32_t*)calloc((size_t)E, sizeof(int32_t));
  for (size_t i = 0; i < NK; ++i) cnt[top_idx[i]]++;
  if (aux) {
    float acc = 0.0f;
    for (int e = 0; e < E; ++e) {
      double s = 0.0;
      for (int n = 0; n < N; ++n) s += probs[(size_t)n * E + e];
      const float pm = R(bf16 && !PLANT(AUX_MEAN_FP32), (float)(s / N));
      const float frac = ((float)cnt[e] / (float)K) / (float)N;
      const float term = pm * frac;
      acc = (e == 0) ? term : acc + term;
    }
    *aux = acc * (float)E;
  }
  if (entropy) {
    double tot = 0.0;
    for (int n = 0; n < N; ++n) {
      float rs = 0.0f;
      for (int e = 0; e < E; ++e) {
        const float q = (PLANT(ENTROPY_FP32) ? probs_raw : probs)[(size_t)n * E + e];
        rs += q * logf(fmaxf(q, 1e-12f));
      }
      tot += rs;
    }
    *entropy = (float)(-(tot / N));
  }

  /* grouping implied by the `top_idx == e` masks: per expert, ascending n */
  int32_t* off = (int32_t*)malloc(sizeof(int32_t) * ((size_t)E + 1));
  off[0] = 0;
  for (int e = 0; e < E; ++e) off[e + 1] = off[e] + cnt[e];
  if (counts) memcpy(counts, cnt, sizeof(int32_t) * (size_t)E);
  if (offsets) memcpy(offsets, off, sizeof(int32_t) * ((size_t)E + 1));
  int32_t* grp = (int32_t*)malloc(sizeof(int32_t) * (NK > 0 ? NK : 1));
  {
    int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    memcpy(fill, off, sizeof(int32_t) * (size_t)E);
    for (int n = 0; n < N; ++n) {
      /* experts of a row in ascending id, so each expert's list is ascending in n */
      for (int e = 0; e < E; ++e)
        for (int k = 0; k < K; ++k)
          if (top_idx[(size_t)n * K + k] == e) grp[fill[e]++] = n;
    }
    free(fill);
  }
  if (perm) memcpy(perm, grp, sizeof(int32_t) * NK);

  if (delta) {
    /* row mask for the optional subset */
    unsigned char* want = (unsigned char*)malloc((size_t)N);
    if (rows) {
      memset(want, 0, (size_t)N);
      for (int i = 0; i < n_rows; ++i)
        if (rows[i] >= 0 && rows[i] < N) want[rows[i]] = 1;
    } else {
      memset(want, 1, (size_t)N);
    }
    for (int n = 0; n < N; ++n)
      if (want[n])
        for (int d = 0; d < D; ++d) delta[(size_t)n * D + d] = 0.0f;
    const int ybf = bf16 && hidden_is_bf16(etype, act);
    const size_t DF = (size_t)D * F;
    for (int e = 0; e < E; ++e) {
      const float* we = expert_w + (size_t)e * wpe * DF;
      const float* wg = (wpe == 3) ? we : NULL;
      const float* wu = (wpe == 3) ? we + DF : we;
      const float* wd = we + (size_t)(wpe - 1) * DF;
      /* rows this expert runs on */
      int nrow = 0;
      int32_t* list = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
      if (dense) {
        for (int n = 0; n < N; ++n)
          if (want[n]) list[nrow++] = n;
      } else {
        for (int i = off[e]; i < off[e + 1]; ++i)
          if (want[grp[i]]) list[nrow++] = grp[i];
      }
#pragma omp parallel for schedule(dynamic, 1)
      for (int b0 = 0; b0 < nrow; b0 += 8) {
        const int nb = (nrow - b0 < 8) ? nrow - b0 : 8;
        const float* ar[8];
        float* g = (float*)malloc(sizeof(float) * (size_t)nb * F);
        float* u = (float*)malloc(sizeof(float) * (size_t)nb * F);
        float* y = (float*)malloc(sizeof(float) * (size_t)nb * D);
        for (int r = 0; r < nb; ++r) ar[r] = x + (size_t)list[b0 + r] * D;
        if (wg) gemm_rows(ar, nb, wg, D, F, g);
        gemm_rows(ar, nb, wu, D, F, u);
        const int rp = bf16 && !PLANT(PROJ_FP32); /* projections are bf16 matmuls */
        for (int i = 0; i < nb * F; ++i) {
          const float gi = wg ? R(rp, g[i]) : 0.0f;
          u[i] = oracle_hidden(bf16, etype, act, slope, gi, R(rp, u[i]));
        }
        const float* hr[8];
        for (int r = 0; r < nb; ++r) hr[r] = u + (size_t)r * F;
        gemm_rows(hr, nb, wd, F, D, y);
        for (int r = 0; r < nb; ++r) {
          const int n = list[b0 + r];
          float gate = 0.0f; /* sum_k where(top_idx == e, top_norm, 0), gpu/ir.cpp:1121 */
          for (int k = 0; k < K; ++k)
            gate = gate + ((top_idx[(size_t)n * K + k] == e) ? gates[(size_t)n * K + k] : 0.0f);
          float* o = delta + (size_t)n * D;
          const float* yr = y + (size_t)r * D;
          for (int d = 0; d < D; ++d) {
            const float yv = ybf ? oracle_round_bf16(yr[d]) : yr[d];
            const volatile float prod = yv * gate;
            o[d] = o[d] + prod;
          }
        }
        free(g);
        free(u);
        free(y);
      }
      free(list);
    }
    free(want);
  }

  free(cnt);
  free(off);
  free(grp);
  free(probs_raw);
  if (!logits_out) free(logits);
  if (!probs_out) free(probs);
  if (!top_idx_out) free(top_idx);
  if (!gates_out) free(gates);
  return 0;
}

/* Vectorised helpers for the tests. */
void oracle_exp_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_exp(x[i]);
}
void oracle_round_bf16_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_round_bf16(x[i]);
}
void oracle_hidden_array(int bf16, int etype, int act, float slope, const float* g,
                         const float* u, float* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = oracle_hidden(bf16, etype, act, slope, g[i], u[i]);
}

/*
 * RMSNorm in front of op 74 (block level, arch/moe.go:152-166), following
 * gpu/ir.cpp:4949-4960: y = astype(x_f32 * (1 / sqrt(mean(x^2) + eps)) *
 * scale, x.dtype).  MLX's reduction order is not specified; this build fixes
 * it (and the device kernel follows it): 64 partial sums, partial l holding
 * x[d]^2 (product rounded, then added) for d = 256*i + 4*l + j in (i, j)
 * order; the partials meet in an xor butterfly over distances 32..1; the
 * mean is sum * (float)(1/D).  sqrt and the division are correctly rounded.
 * out_bf16 rounds y to bf16 (the bf16 flow), else y stays fp32.
 */
void oracle_rmsnorm(int N, int D, const float* x, const float* scale, float eps, int out_bf16,
                    float* out) {
  const float inv_d = (float)(1.0 / (double)D);
  for (int n = 0; n < N; ++n) {
    const float* xr = x + (size_t)n * D;
    float lanes[64], tmp[64];
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (int d0 = 0; d0 < D; d0 += 256)
        for (int j = 0; j < 4; ++j) {
          const int d = d0 + 4 * l + j;
          if (d < D) {
            const float p = xr[d] * xr[d];
            acc = acc + p;
          }
        }
      lanes[l] = acc;
    }
    for (int s = 32; s >= 1; s >>= 1) {
      for (int l = 0; l < 64; ++l) tmp[l] = lanes[l] + lanes[l ^ s];
      memcpy(lanes, tmp, sizeof(lanes));
    }
    const float ms = lanes[0] * inv_d;
    const float r = 1.0f / sqrtf(ms + eps);
    for (int d = 0; d < D; ++d) {
      const float y = (xr[d] * r) * scale[d];
      out[(size_t)n * D + d] = out_bf16 ? oracle_round_bf16(y) : y;
    }
  }
}
