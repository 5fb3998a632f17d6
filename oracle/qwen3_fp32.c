/* Host-independent fp32 restatement of the Qwen3 bf16 decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/ (through oracle/qwen3_fp32.py) load
 * this library, as a checker; the product path never calls it.
 *
 * What it restates: the reference's correctness oracle, HF transformers'
 * Qwen3 bf16 eager decode (reference qwen_megakernel/bench.py:83-133; HF
 * modeling_qwen3.py), with the same bf16 rounding points as
 * oracle/qwen3_ref.py and oracle/qwen3_exact.py, computed the way an fp32
 * implementation computes them -- but with every fp32 sum taken in one fixed
 * order, so that the result depends on the inputs alone and not on a CPU's
 * BLAS or vector width:
 *
 *   - bf16 x bf16 products are exact in fp32 (8 x 8 significant bits);
 *   - every sum (dot products, the RMSNorm mean of squares, the softmax
 *     denominator, P @ V) is taken in one of four fixed orders, chosen per
 *     call (tree_sum below): a pairwise tree, left to right, eight
 *     interleaved partial sums, right to left.  Different orders give
 *     different fp32 results on the same inputs; their spread is the size of
 *     error an fp32 implementation carries;
 *   - exp is evaluated in float64 and rounded to fp32 (one rounding of an
 *     almost exact value); 1/sqrt, divisions and the remaining products are
 *     single IEEE fp32 operations, as torch's CPU kernels perform them.
 *
 * Rounding points (HF modeling_qwen3.py, transformers 5.15.0; the same list
 * as oracle/qwen3_exact.py):
 *   RMSNorm       bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps))))   (:59-64)
 *   Linear        bf16(sum of products)                             (:82, :232-246, :495)
 *   q/k head norm RMSNorm over head_dim                             (:252-253)
 *   RoPE          bf16(bf16(x cos) + bf16(rotate_half(x) sin))      (:140-169)
 *   attention     s = bf16(q.k), bf16(s * scale), p = bf16(e / L) with
 *                 e = exp(s - max), computed as e * (1 / L) (torch's
 *                 softmax multiplies by the reciprocal), out = bf16(p . v)
 *                                                                   (:185-203)
 *   residual      bf16(a + b)                                        (:316, :322)
 *   MLP           bf16(bf16(g / (1 + exp(-g))) * u)                  (:82)
 *   logits        bf16, argmax first index                          (:432)
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off: no fused
 * multiply-add may merge a product into a sum).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint16_t bf16;

static inline float bf(bf16 h) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}

/* fp32 -> bf16, round to nearest, ties to even (the values here are finite). */
static inline bf16 rbf(float f) {
  union { uint32_t u; float f; } c;
  c.f = f;
  uint32_t u = c.u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16)(u >> 16);
}

static inline float rf(float f) { return bf(rbf(f)); }

static inline float exp_f(float x) { return (float)exp((double)x); }

static int pow2_at_least(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

/* The summation order of every fp32 sum (set per call of qf_forward):
 *   0  pairwise tree over buf[0..n) padded with zeros to a power of two: level by level, element i of
 *      the first half plus element i of the second half;
 *   1  left to right;
 *   2  eight interleaved partial sums (term i into sum i % 8, left to right), then the eight sums by
 *      the tree of order 0 -- the order of an 8-lane vector loop;
 *   3  right to left.
 * buf has room for pow2_at_least(n) floats. */
static int g_order = 0;

static float tree_sum(float* buf, int n) {
  if (g_order == 1 || g_order == 3) {
    float a = 0.0f;
    if (g_order == 1)
      for (int i = 0; i < n; i++) a = a + buf[i];
    else
      for (int i = n - 1; i >= 0; i--) a = a + buf[i];
    return a;
  }
  if (g_order == 2) {
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; i++) l[i & 7] = l[i & 7] + buf[i];
    for (int h = 4; h >= 1; h >>= 1)
      for (int i = 0; i < h; i++) l[i] = l[i] + l[i + h];
    return l[0];
  }
  int p = pow2_at_least(n);
  for (int i = n; i < p; i++) buf[i] = 0.0f;
  while (p > 1) {
    const int h = p >> 1;
    for (int i = 0; i < h; i++) buf[i] = buf[i] + buf[i + h];
    p = h;
  }
  return buf[0];
}

static float dot_bf16(const bf16* a, const bf16* b, int n, float* buf) {
  for (int i = 0; i < n; i++) buf[i] = bf(a[i]) * bf(b[i]);
  return tree_sum(buf, n);
}

typedef struct {
  int num_layers, hidden, inter, nq, nkv, hd, vocab, max_seq;
  float eps;   /* the fp32 value HF adds */
  float scale; /* the fp32 attention scale */
  const bf16* embed;
  const bf16* lm_head;
  const bf16* final_norm;
  const bf16* cos_t; /* [max_seq][hd] */
  const bf16* sin_t;
  const bf16* const* layers; /* 11 per layer: in_ln, wq, wk, wv, q_norm, k_norm, wo, post_ln, wg, wu, wd */
  bf16* k_cache;             /* [L][NKV][max_seq][hd] */
  bf16* v_cache;
} QfModel;

/* bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) over n elements, x given as fp32 holding bf16 values. */
static void rms_norm(const float* x, const bf16* w, int n, float eps, float* out, float* buf) {
  for (int i = 0; i < n; i++) buf[i] = x[i] * x[i];
  const float var = tree_sum(buf, n) / (float)n;
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int i = 0; i < n; i++) out[i] = rf(bf(w[i]) * rf(x[i] * rstd));
}

/* out[t][r] = bf16(x[t] . W[r]) for rows r < nout, K = k, T rows of x (bf16 bits). */
static void linear(const bf16* x, int T, const bf16* W, int nout, int k, float* out, int ldo) {
#pragma omp parallel
  {
    float* buf = (float*)malloc(sizeof(float) * (size_t)pow2_at_least(k));
#pragma omp for schedule(static)
    for (int r = 0; r < nout; r++) {
      const bf16* wr = W + (size_t)r * k;
      for (int t = 0; t < T; t++) out[(size_t)t * ldo + r] = rf(dot_bf16(x + (size_t)t * k, wr, k, buf));
    }
    free(buf);
  }
}

/* Logits of T final hidden rows: bf16 values as fp32, [T][vocab]. */
static void lm_logits(const QfModel* m, const bf16* n, int T, float* logits) {
  linear(n, T, m->lm_head, m->vocab, m->hidden, logits, m->vocab);
}

static void to_bf16_bits(const float* x, bf16* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = rbf(x[i]);
}

/* Row 0 of pv ([P2][hd], n rows used) becomes the sum of the n rows, for every column at once, in the
 * order tree_sum uses. */
static void sum_rows(float* pv, int n, int P2, int hd) {
  if (g_order == 1 || g_order == 3) {
    float* a = pv;
    if (g_order == 3) {
      a = pv + (size_t)(n - 1) * hd;
      for (int i = n - 2; i >= 0; i--)
        for (int d = 0; d < hd; d++) a[d] = a[d] + pv[(size_t)i * hd + d];
    } else {
      for (int i = 1; i < n; i++)
        for (int d = 0; d < hd; d++) a[d] = a[d] + pv[(size_t)i * hd + d];
    }
    /* 0 + x = x, so starting from the first term is the left-to-right sum */
    if (a != pv) memcpy(pv, a, sizeof(float) * hd);
    return;
  }
  if (g_order == 2) {
    /* rows i and i + 8j into row i % 8, left to right, then the eight rows by the tree */
    for (int i = 8; i < n; i++)
      for (int d = 0; d < hd; d++) pv[(size_t)(i & 7) * hd + d] = pv[(size_t)(i & 7) * hd + d] + pv[(size_t)i * hd + d];
    for (int i = n; i < 8; i++) memset(pv + (size_t)i * hd, 0, sizeof(float) * hd);
    for (int h = 4; h >= 1; h >>= 1)
      for (int i = 0; i < h; i++)
        for (int d = 0; d < hd; d++) pv[(size_t)i * hd + d] = pv[(size_t)i * hd + d] + pv[(size_t)(i + h) * hd + d];
    return;
  }
  for (int i = n; i < P2; i++) memset(pv + (size_t)i * hd, 0, sizeof(float) * hd);
  int w = P2;
  while (w > 1) {
    const int half = w >> 1;
    for (int i = 0; i < half; i++) {
      float* a = pv + (size_t)i * hd;
      const float* b = pv + (size_t)(i + half) * hd;
      for (int d = 0; d < hd; d++) a[d] = a[d] + b[d];
    }
    w = half;
  }
}

/* Attention of one row: q (bf16 bits, [GQ heads][hd]) of KV head g at position p; cache rows for
 * positions < p are in kc / vc ([max_seq][hd] of this head and layer), the row's own key and value
 * (position p) in k_own / v_own.  Writes bf16 values (as fp32) of the GQ heads' outputs. */
static void attend(const QfModel* m, const bf16* q, int gq, const bf16* kc, const bf16* vc, const bf16* k_own,
                   const bf16* v_own, int p, float* out) {
  const int hd = m->hd, C = p + 1, P2 = pow2_at_least(C);
  float* s = (float*)malloc(sizeof(float) * (size_t)P2);
  float* buf = (float*)malloc(sizeof(float) * (size_t)(P2 > hd ? P2 : hd));
  float* pv = (float*)malloc(sizeof(float) * (size_t)(P2 > 8 ? P2 : 8) * hd);  /* order 2 uses 8 rows */
  for (int h = 0; h < gq; h++) {
    const bf16* qh = q + (size_t)h * hd;
    float mx = -INFINITY;
    for (int i = 0; i < C; i++) {
      const bf16* kr = i < p ? kc + (size_t)i * hd : k_own;
      const float sc = rf(rf(dot_bf16(qh, kr, hd, buf)) * m->scale);
      s[i] = sc;
      if (sc > mx) mx = sc;
    }
    for (int i = 0; i < C; i++) s[i] = exp_f(s[i] - mx);
    for (int i = 0; i < C; i++) buf[i] = s[i];
    const float inv = 1.0f / tree_sum(buf, C);
    /* pv[i][d] = p_i * v_i[d]; the tree runs over i for every d at once */
    for (int i = 0; i < C; i++) {
      const float pr = rf(s[i] * inv);
      const bf16* vr = i < p ? vc + (size_t)i * hd : v_own;
      for (int d = 0; d < hd; d++) pv[(size_t)i * hd + d] = pr * bf(vr[d]);
    }
    sum_rows(pv, C, P2, hd);
    for (int d = 0; d < hd; d++) out[(size_t)h * hd + d] = rf(pv[d]);
  }
  free(pv);
  free(buf);
  free(s);
}

/* T tokens at positions p0 .. p0+T-1.  given_cache = 0: the rows' K/V are written into the cache
 * at their positions, and row i attends to positions 0..p0+i of the cache.  given_cache = 1: the
 * cache already holds another decoder's rows for every position below p0+T; row i attends to the
 * cache's rows below p0+i and to its own K/V at p0+i, the cache is left as it is, and the rows' own
 * K/V are written to own_k / own_v ([L][NKV][T][hd]) when given.  ``order`` (0..3) is the summation
 * order of every sum (tree_sum).  emit[j] (n_emit rows) selects
 * the rows whose logits are written to logits ([n_emit][vocab]).  Returns 0, or -1 on bad
 * arguments. */
int qf_forward(const QfModel* m, const int* tokens, int T, int p0, int given_cache, const int* emit, int n_emit,
               float* logits, bf16* own_k, bf16* own_v, int order) {
  const int H = m->hidden, I = m->inter, NQ = m->nq, NKV = m->nkv, HD = m->hd, GQ = NQ / NKV;
  const int QS = NQ * HD, KVS = NKV * HD;
  if (T < 1 || p0 < 0 || p0 + T > m->max_seq || n_emit < 0 || NQ % NKV || order < 0 || order > 3) return -1;
  g_order = order;
  for (int t = 0; t < T; t++)
    if (tokens[t] < 0 || tokens[t] >= m->vocab) return -1;
  for (int j = 0; j < n_emit; j++)
    if (emit[j] < 0 || emit[j] >= T) return -1;
  const int HP = pow2_at_least(H > I ? H : I);
  float* x = (float*)malloc(sizeof(float) * (size_t)T * H);     /* residual stream, bf16 values */
  float* nrm = (float*)malloc(sizeof(float) * (size_t)T * H);
  bf16* nb = (bf16*)malloc(sizeof(bf16) * (size_t)T * (H > I ? H : I));
  float* q = (float*)malloc(sizeof(float) * (size_t)T * QS);
  float* k = (float*)malloc(sizeof(float) * (size_t)T * KVS);
  float* v = (float*)malloc(sizeof(float) * (size_t)T * KVS);
  bf16* qb = (bf16*)malloc(sizeof(bf16) * (size_t)T * QS);
  bf16* kb = (bf16*)malloc(sizeof(bf16) * (size_t)T * KVS);
  bf16* vb = (bf16*)malloc(sizeof(bf16) * (size_t)T * KVS);
  float* att = (float*)malloc(sizeof(float) * (size_t)T * QS);
  bf16* attb = (bf16*)malloc(sizeof(bf16) * (size_t)T * QS);
  float* o = (float*)malloc(sizeof(float) * (size_t)T * H);
  float* g = (float*)malloc(sizeof(float) * (size_t)T * I);
  float* u = (float*)malloc(sizeof(float) * (size_t)T * I);
  float* buf = (float*)malloc(sizeof(float) * (size_t)HP);
  for (int t = 0; t < T; t++)
    for (int i = 0; i < H; i++) x[(size_t)t * H + i] = bf(m->embed[(size_t)tokens[t] * H + i]);
  const size_t lstride = (size_t)NKV * m->max_seq * HD;
  for (int L = 0; L < m->num_layers; L++) {
    const bf16* const* w = m->layers + 11 * L;
    for (int t = 0; t < T; t++) rms_norm(x + (size_t)t * H, w[0], H, m->eps, nrm + (size_t)t * H, buf);
    to_bf16_bits(nrm, nb, (size_t)T * H);
    linear(nb, T, w[1], QS, H, q, QS);
    linear(nb, T, w[2], KVS, H, k, KVS);
    linear(nb, T, w[3], KVS, H, v, KVS);
    /* q/k head norms, RoPE */
    for (int t = 0; t < T; t++) {
      const int pos = p0 + t;
      const bf16* cr = m->cos_t + (size_t)pos * HD;
      const bf16* sr = m->sin_t + (size_t)pos * HD;
      for (int hh = 0; hh < NQ + NKV; hh++) {
        float* src = hh < NQ ? q + (size_t)t * QS + (size_t)hh * HD : k + (size_t)t * KVS + (size_t)(hh - NQ) * HD;
        const bf16* wn = hh < NQ ? w[4] : w[5];
        float n[512], y[512];
        rms_norm(src, wn, HD, m->eps, n, buf);
        const int half = HD / 2;
        for (int d = 0; d < HD; d++) {
          const float rot = d < half ? -n[d + half] : n[d - half];
          y[d] = rf(rf(n[d] * bf(cr[d])) + rf(rot * bf(sr[d])));
        }
        memcpy(src, y, sizeof(float) * HD);
      }
    }
    to_bf16_bits(q, qb, (size_t)T * QS);
    to_bf16_bits(k, kb, (size_t)T * KVS);
    to_bf16_bits(v, vb, (size_t)T * KVS);
    bf16* kcl = m->k_cache + (size_t)L * lstride;
    bf16* vcl = m->v_cache + (size_t)L * lstride;
    if (!given_cache) {
      for (int t = 0; t < T; t++)
        for (int g2 = 0; g2 < NKV; g2++) {
          memcpy(kcl + ((size_t)g2 * m->max_seq + p0 + t) * HD, kb + (size_t)t * KVS + (size_t)g2 * HD, 2 * HD);
          memcpy(vcl + ((size_t)g2 * m->max_seq + p0 + t) * HD, vb + (size_t)t * KVS + (size_t)g2 * HD, 2 * HD);
        }
    } else if (own_k && own_v) {
      for (int g2 = 0; g2 < NKV; g2++)
        for (int t = 0; t < T; t++) {
          memcpy(own_k + (((size_t)L * NKV + g2) * T + t) * HD, kb + (size_t)t * KVS + (size_t)g2 * HD, 2 * HD);
          memcpy(own_v + (((size_t)L * NKV + g2) * T + t) * HD, vb + (size_t)t * KVS + (size_t)g2 * HD, 2 * HD);
        }
    }
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int t = 0; t < T; t++)
      for (int g2 = 0; g2 < NKV; g2++) {
        const bf16* kc = kcl + (size_t)g2 * m->max_seq * HD;
        const bf16* vc = vcl + (size_t)g2 * m->max_seq * HD;
        attend(m, qb + (size_t)t * QS + (size_t)g2 * GQ * HD, GQ, kc, vc, kb + (size_t)t * KVS + (size_t)g2 * HD,
               vb + (size_t)t * KVS + (size_t)g2 * HD, p0 + t, att + (size_t)t * QS + (size_t)g2 * GQ * HD);
      }
    to_bf16_bits(att, attb, (size_t)T * QS);
    linear(attb, T, w[6], H, QS, o, H);
    for (size_t i = 0; i < (size_t)T * H; i++) x[i] = rf(x[i] + o[i]);
    for (int t = 0; t < T; t++) rms_norm(x + (size_t)t * H, w[7], H, m->eps, nrm + (size_t)t * H, buf);
    to_bf16_bits(nrm, nb, (size_t)T * H);
    linear(nb, T, w[8], I, H, g, I);
    linear(nb, T, w[9], I, H, u, I);
    for (size_t i = 0; i < (size_t)T * I; i++) {
      const float sg = rf(g[i] / (1.0f + exp_f(-g[i])));
      nb[i] = rbf(sg * u[i]);
    }
    linear(nb, T, w[10], H, I, o, H);
    for (size_t i = 0; i < (size_t)T * H; i++) x[i] = rf(x[i] + o[i]);
  }
  if (n_emit > 0) {
    for (int j = 0; j < n_emit; j++) rms_norm(x + (size_t)emit[j] * H, m->final_norm, H, m->eps, nrm + (size_t)j * H, buf);
    to_bf16_bits(nrm, nb, (size_t)n_emit * H);
    lm_logits(m, nb, n_emit, logits);
  }
  free(buf); free(u); free(g); free(o); free(attb); free(att); free(vb); free(kb); free(qb);
  free(v); free(k); free(q); free(nb); free(nrm); free(x);
  return 0;
}

/* The same tree sum, exported so that tests can pin its order. */
float qf_tree_sum(const float* x, int n, float* work, int order) {
  memcpy(work, x, sizeof(float) * (size_t)n);
  g_order = order;
  return tree_sum(work, n);
}
