/*
 * flock_oracle.c -- CPU restatement of flock's strict-f32 attention references.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker: it is loaded by tests/,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by nothing
 * else. The product path (flock_amd/, libflock_attn.so) never links or calls it.
 *
 * Every function restates one function of the reference's TypeScript oracle,
 * rounding point for rounding point. The reference evaluates in JS doubles and
 * rounds to f32 with Math.fround at explicit points; this file does the same
 * with (double) arithmetic and (float) casts:
 *
 *   fr(x)            Math.fround(x)                      -> (float)(x)
 *   fma32(a, b, c)   Math.fround(a*b + c), kernels/lib.ts:169-171
 *                    -> (float)((double)a*b + (double)c). The f64 product of
 *                    two floats is exact; the sum then rounds to f64 and again
 *                    to f32 (a double rounding, NOT always identical to fmaf).
 *
 * Transcendentals (exp, cos, sin, sqrt, pow) are evaluated in double with libm
 * and rounded to f32 where the reference rounds. V8's Math.* may differ from
 * glibc in the last f64 ulp; that survives the f32 rounding only rarely.
 *
 * Compile WITHOUT -ffast-math and with -ffp-contract=off (see oracle/Makefile).
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   flko_rmsnorm        zero-vector KAT (test_ops.ts:167-181); f64 closed form;
 *                       tree order vs a serial-sum mutant on crafted inputs.
 *   flko_rope           planted pairing KAT (test_ops.ts:229-263) for both
 *                       pairings; f64 closed-form rotation; norm preservation.
 *   flko_rope_inv_freq  numpy float64 1/base**(2j/d), rounded to f32.
 *   flko_attn           GQA planted KAT (test_ops.ts:357-392); f64 closed-form
 *                       softmax(q k^T / sqrt d) v; one-key and uniform-key
 *                       special cases.
 *   flko_attn_prefill   f64 closed form with causal bound; last query == attn
 *                       (test_head.ts:321-351); causality bit-identity
 *                       (test_head.ts:353-389).
 *   flko_argmax         lowest-index tie rule on constructed ties.
 *   error metrics       hand-computed values.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float fr(double x) { return (float)x; }

/* kernels/lib.ts:169-171 */
static inline float fma32(float a, float b, float c) {
  return (float)((double)a * (double)b + (double)c);
}

/* kernels/ops_ref.ts:176-182 (treeSum) and head_ref.ts:186-192 (treeReduce with
 * f32 add). Pairwise tree over `len` (a power of two) entries, in place. */
static float tree_sum(float* buf, int len) {
  for (int stride = len >> 1; stride > 0; stride >>= 1)
    for (int i = 0; i < stride; i++) buf[i] = fr((double)buf[i] + (double)buf[i + stride]);
  return buf[0];
}

/* head_ref.ts:186-192 with Math.max. */
static float tree_max(float* buf, int len) {
  for (int stride = len >> 1; stride > 0; stride >>= 1)
    for (int i = 0; i < stride; i++) buf[i] = buf[i] > buf[i + stride] ? buf[i] : buf[i + stride];
  return buf[0];
}

/*
 * rmsnormRef, kernels/ops_ref.ts:20-49.
 * x, o: [n_vecs][n]; g: [n]. `wg` strided fma32 partials, then a pairwise tree.
 * scale = fr(1 / sqrt(fr(fr(sum / n) + eps))) -- one rounding of 1/sqrt.
 * o = fr(fr(x * scale) * g).
 */
void flko_rmsnorm(const float* x, const float* g, float* o, int n, int n_vecs,
                  double eps, int wg) {
  float* part = (float*)malloc(sizeof(float) * (size_t)wg);
  for (int v = 0; v < n_vecs; v++) {
    const float* xv = x + (size_t)v * n;
    float* ov = o + (size_t)v * n;
    for (int t = 0; t < wg; t++) {
      float acc = 0.0f;
      for (int i = t; i < n; i += wg) acc = fma32(xv[i], xv[i], acc);
      part[t] = acc;
    }
    const float sum = tree_sum(part, wg);
    const float mean = fr((double)sum / (double)n);
    const float scale = fr(1.0 / sqrt((double)fr((double)mean + eps)));
    for (int i = 0; i < n; i++) ov[i] = fr((double)fr((double)xv[i] * scale) * (double)g[i]);
  }
  free(part);
}

/*
 * ropeRef, kernels/ops_ref.ts:65-92. In place on x: [n_tokens][n_heads][head_dim].
 * pairing 0 = "neox" (j, j + d/2), 1 = "norm" (2j, 2j + 1).
 * theta = fr((pos0 + t) * inv_freq[j]); c, s = fr(cos/sin(theta));
 * x[ia] = fr(-b*s + fr(a*c)); x[ib] = fr(b*c + fr(a*s)).
 */
void flko_rope(float* x, int n_tokens, int n_heads, int head_dim, int pos0,
               const float* inv_freq, int pairing) {
  const int half = head_dim / 2;
  for (int t = 0; t < n_tokens; t++)
    for (int h = 0; h < n_heads; h++)
      for (int j = 0; j < half; j++) {
        const float theta = fr((double)(pos0 + t) * (double)inv_freq[j]);
        const float c = fr(cos((double)theta)), s = fr(sin((double)theta));
        const size_t base = ((size_t)t * n_heads + h) * head_dim;
        const size_t ia = base + (pairing == 1 ? 2 * j : j);
        const size_t ib = base + (pairing == 1 ? 2 * j + 1 : j + half);
        const float a = x[ia], b = x[ib];
        x[ia] = fr(-(double)b * (double)s + (double)fr((double)a * (double)c));
        x[ib] = fr((double)b * (double)c + (double)fr((double)a * (double)s));
      }
}

/* ropeInvFreq, kernels/ops_ref.ts:95-100 (same as layer.ts:180-186). */
void flko_rope_inv_freq(int head_dim, double base, float* out) {
  for (int j = 0; j < head_dim / 2; j++)
    out[j] = fr(1.0 / pow(base, (2.0 * j) / (double)head_dim));
}

/*
 * attnRef, kernels/ops_ref.ts:135-174. Decode GQA attention for one query.
 * q: [H][d]; k, v: [n_keys][Hkv][d]; o: [H][d]. Head h reads kv head
 * h / (H / Hkv). Serial fma32 dot, fr(acc * scale), max, fr(exp(fr(s - max))),
 * serial f32 sum, inv = fr(1 / sum), serial fma32 P.V, fr(acc * inv).
 * Heads are independent, so they run in parallel; each head's arithmetic is
 * the serial order above.
 */
void flko_attn(const float* q, const float* k, const float* v, float* o, int H, int Hkv,
               int d, int n_keys) {
  const int group = H / Hkv;
  const float scale = fr(1.0 / sqrt((double)d));
#pragma omp parallel for schedule(static)
  for (int h = 0; h < H; h++) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(n_keys > 0 ? n_keys : 1));
    const int kvh = h / group;
    for (int t = 0; t < n_keys; t++) {
      float acc = 0.0f;
      const float* kr = k + ((size_t)t * Hkv + kvh) * d;
      for (int i = 0; i < d; i++) acc = fma32(q[(size_t)h * d + i], kr[i], acc);
      scores[t] = fr((double)acc * scale);
    }
    double mx = -INFINITY;
    for (int t = 0; t < n_keys; t++) mx = fmax(mx, (double)scores[t]);
    float sum = 0.0f;
    for (int t = 0; t < n_keys; t++) {
      scores[t] = fr(exp((double)fr((double)scores[t] - mx)));
      sum = fr((double)sum + (double)scores[t]);
    }
    const float inv = fr(1.0 / (double)sum);
    /* ops_ref.ts:166-172 walks t serially for each channel i. The loops are
     * interchanged here (one accumulator per channel, keys outer) for cache
     * locality; every acc[i] still sees the same fma32 sequence t = 0, 1, ... */
    float* acc = (float*)calloc((size_t)d, sizeof(float));
    for (int t = 0; t < n_keys; t++) {
      const float* vr = v + ((size_t)t * Hkv + kvh) * d;
      const float p = scores[t];
      for (int i = 0; i < d; i++) acc[i] = fma32(p, vr[i], acc[i]);
    }
    for (int i = 0; i < d; i++) o[(size_t)h * d + i] = fr((double)acc[i] * inv);
    free(acc);
    free(scores);
  }
}

/*
 * attnPrefillRef, kernels/head_ref.ts:99-183. Causal GQA over n_q queries with
 * the streaming (online) softmax, tile by tile. q, o: [n_q][H][d]; k, v:
 * [>= pos0 + n_q][Hkv][d]. Query i attends to keys 0 .. pos0 + i.
 * Per tile: serial fma32 dots, fr(s * scale); tile max by strided-then-tree
 * reduction over `wg` partials; corr = fr(exp(fr(m - mNew))); e = fr(exp(fr(s -
 * mNew))) with per-partial f32 sums then a tree; acc = fr(acc * corr) followed
 * by a serial fma32 chain; l = fma32(l, corr, tileSum); o = fr(acc / l).
 * (query, head) pairs are independent and run in parallel.
 */
void flko_attn_prefill(const float* q, const float* k, const float* v, float* o, int H,
                       int Hkv, int d, int n_q, int pos0, int tile, int wg) {
  const int group = H / Hkv;
  const float scale = fr(1.0 / sqrt((double)d));
#pragma omp parallel for schedule(dynamic, 1)
  for (int pair = 0; pair < n_q * H; pair++) {
    const int qi = pair / H, h = pair % H;
    float* tile_s = (float*)malloc(sizeof(float) * (size_t)tile);
    float* part = (float*)malloc(sizeof(float) * (size_t)wg);
    float* acc = (float*)malloc(sizeof(float) * (size_t)d);
    const int kvh = h / group;
    const size_t qbase = ((size_t)qi * H + h) * d;
    const int n_keys = pos0 + qi + 1;
    double m = -INFINITY;
    float l = 0.0f;
    for (int i = 0; i < d; i++) acc[i] = 0.0f;
    for (int base = 0; base < n_keys; base += tile) {
      const int n_this = tile < n_keys - base ? tile : n_keys - base;
      for (int j = 0; j < n_this; j++) {
        const float* kr = k + ((size_t)(base + j) * Hkv + kvh) * d;
        float s = 0.0f;
        for (int i = 0; i < d; i++) s = fma32(q[qbase + i], kr[i], s);
        tile_s[j] = fr((double)s * scale);
      }
      for (int t = 0; t < wg; t++) {
        float tm = -INFINITY;
        for (int j = t; j < n_this; j += wg) tm = tm > tile_s[j] ? tm : tile_s[j];
        part[t] = tm;
      }
      const float tile_max = tree_max(part, wg);
      const double m_new = fmax(m, (double)tile_max);
      const float corr = fr(exp((double)fr(m - m_new)));
      for (int t = 0; t < wg; t++) {
        float ts = 0.0f;
        for (int j = t; j < n_this; j += wg) {
          const float e = fr(exp((double)fr((double)tile_s[j] - m_new)));
          tile_s[j] = e;
          ts = fr((double)ts + (double)e);
        }
        part[t] = ts;
      }
      const float tile_sum = tree_sum(part, wg);
      for (int i = 0; i < d; i++) {
        float a = fr((double)acc[i] * (double)corr);
        for (int j = 0; j < n_this; j++)
          a = fma32(tile_s[j], v[((size_t)(base + j) * Hkv + kvh) * d + i], a);
        acc[i] = a;
      }
      l = fma32(l, corr, tile_sum);
      m = m_new;
    }
    for (int i = 0; i < d; i++) o[qbase + i] = fr((double)acc[i] / (double)l);
    free(tile_s);
    free(part);
    free(acc);
  }
}

/* argmaxRef, kernels/head_ref.ts:65-74: lowest index wins ties. */
int flko_argmax(const float* x, int n) {
  int bi = 0;
  float bv = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > bv) {
      bv = x[i];
      bi = i;
    }
  return bi;
}

/* relErr, kernels/ops_ref.ts:185-191. */
double flko_rel_err(const float* a, const float* b, int64_t n, double floor_) {
  double worst = 0.0;
  for (int64_t i = 0; i < n; i++) {
    const double den = fmax(floor_, fabs((double)b[i]));
    worst = fmax(worst, fabs((double)a[i] - (double)b[i]) / den);
  }
  return worst;
}

/* absErrScaled, kernels/ops_ref.ts:206-210. */
double flko_abs_err_scaled(const float* a, const float* b, int64_t n, double scale) {
  double worst = 0.0;
  for (int64_t i = 0; i < n; i++) worst = fmax(worst, fabs((double)a[i] - (double)b[i]));
  return worst / scale;
}

/* amax, kernels/ops_ref.ts:213-217. */
double flko_amax(const float* a, int64_t n) {
  double m = 0.0;
  for (int64_t i = 0; i < n; i++) m = fmax(m, fabs((double)a[i]));
  return m;
}

/*
 * Attention slice of layerForwardRef, kernels/layer_ref.ts:46-70 (the matvecs
 * and FFN are outside this path): per-head rmsnorm of q and k, RoPE at `pos`,
 * append (k_normed_roped, v_raw) to the cache at row `pos`, then attnRef over
 * pos + 1 keys. kcache/vcache: [>= pos + 1][Hkv][d], rows < pos already filled.
 * qn_out receives the normed+roped q (the attention input).
 */
void flko_layer_attn_decode(const float* q_raw, const float* k_raw, const float* v_raw,
                            const float* gq, const float* gk, const float* inv_freq,
                            double eps, int pairing, float* kcache, float* vcache,
                            float* qn_out, float* o, int pos, int H, int Hkv, int d) {
  float* kn = (float*)malloc(sizeof(float) * (size_t)Hkv * d);
  flko_rmsnorm(q_raw, gq, qn_out, d, H, eps, 128);
  flko_rmsnorm(k_raw, gk, kn, d, Hkv, eps, 128);
  flko_rope(qn_out, 1, H, d, pos, inv_freq, pairing);
  flko_rope(kn, 1, Hkv, d, pos, inv_freq, pairing);
  memcpy(kcache + (size_t)pos * Hkv * d, kn, sizeof(float) * (size_t)Hkv * d);
  memcpy(vcache + (size_t)pos * Hkv * d, v_raw, sizeof(float) * (size_t)Hkv * d);
  flko_attn(qn_out, kcache, vcache, o, H, Hkv, d, pos + 1);
  free(kn);
}

/*
 * Attention slice of layerPrefillRef, kernels/layer_ref.ts:137-165: n tokens at
 * positions pos0 .. pos0 + n - 1. Norms over n*H and n*Hkv head vectors, RoPE
 * with token i at pos0 + i, append n rows at pos0, then attnPrefillRef.
 */
void flko_layer_attn_prefill(const float* q_raw, const float* k_raw, const float* v_raw,
                             const float* gq, const float* gk, const float* inv_freq,
                             double eps, int pairing, float* kcache, float* vcache,
                             float* qn_out, float* o, int n, int pos0, int H, int Hkv,
                             int d) {
  float* kn = (float*)malloc(sizeof(float) * (size_t)n * Hkv * d);
  flko_rmsnorm(q_raw, gq, qn_out, d, n * H, eps, 128);
  flko_rmsnorm(k_raw, gk, kn, d, n * Hkv, eps, 128);
  flko_rope(qn_out, n, H, d, pos0, inv_freq, pairing);
  flko_rope(kn, n, Hkv, d, pos0, inv_freq, pairing);
  memcpy(kcache + (size_t)pos0 * Hkv * d, kn, sizeof(float) * (size_t)n * Hkv * d);
  memcpy(vcache + (size_t)pos0 * Hkv * d, v_raw, sizeof(float) * (size_t)n * Hkv * d);
  flko_attn_prefill(qn_out, kcache, vcache, o, H, Hkv, d, n, pos0, 64, 128);
  free(kn);
}

/* Threads the parallel loops above use (1 unless built with OpenMP). */
int flko_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}
