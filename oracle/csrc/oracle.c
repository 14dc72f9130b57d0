/*
 * CPU oracle helpers in C (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).
 *
 *  - oracle_hist_exact: exact integer histogram (restates
 *    warpgbm/cuda/histogram_kernel.cu:33-59 with integer sums) for inputs
 *    too large for the numpy restatement to finish quickly.
 *  - oracle_expf / oracle_softmax_residual / oracle_softmax_rows: the softmax
 *    of warpgbm/metrics.py:12-15 and the gradients of warpgbm/core.py:186-214,
 *    with an exp written from the mathematics (Cody-Waite reduction by ln 2,
 *    degree-7 Taylor polynomial in Horner form with fmaf, ldexpf scaling)
 *    so that results are reproducible to the bit on any IEEE machine.
 *
 *  - oracle_quantile_edges_matrix / oracle_bin_matrix / oracle_predict_tables:
 *    the quantile edges of core.py:527-533 (torch.quantile over each sorted
 *    column), binner.cu:12-25 and predict.cu:13-44, for full-size checks.
 *
 * The loops over independent features / columns / rows run on OpenMP
 * threads; every output element is produced by one thread in a fixed order,
 * so results do not depend on the thread count.
 *
 * Built by oracle/build.py with gcc -O2 -fopenmp -ffp-contract=off.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* threads the OpenMP loops below use (OMP_NUM_THREADS, else all cores) */
int oracle_num_threads(void) { return omp_get_max_threads(); }

/* rows [p0, p1) of the call into Q, C restricted to features [f0, f1) */
static void hist_rows(const int8_t* codes, int64_t stride, const int32_t* q, const int32_t* rows,
                      int64_t p0, int64_t p1, const int32_t* feats, int32_t f0, int32_t f1,
                      const int32_t* era, int32_t num_eras, int32_t num_bins, int64_t per_era,
                      int64_t* Q, int64_t* C) {
  for (int64_t p = p0; p < p1; ++p) {
    const int64_t s = rows ? rows[p] : p;
    const int e = num_eras == 1 ? 0 : era[s];
    if (e < 0 || e >= num_eras) continue;
    const int8_t* row = codes + s * stride;
    const int64_t qs = q[s];
    int64_t* Qe = Q + e * per_era;
    int64_t* Ce = C + e * per_era;
    for (int32_t f = f0; f < f1; ++f) {
      const int b = row[feats ? feats[f] : f];
      if (b < 0 || b >= num_bins) continue;
      Qe[(int64_t)f * num_bins + b] += qs;
      Ce[(int64_t)f * num_bins + b] += 1;
    }
  }
}

void oracle_hist_exact(const int8_t* codes, int64_t stride, const int32_t* q,
                       const int32_t* rows, int64_t n_rows, const int32_t* feats,
                       int32_t n_feats, const int32_t* era, int32_t num_eras, int32_t num_bins,
                       int64_t* Q, int64_t* C) {
  const int64_t per_era = (int64_t)n_feats * num_bins;
  const int64_t words = per_era * num_eras;
  const int nt = omp_get_max_threads();
  memset(Q, 0, sizeof(int64_t) * words);
  memset(C, 0, sizeof(int64_t) * words);
  if (nt > 1 && words * 16 <= (int64_t)8 << 20 && n_rows >= 4096) {
    /* small histograms: rows split over the threads, each into a private
     * copy, then the copies added (integer sums: the order is immaterial) */
    int64_t* priv = (int64_t*)calloc((size_t)nt * 2 * words, sizeof(int64_t));
    if (priv) {
#pragma omp parallel num_threads(nt)
      {
        const int t = omp_get_thread_num();
        const int64_t p0 = n_rows * t / nt, p1 = n_rows * (t + 1) / nt;
        int64_t* Qt = priv + (int64_t)t * 2 * words;
        hist_rows(codes, stride, q, rows, p0, p1, feats, 0, n_feats, era, num_eras, num_bins,
                  per_era, Qt, Qt + words);
      }
#pragma omp parallel for schedule(static)
      for (int64_t w = 0; w < words; ++w) {
        int64_t a = 0, c = 0;
        for (int t = 0; t < nt; ++t) {
          a += priv[(int64_t)t * 2 * words + w];
          c += priv[(int64_t)t * 2 * words + words + w];
        }
        Q[w] = a;
        C[w] = c;
      }
      free(priv);
      return;
    }
  }
  /* large histograms: each thread owns one contiguous range of features,
   * reads those bytes of every row and is the only writer of their bins */
#pragma omp parallel num_threads(nt)
  {
    const int t = omp_get_thread_num();
    const int32_t f0 = (int32_t)((int64_t)n_feats * t / nt);
    const int32_t f1 = (int32_t)((int64_t)n_feats * (t + 1) / nt);
    if (f1 > f0)
      hist_rows(codes, stride, q, rows, 0, n_rows, feats, f0, f1, era, num_eras, num_bins,
                per_era, Q, C);
  }
}

/* torch.quantile (linear) edges from an ascending-sorted column s[0..n-1]:
 * rank = q*(n-1) in float32, lo/hi = floor/ceil, w = rank - lo, d = s[hi]-s[lo],
 * edge = w < 0.5 ? fma(w, d, s[lo]) : fma(w - 1, d, s[hi]); NaN column -> NaN */
void oracle_quantile_sorted(const float* s, int64_t n, const float* q, int32_t nq, float* out) {
  const int64_t last = n - 1;
  const int has_nan = s[last] != s[last];
  for (int32_t j = 0; j < nq; ++j) {
    const float rank = has_nan ? (float)last : q[j] * (float)last;
    const int64_t lo = (int64_t)rank;
    const int64_t hi = (int64_t)ceilf(rank);
    const float w = rank - (float)lo;
    const float a = s[lo], b = s[hi], d = b - a;
    out[j] = w < 0.5f ? fmaf(w, d, a) : fmaf(w - 1.0f, d, b);
  }
}

float oracle_expf(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.5f) return INFINITY;
  /* ln 2 split into a 15-significant-bit head (k * head is exact for the
   * |k| <= 150 used here) and the remaining tail */
  const float log2e = 1.44269504088896341f;
  const float head = 0.693145751953125f;
  const float tail = 1.42860682030941723212e-6f;
  const float k = rintf(x * log2e);
  float r = fmaf(k, -head, x);
  r = fmaf(k, -tail, r);
  /* e^r = sum_{i<=7} r^i / i!  on |r| <= ln2/2 */
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

void oracle_expf_array(const float* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_expf(x[i]);
}

/* r[k * n + i] = -(softmax(logits[i, :])_k - [k == label_i]) */
void oracle_softmax_residual(const float* logits, const int32_t* labels, int64_t n, int32_t K,
                             float* r) {
  for (int64_t i = 0; i < n; ++i) {
    const float* x = logits + i * K;
    float m = x[0];
    for (int k = 1; k < K; ++k) m = x[k] > m ? x[k] : m;
    float s = 0.0f;
    for (int k = 0; k < K; ++k) s = s + oracle_expf(x[k] - m);
    for (int k = 0; k < K; ++k) {
      const float p = oracle_expf(x[k] - m) / s;
      const float g = p - (k == labels[i] ? 1.0f : 0.0f);
      r[(int64_t)k * n + i] = -g;
    }
  }
}

void oracle_softmax_rows(float* x, int64_t n, int32_t K) {
  for (int64_t i = 0; i < n; ++i) {
    float* v = x + i * K;
    float m = v[0];
    for (int k = 1; k < K; ++k) m = v[k] > m ? v[k] : m;
    float s = 0.0f;
    for (int k = 0; k < K; ++k) {
      v[k] = oracle_expf(v[k] - m);
      s = s + v[k];
    }
    for (int k = 0; k < K; ++k) v[k] = v[k] / s;
  }
}

/* ---- full-size helpers ------------------------------------------------- */

/* order-preserving key of a float (NaN above +inf, -0.0 just below +0.0) */
static inline uint32_t f32_key(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if (x != x) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ascending sort of n floats by their key (LSD radix, 4 passes of 8 bits) */
static void sort_f32(float* a, float* tmp, int64_t n) {
  for (int pass = 0; pass < 4; ++pass) {
    int64_t cnt[257];
    memset(cnt, 0, sizeof(cnt));
    const int sh = pass * 8;
    for (int64_t i = 0; i < n; ++i) cnt[((f32_key(a[i]) >> sh) & 255u) + 1]++;
    for (int k = 0; k < 256; ++k) cnt[k + 1] += cnt[k];
    for (int64_t i = 0; i < n; ++i) tmp[cnt[(f32_key(a[i]) >> sh) & 255u]++] = a[i];
    memcpy(a, tmp, sizeof(float) * n);
  }
}

/* edges[f, j] = torch.quantile(X[:, f], q[j]) for every column f of the
 * row-major X [n, ldx]: the column sorted (NaN last), then the linear
 * interpolation of oracle_quantile_sorted */
void oracle_quantile_edges_matrix(const float* X, int64_t n, int64_t F, int64_t ldx,
                                  const float* q, int32_t nq, float* edges) {
  if (n <= 0) {
    for (int64_t k = 0; k < F * nq; ++k) edges[k] = NAN;
    return;
  }
#pragma omp parallel
  {
    float* col = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
    float* tmp = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
#pragma omp for schedule(dynamic, 1)
    for (int64_t f = 0; f < F; ++f) {
      for (int64_t i = 0; i < n; ++i) col[i] = X[i * ldx + f];
      sort_f32(col, tmp, n);
      oracle_quantile_sorted(col, n, q, nq, edges + f * nq);
    }
    free(col);
    free(tmp);
  }
}

/* codes[i, f] = number of leading edges e[f, j] with x >= e (binner.cu:17-23:
 * the scan stops at the first edge x is below; NaN -> 0) */
void oracle_bin_matrix(const float* X, int64_t n, int64_t F, int64_t ldx, const float* edges,
                       int32_t ne, int8_t* codes, int64_t ldc) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    for (int64_t f = 0; f < F; ++f) {
      const float x = X[i * ldx + f];
      const float* e = edges + f * ne;
      int b = 0;
      while (b < ne && x >= e[b]) ++b;
      codes[i * ldc + f] = (int8_t)b;
    }
  }
}

/* out[i, cls[t]] = out[i, cls[t]] + lr * leaf_t(i) for t = 0..T-1 in order,
 * leaf_t(i) found by walking the pre-order table tables[t] [M, 6]
 * (feature, bin, left, right, is_leaf, value): while is_leaf <= 0.5,
 * code <= bin goes left (predict.cu:23-44) */
void oracle_predict_tables(const int8_t* codes, int64_t n, int64_t ldc, const float* tables,
                           int32_t T, int32_t M, const int32_t* cls, int32_t K, float lr,
                           float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int8_t* row = codes + i * ldc;
    for (int32_t t = 0; t < T; ++t) {
      const float* tb = tables + (int64_t)t * M * 6;
      int32_t nd = 0;
      int guard = 0;
      while (tb[nd * 6 + 4] <= 0.5f && guard++ <= M) {
        const int32_t f = (int32_t)tb[nd * 6 + 0];
        const int32_t b = (int32_t)tb[nd * 6 + 1];
        nd = (int32_t)(row[f] <= b ? tb[nd * 6 + 2] : tb[nd * 6 + 3]);
      }
      const float v = lr * tb[nd * 6 + 5];
      float* o = out + i * K + (cls ? cls[t] : 0);
      *o = *o + v;
    }
  }
}

/* Per-era gain and direction of best_split_kernel.cu:25-54 (the restatement
 * of ops.split_scan) straight from exact histograms: G = float(ldexp(Q, -s)),
 * H = float(C), then sequential float32 totals and prefix; gain/dir are
 * [EF, B-1] for the EF (era, feature) rows of Q, C [EF, B]. */
void oracle_split_scan_q(const int64_t* Q, const int64_t* Cn, int64_t EF, int32_t B, int32_t F,
                         const int32_t* s_era, float mcw, float eps, float* gain, float* dirn) {
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < EF; ++k) {
    const int32_t s = s_era[k / F]; /* the shift of row k's era */
    const int64_t* q = Q + k * B;
    const int64_t* c = Cn + k * B;
    float Gt = 0.0f, Ht = 0.0f;
    for (int32_t b = 0; b < B; ++b) {
      Gt = Gt + (float)ldexp((double)q[b], -s);
      Ht = Ht + (float)c[b];
    }
    const float tot = (Gt * Gt) / (Ht + eps);
    float GL = 0.0f, HL = 0.0f;
    for (int32_t b = 0; b + 1 < B; ++b) {
      GL = GL + (float)ldexp((double)q[b], -s);
      HL = HL + (float)c[b];
      const float GR = Gt - GL, HR = Ht - HL;
      float g = 0.0f, d = 0.0f;
      if (HL >= mcw && HR >= mcw) {
        const float a = (GL * GL) / (HL + eps);
        const float r = (GR * GR) / (HR + eps);
        g = (a + r) - tot;
        d = GL / (HL + eps) > GR / (HR + eps) ? 1.0f : -1.0f;
      }
      gain[k * (B - 1) + b] = g;
      dirn[k * (B - 1) + b] = d;
    }
  }
}

/* largest |r| of the rows of each era among rows[0..n) (float bits of
 * |r|, as an unsigned compare orders non-negative floats; a NaN compares
 * above every finite value and +inf): out[e] for e < num_eras */
void oracle_era_absmax(const float* r, const int32_t* rows, int64_t n, const int32_t* era,
                       int32_t num_eras, uint32_t* out) {
  memset(out, 0, sizeof(uint32_t) * (size_t)num_eras);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t s = rows[i];
    const int e = era[s];
    if (e < 0 || e >= num_eras) continue;
    uint32_t b;
    memcpy(&b, &r[s], sizeof b);
    b &= 0x7fffffffu;
    if (b > out[e]) out[e] = b;
  }
}
