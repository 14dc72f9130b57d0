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
 * Built by oracle/build.py with gcc -O2 -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

void oracle_hist_exact(const int8_t* codes, int64_t stride, const int32_t* q,
                       const int32_t* rows, int64_t n_rows, const int32_t* feats,
                       int32_t n_feats, const int32_t* era, int32_t num_eras, int32_t num_bins,
                       int64_t* Q, int64_t* C) {
  const int64_t per_era = (int64_t)n_feats * num_bins;
  memset(Q, 0, sizeof(int64_t) * per_era * num_eras);
  memset(C, 0, sizeof(int64_t) * per_era * num_eras);
  for (int64_t p = 0; p < n_rows; ++p) {
    const int64_t s = rows ? rows[p] : p;
    const int e = num_eras == 1 ? 0 : era[s];
    if (e < 0 || e >= num_eras) continue;
    const int8_t* row = codes + s * stride;
    const int64_t qs = q[s];
    int64_t* Qe = Q + e * per_era;
    int64_t* Ce = C + e * per_era;
    for (int32_t f = 0; f < n_feats; ++f) {
      const int b = row[feats ? feats[f] : f];
      if (b < 0 || b >= num_bins) continue;
      Qe[(int64_t)f * num_bins + b] += qs;
      Ce[(int64_t)f * num_bins + b] += 1;
    }
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
