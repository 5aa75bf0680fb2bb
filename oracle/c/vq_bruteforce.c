/*
 * fp64 brute-force checker for the residual-VQ hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle/jointkv_oracle.py).  Independent of
 * the torch restatement: distances are summed directly as sum_i (r_i-c_i)^2
 * in double precision, residuals are carried in double, and ties go to the
 * lowest index.  Used to pin the oracle's codes, margins and the closed-form
 * straight-through gradient.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/*
 * Greedy residual VQ on one problem.
 *   x       [N][D]   states (already in search coordinates)
 *   tables  [S][K][D] codewords (search coordinates)
 *   codes   [N][S]   out: chosen index per stage
 *   d1, d2  [N][S]   out: best and second-best squared distance per stage
 *                    (d2 = INFINITY when K == 1)
 */
void bf_rvq_encode(const double* x, const double* tables, int64_t N, int64_t S, int64_t K,
                   int64_t D, int32_t* codes, double* d1, double* d2) {
  double r[4096];
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t i = 0; i < D; ++i) r[i] = x[n * D + i];
    for (int64_t s = 0; s < S; ++s) {
      const double* tab = tables + s * K * D;
      double best = INFINITY, second = INFINITY;
      int64_t bk = 0;
      for (int64_t k = 0; k < K; ++k) {
        double acc = 0.0;
        for (int64_t i = 0; i < D; ++i) {
          double diff = r[i] - tab[k * D + i];
          acc += diff * diff;
        }
        if (acc < best) {
          second = best;
          best = acc;
          bk = k;
        } else if (acc < second) {
          second = acc;
        }
      }
      codes[n * S + s] = (int32_t)bk;
      d1[n * S + s] = best;
      d2[n * S + s] = second;
      for (int64_t i = 0; i < D; ++i) r[i] -= tab[bk * D + i];
    }
  }
}

/*
 * Straight-through codebook gradient of one problem with one exit at depth
 * `depth`:  grad[s][k][:] += g[n][:] for every n and s < depth with
 * codes[n][s] == k.  grad [S][K][D] must be zeroed by the caller.
 */
void bf_scatter(const double* g, const int32_t* codes, int64_t N, int64_t S, int64_t K, int64_t D,
                int64_t depth, double* grad) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t s = 0; s < S && s < depth; ++s) {
      int64_t k = codes[n * S + s];
      if (k < 0 || k >= K) continue;
      for (int64_t i = 0; i < D; ++i) grad[(s * K + k) * D + i] += g[n * D + i];
    }
}

/* Softmax attention of one query row over T keys in fp64. */
void bf_attention_row(const double* q, const double* k, const double* v, int64_t T, int64_t D,
                      double* out) {
  double m = -INFINITY;
  double scale = 1.0 / sqrt((double)D);
  for (int64_t t = 0; t < T; ++t) {
    double s = 0.0;
    for (int64_t i = 0; i < D; ++i) s += q[i] * k[t * D + i];
    s *= scale;
    if (s > m) m = s;
  }
  double l = 0.0;
  memset(out, 0, sizeof(double) * (size_t)D);
  for (int64_t t = 0; t < T; ++t) {
    double s = 0.0;
    for (int64_t i = 0; i < D; ++i) s += q[i] * k[t * D + i];
    double p = exp(s * scale - m);
    l += p;
    for (int64_t i = 0; i < D; ++i) out[i] += p * v[t * D + i];
  }
  for (int64_t i = 0; i < D; ++i) out[i] /= l;
}
