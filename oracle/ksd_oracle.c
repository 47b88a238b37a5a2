/*
 * ksd_oracle.c — CPU restatement of KSDraft's INT8-tier arithmetic, used ONLY as the
 * checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. Nothing
 * in the product (ksdraft_amd/) links or calls it.
 *
 * Plain C, built with gcc -O2 -ffp-contract=off (so a*b+c is two roundings unless
 * written fmaf, which glibc rounds correctly). fp16 values are handled as uint16_t bit
 * patterns with an exact decoder (half_to_float).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* exact fp16 -> fp32 decode (every fp16 value, subnormals included, is an fp32) */
float ksd_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  float f;
  if (exp == 0) {
    f = ldexpf((float)man, -24); /* subnormal: man * 2^-24 */
  } else if (exp == 31) {
    uint32_t bits = 0x7f800000u | (man << 13);
    memcpy(&f, &bits, 4);
  } else {
    uint32_t bits = ((exp + 112u) << 23) | (man << 13);
    memcpy(&f, &bits, 4);
  }
  uint32_t b;
  memcpy(&b, &f, 4);
  b |= sign;
  memcpy(&f, &b, 4);
  return f;
}

/*
 * Exact int32 group partials P_g[m,n] = sum_{k in group g} a[m,k]*w[n,k]
 * (the int32 tl.dot of reference ksdraft/kernels/gemm.py:42). out is (G, M, N).
 */
void ksd_oracle_partials(const int8_t *a, const int8_t *w, int64_t M, int64_t N, int64_t K,
                         int group, int32_t *out) {
  const int64_t G = K / group;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const int8_t *ar = a + m * K;
      const int8_t *wr = w + n * K;
      for (int64_t g = 0; g < G; ++g) {
        int32_t p = 0;
        for (int64_t k = g * group; k < (g + 1) * group; ++k) p += (int32_t)ar[k] * (int32_t)wr[k];
        out[(g * M + m) * N + n] = p;
      }
    }
}

/*
 * W8A8 GEMM in the ordered per-group contract the GPU kernel implements:
 *   acc = 0; for g = 0..G-1: acc = fmaf((float)P_g, sa[m,g]*sw[n,g], acc); y = acc (+ bias[n])
 * Per-group rescale order follows reference ksdraft/kernels/gemm.py:34-45; bias is
 * added in fp32 afterwards as in ksdraft/kernels/linear.py:71-72.
 * rows: optional list of `n_rows` row indices to evaluate (NULL = all M rows); y holds
 * one output row per evaluated row.
 */
void ksd_oracle_gemm_ordered(const int8_t *a, const uint16_t *as, const int8_t *w,
                             const uint16_t *ws, int64_t M, int64_t N, int64_t K, int group,
                             const float *bias, const int64_t *rows, int64_t n_rows, int splits,
                             float *y) {
  const int64_t G = K / group;
  const int64_t R = rows ? n_rows : M;
  if (splits < 1) splits = 1;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t r = 0; r < R; ++r)
    for (int64_t n = 0; n < N; ++n) {
      const int64_t m = rows ? rows[r] : r;
      const int8_t *ar = a + m * K;
      const int8_t *wr = w + n * K;
      float total = 0.0f;
      /* K part q: groups [floor(q G / S), floor((q+1) G / S)), summed from zero in order;
         the parts are added in ascending order */
      for (int q = 0; q < splits; ++q) {
        const int64_t g0 = (int64_t)q * G / splits, g1 = (int64_t)(q + 1) * G / splits;
        float acc = 0.0f;
        for (int64_t g = g0; g < g1; ++g) {
          int32_t p = 0;
          for (int64_t k = g * group; k < (g + 1) * group; ++k) p += (int32_t)ar[k] * (int32_t)wr[k];
          const float s = ksd_half_to_float(as[m * G + g]) * ksd_half_to_float(ws[n * G + g]);
          acc = fmaf((float)p, s, acc);
        }
        total = q == 0 ? acc : total + acc;
      }
      if (bias) total = total + bias[n];
      y[r * N + n] = total;
    }
}

/* ------------------------------------------------------------------ Rosa
 * Longest-suffix match of reference ksdraft/model/rosa.py:40-98, by brute force over
 * every pair (t, j < t): L(t, j) = min(common suffix length of q[0..t] and k[0..j],
 * j + 1, lmax). The decision at t is the latest j with the largest L >= 1; sign is +1 when
 * v[j + 1] is set, else -1; -1 when no j has L >= 1. Bits are uint8 {0,1}, (streams, T).
 * match_j / match_len (optional) receive j* (-1 if none) and L*. */
static void rosa_match_stream(const uint8_t *q, const uint8_t *k, const uint8_t *v, int64_t T,
                              int lmax, float *sign, int32_t *mj, int32_t *ml) {
  for (int64_t t = 0; t < T; ++t) {
    int64_t best_j = -1;
    int best_l = 0;
    for (int64_t j = t - 1; j >= 0; --j) {
      int cap = (int)(j + 1 < lmax ? j + 1 : lmax);
      if (cap <= best_l) continue; /* cannot beat (and ties lose to a later j) */
      int l = 0;
      while (l < cap && q[t - l] == k[j - l]) ++l;
      if (l > best_l) {
        best_l = l;
        best_j = j;
      }
    }
    if (sign) sign[t] = (best_l >= 1 && v[best_j + 1]) ? 1.0f : -1.0f;
    if (mj) mj[t] = best_l >= 1 ? (int32_t)best_j : -1;
    if (ml) ml[t] = best_l;
  }
}

void ksd_oracle_rosa_match(const uint8_t *q, const uint8_t *k, const uint8_t *v,
                           int64_t n_streams, int64_t T, int lmax, float *sign,
                           int32_t *match_j, int32_t *match_len) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t s = 0; s < n_streams; ++s)
    rosa_match_stream(q + s * T, k + s * T, v + s * T, T, lmax, sign ? sign + s * T : 0,
                      match_j ? match_j + s * T : 0, match_len ? match_len + s * T : 0);
}

/* First-order single-bit credits of reference ksdraft/kernels/rosa_credit_gpu.py:28-51,
 * by definition: for every bit of q, k and v, flip it, redo the whole match and sum
 * (sign' - sign) * grad_sign over t (in double). credits: (n_streams, 3, T). */
void ksd_oracle_rosa_credits(const uint8_t *q, const uint8_t *k, const uint8_t *v,
                             const float *grad_sign, int64_t n_streams, int64_t T, int lmax,
                             double *credits) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t s = 0; s < n_streams; ++s) {
    uint8_t *b[3];
    float *base = (float *)malloc(sizeof(float) * T);
    float *pert = (float *)malloc(sizeof(float) * T);
    for (int w = 0; w < 3; ++w) b[w] = (uint8_t *)malloc(T);
    memcpy(b[0], q + s * T, T);
    memcpy(b[1], k + s * T, T);
    memcpy(b[2], v + s * T, T);
    const float *g = grad_sign + s * T;
    rosa_match_stream(b[0], b[1], b[2], T, lmax, base, 0, 0);
    for (int w = 0; w < 3; ++w) {
      for (int64_t p = 0; p < T; ++p) {
        b[w][p] ^= 1;
        rosa_match_stream(b[0], b[1], b[2], T, lmax, pert, 0, 0);
        b[w][p] ^= 1;
        double c = 0.0;
        for (int64_t t = 0; t < T; ++t) c += (double)(pert[t] - base[t]) * (double)g[t];
        credits[(s * 3 + w) * T + p] = c;
      }
    }
    for (int w = 0; w < 3; ++w) free(b[w]);
    free(base);
    free(pert);
  }
}

/* Checker of a device-code identity (test infrastructure): the number of fp32 bit patterns
 * u in [lo, hi) for which the reciprocal division by 127 of the library's group scale,
 *     q0 = x * RN(1/127),  q1 = fma(fma(-q0, 127, x), RN(1/127), q0)   (q0 if q1 is not finite)
 * differs from the IEEE quotient x / 127. */
uint64_t ksd_check_div127(uint32_t lo, uint32_t hi) {
  const float r = 1.0f / 127.0f;
  uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i) {
    const uint32_t u = (uint32_t)i;
    float x;
    memcpy(&x, &u, 4);
    const float q0 = x * r;
    float q1 = fmaf(fmaf(-q0, 127.0f, x), r, q0);
    if (!isfinite(q1)) q1 = q0;
    const float ref = x / 127.0f;
    if (!(q1 == ref || (isnan(q1) && isnan(ref)))) ++bad;
  }
  return bad;
}
