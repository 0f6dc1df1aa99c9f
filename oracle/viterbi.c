/*
 * C restatement of the reference's tail-biting trellis encoder (TEST INFRASTRUCTURE
 * ONLY: used to build fixtures, never by the product path).
 *
 * Restates src/trellis/qtip.py:124-144 (viterbi_tb, QTIP Algorithm 4 two-pass
 * tail-biting) and :147-196 (_viterbi_pass, exact DP over (L-K)-bit edges with an
 * fp32 cost vector and uint8 backpointers), parameterised by L, K and T so tests can
 * brute-force tiny trellises.
 *
 * State convention (qtip.py:168-182): state s = (q << (L-K)) | e, where e is the low
 * L-K bits (the "edge" the cost vector is indexed by after the step) and q the top K
 * bits; the predecessor edge of s is s >> K. Fresh symbol bits are s & (2^K - 1).
 * Ties in the min over q keep the smallest q (the reference pins MSE, not tie bits:
 * tests/test_triton_kernel.py:24-44).
 */
#include <float.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* One DP pass over one sequence. overlap < 0: unconstrained start and free end
 * (qtip.py:161-162, :185-186); overlap >= 0: start cost 0 only at edge `overlap`,
 * final edge forced to `overlap` (qtip.py:163-165, :187-188). */
static void viterbi_pass_one(const float *w, int T, int L, int K, const float *lut,
                             int64_t overlap, float *cost, float *ncost, uint8_t *bp,
                             int32_t *states) {
  const int E = 1 << (L - K);
  const int Q = 1 << K;
  const int H = E >> K;
  const float INF = FLT_MAX / 4.0f; /* torch.finfo(float32).max / 4 (qtip.py:159) */
  if (overlap < 0) {
    for (int e = 0; e < E; ++e) cost[e] = 0.0f;
  } else {
    for (int e = 0; e < E; ++e) cost[e] = INF;
    cost[overlap] = 0.0f;
  }
  for (int t = 0; t < T; ++t) {
    const float wt = w[t];
    uint8_t *bpt = bp + (size_t)t * E;
    for (int e = 0; e < E; ++e) ncost[e] = FLT_MAX;
    for (int q = 0; q < Q; ++q) {
      const float *lq = lut + ((size_t)q << (L - K));
      const float *cq = cost + (size_t)q * H;
      for (int e = 0; e < E; ++e) {
        float d = wt - lq[e];
        float c = d * d + cq[e >> K];
        if (c < ncost[e]) {
          ncost[e] = c;
          bpt[e] = (uint8_t)q;
        }
      }
    }
    float *tmp = cost;
    cost = ncost;
    ncost = tmp;
  }
  /* after an even number of swaps `cost` may alias either buffer: the final costs are
   * in `cost` (local). */
  int64_t e;
  if (overlap < 0) {
    e = 0;
    float best = cost[0];
    for (int i = 1; i < E; ++i)
      if (cost[i] < best) {
        best = cost[i];
        e = i;
      }
  } else {
    e = overlap;
  }
  for (int t = T - 1; t >= 0; --t) {
    int64_t q = bp[(size_t)t * E + e];
    int64_t s = (q << (L - K)) | e;
    states[t] = (int32_t)s;
    e = s >> K;
  }
}

/* Batched single pass (used by tests for brute-force optimality checks). */
int trellis_oracle_viterbi_pass(const float *w, int n, int T, int L, int K,
                                const float *lut, const int64_t *overlap,
                                int32_t *states_out, int nthreads) {
  if (L <= K || L > 20 || K < 1 || K > 8 || T < 1) return 1;
  const int E = 1 << (L - K);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    float *cost = (float *)malloc(sizeof(float) * E);
    float *ncost = (float *)malloc(sizeof(float) * E);
    uint8_t *bp = (uint8_t *)malloc((size_t)T * E);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int i = 0; i < n; ++i) {
      viterbi_pass_one(w + (size_t)i * T, T, L, K, lut, overlap ? overlap[i] : -1, cost,
                       ncost, bp, states_out + (size_t)i * T);
    }
    free(cost);
    free(ncost);
    free(bp);
  }
  return 0;
}

/* Tail-biting encode (qtip.py:124-144): pass 1 on the sequence rolled by T/2,
 * overlap = state at rolled position T/2 >> K, pass 2 constrained to that overlap.
 * Outputs K-bit symbols, the fp32 dequantized values lut[state] and the states. */
int trellis_oracle_viterbi_tb(const float *w, int n, int T, int L, int K, const float *lut,
                              int32_t *bits_out, float *dq_out, int32_t *states_out,
                              int nthreads) {
  if (L <= K || L > 20 || K < 1 || K > 8 || T < 2) return 1;
  const int E = 1 << (L - K);
  const int roll = T / 2;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    float *cost = (float *)malloc(sizeof(float) * E);
    float *ncost = (float *)malloc(sizeof(float) * E);
    uint8_t *bp = (uint8_t *)malloc((size_t)T * E);
    float *wr = (float *)malloc(sizeof(float) * T);
    int32_t *st1 = (int32_t *)malloc(sizeof(int32_t) * T);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int i = 0; i < n; ++i) {
      const float *wi = w + (size_t)i * T;
      /* torch.roll(w, roll, dims=1): wr[t] = w[(t - roll) mod T] */
      for (int t = 0; t < T; ++t) wr[t] = wi[((t - roll) % T + T) % T];
      viterbi_pass_one(wr, T, L, K, lut, -1, cost, ncost, bp, st1);
      int64_t overlap = st1[roll] >> K;
      int32_t *st2 = states_out + (size_t)i * T;
      viterbi_pass_one(wi, T, L, K, lut, overlap, cost, ncost, bp, st2);
      for (int t = 0; t < T; ++t) {
        bits_out[(size_t)i * T + t] = st2[t] & ((1 << K) - 1);
        dq_out[(size_t)i * T + t] = lut[st2[t]];
      }
    }
    free(cost);
    free(ncost);
    free(bp);
    free(wr);
    free(st1);
  }
  return 0;
}
