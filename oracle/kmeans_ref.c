/*
 * CPU oracle for the token k-means used by the Q / V reorder.
 * TEST INFRASTRUCTURE ONLY (tests, smoke and the bench CPU baseline).
 *
 * The reference delegates clustering to flash-kmeans 0.3.0 @ git 3f1ea6ba
 * (uv.lock:387-389), called at kmeans.py:78-81 with max_iters, tol=0.0 and a
 * torch.manual_seed(seed) init.  That package is not available here, so this
 * build fixes its own deterministic Lloyd specification, implemented
 * identically here and in the HIP kernels:
 *
 *   init   : centroid j of slice bh = token  j*stride + (mix(seed,bh,j) % stride),
 *            stride = S / K (integer division), mix = splitmix64 finaliser of
 *            seed + 0x9E3779B97F4A7C15 * (bh*K + j + 1).
 *   assign : cn_j  = sum_d fmaf(c_jd, c_jd, .)   (sequential d = 0..D-1, from 0)
 *            dot_j = sum_d fmaf(x_d,  c_jd, .)   (sequential d)
 *            score_j = fmaf(-2, dot_j, cn_j); label = first j with minimal score.
 *   update : per 1024-token chunk, fp64 sums per (cluster, d) in token order;
 *            chunk partials added in chunk order; c_jd = (float)(sum / count),
 *            an empty cluster keeps its centroid.
 *   loop   : `iters` rounds of (assign, update); the labels returned are those
 *            of the last assign (flash-kmeans order).  Iterating after a fixed
 *            point changes nothing, so the tol=0 early exit needs no modelling.
 *
 * Inputs x are fp32 (the reference clusters x.float(), kmeans.py:77).
 * Parity of the labels against flash-kmeans itself is unpinned (absent
 * dependency); this file is pinned by tests/test_oracle_kmeans.py against a
 * brute-force Python restatement and clustering invariants.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KM_CHUNK 1024

uint64_t lbfq_ref_kmeans_mix(uint64_t seed, uint64_t bh, uint64_t K, uint64_t j) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ULL * (bh * K + j + 1ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

static void assign(const float *x, int S, int D, int K, const float *c, int32_t *labels) {
  float *cn = (float *)malloc(sizeof(float) * K);
  for (int j = 0; j < K; ++j) {
    float a = 0.0f;
    for (int d = 0; d < D; ++d) a = fmaf(c[j * D + d], c[j * D + d], a);
    cn[j] = a;
  }
  for (int t = 0; t < S; ++t) {
    const float *xt = x + (size_t)t * D;
    float best = INFINITY;
    int bj = 0;
    for (int j = 0; j < K; ++j) {
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot = fmaf(xt[d], c[j * D + d], dot);
      float sc = fmaf(-2.0f, dot, cn[j]);
      if (sc < best) { best = sc; bj = j; }
    }
    labels[t] = bj;
  }
  free(cn);
}

static void update(const float *x, int S, int D, int K, const int32_t *labels, float *c) {
  double *total = (double *)calloc((size_t)K * D, sizeof(double));
  double *part = (double *)malloc(sizeof(double) * K * D);
  int64_t *count = (int64_t *)calloc(K, sizeof(int64_t));
  for (int c0 = 0; c0 < S; c0 += KM_CHUNK) {
    memset(part, 0, sizeof(double) * K * D);
    int c1 = c0 + KM_CHUNK < S ? c0 + KM_CHUNK : S;
    for (int t = c0; t < c1; ++t) {
      int l = labels[t];
      count[l] += 1;
      for (int d = 0; d < D; ++d) part[l * D + d] += (double)x[(size_t)t * D + d];
    }
    for (int i = 0; i < K * D; ++i) total[i] += part[i];
  }
  for (int j = 0; j < K; ++j) {
    if (count[j] == 0) continue;
    for (int d = 0; d < D; ++d) c[j * D + d] = (float)(total[j * D + d] / (double)count[j]);
  }
  free(total); free(part); free(count);
}

/* x: (BH, S, D) fp32; labels: (BH, S) int32; centroids: (BH, K, D) fp32. */
int lbfq_ref_kmeans(const float *x, int BH, int S, int D, int K, int iters, uint64_t seed,
                    int32_t *labels, float *centroids) {
  if (K <= 0 || K > S) return -1;
  int stride = S / K;
  for (int bh = 0; bh < BH; ++bh) {
    const float *xb = x + (size_t)bh * S * D;
    float *cb = centroids + (size_t)bh * K * D;
    int32_t *lb = labels + (size_t)bh * S;
    for (int j = 0; j < K; ++j) {
      int idx = j * stride + (int)(lbfq_ref_kmeans_mix(seed, (uint64_t)bh, (uint64_t)K, (uint64_t)j) % (uint64_t)stride);
      memcpy(cb + (size_t)j * D, xb + (size_t)idx * D, sizeof(float) * D);
    }
    if (iters <= 0) { assign(xb, S, D, K, cb, lb); continue; }
    for (int it = 0; it < iters; ++it) {
      assign(xb, S, D, K, cb, lb);
      update(xb, S, D, K, lb, cb);
    }
  }
  return 0;
}
