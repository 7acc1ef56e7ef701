/*
 * Synthetic MoE routing traces for the expert-cache workloads (host code, plain C).
 *
 * One deterministic PRNG (splitmix64) per call, seeded by the caller (one seed per layer),
 * so a trace is a pure function of (shape, seed) on every machine. Two routing models:
 *
 *  ectrace_locality  Zipf(s) popularity over a seeded permutation of the experts, with
 *                    temporal locality per token: each of the token's previous-step experts
 *                    is kept with probability `keep`, the rest of its top-k is drawn by Zipf
 *                    without replacement. s = 0 gives uniform routing.
 *  ectrace_grouped   group-limited routing: per token, `topk_groups` distinct groups drawn by
 *                    Zipf(s) over a seeded group permutation, then top-k distinct experts by
 *                    Zipf(s) over their within-group rank (a seeded permutation per group).
 *
 * Output: int32 out[T][tokens * k], token-major within a step, ids in generation order.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

typedef struct {
  uint64_t s;
} rng_t;

static inline uint64_t next_u64(rng_t* r) {
  uint64_t z = (r->s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline double next_u01(rng_t* r) {
  return (double)(next_u64(r) >> 11) * (1.0 / 9007199254740992.0);
}

static inline int next_below(rng_t* r, int n) {
  int v = (int)(next_u01(r) * (double)n);
  return v < n ? v : n - 1;
}

static void permute(rng_t* r, int* p, int n) {
  for (int i = 0; i < n; i++) p[i] = i;
  for (int i = n - 1; i > 0; i--) {
    const int j = next_below(r, i + 1);
    const int t = p[i];
    p[i] = p[j];
    p[j] = t;
  }
}

/* cdf[i] = sum over ranks 1..i+1 of rank^-s */
static void zipf_cdf(double* cdf, int n, double s) {
  double acc = 0.0;
  for (int i = 0; i < n; i++) {
    acc += pow((double)(i + 1), -s);
    cdf[i] = acc;
  }
}

/* index of the first cdf entry above u * total */
static int zipf_draw(rng_t* r, const double* cdf, int n) {
  const double x = next_u01(r) * cdf[n - 1];
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (cdf[mid] > x)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}

static int contains(const int32_t* v, int n, int32_t x) {
  for (int i = 0; i < n; i++)
    if (v[i] == x) return 1;
  return 0;
}

int ectrace_locality(int32_t* out, int T, int tokens, int k, int E, double s, double keep,
                     uint64_t seed) {
  if (T < 0 || tokens <= 0 || k <= 0 || E <= 0 || k > E) return -1;
  rng_t r = {seed};
  int* perm = (int*)malloc(sizeof(int) * (size_t)E);
  double* cdf = (double*)malloc(sizeof(double) * (size_t)E);
  int32_t* prev = (int32_t*)malloc(sizeof(int32_t) * (size_t)tokens * (size_t)k);
  int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
  permute(&r, perm, E);
  zipf_cdf(cdf, E, s);
  for (int t = 0; t < T; t++) {
    for (int tok = 0; tok < tokens; tok++) {
      int32_t* pv = prev + (size_t)tok * k;
      int n = 0;
      if (t > 0)
        for (int i = 0; i < k; i++)
          if (next_u01(&r) < keep) cur[n++] = pv[i];
      while (n < k) {
        const int32_t e = perm[zipf_draw(&r, cdf, E)];
        if (!contains(cur, n, e)) cur[n++] = e;
      }
      memcpy(out + ((size_t)t * tokens + tok) * k, cur, sizeof(int32_t) * (size_t)k);
      memcpy(pv, cur, sizeof(int32_t) * (size_t)k);
    }
  }
  free(perm);
  free(cdf);
  free(prev);
  free(cur);
  return 0;
}

int ectrace_grouped(int32_t* out, int T, int tokens, int k, int E, int ngroups,
                    int topk_groups, double s, uint64_t seed) {
  if (T < 0 || tokens <= 0 || k <= 0 || E <= 0 || ngroups <= 0 || E % ngroups) return -1;
  const int gs = E / ngroups;
  if (topk_groups <= 0 || topk_groups > ngroups || k > topk_groups * gs) return -1;
  rng_t r = {seed};
  int* gperm = (int*)malloc(sizeof(int) * (size_t)ngroups);
  int* eperm = (int*)malloc(sizeof(int) * (size_t)E); /* per group: gs entries */
  double* gcdf = (double*)malloc(sizeof(double) * (size_t)ngroups);
  double* ucdf = (double*)malloc(sizeof(double) * (size_t)topk_groups * gs);
  int32_t* gsel = (int32_t*)malloc(sizeof(int32_t) * (size_t)topk_groups);
  int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
  permute(&r, gperm, ngroups);
  for (int g = 0; g < ngroups; g++) permute(&r, eperm + (size_t)g * gs, gs);
  zipf_cdf(gcdf, ngroups, s);
  /* the chosen groups' within-group Zipf weights, concatenated */
  double acc = 0.0;
  for (int i = 0; i < topk_groups * gs; i++) {
    acc += pow((double)(i % gs + 1), -s);
    ucdf[i] = acc;
  }
  for (int t = 0; t < T; t++) {
    for (int tok = 0; tok < tokens; tok++) {
      int ng = 0;
      while (ng < topk_groups) {
        const int32_t g = gperm[zipf_draw(&r, gcdf, ngroups)];
        if (!contains(gsel, ng, g)) gsel[ng++] = g;
      }
      int n = 0;
      while (n < k) {
        const int x = zipf_draw(&r, ucdf, topk_groups * gs);
        const int g = gsel[x / gs];
        const int32_t e = g * gs + eperm[(size_t)g * gs + x % gs];
        if (!contains(cur, n, e)) cur[n++] = e;
      }
      memcpy(out + ((size_t)t * tokens + tok) * k, cur, sizeof(int32_t) * (size_t)k);
    }
  }
  free(gperm);
  free(eperm);
  free(gcdf);
  free(ucdf);
  free(gsel);
  free(cur);
  return 0;
}
