/*
 * gen_expf_table.c -- build-time generator of the glibc expf / logf exception
 * tables used by the kernels to reproduce Rust's f32::exp and f32::ln bits.
 *
 * Rust's f32::exp and f32::ln on Linux call glibc's expf and logf, which are
 * not correctly rounded.  The device computes y = tc_exp_d(x) (resp.
 * tc_log_d(x)) in double and rounds it once (tc_expf_cr, tc_logf_cr).  This
 * program walks every float input of the ranges the kernels use, compares
 * glibc with the device routine, and checks:
 *
 *   1. every disagreement lies within the band (in float ulps, measured on y)
 *      of a rounding midpoint, and glibc's value is the neighbour across it;
 *   2. the device routine is correctly rounded (checked against expl / logl
 *      wherever those are far enough from a midpoint to decide);
 *   3. outside the band the two always agree;
 *   4. tc_expf_fast (the f32 routine the kernels use for approximate terms)
 *      is within TC_EXPF_FAST_ULPS of tc_expf_cr on [-87, 0].
 *
 * Ranges: expf on [-104, 88.72283935546875]; logf on [1, 2^24) (the kernels
 * take the log of a softmax denominator, which lies in [1, V]).  The sorted
 * bit patterns of the disagreeing inputs are written as C includes with an
 * index for a two-step lookup.  Any failed check aborts the build.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tc_math.h"

#define BAND 0.002
#define LOG_BUCKET_SHIFT 12

static float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

typedef struct {
  uint32_t* keys;
  size_t n;
  long long band;
  long long bad_cr;
  long long fail;
  long long fast_bad;
  double max_exc_dist;
} scan_result;

static void push(uint32_t** k, size_t* n, size_t* cap, uint32_t v) {
  if (*n == *cap) { *cap = *cap ? *cap * 2 : 4096; *k = (uint32_t*)realloc(*k, *cap * sizeof(uint32_t)); }
  (*k)[(*n)++] = v;
}

static void merge(scan_result* R, uint32_t* lk, size_t ln, long long band, long long bad, long long fail,
                  long long fast_bad, double maxd) {
  R->keys = (uint32_t*)realloc(R->keys, (R->n + ln + 1) * sizeof(uint32_t));
  memcpy(R->keys + R->n, lk, ln * sizeof(uint32_t));
  R->n += ln;
  R->band += band;
  R->bad_cr += bad;
  R->fail += fail;
  R->fast_bad += fast_bad;
  if (maxd > R->max_exc_dist) R->max_exc_dist = maxd;
}

/* expf over the bit patterns lo..hi (inclusive, one sign). */
static void scan_expf(uint32_t lo, uint32_t hi, scan_result* R) {
#pragma omp parallel
  {
    size_t lcap = 0, ln = 0;
    uint32_t* lk = NULL;
    long long lband = 0, lbad = 0, lfail = 0, lfast = 0;
    double lmax = 0.0;
#pragma omp for schedule(static, 65536)
    for (long long u = lo; u <= (long long)hi; u++) {
      float x = bf((uint32_t)u);
      double y = tc_exp_d((double)x);
      float r = tc_expf_cr(x);
      float g = expf(x);
      double d = (r != 0.0f || y > 0.0) ? tc_mid_dist(y, r) : 0.5;
      int in_band = d < BAND;
      lband += in_band;
      long double yl = expl((long double)x);
      float c = (float)yl;
      if (c != r && tc_mid_dist((double)yl, c) > 1e-6) lbad++;
      if (g != r) {
        if (!in_band || fb(g) != tc_toward(y, r)) lfail++;
        if (d > lmax) lmax = d;
        push(&lk, &ln, &lcap, (uint32_t)u);
      }
      if (x <= 0.0f && x >= -87.0f) {
        long long df = (long long)fb(tc_expf_fast(x)) - (long long)fb(r);
        if (df < 0) df = -df;
        if (df > TC_EXPF_FAST_ULPS) lfast++;
      }
    }
#pragma omp critical
    merge(R, lk, ln, lband, lbad, lfail, lfast, lmax);
    free(lk);
  }
}

/* logf over [1, 2^24). */
static void scan_logf(double band, scan_result* R) {
  uint32_t lo = fb(1.0f), hi = fb(16777216.0f);
#pragma omp parallel
  {
    size_t lcap = 0, ln = 0;
    uint32_t* lk = NULL;
    long long lband = 0, lbad = 0, lfail = 0;
    double lmax = 0.0;
#pragma omp for schedule(static, 65536)
    for (long long u = lo; u < (long long)hi; u++) {
      float x = bf((uint32_t)u);
      double y = tc_log_d((double)x);
      float r = tc_logf_cr(x);
      float g = logf(x);
      double d = (x != 1.0f) ? tc_mid_dist(y, r) : 0.5;
      int in_band = d < band;
      lband += in_band;
      long double yl = logl((long double)x);
      float c = (float)yl;
      if (c != r && tc_mid_dist((double)yl, c) > 1e-6) lbad++;
      if (g != r) {
        if (!in_band || fb(g) != tc_toward(y, r)) lfail++;
        if (d > lmax) lmax = d;
        push(&lk, &ln, &lcap, (uint32_t)u);
      }
    }
#pragma omp critical
    merge(R, lk, ln, lband, lbad, lfail, 0, lmax);
    free(lk);
  }
}

static int cmp_u32(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return (x > y) - (x < y);
}

static void write_keys(FILE* f, const char* name, const uint32_t* keys, size_t n) {
  fprintf(f, "__device__ const uint32_t %s[%zu] = {\n", name, n ? n : 1);
  for (size_t i = 0; i < n; i++) fprintf(f, "0x%08xu,%s", keys[i], (i % 8 == 7) ? "\n" : "");
  if (!n) fprintf(f, "0u");
  fprintf(f, "};\n");
}

int main(int argc, char** argv) {
  if (argc != 3) { fprintf(stderr, "usage: %s expf.inc logf.inc\n", argv[0]); return 2; }
  /* ---------------- expf ---------------- */
  scan_result E = {0};
  scan_expf(0x80000000u, fb(-104.0f), &E);
  scan_expf(0x00000000u, fb(88.72283935546875f), &E);
  if (E.fail) { fprintf(stderr, "gen: an expf disagreement lies outside the band\n"); return 1; }
  if (E.bad_cr) { fprintf(stderr, "gen: tc_expf_cr is not correctly rounded on %lld inputs\n", E.bad_cr); return 1; }
  if (E.fast_bad) {
    fprintf(stderr, "gen: tc_expf_fast is off by more than %d ulp on %lld inputs\n", TC_EXPF_FAST_ULPS, E.fast_bad);
    return 1;
  }
  qsort(E.keys, E.n, sizeof(uint32_t), cmp_u32);
  FILE* f = fopen(argv[1], "w");
  if (!f) { perror("fopen"); return 1; }
  fprintf(f, "// generated by gen_expf_table.c -- do not edit\n");
  fprintf(f, "// inputs in [-104, 88.72283935546875] where glibc expf != tc_expf_cr: %zu\n", E.n);
  fprintf(f, "// inputs within %.4g ulp of a midpoint: %lld\n", BAND, E.band);
  fprintf(f, "#define TC_EXPF_BAND %.17g\n", BAND);
  fprintf(f, "#define TC_EXPF_EXC_N %zuu\n", E.n);
  write_keys(f, "tc_expf_exc_keys", E.keys, E.n);
  /* index: first entry whose upper 16 bits are >= h, for h = 0 .. 65536 */
  fprintf(f, "__device__ const uint32_t tc_expf_exc_index[65537] = {\n");
  size_t j = 0;
  for (uint32_t h = 0; h <= 65536u; h++) {
    while (j < E.n && (E.keys[j] >> 16) < h) j++;
    fprintf(f, "%zuu,%s", j, (h % 16 == 15) ? "\n" : "");
  }
  fprintf(f, "};\n");
  fclose(f);
  printf("expf exceptions: %zu (band members %lld, widest %.5f ulp)\n", E.n, E.band, E.max_exc_dist);

  /* ---------------- logf ---------------- */
  /* first pass with the widest band to find how far from a midpoint glibc can
   * disagree, then the real pass with that band (plus margin) */
  scan_result L0 = {0};
  scan_logf(0.5, &L0);
  if (L0.fail) { fprintf(stderr, "gen: a logf disagreement is not the neighbour across the midpoint\n"); return 1; }
  if (L0.bad_cr > 1) { fprintf(stderr, "gen: tc_logf_cr is not correctly rounded on %lld inputs\n", L0.bad_cr); return 1; }
  double lband = L0.max_exc_dist * 1.0001 + 1e-9;
  if (lband > 0.5) lband = 0.5;
  free(L0.keys);
  scan_result L = {0};
  scan_logf(lband, &L);
  if (L.fail) { fprintf(stderr, "gen: a logf disagreement lies outside the band\n"); return 1; }
  qsort(L.keys, L.n, sizeof(uint32_t), cmp_u32);
  f = fopen(argv[2], "w");
  if (!f) { perror("fopen"); return 1; }
  fprintf(f, "// generated by gen_expf_table.c -- do not edit\n");
  fprintf(f, "// inputs in [1, 2^24) where glibc logf != tc_logf_cr: %zu\n", L.n);
  fprintf(f, "// inputs within %.6g ulp of a midpoint: %lld\n", lband, L.band);
  fprintf(f, "#define TC_LOGF_BAND %.17g\n", lband);
  fprintf(f, "#define TC_LOGF_EXC_N %zuu\n", L.n);
  fprintf(f, "#define TC_LOGF_BUCKET_SHIFT %d\n", LOG_BUCKET_SHIFT);
  write_keys(f, "tc_logf_exc_keys", L.keys, L.n);
  /* index by bucket b = (bits - bits(1.0f)) >> LOG_BUCKET_SHIFT: first entry of bucket b */
  uint32_t nb = (fb(16777216.0f) - fb(1.0f)) >> LOG_BUCKET_SHIFT;
  fprintf(f, "#define TC_LOGF_NBUCKETS %uu\n", nb);
  fprintf(f, "__device__ const uint32_t tc_logf_exc_index[%u] = {\n", nb + 1);
  j = 0;
  for (uint32_t b = 0; b <= nb; b++) {
    while (j < L.n && ((L.keys[j] - fb(1.0f)) >> LOG_BUCKET_SHIFT) < b) j++;
    fprintf(f, "%zuu,%s", j, (b % 16 == 15) ? "\n" : "");
  }
  fprintf(f, "};\n");
  fclose(f);
  printf("logf exceptions: %zu (band %.5f ulp, band members %lld)\n", L.n, lband, L.band);
  return 0;
}
