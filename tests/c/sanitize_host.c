/* Driver for the host packers under AddressSanitizer and UndefinedBehaviorSanitizer: built
 * by the CPU test suite together with csrc/fourbit_host.cpp only (no GPU code), with
 * -fsanitize=address,undefined, and run.  Every host entry point is called on edge shapes
 * (one row, one group, ragged row counts, a K of 43 blocks of 256), with ties, zeros,
 * masked groups and subnormals, single- and multi-threaded; the layout transform must
 * round-trip and the decode must reproduce the packed levels.  Any out-of-bounds access,
 * use after free, leak or undefined operation aborts the run.  Prints "ok" on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fourbit.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static double urand(void) {
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return (double)(rng >> 11) / 9007199254740992.0;
}
static float nrand(void) {
  double u = urand() + 1e-12, v = urand();
  return (float)(sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}

#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      exit(1);                                                        \
    }                                                                 \
  } while (0)

static void fill(float* w, int64_t n, int kind) {
  for (int64_t i = 0; i < n; ++i) {
    float v = 0.02f * nrand();
    if (kind == 1 && urand() < 0.5) v = 0.0f;                 /* ties at zero */
    if (kind == 2) v = (float)((int)(urand() * 5) - 2) * 0.25f; /* few distinct values */
    if (kind == 3 && urand() < 0.1) v = 1e-40f * (float)(i % 7); /* subnormals */
    w[i] = v;
  }
}

static void one_shape(int N, int K, int kind, int threads) {
  const int64_t n = (int64_t)N * K;
  float* w = malloc(sizeof(float) * n);
  float* w2 = malloc(sizeof(float) * n);
  uint8_t* keep = malloc(n);
  uint8_t* codes = malloc(n / 2);
  uint8_t* codes2 = malloc(n / 2);
  uint16_t* book = malloc(sizeof(uint16_t) * (n / 128) * 16);
  uint16_t* book2 = malloc(sizeof(uint16_t) * (n / 128) * 16);
  uint8_t* scales = malloc(n / 32);
  float* levels = malloc(sizeof(float) * n);
  float* scale = malloc(sizeof(float) * N);
  fill(w, n, kind);
  for (int64_t i = 0; i < n; ++i) keep[i] = urand() < 0.8;

  CHECK(fb_quantize_gf4(w, N, K, codes, book, threads) == FB_OK);
  CHECK(fb_quantize_gf4_masked(w, keep, N, K, codes2, book2, threads) == FB_OK);
  CHECK(fb_quantize_e2m1(w, N, K, codes2, scales, threads) == FB_OK);

  /* integer levels, at most 16 distinct per 128-group */
  for (int r = 0; r < N; ++r) {
    scale[r] = 0.01f + 0.001f * (float)r;
    for (int k = 0; k < K; ++k) levels[(int64_t)r * K + k] = (float)((int)(urand() * 16) - 8);
  }
  CHECK(fb_pack_levels_gf4(levels, scale, N, K, codes2, book2, threads) == FB_OK);

  /* device layout round trip and exact decode, both formats */
  fb_shape_t s = {N, K, 1, 128, FB_FMT_GF4, 0, FB_DT_F16, FB_DT_F16};
  size_t bytes = fb_device_bytes(&s);
  CHECK(bytes > 0);
  uint8_t* dev = malloc(bytes);
  CHECK(fb_to_device(codes2, book2, dev, &s) == FB_OK);
  memset(codes, 0, n / 2);
  CHECK(fb_from_device(dev, codes, book, &s) == FB_OK);
  CHECK(memcmp(codes, codes2, n / 2) == 0);
  CHECK(memcmp(book, book2, sizeof(uint16_t) * (n / 128) * 16) == 0);
  CHECK(fb_dequant_host(codes2, book2, w2, &s) == FB_OK);
  for (int r = 0; r < N; ++r)
    for (int k = 0; k < K; ++k) {
      const float want = levels[(int64_t)r * K + k] * scale[r];
      const float got = w2[(int64_t)r * K + k];
      CHECK(fabsf(got - want) <= 1e-3f * fabsf(want) + 1e-7f); /* fp16 of the fp32 product */
    }
  free(dev);
  fb_shape_t e = {N, K, 1, 32, FB_FMT_E2M1, 0, FB_DT_BF16, FB_DT_F16};
  dev = malloc(fb_device_bytes(&e));
  CHECK(fb_quantize_e2m1(w, N, K, codes2, scales, threads) == FB_OK);
  CHECK(fb_to_device(codes2, scales, dev, &e) == FB_OK);
  CHECK(fb_from_device(dev, codes, scales, &e) == FB_OK);
  CHECK(memcmp(codes, codes2, n / 2) == 0);
  CHECK(fb_dequant_host(codes2, scales, w2, &e) == FB_OK);
  free(dev);

  /* rotation in place, then back (H is its own inverse up to rounding) */
  if (K % 256 == 0) {
    memcpy(w2, w, sizeof(float) * n);
    CHECK(fb_fwht_rows_f32(w2, N, K, 256, threads) == FB_OK);
    CHECK(fb_fwht_rows_f32(w2, N, K, 256, threads) == FB_OK);
    for (int64_t i = 0; i < n; ++i) CHECK(fabsf(w2[i] - w[i]) <= 1e-6f + 1e-5f * fabsf(w[i]));
  }

  /* the two-class split over the whole array */
  int64_t split = -1;
  double gvf = -1;
  CHECK(fb_jenks2_host(w, n, keep, &split, &gvf) == FB_OK);
  CHECK(split >= 0 && split < n && gvf >= -1e-9 && gvf <= 1.0 + 1e-9);

  free(w);
  free(w2);
  free(keep);
  free(codes);
  free(codes2);
  free(book);
  free(book2);
  free(scales);
  free(levels);
  free(scale);
}

int main(void) {
  static const int shapes[][2] = {{1, 128}, {3, 256}, {17, 384}, {2, 11008}, {16, 1024}};
  for (size_t i = 0; i < sizeof(shapes) / sizeof(shapes[0]); ++i)
    for (int kind = 0; kind < 4; ++kind)
      one_shape(shapes[i][0], shapes[i][1], kind, (int)(i % 3) + 1);
  /* the split alone across its block (256) and superblock (65,536) edges */
  static const int64_t sizes[] = {1, 2, 255, 256, 257, 65535, 65536, 65537, 131073};
  for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); ++i) {
    const int64_t n = sizes[i];
    float* w = malloc(sizeof(float) * n);
    uint8_t* keep = malloc(n);
    fill(w, n, (int)(i % 4));
    int64_t split = -1;
    double gvf = 0;
    CHECK(fb_jenks2_host(w, n, keep, &split, &gvf) == FB_OK);
    int64_t kept = 0;
    for (int64_t j = 0; j < n; ++j) kept += keep[j];
    CHECK(kept == n - split);
    free(w);
    free(keep);
  }
  /* every filter on its own, at the per-filter sizes' edges (1, a 256-block, the maximum) */
  static const int fsz[] = {1, 9, 25, 255, 256, 257, FB_JENKS2_FILTER_MAX};
  for (size_t i = 0; i < sizeof(fsz) / sizeof(fsz[0]); ++i) {
    const int n = fsz[i];
    const int64_t nf = 7;
    float* w = malloc(sizeof(float) * nf * n);
    uint8_t* keep = malloc((size_t)nf * n);
    int32_t* split = malloc(sizeof(int32_t) * nf);
    double* gvf = malloc(sizeof(double) * nf);
    fill(w, nf * n, (int)(i % 4));
    CHECK(fb_jenks2_filters_host(w, nf, n, keep, split, gvf, (int)(i % 3) + 1) == FB_OK);
    for (int64_t f = 0; f < nf; ++f) {
      int64_t kept = 0;
      for (int j = 0; j < n; ++j) kept += keep[f * n + j];
      CHECK(split[f] >= 0 && split[f] < n && kept == n - split[f]);
    }
    free(w);
    free(keep);
    free(split);
    free(gvf);
  }
  /* the per-split SSD of sorted arrays, fp32 and fp64, whole and per filter */
  for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); ++i) {
    const int64_t n = sizes[i];
    float* w = malloc(sizeof(float) * n);
    float* ssd = malloc(sizeof(float) * n);
    double* wd = malloc(sizeof(double) * n);
    double* ssdd = malloc(sizeof(double) * n);
    fill(w, n, (int)(i % 4));
    for (int64_t j = 0; j < n; ++j) wd[j] = w[j];
    CHECK(fb_jenks2_ssd_host(w, n, FB_DT_F32, ssd) == FB_OK);
    CHECK(fb_jenks2_ssd_host(wd, n, FB_DT_F64, ssdd) == FB_OK);
    for (int64_t j = 0; j < n; ++j) CHECK(ssd[j] == (float)ssdd[j]);
    if (n <= FB_JENKS2_FILTER_MAX) {
      CHECK(fb_jenks2_ssd_filters_host(wd, 1, (int32_t)n, FB_DT_F64, ssdd, 2) == FB_OK);
      CHECK(fb_jenks2_ssd_filters_host(w, 1, (int32_t)n, FB_DT_F32, ssd, 1) == FB_OK);
      for (int64_t j = 0; j < n; ++j) CHECK(ssd[j] == (float)ssdd[j]);
    }
    free(w);
    free(ssd);
    free(wd);
    free(ssdd);
  }
  /* errors are reported, not crashed on */
  float bad[2] = {1.0f, NAN};
  uint8_t k2[2];
  int64_t sp;
  double gv;
  CHECK(fb_jenks2_host(bad, 2, k2, &sp, &gv) == FB_ERR_VALUE);
  CHECK(fb_jenks2_host(bad, 0, k2, &sp, &gv) == FB_ERR_SHAPE);
  int32_t sp32;
  CHECK(fb_jenks2_filters_host(bad, 1, 2, k2, &sp32, &gv, 1) == FB_ERR_VALUE);
  CHECK(fb_jenks2_filters_host(bad, 1, FB_JENKS2_FILTER_MAX + 1, k2, &sp32, &gv, 1) == FB_ERR_SHAPE);
  printf("ok\n");
  return 0;
}
