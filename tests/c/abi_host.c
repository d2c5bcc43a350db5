/* A C caller of libfourbit's host-side C ABI (include/fourbit.h), as a native binding of
 * the reference's FFI would call it: plain pointers and sizes, status codes, no torch.
 * Every check is a known answer that follows from the format definitions:
 *  - GF4 on a group of 16 distinct fp16-exact values, 8 copies each: the optimal 16-class
 *    partition has SSD 0 and is unique, so the codebook is those values in ascending
 *    order and the decode reproduces the input exactly; an all-zero row decodes to 0;
 *  - E2M1 on values of the grid with amax 6: scale byte 127 (2^0) and an exact decode;
 *  - integer levels -8..7 with scale 0.5 decode to level * 0.5;
 *  - the normalised FWHT of a one-hot row of width 4 is 0.5 everywhere;
 *  - the device layout round trip returns the canonical bytes;
 *  - validation rejects bad shapes with the documented codes.
 * Built and run by tests/test_host.py::test_c_abi_from_c (gcc, no GPU needed).
 * Prints "ok" and exits 0 when every check holds. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fourbit.h"

static int failures = 0;

#define CHECK(cond)                                              \
  do {                                                           \
    if (!(cond)) {                                               \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                \
    }                                                            \
  } while (0)

/* fp16 bits of a float that fp16 represents exactly as a normal number (or zero). */
static uint16_t half_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  if ((u & 0x7FFFFFFFu) == 0) return (uint16_t)sign;
  const int e = (int)((u >> 23) & 0xFF) - 127 + 15;
  return (uint16_t)(sign | ((uint32_t)e << 10) | ((u & 0x7FFFFFu) >> 13));
}

static void check_validation(void) {
  fb_shape_t s = {64, 1024, 1, 128, FB_FMT_GF4, 0, FB_DT_F16, FB_DT_F16};
  CHECK(fb_abi_version() > 0);
  CHECK(fb_validate(&s) == FB_OK);
  s.K = 100;
  CHECK(fb_validate(&s) == FB_ERR_SHAPE);
  s.K = 1024;
  s.group = 64;
  CHECK(fb_validate(&s) == FB_ERR_GROUP);
  s.group = 128;
  s.fwht_block = 8192;
  CHECK(fb_validate(&s) == FB_ERR_FWHT);
  CHECK(strstr(fb_strerror(FB_ERR_SHAPE), "fourbit") != NULL);
  CHECK(fb_validate(NULL) == FB_ERR_NULL);
  /* one block: 16 rows x 512 K of GF4 is 6144 bytes */
  fb_shape_t b = {16, 512, 1, 128, FB_FMT_GF4, 0, FB_DT_F16, FB_DT_F16};
  CHECK(fb_device_bytes(&b) == 6144);
  CHECK(fb_workspace_bytes(&b) == 0);
}

static void check_gf4(void) {
  enum { N = 2, K = 128 };
  float w[N * K], back[N * K];
  uint8_t codes[N * K / 2];
  uint16_t cb[N * (K / 128) * 16];
  /* row 0: v_j = (j - 8) / 4, j = 0..15, eight copies each, in a scrambled order */
  for (int i = 0; i < K; ++i) {
    const int j = (i * 7 + 3) % 16;
    w[i] = (float)(j - 8) * 0.25f;
  }
  for (int i = 0; i < K; ++i) w[K + i] = 0.0f; /* row 1: zeros */
  CHECK(fb_quantize_gf4(w, N, K, codes, cb, 2) == FB_OK);
  for (int j = 0; j < 16; ++j) CHECK(cb[j] == half_bits((float)(j - 8) * 0.25f));
  for (int i = 0; i < K; ++i) {
    const int code = (codes[i / 2] >> ((i & 1) * 4)) & 15;
    CHECK(code == (i * 7 + 3) % 16);
  }
  fb_shape_t s = {N, K, 1, 128, FB_FMT_GF4, 0, FB_DT_F16, FB_DT_F16};
  CHECK(fb_dequant_host(codes, cb, back, &s) == FB_OK);
  for (int i = 0; i < N * K; ++i) CHECK(back[i] == w[i]);

  /* device layout round trip */
  const size_t nb = fb_device_bytes(&s);
  uint8_t* dev = (uint8_t*)malloc(nb);
  uint8_t codes2[N * K / 2];
  uint16_t cb2[N * (K / 128) * 16];
  CHECK(dev != NULL);
  CHECK(fb_to_device(codes, cb, dev, &s) == FB_OK);
  CHECK(fb_from_device(dev, codes2, cb2, &s) == FB_OK);
  CHECK(memcmp(codes, codes2, sizeof codes) == 0);
  CHECK(memcmp(cb, cb2, sizeof cb) == 0);
  free(dev);
}

static void check_e2m1(void) {
  enum { N = 1, K = 128 };
  static const float grid[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float w[K], back[K];
  uint8_t codes[K / 2], scales[K / 32];
  /* every 32-group holds 6 (i % 8 == 7), so amax = 6: e = floor(log2 6) - 2 = 0 */
  for (int i = 0; i < K; ++i) w[i] = (i & 8 ? -1.0f : 1.0f) * grid[i % 8];
  CHECK(fb_quantize_e2m1(w, N, K, codes, scales, 1) == FB_OK);
  for (int g = 0; g < K / 32; ++g) CHECK(scales[g] == 127);
  for (int i = 0; i < K; ++i) {
    const int c = (codes[i / 2] >> ((i & 1) * 4)) & 15;
    CHECK((c & 7) == i % 8);
  }
  fb_shape_t s = {N, K, 1, 32, FB_FMT_E2M1, 0, FB_DT_BF16, FB_DT_F16};
  CHECK(fb_dequant_host(codes, scales, back, &s) == FB_OK);
  for (int i = 0; i < K; ++i) CHECK(back[i] == w[i]);
}

static void check_levels_and_fwht(void) {
  enum { N = 1, K = 128 };
  float lv[K], sc[N] = {0.5f}, back[K];
  uint8_t codes[K / 2];
  uint16_t cb[16];
  for (int i = 0; i < K; ++i) lv[i] = (float)(i % 16 - 8);
  CHECK(fb_pack_levels_gf4(lv, sc, N, K, codes, cb, 1) == FB_OK);
  fb_shape_t s = {N, K, 1, 128, FB_FMT_GF4, 0, FB_DT_F16, FB_DT_F16};
  CHECK(fb_dequant_host(codes, cb, back, &s) == FB_OK);
  for (int i = 0; i < K; ++i) CHECK(back[i] == lv[i] * 0.5f);

  float r[4] = {1.0f, 0.0f, 0.0f, 0.0f};
  CHECK(fb_fwht_rows_f32(r, 1, 4, 4, 1) == FB_OK);
  for (int i = 0; i < 4; ++i) CHECK(r[i] == 0.5f);
}

int main(void) {
  check_validation();
  check_gf4();
  check_e2m1();
  check_levels_and_fwht();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
