/* abi_check.c -- the C ABI of include/imq.h driven from plain C11, the way a
 * C caller (the reference's Swift module through a module map, or any FFI)
 * binds it: opaque context and stream, device memory as void pointers, every
 * call returning a status.
 *
 * Usage: abi_check [--no-device]
 *   --no-device  only calls that need no GPU: ABI version, status strings and
 *                argument validation on a null context.
 *   (default)    also, on device 0: upload a seeded problem, imq_dequantize
 *                checked element by element against the format's closed form
 *                RNE_bf16(fl32(s*q + b)) computed here; imq_qmm_t at M = 1
 *                (the qGEMV regime) and M = 40 (the MFMA regime) with one-hot
 *                activation rows, whose outputs are single dequantized weights
 *                bit for bit; status codes for malformed and unsupported calls.
 *
 * Prints "abi_check: <n> checks passed" and exits 0, or names the first
 * failure and exits 1.
 *
 * The closed form follows Sources/ImarelloDirect/DirectTEEncoder.swift:39-46
 * (bf16 <-> f32, integer RNE) and :106-123 (nibble k % 8 of word k / 8, one
 * scale/bias pair per 64 elements of a row). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "imq.h"

static int checks = 0;

#define CHECK(cond, ...)                                \
  do {                                                  \
    ++checks;                                           \
    if (!(cond)) {                                      \
      fprintf(stderr, "abi_check: FAILED: " __VA_ARGS__); \
      fprintf(stderr, "\n");                            \
      exit(1);                                          \
    }                                                   \
  } while (0)

#define OK(ctx, call)                                                              \
  do {                                                                             \
    int st_ = (call);                                                              \
    CHECK(st_ == IMQ_OK, "%s -> %s (%s)", #call, imq_status_string(st_),           \
          imq_last_error(ctx));                                                    \
  } while (0)

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static uint32_t rng_state = 12345u;
static uint32_t next_u32(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 17;
  rng_state ^= rng_state << 5;
  return rng_state;
}
static float next_unit(void) { return (float)(next_u32() >> 8) / 16777216.0f; }

static void no_device_checks(void) {
  CHECK(imq_abi_version() == IMQ_ABI_VERSION, "imq_abi_version");
  CHECK(strcmp(imq_status_string(IMQ_OK), "IMQ_OK") == 0, "status string IMQ_OK");
  CHECK(strcmp(imq_status_string(IMQ_EUNSUPPORTED), "IMQ_EUNSUPPORTED") == 0,
        "status string IMQ_EUNSUPPORTED");
  int st = imq_qmm_t(NULL, NULL, NULL, NULL, NULL, NULL, 64, 8, 1, 64, 4, IMQ_BF16, NULL);
  CHECK(st == IMQ_EINVAL, "null context -> %s", imq_status_string(st));
  CHECK(strstr(imq_last_error(NULL), "null context") != NULL, "null-context message: %s",
        imq_last_error(NULL));
  imq_ctx** no_out = NULL;
  CHECK(imq_create(0, no_out) == IMQ_EINVAL, "imq_create with a null output pointer");
  st = imq_cast_prescale(NULL, NULL, NULL, 4, 16.0f, IMQ_F16, NULL);
  CHECK(st == IMQ_EINVAL, "prescale without a context -> %s", imq_status_string(st));
}

int main(int argc, char** argv) {
  const int device = !(argc > 1 && strcmp(argv[1], "--no-device") == 0);
  no_device_checks();
  if (!device) {
    printf("abi_check: %d checks passed (no device)\n", checks);
    return 0;
  }

  enum { N = 320, K = 512, G = K / 64, MB = 40 };
  uint32_t* w = malloc(sizeof(uint32_t) * N * (K / 8));
  uint16_t* s = malloc(sizeof(uint16_t) * N * G);
  uint16_t* b = malloc(sizeof(uint16_t) * N * G);
  uint16_t* deq = malloc(sizeof(uint16_t) * N * K);
  uint16_t* want = malloc(sizeof(uint16_t) * N * K);
  uint16_t* x = calloc((size_t)MB * K, sizeof(uint16_t));
  uint16_t* y = malloc(sizeof(uint16_t) * MB * N);
  int cols[MB];
  if (!w || !s || !b || !deq || !want || !x || !y) return 2;
  for (int i = 0; i < N * (K / 8); ++i) w[i] = next_u32();
  for (int i = 0; i < N * G; ++i) {
    const float sc = 0.001f + 0.02f * next_unit();
    s[i] = f32_to_bf16(sc);
    b[i] = f32_to_bf16(-8.0f * bf16_to_f32(s[i]) + 0.004f * (next_unit() - 0.5f));
  }
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const uint32_t q = (w[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 0xFu;
      const float sq = bf16_to_f32(s[n * G + k / 64]) * (float)q; /* exact in f32 */
      want[n * K + k] = f32_to_bf16(sq + bf16_to_f32(b[n * G + k / 64]));
    }
  for (int i = 0; i < MB; ++i) {
    cols[i] = (int)(next_u32() % K);
    x[i * K + cols[i]] = 0x3F80; /* 1.0 */
  }

  imq_ctx* ctx = NULL;
  OK(NULL, imq_create(0, &ctx));
  imq_stream stream = NULL;
  OK(ctx, imq_stream_create(ctx, &stream));
  void *dw, *ds, *db, *dx, *dy, *dd;
  OK(ctx, imq_malloc(ctx, sizeof(uint32_t) * N * (K / 8), &dw));
  OK(ctx, imq_malloc(ctx, sizeof(uint16_t) * N * G, &ds));
  OK(ctx, imq_malloc(ctx, sizeof(uint16_t) * N * G, &db));
  OK(ctx, imq_malloc(ctx, sizeof(uint16_t) * MB * K, &dx));
  OK(ctx, imq_malloc(ctx, sizeof(uint16_t) * MB * N, &dy));
  OK(ctx, imq_malloc(ctx, sizeof(uint16_t) * N * K, &dd));
  OK(ctx, imq_memcpy_h2d(ctx, dw, w, sizeof(uint32_t) * N * (K / 8), stream));
  OK(ctx, imq_memcpy_h2d(ctx, ds, s, sizeof(uint16_t) * N * G, stream));
  OK(ctx, imq_memcpy_h2d(ctx, db, b, sizeof(uint16_t) * N * G, stream));
  OK(ctx, imq_memcpy_h2d(ctx, dx, x, sizeof(uint16_t) * MB * K, stream));

  OK(ctx, imq_dequantize(ctx, dw, ds, db, dd, K, N, 64, 4, IMQ_BF16, stream));
  OK(ctx, imq_memcpy_d2h(ctx, deq, dd, sizeof(uint16_t) * N * K, stream));
  OK(ctx, imq_stream_sync(ctx, stream));
  for (int i = 0; i < N * K; ++i)
    CHECK(deq[i] == want[i], "dequant element (%d, %d): 0x%04x, closed form 0x%04x", i / K,
          i % K, deq[i], want[i]);

  const int ms[2] = {1, MB};
  for (int t = 0; t < 2; ++t) {
    const int m = ms[t];
    OK(ctx, imq_qmm_t(ctx, dw, ds, db, dx, dy, K, N, m, 64, 4, IMQ_BF16, stream));
    OK(ctx, imq_memcpy_d2h(ctx, y, dy, sizeof(uint16_t) * m * N, stream));
    OK(ctx, imq_stream_sync(ctx, stream));
    for (int i = 0; i < m; ++i)
      for (int n = 0; n < N; ++n)
        CHECK(y[i * N + n] == want[n * K + cols[i]],
              "qmm_t M=%d one-hot row %d, column %d: 0x%04x, weight 0x%04x", m, i, n,
              y[i * N + n], want[n * K + cols[i]]);
  }

  /* x / 16 to f16, closed forms: 1, -2, 2^-5, the f16 maximum, and the tie
   * 1 + 3 * 2^-11 that rounds to the even 1 + 2^-9. */
  {
    const float px[5] = {16.0f, -32.0f, 0.5f, 65504.0f * 16.0f, 16.0f * (1.0f + 3.0f / 2048.0f)};
    const uint16_t pwant[5] = {0x3C00, 0xC000, 0x2800, 0x7BFF, 0x3C02};
    uint16_t py[5] = {0};
    void *dpx, *dpy;
    OK(ctx, imq_malloc(ctx, sizeof(px), &dpx));
    OK(ctx, imq_malloc(ctx, sizeof(py), &dpy));
    OK(ctx, imq_memcpy_h2d(ctx, dpx, px, sizeof(px), stream));
    OK(ctx, imq_cast_prescale(ctx, dpx, dpy, 5, 16.0f, IMQ_F16, stream));
    OK(ctx, imq_memcpy_d2h(ctx, py, dpy, sizeof(py), stream));
    OK(ctx, imq_stream_sync(ctx, stream));
    for (int i = 0; i < 5; ++i)
      CHECK(py[i] == pwant[i], "prescale element %d: 0x%04x, closed form 0x%04x", i, py[i], pwant[i]);
    int pst = imq_cast_prescale(ctx, dpx, dpy, 5, 0.0f, IMQ_F16, stream);
    CHECK(pst == IMQ_EINVAL, "prescale by 0 -> %s", imq_status_string(pst));
    pst = imq_cast_prescale(ctx, dpx, dpy, 5, 16.0f, IMQ_F32, stream);
    CHECK(pst == IMQ_EUNSUPPORTED, "prescale to f32 -> %s", imq_status_string(pst));
    OK(ctx, imq_cast_prescale(ctx, NULL, NULL, 0, 16.0f, IMQ_F16, stream));
    OK(ctx, imq_free(ctx, dpx));
    OK(ctx, imq_free(ctx, dpy));
  }

  int st = imq_qmm_t(ctx, dw, ds, db, dx, dy, 100, N, 1, 64, 4, IMQ_BF16, stream);
  CHECK(st == IMQ_EINVAL, "K = 100 -> %s", imq_status_string(st));
  st = imq_qmm_t(ctx, dw, ds, db, dx, dy, K, N, 1, 32, 4, IMQ_BF16, stream);
  CHECK(st == IMQ_EUNSUPPORTED, "group size 32 -> %s", imq_status_string(st));
  st = imq_qmm_t(ctx, dw, ds, db, dx, dy, K, N, 1, 64, 8, IMQ_BF16, stream);
  CHECK(st == IMQ_EUNSUPPORTED, "8 bits -> %s", imq_status_string(st));
  st = imq_qgemm(ctx, dw, ds, db, dx, dy, K, N, 1, 64, 4, IMQ_F32, stream);
  CHECK(st == IMQ_EUNSUPPORTED, "f32 qgemm -> %s", imq_status_string(st));
  CHECK(strlen(imq_last_error(ctx)) > 0, "an error message after a failed call");

  void* bufs[6] = {dw, ds, db, dx, dy, dd};
  for (int i = 0; i < 6; ++i) OK(ctx, imq_free(ctx, bufs[i]));
  OK(ctx, imq_stream_destroy(ctx, stream));
  OK(NULL, imq_destroy(ctx));
  free(w), free(s), free(b), free(deq), free(want), free(x), free(y);
  printf("abi_check: %d checks passed\n", checks);
  return 0;
}
