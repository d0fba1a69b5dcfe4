/*
 * capi_selftest.c -- a plain C consumer of include/thin_hip.h: device memory
 * from hipMalloc, its own stream, no PyTorch in the process.  It drives a few
 * entry points on inputs whose results are exact (small integers, bit copies)
 * and checks them on the host; exit status 0 means every check passed.
 *
 *   thintnpu_amd/capi_selftest        (built by thintnpu_amd/build.py)
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "thin_hip.h"

static int failures = 0;

#define CHECK(cond, ...)                 \
  do {                                   \
    if (!(cond)) {                       \
      printf("FAIL %s:%d: ", __FILE__, __LINE__); \
      printf(__VA_ARGS__);               \
      printf("\n");                      \
      ++failures;                        \
    }                                    \
  } while (0)

#define HIP(call)                                                        \
  do {                                                                   \
    hipError_t e_ = (call);                                              \
    if (e_ != hipSuccess) {                                              \
      printf("FAIL %s: %s\n", #call, hipGetErrorString(e_));             \
      return 2;                                                          \
    }                                                                    \
  } while (0)

/* fp16 bits of a small integer (|v| <= 2048, exact) and back */
static uint16_t half_of_int(int v) {
  if (v == 0) return 0;
  uint16_t sign = v < 0 ? 0x8000u : 0;
  unsigned a = (unsigned)(v < 0 ? -v : v);
  int e = 31 - __builtin_clz(a);                 /* a = 1.f * 2^e, e <= 11 */
  unsigned mant = (e <= 10 ? a << (10 - e) : a >> (e - 10)) & 0x3ffu;  /* exact: a has <= 11 bits */
  return (uint16_t)(sign | (unsigned)(e + 15) << 10 | mant);
}
static int int_of_half(uint16_t h) {
  if ((h & 0x7fffu) == 0) return 0;
  int e = (int)((h >> 10) & 0x1fu) - 15;
  unsigned mant = (h & 0x3ffu) | 0x400u;
  int v = e >= 10 ? (int)(mant << (e - 10)) : (int)(mant >> (10 - e));
  return (h & 0x8000u) ? -v : v;
}

static thin_desc desc(void* data, int32_t dtype, int32_t rank, const int64_t* sizes) {
  thin_desc d;
  memset(&d, 0, sizeof d);
  d.data = data;
  d.dtype = dtype;
  d.rank = rank;
  int64_t stride = 1;
  for (int i = rank - 1; i >= 0; --i) {
    d.sizes[i] = sizes[i];
    d.strides[i] = stride;
    stride *= sizes[i];
  }
  return d;
}

int main(void) {
  hipStream_t s;
  HIP(hipStreamCreate(&s));
  printf("library: %s\n", thin_version());

  /* 1. fp32 add with alpha: out = x + 2 y */
  {
    enum { N = 1000 };
    float hx[N], hy[N], ho[N];
    for (int i = 0; i < N; ++i) { hx[i] = (float)i; hy[i] = (float)(3 * i); }
    float *dx, *dy, *dout;
    HIP(hipMalloc((void**)&dx, sizeof hx));
    HIP(hipMalloc((void**)&dy, sizeof hy));
    HIP(hipMalloc((void**)&dout, sizeof ho));
    HIP(hipMemcpy(dx, hx, sizeof hx, hipMemcpyHostToDevice));
    HIP(hipMemcpy(dy, hy, sizeof hy, hipMemcpyHostToDevice));
    const int64_t sz[1] = {N};
    thin_desc x = desc(dx, THIN_F32, 1, sz), y = desc(dy, THIN_F32, 1, sz), o = desc(dout, THIN_F32, 1, sz);
    CHECK(thin_binary(THIN_ADD, &x, &y, &o, 2.0f, s) == THIN_OK, "thin_binary: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(ho, dout, sizeof ho, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int i = 0; i < N; ++i) bad += ho[i] != (float)(7 * i);
    CHECK(bad == 0, "add: %d wrong", bad);
    HIP(hipFree(dx));
    HIP(hipFree(dy));
    HIP(hipFree(dout));
  }

  /* 2. fp16 cat along dim 1: [2,3] ++ [2,5] -> [2,8] (bit copy) */
  {
    uint16_t ha[6], hb[10], ho[16];
    for (int i = 0; i < 6; ++i) ha[i] = (uint16_t)(0x1000 + i);
    for (int i = 0; i < 10; ++i) hb[i] = (uint16_t)(0x7e00 + i); /* NaN payloads move unchanged */
    uint16_t *da, *db, *dout;
    HIP(hipMalloc((void**)&da, sizeof ha));
    HIP(hipMalloc((void**)&db, sizeof hb));
    HIP(hipMalloc((void**)&dout, sizeof ho));
    HIP(hipMemcpy(da, ha, sizeof ha, hipMemcpyHostToDevice));
    HIP(hipMemcpy(db, hb, sizeof hb, hipMemcpyHostToDevice));
    const int64_t sa[2] = {2, 3}, sb[2] = {2, 5}, so[2] = {2, 8};
    thin_desc in[2] = {desc(da, THIN_F16, 2, sa), desc(db, THIN_F16, 2, sb)};
    thin_desc o = desc(dout, THIN_F16, 2, so);
    CHECK(thin_cat(in, 2, 1, &o, s) == THIN_OK, "thin_cat: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(ho, dout, sizeof ho, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int r = 0; r < 2; ++r)
      for (int c = 0; c < 8; ++c) bad += ho[r * 8 + c] != (c < 3 ? ha[r * 3 + c] : hb[r * 5 + c - 3]);
    CHECK(bad == 0, "cat: %d wrong", bad);
    HIP(hipFree(da));
    HIP(hipFree(db));
    HIP(hipFree(dout));
  }

  /* 3. bmm of small integers (every sum exact): [2,3,4] x [2,4,5] */
  {
    enum { B = 2, M = 3, K = 4, N = 5 };
    int ia[B * M * K], ib[B * K * N];
    uint16_t ha[B * M * K], hb[B * K * N], ho[B * M * N];
    for (int i = 0; i < B * M * K; ++i) { ia[i] = (i * 7) % 9 - 4; ha[i] = half_of_int(ia[i]); }
    for (int i = 0; i < B * K * N; ++i) { ib[i] = (i * 5) % 7 - 3; hb[i] = half_of_int(ib[i]); }
    uint16_t *da, *db, *dout;
    HIP(hipMalloc((void**)&da, sizeof ha));
    HIP(hipMalloc((void**)&db, sizeof hb));
    HIP(hipMalloc((void**)&dout, sizeof ho));
    HIP(hipMemcpy(da, ha, sizeof ha, hipMemcpyHostToDevice));
    HIP(hipMemcpy(db, hb, sizeof hb, hipMemcpyHostToDevice));
    const int64_t sa[3] = {B, M, K}, sb[3] = {B, K, N};
    thin_desc a = desc(da, THIN_F16, 3, sa), b = desc(db, THIN_F16, 3, sb);
    thin_bmm_layout L;
    memset(&L, 0, sizeof L);
    L.a_channels = -1;
    L.b_channels = -1;
    int32_t rank = 0;
    int64_t osz[4] = {0, 0, 0, 0};
    CHECK(thin_layout_bmm_shape(&a, &b, &L, &rank, osz) == THIN_OK && rank == 3 && osz[0] == B && osz[1] == M &&
              osz[2] == N,
          "thin_layout_bmm_shape: %s", thin_last_error());
    thin_desc o = desc(dout, THIN_F16, 3, osz);
    CHECK(thin_layout_bmm(&a, &b, &L, &o, s) == THIN_OK, "thin_layout_bmm: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(ho, dout, sizeof ho, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int bt = 0; bt < B; ++bt)
      for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
          int acc = 0;
          for (int k = 0; k < K; ++k) acc += ia[(bt * M + i) * K + k] * ib[(bt * K + k) * N + j];
          bad += int_of_half(ho[(bt * M + i) * N + j]) != acc;
        }
    CHECK(bad == 0, "bmm: %d wrong", bad);
    /* mismatched reduction sizes are rejected with the reference's message */
    const int64_t sbad[3] = {B, K + 1, N};
    thin_desc bb = desc(db, THIN_F16, 3, sbad);
    CHECK(thin_layout_bmm_shape(&a, &bb, &L, &rank, osz) == THIN_ERR_INVALID &&
              strstr(thin_last_error(), "do not match") != NULL,
          "bmm mismatch not rejected: %s", thin_last_error());
    HIP(hipFree(da));
    HIP(hipFree(db));
    HIP(hipFree(dout));
  }

  /* 4. channel_select: [1,4,3,16] (64 channels, 2 groups of 32), channels
   *    [4, 12) of each group -> [1,1,3,16] */
  {
    enum { C1 = 4, T = 3 };
    uint16_t hx[C1 * T * 16], ho[1 * T * 16];
    for (int i = 0; i < C1 * T * 16; ++i) hx[i] = (uint16_t)i;
    uint16_t *dx, *dout;
    HIP(hipMalloc((void**)&dx, sizeof hx));
    HIP(hipMalloc((void**)&dout, sizeof ho));
    HIP(hipMemcpy(dx, hx, sizeof hx, hipMemcpyHostToDevice));
    const int64_t sx[4] = {1, C1, T, 16};
    thin_desc x = desc(dx, THIN_F16, 4, sx);
    int64_t osz[4];
    CHECK(thin_channel_select_shape(&x, 2, 4, 8, osz) == THIN_OK && osz[1] == 1 && osz[2] == T,
          "thin_channel_select_shape: %s", thin_last_error());
    thin_desc o = desc(dout, THIN_F16, 4, osz);
    CHECK(thin_channel_select(&x, 2, 4, 8, &o, s) == THIN_OK, "thin_channel_select: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(ho, dout, sizeof ho, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int t = 0; t < T; ++t)
      for (int lane = 0; lane < 16; ++lane) {
        const int c = lane, sc = (c / 8) * 32 + 4 + c % 8;
        bad += ho[t * 16 + lane] != hx[(sc / 16) * T * 16 + t * 16 + sc % 16];
      }
    CHECK(bad == 0, "channel_select: %d wrong", bad);
    HIP(hipFree(dx));
    HIP(hipFree(dout));
  }

  /* 5. pack NCHW [1,20,3,5] -> NC1HWC0 [1,2,3,5,16] (channels 20..31 zero),
   *    then unpack back to NCHW: both bit copies */
  {
    enum { C = 20, H = 3, W = 5, C1 = 2 };
    uint16_t hx[C * H * W], hb[C1 * H * W * 16], hu[C * H * W];
    for (int i = 0; i < C * H * W; ++i) hx[i] = (uint16_t)(0x3c00 + i);
    uint16_t *dx, *db, *du;
    HIP(hipMalloc((void**)&dx, sizeof hx));
    HIP(hipMalloc((void**)&db, sizeof hb));
    HIP(hipMalloc((void**)&du, sizeof hu));
    HIP(hipMemcpy(dx, hx, sizeof hx, hipMemcpyHostToDevice));
    const int64_t sx[4] = {1, C, H, W}, sb[5] = {1, C1, H, W, 16};
    thin_desc x = desc(dx, THIN_F16, 4, sx), b = desc(db, THIN_F16, 5, sb), u = desc(du, THIN_F16, 4, sx);
    CHECK(thin_pack_nc1hwc0(&x, &b, s) == THIN_OK, "thin_pack_nc1hwc0: %s", thin_last_error());
    CHECK(thin_unpack_nc1hwc0(&b, &u, s) == THIN_OK, "thin_unpack_nc1hwc0: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(hb, db, sizeof hb, hipMemcpyDeviceToHost));
    HIP(hipMemcpy(hu, du, sizeof hu, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int c = 0; c < C1 * 16; ++c)
      for (int p = 0; p < H * W; ++p) {
        const uint16_t want = c < C ? hx[c * H * W + p] : 0;
        bad += hb[((c / 16) * H * W + p) * 16 + c % 16] != want;
      }
    CHECK(bad == 0, "pack: %d wrong", bad);
    CHECK(memcmp(hu, hx, sizeof hx) == 0, "unpack did not restore the NCHW input");
    HIP(hipFree(dx));
    HIP(hipFree(db));
    HIP(hipFree(du));
  }

  /* 6. nearest 2x upsample [1,1,2,3,16] -> [1,1,4,6,16] and a k3 max pool of
   *    the result (distinct small integers: every maximum exact), then fill */
  {
    enum { H = 2, W = 3 };
    uint16_t hx[H * W * 16], hy[4 * H * W * 16], hp[4 * H * W * 16];
    for (int i = 0; i < H * W * 16; ++i) hx[i] = half_of_int((i * 37) % 101 - 50);
    uint16_t *dx, *dy, *dp;
    HIP(hipMalloc((void**)&dx, sizeof hx));
    HIP(hipMalloc((void**)&dy, sizeof hy));
    HIP(hipMalloc((void**)&dp, sizeof hp));
    HIP(hipMemcpy(dx, hx, sizeof hx, hipMemcpyHostToDevice));
    const int64_t sx[5] = {1, 1, H, W, 16}, sy[5] = {1, 1, 2 * H, 2 * W, 16};
    thin_desc x = desc(dx, THIN_F16, 5, sx), y = desc(dy, THIN_F16, 5, sy), p = desc(dp, THIN_F16, 5, sy);
    CHECK(thin_upsample2x_nc1hwc0(&x, &y, s) == THIN_OK, "thin_upsample2x_nc1hwc0: %s", thin_last_error());
    CHECK(thin_maxpool_nc1hwc0(&y, 3, &p, s) == THIN_OK, "thin_maxpool_nc1hwc0: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(hy, dy, sizeof hy, hipMemcpyDeviceToHost));
    HIP(hipMemcpy(hp, dp, sizeof hp, hipMemcpyDeviceToHost));
    int bad_up = 0, bad_pool = 0;
    for (int r = 0; r < 2 * H; ++r)
      for (int c = 0; c < 2 * W; ++c)
        for (int l = 0; l < 16; ++l) {
          bad_up += hy[(r * 2 * W + c) * 16 + l] != hx[((r / 2) * W + c / 2) * 16 + l];
          int best = -100000;
          for (int dr = -1; dr <= 1; ++dr)
            for (int dc = -1; dc <= 1; ++dc) {
              const int rr = r + dr, cc = c + dc;
              if (rr < 0 || rr >= 2 * H || cc < 0 || cc >= 2 * W) continue; /* taps outside the plane skipped */
              const int v = int_of_half(hx[((rr / 2) * W + cc / 2) * 16 + l]);
              if (v > best) best = v;
            }
          bad_pool += int_of_half(hp[(r * 2 * W + c) * 16 + l]) != best;
        }
    CHECK(bad_up == 0, "upsample2x: %d wrong", bad_up);
    CHECK(bad_pool == 0, "maxpool k3: %d wrong", bad_pool);
    /* fill the pooled tensor with 3.0 (fp16 0x4200) */
    CHECK(thin_fill(&p, 3.0, 0, s) == THIN_OK, "thin_fill: %s", thin_last_error());
    HIP(hipStreamSynchronize(s));
    HIP(hipMemcpy(hp, dp, sizeof hp, hipMemcpyDeviceToHost));
    int bad_fill = 0;
    for (int i = 0; i < 4 * H * W * 16; ++i) bad_fill += hp[i] != 0x4200u;
    CHECK(bad_fill == 0, "fill: %d wrong", bad_fill);
    /* an even pool kernel is rejected */
    CHECK(thin_maxpool_nc1hwc0(&y, 4, &p, s) == THIN_ERR_INVALID, "maxpool k4 not rejected");
    HIP(hipFree(dx));
    HIP(hipFree(dy));
    HIP(hipFree(dp));
  }

  HIP(hipStreamDestroy(s));
  if (failures) {
    printf("%d check(s) failed\n", failures);
    return 1;
  }
  printf("capi selftest ok\n");
  return 0;
}
