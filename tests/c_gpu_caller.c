/* A plain C99 program that runs libhprms.so on the GPU through its C ABI
 * alone: HIP runtime calls for device memory and a stream, no torch and no
 * Python.  Each case fills seeded inputs on the host, runs one entry point,
 * copies the results back and checks them against the CPU oracle
 * (oracle/libhprms_oracle.so, test infrastructure): residuals and the
 * streamer's output bit for bit, normalised outputs within 1 ulp.
 * Built by hp_rms_norm_amd/build.py (gcc) and run by tests/test_gpu_c_caller.py.
 * Prints one line per case, then "ok"; exits 1 on a mismatch, 2 on a HIP or
 * library error. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "hp_rms_norm_amd.h"

/* the oracle's entry points (oracle/hprms_oracle.c) */
int hprms_oracle_fused_add_rmsnorm(uint16_t* input, const uint16_t* weight, uint16_t* residual, int64_t rows,
                                   int64_t hidden, int64_t input_row_stride, int64_t residual_row_stride, int dtype,
                                   double eps, int threads, int mutation);
int hprms_oracle_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* weight, int64_t rows, int64_t hidden,
                         int64_t out_row_stride, int64_t in_row_stride, int dtype, double eps, int threads);
int hprms_oracle_streamer(uint16_t* out, const uint16_t* in, int64_t rows, int64_t hidden, int64_t out_row_stride,
                          int64_t in_row_stride, int dtype, int op, int threads);
uint16_t hprms_oracle_f32_to_bf16(float f);
uint16_t hprms_oracle_f32_to_f16(float f);
int hprms_oracle_max_threads(void);

#define HIP_CHECK(call)                                                          \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));         \
      exit(2);                                                                   \
    }                                                                            \
  } while (0)
#define HPRMS_CHECK(call)                                                        \
  do {                                                                           \
    int rc_ = (call);                                                            \
    if (rc_ != HPRMS_OK) {                                                       \
      fprintf(stderr, "%s failed: %s (%d)\n", #call, hprms_last_error(), rc_);   \
      exit(2);                                                                   \
    }                                                                            \
  } while (0)

static uint64_t rng_state;
static double uniform(void) {
  rng_state = rng_state * 6364136223846793005ULL + 1442695040888963407ULL;
  return ((double)(rng_state >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
static float normal(void) { return (float)(sqrt(-2.0 * log(uniform())) * cos(6.283185307179586 * uniform())); }
static uint16_t to16(float f, int dtype) {
  return dtype == HPRMS_DTYPE_BF16 ? hprms_oracle_f32_to_bf16(f) : hprms_oracle_f32_to_f16(f);
}
static const char* dname(int dtype) { return dtype == HPRMS_DTYPE_BF16 ? "bf16" : "fp16"; }

/* ulps between two 16-bit floats of one format on the ordered line (-0 = +0);
 * NaN against NaN is 0, NaN against a number is far */
static int is_nan16(uint16_t h, int dtype) { return (h & 0x7fffu) > (dtype == HPRMS_DTYPE_BF16 ? 0x7f80u : 0x7c00u); }
static int64_t ulps16(uint16_t a, uint16_t b, int dtype) {
  if (is_nan16(a, dtype) || is_nan16(b, dtype)) return is_nan16(a, dtype) && is_nan16(b, dtype) ? 0 : 1 << 20;
  const int64_t oa = (a & 0x8000u) ? -(int64_t)(a & 0x7fffu) : (int64_t)(a & 0x7fffu);
  const int64_t ob = (b & 0x8000u) ? -(int64_t)(b & 0x7fffu) : (int64_t)(b & 0x7fffu);
  return oa > ob ? oa - ob : ob - oa;
}

static int failures = 0;

/* rows x hidden elements of got and want, at their row strides: the largest
 * ulp distance, and how many differ */
static int64_t compare(const uint16_t* got, int64_t gs, const uint16_t* want, int64_t ws, int64_t rows,
                       int64_t hidden, int dtype, int64_t* ndiff) {
  int64_t worst = 0;
  *ndiff = 0;
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < hidden; ++j) {
      const int64_t d = ulps16(got[i * gs + j], want[i * ws + j], dtype);
      if (d) ++*ndiff;
      if (d > worst) worst = d;
    }
  return worst;
}

static void report(const char* what, int64_t worst, int64_t ndiff, int64_t limit) {
  printf("  %s: max %lld ulp, %lld elements differ%s\n", what, (long long)worst, (long long)ndiff,
         worst > limit ? "  <-- FAIL" : "");
  if (worst > limit) ++failures;
}

static uint16_t* host16(int64_t n) {
  uint16_t* p = (uint16_t*)malloc((size_t)n * 2);
  if (!p) {
    fprintf(stderr, "out of host memory\n");
    exit(2);
  }
  return p;
}
static void* dev(size_t bytes) {
  void* p = NULL;
  HIP_CHECK(hipMalloc(&p, bytes));
  return p;
}
static void fill(uint16_t* p, int64_t n, float mean, float sd, int dtype) {
  for (int64_t i = 0; i < n; ++i) p[i] = to16(mean + sd * normal(), dtype);
}

/* the fused op in place; input and residual rows at strides si, sr */
static void case_fused(hipStream_t st, int64_t rows, int64_t hidden, int64_t si, int64_t sr, int dtype,
                       uint64_t seed) {
  rng_state = seed;
  uint16_t *x = host16(rows * si), *r = host16(rows * sr), *w = host16(hidden);
  uint16_t *gx = host16(rows * si), *gr = host16(rows * sr);
  fill(x, rows * si, 0.f, 1.f, dtype);
  fill(r, rows * sr, 0.f, 1.f, dtype);
  fill(w, hidden, 1.f, 0.1f, dtype);
  void *dx = dev((size_t)(rows * si * 2)), *dr = dev((size_t)(rows * sr * 2)), *dw = dev((size_t)hidden * 2);
  HIP_CHECK(hipMemcpy(dx, x, (size_t)(rows * si * 2), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dr, r, (size_t)(rows * sr * 2), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dw, w, (size_t)hidden * 2, hipMemcpyHostToDevice));
  printf("case fused_add_rmsnorm %lldx%lld %s (row strides %lld, %lld)\n", (long long)rows, (long long)hidden,
         dname(dtype), (long long)si, (long long)sr);
  fflush(stdout);
  HPRMS_CHECK(hprms_fused_add_rmsnorm(dx, dw, dr, rows, hidden, si, sr, dtype, 1e-6, st));
  HIP_CHECK(hipStreamSynchronize(st));
  HIP_CHECK(hipMemcpy(gx, dx, (size_t)(rows * si * 2), hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(gr, dr, (size_t)(rows * sr * 2), hipMemcpyDeviceToHost));
  if (hprms_oracle_fused_add_rmsnorm(x, w, r, rows, hidden, si, sr, dtype, 1e-6, hprms_oracle_max_threads(), 0)) {
    fprintf(stderr, "oracle refused the case\n");
    exit(2);
  }
  int64_t n;
  int64_t worst = compare(gr, sr, r, sr, rows, hidden, dtype, &n);
  report("residual", worst, n, 0);
  worst = compare(gx, si, x, si, rows, hidden, dtype, &n);
  report("output", worst, n, 1);
  HIP_CHECK(hipFree(dx));
  HIP_CHECK(hipFree(dr));
  HIP_CHECK(hipFree(dw));
  free(x), free(r), free(w), free(gx), free(gr);
}

/* plain RMSNorm out of place, and the fused op out of place */
static void case_plain_and_out(hipStream_t st, int64_t rows, int64_t hidden, int dtype, uint64_t seed) {
  rng_state = seed;
  const int64_t n = rows * hidden;
  uint16_t *x = host16(n), *r = host16(n), *w = host16(hidden), *o = host16(n), *ro = host16(n);
  fill(x, n, 0.f, 1.f, dtype);
  fill(r, n, 0.f, 1.f, dtype);
  fill(w, hidden, 1.f, 0.1f, dtype);
  void *dx = dev((size_t)n * 2), *dr = dev((size_t)n * 2), *dw = dev((size_t)hidden * 2);
  void *dout = dev((size_t)n * 2), *dro = dev((size_t)n * 2);
  HIP_CHECK(hipMemcpy(dx, x, (size_t)n * 2, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dr, r, (size_t)n * 2, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(dw, w, (size_t)hidden * 2, hipMemcpyHostToDevice));
  printf("case rmsnorm %lldx%lld %s\n", (long long)rows, (long long)hidden, dname(dtype));
  fflush(stdout);
  HPRMS_CHECK(hprms_rmsnorm(dout, dx, dw, rows, hidden, hidden, hidden, dtype, 1e-6, st));
  HIP_CHECK(hipStreamSynchronize(st));
  HIP_CHECK(hipMemcpy(o, dout, (size_t)n * 2, hipMemcpyDeviceToHost));
  uint16_t* want = host16(n);
  hprms_oracle_rmsnorm(want, x, w, rows, hidden, hidden, hidden, dtype, 1e-6, hprms_oracle_max_threads());
  int64_t nd;
  int64_t worst = compare(o, hidden, want, hidden, rows, hidden, dtype, &nd);
  report("output", worst, nd, 1);

  printf("case fused_add_rmsnorm_out %lldx%lld %s\n", (long long)rows, (long long)hidden, dname(dtype));
  fflush(stdout);
  HPRMS_CHECK(hprms_fused_add_rmsnorm_out(dout, dro, dx, dr, dw, rows, hidden, hidden, hidden, hidden, hidden, dtype,
                                          1e-6, st));
  HIP_CHECK(hipStreamSynchronize(st));
  HIP_CHECK(hipMemcpy(o, dout, (size_t)n * 2, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(ro, dro, (size_t)n * 2, hipMemcpyDeviceToHost));
  uint16_t* gx = host16(n);
  HIP_CHECK(hipMemcpy(gx, dx, (size_t)n * 2, hipMemcpyDeviceToHost));
  worst = compare(gx, hidden, x, hidden, rows, hidden, dtype, &nd);
  report("input untouched", worst, nd, 0);
  hprms_oracle_fused_add_rmsnorm(x, w, r, rows, hidden, hidden, hidden, dtype, 1e-6, hprms_oracle_max_threads(), 0);
  worst = compare(ro, hidden, r, hidden, rows, hidden, dtype, &nd);
  report("residual output", worst, nd, 0);
  worst = compare(o, hidden, x, hidden, rows, hidden, dtype, &nd);
  report("output", worst, nd, 1);
  HIP_CHECK(hipFree(dx));
  HIP_CHECK(hipFree(dr));
  HIP_CHECK(hipFree(dw));
  HIP_CHECK(hipFree(dout));
  HIP_CHECK(hipFree(dro));
  free(x), free(r), free(w), free(o), free(ro), free(want), free(gx);
}

/* the streamer (op 0: the reference's copying relu; op 1: a true ReLU) */
static void case_streamer(hipStream_t st, int64_t rows, int64_t hidden, int dtype, int op, uint64_t seed) {
  rng_state = seed;
  const int64_t n = rows * hidden;
  uint16_t *x = host16(n), *o = host16(n), *want = host16(n);
  fill(x, n, 0.f, 1.f, dtype);
  void *dx = dev((size_t)n * 2), *dout = dev((size_t)n * 2);
  HIP_CHECK(hipMemcpy(dx, x, (size_t)n * 2, hipMemcpyHostToDevice));
  printf("case streamer op %d %lldx%lld %s\n", op, (long long)rows, (long long)hidden, dname(dtype));
  fflush(stdout);
  HPRMS_CHECK(hprms_streamer(dout, dx, rows, hidden, hidden, hidden, dtype, op, st));
  HIP_CHECK(hipStreamSynchronize(st));
  HIP_CHECK(hipMemcpy(o, dout, (size_t)n * 2, hipMemcpyDeviceToHost));
  hprms_oracle_streamer(want, x, rows, hidden, hidden, hidden, dtype, op, hprms_oracle_max_threads());
  int64_t nd;
  const int64_t worst = compare(o, hidden, want, hidden, rows, hidden, dtype, &nd);
  report("output", worst, nd, 0);
  HIP_CHECK(hipFree(dx));
  HIP_CHECK(hipFree(dout));
  free(x), free(o), free(want);
}

int main(void) {
  int ndev = 0;
  HIP_CHECK(hipGetDeviceCount(&ndev));
  if (ndev < 1) {
    fprintf(stderr, "no HIP device\n");
    return 2;
  }
  HIP_CHECK(hipSetDevice(0));
  hipStream_t st;
  HIP_CHECK(hipStreamCreate(&st));
  printf("abi version %d, %d CUs\n", hprms_abi_version(), hprms_device_cu_count(0));
  case_fused(st, 4096, 4096, 4096, 4096, HPRMS_DTYPE_BF16, 1);   /* C1 */
  case_fused(st, 4096, 5120, 5120, 5120, HPRMS_DTYPE_FP16, 2);   /* C5 */
  case_fused(st, 7, 8192, 8192, 8192, HPRMS_DTYPE_BF16, 3);      /* a decode batch */
  case_fused(st, 300, 1000, 1003, 1010, HPRMS_DTYPE_BF16, 4);    /* rows off the 16-byte grid, odd strides */
  case_plain_and_out(st, 64, 2048, HPRMS_DTYPE_BF16, 5);
  case_streamer(st, 4096, 14336, HPRMS_DTYPE_BF16, 0, 6);         /* the streamer's benchmark shape */
  case_streamer(st, 37, 999, HPRMS_DTYPE_FP16, 1, 7);
  HIP_CHECK(hipStreamDestroy(st));
  if (failures) {
    printf("%d checks failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
