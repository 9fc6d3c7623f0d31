/*
 * hprms_oracle.c - CPU restatement of hp_rms_norm's fused residual-add + RMSNorm
 * path and of its streamer.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product (hp_rms_norm_amd, libhprms.so) never
 * links, loads or calls it.
 *
 * Algorithm followed (paths under the reference repository):
 *   - the reference's own test oracle, test/test_hp_rms_norm.py:6-19:
 *       inp_res = inp + res                         (bf16/fp16 tensor add)
 *       out = torch.rms_norm(inp_res, (H,), weight, eps)
 *   - the in-place contract of the op: residual <- inp_res, input <- out
 *     (hp_rms_norm/csrc/cuda/hp_rms_norm.cuh:207,251; hp_rms_norm/ops.py:4-15)
 *   - the streamer's observable behaviour, an identity copy
 *     (hp_rms_norm/csrc/cuda/activation_kernels.cuh:99-119, test/test_relu.py:24)
 *
 * Arithmetic, element by element, in IEEE binary32 with round-to-nearest-even:
 *   s   = rne16(f32(x) + f32(r))                 stored to residual
 *   ms  = fp32 mean of f32(s)^2 over the row     (each square a binary32
 *                                                 product, summed in binary64,
 *                                                 then rounded once to
 *                                                 binary32: no reduction-order
 *                                                 error; a sum past binary32's
 *                                                 range is +inf, see mean_square)
 *   inv = 1 / sqrt(ms + (float)eps)              two correctly rounded ops
 *   out = rne16((f32(s) * inv) * f32(w))          stored to input
 * The 16-bit conversions below are written from the IEEE 754 definitions
 * (bfloat16 = the top half of a binary32; binary16 with subnormals).
 *
 * With the FP8 output (hprms_oracle_fused_add_rmsnorm_fp8) the 16-bit output
 * y is quantised per row: scale = max(amax|y| / 448, FLT_MIN),
 * q = e4m3fn(clamp(y * (1 / scale), +-448)); this is the composition of the op
 * with per-token dynamic FP8 quantisation as torch evaluates it.
 *
 * The partial-sum form (hprms_oracle_reduce_add_rmsnorm) first forms
 * a = rne16(((f32(p0) + f32(p1)) + ...) + f32(p[P-1])), summed in binary32 in
 * part order and rounded once (an all-reduce of the parts), then applies the
 * fused op to a with the output written to `out`.  It has no counterpart in
 * the reference; with P = 1 it is the fused op.
 *
 * The MX forms (hprms_oracle_fused_add_rmsnorm_mx) quantise the 16-bit
 * output y in blocks of 32 consecutive elements of a row, as the OCP
 * Microscaling Formats (MX) v1.0 specification defines it: scale exponent
 * s = floor(log2(max |y| over the block)) - emax (emax = 8 for E4M3 elements,
 * 2 for E2M1), clamped to [-127, 127] and stored as E8M0 (s + 127; 0xFF when
 * the block holds a NaN or an infinity); elements = y / 2^s rounded to nearest
 * even in the element format, saturated to its largest normal (448 / 6).  E2M1
 * codes pack two to a byte, the even element in the low nibble.
 *
 * Parity pins (tests/test_oracle.py): golden vectors made by the reference's
 * own formula in torch (tests/golden/), the live torch formula on ordinary
 * rows and on rows of special values (NaN, infinities, zero rows with
 * eps = 0, binary32 overflow of the squares and of their sum, subnormals), a
 * binary64 brute force, closed forms (constant rows, power-of-two scaling),
 * numpy's binary16 conversion, and planted mistakes (the `mutation`
 * argument) that the pins must reject.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_BF16 0
#define ORACLE_FP16 1

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- 16-bit <-> binary32 conversions --------------------------------------- */

float hprms_oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round-to-nearest-even of a binary32 to bfloat16.  NaN -> 0x7FC0. */
uint16_t hprms_oracle_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float hprms_oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));   /* inf / NaN */
  if (e == 0) {                                                /* zero / subnormal: m * 2^-24 */
    float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Round-to-nearest-even of a binary32 to binary16, with subnormals and
 * overflow to infinity.  NaN -> 0x7E00 with the input's sign. */
uint16_t hprms_oracle_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7E00;
  if (a >= 0x477FF000u) return sign | 0x7C00;      /* |f| >= 65520 rounds to inf */
  if (a >= 0x38800000u) {                          /* normal result, |f| >= 2^-14 */
    uint32_t t = a - 0x38000000u;                  /* rebias 127 -> 15 */
    t += 0xFFFu + ((t >> 13) & 1u);
    return sign | (uint16_t)(t >> 13);
  }
  if (a <= 0x33000000u) return sign;               /* |f| <= 2^-25 rounds to 0 */
  /* subnormal result: round(mant * 2^(e-150) / 2^-24) */
  uint32_t e = a >> 23;
  uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  uint32_t shift = 126u - e;                       /* 14 .. 24 */
  uint32_t q = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  return sign | (uint16_t)q;
}

static inline float to_f32(uint16_t h, int dtype) {
  return dtype == ORACLE_BF16 ? hprms_oracle_bf16_to_f32(h) : hprms_oracle_f16_to_f32(h);
}
static inline uint16_t from_f32(float f, int dtype) {
  return dtype == ORACLE_BF16 ? hprms_oracle_f32_to_bf16(f) : hprms_oracle_f32_to_f16(f);
}
/* rounding by truncation: only for the planted-mistake mode */
static inline uint16_t from_f32_trunc(float f, int dtype) {
  if (dtype == ORACLE_BF16) return (uint16_t)(f2u(f) >> 16);
  return hprms_oracle_f32_to_f16(u2f(f2u(f) & 0xffffe000u));
}

/* ---- planted mistakes (tests only; 0 = the algorithm) ---------------------- */
enum {
  MUT_NONE = 0,
  MUT_DROP_EPS = 1,        /* rsqrt(mean) */
  MUT_MEAN_H_MINUS_1 = 2,  /* divide the sum of squares by H-1 */
  MUT_WEIGHT_REVERSED = 3, /* weight[H-1-j] */
  MUT_TRUNC_RESIDUAL = 4,  /* residual rounded by truncation */
  MUT_NORM_INPUT = 5,      /* normalise the pre-add input instead of the sum */
  MUT_L1_MEAN = 6,         /* mean of |s| instead of s^2 (then squared) */
  MUT_UNROUNDED_SQUARES = 7, /* squares of the unrounded fp32 sum (the reference kernel's order) */
  MUT_WEIGHT_TWICE = 8,    /* (s * inv) * w * w */
  MUT_BINARY64_SQUARES = 9 /* squares and mean in binary64: no binary32 overflow */
};

static int check_rows(int64_t rows, int64_t hidden, int64_t s0, int64_t s1) {
  return rows >= 0 && hidden >= 1 && s0 >= hidden && s1 >= hidden;
}

/* The mean of a row's squares as the reference's formula forms it in
 * binary32 (test/test_hp_rms_norm.py:13-18: torch.rms_norm upcasts the row
 * to fp32 and takes the mean of its squares).  The caller adds each square
 * as a binary32 product, which is exact for 16-bit inputs unless it
 * overflows to +inf or falls below the normal range, where it rounds as
 * binary32 does.  sum_sq is their sum in binary64, free of reduction-order
 * error.  A sum past binary32's range is +inf, as any binary32 summation of
 * the same squares gives (a row of 256 values of 3e18 has finite squares
 * and an infinite fp32 sum); otherwise the mean is rounded once. */
static inline float mean_square(double sum_sq, double n) {
  if (isinf((float)sum_sq)) return INFINITY;
  return (float)(sum_sq / n);
}

/* One row of the fused op.  x: input row (overwritten with the output),
 * r: residual row (overwritten with the rounded sum). */
static void fused_row(uint16_t* x, const uint16_t* w, uint16_t* r, int64_t H,
                      int dtype, float epsf, int mutation) {
  double acc = 0.0;
  for (int64_t j = 0; j < H; ++j) {
    float sum = to_f32(x[j], dtype) + to_f32(r[j], dtype);
    uint16_t s = mutation == MUT_TRUNC_RESIDUAL ? from_f32_trunc(sum, dtype) : from_f32(sum, dtype);
    float sf = to_f32(s, dtype);
    if (mutation == MUT_UNROUNDED_SQUARES) sf = sum;
    if (mutation == MUT_NORM_INPUT) sf = to_f32(x[j], dtype);
    if (mutation == MUT_L1_MEAN) acc += fabs((double)sf);
    else if (mutation == MUT_BINARY64_SQUARES) acc += (double)sf * (double)sf;
    else acc += (double)(sf * sf);
    r[j] = s;
  }
  if (mutation == MUT_L1_MEAN) acc = (acc / (double)H) * (acc / (double)H) * (double)H;
  double denom = mutation == MUT_MEAN_H_MINUS_1 && H > 1 ? (double)(H - 1) : (double)H;
  float ms = mutation == MUT_BINARY64_SQUARES ? (float)(acc / denom) : mean_square(acc, denom);
  float v = mutation == MUT_DROP_EPS ? ms : ms + epsf;
  float inv = 1.0f / sqrtf(v);
  for (int64_t j = 0; j < H; ++j) {
    float sf = to_f32(mutation == MUT_NORM_INPUT ? x[j] : r[j], dtype);
    float wf = to_f32(w[mutation == MUT_WEIGHT_REVERSED ? H - 1 - j : j], dtype);
    float y = (sf * inv) * wf;
    if (mutation == MUT_WEIGHT_TWICE) y = y * wf;
    x[j] = from_f32(y, dtype);
  }
}

/* Fused residual-add + RMSNorm over [rows, hidden], in place.
 * Returns 0, or -22 on a bad argument. */
int hprms_oracle_fused_add_rmsnorm(uint16_t* input, const uint16_t* weight, uint16_t* residual,
                                   int64_t rows, int64_t hidden,
                                   int64_t input_row_stride, int64_t residual_row_stride,
                                   int dtype, double eps, int threads, int mutation) {
  if (!check_rows(rows, hidden, input_row_stride, residual_row_stride)) return -22;
  if (dtype != ORACLE_BF16 && dtype != ORACLE_FP16) return -22;
  if (rows == 0) return 0;
  if (!input || !weight || !residual) return -22;
  float epsf = (float)eps;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i)
    fused_row(input + i * input_row_stride, weight, residual + i * residual_row_stride,
              hidden, dtype, epsf, mutation);
  (void)threads;
  return 0;
}

/* Plain RMSNorm, out = rne16((f32(in) * inv) * f32(w)); out may equal in. */
int hprms_oracle_rmsnorm(uint16_t* out, const uint16_t* in, const uint16_t* weight,
                         int64_t rows, int64_t hidden, int64_t out_row_stride,
                         int64_t in_row_stride, int dtype, double eps, int threads) {
  if (!check_rows(rows, hidden, out_row_stride, in_row_stride)) return -22;
  if (dtype != ORACLE_BF16 && dtype != ORACLE_FP16) return -22;
  if (rows == 0) return 0;
  if (!out || !in || !weight) return -22;
  float epsf = (float)eps;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i) {
    const uint16_t* x = in + i * in_row_stride;
    uint16_t* o = out + i * out_row_stride;
    double acc = 0.0;
    for (int64_t j = 0; j < hidden; ++j) {
      float v = to_f32(x[j], dtype);
      acc += (double)(v * v);
    }
    float inv = 1.0f / sqrtf(mean_square(acc, (double)hidden) + epsf);
    for (int64_t j = 0; j < hidden; ++j)
      o[j] = from_f32((to_f32(x[j], dtype) * inv) * to_f32(weight[j], dtype), dtype);
  }
  (void)threads;
  return 0;
}

/* Streamer: op 0 = identity copy, op 1 = ReLU: strictly negative values
 * (sign set, nonzero magnitude, not NaN) become +0; -0, NaN and everything
 * else pass through unchanged, as torch.relu does. */
int hprms_oracle_streamer(uint16_t* out, const uint16_t* in, int64_t rows, int64_t hidden,
                          int64_t out_row_stride, int64_t in_row_stride, int dtype, int op,
                          int threads) {
  if (!check_rows(rows, hidden, out_row_stride, in_row_stride)) return -22;
  if ((dtype != ORACLE_BF16 && dtype != ORACLE_FP16) || (op != 0 && op != 1)) return -22;
  if (rows == 0) return 0;
  if (!out || !in) return -22;
  uint16_t nan_floor = dtype == ORACLE_BF16 ? 0x7f80u : 0x7c00u; /* |h| above this is NaN */
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i) {
    const uint16_t* x = in + i * in_row_stride;
    uint16_t* o = out + i * out_row_stride;
    for (int64_t j = 0; j < hidden; ++j) {
      uint16_t h = x[j];
      if (op == 1 && (h & 0x8000u) && (h & 0x7fffu) != 0 && (h & 0x7fffu) <= nan_floor) h = 0;
      o[j] = h;
    }
  }
  (void)threads;
  return 0;
}

int hprms_oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---- FP8 (OCP e4m3fn) quantised output ---------------------------------------- */

/* Round-to-nearest-even of a binary32 to OCP FP8 e4m3fn (bias 7, 3 mantissa
 * bits, subnormals m * 2^-9, no infinities, 0x7F / 0xFF = NaN, max 448).  Not
 * saturating: magnitudes that round past 448 become NaN, as torch's
 * float8_e4m3fn conversion does; callers clamp first. */
uint8_t hprms_oracle_f32_to_e4m3(float f) {
  uint32_t u = f2u(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x43E80000u) return sign | 0x7F;          /* NaN, inf, or rounds past 448 */
  if (a >= 0x3C800000u) {                           /* normal result, |f| >= 2^-6 */
    uint32_t t = a - 0x3C000000u;                   /* rebias 127 -> 7 */
    t += 0x7FFFFu + ((t >> 20) & 1u);
    return sign | (uint8_t)(t >> 20);
  }
  if (a <= 0x3A800000u) return sign;                /* |f| <= 2^-10 rounds to 0 */
  uint32_t e = a >> 23;                             /* subnormal: round(|f| / 2^-9) */
  uint32_t mant = (a & 0x7fffffu) | 0x800000u;
  uint32_t shift = 141u - e;                        /* 21 .. 24 */
  uint32_t q = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  return sign | (uint8_t)q;
}

float hprms_oracle_e4m3_to_f32(uint8_t h) {
  float sgn = (h & 0x80) ? -1.0f : 1.0f;
  uint32_t e = (h >> 3) & 0xFu, m = h & 7u;
  if (e == 0xF && m == 7) return sgn * NAN;
  if (e == 0) return sgn * (float)m * 0.001953125f;            /* m * 2^-9 */
  return sgn * ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
}

/* Fused residual-add + RMSNorm with a per-row FP8 output (the op's 16-bit
 * output y, then dynamic per-token quantisation):
 *   residual <- rne16(x + r)                      (in place; input untouched)
 *   y        = the 16-bit output of the fused op  (as above)
 *   amax     = max |y| over the row               (NaN if any y is NaN)
 *   scale    = max(amax / 448, FLT_MIN)           -> scale[row]
 *   q        = e4m3fn(clamp(y * (1 / scale), -448, 448)) -> q[row, :]
 * q has its own row stride in bytes (elements). */
int hprms_oracle_fused_add_rmsnorm_fp8(uint8_t* q, float* scale, const uint16_t* input,
                                       const uint16_t* weight, uint16_t* residual,
                                       int64_t rows, int64_t hidden, int64_t q_row_stride,
                                       int64_t input_row_stride, int64_t residual_row_stride,
                                       int dtype, double eps, int threads) {
  if (!check_rows(rows, hidden, input_row_stride, residual_row_stride) || q_row_stride < hidden) return -22;
  if (dtype != ORACLE_BF16 && dtype != ORACLE_FP16) return -22;
  if (rows == 0) return 0;
  if (!q || !scale || !input || !weight || !residual) return -22;
  float epsf = (float)eps;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i) {
    const uint16_t* xr = input + i * input_row_stride;
    uint16_t* rr = residual + i * residual_row_stride;
    uint8_t* qr = q + i * q_row_stride;
    uint16_t* y = (uint16_t*)malloc((size_t)hidden * sizeof(uint16_t));
    if (!y) continue;
    for (int64_t j = 0; j < hidden; ++j) y[j] = xr[j];
    fused_row(y, weight, rr, hidden, dtype, epsf, MUT_NONE);
    float amax = 0.0f;
    int nan = 0;
    for (int64_t j = 0; j < hidden; ++j) {
      float v = fabsf(to_f32(y[j], dtype));
      if (v != v) nan = 1;
      else if (v > amax) amax = v;
    }
    float sc = nan ? NAN : amax / 448.0f;
    if (sc < FLT_MIN) sc = FLT_MIN;                 /* NaN compares false and stays */
    float inv = 1.0f / sc;
    scale[i] = sc;
    for (int64_t j = 0; j < hidden; ++j) {
      float v = to_f32(y[j], dtype) * inv;
      v = v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
      qr[j] = hprms_oracle_f32_to_e4m3(v);
    }
    free(y);
  }
  (void)threads;
  return 0;
}

/* planted mistakes of the partial-sum step (tests only; 0 = the algorithm) */
enum {
  RMUT_STEP_ROUNDING = 1, /* round to 16 bits after every addition (a ring all-reduce in bf16) */
  RMUT_NO_ROUNDING = 2,   /* add the residual to the unrounded fp32 sum */
  RMUT_REVERSED = 3       /* sum the parts in reverse order */
};

/* Partial-sum reduction + fused op: out[r] = fused output of a = rne16(sum of
 * the parts), residual <- rne16(a + residual).  The parts share one row
 * stride; out has its own.  Returns 0, or -22 on a bad argument. */
int hprms_oracle_reduce_add_rmsnorm(uint16_t* out, const uint16_t* const* parts, int nparts,
                                    const uint16_t* weight, uint16_t* residual, int64_t rows,
                                    int64_t hidden, int64_t out_row_stride, int64_t part_row_stride,
                                    int64_t residual_row_stride, int dtype, double eps, int threads,
                                    int mutation) {
  if (!check_rows(rows, hidden, out_row_stride, residual_row_stride) || part_row_stride < hidden) return -22;
  if ((dtype != ORACLE_BF16 && dtype != ORACLE_FP16) || nparts < 1) return -22;
  if (rows == 0) return 0;
  if (!out || !parts || !weight || !residual) return -22;
  for (int g = 0; g < nparts; ++g)
    if (!parts[g]) return -22;
  float epsf = (float)eps;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i) {
    uint16_t* o = out + i * out_row_stride;
    uint16_t* rr = residual + i * residual_row_stride;
    const int64_t off = i * part_row_stride;
    for (int64_t j = 0; j < hidden; ++j) {
      const int first = mutation == RMUT_REVERSED ? nparts - 1 : 0;
      float acc = to_f32(parts[first][off + j], dtype);
      for (int t = 1; t < nparts; ++t) {
        const int g = mutation == RMUT_REVERSED ? nparts - 1 - t : t;
        acc = acc + to_f32(parts[g][off + j], dtype);
        if (mutation == RMUT_STEP_ROUNDING) acc = to_f32(from_f32(acc, dtype), dtype);
      }
      if (mutation == RMUT_NO_ROUNDING) {
        /* fold the residual into the unrounded sum; fused_row then adds 0 */
        acc = acc + to_f32(rr[j], dtype);
        rr[j] = 0;
      }
      o[j] = from_f32(acc, dtype);
    }
    fused_row(o, weight, rr, hidden, dtype, epsf, MUT_NONE);
  }
  (void)threads;
  return 0;
}

/* ---- OCP MX block formats ------------------------------------------------ */

/* E2M1 magnitudes by code: 0, 0.5, 1, 1.5, 2, 3, 4, 6. */
static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

/* binary32 -> E2M1 code (sign in bit 3): the nearest magnitude, ties to the
 * even code, saturating at 6.  E2M1 has no NaN (an MX block marks NaN in its
 * scale); NaN is given the largest code with NaN's sign, as the gfx950
 * conversion instruction gives it. */
uint8_t hprms_oracle_f32_to_e2m1(float f) {
  uint8_t sign = (f2u(f) >> 31) ? 8u : 0u;
  float a = fabsf(f);
  if (a != a) return (uint8_t)(sign | 7);
  if (a >= 6.0f) return (uint8_t)(sign | 7);  /* saturation, infinity included */
  int best = 0;
  float bd = INFINITY;
  for (int c = 0; c < 8; ++c) {
    float d = fabsf(a - kE2M1[c]);
    if (d < bd || (d == bd && (c & 1) == 0)) {
      bd = d;
      best = c;
    }
  }
  return (uint8_t)(sign | best);
}

float hprms_oracle_e2m1_to_f32(uint8_t c) {
  float v = kE2M1[c & 7];
  return (c & 8) ? -v : v;
}

/* planted mistakes of the MX step (tests only; 0 = the algorithm) */
enum {
  XMUT_CEIL_SCALE = 1,   /* ceil(log2 amax) instead of floor */
  XMUT_EMAX_PLUS_1 = 2,  /* emax one too large */
  XMUT_TRUNCATE = 3,     /* elements truncated instead of rounded */
  XMUT_NIBBLES = 4       /* E2M1: odd element in the low nibble */
};

/* E8M0 scale exponent of a block from its largest magnitude; returns 128 for
 * NaN / infinity (encoded 0xFF). */
static int mx_scale_exp(float amax, int emax, int mutation) {
  if (amax != amax || isinf(amax)) return 128;
  if (amax == 0.0f) return -127;
  int e;
  float m = frexpf(amax, &e);           /* amax = m * 2^e, m in [0.5, 1) */
  int fl = e - 1;                       /* floor(log2(amax)) */
  if (mutation == XMUT_CEIL_SCALE && m != 0.5f) fl = e;
  int s = fl - (mutation == XMUT_EMAX_PLUS_1 ? emax + 1 : emax);
  if (s < -127) s = -127;
  if (s > 127) s = 127;
  return s;
}

/* The MX step on rows of 16-bit values y: scales[b] (E8M0) and q for each
 * block of 32.  elem 0 = MXFP8 (one E4M3 byte per element), elem 1 = MXFP4
 * (two E2M1 codes per byte, the even element in the low nibble). */
static void mx_quantize_row(const uint16_t* y, int64_t hidden, int elem, int dtype, uint8_t* qr, uint8_t* sr,
                            int mutation) {
  const int emax = elem == 0 ? 8 : 2;
  for (int64_t b = 0; b < hidden / 32; ++b) {
    float amax = 0.0f;
    int nan = 0;
    for (int j = 0; j < 32; ++j) {
      float v = fabsf(to_f32(y[b * 32 + j], dtype));
      if (v != v) nan = 1;
      else if (v > amax) amax = v;
    }
    int s = mx_scale_exp(nan ? NAN : amax, emax, mutation);
    sr[b] = (uint8_t)(s == 128 ? 0xFF : s + 127);
    for (int j = 0; j < 32; ++j) {
      /* a NaN block keeps its values unscaled; the 0xFF scale marks it */
      float v = s == 128 ? to_f32(y[b * 32 + j], dtype) : ldexpf(to_f32(y[b * 32 + j], dtype), -s);
      int64_t col = b * 32 + j;
      if (elem == 0) {
        if (mutation == XMUT_TRUNCATE) v = truncf(v * 8.0f) / 8.0f;
        v = v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
        qr[col] = hprms_oracle_f32_to_e4m3(v);
      } else {
        if (mutation == XMUT_TRUNCATE) v = (v < 0 ? -1.0f : 1.0f) * floorf(fabsf(v) * 2.0f) / 2.0f;
        uint8_t c = hprms_oracle_f32_to_e2m1(v);
        int hi = (int)(col & 1) ^ (mutation == XMUT_NIBBLES);
        uint8_t* dst = &qr[col / 2];
        if (hi) *dst = (uint8_t)((*dst & 0x0F) | (c << 4));
        else *dst = (uint8_t)((*dst & 0xF0) | c);
      }
    }
  }
}

/* The MX step alone, on [rows, hidden] 16-bit values (contiguous rows). */
int hprms_oracle_mx_quantize(uint8_t* q, uint8_t* scales, const uint16_t* y, int64_t rows, int64_t hidden,
                             int elem, int dtype, int mutation) {
  if (rows < 0 || hidden < 32 || hidden % 32 || (elem != 0 && elem != 1)) return -22;
  if (dtype != ORACLE_BF16 && dtype != ORACLE_FP16) return -22;
  const int64_t qw = elem == 0 ? hidden : hidden / 2;
  for (int64_t i = 0; i < rows; ++i)
    mx_quantize_row(y + i * hidden, hidden, elem, dtype, q + i * qw, scales + i * (hidden / 32), mutation);
  return 0;
}

/* Fused op with an OCP MX output (the step above applied to the fused op's
 * 16-bit output).  q has q_row_stride bytes per row, scales
 * scale_row_stride bytes per row (hidden / 32 used).  The residual is updated
 * in place; input is only read.  hidden % 32 == 0. */
int hprms_oracle_fused_add_rmsnorm_mx(uint8_t* q, uint8_t* scales, const uint16_t* input,
                                      const uint16_t* weight, uint16_t* residual, int64_t rows,
                                      int64_t hidden, int64_t q_row_stride, int64_t scale_row_stride,
                                      int64_t input_row_stride, int64_t residual_row_stride, int elem,
                                      int dtype, double eps, int threads, int mutation) {
  if (!check_rows(rows, hidden, input_row_stride, residual_row_stride)) return -22;
  if ((dtype != ORACLE_BF16 && dtype != ORACLE_FP16) || (elem != 0 && elem != 1) || hidden % 32) return -22;
  if (q_row_stride < (elem == 0 ? hidden : hidden / 2) || scale_row_stride < hidden / 32) return -22;
  if (rows == 0) return 0;
  if (!q || !scales || !input || !weight || !residual) return -22;
  float epsf = (float)eps;
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t i = 0; i < rows; ++i) {
    uint16_t* y = (uint16_t*)malloc((size_t)hidden * sizeof(uint16_t));
    if (!y) continue;
    memcpy(y, input + i * input_row_stride, (size_t)hidden * sizeof(uint16_t));
    fused_row(y, weight, residual + i * residual_row_stride, hidden, dtype, epsf, MUT_NONE);
    mx_quantize_row(y, hidden, elem, dtype, q + i * q_row_stride, scales + i * scale_row_stride, mutation);
    free(y);
  }
  (void)threads;
  return 0;
}

void hprms_oracle_e2m1_from_f32(const float* src, uint8_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = hprms_oracle_f32_to_e2m1(src[i]);
}

void hprms_oracle_e4m3_from_f32(const float* src, uint8_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = hprms_oracle_f32_to_e4m3(src[i]);
}

/* Array forms of the conversions, for the conversion pins. */
void hprms_oracle_from_f32(const float* src, uint16_t* dst, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) dst[i] = from_f32(src[i], dtype);
}
void hprms_oracle_to_f32(const uint16_t* src, float* dst, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) dst[i] = to_f32(src[i], dtype);
}
