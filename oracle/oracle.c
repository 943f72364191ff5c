/*
 * oracle.c -- CPU restatement of genovationtech/nve's quantized decode GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU baseline
 * of bench.py.  The product library never links or calls this file.
 *
 * Parity pins (tests/test_oracle.py), one line per function:
 *   orc_quantize_block_q4   hand-derived known answers (ties at k+0.5 under
 *                           half-away-from-zero, all-zero block, 1/scale = inf with
 *                           saturating casts, scale underflow to 0) and the
 *                           reference's own unit tests src/quantize.rs:2234-2252,
 *                           2274-2290 with their inputs and tolerances.
 *   orc_quantize_block_q4_weighted  hand-derived known answers (an importance-0
 *                           outlier makes the second candidate exact and win; a
 *                           single non-zero value reduces to orc_quantize_block_q4;
 *                           blocks below 1e-10 -> scale 0, nibbles 8) and brute force:
 *                           the chosen scale's weighted error, re-evaluated in
 *                           float64, is within rounding of the least over all 8
 *                           candidates, which are the 8 largest |v| (numpy sort).
 *   orc_q4_from_f32_awq     awq = 1 reduces to orc_q4_from_f32 (kquant 0) and to
 *                           the weighted quantizer with unit importance (kquant 1);
 *                           awq = 2^e scaling commutes exactly (scales x 2^e, same
 *                           nibbles); the reference unit test src/quantize.rs:2520-
 *                           2544 (uniform awq 1.5: matvec within 5.0 of the plain
 *                           one); inv_scales closed form incl. |s| <= 1e-10 -> 0.
 *   orc_q4_from_f32         |deq - w| <= scale/2 and nibble in [1,15] invariants
 *                           on random matrices; byte layout KAT.
 *   orc_q4_to_f32           KAT on one hand-packed block.
 *   orc_extract_for_gpu     brute-force bijection check against an independent
 *                           numpy unpacking of both orders.
 *   orc_q4_dot_row_scalar   numpy float64 dequant-dot on tiny shapes (tolerance)
 *                           and exact agreement with a float32 loop in the same
 *                           order written in numpy.
 *   orc_q4_dot_row_avx2     tolerance against the float64 dot; FMA/hsum order is
 *                           pinned only by following src/quantize.rs:883-938
 *                           (the rustc binary cannot be built here).
 *   orc_q4_matvec_f32       equals row-wise orc_q4_dot_row_* for every row and
 *                           thread count (row split must not change results).
 *   orc_quantize_q8_group   KATs: +-amax -> +-127, RNE ties (2.5 -> 2, 3.5 -> 4),
 *                           NaN / Inf groups (the fmaxf tree drops NaN, NaN codes
 *                           are 0, an infinite amax zeroes the group),
 *                           all-zero group -> scale 1, q 0; brute force with numpy
 *                           float32 ops.
 *   orc_quantize_q8_rows_bf16 same KAT family with a bf16 scale.
 *   orc_w4a8_block_acc      brute force from the CPU-order blocks (independent
 *                           unpacking) in numpy int64.
 *   orc_matvec_w4a8_f64     numpy float64 of sum_b ws*xs*acc from numpy's acc.
 *   orc_matvec_w4a16_f64    numpy float64 of (dequantized W from orc_q4_to_f32
 *                           applied to the CPU-order data) @ x.
 *   orc_use_w4a8            truth table over importance / threshold / env.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define Q4_BLOCK 32
#define Q4_BYTES 20

/* ------------------------------------------------------------------------ */
int8_t orc_rust_f32_as_i8(float v) {
  /* Rust float->int `as` casts saturate and map NaN to 0. */
  if (isnan(v)) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v; /* truncation toward zero, in range */
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while (!(man & 0x400u));
      man &= 0x3ffu;
      x = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (man << 13);
  } else {
    x = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
  int e = (int)exp - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t h = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t x = (uint32_t)h << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

/* ------------------------------------------------------------------------ */
/* src/quantize.rs:711-731 */
void orc_quantize_block_q4(const float *v, uint8_t *out) {
  float amax = 0.0f;
  for (int i = 0; i < Q4_BLOCK; i++) amax = fmaxf(amax, fabsf(v[i])); /* f32::max fold */
  float scale = amax > 0.0f ? amax / 7.0f : 0.0f;
  float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  memcpy(out, &scale, 4); /* little-endian host */
  for (int i = 0; i < 16; i++) {
    int8_t a = orc_rust_f32_as_i8(roundf(v[2 * i] * inv)); /* f32::round: half away */
    int8_t b = orc_rust_f32_as_i8(roundf(v[2 * i + 1] * inv));
    a = (int8_t)((a < -8 ? -8 : (a > 7 ? 7 : a)) + 8);
    b = (int8_t)((b < -8 ? -8 : (b > 7 ? 7 : b)) + 8);
    out[4 + i] = (uint8_t)((uint8_t)a | ((uint8_t)b << 4));
  }
}

/* src/quantize.rs:741-793: k-quant candidate search.  Candidates are the 8 largest
 * |v| in descending order (746-751; for finite inputs the order among equal values is
 * immaterial); the loop stops at the first candidate below 1e-10; the error is summed
 * in f32 as error += (imp * diff) * diff (no contraction: -ffp-contract=off). */
void orc_quantize_block_q4_weighted(const float *v, const float *imp, uint8_t *out) {
  float a[Q4_BLOCK];
  for (int i = 0; i < Q4_BLOCK; i++) a[i] = fabsf(v[i]);
  for (int i = 1; i < Q4_BLOCK; i++) { /* insertion sort, descending */
    float t = a[i];
    int j = i - 1;
    while (j >= 0 && a[j] < t) {
      a[j + 1] = a[j];
      j--;
    }
    a[j + 1] = t;
  }
  float best_scale = 0.0f, best_err = 3.40282347e38f; /* f32::MAX */
  for (int c = 0; c < 8; c++) {
    float amax = a[c];
    if (amax < 1e-10f) break;
    float cs = amax / 7.0f;
    float ci = 1.0f / cs;
    float err = 0.0f;
    for (int j = 0; j < Q4_BLOCK; j++) {
      int q = orc_rust_f32_as_i8(roundf(v[j] * ci));
      q = q < -8 ? -8 : (q > 7 ? 7 : q);
      float deq = (float)q * cs;
      float diff = v[j] - deq;
      err += imp[j] * diff * diff;
    }
    if (err < best_err) {
      best_err = err;
      best_scale = cs;
    }
  }
  float inv = best_scale > 0.0f ? 1.0f / best_scale : 0.0f;
  memcpy(out, &best_scale, 4);
  for (int i = 0; i < 16; i++) {
    int qa = orc_rust_f32_as_i8(roundf(v[2 * i] * inv));
    int qb = orc_rust_f32_as_i8(roundf(v[2 * i + 1] * inv));
    qa = (qa < -8 ? -8 : (qa > 7 ? 7 : qa)) + 8;
    qb = (qb < -8 ? -8 : (qb > 7 ? 7 : qb)) + 8;
    out[4 + i] = (uint8_t)((uint8_t)qa | ((uint8_t)qb << 4));
  }
}

/* src/quantize.rs:271-306 (kquant = 0) and 308-346 (kquant = 1): row_f32[j] *= awq[j],
 * then the plain or the weighted block quantizer (importance awq[j] * awq[j]);
 * inv_scales[j] = |awq[j]| > 1e-10 ? 1 / awq[j] : 0 (may be NULL). */
void orc_q4_from_f32_awq(const float *w, int64_t n, int64_t k, const float *awq, int kquant, uint8_t *data,
                         float *inv_scales) {
  int64_t bpr = k / Q4_BLOCK;
  float *row = (float *)malloc((size_t)k * sizeof(float));
  float *imp = (float *)malloc((size_t)k * sizeof(float));
  for (int64_t j = 0; j < k; j++) imp[j] = awq[j] * awq[j];
  for (int64_t r = 0; r < n; r++) {
    for (int64_t j = 0; j < k; j++) row[j] = w[r * k + j] * awq[j];
    for (int64_t b = 0; b < bpr; b++) {
      uint8_t *o = data + (r * bpr + b) * Q4_BYTES;
      if (kquant)
        orc_quantize_block_q4_weighted(row + b * Q4_BLOCK, imp + b * Q4_BLOCK, o);
      else
        orc_quantize_block_q4(row + b * Q4_BLOCK, o);
    }
  }
  free(row);
  free(imp);
  if (inv_scales)
    for (int64_t j = 0; j < k; j++) inv_scales[j] = fabsf(awq[j]) > 1e-10f ? 1.0f / awq[j] : 0.0f;
}

/* src/quantize.rs:347-375 */
void orc_q4_from_f32(const float *w, int64_t n, int64_t k, uint8_t *data) {
  int64_t bpr = k / Q4_BLOCK;
  for (int64_t r = 0; r < n; r++)
    for (int64_t b = 0; b < bpr; b++)
      orc_quantize_block_q4(w + r * k + b * Q4_BLOCK, data + (r * bpr + b) * Q4_BYTES);
}

/* src/quantize.rs:396-426 */
void orc_q4_to_f32(const uint8_t *data, int64_t n, int64_t k, const float *awq_inv,
                   float *out) {
  int64_t bpr = k / Q4_BLOCK;
  for (int64_t r = 0; r < n; r++) {
    for (int64_t b = 0; b < bpr; b++) {
      const uint8_t *blk = data + (r * bpr + b) * Q4_BYTES;
      float scale;
      memcpy(&scale, blk, 4);
      float *o = out + r * k + b * Q4_BLOCK;
      for (int i = 0; i < 16; i++) {
        int q0 = (blk[4 + i] & 0x0f) - 8;
        int q1 = ((blk[4 + i] >> 4) & 0x0f) - 8;
        o[2 * i] = (float)q0 * scale;
        o[2 * i + 1] = (float)q1 * scale;
      }
    }
    if (awq_inv)
      for (int64_t c = 0; c < k; c++) out[r * k + c] *= awq_inv[c];
  }
}

/* src/quantize.rs:437-463 */
void orc_extract_for_gpu(const uint8_t *data, int64_t n, int64_t k, uint8_t *nibbles,
                         float *scales) {
  int64_t bpr = k / Q4_BLOCK;
  for (int64_t r = 0; r < n; r++) {
    for (int64_t b = 0; b < bpr; b++) {
      const uint8_t *blk = data + (r * bpr + b) * Q4_BYTES;
      memcpy(&scales[r * bpr + b], blk, 4);
      const uint8_t *cpu = blk + 4;
      uint8_t *g = nibbles + (r * bpr + b) * 16;
      for (int j = 0; j < 16; j++) {
        int half = j >> 1;
        uint8_t ej = (j & 1) == 0 ? (cpu[half] & 0x0f) : (cpu[half] >> 4);
        uint8_t ej16 = (j & 1) == 0 ? (cpu[half + 8] & 0x0f) : (cpu[half + 8] >> 4);
        g[j] = (uint8_t)(ej | (ej16 << 4));
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* src/quantize.rs:853-879 */
float orc_q4_dot_row_scalar(const uint8_t *row, const float *x, int64_t blocks) {
  float total = 0.0f;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t *blk = row + b * Q4_BYTES;
    float scale;
    memcpy(&scale, blk, 4);
    const float *xb = x + b * Q4_BLOCK;
    float block_sum = 0.0f;
    for (int i = 0; i < 16; i++) {
      int q0 = (blk[4 + i] & 0x0f) - 8;
      int q1 = ((blk[4 + i] >> 4) & 0x0f) - 8;
      block_sum += (float)q0 * xb[2 * i];
      block_sum += (float)q1 * xb[2 * i + 1];
    }
    total += block_sum * scale;
  }
  return total;
}

#if defined(__x86_64__)
/* src/quantize.rs:883-938: per block four 8-lane FMAs into block_acc, then
 * total = fma(block_acc, scale, total); final (lo+hi), movehl, shuffle hsum. */
__attribute__((target("avx2,fma"))) static float q4_dot_row_avx2_impl(const uint8_t *row,
                                                                      const float *x,
                                                                      int64_t blocks) {
  __m256 total_acc = _mm256_setzero_ps();
  const __m256i offset_8 = _mm256_set1_epi32(8);
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t *blk = row + b * Q4_BYTES;
    float scale;
    memcpy(&scale, blk, 4);
    __m256 scale_vec = _mm256_set1_ps(scale);
    const uint8_t *nib = blk + 4;
    const float *xp = x + b * Q4_BLOCK;
    __m256 block_acc = _mm256_setzero_ps();
    for (int g = 0; g < 4; g++) {
      uint32_t b0 = nib[g * 4], b1 = nib[g * 4 + 1], b2 = nib[g * 4 + 2], b3 = nib[g * 4 + 3];
      __m256i vals = _mm256_set_epi32((int)((b3 >> 4) & 15), (int)(b3 & 15), (int)((b2 >> 4) & 15),
                                      (int)(b2 & 15), (int)((b1 >> 4) & 15), (int)(b1 & 15),
                                      (int)((b0 >> 4) & 15), (int)(b0 & 15));
      __m256 fv = _mm256_cvtepi32_ps(_mm256_sub_epi32(vals, offset_8));
      block_acc = _mm256_fmadd_ps(fv, _mm256_loadu_ps(xp + g * 8), block_acc);
    }
    total_acc = _mm256_fmadd_ps(block_acc, scale_vec, total_acc);
  }
  __m128 hi = _mm256_extractf128_ps(total_acc, 1);
  __m128 lo = _mm256_castps256_ps128(total_acc);
  __m128 s128 = _mm_add_ps(lo, hi);
  __m128 s64 = _mm_add_ps(s128, _mm_movehl_ps(s128, s128));
  __m128 s32 = _mm_add_ss(s64, _mm_shuffle_ps(s64, s64, 1));
  return _mm_cvtss_f32(s32);
}
#endif

float orc_q4_dot_row_avx2(const uint8_t *row, const float *x, int64_t blocks) {
#if defined(__x86_64__)
  if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
    return q4_dot_row_avx2_impl(row, x, blocks);
#endif
  return orc_q4_dot_row_scalar(row, x, blocks);
}

/* ---- row-parallel helpers ---------------------------------------------- */
typedef struct {
  int64_t r0, r1;
  const void *a, *b, *c, *d;
  int64_t k;
  void *out;
  int mode;
} rows_job;

static void *q4_rows_worker(void *p) {
  rows_job *j = (rows_job *)p;
  const uint8_t *data = (const uint8_t *)j->a;
  const float *x = (const float *)j->b;
  float *y = (float *)j->out;
  int64_t bpr = j->k / Q4_BLOCK;
  for (int64_t r = j->r0; r < j->r1; r++) {
    const uint8_t *row = data + r * bpr * Q4_BYTES;
    y[r] = j->mode ? orc_q4_dot_row_avx2(row, x, bpr) : orc_q4_dot_row_scalar(row, x, bpr);
  }
  return NULL;
}

static void run_rows(void *(*fn)(void *), rows_job *proto, int64_t n, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if (threads == 1 || n < 32) {
    rows_job j = *proto;
    j.r0 = 0;
    j.r1 = n;
    fn(&j);
    return;
  }
  pthread_t tid[256];
  rows_job jobs[256];
  int64_t per = (n + threads - 1) / threads;
  int started = 0;
  for (int t = 0; t < threads; t++) {
    jobs[t] = *proto;
    jobs[t].r0 = t * per;
    jobs[t].r1 = (t + 1) * per < n ? (t + 1) * per : n;
    if (jobs[t].r0 >= jobs[t].r1) break;
    if (pthread_create(&tid[t], NULL, fn, &jobs[t]) != 0) {
      fn(&jobs[t]);
      tid[t] = 0;
    }
    started = t + 1;
  }
  for (int t = 0; t < started; t++)
    if (tid[t]) pthread_join(tid[t], NULL);
}

/* src/quantize.rs:466-488 (+1107-1111) */
void orc_q4_matvec_f32(const uint8_t *data, int64_t n, int64_t k, const float *x,
                       const float *awq_inv, float *y, int threads, int use_avx2) {
  float *xe = NULL;
  if (awq_inv) {
    xe = (float *)malloc(sizeof(float) * (size_t)k);
    for (int64_t i = 0; i < k; i++) xe[i] = x[i] * awq_inv[i];
    x = xe;
  }
  rows_job proto = {0, 0, data, x, NULL, NULL, k, y, use_avx2};
  run_rows(q4_rows_worker, &proto, n, n >= 32 ? threads : 1);
  free(xe);
}

/* ------------------------------------------------------------------------ */
static int8_t q8_round_clamp(float v) {
  float r = rintf(v); /* round-to-nearest-even (default FP environment) */
  if (isnan(r)) return 0;
  if (r < -127.0f) return -127;
  if (r > 127.0f) return 127;
  return (int8_t)r;
}

/* cuda/nve_kernels.cu:712-745 */
void orc_quantize_q8_group(const float *x, int64_t k, int8_t *xq, float *scales) {
  for (int64_t g = 0; g < k / 32; g++) {
    const float *v = x + g * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    scales[g] = scale;
    float inv = 1.0f / scale;
    for (int i = 0; i < 32; i++) xq[g * 32 + i] = q8_round_clamp(v[i] * inv);
  }
}

void orc_quantize_q8_rows_bf16(const float *x, int64_t m, int64_t k, int8_t *xq,
                               uint16_t *scales_bf16) {
  for (int64_t r = 0; r < m; r++) {
    const float *v = x + r * k;
    float amax = 0.0f;
    for (int64_t i = 0; i < k; i++) amax = fmaxf(amax, fabsf(v[i]));
    float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    uint16_t sb = orc_f32_to_bf16(s);
    scales_bf16[r] = sb;
    float inv = 1.0f / orc_bf16_to_f32(sb);
    for (int64_t i = 0; i < k; i++) xq[r * k + i] = q8_round_clamp(v[i] * inv);
  }
}

/* Integer part of cuda/nve_kernels.cu:796-878.  GPU byte j of a block holds
 * element j (low nibble) and element j+16 (high nibble). */
void orc_w4a8_block_acc(const int8_t *xq, const uint8_t *nibbles, int64_t n, int64_t k,
                        int32_t *acc) {
  int64_t bpr = k / 32;
  for (int64_t r = 0; r < n; r++) {
    for (int64_t b = 0; b < bpr; b++) {
      const uint8_t *g = nibbles + (r * bpr + b) * 16;
      const int8_t *xb = xq + b * 32;
      int32_t s = 0;
      for (int j = 0; j < 16; j++) {
        s += ((int32_t)(g[j] & 0x0f) - 8) * (int32_t)xb[j];
        s += ((int32_t)(g[j] >> 4) - 8) * (int32_t)xb[j + 16];
      }
      acc[r * bpr + b] = s;
    }
  }
}

void orc_matvec_w4a8_f64(const int8_t *xq, const float *xs, int xs_mode,
                         const uint8_t *nibbles, const float *ws, int64_t n, int64_t k,
                         double *y) {
  int64_t bpr = k / 32;
  int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)bpr);
  for (int64_t r = 0; r < n; r++) {
    orc_w4a8_block_acc(xq, nibbles + r * bpr * 16, 1, k, acc);
    double s = 0.0;
    for (int64_t b = 0; b < bpr; b++) {
      double sx = xs_mode == 0 ? (double)xs[b] : (double)xs[0];
      s += (double)ws[r * bpr + b] * sx * (double)acc[b];
    }
    y[r] = s;
  }
  free(acc);
}

static void *w4a8_rows_worker(void *p) {
  rows_job *j = (rows_job *)p;
  const int8_t *xq = (const int8_t *)j->a;
  const float *xs = (const float *)j->b;
  const uint8_t *nib = (const uint8_t *)j->c;
  const float *ws = (const float *)j->d;
  float *y = (float *)j->out;
  int64_t bpr = j->k / 32;
  int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)bpr);
  for (int64_t r = j->r0; r < j->r1; r++) {
    orc_w4a8_block_acc(xq, nib + r * bpr * 16, 1, j->k, acc);
    float s = 0.0f;
    for (int64_t b = 0; b < bpr; b++) s += ws[r * bpr + b] * xs[b] * (float)acc[b];
    y[r] = s;
  }
  free(acc);
  return NULL;
}

void orc_matvec_w4a8_f32(const int8_t *xq, const float *xs, const uint8_t *nibbles,
                         const float *ws, int64_t n, int64_t k, float *y, int threads) {
  rows_job proto = {0, 0, xq, xs, nibbles, ws, k, y, 0};
  run_rows(w4a8_rows_worker, &proto, n, threads);
}

/* cuda/nve_kernels.cu:330-371 formula, in float64 */
void orc_matvec_w4a16_f64(const float *x, const float *awq, const uint8_t *nibbles,
                          const float *scales, int64_t n, int64_t k, double *y) {
  int64_t bpr = k / 32;
  for (int64_t r = 0; r < n; r++) {
    double s = 0.0;
    for (int64_t b = 0; b < bpr; b++) {
      const uint8_t *g = nibbles + (r * bpr + b) * 16;
      double sc = (double)scales[r * bpr + b];
      for (int lane = 0; lane < 32; lane++) {
        int64_t col = b * 32 + lane;
        double xi = (double)x[col];
        if (awq) xi *= (double)awq[col];
        uint8_t bv = g[lane & 15];
        int nib = lane < 16 ? (bv & 0x0f) : (bv >> 4);
        s += xi * (double)(nib - 8) * sc;
      }
    }
    y[r] = s;
  }
}

/* src/gpu_layer.rs:1013-1025 */
int orc_use_w4a8(double importance, int no_w4a8_env, double threshold) {
  if (no_w4a8_env) return 0;
  return importance < threshold ? 1 : 0;
}
