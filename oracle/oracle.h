/*
 * oracle.h -- CPU restatement of genovationtech/nve's quantized decode GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels in
 * nve_amd/csrc and the CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (libnve_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Integer/byte functions are exact restatements;
 * floating-point functions state their evaluation order.
 *
 * Parity pins (which check guards which function) are listed in the header
 * comment of oracle.c.
 */
#ifndef NVE_ORACLE_H
#define NVE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions --------------------------------------------------- */
/* Rust `f32 as i8`: saturating, NaN -> 0 (Rust reference semantics of `as`). */
int8_t orc_rust_f32_as_i8(float v);
/* IEEE binary16 <-> binary32, round-to-nearest-even (the `half` crate's f16). */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
/* bfloat16 <-> binary32.  bf16->f32 is `bits << 16` (src/tensor.rs:1007-1016 via
 * half::bf16::to_f32); f32->bf16 rounds to nearest even, NaN stays NaN. */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* ---- Q4_0 format (src/quantize.rs) --------------------------------------- */
/* quantize_block_q4, src/quantize.rs:711-731: 32 f32 -> 20 bytes
 * [f32 LE scale][16 bytes, byte i = q[2i] | q[2i+1] << 4]. */
void orc_quantize_block_q4(const float *v32, uint8_t *out20);
/* QuantizedTensor::from_f32, src/quantize.rs:347-375 (K % 32 == 0). */
void orc_quantize_block_q4_weighted(const float *v, const float *imp, uint8_t *out);
void orc_q4_from_f32_awq(const float *w, int64_t n, int64_t k, const float *awq, int kquant, uint8_t *data,
                         float *inv_scales);
void orc_q4_from_f32(const float *w, int64_t n, int64_t k, uint8_t *data);
/* QuantizedTensor::to_f32_vec, src/quantize.rs:396-426 (awq_inv nullable). */
void orc_q4_to_f32(const uint8_t *data, int64_t n, int64_t k, const float *awq_inv,
                   float *out);
/* QuantizedTensor::extract_for_gpu, src/quantize.rs:437-463:
 * CPU order {2i,2i+1} -> GPU order byte j = e_j | e_{j+16} << 4. */
void orc_extract_for_gpu(const uint8_t *data, int64_t n, int64_t k, uint8_t *nibbles,
                         float *scales);

/* ---- reference CPU quantized GEMV ---------------------------------------- */
/* q4_dot_row_scalar, src/quantize.rs:853-879. */
float orc_q4_dot_row_scalar(const uint8_t *row, const float *x, int64_t blocks);
/* q4_dot_row_avx2, src/quantize.rs:883-938 (same FMA/hsum order).  Returns the
 * scalar result when built without AVX2+FMA. */
float orc_q4_dot_row_avx2(const uint8_t *row, const float *x, int64_t blocks);
/* QuantizedTensor::matvec_f32, src/quantize.rs:466-488 with the AWQ pre-scale of
 * src/quantize.rs:1107-1111.  Rows split over `threads` workers when n >= 32
 * (rayon par_iter in the reference); use_avx2 selects q4_dot_row_avx2. */
void orc_q4_matvec_f32(const uint8_t *data, int64_t n, int64_t k, const float *x,
                       const float *awq_inv, float *y, int threads, int use_avx2);

/* ---- W4A8 (cuda/nve_kernels.cu) ------------------------------------------ */
/* _nve_quantize_f16_q8, cuda/nve_kernels.cu:712-745, per group of 32:
 * amax; scale = amax > 0 ? amax/127 : 1; q = clamp(rne(x * (1/scale)), -127, 127).
 * Division and reciprocal are IEEE binary32 (the reference's --use_fast_math
 * approximations are not reproduced).  x holds the activation values already
 * widened to f32 (exact for fp16/bf16 inputs). */
void orc_quantize_q8_group(const float *x, int64_t k, int8_t *xq, float *scales);
/* Per-token (per-row) variant asked for by the batched configurations; it has no
 * reference counterpart.  Per row m: amax; s = amax > 0 ? amax/127 : 1;
 * sb = bf16_rne(s); inv = 1/f32(sb); q = clamp(rne(x*inv), -127, 127). */
void orc_quantize_q8_rows_bf16(const float *x, int64_t m, int64_t k, int8_t *xq,
                               uint16_t *scales_bf16);
/* Exact int32 block accumulators of _nve_matvec_w4a8 (cuda/nve_kernels.cu:
 * 796-878, lines 835-853): acc[n][b] = sum_i (nib_i - 8) * xq_i over block b,
 * nibbles in GPU order.  acc is [n, k/32]. */
void orc_w4a8_block_acc(const int8_t *xq, const uint8_t *nibbles, int64_t n, int64_t k,
                        int32_t *acc);
/* fp64 evaluation of y[n] = sum_b ws[n,b] * xs(b) * acc[n][b]
 * (cuda/nve_kernels.cu:855-858).  xs_mode 0: xs is f32 [k/32] (group mode);
 * xs_mode 1: xs is one f32 per-token scale (xs[0]) applied to every block. */
void orc_matvec_w4a8_f64(const int8_t *xq, const float *xs, int xs_mode,
                         const uint8_t *nibbles, const float *ws, int64_t n, int64_t k,
                         double *y);
/* The same product evaluated in binary32 in the reference kernel's per-block
 * order (ws * xs * (float)acc, cuda/nve_kernels.cu:855-858), summed serially.
 * This is the CPU baseline for the W4A8 restatement. */
void orc_matvec_w4a8_f32(const int8_t *xq, const float *xs, const uint8_t *nibbles,
                         const float *ws, int64_t n, int64_t k, float *y, int threads);

/* ---- W4A16 (cuda/nve_kernels.cu:330-371) ---------------------------------- */
/* fp64 of y[n] = sum_k x[k] * awq[k] * (nib - 8) * s[n, k/32]; awq nullable;
 * x already widened to f32 from fp16/bf16. */
void orc_matvec_w4a16_f64(const float *x, const float *awq, const uint8_t *nibbles,
                          const float *scales, int64_t n, int64_t k, double *y);

/* ---- per-layer precision dispatch (src/gpu_layer.rs:1013-1025) ------------ */
/* use_w4a8 = !no_w4a8_env && importance < threshold (default 0.7). */
int orc_use_w4a8(double importance, int no_w4a8_env, double threshold);

#ifdef __cplusplus
}
#endif
#endif
