/*
 * nve_kernels.h -- C ABI of libnve_hip.so, the MI355X (gfx950) quantized decode GEMV
 * library.  Drop-in for the launchers that genovationtech/nve binds in
 * src/cuda_kernels.rs (extern block, lines 57-289) and defines in cuda/nve_kernels.cu.
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer the caller allocated; nothing here allocates
 *     device memory (except the hipBLASLt handle nve_hip_gemm_w4a16_ws creates once per
 *     device), and every launch is asynchronous on `stream` (a hipStream_t; NULL = the
 *     default stream).
 *   - Weights use the reference's GPU layout (QuantizedTensor::extract_for_gpu,
 *     src/quantize.rs:437-463): nibbles u8 [N, K/2], byte j of each 32-weight block
 *     = element j (low nibble) | element j+16 (high nibble); scales f32 [N, K/32];
 *     weight value = (nibble - 8) * scale.
 *   - The `nve_hip_*` functions return an nve_status (0 = success, > 0 = a
 *     hipError_t from the launch, < 0 = an argument error below).  The drop-in
 *     `void` launchers with the reference's names call them, and on failure print
 *     one line to stderr and record the status for nve_hip_last_status().
 *   - Alignment: the main kernels stream 16-byte words and want nibbles, int8
 *     activations and fp16/bf16 vectors 16-byte aligned, scales and awq 4-byte aligned.
 *     The reference's five launchers and their twins (nve_quantize_f16_q8 /
 *     nve_hip_quantize_q8, nve_matvec_w4a8 / nve_hip_matvec_w4a8, nve_matvec_w4a16 /
 *     nve_hip_matvec_w4a16, nve_qkv_matvec_w4a16 / nve_hip_qkv_matvec_w4a16 /
 *     nve_hip_grouped_matvec_w4a16, nve_dequant_w4a16 / nve_hip_dequant_w4) also accept
 *     the reference's own contract (cuda/nve_kernels.cu:789-794, 829-832, 330-433):
 *     W4A8 nibbles 2-byte and xq 4-byte aligned, W4A16 / dequant nibbles at any byte,
 *     16-bit vectors 2-byte, f32 vectors 4-byte aligned; such calls run kernels that
 *     load at the reference's granularity (same results, lower bandwidth).  Below that
 *     contract: NVE_ERR_ALIGN.  Every other entry point keeps the 16-byte rule.
 *   - Limits: K % 32 == 0, 32 <= K <= NVE_MAX_K, 1 <= N; M <= NVE_MAX_M.
 */
#ifndef NVE_KERNELS_H
#define NVE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define NVE_OK 0
#define NVE_ERR_NULL (-1)      /* a required pointer is NULL */
#define NVE_ERR_SHAPE (-2)     /* N < 1, K % 32 != 0, K out of range, M out of range */
#define NVE_ERR_ALIGN (-3)     /* a pointer violates the alignment above */
#define NVE_ERR_DTYPE (-4)     /* unsupported dtype / mode code */
#define NVE_ERR_TOO_LARGE (-5) /* a size exceeds a documented maximum */

/* ---- dtype codes ------------------------------------------------------------ */
#define NVE_DT_F16 0
#define NVE_DT_BF16 1
#define NVE_DT_F32 2
#define NVE_DT_F32_ACCUM 3 /* GEMV output mode only: fp32 out[n] += y (residual add) */

/* ---- activation-scale modes for the W4A8 kernels ------------------------- */
#define NVE_XS_GROUP32_F32 0 /* one f32 scale per 32 activations (reference mode) */
#define NVE_XS_ROW_BF16 1    /* one bf16 scale per activation row (per-token mode) */

#define NVE_MAX_K 32768
#define NVE_MAX_M 16

/* =========================================================================
 * Drop-in launchers: same symbol names and argument order as the reference.
 * ========================================================================= */

/* Replaces nve_quantize_f16_q8 (cuda/nve_kernels.cu:747-757; Rust decl
 * src/cuda_kernels.rs:251-257).  x fp16 [K] -> xq int8 [K], scales f32 [K/32]:
 * per group amax; scale = amax > 0 ? amax/127 : 1; q = clamp(rne(x/scale*), +-127)
 * with IEEE division (the reference's --use_fast_math reciprocal is not copied). */
void nve_quantize_f16_q8(const uint16_t *x, int8_t *xq, float *scales, int K, void *stream);

/* Replaces nve_matvec_w4a8 (cuda/nve_kernels.cu:880-894; Rust decl
 * src/cuda_kernels.rs:261-270).  out fp16 [N] = sum_b ws[n,b] * xs[b] * acc[n,b],
 * acc = exact int32 sum over the block of (nibble - 8) * xq. */
void nve_matvec_w4a8(const int8_t *xq, const float *xq_scales, const uint8_t *nibbles,
                     const float *wt_scales, uint16_t *out, int N, int K, void *stream);

/* Replaces nve_matvec_w4a16 (cuda/nve_kernels.cu:373-388; Rust decl
 * src/cuda_kernels.rs:117-130).  out fp16 [N] = sum_k x[k] * awq[k] * (nib-8) * s;
 * awq may be NULL. */
void nve_matvec_w4a16(const uint16_t *x, const uint8_t *nibbles, const float *scales,
                      const float *awq, uint16_t *out, int N, int K, void *stream);

/* Replaces nve_qkv_matvec_w4a16 (cuda/nve_kernels.cu:680-700; Rust decl
 * src/cuda_kernels.rs:170-180): the three W4A16 projections sharing x in one launch. */
void nve_qkv_matvec_w4a16(const uint16_t *x, const uint8_t *q_nib, const float *q_sc,
                          const float *q_awq, int Nq, const uint8_t *k_nib, const float *k_sc,
                          const float *k_awq, int Nk, const uint8_t *v_nib, const float *v_sc,
                          const float *v_awq, int Nv, uint16_t *q_out, uint16_t *k_out,
                          uint16_t *v_out, int K, void *stream);

/* Replaces nve_dequant_w4a16 (cuda/nve_kernels.cu:397-433; the prefill path's weight
 * expansion before a dense matmul).  out fp16 [N, K] = f16_rne(f32(nib - 8) * scale
 * [* awq[k]]); awq may be NULL. */
void nve_dequant_w4a16(const uint8_t *nibbles, const float *scales, const float *awq, uint16_t *out,
                       int N, int K, void *stream);

/* =========================================================================
 * Status-returning entry points (dtype-generic twins of the launchers above).
 * ========================================================================= */

/* Twin of nve_quantize_f16_q8 for x of dtype x_dtype (F16, BF16 or F32), group-32
 * f32 scales.  M rows of K activations each (xq [M,K], scales [M,K/32]). */
int nve_hip_quantize_q8(const void *x, int x_dtype, int M, int K, int8_t *xq, float *scales,
                        void *stream);

/* Per-token variant (no reference counterpart; the batched configurations ask for
 * it): one bf16 scale per row.  s = amax > 0 ? amax/127 : 1; sb = bf16_rne(s);
 * q = clamp(rne(x * (1/float(sb))), +-127).  xq [M,K], scales_bf16 [M]. */
int nve_hip_quantize_q8_rows(const void *x, int x_dtype, int M, int K, int8_t *xq,
                             uint16_t *scales_bf16, void *stream);

/* Twin of nve_matvec_w4a8 with a selectable output dtype (F16, BF16 or F32; the
 * F32 output is the value before any rounding to 16 bits; F32_ACCUM adds the fp32
 * value into out, which fuses a residual add into the GEMV).  The same output codes
 * apply to every GEMV entry point below except the batched one. */
int nve_hip_matvec_w4a8(const int8_t *xq, const float *xq_scales, const uint8_t *nibbles,
                        const float *wt_scales, void *out, int out_dtype, int N, int K,
                        void *stream);

/* Fused Q/K/V W4A8: the three projections that share one quantized activation
 * vector in one launch (the reference issues three nve_matvec_w4a8 launches,
 * src/gpu_layer.rs:659-661). */
int nve_hip_qkv_matvec_w4a8(const int8_t *xq, const float *xq_scales, const uint8_t *q_nib,
                            const float *q_sc, int Nq, const uint8_t *k_nib, const float *k_sc,
                            int Nk, const uint8_t *v_nib, const float *v_sc, int Nv, void *q_out,
                            void *k_out, void *v_out, int out_dtype, int K, void *stream);

/* One weight matrix of a grouped launch (row-major packed W4 in the layout above). */
typedef struct nve_w4_mat {
  const uint8_t *nibbles; /* [n, K/2] */
  const float *scales;    /* [n, K/32] */
  const float *awq;       /* [K] or NULL (W4A16 only; ignored by W4A8) */
  void *out;              /* [n] of the call's out_dtype */
  int n;
} nve_w4_mat;

/* Grouped W4A8: 1..3 matrices that share K and one quantized activation vector
 * (Q/K/V, or gate/up of a SwiGLU FFN, src/gpu_layer.rs:936-939) in one launch.
 * mats is a host array of `count` entries. */
int nve_hip_grouped_matvec_w4a8(const int8_t *xq, const float *xq_scales, const nve_w4_mat *mats,
                                int count, int out_dtype, int K, void *stream);

/* W4A8 GEMV that quantizes its own activations: nve_quantize_f16_q8 and
 * nve_matvec_w4a8 in one launch (no reference counterpart; the reference issues the two
 * launches, src/gpu_layer.rs:658-662).  x [K] of x_dtype (F16, BF16 or F32) is
 * quantized to int8 with group-32 scales inside every workgroup exactly as
 * nve_hip_quantize_q8 does it, so results are bit-identical to the two-launch sequence.
 * out_dtype F16 or F32; K <= 16384 (NVE_ERR_TOO_LARGE above). */
int nve_hip_matvec_w4a8_x(const void *x, int x_dtype, const uint8_t *nibbles, const float *wt_scales,
                          void *out, int out_dtype, int N, int K, void *stream);
/* Grouped form (1..3 matrices sharing x and K). */
int nve_hip_grouped_matvec_w4a8_x(const void *x, int x_dtype, const nve_w4_mat *mats, int count,
                                  int out_dtype, int K, void *stream);

/* Batched W4A8 (small-batch decode, 1 <= M <= NVE_MAX_M).  xq [M,K]; xs_mode
 * NVE_XS_GROUP32_F32: xq_scales f32 [M, K/32]; NVE_XS_ROW_BF16: bf16 [M].
 * out [M, N] of out_dtype.  M = 1 runs on the one-shot W4A8 GEMV (per-token mode: unit
 * block scales, the row scale applied to the row sums), M >= 2 on int8 MFMA (K % 128 == 0
 * and N <= 16384: the LDS-ring kernel; otherwise a register kernel, and for M = 2 a
 * v_dot4 kernel with both rows staged in LDS where they fit in 40 KB). */
int nve_hip_matvec_w4a8_batched(int M, const int8_t *xq, const void *xq_scales, int xs_mode,
                                const uint8_t *nibbles, const float *wt_scales, void *out,
                                int out_dtype, int N, int K, void *stream);

/* Debug export of the exact int32 block accumulators of the W4A8 kernels:
 * acc [N, K/32], acc[n,b] = sum over block b of (nibble - 8) * xq.  Computed by the
 * same device routine the GEMV kernels use (cuda/nve_kernels.cu:835-853). */
int nve_hip_w4a8_block_acc(const int8_t *xq, const uint8_t *nibbles, int32_t *acc, int N,
                           int K, void *stream);

/* Twin of nve_matvec_w4a16: x_dtype F16 or BF16, awq nullable, out_dtype F16, BF16
 * or F32. */
int nve_hip_matvec_w4a16(const void *x, int x_dtype, const uint8_t *nibbles,
                         const float *scales, const float *awq, void *out, int out_dtype,
                         int N, int K, void *stream);

/* Grouped W4A16: 1..3 matrices sharing K and x in one launch (see the W4A8 twin). */
int nve_hip_grouped_matvec_w4a16(const void *x, int x_dtype, const nve_w4_mat *mats, int count,
                                 int out_dtype, int K, void *stream);

/* Twin of nve_qkv_matvec_w4a16 with dtype codes. */
int nve_hip_qkv_matvec_w4a16(const void *x, int x_dtype, const uint8_t *q_nib,
                             const float *q_sc, const float *q_awq, int Nq,
                             const uint8_t *k_nib, const float *k_sc, const float *k_awq,
                             int Nk, const uint8_t *v_nib, const float *v_sc,
                             const float *v_awq, int Nv, void *q_out, void *k_out,
                             void *v_out, int out_dtype, int K, void *stream);

/* ---- weight preparation (run once per layer upload) ------------------------ */

/* QuantizedTensor::from_f32 / from_compact + extract_for_gpu on the device
 * (src/quantize.rs:347-375, 242-268, 711-731, 437-463): w [N,K] of w_dtype (F32,
 * BF16 or F16) -> nibbles in GPU order + f32 scales, bit-identical to the reference
 * quantizer (f32::round half away from zero, saturating `as i8`). */
int nve_hip_q4_quantize(const void *w, int w_dtype, int N, int K, uint8_t *nibbles,
                        float *scales, void *stream);

/* QuantizedTensor::from_compact_awq (kquant = 0, src/quantize.rs:271-306) and
 * from_compact_awq_kquant (kquant = 1, 308-346) + extract_for_gpu on the device:
 * column j of w [N,K] is multiplied by awq[j] (f32) before quantization; with kquant
 * the block scale is the candidate amax_c / 7 (c-th largest |v|, c < 8, stopping at
 * the first below 1e-10) that minimises sum_j awq[j]^2 (v_j - q_j scale)^2 (first
 * minimum; quantize_block_q4_weighted, 741-793), else the plain amax / 7.  Writes the
 * AWQ inverse scales awq_inv[j] = |awq[j]| > 1e-10 ? 1/awq[j] : 0 when awq_inv is not
 * NULL (the GEMVs' awq argument).  awq [K] f32 16-byte aligned.  Bit-identical to the
 * reference for finite inputs. */
int nve_hip_q4_quantize_awq(const void *w, int w_dtype, const float *awq, int kquant, int N, int K,
                            uint8_t *nibbles, float *scales, float *awq_inv, void *stream);

/* QuantizedTensor::extract_for_gpu (src/quantize.rs:437-463) on the device: the
 * reference's CPU Q4_0 bytes (20-byte blocks [f32 scale][16 B, byte i = e_2i |
 * e_2i+1 << 4], row-major) -> nibbles in GPU order + scales.  q4_blocks 4-byte
 * aligned. */
int nve_hip_q4_repack(const uint8_t *q4_blocks, int N, int K, uint8_t *nibbles,
                      float *scales, void *stream);

/* Twin of nve_dequant_w4a16 with the output dtype F16, BF16 or F32 (F32 = the value
 * before rounding; bit-identical to QuantizedTensor::to_f32_vec, src/quantize.rs:396-426,
 * applied to the same weights). */
int nve_hip_dequant_w4(const uint8_t *nibbles, const float *scales, const float *awq, void *out,
                       int out_dtype, int N, int K, void *stream);

/* Prefill product Y[M, N] = X[M, K] * W[N, K]^T for int4 weights (the reference's
 * GpuWeight::matmul_x for seq > 1, src/gpu_layer.rs:219-237: nve_dequant_w4a16 to fp16
 * then a dense GEMM) in one kernel: each weight is rounded exactly as the dequant
 * rounds it (to x's dtype: F16 as the reference, or BF16) and the products accumulate
 * in fp32 on MFMA (M <= 320: weight-streaming kernels, where K % 128 == 0 and N <= 16384 an
 * LDS ring in launches of up to 64 rows (32 with awq), else M <= 16 only; with K % 128 ==
 * 0, 128 x 128 or 256 x 128 output tiles with the weights dequantized in registers above
 * M = 320 (128 with awq), and from M = 128 (65 with awq) where N / 128 * M / 128 >= 96
 * tiles; otherwise 128 x 128 tiles dequantized in LDS).  x [M, K]
 * row-major F16/BF16 (16-byte aligned); awq [K] or NULL; out [M, N] row-major F16,
 * BF16 or F32.  K % 64 == 0.  Bit-reproducible: the same inputs give the same bits on
 * every call (no atomic accumulation; nve_hip_gemm_w4a16_ws can also split K over
 * workgroups for small tile grids, with its fp32 partials in the workspace, added in a
 * fixed order). */
int nve_hip_gemm_w4a16(const void *x, int x_dtype, int M, const uint8_t *nibbles, const float *scales,
                       const float *awq, void *out, int out_dtype, int N, int K, void *stream);

/* The same product with the reference's own two-step method where it is faster
 * (GpuWeight::matmul_x, src/gpu_layer.rs:219-237), and bit-reproducible everywhere.
 * The workspace (nve_hip_gemm_w4a16_workspace_bytes(M, N, K) bytes, 256-byte aligned)
 * holds: for M > 512 (M > 384 with awq), with out F32 or x's dtype, the weights
 * dequantized by nve_hip_dequant_w4 (bit-identical to the reference dequant), which
 * hipBLASLt then multiplies with fp32 accumulation; otherwise the fp32 partials of the fused kernels'
 * K split where their tile grid leaves CUs idle, added in a fixed order and rounded once
 * to out_dtype (0 bytes when the shape does not split).  With a NULL
 * or smaller workspace it runs nve_hip_gemm_w4a16.  The first call per device and
 * shape creates the hipBLASLt handle and selects the algorithm; made under graph
 * capture, such a call runs the fused kernel instead, so make it once before
 * capturing.  No counterpart in the reference's FFI (it makes two calls). */
size_t nve_hip_gemm_w4a16_workspace_bytes(int M, int N, int K);
int nve_hip_gemm_w4a16_ws(const void *x, int x_dtype, int M, const uint8_t *nibbles, const float *scales,
                          const float *awq, void *out, int out_dtype, int N, int K, void *workspace,
                          size_t workspace_bytes, void *stream);

/* ---- per-layer precision dispatch (src/gpu_layer.rs:1013-1025) -------------- */
/* Returns 1 (W4A8) when NVE_NO_W4A8 is unset and layer_importance < threshold,
 * where threshold = NVE_W4A8_THRESHOLD parsed as a double, default 0.7; else 0. */
int nve_use_w4a8(double layer_importance);

/* ---- kernel selection ---------------------------------------------------------- */
#define NVE_GEMV_AUTO 0       /* persistent kernel when every wave gets >= 2 row tiles */
#define NVE_GEMV_ONESHOT 1    /* one row tile per wave */
#define NVE_GEMV_PERSISTENT 2 /* persistent, double-buffered kernel whenever K allows */
/* Process-wide choice between the two GEMV kernel shapes (both compute bit-identical
 * results), the persistent grid's workgroups per CU (1..8) and its per-lane buffer
 * depth in 32-weight blocks (4 or 8); values <= 0 keep the current setting.  Returns
 * the previous policy.  Not thread-safe; meant for tests and tuning. */
int nve_hip_set_gemv_policy(int policy, int persistent_wg_per_cu, int persistent_depth);

/* ---- decode step (Llama-style decoder layer around the GEMV path) --------------
 * Restates gpu_layer_forward_decode (src/gpu_layer.rs:1005-1084) for one token:
 *   h += o_proj(attn(rope(q), rope(k) ++ K cache, V cache))    with x = rmsnorm(h)
 *   h += down(silu(gate(x2)) * up(x2))                         with x2 = rmsnorm(h)
 * Precision per layer: W4A8 (every GEMV input quantized to int8 with group-32
 * scales, nve_quantize_f16_q8 semantics) or W4A16 (fp16 GEMV inputs, the reference's
 * decode type).  Five launches
 * per layer: Q/K/V with the RMSNorm computed in its staging; attention (RoPE, cache
 * append, softmax, output converted to the o_proj input -- or, for caches of more than
 * 256 slots, split over 4 workgroups per head (8 above 1024 slots when
 * num_heads * head_dim <= 4096) whose partial softmax states the o_proj staging merges;
 * NVE_ATTN_SPLIT=1/2/4/8 in the environment overrides); o_proj
 * with the residual add; gate/up with the RMSNorm in its staging and silu(gate) * up in its epilogue;
 * down with the residual add.  (NVE_DECODE_FUSE=0 in the environment selects
 * standalone RMSNorm / SiLU-mul kernels instead.)  The position of the token is read from
 * device memory (*pos), so a whole step can be captured in a HIP graph and replayed.
 * RMSNorm accumulates in f64 (src/ops.rs:12-30); RoPE pairs (i, i+D/2) with
 * caller-provided cos/sin tables [max_seq, D/2] (src/ops.rs:264-276); attention is
 * GQA with scale 1/sqrt(D) (src/attention.rs:149-228); the KV cache is bf16. */
typedef struct nve_decode_config {
  int hidden;       /* H, multiple of 32 */
  int num_heads;    /* query heads */
  int num_kv_heads; /* key/value heads (num_heads / num_kv_heads <= 8) */
  int head_dim;     /* D: 64, 128 or 256 */
  int ffn;          /* F, multiple of 32 */
  int max_seq;      /* KV-cache capacity (positions): <= 16384 (8192 for D = 256) */
  int vocab;        /* lm_head rows (0 if the workspace is not used by the head) */
  float eps;        /* RMSNorm epsilon */
} nve_decode_config;

typedef struct nve_w4_weight {
  const uint8_t *nibbles; /* [n, k/2], GPU nibble order */
  const float *scales;    /* [n, k/32] */
  int n;
  int k;
} nve_w4_weight;

typedef struct nve_layer_weights {
  const uint16_t *input_norm;     /* bf16 [H] */
  const uint16_t *post_attn_norm; /* bf16 [H] */
  nve_w4_weight q, k, v, o, gate, up, down;
} nve_layer_weights;

typedef struct nve_decode_io {
  float *hidden;          /* fp32 [H] residual stream, updated in place */
  uint16_t *k_cache;      /* bf16 [num_kv_heads, max_seq, D] of this layer */
  uint16_t *v_cache;      /* bf16 [num_kv_heads, max_seq, D] */
  const int *pos;         /* device int: position of this token (< max_seq) */
  const float *rope_cos;  /* f32 [max_seq, D/2] */
  const float *rope_sin;  /* f32 [max_seq, D/2] */
  void *workspace;        /* nve_hip_decode_workspace_bytes() bytes, 256-byte aligned
                             (scratch: every call writes what it reads, no
                             initialisation needed); one workspace per stream:
                             calls sharing one must not overlap */
} nve_decode_io;

typedef struct nve_decode_head {
  float *hidden;              /* fp32 [H]: final residual in; embedding of the chosen token out */
  const uint16_t *final_norm; /* bf16 [H] */
  nve_w4_weight lm_head;      /* [vocab, H] */
  const uint16_t *embed;      /* bf16 [vocab, H] token embeddings */
  float *logits;              /* fp32 [vocab] or NULL (workspace) */
  int *token_out;             /* device int: greedy token (first maximum, src/ops.rs:485-495) */
  int *pos;                   /* device int, incremented after the step */
  void *workspace;
} nve_decode_head;

/* Size of the decode workspace shared by the layer and head calls of one model. */
size_t nve_hip_decode_workspace_bytes(const nve_decode_config *cfg);
/* One decoder layer for one token; use_w4a8 selects the layer's precision (see
 * nve_use_w4a8). */
int nve_hip_layer_forward_decode(const nve_decode_config *cfg, const nve_layer_weights *w,
                                 const nve_decode_io *io, int use_w4a8, void *stream);
/* The same layer without a caller workspace.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  io->workspace is not read (may be
 * NULL); the scratch is a 1 MiB array inside the library, one per GPU, held until the
 * process ends and looked up once per device.  Nothing is allocated on any call.
 * Layers whose workspace (nve_hip_decode_workspace_bytes of cfg with vocab = 0) exceeds
 * 1 MiB return NVE_ERR_TOO_LARGE.  Calls that overlap on one GPU (concurrent streams)
 * share the array and race; every call writes the scratch it reads. */
int nve_hip_layer_forward_decode_noalloc(const nve_decode_config *cfg, const nve_layer_weights *w,
                                         const nve_decode_io *io, int use_w4a8, void *stream);
/* Final RMSNorm, lm_head GEMV (fp32 logits), greedy argmax, embedding of the chosen
 * token into hidden, *pos += 1. */
int nve_hip_decode_head(const nve_decode_config *cfg, const nve_decode_head *head, int use_w4a8,
                        void *stream);
/* Diagnostic: one fused launch of the layer, issued exactly as
 * nve_hip_layer_forward_decode issues it (same kernels, arguments and workspace), with
 * its input and output exposed so that each fused producer and epilogue can be checked
 * on its own (no reference counterpart; the tests use it).  io->workspace is required.
 *   NVE_STAGE_QKV      RMSNorm(io->hidden) -> grouped Q/K/V GEMV -> RoPE: out = q
 *                      rotated and scaled by log2(e)/sqrt(D) (f32 [heads * D]); the new
 *                      key (rotated) and value rows go to the caches at *io->pos (bf16).
 *   NVE_STAGE_O_MERGE  in = key-split attention partials, f32 [split][heads][D + 4]
 *                      records (m, l, -, -, acc[D]), merged in the o_proj staging;
 *                      io->hidden += o_proj(merged).  split =
 *                      nve_hip_decode_attn_splits(cfg); NVE_ERR_SHAPE when it is 1.
 *   NVE_STAGE_GATE_UP  RMSNorm(io->hidden) -> gate/up pair -> out = silu(gate) * up,
 *                      fp16 [ffn].
 *   NVE_STAGE_DOWN     in = fp16 [ffn] -> down GEMV; io->hidden += y.
 * in / out 16-byte aligned. */
#define NVE_STAGE_QKV 0
#define NVE_STAGE_O_MERGE 1
#define NVE_STAGE_GATE_UP 2
#define NVE_STAGE_DOWN 3
int nve_hip_decode_stage(const nve_decode_config *cfg, const nve_layer_weights *w, const nve_decode_io *io,
                         int use_w4a8, int stage, const void *in, void *out, void *stream);
/* Key splits the layer's attention uses for cfg (1, 2, 4 or 8; NVE_ATTN_SPLIT in the
 * environment overrides, as for the layer). */
int nve_hip_decode_attn_splits(const nve_decode_config *cfg);
/* hidden = embed[*token] (bf16 -> fp32), embed [vocab, hidden_size].  The token is read
 * on the device: one outside [0, vocab) is clamped into it (no out-of-table read). */
int nve_hip_embed(const uint16_t *embed, const int *token, float *hidden, int hidden_size, int vocab,
                  void *stream);

/* ---- measurement and diagnostics ------------------------------------------ */
/* Read-only HBM streaming probe: reads `bytes` (multiple of 16, 16-byte aligned)
 * from buf and writes one f32 per workgroup-slot into sink[0..1023]. */
int nve_hip_stream_read(const void *buf, size_t bytes, float *sink, void *stream);
/* The same probe in a chosen form: mode 0 = one-shot (as nve_hip_stream_read: one
 * wave per 8 KiB), mode 1 / 2 = grid-stride over 1 / 2 workgroups per CU.  The bench
 * takes the faster form at each byte count as the same-size read ceiling. */
int nve_hip_stream_read_mode(const void *buf, size_t bytes, float *sink, int mode, void *stream);
int nve_hip_last_status(void);
const char *nve_hip_status_string(int status);
/* Library version string. */
const char *nve_hip_version(void);
/* Hash of the sources and compile flags the library was built from (32 hex digits;
 * no reference counterpart).  A loader compares it with the hash of the sources it
 * ships with and refuses a library built from other sources. */
const char *nve_hip_build_id(void);

#ifdef __cplusplus
}
#endif
#endif
