// capi.hip -- the extern "C" boundary of libnve_hip.so (declared in
// include/nve_kernels.h): argument validation, status codes, and the drop-in
// launchers with the reference's names (cuda/nve_kernels.cu:373, 680, 747, 880).
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "act_producer.h"
#include "w4_launch.h"

namespace nve_host {

static thread_local int g_last_status = NVE_OK;

int set_status(int st) {
  g_last_status = st;
  return st;
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NVE_OK : (int)e;
}

static int from_hip(hipError_t e) { return set_status(e == hipSuccess ? NVE_OK : (int)e); }

static bool dtype_ok(int dt) { return dt == NVE_DT_F16 || dt == NVE_DT_BF16 || dt == NVE_DT_F32; }
// GEMV outputs additionally accept the fp32 accumulate mode.
static bool out_ok(int dt) { return dtype_ok(dt) || dt == NVE_DT_F32_ACCUM; }
static bool out_aligned(const void* p, int dt) { return aligned(p, dt >= NVE_DT_F32 ? 4 : 2); }

// Common GEMV argument checks; nib_align = the nibble alignment the caller's path needs
// (16 for the main kernels; 2 or 1 where the reference-contract kernels of
// gemv_unaligned.hip can serve the call).
static int check_gemv(const void* nib, const void* sc, const void* out, int N, int K, uintptr_t nib_align = 16) {
  if (!nib || !sc || !out) return NVE_ERR_NULL;
  if (N < 1 || K < 32 || K % 32 != 0) return NVE_ERR_SHAPE;
  if (K > NVE_MAX_K) return NVE_ERR_TOO_LARGE;
  if (!aligned(nib, nib_align) || !aligned(sc, 4) || !aligned(out, 2)) return NVE_ERR_ALIGN;
  return NVE_OK;
}
static uintptr_t dt_size(int dt) { return dt == NVE_DT_F32 ? 4 : 2; }

static void report(const char* fn, int st) {
  if (st != NVE_OK) fprintf(stderr, "nve_hip: %s failed: %s (%d)\n", fn, nve_hip_status_string(st), st);
}

hipError_t launch_q8_group(const void* x, int xdt, size_t total, int8_t* xq, float* scales,
                           hipStream_t stream);
hipError_t launch_q8_rows(const void* x, int xdt, int M, int K, int8_t* xq, uint16_t* scales,
                          hipStream_t stream);
hipError_t launch_q4_quantize(const void* w, int wdt, size_t nblocks, uint8_t* nib, float* scales,
                              hipStream_t stream);
hipError_t launch_q4_quantize_awq(const void* w, int wdt, size_t nblocks, int bpr, const float* awq, int kquant,
                                  uint8_t* nib, float* scales, float* awq_inv, hipStream_t stream);
hipError_t launch_gemm_w4a16(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc, const float* awq,
                             void* out, int out_dt, int N, int K, hipStream_t s);
hipError_t launch_dequant_w4(const uint8_t* nib, const float* scales, const float* awq, void* out, int out_dt,
                             int N, int K, hipStream_t stream);
size_t gemm_w4a16_ws_bytes(int M, int N, int K);
hipError_t launch_gemm_w4a16_ws(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                const float* awq, void* out, int out_dt, int N, int K, void* ws, size_t ws_bytes,
                                hipStream_t s);
hipError_t launch_q4_repack(const uint8_t* q4, size_t nblocks, uint8_t* nib, float* scales,
                            hipStream_t stream);
hipError_t launch_stream_read(const void* buf, size_t bytes, float* sink, int mode, hipStream_t stream);
hipError_t launch_w4a8_unaligned(const int8_t* xq, const float* xs, const uint8_t* nib, const float* ws, void* out,
                                 int out_dt, int N, int K, hipStream_t s);
hipError_t launch_w4a16_unaligned(const void* x, int x_dt, const uint8_t* nib, const float* sc, const float* awq,
                                  void* out, int out_dt, int N, int K, hipStream_t s);
hipError_t launch_q8_group_unaligned(const void* x, int xdt, size_t total, int8_t* xq, float* scales,
                                     hipStream_t s);
hipError_t launch_dequant_w4_unaligned(const uint8_t* nib, const float* scales, const float* awq, void* out,
                                       int out_dt, int N, int K, hipStream_t s);
hipError_t launch_w4a8_batched(int M, const int8_t* xq, const void* xs, int xs_mode,
                               const uint8_t* nib, const float* ws, void* out, int out_dt, int N,
                               int K, hipStream_t stream);

}  // namespace nve_host

using namespace nve_host;

extern "C" {

const char* nve_hip_status_string(int st) {
  switch (st) {
    case NVE_OK: return "ok";
    case NVE_ERR_NULL: return "null pointer argument";
    case NVE_ERR_SHAPE: return "invalid shape (need N >= 1, K % 32 == 0, 32 <= K, 1 <= M <= NVE_MAX_M)";
    case NVE_ERR_ALIGN: return "misaligned pointer";
    case NVE_ERR_DTYPE: return "unsupported dtype or mode";
    case NVE_ERR_TOO_LARGE: return "size exceeds a documented maximum";
    default: return st > 0 ? hipGetErrorString((hipError_t)st) : "unknown error";
  }
}

int nve_hip_last_status(void) { return g_last_status; }

const char* nve_hip_version(void) { return "nve_hip 0.1.0 gfx950"; }

#ifndef NVE_BUILD_ID
#error "NVE_BUILD_ID must be defined by the build (hash of the sources it compiles)"
#endif
const char* nve_hip_build_id(void) { return NVE_BUILD_ID; }

// ---- activation quantization --------------------------------------------------
int nve_hip_quantize_q8(const void* x, int x_dtype, int M, int K, int8_t* xq, float* scales,
                        void* stream) {
  if (!x || !xq || !scales) return set_status(NVE_ERR_NULL);
  if (!dtype_ok(x_dtype)) return set_status(NVE_ERR_DTYPE);
  if (M < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(scales, 4)) return set_status(NVE_ERR_ALIGN);
  if (aligned(x, 16) && aligned(xq, 4))
    return from_hip(launch_q8_group(x, x_dtype, (size_t)M * K, xq, scales, (hipStream_t)stream));
  // the reference's contract: x aligned to its element size, xq to a byte
  if (!aligned(x, dt_size(x_dtype))) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_q8_group_unaligned(x, x_dtype, (size_t)M * K, xq, scales, (hipStream_t)stream));
}

int nve_hip_quantize_q8_rows(const void* x, int x_dtype, int M, int K, int8_t* xq,
                             uint16_t* scales_bf16, void* stream) {
  if (!x || !xq || !scales_bf16) return set_status(NVE_ERR_NULL);
  if (!dtype_ok(x_dtype)) return set_status(NVE_ERR_DTYPE);
  if (M < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(x, 16) || !aligned(xq, 4) || !aligned(scales_bf16, 2)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_q8_rows(x, x_dtype, M, K, xq, scales_bf16, (hipStream_t)stream));
}

// ---- W4A8 --------------------------------------------------------------------------
int nve_hip_matvec_w4a8(const int8_t* xq, const float* xq_scales, const uint8_t* nibbles,
                        const float* wt_scales, void* out, int out_dtype, int N, int K,
                        void* stream) {
  if (!xq || !xq_scales) return set_status(NVE_ERR_NULL);
  int st = check_gemv(nibbles, wt_scales, out, N, K, 2);
  if (st != NVE_OK) return set_status(st);
  if (!out_ok(out_dtype)) return set_status(NVE_ERR_DTYPE);
  if (!aligned(xq, 4) || !aligned(xq_scales, 4) || !out_aligned(out, out_dtype)) return set_status(NVE_ERR_ALIGN);
  // nibbles 2-byte / xq 4-byte aligned (the reference's contract) but not 16: the
  // reference-granularity kernel
  if (!aligned(nibbles, 16) || !aligned(xq, 16))
    return from_hip(launch_w4a8_unaligned(xq, xq_scales, nibbles, wt_scales, out, out_dtype, N, K,
                                          (hipStream_t)stream));
  W4Segs s{};
  s.nseg = 1;
  s.nib[0] = nibbles;
  s.sc[0] = wt_scales;
  s.out[0] = out;
  s.n[0] = N;
  return from_hip(launch_w4a8(xq, xq_scales, s, out_dtype, K, (hipStream_t)stream));
}

int nve_hip_grouped_matvec_w4a8(const int8_t* xq, const float* xq_scales, const nve_w4_mat* mats,
                                int count, int out_dtype, int K, void* stream) {
  if (!xq || !xq_scales || !mats) return set_status(NVE_ERR_NULL);
  if (count < 1 || count > 3) return set_status(NVE_ERR_SHAPE);
  if (!out_ok(out_dtype)) return set_status(NVE_ERR_DTYPE);
  W4Segs s{};
  s.nseg = count;
  for (int i = 0; i < count; ++i) {
    int st = check_gemv(mats[i].nibbles, mats[i].scales, mats[i].out, mats[i].n, K);
    if (st != NVE_OK) return set_status(st);
    if (!out_aligned(mats[i].out, out_dtype)) return set_status(NVE_ERR_ALIGN);
    s.nib[i] = mats[i].nibbles;
    s.sc[i] = mats[i].scales;
    s.out[i] = mats[i].out;
    s.n[i] = mats[i].n;
  }
  if (!aligned(xq, 16) || !aligned(xq_scales, 4)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_w4a8(xq, xq_scales, s, out_dtype, K, (hipStream_t)stream));
}

// W4A8 GEMVs that quantize their own activations (nve_quantize_f16_q8 fused into the
// staging of every workgroup; one staging pass, so K <= 16384).
static int src_of(int x_dtype) {
  return x_dtype == NVE_DT_F16 ? nve::SRC_F16 : (x_dtype == NVE_DT_BF16 ? nve::SRC_BF16 : nve::SRC_F32);
}

int nve_hip_grouped_matvec_w4a8_x(const void* x, int x_dtype, const nve_w4_mat* mats, int count, int out_dtype, int K,
                                  void* stream) {
  if (!x || !mats) return set_status(NVE_ERR_NULL);
  if (count < 1 || count > 3) return set_status(NVE_ERR_SHAPE);
  if (!dtype_ok(x_dtype)) return set_status(NVE_ERR_DTYPE);
  if (out_dtype != NVE_DT_F16 && out_dtype != NVE_DT_F32) return set_status(NVE_ERR_DTYPE);
  W4Segs s{};
  s.nseg = count;
  for (int i = 0; i < count; ++i) {
    int st = check_gemv(mats[i].nibbles, mats[i].scales, mats[i].out, mats[i].n, K);
    if (st != NVE_OK) return set_status(st);
    if (!out_aligned(mats[i].out, out_dtype)) return set_status(NVE_ERR_ALIGN);
    s.nib[i] = mats[i].nibbles;
    s.sc[i] = mats[i].scales;
    s.out[i] = mats[i].out;
    s.n[i] = mats[i].n;
  }
  if (K > 16384) return set_status(NVE_ERR_TOO_LARGE);
  if (!aligned(x, 16)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_w4a8_fused(src_of(x_dtype), nve::PAIR_NONE, nve::ProdArgs{x, nullptr, 0.0f}, s, out_dtype, K,
                                    (hipStream_t)stream, nve::EpiArgs{}));
}

int nve_hip_matvec_w4a8_x(const void* x, int x_dtype, const uint8_t* nibbles, const float* wt_scales, void* out,
                          int out_dtype, int N, int K, void* stream) {
  const nve_w4_mat m = {nibbles, wt_scales, nullptr, out, N};
  return nve_hip_grouped_matvec_w4a8_x(x, x_dtype, &m, 1, out_dtype, K, stream);
}

int nve_hip_qkv_matvec_w4a8(const int8_t* xq, const float* xq_scales, const uint8_t* q_nib,
                            const float* q_sc, int Nq, const uint8_t* k_nib, const float* k_sc,
                            int Nk, const uint8_t* v_nib, const float* v_sc, int Nv, void* q_out,
                            void* k_out, void* v_out, int out_dtype, int K, void* stream) {
  const nve_w4_mat m[3] = {{q_nib, q_sc, nullptr, q_out, Nq},
                           {k_nib, k_sc, nullptr, k_out, Nk},
                           {v_nib, v_sc, nullptr, v_out, Nv}};
  return nve_hip_grouped_matvec_w4a8(xq, xq_scales, m, 3, out_dtype, K, stream);
}

int nve_hip_w4a8_block_acc(const int8_t* xq, const uint8_t* nibbles, int32_t* acc, int N, int K,
                           void* stream) {
  if (!xq || !nibbles || !acc) return set_status(NVE_ERR_NULL);
  if (N < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(xq, 16) || !aligned(nibbles, 16) || !aligned(acc, 4)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_w4a8_block_acc(xq, nibbles, acc, N, K, (hipStream_t)stream));
}

int nve_hip_matvec_w4a8_batched(int M, const int8_t* xq, const void* xq_scales, int xs_mode,
                                const uint8_t* nibbles, const float* wt_scales, void* out,
                                int out_dtype, int N, int K, void* stream) {
  if (!xq || !xq_scales) return set_status(NVE_ERR_NULL);
  int st = check_gemv(nibbles, wt_scales, out, N, K);
  if (st != NVE_OK) return set_status(st);
  if (M < 1 || M > NVE_MAX_M) return set_status(NVE_ERR_SHAPE);
  if (!dtype_ok(out_dtype) || (xs_mode != NVE_XS_GROUP32_F32 && xs_mode != NVE_XS_ROW_BF16))
    return set_status(NVE_ERR_DTYPE);
  if (!aligned(xq, 16) || !aligned(xq_scales, xs_mode == NVE_XS_ROW_BF16 ? 2 : 4) ||
      (out_dtype == NVE_DT_F32 && !aligned(out, 4)))
    return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_w4a8_batched(M, xq, xq_scales, xs_mode, nibbles, wt_scales, out, out_dtype, N,
                                      K, (hipStream_t)stream));
}

// ---- W4A16 --------------------------------------------------------------------------
int nve_hip_matvec_w4a16(const void* x, int x_dtype, const uint8_t* nibbles, const float* scales,
                         const float* awq, void* out, int out_dtype, int N, int K, void* stream) {
  if (!x) return set_status(NVE_ERR_NULL);
  int st = check_gemv(nibbles, scales, out, N, K, 1);
  if (st != NVE_OK) return set_status(st);
  if ((x_dtype != NVE_DT_F16 && x_dtype != NVE_DT_BF16) || !out_ok(out_dtype))
    return set_status(NVE_ERR_DTYPE);
  if (!aligned(x, 2) || (awq && !aligned(awq, 4)) || !out_aligned(out, out_dtype)) return set_status(NVE_ERR_ALIGN);
  // aligned only to the reference's contract (nibbles 1, x 2, awq 4 bytes): the
  // reference-granularity kernel
  if (!aligned(nibbles, 16) || !aligned(x, 16) || (awq && !aligned(awq, 16)))
    return from_hip(launch_w4a16_unaligned(x, x_dtype, nibbles, scales, awq, out, out_dtype, N, K,
                                           (hipStream_t)stream));
  W4Segs s{};
  s.nseg = 1;
  s.nib[0] = nibbles;
  s.sc[0] = scales;
  s.awq[0] = awq;
  s.out[0] = out;
  s.n[0] = N;
  return from_hip(launch_w4a16(x, x_dtype, s, out_dtype, K, (hipStream_t)stream));
}

int nve_hip_grouped_matvec_w4a16(const void* x, int x_dtype, const nve_w4_mat* mats, int count,
                                 int out_dtype, int K, void* stream) {
  if (!x || !mats) return set_status(NVE_ERR_NULL);
  if (count < 1 || count > 3) return set_status(NVE_ERR_SHAPE);
  if ((x_dtype != NVE_DT_F16 && x_dtype != NVE_DT_BF16) || !out_ok(out_dtype))
    return set_status(NVE_ERR_DTYPE);
  W4Segs s{};
  s.nseg = count;
  bool fast = aligned(x, 16);
  for (int i = 0; i < count; ++i) {
    int st = check_gemv(mats[i].nibbles, mats[i].scales, mats[i].out, mats[i].n, K, 1);
    if (st != NVE_OK) return set_status(st);
    if ((mats[i].awq && !aligned(mats[i].awq, 4)) || !out_aligned(mats[i].out, out_dtype))
      return set_status(NVE_ERR_ALIGN);
    fast = fast && aligned(mats[i].nibbles, 16) && (!mats[i].awq || aligned(mats[i].awq, 16));
    s.nib[i] = mats[i].nibbles;
    s.sc[i] = mats[i].scales;
    s.awq[i] = mats[i].awq;
    s.out[i] = mats[i].out;
    s.n[i] = mats[i].n;
  }
  if (!aligned(x, 2)) return set_status(NVE_ERR_ALIGN);
  if (fast) return from_hip(launch_w4a16(x, x_dtype, s, out_dtype, K, (hipStream_t)stream));
  // aligned only to the reference's contract: one reference-granularity launch per matrix
  for (int i = 0; i < count; ++i) {
    const hipError_t e = launch_w4a16_unaligned(x, x_dtype, s.nib[i], s.sc[i], s.awq[i], s.out[i], out_dtype, s.n[i],
                                                K, (hipStream_t)stream);
    if (e != hipSuccess) return from_hip(e);
  }
  return set_status(NVE_OK);
}

int nve_hip_qkv_matvec_w4a16(const void* x, int x_dtype, const uint8_t* q_nib, const float* q_sc,
                             const float* q_awq, int Nq, const uint8_t* k_nib, const float* k_sc,
                             const float* k_awq, int Nk, const uint8_t* v_nib, const float* v_sc,
                             const float* v_awq, int Nv, void* q_out, void* k_out, void* v_out,
                             int out_dtype, int K, void* stream) {
  const nve_w4_mat m[3] = {{q_nib, q_sc, q_awq, q_out, Nq},
                           {k_nib, k_sc, k_awq, k_out, Nk},
                           {v_nib, v_sc, v_awq, v_out, Nv}};
  return nve_hip_grouped_matvec_w4a16(x, x_dtype, m, 3, out_dtype, K, stream);
}

// ---- weight preparation -------------------------------------------------------------
int nve_hip_q4_quantize(const void* w, int w_dtype, int N, int K, uint8_t* nibbles, float* scales,
                        void* stream) {
  if (!w || !nibbles || !scales) return set_status(NVE_ERR_NULL);
  if (!dtype_ok(w_dtype)) return set_status(NVE_ERR_DTYPE);
  if (N < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(w, w_dtype == NVE_DT_F32 ? 4 : 2) || !aligned(nibbles, 16) || !aligned(scales, 4))
    return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_q4_quantize(w, w_dtype, (size_t)N * (K / 32), nibbles, scales, (hipStream_t)stream));
}

int nve_hip_q4_quantize_awq(const void* w, int w_dtype, const float* awq, int kquant, int N, int K,
                            uint8_t* nibbles, float* scales, float* awq_inv, void* stream) {
  if (!w || !awq || !nibbles || !scales) return set_status(NVE_ERR_NULL);
  if (!dtype_ok(w_dtype)) return set_status(NVE_ERR_DTYPE);
  if (N < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(w, w_dtype == NVE_DT_F32 ? 4 : 2) || !aligned(awq, 16) || !aligned(nibbles, 16) ||
      !aligned(scales, 4) || (awq_inv && !aligned(awq_inv, 4)))
    return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_q4_quantize_awq(w, w_dtype, (size_t)N * (K / 32), K / 32, awq, kquant != 0, nibbles,
                                         scales, awq_inv, (hipStream_t)stream));
}

int nve_hip_q4_repack(const uint8_t* q4_blocks, int N, int K, uint8_t* nibbles, float* scales,
                      void* stream) {
  if (!q4_blocks || !nibbles || !scales) return set_status(NVE_ERR_NULL);
  if (N < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(q4_blocks, 4) || !aligned(nibbles, 16) || !aligned(scales, 4)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_q4_repack(q4_blocks, (size_t)N * (K / 32), nibbles, scales, (hipStream_t)stream));
}

int nve_hip_dequant_w4(const uint8_t* nibbles, const float* scales, const float* awq, void* out, int out_dtype,
                       int N, int K, void* stream) {
  if (!nibbles || !scales || !out) return set_status(NVE_ERR_NULL);
  if (out_dtype != NVE_DT_F16 && out_dtype != NVE_DT_BF16 && out_dtype != NVE_DT_F32) return set_status(NVE_ERR_DTYPE);
  if (N < 1 || K < 32 || K % 32 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(scales, 4) || !aligned(out, dt_size(out_dtype)) || (awq && !aligned(awq, 4)))
    return set_status(NVE_ERR_ALIGN);
  if (aligned(nibbles, 16) && aligned(out, 16) && (!awq || aligned(awq, 16)))
    return from_hip(launch_dequant_w4(nibbles, scales, awq, out, out_dtype, N, K, (hipStream_t)stream));
  // aligned only to the reference's contract (nibbles 1 byte, out its element size)
  return from_hip(launch_dequant_w4_unaligned(nibbles, scales, awq, out, out_dtype, N, K, (hipStream_t)stream));
}

int nve_hip_gemm_w4a16(const void* x, int x_dtype, int M, const uint8_t* nibbles, const float* scales,
                       const float* awq, void* out, int out_dtype, int N, int K, void* stream) {
  if (!x || !nibbles || !scales || !out) return set_status(NVE_ERR_NULL);
  if (x_dtype != NVE_DT_F16 && x_dtype != NVE_DT_BF16) return set_status(NVE_ERR_DTYPE);
  if (out_dtype != NVE_DT_F16 && out_dtype != NVE_DT_BF16 && out_dtype != NVE_DT_F32) return set_status(NVE_ERR_DTYPE);
  if (M < 1 || N < 1 || K < 64 || K % 64 != 0) return set_status(NVE_ERR_SHAPE);
  if (K > NVE_MAX_K) return set_status(NVE_ERR_TOO_LARGE);
  if (!aligned(x, 16) || !aligned(nibbles, 16) || !aligned(scales, 4) || (awq && !aligned(awq, 16)) ||
      !aligned(out, out_dtype == NVE_DT_F32 ? 4 : 2))
    return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_gemm_w4a16(x, x_dtype, M, nibbles, scales, awq, out, out_dtype, N, K, (hipStream_t)stream));
}

size_t nve_hip_gemm_w4a16_workspace_bytes(int M, int N, int K) {
  return (M < 1 || N < 1 || K < 64) ? 0 : gemm_w4a16_ws_bytes(M, N, K);
}

int nve_hip_gemm_w4a16_ws(const void* x, int x_dtype, int M, const uint8_t* nibbles, const float* scales,
                          const float* awq, void* out, int out_dtype, int N, int K, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (!x || !nibbles || !scales || !out) return set_status(NVE_ERR_NULL);
  if (x_dtype != NVE_DT_F16 && x_dtype != NVE_DT_BF16) return set_status(NVE_ERR_DTYPE);
  if (out_dtype != NVE_DT_F16 && out_dtype != NVE_DT_BF16 && out_dtype != NVE_DT_F32) return set_status(NVE_ERR_DTYPE);
  if (M < 1 || N < 1 || K < 64 || K % 64 != 0) return set_status(NVE_ERR_SHAPE);
  if (K > NVE_MAX_K) return set_status(NVE_ERR_TOO_LARGE);
  if (!aligned(x, 16) || !aligned(nibbles, 16) || !aligned(scales, 4) || (awq && !aligned(awq, 16)) ||
      !aligned(out, out_dtype == NVE_DT_F32 ? 4 : 2) || (workspace && !aligned(workspace, 256)))
    return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_gemm_w4a16_ws(x, x_dtype, M, nibbles, scales, awq, out, out_dtype, N, K, workspace,
                                       workspace_bytes, (hipStream_t)stream));
}

// ---- dispatch -------------------------------------------------------------------------
// src/gpu_layer.rs:1013-1025: NVE_NO_W4A8 set (any value) -> W4A16; otherwise W4A8
// when importance < NVE_W4A8_THRESHOLD, a double parsed like Rust's str::parse::<f64>
// (no surrounding whitespace, no hex), falling back to 0.7 when unset or unparsable.
static bool parse_f64_strict(const char* s, double* out) {
  if (!s || !*s) return false;
  const char* p = s;
  if (*p == '+' || *p == '-') ++p;
  if (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r' || *p == '\f' || *p == '\v') return false;
  if (p[0] == '0' && (p[1] == 'x' || p[1] == 'X')) return false;
  if (*s == ' ' || *s == '\t' || *s == '\n') return false;
  char* end = nullptr;
  errno = 0;
  const double v = strtod(s, &end);
  if (end == s || *end != '\0') return false;
  *out = v;
  return true;
}

int nve_use_w4a8(double layer_importance) {
  if (getenv("NVE_NO_W4A8") != nullptr) return 0;
  double threshold = 0.7;
  double parsed;
  if (parse_f64_strict(getenv("NVE_W4A8_THRESHOLD"), &parsed)) threshold = parsed;
  return layer_importance < threshold ? 1 : 0;
}

// ---- decode step --------------------------------------------------------------------
size_t nve_hip_decode_workspace_bytes(const nve_decode_config* cfg) {
  return cfg ? decode_workspace_bytes(*cfg) : 0;
}

static int check_w4(const nve_w4_weight& w, int n, int k) {
  if (!w.nibbles || !w.scales) return NVE_ERR_NULL;
  if (w.n != n || w.k != k) return NVE_ERR_SHAPE;
  if (!aligned(w.nibbles, 16) || !aligned(w.scales, 4)) return NVE_ERR_ALIGN;
  return NVE_OK;
}

// Arguments of the decode layer; need_ws: the caller passes the workspace.
static int check_layer_args(const nve_decode_config* cfg, const nve_layer_weights* w, const nve_decode_io* io,
                            bool need_ws) {
  if (!cfg || !w || !io) return NVE_ERR_NULL;
  int st = check_decode(*cfg);
  if (st != NVE_OK) return st;
  const int H = cfg->hidden, F = cfg->ffn, QD = cfg->num_heads * cfg->head_dim,
            KD = cfg->num_kv_heads * cfg->head_dim;
  const nve_w4_weight* mats[7] = {&w->q, &w->k, &w->v, &w->o, &w->gate, &w->up, &w->down};
  const int ns[7] = {QD, KD, KD, H, F, F, H}, ks[7] = {H, H, H, QD, H, H, F};
  for (int i = 0; i < 7; ++i)
    if ((st = check_w4(*mats[i], ns[i], ks[i])) != NVE_OK) return st;
  if (!w->input_norm || !w->post_attn_norm || !io->hidden || !io->k_cache || !io->v_cache || !io->pos ||
      !io->rope_cos || !io->rope_sin || (need_ws && !io->workspace))
    return NVE_ERR_NULL;
  if ((need_ws && !aligned(io->workspace, 256)) || !aligned(io->hidden, 16) || !aligned(io->k_cache, 16) ||
      !aligned(io->v_cache, 16))
    return NVE_ERR_ALIGN;
  return NVE_OK;
}

int nve_hip_layer_forward_decode(const nve_decode_config* cfg, const nve_layer_weights* w, const nve_decode_io* io,
                                 int use_w4a8, void* stream) {
  const int st = check_layer_args(cfg, w, io, true);
  if (st != NVE_OK) return set_status(st);
  return set_status(layer_forward_decode(*cfg, *w, *io, use_w4a8 != 0, (hipStream_t)stream));
}

int nve_hip_layer_forward_decode_noalloc(const nve_decode_config* cfg, const nve_layer_weights* w,
                                         const nve_decode_io* io, int use_w4a8, void* stream) {
  const int st = check_layer_args(cfg, w, io, false);
  if (st != NVE_OK) return set_status(st);
  return set_status(layer_forward_decode_noalloc(*cfg, *w, *io, use_w4a8 != 0, (hipStream_t)stream));
}

int nve_hip_decode_stage(const nve_decode_config* cfg, const nve_layer_weights* w, const nve_decode_io* io,
                         int use_w4a8, int stage, const void* in, void* out, void* stream) {
  const int st = check_layer_args(cfg, w, io, true);
  if (st != NVE_OK) return set_status(st);
  if (stage < NVE_STAGE_QKV || stage > NVE_STAGE_DOWN) return set_status(NVE_ERR_DTYPE);
  const bool need_in = stage == NVE_STAGE_O_MERGE || stage == NVE_STAGE_DOWN;
  const bool need_out = stage == NVE_STAGE_QKV || stage == NVE_STAGE_GATE_UP;
  if ((need_in && !in) || (need_out && !out)) return set_status(NVE_ERR_NULL);
  if ((in && !aligned(in, 16)) || (out && !aligned(out, 16))) return set_status(NVE_ERR_ALIGN);
  return set_status(decode_stage(*cfg, *w, *io, use_w4a8 != 0, stage, in, out, (hipStream_t)stream));
}

int nve_hip_decode_attn_splits(const nve_decode_config* cfg) {
  if (!cfg) return set_status(NVE_ERR_NULL);
  const int st = check_decode(*cfg);
  if (st != NVE_OK) return set_status(st);
  return attn_splits(*cfg);  // a count, not a status
}

int nve_hip_decode_head(const nve_decode_config* cfg, const nve_decode_head* hd, int use_w4a8, void* stream) {
  if (!cfg || !hd) return set_status(NVE_ERR_NULL);
  int st = check_decode(*cfg);
  if (st != NVE_OK) return set_status(st);
  if ((st = check_w4(hd->lm_head, hd->lm_head.n, cfg->hidden)) != NVE_OK) return set_status(st);
  if (hd->lm_head.n < 1 || (!hd->logits && hd->lm_head.n > cfg->vocab)) return set_status(NVE_ERR_SHAPE);
  if (!hd->hidden || !hd->final_norm || !hd->embed || !hd->token_out || !hd->pos || !hd->workspace)
    return set_status(NVE_ERR_NULL);
  if (!aligned(hd->workspace, 256) || !aligned(hd->hidden, 16) || (hd->logits && !aligned(hd->logits, 4)))
    return set_status(NVE_ERR_ALIGN);
  return set_status(decode_head(*cfg, *hd, use_w4a8 != 0, (hipStream_t)stream));
}

int nve_hip_embed(const uint16_t* embed, const int* token, float* hidden, int hidden_size, int vocab,
                  void* stream) {
  if (!embed || !token || !hidden) return set_status(NVE_ERR_NULL);
  if (hidden_size < 1 || vocab < 1) return set_status(NVE_ERR_SHAPE);
  return from_hip(launch_embed(embed, token, hidden, hidden_size, vocab, (hipStream_t)stream));
}

// ---- kernel selection ---------------------------------------------------------------
int nve_hip_set_gemv_policy(int policy, int persistent_wg_per_cu, int persistent_depth) {
  if (policy != NVE_GEMV_AUTO && policy != NVE_GEMV_ONESHOT && policy != NVE_GEMV_PERSISTENT)
    return set_status(NVE_ERR_DTYPE);
  const int prev = gemv_policy();
  set_gemv_policy(policy, persistent_wg_per_cu, persistent_depth);
  return prev;
}

// ---- measurement ----------------------------------------------------------------------
int nve_hip_stream_read(const void* buf, size_t bytes, float* sink, void* stream) {
  if (!buf || !sink) return set_status(NVE_ERR_NULL);
  if (bytes == 0 || bytes % 16 != 0) return set_status(NVE_ERR_SHAPE);
  if (!aligned(buf, 16) || !aligned(sink, 4)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_stream_read(buf, bytes, sink, 0, (hipStream_t)stream));
}

int nve_hip_stream_read_mode(const void* buf, size_t bytes, float* sink, int mode, void* stream) {
  if (!buf || !sink) return set_status(NVE_ERR_NULL);
  if (bytes == 0 || bytes % 16 != 0) return set_status(NVE_ERR_SHAPE);
  if (mode < 0 || mode > 2) return set_status(NVE_ERR_DTYPE);
  if (!aligned(buf, 16) || !aligned(sink, 4)) return set_status(NVE_ERR_ALIGN);
  return from_hip(launch_stream_read(buf, bytes, sink, mode, (hipStream_t)stream));
}

// ---- drop-in launchers (reference names and argument order) ----------------------
void nve_quantize_f16_q8(const uint16_t* x, int8_t* xq, float* scales, int K, void* stream) {
  report("nve_quantize_f16_q8", nve_hip_quantize_q8(x, NVE_DT_F16, 1, K, xq, scales, stream));
}

void nve_matvec_w4a8(const int8_t* xq, const float* xq_scales, const uint8_t* nibbles,
                     const float* wt_scales, uint16_t* out, int N, int K, void* stream) {
  report("nve_matvec_w4a8",
         nve_hip_matvec_w4a8(xq, xq_scales, nibbles, wt_scales, out, NVE_DT_F16, N, K, stream));
}

void nve_matvec_w4a16(const uint16_t* x, const uint8_t* nibbles, const float* scales,
                      const float* awq, uint16_t* out, int N, int K, void* stream) {
  report("nve_matvec_w4a16",
         nve_hip_matvec_w4a16(x, NVE_DT_F16, nibbles, scales, awq, out, NVE_DT_F16, N, K, stream));
}

void nve_dequant_w4a16(const uint8_t* nibbles, const float* scales, const float* awq, uint16_t* out, int N, int K,
                       void* stream) {
  report("nve_dequant_w4a16", nve_hip_dequant_w4(nibbles, scales, awq, out, NVE_DT_F16, N, K, stream));
}

void nve_qkv_matvec_w4a16(const uint16_t* x, const uint8_t* q_nib, const float* q_sc,
                          const float* q_awq, int Nq, const uint8_t* k_nib, const float* k_sc,
                          const float* k_awq, int Nk, const uint8_t* v_nib, const float* v_sc,
                          const float* v_awq, int Nv, uint16_t* q_out, uint16_t* k_out,
                          uint16_t* v_out, int K, void* stream) {
  report("nve_qkv_matvec_w4a16",
         nve_hip_qkv_matvec_w4a16(x, NVE_DT_F16, q_nib, q_sc, q_awq, Nq, k_nib, k_sc, k_awq, Nk, v_nib,
                                  v_sc, v_awq, Nv, q_out, k_out, v_out, NVE_DT_F16, K, stream));
}

}  // extern "C"
