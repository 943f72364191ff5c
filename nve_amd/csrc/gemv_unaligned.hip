// gemv_unaligned.hip -- the drop-in launchers' path for buffers that meet only the
// reference's own alignment assumptions.
//
// The reference kernels read nibbles two bytes at a time (W4A8, get_int_b2,
// cuda/nve_kernels.cu:789-794) or one byte at a time (W4A16 and dequant, 330-433), the
// int8 activations four bytes at a time (829-832) and fp16 vectors one element at a
// time, so a caller may hand them a view into a larger buffer at any such offset
// (candle passes device_ptr + start_offset, src/cuda_kernels.rs:300-339).  The main
// kernels of this library stream 16-byte words and require 16-byte alignment; when a
// drop-in call's pointers meet only the reference's contract, capi.hip routes it
// here.  These kernels load with exactly the reference's granularity and compute the
// same quantities as the main kernels:
//   * W4A8: the same exact int32 block accumulator (w4a8_block_dot) and the same
//     y += ws * xs * acc per block, one wave per row;
//   * W4A16: per block sum_i (x_i * awq_i) * (n_i - 8) in fp32, times the block scale;
//   * group-32 int8 quantization: the same scale, reciprocal and rounding as
//     q8_group_kernel (bit-identical codes and scales);
//   * dequant: the same f32 value (n - 8) * s [* awq] and the same final rounding as
//     dequant_w4_kernel (bit-identical).
// They are correctness paths: aligned buffers never take them.
#include "common.h"
#include "w4a8_ops.h"

namespace nve {

// One wave per output row (4 rows per 256-thread workgroup); lane l sums the blocks
// l, l+64, ... of its row.  nib: 2-byte aligned, xq: 4-byte aligned.
template <int OUT_DT>
__global__ __launch_bounds__(256) void w4a8_gemv_unaligned_kernel(const int8_t* __restrict__ xq,
                                                                  const float* __restrict__ xs,
                                                                  const uint8_t* __restrict__ nib,
                                                                  const float* __restrict__ ws, void* __restrict__ out,
                                                                  int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;  // wave-uniform
  const int nb = K >> 5;
  const uint16_t* rn = (const uint16_t*)(nib + (size_t)row * (size_t)(K >> 1));
  const float* rs = ws + (size_t)row * nb;
  float acc = 0.0f;
  for (int b = lane; b < nb; b += 64) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)rn[8 * b + 2 * i] | ((uint32_t)rn[8 * b + 2 * i + 1] << 16);
    const int* xb = (const int*)(xq + 32 * (size_t)b);
    const int4 lo = make_int4(xb[0], xb[1], xb[2], xb[3]);
    const int4 hi = make_int4(xb[4], xb[5], xb[6], xb[7]);
    const int a = w4a8_block_dot(make_uint4(w[0], w[1], w[2], w[3]), lo, hi, sum_i8x16(lo) + sum_i8x16(hi));
    acc = fmaf(rs[b] * xs[b], (float)a, acc);
  }
  const float v = wave_sum_to_lane63(acc);
  if (lane == 63) store_out<OUT_DT>(out, (size_t)row, v);
}

// W4A16, one wave per row.  nib: any alignment; x: 2-byte aligned; awq: 4-byte.
template <int XDT, int OUT_DT>
__global__ __launch_bounds__(256) void w4a16_gemv_unaligned_kernel(const void* __restrict__ x,
                                                                   const uint8_t* __restrict__ nib,
                                                                   const float* __restrict__ sc,
                                                                   const float* __restrict__ awq,
                                                                   void* __restrict__ out, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const int nb = K >> 5;
  const uint8_t* rn = nib + (size_t)row * (size_t)(K >> 1);
  const float* rs = sc + (size_t)row * nb;
  float acc = 0.0f;
  for (int b = lane; b < nb; b += 64) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t byte = rn[16 * b + j];
      const int k0 = 32 * b + j, k1 = k0 + 16;
      float x0 = load_act<XDT>(x, k0), x1 = load_act<XDT>(x, k1);
      if (awq) {
        x0 *= awq[k0];
        x1 *= awq[k1];
      }
      s = fmaf(x0, (float)((int)(byte & 15u) - 8), s);
      s = fmaf(x1, (float)((int)(byte >> 4) - 8), s);
    }
    acc = fmaf(s, rs[b], acc);
  }
  const float v = wave_sum_to_lane63(acc);
  if (lane == 63) store_out<OUT_DT>(out, (size_t)row, v);
}

// Group-32 int8 quantization, one thread per group (x aligned to its element size).
template <int XDT>
__global__ __launch_bounds__(256) void q8_group_unaligned_kernel(const void* __restrict__ x, int8_t* __restrict__ xq,
                                                                 float* __restrict__ scales, size_t groups) {
  const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  float m = 0.0f;
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(load_act<XDT>(x, 32 * g + i)));
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  for (int i = 0; i < 32; ++i) xq[32 * g + i] = q8_round_clamp(load_act<XDT>(x, 32 * g + i) * inv);
  scales[g] = scale;
}

// Dequantization, one thread per weight (nib: any alignment; out: its element size).
template <int OUT_DT>
__global__ __launch_bounds__(256) void dequant_w4_unaligned_kernel(const uint8_t* __restrict__ nib,
                                                                   const float* __restrict__ scales,
                                                                   const float* __restrict__ awq,
                                                                   void* __restrict__ out, size_t total, int K) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const size_t row = i / (size_t)K;
  const int col = (int)(i % (size_t)K);
  const int b = col >> 5, p = col & 31;
  const uint32_t byte = nib[row * (size_t)(K >> 1) + 16 * b + (p & 15)];
  const int n = p < 16 ? (int)(byte & 15u) : (int)(byte >> 4);
  float v = (float)(n - 8) * scales[row * (size_t)(K >> 5) + b];
  if (awq) v *= awq[col];
  store_out<OUT_DT>(out, i, v);
}

}  // namespace nve

namespace nve_host {

hipError_t launch_w4a8_unaligned(const int8_t* xq, const float* xs, const uint8_t* nib, const float* ws, void* out,
                                 int out_dt, int N, int K, hipStream_t s) {
  const dim3 grid((N + 3) / 4);
#define NVE_U8(DT) hipLaunchKernelGGL(nve::w4a8_gemv_unaligned_kernel<DT>, grid, dim3(256), 0, s, xq, xs, nib, ws, out, N, K)
  switch (out_dt) {
    case NVE_DT_F16: NVE_U8(NVE_DT_F16); break;
    case NVE_DT_BF16: NVE_U8(NVE_DT_BF16); break;
    case NVE_DT_F32_ACCUM: NVE_U8(NVE_DT_F32_ACCUM); break;
    default: NVE_U8(NVE_DT_F32); break;
  }
#undef NVE_U8
  return hipGetLastError();
}

hipError_t launch_w4a16_unaligned(const void* x, int x_dt, const uint8_t* nib, const float* sc, const float* awq,
                                  void* out, int out_dt, int N, int K, hipStream_t s) {
  const dim3 grid((N + 3) / 4);
#define NVE_U16(XD, OD) \
  hipLaunchKernelGGL((nve::w4a16_gemv_unaligned_kernel<XD, OD>), grid, dim3(256), 0, s, x, nib, sc, awq, out, N, K)
#define NVE_U16_X(XD)                                        \
  switch (out_dt) {                                          \
    case NVE_DT_F16: NVE_U16(XD, NVE_DT_F16); break;         \
    case NVE_DT_BF16: NVE_U16(XD, NVE_DT_BF16); break;       \
    case NVE_DT_F32_ACCUM: NVE_U16(XD, NVE_DT_F32_ACCUM); break; \
    default: NVE_U16(XD, NVE_DT_F32); break;                 \
  }
  if (x_dt == NVE_DT_BF16) {
    NVE_U16_X(NVE_DT_BF16)
  } else {
    NVE_U16_X(NVE_DT_F16)
  }
#undef NVE_U16_X
#undef NVE_U16
  return hipGetLastError();
}

hipError_t launch_q8_group_unaligned(const void* x, int xdt, size_t total, int8_t* xq, float* scales,
                                     hipStream_t s) {
  const size_t groups = total / 32;
  const unsigned grid = (unsigned)((groups + 255) / 256);
  if (xdt == NVE_DT_F16)
    hipLaunchKernelGGL(nve::q8_group_unaligned_kernel<NVE_DT_F16>, dim3(grid), dim3(256), 0, s, x, xq, scales, groups);
  else if (xdt == NVE_DT_BF16)
    hipLaunchKernelGGL(nve::q8_group_unaligned_kernel<NVE_DT_BF16>, dim3(grid), dim3(256), 0, s, x, xq, scales, groups);
  else
    hipLaunchKernelGGL(nve::q8_group_unaligned_kernel<NVE_DT_F32>, dim3(grid), dim3(256), 0, s, x, xq, scales, groups);
  return hipGetLastError();
}

hipError_t launch_dequant_w4_unaligned(const uint8_t* nib, const float* scales, const float* awq, void* out,
                                       int out_dt, int N, int K, hipStream_t s) {
  const size_t total = (size_t)N * K;
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (out_dt == NVE_DT_F32)
    hipLaunchKernelGGL(nve::dequant_w4_unaligned_kernel<NVE_DT_F32>, dim3(grid), dim3(256), 0, s, nib, scales, awq,
                       out, total, K);
  else if (out_dt == NVE_DT_BF16)
    hipLaunchKernelGGL(nve::dequant_w4_unaligned_kernel<NVE_DT_BF16>, dim3(grid), dim3(256), 0, s, nib, scales, awq,
                       out, total, K);
  else
    hipLaunchKernelGGL(nve::dequant_w4_unaligned_kernel<NVE_DT_F16>, dim3(grid), dim3(256), 0, s, nib, scales, awq,
                       out, total, K);
  return hipGetLastError();
}

}  // namespace nve_host
