// w4a16_ops.h -- W4A16 device pieces shared by the one-shot and persistent GEMV
// kernels: activation staging into LDS (fp16 pair planes, or fp32 planes with AWQ)
// and the per-block dot products.
#pragma once

#include "common.h"

namespace nve {

enum { MODE_F16 = 0, MODE_BF16 = 1, MODE_F32 = 2 };

// ---- LDS layouts (nb blocks + 1 spare slot for threads past the end) --------
// DOT modes: 4 slot planes of int4 per block, slot i holds the activation pairs that
// meet nibble dword i:  {(x4i, x4i+2), (x16+4i, x18+4i), (x4i+1, x4i+3),
// (x17+4i, x19+4i)}; then (MODE_BF16) one float 2^-e per block.
// MODE_F32: 8 planes of float4, plane t holds x[4t .. 4t+3] of the block.
__host__ __device__ constexpr size_t w4a16_lds_bytes(int mode, int K) {
  return mode == MODE_F32 ? (size_t)(K / 32 + 1) * 128
                          : (size_t)(K / 32 + 1) * (64 + (mode == MODE_BF16 ? 4 : 0));
}

__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t c) {
  return (a & 0xffffu) | (c << 16);  // (a.lo, c.lo)
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t c) {
  return (a >> 16) | (c & 0xffff0000u);  // (a.hi, c.hi)
}

// Stage one 16-byte chunk (8 activations) into the DOT-mode planes.  Chunk i is
// quarter q = i & 3 of block i >> 2 and covers 4-groups g = 2q, 2q+1.
template <int MODE>
__device__ __forceinline__ void w4a16_stage_put_dot(uint4 v, int i, bool valid, int nb, int* s_p,
                                                    float* s_mul) {
  const int q = i & 3;
  const int b = valid ? (i >> 2) : nb;
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if (MODE == MODE_BF16) {
    // Block max over the 4 lanes holding the block (aligned quads of threads; the
    // quads are all valid or all not, since nchunk is a multiple of 4).
    float m = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      m = fmaxf(m, fabsf(bf16_bits_to_f32(w[t] & 0xffffu)));
      m = fmaxf(m, fabsf(bf16_bits_to_f32(w[t] >> 16)));
    }
    m = quad_max_f(m);
    int ex = 0;
    (void)frexpf(m, &ex);  // m = f * 2^ex, f in [0.5, 1)
    int e = m > 0.0f ? 15 - ex : 0;
    e = max(-15, min(e, 126));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const _Float16 lo = (_Float16)ldexpf(bf16_bits_to_f32(w[t] & 0xffffu), e);
      const _Float16 hi = (_Float16)ldexpf(bf16_bits_to_f32(w[t] >> 16), e);
      w[t] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    if (q == 0) s_mul[b] = ldexpf(1.0f, -e);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int g = 2 * q + h;              // 4-group within the block
    const uint32_t a = w[2 * h], c = w[2 * h + 1];  // (e0,e1), (e2,e3)
    int* slot = s_p + ((size_t)(g & 3) * (nb + 1) + b) * 4;
    const int off = g < 4 ? 0 : 1;
    slot[off] = (int)pair_lo(a, c);       // (e0, e2)
    slot[off + 2] = (int)pair_hi(a, c);   // (e1, e3)
  }
}

// Stage one chunk (8 activations, fp16 or bf16) times awq into the fp32 planes.
template <int XDT>
__device__ __forceinline__ void w4a16_stage_put_f32(uint4 v, float4 a0, float4 a1, int i, bool valid,
                                                    int nb, float4* s_f) {
  const int q = i & 3;
  const int b = valid ? (i >> 2) : nb;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float x[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    x[2 * t] = XDT == NVE_DT_BF16 ? bf16_bits_to_f32(w[t] & 0xffffu) : f16_bits_to_f32(w[t] & 0xffffu);
    x[2 * t + 1] = XDT == NVE_DT_BF16 ? bf16_bits_to_f32(w[t] >> 16) : f16_bits_to_f32(w[t] >> 16);
  }
  const float4 lo = make_float4(x[0] * a0.x, x[1] * a0.y, x[2] * a0.z, x[3] * a0.w);
  const float4 hi = make_float4(x[4] * a1.x, x[5] * a1.y, x[6] * a1.z, x[7] * a1.w);
  s_f[(size_t)(2 * q) * (nb + 1) + b] = lo;
  s_f[(size_t)(2 * q + 1) * (nb + 1) + b] = hi;
}

// Block dot product, DOT modes: 4 nibble dwords against 4 slot planes.  `magic`
// holds 0x64006400 in a VGPR (opaque to the compiler) so each mask-and-merge is one
// v_and_or_b32 (mask from an SGPR, magic from the VGPR) instead of v_and + v_or with
// two literals (gfx9 VOP3 encodings take no literal operand).
__device__ __forceinline__ float w4a16_block_dot_h(uint4 wq, const int4* __restrict__ s_p4,
                                                   int plane_stride, int b, uint32_t magic) {
  const half2_t k1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const half2_t k72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const half2_t k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t d[4] = {wq.x, wq.y, wq.z, wq.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int4 p = s_p4[i * plane_stride + b];
    const uint32_t d0 = d[i], d8 = d[i] >> 8;
    const half2_t w0 = __builtin_bit_cast(half2_t, (d0 & 0x000F000Fu) | magic) + k1032;
    const half2_t w1 = __builtin_bit_cast(half2_t, (d0 & 0x00F000F0u) | magic) * k16th + k72;
    const half2_t w2 = __builtin_bit_cast(half2_t, (d8 & 0x000F000Fu) | magic) + k1032;
    const half2_t w3 = __builtin_bit_cast(half2_t, (d8 & 0x00F000F0u) | magic) * k16th + k72;
    s = __builtin_amdgcn_fdot2(w0, __builtin_bit_cast(half2_t, p.x), s, false);
    s = __builtin_amdgcn_fdot2(w1, __builtin_bit_cast(half2_t, p.y), s, false);
    s = __builtin_amdgcn_fdot2(w2, __builtin_bit_cast(half2_t, p.z), s, false);
    s = __builtin_amdgcn_fdot2(w3, __builtin_bit_cast(half2_t, p.w), s, false);
  }
  return s;
}

// Block dot product, MODE_F32.
__device__ __forceinline__ float w4a16_block_dot_f(uint4 wq, const float4* __restrict__ s_f,
                                                   int plane_stride, int b) {
  const uint32_t d[4] = {wq.x, wq.y, wq.z, wq.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 xl = s_f[i * plane_stride + b];
    const float4 xh = s_f[(4 + i) * plane_stride + b];
    const uint32_t lo = d[i] & 0x0F0F0F0Fu, hi = (d[i] >> 4) & 0x0F0F0F0Fu;
    s = fmaf((float)(lo & 0xffu) - 8.0f, xl.x, s);
    s = fmaf((float)((lo >> 8) & 0xffu) - 8.0f, xl.y, s);
    s = fmaf((float)((lo >> 16) & 0xffu) - 8.0f, xl.z, s);
    s = fmaf((float)(lo >> 24) - 8.0f, xl.w, s);
    s = fmaf((float)(hi & 0xffu) - 8.0f, xh.x, s);
    s = fmaf((float)((hi >> 8) & 0xffu) - 8.0f, xh.y, s);
    s = fmaf((float)((hi >> 16) & 0xffu) - 8.0f, xh.z, s);
    s = fmaf((float)(hi >> 24) - 8.0f, xh.w, s);
  }
  return s;
}

// Policy used by the persistent kernel (w4_persistent.h).  MODE_F32 (AWQ) is served
// by the one-shot kernel only.
template <int MODE>
struct W4A16Policy {
  static_assert(MODE == MODE_F16 || MODE == MODE_BF16, "persistent W4A16 covers the DOT modes");
  struct Args {
    const void* x;
  };
  template <int NJ>
  struct Stage {
    uint4 v[NJ];
  };
  struct XFrag {
    int b;        // block index into the slot planes
    float mul;    // 2^-e (MODE_BF16) or 1, times 0 for lanes past the end
  };
  static __host__ __device__ size_t lds_bytes(int K) { return w4a16_lds_bytes(MODE, K); }
  template <int NJ>
  static __device__ __forceinline__ void stage_issue(Stage<NJ>& s, const Args& a, int K) {
    const int nchunk = K >> 3;
#pragma unroll
    for (int i = 0; i < NJ; ++i)
      s.v[i] = ((const uint4*)a.x)[min((int)threadIdx.x + 256 * i, nchunk - 1)];
  }
  template <int NJ>
  static __device__ __forceinline__ void stage_write(const Stage<NJ>& s, const Args&, int4* lds, int K) {
    const int nb = K >> 5, nchunk = K >> 3;
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int c = (int)threadIdx.x + 256 * i;
      w4a16_stage_put_dot<MODE>(s.v[i], c, c < nchunk, nb, (int*)lds, (float*)(lds + 4 * (nb + 1)));
    }
  }
  static __device__ __forceinline__ XFrag load_x(const int4* lds, int nb, int bb, bool valid) {
    XFrag f;
    f.b = bb;
    f.mul = valid ? 1.0f : 0.0f;
    if (MODE == MODE_BF16) f.mul *= ((const float*)(lds + 4 * (nb + 1)))[bb];
    return f;
  }
  struct Ctx {
    uint32_t magic;  // 0x64006400 held in a VGPR (see w4a16_block_dot_h)
  };
  static __device__ __forceinline__ Ctx make_ctx() {
    Ctx c;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.magic));
    return c;
  }
  static __device__ __forceinline__ void accum(float& acc, uint4 w, float ws, const XFrag& f, const int4* lds,
                                               int nb, const Ctx& c) {
    const float s = w4a16_block_dot_h(w, lds, nb + 1, f.b, c.magic);
    acc = fmaf(s * f.mul, ws, acc);
  }
};

}  // namespace nve
