// gemv_w4a16.hip -- W4A16 decode GEMV for gfx950 (int4 weights x fp16/bf16 activations).
//
// Computes (cuda/nve_kernels.cu:330-371 restated for CDNA4):
//   y[n] = sum_b s[n,b] * sum_{i<32} x[32b+i] * awq[32b+i] * (nib_i - 8)
// with fp32 accumulation.
//
// Work split and load pipeline are those of the W4A8 kernel (gemv_w4a8.hip): wave
// owns R rows, lane l owns blocks l, l+64, ..., every weight load is a coalesced
// 1 KiB / 256 B wave span, all loads issued before the arithmetic, activations staged
// once per workgroup in LDS while the weight loads are in flight.
//
// Arithmetic (three modes, chosen on the host):
//   MODE_F16   x fp16, no AWQ.  Weights become exact fp16 pairs (nib - 8) with a
//              magic-number trick: (d & 0x000F000F) | 0x64006400 is the fp16 pair
//              (1024 + n0, 1024 + n1), minus 1032 gives n - 8 exactly; the nibbles at
//              bits 4-7 / 20-23 give 1024 + 16n, and *1/16 - 72 gives n - 8 exactly.
//              Each pair meets a pair of activations in one v_dot2c_f32_f16 (exact
//              products, fp32 accumulation).  The activations are staged in LDS in
//              the pair order the nibble layout produces, so no shuffles are needed.
//   MODE_BF16  x bf16, no AWQ.  Same arithmetic; each 32-value block of x is staged
//              as fp16 after an exact power-of-two rescale 2^e chosen so the block
//              maximum lands in [2^14, 2^15), and the block result is multiplied by
//              2^-e.  A bf16 value has 8 significant bits, so the fp16 copy is exact
//              for every element whose magnitude is at least 2^-31 of its block's
//              maximum; smaller elements keep an absolute error below 2^-39 of the
//              block maximum (far below fp32 accumulation rounding).  Precondition:
//              block maxima below 2^31 (e >= -15).
//   MODE_F32   AWQ present (x fp16 or bf16): x*awq is formed in fp32 as the
//              reference does and staged as fp32; weights are converted with
//              v_cvt_f32_ubyte and an exact -8.  Slower (about 3 VALU ops/weight).
#include "common.h"
#include "w4_launch.h"

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

// Block dot product, DOT modes: 4 nibble dwords against 4 slot planes.
__device__ __forceinline__ float w4a16_block_dot_h(uint4 wq, const int4* __restrict__ s_p4,
                                                   int plane_stride, int b) {
  const half2_t k1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const half2_t k72 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const half2_t k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t d[4] = {wq.x, wq.y, wq.z, wq.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int4 p = s_p4[i * plane_stride + b];
    const uint32_t d0 = d[i], d8 = d[i] >> 8;
    const half2_t w0 = __builtin_bit_cast(half2_t, (d0 & 0x000F000Fu) | 0x64006400u) + k1032;
    const half2_t w1 = __builtin_bit_cast(half2_t, (d0 & 0x00F000F0u) | 0x64006400u) * k16th + k72;
    const half2_t w2 = __builtin_bit_cast(half2_t, (d8 & 0x000F000Fu) | 0x64006400u) + k1032;
    const half2_t w3 = __builtin_bit_cast(half2_t, (d8 & 0x00F000F0u) | 0x64006400u) * k16th + k72;
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

template <int MODE, int XDT, int OUT_DT, int R, int NJ, bool MULTI>
__global__ __launch_bounds__(256) void w4a16_gemv_kernel(const void* __restrict__ x, W4Segs segs,
                                                         int K) {
  constexpr int SPT = NJ;  // staging passes: K/8 chunks <= 256*NJ
  extern __shared__ int4 lds[];
  const int nb = K >> 5;
  const int nchunk = K >> 3;
  const int ps = nb + 1;  // plane stride (blocks + spare)
  int* s_p = (int*)lds;
  float* s_mul = (float*)(lds + 4 * ps);
  float4* s_f = (float4*)lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  const int wg = blockIdx.x;
  const int sg = (segs.nseg > 1 && wg >= segs.wg_begin[1]) + (segs.nseg > 2 && wg >= segs.wg_begin[2]);
  const uint8_t* __restrict__ nib = sg == 0 ? segs.nib[0] : (sg == 1 ? segs.nib[1] : segs.nib[2]);
  const float* __restrict__ ws = sg == 0 ? segs.sc[0] : (sg == 1 ? segs.sc[1] : segs.sc[2]);
  const float* __restrict__ awq = sg == 0 ? segs.awq[0] : (sg == 1 ? segs.awq[1] : segs.awq[2]);
  void* __restrict__ out = sg == 0 ? segs.out[0] : (sg == 1 ? segs.out[1] : segs.out[2]);
  const int N = sg == 0 ? segs.n[0] : (sg == 1 ? segs.n[1] : segs.n[2]);
  const int wg0 = sg == 0 ? 0 : (sg == 1 ? segs.wg_begin[1] : segs.wg_begin[2]);
  const int row0 = ((wg - wg0) * 4 + wave) * R;
  const uint4* __restrict__ x4 = (const uint4*)x;

  // (1) activation staging loads (clamped index, unconditional)
  uint4 stv[SPT];
  float4 sta0[MODE == MODE_F32 ? SPT : 1], sta1[MODE == MODE_F32 ? SPT : 1];
  if (!MULTI) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = min((int)threadIdx.x + 256 * s, nchunk - 1);
      stv[s] = x4[i];
      if (MODE == MODE_F32) {
        // A fused Q/K/V launch may mix matrices with and without AWQ scales.
        if (awq) {
          sta0[s] = ((const float4*)awq)[2 * i];
          sta1[s] = ((const float4*)awq)[2 * i + 1];
        } else {
          sta0[s] = sta1[s] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // (2) weight loads
  uint4 wv[R][NJ];
  float wsc[R][NJ];
  const size_t row_bytes = (size_t)(K >> 1);
  auto issue = [&](int jb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, N - 1);
      const uint4* rn = (const uint4*)(nib + (size_t)row * row_bytes);
      const float* rs = ws + (size_t)row * nb;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int bb = min(jb + lane + 64 * j, nb - 1);
        wv[r][j] = rn[bb];
        wsc[r][j] = rs[bb];
      }
    }
  };
  issue(0);
  __builtin_amdgcn_sched_barrier(0);

  // (3) LDS writes
  if (!MULTI) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = (int)threadIdx.x + 256 * s;
      if (MODE == MODE_F32)
        w4a16_stage_put_f32<XDT>(stv[s], sta0[s], sta1[s], i, i < nchunk, nb, s_f);
      else
        w4a16_stage_put_dot<MODE>(stv[s], i, i < nchunk, nb, s_p, s_mul);
    }
  } else {
    for (int base = 0; base < nchunk; base += 256) {
      const int i = base + (int)threadIdx.x;
      const int ic = min(i, nchunk - 1);
      if (MODE == MODE_F32) {
        const float4 one = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        w4a16_stage_put_f32<XDT>(x4[ic], awq ? ((const float4*)awq)[2 * ic] : one,
                                 awq ? ((const float4*)awq)[2 * ic + 1] : one, i, i < nchunk, nb, s_f);
      }
      else
        w4a16_stage_put_dot<MODE>(x4[ic], i, i < nchunk, nb, s_p, s_mul);
    }
  }
  lds_barrier();

  // (4) arithmetic
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int jb = 0;;) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int b = jb + lane + 64 * j;
      const int bb = min(b, nb - 1);
      float mul = b < nb ? 1.0f : 0.0f;  // lanes past the end contribute nothing
      if (MODE == MODE_BF16) mul *= s_mul[bb];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float s = MODE == MODE_F32 ? w4a16_block_dot_f(wv[r][j], s_f, ps, bb)
                                         : w4a16_block_dot_h(wv[r][j], (const int4*)s_p, ps, bb);
        acc[r] = fmaf(s * mul, wsc[r][j], acc[r]);
      }
    }
    if (!MULTI) break;
    jb += 64 * NJ;
    if (jb >= nb) break;
    issue(jb);
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum_to_lane63(acc[r]);
    if (lane == 63 && row0 + r < N) store_out<OUT_DT>(out, (size_t)(row0 + r), v);
  }
}

}  // namespace nve

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace nve_host {

template <int MODE, int XDT, int OUT_DT, int R, int NJ, bool MULTI>
static hipError_t launch_w4a16_t(const void* x, const W4Segs& segs, int K, hipStream_t stream) {
  const size_t lds = nve::w4a16_lds_bytes(MODE, K);
  auto kern = nve::w4a16_gemv_kernel<MODE, XDT, OUT_DT, R, NJ, MULTI>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(segs.wg_total), dim3(256), lds, stream, x, segs, K);
  return hipGetLastError();
}

template <int MODE, int XDT, int OUT_DT>
static hipError_t launch_w4a16_m(const void* x, W4Segs segs, int K, hipStream_t stream) {
  const W4Tiling t = choose_w4_tiling(segs, K);
  finalize_segments(segs, t.R);
#define NVE_W4A16_CASE(RR, JJ, MM) \
  if (t.R == RR && t.NJ == JJ && t.multi == MM) \
    return launch_w4a16_t<MODE, XDT, OUT_DT, RR, JJ, MM>(x, segs, K, stream);
  NVE_W4_TILING_CASES(NVE_W4A16_CASE)
#undef NVE_W4A16_CASE
  return hipErrorInvalidValue;
}

template <int OUT_DT>
static hipError_t launch_w4a16_o(const void* x, int x_dt, const W4Segs& segs, int K,
                                 hipStream_t stream) {
  bool has_awq = false;
  for (int i = 0; i < segs.nseg; ++i) has_awq |= segs.awq[i] != nullptr;
  if (has_awq) {
    // MODE_F32 treats a segment whose awq pointer is NULL as awq = 1.
    if (x_dt == NVE_DT_BF16) return launch_w4a16_m<nve::MODE_F32, NVE_DT_BF16, OUT_DT>(x, segs, K, stream);
    return launch_w4a16_m<nve::MODE_F32, NVE_DT_F16, OUT_DT>(x, segs, K, stream);
  }
  if (x_dt == NVE_DT_BF16) return launch_w4a16_m<nve::MODE_BF16, NVE_DT_BF16, OUT_DT>(x, segs, K, stream);
  return launch_w4a16_m<nve::MODE_F16, NVE_DT_F16, OUT_DT>(x, segs, K, stream);
}

hipError_t launch_w4a16(const void* x, int x_dt, const W4Segs& segs, int out_dt, int K,
                        hipStream_t stream) {
  switch (out_dt) {
    case NVE_DT_F16: return launch_w4a16_o<NVE_DT_F16>(x, x_dt, segs, K, stream);
    case NVE_DT_BF16: return launch_w4a16_o<NVE_DT_BF16>(x, x_dt, segs, K, stream);
    default: return launch_w4a16_o<NVE_DT_F32>(x, x_dt, segs, K, stream);
  }
}

}  // namespace nve_host
