// prep.hip -- activation quantization (W4A8 input), device-side Q4_0 weight
// quantization / repack (layer upload), and the HBM streaming probe.
#include "common.h"
#include "w4_launch.h"

namespace nve {

// ---- activation quantization, group-32 f32 scales --------------------------
// cuda/nve_kernels.cu:712-745 restated: per group of 32, amax; scale = amax > 0 ?
// amax/127 : 1; q = clamp(rne(x * (1/scale)), -127, 127).  Division and reciprocal
// are IEEE binary32 (correctly rounded); rne is v_rndne_f32.
// Thread layout: 8 lanes per group, 4 activations per lane.
template <int XDT>
__device__ __forceinline__ void load4(const void* x, size_t i4, float v[4]) {
  if (XDT == NVE_DT_F32) {
    const float4 f = ((const float4*)x)[i4];
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    const uint2 h = ((const uint2*)x)[i4];
    const uint32_t w[2] = {h.x, h.y};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v[2 * t] = XDT == NVE_DT_BF16 ? bf16_bits_to_f32(w[t] & 0xffffu) : f16_bits_to_f32(w[t] & 0xffffu);
      v[2 * t + 1] = XDT == NVE_DT_BF16 ? bf16_bits_to_f32(w[t] >> 16) : f16_bits_to_f32(w[t] >> 16);
    }
  }
}

template <int XDT>
__global__ __launch_bounds__(256) void q8_group_kernel(const void* __restrict__ x, int8_t* __restrict__ xq,
                                                       float* __restrict__ scales, size_t total4) {
  const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;  // index of 4-element chunk
  const size_t ic = i4 < total4 ? i4 : total4 - 1;            // total4 is a multiple of 8
  float v[4];
  load4<XDT>(x, ic, v);
  float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  m = quad_max_f(m);
  m = fmaxf(m, dpp_mov<0x141>(m));  // row_half_mirror: the other quad of the 8 lanes
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  if (i4 < total4) {
    char4 q;
    q.x = q8_round_clamp(v[0] * inv);
    q.y = q8_round_clamp(v[1] * inv);
    q.z = q8_round_clamp(v[2] * inv);
    q.w = q8_round_clamp(v[3] * inv);
    ((char4*)xq)[i4] = q;
    if ((i4 & 7) == 0) scales[i4 >> 3] = scale;
  }
}

// ---- activation quantization, one bf16 scale per row ---------------------------
template <int XDT>
__global__ __launch_bounds__(256) void q8_rows_kernel(const void* __restrict__ x, int8_t* __restrict__ xq,
                                                      uint16_t* __restrict__ scales, int K) {
  __shared__ float red[4];
  const size_t row = blockIdx.x;
  const size_t base4 = row * (size_t)(K / 4);
  float m = 0.0f;
  for (int c = threadIdx.x; c < K / 4; c += 256) {
    float v[4];
    load4<XDT>(x, base4 + c, v);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  // wave max via DPP, then across the 4 waves through LDS
  m = fmaxf(m, dpp_mov<0xB1>(m));
  m = fmaxf(m, dpp_mov<0x4E>(m));
  m = fmaxf(m, dpp_mov<0x141>(m));
  m = fmaxf(m, dpp_mov<0x140>(m));
  m = fmaxf(m, dpp_mov<0x142, 0xA>(m));
  m = fmaxf(m, dpp_mov<0x143, 0xC>(m));
  m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 63));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = m > 0.0f ? m / 127.0f : 1.0f;
  const uint16_t sb = f32_to_bf16_bits(s);
  const float inv = 1.0f / bf16_bits_to_f32(sb);
  if (threadIdx.x == 0) scales[row] = sb;
  for (int c = threadIdx.x; c < K / 4; c += 256) {
    float v[4];
    load4<XDT>(x, base4 + c, v);
    char4 q;
    q.x = q8_round_clamp(v[0] * inv);
    q.y = q8_round_clamp(v[1] * inv);
    q.z = q8_round_clamp(v[2] * inv);
    q.w = q8_round_clamp(v[3] * inv);
    ((char4*)xq)[base4 + c] = q;
  }
}

// ---- Q4_0 weight quantization on the device ------------------------------------
// src/quantize.rs:711-731 per 32-value block, written straight into the GPU layout
// of extract_for_gpu (src/quantize.rs:437-463).  Rust semantics: f32::round rounds
// half away from zero (roundf); `as i8` saturates and maps NaN to 0.
__device__ __forceinline__ int rust_as_i8(float v) {
  if (v != v) return 0;
  v = fminf(fmaxf(v, -128.0f), 127.0f);
  return (int)v;
}

template <int WDT>
__device__ __forceinline__ float load_w(const void* w, size_t i) {
  return load_act<WDT>(w, i);
}

// Q4 modes: plain (from_f32 / from_compact), AWQ (from_compact_awq: column j scaled by
// awq[j] before the plain block quantizer, src/quantize.rs:271-306) and AWQ k-quant
// (from_compact_awq_kquant, 308-346: the block scale is the candidate amax_c / 7 over
// the 8 largest |v| that minimises sum_j awq[j]^2 (v_j - deq_j)^2, 741-793).
enum { Q4_PLAIN = 0, Q4_AWQ = 1, Q4_AWQ_KQUANT = 2 };

template <int WDT, int MODE>
__global__ __launch_bounds__(256) void q4_quantize_kernel(const void* __restrict__ w, uint8_t* __restrict__ nib,
                                                          float* __restrict__ scales, size_t nblocks,
                                                          const float* __restrict__ awq, float* __restrict__ awq_inv,
                                                          int bpr) {
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblocks) return;
  float v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = load_w<WDT>(w, blk * 32 + i);
  const int col0 = MODE == Q4_PLAIN ? 0 : (int)(blk % (size_t)bpr) * 32;
  float scale;
  if constexpr (MODE != Q4_PLAIN) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 a4 = ((const float4*)(awq + col0))[t];
      v[4 * t] *= a4.x;
      v[4 * t + 1] *= a4.y;
      v[4 * t + 2] *= a4.z;
      v[4 * t + 3] *= a4.w;
    }
    // the workgroups of row 0 also write the inverse scales (|s| > 1e-10 ? 1/s : 0)
    if (awq_inv && blk < (size_t)bpr)
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const float sc = awq[col0 + i];
        awq_inv[col0 + i] = fabsf(sc) > 1e-10f ? 1.0f / sc : 0.0f;
      }
  }
  if constexpr (MODE == Q4_AWQ_KQUANT) {
    // Candidate c is the c-th largest |v| (descending sort, src/quantize.rs:746-751):
    // the element whose rank -- the count of larger values plus equal values at lower
    // indices -- is c.  Equal values are interchangeable, so any sort order gives the
    // same candidates (finite inputs).
    float a[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) a[i] = fabsf(v[i]);
    float cand[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) cand[c] = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      int r = 0;
#pragma unroll
      for (int j = 0; j < 32; ++j) r += (a[j] > a[i]) | (j < i && a[j] == a[i]);
#pragma unroll
      for (int c = 0; c < 8; ++c) cand[c] = r == c ? a[i] : cand[c];
    }
    float best_scale = 0.0f, best_err = 3.40282347e38f;  // f32::MAX
    bool live = true;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      live = live && !(cand[c] < 1e-10f);  // the reference breaks at the first tiny candidate
      if (live) {
        const float cs = cand[c] / 7.0f;
        const float ci = 1.0f / cs;
        float err = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          int q = rust_as_i8(roundf(v[j] * ci));
          q = q < -8 ? -8 : (q > 7 ? 7 : q);
          const float aj = awq[col0 + j];
          // (imp * d) * d + err, each product and the sum rounded on its own (Rust
          // does not contract to FMA)
          const float d = __fsub_rn(v[j], __fmul_rn((float)q, cs));
          err = __fadd_rn(err, __fmul_rn(__fmul_rn(__fmul_rn(aj, aj), d), d));
        }
        if (err < best_err) {
          best_err = err;
          best_scale = cs;
        }
      }
    }
    scale = best_scale;
  } else {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    scale = amax > 0.0f ? amax / 7.0f : 0.0f;
  }
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  int q[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    int t = rust_as_i8(roundf(v[i] * inv));
    t = t < -8 ? -8 : (t > 7 ? 7 : t);
    q[i] = t + 8;
  }
  uint32_t d[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t acc = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = 4 * k + t;  // GPU byte j = element j | element j+16 << 4
      acc |= (uint32_t)(q[j] | (q[j + 16] << 4)) << (8 * t);
    }
    d[k] = acc;
  }
  ((uint4*)nib)[blk] = make_uint4(d[0], d[1], d[2], d[3]);
  scales[blk] = scale;
}

// ---- reference CPU Q4_0 bytes -> GPU layout (extract_for_gpu on the device) -------
__global__ __launch_bounds__(256) void q4_repack_kernel(const uint8_t* __restrict__ q4, uint8_t* __restrict__ nib,
                                                        float* __restrict__ scales, size_t nblocks) {
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblocks) return;
  const uint32_t* src = (const uint32_t*)(q4 + blk * 20);  // 20-byte blocks, 4-byte aligned
  uint32_t c[4];
  const uint32_t s = src[0];
#pragma unroll
  for (int k = 0; k < 4; ++k) c[k] = src[1 + k];
  // CPU byte i = e_2i | e_2i+1 << 4.  Element e: byte e/2, high nibble if e odd.
  auto elem = [&](int e) -> uint32_t {
    const int byte = e >> 1;
    const uint32_t bv = (c[byte >> 2] >> (8 * (byte & 3))) & 0xffu;
    return (e & 1) ? (bv >> 4) : (bv & 0xfu);
  };
  uint32_t d[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t acc = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int j = 4 * k + t;
      acc |= (elem(j) | (elem(j + 16) << 4)) << (8 * t);
    }
    d[k] = acc;
  }
  ((uint4*)nib)[blk] = make_uint4(d[0], d[1], d[2], d[3]);
  scales[blk] = __builtin_bit_cast(float, s);
}

// ---- HBM streaming probe --------------------------------------------------------
// Each wave reads 8 contiguous 1 KiB spans (lane l: 16 B at span*1024 + 16*l) with
// nontemporal loads, xors them and writes one word only on an impossible value, so
// the loads cannot be removed.  One launch covers the buffer once.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ buf, size_t n16,
                                                          float* __restrict__ sink) {
  const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    size_t i = (wave * 8 + j) * 64 + lane;
    if (i >= n16) i = n16 - 1;
    v[j] = ld_stream(buf + i);
  }
  uint32_t a = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) a ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  if (a == 0x12345678u) sink[blockIdx.x & 1023] = 1.0f;
}

// Grid-stride form of the same probe: a fixed grid (one or two workgroups per CU)
// whose waves each read 8 x 1 KiB per iteration, stepping by the grid's span until
// the buffer is covered.  Fewer, longer-lived waves than the one-shot form: the better
// of the two at large sizes.
__global__ __launch_bounds__(256) void stream_read_gs_kernel(const uint4* __restrict__ buf, size_t n16,
                                                             float* __restrict__ sink) {
  const size_t nwaves = (size_t)gridDim.x * 4;
  const int lane = threadIdx.x & 63;
  uint32_t a = 0;
  for (size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6); wave * 512 < n16; wave += nwaves) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      size_t i = (wave * 8 + j) * 64 + lane;
      if (i >= n16) i = n16 - 1;
      v[j] = ld_stream(buf + i);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) a ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  if (a == 0x12345678u) sink[blockIdx.x & 1023] = 1.0f;
}

// ---- W4 dequantization (prefill path) ---------------------------------------
// _nve_dequant_w4a16 (cuda/nve_kernels.cu:397-433): w[n, k] = f32(nibble - 8) * scale,
// times awq[k] when given (a second f32 rounding, as QuantizedTensor::to_f32_vec does
// it, src/quantize.rs:396-426), then rounded to the output type (RNE).  One thread per
// run of 8 consecutive outputs: run q of a 32-weight block is the low (q = 0, 1) or high
// (q = 2, 3) nibbles of bytes 8 (q % 2) .. + 7, so four consecutive lanes cover a block and
// a wave's stores are one contiguous span (1 KiB at fp16; one thread per block, 64-byte
// runs per lane, wrote 16-byte pieces 64 bytes apart: 38.6 us for the 8B gate).
template <int OUT_DT>
__global__ __launch_bounds__(256) void dequant_w4_kernel(const uint8_t* __restrict__ nib,
                                                         const float* __restrict__ scales,
                                                         const float* __restrict__ awq, void* __restrict__ out,
                                                         size_t nruns, int nb) {
  const size_t run = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (run >= nruns) return;
  const size_t blk = run >> 2;
  const int q = (int)(run & 3);
  const uint2 w = ((const uint2*)nib)[2 * blk + (q & 1)];
  const float s = scales[blk];
  const uint32_t sh = q >= 2 ? 4u : 0u;
  const uint32_t d[2] = {w.x >> sh, w.y >> sh};
  float v[8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * t + e] = (float)((int)((d[t] >> (8 * e)) & 15u) - 8) * s;
  if (awq) {
    const float* a = awq + (size_t)(blk % (size_t)nb) * 32 + 8 * q;
    const float4 a0 = ((const float4*)a)[0], a1 = ((const float4*)a)[1];
    v[0] *= a0.x, v[1] *= a0.y, v[2] *= a0.z, v[3] *= a0.w;
    v[4] *= a1.x, v[5] *= a1.y, v[6] *= a1.z, v[7] *= a1.w;
  }
  if (OUT_DT == NVE_DT_F32) {
    float4* o = (float4*)((float*)out + run * 8);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t p[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float a = v[2 * t], b = v[2 * t + 1];
      if (OUT_DT == NVE_DT_BF16) {
        typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
        const bf2_t h = {(__bf16)a, (__bf16)b};  // v_cvt_pk_bf16_f32, round to nearest even
        p[t] = __builtin_bit_cast(uint32_t, h);
      } else
        p[t] = (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(a)) |
               ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(b)) << 16);
    }
    ((uint4*)((uint16_t*)out + run * 8))[0] = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

}  // namespace nve

namespace nve_host {

hipError_t launch_dequant_w4(const uint8_t* nib, const float* scales, const float* awq, void* out, int out_dt,
                             int N, int K, hipStream_t stream) {
  const size_t nruns = (size_t)N * (K / 32) * 4;
  const unsigned grid = (unsigned)((nruns + 255) / 256);
  if (out_dt == NVE_DT_F32)
    hipLaunchKernelGGL(nve::dequant_w4_kernel<NVE_DT_F32>, dim3(grid), dim3(256), 0, stream, nib, scales, awq, out,
                       nruns, K / 32);
  else if (out_dt == NVE_DT_BF16)
    hipLaunchKernelGGL(nve::dequant_w4_kernel<NVE_DT_BF16>, dim3(grid), dim3(256), 0, stream, nib, scales, awq, out,
                       nruns, K / 32);
  else
    hipLaunchKernelGGL(nve::dequant_w4_kernel<NVE_DT_F16>, dim3(grid), dim3(256), 0, stream, nib, scales, awq, out,
                       nruns, K / 32);
  return hipGetLastError();
}

hipError_t launch_q8_group(const void* x, int xdt, size_t total, int8_t* xq, float* scales,
                           hipStream_t stream) {
  const size_t total4 = total / 4;
  const unsigned grid = (unsigned)((total4 + 255) / 256);
  if (xdt == NVE_DT_F16)
    hipLaunchKernelGGL(nve::q8_group_kernel<NVE_DT_F16>, dim3(grid), dim3(256), 0, stream, x, xq, scales, total4);
  else if (xdt == NVE_DT_BF16)
    hipLaunchKernelGGL(nve::q8_group_kernel<NVE_DT_BF16>, dim3(grid), dim3(256), 0, stream, x, xq, scales, total4);
  else
    hipLaunchKernelGGL(nve::q8_group_kernel<NVE_DT_F32>, dim3(grid), dim3(256), 0, stream, x, xq, scales, total4);
  return hipGetLastError();
}

hipError_t launch_q8_rows(const void* x, int xdt, int M, int K, int8_t* xq, uint16_t* scales,
                          hipStream_t stream) {
  if (xdt == NVE_DT_F16)
    hipLaunchKernelGGL(nve::q8_rows_kernel<NVE_DT_F16>, dim3(M), dim3(256), 0, stream, x, xq, scales, K);
  else if (xdt == NVE_DT_BF16)
    hipLaunchKernelGGL(nve::q8_rows_kernel<NVE_DT_BF16>, dim3(M), dim3(256), 0, stream, x, xq, scales, K);
  else
    hipLaunchKernelGGL(nve::q8_rows_kernel<NVE_DT_F32>, dim3(M), dim3(256), 0, stream, x, xq, scales, K);
  return hipGetLastError();
}

hipError_t launch_q4_quantize_awq(const void* w, int wdt, size_t nblocks, int bpr, const float* awq, int kquant,
                                  uint8_t* nib, float* scales, float* awq_inv, hipStream_t stream) {
  const unsigned grid = (unsigned)((nblocks + 255) / 256);
#define NVE_Q4Q(DT, MODE)                                                                                      \
  hipLaunchKernelGGL((nve::q4_quantize_kernel<DT, MODE>), dim3(grid), dim3(256), 0, stream, w, nib, scales, \
                     nblocks, awq, awq_inv, bpr)
#define NVE_Q4Q_DT(DT)                                   \
  if (!awq) NVE_Q4Q(DT, nve::Q4_PLAIN);                  \
  else if (kquant) NVE_Q4Q(DT, nve::Q4_AWQ_KQUANT);      \
  else NVE_Q4Q(DT, nve::Q4_AWQ);
  if (wdt == NVE_DT_F32) {
    NVE_Q4Q_DT(NVE_DT_F32)
  } else if (wdt == NVE_DT_BF16) {
    NVE_Q4Q_DT(NVE_DT_BF16)
  } else {
    NVE_Q4Q_DT(NVE_DT_F16)
  }
#undef NVE_Q4Q_DT
#undef NVE_Q4Q
  return hipGetLastError();
}

hipError_t launch_q4_quantize(const void* w, int wdt, size_t nblocks, uint8_t* nib, float* scales,
                              hipStream_t stream) {
  return launch_q4_quantize_awq(w, wdt, nblocks, 1, nullptr, 0, nib, scales, nullptr, stream);
}

hipError_t launch_q4_repack(const uint8_t* q4, size_t nblocks, uint8_t* nib, float* scales,
                            hipStream_t stream) {
  const unsigned grid = (unsigned)((nblocks + 255) / 256);
  hipLaunchKernelGGL(nve::q4_repack_kernel, dim3(grid), dim3(256), 0, stream, q4, nib, scales, nblocks);
  return hipGetLastError();
}

hipError_t launch_stream_read(const void* buf, size_t bytes, float* sink, int mode, hipStream_t stream) {
  const size_t n16 = bytes / 16;
  const size_t grid = (n16 + 2047) / 2048;  // 4 waves x 8 spans x 64 lanes per workgroup
  if (mode == 0) {
    hipLaunchKernelGGL(nve::stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, stream, (const uint4*)buf, n16,
                       sink);
  } else {
    const size_t gs = (size_t)256 * mode;  // mode = workgroups per CU of the 256-CU MI355X
    hipLaunchKernelGGL(nve::stream_read_gs_kernel, dim3((unsigned)(grid < gs ? grid : gs)), dim3(256), 0, stream,
                       (const uint4*)buf, n16, sink);
  }
  return hipGetLastError();
}

}  // namespace nve_host
