// gemv_w4a8_batched.hip -- small-batch W4A8 (M <= 16 activation rows).
//
// y[m, n] = sum_b ws[n,b] * xs(m,b) * acc[m,n,b],  acc = sum (nib - 8) * xq[m, .]
// xs(m,b) is xq_scales[m*(K/32) + b] (group mode, the reference's scheme per row)
// or the per-row bf16 scale (per-token mode, applied once per row: the sum over
// blocks is formed with ws only and multiplied by the row scale at the end).
//
// v_dot4 kernel (used for every M here): one wave per output row, lane l owns
// blocks l, l+64, ...; the nibbles are turned into signed int8 (nib - 8) once per
// block with (t + 0x78787878) ^ 0x80808080 (no carries cross bytes for t <= 15), and
// every activation row reuses them through 8 v_dot4_i32_i8.
#include "common.h"
#include "w4_launch.h"

namespace nve {

__device__ __forceinline__ int s8_from_nib(uint32_t t) {  // t: 4 bytes, each 0..15
  return (int)((t + 0x78787878u) ^ 0x80808080u);
}

template <int OUT_DT, int XS_MODE>
__global__ __launch_bounds__(256) void w4a8_batched_dot4_kernel(int M, const int8_t* __restrict__ xq,
                                                                const void* __restrict__ xs,
                                                                const uint8_t* __restrict__ nib,
                                                                const float* __restrict__ ws,
                                                                void* __restrict__ out, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nb = K >> 5;
  const int rowc = min(row, N - 1);
  const uint4* rn = (const uint4*)(nib + (size_t)rowc * (size_t)(K >> 1));
  const float* rs = ws + (size_t)rowc * nb;
  float acc[NVE_MAX_M];
#pragma unroll
  for (int m = 0; m < NVE_MAX_M; ++m) acc[m] = 0.0f;

  for (int b = lane; b < nb; b += 64) {
    const uint4 w = rn[b];
    const float wsc = rs[b];
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    int lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = s8_from_nib(d[i] & 0x0F0F0F0Fu);
      hi[i] = s8_from_nib((d[i] >> 4) & 0x0F0F0F0Fu);
    }
#pragma unroll
    for (int m = 0; m < NVE_MAX_M; ++m) {
      if (m < M) {
        const int4* xr = (const int4*)(xq + (size_t)m * K) + 2 * b;
        const int4 a = xr[0], c = xr[1];
        int s = 0;
        s = __builtin_amdgcn_sdot4(lo[0], a.x, s, false);
        s = __builtin_amdgcn_sdot4(hi[0], c.x, s, false);
        s = __builtin_amdgcn_sdot4(lo[1], a.y, s, false);
        s = __builtin_amdgcn_sdot4(hi[1], c.y, s, false);
        s = __builtin_amdgcn_sdot4(lo[2], a.z, s, false);
        s = __builtin_amdgcn_sdot4(hi[2], c.z, s, false);
        s = __builtin_amdgcn_sdot4(lo[3], a.w, s, false);
        s = __builtin_amdgcn_sdot4(hi[3], c.w, s, false);
        if (XS_MODE == NVE_XS_GROUP32_F32) {
          const float xsf = ((const float*)xs)[(size_t)m * nb + b];
          acc[m] = fmaf(wsc * xsf, (float)s, acc[m]);
        } else {
          acc[m] = fmaf(wsc, (float)s, acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < NVE_MAX_M; ++m) {
    if (m < M) {
      float v = wave_sum_to_lane63(acc[m]);
      if (XS_MODE == NVE_XS_ROW_BF16) v *= bf16_bits_to_f32(((const uint16_t*)xs)[m]);
      if (lane == 63 && row < N) store_out<OUT_DT>(out, (size_t)m * N + row, v);
    }
  }
}

}  // namespace nve

namespace nve_host {

template <int OUT_DT>
static hipError_t launch_batched_o(int M, const int8_t* xq, const void* xs, int xs_mode,
                                   const uint8_t* nib, const float* ws, void* out, int N, int K,
                                   hipStream_t stream) {
  const dim3 grid((N + 3) / 4);
  if (xs_mode == NVE_XS_ROW_BF16)
    hipLaunchKernelGGL((nve::w4a8_batched_dot4_kernel<OUT_DT, NVE_XS_ROW_BF16>), grid, dim3(256), 0, stream,
                       M, xq, xs, nib, ws, out, N, K);
  else
    hipLaunchKernelGGL((nve::w4a8_batched_dot4_kernel<OUT_DT, NVE_XS_GROUP32_F32>), grid, dim3(256), 0,
                       stream, M, xq, xs, nib, ws, out, N, K);
  return hipGetLastError();
}

hipError_t launch_w4a8_batched(int M, const int8_t* xq, const void* xs, int xs_mode,
                               const uint8_t* nib, const float* ws, void* out, int out_dt, int N,
                               int K, hipStream_t stream) {
  switch (out_dt) {
    case NVE_DT_F16: return launch_batched_o<NVE_DT_F16>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
    case NVE_DT_BF16: return launch_batched_o<NVE_DT_BF16>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
    default: return launch_batched_o<NVE_DT_F32>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
  }
}

}  // namespace nve_host
