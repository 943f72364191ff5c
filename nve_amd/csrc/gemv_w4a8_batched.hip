// gemv_w4a8_batched.hip -- small-batch W4A8 (M <= 16 activation rows).
//
// y[m, n] = sum_b ws[n,b] * xs(m,b) * acc[m,n,b],  acc = sum (nib - 8) * xq[m, .]
// xs(m,b) is xq_scales[m*(K/32) + b] (group mode, the reference's scheme per row)
// or the per-row bf16 scale (per-token mode, applied once per row: the sum over
// blocks is formed with ws only and multiplied by the row scale at the end).
//
// v_dot4 kernel (M < 4): one wave per output row, lane l owns
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

// ---------------------------------------------------------------------------
// int8 MFMA kernel (M >= 4).
//
// Workgroup = one 16-row tile of W, KW waves splitting K (wave w takes block quads
// w, w+KW, ...; U quads' loads are issued together).  Per quad (4 consecutive
// 32-weight blocks) lane (n = lane%16,
// g = lane/16) loads the whole 16-byte block 4q+g of row n (one dwordx4; a wave
// instruction reads 16 rows x 64 contiguous bytes).  Two permlane32 swaps and two
// permlane16 swaps transpose the 4x4 (lane group x dword) grid so that register j
// holds, in lane (n, g), dword g of block 4q+j: the 8 weights that lane contributes
// to the MFMA over block 4q+j (low nibbles = elements 4g..4g+3, high nibbles =
// elements 16+4g..16+4g+3).  Nibbles become signed int8 (nib - 8) in registers; the
// activations are loaded the same way (lane (m, g) reads the 32 bytes of block 4q+g
// of row m, two dwordx4) and transposed, so the activation operand of lane (m, g)
// holds xq[m] at the same 8 positions,
// and one v_mfma_i32_16x16x32_i8 per block gives the exact int32 accumulators
// D[n][m] for all 16 activation rows (rows m >= M are zero).  The fp32 epilogue
// applies ws[n,b] * xs[m,b] per block; the KW partial sums meet in LDS.
typedef int v4i_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void transpose4(uint32_t& c0, uint32_t& c1, uint32_t& c2, uint32_t& c3) {
  // (lane group g, register c) -> (lane group c, register g)
  auto s02 = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
  auto s13 = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
  c0 = s02[0];
  c2 = s02[1];
  c1 = s13[0];
  c3 = s13[1];
  auto s01 = __builtin_amdgcn_permlane16_swap(c0, c1, false, false);
  auto s23 = __builtin_amdgcn_permlane16_swap(c2, c3, false, false);
  c0 = s01[0];
  c1 = s01[1];
  c2 = s23[0];
  c3 = s23[1];
}

__device__ __forceinline__ long a_operand(uint32_t d) {
  const uint32_t lo = s8_from_nib(d & 0x0F0F0F0Fu);
  const uint32_t hi = s8_from_nib((d >> 4) & 0x0F0F0F0Fu);
  return (long)(((unsigned long)hi << 32) | lo);
}

template <int OUT_DT, int XS_MODE, int KW, int U>
__global__ __launch_bounds__(64 * KW) void w4a8_batched_mfma_kernel(int M, const int8_t* __restrict__ xq,
                                                                    const void* __restrict__ xs,
                                                                    const uint8_t* __restrict__ nib,
                                                                    const float* __restrict__ ws,
                                                                    void* __restrict__ out, int N, int K) {
  __shared__ float s_ws[KW][U][4][16];  // per wave: scales of the current quads, [u][block j][row n]
  __shared__ float s_red[KW][16][17];   // per wave partial sums [n][m] (+1 pad)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;  // weight row within the tile (A operand) / activation row m (B, D)
  const int g = lane >> 4;   // k group
  const int row0 = blockIdx.x * 16;
  const int nb = K >> 5;
  const int nq = (nb + 3) >> 2;
  const int row = min(row0 + nl, N - 1);
  const uint4* wrow = (const uint4*)(nib + (size_t)row * (size_t)(K >> 1));
  const float* srow = ws + (size_t)row * nb;
  const int m = nl;
  const int mc = min(m, M - 1);
  const bool m_ok = m < M;
  const uint4* xrow = (const uint4*)(xq + (size_t)mc * K);  // 2 x 16 B per block

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int q0 = wave; q0 < nq; q0 += KW * U) {
    // All loads of the U quads first (clamped, unconditional).  Lane (n, g) loads
    // weight block 4q+g of row n; lane (m, g) loads the 32 activation bytes of block
    // 4q+g of row m; both grids are transposed to MFMA operand order below.
    uint4 w[U], xa[U], xb[U];
    float sc[U], xsv[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = min(q0 + KW * u, nq - 1);
      const int bl = min(4 * q + g, nb - 1);
      w[u] = ld_stream(wrow + bl);
      sc[u] = ld_stream(srow + bl);
      xa[u] = xrow[2 * bl];
      xb[u] = xrow[2 * bl + 1];
      if (XS_MODE == NVE_XS_GROUP32_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xsv[u][j] = ((const float*)xs)[(size_t)mc * nb + min(4 * q + j, nb - 1)];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) s_ws[wave][u][g][nl] = sc[u];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int bq = 4 * (q0 + KW * u);
      uint32_t c0 = w[u].x, c1 = w[u].y, c2 = w[u].z, c3 = w[u].w;
      transpose4(c0, c1, c2, c3);
      // activations: dword i of a block holds elements 4i..4i+3; lane g needs dwords
      // g (elements 4g..) and 4+g (elements 16+4g..) of each block of the quad
      uint32_t l0 = xa[u].x, l1 = xa[u].y, l2 = xa[u].z, l3 = xa[u].w;
      uint32_t h0 = xb[u].x, h1 = xb[u].y, h2 = xb[u].z, h3 = xb[u].w;
      transpose4(l0, l1, l2, l3);
      transpose4(h0, h1, h2, h3);
      const uint32_t cj[4] = {c0, c1, c2, c3};
      const uint32_t lj[4] = {l0, l1, l2, l3};
      const uint32_t hj[4] = {h0, h1, h2, h3};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (bq + j < nb) {  // wave-uniform
          const long a = a_operand(cj[j]);
          const long bx = m_ok ? (long)(((unsigned long)hj[j] << 32) | lj[j]) : 0L;
          v4i_t d = {0, 0, 0, 0};
          d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bx, d, 0, 0, 0);
          const float4 wsv = *(const float4*)&s_ws[wave][u][j][4 * g];  // rows 4g..4g+3
          const float xsf = XS_MODE == NVE_XS_GROUP32_F32 ? xsv[u][j] : 1.0f;
          acc[0] = fmaf(wsv.x * xsf, (float)d[0], acc[0]);
          acc[1] = fmaf(wsv.y * xsf, (float)d[1], acc[1]);
          acc[2] = fmaf(wsv.z * xsf, (float)d[2], acc[2]);
          acc[3] = fmaf(wsv.w * xsf, (float)d[3], acc[3]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  }
  // D layout: lane holds column m = lane%16, rows 4g..4g+3.
#pragma unroll
  for (int v = 0; v < 4; ++v) s_red[wave][4 * g + v][m] = acc[v];
  __syncthreads();
  for (int t = threadIdx.x; t < 256; t += 64 * KW) {
    const int n = t >> 4, mm = t & 15;
    float y = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < KW; ++w2) y += s_red[w2][n][mm];
    if (mm < M && row0 + n < N) {
      if (XS_MODE == NVE_XS_ROW_BF16) y *= bf16_bits_to_f32(((const uint16_t*)xs)[mm]);
      store_out<OUT_DT>(out, (size_t)mm * N + row0 + n, y);
    }
  }
}

}  // namespace nve

namespace nve_host {

// The MFMA path serves M >= 4 unless the kernel-selection policy forces one-shot
// v_dot4 kernels (nve_hip_set_gemv_policy(NVE_GEMV_ONESHOT, ...)).
static bool batched_use_mfma() { return gemv_policy() != NVE_GEMV_ONESHOT; }

template <int OUT_DT, int XS, int KW>
static hipError_t launch_mfma(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                              void* out, int N, int K, hipStream_t stream) {
  hipLaunchKernelGGL((nve::w4a8_batched_mfma_kernel<OUT_DT, XS, KW, 4>), dim3((N + 15) / 16), dim3(64 * KW), 0,
                     stream, M, xq, xs, nib, ws, out, N, K);
  return hipGetLastError();
}

template <int OUT_DT>
static hipError_t launch_batched_o(int M, const int8_t* xq, const void* xs, int xs_mode,
                                   const uint8_t* nib, const float* ws, void* out, int N, int K,
                                   hipStream_t stream) {
  if (M >= 4 && batched_use_mfma()) {
    // 8 waves per tile when there are too few 16-row tiles to give every CU two
    // workgroups, 4 otherwise.
    const bool wide = (N + 15) / 16 < 512;
    if (xs_mode == NVE_XS_ROW_BF16)
      return wide ? launch_mfma<OUT_DT, NVE_XS_ROW_BF16, 8>(M, xq, xs, nib, ws, out, N, K, stream)
                  : launch_mfma<OUT_DT, NVE_XS_ROW_BF16, 4>(M, xq, xs, nib, ws, out, N, K, stream);
    return wide ? launch_mfma<OUT_DT, NVE_XS_GROUP32_F32, 8>(M, xq, xs, nib, ws, out, N, K, stream)
                : launch_mfma<OUT_DT, NVE_XS_GROUP32_F32, 4>(M, xq, xs, nib, ws, out, N, K, stream);
  }
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
