// gemm_w4a16.hip -- W4A16 prefill GEMM for gfx950: Y[M, N] = X[M, K] * W[N, K]^T with
// int4 weights in the reference GPU layout and fp16 / bf16 activations.
//
// The reference's prefill path (GpuWeight::matmul_x, src/gpu_layer.rs:219-237) expands
// the weights to an fp16 matrix with nve_dequant_w4a16 (cuda/nve_kernels.cu:397-433)
// and multiplies with a dense fp16 GEMM.  This kernel computes the same product
// without the expanded matrix ever reaching HBM: each workgroup dequantizes its
// 128 x 64 weight slice once into LDS, rounded exactly as the reference's dequant
// rounds it (f32 (nibble - 8) * scale [* awq], then RNE to the activation type), and
// the tile product runs on v_mfma_f32_16x16x32_{f16,bf16} with fp32 accumulation.
// Weight traffic: 0.625 B per weight instead of 0.625 + 2 (write) + 2 (read).
//
// Tiling: 128 x 128 output tile per workgroup of 8 waves (4 x 2), 32 x 64 per wave as
// 2 x 4 MFMA tiles of 16 x 16; K advances 64 per slice (two Q4 blocks).  The global
// loads (X rows, nibbles, scales) of the next slice are in flight while a slice is
// staged and multiplied, so HBM latency overlaps the
// math; small-M launches also split K over workgroups (fp32 atomic accumulation).  LDS rows are padded
// (72 elements) so the ds_read_b128 of a fragment spreads over the banks.
//
// MFMA operand layout (16x16x32): lane l supplies A[l%16][8(l/16) .. +7] and
// B[8(l/16) .. +7][l%16]; it receives D[4(l/16) .. +3][l%16].
#include "common.h"
#include "w4_launch.h"

namespace nve {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_LD = GM_BK + 8;

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if (BF16) return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
  return (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(a)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(b)) << 16);
}

template <bool BF16>
__device__ __forceinline__ f4_t mfma16(uint4 a, uint4 b, f4_t c) {
  if (BF16) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

template <bool AWQ>
struct GemmStage {
  uint4 rx0, rx1;  // two 16-byte pieces of the X slice (rows r and r + 64)
  uint2 rn;        // half a Q4 block: bytes 8h .. 8h+7 (elements 8h..8h+7 and 16+8h..16+8h+7)
  float rs;
  float4 ra[AWQ ? 4 : 1];
};

// Thread t of the 512: X pieces (row t/8 and t/8 + 64, columns 8 (t%8) .. +7); weight
// half-block h = t & 1 of block t/2 (tile row t/4, block (t/2) & 1 of the slice).
template <bool AWQ>
__device__ __forceinline__ void gemm_issue(GemmStage<AWQ>& st, const uint16_t* __restrict__ x,
                                           const uint8_t* __restrict__ nib, const float* __restrict__ scales,
                                           const float* __restrict__ awq, int tid, int m0, int M, int K, int wn_g,
                                           int wblk, int k0) {
  const int r = tid >> 3, c8 = tid & 7;
  const uint16_t* xp = x + (size_t)k0 + 8 * c8;
  st.rx0 = *(const uint4*)(xp + (size_t)min(m0 + r, M - 1) * K);
  st.rx1 = *(const uint4*)(xp + (size_t)min(m0 + r + 64, M - 1) * K);
  const int b = (k0 >> 5) + wblk, h = tid & 1;
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 nv = __builtin_nontemporal_load((const u32x2*)(nib + (size_t)wn_g * (K >> 1) + 16 * b + 8 * h));
  st.rn = make_uint2(nv.x, nv.y);
  st.rs = scales[(size_t)wn_g * (K >> 5) + b];
  if (AWQ) {
    const float4* ap = (const float4*)(awq + 32 * b + 8 * h);
    st.ra[0] = ap[0];
    st.ra[1] = ap[1];
    st.ra[2] = ap[4];  // elements 16 + 8h ..
    st.ra[3] = ap[5];
  }
}

// X slice to LDS; the half block dequantized and rounded to the activation type into
// LDS: elements 8h .. 8h+7 (low nibbles of its bytes) and 16+8h .. 16+8h+7 (high).
template <bool BF16, bool AWQ>
__device__ __forceinline__ void gemm_stage(const GemmStage<AWQ>& st, uint16_t* sX, uint16_t* sW, int tid, int wrow,
                                           int wblk) {
  const int r = tid >> 3, c8 = tid & 7;
  uint16_t* xd = sX + r * GM_LD + 8 * c8;
  *(uint4*)(xd) = st.rx0;
  *(uint4*)(xd + 64 * GM_LD) = st.rx1;
  const int h = tid & 1;
  const uint32_t d[2] = {st.rn.x, st.rn.y};
  float lo[8], hi[8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t byte = (d[t] >> (8 * e)) & 0xffu;
      lo[4 * t + e] = (float)((int)(byte & 15u) - 8) * st.rs;
      hi[4 * t + e] = (float)((int)(byte >> 4) - 8) * st.rs;
    }
  if (AWQ) {
    const float a[16] = {st.ra[0].x, st.ra[0].y, st.ra[0].z, st.ra[0].w, st.ra[1].x, st.ra[1].y, st.ra[1].z, st.ra[1].w,
                         st.ra[2].x, st.ra[2].y, st.ra[2].z, st.ra[2].w, st.ra[3].x, st.ra[3].y, st.ra[3].z, st.ra[3].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo[i] *= a[i];
      hi[i] *= a[8 + i];
    }
  }
  uint16_t* dst = sW + wrow * GM_LD + 32 * wblk + 8 * h;
  // (pack2 rounds each product as an f32 value first: two roundings, as the
  // reference's dequant does them)
  *(uint4*)(dst) = make_uint4(pack2<BF16>(lo[0], lo[1]), pack2<BF16>(lo[2], lo[3]), pack2<BF16>(lo[4], lo[5]),
                              pack2<BF16>(lo[6], lo[7]));
  *(uint4*)(dst + 16) = make_uint4(pack2<BF16>(hi[0], hi[1]), pack2<BF16>(hi[2], hi[3]), pack2<BF16>(hi[4], hi[5]),
                                   pack2<BF16>(hi[6], hi[7]));
}

// The wave's 2 x 4 MFMA tiles (32 rows x 64 columns) over one staged K slice.
template <bool BF16>
__device__ __forceinline__ void gemm_mfma(const uint16_t* sX, const uint16_t* sW, int wm, int wn, int lane,
                                          f4_t (&acc)[2][4]) {
  const int fr = lane & 15, fk = 8 * (lane >> 4);
#pragma unroll
  for (int kk = 0; kk < GM_BK; kk += 32) {
    uint4 a[2], b[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = *(const uint4*)(sX + (32 * wm + 16 * i + fr) * GM_LD + kk + fk);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *(const uint4*)(sW + (64 * wn + 16 * j + fr) * GM_LD + kk + fk);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<BF16>(a[i], b[j], acc[i][j]);
  }
}

// SPLIT: the K range is divided over gridDim.z workgroups per output tile, which add
// their fp32 partial sums into a zeroed fp32 output (launches whose tile grid alone
// would leave most CUs idle: small M).
template <bool BF16, bool AWQ, int OUT_DT, bool SPLIT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 4))) void gemm_w4a16_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ nib,
                                                         const float* __restrict__ scales,
                                                         const float* __restrict__ awq, void* __restrict__ out,
                                                         int M, int N, int K, int k_split) {
  __shared__ __align__(16) uint16_t sX[GM_BM * GM_LD];
  __shared__ __align__(16) uint16_t sW[GM_BN * GM_LD];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves: 32 rows x 64 columns each
  const int m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;

  GemmStage<AWQ> st;
  const int wrow = tid >> 2, wblk = (tid >> 1) & 1;  // weight row in the tile, block within the slice
  const int wn_g = min(n0 + wrow, N - 1);

  f4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int fr = lane & 15;
  const int kb = SPLIT ? blockIdx.z * k_split : 0;
  const int ke = SPLIT ? min(K, kb + k_split) : K;
  // the next slice is in flight while a slice is staged and multiplied; the issue is
  // unconditional (the last slice re-reads itself), which keeps the staging registers
  // out of a conditional merge
  gemm_issue<AWQ>(st, x, nib, scales, awq, tid, m0, M, K, wn_g, wblk, kb);
  for (int k0 = kb; k0 < ke; k0 += GM_BK) {
    gemm_stage<BF16, AWQ>(st, sX, sW, tid, wrow, wblk);
    lds_barrier();
    gemm_issue<AWQ>(st, x, nib, scales, awq, tid, m0, M, K, wn_g, wblk, min(k0 + GM_BK, ke - GM_BK));
    gemm_mfma<BF16>(sX, sW, wm, wn, lane, acc);
    lds_barrier();  // the tile is rewritten by the next slice
  }

  // D[4(l/16) + e][l%16] of tile (i, j)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + fr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 32 * wm + 16 * i + 4 * (lane >> 4) + e;
        if (m < M && n < N) {
          if (SPLIT)
            atomicAdd((float*)out + (size_t)m * N + n, acc[i][j][e]);
          else
            store_out<OUT_DT>(out, (size_t)m * N + n, acc[i][j][e]);
        }
      }
    }
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float4* __restrict__ p, size_t n4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) p[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

}  // namespace nve

namespace nve_host {

template <bool BF16, bool AWQ>
static hipError_t launch_gemm_t(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                void* out, int out_dt, int N, int K, hipStream_t s) {
  const int tn = (N + nve::GM_BN - 1) / nve::GM_BN, tm = (M + nve::GM_BM - 1) / nve::GM_BM;
  // split K while the tile grid covers fewer than 512 workgroups (two per CU), keeping
  // at least 4 K iterations per split; fp32 output only (partials are added atomically)
  int split = 1;
  const int kit = K / nve::GM_BK;
  if (out_dt == NVE_DT_F32)
    while (tn * tm * split < 512 && kit / (2 * split) >= 4) split *= 2;
  if (split > 1) {
    const size_t n = (size_t)M * N;  // M * N * 4 bytes; zeroed with float4 stores when possible
    if (n % 4 == 0 && ((uintptr_t)out & 15) == 0) {
      hipLaunchKernelGGL(nve::zero_f32_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, (float4*)out, n / 4);
    } else {
      split = 1;
    }
  }
  const int k_split = ((kit + split - 1) / split) * nve::GM_BK;
  const dim3 grid(tn, tm, split);
#define NVE_GEMM(OD, SP)                                                                                       \
  hipLaunchKernelGGL((nve::gemm_w4a16_kernel<BF16, AWQ, OD, SP>), grid, dim3(512), 0, s, (const uint16_t*)x, nib, \
                     sc, awq, out, M, N, K, k_split)
  if (split > 1) {
    NVE_GEMM(NVE_DT_F32, true);
  } else {
    switch (out_dt) {
      case NVE_DT_F16: NVE_GEMM(NVE_DT_F16, false); break;
      case NVE_DT_BF16: NVE_GEMM(NVE_DT_BF16, false); break;
      default: NVE_GEMM(NVE_DT_F32, false); break;
    }
  }
#undef NVE_GEMM
  return hipGetLastError();
}

hipError_t launch_gemm_w4a16(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc, const float* awq,
                             void* out, int out_dt, int N, int K, hipStream_t s) {
  const bool bf = x_dt == NVE_DT_BF16;
  if (awq) return bf ? launch_gemm_t<true, true>(x, M, nib, sc, awq, out, out_dt, N, K, s)
                     : launch_gemm_t<false, true>(x, M, nib, sc, awq, out, out_dt, N, K, s);
  return bf ? launch_gemm_t<true, false>(x, M, nib, sc, awq, out, out_dt, N, K, s)
            : launch_gemm_t<false, false>(x, M, nib, sc, awq, out, out_dt, N, K, s);
}

}  // namespace nve_host
