// gemm_w4a16.hip -- W4A16 prefill GEMM for gfx950: Y[M, N] = X[M, K] * W[N, K]^T with
// int4 weights in the reference GPU layout and fp16 / bf16 activations.
//
// The reference's prefill path (GpuWeight::matmul_x, src/gpu_layer.rs:219-237) expands
// the weights to an fp16 matrix with nve_dequant_w4a16 (cuda/nve_kernels.cu:397-433)
// and multiplies with a dense fp16 GEMM.  This kernel computes the same product
// without the expanded matrix ever reaching HBM: each workgroup dequantizes its
// 128 x 64 weight slice once into LDS, rounded exactly as the reference's dequant
// rounds it (f32 (nibble - 8) * scale [* awq], then RNE to the activation type), and
// the tile product runs on v_mfma_f32_32x32x16_{f16,bf16} with fp32 accumulation.
// Weight traffic: 0.625 B per weight instead of 0.625 + 2 (write) + 2 (read).
//
// Tiling: 128 x 128 output tile per workgroup of 4 waves (2 x 2), 64 x 64 per wave as
// 2 x 2 MFMA tiles of 32 x 32 (v_mfma_f32_32x32x16: half the LDS operand traffic per
// flop of 16 x 16 tiles); K advances 64 per slice (two Q4 blocks).  The global
// loads (X rows, nibbles, scales) run two slices ahead of the MFMAs and the LDS is
// double-buffered, so the dequantization of slice t+1 overlaps the MFMAs of slice t and
// HBM latency overlaps the math; launches with few output tiles also split K over
// workgroups (fp32 atomic accumulation).  LDS rows are padded (72 elements) so the
// ds_read_b128 of a fragment spreads over the banks.  M <= 16 runs a separate
// weight-streaming kernel (gemm_w4a16_small_kernel below).

#include "common.h"
#include "lds_ring.h"
#include "w4_launch.h"

namespace nve {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_LD = GM_BK + 8;

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if (BF16) {
    // one v_cvt_pk_bf16_f32 (round to nearest even) of the materialised f32 values
    typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
    asm volatile("" : "+v"(a), "+v"(b));
    const bf2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  return (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(a)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(b)) << 16);
}

template <bool BF16>
__device__ __forceinline__ f4_t mfma16(uint4 a, uint4 b, f4_t c) {
  if (BF16) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

typedef float f16x_t __attribute__((ext_vector_type(16)));

template <bool BF16>
__device__ __forceinline__ f16x_t mfma32(uint4 a, uint4 b, f16x_t c) {
  if (BF16) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// Staging of one K slice, written as macros over the kernel's local registers (passing
// a staging struct by reference to helper functions left it in scratch memory).
// Thread t: X pieces (row t/8 + 32 i, columns 8 (t%8) .. +7); weight block t & 1 of
// tile row t/2 (nontemporal: read once).
#define GEMM_ISSUE(K0)                                                                          \
  do {                                                                                          \
    const uint16_t* xp_ = x + (size_t)(K0) + 8 * xc8;                                           \
    rx0 = *(const uint4*)(xp_ + (size_t)min(m0 + xr, M - 1) * K);                               \
    rx1 = *(const uint4*)(xp_ + (size_t)min(m0 + xr + 32, M - 1) * K);                          \
    rx2 = *(const uint4*)(xp_ + (size_t)min(m0 + xr + 64, M - 1) * K);                          \
    rx3 = *(const uint4*)(xp_ + (size_t)min(m0 + xr + 96, M - 1) * K);                          \
    const int b_ = ((K0) >> 5) + wblk;                                                          \
    rn = ld_stream((const uint4*)(nib + (size_t)wn_g * (K >> 1)) + b_);                         \
    rs = scales[(size_t)wn_g * (K >> 5) + b_];                                                  \
    if (AWQ) {                                                                                  \
      _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) ra[i_] = ((const float4*)(awq + 32 * b_))[i_]; \
    }                                                                                           \
  } while (0)

// X pieces to LDS; the weight block dequantized and rounded to the activation type into
// LDS.  (nibble - 8) * s is formed as fma(nibble, s, -8 s): -8 s is exact and n s - 8 s
// is the exact product (n - 8) s, so the fma's single rounding equals the f32 product
// the reference forms; byte extracts of the masked dword become v_cvt_f32_ubyte{0..3}
// (element j = low nibble of byte j, element j + 16 = high nibble).  pack2 then rounds
// each f32 value to the 16-bit type (two roundings, as the reference's dequant).
#define GEMM_STAGE(DX, DW)                                                                      \
  do {                                                                                          \
    uint16_t* xd_ = (DX) + xr * GM_LD + 8 * xc8;                                                \
    *(uint4*)(xd_) = rx0;                                                                       \
    *(uint4*)(xd_ + 32 * GM_LD) = rx1;                                                          \
    *(uint4*)(xd_ + 64 * GM_LD) = rx2;                                                          \
    *(uint4*)(xd_ + 96 * GM_LD) = rx3;                                                          \
    const uint32_t d_[4] = {rn.x, rn.y, rn.z, rn.w};                                            \
    const float s8_ = -8.0f * rs;                                                               \
    float v_[32];                                                                               \
    _Pragma("unroll") for (int t_ = 0; t_ < 4; ++t_) {                                          \
      const uint32_t lo_ = d_[t_] & 0x0F0F0F0Fu, hi_ = (d_[t_] >> 4) & 0x0F0F0F0Fu;             \
      v_[4 * t_ + 0] = fmaf((float)(lo_ & 0xffu), rs, s8_);                                     \
      v_[4 * t_ + 1] = fmaf((float)((lo_ >> 8) & 0xffu), rs, s8_);                              \
      v_[4 * t_ + 2] = fmaf((float)((lo_ >> 16) & 0xffu), rs, s8_);                             \
      v_[4 * t_ + 3] = fmaf((float)(lo_ >> 24), rs, s8_);                                       \
      v_[16 + 4 * t_ + 0] = fmaf((float)(hi_ & 0xffu), rs, s8_);                                \
      v_[16 + 4 * t_ + 1] = fmaf((float)((hi_ >> 8) & 0xffu), rs, s8_);                         \
      v_[16 + 4 * t_ + 2] = fmaf((float)((hi_ >> 16) & 0xffu), rs, s8_);                        \
      v_[16 + 4 * t_ + 3] = fmaf((float)(hi_ >> 24), rs, s8_);                                  \
    }                                                                                           \
    if (AWQ) {                                                                                  \
      _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_) {                                        \
        v_[4 * i_] *= ra[i_].x;                                                                 \
        v_[4 * i_ + 1] *= ra[i_].y;                                                             \
        v_[4 * i_ + 2] *= ra[i_].z;                                                             \
        v_[4 * i_ + 3] *= ra[i_].w;                                                             \
      }                                                                                         \
    }                                                                                           \
    uint16_t* dst_ = (DW) + wrow * GM_LD + 32 * wblk;                                           \
    _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_)                                            \
      *(uint4*)(dst_ + 8 * q_) =                                                                \
          make_uint4(pack2<BF16>(v_[8 * q_], v_[8 * q_ + 1]), pack2<BF16>(v_[8 * q_ + 2], v_[8 * q_ + 3]), \
                     pack2<BF16>(v_[8 * q_ + 4], v_[8 * q_ + 5]), pack2<BF16>(v_[8 * q_ + 6], v_[8 * q_ + 7])); \
  } while (0)

// The wave's 2 x 2 tiles of 32 x 32 (64 rows x 64 columns) over one staged K slice:
// v_mfma_f32_32x32x16, lane l supplies A[l%32][8(l/32) .. +7] and B[8(l/32) .. +7][l%32].
template <bool BF16>
__device__ __forceinline__ void gemm_mfma(const uint16_t* sX, const uint16_t* sW, int wm, int wn, int lane,
                                          f16x_t (&acc)[2][2]) {
  const int fr = lane & 31, fk = 8 * (lane >> 5);
#pragma unroll
  for (int kk = 0; kk < GM_BK; kk += 16) {
    uint4 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = *(const uint4*)(sX + (64 * wm + 32 * i + fr) * GM_LD + kk + fk);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = *(const uint4*)(sW + (64 * wn + 32 * j + fr) * GM_LD + kk + fk);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<BF16>(a[i], b[j], acc[i][j]);
  }
}

// SPLIT: the K range is divided over gridDim.z workgroups per output tile (launches
// whose tile grid alone would leave most CUs idle: small M).  SPLIT_PARTS: workgroup z
// stores its partial tile to out + z * M * N and split_reduce_kernel adds the partials
// in the order z = 0, 1, ... (bit-reproducible; no atomic accumulation anywhere).
enum { SPLIT_NONE = 0, SPLIT_PARTS = 2 };
template <bool BF16, bool AWQ, int OUT_DT, int SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_w4a16_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ nib, const float* __restrict__ scales,
    const float* __restrict__ awq, void* __restrict__ out, int M, int N, int K, int k_split) {
  // two LDS buffers: slice t+1 is staged (dequantized) into one while the MFMAs of
  // slice t read the other, so VALU and MFMA work of a wave overlap
  __shared__ __align__(16) uint16_t sX[2][GM_BM * GM_LD];
  __shared__ __align__(16) uint16_t sW[2][GM_BN * GM_LD];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 2 x 2 waves: 64 rows x 64 columns each
  const int m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;

  uint4 rx0, rx1, rx2, rx3, rn;
  float rs;
  float4 ra[AWQ ? 8 : 1];
  const int xr = tid >> 3, xc8 = tid & 7;
  const int wrow = tid >> 1, wblk = tid & 1;  // weight row in the tile, block within the slice
  const int wn_g = min(n0 + wrow, N - 1);

  f16x_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f16x_t{};

  const int kb = SPLIT ? blockIdx.z * k_split : 0;
  const int ke = SPLIT ? min(K, kb + k_split) : K;
  // global loads run two slices ahead of the MFMAs, staging one slice ahead; the
  // issues are unconditional (slices past the range re-read the last one), which keeps
  // the staging registers out of a conditional merge
  const int klast = ke - GM_BK;
  GEMM_ISSUE(kb);
  GEMM_STAGE(sX[0], sW[0]);
  GEMM_ISSUE(min(kb + GM_BK, klast));
  lds_barrier();
  for (int k0 = kb; k0 < ke; k0 += 2 * GM_BK) {
    // slice k0 is in buffer 0; stage k0 + BK into buffer 1 while multiplying buffer 0
    GEMM_STAGE(sX[1], sW[1]);
    GEMM_ISSUE(min(k0 + 2 * GM_BK, klast));
    gemm_mfma<BF16>(sX[0], sW[0], wm, wn, lane, acc);
    lds_barrier();
    // slice k0 + BK is in buffer 1; stage k0 + 2 BK into buffer 0 while multiplying it
    GEMM_STAGE(sX[0], sW[0]);
    GEMM_ISSUE(min(k0 + 3 * GM_BK, klast));
    if (k0 + GM_BK < ke) gemm_mfma<BF16>(sX[1], sW[1], wm, wn, lane, acc);
    lds_barrier();
  }

  // 32x32 result layout: register r of lane l holds D[8 (r/4) + 4 (l/32) + r%4][l%32]
  const int fr = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wn + 32 * j + fr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < M && n < N) {
          if (SPLIT == SPLIT_PARTS)
            ((float*)out)[(size_t)blockIdx.z * M * N + (size_t)m * N + n] = acc[i][j][r];
          else
            store_out<OUT_DT>(out, (size_t)m * N + n, acc[i][j][r]);
        }
      }
    }
}

// ---- small M (M <= 16): weight-streaming form ---------------------------------
// For a few activation rows the tile GEMM above re-dequantizes little and streams
// less: this kernel is the batched-GEMV layout of the W4A8 MFMA kernel with a fp16 /
// bf16 MFMA (v_mfma_f32_16x16x32_{f16,bf16}).  The activation rows are the A operand
// (rows i; activation row m sits in A row 4 (m % 4) + m / 4), a 16-row weight tile
// the B operand; lane group g of a block takes the k-set {4g..4g+3} u {16+4g..16+4g+3}
// -- the low and high nibbles of nibble dword g -- in A and B alike.  The B operand is
// the reference dequant, rounded exactly as nve_dequant_w4a16 rounds it:
// fma(n, s, -8 s) (= the f32 product (n - 8) s) [* awq], materialised as f32, then RNE
// to fp16 / bf16 (v_cvt_pk_{f16,bf16}_f32); the fp32 MFMA accumulator runs over all of
// K, so there is no per-block epilogue.  Loads are issued row-major (4 consecutive
// lanes on 64 contiguous bytes of one row) and moved to the operand lanes with
// ds_bpermute and the 4x4 lane-group transpose; a workgroup owns T tiles and its 16
// waves deal the K quads (4 blocks) round-robin.
template <bool BF16, bool AWQ, int T>
struct SmallQuad {
  uint2 xl[4], xh[4];  // block 4q+j of activation row r: elements 4p..4p+3, 16+4p..16+4p+3
  uint4 w[T];          // block 4q+p of weight row r
  float4 sc[T];        // scales of the quad's 4 blocks, weight row r
  float4 al[AWQ ? 4 : 1], ah[AWQ ? 4 : 1];  // awq at the lane's k-set of each block
};

template <bool BF16>
__device__ __forceinline__ uint32_t cvt_pk(float a, float b) {
  // the f32 values are materialised first: a fused multiply-convert would round the
  // exact product once instead of rounding the f32 product
  asm volatile("" : "+v"(a), "+v"(b));
  if (BF16) {
    typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
    const bf2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  const half2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

template <bool BF16, bool AWQ, int T>
__device__ __forceinline__ void small_issue(SmallQuad<BF16, AWQ, T>& st, const uint2* xrow, const float* awq,
                                            const uint4* const (&wrow)[T], const float* const (&srow)[T],
                                            int vec_sc, int q, int nb, int g, int lp) {
  // activations (block 4q+j: 8-byte pieces p and 4+p of the 64-byte block row), weights
  // and scales (clamped to the last block: weighted 0 at use)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = min(4 * q + j, nb - 1);
    st.xl[j] = xrow[8 * b + lp];
    st.xh[j] = xrow[8 * b + 4 + lp];
    if (AWQ) {
      st.al[j] = *(const float4*)(awq + 32 * b + 4 * g);
      st.ah[j] = *(const float4*)(awq + 32 * b + 16 + 4 * g);
    }
  }
  const int bl = min(4 * q + lp, nb - 1);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    st.w[t] = ld_stream(wrow[t] + bl);
    if (vec_sc) {
      st.sc[t] = ((const float4*)srow[t])[q];
    } else {
      st.sc[t].x = srow[t][min(4 * q + 0, nb - 1)];
      st.sc[t].y = srow[t][min(4 * q + 1, nb - 1)];
      st.sc[t].z = srow[t][min(4 * q + 2, nb - 1)];
      st.sc[t].w = srow[t][min(4 * q + 3, nb - 1)];
    }
  }
}

template <bool BF16, bool AWQ, int T>
__device__ __forceinline__ void small_compute(const SmallQuad<BF16, AWQ, T>& st, int q, int nb, bool m_ok, int src_w,
                                              int src_x, f4_t (&acc)[T]) {
  // A operands: lane (i, g) <- load lane (m(i), g)
  uint4 a[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t d0 = lane_fetch(st.xl[j].x, src_x), d1 = lane_fetch(st.xl[j].y, src_x);
    const uint32_t d2 = lane_fetch(st.xh[j].x, src_x), d3 = lane_fetch(st.xh[j].y, src_x);
    a[j] = m_ok ? make_uint4(d0, d1, d2, d3) : make_uint4(0, 0, 0, 0);
  }
  const bool full = 4 * q + 3 < nb;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint4 w = lane_fetch4(st.w[t], src_w);
    uint32_t c0 = w.x, c1 = w.y, c2 = w.z, c3 = w.w;
    transpose4(c0, c1, c2, c3);  // lane (n, g): nibble dword g of blocks 4q+0..3
    const uint32_t cj[4] = {c0, c1, c2, c3};
    const uint4 sw = lane_fetch4(make_uint4(__float_as_uint(st.sc[t].x), __float_as_uint(st.sc[t].y),
                                            __float_as_uint(st.sc[t].z), __float_as_uint(st.sc[t].w)),
                                 src_w);
    const float scj[4] = {__uint_as_float(sw.x), __uint_as_float(sw.y), __uint_as_float(sw.z),
                          __uint_as_float(sw.w)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = scj[j], s8 = -8.0f * s;
      const uint32_t lo = cj[j] & 0x0F0F0F0Fu, hi = (cj[j] >> 4) & 0x0F0F0F0Fu;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = fmaf((float)((lo >> (8 * e)) & 0xffu), s, s8);
        v[4 + e] = fmaf((float)((hi >> (8 * e)) & 0xffu), s, s8);
      }
      if (AWQ) {
        const float al[4] = {st.al[j].x, st.al[j].y, st.al[j].z, st.al[j].w};
        const float ah[4] = {st.ah[j].x, st.ah[j].y, st.ah[j].z, st.ah[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] *= al[e];
          v[4 + e] *= ah[e];
        }
      }
      uint4 b = make_uint4(cvt_pk<BF16>(v[0], v[1]), cvt_pk<BF16>(v[2], v[3]), cvt_pk<BF16>(v[4], v[5]),
                           cvt_pk<BF16>(v[6], v[7]));
      // blocks past the end (last quad only) were loaded clamped: multiply zeros
      if (!(full || 4 * q + j < nb)) b = make_uint4(0, 0, 0, 0);
      acc[t] = mfma16<BF16>(a[j], b, acc[t]);
    }
  }
}

template <bool BF16, bool AWQ, int OUT_DT, int KS, int T>
__global__ __launch_bounds__(64 * KS) void gemm_w4a16_small_kernel(const uint16_t* __restrict__ x,
                                                                   const uint8_t* __restrict__ nib,
                                                                   const float* __restrict__ ws,
                                                                   const float* __restrict__ awq,
                                                                   void* __restrict__ out, int M, int N, int K,
                                                                   int vec_sc) {
  __shared__ float s_red[KS][T * 16][17];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;  // operand layout
  const int lr = lane >> 2, lp = lane & 3;  // load layout
  const int row0 = blockIdx.x * (16 * T);
  const int nb = K >> 5;
  const int nq = (nb + 3) >> 2;
  const size_t row_bytes = (size_t)(K >> 1);
  const uint4* wrow[T];
  const float* srow[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int r = min(row0 + 16 * t + lr, N - 1);
    wrow[t] = (const uint4*)(nib + (size_t)r * row_bytes);
    srow[t] = ws + (size_t)r * nb;
  }
  const uint2* xrow = (const uint2*)(x + (size_t)min(lr, M - 1) * K);  // 8-byte units
  const int am = 4 * (nl & 3) + (nl >> 2);
  const bool m_ok = am < M;
  const int src_w = 4 * nl + g, src_x = 4 * am + g;
  f4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int q = wave; q < nq; q += KS) {
    SmallQuad<BF16, AWQ, T> st;
    small_issue<BF16, AWQ, T>(st, xrow, awq, wrow, srow, vec_sc, q, nb, g, lp);
    small_compute<BF16, AWQ, T>(st, q, nb, m_ok, src_w, src_x, acc);
  }
  // D layout: lane (n, g) holds rows i = 4g + e (activation row 4e + g) of column n
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_red[wave][16 * t + nl][4 * e + g] = acc[t][e];
  __syncthreads();
  for (int i = threadIdx.x; i < T * 16 * 16; i += 64 * KS) {
    const int mm = i / (16 * T), r = i % (16 * T);
    float y = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < KS; ++w2) y += s_red[w2][r][mm];
    if (mm < M && row0 + r < N) store_out<OUT_DT>(out, (size_t)mm * N + row0 + r, y);
  }
}

// ---- small M (M <= 64), K % 128 == 0: the LDS-ring form ------------------------------
// The weight-streaming kernel above with the W4A8 batched kernel's LDS ring
// (gemv_w4a8_batched.hip) in place of its VGPR loads and ds_bpermute moves: every load
// is a global -> LDS transfer into a per-wave slot holding one K quad --
//   W  T x 1 KiB   weight tile t, 16 rows x 64 B (4 lanes per row), pieces swizzled as
//                  in the W4A8 ring (load lane (row a, slot s) fetches piece (s - a/2) & 3)
//   SC T x 256 B   the tile's 16 x 4 block scales
//   A  EU x 1 KiB  activation rows 4a..4a+3 of the quad, 256 B each (4 blocks of 32
//                  fp16 / bf16), the 16-byte pieces of row r stored at piece ^ (r & 15)
//                  so that the 16 rows' reads of one k-set fall on different banks
//   AW 512 B       (AWQ) the quad's 128 activation-scale factors, one transfer of 32 lanes
// -- and the operand lanes read the slot: the weight piece (ds_read_b128 and the 4x4
// permlane transpose: nibble dword g of the 4 blocks), the row's scales, and per block
// the two 8-byte k-runs {4g..4g+3} and {16+4g..16+4g+3} of the activation row.  The
// nibbles are extracted low / high per byte, which yields that same k order, so the B
// operand (the reference dequant f16/bf16(fma(n, s, -8 s)), as above) needs no permute.
// KS waves with S quads in flight each (the launcher: 16 waves, one quad; 8 waves where
// 32 activation rows form two operand groups); workgroups take ceil(N / 256) rows each
// (one per CU), the last tile partly masked (masked lanes issue no transfers; lane 0
// always does, so every wave instruction counts once and the vmcnt waits are exact).
template <int T, int EU, bool AWQ>
struct W16Ring {
  static constexpr int W = 0, SC = T * 1024, A = SC + T * 256, AW = A + EU * 1024;
  static constexpr int SLOT = AW + (AWQ ? 512 : 0);
  static constexpr int LOADS = 2 * T + EU + (AWQ ? 1 : 0);
};

template <bool BF16, bool AWQ, int OUT_DT, int T, int EU, int KS, int S>
__global__ __launch_bounds__(64 * KS) void gemm_w4a16_ring_kernel(const uint16_t* __restrict__ x,
                                                               const uint8_t* __restrict__ nib,
                                                               const float* __restrict__ ws,
                                                               const float* __restrict__ awq,
                                                               void* __restrict__ out, int M, int N, int K,
                                                               int rows_per_wg) {
  static_assert(S >= 1 && S <= 2, "ring depth");
  using L = W16Ring<T, EU, AWQ>;
  // EU activation transfers of 4 rows: up to 16 rows form one A operand group, 32 / 64
  // rows (EU = 8 / 16) two / four groups that share every dequantized weight fragment
  constexpr int MG = EU > 4 ? EU / 4 : 1, EG = EU > 4 ? 4 : EU;
  constexpr int kRing = KS * S * L::SLOT;
  constexpr int kRed = KS * T * 16 * (4 * EU + 1) * 4;
  __shared__ __attribute__((aligned(16))) char smem[kRing > kRed ? kRing : kRed];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nl = lane & 15, g = lane >> 4;  // operand layout
  const int lr = lane >> 2, lp = lane & 3;  // weight load layout
  const int row0 = blockIdx.x * rows_per_wg;
  const int nb = K >> 5, nq = nb >> 2;
  const int nqw = (nq + KS - 1) / KS;
  char* const ring = smem + wave * (S * L::SLOT);

  const uint8_t* wsrc[T];
  const float* ssrc[T];
  bool wok[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int rr = 16 * t + lr;
    const int r = min(row0 + rr, N - 1);
    wok[t] = (rr < rows_per_wg && row0 + rr < N) || lane == 0;
    wsrc[t] = nib + (size_t)r * (K >> 1) + 16 * ((lp - (lr >> 1)) & 3);
    ssrc[t] = ws + (size_t)r * nb + lp;
  }
  // activation transfer a: lane l -> row 4a + l / 16, stored piece l % 16 = source piece ^ row
  const char* asrc[EU];
  bool aok[EU];
#pragma unroll
  for (int a = 0; a < EU; ++a) {
    const int m = 4 * a + (lane >> 4);
    aok[a] = m < M || lane == 0;
    asrc[a] = (const char*)(x + (size_t)min(m, M - 1) * K) + 16 * ((lane & 15) ^ (m & 15));
  }
  auto issue = [&](int i) {
    const int q = min(wave + KS * i, nq - 1);
    char* const sb = ring + (i % S) * L::SLOT;
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (wok[t]) lds_dma16(wsrc[t] + 64 * q, sb + L::W + t * 1024);
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (wok[t]) lds_dma4(ssrc[t] + 4 * q, sb + L::SC + t * 256);
#pragma unroll
    for (int a = 0; a < EU; ++a)
      if (aok[a]) lds_dma16(asrc[a] + 256 * q, sb + L::A + a * 1024);
    if (AWQ && lane < 32) lds_dma16(awq + 128 * q + 4 * lane, sb + L::AW);
  };

  // A row nl of group G holds activation row 16 G + am (rows >= M read row M - 1,
  // never stored)
  const int am = 4 * (nl & 3) + (nl >> 2);
  const uint32_t rd_w = 16 * (4 * nl + ((g + (nl >> 1)) & 3));
  uint32_t rd_lo[MG][4], rd_hi[MG][4];
#pragma unroll
  for (int G = 0; G < MG; ++G) {
    const int ar = min(16 * G + am, M - 1);
    const uint32_t rb = L::A + (ar >> 2) * 1024 + (ar & 3) * 256 + 8 * (g & 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rd_lo[G][j] = rb + 16 * ((4 * j + (g >> 1)) ^ (ar & 15));
      rd_hi[G][j] = rb + 16 * ((4 * j + 2 + (g >> 1)) ^ (ar & 15));
    }
  }
  f4_t acc[T][MG];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int G = 0; G < MG; ++G) acc[t][G] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int i) {
    if (wave + KS * i >= nq) return;  // clamped duplicate quad (wave-uniform)
    const uint32_t sb = lds_addr(ring + (i % S) * L::SLOT);
    u32x2_t xl[MG][4], xh[MG][4];
#pragma unroll
    for (int G = 0; G < MG; ++G)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xl[G][j] = ds_read64(sb + rd_lo[G][j]);
        xh[G][j] = ds_read64(sb + rd_hi[G][j]);
      }
    u32x4_t wr[T], sr[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      wr[t] = ds_read128(sb + L::W + t * 1024 + rd_w);
      sr[t] = ds_read128(sb + L::SC + t * 256 + nl * 16);
    }
    // awq at the lane's k-runs of each block
    u32x4_t al[AWQ ? 4 : 1], ah[AWQ ? 4 : 1];
    if constexpr (AWQ) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        al[j] = ds_read128(sb + L::AW + 4 * (32 * j + 4 * g));
        ah[j] = ds_read128(sb + L::AW + 4 * (32 * j + 16 + 4 * g));
      }
    }
    lgkm_wait();
    if constexpr (AWQ) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tie(al[j]);
        tie(ah[j]);
      }
    }
#pragma unroll
    for (int G = 0; G < MG; ++G)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tie(xl[G][j]);
        tie(xh[G][j]);
      }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      tie(wr[t]);
      tie(sr[t]);
    }
    uint4 a[MG][4];
#pragma unroll
    for (int G = 0; G < MG; ++G)
#pragma unroll
      for (int j = 0; j < 4; ++j) a[G][j] = make_uint4(xl[G][j].x, xl[G][j].y, xh[G][j].x, xh[G][j].y);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t c0 = wr[t].x, c1 = wr[t].y, c2 = wr[t].z, c3 = wr[t].w;
      transpose4(c0, c1, c2, c3);  // lane (n, g): nibble dword g of blocks 4q+0..3
      const uint32_t cj[4] = {c0, c1, c2, c3};
      const float scj[4] = {__uint_as_float(sr[t].x), __uint_as_float(sr[t].y), __uint_as_float(sr[t].z),
                            __uint_as_float(sr[t].w)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float s = scj[j], s8 = -8.0f * s;
        const uint32_t lo = cj[j] & 0x0F0F0F0Fu, hi = (cj[j] >> 4) & 0x0F0F0F0Fu;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = fmaf((float)((lo >> (8 * e)) & 0xffu), s, s8);
          v[4 + e] = fmaf((float)((hi >> (8 * e)) & 0xffu), s, s8);
        }
        if constexpr (AWQ) {
          const uint32_t l4[4] = {al[j].x, al[j].y, al[j].z, al[j].w};
          const uint32_t h4[4] = {ah[j].x, ah[j].y, ah[j].z, ah[j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] *= __uint_as_float(l4[e]);
            v[4 + e] *= __uint_as_float(h4[e]);
          }
        }
        const uint4 b = make_uint4(cvt_pk<BF16>(v[0], v[1]), cvt_pk<BF16>(v[2], v[3]), cvt_pk<BF16>(v[4], v[5]),
                                   cvt_pk<BF16>(v[6], v[7]));
#pragma unroll
        for (int G = 0; G < MG; ++G) acc[t][G] = mfma16<BF16>(a[G][j], b, acc[t][G]);
      }
    }
  };

  // S quads in flight: the transfers of quad i + S - 1 are issued before quad i is
  // computed; every quad is the same LOADS transfers (clamped quads past the wave's
  // share included), so the waits are exact.
#pragma unroll
  for (int k = 0; k < S; ++k)
    if (k < nqw) issue(k);
  int i = 0;
  for (; i + S < nqw; ++i) {
    wait_vmcnt<(S - 1) * L::LOADS>();
    __builtin_amdgcn_sched_barrier(0);
    compute(i);
    __builtin_amdgcn_sched_barrier(0);
    issue(i + S);
  }
  for (; i < nqw; ++i) {
    if (i + 1 < nqw) wait_vmcnt<(S - 1) * L::LOADS>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    compute(i);
  }

  __syncthreads();  // every wave is done with its slot: reuse the LDS for the reduction
  float(*s_red)[T * 16][4 * EU + 1] = (float(*)[T * 16][4 * EU + 1])smem;
  // D layout: lane (n, g) of group G holds rows i = 4g + e (activation row
  // 16 G + 4e + g) of column n
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int G = 0; G < MG; ++G)
#pragma unroll
      for (int e = 0; e < EG; ++e) s_red[wave][16 * t + nl][16 * G + 4 * e + g] = acc[t][G][e];
  __syncthreads();
  const int rows = min(rows_per_wg, N - row0);
  for (int xi = threadIdx.x; xi < T * 16 * 4 * EU; xi += 64 * KS) {
    const int mm = xi / (16 * T), r = xi % (16 * T);
    float y = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < KS; ++w2) y += s_red[w2][r][mm];
    if (mm < M && r < rows) store_out<OUT_DT>(out, (size_t)mm * N + row0 + r, y);
  }
}

// out[i] = sum over z = 0 .. split-1 of part[z * n + i], in that order.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           size_t n, int split) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float y = part[i];
  for (int z = 1; z < split; ++z) y += part[(size_t)z * n + i];
  out[i] = y;
}

#undef GEMM_ISSUE
#undef GEMM_STAGE

}  // namespace nve

namespace nve_host {

constexpr int kGemmSmallM = 16;
// the register-dequant tile kernel's first M: without K-split partials, and with them
// (from the first M the ring takes in two launches; workspace path, fp32 out, us: 8B gate
// M = 80 / 96 / 112 32.5 / 32.9 / 33.4 against 35.8 / 37.7 / 43.8 for the ring launches,
// 8B down 29.8 / 30.0 / 31.2 against 39.8 / 45.8 / 54.4; at M = 64, one ring launch, 31.5
// / 28.9 against 24.1 / 28.3)
constexpr int kGemmTileMinM = 128;
constexpr int kGemmTileSplitMinM = 65;
constexpr int kSmallKS = 16;

// K splits of the tiled kernel: split while the tile grid covers fewer than 512
// workgroups (two per CU), keeping at least 4 K iterations per split; fp32 output only.
static int gemm_split(int M, int N, int K, int out_dt) {
  const int tn = (N + nve::GM_BN - 1) / nve::GM_BN, tm = (M + nve::GM_BM - 1) / nve::GM_BM;
  int split = 1;
  const int kit = K / nve::GM_BK;
  if (out_dt == NVE_DT_F32 && M > kGemmSmallM)
    while (tn * tm * split < 512 && kit / (2 * split) >= 4) split *= 2;
  return split;
}

// Bytes of fp32 partials the bit-reproducible splits need (0: no split): that of this
// file's tiled kernel or that of the register-dequant tile kernel, whichever is larger.
size_t gemm_split_parts_bytes(int M, int N, int K) {
  const int split = gemm_split(M, N, K, NVE_DT_F32);
  const size_t own = split > 1 ? (size_t)split * M * N * sizeof(float) : 0;
  const size_t tile = M >= kGemmTileSplitMinM ? gemm_tile_parts_bytes(M, N, K) : 0;
  return own > tile ? own : tile;
}

// parts (parts_bytes >= gemm_split_parts_bytes): a split launch stores its partials
// there and adds them in a fixed order; without them the product is not split, so every
// call gives the same bits.
template <bool BF16, bool AWQ>
static hipError_t launch_gemm_t(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                void* out, int out_dt, int N, int K, float* parts, size_t parts_bytes,
                                hipStream_t s) {
  const int tn = (N + nve::GM_BN - 1) / nve::GM_BN, tm = (M + nve::GM_BM - 1) / nve::GM_BM;
  int split = gemm_split(M, N, K, out_dt);
  const int kit = K / nve::GM_BK;
  const size_t n = (size_t)M * N;
  if (split > 1 && !(parts && parts_bytes >= (size_t)split * n * sizeof(float)))
    split = 1;  // no room for the partials: one pass over K
  const int k_split = ((kit + split - 1) / split) * nve::GM_BK;
  const dim3 grid(tn, tm, split);
#define NVE_GEMM(OD, SP, O)                                                                                    \
  hipLaunchKernelGGL((nve::gemm_w4a16_kernel<BF16, AWQ, OD, SP>), grid, dim3(256), 0, s, (const uint16_t*)x, nib, \
                     sc, awq, O, M, N, K, k_split)
  if (split > 1) {
    NVE_GEMM(NVE_DT_F32, nve::SPLIT_PARTS, (void*)parts);
    hipLaunchKernelGGL(nve::split_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, parts,
                       (float*)out, n, split);
  } else {
    switch (out_dt) {
      case NVE_DT_F16: NVE_GEMM(NVE_DT_F16, nve::SPLIT_NONE, out); break;
      case NVE_DT_BF16: NVE_GEMM(NVE_DT_BF16, nve::SPLIT_NONE, out); break;
      default: NVE_GEMM(NVE_DT_F32, nve::SPLIT_NONE, out); break;
    }
  }
#undef NVE_GEMM
  return hipGetLastError();
}

// M <= 16: the weight-streaming kernel (two 16-row tiles per workgroup while that
// leaves at least 256 workgroups, else one; 16 waves per workgroup).
template <bool BF16, bool AWQ, int OUT_DT>
static hipError_t launch_small_o(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                 void* out, int N, int K, hipStream_t s) {
  const int vec_sc = (K % 128 == 0) && aligned(sc, 16);
  if ((N + 31) / 32 >= 256)
    hipLaunchKernelGGL((nve::gemm_w4a16_small_kernel<BF16, AWQ, OUT_DT, kSmallKS, 2>), dim3((N + 31) / 32),
                       dim3(64 * kSmallKS), 0, s, (const uint16_t*)x, nib, sc, awq, out, M, N, K, vec_sc);
  else
    hipLaunchKernelGGL((nve::gemm_w4a16_small_kernel<BF16, AWQ, OUT_DT, kSmallKS, 1>), dim3((N + 15) / 16),
                       dim3(64 * kSmallKS), 0, s, (const uint16_t*)x, nib, sc, awq, out, M, N, K, vec_sc);
  return hipGetLastError();
}

// M <= 64 (32 with AWQ), K % 128 == 0, N <= 16384: the LDS-ring kernel, ceil(N / 256)
// rows per workgroup (16 below 4096 rows), one activation transfer per 4 rows of M.
template <bool BF16, bool AWQ, int OUT_DT, int T>
static hipError_t launch_ring_t(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq, void* out,
                                int N, int K, int rpw, hipStream_t s) {
  const dim3 grid((N + rpw - 1) / rpw);
  // 16 waves, one quad in flight each (8B gate, fp16 x, M = 1 / 4 / 16: 12.1 / 11.9-12.1 /
  // 12.5-12.8 us; 8 waves with two quads in flight 12.6 / 12.5-12.6 / 13.3-13.4, 8 waves
  // with one 13.4-13.7 / 13.1 / 13.9-14.0)
  // M = 17-32 / 33-64: two / four 16-row operand groups per dequantized weight fragment;
  // their 8 / 16 KiB of activation rows per slot leave LDS for 8 / 6 waves (four groups
  // without AWQ only: with it the kernel needs more than 256 VGPRs)
#define NVE_R16(EU, KS) \
  hipLaunchKernelGGL((nve::gemm_w4a16_ring_kernel<BF16, AWQ, OUT_DT, T, EU, KS, 1>), grid, dim3(64 * KS), 0, s, \
                     (const uint16_t*)x, nib, sc, awq, out, M, N, K, rpw)
  if (M <= 4) NVE_R16(1, 16);
  else if (M <= 8) NVE_R16(2, 16);
  else if (M <= 16) NVE_R16(4, 16);
  else if (AWQ || M <= 32) NVE_R16(8, 8);
  else if constexpr (!AWQ) NVE_R16(16, 6);
#undef NVE_R16
  return hipGetLastError();
}

template <bool BF16, bool AWQ, int OUT_DT>
static hipError_t launch_ring_o(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq, void* out,
                                int N, int K, hipStream_t s) {
  const int rpw = N <= 4096 ? 16 : (N + 255) / 256;
  const int T = (rpw + 15) / 16;
  if (T == 1) return launch_ring_t<BF16, AWQ, OUT_DT, 1>(x, M, nib, sc, awq, out, N, K, rpw, s);
  if (T == 2) return launch_ring_t<BF16, AWQ, OUT_DT, 2>(x, M, nib, sc, awq, out, N, K, rpw, s);
  if (T == 3) return launch_ring_t<BF16, AWQ, OUT_DT, 3>(x, M, nib, sc, awq, out, N, K, rpw, s);
  return launch_ring_t<BF16, AWQ, OUT_DT, 4>(x, M, nib, sc, awq, out, N, K, rpw, s);
}

// rows one ring launch takes (without / with AWQ) and the M up to which launches of that
// many rows beat the tiled kernel
static int ring_rows(bool awq) { return awq ? 32 : 64; }
// 8B gate, 64-row launches: 62.5 / 83.0 / 103.7 / 124.5 us at M = 192 / 256 / 320 / 384
// against 76.7 / 88.1 / 109.8 / 116.4 for the tiled kernel; 32-row launches (AWQ) stop
// winning above 128 rows
static int ring_chunked_max(bool awq) { return awq ? 128 : 320; }
static bool ring_fits(int M, int N, int K, bool awq) {
  return M <= ring_rows(awq) && K % 128 == 0 && N <= 16384;
}

template <bool BF16, bool AWQ>
static hipError_t launch_small(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                               void* out, int out_dt, int N, int K, hipStream_t s) {
  if (ring_fits(M, N, K, AWQ)) {
    switch (out_dt) {
      case NVE_DT_F16: return launch_ring_o<BF16, AWQ, NVE_DT_F16>(x, M, nib, sc, awq, out, N, K, s);
      case NVE_DT_BF16: return launch_ring_o<BF16, AWQ, NVE_DT_BF16>(x, M, nib, sc, awq, out, N, K, s);
      default: return launch_ring_o<BF16, AWQ, NVE_DT_F32>(x, M, nib, sc, awq, out, N, K, s);
    }
  }
  switch (out_dt) {
    case NVE_DT_F16: return launch_small_o<BF16, AWQ, NVE_DT_F16>(x, M, nib, sc, awq, out, N, K, s);
    case NVE_DT_BF16: return launch_small_o<BF16, AWQ, NVE_DT_BF16>(x, M, nib, sc, awq, out, N, K, s);
    default: return launch_small_o<BF16, AWQ, NVE_DT_F32>(x, M, nib, sc, awq, out, N, K, s);
  }
}

hipError_t launch_gemm_w4a16_parts(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                   const float* awq, void* out, int out_dt, int N, int K, float* parts,
                                   size_t parts_bytes, hipStream_t s) {
  const bool bf = x_dt == NVE_DT_BF16;
  // from M = 128 (K % 128 == 0) the 128- / 256-row tile kernel of
  // gemm_w4a16_tile.hip (with AWQ from M = 65); with K-split partials from M = 65.  Without
  // them it runs up to the ring launches' range (320 rows, AWQ 128) only where its 128-row
  // grid has at least 96 workgroups: one workgroup streams all of K, so a narrow grid
  // leaves the chip idle (fp16 out, us: 8B gate M = 128 / 192 / 256 45.5 / 51.2 / 51.4
  // against 47.9 / 72.0 / 95.5 for the ring launches; 8B down, 32 column tiles, M = 256:
  // 133.8 against 120.9 for the ring; above that range the tile kernel beats the 128 x
  // 128-tile kernel below at both: gate M = 512 81.4 against 124.6, down 143 against
  // 243).  With the partials a narrow grid is split over K instead.
  if (M >= kGemmTileSplitMinM && gemm_tile_fits(M, N, K, awq != nullptr)) {
    const size_t tp = gemm_tile_parts_bytes(M, N, K);
    const bool split = parts && tp > 0 && parts_bytes >= tp;
    // (AWQ: from M = 65, where the 32-row ring launches number three or more)
    const int tile_min = awq ? kGemmTileSplitMinM : kGemmTileMinM;
    if (split || M > ring_chunked_max(awq != nullptr) || (M >= tile_min && gemm_tile_grid128(M, N) >= 96))
      return launch_gemm_w4a16_tile(x, x_dt, M, nib, sc, awq, out, out_dt, N, K, split ? parts : nullptr,
                                    parts_bytes, s);
  }
  // up to M = 320 (AWQ: 128) where the ring fits: ring launches of up to 64 (AWQ: 32)
  // activation rows each (8B gate, 32-row launches: 27 us at M = 48 and about 58 us at 128, against
  // 45 / 71 us for the tiled kernel); a row's result does not depend on the rows
  // launched with it
  const int rr = ring_rows(awq != nullptr);
  if (M > rr && M <= ring_chunked_max(awq != nullptr) && ring_fits(rr, N, K, awq != nullptr)) {
    const size_t osz = out_dt == NVE_DT_F32 ? 4 : 2;
    for (int m0 = 0; m0 < M; m0 += rr) {
      const int mc = M - m0 < rr ? M - m0 : rr;
      const void* xc = (const char*)x + (size_t)m0 * K * 2;
      void* oc = (char*)out + (size_t)m0 * N * osz;
      hipError_t e;
      if (awq) e = bf ? launch_small<true, true>(xc, mc, nib, sc, awq, oc, out_dt, N, K, s)
                      : launch_small<false, true>(xc, mc, nib, sc, awq, oc, out_dt, N, K, s);
      else e = bf ? launch_small<true, false>(xc, mc, nib, sc, awq, oc, out_dt, N, K, s)
                  : launch_small<false, false>(xc, mc, nib, sc, awq, oc, out_dt, N, K, s);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  if (M <= kGemmSmallM || ring_fits(M, N, K, awq != nullptr)) {
    if (awq) return bf ? launch_small<true, true>(x, M, nib, sc, awq, out, out_dt, N, K, s)
                       : launch_small<false, true>(x, M, nib, sc, awq, out, out_dt, N, K, s);
    return bf ? launch_small<true, false>(x, M, nib, sc, awq, out, out_dt, N, K, s)
              : launch_small<false, false>(x, M, nib, sc, awq, out, out_dt, N, K, s);
  }
#define NVE_GT(B, A) launch_gemm_t<B, A>(x, M, nib, sc, awq, out, out_dt, N, K, parts, parts_bytes, s)
  if (awq) return bf ? NVE_GT(true, true) : NVE_GT(false, true);
  return bf ? NVE_GT(true, false) : NVE_GT(false, false);
#undef NVE_GT
}

hipError_t launch_gemm_w4a16(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc, const float* awq,
                             void* out, int out_dt, int N, int K, hipStream_t s) {
  return launch_gemm_w4a16_parts(x, x_dt, M, nib, sc, awq, out, out_dt, N, K, nullptr, 0, s);
}

}  // namespace nve_host
