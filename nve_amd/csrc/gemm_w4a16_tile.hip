// gemm_w4a16_tile.hip -- large-M W4A16 prefill GEMM for gfx950: Y[M, N] = X[M, K] W[N, K]^T
// with int4 weights in the reference GPU layout and fp16 / bf16 activations, fp32
// accumulation.  Same product as the reference's prefill path (GpuWeight::matmul_x,
// src/gpu_layer.rs:219-237: nve_dequant_w4a16, cuda/nve_kernels.cu:397-433, then a dense
// GEMM), with every weight dequantized exactly as that dequant rounds it
// (f32 fma(n, s, -8 s) = (n - 8) s, then RNE to the activation type) but only into LDS.
//
// Tile: 256 x 128 outputs per workgroup of 4 waves (2 x 2), 128 x 64 per wave as 4 x 2
// tiles of v_mfma_f32_32x32x16 (8 MFMAs per 6 LDS fragment reads); K advances 64 per
// slice.  A three-slot LDS ring (48 KiB per slot: the 256 x 64 activation slice and the
// 128 x 64 dequantized weight slice, 144 KiB, one workgroup per CU):
//   * activation slices are global -> LDS transfers issued two slices ahead;
//   * raw weight blocks (16 B of nibbles + the f32 scale per thread) are loaded three
//     slices ahead into registers and dequantized into the next slice's slot while the
//     MFMAs of the current slice run;
//   * one barrier per slice.
// LDS rows are 128 B (8 chunks of 8 values); chunk c of row r sits at chunk position
// c ^ ((r >> 1) & 7), so the 16 lanes of each ds_read_b128 phase (rows r .. r + 15 of one
// chunk) cover all 64 banks.  LDS reads and the dequantized writes are inline asm with
// explicit waits: the compiler cannot tell the ring slots apart and would drain every
// transfer in flight before each access.
// Workgroup ids are mapped so that each XCD (workgroups are dealt to the 8 XCDs
// round-robin) runs consecutive tiles of one activation row block: its 2 MiB X slice
// column stays in that XCD's L2 while the weight tiles stream through.
#include "common.h"
#include "lds_ring.h"
#include "w4_launch.h"

namespace nve {

constexpr int TL_BM = 256, TL_BN = 128, TL_BK = 64;
// LDS: three activation slots, two dequantized weight slots, three raw weight slots
constexpr int TL_X = TL_BM * TL_BK * 2;   // 32 KiB: 256 rows x 64 values
constexpr int TL_D = TL_BN * TL_BK * 2;   // 16 KiB: 128 rows x 64 values
constexpr int TL_R = TL_BN * 2 * 20;      // 5 KiB: 256 blocks x (16 B nibbles, 4 B scale)
constexpr int TL_RS = 5;                  // raw weight slots: issued TL_RS slices ahead
constexpr int TL_D0 = 3 * TL_X, TL_R0 = TL_D0 + 2 * TL_D;
constexpr int TL_LDS = TL_R0 + TL_RS * TL_R;  // 153 KiB

typedef _Float16 tl_h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 tl_b8_t __attribute__((ext_vector_type(8)));
typedef float tl_f16x_t __attribute__((ext_vector_type(16)));

template <bool BF16>
__device__ __forceinline__ tl_f16x_t tl_mfma(u32x4_t a, u32x4_t b, tl_f16x_t c) {
  if (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(tl_b8_t, a), __builtin_bit_cast(tl_b8_t, b), c,
                                                   0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(tl_h8_t, a), __builtin_bit_cast(tl_h8_t, b), c, 0,
                                                0, 0);
}

__device__ __forceinline__ void tl_ds_write128(uint32_t a, u32x4_t v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v));
}
template <int OFF>
__device__ __forceinline__ u32x4_t tl_ds_read128(uint32_t a) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

// The reference dequant of 8 nibbles (bytes of lo / hi already masked to one nibble
// each), rounded to the activation type and packed in k order.
template <bool BF16>
__device__ __forceinline__ uint32_t tl_pack2(float a, float b) {
  if (BF16) return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
  return (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(a)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(b)) << 16);
}
typedef float tl_f2_t __attribute__((ext_vector_type(2)));
typedef _Float16 tl_h2_t __attribute__((ext_vector_type(2)));
template <bool BF16>
__device__ __forceinline__ u32x4_t tl_dequant8(uint32_t lo, uint32_t hi, float s, float s8) {
  // the masked dwords are opaque to the compiler, so each byte goes through one
  // v_cvt_f32_ubyte{0..3} (instead of a bit-field extract and a conversion)
  asm("" : "+v"(lo), "+v"(hi));
  float v[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    v[t] = fmaf((float)((lo >> (8 * t)) & 0xffu), s, s8);
    v[4 + t] = fmaf((float)((hi >> (8 * t)) & 0xffu), s, s8);
  }
  u32x4_t r;
  if constexpr (BF16) {
    r.x = tl_pack2<true>(v[0], v[1]);
    r.y = tl_pack2<true>(v[2], v[3]);
    r.z = tl_pack2<true>(v[4], v[5]);
    r.w = tl_pack2<true>(v[6], v[7]);
  } else {
    // each value is an f32 first (the fma's rounding), then one v_cvt_pk_f16_f32 per pair
    // (round to nearest even): the reference dequant's two roundings
#pragma unroll
    for (int t = 0; t < 8; ++t) asm("" : "+v"(v[t]));
    r.x = __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){v[0], v[1]}, tl_h2_t));
    r.y = __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){v[2], v[3]}, tl_h2_t));
    r.z = __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){v[4], v[5]}, tl_h2_t));
    r.w = __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){v[6], v[7]}, tl_h2_t));
  }
  return r;
}

template <bool BF16, int OUT_DT>
__global__ __launch_bounds__(256, 1) void gemm_w4a16_tile_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ nib,
                                                                 const float* __restrict__ sc, void* __restrict__ out,
                                                                 int M, int N, int K, int n_tiles) {
  extern __shared__ __align__(16) char tl_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-grouped tile order: block b runs on XCD b % 8; the blocks of one XCD take
  // consecutive linear tiles (row block major)
  const int total = gridDim.x, b = blockIdx.x, xcd = b & 7;
  const int per = total >> 3, extra = total & 7;
  const int lin = xcd * per + min(xcd, extra) + (b >> 3);
  const int m0 = (lin / n_tiles) * TL_BM, n0 = (lin % n_tiles) * TL_BN;
  const int T = K / TL_BK;
  const uint32_t lds0 = lds_addr(tl_lds);

  // activation transfers: instruction i of wave w fills tile rows 64 w + 8 i .. + 7 (1 KiB);
  // lane l writes row 64 w + 8 i + l / 8 at chunk position l % 8, i.e. global chunk
  // (l % 8) ^ ((row >> 1) & 7)
  // (byte offsets from x: the host routes M K >= 2^30 elsewhere)
  // buffer resources (raw buffers, 32-bit offsets): transfers take the per-lane offset in a
  // VGPR and the slice offset in an SGPR
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc((void*)nib, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)sc, (short)0, 0x7fffffff, 0x00020000);
  uint32_t xoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xoff[i] = ((uint32_t)min(m0 + r, M - 1) * (uint32_t)K + 8u * c) * 2u;
  }
  // this thread's weight block of each slice: tile row wr, block wb (of the slice's two);
  // its nibbles (16 B) and scale reach the raw slot by transfer at R + 16 tid and
  // R + 4096 + 4 tid, where the thread reads them back
  const int wr = tid >> 1, wb = tid & 1;
  const int wrow = min(n0 + wr, N - 1);
  const uint32_t noff = (uint32_t)wrow * (uint32_t)(K / 2) + 16u * wb;
  const uint32_t soff = ((uint32_t)wrow * (uint32_t)(K / 32) + wb) * 4u;
  const uint32_t wdst = wr * 128;  // + dequantized slot base + chunk position * 16
  const int wsw = (wr >> 1) & 7;

  // fragment offsets: A rows 128 wm + 32 i + l % 32 (tile i at +4096 i), B rows
  // 64 wn + 32 j + l % 32 (tile j at +4096 j); the chunk position of step kk depends on
  // l % 32 and l / 32 only
  const int fr = lane & 31, fsw = (fr >> 1) & 7, fhi = lane >> 5;
  const uint32_t arow = (128 * wm + fr) * 128, brow = (64 * wn + fr) * 128;
  uint32_t koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = ((2 * kk + fhi) ^ fsw) * 16;

  tl_f16x_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = tl_f16x_t{};

  // transfers of slice t (clamped to the last slice: the ones past the end re-read it,
  // which keeps every iteration's transfer count equal)
  auto issue_raw = [&](int t, int rslot) {
    const int tc = min(t, T - 1);
    char* const rb = tl_lds + TL_R0 + rslot * TL_R;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(nr, (lds_void_t*)(rb + wave * 1024), 16, noff, tc * 32, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void_t*)(rb + 4096 + wave * 256), 4, soff, tc * 8, 0, 0);
  };
  auto issue_x = [&](int t, int xslot) {
    const int ko = min(t, T - 1) * (TL_BK * 2);
    char* const base = tl_lds + xslot * TL_X + wave * 64 * 128;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t*)(base + i * 1024), 16, xoff[i], ko, 0, 0);
  };
  // this thread's raw block of raw slot rslot (read back from its own transfers)
  auto raw_read = [&](int rslot, u32x4_t& q, uint32_t& sbits) {
    const uint32_t rb = lds0 + TL_R0 + rslot * TL_R;
    q = ds_read128(rb + 16 * tid);
    asm volatile("ds_read_b32 %0, %1 offset:4096" : "=v"(sbits) : "v"(rb + 4 * tid));
  };
  // chunk cl (values 8 cl .. 8 cl + 7 of the block: low (cl < 2) or high nibbles of
  // bytes 8 (cl & 1) .. + 7) of the raw block, dequantized into dequantized slot dslot
  auto chunk_values = [&](int cl, const u32x4_t& q, float s, float s8) {
    const uint32_t a = (cl & 1) ? q.z : q.x, b2 = (cl & 1) ? q.w : q.y;
    const uint32_t lo = cl < 2 ? (a & 0x0F0F0F0Fu) : ((a >> 4) & 0x0F0F0F0Fu);
    const uint32_t hi = cl < 2 ? (b2 & 0x0F0F0F0Fu) : ((b2 >> 4) & 0x0F0F0F0Fu);
    return tl_dequant8<BF16>(lo, hi, s, s8);
  };
  auto chunk_addr = [&](int cl, int dslot) {
    return lds0 + TL_D0 + dslot * TL_D + wdst + (((4 * wb + cl) ^ wsw) * 16);
  };
  auto dequant_chunk = [&](int cl, const u32x4_t& q, float s, float s8, int dslot) {
    tl_ds_write128(chunk_addr(cl, dslot), chunk_values(cl, q, s, s8));
  };
  auto dequant = [&](int rslot, int dslot) {
    u32x4_t q;
    uint32_t sbits;
    raw_read(rslot, q, sbits);
    lgkm_wait();
    tie(q);
    tie(sbits);
    const float s = __builtin_bit_cast(float, sbits), s8 = -8.0f * s;
#pragma unroll
    for (int cl = 0; cl < 4; ++cl) dequant_chunk(cl, q, s, s8, dslot);
  };
  auto rd = [&](uint32_t xa, uint32_t da, int kk, u32x4_t (&fa)[4], u32x4_t (&fb)[2]) {
    const uint32_t a = xa + arow + koff[kk], b = da + brow + koff[kk];
    fa[0] = tl_ds_read128<0>(a);
    fa[1] = tl_ds_read128<4096>(a);
    fa[2] = tl_ds_read128<8192>(a);
    fa[3] = tl_ds_read128<12288>(a);
    fb[0] = tl_ds_read128<0>(b);
    fb[1] = tl_ds_read128<4096>(b);
  };
  // the MFMAs of one slice; fragments of step kk + 1 are read while step kk multiplies,
  // and chunk kk of the next slice's weight block is dequantized after the MFMAs of step
  // kk are issued (VALU work beside the matrix pipe)
  auto mma = [&](int xslot, int dslot, int rslot_next, int dslot_next) {
    const uint32_t xa = lds0 + xslot * TL_X, da = lds0 + TL_D0 + dslot * TL_D;
    u32x4_t fa[4], fb[2], q;
    uint32_t sbits;
    rd(xa, da, 0, fa, fb);
    raw_read(rslot_next, q, sbits);
    float s = 0.0f, s8 = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      lgkm_wait();
#pragma unroll
      for (int i = 0; i < 4; ++i) tie(fa[i]);
#pragma unroll
      for (int j = 0; j < 2; ++j) tie(fb[j]);
      if (kk == 0) {
        tie(q);
        tie(sbits);
        s = __builtin_bit_cast(float, sbits);
        s8 = -8.0f * s;
      }
      u32x4_t ca[4], cb[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) ca[i] = fa[i];
#pragma unroll
      for (int j = 0; j < 2; ++j) cb[j] = fb[j];
      if (kk < 3) rd(xa, da, kk + 1, fa, fb);
      // one scheduling region: the 8 MFMAs of the step with the chunk's dequantization
      // spread between them (each MFMA followed by three VALU instructions)
      const u32x4_t wv = chunk_values(kk, q, s, s8);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = tl_mfma<BF16>(ca[i], cb[j], acc[i][j]);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
      tl_ds_write128(chunk_addr(kk, dslot_next), wv);
    }
  };

  // Pipeline (one barrier per slice): iteration t multiplies slice t (activation slot
  // t % 3, dequantized slot t % 2), dequantizes the raw weights of slice t + 1 (raw slot
  // (t + 1) % TL_RS) and issues the transfers of raw weights t + TL_RS and activations
  // t + 2 (10 per thread: 2 + 8).  At the top of iteration t, this thread's transfers of
  // activations t and raw weights t + 1 are the ones older than the last 10.
  // prologue order raw 0 .. TL_RS - 2, x 0, raw TL_RS - 1, x 1: the top of iteration 0
  // needs x 0 and raw 1, older than the last 10 (raw TL_RS - 1, x 1) -- as in the steady
  // state, where iteration t issues raw t + TL_RS and x t + 2
#pragma unroll
  for (int u = 0; u < TL_RS - 1; ++u) issue_raw(u, u);
  issue_x(0, 0);
  issue_raw(TL_RS - 1, TL_RS - 1);
  issue_x(1, 1);
  wait_vmcnt<10 + 8>();  // raw 0 landed
  dequant(0, 0);

  int xs = 0, ds = 0, rs = 1;  // slots of activations t, dequantized t, raw t + 1
  for (int t = 0; t < T; ++t) {
    const int xs2 = xs == 0 ? 2 : xs - 1;          // (t + 2) % 3
    const int rs2 = rs == 0 ? TL_RS - 1 : rs - 1;  // (t + TL_RS) % TL_RS: the slot raw t left
    wait_vmcnt<10>();
    lgkm_wait();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue_raw(t + TL_RS, rs2);
    issue_x(t + 2, xs2);
    __builtin_amdgcn_sched_barrier(0);
    mma(xs, ds, rs, ds ^ 1);
    xs = xs == 2 ? 0 : xs + 1;
    rs = rs == TL_RS - 1 ? 0 : rs + 1;
    ds ^= 1;
  }
  // the transfers issued past the last slice (clamped re-reads) land before the
  // workgroup's LDS is released
  wait_vmcnt<0>();
  lgkm_wait();

  // 32 x 32 result layout: register r of lane l holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wn + 32 * j + fr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 128 * wm + 32 * i + 8 * (r >> 2) + 4 * fhi + (r & 3);
        if (m < M && n < N) store_out<OUT_DT>(out, (size_t)m * N + n, acc[i][j][r]);
      }
    }
}

}  // namespace nve

namespace nve_host {

// The tile kernel serves K % 64 == 0 without AWQ; anything else is the caller's to route.
bool gemm_tile_fits(int M, int N, int K, bool awq) {
  return !awq && K % 64 == 0 && M >= 1 && N >= 1 && (long)M * K < (1L << 30);
}

template <bool BF16, int OUT_DT>
static hipError_t launch_tile_t(const void* x, int M, const uint8_t* nib, const float* sc, void* out, int N, int K,
                                hipStream_t s) {
  auto kern = nve::gemm_w4a16_tile_kernel<BF16, OUT_DT>;
  static thread_local int attr_dev = -1;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (attr_dev != dev) {
    e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, nve::TL_LDS);
    if (e != hipSuccess) return e;
    attr_dev = dev;
  }
  const int nt = (N + nve::TL_BN - 1) / nve::TL_BN, mt = (M + nve::TL_BM - 1) / nve::TL_BM;
  hipLaunchKernelGGL(kern, dim3(nt * mt), dim3(256), nve::TL_LDS, s, (const uint16_t*)x, nib, sc, out, M, N, K, nt);
  return hipGetLastError();
}

hipError_t launch_gemm_w4a16_tile(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc, void* out,
                                  int out_dt, int N, int K, hipStream_t s) {
  if (K % nve::TL_BK != 0) return hipErrorInvalidValue;
  const bool bf = x_dt == NVE_DT_BF16;
#define NVE_TL(B)                                                                       \
  switch (out_dt) {                                                                     \
    case NVE_DT_F16: return launch_tile_t<B, NVE_DT_F16>(x, M, nib, sc, out, N, K, s);   \
    case NVE_DT_BF16: return launch_tile_t<B, NVE_DT_BF16>(x, M, nib, sc, out, N, K, s); \
    default: return launch_tile_t<B, NVE_DT_F32>(x, M, nib, sc, out, N, K, s);           \
  }
  if (bf) { NVE_TL(true) }
  NVE_TL(false)
#undef NVE_TL
}

}  // namespace nve_host
