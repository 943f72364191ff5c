// gemm_w4a16_tile.hip -- large-M W4A16 prefill GEMM for gfx950: Y[M, N] = X[M, K] W[N, K]^T
// with int4 weights in the reference GPU layout and fp16 / bf16 activations, fp32
// accumulation.  Same product as the reference's prefill path (GpuWeight::matmul_x,
// src/gpu_layer.rs:219-237: nve_dequant_w4a16, cuda/nve_kernels.cu:397-433, then a dense
// GEMM), with every weight dequantized exactly as that dequant rounds it
// (f32 fma(n, s, -8 s) = (n - 8) s [times awq[k] in f32], then RNE to the activation type)
// but only in registers.
//
// Tile: 256 x 128 outputs per workgroup of 4 waves (2 x 2), 128 x 64 per wave as 4 x 2
// tiles of v_mfma_f32_32x32x16, or 128 x 128 outputs as 4 waves (1 x 4) of 128 x 32 (4 x 1
// tiles: each wave dequantizes only its own columns, and a given M has twice the
// workgroups; the host takes it while that grid is one round); K advances 64 per slice
// (two Q4 blocks), two slices per barrier (the barrier and each slice's first LDS reads
// cost about 450 cycles of a 2,700-cycle slice).
//   * Activation slices: global -> LDS transfers (buffer_load ... lds) one iteration ahead
//     into two slots of two slices; the A operands are read from LDS (ds_read_b128).
//   * Weights: the raw blocks (16 B of nibbles and the f32 scale per block row) go to a
//     three-slot LDS ring two iterations ahead; each wave reads the 8-byte nibble runs of its
//     64 rows once per slice and forms its B operands in registers (v_cvt_f32_ubyte, fma,
//     v_cvt_pk), spread between its MFMAs.  With 256-row tiles the two waves sharing a
//     column block both dequantize it; that VALU work runs beside the matrix pipe, while an LDS copy of the
//     dequantized weights would cost more LDS bandwidth than the MFMAs leave (measured:
//     one ds_read_b128 per 32x32x16 MFMA already stretches it from 33 to 47 cycles).
//   * One barrier per two slices.
// LDS rows of the activation ring are 128 B (8 chunks of 8 values); chunk c of row r sits
// at chunk position c ^ ((r >> 1) & 7), so the 16 lanes of each ds_read_b128 phase
// (rows r .. r + 15 of one chunk) cover all 64 banks.  LDS reads are inline asm with
// explicit waits: the compiler cannot tell the ring slots apart and would drain every
// transfer in flight before each access.
// Workgroup ids are mapped so that each XCD (workgroups are dealt to the 8 XCDs
// round-robin) runs consecutive tiles of one activation row block: its 2 MiB X slice
// column stays in that XCD's L2 while the weight tiles stream through.
#include "common.h"
#include "lds_ring.h"
#include "w4_launch.h"

namespace nve {

// BM = 256 or 128 activation rows per tile; each wave owns 128 of them and BN / (4 / (BM /
// 128)) columns: BM = 256 as 2 x 2 waves of 128 x 64, BM = 128 as 1 x 4 waves of 128 x 32
constexpr int TL_BN = 128, TL_BK = 64;
__host__ __device__ constexpr int tl_x_bytes(int bm) { return bm * TL_BK * 2; }  // one 64-wide slice
// raw weights of one slice: 256 blocks x (16 B nibbles, 4 B scale) = 5 KiB, and with AWQ the
// slice's 64 factors (256 B) after them
__host__ __device__ constexpr int tl_r_bytes(bool awq) { return TL_BN * 2 * 20 + (awq ? 256 : 0); }
// An iteration (one barrier) covers two slices: two activation slots of two slices each,
// three raw weight slots of two slices each (BM = 256: 158 KiB, 159.5 with AWQ; 128: 94 KiB)
__host__ __device__ constexpr int tl_r0(int bm) { return 2 * 2 * tl_x_bytes(bm); }
__host__ __device__ constexpr int tl_lds_bytes(int bm, bool awq) { return tl_r0(bm) + 3 * 2 * tl_r_bytes(awq); }

typedef _Float16 tl_h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 tl_b8_t __attribute__((ext_vector_type(8)));
typedef float tl_f16x_t __attribute__((ext_vector_type(16)));
typedef float tl_f2_t __attribute__((ext_vector_type(2)));
typedef _Float16 tl_h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 tl_b2_t __attribute__((ext_vector_type(2)));
typedef unsigned int tl_u2_t __attribute__((ext_vector_type(2)));

template <bool BF16>
__device__ __forceinline__ tl_f16x_t tl_mfma(u32x4_t a, u32x4_t b, tl_f16x_t c) {
  if (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(tl_b8_t, a), __builtin_bit_cast(tl_b8_t, b), c,
                                                   0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(tl_h8_t, a), __builtin_bit_cast(tl_h8_t, b), c, 0,
                                                0, 0);
}

template <int OFF>
__device__ __forceinline__ u32x4_t tl_ds_read128(uint32_t a) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int OFF>
__device__ __forceinline__ tl_u2_t tl_ds_read64(uint32_t a) {
  tl_u2_t v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t tl_ds_read32(uint32_t a) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

template <bool BF16>
__device__ __forceinline__ uint32_t tl_pack2(float a, float b) {
  // each value is an f32 first (the fma's rounding), then one v_cvt_pk_{f16,bf16}_f32
  // (round to nearest even): the reference dequant's two roundings
  asm("" : "+v"(a), "+v"(b));
  if (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){a, b}, tl_b2_t));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((tl_f2_t){a, b}, tl_h2_t));
}
// The reference dequant of 8 nibbles -- one per byte of lo (values 0..3) and hi (values
// 4..7), already masked -- [times the AWQ factors a0 (values 0..3) and a1 (4..7), each an
// f32 product of the f32 dequantized value as the reference forms it,] rounded to the
// activation type and packed in k order.
template <bool BF16, bool AWQ>
__device__ __forceinline__ u32x4_t tl_dequant8(uint32_t lo, uint32_t hi, float s, float s8, const u32x4_t& a0,
                                               const u32x4_t& a1) {
  // the masked dwords are opaque to the compiler, so each byte goes through one
  // v_cvt_f32_ubyte{0..3} (instead of a bit-field extract and a conversion)
  asm("" : "+v"(lo), "+v"(hi));
  float v[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    v[t] = fmaf((float)((lo >> (8 * t)) & 0xffu), s, s8);
    v[4 + t] = fmaf((float)((hi >> (8 * t)) & 0xffu), s, s8);
  }
  if constexpr (AWQ) {
    const uint32_t f[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= __builtin_bit_cast(float, f[e]);
  }
  u32x4_t r;
  r.x = tl_pack2<BF16>(v[0], v[1]);
  r.y = tl_pack2<BF16>(v[2], v[3]);
  r.z = tl_pack2<BF16>(v[4], v[5]);
  r.w = tl_pack2<BF16>(v[6], v[7]);
  return r;
}

// SPLIT: blockIdx.y = z takes slices z ks .. z ks + ks - 1 of K (ks even) and stores its
// fp32 partial tile to out + z M N (tl_reduce_kernel adds the partials in order).
// AWQ: the weights are multiplied by awq[k] after the dequant, as the reference does.
template <bool BF16, bool AWQ, int OUT_DT, int BM, bool SPLIT>
__global__ __launch_bounds__(256, 1) void gemm_w4a16_tile_kernel(const uint16_t* __restrict__ x,
                                                                 const uint8_t* __restrict__ nib,
                                                                 const float* __restrict__ sc,
                                                                 const float* __restrict__ awq, void* __restrict__ out,
                                                                 int M, int N, int K, int n_tiles, int ks) {
  static_assert(!SPLIT || OUT_DT == NVE_DT_F32, "split partials are fp32");
  extern __shared__ __align__(16) char tl_lds[];
  static_assert(BM == 256 || BM == 128, "row tile");
  constexpr int WM = BM / 128;    // waves along M (each 128 rows)
  constexpr int TJ = WM;          // 32-column MFMA tiles per wave: BN / (4 / WM) / 32
  constexpr int NX = BM / 32;     // activation transfers (1 KiB) per wave and slice
  constexpr int TL_X = tl_x_bytes(BM), TL_R0 = tl_r0(BM), TL_R = tl_r_bytes(AWQ);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / (4 / WM), wn = wave % (4 / WM);

  // XCD-grouped tile order: block b runs on XCD b % 8; the blocks of one XCD take
  // consecutive linear tiles (row block major)
  const int total = gridDim.x, b = blockIdx.x, xcd = b & 7;
  const int per = total >> 3, extra = total & 7;
  const int lin = xcd * per + min(xcd, extra) + (b >> 3);
  const int m0 = (lin / n_tiles) * BM, n0 = (lin % n_tiles) * TL_BN;
  // this workgroup's slices: t0 .. t0 + T - 1
  const int t0 = SPLIT ? (int)blockIdx.y * ks : 0;
  const int T = SPLIT ? min(K / TL_BK - t0, ks) : K / TL_BK;
  const uint32_t lds0 = lds_addr(tl_lds);

  // buffer resources (raw buffers, 32-bit offsets: the host routes M K >= 2^30
  // elsewhere): transfers take the per-lane offset in a VGPR, the slice offset in an SGPR
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc((void*)nib, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)sc, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t ar =
      __builtin_amdgcn_make_buffer_rsrc((void*)(AWQ ? awq : sc), (short)0, 0x7fffffff, 0x00020000);
  // activation transfers: instruction i of wave w fills tile rows (BM / 4) w + 8 i .. + 7
  // (1 KiB); lane l writes row (BM / 4) w + 8 i + l / 8 at chunk position l % 8, i.e. global
  // chunk (l % 8) ^ ((row >> 1) & 7)
  uint32_t xoff[8];
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const int r = (BM / 4) * wave + 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    xoff[i] = ((uint32_t)min(m0 + r, M - 1) * (uint32_t)K + 8u * c) * 2u;
  }
  // raw weights of a slice: block q = tid (tile row q / 2, block q % 2 of the slice): its
  // 16 B of nibbles go to R + 16 q, its scale to R + 4096 + 4 q
  const int rrow = min(n0 + (tid >> 1), N - 1);
  const uint32_t noff = (uint32_t)rrow * (uint32_t)(K / 2) + 16u * (tid & 1);
  const uint32_t soff = ((uint32_t)rrow * (uint32_t)(K / 32) + (tid & 1)) * 4u;

  // A fragments: rows 128 wm + 32 i + l % 32 (tile i at +4096 i); chunk position of step
  // kk: (2 kk + l / 32) ^ (((l % 32) >> 1) & 7)
  const int fr = lane & 31, fsw = (fr >> 1) & 7, fhi = lane >> 5;
  const uint32_t arow = (128 * wm + fr) * 128;
  uint32_t koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = ((2 * kk + fhi) ^ fsw) * 16;
  // B operands: lane l of step kk takes row 32 (TJ wn + j) + l % 32, values 16 kk + 8 (l / 32)
  // .. + 7 of the slice = block kk / 2, nibble bytes 8 (l / 32) .. + 7, low nibbles for even
  // kk and high for odd: one 8-byte read per (j, block) serves two steps
  const uint32_t bq = (uint32_t)(2 * (32 * TJ * wn + fr)) * 16 + 8 * fhi;  // + j * 1024 + block * 16
  const uint32_t bs = 4096 + (uint32_t)(2 * (32 * TJ * wn + fr)) * 4;      // + j * 256 + block * 4

  tl_f16x_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = tl_f16x_t{};

  // transfers of slice t (clamped to the last slice: the ones past the end re-read it,
  // which keeps every iteration's transfer count equal)
  auto issue_raw = [&](int t, int rslot) {
    const int tc = t0 + min(t, T - 1);
    char* const rb = tl_lds + TL_R0 + (2 * rslot + (t & 1)) * TL_R;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(nr, (lds_void_t*)(rb + wave * 1024), 16, noff, tc * 32, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void_t*)(rb + 4096 + wave * 256), 4, soff, tc * 8, 0, 0);
    // the slice's 64 AWQ factors, one per lane of wave 0 (the others' transfer counts are
    // unchanged; wave 0 waits for two more per iteration)
    if (AWQ && wave == 0)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void_t*)(rb + 5120), 4, 4u * lane, tc * 256, 0, 0);
  };
  // activation transfers i0 .. i1 - 1 of slice t
  auto issue_x_part = [&](int t, int xslot, int i0, int i1) {
    const int ko = (t0 + min(t, T - 1)) * (TL_BK * 2);
    char* const base = tl_lds + (2 * xslot + (t & 1)) * TL_X + wave * (BM / 4) * 128;
#pragma unroll
    for (int i = i0; i < i1; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void_t*)(base + i * 1024), 16, xoff[i], ko, 0, 0);
  };
  auto issue_x = [&](int t, int xslot) { issue_x_part(t, xslot, 0, NX); };  // slice t into its half of xslot
  auto rd_a = [&](uint32_t xa, int kk, u32x4_t (&fa)[4]) {
    const uint32_t a = xa + arow + koff[kk];
    fa[0] = tl_ds_read128<0>(a);
    fa[1] = tl_ds_read128<4096>(a);
    fa[2] = tl_ds_read128<8192>(a);
    fa[3] = tl_ds_read128<12288>(a);
  };
  // B operand of step kk for one column tile from its raw run q (block kk / 2)
  auto b_operand = [&](const tl_u2_t& q, float s, int kk, const u32x4_t& a0, const u32x4_t& a1) {
    const uint32_t lo = (kk & 1) ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
    const uint32_t hi = (kk & 1) ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
    return tl_dequant8<BF16, AWQ>(lo, hi, s, -8.0f * s, a0, a1);
  };
  // AWQ factors of the lane's 8 values of step kk: slice values 16 kk + 8 (l / 32) .. + 7
  const uint32_t aoff = 5120 + 32 * fhi;  // + 64 kk
  // the MFMAs of one slice (activations at LDS xa, raw weights at rb): A fragments of step
  // kk + 1 are read and B operands of step kk + 1 formed while step kk multiplies (each
  // MFMA followed by VALU work); iss(kk) issues transfers of later slices beside the
  // MFMAs of step kk: issued back to back after the barrier, the four waves' transfers
  // held the address pipeline for about 500 cycles with no matrix work in flight
  auto mma = [&](uint32_t xa, uint32_t rb, auto&& iss) {
    tl_u2_t q[2][2];  // [j][block]
    uint32_t sbits[2][2];
    u32x4_t fa[4];
    u32x4_t aw[4][2] = {};  // AWQ factors of steps 0..3 (unused without AWQ)
    if constexpr (AWQ) {
      aw[0][0] = tl_ds_read128<0>(rb + aoff);
      aw[0][1] = tl_ds_read128<16>(rb + aoff);
      aw[1][0] = tl_ds_read128<64>(rb + aoff);
      aw[1][1] = tl_ds_read128<80>(rb + aoff);
      aw[2][0] = tl_ds_read128<128>(rb + aoff);
      aw[2][1] = tl_ds_read128<144>(rb + aoff);
      aw[3][0] = tl_ds_read128<192>(rb + aoff);
      aw[3][1] = tl_ds_read128<208>(rb + aoff);
    }
    q[0][0] = tl_ds_read64<0>(rb + bq);
    q[0][1] = tl_ds_read64<16>(rb + bq);
    sbits[0][0] = tl_ds_read32<0>(rb + bs);
    sbits[0][1] = tl_ds_read32<4>(rb + bs);
    if (TJ == 2) {
      q[1][0] = tl_ds_read64<1024>(rb + bq);
      q[1][1] = tl_ds_read64<1040>(rb + bq);
      sbits[1][0] = tl_ds_read32<256>(rb + bs);
      sbits[1][1] = tl_ds_read32<260>(rb + bs);
    }
    rd_a(xa, 0, fa);
    lgkm_wait();
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        tie(q[j][h]);
        tie(sbits[j][h]);
      }
    if constexpr (AWQ) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        tie(aw[kk][0]);
        tie(aw[kk][1]);
      }
    }
    float s[2][2];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) s[j][h] = __builtin_bit_cast(float, sbits[j][h]);
    u32x4_t fb[2];
#pragma unroll
    for (int j = 0; j < TJ; ++j) fb[j] = b_operand(q[j][0], s[j][0], 0, aw[0][0], aw[0][1]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk > 0) lgkm_wait();
#pragma unroll
      for (int i = 0; i < 4; ++i) tie(fa[i]);
      u32x4_t ca[4], cb[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) ca[i] = fa[i];
#pragma unroll
      for (int j = 0; j < TJ; ++j) cb[j] = fb[j];
      if (kk < 3) rd_a(xa, kk + 1, fa);
      iss(kk);
      // one scheduling region: the 8 MFMAs of step kk with the next step's B operands
      // formed between them
      if (kk < 3) {
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          fb[j] = b_operand(q[j][(kk + 1) >> 1], s[j][(kk + 1) >> 1], kk + 1, aw[kk + 1][0], aw[kk + 1][1]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = tl_mfma<BF16>(ca[i], cb[j], acc[i][j]);
      if (kk < 3) {
#pragma unroll
        for (int m = 0; m < 4 * TJ; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
      }
    }
  };

  // Pipeline: iteration u (one barrier) multiplies slices 2u and 2u + 1 (activation slot
  // u % 2, raw weight slot u % 3); beside the MFMAs of slice 2u it issues the activation
  // transfers of slices 2u + 2 and 2u + 3 (16 per thread, into the slot iteration u - 1
  // read), beside those of slice 2u + 1 the raw weight transfers of slices 2u + 4 and
  // 2u + 5 (4 per thread, into the slot iteration u - 1 read).  At the top of iteration u
  // this thread's activation transfers for it and raw transfers (issued an iteration
  // earlier still) are all but the last 4 (the raw transfers of iteration u - 1); the
  // barrier then makes every thread's transfers visible and every read of the slots about
  // to be refilled finished.  Prologue order raw 0-1, x 0-1, raw 2-3: the same at u = 0.
  issue_raw(0, 0);
  issue_raw(1, 0);
  issue_x(0, 0);
  issue_x(1, 0);
  issue_raw(2, 1);
  issue_raw(3, 1);

  int xs = 0, rs = 0;  // slots of iteration u's activations and raw weights
  for (int t = 0; t < T; t += 2) {
    const int rs2 = rs == 0 ? 2 : rs - 1;  // (u + 2) % 3 = (u - 1) % 3
    if (AWQ && wave == 0)
      wait_vmcnt<6>();
    else
      wait_vmcnt<4>();
    lgkm_wait();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t xa = lds0 + 2 * xs * TL_X, rb = lds0 + TL_R0 + 2 * rs * TL_R;
    mma(xa, rb, [&](int kk) {
      issue_x_part(t + 2 + (kk >> 1), xs ^ 1, (NX / 2) * (kk & 1), (NX / 2) * (kk & 1) + NX / 2);
    });
    mma(xa + TL_X, rb + TL_R, [&](int kk) {
      if (kk == 0) issue_raw(t + 4, rs2);
      if (kk == 1) issue_raw(t + 5, rs2);
    });
    xs ^= 1;
    rs = rs == 2 ? 0 : rs + 1;
  }
  // the transfers issued past the last slice (clamped re-reads) land before the
  // workgroup's LDS is released
  wait_vmcnt<0>();
  lgkm_wait();

  // 32 x 32 result layout: register r of lane l holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = n0 + 32 * (TJ * wn + j) + fr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + 128 * wm + 32 * i + 8 * (r >> 2) + 4 * fhi + (r & 3);
        if (m < M && n < N) {
          if constexpr (SPLIT)
            ((float*)out)[(size_t)blockIdx.y * M * N + (size_t)m * N + n] = acc[i][j][r];
          else
            store_out<OUT_DT>(out, (size_t)m * N + n, acc[i][j][r]);
        }
      }
    }
}

// out[i] = sum over z = 0 .. split - 1 of part[z n + i], in that order, rounded to OUT_DT
template <int OUT_DT>
__global__ __launch_bounds__(256) void tl_reduce_kernel(const float* __restrict__ part, void* __restrict__ out,
                                                        size_t n, int split) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float y = part[i];
  for (int z = 1; z < split; ++z) y += part[(size_t)z * n + i];
  store_out<OUT_DT>(out, i, y);
}

}  // namespace nve

namespace nve_host {

// The tile kernel serves K % 128 == 0 (two slices per iteration), where every byte offset
// fits its buffer resource (2^31 - 1 bytes; reads past it would return zeros): activations
// M K, nibbles N K / 2 and scales N K / 8 bytes (AWQ factors: 4 K).
long gemm_tile_grid128(int M, int N) {
  return (long)((M + 127) / 128) * ((N + nve::TL_BN - 1) / nve::TL_BN);
}

// K split of a 128-row tile grid that leaves CUs idle: as many splits as keep the grid
// within one round (256 workgroups) and at least 4 iterations (8 slices) each; *ks =
// slices per split (even), and the returned count has no empty split.
static int tile_split(int M, int N, int K, int* ks) {
  const long g = gemm_tile_grid128(M, N);
  const int kit = K / (2 * nve::TL_BK);
  const int by_grid = g >= 256 ? 1 : (int)(256 / g), by_k = kit / 4 > 1 ? kit / 4 : 1;
  const int split = by_grid < by_k ? by_grid : by_k;
  const int per = 2 * ((kit + split - 1) / split);
  if (ks) *ks = per;
  return (2 * kit + per - 1) / per;
}

size_t gemm_tile_parts_bytes(int M, int N, int K) {
  if (!gemm_tile_fits(M, N, K, false)) return 0;
  const int split = tile_split(M, N, K, nullptr);
  return split > 1 ? (size_t)split * M * N * sizeof(float) : 0;
}

bool gemm_tile_fits(int M, int N, int K, bool /*awq*/) {
  return K % 128 == 0 && M >= 1 && N >= 1 && (long)M * K < (1L << 30) && (long)N * (K / 2) < (1L << 31);
}

template <bool BF16, bool AWQ, int OUT_DT, int BM, bool SPLIT = false>
static hipError_t launch_tile_bm(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                 void* out, int N, int K, hipStream_t s, int split = 1, int ks = 0) {
  auto kern = nve::gemm_w4a16_tile_kernel<BF16, AWQ, OUT_DT, BM, SPLIT>;
  constexpr int lds = nve::tl_lds_bytes(BM, AWQ);
  static thread_local int attr_dev = -1;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (attr_dev != dev) {
    e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_dev = dev;
  }
  const int nt = (N + nve::TL_BN - 1) / nve::TL_BN, mt = (M + BM - 1) / BM;
  hipLaunchKernelGGL(kern, dim3(nt * mt, split), dim3(256), lds, s, (const uint16_t*)x, nib, sc, awq, out, M, N, K,
                     nt, ks);
  return hipGetLastError();
}

// 128-row tiles while their grid is one round (at most one workgroup per CU), else 256
// (8B gate, fp16 out, us: M = 256 51.4 against 71.2 with 256-row tiles; M = 512 103.3
// against 81.4, the 128-row grid there being 448 workgroups)
template <bool BF16, bool AWQ, int OUT_DT>
static hipError_t launch_tile_t(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                void* out, int N, int K, hipStream_t s) {
  if (gemm_tile_grid128(M, N) <= 256)
    return launch_tile_bm<BF16, AWQ, OUT_DT, 128>(x, M, nib, sc, awq, out, N, K, s);
  return launch_tile_bm<BF16, AWQ, OUT_DT, 256>(x, M, nib, sc, awq, out, N, K, s);
}

// With parts (parts_bytes >= gemm_tile_parts_bytes) a small grid is split over K: fp32
// partials there, added in a fixed order and rounded to out_dt by a second launch.
template <bool BF16, bool AWQ>
static hipError_t launch_tile_split(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                   void* out, int out_dt, int N, int K, float* parts, int split, int ks,
                                   hipStream_t s) {
  hipError_t e = launch_tile_bm<BF16, AWQ, NVE_DT_F32, 128, true>(x, M, nib, sc, awq, parts, N, K, s, split, ks);
  if (e != hipSuccess) return e;
  const size_t n = (size_t)M * N;
  const dim3 g((unsigned)((n + 255) / 256));
  switch (out_dt) {
    case NVE_DT_F16: hipLaunchKernelGGL(nve::tl_reduce_kernel<NVE_DT_F16>, g, dim3(256), 0, s, parts, out, n, split); break;
    case NVE_DT_BF16: hipLaunchKernelGGL(nve::tl_reduce_kernel<NVE_DT_BF16>, g, dim3(256), 0, s, parts, out, n, split); break;
    default: hipLaunchKernelGGL(nve::tl_reduce_kernel<NVE_DT_F32>, g, dim3(256), 0, s, parts, out, n, split); break;
  }
  return hipGetLastError();
}

template <bool BF16, bool AWQ>
static hipError_t launch_tile_x(const void* x, int M, const uint8_t* nib, const float* sc, const float* awq,
                                void* out, int out_dt, int N, int K, float* parts, size_t parts_bytes,
                                hipStream_t s) {
  if (parts) {
    int ks = 0;
    const int split = tile_split(M, N, K, &ks);
    if (split > 1 && parts_bytes >= (size_t)split * M * N * sizeof(float))
      return launch_tile_split<BF16, AWQ>(x, M, nib, sc, awq, out, out_dt, N, K, parts, split, ks, s);
  }
  switch (out_dt) {
    case NVE_DT_F16: return launch_tile_t<BF16, AWQ, NVE_DT_F16>(x, M, nib, sc, awq, out, N, K, s);
    case NVE_DT_BF16: return launch_tile_t<BF16, AWQ, NVE_DT_BF16>(x, M, nib, sc, awq, out, N, K, s);
    default: return launch_tile_t<BF16, AWQ, NVE_DT_F32>(x, M, nib, sc, awq, out, N, K, s);
  }
}

hipError_t launch_gemm_w4a16_tile(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                  const float* awq, void* out, int out_dt, int N, int K, float* parts,
                                  size_t parts_bytes, hipStream_t s) {
  if (K % (2 * nve::TL_BK) != 0) return hipErrorInvalidValue;
  const bool bf = x_dt == NVE_DT_BF16;
  if (awq)
    return bf ? launch_tile_x<true, true>(x, M, nib, sc, awq, out, out_dt, N, K, parts, parts_bytes, s)
              : launch_tile_x<false, true>(x, M, nib, sc, awq, out, out_dt, N, K, parts, parts_bytes, s);
  return bf ? launch_tile_x<true, false>(x, M, nib, sc, awq, out, out_dt, N, K, parts, parts_bytes, s)
            : launch_tile_x<false, false>(x, M, nib, sc, awq, out, out_dt, N, K, parts, parts_bytes, s);
}

}  // namespace nve_host
