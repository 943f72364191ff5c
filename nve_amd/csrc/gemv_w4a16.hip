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

#include "act_producer.h"
#include "w4a16_ops.h"

namespace nve {

// SRC != SRC_PLAIN (MODE_F16 only): the activations are computed in the staging from
// the producer's inputs (act_producer.h) and rounded to fp16, the activation type of the
// reference's decode path (its W4A16 kernel takes fp16 x, src/cuda_kernels.rs:117-126).
// PAIR (act_producer.h): PAIR_SWIGLU -- segment 0 (gate) and the matrix in nib[1] /
// sc[1] (up) share N; a wave computes R/2 rows of each and writes silu(gate) * up
// (src/ops.rs:62-64).  PAIR_ROPE -- segments q, k, v, each N = rows / 2 pairs; a wave
// computes both rows of R/2 RoPE pairs and writes the attention's input (rope_store).
template <int MODE, int XDT, int OUT_DT, int R, int NJ, bool MULTI, int SRC = SRC_PLAIN, int PAIR = PAIR_NONE>
__global__ __launch_bounds__(256) void w4a16_gemv_kernel(const void* __restrict__ x, W4Segs segs,
                                                         int K, ProdArgs pa, EpiArgs ra) {
  constexpr bool SWI = PAIR == PAIR_SWIGLU, ROPE = PAIR == PAIR_ROPE;
  static_assert(SRC == SRC_PLAIN || (!MULTI && MODE == MODE_F16), "fused producers: one-pass fp16 staging");
  static_assert(PAIR == PAIR_NONE || (R % 2 == 0 && !MULTI && MODE != MODE_F32), "paired rows: even R, one pass");
  constexpr int RH = PAIR != PAIR_NONE ? R / 2 : R;  // output rows (pairs) per wave
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
  const int row0 = ((wg - wg0) * 4 + wave) * RH;
  const uint4* __restrict__ x4 = (const uint4*)x;

  // (1) activation staging loads (clamped index, unconditional)
  uint4 stv[SRC == SRC_PLAIN ? SPT : 1];
  float4 sta0[MODE == MODE_F32 ? SPT : 1], sta1[MODE == MODE_F32 ? SPT : 1];
  ProdChunk<SRC, 8> pc[SRC == SRC_PLAIN ? 1 : SPT];
  if constexpr (SRC != SRC_PLAIN) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) prod_issue<SRC, 8>(pc[s], pa, (int)threadIdx.x + 256 * s, nchunk);
  } else if (!MULTI) {
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
  // Residual add (F32_ACCUM): the output rows' current values are fetched with the
  // staging loads rather than by a dependent load in the epilogue (one writer per row).
  constexpr bool ACC = OUT_DT == NVE_DT_F32_ACCUM;
  float prev[ACC ? RH : 1];
  if constexpr (ACC) {
#pragma unroll
    for (int r = 0; r < RH; ++r) prev[r] = ((const float*)out)[min(row0 + r, N - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);

  // (2) weight loads
  uint4 wv[R][NJ];
  float wsc[R][NJ];
  const size_t row_bytes = (size_t)(K >> 1);
  auto issue = [&](int jb, int e0 = 0, int e1 = R * NJ) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = min(row0 + (PAIR != PAIR_NONE ? r % RH : r), N - 1);
      const int row = ROPE ? rope_row(rr, ra.half, r >= RH) : rr;
      const uint8_t* mn = (SWI && r >= RH) ? segs.nib[1] : nib;
      const float* ms = (SWI && r >= RH) ? segs.sc[1] : ws;
      const uint4* rn = (const uint4*)(mn + (size_t)row * row_bytes);
      const float* rs = ms + (size_t)row * nb;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (r * NJ + j < e0 || r * NJ + j >= e1) continue;
        const int bb = min(jb + lane + 64 * j, nb - 1);
        wv[r][j] = ld_stream(rn + bb);
        wsc[r][j] = ld_stream(rs + bb);
      }
    }
  };
  // SRC_NORM / SRC_F32: weight loads issued once the norm statistic is known / the vector
  // is staged (see gemv_w4a8.hip)
  constexpr bool kLateWeights = SRC == SRC_NORM || SRC == SRC_F32;
  // A late-issue launch still sends the first two of each lane's weight loads ((row,
  // chunk) order; at most half of them) with its staging loads: the 3B decode step runs
  // at 1196 against 1182 tok/s (512 cached keys; 893 against 885 at 7000); one or three
  // early loads in the Q/K/V launch, one or four in gate/up, one or three in down
  // measured equal or slower.
  constexpr int kEarly = kLateWeights ? (R * NJ / 2 < 2 ? R * NJ / 2 : 2) : R * NJ;
  if (kEarly > 0) issue(0, 0, kEarly);
  // A late issue is fenced on both sides so that the loads leave as one group at that
  // point: left to itself the scheduler spreads them through the quantization and hoists
  // the unpacking of the first ones above the LDS stores, which then wait for HBM before
  // the rest are even issued.
  auto issue_pinned = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    issue(0, kEarly);
    __builtin_amdgcn_sched_barrier(0);
  };
  // RoPE rows of this wave's pairs (used by lane 63 in the epilogue)
  int rpos = 0;
  float rc[ROPE ? RH : 1], rs[ROPE ? RH : 1];
  if constexpr (ROPE) {
    rpos = rope_pos(ra);
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const int d = min(row0 + r, N - 1) % ra.half;
      rc[r] = ra.cos[(size_t)rpos * ra.half + d];
      rs[r] = ra.sin[(size_t)rpos * ra.half + d];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // (3) LDS writes
  if constexpr (SRC != SRC_PLAIN) {
    double inv = 0.0;
    if (SRC == SRC_NORM)
      inv = prod_norm_inv(prod_sumsq<SRC, 8, SPT>(pc, nchunk), K, pa.eps,
                          (double*)((char*)lds + w4a16_lds_bytes(MODE, K)));
    if (kLateWeights && SRC == SRC_NORM) issue_pinned();
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = (int)threadIdx.x + 256 * s;
      float v[8];
      prod_values<SRC, 8>(pc[s], inv, v);
      w4a16_stage_put_dot<MODE>(prod_f16x8(v), i, i < nchunk, nb, s_p, s_mul);
    }
    if (kLateWeights && SRC != SRC_NORM) issue_pinned();
  } else if (!MULTI) {
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
  // the weight arithmetic stays below the staging barrier
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();

  // (4) arithmetic
  uint32_t magic;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
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
                                         : w4a16_block_dot_h(wv[r][j], (const int4*)s_p, ps, bb, magic);
        acc[r] = fmaf(s * mul, wsc[r][j], acc[r]);
      }
    }
    if (!MULTI) break;
    jb += 64 * NJ;
    if (jb >= nb) break;
    issue(jb);
  }

  if constexpr (SWI) {
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const float g = wave_sum_to_lane63(acc[r]);
      const float u = wave_sum_to_lane63(acc[r + RH]);
      if (lane == 63 && row0 + r < N) store_out<OUT_DT>(out, (size_t)(row0 + r), g / (1.0f + expf(-g)) * u);
    }
  } else if constexpr (ROPE) {
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const float x0 = wave_sum_to_lane63(acc[r]);
      const float x1 = wave_sum_to_lane63(acc[r + RH]);
      if (lane == 63 && row0 + r < N) rope_store(ra, sg, row0 + r, x0, x1, rc[r], rs[r], rpos);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum_to_lane63(acc[r]);
      if (lane == 63 && row0 + r < N) {
        if constexpr (ACC)
          ((float*)out)[row0 + r] = prev[r] + v;
        else
          store_out<OUT_DT>(out, (size_t)(row0 + r), v);
      }
    }
  }
}

}  // namespace nve

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace nve_host {

template <int MODE, int XDT, int OUT_DT, int R, int NJ, bool MULTI, int SRC = nve::SRC_PLAIN,
          int PAIR = nve::PAIR_NONE>
static hipError_t launch_w4a16_t(const void* x, const W4Segs& segs, int K, hipStream_t stream,
                                 const nve::ProdArgs& pa = nve::ProdArgs{}, const nve::EpiArgs& ra = nve::EpiArgs{}) {
  const size_t lds = nve::w4a16_lds_bytes(MODE, K) + (SRC == nve::SRC_NORM ? 64 : 0);
  auto kern = nve::w4a16_gemv_kernel<MODE, XDT, OUT_DT, R, NJ, MULTI, SRC, PAIR>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(segs.wg_total), dim3(256), lds, stream, x, segs, K, pa, ra);
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

template <int OUT_DT, int SRC, int PAIR>
static hipError_t launch_w4a16_fused_t(const nve::ProdArgs& pa, W4Segs segs, int K, hipStream_t stream,
                                       const nve::EpiArgs& ra) {
  const W4Tiling t = nve::attn_splits_of(SRC) ? choose_merge_tiling(segs, K) : choose_w4_tiling(segs, K);
  if (t.multi) return hipErrorInvalidValue;
  if (PAIR != nve::PAIR_NONE) {
    const int R = t.R < 2 ? 2 : t.R;
    if (PAIR == nve::PAIR_SWIGLU) segs.nseg = 1;  // gate in slot 0, up in slot 1 (read by the kernel directly)
    if (PAIR == nve::PAIR_ROPE)
      for (int i = 0; i < segs.nseg; ++i) segs.n[i] /= 2;  // RoPE pairs per matrix
    finalize_segments(segs, R / 2);
#define NVE_W4A16_PAIR_CASE(RR, JJ) \
    if (R == RR && t.NJ == JJ) \
      return launch_w4a16_t<nve::MODE_F16, NVE_DT_F16, OUT_DT, RR, JJ, false, SRC, PAIR>(nullptr, segs, K, stream, pa, ra);
    NVE_W4_SWIGLU_CASES(NVE_W4A16_PAIR_CASE)
#undef NVE_W4A16_PAIR_CASE
    return hipErrorInvalidValue;
  }
  finalize_segments(segs, t.R);
#define NVE_W4A16_CASE(RR, JJ, MM) \
  if (t.R == RR && t.NJ == JJ && !MM) \
    return launch_w4a16_t<nve::MODE_F16, NVE_DT_F16, OUT_DT, RR, JJ, false, SRC>(nullptr, segs, K, stream, pa);
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
  bool has_awq = false;
  for (int i = 0; i < segs.nseg; ++i) has_awq |= segs.awq[i] != nullptr;
  if (!has_awq && use_persistent(segs, K, true)) return launch_w4a16_persistent(x, x_dt, segs, out_dt, K, stream);
  switch (out_dt) {
    case NVE_DT_F16: return launch_w4a16_o<NVE_DT_F16>(x, x_dt, segs, K, stream);
    case NVE_DT_BF16: return launch_w4a16_o<NVE_DT_BF16>(x, x_dt, segs, K, stream);
    case NVE_DT_F32_ACCUM: return launch_w4a16_o<NVE_DT_F32_ACCUM>(x, x_dt, segs, K, stream);
    default: return launch_w4a16_o<NVE_DT_F32>(x, x_dt, segs, K, stream);
  }
}

// Decode-layer W4A16 GEMVs with a fused producer (act_producer.h), fp16 staging:
//   NORM, F32, rope    Q/K/V from the residual and the norm weights, RoPE + KV append
//                      in the epilogue (PAIR_ROPE);
//   NORM, F32          Q/K/V from the residual and the norm weights;
//   NORM, F16, swiglu  gate/up -> silu(gate) * up rounded to fp16 (the down input);
//   ATTN2/4, F32_ACCUM o_proj from the key-split attention partials.
hipError_t launch_w4a16_fused(int src, int pair, const nve::ProdArgs& pa, const W4Segs& segs, int out_dt, int K,
                              hipStream_t stream, const nve::EpiArgs& ra) {
  if (src == nve::SRC_NORM && out_dt == NVE_DT_F32 && pair == nve::PAIR_ROPE)
    return launch_w4a16_fused_t<NVE_DT_F32, nve::SRC_NORM, nve::PAIR_ROPE>(pa, segs, K, stream, ra);
  if (src == nve::SRC_NORM && out_dt == NVE_DT_F32 && pair == nve::PAIR_NONE)
    return launch_w4a16_fused_t<NVE_DT_F32, nve::SRC_NORM, nve::PAIR_NONE>(pa, segs, K, stream, ra);
  if (src == nve::SRC_NORM && out_dt == NVE_DT_F16 && pair == nve::PAIR_SWIGLU)
    return launch_w4a16_fused_t<NVE_DT_F16, nve::SRC_NORM, nve::PAIR_SWIGLU>(pa, segs, K, stream, ra);
  if (pair != nve::PAIR_NONE || out_dt != NVE_DT_F32_ACCUM) return hipErrorInvalidValue;
  if (src == nve::SRC_ATTN2) return launch_w4a16_fused_t<NVE_DT_F32_ACCUM, nve::SRC_ATTN2, nve::PAIR_NONE>(pa, segs, K, stream, ra);
  if (src == nve::SRC_ATTN4) return launch_w4a16_fused_t<NVE_DT_F32_ACCUM, nve::SRC_ATTN4, nve::PAIR_NONE>(pa, segs, K, stream, ra);
  if (src == nve::SRC_ATTN8) return launch_w4a16_fused_t<NVE_DT_F32_ACCUM, nve::SRC_ATTN8, nve::PAIR_NONE>(pa, segs, K, stream, ra);
  return hipErrorInvalidValue;
}

}  // namespace nve_host
