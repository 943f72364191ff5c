// gemv_w4a8.hip -- W4A8 decode GEMV for gfx950 (int4 weights x int8 activations).
//
// Computes, per output row n (cuda/nve_kernels.cu:796-878 restated for CDNA4):
//   acc[n,b] = sum_{i<32} (nib_i - 8) * xq[32b + i]            exact int32
//   y[n]     = sum_b ws[n,b] * xs[b] * acc[n,b]                fp32
//
// MI355X design:
//   * Each wave owns R output rows.  Lane l of the wave handles the 32-weight blocks
//     b = l, l+64, l+128, ... of those rows, so every weight load instruction of the
//     wave is one contiguous 1 KiB (nibbles, global_load_dwordx4) or 256 B (scales,
//     global_load_dword) span of HBM: fully coalesced for any K.
//   * All R x NJ block loads of a wave are issued before any arithmetic (NJ = blocks
//     per lane), so each lane keeps R*NJ*20 bytes in flight; R is picked so that
//     R*NJ ~ 8 (160 B/lane, 10 KiB/wave).
//   * The activation vector is staged once per workgroup in LDS: xq split into two
//     planes (elements 0-15 and 16-31 of each block, 16 B per block per plane, so a
//     wave's ds_read_b128 walks consecutive 16 B words without bank conflicts) and a
//     {sum(xq), xs} pair per block.  The staging loads are issued before the weight
//     loads and the barrier only waits for LDS traffic, so weight loads stay in
//     flight across it.
//   * The block dot product is 8 v_dot4_i32_i8 on the raw nibbles (0..15) with the
//     -8 offset removed exactly once per block via -8 * sum(xq) (the reference's
//     bias correction, cuda/nve_kernels.cu:845-853).
//   * Row sums are finished with a DPP wave reduction (no LDS round trip).
//   * Up to three weight matrices sharing the same activations (Q/K/V) run in one
//     launch: workgroups are partitioned into segments, one per matrix.
#include "common.h"
#include "w4_launch.h"

#include "act_producer.h"
#include "w4a8_ops.h"

namespace nve {

// R rows per wave, NJ 64-block chunks per lane in registers.  MULTI = K needs more
// than one pass of NJ chunks (K > 64*NJ*32); then staging runs as a loop.  SRC !=
// SRC_PLAIN computes the activations in the staging from the producer's inputs
// (act_producer.h) and quantizes them in place of reading xq / xs.
// PAIR (act_producer.h): PAIR_SWIGLU -- segment 0 (gate) and the matrix in nib[1] /
// sc[1] (up) share N; a wave computes R/2 rows of each and writes silu(gate) * up
// (src/ops.rs:62-64).  PAIR_ROPE -- segments q, k, v, each N = rows / 2 pairs; a wave
// computes both rows of R/2 RoPE pairs and writes the attention's input (rope_store).
template <int OUT_DT, int R, int NJ, bool MULTI, int SRC = SRC_PLAIN, int PAIR = PAIR_NONE>
__global__ __launch_bounds__(256) void w4a8_gemv_kernel(const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xs,
                                                        W4Segs segs, int K, ProdArgs pa, EpiArgs ra) {
  constexpr bool SWI = PAIR == PAIR_SWIGLU, ROPE = PAIR == PAIR_ROPE, PAIRED = SWI || ROPE;
  static_assert(SRC == SRC_PLAIN || !MULTI, "fused producers stage in one pass");
  static_assert(!PAIRED || (R % 2 == 0 && !MULTI), "paired rows: even R, one pass");
  static_assert(PAIR != PAIR_ARGMAX || OUT_DT == NVE_DT_F32, "greedy candidates over f32 logits");
  constexpr int RH = PAIRED ? R / 2 : R;  // output rows (pairs) per wave
  constexpr int SPT = (NJ + 1) / 2;  // staging passes: 2*nb <= 128*NJ chunks of 16 B
  // DIRECT: a pre-quantized vector (no producer) with at most two 64-block chunks per
  // lane skips the LDS: each lane loads the int8 activations and scales of exactly the
  // blocks it multiplies (the same blocks for all R rows), ahead of its weight loads,
  // so no LDS write, barrier or LDS read sits between the loads and the arithmetic
  // (8B lm_head 49.7 -> 49.1 us, q 3.55 -> 3.46; at four chunks, 1B down, it lost 0.3 us
  // to the per-lane block sums).
  constexpr bool DIRECT = SRC == SRC_PLAIN && !MULTI && NJ <= 2;
  extern __shared__ int4 lds[];
  const int nb = K >> 5;
  const int nchunk = 2 * nb;
  int4* s_lo = lds;
  int4* s_hi = lds + (nb + 1);
  int2* s_bs = (int2*)(lds + 2 * (nb + 1));
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // Segment (matrix) of this workgroup: uniform, resolved with scalar selects.
  const int wg = blockIdx.x;
  const int sg = (segs.nseg > 1 && wg >= segs.wg_begin[1]) + (segs.nseg > 2 && wg >= segs.wg_begin[2]);
  const uint8_t* __restrict__ nib = sg == 0 ? segs.nib[0] : (sg == 1 ? segs.nib[1] : segs.nib[2]);
  const float* __restrict__ ws = sg == 0 ? segs.sc[0] : (sg == 1 ? segs.sc[1] : segs.sc[2]);
  void* __restrict__ out = sg == 0 ? segs.out[0] : (sg == 1 ? segs.out[1] : segs.out[2]);
  const int N = sg == 0 ? segs.n[0] : (sg == 1 ? segs.n[1] : segs.n[2]);
  const int wg0 = sg == 0 ? 0 : (sg == 1 ? segs.wg_begin[1] : segs.wg_begin[2]);
  const int row0 = ((wg - wg0) * 4 + wave) * RH;

  W4A8Stage<SRC == SRC_PLAIN ? SPT : 1> st;
  ProdChunk<SRC, 16> pc[SRC == SRC_PLAIN ? 1 : SPT];
  if constexpr (SRC != SRC_PLAIN) {
#pragma unroll
    for (int s = 0; s < SPT; ++s) prod_issue<SRC, 16>(pc[s], pa, (int)threadIdx.x + 256 * s, nchunk);
  } else if (!MULTI && !DIRECT) {
    w4a8_stage_issue<SPT>(st, xq, xs, nchunk, pa.row_scale != nullptr);
  }
  int4 xlo[DIRECT ? NJ : 1], xhi[DIRECT ? NJ : 1];
  float xsr[DIRECT ? NJ : 1];
  if constexpr (DIRECT) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bb = min(lane + 64 * j, nb - 1);
      xlo[j] = ((const int4*)xq)[2 * bb];
      xhi[j] = ((const int4*)xq)[2 * bb + 1];
      xsr[j] = pa.row_scale != nullptr ? 1.0f : xs[bb];
    }
  }
  // Residual add (F32_ACCUM): the output rows' current values are fetched here, with
  // the staging loads, instead of by a dependent load in the epilogue.  The residual
  // was written by the previous launch and that load would otherwise add a full
  // memory round trip to the end of the kernel.  Each row has one writer (lane 63 of
  // its wave), so the read-add-write stays race-free.
  constexpr bool ACC = OUT_DT == NVE_DT_F32_ACCUM;
  float prev[ACC ? RH : 1];
  if constexpr (ACC) {
#pragma unroll
    for (int r = 0; r < RH; ++r) prev[r] = ((const float*)out)[min(row0 + r, N - 1)];
  }
  // Keep the issue order: staging loads, then weight loads, then LDS writes (which
  // then wait only for the older staging loads).
  __builtin_amdgcn_sched_barrier(0);

  // Weight loads.  Blocks past the end of the row (b >= nb, only in the last chunk
  // of a row) re-load block nb-1 and are zeroed at use, so no load is predicated.
  uint4 wv[R][NJ];
  float wsc[R][NJ];
  const size_t row_bytes = (size_t)(K >> 1);
  auto issue = [&](int jb, int e0 = 0, int e1 = R * NJ) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int rr = min(row0 + (PAIRED ? r % RH : r), N - 1);
      const int row = ROPE ? rope_row(rr, ra.half, r >= RH) : rr;
      const uint8_t* mn = (SWI && r >= RH) ? segs.nib[1] : nib;
      const float* ms = (SWI && r >= RH) ? segs.sc[1] : ws;
      const uint4* rn = (const uint4*)(mn + (size_t)row * row_bytes);
      const float* rs = ms + (size_t)row * nb;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (r * NJ + j < e0 || r * NJ + j >= e1) continue;
        const int b = jb + lane + 64 * j;
        const int bb = min(b, nb - 1);
        wv[r][j] = ld_stream(rn + bb);
        wsc[r][j] = ld_stream(rs + bb);
      }
    }
  };
  // With the RMSNorm in the staging (SRC_NORM) the weight loads are issued once the norm
  // statistic is known, and with an f32 producer vector (SRC_F32) once it is staged: the
  // vector was just written by the previous launch and is fetched past the L2, and
  // issued beside this launch's whole weight stream its loads return late (timestamps in
  // the gate/up launch of the 3B decode step: the norm statistic at 3.8 us median with
  // the weights issued first, 2.0 us with them issued after it, kernel end 7.4 -> 6.6
  // us).  The attention-merge producers keep the early issue (late was measured slower).
  // The decode step's down projection (fp16 SwiGLU output, residual add) is such a
  // just-written vector too.
  constexpr bool kLateWeights =
      SRC == SRC_NORM || SRC == SRC_F32 || (SRC == SRC_F16 && OUT_DT == NVE_DT_F32_ACCUM);
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

  if constexpr (SRC != SRC_PLAIN) {
    double inv = 0.0;
    if (SRC == SRC_NORM)
      inv = prod_norm_inv(prod_sumsq<SRC, 16, SPT>(pc, nchunk), K, pa.eps,
                          (double*)((char*)lds + w4a8_lds_bytes(K)));
    if (kLateWeights && SRC == SRC_NORM) issue_pinned();
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = (int)threadIdx.x + 256 * s;
      float v[16];
      prod_values<SRC, 16>(pc[s], inv, v);
      float scale;
      const int4 q = prod_quant16(v, scale);
      w4a8_stage_put(q, scale, i, i < nchunk, nb, s_lo, s_hi, s_bs);
    }
    if (kLateWeights && SRC != SRC_NORM) issue_pinned();
  } else if (DIRECT) {
  } else if (!MULTI) {
    w4a8_stage_write<SPT>(st, s_lo, s_hi, s_bs, nchunk);
  } else {
    w4a8_stage_loop(xq, xs, s_lo, s_hi, s_bs, nchunk, pa.row_scale != nullptr);
  }
  // the weight arithmetic stays below the staging barrier
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!DIRECT) lds_barrier();

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  for (int jb = 0;;) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int b = jb + lane + 64 * j;
      const int bb = min(b, nb - 1);
      int4 lo, hi;
      int sumq;
      float xsb;
      if constexpr (DIRECT) {
        lo = xlo[j];
        hi = xhi[j];
        sumq = sum_i8x16(lo) + sum_i8x16(hi);
        xsb = xsr[j];
      } else {
        lo = s_lo[bb];
        hi = s_hi[bb];
        const int2 bs = s_bs[bb];
        sumq = bs.x;
        xsb = __builtin_bit_cast(float, bs.y);
      }
      // Lanes past the end of the row contribute nothing.
      const float xsf = b < nb ? xsb : 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int a = w4a8_block_dot(wv[r][j], lo, hi, sumq);
        acc[r] = fmaf(wsc[r][j] * xsf, (float)a, acc[r]);
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
    const float rsc = (SRC == SRC_PLAIN && pa.row_scale) ? bf16_bits_to_f32(*pa.row_scale) : 1.0f;
    float best = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v = wave_sum_to_lane63(acc[r]);
      if (SRC == SRC_PLAIN && pa.row_scale) v *= rsc;
      if (lane == 63 && row0 + r < N) {
        if constexpr (ACC)
          ((float*)out)[row0 + r] = prev[r] + v;
        else
          store_out<OUT_DT>(out, (size_t)(row0 + r), v);
        // the merge rule of the greedy head: larger value, or the lower index of equal
        // ones (-inf included); NaN never wins
        if (PAIR == PAIR_ARGMAX && (v > best || (v == best && row0 + r < bi))) best = v, bi = row0 + r;
      }
    }
    if constexpr (PAIR == PAIR_ARGMAX) {
      // the workgroup's candidate: lane 63 of each wave holds its rows' candidate
      __shared__ float s_av[4];
      __shared__ int s_ai[4];
      if (lane == 63) s_av[wave] = best, s_ai[wave] = bi;
      __syncthreads();
      if (threadIdx.x == 0) {
        best = s_av[0];
        bi = s_ai[0];
        for (int w = 1; w < 4; ++w)
          if (s_av[w] > best || (s_av[w] == best && s_ai[w] < bi)) best = s_av[w], bi = s_ai[w];
        ra.arg_v[wg - wg0] = best;
        ra.arg_i[wg - wg0] = bi;
      }
    }
  }
}

// Debug export: exact int32 block accumulators acc[n, b] through w4a8_block_dot.
__global__ __launch_bounds__(256) void w4a8_block_acc_kernel(const int8_t* __restrict__ xq,
                                                             const uint8_t* __restrict__ nib,
                                                             int32_t* __restrict__ acc, int N,
                                                             int K) {
  const int nb = K >> 5;
  const size_t total = (size_t)N * nb;
  for (size_t t = (size_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (size_t)gridDim.x * 256) {
    const size_t n = t / nb;
    const int b = (int)(t % nb);
    const uint4 w = ((const uint4*)(nib + n * (size_t)(K >> 1)))[b];
    const int4 lo = ((const int4*)xq)[2 * b];
    const int4 hi = ((const int4*)xq)[2 * b + 1];
    acc[t] = w4a8_block_dot(w, lo, hi, sum_i8x16(lo) + sum_i8x16(hi));
  }
}

}  // namespace nve

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace nve_host {

template <int OUT_DT, int R, int NJ, bool MULTI, int SRC, int PAIR>
static hipError_t launch_w4a8_t(const int8_t* xq, const float* xs, const W4Segs& segs, int K,
                                int grid, const nve::ProdArgs& pa, hipStream_t stream,
                                const nve::EpiArgs& ra = nve::EpiArgs{}) {
  constexpr bool direct = SRC == nve::SRC_PLAIN && !MULTI && NJ <= 2;  // no LDS staging (see the kernel)
  const size_t lds = direct ? 0 : nve::w4a8_lds_bytes(K) + (SRC == nve::SRC_NORM ? 64 : 0);
  auto kern = nve::w4a8_gemv_kernel<OUT_DT, R, NJ, MULTI, SRC, PAIR>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, stream, xq, xs, segs, K, pa, ra);
  return hipGetLastError();
}

template <int OUT_DT>
static hipError_t launch_w4a8_dt(const int8_t* xq, const float* xs, W4Segs segs, int K,
                                 hipStream_t stream, const nve::ProdArgs& pa = nve::ProdArgs{}) {
  const W4Tiling t = choose_w4_tiling(segs, K);
  finalize_segments(segs, t.R);
  const int grid = segs.wg_total;
#define NVE_W4A8_CASE(RR, JJ, MM) \
  if (t.R == RR && t.NJ == JJ && t.multi == MM) \
    return launch_w4a8_t<OUT_DT, RR, JJ, MM, nve::SRC_PLAIN, nve::PAIR_NONE>(xq, xs, segs, K, grid, pa, stream);
  NVE_W4_TILING_CASES(NVE_W4A8_CASE)
#undef NVE_W4A8_CASE
  return hipErrorInvalidValue;
}

// Fused-producer launches (one-shot kernels, one staging pass: K <= 16384).
template <int OUT_DT, int SRC, int PAIR>
static hipError_t launch_w4a8_fused_t(const nve::ProdArgs& pa, W4Segs segs, int K, hipStream_t stream,
                                      const nve::EpiArgs& ra) {
  const W4Tiling t = nve::attn_splits_of(SRC) ? choose_merge_tiling(segs, K) : choose_w4_tiling(segs, K);
  if (t.multi) return hipErrorInvalidValue;
  if (PAIR != nve::PAIR_NONE) {
    const int R = t.R < 2 ? 2 : t.R;
    if (PAIR == nve::PAIR_SWIGLU) segs.nseg = 1;  // gate in slot 0, up in slot 1 (read by the kernel directly)
    if (PAIR == nve::PAIR_ROPE)
      for (int i = 0; i < segs.nseg; ++i) segs.n[i] /= 2;  // RoPE pairs per matrix
    finalize_segments(segs, R / 2);
#define NVE_W4A8_PAIR_CASE(RR, JJ) \
    if (R == RR && t.NJ == JJ) \
      return launch_w4a8_t<OUT_DT, RR, JJ, false, SRC, PAIR>(nullptr, nullptr, segs, K, segs.wg_total, pa, stream, ra);
    NVE_W4_SWIGLU_CASES(NVE_W4A8_PAIR_CASE)
#undef NVE_W4A8_PAIR_CASE
    return hipErrorInvalidValue;
  }
  finalize_segments(segs, t.R);
#define NVE_W4A8_CASE(RR, JJ, MM) \
  if (t.R == RR && t.NJ == JJ && !MM) \
    return launch_w4a8_t<OUT_DT, RR, JJ, false, SRC, nve::PAIR_NONE>(nullptr, nullptr, segs, K, segs.wg_total, pa, stream);
  NVE_W4_TILING_CASES(NVE_W4A8_CASE)
#undef NVE_W4A8_CASE
  return hipErrorInvalidValue;
}

// One activation row with one bf16 scale (per-token mode, the M = 1 case of the batched
// entry point): the one-shot kernel with unit block scales and the row scale applied to
// the row sums.
hipError_t launch_w4a8_rowscale(const int8_t* xq, const uint16_t* row_scale, const W4Segs& segs, int out_dt, int K,
                                hipStream_t stream) {
  nve::ProdArgs pa{};
  pa.row_scale = row_scale;
  const float* no_xs = nullptr;
  switch (out_dt) {
    case NVE_DT_F16: return launch_w4a8_dt<NVE_DT_F16>(xq, no_xs, segs, K, stream, pa);
    case NVE_DT_BF16: return launch_w4a8_dt<NVE_DT_BF16>(xq, no_xs, segs, K, stream, pa);
    default: return launch_w4a8_dt<NVE_DT_F32>(xq, no_xs, segs, K, stream, pa);
  }
}

hipError_t launch_w4a8(const int8_t* xq, const float* xs, const W4Segs& segs, int out_dt, int K,
                       hipStream_t stream) {
  if (use_persistent(segs, K, false)) return launch_w4a8_persistent(xq, xs, segs, out_dt, K, stream);
  switch (out_dt) {
    case NVE_DT_F16: return launch_w4a8_dt<NVE_DT_F16>(xq, xs, segs, K, stream);
    case NVE_DT_BF16: return launch_w4a8_dt<NVE_DT_BF16>(xq, xs, segs, K, stream);
    case NVE_DT_F32_ACCUM: return launch_w4a8_dt<NVE_DT_F32_ACCUM>(xq, xs, segs, K, stream);
    default: return launch_w4a8_dt<NVE_DT_F32>(xq, xs, segs, K, stream);
  }
}

hipError_t launch_w4a8_argmax(const int8_t* xq, const float* xs, const W4Segs& segs_in, int K, float* arg_v,
                              int* arg_i, int* ncand, hipStream_t stream) {
  W4Segs segs = segs_in;
  if (segs.nseg != 1) return hipErrorInvalidValue;
  const W4Tiling t = choose_w4_tiling(segs, K);
  finalize_segments(segs, t.R);
  *ncand = segs.wg_total;
  nve::EpiArgs ra{};
  ra.arg_v = arg_v;
  ra.arg_i = arg_i;
#define NVE_W4A8_ARG_CASE(RR, JJ, MM)            \
  if (t.R == RR && t.NJ == JJ && t.multi == MM) \
    return launch_w4a8_t<NVE_DT_F32, RR, JJ, MM, nve::SRC_PLAIN, nve::PAIR_ARGMAX>(xq, xs, segs, K, segs.wg_total, \
                                                                                  nve::ProdArgs{}, stream, ra);
  NVE_W4_TILING_CASES(NVE_W4A8_ARG_CASE)
#undef NVE_W4A8_ARG_CASE
  return hipErrorInvalidValue;
}

// Decode-layer W4A8 GEMVs with a fused producer (act_producer.h):
//   NORM, F32, rope    Q/K/V from the residual and the norm weights, RoPE + KV append
//                      in the epilogue (PAIR_ROPE; out[] unused);
//   NORM, F32          Q/K/V from the residual and the norm weights;
//   NORM, F32, swiglu  gate/up -> silu(gate) * up (f32);
//   F32, F32_ACCUM     down from that f32 vector, quantized in the staging;
//   ATTN2/4, F32_ACCUM o_proj from the key-split attention partials.
hipError_t launch_w4a8_fused(int src, int pair, const nve::ProdArgs& pa, const W4Segs& segs, int out_dt, int K,
                             hipStream_t stream, const nve::EpiArgs& ra) {
  if (src == nve::SRC_NORM && out_dt == NVE_DT_F16 && pair == nve::PAIR_SWIGLU)
    return launch_w4a8_fused_t<NVE_DT_F16, nve::SRC_NORM, nve::PAIR_SWIGLU>(pa, segs, K, stream, ra);
  if (src == nve::SRC_NORM && out_dt == NVE_DT_F32) {
    if (pair == nve::PAIR_ROPE)
      return launch_w4a8_fused_t<NVE_DT_F32, nve::SRC_NORM, nve::PAIR_ROPE>(pa, segs, K, stream, ra);
    return pair == nve::PAIR_SWIGLU ? launch_w4a8_fused_t<NVE_DT_F32, nve::SRC_NORM, nve::PAIR_SWIGLU>(pa, segs, K, stream, ra)
                                    : launch_w4a8_fused_t<NVE_DT_F32, nve::SRC_NORM, nve::PAIR_NONE>(pa, segs, K, stream, ra);
  }
  if (pair != nve::PAIR_NONE) return hipErrorInvalidValue;
#define NVE_FU(SRC, OD) launch_w4a8_fused_t<OD, SRC, nve::PAIR_NONE>(pa, segs, K, stream, ra)
  if (src == nve::SRC_F32 && out_dt == NVE_DT_F32_ACCUM) return NVE_FU(nve::SRC_F32, NVE_DT_F32_ACCUM);
  if (src == nve::SRC_F16 && out_dt == NVE_DT_F32_ACCUM) return NVE_FU(nve::SRC_F16, NVE_DT_F32_ACCUM);
  if (src == nve::SRC_ATTN2 && out_dt == NVE_DT_F32_ACCUM) return NVE_FU(nve::SRC_ATTN2, NVE_DT_F32_ACCUM);
  if (src == nve::SRC_ATTN4 && out_dt == NVE_DT_F32_ACCUM) return NVE_FU(nve::SRC_ATTN4, NVE_DT_F32_ACCUM);
  if (src == nve::SRC_ATTN8 && out_dt == NVE_DT_F32_ACCUM) return NVE_FU(nve::SRC_ATTN8, NVE_DT_F32_ACCUM);
  // W4A8 GEMV quantizing its own 16-bit / f32 activations (fp16 or fp32 output)
#define NVE_QX(SRC)                                                                    \
  if (src == SRC) {                                                                    \
    if (out_dt == NVE_DT_F16) return NVE_FU(SRC, NVE_DT_F16);                          \
    if (out_dt == NVE_DT_F32) return NVE_FU(SRC, NVE_DT_F32);                          \
    return hipErrorInvalidValue;                                                       \
  }
  NVE_QX(nve::SRC_F16)
  NVE_QX(nve::SRC_BF16)
  NVE_QX(nve::SRC_F32)
#undef NVE_QX
#undef NVE_FU
  return hipErrorInvalidValue;
}

hipError_t launch_w4a8_block_acc(const int8_t* xq, const uint8_t* nib, int32_t* acc, int N, int K,
                                 hipStream_t stream) {
  const size_t total = (size_t)N * (K / 32);
  size_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(nve::w4a8_block_acc_kernel, dim3((unsigned)g), dim3(256), 0, stream, xq, nib, acc,
                     N, K);
  return hipGetLastError();
}

}  // namespace nve_host
