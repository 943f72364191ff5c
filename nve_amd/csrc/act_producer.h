// act_producer.h -- activation producers fused into the GEMV staging.
//
// A decode layer feeds its GEMVs with vectors that a small elementwise kernel would
// otherwise produce just before (RMSNorm of the residual, the int8 quantization of
// silu(gate) * up).  Every
// GEMV workgroup stages the whole activation vector in LDS anyway, so it can compute
// that vector itself from the producer's inputs: the loads are issued with the
// staging loads (ahead of the weight loads), the arithmetic runs while the weight
// loads are in flight, and one kernel launch per producer disappears.  The output of
// a producer is the same f32 value the standalone kernel computes; the GEMV then
// quantizes it to int8 with group-32 scales (W4A8) or rounds it to bf16 (W4A16)
// exactly as the standalone path does.
//
//   SRC_NORM: x_k = h_k * w_k / sqrt(mean(h^2) + eps), sum of squares and scaling in
//             f64 (src/ops.rs:12-30); a = h (f32 [K]), b = w (bf16 [K]).
//   SRC_F32:  x_k = a_k (an f32 vector, e.g. silu(gate) * up written by the SwiGLU
//             epilogue of the gate/up GEMV); b unused.
//   SRC_F16 / SRC_BF16: x_k = a_k of a 16-bit vector (the W4A8 GEMV that quantizes its
//             own activations: nve_quantize_f16_q8 + nve_matvec_w4a8 in one launch).
//   SRC_ATTN1 / 2 / 4 / 8: the decode attention output, merged from the partials of 1,
//             2, 4 or 8 key splits: a = records [split][head] of (m, l, -, -, acc[D]) with
//             m the running max of the scores in log2 units (q . k * log2(e) / sqrt(D)),
//             l the sum of 2^(s - m), acc the unnormalised value sum;
//             x = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s (M = max_s m_s);
//             i0 = head_dim, i1 = num_heads.
#pragma once

#include "common.h"

namespace nve {

enum {
  SRC_PLAIN = 0, SRC_NORM = 1, SRC_F32 = 2, SRC_F16 = 3, SRC_BF16 = 4, SRC_ATTN2 = 5, SRC_ATTN4 = 6, SRC_ATTN8 = 7,
  SRC_ATTN1 = 8
};

__host__ __device__ constexpr int attn_splits_of(int src) {
  return src == SRC_ATTN2 ? 2 : (src == SRC_ATTN4 ? 4 : (src == SRC_ATTN8 ? 8 : (src == SRC_ATTN1 ? 1 : 0)));
}

struct ProdArgs {
  const void* a;
  const void* b;
  float eps;
  int i0, i1;
  // SRC_PLAIN W4A8 only: one bf16 activation scale for the whole row (per-token mode);
  // the block sums are then formed with the weight scales alone and the row sum is
  // multiplied by this scale (NULL: group-32 scales from xs).
  const uint16_t* row_scale;
};

// E activations (8 or 16) of one staging chunk: f32 sources in a, 16-bit sources in h.
template <int SRC, int E>
struct ProdChunk {
  static constexpr bool kHalf = SRC == SRC_F16 || SRC == SRC_BF16;
  static constexpr int kSplits = attn_splits_of(SRC);
  float4 a[kHalf ? 1 : (kSplits ? kSplits * E / 4 : E / 4)];
  uint4 h[kHalf ? E / 8 : 1];
  uint4 b[SRC == SRC_NORM ? E / 8 : 1];
  float2 ml[kSplits ? kSplits : 1];
};

template <int SRC, int E>
__device__ __forceinline__ void prod_issue(ProdChunk<SRC, E>& c, const ProdArgs& p, int chunk, int nchunk) {
  const int i = min(chunk, nchunk - 1);
  if constexpr (ProdChunk<SRC, E>::kSplits > 0) {
    constexpr int S = ProdChunk<SRC, E>::kSplits;
    const int D = p.i0, H = p.i1;
    const int e0 = i * E, hd = e0 / D, d0 = e0 % D;
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      const float* rec = (const float*)p.a + (size_t)(sp * H + hd) * (D + 4);
      c.ml[sp] = *(const float2*)rec;
#pragma unroll
      for (int t = 0; t < E / 4; ++t) c.a[sp * (E / 4) + t] = ((const float4*)(rec + 4 + d0))[t];
    }
    return;
  }
  if constexpr (ProdChunk<SRC, E>::kHalf) {
#pragma unroll
    for (int t = 0; t < E / 8; ++t) c.h[t] = ((const uint4*)p.a)[i * (E / 8) + t];
    return;
  }
#pragma unroll
  for (int t = 0; t < E / 4; ++t) c.a[t] = ((const float4*)p.a)[i * (E / 4) + t];
  if constexpr (SRC == SRC_NORM) {
#pragma unroll
    for (int t = 0; t < E / 8; ++t) c.b[t] = ((const uint4*)p.b)[i * (E / 8) + t];
  }
}

// Sum of squares of the valid chunks of this thread (SRC_NORM), in f64.
template <int SRC, int E, int SPT>
__device__ __forceinline__ double prod_sumsq(const ProdChunk<SRC, E> (&c)[SPT], int nchunk) {
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < SPT; ++s) {
    const bool ok = (int)threadIdx.x + 256 * s < nchunk;
#pragma unroll
    for (int t = 0; t < E / 4; ++t) {
      const float4 v = c[s].a[t];
      const double q = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
      ss += ok ? q : 0.0;
    }
  }
  return ss;
}

// 1 / sqrt(mean(h^2) + eps) over the K elements, reduced over the 256 threads of the
// workgroup (a DPP / permlane wave sum, then 4 partials through LDS).  Every workgroup
// sums in the same order, so all of them produce the same value.  (The wave sum was six
// __shfl_xor steps: twelve dependent ds_bpermute round trips, about 1 us of the
// launch's critical path.)
__device__ __forceinline__ double prod_norm_inv(double ss, int K, float eps, double* s_red) {
  ss = group_sum_f64<64>(ss);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
  lds_barrier();
  const double tot = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  return 1.0 / sqrt(tot / (double)K + (double)eps);
}

template <int SRC, int E>
__device__ __forceinline__ void prod_values(const ProdChunk<SRC, E>& c, double inv, float (&v)[E]) {
  if constexpr (ProdChunk<SRC, E>::kSplits > 0) {
    constexpr int S = ProdChunk<SRC, E>::kSplits;
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < S; ++sp) M = fmaxf(M, c.ml[sp].x);
    float f[S], L = 0.0f;
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      f[sp] = c.ml[sp].x == -INFINITY ? 0.0f : exp2f(c.ml[sp].x - M);
      L = fmaf(f[sp], c.ml[sp].y, L);
    }
    const float invL = 1.0f / L;
#pragma unroll
    for (int t = 0; t < E / 4; ++t) {
      float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int sp = 0; sp < S; ++sp) {
        const float4 a4 = c.a[sp * (E / 4) + t];
        o[0] = fmaf(f[sp], a4.x, o[0]);
        o[1] = fmaf(f[sp], a4.y, o[1]);
        o[2] = fmaf(f[sp], a4.z, o[2]);
        o[3] = fmaf(f[sp], a4.w, o[3]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * t + e] = o[e] * invL;
    }
    return;
  }
  if constexpr (ProdChunk<SRC, E>::kHalf) {
#pragma unroll
    for (int t = 0; t < E / 8; ++t) {
      const uint32_t d[4] = {c.h[t].x, c.h[t].y, c.h[t].z, c.h[t].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * t + 2 * e] = SRC == SRC_BF16 ? bf16_bits_to_f32(d[e] & 0xffffu) : f16_bits_to_f32(d[e] & 0xffffu);
        v[8 * t + 2 * e + 1] = SRC == SRC_BF16 ? bf16_bits_to_f32(d[e] >> 16) : f16_bits_to_f32(d[e] >> 16);
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < E / 4; ++t) {
    const float a4[4] = {c.a[t].x, c.a[t].y, c.a[t].z, c.a[t].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 4 * t + e;
      if (SRC == SRC_NORM) {
        const uint4 wb = c.b[k / 8];
        const uint32_t wd[4] = {wb.x, wb.y, wb.z, wb.w};
        const uint32_t pair = wd[(k % 8) / 2];
        const float w = bf16_bits_to_f32((k & 1) ? (pair >> 16) : (pair & 0xffffu));
        v[k] = (float)((double)a4[e] * inv * (double)w);
      } else {
        v[k] = a4[e];
      }
    }
  }
}

// W4A8: 16 values of a half block -> 16 int8 codes; the block's scale comes from the
// absmax over the two lanes (2k, 2k+1) holding the block (nve_quantize_f16_q8 rule).
__device__ __forceinline__ int4 prod_quant16(const float (&v)[16], float& scale_out) {
  float m = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(v[e]));
  m = fmaxf(m, dpp_mov<0xB1>(m));  // quad_perm [1,0,3,2]: the pair partner
  const float scale = m > 0.0f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / scale;
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) w |= (uint32_t)(uint8_t)q8_round_clamp(v[4 * t + e] * inv) << (8 * e);
    d[t] = w;
  }
  scale_out = scale;
  return make_int4((int)d[0], (int)d[1], (int)d[2], (int)d[3]);
}

// W4A16: 8 values -> 8 bf16 (round to nearest even), as the standalone producers store.
// Eight producer values rounded once to fp16 (W4A16 staging in MODE_F16).  The values
// are formed in f64 and narrowed to f32 first; f32_to_f16_rne keeps that f32 step (left to
// itself the compiler folds the two truncations into one f64 -> f16 conversion, which
// gfx950 has no instruction for: a 30-instruction integer sequence per value).
__device__ __forceinline__ uint4 prod_f16x8(const float (&v)[8]) {
  uint32_t d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    d[t] = (uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(v[2 * t])) |
           ((uint32_t)__builtin_bit_cast(uint16_t, f32_to_f16_rne(v[2 * t + 1])) << 16);
  return make_uint4(d[0], d[1], d[2], d[3]);
}

}  // namespace nve

namespace nve {

// ---- epilogues of the fused GEMV launches (paired rows, or the greedy candidate) ------
// PAIR_SWIGLU: a wave computes R/2 rows of gate (segment 0) and the same rows of up (the
//   matrix in nib[1] / sc[1]) and writes silu(gate) * up (src/ops.rs:62-64).
// PAIR_ROPE: the Q/K/V launch of a decode layer.  A wave computes, for R/2 pairs p of a
//   head (column d = p % half), rows d and d + half, so it holds both halves of every
//   RoPE pair (src/ops.rs:264-276) and finishes the attention's input in its epilogue:
//   q rotated and multiplied by qscale (f32), the new key rotated and the new value, both
//   rounded to bf16, written straight into the KV cache at the token's position.
// PAIR_ARGMAX: plain rows, stored as usual, and each workgroup's greedy candidate
// (largest value, lowest index among equal ones, NaN never) written to
// arg_v / arg_i[workgroup].
enum { PAIR_NONE = 0, PAIR_SWIGLU = 1, PAIR_ROPE = 2, PAIR_ARGMAX = 3 };

struct EpiArgs {
  float* q;            // f32 [num_heads * D]
  uint16_t* kc;        // bf16 [num_kv_heads, max_seq, D]
  uint16_t* vc;
  const int* pos;      // device position of the token (clamped to [0, max_seq))
  const float* cos;    // f32 [max_seq, D/2]
  const float* sin;
  int max_seq, half;   // half = D / 2
  float qscale;
  float* arg_v;        // PAIR_ARGMAX: per-workgroup candidates
  int* arg_i;
};

__host__ __device__ __forceinline__ int rope_row(int p, int half, bool second) {
  return (p / half) * 2 * half + p % half + (second ? half : 0);
}

__device__ __forceinline__ int rope_pos(const EpiArgs& ra) { return min(max(*ra.pos, 0), ra.max_seq - 1); }

// Segment sg of the Q/K/V launch: 0 = q, 1 = k, 2 = v; x0 / x1 = rows d / d + half.
__device__ __forceinline__ void rope_store(const EpiArgs& ra, int sg, int p, float x0, float x1, float c, float s,
                                           int pos) {
  const int half = ra.half, head = p / half, d = p % half;
  if (sg == 0) {
    float* q = ra.q + (size_t)head * 2 * half;
    q[d] = (x0 * c - x1 * s) * ra.qscale;
    q[d + half] = (x0 * s + x1 * c) * ra.qscale;
  } else {
    uint16_t* row = (sg == 1 ? ra.kc : ra.vc) + ((size_t)head * ra.max_seq + pos) * 2 * half;
    if (sg == 1) {
      row[d] = f32_to_bf16_bits(x0 * c - x1 * s);
      row[d + half] = f32_to_bf16_bits(x0 * s + x1 * c);
    } else {
      row[d] = f32_to_bf16_bits(x0);
      row[d + half] = f32_to_bf16_bits(x1);
    }
  }
}

}  // namespace nve
