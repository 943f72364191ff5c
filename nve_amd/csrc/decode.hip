// decode.hip -- one decode step of a Llama-style decoder on MI355X, built around the
// W4A8 / W4A16 GEMV kernels: RMSNorm (with the W4A8 activation quantization fused
// in), RoPE + KV-cache append fused into split-sequence decode attention, SiLU-mul
// (quantization fused), residual adds fused into the GEMV epilogue (NVE_DT_F32_ACCUM),
// and the head: final norm, lm_head, greedy argmax, next-token embedding, position
// advance.  Positions live in device memory, so a whole step is graph-capturable.
//
// Restates the decode path of the reference: gpu_layer_forward_decode
// (src/gpu_layer.rs:1005-1084), gpu_attn_decode (633-775), gpu_ffn (914-997), and the
// CPU semantics of src/ops.rs (rms_norm 12-30 with f64 accumulation, RoPE half-split
// pairs 264-276, silu 62-64, softmax 152-163, argmax 485-495 first maximum) and
// src/attention.rs:149-228 (GQA, scale 1/sqrt(head_dim)).
#include <math.h>
#include <stdlib.h>

#include "common.h"
#include "act_producer.h"
#include "w4_launch.h"

namespace nve {

// ---- RMSNorm ------------------------------------------------------------------
// y_i = h_i * w_i / sqrt(mean(h^2) + eps): sum of squares and the scaling in f64 as
// src/ops.rs:12-30, output rounded once.  One workgroup of 1024 threads; thread t
// handles elements 4t..4t+3 of each 4096-element pass (8 threads per 32-group, so the
// fused W4A8 quantization is a DPP reduction over 8 lanes).
// OUT: 0 -> fp16 y (a W4A16 layer's input); 1 -> int8 xq + f32 group scales
// (nve_quantize_f16_q8 semantics).
template <int OUT>
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ h,
                                                       const uint16_t* __restrict__ w, float eps, int H,
                                                       uint16_t* __restrict__ y16, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs) {
  __shared__ double red[16];
  double ss = 0.0;
  for (int i = threadIdx.x; i < H; i += 1024) {
    const double v = (double)h[i];
    ss += v * v;
  }
  ss = group_sum_f64<64>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x < 64) {
    double v = threadIdx.x < 16 ? red[threadIdx.x] : 0.0;
    v = group_sum_f64<16>(v);
    if (threadIdx.x == 0) red[0] = v;
  }
  __syncthreads();
  const double inv = 1.0 / sqrt(red[0] / (double)H + (double)eps);
  for (int base = 0; base < H; base += 4096) {
    const int i0 = base + 4 * (int)threadIdx.x;
    const bool ok = i0 < H;  // H % 32 == 0: the 8 lanes of a group agree
    float v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int i = ok ? i0 + t : 0;
      v[t] = (float)((double)h[i] * inv * (double)bf16_bits_to_f32(w[i]));
    }
    if (OUT == 0) {
      if (ok)
#pragma unroll
        for (int t = 0; t < 4; ++t) ((_Float16*)y16)[i0 + t] = f32_to_f16_rne(v[t]);
    } else {
      q8_group8_store(v, ok, xq, xs, (size_t)(ok ? i0 : 0));
    }
  }
}

// ---- attention ------------------------------------------------------------------
// One launch per layer: RoPE on q and on the new key, KV-cache append,
// softmax(q k^T / sqrt(D)) v over the cache, and the conversion of the output to the
// o_proj input (OUT 1: fp16, OUT 2: int8 + group-32 scales).
//
// One workgroup of 8 waves per query head; no cross-workgroup communication.  Keys
// are spread over the waves in tiles: a key's row of D bf16 (D/8 16-byte pieces)
// sits in LPK = D/8 consecutive lanes, one piece per lane, so the q.k dot product is
// a butterfly over those lanes and the value sum accumulates each lane's 8 columns.
// Scores are kept in log2 units (q is pre-multiplied by log2(e) / sqrt(D)), so every
// softmax weight is one exp2 of a score difference.  Every wave keeps its own online
// softmax (running max m, sum l, accumulator rescaled by 2^(m_old - m_new) when the
// maximum grows) over its keys, with the next two tiles' K/V loads in flight while
// the current tile is computed; the 8 wave states are merged once in LDS at the
// end:  out = sum_w 2^(m_w - M) acc_w / sum_w 2^(m_w - M) l_w.
// The new token's key is rotated and rounded to bf16 like every cached entry; the
// workgroup of the kv head's first query head writes it and the value to the cache,
// the others use their own identical copy for that row.
// One key slot per lane per tile (32-key tiles at D = 128): against two slots the 3B
// decode ran 1081 against 1064 tok/s at 512 cached keys and 826 against 820 at 7000
// (with 16 waves) -- a workgroup streams its K/V through one CU, and the smaller tile
// shortens that stream's first wait and its tail.  Eight waves against sixteen: the
// merge at the end combines half the wave states, 1177 against 1173.5 tok/s at 512 keys
// (four key splits), 1168 against 1153 with eight splits, 888.6 against 881.6 at 7000.
template <int D>
struct AttnTile {
  static constexpr int NW = 8;          // waves per workgroup
  static constexpr int P = 1;           // key slots per lane per tile
  static constexpr int LPK = D / 8;     // lanes per key
  static constexpr int KPW = 64 / LPK;  // keys per wave per slot
  static constexpr int KT = NW * KPW * P;
  uint4 k[P], v[P];
};

// Rows past the live length are masked at use, so the load addresses only need to stay
// below `limit` (max_seq for the first tiles, which are issued before the position is
// known; the live length afterwards).
template <int D>
__device__ __forceinline__ void attn_issue(AttnTile<D>& b, const uint16_t* __restrict__ kc,
                                           const uint16_t* __restrict__ vc, size_t cache_base, int t, int limit,
                                           int wave, int krow, int col) {
  using T = AttnTile<D>;
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * T::NW + wave) * T::KPW + krow;
    const size_t off = cache_base + (size_t)(key < limit ? key : limit - 1) * D + col * 8;
    b.k[i] = *(const uint4*)(kc + off);
    b.v[i] = *(const uint4*)(vc + off);
  }
}

// NEWROW: the row at pos comes from the workgroup's own copy in LDS (s_knew / s_vnew)
// rather than the cache (which this launch writes).
template <int D, bool NEWROW = true>
__device__ __forceinline__ void attn_compute(const AttnTile<D>& b, int t, int len, int pos, int wave, int krow,
                                             int col, const float (&qv)[8], const uint16_t* s_knew,
                                             const uint16_t* s_vnew, float& m_run, float& l_run, float (&acc)[8]) {
  using T = AttnTile<D>;
  float s[T::P];
  float m_tile = -INFINITY;
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * T::NW + wave) * T::KPW + krow;
    const uint4 kr = (NEWROW && key == pos) ? *(const uint4*)(s_knew + col * 8) : b.k[i];
    const uint32_t w[4] = {kr.x, kr.y, kr.z, kr.w};
    float d = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      d = fmaf(qv[2 * u + 1], bf16_bits_to_f32(w[u] >> 16), fmaf(qv[2 * u], bf16_bits_to_f32(w[u] & 0xffffu), d));
    d = group_sum<T::LPK>(d);
    s[i] = key < len ? d : -INFINITY;
    m_tile = fmaxf(m_tile, s[i]);
  }
  // the maximum over every key of the wave: the same value in all lanes, so the
  // rescale below is a uniform branch, taken only when the running maximum grows
  m_tile = stride_max<T::LPK>(m_tile);
  if (m_tile > m_run) {
    const float alpha = exp2f(m_run - m_tile);  // 0 while m_run is -inf
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
    m_run = m_tile;
  }
  if (m_run == -INFINITY) return;  // no valid key for this wave yet
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * T::NW + wave) * T::KPW + krow;
    const float p = exp2f(s[i] - m_run);  // masked keys: exp2(-inf) = 0
    l_run += p;
    // rows past the length may hold anything (even NaN): they must not reach acc
    const uint4 vr = (NEWROW && key == pos) ? *(const uint4*)(s_vnew + col * 8)
                                             : (key < len ? b.v[i] : make_uint4(0, 0, 0, 0));
    const uint32_t w[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[2 * u] = fmaf(p, bf16_bits_to_f32(w[u] & 0xffffu), acc[2 * u]);
      acc[2 * u + 1] = fmaf(p, bf16_bits_to_f32(w[u] >> 16), acc[2 * u + 1]);
    }
  }
}

// Merge of the wave states of an attention workgroup and its output: the normalised
// head output converted to the o_proj input (OUT 1: fp16, 2: int8 + group scales), or
// (OUT 3) the split's partial record (m, l, 0, 0, acc[D]).
template <int D, int OUT, int SPLIT>
__device__ __forceinline__ void attn_finish(float m_run, float l_run, float (&acc)[8], int hq, int sp, int num_heads,
                                            int wave, int krow, int col, int tid, float* s_m, float* s_l, float* s_acc, uint16_t* __restrict__ out16,
                                            int8_t* __restrict__ out_q, float* __restrict__ out_s,
                                            float* __restrict__ out_part) {
  using T = AttnTile<D>;
  // merge the rows of the wave (same columns), then the waves through LDS
  l_run = stride_sum<T::LPK>(l_run);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = stride_sum<T::LPK>(acc[e]);
  if (krow == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave * D + col * 8 + e] = acc[e];
    if (col == 0) {
      s_m[wave] = m_run;
      s_l[wave] = l_run;
    }
  }
  lds_barrier();
  if constexpr (OUT == 3) {
    // split partial record (m, l, 0, 0, acc[D]): the first D / 32 waves merge, lane l of
    // wave w owning column 32 w + l % 32 and the waves' halves l / 32 (half of the wave
    // states each); the two halves meet through one xor-32 lane exchange.  Every lane
    // forms M and the weights 2^(m_w - M) itself from the broadcast maxima.
    static_assert(D % 32 == 0 && T::NW % 2 == 0 && D / 32 <= T::NW, "merge layout");
    if (wave < D / 32) {
      const int lane = tid & 63, c = 32 * wave + (lane & 31), h = lane >> 5;
      float mw[T::NW];
#pragma unroll
      for (int w = 0; w < T::NW; w += 4) {
        const float4 m4 = *(const float4*)&s_m[w];
        mw[w] = m4.x, mw[w + 1] = m4.y, mw[w + 2] = m4.z, mw[w + 3] = m4.w;
      }
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < T::NW; ++w) M = fmaxf(M, mw[w]);
      constexpr int HW = T::NW / 2;
      float L = 0.0f, o = 0.0f;
#pragma unroll
      for (int k = 0; k < HW; ++k) {
        const int w = h * HW + k;
        const float mk = s_m[w];  // not mw[w]: a lane-dependent index would put mw in LDS
        const float f = mk == -INFINITY ? 0.0f : exp2f(mk - M);
        L = fmaf(f, s_l[w], L);
        o = fmaf(f, s_acc[w * D + c], o);
      }
      L += __shfl_xor(L, 32);
      o += __shfl_xor(o, 32);
      float* rec = out_part + ((size_t)sp * num_heads + hq) * (D + 4);
      if (tid == 0) *(float4*)rec = make_float4(M, L, 0.0f, 0.0f);
      if (h == 0) rec[4 + c] = o;
    }
    return;
  }
  // one barrier: every output lane reads the wave maxima and sums, forms the wave
  // weights 2^(m_w - M) itself (independent exp2, no second LDS round trip) and sums the
  // wave accumulators of its 4 columns
  if (tid < D / 4) {
    float mw[T::NW], lw[T::NW];
#pragma unroll
    for (int w = 0; w < T::NW; w += 4) {
      const float4 m4 = *(const float4*)&s_m[w];
      const float4 l4 = *(const float4*)&s_l[w];
      mw[w] = m4.x, mw[w + 1] = m4.y, mw[w + 2] = m4.z, mw[w + 3] = m4.w;
      lw[w] = l4.x, lw[w + 1] = l4.y, lw[w + 2] = l4.z, lw[w + 3] = l4.w;
    }
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < T::NW; ++w) M = fmaxf(M, mw[w]);
    float L = 0.0f;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < T::NW; ++w) {
      const float f = mw[w] == -INFINITY ? 0.0f : exp2f(mw[w] - M);
      L = fmaf(f, lw[w], L);
      const float4 a4 = *(const float4*)&s_acc[w * D + 4 * tid];
      o[0] = fmaf(f, a4.x, o[0]);
      o[1] = fmaf(f, a4.y, o[1]);
      o[2] = fmaf(f, a4.z, o[2]);
      o[3] = fmaf(f, a4.w, o[3]);
    }
    const float invL = 1.0f / L;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] *= invL;
    const size_t i0 = (size_t)hq * D + 4 * tid;
    if (OUT == 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) ((_Float16*)out16)[i0 + e] = f32_to_f16_rne(o[e]);
    } else {
      q8_group8_store(o, true, out_q, out_s, i0);
    }
  }
}

// SPLIT > 1 (OUT 3): workgroup (head, sp) takes the tiles t = sp, sp + SPLIT, ... and
// writes its partial state (m, l, 0, 0, acc[D]) -- m in log2 units, acc not yet
// divided by l -- to out_part[sp][head]; the consumer merges the SPLIT partials
// (act_producer.h, SRC_ATTN2 / 4 / 8).  A split with no tile writes m = -inf, l = 0, acc = 0.
// PRE: the Q/K/V launch has already rotated q (and multiplied it by qscale) and
// appended the new key and value to the cache (PAIR_ROPE epilogue): q is read as is, the
// cache holds every row up to pos, and only the first tile's loads are issued before
// the position is known (the others only if the split has them).
template <int D, int OUT, int SPLIT = 1, bool PRE = false>
__global__ __launch_bounds__(64 * AttnTile<D>::NW) void attn_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, const int* __restrict__ d_pos,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int num_heads, int num_kv_heads,
    int max_seq, float qscale, uint16_t* __restrict__ out16, int8_t* __restrict__ out_q,
    float* __restrict__ out_s, float* __restrict__ out_part, int xcd_map) {
  static_assert((OUT == 3) == (SPLIT > 1), "split partials go to out_part");
  using T = AttnTile<D>;
  constexpr int HALF = D / 2;
  __shared__ float s_q[D];
  __shared__ __align__(16) uint16_t s_knew[D];
  __shared__ __align__(16) uint16_t s_vnew[D];
  __shared__ __align__(16) float s_m[T::NW];
  __shared__ __align__(16) float s_l[T::NW];
  __shared__ __align__(16) float s_acc[T::NW * D];

  const int G = num_heads / num_kv_heads;
  // Workgroups are dealt to the 8 XCDs round-robin (XCD = block % 8), each with its own
  // L2.  With xcd_map the G query heads of one (kv head, split) -- which read the same
  // K/V rows -- get block ids 8 apart, so they run on one XCD and share its L2.
  int hq, sp;
  if (xcd_map) {
    const int b = blockIdx.x, x = b % 8, j = b / 8;
    const int pair = (j / G) * 8 + x;  // (kv head, split) pair
    hq = (pair % num_kv_heads) * G + j % G;
    sp = pair / num_kv_heads;
  } else {
    hq = blockIdx.x % num_heads;
    sp = blockIdx.x / num_heads;
  }
  const int kvh = hq / G;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col = lane % T::LPK, krow = lane / T::LPK;
  const size_t cache_base = (size_t)kvh * max_seq * D;

  // three tile buffers in a ring; without PRE the first three tiles' loads are issued at
  // once (their addresses do not depend on the position, rows past the end are masked
  // at use); with PRE only the first, and the next two once the position is known
  AttnTile<D> b0, b1, b2;
  attn_issue<D>(b0, kc, vc, cache_base, sp, max_seq, wave, krow, col);
  if (!PRE) {
    attn_issue<D>(b1, kc, vc, cache_base, sp + SPLIT, max_seq, wave, krow, col);
    attn_issue<D>(b2, kc, vc, cache_base, sp + 2 * SPLIT, max_seq, wave, krow, col);
  }
  if constexpr (PRE) {
    // q (rotated, scaled) is loaded with the first tile, before the position
    float qv[8];
    {
      const float4 qa = *(const float4*)(q + (size_t)hq * D + col * 8);
      const float4 qb = *(const float4*)(q + (size_t)hq * D + col * 8 + 4);
      qv[0] = qa.x, qv[1] = qa.y, qv[2] = qa.z, qv[3] = qa.w, qv[4] = qb.x, qv[5] = qb.y, qv[6] = qb.z, qv[7] = qb.w;
    }
    const int pos = min(max(*d_pos, 0), max_seq - 1);
    const int len = pos + 1;
    const int ntiles = (len + T::KT - 1) / T::KT;
    const int nt = ntiles > sp ? (ntiles - sp + SPLIT - 1) / SPLIT : 0;
    // The ring's loads are issued unconditionally wherever they precede the steady-state
    // loop (rows past the length clamp to the last live row: a tile the split does not
    // have costs one cached row per load), so the waits inside the loop count the two
    // younger tiles' loads exactly: with conditional issues the compiler drained the
    // whole ring (vmcnt(0)) before every third tile.
    attn_issue<D>(b1, kc, vc, cache_base, sp + SPLIT, len, wave, krow, col);
    attn_issue<D>(b2, kc, vc, cache_base, sp + 2 * SPLIT, len, wave, krow, col);
    float m_run = -INFINITY, l_run = 0.0f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    int j = 0;
    for (; j + 5 < nt; j += 3) {  // every refill is a live tile
      attn_compute<D, false>(b0, sp + SPLIT * j, len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run, acc);
      attn_issue<D>(b0, kc, vc, cache_base, sp + SPLIT * (j + 3), len, wave, krow, col);
      attn_compute<D, false>(b1, sp + SPLIT * (j + 1), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
      attn_issue<D>(b1, kc, vc, cache_base, sp + SPLIT * (j + 4), len, wave, krow, col);
      attn_compute<D, false>(b2, sp + SPLIT * (j + 2), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
      attn_issue<D>(b2, kc, vc, cache_base, sp + SPLIT * (j + 5), len, wave, krow, col);
    }
    // the last five tiles at most: b0, b1, b2 hold tiles j, j + 1, j + 2
    if (j < nt)
      attn_compute<D, false>(b0, sp + SPLIT * j, len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run, acc);
    if (j + 3 < nt) attn_issue<D>(b0, kc, vc, cache_base, sp + SPLIT * (j + 3), len, wave, krow, col);
    if (j + 1 < nt)
      attn_compute<D, false>(b1, sp + SPLIT * (j + 1), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
    if (j + 4 < nt) attn_issue<D>(b1, kc, vc, cache_base, sp + SPLIT * (j + 4), len, wave, krow, col);
    if (j + 2 < nt)
      attn_compute<D, false>(b2, sp + SPLIT * (j + 2), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
    if (j + 3 < nt)
      attn_compute<D, false>(b0, sp + SPLIT * (j + 3), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
    if (j + 4 < nt)
      attn_compute<D, false>(b1, sp + SPLIT * (j + 4), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run,
                             acc);
    attn_finish<D, OUT, SPLIT>(m_run, l_run, acc, hq, sp, num_heads, wave, krow, col, tid, s_m, s_l, s_acc,
                               out16, out_q, out_s, out_part);
    return;
  }
  // q, k, v of this head before the position-dependent RoPE rows
  float q0 = 0.0f, q1 = 0.0f, k0 = 0.0f, k1 = 0.0f, v0 = 0.0f, v1 = 0.0f;
  if (tid < HALF) {
    q0 = q[(size_t)hq * D + tid];
    q1 = q[(size_t)hq * D + tid + HALF];
    k0 = k[(size_t)kvh * D + tid];
    k1 = k[(size_t)kvh * D + tid + HALF];
    v0 = v[(size_t)kvh * D + tid];
    v1 = v[(size_t)kvh * D + tid + HALF];
  }
  // a position past the cache is clamped to its last slot (the host bounds the step
  // count; the clamp only keeps every access inside the cache and the RoPE tables)
  const int pos = min(max(*d_pos, 0), max_seq - 1);
  const int len = pos + 1;
  const int ntiles = (len + T::KT - 1) / T::KT;
  // this workgroup's tiles: sp + SPLIT * j for j < nt
  const int nt = ntiles > sp ? (ntiles - sp + SPLIT - 1) / SPLIT : 0;

  if (tid < HALF) {
    const float c = rope_cos[(size_t)pos * HALF + tid], sn = rope_sin[(size_t)pos * HALF + tid];
    s_q[tid] = (q0 * c - q1 * sn) * qscale;
    s_q[tid + HALF] = (q0 * sn + q1 * c) * qscale;
    s_knew[tid] = f32_to_bf16_bits(k0 * c - k1 * sn);
    s_knew[tid + HALF] = f32_to_bf16_bits(k0 * sn + k1 * c);
    s_vnew[tid] = f32_to_bf16_bits(v0);
    s_vnew[tid + HALF] = f32_to_bf16_bits(v1);
  }
  lds_barrier();
  if (hq % G == 0 && sp == 0)
    for (int i = tid; i < D; i += 64 * T::NW) {
      kc[cache_base + (size_t)pos * D + i] = s_knew[i];
      vc[cache_base + (size_t)pos * D + i] = s_vnew[i];
    }
  float qv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qv[e] = s_q[col * 8 + e];

  float m_run = -INFINITY, l_run = 0.0f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  // a buffer is refilled only when a later tile of this workgroup remains: loads past
  // the last tile would only be waited for (their registers are reused by the merge)
  for (int j = 0; j < nt; j += 3) {
    attn_compute<D>(b0, sp + SPLIT * j, len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run, acc);
    if (j + 3 < nt) attn_issue<D>(b0, kc, vc, cache_base, sp + SPLIT * (j + 3), len, wave, krow, col);
    if (j + 1 < nt)
      attn_compute<D>(b1, sp + SPLIT * (j + 1), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run, acc);
    if (j + 4 < nt) attn_issue<D>(b1, kc, vc, cache_base, sp + SPLIT * (j + 4), len, wave, krow, col);
    if (j + 2 < nt)
      attn_compute<D>(b2, sp + SPLIT * (j + 2), len, pos, wave, krow, col, qv, s_knew, s_vnew, m_run, l_run, acc);
    if (j + 5 < nt) attn_issue<D>(b2, kc, vc, cache_base, sp + SPLIT * (j + 5), len, wave, krow, col);
  }
  attn_finish<D, OUT, SPLIT>(m_run, l_run, acc, hq, sp, num_heads, wave, krow, col, tid, s_m, s_l, s_acc,
                             out16, out_q, out_s, out_part);
}

// ---- SiLU * up ------------------------------------------------------------------
// mid = silu(gate) * up (src/ops.rs:62-64: g / (1 + exp(-g))) rounded to fp16.  OUT 0 ->
// fp16, 1 -> int8 + group scales of the fp16 values (fused W4A8 quantization; 8 lanes per
// 32-group).
template <int OUT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                       int F, uint16_t* __restrict__ y16, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs) {
  const int i0 = 4 * ((int)blockIdx.x * 256 + (int)threadIdx.x);
  const bool ok = i0 < F;  // F % 32 == 0
  const int ib = ok ? i0 : 0;
  const float4 g4 = *(const float4*)(gate + ib);
  const float4 u4 = *(const float4*)(up + ib);
  const float gg[4] = {g4.x, g4.y, g4.z, g4.w}, uu[4] = {u4.x, u4.y, u4.z, u4.w};
  float v[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) v[t] = (float)f32_to_f16_rne(gg[t] / (1.0f + expf(-gg[t])) * uu[t]);
  if (OUT == 0) {
    if (ok)
#pragma unroll
      for (int t = 0; t < 4; ++t) ((_Float16*)y16)[i0 + t] = f32_to_f16_rne(v[t]);
  } else {
    q8_group8_store(v, ok, xq, xs, (size_t)ib);
  }
}

// ---- head: greedy argmax (first maximum), next-token embedding, position advance --
// The W4A8 lm_head launch leaves one (value, index) candidate per workgroup (its
// PAIR_ARGMAX epilogue); after a W4A16 lm_head, kArgmaxBlocks workgroups each reduce a
// slice of the logits to one.  One workgroup then reduces the candidates, writes the
// token, embeds its row into hidden and advances the position (the launch boundary
// orders the candidates' writes before their reads -- no device-scope fence or arrival
// counter).  NaN never wins; among equal values the lowest index wins
// (src/ops.rs:485-495 keeps the first maximum).
constexpr int kArgmaxBlocks = 128;

__device__ __forceinline__ void argmax_merge(float& b, int& bi, float o, int oi) {
  if (o > b || (o == b && oi < bi)) {
    b = o;
    bi = oi;
  }
}

// Wave butterfly on DPP / permlane moves (the steps of group_sum): the merge is
// symmetric (larger value, or the lower index of equal values), so both lanes of a pair
// keep the same (value, index) and every lane ends with the wave's result.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& b, int& bi) {
  argmax_merge(b, bi, dpp_mov<CTRL>(b), dpp_mov_i<CTRL>(bi));
}
template <bool X32>
__device__ __forceinline__ void argmax_xor(float& b, int& bi) {
  const uint32_t u = __builtin_bit_cast(uint32_t, b), ui = (uint32_t)bi;
  const auto r = X32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false) : __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const auto ri = X32 ? __builtin_amdgcn_permlane32_swap(ui, ui, false, false)
                      : __builtin_amdgcn_permlane16_swap(ui, ui, false, false);
  // one of the two results is the lane's own pair (a no-op merge), the other its partner's
  argmax_merge(b, bi, __builtin_bit_cast(float, (uint32_t)r[0]), (int)ri[0]);
  argmax_merge(b, bi, __builtin_bit_cast(float, (uint32_t)r[1]), (int)ri[1]);
}

template <int NW>
__device__ __forceinline__ void argmax_block(float& best, int& bi, float* s_v, int* s_i) {
  argmax_dpp<0xB1>(best, bi);   // quad_perm [1,0,3,2]
  argmax_dpp<0x4E>(best, bi);   // quad_perm [2,3,0,1]
  argmax_dpp<0x141>(best, bi);  // row_half_mirror
  argmax_dpp<0x140>(best, bi);  // row_mirror
  argmax_xor<false>(best, bi);
  argmax_xor<true>(best, bi);
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = best;
    s_i[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < NW; ++w) argmax_merge(best, bi, s_v[w], s_i[w]);
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits, int V,
                                                             float* __restrict__ part_v, int* __restrict__ part_i) {
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  // slices of a multiple of 1024 logits: every thread reads whole float4s, four of
  // them issued before any is compared
  const int per = ((V + kArgmaxBlocks - 1) / kArgmaxBlocks + 1023) & ~1023;
  const int lo = blockIdx.x * per, hi = min(V, lo + per);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  if (((uintptr_t)logits & 15) == 0) {
    for (int c = 0; c < per; c += 4096) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = lo + c + 1024 * u + 4 * (int)threadIdx.x;
        v[u] = i + 3 < hi ? *(const float4*)(logits + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = lo + c + 1024 * u + 4 * (int)threadIdx.x;
        if (i + 3 < hi) {
          argmax_merge(best, bi, v[u].x, i);
          argmax_merge(best, bi, v[u].y, i + 1);
          argmax_merge(best, bi, v[u].z, i + 2);
          argmax_merge(best, bi, v[u].w, i + 3);
        } else {
          for (int e = 0; e < 4; ++e)
            if (i + e < hi) argmax_merge(best, bi, logits[i + e], i + e);
        }
      }
    }
  } else {
    for (int i = lo + threadIdx.x; i < hi; i += 256) argmax_merge(best, bi, logits[i], i);
  }
  argmax_block<4>(best, bi, s_v, s_i);
  if (threadIdx.x == 0) {
    part_v[blockIdx.x] = best;
    part_i[blockIdx.x] = bi;
  }
}

// nparts candidates (the argmax_partial_kernel slices, or the per-workgroup candidates
// of the lm_head GEMV's PAIR_ARGMAX epilogue), merged by 1024 threads: every thread's
// loads are issued before any is merged.
__global__ __launch_bounds__(1024) void argmax_embed_kernel(const float* __restrict__ part_v,
                                                            const int* __restrict__ part_i, int nparts,
                                                            const uint16_t* __restrict__ embed, int H,
                                                            float* __restrict__ hidden, int* __restrict__ token_out,
                                                            int* __restrict__ d_pos) {
  __shared__ float s_v[16];
  __shared__ int s_i[16];
  __shared__ int s_tok;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int U = 8;
  for (int base = 0; base < nparts; base += 1024 * U) {
    float v[U];
    int ix[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + 1024 * u + (int)threadIdx.x;
      v[u] = i < nparts ? part_v[i] : -INFINITY;
      ix[u] = i < nparts ? part_i[i] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) argmax_merge(best, bi, v[u], ix[u]);
  }
  argmax_block<16>(best, bi, s_v, s_i);
  if (threadIdx.x == 0) {
    if (bi == 0x7fffffff) bi = 0;  // all NaN / -inf: token 0
    s_tok = bi;
    *token_out = bi;
  }
  __syncthreads();
  const int tok = s_tok;
  for (int i = threadIdx.x; i < H; i += 1024) hidden[i] = bf16_bits_to_f32(embed[(size_t)tok * H + i]);
  if (threadIdx.x == 0) *d_pos += 1;
}

__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ embed, const int* __restrict__ token,
                                                    float* __restrict__ hidden, int H, int vocab) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int t = min(max(*token, 0), vocab - 1);  // a token outside the table is clamped into it
  if (i < H) hidden[i] = bf16_bits_to_f32(embed[(size_t)t * H + i]);
}

}  // namespace nve

// ---------------------------------------------------------------------------
// Host side: workspace layout and the per-layer / head orchestration.
// ---------------------------------------------------------------------------
namespace nve_host {

struct DecodeWs {
  uint16_t* act16;  // [max(H, Hq*D, F)]
  int8_t* xq;          // [max(H, Hq*D, F)]
  float* xs;           // [max/32]
  float* q;            // [Hq*D]
  float* k;            // [Hkv*D]
  float* v;            // [Hkv*D]
  float* gate;         // [F]
  float* up;           // [F]
  float* arg_v;        // [argmax_slots]: greedy candidates of the head
  int* arg_i;          // [argmax_slots]
  float* logits;       // [V] (head only, when the caller passes no logits buffer)
  float* part;         // [kMaxAttnSplit][Hq][D + 4] key-split attention partials
  size_t bytes;
};

constexpr int kMaxAttnSplit = 8;
// cache capacity above which the attention takes eight key splits (where they fit)
constexpr int kAttnSplit8Slots = 1024;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }



// Candidate slots of the greedy head: the lm_head GEMV writes one per workgroup, at
// least four rows each.
static int argmax_slots(const nve_decode_config& c) {
  const int per_wg = ((c.vocab > 0 ? c.vocab : 1) + 3) / 4;
  return per_wg > nve::kArgmaxBlocks ? per_wg : nve::kArgmaxBlocks;
}

static DecodeWs layout_ws(const nve_decode_config& c, void* base) {
  DecodeWs w{};
  const size_t qd = (size_t)c.num_heads * c.head_dim, kd = (size_t)c.num_kv_heads * c.head_dim;
  size_t mx = (size_t)c.hidden;
  if (qd > mx) mx = qd;
  if ((size_t)c.ffn > mx) mx = c.ffn;
  char* p = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  w.act16 = (uint16_t*)take(mx * 2);
  w.xq = (int8_t*)take(mx);
  w.xs = (float*)take(mx / 32 * 4);
  w.q = (float*)take(qd * 4);
  w.k = (float*)take(kd * 4);
  w.v = (float*)take(kd * 4);
  w.gate = (float*)take((size_t)c.ffn * 4);
  w.up = (float*)take((size_t)c.ffn * 4);
  w.arg_v = (float*)take((size_t)argmax_slots(c) * 4);
  w.arg_i = (int*)take((size_t)argmax_slots(c) * 4);
  w.logits = (float*)take((size_t)(c.vocab > 0 ? c.vocab : 1) * 4);
  w.part = (float*)take((size_t)kMaxAttnSplit * c.num_heads * (c.head_dim + 4) * 4);
  w.bytes = off;
  return w;
}

size_t decode_workspace_bytes(const nve_decode_config& c) { return layout_ws(c, nullptr).bytes; }

static int check_cfg(const nve_decode_config& c) {
  if (c.hidden < 32 || c.hidden % 32 || c.num_heads < 1 || c.num_kv_heads < 1 || c.num_heads % c.num_kv_heads ||
      c.num_heads / c.num_kv_heads > 8 || (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) ||
      c.ffn < 32 || c.ffn % 32 || c.max_seq < 1 || ((size_t)c.num_heads * c.head_dim) % 32)
    return NVE_ERR_SHAPE;
  if (c.hidden > NVE_MAX_K || c.ffn > NVE_MAX_K || c.num_heads * c.head_dim > NVE_MAX_K ||
      (size_t)c.num_kv_heads * c.max_seq * c.head_dim > (size_t)INT32_MAX)
    return NVE_ERR_TOO_LARGE;
  return NVE_OK;
}

static W4Segs one_seg(const nve_w4_weight& w, void* out) {
  W4Segs s{};
  s.nseg = 1;
  s.nib[0] = w.nibbles;
  s.sc[0] = w.scales;
  s.out[0] = out;
  s.n[0] = w.n;
  return s;
}

static W4Segs segs3(const nve_w4_weight* w, void* const* outs, int count) {
  W4Segs s{};
  s.nseg = count;
  for (int i = 0; i < count; ++i) {
    s.nib[i] = w[i].nibbles;
    s.sc[i] = w[i].scales;
    s.out[i] = outs[i];
    s.n[i] = w[i].n;
  }
  return s;
}

hipError_t launch_q8_group(const void* x, int xdt, size_t total, int8_t* xq, float* scales, hipStream_t stream);

#define NVE_TRY(x)                              \
  do {                                          \
    const hipError_t e_ = (x);                  \
    if (e_ != hipSuccess) return (int)e_;       \
  } while (0)

static hipError_t launch_rmsnorm(const nve_decode_config& c, const float* h, const uint16_t* w, bool to_q8,
                                 const DecodeWs& ws, hipStream_t s) {
  if (to_q8)
    hipLaunchKernelGGL(nve::rmsnorm_kernel<1>, dim3(1), dim3(1024), 0, s, h, w, c.eps, c.hidden, nullptr, ws.xq,
                       ws.xs);
  else
    hipLaunchKernelGGL(nve::rmsnorm_kernel<0>, dim3(1), dim3(1024), 0, s, h, w, c.eps, c.hidden, ws.act16,
                       nullptr, nullptr);
  return hipGetLastError();
}

// pre: the Q/K/V launch ran the PAIR_ROPE epilogue (q rotated and scaled in ws.q, the
// new key / value already in the cache).
static hipError_t launch_attention(const nve_decode_config& c, const nve_decode_io& io, const DecodeWs& ws,
                                   bool w4a8, int split, bool pre, hipStream_t s) {
  // scores in log2 units: q is pre-multiplied by log2(e) / sqrt(D), so the softmax
  // weights are exp2 of score differences
  const float qscale = 1.4426950408889634f / sqrtf((float)c.head_dim);
  // (kv head, split) pairs a multiple of 8: each XCD gets whole groups of query heads
  const int xcd_map = (c.num_kv_heads * split) % 8 == 0 && c.num_heads / c.num_kv_heads > 1;
#define NVE_ATTN_P(D, OUT, S, P)                                                                             \
  hipLaunchKernelGGL((nve::attn_decode_kernel<D, OUT, S, P>), dim3(c.num_heads * S), dim3(64 * nve::AttnTile<D>::NW), 0, s, ws.q, ws.k, \
                     ws.v, io.k_cache, io.v_cache, io.pos, io.rope_cos, io.rope_sin, c.num_heads,                \
                     c.num_kv_heads, c.max_seq, qscale, ws.act16, ws.xq, ws.xs, ws.part, xcd_map)
#define NVE_ATTN(D, OUT, S)          \
  if (pre) NVE_ATTN_P(D, OUT, S, true); \
  else NVE_ATTN_P(D, OUT, S, false);
#define NVE_ATTN_D(D)                      \
  if (split == 8) { NVE_ATTN(D, 3, 8) }     \
  else if (split == 4) { NVE_ATTN(D, 3, 4) } \
  else if (split == 2) { NVE_ATTN(D, 3, 2) } \
  else if (w4a8) { NVE_ATTN(D, 2, 1) }      \
  else { NVE_ATTN(D, 1, 1) }
  if (c.head_dim == 64) {
    NVE_ATTN_D(64)
  } else if (c.head_dim == 128) {
    NVE_ATTN_D(128)
  } else {
    NVE_ATTN_D(256)
  }
#undef NVE_ATTN_D
#undef NVE_ATTN
#undef NVE_ATTN_P
  return hipGetLastError();
}

// Key splits of the fused decode attention (the partials are merged in the o_proj
// GEMV's staging), chosen from the cache capacity: a workgroup's K/V stream passes
// through one CU (about 60 GB/s), so caches past a few hundred keys need more
// workgroups per head; the merging o_proj launch uses few
// workgroups, so the merge costs little.  Eight splits hold 8 partial chunks in the
// o_proj staging registers, which fits one staging pass (num_heads * head_dim <= 4096);
// wider layers use four.  NVE_ATTN_SPLIT=1/2/4/8 overrides (8 only where it fits).
static int attn_split_max(const nve_decode_config& c) { return c.num_heads * c.head_dim <= 4096 ? 8 : 4; }

static int attn_split(const nve_decode_config& c) {
  const char* e = getenv("NVE_ATTN_SPLIT");
  if (e && (e[0] == '1' || e[0] == '2' || e[0] == '4' || e[0] == '8') && e[1] == 0)
    return e[0] - '0' < attn_split_max(c) ? e[0] - '0' : attn_split_max(c);
  return c.max_seq <= 256 ? 1 : (c.max_seq <= kAttnSplit8Slots ? 4 : attn_split_max(c));
}

// Fused producers in the decode layer (RMSNorm into Q/K/V and gate/up, SiLU * up into
// down); NVE_DECODE_FUSE=0 (read at every call, so a host can switch per call) selects
// the standalone producer kernels instead.
static bool decode_fuse() {
  const char* e = getenv("NVE_DECODE_FUSE");
  return !(e && e[0] == '0' && e[1] == 0);
}

static hipError_t gemv(bool w4a8, const DecodeWs& ws, const W4Segs& sg, int out_dt, int K, hipStream_t s) {
  return w4a8 ? launch_w4a8(ws.xq, ws.xs, sg, out_dt, K, s)
              : launch_w4a16(ws.act16, NVE_DT_F16, sg, out_dt, K, s);
}

static hipError_t gemv_fused(bool w4a8, int src, int pair, const nve::ProdArgs& pa, const W4Segs& sg, int out_dt,
                             int K, hipStream_t s, const nve::EpiArgs& ra = nve::EpiArgs{}) {
  return w4a8 ? launch_w4a8_fused(src, pair, pa, sg, out_dt, K, s, ra)
              : launch_w4a16_fused(src, pair, pa, sg, out_dt, K, s, ra);
}

int layer_forward_decode(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io,
                         bool w4a8, hipStream_t s) {
  const DecodeWs ws = layout_ws(c, io.workspace);
  const int H = c.hidden, F = c.ffn, QD = c.num_heads * c.head_dim;
  const bool fuse = decode_fuse();
  // attention sub-layer: norm -> Q/K/V (one grouped launch) -> attention -> o_proj (+h)
  {
    const nve_w4_weight qkv[3] = {w.q, w.k, w.v};
    void* outs[3] = {ws.q, ws.k, ws.v};
    const W4Segs sg = segs3(qkv, outs, 3);
    if (fuse) {
      // RoPE and the KV-cache append run in the epilogue (PAIR_ROPE)
      const nve::EpiArgs ra{ws.q, io.k_cache, io.v_cache, io.pos, io.rope_cos, io.rope_sin, c.max_seq,
                             c.head_dim / 2, 1.4426950408889634f / sqrtf((float)c.head_dim)};
      NVE_TRY(gemv_fused(w4a8, nve::SRC_NORM, nve::PAIR_ROPE, nve::ProdArgs{io.hidden, w.input_norm, c.eps}, sg,
                         NVE_DT_F32, H, s, ra));
    } else {
      NVE_TRY(launch_rmsnorm(c, io.hidden, w.input_norm, w4a8, ws, s));
      NVE_TRY(gemv(w4a8, ws, sg, NVE_DT_F32, H, s));
    }
  }
  // attention writes the o_proj input directly (int8 + scales, or fp16), or, split over
  // the keys, partials that the o_proj staging merges
  const int split = fuse ? attn_split(c) : 1;
  NVE_TRY(launch_attention(c, io, ws, w4a8, split, fuse, s));
  if (split > 1)
    NVE_TRY(gemv_fused(w4a8, split == 8 ? nve::SRC_ATTN8 : (split == 4 ? nve::SRC_ATTN4 : nve::SRC_ATTN2), nve::PAIR_NONE,
                       nve::ProdArgs{ws.part, nullptr, 0.0f, c.head_dim, c.num_heads}, one_seg(w.o, io.hidden),
                       NVE_DT_F32_ACCUM, QD, s));
  else
    NVE_TRY(gemv(w4a8, ws, one_seg(w.o, io.hidden), NVE_DT_F32_ACCUM, QD, s));
  // FFN sub-layer: norm -> gate/up (one grouped launch) -> silu*up -> down (+h).  Fused:
  // the gate/up launch pairs the rows of both matrices and writes silu(gate) * up
  // rounded to fp16, as the reference's candle FFN holds it (src/gpu_layer.rs:937-946);
  // the W4A8 down GEMV quantizes it in its staging, the W4A16 one reads it as is.
  {
    const nve_w4_weight gu[2] = {w.gate, w.up};
    if (fuse) {
      void* outs[2] = {(void*)ws.act16, nullptr};
      const W4Segs sg = segs3(gu, outs, 2);
      NVE_TRY(gemv_fused(w4a8, nve::SRC_NORM, nve::PAIR_SWIGLU, nve::ProdArgs{io.hidden, w.post_attn_norm, c.eps}, sg,
                         NVE_DT_F16, H, s));
      if (w4a8)
        NVE_TRY(gemv_fused(true, nve::SRC_F16, nve::PAIR_NONE, nve::ProdArgs{ws.act16, nullptr, 0.0f},
                           one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
      else
        NVE_TRY(gemv(false, ws, one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
      return NVE_OK;
    }
    void* outs[2] = {ws.gate, ws.up};
    const W4Segs sg = segs3(gu, outs, 2);
    NVE_TRY(launch_rmsnorm(c, io.hidden, w.post_attn_norm, w4a8, ws, s));
    NVE_TRY(gemv(w4a8, ws, sg, NVE_DT_F32, H, s));
  }
  const dim3 sgrid((F / 4 + 255) / 256);
  if (w4a8)
    hipLaunchKernelGGL(nve::silu_mul_kernel<1>, sgrid, dim3(256), 0, s, ws.gate, ws.up, F, nullptr, ws.xq, ws.xs);
  else
    hipLaunchKernelGGL(nve::silu_mul_kernel<0>, sgrid, dim3(256), 0, s, ws.gate, ws.up, F, ws.act16, nullptr,
                       nullptr);
  NVE_TRY(hipGetLastError());
  NVE_TRY(gemv(w4a8, ws, one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
  return NVE_OK;
}

// One fused launch of the decode layer, exactly as layer_forward_decode issues it (same
// kernel instantiation, arguments and workspace), with its input / output exposed:
//   STAGE_QKV:    RMSNorm(h) -> Q/K/V GEMV -> RoPE; q (scaled) to out f32 [Hq*D], the new
//                 key / value rows to the caches at *pos.
//   STAGE_O_MERGE: attention partials in (f32 [split][Hq][D+4]) merged in the o_proj
//                 staging; h += o_proj(merged).  split = the layer's key-split count.
//   STAGE_GATE_UP: RMSNorm(h) -> gate/up GEMV pair -> silu(gate) * up, fp16 out [F].
//   STAGE_DOWN:   fp16 in [F] -> down GEMV (W4A8: quantized in its staging); h += y.
int decode_stage(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io, bool w4a8,
                 int stage, const void* in, void* out, hipStream_t s) {
  const DecodeWs ws = layout_ws(c, io.workspace);
  const int H = c.hidden, F = c.ffn, QD = c.num_heads * c.head_dim;
  switch (stage) {
    case NVE_STAGE_QKV: {
      const nve_w4_weight qkv[3] = {w.q, w.k, w.v};
      void* outs[3] = {out, ws.k, ws.v};
      const nve::EpiArgs ra{(float*)out, io.k_cache, io.v_cache, io.pos, io.rope_cos, io.rope_sin, c.max_seq,
                             c.head_dim / 2, 1.4426950408889634f / sqrtf((float)c.head_dim)};
      NVE_TRY(gemv_fused(w4a8, nve::SRC_NORM, nve::PAIR_ROPE, nve::ProdArgs{io.hidden, w.input_norm, c.eps},
                         segs3(qkv, outs, 3), NVE_DT_F32, H, s, ra));
      return NVE_OK;
    }
    case NVE_STAGE_O_MERGE: {
      const int split = attn_split(c);
      if (split < 2) return NVE_ERR_SHAPE;  // no partials to merge: o_proj is the plain GEMV
      NVE_TRY(gemv_fused(w4a8, split == 8 ? nve::SRC_ATTN8 : (split == 4 ? nve::SRC_ATTN4 : nve::SRC_ATTN2),
                         nve::PAIR_NONE, nve::ProdArgs{in, nullptr, 0.0f, c.head_dim, c.num_heads},
                         one_seg(w.o, io.hidden), NVE_DT_F32_ACCUM, QD, s));
      return NVE_OK;
    }
    case NVE_STAGE_GATE_UP: {
      const nve_w4_weight gu[2] = {w.gate, w.up};
      void* outs[2] = {out, nullptr};
      NVE_TRY(gemv_fused(w4a8, nve::SRC_NORM, nve::PAIR_SWIGLU, nve::ProdArgs{io.hidden, w.post_attn_norm, c.eps},
                         segs3(gu, outs, 2), NVE_DT_F16, H, s));
      return NVE_OK;
    }
    case NVE_STAGE_DOWN:
      if (w4a8)
        NVE_TRY(gemv_fused(true, nve::SRC_F16, nve::PAIR_NONE, nve::ProdArgs{in, nullptr, 0.0f},
                           one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
      else
        NVE_TRY(launch_w4a16(in, NVE_DT_F16, one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
      return NVE_OK;
    default:
      return NVE_ERR_DTYPE;
  }
}

int attn_splits(const nve_decode_config& c) { return attn_split(c); }

int decode_head(const nve_decode_config& c, const nve_decode_head& hd, bool w4a8, hipStream_t s) {
  const DecodeWs ws = layout_ws(c, hd.workspace);
  float* logits = hd.logits ? hd.logits : ws.logits;
  // (the RMSNorm stays a kernel of its own here: fused into the lm_head staging it
  // would be recomputed by every one of the ~8000 workgroups, measured 44 us vs 42)
  int ncand = nve::kArgmaxBlocks;
  NVE_TRY(launch_rmsnorm(c, hd.hidden, hd.final_norm, w4a8, ws, s));
  if (w4a8 && (hd.lm_head.n + 3) / 4 <= argmax_slots(c)) {
    // the lm_head launch leaves one greedy candidate per workgroup (of >= 4 rows)
    NVE_TRY(launch_w4a8_argmax(ws.xq, ws.xs, one_seg(hd.lm_head, logits), c.hidden, ws.arg_v, ws.arg_i, &ncand, s));
  } else {
    // (also a W4A8 lm_head with more rows than the workspace's vocab has slots for,
    // possible when the caller passes its own logits buffer)
    if (w4a8)
      NVE_TRY(launch_w4a8(ws.xq, ws.xs, one_seg(hd.lm_head, logits), NVE_DT_F32, c.hidden, s));
    else
      NVE_TRY(launch_w4a16(ws.act16, NVE_DT_F16, one_seg(hd.lm_head, logits), NVE_DT_F32, c.hidden, s));
    hipLaunchKernelGGL(nve::argmax_partial_kernel, dim3(nve::kArgmaxBlocks), dim3(256), 0, s, logits, hd.lm_head.n,
                       ws.arg_v, ws.arg_i);
  }
  hipLaunchKernelGGL(nve::argmax_embed_kernel, dim3(1), dim3(1024), 0, s, ws.arg_v, ws.arg_i, ncand, hd.embed,
                     c.hidden, hd.hidden, hd.token_out, hd.pos);
  return (int)hipGetLastError();
}

hipError_t launch_embed(const uint16_t* embed, const int* token, float* hidden, int H, int vocab, hipStream_t s) {
  hipLaunchKernelGGL(nve::embed_kernel, dim3((H + 255) / 256), dim3(256), 0, s, embed, token, hidden, H, vocab);
  return hipGetLastError();
}

int check_decode(const nve_decode_config& c) { return check_cfg(c); }

}  // namespace nve_host

// ---------------------------------------------------------------------------
// The decode layer without a caller workspace (nve_hip_layer_forward_decode_noalloc):
// its scratch is a file-scope device array, one copy per GPU, whose address is looked
// up once per device with hipGetSymbolAddress.  No allocation happens on any call, so
// the entry point can run where hipMalloc cannot (under graph capture, in serving
// loops).  Calls that overlap on one GPU (concurrent streams) share the array and race.
// ---------------------------------------------------------------------------
namespace nve {
constexpr size_t kDecodeScratchBytes = 1u << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];
}  // namespace nve

#include <mutex>

namespace nve_host {

// Device address of this GPU's scratch array (the host-side symbol is only a handle).
static hipError_t decode_scratch_ptr(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(nve::scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return hipSuccess;
}

int layer_forward_decode_noalloc(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io,
                                 bool w4a8, hipStream_t s) {
  // the layer reads no logits: lay the workspace out without them
  nve_decode_config cl = c;
  cl.vocab = 0;
  if (decode_workspace_bytes(cl) > nve::kDecodeScratchBytes) return NVE_ERR_TOO_LARGE;
  void* p = nullptr;
  const hipError_t e = decode_scratch_ptr(&p);
  if (e != hipSuccess) return (int)e;
  nve_decode_io io2 = io;
  io2.workspace = p;
  return layer_forward_decode(cl, w, io2, w4a8, s);
}

}  // namespace nve_host
