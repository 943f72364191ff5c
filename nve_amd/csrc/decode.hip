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

#include "common.h"
#include "w4_launch.h"

namespace nve {

// Keys per attention work item: 64 (32 for head_dim 256, to keep the K/V tiles of a
// workgroup within 64 KB of LDS).
__host__ __device__ constexpr int attn_chunk(int D) { return D == 256 ? 32 : 64; }
// Chunks per kv head the combine holds in LDS (max_seq <= 256 * attn_chunk(D)).
constexpr int kAttnMaxChunks = 256;

// Loads that must see other workgroups' stores from the same launch (after their
// release fence): device-scope atomic loads bypass the CU's vector L1.
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_agent(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- RMSNorm ------------------------------------------------------------------
// y_i = h_i * w_i / sqrt(mean(h^2) + eps): sum of squares and the scaling in f64 as
// src/ops.rs:12-30, output rounded once.  One workgroup of 1024 threads; thread t
// handles elements 4t..4t+3 of each 4096-element pass (8 threads per 32-group, so the
// fused W4A8 quantization is a DPP reduction over 8 lanes).
// OUT: 0 -> bf16 y; 1 -> int8 xq + f32 group scales (nve_quantize_f16_q8 semantics).
template <int OUT>
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* __restrict__ h,
                                                       const uint16_t* __restrict__ w, float eps, int H,
                                                       uint16_t* __restrict__ y_bf16, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs) {
  __shared__ double red[16];
  double ss = 0.0;
  for (int i = threadIdx.x; i < H; i += 1024) {
    const double v = (double)h[i];
    ss += v * v;
  }
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x < 64) {
    double v = threadIdx.x < 16 ? red[threadIdx.x] : 0.0;
    for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
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
        for (int t = 0; t < 4; ++t) y_bf16[i0 + t] = f32_to_bf16_bits(v[t]);
    } else {
      q8_group8_store(v, ok, xq, xs, (size_t)(ok ? i0 : 0));
    }
  }
}

// ---- attention ------------------------------------------------------------------
// One launch per layer: RoPE on q and on the new key, KV-cache append, split-sequence
// softmax(q k^T / sqrt(D)) v over the cached keys, the cross-chunk combine, and the
// conversion of the attention output to the o_proj input (OUT 1: bf16, OUT 2: int8 +
// group-32 scales).
//
// grid (num_kv_heads, ceil(max_seq / KC)), 256 threads; chunks at or past pos + 1
// exit at once.  A workgroup stages its KC keys and values (bf16 rows of D) in LDS
// with every global load issued up front, computes the G = num_heads / num_kv_heads
// query heads of its kv head against them (4 or 8 threads per key for the scores,
// 2-dimension columns x key groups for the value sum), and writes a partial (running
// max m, sum l, unnormalised acc[D]) per query head.  The last workgroup of a kv
// head to finish (a device-scope counter, reset by that workgroup, so replays of a
// captured graph need no memset) combines the partials:
//   out[d] = sum_c e^(m_c - M) acc_c[d] / sum_c e^(m_c - M) l_c.
// The chunk holding pos rotates the new key, rounds key and value to bf16 like every
// cached entry, writes them to the cache and uses them from LDS.
template <int D, int OUT>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, const int* __restrict__ d_pos,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int num_heads, int num_kv_heads,
    int max_seq, float scale, float* __restrict__ part, int* __restrict__ counters,
    uint16_t* __restrict__ out_bf16, int8_t* __restrict__ out_q, float* __restrict__ out_s) {
  constexpr int NT = 256;
  constexpr int KC = attn_chunk(D);
  constexpr int HALF = D / 2;
  constexpr int G_MAX = 8;
  constexpr int ROW = D + 8;                 // padded LDS row, bf16 elements
  constexpr int U4_ROW = D / 8;              // 16-byte pieces per row
  constexpr int U4_T = KC * U4_ROW / NT;     // pieces per thread (2 or 4)
  constexpr int TPK = NT / KC;               // score threads per key (4 or 8)
  constexpr int DPT = D / TPK;               // dims per score thread (16 or 32)
  constexpr int DP = D / 2;                  // value columns (dimension pairs)
  constexpr int KG = NT / DP;                // key groups of the value sum
  constexpr int KPG = KC / KG;               // keys per key group
  static_assert(U4_T * NT == KC * U4_ROW && DPT % 8 == 0 && KG * DP == NT, "attention tiling");
  static_assert(2 * G_MAX * kAttnMaxChunks <= KG * G_MAX * D, "combine weights fit in s_red");

  __shared__ __align__(16) uint16_t s_k[KC * ROW];
  __shared__ __align__(16) uint16_t s_v[KC * ROW];
  __shared__ float s_q[G_MAX * D];
  __shared__ __align__(16) uint16_t s_knew[D];
  __shared__ __align__(16) uint16_t s_vnew[D];
  __shared__ float s_p[G_MAX][KC];
  __shared__ float s_ml[G_MAX][2];
  __shared__ int s_last;
  __shared__ float s_red[KG * G_MAX * D];  // value-sum partials of the key groups (16 KB)

  const int kvh = blockIdx.x;
  const int c = blockIdx.y;
  const int tid = threadIdx.x;
  // a position past the cache is clamped to its last slot (the host bounds the step
  // count; the clamp only keeps every access inside the cache and the RoPE tables)
  const int pos = min(max(*d_pos, 0), max_seq - 1);
  const int len = pos + 1;
  const int t0 = c * KC;
  if (t0 >= len) return;
  const int G = num_heads / num_kv_heads;
  const int nt = min(KC, len - t0);
  const int nchunk = (max_seq + KC - 1) / KC;
  const int used = (len + KC - 1) / KC;
  const size_t cache_base = (size_t)kvh * max_seq * D;
  const bool owner = pos < t0 + KC;  // this chunk holds the new token

  // 1. every K/V load of the tile in flight (rows past nt re-read row t0)
  uint4 rk[U4_T], rv[U4_T];
#pragma unroll
  for (int i = 0; i < U4_T; ++i) {
    const int piece = tid + i * NT;
    const int row = piece / U4_ROW, col = piece % U4_ROW;
    const size_t off = cache_base + (size_t)(t0 + (row < nt ? row : 0)) * D + col * 8;
    rk[i] = *(const uint4*)(kc + off);
    rv[i] = *(const uint4*)(vc + off);
  }
  // 2. rotated q of the G heads; the new key/value (owner)
  const float* cs = rope_cos + (size_t)pos * HALF;
  const float* sn = rope_sin + (size_t)pos * HALF;
  for (int idx = tid; idx < G * HALF; idx += NT) {
    const int g = idx / HALF, i = idx % HALF;
    const float* qh = q + (size_t)(kvh * G + g) * D;
    const float q0 = qh[i], q1 = qh[i + HALF];
    s_q[g * D + i] = q0 * cs[i] - q1 * sn[i];
    s_q[g * D + i + HALF] = q0 * sn[i] + q1 * cs[i];
  }
  if (owner) {
    const float* kh = k + (size_t)kvh * D;
    const float* vh = v + (size_t)kvh * D;
    uint16_t* kdst = kc + cache_base + (size_t)pos * D;
    uint16_t* vdst = vc + cache_base + (size_t)pos * D;
    for (int i = tid; i < HALF; i += NT) {
      const float k0 = kh[i], k1 = kh[i + HALF];
      const uint16_t r0 = f32_to_bf16_bits(k0 * cs[i] - k1 * sn[i]);
      const uint16_t r1 = f32_to_bf16_bits(k0 * sn[i] + k1 * cs[i]);
      s_knew[i] = r0;
      s_knew[i + HALF] = r1;
      kdst[i] = r0;
      kdst[i + HALF] = r1;
    }
    for (int i = tid; i < D; i += NT) {
      const uint16_t r = f32_to_bf16_bits(vh[i]);
      s_vnew[i] = r;
      vdst[i] = r;
    }
  }
  lds_barrier();
  // 3. tile to LDS (the row of pos from the freshly rounded key/value)
  const int prow = owner ? pos - t0 : -1;
#pragma unroll
  for (int i = 0; i < U4_T; ++i) {
    const int piece = tid + i * NT;
    const int row = piece / U4_ROW, col = piece % U4_ROW;
    uint4 a = rk[i], b = rv[i];
    if (row == prow) {
      a = *(const uint4*)(s_knew + col * 8);
      b = *(const uint4*)(s_vnew + col * 8);
    }
    *(uint4*)(s_k + row * ROW + col * 8) = a;
    *(uint4*)(s_v + row * ROW + col * 8) = b;
  }
  lds_barrier();
  // 4. scores: TPK threads per key, DPT dims each
  {
    const int j = tid / TPK, r = tid % TPK;
    float sc[G_MAX];
#pragma unroll
    for (int g = 0; g < G_MAX; ++g) sc[g] = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < DPT; d0 += 8) {
      const uint4 raw = *(const uint4*)(s_k + j * ROW + r * DPT + d0);
      const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int u2 = 0; u2 < 4; ++u2) {
        const float ka = bf16_bits_to_f32(wv[u2] & 0xffffu), kb = bf16_bits_to_f32(wv[u2] >> 16);
        const int dd = r * DPT + d0 + 2 * u2;
#pragma unroll
        for (int g = 0; g < G_MAX; ++g)
          if (g < G) sc[g] = fmaf(s_q[g * D + dd + 1], kb, fmaf(s_q[g * D + dd], ka, sc[g]));
      }
    }
#pragma unroll
    for (int g = 0; g < G_MAX; ++g) {
      if (g >= G) break;
      float s = sc[g];
#pragma unroll
      for (int off = 1; off < TPK; off <<= 1) s += __shfl_xor(s, off, 64);
      if (r == 0) s_p[g][j] = j < nt ? s * scale : -INFINITY;
    }
  }
  lds_barrier();
  // 5. chunk softmax statistics (wave 0; lane = key)
  if (tid < 64) {
    for (int g = 0; g < G; ++g) {
      const float s = tid < KC ? s_p[g][tid] : -INFINITY;
      float m = s;
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      const float p = s == -INFINITY ? 0.0f : expf(s - m);
      float l = p;
      for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
      if (tid < KC) s_p[g][tid] = p;
      if (tid == 0) {
        s_ml[g][0] = m;
        s_ml[g][1] = l;
      }
    }
  }
  lds_barrier();
  // 6. value sum: column pair dp, key group kg
  {
    const int dp = tid % DP, kg = tid / DP;
    float a0[G_MAX], a1[G_MAX];
#pragma unroll
    for (int g = 0; g < G_MAX; ++g) a0[g] = a1[g] = 0.0f;
#pragma unroll 4
    for (int jj = 0; jj < KPG; ++jj) {
      const int j = kg * KPG + jj;
      const uint32_t w2 = *(const uint32_t*)(s_v + j * ROW + 2 * dp);
      const float va = bf16_bits_to_f32(w2 & 0xffffu), vb = bf16_bits_to_f32(w2 >> 16);
#pragma unroll
      for (int g = 0; g < G_MAX; ++g)
        if (g < G) {
          const float p = s_p[g][j];
          a0[g] = fmaf(p, va, a0[g]);
          a1[g] = fmaf(p, vb, a1[g]);
        }
    }
#pragma unroll
    for (int g = 0; g < G_MAX; ++g)
      if (g < G) {
        s_red[(kg * G_MAX + g) * D + 2 * dp] = a0[g];
        s_red[(kg * G_MAX + g) * D + 2 * dp + 1] = a1[g];
      }
  }
  lds_barrier();
  // 7. partials to global, then the per-kv-head arrival counter
  for (int idx = tid; idx < G * D; idx += NT) {
    const int g = idx / D, d = idx % D;
    float a = 0.0f;
#pragma unroll
    for (int kg = 0; kg < KG; ++kg) a += s_red[(kg * G_MAX + g) * D + d];
    float* pp = part + ((size_t)(kvh * G + g) * nchunk + c) * (D + 2);
    pp[2 + d] = a;
    if (d == 0) {
      pp[0] = s_ml[g][0];
      pp[1] = s_ml[g][1];
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&counters[kvh], 1) == used - 1;
  __syncthreads();
  if (!s_last) return;
  // 8. last workgroup of this kv head: combine its G heads and emit the o_proj input.
  // Chunk statistics first (one thread per (head, chunk), all loads in flight), then
  // per-chunk weights f_c = e^(m_c - M) / sum_c' e^(m_c' - M) l_c' in LDS, then the
  // weighted sum of the partial accumulators (loads unrolled by 4).
  __threadfence();
  if (tid == 0) atomicExch(&counters[kvh], 0);
  float* s_f = s_red;  // [G][used] chunk weights, then [G][used] f*l (the value-sum partials are consumed)
  const int ncomb = used;  // <= kAttnMaxChunks (host check): 2 * G * ncomb fits in s_red
  for (int idx = tid; idx < G * ncomb; idx += NT) {
    const int g = idx / ncomb, cc = idx % ncomb;
    const float* p = part + ((size_t)(kvh * G + g) * nchunk + cc) * (D + 2);
    s_f[g * ncomb + cc] = ld_agent(p);
  }
  __syncthreads();
  if (tid < G) {
    const int g = tid;
    float M = -INFINITY;
    for (int cc = 0; cc < ncomb; ++cc) M = fmaxf(M, s_f[g * ncomb + cc]);
    s_ml[g][0] = M;
  }
  __syncthreads();
  for (int idx = tid; idx < G * ncomb; idx += NT) {
    const int g = idx / ncomb, cc = idx % ncomb;
    const float* p = part + ((size_t)(kvh * G + g) * nchunk + cc) * (D + 2);
    const float f = expf(s_f[g * ncomb + cc] - s_ml[g][0]);
    s_f[g * ncomb + cc] = f;
    s_red[G * ncomb + g * ncomb + cc] = f * ld_agent(p + 1);
  }
  __syncthreads();
  if (tid < G) {
    const int g = tid;
    float L = 0.0f;
    for (int cc = 0; cc < ncomb; ++cc) L += s_red[G * ncomb + g * ncomb + cc];
    s_ml[g][1] = 1.0f / L;
  }
  __syncthreads();
  for (int e0 = 4 * tid; e0 < G * D; e0 += 4 * NT) {  // G*D % 32 == 0: 8-lane groups stay whole
    const int g = e0 / D, d = e0 % D;
    const float* pb = part + (size_t)(kvh * G + g) * nchunk * (D + 2) + 2 + d;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int cc = 0;
    for (; cc + 4 <= ncomb; cc += 4) {
      float4 x[4];
#pragma unroll
      for (int u2 = 0; u2 < 4; ++u2) {
        const float* p = pb + (size_t)(cc + u2) * (D + 2);
        x[u2] = make_float4(ld_agent(p), ld_agent(p + 1), ld_agent(p + 2), ld_agent(p + 3));
      }
#pragma unroll
      for (int u2 = 0; u2 < 4; ++u2) {
        const float f = s_f[g * ncomb + cc + u2];
        o[0] = fmaf(f, x[u2].x, o[0]);
        o[1] = fmaf(f, x[u2].y, o[1]);
        o[2] = fmaf(f, x[u2].z, o[2]);
        o[3] = fmaf(f, x[u2].w, o[3]);
      }
    }
    for (; cc < ncomb; ++cc) {
      const float* p = pb + (size_t)cc * (D + 2);
      const float f = s_f[g * ncomb + cc];
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = fmaf(f, ld_agent(p + t), o[t]);
    }
    const float invL = s_ml[g][1];
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] *= invL;
    const size_t i0 = (size_t)(kvh * G + g) * D + d;
    if (OUT == 1) {
#pragma unroll
      for (int t = 0; t < 4; ++t) out_bf16[i0 + t] = f32_to_bf16_bits(o[t]);
    } else {
      q8_group8_store(o, true, out_q, out_s, i0);
    }
  }
}

// Single-pass variant: one workgroup per query head streams every cached key of its
// kv head through LDS in tiles of KT with an online softmax (running max / sum,
// accumulator rescaled per tile) -- no cross-workgroup combine, so no device-scope
// fences.  The next tile's K/V loads are issued before the current tile is computed.
// The workgroup of the kv head's first query head writes the new key/value to the
// cache; the others use their own identical copy for that row.
template <int D, int OUT>
__global__ __launch_bounds__(256) void attn_single_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, const int* __restrict__ d_pos,
    const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, int num_heads, int num_kv_heads,
    int max_seq, float scale, uint16_t* __restrict__ out_bf16, int8_t* __restrict__ out_q,
    float* __restrict__ out_s) {
  constexpr int NT = 256;
  constexpr int KT = attn_chunk(D);
  constexpr int HALF = D / 2;
  constexpr int ROW = D + 8;
  constexpr int U4_ROW = D / 8;
  constexpr int U4_T = KT * U4_ROW / NT;
  constexpr int TPK = NT / KT;
  constexpr int DPT = D / TPK;
  constexpr int DP = D / 2;
  constexpr int KG = NT / DP;
  constexpr int KPG = KT / KG;
  static_assert(U4_T * NT == KT * U4_ROW && DPT % 8 == 0 && KG * DP == NT, "attention tiling");

  __shared__ __align__(16) uint16_t s_k[KT * ROW];
  __shared__ __align__(16) uint16_t s_v[KT * ROW];
  __shared__ float s_q[D];
  __shared__ __align__(16) uint16_t s_knew[D];
  __shared__ __align__(16) uint16_t s_vnew[D];
  __shared__ float s_p[KT];
  __shared__ float s_wm[NT / 64];
  __shared__ float s_wl[NT / 64];
  __shared__ float s_red[KG * D];

  const int hq = blockIdx.x;
  const int G = num_heads / num_kv_heads;
  const int kvh = hq / G;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int pos = min(max(*d_pos, 0), max_seq - 1);  // clamped like the split kernel
  const int len = pos + 1;
  const int ntiles = (len + KT - 1) / KT;
  const size_t cache_base = (size_t)kvh * max_seq * D;

  uint4 rk[U4_T], rv[U4_T];
  auto issue = [&](int t) {
    const int t0 = t * KT;
#pragma unroll
    for (int i = 0; i < U4_T; ++i) {
      const int piece = tid + i * NT;
      const int row = piece / U4_ROW, col = piece % U4_ROW;
      const int tr = t0 + row < len ? t0 + row : t0;
      const size_t off = cache_base + (size_t)tr * D + col * 8;
      rk[i] = *(const uint4*)(kc + off);
      rv[i] = *(const uint4*)(vc + off);
    }
  };
  issue(0);

  const float* cs = rope_cos + (size_t)pos * HALF;
  const float* sn = rope_sin + (size_t)pos * HALF;
  for (int i = tid; i < HALF; i += NT) {
    const float* qh = q + (size_t)hq * D;
    const float q0 = qh[i], q1 = qh[i + HALF];
    s_q[i] = q0 * cs[i] - q1 * sn[i];
    s_q[i + HALF] = q0 * sn[i] + q1 * cs[i];
    const float* kh = k + (size_t)kvh * D;
    const float k0 = kh[i], k1 = kh[i + HALF];
    s_knew[i] = f32_to_bf16_bits(k0 * cs[i] - k1 * sn[i]);
    s_knew[i + HALF] = f32_to_bf16_bits(k0 * sn[i] + k1 * cs[i]);
  }
  for (int i = tid; i < D; i += NT) s_vnew[i] = f32_to_bf16_bits(v[(size_t)kvh * D + i]);
  lds_barrier();
  if (hq % G == 0)
    for (int i = tid; i < D; i += NT) {
      kc[cache_base + (size_t)pos * D + i] = s_knew[i];
      vc[cache_base + (size_t)pos * D + i] = s_vnew[i];
    }

  float m_run = -INFINITY, l_run = 0.0f;
  const int dp = tid % DP, kg = tid / DP;
  float a0 = 0.0f, a1 = 0.0f;
  const int j = tid / TPK, r = tid % TPK;
  for (int t = 0; t < ntiles; ++t) {
    const int t0 = t * KT;
    const int prow = pos - t0;  // row of the new token in this tile (if < KT)
#pragma unroll
    for (int i = 0; i < U4_T; ++i) {
      const int piece = tid + i * NT;
      const int row = piece / U4_ROW, col = piece % U4_ROW;
      uint4 a = rk[i], b = rv[i];
      if (row == prow) {
        a = *(const uint4*)(s_knew + col * 8);
        b = *(const uint4*)(s_vnew + col * 8);
      }
      *(uint4*)(s_k + row * ROW + col * 8) = a;
      *(uint4*)(s_v + row * ROW + col * 8) = b;
    }
    lds_barrier();
    if (t + 1 < ntiles) issue(t + 1);
    // scores
    float s = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < DPT; d0 += 8) {
      const uint4 raw = *(const uint4*)(s_k + j * ROW + r * DPT + d0);
      const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int u2 = 0; u2 < 4; ++u2) {
        const int dd = r * DPT + d0 + 2 * u2;
        s = fmaf(s_q[dd + 1], bf16_bits_to_f32(wv[u2] >> 16), fmaf(s_q[dd], bf16_bits_to_f32(wv[u2] & 0xffffu), s));
      }
    }
#pragma unroll
    for (int off = 1; off < TPK; off <<= 1) s += __shfl_xor(s, off, 64);
    const bool valid = t0 + j < len;
    s = valid ? s * scale : -INFINITY;
    float mw = s;
    for (int off = 32; off > 0; off >>= 1) mw = fmaxf(mw, __shfl_xor(mw, off, 64));
    if ((tid & 63) == 0) s_wm[wave] = mw;
    lds_barrier();
    float m_tile = s_wm[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) m_tile = fmaxf(m_tile, s_wm[w]);
    const float m_new = fmaxf(m_run, m_tile);
    const float p = valid ? expf(s - m_new) : 0.0f;
    if (r == 0) s_p[j] = p;
    float lw = r == 0 ? p : 0.0f;
    for (int off = 32; off > 0; off >>= 1) lw += __shfl_xor(lw, off, 64);
    if ((tid & 63) == 0) s_wl[wave] = lw;
    lds_barrier();
    const float alpha = expf(m_run - m_new);  // 0 on the first tile
    float lt = s_wl[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) lt += s_wl[w];
    l_run = fmaf(l_run, alpha, lt);
    a0 *= alpha;
    a1 *= alpha;
#pragma unroll 4
    for (int jj = 0; jj < KPG; ++jj) {
      const int jv = kg * KPG + jj;
      const uint32_t w2 = *(const uint32_t*)(s_v + jv * ROW + 2 * dp);
      const float pv = s_p[jv];
      a0 = fmaf(pv, bf16_bits_to_f32(w2 & 0xffffu), a0);
      a1 = fmaf(pv, bf16_bits_to_f32(w2 >> 16), a1);
    }
    m_run = m_new;
    lds_barrier();  // tile buffers, s_p and s_wm / s_wl are rewritten next
  }
  s_red[kg * D + 2 * dp] = a0;
  s_red[kg * D + 2 * dp + 1] = a1;
  lds_barrier();
  if (tid < D / 4) {
    const float invL = 1.0f / l_run;
    float o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float a = 0.0f;
#pragma unroll
      for (int g2 = 0; g2 < KG; ++g2) a += s_red[g2 * D + 4 * tid + t];
      o[t] = a * invL;
    }
    const size_t i0 = (size_t)hq * D + 4 * tid;
    if (OUT == 1) {
#pragma unroll
      for (int t = 0; t < 4; ++t) out_bf16[i0 + t] = f32_to_bf16_bits(o[t]);
    } else {
      q8_group8_store(o, true, out_q, out_s, i0);
    }
  }
}

// ---- SiLU * up ------------------------------------------------------------------
// mid = silu(gate) * up (src/ops.rs:62-64: g / (1 + exp(-g))).  OUT 0 -> bf16,
// 1 -> int8 + group scales (fused W4A8 quantization; 8 lanes per 32-group).
template <int OUT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                       int F, uint16_t* __restrict__ y_bf16, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs) {
  const int i0 = 4 * ((int)blockIdx.x * 256 + (int)threadIdx.x);
  const bool ok = i0 < F;  // F % 32 == 0
  const int ib = ok ? i0 : 0;
  const float4 g4 = *(const float4*)(gate + ib);
  const float4 u4 = *(const float4*)(up + ib);
  const float gg[4] = {g4.x, g4.y, g4.z, g4.w}, uu[4] = {u4.x, u4.y, u4.z, u4.w};
  float v[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) v[t] = gg[t] / (1.0f + expf(-gg[t])) * uu[t];
  if (OUT == 0) {
    if (ok)
#pragma unroll
      for (int t = 0; t < 4; ++t) y_bf16[i0 + t] = f32_to_bf16_bits(v[t]);
  } else {
    q8_group8_store(v, ok, xq, xs, (size_t)ib);
  }
}

// ---- head: greedy argmax (first maximum), next-token embedding, position advance --
// grid kArgmaxBlocks x 256: each workgroup reduces a slice of the logits to (value,
// index); the last to arrive (device-scope counter, reset by it) reduces the partials,
// writes the token, embeds its row into hidden and advances the position.  NaN never
// wins; among equal values the lowest index wins (src/ops.rs:485-495 keeps the first
// maximum).
constexpr int kArgmaxBlocks = 128;

__device__ __forceinline__ void argmax_merge(float& b, int& bi, float o, int oi) {
  if (o > b || (o == b && oi < bi)) {
    b = o;
    bi = oi;
  }
}

__device__ __forceinline__ void argmax_block(float& best, int& bi, float* s_v, int* s_i) {
  for (int off = 32; off > 0; off >>= 1) argmax_merge(best, bi, __shfl_xor(best, off, 64), __shfl_xor(bi, off, 64));
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = best;
    s_i[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < 4; ++w) argmax_merge(best, bi, s_v[w], s_i[w]);
}

__global__ __launch_bounds__(256) void argmax_embed_kernel(const float* __restrict__ logits, int V,
                                                           const uint16_t* __restrict__ embed, int H,
                                                           float* __restrict__ hidden, int* __restrict__ token_out,
                                                           int* __restrict__ d_pos, float* __restrict__ part_v,
                                                           int* __restrict__ part_i, int* __restrict__ counter) {
  __shared__ float s_v[4];
  __shared__ int s_i[4];
  __shared__ int s_last;
  __shared__ int s_tok;
  const int per = (V + kArgmaxBlocks - 1) / kArgmaxBlocks;
  const int lo = blockIdx.x * per, hi = min(V, lo + per);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = lo + threadIdx.x; i < hi; i += 256) argmax_merge(best, bi, logits[i], i);
  argmax_block(best, bi, s_v, s_i);
  if (threadIdx.x == 0) {
    part_v[blockIdx.x] = best;
    part_i[blockIdx.x] = bi;
    __threadfence();
    s_last = atomicAdd(counter, 1) == kArgmaxBlocks - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  best = -INFINITY;
  bi = 0x7fffffff;
  if (threadIdx.x < kArgmaxBlocks) {
    best = ld_agent(part_v + threadIdx.x);
    bi = ld_agent(part_i + threadIdx.x);
  }
  __syncthreads();  // s_v / s_i reuse
  argmax_block(best, bi, s_v, s_i);
  if (threadIdx.x == 0) {
    if (bi == 0x7fffffff) bi = 0;  // all NaN / -inf: token 0
    s_tok = bi;
    *token_out = bi;
    atomicExch(counter, 0);
  }
  __syncthreads();
  const int tok = s_tok;
  for (int i = threadIdx.x; i < H; i += 256) hidden[i] = bf16_bits_to_f32(embed[(size_t)tok * H + i]);
  if (threadIdx.x == 0) *d_pos += 1;
}

__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ embed, const int* __restrict__ token,
                                                    float* __restrict__ hidden, int H) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < H) hidden[i] = bf16_bits_to_f32(embed[(size_t)(*token) * H + i]);
}

}  // namespace nve

// ---------------------------------------------------------------------------
// Host side: workspace layout and the per-layer / head orchestration.
// ---------------------------------------------------------------------------
namespace nve_host {

struct DecodeWs {
  int* counters;       // [num_kv_heads] attention arrival counters, then [1] argmax (zero at rest)
  uint16_t* act_bf16;  // [max(H, Hq*D, F)]
  int8_t* xq;          // [max(H, Hq*D, F)]
  float* xs;           // [max/32]
  float* q;            // [Hq*D]
  float* k;            // [Hkv*D]
  float* v;            // [Hkv*D]
  float* part;         // [Hq * nchunk * (D+2)] attention partials
  float* gate;         // [F]
  float* up;           // [F]
  float* arg_v;        // [kArgmaxBlocks]
  int* arg_i;          // [kArgmaxBlocks]
  float* logits;       // [V] (head only, when the caller passes no logits buffer)
  size_t bytes;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int attn_nchunk(const nve_decode_config& c) {
  const int kc = nve::attn_chunk(c.head_dim);
  return (c.max_seq + kc - 1) / kc;
}

static DecodeWs layout_ws(const nve_decode_config& c, void* base) {
  DecodeWs w{};
  const size_t qd = (size_t)c.num_heads * c.head_dim, kd = (size_t)c.num_kv_heads * c.head_dim;
  size_t mx = (size_t)c.hidden;
  if (qd > mx) mx = qd;
  if ((size_t)c.ffn > mx) mx = c.ffn;
  const size_t nchunk = attn_nchunk(c);
  char* p = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  w.counters = (int*)take(((size_t)c.num_kv_heads + 1) * 4);
  w.act_bf16 = (uint16_t*)take(mx * 2);
  w.xq = (int8_t*)take(mx);
  w.xs = (float*)take(mx / 32 * 4);
  w.q = (float*)take(qd * 4);
  w.k = (float*)take(kd * 4);
  w.v = (float*)take(kd * 4);
  w.part = (float*)take((size_t)c.num_heads * nchunk * (c.head_dim + 2) * 4);
  w.gate = (float*)take((size_t)c.ffn * 4);
  w.up = (float*)take((size_t)c.ffn * 4);
  w.arg_v = (float*)take(nve::kArgmaxBlocks * 4);
  w.arg_i = (int*)take(nve::kArgmaxBlocks * 4);
  w.logits = (float*)take((size_t)(c.vocab > 0 ? c.vocab : 1) * 4);
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
      attn_nchunk(c) > nve::kAttnMaxChunks)
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
    hipLaunchKernelGGL(nve::rmsnorm_kernel<0>, dim3(1), dim3(1024), 0, s, h, w, c.eps, c.hidden, ws.act_bf16,
                       nullptr, nullptr);
  return hipGetLastError();
}

// Longest cache served by the single-pass attention kernel; longer caches use the
// split-sequence kernel.
constexpr int kAttnSinglePassMax = 8192;

static hipError_t launch_attention(const nve_decode_config& c, const nve_decode_io& io, const DecodeWs& ws,
                                   bool w4a8, hipStream_t s) {
  const float scale = 1.0f / sqrtf((float)c.head_dim);
  const bool single = c.max_seq <= kAttnSinglePassMax;
  const dim3 grid(c.num_kv_heads, attn_nchunk(c));
#define NVE_ATTN(D, OUT)                                                                                         \
  if (single)                                                                                                    \
    hipLaunchKernelGGL((nve::attn_single_kernel<D, OUT>), dim3(c.num_heads), dim3(256), 0, s, ws.q, ws.k, ws.v,  \
                       io.k_cache, io.v_cache, io.pos, io.rope_cos, io.rope_sin, c.num_heads, c.num_kv_heads,   \
                       c.max_seq, scale, ws.act_bf16, ws.xq, ws.xs);                                            \
  else                                                                                                           \
    hipLaunchKernelGGL((nve::attn_decode_kernel<D, OUT>), grid, dim3(256), 0, s, ws.q, ws.k, ws.v, io.k_cache,   \
                       io.v_cache, io.pos, io.rope_cos, io.rope_sin, c.num_heads, c.num_kv_heads, c.max_seq,    \
                       scale, ws.part, ws.counters, ws.act_bf16, ws.xq, ws.xs)
  if (c.head_dim == 64) {
    if (w4a8) NVE_ATTN(64, 2); else NVE_ATTN(64, 1);
  } else if (c.head_dim == 128) {
    if (w4a8) NVE_ATTN(128, 2); else NVE_ATTN(128, 1);
  } else {
    if (w4a8) NVE_ATTN(256, 2); else NVE_ATTN(256, 1);
  }
#undef NVE_ATTN
  return hipGetLastError();
}

int layer_forward_decode(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io,
                         bool w4a8, hipStream_t s) {
  const DecodeWs ws = layout_ws(c, io.workspace);
  const int H = c.hidden, F = c.ffn, QD = c.num_heads * c.head_dim;
  // attention sub-layer: norm -> Q/K/V (one grouped launch) -> attention -> o_proj (+h)
  NVE_TRY(launch_rmsnorm(c, io.hidden, w.input_norm, w4a8, ws, s));
  {
    const nve_w4_weight qkv[3] = {w.q, w.k, w.v};
    void* outs[3] = {ws.q, ws.k, ws.v};
    const W4Segs sg = segs3(qkv, outs, 3);
    if (w4a8)
      NVE_TRY(launch_w4a8(ws.xq, ws.xs, sg, NVE_DT_F32, H, s));
    else
      NVE_TRY(launch_w4a16(ws.act_bf16, NVE_DT_BF16, sg, NVE_DT_F32, H, s));
  }
  // attention writes the o_proj input directly (int8 + scales, or bf16)
  NVE_TRY(launch_attention(c, io, ws, w4a8, s));
  if (w4a8)
    NVE_TRY(launch_w4a8(ws.xq, ws.xs, one_seg(w.o, io.hidden), NVE_DT_F32_ACCUM, QD, s));
  else
    NVE_TRY(launch_w4a16(ws.act_bf16, NVE_DT_BF16, one_seg(w.o, io.hidden), NVE_DT_F32_ACCUM, QD, s));
  // FFN sub-layer: norm -> gate/up (one grouped launch) -> silu*up -> down (+h)
  NVE_TRY(launch_rmsnorm(c, io.hidden, w.post_attn_norm, w4a8, ws, s));
  {
    const nve_w4_weight gu[2] = {w.gate, w.up};
    void* outs[2] = {ws.gate, ws.up};
    const W4Segs sg = segs3(gu, outs, 2);
    if (w4a8)
      NVE_TRY(launch_w4a8(ws.xq, ws.xs, sg, NVE_DT_F32, H, s));
    else
      NVE_TRY(launch_w4a16(ws.act_bf16, NVE_DT_BF16, sg, NVE_DT_F32, H, s));
  }
  const dim3 sgrid((F / 4 + 255) / 256);
  if (w4a8) {
    hipLaunchKernelGGL(nve::silu_mul_kernel<1>, sgrid, dim3(256), 0, s, ws.gate, ws.up, F, nullptr, ws.xq, ws.xs);
    NVE_TRY(hipGetLastError());
    NVE_TRY(launch_w4a8(ws.xq, ws.xs, one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
  } else {
    hipLaunchKernelGGL(nve::silu_mul_kernel<0>, sgrid, dim3(256), 0, s, ws.gate, ws.up, F, ws.act_bf16, nullptr,
                       nullptr);
    NVE_TRY(hipGetLastError());
    NVE_TRY(launch_w4a16(ws.act_bf16, NVE_DT_BF16, one_seg(w.down, io.hidden), NVE_DT_F32_ACCUM, F, s));
  }
  return NVE_OK;
}

int decode_head(const nve_decode_config& c, const nve_decode_head& hd, bool w4a8, hipStream_t s) {
  const DecodeWs ws = layout_ws(c, hd.workspace);
  NVE_TRY(launch_rmsnorm(c, hd.hidden, hd.final_norm, w4a8, ws, s));
  float* logits = hd.logits ? hd.logits : ws.logits;
  if (w4a8)
    NVE_TRY(launch_w4a8(ws.xq, ws.xs, one_seg(hd.lm_head, logits), NVE_DT_F32, c.hidden, s));
  else
    NVE_TRY(launch_w4a16(ws.act_bf16, NVE_DT_BF16, one_seg(hd.lm_head, logits), NVE_DT_F32, c.hidden, s));
  hipLaunchKernelGGL(nve::argmax_embed_kernel, dim3(nve::kArgmaxBlocks), dim3(256), 0, s, logits, hd.lm_head.n,
                     hd.embed, c.hidden, hd.hidden, hd.token_out, hd.pos, ws.arg_v, ws.arg_i,
                     ws.counters + c.num_kv_heads);
  return (int)hipGetLastError();
}

hipError_t launch_embed(const uint16_t* embed, const int* token, float* hidden, int H, hipStream_t s) {
  hipLaunchKernelGGL(nve::embed_kernel, dim3((H + 255) / 256), dim3(256), 0, s, embed, token, hidden, H);
  return hipGetLastError();
}

int check_decode(const nve_decode_config& c) { return check_cfg(c); }

}  // namespace nve_host
