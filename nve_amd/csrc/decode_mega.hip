// decode_mega.hip -- one decoder layer of the decode step as ONE persistent kernel.
//
// The five-launch layer (decode.hip: Q/K/V, attention, o_proj, gate/up, down) pays a
// kernel boundary and a cold start per launch: the next launch's weight loads cannot
// be issued before the previous launch has drained, so every sub-layer waits for its
// first HBM bytes after the boundary.  Here one workgroup per CU (8 compute waves plus
// one control wave) runs all five phases of the layer, and the phases are separated by
// a grid barrier instead of a launch.  Weights do not depend on the activations, so
// each phase's weight loads are issued BEFORE the barrier that precedes the phase and
// stream in while the barrier completes; only the activation hand-off (a few KB per
// workgroup) waits for it.  The arithmetic of every phase is that of the five-launch
// path (same block dot products, same producers, same attention and merge).
//
// Grid barrier (hierarchical, sense-reversing, counters at rest are zero): the control
// wave of each workgroup adds one to its XCD's counter (workgroups are dealt to the 8
// XCDs round-robin, so XCD = blockIdx % 8); the last arriver of an XCD resets the
// counter and adds one to the global counter; the last XCD resets that and bumps the
// global generation; each XCD's last arriver then bumps its XCD generation, which the
// other workgroups of the XCD poll.  A flat counter polled by every workgroup costs
// about twice as much on this part (measured).  Spins are bounded; a spin that gives up
// sets an error word in the workspace and the kernel finishes (with wrong results)
// instead of hanging.
//
// Coherence: data passed between workgroups in a phase hand-off is stored with
// agent-scope (write-through, sc1) stores whose completion the storing wave waits for
// before its workgroup arrives at the barrier; the consumers read it with plain loads,
// which is correct because every such buffer is written once per launch and not read
// before the barrier that follows its writes (so no XCD's L2 can hold a stale copy):
// q/k/v, the attention partials, h_mid (the residual after the attention sub-layer,
// kept apart from h, which every workgroup reads at the start) and mid.
//
// The kernel needs every workgroup resident at once (one per CU); the host launches it
// only with grid = CU count and falls back to the five-launch path where the shapes do
// not fit its register tiling.
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <set>
#include <utility>

#include "common.h"
#include "act_producer.h"
#include "w4_launch.h"
#include "w4a16_ops.h"
#include "w4a8_ops.h"
#include "decode_mega.h"

namespace nve {
namespace mega {

constexpr int NW = 8;           // compute waves per workgroup
constexpr int NT = NW * 64;     // compute threads
constexpr int kThreads = NT + 64;  // + the control wave
constexpr int kWord = 64;       // barrier words are 256 B apart
constexpr int kBarWords = 20;   // [0,8) XCD counters, [8,16) XCD generations, 16 global counter,
                                // 17 global generation, 18 error word
constexpr long kSpinLimit = 20000;  // polls of about 1 us: a barrier gives up after ~20 ms


// ---- coherent hand-off stores and the grid barrier ----------------------------------
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coh(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void spin_while_eq(unsigned* p, unsigned v, unsigned* err) {
  for (long i = 0; ld_coh(p) == v; ++i) {
    if (i > kSpinLimit) {
      __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Lane 0 of the control wave; every compute wave's hand-off stores have completed.
__device__ void grid_arrive_wait(unsigned* bar, int per_xcd) {
  const int x = blockIdx.x & 7;
  unsigned* xcnt = bar + x * kWord;
  unsigned* xgen = bar + (8 + x) * kWord;
  unsigned* gcnt = bar + 16 * kWord;
  unsigned* ggen = bar + 17 * kWord;
  unsigned* err = bar + 18 * kWord;
  // the generation is read before arriving (it cannot move until this workgroup has
  // arrived), and the read completes before the arrival is issued
  const unsigned g0 = ld_coh(xgen);
  wait_mem();
  const unsigned old = __hip_atomic_fetch_add(xcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old + 1 == (unsigned)per_xcd) {
    __hip_atomic_store(xcnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned G0 = ld_coh(ggen);
    wait_mem();
    const unsigned o2 = __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (o2 + 1 == 8u) {
      __hip_atomic_store(gcnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_mem();
      __hip_atomic_fetch_add(ggen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      spin_while_eq(ggen, G0, err);
    }
    wait_mem();
    __hip_atomic_fetch_add(xgen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    spin_while_eq(xgen, g0, err);
  }
  wait_mem();
}

// Whole-workgroup grid barrier in two halves, both called by all 9 waves.
// grid_sync_arrive: compute waves have waited for their hand-off stores (wait_mem);
// after the LDS barrier the control wave arrives and waits for the grid while the
// compute waves go on to issue the next phase's weight loads (issuing them takes about
// as long as they take to stream in: the load queues are bounded, so issuing them
// before the arrival would delay the whole grid).  grid_sync_wait: the second LDS
// barrier, which the control wave reaches once the grid has arrived; the compute
// waves' loads stay in flight across it (it waits only for LDS traffic).
__device__ __forceinline__ void grid_sync_arrive(unsigned* bar, int per_xcd) {
  lds_barrier();
  if (threadIdx.x == NT) grid_arrive_wait(bar, per_xcd);
}
__device__ __forceinline__ void grid_sync_wait() { lds_barrier(); }

// ---- weights of one GEMV phase: R rows per wave, NJ 64-block chunks per lane ---------
struct Mats {
  // matrices concatenated by rows (SWI: gate in 0, up in 1, paired); named members, not
  // arrays, so the row -> matrix selection stays a scalar select
  const uint8_t *nib0, *nib1, *nib2;
  const float *sc0, *sc1, *sc2;
  int n0, n1, count;
};

template <int R, int NJ>
struct WBuf {
  uint4 w[R][NJ];
  float s[R][NJ];
};

// Row g of the concatenation -> (matrix, row); g < total.
__device__ __forceinline__ int mat_of(const Mats& m, int g, int& row) {
  if (m.count > 1 && g >= m.n0) {
    if (m.count > 2 && g >= m.n0 + m.n1) {
      row = g - m.n0 - m.n1;
      return 2;
    }
    row = g - m.n0;
    return 1;
  }
  row = g;
  return 0;
}

template <int R, int NJ, bool SWI>
__device__ __forceinline__ void issue_weights(WBuf<R, NJ>& b, const Mats& m, int g0, int total, int K, int lane) {
  constexpr int RH = SWI ? R / 2 : R;
  const int nb = K >> 5;
  const size_t row_bytes = (size_t)(K >> 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    int row;
    int mi;
    if (SWI) {
      row = min(g0 + r % RH, total - 1);
      mi = r < RH ? 0 : 1;
    } else {
      mi = mat_of(m, min(g0 + r, total - 1), row);
    }
    // the selected pointer is formed as matrix 0's pointer plus a scalar byte offset: a
    // select of the three pointers is turned into an indexed load from a stack copy of
    // the struct, and a pointer rebuilt from an integer loses its global address space
    const intptr_t dn = ((intptr_t)m.nib1 - (intptr_t)m.nib0) * (mi == 1) + ((intptr_t)m.nib2 - (intptr_t)m.nib0) * (mi == 2);
    const intptr_t ds = ((intptr_t)m.sc1 - (intptr_t)m.sc0) * (mi == 1) + ((intptr_t)m.sc2 - (intptr_t)m.sc0) * (mi == 2);
    const uint8_t* nib = m.nib0 + dn;
    const float* sc = (const float*)((const char*)m.sc0 + ds);
    const uint4* rn = (const uint4*)(nib + (size_t)row * row_bytes);
    const float* rs = sc + (size_t)row * nb;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bb = min(lane + 64 * j, nb - 1);
      b.w[r][j] = ld_stream(rn + bb);
      b.s[r][j] = ld_stream(rs + bb);
    }
  }
}

// ---- activation staging (compute threads; SPT passes of NT chunks) --------------------
// f64 sum of squares over the workgroup, fixed order: thread partials, wave butterfly,
// then the NW wave sums in order.
template <int SRC, int E, int SPT>
__device__ __forceinline__ double stage_sumsq(const ProdChunk<SRC, E> (&pc)[SPT], int nchunk) {
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < SPT; ++s) {
    const bool ok = (int)threadIdx.x + NT * s < nchunk;
#pragma unroll
    for (int t = 0; t < E / 4; ++t) {
      const float4 v = pc[s].a[t];
      const double q = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
      ss += ok ? q : 0.0;
    }
  }
  return group_sum_f64<64>(ss);
}

template <bool W4A8>
__host__ __device__ constexpr size_t stage_bytes(int K) {
  return W4A8 ? w4a8_lds_bytes(K) : w4a16_lds_bytes(MODE_F16, K);
}

// Issue the staging loads of one phase (compute waves).
template <int SRC, int E, int SPT>
__device__ __forceinline__ void stage_issue(ProdChunk<SRC, E> (&pc)[SPT], const ProdArgs& pa, int nchunk) {
#pragma unroll
  for (int s = 0; s < SPT; ++s) prod_issue<SRC, E>(pc[s], pa, (int)threadIdx.x + NT * s, nchunk);
}

// Write the staged activations into LDS (compute waves), given inv (SRC_NORM).
template <bool W4A8, int SRC, int E, int SPT>
__device__ __forceinline__ void stage_write(const ProdChunk<SRC, E> (&pc)[SPT], double inv, int K, int4* lds) {
  const int nb = K >> 5;
  if constexpr (W4A8) {
    const int nchunk = 2 * nb;
    int4* s_lo = lds;
    int4* s_hi = lds + (nb + 1);
    int2* s_bs = (int2*)(lds + 2 * (nb + 1));
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = (int)threadIdx.x + NT * s;
      float v[16];
      prod_values<SRC, 16>(pc[s], inv, v);
      if constexpr (SRC == SRC_F32) {  // the SwiGLU output, held in fp16 as in the launches
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = (float)f32_to_f16_rne(v[k]);
      }
      float scale;
      const int4 q = prod_quant16(v, scale);
      w4a8_stage_put(q, scale, i, i < nchunk, nb, s_lo, s_hi, s_bs);
    }
  } else {
    const int nchunk = K >> 3;
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = (int)threadIdx.x + NT * s;
      float v[8];
      prod_values<SRC, 8>(pc[s], inv, v);
      w4a16_stage_put_dot<MODE_F16>(prod_f16x8(v), i, i < nchunk, nb, (int*)lds, nullptr);
    }
  }
}

// ---- GEMV arithmetic on prefetched weights (W4A8 / W4A16, the five-launch kernels' order)
template <bool W4A8, int R, int NJ>
__device__ __forceinline__ void gemv_dot(const WBuf<R, NJ>& b, const int4* lds, int K, int lane, float (&acc)[R]) {
  const int nb = K >> 5;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  if constexpr (W4A8) {
    const int4* s_lo = lds;
    const int4* s_hi = lds + (nb + 1);
    const int2* s_bs = (const int2*)(lds + 2 * (nb + 1));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bi = lane + 64 * j;
      const int bb = min(bi, nb - 1);
      const int4 lo = s_lo[bb];
      const int4 hi = s_hi[bb];
      const int2 bs = s_bs[bb];
      const float xsf = bi < nb ? __builtin_bit_cast(float, bs.y) : 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int a = w4a8_block_dot(b.w[r][j], lo, hi, bs.x);
        acc[r] = fmaf(b.s[r][j] * xsf, (float)a, acc[r]);
      }
    }
  } else {
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    const int ps = nb + 1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bi = lane + 64 * j;
      const int bb = min(bi, nb - 1);
      const float mul = bi < nb ? 1.0f : 0.0f;  // fp16 staging: no block multiplier
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float s = w4a16_block_dot_h(b.w[r][j], lds, ps, bb, magic);
        acc[r] = fmaf(s * mul, b.s[r][j], acc[r]);
      }
    }
  }
}

// ---- attention (RoPE, cache append, one key split of one query head) ------------------
template <int D>
struct ATile {
  static constexpr int P = 2;
  static constexpr int LPK = D / 8;
  static constexpr int KPW = 64 / LPK;
  static constexpr int KT = NW * KPW * P;  // keys per tile
  uint4 k[P], v[P];
};

template <int D>
__device__ __forceinline__ void atile_issue(ATile<D>& b, const uint16_t* kc, const uint16_t* vc, size_t base, int t,
                                            int limit, int wave, int krow, int col) {
  using T = ATile<D>;
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * NW + wave) * T::KPW + krow;
    const size_t off = base + (size_t)(key < limit ? key : limit - 1) * D + col * 8;
    b.k[i] = *(const uint4*)(kc + off);
    b.v[i] = *(const uint4*)(vc + off);
  }
}

template <int D>
__device__ __forceinline__ void atile_compute(const ATile<D>& b, int t, int len, int pos, int wave, int krow, int col,
                                              const float (&qv)[8], const uint16_t* s_knew, const uint16_t* s_vnew,
                                              float& m_run, float& l_run, float (&acc)[8]) {
  using T = ATile<D>;
  float s[T::P];
  float m_tile = -INFINITY;
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * NW + wave) * T::KPW + krow;
    const uint4 kr = key == pos ? *(const uint4*)(s_knew + col * 8) : b.k[i];
    const uint32_t w[4] = {kr.x, kr.y, kr.z, kr.w};
    float d = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      d = fmaf(qv[2 * u + 1], bf16_bits_to_f32(w[u] >> 16), fmaf(qv[2 * u], bf16_bits_to_f32(w[u] & 0xffffu), d));
    d = group_sum<T::LPK>(d);
    s[i] = key < len ? d : -INFINITY;
    m_tile = fmaxf(m_tile, s[i]);
  }
  m_tile = stride_max<T::LPK>(m_tile);
  if (m_tile > m_run) {
    const float alpha = exp2f(m_run - m_tile);
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= alpha;
    m_run = m_tile;
  }
  if (m_run == -INFINITY) return;
#pragma unroll
  for (int i = 0; i < T::P; ++i) {
    const int key = t * T::KT + (i * NW + wave) * T::KPW + krow;
    const float p = exp2f(s[i] - m_run);
    l_run += p;
    const uint4 vr = key == pos ? *(const uint4*)(s_vnew + col * 8) : (key < len ? b.v[i] : make_uint4(0, 0, 0, 0));
    const uint32_t w[4] = {vr.x, vr.y, vr.z, vr.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[2 * u] = fmaf(p, bf16_bits_to_f32(w[u] & 0xffffu), acc[2 * u]);
      acc[2 * u + 1] = fmaf(p, bf16_bits_to_f32(w[u] >> 16), acc[2 * u + 1]);
    }
  }
}

// LDS of the attention phase (lives in the same dynamic LDS as the staging planes).
template <int D>
struct ALds {
  float q[D];
  uint16_t knew[D];
  uint16_t vnew[D];
  float m[NW], l[NW], f[NW], ml[2];
  float acc[NW * D];
};

// Phase timestamps of workgroup b (diagnostics; a.trace == NULL in normal runs): wave 0,
// lane 0 writes the 100 MHz realtime counter at each phase point.
#define MEGA_MARK(k)                                                                       \
  do {                                                                                     \
    if (a.trace && tid == 0) a.trace[blockIdx.x * 16 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)

// ---- the layer kernel ---------------------------------------------------------------------
// Phase shapes: A = Q/K/V (RA rows per wave, NJA chunks), C = o_proj, D = gate/up
// (RD = 2 x pairs), E = down.  SPT* = staging passes.  S = key splits.
template <bool W4A8, int HD, int S, int RA, int NJA, int RC, int NJC, int RD, int NJD, int RE, int NJE>
__global__ __launch_bounds__(kThreads) void layer_mega_kernel(Args a) {
  extern __shared__ int4 lds[];
  const int tid = threadIdx.x;
  // wave-uniform (scalar) wave index: every row -> matrix selection below is then scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool cw = wave < NW;  // compute wave
  const int gw = blockIdx.x * NW + wave;
  const int per_xcd = gridDim.x / 8;
  const int H = a.H, QD = a.QD, KD = a.KD, F = a.F;
  constexpr int E8 = W4A8 ? 16 : 8;  // activations per staging chunk
  double* s_red = (double*)((char*)lds + a.red_off);  // NW doubles past every phase's planes

  MEGA_MARK(0);
  const int pos = min(max(*a.pos, 0), a.max_seq - 1);
  const int len = pos + 1;

  // ================= phase A: Q/K/V with the input RMSNorm =================
  const Mats ma = {a.nib[0], a.nib[1], a.nib[2], a.sc[0], a.sc[1], a.sc[2], QD, KD, 3};
  const int totA = QD + 2 * KD;
  const bool actA = cw && gw * RA < totA;
  {
    constexpr int SPTA = 1;  // H/E8 <= NT (checked on the host)
    ProdChunk<SRC_NORM, E8> pc[SPTA];
    const ProdArgs pa{a.h, a.norm1, a.eps, 0, 0};
    const int nchunk = H / E8;
    if (cw) stage_issue<SRC_NORM, E8, SPTA>(pc, pa, nchunk);
    __builtin_amdgcn_sched_barrier(0);
    WBuf<RA, NJA> wa;
    if (actA) issue_weights<RA, NJA, false>(wa, ma, gw * RA, totA, H, lane);
    __builtin_amdgcn_sched_barrier(0);
    double ss = cw ? stage_sumsq<SRC_NORM, E8, SPTA>(pc, nchunk) : 0.0;
    if (cw && lane == 0) s_red[wave] = ss;
    lds_barrier();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_red[w];
    const double inv = 1.0 / sqrt(tot / (double)H + (double)a.eps);
    if (cw) stage_write<W4A8, SRC_NORM, E8, SPTA>(pc, inv, H, lds);
    lds_barrier();
    MEGA_MARK(1);
    if (actA) {
      float acc[RA];
      gemv_dot<W4A8, RA, NJA>(wa, lds, H, lane, acc);
#pragma unroll
      for (int r = 0; r < RA; ++r) {
        const float y = wave_sum_to_lane63(acc[r]);
        const int g = gw * RA + r;
        if (lane == 63 && g < totA) {
          int row;
          const int mi = mat_of(ma, g, row);
          st_coh((mi == 0 ? a.q : (mi == 1 ? a.k : a.v)) + row, y);
        }
      }
    }
    wait_mem();
    MEGA_MARK(2);
  }

  // ================= phase B: attention (one key split of one query head) =============
  using T = ATile<HD>;
  ALds<HD>& al = *(ALds<HD>*)lds;
  const int G = a.heads / a.kv_heads;
  int hq, sp;
  if (a.xcd_map) {
    const int b = blockIdx.x, x = b % 8, j = b / 8;
    const int pair = (j / G) * 8 + x;
    hq = (pair % a.kv_heads) * G + j % G;
    sp = pair / a.kv_heads;
  } else {
    hq = blockIdx.x % a.heads;
    sp = blockIdx.x / a.heads;
  }
  const bool attn = (int)blockIdx.x < a.heads * S;  // workgroup-uniform
  const int kvh = hq / G;
  const int col = lane % T::LPK, krow = lane / T::LPK;
  const size_t cache_base = (size_t)kvh * a.max_seq * HD;
  const int ntiles = (len + T::KT - 1) / T::KT;
  const int nt = ntiles > sp ? (ntiles - sp + S - 1) / S : 0;
  // o_proj weights: workgroups without an attention share prefetch them now
  const Mats mc = {a.nib[3], nullptr, nullptr, a.sc[3], nullptr, nullptr, H, 0, 1};
  const bool actC = cw && gw * RC < H;
  WBuf<RC, NJC> wc;
  T b0, b1, b2;
  grid_sync_arrive(a.bar, per_xcd);
  if (!attn && actC) issue_weights<RC, NJC, false>(wc, mc, gw * RC, H, QD, lane);
  if (attn && cw) {
    atile_issue<HD>(b0, a.kc, a.vc, cache_base, sp, len, wave, krow, col);
    atile_issue<HD>(b1, a.kc, a.vc, cache_base, sp + S, len, wave, krow, col);
    atile_issue<HD>(b2, a.kc, a.vc, cache_base, sp + 2 * S, len, wave, krow, col);
  }
  grid_sync_wait();
  MEGA_MARK(3);
  {
    constexpr int HALF = HD / 2;
    if (attn && tid < HALF) {
      const float q0 = a.q[(size_t)hq * HD + tid], q1 = a.q[(size_t)hq * HD + tid + HALF];
      const float k0 = a.k[(size_t)kvh * HD + tid], k1 = a.k[(size_t)kvh * HD + tid + HALF];
      const float v0 = a.v[(size_t)kvh * HD + tid], v1 = a.v[(size_t)kvh * HD + tid + HALF];
      const float c = a.rcos[(size_t)pos * HALF + tid], sn = a.rsin[(size_t)pos * HALF + tid];
      al.q[tid] = (q0 * c - q1 * sn) * a.qscale;
      al.q[tid + HALF] = (q0 * sn + q1 * c) * a.qscale;
      al.knew[tid] = f32_to_bf16_bits(k0 * c - k1 * sn);
      al.knew[tid + HALF] = f32_to_bf16_bits(k0 * sn + k1 * c);
      al.vnew[tid] = f32_to_bf16_bits(v0);
      al.vnew[tid + HALF] = f32_to_bf16_bits(v1);
    }
    lds_barrier();
    if (attn) {
      if (hq % G == 0 && sp == 0)
        for (int i = tid; i < HD; i += kThreads) {
          a.kc[cache_base + (size_t)pos * HD + i] = al.knew[i];
          a.vc[cache_base + (size_t)pos * HD + i] = al.vnew[i];
        }
    }
    float m_run = -INFINITY, l_run = 0.0f, acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    if (attn && cw) {
      float qv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[e] = al.q[col * 8 + e];
      for (int j = 0; j < nt; j += 3) {
        atile_compute<HD>(b0, sp + S * j, len, pos, wave, krow, col, qv, al.knew, al.vnew, m_run, l_run, acc);
        if (j + 3 < nt) atile_issue<HD>(b0, a.kc, a.vc, cache_base, sp + S * (j + 3), len, wave, krow, col);
        if (j + 1 < nt)
          atile_compute<HD>(b1, sp + S * (j + 1), len, pos, wave, krow, col, qv, al.knew, al.vnew, m_run, l_run, acc);
        if (j + 4 < nt) atile_issue<HD>(b1, a.kc, a.vc, cache_base, sp + S * (j + 4), len, wave, krow, col);
        if (j + 2 < nt)
          atile_compute<HD>(b2, sp + S * (j + 2), len, pos, wave, krow, col, qv, al.knew, al.vnew, m_run, l_run, acc);
        if (j + 5 < nt) atile_issue<HD>(b2, a.kc, a.vc, cache_base, sp + S * (j + 5), len, wave, krow, col);
      }
      l_run = stride_sum<T::LPK>(l_run);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = stride_sum<T::LPK>(acc[e]);
      if (krow == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) al.acc[wave * HD + col * 8 + e] = acc[e];
        if (col == 0) {
          al.m[wave] = m_run;
          al.l[wave] = l_run;
        }
      }
    }
    lds_barrier();
    if (attn && tid < NW) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, al.m[w]);
      al.f[tid] = al.m[tid] == -INFINITY ? 0.0f : exp2f(al.m[tid] - M);
      if (tid == 0) {
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) L = fmaf(al.m[w] == -INFINITY ? 0.0f : exp2f(al.m[w] - M), al.l[w], L);
        al.ml[0] = M;
        al.ml[1] = L;
      }
    }
    lds_barrier();
    if (attn && tid < HD / 4) {
      float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = al.f[w];
        const float4 a4 = *(const float4*)&al.acc[w * HD + 4 * tid];
        o[0] = fmaf(f, a4.x, o[0]);
        o[1] = fmaf(f, a4.y, o[1]);
        o[2] = fmaf(f, a4.z, o[2]);
        o[3] = fmaf(f, a4.w, o[3]);
      }
      float* rec = a.part + ((size_t)sp * a.heads + hq) * (HD + 4);
      if (tid == 0) {
        st_coh(rec, al.ml[0]);
        st_coh(rec + 1, al.ml[1]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) st_coh(rec + 4 + 4 * tid + e, o[e]);
    }
    wait_mem();
    MEGA_MARK(4);
  }
  grid_sync_arrive(a.bar, per_xcd);
  if (attn && actC) issue_weights<RC, NJC, false>(wc, mc, gw * RC, H, QD, lane);
  grid_sync_wait();
  MEGA_MARK(5);

  // ================= phase C: o_proj, merging the key-split partials; h_mid = h + y ======
  {
    constexpr int SRCC = S == 1 ? SRC_ATTN1 : (S == 2 ? SRC_ATTN2 : (S == 4 ? SRC_ATTN4 : SRC_ATTN8));
    ProdChunk<SRCC, E8> pc[1];
    const ProdArgs pa{a.part, nullptr, 0.0f, HD, a.heads};
    const int nchunk = QD / E8;
    if (cw) stage_issue<SRCC, E8, 1>(pc, pa, nchunk);
    if (cw) stage_write<W4A8, SRCC, E8, 1>(pc, 0.0, QD, lds);
    lds_barrier();
    if (actC) {
      float acc[RC];
      gemv_dot<W4A8, RC, NJC>(wc, lds, QD, lane, acc);
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        const float y = wave_sum_to_lane63(acc[r]);
        const int n = gw * RC + r;
        if (lane == 63 && n < H) st_coh(a.hmid + n, a.h[n] + y);
      }
    }
    wait_mem();
    MEGA_MARK(6);
  }
  const Mats md = {a.nib[4], a.nib[5], nullptr, a.sc[4], a.sc[5], nullptr, F, F, 2};
  constexpr int RDH = RD / 2;
  const bool actD = cw && gw * RDH < F;
  WBuf<RD, NJD> wd;
  // (the arrival's LDS barrier also orders phase C's LDS reads before phase D's writes)
  grid_sync_arrive(a.bar, per_xcd);
  if (actD) issue_weights<RD, NJD, true>(wd, md, gw * RDH, F, H, lane);
  grid_sync_wait();
  MEGA_MARK(7);

  // ================= phase D: gate/up with the post-attention RMSNorm; mid = silu(g) * u ===
  {
    ProdChunk<SRC_NORM, E8> pc[1];
    const ProdArgs pa{a.hmid, a.norm2, a.eps, 0, 0};
    const int nchunk = H / E8;
    if (cw) stage_issue<SRC_NORM, E8, 1>(pc, pa, nchunk);
    double ss = cw ? stage_sumsq<SRC_NORM, E8, 1>(pc, nchunk) : 0.0;
    if (cw && lane == 0) s_red[wave] = ss;
    lds_barrier();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_red[w];
    const double inv = 1.0 / sqrt(tot / (double)H + (double)a.eps);
    if (cw) stage_write<W4A8, SRC_NORM, E8, 1>(pc, inv, H, lds);
    lds_barrier();
    if (actD) {
      float acc[RD];
      gemv_dot<W4A8, RD, NJD>(wd, lds, H, lane, acc);
#pragma unroll
      for (int r = 0; r < RDH; ++r) {
        const float g = wave_sum_to_lane63(acc[r]);
        const float u = wave_sum_to_lane63(acc[r + RDH]);
        const int n = gw * RDH + r;
        if (lane == 63 && n < F) st_coh(a.mid + n, g / (1.0f + expf(-g)) * u);
      }
    }
    wait_mem();
    MEGA_MARK(8);
  }
  const Mats me = {a.nib[6], nullptr, nullptr, a.sc[6], nullptr, nullptr, H, 0, 1};
  const bool actE = cw && gw * RE < H;
  WBuf<RE, NJE> we;
  grid_sync_arrive(a.bar, per_xcd);
  if (actE) issue_weights<RE, NJE, false>(we, me, gw * RE, H, F, lane);
  grid_sync_wait();
  MEGA_MARK(9);

  // ================= phase E: down (mid quantized / rounded in the staging); h = h_mid + y ==
  {
    constexpr int SPTE = W4A8 ? 1 : 2;  // F / E8 <= SPTE * NT (the host admits F <= 8192)
    ProdChunk<SRC_F32, E8> pc[SPTE];
    const ProdArgs pa{a.mid, nullptr, 0.0f, 0, 0};
    const int nchunk = F / E8;
    if (cw) stage_issue<SRC_F32, E8, SPTE>(pc, pa, nchunk);
    if (cw) stage_write<W4A8, SRC_F32, E8, SPTE>(pc, 0.0, F, lds);
    lds_barrier();
    if (actE) {
      float acc[RE];
      gemv_dot<W4A8, RE, NJE>(we, lds, F, lane, acc);
#pragma unroll
      for (int r = 0; r < RE; ++r) {
        const float y = wave_sum_to_lane63(acc[r]);
        const int n = gw * RE + r;
        if (lane == 63 && n < H) a.h[n] = a.hmid[n] + y;
      }
    }
    MEGA_MARK(10);
  }
}

__global__ void zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace mega
}  // namespace nve

namespace nve_host {

size_t mega_bar_bytes() { return (size_t)nve::mega::kBarWords * nve::mega::kWord * sizeof(unsigned); }

// Shape classes with a compiled tiling: (rows per wave, 64-block chunks per lane) of
// the Q/K/V, o_proj, gate/up (2 x pairs) and down phases, and the head size.
//   0: Llama-3.2-3B layers (hidden 3072, 24 x 128 query / 8 x 128 key heads, FFN 8192)
//   1: small layers (hidden 256, 4 x 64 / 2 x 64, FFN 512; the test models)
#define NVE_MEGA_CLASSES(X) \
  X(0, 128, 3, 2, 2, 2, 8, 2, 2, 4) \
  X(1, 64, 1, 1, 1, 1, 2, 1, 1, 1)

static int cdiv(int a, int b) { return (a + b - 1) / b; }

// Grid = CU count (one workgroup per CU; 8 compute waves each).
static int mega_grid() {
  static int g = -1;
  if (g < 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 0;
    g = (n >= 8 && n % 8 == 0) ? n : 0;
  }
  return g;
}

// Shape class of a layer, or -1 when no compiled tiling matches (the five-launch path
// then serves it).
int mega_class(const nve_decode_config& c, int split) {
  const int grid = mega_grid();
  if (grid == 0) return -1;
  const int waves = grid * nve::mega::NW;
  const int H = c.hidden, QD = c.num_heads * c.head_dim, KD = c.num_kv_heads * c.head_dim, F = c.ffn;
  if (c.num_heads * split > grid || F > 8192 || H / 8 > nve::mega::NT || QD / 8 > nve::mega::NT) return -1;
  const int ra = cdiv(QD + 2 * KD, waves), nja = cdiv(H / 32, 64);
  const int rc = cdiv(H, waves), njc = cdiv(QD / 32, 64);
  const int rd = 2 * cdiv(F, waves), njd = cdiv(H / 32, 64);
  const int re = cdiv(H, waves), nje = cdiv(F / 32, 64);
#define NVE_MEGA_MATCH(ID, HD, RA, NJA, RC, NJC, RD, NJD, RE, NJE)                                              \
  if (c.head_dim == HD && ra == RA && nja == NJA && rc == RC && njc == NJC && rd == RD && njd == NJD && re == RE && \
      nje == NJE)                                                                                              \
    return ID;
  NVE_MEGA_CLASSES(NVE_MEGA_MATCH)
#undef NVE_MEGA_MATCH
  return -1;
}

// Barrier words of a workspace start at zero: the first layer call with a workspace on
// a device zeroes them (after that they return to zero at every completed barrier).
static hipError_t mega_init_bar(unsigned* bar, hipStream_t s) {
  static std::mutex mu;
  static std::set<std::pair<int, void*>> seen;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (!seen.insert({dev, (void*)bar}).second) return hipSuccess;
  }
  const int n = nve::mega::kBarWords * nve::mega::kWord;
  hipLaunchKernelGGL(nve::mega::zero_words_kernel, dim3((n + 255) / 256), dim3(256), 0, s, bar, n);
  return hipGetLastError();
}

template <bool W4A8, int HD, int S, int RA, int NJA, int RC, int NJC, int RD, int NJD, int RE, int NJE>
static hipError_t launch_mega_t(nve::mega::Args a, hipStream_t s) {
  const size_t stage = std::max({nve::mega::stage_bytes<W4A8>(a.H), nve::mega::stage_bytes<W4A8>(a.QD),
                                 nve::mega::stage_bytes<W4A8>(a.F), sizeof(nve::mega::ALds<HD>)});
  a.red_off = (int)((stage + 15) & ~(size_t)15);
  const size_t lds = (size_t)a.red_off + 8 * nve::mega::NW;
  auto kern = nve::mega::layer_mega_kernel<W4A8, HD, S, RA, NJA, RC, NJC, RD, NJD, RE, NJE>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(mega_grid()), dim3(nve::mega::kThreads), lds, s, a);
  return hipGetLastError();
}

hipError_t launch_layer_mega(int cls, bool w4a8, int split, const nve::mega::Args& a, hipStream_t s) {
  hipError_t e = mega_init_bar(a.bar, s);
  if (e != hipSuccess) return e;
#define NVE_MEGA_S(W, ID, HD, RA, NJA, RC, NJC, RD, NJD, RE, NJE)                                           \
  switch (split) {                                                                                       \
    case 1: return launch_mega_t<W, HD, 1, RA, NJA, RC, NJC, RD, NJD, RE, NJE>(a, s);                     \
    case 2: return launch_mega_t<W, HD, 2, RA, NJA, RC, NJC, RD, NJD, RE, NJE>(a, s);                     \
    case 4: return launch_mega_t<W, HD, 4, RA, NJA, RC, NJC, RD, NJD, RE, NJE>(a, s);                     \
    default: return launch_mega_t<W, HD, 8, RA, NJA, RC, NJC, RD, NJD, RE, NJE>(a, s);                    \
  }
#define NVE_MEGA_LAUNCH(ID, HD, RA, NJA, RC, NJC, RD, NJD, RE, NJE)           \
  if (cls == ID) {                                                          \
    if (w4a8) {                                                             \
      NVE_MEGA_S(true, ID, HD, RA, NJA, RC, NJC, RD, NJD, RE, NJE)            \
    } else {                                                                \
      NVE_MEGA_S(false, ID, HD, RA, NJA, RC, NJC, RD, NJD, RE, NJE)           \
    }                                                                       \
  }
  NVE_MEGA_CLASSES(NVE_MEGA_LAUNCH)
#undef NVE_MEGA_LAUNCH
#undef NVE_MEGA_S
  return hipErrorInvalidValue;
}

}  // namespace nve_host
