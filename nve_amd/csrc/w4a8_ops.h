// w4a8_ops.h -- W4A8 device pieces shared by the one-shot and persistent GEMV
// kernels: the exact int32 block dot product (v_dot4) and the LDS staging of the
// quantized activation vector.
#pragma once

#include "common.h"

namespace nve {

// Exact int32 accumulator of one Q4_0 block (GPU nibble order) against 32 int8
// activations: lo = elements 0..15, hi = elements 16..31 (4 per dword).
__device__ __forceinline__ int w4a8_block_dot(uint4 w, int4 lo, int4 hi, int sumq) {
  const unsigned M = 0x0F0F0F0Fu;
  int s = 0;
  s = __builtin_amdgcn_sdot4((int)(w.x & M), lo.x, s, false);
  s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & M), hi.x, s, false);
  s = __builtin_amdgcn_sdot4((int)(w.y & M), lo.y, s, false);
  s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & M), hi.y, s, false);
  s = __builtin_amdgcn_sdot4((int)(w.z & M), lo.z, s, false);
  s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & M), hi.z, s, false);
  s = __builtin_amdgcn_sdot4((int)(w.w & M), lo.w, s, false);
  s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & M), hi.w, s, false);
  return s - 8 * sumq;
}

__device__ __forceinline__ int sum_i8x16(int4 v) {
  int s = 0;
  s = __builtin_amdgcn_sdot4(v.x, 0x01010101, s, false);
  s = __builtin_amdgcn_sdot4(v.y, 0x01010101, s, false);
  s = __builtin_amdgcn_sdot4(v.z, 0x01010101, s, false);
  s = __builtin_amdgcn_sdot4(v.w, 0x01010101, s, false);
  return s;
}

// LDS layout for K activations (nb = K/32 blocks, plus one spare slot written by
// threads past the end of the vector):
//   int4 lo[nb+1]; int4 hi[nb+1]; int2 bs[nb+1] = {sum(xq of block), bits(xs[b])}
__host__ __device__ constexpr size_t w4a8_lds_bytes(int K) {
  return (size_t)(K / 32 + 1) * (16 + 16 + 8);
}

// Stage xq/xs into LDS.  Thread t handles 16-byte chunks i = t + 256*s; chunk i is
// half (i & 1) of block i >> 1, and lanes 2k / 2k+1 hold the two halves of a block
// so the per-block sum(xq) is a DPP pair sum.  Loads are unconditional (clamped
// index) so the compiler can count outstanding loads exactly; only LDS writes are
// predicated.
template <int SPT>
struct W4A8Stage {
  int4 v[SPT];
  float xs[SPT];
};

// xs_one: every block scale is 1 (the per-token mode applies one row scale at the end);
// xs is not read.
template <int SPT>
__device__ __forceinline__ void w4a8_stage_issue(W4A8Stage<SPT>& st, const int8_t* __restrict__ xq,
                                                 const float* __restrict__ xs, int nchunk, bool xs_one = false) {
#pragma unroll
  for (int s = 0; s < SPT; ++s) {
    const int i = min((int)threadIdx.x + 256 * s, nchunk - 1);
    st.v[s] = ((const int4*)xq)[i];
    st.xs[s] = xs_one ? 1.0f : xs[i >> 1];
  }
}

__device__ __forceinline__ void w4a8_stage_put(int4 v, float xsb, int i, bool valid, int nb,
                                               int4* s_lo, int4* s_hi, int2* s_bs) {
  // Both lanes of a pair write the same {sum, xs} word and each writes its half to
  // the lo or hi plane by address select: no branches, so no load is sunk.  Lanes
  // past the end (valid == false) write to the spare slot nb.
  const int b = valid ? (i >> 1) : nb;
  const int q = pair_sum_i(sum_i8x16(v));
  int4* dst = (i & 1) ? s_hi : s_lo;
  dst[b] = v;
  s_bs[b] = make_int2(q, __builtin_bit_cast(int, xsb));
}

template <int SPT>
__device__ __forceinline__ void w4a8_stage_write(const W4A8Stage<SPT>& st, int4* s_lo, int4* s_hi,
                                                 int2* s_bs, int nchunk) {
#pragma unroll
  for (int s = 0; s < SPT; ++s) {
    // nchunk is even, so the two lanes of a pair are both valid or both not.
    const int i = threadIdx.x + 256 * s;
    w4a8_stage_put(st.v[s], st.xs[s], i, i < nchunk, nchunk >> 1, s_lo, s_hi, s_bs);
  }
}

// Staging for K > 16384 (MULTI kernels): loads and LDS writes in one loop.
__device__ __forceinline__ void w4a8_stage_loop(const int8_t* __restrict__ xq,
                                                const float* __restrict__ xs, int4* s_lo,
                                                int4* s_hi, int2* s_bs, int nchunk, bool xs_one = false) {
  for (int base = 0; base < nchunk; base += 256) {
    const int i = base + threadIdx.x;
    const int ic = min(i, nchunk - 1);
    w4a8_stage_put(((const int4*)xq)[ic], xs_one ? 1.0f : xs[ic >> 1], i, i < nchunk, nchunk >> 1, s_lo, s_hi,
                   s_bs);
  }
}

// Policy used by the persistent kernel (w4_persistent.h).
struct W4A8Policy {
  struct Args {
    const int8_t* xq;
    const float* xs;
  };
  template <int NJ>
  struct Stage {
    W4A8Stage<(NJ + 1) / 2> st;
  };
  struct XFrag {
    int4 lo, hi;
    int sumq;
    float xs;
  };
  static __host__ __device__ size_t lds_bytes(int K) { return w4a8_lds_bytes(K); }
  template <int NJ>
  static __device__ __forceinline__ void stage_issue(Stage<NJ>& s, const Args& a, int K) {
    w4a8_stage_issue<(NJ + 1) / 2>(s.st, a.xq, a.xs, 2 * (K >> 5));
  }
  template <int NJ>
  static __device__ __forceinline__ void stage_write(const Stage<NJ>& s, const Args&, int4* lds, int K) {
    const int nb = K >> 5;
    w4a8_stage_write<(NJ + 1) / 2>(s.st, lds, lds + (nb + 1), (int2*)(lds + 2 * (nb + 1)), 2 * nb);
  }
  static __device__ __forceinline__ XFrag load_x(const int4* lds, int nb, int bb, bool valid) {
    const int2 bs = ((const int2*)(lds + 2 * (nb + 1)))[bb];
    XFrag f;
    f.lo = lds[bb];
    f.hi = lds[(nb + 1) + bb];
    f.sumq = bs.x;
    f.xs = valid ? __builtin_bit_cast(float, bs.y) : 0.0f;
    return f;
  }
  struct Ctx {};
  static __device__ __forceinline__ Ctx make_ctx() { return Ctx{}; }
  // y += ws * xs * acc (the reference's per-block order, cuda/nve_kernels.cu:855-858)
  static __device__ __forceinline__ void accum(float& acc, uint4 w, float ws, const XFrag& x, const int4*,
                                               int, const Ctx&) {
    const int a = w4a8_block_dot(w, x.lo, x.hi, x.sumq);
    acc = fmaf(ws * x.xs, (float)a, acc);
  }
};

}  // namespace nve
