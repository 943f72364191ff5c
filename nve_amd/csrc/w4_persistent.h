// w4_persistent.h -- persistent, double-buffered W4 GEMV kernel (W4A8 and W4A16).
//
// The one-shot kernels give every wave a single R-row tile: all of a wave's loads
// are issued at once and its arithmetic runs only after they land, so at large N
// the arithmetic of the last-served waves trails the HBM stream.  Here a fixed grid
// (a few workgroups per CU) walks the tiles: wave w handles tiles w, w+W, w+2W, ...
// (W = waves in the grid) and, while it computes tile t from one register buffer,
// the loads of tile t+W are already in flight into the other.  The activation vector
// is staged into LDS once per workgroup instead of once per tile.
//
// Loads are never predicated (the compiler then counts outstanding loads exactly and
// waits only for the older buffer): the prefetch after a wave's last tile re-reads
// tile 0 of its matrix, which every wave of that matrix shares, so it is served from
// L2.
#pragma once

#include "common.h"
#include "w4_launch.h"

namespace nve {

template <int R, int NJ>
struct W4Buf {
  uint4 w[R][NJ];
  float s[R][NJ];
};

template <int R, int NJ>
__device__ __forceinline__ void w4_issue(W4Buf<R, NJ>& buf, const W4Wave& wv, int t, int K, int lane) {
  const int nb = K >> 5;
  const size_t row_bytes = (size_t)(K >> 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(t * R + r, wv.n - 1);
    const uint4* rn = (const uint4*)(wv.nib + (size_t)row * row_bytes);
    const float* rs = wv.ws + (size_t)row * nb;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bb = min(lane + 64 * j, nb - 1);
      buf.w[r][j] = ld_stream(rn + bb);
      buf.s[r][j] = ld_stream(rs + bb);
    }
  }
}

// Results of up to kMaxTilesPerWave tiles per wave are parked in LDS (written by
// lane 63 with ds_write) and stored to global memory after the loop: a global store
// inside the loop would sit in the in-order vmcnt queue behind the prefetch loads and
// any later reuse of its data register would wait for the whole prefetch.
constexpr int kMaxTilesPerWave = kPersistentMaxTilesPerWave;

template <class P, int R, int NJ>
__device__ __forceinline__ void w4_compute(const W4Buf<R, NJ>& buf, int K, int lane, const int4* lds,
                                           float* res, const typename P::Ctx& ctx) {
  const int nb = K >> 5;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int b = lane + 64 * j;
    const int bb = min(b, nb - 1);
    const typename P::XFrag xf = P::load_x(lds, nb, bb, b < nb);
#pragma unroll
    for (int r = 0; r < R; ++r) P::accum(acc[r], buf.w[r][j], buf.s[r][j], xf, lds, nb, ctx);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum_to_lane63(acc[r]);
    if (lane == 63) res[r] = v;
  }
}

template <class P, int OUT_DT, int R, int NJ>
__global__ __launch_bounds__(256) void w4_persistent_kernel(const typename P::Args args, W4Segs segs, int K) {
  extern __shared__ int4 lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // wave-uniform values live in SGPRs
  const int w = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + wave);
  const W4Wave wv = resolve_wave(segs, w);
  const int W = __builtin_amdgcn_readfirstlane(wv.stride);
  const int T = __builtin_amdgcn_readfirstlane(wv.tiles);
  const int t0 = __builtin_amdgcn_readfirstlane(wv.t0);
  float* res = (float*)((char*)lds + P::lds_bytes(K)) + wave * (kMaxTilesPerWave * R);

  typename P::template Stage<NJ> st;
  P::template stage_issue<NJ>(st, args, K);
  __builtin_amdgcn_sched_barrier(0);
  W4Buf<R, NJ> a, b;
  w4_issue<R, NJ>(a, wv, t0 < T ? t0 : 0, K, lane);
  __builtin_amdgcn_sched_barrier(0);
  P::template stage_write<NJ>(st, args, lds, K);
  lds_barrier();
  if (t0 >= T) return;  // wave-uniform; no barrier follows
  const typename P::Ctx ctx = P::make_ctx();
  // Tiles of this wave: t0, t0+W, ...; at most kMaxTilesPerWave (the host sizes the
  // grid for that).  The loop is fully unrolled, so there is no back-edge: the
  // compiler's waitcnt analysis sees straight-line code and waits, before each
  // compute, only for the older of the two buffers.
  const int cnt = __builtin_amdgcn_readfirstlane(min((T - t0 + W - 1) / W, kMaxTilesPerWave));
  int k = 0;
#pragma unroll
  for (int i = 0; i < kMaxTilesPerWave; ++i) {
    if (i >= cnt) break;
    const int tn = t0 + (i + 1) * W;
    if (i & 1) {
      w4_issue<R, NJ>(a, wv, i + 1 < cnt ? tn : 0, K, lane);
      __builtin_amdgcn_sched_barrier(0);
      w4_compute<P, R, NJ>(b, K, lane, lds, res + R * i, ctx);
    } else {
      w4_issue<R, NJ>(b, wv, i + 1 < cnt ? tn : 0, K, lane);
      __builtin_amdgcn_sched_barrier(0);
      w4_compute<P, R, NJ>(a, K, lane, lds, res + R * i, ctx);
    }
    k = i + 1;
  }
  // Flush: lane r of the wave stores row r of each of the wave's k tiles.
  for (int i = 0; i < k; ++i) {
    const int row = (t0 + i * W) * R + lane;
    if (lane < R && row < wv.n) store_out<OUT_DT>(wv.out, (size_t)row, res[R * i + lane]);
  }
}

}  // namespace nve
