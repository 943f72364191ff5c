// gemv_w4a8_batched.hip -- small-batch W4A8 (M <= 16 activation rows).
//
// y[m, n] = sum_b ws[n,b] * xs(m,b) * acc[m,n,b],  acc = sum (nib - 8) * xq[m, .]
// xs(m,b) is xq_scales[m*(K/32) + b] (group mode, the reference's scheme per row)
// or the per-row bf16 scale (per-token mode, applied once per row: the sum over
// blocks is formed with ws only and multiplied by the row scale at the end).
//
// M = 1 runs the one-shot W4A8 GEMV (gemv_w4a8.hip); M >= 2 the LDS-ring int8 MFMA
// kernel where K % 128 == 0 and N <= 16384, otherwise the staged v_dot4 kernel for M = 2
// (where its LDS fits) and the register int8 MFMA kernel.
// v_dot4 kernel (any M >= 2 under NVE_GEMV_ONESHOT): one wave per output row, lane l owns
// blocks l, l+64, ...; the nibbles are turned into signed int8 (nib - 8) once per
// block with (t + 0x78787878) ^ 0x80808080 (no carries cross bytes for t <= 15), and
// every activation row reuses them through 8 v_dot4_i32_i8.
#include "common.h"
#include "lds_ring.h"
#include "w4_launch.h"
#include "w4a8_ops.h"

namespace nve {

__device__ __forceinline__ int s8_from_nib(uint32_t t) {  // t: 4 bytes, each 0..15
  return (int)((t + 0x78787878u) ^ 0x80808080u);
}

template <int OUT_DT, int XS_MODE>
__global__ __launch_bounds__(256) void w4a8_batched_dot4_kernel(int M, const int8_t* __restrict__ xq,
                                                                const void* __restrict__ xs,
                                                                const uint8_t* __restrict__ nib,
                                                                const float* __restrict__ ws,
                                                                void* __restrict__ out, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nb = K >> 5;
  const int rowc = min(row, N - 1);
  const uint4* rn = (const uint4*)(nib + (size_t)rowc * (size_t)(K >> 1));
  const float* rs = ws + (size_t)rowc * nb;
  float acc[NVE_MAX_M];
#pragma unroll
  for (int m = 0; m < NVE_MAX_M; ++m) acc[m] = 0.0f;

  for (int b = lane; b < nb; b += 64) {
    const uint4 w = rn[b];
    const float wsc = rs[b];
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    int lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo[i] = s8_from_nib(d[i] & 0x0F0F0F0Fu);
      hi[i] = s8_from_nib((d[i] >> 4) & 0x0F0F0F0Fu);
    }
#pragma unroll
    for (int m = 0; m < NVE_MAX_M; ++m) {
      if (m < M) {
        const int4* xr = (const int4*)(xq + (size_t)m * K) + 2 * b;
        const int4 a = xr[0], c = xr[1];
        int s = 0;
        s = __builtin_amdgcn_sdot4(lo[0], a.x, s, false);
        s = __builtin_amdgcn_sdot4(hi[0], c.x, s, false);
        s = __builtin_amdgcn_sdot4(lo[1], a.y, s, false);
        s = __builtin_amdgcn_sdot4(hi[1], c.y, s, false);
        s = __builtin_amdgcn_sdot4(lo[2], a.z, s, false);
        s = __builtin_amdgcn_sdot4(hi[2], c.z, s, false);
        s = __builtin_amdgcn_sdot4(lo[3], a.w, s, false);
        s = __builtin_amdgcn_sdot4(hi[3], c.w, s, false);
        if (XS_MODE == NVE_XS_GROUP32_F32) {
          const float xsf = ((const float*)xs)[(size_t)m * nb + b];
          acc[m] = fmaf(wsc * xsf, (float)s, acc[m]);
        } else {
          acc[m] = fmaf(wsc, (float)s, acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < NVE_MAX_M; ++m) {
    if (m < M) {
      float v = wave_sum_to_lane63(acc[m]);
      if (XS_MODE == NVE_XS_ROW_BF16) v *= bf16_bits_to_f32(((const uint16_t*)xs)[m]);
      if (lane == 63 && row < N) store_out<OUT_DT>(out, (size_t)m * N + row, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Staged v_dot4 kernel (small M): the one-row GEMV's structure (gemv_w4a8.hip) with
// the M activation rows staged in LDS, each in the one-row kernel's planes (lo / hi
// halves of every block, {sum(xq), bits(xs)}).  A wave owns R weight rows, lane l owns
// blocks l, l + 64, ...; every weight load is issued before any arithmetic; a block's
// nibbles are masked once and meet each activation row through 8 v_dot4 (the block
// order per lane and the fma per block are the one-row kernel's, so the per-row result
// is the same arithmetic as M one-row launches).  Per-token mode stages unit block
// scales and multiplies each row sum by the row's bf16 scale.
__host__ __device__ constexpr int staged_row_int4(int K) {  // LDS int4 units per activation row
  return 2 * (K / 32 + 1) + (K / 32 + 2) / 2;
}

template <int OUT_DT, int XS_MODE, int MM, int R, int NJ>
__global__ __launch_bounds__(256) void w4a8_batched_staged_kernel(int M, const int8_t* __restrict__ xq,
                                                                  const void* __restrict__ xs,
                                                                  const uint8_t* __restrict__ nib,
                                                                  const float* __restrict__ ws,
                                                                  void* __restrict__ out, int N, int K) {
  constexpr int SPT = (NJ + 1) / 2;  // staging passes per row: 2*nb <= 128*NJ chunks of 16 B
  extern __shared__ int4 lds[];
  const int nb = K >> 5;
  const int nchunk = 2 * nb;
  const int rs = staged_row_int4(K);
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;

  // (1) staging loads of every activation row (clamped index, unconditional)
  int4 sv[MM][SPT];
  float sx[MM][SPT];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const int mc = min(m, M - 1);
#pragma unroll
    for (int s = 0; s < SPT; ++s) {
      const int i = min((int)threadIdx.x + 256 * s, nchunk - 1);
      sv[m][s] = ((const int4*)(xq + (size_t)mc * K))[i];
      sx[m][s] = XS_MODE == NVE_XS_GROUP32_F32 ? ((const float*)xs)[(size_t)mc * nb + (i >> 1)] : 1.0f;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // (2) weight loads (blocks past the end of a row re-load block nb-1, zeroed at use)
  uint4 wv[R][NJ];
  float wsc[R][NJ];
  const size_t row_bytes = (size_t)(K >> 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, N - 1);
    const uint4* rn = (const uint4*)(nib + (size_t)row * row_bytes);
    const float* rsc = ws + (size_t)row * nb;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bb = min(lane + 64 * j, nb - 1);
      wv[r][j] = ld_stream(rn + bb);
      wsc[r][j] = ld_stream(rsc + bb);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // (3) LDS writes (wait only for the older staging loads)
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m < M) {
      int4* base = lds + (size_t)m * rs;
#pragma unroll
      for (int s = 0; s < SPT; ++s) {
        const int i = (int)threadIdx.x + 256 * s;
        w4a8_stage_put(sv[m][s], sx[m][s], i, i < nchunk, nb, base, base + (nb + 1), (int2*)(base + 2 * (nb + 1)));
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();

  // (4) arithmetic
  float acc[R][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.0f;
  const unsigned MASK = 0x0F0F0F0Fu;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int b = lane + 64 * j;
    const int bb = min(b, nb - 1);
    int4 lo[MM], hi[MM];
    int sq[MM];
    float xsf[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (m < M) {
        const int4* base = lds + (size_t)m * rs;
        lo[m] = base[bb];
        hi[m] = base[(nb + 1) + bb];
        const int2 bs = ((const int2*)(base + 2 * (nb + 1)))[bb];
        sq[m] = bs.x;
        xsf[m] = b < nb ? __builtin_bit_cast(float, bs.y) : 0.0f;  // lanes past the end add nothing
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint4 w = wv[r][j];
      const int w0 = (int)(w.x & MASK), w1 = (int)((w.x >> 4) & MASK), w2 = (int)(w.y & MASK),
                w3 = (int)((w.y >> 4) & MASK), w4 = (int)(w.z & MASK), w5 = (int)((w.z >> 4) & MASK),
                w6 = (int)(w.w & MASK), w7 = (int)((w.w >> 4) & MASK);
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (m < M) {
          int d = 0;
          d = __builtin_amdgcn_sdot4(w0, lo[m].x, d, false);
          d = __builtin_amdgcn_sdot4(w1, hi[m].x, d, false);
          d = __builtin_amdgcn_sdot4(w2, lo[m].y, d, false);
          d = __builtin_amdgcn_sdot4(w3, hi[m].y, d, false);
          d = __builtin_amdgcn_sdot4(w4, lo[m].z, d, false);
          d = __builtin_amdgcn_sdot4(w5, hi[m].z, d, false);
          d = __builtin_amdgcn_sdot4(w6, lo[m].w, d, false);
          d = __builtin_amdgcn_sdot4(w7, hi[m].w, d, false);
          acc[r][m] = fmaf(wsc[r][j] * xsf[m], (float)(d - 8 * sq[m]), acc[r][m]);
        }
      }
    }
  }
  // (5) row sums
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    if (m < M) {
      const float rsc = XS_MODE == NVE_XS_ROW_BF16 ? bf16_bits_to_f32(((const uint16_t*)xs)[m]) : 1.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v = wave_sum_to_lane63(acc[r][m]);
        if (XS_MODE == NVE_XS_ROW_BF16) v *= rsc;
        if (lane == 63 && row0 + r < N) store_out<OUT_DT>(out, (size_t)m * N + row0 + r, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// int8 MFMA kernel (M >= 2).
//
// The activation rows are the A operand of v_mfma_i32_16x16x32_i8 (rows i) and a
// 16-row weight tile the B operand (columns n), one 32-weight block per MFMA, so a
// block's output D[i][n] lands with weight row n = lane % 16 in every lane and the
// block's weight scale is one value per lane.  Nibbles enter the MFMA raw (0..15 is
// a valid int8); the -8 offset is the accumulator input C[i][.] = -8 * sum_k xq[i, k],
// itself one MFMA of the activation operand with a B operand of all -8 bytes: the
// int32 block accumulators are exact, as in the one-row kernels.
//
// Memory access: the operand layout (lane = (row % 16, k group)) puts 4 different
// rows in 4 consecutive lanes, and the texture path serves a wave load one 64-byte
// piece per 4 consecutive lanes only when those lanes read 64 contiguous bytes;
// loaded in operand order, every lane costs a separate cache access (measured 17x
// the accesses of the one-row GEMV on the same bytes).  So every load is issued in
// row-major lane order -- lane (r = lane / 4, p = lane % 4) reads piece p of row r,
// 16 rows x 64 contiguous bytes per instruction -- and the registers are moved to the
// operand lanes with ds_bpermute (through the LDS crossbar, no LDS storage), then the
// 4x4 (lane group x dword) transpose of two permlane32 + two permlane16 swaps.
//
// Activation row m sits in A row i = 4 (m % 4) + m / 4, so D row 4g + e (lane group
// g, element e) is activation row 4e + g: for M <= 4 only element 0 of each lane is
// live, for M <= 8 elements 0-1 (EU = ceil(M / 4) elements are scaled and summed).
// A workgroup owns T weight tiles; its KS waves take the quads (4 blocks) q = wave,
// wave + KS, ... of K and meet in LDS.
typedef int v4i_t __attribute__((ext_vector_type(4)));

// One quad of K: activations (two 16-byte halves of block 4q+p of activation row r)
// and, per tile, weights (block 4q+p of weight row r) and the quad's 4 weight scales,
// all in the row-major load layout.
template <int T>
struct BQuad {
  uint4 xa, xb;
  uint4 w[T];
  float4 sc[T];
};

template <int T>
__device__ __forceinline__ void bquad_issue(BQuad<T>& st, const uint4* xrow, const uint4* const (&wrow)[T],
                                            const float* const (&srow)[T], bool vec_sc, int q, int nq, int nb,
                                            int p) {
  q = min(q, nq - 1);
  const int bl = min(4 * q + p, nb - 1);
  st.xa = xrow[2 * bl];
  st.xb = xrow[2 * bl + 1];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    st.w[t] = ld_stream(wrow[t] + bl);
    if (vec_sc) {
      st.sc[t] = ((const float4*)srow[t])[q];
    } else {
      st.sc[t].x = srow[t][min(4 * q + 0, nb - 1)];
      st.sc[t].y = srow[t][min(4 * q + 1, nb - 1)];
      st.sc[t].z = srow[t][min(4 * q + 2, nb - 1)];
      st.sc[t].w = srow[t][min(4 * q + 3, nb - 1)];
    }
  }
}

template <int XS_MODE, int T, int EU>
__device__ __forceinline__ void bquad_compute(const BQuad<T>& st, int q, int nb, bool m_ok, int src_w, int src_x,
                                              const float* xs_g, int M, int g, float (&acc)[T][EU]) {
  constexpr long kMinus8 = (long)0xF8F8F8F8F8F8F8F8ull;
  // A operand: lane (i, g) <- load lane (m(i), g); then dword g of each block's halves
  const uint4 xa = lane_fetch4(st.xa, src_x), xb = lane_fetch4(st.xb, src_x);
  uint32_t l0 = xa.x, l1 = xa.y, l2 = xa.z, l3 = xa.w;
  uint32_t h0 = xb.x, h1 = xb.y, h2 = xb.z, h3 = xb.w;
  transpose4(l0, l1, l2, l3);
  transpose4(h0, h1, h2, h3);
  const uint32_t lj[4] = {l0, l1, l2, l3};
  const uint32_t hj[4] = {h0, h1, h2, h3};
  long a[4];
  v4i_t cm[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = m_ok ? (long)(((unsigned long)hj[j] << 32) | lj[j]) : 0L;
    const v4i_t z = {0, 0, 0, 0};
    cm[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], kMinus8, z, 0, 0, 0);
  }
  // group scales xs[m = 4e + g][4q + j]
  float xsv[4][EU];
  if (XS_MODE == NVE_XS_GROUP32_F32) {
#pragma unroll
    for (int e = 0; e < EU; ++e) {
      const float* r = xs_g + (size_t)min(4 * e + g, M - 1) * nb;
#pragma unroll
      for (int j = 0; j < 4; ++j) xsv[j][e] = r[min(4 * q + j, nb - 1)];
    }
  }
  const bool full = 4 * q + 3 < nb;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint4 w = lane_fetch4(st.w[t], src_w);
    uint32_t c0 = w.x, c1 = w.y, c2 = w.z, c3 = w.w;
    transpose4(c0, c1, c2, c3);
    const uint32_t cj[4] = {c0, c1, c2, c3};
    const uint4 sw = lane_fetch4(make_uint4(__float_as_uint(st.sc[t].x), __float_as_uint(st.sc[t].y),
                                            __float_as_uint(st.sc[t].z), __float_as_uint(st.sc[t].w)),
                                 src_w);
    float scj[4] = {__uint_as_float(sw.x), __uint_as_float(sw.y), __uint_as_float(sw.z), __uint_as_float(sw.w)};
    // blocks past the end (last quad only) were loaded clamped: weight them 0
#pragma unroll
    for (int j = 1; j < 4; ++j) scj[j] = (full || 4 * q + j < nb) ? scj[j] : 0.0f;
    v4i_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = cj[j] & 0x0F0F0F0Fu, hi = (cj[j] >> 4) & 0x0F0F0F0Fu;
      d[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], (long)(((unsigned long)hi << 32) | lo), cm[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < EU; ++e) {
        const float f = XS_MODE == NVE_XS_GROUP32_F32 ? scj[j] * xsv[j][e] : scj[j];
        acc[t][e] = fmaf(f, (float)d[j][e], acc[t][e]);
      }
  }
}

template <int OUT_DT, int XS_MODE, int KS, int T, int EU>
__global__ __launch_bounds__(64 * KS) void w4a8_batched_mfma_kernel(int M, const int8_t* __restrict__ xq,
                                                                    const void* __restrict__ xs,
                                                                    const uint8_t* __restrict__ nib,
                                                                    const float* __restrict__ ws,
                                                                    void* __restrict__ out, int N, int K,
                                                                    int vec_sc) {
  __shared__ float s_red[KS][T * 16][4 * EU + 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;  // operand layout
  const int lr = lane >> 2, lp = lane & 3;  // load layout: 4 consecutive lanes per row
  const int row0 = blockIdx.x * (16 * T);
  const int nb = K >> 5;
  const int nq = (nb + 3) >> 2;
  const size_t row_bytes = (size_t)(K >> 1);
  const uint4* wrow[T];
  const float* srow[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int r = min(row0 + 16 * t + lr, N - 1);
    wrow[t] = (const uint4*)(nib + (size_t)r * row_bytes);
    srow[t] = ws + (size_t)r * nb;
  }
  const uint4* xrow = (const uint4*)(xq + (size_t)min(lr, M - 1) * K);
  const int am = 4 * (nl & 3) + (nl >> 2);  // activation row of A row nl
  const bool m_ok = am < M;
  const int src_w = 4 * nl + g;  // load lane holding (weight row nl, piece g)
  const int src_x = 4 * am + g;  // load lane holding (activation row am, piece g)
  float acc[T][EU];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int e = 0; e < EU; ++e) acc[t][e] = 0.0f;
  for (int q = wave; q < nq; q += KS) {
    BQuad<T> st;
    bquad_issue<T>(st, xrow, wrow, srow, vec_sc != 0, q, nq, nb, lp);
    bquad_compute<XS_MODE, T, EU>(st, q, nb, m_ok, src_w, src_x, (const float*)xs, M, g, acc);
  }
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int e = 0; e < EU; ++e) s_red[wave][16 * t + nl][4 * e + g] = acc[t][e];
  __syncthreads();
  for (int i = threadIdx.x; i < T * 16 * 4 * EU; i += 64 * KS) {
    const int mm = i / (16 * T), r = i % (16 * T);
    float y = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < KS; ++w2) y += s_red[w2][r][mm];
    if (mm < M && row0 + r < N) {
      if (XS_MODE == NVE_XS_ROW_BF16) y *= bf16_bits_to_f32(((const uint16_t*)xs)[mm]);
      store_out<OUT_DT>(out, (size_t)mm * N + row0 + r, y);
    }
  }
}


// ---------------------------------------------------------------------------
// LDS-ring int8 MFMA kernel (M >= 2, K % 128 == 0, N <= 256 * 64).
//
// Same operand mapping as the kernel above; what changes is how the bytes reach the
// operand lanes.  The register kernel moves every loaded dword to its operand lane
// with ds_bpermute (about 200 instructions per wave and quad at one tile) and holds its
// loads in VGPRs.  Here every load is a global -> LDS transfer (global_load_lds, no
// VGPRs in flight) into a per-wave ring of S slots, each holding one K quad:
//   W  T x 1 KiB   weight tile t, the row-major load layout (16 rows x 64 B, 4 lanes per row)
//   SC T x 256 B   the tile's 16 x 4 block scales (row-major)
//   A  MA x 1 KiB  activation rows 8a..8a+7, 128 B each (blocks 4q..4q+3)
//   XS 256 B       (group-scale mode) the quad's 4 scales of each activation row
// and the operand lanes read the slot directly: the tile's dword g of the 4 blocks is
// one ds_read_b128 (piece g of row n) and the 4x4 permlane transpose; the activation
// operand (dword g of both halves of each block) four ds_read2_b32; the scales one
// ds_read_b128.  A transfer writes its lanes' 16 bytes contiguously, so rows sit 64 B
// (weights) or 128 B (activations) apart and a column read would hit one bank group
// (8-way and 16-way conflicts on the CU's shared LDS, which bound the kernel); the
// sources are swizzled instead -- load lane (row a, slot s) fetches weight piece
// (s - a / 2) & 3, activation row m's blocks are rotated by m % 4 -- so each transfer
// still covers whole rows (coalesced) and the operand reads are conflict-free.
// The issue is unconditional (quads past the wave's share are clamped to the last
// quad), so every quad is the same number of transfers and the waits are exact vmcnt
// immediates: S quads in flight through the steady loop, an unrolled drain.
// Workgroups take ceil(N / 256) consecutive rows each (T = ceil(rows / 16) tiles, the
// last one partly masked), so the grid is at most one workgroup per CU and every CU
// streams the same number of weight bytes; masked lanes issue no loads.
template <int T, int EU, int XS_MODE>
struct RingLayout {
  static constexpr int MA = EU == 4 ? 2 : 1;  // activation transfers per quad
  static constexpr int XG = XS_MODE == NVE_XS_GROUP32_F32 ? 1 : 0;
  static constexpr int W = 0, SC = T * 1024, A = SC + T * 256, XS = A + MA * 1024;
  static constexpr int SLOT = XS + XG * 256;
  static constexpr int LOADS = 2 * T + MA + XG;  // vmcnt events per quad
};

template <int OUT_DT, int XS_MODE, int KS, int T, int EU, int S>
__global__ __launch_bounds__(64 * KS) void w4a8_batched_mfma_lds_kernel(int M, const int8_t* __restrict__ xq,
                                                                        const void* __restrict__ xs,
                                                                        const uint8_t* __restrict__ nib,
                                                                        const float* __restrict__ ws,
                                                                        void* __restrict__ out, int N, int K,
                                                                        int rows_per_wg) {
  static_assert(S >= 1 && S <= 4, "ring depth");
  using L = RingLayout<T, EU, XS_MODE>;
  constexpr int kRing = KS * S * L::SLOT;
  constexpr int kRed = KS * T * 16 * (4 * EU + 1) * 4;
  __shared__ __attribute__((aligned(16))) char smem[kRing > kRed ? kRing : kRed];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nl = lane & 15, g = lane >> 4;  // operand layout
  const int lr = lane >> 2, lp = lane & 3;  // load layout
  const int row0 = blockIdx.x * rows_per_wg;
  const int nb = K >> 5, nq = nb >> 2;
  const int nqw = (nq + KS - 1) / KS;  // quads per wave (the host guarantees nqw >= S)
  char* const ring = smem + wave * (S * L::SLOT);

  // per-lane sources at quad 0 (advanced by the quad index at issue)
  const uint8_t* wsrc[T];
  const float* ssrc[T];
  bool wok[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int rr = 16 * t + lr;
    const int r = min(row0 + rr, N - 1);
    // masked lanes load nothing; lane 0 always loads (a clamped row if need be), so no
    // transfer is skipped by the whole wave and the vmcnt immediates stay exact
    wok[t] = (rr < rows_per_wg && row0 + rr < N) || lane == 0;
    wsrc[t] = nib + (size_t)r * (K >> 1) + 16 * ((lp - (lr >> 1)) & 3);  // swizzled piece
    ssrc[t] = ws + (size_t)r * nb + lp;
  }
  const int8_t* asrc[L::MA];
  bool aok[L::MA];
#pragma unroll
  for (int a = 0; a < L::MA; ++a) {
    const int m = 8 * a + (lane >> 3);
    aok[a] = m < M;  // lane 0 holds row 0, or row 8 where a second transfer exists (M > 8)
    asrc[a] = xq + (size_t)min(m, M - 1) * K + 16 * (((lane & 7) - 2 * (lane >> 3)) & 7);  // rotated blocks
  }
  const float* xsrc = (const float*)xs + (size_t)min(lr, M - 1) * nb + lp;
  const bool xok = lr < M;

  auto issue = [&](int i) {
    const int q = min(wave + KS * i, nq - 1);
    char* const sb = ring + (i % S) * L::SLOT;
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (wok[t]) lds_dma16(wsrc[t] + 64 * q, sb + L::W + t * 1024);
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (wok[t]) lds_dma4(ssrc[t] + 4 * q, sb + L::SC + t * 256);
#pragma unroll
    for (int a = 0; a < L::MA; ++a)
      if (aok[a]) lds_dma16(asrc[a] + 128 * q, sb + L::A + a * 1024);
    if (L::XG && xok) lds_dma4(xsrc + 4 * q, sb + L::XS);
  };

  const int am = 4 * (nl & 3) + (nl >> 2);  // activation row of A row nl
  // slot offsets read by this lane (see the swizzles above): weight piece g of row nl,
  // and the lo / hi halves of block j of activation row am (rows >= M read row M - 1)
  const uint32_t rd_w = 16 * (4 * nl + ((g + (nl >> 1)) & 3));
  uint32_t rd_a[4];
  {
    const int ar = min(am, M - 1);
    const uint32_t rb = L::A + (L::MA == 2 ? (ar >> 3) * 1024 : 0) + (ar & 7) * 128 + 4 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) rd_a[j] = rb + 32 * ((j + (ar & 7)) & 3);
  }
  constexpr long kMinus8 = (long)0xF8F8F8F8F8F8F8F8ull;
  float acc[T][EU];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int e = 0; e < EU; ++e) acc[t][e] = 0.0f;

  auto compute = [&](int i) {
    if (wave + KS * i >= nq) return;  // clamped duplicate quad (wave-uniform)
    const uint32_t sb = lds_addr(ring + (i % S) * L::SLOT);
    u32x2_t ar[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ar[j] = ds_read2<0, 4>(sb + rd_a[j]);
    u32x4_t xr[EU];
    if (XS_MODE == NVE_XS_GROUP32_F32) {
#pragma unroll
      for (int e = 0; e < EU; ++e) xr[e] = ds_read128(sb + L::XS + (4 * e + g) * 16);
    }
    u32x4_t wr[T], sr[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      wr[t] = ds_read128(sb + L::W + t * 1024 + rd_w);
      sr[t] = ds_read128(sb + L::SC + t * 256 + nl * 16);
    }
    lgkm_wait();
#pragma unroll
    for (int j = 0; j < 4; ++j) tie(ar[j]);
    if (XS_MODE == NVE_XS_GROUP32_F32) {
#pragma unroll
      for (int e = 0; e < EU; ++e) tie(xr[e]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      tie(wr[t]);
      tie(sr[t]);
    }
    long a[4];
    v4i_t cm[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = (long)(((unsigned long)ar[j].y << 32) | ar[j].x);  // rows >= M: row M - 1, never stored
      const v4i_t z = {0, 0, 0, 0};
      cm[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], kMinus8, z, 0, 0, 0);
    }
    float4 xv[EU];
    if (XS_MODE == NVE_XS_GROUP32_F32) {
#pragma unroll
      for (int e = 0; e < EU; ++e)
        xv[e] = make_float4(__uint_as_float(xr[e].x), __uint_as_float(xr[e].y), __uint_as_float(xr[e].z),
                            __uint_as_float(xr[e].w));
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t c0 = wr[t].x, c1 = wr[t].y, c2 = wr[t].z, c3 = wr[t].w;
      transpose4(c0, c1, c2, c3);
      const uint32_t cj[4] = {c0, c1, c2, c3};
      const float scj[4] = {__uint_as_float(sr[t].x), __uint_as_float(sr[t].y), __uint_as_float(sr[t].z),
                            __uint_as_float(sr[t].w)};
      v4i_t d[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = cj[j] & 0x0F0F0F0Fu, hi = (cj[j] >> 4) & 0x0F0F0F0Fu;
        d[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j], (long)(((unsigned long)hi << 32) | lo), cm[j], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < EU; ++e) {
          float f = scj[j];
          if (XS_MODE == NVE_XS_GROUP32_F32) f *= (j == 0 ? xv[e].x : j == 1 ? xv[e].y : j == 2 ? xv[e].z : xv[e].w);
          acc[t][e] = fmaf(f, (float)d[j][e], acc[t][e]);
        }
    }
  };

#pragma unroll
  for (int i = 0; i < S; ++i) issue(i);
  int i = 0;
  for (; i + S < nqw; ++i) {
    wait_vmcnt<(S - 1) * L::LOADS>();
    __builtin_amdgcn_sched_barrier(0);
    compute(i);
    __builtin_amdgcn_sched_barrier(0);
    issue(i + S);
  }
#pragma unroll
  for (int k = 0; k < S; ++k) {
    if (k == 0) wait_vmcnt<(S - 1) * L::LOADS>();
    if (k == 1) wait_vmcnt<(S > 1 ? S - 2 : 0) * L::LOADS>();
    if (k == 2) wait_vmcnt<(S > 2 ? S - 3 : 0) * L::LOADS>();
    if (k == 3) wait_vmcnt<(S > 3 ? S - 4 : 0) * L::LOADS>();
    __builtin_amdgcn_sched_barrier(0);
    compute(i + k);
  }

  __syncthreads();  // every wave is done with its ring: reuse the LDS for the reduction
  float(*s_red)[T * 16][4 * EU + 1] = (float(*)[T * 16][4 * EU + 1])smem;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int e = 0; e < EU; ++e) s_red[wave][16 * t + nl][4 * e + g] = acc[t][e];
  __syncthreads();
  const int rows = min(rows_per_wg, N - row0);
  for (int x = threadIdx.x; x < T * 16 * 4 * EU; x += 64 * KS) {
    const int mm = x / (16 * T), r = x % (16 * T);
    float y = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < KS; ++w2) y += s_red[w2][r][mm];
    if (mm < M && r < rows) {
      if (XS_MODE == NVE_XS_ROW_BF16) y *= bf16_bits_to_f32(((const uint16_t*)xs)[mm]);
      store_out<OUT_DT>(out, (size_t)mm * N + row0 + r, y);
    }
  }
}

}  // namespace nve

namespace nve_host {

// The MFMA path serves M >= 2 (measured faster than v_dot4 from M = 2 on) unless
// the kernel-selection policy forces one-shot v_dot4 kernels (nve_hip_set_gemv_policy(NVE_GEMV_ONESHOT, ...)).
static bool batched_use_mfma() { return gemv_policy() != NVE_GEMV_ONESHOT; }

// 16 waves per workgroup (the K quads are dealt round-robin) and 1, 2 or 4 16-row tiles
// per workgroup: the fewest that keep the grid within one workgroup per CU (one
// 1024-thread workgroup fits a CU), since a second round of workgroups starts only as
// the first drains (8B gate, 14336 rows: 224 workgroups of 4 tiles take 10.9 / 11.2 /
// 11.8 us at M = 4 / 8 / 16 against 11.6 / 12.1 / 13.2 for 448 of 2).
template <int OUT_DT, int XS, int EU>
static hipError_t launch_mfma(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                              void* out, int N, int K, hipStream_t stream) {
  const int vec_sc = (K % 128 == 0) && aligned(ws, 16);
  constexpr int kCU = 256;
  if ((N + 15) / 16 <= kCU)
    hipLaunchKernelGGL((nve::w4a8_batched_mfma_kernel<OUT_DT, XS, 16, 1, EU>), dim3((N + 15) / 16), dim3(1024), 0,
                       stream, M, xq, xs, nib, ws, out, N, K, vec_sc);
  else if ((N + 31) / 32 <= kCU)
    hipLaunchKernelGGL((nve::w4a8_batched_mfma_kernel<OUT_DT, XS, 16, 2, EU>), dim3((N + 31) / 32), dim3(1024), 0,
                       stream, M, xq, xs, nib, ws, out, N, K, vec_sc);
  else
    hipLaunchKernelGGL((nve::w4a8_batched_mfma_kernel<OUT_DT, XS, 16, 4, EU>), dim3((N + 63) / 64), dim3(1024), 0,
                       stream, M, xq, xs, nib, ws, out, N, K, vec_sc);
  return hipGetLastError();
}

// LDS-ring kernel configuration: 16 waves per workgroup, one quad in flight per wave.
// Measured on the 8B gate (T = 4) and down (T = 1) shapes at M = 4 / 8 / 16 (us):
//   16 waves, depth 1:                 gate 9.07 / 9.30 / 10.26   down 9.16 / 9.69 / 11.25
//   16 waves, depth 2 (down):                                     down 9.21 / 10.48 / 12.21
//   16 waves, depth 3 (down), 8 waves, depth 3 (gate):
//                                      gate 9.95 / 10.31 / 10.46  down 9.73 / 10.47 / 12.34
// Deeper rings do not help (sixteen waves already keep 40-118 KiB per CU in flight).
template <int T, int EU>
struct RingCfg {
  static constexpr int KS = 16;
  static constexpr int S = 1;
};

template <int OUT_DT, int XS, int T, int EU>
static hipError_t launch_ring_t(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                                void* out, int N, int K, int rpw, hipStream_t stream) {
  using C = RingCfg<T, EU>;
  const int nq = K / 128;
  if ((nq + C::KS - 1) / C::KS < C::S) return hipErrorNotSupported;
  const int grid = (N + rpw - 1) / rpw;
  hipLaunchKernelGGL((nve::w4a8_batched_mfma_lds_kernel<OUT_DT, XS, C::KS, T, EU, C::S>), dim3(grid),
                     dim3(64 * C::KS), 0, stream, M, xq, xs, nib, ws, out, N, K, rpw);
  return hipGetLastError();
}

// hipErrorNotSupported: the shape is outside the ring kernel's range (the caller takes
// the register kernel).
template <int OUT_DT, int XS, int EU>
static hipError_t launch_ring(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                              void* out, int N, int K, hipStream_t stream) {
  constexpr int kCU = 256;
  if (K % 128 != 0 || N > kCU * 64 || !aligned(ws, 4) || !aligned(xq, 16) || !aligned(nib, 16))
    return hipErrorNotSupported;
  const int rpw = N <= 16 * kCU ? 16 : (N + kCU - 1) / kCU;
  switch ((rpw + 15) / 16) {
    case 1: return launch_ring_t<OUT_DT, XS, 1, EU>(M, xq, xs, nib, ws, out, N, K, rpw, stream);
    case 2: return launch_ring_t<OUT_DT, XS, 2, EU>(M, xq, xs, nib, ws, out, N, K, rpw, stream);
    case 3: return launch_ring_t<OUT_DT, XS, 3, EU>(M, xq, xs, nib, ws, out, N, K, rpw, stream);
    default: return launch_ring_t<OUT_DT, XS, 4, EU>(M, xq, xs, nib, ws, out, N, K, rpw, stream);
  }
}

template <int OUT_DT, int XS>
static hipError_t launch_mfma_m(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                                void* out, int N, int K, hipStream_t stream) {
  {
    const hipError_t e = M <= 4   ? launch_ring<OUT_DT, XS, 1>(M, xq, xs, nib, ws, out, N, K, stream)
                         : M <= 8 ? launch_ring<OUT_DT, XS, 2>(M, xq, xs, nib, ws, out, N, K, stream)
                                  : launch_ring<OUT_DT, XS, 4>(M, xq, xs, nib, ws, out, N, K, stream);
    if (e != hipErrorNotSupported) return e;
  }
  if (M <= 4) return launch_mfma<OUT_DT, XS, 1>(M, xq, xs, nib, ws, out, N, K, stream);
  if (M <= 8) return launch_mfma<OUT_DT, XS, 2>(M, xq, xs, nib, ws, out, N, K, stream);
  return launch_mfma<OUT_DT, XS, 4>(M, xq, xs, nib, ws, out, N, K, stream);
}

// Staged v_dot4 kernel: the one-row GEMV's tiling (R rows per wave, NJ 64-block chunks
// per lane, one staging pass), the activation rows in LDS.  It serves M = 2 outside the
// LDS-ring kernel's range where the two staged rows take at most 40 KB of LDS (8B gate
// 14336x4096: 9.2 us against 11.3 us on the register MFMA kernel; down 4096x14336: 10.4
// against 10.5).  From M = 3 the per-workgroup staging
// (every workgroup stages every row) and the M-fold LDS operand reads cost more than the
// MFMA kernel's transposes (gate M = 4: 12.1 against 11.6 us).
static constexpr int kStagedM = 2;
static size_t staged_lds_bytes(int M, int K) { return (size_t)M * nve::staged_row_int4(K) * 16; }

static bool staged_fits(int M, int N, int K) {
  if (M != kStagedM) return false;
  W4Segs s{};
  s.nseg = 1;
  s.n[0] = N;
  return !choose_w4_tiling(s, K).multi && staged_lds_bytes(M, K) <= 40 * 1024;
}

template <int OUT_DT, int XS>
static hipError_t launch_staged(int M, const int8_t* xq, const void* xs, const uint8_t* nib, const float* ws,
                                void* out, int N, int K, hipStream_t stream) {
  W4Segs s{};
  s.nseg = 1;
  s.n[0] = N;
  const W4Tiling t = choose_w4_tiling(s, K);
  const size_t lds = staged_lds_bytes(M, K);
  const int grid = (N + 4 * t.R - 1) / (4 * t.R);
#define NVE_STAGED_CASE(RR, JJ, MM)                                                                          \
  if (!MM && t.R == RR && t.NJ == JJ) {                                                                      \
    auto kern = nve::w4a8_batched_staged_kernel<OUT_DT, XS, kStagedM, RR, JJ>;                           \
    if (lds > 65536) {                                                                                       \
      hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
      if (e != hipSuccess) return e;                                                                         \
    }                                                                                                        \
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, stream, M, xq, xs, nib, ws, out, N, K);             \
    return hipGetLastError();                                                                                \
  }
  NVE_W4_TILING_CASES(NVE_STAGED_CASE)
#undef NVE_STAGED_CASE
  return hipErrorInvalidValue;
}

template <int OUT_DT>
static hipError_t launch_batched_o(int M, const int8_t* xq, const void* xs, int xs_mode,
                                   const uint8_t* nib, const float* ws, void* out, int N, int K,
                                   hipStream_t stream) {
  if (M == 1) {
    // one row: the one-shot GEMV (its staged activations and per-lane block order), with
    // the row's bf16 scale applied to the row sums in per-token mode
    W4Segs s{};
    s.nseg = 1;
    s.nib[0] = nib;
    s.sc[0] = ws;
    s.out[0] = out;
    s.n[0] = N;
    if (xs_mode == NVE_XS_ROW_BF16) return launch_w4a8_rowscale(xq, (const uint16_t*)xs, s, OUT_DT, K, stream);
    return launch_w4a8(xq, (const float*)xs, s, OUT_DT, K, stream);
  }
  if (M == 2 && batched_use_mfma()) {
    // the LDS-ring MFMA kernel where it applies (8B gate: 8.9 us against 9.3 on the
    // staged v_dot4 kernel, down 9.2 against 10.3), else the staged kernel below
    const hipError_t e = xs_mode == NVE_XS_ROW_BF16
                             ? launch_ring<OUT_DT, NVE_XS_ROW_BF16, 1>(M, xq, xs, nib, ws, out, N, K, stream)
                             : launch_ring<OUT_DT, NVE_XS_GROUP32_F32, 1>(M, xq, xs, nib, ws, out, N, K, stream);
    if (e != hipErrorNotSupported) return e;
  }
  if (staged_fits(M, N, K)) {
    if (xs_mode == NVE_XS_ROW_BF16)
      return launch_staged<OUT_DT, NVE_XS_ROW_BF16>(M, xq, xs, nib, ws, out, N, K, stream);
    return launch_staged<OUT_DT, NVE_XS_GROUP32_F32>(M, xq, xs, nib, ws, out, N, K, stream);
  }
  if (batched_use_mfma()) {
    if (xs_mode == NVE_XS_ROW_BF16)
      return launch_mfma_m<OUT_DT, NVE_XS_ROW_BF16>(M, xq, xs, nib, ws, out, N, K, stream);
    return launch_mfma_m<OUT_DT, NVE_XS_GROUP32_F32>(M, xq, xs, nib, ws, out, N, K, stream);
  }
  const dim3 grid((N + 3) / 4);
  if (xs_mode == NVE_XS_ROW_BF16)
    hipLaunchKernelGGL((nve::w4a8_batched_dot4_kernel<OUT_DT, NVE_XS_ROW_BF16>), grid, dim3(256), 0, stream,
                       M, xq, xs, nib, ws, out, N, K);
  else
    hipLaunchKernelGGL((nve::w4a8_batched_dot4_kernel<OUT_DT, NVE_XS_GROUP32_F32>), grid, dim3(256), 0,
                       stream, M, xq, xs, nib, ws, out, N, K);
  return hipGetLastError();
}

hipError_t launch_w4a8_batched(int M, const int8_t* xq, const void* xs, int xs_mode,
                               const uint8_t* nib, const float* ws, void* out, int out_dt, int N,
                               int K, hipStream_t stream) {
  switch (out_dt) {
    case NVE_DT_F16: return launch_batched_o<NVE_DT_F16>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
    case NVE_DT_BF16: return launch_batched_o<NVE_DT_BF16>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
    default: return launch_batched_o<NVE_DT_F32>(M, xq, xs, xs_mode, nib, ws, out, N, K, stream);
  }
}

}  // namespace nve_host
