// w4_launch.h -- workgroup tiling shared by the W4A8 and W4A16 GEMV launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nve_kernels.h"

// Up to three weight matrices that share one activation vector and K (Q/K/V).
// Workgroups [wg_begin[s], wg_begin[s+1]) compute matrix s.
struct W4Segs {
  const uint8_t* nib[3];
  const float* sc[3];
  const float* awq[3];
  void* out[3];
  int n[3];
  int wg_begin[3];    // one-shot kernels: first workgroup of each matrix
  int nseg;
  int wg_total;
  int tile_begin[4];  // persistent kernels: first R-row tile of each matrix (+ end)
  int tiles_total;
  int wave_begin[4];  // persistent kernels: first wave of each matrix (+ end)
};

struct W4Tiling {
  int R;   // output rows per wave
  int NJ;  // 64-block chunks per lane held in registers at once
  bool multi;  // K needs more than one pass of NJ chunks
};

// Excess of the busiest CU over the mean when `wgs` one-shot workgroups are dealt to
// the 256 CUs (1.0 = every CU gets the same number).
inline double w4_grid_imbalance(long wgs) {
  const long rounds = (wgs + 255) / 256;
  return (double)(rounds * 256) / (double)wgs;
}

// Rows per wave are chosen so a lane keeps about 8 blocks (160 B) of weights in
// flight, then halved while the launch would have fewer than 512 workgroups (two per
// CU of the 256-CU MI355X), and halved again while that evens out the workgroups per
// CU: all of a one-shot grid is resident at once, and a CU holding one workgroup more
// than the others finishes a workgroup's latency later (8B gate, 14336 rows: 896
// workgroups = 3.5 per CU at 4 rows per wave, 7.23 us W4A8 / 8.72 us W4A16; 1792 = 7
// per CU at 2 rows, 7.05 / 8.11 us).
inline W4Tiling choose_w4_tiling(const W4Segs& s, int K) {
  const int nb = K / 32;
  int nj = (nb + 63) / 64;
  const bool multi = nj > 8;
  if (multi) nj = 8;
  int r = nj == 1 ? 8 : (nj == 2 ? 4 : (nj <= 4 ? 2 : 1));
  long ntot = 0;
  for (int i = 0; i < s.nseg; ++i) ntot += s.n[i];
  auto wgs = [&](int rr) {
    long w = 0;
    for (int i = 0; i < s.nseg; ++i) w += (s.n[i] + 4L * rr - 1) / (4L * rr);
    return w;
  };
  while (r > 1 && (ntot + 4L * r - 1) / (4L * r) < 512) r /= 2;
  while (r > 1 && w4_grid_imbalance(wgs(r)) > 1.05 && w4_grid_imbalance(wgs(r / 2)) < w4_grid_imbalance(wgs(r)))
    r /= 2;
  return W4Tiling{r, nj, multi};
}

// Launches whose staging merges the key-split attention partials (o_proj after split
// attention): every workgroup reads the partial records of every head, so that work
// grows with the number of workgroups; these take the largest R of the table for their
// NJ (fewest workgroups) instead of filling 512 workgroups.
inline W4Tiling choose_merge_tiling(const W4Segs& s, int K) {
  W4Tiling t = choose_w4_tiling(s, K);
  t.R = t.NJ == 1 ? 8 : (t.NJ == 2 ? 4 : (t.NJ <= 4 ? 2 : 1));
  return t;
}

inline void finalize_segments(W4Segs& s, int R) {
  int wg = 0;
  for (int i = 0; i < 3; ++i) {
    s.wg_begin[i] = wg;
    if (i < s.nseg) wg += (s.n[i] + 4 * R - 1) / (4 * R);
  }
  s.wg_total = wg;
}

// Every (R, NJ) pair choose_w4_tiling can return.
#define NVE_W4_TILING_CASES(X)                                                           \
  X(8, 1, false) X(4, 1, false) X(2, 1, false) X(1, 1, false) X(4, 2, false) X(2, 2, false) \
  X(1, 2, false) X(2, 3, false) X(1, 3, false) X(2, 4, false) X(1, 4, false) X(1, 5, false) \
  X(1, 6, false) X(1, 7, false) X(1, 8, false) X(1, 8, true)

// (R, NJ) pairs of the SwiGLU-paired launches (R even: R/2 gate + R/2 up rows).
#define NVE_W4_SWIGLU_CASES(X) \
  X(8, 1) X(4, 1) X(2, 1) X(4, 2) X(2, 2) X(2, 3) X(2, 4) X(2, 5) X(2, 6) X(2, 7) X(2, 8)

// Persistent kernels: R*NJ ~ depth (4 or 8) blocks per lane per buffer, two buffers.
inline W4Tiling choose_persistent_tiling(int K, int depth) {
  const int nb = K / 32;
  const int nj = (nb + 63) / 64;
  int r;
  if (depth >= 8)
    r = nj == 1 ? 8 : (nj == 2 ? 4 : (nj <= 4 ? 2 : 1));
  else
    r = nj == 1 ? 4 : (nj == 2 ? 2 : 1);
  return W4Tiling{r, nj, false};
}

inline void finalize_tiles(W4Segs& s, int R) {
  int t = 0;
  for (int i = 0; i < 4; ++i) {
    s.tile_begin[i] = t;
    if (i < s.nseg) t += (s.n[i] + R - 1) / R;
  }
  s.tiles_total = t;
}

// Split `waves` between the matrices in proportion to their tiles (at least one wave
// each, never more waves than tiles); returns the number of waves actually used.
inline int assign_waves(W4Segs& s, int waves) {
  int used = 0;
  for (int i = 0; i < 4; ++i) {
    s.wave_begin[i] = used;
    if (i < s.nseg) {
      const int ti = s.tile_begin[i + 1] - s.tile_begin[i];
      long w = ((long)waves * ti + s.tiles_total - 1) / s.tiles_total;
      if (w < 1) w = 1;
      if (w > ti) w = ti;
      used += (int)w;
    }
  }
  return used;
}

// The rows of one wave all come from one matrix: the host splits the grid's waves
// between the matrices of a grouped launch in proportion to their tile counts
// (W4Segs::wave_begin), so the segment lookup happens once per wave, outside the
// tile loop, and the loop itself is pure scalar arithmetic on an SGPR tile index.
struct W4Wave {
  const uint8_t* nib;
  const float* ws;
  void* out;
  int n;
  int t0;      // first tile of this wave within its matrix
  int stride;  // waves assigned to the matrix
  int tiles;   // tiles of the matrix
};

// Waves past the last assigned one (the grid is a whole number of 4-wave workgroups)
// are idle: they map onto wave 0's matrix with no tiles, so their one unconditional
// prefetch reads tile 0 of a real matrix and nothing else runs.  Segments >= nseg
// have wave_begin == wave_begin[nseg], so no active wave can select them.
__host__ __device__ inline W4Wave resolve_wave(const W4Segs& g, int w) {
  const int wtot = g.wave_begin[g.nseg];
  const bool idle = w >= wtot;
  const int wc = idle ? 0 : w;
  const int sg = wc >= g.wave_begin[2] ? 2 : (wc >= g.wave_begin[1] ? 1 : 0);
  W4Wave r;
  r.nib = g.nib[sg];
  r.ws = g.sc[sg];
  r.out = g.out[sg];
  r.n = g.n[sg];
  r.t0 = wc - g.wave_begin[sg];
  r.stride = g.wave_begin[sg + 1] - g.wave_begin[sg];
  r.tiles = idle ? 0 : g.tile_begin[sg + 1] - g.tile_begin[sg];
  return r;
}

// Persistent tile results parked per wave in LDS (see w4_persistent.h).
constexpr int kPersistentMaxTilesPerWave = 8;

// Grid plan of a persistent launch: fills tile_begin / wave_begin and returns the
// number of 4-wave workgroups (0 if the shape cannot be planned within the per-wave
// tile limit).  Wave w of the grid runs tiles t0, t0+stride, ... of its matrix.
inline int plan_persistent(W4Segs& s, int R, int waves_wanted) {
  finalize_tiles(s, R);
  int waves = waves_wanted;
  const int min_waves = (s.tiles_total + kPersistentMaxTilesPerWave - 1) / kPersistentMaxTilesPerWave + s.nseg;
  if (waves < min_waves) waves = min_waves;
  waves = assign_waves(s, waves);
  for (int i = 0; i < s.nseg; ++i) {
    const int ti = s.tile_begin[i + 1] - s.tile_begin[i];
    const int wi = s.wave_begin[i + 1] - s.wave_begin[i];
    if (wi < 1 || (ti + wi - 1) / wi > kPersistentMaxTilesPerWave) return 0;
  }
  return (waves + 3) / 4;
}

#define NVE_W4_PERSISTENT_CASES(X) \
  X(8, 1) X(4, 1) X(4, 2) X(2, 2) X(2, 3) X(1, 3) X(2, 4) X(1, 4) X(1, 5) X(1, 6) X(1, 7) X(1, 8)

namespace nve_host {
// Workgroups per CU for the persistent kernels (NVE_PERSISTENT_OCC overrides; 0 turns
// the persistent kernels off).
int persistent_occupancy();
int persistent_depth();
int gemv_policy();
void set_gemv_policy(int policy, int occ, int depth);
bool use_persistent(const W4Segs& s, int K, bool w4a16);
hipError_t launch_w4a8_persistent(const int8_t* xq, const float* xs, W4Segs segs, int out_dt, int K,
                                  hipStream_t stream);
hipError_t launch_w4a16_persistent(const void* x, int x_dt, W4Segs segs, int out_dt, int K,
                                   hipStream_t stream);
size_t decode_workspace_bytes(const nve_decode_config& c);
int check_decode(const nve_decode_config& c);
int layer_forward_decode(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io,
                         bool w4a8, hipStream_t s);
int decode_head(const nve_decode_config& c, const nve_decode_head& hd, bool w4a8, hipStream_t s);
int decode_stage(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io, bool w4a8,
                 int stage, const void* in, void* out, hipStream_t s);
int attn_splits(const nve_decode_config& c);
int layer_forward_decode_noalloc(const nve_decode_config& c, const nve_layer_weights& w, const nve_decode_io& io,
                                 bool w4a8, hipStream_t s);
// Fused-producer GEMVs (act_producer.h).
}  // namespace nve_host
namespace nve {
struct ProdArgs;
struct EpiArgs;
}
namespace nve_host {
// pair: nve::PAIR_NONE / PAIR_SWIGLU / PAIR_ROPE (act_producer.h); ra is read by PAIR_ROPE only.
hipError_t launch_w4a8_fused(int src, int pair, const nve::ProdArgs& pa, const W4Segs& segs, int out_dt, int K,
                             hipStream_t stream, const nve::EpiArgs& ra);
hipError_t launch_w4a16_fused(int src, int pair, const nve::ProdArgs& pa, const W4Segs& segs, int out_dt, int K,
                              hipStream_t stream, const nve::EpiArgs& ra);
// Large-M W4A16 GEMM (gemm_w4a16_tile.hip): K % 128 == 0, M K < 2^30, N K / 2 < 2^31;
// gemm_tile_grid128 = its workgroup count with 128-row tiles.
bool gemm_tile_fits(int M, int N, int K, bool awq);
long gemm_tile_grid128(int M, int N);
// fp32 partial bytes of its K split where the 128-row grid leaves CUs idle (0: no split)
size_t gemm_tile_parts_bytes(int M, int N, int K);
hipError_t launch_gemm_w4a16_tile(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                  const float* awq, void* out, int out_dt, int N, int K, float* parts,
                                  size_t parts_bytes, hipStream_t s);
hipError_t launch_embed(const uint16_t* embed, const int* token, float* hidden, int H, int vocab, hipStream_t s);
hipError_t launch_w4a8(const int8_t* xq, const float* xs, const W4Segs& segs, int out_dt, int K,
                       hipStream_t stream);
hipError_t launch_w4a8_rowscale(const int8_t* xq, const uint16_t* row_scale, const W4Segs& segs, int out_dt, int K,
                                hipStream_t stream);
// One-shot W4A8 GEMV to f32 logits that also writes each workgroup's greedy candidate
// (PAIR_ARGMAX) to arg_v / arg_i; *ncand = the number of workgroups (<= ceil(N / 4)).
hipError_t launch_w4a8_argmax(const int8_t* xq, const float* xs, const W4Segs& segs, int K, float* arg_v,
                              int* arg_i, int* ncand, hipStream_t stream);
hipError_t launch_w4a8_block_acc(const int8_t* xq, const uint8_t* nib, int32_t* acc, int N, int K,
                                 hipStream_t stream);
hipError_t launch_w4a16(const void* x, int x_dt, const W4Segs& segs, int out_dt, int K,
                        hipStream_t stream);
}  // namespace nve_host
