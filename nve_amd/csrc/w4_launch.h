// w4_launch.h -- workgroup tiling shared by the W4A8 and W4A16 GEMV launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Up to three weight matrices that share one activation vector and K (Q/K/V).
// Workgroups [wg_begin[s], wg_begin[s+1]) compute matrix s.
struct W4Segs {
  const uint8_t* nib[3];
  const float* sc[3];
  const float* awq[3];
  void* out[3];
  int n[3];
  int wg_begin[3];
  int nseg;
  int wg_total;
};

struct W4Tiling {
  int R;   // output rows per wave
  int NJ;  // 64-block chunks per lane held in registers at once
  bool multi;  // K needs more than one pass of NJ chunks
};

// Rows per wave are chosen so a lane keeps about 8 blocks (160 B) of weights in
// flight, then halved while the launch would have fewer than 512 workgroups (two per
// CU of the 256-CU MI355X).
inline W4Tiling choose_w4_tiling(const W4Segs& s, int K) {
  const int nb = K / 32;
  int nj = (nb + 63) / 64;
  const bool multi = nj > 8;
  if (multi) nj = 8;
  int r = nj == 1 ? 8 : (nj == 2 ? 4 : (nj <= 4 ? 2 : 1));
  long ntot = 0;
  for (int i = 0; i < s.nseg; ++i) ntot += s.n[i];
  while (r > 1 && (ntot + 4L * r - 1) / (4L * r) < 512) r /= 2;
  return W4Tiling{r, nj, multi};
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

namespace nve_host {
hipError_t launch_w4a8(const int8_t* xq, const float* xs, const W4Segs& segs, int out_dt, int K,
                       hipStream_t stream);
hipError_t launch_w4a8_block_acc(const int8_t* xq, const uint8_t* nib, int32_t* acc, int N, int K,
                                 hipStream_t stream);
hipError_t launch_w4a16(const void* x, int x_dt, const W4Segs& segs, int out_dt, int K,
                        hipStream_t stream);
}  // namespace nve_host
