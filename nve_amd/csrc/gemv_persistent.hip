// gemv_persistent.hip -- instantiations and launchers of the persistent W4A8 / W4A16
// GEMV kernels (w4_persistent.h).  Used when a launch has enough row tiles to give
// every wave of the grid several of them; smaller launches use the one-shot kernels.
#include <stdlib.h>

#include "w4_persistent.h"
#include "w4a16_ops.h"
#include "w4a8_ops.h"

namespace nve_host {

// Kernel-selection policy (nve_hip_set_gemv_policy): 0 auto, 1 one-shot only,
// 2 persistent whenever the shape allows it.  Workgroups per CU of the persistent grid.
static int g_policy = NVE_GEMV_AUTO;
static int g_occ = 2;
static int g_depth = 4;

int gemv_policy() { return g_policy; }
int persistent_occupancy() { return g_occ; }
int persistent_depth() { return g_depth; }

void set_gemv_policy(int policy, int occ, int depth) {
  g_policy = policy;
  if (occ > 0) g_occ = occ > 8 ? 8 : occ;
  if (depth > 0) g_depth = depth >= 8 ? 8 : 4;
}

static constexpr int kNumCU = 256;  // MI355X

// AUTO picks per precision from measurements on MI355X (8B layer shapes, weights
// streamed from HBM): the W4A8 kernel is light on VALU and its one-shot form stays
// closest to the streaming floor at every shape; the W4A16 kernel (about twice the
// VALU work per block) gains from the persistent form with one workgroup per CU where
// the one-shot form's K-long LDS staging limits its workgroups per CU (K > 8192: 8B
// down 9.0 against 10.0 us), and loses at lm_head size and, with a balanced one-shot
// grid, at the K = 4096 shapes (8B gate 8.1 one-shot against 8.4 us).
bool use_persistent(const W4Segs& s0, int K, bool w4a16) {
  if (g_policy == NVE_GEMV_ONESHOT || K / 32 > 64 * 8) return false;
  W4Segs s = s0;
  if (g_policy == NVE_GEMV_PERSISTENT) {
    const W4Tiling t = choose_persistent_tiling(K, g_depth);
    return plan_persistent(s, t.R, 4 * kNumCU * g_occ) > 0;
  }
  if (!w4a16 || K <= 8192) return false;
  long rows = 0;
  for (int i = 0; i < s.nseg; ++i) rows += s.n[i];
  const W4Tiling t = choose_persistent_tiling(K, 4);
  if (plan_persistent(s, t.R, 4 * kNumCU) <= 0) return false;
  return s.tiles_total >= 4 * 4 * kNumCU && rows <= 65536;
}

static int launch_occ() { return g_policy == NVE_GEMV_PERSISTENT ? g_occ : 1; }
static int launch_depth() { return g_policy == NVE_GEMV_PERSISTENT ? g_depth : 4; }

template <class P, int OUT_DT, int R, int NJ>
static hipError_t launch_p(const typename P::Args& a, W4Segs segs, int K, hipStream_t stream) {
  const size_t lds = P::lds_bytes(K) + 4 * (size_t)nve::kMaxTilesPerWave * R * sizeof(float);
  auto kern = nve::w4_persistent_kernel<P, OUT_DT, R, NJ>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  const int grid = plan_persistent(segs, R, 4 * kNumCU * launch_occ());
  if (grid <= 0) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, stream, a, segs, K);
  return hipGetLastError();
}

template <class P, int OUT_DT>
static hipError_t launch_p_dt(const typename P::Args& a, W4Segs segs, int K, hipStream_t stream) {
  const W4Tiling t = choose_persistent_tiling(K, launch_depth());
#define NVE_P_CASE(RR, JJ) \
  if (t.R == RR && t.NJ == JJ) return launch_p<P, OUT_DT, RR, JJ>(a, segs, K, stream);
  NVE_W4_PERSISTENT_CASES(NVE_P_CASE)
#undef NVE_P_CASE
  return hipErrorInvalidValue;
}

template <class P>
static hipError_t launch_p_any(const typename P::Args& a, const W4Segs& segs, int out_dt, int K,
                               hipStream_t stream) {
  switch (out_dt) {
    case NVE_DT_F16: return launch_p_dt<P, NVE_DT_F16>(a, segs, K, stream);
    case NVE_DT_BF16: return launch_p_dt<P, NVE_DT_BF16>(a, segs, K, stream);
    case NVE_DT_F32_ACCUM: return launch_p_dt<P, NVE_DT_F32_ACCUM>(a, segs, K, stream);
    default: return launch_p_dt<P, NVE_DT_F32>(a, segs, K, stream);
  }
}

hipError_t launch_w4a8_persistent(const int8_t* xq, const float* xs, W4Segs segs, int out_dt, int K,
                                  hipStream_t stream) {
  const nve::W4A8Policy::Args a{xq, xs};
  return launch_p_any<nve::W4A8Policy>(a, segs, out_dt, K, stream);
}

hipError_t launch_w4a16_persistent(const void* x, int x_dt, W4Segs segs, int out_dt, int K,
                                   hipStream_t stream) {
  if (x_dt == NVE_DT_BF16) {
    const nve::W4A16Policy<nve::MODE_BF16>::Args a{x};
    return launch_p_any<nve::W4A16Policy<nve::MODE_BF16>>(a, segs, out_dt, K, stream);
  }
  const nve::W4A16Policy<nve::MODE_F16>::Args a{x};
  return launch_p_any<nve::W4A16Policy<nve::MODE_F16>>(a, segs, out_dt, K, stream);
}

}  // namespace nve_host
