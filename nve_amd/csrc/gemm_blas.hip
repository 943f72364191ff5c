// gemm_blas.hip -- the reference's own prefill method for large M.
//
// GpuWeight::matmul_x (src/gpu_layer.rs:219-237) expands the int4 weights to a dense
// 16-bit matrix with nve_dequant_w4a16 and multiplies with the vendor GEMM.  The fused
// kernels (gemm_w4a16.hip, gemm_w4a16_tile.hip) win up to M = 512; they re-dequantize
// each weight slice once per activation row block, so above M = 512 the reference's
// two-step method is the faster one on this part.  nve_hip_gemm_w4a16_ws
// takes that path when the caller provides the workspace: the weights are dequantized
// into it (dequant_w4_kernel, bit-identical to the reference dequant) and hipBLASLt
// computes Y = X W^T with fp32 accumulation.  Column-major view: D (N x M, ld N) =
// op(A) op(B) with A = the dequantized W seen as K x N (ld K, transposed) and B = X
// seen as K x M (ld K), which is the row-major Y [M, N].
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "common.h"
#include "w4_launch.h"

namespace nve_host {

hipError_t launch_gemm_w4a16(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc, const float* awq,
                             void* out, int out_dt, int N, int K, hipStream_t s);
hipError_t launch_dequant_w4(const uint8_t* nib, const float* scales, const float* awq, void* out, int out_dt,
                             int N, int K, hipStream_t stream);
hipError_t launch_gemm_w4a16_parts(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                   const float* awq, void* out, int out_dt, int N, int K, float* parts,
                                   size_t parts_bytes, hipStream_t s);
size_t gemm_split_parts_bytes(int M, int N, int K);

namespace {

// from here on dequant + GEMM is faster (fp16 out, us: 8B gate M = 640 96.8 against 145.9
// for the tile kernel, 8B down 116.2 against 135.5; at M = 384-512 the two are within 10%,
// the tile kernel ahead at down); with AWQ factors from 385 rows, where the tile kernel's
// extra multiply and factor reads put it behind at the gate (fp32 out, M = 512: 88.0 against
// 80.8; down 103.1 against 104.5)
constexpr int kGemmBlasMinM = 513;
constexpr int kGemmBlasMinMAwq = 385;
constexpr size_t kBlasWorkspace = 32u << 20;
constexpr int kBlasCandidates = 32;  // heuristic candidates timed on the first call per shape
constexpr int kBlasTimedRuns = 5;    // timed runs per candidate (after one untimed run)

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

hipDataType blas_type(int nve_dt) {
  return nve_dt == NVE_DT_F16 ? HIP_R_16F : (nve_dt == NVE_DT_BF16 ? HIP_R_16BF : HIP_R_32F);
}

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;                                     // per device
// Selected algorithm per (dev, M, N, K, x, out); ok == false marks a shape for which no
// candidate ran (that shape is served by the fused kernel from then on).
struct AlgoChoice {
  bool ok;
  hipblasLtMatmulAlgo_t algo;
};
std::map<std::tuple<int, int, int, int, int, int>, AlgoChoice> g_algo;

struct Descs {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  ~Descs() {
    if (d) hipblasLtMatrixLayoutDestroy(d);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (op) hipblasLtMatmulDescDestroy(op);
  }
};

bool make_descs(Descs& ds, int M, int N, int K, int x_dt, int out_dt) {
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  return hipblasLtMatmulDescCreate(&ds.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) ==
             HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(ds.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) ==
             HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&ds.a, blas_type(x_dt), K, N, K) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&ds.b, blas_type(x_dt), K, M, K) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&ds.d, blas_type(out_dt), N, M, N) == HIPBLAS_STATUS_SUCCESS;
}

// Heuristic candidates for the shape, each timed (kBlasTimedRuns runs after one untimed
// run) on the caller's stream; only
// a candidate in the success state, within the workspace limit, whose runs all
// returned success can be chosen.  ok == false when none qualifies (or no candidate
// exists).  A single candidate is still run once to check it.  `out` and the
// dequantized-weight part of `ws` hold scratch until the caller's product overwrites
// them.
AlgoChoice select_algo(hipblasLtHandle_t h, const Descs& ds, const void* x, void* ws, void* out,
                       const uint8_t* nib, const float* sc, const float* awq, int x_dt, int N, int K,
                       hipStream_t s, hipError_t* err) {
  *err = hipSuccess;
  AlgoChoice none{false, {}};
  hipblasLtMatmulPreference_t pref = nullptr;
  const uint64_t wsz = kBlasWorkspace;
  hipblasLtMatmulHeuristicResult_t res[kBlasCandidates];
  int found = 0;
  const bool ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz,
                                                        sizeof wsz) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulAlgoGetHeuristic(h, ds.op, ds.a, ds.b, ds.d, ds.d, pref, kBlasCandidates, res,
                                                  &found) == HIPBLAS_STATUS_SUCCESS &&
                  found > 0;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!ok) return none;
  *err = launch_dequant_w4(nib, sc, awq, ws, x_dt, N, K, s);
  if (*err != hipSuccess) return none;
  void* bws = (char*)ws + round256((size_t)N * K * 2);
  const float alpha = 1.0f, beta = 0.0f;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return none;
  if (hipEventCreate(&e1) != hipSuccess) {
    hipEventDestroy(e0);
    return none;
  }
  int best = -1;
  float best_ms = 1e30f;
  for (int c = 0; c < found; ++c) {
    if (res[c].state != HIPBLAS_STATUS_SUCCESS || res[c].workspaceSize > kBlasWorkspace) continue;
    bool run_ok = hipblasLtMatmul(h, ds.op, &alpha, ws, ds.a, x, ds.b, &beta, out, ds.d, out, ds.d, &res[c].algo,
                                  bws, kBlasWorkspace, s) == HIPBLAS_STATUS_SUCCESS;
    hipEventRecord(e0, s);
    for (int r = 0; run_ok && r < kBlasTimedRuns; ++r)
      run_ok = hipblasLtMatmul(h, ds.op, &alpha, ws, ds.a, x, ds.b, &beta, out, ds.d, out, ds.d, &res[c].algo,
                               bws, kBlasWorkspace, s) == HIPBLAS_STATUS_SUCCESS;
    hipEventRecord(e1, s);
    float ms = 1e30f;
    const bool synced = hipEventSynchronize(e1) == hipSuccess;
    run_ok = run_ok && synced && hipGetLastError() == hipSuccess;
    if (run_ok) hipEventElapsedTime(&ms, e0, e1);
    if (run_ok && (best < 0 || ms < best_ms)) {
      best_ms = ms;
      best = c;
    }
  }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (best < 0) return none;
  return AlgoChoice{true, res[best].algo};
}

}  // namespace

// Below kGemmBlasMinMAwq: the fp32 partials of the fused kernels' K split (0 when that
// shape does not split); from it on also room for the dequantized weights + the hipBLASLt
// workspace (used from kGemmBlasMinM, or kGemmBlasMinMAwq with AWQ factors).
size_t gemm_w4a16_ws_bytes(int M, int N, int K) {
  if (M < kGemmBlasMinMAwq) return round256(gemm_split_parts_bytes(M, N, K));
  const size_t blas = round256((size_t)N * K * 2) + kBlasWorkspace;
  const size_t parts = round256(gemm_split_parts_bytes(M, N, K));
  return blas > parts ? blas : parts;
}

// Dequant + hipBLASLt when M >= kGemmBlasMinM (kGemmBlasMinMAwq with AWQ factors), the
// workspace is large enough and the output is F32 or x's dtype; otherwise the fused
// kernel.  The first call per device and
// shape creates the hipBLASLt handle and picks the fastest of up to kBlasCandidates
// heuristic algorithms by timing them on the caller's stream; under graph capture a
// device or shape without that state takes the fused kernel instead.
hipError_t launch_gemm_w4a16_ws(const void* x, int x_dt, int M, const uint8_t* nib, const float* sc,
                                const float* awq, void* out, int out_dt, int N, int K, void* ws, size_t ws_bytes,
                                hipStream_t s) {
  // the fused kernel, with its K-split partials (if any) in the workspace: added in a
  // fixed order, so the result does not vary between calls
  auto fused = [&]() {
    return launch_gemm_w4a16_parts(x, x_dt, M, nib, sc, awq, out, out_dt, N, K, (float*)ws, ws ? ws_bytes : 0, s);
  };
  const int blas_min = awq ? kGemmBlasMinMAwq : kGemmBlasMinM;
  const size_t need = M >= blas_min ? round256((size_t)N * K * 2) + kBlasWorkspace : 0;
  if (need == 0 || ws == nullptr || ws_bytes < need || (out_dt != NVE_DT_F32 && out_dt != x_dt)) return fused();
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return e;
  const bool capturing = cap != hipStreamCaptureStatusNone;
  hipblasLtHandle_t h = nullptr;
  Descs ds;
  if (!make_descs(ds, M, N, K, x_dt, out_dt)) return hipErrorNotSupported;
  const auto key = std::make_tuple(dev, M, N, K, x_dt, out_dt);
  bool known = false;
  AlgoChoice choice{false, {}};
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto hi = g_handles.find(dev);
    auto ai = g_algo.find(key);
    known = ai != g_algo.end();
    if (known) choice = ai->second;
    // Handle creation and the first call's timing (event synchronisation) cannot run
    // under graph capture: an unseen device or shape is served by the fused kernel.
    if (capturing && (hi == g_handles.end() || !known)) return fused();
    if (hi == g_handles.end()) {
      if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return hipErrorNotSupported;
      g_handles[dev] = h;
    } else {
      h = hi->second;
    }
  }
  if (!known) {
    // First call for this shape: pick an algorithm outside the lock (two threads that
    // race here both time the candidates; the first result stored is kept).
    choice = select_algo(h, ds, x, ws, out, nib, sc, awq, x_dt, N, K, s, &e);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_mu);
    choice = g_algo.emplace(key, choice).first->second;
  }
  if (!choice.ok) return fused();
  const hipblasLtMatmulAlgo_t algo = choice.algo;
  void* wdq = ws;
  void* blas_ws = (char*)ws + round256((size_t)N * K * 2);
  e = launch_dequant_w4(nib, sc, awq, wdq, x_dt, N, K, s);
  if (e != hipSuccess) return e;
  const float alpha = 1.0f, beta = 0.0f;
  if (hipblasLtMatmul(h, ds.op, &alpha, wdq, ds.a, x, ds.b, &beta, out, ds.d, out, ds.d, &algo, blas_ws,
                      kBlasWorkspace, s) != HIPBLAS_STATUS_SUCCESS)
    return hipErrorLaunchFailure;
  return hipGetLastError();
}

}  // namespace nve_host
