"""GPU parity of the W4A16 prefill GEMM (nve_hip_gemm_w4a16) and of the weight
dequantization it fuses.

Reference semantics (GpuWeight::matmul_x for seq > 1, src/gpu_layer.rs:219-237): the
int4 weights are expanded with nve_dequant_w4a16 (f32 (nibble - 8) * scale [* awq],
rounded to fp16) and multiplied by the fp16 activations in a dense GEMM.  The oracle
forms the same rounded weights from QuantizedTensor::to_f32_vec (restated in
oracle/oracle.c) and multiplies in float64; the kernel accumulates in fp32 on MFMA.
Bars: the weights the GEMM multiplies are bit-identical to the reference's dequant
(checked exactly with an identity activation matrix); products: the W4A16 bar,
rel = max_i |y_i - ref_i| / max(|ref_i|, 1e-3 rms(ref)) <= 2e-3 for fp32 output
(fp32 accumulation over K terms in MFMA order; measured ~1e-3 at the near-zero floor
for K = 8192), plus 2^-8 (bf16) / 2^-11 (fp16) for rounded outputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import rel_err_floor, to_bf16, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def hk(torch_dev):
    from nve_amd import hip_kernels
    return hip_kernels


def _round(a, dt):
    return a.astype(np.float16).astype(np.float32) if dt == "f16" else to_bf16(a)


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (7, 300, 4096), (2, 1000, 4096), (16, 200, 192), (16, 8200, 1024),
                                   (1, 4097, 256), (4, 14336, 4096), (9, 4096, 14336), (16, 16384, 512),
                                   (24, 14336, 4096), (32, 4096, 14336), (20, 300, 256), (48, 14336, 4096),
                                   (100, 2000, 1024), (48, 16400, 512), (33, 200, 4160), (64, 14336, 4096), (60, 300, 512), (320, 1000, 1024), (129, 700, 512),
                                   (17, 96, 1024), (32, 520, 1024), (33, 300, 2048), (128, 128, 1024), (200, 520, 3072), (512, 256, 8192),
                                   (300, 1000, 512), (600, 520, 2048), (1100, 300, 1024), (200, 8192, 1024),
                                   (520, 8300, 512)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
def test_gemm_w4a16_parity(orc, torch_dev, hk, m, n, k, xdt, with_awq):
    torch = torch_dev
    print(f"gemm m={m} n={n} k={k} x={xdt} awq={with_awq}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k)
    data = orc.q4_from_f32(weights(n, k, seed=m + n, std=0.05))
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = rng.uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    wref = _round(orc.q4_to_f32(data, n, k, awq), xdt).astype(np.float64)
    x = _round(rng.standard_normal((m, k)).astype(np.float32), xdt)
    ref = x.astype(np.float64) @ wref.T
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    xt = torch.from_numpy(x).cuda().to(tdt)
    y = hk.gemm_w4a16(xt, torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda(), n, k,
                      None if awq is None else torch.from_numpy(awq).cuda(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err_floor(y.cpu().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
def test_gemm_w4a16_weights_match_dequant_exactly(orc, torch_dev, hk, xdt, with_awq):
    """X = I: every output is one product 1 * w (exact in fp32), so Y^T is the weight
    matrix as the GEMM rounded it, which must equal the reference dequant bit for bit
    (including halfway cases, where a fused multiply-convert would round differently)."""
    torch = torch_dev
    n, k = 130, 512
    data = orc.q4_from_f32(weights(n, k, seed=31, std=0.3))
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = np.random.default_rng(32).uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    wref = _round(orc.q4_to_f32(data, n, k, awq), xdt)
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    eye = torch.eye(k, dtype=tdt, device="cuda")
    y = hk.gemm_w4a16(eye, torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda(), n, k,
                      None if awq is None else torch.from_numpy(awq).cuda(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().T.view(np.uint32), wref.view(np.uint32))


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
@pytest.mark.parametrize("n,k,mb", [(70, 448, 16), (70, 512, 16), (4100, 256, 16), (70, 512, 32), (4100, 256, 24), (70, 512, 48), (70, 512, 64)])
def test_gemm_w4a16_small_m_weights_match_dequant_exactly(orc, torch_dev, hk, xdt, with_awq, n, k, mb):
    """M <= 32 runs a weight-streaming kernel: mb rows of the identity at a time
    (X = I[k0 : k0 + mb]) read back mb columns of the weight matrix as the kernel
    rounded it, which must equal the reference dequant bit for bit.  K = 448 leaves a
    partial last quad of blocks (the register kernel, M <= 16); K = 512 and 256 run the
    LDS-ring kernel (16-row workgroups at 70 rows, 17-row workgroups at 4100: a partly
    masked second tile; mb = 24 / 32: two operand groups of activation rows; mb = 64: four,
    or two launches of 32 rows with AWQ)."""
    torch = torch_dev
    print(f"identity n={n} k={k} mb={mb} x={xdt} awq={with_awq}", flush=True)
    data = orc.q4_from_f32(weights(n, k, seed=41, std=0.3))
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = np.random.default_rng(42).uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    wref = _round(orc.q4_to_f32(data, n, k, awq), xdt)
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    eye = torch.eye(k, dtype=tdt, device="cuda")
    tn, ts = torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda()
    ta = None if awq is None else torch.from_numpy(awq).cuda()
    got = np.zeros((k, n), np.float32)
    for k0 in range(0, k, mb):
        y = hk.gemm_w4a16(eye[k0:k0 + mb].contiguous(), tn, ts, n, k, ta, out_dtype=torch.float32)
        got[k0:k0 + mb] = y.cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(got.T.view(np.uint32), wref.view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(330, 130, 256), (321, 1000, 512), (130, 16000, 256), (1100, 300, 1024),
                                   (600, 8200, 256), (513, 4100, 512), (300, 200, 192), (330, 200, 128)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
def test_gemm_w4a16_tile_weights_match_dequant_exactly(orc, torch_dev, hk, m, n, k, xdt, with_awq):
    """With K % 128 == 0 the tile kernel (gemm_w4a16_tile.hip) runs above 320 rows (with
    AWQ above 128), and from 128 rows where its 128-row grid has at least 128 workgroups; it
    takes 128-row tiles while that grid has at most 256 workgroups, else 256-row tiles
    (here: 128 rows at 3 x 2, 3 x 8, 2 x 125, 9 x 3 and 5 x 33 tiles, 256 rows at 3 x 65;
    K % 128 == 64, here K = 192, runs the 128 x 128-tile kernel).  One-hot activation rows
    (row i picks column k_i) make each output one product 1 * w, so Y[i, :] is weight
    column k_i as the kernel rounded it, which must equal the reference dequant bit for
    bit.  Ragged M and N, K = 256 (two iterations of two 64-wide slices) and K = 128 (one
    iteration, every later slice's transfers clamped to its last slice), and tile grids that are
    not a multiple of 8 workgroups (the XCD-grouped tile order); fp32 output, and fp16 /
    bf16 output for fp16 / bf16 x (exact too).  With AWQ every weight is the reference's
    f32 dequant times awq[k], then rounded."""
    torch = torch_dev
    print(f"tile identity m={m} n={n} k={k} x={xdt} awq={with_awq}", flush=True)
    data = orc.q4_from_f32(weights(n, k, seed=m + n, std=0.3))
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = np.random.default_rng(n + k).uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    wref = _round(orc.q4_to_f32(data, n, k, awq), xdt)
    ta = None if awq is None else torch.from_numpy(awq).cuda()
    ks = np.random.default_rng(m + k).integers(0, k, m)
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    x = torch.zeros((m, k), dtype=tdt, device="cuda")
    x[torch.arange(m, device="cuda"), torch.from_numpy(ks).cuda()] = 1
    tn, ts = torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda()
    y = hk.gemm_w4a16(x, tn, ts, n, k, ta, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), np.ascontiguousarray(wref[:, ks].T).view(np.uint32))
    if xdt == "f16":
        y16 = hk.gemm_w4a16(x, tn, ts, n, k, ta, out_dtype=torch.float16)
        assert np.array_equal(y16.cpu().numpy(), wref[:, ks].T.astype(np.float16))
    else:
        yb = hk.gemm_w4a16(x, tn, ts, n, k, ta, out_dtype=torch.bfloat16)
        assert np.array_equal(yb.float().cpu().numpy().view(np.uint32),
                              np.ascontiguousarray(wref[:, ks].T).view(np.uint32))


def test_gemm_w4a16_tile_wide_n_exact(orc, torch_dev, hk):
    """The tile kernel at an lm_head-wide N (128256 rows of weights, 1002 column tiles):
    at M = 300 its 256-row grid is 2 x 1002 workgroups, about eight rounds on 256 CUs,
    with the XCD-grouped order spread over them.  One-hot activation rows: every output
    is one weight as the reference dequant rounds it, compared bit for bit."""
    torch = torch_dev
    m, n, k = 300, 128256, 256
    data = orc.q4_from_f32(weights(n, k, seed=77, std=0.3))
    nib, sc = orc.extract_for_gpu(data, n, k)
    wref = orc.q4_to_f32(data, n, k, None).astype(np.float16)
    ks = np.random.default_rng(78).integers(0, k, m)
    x = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    x[torch.arange(m, device="cuda"), torch.from_numpy(ks).cuda()] = 1
    y = hk.gemm_w4a16(x, torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda(), n, k, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), np.ascontiguousarray(wref[:, ks].T))


@pytest.mark.parametrize("odt,tol", [("bf16", 2.0 ** -8 + 2e-3), ("f16", 2.0 ** -11 + 2e-3)])
@pytest.mark.parametrize("m", [33, 5, 130, 300])
def test_gemm_w4a16_rounded_outputs(orc, torch_dev, hk, odt, tol, m):
    torch = torch_dev
    n, k = 192, 2048
    rng = np.random.default_rng(5)
    data = orc.q4_from_f32(weights(n, k, seed=9, std=0.05))
    nib, sc = orc.extract_for_gpu(data, n, k)
    wref = orc.q4_to_f32(data, n, k).astype(np.float16).astype(np.float64)
    x = rng.standard_normal((m, k)).astype(np.float16)
    ref = x.astype(np.float64) @ wref.T
    out_dt = torch.bfloat16 if odt == "bf16" else torch.float16
    y = hk.gemm_w4a16(torch.from_numpy(x).cuda(), torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda(), n, k,
                      out_dtype=out_dt)
    torch.cuda.synchronize()
    assert rel_err_floor(y.float().cpu().numpy(), ref) <= tol


@pytest.mark.parametrize("m,n,k", [(520, 256, 1024), (600, 520, 2048), (1024, 384, 4096)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
def test_gemm_w4a16_ws_blas_path(orc, torch_dev, hk, m, n, k, xdt, with_awq):
    """nve_hip_gemm_w4a16_ws above M = 512 with its workspace: dequant (bit-identical
    weights) + hipBLASLt, the reference's own prefill method, to the same bar."""
    _ws_blas_check(orc, torch_dev, hk, m, n, k, xdt, with_awq)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_gemm_w4a16_ws_blas_path_awq_from_385(orc, torch_dev, hk, xdt):
    """With AWQ factors the workspace path takes dequant + hipBLASLt from M = 385."""
    _ws_blas_check(orc, torch_dev, hk, 400, 256, 1024, xdt, True)


def _ws_blas_check(orc, torch_dev, hk, m, n, k, xdt, with_awq):
    torch = torch_dev
    print(f"gemm_ws m={m} n={n} k={k} x={xdt} awq={with_awq}", flush=True)
    rng = np.random.default_rng(m + 3 * n + k)
    data = orc.q4_from_f32(weights(n, k, seed=m + 2 * n, std=0.05))
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = rng.uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    wref = _round(orc.q4_to_f32(data, n, k, awq), xdt).astype(np.float64)
    x = _round(rng.standard_normal((m, k)).astype(np.float32), xdt)
    ref = x.astype(np.float64) @ wref.T
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    xt = torch.from_numpy(x).cuda().to(tdt)
    wsb = hk.gemm_w4a16_workspace_bytes(m, n, k)
    assert wsb >= n * k * 2
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    args = (xt, torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda(), n, k, ws,
            None if awq is None else torch.from_numpy(awq).cuda())
    y = hk.gemm_w4a16_ws(*args, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err_floor(y.cpu().numpy().astype(np.float64), ref) <= 2e-3
    # the workspace holds the reference dequant of the weights, bit for bit
    wdq = ws[: n * k * 2].view(tdt).view(n, k).float().cpu().numpy()
    assert np.array_equal(wdq, wref.astype(np.float32))
    # output in x's dtype: the fp32 result rounded once
    y16 = hk.gemm_w4a16_ws(*args, out_dtype=tdt).float().cpu().numpy().astype(np.float64)
    assert rel_err_floor(y16, ref) <= 2e-3 + (2.0 ** -8 if xdt == "bf16" else 2.0 ** -11)


def test_gemm_w4a16_ws_falls_back(orc, torch_dev, hk):
    """Up to M = 512 (no AWQ factors), or without a workspace, nve_hip_gemm_w4a16_ws is the fused kernel
    (compared at fp16 output: with a workspace an fp32 product at small M splits K, whose
    partials then add in a different order than one pass)."""
    torch = torch_dev
    # up to M = 384 the workspace holds only K-split partials (none for M <= 16); from 385
    # also room for the dequantized weights (used with AWQ factors up to 512, else above)
    assert hk.gemm_w4a16_workspace_bytes(16, 256, 1024) == 0
    assert hk.gemm_w4a16_workspace_bytes(384, 256, 1024) == 4 * 384 * 256 * 4
    assert hk.gemm_w4a16_workspace_bytes(385, 256, 1024) > (256 * 1024 * 2)
    assert hk.gemm_w4a16_workspace_bytes(513, 256, 1024) > (256 * 1024 * 2)
    n, k = 256, 1024
    data = orc.q4_from_f32(weights(n, k, seed=5, std=0.05))
    nib, sc = (torch.from_numpy(a).cuda() for a in orc.extract_for_gpu(data, n, k))
    for m in (64, 300, 512, 600):
        x = torch.randn((m, k), device="cuda").to(torch.float16)
        a = hk.gemm_w4a16(x, nib, sc, n, k, out_dtype=torch.float16).cpu()
        b = hk.gemm_w4a16_ws(x, nib, sc, n, k, None, out_dtype=torch.float16).cpu()
        assert torch.equal(a, b), m


def test_gemm_w4a16_ws_graph_capture(orc, torch_dev, hk):
    """Under HIP graph capture: a shape first seen during capture takes the fused kernel
    (no handle creation or timing in the graph; with the workspace's K-split partials,
    as an eager call whose workspace only fits those); after an eager call has selected the
    algorithm, the captured graph replays the BLAS path.  Every replay matches eager."""
    torch = torch_dev
    # N = 544 is used by no other test: the algorithm cache is process-wide, so the cold
    # case must be a shape nothing earlier in the process has sent down the BLAS path.
    n, k = 544, 1024
    data = orc.q4_from_f32(weights(n, k, seed=9, std=0.05))
    nib, sc = (torch.from_numpy(a).cuda() for a in orc.extract_for_gpu(data, n, k))
    for m, warm in ((520, False), (640, True)):
        print(f"gemm_ws capture m={m} warm={warm}", flush=True)
        x = torch.randn((m, k), device="cuda").to(torch.float16)
        ws = torch.empty(hk.gemm_w4a16_workspace_bytes(m, n, k), dtype=torch.uint8, device="cuda")
        out = torch.empty((m, n), dtype=torch.float16, device="cuda")
        # the fused path with this workspace (K-split partials): a workspace slice too
        # small for the BLAS path but large enough for the partials
        assert m * n * 32 < n * k * 2 + (32 << 20)
        eager_fused = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws[: m * n * 32], out_dtype=torch.float16)
        if warm:
            eager = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, out_dtype=torch.float16)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out.copy_(hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, out_dtype=torch.float16))
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            if warm:
                assert torch.equal(out, eager)
            else:
                assert torch.equal(out, eager_fused)


@pytest.mark.parametrize("m,n,k", [(64, 512, 4160), (40, 1000, 2112), (200, 256, 8192)])
def test_gemm_w4a16_ws_split_k_reproducible(orc, torch_dev, hk, m, n, k):
    """With a workspace, a K-split fp32 product stores its partials there and adds them
    in a fixed order: every call -- eager or replayed from a HIP graph -- gives the same
    bits, within the W4A16 bar of the oracle and within fp32 rounding of the unsplit
    product of nve_hip_gemm_w4a16 (which is itself the same on every call)."""
    torch = torch_dev
    wsb = hk.gemm_w4a16_workspace_bytes(m, n, k)
    assert wsb > 0
    data = orc.q4_from_f32(weights(n, k, seed=m + n, std=0.05))
    nib_h, sc_h = orc.extract_for_gpu(data, n, k)
    nib, sc = torch.from_numpy(nib_h).cuda(), torch.from_numpy(sc_h).cuda()
    xh = np.random.default_rng(m).standard_normal((m, k)).astype(np.float16)
    x = torch.from_numpy(xh).cuda()
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    a = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws)
    b = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws)
    unsplit = hk.gemm_w4a16(x, nib, sc, n, k)
    assert torch.equal(unsplit, hk.gemm_w4a16(x, nib, sc, n, k))  # no workspace: one pass, same bits
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out.copy_(hk.gemm_w4a16_ws(x, nib, sc, n, k, ws))
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, a)
    assert torch.equal(a, b)
    assert torch.allclose(a, unsplit, rtol=1e-5, atol=1e-5 * float(a.abs().max()))
    wref = _round(orc.q4_to_f32(data, n, k, None), "f16").astype(np.float64)
    ref = xh.astype(np.float64) @ wref.T
    assert rel_err_floor(a.cpu().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("m,n,k", [(200, 520, 2048), (300, 1000, 1152), (130, 4100, 8192), (513, 300, 1024),
                                   (100, 520, 2048), (65, 4101, 1024), (130, 520, 2688)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("with_awq", [False, True])
def test_gemm_w4a16_ws_tile_split(orc, torch_dev, hk, m, n, k, xdt, with_awq):
    """With a workspace, the register-dequant tile kernel splits K where its 128-row grid
    leaves CUs idle, from M = 65 (here 2 x 5 tiles in 4 splits, 3 x 8 in 2 of 10 and 8
    slices, 2 x 33 in 3 of 44, 44 and 40, 5 x 3 in 2, 1 x 5 in 4, 1 x 33 in 2 with an odd
    M N, 2 x 5 in 5 of 10, 10, 10, 10 and 2 slices; M = 513 takes the fused path when the output type is neither fp32 nor
    x's): each split stores fp32 partials, one more launch adds them in split order and
    rounds once to the output type.  Every call and every graph replay gives the same
    bits; an fp16 / bf16 output is exactly the fp32 result rounded; the product is within
    fp32 rounding of the unsplit one and within the W4A16 bar of the oracle; with and
    without AWQ."""
    torch = torch_dev
    print(f"tile split m={m} n={n} k={k} x={xdt} awq={with_awq}", flush=True)
    wsb = hk.gemm_w4a16_workspace_bytes(m, n, k)
    assert wsb >= 2 * m * n * 4
    data = orc.q4_from_f32(weights(n, k, seed=m + n, std=0.05))
    nib_h, sc_h = orc.extract_for_gpu(data, n, k)
    nib, sc = torch.from_numpy(nib_h).cuda(), torch.from_numpy(sc_h).cuda()
    awq = np.random.default_rng(n).uniform(0.5, 2.0, k).astype(np.float32) if with_awq else None
    ta = None if awq is None else torch.from_numpy(awq).cuda()
    xr = _round(np.random.default_rng(m + k).standard_normal((m, k)).astype(np.float32), xdt)
    tdt = torch.float16 if xdt == "f16" else torch.bfloat16
    x = torch.from_numpy(xr).cuda().to(tdt)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    if m <= 512:
        a = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta)
        assert torch.equal(a, hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta))
        unsplit = hk.gemm_w4a16(x, nib, sc, n, k, ta)
        assert torch.allclose(a, unsplit, rtol=1e-5, atol=1e-5 * float(a.abs().max()))
        wref = _round(orc.q4_to_f32(data, n, k, awq), xdt).astype(np.float64)
        assert rel_err_floor(a.cpu().numpy(), xr.astype(np.float64) @ wref.T) <= 2e-3
        for odt in (torch.float16, torch.bfloat16):
            assert torch.equal(hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta, out_dtype=odt), a.to(odt))
    else:
        odt = torch.bfloat16 if xdt == "f16" else torch.float16  # not BLAS-eligible: fused
        a = hk.gemm_w4a16(x, nib, sc, n, k, ta).to(odt)
        b = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta, out_dtype=odt)
        assert torch.allclose(a.float(), b.float(), rtol=2 ** -7, atol=1e-5 * float(a.float().abs().max()))
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    ref16 = hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta, out_dtype=torch.float16)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out.copy_(hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, ta, out_dtype=torch.float16))
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref16)


@pytest.mark.parametrize("m", [8, 48, 200])
def test_gemm_w4a16_ring_graph_replay_matches_eager(orc, torch_dev, hk, m):
    """The LDS-ring prefill path (one launch at M = 8 and 48, four 64-row launches at
    M = 200) captured in a HIP graph: every replay, with eager work and
    synchronisations between the replays, equals the eager call bit for bit."""
    torch = torch_dev
    n, k = 700, 1024
    print(f"ring graph m={m}", flush=True)
    data = orc.q4_from_f32(weights(n, k, seed=m, std=0.05))
    nib_h, sc_h = orc.extract_for_gpu(data, n, k)
    nib, sc = torch.from_numpy(nib_h).cuda(), torch.from_numpy(sc_h).cuda()
    x = torch.from_numpy(np.random.default_rng(m).standard_normal((m, k)).astype(np.float16)).cuda()
    eager = hk.gemm_w4a16(x, nib, sc, n, k, None, out_dtype=torch.float32)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out.copy_(hk.gemm_w4a16(x, nib, sc, n, k, None, out_dtype=torch.float32))
    for r in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), r
        hk.gemm_w4a16(x, nib, sc, n, k, None, out_dtype=torch.float32)
        torch.cuda.synchronize()
