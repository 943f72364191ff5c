"""The persistent (double-buffered) GEMV kernels against the one-shot kernels and the
oracle.  Both kernel shapes compute every row with the same per-lane block order and
the same DPP reduction, so their outputs must be bit-identical."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import activations, rel_err_floor, to_bf16, to_f16, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nve_amd import hip_kernels as hk
    from nve_amd._lib import GEMV_AUTO, GEMV_ONESHOT, GEMV_PERSISTENT, lib
    L = lib()
    yield torch, hk, L, (GEMV_AUTO, GEMV_ONESHOT, GEMV_PERSISTENT)
    L.nve_hip_set_gemv_policy(GEMV_AUTO, 2, 4)


def _problem(orc, n, k, seed):
    data = orc.q4_from_f32(weights(n, k, seed=seed))
    return orc.extract_for_gpu(data, n, k)


SHAPES = [(1, 32), (5, 96), (37, 1056), (1000, 2048), (3000, 3072), (4096, 4096), (333, 8192),
          (200, 14336), (64, 16384)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("occ,depth", [(1, 4), (2, 4), (4, 4), (2, 8), (3, 8)])
def test_persistent_w4a8_matches_oneshot_and_oracle(orc, env, n, k, occ, depth):
    torch, hk, L, (AUTO, ONESHOT, PERSIST) = env
    nib, ws = _problem(orc, n, k, seed=n + 3 * k)
    x = to_f16(activations(k, seed=k))
    tn, tw = torch.from_numpy(nib).cuda(), torch.from_numpy(ws).cuda()
    xq, xs = hk.quantize_f16_q8(torch.from_numpy(x.astype(np.float16)).cuda())
    L.nve_hip_set_gemv_policy(ONESHOT, occ, 4)
    y1 = hk.matvec_w4a8(xq, xs, tn, tw, n, k, out_dtype=torch.float32)
    L.nve_hip_set_gemv_policy(PERSIST, occ, depth)
    y2 = hk.matvec_w4a8(xq, xs, tn, tw, n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    L.nve_hip_set_gemv_policy(AUTO, 2, 4)
    assert torch.equal(y1, y2)
    q, s = orc.quantize_q8_group(x)
    assert rel_err_floor(y2.cpu().numpy()[0], orc.matvec_w4a8_f64(q, s, nib, ws, n, k)) <= 1e-3


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("depth", [4, 8])
def test_persistent_w4a16_matches_oneshot_and_oracle(orc, env, n, k, xdt, depth):
    torch, hk, L, (AUTO, ONESHOT, PERSIST) = env
    nib, sc = _problem(orc, n, k, seed=2 * n + k)
    x = activations(k, seed=k + 1)
    if xdt == "f16":
        xv = to_f16(x)
        xt = torch.from_numpy(x.astype(np.float16)).cuda()
    else:
        xv = to_bf16(x)
        xt = torch.from_numpy(xv).cuda().to(torch.bfloat16)
    tn, ts = torch.from_numpy(nib).cuda(), torch.from_numpy(sc).cuda()
    L.nve_hip_set_gemv_policy(ONESHOT, 2, 4)
    y1 = hk.fused_matvec_w4a16(xt, tn, ts, None, n, k, out_dtype=torch.float32)
    L.nve_hip_set_gemv_policy(PERSIST, 2, depth)
    y2 = hk.fused_matvec_w4a16(xt, tn, ts, None, n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    L.nve_hip_set_gemv_policy(AUTO, 2, 4)
    assert torch.equal(y1, y2)
    assert rel_err_floor(y2.cpu().numpy()[0], orc.matvec_w4a16_f64(xv, nib, sc, n, k)) <= 2e-3


@pytest.mark.parametrize("ns", [(3072, 1024, 1024), (5, 4000, 37), (14336, 14336, 1)])
@pytest.mark.parametrize("prec", ["w4a8", "w4a16"])
def test_persistent_grouped_segments(orc, env, ns, prec):
    torch, hk, L, (AUTO, ONESHOT, PERSIST) = env
    from nve_amd._lib import W4Mat
    k = 3072
    mats = [_problem(orc, n, k, seed=90 + i) for i, n in enumerate(ns)]
    t = [(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()) for a, b in mats]
    x = to_f16(activations(k, seed=5))
    x16 = torch.from_numpy(x.astype(np.float16)).cuda()
    xq, xs = hk.quantize_f16_q8(x16)
    results = {}
    for pol in (ONESHOT, PERSIST):
        L.nve_hip_set_gemv_policy(pol, 2, 4)
        outs = [torch.empty(n, dtype=torch.float32, device="cuda") for n in ns]
        arr = (W4Mat * 3)()
        for i in range(3):
            arr[i] = W4Mat(t[i][0].data_ptr(), t[i][1].data_ptr(), None, outs[i].data_ptr(), ns[i])
        s = torch.cuda.current_stream().cuda_stream
        if prec == "w4a8":
            st = L.nve_hip_grouped_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), arr, 3, 2, k, s)
        else:
            st = L.nve_hip_grouped_matvec_w4a16(x16.data_ptr(), 0, arr, 3, 2, k, s)
        assert st == 0
        torch.cuda.synchronize()
        results[pol] = outs
    L.nve_hip_set_gemv_policy(AUTO, 2, 4)
    q, sx = orc.quantize_q8_group(x)
    for i, n in enumerate(ns):
        assert torch.equal(results[ONESHOT][i], results[PERSIST][i])
        y = results[PERSIST][i].cpu().numpy()
        if prec == "w4a8":
            ref = orc.matvec_w4a8_f64(q, sx, mats[i][0], mats[i][1], n, k)
            assert rel_err_floor(y, ref) <= 1e-3
        else:
            ref = orc.matvec_w4a16_f64(x, mats[i][0], mats[i][1], n, k)
            assert rel_err_floor(y, ref) <= 2e-3


def test_graph_replay_matches_eager(orc, env):
    """The GEMV launches captured in a HIP graph and replayed several times, with eager
    work in between, give the eager result on every replay."""
    torch, hk, L, _ = env
    n, k = 8192, 4096
    nib, ws = _problem(orc, n, k, seed=4)
    tn, tw = torch.from_numpy(nib).cuda(), torch.from_numpy(ws).cuda()
    x16 = torch.from_numpy(activations(k, seed=8).astype(np.float16)).cuda()
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
    y8 = torch.empty(n, dtype=torch.float32, device="cuda")
    y16 = torch.empty(n, dtype=torch.float32, device="cuda")

    def step():
        s = torch.cuda.current_stream().cuda_stream
        assert L.nve_hip_quantize_q8(x16.data_ptr(), 0, 1, k, xq.data_ptr(), xs.data_ptr(), s) == 0
        assert L.nve_hip_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), tn.data_ptr(), tw.data_ptr(), y8.data_ptr(), 2,
                                     n, k, s) == 0
        assert L.nve_hip_matvec_w4a16(x16.data_ptr(), 0, tn.data_ptr(), tw.data_ptr(), None, y16.data_ptr(), 2,
                                      n, k, s) == 0
    step()
    torch.cuda.synchronize()
    e8, e16 = y8.clone(), y16.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(4):
        y8.zero_()
        y16.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y8, e8) and torch.equal(y16, e16)
