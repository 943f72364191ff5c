"""GPU parity: the HIP kernels in libnve_hip.so, called through the C ABI, against the
CPU oracle on identical seeded inputs.

Bars (stated by the task for this path):
  * W4A8 int32 block accumulators and int8 activations: bit-exact.
  * W4A8 fp32 output: relative error <= 1e-3 against the fp64 evaluation of
    sum_b ws*xs*acc, with rel = max_i |y_i - ref_i| / max(|ref_i|, 1e-3*rms(ref)).
  * W4A16 output: same metric <= 2e-3 against the fp64 dequantized product.
  * Device Q4_0 quantization and repack: bit-exact bytes.
Large shapes are checked on a seeded sample of rows (every addressing path of the
kernel is exercised, the oracle only evaluates the sampled rows).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import activations, rel_err_floor, to_bf16, to_f16, weights

pytestmark = pytest.mark.gpu

TOL_W4A8 = 1e-3
TOL_W4A16 = 2e-3


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


def up(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def down(t):
    return t.detach().cpu().numpy()


def _problem(orc, n, k, seed, std=0.02):
    w = weights(n, k, seed=seed, std=std)
    data = orc.q4_from_f32(w)
    nib, sc = orc.extract_for_gpu(data, n, k)
    return w, data, nib, sc


# ---------------------------------------------------------------------------
# activation quantization
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("k", [32, 64, 2048, 3072, 4096, 14336])
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
def test_quantize_q8_group_exact(orc, torch_dev, hk, k, xdt):
    torch = torch_dev
    x = activations(k, seed=100 + k)
    if xdt == "f16":
        xv, xt = to_f16(x), up(torch, x.astype(np.float16))
    elif xdt == "bf16":
        xv = to_bf16(x)
        xt = up(torch, xv).to(torch.bfloat16)
    else:
        xv, xt = x, up(torch, x)
    xq, xs = hk.quantize_f16_q8(xt)
    q_ref, s_ref = orc.quantize_q8_group(xv)
    assert np.array_equal(down(xq), q_ref)
    assert np.array_equal(down(xs), s_ref)


def test_quantize_q8_kat_ties_and_zero_group(orc, torch_dev, hk):
    torch = torch_dev
    x = np.zeros(64, np.float32)
    x[:8] = [127.0, 2.5, 3.5, -2.5, -127.0, 0.5, 1.5, -0.5]
    xq, xs = hk.quantize_f16_q8(up(torch, x.astype(np.float16)))
    assert list(down(xq)[:8]) == [127, 2, 4, -2, -127, 0, 2, 0]
    assert np.all(down(xq)[32:] == 0) and np.all(down(xs) == 1.0)


@pytest.mark.parametrize("xdt", ["f16", "f32"])
def test_quantize_q8_nonfinite(orc, torch_dev, hk, xdt):
    """NaN / +-Inf activations: the same codes and scales as the reference kernel's
    semantics restated in the oracle (NaN ignored by the max, scale inf -> codes 0)."""
    torch = torch_dev
    from test_oracle import _nonfinite_groups
    x = _nonfinite_groups()
    xt = up(torch, x.astype(np.float16)) if xdt == "f16" else up(torch, x)
    xq, xs = hk.quantize_f16_q8(xt)
    q_ref, s_ref = orc.quantize_q8_group(x)
    assert np.array_equal(down(xq), q_ref)
    assert np.array_equal(down(xs).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("m,k", [(1, 2048), (4, 4096), (16, 14336), (3, 96)])
def test_quantize_q8_rows_exact(orc, torch_dev, hk, m, k):
    torch = torch_dev
    x = to_bf16(activations(k, seed=7 * m + k, m=m))
    xq, xs = hk.quantize_q8_rows(up(torch, x).to(torch.bfloat16), per_token=True)
    q_ref, s_ref = orc.quantize_q8_rows_bf16(x)
    assert np.array_equal(down(xq), q_ref)
    assert np.array_equal(down(xs.view(torch.int16)).view(np.uint16), s_ref)
    xq2, xs2 = hk.quantize_q8_rows(up(torch, x).to(torch.bfloat16), per_token=False)
    q2, s2 = orc.quantize_q8_group(x)
    assert np.array_equal(down(xq2), q2) and np.array_equal(down(xs2), s2)


# ---------------------------------------------------------------------------
# W4A8 GEMV
# ---------------------------------------------------------------------------
W4A8_SHAPES = [
    (1, 32), (3, 64), (5, 96), (37, 160), (130, 1056), (2048, 2048), (512, 2048), (1000, 3072),
    (256, 4096), (300, 8192), (96, 14336), (64, 16384), (40, 16416), (24, 28672), (16, 32768),
]


@pytest.mark.parametrize("n,k", W4A8_SHAPES)
def test_w4a8_gemv_parity(orc, torch_dev, hk, n, k):
    torch = torch_dev
    _, _, nib, ws = _problem(orc, n, k, seed=n * 31 + k)
    x = to_f16(activations(k, seed=k + 1))
    xq_ref, xs_ref = orc.quantize_q8_group(x)
    tnib, tws = up(torch, nib), up(torch, ws)
    xq, xs = hk.quantize_f16_q8(up(torch, x.astype(np.float16)))
    assert np.array_equal(down(xq), xq_ref)
    acc = hk.w4a8_block_acc(xq, tnib, n, k)
    assert np.array_equal(down(acc), orc.w4a8_block_acc(xq_ref, nib, n, k))
    y = hk.matvec_w4a8(xq, xs, tnib, tws, n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = orc.matvec_w4a8_f64(xq_ref, xs_ref, nib, ws, n, k)
    assert rel_err_floor(down(y)[0], ref) <= TOL_W4A8
    y16 = hk.matvec_w4a8(xq, xs, tnib, tws, n, k)  # reference dtype (fp16)
    assert np.array_equal(down(y16)[0], down(y)[0].astype(np.float16))


def test_w4a8_dropin_void_launchers(orc, torch_dev):
    """nve_quantize_f16_q8 / nve_matvec_w4a8 with the reference's argument order."""
    torch = torch_dev
    from nve_amd._lib import lib
    L = lib()
    n, k = 700, 2048
    _, _, nib, ws = _problem(orc, n, k, seed=5)
    x = to_f16(activations(k, seed=6))
    tx = up(torch, x.astype(np.float16))
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    L.nve_quantize_f16_q8(tx.data_ptr(), xq.data_ptr(), xs.data_ptr(), k, s)
    tnib, tws = up(torch, nib), up(torch, ws)
    L.nve_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), tnib.data_ptr(), tws.data_ptr(), out.data_ptr(), n, k, s)
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    xq_ref, xs_ref = orc.quantize_q8_group(x)
    ref = orc.matvec_w4a8_f64(xq_ref, xs_ref, nib, ws, n, k)
    assert rel_err_floor(down(out).astype(np.float64), ref) <= 1e-3 + 2.0**-11


def test_w4a8_fused_qkv_equals_separate(orc, torch_dev, hk):
    torch = torch_dev
    from nve_amd.gpu_layer import GpuW4
    k = 3072
    mats = []
    for i, n in enumerate((3072, 1024, 1024)):
        _, _, nib, ws = _problem(orc, n, k, seed=50 + i)
        mats.append(GpuW4(up(torch, nib), up(torch, ws), None, n, k))
    xq, xs = hk.quantize_f16_q8(up(torch, activations(k, seed=9).astype(np.float16)))
    fused = hk.qkv_matvec_w4a8(xq, xs, *mats, out_dtype=torch.float32)
    for f, m in zip(fused, mats):
        sep = hk.matvec_w4a8(xq, xs, m.nibbles, m.scales, m.n, m.k, out_dtype=torch.float32)
        assert torch.equal(f, sep)


# ---------------------------------------------------------------------------
# W4A16 GEMV
# ---------------------------------------------------------------------------
W4A16_SHAPES = [(1, 32), (7, 96), (37, 160), (2048, 2048), (512, 2048), (1000, 3072), (256, 4096),
                (300, 8192), (96, 14336), (40, 16416), (16, 32768)]


@pytest.mark.parametrize("n,k", W4A16_SHAPES)
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_w4a16_gemv_parity(orc, torch_dev, hk, n, k, xdt):
    torch = torch_dev
    _, _, nib, sc = _problem(orc, n, k, seed=n * 17 + k)
    x = activations(k, seed=k + 3)
    if xdt == "f16":
        xv = to_f16(x)
        xt = up(torch, x.astype(np.float16))
    else:
        xv = to_bf16(x)
        xt = up(torch, xv).to(torch.bfloat16)
    y = hk.fused_matvec_w4a16(xt, up(torch, nib), up(torch, sc), None, n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = orc.matvec_w4a16_f64(xv, nib, sc, n, k)
    assert rel_err_floor(down(y)[0], ref) <= TOL_W4A16


@pytest.mark.parametrize("n,k", [(64, 2048), (33, 4096), (20, 16416)])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_w4a16_awq_parity(orc, torch_dev, hk, n, k, xdt):
    torch = torch_dev
    _, _, nib, sc = _problem(orc, n, k, seed=n + k)
    x = activations(k, seed=4)
    awq = np.exp(np.random.default_rng(5).standard_normal(k) * 0.3).astype(np.float32)
    xv = to_f16(x) if xdt == "f16" else to_bf16(x)
    xt = up(torch, x.astype(np.float16)) if xdt == "f16" else up(torch, xv).to(torch.bfloat16)
    y = hk.fused_matvec_w4a16(xt, up(torch, nib), up(torch, sc), up(torch, awq), n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = orc.matvec_w4a16_f64(xv, nib, sc, n, k, awq=awq)
    assert rel_err_floor(down(y)[0], ref) <= TOL_W4A16


def test_w4a16_bf16_wide_dynamic_range(orc, torch_dev, hk):
    """Blocks whose values span 2^-30 .. 2^20 (exercises the per-block fp16 rescale)."""
    torch = torch_dev
    n, k = 64, 1024
    _, _, nib, sc = _problem(orc, n, k, seed=77)
    g = np.random.default_rng(78)
    x = (g.standard_normal(k) * np.exp2(g.integers(-30, 21, size=k))).astype(np.float32)
    xv = to_bf16(x)
    y = hk.fused_matvec_w4a16(up(torch, xv).to(torch.bfloat16), up(torch, nib), up(torch, sc), None, n, k,
                              out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err_floor(down(y)[0], orc.matvec_w4a16_f64(xv, nib, sc, n, k)) <= TOL_W4A16


def test_w4a16_dropin_and_qkv(orc, torch_dev, hk):
    torch = torch_dev
    from nve_amd._lib import lib
    L = lib()
    k = 2048
    x = to_f16(activations(k, seed=12))
    tx = up(torch, x.astype(np.float16))
    probs = [_problem(orc, n, k, seed=60 + i) for i, n in enumerate((2048, 512, 512))]
    t = [(up(torch, p[2]), up(torch, p[3])) for p in probs]
    ns = (2048, 512, 512)
    outs = [torch.empty(n, dtype=torch.float16, device="cuda") for n in ns]
    s = torch.cuda.current_stream().cuda_stream
    L.nve_qkv_matvec_w4a16(tx.data_ptr(), t[0][0].data_ptr(), t[0][1].data_ptr(), None, ns[0],
                           t[1][0].data_ptr(), t[1][1].data_ptr(), None, ns[1],
                           t[2][0].data_ptr(), t[2][1].data_ptr(), None, ns[2],
                           outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), k, s)
    single = torch.empty(2048, dtype=torch.float16, device="cuda")
    L.nve_matvec_w4a16(tx.data_ptr(), t[0][0].data_ptr(), t[0][1].data_ptr(), None, single.data_ptr(), 2048, k, s)
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    assert torch.equal(single, outs[0])
    for o, p, n in zip(outs, probs, ns):
        ref = orc.matvec_w4a16_f64(x, p[2], p[3], n, k)
        assert rel_err_floor(down(o).astype(np.float64), ref) <= TOL_W4A16 + 2.0**-11


# ---------------------------------------------------------------------------
# weight preparation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("wdt", ["f32", "bf16", "f16"])
def test_q4_quantize_device_bit_exact(orc, torch_dev, hk, wdt):
    torch = torch_dev
    n, k = 257, 640
    w = weights(n, k, seed=3, std=1.0)
    # known-answer blocks in the first row: ramp, ties, zero, 1/scale = inf, underflow
    w[0, 0:32] = (np.arange(32) - 16) * 0.5
    w[0, 32:64] = 0.0
    w[0, 32:42] = [7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 6.5, -6.5, 3.5]
    w[0, 64:96] = 0.0
    if wdt == "f32":
        w[0, 96:128] = 0.0
        w[0, 96], w[0, 97], w[0, 99] = 1e-38, -1e-38, 5e-39
        w[0, 128:160] = 0.0
        w[0, 130] = 2.0**-149
        wt, wv = up(torch, w), w
    elif wdt == "bf16":
        wv = to_bf16(w)
        wt = up(torch, wv).to(torch.bfloat16)
    else:
        wv = to_f16(w)
        wt = up(torch, w.astype(np.float16))
    nib, sc = hk.q4_quantize(wt)
    nib_ref, sc_ref = orc.extract_for_gpu(orc.q4_from_f32(wv), n, k)
    assert np.array_equal(down(nib), nib_ref)
    assert np.array_equal(down(sc).view(np.uint32), sc_ref.view(np.uint32))


@pytest.mark.parametrize("kquant", [False, True])
@pytest.mark.parametrize("wdt", ["f32", "bf16", "f16"])
def test_q4_quantize_awq_device_bit_exact(orc, torch_dev, hk, wdt, kquant):
    """from_compact_awq(_kquant) + extract_for_gpu on the device against the oracle's
    restatement (src/quantize.rs:271-346, 741-793) on the same weights."""
    torch = torch_dev
    n, k = 131, 1024
    w = weights(n, k, seed=31, std=0.5)
    rng = np.random.default_rng(32)
    awq = rng.uniform(0.25, 4.0, k).astype(np.float32)
    awq[5], awq[40] = 0.0, -2.0  # a dead channel (inverse 0) and a negative scale
    # special blocks in row 0: a constant block with a dead channel (awq 0 zeroes
    # both the value and its importance), a ramp with unit awq, a tiny block (every
    # |v| < 1e-10: no candidate, scale 0)
    awq[64:96] = 1.0
    w[0, 0:32] = 3.5
    w[0, 5] = 7.0
    w[0, 32:64] = (np.arange(32) - 16) * 0.5
    w[0, 64:96] = 5e-11 if wdt == "f32" else 0.0
    w[1, ::7] *= 20.0  # outliers
    if wdt == "f32":
        wt, wv = up(torch, w), w
    elif wdt == "bf16":
        wv = to_bf16(w)
        wt = up(torch, wv).to(torch.bfloat16)
    else:
        wv = to_f16(w)
        wt = up(torch, w.astype(np.float16))
    nib, sc, inv = hk.q4_quantize_awq(wt, up(torch, awq), kquant=kquant)
    data_ref, inv_ref = orc.q4_from_f32_awq(wv, awq, kquant)
    nib_ref, sc_ref = orc.extract_for_gpu(data_ref, n, k)
    assert np.array_equal(down(nib), nib_ref)
    assert np.array_equal(down(sc).view(np.uint32), sc_ref.view(np.uint32))
    assert np.array_equal(down(inv).view(np.uint32), inv_ref.view(np.uint32))


def test_q4_quantize_awq_feeds_w4a16_gemv(orc, torch_dev, hk):
    """AWQ end to end: the device-quantized weights and inverse scales through the
    W4A16 GEMV against the float64 dequantized product (bar 2e-3)."""
    torch = torch_dev
    n, k = 512, 2048
    w = weights(n, k, seed=41, std=0.02)
    awq = np.random.default_rng(42).uniform(0.5, 2.0, k).astype(np.float32)
    nib, sc, inv = hk.q4_quantize_awq(up(torch, w), up(torch, awq), kquant=True)
    x = activations(k, seed=43)
    xb = to_bf16(x)
    y = down(hk.fused_matvec_w4a16(up(torch, xb).to(torch.bfloat16), nib, sc, inv, n, k, out_dtype=torch.float32))
    ref = orc.matvec_w4a16_f64(xb, down(nib), down(sc), n, k, awq=down(inv))
    assert rel_err_floor(y, ref) <= 2e-3


def test_q4_repack_device_bit_exact(orc, torch_dev, hk):
    torch = torch_dev
    n, k = 129, 4096
    data = orc.q4_from_f32(weights(n, k, seed=4))
    nib, sc = hk.q4_repack(up(torch, data), n, k)
    nib_ref, sc_ref = orc.extract_for_gpu(data, n, k)
    assert np.array_equal(down(nib), nib_ref) and np.array_equal(down(sc), sc_ref)


@pytest.mark.parametrize("with_awq", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_dequant_w4_bit_exact(orc, torch_dev, hk, dtype, with_awq):
    """nve_dequant_w4a16 / nve_hip_dequant_w4 against QuantizedTensor::to_f32_vec
    (restated as orc.q4_to_f32) on the same weights, then rounded like the kernel."""
    torch = torch_dev
    n, k = 67, 2048
    w = weights(n, k, seed=21, std=0.5)
    data = orc.q4_from_f32(w)
    nib, sc = orc.extract_for_gpu(data, n, k)
    awq = (np.random.default_rng(22).uniform(0.25, 4.0, k).astype(np.float32)) if with_awq else None
    ref = orc.q4_to_f32(data, n, k, awq)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    out = hk.dequant_w4(up(torch, nib), up(torch, sc), n, k, None if awq is None else up(torch, awq), dtype=tdt)
    torch.cuda.synchronize()
    if dtype == "f32":
        assert np.array_equal(down(out).view(np.uint32), ref.view(np.uint32))
    elif dtype == "f16":
        assert np.array_equal(down(out).view(np.uint16), ref.astype(np.float16).view(np.uint16))
    else:
        got = down(out.view(torch.int16)).view(np.uint16)
        assert np.array_equal(got, orc.f32_to_bf16_bits(ref).reshape(ref.shape))


def test_dequant_w4a16_drop_in(orc, torch_dev, hk):
    from nve_amd._lib import lib
    torch = torch_dev
    n, k = 40, 4096
    data = orc.q4_from_f32(weights(n, k, seed=23))
    nib, sc = orc.extract_for_gpu(data, n, k)
    out = torch.empty((n, k), dtype=torch.float16, device="cuda")
    tn, ts = up(torch, nib), up(torch, sc)
    lib().nve_dequant_w4a16(tn.data_ptr(), ts.data_ptr(), None, out.data_ptr(), n, k,
                            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert lib().nve_hip_last_status() == 0
    assert np.array_equal(down(out).view(np.uint16), orc.q4_to_f32(data, n, k).astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# batched W4A8
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("n,k", [(300, 4096), (14336, 4096)])
def test_w4a8_batched_parity(orc, torch_dev, hk, m, per_token, n, k):
    """configs[3] at the Llama-3.1-8B gate shape (and a small ragged one)."""
    torch = torch_dev
    _, _, nib, ws = _problem(orc, n, k, seed=m)
    x = to_bf16(activations(k, seed=200 + m, m=m))
    xq, xs = hk.quantize_q8_rows(up(torch, x).to(torch.bfloat16), per_token=per_token)
    y = hk.matvec_w4a8_batched(xq, xs, up(torch, nib), up(torch, ws), n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y = down(y)
    for r in range(m):
        if per_token:
            q, s = orc.quantize_q8_rows_bf16(x[r])
            ref = orc.matvec_w4a8_f64(q[0], orc.bf16_bits_to_f32(s), nib, ws, n, k, xs_mode=1)
        else:
            q, s = orc.quantize_q8_group(x[r])
            ref = orc.matvec_w4a8_f64(q, s, nib, ws, n, k)
        assert rel_err_floor(y[r], ref) <= TOL_W4A8, r


# ---------------------------------------------------------------------------
# full-size suites (Llama-3.2-1B, Llama-3.1-8B layer shapes) on sampled rows
# ---------------------------------------------------------------------------
SUITE_1B = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192)]
SUITE_8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


@pytest.mark.parametrize("n,k", SUITE_1B + SUITE_8B)
def test_suite_shapes_sampled_rows(orc, torch_dev, hk, n, k):
    torch = torch_dev
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    nib, sc = hk.q4_quantize(w)
    rows = np.sort(np.random.default_rng(n).choice(n, size=min(n, 192), replace=False))
    rows[-1] = n - 1
    rows_t = torch.from_numpy(rows).cuda()
    w_rows = down(w[rows_t])
    nib_ref, sc_ref = orc.extract_for_gpu(orc.q4_from_f32(w_rows), len(rows), k)
    nib_s, sc_s = down(nib[rows_t]), down(sc[rows_t])
    del w
    assert np.array_equal(nib_s, nib_ref) and np.array_equal(sc_s, sc_ref)
    x = activations(k, seed=k)
    # W4A8
    x16 = to_f16(x)
    xq, xs = hk.quantize_f16_q8(up(torch, x.astype(np.float16)))
    y8 = down(hk.matvec_w4a8(xq, xs, nib, sc, n, k, out_dtype=torch.float32))[0][rows]
    xq_ref, xs_ref = orc.quantize_q8_group(x16)
    assert rel_err_floor(y8, orc.matvec_w4a8_f64(xq_ref, xs_ref, nib_ref, sc_ref, len(rows), k)) <= TOL_W4A8
    # W4A16 (bf16 activations)
    xb = to_bf16(x)
    y16 = down(hk.fused_matvec_w4a16(up(torch, xb).to(torch.bfloat16), nib, sc, None, n, k,
                                     out_dtype=torch.float32))[0][rows]
    assert rel_err_floor(y16, orc.matvec_w4a16_f64(xb, nib_ref, sc_ref, len(rows), k)) <= TOL_W4A16


def test_dispatch_project(orc, torch_dev, hk, monkeypatch):
    """gpu_layer.use_w4a8 + project: the branch taken follows the env rules."""
    torch = torch_dev
    from nve_amd.gpu_layer import GpuW4, project, use_w4a8
    n, k = 256, 2048
    _, _, nib, sc = _problem(orc, n, k, seed=1)
    w = GpuW4(up(torch, nib), up(torch, sc), None, n, k)
    x = to_f16(activations(k, seed=2))
    xt = up(torch, x.astype(np.float16))
    monkeypatch.delenv("NVE_NO_W4A8", raising=False)
    monkeypatch.delenv("NVE_W4A8_THRESHOLD", raising=False)
    assert use_w4a8(0.0) and not use_w4a8(1.0)
    y8 = down(project(xt, w, use_w4a8(0.0), out_dtype=torch.float32))[0]
    y16 = down(project(xt, w, use_w4a8(1.0), out_dtype=torch.float32))[0]
    q, s = orc.quantize_q8_group(x)
    assert rel_err_floor(y8, orc.matvec_w4a8_f64(q, s, nib, sc, n, k)) <= TOL_W4A8
    assert rel_err_floor(y16, orc.matvec_w4a16_f64(x, nib, sc, n, k)) <= TOL_W4A16


@pytest.mark.parametrize("m", [2, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("n,k", [(16, 32), (17, 96), (300, 160), (1000, 2048), (8200, 4096), (70, 14336),
                                 (4096, 14336), (14336, 4096), (6000, 4096), (12000, 4096), (4097, 2048),
                                 (16384, 1024), (16400, 1024)])
@pytest.mark.parametrize("per_token", [False, True])
def test_w4a8_batched_mfma_shapes(orc, torch_dev, hk, m, n, k, per_token):
    """M >= 3 runs on the int8 MFMA kernels (M = 2 on the staged v_dot4 kernel where it
    fits): ragged N, K with a partial last block quad (K % 128 != 0: the register kernel
    with scalar scale loads), the LDS-ring kernel at 1-4 tiles per workgroup with a
    partly masked last tile (4097, 6000, 8200, 12000, 14336 rows: 17, 24, 33, 47, 56 rows
    per workgroup; 16384 rows: four full tiles, the largest ring shape; 16400 rows: past
    it, on the register kernel), every live-element count (M = 4, 5-8, 13-16)."""
    torch = torch_dev
    _, _, nib, ws = _problem(orc, n, k, seed=m * 7 + n)
    x = to_bf16(activations(k, seed=300 + m, m=m))
    xq, xs = hk.quantize_q8_rows(up(torch, x).to(torch.bfloat16), per_token=per_token)
    y = down(hk.matvec_w4a8_batched(xq, xs, up(torch, nib), up(torch, ws), n, k, out_dtype=torch.float32))
    for r in range(m):
        if per_token:
            q, s = orc.quantize_q8_rows_bf16(x[r])
            ref = orc.matvec_w4a8_f64(q[0], orc.bf16_bits_to_f32(s), nib, ws, n, k, xs_mode=1)
        else:
            q, s = orc.quantize_q8_group(x[r])
            ref = orc.matvec_w4a8_f64(q, s, nib, ws, n, k)
        assert rel_err_floor(y[r], ref) <= TOL_W4A8, r


@pytest.mark.parametrize("per_token", [False, True])
def test_w4a8_batched_graph_replay_matches_eager(orc, torch_dev, hk, per_token):
    """The batched kernels (M = 2 and 5 on the LDS-ring kernel, 16 rows on it at T = 2,
    M = 3 on the register kernel at K % 128 != 0) captured in one HIP graph and replayed
    several times, with eager work in between: every replay equals the eager result."""
    torch = torch_dev
    cases = []
    for m, n, k in ((2, 6000, 4096), (5, 6000, 4096), (16, 6000, 4096), (3, 300, 160)):
        _, _, nib, ws = _problem(orc, n, k, seed=m + n)
        x = to_bf16(activations(k, seed=50 + m, m=m))
        xq, xs = hk.quantize_q8_rows(up(torch, x).to(torch.bfloat16), per_token=per_token)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        cases.append((xq, xs, up(torch, nib), up(torch, ws), n, k, out))

    def step():
        for xq, xs, nib, ws, n, k, out in cases:
            hk.matvec_w4a8_batched(xq, xs, nib, ws, n, k, out=out)
    step()
    torch.cuda.synchronize()
    eager = [c[-1].clone() for c in cases]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        for c in cases:
            c[-1].fill_(float("nan"))
        step()  # eager work between replays
        torch.cuda.synchronize()
        for c in cases:
            c[-1].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[-1], e)


# ---------------------------------------------------------------------------
# W4A8 GEMV with the activation quantization fused in (nve_hip_matvec_w4a8_x)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,k", [(300, 4096), (4096, 14336), (128256 // 64, 4096), (64, 32)])
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("odt", ["f32", "f16"])
def test_w4a8_fused_quantize_bit_identical(orc, torch_dev, hk, n, k, xdt, odt):
    """One launch = nve_hip_quantize_q8 + nve_hip_matvec_w4a8, bit for bit; and the
    int8 codes it forms are the oracle's (checked through the two-launch path)."""
    torch = torch_dev
    _, _, nib, ws = _problem(orc, n, k, seed=n + k)
    x = activations(k, seed=k + 3)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[xdt]
    xt = up(torch, x).to(tdt)
    odt_t = torch.float32 if odt == "f32" else torch.float16
    tn, tw = up(torch, nib), up(torch, ws)
    y1 = hk.matvec_w4a8_x(xt, tn, tw, n, k, out_dtype=odt_t)
    xq, xs = hk.quantize_f16_q8(xt)
    y2 = torch.empty(n, dtype=odt_t, device="cuda")
    hk.matvec_w4a8_into(xq, xs, tn, tw, y2, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16 if odt == "f16" else torch.int32),
                       y2.view(torch.int16 if odt == "f16" else torch.int32))
    xq_ref, _ = orc.quantize_q8_group(down(xt.float()))
    assert np.array_equal(down(xq), xq_ref)


@pytest.mark.parametrize("xdt", ["f16", "f32"])
def test_w4a8_fused_quantize_nonfinite(orc, torch_dev, hk, xdt):
    """NaN / +-Inf activations through the fused quantize + GEMV: bit-identical to the
    two-launch sequence (the infinite-scale groups make their outputs NaN in both)."""
    torch = torch_dev
    from test_oracle import _nonfinite_groups
    n, k = 96, 256
    _, _, nib, ws = _problem(orc, n, k, seed=5)
    x = np.tile(_nonfinite_groups(), 2)
    x[128:] = np.where(np.isfinite(x[128:]), x[128:], 0.5)  # second half finite
    xt = up(torch, x.astype(np.float16)) if xdt == "f16" else up(torch, x)
    tn, tw = up(torch, nib), up(torch, ws)
    y1 = hk.matvec_w4a8_x(xt, tn, tw, n, k, out_dtype=torch.float32)
    xq, xs = hk.quantize_f16_q8(xt)
    y2 = torch.empty(n, dtype=torch.float32, device="cuda")
    hk.matvec_w4a8_into(xq, xs, tn, tw, y2, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    q_ref, s_ref = orc.quantize_q8_group(down(xt.float()))
    assert np.array_equal(down(xq), q_ref) and np.array_equal(down(xs).view(np.uint32), s_ref.view(np.uint32))


def test_w4a8_fused_quantize_grouped(orc, torch_dev, hk):
    torch = torch_dev
    k = 4096
    mats, refs = [], []
    x = up(torch, activations(k, seed=77)).to(torch.float16)
    xq, xs = hk.quantize_f16_q8(x)
    for i, n in enumerate((4096, 1024, 1024)):
        _, _, nib, ws = _problem(orc, n, k, seed=90 + i)
        tn, tw = up(torch, nib), up(torch, ws)
        mats.append((tn, tw, n))
        r = torch.empty(n, dtype=torch.float32, device="cuda")
        hk.matvec_w4a8_into(xq, xs, tn, tw, r, n, k)
        refs.append(r)
    outs = hk.grouped_matvec_w4a8_x(x, mats, k)
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert torch.equal(o, r)
