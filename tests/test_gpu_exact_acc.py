"""Exact int32 accumulators of every shipping W4A8 kernel, seen through its fp32 output.

The W4A8 GEMV computes y[n] = sum_b ws[n,b] * xs[b] * acc[n,b] with acc[n,b] the exact
int32 sum over block b of (nibble - 8) * xq (cuda/nve_kernels.cu:835-858).  When every
weight scale and activation scale is a power of two, ws * xs = c_b * 2^e with small
integers c_b, and when sum_b |c_b * acc[n,b]| < 2^24 every product, every partial sum
(in any order, any split over lanes / waves / MFMA tiles) and the result are exactly
representable in fp32.  The fp32 output must then equal 2^e * sum_b c_b * acc[n,b]
bit for bit: a single accumulator that is off by one, a block paired with the wrong
scale, or a dropped or doubled block changes the output.  The accumulators themselves
come from the oracle (orc_w4a8_block_acc, pinned against a brute-force unpacking in
test_oracle.py), so this compares the production kernels with the oracle exactly --
not the debug export nve_hip_w4a8_block_acc, which shares only the block dot.

Kernels covered: the one-shot GEMV, the persistent GEMV, the GEMV that quantizes its
own fp16 / bf16 / fp32 input (inputs built so the quantizer returns the chosen int8
codes with power-of-two scales), the grouped launches (pre-quantized and quantizing,
1-3 matrices), the drop-in nve_matvec_w4a8 (fp16 output = the exact value rounded
once), and the batched kernel at M = 1 (v_dot4) and M = 2..16 (int8 MFMA) in both
activation-scale modes.  Shapes include the Llama-3.1-8B layer shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIM = 1 << 24


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nve_amd import hip_kernels as hk
    from nve_amd._lib import GEMV_AUTO, GEMV_ONESHOT, GEMV_PERSISTENT, lib
    L = lib()
    yield torch, hk, L, {"auto": GEMV_AUTO, "oneshot": GEMV_ONESHOT, "persistent": GEMV_PERSISTENT}
    L.nve_hip_set_gemv_policy(GEMV_AUTO, 2, 4)


def _pow2(g, shape, lo, hi):
    return np.ldexp(np.float32(1.0), g.integers(lo, hi + 1, size=shape)).astype(np.float32)


def _weights(n, k, seed, ws_spread):
    """Random nibbles (every byte value is a valid pair of codes) and power-of-two
    weight scales 2^-9 .. 2^(-9+ws_spread)."""
    g = np.random.default_rng(seed)
    nib = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    ws = _pow2(g, (n, k // 32), -9, -9 + ws_spread)
    return nib, ws


def _acts(k, seed, m=1):
    """int8 codes in [-127, 127] with +-127 in every group (so a quantizer that sees
    xq * 2^e returns exactly these codes and the scale 2^e), and power-of-two group
    exponents e in [-4, -3]."""
    g = np.random.default_rng(seed)
    xq = g.integers(-127, 128, size=(m, k), dtype=np.int16)
    pos = g.integers(0, 32, size=(m, k // 32))
    sign = np.where(g.random((m, k // 32)) < 0.5, -127, 127)
    for b in range(k // 32):
        xq[np.arange(m), 32 * b + pos[:, b]] = sign[:, b]
    e = g.integers(-4, -2, size=(m, k // 32))
    return xq.astype(np.int8), e


def _expected(orc, xq_row, xs_row, nib, ws, n, k):
    """Exact 2^e * sum_b c_b * acc[n, b] as float32, asserting the < 2^24 precondition."""
    acc = orc.w4a8_block_acc(xq_row, nib, n, k).astype(np.int64)
    sc = ws.astype(np.float64) * xs_row.astype(np.float64)[None, :]
    e_min = np.floor(np.log2(sc.min()))
    c = np.rint(sc / 2.0 ** e_min).astype(np.int64)
    assert np.all(c.astype(np.float64) * 2.0 ** e_min == sc)
    terms = c * acc
    assert int(np.abs(terms).sum(axis=1).max()) < LIM, "test precondition: exact fp32 sums"
    y = terms.sum(axis=1).astype(np.float64) * 2.0 ** e_min
    y32 = y.astype(np.float32)
    assert np.all(y32.astype(np.float64) == y)
    return y32


def _spread(k):
    # keep sum |c * acc| < 2^24: wider scale spreads only for short rows
    return 2 if k <= 8192 else (1 if k <= 16384 else 0)


SHAPES = [(1, 32), (5, 96), (37, 160), (130, 1056), (2048, 2048), (1024, 4096), (4096, 4096), (14336, 4096),
          (4096, 14336), (300, 8192), (64, 16384), (40, 16416), (16, 32768)]


def _up(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("policy", ["oneshot", "persistent"])
def test_w4a8_gemv_exact(orc, env, n, k, policy):
    torch, hk, L, pol = env
    print(f"exact w4a8 gemv n={n} k={k} policy={policy}", flush=True)
    nib, ws = _weights(n, k, seed=n * 7 + k, ws_spread=_spread(k))
    xq, e = _acts(k, seed=k + 3)
    xs = np.ldexp(np.float32(1.0), e[0]).astype(np.float32)
    ref = _expected(orc, xq[0], xs, nib, ws, n, k)
    tn, tw, tq, ts = _up(torch, nib), _up(torch, ws), _up(torch, xq[0]), _up(torch, xs)
    L.nve_hip_set_gemv_policy(pol[policy], 2, 4)
    try:
        y = hk.matvec_w4a8(tq, ts, tn, tw, n, k, out_dtype=torch.float32)
        y16 = hk.matvec_w4a8(tq, ts, tn, tw, n, k)
        torch.cuda.synchronize()
    finally:
        L.nve_hip_set_gemv_policy(pol["auto"], 2, 4)
    got = y.cpu().numpy()[0]
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), int(np.sum(got != ref))
    assert np.array_equal(y16.cpu().numpy()[0], ref.astype(np.float16))


def test_w4a8_dropin_exact(orc, env):
    """The reference-named void launcher (fp16 output)."""
    torch, hk, L, pol = env
    n, k = 4096, 4096
    nib, ws = _weights(n, k, seed=99, ws_spread=2)
    xq, e = _acts(k, seed=98)
    xs = np.ldexp(np.float32(1.0), e[0]).astype(np.float32)
    ref = _expected(orc, xq[0], xs, nib, ws, n, k)
    tn, tw, tq, ts = _up(torch, nib), _up(torch, ws), _up(torch, xq[0]), _up(torch, xs)
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    L.nve_matvec_w4a8(tq.data_ptr(), ts.data_ptr(), tn.data_ptr(), tw.data_ptr(), out.data_ptr(), n, k,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref.astype(np.float16))


def _x_for(xq_row, e_row, xdt):
    """The activation vector whose group-32 quantization is (xq_row, 2^e_row)."""
    x = xq_row.astype(np.float32) * np.repeat(np.ldexp(np.float32(1.0), e_row), 32).astype(np.float32)
    return x


@pytest.mark.parametrize("n,k", [(1, 32), (37, 160), (2048, 2048), (1024, 4096), (14336, 4096), (4096, 14336),
                                 (64, 16384)])
@pytest.mark.parametrize("xdt", ["f16", "bf16", "f32"])
def test_w4a8_quantizing_gemv_exact(orc, env, n, k, xdt):
    """nve_hip_matvec_w4a8_x: quantization inside the GEMV, then the exact block sums."""
    torch, hk, L, pol = env
    print(f"exact w4a8_x n={n} k={k} x={xdt}", flush=True)
    nib, ws = _weights(n, k, seed=n + 5 * k, ws_spread=_spread(k))
    xq, e = _acts(k, seed=2 * k + 1)
    xs = np.ldexp(np.float32(1.0), e[0]).astype(np.float32)
    ref = _expected(orc, xq[0], xs, nib, ws, n, k)
    x = _x_for(xq[0], e[0], xdt)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[xdt]
    xt = _up(torch, x).to(tdt)
    assert np.array_equal(xt.float().cpu().numpy(), x)  # representable in the input dtype
    qq, qs = hk.quantize_f16_q8(xt)
    assert np.array_equal(qq.cpu().numpy(), xq[0]) and np.array_equal(qs.cpu().numpy(), xs)
    y = hk.matvec_w4a8_x(xt, _up(torch, nib), _up(torch, ws), n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), int(np.sum(got != ref))


@pytest.mark.parametrize("ns,k", [((4096, 1024, 1024), 4096), ((14336, 14336), 4096), ((5, 300, 37), 1056),
                                  ((3072,), 3072)])
@pytest.mark.parametrize("mode", ["xq_oneshot", "xq_persistent", "x_f16"])
def test_w4a8_grouped_exact(orc, env, ns, k, mode):
    """Grouped launches: nve_hip_grouped_matvec_w4a8 (both kernel shapes) and the
    quantizing nve_hip_grouped_matvec_w4a8_x; every matrix's output exact."""
    torch, hk, L, pol = env
    from nve_amd._lib import W4Mat
    print(f"exact grouped ns={ns} k={k} mode={mode}", flush=True)
    xq, e = _acts(k, seed=k + len(ns))
    xs = np.ldexp(np.float32(1.0), e[0]).astype(np.float32)
    mats, refs, outs, keep = [], [], [], []
    for i, n in enumerate(ns):
        nib, ws = _weights(n, k, seed=31 * i + n, ws_spread=_spread(k))
        refs.append(_expected(orc, xq[0], xs, nib, ws, n, k))
        tn, tw = _up(torch, nib), _up(torch, ws)
        o = torch.empty(n, dtype=torch.float32, device="cuda")
        keep += [tn, tw]
        outs.append(o)
        mats.append(W4Mat(tn.data_ptr(), tw.data_ptr(), None, o.data_ptr(), n))
    arr = (W4Mat * len(mats))(*mats)
    s = torch.cuda.current_stream().cuda_stream
    if mode == "x_f16":
        xt = _up(torch, _x_for(xq[0], e[0], "f16")).to(torch.float16)
        st = L.nve_hip_grouped_matvec_w4a8_x(xt.data_ptr(), 0, arr, len(mats), 2, k, s)
    else:
        tq, ts = _up(torch, xq[0]), _up(torch, xs)
        L.nve_hip_set_gemv_policy(pol["oneshot" if mode == "xq_oneshot" else "persistent"], 2, 4)
        try:
            st = L.nve_hip_grouped_matvec_w4a8(tq.data_ptr(), ts.data_ptr(), arr, len(mats), 2, k, s)
            torch.cuda.synchronize()
        finally:
            L.nve_hip_set_gemv_policy(pol["auto"], 2, 4)
    assert st == 0
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        got = o.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), r.view(np.uint32)), int(np.sum(got != r))


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (37, 160), (300, 2048), (6000, 4096), (8200, 4096)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("xs_mode", ["group_f32", "row_bf16"])
def test_w4a8_batched_exact(orc, env, n, k, m, xs_mode):
    """Batched W4A8: M = 1 on the one-row GEMV; M >= 2 on the LDS-ring int8 MFMA kernel
    (with the -8 correction MFMA) where K % 128 == 0 and each wave has a full ring of
    quads; otherwise M = 2 on the staged v_dot4 kernel (the shapes here all fit its LDS)
    and M >= 3 on the register MFMA kernel;
    every row of every activation exact.  Row mode: one power-of-two bf16 scale per
    activation row (bf16 2^e is exact)."""
    torch, hk, L, pol = env
    print(f"exact batched n={n} k={k} m={m} xs={xs_mode}", flush=True)
    nib, ws = _weights(n, k, seed=n + k + m, ws_spread=_spread(k))
    xq, e = _acts(k, seed=k + 17 * m, m=m)
    if xs_mode == "row_bf16":
        e = np.repeat(e[:, :1], k // 32, axis=1)
    xs = np.ldexp(np.float32(1.0), e).astype(np.float32)
    refs = np.stack([_expected(orc, xq[i], xs[i], nib, ws, n, k) for i in range(m)])
    tq = _up(torch, xq)
    if xs_mode == "row_bf16":
        ts = _up(torch, xs[:, 0].copy()).to(torch.bfloat16)
    else:
        ts = _up(torch, xs)
    y = hk.matvec_w4a8_batched(tq, ts, _up(torch, nib), _up(torch, ws), n, k, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    bad = got.view(np.uint32) != refs.view(np.uint32)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} outputs differ"


@pytest.mark.parametrize("n,k", [(300, 2048), (4096, 14336)])
@pytest.mark.parametrize("m", [3, 5])
@pytest.mark.parametrize("xs_mode", ["group_f32", "row_bf16"])
def test_w4a8_batched_dot4_exact(orc, env, n, k, m, xs_mode):
    """The v_dot4 batched kernel (one wave per row, activations read per row), which the
    one-shot kernel policy selects for M >= 3: exact like the other batched kernels."""
    torch, hk, L, pol = env
    print(f"exact batched dot4 n={n} k={k} m={m} xs={xs_mode}", flush=True)
    nib, ws = _weights(n, k, seed=n + k + m + 1, ws_spread=_spread(k))
    xq, e = _acts(k, seed=k + 19 * m, m=m)
    if xs_mode == "row_bf16":
        e = np.repeat(e[:, :1], k // 32, axis=1)
    xs = np.ldexp(np.float32(1.0), e).astype(np.float32)
    refs = np.stack([_expected(orc, xq[i], xs[i], nib, ws, n, k) for i in range(m)])
    tq = _up(torch, xq)
    ts = _up(torch, xs[:, 0].copy()).to(torch.bfloat16) if xs_mode == "row_bf16" else _up(torch, xs)
    L.nve_hip_set_gemv_policy(pol["oneshot"], 2, 4)
    try:
        y = hk.matvec_w4a8_batched(tq, ts, _up(torch, nib), _up(torch, ws), n, k, out_dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        L.nve_hip_set_gemv_policy(pol["auto"], 2, 4)
    got = y.cpu().numpy()
    bad = got.view(np.uint32) != refs.view(np.uint32)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} outputs differ"
