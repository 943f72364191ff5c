"""Pins for the CPU oracle (oracle/oracle.c) -- known answers, reference unit tests,
independent brute force and invariants.  CPU only.

Reference test inputs re-expressed here: src/quantize.rs:2234-2252
(test_quantize_block_q4_roundtrip) and 2274-2290 (test_q4_matvec).
"""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest

from helpers import activations, rel_err_floor, weights

F32 = np.float32


def _scale_bytes(v: float) -> list[int]:
    return list(struct.pack("<f", float(F32(v))))


# ---------------------------------------------------------------------------
# scalar semantics
# ---------------------------------------------------------------------------
def test_rust_as_i8_saturates(orc):
    L = orc.lib()
    cases = {math.nan: 0, math.inf: 127, -math.inf: -128, 127.9: 127, 300.0: 127,
             -128.5: -128, -1e9: -128, 3.99: 3, -3.99: -3, 0.0: 0}
    for v, want in cases.items():
        assert L.orc_rust_f32_as_i8(v) == want, v


def test_half_conversions_match_numpy(orc):
    L = orc.lib()
    g = np.random.default_rng(1)
    vals = np.concatenate([g.standard_normal(2000).astype(F32) * F32(100),
                           np.array([0.0, -0.0, 65504.0, 65520.0, 1e-7, 6e-8, 2.98e-8, 1e6, np.inf, -np.inf], F32)])
    for v in vals:
        with np.errstate(over="ignore"):
            want = int(np.float16(v).view(np.uint16))
        assert L.orc_f32_to_f16(float(v)) == want, v
    for h in range(0, 65536, 7):
        f = np.uint16(h).view(np.float16)
        want = np.float32(f)
        got = L.orc_f16_to_f32(h)
        if np.isnan(want):
            assert math.isnan(got)
        else:
            assert got == want, hex(h)


def test_bf16_conversion_rne(orc):
    # 1 + 2^-8 is a tie between 1.0 and 1 + 2^-7: even mantissa -> 1.0 (0x3F80)
    assert orc.f32_to_bf16_bits(np.array([1.0 + 2**-8]))[0] == 0x3F80
    # 1 + 3*2^-8 ties between 1+2^-7 (odd) and 1+2^-6 (even) -> 0x3F82
    assert orc.f32_to_bf16_bits(np.array([1.0 + 3 * 2**-8]))[0] == 0x3F82
    assert orc.f32_to_bf16_bits(np.array([0.7874015748]))[0] == 0x3F4A
    assert orc.bf16_bits_to_f32([0x3F4A])[0] == F32(0.7890625)


# ---------------------------------------------------------------------------
# quantize_block_q4 (src/quantize.rs:711-731): hand-derived known answers
# ---------------------------------------------------------------------------
def test_q4_block_kat_reference_ramp(orc):
    # values (i - 16) * 0.5 (the reference unit test's input): amax 8, scale
    # fl(8/7) = 1.14285719..., inv = fl(1/scale) = 0.87499994 (just below 7/8), so
    # v*inv = (i-16)*7/16 except at v = +-4 where it is +-3.4999998 and rounds to +-3
    # (a quantizer that divided v/scale instead would get +-3.5 -> +-4).  Nibbles
    # worked out by hand with half-away-from-zero rounding.
    v = (np.arange(32, dtype=F32) - F32(16)) * F32(0.5)
    out = orc.quantize_block_q4(v)
    assert list(out[:4]) == _scale_bytes(F32(8.0) / F32(7.0))
    assert F32(1.0) / (F32(8.0) / F32(7.0)) == F32(0.87499994)
    want = [0x11, 0x22, 0x33, 0x44, 0x55, 0x65, 0x76, 0x87,
            0x88, 0x99, 0xAA, 0xBB, 0xCB, 0xDC, 0xED, 0xFE]
    assert list(out[4:]) == want


def test_q4_block_kat_ties_half_away_from_zero(orc):
    # amax 7 -> scale 1, inv 1; ties k+0.5 with even k separate f32::round (half away
    # from zero) from round-half-even.
    v = np.zeros(32, F32)
    v[:10] = [7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 6.5, -6.5, 3.5]
    out = orc.quantize_block_q4(v)
    assert list(out[:4]) == _scale_bytes(1.0)
    q = [15, 11, 5, 9, 7, 10, 6, 15, 1, 12] + [8] * 22
    want = [q[2 * i] | (q[2 * i + 1] << 4) for i in range(16)]
    assert list(out[4:]) == want


def test_q4_block_kat_zero_block(orc):
    out = orc.quantize_block_q4(np.zeros(32, F32))
    assert list(out) == [0, 0, 0, 0] + [0x88] * 16


def test_q4_block_kat_infinite_inverse_scale(orc):
    # amax = 1e-38 (subnormal): scale = amax/7 > 0 but 1/scale overflows to +inf.
    # Saturating casts: +inf -> 127 -> clamp 7 -> nibble 15; -inf -> -128 -> -8 -> 0;
    # 0 * inf = NaN -> 0 -> nibble 8.  (Nibble 0 is reachable only here.)
    v = np.zeros(32, F32)
    v[0], v[1], v[3] = F32(1e-38), F32(-1e-38), F32(5e-39)
    s = F32(1e-38) / F32(7.0)
    with np.errstate(over="ignore"):
        assert s > 0 and np.isinf(F32(1.0) / s)
    out = orc.quantize_block_q4(v)
    assert list(out[:4]) == list(struct.pack("<f", float(s)))
    assert list(out[4:]) == [0x0F, 0xF8] + [0x88] * 14


def test_q4_block_kat_scale_underflow(orc):
    v = np.zeros(32, F32)
    v[7] = F32(2.0**-149)  # amax/7 rounds to 0 -> scale 0, inv 0, all nibbles 8
    out = orc.quantize_block_q4(v)
    assert list(out) == [0, 0, 0, 0] + [0x88] * 16


def test_q4_block_single_nonzero(orc):
    v = np.zeros(32, F32)
    v[5] = -3.0
    out = orc.quantize_block_q4(v)
    nib = [out[4 + i // 2] >> (4 * (i & 1)) & 15 for i in range(32)]
    assert nib[5] == 1 and all(n == 8 for i, n in enumerate(nib) if i != 5)


def test_reference_unit_test_roundtrip(orc):
    # src/quantize.rs:2234-2252: |orig - deq| < 2.0
    v = (np.arange(32, dtype=F32) - 16) * F32(0.5)
    data = orc.quantize_block_q4(v)
    deq = orc.q4_to_f32(data, 1, 32)[0]
    assert np.all(np.abs(v - deq) < 2.0)


def test_reference_unit_test_matvec(orc):
    # src/quantize.rs:2274-2290: 2x32 one-hot rows, x[0]=5, x[1]=3, y within 2.0
    w = np.zeros((2, 32), F32)
    w[0, 0] = 1.0
    w[1, 1] = 1.0
    data = orc.q4_from_f32(w)
    x = np.zeros(32, F32)
    x[0], x[1] = 5.0, 3.0
    for avx in (False, True):
        y = orc.q4_matvec_f32(data, 2, 32, x, avx2=avx)
        assert abs(y[0] - 5.0) < 2.0 and abs(y[1] - 3.0) < 2.0
        # one-hot rows dequantize to 7 * fl(1/7) = 1 + 1 ulp-ish: y within 1e-6
        assert abs(y[0] - 5.0) < 1e-5 and abs(y[1] - 3.0) < 1e-5


def test_q4_invariants_random(orc):
    w = weights(64, 256, seed=11)
    data = orc.q4_from_f32(w).reshape(64, 8, 20)
    sc = data[:, :, :4].copy().view(np.float32)[..., 0]
    nib = data[:, :, 4:]
    lo, hi = nib & 15, nib >> 4
    assert lo.min() >= 1 and hi.min() >= 1  # nibble 0 unreachable for finite input
    deq = orc.q4_to_f32(orc.q4_from_f32(w), 64, 256).reshape(64, 8, 32)
    err = np.abs(deq - w.reshape(64, 8, 32))
    assert np.all(err <= sc[..., None] * 0.5 * (1 + 1e-5) + 1e-30)


def test_q4_to_f32_kat_and_awq(orc):
    blk = np.array(_scale_bytes(0.5) + [0x80] + [0x8F] + [0x88] * 14, np.uint8)
    deq = orc.q4_to_f32(blk, 1, 32)[0]
    want = np.zeros(32, F32)
    want[0] = -4.0   # nibble 0
    want[1] = 0.0    # nibble 8
    want[2] = 3.5    # nibble 15
    want[3] = 0.0
    assert np.array_equal(deq, want)
    awq = np.full(32, 2.0, F32)
    assert np.array_equal(orc.q4_to_f32(blk, 1, 32, awq_inv=awq)[0], want * 2)


# ---------------------------------------------------------------------------
# extract_for_gpu (src/quantize.rs:437-463)
# ---------------------------------------------------------------------------
def _cpu_elems(data, n, k):
    b = data.reshape(n, k // 32, 20)[:, :, 4:]
    e = np.empty((n, k // 32, 32), np.uint8)
    e[:, :, 0::2] = b & 15
    e[:, :, 1::2] = b >> 4
    return e


def _gpu_elems(nib, n, k):
    # Read side of the reference kernels: lane t < 16 takes the low nibble of byte t,
    # lane t >= 16 the high nibble of byte t-16 (cuda/nve_kernels.cu:357-362).
    g = nib.reshape(n, k // 32, 16)
    return np.concatenate([g & 15, g >> 4], axis=2)


def test_extract_for_gpu_bijection(orc):
    n, k = 24, 320
    data = orc.q4_from_f32(weights(n, k, seed=5, std=1.0))
    nib, sc = orc.extract_for_gpu(data, n, k)
    assert np.array_equal(_gpu_elems(nib, n, k), _cpu_elems(data, n, k))
    assert np.array_equal(sc, data.reshape(n, k // 32, 20)[:, :, :4].copy().view(np.float32)[..., 0])


def test_extract_for_gpu_kat_one_block(orc):
    # elements e_i = i & 15 in CPU order -> GPU byte j = e_j | e_{j+16} << 4
    cpu = bytes([(2 * i & 15) | ((2 * i + 1) & 15) << 4 for i in range(16)])
    blk = np.frombuffer(_scale_bytes_raw(1.25) + cpu, np.uint8)
    nib, sc = orc.extract_for_gpu(blk, 1, 32)
    assert sc[0, 0] == F32(1.25)
    assert list(nib[0]) == [(j & 15) | (((j + 16) & 15) << 4) for j in range(16)]


def _scale_bytes_raw(v):
    return struct.pack("<f", v)


# ---------------------------------------------------------------------------
# CPU GEMV (src/quantize.rs:466-488, 844-938)
# ---------------------------------------------------------------------------
def _f64_ref(data, n, k, x, awq_inv=None):
    w = orc_mod().q4_to_f32(data, n, k).astype(np.float64)
    xe = x.astype(np.float64) if awq_inv is None else (x * awq_inv).astype(np.float64)
    return w @ xe, np.abs(w) @ np.abs(xe)


def orc_mod():
    from oracle import oracle
    return oracle


@pytest.mark.parametrize("n,k", [(1, 32), (7, 96), (33, 2048), (64, 4096)])
def test_cpu_gemv_scalar_and_avx2_vs_f64(orc, n, k):
    w = weights(n, k, seed=n * 7 + k)
    x = activations(k, seed=k)
    data = orc.q4_from_f32(w)
    ref, mag = _f64_ref(data, n, k, x)
    bound = 2 * (k + 8) * 2.0**-24 * mag  # gamma_n * sum |w x|, generous constant
    for avx in (False, True):
        y = orc.q4_matvec_f32(data, n, k, x, avx2=avx)
        assert np.all(np.abs(y - ref) <= bound), (avx, np.max(np.abs(y - ref) / bound))


def test_cpu_gemv_row_split_invariant(orc):
    n, k = 97, 1024
    data = orc.q4_from_f32(weights(n, k, seed=3))
    x = activations(k, seed=4)
    rows = np.array([orc.q4_dot_row(data[i], x, avx2=True) for i in range(n)], F32)
    for t in (1, 3, 8):
        assert np.array_equal(orc.q4_matvec_f32(data, n, k, x, threads=t), rows)


def test_cpu_gemv_awq(orc):
    n, k = 40, 512
    data = orc.q4_from_f32(weights(n, k, seed=8))
    x = activations(k, seed=9)
    awq_inv = (1.0 / np.linspace(0.5, 2.0, k)).astype(F32)
    ref, mag = _f64_ref(data, n, k, x, awq_inv)
    y = orc.q4_matvec_f32(data, n, k, x, awq_inv=awq_inv)
    assert np.all(np.abs(y - ref) <= 2 * (k + 8) * 2.0**-24 * mag)


# ---------------------------------------------------------------------------
# W4A8 activation quantization (cuda/nve_kernels.cu:712-745)
# ---------------------------------------------------------------------------
def test_q8_group_kat(orc):
    x = np.zeros(64, F32)
    x[:8] = [127.0, 2.5, 3.5, -2.5, -127.0, 0.5, 1.5, -0.5]  # scale 1: RNE ties
    xq, sc = orc.quantize_q8_group(x)
    assert sc[0] == 1.0 and sc[1] == 1.0  # second group all zero -> scale 1
    assert list(xq[:8]) == [127, 2, 4, -2, -127, 0, 2, 0]
    assert np.all(xq[32:] == 0)


def _nonfinite_groups():
    x = np.zeros(128, F32)
    x[0], x[1], x[2] = np.nan, 3.0, -1.5   # NaN dropped by fmaxf: amax 3
    x[32], x[33] = np.inf, 1.0             # amax inf: scale inf, 1/scale 0
    x[64:96] = np.nan                      # all NaN: amax not > 0 -> scale 1
    x[96], x[97] = -np.inf, -2.0
    return x


def test_q8_group_kat_nonfinite(orc):
    """cuda/nve_kernels.cu:712-745 on NaN / Inf: the fmaxf tree ignores NaN, a group
    whose amax is not > 0 keeps scale 1, __float2int_rn(NaN) is 0, and an infinite
    amax gives scale inf, 1/scale = 0, so every code of that group is 0 (inf * 0 is
    NaN -> 0)."""
    xq, sc = orc.quantize_q8_group(_nonfinite_groups())
    assert sc[0] == F32(3.0) / F32(127.0)
    assert list(xq[:3]) == [0, 127, -64]   # -1.5 * 127 / 3 = -63.5 -> -64 (RNE)
    assert np.isposinf(sc[1]) and np.all(xq[32:64] == 0)
    assert sc[2] == 1.0 and np.all(xq[64:96] == 0)
    assert np.isposinf(sc[3]) and np.all(xq[96:128] == 0)


def test_q8_group_brute_force(orc):
    x = activations(4096, seed=21)
    xq, sc = orc.quantize_q8_group(x)
    g = x.reshape(-1, 32)
    amax = np.max(np.abs(g), axis=1)
    s = np.where(amax > 0, amax / F32(127.0), F32(1.0)).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    q = np.clip(np.rint((g * inv[:, None]).astype(F32)), -127, 127).astype(np.int8)
    assert np.array_equal(sc, s) and np.array_equal(xq.reshape(-1, 32), q)
    assert np.all(np.max(np.abs(xq.reshape(-1, 32).astype(int)), axis=1) == 127)


def test_q8_rows_bf16_kat(orc):
    x = np.zeros((2, 64), F32)
    x[0, :5] = [254.0, 1.0, -1.0, 3.0, -254.0]   # s = 2 exactly, inv 0.5
    x[1, :2] = [100.0, -50.0]                    # s = 100/127 -> bf16 0x3F4A = 0.7890625
    xq, sc = orc.quantize_q8_rows_bf16(x)
    assert sc[0] == 0x4000 and sc[1] == 0x3F4A
    assert list(xq[0, :5]) == [127, 0, 0, 2, -127]
    inv = F32(1.0) / F32(0.7890625)
    assert xq[1, 0] == int(np.rint(F32(100.0) * inv)) == 127
    assert xq[1, 1] == int(np.rint(F32(-50.0) * inv)) == -63


# ---------------------------------------------------------------------------
# W4A8 integer accumulators and fp64 product
# ---------------------------------------------------------------------------
def test_w4a8_block_acc_brute_force(orc):
    n, k = 37, 1024
    data = orc.q4_from_f32(weights(n, k, seed=31, std=1.0))
    nib, ws = orc.extract_for_gpu(data, n, k)
    xq, xs = orc.quantize_q8_group(activations(k, seed=32))
    acc = orc.w4a8_block_acc(xq, nib, n, k)
    e = _cpu_elems(data, n, k).astype(np.int64) - 8  # independent (CPU-order) unpack
    want = np.einsum("nbi,bi->nb", e, xq.reshape(k // 32, 32).astype(np.int64))
    assert np.array_equal(acc.astype(np.int64), want)
    y = orc.matvec_w4a8_f64(xq, xs, nib, ws, n, k)
    y_np = (ws.astype(np.float64) * xs.astype(np.float64)[None, :] * want).sum(axis=1)
    assert np.allclose(y, y_np, rtol=1e-12, atol=0)
    y32 = orc.matvec_w4a8_f32(xq, xs, nib, ws, n, k, threads=4)
    assert rel_err_floor(y32, y) < 1e-4


def test_w4a8_extreme_accumulator(orc):
    # every weight nibble 0 (-8) and xq -127: acc = 32 * 1016 per block
    n, k = 2, 64
    nib = np.zeros((n, k // 2), np.uint8)
    xq = np.full(k, -127, np.int8)
    assert np.all(orc.w4a8_block_acc(xq, nib, n, k) == 32 * 8 * 127)


# ---------------------------------------------------------------------------
# W4A16 fp64 reference (cuda/nve_kernels.cu:330-371)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("awq", [False, True])
def test_w4a16_f64_vs_dequant(orc, awq):
    n, k = 29, 640
    data = orc.q4_from_f32(weights(n, k, seed=41))
    nib, sc = orc.extract_for_gpu(data, n, k)
    x = activations(k, seed=42).astype(np.float16).astype(F32)
    a = np.linspace(0.25, 4.0, k).astype(F32) if awq else None
    y = orc.matvec_w4a16_f64(x, nib, sc, n, k, awq=a)
    # exact dequantization in float64 from an independent CPU-order unpack
    e = _cpu_elems(data, n, k).astype(np.float64) - 8.0
    sc64 = data.reshape(n, k // 32, 20)[:, :, :4].copy().view(np.float32)[..., 0].astype(np.float64)
    w = (e * sc64[..., None]).reshape(n, k)
    xe = x.astype(np.float64) * (a.astype(np.float64) if awq else 1.0)
    assert np.allclose(y, w @ xe, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# dispatch (src/gpu_layer.rs:1013-1025)
# ---------------------------------------------------------------------------
def test_dispatch_truth_table(orc):
    assert orc.use_w4a8(0.0, False) is True
    assert orc.use_w4a8(0.69, False) is True
    assert orc.use_w4a8(0.7, False) is False   # strict <
    assert orc.use_w4a8(1.0, False) is False
    assert orc.use_w4a8(0.0, True) is False     # NVE_NO_W4A8 wins
    assert orc.use_w4a8(0.5, False, threshold=0.4) is False
    assert orc.use_w4a8(0.3, False, threshold=0.4) is True
