"""Pins of the AWQ / k-quant Q4 quantizers of the oracle (src/quantize.rs:271-346,
741-793): hand-derived known answers, reductions to the plain quantizer, exact
power-of-two scaling, a float64 brute force over the 8 candidates, and the
reference's own AWQ unit test (src/quantize.rs:2520-2544)."""
from __future__ import annotations

import struct

import numpy as np

from helpers import weights

F32 = np.float32


def _scale(out) -> float:
    return struct.unpack("<f", bytes(out[:4]))[0]


def _nibbles(out) -> list[int]:
    """CPU order: byte i = e_2i | e_2i+1 << 4."""
    return [int(out[4 + i // 2]) >> (4 * (i & 1)) & 15 for i in range(32)]


def test_weighted_kat_zero_importance_outlier(orc):
    # v = [7, 3.5 x 31], importance 0 on the outlier: candidate 0 (scale 1) leaves
    # 3.5 -> 4 (error 31 * 0.25); candidate 1 (scale 0.5) is exact on the 31 values.
    v = np.full(32, 3.5, F32)
    v[0] = 7.0
    imp = np.ones(32, F32)
    imp[0] = 0.0
    out = orc.quantize_block_q4_weighted(v, imp)
    assert _scale(out) == 0.5
    assert _nibbles(out) == [15] * 32  # 7 * 2 = 14 clamps to 7; 3.5 * 2 = 7


def test_weighted_kat_uniform_importance(orc):
    # same block, unit importance: candidate 0 costs 7.75, candidates 1-7 cost 12.25
    v = np.full(32, 3.5, F32)
    v[0] = 7.0
    out = orc.quantize_block_q4_weighted(v, np.ones(32, F32))
    assert _scale(out) == 1.0
    assert _nibbles(out) == [15] + [12] * 31  # round(3.5) = 4 (half away from zero)


def test_weighted_kat_first_minimum_wins(orc):
    # two non-zero values, both with importance 0: every candidate has error 0, so
    # the first (largest amax, scale 1) is kept; the loop stops at the zero candidate.
    v = np.zeros(32, F32)
    v[3], v[9] = 7.0, -3.5
    out = orc.quantize_block_q4_weighted(v, np.zeros(32, F32))
    assert _scale(out) == 1.0
    nib = _nibbles(out)
    assert nib[3] == 15 and nib[9] == 4 and all(n == 8 for i, n in enumerate(nib) if i not in (3, 9))


def test_weighted_kat_tiny_block(orc):
    # every |v| < 1e-10: no candidate, scale 0, all nibbles 8 (the plain quantizer
    # would use amax / 7 > 0 here)
    v = np.full(32, 5e-11, F32)
    v[::2] *= -1
    out = orc.quantize_block_q4_weighted(v, np.ones(32, F32))
    assert _scale(out) == 0.0 and _nibbles(out) == [8] * 32
    assert _scale(orc.quantize_block_q4(v)) > 0.0


def test_weighted_single_nonzero_equals_plain(orc):
    rng = np.random.default_rng(3)
    for _ in range(20):
        v = np.zeros(32, F32)
        v[rng.integers(32)] = F32(rng.normal() * 10)
        imp = rng.random(32).astype(F32) + F32(0.1)
        assert np.array_equal(orc.quantize_block_q4_weighted(v, imp), orc.quantize_block_q4(v))


def _round_away(x):
    return np.where(x >= 0, np.floor(x + 0.5), -np.floor(-x + 0.5))


def test_weighted_brute_force_f64(orc):
    """The chosen scale is one of the 8 largest |v| / 7 and its importance-weighted
    error, evaluated in float64, is the least over those candidates up to the f32
    rounding of the reference's own error sum."""
    rng = np.random.default_rng(7)
    for t in range(300):
        v = (rng.standard_normal(32) * (0.02 if t % 2 else 1.0)).astype(F32)
        if t % 5 == 0:
            v[rng.integers(32)] *= F32(20.0)  # an outlier
        imp = (rng.random(32) ** 2).astype(F32)
        out = orc.quantize_block_q4_weighted(v, imp)
        s = _scale(out)
        cands = np.sort(np.abs(v).astype(np.float64))[::-1][:8]
        cands = cands[cands >= 1e-10]
        errs = []
        for a in cands:
            cs = F32(F32(a) / F32(7.0))
            ci = F32(F32(1.0) / cs)
            q = np.clip(_round_away((v * ci).astype(np.float64)), -8, 7)
            errs.append(float(np.sum(imp.astype(np.float64) * (v.astype(np.float64) - q * float(cs)) ** 2)))
        scales = [float(F32(F32(a) / F32(7.0))) for a in cands]
        assert s in scales, (t, s, scales)
        e = errs[scales.index(s)]
        assert e <= min(errs) * (1 + 1e-4) + 1e-12, (t, e, min(errs))
        # the nibbles are the plain rounding at the chosen scale
        inv = F32(1.0) / F32(s)
        q = np.clip(_round_away((v * inv).astype(np.float64)), -8, 7).astype(int) + 8
        assert _nibbles(out) == list(q)


def test_awq_unit_scales_reduce_to_plain(orc):
    w = weights(8, 128, seed=5)
    ones = np.ones(128, F32)
    data0, inv = orc.q4_from_f32_awq(w, ones, kquant=False)
    assert np.array_equal(data0, orc.q4_from_f32(w))
    assert np.array_equal(inv, ones)
    data1, _ = orc.q4_from_f32_awq(w, ones, kquant=True)
    blocks = w.reshape(-1, 32)
    ref = np.stack([orc.quantize_block_q4_weighted(b, ones[:32]) for b in blocks]).reshape(8, -1)
    assert np.array_equal(data1, ref)


def test_awq_power_of_two_commutes(orc):
    """A uniform awq = 2^e scales every value, candidate and error exactly: the same
    nibbles, scales multiplied by 2^e."""
    w = weights(6, 96, seed=9)
    base0, _ = orc.q4_from_f32_awq(w, np.ones(96, F32), kquant=False)
    base1, _ = orc.q4_from_f32_awq(w, np.ones(96, F32), kquant=True)
    for e in (-3, 1, 4):
        a = np.full(96, 2.0 ** e, F32)
        for kq, base in ((False, base0), (True, base1)):
            d, inv = orc.q4_from_f32_awq(w, a, kquant=kq)
            d, b = d.reshape(-1, 20), base.reshape(-1, 20)
            assert np.array_equal(d[:, 4:], b[:, 4:])
            assert np.array_equal(d[:, :4].copy().view(F32)[:, 0], b[:, :4].copy().view(F32)[:, 0] * F32(2.0 ** e))
            assert np.all(inv == F32(2.0 ** -e))


def test_awq_inverse_scales_closed_form(orc):
    a = np.zeros(32, F32)
    a[:6] = [2.0, -4.0, 1e-11, 0.0, -1e-10, 1e-9]
    a[6:] = 1.0
    _, inv = orc.q4_from_f32_awq(np.ones((1, 32), F32), a, kquant=False)
    assert inv[0] == 0.5 and inv[1] == -0.25 and inv[2] == 0.0 and inv[3] == 0.0
    assert inv[4] == 0.0  # |s| > 1e-10 is strict
    assert inv[5] == F32(1.0) / F32(1e-9)


def test_reference_unit_test_awq_scaling(orc):
    # src/quantize.rs:2520-2544: rows (i-16)*0.3 and (i-16)*0.1; the AWQ copy is
    # quantized from the bf16-rounded values with uniform awq 1.5; matvec with x = 1
    # (AWQ: x * inv_scales) within 5.0 of the plain quantization.
    vals = np.concatenate([(np.arange(32, dtype=F32) - 16) * F32(0.3),
                           (np.arange(32, dtype=F32) - 16) * F32(0.1)]).reshape(2, 32).astype(F32)
    x = np.ones(32, F32)
    y0 = orc.q4_matvec_f32(orc.q4_from_f32(vals), 2, 32, x)
    vb = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(vals)).astype(F32).reshape(2, 32)
    for kq in (False, True):
        data, inv = orc.q4_from_f32_awq(vb, np.full(32, 1.5, F32), kquant=kq)
        y1 = orc.q4_matvec_f32(data, 2, 32, x, awq_inv=inv)
        assert np.all(np.abs(y0 - y1) < 5.0)
        # tighter: both are within one quantization step sum of the exact row sums
        assert np.all(np.abs(y1 - vals.sum(axis=1)) < 0.3 * 32)
