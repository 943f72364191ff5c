"""CPU pins of the decode-step restatement (oracle/decode_ref.py) and of the host-side
tables the decode path builds (RoPE tables, precision mask)."""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import rng, weights


@pytest.fixture(scope="module")
def dr(orc):
    from oracle import decode_ref
    return decode_ref


def test_gpu_to_cpu_blocks_inverts_extract_for_gpu(orc, dr):
    n, k = 7, 96
    data = orc.q4_from_f32(weights(n, k, seed=3))
    nib, sc = orc.extract_for_gpu(data, n, k)
    back = dr.gpu_to_cpu_blocks(nib, sc)
    assert np.array_equal(back, data)


def test_rms_norm_closed_form(dr):
    # constant vector c: mean(x^2) = c^2, y = w * c / sqrt(c^2 + eps)
    x = np.full(64, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = dr.rms_norm(x, w, 1e-5)
    exp = (w.astype(np.float64) * 3.0 / math.sqrt(9.0 + 1e-5)).astype(np.float32)
    assert np.array_equal(y, exp)
    # scale invariance (eps -> 0)
    v = rng(1).standard_normal(256).astype(np.float32)
    assert np.allclose(dr.rms_norm(v, w.repeat(4), 0.0), dr.rms_norm(v * 8, w.repeat(4), 0.0), rtol=1e-6)


def test_rope_matches_complex_rotation(dr):
    from nve_amd.decode import rope_tables
    d, heads = 64, 3
    cos, sin = rope_tables(d, 16, 10000.0)
    x = rng(2).standard_normal(heads * d).astype(np.float32)
    pos = 11
    y = dr.rope(x, cos, sin, pos, heads, d).reshape(heads, d)
    xr = x.reshape(heads, d).astype(np.float64)
    z = (xr[:, :d // 2] + 1j * xr[:, d // 2:]) * np.exp(1j * pos / 10000.0 ** (2.0 * np.arange(d // 2) / d))
    assert np.allclose(y[:, :d // 2], z.real, atol=1e-5)
    assert np.allclose(y[:, d // 2:], z.imag, atol=1e-5)
    # norm preserved per pair, position 0 is the identity
    assert np.array_equal(dr.rope(x, cos, sin, 0, heads, d), x)


def test_rope_tables_llama3_scaling_bands():
    from nve_amd.decode import RopeScaling, rope_tables
    d, theta = 128, 500000.0
    sc = RopeScaling()
    c0, s0 = rope_tables(d, 2, theta)
    c1, s1 = rope_tables(d, 2, theta, sc)
    inv = 1.0 / theta ** (2.0 * np.arange(d // 2) / d)
    ang0 = np.arctan2(s0[1].astype(np.float64), c0[1])
    ang1 = np.arctan2(s1[1].astype(np.float64), c1[1])
    wl = 2 * np.pi / inv
    high = wl < sc.original_max_position_embeddings / sc.high_freq_factor  # unscaled band
    low = wl > sc.original_max_position_embeddings / sc.low_freq_factor   # divided by factor
    assert high.any() and low.any()
    assert np.allclose(ang1[high], ang0[high], atol=1e-6)
    assert np.allclose(ang1[low], inv[low] / sc.factor, rtol=1e-5, atol=1e-9)
    mid = ~high & ~low
    assert np.all(ang1[mid] < inv[mid]) and np.all(ang1[mid] > inv[mid] / sc.factor)


def test_attention_matches_bruteforce(dr):
    heads, kv, d, L = 6, 2, 64, 37
    g = rng(5)
    q = g.standard_normal(heads * d).astype(np.float32)
    kc = g.standard_normal((kv, 50, d)).astype(np.float32)
    vc = g.standard_normal((kv, 50, d)).astype(np.float32)
    out = dr.attention(q, kc, vc, L, heads, kv, d).reshape(heads, d)
    for h in range(heads):
        j = h // (heads // kv)
        s = [float(np.dot(q[h * d:(h + 1) * d].astype(np.float64), kc[j, t])) / math.sqrt(d) for t in range(L)]
        e = np.exp(np.array(s) - max(s))
        ref = (e / e.sum()) @ vc[j, :L].astype(np.float64)
        assert np.allclose(out[h], ref, atol=1e-9)
    # a single key: the output is that key's value
    one = dr.attention(q, kc, vc, 1, heads, kv, d).reshape(heads, d)
    assert np.allclose(one[0], vc[0, 0])


def test_silu_known_values(dr):
    x = np.array([0.0, 1.0, -1.0, 20.0], np.float32)
    assert np.allclose(dr.silu(x), [0.0, 1 / (1 + math.exp(-1)), -1 / (1 + math.e), 20.0], rtol=1e-6)


def test_activation_roundings_known_answers(dr):
    """bf16 (KV cache, W4A8 staging inputs) and fp16 (W4A16 activations) rounding: ties
    to even, the last finite values, overflow and fp16 subnormals, by value."""
    bmax = (2 - 2.0 ** -7) * 2.0 ** 127  # largest finite bf16
    b = dr.bf16_round(np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 1 + 2.0 ** -9, -2.5, bmax, 0.0], np.float32))
    assert b.tolist() == [1.0, 1 + 2.0 ** -6, 1.0, -2.5, bmax, 0.0]
    h = dr.f16_round(np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 65504.0, 65520.0, -65520.0, 2.0 ** -24,
                               2.0 ** -25, 3 * 2.0 ** -26, 0.1], np.float32))
    assert h[:3].tolist() == [1.0, 1 + 2.0 ** -9, 65504.0]
    assert h[3] == np.inf and h[4] == -np.inf
    assert h[5:8].tolist() == [2.0 ** -24, 0.0, 2.0 ** -24]
    assert h[8] == np.float32(0.0999755859375)  # 0x2E66


def test_precision_mask_counts_and_seed():
    from nve_amd.decode import precision_mask
    m = precision_mask(28, 0.3, 7)
    assert m.sum() == 8 and set(np.unique(m)) <= {0.0, 1.0}
    assert np.array_equal(m, precision_mask(28, 0.3, 7))
    assert precision_mask(28, 0.0, 7).sum() == 0
