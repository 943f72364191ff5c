"""Shared input generators and error metrics for the tests (seeded numpy PCG64)."""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def weights(n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    return (rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)


def activations(k: int, seed: int, outlier_frac: float = 0.005, outlier_sigma: float = 20.0, m: int | None = None):
    """x ~ N(0,1) with a seeded 0.5% of channels (at least one) set to +-20 sigma."""
    g = rng(seed)
    shape = (k,) if m is None else (m, k)
    x = g.standard_normal(shape, dtype=np.float32)
    n_out = max(1, int(round(outlier_frac * k))) if outlier_frac > 0 else 0
    if n_out:
        idx = g.choice(k, size=n_out, replace=False)
        sign = np.where(g.random(n_out) < 0.5, -1.0, 1.0).astype(np.float32)
        x[..., idx] = sign * np.float32(outlier_sigma)
    return x.astype(np.float32)


def to_f16(x: np.ndarray) -> np.ndarray:
    """Round to fp16 and back (the activation dtype of the reference)."""
    return x.astype(np.float16).astype(np.float32)


def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 and back to f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def rel_err_floor(y, ref) -> float:
    """max_i |y_i - ref_i| / max(|ref_i|, 1e-3 * rms(ref))  (strict, elementwise)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    den = np.maximum(np.abs(ref), 1e-3 * rms)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(np.abs(y - ref) / den)) if ref.size else 0.0


def rel_err_norm(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = float(np.linalg.norm(ref))
    return float(np.linalg.norm(y - ref)) / (d if d else 1.0)
