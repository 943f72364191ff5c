"""ctypes/numpy wrapper of liboracle.so (the C restatement in oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  Each function names the reference lines it restates (see oracle.h).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        p = C.c_void_p
        i64 = C.c_int64
        L.orc_rust_f32_as_i8.argtypes = [C.c_float]
        L.orc_rust_f32_as_i8.restype = C.c_int8
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_quantize_block_q4.argtypes = [p, p]
        L.orc_q4_from_f32.argtypes = [p, i64, i64, p]
        L.orc_quantize_block_q4_weighted.argtypes = [p, p, p]
        L.orc_q4_from_f32_awq.argtypes = [p, i64, i64, p, C.c_int, p, p]
        L.orc_q4_to_f32.argtypes = [p, i64, i64, p, p]
        L.orc_extract_for_gpu.argtypes = [p, i64, i64, p, p]
        L.orc_q4_dot_row_scalar.argtypes = [p, p, i64]
        L.orc_q4_dot_row_scalar.restype = C.c_float
        L.orc_q4_dot_row_avx2.argtypes = [p, p, i64]
        L.orc_q4_dot_row_avx2.restype = C.c_float
        L.orc_q4_matvec_f32.argtypes = [p, i64, i64, p, p, p, C.c_int, C.c_int]
        L.orc_quantize_q8_group.argtypes = [p, i64, p, p]
        L.orc_quantize_q8_rows_bf16.argtypes = [p, i64, i64, p, p]
        L.orc_w4a8_block_acc.argtypes = [p, p, i64, i64, p]
        L.orc_matvec_w4a8_f64.argtypes = [p, p, C.c_int, p, p, i64, i64, p]
        L.orc_matvec_w4a8_f32.argtypes = [p, p, p, p, i64, i64, p, C.c_int]
        L.orc_matvec_w4a16_f64.argtypes = [p, p, p, p, i64, i64, p]
        L.orc_use_w4a8.argtypes = [C.c_double, C.c_int, C.c_double]
        L.orc_use_w4a8.restype = C.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- Q4_0 format (src/quantize.rs) -------------------------------------------
def quantize_block_q4(v32) -> np.ndarray:
    """src/quantize.rs:711-731 -> 20 bytes."""
    v = _c(v32, np.float32)
    assert v.size == 32
    out = np.zeros(20, np.uint8)
    lib().orc_quantize_block_q4(_ptr(v), _ptr(out))
    return out


def q4_from_f32(w) -> np.ndarray:
    """QuantizedTensor::from_f32 (src/quantize.rs:347-375): [N,K] f32 -> bytes [N, K/32*20]."""
    w = _c(w, np.float32)
    n, k = w.shape
    assert k % 32 == 0
    out = np.zeros((n, k // 32 * 20), np.uint8)
    lib().orc_q4_from_f32(_ptr(w), n, k, _ptr(out))
    return out


def quantize_block_q4_weighted(v32, imp32) -> np.ndarray:
    """src/quantize.rs:741-793 -> 20 bytes."""
    v, imp = _c(v32, np.float32), _c(imp32, np.float32)
    assert v.size == 32 and imp.size == 32
    out = np.zeros(20, np.uint8)
    lib().orc_quantize_block_q4_weighted(_ptr(v), _ptr(imp), _ptr(out))
    return out


def q4_from_f32_awq(w, awq, kquant: bool) -> tuple[np.ndarray, np.ndarray]:
    """QuantizedTensor::from_compact_awq (kquant False, src/quantize.rs:271-306) /
    from_compact_awq_kquant (True, 308-346) on the f32 rows -> (bytes, inv_scales)."""
    w, awq = _c(w, np.float32), _c(awq, np.float32)
    n, k = w.shape
    assert k % 32 == 0 and awq.size == k
    out = np.zeros((n, k // 32 * 20), np.uint8)
    inv = np.zeros(k, np.float32)
    lib().orc_q4_from_f32_awq(_ptr(w), n, k, _ptr(awq), int(bool(kquant)), _ptr(out), _ptr(inv))
    return out, inv


def q4_to_f32(data, n, k, awq_inv=None) -> np.ndarray:
    """QuantizedTensor::to_f32_vec (src/quantize.rs:396-426)."""
    data = _c(data, np.uint8)
    out = np.zeros((n, k), np.float32)
    aw = None if awq_inv is None else _c(awq_inv, np.float32)
    lib().orc_q4_to_f32(_ptr(data), n, k, _ptr(aw), _ptr(out))
    return out


def extract_for_gpu(data, n, k):
    """QuantizedTensor::extract_for_gpu (src/quantize.rs:437-463) -> (nibbles [N,K/2], scales [N,K/32])."""
    data = _c(data, np.uint8)
    nib = np.zeros((n, k // 2), np.uint8)
    sc = np.zeros((n, k // 32), np.float32)
    lib().orc_extract_for_gpu(_ptr(data), n, k, _ptr(nib), _ptr(sc))
    return nib, sc


def q4_dot_row(row, x, avx2: bool) -> float:
    """q4_dot_row_avx2 / q4_dot_row_scalar (src/quantize.rs:853-938)."""
    row = _c(row, np.uint8)
    x = _c(x, np.float32)
    f = lib().orc_q4_dot_row_avx2 if avx2 else lib().orc_q4_dot_row_scalar
    return float(f(_ptr(row), _ptr(x), row.size // 20))


def q4_matvec_f32(data, n, k, x, awq_inv=None, threads: int = 1, avx2: bool = True) -> np.ndarray:
    """QuantizedTensor::matvec_f32 (src/quantize.rs:466-488, 1107-1111)."""
    data = _c(data, np.uint8)
    x = _c(x, np.float32)
    y = np.zeros(n, np.float32)
    aw = None if awq_inv is None else _c(awq_inv, np.float32)
    lib().orc_q4_matvec_f32(_ptr(data), n, k, _ptr(x), _ptr(aw), _ptr(y), threads, 1 if avx2 else 0)
    return y


# ---- W4A8 (cuda/nve_kernels.cu) -----------------------------------------------
def quantize_q8_group(x):
    """_nve_quantize_f16_q8 (cuda/nve_kernels.cu:712-745), rows of x independently."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    xq = np.zeros(x.shape, np.int8)
    sc = np.zeros(x.shape[:-1] + (k // 32,), np.float32)
    lib().orc_quantize_q8_group(_ptr(x), x.size, _ptr(xq), _ptr(sc))
    return xq, sc


def quantize_q8_rows_bf16(x):
    """Per-token int8 quantization with one bf16 scale per row (no reference counterpart)."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    m, k = x.shape
    xq = np.zeros((m, k), np.int8)
    sc = np.zeros(m, np.uint16)
    lib().orc_quantize_q8_rows_bf16(_ptr(x), m, k, _ptr(xq), _ptr(sc))
    return xq, sc


def w4a8_block_acc(xq, nib, n, k) -> np.ndarray:
    """Exact int32 accumulators of _nve_matvec_w4a8 (cuda/nve_kernels.cu:835-853)."""
    xq = _c(xq, np.int8)
    nib = _c(nib, np.uint8)
    acc = np.zeros((n, k // 32), np.int32)
    lib().orc_w4a8_block_acc(_ptr(xq), _ptr(nib), n, k, _ptr(acc))
    return acc


def matvec_w4a8_f64(xq, xs, nib, ws, n, k, xs_mode: int = 0) -> np.ndarray:
    xq = _c(xq, np.int8)
    xs = _c(xs, np.float32)
    nib = _c(nib, np.uint8)
    ws = _c(ws, np.float32)
    y = np.zeros(n, np.float64)
    lib().orc_matvec_w4a8_f64(_ptr(xq), _ptr(xs), xs_mode, _ptr(nib), _ptr(ws), n, k, _ptr(y))
    return y


def matvec_w4a8_f32(xq, xs, nib, ws, n, k, threads: int = 1) -> np.ndarray:
    xq = _c(xq, np.int8)
    xs = _c(xs, np.float32)
    nib = _c(nib, np.uint8)
    ws = _c(ws, np.float32)
    y = np.zeros(n, np.float32)
    lib().orc_matvec_w4a8_f32(_ptr(xq), _ptr(xs), _ptr(nib), _ptr(ws), n, k, _ptr(y), threads)
    return y


# ---- W4A16 (cuda/nve_kernels.cu:330-371) --------------------------------------
def matvec_w4a16_f64(x, nib, sc, n, k, awq=None) -> np.ndarray:
    x = _c(x, np.float32)
    nib = _c(nib, np.uint8)
    sc = _c(sc, np.float32)
    aw = None if awq is None else _c(awq, np.float32)
    y = np.zeros(n, np.float64)
    lib().orc_matvec_w4a16_f64(_ptr(x), _ptr(aw), _ptr(nib), _ptr(sc), n, k, _ptr(y))
    return y


# ---- dispatch (src/gpu_layer.rs:1013-1025) -------------------------------------
def use_w4a8(importance: float, no_w4a8_env: bool, threshold: float = 0.7) -> bool:
    return bool(lib().orc_use_w4a8(importance, 1 if no_w4a8_env else 0, threshold))


# ---- conversions -----------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    return np.array([lib().orc_f32_to_bf16(float(v)) for v in x], np.uint16)


def bf16_bits_to_f32(h) -> np.ndarray:
    h = np.asarray(h, np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)
