"""File-level weight loading into the packed W4 device layout.

Quantize-on-load from a safetensors checkpoint, as the reference's paged model does it
(src/paged_model.rs:1003-1016: "loads bf16, quantizes, drops bf16"; the quantized set
is GenericBlockWeights::quantize_q4, src/generic_model.rs:69-85): the seven projections
of every decoder block (q/k/v/o/gate/up/down) become Q4_0 (QuantizedTensor::from_compact,
src/quantize.rs:242-268) in the GPU layout (extract_for_gpu, 437-463), quantized on the
device; every other tensor (embeddings, norms, biases, lm_head) is uploaded as stored.
Tensors are read one at a time, so host memory holds at most one of them.

Q4_0 block files: the reference's QuantizedTensor.data byte layout (row-major blocks of
20 bytes: f32 little-endian scale, then 16 bytes with byte i = q[2i] | q[2i+1] << 4,
src/quantize.rs:711-731), memory-mapped and repacked on the device (nve_hip_q4_repack).
"""
from __future__ import annotations

import os
from typing import Callable, Iterable

import numpy as np
import torch

from .gpu_layer import GpuW4

PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
Q4_BLOCK_BYTES = 20


def is_block_projection(name: str) -> bool:
    """True for '<...>.<proj>.weight' with <proj> one of the seven block projections
    (the tensors GenericBlockWeights::quantize_q4 converts)."""
    parts = name.split(".")
    return len(parts) >= 2 and parts[-1] == "weight" and parts[-2] in PROJECTIONS


def quantizable(name: str, shape: Iterable[int]) -> bool:
    """A block projection whose rows are whole Q4 blocks (from_compact / from_f32
    assert K % 32 == 0, src/quantize.rs:245, 349)."""
    shape = tuple(shape)
    return is_block_projection(name) and len(shape) == 2 and shape[1] % 32 == 0


def load_safetensors_w4(paths: str | Iterable[str], device: str = "cuda",
                        awq: Callable[[str], torch.Tensor | None] | None = None,
                        kquant: bool = True) -> dict[str, GpuW4 | torch.Tensor]:
    """Read one or more .safetensors files; block projections -> GpuW4 (quantized on
    `device`), everything else -> a device tensor of the stored dtype.

    awq: optional callable name -> f32 [K] per-input-channel scales (or None) for the
    AWQ quantize-on-load path (from_compact_awq_kquant with kquant, the reference's Q4
    AWQ load, src/generic_model.rs:172; from_compact_awq without)."""
    from safetensors import safe_open

    if isinstance(paths, (str, os.PathLike)):
        paths = [paths]
    out: dict[str, GpuW4 | torch.Tensor] = {}
    for path in paths:
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for name in f.keys():
                t = f.get_tensor(name)
                if quantizable(name, t.shape):
                    w = t.to(device)
                    if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                        w = w.float()
                    a = awq(name) if awq is not None else None
                    out[name] = GpuW4.quantize(w, awq=None if a is None else a.to(device, torch.float32),
                                               kquant=kquant)
                    del w
                else:
                    out[name] = t.to(device)
                del t
    return out


def q4_block_bytes(n: int, k: int) -> int:
    if k % 32:
        raise ValueError(f"K = {k} is not a multiple of 32")
    return n * (k // 32) * Q4_BLOCK_BYTES


def read_q4_blocks(path: str, n: int, k: int, offset: int = 0) -> np.ndarray:
    """Memory-map the Q4_0 bytes of an [n, k] matrix at `offset` of `path` (u8 [n, k/32*20])."""
    size = q4_block_bytes(n, k)
    if os.path.getsize(path) < offset + size:
        raise ValueError(f"{path}: {os.path.getsize(path)} bytes, need {offset + size} for [{n}, {k}] at {offset}")
    return np.memmap(path, dtype=np.uint8, mode="r", offset=offset, shape=(n, size // n))


def write_q4_blocks(path: str, q4: np.ndarray, append: bool = False) -> int:
    """Write Q4_0 block bytes (u8, n * k/32 * 20); returns the offset they start at."""
    q4 = np.ascontiguousarray(q4, dtype=np.uint8)
    with open(path, "ab" if append else "wb") as f:
        off = f.tell()
        f.write(q4.tobytes())
    return off


def load_q4_file(path: str, n: int, k: int, offset: int = 0, device: str = "cuda",
                 awq_inv: torch.Tensor | None = None) -> GpuW4:
    """Q4_0 block bytes from a file -> GpuW4 (upload + device repack; the ws_to_gpu path,
    src/gpu_layer.rs:57-77).  awq_inv: the matrix's AWQ inverse scales f32 [K], if any."""
    blocks = read_q4_blocks(path, n, k, offset)
    q4 = torch.from_numpy(np.array(blocks)).to(device)
    return GpuW4.from_q4_bytes(q4, n, k, awq=awq_inv)
