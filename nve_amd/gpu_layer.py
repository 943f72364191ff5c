"""Per-layer precision dispatch and the packed-W4 device weight (src/gpu_layer.rs).

GpuW4        -- src/gpu_layer.rs:199-205 (nibbles U8 [N,K/2], scales F32 [N,K/32],
                optional AWQ F32 [K], n, k)
ws_to_gpu    -- src/gpu_layer.rs:57-77 (Q4_0 upload: extract_for_gpu + H2D); here the
                CPU Q4_0 bytes are uploaded and repacked on the device, or an f32/bf16
                matrix is quantized on the device (quantize-on-load).
use_w4a8     -- src/gpu_layer.rs:1013-1025, evaluated by the C ABI (nve_use_w4a8) so
                the environment rules are the library's, not a Python copy.
project      -- the W4A8 / W4A16 branch of one projection (src/gpu_layer.rs:650-687,
                736-743, 936-976).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import hip_kernels as hk
from ._lib import lib


@dataclass
class GpuW4:
    nibbles: torch.Tensor  # u8 [N, K/2], GPU nibble order
    scales: torch.Tensor   # f32 [N, K/32]
    awq_scales: torch.Tensor | None
    n: int
    k: int

    @staticmethod
    def from_q4_bytes(q4: torch.Tensor, n: int, k: int, awq: torch.Tensor | None = None) -> "GpuW4":
        """Upload of a reference QuantizedTensor (CPU Q4_0 bytes, src/gpu_layer.rs:57-77)."""
        nib, sc = hk.q4_repack(q4, n, k)
        return GpuW4(nib, sc, awq, n, k)

    @staticmethod
    def quantize(w: torch.Tensor, awq: torch.Tensor | None = None, kquant: bool = True) -> "GpuW4":
        """Quantize-on-load of a device matrix [N,K]: QuantizedTensor::from_f32 /
        from_compact semantics, or with per-channel AWQ scales awq f32 [K]
        from_compact_awq_kquant (kquant, the reference's Q4 AWQ load path,
        src/generic_model.rs:172) / from_compact_awq; the inverse scales become the
        W4A16 GEMV's awq argument.  As in the reference (src/gpu_layer.rs:656-661),
        the W4A8 kernels ignore AWQ scales: run AWQ weights on W4A16."""
        n, k = w.shape
        if awq is None:
            nib, sc = hk.q4_quantize(w.contiguous())
            return GpuW4(nib, sc, None, n, k)
        nib, sc, inv = hk.q4_quantize_awq(w.contiguous(), awq.contiguous(), kquant=kquant)
        return GpuW4(nib, sc, inv, n, k)

    @property
    def nbytes(self) -> int:
        return self.nibbles.numel() + self.scales.numel() * 4


def use_w4a8(layer_importance: float) -> bool:
    """W4A8 when NVE_NO_W4A8 is unset and importance < NVE_W4A8_THRESHOLD (0.7)."""
    return bool(lib().nve_use_w4a8(float(layer_importance)))


def project(x: torch.Tensor, w: GpuW4, use_w4a8_: bool, xq=None, out_dtype=torch.float16):
    """One decode projection x[1,K] -> [1,N] on the layer's precision.

    For W4A8 the caller may pass an already-quantized (xq, xs) pair to share it
    between projections, as src/gpu_layer.rs:658-661 does for Q/K/V."""
    if use_w4a8_:
        if xq is None:
            xq = hk.quantize_f16_q8(x)
        return hk.matvec_w4a8(xq[0], xq[1], w.nibbles, w.scales, w.n, w.k, out_dtype=out_dtype)
    return hk.fused_matvec_w4a16(x, w.nibbles, w.scales, w.awq_scales, w.n, w.k, out_dtype=out_dtype)
