"""Host-side mirror of the reference's GEMV operator API (src/cuda_kernels.rs).

Same function names, argument meaning and output shapes as the Rust wrappers; torch
device tensors take the place of candle tensors, and each call goes through the C ABI
of libnve_hip.so on torch's current HIP stream.  As in the reference, the plain
wrappers allocate their outputs and the `_into` variants write into caller buffers.

Reference wrappers mirrored here (file:line in src/cuda_kernels.rs):
  quantize_f16_q8            525-540
  matvec_w4a8                552-573
  fused_matvec_w4a16         463-486
  fused_qkv_matvec_w4a16     622-662
  fused_matvec_w4a16_into    727-745
  fused_qkv_matvec_w4a16_into 748-786
Additions for the MI355X build (no reference counterpart): fp32/bf16 outputs, the
fused W4A8 Q/K/V launch, the batched W4A8 GEMV, per-token activation quantization,
device-side Q4_0 quantization/repack and the int32 accumulator debug export.
"""
from __future__ import annotations

import torch

from ._lib import (DT_BF16, DT_F16, DT_F32, XS_GROUP32_F32, XS_ROW_BF16, W4Mat, check, lib)

_DT = {torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.float32: DT_F32}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dt(t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return _DT[t.dtype]


def _dev(t: torch.Tensor, name: str) -> int:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _opt(t: torch.Tensor | None, name: str) -> int | None:
    return None if t is None else _dev(t, name)


# ---------------------------------------------------------------------------
# W4A8
# ---------------------------------------------------------------------------
def quantize_f16_q8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [K] or [1,K] (fp16, bf16 or fp32) -> (xq int8 [K], scales f32 [K/32]).

    src/cuda_kernels.rs:525-540 (asserts K % 32 == 0 like the reference).
    """
    k = x.numel()
    if k % 32 != 0:
        raise ValueError("quantize_f16_q8: K must be multiple of 32")
    xf = x.reshape(-1)
    xq = torch.empty(k, dtype=torch.int8, device=x.device)
    sc = torch.empty(k // 32, dtype=torch.float32, device=x.device)
    check("nve_hip_quantize_q8",
          lib().nve_hip_quantize_q8(_dev(xf, "x"), _dt(xf), 1, k, xq.data_ptr(), sc.data_ptr(), _stream()))
    return xq, sc


def quantize_q8_rows(x: torch.Tensor, per_token: bool = False):
    """Quantize M rows of activations [M,K].

    per_token=False: group-32 f32 scales [M, K/32] (reference scheme per row).
    per_token=True : one bf16 scale per row, returned as a bfloat16 tensor [M].
    """
    if x.dim() == 1:
        x = x[None]
    m, k = x.shape
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    if per_token:
        sc = torch.empty(m, dtype=torch.bfloat16, device=x.device)
        check("nve_hip_quantize_q8_rows",
              lib().nve_hip_quantize_q8_rows(_dev(x, "x"), _dt(x), m, k, xq.data_ptr(), sc.data_ptr(), _stream()))
    else:
        sc = torch.empty((m, k // 32), dtype=torch.float32, device=x.device)
        check("nve_hip_quantize_q8",
              lib().nve_hip_quantize_q8(_dev(x, "x"), _dt(x), m, k, xq.data_ptr(), sc.data_ptr(), _stream()))
    return xq, sc


def matvec_w4a8_into(xq, xq_scales, nibbles, wt_scales, out, n: int, k: int) -> None:
    check("nve_hip_matvec_w4a8",
          lib().nve_hip_matvec_w4a8(_dev(xq, "xq"), _dev(xq_scales, "xq_scales"), _dev(nibbles, "nibbles"),
                                    _dev(wt_scales, "wt_scales"), _dev(out, "out"), _dt(out), n, k, _stream()))


def matvec_w4a8(xq, xq_scales, nibbles, wt_scales, n: int, k: int,
                out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """xq[K] x W_int4[N,K]^T -> [1, N] (fp16 like the reference, src/cuda_kernels.rs:552-573)."""
    out = torch.empty((1, n), dtype=out_dtype, device=xq.device)
    matvec_w4a8_into(xq, xq_scales, nibbles, wt_scales, out, n, k)
    return out


def qkv_matvec_w4a8(xq, xq_scales, wq, wk, wv, out_dtype: torch.dtype = torch.float16):
    """The three W4A8 projections of one layer in one launch.  wq/wk/wv: GpuW4-like
    objects with .nibbles, .scales, .n, .k."""
    dev = xq.device
    outs = [torch.empty((1, w.n), dtype=out_dtype, device=dev) for w in (wq, wk, wv)]
    check("nve_hip_qkv_matvec_w4a8",
          lib().nve_hip_qkv_matvec_w4a8(
              _dev(xq, "xq"), _dev(xq_scales, "xq_scales"),
              _dev(wq.nibbles, "q_nib"), _dev(wq.scales, "q_sc"), wq.n,
              _dev(wk.nibbles, "k_nib"), _dev(wk.scales, "k_sc"), wk.n,
              _dev(wv.nibbles, "v_nib"), _dev(wv.scales, "v_sc"), wv.n,
              outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), _DT[out_dtype], wq.k, _stream()))
    return tuple(outs)


def matvec_w4a8_batched(xq, xq_scales, nibbles, wt_scales, n: int, k: int,
                        out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None) -> torch.Tensor:
    """xq [M,K] int8 with group scales f32 [M,K/32] or per-token bf16 [M] -> out [M,N]."""
    m = xq.shape[0]
    mode = XS_ROW_BF16 if xq_scales.dtype == torch.bfloat16 else XS_GROUP32_F32
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=xq.device)
    check("nve_hip_matvec_w4a8_batched",
          lib().nve_hip_matvec_w4a8_batched(m, _dev(xq, "xq"), _dev(xq_scales, "xq_scales"), mode,
                                            _dev(nibbles, "nibbles"), _dev(wt_scales, "wt_scales"),
                                            _dev(out, "out"), _dt(out), n, k, _stream()))
    return out


def w4a8_block_acc(xq, nibbles, n: int, k: int) -> torch.Tensor:
    """Debug: exact int32 block accumulators [N, K/32]."""
    acc = torch.empty((n, k // 32), dtype=torch.int32, device=xq.device)
    check("nve_hip_w4a8_block_acc",
          lib().nve_hip_w4a8_block_acc(_dev(xq, "xq"), _dev(nibbles, "nibbles"), acc.data_ptr(), n, k, _stream()))
    return acc


# ---------------------------------------------------------------------------
# W4A16
# ---------------------------------------------------------------------------
def fused_matvec_w4a16_into(x, nibbles, scales, awq_scales, out, n: int, k: int) -> None:
    """src/cuda_kernels.rs:727-745."""
    check("nve_hip_matvec_w4a16",
          lib().nve_hip_matvec_w4a16(_dev(x, "x"), _dt(x), _dev(nibbles, "nibbles"), _dev(scales, "scales"),
                                     _opt(awq_scales, "awq_scales"), _dev(out, "out"), _dt(out), n, k,
                                     _stream()))


def fused_matvec_w4a16(x, nibbles, scales, awq_scales, n: int, k: int,
                       out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x[1,K] (fp16/bf16) x W_int4[N,K]^T -> [1,N] (src/cuda_kernels.rs:463-486).
    The output dtype defaults to the activation dtype."""
    out = torch.empty((1, n), dtype=out_dtype or x.dtype, device=x.device)
    fused_matvec_w4a16_into(x.reshape(-1), nibbles, scales, awq_scales, out, n, k)
    return out


def fused_qkv_matvec_w4a16_into(x, q_nib, q_sc, q_awq, nq, k_nib, k_sc, k_awq, nk, v_nib, v_sc, v_awq, nv,
                                k_dim, q_out, k_out, v_out) -> None:
    """src/cuda_kernels.rs:748-786 (argument order of the reference)."""
    check("nve_hip_qkv_matvec_w4a16",
          lib().nve_hip_qkv_matvec_w4a16(
              _dev(x, "x"), _dt(x),
              _dev(q_nib, "q_nib"), _dev(q_sc, "q_sc"), _opt(q_awq, "q_awq"), nq,
              _dev(k_nib, "k_nib"), _dev(k_sc, "k_sc"), _opt(k_awq, "k_awq"), nk,
              _dev(v_nib, "v_nib"), _dev(v_sc, "v_sc"), _opt(v_awq, "v_awq"), nv,
              _dev(q_out, "q_out"), _dev(k_out, "k_out"), _dev(v_out, "v_out"), _dt(q_out), k_dim, _stream()))


def fused_qkv_matvec_w4a16(x, q_nib, q_sc, q_awq, nq, k_nib, k_sc, k_awq, nk, v_nib, v_sc, v_awq, nv, k_dim,
                           out_dtype: torch.dtype | None = None):
    """src/cuda_kernels.rs:622-662 -> ([1,Nq], [1,Nk], [1,Nv])."""
    dt = out_dtype or x.dtype
    outs = [torch.empty((1, m), dtype=dt, device=x.device) for m in (nq, nk, nv)]
    fused_qkv_matvec_w4a16_into(x.reshape(-1), q_nib, q_sc, q_awq, nq, k_nib, k_sc, k_awq, nk, v_nib, v_sc, v_awq,
                                nv, k_dim, *outs)
    return tuple(outs)


# ---------------------------------------------------------------------------
# weight preparation (once per layer upload)
# ---------------------------------------------------------------------------
def q4_quantize(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """QuantizedTensor::from_f32/from_compact + extract_for_gpu on the device:
    w [N,K] (f32/bf16/f16) -> (nibbles u8 [N,K/2] GPU order, scales f32 [N,K/32])."""
    n, k = w.shape
    nib = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    sc = torch.empty((n, k // 32), dtype=torch.float32, device=w.device)
    check("nve_hip_q4_quantize",
          lib().nve_hip_q4_quantize(_dev(w, "w"), _dt(w), n, k, nib.data_ptr(), sc.data_ptr(), _stream()))
    return nib, sc


def q4_quantize_awq(w: torch.Tensor, awq: torch.Tensor, kquant: bool = True
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """QuantizedTensor::from_compact_awq(_kquant) + extract_for_gpu on the device
    (src/quantize.rs:271-346): w [N,K] (f32/bf16/f16), awq f32 [K] ->
    (nibbles, scales, awq_inv f32 [K]); awq_inv is the GEMVs' awq argument."""
    n, k = w.shape
    if awq.dtype != torch.float32 or awq.numel() != k:
        raise ValueError("awq must be float32 [K]")
    nib = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    sc = torch.empty((n, k // 32), dtype=torch.float32, device=w.device)
    inv = torch.empty(k, dtype=torch.float32, device=w.device)
    check("nve_hip_q4_quantize_awq",
          lib().nve_hip_q4_quantize_awq(_dev(w, "w"), _dt(w), _dev(awq, "awq"), int(bool(kquant)), n, k,
                                        nib.data_ptr(), sc.data_ptr(), inv.data_ptr(), _stream()))
    return nib, sc, inv


def q4_repack(q4_blocks: torch.Tensor, n: int, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """extract_for_gpu on the device: reference CPU Q4_0 bytes [N, K/32*20] -> (nibbles, scales)."""
    nib = torch.empty((n, k // 2), dtype=torch.uint8, device=q4_blocks.device)
    sc = torch.empty((n, k // 32), dtype=torch.float32, device=q4_blocks.device)
    check("nve_hip_q4_repack",
          lib().nve_hip_q4_repack(_dev(q4_blocks, "q4_blocks"), n, k, nib.data_ptr(), sc.data_ptr(), _stream()))
    return nib, sc


def matvec_w4a8_x(x: torch.Tensor, nibbles: torch.Tensor, scales: torch.Tensor, n: int, k: int,
                  out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """quantize_f16_q8 + matvec_w4a8 (src/cuda_kernels.rs:525-573) in one launch: x [K]
    (fp16 / bf16 / fp32) is quantized inside the GEMV; bit-identical to the pair."""
    out = torch.empty(n, dtype=out_dtype, device=x.device)
    check("nve_hip_matvec_w4a8_x",
          lib().nve_hip_matvec_w4a8_x(_dev(x, "x"), _dt(x), _dev(nibbles, "nibbles"), _dev(scales, "scales"),
                                      out.data_ptr(), _dt(out), n, k, _stream()))
    return out


def grouped_matvec_w4a8_x(x: torch.Tensor, mats, k: int, out_dtype: torch.dtype = torch.float32) -> list:
    """Grouped form of matvec_w4a8_x: mats = [(nibbles, scales, n), ...] (1..3) sharing x."""
    outs = [torch.empty(n, dtype=out_dtype, device=x.device) for _, _, n in mats]
    arr = (W4Mat * len(mats))(*[W4Mat(_dev(nb, "nibbles"), _dev(sc, "scales"), None, o.data_ptr(), n)
                               for (nb, sc, n), o in zip(mats, outs)])
    check("nve_hip_grouped_matvec_w4a8_x",
          lib().nve_hip_grouped_matvec_w4a8_x(_dev(x, "x"), _dt(x), arr, len(mats), _dt(outs[0]), k, _stream()))
    return outs


def dequant_w4(nibbles: torch.Tensor, scales: torch.Tensor, n: int, k: int, awq: torch.Tensor | None = None,
               dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """nve_dequant_w4a16 (cuda/nve_kernels.cu:397-433), the prefill path's weight expansion:
    W [N, K] = (nibble - 8) * scale [* awq], in fp16 (the reference), bf16 or fp32."""
    out = torch.empty((n, k), dtype=dtype, device=nibbles.device)
    check("nve_hip_dequant_w4",
          lib().nve_hip_dequant_w4(_dev(nibbles, "nibbles"), _dev(scales, "scales"),
                                   None if awq is None else _dev(awq, "awq"), out.data_ptr(), _dt(out), n, k,
                                   _stream()))
    return out


def gemm_w4a16(x: torch.Tensor, nibbles: torch.Tensor, scales: torch.Tensor, n: int, k: int,
               awq: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Prefill x [M, K] @ W^T for int4 W: GpuWeight::matmul_x with seq > 1
    (src/gpu_layer.rs:219-237, dequant to fp16 then matmul) fused into one MFMA kernel."""
    m = x.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    check("nve_hip_gemm_w4a16",
          lib().nve_hip_gemm_w4a16(_dev(x, "x"), _dt(x), m, _dev(nibbles, "nibbles"), _dev(scales, "scales"),
                                   None if awq is None else _dev(awq, "awq"), out.data_ptr(), _dt(out), n, k,
                                   _stream()))
    return out


def gemm_w4a16_workspace_bytes(m: int, n: int, k: int) -> int:
    """Workspace that lets gemm_w4a16_ws take the dequant + hipBLASLt path (0: it will not)."""
    return int(lib().nve_hip_gemm_w4a16_workspace_bytes(m, n, k))


def gemm_w4a16_ws(x: torch.Tensor, nibbles: torch.Tensor, scales: torch.Tensor, n: int, k: int,
                  workspace: torch.Tensor | None, awq: torch.Tensor | None = None,
                  out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """gemm_w4a16 with the reference's two-step method (dequant + vendor GEMM) where it
    is faster (M > 512, given `workspace` of gemm_w4a16_workspace_bytes bytes)."""
    m = x.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    ws_ptr = None if workspace is None else _dev(workspace, "workspace")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check("nve_hip_gemm_w4a16_ws",
          lib().nve_hip_gemm_w4a16_ws(_dev(x, "x"), _dt(x), m, _dev(nibbles, "nibbles"), _dev(scales, "scales"),
                                      None if awq is None else _dev(awq, "awq"), out.data_ptr(), _dt(out), n, k,
                                      ws_ptr, ws_bytes, _stream()))
    return out


def stream_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """HBM streaming probe (reads every byte of buf once)."""
    check("nve_hip_stream_read",
          lib().nve_hip_stream_read(_dev(buf, "buf"), buf.numel() * buf.element_size(), _dev(sink, "sink"),
                                    _stream()))
