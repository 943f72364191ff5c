"""CPU restatement of one decode step (TEST INFRASTRUCTURE ONLY).

Two uses:
  * `emulate_step` -- the checker for nve_amd.decode: the same layer math as the HIP
    path (W4A8 layers quantize their activations with the group-32 quantizer,
    W4A16 layers see fp16 activations as the reference's decode path does, whose W4A16
    kernel takes fp16 x, src/cuda_kernels.rs:117-126; bf16 KV cache; fp32 residual), evaluated with
    float64 dot products on the oracle's restated kernels.
  * `reference_step` -- the reference's CPU decode path for the bench's CPU baseline:
    every projection through QuantizedTensor::matvec_f32 (src/quantize.rs:466-488,
    q4_dot_row_avx2 restated in oracle.c, row-parallel over the host cores) with f32
    activations, as PagedModel::forward_single's CPU branch does
    (src/paged_model.rs:1352-1434).

Both follow src/ops.rs (rms_norm 12-30 in f64; RoPE half-split pairs 264-276; silu
62-64; softmax 152-163; argmax 485-495) and src/attention.rs:149-228 (GQA,
scale 1/sqrt(head_dim)).
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc

F32 = np.float32


def bf16_round(x) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def f16_round(x) -> np.ndarray:
    """f32 -> fp16 -> f32: round to nearest even, fp16 subnormals kept, overflow to inf
    (what the W4A16 staging's v_cvt_f16_f32 does)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """src/ops.rs:12-30: f64 sum of squares and scaling, rounded to f32."""
    xd = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.sum(xd * xd) / x.size + eps)
    return (xd * inv * w.astype(np.float64)).astype(F32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, pos: int, nheads: int, d: int) -> np.ndarray:
    """RopeFreqs::apply_q per head (src/ops.rs:264-276), f32 arithmetic."""
    half = d // 2
    y = x.reshape(nheads, d).astype(F32).copy()
    c, s = cos[pos].astype(F32), sin[pos].astype(F32)
    x0, x1 = y[:, :half].copy(), y[:, half:].copy()
    y[:, :half] = x0 * c - x1 * s
    y[:, half:] = x0 * s + x1 * c
    return y.reshape(-1)


def silu(x: np.ndarray) -> np.ndarray:
    x = x.astype(F32)
    return x / (F32(1.0) + np.exp(-x))


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, length: int, heads: int, kv_heads: int,
              d: int) -> np.ndarray:
    """gqa_forward_single's score / softmax / value sum (src/attention.rs:186-220) over
    keys 0..length-1, in float64."""
    g = heads // kv_heads
    out = np.zeros((heads, d), np.float64)
    qh = q.reshape(heads, d).astype(np.float64)
    scale = 1.0 / np.sqrt(np.float32(d))
    for h in range(heads):
        kv = h // g
        k = kc[kv, :length].astype(np.float64)
        v = vc[kv, :length].astype(np.float64)
        s = k @ qh[h] * float(scale)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v
    return out.reshape(-1)


def gpu_to_cpu_blocks(nib: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """Inverse of extract_for_gpu (src/quantize.rs:437-463): GPU nibble order + scales ->
    the CPU Q4_0 blocks [f32 scale][16 B, byte i = e_2i | e_2i+1 << 4]."""
    n, kb = sc.shape
    g = nib.reshape(n, kb, 16)
    e = np.concatenate([g & 15, g >> 4], axis=2)  # elements 0..31
    cpu = (e[:, :, 0::2] | (e[:, :, 1::2] << 4)).astype(np.uint8)
    out = np.empty((n, kb, 20), np.uint8)
    out[:, :, :4] = np.ascontiguousarray(sc, np.float32).view(np.uint8).reshape(n, kb, 4)
    out[:, :, 4:] = cpu
    return out.reshape(n, kb * 20)


class HostModel:
    """Host copy of a nve_amd.decode.DecodeModel (weights, norms, caches, tables)."""

    def __init__(self, m, with_cpu_blocks: bool = False):
        s = m.shape
        self.shape = s
        self.max_seq = m.max_seq
        self.prefill = m.prefill
        self.use_w4a8 = list(m.use_w4a8)
        self.lm_head_w4a8 = m.lm_head_w4a8

        def w(t):
            nib, sc = t[0].cpu().numpy(), t[1].cpu().numpy()
            return (nib, sc, gpu_to_cpu_blocks(nib, sc) if with_cpu_blocks else None)

        def b(t):
            return bf16_to_f32(t.view(dtype=__import__("torch").int16).cpu().numpy().view(np.uint16))

        self.layers = []
        for lw in m.layers:
            self.layers.append({
                "input_norm": b(lw["input_norm"]), "post_attn_norm": b(lw["post_attn_norm"]),
                **{nm: w(lw[nm]) for nm in ("q", "k", "v", "o", "gate", "up", "down")},
                "k_cache": b(lw["k_cache"]).reshape(lw["k_cache"].shape),
                "v_cache": b(lw["v_cache"]).reshape(lw["v_cache"].shape),
            })
        self.final_norm = b(m.final_norm)
        self.lm_head = w(m.lm_head)
        self.embed = b(m.embed).reshape(m.embed.shape)
        self.cos = m.rope_cos.cpu().numpy()
        self.sin = m.rope_sin.cpu().numpy()


def _gemv_emulated(x: np.ndarray, wt, w4a8: bool) -> np.ndarray:
    nib, sc, _ = wt
    n, k = nib.shape[0], nib.shape[1] * 2
    if w4a8:
        q, s = orc.quantize_q8_group(x.astype(F32))
        return orc.matvec_w4a8_f64(q, s, nib, sc, n, k).astype(F32)
    return orc.matvec_w4a16_f64(f16_round(x), nib, sc, n, k).astype(F32)


def emulate_layer(hm: HostModel, li: int, h: np.ndarray, pos: int) -> np.ndarray:
    """One layer (gpu_layer_forward_decode, src/gpu_layer.rs:1005-1084) with the HIP
    path's precisions; appends the layer's bf16 K/V row at pos to the host caches."""
    s = hm.shape
    d = s.head_dim
    lw = hm.layers[li]
    w8 = bool(hm.use_w4a8[li])
    h = h.astype(F32).copy()
    x = rms_norm(h, lw["input_norm"], s.eps)
    q = _gemv_emulated(x, lw["q"], w8)
    k = _gemv_emulated(x, lw["k"], w8)
    v = _gemv_emulated(x, lw["v"], w8)
    q = rope(q, hm.cos, hm.sin, pos, s.heads, d)
    k = rope(k, hm.cos, hm.sin, pos, s.kv_heads, d)
    lw["k_cache"][:, pos] = bf16_round(k).reshape(s.kv_heads, d)
    lw["v_cache"][:, pos] = bf16_round(v).reshape(s.kv_heads, d)
    a = attention(q, lw["k_cache"], lw["v_cache"], pos + 1, s.heads, s.kv_heads, d).astype(F32)
    h = (h + _gemv_emulated(a, lw["o"], w8)).astype(F32)
    x2 = rms_norm(h, lw["post_attn_norm"], s.eps)
    gt = _gemv_emulated(x2, lw["gate"], w8)
    up = _gemv_emulated(x2, lw["up"], w8)
    mid = f16_round(silu(gt) * up)  # held in fp16 (src/gpu_layer.rs:937-946)
    return (h + _gemv_emulated(mid, lw["down"], w8)).astype(F32)


def emulate_head(hm: HostModel, h: np.ndarray):
    """Final norm, lm_head, greedy argmax (first maximum, src/ops.rs:485-495)."""
    xf = rms_norm(h, hm.final_norm, hm.shape.eps)
    logits = _gemv_emulated(xf, hm.lm_head, bool(hm.lm_head_w4a8))
    return logits, int(np.argmax(logits))


def emulate_step(hm: HostModel, hidden: np.ndarray, pos: int):
    """One token through every layer and the head with the HIP path's precisions.
    Mutates the host KV caches; returns (next hidden, logits, token)."""
    h = hidden.astype(F32)
    for li in range(len(hm.layers)):
        h = emulate_layer(hm, li, h, pos)
    logits, tok = emulate_head(hm, h)
    return hm.embed[tok].astype(F32), logits, tok


def reference_step(hm: HostModel, hidden: np.ndarray, pos: int, threads: int):
    """The reference CPU decode path: Q4 x f32 matvec_f32 for every projection (AVX2
    restated, row-parallel), f32 activations, f32 KV values.  Returns
    (next hidden, token)."""
    s = hm.shape
    d = s.head_dim

    def mv(x, wt):
        nib, _, blocks = wt
        n, k = nib.shape[0], nib.shape[1] * 2
        return orc.q4_matvec_f32(blocks, n, k, x, threads=threads)

    h = hidden.astype(F32).copy()
    for lw in hm.layers:
        x = rms_norm(h, lw["input_norm"], s.eps)
        q = rope(mv(x, lw["q"]), hm.cos, hm.sin, pos, s.heads, d)
        k = rope(mv(x, lw["k"]), hm.cos, hm.sin, pos, s.kv_heads, d)
        v = mv(x, lw["v"])
        lw["k_cache"][:, pos] = k.reshape(s.kv_heads, d)
        lw["v_cache"][:, pos] = v.reshape(s.kv_heads, d)
        a = attention(q, lw["k_cache"], lw["v_cache"], pos + 1, s.heads, s.kv_heads, d).astype(F32)
        h = h + mv(a, lw["o"])
        x2 = rms_norm(h, lw["post_attn_norm"], s.eps)
        mid = silu(mv(x2, lw["gate"])) * mv(x2, lw["up"])
        h = h + mv(mid.astype(F32), lw["down"])
    logits = mv(rms_norm(h, hm.final_norm, s.eps), hm.lm_head)
    tok = int(np.argmax(logits))
    return hm.embed[tok].astype(F32), tok
