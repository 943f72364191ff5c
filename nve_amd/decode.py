"""Synthetic Llama-style decoder on the W4A8 / W4A16 decode path.

The host side of one decode step (the reference's gpu_layer_forward_decode,
src/gpu_layer.rs:1005-1084, driven per layer from PagedModel::forward_single,
src/paged_model.rs:1307-1341): per layer, the precision comes from the dispatch rule
(nve_use_w4a8 on the layer's importance) and the layer runs through the native entry
point nve_hip_layer_forward_decode; the head (final norm, lm_head, greedy argmax,
next-token embedding, position advance) through nve_hip_decode_head.  The token
position is device-resident, so one step is captured as a HIP graph and replayed per
token.

Weights are random-init N(0, 0.02) and int4 group-quantized on the device; a seeded
mask routes a fraction of the layers to W4A16 (importance 1.0) and the rest to W4A8
(importance 0.0); the KV cache is prefilled with N(0,1) bf16 values.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import hip_kernels as hk
from ._lib import (DecodeConfig, DecodeHead, DecodeIO, LayerWeights, W4Weight, check, lib)


@dataclass
class RopeScaling:
    """Llama-3 frequency scaling (src/config.rs RopeScalingConfig, rope_type "llama3")."""
    factor: float = 32.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192


@dataclass
class ModelShape:
    hidden: int = 3072
    layers: int = 28
    heads: int = 24
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 8192
    vocab: int = 128256
    eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: RopeScaling | None = None


LLAMA_3_2_3B = ModelShape()  # config 5 names theta 500000 and no frequency scaling


def rope_tables(head_dim: int, max_seq: int, theta: float, scaling: RopeScaling | None = None):
    """RopeFreqs::new (src/ops.rs:174-226): inv_freq in f64 (llama3 scaling applied per
    frequency by wavelength band), angle = pos * inv_freq in f64, cos/sin rounded to
    f32.  Returns (cos, sin), each [max_seq, D/2]."""
    half = head_dim // 2
    inv = 1.0 / np.power(theta, 2.0 * np.arange(half, dtype=np.float64) / head_dim)
    if scaling is not None:
        old = float(scaling.original_max_position_embeddings)
        lo, hi, f = scaling.low_freq_factor, scaling.high_freq_factor, scaling.factor
        wavelen = 2.0 * math.pi / inv
        smooth = (old / wavelen - lo) / (hi - lo)
        mid = (1.0 - smooth) * (inv / f) + smooth * inv
        inv = np.where(wavelen > old / lo, inv / f, np.where(wavelen > old / hi, mid, inv))
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def precision_mask(layers: int, w4a16_frac: float, seed: int) -> np.ndarray:
    """Seeded per-layer importance: round(frac * layers) layers get 1.0 (W4A16 under
    the default threshold 0.7), the rest 0.0 (W4A8)."""
    imp = np.zeros(layers, np.float64)
    n16 = int(round(w4a16_frac * layers))
    if n16:
        imp[np.random.default_rng(seed).choice(layers, size=n16, replace=False)] = 1.0
    return imp


def _w4(t: tuple[torch.Tensor, torch.Tensor], n: int, k: int) -> W4Weight:
    return W4Weight(t[0].data_ptr(), t[1].data_ptr(), n, k)


class DecodeModel:
    """Device-resident synthetic decoder; weights and caches are torch tensors (plumbing),
    every computation runs in libnve_hip.so."""

    def __init__(self, shape: ModelShape = LLAMA_3_2_3B, *, max_seq: int = 1024, prefill: int = 512,
                 w4a16_frac: float = 0.3, seed: int = 0x4E5645, lm_head_w4a8: bool = True,
                 importance: np.ndarray | None = None, device: str = "cuda"):
        assert prefill < max_seq
        self.shape = s = shape
        self.max_seq = max_seq
        self.prefill = prefill
        self.device = device
        g = torch.Generator(device=device).manual_seed(seed)
        H, F, D = s.hidden, s.ffn, s.head_dim
        QD, KD = s.heads * D, s.kv_heads * D
        self.importance = precision_mask(s.layers, w4a16_frac, seed) if importance is None else importance
        L = lib()
        self.use_w4a8 = [int(L.nve_use_w4a8(float(x))) for x in self.importance]
        self.lm_head_w4a8 = int(lm_head_w4a8)

        def qw(n, k):
            w = torch.randn((n, k), generator=g, device=device, dtype=torch.float32).mul_(0.02)
            return hk.q4_quantize(w)

        def norm_w(n):
            return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

        self.layers = []
        for _ in range(s.layers):
            lw = {"input_norm": norm_w(H), "post_attn_norm": norm_w(H),
                  "q": qw(QD, H), "k": qw(KD, H), "v": qw(KD, H), "o": qw(H, QD),
                  "gate": qw(F, H), "up": qw(F, H), "down": qw(H, F)}
            kc = torch.zeros((s.kv_heads, max_seq, D), dtype=torch.bfloat16, device=device)
            vc = torch.zeros_like(kc)
            if prefill:
                kc[:, :prefill].copy_(torch.randn((s.kv_heads, prefill, D), generator=g, device=device))
                vc[:, :prefill].copy_(torch.randn((s.kv_heads, prefill, D), generator=g, device=device))
            lw["k_cache"], lw["v_cache"] = kc, vc
            self.layers.append(lw)
        self.final_norm = norm_w(H)
        self.lm_head = qw(s.vocab, H)
        self.embed = torch.randn((s.vocab, H), generator=g, device=device).to(torch.bfloat16)
        cos, sin = rope_tables(D, max_seq, s.rope_theta, s.rope_scaling)
        self.rope_cos = torch.from_numpy(cos).to(device)
        self.rope_sin = torch.from_numpy(sin).to(device)

        self.cfg = DecodeConfig(H, s.heads, s.kv_heads, D, F, max_seq, s.vocab, s.eps)
        ws_bytes = int(L.nve_hip_decode_workspace_bytes(C.byref(self.cfg)))
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)  # scratch
        self.hidden = torch.zeros(H, dtype=torch.float32, device=device)
        self.pos = torch.full((1,), prefill, dtype=torch.int32, device=device)
        self.token = torch.zeros(1, dtype=torch.int32, device=device)
        self.logits = torch.empty(s.vocab, dtype=torch.float32, device=device)

        # C structs (kept alive with the model)
        self._lw = []
        self._io = []
        for lw in self.layers:
            w = LayerWeights(lw["input_norm"].data_ptr(), lw["post_attn_norm"].data_ptr(),
                             _w4(lw["q"], QD, H), _w4(lw["k"], KD, H), _w4(lw["v"], KD, H), _w4(lw["o"], H, QD),
                             _w4(lw["gate"], F, H), _w4(lw["up"], F, H), _w4(lw["down"], H, F))
            io = DecodeIO(self.hidden.data_ptr(), lw["k_cache"].data_ptr(), lw["v_cache"].data_ptr(),
                          self.pos.data_ptr(), self.rope_cos.data_ptr(), self.rope_sin.data_ptr(),
                          self.workspace.data_ptr())
            self._lw.append(w)
            self._io.append(io)
        self._head = DecodeHead(self.hidden.data_ptr(), self.final_norm.data_ptr(), _w4(self.lm_head, s.vocab, H),
                                self.embed.data_ptr(), self.logits.data_ptr(), self.token.data_ptr(),
                                self.pos.data_ptr(), self.workspace.data_ptr())
        self.graph = None
        self.length = prefill  # host shadow of the device position

    # -- state ------------------------------------------------------------------
    def start(self, token: int) -> None:
        """Reset the position to the prefill length and embed `token` as the input."""
        if not 0 <= int(token) < self.shape.vocab:
            raise ValueError(f"token {token} outside the vocabulary")
        self.pos.fill_(self.prefill)
        self.length = self.prefill
        self.token.fill_(int(token))
        check("nve_hip_embed", lib().nve_hip_embed(self.embed.data_ptr(), self.token.data_ptr(),
                                                    self.hidden.data_ptr(), self.shape.hidden,
                                                    torch.cuda.current_stream().cuda_stream))

    def _advance(self, n: int) -> None:
        if self.length + n > self.max_seq:
            raise ValueError(f"{n} more tokens would pass the KV cache ({self.length} of {self.max_seq} used)")
        self.length += n

    def step(self) -> None:
        """One token: every layer at its precision, then the head (enqueued, async)."""
        self._advance(1)
        self._enqueue()

    def _enqueue(self) -> None:
        for i in range(self.shape.layers):
            self.layer(i)
        self.head()

    def layer(self, i: int) -> None:
        """Layer i at its precision on the current hidden state and position (enqueued;
        does not advance the position)."""
        check("nve_hip_layer_forward_decode",
              lib().nve_hip_layer_forward_decode(C.byref(self.cfg), C.byref(self._lw[i]), C.byref(self._io[i]),
                                                 self.use_w4a8[i], torch.cuda.current_stream().cuda_stream))

    def head(self) -> None:
        """Final norm, lm_head, argmax, next-token embedding, position + 1 (enqueued)."""
        check("nve_hip_decode_head",
              lib().nve_hip_decode_head(C.byref(self.cfg), C.byref(self._head), self.lm_head_w4a8,
                                        torch.cuda.current_stream().cuda_stream))

    def capture(self) -> None:
        """Capture one step as a HIP graph (position and token stay device-side)."""
        pos0, len0 = self.pos.clone(), self.length
        hid0, tok0 = self.hidden.clone(), self.token.clone()
        self._enqueue()  # warm (kernel attributes, lazy init) before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._enqueue()
        torch.cuda.synchronize()
        # the warm-up step advanced the state (capture executes nothing): restore it; the
        # KV slot it wrote is rewritten by the next step
        self.pos.copy_(pos0)
        self.hidden.copy_(hid0)
        self.token.copy_(tok0)
        self.length = len0
        self.graph = g

    def generate(self, n: int, use_graph: bool = True) -> None:
        """n greedy tokens; the graph path replays the captured step."""
        if use_graph and self.graph is None:
            raise RuntimeError("capture() before generate(use_graph=True)")
        self._advance(n)
        for _ in range(n):
            if use_graph:
                self.graph.replay()
            else:
                self._enqueue()

    def step_bytes(self) -> int:
        """Algorithmic HBM bytes of one step: weights + scales of every GEMV, the KV
        cache read at the current length, embedding row, norms (approximate: weights
        dominate)."""
        s = self.shape
        H, F, D = s.hidden, s.ffn, s.head_dim
        QD, KD = s.heads * D, s.kv_heads * D
        per_layer = (QD + 2 * KD) * H + H * QD + 2 * F * H + H * F
        wbytes = per_layer * 0.625 * s.layers + s.vocab * H * 0.625
        return int(wbytes)

    def kv_bytes(self, length: int) -> int:
        s = self.shape
        return 2 * s.layers * s.kv_heads * length * s.head_dim * 2
