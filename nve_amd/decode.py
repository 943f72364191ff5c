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


def shape_from_hf_config(cfg: dict) -> ModelShape:
    """ModelShape from a Hugging Face Llama config.json dict (the fields the reference's
    generic loader reads from a checkpoint's config, src/arch.rs:200-262:
    hidden_size, num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
    intermediate_size, vocab_size, rms_norm_eps, rope_theta -- default 10000 as at
    src/arch.rs:221 -- and rope_scaling with rope_type "llama3"; rope_type "default"
    means no scaling)."""
    heads = int(cfg["num_attention_heads"])
    hidden = int(cfg["hidden_size"])
    rs = cfg.get("rope_scaling") or None
    scaling = None
    rtype = rs.get("rope_type", rs.get("type")) if rs else None
    if rtype == "default":
        rs = None
    if rs and rtype == "llama3":
        scaling = RopeScaling(float(rs["factor"]), float(rs.get("low_freq_factor", 1.0)),
                              float(rs.get("high_freq_factor", 4.0)),
                              int(rs.get("original_max_position_embeddings", 8192)))
    elif rs:
        raise ValueError(f"rope_scaling {rs} is not supported (llama3 only)")
    return ModelShape(hidden=hidden, layers=int(cfg["num_hidden_layers"]), heads=heads,
                      kv_heads=int(cfg.get("num_key_value_heads", heads)),
                      head_dim=int(cfg.get("head_dim") or hidden // heads), ffn=int(cfg["intermediate_size"]),
                      vocab=int(cfg["vocab_size"]), eps=float(cfg.get("rms_norm_eps", 1e-5)),
                      rope_theta=float(cfg.get("rope_theta", 10000.0)), rope_scaling=scaling)


def checkpoint_weights(w: dict, s: ModelShape, device: str = "cuda", tie_word_embeddings: bool = True) -> dict:
    """Decode-model weights from a loaded checkpoint (nve_amd.loader.load_safetensors_w4:
    block projections as GpuW4, every other tensor as stored), Hugging Face Llama names:
    model.layers.{i}.{input_layernorm, post_attention_layernorm}.weight,
    model.layers.{i}.self_attn.{q,k,v,o}_proj.weight, model.layers.{i}.mlp.{gate,up,down}_proj.weight,
    model.norm.weight, model.embed_tokens.weight and lm_head.weight (absent: tied to the
    embeddings when tie_word_embeddings -- config.json's field of that name -- is true,
    a KeyError otherwise).  Norms and embeddings become bf16; the lm_head is quantized to W4 on
    the device (the decode head's GEMV is W4A8 / W4A16).  AWQ-scaled projections are
    refused: the decode layer's GEMVs take no awq vector."""
    from .gpu_layer import GpuW4

    H, D = s.hidden, s.head_dim
    QD, KD, F = s.heads * D, s.kv_heads * D, s.ffn
    dims = {"q": (QD, H), "k": (KD, H), "v": (KD, H), "o": (H, QD), "gate": (F, H), "up": (F, H), "down": (H, F)}
    src = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
           "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}

    def get(name):
        if name not in w:
            raise KeyError(f"checkpoint has no tensor {name}")
        return w[name]

    def bf16(t, shape):
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"shape {tuple(t.shape)}, expected {tuple(shape)}")
        return t.to(device=device, dtype=torch.bfloat16).contiguous()

    def w4(name, n, k):
        g = get(name)
        if not isinstance(g, GpuW4):
            raise ValueError(f"{name} was not quantized on load")
        if (g.n, g.k) != (n, k):
            raise ValueError(f"{name}: [{g.n}, {g.k}], expected [{n}, {k}]")
        if g.awq_scales is not None:
            raise ValueError(f"{name}: AWQ-scaled weights are not supported by the decode layer")
        return g.nibbles, g.scales

    layers = []
    for i in range(s.layers):
        p = f"model.layers.{i}."
        lw = {"input_norm": bf16(get(p + "input_layernorm.weight"), (H,)),
              "post_attn_norm": bf16(get(p + "post_attention_layernorm.weight"), (H,))}
        for nm, (n, k) in dims.items():
            lw[nm] = w4(p + src[nm] + ".weight", n, k)
        layers.append(lw)
    embed = bf16(get("model.embed_tokens.weight"), (s.vocab, H))
    if "lm_head.weight" not in w and not tie_word_embeddings:
        raise KeyError("checkpoint has no tensor lm_head.weight and tie_word_embeddings is false")
    head = w.get("lm_head.weight", embed)
    if isinstance(head, GpuW4):
        lm_head = w4("lm_head.weight", s.vocab, H)
    else:
        g = GpuW4.quantize(bf16(head, (s.vocab, H)))
        lm_head = (g.nibbles, g.scales)
    return {"layers": layers, "final_norm": bf16(get("model.norm.weight"), (H,)), "lm_head": lm_head,
            "embed": embed}


class DecodeModel:
    """Device-resident synthetic decoder; weights and caches are torch tensors (plumbing),
    every computation runs in libnve_hip.so."""

    def __init__(self, shape: ModelShape = LLAMA_3_2_3B, *, max_seq: int = 1024, prefill: int = 512,
                 w4a16_frac: float = 0.3, seed: int = 0x4E5645, lm_head_w4a8: bool = True,
                 importance: np.ndarray | None = None, device: str = "cuda", weights: dict | None = None):
        """weights: None for seeded random weights, or a checkpoint loaded with
        nve_amd.loader.load_safetensors_w4 (Hugging Face Llama tensor names; see
        checkpoint_weights).  `prefill` cached positions hold seeded N(0, 1) keys and
        values either way (0 for an empty cache)."""
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

        loaded = checkpoint_weights(weights, s, device) if weights is not None else None
        self.layers = []
        for li in range(s.layers):
            if loaded is not None:
                lw = dict(loaded["layers"][li])
            else:
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
        if loaded is not None:
            self.final_norm, self.lm_head, self.embed = loaded["final_norm"], loaded["lm_head"], loaded["embed"]
        else:
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
                                                    self.hidden.data_ptr(), self.shape.hidden, self.shape.vocab,
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

    def capture(self, steps_per_graph: int = 1) -> None:
        """Capture one step as a HIP graph (position and token stay device-side), and,
        with steps_per_graph > 1, also that many consecutive steps as one graph: every
        step reads the token and position the previous one left on the device, so a
        replay of the longer graph is that many greedy tokens, with one graph launch
        instead of one per token."""
        if steps_per_graph < 1:
            raise ValueError("steps_per_graph must be >= 1")
        pos0, len0 = self.pos.clone(), self.length
        hid0, tok0 = self.hidden.clone(), self.token.clone()
        self._enqueue()  # warm (kernel attributes, lazy init) before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._enqueue()
        gm = None
        if steps_per_graph > 1:
            gm = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gm):
                for _ in range(steps_per_graph):
                    self._enqueue()
        torch.cuda.synchronize()
        # the warm-up step advanced the state (capture executes nothing): restore it; the
        # KV slot it wrote is rewritten by the next step
        self.pos.copy_(pos0)
        self.hidden.copy_(hid0)
        self.token.copy_(tok0)
        self.length = len0
        self.graph = g
        self.graph_multi = gm
        self.steps_per_graph = steps_per_graph

    def generate(self, n: int, use_graph: bool = True) -> None:
        """n greedy tokens; the graph path replays the captured steps (the multi-step
        graph while at least steps_per_graph tokens remain, then the one-step graph)."""
        if use_graph and self.graph is None:
            raise RuntimeError("capture() before generate(use_graph=True)")
        self._advance(n)
        if not use_graph:
            for _ in range(n):
                self._enqueue()
            return
        q, r = (divmod(n, self.steps_per_graph) if getattr(self, "graph_multi", None) is not None else (0, n))
        for _ in range(q):
            self.graph_multi.replay()
        for _ in range(r):
            self.graph.replay()

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
