"""Quantize-on-load from safetensors and Q4_0 block files (nve_amd/loader.py) on the
device, against the oracle's QuantizedTensor::from_f32 + extract_for_gpu (bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _ref(orc, w32: np.ndarray):
    n, k = w32.shape
    return orc.extract_for_gpu(orc.q4_from_f32(w32.astype(np.float32)), n, k)


def test_safetensors_quantize_on_load(torch_dev, orc, tmp_path):
    torch = torch_dev
    from safetensors.torch import save_file
    from nve_amd.gpu_layer import GpuW4
    from nve_amd.loader import load_safetensors_w4
    q = torch.from_numpy(weights(64, 128, seed=3)).to(torch.bfloat16)
    down = torch.from_numpy(weights(32, 96, seed=4)).to(torch.float16)
    up = torch.from_numpy(weights(48, 64, seed=5))                        # f32 checkpoint
    odd = torch.from_numpy(weights(8, 40, seed=6)).to(torch.bfloat16)     # K % 32 != 0: kept
    norm = torch.from_numpy(weights(1, 128, seed=7)[0] + 1.0).to(torch.bfloat16)
    emb = torch.from_numpy(weights(16, 128, seed=8)).to(torch.bfloat16)
    path = tmp_path / "model.safetensors"
    save_file({"model.layers.0.self_attn.q_proj.weight": q, "model.layers.0.mlp.down_proj.weight": down,
               "model.layers.1.mlp.up_proj.weight": up, "model.layers.0.self_attn.k_proj.weight": odd,
               "model.layers.0.input_layernorm.weight": norm, "model.embed_tokens.weight": emb}, str(path))
    out = load_safetensors_w4(str(path))
    assert set(out) == {"model.layers.0.self_attn.q_proj.weight", "model.layers.0.mlp.down_proj.weight",
                        "model.layers.1.mlp.up_proj.weight", "model.layers.0.self_attn.k_proj.weight",
                        "model.layers.0.input_layernorm.weight", "model.embed_tokens.weight"}
    for name, src in (("model.layers.0.self_attn.q_proj.weight", q), ("model.layers.0.mlp.down_proj.weight", down),
                      ("model.layers.1.mlp.up_proj.weight", up)):
        g = out[name]
        assert isinstance(g, GpuW4) and (g.n, g.k) == tuple(src.shape) and g.awq_scales is None
        nib_ref, sc_ref = _ref(orc, src.float().numpy())
        assert np.array_equal(g.nibbles.cpu().numpy().reshape(-1), nib_ref.reshape(-1)), name
        assert np.array_equal(g.scales.cpu().numpy().reshape(-1), sc_ref.reshape(-1)), name
    for name, src in (("model.layers.0.self_attn.k_proj.weight", odd), ("model.layers.0.input_layernorm.weight", norm),
                      ("model.embed_tokens.weight", emb)):
        t = out[name]
        assert not isinstance(t, GpuW4) and t.is_cuda and t.dtype == src.dtype
        assert torch.equal(t.cpu(), src)


def test_safetensors_awq_on_load(torch_dev, orc, tmp_path):
    """The AWQ path: from_compact_awq_kquant with the caller's per-channel scales."""
    torch = torch_dev
    from safetensors.torch import save_file
    from nve_amd.loader import load_safetensors_w4
    w = torch.from_numpy(weights(24, 64, seed=9)).to(torch.bfloat16)
    awq = (np.random.default_rng(1).random(64) * 2 + 0.25).astype(np.float32)
    path = tmp_path / "m.safetensors"
    save_file({"model.layers.0.mlp.gate_proj.weight": w}, str(path))
    for kq in (True, False):
        g = load_safetensors_w4(str(path), awq=lambda nm: torch.from_numpy(awq), kquant=kq)[
            "model.layers.0.mlp.gate_proj.weight"]
        data_ref, inv_ref = orc.q4_from_f32_awq(w.float().numpy(), awq, kq)
        nib_ref, sc_ref = orc.extract_for_gpu(data_ref, 24, 64)
        assert np.array_equal(g.nibbles.cpu().numpy().reshape(-1), nib_ref.reshape(-1))
        assert np.array_equal(g.scales.cpu().numpy().reshape(-1), sc_ref.reshape(-1))
        assert np.array_equal(g.awq_scales.cpu().numpy(), inv_ref)


def test_q4_file_load(torch_dev, orc, tmp_path):
    from nve_amd.loader import load_q4_file, write_q4_blocks
    wa, wb = weights(40, 128, seed=10), weights(8, 4096, seed=11)
    path = str(tmp_path / "w.q4")
    write_q4_blocks(path, orc.q4_from_f32(wa))
    off = write_q4_blocks(path, orc.q4_from_f32(wb), append=True)
    for w, o in ((wa, 0), (wb, off)):
        n, k = w.shape
        g = load_q4_file(path, n, k, offset=o)
        nib_ref, sc_ref = _ref(orc, w)
        assert np.array_equal(g.nibbles.cpu().numpy().reshape(-1), nib_ref.reshape(-1))
        assert np.array_equal(g.scales.cpu().numpy().reshape(-1), sc_ref.reshape(-1))
