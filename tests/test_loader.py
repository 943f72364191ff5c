"""Host side of the file-level loaders (nve_amd/loader.py): which tensors are quantized
on load (GenericBlockWeights::quantize_q4, src/generic_model.rs:69-85) and the Q4_0
block file format (QuantizedTensor.data, src/quantize.rs:711-731)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import weights


def test_projection_selection():
    from nve_amd.loader import is_block_projection, quantizable
    for nm in ("model.layers.3.self_attn.q_proj.weight", "model.layers.0.self_attn.k_proj.weight",
               "model.layers.0.self_attn.v_proj.weight", "model.layers.0.self_attn.o_proj.weight",
               "model.layers.7.mlp.gate_proj.weight", "model.layers.7.mlp.up_proj.weight",
               "model.layers.7.mlp.down_proj.weight"):
        assert is_block_projection(nm), nm
        assert quantizable(nm, (64, 128))
    for nm in ("model.embed_tokens.weight", "lm_head.weight", "model.norm.weight",
               "model.layers.0.input_layernorm.weight", "model.layers.0.self_attn.q_proj.bias",
               "model.layers.0.post_attention_layernorm.weight", "q_proj"):
        assert not is_block_projection(nm), nm
    # rows must be whole blocks, and only matrices are quantized
    assert not quantizable("model.layers.0.self_attn.k_proj.weight", (8, 40))
    assert not quantizable("model.layers.0.self_attn.k_proj.weight", (128,))


def test_q4_block_file_round_trip(orc, tmp_path):
    from nve_amd.loader import q4_block_bytes, read_q4_blocks, write_q4_blocks
    a = orc.q4_from_f32(weights(6, 96, seed=1))
    b = orc.q4_from_f32(weights(3, 64, seed=2))
    assert a.size == q4_block_bytes(6, 96) and b.size == q4_block_bytes(3, 64)
    path = str(tmp_path / "w.q4")
    assert write_q4_blocks(path, a) == 0
    off = write_q4_blocks(path, b, append=True)
    assert off == a.size
    ra = read_q4_blocks(path, 6, 96)
    rb = read_q4_blocks(path, 3, 64, offset=off)
    assert ra.shape == (6, 3 * 20) and rb.shape == (3, 2 * 20)
    assert np.array_equal(np.asarray(ra).ravel(), a.ravel())
    assert np.array_equal(np.asarray(rb).ravel(), b.ravel())
    # the first block: f32 LE scale, then 16 nibble bytes
    w0 = weights(6, 96, seed=1)[0, :32]
    amax = np.abs(w0).max()
    assert np.frombuffer(bytes(ra[0, :4]), "<f4")[0] == np.float32(amax) / np.float32(7.0)


def test_q4_block_file_errors(tmp_path):
    from nve_amd.loader import q4_block_bytes, read_q4_blocks
    with pytest.raises(ValueError):
        q4_block_bytes(4, 40)
    path = tmp_path / "short.q4"
    path.write_bytes(b"\0" * 100)
    with pytest.raises(ValueError):
        read_q4_blocks(str(path), 2, 96)  # needs 2 * 3 * 20 = 120 bytes
    read_q4_blocks(str(path), 2, 64)      # 80 bytes: fits
    with pytest.raises(ValueError):
        read_q4_blocks(str(path), 2, 64, offset=40)


def test_shape_from_hf_config():
    """config.json fields -> ModelShape (the fields src/arch.rs:200-262 reads)."""
    from nve_amd.decode import ModelShape, shape_from_hf_config
    cfg = {"hidden_size": 3072, "num_hidden_layers": 28, "num_attention_heads": 24, "num_key_value_heads": 8,
           "intermediate_size": 8192, "vocab_size": 128256, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
           "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                            "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}}
    s = shape_from_hf_config(cfg)
    assert (s.hidden, s.layers, s.heads, s.kv_heads, s.head_dim, s.ffn, s.vocab) == \
        (3072, 28, 24, 8, 128, 8192, 128256)
    assert s.rope_scaling.factor == 32.0 and s.rope_scaling.original_max_position_embeddings == 8192
    # head_dim given explicitly wins; no kv heads means multi-head attention; no scaling
    s = shape_from_hf_config({"hidden_size": 256, "num_hidden_layers": 2, "num_attention_heads": 2,
                              "head_dim": 64, "intermediate_size": 512, "vocab_size": 100})
    assert (s.head_dim, s.kv_heads, s.rope_scaling, s.rope_theta, s.eps) == (64, 2, None, 10000.0, 1e-5)
    assert isinstance(s, ModelShape)
    with pytest.raises(ValueError):
        shape_from_hf_config({**cfg, "rope_scaling": {"rope_type": "yarn", "factor": 4.0}})
    # rope_type "default" is no scaling
    assert shape_from_hf_config({**cfg, "rope_scaling": {"rope_type": "default"}}).rope_scaling is None


def test_checkpoint_weights_rejects_mismatch():
    """A missing tensor is a KeyError; a norm, embedding or projection whose shape does
    not match the config, or a projection that was not quantized on load, a ValueError."""
    import torch
    from nve_amd.decode import ModelShape, checkpoint_weights
    s = ModelShape(hidden=64, layers=1, heads=2, kv_heads=1, head_dim=32, ffn=128, vocab=64)
    with pytest.raises(KeyError):
        checkpoint_weights({}, s, device="cpu")
    p = "model.layers.0."
    w = {p + "input_layernorm.weight": torch.ones(64), p + "post_attention_layernorm.weight": torch.ones(32)}
    with pytest.raises(ValueError):
        checkpoint_weights(w, s, device="cpu")
    w[p + "post_attention_layernorm.weight"] = torch.ones(64)
    w[p + "self_attn.q_proj.weight"] = torch.ones(64, 64)  # stored dense: not quantized on load
    with pytest.raises(ValueError):
        checkpoint_weights(w, s, device="cpu")


def test_checkpoint_weights_untied_needs_lm_head():
    """tie_word_embeddings = false and no lm_head.weight: a KeyError, not a silent tie."""
    from nve_amd.decode import ModelShape, checkpoint_weights
    s = ModelShape(hidden=64, layers=0, heads=2, kv_heads=1, head_dim=32, ffn=128, vocab=64)
    import torch
    w = {"model.embed_tokens.weight": torch.ones(64, 64), "model.norm.weight": torch.ones(64)}
    with pytest.raises(KeyError, match="lm_head"):
        checkpoint_weights(w, s, device="cpu", tie_word_embeddings=False)
