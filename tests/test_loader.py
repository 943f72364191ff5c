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
