"""nve_hip_layer_forward_decode_noalloc: the decode layer with its scratch in a
file-scope device array of the library (1 MiB) instead of a caller workspace.

Checked through the C ABI against nve_hip_layer_forward_decode on the same state:
two calls in a row, the second on a smaller model, each for a W4A8 and a W4A16 layer;
the residual stream and the KV-cache rows written must match bit for bit (the same
kernels run on the same inputs).  A configuration whose layer workspace exceeds the
array is refused with NVE_ERR_TOO_LARGE before anything runs.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nve_amd._lib import lib
    return torch, lib()


def _model(shape_kw, max_seq, prefill, seed):
    from nve_amd.decode import DecodeModel, ModelShape
    s = ModelShape(**shape_kw)
    return DecodeModel(s, max_seq=max_seq, prefill=prefill, importance=np.array([0.0, 1.0][:s.layers]), seed=seed)


def _state(m, li):
    return (m.hidden.clone(), m.layers[li]["k_cache"].clone(), m.layers[li]["v_cache"].clone())


def _restore(m, li, st):
    m.hidden.copy_(st[0])
    m.layers[li]["k_cache"].copy_(st[1])
    m.layers[li]["v_cache"].copy_(st[2])


def _compare(torch, L, m, token):
    stream = torch.cuda.current_stream().cuda_stream
    m.start(token)
    for li in range(m.shape.layers):
        print(f"noalloc layer {li} w4a8={m.use_w4a8[li]} hidden={m.shape.hidden}", flush=True)
        before = _state(m, li)
        assert L.nve_hip_layer_forward_decode(C.byref(m.cfg), C.byref(m._lw[li]), C.byref(m._io[li]),
                                              m.use_w4a8[li], stream) == 0
        torch.cuda.synchronize()
        ref = _state(m, li)
        _restore(m, li, before)
        io = type(m._io[li])(m._io[li].hidden, m._io[li].k_cache, m._io[li].v_cache, m._io[li].pos,
                             m._io[li].rope_cos, m._io[li].rope_sin, None)  # no workspace
        assert L.nve_hip_layer_forward_decode_noalloc(C.byref(m.cfg), C.byref(m._lw[li]), C.byref(io),
                                                      m.use_w4a8[li], stream) == 0
        torch.cuda.synchronize()
        got = _state(m, li)
        for a, b in zip(ref, got):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
        assert not torch.equal(ref[0], before[0])  # the layer did change the residual


def test_noalloc_layer_matches_workspace_layer(env):
    torch, L = env
    big = _model(dict(hidden=512, layers=2, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=256,
                      rope_theta=10000.0), max_seq=600, prefill=520, seed=5)  # 4-way key split
    _compare(torch, L, big, 3)
    small = _model(dict(hidden=128, layers=2, heads=2, kv_heads=1, head_dim=64, ffn=256, vocab=128,
                        rope_theta=10000.0), max_seq=40, prefill=10, seed=6)
    _compare(torch, L, small, 7)


def test_noalloc_rejects_oversized_config(env):
    """512 heads of 64: the key-split partials alone exceed the 1 MiB array."""
    torch, L = env
    from nve_amd._lib import DecodeConfig, DecodeIO, LayerWeights, W4Weight
    P = 0x10000
    H, QD, KD, F = 4096, 512 * 64, 64 * 64, 4096
    cfg = DecodeConfig(H, 512, 64, 64, F, 4096, 0, 1e-5)

    def w(n, k):
        return W4Weight(P, P, n, k)

    lw = LayerWeights(P, P, w(QD, H), w(KD, H), w(KD, H), w(H, QD), w(F, H), w(F, H), w(H, F))
    io = DecodeIO(P, P, P, P, P, P, None)
    assert L.nve_hip_layer_forward_decode_noalloc(C.byref(cfg), C.byref(lw), C.byref(io), 1, None) == -5
