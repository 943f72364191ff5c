"""The C ABI library loads, exports every symbol include/nve_kernels.h declares, and
rejects bad arguments with the documented status codes before touching the GPU.
CPU only (no compute calls)."""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nve_kernels.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nve_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from nve_amd._lib import lib
    return lib()


def test_header_declarations_found():
    names = _declared()
    for must in ("nve_quantize_f16_q8", "nve_matvec_w4a8", "nve_matvec_w4a16", "nve_qkv_matvec_w4a16"):
        assert must in names


def test_every_declared_symbol_is_exported(L):
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from nve_amd._lib import SIGNATURES
    assert sorted(SIGNATURES) == _declared()


def test_version_and_status_strings(L):
    assert b"gfx950" in L.nve_hip_version()
    assert b"null" in L.nve_hip_status_string(-1)
    assert b"shape" in L.nve_hip_status_string(-2)
    assert b"align" in L.nve_hip_status_string(-3)


P16 = 0x10000  # an aligned fake device address; validation fails before any use


def test_w4a8_argument_errors(L):
    f = L.nve_hip_matvec_w4a8
    assert f(None, P16, P16, P16, P16, 2, 8, 64, None) == -1           # null xq
    assert f(P16, P16, P16, P16, P16, 2, 8, 48, None) == -2            # K % 32
    assert f(P16, P16, P16, P16, P16, 2, 0, 64, None) == -2            # N = 0
    assert f(P16, P16, P16, P16, P16, 2, 8, 65536, None) == -5         # K > NVE_MAX_K
    # the reference's contract: nibbles 2-byte, xq 4-byte aligned (the main kernels need
    # 16; weaker alignment down to the contract is served, below it refused)
    assert f(P16, P16, P16 + 1, P16, P16, 2, 8, 64, None) == -3        # nibbles odd
    assert f(P16 + 2, P16, P16, P16, P16, 2, 8, 64, None) == -3        # xq not 4-byte aligned
    assert f(P16, P16, P16, P16, P16, 7, 8, 64, None) == -4            # out dtype
    assert L.nve_hip_last_status() == -4


def test_w4a16_argument_errors(L):
    f = L.nve_hip_matvec_w4a16
    assert f(None, 0, P16, P16, None, P16, 0, 8, 64, None) == -1
    assert f(P16, 2, P16, P16, None, P16, 0, 8, 64, None) == -4        # f32 x not accepted
    assert f(P16, 0, P16, P16, P16 + 2, P16, 0, 8, 64, None) == -3     # awq not 4-byte aligned
    assert f(P16 + 1, 0, P16, P16, None, P16, 0, 8, 64, None) == -3    # fp16 x odd
    assert f(P16, 0, P16, P16, None, P16, 0, -1, 64, None) == -2


def test_batched_and_prep_argument_errors(L):
    assert L.nve_hip_matvec_w4a8_batched(0, P16, P16, 0, P16, P16, P16, 2, 8, 64, None) == -2
    assert L.nve_hip_matvec_w4a8_batched(17, P16, P16, 0, P16, P16, P16, 2, 8, 64, None) == -2
    assert L.nve_hip_matvec_w4a8_batched(4, P16, P16, 5, P16, P16, P16, 2, 8, 64, None) == -4
    assert L.nve_hip_quantize_q8(P16, 0, 1, 40, P16, P16, None) == -2
    assert L.nve_hip_quantize_q8(P16 + 1, 0, 1, 64, P16, P16, None) == -3   # fp16 x odd
    assert L.nve_hip_quantize_q8(P16 + 2, 2, 1, 64, P16, P16, None) == -3   # f32 x not 4-byte aligned
    assert L.nve_hip_quantize_q8_rows(P16, 9, 1, 64, P16, P16, None) == -4
    assert L.nve_hip_q4_quantize(P16, 2, 4, 33, P16, P16, None) == -2
    assert L.nve_hip_q4_repack(P16, 4, 64, P16 + 8, P16, None) == -3
    assert L.nve_hip_w4a8_block_acc(None, P16, P16, 1, 32, None) == -1
    assert L.nve_hip_stream_read(P16, 24, P16, None) == -2
    assert L.nve_hip_qkv_matvec_w4a16(P16, 0, P16, P16, None, 8, P16, P16, None, 0, P16, P16, None, 8,
                                      P16, P16, P16, 0, 64, None) == -2


def test_decode_argument_errors(L):
    from nve_amd._lib import DecodeConfig, DecodeHead, DecodeIO, LayerWeights, W4Weight
    H, F, D, hq, hkv = 256, 512, 64, 4, 2

    def w(n, k):
        return W4Weight(P16, P16, n, k)

    def weights(**over):
        d = dict(q=w(hq * D, H), k=w(hkv * D, H), v=w(hkv * D, H), o=w(H, hq * D), gate=w(F, H), up=w(F, H),
                 down=w(H, F))
        d.update(over)
        return LayerWeights(P16, P16, d["q"], d["k"], d["v"], d["o"], d["gate"], d["up"], d["down"])

    io = DecodeIO(P16, P16, P16, P16, P16, P16, P16)
    f = L.nve_hip_layer_forward_decode

    def call(cfg, wts=None, iox=io):
        return f(C.byref(cfg), C.byref(wts or weights()), C.byref(iox), 1, None)

    assert call(DecodeConfig(H, hq, hkv, 96, F, 64, 512, 1e-5)) == -2        # head_dim 96
    assert call(DecodeConfig(H, 12, 1, D, F, 64, 512, 1e-5)) == -2           # 12 q heads per kv head
    assert call(DecodeConfig(H + 16, hq, hkv, D, F, 64, 512, 1e-5)) == -2    # H % 32
    assert call(DecodeConfig(H, hq, hkv, D, F, 1 << 26, 512, 1e-5)) == -5    # cache index past int32
    cfg = DecodeConfig(H, hq, hkv, D, F, 64, 512, 1e-5)
    assert call(cfg, weights(gate=w(F, H + 32))) == -2                       # weight shape mismatch
    assert call(cfg, weights(down=W4Weight(None, P16, H, F))) == -1
    assert call(cfg, weights(o=W4Weight(P16 + 4, P16, H, hq * D))) == -3
    assert call(cfg, iox=DecodeIO(P16, P16, P16, None, P16, P16, P16)) == -1  # pos
    assert call(cfg, iox=DecodeIO(P16, P16, P16, P16, P16, P16, P16 + 16)) == -3  # workspace alignment
    # the stage entry point: same layer checks, plus its stage code and in / out
    st = L.nve_hip_decode_stage
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, 4, P16, P16, None) == -4      # stage code
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, -1, P16, P16, None) == -4
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, 0, None, None, None) == -1    # QKV needs out
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, 1, None, None, None) == -1    # merge needs in
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, 2, None, P16 + 8, None) == -3  # out alignment
    assert st(C.byref(cfg), C.byref(weights()), C.byref(io), 1, 3, P16 + 4, None, None) == -3  # in alignment
    assert st(C.byref(DecodeConfig(H, hq, hkv, 96, F, 64, 512, 1e-5)), C.byref(weights()), C.byref(io), 1, 0,
              None, P16, None) == -2
    iow = DecodeIO(P16, P16, P16, P16, P16, P16, None)
    assert st(C.byref(cfg), C.byref(weights()), C.byref(iow), 1, 0, None, P16, None) == -1    # workspace
    bad = DecodeHead(P16, P16, w(512, H + 32), P16, P16, P16, P16, P16)
    assert L.nve_hip_decode_head(C.byref(cfg), C.byref(bad), 1, None) == -2
    assert L.nve_hip_embed(None, P16, P16, H, 512, None) == -1
    assert L.nve_hip_embed(P16, P16, P16, H, 0, None) == -2
    assert L.nve_hip_decode_workspace_bytes(C.byref(cfg)) % 256 == 0


def test_attention_split_rule(L, monkeypatch):
    """Key splits of the decode attention (host rule): 1 up to 256 cache slots, 4 up to
    1024, 8 above where num_heads * head_dim <= 4096 (else 4); NVE_ATTN_SPLIT overrides
    within that maximum."""
    from nve_amd._lib import DecodeConfig
    monkeypatch.delenv("NVE_ATTN_SPLIT", raising=False)

    def splits(seq, heads=24, d=128):
        return L.nve_hip_decode_attn_splits(C.byref(DecodeConfig(3072, heads, 8, d, 8192, seq, 0, 1e-5)))
    assert [splits(s) for s in (1, 256, 257, 1024, 1025, 8192)] == [1, 1, 4, 4, 8, 8]
    assert splits(8192, heads=48) == 4                  # 48 x 128 > 4096: four splits at most
    for v, want in (("1", 1), ("2", 2), ("4", 4), ("8", 8), ("3", 4), ("16", 4)):
        monkeypatch.setenv("NVE_ATTN_SPLIT", v)
        assert splits(1024) == want, v                  # invalid values keep the default
    monkeypatch.setenv("NVE_ATTN_SPLIT", "8")
    assert splits(1024, heads=48) == 4
    assert L.nve_hip_decode_attn_splits(C.byref(DecodeConfig(3072, 24, 8, 96, 8192, 64, 0, 1e-5))) == -2


def test_stream_read_mode_argument_errors(L):
    f = L.nve_hip_stream_read_mode
    assert f(None, 64, P16, 0, None) == -1
    assert f(P16, 24, P16, 1, None) == -2       # not a multiple of 16
    assert f(P16, 0, P16, 2, None) == -2
    assert f(P16, 64, P16, 3, None) == -4       # mode
    assert f(P16 + 8, 64, P16, 0, None) == -3   # buffer alignment


def test_dispatch_env_rules(L, orc, monkeypatch):
    """nve_use_w4a8 (src/gpu_layer.rs:1013-1025) against the oracle's truth table."""
    monkeypatch.delenv("NVE_NO_W4A8", raising=False)
    monkeypatch.delenv("NVE_W4A8_THRESHOLD", raising=False)
    for imp in (0.0, 0.3, 0.6999, 0.7, 0.71, 1.0):
        assert L.nve_use_w4a8(imp) == int(orc.use_w4a8(imp, False)), imp
    monkeypatch.setenv("NVE_W4A8_THRESHOLD", "0.25")
    for imp in (0.0, 0.2499, 0.25, 0.5):
        assert L.nve_use_w4a8(imp) == int(orc.use_w4a8(imp, False, 0.25)), imp
    for bad in ("abc", " 0.25", "0x1p-2", "0.25 ", ""):
        monkeypatch.setenv("NVE_W4A8_THRESHOLD", bad)  # unparsable -> default 0.7
        assert L.nve_use_w4a8(0.5) == 1 and L.nve_use_w4a8(0.7) == 0, repr(bad)
    monkeypatch.setenv("NVE_W4A8_THRESHOLD", "1e-1")
    assert L.nve_use_w4a8(0.05) == 1 and L.nve_use_w4a8(0.1) == 0
    monkeypatch.setenv("NVE_NO_W4A8", "1")
    assert L.nve_use_w4a8(0.0) == 0
    monkeypatch.setenv("NVE_NO_W4A8", "")  # set but empty still counts as set
    assert L.nve_use_w4a8(0.0) == 0


def test_product_path_has_no_oracle_dependency():
    """Nothing under nve_amd/ imports or links the oracle."""
    for p in (ROOT / "nve_amd").rglob("*"):
        if p.suffix in (".py", ".hip", ".h", ".cpp"):
            assert "oracle" not in p.read_text(), p


def test_build_id_matches_sources(L):
    """The loaded library was built from the sources in this tree (the loader refuses
    any other, so tests and the bench never measure a stale binary)."""
    from nve_amd.build_ext import source_id
    bid = L.nve_hip_build_id().decode()
    assert len(bid) == 32 and bid == source_id()


def test_build_id_changes_with_sources(tmp_path, monkeypatch):
    from nve_amd import build_ext
    a = build_ext.source_id()
    d = tmp_path / "csrc"
    d.mkdir()
    for f in build_ext.CSRC.iterdir():
        if f.is_file():
            (d / f.name).write_bytes(f.read_bytes())
    monkeypatch.setattr(build_ext, "CSRC", d)
    assert build_ext.source_id() == a
    (d / "common.h").write_bytes((d / "common.h").read_bytes() + b"\n")
    assert build_ext.source_id() != a
