"""bench.py's command-line contract that runs without a GPU: more than one GPU is
refused with a message (this build measures one MI355X), and the bench helpers that
mirror library policy agree with it."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_multi_gpu_refused_with_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=str(ROOT))
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


def test_attn_key_split_mirror(monkeypatch):
    import bench
    from nve_amd.decode import LLAMA_3_2_3B, ModelShape
    monkeypatch.delenv("NVE_ATTN_SPLIT", raising=False)
    assert [bench.attn_key_split(LLAMA_3_2_3B, ms) for ms in (128, 256, 257, 1024, 1025, 8192)] == [1, 1, 4, 4, 8, 8]
    wide = ModelShape(hidden=4096, layers=1, heads=64, kv_heads=8, head_dim=128, ffn=8192, vocab=32)
    assert bench.attn_key_split(wide, 8192) == 4       # num_heads * head_dim > 4096: four
    monkeypatch.setenv("NVE_ATTN_SPLIT", "8")
    assert bench.attn_key_split(LLAMA_3_2_3B, 512) == 8 and bench.attn_key_split(wide, 512) == 4
