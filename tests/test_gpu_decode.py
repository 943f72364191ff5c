"""GPU parity of the decode step (nve_hip_layer_forward_decode + nve_hip_decode_head)
against the CPU restatement oracle/decode_ref.emulate_step, on small synthetic models.

Every layer and the head are teacher-forced: the oracle's layer starts from the GPU's
hidden state before that layer, so each is checked on its own.  Bars:
  * a layer's contribution (h_out - h_in) and the logits: ||gpu - oracle|| / ||oracle||
    <= 2e-3 (W4A8 activations are re-quantized at every projection input, so a
    last-ulp difference upstream can move an int8 code);
  * token: the GPU's token is the first maximum of the GPU's own logits (exact), and
    equals the oracle's whenever the oracle's top-2 gap exceeds the logit error;
  * KV cache: the slot written at pos equals the oracle's bf16 row to 1 bf16 ulp
    (plus 2e-3 of the row's rms for entries near zero);
  * HIP graph replay reproduces the eager sequence bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import rel_err_norm

pytestmark = pytest.mark.gpu

TOL_LAYER = 2e-3


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _model(torch, heads, kv, d, *, layers=3, hidden=256, ffn=512, vocab=512, max_seq=160, prefill=60,
           importance=(0.0, 1.0, 0.0), lm_head_w4a8=True, seed=11):
    from nve_amd.decode import DecodeModel, ModelShape
    shape = ModelShape(hidden=hidden, layers=layers, heads=heads, kv_heads=kv, head_dim=d, ffn=ffn, vocab=vocab,
                       rope_theta=10000.0)
    imp = np.array(importance[:layers], np.float64)
    return DecodeModel(shape, max_seq=max_seq, prefill=prefill, importance=imp, lm_head_w4a8=lm_head_w4a8,
                       seed=seed)


def _run_teacher_forced(torch, m, steps, token0=5, checked=None, record=None):
    """Layer by layer: the oracle's layer i starts from the GPU's hidden state before
    layer i, so every layer and the head are checked on their own.  checked: the layers
    to compare (None = all; the others only run).  record: a list that receives each
    step's (token, logits)."""
    from oracle import decode_ref as dr
    hm = dr.HostModel(m)
    m.start(token0)
    pos = m.prefill
    errs = []
    for i in range(steps):
        print(f"decode step {i} pos {pos}", flush=True)
        m._advance(1)
        for li in range(m.shape.layers):
            if checked is not None and li not in checked:
                m.layer(li)
                continue
            torch.cuda.synchronize()
            h_in = m.hidden.cpu().numpy().copy()
            m.layer(li)
            torch.cuda.synchronize()
            h_gpu = m.hidden.cpu().numpy()
            h_ora = dr.emulate_layer(hm, li, h_in, pos)
            err = rel_err_norm(h_gpu - h_in, h_ora - h_in)  # the layer's own contribution
            errs.append(("layer", li, m.use_w4a8[li], err))
            assert err <= TOL_LAYER, (i, li, err)
            for name in ("k_cache", "v_cache"):
                g_row = dr.bf16_to_f32(m.layers[li][name][:, pos].view(torch.int16).cpu().numpy().view(np.uint16))
                o_row = hm.layers[li][name][:, pos]
                # one bf16 ulp, plus the projection's own error on near-zero entries
                tol = np.abs(o_row) * 2.0 ** -7 + TOL_LAYER * np.sqrt(np.mean(o_row ** 2))
                assert np.all(np.abs(g_row - o_row) <= tol), (i, li, name)
        h_in = m.hidden.cpu().numpy().copy()
        m.head()
        torch.cuda.synchronize()
        g_logits = m.logits.cpu().numpy()
        g_tok = int(m.token.item())
        o_logits, o_tok = dr.emulate_head(hm, h_in)
        err = rel_err_norm(g_logits, o_logits)
        errs.append(("head", -1, m.lm_head_w4a8, err))
        assert err <= TOL_LAYER, (i, err)
        assert g_tok == int(np.argmax(g_logits))
        top = np.sort(o_logits)[-2:]
        if top[1] - top[0] > 4 * TOL_LAYER * np.linalg.norm(o_logits) / np.sqrt(o_logits.size):
            assert g_tok == o_tok, (i, g_tok, o_tok)
        if record is not None:
            record.append((g_tok, g_logits.copy()))
        # the head embedded the GPU's token and advanced the position
        assert np.array_equal(m.hidden.cpu().numpy(), hm.embed[g_tok])
        assert int(m.pos.item()) == pos + 1
        pos += 1
    print("max errors:", {k: max(e[3] for e in errs if (e[0], e[2]) == k)
                          for k in {(e[0], e[2]) for e in errs}}, flush=True)
    return m


@pytest.mark.parametrize("fuse,split", [("1", "8"), ("1", "4"), ("1", "2"), ("1", "1"), ("0", "1")])
@pytest.mark.parametrize("heads,kv,d", [(4, 2, 64), (6, 2, 128), (8, 1, 64), (2, 2, 256), (24, 8, 128)])
def test_decode_step_mixed_precision(torch_dev, heads, kv, d, fuse, split, monkeypatch):
    """Every layer path: the five launches with producers fused into the
    GEMV staging, and standalone RMSNorm / SiLU-mul kernels (NVE_DECODE_FUSE=0); fused
    attention split over 1, 2, 4 or 8 workgroups per head (at 61..66 keys most splits
    have no tile: their partials are empty and must drop out of the merge)."""
    monkeypatch.setenv("NVE_DECODE_FUSE", fuse)
    monkeypatch.setenv("NVE_ATTN_SPLIT", split)
    m = _model(torch_dev, heads, kv, d)
    _run_teacher_forced(torch_dev, m, steps=6)  # pos 60..65 crosses a 64-key boundary


@pytest.mark.parametrize("importance,lm8", [((0.0, 0.0), True), ((1.0, 1.0), False)])
def test_decode_step_single_precision(torch_dev, importance, lm8):
    m = _model(torch_dev, 4, 1, 128, layers=2, importance=importance, lm_head_w4a8=lm8, prefill=1, max_seq=64)
    _run_teacher_forced(torch_dev, m, steps=3)


def test_decode_empty_prefill_and_last_slot(torch_dev):
    # prefill 0: the first step attends to its own key only; the last steps fill the cache
    m = _model(torch_dev, 4, 2, 64, layers=2, prefill=0, max_seq=4)
    _run_teacher_forced(torch_dev, m, steps=4)
    with pytest.raises(ValueError):
        m.step()


def test_decode_graph_replay_matches_eager(torch_dev):
    torch = torch_dev
    m = _model(torch, 4, 2, 64, max_seq=96, prefill=40)
    n = 8
    m.start(9)
    toks, logits = [], []
    for _ in range(n):
        m.step()
        toks.append(int(m.token.item()))
        logits.append(m.logits.cpu().numpy().copy())
    m.start(9)
    m.capture()
    for r in range(n):
        m.generate(1)
        torch.cuda.synchronize()
        assert int(m.token.item()) == toks[r], r
        assert np.array_equal(m.logits.cpu().numpy(), logits[r]), r
    assert int(m.pos.item()) == 40 + n


def test_decode_multi_step_graph_matches_eager(torch_dev):
    """Graphs of several consecutive tokens (each step reads the token and position the
    previous one left on the device): 11 tokens as two 4-token replays and three 1-token
    replays give the eager tokens, logits, hidden state and position bit for bit."""
    torch = torch_dev
    m = _model(torch, 4, 2, 64, layers=2, max_seq=96, prefill=40)
    n = 11
    m.start(5)
    toks = []
    for _ in range(n):
        m.step()
        toks.append(int(m.token.item()))
    torch.cuda.synchronize()
    logits, hidden = m.logits.cpu().clone(), m.hidden.cpu().clone()
    m.start(5)
    m.capture(steps_per_graph=4)
    m.generate(4)
    torch.cuda.synchronize()
    assert int(m.token.item()) == toks[3] and int(m.pos.item()) == 44
    m.generate(n - 4)
    torch.cuda.synchronize()
    assert int(m.token.item()) == toks[-1]
    assert int(m.pos.item()) == 40 + n and m.length == 40 + n
    assert torch.equal(m.logits.cpu(), logits) and torch.equal(m.hidden.cpu(), hidden)


@pytest.mark.parametrize("split", ["2", "4", "8"])
def test_decode_graph_replay_split_attention(torch_dev, split, monkeypatch):
    """Key-split attention (partials merged in the o_proj staging) under HIP graph
    replay: every replayed token and its logits equal the eager sequence bit for bit,
    with tile counts per split that change as the position crosses tile edges."""
    torch = torch_dev
    monkeypatch.setenv("NVE_ATTN_SPLIT", split)
    m = _model(torch, 4, 2, 64, layers=2, max_seq=1100, prefill=1020)
    n = 6
    m.start(3)
    toks, logits = [], []
    for _ in range(n):
        m.step()
        toks.append(int(m.token.item()))
        logits.append(m.logits.cpu().numpy().copy())
    m.start(3)
    m.capture()
    for r in range(n):
        m.generate(1)
        torch.cuda.synchronize()
        assert int(m.token.item()) == toks[r], r
        assert np.array_equal(m.logits.cpu().numpy(), logits[r]), r


@pytest.mark.parametrize("fuse", ["1", "0"])
def test_decode_3b_shape_smoke(torch_dev, fuse, monkeypatch):
    """The Llama-3.2-3B shapes (head_dim 128, GQA 3, ffn 8192, vocab 128256) on 2 layers:
    one teacher-forced step against the oracle over the full logits, for the five
    launches and the unfused path."""
    monkeypatch.setenv("NVE_DECODE_FUSE", fuse)
    from nve_amd.decode import ModelShape, DecodeModel
    s = ModelShape(layers=2)
    m = DecodeModel(s, max_seq=130, prefill=128, importance=np.array([0.0, 1.0]))
    _run_teacher_forced(torch_dev, m, steps=1)


@pytest.mark.parametrize("split", ["1", "4", "8"])
def test_decode_long_cache(torch_dev, split, monkeypatch):
    """A cache of 8190+ keys: many tiles per workgroup (256 keys per tile at head_dim
    64 -> 32 tiles, 8 per split at 4 splits, 4 at 8), pos 8190..8192 crosses a tile
    edge."""
    monkeypatch.setenv("NVE_ATTN_SPLIT", split)
    m = _model(torch_dev, 4, 2, 64, layers=2, importance=(0.0, 1.0), max_seq=8256, prefill=8190)
    _run_teacher_forced(torch_dev, m, steps=3)


@pytest.mark.parametrize("tied", [True, False])
def test_decode_from_checkpoint(torch_dev, tmp_path, tied):
    """A Hugging Face Llama checkpoint (config.json + safetensors, bf16) loaded with
    load_safetensors_w4 drives the decode step: projections are the on-load Q4_0 of the
    stored matrices, norms and embeddings the stored bf16, the lm_head the Q4_0 of
    lm_head.weight or, tied, of the embeddings; the step matches the oracle."""
    import json
    from safetensors.torch import save_file
    from nve_amd import hip_kernels as hk
    from nve_amd.decode import DecodeModel, shape_from_hf_config
    from nve_amd.loader import load_safetensors_w4

    torch = torch_dev
    cfg = {"hidden_size": 256, "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
           "intermediate_size": 512, "vocab_size": 384, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
           "rope_scaling": {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                            "high_freq_factor": 4.0, "original_max_position_embeddings": 64}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    s = shape_from_hf_config(json.loads((tmp_path / "config.json").read_text()))
    assert (s.head_dim, s.kv_heads, s.rope_scaling.factor) == (64, 2, 8.0)
    g = torch.Generator().manual_seed(3)
    H, F, QD, KD = s.hidden, s.ffn, s.heads * s.head_dim, s.kv_heads * s.head_dim

    def mat(n, k):
        return (torch.randn((n, k), generator=g) * 0.05).to(torch.bfloat16)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": mat(s.vocab, H), "model.norm.weight": norm(H)}
    for i in range(s.layers):
        p = f"model.layers.{i}."
        t.update({p + "input_layernorm.weight": norm(H), p + "post_attention_layernorm.weight": norm(H),
                  p + "self_attn.q_proj.weight": mat(QD, H), p + "self_attn.k_proj.weight": mat(KD, H),
                  p + "self_attn.v_proj.weight": mat(KD, H), p + "self_attn.o_proj.weight": mat(H, QD),
                  p + "mlp.gate_proj.weight": mat(F, H), p + "mlp.up_proj.weight": mat(F, H),
                  p + "mlp.down_proj.weight": mat(H, F)})
    if not tied:
        t["lm_head.weight"] = mat(s.vocab, H)
    # two shards, as large checkpoints come
    names = sorted(t)
    save_file({n: t[n] for n in names[::2]}, str(tmp_path / "model-00001.safetensors"))
    save_file({n: t[n] for n in names[1::2]}, str(tmp_path / "model-00002.safetensors"))
    w = load_safetensors_w4([tmp_path / "model-00001.safetensors", tmp_path / "model-00002.safetensors"])
    m = DecodeModel(s, max_seq=48, prefill=20, importance=np.array([0.0, 1.0]), weights=w)

    nib, sc = hk.q4_quantize(t["model.layers.1.mlp.down_proj.weight"].cuda())
    assert torch.equal(m.layers[1]["down"][0], nib) and torch.equal(m.layers[1]["down"][1], sc)
    assert torch.equal(m.layers[0]["input_norm"].cpu(), t["model.layers.0.input_layernorm.weight"])
    assert torch.equal(m.embed.cpu(), t["model.embed_tokens.weight"])
    head = t["model.embed_tokens.weight" if tied else "lm_head.weight"]
    nib, sc = hk.q4_quantize(head.cuda())
    assert torch.equal(m.lm_head[0], nib) and torch.equal(m.lm_head[1], sc)
    _run_teacher_forced(torch, m, steps=3)



def test_decode_bench_model_sampled_layers(torch_dev):
    """The bench's own decode model (Llama-3.2-3B shapes, 28 layers with the seeded
    8 W4A16 / 20 W4A8 mask, W4A8 lm_head, 512 cached keys in a 1024-slot cache, four-way
    key-split attention): layers 0, 13 and 27 and the head teacher-forced against the
    oracle for two tokens, then the captured HIP graph replays the same two tokens bit
    for bit."""
    torch = torch_dev
    from nve_amd.decode import LLAMA_3_2_3B, DecodeModel
    m = DecodeModel(LLAMA_3_2_3B, max_seq=1024, prefill=512)
    assert sum(1 for u in m.use_w4a8 if not u) == 8
    checked = {0, 13, 27}
    print("bench model: layer precisions (1 = W4A8)", [m.use_w4a8[i] for i in sorted(checked)], flush=True)
    rec = []
    _run_teacher_forced(torch, m, steps=2, token0=1, checked=checked, record=rec)
    m.start(1)
    m.capture()
    for r in range(2):
        m.generate(1)
        torch.cuda.synchronize()
        assert int(m.token.item()) == rec[r][0], r
        assert np.array_equal(m.logits.cpu().numpy(), rec[r][1]), r


@pytest.mark.parametrize("lm8", [True, False])
def test_head_argmax_ties_nan_and_slices(torch_dev, lm8):
    """Greedy argmax of the head across all 128 partial workgroups (vocab 200000: every
    slice holds logits): among equal logits the lowest index wins, NaN never wins
    (src/ops.rs:485-495 keeps the first maximum), including ties that span slices."""
    torch = torch_dev
    vocab = 200_000
    m = _model(torch, 4, 2, 64, layers=1, vocab=vocab, lm_head_w4a8=lm8, prefill=4, max_seq=16)
    nib, sc = m.lm_head
    nb = sc.numel() // vocab
    sc0, nib0 = sc.clone(), nib.clone()

    def run():
        m.start(3)
        m.head()
        torch.cuda.synchronize()
        return int(m.token.item()), m.logits.cpu().numpy()

    # every logit 0: the first index
    sc.zero_()
    tok, lg = run()
    assert np.all(lg == 0.0) and tok == 0
    # NaN rows in front of the zeros: the first non-NaN row
    for k in (1, 5000, 150_001):
        sc.zero_()
        sc.view(vocab, nb)[:k] = float("nan")
        tok, lg = run()
        assert np.isnan(lg[:k]).all() and tok == k, (k, tok)
    # one row copied to later slices, everything else 0: the first maximum
    r0, copies = 70_000, (70_001, 140_000, 199_999)
    sc.zero_()
    sc.view(vocab, nb)[r0] = sc0.view(vocab, nb)[r0]
    rb = nib.numel() // vocab
    for r in copies:
        sc.view(vocab, nb)[r] = sc0.view(vocab, nb)[r0]
        nib.view(vocab, rb)[r] = nib0.view(vocab, rb)[r0]
    nib.view(vocab, rb)[r0] = nib0.view(vocab, rb)[r0]
    tok, lg = run()
    assert lg[r0] != 0.0 and all(lg[r] == lg[r0] for r in copies)
    expect = r0 if lg[r0] > 0 else 0
    assert tok == expect, (tok, expect, lg[r0])
    # a NaN among the copies changes nothing for the others
    sc.view(vocab, nb)[r0] = float("nan")
    tok, lg = run()
    assert tok == (copies[0] if lg[copies[0]] > 0 else 0), tok


@pytest.mark.parametrize("lm8", [True, False])
def test_head_with_caller_logits_and_more_rows_than_vocab(torch_dev, lm8):
    """A caller that passes its own logits buffer may hand the head an lm_head with more
    rows than the config's vocabulary (nve_decode_head): the W4A8 head then has more
    workgroups than the workspace has greedy-candidate slots and takes the launch over
    the logits instead.  Extra rows that copy rows 0..39 tie with them, so the token is
    the same as with the plain lm_head (the first maximum) and the copied logits equal
    the originals."""
    torch = torch_dev
    import ctypes as C
    from nve_amd._lib import DecodeHead, W4Weight, check, lib
    vocab, extra = 512, 40
    m = _model(torch, 4, 2, 64, layers=1, vocab=vocab, lm_head_w4a8=lm8, prefill=4, max_seq=16)
    nib, sc = m.lm_head
    H = m.shape.hidden
    nib2 = torch.cat([nib.view(vocab, -1), nib.view(vocab, -1)[:extra]]).contiguous()
    sc2 = torch.cat([sc.view(vocab, -1), sc.view(vocab, -1)[:extra]]).contiguous()
    logits2 = torch.full((vocab + extra,), float("nan"), dtype=torch.float32, device="cuda")
    tok2 = torch.zeros(1, dtype=torch.int32, device="cuda")
    for step in range(3):
        m.start(3 + step)
        m.head()
        torch.cuda.synchronize()
        tok, lg = int(m.token.item()), m.logits.cpu().numpy()
        m.start(3 + step)
        hd = DecodeHead(m.hidden.data_ptr(), m.final_norm.data_ptr(),
                        W4Weight(nib2.data_ptr(), sc2.data_ptr(), vocab + extra, H), m.embed.data_ptr(),
                        logits2.data_ptr(), tok2.data_ptr(), m.pos.data_ptr(), m.workspace.data_ptr())
        check("nve_hip_decode_head",
              lib().nve_hip_decode_head(C.byref(m.cfg), C.byref(hd), int(lm8), torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        lg2 = logits2.cpu().numpy()
        print(f"lm8={lm8} step {step}: token {tok} / {int(tok2.item())}", flush=True)
        assert np.array_equal(lg2[:vocab], lg) and np.array_equal(lg2[vocab:], lg[:extra])
        assert int(tok2.item()) == tok


def test_embed_token_clamped(torch_dev):
    """nve_hip_embed: the row of the token, bf16 -> fp32 exactly; a token outside
    [0, vocab) (read on the device) is clamped to the first / last row."""
    torch = torch_dev
    from nve_amd._lib import lib
    vocab, H = 37, 200
    emb = torch.randn((vocab, H), device="cuda").to(torch.bfloat16)
    hidden = torch.empty(H, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    for tok, row in ((5, 5), (vocab - 1, vocab - 1), (vocab + 9, vocab - 1), (-4, 0)):
        t = torch.tensor([tok], dtype=torch.int32, device="cuda")
        assert lib().nve_hip_embed(emb.data_ptr(), t.data_ptr(), hidden.data_ptr(), H, vocab, s) == 0
        torch.cuda.synchronize()
        assert torch.equal(hidden, emb[row].float()), (tok, row)
