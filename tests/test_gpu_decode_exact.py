"""Exact outputs of the decode step's fused launches, each driven on its own.

nve_hip_decode_stage issues one of the decode layer's fused launches exactly as
nve_hip_layer_forward_decode issues it (same kernel instantiation, arguments and
workspace); nve_hip_decode_head is the head itself.  Inputs are built so that every
fused producer yields known int8 codes (W4A8) or exact fp16 values (W4A16), and the
weight scales are powers of two, so each GEMV result is an exact fp32 number (the
argument of test_gpu_exact_acc.py).  Every epilogue then applies at most one or two
IEEE roundings, which numpy replays, so the outputs must match bit for bit:

  * RMSNorm producer (Q/K/V, gate/up, head): h = +-2^a, eps = 0 -> mean(h^2) = 4^a,
    1/sqrt = 2^-a exactly, so x = sign(h) * w_norm with w_norm integers in [-127, 127]
    and +-127 in every 32-group: the group scale is 1.0 and the codes are x itself.
  * RoPE pair + KV append (Q/K/V): cos / sin tables in {0, +-1} per column, so the
    rotation is exact; q = f32(rotated * qscale), the new key / value rows bf16(...).
  * attention-merge o_proj: partials with equal running maxima (weight 2^0 = 1) or
    empty (-inf, dropped), integer accumulators and l summing to a power of two, so the
    merged input is the chosen codes; residual: h_out = f32(h + y).
  * SwiGLU pair (gate/up): silu(g) = g where 1 + exp(-g) rounds to 1 (g >= 20) and -0
    where exp(-g) overflows (g <= -100); rows in between are not compared;
    out = f16(f32(silu(g) * up)).
  * down with its input quantized in the staging (W4A8) or read as fp16 (W4A16):
    codes * 2^e with +-127 per group; residual add as above.
  * head: final RMSNorm as above, lm_head logits (fp32) bit-exact, greedy token = first
    maximum, its embedding written to hidden, pos advanced.

A wrong accumulator, a row paired with the wrong partner, a block with the wrong scale,
a swapped cos / sin, a dropped split or a residual added twice changes some output.
Accumulators come from the oracle (orc_w4a8_block_acc)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIM = 1 << 24
QSCALE_NUM = np.float32(1.4426950408889634)


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nve_amd import _lib
    return torch, _lib, _lib.lib()


def _bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16(x):
    return (_bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def _codes(g, k, lo=1):
    """int codes in [-127, 127] with +-127 in every 32-group."""
    c = g.integers(-127, 128, size=k).astype(np.int64)
    if lo:
        c[c == 0] = 1
    pos = g.integers(0, 32, size=k // 32)
    c[32 * np.arange(k // 32) + pos] = np.where(g.random(k // 32) < 0.5, -127, 127)
    return c


def _w4(g, n, k, lo, hi):
    nib = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    ws = np.ldexp(np.float32(1.0), g.integers(lo, hi + 1, size=(n, k // 32))).astype(np.float32)
    return nib, ws


def _exact(orc, codes, nib, ws, n, k, xs_exp=None):
    """Exact y[n] = sum_b ws[n,b] * 2^xs_exp[b] * acc[n,b] (asserting fp32 exactness)."""
    acc = orc.w4a8_block_acc(codes.astype(np.int8), nib, n, k).astype(np.int64)
    sc = ws.astype(np.float64)
    if xs_exp is not None:
        sc = sc * np.ldexp(1.0, xs_exp)[None, :]
    e_min = np.floor(np.log2(sc.min()))
    c = np.rint(sc / 2.0 ** e_min).astype(np.int64)
    assert np.all(c * 2.0 ** e_min == sc)
    t = c * acc
    assert int(np.abs(t).sum(axis=1).max()) < LIM, "test precondition: exact fp32 sums"
    y = t.sum(axis=1).astype(np.float64) * 2.0 ** e_min
    assert np.all(y.astype(np.float32).astype(np.float64) == y)
    return y.astype(np.float32)


class Layer:
    """One decode layer's buffers on the device, with exact-friendly contents."""

    def __init__(self, torch, L, orc, H, heads, kv, D, F, max_seq, seed, vocab=0):
        self.torch, self.L = torch, L
        g = np.random.default_rng(seed)
        self.g = g
        self.H, self.heads, self.kv, self.D, self.F, self.S = H, heads, kv, D, F, max_seq
        QD, KD = heads * D, kv * D
        self.QD, self.KD = QD, KD
        from nve_amd._lib import DecodeConfig
        self.cfg = DecodeConfig(H, heads, kv, D, F, max_seq, vocab, 0.0)
        sp = lambda k: 2 if k <= 4096 else (1 if k <= 8192 else 0)  # noqa: E731
        self.mats = {
            "q": _w4(g, QD, H, -9, -9 + sp(H)), "k": _w4(g, KD, H, -9, -9 + sp(H)), "v": _w4(g, KD, H, -9, -9 + sp(H)),
            "o": _w4(g, H, QD, -9, -9 + sp(QD)),
            # gate large (|g| mostly far from 0), up small (product within fp16)
            "gate": _w4(g, F, H, -4 - sp(H) // 2, -4), "up": _w4(g, F, H, -10, -10 + sp(H) // 2),
            "down": _w4(g, H, F, -9, -9 + sp(F)),
        }
        self.dev = {nm: (self.up(nib), self.up(ws)) for nm, (nib, ws) in self.mats.items()}
        self.wn1 = _codes(g, H)
        self.wn2 = _codes(g, H)
        self.dn1 = self.up(_bf16_bits(self.wn1.astype(np.float32)))
        self.dn2 = self.up(_bf16_bits(self.wn2.astype(np.float32)))
        self.kc = torch.zeros((kv, max_seq, D), dtype=torch.bfloat16, device="cuda")
        self.vc = torch.zeros((kv, max_seq, D), dtype=torch.bfloat16, device="cuda")
        self.hid = torch.zeros(H, dtype=torch.float32, device="cuda")
        self.pos = torch.zeros(1, dtype=torch.int32, device="cuda")
        half = D // 2
        # per-column rotation (cos, sin) in {(1,0), (0,1), (-1,0), (0,-1)} at every position
        rot = g.integers(0, 4, size=half)
        cs = np.array([[1, 0], [0, 1], [-1, 0], [0, -1]], np.float32)[rot]
        self.cos_np = np.tile(cs[:, 0], (max_seq, 1)).astype(np.float32)
        self.sin_np = np.tile(cs[:, 1], (max_seq, 1)).astype(np.float32)
        self.cos, self.sin = self.up(self.cos_np), self.up(self.sin_np)
        ws_bytes = L.nve_hip_decode_workspace_bytes(C.byref(self.cfg))
        self.ws = torch.empty(ws_bytes + 256, dtype=torch.uint8, device="cuda")
        from nve_amd._lib import W4Weight, LayerWeights, DecodeIO
        wt = {nm: W4Weight(self.dev[nm][0].data_ptr(), self.dev[nm][1].data_ptr(), n, k)
              for nm, n, k in (("q", QD, H), ("k", KD, H), ("v", KD, H), ("o", H, QD), ("gate", F, H), ("up", F, H),
                               ("down", H, F))}
        self.w = LayerWeights(self.dn1.data_ptr(), self.dn2.data_ptr(), *[wt[nm] for nm in
                                                                          ("q", "k", "v", "o", "gate", "up", "down")])
        wsp = (self.ws.data_ptr() + 255) // 256 * 256
        self.io = DecodeIO(self.hid.data_ptr(), self.kc.data_ptr(), self.vc.data_ptr(), self.pos.data_ptr(),
                           self.cos.data_ptr(), self.sin.data_ptr(), wsp)

    def up(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def norm_hidden(self, a=3):
        """h = +-2^a: mean(h^2) = 4^a, so RMSNorm with eps = 0 scales by 2^-a exactly."""
        sgn = np.where(self.g.random(self.H) < 0.5, -1.0, 1.0).astype(np.float32)
        h = (sgn * np.float32(2.0 ** a)).astype(np.float32)
        self.hid.copy_(self.up(h))
        return sgn.astype(np.int64)

    def stage(self, w4a8, stage, inp=None, out=None):
        st = self.L.nve_hip_decode_stage(C.byref(self.cfg), C.byref(self.w), C.byref(self.io), int(w4a8), stage,
                                         inp.data_ptr() if inp is not None else None,
                                         out.data_ptr() if out is not None else None,
                                         self.torch.cuda.current_stream().cuda_stream)
        assert st == 0, st
        self.torch.cuda.synchronize()


SHAPES = [  # H, heads, kv, D, F, max_seq
    (256, 4, 2, 64, 512, 600),
    (1024, 8, 2, 128, 2816, 1100),
    (3072, 24, 8, 128, 8192, 1024),
]


@pytest.mark.parametrize("w4a8", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_stage_qkv_rope_kv_append(orc, env, shape, w4a8):
    torch, _lib, L = env
    H, heads, kv, D, F, S = shape
    print(f"exact decode stage QKV shape={shape} w4a8={w4a8}", flush=True)
    ly = Layer(torch, L, orc, H, heads, kv, D, F, S, seed=H + 7 * w4a8)
    codes = ly.norm_hidden() * ly.wn1
    pos = S - 5
    ly.pos.fill_(pos)
    q = torch.full((ly.QD,), float("nan"), dtype=torch.float32, device="cuda")
    kc0, vc0 = ly.kc.clone(), ly.vc.clone()
    ly.stage(w4a8, _lib.STAGE_QKV, out=q)
    y = {nm: _exact(orc, codes, *ly.mats[nm], n, H) for nm, n in (("q", ly.QD), ("k", ly.KD), ("v", ly.KD))}
    half = D // 2
    c, s = ly.cos_np[pos], ly.sin_np[pos]
    qs = np.float32(QSCALE_NUM / np.sqrt(np.float32(D)))

    def rot(v):
        v = v.reshape(-1, D)
        x0, x1 = v[:, :half], v[:, half:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=1).astype(np.float32)

    q_ref = (rot(y["q"]) * qs).astype(np.float32).reshape(-1)
    got = q.cpu().numpy()
    assert np.array_equal(got, q_ref), int(np.sum(got != q_ref))
    k_ref = _bf16_bits(rot(y["k"]))
    v_ref = _bf16_bits(y["v"].reshape(-1, D))
    kg = ly.kc.view(torch.int16).cpu().numpy().view(np.uint16)
    vg = ly.vc.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(kg[:, pos], k_ref) and np.array_equal(vg[:, pos], v_ref)
    # nothing else in the caches moved
    mask = np.ones(S, bool)
    mask[pos] = False
    assert torch.equal(ly.kc[:, torch.from_numpy(mask).cuda()], kc0[:, torch.from_numpy(mask).cuda()])
    assert torch.equal(ly.vc[:, torch.from_numpy(mask).cuda()], vc0[:, torch.from_numpy(mask).cuda()])


@pytest.mark.parametrize("split", ["2", "4", "8"])
@pytest.mark.parametrize("w4a8", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_stage_o_proj_merge_residual(orc, env, shape, w4a8, split, monkeypatch):
    torch, _lib, L = env
    H, heads, kv, D, F, S = shape
    monkeypatch.setenv("NVE_ATTN_SPLIT", split)
    print(f"exact decode stage O_MERGE shape={shape} w4a8={w4a8} split={split}", flush=True)
    ly = Layer(torch, L, orc, H, heads, kv, D, F, S, seed=3 * H + int(split) + 11 * w4a8)
    sp = L.nve_hip_decode_attn_splits(C.byref(ly.cfg))
    assert sp == min(int(split), 8 if heads * D <= 4096 else 4)
    g = ly.g
    QD = ly.QD
    codes = np.concatenate([_codes(g, 32, lo=0) for _ in range(QD // 32)])
    part = np.zeros((sp, heads, D + 4), np.float32)
    for hd in range(heads):
        active = g.random(sp) < 0.6
        active[g.integers(0, sp)] = True
        act = np.flatnonzero(active)
        j = int(g.integers(0, 4))
        L_tot = 2 ** j
        # l: positive integers summing to 2^j when there are enough units, else a 2^j on one split
        ls = np.zeros(sp, np.float32)
        if len(act) <= L_tot:
            cuts = np.sort(g.choice(np.arange(1, L_tot), size=len(act) - 1, replace=False)) if len(act) > 1 else []
            ls[act] = np.diff(np.concatenate([[0], cuts, [L_tot]]))
        else:
            ls[act[0]] = L_tot
        tgt = codes[hd * D:(hd + 1) * D] * L_tot
        accs = np.zeros((sp, D), np.int64)
        rest = tgt.copy()
        for a in act[:-1]:
            accs[a] = g.integers(-300, 301, size=D)
            rest -= accs[a]
        accs[act[-1]] = rest
        for s_ in range(sp):
            if active[s_]:
                part[s_, hd, 0] = 0.0
                part[s_, hd, 1] = ls[s_]
                part[s_, hd, 4:] = accs[s_]
            else:
                part[s_, hd, 0] = -np.inf
    h0 = (g.standard_normal(H) * 4).astype(np.float32)
    ly.hid.copy_(ly.up(h0))
    ly.stage(w4a8, _lib.STAGE_O_MERGE, inp=ly.up(part))
    y = _exact(orc, codes, *ly.mats["o"], H, QD)
    ref = (h0 + y).astype(np.float32)
    got = ly.hid.cpu().numpy()
    assert np.array_equal(got, ref), int(np.sum(got != ref))


@pytest.mark.parametrize("w4a8", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_stage_gate_up_swiglu(orc, env, shape, w4a8):
    torch, _lib, L = env
    H, heads, kv, D, F, S = shape
    print(f"exact decode stage GATE_UP shape={shape} w4a8={w4a8}", flush=True)
    ly = Layer(torch, L, orc, H, heads, kv, D, F, S, seed=5 * H + w4a8)
    codes = ly.norm_hidden(a=-2) * ly.wn2
    out = torch.full((F,), float("nan"), dtype=torch.float16, device="cuda")
    ly.stage(w4a8, _lib.STAGE_GATE_UP, out=out)
    gy = _exact(orc, codes, *ly.mats["gate"], F, H)
    uy = _exact(orc, codes, *ly.mats["up"], F, H)
    got = out.cpu().numpy()
    pos_rows, neg_rows = gy >= 20, gy <= -100
    assert (pos_rows | neg_rows).mean() > 0.8, "test precondition: most gate rows far from zero"
    ref_pos = (gy * uy).astype(np.float32).astype(np.float16)
    assert np.array_equal(got[pos_rows].view(np.uint16), ref_pos[pos_rows].view(np.uint16))
    assert np.all(got[neg_rows] == 0)
    # the rows in between: silu(g) * up within fp16 rounding of the f64 value
    mid = ~(pos_rows | neg_rows)
    gm = gy[mid].astype(np.float64)
    r = gm / (1 + np.exp(-gm)) * uy[mid]
    assert np.all(np.abs(got[mid].astype(np.float64) - r) <= 2e-3 * np.abs(r) + 1e-6)


@pytest.mark.parametrize("w4a8", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_stage_down_residual(orc, env, shape, w4a8):
    torch, _lib, L = env
    H, heads, kv, D, F, S = shape
    print(f"exact decode stage DOWN shape={shape} w4a8={w4a8}", flush=True)
    ly = Layer(torch, L, orc, H, heads, kv, D, F, S, seed=9 * H + w4a8)
    g = ly.g
    codes = _codes(g, F, lo=0)
    e = g.integers(-4, -2, size=F // 32)
    x16 = (codes.astype(np.float64) * np.ldexp(1.0, np.repeat(e, 32))).astype(np.float16)
    assert np.all(x16.astype(np.float64) == codes * np.ldexp(1.0, np.repeat(e, 32)))
    h0 = (g.standard_normal(H) * 4).astype(np.float32)
    ly.hid.copy_(ly.up(h0))
    ly.stage(w4a8, _lib.STAGE_DOWN, inp=ly.up(x16))
    y = _exact(orc, codes, *ly.mats["down"], H, F, xs_exp=e)
    ref = (h0 + y).astype(np.float32)
    got = ly.hid.cpu().numpy()
    assert np.array_equal(got, ref), int(np.sum(got != ref))


@pytest.mark.parametrize("w4a8", [True, False])
@pytest.mark.parametrize("H,vocab", [(256, 1000), (3072, 128256)])
def test_head_logits_and_token_exact(orc, env, H, vocab, w4a8):
    torch, _lib, L = env
    print(f"exact decode head H={H} vocab={vocab} w4a8={w4a8}", flush=True)
    from nve_amd._lib import DecodeConfig, DecodeHead, W4Weight
    cfg = DecodeConfig(H, 4, 2, 64, 512, 64, vocab, 0.0)
    g = np.random.default_rng(H + vocab + w4a8)
    nib, ws = _w4(g, vocab, H, -9, -9 + (2 if H <= 4096 else 1))
    wn = _codes(g, H)
    sgn = np.where(g.random(H) < 0.5, -1, 1).astype(np.int64)
    codes = sgn * wn
    h = (sgn * 2.0 ** 5).astype(np.float32)
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    d_nib, d_ws, d_wn = up(nib), up(ws), up(_bf16_bits(wn.astype(np.float32)))
    emb = up(g.integers(0, 1 << 16, size=(vocab, H), dtype=np.uint16) & 0x7F7F)  # finite bf16
    hid = up(h)
    logits = torch.full((vocab,), float("nan"), dtype=torch.float32, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    pos = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    wsb = torch.empty(L.nve_hip_decode_workspace_bytes(C.byref(cfg)) + 256, dtype=torch.uint8, device="cuda")
    hd = DecodeHead(hid.data_ptr(), d_wn.data_ptr(), W4Weight(d_nib.data_ptr(), d_ws.data_ptr(), vocab, H),
                    emb.data_ptr(), logits.data_ptr(), tok.data_ptr(), pos.data_ptr(),
                    (wsb.data_ptr() + 255) // 256 * 256)
    assert L.nve_hip_decode_head(C.byref(cfg), C.byref(hd), int(w4a8), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    y = _exact(orc, codes, nib, ws, vocab, H)
    got = logits.cpu().numpy()
    assert np.array_equal(got, y), int(np.sum(got != y))
    t = int(np.argmax(y))
    assert int(tok.item()) == t
    e = emb.cpu().numpy()[t].astype(np.uint32) << 16
    assert np.array_equal(hid.cpu().numpy(), e.view(np.float32))
    assert int(pos.item()) == 8
