"""The reference's alignment contract at the drop-in launchers.

The reference kernels load nibbles two bytes (W4A8, get_int_b2,
cuda/nve_kernels.cu:789-794) or one byte at a time (W4A16 and dequant, 330-433), the
int8 activations four bytes at a time (829-832) and 16-bit vectors per element, so a
Rust caller may pass views at such offsets (device_ptr + start_offset,
src/cuda_kernels.rs:300-339).  Every case here places buffers at +1 / +2 / +4 / +8
bytes from a 256-byte-aligned allocation and checks the results against the oracle
with the same bars as the aligned tests (bit-exact for the quantizer, the dequant and
the W4A8 accumulators, 1e-3 / 2e-3 for the scaled outputs), and against the aligned
call where both must agree bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import activations, rel_err_floor, to_f16, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from nve_amd import hip_kernels as hk
    from nve_amd._lib import lib
    return torch, hk, lib()


class Placed:
    """A host array copied to device memory at byte offset `off` of a fresh allocation."""

    def __init__(self, torch, a: np.ndarray, off: int):
        raw = np.ascontiguousarray(a).view(np.uint8).ravel()
        self.buf = torch.zeros(raw.size + off + 64, dtype=torch.uint8, device="cuda")
        self.buf[off:off + raw.size] = torch.from_numpy(raw).cuda()
        self.off, self.nbytes, self.dtype, self.shape = off, raw.size, a.dtype, a.shape
        assert self.buf.data_ptr() % 256 == 0

    @property
    def ptr(self) -> int:
        return self.buf.data_ptr() + self.off

    def get(self) -> np.ndarray:
        return self.buf[self.off:self.off + self.nbytes].cpu().numpy().view(self.dtype).reshape(self.shape)


def _stream(torch):
    return torch.cuda.current_stream().cuda_stream


def _problem(orc, n, k, seed):
    data = orc.q4_from_f32(weights(n, k, seed=seed))
    return orc.extract_for_gpu(data, n, k)


@pytest.mark.parametrize("x_off,xq_off", [(2, 0), (0, 1), (6, 3), (2, 4)])
def test_quantize_f16_q8_offsets(orc, env, x_off, xq_off):
    torch, hk, L = env
    k = 4096
    x = to_f16(activations(k, seed=5))
    px = Placed(torch, x.astype(np.float16), x_off)
    pq = Placed(torch, np.zeros(k, np.int8), xq_off)
    ps = Placed(torch, np.zeros(k // 32, np.float32), 0)
    L.nve_quantize_f16_q8(px.ptr, pq.ptr, ps.ptr, k, _stream(torch))
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    q_ref, s_ref = orc.quantize_q8_group(x)
    assert np.array_equal(pq.get(), q_ref) and np.array_equal(ps.get(), s_ref)


@pytest.mark.parametrize("nib_off,xq_off,out_off", [(2, 0, 0), (0, 4, 0), (2, 4, 2), (14, 12, 6), (8, 8, 0)])
@pytest.mark.parametrize("n,k", [(300, 4096), (4096, 4096), (37, 160)])
def test_matvec_w4a8_offsets(orc, env, nib_off, xq_off, out_off, n, k):
    torch, hk, L = env
    print(f"align w4a8 n={n} k={k} offs={nib_off},{xq_off},{out_off}", flush=True)
    nib, ws = _problem(orc, n, k, seed=n + k)
    x = to_f16(activations(k, seed=k))
    xq, xs = orc.quantize_q8_group(x)
    pn, pq = Placed(torch, nib, nib_off), Placed(torch, xq, xq_off)
    tws, txs = torch.from_numpy(ws).cuda(), torch.from_numpy(xs).cuda()
    # fp32 twin: the accumulators through the bar; the void drop-in: fp16 output
    p32 = Placed(torch, np.zeros(n, np.float32), 4 * (out_off // 4))
    assert L.nve_hip_matvec_w4a8(pq.ptr, txs.data_ptr(), pn.ptr, tws.data_ptr(), p32.ptr, 2, n, k,
                                 _stream(torch)) == 0
    p16 = Placed(torch, np.zeros(n, np.float16), out_off)
    L.nve_matvec_w4a8(pq.ptr, txs.data_ptr(), pn.ptr, tws.data_ptr(), p16.ptr, n, k, _stream(torch))
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    ref = orc.matvec_w4a8_f64(xq, xs, nib, ws, n, k)
    assert rel_err_floor(p32.get(), ref) <= 1e-3
    assert np.array_equal(p16.get(), p32.get().astype(np.float16))


def test_matvec_w4a8_offsets_exact(orc, env):
    """Power-of-two scales: the misaligned path's fp32 output equals the exact integer
    sum (see test_gpu_exact_acc.py) and the aligned kernel's output bit for bit."""
    torch, hk, L = env
    from test_gpu_exact_acc import _acts, _expected, _weights
    n, k = 1024, 4096
    nib, ws = _weights(n, k, seed=3, ws_spread=2)
    xq, e = _acts(k, seed=4)
    xs = np.ldexp(np.float32(1.0), e[0]).astype(np.float32)
    ref = _expected(orc, xq[0], xs, nib, ws, n, k)
    pn, pq = Placed(torch, nib, 2), Placed(torch, xq[0], 4)
    tws, txs = torch.from_numpy(ws).cuda(), torch.from_numpy(xs).cuda()
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    assert L.nve_hip_matvec_w4a8(pq.ptr, txs.data_ptr(), pn.ptr, tws.data_ptr(), out.data_ptr(), 2, n, k,
                                 _stream(torch)) == 0
    aligned = hk.matvec_w4a8(torch.from_numpy(xq[0]).cuda(), txs, torch.from_numpy(nib).cuda(), tws, n, k,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert torch.equal(out, aligned[0])


@pytest.mark.parametrize("nib_off,x_off,awq_off,out_off", [(1, 0, 0, 0), (0, 2, 0, 0), (0, 0, 4, 2), (3, 6, 12, 2),
                                                           (2, 2, None, 0)])
@pytest.mark.parametrize("n,k", [(300, 4096), (37, 160)])
def test_matvec_w4a16_offsets(orc, env, nib_off, x_off, awq_off, out_off, n, k):
    torch, hk, L = env
    print(f"align w4a16 n={n} k={k} offs={nib_off},{x_off},{awq_off},{out_off}", flush=True)
    nib, sc = _problem(orc, n, k, seed=2 * n + k)
    x = to_f16(activations(k, seed=k + 9))
    awq = None if awq_off is None else (np.random.default_rng(1).uniform(0.5, 2.0, k).astype(np.float32))
    pn, px = Placed(torch, nib, nib_off), Placed(torch, x.astype(np.float16), x_off)
    pa = None if awq is None else Placed(torch, awq, awq_off)
    tsc = torch.from_numpy(sc).cuda()
    p16 = Placed(torch, np.zeros(n, np.float16), out_off)
    L.nve_matvec_w4a16(px.ptr, pn.ptr, tsc.data_ptr(), None if pa is None else pa.ptr, p16.ptr, n, k, _stream(torch))
    p32 = Placed(torch, np.zeros(n, np.float32), 0)
    assert L.nve_hip_matvec_w4a16(px.ptr, 0, pn.ptr, tsc.data_ptr(), None if pa is None else pa.ptr, p32.ptr, 2, n, k,
                                  _stream(torch)) == 0
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    ref = orc.matvec_w4a16_f64(x, nib, sc, n, k, awq=awq)
    assert rel_err_floor(p32.get(), ref) <= 2e-3
    assert np.array_equal(p16.get(), p32.get().astype(np.float16))


def test_qkv_matvec_w4a16_offsets(orc, env):
    """The fused Q/K/V drop-in with one misaligned projection (every matrix checked)."""
    torch, hk, L = env
    k = 2048
    ns = (2048, 512, 512)
    x = to_f16(activations(k, seed=77))
    px = Placed(torch, x.astype(np.float16), 2)
    probs = [_problem(orc, n, k, seed=100 + n + i) for i, n in enumerate(ns)]
    pn = [Placed(torch, p[0], off) for p, off in zip(probs, (0, 1, 0))]
    ts = [torch.from_numpy(p[1]).cuda() for p in probs]
    outs = [Placed(torch, np.zeros(n, np.float16), 2) for n in ns]
    L.nve_qkv_matvec_w4a16(px.ptr, pn[0].ptr, ts[0].data_ptr(), None, ns[0], pn[1].ptr, ts[1].data_ptr(), None, ns[1],
                           pn[2].ptr, ts[2].data_ptr(), None, ns[2], outs[0].ptr, outs[1].ptr, outs[2].ptr, k,
                           _stream(torch))
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    for (nib, sc), o, n in zip(probs, outs, ns):
        ref = orc.matvec_w4a16_f64(x, nib, sc, n, k)
        assert rel_err_floor(o.get().astype(np.float32), ref) <= 2e-3 + 2 ** -11  # fp16 output rounding


@pytest.mark.parametrize("nib_off,out_off,awq_off", [(1, 0, None), (0, 2, None), (5, 6, 4), (0, 0, 8)])
def test_dequant_w4a16_offsets(orc, env, nib_off, out_off, awq_off):
    """Misaligned dequant: bit-identical to the aligned kernel (which matches the
    reference's to_f32_vec rounding, test_gpu_gemm.py)."""
    torch, hk, L = env
    n, k = 96, 1024
    nib, sc = _problem(orc, n, k, seed=8)
    awq = None if awq_off is None else np.random.default_rng(2).uniform(0.5, 2.0, k).astype(np.float32)
    pn = Placed(torch, nib, nib_off)
    pa = None if awq is None else Placed(torch, awq, awq_off)
    po = Placed(torch, np.zeros((n, k), np.float16), out_off)
    tsc = torch.from_numpy(sc).cuda()
    L.nve_dequant_w4a16(pn.ptr, tsc.data_ptr(), None if pa is None else pa.ptr, po.ptr, n, k, _stream(torch))
    ref = hk.dequant_w4(torch.from_numpy(nib).cuda(), tsc, n, k,
                        awq=None if awq is None else torch.from_numpy(awq).cuda())
    torch.cuda.synchronize()
    assert L.nve_hip_last_status() == 0
    assert np.array_equal(po.get().view(np.uint16), ref.cpu().numpy().view(np.uint16))
