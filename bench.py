#!/usr/bin/env python3
"""Benchmark of the MI355X quantized decode GEMV path (W4A8 / W4A16).

Workload: the Llama-3.1-8B layer-shape suite at batch 1 --
q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096, down 4096x14336,
lm_head 128256x4096 -- in W4A8 (fp16 activations quantized per 32-group to int8 by
nve_quantize_f16_q8, int8 x int4 on v_dot4) and in W4A16 (bf16 activations).
Weights: N(0, 0.02) from a seeded generator, int4 group-quantized on the device by
the library's Q4_0 quantizer (src/quantize.rs:711-731 semantics).  Activations:
N(0,1) with 0.5% of channels at +-20 sigma.

One step = one pass over the suite in both precisions (W4A8: 5 GEMV launches,
Q/K/V and gate/up each as one grouped launch, the K = 4096 ones quantizing their
fp16 input in-kernel and down after one separate quantization launch; W4A16: 5 GEMV
launches), captured as HIP graphs of four consecutive steps (plus one-step graphs for a
remainder, so exactly K steps run); consecutive steps use different weight copies
(>= 1 GB in rotation), so the 256 MB MALL cannot serve the weights and every byte comes
from HBM.

value = algorithmic bytes of one step / measured step time (GB/s), with the
algorithmic bytes of a GEMV = N*K/2 (nibbles) + N*K/32*4 (f32 scales) + activation
bytes (W4A8: K + K/32*4, W4A16: 2K) + output bytes.

The roofline object reports the dominant kernel of the step: the lm_head launches
(128256x4096, fp32 logits), which take more than half of the step.  Both lm_head
launches of the step are timed with the step's own entry points and arguments (so the
same kernel instantiations: the W4A8 GEMV that quantizes its fp16 input in-kernel,
nve_hip_matvec_w4a8_x, and the W4A16 GEMV on bf16 activations), each on its own in a
graph of back-to-back launches over rotating weight copies, with HIP events on the
stream the graph is replayed on; `roofline` is the slower of the two and
`roofline_other` the other.  cpu_baseline times the reference's CPU quantized GEMV
(QuantizedTensor::matvec_f32 + q4_dot_row_avx2, restated in oracle/) on every host
core this process may run on (os.sched_getaffinity, as rayon's default pool) over a
bounded sample.

Also in the line (measured beside the step, not part of `value`): every suite shape
timed on its own (graphs of 200 back-to-back launches over 8 weight copies; GB/s and
GEMV/s), the same table at the Llama-3.2-1B shapes, the batched
W4A8 sweep, the 3B decode step and the prefill GEMM.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W4A8/W4A16 GEMV GB/s & % HBM peak at 8B shapes; decode tok/s (1 GPU)"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16

SUITE_8B = [  # name, N, K
    ("q_proj", 4096, 4096),
    ("k_proj", 1024, 4096),
    ("v_proj", 1024, 4096),
    ("o_proj", 4096, 4096),
    ("gate_proj", 14336, 4096),
    ("up_proj", 14336, 4096),
    ("down_proj", 4096, 14336),
    ("lm_head", 128256, 4096),
]

SUITE_1B = [  # BASELINE config 2 (Llama-3.2-1B layer shapes); reported beside the 8B suite
    ("q_proj", 2048, 2048),
    ("k_proj", 512, 2048),
    ("v_proj", 512, 2048),
    ("o_proj", 2048, 2048),
    ("gate_proj", 8192, 2048),
    ("up_proj", 8192, 2048),
    ("down_proj", 2048, 8192),
]


def weight_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * (k // 32) * 4


def gemv_bytes(n: int, k: int, prec: str, out_bytes: int) -> int:
    act = (k + (k // 32) * 4) if prec == "w4a8" else 2 * k
    return weight_bytes(n, k) + act + n * out_bytes


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
def make_inputs(torch, hk, copies_layer: int, copies_head: int, seed: int = 0x4E5645, suite=SUITE_8B):
    """Quantized weight copies for every suite shape (device-side generation)."""
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(seed)
    weights = {}
    for name, n, k in suite:
        c = copies_head if name == "lm_head" else copies_layer
        sets = []
        for _ in range(c):
            w = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32).mul_(0.02)
            nib, sc = hk.q4_quantize(w)
            del w
            sets.append((nib, sc))
        weights[name] = sets
    torch.cuda.synchronize()
    return weights


def make_activation(torch, k: int, seed: int):
    import numpy as np
    r = np.random.default_rng(seed)
    x = r.standard_normal(k).astype(np.float32)
    idx = r.choice(k, size=max(1, round(0.005 * k)), replace=False)
    x[idx] = np.where(r.random(idx.size) < 0.5, -20.0, 20.0)
    return torch.from_numpy(x).cuda()


class Step:
    """One pass over the suite in both precisions on weight copy `ci`, as raw C-ABI
    launches into preallocated buffers (capturable)."""

    def __init__(self, torch, lib, weights, acts):
        self.t = torch
        self.L = lib
        self.w = weights
        self.acts = acts
        dev = "cuda"
        self.bufs = {}
        for name, n, k in SUITE_8B:
            odt = torch.float32 if name == "lm_head" else torch.float16
            self.bufs[name] = (torch.empty(n, dtype=odt, device=dev),
                               torch.empty(n, dtype=torch.float32 if name == "lm_head" else torch.bfloat16,
                                           device=dev))
        self.xq = {k: (torch.empty(k, dtype=torch.int8, device=dev), torch.empty(k // 32, dtype=torch.float32,
                                                                                  device=dev))
                   for k in (4096, 14336)}

    def _quant(self, x16, k, s):
        xq, xs = self.xq[k]
        st = self.L.nve_hip_quantize_q8(x16.data_ptr(), 0, 1, k, xq.data_ptr(), xs.data_ptr(), s)
        assert st == 0, st
        return xq, xs

    def w4a8(self, name, ci, xq, xs, s):
        n, k = [(n, k) for nm, n, k in SUITE_8B if nm == name][0]
        nib, sc = self.w[name][ci % len(self.w[name])]
        out = self.bufs[name][0]
        odt = 2 if out.dtype == self.t.float32 else 0
        st = self.L.nve_hip_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), nib.data_ptr(), sc.data_ptr(),
                                        out.data_ptr(), odt, n, k, s)
        assert st == 0, st

    def w4a8_x(self, name, ci, x16, s):
        """W4A8 GEMV that quantizes its fp16 activations itself (one launch)."""
        n, k = [(n, k) for nm, n, k in SUITE_8B if nm == name][0]
        nib, sc = self.w[name][ci % len(self.w[name])]
        out = self.bufs[name][0]
        odt = 2 if out.dtype == self.t.float32 else 0
        st = self.L.nve_hip_matvec_w4a8_x(x16.data_ptr(), 0, nib.data_ptr(), sc.data_ptr(), out.data_ptr(), odt, n, k,
                                          s)
        assert st == 0, st

    def w4a16(self, name, ci, xb, s):
        n, k = [(n, k) for nm, n, k in SUITE_8B if nm == name][0]
        nib, sc = self.w[name][ci % len(self.w[name])]
        out = self.bufs[name][1]
        odt = 2 if out.dtype == self.t.float32 else 1
        st = self.L.nve_hip_matvec_w4a16(xb.data_ptr(), 1, nib.data_ptr(), sc.data_ptr(), None, out.data_ptr(),
                                         odt, n, k, s)
        assert st == 0, st

    def grouped(self, prec, names, ci, x, xs, s):
        from nve_amd._lib import W4Mat
        k = [kk for nm, _, kk in SUITE_8B if nm == names[0]][0]
        arr = (W4Mat * len(names))()
        for i, name in enumerate(names):
            n = [nn for nm, nn, _ in SUITE_8B if nm == name][0]
            nib, sc = self.w[name][ci % len(self.w[name])]
            out = self.bufs[name][1 if prec == "w4a16" else 0]
            arr[i] = W4Mat(nib.data_ptr(), sc.data_ptr(), None, out.data_ptr(), n)
        if prec == "w4a8x":
            st = self.L.nve_hip_grouped_matvec_w4a8_x(x.data_ptr(), 0, arr, len(names), 0, k, s)
        elif prec == "w4a8":
            st = self.L.nve_hip_grouped_matvec_w4a8(x.data_ptr(), xs.data_ptr(), arr, len(names), 0, k, s)
        else:
            st = self.L.nve_hip_grouped_matvec_w4a16(x.data_ptr(), 1, arr, len(names), 1, k, s)
        assert st == 0, st

    def run(self, ci):
        s = self.t.cuda.current_stream().cuda_stream
        a = self.acts
        # W4A8: the reference quantizes once for q/k/v (src/gpu_layer.rs:658-661),
        # re-quantizes for o, once for gate/up, again for down, and for the lm_head
        # input.  Here the K = 4096 launches quantize their fp16 input inside the GEMV
        # (nve_hip_*matvec_w4a8_x, bit-identical; q/k/v and gate/up grouped); down
        # (K = 14336, where a per-workgroup quantization reads 28 KB of L2 per workgroup)
        # keeps the separate quantization launch.
        self.grouped("w4a8x", ("q_proj", "k_proj", "v_proj"), ci, a["h16"], None, s)
        self.w4a8_x("o_proj", ci, a["attn16"], s)
        self.grouped("w4a8x", ("gate_proj", "up_proj"), ci, a["h216"], None, s)
        xq, xs = self._quant(a["mid16"], 14336, s)
        self.w4a8("down_proj", ci, xq, xs, s)
        self.w4a8_x("lm_head", ci, a["final16"], s)
        # W4A16 (bf16 activations)
        self.grouped("w4a16", ("q_proj", "k_proj", "v_proj"), ci, a["hb"], None, s)
        self.w4a16("o_proj", ci, a["attnb"], s)
        self.grouped("w4a16", ("gate_proj", "up_proj"), ci, a["h2b"], None, s)
        self.w4a16("down_proj", ci, a["midb"], s)
        self.w4a16("lm_head", ci, a["finalb"], s)

    def step_bytes(self) -> int:
        """Algorithmic bytes of one step: weights + scales of every GEMV, each launch's
        activation read (int8 + group scales, or fp16 for the launches that quantize
        in-kernel / bf16 for W4A16) counted once per launch, outputs, and the separate
        quantization of the down input (fp16 read, int8 + scales written)."""
        tot = 0
        for name, n, k in SUITE_8B:
            ob = 4 if name == "lm_head" else 2
            tot += weight_bytes(n, k) * 2 + n * ob * 2  # both precisions
        kq = 14336
        tot += 4096 * 2 * 4 + (kq + kq // 32 * 4)       # W4A8 inputs: 4 fp16 launches, down int8
        tot += 2 * kq + kq + kq // 32 * 4               # the down input's quantization
        tot += 2 * 4096 * 4 + 2 * kq                    # W4A16 inputs (bf16), 5 launches
        return tot


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# Launches per graph of the per-kernel tables: a graph replay costs the host-side launch
# and the first dispatch's wait (tens of us at a replay boundary), which 200 back-to-back
# launches amortise to about 1% of an 8B gate launch (MI355X: k_proj 2.55 -> 2.10 us,
# gate 7.36 -> 7.20 us, lm_head 49.3 -> 48.1 us per launch from 40 to 200 launches).
# Steps per graph of the timed step, for the same reason (a step is 11 launches).
STEPS_PER_GRAPH = 4


def time_graphs(torch, graphs, reps: int) -> float:
    """Replay `graphs` round-robin `reps` times; returns ms per replay."""
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def kernel_table(torch, L, weights, acts, launches_per_graph: int = 200, suite=SUITE_8B):
    """Average launch duration of every (shape, precision) GEMV, each timed on its own in
    a graph of back-to-back launches over rotating weight copies.  acts: fp16 / bf16
    activations keyed "h16" / "hb" (the hidden size) and "mid16" / "midb" (the FFN
    size, down_proj's K)."""
    rows = {}
    s_bufs = {}
    hid = [k for nm, _, k in suite if nm == "q_proj"][0]
    for name, n, k in suite:
        sets = weights[name]
        for prec in ("w4a8", "w4a16"):
            odt_t = torch.float32 if name == "lm_head" else (torch.float16 if prec == "w4a8" else torch.bfloat16)
            out = torch.empty(n, dtype=odt_t, device="cuda")
            odt = {torch.float32: 2, torch.float16: 0, torch.bfloat16: 1}[odt_t]
            if prec == "w4a8":
                xq = torch.empty(k, dtype=torch.int8, device="cuda")
                xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
                x16 = acts["h16"] if k == hid else acts["mid16"]
                assert L.nve_hip_quantize_q8(x16.data_ptr(), 0, 1, k, xq.data_ptr(), xs.data_ptr(), None) == 0

                def body(sets=sets, xq=xq, xs=xs, out=out, odt=odt, n=n, k=k):
                    s = torch.cuda.current_stream().cuda_stream
                    for i in range(launches_per_graph):
                        nib, sc = sets[i % len(sets)]
                        assert L.nve_hip_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), nib.data_ptr(), sc.data_ptr(),
                                                     out.data_ptr(), odt, n, k, s) == 0
            else:
                xb = acts["hb"] if k == hid else acts["midb"]

                def body(sets=sets, xb=xb, out=out, odt=odt, n=n, k=k):
                    s = torch.cuda.current_stream().cuda_stream
                    for i in range(launches_per_graph):
                        nib, sc = sets[i % len(sets)]
                        assert L.nve_hip_matvec_w4a16(xb.data_ptr(), 1, nib.data_ptr(), sc.data_ptr(), None,
                                                      out.data_ptr(), odt, n, k, s) == 0
            body()
            g = capture(torch, body)
            time_graphs(torch, [g], 2)
            reps = 3 if name == "lm_head" else 10
            ms = time_graphs(torch, [g], reps)
            us = ms * 1e3 / launches_per_graph
            ob = 4 if name == "lm_head" else 2
            b = gemv_bytes(n, k, prec, ob)
            rows[f"{name}/{prec}"] = {
                "N": n, "K": k, "us": round(us, 3), "gemv_per_s": round(1e6 / us), "bytes": b,
                "GBs": round(b / us / 1e3, 1), "frac_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
            }
            s_bufs[(name, prec)] = (g, out)
            log(f"  {name:10s} {prec:6s} {us:8.2f} us {b / us / 1e3:8.1f} GB/s {100 * b / us / 1e3 / HBM_PEAK_GBS:5.1f}%")
    # grouped launches (one launch for matrices sharing the input)
    from nve_amd._lib import W4Mat
    for label, names in (("qkv_grouped", ("q_proj", "k_proj", "v_proj")), ("gate_up_grouped", ("gate_proj", "up_proj"))):
        k = hid
        for prec in ("w4a8", "w4a16"):
            outs = [torch.empty([n for nm, n, _ in suite if nm == x][0], dtype=torch.float16 if prec == "w4a8"
                                else torch.bfloat16, device="cuda") for x in names]
            xq = torch.empty(k, dtype=torch.int8, device="cuda")
            xs = torch.empty(k // 32, dtype=torch.float32, device="cuda")
            assert L.nve_hip_quantize_q8(acts["h16"].data_ptr(), 0, 1, k, xq.data_ptr(), xs.data_ptr(), None) == 0
            copies = len(weights[names[0]])
            arrs = []
            for ci in range(copies):
                arr = (W4Mat * len(names))()
                for i, nm in enumerate(names):
                    nib, sc = weights[nm][ci]
                    arr[i] = W4Mat(nib.data_ptr(), sc.data_ptr(), None, outs[i].data_ptr(), outs[i].numel())
                arrs.append(arr)

            def body(prec=prec, arrs=arrs, xq=xq, xs=xs, names=names):
                s = torch.cuda.current_stream().cuda_stream
                for i in range(launches_per_graph):
                    a = arrs[i % len(arrs)]
                    if prec == "w4a8":
                        assert L.nve_hip_grouped_matvec_w4a8(xq.data_ptr(), xs.data_ptr(), a, len(names), 0, k, s) == 0
                    else:
                        assert L.nve_hip_grouped_matvec_w4a16(acts["hb"].data_ptr(), 1, a, len(names), 1, k, s) == 0
            body()
            g = capture(torch, body)
            time_graphs(torch, [g], 2)
            us = time_graphs(torch, [g], 10) * 1e3 / launches_per_graph
            b = sum(gemv_bytes([n for nm, n, _ in suite if nm == x][0], k, prec, 2) for x in names)
            b -= (len(names) - 1) * ((k + (k // 32) * 4) if prec == "w4a8" else 2 * k)  # one shared input
            rows[f"{label}/{prec}"] = {"N": sum(o.numel() for o in outs), "K": k, "us": round(us, 3),
                                       "gemv_per_s": round(1e6 / us), "bytes": b,
                                       "GBs": round(b / us / 1e3, 1), "frac_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
            log(f"  {label:15s} {prec:6s} {us:8.2f} us {b / us / 1e3:8.1f} GB/s {100 * b / us / 1e3 / HBM_PEAK_GBS:5.1f}%")
    # the reference's own W4A16 entry point: nve_matvec_w4a16 (fp16 in, fp16 out, no AWQ)
    for name, n, k in suite:
        if name not in ("gate_proj", "down_proj", "lm_head"):
            continue
        sets = weights[name]
        x16 = acts["h16"] if k == hid else acts["mid16"]
        out = torch.empty(n, dtype=torch.float16, device="cuda")

        def body(sets=sets, x16=x16, out=out, n=n, k=k):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(launches_per_graph):
                nib, sc = sets[i % len(sets)]
                L.nve_matvec_w4a16(x16.data_ptr(), nib.data_ptr(), sc.data_ptr(), None, out.data_ptr(), n, k, s)
        body()
        g = capture(torch, body)
        time_graphs(torch, [g], 2)
        us = time_graphs(torch, [g], 3 if name == "lm_head" else 10) * 1e3 / launches_per_graph
        b = gemv_bytes(n, k, "w4a16", 2)
        rows[f"{name}/w4a16_f16_dropin"] = {"N": n, "K": k, "us": round(us, 3), "gemv_per_s": round(1e6 / us),
                                             "bytes": b, "GBs": round(b / us / 1e3, 1),
                                             "frac_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"  {name:10s} w4a16 fp16 drop-in {us:8.2f} us {b / us / 1e3:8.1f} GB/s")
    return rows


def step_head_kernels(torch, step, launches_per_graph: int = 200) -> dict:
    """The step's two lm_head launches, each with the step's own entry point and
    arguments (same kernel instantiation as in the timed step), timed on their own: a
    graph of back-to-back launches over the rotating lm_head copies, HIP events on the
    stream the graph is replayed on."""
    n, k = 128256, 4096
    copies = len(step.w["lm_head"])
    res = {}
    for label, fn in (("w4a8_x", lambda ci, s: step.w4a8_x("lm_head", ci, step.acts["final16"], s)),
                      ("w4a16", lambda ci, s: step.w4a16("lm_head", ci, step.acts["finalb"], s))):
        def body(fn=fn):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(launches_per_graph):
                fn(i % copies, s)
        body()
        g = capture(torch, body)
        time_graphs(torch, [g], 2)
        us = time_graphs(torch, [g], 5) * 1e3 / launches_per_graph
        prec = "w4a8" if label == "w4a8_x" else "w4a16"
        b = gemv_bytes(n, k, prec, 4)
        if label == "w4a8_x":
            b += 2 * k - (k + (k // 32) * 4)  # reads the fp16 vector instead of int8 + scales
        res[label] = {"us": round(us, 3), "bytes": b, "GBs": round(b / us / 1e3, 1)}
        log(f"  step lm_head {label:7s} {us:8.2f} us {b / us / 1e3:8.1f} GB/s")
    return res


def batched_sweep(torch, L, weights, launches_per_graph: int = 200):
    """W4A8 at M in {1,2,4,8,16} activation rows (per-row absmax
    int8, bf16 scales) on the 8B gate (14336x4096) and down (4096x14336) shapes.
    M >= 2 runs on int8 MFMA (v_mfma_i32_16x16x32_i8, 16 activation columns per
    instruction, so the issued MFMA work is 2*16*N*K per launch whatever M is)."""
    import numpy as np
    rows = {}
    for name in ("gate_proj", "down_proj"):
        n, k = [(nn, kk) for nm, nn, kk in SUITE_8B if nm == name][0]
        sets = weights[name]
        for m in (1, 2, 4, 8, 16):
            r = np.random.default_rng(100 + m)
            x = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).cuda().to(torch.bfloat16)
            xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
            xs = torch.empty(m, dtype=torch.bfloat16, device="cuda")
            assert L.nve_hip_quantize_q8_rows(x.data_ptr(), 1, m, k, xq.data_ptr(), xs.data_ptr(), None) == 0
            out = torch.empty((m, n), dtype=torch.float16, device="cuda")

            def body(sets=sets, xq=xq, xs=xs, out=out, m=m, n=n, k=k):
                s = torch.cuda.current_stream().cuda_stream
                for i in range(launches_per_graph):
                    nib, sc = sets[i % len(sets)]
                    assert L.nve_hip_matvec_w4a8_batched(m, xq.data_ptr(), xs.data_ptr(), 1, nib.data_ptr(),
                                                         sc.data_ptr(), out.data_ptr(), 0, n, k, s) == 0
            body()
            g = capture(torch, body)
            time_graphs(torch, [g], 2)
            us = time_graphs(torch, [g], 10) * 1e3 / launches_per_graph
            b = weight_bytes(n, k) + m * (k + 2) + m * n * 2
            rec = {"M": m, "N": n, "K": k, "us": round(us, 3), "GBs": round(b / us / 1e3, 1),
                   "frac_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                   "useful_int8_TOPs": round(2 * m * n * k / us / 1e6, 2),
                   "kernel": "mfma_i32_16x16x32_i8" if m >= 2 else "w4a8_gemv (one-shot, v_dot4)"}
            if m >= 2:
                issued = 2 * 16 * n * k / us / 1e6
                rec["issued_mfma_TOPs"] = round(issued, 2)
                rec["mfma_util_vs_5000_TOPs"] = round(issued / 5000.0, 4)
            rows[f"{name}/M{m}"] = rec
            log(f"  {name:10s} M={m:2d} {us:8.2f} us {b / us / 1e3:8.1f} GB/s {100 * b / us / 1e3 / HBM_PEAK_GBS:5.1f}%"
                f"  {rec['kernel']}")
    return rows


def stream_probe(torch, L) -> float:
    buf = torch.empty(2 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1024, device="cuda")

    def body():
        s = torch.cuda.current_stream().cuda_stream
        for _ in range(5):
            assert L.nve_hip_stream_read(buf.data_ptr(), buf.numel(), sink.data_ptr(), s) == 0
    body()
    g = capture(torch, body)
    ms = time_graphs(torch, [g], 3) / 5
    del buf
    return buf_gbs(2 << 30, ms)


def same_size_read(torch, L, nbytes: int, copies: int, launches_per_graph: int = 200) -> dict:
    """The streaming-read ceiling at one byte count: the library's read probe
    (nve_hip_stream_read_mode) over `copies` rotating buffers of `nbytes` each -- the
    same rotation the GEMV table uses for that shape, so the MALL serves neither more
    nor less -- timed like the GEMVs (a graph of back-to-back launches, HIP events on
    the replay stream).  Every probe form (one-shot, grid-stride at 1 and 2 workgroups
    per CU) is timed; the fastest is the ceiling."""
    stride = (nbytes + 4095) // 4096 * 4096
    n16 = (nbytes + 15) // 16 * 16
    buf = torch.empty(stride * copies, dtype=torch.uint8, device="cuda")
    buf.fill_(0x5A)
    sink = torch.zeros(1024, device="cuda")
    best = None
    for mode in (0, 1, 2):
        def body(mode=mode):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(launches_per_graph):
                assert L.nve_hip_stream_read_mode(buf.data_ptr() + (i % copies) * stride, n16, sink.data_ptr(),
                                                  mode, s) == 0
        body()
        g = capture(torch, body)
        time_graphs(torch, [g], 2)
        us = time_graphs(torch, [g], 10) * 1e3 / launches_per_graph
        if best is None or us < best["us"]:
            best = {"us": round(us, 3), "GBs": round(nbytes / us / 1e3, 1),
                    "form": ("one-shot", "grid-stride 1 wg/CU", "grid-stride 2 wg/CU")[mode]}
    del buf, g
    return best


def add_read_ceiling(torch, L, table: dict, copies_of) -> dict:
    """Annotate every row of a kernel table with the same-size read ceiling:
    read_us and frac_of_same_size_read = read_us / us (1.0 = the GEMV streams its
    bytes as fast as a pure read of the same size)."""
    cache = {}
    for key, row in table.items():
        c = copies_of(key)
        if (row["bytes"], c) not in cache:
            cache[(row["bytes"], c)] = same_size_read(torch, L, row["bytes"], c)
        r = cache[(row["bytes"], c)]
        row["read_us"] = r["us"]
        row["frac_of_same_size_read"] = round(r["us"] / row["us"], 4)
    return {str(b): {"copies": c, **r} for (b, c), r in sorted(cache.items())}


def buf_gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9


def host_cpus() -> tuple[int, str, str | None]:
    """(threads to use = every core this process may run on, CPU model string, the
    cgroup CPU quota if one is set)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    quota = None
    try:
        q = open("/sys/fs/cgroup/cpu.max").read().split()
        if q and q[0] != "max":
            quota = f"{int(q[0]) / int(q[1]):.1f} CPUs"
    except (OSError, ValueError, IndexError):
        pass
    return n, model, quota


def cpu_baseline(target_s: float = 12.0) -> dict:
    """The reference's CPU quantized GEMV (q4_dot_row_avx2 + row-parallel matvec_f32,
    restated in oracle/) over 8B gate_proj + down_proj, on every host core this
    process may use (rayon's default pool, src/quantize.rs:476)."""
    import numpy as np
    from oracle import oracle as orc
    threads, model, quota = host_cpus()
    r = np.random.default_rng(7)
    mats = []
    for n, k in ((14336, 4096), (4096, 14336)):
        w = (r.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        mats.append((orc.q4_from_f32(w), n, k, r.standard_normal(k).astype(np.float32)))
        del w
    b = sum(weight_bytes(n, k) + 4 * k + 4 * n for _, n, k, _ in mats)
    for data, n, k, x in mats:  # warm
        orc.q4_matvec_f32(data, n, k, x, threads=threads)
    reps = 0
    t0 = time.perf_counter()
    while True:
        for data, n, k, x in mats:
            orc.q4_matvec_f32(data, n, k, x, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    gbs = b * reps / el / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port", "cpu_model": model,
            "cgroup_cpu_quota": quota,
            "sample": f"8B gate_proj 14336x4096 + down_proj 4096x14336, W4 x f32 (QuantizedTensor::matvec_f32 / "
                      f"q4_dot_row_avx2 restated in oracle/oracle.c), {reps} passes in {el:.1f} s, "
                      f"{threads} threads; GB/s over the same algorithmic bytes as the GPU"}


def attn_key_split(shape, max_seq: int) -> int:
    """The key split the library's decode attention takes (decode.hip attn_split): 1 up
    to 256 cache slots, 4 up to 1024, else 8 when num_heads * head_dim <= 4096 (else 4);
    NVE_ATTN_SPLIT overrides, capped the same way."""
    cap = 8 if shape.heads * shape.head_dim <= 4096 else 4
    e = os.environ.get("NVE_ATTN_SPLIT")
    if e in ("1", "2", "4", "8"):
        return min(int(e), cap)
    return 1 if max_seq <= 256 else (4 if max_seq <= 1024 else cap)


DECODE_STEPS_PER_GRAPH = 8


def decode_3b(torch, tokens: int, warm: int, cpu_tokens: int, no_cpu: bool, prefill: int = 512,
              max_seq: int = 1024, steps_per_graph: int = DECODE_STEPS_PER_GRAPH) -> dict:
    """synthetic Llama-3.2-3B decode at batch 1, greedy.  28 layers
    (a seeded 30% = 8 W4A16, 20 W4A8; W4A8 lm_head), 512 prefilled N(0,1) bf16 KV
    positions, HIP graphs of `steps_per_graph` consecutive tokens (all layers + head per
    token; token and position device-resident, so each step feeds the next) and a one-token
    graph for a remainder, `tokens` greedy tokens timed with HIP events on the replay
    stream.  The CPU leg runs
    the reference's CPU decode path (Q4 x f32 matvec_f32, AVX2 restated in oracle/, all
    projections; f32 attention) on the same weights for `cpu_tokens` tokens.  prefill /
    max_seq: the cached positions and the cache capacity (also run at 7000 / 8192 as
    the long-context line, GPU only)."""
    from nve_amd.decode import LLAMA_3_2_3B, DecodeModel
    s = LLAMA_3_2_3B
    if prefill + warm + 1 >= max_seq:
        raise SystemExit(f"decode: prefill ({prefill}) + warm-up ({warm}) + 1 must be below max_seq ({max_seq})")
    tokens = min(tokens, max_seq - prefill - warm - 1)
    assert tokens >= 1
    m = DecodeModel(s, max_seq=max_seq, prefill=prefill)
    m.capture(steps_per_graph)
    m.start(1)
    m.generate(warm)
    torch.cuda.synchronize()
    m.start(1)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    m.generate(tokens)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / tokens
    wb = m.step_bytes()
    kvb = m.kv_bytes(prefill + tokens // 2)  # mean cache length over the timed tokens
    tok_s = 1e3 / ms
    n16 = sum(1 for u in m.use_w4a8 if not u)
    rec = {"tok_per_s": round(tok_s, 1), "ms_per_token": round(ms, 4), "tokens": tokens, "warmup": warm,
           "layers_w4a8": s.layers - n16, "layers_w4a16": n16, "kv_prefill": prefill, "kv_capacity": max_seq,
           "bytes_per_token": wb + kvb,
           "GBs": round((wb + kvb) / (ms * 1e-3) / 1e9, 1),
           "frac_hbm_peak": round((wb + kvb) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           # per layer: Q/K/V (norm fused), attention, o_proj, gate/up (norm + SwiGLU fused),
           # down; head: final norm, lm_head (a W4A8 one leaves the argmax candidates, a
           # W4A16 one is followed by an argmax-partials launch), argmax + next embedding
           "launches_per_token": 5 * s.layers + (3 if m.lm_head_w4a8 else 4),
           "attn_key_split": attn_key_split(s, max_seq), "tokens_per_graph": steps_per_graph}
    log(f"decode 3B: {ms * 1e3:.1f} us/token, {tok_s:.1f} tok/s, {rec['GBs']} GB/s")
    if not no_cpu:
        import numpy as np
        from oracle import decode_ref as dr
        log("decode 3B CPU leg: copying weights to host")
        hm = dr.HostModel(m, with_cpu_blocks=True)
        threads, model, quota = host_cpus()
        h = hm.embed[1].copy()
        h, _ = dr.reference_step(hm, h, prefill, threads)  # warm
        t0 = time.perf_counter()
        for i in range(cpu_tokens):
            h, _ = dr.reference_step(hm, h, prefill + 1 + i, threads)
        el = time.perf_counter() - t0
        rec["cpu_baseline"] = {"value": round(cpu_tokens / el, 2), "unit": "tok/s", "cores": threads, "kind": "port",
                               "cpu_model": model, "cgroup_cpu_quota": quota,
                               "sample": f"{cpu_tokens} greedy tokens (after 1 warm) of the same 3B model on the "
                                         f"reference CPU decode path (QuantizedTensor::matvec_f32 / q4_dot_row_avx2 "
                                         f"restated in oracle/, f32 activations), {el:.1f} s"}
        log(f"decode 3B CPU: {cpu_tokens / el:.2f} tok/s on {threads} threads")
        del hm
    del m
    torch.cuda.empty_cache()
    return rec


def prefill_gemm(torch, hk, reps: int = 20) -> dict:
    """The prefill-adjacency row: W4A16 GEMM X[M, K] @ W^T at the 8B gate shape
    (14336 x 4096), fp16 activations, fp32 output, M in {1, 4, 16, 128, 256, 512, 2048}:
    the fused MFMA kernels of nve_hip_gemm_w4a16 (weight-streaming at M = 1-128 at this
    shape, then the register-dequant tile kernel: 128-row tiles at M = 256, 256-row tiles
    from M = 512)
    against the reference's own method on the same GPU
    (nve_dequant_w4a16 to fp16, then a dense fp16 GEMM -- torch.matmul, i.e. the
    vendor BLAS -- as GpuWeight::matmul_x does with candle, src/gpu_layer.rs:219-237).
    Times: HIP events over graphs of `reps` launches; TFLOP/s = 2 M N K / time.
    library_us: nve_hip_gemm_w4a16_ws with its workspace (dequant + hipBLASLt above
    M = 512, the fused kernels up to it), fp32 output; library_f16_out_us: the same
    with fp16 output, the output type of the reference-method timing.  awq_rows: the
    library entry and the two-step method with AWQ factors at M = 128 and 512."""
    g = torch.Generator(device="cuda").manual_seed(17)
    n, k = 14336, 4096
    nib, sc = hk.q4_quantize(torch.randn((n, k), generator=g, device="cuda").mul_(0.02))
    out = {"shape": f"{n}x{k}", "x_dtype": "f16", "peak_TFLOPs": MFMA_F16_PEAK_TFLOPS, "rows": []}
    for m in (1, 4, 16, 128, 256, 512, 2048):
        x = torch.randn((m, k), generator=g, device="cuda").half()
        wf = hk.dequant_w4(nib, sc, n, k)

        def timed(fn):
            fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(reps):
                    fn()
            gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / reps

        us = timed(lambda: hk.gemm_w4a16(x, nib, sc, n, k))
        us_ref = timed(lambda: hk.dequant_w4(nib, sc, n, k)) + timed(lambda: torch.matmul(x, wf.t()))
        wsb = hk.gemm_w4a16_workspace_bytes(m, n, k)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda") if wsb else None
        us_lib = timed(lambda: hk.gemm_w4a16_ws(x, nib, sc, n, k, ws))
        # fp16 output, as torch.matmul writes in the reference-method timing above
        us_lib16 = timed(lambda: hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, out_dtype=torch.float16))
        fl = 2.0 * m * n * k
        out["rows"].append({"M": m, "fused_us": round(us, 1), "fused_TFLOPs": round(fl / us / 1e6, 1),
                            "frac_mfma_peak": round(fl / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
                            "dequant_plus_blas_us": round(us_ref, 1),
                            "library_us": round(us_lib, 1),
                            "library_f16_out_us": round(us_lib16, 1),
                            # the library's rule (gemm_blas.hip): dequant + hipBLASLt above M = 512
                            # with a workspace; up to it the fused kernels
                            "library_path": "dequant + hipBLASLt" if m > 512 and wsb else "fused"})
        log(f"  prefill GEMM M={m}: {us:.1f} us ({fl / us / 1e6:.0f} TFLOP/s), dequant+BLAS {us_ref:.1f} us, "
            f"nve_hip_gemm_w4a16_ws {us_lib:.1f} us (fp16 out {us_lib16:.1f} us)")
        del x, wf, ws
    # with AWQ factors (the reference dequant multiplies each f32 weight by awq[k] before the
    # fp16 rounding): the library entry with its workspace against the same two-step method
    awq = torch.rand(k, generator=g, device="cuda").add_(0.5)
    out["awq_rows"] = []
    for m in (128, 512):
        x = torch.randn((m, k), generator=g, device="cuda").half()
        wf = hk.dequant_w4(nib, sc, n, k, awq)
        wsb = hk.gemm_w4a16_workspace_bytes(m, n, k)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda") if wsb else None
        us_lib = timed(lambda: hk.gemm_w4a16_ws(x, nib, sc, n, k, ws, awq))
        us_ref = timed(lambda: hk.dequant_w4(nib, sc, n, k, awq)) + timed(lambda: torch.matmul(x, wf.t()))
        out["awq_rows"].append({"M": m, "library_us": round(us_lib, 1), "dequant_plus_blas_us": round(us_ref, 1)})
        log(f"  prefill GEMM with AWQ M={m}: nve_hip_gemm_w4a16_ws {us_lib:.1f} us, dequant+BLAS {us_ref:.1f} us")
        del x, wf, ws
    return out


def decode_traffic_probe(torch) -> None:
    """Six eager 3B decode steps (the bench's model: max_seq 1024, 512 prefilled
    positions) for per-dispatch HBM counters; eager launches because counter collection
    over HIP-graph replays crashed the profiler's host library."""
    from nve_amd.decode import LLAMA_3_2_3B, DecodeModel
    m = DecodeModel(LLAMA_3_2_3B, max_seq=1024, prefill=512)
    m.start(1)
    for _ in range(6):
        m.step()
    torch.cuda.synchronize()
    log(f"decode traffic probe: 6 steps, algorithmic bytes per step {m.step_bytes()}")


def prefill_probe(torch, hk):
    """Eager launches for rocprofv3 --pmc of the fused prefill GEMM at large M (counter
    collection over HIP-graph replays is not used): the 8B gate shape 14336x4096, fp16
    x, fp16 output (one pass over K, no split), M = 512 then M = 2048, 5 launches each."""
    g = torch.Generator(device="cuda").manual_seed(17)
    n, k = 14336, 4096
    nib, sc = hk.q4_quantize(torch.randn((n, k), generator=g, device="cuda").mul_(0.02))
    for m in (512, 2048):
        x = torch.randn((m, k), generator=g, device="cuda").half()
        for _ in range(5):
            hk.gemm_w4a16(x, nib, sc, n, k, out_dtype=torch.float16)
        torch.cuda.synchronize()
    print(json.dumps({"probe": "prefill", "shape": f"{n}x{k}", "M": [512, 2048], "launches_each": 5}), flush=True)


def prefill_ws_probe(torch, hk):
    """Eager launches of nve_hip_gemm_w4a16_ws (fp16 x, fp32 out, with its workspace) for
    a rocprofv3 kernel trace of the K-split tile path: the 8B gate (14336x4096) and down
    (4096x14336) shapes at M = 96, 128, 256, 512, one warm-up then 5 launches each."""
    g = torch.Generator(device="cuda").manual_seed(17)
    cases = []
    for n, k in ((14336, 4096), (4096, 14336)):
        nib, sc = hk.q4_quantize(torch.randn((n, k), generator=g, device="cuda").mul_(0.02))
        for m in (96, 128, 256, 512):
            x = torch.randn((m, k), generator=g, device="cuda").half()
            ws = torch.empty(hk.gemm_w4a16_workspace_bytes(m, n, k), dtype=torch.uint8, device="cuda")
            for _ in range(6):
                hk.gemm_w4a16_ws(x, nib, sc, n, k, ws)
            torch.cuda.synchronize()
            cases.append({"N": n, "K": k, "M": m, "workspace_bytes": ws.numel()})
            del x, ws
    print(json.dumps({"probe": "prefill_ws", "launches_each": 6, "cases": cases}), flush=True)


def batched_probe(torch, L, hk):
    """Short eager run for rocprofv3 --pmc of the batched W4A8 kernels (MFMA counters):
    the configs[3] shapes (8B gate and down) at M in {1, 2, 4, 8, 16}, 10 launches each
    over 4 weight copies, in the order printed."""
    import numpy as np
    g = torch.Generator(device="cuda").manual_seed(12)
    order = []
    for name in ("gate_proj", "down_proj"):
        n, k = [(nn, kk) for nm, nn, kk in SUITE_8B if nm == name][0]
        sets = []
        for _ in range(4):
            w = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32).mul_(0.02)
            sets.append(hk.q4_quantize(w))
            del w
        for m in (1, 2, 4, 8, 16):
            r = np.random.default_rng(100 + m)
            x = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).cuda().to(torch.bfloat16)
            xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
            xs = torch.empty(m, dtype=torch.bfloat16, device="cuda")
            assert L.nve_hip_quantize_q8_rows(x.data_ptr(), 1, m, k, xq.data_ptr(), xs.data_ptr(), None) == 0
            out = torch.empty((m, n), dtype=torch.float16, device="cuda")
            s = torch.cuda.current_stream().cuda_stream
            for i in range(10):
                nib, sc = sets[i % 4]
                assert L.nve_hip_matvec_w4a8_batched(m, xq.data_ptr(), xs.data_ptr(), 1, nib.data_ptr(), sc.data_ptr(),
                                                     out.data_ptr(), 0, n, k, s) == 0
            torch.cuda.synchronize()
            order.append({"shape": name, "N": n, "K": k, "M": m, "launches": 10})
        del sets
    print(json.dumps({"probe": "batched", "order": order}), flush=True)


def suite_probe(torch, L, hk):
    """The per-shape tables of the bench (8B suite, both precisions, grouped launches;
    batched W4A8 sweep) on their own, for a rocprofv3 kernel trace: each (shape,
    precision) runs as graphs of back-to-back launches separated by host
    synchronisations, in the order printed at the end."""
    weights = make_inputs(torch, hk, 8, 4)
    acts = {}
    for nm, k, sd in (("h", 4096, 1), ("mid", 14336, 4)):
        x = make_activation(torch, k, sd)
        acts[nm + "16"] = x.to(torch.float16)
        acts[nm + "b"] = x.to(torch.bfloat16)
    table = kernel_table(torch, L, weights, acts)
    sweep = batched_sweep(torch, L, weights)
    print(json.dumps({"probe": "suite", "order": list(table) + list(sweep)}), flush=True)


def traffic_probe(torch, L, hk):
    """Short run for rocprofv3 --pmc (FETCH_SIZE / WRITE_SIZE): a plain device copy of
    256 MiB (calibration: 256 MiB read + 256 MiB written), then the step's two lm_head
    launches (128256x4096, fp32 logits) 5 times each on 5 distinct weight copies: W4A8
    quantizing its fp16 input in-kernel (nve_hip_matvec_w4a8_x), then W4A16 on bf16
    activations.  Prints the launch order so per-dispatch counters can be matched."""
    g = torch.Generator(device="cuda").manual_seed(11)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.random_(generator=g)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    n, k = 128256, 4096
    sets = []
    for _ in range(5):
        w = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32).mul_(0.02)
        sets.append(hk.q4_quantize(w))
        del w
    x = make_activation(torch, k, 5)
    x16, xb = x.to(torch.float16), x.to(torch.bfloat16)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    s = torch.cuda.current_stream().cuda_stream
    for nib, sc in sets:
        assert L.nve_hip_matvec_w4a8_x(x16.data_ptr(), 0, nib.data_ptr(), sc.data_ptr(), out.data_ptr(), 2, n, k,
                                       s) == 0
    for nib, sc in sets:
        assert L.nve_hip_matvec_w4a16(xb.data_ptr(), 1, nib.data_ptr(), sc.data_ptr(), None, out.data_ptr(), 2, n, k,
                                      s) == 0
    torch.cuda.synchronize()
    b8 = gemv_bytes(n, k, "w4a8", 4) + 2 * k - (k + (k // 32) * 4)
    print(json.dumps({"probe": "traffic", "copy_bytes": 256 << 20,
                      "launches": [{"label": "w4a8_x", "count": 5, "bytes": b8},
                                   {"label": "w4a16", "count": 5, "bytes": gemv_bytes(n, k, "w4a16", 4)}]}),
          flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--cpu-decode-tokens", type=int, default=3)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--decode-prefill", type=int, default=512,
                    help="cached positions before the timed tokens (--decode-only)")
    ap.add_argument("--decode-max-seq", type=int, default=1024, help="KV cache slots (--decode-only)")
    ap.add_argument("--decode-steps-per-graph", type=int, default=DECODE_STEPS_PER_GRAPH,
                    help="tokens per replayed HIP graph in the decode measurement")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the 3B decode measurement (for profiling; no bench line)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="short run for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (no bench line)")
    ap.add_argument("--batched-probe", action="store_true",
                    help="eager batched W4A8 launches for rocprofv3 --pmc MFMA counters (no bench line)")
    ap.add_argument("--suite-probe", action="store_true",
                    help="only the per-shape 8B table and the batched sweep, for rocprofv3 --kernel-trace "
                         "per-shape kernel durations (no bench line)")
    ap.add_argument("--prefill-ws-probe", action="store_true",
                    help="eager nve_hip_gemm_w4a16_ws launches (8B gate / down, M = 96-512) for a rocprofv3 "
                         "kernel trace of the K-split tile path (no bench line)")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="eager fused prefill GEMM launches at M = 512 / 2048 for rocprofv3 --pmc (no bench line)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the W4A16 prefill GEMM rows (for profiling; no bench line)")
    ap.add_argument("--decode-traffic-probe", action="store_true",
                    help="6 eager (not graph-replayed) 3B decode steps for rocprofv3 --pmc (no bench line)")
    args = ap.parse_args()
    if args.decode_prefill < 0 or args.decode_prefill + 16 + 1 >= args.decode_max_seq:
        ap.error("--decode-prefill + 17 (16 warm-up tokens and one timed) must be below --decode-max-seq")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).", file=sys.stderr)
        sys.exit(2)

    import torch
    from nve_amd._lib import lib
    from nve_amd import hip_kernels as hk
    L = lib()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.traffic_probe:
        traffic_probe(torch, L, hk)
        return
    if args.decode_traffic_probe:
        decode_traffic_probe(torch)
        return
    if args.batched_probe:
        batched_probe(torch, L, hk)
        return
    if args.suite_probe:
        suite_probe(torch, L, hk)
        return
    if args.prefill_ws_probe:
        prefill_ws_probe(torch, hk)
        return
    if args.prefill_probe:
        prefill_probe(torch, hk)
        return
    if args.prefill_only:
        print(json.dumps({"prefill_w4a16_gemm": prefill_gemm(torch, hk)}))
        return
    if args.decode_only:
        print(json.dumps({"decode_3b": decode_3b(torch, args.decode_tokens, 16, args.cpu_decode_tokens, True,
                                                 prefill=args.decode_prefill, max_seq=args.decode_max_seq,
                                                 steps_per_graph=args.decode_steps_per_graph)}))
        return

    # weight copies: layer set 136 MB -> 8 copies (1.09 GB); lm_head 328 MB -> 4 copies
    copies_layer, copies_head = 8, 4
    log(f"generating weights ({copies_layer} layer copies, {copies_head} lm_head copies)")
    weights = make_inputs(torch, hk, copies_layer, copies_head)
    acts = {}
    for nm, k, sd in (("h", 4096, 1), ("attn", 4096, 2), ("h2", 4096, 3), ("mid", 14336, 4), ("final", 4096, 5)):
        x = make_activation(torch, k, sd)
        acts[nm + "16"] = x.to(torch.float16)
        acts[nm + "b"] = x.to(torch.bfloat16)

    step = Step(torch, L, weights, acts)
    n_graphs = max(copies_layer, copies_head)
    step.run(0)
    torch.cuda.synchronize()
    # one-step graphs (per weight copy) and STEPS_PER_GRAPH-step graphs over consecutive
    # copies; K timed steps = K // STEPS_PER_GRAPH multi-step replays + K % STEPS_PER_GRAPH
    # one-step replays, every step on the next weight copy
    graphs = [capture(torch, lambda ci=ci: step.run(ci)) for ci in range(n_graphs)]

    def run_steps(ci0):
        for j in range(STEPS_PER_GRAPH):
            step.run(ci0 + j)
    multi = [capture(torch, lambda ci=ci: run_steps(ci)) for ci in range(0, n_graphs, STEPS_PER_GRAPH)]

    def time_steps(k: int) -> float:
        """ms per step over exactly k steps (HIP events on the replay stream)."""
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        q, r = divmod(k, STEPS_PER_GRAPH)
        for i in range(q):
            multi[i % len(multi)].replay()
        for j in range(r):
            graphs[(q * STEPS_PER_GRAPH + j) % n_graphs].replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k
    # The per-shape table runs before the step is timed (same weight copies, ~10 s of
    # GPU work, no host-only gap before the step's warmup): right after set-up the step
    # runs up to 15% slower for its first few hundred replays (194, 181, 176 us for the
    # first three 20-step passes, 168 us from about the 300th), and the step is meant
    # to be timed in that steady state.
    # and every launch runs slower right after set-up (the first lm_head graph a process
    # times, about 10 us above the steady 49-50 us), so the table starts after 300 step
    # replays (about 50 ms)
    time_steps(300)
    log("per-kernel table:")
    table = kernel_table(torch, L, weights, acts)
    time_steps(max(args.warmup, 1))
    ms = time_steps(args.steps)
    sb = step.step_bytes()
    value = sb / (ms * 1e-3) / 1e9
    log(f"step: {ms * 1e3:.1f} us, {sb / 1e6:.1f} MB algorithmic, {value:.1f} GB/s")

    log("same-size read ceilings (8B rows):")
    read_8b = add_read_ceiling(torch, L, table, lambda key: copies_head if key.startswith("lm_head") else copies_layer)
    for b, r in read_8b.items():
        log(f"  {int(b) / 1e6:8.2f} MB  {r['us']:8.2f} us {r['GBs']:8.1f} GB/s ({r['form']})")
    log("the step's lm_head launches:")
    heads = step_head_kernels(torch, step)
    for h in heads.values():
        h["read_us"] = same_size_read(torch, L, h["bytes"], copies_head)["us"]
    log("batched W4A8 sweep (per-token int8 activations):")
    sweep = batched_sweep(torch, L, weights)
    stream_gbs = stream_probe(torch, L)
    log(f"HBM streaming probe: {stream_gbs:.1f} GB/s")

    def agg(prec, names):
        b = sum(table[f"{n}/{prec}"]["bytes"] for n in names)
        t = sum(table[f"{n}/{prec}"]["us"] for n in names)
        return round(b / t / 1e3, 1)

    layer_names = [n for n, _, _ in SUITE_8B if n != "lm_head"]
    rot_gb = round(sum(weight_bytes(n, k) * len(weights[nm]) for nm, n, k in SUITE_8B) / 1e9, 2)
    del weights, step, graphs, multi
    torch.cuda.empty_cache()
    # the Llama-3.2-1B layer shapes, same method (16 weight copies)
    log("per-kernel table, Llama-3.2-1B shapes:")
    w1b = make_inputs(torch, hk, 16, 1, seed=0x4E5646, suite=SUITE_1B)
    acts1b = {}
    for nm, k, sd in (("h", 2048, 11), ("mid", 8192, 14)):
        x = make_activation(torch, k, sd)
        acts1b[nm + "16"] = x.to(torch.float16)
        acts1b[nm + "b"] = x.to(torch.bfloat16)
    table_1b = kernel_table(torch, L, w1b, acts1b, suite=SUITE_1B)
    read_1b = add_read_ceiling(torch, L, table_1b, lambda key: 16)
    del w1b, acts1b
    torch.cuda.empty_cache()
    decode = None if args.no_decode else decode_3b(torch, args.decode_tokens, 16, args.cpu_decode_tokens,
                                                   args.no_cpu)
    decode_long = None
    if not args.no_decode:
        torch.cuda.empty_cache()
        decode_long = decode_3b(torch, 128, 8, 0, True, prefill=7000, max_seq=8192)
    log("prefill W4A16 GEMM:")
    prefill = prefill_gemm(torch, hk)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    # HBM bytes per launch of the step's lm_head kernels, from the calibrated rocprofv3
    # FETCH_SIZE / WRITE_SIZE passes over `bench.py --traffic-probe` (recorded in
    # profiles/lm_head_8b_step_kernels_traffic.md)
    traffic = {}
    tf = ROOT / "profiles" / "lm_head_8b_step_kernels_traffic.md"
    if tf.exists():
        import re
        m = re.search(r"```json\n(.*?)\n```", tf.read_text(), re.S)
        if m:
            traffic = json.loads(m.group(1)).get("hbm_bytes_per_launch", {})
    kernels = {"w4a8_x": "w4a8_gemv_kernel<F32, R=4, NJ=2, SRC_F16> (nve_hip_matvec_w4a8_x, lm_head 128256x4096, "
                         "fp16 input quantized in-kernel, fp32 logits)",
               "w4a16": "w4a16_gemv_kernel<bf16 x, F32 out> (nve_hip_matvec_w4a16, lm_head 128256x4096, fp32 logits)"}
    order = sorted(heads, key=lambda kk: -heads[kk]["us"])

    def roof(label):
        h = heads[label]
        return {"kernel": kernels[label], "bound": "hbm", "achieved": h["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(h["GBs"] / HBM_PEAK_GBS, 4), "traffic": traffic.get(label),
                "achievable_peak": round(stream_gbs, 1), "frac_of_achievable": round(h["GBs"] / stream_gbs, 4),
                "same_size_read_us": h["read_us"], "frac_of_same_size_read": round(h["read_us"] / h["us"], 4),
                "bytes_per_launch": h["bytes"], "us_per_launch": h["us"]}

    rec = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x int8 -> int32 (W4A8); int4 x bf16 -> fp32 (W4A16)",
        "data": "synthetic (seeded N(0,0.02) weights int4-quantized on device; N(0,1) activations, 0.5% at 20 sigma)",
        "config": {
            "workload": "Llama-3.1-8B layer-shape suite, batch 1, W4A8 + W4A16(bf16): q,k,v,o,gate,up,down,lm_head; "
                        "one step = both precisions over all shapes incl. the W4A8 activation quantizations "
                        "(in-kernel for K=4096, one launch for the down input)",
            "weights_in_rotation_GB": rot_gb,
            "step_bytes": sb,
            "graph": f"HIP graphs of {STEPS_PER_GRAPH} steps (and of 1 step for a remainder), each step on the next "
                     "weight copy, replayed round-robin",
        },
        "roofline": roof(order[0]),
        "roofline_other": roof(order[1]),
        "cpu_baseline": cpu,
        "suite_8b": table,
        "suite_8b_aggregate_GBs": {"w4a8_layers": agg("w4a8", layer_names), "w4a16_layers": agg("w4a16", layer_names),
                                   "w4a8_all": agg("w4a8", [n for n, _, _ in SUITE_8B]),
                                   "w4a16_all": agg("w4a16", [n for n, _, _ in SUITE_8B])},
        "suite_1b": table_1b,
        "hbm_stream_probe_GBs": round(stream_gbs, 1),
        "same_size_read_8b": read_8b,
        "same_size_read_1b": read_1b,
        "batched_w4a8_8b": sweep,
        "decode_3b": decode,
        "decode_3b_long_context": decode_long,
        "prefill_w4a16_gemm": prefill,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
