#!/usr/bin/env python3
"""Benchmark of the quantized linear path on one MI355X.

Headline (BASELINE.json metric, config C2): W4A16 AWQ-style g128 decode GEMV,
N=11008, K=4096, M=1, bf16 activations, in achieved HBM GB/s of algorithmic
bytes.  A "step" is one GEMV call; the 16 weight copies rotate so each call
streams its 23.5 MB from HBM rather than from the 256 MB Infinity Cache.

The JSON line also carries the roofline of the dominant kernel, the CPU
baseline (the oracle's C restatement on one host core, a bounded sample), and
`extra` measurements for the other configs (W8A8 int8/fp8 GEMM at M=2048 in
TOPS, W4A16 at M=4/16, GPTQ act-order, the W8 GEMV).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu] [--no-extra]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "sneppx-alg_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5033.2        # dense int8 MFMA (256 CU x 8192 op/clk x 2.4 GHz)
FP8_PEAK_TOPS = 5033.2         # dense fp8 MFMA
BF16_PEAK_TFLOPS = 2516.6      # dense bf16 MFMA
FP4_PEAK_TFLOPS = 10066.3      # dense fp4 MFMA (MXFP4)
FP6_PEAK_TFLOPS = 10066.3      # dense fp6 MFMA (MXFP6)
# MFMA-heavy kernels reach their steady shader clock only after ~30 ms of
# work: C4 fp8 measured 2278 TOPS timed after 30 warm-up launches and
# 2527-2553 TOPS after 300-3000 (one box, 200 timed launches each), so the
# GEMM lines warm up for 300 launches (~30 ms) before their timed launches.
GEMM_WARMUP, GEMM_STEPS = 300, 200
MX_BENCH = {"mxfp4_e2m1": FP4_PEAK_TFLOPS, "nvfp4_e2m1": FP4_PEAK_TFLOPS, "mxfp8_e4m3": FP8_PEAK_TOPS,
            "mxfp8_e5m2": FP8_PEAK_TOPS, "mxfp6_e3m2": FP6_PEAK_TFLOPS, "mxfp6_e2m3": FP6_PEAK_TFLOPS}
SNEPPX_BFLOAT16 = 3            # SNEPPXDtype of include/sneppx_qlinear.h
GRAPH_HOLD_CYCLES = 400_000    # GPU spin (~0.2 ms) ahead of a timed graph replay
DECODE_GRAPH = False           # time the decode GEMV lines as one HIP graph replay (--graph)
METRIC = "W4A16 GEMV achieved HBM GB/s (% peak); W8A8 GEMM TOPS at M=2048 (% peak)"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=16, help="rotating weight copies (>256 MB total)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extra", action="store_true", help="headline config only")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--m", type=int, default=1, help="activation rows for --only gemv")
    p.add_argument("--graph", action="store_true", help="--only: time the decode lines as a HIP graph replay")
    p.add_argument("--only", choices=["gemv", "gemm-i8", "gemm-fp8", "gemm-dyn", "gemm-w4", "chain", "mx", "decode",
                                      "shard", "copy", "fit"],
                   help="run one kernel family and exit (for rocprofv3 --pmc passes)")
    return p.parse_args()


def w4_bytes(M, N, K, G, zeros=True, gidx=False):
    b = N * K // 2 + N * G * 2 + M * K * 2 + M * N * 2
    if zeros:
        b += N * ((G + 7) // 8) * 4
    if gidx:
        b += K * 4
    return b


def _graph(graph):
    """A decode bench's timing mode: its own argument, else --graph."""
    return DECODE_GRAPH if graph is None else graph


class Timer:
    """HIP events recorded on the stream the kernels are launched on."""

    def __init__(self, lib, stream):
        self.lib, self.stream = lib, stream

    def run(self, calls, steps, warmup, loop=None, graph=False):
        """Back-to-back time of `steps` calls between two events; `loop(n)`,
        when given, issues n calls from C (bench_loop.c) instead of Python.
        graph: the `steps` calls are captured once into a HIP graph and the
        timed region is one replay of it (one host call for the whole run,
        as a decode loop runs its captured steps), the calls' own kernels
        back to back on the GPU."""
        import torch

        def issue(n):
            if loop:
                loop(n)
            else:
                for i in range(n):
                    calls[i % len(calls)]()
        a, b = self.lib.event(), self.lib.event()
        g = None
        if graph:
            issue(1)                   # any workspace exists before the capture
            torch.cuda.synchronize()
            g = self.lib.capture(lambda: issue(steps), self.stream)
        torch.cuda.synchronize()
        issue(warmup)
        if g is not None:
            self.lib.graph_launch(g, self.stream)     # untimed replay: the graph's first upload
            # a bounded spin on the GPU keeps the queue busy while the host
            # submits the timed replay, so its first kernel follows at once
            torch.cuda._sleep(GRAPH_HOLD_CYCLES)
        # whole-job time: back-to-back launches between two events.  The
        # start event is queued right behind the warm-up launches (no host
        # synchronisation in between), so the timed launches begin on a busy
        # queue: the first launch's wake-up latency stays in the warm-up and
        # a short run times the same steady state as a long one.
        self.lib.record(a, self.stream)
        if g is not None:
            self.lib.graph_launch(g, self.stream)
        else:
            issue(steps)
        self.lib.record(b, self.stream)
        torch.cuda.synchronize()
        total_ms = self.lib.elapsed_ms(a, b)
        if g is not None:
            self.lib.graph_destroy(g)
        # per-launch duration: an event pair around every launch
        evs = [(self.lib.event(), self.lib.event()) for _ in range(steps)]
        for i in range(steps):
            self.lib.record(evs[i][0], self.stream)
            calls[i % len(calls)]()
            self.lib.record(evs[i][1], self.stream)
        torch.cuda.synchronize()
        per = sorted(self.lib.elapsed_ms(s, e) for s, e in evs)
        self.pcts = (per[len(per) // 10], per[(9 * len(per)) // 10])     # p10, p90 of the last run
        for s, e in evs:
            self.lib.fn["snx_hip_event_destroy"](s)
            self.lib.fn["snx_hip_event_destroy"](e)
        self.lib.fn["snx_hip_event_destroy"](a)
        self.lib.fn["snx_hip_event_destroy"](b)
        return total_ms, sum(per) / len(per), per[len(per) // 2]


_BENCHLIB = None


def bench_loops():
    """ctypes view of libsneppx_bench.so (C launch loops over the decode
    entry points); None when it is not built."""
    global _BENCHLIB
    if _BENCHLIB is None:
        path = os.path.join(REPO, "sneppx-alg_amd", "libsneppx_bench.so")
        _BENCHLIB = C.CDLL(path) if os.path.exists(path) else False
        if _BENCHLIB:
            for name in ("snxb_loop_w4a16", "snxb_loop_w4a16_actorder", "snxb_loop_w8_gemv", "snxb_loop_decode"):
                getattr(_BENCHLIB, name).restype = C.c_int
    return _BENCHLIB or None


def ptr_array(tensors):
    arr = (C.c_void_p * len(tensors))()
    for i, t in enumerate(tensors):
        arr[i] = t.data_ptr()
    return arr


def make_loop(name, *args):
    """A loop(n) that issues n calls of a decode entry point from C, or None."""
    bl = bench_loops()
    if bl is None:
        return None
    f = getattr(bl, name)
    conv = [C.c_void_p(a.data_ptr()) if hasattr(a, "data_ptr") else
            (C.c_size_t(a) if isinstance(a, int) and not isinstance(a, bool) else a) for a in args]

    def loop(n):
        if f(C.c_int(n), *conv) != 0:
            raise RuntimeError(f"{name} failed")
    return loop


def bound(lib, name, *args):
    """A zero-argument launcher for one C entry point with its arguments
    converted once (device pointers as c_void_p), so the timed loop measures
    the GPU rather than Python's argument handling; checked once here."""
    import ctypes as C
    f = lib.fn[name]
    conv = tuple(C.c_void_p(a.data_ptr()) if hasattr(a, "data_ptr") else a for a in args)
    lib.check(f(*conv), name)
    return lambda: f(*conv)


def make_w4(lib, N, K, group, copies, seed, torch):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    G = K // group
    qw = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
    sc = torch.empty((N, G), dtype=torch.int16, device="cuda")
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device="cuda")
    lib.dev_quantize_w4_awq(w, qw, sc, qz, group)
    del w
    return [(qw.clone(), sc.clone(), qz.clone()) for _ in range(copies)], G


def bench_w4a16(lib, timer, torch, M, N, K, group, copies, steps, warmup, seed=2, graph=None):
    ws, G = make_w4(lib, N, K, group, copies, seed, torch)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    st = timer.stream
    calls = [bound(lib, "SNEPPX_qlinear_w4a16", x, c[0], c[1], c[2], None, G, None, y, SNEPPX_BFLOAT16,
                   M, N, K, group, C.c_void_p(st)) for c in ws]
    qwa, sca, qza = ptr_array([c[0] for c in ws]), ptr_array([c[1] for c in ws]), ptr_array([c[2] for c in ws])
    loop = make_loop("snxb_loop_w4a16", C.c_int(len(ws)), x, qwa, sca, qza, y, C.c_int(SNEPPX_BFLOAT16),
                     M, N, K, C.c_int(group), C.c_void_p(st))
    total, mean_launch, med_launch = timer.run(calls, steps, warmup, loop, graph=_graph(graph))
    nbytes = w4_bytes(M, N, K, G)
    return {
        "bytes": nbytes, "ms_per_step": total / steps, "launch_ms_mean": mean_launch,
        "launch_ms_median": med_launch, "gbs": nbytes / (total / steps) / 1e6,
        "gbs_kernel": nbytes / mean_launch / 1e6,
    }, (ws, x, y, G)


LLAMA3_LINEARS = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}


def llama_linears(tp=1):
    """[N, K] of the Llama-3-8B layer's linears on one GPU of a tp-way
    tensor-parallel layer: QKV and gate/up column-parallel (N / tp), O and
    down row-parallel (K / tp)."""
    return {"qkv": (6144 // tp, 4096), "o": (4096, 4096 // tp), "gate_up": (28672 // tp, 4096),
            "down": (4096, 14336 // tp)}


def bench_decode(lib, timer, torch, copies, steps, warmup, layer, tp=1, graph=None):
    """One token (M = 1) through C5's Llama-3-8B linears: the gate/up
    projection with its SwiGLU step as one launch (layer False), or the
    layer's four linears back to back (QKV, O, gate/up + SwiGLU, down; the
    attention and norms between them are not part of it), weights rotated
    over `copies` copies so they stream from HBM.  tp > 1: one GPU's shard
    of a tp-way tensor-parallel layer (the reductions after O and down are
    not part of it)."""
    shapes = llama_linears(tp)
    H, QKV, A, F = 4096, shapes["qkv"][0], shapes["o"][1], shapes["gate_up"][0] // 2
    names = list(shapes) if layer else ["gate_up"]
    ws = {}
    for i, (n, (N, K)) in enumerate(shapes.items()):
        if n in names:
            ws[n], _ = make_w4(lib, N, K, 128, copies, 40 + i, torch)
    g = torch.Generator(device="cuda").manual_seed(47)
    x = torch.randn((1, H), device="cuda", generator=g).to(torch.bfloat16)
    bufs = {n: torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
            for n, N in (("qkv", QKV), ("o", H), ("h", F), ("y", H))}
    st = timer.stream
    # copy c, linear j at [4 c + j]; absent linears repeat gate/up (never read)
    flat = [ws[n][c] if n in ws else ws["gate_up"][c] for c in range(copies) for n in shapes]
    qwa, sca, qza = (ptr_array([t[i] for t in flat]) for i in range(3))
    loop = make_loop("snxb_loop_decode", C.c_int(copies), C.c_int(1 if layer else 0), x, qwa, sca, qza,
                     bufs["qkv"], bufs["o"], bufs["h"], bufs["y"], H, QKV, F, A, C.c_void_p(st))

    def step(c):
        calls = []
        gu = ws["gate_up"][c]
        if layer:
            q, o, d = ws["qkv"][c], ws["o"][c], ws["down"][c]
            calls.append(bound(lib, "SNEPPX_qlinear_w4a16", x, q[0], q[1], q[2], None, 0, None, bufs["qkv"],
                               SNEPPX_BFLOAT16, 1, QKV, H, 128, C.c_void_p(st)))
            calls.append(bound(lib, "SNEPPX_qlinear_w4a16", bufs["qkv"], o[0], o[1], o[2], None, 0, None,
                               bufs["o"], SNEPPX_BFLOAT16, 1, H, A, 128, C.c_void_p(st)))
        calls.append(bound(lib, "SNEPPX_qlinear_w4a16_swiglu", bufs["o"] if layer else x, gu[0], gu[1], gu[2],
                           None, bufs["h"], 1, F, H, 128, C.c_void_p(st)))
        if layer:
            calls.append(bound(lib, "SNEPPX_qlinear_w4a16", bufs["h"], d[0], d[1], d[2], None, 0, None,
                               bufs["y"], SNEPPX_BFLOAT16, 1, H, F, 128, C.c_void_p(st)))
        return lambda: [f() for f in calls]
    total, mean_step, _ = timer.run([step(c) for c in range(copies)], steps, warmup, loop, graph=_graph(graph))
    nbytes = sum(w4_bytes(1, N, K, K // 128) for n, (N, K) in shapes.items() if n in names)
    nbytes -= 2 * F if "gate_up" in names else 0        # gate/up writes F outputs, not 2 F
    host = {n: tuple(t.cpu() for t in ws[n][0]) for n in names}
    return {"bytes": nbytes, "ms_per_step": total / steps, "gbs": nbytes / (total / steps) / 1e6,
            "host": {"w": host, "x": _u16(x), "shapes": shapes}}


def bench_w4a16_gptq(lib, timer, torch, M, N, K, copies, steps, warmup, graph=None):
    """C3: GPTQ act-order weights, prepared once into group-contiguous column
    order (SNEPPX_qlinear_w4_actorder_prepare), then the decode linear that
    gathers the activations by the permutation."""
    g = torch.Generator(device="cuda").manual_seed(7)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(7))
    g_idx = (perm // 128).to(torch.int32).cuda()
    G = K // 128
    qw = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
    sc = torch.empty((N, G), dtype=torch.int16, device="cuda")
    lib.dev_quantize_w4_gptq(w, g_idx, G, qw, sc)
    del w
    qs = torch.empty_like(qw)
    order = torch.empty(K, dtype=torch.int16, device="cuda")
    lib.qlinear_w4_actorder_prepare(qw, g_idx, G, qs, order)
    host = {"qw": _u32(qw), "sc": _u16(sc), "g_idx": g_idx.cpu().numpy()}
    del qw
    ws = [(qs.clone(), sc.clone()) for _ in range(copies)]
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    st = timer.stream
    calls = [bound(lib, "SNEPPX_qlinear_w4a16_actorder", x, c[0], c[1], None, order, None, y,
                   SNEPPX_BFLOAT16, M, N, K, 128, C.c_void_p(st)) for c in ws]
    qwa, sca = ptr_array([c[0] for c in ws]), ptr_array([c[1] for c in ws])
    loop = make_loop("snxb_loop_w4a16_actorder", C.c_int(len(ws)), x, qwa, sca, order, y,
                     C.c_int(SNEPPX_BFLOAT16), M, N, K, C.c_int(128), C.c_void_p(st))
    total, mean_launch, _ = timer.run(calls, steps, warmup, loop, graph=_graph(graph))
    nbytes = w4_bytes(M, N, K, G, zeros=False) + K * 2      # + uint16 perm
    host["x"] = _u16(x)
    return {"bytes": nbytes, "ms_per_step": total / steps, "gbs": nbytes / (total / steps) / 1e6,
            "gbs_kernel": nbytes / mean_launch / 1e6, "host": host}


def bench_w8(lib, timer, torch, N, K, copies, steps, warmup, graph=None):
    g = torch.Generator(device="cuda").manual_seed(11)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    s = torch.empty(N, device="cuda")
    lib.dev_quantize_int8_channel(w, q, s)
    # the config text says round-half-even; the reference rounds half away
    # from zero (roundf).  Codes use the reference; count where they differ.
    q_even = torch.empty_like(q)
    s_even = torch.empty_like(s)
    lib.dev_quantize_int8_channel(w, q_even, s_even, half_even=True)
    mismatch = int((q != q_even).sum().item())
    del w, q_even, s_even
    ws = [(q.clone(), s.clone()) for _ in range(copies)]
    x = torch.randn((1, K), device="cuda", generator=g)
    y = torch.empty((1, N), device="cuda")
    st = timer.stream
    calls = [bound(lib, "SNEPPX_qlinear_w8_gemv", x, c[0], c[1], None, y, 1, N, K, C.c_void_p(st))
             for c in ws]
    loop = make_loop("snxb_loop_w8_gemv", C.c_int(len(ws)), x, ptr_array([c[0] for c in ws]),
                     ptr_array([c[1] for c in ws]), y, 1, N, K, C.c_void_p(st))
    total, mean_launch, _ = timer.run(calls, steps, warmup, loop, graph=_graph(graph))
    nbytes = N * K + N * 4 + K * 4 + N * 4
    host = {"q": q.cpu().numpy(), "s": s.cpu().numpy(), "x": x.cpu().numpy()}
    return {"bytes": nbytes, "ms_per_step": total / steps, "gbs": nbytes / (total / steps) / 1e6,
            "gbs_kernel": nbytes / mean_launch / 1e6, "codes_differing_half_even": mismatch,
            "host": host}


def bench_host_api(lib, N, K, reps=5):
    """The reference's host-pointer entry point SNEPPX_quantize_int8_channel
    (quantize_int8.c:157-177) on the C1 weight: pageable host fp32 in, host
    int8 codes + scales out, copies over PCIe included (the drop-in path a C
    caller of quantization.h gets)."""
    import numpy as np
    w = np.random.default_rng(11).normal(0, 0.02, (N, K)).astype(np.float32)
    lib.quantize_int8_channel(w)   # warm-up (first allocation)
    t0 = time.perf_counter()
    for _ in range(reps):
        rc, q, s = lib.quantize_int8_channel(w)
    per = (time.perf_counter() - t0) / reps
    return {"ms_per_call": per * 1e3, "rc": rc,
            "gbs_pcie_inclusive": (N * K * 4 + N * K + N * 4) / per / 1e9}


def bench_w8a8(lib, timer, torch, M, N, K, steps, warmup, fp8=False):
    g = torch.Generator(device="cuda").manual_seed(13)
    a32 = torch.randn((M, K), device="cuda", generator=g)
    w32 = torch.randn((N, K), device="cuda", generator=g) * 0.02
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    st = timer.stream
    if fp8:
        A = torch.empty((M, K), dtype=torch.uint8, device="cuda")
        W = torch.empty((N, K), dtype=torch.uint8, device="cuda")
        sA, sW = torch.empty(1, device="cuda"), torch.empty(1, device="cuda")
        lib.dev_quantize_fp8_e4m3_scaled(a32, A, sA)
        lib.dev_quantize_fp8_e4m3_scaled(w32, W, sW)
        calls = [lambda: lib.qlinear_w8a8_fp8(A, sA, W, sW, out, stream=st)]
    else:
        A = torch.empty((M, K), dtype=torch.int8, device="cuda")
        W = torch.empty((N, K), dtype=torch.int8, device="cuda")
        sA, sW = torch.empty(M, device="cuda"), torch.empty(N, device="cuda")
        lib.dev_quantize_int8_channel(a32, A, sA)
        lib.dev_quantize_int8_channel(w32, W, sW)
        calls = [lambda: lib.qlinear_w8a8_i8(A, sA, W, sW, out, stream=st)]
    del a32, w32
    with ClockSampler() as clk:
        total, mean_launch, _ = timer.run(calls, steps, warmup)
    ops = 2 * M * N * K
    host = {"A": A[:CPU_ROWS].cpu().numpy(), "W": W.cpu().numpy(), "sA": sA[:CPU_ROWS].cpu().numpy(),
            "sW": sW.cpu().numpy(), "M": M}
    return {"ops": ops, "ms_per_step": total / steps, "tops": ops / (total / steps) / 1e9,
            "tops_kernel": ops / mean_launch / 1e9, "host": host, "sclk_dpm_mhz_median": clk.median()}


def bench_w8a8_dyn(lib, timer, torch, M, N, K, steps, warmup, fp8=False):
    """C4 as a layer runs it: bf16 activations in, quantized inside the timed
    call (int8 per token / fp8 per tensor), the W8A8 GEMM, bf16 out."""
    g = torch.Generator(device="cuda").manual_seed(13)
    A = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w32 = torch.randn((N, K), device="cuda", generator=g) * 0.02
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    if fp8:
        W = torch.empty((N, K), dtype=torch.uint8, device="cuda")
        sW = torch.empty(1, device="cuda")
        lib.dev_quantize_fp8_e4m3_scaled(w32, W, sW)
    else:
        W = torch.empty((N, K), dtype=torch.int8, device="cuda")
        sW = torch.empty(N, device="cuda")
        lib.dev_quantize_int8_channel(w32, W, sW)
    del w32
    st = timer.stream
    Ab = A.view(torch.int16)
    total, mean_launch, _ = timer.run([lambda: lib.qlinear_w8a8_dyn(Ab, W, sW, out, fp8=fp8, stream=st)],
                                      steps, warmup)
    ops = 2 * M * N * K
    return {"ops": ops, "ms_per_step": total / steps, "tops": ops / (total / steps) / 1e9,
            "tops_kernel": ops / mean_launch / 1e9}


def bench_mx(lib, timer, torch, M, N, K, steps, warmup, fmt="mxfp4_e2m1", mfma_form=False):
    """MX x MX GEMM (f4 row): operands quantized on the GPU with the
    reference's MX rule, the product on the scaled f8f6f4 matrix cores.
    mfma_form: FP8 operands converted to the matrix cores' encoding before
    the timed region (weights kept converted); otherwise every call converts
    both operands."""
    g = torch.Generator(device="cuda").manual_seed(19)
    a = torch.randn((M, K), device="cuda", generator=g)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    pa, sa = lib.dev_quantize_mx(a, fmt)
    pw, sw = lib.dev_quantize_mx(w, fmt)
    del a, w
    if mfma_form:
        pa, sa, _ = lib.mx_to_mfma(pa, sa, M, K, fmt)
        pw, sw, _ = lib.mx_to_mfma(pw, sw, N, K, fmt)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    st = timer.stream
    if fmt == "mxfp4_e2m1" and not mfma_form:
        call = lambda: lib.qlinear_mxfp4_gemm(pa, sa, pw, sw, out, M, N, K, stream=st)
    else:
        call = lambda: lib.qlinear_mx_gemm(pa, sa, pw, sw, fmt, out, M, N, K, stream=st, mfma_form=mfma_form)
    total, mean_launch, _ = timer.run([call], steps, warmup)
    flops = 2 * M * N * K
    rb = pa.shape[1] if pa.dim() == 2 else pa.numel() // M          # code bytes per row
    per_tensor = sa.numel() == 1                                     # NVFP4: one exponent per operand
    host = {"pa": pa.reshape(M, -1)[:CPU_ROWS].cpu().numpy(),
            "sa": sa.reshape(-1).cpu().numpy() if per_tensor else sa.reshape(M, -1)[:CPU_ROWS].cpu().numpy(),
            "pw": pw.reshape(N, -1).cpu().numpy(),
            "sw": sw.reshape(-1).cpu().numpy() if per_tensor else sw.reshape(N, -1).cpu().numpy(),
            "M": M, "N": N, "K": K, "fmt": fmt, "flops": flops, "row_bytes": rb}
    return {"ms_per_step": total / steps, "tflops": flops / (total / steps) / 1e9,
            "tflops_kernel": flops / mean_launch / 1e9, "host": host}


def bench_vendor_w8a8(torch, M, N, K, steps, warmup):
    """The same C4 shape through the vendor GEMM library (hipBLASLt behind
    torch._int_mm / torch._scaled_mm), timed the same way: a reference point
    for what the hardware delivers on this shape, not part of this library."""
    out = []
    g = torch.Generator(device="cuda").manual_seed(17)
    a = torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=g)
    af = (torch.randn((M, K), device="cuda", generator=g)).to(torch.float8_e4m3fn)
    wf = (torch.randn((N, K), device="cuda", generator=g)).to(torch.float8_e4m3fn)
    one = torch.ones((), device="cuda")
    cases = [("int8 torch._int_mm", lambda: torch._int_mm(a, w.t())),
             ("fp8 e4m3 torch._scaled_mm", lambda: torch._scaled_mm(af, wf.t(), scale_a=one, scale_b=one,
                                                                    out_dtype=torch.bfloat16))]
    for name, f in cases:
        try:
            for _ in range(warmup):
                f()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                f()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            out.append({"workload": f"vendor reference (hipBLASLt, not this library): {name} M={M} N={N} K={K}",
                        "value": round(2 * M * N * K / ms / 1e9, 1), "unit": "TOPS", "ms_per_step": round(ms, 4),
                        "steps": steps, "warmup": warmup})
        except Exception as e:   # a torch build without the op: report, do not fail the bench
            out.append({"workload": f"vendor reference: {name}", "value": None, "error": str(e)[:120]})
    del a, w, af, wf
    return out


def llama_tokens(seed=5):
    """C5 ragged continuous batch: 16 decode rows + 8 prefill chunks of
    lengths uniform in [32, 512] (seeded), packed into one token matrix."""
    import numpy as np
    lens = np.random.RandomState(seed).randint(32, 513, size=8)
    return 16 + int(lens.sum()), [int(v) for v in lens]


def bench_chain(lib, timer, torch, steps, warmup, tp=1):
    """C5: one Llama-3-8B decoder layer's linears in W4A16 g128 (AWQ-style,
    random init): QKV 4096->6144, O 4096->4096, gate/up 4096->2x14336 with
    SiLU(gate)*up in the GEMM's epilogue, down 14336->4096, on T packed
    tokens; gate/up and down run as one MLP call (SNEPPX_qlinear_w4a16_mlp:
    the SwiGLU rows are written as the down projection's prepared input).
    The O input is a
    synthetic bf16 tensor (attention is not part of this path); the gate/up
    input is the O output.  tp > 1: one GPU's shard of a tp-way
    tensor-parallel layer (QKV, gate/up N / tp; O, down K / tp; the
    reductions after O and down are not part of it)."""
    T, lens = llama_tokens()
    H = 4096
    shapes = llama_linears(tp)
    F, A = shapes["gate_up"][0] // 2, shapes["o"][1]
    g = torch.Generator(device="cuda").manual_seed(17)
    ws = {}
    for name, (N, K) in shapes.items():
        w = torch.randn((N, K), device="cuda", generator=g) * 0.02
        G = K // 128
        qw = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
        sc = torch.empty((N, G), dtype=torch.int16, device="cuda")
        qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device="cuda")
        lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
        del w
        ws[name] = (qw, sc, qz, G)
    x = torch.randn((T, H), device="cuda", generator=g).to(torch.bfloat16)
    attn = torch.randn((T, A), device="cuda", generator=g).to(torch.bfloat16)
    y_qkv = torch.empty((T, shapes["qkv"][0]), dtype=torch.bfloat16, device="cuda")
    y_o = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    y_gu = torch.empty((T, 2 * F), dtype=torch.bfloat16, device="cuda")
    act = torch.empty((T, F), dtype=torch.bfloat16, device="cuda")
    y_d = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    st = timer.stream

    def lin(name, inp, out):
        qw, sc, qz, G = ws[name]
        lib.qlinear_w4a16(inp, qw, sc, qz, None, G, out, 128, stream=st)

    def gate_up_swiglu(inp, out):
        qw, sc, qz, G = ws["gate_up"]
        lib.qlinear_w4a16_swiglu(inp, qw, sc, qz, out, 128, stream=st)

    def mlp(inp, out):
        lib.qlinear_w4a16_mlp(inp, ws["gate_up"][:3], ws["down"][:3], out, 128, stream=st)

    def layer():
        lin("qkv", x, y_qkv)
        lin("o", attn, y_o)
        mlp(y_o, y_d)                      # gate/up + SiLU(gate) * up -> down

    with ClockSampler() as clk:
        total, _, _ = timer.run([layer], steps, warmup)
    per = {}
    for name, fn in (("qkv", lambda: lin("qkv", x, y_qkv)), ("o", lambda: lin("o", attn, y_o)),
                     ("gate_up+swiglu", lambda: gate_up_swiglu(y_o, act)),
                     ("down", lambda: lin("down", act, y_d))):
        t, _, _ = timer.run([fn], steps, 2)
        N, K = shapes[name.split("+")[0]]
        per[name] = {"us": round(t / steps * 1e3, 1), "tflops": round(2 * T * N * K / (t / steps) / 1e9, 1)}
    t, _, _ = timer.run([lambda: mlp(y_o, y_d)], steps, 2)
    fl = 2 * T * (shapes["gate_up"][0] * shapes["gate_up"][1] + shapes["down"][0] * shapes["down"][1])
    per["mlp (gate_up+swiglu -> down, one call)"] = {"us": round(t / steps * 1e3, 1),
                                                     "tflops": round(fl / (t / steps) / 1e9, 1)}
    # the unfused form for comparison: the [T][2F] projection in bf16, then the SwiGLU pass
    t, _, _ = timer.run([lambda: (lin("gate_up", y_o, y_gu), lib.qlinear_silu_mul(y_gu, act, stream=st))],
                        steps, 2)
    per["gate_up then silu_mul (unfused)"] = {"us": round(t / steps * 1e3, 1)}
    flops = 2 * T * sum(N * K for N, K in shapes.values())
    host = {"x": _u16(x[:2 * CPU_ROWS]), "attn": _u16(attn[:2 * CPU_ROWS]), "shapes": shapes,
            "w": {name: (_u32(qw), _u16(sc), _u32(qz)) for name, (qw, sc, qz, G) in ws.items()}}
    return {"T": T, "chunk_lens": lens, "flops": flops, "ms_per_step": total / steps,
            "sclk_dpm_mhz_median": clk.median(),
            "tflops": flops / (total / steps) / 1e9, "per_linear": per, "host": host}


CPU_ROWS = 16     # activation rows of the C4 / C5 CPU slices

SHARD_TP = 8      # the tensor-parallel degree whose per-GPU shapes the shard lines measure


def _copies_for(nbytes, floor=16):
    """Rotating weight copies that together exceed the 256 MB Infinity Cache
    with room to spare (>= 320 MB), so every call streams from HBM."""
    return max(floor, -(-320_000_000 // nbytes))


def bench_shards(lib, timer, torch, steps, warmup, tp=SHARD_TP, log=None):
    """Every config at one GPU's share of a tp-way tensor-parallel layer: the
    decode GEMVs and the W8A8 GEMM column-parallel (N / tp), the Llama-3-8B
    layer's QKV and gate/up column-parallel and O and down row-parallel
    (K / tp).  The collectives that would join the shards are not part of
    it.  Returns (extra entries, CPU jobs)."""
    out, jobs = [], []
    tag = f"TP={tp} shard: "
    # The shard's decode kernels (0.7-8 MB, 3-4 us) are shorter than the
    # host's ~3 us launch path, so launched one by one they time the host.
    # A decode loop runs such steps as a captured HIP graph: the value is one
    # graph replay of the timed steps; the eager figure stays beside it.
    how = " (HIP graph replay)"

    def both(fn, *a, **kw):
        r = fn(*a, graph=True, **kw)
        r_eager = fn(*a, graph=False, **kw)
        r0 = r_eager[0] if isinstance(r_eager, tuple) else r_eager
        return r, round(r0["gbs"], 1)
    N2, K = 11008 // tp, 4096
    for m in (1, 16):
        cp = _copies_for(w4_bytes(m, N2, K, K // 128))
        (r, (ws_m, x_m, _, _)), eager = both(bench_w4a16, lib, timer, torch, m, N2, K, 128, cp, steps, warmup)
        out.append({"workload": f"{tag}C2 W4A16 g128 GEMV N={N2} K={K} M={m}{how}", "value": round(r["gbs"], 1),
                    "unit": "GB/s", "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4), "eager_gbs": eager,
                    "kernel_gbs": round(r["gbs_kernel"], 1), "ms_per_step": round(r["ms_per_step"], 5),
                    "weight_copies": cp})
        jobs.append((out[-1], "w4", {"qw": _u32(ws_m[0][0]), "sc": _u16(ws_m[0][1]), "qz": _u32(ws_m[0][2]),
                                     "x": _u16(x_m), "bytes": r["bytes"]}))
        del ws_m, x_m
    cp = _copies_for(w4_bytes(1, N2, K, K // 128, zeros=False))
    r, eager = both(bench_w4a16_gptq, lib, timer, torch, 1, N2, K, cp, steps, warmup)
    out.append({"workload": f"{tag}C3 GPTQ act-order W4A16 (prepared) N={N2} K={K} M=1{how}",
                "value": round(r["gbs"], 1), "unit": "GB/s", "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
                "eager_gbs": eager, "kernel_gbs": round(r["gbs_kernel"], 1),
                "ms_per_step": round(r["ms_per_step"], 5), "weight_copies": cp})
    jobs.append((out[-1], "w4_gidx", dict(r["host"], bytes=r["bytes"])))
    N1 = 4096 // tp
    cp = _copies_for(N1 * K)
    r, eager = both(bench_w8, lib, timer, torch, N1, K, cp, steps, warmup)
    out.append({"workload": f"{tag}C1 W8 weight-only GEMV N={N1} K={K} M=1 fp32{how}", "value": round(r["gbs"], 1),
                "unit": "GB/s", "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4), "eager_gbs": eager,
                "kernel_gbs": round(r["gbs_kernel"], 1), "ms_per_step": round(r["ms_per_step"], 5),
                "weight_copies": cp})
    jobs.append((out[-1], "w8", r["host"]))
    sh = llama_linears(tp)
    for layer in (False, True):
        per_copy = sum(w4_bytes(1, N, K_, K_ // 128) for n, (N, K_) in sh.items() if layer or n == "gate_up")
        cp = _copies_for(per_copy)
        r, eager = both(bench_decode, lib, timer, torch, cp, steps, warmup, layer, tp=tp)
        what = ("Llama-3-8B layer linears at decode (QKV {qkv[0]}x{qkv[1]}, O {o[0]}x{o[1]}, gate/up "
                "{gate_up[0]}x{gate_up[1]} + SwiGLU fused, down {down[0]}x{down[1]}; 4 launches)".format(**sh)
                if layer else f"Llama-3-8B gate/up projection + SwiGLU fused, one launch "
                              f"(F={sh['gate_up'][0] // 2}, K={sh['gate_up'][1]})")
        out.append({"workload": f"{tag}{what} W4A16 g128 M=1{how}", "value": round(r["gbs"], 1), "unit": "GB/s",
                    "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4), "eager_gbs": eager, "bytes": r["bytes"],
                    "ms_per_step": round(r["ms_per_step"], 5), "weight_copies": cp})
        jobs.append((out[-1], "decode", dict(r["host"], bytes=r["bytes"], layer=layer)))
    r = bench_chain(lib, timer, torch, 10, 30, tp=tp)
    out.append({"workload": f"{tag}C5 Llama-3-8B layer W4A16 g128 linear chain T={r['T']}",
                "value": round(r["tflops"], 1), "unit": "TFLOP/s",
                "frac_of_peak": round(r["tflops"] / BF16_PEAK_TFLOPS, 4),
                "ms_per_step": round(r["ms_per_step"], 4), "steps": 10, "warmup": 30,
                "per_linear": r["per_linear"]})
    jobs.append((out[-1], "chain", dict(r["host"], T=r["T"], flops=r["flops"])))
    N4 = 14336 // tp
    for fp8 in (False, True):
        r = bench_w8a8(lib, timer, torch, 2048, N4, 4096, GEMM_STEPS, GEMM_WARMUP, fp8=fp8)
        peak = FP8_PEAK_TOPS if fp8 else INT8_PEAK_TOPS
        out.append({"workload": f"{tag}C4 W8A8 {'fp8 e4m3' if fp8 else 'int8'} GEMM M=2048 N={N4} K=4096",
                    "value": round(r["tops"], 1), "unit": "TOPS", "frac_of_peak": round(r["tops"] / peak, 4),
                    "ms_per_step": round(r["ms_per_step"], 4), "steps": GEMM_STEPS, "warmup": GEMM_WARMUP})
        jobs.append((out[-1], "fp8" if fp8 else "i8", r["host"]))
    if log:
        for e in out:
            log(f"[bench] {e['workload']}: {e['value']} {e['unit']} ({e['frac_of_peak']})")
    return out, jobs


def _u32(t):
    import numpy as np
    return t.cpu().numpy().view(np.uint32)


def _u16(t):
    import numpy as np
    import torch
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _bf16_np(a):
    """float32 -> bf16 bits, round to nearest even (the GPU's output rounding)."""
    import numpy as np
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def _per_call(fn, seconds, max_reps=200):
    """Seconds per call of fn(), repeated for about `seconds` (at least once)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            return el / reps, reps, el


def _cpu_entry(value, unit, sample, kind="port"):
    return {"value": value, "unit": unit, "cores": 1, "kind": kind, "sample": sample,
            "build": "oracle/liboracle_perf.so (-O3 -march=x86-64-v3), one thread"}


def cpu_legs(orc, jobs, seconds):
    """The oracle's C restatement of the reference CPU path for every extra
    config (dequantise, then the k-ascending fp32 dot of tensor.c:1820-1823),
    one host thread; each job fills the `cpu_baseline` of its extra entry."""
    import numpy as np
    for entry, kind, h in jobs:
        if kind == "w8":                       # C1, full shape
            per, reps, el = _per_call(lambda: orc.w8_linear(h["x"], h["q"], h["s"]), seconds)
            N, K = h["q"].shape
            nbytes = N * K + N * 4 + K * 4 + N * 4
            entry["cpu_baseline"] = _cpu_entry(round(nbytes / per / 1e9, 3), "GB/s",
                                               f"full C1 shape, {reps} calls in {el:.1f} s ({per * 1e3:.2f} ms/call)")
        elif kind in ("w4", "w4_gidx"):         # C2 / C3, full shape
            N = h["qw"].shape[0]
            K = h["qw"].shape[1] * 8
            gi = h.get("g_idx")
            per, reps, el = _per_call(lambda: orc.w4a16_linear(h["x"], h["qw"], h["sc"], h.get("qz"), gi,
                                                               N, K, 128), seconds)
            entry["cpu_baseline"] = _cpu_entry(round(h["bytes"] / per / 1e9, 4), "GB/s",
                                               f"full shape M={h['x'].shape[0]}, {reps} calls in {el:.1f} s "
                                               f"({per * 1e3:.1f} ms/call)")
        elif kind in ("i8", "fp8"):            # C4: rows of A, extrapolated to M
            A, W, M = h["A"], h["W"], h["M"]
            N, K = W.shape
            if kind == "i8":
                a_deq = (A.astype(np.float32) * h["sA"][:, None]).astype(np.float32)   # (float)q * s
                fn = lambda: orc.w8_linear(a_deq, W, h["sW"])                          # noqa: E731
            else:
                fn = lambda: orc.fp8_gemm(A, W, np.float32(h["sA"][0]), np.float32(h["sW"][0]))  # noqa: E731
            per, reps, el = _per_call(fn, seconds, max_reps=3)
            full = per * M / A.shape[0]
            entry["cpu_baseline"] = _cpu_entry(round(2 * M * N * K / full / 1e12, 6), "TOPS",
                                               f"{A.shape[0]} of {M} rows of A against all of W, "
                                               f"{per:.2f} s per slice, extrapolated linearly to M={M} "
                                               f"({full:.0f} s per call)")
        elif kind == "decode":                 # C5 linears at M = 1 (full or one shard's shapes)
            w = {n: (v[0].numpy().view(np.uint32), v[1].numpy().view(np.uint16), v[2].numpy().view(np.uint32))
                 for n, v in h["w"].items()}
            sh = h["shapes"]

            def token():
                xs = h["x"]
                if h["layer"]:
                    rc, q = orc.w4a16_linear(xs, *w["qkv"], None, *sh["qkv"], 128)
                    xs = _bf16_np(q[:, :sh["o"][1]])
                    rc, o = orc.w4a16_linear(xs, *w["o"], None, *sh["o"], 128)
                    xs = _bf16_np(o)
                rc, gu = orc.w4a16_linear(xs, *w["gate_up"], None, *sh["gate_up"], 128)
                F = sh["gate_up"][0] // 2
                g = gu[:, :F]
                with np.errstate(over="ignore"):
                    act = _bf16_np((g / (np.float32(1) + np.exp(-g)) * gu[:, F:]).astype(np.float32))
                if h["layer"]:
                    orc.w4a16_linear(act, *w["down"], None, *sh["down"], 128)
            per, reps, el = _per_call(token, seconds, max_reps=20)
            entry["cpu_baseline"] = _cpu_entry(round(h["bytes"] / per / 1e9, 4), "GB/s",
                                               f"the same shapes M=1, {reps} calls in {el:.1f} s "
                                               f"({per * 1e3:.1f} ms/call)")
        elif kind == "mx":                     # MX GEMM: decode W once, rows of A extrapolated
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import mx_oracle
            from threadpoolctl import threadpool_limits
            M, N, K, fmt, r = h["M"], h["N"], h["K"], h["fmt"], h["pa"].shape[0]
            nw = min(N, 512)                   # rows of W decoded (the numpy bit unpack is slow)
            with threadpool_limits(limits=1):
                t0 = time.perf_counter()
                sw_rows = h["sw"] if h["sw"].size == 1 else h["sw"][:nw]     # per-tensor NVFP4: one exponent
                wd = mx_oracle.dequantize(h["pw"][:nw].reshape(-1), sw_rows.reshape(-1), (nw, K),
                                          fmt).astype(np.float32)
                t_w = time.perf_counter() - t0
                t0 = time.perf_counter()
                ad = mx_oracle.dequantize(h["pa"].reshape(-1), h["sa"].reshape(-1), (r, K), fmt).astype(np.float32)
                ad @ wd.T
                t_rows = time.perf_counter() - t0
            full = (t_w + t_rows * M / r) * N / nw
            entry["cpu_baseline"] = _cpu_entry(round(h["flops"] / full / 1e12, 6), "TFLOP/s",
                                               f"numpy oracle dequantize of {nw} rows of W ({t_w:.1f} s) + {r} rows "
                                               f"of A dequantized and multiplied with them in fp32 ({t_rows:.2f} s), "
                                               f"extrapolated linearly to M={M}, N={N} ({full:.0f} s per call)")
            entry["cpu_baseline"]["build"] = "oracle/mx_oracle.py (numpy), BLAS limited to one thread"
        elif kind == "chain":                  # C5: token slices, extrapolated to T
            shapes, w = h["shapes"], h["w"]

            def layer(rows):
                xs, at = h["x"][:rows], h["attn"][:rows]
                for name, inp in (("qkv", xs), ("o", at)):
                    N, K = shapes[name]
                    orc.w4a16_linear(inp, *w[name], None, N, K, 128)
                N, K = shapes["gate_up"]
                rc, gu = orc.w4a16_linear(xs, *w["gate_up"], None, N, K, 128)
                F = N // 2
                g = gu[:, :F]
                with np.errstate(over="ignore"):
                    act = (g / (np.float32(1) + np.exp(-g)) * gu[:, F:]).astype(np.float32)
                ab = act.view(np.uint32)
                ab = ((ab + 0x7FFF + ((ab >> 16) & 1)) >> 16).astype(np.uint16)   # bf16, as the GPU chain
                N, K = shapes["down"]
                orc.w4a16_linear(ab, *w["down"], None, N, K, 128)
            lo, hi = CPU_ROWS // 2, CPU_ROWS
            t_lo, _, _ = _per_call(lambda: layer(lo), 0.0, max_reps=1)
            t_hi, _, _ = _per_call(lambda: layer(hi), 0.0, max_reps=1)
            T = h["T"]
            full = t_lo + (T - lo) * (t_hi - t_lo) / (hi - lo)
            entry["cpu_baseline"] = _cpu_entry(round(h["flops"] / full / 1e12, 6), "TFLOP/s",
                                               f"the layer on {lo} and {hi} tokens ({t_lo:.2f} / {t_hi:.2f} s), "
                                               f"extrapolated linearly to T={T} ({full:.0f} s per layer)")


def cpu_baseline(ws_host, x_host, N, K, group, seconds):
    """The oracle's C restatement (C2 GEMV: dequantise + k-ascending fp32 dot,
    the reference tensor.c:1820-1823 order), one host thread, -O3.  Also times
    the restated SNEPPX_quantize_int8_channel on the C1 weight (the host API
    function the drop-in replaces), for the PCIe-inclusive comparison."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    from py_oracle import Oracle
    orc = Oracle(perf=True)
    qw, sc, qz = ws_host
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.w4a16_linear(x_host, qw, sc, qz, None, N, K, group)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 200:
            break
    per = el / reps
    nbytes = w4_bytes(1, N, K, K // group)
    # the same restatement on every host thread, rows split evenly (a labelled
    # second figure; the reference path itself is single-threaded)
    import threading
    nth = max(1, min(16, os.cpu_count() or 1))
    bounds = [N * i // nth for i in range(nth + 1)]

    def part(i):
        lo, hi = bounds[i], bounds[i + 1]
        orc.w4a16_linear(x_host, qw[lo:hi], sc[lo:hi], qz[lo:hi], None, hi - lo, K, group)

    treps, t0 = 0, time.perf_counter()
    while True:
        ths = [threading.Thread(target=part, args=(i,)) for i in range(nth)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        treps += 1
        tel = time.perf_counter() - t0
        if tel >= seconds / 3 or treps >= 200:
            break
    w = np.random.default_rng(11).normal(0, 0.02, (4096, 4096)).astype(np.float32)
    t1 = time.perf_counter()
    for _ in range(3):
        orc.quantize_int8_channel(w)
    q_ms = (time.perf_counter() - t1) / 3 * 1e3
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"full C2 shape N={N} K={K} M=1, {reps} calls in {el:.1f} s "
                      f"({per * 1e3:.1f} ms/call), oracle/liboracle_perf.so (-O3 -march=x86-64-v3)",
            "quantize_int8_channel_4096x4096_ms": round(q_ms, 2),
            "restatement_threads": {"value": round(nbytes / (tel / treps) / 1e9, 3), "unit": "GB/s",
                                    "cores": nth, "sample": f"rows split over {nth} host threads, "
                                                            f"{treps} calls in {tel:.1f} s"},
            "host_cpu": _cpu_name(), "host_threads_available": os.cpu_count()}


def load_traffic(kernel):
    """HBM bytes per dispatch of `kernel` from profiles/traffic.json (written
    from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes, calibrated on a copy
    of known size); None when absent."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    if not rec:
        return None
    return int(rec["fetch_bytes"] + rec["write_bytes"])


def intercept_fit(lib, timer, torch, steps, warmup, K=4096):
    """Per-launch time of the M = 1 W4A16 GEMV (k_w4a16_gemv1) at six sizes
    of N, and of a plain streaming read of the same bytes in the GEMV's
    access shape (stream_read.hip: 16-byte nontemporal loads, 1 KB per wave
    instruction, four per thread in flight, no arithmetic), each rotating
    over enough copies to stream from HBM; least-squares fits
    t = a + bytes / bw.  The intercept a is what a launch costs beyond its
    bytes; the GEMV's minus the read's is what its own work adds.  The GEMV
    is timed eagerly (launched from C) and as a graph replay, the read as a
    graph replay."""
    import numpy as np
    bl = bench_loops()
    bl.snxb_stream_read.restype = C.c_int
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    rows = []
    for N in (2048, 4096, 8192, 11008, 16384, 28672):
        nbytes = w4_bytes(1, N, K, K // 128)
        cp = _copies_for(nbytes)
        r, (ws, x, y, G) = bench_w4a16(lib, timer, torch, 1, N, K, 128, cp, steps, warmup, graph=False)
        rg, _ = bench_w4a16(lib, timer, torch, 1, N, K, 128, cp, steps, warmup, graph=True)
        del ws, x, y
        rb = nbytes // 16 * 16
        bufs = [torch.ones(rb // 4, dtype=torch.int32, device="cuda") for _ in range(cp)]
        st = C.c_void_p(timer.stream)
        calls = [lambda b=b: bl.snxb_stream_read(C.c_void_p(b.data_ptr()), C.c_size_t(rb),
                                                 C.c_void_p(sink.data_ptr()), st) for b in bufs]
        t_read, _, _ = timer.run(calls, steps, warmup, graph=True)
        del bufs
        rows.append({"N": N, "bytes": nbytes, "copies": cp, "gemv_us": round(r["ms_per_step"] * 1e3, 3),
                     "gemv_graph_us": round(rg["ms_per_step"] * 1e3, 3),
                     "read_graph_us": round(t_read / steps * 1e3, 3)})
    b = np.array([r["bytes"] for r in rows], np.float64)
    out = {"K": K, "steps": steps, "rows": rows}
    for key in ("gemv_us", "gemv_graph_us", "read_graph_us"):
        t = np.array([r[key] for r in rows], np.float64)
        slope, icpt = np.polyfit(b, t, 1)
        out[key.replace("_us", "_fit")] = {"intercept_us": round(float(icpt), 3),
                                           "bw_tbs": round(float(1e-6 / slope), 3),
                                           "max_resid_us": round(float(np.abs(t - (icpt + slope * b)).max()), 3)}
    return out


def run_only(args, lib, timer, torch, N, K, group):
    """One kernel family, for profiler passes (prints one line, no JSON)."""
    steps = args.steps
    if args.only == "gemv":
        r, _ = bench_w4a16(lib, timer, torch, args.m, N, K, group, args.copies, steps, args.warmup)
        print(f"gemv C2 M={args.m}: {r['ms_per_step'] * 1e3:.3f} us/launch, {r['gbs']:.0f} GB/s")
    elif args.only == "fit":
        print(json.dumps(intercept_fit(lib, timer, torch, steps, args.warmup)), flush=True)
    elif args.only == "gemm-dyn":
        for fp8 in (False, True):
            r = bench_w8a8_dyn(lib, timer, torch, 2048, 14336, 4096, steps, args.warmup, fp8=fp8)
            print(f"gemm-{'fp8' if fp8 else 'i8'} from bf16 A: {r['ms_per_step'] * 1e3:.1f} us/call, "
                  f"{r['tops']:.0f} TOPS")
    elif args.only in ("gemm-i8", "gemm-fp8"):
        r = bench_w8a8(lib, timer, torch, 2048, 14336, 4096, steps, args.warmup, fp8=args.only == "gemm-fp8")
        print(f"{args.only}: {r['ms_per_step'] * 1e3:.1f} us/launch, {r['tops']:.0f} TOPS")
    elif args.only == "gemm-w4":
        # the chain's widest linear alone (gate/up, 4096 -> 2 x 14336)
        T, _ = llama_tokens()
        N2, K2 = 28672, 4096
        w = torch.randn((N2, K2), device="cuda") * 0.02
        qw = torch.empty((N2, K2 // 8), dtype=torch.int32, device="cuda")
        sc = torch.empty((N2, K2 // 128), dtype=torch.int16, device="cuda")
        qz = torch.empty((N2, K2 // 1024), dtype=torch.int32, device="cuda")
        lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
        del w
        x = torch.randn((T, K2), device="cuda").to(torch.bfloat16)
        y = torch.empty((T, N2), dtype=torch.bfloat16, device="cuda")
        st = timer.stream
        t, _, _ = timer.run([lambda: lib.qlinear_w4a16(x, qw, sc, qz, None, K2 // 128, y, 128, stream=st)], steps, 2)
        print(f"gemm-w4 T={T} N={N2} K={K2}: {t / steps * 1e3:.1f} us, {2 * T * N2 * K2 / (t / steps) / 1e9:.0f} TFLOP/s")
    elif args.only == "decode":
        for layer in (False, True):
            r = bench_decode(lib, timer, torch, 4 if layer else 8, steps, args.warmup, layer)
            print(f"decode {'layer' if layer else 'gate/up+swiglu'}: {r['ms_per_step'] * 1e3:.2f} us, "
                  f"{r['gbs']:.0f} GB/s ({r['gbs'] / HBM_PEAK_GBS:.3f})")
    elif args.only == "mx":
        for fmt in MX_BENCH:
            r = bench_mx(lib, timer, torch, 2048, 14336, 4096, steps, args.warmup, fmt)
            print(f"{fmt} gemm: {r['ms_per_step'] * 1e3:.1f} us, {r['tflops']:.0f} TFLOP/s")
    elif args.only == "shard":
        bench_shards(lib, timer, torch, max(50, steps // 4), 10,
                     log=lambda t: print(t, flush=True))
    elif args.only == "chain":
        r = bench_chain(lib, timer, torch, steps, 2)
        print(f"chain T={r['T']}: {r['ms_per_step'] * 1e3:.0f} us, {r['tflops']:.0f} TFLOP/s {r['per_linear']}")
    else:
        # a plain device copy of known size, the calibration for FETCH/WRITE_SIZE
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {steps} x {n} bytes")


def _gpu_sclk_mhz():
    """Current shader clock of the first GPU from sysfs (the line marked '*'
    of pp_dpm_sclk), or None where the file is absent or unreadable."""
    import glob
    for path in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
        try:
            for line in open(path):
                if line.rstrip().endswith("*"):
                    return int("".join(ch for ch in line.split(":", 1)[1] if ch.isdigit()))
        except (OSError, ValueError, IndexError):
            continue
    return None


class ClockSampler:
    """Median shader clock level (MHz) the driver reports in sysfs
    (pp_dpm_sclk, the active DPM level) over a timed region, sampled every
    2 ms from a host thread; None where sysfs gives no reading.  The level
    is the clock requested, not the effective clock under the power limit,
    which the SQ counters give (CU-busy cycles / kernel time)."""

    def __enter__(self):
        import threading
        self.samples, self._stop = [], False

        def run():
            while not self._stop:
                c = _gpu_sclk_mhz()
                if c:
                    self.samples.append(c)
                time.sleep(0.002)
        self._t = threading.Thread(target=run, daemon=True)
        self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop = True
        self._t.join()

    def median(self):
        if not self.samples:
            return None
        v = sorted(self.samples)
        return v[len(v) // 2]


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only: the quantized GEMV/GEMM "
                                   "path has no collective step; run with --gpus 1"}))
        sys.exit(2)
    import torch
    import sneppx_quant
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    lib = sneppx_quant.load()
    arch, cus, clk = lib.device_info()
    # one stream of our own (default priority) for every launch: a graph
    # cannot be captured on the null stream
    bench_stream = torch.cuda.Stream()
    torch.cuda.set_stream(bench_stream)
    stream = bench_stream.cuda_stream
    timer = Timer(lib, stream)

    N, K, group, M = 11008, 4096, 128, 1
    if args.only:
        global DECODE_GRAPH
        DECODE_GRAPH = args.graph
        run_only(args, lib, timer, torch, N, K, group)
        return
    head, keep = bench_w4a16(lib, timer, torch, M, N, K, group, args.copies, args.steps, args.warmup)
    head_pcts, head_sclk = timer.pcts, _gpu_sclk_mhz()
    print(f"[bench] C2 M=1: {head['gbs']:.0f} GB/s whole-job, kernel {head['launch_ms_mean'] * 1e3:.2f} us",
          file=sys.stderr, flush=True)

    extra, cpu_jobs, gemm = [], [], {}
    if not args.no_extra:
        for m in (4, 16):
            r, (ws_m, x_m, _, _) = bench_w4a16(lib, timer, torch, m, N, K, group, args.copies,
                                               max(50, args.steps // 4), 10)
            extra.append({"workload": f"C2 W4A16 g128 GEMV N={N} K={K} M={m}", "value": round(r["gbs"], 1),
                          "unit": "GB/s", "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
                          "kernel_gbs": round(r["gbs_kernel"], 1), "ms_per_step": round(r["ms_per_step"], 5)})
            cpu_jobs.append((extra[-1], "w4", {"qw": _u32(ws_m[0][0]), "sc": _u16(ws_m[0][1]),
                                               "qz": _u32(ws_m[0][2]), "x": _u16(x_m), "bytes": r["bytes"]}))
            del ws_m, x_m
        for m in (1, 8):
            r = bench_w4a16_gptq(lib, timer, torch, m, N, K, args.copies, max(50, args.steps // 4), 10)
            extra.append({"workload": f"C3 GPTQ act-order W4A16 (prepared) N={N} K={K} M={m}",
                          "value": round(r["gbs"], 1), "unit": "GB/s",
                          "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
                          "kernel_gbs": round(r["gbs_kernel"], 1), "ms_per_step": round(r["ms_per_step"], 5)})
            cpu_jobs.append((extra[-1], "w4_gidx", dict(r["host"], bytes=r["bytes"])))
        for layer in (False, True):
            r = bench_decode(lib, timer, torch, 4 if layer else 8, max(50, args.steps // 4), 10, layer)
            what = ("Llama-3-8B layer linears at decode (QKV, O, gate/up + SwiGLU fused, down; "
                    "4 launches, attention and norms excluded)" if layer else
                    "Llama-3-8B gate/up projection + SwiGLU fused, one launch (F=14336, K=4096)")
            extra.append({"workload": f"{what} W4A16 g128 M=1", "value": round(r["gbs"], 1), "unit": "GB/s",
                          "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4), "bytes": r["bytes"],
                          "ms_per_step": round(r["ms_per_step"], 5)})
            cpu_jobs.append((extra[-1], "decode", dict(r["host"], bytes=r["bytes"], layer=layer)))
            print(f"[bench] {what}: {r['gbs']:.0f} GB/s, {r['ms_per_step'] * 1e3:.2f} us",
                  file=sys.stderr, flush=True)
        # the headline kernel with one weight copy, which stays in the 256 MB
        # Infinity Cache between calls: what the launch and the kernel cost
        # when HBM is not the limit (labelled; not the metric)
        r, _ = bench_w4a16(lib, timer, torch, 1, N, K, group, 1, max(50, args.steps // 4), 10)
        extra.append({"workload": f"C2 W4A16 g128 GEMV N={N} K={K} M=1, one weight copy resident in the "
                                  "Infinity Cache (cache-hot, not HBM-bound; the headline rotates 16 copies)",
                      "value": round(r["gbs"], 1), "unit": "GB/s", "ms_per_step": round(r["ms_per_step"], 5)})
        print(f"[bench] C2 M=1 cache-hot: {r['gbs']:.0f} GB/s, {r['ms_per_step'] * 1e3:.2f} us",
              file=sys.stderr, flush=True)
        r = bench_w8(lib, timer, torch, 4096, 4096, 20, max(50, args.steps // 4), 10)
        extra.append({"workload": "C1 W8 weight-only GEMV N=4096 K=4096 M=1 fp32", "value": round(r["gbs"], 1),
                      "unit": "GB/s", "frac_of_peak": round(r["gbs"] / HBM_PEAK_GBS, 4),
                      "kernel_gbs": round(r["gbs_kernel"], 1), "ms_per_step": round(r["ms_per_step"], 5),
                      "codes_differing_half_even": r["codes_differing_half_even"]})
        cpu_jobs.append((extra[-1], "w8", r["host"]))
        h = bench_host_api(lib, 4096, 4096)
        extra.append({"workload": "host API SNEPPX_quantize_int8_channel 4096x4096 (host buffers, PCIe included)",
                      "value": round(h["ms_per_call"], 3), "unit": "ms", "higher_is_better": False,
                      "gbs_pcie_inclusive": round(h["gbs_pcie_inclusive"], 2)})
        r = bench_chain(lib, timer, torch, 10, 30)
        extra.append({"workload": f"C5 Llama-3-8B layer W4A16 g128 linear chain T={r['T']} "
                                  f"(16 decode + 8 prefill chunks {r['chunk_lens']})",
                      "value": round(r["tflops"], 1), "unit": "TFLOP/s",
                      "frac_of_peak": round(r["tflops"] / BF16_PEAK_TFLOPS, 4),
                      "ms_per_step": round(r["ms_per_step"], 4), "steps": 10, "warmup": 30,
                      "sclk_dpm_mhz_median": r["sclk_dpm_mhz_median"], "per_linear": r["per_linear"]})
        cpu_jobs.append((extra[-1], "chain", dict(r["host"], T=r["T"], flops=r["flops"])))
        print(f"[bench] C5 chain T={r['T']}: {r['ms_per_step'] * 1e3:.0f} us, {r['tflops']:.0f} TFLOP/s",
              file=sys.stderr, flush=True)
        for fp8 in (False, True):
            r = bench_w8a8(lib, timer, torch, 2048, 14336, 4096, GEMM_STEPS, GEMM_WARMUP, fp8=fp8)
            peak = FP8_PEAK_TOPS if fp8 else INT8_PEAK_TOPS
            kind = "fp8" if fp8 else "int8"
            extra.append({"workload": f"C4 W8A8 {'fp8 e4m3' if fp8 else 'int8'} GEMM M=2048 N=14336 K=4096",
                          "value": round(r["tops"], 1), "unit": "TOPS",
                          "frac_of_peak": round(r["tops"] / peak, 4), "ms_per_step": round(r["ms_per_step"], 4),
                          "kernel_tops": round(r["tops_kernel"], 1), "steps": GEMM_STEPS, "warmup": GEMM_WARMUP,
                          "sclk_dpm_mhz_median": r["sclk_dpm_mhz_median"]})
            gemm[kind] = dict(r, peak=peak, line=extra[-1])
            cpu_jobs.append((extra[-1], "fp8" if fp8 else "i8", r["host"]))
            print(f"[bench] C4 W8A8 {kind} GEMM M=2048 N=14336 K=4096: {r['tops']:.0f} TOPS "
                  f"({r['tops'] / peak:.4f} of {peak:.0f}), {r['ms_per_step'] * 1e3:.1f} us/launch",
                  file=sys.stderr, flush=True)
        for fp8 in (False, True):
            r = bench_w8a8_dyn(lib, timer, torch, 2048, 14336, 4096, GEMM_STEPS, GEMM_WARMUP, fp8=fp8)
            peak = FP8_PEAK_TOPS if fp8 else INT8_PEAK_TOPS
            kind = "fp8" if fp8 else "int8"
            rule = "per tensor" if fp8 else "per token"
            extra.append({"workload": f"C4 W8A8 {'fp8 e4m3' if fp8 else 'int8'} M=2048 N=14336 K=4096 from bf16 A "
                                      f"(A quantized {rule} inside the timed call, bf16 out)",
                          "value": round(r["tops"], 1), "unit": "TOPS", "frac_of_peak": round(r["tops"] / peak, 4),
                          "ms_per_step": round(r["ms_per_step"], 4), "steps": GEMM_STEPS, "warmup": GEMM_WARMUP})
            gemm[kind]["dyn_tops"] = r["tops"]
            gemm[kind]["dyn_us"] = r["ms_per_step"] * 1e3
            print(f"[bench] C4 W8A8 {kind} from bf16 A (quantized {rule} in the call): {r['tops']:.0f} TOPS "
                  f"({r['tops'] / peak:.4f}), {r['ms_per_step'] * 1e3:.1f} us/call", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        extra.extend(bench_vendor_w8a8(torch, 2048, 14336, 4096, GEMM_STEPS, GEMM_WARMUP))
        for fmt, peak in MX_BENCH.items():
            for kept in ((False, True) if fmt.startswith("mxfp8") else (False,)):
                r = bench_mx(lib, timer, torch, 2048, 14336, 4096, GEMM_STEPS, GEMM_WARMUP, fmt, mfma_form=kept)
                how = ("operands kept in matrix-core form" if kept else
                       "both operands converted every call" if fmt.startswith("mxfp8") else
                       "per-tensor exponents fed to every 32-block" if fmt.startswith("nvfp4") else
                       "reference MX encoding")
                extra.append({"workload": f"{fmt.upper()} GEMM M=2048 N=14336 K=4096 ({how}, bf16 out)",
                              "value": round(r["tflops"], 1), "unit": "TFLOP/s",
                              "frac_of_peak": round(r["tflops"] / peak, 4),
                              "ms_per_step": round(r["ms_per_step"], 4), "steps": GEMM_STEPS,
                              "warmup": GEMM_WARMUP})
                print(f"[bench] {extra[-1]['workload']}: {r['tflops']:.0f} TFLOP/s", file=sys.stderr, flush=True)
                if not kept:
                    cpu_jobs.append((extra[-1], "mx", r["host"]))
        # one GPU's share of a tensor-parallel layer (the collectives are not part of it)
        shard, shard_jobs = bench_shards(lib, timer, torch, max(50, args.steps // 4), 10,
                                         log=lambda t: print(t, file=sys.stderr, flush=True))
        extra.extend(shard)
        cpu_jobs.extend(shard_jobs)

    cpu = None
    if not args.no_cpu:
        ws, x, y, G = keep
        qw, sc, qz = ws[0]
        import numpy as np
        host = (qw.cpu().numpy().view(np.uint32), sc.cpu().numpy().view(np.uint16),
                qz.cpu().numpy().view(np.uint32))
        xh = x.cpu().view(torch.int16).numpy().view(np.uint16)
        cpu = cpu_baseline(host, xh, N, K, group, args.cpu_seconds)
        print(f"[bench] CPU baseline C2: {cpu['value']} GB/s", file=sys.stderr, flush=True)
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        from py_oracle import Oracle
        cpu_legs(Oracle(perf=True), cpu_jobs, min(3.0, args.cpu_seconds))
        print(f"[bench] CPU legs done ({len(cpu_jobs)} configs)", file=sys.stderr, flush=True)
        for kind, g in gemm.items():
            cb = g["line"].get("cpu_baseline") or {}
            print(f"[bench] CPU baseline C4 {kind}: {cb.get('value')} {cb.get('unit')} ({cb.get('sample')})",
                  file=sys.stderr, flush=True)

    # per-launch duration = back-to-back time / launches (>= kernel time; it
    # matches rocprofv3's kernel-trace average to within the launch gap)
    achieved = head["bytes"] / head["ms_per_step"] / 1e6
    traffic = load_traffic("k_w4a16_gemv1")
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn N(0,0.02) weights quantized on the GPU, N(0,1) bf16 activations)",
        "config": {"workload": "C2 W4A16 AWQ-style g128 decode GEMV", "N": N, "K": K, "M": M,
                   "group": group, "weight_copies": args.copies,
                   "bytes_per_step": head["bytes"], "device": arch, "cus": cus,
                   "seeds": {"weights": 2, "activations": 3}, "gpu_clock_max_mhz": clk // 1000,
                   "gpu_sclk_mhz_after_run": head_sclk},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_w4a16_gemv1", "algorithmic_bytes": head["bytes"],
                     "launch_us": round(head["ms_per_step"] * 1e3, 3),
                     "event_pair_us_median": round(head["launch_ms_median"] * 1e3, 3),
                     "event_pair_us_p10_p90": [round(head_pcts[0] * 1e3, 3), round(head_pcts[1] * 1e3, 3)]},
        "cpu_baseline": cpu,
        "roofline_gemm": roofline_gemm(gemm),
        "extra": extra,
    }
    # the metric's second half (C4 W8A8 at M=2048) as flat scalars of the
    # headline roofline too, next to the GEMV figures
    for kind, g in gemm.items():
        line["roofline"][f"c4_{kind}_tops"] = round(g["tops"], 1)
        line["roofline"][f"c4_{kind}_frac"] = round(g["tops"] / g["peak"], 4)
        line["roofline"][f"c4_{kind}_us"] = round(g["ms_per_step"] * 1e3, 2)
        if "dyn_tops" in g:
            line["roofline"][f"c4_{kind}_bf16_in_tops"] = round(g["dyn_tops"], 1)
            line["roofline"][f"c4_{kind}_bf16_in_frac"] = round(g["dyn_tops"] / g["peak"], 4)
        cb = g["line"].get("cpu_baseline") or {}
        if cb.get("value") is not None:
            line["cpu_baseline"] = dict(line["cpu_baseline"] or {})
            line["cpu_baseline"][f"c4_{kind}_{cb.get('unit', 'TOPS')}"] = cb["value"]
    print(json.dumps(line), flush=True)


def roofline_gemm(gemm):
    """Roofline of the W8A8 GEMM (k_gemm_8wp) at C4: algorithmic ops per
    launch over the back-to-back launch time, against dense int8 / fp8 MFMA
    peak, with the HBM traffic the counters measured for one launch and the
    same-run CPU baseline."""
    if not gemm:
        return None
    out = {"bound": "mfma", "kernel": "k_gemm_8wp", "unit": "TOPS", "workload": "C4 M=2048 N=14336 K=4096",
           "ops_per_launch": 2 * 2048 * 14336 * 4096}
    for kind, g in gemm.items():
        out[kind] = {"achieved": round(g["tops"], 1), "peak": g["peak"], "frac": round(g["tops"] / g["peak"], 4),
                     "kernel_event_pair_tops": round(g["tops_kernel"], 1),
                     "launch_us": round(g["ms_per_step"] * 1e3, 2),
                     "traffic": load_traffic(f"k_gemm_8wp<{kind}>"),
                     "sclk_dpm_mhz_median": g.get("sclk_dpm_mhz_median"),
                     "cpu_baseline": g["line"].get("cpu_baseline")}
    return out


if __name__ == "__main__":
    main()
