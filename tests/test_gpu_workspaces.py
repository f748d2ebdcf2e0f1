"""Scratch workspaces under thread churn: 48 short-lived host threads, each
running a decode linear that needs split-K scratch (W4A16 at M = 8, K =
8192) on the same stream, leave at most as many workspaces as the threads
alive at once need, every result equals the single-threaded one, and
SNEPPX_qlinear_release_workspaces returns the count to where it started."""
import threading

import numpy as np
import pytest
import torch

DEV = "cuda"


@pytest.mark.gpu
def test_workspaces_bounded_under_thread_churn(lib):
    import ctypes as C
    print("[gpu] workspaces: 48 threads x W4A16 M=8 N=1000 K=8192", flush=True)
    N, K, g, M = 1000, 8192, 128, 8
    w = torch.randn((N, K), device=DEV) * 0.02
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, K // g), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (K // g + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, g)
    x = torch.randn((M, K), device=DEV).to(torch.bfloat16)
    stream = torch.cuda.Stream()
    want = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(x, qw, sc, qz, None, K // g, want, g, stream=stream.cuda_stream)
    torch.cuda.synchronize()
    count = lib.fn["snx_workspace_count"]
    start = count()
    errors = []

    def worker():
        try:
            y = torch.empty((M, N), device=DEV)
            lib.qlinear_w4a16(x, qw, sc, qz, None, K // g, y, g, stream=stream.cuda_stream)
            torch.cuda.synchronize()
            if not torch.equal(y, want):
                errors.append("result differs")
        except Exception as e:      # reported in the main thread
            errors.append(str(e))

    for wave in range(12):
        ts = [threading.Thread(target=worker) for _ in range(4)]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=60)
        assert not any(t.is_alive() for t in ts)
    assert not errors, errors[:3]
    held = count() - start
    print(f"[gpu] workspaces held after 48 threads: {held}", flush=True)
    assert 0 < held <= 4 * 4, held          # 4 threads alive at once, a few slots each
    assert lib.fn["SNEPPX_qlinear_release_workspaces"](C.c_void_p(stream.cuda_stream)) == 0
    torch.cuda.synchronize()
    assert count() <= start
