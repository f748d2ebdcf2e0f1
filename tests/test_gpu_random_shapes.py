"""Seeded random shapes through every quantized linear entry point, against
the CPU oracle: W4A16 (every dispatch path: M = 1, small M, the prefill GEMM,
group sizes 32..256, with and without zero words and bias, bf16 and fp32
outputs), GPTQ act-order (prepared), W8A8 int8 (int32 accumulators exact,
bf16 outputs vs the float64 epilogue), W8A8 fp8 and the W8 GEMV.  Each case
is drawn from its own seed, so a failure names a reproducible shape; sizes
are bounded so the oracle finishes in well under a second per case."""
import numpy as np
import pytest
import torch

from test_gpu_qlinear import DEV, TOL_BF16, TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def _u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


def _gen(rng):
    return torch.Generator(device=DEV).manual_seed(int(rng.integers(1 << 30)))


@pytest.mark.parametrize("seed", range(24))
def test_w4a16_random_shape(lib, oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    group = int(rng.choice([32, 64, 128, 128, 256]))
    M = int(rng.choice([1, 1, 2, 3, 4, 5, 8, 11, 16, 17, 40, 256, 257, 300]))
    while True:
        K = group * int(rng.integers(1, max(2, 4096 // group)))
        N = int(rng.integers(1, 2500))
        if M * N * K <= 2e8:
            break
    if rng.random() < 0.5:
        N = (N + 7) // 8 * 8
    zeros, bias, f32 = rng.random() < 0.7, rng.random() < 0.3, rng.random() < 0.5
    print(f"[gpu] w4a16 random seed={seed} M={M} N={N} K={K} group={group} zeros={zeros} bias={bias} "
          f"f32={f32}", flush=True)
    G = K // group
    g = _gen(rng)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, group)
    x = (torch.randn((M, K), device=DEV, generator=g) + float(rng.normal(0, 0.5))).to(torch.bfloat16)
    b = torch.randn(N, device=DEV, generator=g) if bias else None
    y = torch.empty((M, N), dtype=torch.float32 if f32 else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(x, qw, sc, qz if zeros else None, None, G, y, group, bias=b)
    torch.cuda.synchronize()
    rc, want = oracle.w4a16_linear(_u16(x), _u32(qw), _u16(sc), _u32(qz) if zeros else None, None, N, K, group,
                                   bias=None if b is None else b.cpu().numpy())
    assert rc == 0
    assert rel_err(y.float().cpu().numpy(), want) <= (TOL_F32 if f32 else TOL_BF16)


@pytest.mark.parametrize("seed", range(8))
def test_w4a16_actorder_random_shape(lib, oracle, seed):
    rng = np.random.default_rng(2000 + seed)
    M = int(rng.choice([1, 2, 4, 8, 9, 16, 40]))
    K = 128 * int(rng.integers(1, 48))
    N = int(rng.integers(8, 2000)) // 8 * 8
    f32 = rng.random() < 0.5
    G = K // 128
    print(f"[gpu] act-order random seed={seed} M={M} N={N} K={K} f32={f32}", flush=True)
    g_idx = torch.from_numpy((rng.permutation(K) // 128).astype(np.int32)).to(DEV)
    g = _gen(rng)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    lib.dev_quantize_w4_gptq(w, g_idx, G, qw, sc)
    qs = torch.empty_like(qw)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(qw, g_idx, G, qs, perm)
    x = torch.randn((M, K), device=DEV, generator=g).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.float32 if f32 else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16_actorder(x, qs, sc, None, perm, y, 128)
    torch.cuda.synchronize()
    rc, want = oracle.w4a16_linear(_u16(x), _u32(qw), _u16(sc), None, g_idx.cpu().numpy(), N, K, 128)
    assert rc == 0
    assert rel_err(y.float().cpu().numpy(), want) <= (TOL_F32 if f32 else TOL_BF16)


@pytest.mark.parametrize("seed", range(8))
def test_w8a8_random_shape(lib, oracle, seed):
    rng = np.random.default_rng(3000 + seed)
    fp8 = seed % 2 == 1
    M, N = int(rng.integers(1, 1200)), int(rng.integers(1, 1200))
    K = (32 if fp8 else 16) * int(rng.integers(1, 80))
    print(f"[gpu] w8a8 random seed={seed} {'fp8' if fp8 else 'int8'} M={M} N={N} K={K}", flush=True)
    g = _gen(rng)
    a32 = torch.randn((M, K), device=DEV, generator=g)
    w32 = torch.randn((N, K), device=DEV, generator=g) * 0.02
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    if fp8:
        A = torch.empty((M, K), dtype=torch.uint8, device=DEV)
        W = torch.empty((N, K), dtype=torch.uint8, device=DEV)
        sA, sW = torch.empty(1, device=DEV), torch.empty(1, device=DEV)
        lib.dev_quantize_fp8_e4m3_scaled(a32, A, sA)
        lib.dev_quantize_fp8_e4m3_scaled(w32, W, sW)
        lib.qlinear_w8a8_fp8(A, sA, W, sW, out)
        torch.cuda.synchronize()
        want = oracle.fp8_gemm(A.cpu().numpy(), W.cpu().numpy(), float(sA.item()), float(sW.item()))
    else:
        A = torch.empty((M, K), dtype=torch.int8, device=DEV)
        W = torch.empty((N, K), dtype=torch.int8, device=DEV)
        sA, sW = torch.empty(M, device=DEV), torch.empty(N, device=DEV)
        lib.dev_quantize_int8_channel(a32, A, sA)
        lib.dev_quantize_int8_channel(w32, W, sW)
        acc = torch.empty((M, N), dtype=torch.int32, device=DEV)
        lib.qlinear_i8_gemm_i32(A, W, acc)
        lib.qlinear_w8a8_i8(A, sA, W, sW, out)
        torch.cuda.synchronize()
        exact = A.cpu().numpy().astype(np.int64) @ W.cpu().numpy().astype(np.int64).T
        assert np.array_equal(acc.cpu().numpy().astype(np.int64), exact)
        want = oracle.w8a8_epilogue(exact.astype(np.int32), sA.cpu().numpy(), sW.cpu().numpy())
    assert rel_err(out.float().cpu().numpy(), want) <= TOL_BF16


@pytest.mark.parametrize("seed", range(6))
def test_w8_gemv_random_shape(lib, oracle, seed):
    rng = np.random.default_rng(4000 + seed)
    M = int(rng.choice([1, 1, 2, 3, 5]))
    N, K = int(rng.integers(1, 4000)), 16 * int(rng.integers(1, 1024))
    print(f"[gpu] w8 gemv random seed={seed} M={M} N={N} K={K}", flush=True)
    g = _gen(rng)
    w32 = torch.randn((N, K), device=DEV, generator=g) * 0.02
    q = torch.empty((N, K), dtype=torch.int8, device=DEV)
    s = torch.empty(N, device=DEV)
    lib.dev_quantize_int8_channel(w32, q, s)
    x = torch.randn((M, K), device=DEV, generator=g) + float(rng.normal(0, 1))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w8_gemv(x, q, s, y)
    torch.cuda.synchronize()
    rc, want = oracle.w8_linear(x.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy())
    assert rc == 0
    assert rel_err(y.cpu().numpy(), want) <= TOL_F32
