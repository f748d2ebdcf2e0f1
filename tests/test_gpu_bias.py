"""The bias term of the quantized linears: y = x . W^T + bias
(QuantizedLinear.forward, bindings/python/.../quantization.py:451-454),
through every kernel path the entry points dispatch to, against the oracle
linear followed by the oracle's bias step (one fp32 add).

Bar as for the linears without bias: fp32 outputs within normwise 1e-4,
bf16 outputs within 1e-2."""
import numpy as np
import pytest
import torch

from test_gpu_qlinear import (DEV, TOL_BF16, TOL_F32, _w4_case, bf16_bits, bf16_to_f32, rel_err,
                              to_dev, u16)

pytestmark = pytest.mark.gpu


def _bias(N, seed):
    return np.random.default_rng(seed).normal(0, 1, N).astype(np.float32)


@pytest.mark.parametrize("M,N,K", [(1, 300, 4096), (3, 100, 4096), (2, 37, 100)])
def test_w8_gemv_bias(lib, oracle, M, N, K):
    # the M = 1 streaming kernel, the 4-row kernel, the any-K kernel
    print(f"[gpu] w8 gemv bias M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    b = _bias(N, K)
    rc, q, s = oracle.quantize_int8_channel(w)
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w8_gemv(to_dev(x), to_dev(q), to_dev(s), y, bias=to_dev(b))
    torch.cuda.synchronize()
    rc, yo = oracle.w8_linear(x, q, s, bias=b)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M,N,K,group,out", [
    (1, 1000, 4096, 128, "f32"),     # streaming M = 1 kernel
    (1, 1000, 4096, 128, "bf16"),
    (4, 1000, 4096, 128, "f32"),     # persistent small-M kernel
    (8, 500, 14336, 128, "f32"),     # split-K + ordered reduction
    (2, 300, 1024, 256, "bf16"),     # LDS-staged small-M kernel (group 256)
    (33, 200, 4096, 128, "f32"),     # 64-row GEMV slices
    (300, 520, 1024, 128, "f32"),    # prefill GEMM
    (300, 520, 1024, 128, "bf16"),
    (2, 30, 96, 32, "f32"),          # generic kernel (group 32)
])
def test_w4a16_bias(lib, oracle, M, N, K, group, out):
    print(f"[gpu] w4a16 bias M={M} N={N} K={K} g={group} {out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, M + N)
    x = bf16_bits(np.random.default_rng(M).normal(0, 1, (M, K)).astype(np.float32))
    b = _bias(N, N)
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, group, bias=to_dev(b))
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group, bias=b)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


@pytest.mark.parametrize("M", [1, 8, 300])
def test_w4a16_actorder_bias(lib, oracle, M):
    # prepared act-order: M = 1 and M = 8 gather in the decode kernels,
    # M = 300 gathers once and runs the prefill GEMM
    N, K = 600, 4096
    print(f"[gpu] w4a16 act-order bias M={M}", flush=True)
    rng = np.random.default_rng(M)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 5, g_idx=g_idx)
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    b = _bias(N, M)
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16_actorder(to_dev(x), qs, to_dev(sc), None, perm, y, 128, bias=to_dev(b))
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None, g_idx, N, K, 128, bias=b)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(256, 512, 256), (130, 7205, 256), (64, 64, 64)])
def test_w8a8_i8_bias(lib, oracle, M, N, K):
    # persistent kernel, the N % 8 != 0 kernel, the small-shape kernel
    print(f"[gpu] w8a8 i8 bias {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + N)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    sA = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sW = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    b = _bias(N, K)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_i8(to_dev(A), to_dev(sA), to_dev(W), to_dev(sW), out, bias=to_dev(b))
    torch.cuda.synchronize()
    want = oracle.w8a8_epilogue(oracle.i8_gemm_i32(A, W), sA, sW, bias=b)
    assert rel_err(bf16_to_f32(u16(out)), want) <= TOL_BF16


@pytest.mark.parametrize("M,N,K", [(256, 448, 256), (64, 64, 128)])
def test_w8a8_fp8_bias(lib, oracle, M, N, K):
    print(f"[gpu] w8a8 fp8 bias {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + K)
    rc, A, sa = oracle.quantize_fp8_e4m3_scaled(rng.normal(0, 1, (M, K)).astype(np.float32))
    rc, W, sw = oracle.quantize_fp8_e4m3_scaled(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    b = (0.05 * _bias(N, N)).astype(np.float32)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_fp8(to_dev(A), to_dev(np.array([sa], np.float32)), to_dev(W),
                         to_dev(np.array([sw], np.float32)), out, bias=to_dev(b))
    torch.cuda.synchronize()
    want = oracle.fp8_gemm(A, W, sa, sw, bias=b)
    assert rel_err(bf16_to_f32(u16(out)), want) <= TOL_BF16


@pytest.mark.parametrize("fmt,M", [("w4", 1), ("w4", 300), ("w8", 3)])
def test_qlayer_bias_forward_and_file_round_trip(lib, oracle, tmp_path, fmt, M):
    K, N = 1024, 520
    print(f"[gpu] qlayer bias {fmt} M={M}", flush=True)
    rng = np.random.default_rng(M)
    w_kn = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    b = _bias(N, 7)
    layer = lib.qlayer_create_kn(w_kn, fmt, 128)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y0 = layer.matmul_host(x)
    layer.set_bias(b)
    y = layer.matmul_host(x)
    wt = np.ascontiguousarray(w_kn.T)
    if fmt == "w4":
        rc, qw, sc, qz = oracle.w4_awq_quantize(wt, 128)
        rc, yo = oracle.w4a16_linear(bf16_bits(x), qw, sc, qz, None, N, K, 128, bias=b)
    else:
        rc, q, s = oracle.quantize_int8_channel(wt)
        rc, yo = oracle.w8_linear(x, q, s, bias=b)
    assert rel_err(y, yo) <= TOL_F32
    assert not np.array_equal(y, y0)
    # the bias travels with the layer through a file
    path = str(tmp_path / "b.safetensors")
    wr = lib.qstore_writer(path)
    layer.save(wr, "proj")
    wr.close()
    with lib.qstore_open(path) as st:
        np.testing.assert_array_equal(st.host("proj.bias"), b)
        layer2 = lib.qlayer_load(st, "proj")
    np.testing.assert_array_equal(layer2.matmul_host(x), y)
    # a device bias, then none
    layer.set_bias(torch.from_numpy(b).to(DEV))
    np.testing.assert_array_equal(layer.matmul_host(x), y)
    layer.set_bias(None)
    np.testing.assert_array_equal(layer.matmul_host(x), y0)


@pytest.mark.parametrize("fmt", ["w4", "w8"])
def test_matmul_host_is_reentrant(lib, fmt):
    """SNEPPX_qlayer_matmul_host replaces the reentrant matmul_3d
    (attention.c:324-346): two host threads calling it at once on one layer,
    with different row counts and inputs, get the single-threaded results."""
    import threading
    K, N = 2048, 1000
    layer = lib.qlayer_create_kn(np.random.default_rng(1).normal(0, 0.02, (K, N)).astype(np.float32), fmt, 128)
    xs = [np.random.default_rng(10 + t).normal(0, 1, (m, K)).astype(np.float32) for t, m in enumerate((3, 37))]
    want = [layer.matmul_host(x) for x in xs]
    errors = []

    def worker(t):
        try:
            for _ in range(25):
                got = layer.matmul_host(xs[t])
                if not np.array_equal(got, want[t]):
                    errors.append(f"thread {t}: result differs")
                    return
        except Exception as e:      # reported in the main thread
            errors.append(f"thread {t}: {e}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "matmul_host threads did not finish"
    assert not errors, errors
