"""Device quantizers and quantized linears (include/sneppx_qlinear.h) on the
GPU against the CPU oracle.

Bar: codes / packing / scales bit-exact; int32 GEMM accumulators bit-exact;
fp32-output linears within normwise relative error 1e-4 and bf16-output
linears within 1e-2 of the fp32 oracle, ||y - y_ref||_inf / ||y_ref||_inf."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 1e-2
DEV = "cuda"


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_to_f32(h):
    return (np.asarray(h, np.uint32) << 16).view(np.float32)


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------ quantizers
@pytest.mark.parametrize("shape", [(1, 1), (5, 333), (4096, 4096), (256, 14336)])
def test_dev_int8_channel_bit_exact(lib, oracle, shape):
    print(f"[gpu] int8 channel {shape}", flush=True)
    rng = np.random.default_rng(sum(shape))
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    w[0, 0] = 0.5 * np.abs(w[0]).max() / 127 * 3          # a tie when scaled
    q, s = torch.empty(shape, dtype=torch.int8, device=DEV), torch.empty(shape[0], device=DEV)
    lib.dev_quantize_int8_channel(to_dev(w), q, s)
    torch.cuda.synchronize()
    rc, qo, so = oracle.quantize_int8_channel(w)
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("shape", [(8, 512), (4096, 4096)])
def test_dev_int8_channel_half_even_bit_exact(lib, oracle, shape):
    print(f"[gpu] int8 channel half-even {shape}", flush=True)
    rng = np.random.default_rng(shape[0])
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    w[:4, 0] = 127.0                                       # scale 1: the next values are ties
    w[:4, 1:5] = np.array([0.5, 1.5, -2.5, 126.5], np.float32)
    q, s = torch.empty(shape, dtype=torch.int8, device=DEV), torch.empty(shape[0], device=DEV)
    lib.dev_quantize_int8_channel(to_dev(w), q, s, half_even=True)
    torch.cuda.synchronize()
    rc, qo, so = oracle.quantize_int8_channel_rne(w)
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert list(q.cpu().numpy()[0, 1:5]) == [0, 2, -2, 126]


@pytest.mark.parametrize("N,K,group", [(24, 512, 128), (11008, 4096, 128), (40, 256, 64), (8, 64, 8)])
def test_dev_w4_awq_bit_exact(lib, oracle, N, K, group):
    print(f"[gpu] w4 awq {N}x{K} g{group}", flush=True)
    rng = np.random.default_rng(N + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[1, :group] = 0.125                                   # degenerate group
    w[2, 0] = np.nan                                       # NaN first element of a group
    G = K // group
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(to_dev(w), qw, sc, qz, group)
    torch.cuda.synchronize()
    rc, qwo, sco, qzo = oracle.w4_awq_quantize(w, group)
    assert np.array_equal(qw.cpu().numpy().view(np.uint32), qwo)
    assert np.array_equal(u16(sc), sco)
    assert np.array_equal(qz.cpu().numpy().view(np.uint32), qzo)


@pytest.mark.parametrize("N,K", [(16, 512), (11008, 4096)])
def test_dev_w4_gptq_actorder_bit_exact(lib, oracle, N, K):
    print(f"[gpu] w4 gptq act-order {N}x{K}", flush=True)
    rng = np.random.default_rng(K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[3, 7] = np.inf                                      # poisons the rest of its group
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    G = K // 128
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    lib.dev_quantize_w4_gptq(to_dev(w), to_dev(g_idx), G, qw, sc)
    torch.cuda.synchronize()
    rc, qwo, sco = oracle.w4_gptq_quantize(w, g_idx, G)
    assert np.array_equal(qw.cpu().numpy().view(np.uint32), qwo)
    assert np.array_equal(u16(sc), sco)


def test_dev_w4_gptq_rejects_bad_g_idx(lib):
    w = torch.zeros((2, 16), device=DEV)
    g = torch.tensor([0] * 15 + [5], dtype=torch.int32, device=DEV)
    qw = torch.empty((2, 2), dtype=torch.int32, device=DEV)
    sc = torch.empty((2, 2), dtype=torch.int16, device=DEV)
    with pytest.raises(Exception, match="g_idx"):
        lib.dev_quantize_w4_gptq(w, g, 2, qw, sc)


@pytest.mark.parametrize("n", [1, 1000, 2048 * 4096])
def test_dev_fp8_scaled_bit_exact(lib, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.normal(0, 1, n).astype(np.float32)
    out = torch.empty(n, dtype=torch.uint8, device=DEV)
    s = torch.empty(1, device=DEV)
    lib.dev_quantize_fp8_e4m3_scaled(to_dev(x), out, s)
    torch.cuda.synchronize()
    rc, co, so = oracle.quantize_fp8_e4m3_scaled(x)
    assert np.array_equal(out.cpu().numpy(), co) and s.item() == so


def test_dev_fp8_scaled_division_rule(lib, oracle):
    """Tensors whose largest element is coded 0x77 under x / s and 0x76
    under x * (1/s), and the other way round: the kernel must give the
    oracle's (division) codes for both."""
    rng = np.random.default_rng(23)
    am = rng.uniform(0.5, 8.0, 4000).astype(np.float32)
    sc = (am / np.float32(240)).astype(np.float32)
    vd = (am / sc).astype(np.float32)
    vm = (am * (np.float32(1) / sc).astype(np.float32)).astype(np.float32)
    picks = np.concatenate([am[(vd >= 240) & (vm < 240)][:8], am[(vd < 240) & (vm >= 240)][:8]])
    assert len(picks) == 16
    for i, a in enumerate(picks):
        x = np.clip(rng.normal(0, float(a) / 4, 4099), -a, a).astype(np.float32)
        x[(37 * i) % 4099] = a if i % 2 else -a
        out = torch.empty(x.size, dtype=torch.uint8, device=DEV)
        s = torch.empty(1, device=DEV)
        lib.dev_quantize_fp8_e4m3_scaled(to_dev(x), out, s)
        torch.cuda.synchronize()
        rc, co, so = oracle.quantize_fp8_e4m3_scaled(x)
        assert np.array_equal(out.cpu().numpy(), co) and s.item() == so, a


# ---------------------------------------------------------------- linears
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (4, 1000, 4096), (2, 37, 100), (1, 17, 1024),
                                   (1, 1001, 2048), (1, 300, 8192), (1, 1, 4096), (1, 4096, 14336),
                                   (1, 33, 3072), (1, 100, 16384)])
def test_w8_gemv(lib, oracle, M, N, K):
    print(f"[gpu] w8 gemv M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * N + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    rc, q, s = oracle.quantize_int8_channel(w)
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w8_gemv(to_dev(x), to_dev(q), to_dev(s), y)
    torch.cuda.synchronize()
    rc, yo = oracle.w8_linear(x, q, s)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


def _w4_case(oracle, N, K, group, seed, g_idx=None, sym=False):
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    if g_idx is not None:
        G = int(g_idx.max()) + 1
        rc, qw, sc = oracle.w4_gptq_quantize(w, g_idx, G)
        return qw, sc, None, G
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, group)
    if sym:
        qz = None
    return qw, sc, qz, K // group


@pytest.mark.parametrize("M", [1, 4, 16, 33])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_w4a16_gemv_awq(lib, oracle, M, out):
    N, K, group = 11008 if M <= 4 else 1376, 4096, 128
    print(f"[gpu] w4a16 gemv M={M} N={N} out={out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, M)
    x = bf16_bits(np.random.default_rng(5 + M).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 14336), (2, 64, 2048), (3, 200, 4096)])
def test_w4a16_gemv_shapes(lib, oracle, M, N, K):
    # down-projection width, and the small-M kernel's scalar-scale path
    group = 128
    print(f"[gpu] w4a16 gemv M={M} N={N} K={K}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, K + M)
    x = bf16_bits(np.random.default_rng(M).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("N,K,sym,out", [
    (1, 2048, False, "f32"), (17, 4096, True, "bf16"), (1001, 6144, False, "f32"),
    (300, 8192, True, "f32"), (16, 8192, False, "bf16"), (11008, 2048, False, "f32"),
    (4096, 14336, False, "f32"), (33, 10240, True, "bf16"), (250, 12288, False, "bf16"),
    (19, 16384, True, "f32")])
def test_w4a16_gemv_m1_group128(lib, oracle, N, K, sym, out):
    # the M = 1, group-128 decode kernel at every K it takes (2048 T, T <= 8),
    # row counts that leave part of the last workgroup empty, with and
    # without zero points, fp32 and bf16 outputs
    group = 128
    print(f"[gpu] w4a16 gemv M=1 N={N} K={K} sym={sym} out={out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, N + K, sym=sym)
    x = bf16_bits(np.random.default_rng(K).normal(0, 1, (1, K)).astype(np.float32))
    y = torch.empty((1, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None if sym else to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None if sym else qz, None, N, K, group)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


@pytest.mark.parametrize("N,K,sym,out,bias,soff", [
    (4096, 1792, False, "bf16", False, 0), (4096, 1792, True, "f32", True, 2), (17, 256, False, "f32", False, 2),
    (4096, 512, False, "f32", True, 0), (1001, 2304, True, "bf16", False, 2), (4096, 3584, False, "f32", False, 0),
    (300, 7168, False, "f32", True, 2), (16, 10496, True, "bf16", False, 0), (33, 16128, False, "f32", False, 2)])
def test_w4a16_gemv_m1_ragged_k(lib, oracle, N, K, sym, out, bias, soff):
    # the M = 1 kernel's ragged form: K a multiple of 256 but not of 2048
    # (the down / O projections of a tensor-parallel shard: 4096 x 1792 and
    # 4096 x 512 at TP = 8, 4096 x 3584 at TP = 4, 4096 x 7168 at TP = 2),
    # group scales that are 4-byte but not 16-byte aligned (soff = 2 fp16
    # values into the buffer), with and without zero points and a bias
    group = 128
    print(f"[gpu] w4a16 gemv M=1 ragged N={N} K={K} sym={sym} out={out} bias={bias} soff={soff}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, 3 * N + K, sym=sym)
    x = bf16_bits(np.random.default_rng(K + 1).normal(0, 1, (1, K)).astype(np.float32))
    b = np.random.default_rng(K + 2).normal(0, 1, N).astype(np.float32) if bias else None
    scb = torch.zeros(N * G + soff, dtype=torch.int16, device=DEV)
    scb[soff:] = to_dev(sc.view(np.int16).reshape(-1))
    sc_d = scb[soff:].view(N, G)
    assert sc_d.data_ptr() % 16 == (4 * (soff // 2)) % 16
    y = torch.empty((1, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), sc_d, None if sym else to_dev(qz), None, G, y, group,
                      bias=None if b is None else to_dev(b))
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None if sym else qz, None, N, K, group)
    if b is not None:
        yo = oracle.add_bias(yo, b)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


@pytest.mark.parametrize("K,zeros", [(1792, False), (3584, True), (512, True)])
def test_w4a16_actorder_prepared_ragged_k(lib, oracle, K, zeros):
    """Act-order weights at the row-parallel shard widths (K not a multiple
    of 2048) through the M = 1 kernel's ragged form with the activation
    gather, against the oracle on the original column order."""
    N = 1040
    print(f"[gpu] w4a16 act-order M=1 ragged K={K} zeros={zeros}", flush=True)
    rng = np.random.default_rng(K)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 29, g_idx=g_idx)
    qz = rng.integers(0, 2**32, (N, (G + 7) // 8), dtype=np.uint64).astype(np.uint32) if zeros else None
    x = bf16_bits(rng.normal(0, 1, (1, K)).astype(np.float32))
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    y = torch.empty((1, N), dtype=torch.float32, device=DEV)
    lib.qlinear_w4a16_actorder(to_dev(x), qs, to_dev(sc), None if qz is None else to_dev(qz), perm, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, g_idx, N, K, 128)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M,zeros", [(11, False), (16, True), (12, True)])
def test_w4a16_actorder_prepared_small_m_two_early_groups(lib, oracle, M, zeros):
    """Act-order weights at 11 <= M <= 16 through the small-M kernel's form
    that issues two row groups' weight loads ahead of the activation copy
    (N = 11008: three groups per workgroup), against the oracle on the
    original column order."""
    N, K = 11008, 4096
    print(f"[gpu] w4a16 act-order prepared M={M} zeros={zeros}", flush=True)
    rng = np.random.default_rng(100 + M)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 31, g_idx=g_idx)
    qz = rng.integers(0, 2**32, (N, (G + 7) // 8), dtype=np.uint64).astype(np.uint32) if zeros else None
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    y = torch.empty((M, N), dtype=torch.float32, device=DEV)
    lib.qlinear_w4a16_actorder(to_dev(x), qs, to_dev(sc), None if qz is None else to_dev(qz), perm, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, g_idx, N, K, 128)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M,N,K,sym,out", [
    (2, 8197, 1024, False, "f32"), (3, 45, 2048, True, "bf16"), (5, 4099, 3072, False, "f32"),
    (8, 11008, 4096, True, "f32"), (16, 300, 4096, False, "bf16"), (16, 9000, 2048, True, "f32"),
    (7, 17, 4096, False, "f32")])
def test_w4a16_gemv_small_m_persistent(lib, oracle, M, N, K, sym, out):
    # the persistent 2 <= M <= 16 kernel: every K it takes (1024 .. 4096),
    # more row groups than workgroups (three per workgroup at N = 8197, 9000,
    # 11008), fewer (N = 17, 45), N not a multiple of 16, with and without
    # zero points, fp32 and bf16 outputs
    group = 128
    print(f"[gpu] w4a16 small-M M={M} N={N} K={K} sym={sym} out={out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, 90 + M + K, sym=sym)
    x = bf16_bits(np.random.default_rng(100 + M).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None if qz is None else to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


def test_w4a16_gemv_symmetric_and_tails(lib, oracle):
    # symmetric zero 8 (no qzeros), N not a multiple of 16, K of 1024
    N, K, group, M = 45, 1024, 256, 3
    qw, sc, _, G = _w4_case(oracle, N, K, group, 9, sym=True)
    x = bf16_bits(np.random.default_rng(3).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None, None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None, None, N, K, group)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M", [1, 8])
def test_w4a16_gptq_actorder(lib, oracle, M):
    N, K = 2048, 4096
    rng = np.random.default_rng(M)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 21, g_idx=g_idx)
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None, to_dev(g_idx), G, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None, g_idx, N, K, 128)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


def _unpack_nibbles(qw, K):
    q = np.asarray(qw, np.uint32)
    return np.stack([(q >> (4 * e)) & 15 for e in range(8)], axis=-1).reshape(q.shape[0], K)


def test_actorder_prepare_permutes_columns(lib, oracle):
    N, K = 96, 1024
    rng = np.random.default_rng(31)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 22, g_idx=g_idx)
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    torch.cuda.synchronize()
    p = perm.cpu().numpy().view(np.uint16).astype(np.int64)
    assert np.array_equal(p, np.argsort(g_idx, kind="stable"))
    assert np.array_equal(_unpack_nibbles(qs.cpu().numpy().view(np.uint32), K),
                          _unpack_nibbles(qw, K)[:, p])


def test_actorder_prepare_rejects_uneven_groups(lib, oracle):
    N, K = 16, 256
    g_idx = np.zeros(K, np.int32)
    g_idx[200:] = 1                       # group 0 holds 200 columns, group 1 holds 56
    qw = np.zeros((N, K // 8), np.uint32)
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    with pytest.raises(Exception, match="columns"):
        lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), 2, qs, perm)


@pytest.mark.parametrize("M,ydt,K", [(1, torch.float32, 4096), (1, torch.bfloat16, 4096),
                                     (1, torch.float32, 8192), (1, torch.float32, 2048),
                                     (3, torch.float32, 4096), (4, torch.bfloat16, 4096),
                                     (8, torch.float32, 4096), (300, torch.float32, 4096),
                                     (2, torch.bfloat16, 2048), (16, torch.float32, 1024),
                                     (1, torch.float32, 14336), (1, torch.bfloat16, 16384)])
def test_w4a16_actorder_prepared(lib, oracle, M, ydt, K):
    """Prepared (group-contiguous) weights give the layer's result on the
    original column order: compared with the oracle on qweight + g_idx."""
    N = 1040
    rng = np.random.default_rng(40 + M)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 23, g_idx=g_idx)
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    y = torch.empty((M, N), dtype=ydt, device=DEV)
    lib.qlinear_w4a16_actorder(to_dev(x), qs, to_dev(sc), None, perm, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, None, g_idx, N, K, 128)
    tol = TOL_F32 if ydt == torch.float32 else TOL_BF16
    assert rel_err(y.float().cpu().numpy(), yo) <= tol


@pytest.mark.parametrize("M,N,K,group,sym,out", [
    (5, 11008, 4096, 128, False, "f32"),     # persistent small-M kernel (group 128, K <= 4096)
    (8, 1000, 1408, 128, True, "f32"),       # 11 steps: spans of 128, N tail
    (12, 64, 4096, 256, False, "bf16"),      # one row block, group 256
    (16, 4096, 14336, 128, False, "f32"),    # down-projection width
    (2, 4096, 14336, 128, True, "bf16"),     # M <= 4 beyond the LDS-staged small-M kernel
    (3, 77, 14336, 128, False, "f32"),
    (4, 1000, 6144, 256, False, "f32"),
])
def test_w4a16_splitk_decode(lib, oracle, M, N, K, group, sym, out):
    print(f"[gpu] w4a16 split-K M={M} N={N} K={K} g={group} sym={sym} out={out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, 70 + M, sym=sym)
    x = bf16_bits(np.random.default_rng(80 + M).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None if qz is None else to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


# ------------------------------------------------------ W4A16 prefill GEMM
@pytest.mark.parametrize("M,N,K,group,sym,out", [
    (256, 512, 1024, 128, False, "f32"),     # whole tiles
    (300, 1000, 512, 256, True, "f32"),      # M and N tails, group 256, symmetric
    (257, 256, 4096, 128, False, "bf16"),    # one row into the second M tile
    (600, 136, 2048, 512, False, "f32"),     # N narrower than one tile, group 512
])
def test_w4a16_gemm(lib, oracle, M, N, K, group, sym, out):
    print(f"[gpu] w4a16 gemm M={M} N={N} K={K} g={group} sym={sym} out={out}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, 50 + M, sym=sym)
    x = bf16_bits(np.random.default_rng(60 + M).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), None if qz is None else to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)


@pytest.mark.parametrize("N,out,yoff", [(1001, "f32", 0), (1004, "bf16", 0), (1000, "bf16", 2), (1000, "f32", 1),
                                        (1000, "bf16", 0), (1000, "f32", 0)])
def test_w4a16_gemm_output_rows_staged_or_not(lib, oracle, N, out, yoff):
    """The prefill GEMM writes 16-byte row pieces staged through LDS when the
    output rows allow it (16-byte aligned, N a multiple of 8 bf16 / 4 fp32
    values) and one value per store otherwise: N = 1001 / 1004 and outputs
    offset by 2 or 1 values take the second path; both against the oracle,
    with a bias."""
    M, K, group = 300, 1024, 128
    print(f"[gpu] w4a16 gemm epilogue N={N} out={out} yoff={yoff}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, group, N + 3)
    x = bf16_bits(np.random.default_rng(N).normal(0, 1, (M, K)).astype(np.float32))
    b = np.random.default_rng(N + 1).normal(0, 1, N).astype(np.float32)
    dt = torch.float32 if out == "f32" else torch.bfloat16
    buf = torch.zeros(M * N + yoff, dtype=dt, device=DEV)
    y = buf[yoff:].view(M, N)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, group, bias=to_dev(b))
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group, bias=b)
    got = y.cpu().numpy() if out == "f32" else bf16_to_f32(u16(y))
    assert rel_err(got, yo) <= (TOL_F32 if out == "f32" else TOL_BF16)
    if yoff:
        assert float(buf[:yoff].abs().max()) == 0.0       # nothing written before the output


@pytest.mark.parametrize("M,N,K", [(2192, 6144, 4096), (1849, 6144, 4096), (600, 4096, 14336),
                                   (1849, 768, 4096)])
def test_w4a16_gemm_llama_shapes_sampled_rows(lib, oracle, M, N, K):
    """Full-size QKV (T=2192; and T=1849, whose 360 tiles exceed a round of
    256 CUs by 104: the full round whole-K, the 104 in two K spans) and
    down-projection shapes, and the QKV projection of one GPU's
    tensor-parallel shard (N = 6144 / 8: 45 tiles, K in 4 spans; the down
    shape at M = 600 runs 2): weights quantized on
    the GPU (bit-exact quantizer), every output row of a sample checked
    against the oracle, including the last, partial M tile; a second call
    gives bit-identical output (the span sums' order does not depend on
    which wave arrives last)."""
    print(f"[gpu] w4a16 gemm llama M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    G = K // 128
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
    del w
    x = torch.randn((M, K), device=DEV, generator=g).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(x, qw, sc, qz, None, G, y, 128)
    torch.cuda.synchronize()
    rows = np.array(sorted({0, 1, 63, 64, 127, 128, 255, M // 2, M - 129, M - 17, M - 2, M - 1}))
    xh = u16(x)[rows]
    rc, yo = oracle.w4a16_linear(xh, qw.cpu().numpy().view(np.uint32), u16(sc),
                                 qz.cpu().numpy().view(np.uint32), None, N, K, 128)
    got = bf16_to_f32(u16(y)[rows])
    assert rel_err(got, yo) <= TOL_BF16
    again = torch.empty_like(y)
    lib.qlinear_w4a16(x, qw, sc, qz, None, G, again, 128)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), again.view(torch.int16))


def test_w4a16_odd_group_uses_generic_path(lib, oracle):
    N, K, group, M = 30, 96, 32, 2
    qw, sc, qz, G = _w4_case(oracle, N, K, group, 4)
    x = bf16_bits(np.random.default_rng(4).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (200, 136, 4096), (17, 33, 48)])
def test_i8_gemm_accumulators_bit_exact(lib, oracle, M, N, K):
    print(f"[gpu] i8 gemm {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    Cm = torch.empty((M, N), dtype=torch.int32, device=DEV)
    lib.qlinear_i8_gemm_i32(to_dev(A), to_dev(W), Cm)
    torch.cuda.synchronize()
    assert np.array_equal(Cm.cpu().numpy(), oracle.i8_gemm_i32(A, W))


def test_w8a8_i8_full_shape_subtiles(lib, oracle):
    # C4 at full size: accumulators exact on sampled 64x64 sub-tiles, the
    # bf16 epilogue within 1e-2 of fp32 on dequantised operands.
    M, N, K = 2048, 14336, 4096
    print(f"[gpu] w8a8 i8 {M}x{N}x{K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(0)
    a32 = torch.randn((M, K), device=DEV, generator=g)
    w32 = torch.randn((N, K), device=DEV, generator=g) * 0.02
    A = torch.empty((M, K), dtype=torch.int8, device=DEV)
    W = torch.empty((N, K), dtype=torch.int8, device=DEV)
    sA, sW = torch.empty(M, device=DEV), torch.empty(N, device=DEV)
    lib.dev_quantize_int8_channel(a32, A, sA)
    lib.dev_quantize_int8_channel(w32, W, sW)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_i8(A, sA, W, sW, out)
    Cm = torch.empty((M, N), dtype=torch.int32, device=DEV)
    lib.qlinear_i8_gemm_i32(A, W, Cm)
    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    An, Wn, Cn = A.cpu().numpy(), W.cpu().numpy(), Cm.cpu().numpy()
    sAn, sWn, outn = sA.cpu().numpy(), sW.cpu().numpy(), bf16_to_f32(u16(out))
    for _ in range(6):
        m0, n0 = int(rng.integers(0, M - 64)), int(rng.integers(0, N - 64))
        ref = oracle.i8_gemm_i32(An[m0:m0 + 64], Wn[n0:n0 + 64])
        assert np.array_equal(Cn[m0:m0 + 64, n0:n0 + 64], ref)
        deq = oracle.w8a8_epilogue(ref, sAn[m0:m0 + 64], sWn[n0:n0 + 64])
        assert rel_err(outn[m0:m0 + 64, n0:n0 + 64], deq) <= TOL_BF16
    # last rows / columns too
    ref = oracle.i8_gemm_i32(An[-64:], Wn[-64:])
    assert np.array_equal(Cn[-64:, -64:], ref)


@pytest.mark.parametrize("M,N,K", [(2148, 7208, 384), (300, 1000, 128), (130, 7205, 256)])
def test_w8a8_i8_persistent_ragged(lib, oracle, M, N, K):
    # 297 tiles for 256 workgroups (several tiles per workgroup, tile order
    # without the XCD grouping), ragged edge tiles, odd and single-stage K
    # loops, and N % 8 != 0 (bf16 output through the non-persistent kernel).
    print(f"[gpu] w8a8 i8 persistent {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    sA = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sW = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_i8(to_dev(A), to_dev(sA), to_dev(W), to_dev(sW), out)
    Cm = torch.empty((M, N), dtype=torch.int32, device=DEV)
    lib.qlinear_i8_gemm_i32(to_dev(A), to_dev(W), Cm)
    torch.cuda.synchronize()
    Cn, outn = Cm.cpu().numpy(), bf16_to_f32(u16(out))
    blocks = [(0, 0), (M - 64, N - 64), (M - 64, 0), (0, N - 64)]
    blocks += [(int(rng.integers(0, M - 64)), int(rng.integers(0, N - 64))) for _ in range(6)]
    for m0, n0 in blocks:
        ref = oracle.i8_gemm_i32(A[m0:m0 + 64], W[n0:n0 + 64])
        assert np.array_equal(Cn[m0:m0 + 64, n0:n0 + 64], ref), (m0, n0)
        deq = oracle.w8a8_epilogue(ref, sA[m0:m0 + 64], sW[n0:n0 + 64])
        assert rel_err(outn[m0:m0 + 64, n0:n0 + 64], deq) <= TOL_BF16, (m0, n0)


@pytest.mark.parametrize("M,N,K", [(64, 64, 128), (130, 200, 4096)])
def test_fp8_gemm(lib, oracle, M, N, K):
    print(f"[gpu] fp8 gemm {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M * N)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    rc, ca, sa = oracle.quantize_fp8_e4m3_scaled(a)
    rc, cw, sw = oracle.quantize_fp8_e4m3_scaled(w)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_fp8(to_dev(ca), to_dev(np.array([sa], np.float32)), to_dev(cw),
                         to_dev(np.array([sw], np.float32)), out)
    torch.cuda.synchronize()
    ref = oracle.fp8_gemm(ca, cw, sa, sw)
    assert rel_err(bf16_to_f32(u16(out)), ref) <= TOL_BF16


# ------------------------------------------------------------ SwiGLU step
@pytest.mark.parametrize("T,F", [(1, 8), (37, 14336), (300, 1000)])
def test_silu_mul(lib, T, F):
    rng = np.random.default_rng(T)
    gu = bf16_bits(rng.normal(0, 2, (T, 2 * F)).astype(np.float32))
    out = torch.empty((T, F), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_silu_mul(to_dev(gu), out)
    torch.cuda.synchronize()
    g = bf16_to_f32(gu[:, :F]).astype(np.float64)
    u = bf16_to_f32(gu[:, F:]).astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    got = bf16_to_f32(u16(out)).astype(np.float64)
    # one bf16 rounding of the fp32 value: |err| <= 2^-8 |want| (+ fp32 slack)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)


@pytest.mark.parametrize("T,F", [(1, 8), (37, 14336), (300, 1000), (2, 32768)])
def test_silu_mul_quant_int8_equals_quantizing_the_silu_output(lib, oracle, T, F):
    print(f"[gpu] silu_mul_quant_int8 T={T} F={F}", flush=True)
    rng = np.random.default_rng(T + F)
    gu = bf16_bits(rng.normal(0, 2, (T, 2 * F)).astype(np.float32))
    if T >= 37:
        gu[3] = 0                                            # an all-zero row: scale 1, codes 0
        gu[5, :F] = bf16_bits(np.full(F, 60.0, np.float32))  # saturating gate
    g = to_dev(gu)
    h = torch.empty((T, F), dtype=torch.bfloat16, device=DEV)
    q = torch.empty((T, F), dtype=torch.int8, device=DEV)
    s = torch.empty(T, device=DEV)
    lib.qlinear_silu_mul(g, h)
    lib.qlinear_silu_mul_quant_int8(g, q, s)
    torch.cuda.synchronize()
    rc, qo, so = oracle.quantize_int8_channel(bf16_to_f32(u16(h)).reshape(T, F))
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 4096), (2048, 4096), (3, 14336), (5, 1000), (9, 2048),
                                       (4, 6000), (3, 8192), (300, 136)])
def test_dev_int8_channel_bf16_bit_exact(lib, oracle, rows, cols):
    """Per-token int8 of bf16 rows (one-pass register kernel for cols % 8 == 0
    up to 8192 in its 1 / 2 / 4-chunk forms, the two-pass kernel otherwise)
    bit-exact vs the oracle, incl. NaN (ignored by the max, code -128), +-inf
    (scale inf, codes 0 or NaN-clamped), an all-zero row (scale 1), bf16
    denormals and exact .5 ties."""
    rng = np.random.default_rng(rows * cols)
    x = rng.normal(0, 3, (rows, cols)).astype(np.float32)
    if rows >= 3 and cols >= 8:
        x[0, :4] = [np.nan, 1.0, -2.5, 127.0]
        x[0, 4:8] = [0.5, 1.5, -0.5, 2.5]           # with max 127: exact ties
        x[0, 8:] = np.clip(x[0, 8:], -126, 126)
        x[1, :] = 0.0
        x[2, :2] = [np.inf, -1e-39]
    xb = bf16_bits(x)
    q = torch.empty((rows, cols), dtype=torch.int8, device=DEV)
    s = torch.empty(rows, device=DEV)
    lib.dev_quantize_int8_channel_bf16(to_dev(xb), q, s)
    torch.cuda.synchronize()
    rc, qo, so = oracle.quantize_int8_channel(bf16_to_f32(xb).reshape(rows, cols))
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_silu_mul_quant_int8_rejects_bad_shapes(lib):
    g = torch.zeros((2, 2 * 12), dtype=torch.int16, device=DEV)
    with pytest.raises(Exception, match="multiple of 8"):
        lib.qlinear_silu_mul_quant_int8(g, torch.empty((2, 12), dtype=torch.int8, device=DEV),
                                        torch.empty(2, device=DEV))


# ---------------------------------------------------------- QAT fake-quant
@pytest.mark.parametrize("n,scale,bits", [(1, 0.5, 8), (1000, 0.02, 4), (1 << 20, 0.003, 8), (77, 1.0, 16)])
def test_dev_fake_quant_bit_exact(lib, oracle, n, scale, bits):
    rng = np.random.default_rng(n + bits)
    x = rng.normal(0, 1, n).astype(np.float32)
    x[: min(n, 4)] = np.array([1.4, -0.6, 200.0, np.nan], np.float32)[: min(n, 4)]   # test_fake_quant.c KATs
    y = torch.empty(n, device=DEV)
    lib.dev_fake_quant(to_dev(x), y, scale, bits)
    torch.cuda.synchronize()
    rc, yo = oracle.fake_quant(x, scale, bits)
    assert rc == 0
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yo.view(np.uint32))


def test_dev_fake_quant_rejects_bad_arguments(lib):
    x = torch.zeros(4, device=DEV)
    for scale, bits in ((0.0, 8), (-1.0, 8), (1.0, 1), (1.0, 17)):
        with pytest.raises(Exception):
            lib.dev_fake_quant(x, x, scale, bits)


# ------------------------------------------- the bench's exact shapes, fp8 C4
def _fp8_blocks(M, N, rng, extra=6):
    blocks = [(0, 0), (M - 64, N - 64), (M - 64, 0), (0, N - 64)]
    return blocks + [(int(rng.integers(0, M - 64)), int(rng.integers(0, N - 64))) for _ in range(extra)]


def test_w8a8_fp8_full_shape_subtiles(lib, oracle):
    """C4 fp8 at full size through the multi-tile kernel (XCD-aware tile
    map): sampled 64x64 sub-tiles plus the four corner blocks against the
    oracle's fp8 product of the same codes."""
    M, N, K = 2048, 14336, 4096
    print(f"[gpu] w8a8 fp8 {M}x{N}x{K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3)
    a32 = torch.randn((M, K), device=DEV, generator=g)
    w32 = torch.randn((N, K), device=DEV, generator=g) * 0.02
    A = torch.empty((M, K), dtype=torch.uint8, device=DEV)
    W = torch.empty((N, K), dtype=torch.uint8, device=DEV)
    sA, sW = torch.empty(1, device=DEV), torch.empty(1, device=DEV)
    lib.dev_quantize_fp8_e4m3_scaled(a32, A, sA)
    lib.dev_quantize_fp8_e4m3_scaled(w32, W, sW)
    del a32, w32
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_fp8(A, sA, W, sW, out)
    torch.cuda.synchronize()
    An, Wn, outn = A.cpu().numpy(), W.cpu().numpy(), bf16_to_f32(u16(out))
    sa, sw = np.float32(sA.item()), np.float32(sW.item())
    for m0, n0 in _fp8_blocks(M, N, np.random.default_rng(2)):
        ref = oracle.fp8_gemm(An[m0:m0 + 64], Wn[n0:n0 + 64], sa, sw)
        assert rel_err(outn[m0:m0 + 64, n0:n0 + 64], ref) <= TOL_BF16, (m0, n0)


@pytest.mark.parametrize("M,N,K", [(2148, 7208, 384), (300, 1000, 128), (130, 7205, 256)])
def test_w8a8_fp8_ragged_multi_tile(lib, oracle, M, N, K):
    # several tile rows and columns, ragged edge tiles, one- and three-stage
    # K loops, N not a multiple of 8
    print(f"[gpu] w8a8 fp8 ragged {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    rc, A, sa = oracle.quantize_fp8_e4m3_scaled(rng.normal(0, 1, (M, K)).astype(np.float32))
    rc, W, sw = oracle.quantize_fp8_e4m3_scaled(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w8a8_fp8(to_dev(A), to_dev(np.array([sa], np.float32)), to_dev(W),
                         to_dev(np.array([sw], np.float32)), out)
    torch.cuda.synchronize()
    outn = bf16_to_f32(u16(out))
    for m0, n0 in _fp8_blocks(M, N, rng):
        ref = oracle.fp8_gemm(A[m0:m0 + 64], W[n0:n0 + 64], sa, sw)
        assert rel_err(outn[m0:m0 + 64, n0:n0 + 64], ref) <= TOL_BF16, (m0, n0)


@pytest.mark.parametrize("kind,N,bias", [("i8", 1792, False), ("fp8", 1792, True), ("i8", 3584, True),
                                         ("fp8", 3584, False)])
def test_w8a8_tensor_parallel_shard_split_k(lib, oracle, kind, N, bias):
    """C4 on one GPU's column shard of a tensor-parallel layer: at N = 14336
    / 8 the 64 tiles fill a quarter of the CUs, so the persistent kernel
    splits K into 2 spans and the last-arriving wave of each (tile, wave)
    adds the spans' partial sums in span order; N = 14336 / 4 (128 tiles)
    runs unsplit.  Sampled 64x64 sub-tiles and the
    corners against the oracle (int8 accumulators bit-exact); a call of
    another split shape in between, then a repeat giving bit-identical
    output (the arrival counters return to 0; the sums' order does not
    depend on which wave arrives last)."""
    M, K = 2048, 4096
    print(f"[gpu] w8a8 {kind} shard {M}x{N}x{K} bias={bias}", flush=True)
    rng = np.random.default_rng(N + (7 if kind == "fp8" else 0))
    b = rng.normal(0, 1, N).astype(np.float32) if bias else None
    bd = None if b is None else to_dev(b)
    g = torch.Generator(device=DEV).manual_seed(N)
    a32 = torch.randn((M, K), device=DEV, generator=g)
    w32 = torch.randn((N, K), device=DEV, generator=g) * 0.02
    fp8 = kind == "fp8"
    A = torch.empty((M, K), dtype=torch.uint8 if fp8 else torch.int8, device=DEV)
    W = torch.empty((N, K), dtype=torch.uint8 if fp8 else torch.int8, device=DEV)
    if fp8:
        sA, sW = torch.empty(1, device=DEV), torch.empty(1, device=DEV)
        lib.dev_quantize_fp8_e4m3_scaled(a32, A, sA)
        lib.dev_quantize_fp8_e4m3_scaled(w32, W, sW)
        run = lambda o, A_=A, W_=W, sA_=sA, sW_=sW: lib.qlinear_w8a8_fp8(A_, sA_, W_, sW_, o, bias=bd)  # noqa: E731
    else:
        sA, sW = torch.empty(M, device=DEV), torch.empty(N, device=DEV)
        lib.dev_quantize_int8_channel(a32, A, sA)
        lib.dev_quantize_int8_channel(w32, W, sW)
        run = lambda o, A_=A, W_=W, sA_=sA, sW_=sW: lib.qlinear_w8a8_i8(A_, sA_, W_, sW_, o, bias=bd)  # noqa: E731
    del a32, w32
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    run(out)
    # another split shape on the same stream (10 tiles), then a repeat
    small = torch.empty((300, 1000), dtype=torch.bfloat16, device=DEV)
    if fp8:
        lib.qlinear_w8a8_fp8(A[:300, :1024].contiguous(), sA, W[:1000, :1024].contiguous(), sW, small)
    else:
        lib.qlinear_w8a8_i8(A[:300, :1024].contiguous(), sA[:300].contiguous(), W[:1000, :1024].contiguous(),
                            sW[:1000].contiguous(), small)
    again = torch.empty_like(out)
    run(again)
    Cm = None
    if not fp8:
        Cm = torch.empty((M, N), dtype=torch.int32, device=DEV)
        lib.qlinear_i8_gemm_i32(A, W, Cm)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    An, Wn, outn = A.cpu().numpy(), W.cpu().numpy(), bf16_to_f32(u16(out))
    blocks = [(0, 0), (M - 64, N - 64), (M - 64, 0), (0, N - 64)]
    blocks += [(int(rng.integers(0, M - 64)), int(rng.integers(0, N - 64))) for _ in range(4)]
    for m0, n0 in blocks:
        if fp8:
            ref = oracle.fp8_gemm(An[m0:m0 + 64], Wn[n0:n0 + 64], np.float32(sA.item()), np.float32(sW.item()))
        else:
            acc = oracle.i8_gemm_i32(An[m0:m0 + 64], Wn[n0:n0 + 64])
            assert np.array_equal(Cm.cpu().numpy()[m0:m0 + 64, n0:n0 + 64], acc), (m0, n0)
            ref = oracle.w8a8_epilogue(acc, sA.cpu().numpy()[m0:m0 + 64], sW.cpu().numpy()[n0:n0 + 64])
        if b is not None:
            ref = oracle.add_bias(ref, b[n0:n0 + 64])
        assert rel_err(outn[m0:m0 + 64, n0:n0 + 64], ref) <= TOL_BF16, (m0, n0)


def _random_qzeros(rng, N, G):
    z = rng.integers(0, 16, (N, ((G + 7) // 8) * 8)).astype(np.uint32)
    z[:, G:] = 0
    return (z.reshape(N, -1, 8) << (4 * np.arange(8, dtype=np.uint32))).sum(-1).astype(np.uint32)


@pytest.mark.parametrize("M,N,K,zeros", [(1, 11008, 4096, False), (8, 11008, 4096, False),
                                         (1, 11008, 4096, True), (8, 11008, 4096, True),
                                         (1, 4096, 14336, True), (8, 4096, 14336, True)])
def test_w4a16_actorder_prepared_bench_shapes(lib, oracle, M, N, K, zeros):
    """C3 at the bench's shape (N = 11008, three row groups per workgroup in
    the small-M kernel), and act-order weights that carry zero points (the
    prepared M = 1 and small-M kernels built with zeros), also at the
    down-projection width."""
    print(f"[gpu] w4a16 act-order prepared M={M} N={N} K={K} zeros={zeros}", flush=True)
    rng = np.random.default_rng(M + N + K + zeros)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    qw, sc, _, G = _w4_case(oracle, N, K, 128, 29 + M, g_idx=g_idx)
    qz = _random_qzeros(rng, N, G) if zeros else None
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    qs = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    perm = torch.empty(K, dtype=torch.int16, device=DEV)
    lib.qlinear_w4_actorder_prepare(to_dev(qw), to_dev(g_idx), G, qs, perm)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16_actorder(to_dev(x), qs, to_dev(sc), None if qz is None else to_dev(qz), perm, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, g_idx, N, K, 128)
    assert rel_err(bf16_to_f32(u16(y)), yo) <= TOL_BF16


def test_w4a16_gemv_m16_bench_shape(lib, oracle):
    # C2 M = 16 exactly as the bench runs it (N = 11008, zero points, bf16 out)
    M, N, K = 16, 11008, 4096
    print(f"[gpu] w4a16 gemv M={M} N={N} K={K}", flush=True)
    qw, sc, qz, G = _w4_case(oracle, N, K, 128, 116)
    x = bf16_bits(np.random.default_rng(216).normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, G, y, 128)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, 128)
    assert rel_err(bf16_to_f32(u16(y)), yo) <= TOL_BF16


@pytest.mark.parametrize("K", [14336, 16384])
@pytest.mark.parametrize("mean", [3.0, -1.0])
def test_w8_gemv_activations_far_from_zero_mean(lib, oracle, K, mean):
    # the unsigned-byte form takes 128 * sum(x) off; with x ~ N(mean, 1) that
    # term is large, so it must come off per slot, not once per row
    N = 300
    print(f"[gpu] w8 gemv mean={mean} K={K}", flush=True)
    rng = np.random.default_rng(K + int(mean))
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = (rng.normal(0, 1, (1, K)) + mean).astype(np.float32)
    rc, q, s = oracle.quantize_int8_channel(w)
    y = torch.empty((1, N), device=DEV)
    lib.qlinear_w8_gemv(to_dev(x), to_dev(q), to_dev(s), y)
    torch.cuda.synchronize()
    rc, yo = oracle.w8_linear(x, q, s)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32


# ------------------------------------------- gate/up projection + SwiGLU fused
@pytest.mark.parametrize("M,F,K,sym,bias", [
    (300, 1000, 1024, False, False),    # fused GEMM epilogue, F not a multiple of 128
    (256, 512, 4096, True, True),       # one M tile, symmetric, bias
    (600, 14336, 4096, False, False),   # the Llama MLP width (sampled rows)
    (4, 1000, 4096, False, True),       # decode rows: fp32 projection, then the same rule
    (1, 512, 2048, True, False),        # one row: gate and up rows in one wave of the M = 1 kernel
    (1, 14336, 4096, False, True),      # the Llama-3-8B MLP width at decode
    (1, 11008, 4096, False, False),
    (1, 1000, 4096, False, True),       # ragged row shares
    (1, 3000, 14336, False, True),      # K = 14336
    (1, 24, 2048, True, True),          # fewer workgroups than CUs, short shares
])
def test_w4a16_swiglu(lib, oracle, M, F, K, sym, bias):
    """out = bf16(silu(g) * u), g / u the gate / up halves of the stacked
    [2F][K] projection (gated_activations.c:33-52 SWIGLU on the fp32 linear),
    against the oracle linear and a float64 SiLU."""
    print(f"[gpu] w4a16 swiglu M={M} F={F} K={K} sym={sym} bias={bias}", flush=True)
    rng = np.random.default_rng(M + F)
    qw, sc, qz, G = _w4_case(oracle, 2 * F, K, 128, M + K, sym=sym)
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    b = rng.normal(0, 0.5, 2 * F).astype(np.float32) if bias else None
    out = torch.empty((M, F), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16_swiglu(to_dev(x), to_dev(qw), to_dev(sc), None if qz is None else to_dev(qz), out, 128,
                             bias=None if b is None else to_dev(b))
    torch.cuda.synchronize()
    rows = np.arange(M) if M * F <= 300 * 1000 else np.array(sorted({0, 1, 127, 128, M // 2, M - 2, M - 1}))
    rc, gu = oracle.w4a16_linear(x[rows], qw, sc, qz, None, 2 * F, K, 128, bias=b)
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * u
    got = bf16_to_f32(u16(out)[rows]).astype(np.float64)
    assert rel_err(got, want) <= TOL_BF16
    # elementwise: one bf16 rounding plus the fp32 linear's own error
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-4 * np.abs(want).max())


@pytest.mark.parametrize("M,K,group", [(1, 4096, 128), (4, 4096, 128), (2, 1024, 256), (8, 14336, 128),
                                       (3, 96, 32)])
def test_w4a16_subnormal_fp16_scales(lib, oracle, M, K, group):
    """Rows of tiny weights get fp16-subnormal group scales (range/15 below
    2^-14); every decode kernel must decode them exactly (the hardware
    fp16 -> fp32 conversion keeps fp16 denormals).  The tiny rows are checked
    as a group, normwise among themselves, so the large rows cannot hide
    them; a scale flushed to zero would give a relative error of 1."""
    N = 48
    print(f"[gpu] w4a16 subnormal scales M={M} K={K} g={group}", flush=True)
    rng = np.random.default_rng(K + M)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[::3] *= 1e-4                                          # scales ~ 1e-5: subnormal fp16
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, group)
    assert ((sc[::3] & 0x7C00) == 0).mean() > 0.9            # mostly subnormal scales
    x = bf16_bits(rng.normal(0, 1, (M, K)).astype(np.float32))
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(to_dev(x), to_dev(qw), to_dev(sc), to_dev(qz), None, K // group, y, group)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(x, qw, sc, qz, None, N, K, group)
    got = y.cpu().numpy()
    assert np.abs(yo[:, ::3]).max() < 1e-3 * np.abs(yo[:, 1::3]).max()
    assert rel_err(got[:, ::3], yo[:, ::3]) <= TOL_F32


@pytest.mark.parametrize("tp", [1, 8])
def test_decode_token_through_llama3_layer_linears(lib, oracle, tp):
    """One token (M = 1) through the four linears of a Llama-3-8B layer as the
    bench's decode lines run them (QKV 6144x4096, O 4096x4096 on the first
    4096 QKV outputs, gate/up + SwiGLU 2x14336x4096 in one launch, down
    4096x14336), or one GPU's shard of them at tp = 8 (QKV 768x4096, O
    4096x512, gate/up 2x1792x4096, down 4096x1792), each stage against the
    oracle fed the same bf16 input."""
    print(f"[gpu] decode token through the Llama-3-8B layer linears tp={tp}", flush=True)
    H, F, QKV, A = 4096, 14336 // tp, 6144 // tp, 4096 // tp
    rng = np.random.default_rng(77)
    w = {n: _w4_case(oracle, N, K, 128, 80 + i)
         for i, (n, N, K) in enumerate((("qkv", QKV, H), ("o", H, A), ("gu", 2 * F, H), ("down", H, F)))}
    x = bf16_bits(rng.normal(0, 1, (1, H)).astype(np.float32))
    dev = {n: tuple(to_dev(a) for a in v[:3]) for n, v in w.items()}
    qkv = torch.empty((1, QKV), dtype=torch.bfloat16, device=DEV)
    o = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
    h = torch.empty((1, F), dtype=torch.bfloat16, device=DEV)
    y = torch.empty((1, H), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16(to_dev(x), *dev["qkv"], None, H // 128, qkv, 128)
    lib.qlinear_w4a16(qkv[:, :A], *dev["o"], None, A // 128, o, 128)       # the first A values
    lib.qlinear_w4a16_swiglu(o, *dev["gu"], h, 128)
    lib.qlinear_w4a16(h, *dev["down"], None, F // 128, y, 128)
    torch.cuda.synchronize()
    # each stage against the oracle on the GPU's own (bf16) input to it
    steps = (("qkv", x, qkv, QKV, H), ("o", u16(qkv)[:, :A], o, H, A), ("down", u16(h), y, H, F))
    for name, inp, got, N, K in steps:
        qw, sc, qz, _ = w[name]
        rc, want = oracle.w4a16_linear(np.ascontiguousarray(inp), qw, sc, qz, None, N, K, 128)
        assert rel_err(bf16_to_f32(u16(got)), want) <= TOL_BF16, name
    qw, sc, qz, _ = w["gu"]
    rc, gu = oracle.w4a16_linear(u16(o), qw, sc, qz, None, 2 * F, H, 128)
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    assert rel_err(bf16_to_f32(u16(h)), g / (1.0 + np.exp(-g)) * u) <= TOL_BF16


@pytest.mark.parametrize("M,N,K", [(2048, 14336, 4096), (300, 1000, 1024), (257, 448, 10016), (1, 256, 4096)])
@pytest.mark.parametrize("fp8", [False, True])
def test_w8a8_dyn_equals_quantize_then_gemm(lib, M, N, K, fp8):
    """C4 from bf16 activations: the one-call form (A quantized inside) gives
    the bits of quantizing A with the standalone entry point and calling the
    GEMM (int8 per token; fp8 per tensor on A converted to fp32, exact)."""
    print(f"[gpu] w8a8 dyn {'fp8' if fp8 else 'int8'} M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    A = torch.randn((M, K), device=DEV, generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    bias = torch.randn(N, device=DEV, generator=g)
    out1 = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    out2 = torch.empty_like(out1)
    if fp8:
        W = torch.empty((N, K), dtype=torch.uint8, device=DEV)
        sW = torch.empty(1, device=DEV)
        lib.dev_quantize_fp8_e4m3_scaled(w, W, sW)
        lib.qlinear_w8a8_dyn(A.view(torch.int16), W, sW, out1, fp8=True, bias=bias)
        Aq = torch.empty((M, K), dtype=torch.uint8, device=DEV)
        sA = torch.empty(1, device=DEV)
        lib.dev_quantize_fp8_e4m3_scaled(A.float(), Aq, sA)
        lib.qlinear_w8a8_fp8(Aq, sA, W, sW, out2, bias=bias)
    else:
        W = torch.empty((N, K), dtype=torch.int8, device=DEV)
        sW = torch.empty(N, device=DEV)
        lib.dev_quantize_int8_channel(w, W, sW)
        lib.qlinear_w8a8_dyn(A.view(torch.int16), W, sW, out1, bias=bias)
        Aq = torch.empty((M, K), dtype=torch.int8, device=DEV)
        sA = torch.empty(M, device=DEV)
        lib.dev_quantize_int8_channel_bf16(A.view(torch.int16), Aq, sA)
        lib.qlinear_w8a8_i8(Aq, sA, W, sW, out2, bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    ref = (A.float() @ w.T + bias).double()
    err = (out1.double() - ref).abs().max() / ref.abs().max()
    # quantization error of both operands against the unquantized product,
    # a sanity bound, not the parity bar (that is the bit equality above):
    # the reference's e4m3 encoder truncates toward zero, so its errors share
    # a sign and add up over K
    assert err < (0.15 if fp8 else 0.05), err
