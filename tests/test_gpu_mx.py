"""MX encode/decode on the GPU (include/sneppx_mx.h) against the reference's
own vectors (tests/golden/mx_ref.npz) and the oracle (oracle/mx_oracle.py).

Bar: packed codes and int8 exponents bit-exact; decoded values equal to the
reference's float64 results rounded to float32; per-tensor errors where the
reference raises."""
import os
import zlib

import numpy as np
import pytest
import torch

import mx_oracle as mx

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "mx_ref.npz")


def test_golden_vectors_bit_exact(lib):
    z = np.load(GOLD)
    keys = sorted({k.rsplit("__", 1)[0] for k in z.files})
    for key in keys:
        fmt, name, bs = key.split("__")
        bs = int(bs) or None
        x = z[key + "__x"]
        xd = torch.from_numpy(x).to(DEV)
        if key + "__error" in z.files:
            with pytest.raises(Exception, match="OverflowError"):
                lib.dev_quantize_mx(xd, fmt, bs)
            continue
        packed, scales = lib.dev_quantize_mx(xd, fmt, bs)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(packed.cpu().numpy(), z[key + "__packed"], err_msg=key)
        np.testing.assert_array_equal(scales.cpu().numpy().reshape(z[key + "__scales"].shape),
                                      z[key + "__scales"], err_msg=key)
        # decode the reference's own codes
        y = lib.dev_dequantize_mx(torch.from_numpy(z[key + "__packed"]).to(DEV),
                                  torch.from_numpy(z[key + "__scales"].ravel().copy()).to(DEV),
                                  x.shape, fmt, bs)
        ref = z[key + "__deq"].astype(np.float32)
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.reshape(got.shape).view(np.uint32)), key


@pytest.mark.parametrize("fmt", mx.FORMATS)
@pytest.mark.parametrize("shape,bs", [((64, 4096), None), ((3, 1000), None), ((7, 96), 16),
                                      ((5, 200), 64), ((2, 333), -1)])
def test_random_tensors_match_the_oracle(lib, fmt, shape, bs):
    print(f"[gpu] mx {fmt} {shape} bs={bs}", flush=True)
    rng = np.random.default_rng(zlib.crc32(repr((fmt, shape, bs)).encode()))
    x = (rng.normal(0, 1, shape) * 10.0 ** rng.integers(-6, 6, (shape[0], 1))).astype(np.float32)
    x[0, :5] = [0.0, -0.0, 1e-40, -3.0, 6.0]
    packed, scales = lib.dev_quantize_mx(torch.from_numpy(x).to(DEV), fmt, bs)
    torch.cuda.synchronize()
    po, so = mx.quantize(x, fmt, bs)
    np.testing.assert_array_equal(packed.cpu().numpy(), po)
    np.testing.assert_array_equal(scales.cpu().numpy().ravel(), so.ravel())
    y = lib.dev_dequantize_mx(packed, scales.reshape(-1), shape, fmt, bs)
    yo = mx.dequantize(po, so, shape, fmt, bs).astype(np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yo.view(np.uint32))


def test_nonfinite_blocks_and_per_tensor_errors(lib):
    x = np.random.default_rng(0).normal(0, 1, (3, 64)).astype(np.float32)
    x[0, 3] = np.nan
    x[1, 40] = np.inf
    x[2, 7] = -np.inf
    for fmt in mx.FORMATS[:5]:
        packed, scales = lib.dev_quantize_mx(torch.from_numpy(x).to(DEV), fmt)
        po, so = mx.quantize(x, fmt)
        np.testing.assert_array_equal(packed.cpu().numpy(), po)
        np.testing.assert_array_equal(scales.cpu().numpy().ravel(), so.ravel())
    # per tensor: NaN -> peak 1.0 (no error); an infinity raises
    xn = x.copy()
    xn[1, 40] = 1.0
    xn[2, 7] = 2.0
    packed, scales = lib.dev_quantize_mx(torch.from_numpy(xn).to(DEV), "nvfp4_e2m1")
    po, so = mx.quantize(xn, "nvfp4_e2m1")
    np.testing.assert_array_equal(packed.cpu().numpy(), po)
    assert int(scales.cpu()[0]) == int(so[0])
    with pytest.raises(Exception, match="infinite peak"):
        lib.dev_quantize_mx(torch.from_numpy(x[1:2]).to(DEV), "nvfp4_e2m1")


def test_rejects_block_sizes_that_are_not_byte_aligned(lib):
    with pytest.raises(Exception, match="block size"):
        lib.dev_quantize_mx(torch.zeros((2, 30), device=DEV), "mxfp6_e2m3", 12)


@pytest.mark.parametrize("M,N,K,out", [(128, 128, 64, "f32"), (300, 200, 512, "f32"), (1, 4096, 4096, "bf16"),
                                       (2048, 1024, 4096, "f32"), (257, 450, 768, "f32"),
                                       (384, 448, 1024, "bf16"), (300, 260, 3072, "bf16")])
def test_mxfp4_gemm_against_dequantized_product(lib, M, N, K, out):
    print(f"[gpu] mxfp4 gemm M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    w = (rng.normal(0, 0.02, (N, K)) * 10.0 ** rng.integers(-2, 2, (N, 1))).astype(np.float32)
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(a).to(DEV), "mxfp4_e2m1")
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(w).to(DEV), "mxfp4_e2m1")
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_mxfp4_gemm(pa, sa, pw, sw, y, M, N, K)
    torch.cuda.synchronize()
    da = mx.dequantize(pa.cpu().numpy(), sa.cpu().numpy(), (M, K), "mxfp4_e2m1")
    dw = mx.dequantize(pw.cpu().numpy(), sw.cpu().numpy(), (N, K), "mxfp4_e2m1")
    ref = da @ dw.T
    got = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= (1e-5 if out == "f32" else 1e-2), err


def test_mxfp4_gemm_rejects_k_not_multiple_of_64(lib):
    z = torch.zeros(64, dtype=torch.uint8, device=DEV)
    s = torch.zeros(8, dtype=torch.int8, device=DEV)
    with pytest.raises(Exception, match="multiple of 64"):
        lib.qlinear_mxfp4_gemm(z, s, z, s, torch.empty((2, 2), device=DEV), 2, 2, 96)


MX_BLOCK32 = ["mxfp8_e4m3", "mxfp8_e5m2", "mxfp6_e3m2", "mxfp6_e2m3"]


def _mx_operand(rng, rows, K, spread):
    x = rng.normal(0, 1, (rows, K)) * 10.0 ** rng.integers(-spread, spread + 1, (rows, 1))
    return x.astype(np.float32)


def _mfma_values(packed, scales, rows, K, fmt):
    """float64 values of the matrix-core form of a reference MX tensor: the
    oracle's re-encoding, decoded as the OCP format (FP6: the reference's own
    codes and decode)."""
    p2, s2, _ = mx.to_mfma(packed, scales, rows, K, fmt)
    sp = mx.SPECS[fmt]
    if sp.bits != 8:
        return mx.dequantize(p2, s2, (rows, K), fmt).astype(np.float64)
    v = mx.ocp_decode(p2.astype(np.int64), fmt).reshape(rows, K // 32, 32)
    return (v * 2.0 ** s2.astype(np.float64)[..., None]).reshape(rows, K)


@pytest.mark.parametrize("fmt", MX_BLOCK32)
def test_to_mfma_bit_exact(lib, fmt):
    print(f"[gpu] mx_to_mfma {fmt}", flush=True)
    rng = np.random.default_rng(7)
    rows, cols = 96, 1024
    x = _mx_operand(rng, rows, cols, 3)
    x[0, :32] = 480.0 / 7     # a block whose peak lands on the format's largest element
    p, s = lib.dev_quantize_mx(torch.from_numpy(x).to(DEV), fmt)
    p2, s2, rounded = lib.mx_to_mfma(p, s, rows, cols, fmt)
    torch.cuda.synchronize()
    ep, es, er = mx.to_mfma(p.cpu().numpy(), s.cpu().numpy(), rows, cols, fmt)
    assert np.array_equal(p2.cpu().numpy().reshape(-1), ep)
    assert np.array_equal(s2.cpu().numpy().reshape(es.shape), es)
    assert int(rounded.item()) == er
    if mx.SPECS[fmt].bits == 8:
        assert not np.array_equal(es, s.cpu().numpy().reshape(es.shape))


@pytest.mark.parametrize("fmt", MX_BLOCK32)
@pytest.mark.parametrize("M,N,K", [(256, 224, 128), (300, 500, 384), (1, 17, 256), (513, 449, 1024)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_mx_gemm_against_dequantized_product(lib, fmt, M, N, K, out):
    """MXFP8 / MXFP6 GEMM on the scaled matrix cores against the float64
    product of the operands' matrix-core values (the oracle's re-encoding),
    which lies within 1e-6 of the reference's own dequantized product."""
    print(f"[gpu] mx gemm {fmt} M={M} N={N} K={K} {out}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    a, w = _mx_operand(rng, M, K, 1), _mx_operand(rng, N, K, 2) * 0.02
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(a).to(DEV), fmt)
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(w).to(DEV), fmt)
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_mx_gemm(pa, sa, pw, sw, fmt, y, M, N, K)
    torch.cuda.synchronize()
    hpa, hsa, hpw, hsw = (t.cpu().numpy() for t in (pa, sa, pw, sw))
    va, vw = _mfma_values(hpa, hsa, M, K, fmt), _mfma_values(hpw, hsw, N, K, fmt)
    ref = va @ vw.T
    got = y.float().cpu().numpy().astype(np.float64)
    if out == "f32":
        # exact products; the scaled matrix cores sum each 128-element step
        # keeping about 16 bits relative to its sum of |products| (measured
        # 2.1e-5 of sum |a_k w_k| for the FP8 and E3M2 formats, 0 for E2M3),
        # then add it to the fp32 accumulator: bound 2^-13 sum_k |a_k w_k|
        absprod = np.abs(va) @ np.abs(vw).T
        rel = (np.abs(got - ref) / np.maximum(absprod, 1e-300)).max()
        print(f"[gpu]   max |err| / sum|a w| = {rel:.3g}", flush=True)
        assert rel <= 2.0 ** -13, rel
    else:
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-2
    # the re-encoding moves the reference's own product by far less than that
    refd = mx.dequantize(hpa, hsa, (M, K), fmt) @ mx.dequantize(hpw, hsw, (N, K), fmt).T
    assert np.abs(ref - refd).max() <= 1e-6 * np.abs(refd).max()


@pytest.mark.parametrize("fmt", ["mxfp8_e4m3", "mxfp6_e2m3"])
def test_mx_gemm_on_weights_kept_in_matrix_core_form(lib, fmt):
    """Weights converted once (mx_to_mfma) and the activations per call give
    the same bits as the converting entry point."""
    print(f"[gpu] mx gemm mfma-form {fmt}", flush=True)
    rng = np.random.default_rng(11)
    M, N, K = 130, 260, 512
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(_mx_operand(rng, M, K, 1)).to(DEV), fmt)
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(_mx_operand(rng, N, K, 1)).to(DEV), fmt)
    y1 = torch.empty((M, N), device=DEV)
    y2 = torch.empty_like(y1)
    lib.qlinear_mx_gemm(pa, sa, pw, sw, fmt, y1, M, N, K)
    a2, sa2, _ = lib.mx_to_mfma(pa, sa, M, K, fmt)
    w2, sw2, _ = lib.mx_to_mfma(pw, sw, N, K, fmt)
    lib.qlinear_mx_gemm(a2, sa2, w2, sw2, fmt, y2, M, N, K, mfma_form=True)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_mx_gemm_rejects_bad_shapes(lib):
    z = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    s = torch.zeros(128, dtype=torch.int8, device=DEV)
    y = torch.empty((2, 2), device=DEV)
    with pytest.raises(Exception, match="multiple of 128"):
        lib.qlinear_mx_gemm(z, s, z, s, "mxfp8_e4m3", y, 2, 2, 96)
    # blocks the matrix cores cannot scale exactly (not a multiple of 32)
    with pytest.raises(Exception, match="blocks of 32"):
        lib.qlinear_mx_gemm_bs(z, s, z, s, "mxfp4_e2m1", y, 2, 2, 128, block_size=16)
    with pytest.raises(Exception, match="multiple of the block"):
        lib.qlinear_mx_gemm_bs(z, s, z, s, "mxfp4_e2m1", y, 2, 2, 192, block_size=128)


def _expanded(scales, rows, K, bs, fmt):
    """block-32 exponents [rows][K/32] of an operand quantized with block bs
    (None: the format's default; per tensor when <= 0): what the GEMM's scale
    expansion stands for."""
    s = np.asarray(scales, np.int64).reshape(-1)
    if bs is None:
        bs = mx.SPECS[fmt].block_size
    if bs <= 0:
        return np.full((rows, K // 32), s[0], np.int64)
    return np.repeat(s.reshape(rows, K // bs), bs // 32, axis=1)


def _values(packed, scales, rows, K, fmt, bs):
    """float64 matrix-core values of an operand: its block-32 exponents, the
    FP8 codes through the oracle's re-encoding (exact but for the counted
    half-to-even elements), FP6 / FP4 as the reference decodes them."""
    ef = "mxfp4_e2m1" if fmt == "nvfp4_e2m1" else fmt
    s32 = _expanded(scales, rows, K, bs, fmt)
    if mx.SPECS[ef].bits == 8:
        return _mfma_values(np.asarray(packed).reshape(-1), s32.astype(np.int8), rows, K, ef)
    return mx.dequantize(np.asarray(packed).reshape(-1), s32.astype(np.int8), (rows, K), ef).astype(np.float64)


@pytest.mark.parametrize("M,N,K", [(256, 224, 256), (300, 500, 512), (1, 17, 128), (2048, 1024, 1024)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_nvfp4_gemm_against_dequantized_product(lib, M, N, K, out):
    """NVFP4 (E2M1 codes, one per-tensor exponent each, mx_formats.py:72-73,
    165-172) through the E2M1 matrix-core kernels against the float64
    product of the reference's dequantized operands."""
    print(f"[gpu] nvfp4 gemm M={M} N={N} K={K} {out}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K)
    a = rng.normal(0, 1, (M, K)).astype(np.float32)
    w = (rng.normal(0, 0.02, (N, K))).astype(np.float32)
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(a).to(DEV), "nvfp4_e2m1")
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(w).to(DEV), "nvfp4_e2m1")
    assert sa.numel() == 1 and sw.numel() == 1
    y = torch.empty((M, N), dtype=torch.float32 if out == "f32" else torch.bfloat16, device=DEV)
    lib.qlinear_mx_gemm(pa, sa, pw, sw, "nvfp4_e2m1", y, M, N, K)
    torch.cuda.synchronize()
    da = mx.dequantize(pa.cpu().numpy(), sa.cpu().numpy(), (M, K), "nvfp4_e2m1").astype(np.float64)
    dw = mx.dequantize(pw.cpu().numpy(), sw.cpu().numpy(), (N, K), "nvfp4_e2m1").astype(np.float64)
    ref = da @ dw.T
    got = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= (1e-5 if out == "f32" else 1e-2), err


def test_nvfp4_gemm_extreme_exponents(lib):
    """An operand whose per-tensor exponent is -128 (peak just above FLT_MIN)
    against one near 2^100: the product's exponent is split between the two
    E8M0 scales, so neither is clamped (clamping -128 to -127 would double
    every output)."""
    print("[gpu] nvfp4 gemm extreme exponents", flush=True)
    rng = np.random.default_rng(31)
    M, N, K = 130, 260, 512
    a = (rng.uniform(-1, 1, (M, K)) * 1.7e-38).astype(np.float32)
    a[0, 0] = 1.7e-38
    w = (rng.normal(0, 1, (N, K)) * 2.0 ** 100).astype(np.float32)
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(a).to(DEV), "nvfp4_e2m1")
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(w).to(DEV), "nvfp4_e2m1")
    assert int(sa.cpu()[0]) == -128 and int(sw.cpu()[0]) > 90
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_mx_gemm(pa, sa, pw, sw, "nvfp4_e2m1", y, M, N, K)
    torch.cuda.synchronize()
    da = mx.dequantize(pa.cpu().numpy(), sa.cpu().numpy(), (M, K), "nvfp4_e2m1").astype(np.float64)
    dw = mx.dequantize(pw.cpu().numpy(), sw.cpu().numpy(), (N, K), "nvfp4_e2m1").astype(np.float64)
    ref = da @ dw.T
    got = y.cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("fmt,bs", [("mxfp4_e2m1", 64), ("mxfp4_e2m1", -1), ("mxfp8_e4m3", 128),
                                    ("mxfp8_e5m2", -1), ("mxfp6_e3m2", 64), ("mxfp6_e2m3", -1),
                                    ("nvfp4_e2m1", 32), ("nvfp4_e2m1", 256)])
def test_mx_gemm_other_blocks(lib, fmt, bs):
    """Operands quantized with a block override or per tensor (the
    reference's block_size argument, mx_formats.py:147-150,165) against the
    float64 product of their matrix-core values."""
    print(f"[gpu] mx gemm {fmt} block {bs}", flush=True)
    rng = np.random.default_rng(abs(bs) + len(fmt))
    M, N, K = 300, 260, 1024
    a, w = _mx_operand(rng, M, K, 1), _mx_operand(rng, N, K, 1) * 0.02
    pa, sa = lib.dev_quantize_mx(torch.from_numpy(a).to(DEV), fmt, bs)
    pw, sw = lib.dev_quantize_mx(torch.from_numpy(w).to(DEV), fmt, bs)
    y = torch.empty((M, N), device=DEV)
    lib.qlinear_mx_gemm_bs(pa, sa.reshape(-1), pw, sw.reshape(-1), fmt, y, M, N, K, block_size=bs)
    torch.cuda.synchronize()
    hpa, hsa, hpw, hsw = (t.cpu().numpy() for t in (pa, sa, pw, sw))
    va, vw = _values(hpa, hsa, M, K, fmt, bs), _values(hpw, hsw, N, K, fmt, bs)
    ref = va @ vw.T
    got = y.cpu().numpy().astype(np.float64)
    absprod = np.abs(va) @ np.abs(vw).T
    assert (np.abs(got - ref) / np.maximum(absprod, 1e-300)).max() <= 2.0 ** -13
    refd = mx.dequantize(hpa, hsa, (M, K), fmt, bs) @ mx.dequantize(hpw, hsw, (N, K), fmt, bs).T
    assert np.abs(ref - refd).max() <= 1e-6 * np.abs(refd).max()


@pytest.mark.parametrize("fmt", ["mxfp4_e2m1", "nvfp4_e2m1", "mxfp8_e4m3", "mxfp6_e3m2", "mxfp6_e2m3"])
def test_mx_gemm_full_c4_shape_sampled(lib, fmt):
    """The bench's 2048 x 14336 x 4096 MX GEMMs (bf16 out): the four corner
    and eight random 64 x 64 output tiles against the float64 product of the
    matrix-core values of those rows and columns (tolerance 1e-2 of the
    tile's largest output)."""
    print(f"[gpu] mx gemm {fmt} 2048x14336x4096 sampled", flush=True)
    M, N, K = 2048, 14336, 4096
    g = torch.Generator(device=DEV).manual_seed(19)
    a = torch.randn((M, K), device=DEV, generator=g)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    pa, sa = lib.dev_quantize_mx(a, fmt)
    pw, sw = lib.dev_quantize_mx(w, fmt)
    del a, w
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_mx_gemm(pa, sa.reshape(-1), pw, sw.reshape(-1), fmt, y, M, N, K)
    torch.cuda.synchronize()
    rb = K * mx.SPECS["mxfp4_e2m1" if fmt == "nvfp4_e2m1" else fmt].bits // 8
    hpa, hpw = pa.reshape(M, rb).cpu().numpy(), pw.reshape(N, rb).cpu().numpy()
    hsa, hsw = sa.cpu().numpy().reshape(-1), sw.cpu().numpy().reshape(-1)
    bs = None if fmt == "nvfp4_e2m1" else 32
    rng = np.random.default_rng(5)
    tiles = [(0, 0), (M - 64, 0), (0, N - 64), (M - 64, N - 64)] + \
        [(int(rng.integers(0, M // 64)) * 64, int(rng.integers(0, N // 64)) * 64) for _ in range(8)]
    got_all = y.float()
    for m0, n0 in tiles:
        if fmt == "nvfp4_e2m1":
            ssa, ssw = hsa, hsw
        else:
            ssa = hsa.reshape(M, K // 32)[m0:m0 + 64].ravel()
            ssw = hsw.reshape(N, K // 32)[n0:n0 + 64].ravel()
        va = _values(hpa[m0:m0 + 64].ravel(), ssa, 64, K, fmt, bs)
        vw = _values(hpw[n0:n0 + 64].ravel(), ssw, 64, K, fmt, bs)
        ref = va @ vw.T
        got = got_all[m0:m0 + 64, n0:n0 + 64].cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err <= 1e-2, (m0, n0, err)
