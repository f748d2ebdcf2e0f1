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
                                       (384, 448, 1024, "bf16")])
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
