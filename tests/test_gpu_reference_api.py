"""The reference's host-pointer quantization API served by the HIP kernels,
against the reference's own outputs (golden fixtures) and the oracle.

Bit-exact: every code, scale, zero point and dequantised value."""
import numpy as np
import pytest

import golden_checks as gc
from helpers import bits_equal

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("check", [gc.check_int8_int4, gc.check_channel, gc.check_fp8,
                                   gc.check_awq, gc.check_gptq, gc.check_meta])
def test_library_matches_reference_fixtures(lib, golden, check):
    print(f"[gpu] fixtures via {check.__name__}", flush=True)
    bad = check(lib, golden)
    assert not bad, "\n".join(bad[:20])


def test_fp8_codecs_over_every_deciding_bit(lib, oracle):
    # codes depend on bits 20..31 only: 2^16 high halves x a few low halves
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    for lo in (0, 1, 0x7FFF, 0x8000, 0xFFFF):
        x = (hi | np.uint32(lo)).view(np.float32)
        for fmt in ("e4m3", "e5m2"):
            rc, got = lib.quantize_fp8(x, fmt)
            assert rc == 0 and np.array_equal(got, oracle.quantize_fp8(x, fmt)[1]), (fmt, lo)
    codes = np.arange(256, dtype=np.uint8)
    for fmt in ("e4m3", "e5m2"):
        assert bits_equal(lib.dequantize_fp8(codes, fmt)[1], oracle.dequantize_fp8(codes, fmt)[1])
        for c in range(256):
            a = lib.fn[f"SNEPPX_fp8_{fmt}_to_float"](c)
            b = oracle.raw[f"fp8_{fmt}_to_float"](c)
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


def _specials(rng, n):
    x = rng.normal(0, 1, n).astype(np.float32)
    sp = np.array([np.nan, np.inf, -np.inf, -0.0, 1e-40, 3e38, 0.5, 2.5, -2.5], np.float32)
    x[rng.choice(n, len(sp), replace=False)] = sp
    return x


@pytest.mark.parametrize("seed", range(3))
def test_random_and_ragged_inputs_match_oracle(lib, oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    for n in (1, 2, 3, 63, 64, 65, 4095, 100003):
        for x in (rng.normal(0, 1, n).astype(np.float32),
                  _specials(rng, max(n, 16)),
                  np.full(n, 0.75, np.float32)):
            for fn in ("quantize_int8_sym", "quantize_int8_asym", "quantize_int4_sym"):
                a, b = getattr(lib, fn)(x), getattr(oracle, fn)(x)
                assert all(bits_equal(np.asarray(u), np.asarray(v)) for u, v in zip(a, b)), (fn, n)
    for rows, cols in ((1, 1), (3, 1), (7, 333), (130, 4096)):
        x = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        a, b = lib.quantize_int8_channel(x), oracle.quantize_int8_channel(x)
        assert bits_equal(a[1], b[1]) and bits_equal(a[2], b[2])
        for g in (0, 128, 7, 1000):
            a, b = lib.awq_quantize(x, g), oracle.awq_quantize(x, g)
            assert a[0] == b[0] and bits_equal(a[1], b[1]) and bits_equal(a[2], b[2])
            for bits, sym in ((4, 1), (8, 0), (3, 1), (16, 1)):
                a, b = lib.gptq_quantize(x, g, bits, sym), oracle.gptq_quantize(x, g, bits, sym)
                assert bits_equal(a[3], b[3]) and bits_equal(a[4], b[4])
                if bits <= 8:
                    assert bits_equal(a[2], b[2])


def test_error_conventions_match_reference(lib):
    empty = np.zeros(0, np.float32)
    assert lib.quantize_int8_sym(empty)[0] == -1
    assert lib.quantize_int8_asym(empty)[0] == -1
    assert lib.quantize_int4_sym(empty)[0] == -1
    assert lib.quantize_fp8(empty, "e4m3")[0] == 0
    assert lib.dequantize_fp8(np.zeros(0, np.uint8), "e5m2")[0] == 0
    assert lib.gptq_compute_hessian(np.zeros((0, 3), np.float32))[0] == -1


def test_scale_search_and_hessian_random(lib, oracle):
    rng = np.random.default_rng(77)
    w = rng.normal(0, 0.02, (3, 300)).astype(np.float32)
    act = rng.uniform(-0.3, 1.4, 300).astype(np.float32)
    a, b = lib.awq_scale_weights(w, act), oracle.awq_scale_weights(w, act)
    assert a[0] == 0 and bits_equal(a[1], b[1]) and bits_equal(a[2], b[2])
    acts = rng.normal(0, 1, (37, 70)).astype(np.float32)
    a, b = lib.gptq_compute_hessian(acts), oracle.gptq_compute_hessian(acts)
    assert bits_equal(a[1], b[1])
    for n in (1, 5, 130):
        wb = rng.normal(0, 1, n).astype(np.float32)
        h = rng.normal(0, 0.5, (n, n)).astype(np.float32)
        a, b = lib.gptq_quantize_block(wb, h, 4, 1), oracle.gptq_quantize_block(wb, h, 4, 1)
        assert all(bits_equal(np.asarray(u), np.asarray(v)) for u, v in zip(a, b))
