"""The CPU oracle against the reference compiled unchanged (oracle/_ref), on
seeded random and special-value inputs beyond the committed fixtures.

Runs wherever oracle/_ref/libsnxref.so exists.  It is built from the
reference's sources in the build container (`make -C oracle ref`), kept out
of git history, and travels to the GPU box with the rest of the built
libraries; the reference's source files never do.  Where the library is
absent, the committed fixtures carry the same evidence."""
import numpy as np
import pytest

from helpers import bits_equal
from py_oracle import Reference, reference_available

pytestmark = pytest.mark.skipif(not reference_available(), reason="oracle/_ref not built here")

SPECIALS = np.array([np.nan, np.inf, -np.inf, -0.0, 1e-40, -1e-40, 3e38, -3e38, 0.5, 2.5,
                     -2.5, 1e-45], np.float32)


@pytest.fixture(scope="module")
def ref():
    return Reference()


def _inputs(rng, n):
    x = rng.normal(0, 1, n).astype(np.float32)
    y = x.copy()
    k = min(n, len(SPECIALS))
    y[rng.choice(n, k, replace=False)] = SPECIALS[:k]
    z = (rng.integers(-300, 300, n) / 2).astype(np.float32)
    return [x, y, z]


def _same(a, b):
    return all(bits_equal(np.asarray(u), np.asarray(v)) for u, v in zip(a, b))


@pytest.mark.parametrize("seed", range(4))
def test_vector_codecs_random(oracle, ref, seed):
    rng = np.random.default_rng(100 + seed)
    for _ in range(10):
        n = int(rng.integers(1, 5000))
        for x in _inputs(rng, n):
            for fn in ("quantize_int8_sym", "quantize_int8_asym", "quantize_int4_sym"):
                assert _same(getattr(oracle, fn)(x), getattr(ref, fn)(x)), fn
            for fmt in ("e4m3", "e5m2"):
                assert _same(oracle.quantize_fp8(x, fmt), ref.quantize_fp8(x, fmt))
            rows = int(rng.integers(1, 9))
            xx = x[: rows * (n // rows)].reshape(rows, -1) if n >= rows else x.reshape(1, -1)
            assert _same(oracle.quantize_int8_channel(xx), ref.quantize_int8_channel(xx))


def test_fp8_encoders_over_every_deciding_bit(oracle, ref):
    # The codes depend only on bits 20..31 of the fp32 input (sign, exponent,
    # top 3 mantissa bits; e5m2 uses fewer), so all 2^16 high halves times a
    # few low halves covers every case the encoders distinguish.
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    for lo in (0, 1, 0x7FFF, 0x8000, 0xFFFF, 0x1234):
        x = (hi | np.uint32(lo)).view(np.float32)
        for fmt in ("e4m3", "e5m2"):
            assert np.array_equal(oracle.quantize_fp8(x, fmt)[1], ref.quantize_fp8(x, fmt)[1])


@pytest.mark.parametrize("seed", range(3))
def test_group_quantizers_random(oracle, ref, seed):
    rng = np.random.default_rng(200 + seed)
    for x in _inputs(rng, 4 * 300):
        x = x.reshape(4, 300)
        for g in (0, 128, 7, 64, 300, 1000):
            assert _same(oracle.awq_quantize(x, g), ref.awq_quantize(x, g))
            for bits in (4, 8, 3, 1, 16, 0, 17):
                for sym in (0, 1):
                    a = oracle.gptq_quantize(x, g, bits, sym)
                    b = ref.gptq_quantize(x, g, bits, sym)
                    assert a[0] == b[0] and bits_equal(a[2], b[2]) and bits_equal(a[3], b[3])
                    assert bits_equal(a[4], b[4])


def test_gptq_literal_equals_closed_form(oracle, ref):
    # The oracle's literal Cholesky-of-I restatement, its closed form and the
    # reference agree, including groups poisoned by NaN / Inf.
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (3, 300)).astype(np.float32)
    x[1, 10] = np.nan
    x[2, 200] = np.inf
    for g in (128, 64):
        for bits in (4, 8, 1):
            for sym in (0, 1):
                lit = oracle.gptq_quantize_literal(x, g, bits, sym)
                cf = oracle.gptq_quantize(x, g, bits, sym)
                rf = ref.gptq_quantize(x, g, bits, sym)
                assert bits_equal(lit[2], rf[2]) and bits_equal(cf[2], rf[2])
                assert bits_equal(lit[3], rf[3]) and bits_equal(cf[3], rf[3])


@pytest.mark.parametrize("seed", range(3))
def test_scale_search_hessian_block_random(oracle, ref, seed):
    rng = np.random.default_rng(300 + seed)
    rows, cols = int(rng.integers(1, 4)), int(rng.integers(1, 300))
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    act = rng.uniform(-0.5, 1.5, cols).astype(np.float32)
    assert _same(oracle.awq_scale_weights(w, act), ref.awq_scale_weights(w, act))
    a = rng.normal(0, 1, (int(rng.integers(1, 30)), int(rng.integers(1, 40)))).astype(np.float32)
    assert _same(oracle.gptq_compute_hessian(a), ref.gptq_compute_hessian(a))
    n = int(rng.integers(1, 64))
    wb = rng.normal(0, 1, n).astype(np.float32)
    h = rng.normal(0, 1, (n, n)).astype(np.float32)
    for bits in (2, 4, 8):
        for sym in (0, 1):
            assert _same(oracle.gptq_quantize_block(wb, h, bits, sym),
                         ref.gptq_quantize_block(wb, h, bits, sym))
