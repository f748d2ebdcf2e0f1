"""The MX oracle (oracle/mx_oracle.py) against vectors of the reference's own
module (tests/golden/mx_ref.npz, written by tests/golden/make_mx_golden.py)
and against what the formats fix mathematically.  CPU only."""
import os

import numpy as np
import pytest

import mx_oracle as mx

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mx_ref.npz")


def _cases():
    z = np.load(GOLD)
    keys = sorted({k.rsplit("__", 1)[0] for k in z.files})
    return z, keys


def test_golden_vectors_all_formats_blocks_and_specials():
    z, keys = _cases()
    assert len(keys) == 99
    for key in keys:
        fmt, name, bs = key.split("__")
        bs = int(bs) or None
        x = z[key + "__x"]
        if key + "__error" in z.files:
            with pytest.raises(OverflowError):
                mx.quantize(x, fmt, bs)
            continue
        packed, scales = mx.quantize(x, fmt, bs)
        np.testing.assert_array_equal(packed, z[key + "__packed"], err_msg=key)
        np.testing.assert_array_equal(scales.reshape(z[key + "__scales"].shape), z[key + "__scales"], err_msg=key)
        deq = mx.dequantize(z[key + "__packed"], z[key + "__scales"], x.shape, fmt, bs)
        ref = z[key + "__deq"]
        assert np.array_equal(deq.reshape(ref.shape), ref, equal_nan=True), key


@pytest.mark.parametrize("fmt", [f for f in mx.FORMATS if f != "nvfp4_e2m1"])
def test_every_code_decodes_and_reencodes_to_itself(fmt):
    # each element value, placed in a block whose peak keeps the scale
    # exponent at 0 (3/4 of the largest element, or the value itself when
    # larger), encodes back to its own code; -0 encodes as +0.  The largest
    # element itself is an exact tie of the scale rule and is left out.
    sp = mx.SPECS[fmt]
    codes = np.arange(1 << sp.bits)
    vals = mx.decode(codes, sp)
    for c, v in zip(codes, vals):
        if abs(v) == mx.max_element(sp):
            continue
        blk = np.zeros(32, np.float32)
        blk[0] = 0.75 * mx.max_element(sp)
        blk[1] = v
        packed, scales = mx.quantize(blk, fmt)
        assert scales[0, 0] == 0
        got = mx.unpack(packed, sp.bits, 32)[1]
        want = 0 if v == 0 else c
        assert got == want, (fmt, c, v, got)


@pytest.mark.parametrize("fmt", mx.FORMATS)
def test_dequantized_values_are_within_half_a_step(fmt):
    # away from the no-carry clip at the top of each binade, the encoder
    # rounds to nearest: |x - deq| <= half the local step
    sp = mx.SPECS[fmt]
    x = np.random.default_rng(1).normal(0, 1, (16, 128)).astype(np.float32)
    packed, scales = mx.quantize(x, fmt)
    deq = mx.dequantize(packed, scales, x.shape, fmt)
    s = np.repeat(scales.astype(np.float64), 32, axis=1) if sp.block_size else float(scales[0])
    v = np.abs(x) / 2.0 ** s
    e = np.clip(np.floor(np.log2(np.maximum(v, 1e-300))), 1 - sp.bias, None)
    step = 2.0 ** (e - sp.mant_bits) * 2.0 ** s
    # where rounding would carry into the next exponent the reference clips
    # the mantissa instead: at the top of every binade, and at the top of the
    # subnormal range (exponent -bias values are encoded as subnormals)
    top = (v / 2.0 ** e) >= 2.0 - 2.0 ** (-sp.mant_bits - 1)
    top |= (v < 2.0 ** (1 - sp.bias)) & (v >= (2 ** sp.mant_bits - 0.5) * 2.0 ** (1 - sp.bias - sp.mant_bits))
    err = np.abs(x - deq)
    assert np.all(err[~top] <= 0.5 * step[~top] * (1 + 1e-12))
    assert np.all(err[top] <= step[top] * (1 + 1e-12))


def test_scale_maps_the_block_peak_into_the_top_binade():
    for fmt in mx.FORMATS:
        sp = mx.SPECS[fmt]
        rng = np.random.default_rng(3)
        x = (rng.normal(0, 1, (32, 32)) * 10.0 ** rng.integers(-8, 8, (32, 1))).astype(np.float32)
        packed, scales = mx.quantize(x, fmt, 32 if sp.block_size == 0 else None)
        peak = np.abs(x).max(axis=1)
        r = peak / 2.0 ** scales.reshape(-1).astype(np.float64)
        m = mx.max_element(sp)
        assert np.all(r <= m) and np.all(r > m / 2)


def test_pack_unpack_bitstream():
    rng = np.random.default_rng(0)
    for bits in (4, 6, 8):
        c = rng.integers(0, 1 << bits, 101)
        p = mx.pack(c, bits)
        assert p.size == (101 * bits + 7) // 8
        np.testing.assert_array_equal(mx.unpack(p, bits, 101), c)
    # 6-bit: codes 1, 2, 3, 4 -> bits 000001 000010 000011 000100, little end first
    assert mx.pack([1, 2, 3, 4], 6).tolist() == [0x81, 0x30, 0x10]


@pytest.mark.parametrize("fmt", ["mxfp8_e4m3", "mxfp8_e5m2"])
@pytest.mark.parametrize("seed", [0, 1])
def test_to_mfma_keeps_every_value(fmt, seed):
    """The matrix-core form decodes (as the OCP format) to the reference's
    values: exactly, except the counted half-to-even elements, which move by
    at most half a smallest subnormal at the new exponent; no code the
    matrix cores would read as NaN or inf remains; untouched blocks keep
    their bytes and exponent."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(3, (64, 512)) * 10.0 ** rng.integers(-3, 3, (64, 1))).astype(np.float32)
    x[0, :32] = np.linspace(-1, 1, 32)
    x[0, 5] = 480.0 / 7                      # scaled peak at the format's largest element
    packed, scales = mx.quantize(x, fmt)
    sp = mx.SPECS[fmt]
    p2, s2, rounded = mx.to_mfma(packed, scales, 64, 512, fmt)
    ref = mx.decode(packed.astype(np.int64), sp).reshape(64, 16, 32) * 2.0 ** scales.astype(np.float64)[..., None]
    hw = mx.ocp_decode(p2.astype(np.int64), fmt).reshape(64, 16, 32) * 2.0 ** s2.astype(np.float64)[..., None]
    assert np.isfinite(hw).all()
    changed = s2 != scales
    assert changed.any() and (s2[changed] == scales[changed] + 1).all()
    same = ~changed
    assert np.array_equal(p2.reshape(64, 16, 32)[same], packed.reshape(64, 16, 32)[same])
    diff = np.abs(hw - ref)
    unit = 2.0 ** (1 - sp.bias - sp.mant_bits) * 2.0 ** s2.astype(np.float64)[..., None]
    assert (diff <= 0.5 * unit).all()
    assert (diff > 0).sum() == rounded
    # the reference-only codes are common: about one block in twenty for E4M3
    assert changed.mean() > (0.01 if fmt == "mxfp8_e4m3" else 0.2)


def test_to_mfma_known_answers():
    # E4M3 block: 0x7F (480) and 0x7E (448) -> 0x77 (240) and 0x76 (224), s + 1;
    # subnormal / smallest-normal halving: units k = 1, 3, 5, 7, 9, 15 -> 0, 2, 2, 4, 4, 8
    blk = np.zeros(32, np.uint8)
    blk[:8] = [0x7F, 0x7E, 0x01, 0x03, 0x05, 0x07, 0x09, 0x0F]
    blk[8] = 0x80 | 0x7F
    p2, s2, rounded = mx.to_mfma(blk, np.array([3], np.int8), 1, 32, "mxfp8_e4m3")
    assert list(p2[:9]) == [0x77, 0x76, 0x00, 0x02, 0x02, 0x04, 0x04, 0x08, 0xF7]
    assert s2[0, 0] == 4 and rounded == 6
    assert mx.ocp_decode(np.array([0x7F, 0x77, 0x7E]), "mxfp8_e4m3")[1:].tolist() == [240.0, 448.0]
    assert np.isnan(mx.ocp_decode(np.array([0x7F]), "mxfp8_e4m3")[0])
    # E5M2 field 31 (65536 .. 114688 in the reference, inf / NaN in OCP) -> field 30
    b5 = np.zeros(32, np.uint8)
    b5[:3] = [0x7C, 0x7F, 0x05]
    p5, s5, r5 = mx.to_mfma(b5, np.array([-2], np.int8), 1, 32, "mxfp8_e5m2")
    assert list(p5[:3]) == [0x78, 0x7B, 0x02] and s5[0, 0] == -1 and r5 == 1
    # a block at exponent 127 cannot move up and stays as it is
    p7, s7, _ = mx.to_mfma(blk, np.array([127], np.int8), 1, 32, "mxfp8_e4m3")
    assert np.array_equal(p7, blk) and s7[0, 0] == 127
