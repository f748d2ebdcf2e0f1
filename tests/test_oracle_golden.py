"""The CPU oracle against the reference's own outputs (golden fixtures) and
against the reference's known-answer tests.  CPU only."""
import math

import numpy as np
import pytest

import golden_checks as gc


@pytest.mark.parametrize("check", [gc.check_int8_int4, gc.check_channel, gc.check_fp8,
                                   gc.check_awq, gc.check_gptq, gc.check_meta])
def test_oracle_matches_reference_fixtures(oracle, golden, check):
    bad = check(oracle, golden)
    assert not bad, "\n".join(bad[:20])


def test_kat_int8_ties_away_from_zero(oracle):
    # quantize_int8.c:61 uses roundf: 0.5 -> 1, 2.5 -> 3, -2.5 -> -3
    rc, q, s = oracle.quantize_int8_sym(np.array([127, .5, 2.5, -2.5], np.float32))
    assert rc == 0 and s == 1.0 and q.tolist() == [127, 1, 3, -3]


def test_kat_int4_nibble_order(oracle):
    # element 2i in the low nibble, 2i+1 in the high nibble (quantize_int8.c:206-216)
    rc, p, s = oracle.quantize_int4_sym(np.array([7, -7, 3.5, -3.5, 1, 0], np.float32))
    assert rc == 0 and s == 1.0 and p.tolist() == [0x97, 0xC4, 0x01]


def test_kat_fp8_codes(oracle):
    e4 = {0.0: 0x00, 1.0: 0x38, -1.0: 0xB8, 2.5: 0x42, 127.0: 0x6F, -64.0: 0xE8, 0.125: 0x20,
          240.0: 0x77, 256.0: 0x78, 300.0: 0x79, 448.0: 0x7E, 600.0: 0x78, 0.015625: 0x08,
          0.0156: 0x00}
    for v, c in e4.items():
        assert oracle.raw["float_to_fp8_e4m3"](v) == c, v
    assert oracle.raw["fp8_e4m3_to_float"](0x6F) == 120.0
    assert math.isinf(oracle.raw["fp8_e4m3_to_float"](0x78))
    assert math.isnan(oracle.raw["fp8_e4m3_to_float"](0x7E))
    assert oracle.raw["fp8_e4m3_to_float"](0x80) == 0.0
    e5 = {1.0: 0x3C, 1.25: 0x3C, 1.5: 0x3D, 1.75: 0x3D, 3.0: 0x41, 256.0: 0x5C, -128.0: 0xD8,
          0.25: 0x34}
    for v, c in e5.items():
        assert oracle.raw["float_to_fp8_e5m2"](v) == c, v
    assert oracle.raw["fp8_e5m2_to_float"](0x3D) == 1.25
    assert oracle.raw["fp8_e5m2_to_float"](0x41) == 2.5


def test_kat_awq_and_gptq(oracle):
    # test_quantize.c:134-138: 2x4, group 2 -> scales 2/127, 4/127 per row
    rc, q, s = oracle.awq_quantize(np.array([[1, 2, 3, 4], [-1, -2, -3, -4]], np.float32), 2)
    assert rc == 0
    np.testing.assert_array_equal(s, np.float32([[2 / 127, 4 / 127], [2 / 127, 4 / 127]]))
    # gptq bits 4, group 3 on one row
    rc, _, q, s, z = oracle.gptq_quantize(np.array([[.7, -.1, .35, .2, -.6, .05]], np.float32), 3, 4, 1)
    assert rc == 0 and q.ravel().tolist() == [7, -1, 4, 2, -7, 1] and z.ravel().tolist() == [0, 0]
    assert s.ravel()[0] == np.float32(float.fromhex("0x1.99999ap-4"))
    assert s.ravel()[1] == np.float32(float.fromhex("0x1.5f15f2p-4"))
    # test_quantize.c:146-148 Hessian: [[17,0,22],[0,45,0],[22,0,29]] + 1.7e-4 on the diagonal
    rc, h = oracle.gptq_compute_hessian(np.array([1, 0, 2, 0, 3, 0, 4, 0, 5, 0, 6, 0],
                                                 np.float32).reshape(4, 3))
    reg = np.float32(1e-5) * np.float32(17)
    want = np.array([[17, 0, 22], [0, 45, 0], [22, 0, 29]], np.float32) + np.eye(3, dtype=np.float32) * reg
    np.testing.assert_array_equal(h, want)


def test_fake_quant_reference_kats(oracle):
    # tests/unit/test_fake_quant.c:28-31 (scale 1, 8 bits)
    rc, y = oracle.fake_quant(np.array([1.4, -0.6, 200, -200], np.float32), 1.0, 8)
    assert rc == 0 and y.tolist() == [1.0, -1.0, 127.0, -128.0]
    # floor(x + 0.5): ties go toward +inf, unlike roundf
    rc, y = oracle.fake_quant(np.array([0.5, -0.5, 1.5, -1.5, 2.5], np.float32), 1.0, 8)
    assert y.tolist() == [1.0, 0.0, 2.0, -1.0, 3.0]
    assert oracle.fake_quant(np.ones(2, np.float32), 0.0, 8)[0] == -1
    assert oracle.fake_quant(np.ones(2, np.float32), 1.0, 1)[0] == -1


def test_error_conventions(oracle):
    empty = np.zeros(0, np.float32)
    assert oracle.quantize_int8_sym(empty)[0] == -1          # n == 0 -> -1
    assert oracle.quantize_int4_sym(empty)[0] == -1
    assert oracle.quantize_fp8(empty, "e4m3")[0] == 0         # fp8 arrays accept n == 0
    assert oracle.dequantize_fp8(np.zeros(0, np.uint8), "e5m2")[0] == 0


def test_fp8_decode_is_exhaustive_and_roundtrips(oracle):
    codes = np.arange(256, dtype=np.uint8)
    for fmt in ("e4m3", "e5m2"):
        _, dec = oracle.dequantize_fp8(codes, fmt)
        finite = np.isfinite(dec)
        _, back = oracle.quantize_fp8(dec[finite], fmt)
        if fmt == "e4m3":
            # exact round trip for every normal code the encoder can emit
            emit = finite & ((codes & 0x78) != 0)
            assert np.array_equal(back[emit[finite]], codes[emit])
