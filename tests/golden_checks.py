"""Fixture-driven parity checks shared by the oracle tests (CPU) and the
product tests (GPU).

`impl` is anything with the numpy-facing methods of oracle/py_oracle._Lib:
the oracle itself, or the product binding in sneppx-alg_amd/sneppx_quant.py
(which calls the HIP library through its C-ABI).  Each check returns a list
of human-readable mismatches; an empty list is a pass.  Expected values are
the reference's own outputs (tests/golden/gen_golden.py).
"""
import hashlib

import numpy as np

from helpers import bits_equal, cases


def _cmp(bad, name, got, want):
    if not bits_equal(got, want):
        g, w = np.asarray(got), np.asarray(want)
        if g.shape == w.shape and g.size:
            gi = g.view(np.uint32) if g.dtype == np.float32 else g
            wi = w.view(np.uint32) if w.dtype == np.float32 else w
            idx = np.flatnonzero(gi.ravel() != wi.ravel())
            bad.append(f"{name}: {idx.size} differ, first at {idx[:5]}: "
                       f"got {g.ravel()[idx[:3]]} want {w.ravel()[idx[:3]]}")
        else:
            bad.append(f"{name}: got {g!r} want {w!r}")


def check_int8_int4(impl, golden):
    bad = []
    for case, f in cases(golden, "int8_sym").items():
        rc, q, s = impl.quantize_int8_sym(f["x"])
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".q", q, f["q"])
        _cmp(bad, case + ".s", np.float32(s), f["s"])
    for case, f in cases(golden, "int8_asym").items():
        rc, q, s, z = impl.quantize_int8_asym(f["x"])
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".q", q, f["q"])
        _cmp(bad, case + ".s", np.float32(s), f["s"]); _cmp(bad, case + ".z", z, f["z"])
    for case, f in cases(golden, "int4_sym").items():
        rc, p, s = impl.quantize_int4_sym(f["x"])
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".p", p, f["p"])
        _cmp(bad, case + ".s", np.float32(s), f["s"])
    for case, f in cases(golden, "deq").items():
        s, z = np.float32(f["s"]), int(f["z"])
        _cmp(bad, case + ".sym", impl.dequantize_int8_sym(f["codes"], s)[1], f["y_sym"])
        _cmp(bad, case + ".asym", impl.dequantize_int8_asym(f["codes"], s, z)[1], f["y_asym"])
        _cmp(bad, case + ".int4",
             impl.dequantize_int4_sym(f["codes"].view(np.uint8), 512, s)[1], f["y_int4"])
    return bad


def c1_weights(seed, rows, cols):
    return np.random.default_rng(int(seed)).normal(0.0, 0.02, (int(rows), int(cols))).astype(np.float32)


def check_channel(impl, golden):
    bad = []
    for case, f in cases(golden, "int8_channel").items():
        if case == "int8_channel_c1":
            x = c1_weights(f["seed"], f["rows"], f["cols"])
            if hashlib.sha256(x.tobytes()).hexdigest() != str(f["sha"]):
                bad.append("int8_channel_c1: regenerated input differs from the fixture's SHA-256")
                continue
        else:
            x = f["x"]
        rc, q, s = impl.quantize_int8_channel(x)
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".q", q, f["q"])
        _cmp(bad, case + ".s", s, f["s"])
    return bad


def check_fp8(impl, golden):
    bad = []
    for fmt in ("e4m3", "e5m2"):
        f = cases(golden, "fp8_" + fmt)["fp8_" + fmt]
        _cmp(bad, fmt + ".dec", impl.dequantize_fp8(f["codes"], fmt)[1].view(np.uint32), f["dec_bits"])
        _cmp(bad, fmt + ".enc", impl.quantize_fp8(f["x"], fmt)[1], f["enc"])
    k = cases(golden, "fp8_kat")["fp8_kat"]
    _cmp(bad, "kat.e4m3", impl.quantize_fp8(k["x"], "e4m3")[1], k["e4m3"])
    _cmp(bad, "kat.e5m2", impl.quantize_fp8(k["x"], "e5m2")[1], k["e5m2"])
    return bad


def check_awq(impl, golden):
    bad = []
    for case, f in cases(golden, "awq").items():
        if case.startswith("awq_sw"):
            rc, w, s = impl.awq_scale_weights(f["x"], f["act"])
            _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".w", w, f["w"])
            _cmp(bad, case + ".s", s, f["s"])
        else:
            rc, q, s = impl.awq_quantize(f["x"], int(f["g"]))
            _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".q", q, f["q"])
            _cmp(bad, case + ".s", s, f["s"])
    return bad


def check_gptq(impl, golden):
    bad = []
    for case, f in cases(golden, "hessian").items():
        rc, h = impl.gptq_compute_hessian(f["act"])
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".h", h, f["h"])
    for case, f in cases(golden, "gptq_block").items():
        rc, w, qw, s, z = impl.gptq_quantize_block(f["w_in"], f["h"], int(f["bits"]), int(f["sym"]))
        _cmp(bad, case + ".w", w, f["w"]); _cmp(bad, case + ".qw", qw, f["qw"])
        _cmp(bad, case + ".s", np.float32(s), f["s"]); _cmp(bad, case + ".z", z, f["z"])
    for case, f in cases(golden, "gptq").items():
        if case.startswith("gptq_block"):
            continue
        rc, _, q, s, z = impl.gptq_quantize(f["x"], int(f["g"]), int(f["bits"]), int(f["sym"]))
        _cmp(bad, case + ".rc", rc, f["rc"]); _cmp(bad, case + ".s", s, f["s"])
        _cmp(bad, case + ".z", z, f["z"])
        b = int(f["bits"])
        if not 1 <= b <= 16:
            b = 8                      # gptq.c:196
        if b <= 8:                     # wider codes are never stored (gptq.c:227-234)
            _cmp(bad, case + ".q", q, f["q"])
    return bad


def check_meta(impl, golden):
    bad = []
    f = cases(golden, "meta")["meta"]
    for m, p, nm in zip(f["modes"], f["params"], f["names"]):
        rc, got = impl.quant_params_create(int(m))
        if rc != 0 or not np.array_equal(np.array(got, np.float64), p):
            bad.append(f"params({m}): {got} vs {p}")
        if impl.quant_mode_name(int(m)) != str(nm):
            bad.append(f"name({m}): {impl.quant_mode_name(int(m))} vs {nm}")
    return bad
