"""Writes tests/golden/mx_ref.npz: input/output vectors of the reference's MX
(micro-scaling) encoder/decoder, bindings/python/SneppX_ALG/interface_bindings/
mx_formats.py:99-222 (quantize_mx / dequantize_mx), which the reference's own
tests (tests/python/test_mx_formats.py) check only through SNR bounds.

Run in the build container only (it imports the reference module from
/root/reference); the .npz it writes is the committed fixture:

    python3 tests/golden/make_mx_golden.py
"""
import importlib.util
import os
import warnings

import numpy as np

REF = "/root/reference/bindings/python/SneppX_ALG/interface_bindings/mx_formats.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mx_ref.npz")

FORMATS = ["mxfp8_e4m3", "mxfp8_e5m2", "mxfp6_e3m2", "mxfp6_e2m3", "mxfp4_e2m1", "nvfp4_e2m1"]
MAXEL = {"mxfp8_e4m3": 480.0, "mxfp8_e5m2": 114688.0, "mxfp6_e3m2": 28.0, "mxfp6_e2m3": 7.5,
         "mxfp4_e2m1": 6.0, "nvfp4_e2m1": 6.0}


def inputs(fmt):
    rng = np.random.default_rng(FORMATS.index(fmt) + 1)
    m = MAXEL[fmt]
    cases = {
        "normal": rng.normal(0, 1, (8, 96)),
        "small": rng.normal(0, 0.01, (4, 64)),
        "large": rng.normal(0, 1e4, (4, 64)),
        "ragged": rng.normal(0, 1, (5, 50)),
        "wide_range": rng.normal(0, 1, (6, 32)) * 10.0 ** rng.integers(-30, 30, (6, 1)),
    }
    # exact ties: block peaks equal to max_element * 2^k, element values on
    # rounding midpoints, powers of two, zeros of both signs, subnormal range
    ties = np.zeros((6, 32))
    for r, k in enumerate([-3, -1, 0, 1, 2, 7]):
        row = rng.normal(0, 0.2, 32) * m * 2.0 ** k
        row[r] = m * 2.0 ** k
        row[31 - r] = -m * 2.0 ** k
        ties[r] = row
    cases["ties"] = ties
    grid = []
    for e in range(-12, 9):
        for f in (1.0, 1.125, 1.25, 1.5, 1.75, 1.875, 1.9375, 1.96875, 1.984375, 1.0625):
            grid.append(f * 2.0 ** e)
    g = np.array(grid[:192])
    cases["grid"] = np.concatenate([g, -g[:64]]).reshape(-1, 32)
    z = np.zeros((2, 32))
    z[1, ::3] = -0.0
    z[1, 1] = 1e-42
    cases["zeros"] = z
    # non-finite blocks (the encoder's float->int64 casts of NaN/inf, as numpy
    # does them on x86-64) next to finite ones
    nf = rng.normal(0, 1, (4, 64))
    nf[0, 3] = np.nan
    nf[1, 40] = np.inf
    nf[2, 0] = -np.inf
    nf[2, 33] = np.nan
    nf[3, 5] = 0.0
    nf[3, 7] = np.inf
    cases["nonfinite"] = nf
    return {k: np.asarray(v, np.float32) for k, v in cases.items()}


def main():
    spec = importlib.util.spec_from_file_location("ref_mx_formats", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = {}
    for fmt in FORMATS:
        for name, x in inputs(fmt).items():
            for bs in (None, 16) if fmt != "nvfp4_e2m1" else (None,):
                key = f"{fmt}__{name}__{bs or 0}"
                with warnings.catch_warnings():
                    warnings.simplefilter("ignore")
                    try:
                        packed, scales = mod.quantize_mx(x, format=fmt, block_size=bs)
                    except OverflowError:
                        # per-tensor scale outside int8 (mx_formats.py:173): recorded as an error
                        out[key + "__x"] = x
                        out[key + "__error"] = np.array(1, np.int8)
                        continue
                    deq = mod.dequantize_mx(packed, scales, x.shape, format=fmt, block_size=bs)
                out[key + "__x"] = x
                out[key + "__packed"] = np.asarray(packed, np.uint8)
                out[key + "__scales"] = np.asarray(scales, np.int8)
                out[key + "__deq"] = np.asarray(deq, np.float64)
    np.savez_compressed(OUT, **out)
    print(f"wrote {sum(k.endswith('__x') for k in out)} cases to {OUT}")


if __name__ == "__main__":
    main()
