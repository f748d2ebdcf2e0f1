"""CPU statement of the reference's MX (micro-scaling) encoder and decoder.

TEST INFRASTRUCTURE ONLY: imported by tests/ (the checker); the product path
is sneppx-alg_amd (HIP) and never calls this.

Follows bindings/python/SneppX_ALG/interface_bindings/mx_formats.py:
  - formats and their parameters            mx_formats.py:53-72
  - element decode                          mx_formats.py:75-96
  - element encode (no carry into the exponent: a mantissa that rounds up to
    2^m_bits is clipped to 2^m_bits - 1)     mx_formats.py:99-123
  - largest element, shared-scale exponent  mx_formats.py:126-141
  - quantize_mx / dequantize_mx             mx_formats.py:144-222
for 2-D inputs blocked along the last axis (block_axis=-1).

Where the reference relies on numpy casting a NaN or an infinity to int64
(the exponent of a non-finite element or block), this states what that cast
does on x86-64 - it yields INT64_MIN - explicitly:
  * a block containing NaN or +-inf gets scale exponent INT64_MIN, stored as
    int8 0; its elements are divided by 2**INT64_MIN = 0.0, so finite nonzero
    and infinite elements encode as sign | largest subnormal mantissa and
    zeros / NaNs as code 0;
  * per tensor (block size 0), a NaN peak is replaced by 1.0 (a false `> 0`)
    and an infinite peak raises, as int(ceil(inf)) does.
Pinned against tests/golden/mx_ref.npz (vectors of the reference module
itself) in tests/test_mx_oracle.py.
"""
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Spec:
    name: str
    bits: int
    exp_bits: int
    mant_bits: int
    bias: int
    block_size: int


SPECS = {
    "mxfp8_e4m3": Spec("mxfp8_e4m3", 8, 4, 3, 7, 32),
    "mxfp8_e5m2": Spec("mxfp8_e5m2", 8, 5, 2, 15, 32),
    "mxfp6_e3m2": Spec("mxfp6_e3m2", 6, 3, 2, 3, 32),
    "mxfp6_e2m3": Spec("mxfp6_e2m3", 6, 2, 3, 1, 32),
    "mxfp4_e2m1": Spec("mxfp4_e2m1", 4, 2, 1, 1, 32),
    "nvfp4_e2m1": Spec("nvfp4_e2m1", 4, 2, 1, 1, 0),
}
FORMATS = list(SPECS)


def max_element(sp):
    """(2 - 2^-m) * 2^(e_max_field - bias): every exponent field is finite."""
    return (2.0 - 2.0 ** (-sp.mant_bits)) * 2.0 ** ((1 << sp.exp_bits) - 1 - sp.bias)


def _floor_log2(mag):
    """floor(log2(mag)) for positive finite float64 values (exact via frexp)."""
    _, e = np.frexp(mag)
    return e.astype(np.int64) - 1


def encode(v, sp):
    """Codes (int64, 0 .. 2^bits-1) of float64 values v already divided by
    their block scale."""
    v = np.asarray(v, np.float64)
    sign = (v < 0).astype(np.int64)
    mag = np.abs(v)
    finite = np.isfinite(mag)
    fmax = (1 << sp.exp_bits) - 1
    mmax = (1 << sp.mant_bits) - 1
    # exponent: floor(log2(mag)); zeros take log2(1e-30); non-finite -> INT64_MIN
    m0 = np.where(mag == 0, 1e-30, np.where(finite, mag, 1.0))
    e = np.where(finite, _floor_log2(m0), np.iinfo(np.int64).min)
    e = np.clip(e, -sp.bias, fmax - sp.bias)
    sub = e <= -sp.bias
    field = np.where(sub, 0, np.clip(e + sp.bias, 1, fmax))
    with np.errstate(over="ignore", invalid="ignore"):
        sub_m = np.round(mag * 2.0 ** (sp.mant_bits + sp.bias - 1))
        nor_m = np.round((mag / 2.0 ** e - 1.0) * (1 << sp.mant_bits))
    mant = np.where(sub, sub_m, nor_m)
    # a NaN mantissa casts to INT64_MIN, whose low bits are zero
    mant = np.where(np.isnan(mant), 0, np.clip(mant, 0, mmax)).astype(np.int64)
    return (sign << (sp.bits - 1)) | (field << sp.mant_bits) | mant


def pack(codes, bits):
    """Little-endian bitstream: code i in bits [bits*i, bits*(i+1))."""
    codes = np.asarray(codes, np.int64).ravel()
    n = codes.size
    nbytes = (n * bits + 7) // 8
    out = np.zeros(nbytes, np.uint8)
    for b in range(bits):
        pos = np.arange(n) * bits + b
        bit = ((codes >> b) & 1).astype(np.uint8)
        np.add.at(out, pos >> 3, (bit << (pos & 7)).astype(np.uint8))
    return out


def unpack(packed, bits, n):
    packed = np.asarray(packed, np.uint8)
    pos = np.arange(n)[:, None] * bits + np.arange(bits)[None, :]
    bit = (packed[pos >> 3] >> (pos & 7)) & 1
    return (bit.astype(np.int64) << np.arange(bits)).sum(axis=1)


def decode(codes, sp):
    codes = np.asarray(codes, np.int64)
    sign = (codes >> (sp.bits - 1)) & 1
    e = (codes >> sp.mant_bits) & ((1 << sp.exp_bits) - 1)
    m = codes & ((1 << sp.mant_bits) - 1)
    val = np.where(e == 0, m / (1 << sp.mant_bits) * 2.0 ** (1 - sp.bias),
                   (1.0 + m / (1 << sp.mant_bits)) * 2.0 ** (e - sp.bias))
    return np.where(sign == 1, -val, val)


def scale_exponent(peak, sp):
    """ceil(log2(peak) - log2(max_element)) evaluated as the reference does
    (mx_formats.py:141, :195-196): log2 in the precision of `peak` (float32
    for block peaks, whose log2 numpy rounds to float32 - which moves exact
    ties peak = max_element * 2^k up by one where that rounding goes up),
    minus a float64 log2(max_element)."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.ceil(np.log2(peak) - np.log2(np.float64(max_element(sp))))


def quantize(x, fmt, block_size=None):
    """x float32 [rows, cols] -> (packed uint8, scales int8): blocked
    [rows, nblocks] (blocks of block_size along cols, zero-padded), or [1]
    per tensor.  Raises OverflowError where the reference does."""
    x = np.asarray(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    sp = SPECS[fmt]
    bs = block_size or sp.block_size
    rows, cols = x.shape
    if bs <= 0:
        peak = float(np.abs(x).max()) if x.size else 1.0
        peak = peak if peak > 0 else 1.0            # NaN > 0 is False
        s = scale_exponent(peak, sp)
        if not np.isfinite(s):
            raise OverflowError("cannot convert float infinity to integer")
        s = int(s)
        if not -128 <= s <= 127:
            raise OverflowError(f"Python integer {s} out of bounds for int8")
        # float32 / (Python float) stays float32 (mx_formats.py:171): the
        # division rounds once in float32
        scaled = (x.ravel() / np.float32(2.0 ** s)).astype(np.float64)
        codes = encode(scaled, sp)
        return pack(codes, sp.bits), np.array([s], np.int8)
    pad = (-cols) % bs
    xp = np.concatenate([x, np.zeros((rows, pad), np.float32)], axis=1) if pad else x
    nb = xp.shape[1] // bs
    blk32 = xp.reshape(rows, nb, bs)
    blk = blk32.astype(np.float64)
    peak = np.abs(blk32).max(axis=-1)               # float32; NaN propagates, as np.max does
    peak = np.where(peak <= 0, np.float32(1.0), peak)
    s = scale_exponent(peak, sp)
    bad = ~np.isfinite(s)
    s_int = np.where(bad, np.iinfo(np.int64).min, np.where(bad, 0, s)).astype(np.int64)
    with np.errstate(divide="ignore", invalid="ignore"):
        div = np.where(bad, 0.0, 2.0 ** np.where(bad, 0, s_int).astype(np.float64))
        scaled = blk / div[..., None]
    codes = encode(scaled.ravel(), sp)
    return pack(codes, sp.bits), s_int.astype(np.int8)   # int8 cast wraps, as astype does


def dequantize(packed, scales, shape, fmt, block_size=None):
    """float64 [rows, cols], as the reference's dequantize_mx returns."""
    sp = SPECS[fmt]
    bs = block_size or sp.block_size
    rows, cols = (1, shape[0]) if len(shape) == 1 else shape
    if bs <= 0:
        codes = unpack(packed, sp.bits, rows * cols)
        s = float(np.asarray(scales, np.float32).reshape(-1)[0])
        return (decode(codes, sp) * 2.0 ** s).reshape(rows, cols)
    nb = (cols + bs - 1) // bs
    codes = unpack(packed, sp.bits, rows * nb * bs)
    vals = decode(codes, sp).reshape(rows, nb, bs)
    s = np.asarray(scales, np.float32).reshape(rows, nb).astype(np.float64)
    return (vals * 2.0 ** s[..., None]).reshape(rows, nb * bs)[:, :cols]


# ------------------------------------------------------------------------
# Matrix-core form of the reference's codes (build-defined, no reference
# counterpart).  The gfx950 scaled MFMA decodes FP8 operands as the OCP
# formats, in which the all-ones exponent field is not finite; the
# reference's MXFP8 decode (mx_formats.py:75-96) makes it finite.  FP6 / FP4
# agree with OCP everywhere.

def ocp_decode(codes, fmt):
    """Value of each code as the OCP format the matrix cores use: E4M3FN
    (0x7F / 0xFF NaN, every other code as the reference decodes it), E5M2
    (exponent field 31: +-inf for mantissa 0, else NaN); FP6 / FP4 as the
    reference.  Independent of the reference decoder above: the OCP MX spec's
    formats written out directly."""
    sp = SPECS[fmt]
    c = np.asarray(codes, np.int64)
    sign = np.where((c >> (sp.bits - 1)) & 1, -1.0, 1.0)
    e = (c >> sp.mant_bits) & ((1 << sp.exp_bits) - 1)
    m = c & ((1 << sp.mant_bits) - 1)
    sub = m * 2.0 ** (1 - sp.bias - sp.mant_bits)
    norm = (2 ** sp.mant_bits + m) * 2.0 ** (e.astype(np.float64) - sp.bias - sp.mant_bits)
    val = sign * np.where(e == 0, sub, norm)
    top = (1 << sp.exp_bits) - 1
    if fmt == "mxfp8_e4m3":
        val = np.where((e == top) & (m == (1 << sp.mant_bits) - 1), np.nan, val)
    elif fmt == "mxfp8_e5m2":
        val = np.where(e == top, np.where(m == 0, sign * np.inf, np.nan), val)
    return val


def to_mfma(packed, scales, rows, cols, fmt):
    """Codes and exponents of a block-32 tensor that the matrix cores decode
    to the reference's values: an FP8 block holding an all-ones-exponent code
    is written one binade lower (every value / 2) with exponent s + 1, unless
    s is already 127; a value of an odd number of smallest-subnormal units at
    the new exponent rounds half to even.  Returns (packed, scales, rounded)."""
    sp = SPECS[fmt]
    scales = np.asarray(scales, np.int8).reshape(rows, cols // 32).copy()
    if sp.bits != 8:
        return np.asarray(packed, np.uint8).copy(), scales, 0
    codes = np.asarray(packed, np.uint8).reshape(rows, cols // 32, 32).astype(np.int64)
    mb = sp.mant_bits
    e = (codes & 0x7F) >> mb
    ref_only = e == (1 << sp.exp_bits) - 1
    if fmt == "mxfp8_e4m3":
        ref_only &= (codes & ((1 << mb) - 1)) == (1 << mb) - 1
    fix = ref_only.any(axis=-1) & (scales.astype(np.int64) < 127)
    sign, mag = codes & 0x80, codes & 0x7F
    m = mag & ((1 << mb) - 1)
    k = np.where(e == 0, m, (1 << mb) + m)            # value in smallest-subnormal units (fields 0, 1)
    h = k >> 1
    h = h + ((k & 1) & (h & 1))                       # half to even
    halved = np.where(e >= 2, mag - (1 << mb), h) | sign
    out = np.where(fix[..., None], halved, codes).astype(np.uint8)
    rounded = int(((e < 2) & (k & 1).astype(bool) & fix[..., None]).sum())
    scales = np.where(fix, scales.astype(np.int64) + 1, scales).astype(np.int8)
    return out.reshape(-1), scales, rounded
