"""Write tests/golden/ref_quant.npz from the reference compiled unchanged.

Run in the build container only (it needs /root/reference):

    make -C oracle ref && python tests/golden/gen_golden.py

Every expected output in the fixture comes from oracle/_ref/libsnxref.so,
i.e. the reference's kernel/quantization/{quantize_int8,quantize_fp8,awq,
gptq}.c built with -O2 -ffp-contract=off.  Inputs are stored verbatim (small
cases) or as a numpy seed plus the SHA-256 of the generated array (the
256x4096 C1-shaped case), so the fixture stays a few hundred KB.

Keys are "<case>__<field>"; tests/test_oracle_golden.py and the GPU parity
tests read them back.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
from py_oracle import Reference  # noqa: E402

OUT = os.path.join(HERE, "ref_quant.npz")
SPECIALS = np.array([np.nan, np.inf, -np.inf, -0.0, 1e-40, -1e-40, 3e38, -3e38,
                     0.5, 2.5, -2.5, 1e-45, 1.17549435e-38], np.float32)


def with_specials(rng, n):
    x = rng.normal(0, 1, n).astype(np.float32)
    idx = rng.choice(n, len(SPECIALS), replace=False)
    x[idx] = SPECIALS
    return x


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_weights(seed: int, rows: int, cols: int) -> np.ndarray:
    return np.random.default_rng(seed).normal(0.0, 0.02, (rows, cols)).astype(np.float32)


def fp8_encode_sample() -> np.ndarray:
    """Stratified fp32 bit patterns: every exponent, both signs, edge and
    random mantissas (the full 2^32 sweep runs in tests against the oracle)."""
    rng = np.random.default_rng(7)
    mant = np.concatenate([np.array([0, 1, 0x7FFFFF, 0x080000, 0x0FFFFF, 0x100000,
                                     0x1FFFFF, 0x200000, 0x3FFFFF, 0x400000, 0x7FFFFE],
                                    np.uint32), rng.integers(0, 1 << 23, 21, dtype=np.uint32)])
    e = np.arange(256, dtype=np.uint32)
    bits = (e[:, None] << 23 | mant[None, :]).ravel()
    bits = np.concatenate([bits, bits | np.uint32(0x80000000)])
    return bits.view(np.float32)


def main() -> None:
    ref = Reference()
    rng = np.random.default_rng(2024)
    fx: dict[str, np.ndarray] = {}

    def put(case, **kw):
        for k, v in kw.items():
            fx[f"{case}__{k}"] = np.asarray(v)

    # --- int8 / int4 vector codecs (quantize_int8.c) -------------------------
    vec_inputs = [
        np.array([127, .5, 2.5, -2.5], np.float32),                 # ties away from zero
        np.array([-1.0, 0.0, 1.0, 2.5], np.float32),                # test_quantize.c:30
        np.array([0.5, 1.5, 2.0, 0.0, -1.0], np.float32),           # test_quantize.c:63
        np.array([1.0, -1.0, 3.5, -3.0, 0.5, -0.5], np.float32),    # test_quantize.c:95
        np.array([7, -7, 3.5, -3.5, 1, 0], np.float32),             # int4 KAT
        np.zeros(4, np.float32), np.full(5, 0.25, np.float32),
        np.array([1e-39, -1e-39, 0.0], np.float32), np.array([3.0], np.float32),
        rng.normal(0, 1, 1001).astype(np.float32),
        rng.normal(0, 0.02, 4096).astype(np.float32),
        with_specials(rng, 257), with_specials(rng, 64),
        (rng.integers(-400, 400, 777) / 4).astype(np.float32),
        np.array([np.nan, 1.0, -2.0, 0.5], np.float32),
    ]
    for i, x in enumerate(vec_inputs):
        rc, q, s = ref.quantize_int8_sym(x)
        put(f"int8_sym_{i}", x=x, rc=rc, q=q, s=s)
        rc, q, s, z = ref.quantize_int8_asym(x)
        put(f"int8_asym_{i}", x=x, rc=rc, q=q, s=s, z=z)
        rc, p, s = ref.quantize_int4_sym(x)
        put(f"int4_sym_{i}", x=x, rc=rc, p=p, s=s)
    codes = np.arange(-128, 128, dtype=np.int8)
    for i, (s, z) in enumerate([(0.0157480314, 0), (1.0, 0), (0.0117647059, 85), (3.5e-3, 255),
                                (-0.5, 7), (np.float32(np.inf), 1), (1e-38, 128)]):
        _, y = ref.dequantize_int8_sym(codes, np.float32(s))
        _, ya = ref.dequantize_int8_asym(codes, np.float32(s), z)
        _, y4 = ref.dequantize_int4_sym(codes.view(np.uint8), 512, np.float32(s))
        put(f"deq_{i}", codes=codes, s=np.float32(s), z=z, y_sym=y, y_asym=ya, y_int4=y4)

    # --- per-channel int8 (quantize_int8.c:157-177) ---------------------------
    ch = [rng.normal(0, 0.02, (64, 257)).astype(np.float32),
          with_specials(rng, 8 * 33).reshape(8, 33),
          np.zeros((3, 5), np.float32)]
    ch[0][5] = 0.0
    ch[0][9, 3] = 0.5 * (np.abs(ch[0][9]).max() / 127) * 3    # a tie candidate
    for i, x in enumerate(ch):
        rc, q, s = ref.quantize_int8_channel(x)
        put(f"int8_channel_{i}", x=x, rc=rc, q=q, s=s)
    # C1-shaped slice: 256 rows of the 4096-wide N(0, 0.02) matrix, by seed
    w = c1_weights(11, 256, 4096)
    rc, q, s = ref.quantize_int8_channel(w)
    put("int8_channel_c1", seed=11, rows=256, cols=4096, sha=sha(w), rc=rc, q=q, s=s)

    # --- FP8 codecs (quantize_fp8.c) ------------------------------------------
    allc = np.arange(256, dtype=np.uint8)
    xs = fp8_encode_sample()
    for fmt in ("e4m3", "e5m2"):
        _, dec = ref.dequantize_fp8(allc, fmt)
        _, enc = ref.quantize_fp8(xs, fmt)
        put(f"fp8_{fmt}", codes=allc, dec_bits=dec.view(np.uint32), x=xs, enc=enc)
    kat = np.array([0, 1, -1, 2.5, 127, -64, 0.125, 240, 255, 256, 300, 448, 600,
                    0.015625, 0.0156, -0.0, 1.25, 1.5, 1.75, 3.0, 0.25, -128], np.float32)
    put("fp8_kat", x=kat, e4m3=ref.quantize_fp8(kat, "e4m3")[1], e5m2=ref.quantize_fp8(kat, "e5m2")[1])

    # --- AWQ (awq.c) ----------------------------------------------------------
    awq_in = [(np.array([[1, 2, 3, 4], [-1, -2, -3, -4]], np.float32), 2),   # test_quantize.c:134-138
              (rng.normal(0, 0.02, (8, 300)).astype(np.float32), 128),
              (rng.normal(0, 0.02, (4, 256)).astype(np.float32), 0),
              (rng.normal(0, 1, (5, 100)).astype(np.float32), 7),
              (with_specials(rng, 4 * 64).reshape(4, 64), 16)]
    for i, (x, g) in enumerate(awq_in):
        rc, q, s = ref.awq_quantize(x, g)
        put(f"awq_{i}", x=x, g=g, rc=rc, q=q, s=s)
    sw_in = [(rng.normal(0, 0.02, (2, 256)).astype(np.float32),
              rng.uniform(0.05, 1.5, 256).astype(np.float32)),
             (rng.normal(0, 1, (3, 130)).astype(np.float32),
              np.concatenate([np.array([np.nan, -1.0, 0.999, 1.0, 0.0], np.float32),
                              rng.uniform(-0.2, 1.2, 125).astype(np.float32)]))]
    for i, (x, a) in enumerate(sw_in):
        rc, wo, so = ref.awq_scale_weights(x, a)
        put(f"awq_sw_{i}", x=x, act=a, rc=rc, w=wo, s=so)

    # --- GPTQ (gptq.c) --------------------------------------------------------
    acts = np.array([1, 0, 2, 0, 3, 0, 4, 0, 5, 0, 6, 0], np.float32).reshape(4, 3)  # test_quantize.c:146-148
    for i, a in enumerate([acts, rng.normal(0, 1, (20, 17)).astype(np.float32)]):
        rc, h = ref.gptq_compute_hessian(a)
        put(f"hessian_{i}", act=a, rc=rc, h=h)
    for i, (n, bits, sym) in enumerate([(6, 4, 1), (40, 4, 0), (33, 8, 1), (17, 3, 1)]):
        wb = rng.normal(0, 1, n).astype(np.float32)
        hb = rng.normal(0, 0.3, (n, n)).astype(np.float32) + np.eye(n, dtype=np.float32)
        if i == 0:
            wb = np.array([.7, -.1, .35, .2, -.6, .05], np.float32)
        rc, wo, qw, s, z = ref.gptq_quantize_block(wb, hb, bits, sym)
        put(f"gptq_block_{i}", w_in=wb, h=hb, bits=bits, sym=sym, rc=rc, w=wo, qw=qw, s=s, z=z)
    gq_in = [rng.normal(0, 0.02, (6, 300)).astype(np.float32),
             with_specials(rng, 3 * 300).reshape(3, 300),
             np.array([[.7, -.1, .35, .2, -.6, .05]], np.float32)]
    cfgs = [(128, 4, 1), (128, 4, 0), (0, 8, 1), (64, 3, 1), (3, 4, 1), (128, 16, 1), (128, 1, 1)]
    for i, x in enumerate(gq_in):
        for j, (g, bits, sym) in enumerate(cfgs):
            rc, _, q, s, z = ref.gptq_quantize(x, g, bits, sym)
            put(f"gptq_{i}_{j}", x=x, g=g, bits=bits, sym=sym, rc=rc, q=q, s=s, z=z)

    # --- a21 reduction: GPTQ act-order == gptq_quantize on permuted columns ----
    N, K, gsz = 16, 512, 128
    wa = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    g_idx = (rng.permutation(K) // gsz).astype(np.int32)
    perm = np.argsort(g_idx, kind="stable").astype(np.int32)
    rc, _, q, s, z = ref.gptq_quantize(np.ascontiguousarray(wa[:, perm]), gsz, 4, 1)
    put("actorder", w=wa, g_idx=g_idx, perm=perm, rc=rc, q_perm=q, s=s)

    # --- metadata (awq.c:171-223) ----------------------------------------------
    modes = np.arange(-1, 10, dtype=np.int32)
    params = np.array([ref.quant_params_create(int(m))[1] for m in modes], np.float64)
    names = np.array([ref.quant_mode_name(int(m)) for m in modes])
    put("meta", modes=modes, params=params, names=names)

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {len(fx)} arrays, {os.path.getsize(OUT) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
