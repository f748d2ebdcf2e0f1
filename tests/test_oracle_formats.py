"""Pins for the oracle's build-defined formats (W4 AWQ-style, GPTQ act-order,
W8/W4A16 linears, W8A8 int8/fp8) and its fp16/bf16 conversions.  CPU only.

None of these re-types the oracle's formula: each checks an independent
property (a library conversion, brute-force optimality, a reduction to the
reference's own gptq_quantize output, exact integer arithmetic, float64
products)."""
import numpy as np
import pytest
import torch

from helpers import cases


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_to_f32(h):
    return (np.asarray(h, np.uint32) << 16).view(np.float32)


def test_f16_and_bf16_conversions_match_libraries(oracle):
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.normal(0, 1, 2000), rng.normal(0, 1e-6, 500), rng.normal(0, 3e4, 500),
        [0.0, -0.0, 65504, 65519.99, 65520, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
         2.0 ** -14, 2.0 ** -14 * 0.99, 3e-8, np.inf, -np.inf],
        (np.arange(1, 4000) * 2.0 ** -24) * 1.5,
    ]).astype(np.float32)
    want16 = vals.astype(np.float16).view(np.uint16)
    got16 = np.array([oracle.f32_to_f16(v) for v in vals], np.uint16)
    assert np.array_equal(got16, want16)
    back = np.array([oracle.f16_to_f32(h) for h in want16], np.float32)
    assert np.array_equal(back.view(np.uint32), want16.view(np.float16).astype(np.float32).view(np.uint32))
    got_b = np.array([oracle.f32_to_bf16(v) for v in vals], np.uint16)
    assert np.array_equal(got_b, bf16_bits(vals))
    # W4 scale clamps
    assert oracle.raw["w4_scale_to_f16"](0.0) == 0x0001
    assert oracle.raw["w4_scale_to_f16"](1e-30) == 0x0001
    assert oracle.raw["w4_scale_to_f16"](1e6) == 0x7BFF


def test_w4_nibble_order_is_the_reference_int4_byte_order(oracle):
    # The reference packs element 2i low / 2i+1 high (quantize_int8.c:206-216);
    # read as little-endian u32, element j sits at bits 4j.  The W4 format uses
    # exactly that order, so dequantising reference int4 bytes with scale 1 and
    # zero 0 must give back the reference's unsigned nibbles.
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, 64).astype(np.float32)
    rc, packed, s = oracle.quantize_int4_sym(x)
    words = packed.view(np.uint32).reshape(1, 8)
    scales = np.full((1, 1), 0x3C00, np.uint16)        # 1.0
    zeros = np.zeros((1, 1), np.uint32)
    rc, deq = oracle.w4_dequantize(words, scales, zeros, None, 1, 64, 64)
    nib = np.stack([packed & 0xF, packed >> 4], 1).ravel().astype(np.float32)
    assert rc == 0 and np.array_equal(deq.ravel(), nib)


@pytest.mark.parametrize("seed", [0, 1])
def test_w4_awq_codes_are_nearest_levels(oracle, seed):
    rng = np.random.default_rng(seed)
    N, K, g = 24, 512, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w[3, :128] = 0.125                                  # constant group -> degenerate path
    w[4, 128:256] = np.abs(w[4, 128:256]) + 0.01        # all-positive group -> zero clamps to 0
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, g)
    assert rc == 0
    nib = ((qw[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K).astype(np.int64)
    z = ((qz[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, -1)[:, :K // g].astype(np.int64)
    s = sc.view(np.float16).astype(np.float32)
    for n in range(N):
        for j in range(K // g):
            wg = w[n, j * g:(j + 1) * g].astype(np.float64)
            q = nib[n, j * g:(j + 1) * g]
            if n == 3 and j == 0:
                assert sc[n, j] == 0x3C00 and z[n, j] == 0 and not q.any()
                continue
            lo, hi = wg.min(), wg.max()
            assert s[n, j] == np.float32(np.float16((np.float32(hi) - np.float32(lo)) / np.float32(15)))
            levels = (np.arange(16)[None, :] - z[n, j]) * float(s[n, j])
            err = np.abs(levels - wg[:, None])
            chosen = err[np.arange(g), q]
            assert np.all(chosen <= err.min(1) + 1e-6 * float(s[n, j])), (n, j)
            if 0 < z[n, j] < 15:
                assert np.all(chosen <= 0.5 * float(s[n, j]) * (1 + 1e-5) + 1e-12)


def test_actorder_reduces_to_reference_gptq(oracle, golden):
    # a21: codes of the act-order format == the reference's gptq_quantize
    # (bits 4, sym, g 128) run on W[:, stable_argsort(g_idx)]; scales are the
    # reference's fp32 scales rounded to fp16.
    f = cases(golden, "actorder")["actorder"]
    w, g_idx, perm = f["w"], f["g_idx"], f["perm"]
    N, K = w.shape
    G = int(g_idx.max()) + 1
    rc, qw, sc = oracle.w4_gptq_quantize(w, g_idx, G)
    assert rc == 0
    nib = ((qw[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(N, K).astype(np.int32)
    assert np.array_equal(nib[:, perm] - 8, f["q_perm"].astype(np.int32))
    want_sc = f["s"].astype(np.float16).view(np.uint16)
    assert np.array_equal(sc, want_sc)


def test_linears_against_float64(oracle):
    rng = np.random.default_rng(5)
    M, N, K, g = 3, 40, 256, 128
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    xb = bf16_bits(x)
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, g)
    rc, deq = oracle.w4_dequantize(qw, sc, qz, None, N, K, g)
    rc, y = oracle.w4a16_linear(xb, qw, sc, qz, None, N, K, g)
    want = bf16_to_f32(xb).astype(np.float64) @ deq.astype(np.float64).T
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    # W8 weight-only
    rc, q, s = oracle.quantize_int8_channel(w)
    rc, y8 = oracle.w8_linear(x, q, s)
    want8 = x.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T
    assert np.abs(y8 - want8).max() <= 1e-5 * np.abs(want8).max()
    # int8 GEMM accumulators are exact
    A = rng.integers(-128, 128, (7, 300)).astype(np.int8)
    B = rng.integers(-128, 128, (9, 300)).astype(np.int8)
    assert np.array_equal(oracle.i8_gemm_i32(A, B), A.astype(np.int64) @ B.astype(np.int64).T)
    # fp8 GEMM on decoded operands
    a = rng.normal(0, 1, (5, 64)).astype(np.float32)
    b = rng.normal(0, 0.02, (6, 64)).astype(np.float32)
    _, ca, sa = oracle.quantize_fp8_e4m3_scaled(a)
    _, cb, sb = oracle.quantize_fp8_e4m3_scaled(b)
    assert sa == np.float32(np.abs(a).max()) / np.float32(240)
    out = oracle.fp8_gemm(ca, cb, sa, sb)
    _, da = oracle.dequantize_fp8(ca.ravel(), "e4m3")
    _, db = oracle.dequantize_fp8(cb.ravel(), "e4m3")
    want = (da.reshape(5, 64).astype(np.float64) @ db.reshape(6, 64).astype(np.float64).T) * float(sa) * float(sb)
    assert np.abs(out - want).max() <= 1e-5 * np.abs(want).max()
    # codes stay below the reference's field-15 (inf/nan) range when |x/s| <= 240
    assert ((ca & 0x78) != 0x78).all() and ((cb & 0x78) != 0x78).all()


def test_half_even_option_matches_numpy_rint_and_differs_only_at_ties(oracle):
    """The build's SNEPPX_ROUND_HALF_EVEN option (C1 config text) against
    numpy's rint on the same fp32 products; the reference's roundf path
    differs from it exactly at the odd .5 ties."""
    rng = np.random.default_rng(17)
    w = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    # plant exact ties: scale is max/127, so max=127 makes x*inv = x
    w[:8, 0] = 127.0
    w[:8, 1:9] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32)
    rc, q_even, s_even = oracle.quantize_int8_channel_rne(w)
    rc2, q_away, s_away = oracle.quantize_int8_channel(w)
    assert rc == 0 and rc2 == 0
    assert np.array_equal(s_even.view(np.uint32), s_away.view(np.uint32))
    inv = (np.float32(1.0) / s_even).astype(np.float32)
    prod = (w * inv[:, None]).astype(np.float32)
    want = np.clip(np.rint(prod), -128, 127).astype(np.int8)
    assert np.array_equal(q_even, want)
    assert list(q_even[0, 1:9]) == [0, 2, 2, 0, -2, -2, 126, -126]
    assert list(q_away[0, 1:9]) == [1, 2, 3, -1, -2, -3, 127, -127]
    ties = (np.abs(prod - np.trunc(prod)) == 0.5)
    diff = q_even != q_away
    assert diff.sum() > 0 and np.all(ties[diff])


def _nibbles(qw, K):
    q = np.asarray(qw, np.uint32)
    return ((q[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(q.shape[0], K).astype(np.int64)


def _roundf(v):
    """C roundf (ties away from zero) on float32 values, exact in float64."""
    v = np.asarray(v, np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_w4_awq_ties_and_divide_first(oracle):
    """The W4 code rule is quantize_int8.c:114-120 with 255 -> 15:
    roundf(w / s + z) - a division, then an fp32 add, then ties away from
    zero.  Planted exact ties (w / s + z = k + 0.5 exactly) must give k + 1
    (rint would give the even neighbour), and values where w * (1/s) and w / s
    round to different codes must take the division's code."""
    s = np.float32(3.0 / 1024.0)                      # exact in fp16 and fp32
    g = 128
    row = np.zeros(g, np.float32)
    row[0], row[1] = -5 * s, 10 * s                   # lo, hi: (hi - lo)/15 = s, z = 5
    ks = np.arange(15)
    row[2:17] = (ks + 0.5 - 5) * s                    # w/s + z = k + 0.5 exactly
    # values where multiply-by-reciprocal and divide disagree on the code
    inv = np.float32(1.0) / s
    found = []
    base = ((np.arange(-4, 10) + 0.5) * s).astype(np.float32)
    for b in base:
        for d in range(-64, 65):
            w = np.nextafter(b, np.float32(np.inf if d > 0 else -np.inf)) if d else b
            for _ in range(abs(d) - 1):
                w = np.nextafter(w, np.float32(np.inf if d > 0 else -np.inf))
            q_div = _roundf(np.float32(np.float32(w / s) + np.float32(5)))
            q_mul = _roundf(np.float32(np.float32(w * inv) + np.float32(5)))
            if q_div != q_mul and -5 * s < w < 10 * s:
                found.append((np.float32(w), int(q_div), int(q_mul)))
    assert found, "no multiply/divide disagreement near the ties"
    found = found[: g - 17]
    row[17:17 + len(found)] = [f[0] for f in found]
    w = np.tile(row, (2, 1))
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, g)
    assert rc == 0
    assert sc[0, 0] == np.float16(s).view(np.uint16) and (qz[0, 0] & 0xF) == 5
    nib = _nibbles(qw, g)[0]
    assert nib[0] == 0 and nib[1] == 15
    assert list(nib[2:17]) == list(ks + 1)            # ties away from zero
    got = nib[17:17 + len(found)]
    assert list(got) == [f[1] for f in found]         # the division's codes
    assert all(g_ != f[2] for g_, f in zip(got, found))


def test_w8a8_epilogue_against_float64(oracle):
    """out[m][n] = acc * sA[m] * sW[n]: per-token scales index rows and
    per-channel scales index columns (M != N, distinct scales, so a swapped
    or transposed index fails); fp32 rounding only."""
    rng = np.random.default_rng(8)
    M, N = 7, 11
    acc = rng.integers(-2 ** 26, 2 ** 26, (M, N)).astype(np.int32)
    sA = rng.uniform(1e-3, 2e-2, M).astype(np.float32)
    sW = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    out = oracle.w8a8_epilogue(acc, sA, sW)
    want = acc.astype(np.float64) * sA[:, None].astype(np.float64) * sW[None, :].astype(np.float64)
    assert np.all(np.abs(out - want) <= 2.5 * 2.0 ** -24 * np.abs(want))
    bias = rng.normal(0, 1, N).astype(np.float32)
    outb = oracle.w8a8_epilogue(acc, sA, sW, bias)
    wantb = want + bias.astype(np.float64)
    assert np.all(np.abs(outb - wantb) <= 2.0 ** -22 * (np.abs(want) + np.abs(wantb)))
    # the full W8A8 reference on dequantised operands (float64) is what the
    # epilogue of the exact int32 product equals
    A = rng.integers(-127, 128, (M, 96)).astype(np.int8)
    W = rng.integers(-127, 128, (N, 96)).astype(np.int8)
    out2 = oracle.w8a8_epilogue(oracle.i8_gemm_i32(A, W), sA, sW)
    deq = (A.astype(np.float64) * sA[:, None]) @ (W.astype(np.float64) * sW[:, None]).T
    assert np.all(np.abs(out2 - deq) <= 2.5 * 2.0 ** -24 * np.abs(deq) + 1e-30)


def test_matmul_order_and_layout(oracle):
    """tensor.c:1820-1823: k-ascending fp32 sum from 0.0f.  [1, 1e8, -1e8]
    summed in that order is 0 (1 is absorbed by 1e8); reversed it is 1.  The
    [K,N] and [N,K] forms are transposes of one another and equal float64
    within fp32 rounding."""
    a = np.array([[1.0, 1e8, -1e8]], np.float32)
    ones = np.ones((3, 1), np.float32)
    assert oracle.matmul_kn(a, ones)[0, 0] == 0.0
    assert oracle.matmul_nk(a, ones.T)[0, 0] == 0.0
    assert oracle.matmul_kn(a[:, ::-1].copy(), ones)[0, 0] == 1.0
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (5, 64)).astype(np.float32)
    b = rng.normal(0, 1, (64, 7)).astype(np.float32)
    ykn = oracle.matmul_kn(x, b)
    ynk = oracle.matmul_nk(x, np.ascontiguousarray(b.T))
    assert np.array_equal(ykn.view(np.uint32), ynk.view(np.uint32))
    want = x.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(ykn - want).max() <= 1e-5 * np.abs(want).max()


def test_bias_step(oracle):
    """quantization.py:451-454: y = x @ W^T + bias.  Zero weights give the
    bias exactly; otherwise float64 within fp32 rounding."""
    rng = np.random.default_rng(10)
    M, N, K, g = 3, 24, 256, 128
    bias = rng.normal(0, 1, N).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    q0 = np.zeros((N, K), np.int8)
    rc, y0 = oracle.w8_linear(x, q0, np.ones(N, np.float32), bias)
    assert rc == 0 and np.array_equal(y0, np.tile(bias, (M, 1)))
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    rc, qw, sc, qz = oracle.w4_awq_quantize(w, g)
    xb = bf16_bits(x)
    rc, deq = oracle.w4_dequantize(qw, sc, qz, None, N, K, g)
    rc, y = oracle.w4a16_linear(xb, qw, sc, qz, None, N, K, g, bias)
    want = bf16_to_f32(xb).astype(np.float64) @ deq.astype(np.float64).T + bias
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    rc, ynb = oracle.w4a16_linear(xb, qw, sc, qz, None, N, K, g)
    assert np.array_equal(y, (ynb + bias[None, :]).astype(np.float32))


def _planted_fp8_amax(rng, want_div_at_240):
    """amax values whose per-tensor fp8 codes differ between x / s and
    x * (1/s) with s = amax / 240: with want_div_at_240 the quotient is 240
    (code 0x77) and the product 239.99998 (0x76), else the other way."""
    am = rng.uniform(0.5, 8.0, 4000).astype(np.float32)
    s = (am / np.float32(240)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    vd = (am / s).astype(np.float32)
    vm = (am * inv).astype(np.float32)
    sel = (vd >= 240) & (vm < 240) if want_div_at_240 else (vd < 240) & (vm >= 240)
    return am[sel]


def test_fp8_per_tensor_rule_is_division(oracle):
    """The per-tensor fp8 quantizer encodes x / s (one correctly rounded
    division), not x * (1/s).  Each planted tensor's largest element lands
    at 240 under one rule and 239.99998 under the other, which the
    reference's truncating encoder sends to 0x77 and 0x76; the oracle must
    give the division's code for every element, in both directions.  The
    expected codes use the reference array encoder (quantize_fp8.c:111-121,
    pinned exhaustively against the reference build) on numpy's fp32
    quotient."""
    rng = np.random.default_rng(21)
    for want_div_at_240 in (True, False):
        amaxes = _planted_fp8_amax(rng, want_div_at_240)[:24]
        assert len(amaxes) >= 8
        for i, am in enumerate(amaxes):
            x = rng.normal(0, float(am) / 4, 257).astype(np.float32)
            x = np.clip(x, -am, am)
            x[i % 257] = am if i % 2 == 0 else -am
            rc, c, s = oracle.quantize_fp8_e4m3_scaled(x)
            assert rc == 0 and s == (np.float32(am) / np.float32(240)).astype(np.float32)
            _, want = oracle.quantize_fp8((x / s).astype(np.float32))
            _, mul = oracle.quantize_fp8((x * (np.float32(1) / s)).astype(np.float32))
            assert np.array_equal(c, want), (am, np.flatnonzero(c != want))
            top = c[i % 257] & 0x7F
            assert top == (0x77 if want_div_at_240 else 0x76)
            assert (mul[i % 257] & 0x7F) == (0x76 if want_div_at_240 else 0x77)
            assert not np.array_equal(c, mul)
    # degenerate tensor: scale 1, raw codes
    rc, c, s = oracle.quantize_fp8_e4m3_scaled(np.zeros(5, np.float32))
    assert rc == 0 and s == 1.0 and not c.any()


def test_actorder_dequant_gathers_by_g_idx(oracle, golden):
    """orc_w4_dequantize with g_idx reads scale[n][g_idx[k]] for column k.
    Closed form against the reference's own GPTQ output: after the stable
    argsort perm of g_idx, column perm[i] holds the reference code
    q_perm[n][i] of group i // 128, so its dequantised value is exactly
    q_perm * fp16(s) (a product of a 4-bit integer and an fp16 value is
    exact in fp32).  A k // 128 gather (the no-g_idx path) fails it."""
    f = cases(golden, "actorder")["actorder"]
    w, g_idx, perm, q_perm, s = f["w"], f["g_idx"], f["perm"], f["q_perm"], f["s"]
    N, K = w.shape
    G = int(g_idx.max()) + 1
    gs = K // G
    rc, qw, sc = oracle.w4_gptq_quantize(w, g_idx, G)
    assert rc == 0
    rc, deq = oracle.w4_dequantize(qw, sc, None, g_idx, N, K, gs)
    assert rc == 0
    s16 = s.astype(np.float16).astype(np.float32)
    want = np.zeros((N, K), np.float32)
    grp_sorted = np.arange(K) // gs
    want[:, perm] = q_perm.astype(np.float32) * s16[:, grp_sorted]
    assert np.array_equal(deq, want)
    # the planted mistake: gather by k // group instead of g_idx[k]
    rc, wrong = oracle.w4_dequantize(qw, sc, None, None, N, K, gs)
    assert rc == 0 and not np.array_equal(wrong, want)


def test_actorder_dequant_error_bound_with_spread_groups(oracle):
    """Invariant: after the act-order quantize, every element satisfies
    |deq - w| <= s/2 + 7 |fp16(s) - s| with its own group's fp32 scale
    s = max|w_group| / 7 (codes come from the fp32 scale, dequantisation
    uses the stored fp16 one).  Groups get magnitudes 2^j apart, so reading
    a neighbour's scale (a k // 128 gather) breaks the bound."""
    rng = np.random.default_rng(22)
    N, K, gs = 6, 1024, 128
    G = K // gs
    perm = rng.permutation(K)
    g_idx = (perm // gs).astype(np.int32)               # each group: 128 scattered columns
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    w *= (2.0 ** g_idx.astype(np.float32))[None, :]
    rc, qw, sc = oracle.w4_gptq_quantize(w, g_idx, G)
    assert rc == 0
    gmax = np.zeros((N, G), np.float32)
    for j in range(G):
        gmax[:, j] = np.abs(w[:, g_idx == j]).max(1)
    s32 = (gmax / np.float32(7)).astype(np.float32)
    s16 = sc.view(np.float16).astype(np.float64)
    bound = 0.5 * s32.astype(np.float64) + 7 * np.abs(s16 - s32) + 1e-12
    rc, deq = oracle.w4_dequantize(qw, sc, None, g_idx, N, K, gs)
    assert rc == 0
    err = np.abs(deq.astype(np.float64) - w.astype(np.float64))
    assert np.all(err <= bound[:, g_idx] * (1 + 1e-6))
    rc, wrong = oracle.w4_dequantize(qw, sc, None, None, N, K, gs)
    err_w = np.abs(wrong.astype(np.float64) - w.astype(np.float64))
    assert (err_w > bound[:, g_idx] * (1 + 1e-6)).mean() > 0.5
