"""SNEPPX_qlinear_w4a16_mlp: a SwiGLU MLP block, y = down(silu(gate(x)) * up(x)).

For prefill row counts the gate/up GEMM's SwiGLU epilogue writes the down
GEMM's prepared input itself (slot order and 128-column step sums) instead of
plain rows that the down projection's activation pass would then reorder and
sum; the result must be bit-identical to the two calls it replaces
(SNEPPX_qlinear_w4a16_swiglu, then SNEPPX_qlinear_w4a16 on its output), and
other shapes run exactly those two calls.  One small case is also checked
against the oracle linears with the SwiGLU rule of
kernel/activations/gated_activations.c:33-52 in float64."""
import numpy as np
import pytest
import torch

from test_gpu_qlinear import DEV, TOL_BF16, _w4_case, bf16_bits, bf16_to_f32, rel_err, to_dev, u16

pytestmark = pytest.mark.gpu


def _dev_w4(lib, N, K, seed, sym=False):
    """AWQ-style W4 g128 weights quantized on the device (large shapes)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, K // 128), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (K // 128 + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
    return qw, sc, None if sym else qz


@pytest.mark.parametrize("M,H,F,N,sym,bias,out", [
    (1849, 4096, 14336, 4096, False, False, "bf16"),   # the C5 Llama-3-8B MLP at T = 1849
    (300, 256, 384, 512, False, True, "bf16"),        # ragged M, biases on both projections
    (256, 512, 256, 640, True, True, "f32"),          # one M tile, symmetric weights, fp32 out
    (600, 1024, 2048, 256, False, False, "bf16"),     # few down tiles: the down GEMM in K spans
    (257, 1024, 1024, 768, False, True, "f32"),       # one row past a tile
    (8, 512, 384, 256, False, True, "bf16"),          # decode rows: the two calls
    (1, 4096, 1792, 4096, False, False, "bf16"),      # one token, a TP=8 shard's MLP (ragged K of down)
    (1, 4096, 14336, 4096, False, True, "bf16"),      # one token, the C5 MLP, biases on both
    (1, 4096, 14336, 4096, True, False, "bf16"),      # the same without zero words
    (1, 8192, 2816, 1024, False, True, "bf16"),       # H = 8192, ragged F
    (1, 4096, 2048, 300, True, True, "bf16"),         # few down rows
    (1, 4096, 1792, 4096, False, True, "f32"),        # fp32 output
])
def test_mlp_equals_swiglu_then_down(lib, M, H, F, N, sym, bias, out):
    print(f"[gpu] w4a16 mlp M={M} H={H} F={F} N={N} sym={sym} bias={bias} out={out}", flush=True)
    gu = _dev_w4(lib, 2 * F, H, 11 + F, sym)
    dn = _dev_w4(lib, N, F, 12 + N, sym)
    g = torch.Generator(device=DEV).manual_seed(M + H)
    x = torch.randn((M, H), device=DEV, generator=g).to(torch.bfloat16)
    gb = torch.randn(2 * F, device=DEV, generator=g) * 0.5 if bias else None
    db = torch.randn(N, device=DEV, generator=g) * 0.5 if bias else None
    dt = torch.float32 if out == "f32" else torch.bfloat16
    y = torch.empty((M, N), dtype=dt, device=DEV)
    lib.qlinear_w4a16_mlp(x, gu, dn, y, 128, gu_bias=gb, dn_bias=db)
    act = torch.empty((M, F), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16_swiglu(x, *gu, act, 128, bias=gb)
    y2 = torch.empty((M, N), dtype=dt, device=DEV)
    lib.qlinear_w4a16(act, *dn, None, F // 128, y2, 128, bias=db)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    iv = torch.int32 if out == "f32" else torch.int16
    assert torch.equal(y.view(iv), y2.view(iv))
    # again with the workspaces warm: same bits
    for _ in range(3):
        y.zero_()
        lib.qlinear_w4a16_mlp(x, gu, dn, y, 128, gu_bias=gb, dn_bias=db)
        torch.cuda.synchronize()
        assert torch.equal(y.view(iv), y2.view(iv))


def test_mlp_against_oracle(lib, oracle):
    """The fused path on a small prefill shape against the oracle: gate/up
    linear in fp32, SwiGLU in float64 rounded to bf16 (the GPU's act), down
    linear on that act."""
    M, H, F, N = 300, 256, 384, 512
    print(f"[gpu] w4a16 mlp vs oracle M={M} H={H} F={F} N={N}", flush=True)
    rng = np.random.default_rng(5)
    gq, gs, gz, _ = _w4_case(oracle, 2 * F, H, 128, 21)
    dq, ds, dz, _ = _w4_case(oracle, N, F, 128, 22)
    x = bf16_bits(rng.normal(0, 1, (M, H)).astype(np.float32))
    gb = rng.normal(0, 0.5, 2 * F).astype(np.float32)
    db = rng.normal(0, 0.5, N).astype(np.float32)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    lib.qlinear_w4a16_mlp(to_dev(x), (to_dev(gq), to_dev(gs), to_dev(gz)), (to_dev(dq), to_dev(ds), to_dev(dz)),
                          y, 128, gu_bias=to_dev(gb), dn_bias=to_dev(db))
    torch.cuda.synchronize()
    rc, guo = oracle.w4a16_linear(x, gq, gs, gz, None, 2 * F, H, 128, bias=gb)
    g, u = guo[:, :F].astype(np.float64), guo[:, F:].astype(np.float64)
    act = bf16_bits((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
    rc, want = oracle.w4a16_linear(act, dq, ds, dz, None, N, F, 128, bias=db)
    assert rel_err(bf16_to_f32(u16(y)), want) <= TOL_BF16
