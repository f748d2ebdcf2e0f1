"""Decode linears captured into a HIP graph (snx_hip_stream_begin_capture /
end_capture / graph_launch): every replay gives the eager bits, with eager
work on the same stream and on the default stream between the replays.
Covers the M = 1 W4A16 GEMV (full and ragged K), its GLU (gate/up +
SwiGLU) form, the decode MLP call (gate/up + SwiGLU, then down), the
prepared act-order GEMV and the W8 GEMV, chained as a decode step chains them (one linear's output is the
next one's input)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _w4(lib, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, K // 128), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (K // 128 + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
    return qw, sc, qz


def test_decode_step_graph_replays_match_eager(lib):
    print("[gpu] graph: W4 GEMV, GLU, ragged-K GEMV, act-order, W8 GEMV, MLP call chained; 4 replays", flush=True)
    H, F, N2, NG, N8 = 4096, 1792, 3072, 2048, 1000
    s = torch.cuda.Stream()
    st = s.cuda_stream
    with torch.cuda.stream(s):
        w_a = _w4(lib, H, H, 1)                 # H -> H
        w_gu = _w4(lib, 2 * F, H, 2)            # H -> 2F, SwiGLU -> F
        w_b = _w4(lib, N2, F, 3)                # F (ragged K = 1792) -> N2
        # GPTQ act-order N2 -> NG, prepared once
        g_idx = torch.from_numpy((np.random.default_rng(4).permutation(N2) // 128).astype(np.int32)).to(DEV)
        G = N2 // 128
        wg = torch.randn((NG, N2), device=DEV, generator=torch.Generator(device=DEV).manual_seed(5)) * 0.02
        qw_g = torch.empty((NG, N2 // 8), dtype=torch.int32, device=DEV)
        sc_g = torch.empty((NG, G), dtype=torch.int16, device=DEV)
        lib.dev_quantize_w4_gptq(wg, g_idx, G, qw_g, sc_g)
        qs = torch.empty_like(qw_g)
        perm = torch.empty(N2, dtype=torch.int16, device=DEV)
        lib.qlinear_w4_actorder_prepare(qw_g, g_idx, G, qs, perm)
        # W8 NG -> N8 (fp32 activations)
        w8 = torch.randn((N8, NG), device=DEV) * 0.02
        q8 = torch.empty((N8, NG), dtype=torch.int8, device=DEV)
        s8 = torch.empty(N8, device=DEV)
        lib.dev_quantize_int8_channel(w8, q8, s8)
        w_dn = _w4(lib, H, F, 6)                # the MLP's down projection F -> H
        x = torch.randn((1, H), device=DEV).to(torch.bfloat16)
        outs = [torch.empty((1, H), dtype=torch.bfloat16, device=DEV),
                torch.empty((1, F), dtype=torch.bfloat16, device=DEV),
                torch.empty((1, N2), dtype=torch.bfloat16, device=DEV),
                torch.empty((1, NG), device=DEV),
                torch.empty((1, N8), device=DEV),
                torch.empty((1, H), dtype=torch.bfloat16, device=DEV)]
        y1, h, y2, y3, y4, y5 = outs

        def step():
            lib.qlinear_w4a16(x, w_a[0], w_a[1], w_a[2], None, H // 128, y1, 128, stream=st)
            lib.qlinear_w4a16_swiglu(y1, w_gu[0], w_gu[1], w_gu[2], h, 128, stream=st)
            lib.qlinear_w4a16(h, w_b[0], w_b[1], w_b[2], None, F // 128, y2, 128, stream=st)
            lib.qlinear_w4a16_actorder(y2, qs, sc_g, None, perm, y3, 128, stream=st)
            lib.qlinear_w8_gemv(y3, q8, s8, y4, stream=st)
            lib.qlinear_w4a16_mlp(y1, w_gu, w_dn, y5, 128, stream=st)

        step()
        s.synchronize()
        want = [t.clone() for t in outs]
        assert all(torch.isfinite(t.float()).all() for t in want)
        graph = lib.capture(step, st)
        try:
            for rep in range(4):
                for t in outs:
                    t.fill_(7)                                    # eager work on the stream between replays
                junk = torch.randn(1 << 20, device=DEV).sum()       # and elsewhere
                lib.graph_launch(graph, st)
                s.synchronize()
                for i, (t, w) in enumerate(zip(outs, want)):
                    assert torch.equal(t, w), (rep, i)
                assert torch.isfinite(junk)
                step()                                            # eager again: the same bits
                s.synchronize()
                assert all(torch.equal(t, w) for t, w in zip(outs, want))
        finally:
            lib.graph_destroy(graph)
