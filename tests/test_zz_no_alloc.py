"""The allocation-free entry point SNEPPX_qlinear_w4a16_noalloc against
SNEPPX_qlinear_w4a16 through the C-ABI: same kernels, so bit-identical
outputs, on two calls in a row per path (the second smaller, reusing the
static scratch array the first one filled), and a clear error for a call
whose scratch would exceed the array.  Where the allocating entry point
splits the prefill GEMM's K into spans (few tiles), the allocation-free one
runs it whole: the same product with another fp32 summation order, checked
to the bf16 tolerance."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH = 32 << 20          # SNEPPX_NOALLOC_SCRATCH_BYTES


def _layer(lib, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn((N, K), device=DEV, generator=g) * 0.02
    G = K // 128
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, 128)
    return qw, sc, qz, G


def _both(lib, M, N, K, seed, ydt=torch.bfloat16, bias=False):
    qw, sc, qz, G = _layer(lib, N, K, seed)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    x = torch.randn((M, K), device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randn(N, device=DEV, generator=g) if bias else None
    y_ref = torch.full((M, N), 7, dtype=ydt, device=DEV)
    y = torch.full((M, N), 9, dtype=ydt, device=DEV)
    lib.qlinear_w4a16(x, qw, sc, qz, None, G, y_ref, 128, bias=b)
    lib.qlinear_w4a16_noalloc(x, qw, sc, qz, None, G, y, 128, bias=b)
    torch.cuda.synchronize()
    return y, y_ref


@pytest.mark.parametrize("first,second", [
    ((16, 11008, 14336), (8, 4096, 14336)),     # split-K partials: 9.9 MB, then 1.8 MB
    ((1849, 4096, 4096), (300, 11008, 4096)),   # prefill GEMM, prepared activations: 15 MB, then 2.5 MB
    ((1, 11008, 4096), (4, 1000, 4096)),        # kernels without scratch
])
def test_noalloc_matches_the_allocating_entry_point(lib, first, second):
    for i, (M, N, K) in enumerate((first, second)):
        print(f"[gpu] noalloc M={M} N={N} K={K}", flush=True)
        y, y_ref = _both(lib, M, N, K, seed=M + N + i, bias=(i == 1))
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), (M, N, K)


def test_noalloc_where_the_allocating_entry_point_splits_k(lib):
    # 12 tiles: the allocating entry point runs K in 4 spans, this one whole
    for M, N, K in ((300, 1000, 4096), (1849, 768, 4096)):
        print(f"[gpu] noalloc vs split M={M} N={N} K={K}", flush=True)
        y, y_ref = _both(lib, M, N, K, seed=M + N)
        a, b = y.float(), y_ref.float()
        assert float((a - b).abs().max() / b.abs().max()) <= 1e-2, (M, N, K)


def test_noalloc_fp32_output_and_bias(lib):
    y, y_ref = _both(lib, 12, 2048, 8192, seed=3, ydt=torch.float32, bias=True)
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32))


def test_noalloc_rejects_calls_beyond_its_scratch(lib):
    # prefill at K = 14336 and M = 2048 needs 2 M K = 58.7 MB of prepared activations
    M, N, K = 2048, 256, 14336
    assert 2 * M * K > SCRATCH
    qw, sc, qz, G = _layer(lib, N, K, 5)
    x = torch.zeros((M, K), dtype=torch.bfloat16, device=DEV)
    y = torch.full((M, N), 3, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(Exception, match="static buffer"):
        lib.qlinear_w4a16_noalloc(x, qw, sc, qz, None, G, y, 128)
    torch.cuda.synchronize()
    assert bool((y == 3).all())                # nothing was launched
