"""Quantized layers at the reference's linear call sites (include/sneppx_qlayer.h).

The reference multiplies x [M, K] by W [K, N] in fp32 (attention.c:324-345,
inference_engine.c:264).  A layer built from that W must hold exactly the
codes the oracle gives for W^T (the output-major layout of the linears), and
its products must match the oracle linear on those codes: fp32 activations
(W8) within 1e-4, bf16 activations (W4) within 1e-4 of the oracle fed the
same bf16-rounded activations.  Layers saved and loaded compute bit-identical
outputs."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_F32 = 1e-4


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _weights(K, N, seed):
    return np.random.default_rng(seed).normal(0, 0.02, (K, N)).astype(np.float32)


@pytest.mark.parametrize("K,N,M", [(512, 96, 1), (4096, 6144, 4), (4096, 11008, 37), (4096, 4096, 300)])
def test_w4_layer_from_reference_layout(lib, oracle, tmp_path, K, N, M):
    print(f"[gpu] qlayer w4 K={K} N={N} M={M}", flush=True)
    w_kn = _weights(K, N, K + N)
    layer = lib.qlayer_create_kn(w_kn, "w4", 128)
    assert (layer.K, layer.N, layer.format) == (K, N, "w4")
    # codes: bit-exact with the oracle quantizing W^T
    path = str(tmp_path / "l.safetensors")
    wr = lib.qstore_writer(path)
    layer.save(wr, "l")
    wr.close()
    rc, qw, sc, qz = oracle.w4_awq_quantize(np.ascontiguousarray(w_kn.T), 128)
    with lib.qstore_open(path) as st:
        np.testing.assert_array_equal(st.host("l.qweight").view(np.uint32), qw)
        np.testing.assert_array_equal(st.host("l.scales").view(np.uint16), sc)
        np.testing.assert_array_equal(st.host("l.qzeros").view(np.uint32), qz)
    # forward with fp32 activations (rounded to bf16 on the way in)
    x = np.random.default_rng(M).normal(0, 1, (M, K)).astype(np.float32)
    y = torch.empty((M, N), device=DEV)
    layer.forward_f32(torch.from_numpy(x).to(DEV), y)
    torch.cuda.synchronize()
    rc, yo = oracle.w4a16_linear(bf16_bits(x), qw, sc, qz, None, N, K, 128)
    assert rel_err(y.cpu().numpy(), yo) <= TOL_F32
    # host buffers in and out: the same numbers
    yh = layer.matmul_host(x)
    np.testing.assert_array_equal(yh, y.cpu().numpy())


@pytest.mark.parametrize("K,N,M", [(4096, 4096, 1), (1024, 300, 5)])
def test_w8_layer_from_reference_layout(lib, oracle, tmp_path, K, N, M):
    w_kn = _weights(K, N, 3)
    layer = lib.qlayer_create_kn(w_kn, "w8")
    path = str(tmp_path / "w8.safetensors")
    wr = lib.qstore_writer(path)
    layer.save(wr, "w8")
    wr.close()
    rc, q, s = oracle.quantize_int8_channel(np.ascontiguousarray(w_kn.T))
    with lib.qstore_open(path) as st:
        np.testing.assert_array_equal(st.host("w8.weight"), q)
        np.testing.assert_array_equal(st.host("w8.weight_scale").view(np.uint32), s.view(np.uint32))
    x = np.random.default_rng(1).normal(0, 1, (M, K)).astype(np.float32)
    y = layer.matmul_host(x)
    rc, yo = oracle.w8_linear(x, q, s)
    assert rel_err(y, yo) <= TOL_F32
    with pytest.raises(Exception, match="fp32 activations"):
        layer.forward_bf16(torch.zeros((M, K), dtype=torch.int16, device=DEV),
                           torch.zeros((M, N), dtype=torch.int16, device=DEV))


def test_lm_head_shape_and_device_weight(lib, oracle):
    # inference_engine.c:264: logits = flat [1, d_model] . unembed [d_model, vocab]
    K, N = 4096, 32000
    w_kn = _weights(K, N, 11)
    layer = lib.qlayer_create_kn(torch.from_numpy(w_kn).to(DEV), "w4", 128)
    x = np.random.default_rng(2).normal(0, 1, (1, K)).astype(np.float32)
    xb = torch.from_numpy(bf16_bits(x).view(np.int16)).to(DEV)
    y = torch.empty((1, N), dtype=torch.int16, device=DEV)
    layer.forward_bf16(xb, y)
    torch.cuda.synchronize()
    rc, qw, sc, qz = oracle.w4_awq_quantize(np.ascontiguousarray(w_kn.T), 128)
    rc, yo = oracle.w4a16_linear(bf16_bits(x), qw, sc, qz, None, N, K, 128)
    got = (y.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    assert rel_err(got, yo) <= 1e-2


@pytest.mark.parametrize("M,zeros", [(3, False), (1, True), (8, True)])
def test_loaded_actorder_layer_is_prepared_and_exact(lib, oracle, tmp_path, M, zeros):
    # GPTQ act-order files with and without zero points (qzeros [N][G/8]):
    # loading prepares them, and M = 1 / 8 run the prepared decode kernels
    K, N = 2048, 512
    rng = np.random.default_rng(8 + M)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    rc, qw, sc = oracle.w4_gptq_quantize(w, g_idx, 16)
    qz = None
    if zeros:
        z = rng.integers(0, 16, (N, 16)).astype(np.uint32)
        qz = (z.reshape(N, 2, 8) << (4 * np.arange(8, dtype=np.uint32))).sum(-1).astype(np.uint32)
    path = str(tmp_path / "gptq.safetensors")
    wr = lib.qstore_writer(path)
    wr.add_host("g.qweight", "I32", qw.view(np.int32))
    wr.add_host("g.scales", "F16", sc.view(np.float16))
    wr.add_host("g.g_idx", "I32", g_idx)
    if zeros:
        wr.add_host("g.qzeros", "I32", qz.view(np.int32))
    wr.close()
    with lib.qstore_open(path) as st:
        layer = lib.qlayer_load(st, "g")
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    y = layer.matmul_host(x)
    rc, yo = oracle.w4a16_linear(bf16_bits(x), qw, sc, qz, g_idx, N, K, 128)
    assert rel_err(y, yo) <= TOL_F32
    # saved again, it round-trips to the same tensors
    path2 = str(tmp_path / "gptq2.safetensors")
    wr = lib.qstore_writer(path2)
    layer.save(wr, "g")
    wr.close()
    with lib.qstore_open(path2) as st:
        np.testing.assert_array_equal(st.host("g.qweight").view(np.uint32), qw)
        np.testing.assert_array_equal(st.host("g.g_idx"), g_idx)


def test_layer_round_trip_through_a_file_is_bit_identical(lib, tmp_path):
    K, N, M = 4096, 1024, 7
    layer = lib.qlayer_create_kn(_weights(K, N, 5), "w4", 128)
    path = str(tmp_path / "rt.safetensors")
    wr = lib.qstore_writer(path)
    layer.save(wr, "model.layers.7.self_attn.q_proj")
    wr.close()
    with lib.qstore_open(path) as st:
        layer2 = lib.qlayer_load(st, "model.layers.7.self_attn.q_proj")
    x = np.random.default_rng(0).normal(0, 1, (M, K)).astype(np.float32)
    np.testing.assert_array_equal(layer.matmul_host(x), layer2.matmul_host(x))


def test_create_rejects_bad_arguments(lib):
    with pytest.raises(Exception, match="group"):
        lib.qlayer_create_kn(_weights(100, 8, 0), "w4", 128)    # 128 does not divide 100
    with pytest.raises(Exception, match="group"):
        lib.qlayer_create_kn(_weights(128, 8, 0), "w4", 12)     # not a multiple of 8

