"""Quantized layers to disk and back (include/sneppx_qstore.h) and the device
model-zoo INT8 rule (weights.c:225-252), on the GPU.

Bar: everything here is integer or byte work - codes, scales and loaded
buffers are bit-exact; a linear run on loaded weights equals the same linear
on the weights that were saved, bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("n", [1, 3, 1000, 1 << 20])
def test_modelzoo_int8_device_and_host_bit_exact(lib, oracle, n):
    print(f"[gpu] modelzoo int8 n={n}", flush=True)
    rng = np.random.default_rng(n)
    x = rng.normal(0, 1, n).astype(np.float32)
    if n >= 1000:
        x[::97] = np.nan
        x[5] = -7.25
    rc, qo, mo = oracle.quantize_int8_modelzoo(x)
    q = torch.empty(n, dtype=torch.int8, device=DEV)
    m = torch.empty(1, device=DEV)
    lib.dev_quantize_int8_modelzoo(to_dev(x), q, m)
    torch.cuda.synchronize()
    assert host(m)[0] == mo
    np.testing.assert_array_equal(host(q), qo)
    rc2, qh, mh = lib.quantize_int8_modelzoo(x)
    assert rc2 == 0 and mh == mo
    np.testing.assert_array_equal(qh, qo)


def test_modelzoo_int8_special_values(lib, oracle):
    for x in [np.zeros(7, np.float32),
              np.array([1.0, np.inf, -2.0], np.float32),
              np.array([1e-45, -2e-45, 0.0], np.float32),
              np.array([np.nan, np.nan], np.float32),
              np.array([3.0e38, -3.4e38, 1.0], np.float32)]:
        rc, qo, mo = oracle.quantize_int8_modelzoo(x)
        rc2, qh, mh = lib.quantize_int8_modelzoo(x)
        assert rc2 == 0
        np.testing.assert_array_equal(qh, qo)
        assert mh == mo or (np.isnan(mh) and np.isnan(mo))


def _w4_device(lib, N, K, group, seed):
    w = torch.from_numpy(np.random.default_rng(seed).normal(0, 0.02, (N, K)).astype(np.float32)).to(DEV)
    G = K // group
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    qz = torch.empty((N, (G + 7) // 8), dtype=torch.int32, device=DEV)
    lib.dev_quantize_w4_awq(w, qw, sc, qz, group)
    return qw, sc, qz, G


@pytest.mark.parametrize("N,K,group", [(24, 512, 128), (4096, 4096, 128), (40, 1024, 256)])
def test_w4_layer_save_load_round_trip(lib, tmp_path, N, K, group):
    print(f"[gpu] qstore w4 N={N} K={K} g={group}", flush=True)
    qw, sc, qz, G = _w4_device(lib, N, K, group, N)
    path = str(tmp_path / "w4.safetensors")
    w = lib.qstore_writer(path)
    w.save_w4("model.layers.0.mlp.up_proj", qw, sc, qz, None, N, K, group, G)
    w.close()
    with lib.qstore_open(path) as st:
        assert st.query_w4("model.layers.0.mlp.up_proj") == (N, K, G, group, True, False)
        assert st.metadata("model.layers.0.mlp.up_proj.format") == "w4"
        assert st.metadata("model.layers.0.mlp.up_proj.group_size") == str(group)
        qw2, sc2, qz2 = torch.zeros_like(qw), torch.zeros_like(sc), torch.zeros_like(qz)
        st.load_w4("model.layers.0.mlp.up_proj", qw2, sc2, qz2)
        with pytest.raises(Exception, match="destinations must match"):
            st.load_w4("model.layers.0.mlp.up_proj", qw2, sc2, None)
    torch.cuda.synchronize()
    for a, b in ((qw, qw2), (sc, sc2), (qz, qz2)):
        np.testing.assert_array_equal(host(a), host(b))
    # the loaded layer computes exactly what the saved one does
    M = 3
    x = torch.randn((M, K), device=DEV).to(torch.bfloat16)
    y1 = torch.empty((M, N), device=DEV)
    y2 = torch.empty((M, N), device=DEV)
    lib.qlinear_w4a16(x.view(torch.int16), qw, sc, qz, None, G, y1, group)
    lib.qlinear_w4a16(x.view(torch.int16), qw2, sc2, qz2, None, G, y2, group)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_w4_gptq_layer_with_g_idx_round_trip(lib, tmp_path):
    N, K = 64, 1024
    rng = np.random.default_rng(9)
    g_idx = (rng.permutation(K) // 128).astype(np.int32)
    G = 8
    w = torch.from_numpy(rng.normal(0, 0.02, (N, K)).astype(np.float32)).to(DEV)
    qw = torch.empty((N, K // 8), dtype=torch.int32, device=DEV)
    sc = torch.empty((N, G), dtype=torch.int16, device=DEV)
    gi = to_dev(g_idx)
    lib.dev_quantize_w4_gptq(w, gi, G, qw, sc)
    path = str(tmp_path / "gptq.safetensors")
    wr = lib.qstore_writer(path)
    wr.save_w4("q", qw, sc, None, gi, N, K, 0, G)
    wr.close()
    with lib.qstore_open(path) as st:
        assert st.query_w4("q") == (N, K, G, 0, False, True)
        qw2, sc2, gi2 = torch.zeros_like(qw), torch.zeros_like(sc), torch.zeros_like(gi)
        st.load_w4("q", qw2, sc2, None, gi2)
    torch.cuda.synchronize()
    for a, b in ((qw, qw2), (sc, sc2), (gi, gi2)):
        np.testing.assert_array_equal(host(a), host(b))


def test_w8_layer_save_load_round_trip(lib, tmp_path):
    N, K = 300, 4096
    w = torch.from_numpy(np.random.default_rng(4).normal(0, 0.02, (N, K)).astype(np.float32)).to(DEV)
    q = torch.empty((N, K), dtype=torch.int8, device=DEV)
    s = torch.empty(N, device=DEV)
    lib.dev_quantize_int8_channel(w, q, s)
    path = str(tmp_path / "w8.safetensors")
    wr = lib.qstore_writer(path)
    wr.save_w8("o_proj", q, s)
    wr.close()
    with lib.qstore_open(path) as st:
        assert st.query_w8("o_proj") == (N, K)
        q2, s2 = torch.zeros_like(q), torch.zeros_like(s)
        st.load_w8("o_proj", q2, s2)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_save_w4_rejects_inconsistent_group(lib, tmp_path):
    qw, sc, qz, G = _w4_device(lib, 8, 256, 64, 1)
    wr = lib.qstore_writer(str(tmp_path / "bad.safetensors"))
    with pytest.raises(Exception, match="qstore_save_w4"):
        wr.save_w4("x", qw, sc, qz, None, 8, 256, 128, G)   # 256/128 = 2 groups, not 4
    wr.close()
