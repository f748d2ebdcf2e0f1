"""Quantized weights on disk (include/sneppx_qstore.h) and the model-zoo INT8
rule - CPU only: the safetensors reader/writer is host code, and the oracle
of weights.c:225-252 is pinned here against the reference's own weights.c
(oracle/_ref) and hand-computed cases.

Format conformance is checked both ways against the `safetensors` package
(an independent implementation of the file format)."""
import os
import struct

import numpy as np
import pytest

import sneppx_quant as sq

HAVE_LIB = os.path.exists(sq.LIB_PATH)
needs_lib = pytest.mark.skipif(not HAVE_LIB, reason="library not built")


@pytest.fixture(scope="module")
def L():
    return sq.load()


def _arrays():
    rng = np.random.default_rng(7)
    return {
        "layers.0.qweight": ("I32", rng.integers(-2**31, 2**31, (6, 4), dtype=np.int64).astype(np.int32)),
        "layers.0.scales": ("F16", rng.normal(0, 1, (6, 2)).astype(np.float16)),
        "layers.0.weight_scale": ("F32", rng.normal(0, 1, 6).astype(np.float32)),
        "emb": ("F64", rng.normal(0, 1, (2, 3, 2)).astype(np.float64)),
        "codes": ("I8", rng.integers(-128, 128, 17, dtype=np.int64).astype(np.int8)),
        "bytes": ("U8", rng.integers(0, 256, (3, 3), dtype=np.int64).astype(np.uint8)),
        "steps": ("I64", np.arange(5, dtype=np.int64) * 10**12),
        "half16": ("I16", np.arange(-3, 4, dtype=np.int16)),
        "empty": ("F32", np.zeros((0, 4), np.float32)),
        "scalar": ("F32", np.array(3.5, np.float32)),
        "quote\"d\\name": ("F32", np.ones(2, np.float32)),
    }


@needs_lib
def test_round_trip_every_dtype_shape_and_metadata(L, tmp_path):
    path = str(tmp_path / "rt.safetensors")
    arrs = _arrays()
    w = L.qstore_writer(path)
    for name, (dt, a) in arrs.items():
        w.add_host(name, dt, a)
    w.set_metadata("layers.0.format", "w4")
    w.set_metadata("note", "line1\nline2 \"quoted\"")
    w.close()
    raw = open(path, "rb").read()
    (hl,) = struct.unpack("<Q", raw[:8])
    assert hl % 8 == 0                      # data block 8-aligned, padding counted
    with L.qstore_open(path) as st:
        assert sorted(st.names()) == sorted(arrs)
        for name, (dt, a) in arrs.items():
            code, shape, nb = st.info(name)
            assert sq.QST_DTYPES[code] == dt and shape == a.shape and nb == a.nbytes
            np.testing.assert_array_equal(st.host(name), a)
        assert st.metadata("layers.0.format") == "w4"
        assert st.metadata("note") == "line1\nline2 \"quoted\""
        assert st.metadata("absent") is None
        assert st.info("absent") is None


@needs_lib
def test_files_we_write_load_in_the_safetensors_package(L, tmp_path):
    from safetensors.numpy import load_file
    path = str(tmp_path / "ours.safetensors")
    arrs = {k: v for k, v in _arrays().items() if v[0] != "F16" or True}
    w = L.qstore_writer(path)
    for name, (dt, a) in arrs.items():
        w.add_host(name, dt, a)
    w.set_metadata("format", "w4")
    w.close()
    got = load_file(path)
    assert sorted(got) == sorted(arrs)
    for name, (dt, a) in arrs.items():
        np.testing.assert_array_equal(got[name], a)
        assert got[name].dtype == a.dtype


@needs_lib
def test_files_of_the_safetensors_package_load_here(L, tmp_path):
    from safetensors.numpy import save_file
    path = str(tmp_path / "theirs.safetensors")
    rng = np.random.default_rng(3)
    arrs = {"model.layers.3.mlp.down_proj.qweight": rng.integers(0, 2**31, (8, 16)).astype(np.int32),
            "model.layers.3.mlp.down_proj.scales": rng.normal(0, 1, (8, 1)).astype(np.float16),
            "x": rng.normal(0, 1, (5,)).astype(np.float32),
            "b": np.array([True, False, True])}
    save_file(arrs, path, metadata={"quant_method": "awq", "bits": "4"})
    with L.qstore_open(path) as st:
        for name, a in arrs.items():
            np.testing.assert_array_equal(st.host(name), a)
        assert st.metadata("quant_method") == "awq" and st.metadata("bits") == "4"


def _reference_writer_bytes(tensors):
    """The byte layout SNEPPX_safetensors_save writes (fs/format/safetensors.c
    :454-480): JSON entries in insertion order, the u64 length of the
    *unpadded* JSON, the JSON, zero bytes up to an 8-byte boundary, the data.
    Restated here (the reference's safetensors.c does not build on this image:
    it calls _strdup, which glibc lacks)."""
    parts, off, data = [], 0, b""
    codes = {np.dtype(np.float32): "F32", np.dtype(np.int32): "I32", np.dtype(np.float16): "F16",
             np.dtype(np.int8): "I8"}
    for name, a in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        shape = ",".join(str(s) for s in a.shape)
        parts.append(f'"{name}":{{"dtype":"{codes[a.dtype]}","shape":[{shape}],'
                     f'"data_offsets":[{off},{off + len(b)}]}}')
        off += len(b)
        data += b
    hdr = ("{" + ",".join(parts) + "}").encode()
    pad = (8 - (len(hdr) & 7)) & 7
    return struct.pack("<Q", len(hdr)) + hdr + b"\0" * pad + data, pad


@needs_lib
def test_reads_files_of_the_reference_writer(L, tmp_path):
    rng = np.random.default_rng(11)
    for extra in range(8):        # every header length mod 8, so every padding
        t = {"w" * (1 + extra): rng.normal(0, 1, (3, 5)).astype(np.float32),
             "q": rng.integers(-128, 128, 7).astype(np.int8),
             "s": rng.normal(0, 1, 4).astype(np.float16)}
        blob, pad = _reference_writer_bytes(t)
        path = str(tmp_path / f"ref{extra}.safetensors")
        open(path, "wb").write(blob)
        with L.qstore_open(path) as st:
            for name, a in t.items():
                np.testing.assert_array_equal(st.host(name), a)


@needs_lib
@pytest.mark.parametrize("case", ["short", "huge_header", "not_object", "bad_entry", "past_end",
                                  "size_mismatch", "trailing", "byte_overflow"])
def test_malformed_files_are_rejected_with_a_reason(L, tmp_path, case):
    good = b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}'
    body = {
        "short": b"\x01\x02",
        "huge_header": struct.pack("<Q", 10**9) + good,
        "not_object": struct.pack("<Q", 4) + b"[1,2]" [:4],
        "bad_entry": struct.pack("<Q", 40) + b'{"a":{"dtype":"F32","shape":[2]}}      ' + b"\0" * 8,
        "past_end": struct.pack("<Q", len(good)) + good + b"\0" * 4,
        "size_mismatch": struct.pack("<Q", 54) + b'{"a":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}' + b"\0" * 8,
        "trailing": struct.pack("<Q", len(good) + 1) + good + b"x" + b"\0" * 8,
        # 2^62 I32 elements: the byte count wraps to 0, which would match [0, 0]
        "byte_overflow": struct.pack("<Q", 74) + b'{"q":{"dtype":"I32","shape":[4611686018427387904,1],"data_offsets":[0,0]}}',
    }[case]
    path = str(tmp_path / f"{case}.safetensors")
    open(path, "wb").write(body)
    with pytest.raises(sq.SneppxError) as e:
        L.qstore_open(path)
    assert "qstore_open" in str(e.value)


@needs_lib
def test_unknown_dtype_strings_stay_readable_as_bytes(L, tmp_path):
    hdr = b'{"u":{"dtype":"U32","shape":[2],"data_offsets":[0,8]}}'
    hdr += b" " * ((8 - len(hdr) % 8) % 8)
    path = str(tmp_path / "u32.safetensors")
    open(path, "wb").write(struct.pack("<Q", len(hdr)) + hdr + np.array([1, 2], np.uint32).tobytes())
    with L.qstore_open(path) as st:
        code, shape, nb = st.info("u")
        assert code == -1 and shape == (2,) and nb == 8
        np.testing.assert_array_equal(st.host("u").view(np.uint32), [1, 2])


@needs_lib
def test_w4_and_w8_layer_queries(L, tmp_path):
    N, K, g = 6, 256, 64
    G = K // g
    path = str(tmp_path / "layer.safetensors")
    w = L.qstore_writer(path)
    w.add_host("l.qweight", "I32", np.zeros((N, K // 8), np.int32))
    w.add_host("l.scales", "F16", np.ones((N, G), np.float16))
    w.add_host("l.qzeros", "I32", np.zeros((N, (G + 7) // 8), np.int32))
    w.add_host("gp.qweight", "I32", np.zeros((N, K // 8), np.int32))
    w.add_host("gp.scales", "F16", np.ones((N, G), np.float16))
    w.add_host("gp.g_idx", "I32", (np.arange(K) // g).astype(np.int32))
    w.add_host("bad.qweight", "I32", np.zeros((N, K // 8), np.int32))
    w.add_host("bad.scales", "F16", np.ones((N + 1, G), np.float16))
    w.add_host("w8.weight", "I8", np.zeros((N, K), np.int8))
    w.add_host("w8.weight_scale", "F32", np.ones(N, np.float32))
    w.close()
    with L.qstore_open(path) as st:
        assert st.query_w4("l") == (N, K, G, g, True, False)
        assert st.query_w4("gp") == (N, K, G, 0, False, True)
        with pytest.raises(sq.SneppxError, match="inconsistent"):
            st.query_w4("bad")
        with pytest.raises(sq.SneppxError, match="no missing.qweight"):
            st.query_w4("missing")
        assert st.query_w8("w8") == (N, K)


# ------------------------------------------------ model-zoo INT8 oracle pins

def test_modelzoo_oracle_known_answers(oracle):
    # m = 127 / 2 = 63.5; 1*63.5 = 63.5 -> 63 (truncation), -2*63.5 = -127,
    # 0.5*63.5 = 31.75 -> 31, -0.3*63.5 = -19.05 -> -19
    rc, q, m = oracle.quantize_int8_modelzoo(np.array([1.0, -2.0, 0.5, -0.3], np.float32))
    assert rc == 0 and m == np.float32(63.5)
    assert q.tolist() == [63, -127, 31, -19]
    # all zeros: multiplier 1, codes 0
    rc, q, m = oracle.quantize_int8_modelzoo(np.zeros(5, np.float32))
    assert m == 1.0 and not q.any()
    # NaN is skipped by the max scan and codes 0; an infinity makes the
    # multiplier 127/inf = 0, so every code is 0
    rc, q, m = oracle.quantize_int8_modelzoo(np.array([4.0, np.nan, -1.0], np.float32))
    assert m == np.float32(127.0 / 4.0) and q.tolist() == [127, 0, -31]
    rc, q, m = oracle.quantize_int8_modelzoo(np.array([1.0, np.inf], np.float32))
    assert m == 0.0 and q.tolist() == [0, 0]
    assert oracle.quantize_int8_modelzoo(np.zeros(0, np.float32))[0] == -1


def test_modelzoo_oracle_is_truncation_not_rounding(oracle):
    # against numpy's trunc of the same float32 products (the float32
    # multiply is one IEEE rounding in both)
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, 50000).astype(np.float32)
    rc, q, m = oracle.quantize_int8_modelzoo(x)
    mult = np.float32(127.0) / np.float32(np.abs(x).max())
    assert m == mult
    expect = np.trunc(np.clip(x * mult, -128, 127)).astype(np.int8)
    np.testing.assert_array_equal(q, expect)
    assert np.abs(q).max() == 127


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref",
                                                    "libsnxref.so")),
                    reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("seed", range(4))
def test_modelzoo_oracle_equals_reference_weights_c(oracle, seed):
    from py_oracle import Reference
    ref = Reference()
    rng = np.random.default_rng(seed)
    cases = [rng.normal(0, 1, 4096).astype(np.float32),
             (rng.normal(0, 1, 999) * 10.0 ** rng.integers(-40, 38)).astype(np.float32),
             np.array([0.0, -0.0, 1e-45, -1e-45], np.float32),
             np.array([2.0, np.nan, -3.0, np.nan], np.float32),
             np.array([np.inf, -1.0], np.float32),
             np.array([-np.inf, np.nan, 1.0], np.float32)]
    for x in cases:
        rc1, q1, _ = oracle.quantize_int8_modelzoo(x)
        rc2, q2 = ref.modelzoo_quantize_int8(x)
        assert rc1 == rc2 == 0
        np.testing.assert_array_equal(q1, q2)
