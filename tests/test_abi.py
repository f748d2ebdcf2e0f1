"""The C-ABI library builds, loads and exports every function the public
headers declare.  CPU only: no kernel is launched."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")
LIB = os.path.join(REPO, "sneppx-alg_amd", "libsneppx_quant.so")


def declared_functions():
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:SNEPPX|snx)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_the_reference_surface():
    names = declared_functions()
    reference = [
        "SNEPPX_quantize_int8_sym", "SNEPPX_dequantize_int8_sym", "SNEPPX_quantize_int8_asym",
        "SNEPPX_dequantize_int8_asym", "SNEPPX_quantize_int8_channel", "SNEPPX_quantize_int4_sym",
        "SNEPPX_dequantize_int4_sym", "SNEPPX_float_to_fp8_e4m3", "SNEPPX_fp8_e4m3_to_float",
        "SNEPPX_quantize_fp8_e4m3", "SNEPPX_dequantize_fp8_e4m3", "SNEPPX_float_to_fp8_e5m2",
        "SNEPPX_fp8_e5m2_to_float", "SNEPPX_quantize_fp8_e5m2", "SNEPPX_dequantize_fp8_e5m2",
        "SNEPPX_awq_scale_weights", "SNEPPX_awq_quantize", "SNEPPX_gptq_quantize",
        "SNEPPX_gptq_compute_hessian", "SNEPPX_gptq_quantize_block", "SNEPPX_quant_params_create",
        "SNEPPX_quant_mode_name",
    ]
    missing = [n for n in reference if n not in names]
    assert not missing, missing
    assert len(reference) == 22


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    import sneppx_quant  # noqa: F401  (imports torch first, as the product does)
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run __graft_entry__.build())")
def test_library_has_gfx950_code_and_no_other_target():
    # the offload bundle ids embedded in our own build name the targets
    blob = open(LIB, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob))
    assert targets == {b"gfx950"}, targets


def test_binding_refuses_to_run_without_the_library(tmp_path):
    import sneppx_quant
    with pytest.raises(sneppx_quant.SneppxError):
        sneppx_quant.Library(str(tmp_path / "missing.so"))
