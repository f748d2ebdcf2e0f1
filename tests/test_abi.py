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


REF_KERNEL_INC = "/root/reference/include/neural_core/kernel"
needs_ref_header = pytest.mark.skipif(not os.path.exists(os.path.join(REF_KERNEL_INC, "quantization.h")),
                                      reason="reference tree absent (build container only)")


def _gcc(args, cwd):
    import subprocess
    r = subprocess.run(["gcc", "-std=gnu11", "-Wall", "-Werror", *args], cwd=cwd,
                       capture_output=True, text=True)
    return r.returncode, r.stdout + r.stderr


@needs_ref_header
def test_prototypes_compile_against_the_reference_header(tmp_path):
    """One translation unit includes the reference's quantization.h, then
    include/sneppx_quantization.h: every prototype of ours redeclares the
    reference's, so a changed return or argument type fails to compile.  A
    planted drift (one argument type changed) must fail the same build."""
    ours = open(os.path.join(INCLUDE, "sneppx_quantization.h")).read()
    src = ('#include "quantization.h"\n#include "sneppx_quantization.h"\n'
           "int main(void) { return (int)sizeof(SNEPPXQuantParams) == 0; }\n")
    (tmp_path / "pin.c").write_text(src)
    args = ["-fsyntax-only", f"-I{tmp_path}", f"-I{INCLUDE}", f"-I{REF_KERNEL_INC}",
            "-I/root/reference/include", "pin.c"]
    rc, out = _gcc(args, tmp_path)
    assert rc == 0, out
    drift = ours.replace("int SNEPPX_dequantize_int8_sym(const int8_t* input, float* output,\n"
                         "                               size_t n, float scale);",
                         "int SNEPPX_dequantize_int8_sym(const int8_t* input, float* output,\n"
                         "                               size_t n, double scale);")
    assert drift != ours
    (tmp_path / "sneppx_quantization.h").write_text(drift)   # found first: -I tmp_path
    rc, out = _gcc(args, tmp_path)
    assert rc != 0 and "conflicting types" in out, out


@needs_ref_header
def test_type_abi_matches_the_reference_header(tmp_path):
    """Enum ordinals, struct sizes and field offsets: the same program built
    once against each header prints the same table."""
    import subprocess
    body = r'''
#include <stddef.h>
#include <stdio.h>
#define E(x) printf(#x " %d\n", (int)(x))
#define O(t, f) printf(#t "." #f " %zu\n", offsetof(t, f))
int main(void) {
    E(SNEPPX_QUANT_NONE); E(SNEPPX_QUANT_INT8_SYM); E(SNEPPX_QUANT_INT8_ASYM); E(SNEPPX_QUANT_INT4_SYM);
    E(SNEPPX_QUANT_FP8_E4M3); E(SNEPPX_QUANT_FP8_E5M2); E(SNEPPX_QUANT_AWQ); E(SNEPPX_QUANT_GPTQ);
    E(SNEPPX_QUANT_PER_TENSOR); E(SNEPPX_QUANT_PER_CHANNEL); E(SNEPPX_QUANT_PER_GROUP);
    E(SNEPPX_QUANT_PER_TOKEN);
    E(SNEPPX_FLOAT32); E(SNEPPX_FLOAT16); E(SNEPPX_BFLOAT16); E(SNEPPX_INT8); E(SNEPPX_UINT8);
    E(sizeof(SNEPPXQuantParams)); O(SNEPPXQuantParams, scale); O(SNEPPXQuantParams, zero_point);
    O(SNEPPXQuantParams, qmin); O(SNEPPXQuantParams, qmax); O(SNEPPXQuantParams, scale_max);
    E(sizeof(SNEPPXQuantState)); O(SNEPPXQuantState, scales); O(SNEPPXQuantState, zero_points);
    O(SNEPPXQuantState, num_params); O(SNEPPXQuantState, granularity);
    E(sizeof(SNEPPXGPTQState)); O(SNEPPXGPTQState, weights); O(SNEPPXGPTQState, hessian);
    O(SNEPPXGPTQState, rows); O(SNEPPXGPTQState, cols); O(SNEPPXGPTQState, group_size);
    E(sizeof(SNEPPXDtype)); E(sizeof(SNEPPXQuantMode));
    return 0;
}
'''
    tables = []
    for name, inc, extra in (("ref", "quantization.h", [f"-I{REF_KERNEL_INC}", "-I/root/reference/include"]),
                             ("ours", "sneppx_quantization.h", [f"-I{INCLUDE}"])):
        (tmp_path / f"{name}.c").write_text(f'#include "{inc}"\n' + body)
        rc, out = _gcc([*extra, f"{name}.c", "-o", name], tmp_path)
        assert rc == 0, out
        tables.append(subprocess.run([str(tmp_path / name)], capture_output=True, text=True,
                                     check=True).stdout)
    assert tables[0] == tables[1]
    assert "SNEPPX_QUANT_GPTQ 7" in tables[0] and "SNEPPX_BFLOAT16 3" in tables[0]
