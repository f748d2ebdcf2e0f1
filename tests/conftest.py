"""Shared pytest setup.

Markers: `gpu` tests need an MI355X (HIP device) and call the product library
through its C-ABI; everything else runs on the CPU.
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "oracle"), os.path.join(REPO, "sneppx-alg_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden", "ref_quant.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the product kernels")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def oracle():
    from py_oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def lib():
    """The product library on a real GPU; a missing GPU or library is a failure."""
    import torch
    import sneppx_quant
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a HIP device")
    lib = sneppx_quant.load()
    arch, cus, _ = lib.device_info()
    print(f"[gpu] {arch} with {cus} CUs, library {lib.path}", flush=True)
    return lib
