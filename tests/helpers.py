"""Helpers shared by the test modules (fixture access, bitwise comparison)."""
import numpy as np


def cases(golden, prefix):
    """Group fixture keys '<case>__<field>' whose case starts with prefix."""
    out = {}
    for k, v in golden.items():
        case, field = k.split("__", 1)
        if case == prefix or case.startswith(prefix + "_"):
            out.setdefault(case, {})[field] = v
    return out


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a = a.view(np.uint32)
    if b.dtype == np.float32:
        b = b.view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)
