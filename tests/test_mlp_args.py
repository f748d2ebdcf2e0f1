"""SNEPPX_qlinear_w4a16_mlp rejects bad arguments before it touches the
device: -1 and a reason for NULL pointers, empty shapes, widths that are not
multiples of 8, a group that does not divide both K dimensions, and an output
type other than bf16 / fp32.  CPU only (the pointers passed are never
dereferenced: every check runs first)."""
import ctypes as C

import pytest

import sneppx_quant as sq


@pytest.fixture(scope="module")
def L():
    return sq.load()


def _call(L, x=16, y=16, M=300, H=256, F=384, N=512, group=128, ydt=None):
    p = C.c_void_p(16)                     # stand-in device pointers, never read
    return L.fn["SNEPPX_qlinear_w4a16_mlp"](
        C.c_void_p(x) if x else None, p, p, p, None, p, p, p, None, C.c_void_p(y) if y else None,
        sq.SNEPPX_BFLOAT16 if ydt is None else ydt, M, H, F, N, group, None)


@pytest.mark.parametrize("kw,reason", [
    (dict(x=0), "NULL pointer"),
    (dict(y=0), "NULL pointer"),
    (dict(M=0), "empty shape"),
    (dict(N=0), "empty shape"),
    (dict(F=100), "multiples of 8"),
    (dict(H=260), "multiples of 8"),
    (dict(H=200), "must divide"),
    (dict(F=320, group=256), "must divide"),
    (dict(ydt=99), "y_dtype"),
])
def test_mlp_rejects_bad_arguments(L, kw, reason):
    assert _call(L, **kw) == -1
    assert reason in L.last_error()
