"""ctypes access to the CPU oracle (oracle/liboracle*.so) and, in the build
container only, to the reference compiled unchanged (oracle/_ref/libsnxref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never on the product path.

All wrappers take and return numpy arrays.  Function names drop the `orc_`
prefix; the reference binding exposes the reference's own symbol names.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
ORACLE_PERF_SO = os.path.join(HERE, "liboracle_perf.so")
REF_SO = os.path.join(HERE, "_ref", "libsnxref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C")
_sz = C.c_size_t


class QuantParams(C.Structure):
    """SNEPPXQuantParams (quantization.h:44-50)."""
    _fields_ = [("scale", C.c_float), ("zero_point", C.c_int32), ("qmin", C.c_float),
                ("qmax", C.c_float), ("scale_max", C.c_float)]


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


# Signatures shared by the reference ABI (SNEPPX_*) and the oracle (orc_*).
_COMMON = {
    "quantize_int8_sym": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float)]),
    "dequantize_int8_sym": (C.c_int, [_i8p, _f32p, _sz, C.c_float]),
    "quantize_int8_asym": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float), C.POINTER(C.c_int32)]),
    "dequantize_int8_asym": (C.c_int, [_i8p, _f32p, _sz, C.c_float, C.c_int32]),
    "quantize_int8_channel": (C.c_int, [_f32p, _i8p, _sz, _sz, _f32p]),
    "quantize_int4_sym": (C.c_int, [_f32p, _u8p, _sz, C.POINTER(C.c_float)]),
    "dequantize_int4_sym": (C.c_int, [_u8p, _f32p, _sz, C.c_float]),
    "float_to_fp8_e4m3": (C.c_uint8, [C.c_float]),
    "fp8_e4m3_to_float": (C.c_float, [C.c_uint8]),
    "quantize_fp8_e4m3": (C.c_int, [_f32p, _u8p, _sz]),
    "dequantize_fp8_e4m3": (C.c_int, [_u8p, _f32p, _sz]),
    "float_to_fp8_e5m2": (C.c_uint8, [C.c_float]),
    "fp8_e5m2_to_float": (C.c_float, [C.c_uint8]),
    "quantize_fp8_e5m2": (C.c_int, [_f32p, _u8p, _sz]),
    "dequantize_fp8_e5m2": (C.c_int, [_u8p, _f32p, _sz]),
    "awq_scale_weights": (C.c_int, [_f32p, _sz, _sz, _f32p, _f32p]),
    "awq_quantize": (C.c_int, [_f32p, _i8p, C.c_void_p, _f32p, _sz, _sz, C.c_int]),
    "gptq_compute_hessian": (C.c_int, [_f32p, _f32p, _sz, _sz]),
    "gptq_quantize_block": (C.c_int, [_f32p, _f32p, _f32p, C.POINTER(C.c_float),
                                      C.POINTER(C.c_int32), _sz, C.c_int, C.c_int]),
    "gptq_quantize": (C.c_int, [_f32p, _sz, _sz, C.c_int, C.c_int, _i8p, _f32p,
                                C.c_void_p, C.c_int]),
    "quant_params_create": (C.c_int, [C.POINTER(QuantParams), C.c_int]),
    "quant_mode_name": (C.c_char_p, [C.c_int]),
}

_ORACLE_ONLY = {
    "quantize_int8_channel_rne": (C.c_int, [_f32p, _i8p, _sz, _sz, _f32p]),
    "gptq_quantize_literal": _COMMON["gptq_quantize"],
    "fake_quant": (C.c_int, [_f32p, _f32p, _sz, C.c_float, C.c_int]),
    "quantize_int8_modelzoo": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float)]),
    "matmul_kn": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz]),
    "matmul_nk": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz]),
    "f32_to_bf16": (C.c_uint16, [C.c_float]),
    "f32_to_f16": (C.c_uint16, [C.c_float]),
    "f16_to_f32": (C.c_float, [C.c_uint16]),
    "w4_scale_to_f16": (C.c_uint16, [C.c_float]),
    "w4_awq_quantize": (C.c_int, [_f32p, _sz, _sz, C.c_int, _u32p, _u16p, _u32p]),
    "w4_gptq_quantize": (C.c_int, [_f32p, _i32p, _sz, _sz, _sz, _u32p, _u16p]),
    "w4_dequantize": (C.c_int, [_u32p, _u16p, C.c_void_p, C.c_void_p, _sz, _sz, C.c_int, _f32p]),
    "w4a16_linear": (C.c_int, [_u16p, _u32p, _u16p, C.c_void_p, C.c_void_p, _sz, _sz, _sz,
                               C.c_int, _f32p]),
    "w8_linear": (C.c_int, [_f32p, _i8p, _f32p, _sz, _sz, _sz, _f32p]),
    "i8_gemm_i32": (None, [_i8p, _i8p, _i32p, _sz, _sz, _sz]),
    "w8a8_epilogue": (None, [_i32p, _f32p, _f32p, _sz, _sz, _f32p]),
    "add_bias": (None, [_f32p, _f32p, _sz, _sz]),
    "quantize_fp8_e4m3_scaled": (C.c_int, [_f32p, _u8p, _sz, C.POINTER(C.c_float)]),
    "fp8_gemm": (None, [_u8p, _u8p, C.c_float, C.c_float, _sz, _sz, _sz, _f32p]),
}


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class _Lib:
    """Thin numpy-facing wrapper over one of the shared objects."""

    def __init__(self, path: str, prefix: str, table: dict):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle` / `make -C oracle ref`)")
        self.path = path
        self.lib = C.CDLL(path)
        self.raw = {}
        for name, (res, args) in table.items():
            self.raw[name] = _sig(self.lib, prefix + name, res, args)

    # -- reference surface ---------------------------------------------------
    def quantize_int8_sym(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.size, np.int8)
        s = C.c_float(0)
        rc = self.raw["quantize_int8_sym"](x, q, x.size, C.byref(s))
        return rc, q, np.float32(s.value)

    def dequantize_int8_sym(self, q, scale):
        q = np.ascontiguousarray(q, np.int8)
        y = np.zeros(q.size, np.float32)
        rc = self.raw["dequantize_int8_sym"](q, y, q.size, scale)
        return rc, y

    def quantize_int8_asym(self, x):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.size, np.int8)
        s, z = C.c_float(0), C.c_int32(0)
        rc = self.raw["quantize_int8_asym"](x, q, x.size, C.byref(s), C.byref(z))
        return rc, q, np.float32(s.value), int(z.value)

    def dequantize_int8_asym(self, q, scale, zp):
        q = np.ascontiguousarray(q, np.int8)
        y = np.zeros(q.size, np.float32)
        rc = self.raw["dequantize_int8_asym"](q, y, q.size, scale, zp)
        return rc, y

    def quantize_int8_channel(self, x):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        q = np.zeros((rows, cols), np.int8)
        s = np.zeros(rows, np.float32)
        rc = self.raw["quantize_int8_channel"](x, q, rows, cols, s)
        return rc, q, s

    def quantize_int8_channel_rne(self, x):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        q = np.zeros((rows, cols), np.int8)
        s = np.zeros(rows, np.float32)
        rc = self.raw["quantize_int8_channel_rne"](x, q, rows, cols, s)
        return rc, q, s

    def quantize_int4_sym(self, x):
        x = np.ascontiguousarray(x, np.float32)
        p = np.zeros((x.size + 1) // 2, np.uint8)
        s = C.c_float(0)
        rc = self.raw["quantize_int4_sym"](x, p, x.size, C.byref(s))
        return rc, p, np.float32(s.value)

    def dequantize_int4_sym(self, packed, n, scale):
        packed = np.ascontiguousarray(packed, np.uint8)
        y = np.zeros(n, np.float32)
        rc = self.raw["dequantize_int4_sym"](packed, y, n, scale)
        return rc, y

    def quantize_fp8(self, x, fmt="e4m3"):
        x = np.ascontiguousarray(x, np.float32)
        c = np.zeros(x.size, np.uint8)
        rc = self.raw[f"quantize_fp8_{fmt}"](x, c, x.size)
        return rc, c

    def dequantize_fp8(self, c, fmt="e4m3"):
        c = np.ascontiguousarray(c, np.uint8)
        y = np.zeros(c.size, np.float32)
        rc = self.raw[f"dequantize_fp8_{fmt}"](c, y, c.size)
        return rc, y

    def awq_scale_weights(self, w, act_scales):
        w = np.array(w, np.float32, order="C", copy=True)
        rows, cols = w.shape
        s = np.zeros((rows, cols), np.float32)
        a = np.ascontiguousarray(act_scales, np.float32)
        rc = self.raw["awq_scale_weights"](w, rows, cols, a, s)
        return rc, w, s

    def awq_quantize(self, w, group_size, act_scales=None):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        g = group_size if group_size > 0 else 128
        ng = (cols + g - 1) // g
        q = np.zeros((rows, cols), np.int8)
        s = np.zeros((rows, ng), np.float32)
        a = None if act_scales is None else np.ascontiguousarray(act_scales, np.float32)
        rc = self.raw["awq_quantize"](w, q, _ptr(a), s, rows, cols, group_size)
        return rc, q, s

    def gptq_compute_hessian(self, act):
        act = np.ascontiguousarray(act, np.float32)
        n, dim = act.shape
        h = np.zeros((dim, dim), np.float32)
        rc = self.raw["gptq_compute_hessian"](h, act, n, dim)
        return rc, h

    def gptq_quantize_block(self, w, h_inv, bits, sym):
        w = np.array(w, np.float32, order="C", copy=True)
        h = np.array(h_inv, np.float32, order="C", copy=True)
        qw = np.zeros(w.size, np.float32)
        s, z = C.c_float(0), C.c_int32(-7)
        rc = self.raw["gptq_quantize_block"](w, h, qw, C.byref(s), C.byref(z), w.size, bits, sym)
        return rc, w, qw, np.float32(s.value), int(z.value)

    def gptq_quantize(self, w, group_size, bits, sym, with_zeros=True, name="gptq_quantize"):
        w = np.array(w, np.float32, order="C", copy=True)
        rows, cols = w.shape
        g = group_size if group_size > 0 else 128
        ng = (cols + g - 1) // g
        q = np.full((rows, cols), 0x55, np.int8)
        s = np.zeros((rows, ng), np.float32)
        z = np.full((rows, ng), -7, np.int32) if with_zeros else None
        rc = self.raw[name](w, rows, cols, group_size, bits, q, s, _ptr(z), sym)
        return rc, w, q, s, z

    def quant_params_create(self, mode):
        p = QuantParams()
        rc = self.raw["quant_params_create"](C.byref(p), mode)
        return rc, (p.scale, p.zero_point, p.qmin, p.qmax, p.scale_max)

    def quant_mode_name(self, mode):
        return self.raw["quant_mode_name"](mode).decode()


class Oracle(_Lib):
    """The restatement (orc_*) plus the build-defined formats."""

    def __init__(self, perf: bool = False):
        table = dict(_COMMON)
        table.update(_ORACLE_ONLY)
        super().__init__(ORACLE_PERF_SO if perf else ORACLE_SO, "orc_", table)

    def gptq_quantize_literal(self, w, group_size, bits, sym, with_zeros=True):
        return self.gptq_quantize(w, group_size, bits, sym, with_zeros, name="gptq_quantize_literal")

    def fake_quant(self, x, scale, bits):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(x.size, np.float32)
        rc = self.raw["fake_quant"](x, y, x.size, scale, bits)
        return rc, y

    def quantize_int8_modelzoo(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        m = C.c_float(0)
        rc = self.raw["quantize_int8_modelzoo"](x, q, x.size, C.byref(m))
        return rc, q, np.float32(m.value)

    def matmul_nk(self, a, w):
        a = np.ascontiguousarray(a, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        M, K = a.shape
        N = w.shape[0]
        y = np.zeros((M, N), np.float32)
        self.raw["matmul_nk"](a, w, y, M, K, N)
        return y

    def matmul_kn(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        M, K = a.shape
        N = b.shape[1]
        y = np.zeros((M, N), np.float32)
        self.raw["matmul_kn"](a, b, y, M, K, N)
        return y

    def f32_to_f16(self, v):
        return self.raw["f32_to_f16"](float(v))

    def f16_to_f32(self, h):
        return self.raw["f16_to_f32"](int(h))

    def f32_to_bf16(self, v):
        return self.raw["f32_to_bf16"](float(v))

    def w4_awq_quantize(self, w, group):
        w = np.ascontiguousarray(w, np.float32)
        N, K = w.shape
        G = K // group
        qw = np.zeros((N, K // 8), np.uint32)
        sc = np.zeros((N, G), np.uint16)
        qz = np.zeros((N, (G + 7) // 8), np.uint32)
        rc = self.raw["w4_awq_quantize"](w, N, K, group, qw, sc, qz)
        return rc, qw, sc, qz

    def w4_gptq_quantize(self, w, g_idx, G):
        w = np.ascontiguousarray(w, np.float32)
        g_idx = np.ascontiguousarray(g_idx, np.int32)
        N, K = w.shape
        qw = np.zeros((N, K // 8), np.uint32)
        sc = np.zeros((N, G), np.uint16)
        rc = self.raw["w4_gptq_quantize"](w, g_idx, N, K, G, qw, sc)
        return rc, qw, sc

    def w4_dequantize(self, qweight, scales, qzeros, g_idx, N, K, group):
        qweight = np.ascontiguousarray(qweight, np.uint32)
        scales = np.ascontiguousarray(scales, np.uint16)
        qz = None if qzeros is None else np.ascontiguousarray(qzeros, np.uint32)
        gi = None if g_idx is None else np.ascontiguousarray(g_idx, np.int32)
        out = np.zeros((N, K), np.float32)
        rc = self.raw["w4_dequantize"](qweight, scales, _ptr(qz), _ptr(gi), N, K, group, out)
        return rc, out

    def add_bias(self, y, bias):
        """y + bias[n] in fp32 (quantization.py:453-454), on a copy of y."""
        y = np.array(y, np.float32, copy=True, order="C")
        M, N = y.shape
        self.raw["add_bias"](y, np.ascontiguousarray(bias, np.float32), M, N)
        return y

    def _bias(self, rc, y, bias):
        return (rc, y) if bias is None or rc != 0 else (rc, self.add_bias(y, bias))

    def w4a16_linear(self, x_bf16, qweight, scales, qzeros, g_idx, N, K, group, bias=None):
        x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
        M = x_bf16.shape[0]
        qweight = np.ascontiguousarray(qweight, np.uint32)
        scales = np.ascontiguousarray(scales, np.uint16)
        qz = None if qzeros is None else np.ascontiguousarray(qzeros, np.uint32)
        gi = None if g_idx is None else np.ascontiguousarray(g_idx, np.int32)
        y = np.zeros((M, N), np.float32)
        rc = self.raw["w4a16_linear"](x_bf16, qweight, scales, _ptr(qz), _ptr(gi), M, N, K, group, y)
        return self._bias(rc, y, bias)

    def w8_linear(self, x, q, s, bias=None):
        x = np.ascontiguousarray(x, np.float32)
        q = np.ascontiguousarray(q, np.int8)
        s = np.ascontiguousarray(s, np.float32)
        M, K = x.shape
        N = q.shape[0]
        y = np.zeros((M, N), np.float32)
        rc = self.raw["w8_linear"](x, q, s, M, N, K, y)
        return self._bias(rc, y, bias)

    def i8_gemm_i32(self, A, W):
        A = np.ascontiguousarray(A, np.int8)
        W = np.ascontiguousarray(W, np.int8)
        M, K = A.shape
        N = W.shape[0]
        Cm = np.zeros((M, N), np.int32)
        self.raw["i8_gemm_i32"](A, W, Cm, M, N, K)
        return Cm

    def w8a8_epilogue(self, acc, sA, sW, bias=None):
        acc = np.ascontiguousarray(acc, np.int32)
        M, N = acc.shape
        out = np.zeros((M, N), np.float32)
        self.raw["w8a8_epilogue"](acc, np.ascontiguousarray(sA, np.float32),
                                  np.ascontiguousarray(sW, np.float32), M, N, out)
        return out if bias is None else self.add_bias(out, bias)

    def quantize_fp8_e4m3_scaled(self, x):
        x = np.ascontiguousarray(x, np.float32)
        c = np.zeros(x.shape, np.uint8)
        s = C.c_float(0)
        rc = self.raw["quantize_fp8_e4m3_scaled"](x, c, x.size, C.byref(s))
        return rc, c, np.float32(s.value)

    def fp8_gemm(self, A, W, sA, sW, bias=None):
        A = np.ascontiguousarray(A, np.uint8)
        W = np.ascontiguousarray(W, np.uint8)
        M, K = A.shape
        N = W.shape[0]
        out = np.zeros((M, N), np.float32)
        self.raw["fp8_gemm"](A, W, sA, sW, M, N, K, out)
        return out if bias is None else self.add_bias(out, bias)


class _WeightTensor(C.Structure):
    """WeightTensor (include/neural_core/model_zoo/weights.h:39-48)."""
    _fields_ = [("name", C.c_char_p), ("shape", C.POINTER(C.c_int64)), ("ndim", C.c_int),
                ("numel", C.c_size_t), ("dtype", C.c_void_p), ("data", C.c_void_p),
                ("data_size", C.c_size_t), ("owns_data", C.c_int)]


class Reference(_Lib):
    """The reference's kernel/quantization sources and model_zoo/weights.c
    compiled unchanged (build container only)."""

    def __init__(self):
        super().__init__(REF_SO, "SNEPPX_", _COMMON)

    def modelzoo_quantize_int8(self, x):
        """weight_tensor_quantize_int8 (weights.c:225-252) on a float32 vector:
        the tensor's buffers are malloc'd by libc because the function frees
        and replaces them; returns (rc, int8 codes)."""
        libc = C.CDLL(None)
        libc.malloc.restype = C.c_void_p
        libc.malloc.argtypes = [C.c_size_t]
        libc.free.argtypes = [C.c_void_p]
        libc.strdup.restype = C.c_void_p
        libc.strdup.argtypes = [C.c_char_p]
        f = self.lib.weight_tensor_quantize_int8
        f.restype, f.argtypes = C.c_int, [C.POINTER(_WeightTensor)]
        x = np.ascontiguousarray(x, np.float32).ravel()
        t = _WeightTensor()
        t.numel = x.size
        t.data = libc.malloc(max(x.nbytes, 1))
        C.memmove(t.data, x.ctypes.data, x.nbytes)
        t.data_size = x.nbytes
        t.dtype = libc.strdup(b"float32")
        rc = f(C.byref(t))
        q = np.zeros(x.size, np.int8)
        if rc == 0:
            C.memmove(q.ctypes.data, t.data, x.size)
        libc.free(t.data)
        libc.free(t.dtype)
        return rc, q


def reference_available() -> bool:
    return os.path.exists(REF_SO)
