"""Python access to libsneppx_quant.so (the HIP-backed quantized linear path).

Two layers, both thin ctypes bindings over the C-ABI in include/:

* `Library` - the reference's host-pointer quantization API
  (include/sneppx_quantization.h) with numpy in / numpy out, mirroring the
  return tuples of the reference's C functions (rc first, then outputs).
* device entry points (include/sneppx_qlinear.h) taking torch tensors that
  live on the GPU; they launch on torch's current stream unless a stream is
  given.  torch is only the allocator/stream plumbing here.

There is no fallback: if the shared library is missing, `load()` raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

try:  # torch first: its libamdhip64 must be the one the library binds to
    import torch
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsneppx_quant.so")

# SNEPPXDtype ordinals (multidimensional_tensor_engine.h:27-41)
SNEPPX_FLOAT32 = 0
SNEPPX_FLOAT16 = 2
SNEPPX_BFLOAT16 = 3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C")
_sz = C.c_size_t
_vp = C.c_void_p

EXPORTS = {
    # reference surface
    "SNEPPX_quantize_int8_sym": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float)]),
    "SNEPPX_dequantize_int8_sym": (C.c_int, [_i8p, _f32p, _sz, C.c_float]),
    "SNEPPX_quantize_int8_asym": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float), C.POINTER(C.c_int32)]),
    "SNEPPX_dequantize_int8_asym": (C.c_int, [_i8p, _f32p, _sz, C.c_float, C.c_int32]),
    "SNEPPX_quantize_int8_channel": (C.c_int, [_f32p, _i8p, _sz, _sz, _f32p]),
    "SNEPPX_quantize_int4_sym": (C.c_int, [_f32p, _u8p, _sz, C.POINTER(C.c_float)]),
    "SNEPPX_dequantize_int4_sym": (C.c_int, [_u8p, _f32p, _sz, C.c_float]),
    "SNEPPX_float_to_fp8_e4m3": (C.c_uint8, [C.c_float]),
    "SNEPPX_fp8_e4m3_to_float": (C.c_float, [C.c_uint8]),
    "SNEPPX_quantize_fp8_e4m3": (C.c_int, [_f32p, _u8p, _sz]),
    "SNEPPX_dequantize_fp8_e4m3": (C.c_int, [_u8p, _f32p, _sz]),
    "SNEPPX_float_to_fp8_e5m2": (C.c_uint8, [C.c_float]),
    "SNEPPX_fp8_e5m2_to_float": (C.c_float, [C.c_uint8]),
    "SNEPPX_quantize_fp8_e5m2": (C.c_int, [_f32p, _u8p, _sz]),
    "SNEPPX_dequantize_fp8_e5m2": (C.c_int, [_u8p, _f32p, _sz]),
    "SNEPPX_awq_scale_weights": (C.c_int, [_f32p, _sz, _sz, _f32p, _f32p]),
    "SNEPPX_awq_quantize": (C.c_int, [_f32p, _i8p, _vp, _f32p, _sz, _sz, C.c_int]),
    "SNEPPX_gptq_quantize": (C.c_int, [_f32p, _sz, _sz, C.c_int, C.c_int, _i8p, _f32p, _vp, C.c_int]),
    "SNEPPX_gptq_compute_hessian": (C.c_int, [_f32p, _f32p, _sz, _sz]),
    "SNEPPX_gptq_quantize_block": (C.c_int, [_f32p, _f32p, _f32p, C.POINTER(C.c_float),
                                             C.POINTER(C.c_int32), _sz, C.c_int, C.c_int]),
    "SNEPPX_quant_params_create": (C.c_int, [_vp, C.c_int]),
    "SNEPPX_quant_mode_name": (C.c_char_p, [C.c_int]),
    # device entry points
    "SNEPPX_qlinear_last_error": (C.c_char_p, []),
    "SNEPPX_dev_quantize_int8_channel": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_dev_quantize_int8_channel_rounding": (C.c_int, [_vp, _vp, _vp, _sz, _sz, C.c_int, _vp]),
    "SNEPPX_dev_fake_quant": (C.c_int, [_vp, _vp, _sz, C.c_float, C.c_int, _vp]),
    "SNEPPX_dev_quantize_w4_awq": (C.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, C.c_int, _vp]),
    "SNEPPX_dev_quantize_w4_gptq": (C.c_int, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_dev_quantize_fp8_e4m3_scaled": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "SNEPPX_qlinear_w8_gemv": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w4a16": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, C.c_int, _sz, _sz,
                                       _sz, C.c_int, _vp]),
    "SNEPPX_qlinear_w4a16_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, C.c_int, _sz, _sz,
                                               _sz, C.c_int, _vp]),
    "SNEPPX_qlinear_w4_actorder_prepare": (C.c_int, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w4a16_actorder": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, _sz, _sz,
                                                _sz, C.c_int, _vp]),
    "SNEPPX_qlinear_silu_mul": (C.c_int, [_vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w4a16_swiglu": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, C.c_int, _vp]),
    "SNEPPX_qlinear_w4a16_mlp": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_int, _sz, _sz,
                                           _sz, _sz, C.c_int, _vp]),
    "SNEPPX_qlinear_silu_mul_quant_int8": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_dev_quantize_int8_channel_bf16": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w8a8_i8": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_i8_gemm_i32": (C.c_int, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w8a8_fp8": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    # quantized weights on disk + model-zoo int8 (include/sneppx_qstore.h)
    "SNEPPX_qstore_open": (_vp, [C.c_char_p]),
    "SNEPPX_qstore_close": (None, [_vp]),
    "SNEPPX_qstore_count": (_sz, [_vp]),
    "SNEPPX_qstore_name": (C.c_char_p, [_vp, _sz]),
    "SNEPPX_qstore_info": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int), C.POINTER(_sz),
                                     C.POINTER(_sz), C.POINTER(_sz)]),
    "SNEPPX_qstore_data": (_vp, [_vp, C.c_char_p, C.POINTER(_sz)]),
    "SNEPPX_qstore_read_device": (C.c_int, [_vp, C.c_char_p, _vp, _sz, _vp]),
    "SNEPPX_qstore_metadata": (C.c_char_p, [_vp, C.c_char_p]),
    "SNEPPX_qstore_writer_open": (_vp, [C.c_char_p]),
    "SNEPPX_qstore_writer_add_host": (C.c_int, [_vp, C.c_char_p, C.c_int, C.POINTER(_sz), _sz, _vp]),
    "SNEPPX_qstore_writer_add_device": (C.c_int, [_vp, C.c_char_p, C.c_int, C.POINTER(_sz), _sz, _vp,
                                                  _vp]),
    "SNEPPX_qstore_writer_set_metadata": (C.c_int, [_vp, C.c_char_p, C.c_char_p]),
    "SNEPPX_qstore_writer_close": (C.c_int, [_vp]),
    "SNEPPX_qstore_save_w4": (C.c_int, [_vp, C.c_char_p, _vp, _vp, _vp, _vp, _sz, _sz, C.c_int, _sz,
                                        _vp]),
    "SNEPPX_qstore_query_w4": (C.c_int, [_vp, C.c_char_p, C.POINTER(_sz), C.POINTER(_sz),
                                         C.POINTER(_sz), C.POINTER(C.c_int), C.POINTER(C.c_int),
                                         C.POINTER(C.c_int)]),
    "SNEPPX_qstore_load_w4": (C.c_int, [_vp, C.c_char_p, _vp, _vp, _vp, _vp, _vp]),
    "SNEPPX_qstore_save_w8": (C.c_int, [_vp, C.c_char_p, _vp, _vp, _sz, _sz, _vp]),
    "SNEPPX_qstore_query_w8": (C.c_int, [_vp, C.c_char_p, C.POINTER(_sz), C.POINTER(_sz)]),
    "SNEPPX_qstore_load_w8": (C.c_int, [_vp, C.c_char_p, _vp, _vp, _vp]),
    "SNEPPX_quantize_int8_modelzoo": (C.c_int, [_f32p, _i8p, _sz, C.POINTER(C.c_float)]),
    "SNEPPX_dev_quantize_int8_modelzoo": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    # quantized layers for the reference's linear call sites (include/sneppx_qlayer.h)
    "SNEPPX_qlayer_create_kn": (_vp, [_f32p, _sz, _sz, C.c_int, C.c_int, _vp]),
    "SNEPPX_qlayer_create_kn_device": (_vp, [_vp, _sz, _sz, C.c_int, C.c_int, _vp]),
    "SNEPPX_qlayer_load": (_vp, [_vp, C.c_char_p, _vp]),
    "SNEPPX_qlayer_save": (C.c_int, [_vp, _vp, C.c_char_p, _vp]),
    "SNEPPX_qlayer_destroy": (None, [_vp]),
    "SNEPPX_qlayer_set_bias": (C.c_int, [_vp, _f32p, _vp]),
    "SNEPPX_qlayer_set_bias_device": (C.c_int, [_vp, _vp, _vp]),
    "SNEPPX_qlayer_in_features": (_sz, [_vp]),
    "SNEPPX_qlayer_out_features": (_sz, [_vp]),
    "SNEPPX_qlayer_format": (C.c_int, [_vp]),
    "SNEPPX_qlayer_forward_f32": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "SNEPPX_qlayer_forward_bf16": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "SNEPPX_qlayer_matmul_host": (C.c_int, [_vp, _f32p, _f32p, _sz]),
    # MX formats (include/sneppx_mx.h)
    "SNEPPX_mx_bits": (C.c_int, [C.c_int]),
    "SNEPPX_mx_default_block": (C.c_int, [C.c_int]),
    "SNEPPX_mx_packed_bytes": (_sz, [C.c_int, _sz, _sz, C.c_int]),
    "SNEPPX_mx_scale_count": (_sz, [C.c_int, _sz, _sz, C.c_int]),
    "SNEPPX_dev_quantize_mx": (C.c_int, [_vp, _vp, _vp, _sz, _sz, C.c_int, C.c_int, _vp]),
    "SNEPPX_dev_dequantize_mx": (C.c_int, [_vp, _vp, _vp, _sz, _sz, C.c_int, C.c_int, _vp]),
    "SNEPPX_qlinear_mxfp4_gemm": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_mx_gemm": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_mx_gemm_mfma": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_mx_gemm_bs": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, _vp, C.c_int, _sz, _sz, _sz,
                                            _vp]),
    "SNEPPX_mx_to_mfma": (C.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, C.c_int, _vp, _vp]),
    # thin HIP ABI
    "snx_hip_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "snx_hip_event_create": (C.c_int, [C.POINTER(_vp)]),
    "snx_hip_event_destroy": (C.c_int, [_vp]),
    "snx_hip_event_record": (C.c_int, [_vp, _vp]),
    "snx_hip_event_sync": (C.c_int, [_vp]),
    "snx_hip_event_elapsed_ms": (C.c_int, [C.POINTER(C.c_float), _vp, _vp]),
    "snx_hip_stream_sync": (C.c_int, [_vp]),
    "snx_hip_device_info": (C.c_int, [C.c_char_p, _sz, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "SNEPPX_qlinear_release_workspaces": (C.c_int, [_vp]),
    "SNEPPX_qlinear_w8a8_i8_dyn": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "SNEPPX_qlinear_w8a8_fp8_dyn": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "snx_hip_stream_begin_capture": (C.c_int, [_vp]),
    "snx_hip_stream_end_capture": (C.c_int, [_vp, C.POINTER(_vp)]),
    "snx_hip_graph_launch": (C.c_int, [_vp, _vp]),
    "snx_hip_graph_destroy": (C.c_int, [_vp]),
    "snx_workspace_count": (C.c_long, []),
}


class QuantParams(C.Structure):
    """SNEPPXQuantParams (quantization.h:42-48)."""
    _fields_ = [("scale", C.c_float), ("zero_point", C.c_int32), ("qmin", C.c_float),
                ("qmax", C.c_float), ("scale_max", C.c_float)]


class SneppxError(RuntimeError):
    pass


def _ptr(t):
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def _bias_ptr(bias, n, like):
    """Pointer of an optional bias after checking what the kernels read: fp32,
    contiguous, on the output's device, exactly n elements (2F for the stacked
    gate/up of the SwiGLU form).  Anything else raises ValueError rather than
    letting a kernel read past the end or reinterpret bf16 bits."""
    if bias is None:
        return None
    if not isinstance(bias, torch.Tensor):
        raise ValueError("bias must be a torch tensor on the device (fp32 [N])")
    if bias.dtype != torch.float32:
        raise ValueError(f"bias must be float32, got {bias.dtype}")
    if not bias.is_contiguous():
        raise ValueError("bias must be contiguous")
    if bias.device != like.device:
        raise ValueError(f"bias is on {bias.device}, the output on {like.device}")
    if bias.numel() != n:
        raise ValueError(f"bias has {bias.numel()} elements, the linear needs {n}")
    return C.c_void_p(bias.data_ptr())


class Library:
    """ctypes view of libsneppx_quant.so."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise SneppxError(f"{path} is not built; run `make -C sneppx-alg_amd` "
                              "(or __graft_entry__.build()) - there is no CPU fallback")
        self.path = path
        self.lib = C.CDLL(path)
        self.fn = {}
        for name, (res, args) in EXPORTS.items():
            f = getattr(self.lib, name)
            f.restype, f.argtypes = res, args
            self.fn[name] = f

    def last_error(self) -> str:
        return self.fn["SNEPPX_qlinear_last_error"]().decode()

    def check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise SneppxError(f"{what} failed: {self.last_error()}")

    # ---------------- reference host API (numpy) -------------------------
    def quantize_int8_sym(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        s = C.c_float(0)
        rc = self.fn["SNEPPX_quantize_int8_sym"](x, q, x.size, C.byref(s))
        return rc, q, np.float32(s.value)

    def dequantize_int8_sym(self, q, scale):
        q = np.ascontiguousarray(q, np.int8).ravel()
        y = np.zeros(q.size, np.float32)
        return self.fn["SNEPPX_dequantize_int8_sym"](q, y, q.size, scale), y

    def quantize_int8_asym(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        s, z = C.c_float(0), C.c_int32(0)
        rc = self.fn["SNEPPX_quantize_int8_asym"](x, q, x.size, C.byref(s), C.byref(z))
        return rc, q, np.float32(s.value), int(z.value)

    def dequantize_int8_asym(self, q, scale, zp):
        q = np.ascontiguousarray(q, np.int8).ravel()
        y = np.zeros(q.size, np.float32)
        return self.fn["SNEPPX_dequantize_int8_asym"](q, y, q.size, scale, zp), y

    def quantize_int8_channel(self, x):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        q = np.zeros((rows, cols), np.int8)
        s = np.zeros(rows, np.float32)
        rc = self.fn["SNEPPX_quantize_int8_channel"](x, q, rows, cols, s)
        return rc, q, s

    def quantize_int4_sym(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        p = np.zeros((x.size + 1) // 2, np.uint8)
        s = C.c_float(0)
        rc = self.fn["SNEPPX_quantize_int4_sym"](x, p, x.size, C.byref(s))
        return rc, p, np.float32(s.value)

    def dequantize_int4_sym(self, packed, n, scale):
        packed = np.ascontiguousarray(packed, np.uint8)
        y = np.zeros(n, np.float32)
        return self.fn["SNEPPX_dequantize_int4_sym"](packed, y, n, scale), y

    def quantize_fp8(self, x, fmt="e4m3"):
        x = np.ascontiguousarray(x, np.float32).ravel()
        c = np.zeros(x.size, np.uint8)
        return self.fn[f"SNEPPX_quantize_fp8_{fmt}"](x, c, x.size), c

    def dequantize_fp8(self, c, fmt="e4m3"):
        c = np.ascontiguousarray(c, np.uint8).ravel()
        y = np.zeros(c.size, np.float32)
        return self.fn[f"SNEPPX_dequantize_fp8_{fmt}"](c, y, c.size), y

    def awq_scale_weights(self, w, act_scales):
        w = np.array(w, np.float32, order="C", copy=True)
        rows, cols = w.shape
        s = np.zeros((rows, cols), np.float32)
        a = np.ascontiguousarray(act_scales, np.float32)
        rc = self.fn["SNEPPX_awq_scale_weights"](w, rows, cols, a, s)
        return rc, w, s

    def awq_quantize(self, w, group_size, act_scales=None):
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = w.shape
        g = group_size if group_size > 0 else 128
        q = np.zeros((rows, cols), np.int8)
        s = np.zeros((rows, (cols + g - 1) // g), np.float32)
        a = None if act_scales is None else np.ascontiguousarray(act_scales, np.float32)
        rc = self.fn["SNEPPX_awq_quantize"](w, q, None if a is None else a.ctypes.data_as(_vp),
                                            s, rows, cols, group_size)
        return rc, q, s

    def gptq_compute_hessian(self, act):
        act = np.ascontiguousarray(act, np.float32)
        n, dim = act.shape
        h = np.zeros((dim, dim), np.float32)
        return self.fn["SNEPPX_gptq_compute_hessian"](h, act, n, dim), h

    def gptq_quantize_block(self, w, h_inv, bits, sym):
        w = np.array(w, np.float32, order="C", copy=True)
        h = np.array(h_inv, np.float32, order="C", copy=True)
        qw = np.zeros(w.size, np.float32)
        s, z = C.c_float(0), C.c_int32(-7)
        rc = self.fn["SNEPPX_gptq_quantize_block"](w, h, qw, C.byref(s), C.byref(z), w.size, bits, sym)
        return rc, w, qw, np.float32(s.value), int(z.value)

    def gptq_quantize(self, w, group_size, bits, sym, with_zeros=True):
        w = np.array(w, np.float32, order="C", copy=True)
        rows, cols = w.shape
        g = group_size if group_size > 0 else 128
        ng = (cols + g - 1) // g
        q = np.full((rows, cols), 0x55, np.int8)
        s = np.zeros((rows, ng), np.float32)
        z = np.full((rows, ng), -7, np.int32) if with_zeros else None
        rc = self.fn["SNEPPX_gptq_quantize"](w, rows, cols, group_size, bits, q, s,
                                             None if z is None else z.ctypes.data_as(_vp), sym)
        return rc, w, q, s, z

    def quant_params_create(self, mode):
        p = QuantParams()
        rc = self.fn["SNEPPX_quant_params_create"](C.cast(C.pointer(p), _vp), mode)
        return rc, (p.scale, p.zero_point, p.qmin, p.qmax, p.scale_max)

    def quant_mode_name(self, mode):
        return self.fn["SNEPPX_quant_mode_name"](mode).decode()

    # ---------------- device entry points (torch tensors on the GPU) -------
    @staticmethod
    def _stream(stream):
        if stream is not None:
            return C.c_void_p(stream)
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def dev_quantize_int8_channel(self, w, q, scales, stream=None, half_even=False):
        rows, cols = w.shape
        if half_even:
            self.check(self.fn["SNEPPX_dev_quantize_int8_channel_rounding"](
                _ptr(w), _ptr(q), _ptr(scales), rows, cols, 1, self._stream(stream)),
                "dev_quantize_int8_channel_rounding")
        else:
            self.check(self.fn["SNEPPX_dev_quantize_int8_channel"](
                _ptr(w), _ptr(q), _ptr(scales), rows, cols, self._stream(stream)), "dev_quantize_int8_channel")

    def dev_fake_quant(self, x, out, scale, bits, stream=None):
        self.check(self.fn["SNEPPX_dev_fake_quant"](
            _ptr(x), _ptr(out), x.numel(), scale, bits, self._stream(stream)), "dev_fake_quant")

    def dev_quantize_w4_awq(self, w, qweight, scales, qzeros, group, stream=None):
        N, K = w.shape
        self.check(self.fn["SNEPPX_dev_quantize_w4_awq"](
            _ptr(w), _ptr(qweight), _ptr(scales), _ptr(qzeros), N, K, group, self._stream(stream)),
            "dev_quantize_w4_awq")

    def dev_quantize_w4_gptq(self, w, g_idx, G, qweight, scales, stream=None):
        N, K = w.shape
        self.check(self.fn["SNEPPX_dev_quantize_w4_gptq"](
            _ptr(w), _ptr(g_idx), G, _ptr(qweight), _ptr(scales), N, K, self._stream(stream)),
            "dev_quantize_w4_gptq")

    def dev_quantize_fp8_e4m3_scaled(self, x, out, scale, stream=None):
        self.check(self.fn["SNEPPX_dev_quantize_fp8_e4m3_scaled"](
            _ptr(x), _ptr(out), _ptr(scale), x.numel(), self._stream(stream)), "dev_quantize_fp8_e4m3_scaled")

    def qlinear_w8_gemv(self, x, qweight, scales, y, stream=None, bias=None):
        M, K = x.shape
        N = qweight.shape[0]
        self.check(self.fn["SNEPPX_qlinear_w8_gemv"](
            _ptr(x), _ptr(qweight), _ptr(scales), _bias_ptr(bias, N, y), _ptr(y), M, N, K, self._stream(stream)),
            "qlinear_w8_gemv")

    def qlinear_w4a16(self, x, qweight, scales, qzeros, g_idx, G, y, group, stream=None, bias=None):
        M, K = x.shape
        N = qweight.shape[0]
        ydt = SNEPPX_FLOAT32 if y.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_w4a16"](
            _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx), G, _bias_ptr(bias, N, y), _ptr(y),
            ydt, M, N, K, group, self._stream(stream)), "qlinear_w4a16")

    def qlinear_w4a16_noalloc(self, x, qweight, scales, qzeros, g_idx, G, y, group, stream=None,
                              bias=None):
        """SNEPPX_qlinear_w4a16_noalloc: as qlinear_w4a16, scratch from the
        library's static device array instead of a workspace."""
        M, K = x.shape
        N = qweight.shape[0]
        ydt = SNEPPX_FLOAT32 if y.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_w4a16_noalloc"](
            _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx), G, _bias_ptr(bias, N, y), _ptr(y),
            ydt, M, N, K, group, self._stream(stream)), "qlinear_w4a16_noalloc")

    def qlinear_w4_actorder_prepare(self, qweight, g_idx, G, qweight_sorted, perm, stream=None):
        N, K8 = qweight.shape
        self.check(self.fn["SNEPPX_qlinear_w4_actorder_prepare"](
            _ptr(qweight), _ptr(g_idx), G, _ptr(qweight_sorted), _ptr(perm), N, K8 * 8,
            self._stream(stream)), "qlinear_w4_actorder_prepare")

    def qlinear_w4a16_actorder(self, x, qweight_sorted, scales, qzeros, perm, y, group, stream=None,
                               bias=None):
        M, K = x.shape
        N = qweight_sorted.shape[0]
        ydt = SNEPPX_FLOAT32 if y.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_w4a16_actorder"](
            _ptr(x), _ptr(qweight_sorted), _ptr(scales), _ptr(qzeros), _ptr(perm), _bias_ptr(bias, N, y), _ptr(y),
            ydt, M, N, K, group, self._stream(stream)), "qlinear_w4a16_actorder")

    def qlinear_w4a16_swiglu(self, x, qweight, scales, qzeros, out, group, stream=None, bias=None):
        """out [M][F] = bf16(silu(x . Wg^T) * (x . Wu^T)), qweight the stacked [2F][K/8]."""
        M, K = x.shape
        F = out.shape[1]
        self.check(self.fn["SNEPPX_qlinear_w4a16_swiglu"](
            _ptr(x), _ptr(qweight), _ptr(scales), _ptr(qzeros), _bias_ptr(bias, 2 * F, out), _ptr(out), M, F, K, group,
            self._stream(stream)), "qlinear_w4a16_swiglu")

    def qlinear_w4a16_mlp(self, x, gate_up, down, y, group, stream=None, gu_bias=None, dn_bias=None):
        """y [M][N] = down(silu(x . Wg^T) * (x . Wu^T)): gate_up = (qweight [2F][H/8],
        scales, qzeros) of the stacked gate/up projection, down = (qweight [N][F/8],
        scales, qzeros)."""
        M, H = x.shape
        gq, gs, gz = gate_up
        dq, ds, dz = down
        F = gq.shape[0] // 2
        N = dq.shape[0]
        ydt = SNEPPX_FLOAT32 if y.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_w4a16_mlp"](
            _ptr(x), _ptr(gq), _ptr(gs), _ptr(gz), _bias_ptr(gu_bias, 2 * F, y), _ptr(dq), _ptr(ds), _ptr(dz),
            _bias_ptr(dn_bias, N, y), _ptr(y), ydt, M, H, F, N, group, self._stream(stream)), "qlinear_w4a16_mlp")

    def qlinear_silu_mul(self, gate_up, out, stream=None):
        T, F2 = gate_up.shape
        self.check(self.fn["SNEPPX_qlinear_silu_mul"](
            _ptr(gate_up), _ptr(out), T, F2 // 2, self._stream(stream)), "qlinear_silu_mul")

    def qlinear_silu_mul_quant_int8(self, gate_up, q, scales, stream=None):
        T, F2 = gate_up.shape
        self.check(self.fn["SNEPPX_qlinear_silu_mul_quant_int8"](
            _ptr(gate_up), _ptr(q), _ptr(scales), T, F2 // 2, self._stream(stream)),
            "qlinear_silu_mul_quant_int8")

    def dev_quantize_int8_channel_bf16(self, x, q, scales, stream=None):
        rows, cols = x.shape
        self.check(self.fn["SNEPPX_dev_quantize_int8_channel_bf16"](
            _ptr(x), _ptr(q), _ptr(scales), rows, cols, self._stream(stream)),
            "dev_quantize_int8_channel_bf16")

    def qlinear_w8a8_i8(self, A, sA, W, sW, out, stream=None, bias=None):
        M, K = A.shape
        N = W.shape[0]
        self.check(self.fn["SNEPPX_qlinear_w8a8_i8"](
            _ptr(A), _ptr(sA), _ptr(W), _ptr(sW), _bias_ptr(bias, N, out), _ptr(out), M, N, K, self._stream(stream)),
            "qlinear_w8a8_i8")

    def qlinear_w8a8_dyn(self, A, W, sW, out, fp8=False, stream=None, bias=None):
        """C4 from bf16 activations: A quantized inside the call (int8 per
        token, or fp8 per tensor), then the W8A8 GEMM."""
        M, K = A.shape
        N = W.shape[0]
        name = "SNEPPX_qlinear_w8a8_fp8_dyn" if fp8 else "SNEPPX_qlinear_w8a8_i8_dyn"
        self.check(self.fn[name](_ptr(A), _ptr(W), _ptr(sW), _bias_ptr(bias, N, out), _ptr(out), M, N, K,
                                 self._stream(stream)), name[7:])

    def qlinear_i8_gemm_i32(self, A, W, Cm, stream=None):
        M, K = A.shape
        N = W.shape[0]
        self.check(self.fn["SNEPPX_qlinear_i8_gemm_i32"](
            _ptr(A), _ptr(W), _ptr(Cm), M, N, K, self._stream(stream)), "qlinear_i8_gemm_i32")

    def qlinear_w8a8_fp8(self, A, sA, W, sW, out, stream=None, bias=None):
        M, K = A.shape
        N = W.shape[0]
        self.check(self.fn["SNEPPX_qlinear_w8a8_fp8"](
            _ptr(A), _ptr(sA), _ptr(W), _ptr(sW), _bias_ptr(bias, N, out), _ptr(out), M, N, K, self._stream(stream)),
            "qlinear_w8a8_fp8")

    # ---------------- model-zoo int8 (weights.c:225-252) -------------------
    def quantize_int8_modelzoo(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        q = np.zeros(x.size, np.int8)
        m = C.c_float(0)
        rc = self.fn["SNEPPX_quantize_int8_modelzoo"](x, q, x.size, C.byref(m))
        return rc, q, np.float32(m.value)

    def dev_quantize_int8_modelzoo(self, x, q, mult, stream=None):
        self.check(self.fn["SNEPPX_dev_quantize_int8_modelzoo"](
            _ptr(x), _ptr(q), _ptr(mult), x.numel(), self._stream(stream)), "dev_quantize_int8_modelzoo")

    # ---------------- quantized weights on disk (safetensors) --------------
    def qstore_open(self, path):
        h = self.fn["SNEPPX_qstore_open"](os.fsencode(path))
        if not h:
            raise SneppxError(f"qstore_open failed: {self.last_error()}")
        return QStore(self, h)

    def qstore_writer(self, path):
        h = self.fn["SNEPPX_qstore_writer_open"](os.fsencode(path))
        if not h:
            raise SneppxError(f"qstore_writer_open failed: {self.last_error()}")
        return QStoreWriter(self, h)

    # ---------------- quantized layers (reference [K, N] weights) ------------
    def qlayer_create_kn(self, w_kn, fmt="w4", group=128, stream=None):
        """w_kn: numpy fp32 [K, N] (host) or a torch fp32 [K, N] device tensor."""
        code = {"w8": 0, "w4": 1}[fmt]
        if isinstance(w_kn, np.ndarray):
            w = np.ascontiguousarray(w_kn, np.float32)
            K, N = w.shape
            h = self.fn["SNEPPX_qlayer_create_kn"](w, K, N, code, group, self._stream(stream))
        else:
            K, N = w_kn.shape
            h = self.fn["SNEPPX_qlayer_create_kn_device"](_ptr(w_kn), K, N, code, group, self._stream(stream))
        if not h:
            raise SneppxError(f"qlayer_create_kn failed: {self.last_error()}")
        return QLayer(self, h)

    def qlayer_load(self, store, prefix, stream=None):
        h = self.fn["SNEPPX_qlayer_load"](store.h, prefix.encode(), self._stream(stream))
        if not h:
            raise SneppxError(f"qlayer_load failed: {self.last_error()}")
        return QLayer(self, h)

    # ---------------- MX formats (mx_formats.py semantics) ------------------
    def _mx_block(self, fmt, block_size):
        # the reference's `block_size or spec.block_size`, per tensor when <= 0
        if block_size is None:
            return 0
        return block_size if block_size > 0 else -1

    def dev_quantize_mx(self, x, fmt, block_size=None, stream=None):
        """x: float32 device tensor [rows, cols] (or [n]); returns (packed uint8,
        scales int8) device tensors laid out as quantize_mx returns them."""
        code = MX_FORMATS.index(fmt)
        x2 = x if x.dim() == 2 else x.reshape(1, -1)
        rows, cols = x2.shape
        bs = self._mx_block(fmt, block_size)
        nbytes = self.fn["SNEPPX_mx_packed_bytes"](code, rows, cols, bs)
        nsc = self.fn["SNEPPX_mx_scale_count"](code, rows, cols, bs)
        if nbytes == 0 or nsc == 0:
            raise SneppxError(f"dev_quantize_mx: bad block size {block_size}")
        packed = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        scales = torch.empty(nsc, dtype=torch.int8, device=x.device)
        self.check(self.fn["SNEPPX_dev_quantize_mx"](
            _ptr(x2), _ptr(packed), _ptr(scales), rows, cols, code, bs, self._stream(stream)),
            "dev_quantize_mx")
        if nsc > 1 or self.fn["SNEPPX_mx_default_block"](code) > 0 and bs >= 0:
            scales = scales.reshape(rows, -1)
        return packed, scales

    def dev_dequantize_mx(self, packed, scales, shape, fmt, block_size=None, stream=None):
        code = MX_FORMATS.index(fmt)
        rows, cols = (1, shape[0]) if len(shape) == 1 else shape
        y = torch.empty((rows, cols), dtype=torch.float32, device=packed.device)
        self.check(self.fn["SNEPPX_dev_dequantize_mx"](
            _ptr(packed), _ptr(scales), _ptr(y), rows, cols, code, self._mx_block(fmt, block_size),
            self._stream(stream)), "dev_dequantize_mx")
        return y.reshape(shape)

    def qlinear_mxfp4_gemm(self, A, sA, W, sW, out, M, N, K, stream=None):
        ydt = SNEPPX_FLOAT32 if out.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_mxfp4_gemm"](
            _ptr(A), _ptr(sA), _ptr(W), _ptr(sW), _ptr(out), ydt, M, N, K, self._stream(stream)),
            "qlinear_mxfp4_gemm")

    def qlinear_mx_gemm(self, A, sA, W, sW, fmt, out, M, N, K, stream=None, mfma_form=False):
        """out = A W^T for block-32 MX operands of format `fmt` (FP8 / FP6 / FP4);
        mfma_form: operands already converted by mx_to_mfma."""
        ydt = SNEPPX_FLOAT32 if out.dtype == torch.float32 else SNEPPX_BFLOAT16
        name = "SNEPPX_qlinear_mx_gemm_mfma" if mfma_form else "SNEPPX_qlinear_mx_gemm"
        self.check(self.fn[name](
            _ptr(A), _ptr(sA), _ptr(W), _ptr(sW), MX_FORMATS.index(fmt), _ptr(out), ydt, M, N, K,
            self._stream(stream)), name[7:])

    def qlinear_mx_gemm_bs(self, A, sA, W, sW, fmt, out, M, N, K, block_size=None, stream=None):
        """out = A W^T for MX operands quantized with `block_size` (the rule of
        dev_quantize_mx: None = the format's default, <= 0 per tensor)."""
        ydt = SNEPPX_FLOAT32 if out.dtype == torch.float32 else SNEPPX_BFLOAT16
        self.check(self.fn["SNEPPX_qlinear_mx_gemm_bs"](
            _ptr(A), _ptr(sA), _ptr(W), _ptr(sW), MX_FORMATS.index(fmt), self._mx_block(fmt, block_size),
            _ptr(out), ydt, M, N, K, self._stream(stream)), "qlinear_mx_gemm_bs")

    def mx_to_mfma(self, packed, scales, rows, cols, fmt, stream=None):
        """(packed, scales, rounded) in the matrix cores' encoding; rounded is an
        int32 device counter of the elements that rounded half to even."""
        out_p, out_s = torch.empty_like(packed), torch.empty_like(scales)
        rounded = torch.zeros(1, dtype=torch.int32, device=packed.device)
        self.check(self.fn["SNEPPX_mx_to_mfma"](
            _ptr(packed), _ptr(scales), _ptr(out_p), _ptr(out_s), rows, cols, MX_FORMATS.index(fmt),
            _ptr(rounded), self._stream(stream)), "mx_to_mfma")
        return out_p, out_s, rounded

    # ---------------- HIP events on an explicit stream ----------------------
    def event(self):
        e = C.c_void_p()
        self.check(self.fn["snx_hip_event_create"](C.byref(e)), "event_create")
        return e

    def record(self, ev, stream=None):
        self.check(self.fn["snx_hip_event_record"](ev, self._stream(stream)), "event_record")

    def capture(self, fn, stream=None):
        """A HIP graph of everything fn() issues on `stream` (an executable
        graph handle; replay with graph_launch, free with graph_destroy)."""
        st = self._stream(stream)
        self.check(self.fn["snx_hip_stream_begin_capture"](st), "stream_begin_capture")
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = self.fn["snx_hip_stream_end_capture"](st, C.byref(g))
        self.check(rc, "stream_end_capture")
        return g

    def graph_launch(self, g, stream=None):
        self.check(self.fn["snx_hip_graph_launch"](g, self._stream(stream)), "graph_launch")

    def graph_destroy(self, g):
        self.check(self.fn["snx_hip_graph_destroy"](g), "graph_destroy")

    def elapsed_ms(self, a, b):
        self.check(self.fn["snx_hip_event_sync"](b), "event_sync")
        ms = C.c_float(0)
        self.check(self.fn["snx_hip_event_elapsed_ms"](C.byref(ms), a, b), "event_elapsed")
        return ms.value

    def device_info(self):
        buf = C.create_string_buffer(128)
        cu, clk = C.c_int(0), C.c_int(0)
        self.check(self.fn["snx_hip_device_info"](buf, 128, C.byref(cu), C.byref(clk)), "device_info")
        return buf.value.decode(), cu.value, clk.value


# SNEPPXMXFormat order (include/sneppx_mx.h = MX_FORMATS of mx_formats.py)
MX_FORMATS = ["mxfp8_e4m3", "mxfp8_e5m2", "mxfp6_e3m2", "mxfp6_e2m3", "mxfp4_e2m1", "nvfp4_e2m1"]

# dtype codes of include/sneppx_qstore.h (= the reference's SNEPPXSafetensorsDType)
QST_DTYPES = ["F32", "F16", "F64", "I64", "I32", "I16", "I8", "U8", "BOOL", "BF16", "F8_E5M2",
              "F8_E4M3FN"]
QST_NUMPY = {"F32": np.float32, "F16": np.float16, "F64": np.float64, "I64": np.int64,
             "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_,
             "BF16": np.uint16, "F8_E5M2": np.uint8, "F8_E4M3FN": np.uint8}


def _shape_arg(shape):
    return (_sz * max(len(shape), 1))(*shape), len(shape)


class QStore:
    """A safetensors file opened by SNEPPX_qstore_open (read-only mapping)."""

    def __init__(self, lib, handle):
        self.L, self.h = lib, C.c_void_p(handle)

    def close(self):
        if self.h:
            self.L.fn["SNEPPX_qstore_close"](self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self):
        n = self.L.fn["SNEPPX_qstore_count"](self.h)
        return [self.L.fn["SNEPPX_qstore_name"](self.h, i).decode() for i in range(n)]

    def info(self, name):
        dt, nd, nb = C.c_int(0), _sz(0), _sz(0)
        shape = (_sz * 8)()
        if self.L.fn["SNEPPX_qstore_info"](self.h, name.encode(), C.byref(dt), shape, C.byref(nd),
                                           C.byref(nb)):
            return None
        return dt.value, tuple(shape[i] for i in range(nd.value)), nb.value

    def host(self, name):
        """Copy of a tensor's bytes as a numpy array of its dtype and shape."""
        inf = self.info(name)
        if inf is None:
            raise KeyError(name)
        dt, shape, nb = inf
        n = _sz(0)
        p = self.L.fn["SNEPPX_qstore_data"](self.h, name.encode(), C.byref(n))
        raw = np.frombuffer(C.string_at(p, n.value), np.uint8) if n.value else np.zeros(0, np.uint8)
        npdt = QST_NUMPY[QST_DTYPES[dt]] if 0 <= dt < len(QST_DTYPES) else np.uint8
        return raw.view(npdt).reshape(shape) if dt >= 0 else raw

    def metadata(self, key):
        v = self.L.fn["SNEPPX_qstore_metadata"](self.h, key.encode())
        return None if v is None else v.decode()

    def read_device(self, name, t, stream=None):
        self.L.check(self.L.fn["SNEPPX_qstore_read_device"](
            self.h, name.encode(), _ptr(t), t.numel() * t.element_size(), self.L._stream(stream)),
            "qstore_read_device")

    def query_w4(self, prefix):
        N, K, G = _sz(0), _sz(0), _sz(0)
        group, hz, hg = C.c_int(0), C.c_int(0), C.c_int(0)
        self.L.check(self.L.fn["SNEPPX_qstore_query_w4"](
            self.h, prefix.encode(), C.byref(N), C.byref(K), C.byref(G), C.byref(group),
            C.byref(hz), C.byref(hg)), "qstore_query_w4")
        return N.value, K.value, G.value, group.value, bool(hz.value), bool(hg.value)

    def load_w4(self, prefix, qweight, scales, qzeros=None, g_idx=None, stream=None):
        self.L.check(self.L.fn["SNEPPX_qstore_load_w4"](
            self.h, prefix.encode(), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx),
            self.L._stream(stream)), "qstore_load_w4")

    def query_w8(self, prefix):
        N, K = _sz(0), _sz(0)
        self.L.check(self.L.fn["SNEPPX_qstore_query_w8"](self.h, prefix.encode(), C.byref(N), C.byref(K)),
                     "qstore_query_w8")
        return N.value, K.value

    def load_w8(self, prefix, q, scales, stream=None):
        self.L.check(self.L.fn["SNEPPX_qstore_load_w8"](
            self.h, prefix.encode(), _ptr(q), _ptr(scales), self.L._stream(stream)), "qstore_load_w8")


class QStoreWriter:
    """Accumulates tensors and metadata; close() writes the file."""

    def __init__(self, lib, handle):
        self.L, self.h = lib, C.c_void_p(handle)

    def add_host(self, name, dtype, arr):
        arr = np.array(arr, order="C", copy=True)   # keeps 0-d arrays 0-d
        shape, nd = _shape_arg(arr.shape)
        self.L.check(self.L.fn["SNEPPX_qstore_writer_add_host"](
            self.h, name.encode(), QST_DTYPES.index(dtype), shape, nd, arr.ctypes.data_as(_vp)),
            "qstore_writer_add_host")

    def add_device(self, name, dtype, t, stream=None):
        shape, nd = _shape_arg(tuple(t.shape))
        self.L.check(self.L.fn["SNEPPX_qstore_writer_add_device"](
            self.h, name.encode(), QST_DTYPES.index(dtype), shape, nd, _ptr(t), self.L._stream(stream)),
            "qstore_writer_add_device")

    def set_metadata(self, key, value):
        self.L.check(self.L.fn["SNEPPX_qstore_writer_set_metadata"](self.h, key.encode(), value.encode()),
                     "qstore_writer_set_metadata")

    def save_w4(self, prefix, qweight, scales, qzeros, g_idx, N, K, group, G, stream=None):
        self.L.check(self.L.fn["SNEPPX_qstore_save_w4"](
            self.h, prefix.encode(), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(g_idx), N, K,
            group, G, self.L._stream(stream)), "qstore_save_w4")

    def save_w8(self, prefix, q, scales, stream=None):
        N, K = q.shape
        self.L.check(self.L.fn["SNEPPX_qstore_save_w8"](
            self.h, prefix.encode(), _ptr(q), _ptr(scales), N, K, self.L._stream(stream)), "qstore_save_w8")

    def close(self):
        h, self.h = self.h, None
        if h:
            self.L.check(self.L.fn["SNEPPX_qstore_writer_close"](h), "qstore_writer_close")


class QLayer:
    """SNEPPXQLayer: y = x . W for a reference-layout weight W [K, N]."""

    def __init__(self, lib, handle):
        self.L, self.h = lib, C.c_void_p(handle)
        self.K = lib.fn["SNEPPX_qlayer_in_features"](self.h)
        self.N = lib.fn["SNEPPX_qlayer_out_features"](self.h)
        self.format = ["w8", "w4"][lib.fn["SNEPPX_qlayer_format"](self.h)]

    def destroy(self):
        if self.h:
            self.L.fn["SNEPPX_qlayer_destroy"](self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def forward_f32(self, x, y, stream=None):
        M = x.shape[0]
        self.L.check(self.L.fn["SNEPPX_qlayer_forward_f32"](self.h, _ptr(x), _ptr(y), M,
                                                            self.L._stream(stream)), "qlayer_forward_f32")

    def forward_bf16(self, x, y, stream=None):
        M = x.shape[0]
        self.L.check(self.L.fn["SNEPPX_qlayer_forward_bf16"](self.h, _ptr(x), _ptr(y), M,
                                                             self.L._stream(stream)), "qlayer_forward_bf16")

    def set_bias(self, bias, stream=None):
        """bias: numpy fp32 [N] (host), a torch fp32 [N] device tensor, or None."""
        if bias is None:
            rc = self.L.fn["SNEPPX_qlayer_set_bias_device"](self.h, None, self.L._stream(stream))
        elif isinstance(bias, np.ndarray):
            rc = self.L.fn["SNEPPX_qlayer_set_bias"](self.h, np.ascontiguousarray(bias, np.float32),
                                                      self.L._stream(stream))
        else:
            n = self.L.fn["SNEPPX_qlayer_out_features"](self.h)
            rc = self.L.fn["SNEPPX_qlayer_set_bias_device"](self.h, _bias_ptr(bias, n, bias),
                                                             self.L._stream(stream))
        self.L.check(rc, "qlayer_set_bias")

    def matmul_host(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M = x.shape[0]
        y = np.zeros((M, self.N), np.float32)
        self.L.check(self.L.fn["SNEPPX_qlayer_matmul_host"](self.h, x, y, M), "qlayer_matmul_host")
        return y

    def save(self, writer, prefix, stream=None):
        self.L.check(self.L.fn["SNEPPX_qlayer_save"](self.h, writer.h, prefix.encode(),
                                                     self.L._stream(stream)), "qlayer_save")


_LIB = None


def load() -> Library:
    global _LIB
    if _LIB is None:
        _LIB = Library()
    return _LIB
