"""ctypes binding of libvortx_hip.so (the C ABI in include/vortx_hip.h).

The library is loaded from this package directory only; there is no
fallback implementation: if it is missing, importing ``vortx_amd`` raises.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libvortx_hip.so")

(VX_OK, VX_ERR_SHAPE, VX_ERR_UNSUPPORTED, VX_ERR_INVALID, VX_ERR_HIP, VX_ERR_NO_CODE_OBJECT, VX_ERR_IO, VX_ERR_FORMAT,
 VX_ERR_NOT_FOUND) = range(9)
VX_Q4_0, VX_Q8_0, VX_Q4_K = 2, 8, 12
ROUTE_NAIVE, ROUTE_TILED, ROUTE_GEMV, ROUTE_EMPTY = range(4)
NONE_STRIDE = 0xFFFFFFFF
VX_GEMV_X_INT8, VX_GEMV_X_F32 = 1, 2


class VxLayout(C.Structure):
    _fields_ = [("size", C.c_uint32 * 4), ("stride", C.c_uint32 * 4), ("rank", C.c_uint32), ("offset", C.c_uint32)]


class VxCView(C.Structure):
    _fields_ = [("base", C.c_void_p), ("layout", VxLayout)]


class VxMView(C.Structure):
    _fields_ = [("base", C.c_void_p), ("layout", VxLayout)]


class VxQWeight(C.Structure):
    _fields_ = [("base", C.c_void_p), ("qtype", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32),
                ("reserved", C.c_uint32), ("row_stride_bytes", C.c_uint64)]


class VxXq(C.Structure):
    _fields_ = [("base", C.c_void_p), ("K", C.c_uint32), ("B", C.c_uint32)]


class VxGemmOpts(C.Structure):
    _fields_ = [("alpha", C.c_float), ("beta", C.c_float), ("flags", C.c_uint32), ("reserved", C.c_uint32)]


VX_GEMM_BROADCAST, VX_GEMM_TILE_NARROW, VX_GEMM_TILE_WIDE, VX_GEMM_TILE_SMALL = 1, 2, 4, 8


class VxGgufHeader(C.Structure):
    _fields_ = [("version", C.c_uint32), ("reserved", C.c_uint32), ("n_tensors", C.c_uint64), ("n_kv", C.c_uint64),
                ("alignment", C.c_uint64), ("data_offset", C.c_uint64), ("data_size", C.c_uint64),
                ("file_size", C.c_uint64)]


class VxGgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("type", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("size_known", C.c_uint32), ("reserved", C.c_uint32),
                ("data", C.c_void_p)]


class VxGgufKv(C.Structure):
    _fields_ = [("key", C.c_char_p), ("type", C.c_uint32), ("elem_type", C.c_uint32), ("count", C.c_uint64),
                ("data", C.c_void_p), ("nbytes", C.c_uint64)]


# (name, restype, argtypes) for every exported entry point.
_P = C.POINTER
SIGNATURES = [
    ("vx_init", C.c_int, [C.c_int, _P(C.c_void_p)]),
    ("vx_destroy", C.c_int, [C.c_void_p]),
    ("vx_device_info", C.c_int, [C.c_void_p, _P(C.c_int), _P(C.c_int)]),
    ("vx_gemm_f32", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxCView), _P(VxCView)]),
    ("vx_gemm_f32_naive", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxCView), _P(VxCView)]),
    ("vx_gemm_f32_tiled", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxCView), _P(VxCView)]),
    ("vx_gemm_f32_ex", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxCView), _P(VxCView), _P(VxGemmOpts)]),
    ("vx_gemm_f32_route", C.c_int, [_P(VxMView), _P(VxCView), _P(VxCView), _P(C.c_int)]),
    ("vx_gemv_q", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight), _P(VxCView)]),
    ("vx_gemv_q_ex", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight), _P(VxCView), C.c_uint32]),
    ("vx_gemv_q_ws", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight), _P(VxCView), C.c_uint32,
                               C.c_void_p, C.c_uint64]),
    ("vx_gemv_q_ws_size", C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _P(C.c_uint64)]),
    ("vx_gemv_q_read_probe", C.c_int, [C.c_void_p, C.c_void_p, _P(VxQWeight), C.c_void_p]),
    ("vx_launch_floor", C.c_int, [C.c_void_p, C.c_void_p]),
    ("vx_dequantize", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight)]),
    ("vx_xq_size", C.c_int, [C.c_uint32, C.c_uint32, _P(C.c_uint64)]),
    ("vx_quantize_x", C.c_int, [C.c_void_p, C.c_void_p, _P(VxXq), _P(VxCView)]),
    ("vx_gemv_q_xq", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight), _P(VxXq)]),
    ("vx_gemv_q_noalloc", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxQWeight), _P(VxCView), C.c_uint32]),
    ("vx_quantize", C.c_int, [C.c_void_p, C.c_void_p, _P(VxQWeight), _P(VxCView)]),
    ("vx_contiguous", C.c_int, [C.c_void_p, C.c_void_p, _P(VxMView), _P(VxCView), C.c_void_p]),
    ("vx_qtype_info", C.c_int, [C.c_uint32, _P(C.c_uint32), _P(C.c_uint32)]),
    ("vx_layout_contiguous", C.c_int, [_P(C.c_uint32), C.c_uint32, _P(VxLayout)]),
    ("vx_layout_canonicalize", C.c_int, [_P(VxLayout), _P(VxLayout)]),
    ("vx_layout_transpose", C.c_int, [_P(VxLayout), C.c_uint32, C.c_uint32, _P(VxLayout)]),
    ("vx_layout_broadcast", C.c_int, [_P(VxLayout), _P(VxLayout), _P(VxLayout), _P(VxLayout)]),
    ("vx_layout_view", C.c_int, [_P(VxLayout), C.c_uint32, _P(C.c_uint32), C.c_uint32, _P(C.c_uint32),
                                 C.c_uint32, _P(VxLayout)]),
    ("vx_layout_narrow", C.c_int, [_P(VxLayout), C.c_uint32, C.c_uint32, C.c_uint32, _P(VxLayout)]),
    ("vx_layout_unsqueeze", C.c_int, [_P(VxLayout), C.c_uint32, _P(VxLayout)]),
    ("vx_layout_is_contiguous", C.c_int, [_P(VxLayout)]),
    ("vx_gguf_open", C.c_int, [C.c_char_p, _P(C.c_void_p)]),
    ("vx_gguf_close", C.c_int, [C.c_void_p]),
    ("vx_gguf_get_header", C.c_int, [C.c_void_p, _P(VxGgufHeader)]),
    ("vx_gguf_tensor_info", C.c_int, [C.c_void_p, C.c_uint64, _P(VxGgufTensor)]),
    ("vx_gguf_find_tensor", C.c_int, [C.c_void_p, C.c_char_p, _P(C.c_uint64)]),
    ("vx_gguf_kv_info", C.c_int, [C.c_void_p, C.c_uint64, _P(VxGgufKv)]),
    ("vx_gguf_find_key", C.c_int, [C.c_void_p, C.c_char_p, _P(C.c_uint64)]),
    ("vx_gguf_kv_string", C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, _P(C.c_void_p), _P(C.c_uint64)]),
    ("vx_gguf_type_size", C.c_int, [C.c_uint32, _P(C.c_uint32), _P(C.c_uint32)]),
    ("vx_gguf_upload", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]),
    ("vx_gguf_qweight", C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, _P(VxQWeight)]),
    ("vx_gguf_view", C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, _P(VxCView)]),
    ("vx_status_string", C.c_char_p, [C.c_int]),
    ("vx_last_error_message", C.c_char_p, []),
    ("vx_last_hip_error", C.c_int, []),
]

_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no non-HIP fallback)")
        # torch ships its own libamdhip64.so.7 (same SONAME as ROCm's). Load it
        # first so this library binds to the HIP runtime torch already uses:
        # two runtimes in one process do not see the same devices.
        import torch  # noqa: F401
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class VortxError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        name = lib().vx_status_string(status).decode()
        super().__init__(f"{name}: {message}")


def check(status: int) -> None:
    if status != VX_OK:
        raise VortxError(status, lib().vx_last_error_message().decode("utf-8", errors="replace"))
