"""The C-ABI library on the CPU: it loads, exports every entry point that
include/*.h declare, and its host-side validation and routing
behave without a GPU (no kernel is launched here)."""
import ctypes as C
import os
import re

import pytest

import vortx_amd as vx
from vortx_amd import _ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            with open(os.path.join(ROOT, "include", h)) as f:
                src = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
            names |= set(re.findall(r"\b(vx_\w+)\s*\(", src))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    names = _declared()
    assert "vx_gemm_f32" in names and "vx_gemv_q" in names and len(names) >= 20
    lib = C.CDLL(_ffi.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_declarations():
    bound = {n for n, _, _ in _ffi.SIGNATURES}
    assert set(_declared()) <= bound


def _view(cls, base, shape, strides=None, offset=0):
    v = cls()
    v.base = base
    l = vx.TensorLayout.contiguous(shape)
    if strides is not None:
        l = vx.TensorLayout(tuple(list(strides) + [1] * (4 - len(strides))) and l.size,
                            tuple(list(strides) + [1] * (4 - len(strides))), len(shape), offset)
    v.layout = vx.TensorLayout(l.size, l.stride, l.rank, offset)._c()
    return v


def _route(o, l, r):
    rt = C.c_int(-1)
    s = vx.lib().vx_gemm_f32_route(C.byref(o), C.byref(l), C.byref(r), C.byref(rt))
    return s, rt.value


FAKE = 0x10000  # never dereferenced: routing is host logic


@pytest.mark.parametrize("M,N,K,route", [
    (256, 1, 256, vx.ROUTE_GEMV),   # the reference test's shape
    (16, 16, 100, vx.ROUTE_NAIVE),  # M < 32 and N < 32 (gemm.rs:111-112)
    (31, 31, 5, vx.ROUTE_NAIVE),
    (32, 8, 8, vx.ROUTE_TILED),
    (4096, 4096, 4096, vx.ROUTE_TILED),
    (0, 8, 8, vx.ROUTE_EMPTY),
])
def test_route(M, N, K, route):
    s, rt = _route(_view(_ffi.VxMView, FAKE, [M, N]), _view(_ffi.VxCView, FAKE, [M, K]), _view(_ffi.VxCView, FAKE, [K, N]))
    assert s == _ffi.VX_OK and rt == route


def test_shape_mismatch_reports_like_the_reference():
    s, _ = _route(_view(_ffi.VxMView, FAKE, [8, 9]), _view(_ffi.VxCView, FAKE, [8, 5]), _view(_ffi.VxCView, FAKE, [6, 9]))
    assert s == _ffi.VX_ERR_SHAPE
    assert vx.lib().vx_last_error_message().decode().startswith("incompatible gemm shapes")
    # batch dims must match exactly (no broadcasting, gemm.rs:64)
    s, _ = _route(_view(_ffi.VxMView, FAKE, [2, 8, 9]), _view(_ffi.VxCView, FAKE, [1, 8, 5]),
                  _view(_ffi.VxCView, FAKE, [2, 5, 9]))
    assert s == _ffi.VX_ERR_SHAPE


def test_invalid_arguments():
    lib = vx.lib()
    o = _view(_ffi.VxMView, 0, [8, 9])  # null base with elements
    s, _ = _route(o, _view(_ffi.VxCView, FAKE, [8, 5]), _view(_ffi.VxCView, FAKE, [5, 9]))
    assert s == _ffi.VX_ERR_INVALID
    bad = _view(_ffi.VxMView, FAKE, [8, 9])
    bad.layout.rank = 5
    s, _ = _route(bad, _view(_ffi.VxCView, FAKE, [8, 5]), _view(_ffi.VxCView, FAKE, [5, 9]))
    assert s == _ffi.VX_ERR_UNSUPPORTED
    assert lib.vx_gemm_f32(None, None, None, None, None) == _ffi.VX_ERR_INVALID
    assert lib.vx_gemv_q(None, None, None, None, None) == _ffi.VX_ERR_INVALID
    qk, bb = C.c_uint32(), C.c_uint32()
    assert lib.vx_qtype_info(3, C.byref(qk), C.byref(bb)) == _ffi.VX_ERR_INVALID
    assert lib.vx_qtype_info(12, C.byref(qk), C.byref(bb)) == _ffi.VX_OK and (qk.value, bb.value) == (256, 144)
    assert lib.vx_status_string(_ffi.VX_ERR_SHAPE) == b"VX_ERR_SHAPE"


def test_init_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    s = vx.lib().vx_init(0, C.byref(h))
    assert s in (_ffi.VX_ERR_HIP, _ffi.VX_ERR_INVALID) and not h.value
    assert vx.lib().vx_last_error_message()


def test_gemv_q_ws_size():
    """Workspace bytes of vx_gemv_q_ws: the activation split (vx_xq_size) on
    the int8 route at B >= 2, nothing at B = 1, with f32 x or K % 64 != 0."""
    L = vx.lib()
    n = C.c_uint64()
    for qt, K, B, flags, want in [(vx.VX_Q4_0, 4096, 8, 0, vx.xq_size(4096, 8)),
                                  (vx.VX_Q4_K, 4096, 16, 0, vx.xq_size(4096, 16)),
                                  (vx.VX_Q8_0, 11008, 3, 1, vx.xq_size(11008, 3)),
                                  (vx.VX_Q4_0, 4096, 1, 0, 0), (vx.VX_Q4_0, 4096, 8, 2, 0), (vx.VX_Q4_0, 96, 4, 0, 0)]:
        assert L.vx_gemv_q_ws_size(qt, K, B, flags, C.byref(n)) == 0
        assert n.value == want, (qt, K, B, flags)
    assert L.vx_gemv_q_ws_size(3, 4096, 8, 0, C.byref(n)) == _ffi.VX_ERR_INVALID
