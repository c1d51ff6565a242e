"""GGUF model files (include/vortx_gguf.h) from Python.

The parsing, validation and device upload all run in libvortx_hip.so; this
module only turns the C structs into Python values::

    f = GGUFFile("model.gguf")
    dev = torch.empty(f.header["data_size"], dtype=torch.uint8, device="cuda")
    f.upload(ctx, dev)                       # the whole data section, once
    w = f.qweight("blk.0.ffn_up.weight", dev)  # a QWeight into dev
    QuantGemv(0).dispatch(y, w, x)

The reference has no model-file reader; tensor dimensions follow its GGML
convention (GGML_IDS = [1, 0, 2, 3], src/shapes.rs:15-18): a weight with
ggml ne = [K, M] is the row-major [M, K] matrix W of y = W x.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass

from . import _ffi
from ._ffi import check, lib

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR_FMT = {UINT8: "B", INT8: "b", UINT16: "H", INT16: "h", UINT32: "I", INT32: "i", FLOAT32: "f", BOOL: "?",
               UINT64: "Q", INT64: "q", FLOAT64: "d"}


def _text(b: bytes) -> str:
    """GGUF strings are UTF-8; bytes that are not decode as surrogates, so no
    name or key is lost and the original bytes can be recovered."""
    return b.decode("utf-8", errors="surrogateescape")


@dataclass(frozen=True)
class TensorInfo:
    name: str
    type: int          # ggml type id
    ne: tuple          # ggml order, n_dims entries; ne[0] is the innermost dimension
    offset: int        # bytes from the start of the data section
    nbytes: int        # 0 when size_known is False
    size_known: bool


def type_size(ggml_type: int) -> tuple:
    """(elements, bytes) per block of a ggml type."""
    e, b = C.c_uint32(), C.c_uint32()
    check(lib().vx_gguf_type_size(ggml_type, C.byref(e), C.byref(b)))
    return e.value, b.value


class GGUFFile:
    """A mapped, validated GGUF v2/v3 file (vx_gguf_open). Raises VortxError
    (VX_ERR_IO / VX_ERR_FORMAT / VX_ERR_UNSUPPORTED) for unreadable files."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().vx_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        hd = _ffi.VxGgufHeader()
        check(lib().vx_gguf_get_header(h, C.byref(hd)))
        self.header = {k: getattr(hd, k) for k, _ in hd._fields_ if k != "reserved"}
        self.tensors = [self._tensor(i) for i in range(hd.n_tensors)]
        self._by_name = {t.name: i for i, t in enumerate(self.tensors)}
        self.metadata = {}
        for i in range(hd.n_kv):
            kv = _ffi.VxGgufKv()
            check(lib().vx_gguf_kv_info(h, i, C.byref(kv)))
            self.metadata[_text(kv.key)] = self._value(i, kv)

    # ------------------------------------------------------------ queries
    def _tensor(self, i: int) -> TensorInfo:
        t = _ffi.VxGgufTensor()
        check(lib().vx_gguf_tensor_info(self._h, i, C.byref(t)))
        return TensorInfo(_text(t.name), t.type, tuple(t.ne[:t.n_dims]), t.offset, t.nbytes,
                          bool(t.size_known))

    def _string(self, i: int, elem: int) -> str:
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().vx_gguf_kv_string(self._h, i, elem, C.byref(p), C.byref(n)))
        return _text(C.string_at(p, n.value)) if n.value else ""

    def _value(self, i: int, kv: _ffi.VxGgufKv):
        if kv.type == STRING:
            return self._string(i, 0)
        if kv.type == ARRAY:
            if kv.elem_type == STRING:
                return [self._string(i, j) for j in range(kv.count)]
            if kv.elem_type in _SCALAR_FMT:
                raw = C.string_at(kv.data, kv.nbytes) if kv.nbytes else b""
                return list(struct.unpack(f"<{kv.count}{_SCALAR_FMT[kv.elem_type]}", raw))
            return None  # arrays of arrays are validated but not decoded
        raw = C.string_at(kv.data, kv.nbytes)
        return struct.unpack("<" + _SCALAR_FMT[kv.type], raw)[0]

    def index(self, name: str) -> int:
        i = C.c_uint64()
        check(lib().vx_gguf_find_tensor(self._h, name.encode("utf-8", errors="surrogateescape"), C.byref(i)))
        return i.value

    def tensor(self, name: str) -> TensorInfo:
        return self.tensors[self.index(name)]

    def tensor_bytes(self, name: str) -> bytes:
        """A host copy of the tensor's bytes, read from the mapping."""
        t = _ffi.VxGgufTensor()
        check(lib().vx_gguf_tensor_info(self._h, self.index(name), C.byref(t)))
        if not t.size_known:
            raise _ffi.VortxError(_ffi.VX_ERR_UNSUPPORTED, f"no block size for ggml type {t.type}")
        return C.string_at(t.data, t.nbytes) if t.nbytes else b""

    # ------------------------------------------------------------- device
    def upload(self, ctx, device_data, offset: int = 0, nbytes: int | None = None, stream=None) -> None:
        """Copy data-section bytes [offset, offset + nbytes) to the uint8 GPU tensor
        ``device_data`` (vx_gguf_upload); returns once the copy has completed."""
        import torch

        from . import _stream
        if nbytes is None:
            nbytes = self.header["data_size"] - offset
        if not (isinstance(device_data, torch.Tensor) and device_data.is_cuda and device_data.dtype == torch.uint8
                and device_data.is_contiguous() and device_data.numel() >= nbytes):
            raise TypeError("device_data must be a contiguous uint8 GPU tensor of at least nbytes bytes")
        check(lib().vx_gguf_upload(ctx._h, _stream(stream), self._h, offset, nbytes, device_data.data_ptr()))

    def qweight(self, name: str, device_data):
        """The QWeight of a Q4_0 / Q8_0 / Q4_K matrix whose data section was
        uploaded whole into ``device_data`` (vx_gguf_qweight)."""
        from . import QWeight
        i = self.index(name)
        w = _ffi.VxQWeight()
        check(lib().vx_gguf_qweight(self._h, i, device_data.data_ptr(), C.byref(w)))
        t = self.tensors[i]
        return QWeight(device_data[t.offset:t.offset + t.nbytes], w.qtype, w.rows, w.cols, w.row_stride_bytes)

    def view(self, name: str, device_data):
        """``(buffer, TensorLayout)`` of an F32 tensor uploaded whole into
        ``device_data``, in vortx's GGML dimension convention (vx_gguf_view)."""
        import torch

        from . import TensorLayout
        i = self.index(name)
        v = _ffi.VxCView()
        check(lib().vx_gguf_view(self._h, i, device_data.data_ptr(), C.byref(v)))
        t = self.tensors[i]
        buf = device_data[t.offset:t.offset + t.nbytes].view(torch.float32)
        return buf, TensorLayout._py(v.layout)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().vx_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
