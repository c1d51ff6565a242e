"""vortx_amd — MI355X (gfx950) linalg hot path of vortx behind a C ABI.

Python-side mirror of the reference interface for this path:

* :class:`TensorLayout` — vortx's view algebra (src/shapes.rs:51-530),
  computed by the native library;
* :class:`Gemm` — ``Gemm::dispatch`` / ``dispatch_naive`` / ``dispatch_tiled``
  (src/linalg/gemm.rs:47-305) on f32 views: out = lhs * rhs;
* :class:`QuantGemv` — block-quantized GEMV y = W x (Q8_0, Q4_0, Q4_K) and
  dequantize, which the reference does not have;
* :class:`Contiguous` — ``Contiguous::launch`` (src/linalg/contiguous.rs:22-119),
  the strided -> contiguous copy of 4-byte elements;
* :class:`GGUFFile` — GGUF model files (vortx_amd.gguf), which feed real
  quantized weights to :class:`QuantGemv`.

A view is either a torch tensor on the GPU (its sizes, strides and storage
offset become the layout) or a ``(buffer, TensorLayout)`` pair, exactly like
vortx's ``TensorRef { layout, buffer }``. torch only provides device memory
and streams; every launch goes through libvortx_hip.so, and there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _ffi
from ._ffi import (NONE_STRIDE, ROUTE_EMPTY, ROUTE_GEMV, ROUTE_NAIVE, ROUTE_TILED, VX_Q4_0, VX_Q4_K, VX_Q8_0,
                   VortxError, check, lib)

__all__ = ["TensorLayout", "layout_extent", "XQ", "xq_size", "Gemm", "QuantGemv", "QWeight", "Contiguous", "GGUFFile", "VortxError", "VX_Q4_0", "VX_Q8_0", "VX_Q4_K",
           "ROUTE_NAIVE", "ROUTE_TILED", "ROUTE_GEMV", "ROUTE_EMPTY", "qtype_info", "lib"]

# Load eagerly: a missing library must fail at import, not at first call.
lib()


# ---------------------------------------------------------------- layout
@dataclass(frozen=True)
class TensorLayout:
    """vortx's TensorLayout (src/shapes.rs:51-60): element sizes/strides, rank <= 4."""
    size: tuple
    stride: tuple
    rank: int
    offset: int = 0

    def _c(self) -> _ffi.VxLayout:
        l = _ffi.VxLayout()
        for i in range(4):
            l.size[i] = self.size[i] if i < len(self.size) else 1
            l.stride[i] = self.stride[i] if i < len(self.stride) else 1
        l.rank = self.rank
        l.offset = self.offset
        return l

    @staticmethod
    def _py(l: _ffi.VxLayout) -> "TensorLayout":
        return TensorLayout(tuple(l.size), tuple(l.stride), l.rank, l.offset)

    @staticmethod
    def contiguous(size) -> "TensorLayout":
        arr = (C.c_uint32 * max(1, len(size)))(*size)
        out = _ffi.VxLayout()
        check(lib().vx_layout_contiguous(arr, len(size), C.byref(out)))
        return TensorLayout._py(out)

    def dims(self) -> tuple:
        return self.size[:self.rank]

    def canonicalize(self) -> "TensorLayout":
        out = _ffi.VxLayout()
        check(lib().vx_layout_canonicalize(C.byref(self._c()), C.byref(out)))
        return TensorLayout._py(out)

    def transpose(self, a: int, b: int) -> "TensorLayout":
        out = _ffi.VxLayout()
        check(lib().vx_layout_transpose(C.byref(self._c()), a, b, C.byref(out)))
        return TensorLayout._py(out)

    def broadcast(self, other: "TensorLayout"):
        """(self', other') or None when incompatible (src/shapes.rs:346-391)."""
        a, b = _ffi.VxLayout(), _ffi.VxLayout()
        s = lib().vx_layout_broadcast(C.byref(self._c()), C.byref(other._c()), C.byref(a), C.byref(b))
        if s == _ffi.VX_ERR_SHAPE:
            return None
        check(s)
        return TensorLayout._py(a), TensorLayout._py(b)

    def view(self, offset: int, shape, stride=()) -> "TensorLayout":
        sh = (C.c_uint32 * max(1, len(shape)))(*shape)
        st = (C.c_uint32 * max(1, len(stride)))(*[NONE_STRIDE if s is None else s for s in stride])
        out = _ffi.VxLayout()
        check(lib().vx_layout_view(C.byref(self._c()), offset, sh, len(shape), st, len(stride), C.byref(out)))
        return TensorLayout._py(out)

    def narrow(self, axis: int, first: int, count: int) -> "TensorLayout":
        out = _ffi.VxLayout()
        check(lib().vx_layout_narrow(C.byref(self._c()), axis, first, count, C.byref(out)))
        return TensorLayout._py(out)

    def unsqueeze(self, axis: int) -> "TensorLayout":
        out = _ffi.VxLayout()
        check(lib().vx_layout_unsqueeze(C.byref(self._c()), axis, C.byref(out)))
        return TensorLayout._py(out)

    def is_contiguous(self) -> bool:
        return bool(lib().vx_layout_is_contiguous(C.byref(self._c())))


def layout_extent(layout: TensorLayout) -> int:
    """Elements a buffer needs to hold every element of ``layout``: its offset
    plus the largest index sum((size - 1) * stride) plus one (0 when a
    dimension below rank is empty)."""
    dims = layout.size[:layout.rank]
    if any(d == 0 for d in dims):
        return 0
    return layout.offset + sum((d - 1) * st for d, st in zip(dims, layout.stride[:layout.rank])) + 1


def _view_of(v, mutable: bool, any4: bool = False):
    """torch tensor or (buffer, TensorLayout) -> VxCView / VxMView.
    any4: accept any 4-byte element type (bit copies), not only float32."""
    import torch
    ok = (lambda t: t.element_size() == 4) if any4 else (lambda t: t.dtype == torch.float32)
    if isinstance(v, tuple):
        buf, layout = v
        if not (isinstance(buf, torch.Tensor) and ok(buf)):
            raise TypeError("view buffer must be a float32 tensor on the GPU")
        # The C ABI carries no buffer sizes: a layout reaching past the buffer
        # would become an out-of-bounds device access, so it is refused here.
        need = layout_extent(layout)
        if need > buf.numel():
            raise VortxError(_ffi.VX_ERR_INVALID,
                             f"layout {layout} reaches element {need - 1} of a {buf.numel()}-element buffer")
        if not buf.is_cuda:
            raise TypeError("view buffer must be a float32 tensor on the GPU")
        base = buf.data_ptr()
    else:
        if not (isinstance(v, torch.Tensor) and ok(v) and v.is_cuda):
            raise TypeError("views must be float32 tensors on the GPU")
        if v.dim() > 4:
            raise VortxError(_ffi.VX_ERR_UNSUPPORTED, "tensors of ranks > 4 not supported")
        if any(s < 0 for s in v.stride()):
            raise VortxError(_ffi.VX_ERR_UNSUPPORTED, "negative strides")
        base = v.untyped_storage().data_ptr()
        layout = TensorLayout(tuple(v.shape), tuple(v.stride()), v.dim(), v.storage_offset())
    view = (_ffi.VxMView if mutable else _ffi.VxCView)()
    view.base = base
    view.layout = layout._c()
    return view


def _stream(stream) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


# ------------------------------------------------------------------ gemm
class _Context:
    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().vx_init(device, C.byref(h)))
        self._h = h
        self.device = device
        n = C.c_int()
        check(lib().vx_device_info(h, None, C.byref(n)))
        self.num_cus = n.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().vx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gemm(_Context):
    """f32 GEMM on tensor views: out = lhs * rhs (src/linalg/gemm.rs:34-321).

    ``dispatch`` validates like the reference (a shape mismatch raises
    VortxError(VX_ERR_SHAPE) where vortx panics) and routes: naive kernel when
    M < 32 and N < 32, f32 GEMV when N == 1, MFMA tiled kernel otherwise.
    """

    def _call(self, fn, out, lhs, rhs, stream):
        o, l, r = _view_of(out, True), _view_of(lhs, False), _view_of(rhs, False)
        check(fn(self._h, _stream(stream), C.byref(o), C.byref(l), C.byref(r)))

    def dispatch(self, out, lhs, rhs, stream=None) -> None:
        self._call(lib().vx_gemm_f32, out, lhs, rhs, stream)

    def dispatch_ex(self, out, lhs, rhs, alpha: float = 1.0, beta: float = 0.0, broadcast: bool = False,
                    tile: str = "auto", stream=None) -> None:
        """out = alpha * (lhs x rhs) + beta * out (vx_gemm_f32_ex); out is not
        read when beta == 0. ``broadcast``: batch dims of lhs / rhs of size 1
        are reused along out's (src/shapes.rs:346-391 semantics). ``tile``:
        "narrow" / "wide" / "small" pins the MFMA kernel's 128 x 128 / 128 x 256 /
        64 x 64 output tiles (same bits every way), "auto" lets the library choose."""
        o, l, r = _view_of(out, True), _view_of(lhs, False), _view_of(rhs, False)
        flags = (_ffi.VX_GEMM_BROADCAST if broadcast else 0) | {"auto": 0, "narrow": _ffi.VX_GEMM_TILE_NARROW,
                                                                 "wide": _ffi.VX_GEMM_TILE_WIDE,
                                                                 "small": _ffi.VX_GEMM_TILE_SMALL}[tile]
        opts = _ffi.VxGemmOpts(alpha, beta, flags, 0)
        check(lib().vx_gemm_f32_ex(self._h, _stream(stream), C.byref(o), C.byref(l), C.byref(r), C.byref(opts)))

    def dispatch_naive(self, out, lhs, rhs, stream=None) -> None:
        self._call(lib().vx_gemm_f32_naive, out, lhs, rhs, stream)

    def dispatch_tiled(self, out, lhs, rhs, stream=None) -> None:
        self._call(lib().vx_gemm_f32_tiled, out, lhs, rhs, stream)

    @staticmethod
    def route(out, lhs, rhs) -> int:
        o, l, r = _view_of(out, True), _view_of(lhs, False), _view_of(rhs, False)
        rt = C.c_int()
        check(lib().vx_gemm_f32_route(C.byref(o), C.byref(l), C.byref(r), C.byref(rt)))
        return rt.value


# ----------------------------------------------------------------- quant
def qtype_info(qtype: int) -> tuple:
    """(weights per block, bytes per block)."""
    qk, bb = C.c_uint32(), C.c_uint32()
    check(lib().vx_qtype_info(qtype, C.byref(qk), C.byref(bb)))
    return qk.value, bb.value


@dataclass
class QWeight:
    """Row-major block-quantized matrix [rows, cols] in a uint8 GPU tensor."""
    data: object  # torch.uint8 tensor on the GPU, >= rows * row_stride bytes
    qtype: int
    rows: int
    cols: int
    row_stride: int = 0

    def __post_init__(self):
        qk, bb = qtype_info(self.qtype)
        if self.row_stride == 0:
            self.row_stride = self.cols // qk * bb
        # The C ABI carries no buffer size: an undersized buffer would be read
        # out of bounds on the device, so it is refused here.
        if self.rows and self.cols:
            need = (self.rows - 1) * self.row_stride + self.cols // qk * bb
            have = self.data.numel() * self.data.element_size()
            if have < need:
                raise VortxError(_ffi.VX_ERR_INVALID,
                                 f"QWeight needs {need} bytes ({self.rows} rows at stride {self.row_stride}), "
                                 f"the buffer holds {have}")

    def _c(self) -> _ffi.VxQWeight:
        w = _ffi.VxQWeight()
        w.base = self.data.data_ptr()
        w.qtype = self.qtype
        w.rows = self.rows
        w.cols = self.cols
        w.reserved = 0
        w.row_stride_bytes = self.row_stride
        return w


def xq_size(K: int, B: int) -> int:
    """Bytes of the activation split of a [K, B] x (include/vortx_hip.h vx_xq)."""
    n = C.c_uint64()
    check(lib().vx_xq_size(K, B, C.byref(n)))
    return n.value


@dataclass
class XQ:
    """x [K, B] split into two int8 levels per 32-block (vx_xq): a uint8 GPU
    buffer of at least xq_size(K, B) bytes, 16-byte aligned. ``levels()``
    views its level bytes in the device layout ([ceil(K/256), 4, 4, B, 2, 2, 8]
    int8: item, block pair, position group, column, level, block parity,
    byte) and ``scales()`` its [K/32, B, 2] f32 scales."""
    data: object
    K: int
    B: int

    def __post_init__(self):
        need = xq_size(self.K, self.B)
        have = self.data.numel() * self.data.element_size()
        if have < need:
            raise VortxError(_ffi.VX_ERR_INVALID, f"XQ needs {need} bytes, the buffer holds {have}")

    @staticmethod
    def empty(K: int, B: int, device="cuda:0") -> "XQ":
        import torch
        return XQ(torch.empty(xq_size(K, B), dtype=torch.uint8, device=device), K, B)

    def levels(self):
        import torch
        ni = (self.K + 255) // 256
        return self.data[:ni * self.B * 512].view(torch.int8).view(ni, 4, 4, self.B, 2, 2, 8)

    def scales(self):
        import torch
        ni, nb = (self.K + 255) // 256, self.K // 32
        off = ni * self.B * 512
        return self.data[off:off + nb * self.B * 8].view(torch.float32).view(nb, self.B, 2)

    def _c(self) -> _ffi.VxXq:
        q = _ffi.VxXq()
        q.base = self.data.data_ptr()
        q.K = self.K
        q.B = self.B
        return q


class QuantGemv(_Context):
    """y = W x for GGML Q8_0 / Q4_0 / Q4_K weights, f32 accumulate."""

    def quantize_x(self, out: XQ, x, stream=None) -> None:
        """Split x (a [K, B] f32 view, or [K]) into ``out`` (vx_quantize_x)."""
        xv, q = _view_of(x, False), out._c()
        check(lib().vx_quantize_x(self._h, _stream(stream), C.byref(q), C.byref(xv)))

    def dispatch_xq(self, y, w: "QWeight", xq: XQ, stream=None) -> None:
        """y = W x from the split of x (vx_gemv_q_xq)."""
        yv, wc, q = _view_of(y, True), w._c(), xq._c()
        check(lib().vx_gemv_q_xq(self._h, _stream(stream), C.byref(yv), C.byref(wc), C.byref(q)))

    @staticmethod
    def workspace_size(w: "QWeight", B: int, x_f32: bool = False) -> int:
        """Bytes of workspace ``dispatch(..., workspace=)`` may use for B
        columns (vx_gemv_q_ws_size; 0: none)."""
        n = C.c_uint64()
        check(lib().vx_gemv_q_ws_size(w.qtype, w.cols, B, _ffi.VX_GEMV_X_F32 if x_f32 else 0, C.byref(n)))
        return n.value

    @staticmethod
    def workspace(w: "QWeight", B: int, device="cuda:0"):
        """A device workspace for ``dispatch`` on W with B columns (a uint8
        tensor; torch's allocator owns it, the library never does)."""
        import torch
        return torch.empty(max(16, QuantGemv.workspace_size(w, B)), dtype=torch.uint8, device=device)

    def dispatch(self, y, w: QWeight, x, stream=None, x_f32: bool = False, x_int8: bool = False,
                 workspace=None) -> None:
        """y = W x. By default x is split per 32-block into two int8 levels
        (error <= 1.6e-5 of the block's max|x|) and every product is exact in
        int32 (include/vortx_hip.h, vx_gemv_q_ex). ``x_f32=True`` keeps x in
        f32 (f32 FMA on the exactly decoded weights); ``x_int8=True`` names
        the default explicitly. ``workspace``: a uint8 GPU tensor of at least
        ``workspace_size(w, B)`` bytes (vx_gemv_q_ws), where batched shapes
        split x when the GEMV kernel cannot split it itself; without one
        those shapes keep x in f32 (or, with ``x_int8``, raise)."""
        yv, xv, wc = _view_of(y, True), _view_of(x, False), w._c()
        flags = (_ffi.VX_GEMV_X_F32 if x_f32 else 0) | (_ffi.VX_GEMV_X_INT8 if x_int8 else 0)
        if workspace is None:
            check(lib().vx_gemv_q_ex(self._h, _stream(stream), C.byref(yv), C.byref(wc), C.byref(xv), flags))
            return
        import torch
        if not (isinstance(workspace, torch.Tensor) and workspace.is_cuda and workspace.is_contiguous()):
            raise TypeError("workspace must be a contiguous GPU tensor")
        nbytes = workspace.numel() * workspace.element_size()
        check(lib().vx_gemv_q_ws(self._h, _stream(stream), C.byref(yv), C.byref(wc), C.byref(xv), flags,
                                 workspace.data_ptr(), nbytes))

    def read_probe(self, y, w: QWeight, stream=None) -> None:
        """The batch-1 GEMV's loads of W alone (vx_gemv_q_read_probe), one
        word per row to the f32 GPU tensor y (measurement only)."""
        import torch
        if not (isinstance(y, torch.Tensor) and y.is_cuda and y.dtype == torch.float32 and y.is_contiguous()
                and y.numel() >= w.rows):
            raise TypeError("y must be a contiguous float32 GPU tensor of at least w.rows elements")
        wc = w._c()
        check(lib().vx_gemv_q_read_probe(self._h, _stream(stream), C.byref(wc), y.data_ptr()))

    def launch_floor(self, stream=None) -> None:
        """One empty launch on the batch-1 GEMV's grid (vx_launch_floor,
        measurement only): the fixed cost of a launch."""
        check(lib().vx_launch_floor(self._h, _stream(stream)))

    def quantize(self, out: "QWeight", x, stream=None) -> None:
        """Write the blocks of ``out`` from the f32 [rows, cols] view ``x``
        (ggml's reference quantizers; see include/vortx_hip.h vx_quantize)."""
        xv, wc = _view_of(x, False), out._c()
        check(lib().vx_quantize(self._h, _stream(stream), C.byref(wc), C.byref(xv)))

    def dequantize(self, out, w: QWeight, stream=None) -> None:
        ov, wc = _view_of(out, True), w._c()
        check(lib().vx_dequantize(self._h, _stream(stream), C.byref(ov), C.byref(wc)))


class Contiguous(_Context):
    """vortx's Contiguous op (src/linalg/contiguous.rs:11-119): copy a
    strided view of 4-byte elements into a contiguous output of the same
    size. ``offset`` is the optional device u32 tensor of the reference's
    ``launch``: when given, the source's raw buffer is read at that offset and
    the view's own offset is ignored, as in the reference."""

    def launch(self, out, tensor, offset=None, stream=None) -> None:
        import torch
        ov, tv = _view_of(out, True, any4=True), _view_of(tensor, False, any4=True)
        off = None
        if offset is not None:
            if not (isinstance(offset, torch.Tensor) and offset.is_cuda and offset.element_size() == 4
                    and offset.numel() >= 1):
                raise TypeError("offset must be a 4-byte integer tensor on the GPU")
            off = offset.data_ptr()
        check(lib().vx_contiguous(self._h, _stream(stream), C.byref(ov), C.byref(tv), off))


from .gguf import GGUFFile  # noqa: E402  (needs QWeight and TensorLayout above)
