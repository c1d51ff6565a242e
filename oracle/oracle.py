"""Python access to the CPU oracle (oracle/vx_oracle.c) — TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker (or the timed CPU baseline):
the product library ``vortx_amd`` never calls it.

Every function takes and returns numpy arrays. Quantized matrices are
``uint8`` arrays of shape ``[M, row_stride_bytes]``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_0, Q8_0, Q4_K = 2, 8, 12
QTYPE_INFO = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144)}
QTYPE_NAME = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k"}


class OrcView(C.Structure):
    _fields_ = [("base", C.c_void_p), ("size", C.c_uint32 * 4), ("stride", C.c_int64 * 4)]


_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with gcc (oracle/Makefile)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_dequant.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_void_p]
        L.orc_gemv_q_f64.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64,
                                     C.c_void_p, C.c_int64, C.c_int64, C.c_uint32,
                                     C.c_void_p, C.c_int64, C.c_int64]
        L.orc_gemv_q_f32_omp.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64,
                                         C.c_void_p, C.c_uint32, C.c_void_p, C.c_int]
        L.orc_gemm_ref_f32.argtypes = [C.c_void_p, C.POINTER(C.c_int64), C.POINTER(OrcView), C.POINTER(OrcView)]
        L.orc_gemm_f64.argtypes = [C.c_void_p, C.POINTER(OrcView), C.POINTER(OrcView), C.c_void_p, C.c_uint32]
        L.orc_gemm_tiled_f32_omp.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                             C.c_uint32, C.c_int]
        L.orc_q4k_scale_min.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.orc_max_threads.restype = C.c_int
        L.orc_contiguous_u32.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
        L.orc_contiguous_u32.restype = C.c_int
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_quantize.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_void_p, C.c_uint64]
        L.orc_quantize.restype = C.c_int
        L.orc_q4k_fit.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.orc_q4k_fit.restype = C.c_int
        L.orc_quantize_x.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_uint32, C.c_uint32, C.c_void_p,
                                     C.c_void_p]
        L.orc_quantize_x.restype = C.c_int
        for name in ("orc_dequant", "orc_gemv_q_f64", "orc_gemv_q_f32_omp", "orc_gemm_ref_f32",
                     "orc_gemm_f64", "orc_gemm_tiled_f32_omp", "orc_q4k_scale_min"):
            if name != "orc_q4k_scale_min":
                getattr(L, name).restype = C.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ------------------------------------------------------------------ f16
def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.asarray(bits, dtype=np.uint16).ravel()
    out = np.array([L.orc_f16_to_f32(int(b)) for b in flat], dtype=np.float32)
    return out.reshape(np.shape(bits))


# ---------------------------------------------------------------- quant
def row_bytes(qtype: int, K: int) -> int:
    qk, bb = QTYPE_INFO[qtype]
    assert K % qk == 0
    return K // qk * bb


def dequant(qtype: int, w: np.ndarray, M: int, K: int) -> np.ndarray:
    """Decode W (uint8 [M, row_stride]) to f32 [M, K]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.shape[0] == M
    out = np.empty((M, K), dtype=np.float32)
    rc = lib().orc_dequant(qtype, _ptr(w), M, K, w.shape[1], _ptr(out))
    assert rc == 0, rc
    return out


def q4k_scale_min(scales12: bytes, s: int) -> tuple[int, int]:
    buf = np.frombuffer(bytes(scales12), dtype=np.uint8).copy()
    sc, mn = C.c_uint8(), C.c_uint8()
    lib().orc_q4k_scale_min(_ptr(buf), s, C.byref(sc), C.byref(mn))
    return sc.value, mn.value


def gemv_q_f64(qtype: int, w: np.ndarray, M: int, K: int, x_bk: np.ndarray) -> np.ndarray:
    """y[m, b] = sum_k W[m,k] x[b,k] in float64. x_bk is f32 [B, K]; returns [M, B]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x_bk, dtype=np.float32)
    B = x.shape[0]
    assert x.shape[1] == K
    y = np.empty((M, B), dtype=np.float64)
    rc = lib().orc_gemv_q_f64(qtype, _ptr(w), M, K, w.shape[1], _ptr(x), 1, K, B, _ptr(y), B, 1)
    assert rc == 0, rc
    return y


def gemv_q_f32_omp(qtype: int, w: np.ndarray, M: int, K: int, x_bk: np.ndarray, nthreads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x_bk, dtype=np.float32)
    B = x.shape[0]
    y = np.empty((M, B), dtype=np.float32)
    rc = lib().orc_gemv_q_f32_omp(qtype, _ptr(w), M, K, w.shape[1], _ptr(x), B, _ptr(y), nthreads)
    assert rc == 0, rc
    return y


# ----------------------------------------------------------------- gemm
def _canon(arr: np.ndarray):
    """numpy f32 array (any strides, rank <= 4) -> OrcView on its memory, rank 4."""
    assert arr.dtype == np.float32 and arr.ndim <= 4
    shape = (1,) * (4 - arr.ndim) + tuple(arr.shape)
    strides = (0,) * (4 - arr.ndim) + tuple(s // 4 for s in arr.strides)
    v = OrcView()
    v.base = arr.ctypes.data
    for i in range(4):
        v.size[i] = shape[i]
        v.stride[i] = strides[i]
    return v, shape


def gemm_ref_f32(lhs: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """f32 product in the reference kernels' summation order (rank <= 4 views)."""
    lv, ls = _canon(lhs)
    rv, rs = _canon(rhs)
    assert ls[0] == rs[0] and ls[1] == rs[1] and ls[3] == rs[2]
    out = np.empty((ls[0], ls[1], ls[2], rs[3]), dtype=np.float32)
    ost = (C.c_int64 * 4)(*[s // 4 for s in out.strides])
    lib().orc_gemm_ref_f32(_ptr(out), ost, C.byref(lv), C.byref(rv))
    nd = max(lhs.ndim, rhs.ndim)
    return out.reshape(out.shape[4 - nd:]) if nd >= 2 else out.reshape(out.shape[2:])


def gemm_f64(lhs: np.ndarray, rhs: np.ndarray, rows=None) -> np.ndarray:
    """float64 product, canonical [n, c, rows, N] (only `rows` if given)."""
    lv, ls = _canon(lhs)
    rv, rs = _canon(rhs)
    assert ls[0] == rs[0] and ls[1] == rs[1] and ls[3] == rs[2]
    if rows is None:
        R, rp = ls[2], None
    else:
        ra = np.ascontiguousarray(rows, dtype=np.uint32)
        R, rp = len(ra), ra
    out = np.empty((ls[0], ls[1], R, rs[3]), dtype=np.float64)
    lib().orc_gemm_f64(_ptr(out), C.byref(lv), C.byref(rv), None if rp is None else _ptr(rp), R)
    return out


def gemm_tiled_f32_omp(a: np.ndarray, b: np.ndarray, nthreads: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_tiled_f32_omp(_ptr(c), _ptr(a), _ptr(b), M, N, K, nthreads)
    return c


def max_threads() -> int:
    return lib().orc_max_threads()


# ----------------------------------------------------------- contiguous
def canonicalize(shape, stride):
    """src/shapes.rs:145-155: prepend size-1 dims up to rank 4 (their strides
    are those of a contiguous layout of the padded sizes)."""
    shape, stride = list(shape), list(stride)
    pad = 4 - len(shape)
    size = [1] * pad + shape
    st = [0] * 4
    acc = 1
    for k in range(3, -1, -1):
        st[k] = acc
        acc *= size[k]
    st[pad:] = stride
    return size, st


def contiguous_u32(src_flat: np.ndarray, shape, stride, offset: int = 0) -> np.ndarray:
    """vortx-shaders/src/linalg/contiguous.rs:70-90 over a 4-byte element
    buffer (viewed as uint32): the row-major copy of the view (shape, stride)
    starting at element `offset`."""
    buf = np.ascontiguousarray(src_flat).view(np.uint32)
    size, st = canonicalize(shape, stride)
    size_a = np.array(size, dtype=np.uint32)
    st_a = np.array(st, dtype=np.uint32)
    n = int(np.prod(size, dtype=np.int64))
    out = np.empty(max(n, 1), dtype=np.uint32)
    rc = lib().orc_contiguous_u32(_ptr(out), _ptr(buf), _ptr(size_a), _ptr(st_a), offset)
    assert rc == 0
    return out[:n].reshape(shape) if len(shape) else out[:n]


# ------------------------------------------------------------- quantize
def f32_to_f16(vals) -> np.ndarray:
    """orc_f32_to_f16 (round to nearest even) over an array; returns uint16 bits."""
    L = lib()
    flat = np.asarray(vals, dtype=np.float32).ravel()
    return np.array([L.orc_f32_to_f16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(vals))


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    """f32 [M, K] -> uint8 [M, row_bytes]: ggml's reference quantizers
    (quantize_row_{q8_0,q4_0,q4_K}_ref) as restated in vx_oracle.c."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    rb = row_bytes(qtype, K)
    out = np.zeros((M, rb), dtype=np.uint8)
    rc = lib().orc_quantize(qtype, _ptr(x), M, K, K, _ptr(out), rb)
    assert rc == 0, rc
    return out


def q4k_fit(x: np.ndarray, weights: np.ndarray):
    """One Q4_K sub-block's scale/min search (ggml make_qkx2_quants with the
    constants quantize_row_q4_K_ref passes) -> (levels uint8[32], scale, min)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    assert x.shape == w.shape == (32,)
    levels = np.zeros(32, np.uint8)
    sc, mn = C.c_float(), C.c_float()
    assert lib().orc_q4k_fit(_ptr(x), _ptr(w), _ptr(levels), C.byref(sc), C.byref(mn)) == 0
    return levels, sc.value, mn.value


# ---------------------------------------------------- activation split
# Byte position of element i of a 32-block in the level arrays (the order of
# a Q4_0 block's nibbles: byte t holds elements t and t + 16).
XQ_POS = np.array([8 * (i // 4) + i % 4 if i < 16 else 8 * ((i - 16) // 4) + 4 + (i - 16) % 4 for i in range(32)])


def quantize_x(x_bk: np.ndarray):
    """x f32 [B, K] (column b of the GEMV's [K, B] operand in row b) ->
    (levels int8 [K/32, B, 2, 32], scales f32 [K/32, B, 2]) as restated in
    vx_oracle.c orc_quantize_x (levels in XQ_POS order)."""
    x = np.ascontiguousarray(x_bk, dtype=np.float32)
    B, K = x.shape
    assert K % 32 == 0
    levels = np.zeros((K // 32, B, 2, 32), dtype=np.int8)
    scales = np.zeros((K // 32, B, 2), dtype=np.float32)
    rc = lib().orc_quantize_x(_ptr(x), 1, K, K, B, _ptr(levels), _ptr(scales))
    assert rc == 0, rc
    return levels, scales


def xq_decode_f64(levels: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """The x an activation split stands for, in float64: [B, K] with
    x[b, 32 j + i] = c2 (254 q1 + q2) at position XQ_POS[i] of block j."""
    nblk, B = levels.shape[:2]
    lv = levels.astype(np.float64)[:, :, :, XQ_POS]          # [nblk, B, 2, 32] in element order
    val = scales[:, :, 0:1].astype(np.float64) * (254.0 * lv[:, :, 0] + lv[:, :, 1])
    return val.transpose(1, 0, 2).reshape(B, nblk * 32)


def xq_device_levels(levels: np.ndarray) -> np.ndarray:
    """The oracle's levels [K/32, B, 2, 32] (positions in XQ_POS order) in the
    library's device layout [ceil(K/256), 4, 4, B, 2, 2, 8] (item, block pair
    (j%8)/2, position group p/8, column, level, block parity j%2, byte p%8;
    blocks past K/32 zero)."""
    nblk, B = levels.shape[:2]
    ni = -(-nblk // 8)
    pad = np.zeros((ni * 8, B, 2, 32), dtype=np.int8)
    pad[:nblk] = levels
    v = pad.reshape(ni, 4, 2, B, 2, 4, 8)       # item, pair, parity, col, level, group, byte
    return np.ascontiguousarray(v.transpose(0, 1, 5, 3, 4, 2, 6))
