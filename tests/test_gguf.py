"""GGUF reader (include/vortx_gguf.h) on the CPU: a hand-assembled fixture
checked field by field, every truncation of it, writer round trips over all
metadata types and tensor types, malformed files, and the host-side
qweight / view mapping. No GPU call is made here."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import vortx_amd as vx
from oracle import oracle as O
from tests import gguf_writer as W
from vortx_amd import _ffi

HERE = os.path.dirname(os.path.abspath(__file__))


def _tiny() -> bytes:
    out = bytearray()
    with open(os.path.join(HERE, "golden", "gguf_tiny.hex")) as f:
        for line in f:
            line = line.split("#", 1)[0].split()
            out += bytes(int(b, 16) for b in line)
    return bytes(out)


def _write(tmp_path, data: bytes, name="f.gguf") -> str:
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def _status(path) -> int:
    with pytest.raises(vx.VortxError) as e:
        vx.GGUFFile(path)
    return e.value.status


# ---------------------------------------------------------------- fixture
def test_tiny_fixture_every_field(tmp_path):
    data = _tiny()
    assert len(data) == 332
    f = vx.GGUFFile(_write(tmp_path, data))
    assert f.header == {"version": 3, "n_tensors": 2, "n_kv": 3, "alignment": 32, "data_offset": 224,
                        "data_size": 108, "file_size": 332}
    assert f.metadata == {"general.architecture": "llama", "llama.block_count": 2, "t.arr": [-1, 300]}
    w, b = f.tensors
    assert (w.name, w.type, w.ne, w.offset, w.nbytes, w.size_known) == ("w", 8, (32, 2), 0, 68, True)
    assert (b.name, b.type, b.ne, b.offset, b.nbytes, b.size_known) == ("b", 0, (3,), 96, 12, True)
    assert f.index("b") == 1 and f.tensor("w") == w
    wb = np.frombuffer(f.tensor_bytes("w"), np.uint8).reshape(2, 34)
    dq = O.dequant(O.Q8_0, wb, 2, 32)
    assert np.array_equal(dq[0], np.arange(32, dtype=np.float32))
    assert np.array_equal(dq[1], -0.5 * np.arange(-16, 16, dtype=np.float32))
    assert np.array_equal(np.frombuffer(f.tensor_bytes("b"), np.float32), np.float32([1.0, -2.5, 0.125]))
    with pytest.raises(vx.VortxError) as e:
        f.index("missing")
    assert e.value.status == _ffi.VX_ERR_NOT_FOUND
    f.close()


def test_tiny_fixture_as_version_2(tmp_path):
    data = bytearray(_tiny())
    data[4] = 2  # v2 has the v3 layout (v3 only added big-endian files)
    f = vx.GGUFFile(_write(tmp_path, bytes(data)))
    assert f.header["version"] == 2 and [t.name for t in f.tensors] == ["w", "b"]


def test_every_truncation_of_the_fixture_fails(tmp_path):
    data = _tiny()
    for n in range(len(data)):
        p = _write(tmp_path, data[:n], f"t{n}.gguf")
        assert _status(p) == _ffi.VX_ERR_FORMAT, n
        os.remove(p)


@pytest.mark.parametrize("patch,status", [
    ((0, b"GGUG"), _ffi.VX_ERR_FORMAT),                 # magic
    ((4, b"\x01\0\0\0"), _ffi.VX_ERR_UNSUPPORTED),      # version 1 (32-bit counts)
    ((4, b"\0\0\0\x03"), _ffi.VX_ERR_UNSUPPORTED),      # a big-endian file's version
    ((4, b"\x04\0\0\0"), _ffi.VX_ERR_FORMAT),           # unknown version
    ((8, struct.pack("<Q", 1 << 60)), _ffi.VX_ERR_FORMAT),   # n_tensors beyond the file
    ((16, struct.pack("<Q", 1 << 60)), _ffi.VX_ERR_FORMAT),  # n_kv beyond the file
    ((24, struct.pack("<Q", 0)), _ffi.VX_ERR_FORMAT),   # empty key
    ((24, struct.pack("<Q", 1 << 62)), _ffi.VX_ERR_FORMAT),  # key length beyond the file
    ((52, b"\x0d\0\0\0"), _ffi.VX_ERR_FORMAT),          # unknown value type 13
    ((56, struct.pack("<Q", 1 << 61)), _ffi.VX_ERR_FORMAT),  # string length beyond the file
])
def test_patched_fixture_errors(tmp_path, patch, status):
    data = bytearray(_tiny())
    at, b = patch
    data[at:at + len(b)] = b
    assert _status(_write(tmp_path, bytes(data))) == status


def test_unreadable_paths(tmp_path):
    assert _status(str(tmp_path / "missing.gguf")) == _ffi.VX_ERR_IO
    assert _status(str(tmp_path)) == _ffi.VX_ERR_IO


# ------------------------------------------------------------ round trips
ALL_KVS = [
    ("u8", W.UINT8, 255), ("i8", W.INT8, -128), ("u16", W.UINT16, 65535), ("i16", W.INT16, -32768),
    ("u32", W.UINT32, 2 ** 32 - 1), ("i32", W.INT32, -2 ** 31), ("f32", W.FLOAT32, -1.5),
    ("bool.t", W.BOOL, True), ("bool.f", W.BOOL, False), ("s", W.STRING, "héllo ✓"), ("s.empty", W.STRING, ""),
    ("u64", W.UINT64, 2 ** 64 - 1), ("i64", W.INT64, -2 ** 63), ("f64", W.FLOAT64, 1e300),
    ("a.f32", W.ARRAY, (W.FLOAT32, [0.5, -2.0, 3.25])), ("a.u8", W.ARRAY, (W.UINT8, [1, 2, 3])),
    ("a.i64", W.ARRAY, (W.INT64, [-1, 2 ** 62])), ("a.empty", W.ARRAY, (W.INT32, [])),
    ("a.bool", W.ARRAY, (W.BOOL, [True, False, True])),
    ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<s>", "", "▁the", "x" * 300])),
    ("a.nested", W.ARRAY, (W.ARRAY, [(W.INT8, [1, 2]), (W.STRING, ["a", "bc"]), (W.ARRAY, [(W.UINT64, [9])])])),
]


def _tensors(rng):
    def rb(n):
        return rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    return [
        ("tok_embd.weight", [256, 3], 12, rb(3 * 144)),      # Q4_K
        ("blk.0.attn_q.weight", [64, 5], 2, rb(5 * 2 * 18)),  # Q4_0
        ("blk.0.ffn_up.weight", [96, 2], 8, rb(2 * 3 * 34)),  # Q8_0
        ("norm", [7], 0, rb(28)),                             # F32
        ("h", [3, 2, 2], 1, rb(24)),                          # F16
        ("q6", [256, 1], 14, rb(210)),                        # Q6_K
        ("bf", [5, 1, 1, 2], 30, rb(20)),                     # BF16
        ("iq", [256, 2], 16, rb(132)),                        # IQ2_XXS: no block size in this reader
    ]


@pytest.mark.parametrize("alignment", [32, 64, 1, 4096])
def test_writer_roundtrip_every_type(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    tensors = _tensors(rng)
    data = W.build(ALL_KVS, tensors, alignment=alignment)
    f = vx.GGUFFile(_write(tmp_path, data))
    h = f.header
    assert h["alignment"] == alignment and h["n_tensors"] == len(tensors) and h["file_size"] == len(data)
    assert h["data_offset"] % alignment == 0
    for key, t, v in ALL_KVS:
        got = f.metadata[key]
        if key == "a.nested":
            assert got is None
        elif t == W.FLOAT32:
            assert got == np.float32(v)
        elif t == W.ARRAY and v[0] == W.FLOAT32:
            assert got == [float(np.float32(x)) for x in v[1]]
        elif t == W.ARRAY:
            assert got == list(v[1])
        else:
            assert got == v, key
    if alignment != 32:
        assert f.metadata["general.alignment"] == alignment
    for (name, ne, gt, raw), info in zip(tensors, f.tensors):
        assert (info.name, info.type, info.ne) == (name, gt, tuple(ne))
        assert info.offset % alignment == 0
        if gt == 16:
            assert not info.size_known and info.nbytes == 0
            continue
        e, b = vx.gguf.type_size(gt)
        assert info.nbytes == len(raw) == ne[0] // e * b * int(np.prod(ne[1:]))
        assert f.tensor_bytes(name) == raw
        start = h["data_offset"] + info.offset
        assert data[start:start + info.nbytes] == raw


def test_zero_tensors_and_zero_kv(tmp_path):
    f = vx.GGUFFile(_write(tmp_path, W.build([], [])))
    assert f.header["n_tensors"] == 0 and f.header["n_kv"] == 0 and f.header["data_size"] == 0
    assert f.metadata == {} and f.tensors == []


def test_type_sizes():
    for qt in (O.Q4_0, O.Q8_0, O.Q4_K):
        assert vx.gguf.type_size(qt) == O.QTYPE_INFO[qt]
    assert vx.gguf.type_size(0) == (1, 4) and vx.gguf.type_size(30) == (1, 2)
    assert vx.gguf.type_size(14) == (256, 210)
    for t in (4, 16, 31, 1000):
        with pytest.raises(vx.VortxError) as e:
            vx.gguf.type_size(t)
        assert e.value.status == _ffi.VX_ERR_UNSUPPORTED


# -------------------------------------------------------------- malformed
def _bad_files():
    q8 = bytes(34)
    ok_t = [("w", [32, 1], 8, q8)]
    yield "duplicate key", W.build([("k", W.UINT8, 1), ("k", W.UINT8, 2)], ok_t)
    yield "duplicate tensor", W.build([], ok_t + ok_t)
    yield "alignment 0", W.build([("general.alignment", W.UINT32, 0)], ok_t, set_alignment_key=False)
    yield "alignment 3", W.build([("general.alignment", W.UINT32, 3)], ok_t, set_alignment_key=False)
    yield "alignment as u64", W.build([("general.alignment", W.UINT64, 32)], ok_t, set_alignment_key=False)
    yield "ne[0] not a block multiple", W.build([], [("w", [33, 1], 8, bytes(34))])
    yield "unknown array element type", W.build([("a", W.ARRAY, (13, []))], [])
    deep = (W.INT8, [1])
    for _ in range(9):
        deep = (W.ARRAY, [deep])
    yield "arrays nested 10 deep", W.build([("a", W.ARRAY, deep)], [])
    # tensor infos written by hand: n_dims 0 / 5, negative ne, overflowing counts, offsets
    def raw(name, ne, t, off, data=b""):
        head = struct.pack("<4sIQQ", b"GGUF", 3, 1, 0) + W.tensor_info(name, ne, t, off)
        head += b"\0" * ((-len(head)) % 32)
        return head + data
    yield "n_dims 0", raw("w", [], 8, 0, q8)
    yield "n_dims 5", raw("w", [32, 1, 1, 1, 1], 8, 0, q8)
    yield "negative ne", raw("w", [32, 2 ** 63], 8, 0, q8)
    yield "element count overflow", raw("w", [2 ** 40, 2 ** 40], 0, 0)
    yield "byte size overflow", raw("w", [2 ** 32, 2 ** 31 - 1], 0, 0)
    # one row of 2^62 + 1 f32 elements: 4 (2^62 + 1) wraps to 4 bytes in u64
    yield "row byte size overflow (f32)", raw("w", [2 ** 62 + 1], 0, 0, bytes(32))
    yield "row byte size overflow (i64)", raw("w", [2 ** 61 + 1, 1], 27, 0, bytes(32))
    yield "misaligned offset", raw("w", [32, 1], 8, 16, bytes(64))
    yield "data past the end", raw("w", [32, 1], 8, 0, bytes(33))
    yield "offset past the end", raw("w", [32, 1], 8, 1 << 40, q8)
    yield "unknown type past the end", raw("w", [32, 1], 16, 64, q8)


@pytest.mark.parametrize("name,data", list(_bad_files()), ids=[n for n, _ in _bad_files()])
def test_malformed_files(tmp_path, name, data):
    assert _status(_write(tmp_path, data)) == _ffi.VX_ERR_FORMAT


def test_random_corruption_is_rejected_or_consistent(tmp_path):
    """Flipped bytes and cut-offs of a valid file: the reader either rejects
    the file or reports tensors that lie inside the data section."""
    rng = np.random.default_rng(5)
    base = bytearray(W.build(ALL_KVS[:6] + ALL_KVS[19:20], _tensors(rng)[:4], alignment=64))
    p = tmp_path / "c.gguf"
    for i in range(1500):
        data = bytearray(base)
        for _ in range(rng.integers(1, 5)):
            data[rng.integers(0, len(data))] = rng.integers(0, 256)
        if i % 3 == 0:
            data = data[:rng.integers(0, len(data) + 1)]
        p.write_bytes(bytes(data))
        try:
            f = vx.GGUFFile(str(p))
        except vx.VortxError as e:
            assert e.status in (_ffi.VX_ERR_FORMAT, _ffi.VX_ERR_UNSUPPORTED)
            continue
        h = f.header
        for t in f.tensors:
            assert t.offset % h["alignment"] == 0
            assert t.offset + t.nbytes <= h["data_size"]
        f.close()


# -------------------------------------------------- qweight / view (host)
FAKE = 0x7F0000000000  # a device address; these calls only compute fields


def _open(tmp_path, tensors, alignment=32):
    f = vx.GGUFFile(_write(tmp_path, W.build([], tensors, alignment=alignment)))
    return f


def test_qweight_fields(tmp_path):
    rng = np.random.default_rng(0)
    f = _open(tmp_path, _tensors(rng))
    for name in ("tok_embd.weight", "blk.0.attn_q.weight", "blk.0.ffn_up.weight"):
        i, t = f.index(name), f.tensor(name)
        w = _ffi.VxQWeight()
        _ffi.check(vx.lib().vx_gguf_qweight(f._h, i, FAKE, C.byref(w)))
        qk, bb = O.QTYPE_INFO[t.type]
        assert (w.base, w.qtype, w.rows, w.cols, w.row_stride_bytes) == (
            FAKE + t.offset, t.type, t.ne[1], t.ne[0], t.ne[0] // qk * bb)
    for name in ("norm", "h", "q6"):
        w = _ffi.VxQWeight()
        assert vx.lib().vx_gguf_qweight(f._h, f.index(name), FAKE, C.byref(w)) == _ffi.VX_ERR_UNSUPPORTED


def test_qweight_rejects_stacked_matrices(tmp_path):
    f = _open(tmp_path, [("e", [32, 2, 3], 8, bytes(34 * 6))])
    w = _ffi.VxQWeight()
    assert vx.lib().vx_gguf_qweight(f._h, 0, FAKE, C.byref(w)) == _ffi.VX_ERR_UNSUPPORTED


def test_view_follows_ggml_ids(tmp_path):
    """GGML_IDS = [1, 0, 2, 3] (src/shapes.rs:15-18): size[GGML_IDS[i]] = ne[i]."""
    t = [("v1", [7], 0, bytes(28)), ("v2", [5, 3], 0, bytes(60)), ("v3", [4, 3, 2], 0, bytes(96)),
         ("v4", [2, 3, 4, 5], 0, bytes(480)), ("h", [2], 1, bytes(4))]
    f = _open(tmp_path, t)
    want = {"v1": ((7,), (1,)), "v2": ((3, 5), (5, 1)), "v3": ((3, 4, 2), (4, 1, 12)),
            "v4": ((3, 2, 4, 5), (2, 1, 6, 24))}
    for name, (size, stride) in want.items():
        v = _ffi.VxCView()
        _ffi.check(vx.lib().vx_gguf_view(f._h, f.index(name), FAKE, C.byref(v)))
        l = v.layout
        assert v.base == FAKE + f.tensor(name).offset
        assert (l.rank, tuple(l.size[:l.rank]), tuple(l.stride[:l.rank]), l.offset) == (len(size), size, stride, 0)
        # every element of the view addresses its own ggml element exactly once
        idx = np.indices(size).reshape(len(size), -1).T @ np.array(stride)
        assert sorted(idx.tolist()) == list(range(int(np.prod(size))))
    v = _ffi.VxCView()
    assert vx.lib().vx_gguf_view(f._h, f.index("h"), FAKE, C.byref(v)) == _ffi.VX_ERR_UNSUPPORTED


def test_view_rejects_misaligned_f32(tmp_path):
    f = _open(tmp_path, [("a", [1], 1, bytes(2)), ("b", [1], 0, bytes(4))], alignment=2)
    assert f.tensor("b").offset == 2
    v = _ffi.VxCView()
    assert vx.lib().vx_gguf_view(f._h, f.index("b"), FAKE, C.byref(v)) == _ffi.VX_ERR_UNSUPPORTED


def test_nul_in_key_or_tensor_name_is_rejected(tmp_path):
    """Keys and tensor names are handed out NUL-terminated, so one holding a
    NUL byte could not be found by its own name (the sanitized fuzzer found
    such a file); the reader rejects it as malformed."""
    good = W.build([("a.b", W.UINT32, 1)], [("t", [32], 0, bytes(128))])
    assert vx.GGUFFile(_write(tmp_path, good)).header["n_kv"] == 1
    bad_key = W.build([("a\0b", W.UINT32, 1)], [])
    assert _status(_write(tmp_path, bad_key, "k.gguf")) == vx._ffi.VX_ERR_FORMAT
    bad_name = W.build([], [("t\0u", [32], 0, bytes(128))])
    assert _status(_write(tmp_path, bad_name, "n.gguf")) == vx._ffi.VX_ERR_FORMAT
