"""GGUF files on the GPU: the data section uploaded through the pinned
staging path must arrive byte for byte (whole, in pieces, across staging
chunks), and the weights and activations read from the file must give the
oracle's GEMV through vx_gguf_qweight / vx_gguf_view."""
import numpy as np
import pytest
import torch

import vortx_amd as vx
from oracle import oracle as O
from tests import gguf_writer as W
from tests.helpers import assert_close, note
from vortx_amd import _ffi
from vortx_amd import synthetic as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _model(tmp_path, alignment=32, big=False):
    """A file with one matrix per supported format, an activation matrix
    x with ggml ne = [K, B] (vortx [B, K]) and a norm vector."""
    K, B = 1024, 3
    mats = {"blk.0.attn_q.weight": (vx.VX_Q4_0, 200), "blk.0.ffn_up.weight": (vx.VX_Q8_0, 96),
            "blk.0.ffn_down.weight": (vx.VX_Q4_K, 130)}
    if big:  # a 71 MB tensor: more than two 32 MB staging chunks
        mats["output.weight"] = (vx.VX_Q8_0, 8192 * 8192 // K)
    tensors, host = [], {}
    for i, (name, (qt, M)) in enumerate(mats.items()):
        w = S.quant_weights(qt, M, K, seed=30 + i).numpy()
        host[name] = (qt, M, w)
        tensors.append((name, [K, M], qt, w.tobytes()))
    x = S.activations(B, K, seed=9).numpy()
    tensors.append(("x", [K, B], 0, x.tobytes()))
    tensors.append(("output_norm.weight", [K], 0, np.linspace(-1, 1, K, dtype=np.float32).tobytes()))
    p = tmp_path / "model.gguf"
    data = W.build([("general.architecture", W.STRING, "llama")], tensors, alignment=alignment)
    p.write_bytes(data)
    return str(p), data, host, x


@pytest.mark.parametrize("alignment", [32, 256])
def test_upload_whole_data_section_bit_exact(qgemv, tmp_path, alignment):
    path, data, _, _ = _model(tmp_path, alignment)
    f = vx.GGUFFile(path)
    h = f.header
    note(f"gguf upload {h['data_size']} bytes, alignment {alignment}")
    dev = torch.full((h["data_size"],), 0xCD, dtype=torch.uint8, device=DEV)
    f.upload(qgemv, dev)
    got = dev.cpu().numpy().tobytes()
    assert got == data[h["data_offset"]:]


def test_upload_across_staging_chunks_and_pieces(qgemv, tmp_path):
    path, data, _, _ = _model(tmp_path, big=True)
    f = vx.GGUFFile(path)
    h = f.header
    note(f"gguf upload {h['data_size']} bytes in pieces")
    assert h["data_size"] > 2 * (32 << 20)
    body = np.frombuffer(data, np.uint8)[h["data_offset"]:]
    dev = torch.zeros(h["data_size"], dtype=torch.uint8, device=DEV)
    f.upload(qgemv, dev)
    assert torch.equal(dev.cpu(), torch.from_numpy(body.copy()))
    # odd offsets and lengths, on a side stream
    s = torch.cuda.Stream()
    for off, n in [(1, 12345), (33 << 20, (32 << 20) + 7), (h["data_size"] - 5, 5), (777, 0)]:
        part = torch.zeros(max(n, 1), dtype=torch.uint8, device=DEV)
        torch.cuda.synchronize()  # the fill ran on the current stream, the upload goes to s
        f.upload(qgemv, part, offset=off, nbytes=n, stream=s)
        if n:
            assert np.array_equal(part.cpu().numpy(), body[off:off + n]), (off, n)


def test_gemv_on_weights_read_from_the_file(qgemv, tmp_path):
    path, _, host, x = _model(tmp_path)
    f = vx.GGUFFile(path)
    dev = torch.empty(f.header["data_size"], dtype=torch.uint8, device=DEV)
    f.upload(qgemv, dev)
    xb, xl = f.view("x", dev)            # ggml ne = [K, B] -> vortx [B, K]
    assert xl.dims() == (3, 1024)
    xv = (xb, xl.transpose(0, 1))        # the [K, B] operand of y = W x
    for name, (qt, M, w) in host.items():
        note(f"gguf gemv {name}")
        qw = f.qweight(name, dev)
        assert (qw.qtype, qw.rows, qw.cols) == (qt, M, 1024)
        y = torch.full((M, 3), float("nan"), device=DEV)
        qgemv.dispatch(y, qw, xv)
        torch.cuda.synchronize()
        assert_close(y.cpu().numpy(), O.gemv_q_f64(qt, w, M, 1024, x), what=name)
        # and decode straight from the uploaded bytes is the file's decode
        out = torch.empty((M, 1024), device=DEV)
        qgemv.dequantize(out, qw)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), O.dequant(qt, w, M, 1024).view(np.uint32))
    nb, nl = f.view("output_norm.weight", dev)
    assert nl.dims() == (1024,)
    assert np.array_equal(nb.cpu().numpy(), np.linspace(-1, 1, 1024, dtype=np.float32))


def test_upload_errors(qgemv, tmp_path):
    path, _, _, _ = _model(tmp_path)
    f = vx.GGUFFile(path)
    n = f.header["data_size"]
    dev = torch.empty(n, dtype=torch.uint8, device=DEV)
    L = vx.lib()
    assert L.vx_gguf_upload(qgemv._h, None, f._h, 1, n, dev.data_ptr()) == _ffi.VX_ERR_INVALID
    assert L.vx_gguf_upload(qgemv._h, None, f._h, n + 1, 0, dev.data_ptr()) == _ffi.VX_ERR_INVALID
    assert L.vx_gguf_upload(None, None, f._h, 0, n, dev.data_ptr()) == _ffi.VX_ERR_INVALID
    assert L.vx_gguf_upload(qgemv._h, None, None, 0, n, dev.data_ptr()) == _ffi.VX_ERR_INVALID
    assert L.vx_gguf_upload(qgemv._h, None, f._h, 0, n, None) == _ffi.VX_ERR_INVALID
    with pytest.raises(TypeError):
        f.upload(qgemv, dev[:n - 1])
