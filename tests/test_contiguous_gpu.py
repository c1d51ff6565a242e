"""Strided -> contiguous copy (vortx's Contiguous op) on the GPU vs the
reference test and the CPU oracle (oracle/vx_oracle.c orc_contiguous_u32).

The copy moves 4-byte elements as bits, so every comparison is exact.
"""
import numpy as np
import pytest
import torch

import vortx_amd as vx
from oracle import oracle as O
from tests.helpers import note

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def cont():
    return vx.Contiguous(0)


def test_reference_contiguous_transpose(cont):
    """src/linalg/contiguous.rs:162-207: a 256x128 matrix viewed through
    transpose(0, 1) copied into a 128x256 output equals the row-major
    transpose (exact compare, as the reference asserts computed == expected)."""
    note("contiguous reference test")
    g = torch.Generator().manual_seed(7)
    t = torch.rand((256, 128), generator=g) * 2 - 1
    gpu_t = t.to(DEV)
    out = torch.rand((128, 256), generator=g).to(DEV)
    cont.launch(out, gpu_t.t())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), t.t().contiguous())


@pytest.mark.parametrize("shape,perm", [
    ((64, 48), (1, 0)),
    ((4096, 4096), (1, 0)),
    ((3, 130, 70), (2, 0, 1)),
    ((2, 3, 40, 33), (0, 3, 1, 2)),
    ((2, 3, 40, 33), (3, 2, 1, 0)),
    ((5, 1000), (1, 0)),
    ((1000, 5), (1, 0)),
    ((3, 200, 132), (0, 2, 1)),  # 16-byte 128x64 tiles: 3 slices, partial tiles
    ((2, 4100, 4096), (0, 2, 1)),  # 16-byte 128x128 tiles (>= 8 per CU), partial last w-tile
    ((130, 70), (1, 0)),         # H = 70 not a multiple of 4: the 4-byte tiles
    ((17,), (0,)),
])
def test_permuted_views_bit_exact(cont, shape, perm):
    note(f"contiguous permute {shape} {perm}")
    x = torch.randn(shape, device=DEV)
    v = x.permute(*perm)
    out = torch.full(v.shape, float("nan"), device=DEV)
    cont.launch(out, v)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.contiguous_u32(x.cpu().numpy().ravel(), tuple(v.shape), tuple(v.stride()), v.storage_offset())
    assert np.array_equal(got.view(np.uint32), ref.reshape(got.shape))
    assert torch.equal(out.cpu(), v.contiguous().cpu())


def test_strided_offset_and_broadcast_views(cont):
    """Sliced, stepped, offset and stride-0 (broadcast) sources."""
    buf = torch.randn(200000, device=DEV)
    cases = [((3, 50, 60), (20000, 300, 4), 11),
             ((40, 70), (0, 2), 5),            # broadcast rows
             ((6, 7, 8, 9), (1, 6, 42, 336), 100),
             ((123, 77), (150, 1), 7)]
    for shape, stride, off in cases:
        note(f"contiguous strided {shape} {stride} +{off}")
        lay = vx.TensorLayout(tuple(shape), tuple(stride), len(shape), off)
        out = torch.full(shape, float("nan"), device=DEV)
        cont.launch(out, (buf, lay))
        torch.cuda.synchronize()
        ref = O.contiguous_u32(buf.cpu().numpy(), shape, stride, off)
        assert np.array_equal(out.cpu().numpy().view(np.uint32).reshape(-1), ref.reshape(-1))


def test_device_offset_reads_the_raw_buffer(cont):
    """contiguous.rs:63-71: with the `offset` tensor the raw buffer is read
    at that device offset and the view's own offset is ignored."""
    buf = torch.arange(5000, dtype=torch.float32, device=DEV)
    lay = vx.TensorLayout((30, 40), (1, 30), 2, 999)   # view offset 999 must be ignored
    off = torch.tensor([123], dtype=torch.int32, device=DEV)
    out = torch.zeros((30, 40), device=DEV)
    cont.launch(out, (buf, lay), offset=off)
    torch.cuda.synchronize()
    ref = O.contiguous_u32(buf.cpu().numpy(), (30, 40), (1, 30), 123).view(np.float32)
    assert np.array_equal(out.cpu().numpy(), ref)
    # without it, the view offset applies
    cont.launch(out, (buf, lay))
    torch.cuda.synchronize()
    ref = O.contiguous_u32(buf.cpu().numpy(), (30, 40), (1, 30), 999).view(np.float32)
    assert np.array_equal(out.cpu().numpy(), ref)


def test_int32_elements_and_offset_output(cont):
    x = torch.randint(-2**31, 2**31 - 1, (70, 90), dtype=torch.int32, device=DEV)
    big = torch.zeros(70 * 90 + 13, dtype=torch.int32, device=DEV)
    out_lay = vx.TensorLayout((90, 70), (70, 1), 2, 13)
    cont.launch((big, out_lay), x.t())
    torch.cuda.synchronize()
    assert torch.equal(big[13:].view(90, 70).cpu(), x.t().contiguous().cpu())
    assert int(big[:13].abs().sum()) == 0


def test_errors_like_the_reference(cont):
    x = torch.randn(8, 9, device=DEV)
    with pytest.raises(vx.VortxError) as e:
        cont.launch(torch.empty(9, 9, device=DEV), x)
    assert e.value.status == vx._ffi.VX_ERR_SHAPE
    with pytest.raises(vx.VortxError) as e:
        cont.launch(torch.empty(9, 8, device=DEV).t(), x)
    assert e.value.status == vx._ffi.VX_ERR_SHAPE
    assert "Output tensor must be contiguous" in str(e.value)


def test_empty_is_a_no_op(cont):
    out = torch.full((0, 5), 1.0, device=DEV)
    cont.launch(out, torch.empty(5, 0, device=DEV).t())
    torch.cuda.synchronize()
