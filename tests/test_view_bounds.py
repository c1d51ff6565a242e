"""Host-side bounds checks of the Python binding (no GPU needed).

The C ABI takes raw device pointers without sizes, so the binding refuses a
``(buffer, TensorLayout)`` view that reaches past its buffer and a QWeight
whose buffer is smaller than its rows need, before anything is launched.
"""
import pytest
import torch

import vortx_amd as vx
from vortx_amd import _ffi


def test_layout_extent_known_answers():
    L = vx.TensorLayout
    assert vx.layout_extent(L((3, 4), (4, 1), 2, 0)) == 12
    assert vx.layout_extent(L((3, 4), (4, 1), 2, 5)) == 17
    # transposed view of a [4, 3] buffer: last element at 2 * 1 + 3 * 3
    assert vx.layout_extent(L((3, 4), (1, 3), 2, 0)) == 12
    # broadcast (stride 0) dims add nothing
    assert vx.layout_extent(L((7, 4), (0, 1), 2, 0)) == 4
    # an empty dimension needs no storage at all
    assert vx.layout_extent(L((0, 4), (4, 1), 2, 9)) == 0
    # dims past the rank are ignored
    assert vx.layout_extent(L((5, 2, 9, 9), (2, 1, 100, 100), 2, 0)) == 10


@pytest.mark.parametrize("layout,ok", [
    (vx.TensorLayout((4, 4), (4, 1), 2, 0), True),
    (vx.TensorLayout((4, 4), (4, 1), 2, 1), False),     # offset pushes the last element out
    (vx.TensorLayout((4, 5), (4, 1), 2, 0), False),     # a row longer than its stride
    (vx.TensorLayout((4, 4), (1, 4), 2, 0), True),      # transposed, same extent
    (vx.TensorLayout((2, 2, 4), (16, 4, 1), 3, 0), False),
])
def test_view_pair_extent_is_checked_before_launch(layout, ok):
    buf = torch.zeros(16, dtype=torch.float32)  # CPU: only the checks run
    if ok:
        # in bounds: the next check (buffer on the GPU) is the one that fails here
        with pytest.raises(TypeError, match="GPU"):
            vx._view_of((buf, layout), False)
    else:
        with pytest.raises(vx.VortxError) as e:
            vx._view_of((buf, layout), False)
        assert e.value.status == _ffi.VX_ERR_INVALID


@pytest.mark.parametrize("qtype,rows,cols,stride,nbytes,ok", [
    (vx.VX_Q4_0, 4, 64, 0, 4 * 36, True),
    (vx.VX_Q4_0, 4, 64, 0, 4 * 36 - 1, False),
    (vx.VX_Q8_0, 3, 64, 80, 2 * 80 + 68, True),        # padded rows: the last row needs no padding
    (vx.VX_Q8_0, 3, 64, 80, 2 * 80 + 67, False),
    (vx.VX_Q4_K, 2, 512, 0, 2 * 288, True),
    (vx.VX_Q4_K, 2, 512, 0, 288, False),
    (vx.VX_Q4_0, 0, 64, 0, 0, True),                    # no rows: nothing to read
])
def test_qweight_buffer_size_is_checked(qtype, rows, cols, stride, nbytes, ok):
    data = torch.zeros(nbytes, dtype=torch.uint8)
    if ok:
        w = vx.QWeight(data, qtype, rows, cols, row_stride=stride)
        assert w.row_stride == (stride or cols // vx.qtype_info(qtype)[0] * vx.qtype_info(qtype)[1])
    else:
        with pytest.raises(vx.VortxError) as e:
            vx.QWeight(data, qtype, rows, cols, row_stride=stride)
        assert e.value.status == _ffi.VX_ERR_INVALID
