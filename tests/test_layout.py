"""TensorLayout algebra through the C ABI (host only; no GPU).

The broadcast cases restate the reference's own unit tests
(src/shapes.rs:642-783) one for one; canonicalize / transpose / view /
narrow / unsqueeze / is_contiguous follow src/shapes.rs:85-465.
"""
import pytest

import vortx_amd as vx

L = vx.TensorLayout


def test_broadcast_same_shape():  # shapes.rs:646-653
    a, b = L.contiguous([3, 4]), L.contiguous([3, 4])
    ab, bb = a.broadcast(b)
    assert ab == a and bb == b


def test_broadcast_scalar_to_matrix():  # shapes.rs:655-669
    s, m = L.contiguous([1]).broadcast(L.contiguous([3, 4]))
    assert s.size == (1, 1, 1, 1) and m.size == (3, 4, 1, 1)
    assert s.rank == 2 and m.rank == 2
    assert s.stride[0] == 0 and s.stride[1] == 0


def test_broadcast_vector_to_matrix():  # shapes.rs:671-683
    v, m = L.contiguous([3, 1]).broadcast(L.contiguous([3, 4]))
    assert v.size == (3, 1, 1, 1) and m.size == (3, 4, 1, 1)
    assert v.stride[1] == 0


def test_broadcast_row_vector_to_matrix():  # shapes.rs:685-697
    v, m = L.contiguous([1, 4]).broadcast(L.contiguous([3, 4]))
    assert v.size == (1, 4, 1, 1) and m.size == (3, 4, 1, 1)
    assert v.stride[0] == 0


def test_broadcast_different_ranks():  # shapes.rs:699-716
    v, t = L.contiguous([2]).broadcast(L.contiguous([3, 4, 2]))
    assert v.rank == 3 and t.rank == 3
    assert v.size[:3] == (1, 1, 2)
    assert v.stride[0] == 0 and v.stride[1] == 0


def test_broadcast_incompatible_shapes():  # shapes.rs:718-727
    assert L.contiguous([3, 4]).broadcast(L.contiguous([8])) is None
    assert L.contiguous([3, 4]).broadcast(L.contiguous([3])) is None


def test_broadcast_incompatible_inner_dim():  # shapes.rs:729-734
    assert L.contiguous([3, 4]).broadcast(L.contiguous([3, 5])) is None


def test_broadcast_3d_tensors():  # shapes.rs:736-746
    a, b = L.contiguous([2, 1, 4]).broadcast(L.contiguous([2, 3, 4]))
    assert a.stride[1] == 0


def test_broadcast_preserves_order():  # shapes.rs:748-766
    a = L.contiguous([3, 4, 5])
    ab, bb = a.broadcast(L.contiguous([5]))
    assert ab == a
    assert bb.rank == 3 and bb.size[:3] == (1, 1, 5) and bb.stride[:3] == (0, 0, 1)


def test_broadcast_4d_tensors():  # shapes.rs:768-782
    a, b = L.contiguous([2, 3, 1, 5]), L.contiguous([2, 1, 4, 5])
    ab, bb = a.broadcast(b)
    assert ab.size == a.size and bb.size == b.size
    assert ab.rank == 4 and bb.rank == 4
    assert ab.stride[2] == 0 and bb.stride[1] == 0


def test_contiguous_and_canonicalize():
    l = L.contiguous([3, 4])
    assert l.size == (3, 4, 1, 1) and l.stride == (4, 1, 1, 1) and l.rank == 2
    c = l.canonicalize()
    assert c.size == (1, 1, 3, 4) and c.stride == (12, 12, 4, 1) and c.rank == 4
    # rank < 4 canonicalization drops the offset (it travels in the buffer slice)
    off = L((3, 4, 1, 1), (4, 1, 1, 1), 2, 7)
    assert off.canonicalize().offset == 0
    # rank 4 is returned unchanged, offset included
    r4 = L((2, 3, 4, 5), (60, 20, 5, 1), 4, 9)
    assert r4.canonicalize() == r4


def test_transpose_swaps_size_and_stride():
    t = L.contiguous([3, 4]).transpose(0, 1)
    assert t.size[:2] == (4, 3) and t.stride[:2] == (1, 4)
    assert not t.is_contiguous()
    with pytest.raises(vx.VortxError):
        L.contiguous([3, 4]).transpose(0, 2)


def test_view_narrow_unsqueeze():
    base = L.contiguous([4, 6])
    v = base.view(2, [3, 5])
    assert v.size[:2] == (3, 5) and v.stride[:2] == (5, 1) and v.offset == 2
    v2 = base.view(0, [2, 3], [10, None])
    assert v2.stride[:2] == (10, 1)
    with pytest.raises(vx.VortxError):
        base.view(0, [5, 5])  # needs 25 elements, has 24
    with pytest.raises(vx.VortxError):
        base.transpose(0, 1).view(0, [2, 2])  # non-contiguous source
    n = base.narrow(1, 2, 3)
    assert n.size[:2] == (4, 3) and n.offset == 2
    n0 = base.narrow(0, 1, 2)
    assert n0.offset == 6
    with pytest.raises(vx.VortxError):
        base.narrow(0, 3, 2)
    u = L.contiguous([256]).unsqueeze(1)  # Tensor::unsqueeze in the reference GEMM test
    assert u.size[:2] == (256, 1) and u.stride[:2] == (1, 1) and u.rank == 2
    u0 = L.contiguous([3, 4]).unsqueeze(0)
    assert u0.size[:3] == (1, 3, 4) and u0.stride[:3] == (4, 4, 1)


def test_is_contiguous_accepts_zero_strides():
    assert L((3, 4, 1, 1), (0, 1, 1, 1), 2, 0).is_contiguous()
    assert not L((3, 4, 1, 1), (5, 1, 1, 1), 2, 0).is_contiguous()
