"""vx_gemm_f32_ex on the GPU: batch broadcasting (the reference's TODO at
src/linalg/gemm.rs:64, with TensorLayout::broadcast semantics,
src/shapes.rs:346-391) and the alpha / beta epilogue, on every route.

Broadcast results are checked against numpy's own broadcasting matmul in
float64 (independent of the oracle); tolerance normwise 1e-3. The naive
route is also bit-exact: the oracle's reference-order f32 sum S, then
(alpha * S) + (beta * C) with one f32 rounding per operation.
"""
import numpy as np
import pytest
import torch

import vortx_amd as vx
from oracle import oracle as O
from tests.helpers import assert_close, note
from vortx_amd import _ffi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rand(shape, seed):
    return torch.from_numpy(np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)).to(DEV)


# (lhs shape, rhs shape, out shape, route)
BCAST = [
    ((3, 150, 70), (70, 90), (3, 150, 90), vx.ROUTE_TILED),        # rhs shared by a batch of lhs
    ((150, 70), (4, 70, 90), (4, 150, 90), vx.ROUTE_TILED),        # lhs shared
    ((2, 1, 64, 48), (1, 3, 48, 40), (2, 3, 64, 40), vx.ROUTE_TILED),  # both dims, opposite sides
    ((5, 20, 30), (30, 12), (5, 20, 12), vx.ROUTE_NAIVE),
    ((1, 3, 9, 7), (2, 1, 7, 5), (2, 3, 9, 5), vx.ROUTE_NAIVE),
    ((256, 300), (6, 300, 1), (6, 256, 1), vx.ROUTE_GEMV),         # one matrix, a batch of vectors
    ((6, 256, 300), (300, 1), (6, 256, 1), vx.ROUTE_GEMV),
]


def _route(out, lhs, rhs):
    """The route the planner takes once the operands are expanded to out's batch."""
    nb = out.dim() - 2
    le = lhs.expand(*out.shape[:nb], *lhs.shape[-2:]) if lhs.dim() < out.dim() or lhs.shape[:nb] != out.shape[:nb] \
        else lhs
    re = rhs.expand(*out.shape[:nb], *rhs.shape[-2:]) if rhs.dim() < out.dim() or rhs.shape[:nb] != out.shape[:nb] \
        else rhs
    return vx.Gemm.route(out, le, re)


@pytest.mark.parametrize("ls,rs,os_,route", BCAST, ids=[f"{a}x{b}" for a, b, _, _ in BCAST])
def test_broadcast_matches_numpy(gemm, ls, rs, os_, route):
    note(f"gemm_ex broadcast {ls} x {rs} -> {os_}")
    lhs, rhs = _rand(ls, 1), _rand(rs, 2)
    out = torch.full(os_, float("nan"), device=DEV)
    assert _route(out, lhs, rhs) == route
    gemm.dispatch_ex(out, lhs, rhs, broadcast=True)
    torch.cuda.synchronize()
    ref = np.matmul(lhs.cpu().numpy().astype(np.float64), rhs.cpu().numpy().astype(np.float64))
    assert_close(out.cpu().numpy(), ref, what=f"broadcast {ls} x {rs}")
    # without the flag the reference's equality checks apply (src/linalg/gemm.rs:70-104)
    with pytest.raises(vx.VortxError) as e:
        gemm.dispatch_ex(out, lhs, rhs)
    assert e.value.status == _ffi.VX_ERR_SHAPE


def test_broadcast_incompatible_batches(gemm):
    note("gemm_ex broadcast errors")
    out = torch.empty((3, 16, 8), device=DEV)
    for l, r in [((2, 16, 4), (4, 8)), ((16, 4), (2, 4, 8)), ((3, 16, 5), (4, 8))]:
        with pytest.raises(vx.VortxError) as e:
            gemm.dispatch_ex(out, _rand(l, 3), _rand(r, 4), broadcast=True)
        assert e.value.status == _ffi.VX_ERR_SHAPE, (l, r)


# (M, N, K, rhs transposed) covering the naive, GEMV and several MFMA operand modes
EPI = [(20, 25, 33, False), (300, 1, 257, False), (257, 190, 129, False), (256, 256, 256, True),
       (130, 70, 50, "generic")]


@pytest.mark.parametrize("M,N,K,mode", EPI, ids=[f"{m}x{n}x{k}-{t}" for m, n, k, t in EPI])
@pytest.mark.parametrize("alpha,beta", [(0.5, -2.0), (-1.25, 0.75), (3.0, 1.0)])
def test_alpha_beta_epilogue(gemm, M, N, K, mode, alpha, beta):
    note(f"gemm_ex epilogue {M}x{N}x{K} {mode} alpha={alpha} beta={beta}")
    a = _rand((M, K), 5)
    if mode is True:
        b = _rand((N, K), 6).t()                  # B as a transposed [N, K] buffer
    elif mode == "generic":
        b = _rand((K, 2 * N), 6)[:, ::2]          # stride 2 along N: scalar loads
    else:
        b = _rand((K, N), 6)
    c0 = _rand((M, N), 7)
    out = c0.clone()
    gemm.dispatch_ex(out, a, b, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    an, bn, cn = (t.cpu().numpy().astype(np.float64) for t in (a, b, c0))
    ref = alpha * (an @ bn) + beta * cn
    assert_close(out.cpu().numpy(), ref, what="alpha/beta")
    if vx.Gemm.route(out, a, b) == vx.ROUTE_NAIVE:
        s32 = O.gemm_ref_f32(a.cpu().numpy(), b.cpu().numpy())
        want = np.float32(alpha) * s32 + np.float32(beta) * c0.cpu().numpy()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(20, 25, 33), (300, 1, 257), (257, 190, 129)])
def test_beta_zero_never_reads_out(gemm, M, N, K):
    note(f"gemm_ex beta 0 over NaN {M}x{N}x{K}")
    a, b = _rand((M, K), 8), _rand((K, N), 9)
    out = torch.full((M, N), float("nan"), device=DEV)
    gemm.dispatch_ex(out, a, b, alpha=2.0, beta=0.0)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), 2.0 * (a.cpu().numpy().astype(np.float64) @ b.cpu().numpy()), what="beta 0")


@pytest.mark.parametrize("M,N,K", [(20, 25, 33), (300, 1, 257), (257, 190, 129)])
def test_defaults_equal_dispatch_bit_for_bit(gemm, M, N, K):
    """alpha 1, beta 0 multiplies by exactly 1: the same bits as vx_gemm_f32."""
    note(f"gemm_ex defaults {M}x{N}x{K}")
    a, b = _rand((M, K), 10), _rand((K, N), 11)
    o1 = torch.full((M, N), float("nan"), device=DEV)
    o2 = torch.full((M, N), float("nan"), device=DEV)
    gemm.dispatch(o1, a, b)
    gemm.dispatch_ex(o2, a, b)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))
    # alpha 0, beta 1 leaves out exactly as it was
    gemm.dispatch_ex(o2, a, b, alpha=0.0, beta=1.0)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int32), o2.view(torch.int32))


def test_ex_argument_errors(gemm):
    note("gemm_ex argument errors")
    a, b = _rand((40, 30), 12), _rand((30, 50), 13)
    out = torch.empty((40, 50), device=DEV)
    o, l, r = vx._view_of(out, True), vx._view_of(a, False), vx._view_of(b, False)
    L = vx.lib()
    import ctypes as C
    bad = _ffi.VxGemmOpts(1.0, 0.0, 0, 1)          # reserved != 0
    assert L.vx_gemm_f32_ex(gemm._h, None, C.byref(o), C.byref(l), C.byref(r), C.byref(bad)) == _ffi.VX_ERR_INVALID
    bad = _ffi.VxGemmOpts(1.0, 0.0, 6, 0)          # unknown flag
    assert L.vx_gemm_f32_ex(gemm._h, None, C.byref(o), C.byref(l), C.byref(r), C.byref(bad)) == _ffi.VX_ERR_INVALID
    # an out that overlaps itself (stride 0 on a dim of size 50)
    row = torch.empty((40, 1), device=DEV).expand(40, 50)
    with pytest.raises(vx.VortxError) as e:
        gemm.dispatch_ex(row, a, b, beta=1.0)
    assert e.value.status == _ffi.VX_ERR_INVALID
    # NULL opts is vx_gemm_f32
    assert L.vx_gemm_f32_ex(gemm._h, None, C.byref(o), C.byref(l), C.byref(r), None) == _ffi.VX_OK
