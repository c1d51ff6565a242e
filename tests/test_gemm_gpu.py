"""f32 GEMM through the C ABI on the GPU vs the CPU oracle.

Restates the reference's only GEMM test (src/linalg/gemm.rs:365-443:
256x256 matrix times a [256, 1] vector, |gpu - cpu| <= 1e-3 absolute) with
seeded inputs, then covers the routes (naive / GEMV / MFMA tiled), view
semantics (transposed, offset, strided, batched) and the BASELINE.json
shapes. Tolerance: normwise 1e-3 against float64 (tests/helpers.py); the
naive kernel is additionally bit-exact against the oracle's restatement of
the reference's f32 summation order.
"""
import numpy as np
import pytest
import torch

import vortx_amd as vx
from oracle import oracle as O
from tests.helpers import assert_close, note
from vortx_amd import synthetic as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _nan(*shape):
    return torch.full(shape, float("nan"), device=DEV)


def _f64(a, b, rows=None):
    return O.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), rows)


def test_reference_gemm_vector(gemm):
    """gpu_gemm_generic: m [256,256] * v [256] unsqueezed to [256,1]."""
    note("reference gemm 256x256 * 256x1")
    m = torch.rand((256, 256), generator=torch.Generator().manual_seed(0)).to(DEV)
    v = torch.rand((256,), generator=torch.Generator().manual_seed(1)).to(DEV).unsqueeze(1)
    out = _nan(256, 1)
    assert vx.Gemm.route(out, m, v) == vx.ROUTE_GEMV
    gemm.dispatch(out, m, v)
    torch.cuda.synchronize()
    ref = _f64(m, v)[0, 0]
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-3  # approx epsilon = 1e-3
    # the forced tiled kernel (what the reference runs here) agrees too
    out2 = _nan(256, 1)
    gemm.dispatch_tiled(out2, m, v)
    torch.cuda.synchronize()
    assert np.abs(out2.cpu().numpy() - ref).max() <= 1e-3


@pytest.mark.parametrize("M,N,K", [(17, 23, 45), (1, 1, 1), (31, 31, 300), (5, 40, 7)])
def test_naive_bit_exact_reference_order(gemm, M, N, K):
    note(f"naive {M}x{N}x{K}")
    a = S.uniform((M, K), 1, DEV)
    b = S.uniform((K, N), 2, DEV)
    c = _nan(M, N)
    gemm.dispatch_naive(c, a, b)
    torch.cuda.synchronize()
    ref = O.gemm_ref_f32(a.cpu().numpy(), b.cpu().numpy())
    assert np.array_equal(c.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(67, 33, 17), (128, 128, 16), (129, 257, 31), (300, 200, 1000),
                                   (1024, 1024, 1024), (64, 64, 1), (33, 129, 2)])
def test_tiled_parity(gemm, M, N, K):
    note(f"tiled {M}x{N}x{K}")
    a = S.uniform((M, K), M, DEV)
    b = S.uniform((K, N), N, DEV)
    c = _nan(M, N)
    gemm.dispatch(c, a, b)
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), _f64(a, b)[0, 0], what=f"{M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,tr_b", [(67, 33, 17, False), (128, 256, 16, False), (129, 257, 31, True),
                                        (300, 517, 129, False), (513, 1000, 100, True), (1024, 1024, 1024, False)])
def test_wide_tiles_match_narrow(gemm, M, N, K, tr_b):
    """The 128 x 256 tile kernels (chosen for shapes such as 4096^3, forced
    here with VX_GEMM_TILE_WIDE) and the 64 x 64 ones (chosen when the
    128 x 128 tiles are fewer than the CUs, e.g. 1024^3; VX_GEMM_TILE_SMALL)
    give the same bits as the 128 x 128 ones (VX_GEMM_TILE_NARROW) and as the
    default choice: each output is the same sum in the same order. Edge tiles
    in M, N and K."""
    note(f"wide tiles {M}x{N}x{K} trB={tr_b}")
    a = S.uniform((M, K), 5, DEV)
    b = S.uniform((N, K), 6, DEV).t() if tr_b else S.uniform((K, N), 6, DEV)
    c0, c1, c2, c3 = _nan(M, N), _nan(M, N), _nan(M, N), _nan(M, N)
    gemm.dispatch_ex(c0, a, b, tile="narrow")
    gemm.dispatch_ex(c1, a, b, tile="wide")
    gemm.dispatch(c2, a, b)
    gemm.dispatch_ex(c3, a, b, tile="small")
    torch.cuda.synchronize()
    assert torch.equal(c0.view(torch.int32), c1.view(torch.int32))
    assert torch.equal(c0.view(torch.int32), c2.view(torch.int32))
    assert torch.equal(c0.view(torch.int32), c3.view(torch.int32))
    assert_close(c1.cpu().numpy(), _f64(a, b.contiguous())[0, 0])


@pytest.mark.parametrize("tr_a,tr_b", [(False, True), (True, False), (True, True)])
def test_transposed_views(gemm, tr_a, tr_b):
    M, N, K = 200, 150, 130
    note(f"transposed views a={tr_a} b={tr_b}")
    a = S.uniform((K, M), 3, DEV).t() if tr_a else S.uniform((M, K), 3, DEV)
    b = S.uniform((N, K), 4, DEV).t() if tr_b else S.uniform((K, N), 4, DEV)
    c = _nan(M, N)
    gemm.dispatch(c, a, b)
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), _f64(a.contiguous(), b.contiguous())[0, 0])


def test_generic_strides_and_offsets(gemm):
    """Every operand a strided, offset view into a larger buffer."""
    M, N, K = 70, 90, 50
    note("generic strides/offsets")
    A = S.uniform((2 * M + 3, 3 * K), 5, DEV)
    B = S.uniform((K + 1, 2 * N + 1), 6, DEV)
    a = A[3::2, 1::3]
    b = B[1:, 1::2]
    C = _nan(M + 2, 3 * N)
    c = C[2:, ::3]
    gemm.dispatch(c, a, b)
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), _f64(a.contiguous(), b.contiguous())[0, 0])
    mask = torch.ones_like(C, dtype=torch.bool)
    mask[2:, ::3] = False
    assert torch.isnan(C[mask]).all(), "wrote outside the output view"


def test_explicit_layout_views(gemm):
    """(buffer, TensorLayout) views: offset carried by the layout like
    TensorRef::buffer (src/tensor/tensor_ref.rs:101-103)."""
    M, N, K = 48, 40, 36
    note("explicit layouts")
    buf_a = S.uniform((M * K + 10,), 7, DEV)
    buf_b = S.uniform((N * K + 3,), 8, DEV)
    la = vx.TensorLayout((M, K, 1, 1), (K, 1, 1, 1), 2, 10)
    lb = vx.TensorLayout.contiguous([N, K]).transpose(0, 1)  # [K, N] view of an N x K buffer
    lb = vx.TensorLayout(lb.size, lb.stride, lb.rank, 3)
    out = torch.full((M * N,), float("nan"), device=DEV)
    gemm.dispatch((out, vx.TensorLayout.contiguous([M, N])), (buf_a, la), (buf_b, lb))
    torch.cuda.synchronize()
    a = buf_a[10:].reshape(M, K)
    b = buf_b[3:].reshape(N, K).t()
    assert_close(out.reshape(M, N).cpu().numpy(), _f64(a, b.contiguous())[0, 0])


def test_batched(gemm):
    n, c, M, N, K = 2, 3, 65, 70, 40
    note("batched 2x3")
    a = S.uniform((n, c, M, K), 9, DEV)
    b = S.uniform((n, c, K, N), 10, DEV).transpose(2, 3).contiguous().transpose(2, 3)
    out = _nan(n, c, M, N)
    gemm.dispatch(out, a, b)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), O.gemm_f64(a.cpu().numpy(), b.contiguous().cpu().numpy()))
    out3 = _nan(c, M, 5)
    a3, b3 = a[0], S.uniform((c, K, 5), 11, DEV)
    gemm.dispatch(out3, a3, b3)  # rank 3, small N -> naive? (M >= 32 -> tiled)
    torch.cuda.synchronize()
    assert_close(out3.cpu().numpy(), O.gemm_f64(a3.cpu().numpy(), b3.cpu().numpy())[0])


def test_special_cases(gemm):
    note("special cases K=0, identity, zeros")
    M, N = 40, 50
    a0 = torch.empty((M, 0), device=DEV)
    b0 = torch.empty((0, N), device=DEV)
    c = _nan(M, N)
    gemm.dispatch(c, a0, b0)
    torch.cuda.synchronize()
    assert (c == 0).all(), "K = 0 must write zeros"
    eye = torch.eye(64, device=DEV)
    b = S.uniform((64, 96), 12, DEV)
    c = _nan(64, 96)
    gemm.dispatch(c, eye, b)
    torch.cuda.synchronize()
    assert torch.equal(c, b), "identity * B must be exact"
    z = torch.zeros((64, 64), device=DEV)
    c = _nan(64, 96)
    gemm.dispatch(c, z, b)
    torch.cuda.synchronize()
    assert (c == 0).all()
    # integer-valued operands: every product and partial sum is exact in f32
    ai = torch.randint(-8, 9, (96, 80), generator=torch.Generator().manual_seed(3)).float().to(DEV)
    bi = torch.randint(-8, 9, (80, 72), generator=torch.Generator().manual_seed(4)).float().to(DEV)
    c = _nan(96, 72)
    gemm.dispatch(c, ai, bi)
    torch.cuda.synchronize()
    exact = (ai.cpu().numpy().astype(np.int64) @ bi.cpu().numpy().astype(np.int64)).astype(np.float32)
    assert np.array_equal(c.cpu().numpy(), exact)


def test_empty_outputs_are_no_ops(gemm):
    """M = 0, N = 0 or an empty batch: nothing to write, success, no launch
    (the route is VX_ROUTE_EMPTY); a normal call afterwards is exact."""
    note("gemm empty outputs")
    for M, N, K in ((0, 50, 40), (40, 0, 40), (0, 0, 0)):
        gemm.dispatch(torch.empty((M, N), device=DEV), torch.empty((M, K), device=DEV), torch.empty((K, N), device=DEV))
    gemm.dispatch(torch.empty((0, 3, 4), device=DEV), torch.empty((0, 3, 5), device=DEV),
                  torch.empty((0, 5, 4), device=DEV))
    ai = torch.randint(-8, 9, (40, 24), generator=torch.Generator().manual_seed(5)).float().to(DEV)
    bi = torch.randint(-8, 9, (24, 36), generator=torch.Generator().manual_seed(6)).float().to(DEV)
    c = _nan(40, 36)
    gemm.dispatch(c, ai, bi)
    torch.cuda.synchronize()
    exact = (ai.cpu().numpy().astype(np.int64) @ bi.cpu().numpy().astype(np.int64)).astype(np.float32)
    assert np.array_equal(c.cpu().numpy(), exact)


def test_shape_mismatch_is_an_error(gemm):
    a = torch.zeros((40, 30), device=DEV)
    b = torch.zeros((31, 50), device=DEV)
    with pytest.raises(vx.VortxError, match="incompatible gemm shapes"):
        gemm.dispatch(torch.zeros((40, 50), device=DEV), a, b)
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        gemm.dispatch_naive(torch.zeros((40, 50), device=DEV), a, b)


CONFIGS = [(4096, 4096, 4096, False), (4096, 11008, 4096, False), (4096, 4096, 4096, True)]


@pytest.mark.parametrize("M,N,K,tr_b", CONFIGS, ids=["4096^3", "4096x11008x4096", "4096^3-Btransposed"])
def test_gemm_configs_full_f64(gemm, M, N, K, tr_b):
    """BASELINE.json shapes, every output checked against a float64 product
    (numpy's BLAS dgemm on the f32 operands, as the reference's own test
    compares every output, src/linalg/gemm.rs:365-443). The dgemm result is
    itself tied to the oracle's float64 loop (orc_gemm_f64) on 16 rows."""
    note(f"gemm config {M}x{N}x{K} trB={tr_b}")
    a = S.uniform((M, K), 21, DEV)
    b = S.uniform((N, K), 22, DEV).t() if tr_b else S.uniform((K, N), 22, DEV)
    c = _nan(M, N)
    gemm.dispatch(c, a, b)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    a64 = a.cpu().numpy().astype(np.float64)
    b64 = b.contiguous().cpu().numpy().astype(np.float64)
    ref = a64 @ b64
    del a64, b64
    rows = np.random.default_rng(0).choice(M, 16, replace=False).astype(np.uint32)
    orc = _f64(a, b.contiguous(), rows)[0, 0]
    assert np.abs(ref[rows.astype(np.int64)] - orc).max() <= 1e-9 * np.abs(orc).max(), "dgemm differs from the oracle"
    assert_close(got, ref, what=f"full {M}x{N}x{K}")
    # the reference test's own criterion, element by element: |out - ref| <= 1e-3
    assert np.abs(got - ref).max() <= 1e-3


def test_gemm_1024_config(gemm):
    """M = N = K = 1024, full float64 check."""
    note("gemm 1024^3")
    a = S.uniform((1024, 1024), 31, DEV)
    b = S.uniform((1024, 1024), 32, DEV)
    c = _nan(1024, 1024)
    gemm.dispatch(c, a, b)
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), _f64(a, b)[0, 0])


@pytest.mark.parametrize("M,K,pad", [(32, 4, 0), (37, 5, 3), (45, 256, 0), (300, 1000, 4), (129, 4096, 0),
                                     (61, 4099, 1), (33, 11008, 0), (1000, 16384, 0), (35, 20000, 0)])
def test_gemv_route_shapes(gemm, M, K, pad):
    """The N == 1 route (M >= 32; one row per workgroup from K = 4096, four below):
    ragged M and K (K % 4 != 0 with the rows padded to a multiple of 4),
    strided x; float64 reference, normwise tolerance."""
    note(f"f32 gemv {M}x{K} pad {pad}")
    buf = S.uniform((M, K + pad), 5, DEV)
    a = buf[:, :K]
    if (K + pad) % 4:
        pytest.skip("the route needs rows 16-byte aligned")
    xb = S.uniform((K, 3), 6, DEV)
    for x in (xb[:, :1].contiguous(), xb[:, 1:2]):  # contiguous and strided x
        out = _nan(M, 1)
        assert vx.Gemm.route(out, a, x) == vx.ROUTE_GEMV
        gemm.dispatch(out, a, x)
        torch.cuda.synchronize()
        ref = _f64(a, x)[0, 0]
        err = np.abs(out.cpu().numpy() - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err <= 1e-5, (M, K, err)


def test_gemv_route_batch_and_epilogue(gemm):
    """Batched A and x with alpha / beta: out = 0.5 A x + 2 out."""
    note("f32 gemv batch alpha beta")
    a = S.uniform((3, 700, 4096), 7, DEV)
    x = S.uniform((3, 4096, 1), 8, DEV)
    c0 = S.uniform((3, 700, 1), 9, DEV)
    out = c0.clone()
    gemm.dispatch_ex(out, a, x, alpha=0.5, beta=2.0)
    torch.cuda.synchronize()
    ref = 0.5 * (a.double() @ x.double()) + 2.0 * c0.double()
    err = ((out.double() - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-5, err
