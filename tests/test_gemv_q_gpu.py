"""Block-quantized GEMV and dequantize on the GPU vs the CPU oracle.

Decode must be bit-exact (every Q8_0 / Q4_0 / Q4_K weight is exactly
representable in f32); GEMV outputs must be within normwise 1e-3 of the
float64 oracle. The reference has no quantized path, so these are pinned by
the oracle, itself pinned in tests/test_oracle.py.
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
QTYPES = [vx.VX_Q4_0, vx.VX_Q8_0, vx.VX_Q4_K]
QN = {vx.VX_Q4_0: "q4_0", vx.VX_Q8_0: "q8_0", vx.VX_Q4_K: "q4_k"}


def _special_scales(w: np.ndarray, qtype: int) -> np.ndarray:
    """Overwrite some block scales with edge values: f16 subnormals, -0,
    negative, zero, the largest finite half."""
    qk, bb = O.QTYPE_INFO[qtype]
    M, rb = w.shape
    blocks = w.reshape(M, rb // bb, bb).copy()
    specials = np.array([0x0001, 0x03FF, 0x8000, 0xBC00, 0x0000, 0x7BFF, 0x0400, 0x8001], dtype=np.uint16)
    for i, s in enumerate(specials):
        r, b = i % M, (3 * i) % blocks.shape[1]
        blocks[r, b, 0] = s & 0xFF
        blocks[r, b, 1] = s >> 8
        if qtype == vx.VX_Q4_K:  # dmin too
            blocks[r, b, 2] = specials[-1 - i] & 0xFF
            blocks[r, b, 3] = specials[-1 - i] >> 8
    return blocks.reshape(M, rb)


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_dequantize_bit_exact(qgemv, qtype):
    M, K = 37, 1024
    note(f"dequantize {QN[qtype]} {M}x{K}")
    w = _special_scales(S.quant_weights(qtype, M, K, seed=11).numpy(), qtype)
    wd = torch.from_numpy(w).to(DEV)
    out = torch.full((M, K), float("nan"), device=DEV)
    qgemv.dequantize(out, vx.QWeight(wd, qtype, M, K))
    torch.cuda.synchronize()
    ref = O.dequant(qtype, w, M, K)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "decode differs from the oracle bit pattern"


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_dequantize_strided_output(qgemv, qtype):
    M, K = 9, 512
    note(f"dequantize strided {QN[qtype]}")
    w = S.quant_weights(qtype, M, K, seed=12)
    big = torch.full((K, 2 * M), float("nan"), device=DEV)
    out_view = big[:, 1::2].t()  # [M, K] with strides (2, 2M)
    qgemv.dequantize(out_view, vx.QWeight(w.to(DEV), qtype, M, K))
    torch.cuda.synchronize()
    ref = O.dequant(qtype, w.numpy(), M, K)
    assert np.array_equal(out_view.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert torch.isnan(big[:, 0::2]).all(), "wrote outside the view"


def _run_gemv(qgemv, qtype, M, K, B, seed=0, x_kb=None, y_out=None, x_int8=False, x_f32=False, ws=True):
    """One GEMV; ws: with a workspace (vx_gemv_q_ws, the int8 split at every
    batched shape) or without (vx_gemv_q_ex)."""
    w = S.quant_weights(qtype, M, K, seed=seed, device=DEV)
    x = S.activations(B, K, seed=seed + 1, device=DEV)
    y = torch.full((B, M), float("nan"), device=DEV) if y_out is None else y_out
    xv = x.t() if x_kb is None else x_kb(x)
    yv = y.t() if y_out is None else y
    qw = vx.QWeight(w, qtype, M, K)
    wsp = vx.QuantGemv.workspace(qw, B) if ws else None
    qgemv.dispatch(yv, qw, xv, x_int8=x_int8, x_f32=x_f32, workspace=wsp)
    torch.cuda.synchronize()
    ref = O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy())
    return yv.cpu().numpy(), ref


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 8, 16, 21])
# (93, 832): 13 units of 64, so the batched kernel's last round is ragged
# (Q4_K skips: K is not a multiple of 256); (1, 4096): a single row.
# (61, 8128) and (57, 16384): two passes of 64 units (the last one partial)
# and four, the batch-1 kernel's K limit.
@pytest.mark.parametrize("M,K", [(131, 4096), (70, 11008), (257, 1536), (93, 832), (1, 4096), (61, 8128),
                                 (57, 16384)])
def test_gemv_parity_small(qgemv, qtype, B, M, K):
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"gemv {QN[qtype]} M={M} K={K} B={B}")
    got, ref = _run_gemv(qgemv, qtype, M, K, B, seed=M + K + B)
    assert_close(got, ref, what=f"{QN[qtype]} {M}x{K} b{B}")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K", [(9000, 8192), (5000, 16384), (4097, 11008)])
def test_gemv_b1_multipass_several_rows(qgemv, qtype, M, K):
    """Batch 1 with K > 4096 (several passes of 64 units per row) and more
    rows than the grid has waves, so a wave's items run across rows and
    passes through both ring slots."""
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"gemv b1 multipass {QN[qtype]} M={M} K={K}")
    got, ref = _run_gemv(qgemv, qtype, M, K, 1, seed=M + K)
    assert_close(got, ref, what=f"{QN[qtype]} {M}x{K} b1")


# BASELINE.json configs at full size.
FULL = [
    (vx.VX_Q8_0, 4096, 4096, 1), (vx.VX_Q8_0, 4096, 4096, 8),
    (vx.VX_Q4_0, 11008, 4096, 1), (vx.VX_Q4_0, 11008, 4096, 4), (vx.VX_Q4_0, 11008, 4096, 8),
    (vx.VX_Q4_0, 4096, 11008, 1), (vx.VX_Q4_0, 4096, 11008, 4), (vx.VX_Q4_0, 4096, 11008, 8),
    (vx.VX_Q4_K, 14336, 4096, 1), (vx.VX_Q4_K, 14336, 4096, 16),
    (vx.VX_Q4_K, 32000, 4096, 1), (vx.VX_Q4_K, 32000, 4096, 16),
]


@pytest.mark.parametrize("qtype,M,K,B", FULL, ids=[f"{QN[q]}-{m}x{k}-b{b}" for q, m, k, b in FULL])
def test_gemv_parity_configs(qgemv, qtype, M, K, B):
    note(f"gemv config {QN[qtype]} {M}x{K} b{B}")
    got, ref = _run_gemv(qgemv, qtype, M, K, B, seed=7)
    assert_close(got, ref, what=f"{QN[qtype]} {M}x{K} b{B}")
    if B == 1:
        # the exact-f32 batch-1 kernel: f32 accumulation only, so 1e-5 holds
        note(f"gemv config f32-x {QN[qtype]} {M}x{K}")
        got, ref = _run_gemv(qgemv, qtype, M, K, B, seed=8, x_f32=True)
        assert_close(got, ref, tol=1e-5, what=f"f32-x {QN[qtype]} {M}x{K}")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K", [(131, 4096), (70, 11008), (257, 1536), (33, 64 * 300)])
def test_gemv_int8x_path_small(qgemv, qtype, M, K):
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"gemv int8-x {QN[qtype]} M={M} K={K}")
    got, ref = _run_gemv(qgemv, qtype, M, K, 1, seed=M + K, x_int8=True)
    assert_close(got, ref, what="int8-x path")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_gemv_x_edge_values(qgemv, qtype):
    """Both batch-1 x modes (int8 levels, f32) with x blocks that are all
    zero, tiny, huge, or one large outlier among small values; K spanning
    several LDS chunks (the per-row-group kernels)."""
    M, K = 40, 64 * 300
    note(f"gemv i8 edge x {QN[qtype]}")
    w = S.quant_weights(qtype, M, K, seed=3, device=DEV)
    x = S.activations(1, K, seed=4, device=DEV)
    x[0, 0:32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e30
    x[0, 96:128] *= 1e-3
    x[0, 100] = 50.0
    y = torch.full((M,), float("nan"), device=DEV)
    ref = O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy())[:, 0]
    for x_f32 in (False, True):
        y.fill_(float("nan"))
        qgemv.dispatch(y, vx.QWeight(w, qtype, M, K), x[0], x_f32=x_f32)
        torch.cuda.synchronize()
        assert_close(y.cpu().numpy(), ref, what=f"x_f32={x_f32}")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K", [(40, 4096), (11008, 4096), (600, 8192)], ids=["one-item", "one-pass", "two-pass"])
def test_gemv_persistent_x_edge_values(qgemv, qtype, M, K):
    """The persistent batch-1 kernels (one item per wave, one pass, several
    passes) with x blocks that are all zero, tiny above and below 2^-100
    (the latter stored as zero levels), huge, subnormal, or one large outlier
    among small values, split in the kernel; y within tolerance of the
    float64 product."""
    note(f"gemv persistent edge x {QN[qtype]} M={M} K={K}")
    w = S.quant_weights(qtype, M, K, seed=13, device=DEV)
    x = S.activations(1, K, seed=14, device=DEV)
    x[0, 0:32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e-33
    x[0, 96:128] *= 1e30
    x[0, 128:160] *= 1e-3
    x[0, 140] = 50.0
    x[0, 160:192] = 1e-40
    x[0, K - 32:K] *= 1e-20
    y = torch.full((M,), float("nan"), device=DEV)
    ref = O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy())[:, 0]
    qgemv.dispatch(y, vx.QWeight(w, qtype, M, K), x[0])
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), ref, what="persistent int8-x")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("B", [2, 5, 8, 9])
def test_gemv_batched_x_edge_values(qgemv, qtype, B):
    """Batched (matrix-core) path: per column, blocks of x that are zero,
    tiny, huge or hold one outlier. x is split per 32-block into two int8
    levels there (error <= max|x_blk| / 64008 per element), so each column
    is checked on its own at the spec tolerance and at 2e-4."""
    M, K = 70, 4096
    note(f"gemv batched edge x {QN[qtype]} B={B}")
    w = S.quant_weights(qtype, M, K, seed=21, device=DEV)
    x = S.activations(B, K, seed=22, device=DEV)
    x[:, 0:32] = 0.0
    x[1::2, 32:64] *= 1e-30
    x[0::2, 64:96] *= 1e30
    x[:, 96:128] *= 1e-3
    x[:, 100] = 50.0
    ref = O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy())
    qw = vx.QWeight(w, qtype, M, K)
    for wsp in (None, vx.QuantGemv.workspace(qw, B)):
        y = torch.full((B, M), float("nan"), device=DEV)
        qgemv.dispatch(y.t(), qw, x.t(), workspace=wsp)
        torch.cuda.synchronize()
        got = y.cpu().numpy().T
        for b in range(B):
            assert_close(got[:, b], ref[:, b], what=f"column {b}")
            assert_close(got[:, b], ref[:, b], tol=2e-4, what=f"column {b} (two-level bound)")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("path", ["f32", "rows", "rows-f32"])
def test_gemv_alternate_kernels(qgemv, qtype, path):
    """The exact-f32 kernels (VX_GEMV_X_F32, every batch size) and the
    per-row-group batch-1 kernels that take over when x does not fit the
    persistent kernel's LDS (K > 16384; int8 or f32 x). The f32-x kernels
    accumulate in f32 only and are held to 1e-5."""
    M = 131
    K = 16640 if path.startswith("rows") else 4096
    x_f32 = path in ("f32", "rows-f32")
    Bs = [1] if path.startswith("rows") else [1, 2, 4, 8, 16]
    w = S.quant_weights(qtype, M, K, seed=31, device=DEV)
    wn = w.cpu().numpy()
    for B in Bs:
        note(f"gemv {path} {QN[qtype]} K={K} B={B}")
        x = S.activations(B, K, seed=32 + B, device=DEV)
        y = torch.full((B, M), float("nan"), device=DEV)
        qgemv.dispatch(y.t(), vx.QWeight(w, qtype, M, K), x.t(), x_f32=x_f32)
        torch.cuda.synchronize()
        ref = O.gemv_q_f64(qtype, wn, M, K, x.cpu().numpy())
        tol = 1e-5 if x_f32 else 1e-4
        assert_close(y.cpu().numpy().T, ref, tol=tol, what=f"{path} B={B}")


def test_gemv_flag_errors(qgemv):
    M, K = 64, 4096
    w = S.quant_weights(vx.VX_Q4_0, M, K, seed=1, device=DEV)
    x = S.activations(1, K, seed=2, device=DEV)
    y = torch.empty((M,), device=DEV)
    with pytest.raises(vx.VortxError) as e:
        qgemv.dispatch(y, vx.QWeight(w, vx.VX_Q4_0, M, K), x[0], x_f32=True, x_int8=True)
    assert e.value.status == vx._ffi.VX_ERR_INVALID
    yv, xv, wc = vx._view_of(y, True), vx._view_of(x[0], False), vx.QWeight(w, vx.VX_Q4_0, M, K)._c()
    import ctypes as C
    assert vx.lib().vx_gemv_q_ex(qgemv._h, None, C.byref(yv), C.byref(wc), C.byref(xv), 4) == vx._ffi.VX_ERR_INVALID


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_gemv_generic_paths(qgemv, qtype):
    """Odd block counts, padded (unaligned) row strides and strided x / y
    take the byte-level fallback or the scalar x staging."""
    qk, bb = O.QTYPE_INFO[qtype]
    K = 3 * qk if qtype != vx.VX_Q4_K else 512
    M, B = 45, 3
    note(f"gemv generic {QN[qtype]} K={K}")
    w = S.quant_weights(qtype, M, K, seed=5).numpy()
    rb = w.shape[1]
    padded = np.zeros((M, rb + 2), dtype=np.uint8)  # row stride not a multiple of 4
    padded[:, :rb] = w
    wd = torch.from_numpy(padded).to(DEV)
    x = S.activations(B, K, seed=6, device=DEV)
    xbig = torch.zeros((K, 2 * B), device=DEV)
    xbig[:, ::2] = x.t()
    y = torch.full((M, 2 * B), float("nan"), device=DEV)
    qgemv.dispatch(y[:, 1::2], vx.QWeight(wd, qtype, M, K, row_stride=rb + 2), xbig[:, ::2])
    torch.cuda.synchronize()
    ref = O.gemv_q_f64(qtype, w, M, K, x.cpu().numpy())
    assert_close(y[:, 1::2].cpu().numpy(), ref, what="generic")
    assert torch.isnan(y[:, 0::2]).all()


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("x_f32", [False, True], ids=["int8x", "f32x"])
# on 256 CUs: one item per wave (_p1e), two one-pass items (ring of one),
# two and three passes (ring of two; Q8_0 with two items: ring of one)
@pytest.mark.parametrize("M,K", [(300, 4096), (5000, 4096), (600, 8192), (131, 11008)])
def test_gemv_b1_strided_x_matches_contiguous(qgemv, qtype, x_f32, M, K):
    """Batch 1 with x not contiguous along K (stride 3) runs the strided-x
    (_xs) form of the persistent kernels: y equals the contiguous-x run bit
    for bit (the same values staged and split in the same order) and the
    oracle within tolerance."""
    note(f"gemv b=1 strided-x {QN[qtype]} {M}x{K} x_f32={x_f32}")
    w = S.quant_weights(qtype, M, K, seed=31, device=DEV)
    x = S.activations(1, K, seed=32, device=DEV)
    qw = vx.QWeight(w, qtype, M, K)
    y0 = torch.full((1, M), float("nan"), device=DEV)
    qgemv.dispatch(y0.t(), qw, x.t(), x_f32=x_f32)
    xk3 = torch.full((K, 3), float("nan"), device=DEV)
    xk3[:, 0] = x[0]
    y1 = torch.full((1, M), float("nan"), device=DEV)
    qgemv.dispatch(y1.t(), qw, xk3[:, :1], x_f32=x_f32)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
    assert_close(y1.t().cpu().numpy(), O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy()))


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_gemv_strided_x_fast_weights(qgemv, qtype):
    """Aligned weights with x not contiguous along K (scalar staging)."""
    M, K, B = 64, 4096, 2
    note(f"gemv strided-x {QN[qtype]}")
    got, ref = _run_gemv(qgemv, qtype, M, K, B, seed=9, x_kb=lambda x: x.t().contiguous())
    assert_close(got, ref)
    w = S.quant_weights(qtype, M, K, seed=19, device=DEV)
    x = S.activations(B, K, seed=20, device=DEV)
    xkb = torch.empty((K, 3 * B), device=DEV)
    xkb[:, ::3] = x.t()
    y = torch.full((M, B), float("nan"), device=DEV)
    qgemv.dispatch(y, vx.QWeight(w, qtype, M, K), xkb[:, ::3])
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy()))


def test_gemv_shape_errors(qgemv):
    M, K = 8, 64
    w = vx.QWeight(torch.zeros((M, K // 32 * 18), dtype=torch.uint8, device=DEV), vx.VX_Q4_0, M, K)
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        qgemv.dispatch(torch.zeros(M + 1, device=DEV), w, torch.zeros(K, device=DEV))
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        qgemv.dispatch(torch.zeros(M, device=DEV), w, torch.zeros(K + 1, device=DEV))
    bad = vx.QWeight(w.data, vx.VX_Q4_0, M, K)
    bad.qtype = 3  # not a supported GGML type
    with pytest.raises(vx.VortxError, match="VX_ERR_INVALID"):
        qgemv.dispatch(torch.zeros(M, device=DEV), bad, torch.zeros(K, device=DEV))


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("B", [1, 3, 8])
@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -float("inf")], ids=["nan", "inf", "-inf"])
def test_non_finite_x_reaches_its_column_only(qgemv, qtype, B, bad):
    """One non-finite value in column 0 of x makes every y of that column
    non-finite, on the int8 path at batch 1 and on the batched kernel; the
    other columns equal a run without it, bit for bit."""
    M, K = 300, 2048
    note(f"gemv non-finite x {QN[qtype]} B={B} {bad}")
    w = vx.QWeight(S.quant_weights(qtype, M, K, seed=5, device=DEV), qtype, M, K)
    x = S.activations(B, K, seed=6, device=DEV)
    wsp = vx.QuantGemv.workspace(w, B)
    y0 = torch.empty((B, M), device=DEV)
    qgemv.dispatch(y0.t(), w, x.t(), workspace=wsp)
    xb = x.clone()
    xb[0, 777] = bad
    y = torch.empty((B, M), device=DEV)
    qgemv.dispatch(y.t(), w, xb.t(), workspace=wsp)
    torch.cuda.synchronize()
    assert not torch.isfinite(y[0]).any(), "a non-finite x value was lost"
    if B > 1:
        assert torch.equal(y[1:].view(torch.int32), y0[1:].view(torch.int32))


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("path", ["k-large", "k-large-f32", "x-f32", "batched-f32"])
@pytest.mark.parametrize("bad", [float("nan"), float("inf")], ids=["nan", "inf"])
def test_non_finite_x_other_paths(qgemv, qtype, path, bad):
    """The same on the other routes: batch 1 with K > 16384 (the per-row-group
    kernels, int8 or f32 x), f32 x at batch 1 (VX_GEMV_X_F32) and the
    exact-f32 batched kernels (VX_GEMV_X_F32 with B = 3)."""
    M = 96
    K = 16640 if path.startswith("k-large") else 2048
    B = 3 if path == "batched-f32" else 1
    x_f32 = path != "k-large"
    note(f"gemv non-finite x {QN[qtype]} path={path} {bad}")
    w = vx.QWeight(S.quant_weights(qtype, M, K, seed=5, device=DEV), qtype, M, K)
    x = S.activations(B, K, seed=6, device=DEV)
    x[0, K - 5] = bad
    y = torch.empty((B, M), device=DEV)
    qgemv.dispatch(y.t(), w, x.t(), x_f32=x_f32)
    torch.cuda.synchronize()
    assert not torch.isfinite(y[0]).any(), "a non-finite x value was lost"
    if B > 1:
        assert torch.isfinite(y[1:]).all()


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_gemv_without_workspace(qgemv, qtype):
    """vx_gemv_q_ex without a workspace: batched shapes the GEMV kernel can
    split itself (one item per wave, <= 8 columns, x of stride 1 along K)
    give the bits of the workspace route; the others keep x in f32 (held to
    the f32 kernels' 1e-5), or, asked for the int8 split explicitly, fail
    with VX_ERR_UNSUPPORTED and launch nothing."""
    M = 300
    # (K, B, fused): one item per wave (up to 16 columns), two items with up
    # to 8 columns or three with up to 4 fuse; three items with 8 columns,
    # several passes (K past 16 waves x items) or more than 16 columns need
    # the split in memory
    big = 12288 if qtype == vx.VX_Q4_K else 11008
    for K, B, fused in ((4096, 4, True), (2048, 8, True), (4096, 16, True), (8192, 3, True), (big, 8, False),
                        (4096, 20, False)):
        note(f"gemv no-workspace {QN[qtype]} K={K} B={B}")
        w = torch.from_numpy(S.quant_weights(qtype, M, K, seed=42 + K).numpy()).to(DEV)
        qw = vx.QWeight(w, qtype, M, K)
        x = S.activations(B, K, seed=43, device=DEV)
        y0 = torch.full((B, M), float("nan"), device=DEV)
        y1 = torch.full((B, M), float("nan"), device=DEV)
        qgemv.dispatch(y0.t(), qw, x.t(), workspace=vx.QuantGemv.workspace(qw, B))
        qgemv.dispatch(y1.t(), qw, x.t())
        torch.cuda.synchronize()
        ref = O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy())
        assert_close(y0.cpu().numpy().T, ref, what="workspace route")
        if fused:
            assert torch.equal(y0.view(torch.int32), y1.view(torch.int32)), "fused route differs from the split"
        else:
            assert_close(y1.cpu().numpy().T, ref, tol=1e-5, what="f32-x fallback")
            y2 = torch.full((B, M), float("nan"), device=DEV)
            with pytest.raises(vx.VortxError, match="VX_ERR_UNSUPPORTED"):
                qgemv.dispatch(y2.t(), qw, x.t(), x_int8=True)
            torch.cuda.synchronize()
            assert torch.isnan(y2).all(), "a refused call wrote y"


def test_gemv_workspace_errors(qgemv):
    M, K, B = 64, 8192, 4
    qw = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, K, seed=1, device=DEV), vx.VX_Q4_0, M, K)
    x = S.activations(B, K, seed=2, device=DEV)
    y = torch.empty((B, M), device=DEV)
    need = vx.QuantGemv.workspace_size(qw, B)
    assert need == vx.xq_size(K, B) and vx.QuantGemv.workspace_size(qw, 1) == 0
    assert vx.QuantGemv.workspace_size(qw, B, x_f32=True) == 0
    small = torch.empty(need - 16, dtype=torch.uint8, device=DEV)
    with pytest.raises(vx.VortxError, match="VX_ERR_INVALID"):
        qgemv.dispatch(y.t(), qw, x.t(), workspace=small)
    big = torch.empty(need + 16, dtype=torch.uint8, device=DEV)
    with pytest.raises(vx.VortxError, match="VX_ERR_INVALID"):  # not 16-byte aligned
        qgemv.dispatch(y.t(), qw, x.t(), workspace=big[4:])


def test_gemv_two_streams_own_workspaces(qgemv):
    """One context, two streams, each with its own workspace, running
    interleaved batched GEMVs that need the split in memory: every result
    equals the serial run bit for bit (the context holds no per-call state)."""
    cases = [(vx.VX_Q4_K, 2048, 12288, 16), (vx.VX_Q4_0, 1024, 11008, 8), (vx.VX_Q8_0, 512, 8192, 12)]
    data = []
    for i, (qt, M, K, B) in enumerate(cases):
        qw = vx.QWeight(S.quant_weights(qt, M, K, seed=50 + i, device=DEV), qt, M, K)
        data.append((qw, S.activations(B, K, seed=60 + i, device=DEV), B, M))
    serial = []
    ws0 = torch.empty(max(vx.QuantGemv.workspace_size(qw, B) for qw, _, B, _ in data), dtype=torch.uint8, device=DEV)
    for qw, x, B, M in data:
        y = torch.empty((B, M), device=DEV)
        qgemv.dispatch(y.t(), qw, x.t(), workspace=ws0)
        serial.append(y)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [torch.empty_like(ws0), torch.empty_like(ws0)]
    outs = [[torch.full((B, M), float("nan"), device=DEV) for qw, x, B, M in data] for _ in range(2)]
    torch.cuda.current_stream().synchronize()
    for rep in range(4):
        for si in (0, 1):
            for ci in (range(len(data)) if si == 0 else reversed(range(len(data)))):
                qw, x, B, M = data[ci]
                qgemv.dispatch(outs[si][ci].t(), qw, x.t(), stream=streams[si], workspace=wss[si])
    torch.cuda.synchronize()
    for si in (0, 1):
        for ci in range(len(data)):
            assert torch.equal(outs[si][ci].view(torch.int32), serial[ci].view(torch.int32)), (si, ci)


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K", [(11008, 4096), (37, 8192), (4096, 4096)])
def test_read_probe_stays_in_its_rows(qgemv, qtype, M, K):
    """vx_gemv_q_read_probe (measurement kernel) writes exactly y[0..M)."""
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"read probe {QN[qtype]} {M}x{K}")
    qw = vx.QWeight(S.quant_weights(qtype, M, K, seed=3, device=DEV), qtype, M, K)
    y = torch.full((M + 64,), float("nan"), device=DEV)
    qgemv.read_probe(y, qw)
    torch.cuda.synchronize()
    assert not torch.isnan(y[:M]).any(), "a row was not written"
    assert torch.isnan(y[M:]).all(), "wrote past the rows"


def test_launch_floor_runs_eager_and_captured(qgemv):
    """vx_launch_floor (measurement kernel) launches and completes, eagerly
    and replayed from a HIP graph, and touches no memory it is not given."""
    note("launch floor")
    sentinel = torch.full((1024,), 7.0, device=DEV)
    for _ in range(3):
        qgemv.launch_floor()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(4):
                qgemv.launch_floor(stream=s)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    assert torch.equal(sentinel, torch.full((1024,), 7.0, device=DEV))


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_gemv_empty_shapes(qgemv, qtype):
    """Empty shapes, as the GEMM treats them (K = 0 writes zeros, nothing to
    write is a no-op): K = 0 gives y = 0 at B = 1 and B = 3 (with and without
    a workspace, int8 and f32 x); M = 0 and B = 0 launch nothing and return
    success; dequantize of 0 rows likewise. A normal call afterwards still
    matches the oracle."""
    qk, bb = O.QTYPE_INFO[qtype]
    M, K = 70, 2 * qk if qtype == vx.VX_Q4_K else 256
    note(f"gemv empty shapes {QN[qtype]}")
    w0 = vx.QWeight(torch.empty((M, 0), dtype=torch.uint8, device=DEV), qtype, M, 0)
    for B in (1, 3):
        for x_f32 in (False, True):
            x = torch.empty((B, 0), device=DEV)
            for ws in (None, vx.QuantGemv.workspace(w0, B)):
                y = torch.full((B, M), float("nan"), device=DEV)
                qgemv.dispatch(y[0] if B == 1 else y.t(), w0, x[0] if B == 1 else x.t(), x_f32=x_f32, workspace=ws)
                torch.cuda.synchronize()
                assert (y == 0).all(), f"K = 0 must write zeros (B={B}, x_f32={x_f32}, workspace={ws is not None})"
    wm = vx.QWeight(torch.empty((0, K // qk * bb), dtype=torch.uint8, device=DEV), qtype, 0, K)
    qgemv.dispatch(torch.empty(0, device=DEV), wm, S.activations(1, K, seed=3, device=DEV)[0])
    qgemv.dispatch(torch.empty((3, 0), device=DEV).t(), wm, S.activations(3, K, seed=4, device=DEV).t())
    qgemv.dequantize(torch.empty((0, K), device=DEV), wm)
    w = S.quant_weights(qtype, M, K, seed=5, device=DEV)
    qw = vx.QWeight(w, qtype, M, K)
    y = torch.full((M, 0), float("nan"), device=DEV)
    qgemv.dispatch(y, qw, torch.empty((K, 0), device=DEV))
    qgemv.dispatch(y, qw, torch.empty((K, 0), device=DEV), workspace=vx.QuantGemv.workspace(qw, 4))
    # the library is still in a good state
    x = S.activations(2, K, seed=6, device=DEV)
    y = torch.full((2, M), float("nan"), device=DEV)
    qgemv.dispatch(y.t(), qw, x.t())
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy().T, O.gemv_q_f64(qtype, w.cpu().numpy(), M, K, x.cpu().numpy()))
