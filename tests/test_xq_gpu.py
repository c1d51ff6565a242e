"""Activation split (vx_quantize_x) and the batched GEMV on it (vx_gemv_q_xq).

The split must equal the oracle's bytes exactly (tests/test_oracle_xq.py
pins the oracle). The GEMV is checked on a split the ORACLE wrote, against a
float64 evaluation of what the kernel computes from that split (the
quantized part of W times the x the levels stand for, plus each block's
offset term times the exact block sum the split stores), so it is checked
apart from the x rounding: products of levels and weights are exact int32,
only the f32 scaling and accumulation round (tolerance below). The default
vx_gemv_q path at B >= 2 (split into the context's workspace + this GEMV)
is covered by tests/test_gemv_q_gpu.py against the float64 GEMV of x itself.
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
# f32 scaling and accumulation over K/32 block terms of an exact int32 dot:
# well below this (Q4_K subtracts its min term, which can cancel).
XQ_GEMV_TOL = 2e-5


def _logical_levels(q: vx.XQ) -> np.ndarray:
    """Device-layout levels [ceil(K/256), 4, 4, B, 2, 2, 8] (item, block pair,
    position group, column, level, block parity, byte) -> [K/32, B, 2, 32]
    (the oracle's layout); O.xq_device_levels is the inverse."""
    d = q.levels().cpu().numpy()
    ni, B = d.shape[0], d.shape[3]
    lv = d.transpose(0, 1, 5, 3, 4, 2, 6).reshape(ni * 8, B, 2, 32)
    return lv[:q.K // 32]


def _gpu_split(qgemv, x_bk: torch.Tensor, x_view=None) -> vx.XQ:
    B, K = x_bk.shape
    q = vx.XQ.empty(K, B)
    q.data.fill_(0xA5)
    qgemv.quantize_x(q, x_bk.t() if x_view is None else x_view)
    torch.cuda.synchronize()
    return q


@pytest.mark.parametrize("K,B", [(32, 1), (96, 3), (4096, 8), (11008, 4), (1024, 16), (2048, 21)])
def test_split_bytes_equal_oracle(qgemv, K, B):
    note(f"quantize_x K={K} B={B}")
    x = S.activations(B, K, seed=K + B, device=DEV)
    x[:, :32] *= 1e-3
    x[0, min(40, K - 1)] = 77.0
    q = _gpu_split(qgemv, x)
    lv, sc = O.quantize_x(x.cpu().numpy())
    assert np.array_equal(_logical_levels(q), lv), "levels differ from the oracle"
    assert np.array_equal(q.scales().cpu().numpy().view(np.uint32), sc.view(np.uint32)), "scales differ"


def test_split_edge_blocks_equal_oracle(qgemv):
    """Zero, subnormal, below 2^-100, huge, NaN and inf blocks, ties of the
    first rounding: bytes equal the oracle's, NaN scales included."""
    K, B = 512, 3
    note("quantize_x edge blocks")
    x = S.activations(B, K, seed=5, device=DEV)
    x[:, 0:32] = 0.0
    x[0, 32:64] = 1e-40                     # subnormal
    x[1, 64:96] *= 2.0 ** -105              # below the split threshold
    x[2, 96:128] *= 1e30
    x[0, 130] = float("nan")
    x[1, 170] = float("inf")
    x[2, 200] = -float("inf")
    x[0, 224:256] = torch.arange(-16, 16, dtype=torch.float32, device=DEV) + 0.5  # ties at max 15.5
    x[1, 256:288] = 126.0 * torch.linspace(-1, 1, 32, device=DEV)
    q = _gpu_split(qgemv, x)
    lv, sc = O.quantize_x(x.cpu().numpy())
    assert np.array_equal(_logical_levels(q), lv)
    assert np.array_equal(q.scales().cpu().numpy().view(np.uint32), sc.view(np.uint32))


def test_split_strided_x(qgemv):
    """x not contiguous along K (scalar loads) gives the same bytes."""
    K, B = 1024, 5
    note("quantize_x strided")
    x = S.activations(B, K, seed=9, device=DEV)
    xkb = torch.empty((K, 2 * B), device=DEV)
    xkb[:, ::2] = x.t()
    q = _gpu_split(qgemv, x, x_view=xkb[:, ::2])
    lv, sc = O.quantize_x(x.cpu().numpy())
    assert np.array_equal(_logical_levels(q), lv)
    assert np.array_equal(q.scales().cpu().numpy(), sc)


def _oracle_split_on_gpu(x_np: np.ndarray) -> tuple:
    lv, sc = O.quantize_x(x_np)
    B, K = x_np.shape
    q = vx.XQ.empty(K, B)
    raw = np.concatenate([O.xq_device_levels(lv).reshape(-1).view(np.uint8), sc.reshape(-1).view(np.uint8)])
    assert raw.size == vx.xq_size(K, B)
    q.data.copy_(torch.from_numpy(raw))
    return q, lv, sc


def _offset_coefficients(qtype: int, w: np.ndarray, M: int, K: int) -> np.ndarray:
    """[M, K/32] float64: the value a weight of each block (Q4_K: sub-block)
    has when its quant bits are 0, i.e. the coefficient of the block's sum of
    x: -8 d (Q4_0), -dmin m (Q4_K), 0 (Q8_0)."""
    qk, bb = O.QTYPE_INFO[qtype]
    wz = w.reshape(M, K // qk, bb).copy()
    if qtype == vx.VX_Q4_0:
        wz[:, :, 2:] = 0
    elif qtype == vx.VX_Q8_0:
        wz[:, :, 2:] = 0
    else:
        wz[:, :, 16:] = 0
    return O.dequant(qtype, wz.reshape(M, -1), M, K)[:, ::32].astype(np.float64)


def _xq_reference(qtype: int, w: np.ndarray, M: int, K: int, lv: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """[M, B] float64 product the kernel computes from a split: the weights'
    quantized part times x^ = c2 (254 q1 + q2), and each block's offset term
    (its zero-quant value, see _offset_coefficients) times the block's EXACT
    sum S stored in the split (not the sum of x^)."""
    wd = O.dequant(qtype, w, M, K).astype(np.float64)
    xhat = O.xq_decode_f64(lv, sc)                                  # [B, K]
    shat = xhat.reshape(xhat.shape[0], K // 32, 32).sum(-1)         # [B, K/32]
    s_exact = sc[:, :, 1].astype(np.float64).T                      # [B, K/32]
    return wd @ xhat.T + _offset_coefficients(qtype, w, M, K) @ (s_exact - shat).T


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K,B", [(131, 4096, 2), (300, 4096, 8), (70, 11008, 4), (45, 16384, 8), (64, 1536, 16),
                                   (257, 832, 5), (33, 4096, 13), (1, 4096, 3)])
def test_gemv_xq_on_oracle_split(qgemv, qtype, M, K, B):
    """Every route of the kernel: one pass (K <= 4096) and several (K = 11008,
    16384), one and two groups of 8 columns, odd column counts, a partial last
    item (K = 832, 1536: 13 and 24 units of 64), a single row."""
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"gemv_xq {QN[qtype]} {M}x{K} B={B}")
    w = S.quant_weights(qtype, M, K, seed=M + K, device=DEV)
    x = S.activations(B, K, seed=M + B, device=DEV).cpu().numpy()
    q, lv, sc = _oracle_split_on_gpu(x)
    y = torch.full((B, M), float("nan"), device=DEV)
    qgemv.dispatch_xq(y.t(), vx.QWeight(w, qtype, M, K), q)
    torch.cuda.synchronize()
    ref = _xq_reference(qtype, w.cpu().numpy(), M, K, lv, sc)
    assert_close(y.cpu().numpy().T, ref, tol=XQ_GEMV_TOL, what=f"{QN[qtype]} {M}x{K} b{B} vs the split")


def test_one_split_for_three_matrices(qgemv):
    """Quantize x once, multiply it by three matrices of different types: each
    y equals vx_gemv_q on the same x bit for bit (the same kernels on the same
    split), the use the entry point exists for (q / k / v projections)."""
    K, B = 4096, 6
    note("gemv_xq reuse")
    x = S.activations(B, K, seed=3, device=DEV)
    q = _gpu_split(qgemv, x)
    for qtype, M in ((vx.VX_Q4_0, 512), (vx.VX_Q8_0, 300), (vx.VX_Q4_K, 1024)):
        w = vx.QWeight(S.quant_weights(qtype, M, K, seed=M, device=DEV), qtype, M, K)
        y1 = torch.empty((B, M), device=DEV)
        y2 = torch.empty((B, M), device=DEV)
        qgemv.dispatch_xq(y1.t(), w, q)
        qgemv.dispatch(y2.t(), w, x.t(), workspace=vx.QuantGemv.workspace(w, B))
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int32), y2.view(torch.int32)), QN[qtype]


def test_xq_errors(qgemv):
    K, B, M = 256, 2, 16
    x = S.activations(B, K, seed=1, device=DEV)
    w = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, K, seed=2, device=DEV), vx.VX_Q4_0, M, K)
    q = vx.XQ.empty(K, B)
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        qgemv.quantize_x(vx.XQ.empty(K, B + 1), x.t())
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        qgemv.dispatch_xq(torch.empty((B, M + 1), device=DEV).t(), w, q)
    with pytest.raises(vx.VortxError, match="VX_ERR_SHAPE"):
        qgemv.dispatch_xq(torch.empty((B, M), device=DEV).t(), w, vx.XQ.empty(2 * K, B))
    with pytest.raises(vx.VortxError, match="VX_ERR_INVALID"):  # misaligned base
        bad = vx.XQ(torch.empty(vx.xq_size(K, B) + 16, dtype=torch.uint8, device=DEV)[4:], K, B)
        qgemv.quantize_x(bad, x.t())
    with pytest.raises(vx.VortxError, match="VX_ERR_UNSUPPORTED"):  # K % 64 != 0
        w96 = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, 96, seed=2, device=DEV), vx.VX_Q4_0, M, 96)
        q96 = vx.XQ.empty(96, B)
        qgemv.dispatch_xq(torch.empty((B, M), device=DEV).t(), w96, q96)
    with pytest.raises(vx.VortxError, match="VX_ERR_INVALID"):  # buffer too small
        vx.XQ(torch.empty(vx.xq_size(K, B) - 1, dtype=torch.uint8, device=DEV), K, B)


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("M,K,B", [(300, 4096, 8), (131, 4096, 2), (257, 832, 5), (64, 1536, 16), (45, 8192, 3),
                                   (70, 11008, 4), (33, 4096, 13), (100, 2048, 21), (16, 4096, 9),
                                   (300, 4096, 4), (257, 832, 3), (40, 2048, 4), (200, 8192, 7), (257, 12288, 4),
                                   (96, 4096, 16)])
def test_fused_split_equals_split_then_gemv(qgemv, qtype, M, K, B):
    """vx_gemv_q with x stored [B, K] (stride 1 along K) splits x inside the
    GEMV kernels (one launch); stored [K, B] it runs vx_quantize_x into the
    caller's workspace, then the GEMV on the split. Same bytes of x, same
    kernels otherwise: y is equal bit for bit. (The host fuses one pass with one item per wave at B <= 16, two
    at B <= 8 or three at B <= 4; the other shapes check that both storages
    take the split path and agree.)"""
    if K % O.QTYPE_INFO[qtype][0]:
        pytest.skip("K not a multiple of the block size")
    note(f"fused split {QN[qtype]} {M}x{K} B={B}")
    w = vx.QWeight(S.quant_weights(qtype, M, K, seed=M + K, device=DEV), qtype, M, K)
    x = S.activations(B, K, seed=B + 1, device=DEV)
    x[:, :32] = 0.0
    x[0, 32:64] *= 2.0 ** -110
    x[-1, 64:96] *= 1e25
    xkb = x.t().contiguous()  # [K, B] storage: stride B along K
    y1 = torch.full((B, M), float("nan"), device=DEV)
    y2 = torch.full((B, M), float("nan"), device=DEV)
    wsp = vx.QuantGemv.workspace(w, B)  # [K, B] storage: the split goes to the workspace
    qgemv.dispatch(y1.t(), w, x.t(), workspace=wsp)
    qgemv.dispatch(y2.t(), w, xkb, workspace=wsp)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    ref = O.gemv_q_f64(qtype, w.data.cpu().numpy(), M, K, x.cpu().numpy())
    assert_close(y1.cpu().numpy().T, ref, tol=2e-4, what=f"fused {QN[qtype]} {M}x{K} b{B}")


@pytest.mark.parametrize("B,bad", [(6, (1, 4)), (4, (1, 3))])
def test_fused_split_non_finite_column(qgemv, B, bad):
    """A NaN / inf in x reaches every y of its column on the fused path too,
    and only that column, the same way the split path does (B <= 4 runs the
    fused form whose lanes split half the blocks each)."""
    M, K = 200, 4096
    note(f"fused split non-finite B={B}")
    w = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, K, seed=3, device=DEV), vx.VX_Q4_0, M, K)
    x = S.activations(B, K, seed=4, device=DEV)
    x[bad[0], 100] = float("nan")
    x[bad[1], 3000] = float("inf")
    y1 = torch.empty((B, M), device=DEV)
    y2 = torch.empty((B, M), device=DEV)
    wsp = vx.QuantGemv.workspace(w, B)  # [K, B] storage: the split goes to the workspace
    qgemv.dispatch(y1.t(), w, x.t(), workspace=wsp)
    qgemv.dispatch(y2.t(), w, x.t().contiguous(), workspace=wsp)
    torch.cuda.synchronize()
    good = [c for c in range(B) if c not in bad]
    fin = torch.isfinite(y1)
    assert not fin[bad[0]].any() and not fin[bad[1]].any()
    assert fin[good].all()
    assert torch.equal(torch.isfinite(y2), fin)
    assert torch.equal(y1[good].view(torch.int32), y2[good].view(torch.int32))


def _sweep_cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        qtype = QTYPES[rng.integers(len(QTYPES))]
        qk = 256 if qtype == vx.VX_Q4_K else 64
        K = int(qk * rng.integers(1, 12288 // qk + 1))
        M = int(rng.choice([rng.integers(1, 40), rng.integers(40, 600), rng.integers(600, 3000)]))
        B = int(rng.integers(2, 17))
        if M * K * B <= 40_000_000:
            cases.append((qtype, M, K, B))
    return cases


_SWEEP = _sweep_cases()


@pytest.mark.parametrize("qtype,M,K,B", _SWEEP, ids=[f"{QN[q]}-{m}x{k}-b{b}" for q, m, k, b in _SWEEP])
def test_batched_random_shapes(qgemv, qtype, M, K, B):
    """Seeded random shapes across every batched route (fused one-launch
    kernels, split + GEMV with one or two column groups, one or several
    passes, partial tiles and items): x stored [B, K] and [K, B] give the same
    bits, and both stay within the tolerance of the exact f64 product."""
    note(f"batched sweep {QN[qtype]} {M}x{K} B={B}")
    w = vx.QWeight(S.quant_weights(qtype, M, K, seed=M * 7 + K, device=DEV), qtype, M, K)
    x = S.activations(B, K, seed=M + 3 * B, device=DEV)
    y1 = torch.full((B, M), float("nan"), device=DEV)
    y2 = torch.full((B, M), float("nan"), device=DEV)
    wsp = vx.QuantGemv.workspace(w, B)  # [K, B] storage: the split goes to the workspace
    qgemv.dispatch(y1.t(), w, x.t(), workspace=wsp)
    qgemv.dispatch(y2.t(), w, x.t().contiguous(), workspace=wsp)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    ref = O.gemv_q_f64(qtype, w.data.cpu().numpy(), M, K, x.cpu().numpy())
    assert_close(y1.cpu().numpy().T, ref, tol=2e-4, what=f"{QN[qtype]} {M}x{K} b{B}")
