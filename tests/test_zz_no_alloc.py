"""vx_gemv_q_noalloc (the GEMV entry point that allocates nothing) against
vx_gemv_q_ws (the same routes with a caller workspace), both called through
the C ABI: the same kernels on the same inputs, so y must be identical bit
for bit and within tolerance of the oracle. The cases take the route that
splits x into memory (the shapes whose split does not fit the GEMV kernel's
registers), so
every call goes through the module's scratch array; they run largest first
after a call that fills almost all of the scratch with other data, so a
call that read stale scratch contents would show. A split that does not fit
the scratch is refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest
import torch

import vortx_amd as vx
from oracle import oracle as O
from tests.helpers import assert_close, note
from vortx_amd import synthetic as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _gemv(fn, ctx, y, w: vx.QWeight, x, flags=0):
    yv, xv, wc = vx._view_of(y, True), vx._view_of(x, False), w._c()
    return fn(ctx._h, _stream(), C.byref(yv), C.byref(wc), C.byref(xv), flags)


def _gemv_ws(ctx, y, w: vx.QWeight, x, ws, flags=0):
    yv, xv, wc = vx._view_of(y, True), vx._view_of(x, False), w._c()
    return vx.lib().vx_gemv_q_ws(ctx._h, _stream(), C.byref(yv), C.byref(wc), C.byref(xv), flags, ws.data_ptr(),
                                 ws.numel())


@pytest.mark.parametrize("flags", [0, vx._ffi.VX_GEMV_X_F32], ids=["int8-x", "f32-x"])
def test_noalloc_matches_gemv_q_ws_decreasing(qgemv, flags):
    L = vx.lib()
    # fill the scratch with the split of other data (4.1 of its 4 MiB)
    Kf, Bf, Mf = 28672, 64, 16
    wf = vx.QWeight(S.quant_weights(vx.VX_Q8_0, Mf, Kf, seed=5, device=DEV), vx.VX_Q8_0, Mf, Kf)
    xf = S.activations(Bf, Kf, seed=6, device=DEV) * 100.0
    yf = torch.empty((Bf, Mf), device=DEV)
    assert _gemv(L.vx_gemv_q_noalloc, qgemv, yf.t(), wf, xf.t()) == 0
    # shapes the GEMV cannot split x for itself (several passes, or three
    # items with 8 columns), largest split first: 442 KB, 198 KB, 124 KB
    cases = [(vx.VX_Q4_K, 2048, 12288, 16), (vx.VX_Q4_0, 4096, 11008, 8), (vx.VX_Q8_0, 512, 11008, 5)]
    for qtype, M, K, B in cases:
        note(f"noalloc {qtype} {M}x{K} B={B} flags={flags}")
        w = vx.QWeight(S.quant_weights(qtype, M, K, seed=M, device=DEV), qtype, M, K)
        x = S.activations(B, K, seed=K, device=DEV)
        ws = torch.empty(max(16, vx.QuantGemv.workspace_size(w, B, x_f32=bool(flags))), dtype=torch.uint8,
                         device=DEV)
        y0 = torch.full((B, M), float("nan"), device=DEV)
        y1 = torch.full((B, M), float("nan"), device=DEV)
        assert _gemv_ws(qgemv, y0.t(), w, x.t(), ws, flags) == 0
        assert _gemv(L.vx_gemv_q_noalloc, qgemv, y1.t(), w, x.t(), flags) == 0
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int32), y1.view(torch.int32)), (qtype, M, K, B)
        ref = O.gemv_q_f64(qtype, w.data.cpu().numpy(), M, K, x.cpu().numpy())
        assert_close(y1.cpu().numpy().T, ref, what=f"noalloc {qtype} {M}x{K} b{B}")


def test_noalloc_refuses_a_split_larger_than_its_scratch(qgemv):
    K, B, M = 32768, 64, 16  # vx_xq_size = 4.7 MB > 4 MiB
    assert vx.xq_size(K, B) > 4 << 20
    note("noalloc oversize")
    w = vx.QWeight(S.quant_weights(vx.VX_Q8_0, M, K, seed=1, device=DEV), vx.VX_Q8_0, M, K)
    x = S.activations(B, K, seed=2, device=DEV)
    y = torch.full((B, M), float("nan"), device=DEV)
    st = _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y.t(), w, x.t())
    torch.cuda.synchronize()
    assert st == vx._ffi.VX_ERR_UNSUPPORTED
    assert b"scratch" in vx.lib().vx_last_error_message()
    assert torch.isnan(y).all(), "an oversize call wrote y"
    # the largest split that fits (B = 64, K a multiple of 256) runs
    K2, B2 = 28928, 64
    assert vx.xq_size(K2, B2) <= 4 << 20 < vx.xq_size(K2 + 256, B2)
    w2 = vx.QWeight(S.quant_weights(vx.VX_Q8_0, M, K2, seed=3, device=DEV), vx.VX_Q8_0, M, K2)
    x2 = S.activations(B2, K2, seed=4, device=DEV)
    y2 = torch.empty((B2, M), device=DEV)
    y3 = torch.empty((B2, M), device=DEV)
    ws = torch.empty(vx.xq_size(K2, B2), dtype=torch.uint8, device=DEV)
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y2.t(), w2, x2.t()) == 0
    assert _gemv_ws(qgemv, y3.t(), w2, x2.t(), ws) == 0
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int32), y3.view(torch.int32))


def test_noalloc_flag_errors(qgemv):
    M, K = 64, 256
    w = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, K, seed=1, device=DEV), vx.VX_Q4_0, M, K)
    x = S.activations(2, K, seed=2, device=DEV)
    y = torch.empty((2, M), device=DEV)
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y.t(), w, x.t(), 8) == vx._ffi.VX_ERR_INVALID
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y.t(), w, x.t(), 3) == vx._ffi.VX_ERR_INVALID
