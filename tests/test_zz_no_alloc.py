"""vx_gemv_q_noalloc (the GEMV entry point that allocates nothing) against
vx_gemv_q_ex, both called through the C ABI: the same kernels on the same
inputs, so y must be identical bit for bit, on two calls in a row (the
second smaller, reusing the scratch the first one filled), and a split that
does not fit the scratch is refused before anything is launched."""
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


def _gemv(fn, ctx, y, w: vx.QWeight, x, flags=0):
    yv, xv, wc = vx._view_of(y, True), vx._view_of(x, False), w._c()
    return fn(ctx._h, C.c_void_p(torch.cuda.current_stream().cuda_stream), C.byref(yv), C.byref(wc), C.byref(xv),
              flags)


@pytest.mark.parametrize("flags", [0, vx._ffi.VX_GEMV_X_F32], ids=["int8-x", "f32-x"])
def test_noalloc_matches_gemv_q_ex_twice(qgemv, flags):
    L = vx.lib()
    cases = [(vx.VX_Q4_0, 1000, 4096, 8), (vx.VX_Q4_K, 300, 2048, 3), (vx.VX_Q8_0, 200, 1024, 1)]
    for qtype, M, K, B in cases:  # each call smaller than the one before
        note(f"noalloc {qtype} {M}x{K} B={B} flags={flags}")
        w = vx.QWeight(S.quant_weights(qtype, M, K, seed=M, device=DEV), qtype, M, K)
        x = S.activations(B, K, seed=K, device=DEV)
        y0 = torch.full((B, M), float("nan"), device=DEV)
        y1 = torch.full((B, M), float("nan"), device=DEV)
        assert _gemv(L.vx_gemv_q_ex, qgemv, y0.t(), w, x.t(), flags) == 0
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
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y2.t(), w2, x2.t()) == 0
    assert _gemv(vx.lib().vx_gemv_q_ex, qgemv, y3.t(), w2, x2.t()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int32), y3.view(torch.int32))


def test_noalloc_flag_errors(qgemv):
    M, K = 64, 256
    w = vx.QWeight(S.quant_weights(vx.VX_Q4_0, M, K, seed=1, device=DEV), vx.VX_Q4_0, M, K)
    x = S.activations(2, K, seed=2, device=DEV)
    y = torch.empty((2, M), device=DEV)
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y.t(), w, x.t(), 8) == vx._ffi.VX_ERR_INVALID
    assert _gemv(vx.lib().vx_gemv_q_noalloc, qgemv, y.t(), w, x.t(), 3) == vx._ffi.VX_ERR_INVALID
