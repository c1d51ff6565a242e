"""Launches captured into a HIP graph (stream capture) replay with their own
arguments: every replay, with eager work and synchronizations in between,
matches the eager results bit for bit."""
import pytest
import torch

import vortx_amd as vx
from tests.helpers import note
from vortx_amd import synthetic as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("B,use_ws", [(1, False), (4, False), (16, False), (16, True), (5, True)])
def test_gemv_graph_replay_matches_eager(qgemv, B, use_ws):
    """use_ws: one caller workspace shared by the captured launches (one
    stream, so in order); at these shapes (several passes at B = 16, three
    items with 5 columns) the split goes there."""
    M, n = 300, 6
    K = (12288 if B == 16 else 11008) if use_ws else 1024
    note(f"graph replay gemv B={B} workspace={use_ws}")
    ws = [S.quant_weights(vx.VX_Q4_K if B == 16 else vx.VX_Q4_0, M, K, seed=i, device=DEV) for i in range(n)]
    qt = vx.VX_Q4_K if B == 16 else vx.VX_Q4_0
    xs = [S.activations(B, K, seed=50 + i, device=DEV) for i in range(n)]
    ys = [torch.full((B, M), float("nan"), device=DEV) for _ in range(n)]
    wsp = vx.QuantGemv.workspace(vx.QWeight(ws[0], qt, M, K), B) if use_ws else None
    eager = []
    for i in range(n):
        qgemv.dispatch(ys[i].t(), vx.QWeight(ws[i], qt, M, K), xs[i].t(), workspace=wsp)
    torch.cuda.synchronize()
    eager = [y.clone() for y in ys]
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                qgemv.dispatch(ys[i].t(), vx.QWeight(ws[i], qt, M, K), xs[i].t(), stream=s, workspace=wsp)
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i in range(n):
            assert torch.equal(ys[i], eager[i]), f"replay {rep}, launch {i} differs from eager"
        _ = torch.ones(10, device=DEV).sum().item()  # eager work between replays


def test_gemm_graph_replay_matches_eager(gemm):
    note("graph replay gemm")
    a = [S.uniform((200, 96), i, DEV) for i in range(3)]
    b = [S.uniform((96, 150), 10 + i, DEV) for i in range(3)]
    c = [torch.full((200, 150), float("nan"), device=DEV) for _ in range(3)]
    for i in range(3):
        gemm.dispatch(c[i], a[i], b[i])
    torch.cuda.synchronize()
    eager = [t.clone() for t in c]
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(3):
                gemm.dispatch(c[i], a[i], b[i], stream=s)
    for rep in range(3):
        for t in c:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i in range(3):
            assert torch.equal(c[i], eager[i]), f"replay {rep}, launch {i}"
