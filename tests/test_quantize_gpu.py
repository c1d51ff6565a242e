"""f32 -> Q8_0 / Q4_0 / Q4_K quantize kernels vs the CPU oracle: the bytes
must be identical (same algorithm, same f32 operation order, no contraction,
IEEE division and square root, round-to-nearest-even f16)."""
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


def _edge_rows(K, rng):
    """Rows of blocks that are zero, constant, tiny, huge, one outlier,
    all-negative, f16-subnormal scale, near the f16 overflow edge."""
    rows = []
    base = rng.standard_normal(K).astype(np.float32)
    rows.append(np.zeros(K, np.float32))
    rows.append(np.full(K, 0.75, np.float32))
    rows.append(np.full(K, -3.0, np.float32))
    rows.append(base * 1e-6)
    rows.append(base * 1e3)
    r = base * 1e-3
    r[::37] = 50.0
    rows.append(r)
    rows.append(-np.abs(base))
    rows.append(base * 2.0 ** -20)
    rows.append(base * 2000.0)
    rows.append(np.abs(base) + 5.0)
    return np.stack(rows)


def _grid_rows(M, K, rng):
    """Super-blocks of exact grids x = s q - m (power-of-two s, m in {0, s/2, s, 2s},
    q = 0 and 15 in every 32): the Q4_K search's first candidate is an exact fit."""
    e = rng.integers(-8, 0, (M, K // 32))
    s = np.ldexp(np.float32(1), e).astype(np.float32)
    m = s * rng.choice(np.float32([0.0, 0.5, 1.0, 2.0]), (M, K // 32))
    q = rng.integers(0, 16, (M, K // 32, 32))
    q[:, :, 0], q[:, :, 1] = 0, 15
    return (s[..., None] * q - m[..., None]).astype(np.float32).reshape(M, K)


def _tie_rows(M, K, rng):
    """Blocks whose max is 127/16 (Q8_0: id = 16 exactly) and whose other values are
    odd multiples of 1/32, so x * id lands exactly on k + 1/2: rounding ties."""
    k = rng.integers(-127, 127, (M, K)).astype(np.float32)
    x = (k + np.float32(0.5)) / np.float32(16)
    x[:, ::32] = np.float32(127 / 16) * rng.choice(np.float32([-1, 1]), (M, K // 32))
    return x.astype(np.float32)


def _run(qg, qtype, x_np, strided=False):
    M, K = x_np.shape
    rb = S.row_bytes(qtype, K)
    out = torch.full((M, rb), 0xAB, dtype=torch.uint8, device=DEV)
    if strided:
        big = torch.zeros((M, K + 5), device=DEV)
        big[:, 3:3 + K] = torch.from_numpy(x_np)
        xv = big[:, 3:3 + K]
    else:
        xv = torch.from_numpy(x_np).to(DEV)
    qg.quantize(vx.QWeight(out, qtype, M, K), xv)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
@pytest.mark.parametrize("dist", ["normal", "uniform", "edges", "grid", "ties"])
def test_quantize_bytes_match_oracle(qgemv, qtype, dist):
    rng = np.random.default_rng(41)
    K = 1024
    if dist == "normal":
        x = rng.standard_normal((37, K)).astype(np.float32)
    elif dist == "uniform":
        x = rng.uniform(-1, 1, (37, K)).astype(np.float32)
    elif dist == "grid":
        x = _grid_rows(16, K, rng)
    elif dist == "ties":
        x = _tie_rows(16, K, rng)
    else:
        x = _edge_rows(K, rng)
    note(f"quantize {QN[qtype]} {dist}")
    got = _run(qgemv, qtype, x)
    ref = O.quantize(qtype, x)
    if not np.array_equal(got, ref):
        bad = np.argwhere(got != ref)
        pytest.fail(f"{len(bad)} bytes differ, first at {bad[:4].tolist()}")


@pytest.mark.parametrize("qtype", QTYPES, ids=lambda q: QN[q])
def test_quantize_strided_input_and_roundtrip(qgemv, qtype):
    """Non-contiguous x (scalar loads) gives the same bytes; quantize ->
    dequantize -> quantize is a fixed point; the GEMV on the result agrees
    with the f64 product of the dequantized matrix."""
    rng = np.random.default_rng(42)
    M, K = 65, 2048
    x = rng.standard_normal((M, K)).astype(np.float32)
    note(f"quantize strided {QN[qtype]}")
    got = _run(qgemv, qtype, x, strided=True)
    assert np.array_equal(got, O.quantize(qtype, x))
    wd = torch.from_numpy(got).to(DEV)
    dq = torch.empty((M, K), device=DEV)
    qgemv.dequantize(dq, vx.QWeight(wd, qtype, M, K))
    again = _run(qgemv, qtype, dq.cpu().numpy())
    assert np.array_equal(again, got)
    xv = S.activations(1, K, seed=43, device=DEV)
    y = torch.empty(M, device=DEV)
    qgemv.dispatch(y, vx.QWeight(wd, qtype, M, K), xv[0])
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), O.gemv_q_f64(qtype, got, M, K, xv.cpu().numpy())[:, 0])


def test_quantize_large_matches_oracle_rows(qgemv):
    """A 4096 x 4096 Q4_K quantize (the compute-heavy search) on the GPU,
    checked on 64 sampled rows."""
    rng = np.random.default_rng(44)
    x = rng.standard_normal((4096, 4096)).astype(np.float32)
    note("quantize q4_k 4096x4096")
    got = _run(qgemv, vx.VX_Q4_K, x)
    rows = rng.choice(4096, 64, replace=False)
    assert np.array_equal(got[rows], O.quantize(vx.VX_Q4_K, x[rows]))


def test_quantize_errors(qgemv):
    x = torch.randn(8, 64, device=DEV)
    out = torch.zeros((8, S.row_bytes(vx.VX_Q8_0, 64)), dtype=torch.uint8, device=DEV)
    with pytest.raises(vx.VortxError) as e:
        qgemv.quantize(vx.QWeight(out, vx.VX_Q8_0, 8, 64), x[:, :32])
    assert e.value.status == vx._ffi.VX_ERR_SHAPE
    with pytest.raises(vx.VortxError) as e:
        qgemv.quantize(vx.QWeight(out, vx.VX_Q8_0, 8, 64), x.reshape(-1))
    assert e.value.status == vx._ffi.VX_ERR_SHAPE


@pytest.mark.parametrize("qtype", [vx.VX_Q8_0, vx.VX_Q4_0], ids=lambda q: QN[q])
@pytest.mark.parametrize("layout", ["padded-rows", "unaligned-base"])
def test_quantize_output_layouts(qgemv, qtype, layout):
    """Rows padded past their blocks take per-block stores; dense rows are
    staged and copied out, with 2-byte stores when the output base is not
    16-byte aligned. Bytes equal the oracle's and nothing outside the blocks
    is written."""
    rng = np.random.default_rng(45)
    M, K = 45, 1024
    x = rng.standard_normal((M, K)).astype(np.float32)
    rb = S.row_bytes(qtype, K)
    note(f"quantize {QN[qtype]} {layout}")
    if layout == "padded-rows":
        buf = torch.full((M, rb + 6), 0xAB, dtype=torch.uint8, device=DEV)
        qw = vx.QWeight(buf, qtype, M, K, row_stride=rb + 6)
    else:
        flat = torch.full((M * rb + 16,), 0xAB, dtype=torch.uint8, device=DEV)
        buf = flat[2:2 + M * rb].view(M, rb)
        qw = vx.QWeight(buf, qtype, M, K)
    qgemv.quantize(qw, torch.from_numpy(x).to(DEV))
    torch.cuda.synchronize()
    ref = O.quantize(qtype, x)
    got = buf.cpu().numpy()
    assert np.array_equal(got[:, :rb], ref)
    if layout == "padded-rows":
        assert (got[:, rb:] == 0xAB).all(), "wrote into the row padding"
    else:
        f = flat.cpu().numpy()
        assert (f[:2] == 0xAB).all() and (f[2 + M * rb:] == 0xAB).all(), "wrote outside the output"


def test_quantize_q4_k_search_fixture(qgemv):
    """The designed Q4_K sub-blocks of tests/golden/q4k_search.json: the block
    whose result depends on the av_x + |x| weighting equals the fixture's
    bytes; a row of the search-winner sub-blocks equals the oracle's bytes."""
    import json
    import os
    fix = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4k_search.json")))
    x = np.zeros((2, 256), np.float32)
    x[0, :32] = np.array(fix["weighting_block"]["x0_bits"], np.uint32).view(np.float32)
    for i, c in enumerate(fix["fits"]):
        x[1, 32 * i:32 * i + 32] = np.array(c["x_bits"], np.uint32).view(np.float32)
    note("quantize q4_k search fixture")
    got = _run(qgemv, vx.VX_Q4_K, x)
    assert got[0].tobytes().hex() == fix["weighting_block"]["block_hex"]
    assert np.array_equal(got[1], O.quantize(vx.VX_Q4_K, x[1:2])[0])
