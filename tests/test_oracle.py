"""CPU tests that pin the oracle (oracle/vx_oracle.c) before it is trusted.

* f16 -> f32: all 65536 bit patterns against numpy's binary16 conversion.
* Block decode: the hand-built known-answer blocks of tests/golden, plus
  invariants a plausible mistake breaks: one-hot nibble positions, exact
  linearity in d, the Q4_0 / Q8_0 identity (a Q4_0 block equals the Q8_0
  block holding nibble - 8 with the same d), and Q4_K scale unpacking over
  every 6-bit value.
* GEMM: the reference-order f32 restatement and the f64 contraction against
  numpy (BLAS) float64 matmul, integer-exact products, closed forms (K = 0,
  identity, outer product K = 1) and strided / transposed views.
* GEMV: the f64 oracle against numpy's float64 product of the decoded
  matrix; the CPU-baseline kernels against the oracle.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_f16_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(bits)
    exp = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def _golden():
    with open(os.path.join(GOLDEN, "quant_known_answers.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden(), ids=lambda c: c["name"])
def test_decode_known_answers(case):
    blk = np.frombuffer(bytes.fromhex(case["block"]), np.uint8)[None, :]
    qk, bb = O.QTYPE_INFO[case["qtype"]]
    assert blk.shape[1] == bb
    got = O.dequant(case["qtype"], blk, 1, qk)[0]
    exp = np.array(case["expected"], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), np.nonzero(got != exp)


def test_q4k_scale_unpack_matches_golden():
    case = [c for c in _golden() if c["name"] == "q4k_highbits"][0]
    sc12 = bytes.fromhex(case["block"])[4:16]
    for s in range(8):
        assert O.q4k_scale_min(sc12, s) == (case["scales"][s], case["mins"][s])


def _q4k_pack(sc, m):
    b = [0] * 12
    for s in range(4):
        b[s] = (sc[s] & 63) | ((sc[s + 4] >> 4) << 6)
        b[s + 4] = (m[s] & 63) | ((m[s + 4] >> 4) << 6)
        b[s + 8] = (sc[s + 4] & 15) | ((m[s + 4] & 15) << 4)
    return bytes(b)


def test_q4k_scale_unpack_every_value():
    rng = np.random.default_rng(0)
    for v in range(64):
        sc = list(rng.integers(0, 64, 8))
        m = list(rng.integers(0, 64, 8))
        s = v % 8
        sc[s], m[(s + 3) % 8] = v, 63 - v
        packed = _q4k_pack(sc, m)
        for t in range(8):
            assert O.q4k_scale_min(packed, t) == (sc[t], m[t])


def test_q4_0_one_hot_positions():
    """A single non-zero (q - 8) lands at element j (low nibble) or j + 16."""
    for j in range(16):
        for hi in (False, True):
            qs = bytearray([0x88] * 16)
            qs[j] = (0x8F if not hi else 0xF8)
            blk = np.frombuffer(bytes.fromhex("003c") + bytes(qs), np.uint8)[None, :]
            got = O.dequant(O.Q4_0, blk, 1, 32)[0]
            nz = np.nonzero(got)[0]
            assert list(nz) == [j + 16 * hi] and got[nz[0]] == 7.0


def test_q4k_one_hot_positions():
    """Byte l of chunk c: low nibble -> element 64c + l, high -> 64c + 32 + l."""
    sc = [1] * 8
    m = [0] * 8
    head = bytes.fromhex("003c") + bytes.fromhex("0000") + _q4k_pack(sc, m)
    for c in range(4):
        for l in (0, 7, 31):
            for hi in (False, True):
                qs = bytearray(128)
                qs[32 * c + l] = 0x50 if hi else 0x05
                blk = np.frombuffer(head + bytes(qs), np.uint8)[None, :]
                got = O.dequant(O.Q4_K, blk, 1, 256)[0]
                nz = np.nonzero(got)[0]
                assert list(nz) == [64 * c + 32 * hi + l] and got[nz[0]] == 5.0


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K])
def test_decode_linear_in_d(qtype):
    """Doubling d (and dmin) doubles every decoded weight exactly."""
    qk, bb = O.QTYPE_INFO[qtype]
    rng = np.random.default_rng(qtype)
    w = rng.integers(0, 256, size=(16, 4 * bb), dtype=np.uint8)
    blocks = w.reshape(16, 4, bb)
    d = np.abs(rng.standard_normal((16, 4, 2 if qtype == O.Q4_K else 1))).astype(np.float16) + np.float16(0.01)
    blocks[..., 0:d.shape[-1] * 2] = d.view(np.uint8).reshape(16, 4, -1)
    base = O.dequant(qtype, blocks.reshape(16, -1), 16, 4 * qk)
    blocks2 = blocks.copy()
    blocks2[..., 0:d.shape[-1] * 2] = (d * np.float16(2)).view(np.uint8).reshape(16, 4, -1)
    dbl = O.dequant(qtype, blocks2.reshape(16, -1), 16, 4 * qk)
    assert np.array_equal(dbl, 2 * base)


def test_q4_0_equals_q8_0_with_centered_nibbles():
    rng = np.random.default_rng(5)
    nib = rng.integers(0, 16, size=(8, 32))
    d = np.abs(rng.standard_normal(8)).astype(np.float16)
    q40 = np.zeros((8, 18), np.uint8)
    q80 = np.zeros((8, 34), np.uint8)
    q40[:, 0:2] = d.view(np.uint8).reshape(8, 2)
    q80[:, 0:2] = d.view(np.uint8).reshape(8, 2)
    q40[:, 2:] = nib[:, :16] | (nib[:, 16:] << 4)
    q80[:, 2:] = (nib - 8).astype(np.int8).view(np.uint8)
    assert np.array_equal(O.dequant(O.Q4_0, q40, 8, 32), O.dequant(O.Q8_0, q80, 8, 32))


# ------------------------------------------------------------------ gemm
@pytest.mark.parametrize("M,N,K", [(67, 33, 17), (1, 1, 1), (64, 64, 64), (5, 130, 257)])
def test_gemm_oracles_vs_numpy(M, N, K):
    rng = np.random.default_rng(M * N * K)
    a = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(O.gemm_f64(a, b)[0, 0], ref, rtol=1e-12, atol=1e-12)
    got = O.gemm_ref_f32(a, b)
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max()) * K ** 0.5


def test_gemm_ref_order_is_sequential_f32():
    """The restatement accumulates k = 0..K-1 in f32 with one rounding per op."""
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, (3, 50)).astype(np.float32)
    b = rng.uniform(-1, 1, (50, 4)).astype(np.float32)
    exp = np.zeros((3, 4), np.float32)
    for i in range(3):
        for j in range(4):
            s = np.float32(0)
            for k in range(50):
                s = np.float32(s + np.float32(a[i, k] * b[k, j]))
            exp[i, j] = s
    assert np.array_equal(O.gemm_ref_f32(a, b).view(np.uint32), exp.view(np.uint32))


def test_gemm_integer_golden():
    with open(os.path.join(GOLDEN, "gemm_int_small.json")) as f:
        g = json.load(f)
    a = np.array(g["a"], np.float32)
    b = np.array(g["b"], np.float32)
    c = np.array(g["c"], np.float32)
    assert np.array_equal(O.gemm_ref_f32(a, b), c)
    assert np.array_equal(O.gemm_f64(a, b)[0, 0], c.astype(np.float64))


def test_gemm_closed_forms():
    rng = np.random.default_rng(2)
    b = rng.uniform(-1, 1, (6, 5)).astype(np.float32)
    assert np.array_equal(O.gemm_ref_f32(np.eye(6, dtype=np.float32), b), b)
    a0 = np.zeros((4, 0), np.float32)
    b0 = np.zeros((0, 3), np.float32)
    assert np.array_equal(O.gemm_ref_f32(a0, b0), np.zeros((4, 3), np.float32))
    u = rng.uniform(-1, 1, (7, 1)).astype(np.float32)
    v = rng.uniform(-1, 1, (1, 9)).astype(np.float32)
    assert np.array_equal(O.gemm_ref_f32(u, v), (u * v).astype(np.float32))


def test_gemm_strided_and_batched_views():
    rng = np.random.default_rng(4)
    A = rng.uniform(-1, 1, (2, 3, 40, 30)).astype(np.float32)
    Bt = rng.uniform(-1, 1, (2, 3, 20, 30)).astype(np.float32)
    b = Bt.transpose(0, 1, 3, 2)  # transposed view, no copy
    ref = np.einsum("ncik,nckj->ncij", A.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(O.gemm_f64(A, b), ref, rtol=1e-12)
    np.testing.assert_allclose(O.gemm_ref_f32(A, b), ref, rtol=1e-4, atol=1e-5)
    a_str = A[0, 0, ::2, ::3]
    np.testing.assert_allclose(O.gemm_f64(a_str, b[0, 0, ::3, :])[0, 0],
                               a_str.astype(np.float64) @ b[0, 0, ::3, :].astype(np.float64), rtol=1e-12)


def test_cpu_baseline_tiled_matches_reference_order():
    """The OpenMP restatement of gemm_tiled keeps the k order: bit-exact."""
    rng = np.random.default_rng(6)
    a = rng.uniform(-1, 1, (100, 70)).astype(np.float32)
    b = rng.uniform(-1, 1, (70, 90)).astype(np.float32)
    assert np.array_equal(O.gemm_tiled_f32_omp(a, b, 2).view(np.uint32), O.gemm_ref_f32(a, b).view(np.uint32))


# ------------------------------------------------------------------ gemv
@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K])
def test_gemv_oracle_vs_numpy(qtype):
    M, K, B = 37, 512, 3
    rng = np.random.default_rng(qtype)
    w = rng.integers(0, 256, size=(M, O.row_bytes(qtype, K)), dtype=np.uint8)
    qk, bb = O.QTYPE_INFO[qtype]
    blocks = w.reshape(M, K // qk, bb)
    nd = 2 if qtype == O.Q4_K else 1  # d (and dmin) kept in a realistic range
    blocks[..., 0:2 * nd] = (np.abs(rng.standard_normal((M, K // qk, nd))) * 0.01).astype(np.float16).view(
        np.uint8).reshape(M, K // qk, 2 * nd)
    x = rng.standard_normal((B, K)).astype(np.float32)
    W = O.dequant(qtype, w, M, K).astype(np.float64)
    ref = W @ x.T.astype(np.float64)
    np.testing.assert_allclose(O.gemv_q_f64(qtype, w, M, K, x), ref, rtol=1e-12, atol=1e-12)
    got = O.gemv_q_f32_omp(qtype, w, M, K, x, 2)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("shape,stride,offset", [
    ((7,), (3,), 2),
    ((5, 6), (1, 5), 0),            # transposed 6x5
    ((4, 3, 5), (1, 0, 4), 1),      # a broadcast axis (stride 0)
    ((2, 3, 4, 5), (70, 20, 5, 1), 0),
    ((2, 3, 4, 5), (1, 2, 6, 24), 3),
])
def test_oracle_contiguous_matches_numpy(shape, stride, offset):
    """orc_contiguous_u32 (contiguous.rs:70-90) vs numpy's as_strided copy."""
    rng = np.random.default_rng(5)
    span = offset + sum((s - 1) * st for s, st in zip(shape, stride)) + 1
    buf = rng.standard_normal(span + 4).astype(np.float32)
    ref = np.lib.stride_tricks.as_strided(buf[offset:], shape=shape, strides=[s * 4 for s in stride]).copy()
    got = O.contiguous_u32(buf, shape, stride, offset).view(np.float32)
    assert np.array_equal(got.reshape(shape), ref)


def test_oracle_canonicalize_rule():
    """src/shapes.rs:145-155: leading size-1 dims with contiguous strides."""
    assert O.canonicalize((5, 6), (1, 5)) == ([1, 1, 5, 6], [30, 30, 1, 5])
    assert O.canonicalize((2, 3, 4, 5), (9, 8, 7, 6)) == ([2, 3, 4, 5], [9, 8, 7, 6])


# ---------------------------------------------------------------- quantize
def test_oracle_f32_to_f16_matches_numpy():
    """orc_f32_to_f16 is IEEE round-to-nearest-even: numpy's float16 cast on
    random magnitudes from 1e-9 to 1e5, ties, subnormals and the overflow edge."""
    rng = np.random.default_rng(11)
    vals = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-9, 5, 20000)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                      1.5 * 2.0 ** -24, 2.5 * 2.0 ** -24, 6.1e-5, -6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11],
                     dtype=np.float32)
    allv = np.concatenate([vals, edges])
    with np.errstate(over="ignore"):
        ref = allv.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(allv), ref)


def _block(qtype, x):
    return O.quantize(qtype, np.asarray(x, dtype=np.float32).reshape(1, -1))[0]


def test_quantize_q8_0_known_block():
    """amax = 127/16 makes d = 1/16 exactly, so every q = 16 x is exact."""
    q = np.array([127, -127, 0, 1, -1, 64, -64, 100] * 4, dtype=np.int8)
    blk = _block(O.Q8_0, q.astype(np.float32) / 16.0)
    assert blk[:2].tobytes() == np.float16(1 / 16).tobytes()
    assert np.array_equal(blk[2:].view(np.int8), q)


def test_quantize_q4_0_known_block():
    """x = (q - 8) d with the extreme -8 d present: d and the nibbles come
    back exactly (qs byte j = q_j | q_{j+16} << 4)."""
    q = np.array([0, 15, 8, 3, 12, 7, 9, 1] * 4, dtype=np.int32)
    d = 0.25
    blk = _block(O.Q4_0, (q - 8) * d)
    assert blk[:2].tobytes() == np.float16(d).tobytes()
    expect = (q[:16] | (q[16:] << 4)).astype(np.uint8)
    assert np.array_equal(blk[2:], expect)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize_q4_k_exact_grid_known_answer(seed):
    """Sub-block j holds x = s_j q - m_j with power-of-two s_j, m_j in {0, s_j/2, s_j, 2 s_j}
    and both q = 0 and q = 15 present. Then max - min = 15 s_j exactly, so the search's
    first candidate (iscale = 15 / (max - min)) reproduces q with zero error and no later
    candidate can be strictly better: the sub-block fit is (s_j, m_j) exactly. What follows
    is ggml's super-block step in closed form (d = f16(max s / 63), dmin = f16(max m / 63),
    6-bit scales = rne(63 s_j / max s), the same for mins) and a requantization that
    returns q (asserted below from the f16 scales themselves). Pins the 6-bit scale and
    nibble packing, the f16 rounding and the requantization independently of the search."""
    rng = np.random.default_rng(seed)
    e = rng.integers(-6, 0, 8)
    e[rng.integers(0, 8)] = e.max() - 4  # one sub-block 16x smaller: a 6-bit scale of 4
    s = np.ldexp(np.float32(1), e).astype(np.float32)
    m = (s * rng.choice([0.0, 0.5, 1.0, 2.0], 8)).astype(np.float32)
    q = rng.integers(0, 16, (8, 32))
    q[:, 0], q[:, 1] = 0, 15
    x = (s[:, None] * q - m[:, None]).astype(np.float32)
    assert np.array_equal((x + m[:, None]) / s[:, None], q), "grid values are exact in f32"
    blk = _block(O.Q4_K, x.reshape(-1))
    f32 = np.float32
    max_s, max_m = s.max(), m.max()
    d16, dm16 = np.float16(f32(max_s) / f32(63)), np.float16(f32(max_m) / f32(63))
    assert blk[0:2].tobytes() == d16.tobytes() and blk[2:4].tobytes() == dm16.tobytes()
    inv_s = f32(63) / max_s
    inv_m = f32(63) / max_m if max_m > 0 else f32(0)
    ls = np.minimum(np.rint(inv_s * s), 63).astype(int)  # rint: half to even, like nearest_int
    lm = np.minimum(np.rint(inv_m * m), 63).astype(int)
    for j in range(8):
        assert O.q4k_scale_min(bytes(blk[4:16]), j) == (ls[j], lm[j]), j
    # requantization nearest_int((x + dmin lm) / (d ls)) lands on q with margin
    dq = np.float64(d16) * ls
    dm = np.float64(dm16) * lm
    r = (x.astype(np.float64) + dm[:, None]) / dq[:, None]
    assert np.abs(r - q).max() < 0.45
    qs = blk[16:].reshape(4, 32)
    assert np.array_equal(qs & 15, q[0::2]) and np.array_equal(qs >> 4, q[1::2])


@pytest.mark.parametrize("qtype", [O.Q4_0, O.Q8_0, O.Q4_K])
def test_quantize_zero_and_requantize_invariants(qtype):
    qk, bb = O.QTYPE_INFO[qtype]
    zero = O.quantize(qtype, np.zeros((2, 2 * qk), np.float32))
    assert not O.dequant(qtype, zero, 2, 2 * qk).any(), "an all-zero block decodes to zeros"
    if qtype == O.Q4_0:
        # d = max / -8 = -0.0 (f16 0x8000) and every nibble is 8 (value 0)
        blocks = zero.reshape(-1, bb)
        assert (blocks[:, :2] == [0x00, 0x80]).all() and (blocks[:, 2:] == 0x88).all()
    else:
        assert not zero.any()
    rng = np.random.default_rng(12)
    x = rng.standard_normal((24, 1024)).astype(np.float32)
    q = O.quantize(qtype, x)
    dq = O.dequant(qtype, q, 24, 1024)
    q2 = O.quantize(qtype, dq)
    if qtype != O.Q4_K:
        # a dequantized matrix is a fixed point of the symmetric quantizers
        assert np.array_equal(q2, q)
    else:
        # Q4_K's scale/min search (20 candidate steps, then 6-bit rounding of the
        # super-block scales) lands on the same blocks for most inputs but is not
        # a projection; requantizing must stay close to the first decode
        same = (q2.reshape(-1, bb) == q.reshape(-1, bb)).all(axis=1).mean()
        assert same >= 0.95
        dq2 = O.dequant(qtype, q2, 24, 1024)
        assert np.sqrt(((dq2 - dq) ** 2).mean()) <= 0.01 * np.sqrt((dq ** 2).mean())
    # error bounds per block: Q8_0 <= 0.5 d + 127 |d - d16|; Q4_0 <= |d| (d = -max/8 maps the
    # extreme to -8; the opposite side is clamped at +7, one step short of +8) + f16 rounding of d
    err = np.abs(dq - x).reshape(24, -1, 32)
    amax = np.abs(x).reshape(24, -1, 32).max(axis=2)
    if qtype == O.Q8_0:
        assert (err.max(axis=2) <= amax / 127 * (0.5 + 127 * 2.0 ** -11) * 1.0001).all()
    elif qtype == O.Q4_0:
        assert (err.max(axis=2) <= amax / 8 * (1.0 + 8 * 2.0 ** -11) * 1.0001).all()
    else:
        # 4-bit asymmetric with 6-bit scales: rms error of gaussian data ~ 7 %
        assert np.sqrt((err ** 2).mean()) <= 0.09 * np.sqrt((x ** 2).mean())
