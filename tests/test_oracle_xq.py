"""The oracle's activation split (orc_quantize_x), pinned without the GPU.

x is split per 32-element block into two int8 levels with one scale,
x ~= c2 (254 q1 + q2). Nothing in the reference covers this (vortx has no
quantized path), so it is pinned by what the mathematics fixes: exact
recovery of inputs the format represents, the error bound, equivariance under
powers of two and sign, the element order tied to the Q4_0 nibble layout,
and the non-finite / tiny-block rules.
"""
import numpy as np
import pytest

from oracle import oracle as O

# c2 / 2 relative to the block's max|x| (c2 = max / (126 * 254)), plus the
# roundings of the scales: 254 c2 differs from c1 by <= 2^-24 c1 (times |q1| <= 126)
# and i2 c2 from 1 by a few 2^-24 (times |q2| <= 127): < 1e-3 of c2 / 2 together.
BOUND = 1.0 / 64008.0 * (1 + 1e-3)


def _split(x):
    lv, sc = O.quantize_x(np.asarray(x, dtype=np.float32))
    return lv, sc


def test_position_order_is_the_q4_0_nibble_order():
    """Position p of a level array holds the element whose nibble sits at p in
    the pair (low nibbles of dword g, high nibbles of dword g) of a Q4_0
    block's 16 bytes: byte t holds elements t (low) and t + 16 (high)."""
    pos_from_layout = np.empty(32, dtype=int)
    for g in range(4):
        for t in range(4):
            byte = 4 * g + t
            pos_from_layout[byte] = 8 * g + t           # low nibble of byte -> element `byte`
            pos_from_layout[byte + 16] = 8 * g + 4 + t  # high nibble -> element byte + 16
    assert np.array_equal(O.XQ_POS, pos_from_layout)
    assert sorted(O.XQ_POS) == list(range(32))
    for i in range(32):  # one-hot blocks land at their position
        x = np.zeros((1, 32), np.float32)
        x[0, i] = 3.0
        lv, _ = _split(x)
        assert lv[0, 0, 0, O.XQ_POS[i]] == 126 and np.count_nonzero(lv) == 1


def test_exact_grid_is_recovered():
    """With max|x| = 126 the scales are c1 = 1, i1 = 1, i2 = 254: x = a + k/256
    (exact in f32) splits into q1 = a and q2 = the nearest integer to 254 k / 256,
    ties to even (k = 64: 63.5 -> 64, k = -64: -63.5 -> -64, k = 192: 190.5 is
    past |r| < 1/2 so it is never used)."""
    rng = np.random.default_rng(3)
    a = rng.integers(-125, 126, 32)
    k = rng.integers(-127, 128, 32)
    k[:6] = [64, -64, 32, 0, 127, -127]
    a[31] = 126
    k[31] = 0  # the block max (every other |x| < 125.5)
    x = (a + k / 256.0).astype(np.float32)
    assert np.array_equal(x.astype(np.float64), a + k / 256.0)
    lv, sc = _split(x[None, :])
    q1 = lv[0, 0, 0, O.XQ_POS]
    q2 = lv[0, 0, 1, O.XQ_POS]
    assert np.array_equal(q1, a)
    expect_q2 = np.rint(254.0 * k / 256.0)  # numpy rounds half to even
    assert np.array_equal(q2, expect_q2)
    assert q2[0] == 64 and q2[1] == -64 and q2[2] == 32  # 63.5 -> 64, -63.5 -> -64, 31.75 -> 32
    assert sc[0, 0, 0] == np.float32(np.float32(126.0 / 126.0) / np.float32(254.0))
    assert sc[0, 0, 1] == np.float32(x.astype(np.float64).sum())  # integer-grid sum: exact


@pytest.mark.parametrize("dist", ["normal", "uniform", "heavy", "ties"])
def test_error_bound(dist):
    rng = np.random.default_rng(11)
    B, K = 5, 32 * 64
    if dist == "normal":
        x = rng.standard_normal((B, K))
    elif dist == "uniform":
        x = rng.uniform(-1, 1, (B, K)) * 10.0 ** rng.integers(-20, 20, (B, K // 32)).repeat(32, 1)
    elif dist == "heavy":
        x = rng.standard_cauchy((B, K))
    else:  # values at half-level boundaries of the first split
        m = 126.0
        x = (rng.integers(-125, 126, (B, K)) + 0.5) * (m / 126.0)
        x[:, ::32] = m
    x = x.astype(np.float32)
    lv, sc = _split(x)
    xr = O.xq_decode_f64(lv, sc)
    bm = np.abs(x.reshape(B, -1, 32)).max(-1, keepdims=True).astype(np.float64)
    rel = (np.abs(xr - x).reshape(B, -1, 32) / bm).max()
    assert rel <= BOUND, rel


def test_power_of_two_and_sign_equivariance():
    """Every step is a ratio or a product of ratios of x, so scaling x by 2^e
    scales c2 and S by 2^e and leaves the levels; -x negates levels and S."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    lv, sc = _split(x)
    for e in (-40, -7, 9, 60):
        lv2, sc2 = _split(x * np.float32(2.0 ** e))
        assert np.array_equal(lv2, lv)
        assert np.array_equal(sc2, sc * np.float32(2.0 ** e))
    lvn, scn = _split(-x)
    assert np.array_equal(lvn, -lv)
    assert np.array_equal(scn[..., 0], sc[..., 0]) and np.array_equal(scn[..., 1], -sc[..., 1])


def test_sum_is_the_stated_tree():
    """S adds the 32 values as a fixed tree (pairs inside each 4, then the 8
    partial sums pairwise); a block where sequential summation cancels
    differently tells the orders apart."""
    v = np.array([1e8, 1, -1e8, 1] * 8, dtype=np.float32)
    v[5] = 3
    _, sc = _split(v[None, :])
    s4 = [(v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]) for q in range(8)]
    tree = ((s4[0] + s4[1]) + (s4[2] + s4[3])) + ((s4[4] + s4[5]) + (s4[6] + s4[7]))
    seq = np.float32(0)
    for t in v:
        seq = np.float32(seq + t)
    assert sc[0, 0, 1] == tree and tree != seq


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_non_finite_block(bad):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    ref_lv, ref_sc = _split(x)
    x[0, 40] = bad
    lv, sc = _split(x)
    assert not np.isfinite(sc[1, 0, 0]) and (lv[1, 0] == 0).all()  # block 1 of column 0
    other = np.ones(sc.shape[:2], bool)
    other[1, 0] = False
    assert np.array_equal(lv[other], ref_lv[other]) and np.array_equal(sc[other], ref_sc[other])


def test_tiny_and_zero_blocks():
    x = np.zeros((1, 96), np.float32)
    x[0, 32:64] = np.float32(2.0 ** -110) * np.arange(1, 33, dtype=np.float32)
    x[0, 64:96] = np.float32(2.0 ** -99)
    lv, sc = _split(x)
    assert (lv[0:2] == 0).all()                       # zero block and one below 2^-100: no levels
    assert sc[1, 0, 1] == np.float32(2.0 ** -110 * 528)  # S still exact
    assert (lv[2, 0, 0] == 126).all()                 # 2^-99 is split normally
    assert sc[0, 0, 0] == 0 and sc[0, 0, 1] == 0


def test_strided_input_matches_contiguous():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    lv, sc = _split(x)
    xt = np.ascontiguousarray(x.T)  # [K, B] storage: xs_k = B, xs_b = 1
    levels = np.zeros_like(lv)
    scales = np.zeros_like(sc)
    assert O.lib().orc_quantize_x(xt.ctypes.data, 4, 1, 256, 4, levels.ctypes.data, scales.ctypes.data) == 0
    assert np.array_equal(levels, lv) and np.array_equal(scales, sc)


def _unclamped_levels(x):
    """Both levels of every 32-block before any clamp, from the stated
    roundings (f32 scales, exact products, round to nearest even), with the
    magnitude |r i2| that the second rounding sees."""
    v = x.reshape(-1, 32).astype(np.float32)
    m = np.abs(v).max(1)
    m = m[m >= np.float32(2.0 ** -100)]
    v = v[np.abs(v).max(1) >= np.float32(2.0 ** -100)]
    c1 = (m / np.float32(126.0)).astype(np.float32)
    i1 = (np.float32(126.0) / m).astype(np.float32)
    i2 = (i1 * np.float32(254.0)).astype(np.float32)
    q1 = np.rint(v.astype(np.float64) * i1[:, None].astype(np.float64))  # exact product, ties to even
    r = (v.astype(np.float64) - q1 * c1[:, None].astype(np.float64)).astype(np.float32)
    t2 = r.astype(np.float64) * i2[:, None].astype(np.float64)
    return q1, t2


def test_clamps_never_act():
    """The device split computes no clamp (vx_xq_levels4): |v| <= m with
    i1 = RN(126 / m) keeps |q1| <= 126, and |r| <= c1 (0.5 + 126 2^-23) with
    i2 = RN(254 i1) keeps |r i2| <= 127.004, which rounds to |q2| <= 127.
    Checked on random, heavy-tailed and adversarial blocks (values whose first
    level sits on a half, blocks whose scale products c1 i1 stray furthest
    from 1), and the oracle's clamped levels equal the unclamped ones."""
    rng = np.random.default_rng(17)
    blocks = [rng.standard_normal((4000, 32)), rng.standard_cauchy((4000, 32)),
              rng.uniform(-1, 1, (4000, 32)) * 10.0 ** rng.integers(-30, 30, (4000, 1))]
    # first level on a half: v = (k + 1/2 - tiny) c1 for k up to 125, block max m
    ms = (rng.uniform(1, 2, 4000) * 2.0 ** rng.integers(-90, 90, 4000)).astype(np.float32)
    k = rng.integers(-125, 126, (4000, 31)) + rng.choice([-0.5, 0.5], (4000, 31)) * (1 - 1e-7)
    adv = np.concatenate([ms[:, None], k * (ms[:, None] / 126.0)], 1)
    blocks.append(adv)
    x = np.concatenate([b.astype(np.float32) for b in blocks])
    q1, t2 = _unclamped_levels(x)
    assert np.abs(q1).max() <= 126
    assert np.abs(t2).max() <= 127.004, np.abs(t2).max()
    # the split with its clamps gives exactly the rounded, unclamped levels
    lv, _ = _split(x[:2000].reshape(1, -1))
    q1c, t2c = _unclamped_levels(x[:2000])
    got = lv.reshape(-1, 2, 32)
    pos = O.XQ_POS
    assert np.array_equal(got[:, 0, pos], q1c) and np.array_equal(got[:, 1, pos], np.rint(t2c))


def test_device_layout_round_trip_and_coalescing():
    """O.xq_device_levels places level L of column b, block j, position p at
    (j/8) B 512 + ((j%8)/2) B 128 + (p/8) B 32 + b 32 + L 16 + (j%2) 8 + p%8
    (the header's formula), and the 16 bytes a matrix-core lane (b, L, group
    g) loads for a block pair are contiguous, with consecutive (b, L) lanes of
    one load 16 bytes apart."""
    rng = np.random.default_rng(3)
    K, B = 800, 5                      # 25 blocks: a partial last item
    lv = rng.integers(-127, 128, (K // 32, B, 2, 32), dtype=np.int8)
    dev = O.xq_device_levels(lv).reshape(-1)
    assert dev.size == (-(-K // 256)) * B * 512
    for j in (0, 1, 7, 8, 13, 24):
        for b in range(B):
            for L in range(2):
                for p in (0, 5, 8, 17, 31):
                    off = (j // 8) * B * 512 + ((j % 8) // 2) * B * 128 + (p // 8) * B * 32 + b * 32 + L * 16 + \
                        (j % 2) * 8 + p % 8
                    assert dev[off] == lv[j, b, L, p], (j, b, L, p)
    # the inverse used by the GPU tests
    d = dev.reshape(-1, 4, 4, B, 2, 2, 8)
    back = d.transpose(0, 1, 5, 3, 4, 2, 6).reshape(-1, B, 2, 32)[:K // 32]
    assert np.array_equal(back, lv)
