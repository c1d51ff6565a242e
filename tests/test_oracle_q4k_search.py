"""The oracle's Q4_K scale search pinned on designed sub-blocks.

tests/golden/q4k_search.json (written by tests/golden/make_q4k_search.py,
which restates ggml's make_qkx2_quants in float64 and says how the cases were
chosen) holds sub-blocks whose search has one decisive winner: the last
candidate (k = 20, inverse scale 16 / range), the first (k = 0, 14 / range)
and k = 7 (14.7 / range), each produced by no other candidate and each
changed by a one-constant change of nstep (20), rmin (-1) or rdelta (0.1).
A block whose result differs under the weights 1, |x| and x^2 pins the
weighting av_x + |x| of quantize_row_q4_K_ref through the whole quantizer.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

FIX = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4k_search.json")))


@pytest.mark.parametrize("case", FIX["fits"], ids=lambda c: f"winner{c['winner']}")
def test_search_winner(case):
    x = np.array(case["x_bits"], np.uint32).view(np.float32)
    w = np.array(case["w_bits"], np.uint32).view(np.float32)
    levels, scale, mn = O.q4k_fit(x, w)
    assert np.array_equal(levels, np.array(case["levels"], np.uint8)), "a different candidate won"
    # the least-squares (scale, min) of the winning levels, f32 vs f64 evaluation
    assert abs(scale - case["scale"]) <= 1e-5 * abs(case["scale"])
    assert abs(mn - case["min"]) <= 1e-5 * abs(case["scale"])


def test_weighting_av_x_plus_abs_x():
    b = FIX["weighting_block"]
    x = np.zeros(256, np.float32)
    x[:32] = np.array(b["x0_bits"], np.uint32).view(np.float32)
    blk = O.quantize(O.Q4_K, x[None, :])[0]
    assert blk.tobytes().hex() == b["block_hex"]


def test_fixture_is_what_the_statement_gives():
    """The fixture's expectations restated from its own inputs by the
    float64 statement (guards the fixture against hand edits)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "mk", os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "make_q4k_search.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    for case in FIX["fits"]:
        x = np.array(case["x_bits"], np.uint32).view(np.float32)
        w = np.array(case["w_bits"], np.uint32).view(np.float32)
        L, s, m, win, fits = mk.qkx2(x, w)
        assert win == case["winner"] and mk.decisive(fits, win) and L.tolist() == case["levels"]
        for name in case["detects"]:
            assert not mk.same(mk.qkx2(x, w, **mk.MUTATIONS[name]), (L, s, m)), name
