"""Routing trace files (src/main.rs:771-799) and the counts read back from
them (src/route.rs:28-177), on the CPU."""
import math

import numpy as np
import pytest

from moe_amd.layer import Route
from moe_amd.trace import Counts, _f64_text, header_line, route_line, write_trace


# The Rust float writers' notation (ryu's documented layout, which
# serde_json's compact writer prints): decimal while the decimal exponent
# kk = len(digits) + k lies in (-5, 16], else d.ddd e(kk-1) with no '+' and
# no zero padding.  Python's repr differs on every case below but the first
# three, so a writer that fell back to repr fails here.
@pytest.mark.parametrize("v,text", [
    (1.0, "1.0"), (0.5, "0.5"), (-2.5, "-2.5"),
    (1e-4, "0.0001"), (1e-5, "0.00001"), (1.25e-5, "0.0000125"),
    (1e-6, "1e-6"), (1.5e-7, "1.5e-7"), (5e-324, "5e-324"),
    (1e15, "1000000000000000.0"), (1e16, "1e16"), (1.5e16, "1.5e16"), (1e300, "1e300"),
    (0.0, "0.0"), (-0.0, "-0.0"), (float("inf"), "null"), (float("nan"), "null"),
])
def test_float_notation(v, text):
    assert _f64_text(v) == text


def test_f32_weights_widen_to_f64_and_read_back_exactly():
    """A weight goes out as its f32 value widened to f64 (0.1f32 prints
    0.10000000149011612) in the fewest digits that read back to it."""
    rng = np.random.default_rng(3)
    w = np.concatenate([rng.random(2000, dtype=np.float32),
                        np.float32([0.1, 1 / 3, 2.5, 1e-30, 3.4028235e38, 1.4e-45])])
    for x in w:
        s = _f64_text(float(x))
        assert float(s) == float(x)
        digits = s.split("e")[0].replace("-", "").replace(".", "").strip("0")
        assert len(digits) <= 17
        # No shorter digit string reads back to the same f64.
        if len(digits) > 1:
            shorter = float(f"{float(x):.{len(digits) - 2}e}")
            assert shorter != float(x)
    assert _f64_text(float(np.float32(0.1))) == "0.10000000149011612"


def test_lines_have_sorted_keys_and_no_spaces():
    assert header_line("mixtral", 32, 8, 2) == '{"experts":8,"layers":32,"model":"mixtral","top_k":2}'
    r = Route(pos=3, layer=1, experts=[(5, np.float32(0.75)), (2, np.float32(0.25))])
    assert route_line(r) == '{"experts":[[5,0.75],[2,0.25]],"layer":1,"pos":3,"text":null,"token":null}'
    tokens = [10, 11, 12, 13]
    texts = ["a", "b", "c", 'd"\n\x01']
    assert route_line(r, tokens, texts) == \
        '{"experts":[[5,0.75],[2,0.25]],"layer":1,"pos":3,"text":"d\\"\\n\\u0001","token":13}'
    # A position the token list does not cover has no token and no text.
    assert '"text":null,"token":null' in route_line(Route(9, 0, [(1, 1.0)]), tokens, texts)


def _routes():
    # Three tokens over two routed layers (1 and 3), 4 experts, top-2.
    sel = {(0, 1): [(2, 0.6), (0, 0.4)], (1, 1): [(2, 0.7), (3, 0.3)], (2, 1): [(1, 0.5), (2, 0.5)],
           (0, 3): [(0, 0.9), (1, 0.1)], (1, 3): [(0, 0.8), (3, 0.2)], (2, 3): [(0, 0.55), (3, 0.45)]}
    return [Route(p, l, [(e, np.float32(w)) for e, w in ex]) for (p, l), ex in sel.items()]


def test_write_then_read_gives_the_in_memory_counts(tmp_path):
    routes = _routes()
    path = tmp_path / "t.jsonl"
    assert write_trace(str(path), routes, "m", 4, 4, 2, tokens=[7, 8, 9]) == len(routes)
    lines = path.read_text().splitlines()
    assert len(lines) == 1 + len(routes)
    got = Counts.read(str(path))
    want = Counts.from_trace(routes, "m", 4, 2)
    assert got == want
    assert (got.model, got.experts, got.top_k, got.tokens) == ("m", 4, 2, 3)
    assert got.layers() == [1, 3]
    assert got.count(1, 2) == 3 and got.count(3, 0) == 3 and got.count(3, 2) == 0


def test_reader_skips_what_the_reference_skips(tmp_path):
    """Blank and unparsable lines are skipped; any object or value without a
    "pos" key is a header; "pos": null is a route at position 0; experts
    without an integer id are not counted; the expert count falls back to
    the largest id seen + 1."""
    path = tmp_path / "t.jsonl"
    path.write_text("\n".join([
        '{"model":"x","experts":6,"top_k":2}',
        "",
        "not json",
        '{"pos":0,"layer":2,"experts":[[1,0.5],[4,0.5]]}',
        '{"pos":null,"layer":2,"experts":[[1,0.5],["3",0.5],[-1,0.1],[2.0,0.1],[]]}',
        '[1,2,3]',
        '{"pos":5,"layer":2,"experts":"none"}',
    ]) + "\n")
    c = Counts.read(str(path))
    # The array line is a header with no fields: it resets the header's values.
    assert (c.model, c.top_k) == ("", 0)
    assert c.experts == 5  # largest id 4, plus one
    assert c.tokens == 2   # positions 0 and 5
    assert c.counts == {(2, 1): 2, (2, 4): 1}


def test_statistics_closed_forms():
    # Uniform: every expert chosen equally often.
    u = Counts(experts=8, tokens=8, counts={(0, e): 2 for e in range(8)})
    assert abs(float(u.entropy(0)) - 1.0) <= 2 ** -22
    assert u.peak_ratio(0) == 1.0 and u.dead(0) == 0 and u.coverage() == 1.0
    # One expert takes everything: entropy 0, peak ratio E, E-1 dead.
    s = Counts(experts=8, tokens=4, counts={(0, 3): 4})
    assert s.entropy(0) == 0.0 and s.peak_ratio(0) == 8.0 and s.dead(0) == 7
    assert s.coverage() == np.float32(1 / 8)
    # Two experts at 3:1, normalised by ln 4: H = -(3/4 ln 3/4 + 1/4 ln 1/4).
    t = Counts(experts=4, tokens=4, counts={(0, 0): 3, (0, 1): 1})
    h = -(0.75 * math.log(0.75) + 0.25 * math.log(0.25)) / math.log(4)
    assert abs(float(t.entropy(0)) - h) <= 4e-7
    assert t.share(0, 0) == np.float32(0.75)
    # Fewer than two experts, or nothing routed: 0.
    assert Counts(experts=1, counts={(0, 0): 5}).entropy(0) == 0.0
    assert Counts(experts=4).entropy(0) == 0.0 and Counts(experts=4).peak_ratio(0) == 0.0


def test_hottest_orders_by_count_then_key():
    c = Counts(experts=4, counts={(1, 2): 5, (0, 3): 5, (0, 1): 7, (2, 0): 1, (1, 1): 0})
    assert c.hottest() == [(0, 1), (0, 3), (1, 2), (2, 0)]


def test_entropy_uses_f32_arithmetic():
    """Counts whose f32 and f64 entropies differ in the last bit: the f32
    fold (each term rounded to f32, ln from the C library's logf) is what
    the reference computes; an f64 evaluation rounded once at the end gives
    0.9355996 here instead."""
    rng = np.random.default_rng(0)
    E = int(rng.integers(3, 64))
    n = [int(x) for x in rng.integers(0, 1000, E)]
    c = Counts(experts=E, tokens=1, counts={(0, e): v for e, v in enumerate(n)})
    total = sum(n)
    f64 = -sum(v / total * math.log(v / total) for v in n if v) / math.log(E)
    assert E == 54 and np.float32(f64) == np.float32(0.9355996)
    assert c.entropy(0) == np.float32(0.93559957)
    assert c.entropy(0) != np.float32(f64)
