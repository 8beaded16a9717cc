"""The oracle's routed layer inside a tiny forward reproduces the
reference's golden logits (tests/fixtures/*/expected.json) at the
reference's own tolerances, and the fixtures are sensitive enough that a
routing mistake would show."""
import numpy as np
import pytest

from tiny_model import TinyModel, oracle_moe_fn

FIXTURES = ["gqa", "gqa_fullnorm", "gqa_long", "mla"]


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_logits_every_position(oracle, name):
    """tests/oracle.rs:45-76, 100-118: 5e-3 at every position, argmax kept."""
    m = TinyModel(name)
    got = m.forward(oracle_moe_fn(m))
    assert np.abs(got - m.expected).max() < 5e-3
    assert (got.argmax(1) == m.expected.argmax(1)).all()


@pytest.mark.parametrize("name,dt,tol", [("gqa", 8, 0.25), ("mla", 8, 0.25), ("gqa", 6, 0.7), ("mla", 6, 0.7),
                                         ("gqa", 2, 1.5), ("mla", 2, 1.5)])
def test_fixture_packed(oracle, name, dt, tol):
    """tests/oracle.rs:78-94, 483-501: packed checkpoints keep the prediction."""
    m = TinyModel(name, quant_dt=dt)
    got = m.forward(oracle_moe_fn(m))
    assert np.abs(got[-1] - m.expected[-1]).max() < tol
    assert got[-1].argmax() == m.expected[-1].argmax()
    assert np.isfinite(got).all()


@pytest.mark.parametrize("name", ["gqa", "mla"])
def test_layer_is_position_independent(oracle, name):
    """The routed layer sees only its t rows: one token at a time equals the
    batch, bit for bit (what makes batched and incremental prefill agree,
    tests/oracle.rs:60-75)."""
    m = TinyModel(name)
    fn = oracle_moe_fn(m)
    x = np.random.default_rng(0).standard_normal((6, 32)).astype(np.float32)
    layer = next(l for l in range(m.layers) if m.is_moe(l))
    whole = fn(layer, x)
    rows = np.concatenate([fn(layer, x[i:i + 1]) for i in range(6)])
    assert np.array_equal(whole, rows)


@pytest.mark.parametrize("name,mutation", [("gqa", dict(top_k=1)), ("gqa", dict(temp=4.0)),
                                           ("mla", dict(top_k=1)), ("mla", dict(top_k=4)),
                                           ("mla", dict(temp=0.25))])
def test_fixture_detects_routing_mistakes(oracle, name, mutation):
    """A plausible routing error moves the logits past the 5e-3 bar, so the
    fixtures pin the routing rule, not only the expert arithmetic."""
    from oracle import pyoracle as O

    m = TinyModel(name)
    got = m.forward(oracle_moe_fn(m, O.OracleLayer.routing(**mutation)))
    assert np.abs(got - m.expected).max() > 5e-3
