"""The oracle's whole-model forward (embedding, norms, rope schemes, GQA and
MLA attention with windows, dense and routed FFNs, head, greedy decoding)
against the reference's golden logits, its rope unit tests and a float64
restatement; this is what pins the CPU side of the end-to-end checks."""
import math

import numpy as np
import pytest

from tiny_model import TinyModel, host_tensors, oracle_moe_fn

FIXTURES = ["gqa", "gqa_fullnorm", "gqa_long", "mla"]


def _model(name, dt=None):
    from oracle import pyoracle as O

    m, spec, tensors = host_tensors(name, dt)
    return m, spec, O.OracleModel(spec, tensors)


@pytest.mark.parametrize("name", FIXTURES)
def test_forward_all_every_position(oracle, name):
    """tests/oracle.rs:100-118: forward_all at every position within 5e-3,
    argmax kept; the last row equals forward's."""
    m, spec, om = _model(name)
    all_ = om.forward_all(m.tokens, om.new_state(32))
    assert all_.shape == (len(m.tokens), spec.vocab)
    assert np.abs(all_ - m.expected).max() < 5e-3
    assert (all_.argmax(1) == m.expected.argmax(1)).all()
    last = om.forward(m.tokens, om.new_state(32))
    assert np.abs(all_[-1] - last).max() < 1e-6


@pytest.mark.parametrize("name", FIXTURES)
def test_incremental_and_chunked(oracle, name):
    """tests/oracle.rs:45-76: one token at a time within 5e-3 at every step;
    a split prefill lands within 1e-4 of a whole one."""
    m, spec, om = _model(name)
    st = om.new_state(32)
    for i, tok in enumerate(m.tokens):
        got = om.forward([tok], st)
        assert np.abs(got - m.expected[i]).max() < 5e-3, i
    assert st["pos"] == len(m.tokens)
    whole = om.forward(m.tokens, om.new_state(32))
    st2 = om.new_state(32)
    h = len(m.tokens) // 2
    om.forward(m.tokens[:h], st2)
    split = om.forward(m.tokens[h:], st2)
    assert np.abs(whole - split).max() < 1e-4


@pytest.mark.parametrize("name,dt,tol", [("gqa", 8, 0.25), ("mla", 8, 0.25), ("gqa", 6, 0.7), ("mla", 6, 0.7),
                                         ("gqa", 2, 1.5), ("mla", 2, 1.5), ("gqa_long", 8, 0.25),
                                         ("gqa_fullnorm", 8, 0.25)])
def test_packed(oracle, name, dt, tol):
    """tests/oracle.rs:78-94, 483-501: packed weights keep the prediction."""
    m, spec, om = _model(name, dt)
    got = om.forward(m.tokens, om.new_state(32))
    assert np.abs(got - m.expected[-1]).max() < tol
    assert got.argmax() == m.expected[-1].argmax()


@pytest.mark.parametrize("name,dt", [(n, None) for n in FIXTURES] + [("gqa", 8), ("mla", 2)])
def test_matches_float64_restatement(oracle, name, dt):
    """The f32 oracle model against an independent float64 forward over the
    same (dequantised) weights: agreement to f32 rounding, far inside the
    fixtures' bar, so a mistake in either shows."""
    m, spec, om = _model(name, dt)
    ref = m.forward(oracle_moe_fn(m))
    got = om.forward_all(m.tokens, om.new_state(32))
    assert np.abs(got - ref).max() < 2e-4


def test_fixture_catches_rope_mistake(oracle):
    """A rope mistake planted in the oracle (the frequency table reversed)
    moves the mla fixture's logits past 5e-3.  The GQA fixtures' attention
    is close to uniform (tiny random weights): reversing their rope table,
    regrouping GQA heads, dropping gqa_long's window or YaRN's attention
    scale moves their logits by at most 8e-5, so those properties are pinned
    by test_attention_brute_force, the rope closed forms and the reference's
    rope unit tests below, not by the fixtures."""
    m, spec, om = _model("mla")
    om.inv = om.inv[::-1].copy()
    got = om.forward_all(m.tokens, om.new_state(32))
    assert np.abs(got - m.expected).max() > 5e-3


def _attention64(q, kc, vc, t, base, heads, n_kv, qd, vd, scale, window):
    """Causal attention in float64 straight from its definition."""
    rep = heads // n_kv
    out = np.zeros((t, heads, vd))
    for i in range(t):
        p = base + i
        lo = max(p + 1 - window, 0) if window else 0
        for h in range(heads):
            g = h // rep if rep > 1 else min(h, n_kv - 1)
            k = kc[lo:p + 1].reshape(-1, n_kv, qd)[:, g, :].astype(np.float64)
            v = vc[lo:p + 1].reshape(-1, n_kv, vd)[:, g, :].astype(np.float64)
            s = k @ q[i].reshape(heads, qd)[h].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out[i, h] = (w / w.sum()) @ v
    return out.reshape(t, -1)


@pytest.mark.parametrize("heads,n_kv,qd,vd,window,base,t", [(4, 2, 8, 8, 3, 0, 6), (8, 8, 16, 8, 0, 5, 4),
                                                            (6, 2, 32, 16, 5, 40, 9), (4, 1, 64, 64, 1, 3, 2),
                                                            (2, 2, 8, 8, 100, 0, 7)])
def test_attention_brute_force(oracle, heads, n_kv, qd, vd, window, base, t):
    """orc_attention against its float64 definition (windows keep the last
    `window` positions, itself included; GQA groups consecutive heads; MQA
    and window 1 as special cases), and a dropped window fails the check."""
    from oracle import pyoracle as O

    rng = np.random.default_rng(heads * 100 + window)
    ctx = base + t
    q = rng.standard_normal((t, heads * qd)).astype(np.float32)
    kc = rng.standard_normal((ctx, n_kv * qd)).astype(np.float32)
    vc = rng.standard_normal((ctx, n_kv * vd)).astype(np.float32)
    scale = np.float32(1.0 / math.sqrt(qd))
    om = O.OracleModel.__new__(O.OracleModel)
    got = om._attend(q, kc, vc, t, base, heads, n_kv, qd, vd, scale, window)
    want = _attention64(q, kc, vc, t, base, heads, n_kv, qd, vd, float(scale), window)
    assert np.abs(got - want).max() < 1e-5
    if window and window < ctx:
        full = _attention64(q, kc, vc, t, base, heads, n_kv, qd, vd, float(scale), 0)
        assert np.abs(full - want).max() > 1e-2
    if window == 1:
        # One position: the output is that position's value row.
        assert np.abs(got.reshape(t, heads, vd) - vc[base:base + t].reshape(t, n_kv, vd)[:, [h // (heads // n_kv)
                      for h in range(heads)], :]).max() < 1e-6


def test_rmsnorm_and_rope_closed_forms(oracle):
    """rmsnorm of a constant row is the weight times sign (to eps); rope at
    position 0 is the identity and preserves each pair's norm elsewhere;
    rope by p then by q equals rope by p + q to f32 rounding."""
    from oracle import pyoracle as O
    import ctypes as C

    w = np.linspace(0.5, 2.0, 16).astype(np.float32)
    x = np.full((2, 16), 3.0, np.float32)
    x[1] = -0.25
    out = O.rmsnorm_rows(x, w, 1e-6)
    assert np.abs(out[0] - w).max() < 1e-6 and np.abs(out[1] + w).max() < 1e-4
    rng = np.random.default_rng(3)
    inv = (10000.0 ** (-2.0 * np.arange(8) / 16)).astype(np.float32)
    v = rng.standard_normal((3, 16)).astype(np.float32)
    r = v.copy()
    O.lib().orc_rope_rows(O._p(r), 3, 16, 1, 16, 0, 16, O._p(np.array([0, 7, 300], np.int32)), O._p(inv), 8)
    assert np.array_equal(r[0], v[0])
    for i in (1, 2):
        n0 = v[i, :8] ** 2 + v[i, 8:] ** 2
        n1 = r[i, :8] ** 2 + r[i, 8:] ** 2
        assert np.abs(n0 - n1).max() < 1e-4
    a = v[1:2].copy()
    O.lib().orc_rope_rows(O._p(a), 1, 16, 1, 16, 0, 16, O._p(np.array([3], np.int32)), O._p(inv), 8)
    O.lib().orc_rope_rows(O._p(a), 1, 16, 1, 16, 0, 16, O._p(np.array([4], np.int32)), O._p(inv), 8)
    assert np.abs(a[0] - r[1]).max() < 1e-5
    # The second half rotates the opposite way: swapping halves is a mistake the check sees.
    ang = 7 * inv.astype(np.float64)
    want = np.concatenate([v[1, :8] * np.cos(ang) - v[1, 8:] * np.sin(ang), v[1, :8] * np.sin(ang) +
                           v[1, 8:] * np.cos(ang)])
    assert np.abs(r[1] - want).max() < 1e-5


def _rope(cfg):
    from moe_amd.model import Rope

    return Rope.from_config(cfg, 4096)


def _inv(rope, dim):
    from oracle import pyoracle as O

    return O.inv_freqs(rope, dim).astype(np.float64)


def test_rope_unscaled(oracle):
    """src/spec.rs:454-465."""
    r = _rope({"rope_theta": 500000.0})
    assert r.kind == 0 and abs(r.theta - 500000.0) < 1.0
    inv = _inv(r, 8)
    assert inv.size == 4 and abs(inv[0] - 1.0) < 1e-6 and (np.diff(inv) < 0).all()
    assert abs(float(O_attn(r)) - 1.0) < 1e-6
    # The plain geometric series theta^(-2i/d), to f32 rounding.
    want = np.array([500000.0 ** (-2.0 * i / 8) for i in range(4)])
    assert np.abs(inv / want - 1).max() < 1e-6


def O_attn(r):
    from oracle import pyoracle as O

    return O.attn_scale(r)


def test_rope_schemes_recognised():
    """src/spec.rs:467-491."""
    kinds = {"linear": 1, "dynamic": 2, "ntk": 2, "yarn": 3, "llama3": 4}
    for name, kind in kinds.items():
        assert _rope({"rope_scaling": {"rope_type": name, "factor": 4.0}}).kind == kind
        assert _rope({"rope_scaling": {"type": name, "factor": 4.0}}).kind == kind
        assert _rope({"rope_scaling": {"rope_type": name, "factor": 1.0}}).kind == 0
    assert _rope({"rope_scaling": {"factor": 2.0}}).kind == 1


def test_rope_linear_divides(oracle):
    """src/spec.rs:493-504."""
    base = _inv(_rope({"rope_theta": 10000.0}), 16)
    lin = _inv(_rope({"rope_theta": 10000.0, "rope_scaling": {"rope_type": "linear", "factor": 4.0}}), 16)
    assert np.abs(lin - base / 4.0).max() < 1e-9


def test_rope_ntk(oracle):
    """src/spec.rs:506-523, plus NTK's closed form: the base raised to
    theta * s^(d/(d-2))."""
    base = _inv(_rope({"rope_theta": 10000.0}), 64)
    ntk = _inv(_rope({"rope_theta": 10000.0, "rope_scaling": {"rope_type": "dynamic", "factor": 8.0}}), 64)
    lin = _inv(_rope({"rope_theta": 10000.0, "rope_scaling": {"rope_type": "linear", "factor": 8.0}}), 64)
    assert abs(ntk[0] - base[0]) < 1e-9 and abs(lin[0] - base[0] / 8.0) < 1e-9
    assert ntk[-1] <= lin[-1] * 1.05
    th = 10000.0 * 8.0 ** (64 / 62)
    want = np.array([th ** (-2.0 * i / 64) for i in range(32)])
    assert np.abs(ntk / want - 1).max() < 2e-5


def test_rope_llama3(oracle):
    """src/spec.rs:525-545."""
    r = _rope({"rope_theta": 500000.0, "rope_scaling": {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                                       "high_freq_factor": 4.0,
                                                       "original_max_position_embeddings": 8192}})
    base = _inv(_rope({"rope_theta": 500000.0}), 128)
    got = _inv(r, 128)
    assert (got <= base + 1e-9).all() and (got >= base / 8.0 - 1e-9).all()
    assert abs(got[0] - base[0]) < 1e-9 and abs(got[-1] - base[-1] / 8.0) < 1e-9
    # Some pair sits on the ramp strictly between the two.
    assert ((got < base * (1 - 1e-3)) & (got > base / 8.0 * (1 + 1e-3))).any()


def test_rope_yarn(oracle):
    """src/spec.rs:547-565 and 567-577."""
    r = _rope({"rope_theta": 10000.0, "rope_scaling": {"rope_type": "yarn", "factor": 4.0,
                                                      "original_max_position_embeddings": 4096}})
    base = _inv(_rope({"rope_theta": 10000.0}), 64)
    got = _inv(r, 64)
    assert ((got <= base + 1e-9) & (got >= base / 4.0 - 1e-9)).all()
    assert abs(float(O_attn(r)) - (0.1 * math.log(4.0) + 1.0)) < 1e-6
    assert abs(float(O_attn(_rope({"rope_scaling": {"rope_type": "linear", "factor": 4.0}}))) - 1.0) < 1e-9
    r1 = _rope({"rope_scaling": {"rope_type": "yarn", "factor": 40.0, "mscale": 1.0, "mscale_all_dim": 1.0}})
    assert abs(float(O_attn(r1)) - 1.0) < 1e-6
    r2 = _rope({"rope_scaling": {"rope_type": "yarn", "factor": 40.0, "mscale": 1.0, "mscale_all_dim": 0.0}})
    assert float(O_attn(r2)) > 1.0


def test_product_rope_tables_equal_oracle(oracle):
    """The library's inv_freqs and attention scale equal the oracle's bit
    for bit for every scheme."""
    cfgs = [{"rope_theta": 500000.0},
            {"rope_theta": 10000.0, "rope_scaling": {"rope_type": "linear", "factor": 4.0}},
            {"rope_theta": 10000.0, "rope_scaling": {"rope_type": "dynamic", "factor": 8.0}},
            {"rope_theta": 500000.0, "rope_scaling": {"rope_type": "llama3", "factor": 8.0,
                                                      "original_max_position_embeddings": 8192}},
            {"rope_theta": 10000.0, "rope_scaling": {"rope_type": "yarn", "factor": 4.0,
                                                     "original_max_position_embeddings": 32}},
            {"rope_scaling": {"rope_type": "yarn", "factor": 40.0, "mscale": 0.707, "mscale_all_dim": 1.0,
                              "original_max_position_embeddings": 4096}}]
    for cfg in cfgs:
        r = _rope(cfg)
        for dim in (8, 64, 128):
            assert np.array_equal(r.inv_freqs(dim), _inv(r, dim).astype(np.float32)), (cfg, dim)
        assert np.float32(r.attn_scale()) == O_attn(r), cfg


def test_windows_conventions():
    """src/spec.rs:581-607."""
    from moe_amd.model import windows_of

    assert windows_of({}, 4) == [None] * 4
    assert windows_of({"sliding_window": 0}, 3) == [None] * 3
    assert windows_of({"sliding_window": 128}, 3) == [128] * 3
    assert windows_of({"sliding_window": 128, "layer_types": ["sliding_attention", "full_attention",
                                                              "sliding_attention"]}, 3) == [128, None, 128]
    assert windows_of({"sliding_window": 64, "sliding_window_pattern": 4}, 4) == [64, 64, 64, None]
    assert windows_of({"sliding_window": 32, "use_sliding_window": True, "max_window_layers": 2}, 4) == \
        [None, None, 32, 32]
    assert windows_of({"sliding_window": 32, "use_sliding_window": False}, 2) == [None, None]
    # The first numeric key decides, as num() reads it.
    assert windows_of({"sliding_window": 0, "attention_window_size": 8}, 2) == [None, None]


@pytest.mark.parametrize("name", ["gqa", "mla"])
def test_greedy_generation(oracle, name):
    """Greedy decoding picks the first maximum (src/sample.rs:87-95) and
    feeds it back: each step's token is the argmax of a whole-sequence
    forward over everything so far."""
    m, spec, om = _model(name)
    prompt = m.tokens[:3]
    out = om.generate_greedy(prompt, 5, ctx=16)
    seq = list(prompt)
    for tok in out:
        logits = om.forward_all(seq, om.new_state(16))[-1]
        assert tok == int(np.argmax(logits))
        seq.append(tok)
