"""Pins the oracle's dot product (lane and reduction order) and its routing
(softmax / sigmoid, bias, group pruning, top-k, weights, interventions).

Known answers are built so that a different summation order, a dropped
term, a transposed operand or a wrong tie rule gives a different result.
"""
import math

import numpy as np
import pytest

F32 = 0


def test_dot_vector_equals_scalar_restatement(oracle):
    """The AVX2 kernel and the scalar fmaf restatement agree bit for bit, at
    lengths exercising the 16-chunk loop, the 8-chunk step and the tail."""
    rng = np.random.default_rng(1)
    for n in list(range(1, 70)) + [1000, 4096, 4104, 7168, 14336]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert oracle.dot(a, b) == oracle.dot(a, b, scalar=True), n


def test_dot_lane_structure_known_answers(oracle):
    """Products placed so each order gives a different sum.  Lane j of the
    16-chunk loop accumulates elements j, j+16, ...; lanes j and j+8 are added
    first, then j+4 and j, then (q0+q1)+(q2+q3); the scalar tail last."""
    big = np.float32(2.0**24)
    a = np.zeros(16, dtype=np.float32)
    a[0], a[1], a[8], a[9] = big, 1, -big, 1
    b = np.ones(16, dtype=np.float32)
    # lanes: s0 = 2^24 + -2^24 = 0, s1 = 1 + 1 = 2 -> 2.  A left-to-right sum gives 1.
    assert oracle.dot(a, b) == 2.0
    # Lane pairing (j, j+4): s0 = 2^24, s4 = 1 -> q0 = 2^24 (1 lost), q1 = s1 + s5 = 1 + 1.
    a = np.zeros(16, dtype=np.float32)
    a[0], a[4], a[1], a[5] = big, 1, 1, 1
    assert oracle.dot(a, b) == float(big + 2)
    # The 8-chunk step feeds acc0 only: n = 24, element 16 lands in lane 0 with 2^24.
    a = np.zeros(24, dtype=np.float32)
    a[0], a[16], a[8] = big, 1, 1
    # acc0[0] = 2^24 + 1 -> 2^24 (rounded), acc1[0] = 1 -> s0 = 2^24 + 1 -> 2^24.
    assert oracle.dot(a, np.ones(24, dtype=np.float32)) == float(big)
    # The scalar tail is added after the tree: n = 17, tail element 16.
    a = np.zeros(17, dtype=np.float32)
    a[0], a[16] = big, 1
    assert oracle.dot(a, np.ones(17, dtype=np.float32)) == float(big)  # 2^24 + 1 rounds back
    a[16] = 2
    assert oracle.dot(a, np.ones(17, dtype=np.float32)) == float(big + 2)


def test_dot_error_bound(oracle):
    rng = np.random.default_rng(2)
    for n in (64, 4096, 14336):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = (n + 8) * 2.0**-24 * float(np.abs(a.astype(np.float64) * b).sum())
        assert abs(float(oracle.dot(a, b)) - exact) <= bound


def test_matmul_matches_naive(oracle):
    """src/quant.rs:608-627: 35 x 64 weights over 3 tokens vs a triple loop."""
    rows, cols, t = 35, 64, 3
    w = np.array([((i % 13) - 6.0) / 7.0 for i in range(rows * cols)], dtype=np.float32).reshape(rows, cols)
    x = np.array([((i % 9) - 4.0) / 5.0 for i in range(t * cols)], dtype=np.float32).reshape(t, cols)
    qt = oracle.qt(F32, rows, cols, w.view(np.uint8).reshape(-1))
    got = oracle.matmul(qt, x)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - want).max() < 1e-3
    # and each element is exactly one dot() of a row with a token
    for ti in range(t):
        for r in range(rows):
            assert got[ti, r] == oracle.dot(w[r], x[ti])


# ------------------------------------------------------------------ routing


def _layer(oracle, logits_by_expert_basis, **kw):
    """A layer whose router makes logits[t][e] = x[t][e] exactly: W = I."""
    E = logits_by_expert_basis
    H = 16
    router = np.zeros((E, H), dtype=np.float32)
    router[np.arange(E), np.arange(E)] = 1.0
    dummy = np.zeros(18, dtype=np.uint8)
    experts = [[(2, 1, H, np.zeros(9, dtype=np.uint8)), (2, 1, H, np.zeros(9, dtype=np.uint8)),
                (F32, H, 1, np.zeros(4 * H, dtype=np.uint8))] for _ in range(E)]
    del dummy
    return oracle.OracleLayer(H, E, kw.pop("top_k", 2), router, experts, **kw)


def _x(rows):
    x = np.zeros((len(rows), 16), dtype=np.float32)
    for i, r in enumerate(rows):
        x[i, :len(r)] = r
    return x


def test_softmax_top2_closed_form(oracle):
    ol = _layer(oracle, 4)
    sel, w, logits, ties = ol.route(_x([[1.0, 3.0, 2.0, 0.0]]))
    assert logits[0].tolist() == [1.0, 3.0, 2.0, 0.0]
    assert sel[0].tolist() == [1, 2] and ties == 0
    e3, e2 = math.exp(3.0), math.exp(2.0)
    assert w[0] == pytest.approx([e3 / (e3 + e2), e2 / (e3 + e2)], rel=1e-6)
    assert w[0].sum() == pytest.approx(1.0, abs=1e-6)


def test_ties_go_to_the_lower_index(oracle):
    ol = _layer(oracle, 8, top_k=3)
    sel, w, _, ties = ol.route(_x([[0.5, 2.0, 0.5, 2.0, 0.1, 2.0, 0.0, 0.0]]))
    assert sel[0].tolist() == [1, 3, 5]
    assert ties == 1
    assert w[0][0] == w[0][1] == w[0][2]


def test_no_renormalisation_and_scale(oracle):
    ol = _layer(oracle, 4, norm_topk=False, routed_scale=2.0)
    sel, w, _, _ = ol.route(_x([[1.0, 3.0, 2.0, 0.0]]))
    s = sum(math.exp(v) for v in (1.0, 3.0, 2.0, 0.0))
    assert w[0] == pytest.approx([2 * math.exp(3) / s, 2 * math.exp(2) / s], rel=1e-6)


def test_sigmoid_bias_and_group_pruning(oracle):
    """DeepSeek-style: rank = sigmoid(logit) + bias; 4 groups of 2, keep the 2
    groups with the strongest pairs; top-3 from those; weights are the
    unbiased sigmoid scores, renormalised, times the routed scale."""
    logits = [2.0, -1.0, 0.5, 0.4, 3.0, -3.0, 0.1, 0.2]
    bias = np.array([0.0, 0.0, 0.3, 0.3, -1.0, 0.0, 0.0, 0.0], dtype=np.float32)
    ol = _layer(oracle, 8, top_k=3, sigmoid=True, e_bias=bias, n_group=4, topk_group=2, routed_scale=2.5)
    sig = [1 / (1 + math.exp(-v)) for v in logits]
    rank = [s + b for s, b in zip(sig, bias)]
    # group pair sums: g0 = r0 + r1, g1 = r2 + r3, g2 = r4 + r5, g3 = r6 + r7
    sums = [rank[0] + rank[1], rank[2] + rank[3], rank[4] + rank[5], rank[6] + rank[7]]
    keep = sorted(range(4), key=lambda g: -sums[g])[:2]
    assert keep == [1, 0]  # expert 4 has the largest score but its group is pruned by the bias
    cands = [e for e in range(8) if e // 2 in keep]
    top = sorted(cands, key=lambda e: -rank[e])[:3]
    sel, w, _, _ = ol.route(_x([logits]))
    assert sel[0].tolist() == top == [2, 3, 0]
    z = sum(sig[e] for e in top)
    assert w[0] == pytest.approx([2.5 * sig[e] / z for e in top], rel=1e-6)
    assert 4 not in sel[0]


def test_invariants_like_the_reference_trace_test(oracle):
    """tests/oracle.rs:647-671: k experts per token, strongest first, weights
    descending and summing to the routed scale (softmax gate)."""
    rng = np.random.default_rng(3)
    for scale in (1.0, 1.5):
        ol = _layer(oracle, 8, top_k=3, routed_scale=scale)
        x = rng.standard_normal((50, 16)).astype(np.float32)
        sel, w, logits, _ = ol.route(x)
        assert sel.shape == (50, 3)
        for t in range(50):
            assert len(set(sel[t].tolist())) == 3
            assert (np.diff(w[t]) <= 0).all()
            assert abs(w[t].sum() - scale) < 1e-4
            assert (logits[t][sel[t]] >= np.sort(logits[t])[-3]).all()


def test_interventions(oracle):
    """tests/oracle.rs:264-344 restated on the routing table."""
    rng = np.random.default_rng(4)
    ol = _layer(oracle, 8, top_k=2)
    x = rng.standard_normal((40, 16)).astype(np.float32)
    sel, w, _, _ = ol.route(x)
    victim = int(sel[0, 0])
    s2, w2, _, _ = ol.route(x, oracle.OracleLayer.routing(disabled=[victim]))
    assert victim not in s2 and s2.shape == sel.shape
    target = (victim + 1) % 8
    s3, _, _, _ = ol.route(x, oracle.OracleLayer.routing(forced=[target]))
    assert all(target in r for r in s3.tolist())
    assert oracle.OracleLayer.routing(top_k=1) and ol.route(x, oracle.OracleLayer.routing(top_k=1))[0].shape[1] == 1
    assert ol.route(x, oracle.OracleLayer.routing(top_k=8))[0].shape[1] == 8
    _, w5, _, _ = ol.route(x, oracle.OracleLayer.routing(temp=50.0))
    assert np.abs(w5.sum(1) - 1).max() < 1e-3 and (w5 >= 0).all()
    # a forced expert displaces the weakest pick and is re-sorted by rank
    s6, _, lg, _ = ol.route(x[:1], oracle.OracleLayer.routing(forced=[int(np.argsort(x[0, :8])[0])]))
    f = int(np.argsort(x[0, :8])[0])
    assert s6[0].tolist() == [int(sel[0, 0]), f]


def test_forward_single_expert_matches_mlp(oracle):
    """With top_k = E = 1 and weight 1 the layer is exactly one SwiGLU MLP."""
    rng = np.random.default_rng(5)
    H, I = 64, 32
    g = rng.standard_normal((I, H)).astype(np.float32) * 0.1
    u = rng.standard_normal((I, H)).astype(np.float32) * 0.1
    d = rng.standard_normal((H, I)).astype(np.float32) * 0.1
    ex = [[(F32, I, H, g.view(np.uint8).reshape(-1)), (F32, I, H, u.view(np.uint8).reshape(-1)),
           (F32, H, I, d.view(np.uint8).reshape(-1))]]
    ol = oracle.OracleLayer(H, 1, 1, np.ones((1, H), dtype=np.float32), ex)
    x = rng.standard_normal((5, H)).astype(np.float32)
    out, sel, w, hits, stats = ol.forward(x)
    assert (sel == 0).all() and (w == 1.0).all() and hits[:2].tolist() == [1, 0]
    gx, ux = x.astype(np.float64) @ g.T, x.astype(np.float64) @ u.T
    ref = ((gx / (1 + np.exp(-gx))) * ux) @ d.T
    assert np.abs(out - ref).max() < 1e-5 * np.abs(ref).max() + 1e-6
    assert stats.tolist() == [5, 0, 3 * 4 * H * I, 0]


def test_mlp_is_swiglu_of_the_matmuls(oracle):
    """Mlp::forward (src/model.rs:26-35) is down(silu(g) * u) with
    g = matmul(gate, x), u = matmul(up, x) and silu(g) = g / (1 + exp(-g)):
    divide, then multiply, each rounded to f32, exp from glibc.  The
    composition from the pinned matmul and expf equals the oracle's MLP bit
    for bit; dropping the divide's order (g * sigmoid(g)) or fusing breaks
    it somewhere on these inputs."""
    from moe_amd import synth

    H, I, t = 128, 96, 5
    rng = np.random.default_rng(11)
    w = {n: (rng.standard_normal((r, c)) * 0.2).astype(np.float32)
         for n, r, c in [("gate", I, H), ("up", I, H), ("down", H, I)]}
    qts = {n: oracle.qt(F32, a.shape[0], a.shape[1], a.view(np.uint8).reshape(-1)) for n, a in w.items()}
    x = synth.normal(5, 1, t * H).reshape(t, H)
    got = oracle.mlp_forward(qts["gate"], qts["up"], qts["down"], x)
    g = oracle.matmul(qts["gate"], x)
    u = oracle.matmul(qts["up"], x)
    e = oracle.expf_array(-g)
    h = (g / (np.float32(1.0) + e)).astype(np.float32) * u
    want = oracle.matmul(qts["down"], h.astype(np.float32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # A plausible mistake, g * (1 / (1 + e)), rounds differently.
    h2 = (g * (np.float32(1.0) / (np.float32(1.0) + e))).astype(np.float32) * u
    assert not np.array_equal(oracle.matmul(qts["down"], h2).view(np.uint32), got.view(np.uint32))


def test_shared_expert_gate_closed_form(oracle):
    """The shared expert's sigmoid gate (src/model.rs:956-970): the layer's
    output is the routed sum plus s * Mlp_shared(x), s = 1 / (1 + exp(-g)),
    g = shared_gate . x, applied after the routed sum and not scaled by
    routed_scale.  A zero gate row gives s = 1/2 exactly; a general row is
    composed from the pinned matmul, MLP and expf bit for bit.  Plausible
    mistakes — no gate, the gate on the routed sum too, routed_scale on the
    shared expert, or sigmoid(g) written as exp(g) / (1 + exp(g)) — each
    break the equality."""
    from moe_amd import synth

    H, I, Is, t = 64, 32, 48, 6
    rng = np.random.default_rng(17)

    def mats(r_i):
        return [(rng.standard_normal(s) * 0.2).astype(np.float32) for s in ((r_i, H), (r_i, H), (H, r_i))]

    routed = mats(I)
    shared = mats(Is)
    as_qt = lambda ws: [(F32, a.shape[0], a.shape[1], a.view(np.uint8).reshape(-1)) for a in ws]
    x = synth.normal(9, 2, t * H).reshape(t, H)
    qs = [oracle.qt(F32, a.shape[0], a.shape[1], a.view(np.uint8).reshape(-1)) for a in shared]
    qr = [oracle.qt(F32, a.shape[0], a.shape[1], a.view(np.uint8).reshape(-1)) for a in routed]
    y_r = oracle.mlp_forward(*qr, x)   # one routed expert, weight 1 * routed_scale
    y_s = oracle.mlp_forward(*qs, x)
    scale = np.float32(1.5)
    for gate_row in (np.zeros(H, np.float32), (rng.standard_normal(H) * 0.3).astype(np.float32)):
        ol = oracle.OracleLayer(H, 1, 1, np.ones((1, H), dtype=np.float32), [as_qt(routed)],
                                routed_scale=float(scale), shared=as_qt(shared), shared_gate=gate_row)
        out, sel, w, _, _ = ol.forward(x)
        assert (sel == 0).all() and (w == scale).all()
        g = oracle.matmul(oracle.qt(F32, 1, H, gate_row.view(np.uint8)), x).reshape(t)
        s = (np.float32(1.0) / (np.float32(1.0) + oracle.expf_array(-g))).astype(np.float32)
        if not gate_row.any():
            assert (s == np.float32(0.5)).all()
        want = (np.float32(0.0) + scale * y_r).astype(np.float32) + (y_s * s[:, None]).astype(np.float32)
        assert np.array_equal(out.view(np.uint32), want.astype(np.float32).view(np.uint32))
        wrong = [
            (np.float32(0.0) + scale * y_r) + y_s,                                  # gate dropped
            ((np.float32(0.0) + scale * y_r) + y_s) * s[:, None],                   # gate on everything
            (np.float32(0.0) + scale * y_r) + (scale * y_s * s[:, None]),           # routed_scale on shared
        ]
        if gate_row.any():  # at g = 0 both spellings give 1/2
            eg = np.exp(g.astype(np.float32))
            wrong.append((np.float32(0.0) + scale * y_r) + y_s * (eg / (np.float32(1.0) + eg))[:, None])
        for bad in wrong:
            assert not np.array_equal(out.view(np.uint32), bad.astype(np.float32).view(np.uint32))
