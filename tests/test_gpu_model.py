"""Whole decoders on the GPU (the reference's Model::forward,
src/model.rs:565-834, with every operation in libmoe_hip) against the CPU
oracle's whole-model forward and the reference's golden logits, plus the
plain projections (quant::matmul, src/quant.rs:482-506) on the expert
kernels.

Configs: the four golden fixtures (F32 and packed), BASELINE configs[0] (the
tiny Mixtral, 32 greedy tokens from a 16-token random prompt) and configs[4]
(DeepSeek-V2-Lite, 27 layers, 32 sequences of 256 random tokens then 128
greedy steps, the routed layers seeing T = 32 rows per step).
"""
import time

import numpy as np
import pytest

from gpu_util import MODEL_TOL, TOL, log, record, rel_err
from tiny_model import host_tensors

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def ctx():
    import torch

    assert torch.cuda.is_available(), "no GPU visible"
    from moe_amd.layer import Context

    return Context(0)


def gpu_model(ctx, spec, tensors):
    from moe_amd.model import Model, upload_store

    return Model(ctx, spec, upload_store(ctx, tensors))


def np_(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


FIXTURES = ["gqa", "gqa_fullnorm", "gqa_long", "mla"]


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_model_gpu(ctx, oracle, name):
    """tests/oracle.rs:45-118 on the GPU forward: forward_all within 5e-3 of
    the golden logits at every position with the argmax kept, one token at a
    time within 5e-3 at every step, a split prefill within 1e-4 of a whole
    one; and every call within MODEL_TOL of the oracle model."""
    m, spec, tensors = host_tensors(name)
    om = oracle.OracleModel(spec, tensors)
    gm = gpu_model(ctx, spec, tensors)
    try:
        got = np_(gm.forward_all(m.tokens, gm.new_state(1, 32)))
        assert np.abs(got - m.expected).max() < 5e-3
        assert (got.argmax(1) == m.expected.argmax(1)).all()
        ref = om.forward_all(m.tokens, om.new_state(32))
        e = rel_err(got, ref)
        record("test_fixture_model_gpu", f"{name} forward_all", e)
        assert e < MODEL_TOL, e
        st, ost = gm.new_state(1, 32), om.new_state(32)
        worst = 0.0
        for i, tok in enumerate(m.tokens):
            g = np_(gm.forward([[tok]], st))[0]
            assert np.abs(g - m.expected[i]).max() < 5e-3, i
            worst = max(worst, rel_err(g, om.forward([tok], ost)))
        record("test_fixture_model_gpu", f"{name} incremental", worst)
        assert worst < MODEL_TOL, worst
        st2 = gm.new_state(1, 32)
        h = len(m.tokens) // 2
        gm.forward([m.tokens[:h]], st2)
        split = np_(gm.forward([m.tokens[h:]], st2))[0]
        assert np.abs(split - got[-1]).max() < 1e-4
    finally:
        gm.close()


@pytest.mark.parametrize("name,dt,tol", [("gqa", 8, 0.25), ("mla", 8, 0.25), ("gqa", 6, 0.7), ("mla", 6, 0.7),
                                         ("gqa", 2, 1.5), ("mla", 2, 1.5)])
def test_fixture_packed_model_gpu(ctx, oracle, name, dt, tol):
    """tests/oracle.rs:78-94: packed checkpoints keep the prediction, and
    the GPU forward stays within MODEL_TOL of the oracle's."""
    m, spec, tensors = host_tensors(name, dt)
    om = oracle.OracleModel(spec, tensors)
    gm = gpu_model(ctx, spec, tensors)
    try:
        got = np_(gm.forward([m.tokens], gm.new_state(1, 32)))[0]
        assert np.abs(got - m.expected[-1]).max() < tol
        assert got.argmax() == m.expected[-1].argmax()
        e = rel_err(got, om.forward(m.tokens, om.new_state(32)))
        record("test_fixture_packed_model_gpu", f"{name} dt={dt}", e)
        assert e < MODEL_TOL, e
    finally:
        gm.close()


def test_fixture_batched_sequences_gpu(ctx, oracle):
    """Several sequences in one call (the batch the routed layers see) give
    each sequence what it gets alone: three prompts of different lengths,
    then two decode steps, each against the oracle's single-sequence run."""
    m, spec, tensors = host_tensors("mla")
    om = oracle.OracleModel(spec, tensors)
    gm = gpu_model(ctx, spec, tensors)
    try:
        prompts = [m.tokens, m.tokens[:2], [5, 9, 40, 1]]
        st = gm.new_state(3, 16)
        osts = [om.new_state(16) for _ in prompts]
        logits = np_(gm.forward(prompts, st))
        for i, p in enumerate(prompts):
            assert rel_err(logits[i], om.forward(p, osts[i])) < MODEL_TOL
        for step in range(2):
            nxt = [int(v) for v in logits.argmax(1)]
            logits = np_(gm.forward([[t] for t in nxt], st))
            for i in range(3):
                e = rel_err(logits[i], om.forward([nxt[i]], osts[i]))
                assert e < MODEL_TOL, (step, i, e)
        assert st.pos == [len(p) + 2 for p in prompts]
    finally:
        gm.close()


# ---------------------------------------------------------------- (f)3

_LINEAR = {}


def _linear_case(ctx, model, name):
    """One tensor of a synthetic model: (Linear, host bytes, dt, rows, cols)."""
    from moe_amd import synth
    from moe_amd.layer import Store, View
    from moe_amd.model import Linear

    key = (model, name)
    if key not in _LINEAR:
        shape = synth.MODEL_SHAPES[model]
        (n, dt, sh, fill), = [p for p in shape.plan() if p[0] == name]
        rows, cols = sh
        from moe_amd.layer import row_bytes

        buf = np.empty(rows * row_bytes(dt, cols), dtype=np.uint8)
        synth._fill(buf, 11, synth._name_stream(name), dt, rows, cols, 0.0, shape.weight_std)
        region = ctx.upload(buf)
        lin = Linear(ctx, View(dt, rows, cols, region.id, 0))
        lin._region = region
        _LINEAR[key] = (lin, buf, dt, rows, cols)
    return _LINEAR[key]


LINEAR_CASES = [("tiny_mixtral", "model.layers.0.self_attn.q_proj.weight"),
                ("tiny_mixtral", "model.layers.0.self_attn.k_proj.weight"),
                ("tiny_mixtral", "lm_head.weight"),
                ("v2_lite", "model.layers.1.self_attn.q_proj.weight"),
                ("v2_lite", "model.layers.1.self_attn.kv_a_proj_with_mqa.weight"),
                ("v2_lite", "model.layers.1.self_attn.kv_b_proj.weight"),
                ("v2_lite", "model.layers.1.self_attn.o_proj.weight"),
                ("v2_lite", "lm_head.weight")]


@pytest.mark.parametrize("model,name", LINEAR_CASES)
@pytest.mark.parametrize("t", [1, 6, 32, 300])
def test_linear_gpu(ctx, oracle, model, name, t):
    """moe_linear (the f32 GEMV up to 8 rows, the MFMA kernel beyond)
    against oracle.matmul at the configs' projection shapes, with and
    without the fused residual add."""
    import torch

    lin, buf, dt, rows, cols = _linear_case(ctx, model, name)
    rng = np.random.default_rng(rows + t)
    x = rng.standard_normal((t, cols)).astype(np.float32)
    ref = oracle.matmul(oracle.qt(dt, rows, cols, buf), x)
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    y = torch.full((t, rows), float("nan"), dtype=torch.float32, device=dev)
    ws = torch.zeros(lin.workspace_size(t) + 256, dtype=torch.uint8, device=dev)
    off = (-ws.data_ptr()) % 256
    ws = ws[off:off + lin.workspace_size(t)]
    lin(xd, y, ws)
    got = np_(y)
    e = rel_err(got, ref)
    record("test_linear_gpu", f"{model} {name.split('.')[-2]} T={t}", e)
    assert e < TOL, e
    res = rng.standard_normal((t, rows)).astype(np.float32)
    rd = torch.from_numpy(res).to(dev)
    lin(xd, y, ws, residual=rd)
    # residual += y, one f32 addition per element.
    assert np.array_equal(np_(rd), res + got)


@pytest.mark.parametrize("t", [1, 5, 16])
def test_linear_f32_exact_gpu(ctx, oracle, t):
    """F32 weights take the exact kernel: bit-identical to the oracle's dot."""
    import torch
    from moe_amd.layer import View
    from moe_amd.model import Linear

    rng = np.random.default_rng(t)
    w = rng.standard_normal((48, 32)).astype(np.float32)
    region = ctx.upload(w.view(np.uint8).reshape(-1))
    lin = Linear(ctx, View(0, 48, 32, region.id, 0))
    x = rng.standard_normal((t, 32)).astype(np.float32)
    ref = oracle.matmul(oracle.qt(0, 48, 32, w.view(np.uint8).reshape(-1)), x)
    dev = torch.device("cuda:0")
    y = torch.empty((t, 48), dtype=torch.float32, device=dev)
    ws = torch.zeros(512, dtype=torch.uint8, device=dev)
    off = (-ws.data_ptr()) % 256
    lin(torch.from_numpy(x).to(dev), y, ws[off:off + 256])
    assert np.array_equal(np_(y).view(np.uint32), ref.view(np.uint32))
    lin.close()


# ------------------------------------------------------- configs 0 and 4


def test_config1_tiny_mixtral_greedy_gpu(ctx, oracle):
    """the tiny Mixtral (2 layers, hidden 512, 8 heads,
    8 experts top-2 of 1408, vocab 32000, Q8_0 from N(0, 0.02)), 16 random
    prompt ids (seed 0), 32 greedy tokens.  The GPU's token sequence equals
    the CPU path's, and every step's logits are within MODEL_TOL."""
    from moe_amd import synth
    from moe_amd.model import Spec

    cfg, ck = synth.build_host_model(synth.MODEL_SHAPES["tiny_mixtral"], 0)
    spec = Spec.derive(cfg, {k: v.shape for k, v in ck.items()})
    prompt = synth.prompt_ids(0, 16, spec.vocab)
    om = oracle.OracleModel(spec, ck)
    want = om.generate_greedy(prompt, 32)
    gm = gpu_model(ctx, spec, ck)
    try:
        st = gm.new_state(1, 48)
        ost = om.new_state(48)
        toks, worst, feed = [], 0.0, list(prompt)
        for step in range(32):
            g = np_(gm.forward([feed], st))[0]
            r = om.forward(feed, ost)
            worst = max(worst, rel_err(g, r))
            toks.append(int(np.argmax(g)))
            feed = [toks[-1]]
        record("test_config1_tiny_mixtral_greedy_gpu", "32 steps", worst)
        log(f"config 1: {toks}")
        assert toks == want
        assert worst < MODEL_TOL, worst
        assert gm.generate_greedy([prompt], 32)[0] == want
    finally:
        gm.close()


@pytest.mark.timeout(900)
def test_config5_v2_lite_batched_gpu(ctx, oracle):
    """DeepSeek-V2-Lite (27 layers, MLA with kv_lora
    512, layer 0 dense, 64 routed experts top-6 plus 2 shared, vocab 102400,
    Q8_0 from N(0, 0.02)), 32 sequences of 256 random ids, then 128 greedy
    steps of all 32 at once (T = 32 rows per routed layer per step).
    Against the CPU path (the oracle fed the GPU's tokens): the prefill
    logits and all 127 steps after it of sequences 0 and 31 (the batch's
    first and last rows) within MODEL_TOL with the same argmax at every step
    (the smallest top-1 / top-2 logit margin of the CPU path is recorded); and
    sequences 0 and 31 run alone on the GPU produce the same 128 tokens as
    in the batch."""
    import torch

    from moe_amd import synth
    from moe_amd.model import Spec

    t0 = time.time()
    cfg, ck = synth.build_host_model(synth.MODEL_SHAPES["v2_lite"], 0)
    spec = Spec.derive(cfg, {k: v.shape for k, v in ck.items()})
    log(f"config 5: {ck.buf.nbytes / 2**30:.1f} GiB of weights built in {time.time() - t0:.0f} s")
    n_seq, plen, steps = 32, 256, 128
    prompts = [synth.prompt_ids(s, plen, spec.vocab) for s in range(n_seq)]
    gm = gpu_model(ctx, spec, ck)
    log(f"config 5: uploaded at {time.time() - t0:.0f} s")
    try:
        st = gm.new_state(n_seq, plen + steps)
        torch.cuda.synchronize()
        t1 = time.time()
        logits = gm.forward(prompts, st)
        first = np_(logits)
        t2 = time.time()
        toks = [[int(v)] for v in first.argmax(1)]
        last = n_seq - 1
        step_logits = {0: [], last: []}  # GPU logits of the pinned sequences, steps 1 ..
        for step in range(1, steps):
            lg = gm.forward([[tk[-1]] for tk in toks], st)
            nxt = gm.argmax(lg).cpu().tolist()
            step_logits[0].append(lg[0].cpu().numpy())
            step_logits[last].append(lg[last].cpu().numpy())
            for i in range(n_seq):
                toks[i].append(int(nxt[i]))
        torch.cuda.synchronize()
        t3 = time.time()
        log(f"config 5: prefill {n_seq}x{plen} in {t2 - t1:.2f} s, {steps - 1} batched steps in {t3 - t2:.2f} s "
            f"({n_seq * (steps - 1) / (t3 - t2):.0f} tok/s)")
        record("test_config5_v2_lite_batched_gpu", "timing", 0.0, prefill_s=t2 - t1, decode_s=t3 - t2,
               decode_tok_s=n_seq * (steps - 1) / (t3 - t2))
        # Sequences 0 and 31, every step, on the CPU path.
        om = oracle.OracleModel(spec, ck)

        def margin(r):
            top2 = np.partition(r, -2)[-2:]
            return float(top2[1] - top2[0])

        for s, n in ((0, steps - 1), (last, steps - 1)):
            ost = om.new_state(plen + steps)
            r = om.forward(prompts[s], ost)
            worst = rel_err(first[s], r)
            least = (margin(r), 0)
            assert int(np.argmax(r)) == toks[s][0], (s, 0)
            for step in range(1, n + 1):
                r = om.forward([toks[s][step - 1]], ost)
                worst = max(worst, rel_err(step_logits[s][step - 1], r))
                least = min(least, (margin(r), step))
                assert int(np.argmax(r)) == toks[s][step], (s, step)
            log(f"config 5: sequence {s} vs the CPU path over prefill + {n} steps: {worst:.2e}, smallest top-1/top-2 "
                f"margin {least[0]:.3e} at step {least[1]} (at {time.time() - t0:.0f} s)")
            record("test_config5_v2_lite_batched_gpu", f"seq {s} prefill + {n} steps", worst,
                   min_top2_margin=least[0], min_margin_step=least[1])
            assert worst < MODEL_TOL, (s, worst)
        # Batched == alone.
        for s in (0, n_seq - 1):
            alone = gm.generate_greedy([prompts[s]], steps)[0]
            assert alone == toks[s], s
        log(f"config 5: done at {time.time() - t0:.0f} s")
    finally:
        gm.close()
