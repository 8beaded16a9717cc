"""Dense SwiGLU MLPs (Mlp::forward, src/model.rs:20-40; Ffn::Dense at
src/model.rs:840) on the expert kernels, against the CPU path's MLP."""
import numpy as np
import pytest

from gpu_util import TOL, log, record, rel_err

pytestmark = pytest.mark.gpu

SEED = 7


@pytest.fixture(scope="module")
def ctx():
    import torch

    assert torch.cuda.is_available(), "no GPU visible"
    from moe_amd.layer import Context

    return Context(0)


_cache = {}


def mlp_pair(ctx, oracle, name, **kw):
    """(GPU Mlp, oracle QTs, host bytes) for one expert of a shape."""
    from moe_amd import synth
    from moe_amd.layer import Mlp, Store

    key = (name, tuple(sorted(kw.items())))
    if key not in _cache:
        shape = synth.scaled(synth.SHAPES[name], n_experts=1, top_k=1, n_group=1, topk_group=1, shared_inter=0,
                             e_bias_std=0.0, shared_gate=False, zipf=0.0, **kw)
        log(f"building MLP {name} {kw} H={shape.hidden} I={shape.inter}")
        host = synth.build_host_layer(shape, SEED)
        region = ctx.upload(host.buf)
        store = Store(region, host.index)
        H, I, dt = shape.hidden, shape.inter, shape.expert_dt
        mlp = Mlp(ctx, store.view("experts.gate", 0, 0, I), store.view("experts.up", 0, 0, I),
                  store.view("experts.down", 0, 0, H))
        mlp._region = region
        qts = (oracle.qt(dt, I, H, host.tensor("experts.gate")), oracle.qt(dt, I, H, host.tensor("experts.up")),
               oracle.qt(dt, H, I, host.tensor("experts.down")))
        _cache[key] = (mlp, qts, host)
    return _cache[key]


def run(mlp, x, mode=0, residual=None):
    import torch

    dev = torch.device("cuda:0")
    mlp.set_mode(mode)
    try:
        xd = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
        out = torch.full_like(xd, float("nan"))
        res = torch.from_numpy(residual).to(dev) if residual is not None else None
        mlp.forward(xd, out, residual=res)
        torch.cuda.synchronize()
        return out.cpu().numpy(), (res.cpu().numpy() if res is not None else None)
    finally:
        mlp.set_mode(0)


# (shape whose expert is used, extra shape changes, tokens): T = 1 takes the
# one-token kernels, a few tokens the few-tokens kernels, more the MFMA ones.
CASES = [
    ("tiny_mixtral", {}, 1), ("tiny_mixtral", {}, 6), ("tiny_mixtral", {}, 200),
    ("mixtral", {}, 1), ("mixtral", {}, 24), ("mixtral", {}, 320),
    ("deepseek_v3", {"expert_dt": 6}, 1), ("deepseek_v3", {"expert_dt": 6}, 9), ("deepseek_v3", {"expert_dt": 6}, 161),
]


@pytest.mark.parametrize("name,kw,t", CASES, ids=[f"{n}-{'q5' if kw else 'base'}-{t}" for n, kw, t in CASES])
def test_mlp_matches_cpu_path(ctx, oracle, name, kw, t):
    from moe_amd import synth

    mlp, qts, host = mlp_pair(ctx, oracle, name, **kw)
    x = synth.activations(SEED, t, mlp.hidden)
    want = oracle.mlp_forward(*qts, x)
    log(f"MLP {name} {kw} T={t}")
    got, _ = run(mlp, x)
    assert np.isfinite(got).all()
    err = rel_err(got, want)
    record("mlp", f"{name}{' Q5_0' if kw else ''} T={t}", err)
    assert err <= TOL, f"max rel err {err:.2e}"


@pytest.mark.parametrize("t", [1, 5, 33])
def test_mlp_exact_path_bit_identical(ctx, oracle, t):
    """With the exact kernels the routing weight 1 and the combine's 0 + 1 * y
    leave the MLP's output bit for bit the CPU path's."""
    from moe_amd import synth

    mlp, qts, host = mlp_pair(ctx, oracle, "tiny_mixtral")
    x = synth.activations(SEED + 3, t, mlp.hidden)
    want = oracle.mlp_forward(*qts, x)
    got, _ = run(mlp, x, mode=1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_mlp_residual(ctx, oracle):
    from moe_amd import synth

    mlp, qts, host = mlp_pair(ctx, oracle, "tiny_mixtral")
    x = synth.activations(SEED + 5, 3, mlp.hidden)
    r0 = synth.normal(SEED, 77, 3 * mlp.hidden).reshape(3, mlp.hidden)
    got, res = run(mlp, x, residual=r0)
    np.testing.assert_array_equal(res, r0 + got)


def test_mlp_rejects_mismatched_views(ctx, oracle):
    from moe_amd.layer import Mlp, View

    g = View(8, 64, 128, 0, 0)
    with pytest.raises(ValueError):
        Mlp(ctx, g, View(8, 64, 128, 0, 0), View(8, 64, 128, 0, 0))
