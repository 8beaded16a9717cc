"""The reference's golden fixtures through the GPU routed layer.

The numpy tiny forward supplies attention and the rest of the model; every
routed layer runs through libmoe_hip.  The logits must match the reference's
expected.json at its own tolerances (tests/oracle.rs:45-94), and the routed
layer's output must equal the CPU oracle's bit for bit (these widths take the
exact kernels).
"""
import numpy as np
import pytest

from gpu_util import log
from tiny_model import TinyModel, oracle_moe_fn

pytestmark = pytest.mark.gpu


def _align(v, a=256):
    return (v + a - 1) // a * a


def gpu_moe_fn(model: TinyModel, ctx, calls: list):
    """Routed layers on the GPU; records (layer, x, out) of every call."""
    import torch

    from moe_amd import _lib as L
    from moe_amd.layer import MoeLayer, MoeSpec, View

    spec = model.routing_spec()
    layers = {}

    def build(l: int):
        mt = model.moe_tensors(l)
        parts, views = [], {}

        def add(key, dt, rows, cols, data):
            off = sum(len(p) for p in parts)
            data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            pad = np.zeros(_align(len(data)) - len(data), dtype=np.uint8)
            parts.extend([data, pad]) if len(pad) else parts.append(data)
            views[key] = (dt, rows, cols, off)

        E, H = model.n_experts, mt["router"].shape[1]
        add("router", L.DT_F32, E, H, mt["router"])
        if mt["e_bias"] is not None:
            add("e_bias", L.DT_F32, 1, E, mt["e_bias"])
        for e, mats in enumerate(mt["experts"]):
            for m, (dt, rows, cols, data) in enumerate(mats):
                add(("x", e, m), dt, rows, cols, data)
        if mt["shared"] is not None:
            for m, (dt, rows, cols, data) in enumerate(mt["shared"]):
                add(("s", m), dt, rows, cols, data)
        region = ctx.upload(np.concatenate(parts))

        def v(key):
            dt, rows, cols, off = views[key]
            return View(dt, rows, cols, region.id, off)

        ms = MoeSpec(hidden=H, n_experts=E, top_k=spec["top_k"], sigmoid=spec["sigmoid"],
                     norm_topk=spec["norm_topk"], routed_scale=spec["routed_scale"], n_group=spec["n_group"],
                     topk_group=spec["topk_group"])
        layer = MoeLayer(ctx, ms, v("router"), [(v(("x", e, 0)), v(("x", e, 1)), v(("x", e, 2))) for e in range(E)],
                         e_bias=v("e_bias") if "e_bias" in views else None,
                         shared=[v(("s", m)) for m in range(3)] if mt["shared"] is not None else None,
                         layer_index=l)
        layer._region = region
        return layer

    def fn(l: int, xn: np.ndarray) -> np.ndarray:
        if l not in layers:
            layers[l] = build(l)
        xd = torch.from_numpy(np.ascontiguousarray(xn)).cuda()
        out = torch.empty_like(xd)
        layers[l].feed_forward(xd, out)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        calls.append((l, xn.copy(), o))
        return o

    return fn


@pytest.fixture(scope="module")
def ctx():
    from moe_amd.layer import Context

    return Context(0)


@pytest.mark.parametrize("name", ["gqa", "gqa_fullnorm", "gqa_long", "mla"])
def test_fixture_logits_gpu(ctx, oracle, name):
    m = TinyModel(name)
    calls = []
    got = m.forward(gpu_moe_fn(m, ctx, calls))
    d = np.abs(got - m.expected).max()
    log(f"{name}: max |logit diff| {d:.2e}")
    assert d < 5e-3
    assert (got.argmax(1) == m.expected.argmax(1)).all()
    # Bit-identical to the CPU oracle on the same inputs.
    ofn = oracle_moe_fn(m)
    for l, xn, o in calls:
        ref = ofn(l, xn)
        assert np.array_equal(o.view(np.uint32), ref.view(np.uint32)), f"layer {l} differs from the oracle"


@pytest.mark.parametrize("name,dt,tol", [("gqa", 8, 0.25), ("mla", 8, 0.25), ("gqa", 6, 0.7), ("mla", 6, 0.7),
                                         ("gqa", 2, 1.5), ("mla", 2, 1.5)])
def test_fixture_packed_gpu(ctx, oracle, name, dt, tol):
    """Packed Q8_0/Q5_0/Q4_0 checkpoints keep the prediction (tests/oracle.rs:483-501)."""
    m = TinyModel(name, quant_dt=dt)
    calls = []
    got = m.forward(gpu_moe_fn(m, ctx, calls))
    d = np.abs(got[-1] - m.expected[-1]).max()
    assert d < tol, f"{name} dt={dt}: {d}"
    assert got[-1].argmax() == m.expected[-1].argmax()
    assert np.isfinite(got).all()
    ofn = oracle_moe_fn(m)
    for l, xn, o in calls:
        assert np.array_equal(o.view(np.uint32), ofn(l, xn).view(np.uint32))
