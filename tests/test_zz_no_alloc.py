"""The allocation-free entry point (moe_layer_forward_noalloc) against the
ordinary one (moe_layer_forward): the same kernels on the same inputs, so the
outputs, routes, hits and counters must agree bit for bit, on two calls in a
row — the second with fewer tokens, so it reuses the static scratch array
the first one left behind — and on every kernel path a small call takes."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import TOL, log, rel_err, run_gpu

pytestmark = pytest.mark.gpu
SEED = 3


def _noalloc(layer, x):
    import torch

    from moe_amd import _lib as L

    t, H = x.shape
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    out = torch.full((t, H), float("nan"), dtype=torch.float32, device=dev)
    routes = torch.empty((t, layer.k, 2), dtype=torch.int32, device=dev)
    hits = torch.full((layer.spec.n_experts + 1,), -1, dtype=torch.int32, device=dev)
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    rc = L.lib().moe_layer_forward_noalloc(layer.handle, C.c_void_p(xd.data_ptr()), t, C.c_void_p(out.data_ptr()),
                                           None, C.c_void_p(routes.data_ptr()), C.c_void_p(hits.data_ptr()), None,
                                           C.c_void_p(stats.data_ptr()),
                                           C.c_void_p(torch.cuda.current_stream().cuda_stream))
    L.check(rc, "moe_layer_forward_noalloc")
    torch.cuda.synchronize()
    r = routes.cpu().numpy()
    return dict(out=out.cpu().numpy(), sel=r[..., 0], w=r[..., 1].view(np.float32),
                hits=hits.cpu().numpy(), stats=stats.cpu().numpy())


@pytest.mark.parametrize("name,ts", [("tiny_mixtral", (40, 7)), ("mixtral", (12, 1)), ("qwen2_moe", (24, 1))])
def test_noalloc_matches_forward(name, ts):
    import torch

    from moe_amd import synth
    from moe_amd.layer import Context

    assert torch.cuda.is_available(), "no GPU visible"
    ctx = Context(0)
    host = synth.build_host_layer(synth.SHAPES[name], SEED)
    layer = synth.make_layer(ctx, host)
    try:
        for t in ts:  # the second call is smaller and finds the first one's leftovers
            x = synth.activations(SEED + t, t, host.shape.hidden)
            want = run_gpu(layer, x)
            got = _noalloc(layer, x)
            log(f"{name} T={t}: noalloc vs forward max rel err {rel_err(got['out'], want['out']):.2e}")
            assert np.array_equal(got["sel"], want["sel"]) and np.array_equal(got["w"].view(np.uint32),
                                                                                want["w"].view(np.uint32))
            n = int(want["hits"][0])
            assert np.array_equal(got["hits"][:n + 1].view(np.uint32), want["hits"][:n + 1])
            assert np.array_equal(got["stats"][:3].view(np.uint64), want["stats"][:3])
            assert rel_err(got["out"], want["out"]) <= TOL
            assert np.array_equal(got["out"].view(np.uint32), want["out"].view(np.uint32))
    finally:
        layer.close()
        ctx.close()


def test_noalloc_refuses_oversized_calls():
    """A call whose workspace would not fit the static array fails cleanly."""
    import torch

    from moe_amd import _lib as L
    from moe_amd import synth
    from moe_amd.layer import Context

    ctx = Context(0)
    host = synth.build_host_layer(synth.SHAPES["tiny_mixtral"], SEED)
    layer = synth.make_layer(ctx, host)
    try:
        t = 1
        while layer.workspace_size(t) <= 64 << 20:
            t *= 2
        x = torch.zeros((t, 512), dtype=torch.float32, device="cuda:0")
        out = torch.empty_like(x)
        rc = L.lib().moe_layer_forward_noalloc(layer.handle, C.c_void_p(x.data_ptr()), t, C.c_void_p(out.data_ptr()),
                                               None, None, None, None, None, None)
        assert rc == L.MOE_EINVAL
        assert b"scratch" in L.lib().moe_last_error()
    finally:
        layer.close()
        ctx.close()
