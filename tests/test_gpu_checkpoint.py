"""Layers read from checkpoint files: a synthetic layer packed as .moe and
as GGUF, parsed by the library, uploaded with every tensor 256-byte aligned
(the .moe payload is unaligned), bound by name as the reference binds a
layer (src/model.rs:396-441), and run.  The output must equal the same
layer uploaded directly bit for bit (same bytes, same kernels), and the
CPU path within the usual bar."""
import numpy as np
import pytest

from gguf_writer import GgufWriter
from gpu_util import TOL, assert_routing_equal, log, record, rel_err, run_gpu

pytestmark = pytest.mark.gpu

CASES = [
    # (shape, scale, T): softmax top-2; sigmoid + bias + groups + Q5_0 shared expert; two shared experts
    ("tiny_mixtral", {}, 7),
    ("deepseek_v3", dict(hidden=512, inter=128, shared_inter=128), 40),
    ("v2_lite", dict(hidden=1024, inter=256, shared_inter=512), 33),
]


def gguf_of(host, layer: int) -> bytes:
    """The layer under GGUF's names (blk.L.ffn_*_exps, ffn_*_shexp, ...)."""
    names = {"router": "ffn_gate_inp.weight", "e_bias": "exp_probs_b.bias", "experts.gate": "ffn_gate_exps.weight",
             "experts.up": "ffn_up_exps.weight", "experts.down": "ffn_down_exps.weight",
             "shared.gate": "ffn_gate_shexp.weight", "shared.up": "ffn_up_shexp.weight",
             "shared.down": "ffn_down_shexp.weight", "shared_gate": "ffn_gate_inp_shexp.weight"}
    w = GgufWriter(32)
    w.kv_str("general.architecture", "deepseek2")
    for key, rec in host.index.items():
        if key == "e_bias":
            shape = [rec.cols]
        else:
            shape = [rec.slabs, rec.rows, rec.cols] if rec.slabs > 1 else [rec.rows, rec.cols]
        w.tensor(f"blk.{layer}.{names[key]}", shape, rec.dt, host.tensor(key).tobytes())
    return w.build()


@pytest.mark.parametrize("fmt", ["moe", "gguf"])
@pytest.mark.parametrize("name,scale,t", CASES)
def test_layer_from_checkpoint(tmp_path, oracle, fmt, name, scale, t):
    import torch

    from moe_amd import checkpoint, synth
    from moe_amd.layer import Context

    assert torch.cuda.is_available(), "no GPU visible"
    shape = synth.scaled(synth.SHAPES[name], **scale) if scale else synth.SHAPES[name]
    host = synth.build_host_layer(shape, 5)
    layer_no = 3
    path = str(tmp_path / f"layer.{fmt}")
    if fmt == "moe":
        checkpoint.write_moe(path, checkpoint.host_layer_tensors(host, layer=layer_no), config={"n_routed": 1})
    else:
        open(path, "wb").write(gguf_of(host, layer_no))
    ctx = Context(0)
    c = checkpoint.Container(path)
    try:
        names = checkpoint.layer_tensor_names(c, layer_no, shape.n_experts)
        store = checkpoint.upload(ctx, c, names)
        assert all(r.offset % 256 == 0 for r in store.index.values())
        gl = checkpoint.bind_layer(ctx, store, layer_no, shape.spec())
        direct = synth.make_layer(ctx, host)
        x = synth.activations(5, t, shape.hidden)
        g = run_gpu(gl, x)
        d = run_gpu(direct, x)
        assert np.array_equal(g["out"].view(np.uint32), d["out"].view(np.uint32)), "differs from the direct upload"
        out, sel, w, hits, stats = oracle.from_host_layer(host).forward(x)
        assert_routing_equal(g, sel, w, f"{name} from .{fmt}")
        err = rel_err(g["out"], out)
        log(f"{name} from .{fmt}: {len(names)} tensors, max rel err {err:.2e}")
        record("checkpoint", f"{name} from .{fmt} T={t}", err)
        assert err <= TOL
    finally:
        c.close()
