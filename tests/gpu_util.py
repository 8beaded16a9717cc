"""Shared helpers for the GPU parity tests."""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

# Bar of every output comparison: max |gpu - ref| / max |ref| per output
# tensor.  BASELINE.json's north_star asks for 1e-3 with f32 accumulation;
# every kernel path computes in f32 precision (f32 GEMV, three-level int8
# activations with exact integer dots, two-piece f16 MFMA operands with f32
# accumulation).  Measured on MI355X over every case of the GPU tests: the
# f32 GEMV 5e-7 .. 1e-6, the integer-dot paths 3e-7 .. 8e-7, the MFMA path
# 6e-7 .. 2.1e-6 (22-bit activation pieces); the tests hold every path to
# 5e-6, a 2.5x margin over the worst case.
TOL = 5e-6

# Bar of whole-model logits (tests/test_gpu_model.py): max |gpu - oracle| /
# max |oracle| over a call's logits.  Every operation is f32 (the
# projections and routed layers within TOL of the oracle's products, the
# norms, rope and attention in f32 with their own summation order); the
# differences compound over the layers.  Measured on MI355X: 1e-7 .. 1e-6
# on the GQA fixtures and config 1, 3e-7 .. 1.7e-5 on the mla fixture,
# whose logits move 4.8e-6 when one norm weight moves by one ulp on the CPU
# path (the GQA fixtures move 2.2e-7).
MODEL_TOL = 5e-5

# Where the per-case errors go (one JSON object per line), for the table.
ERR_LOG = os.environ.get("MOE_PARITY_LOG", os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                                         "gpurun_out", "parity_errors.jsonl"))


def record(test: str, case: str, err: float, **extra) -> None:
    """Append one measured error to ERR_LOG (best effort)."""
    try:
        os.makedirs(os.path.dirname(ERR_LOG), exist_ok=True)
        with open(ERR_LOG, "a") as f:
            f.write(json.dumps(dict(test=test, case=case, err=err, **extra)) + "\n")
    except OSError:
        pass


PROGRESS_LOG = os.path.join(os.path.dirname(ERR_LOG), "progress.log")


def log(msg: str) -> None:
    """A progress line on stdout and in PROGRESS_LOG (which a captured test
    run still shows growing while a long case runs)."""
    line = f"[{time.strftime('%H:%M:%S')}] {msg}"
    print(line, flush=True)
    sys.stdout.flush()
    try:
        with open(PROGRESS_LOG, "a") as f:
            f.write(line + "\n")
    except OSError:
        pass


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    den = float(np.abs(ref).max())
    return float(np.abs(got.astype(np.float64) - ref).max()) / (den if den > 0 else 1.0)


def run_gpu(layer, x: np.ndarray, mode=None, routing=None, prev=None, residual: np.ndarray = None):
    """One forward through the C ABI; returns host copies of everything."""
    import torch

    from moe_amd import _lib as L

    dev = torch.device("cuda:0")
    if mode is not None:
        layer.set_mode(mode)
    if routing is not None:
        layer.set_routing(routing)
    t, H = x.shape
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    out = torch.full((t, H), float("nan"), dtype=torch.float32, device=dev)
    res = torch.from_numpy(np.ascontiguousarray(residual)).to(dev) if residual is not None else None
    k = layer.k
    routes = torch.empty((t, k, 2), dtype=torch.int32, device=dev)
    E = layer.spec.n_experts
    hits = torch.full((E + 1,), -1, dtype=torch.int32, device=dev)
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    pv = torch.from_numpy(prev.astype(np.int32)).to(dev) if prev is not None else None
    import ctypes as C

    rc = L.lib().moe_layer_forward(layer.handle, C.c_void_p(xd.data_ptr()), t, C.c_void_p(out.data_ptr()),
                                   C.c_void_p(res.data_ptr() if res is not None else None),
                                   C.c_void_p(routes.data_ptr()), C.c_void_p(hits.data_ptr()),
                                   C.c_void_p(pv.data_ptr() if pv is not None else None),
                                   C.c_void_p(stats.data_ptr()),
                                   C.c_void_p(torch.cuda.current_stream().cuda_stream))
    L.check(rc, "moe_layer_forward")
    torch.cuda.synchronize()
    r = routes.cpu().numpy()
    return dict(out=out.cpu().numpy(), sel=r[..., 0].copy(), w=r[..., 1].view(np.float32).copy(),
                hits=hits.cpu().numpy().view(np.uint32), stats=stats.cpu().numpy().view(np.uint64),
                residual=res.cpu().numpy() if res is not None else None)


def assert_routing_equal(g: dict, sel: np.ndarray, w: np.ndarray, what: str) -> None:
    """Selected experts (and their order) and weights bit-exact."""
    if not np.array_equal(g["sel"], sel):
        bad = np.argwhere(g["sel"] != sel)
        t = bad[0][0]
        raise AssertionError(f"{what}: expert selection differs at {len(bad)} slots; token {t}: "
                             f"gpu {g['sel'][t].tolist()} ref {sel[t].tolist()}")
    if not np.array_equal(g["w"].view(np.uint32), w.view(np.uint32)):
        bad = np.argwhere(g["w"].view(np.uint32) != w.view(np.uint32))
        t = bad[0][0]
        raise AssertionError(f"{what}: routing weights differ in {len(bad)} slots; token {t}: "
                             f"gpu {g['w'][t].tolist()} ref {w[t].tolist()}")
