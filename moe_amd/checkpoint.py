"""Single-file checkpoints: the packed ``.moe`` container and GGUF.

The library parses both (``moe_container_open``: src/store.rs:228-279 for
``.moe``, src/gguf.rs:206-276 for GGUF) from a memory map that stays owned
here; the tensors a layer needs are then copied to one device region with
every tensor on a 256-byte boundary (``moe_upload_tensors``), and a
``Store`` over that region addresses experts as row ranges exactly as
``Store::view`` addresses the file (src/store.rs:303-315).

``bind_layer`` finds a routed layer's tensors under the names the reference
looks for (src/model.rs:396-441): a fused ``gate_up_proj`` stack, one 3-D
stack per projection (what GGUF writes), or one tensor per expert (including
Mixtral's ``block_sparse_moe.experts.{e}.{w1,w3,w2}``).  ``write_moe`` writes
the reference's packed format, for tests and for packing synthetic layers.
"""
from __future__ import annotations

import ctypes as C
import json
import mmap
import os
import struct
from typing import Iterable, Optional

import numpy as np

from . import _lib as L
from .layer import MoeLayer, MoeSpec, Rec, Region, Store, row_bytes

KIND_MOE, KIND_GGUF = 1, 2

# quant::Dt::name (src/quant.rs:53-65) for the formats a .moe can hold here.
DT_TO_MOE_NAME = {L.DT_F32: "F32", L.DT_F16: "F16", L.DT_BF16: "BF16", L.DT_Q8_0: "Q8", L.DT_Q4_0: "Q4",
                  L.DT_Q5_0: "Q5"}


class Container:
    """A parsed checkpoint file, memory-mapped for as long as this lives."""

    def __init__(self, path: str):
        self.path = path
        self._file = open(path, "rb")
        size = os.fstat(self._file.fileno()).st_size
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ) if size else None
        self.buf = np.frombuffer(self._map, dtype=np.uint8) if self._map is not None else np.zeros(0, np.uint8)
        h = C.c_void_p()
        L.check(L.lib().moe_container_open(self.buf.ctypes.data_as(C.c_void_p) if size else None, size,
                                           C.byref(h)), f"open {path}")
        self._h = h
        self.kind = int(L.lib().moe_container_kind(h))
        self.recs: dict[str, dict] = {}
        r = L.RecC()
        for i in range(int(L.lib().moe_container_count(h))):
            L.check(L.lib().moe_container_rec(h, i, C.byref(r)), "moe_container_rec")
            self.recs[r.name.decode(errors="surrogateescape")] = dict(dt=r.dt, slabs=r.slabs, rows=r.rows, cols=r.cols, offset=r.offset,
                                              bytes=r.bytes)

    def config(self) -> Optional[dict]:
        """The .moe header's model config (Store::config), if any."""
        s = L.lib().moe_container_config(self._h)
        return None if s is None else json.loads(s.decode())

    def hf_names(self) -> dict[str, str]:
        """Hugging Face name -> file name: identity for a .moe, gguf::rename
        for GGUF (tensors without a counterpart are left out)."""
        if self.kind != KIND_GGUF:
            return {n: n for n in self.recs}
        return {hf: n for n in self.recs if (hf := gguf_rename(n)) is not None}

    def bytes_of(self, name: str) -> np.ndarray:
        r = self.recs[name]
        return self.buf[r["offset"]:r["offset"] + r["bytes"]]

    def close(self) -> None:
        if self._h:
            L.lib().moe_container_close(self._h)
            self._h = None
        self.buf = None
        if self._map is not None:
            self._map.close()
            self._map = None
        self._file.close()

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


def gguf_rename(name: str) -> Optional[str]:
    """gguf::rename (src/gguf.rs:435-487): the Hugging Face name, or None."""
    out = C.create_string_buffer(512)
    rc = L.lib().moe_gguf_rename(name.encode(), out, len(out))
    if rc == 1:
        return None
    L.check(rc, "moe_gguf_rename")
    return out.value.decode()


def upload(ctx, container: Container, names: Iterable[str]) -> Store:
    """Copy the named tensors (Hugging Face names) to one device region, each
    256-byte aligned, and return a Store over it keyed by those names."""
    hf = container.hf_names()
    names = list(names)
    recs = [container.recs[hf[n]] for n in names]
    for n, r in zip(names, recs):
        if r["bytes"] == 0:
            raise L.MoeError(L.MOE_EUNSUP, f"{n}: format {r['dt']} cannot be read by these kernels")
    offs = (C.c_uint64 * len(recs))(*[r["offset"] for r in recs])
    lens = (C.c_uint64 * len(recs))(*[r["bytes"] for r in recs])
    dev = (C.c_uint64 * len(recs))()
    rid = C.c_uint64()
    L.check(L.lib().moe_upload_tensors(ctx.handle, container.buf.ctypes.data_as(C.c_void_p), container.buf.nbytes,
                                       offs, lens, len(recs), dev, C.byref(rid)), "moe_upload_tensors")
    total = max((dev[i] + recs[i]["bytes"] for i in range(len(recs))), default=0)
    region = Region(ctx, rid.value, total)
    index = {n: Rec(r["dt"], r["slabs"], r["rows"], r["cols"], dev[i]) for i, (n, r) in enumerate(zip(names, recs))}
    return Store(region, index)


def layer_tensor_names(container: Container, layer: int, n_experts: int) -> list[str]:
    """The Hugging Face names of one routed layer's tensors present in the
    file (router, bias, experts in any of the three layouts, shared expert
    and its gate)."""
    hf = container.hf_names()
    p = f"model.layers.{layer}."
    want = [p + "mlp.gate.weight", p + "block_sparse_moe.gate.weight", p + "mlp.gate.e_score_correction_bias",
            p + "mlp.experts.gate_up_proj", p + "mlp.experts.gate_proj", p + "mlp.experts.up_proj",
            p + "mlp.experts.down_proj", p + "mlp.shared_expert_gate.weight"]
    for n in ("gate_proj", "up_proj", "down_proj"):
        want += [p + f"mlp.shared_expert.{n}.weight", p + f"mlp.shared_experts.{n}.weight"]
        want += [p + f"mlp.experts.{e}.{n}.weight" for e in range(n_experts)]
    for w in ("w1", "w3", "w2"):
        want += [p + f"block_sparse_moe.experts.{e}.{w}.weight" for e in range(n_experts)]
    return [n for n in want if n in hf]


def bind_layer(ctx, store: Store, layer: int, spec: MoeSpec, layer_index: int = 0) -> MoeLayer:
    """A MoeLayer over a routed layer's tensors, found as src/model.rs:396-441
    finds them; every expert is a row range of its tensor."""
    p = f"model.layers.{layer}."
    E = spec.n_experts

    def g(name):
        return store.get(p + name)

    fused = store.shape(p + "mlp.experts.gate_up_proj")
    names = ("gate_proj", "up_proj", "down_proj")
    stacked = all((sh := store.shape(p + f"mlp.experts.{n}")) is not None and sh[0] >= 2 for n in names)

    def expert(e, which):
        if fused is not None:
            inter = fused[1] // 2
            if which == 0:
                return store.view(p + "mlp.experts.gate_up_proj", e, 0, inter)
            if which == 1:
                return store.view(p + "mlp.experts.gate_up_proj", e, inter, 2 * inter)
            sh = store.shape(p + "mlp.experts.down_proj")
            return None if sh is None else store.view(p + "mlp.experts.down_proj", e, 0, sh[1])
        if stacked:
            n = p + f"mlp.experts.{names[which]}"
            return store.view(n, e, 0, store.shape(n)[1])
        return g(f"mlp.experts.{e}.{names[which]}.weight") or g(
            f"block_sparse_moe.experts.{e}.{('w1', 'w3', 'w2')[which]}.weight")

    experts = []
    for e in range(E):
        trio = [expert(e, w) for w in range(3)]
        if any(v is None for v in trio):
            raise L.MoeError(L.MOE_EINVAL, f"layer {layer}: expert {e} is incomplete")
        experts.append(tuple(trio))
    router = g("mlp.gate.weight") or g("block_sparse_moe.gate.weight")
    if router is None:
        raise L.MoeError(L.MOE_EINVAL, f"layer {layer}: no router")

    def shared(which):
        n = names[which]
        return g(f"mlp.shared_expert.{n}.weight") or g(f"mlp.shared_experts.{n}.weight")

    sh = None if shared(0) is None else (shared(0), shared(1), shared(2))
    layer_obj = MoeLayer(ctx, spec, router, experts, e_bias=g("mlp.gate.e_score_correction_bias"), shared=sh,
                         shared_gate=g("mlp.shared_expert_gate.weight"), layer_index=layer_index)
    layer_obj._region = store.region
    return layer_obj


def write_moe(path: str, tensors: list, config: Optional[dict] = None) -> None:
    """Write a packed .moe file (src/store.rs:473-481): "MOEF", u32 version 1,
    u64 header length, the JSON header, then each tensor's rows back to back
    in name order.  `tensors` holds (name, dt, shape, raw bytes) with shape
    [rows, cols] or [slabs, rows, cols]."""
    entries, off = {}, 0
    items = sorted(tensors, key=lambda t: t[0])
    for name, dt, shape, raw in items:
        rows = int(np.prod(shape[:-1]))
        n = rows * row_bytes(dt, shape[-1])
        if len(raw) != n:
            raise ValueError(f"{name}: {len(raw)} bytes for shape {shape} in format {dt}")
        entries[name] = {"dt": DT_TO_MOE_NAME[dt], "shape": [int(d) for d in shape], "off": off, "len": n}
        off += n
    header = json.dumps({"config": config or {}, "tokenizer": None, "chat_template": None, "tensors": entries},
                        separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(b"MOEF")
        f.write(struct.pack("<IQ", 1, len(header)))
        f.write(header)
        for _, _, _, raw in items:
            f.write(bytes(raw))


def host_layer_tensors(host, layer: int = 0) -> list:
    """A synthetic layer's tensors under Hugging Face names, experts as
    per-projection 3-D stacks (the layout GGUF and DeepSeek checkpoints use)."""
    s = host.shape
    p = f"model.layers.{layer}."
    names = {"router": "mlp.gate.weight", "e_bias": "mlp.gate.e_score_correction_bias",
             "experts.gate": "mlp.experts.gate_proj", "experts.up": "mlp.experts.up_proj",
             "experts.down": "mlp.experts.down_proj", "shared.gate": "mlp.shared_experts.gate_proj.weight",
             "shared.up": "mlp.shared_experts.up_proj.weight", "shared.down": "mlp.shared_experts.down_proj.weight",
             "shared_gate": "mlp.shared_expert_gate.weight"}
    out = []
    for key, rec in host.index.items():
        shape = [rec.slabs, rec.rows, rec.cols] if rec.slabs > 1 else [rec.rows, rec.cols]
        out.append((p + names[key], rec.dt, shape, host.tensor(key).tobytes()))
    return out
