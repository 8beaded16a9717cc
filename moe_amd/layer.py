"""Host mirror of the reference's routed-layer interface, over libmoe_hip.

The reference's boundary is ``Model::feed_forward`` (src/model.rs:836-971)
with its ``Ffn::Moe`` weights (src/model.rs:68-71), router interventions
``Routing`` (src/model.rs:238-280), per-sequence ``State`` (prev selections,
``Stats`` counters and an optional ``Trace`` of ``Route`` records,
src/model.rs:84-137).  The classes here keep those names, argument meanings
and side effects; the arithmetic all happens in the HIP library on the GPU.
Torch is used only as the owner of device memory and streams.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib as L

try:
    import torch
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None


def _stream_ptr(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


# --------------------------------------------------------------- regions


class Region:
    """An uploaded byte range (the device copy of an mmap'd checkpoint range)."""

    def __init__(self, ctx: "Context", rid: int, nbytes: int):
        self.ctx, self.id, self.nbytes = ctx, rid, nbytes

    def device_ptr(self) -> int:
        p = C.c_void_p()
        L.check(L.lib().moe_region_ptr(self.ctx.handle, self.id, C.byref(p)), "moe_region_ptr")
        return p.value


class Context:
    """One device's library context (moe_ctx)."""

    def __init__(self, device: int = 0):
        self.device = device
        h = C.c_void_p()
        L.check(L.lib().moe_ctx_create(device, C.byref(h)), "moe_ctx_create")
        self.handle = h

    def upload(self, data) -> Region:
        """Copy host bytes (bytes, bytearray or a contiguous numpy array) to a
        new 256-byte-aligned device region; offsets inside are preserved."""
        arr = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                                   else data).view(np.uint8).reshape(-1)
        rid = C.c_uint64()
        L.check(L.lib().moe_upload(self.handle, arr.ctypes.data_as(C.c_void_p), arr.nbytes, C.byref(rid)),
                "moe_upload")
        return Region(self, rid.value, arr.nbytes)

    def close(self) -> None:
        if self.handle:
            L.lib().moe_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------- tensor views


def row_bytes(dt: int, cols: int) -> int:
    """Dt::row_bytes (src/quant.rs:68-83)."""
    return int(L.lib().moe_row_bytes(dt, cols))


@dataclass(frozen=True)
class View:
    """A QT (src/quant.rs:97-129): dt, rows x cols, at a byte offset of a region."""

    dt: int
    rows: int
    cols: int
    region: int
    offset: int

    def c(self) -> L.Tensor:
        return L.Tensor(dt=self.dt, rows=self.rows, cols=self.cols, region=self.region, offset=self.offset)

    @property
    def nbytes(self) -> int:
        return self.rows * row_bytes(self.dt, self.cols)


@dataclass(frozen=True)
class Rec:
    """A named tensor in a region (Rec, src/store.rs:25-47): `slabs` leading
    expert dimension (1 for a plain matrix), then rows x cols."""

    dt: int
    slabs: int
    rows: int
    cols: int
    offset: int

    @property
    def nbytes(self) -> int:
        return self.slabs * self.rows * row_bytes(self.dt, self.cols)


class Store:
    """Named tensors in one region, addressed like Store::get/view
    (src/store.rs:291-315): an expert is a row range inside a slab."""

    def __init__(self, region: Region, index: dict[str, Rec]):
        self.region, self.index = region, index

    def shape(self, name: str):
        r = self.index.get(name)
        return None if r is None else (r.slabs, r.rows, r.cols)

    def view(self, name: str, slab: int, r0: int, r1: int) -> Optional[View]:
        r = self.index.get(name)
        if r is None or r1 > r.slabs * r.rows or r0 >= r1:
            return None
        stride = row_bytes(r.dt, r.cols)
        off = r.offset + (slab * r.rows + r0) * stride
        if off + (r1 - r0) * stride > r.offset + r.nbytes:
            return None
        return View(r.dt, r1 - r0, r.cols, self.region.id, off)

    def get(self, name: str) -> Optional[View]:
        r = self.index.get(name)
        return None if r is None else self.view(name, 0, 0, r.slabs * r.rows)


# ----------------------------------------------------- routing and state


@dataclass
class Routing:
    """Router interventions (model::Routing, src/model.rs:238-280)."""

    disabled: list = field(default_factory=list)   # (layer, expert)
    forced: list = field(default_factory=list)     # (layer, expert)
    temp: float = 0.0
    top_k: int = 0

    def is_empty(self) -> bool:
        return not self.disabled and not self.forced and self.temp <= 0.0 and self.top_k == 0

    @staticmethod
    def at(pairs, layer: int) -> list[int]:
        return [e for (l, e) in pairs if l == layer]


@dataclass
class Route:
    """One token's routing at one layer (src/model.rs:84-91)."""

    pos: int
    layer: int
    experts: list  # (expert, weight), strongest first


@dataclass
class Stats:
    """Host snapshot of the Stats counters (src/model.rs:116-137) plus the
    count of tokens whose selection met an exact rank tie."""

    routed: int = 0
    reused: int = 0
    expert_bytes: int = 0
    ties: int = 0

    def reuse_rate(self) -> float:
        return 0.0 if self.routed == 0 else self.reused / self.routed


class State:
    """Per-sequence state for routed layers: position, the previous token's
    selection per layer, counters and an optional trace (src/model.rs:93-189,
    MoE-relevant parts)."""

    def __init__(self, n_layers: int, device: int = 0, trace: bool = False):
        self.pos = 0
        self.device = device
        self.prev: list = [None] * n_layers          # device u32 [E+1] per layer
        self.stats_dev = torch.zeros(4, dtype=torch.int64, device=f"cuda:{device}")
        self.trace: Optional[list] = [] if trace else None

    def stats(self) -> Stats:
        v = self.stats_dev.cpu().tolist()
        return Stats(*[int(x) for x in v])

    def previous(self, layer: int) -> list[int]:
        p = self.prev[layer]
        if p is None:
            return []
        h = p.cpu().numpy().view(np.uint32)
        return h[1:1 + h[0]].tolist()

    def truncate(self, n: int) -> None:
        """Rewind to position n (State::truncate, src/model.rs:176-189)."""
        self.pos = min(n, self.pos)
        self.prev = [None] * len(self.prev)
        if self.trace is not None:
            self.trace = [r for r in self.trace if r.pos < self.pos]


# ---------------------------------------------------------------- layer


@dataclass
class MoeSpec:
    """The Spec fields a routed layer reads (src/spec.rs:199-207)."""

    hidden: int
    n_experts: int
    top_k: int = 2
    sigmoid: bool = False
    norm_topk: bool = True
    routed_scale: float = 1.0
    n_group: int = 1
    topk_group: int = 1


class Mlp:
    """A dense SwiGLU MLP, Mlp::forward (src/model.rs:20-40), as Ffn::Dense
    runs it (src/model.rs:840), on the expert kernels.

    It is a routed layer with one expert and a router row of zeros: the
    softmax over one logit gives the expert weight exp(0) / exp(0) = 1, the
    renormalisation divides by 1, and the combine writes 0 + 1 * y = y, so
    the output is the expert's output unchanged; the routing stages add a
    few microseconds per call."""

    def __init__(self, ctx: "Context", gate: View, up: View, down: View):
        if not (gate.rows == up.rows == down.cols and gate.cols == up.cols == down.rows):
            raise ValueError(f"gate {gate.rows}x{gate.cols}, up {up.rows}x{up.cols}, down {down.rows}x{down.cols}"
                             " do not form an MLP")
        self.hidden, self.inter = gate.cols, gate.rows
        self._router_region = ctx.upload(np.zeros(self.hidden, dtype=np.float32))
        router = View(L.DT_F32, 1, self.hidden, self._router_region.id, 0)
        self.layer = MoeLayer(ctx, MoeSpec(hidden=self.hidden, n_experts=1, top_k=1), router, [(gate, up, down)])

    def set_mode(self, mode: int) -> None:
        self.layer.set_mode(mode)

    def reserve(self, max_t: int) -> None:
        self.layer.reserve(max_t)

    def forward(self, x, out, residual=None, stream=None) -> None:
        """out = down(silu(gate x) * up x) for x [t, hidden] f32 (CUDA);
        residual += out when given."""
        self.layer.feed_forward(x, out, residual=residual, stream=stream)

    def close(self) -> None:
        self.layer.close()


class MoeLayer:
    """Ffn::Moe on the GPU (src/model.rs:68-71, 841-971)."""

    def __init__(self, ctx: Context, spec: MoeSpec, router: View, experts: Sequence, e_bias: Optional[View] = None,
                 shared: Optional[Sequence[View]] = None, shared_gate: Optional[View] = None, layer_index: int = 0):
        self.ctx, self.spec, self.li = ctx, spec, layer_index
        arr = (L.Tensor * (3 * spec.n_experts))()
        if len(experts) != spec.n_experts:
            raise ValueError(f"{len(experts)} experts given, spec says {spec.n_experts}")
        for e, (g, u, d) in enumerate(experts):
            arr[3 * e], arr[3 * e + 1], arr[3 * e + 2] = g.c(), u.c(), d.c()
        self._experts_c = arr
        desc = L.LayerDesc(hidden=spec.hidden, n_experts=spec.n_experts, top_k=spec.top_k,
                           gate=L.GATE_SIGMOID if spec.sigmoid else L.GATE_SOFTMAX,
                           norm_topk=1 if spec.norm_topk else 0, n_group=spec.n_group,
                           topk_group=spec.topk_group, routed_scale=spec.routed_scale,
                           router=router.c(), e_bias=e_bias.c() if e_bias else L.absent(),
                           experts=C.cast(arr, C.POINTER(L.Tensor)))
        for i in range(3):
            desc.shared[i] = shared[i].c() if shared else L.absent()
        desc.shared_gate = shared_gate.c() if shared_gate else L.absent()
        h = C.c_void_p()
        L.check(L.lib().moe_layer_create(ctx.handle, C.byref(desc), C.byref(h)), "moe_layer_create")
        self.handle = h
        self.expert_views = list(experts)
        self.routing = Routing()

    # -- configuration ---------------------------------------------------
    def set_routing(self, routing: Optional[Routing]) -> None:
        """Apply this layer's share of a Routing (src/model.rs:846-888)."""
        self.routing = routing or Routing()
        r = self.routing
        dis = Routing.at(r.disabled, self.li)
        frc = Routing.at(r.forced, self.li)
        da = (C.c_int32 * max(1, len(dis)))(*dis)
        fa = (C.c_int32 * max(1, len(frc)))(*frc)
        rc = L.RoutingC(disabled=C.cast(da, C.POINTER(C.c_int32)), n_disabled=len(dis),
                        forced=C.cast(fa, C.POINTER(C.c_int32)), n_forced=len(frc),
                        temp=float(r.temp), top_k=int(r.top_k))
        L.check(L.lib().moe_layer_set_routing(self.handle, C.byref(rc)), "moe_layer_set_routing")

    def set_mode(self, mode: int) -> None:
        L.check(L.lib().moe_layer_set_mode(self.handle, mode), "moe_layer_set_mode")

    def set_tiled(self, enable: bool = True) -> None:
        """Keep (or drop) the tiled copy of the expert matrices that calls of
        few tokens per expert stream at about twice the row-major rate."""
        L.check(L.lib().moe_layer_set_tiled(self.handle, 1 if enable else 0), "moe_layer_set_tiled")

    def reserve(self, max_t: int, stream=None) -> None:
        """Allocate the workspace for `stream` up front (no later call on it
        allocates; calls beyond max_t tokens fail)."""
        L.check(L.lib().moe_layer_reserve_stream(self.handle, max_t, C.c_void_p(_stream_ptr(stream))),
                "moe_layer_reserve_stream")

    def release_stream(self, stream=None) -> None:
        """Drop the workspace kept for `stream` (freed once its queued work
        has finished); call before destroying a stream whose handle may be
        reused."""
        L.check(L.lib().moe_layer_release_stream(self.handle, C.c_void_p(_stream_ptr(stream))),
                "moe_layer_release_stream")

    def workspace_size(self, max_t: int) -> int:
        """Bytes of a caller-owned workspace for up to max_t tokens."""
        n = C.c_uint64()
        L.check(L.lib().moe_layer_workspace_size(self.handle, max_t, C.byref(n)), "moe_layer_workspace_size")
        return int(n.value)

    @staticmethod
    def new_workspace(nbytes: int, device="cuda"):
        """A zero-filled, 256-byte-aligned device buffer of at least nbytes
        for feed_forward(workspace=...)."""
        buf = torch.zeros(nbytes + 256, dtype=torch.uint8, device=device)
        off = (-buf.data_ptr()) % 256
        return buf[off:off + nbytes]

    @property
    def k(self) -> int:
        return int(L.lib().moe_layer_k(self.handle))

    # -- the forward -------------------------------------------------------
    def feed_forward(self, x, out, state: Optional[State] = None, residual=None, routes=None, stream=None,
                     workspace=None):
        """out = the routed layer over x ([t, H] f32 CUDA tensors); residual
        += out when given.  With a State: its prev selection drives the reuse
        counter and is replaced by this call's, its stats accumulate, and
        with tracing on the routes are appended (src/model.rs:943-954).
        With `workspace` (a device buffer from new_workspace) the call runs
        on it and allocates nothing (moe_layer_forward_ws)."""
        t = int(x.shape[0])
        self._check_io(x, out, residual)
        k = self.k
        want_routes = routes is not None or (state is not None and state.trace is not None)
        if want_routes and routes is None:
            routes = torch.empty((t, k, 2), dtype=torch.int32, device=x.device)
        hits = prev = stats = None
        if state is not None:
            hits = torch.empty(self.spec.n_experts + 1, dtype=torch.int32, device=x.device)
            prev = state.prev[self.li]
            stats = state.stats_dev
        args = (self.handle, C.c_void_p(x.data_ptr()), t, C.c_void_p(out.data_ptr()),
                C.c_void_p(residual.data_ptr() if residual is not None else None),
                C.c_void_p(routes.data_ptr() if routes is not None else None),
                C.c_void_p(hits.data_ptr() if hits is not None else None),
                C.c_void_p(prev.data_ptr() if prev is not None else None),
                C.c_void_p(stats.data_ptr() if stats is not None else None))
        if workspace is None:
            rc = L.lib().moe_layer_forward(*args, C.c_void_p(_stream_ptr(stream)))
            L.check(rc, "moe_layer_forward")
        else:
            rc = L.lib().moe_layer_forward_ws(*args, C.c_void_p(workspace.data_ptr()), workspace.numel(),
                                              C.c_void_p(_stream_ptr(stream)))
            L.check(rc, "moe_layer_forward_ws")
        if state is not None:
            state.prev[self.li] = hits
            if state.trace is not None:
                r = routes.cpu().numpy()
                for i in range(t):
                    ex = r[i, :, 0].view(np.uint32).tolist()
                    w = r[i, :, 1].view(np.float32).tolist()
                    state.trace.append(Route(state.pos + i, self.li, list(zip(ex, w))))
        return routes

    def route(self, x, logits=None, stream=None):
        """Routing only: (experts [t,k] int, weights [t,k] f32) tensors."""
        t = int(x.shape[0])
        routes = torch.empty((t, self.k, 2), dtype=torch.int32, device=x.device)
        rc = L.lib().moe_layer_route(self.handle, C.c_void_p(x.data_ptr()), t, C.c_void_p(routes.data_ptr()),
                                     C.c_void_p(logits.data_ptr() if logits is not None else None),
                                     C.c_void_p(_stream_ptr(stream)))
        L.check(rc, "moe_layer_route")
        return routes[..., 0], routes[..., 1].view(torch.float32)

    def _check_io(self, x, out, residual):
        H = self.spec.hidden
        for name, tsr in (("x", x), ("out", out), ("residual", residual)):
            if tsr is None:
                continue
            if not tsr.is_cuda or tsr.dtype != torch.float32 or not tsr.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 CUDA tensor")
            if tsr.dim() != 2 or tsr.shape[1] != H or tsr.shape[0] != x.shape[0]:
                raise ValueError(f"{name} has shape {tuple(tsr.shape)}, expected ({x.shape[0]}, {H})")
        if x.shape[0] < 1:
            raise ValueError("t must be at least 1 (src/model.rs:649)")

    def close(self) -> None:
        if getattr(self, "handle", None):
            L.lib().moe_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass
