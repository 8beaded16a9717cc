"""ctypes wrapper of the CPU oracle (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (moe_amd/).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmoe_oracle.so"

DT_F32, DT_F16, DT_Q4_0, DT_Q5_0, DT_Q8_0, DT_BF16 = 0, 1, 2, 6, 8, 30


class QT(C.Structure):
    _fields_ = [("dt", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32), ("_pad", C.c_int32),
                ("data", C.c_void_p)]


class Layer(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32), ("sigmoid", C.c_int32),
                ("norm_topk", C.c_int32), ("n_group", C.c_int32), ("topk_group", C.c_int32),
                ("routed_scale", C.c_float), ("router", QT), ("e_bias", C.c_void_p),
                ("experts", C.POINTER(QT)), ("shared", C.POINTER(QT)), ("shared_gate", C.POINTER(QT))]


class Routing(C.Structure):
    _fields_ = [("disabled", C.POINTER(C.c_int32)), ("n_disabled", C.c_int32),
                ("forced", C.POINTER(C.c_int32)), ("n_forced", C.c_int32),
                ("temp", C.c_float), ("top_k", C.c_int32)]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = C.CDLL(str(LIB_PATH))
        vp, sz = C.c_void_p, C.c_size_t
        sigs = {
            "orc_row_bytes": (sz, [C.c_int, sz]),
            "orc_quantize_rows": (None, [C.c_int, vp, sz, sz, vp]),
            "orc_dequant_rows": (None, [C.c_int, vp, sz, sz, vp]),
            "orc_f16_to_f32": (None, [vp, vp, sz]),
            "orc_f32_to_f16": (None, [vp, vp, sz]),
            "orc_dot": (C.c_float, [vp, vp, sz]),
            "orc_dot_scalar": (C.c_float, [vp, vp, sz]),
            "orc_matmul": (None, [C.POINTER(QT), vp, sz, vp]),
            "orc_route": (C.c_int, [C.POINTER(Layer), C.POINTER(Routing), vp, C.c_int, vp, vp, vp]),
            "orc_moe_forward": (C.c_int, [C.POINTER(Layer), C.POINTER(Routing), vp, C.c_int, vp, vp, vp, vp, vp,
                                          vp]),
            "orc_mlp_forward": (None, [C.POINTER(QT), C.POINTER(QT), C.POINTER(QT), vp, C.c_int, vp]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_expf_array": (None, [vp, vp, sz]),
            "orc_set_threads": (None, [C.c_int]),
            "orc_max_threads": (C.c_int, []),
        }
        for name, (res, args) in sigs.items():
            f = getattr(h, name)
            f.restype, f.argtypes = res, args
        _lib = h
    return _lib


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def row_bytes(dt: int, cols: int) -> int:
    return int(lib().orc_row_bytes(dt, cols))


def quantize(dt: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty(rows * row_bytes(dt, cols), dtype=np.uint8)
    lib().orc_quantize_rows(dt, _p(x), rows, cols, _p(out))
    return out


def dequant(dt: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    lib().orc_dequant_rows(dt, _p(data), rows, cols, _p(out))
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32(_p(h), _p(out), h.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16(_p(x), _p(out), x.size)
    return out


def dot(a: np.ndarray, b: np.ndarray, scalar: bool = False) -> np.float32:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    f = lib().orc_dot_scalar if scalar else lib().orc_dot
    return np.float32(f(_p(a), _p(b), a.size))


def qt(dt: int, rows: int, cols: int, data: np.ndarray) -> QT:
    return QT(dt=dt, rows=rows, cols=cols, data=data.ctypes.data)


def matmul(w: QT, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = x.shape[0]
    out = np.empty((t, w.rows), dtype=np.float32)
    lib().orc_matmul(C.byref(w), _p(x), t, _p(out))
    return out


def mlp_forward(gate: QT, up: QT, down: QT, x: np.ndarray) -> np.ndarray:
    """Mlp::forward (src/model.rs:26-35): down(silu(gate x) * up x)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = x.shape[0]
    out = np.empty((t, down.rows), dtype=np.float32)
    lib().orc_mlp_forward(C.byref(gate), C.byref(up), C.byref(down), _p(x), t, _p(out))
    return out


def expf(x: float) -> np.float32:
    return np.float32(lib().orc_expf(float(x)))


def expf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_expf_array(_p(x), _p(y), x.size)
    return y


class OracleLayer:
    """An orc_layer over host buffers; keeps every buffer it points at alive."""

    def __init__(self, hidden: int, n_experts: int, top_k: int, router: np.ndarray, experts: list,
                 sigmoid: bool = False, norm_topk: bool = True, routed_scale: float = 1.0, n_group: int = 1,
                 topk_group: int = 1, e_bias: Optional[np.ndarray] = None, shared: Optional[list] = None,
                 shared_gate: Optional[np.ndarray] = None):
        """router: f32 [E, H]; experts: E tuples of 3 (dt, rows, cols, bytes)."""
        self._keep = [np.ascontiguousarray(router, dtype=np.float32)]
        self.router = self._keep[0]
        self.experts_c = (QT * (3 * n_experts))()
        for e, mats in enumerate(experts):
            for m, (dt, rows, cols, data) in enumerate(mats):
                data = np.ascontiguousarray(data, dtype=np.uint8)
                self._keep.append(data)
                self.experts_c[3 * e + m] = qt(dt, rows, cols, data)
        self.shared_c = None
        if shared is not None:
            self.shared_c = (QT * 3)()
            for m, (dt, rows, cols, data) in enumerate(shared):
                data = np.ascontiguousarray(data, dtype=np.uint8)
                self._keep.append(data)
                self.shared_c[m] = qt(dt, rows, cols, data)
        self.sg_c = None
        if shared_gate is not None:
            sg = np.ascontiguousarray(shared_gate, dtype=np.float32).reshape(1, hidden)
            self._keep.append(sg)
            self.sg_c = qt(DT_F32, 1, hidden, sg.view(np.uint8).reshape(-1))
        eb = None
        if e_bias is not None:
            eb = np.ascontiguousarray(e_bias, dtype=np.float32).reshape(-1)
            self._keep.append(eb)
        self.c = Layer(hidden=hidden, n_experts=n_experts, top_k=top_k, sigmoid=int(sigmoid),
                       norm_topk=int(norm_topk), n_group=n_group, topk_group=topk_group,
                       routed_scale=routed_scale,
                       router=qt(DT_F32, n_experts, hidden, self.router.view(np.uint8).reshape(-1)),
                       e_bias=eb.ctypes.data if eb is not None else None,
                       experts=C.cast(self.experts_c, C.POINTER(QT)),
                       shared=C.cast(self.shared_c, C.POINTER(QT)) if self.shared_c is not None else None,
                       shared_gate=C.pointer(self.sg_c) if self.sg_c is not None else None)
        self.hidden, self.n_experts, self.top_k = hidden, n_experts, top_k

    @staticmethod
    def routing(disabled=(), forced=(), temp: float = 0.0, top_k: int = 0):
        da = (C.c_int32 * max(1, len(disabled)))(*disabled)
        fa = (C.c_int32 * max(1, len(forced)))(*forced)
        r = Routing(disabled=C.cast(da, C.POINTER(C.c_int32)), n_disabled=len(disabled),
                    forced=C.cast(fa, C.POINTER(C.c_int32)), n_forced=len(forced), temp=temp, top_k=top_k)
        r._keep = (da, fa)
        return r

    def k(self, routing: Optional[Routing] = None) -> int:
        top = routing.top_k if routing is not None and routing.top_k > 0 else self.top_k
        return min(top, self.n_experts)

    def route(self, x: np.ndarray, routing: Optional[Routing] = None):
        """(experts [t,k] int32, weights [t,k] f32, logits [t,E] f32, ties)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        t, k = x.shape[0], self.k(routing)
        sel = np.empty((t, k), dtype=np.int32)
        w = np.empty((t, k), dtype=np.float32)
        logits = np.empty((t, self.n_experts), dtype=np.float32)
        ties = lib().orc_route(C.byref(self.c), C.byref(routing) if routing is not None else None, _p(x), t,
                               _p(sel), _p(w), _p(logits))
        return sel, w, logits, ties

    def forward(self, x: np.ndarray, routing: Optional[Routing] = None, prev: Optional[np.ndarray] = None):
        """(out [t,H], experts [t,k], weights [t,k], hits [E+1] u32, stats [4] u64)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        t, k = x.shape[0], self.k(routing)
        out = np.empty((t, self.hidden), dtype=np.float32)
        sel = np.empty((t, k), dtype=np.int32)
        w = np.empty((t, k), dtype=np.float32)
        hits = np.zeros(self.n_experts + 1, dtype=np.uint32)
        stats = np.zeros(4, dtype=np.uint64)
        pv = np.ascontiguousarray(prev, dtype=np.uint32) if prev is not None else None
        rc = lib().orc_moe_forward(C.byref(self.c), C.byref(routing) if routing is not None else None, _p(x), t,
                                   _p(out), _p(sel), _p(w), _p(hits), _p(pv) if pv is not None else None,
                                   _p(stats))
        if rc < 0:
            raise RuntimeError(f"orc_moe_forward failed ({rc})")
        return out, sel, w, hits, stats


def from_host_layer(host) -> OracleLayer:
    """The oracle over a moe_amd.synth.HostLayer's bytes (the same bytes the
    GPU reads)."""
    s = host.shape
    E, H, I = s.n_experts, s.hidden, s.inter
    router = host.tensor("router").view(np.float32).reshape(E, H)
    experts = []
    g, u, d = host.tensor("experts.gate"), host.tensor("experts.up"), host.tensor("experts.down")
    rg, rd = row_bytes(s.expert_dt, H) * I, row_bytes(s.expert_dt, I) * H
    for e in range(E):
        experts.append([(s.expert_dt, I, H, g[e * rg:(e + 1) * rg]), (s.expert_dt, I, H, u[e * rg:(e + 1) * rg]),
                        (s.expert_dt, H, I, d[e * rd:(e + 1) * rd])])
    shared = None
    if s.shared_inter:
        sdt = s.shared_dt if s.shared_dt is not None else s.expert_dt
        Is = s.shared_inter
        shared = [(sdt, Is, H, host.tensor("shared.gate")), (sdt, Is, H, host.tensor("shared.up")),
                  (sdt, H, Is, host.tensor("shared.down"))]
    e_bias = host.tensor("e_bias").view(np.float32) if "e_bias" in host.index else None
    sg = host.tensor("shared_gate").view(np.float32) if "shared_gate" in host.index else None
    return OracleLayer(H, E, s.top_k, router, experts, sigmoid=s.sigmoid, norm_topk=s.norm_topk,
                       routed_scale=s.routed_scale, n_group=s.n_group, topk_group=s.topk_group, e_bias=e_bias,
                       shared=shared, shared_gate=sg)
