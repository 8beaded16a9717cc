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
            "orc_rmsnorm_rows": (None, [vp, sz, sz, sz, vp, C.c_float, vp, sz]),
            "orc_rope_rows": (None, [vp, sz, sz, sz, sz, sz, sz, vp, vp, sz]),
            "orc_inv_freqs": (None, [C.c_int, C.c_float, C.c_float, sz, C.c_float, C.c_float, C.c_float, C.c_float,
                                     sz, vp]),
            "orc_attn_scale": (C.c_float, [C.c_int, C.c_float, C.c_float, C.c_float, C.c_float]),
            "orc_attention": (None, [vp, vp, vp, sz, sz, sz, sz, sz, sz, C.c_float, sz, vp]),
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


# ------------------------------------------------------- the whole model


def inv_freqs(rope, head_dim: int) -> np.ndarray:
    """Rope::inv_freqs (src/spec.rs:89-145) for a rope description with the
    reference's fields (kind 0 none, 1 linear, 2 dynamic, 3 YaRN, 4 Llama 3)."""
    out = np.zeros(head_dim // 2, dtype=np.float32)
    lib().orc_inv_freqs(rope.kind, rope.theta, rope.factor, rope.original_ctx, rope.low_freq_factor,
                        rope.high_freq_factor, rope.beta_fast, rope.beta_slow, head_dim, _p(out))
    return out


def attn_scale(rope) -> np.float32:
    return np.float32(lib().orc_attn_scale(rope.kind, rope.factor, rope.mscale, rope.mscale_all_dim,
                                           rope.attn_factor))


def rmsnorm_rows(x: np.ndarray, w: np.ndarray, eps: float, n: Optional[int] = None) -> np.ndarray:
    """rmsnorm (src/model.rs:211-216) of every row of x (the first n values
    of each row when n is given)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, width = x.shape
    n = width if n is None else n
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty((rows, n), dtype=np.float32)
    lib().orc_rmsnorm_rows(_p(x), rows, n, width, _p(w), eps, _p(out), n)
    return out


class OracleModel:
    """The reference's CPU forward of a whole decoder (src/model.rs:565-834)
    over host tensors: `spec` carries the Spec fields (moe_amd.model.Spec),
    `tensors` maps Hugging Face names to (dt, shape, uint8 bytes) records.
    One sequence per State, as the reference runs them."""

    def __init__(self, spec, tensors: dict):
        self.spec, self.tensors = spec, tensors
        s = spec
        self._keep = []
        self.inv = inv_freqs(s.rope, s.mla.qk_rope if s.mla else s.head_dim)
        self.scale_mult = attn_scale(s.rope)
        self.embed = self._qt("model.embed_tokens.weight")
        self.out_norm = self._f32("model.norm.weight")
        self.lm_head = self._qt("lm_head.weight") if "lm_head.weight" in tensors else self.embed
        self.layers = [self._layer(l) for l in range(s.layers)]

    # -- weights ---------------------------------------------------------
    def _rec(self, name):
        t = self.tensors[name]
        return t.dt, t.shape, np.ascontiguousarray(t.data).view(np.uint8).reshape(-1)

    def _qt(self, name, slab: Optional[int] = None):
        dt, shape, data = self._rec(name)
        rows, cols = (shape[-2] if len(shape) > 1 else 1), shape[-1]
        if slab is not None:
            n = row_bytes(dt, cols) * rows
            data = data[slab * n:(slab + 1) * n]
        self._keep.append(data)
        return qt(dt, rows, cols, data)

    def _qt_tuple(self, name, slab: Optional[int] = None):
        dt, shape, data = self._rec(name)
        rows, cols = (shape[-2] if len(shape) > 1 else 1), shape[-1]
        if slab is not None:
            n = row_bytes(dt, cols) * rows
            data = data[slab * n:(slab + 1) * n]
        return (dt, rows, cols, data)

    def _f32(self, name, optional=False):
        if name not in self.tensors:
            if optional:
                return None
            raise KeyError(name)
        dt, shape, data = self._rec(name)
        assert dt == DT_F32, name
        return data.view(np.float32)

    def _layer(self, l: int) -> dict:
        s, p = self.spec, f"{self.spec.prefix}{l}."
        a = p + "self_attn."
        lay = dict(ln1=self._f32(p + "input_layernorm.weight"), ln2=self._f32(p + "post_attention_layernorm.weight"),
                   o=self._qt(a + "o_proj.weight"), window=s.windows[l] if l < len(s.windows) else None)
        if s.mla is None:
            lay.update(q=self._qt(a + "q_proj.weight"), k=self._qt(a + "k_proj.weight"), v=self._qt(a + "v_proj.weight"),
                       bias=[self._f32(a + f"{m}_proj.bias", True) for m in "qkv"],
                       q_norm=self._f32(a + "q_norm.weight", True), k_norm=self._f32(a + "k_norm.weight", True))
        else:
            has_qa = (a + "q_a_proj.weight") in self.tensors
            lay.update(q_a=self._qt(a + "q_a_proj.weight") if has_qa else None,
                       q_a_norm=self._f32(a + "q_a_layernorm.weight", True),
                       q_b=self._qt(a + ("q_b_proj.weight" if has_qa else "q_proj.weight")),
                       kv_a=self._qt(a + "kv_a_proj_with_mqa.weight"), kv_a_norm=self._f32(a + "kv_a_layernorm.weight"),
                       kv_b=self._qt(a + "kv_b_proj.weight"))
        m = p + "mlp."
        router = m + "gate.weight" if (m + "gate.weight") in self.tensors else p + "block_sparse_moe.gate.weight"
        if router in self.tensors:
            lay["moe"] = self._moe(l, router)
        else:
            lay["mlp"] = tuple(self._qt(m + f"{n}_proj.weight") for n in ("gate", "up", "down"))
        return lay

    def _moe(self, l: int, router_name: str) -> "OracleLayer":
        """The routed layer's tensors in any of the reference's three expert
        layouts (src/model.rs:396-441)."""
        s, p = self.spec, f"{self.spec.prefix}{l}."
        m = p + "mlp."
        router = self._f32(router_name).reshape(s.experts, s.hidden)
        names = ("gate_proj", "up_proj", "down_proj")
        experts = []
        for e in range(s.experts):
            trio = []
            for w, n in enumerate(names):
                if m + f"experts.{n}" in self.tensors:
                    trio.append(self._qt_tuple(m + f"experts.{n}", e))
                elif m + f"experts.{e}.{n}.weight" in self.tensors:
                    trio.append(self._qt_tuple(m + f"experts.{e}.{n}.weight"))
                else:
                    trio.append(self._qt_tuple(p + f"block_sparse_moe.experts.{e}.{('w1', 'w3', 'w2')[w]}.weight"))
            experts.append(trio)
        shared = None
        for stem in ("shared_experts", "shared_expert"):
            if m + f"{stem}.gate_proj.weight" in self.tensors:
                shared = [self._qt_tuple(m + f"{stem}.{n}.weight") for n in names]
        return OracleLayer(s.hidden, s.experts, s.top_k, router, experts, sigmoid=s.sigmoid, norm_topk=s.norm_topk,
                           routed_scale=s.routed_scale, n_group=s.n_group, topk_group=s.topk_group,
                           e_bias=self._f32(m + "gate.e_score_correction_bias", True), shared=shared,
                           shared_gate=self._f32(m + "shared_expert_gate.weight", True))

    # -- the forward -----------------------------------------------------
    def kv_dims(self):
        s = self.spec
        if s.mla:
            return s.heads * (s.mla.qk_nope + s.mla.qk_rope), s.heads * s.mla.v_head
        return s.kv_heads * s.head_dim, s.kv_heads * s.head_dim

    def new_state(self, ctx: int) -> dict:
        kd, vd = self.kv_dims()
        return dict(pos=0, ctx=ctx, k=[np.zeros((ctx, kd), np.float32) for _ in self.layers],
                    v=[np.zeros((ctx, vd), np.float32) for _ in self.layers])

    def _attention(self, li: int, lay: dict, x: np.ndarray, st: dict) -> np.ndarray:
        """Model::attention (src/model.rs:686-834)."""
        s, t, base = self.spec, x.shape[0], st["pos"]
        pos = np.arange(base, base + t, dtype=np.int32)
        if s.mla is None:
            qd = vd = s.head_dim
            n_kv = s.kv_heads
            q, k, v = matmul(lay["q"], x), matmul(lay["k"], x), matmul(lay["v"], x)
            bufs = [q, k, v]
            for i, b in enumerate(lay["bias"]):
                if b is not None:
                    flat = bufs[i].reshape(-1)
                    flat += np.resize(b, flat.size)
            for buf, heads, nrm in ((q, s.heads, lay["q_norm"]), (k, n_kv, lay["k_norm"])):
                if nrm is not None:
                    span = buf.shape[1] if nrm.size == buf.shape[1] else qd
                    buf[:] = rmsnorm_rows(buf.reshape(-1, span), nrm, s.eps).reshape(buf.shape)
                lib().orc_rope_rows(_p(buf), t, buf.shape[1], heads, qd, 0, qd, _p(pos), _p(self.inv), self.inv.size)
            st["k"][li][base:base + t] = k
            st["v"][li][base:base + t] = v
        else:
            m = s.mla
            qd, vd, n_kv = m.qk_nope + m.qk_rope, m.v_head, s.heads
            if lay["q_a"] is not None and lay["q_a_norm"] is not None:
                q = matmul(lay["q_b"], rmsnorm_rows(matmul(lay["q_a"], x), lay["q_a_norm"], s.eps))
            else:
                q = matmul(lay["q_b"], x)
            c = matmul(lay["kv_a"], x)
            cn = rmsnorm_rows(c, lay["kv_a_norm"], s.eps, n=m.kv_lora)
            kv = matmul(lay["kv_b"], cn).reshape(t, s.heads, m.qk_nope + m.v_head)
            kpe = np.ascontiguousarray(c[:, m.kv_lora:])
            lib().orc_rope_rows(_p(kpe), t, m.qk_rope, 1, 0, 0, m.qk_rope, _p(pos), _p(self.inv), self.inv.size)
            lib().orc_rope_rows(_p(q), t, q.shape[1], s.heads, qd, m.qk_nope, m.qk_rope, _p(pos), _p(self.inv),
                                self.inv.size)
            kc = np.concatenate([kv[:, :, :m.qk_nope], np.broadcast_to(kpe[:, None, :], (t, s.heads, m.qk_rope))],
                                axis=2)
            st["k"][li][base:base + t] = kc.reshape(t, -1)
            st["v"][li][base:base + t] = kv[:, :, m.qk_nope:].reshape(t, -1)
        scale = np.float32(self.scale_mult / np.sqrt(np.float32(qd), dtype=np.float32))
        out = self._attend(q, st["k"][li], st["v"][li], t, base, s.heads, n_kv, qd, vd, scale, lay["window"] or 0)
        return matmul(lay["o"], out)

    def _attend(self, q, kc, vc, t, base, heads, n_kv, qd, vd, scale, window) -> np.ndarray:
        """The causal attention loop (src/model.rs:797-831)."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.empty((t, heads * vd), dtype=np.float32)
        lib().orc_attention(_p(q), _p(kc), _p(vc), t, base, heads, n_kv, qd, vd, float(scale), window, _p(out))
        return out

    def trunk(self, tokens, st: dict) -> np.ndarray:
        """Model::trunk (src/model.rs:646-684): the residual stream [t, H]."""
        s = self.spec
        t = len(tokens)
        assert t > 0 and st["pos"] + t <= st["ctx"], "context window exhausted"
        e = self.embed
        rb = row_bytes(e.dt, e.cols)
        data = self.tensors["model.embed_tokens.weight"].data
        x = np.empty((t, s.hidden), dtype=np.float32)
        for i, tok in enumerate(tokens):
            r = int(tok) % s.vocab
            x[i] = dequant(e.dt, np.asarray(data[r * rb:(r + 1) * rb]), 1, e.cols)[0]
        for li, lay in enumerate(self.layers):
            n = rmsnorm_rows(x, lay["ln1"], s.eps)
            x = x + self._attention(li, lay, n, st)
            n = rmsnorm_rows(x, lay["ln2"], s.eps)
            if "moe" in lay:
                delta = lay["moe"].forward(n)[0]
            else:
                delta = mlp_forward(*lay["mlp"], n)
            x = x + delta
        st["pos"] += t
        return x

    def head(self, rows: np.ndarray) -> np.ndarray:
        """Model::head (src/model.rs:636-642) of residual rows."""
        return matmul(self.lm_head, rmsnorm_rows(rows, self.out_norm, self.spec.eps))

    def forward(self, tokens, st: dict) -> np.ndarray:
        """Model::forward: the logits of the last token."""
        x = self.trunk(tokens, st)
        return self.head(x[-1:])[0]

    def forward_all(self, tokens, st: dict) -> np.ndarray:
        """Model::forward_all: logits at every position."""
        return self.head(self.trunk(tokens, st))

    def generate_greedy(self, prompt, max_tokens: int, ctx: Optional[int] = None) -> list:
        """Sampler::default (temp 0: the first index of the maximum,
        src/sample.rs:87-95) in generate's loop (src/generate.rs:142-320)."""
        st = self.new_state(ctx or len(prompt) + max_tokens)
        logits = self.forward(list(prompt), st)
        out = [int(np.argmax(logits))]
        while len(out) < max_tokens:
            logits = self.forward([out[-1]], st)
            out.append(int(np.argmax(logits)))
        return out
