"""A whole decoder on the GPU, its routed layers on the expert kernels.

Mirrors the reference's `Model` (src/model.rs:336-834): the embedding, per
layer RMSNorm -> attention (GQA with optional biases and q/k norms, or MLA
with its latent KV) -> residual, RMSNorm -> FFN (a routed layer, MoeLayer,
or a dense SwiGLU MLP) -> residual, then the final norm and lm_head, and
greedy decoding (src/sample.rs:87-95, src/generate.rs:142-320).  Every
operation runs on the device through libmoe_hip (include/moe_hip.h); torch
holds the buffers.

One call runs several sequences at once: the rows of all sequences go
through the per-row operations (norms, projections, the routed layers)
together, and the attention kernel sends each row to its own sequence's
cache.  This is how the reference's single-sequence forward
(src/model.rs:565, one State per sequence) becomes a batch: with 32
sequences decoding, every routed layer sees T = 32 tokens per step.

`Spec` restates the reference's Spec (src/spec.rs:180-214) with its rope
scaling (src/spec.rs:12-160, 380-411) and windows (src/spec.rs:413-444);
weights are bound by the Hugging Face names the reference reads
(src/model.rs:341-480).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib as L
from .layer import Context, Mlp, MoeLayer, MoeSpec, Rec, Region, Store, View, _stream_ptr, row_bytes

try:
    import torch
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

ROPE_NONE, ROPE_LINEAR, ROPE_DYNAMIC, ROPE_YARN, ROPE_LLAMA3 = 0, 1, 2, 3, 4

# Positions one attention row can cover: moe_attention holds the row's f32
# scores in 64 KiB of LDS.
ATTN_MAX_POSITIONS = 16384


@dataclass
class Rope:
    """src/spec.rs:34-62 (defaults as Rope::default)."""

    kind: int = ROPE_NONE
    theta: float = 10000.0
    factor: float = 1.0
    original_ctx: int = 4096
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    attn_factor: float = 1.0
    mscale: float = 0.0
    mscale_all_dim: float = 0.0

    @staticmethod
    def from_config(cfg: dict, max_ctx: int) -> "Rope":
        """rope_of (src/spec.rs:380-411)."""
        sc = cfg.get("rope_scaling") if isinstance(cfg.get("rope_scaling"), dict) else \
            (cfg.get("rope_parameters") or {})
        theta = cfg.get("rope_theta", (cfg.get("rope_parameters") or {}).get("rope_theta", 10000.0))
        r = Rope(theta=float(theta))
        r.original_ctx = int(sc.get("original_max_position_embeddings", max_ctx))
        named = sc.get("rope_type", sc.get("type", "")) or ""
        factor = float(sc.get("factor", 1.0))
        kinds = {"linear": ROPE_LINEAR, "dynamic": ROPE_DYNAMIC, "ntk": ROPE_DYNAMIC, "yarn": ROPE_YARN,
                 "llama3": ROPE_LLAMA3}
        r.kind = kinds.get(named, ROPE_LINEAR if factor > 1.0 else ROPE_NONE)
        if factor <= 1.0:
            r.kind = ROPE_NONE
        r.factor = factor
        r.low_freq_factor = float(sc.get("low_freq_factor", 1.0))
        r.high_freq_factor = float(sc.get("high_freq_factor", 4.0))
        r.beta_fast = float(sc.get("beta_fast", 32.0))
        r.beta_slow = float(sc.get("beta_slow", 1.0))
        r.attn_factor = float(sc.get("attention_factor", 1.0))
        r.mscale = float(sc.get("mscale", 0.0))
        r.mscale_all_dim = float(sc.get("mscale_all_dim", 0.0))
        return r

    def inv_freqs(self, head_dim: int) -> np.ndarray:
        """Rope::inv_freqs (src/spec.rs:89-145), computed by the library."""
        out = np.zeros(head_dim // 2, dtype=np.float32)
        L.check(L.lib().moe_rope_inv_freqs(self.kind, self.theta, self.factor, self.original_ctx,
                                           self.low_freq_factor, self.high_freq_factor, self.beta_fast,
                                           self.beta_slow, head_dim, out.ctypes.data_as(C.c_void_p)),
                "moe_rope_inv_freqs")
        return out

    def attn_scale(self) -> float:
        """Rope::attn_scale (src/spec.rs:147-160), in f32."""
        f32 = np.float32
        if self.kind != ROPE_YARN:
            return 1.0

        def ms(scale, m):
            return f32(1.0) if f32(scale) <= 1 else f32(f32(f32(0.1) * f32(m)) * f32(math.log(f32(scale)))) + f32(1)

        if self.mscale > 0.0 or self.mscale_all_dim > 0.0:
            return float(f32(ms(self.factor, self.mscale) / max(ms(self.factor, self.mscale_all_dim), f32(1e-6)))
                         * f32(self.attn_factor))
        return float(f32(ms(self.factor, 1.0)) * f32(self.attn_factor))


@dataclass
class Mla:
    """src/spec.rs:170-178."""

    q_lora: int
    kv_lora: int
    qk_nope: int
    qk_rope: int
    v_head: int


@dataclass
class Spec:
    """The fields of the reference's Spec (src/spec.rs:180-214) this forward
    reads."""

    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    rope: Rope = field(default_factory=Rope)
    windows: list = field(default_factory=list)
    max_ctx: int = 4096
    tie: bool = False
    mla: Optional[Mla] = None
    experts: int = 0
    top_k: int = 2
    norm_topk: bool = True
    sigmoid: bool = False
    routed_scale: float = 1.0
    n_group: int = 1
    topk_group: int = 1
    prefix: str = "model.layers."

    def moe_spec(self) -> MoeSpec:
        return MoeSpec(hidden=self.hidden, n_experts=self.experts, top_k=self.top_k, sigmoid=self.sigmoid,
                       norm_topk=self.norm_topk, routed_scale=self.routed_scale, n_group=self.n_group,
                       topk_group=self.topk_group)

    @staticmethod
    def derive(cfg: dict, shapes: dict) -> "Spec":
        """Spec::derive (src/spec.rs:244-338): the config's values, with the
        sizes the checkpoint's shapes fix (vocab and hidden from the
        embedding, key/value heads from k_proj, the expert count from the
        expert tensors) taken from `shapes` (name -> shape, outermost
        first)."""
        def num(*keys, default=None):
            for k in keys:
                v = cfg.get(k)
                if isinstance(v, (int, float)) and not isinstance(v, bool):
                    return v
            return default

        def flag(key, default):
            v = cfg.get(key)
            return v if isinstance(v, bool) else default

        p = "model.layers."
        emb = shapes.get("model.embed_tokens.weight") or shapes.get("embed_tokens.weight")
        if emb is None:
            raise ValueError("no embedding tensor (looked for model.embed_tokens.weight)")
        vocab, hidden = int(emb[-2]), int(emb[-1])
        layers = num("num_hidden_layers", "n_layers", "n_layer")
        if layers is None:
            layers = 0
            while any(n.startswith(f"{p}{layers}.") for n in shapes):
                layers += 1
        layers = int(layers)
        heads = num("num_attention_heads", "n_heads", "n_head")
        if heads is None:
            raise ValueError("config lacks num_attention_heads")
        heads = int(heads)
        mla = None
        kva = shapes.get(f"{p}0.self_attn.kv_a_proj_with_mqa.weight")
        if kva is not None:
            qk_rope = int(num("qk_rope_head_dim", default=64))
            mla = Mla(int(num("q_lora_rank", default=0) or 0), int(num("kv_lora_rank", default=kva[-2] - qk_rope)),
                      int(num("qk_nope_head_dim", default=128)), qk_rope, int(num("v_head_dim", default=128)))
            head_dim, kv_heads = mla.qk_rope, heads
        else:
            q = shapes.get(f"{p}0.self_attn.q_proj.weight")
            if q is None:
                raise ValueError("no self_attn.q_proj.weight in layer 0")
            head_dim = int(num("head_dim", default=q[-2] // heads))
            k = shapes.get(f"{p}0.self_attn.k_proj.weight")
            kv_heads = max(k[-2] // head_dim, 1) if k is not None else heads
        experts = 0
        for l in range(layers):
            for n in ("mlp.experts.gate_up_proj", "mlp.experts.gate_proj", "mlp.experts.down_proj"):
                sh = shapes.get(f"{p}{l}.{n}")
                if sh is not None and len(sh) == 3 and sh[0] > 1:
                    experts = int(sh[0])
                    break
            if experts:
                break
        else:
            while any(f"{p}{l}.mlp.experts.{experts}.down_proj.weight" in shapes
                      or f"{p}{l}.block_sparse_moe.experts.{experts}.w2.weight" in shapes
                      for l in range(min(layers, 2))):
                experts += 1
        sigmoid = cfg.get("scoring_func", "softmax") == "sigmoid" or \
            f"{p}0.mlp.gate.e_score_correction_bias" in shapes
        max_ctx = int(num("max_position_embeddings", default=8192))
        return Spec(hidden=hidden, layers=layers, heads=heads, kv_heads=int(kv_heads), head_dim=int(head_dim),
                    vocab=vocab, eps=float(num("rms_norm_eps", "layer_norm_eps", default=1e-6)),
                    rope=Rope.from_config(cfg, max_ctx), windows=windows_of(cfg, layers), max_ctx=max_ctx,
                    tie=flag("tie_word_embeddings", False) or "lm_head.weight" not in shapes, mla=mla,
                    experts=experts, top_k=int(num("num_experts_per_tok", "moe_top_k", "top_k", default=2)),
                    norm_topk=flag("norm_topk_prob", flag("norm_expert_prob", True)), sigmoid=sigmoid,
                    routed_scale=float(num("routed_scaling_factor", default=1.0)),
                    n_group=int(num("n_group", default=1)), topk_group=int(num("topk_group", default=1)))


def windows_of(cfg: dict, layers: int) -> list:
    """windows_of (src/spec.rs:413-444): the attention window of each layer
    (None = every earlier position)."""
    w = next((cfg[k] for k in ("sliding_window", "attention_window_size")
              if isinstance(cfg.get(k), (int, float)) and not isinstance(cfg.get(k), bool)), None)
    w = int(w) if w and w > 0 else 0
    if not w:
        return [None] * layers
    types = cfg.get("layer_types")
    if isinstance(types, list):
        return [w if (l < len(types) and types[l] in ("sliding_attention", "local_attention")) else None
                for l in range(layers)]
    pattern = cfg.get("sliding_window_pattern")
    if isinstance(pattern, int) and pattern > 1:
        return [None if (l + 1) % pattern == 0 else w for l in range(layers)]
    if cfg.get("use_sliding_window") is False:
        return [None] * layers
    start = int(cfg.get("max_window_layers", 0) or 0)
    return [w if l >= start else None for l in range(layers)]


# ------------------------------------------------------------------- weights


@dataclass
class HostTensor:
    """A checkpoint tensor in host memory: format, shape (outermost first)
    and its stored bytes."""

    dt: int
    shape: tuple
    data: np.ndarray  # uint8

    @property
    def rows(self) -> int:
        return int(np.prod(self.shape[:-1])) if len(self.shape) > 1 else 1

    @property
    def cols(self) -> int:
        return int(self.shape[-1])

    def f32(self) -> np.ndarray:
        """The values (dequantised), [rows, cols]."""
        if self.dt == L.DT_F32:
            return self.data.view(np.float32).reshape(self.rows, self.cols)
        out = np.empty((self.rows, self.cols), dtype=np.float32)
        L.check(L.lib().moe_dequant_rows(self.dt, self.data.ctypes.data_as(C.c_void_p), self.rows, self.cols,
                                         out.ctypes.data_as(C.c_void_p)), "moe_dequant_rows")
        return out


class HostCheckpoint(dict):
    """Named HostTensors whose bytes all live in one host buffer (`buf`, the
    image of an mmap'd checkpoint), each at `offsets[name]`."""

    def __init__(self, buf: np.ndarray):
        super().__init__()
        self.buf, self.offsets = buf, {}

    def add(self, name: str, t: HostTensor, offset: int) -> None:
        self[name] = t
        self.offsets[name] = offset


def upload_store(ctx: Context, tensors: dict) -> Store:
    """Every tensor into one device region, each on a 256-byte boundary
    (moe_upload_tensors), indexed by name as Store::view indexes a file."""
    names = list(tensors)
    offs, lens = [], []
    if isinstance(tensors, HostCheckpoint):
        buf = tensors.buf
        for n in names:
            offs.append(tensors.offsets[n])
            lens.append(tensors[n].data.nbytes)
    else:
        chunks, off = [], 0
        for n in names:
            d = np.ascontiguousarray(tensors[n].data).view(np.uint8).reshape(-1)
            chunks.append(d)
            offs.append(off)
            lens.append(d.nbytes)
            off += d.nbytes
        buf = np.concatenate(chunks) if chunks else np.zeros(1, np.uint8)
    k = len(names)
    o = (C.c_uint64 * k)(*offs)
    ln = (C.c_uint64 * k)(*lens)
    dev = (C.c_uint64 * k)()
    rid = C.c_uint64()
    L.check(L.lib().moe_upload_tensors(ctx.handle, buf.ctypes.data_as(C.c_void_p), buf.nbytes, o, ln, k, dev,
                                       C.byref(rid)), "moe_upload_tensors")
    total = max((dev[i] + lens[i] for i in range(k)), default=0)
    region = Region(ctx, rid.value, total)
    index = {}
    for i, n in enumerate(names):
        t = tensors[n]
        sh = t.shape
        slabs, rows, cols = (sh[0], sh[1], sh[2]) if len(sh) == 3 else (1, sh[0], sh[1]) if len(sh) == 2 else \
            (1, 1, sh[0])
        index[n] = Rec(t.dt, slabs, rows, cols, dev[i])
    return Store(region, index)


# ---------------------------------------------------------------- the model


class Linear:
    """quant::matmul over one weight view (moe_linear)."""

    def __init__(self, ctx: Context, view: View):
        self.view = view
        h = C.c_void_p()
        L.check(L.lib().moe_linear_create(ctx.handle, C.byref(view.c()), C.byref(h)), "moe_linear_create")
        self.handle = h
        self.n, self.k = view.rows, view.cols

    def workspace_size(self, max_t: int) -> int:
        n = C.c_uint64()
        L.check(L.lib().moe_linear_workspace_size(self.handle, max_t, C.byref(n)), "moe_linear_workspace_size")
        return int(n.value)

    def __call__(self, x, y, ws, residual=None, stream=None):
        t = int(x.shape[0])
        L.check(L.lib().moe_linear_forward(self.handle, C.c_void_p(x.data_ptr()), t, C.c_void_p(y.data_ptr()),
                                           C.c_void_p(residual.data_ptr() if residual is not None else None),
                                           C.c_void_p(ws.data_ptr()), ws.numel(), C.c_void_p(_stream_ptr(stream))),
                "moe_linear_forward")
        return y

    def close(self):
        if getattr(self, "handle", None):
            L.lib().moe_linear_destroy(self.handle)
            self.handle = None


class Batch:
    """Which sequence and position each row of a forward call belongs to."""

    def __init__(self, seq: list, pos: list, ctx: int, device):
        self.t = len(seq)
        self.seq = torch.tensor(seq, dtype=torch.int32, device=device)
        self.pos = torch.tensor(pos, dtype=torch.int32, device=device)
        self.dst = torch.tensor([s * ctx + p for s, p in zip(seq, pos)], dtype=torch.int64, device=device)
        self.max_pos = max(pos)


class State:
    """The per-sequence part of the reference's State (src/model.rs:93-189)
    for n_seq sequences: positions and each layer's KV cache
    ([sequence][ctx][keys], [sequence][ctx][values], f32 on the device)."""

    def __init__(self, model: "Model", n_seq: int, ctx: int):
        s = model.spec
        self.ctx, self.n_seq = ctx, n_seq
        self.pos = [0] * n_seq
        kd, vd = model.kv_dims()
        dev = model.device
        self.k = [torch.zeros((n_seq, ctx, kd), dtype=torch.float32, device=dev) for _ in range(s.layers)]
        self.v = [torch.zeros((n_seq, ctx, vd), dtype=torch.float32, device=dev) for _ in range(s.layers)]


class Model:
    """Model (src/model.rs:192-209, 336-834) over weights in one device
    region, bound by the reference's tensor names."""

    def __init__(self, ctx: Context, spec: Spec, store: Store, device="cuda:0"):
        self.ctx, self.spec, self.store, self.device = ctx, spec, store, torch.device(device)
        s = spec
        p = s.prefix
        g = store.get
        self.embed = g("model.embed_tokens.weight")
        self.out_norm = self._vec("model.norm.weight")
        lm = g("lm_head.weight")
        self.lm_head = Linear(ctx, lm if lm is not None else self.embed)
        self.inv_freq = torch.from_numpy(s.rope.inv_freqs(s.mla.qk_rope if s.mla else s.head_dim)).to(self.device)
        self.layers = []
        for l in range(s.layers):
            a = f"{p}{l}.self_attn."
            lay = dict(ln1=self._vec(f"{p}{l}.input_layernorm.weight"),
                       ln2=self._vec(f"{p}{l}.post_attention_layernorm.weight"),
                       o=Linear(ctx, g(a + "o_proj.weight")), window=s.windows[l] if l < len(s.windows) else None)
            if s.mla is None:
                lay.update(q=Linear(ctx, g(a + "q_proj.weight")), k=Linear(ctx, g(a + "k_proj.weight")),
                           v=Linear(ctx, g(a + "v_proj.weight")),
                           bias=[self._vec(a + f"{m}_proj.bias", optional=True) for m in "qkv"],
                           q_norm=self._vec(a + "q_norm.weight", optional=True),
                           k_norm=self._vec(a + "k_norm.weight", optional=True))
            else:
                qa = g(a + "q_a_proj.weight")
                lay.update(q_a=Linear(ctx, qa) if qa is not None else None,
                           q_a_norm=self._vec(a + "q_a_layernorm.weight", optional=True),
                           q_b=Linear(ctx, g(a + "q_b_proj.weight") if qa is not None else g(a + "q_proj.weight")),
                           kv_a=Linear(ctx, g(a + "kv_a_proj_with_mqa.weight")),
                           kv_a_norm=self._vec(a + "kv_a_layernorm.weight"),
                           kv_b=Linear(ctx, g(a + "kv_b_proj.weight")))
            m = f"{p}{l}.mlp."
            if g(m + "gate.weight") is not None or g(f"{p}{l}.block_sparse_moe.gate.weight") is not None:
                from .checkpoint import bind_layer

                lay["moe"] = bind_layer(ctx, store, l, s.moe_spec(), layer_index=l)
            else:
                lay["mlp"] = Mlp(ctx, g(m + "gate_proj.weight"), g(m + "up_proj.weight"), g(m + "down_proj.weight"))
            self.layers.append(lay)
        self._ws = self._mws = None

    # -- helpers ---------------------------------------------------------
    def _vec(self, name: str, optional: bool = False):
        """An F32 vector tensor of the region as a device tensor view."""
        v = self.store.get(name)
        if v is None:
            if optional:
                return None
            raise KeyError(name)
        if v.dt != L.DT_F32:
            raise ValueError(f"{name}: norms and biases must be F32")
        n = v.rows * v.cols
        base = self.store.region.device_ptr() + v.offset
        return _device_floats(base, n, self.device, keep=self.store.region)

    def kv_dims(self):
        """(key, value) floats cached per position (Model::kv_dims, src/model.rs:546-551)."""
        s = self.spec
        if s.mla:
            return s.heads * (s.mla.qk_nope + s.mla.qk_rope), s.heads * s.mla.v_head
        return s.kv_heads * s.head_dim, s.kv_heads * s.head_dim

    def new_state(self, n_seq: int, ctx: int) -> State:
        # moe_attention keeps one row's scores in LDS: at most
        # ATTN_MAX_POSITIONS positions per row (the window, where a layer
        # has one).  A longer context is refused here, before any step.
        layers = self.spec.layers
        wins = list(self.spec.windows) + [None] * max(0, layers - len(self.spec.windows))
        widest = max(min(w, ctx) if w else ctx for w in wins) if wins else ctx
        if widest > ATTN_MAX_POSITIONS:
            raise ValueError(f"a context of {ctx} positions: attention here covers at most "
                             f"{ATTN_MAX_POSITIONS} positions per row")
        return State(self, n_seq, ctx)

    def _workspace(self, t: int):
        lins = [self.lm_head]
        for lay in self.layers:
            lins += [v for k, v in lay.items() if isinstance(v, Linear)]
        need = max(l.workspace_size(t) for l in lins)
        if self._ws is None or self._ws.numel() < need:
            buf = torch.empty(need + 256, dtype=torch.uint8, device=self.device)
            off = (-buf.data_ptr()) % 256
            self._ws = buf[off:off + need]
        return self._ws

    def _ffn_workspace(self, t: int):
        """One workspace every FFN layer runs on in turn (calls on one stream
        are ordered, and each leaves the workspace's persistent counter at
        zero)."""
        need = max((lay["moe"] if "moe" in lay else lay["mlp"].layer).workspace_size(t) for lay in self.layers)
        if self._mws is None or self._mws.numel() < need:
            self._mws = MoeLayer.new_workspace(need, device=self.device)
        return self._mws

    # -- the forward -----------------------------------------------------
    def trunk(self, tokens: list, st: State, seqs: Optional[list] = None, stream=None):
        """Model::trunk (src/model.rs:646-684) for tokens[i] (a list per
        sequence, sequence seqs[i] of the state); returns the residual
        stream [rows, H] and the batch."""
        s = self.spec
        seqs = list(range(len(tokens))) if seqs is None else seqs
        seq_of, pos_of, ids = [], [], []
        for q, toks in zip(seqs, tokens):
            for i, tok in enumerate(toks):
                seq_of.append(q)
                pos_of.append(st.pos[q] + i)
                ids.append(int(tok))
            if st.pos[q] + len(toks) > st.ctx:
                raise ValueError("context window exhausted")
        b = Batch(seq_of, pos_of, st.ctx, self.device)
        t, H = b.t, s.hidden
        sp = _stream_ptr(stream)
        lib = L.lib()
        ws = self._workspace(t)
        mws = self._ffn_workspace(t)
        x = torch.empty((t, H), dtype=torch.float32, device=self.device)
        tok = torch.tensor(ids, dtype=torch.int32, device=self.device)
        e = self.embed
        L.check(lib.moe_embed_rows(C.c_void_p(self.store.region.device_ptr() + e.offset), e.dt, e.rows, e.cols,
                                   C.c_void_p(tok.data_ptr()), t, C.c_void_p(x.data_ptr()), C.c_void_p(sp)),
                "moe_embed_rows")
        norm = torch.empty_like(x)
        for li, lay in enumerate(self.layers):
            self._rmsnorm(x, lay["ln1"], norm, stream)
            self._attention(li, lay, norm, b, st, x, ws, stream)
            self._rmsnorm(x, lay["ln2"], norm, stream)
            out = torch.empty_like(x)
            ffn = lay["moe"] if "moe" in lay else lay["mlp"].layer
            ffn.feed_forward(norm, out, residual=x, stream=stream, workspace=mws)
        for q, toks in zip(seqs, tokens):
            st.pos[q] += len(toks)
        return x, b

    def _rmsnorm(self, x, w, out, stream, rows=None, n=None, xs=None, os_=None):
        rows = x.shape[0] if rows is None else rows
        n = x.shape[-1] if n is None else n
        L.check(L.lib().moe_rmsnorm(C.c_void_p(x.data_ptr()), x.shape[-1] if xs is None else xs,
                                    C.c_void_p(w.data_ptr()), rows, n, self.spec.eps, C.c_void_p(out.data_ptr()),
                                    out.shape[-1] if os_ is None else os_, C.c_void_p(_stream_ptr(stream))),
                "moe_rmsnorm")

    def _rope(self, x, rows, row_stride, heads, head_stride, offset, dim, b: Batch, stream):
        L.check(L.lib().moe_rope(C.c_void_p(x.data_ptr()), rows, row_stride, heads, head_stride, offset, dim,
                                 C.c_void_p(b.pos.data_ptr()), C.c_void_p(self.inv_freq.data_ptr()),
                                 self.inv_freq.numel(), C.c_void_p(_stream_ptr(stream))), "moe_rope")

    def _attention(self, li, lay, x, b: Batch, st: State, resid, ws, stream):
        """Model::attention (src/model.rs:686-834); resid += o(ctx)."""
        s = self.spec
        t, dev, sp = b.t, self.device, C.c_void_p(_stream_ptr(stream))
        lib = L.lib()
        f32 = torch.float32
        if s.mla is None:
            qd = vd = s.head_dim
            n_kv = s.kv_heads
            q = lay["q"](x, torch.empty((t, s.heads * qd), dtype=f32, device=dev), ws, stream=stream)
            k = lay["k"](x, torch.empty((t, n_kv * qd), dtype=f32, device=dev), ws, stream=stream)
            v = lay["v"](x, torch.empty((t, n_kv * vd), dtype=f32, device=dev), ws, stream=stream)
            for buf, bias in zip((q, k, v), lay["bias"]):
                if bias is not None:
                    L.check(lib.moe_add_bias(C.c_void_p(buf.data_ptr()), buf.numel(), C.c_void_p(bias.data_ptr()),
                                             bias.numel(), sp), "moe_add_bias")
            for buf, heads, nrm in ((q, s.heads, lay["q_norm"]), (k, n_kv, lay["k_norm"])):
                if nrm is not None:
                    # One weight across the projection (OLMoE) or one per head (Qwen3).
                    span = buf.shape[1] if nrm.numel() == buf.shape[1] else qd
                    tmp = torch.empty_like(buf)
                    self._rmsnorm(buf, nrm, tmp, stream, rows=buf.numel() // span, n=span, xs=span, os_=span)
                    buf.copy_(tmp)
                self._rope(buf, t, buf.shape[1], heads, qd, 0, qd, b, stream)
            kd, vdim = n_kv * qd, n_kv * vd
            L.check(lib.moe_scatter_rows(C.c_void_p(k.data_ptr()), t, kd, kd, C.c_void_p(st.k[li].data_ptr()), kd,
                                         C.c_void_p(b.dst.data_ptr()), sp), "moe_scatter_rows")
            L.check(lib.moe_scatter_rows(C.c_void_p(v.data_ptr()), t, vdim, vdim, C.c_void_p(st.v[li].data_ptr()),
                                         vdim, C.c_void_p(b.dst.data_ptr()), sp), "moe_scatter_rows")
        else:
            m = s.mla
            qd, vd, n_kv = m.qk_nope + m.qk_rope, m.v_head, s.heads
            if lay["q_a"] is not None:
                cq = lay["q_a"](x, torch.empty((t, m.q_lora), dtype=f32, device=dev), ws, stream=stream)
                cqn = torch.empty_like(cq)
                self._rmsnorm(cq, lay["q_a_norm"], cqn, stream)
                q = lay["q_b"](cqn, torch.empty((t, s.heads * qd), dtype=f32, device=dev), ws, stream=stream)
            else:
                q = lay["q_b"](x, torch.empty((t, s.heads * qd), dtype=f32, device=dev), ws, stream=stream)
            ca = m.kv_lora + m.qk_rope
            c = lay["kv_a"](x, torch.empty((t, ca), dtype=f32, device=dev), ws, stream=stream)
            cn = torch.empty((t, m.kv_lora), dtype=f32, device=dev)
            self._rmsnorm(c, lay["kv_a_norm"], cn, stream, n=m.kv_lora, xs=ca, os_=m.kv_lora)
            kv = lay["kv_b"](cn, torch.empty((t, s.heads * (m.qk_nope + m.v_head)), dtype=f32, device=dev), ws,
                             stream=stream)
            self._rope(c, t, ca, 1, 0, m.kv_lora, m.qk_rope, b, stream)
            self._rope(q, t, s.heads * qd, s.heads, qd, m.qk_nope, m.qk_rope, b, stream)
            L.check(lib.moe_mla_kv_store(C.c_void_p(kv.data_ptr()), C.c_void_p(c.data_ptr()), ca, m.kv_lora, t,
                                         s.heads, m.qk_nope, m.qk_rope, m.v_head, C.c_void_p(st.k[li].data_ptr()),
                                         C.c_void_p(st.v[li].data_ptr()), C.c_void_p(b.dst.data_ptr()), sp),
                    "moe_mla_kv_store")
        scale = float(np.float32(s.rope.attn_scale()) / np.sqrt(np.float32(qd), dtype=np.float32))
        ctxv = torch.empty((t, s.heads * vd), dtype=f32, device=dev)
        win = lay["window"] or 0
        L.check(lib.moe_attention(C.c_void_p(q.data_ptr()), q.shape[1], t, s.heads, n_kv, qd, vd, scale,
                                  C.c_void_p(st.k[li].data_ptr()), C.c_void_p(st.v[li].data_ptr()), st.ctx,
                                  C.c_void_p(b.seq.data_ptr()), C.c_void_p(b.pos.data_ptr()), b.max_pos, win,
                                  C.c_void_p(ctxv.data_ptr()), ctxv.shape[1], sp), "moe_attention")
        y = torch.empty_like(resid)
        lay["o"](ctxv, y, ws, residual=resid, stream=stream)

    def head(self, x, rows, stream=None):
        """Model::head (src/model.rs:636-642) for the chosen rows of the
        residual stream: logits [len(rows), vocab]."""
        s = self.spec
        idx = torch.tensor(rows, dtype=torch.int64, device=self.device)
        last = x.index_select(0, idx).contiguous()
        nx = torch.empty_like(last)
        self._rmsnorm(last, self.out_norm, nx, stream)
        logits = torch.empty((len(rows), s.vocab), dtype=torch.float32, device=self.device)
        return self.lm_head(nx, logits, self._workspace(len(rows)), stream=stream)

    def forward(self, tokens: list, st: State, seqs: Optional[list] = None, stream=None):
        """Model::forward (src/model.rs:565-570) for each sequence: the
        logits of its last token, [len(tokens), vocab]."""
        x, b = self.trunk(tokens, st, seqs, stream)
        ends, r = [], 0
        for toks in tokens:
            r += len(toks)
            ends.append(r - 1)
        return self.head(x, ends, stream)

    def forward_all(self, tokens: list, st: State, stream=None):
        """Model::forward_all (src/model.rs:572-589) for one sequence: logits
        at every position."""
        x, b = self.trunk([tokens], st, [0], stream)
        return self.head(x, list(range(len(tokens))), stream)

    def argmax(self, logits, stream=None):
        out = torch.empty(logits.shape[0], dtype=torch.int32, device=self.device)
        L.check(L.lib().moe_argmax(C.c_void_p(logits.data_ptr()), logits.shape[0], logits.shape[1],
                                   C.c_void_p(out.data_ptr()), C.c_void_p(_stream_ptr(stream))), "moe_argmax")
        return out

    def generate_greedy(self, prompts: list, max_tokens: int, st: Optional[State] = None, stream=None) -> list:
        """Greedy generation (Sampler::default, temp 0: src/sample.rs:87-95;
        the loop of src/generate.rs:142-320 without stop tokens) for every
        prompt at once: the prefill of all prompts is one batch, then each
        step feeds every sequence its last token."""
        n = len(prompts)
        if st is None:
            st = self.new_state(n, max(len(p) for p in prompts) + max_tokens)
        logits = self.forward(prompts, st, stream=stream)
        out = [[] for _ in range(n)]
        nxt = self.argmax(logits, stream).cpu().tolist()
        for i in range(n):
            out[i].append(nxt[i])
        while len(out[0]) < max_tokens:
            logits = self.forward([[t] for t in nxt], st, stream=stream)
            nxt = self.argmax(logits, stream).cpu().tolist()
            for i in range(n):
                out[i].append(nxt[i])
        return out

    def close(self):
        for lay in self.layers:
            for v in lay.values():
                if hasattr(v, "close"):
                    v.close()
        self.lm_head.close()


def _device_floats(ptr: int, n: int, device, keep=None):
    """A float32 tensor holding a copy of the n floats of device memory at
    ptr (a vector inside an uploaded region)."""
    class _View:
        __cuda_array_interface__ = {"shape": (n,), "typestr": "<f4", "data": (ptr, False), "version": 3}

    return torch.as_tensor(_View(), device=device).clone()
