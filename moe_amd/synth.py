"""Seeded synthetic MoE layers at the benchmark shapes.

A layer is laid out as one byte region the way a packed checkpoint lays out
its tensors: the router, the optional correction bias, the experts as three
stacked tensors (``experts.gate`` / ``experts.up`` as [E, I, H] and
``experts.down`` as [E, H, I], GGUF's ``ffn_*_exps`` layout), and the
optional shared expert and its gate.  Every tensor starts on a 256-byte
boundary, and an expert is a row range inside its stack (src/store.rs:303-315,
src/model.rs:396-421).  Values are N(mean, std) from the library's seeded
generator and are quantised with the reference's quantiser.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, replace
from typing import Optional

import numpy as np

from . import _lib as L
from .layer import MoeSpec, Rec, Store, View, row_bytes

# Generator streams of a layer's tensors.
STREAM_ROUTER, STREAM_EBIAS, STREAM_SHGATE = 1, 2, 3
STREAM_SHARED = (4, 5, 6)
STREAM_ACTS = 0xA000


def stream_expert(e: int, which: int) -> int:
    return 16 + 3 * e + which


@dataclass(frozen=True)
class Shape:
    """A routed layer's shape and routing rule."""

    name: str
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    expert_dt: int
    sigmoid: bool = False
    norm_topk: bool = True
    routed_scale: float = 1.0
    n_group: int = 1
    topk_group: int = 1
    shared_inter: int = 0
    shared_dt: Optional[int] = None
    e_bias_std: float = 0.0
    shared_gate: bool = False
    weight_std: float = 0.02
    router_std: float = 0.02
    zipf: float = 0.0          # > 0: router rows rescaled so expert popularity follows Zipf(zipf)

    def spec(self) -> MoeSpec:
        return MoeSpec(hidden=self.hidden, n_experts=self.n_experts, top_k=self.top_k, sigmoid=self.sigmoid,
                       norm_topk=self.norm_topk, routed_scale=self.routed_scale, n_group=self.n_group,
                       topk_group=self.topk_group)

    def expert_bytes(self) -> int:
        return 2 * self.inter * row_bytes(self.expert_dt, self.hidden) + self.hidden * row_bytes(self.expert_dt,
                                                                                                  self.inter)

    def shared_bytes(self) -> int:
        if not self.shared_inter:
            return 0
        dt = self.shared_dt if self.shared_dt is not None else self.expert_dt
        return 2 * self.shared_inter * row_bytes(dt, self.hidden) + self.hidden * row_bytes(dt, self.shared_inter)


SHAPES = {
    # Mixtral-8x7B layer, Q4_0, softmax top-2, renormalised.
    "mixtral": Shape("mixtral", 4096, 14336, 8, 2, L.DT_Q4_0),
    # Qwen3-30B-A3B layer, Q8_0, softmax top-8, renormalised.
    "qwen3": Shape("qwen3", 2048, 768, 128, 8, L.DT_Q8_0),
    # DeepSeek-V3 layer: sigmoid + bias N(0, 0.1), 8 groups keep 4,
    # top-8, scale 2.5, Q4_0 routed experts, one Q5_0 shared expert.
    "deepseek_v3": Shape("deepseek_v3", 7168, 2048, 256, 8, L.DT_Q4_0, sigmoid=True, routed_scale=2.5,
                         n_group=8, topk_group=4, shared_inter=2048, shared_dt=L.DT_Q5_0, e_bias_std=0.1),
    # configs[3] as benchmarked: router rows skewed so expert popularity is
    # Zipf(s = 1.1) (see zipf_router_scales).
    "deepseek_v3_zipf": Shape("deepseek_v3_zipf", 7168, 2048, 256, 8, L.DT_Q4_0, sigmoid=True, routed_scale=2.5,
                              n_group=8, topk_group=4, shared_inter=2048, shared_dt=L.DT_Q5_0, e_bias_std=0.1,
                              zipf=1.1),
    # DeepSeek-V2-Lite MoE layer: 64 experts top-6 plus two shared
    # experts loaded as one 2816-wide MLP (src/model.rs:431-439), Q8_0.  The
    # model's own config sets norm_topk_prob false, which the reference reads.
    "v2_lite": Shape("v2_lite", 2048, 1408, 64, 6, L.DT_Q8_0, norm_topk=False, shared_inter=2816,
                     shared_dt=L.DT_Q8_0),
    # configs[0]'s MoE layer: tiny Mixtral, hidden 512, 8 experts top-2, Q8_0.
    "tiny_mixtral": Shape("tiny_mixtral", 512, 1408, 8, 2, L.DT_Q8_0),
    # A Qwen2-MoE layer (Qwen1.5-MoE-A2.7B: 60 experts of 1408, top-4, not
    # renormalised, one 5632-wide shared expert scaled by the sigmoid of
    # mlp.shared_expert_gate.weight . x, src/model.rs:956-970), Q8_0: the
    # layer family whose shared expert carries a gate.
    "qwen2_moe": Shape("qwen2_moe", 2048, 1408, 60, 4, L.DT_Q8_0, norm_topk=False, shared_inter=5632,
                       shared_dt=L.DT_Q8_0, shared_gate=True),
}


def scaled(shape: Shape, **kw) -> Shape:
    """The same routing rule at other sizes (for quick parity cases)."""
    return replace(shape, **kw)


def _align(v: int, a: int = 256) -> int:
    return (v + a - 1) // a * a


@dataclass
class HostLayer:
    """A layer's bytes in host memory plus its tensor index."""

    shape: Shape
    buf: np.ndarray          # uint8
    index: dict              # name -> Rec

    def tensor(self, name: str) -> np.ndarray:
        r = self.index[name]
        return self.buf[r.offset:r.offset + r.nbytes]


def _fill(dst: np.ndarray, seed: int, stream: int, dt: int, rows: int, cols: int, mean: float, std: float) -> None:
    rc = L.lib().moe_synth_quantized(seed, stream, dt, rows, cols, mean, std, dst.ctypes.data_as(C.c_void_p))
    L.check(rc, "moe_synth_quantized")


STREAM_ZIPF_CAL = 0xB000  # calibration activations of the Zipf skew


def zipf_targets(n_experts: int, s: float, total: float, cap: float) -> np.ndarray:
    """Selections per popularity rank r = 1..E proportional to r^-s, summing to
    `total`, with no rank above `cap` (the excess spread over the others in
    proportion, repeatedly)."""
    w = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    t = w / w.sum() * total
    fixed = np.zeros(n_experts, dtype=bool)
    for _ in range(n_experts):
        over = (t > cap) & ~fixed
        if not over.any():
            break
        fixed |= over
        t[fixed] = cap
        free = ~fixed
        t[free] = w[free] / w[free].sum() * (total - cap * fixed.sum())
    return t


def _route_counts(logits: np.ndarray, bias: np.ndarray, shape: Shape) -> np.ndarray:
    """Selections per expert under the layer's rule (src/model.rs:855-888):
    sigmoid or softmax scores, + bias, group-limited, top-k; float64, for
    calibration only."""
    T, E = logits.shape
    sc = 1.0 / (1.0 + np.exp(-logits)) if shape.sigmoid else np.exp(logits - logits.max(1, keepdims=True))
    rank = sc + bias[None, :]
    if shape.n_group > 1 and shape.topk_group < shape.n_group:
        per = E // shape.n_group
        g = rank.reshape(T, shape.n_group, per)
        gs = np.sort(g, axis=2)[:, :, -2:].sum(axis=2)
        keep = np.argsort(-gs, axis=1, kind="stable")[:, :shape.topk_group]
        mask = np.full((T, shape.n_group), -np.inf)
        np.put_along_axis(mask, keep, 0.0, axis=1)
        rank = (g + mask[:, :, None]).reshape(T, E)
    sel = np.argsort(-rank, axis=1, kind="stable")[:, :shape.top_k]
    return np.bincount(sel.ravel(), minlength=E)


def zipf_router_scales(router: np.ndarray, bias: np.ndarray, shape: Shape, seed: int,
                       n_cal: int = 512) -> np.ndarray:
    """Per-expert scales for the router rows, so that on a calibration batch
    of N(0, 1) tokens the selection histogram comes as close as this family
    allows to Zipf(shape.zipf) over the experts.

    x has zero mean, so scaling a row changes only the spread of its logits;
    under sigmoid scores an expert clears the top-k threshold for at most
    about half of the tokens, so the target is capped at 0.45 of the tokens
    (zipf_targets).  The scales follow a power law of a seeded popularity rank
    r, exp(a - b ln r); (a, b) is the point of a fixed grid whose histogram,
    sorted, is nearest the target in L1 — deterministic, so every build of
    the layer has the same bytes.  With the DeepSeek-V3 rule the correction
    bias (N(0, 0.1)) dominates which experts are popular; the scales set how
    concentrated the histogram is."""
    E = shape.n_experts
    x = activations(seed, n_cal, shape.hidden).astype(np.float64)
    base = x @ router.astype(np.float64).T
    order = np.random.default_rng(seed).permutation(E)  # order[r] = expert of popularity rank r + 1
    log_rank = np.empty(E)
    log_rank[order] = np.log(np.arange(1, E + 1, dtype=np.float64))
    target = zipf_targets(E, shape.zipf, float(n_cal * shape.top_k), 0.45 * n_cal)
    bias64 = bias.astype(np.float64)
    best, best_ab = None, (0.0, 0.0)
    for a in np.linspace(-2.0, 4.0, 13):
        for b in np.linspace(0.0, 3.0, 13):
            counts = _route_counts(base * np.exp(a - b * log_rank)[None, :], bias64, shape)
            err = np.abs(np.sort(counts)[::-1] - target).sum()
            if best is None or err < best:
                best, best_ab = err, (a, b)
    return np.exp(best_ab[0] - best_ab[1] * log_rank)


def zipf_histogram(shape: Shape, seed: int, t: int, act_seed: int = 1) -> dict:
    """The Zipf workload as routed: the layer's router and bias exactly as
    build_host_layer makes them (same streams, same calibration), the
    selections per expert of activations(act_seed, t) under the layer's rule
    (float64, as the calibration counts them), sorted, beside zipf_targets at
    the same total and cap."""
    E, H = shape.n_experts, shape.hidden
    router = np.empty((E, H), dtype=np.float32)
    _fill(router.view(np.uint8).reshape(-1), seed, STREAM_ROUTER, L.DT_F32, E, H, 0.0, shape.router_std)
    bias = np.zeros(E, dtype=np.float32)
    if shape.e_bias_std > 0:
        _fill(bias.view(np.uint8), seed, STREAM_EBIAS, L.DT_F32, 1, E, 0.0, shape.e_bias_std)
    scales = zipf_router_scales(router, bias, shape, seed)
    router *= scales.astype(np.float32)[:, None]
    x = activations(act_seed, t, H).astype(np.float64)
    counts = _route_counts(x @ router.astype(np.float64).T, bias.astype(np.float64), shape)
    target = zipf_targets(E, shape.zipf, float(t * shape.top_k), 0.45 * t)
    return dict(counts=np.sort(counts)[::-1], target=target, hit=int((counts > 0).sum()), t=t, k=shape.top_k)


def build_host_layer(shape: Shape, seed: int) -> HostLayer:
    """Generate and quantise every tensor of a layer into one byte buffer."""
    E, H, I = shape.n_experts, shape.hidden, shape.inter
    plan = [("router", L.DT_F32, 1, E, H)]
    if shape.e_bias_std > 0:
        plan.append(("e_bias", L.DT_F32, 1, 1, E))
    plan += [("experts.gate", shape.expert_dt, E, I, H), ("experts.up", shape.expert_dt, E, I, H),
             ("experts.down", shape.expert_dt, E, H, I)]
    if shape.shared_inter:
        sdt = shape.shared_dt if shape.shared_dt is not None else shape.expert_dt
        Is = shape.shared_inter
        plan += [("shared.gate", sdt, 1, Is, H), ("shared.up", sdt, 1, Is, H), ("shared.down", sdt, 1, H, Is)]
    if shape.shared_gate:
        plan.append(("shared_gate", L.DT_F32, 1, 1, H))
    index, off = {}, 0
    for name, dt, slabs, rows, cols in plan:
        rec = Rec(dt, slabs, rows, cols, off)
        index[name] = rec
        off = _align(off + rec.nbytes)
    buf = np.zeros(max(off, 256), dtype=np.uint8)
    for name, dt, slabs, rows, cols in plan:
        r = index[name]
        dst = buf[r.offset:r.offset + r.nbytes]
        if name == "router":
            _fill(dst, seed, STREAM_ROUTER, dt, rows, cols, 0.0, shape.router_std)
        elif name == "e_bias":
            _fill(dst, seed, STREAM_EBIAS, dt, rows, cols, 0.0, shape.e_bias_std)
        elif name == "shared_gate":
            _fill(dst, seed, STREAM_SHGATE, dt, rows, cols, 0.0, shape.router_std)
        elif name.startswith("experts."):
            which = ("experts.gate", "experts.up", "experts.down").index(name)
            rb = row_bytes(dt, cols) * rows
            for e in range(slabs):
                _fill(dst[e * rb:(e + 1) * rb], seed, stream_expert(e, which), dt, rows, cols, 0.0,
                      shape.weight_std)
        else:
            which = ("shared.gate", "shared.up", "shared.down").index(name)
            _fill(dst, seed, STREAM_SHARED[which], dt, rows, cols, 0.0, shape.weight_std)
    if shape.zipf > 0:
        r = index["router"]
        router = buf[r.offset:r.offset + r.nbytes].view(np.float32).reshape(E, H)
        bias = (buf[index["e_bias"].offset:index["e_bias"].offset + 4 * E].view(np.float32)
                if "e_bias" in index else np.zeros(E, np.float32))
        router *= zipf_router_scales(router, bias, shape, seed).astype(np.float32)[:, None]
    return HostLayer(shape, buf, index)


def activations(seed: int, t: int, hidden: int) -> np.ndarray:
    """x [t, hidden] ~ N(0, 1), f32 (stream depends on t, so every T is its own input)."""
    out = np.empty((t, hidden), dtype=np.float32)
    L.check(L.lib().moe_synth_normal(seed, STREAM_ACTS + t, out.size, 0.0, 1.0, out.ctypes.data_as(C.c_void_p)),
            "moe_synth_normal")
    return out


def normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    L.check(L.lib().moe_synth_normal(seed, stream, n, mean, std, out.ctypes.data_as(C.c_void_p)), "moe_synth_normal")
    return out


def layer_views(store: Store, shape: Shape):
    """(router, e_bias, experts[(gate, up, down)], shared, shared_gate) views,
    each expert a row range of its stack (src/model.rs:396-421)."""
    E, I, H = shape.n_experts, shape.inter, shape.hidden
    experts = [(store.view("experts.gate", e, 0, I), store.view("experts.up", e, 0, I),
                store.view("experts.down", e, 0, H)) for e in range(E)]
    shared = None
    if shape.shared_inter:
        shared = (store.get("shared.gate"), store.get("shared.up"), store.get("shared.down"))
    return (store.get("router"), store.get("e_bias"), experts, shared, store.get("shared_gate"))


def make_layer(ctx, host: HostLayer, layer_index: int = 0):
    """Upload a host layer and bind a MoeLayer over it."""
    from .layer import MoeLayer

    region = ctx.upload(host.buf)
    store = Store(region, host.index)
    router, e_bias, experts, shared, shared_gate = layer_views(store, host.shape)
    layer = MoeLayer(ctx, host.shape.spec(), router, experts, e_bias=e_bias, shared=shared,
                     shared_gate=shared_gate, layer_index=layer_index)
    layer._region = region  # keep the region alive with the layer
    return layer


# ------------------------------------------------------------ whole models


@dataclass(frozen=True)
class ModelShape:
    """A decoder's architecture as a Hugging Face config states it
    (BASELINE.json configs[0] and configs[4])."""

    name: str
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    moe_inter: int
    n_experts: int
    top_k: int
    dt: int
    style: str                      # "mixtral" (block_sparse_moe names) or "deepseek"
    dense_inter: int = 0            # the dense MLP of layers before first_dense
    first_dense: int = 0
    shared_inter: int = 0
    norm_topk: bool = True
    mla: Optional[tuple] = None     # (q_lora, kv_lora, qk_nope, qk_rope, v_head)
    rope_theta: float = 10000.0
    rope_scaling: Optional[dict] = None
    eps: float = 1e-6
    max_pos: int = 4096
    weight_std: float = 0.02

    def config(self) -> dict:
        c = {"hidden_size": self.hidden, "num_hidden_layers": self.layers, "num_attention_heads": self.heads,
             "num_key_value_heads": self.kv_heads, "vocab_size": self.vocab, "rms_norm_eps": self.eps,
             "rope_theta": self.rope_theta, "max_position_embeddings": self.max_pos,
             "num_experts_per_tok": self.top_k, "norm_topk_prob": self.norm_topk, "tie_word_embeddings": False}
        if self.style == "mixtral":
            c.update(architectures=["MixtralForCausalLM"], model_type="mixtral", head_dim=self.head_dim,
                     intermediate_size=self.moe_inter, num_local_experts=self.n_experts)
        else:
            q_lora, kv_lora, nope, rope, v = self.mla
            c.update(architectures=["DeepseekV2ForCausalLM"], model_type="deepseek_v2",
                     q_lora_rank=q_lora or None, kv_lora_rank=kv_lora, qk_nope_head_dim=nope,
                     qk_rope_head_dim=rope, v_head_dim=v, intermediate_size=self.dense_inter,
                     moe_intermediate_size=self.moe_inter, n_routed_experts=self.n_experts,
                     n_shared_experts=self.shared_inter // self.moe_inter, first_k_dense_replace=self.first_dense,
                     scoring_func="softmax", routed_scaling_factor=1.0, n_group=1, topk_group=1)
        if self.rope_scaling:
            c["rope_scaling"] = dict(self.rope_scaling)
        return c

    def plan(self) -> list:
        """(name, dt, shape, fill) of every tensor; fill is "ones" (norms),
        "router" (F32 N(0, std)) or "weight" (N(0, std) in the model's
        format)."""
        H, dt, p = self.hidden, self.dt, "model.layers."
        out = [("model.embed_tokens.weight", dt, (self.vocab, H), "weight"),
               ("model.norm.weight", 0, (H,), "ones"), ("lm_head.weight", dt, (self.vocab, H), "weight")]
        for l in range(self.layers):
            a = f"{p}{l}.self_attn."
            out += [(f"{p}{l}.input_layernorm.weight", 0, (H,), "ones"),
                    (f"{p}{l}.post_attention_layernorm.weight", 0, (H,), "ones")]
            if self.mla is None:
                hd = self.head_dim
                out += [(a + "q_proj.weight", dt, (self.heads * hd, H), "weight"),
                        (a + "k_proj.weight", dt, (self.kv_heads * hd, H), "weight"),
                        (a + "v_proj.weight", dt, (self.kv_heads * hd, H), "weight"),
                        (a + "o_proj.weight", dt, (H, self.heads * hd), "weight")]
            else:
                q_lora, kv_lora, nope, rope, v = self.mla
                if q_lora:
                    out += [(a + "q_a_proj.weight", dt, (q_lora, H), "weight"),
                            (a + "q_a_layernorm.weight", 0, (q_lora,), "ones"),
                            (a + "q_b_proj.weight", dt, (self.heads * (nope + rope), q_lora), "weight")]
                else:
                    out.append((a + "q_proj.weight", dt, (self.heads * (nope + rope), H), "weight"))
                out += [(a + "kv_a_proj_with_mqa.weight", dt, (kv_lora + rope, H), "weight"),
                        (a + "kv_a_layernorm.weight", 0, (kv_lora,), "ones"),
                        (a + "kv_b_proj.weight", dt, (self.heads * (nope + v), kv_lora), "weight"),
                        (a + "o_proj.weight", dt, (H, self.heads * v), "weight")]
            m = f"{p}{l}.mlp."
            if l < self.first_dense:
                I = self.dense_inter
                out += [(m + "gate_proj.weight", dt, (I, H), "weight"), (m + "up_proj.weight", dt, (I, H), "weight"),
                        (m + "down_proj.weight", dt, (H, I), "weight")]
                continue
            I = self.moe_inter
            if self.style == "mixtral":
                b = f"{p}{l}.block_sparse_moe."
                out.append((b + "gate.weight", 0, (self.n_experts, H), "router"))
                for e in range(self.n_experts):
                    out += [(b + f"experts.{e}.w1.weight", dt, (I, H), "weight"),
                            (b + f"experts.{e}.w3.weight", dt, (I, H), "weight"),
                            (b + f"experts.{e}.w2.weight", dt, (H, I), "weight")]
            else:
                out.append((m + "gate.weight", 0, (self.n_experts, H), "router"))
                for e in range(self.n_experts):
                    out += [(m + f"experts.{e}.gate_proj.weight", dt, (I, H), "weight"),
                            (m + f"experts.{e}.up_proj.weight", dt, (I, H), "weight"),
                            (m + f"experts.{e}.down_proj.weight", dt, (H, I), "weight")]
                if self.shared_inter:
                    S = self.shared_inter
                    out += [(m + "shared_experts.gate_proj.weight", dt, (S, H), "weight"),
                            (m + "shared_experts.up_proj.weight", dt, (S, H), "weight"),
                            (m + "shared_experts.down_proj.weight", dt, (H, S), "weight")]
        return out


MODEL_SHAPES = {
    # tiny Mixtral, 2 layers, hidden 512, 8 heads (2 key/value
    # heads: Mixtral's 4:1 grouping), 8 experts of 1408 top-2, vocab 32000,
    # every big weight Q8_0 from N(0, 0.02).
    "tiny_mixtral": ModelShape("tiny_mixtral", 512, 2, 8, 2, 64, 32000, 1408, 8, 2, L.DT_Q8_0, "mixtral",
                               rope_theta=1e6, eps=1e-5, max_pos=32768),
    # DeepSeek-V2-Lite, 27 layers, hidden 2048, 16 MLA heads
    # (no query LoRA, kv_lora 512, 128 + 64 key dims, 128 value dims, YaRN
    # factor 40 as its config states), layer 0 a dense 10944 MLP, then 64
    # routed experts of 1408 top-6 (not renormalised) plus 2 shared experts
    # (one 2816-wide MLP), vocab 102400, Q8_0 from N(0, 0.02).
    "v2_lite": ModelShape("v2_lite", 2048, 27, 16, 16, 64, 102400, 1408, 64, 6, L.DT_Q8_0, "deepseek",
                          dense_inter=10944, first_dense=1, shared_inter=2816, norm_topk=False,
                          mla=(0, 512, 128, 64, 128),
                          rope_scaling={"type": "yarn", "factor": 40.0, "original_max_position_embeddings": 4096,
                                        "beta_fast": 32.0, "beta_slow": 1.0, "mscale": 0.707,
                                        "mscale_all_dim": 0.707},
                          max_pos=163840),
}


def model_shape(name: str, **kw) -> ModelShape:
    """A named model shape, optionally with fields replaced (fewer layers or
    experts for quick cases)."""
    return replace(MODEL_SHAPES[name], **kw)


def _name_stream(name: str) -> int:
    import zlib

    return 0x1000000 + zlib.crc32(name.encode())


def build_host_model(shape: ModelShape, seed: int):
    """Every tensor of a random-init model in one host buffer (each on a
    256-byte boundary): returns (config, HostCheckpoint).  Values come from
    the library's seeded generator, one stream per tensor name, and are
    quantised with the reference's quantiser."""
    from .model import HostCheckpoint, HostTensor

    plan = shape.plan()
    offs, off = [], 0
    for name, dt, sh, fill in plan:
        rows = int(np.prod(sh[:-1])) if len(sh) > 1 else 1
        offs.append(off)
        off = _align(off + rows * row_bytes(dt, sh[-1]))
    buf = np.empty(max(off, 256), dtype=np.uint8)
    ck = HostCheckpoint(buf)
    for (name, dt, sh, fill), o in zip(plan, offs):
        rows = int(np.prod(sh[:-1])) if len(sh) > 1 else 1
        n = rows * row_bytes(dt, sh[-1])
        dst = buf[o:o + n]
        if fill == "ones":
            dst.view(np.float32)[:] = 1.0
        elif fill == "router":
            L.check(L.lib().moe_synth_normal(seed, _name_stream(name), rows * sh[-1], 0.0, shape.weight_std,
                                             dst.ctypes.data_as(C.c_void_p)), "moe_synth_normal")
        else:
            _fill(dst, seed, _name_stream(name), dt, rows, sh[-1], 0.0, shape.weight_std)
        ck.add(name, HostTensor(dt, tuple(sh), dst), o)
    return shape.config(), ck


def prompt_ids(seed: int, n: int, vocab: int) -> list:
    """n token ids uniform in [0, vocab) (numpy's PCG64 seeded with `seed`)."""
    return [int(v) for v in np.random.default_rng(seed).integers(0, vocab, n)]
