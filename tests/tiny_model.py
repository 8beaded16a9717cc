"""A tiny decoder forward in numpy, for the reference's golden fixtures.

Test scaffolding: everything around the routed layer (embedding, RMSNorm,
GQA/MLA attention with RoPE/YaRN and sliding windows, the dense MLP, the
head) is computed here in float64 from the model definitions the fixtures
were generated from (the reference's forward is src/model.rs:646-834; rope
scaling src/spec.rs:89-160; windows src/spec.rs:422-444).  The routed layer
itself is a callback, so the same forward checks the CPU oracle and the GPU
kernels against the fixtures' expected logits.

`quant_dt` applies the reference's pack rule (src/store.rs:418-429): every
"big" weight with a block-divisible width is stored in that format (norms,
biases, routers and the correction bias stay F32), and the non-MoE parts then
read the dequantised values.
"""
from __future__ import annotations

import json
import math
from pathlib import Path
from typing import Callable, Optional

import numpy as np
from safetensors.numpy import load_file

FIXTURES = Path(__file__).resolve().parent / "golden" / "fixtures"


def is_big_weight(name: str) -> bool:
    """src/store.rs:791-793."""
    return not ("norm" in name or name.endswith(".bias") or name.endswith("gate.weight") or "e_score" in name)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    s = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * s * w


def inv_freqs(cfg: dict, dim: int) -> np.ndarray:
    theta = cfg.get("rope_theta", 10000.0)
    base = np.array([theta ** (-2.0 * i / dim) for i in range(dim // 2)])
    sc = cfg.get("rope_scaling") or {}
    kind = sc.get("rope_type", sc.get("type", ""))
    s = sc.get("factor", 1.0)
    if s <= 1.0 or not kind:
        return base
    assert kind == "yarn", kind  # the only scaling the fixtures use
    ctx = sc.get("original_max_position_embeddings", cfg["max_position_embeddings"])
    bf, bs = sc.get("beta_fast", 32.0), sc.get("beta_slow", 1.0)
    ln_base = math.log(theta)

    def bound(b):
        return dim * math.log(ctx / (b * 2 * math.pi)) / (2 * ln_base)

    low, high = math.floor(bound(bf)), math.ceil(bound(bs))
    span = max(high - low, 1e-3)
    ramp = np.clip((np.arange(dim // 2) - low) / span, 0.0, 1.0)
    return (1 - ramp) * (base / s) + ramp * base


def attn_scale(cfg: dict) -> float:
    sc = cfg.get("rope_scaling") or {}
    if sc.get("rope_type", sc.get("type", "")) != "yarn" or sc.get("factor", 1.0) <= 1.0:
        return 1.0
    return 0.1 * math.log(sc["factor"]) + 1.0


def windows(cfg: dict, layers: int) -> list:
    w = cfg.get("sliding_window") or 0
    if not w:
        return [None] * layers
    types = cfg.get("layer_types") or []
    return [w if (l < len(types) and types[l] in ("sliding_attention", "local_attention")) else None
            for l in range(layers)]


def rope(x: np.ndarray, pos: np.ndarray, inv: np.ndarray) -> np.ndarray:
    """Half-split rotary embedding; x [..., t, d] with positions pos [t]."""
    half = x.shape[-1] // 2
    ang = pos[:, None] * inv[None, :half]
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half], x[..., half:2 * half]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)


class TinyModel:
    def __init__(self, name: str, quant_dt: Optional[int] = None):
        d = FIXTURES / name
        self.name = name
        self.cfg = json.loads((d / "config.json").read_text())
        exp = json.loads((d / "expected.json").read_text())
        self.tokens = exp["tokens"]
        self.expected = np.array(exp["logits"], dtype=np.float64)
        self.raw = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in load_file(str(d / "model.safetensors")).items()}
        self.quant_dt = quant_dt
        self.packed = {}   # name -> (dt, rows, cols, bytes) of every tensor the pack rule quantises
        self.w = {}
        for k, v in self.raw.items():
            self.w[k] = v.astype(np.float64)
            if quant_dt is not None and v.ndim == 2 and v.shape[0] > 1 and is_big_weight(k) and v.shape[1] % 32 == 0:
                from oracle import pyoracle as O

                q = O.quantize(quant_dt, v)
                self.packed[k] = (quant_dt, v.shape[0], v.shape[1], q)
                self.w[k] = O.dequant(quant_dt, q, v.shape[0], v.shape[1]).astype(np.float64)
        c = self.cfg
        self.layers = c["num_hidden_layers"]
        self.mla = "kv_lora_rank" in c
        self.n_experts = c.get("num_experts", c.get("n_routed_experts", 0))

    # ------------------------------------------------------------------ MoE
    def is_moe(self, l: int) -> bool:
        return f"model.layers.{l}.mlp.gate.weight" in self.w

    def moe_tensors(self, l: int):
        """The routed layer's weights as (dt, rows, cols, bytes) records (F32
        unless the pack rule quantised them) plus router/bias/shared."""
        p = f"model.layers.{l}.mlp."

        def rec(name):
            if name in self.packed:
                return self.packed[name]
            v = self.raw[name]
            return (0, v.shape[0], v.shape[1], v.view(np.uint8).reshape(-1))

        experts = [[rec(f"{p}experts.{e}.{m}_proj.weight") for m in ("gate", "up", "down")]
                   for e in range(self.n_experts)]
        shared = None
        if f"{p}shared_experts.gate_proj.weight" in self.raw:
            shared = [rec(f"{p}shared_experts.{m}_proj.weight") for m in ("gate", "up", "down")]
        return dict(router=self.raw[f"{p}gate.weight"], e_bias=self.raw.get(f"{p}gate.e_score_correction_bias"),
                    experts=experts, shared=shared)

    def routing_spec(self) -> dict:
        c = self.cfg
        return dict(top_k=c.get("num_experts_per_tok", 2), norm_topk=c.get("norm_topk_prob", True),
                    sigmoid=c.get("scoring_func") == "sigmoid" or any("e_score" in k for k in self.raw),
                    routed_scale=c.get("routed_scaling_factor", 1.0), n_group=c.get("n_group", 1),
                    topk_group=c.get("topk_group", 1))

    # -------------------------------------------------------------- forward
    def _attention(self, l: int, n: np.ndarray, pos: np.ndarray, win) -> np.ndarray:
        c, w = self.cfg, self.w
        p = f"model.layers.{l}.self_attn."
        nh = c["num_attention_heads"]
        t = n.shape[0]
        if self.mla:
            qk_n, qk_r, vh, kvl = c["qk_nope_head_dim"], c["qk_rope_head_dim"], c["v_head_dim"], c["kv_lora_rank"]
            inv = inv_freqs(c, qk_r)
            cq = rmsnorm(n @ w[p + "q_a_proj.weight"].T, w[p + "q_a_layernorm.weight"], c["rms_norm_eps"])
            q = (cq @ w[p + "q_b_proj.weight"].T).reshape(t, nh, qk_n + qk_r).transpose(1, 0, 2)
            ca = n @ w[p + "kv_a_proj_with_mqa.weight"].T
            ckv = rmsnorm(ca[:, :kvl], w[p + "kv_a_layernorm.weight"], c["rms_norm_eps"])
            kpe = rope(ca[:, kvl:], pos, inv)
            kv = (ckv @ w[p + "kv_b_proj.weight"].T).reshape(t, nh, qk_n + vh).transpose(1, 0, 2)
            q = np.concatenate([q[..., :qk_n], rope(q[..., qk_n:], pos, inv)], axis=-1)
            k = np.concatenate([kv[..., :qk_n], np.broadcast_to(kpe, (nh, t, qk_r))], axis=-1)
            v = kv[..., qk_n:]
            qd, rep = qk_n + qk_r, 1
        else:
            hd, nkv = c["head_dim"], c["num_key_value_heads"]
            inv = inv_freqs(c, hd)
            q, k, v = (n @ w[p + f"{m}_proj.weight"].T for m in "qkv")
            for nm, arr_name in (("q_norm", "q"), ("k_norm", "k")):
                key = p + nm + ".weight"
                arr = q if arr_name == "q" else k
                if key in w:
                    g = w[key]
                    if g.shape[0] == arr.shape[1]:
                        arr = rmsnorm(arr, g, c["rms_norm_eps"])
                    else:
                        heads = arr.shape[1] // hd
                        arr = rmsnorm(arr.reshape(t, heads, hd), g, c["rms_norm_eps"]).reshape(t, heads * hd)
                if arr_name == "q":
                    q = arr
                else:
                    k = arr
            q = rope(q.reshape(t, nh, hd).transpose(1, 0, 2), pos, inv)
            k = rope(k.reshape(t, nkv, hd).transpose(1, 0, 2), pos, inv)
            v = v.reshape(t, nkv, hd).transpose(1, 0, 2)
            qd, rep = hd, nh // nkv
        scale = attn_scale(c) / math.sqrt(qd)
        out = np.zeros((t, nh, v.shape[-1]))
        for h in range(nh):
            kh = h // rep
            s = (q[h] @ k[kh].T) * scale
            mask = np.tril(np.ones((t, t), dtype=bool))
            if win:
                mask &= (np.arange(t)[None, :] > np.arange(t)[:, None] - win)
            s = np.where(mask, s, -np.inf)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            s /= s.sum(axis=1, keepdims=True)
            out[:, h] = s @ v[kh]
        return out.reshape(t, -1) @ w[p + "o_proj.weight"].T

    def forward(self, moe_fn: Callable[[int, np.ndarray], np.ndarray], tokens=None) -> np.ndarray:
        """Logits at every position for `tokens` (default: the fixture's),
        computed as one causal batch; `moe_fn(layer, x_norm_f32)` returns the
        routed layer's output for the layer."""
        c, w = self.cfg, self.w
        tokens = self.tokens if tokens is None else tokens
        t = len(tokens)
        pos = np.arange(t, dtype=np.float64)
        wins = windows(c, self.layers)
        x = w["model.embed_tokens.weight"][np.array(tokens) % c["vocab_size"]]
        eps = c["rms_norm_eps"]
        for l in range(self.layers):
            p = f"model.layers.{l}."
            n = rmsnorm(x, w[p + "input_layernorm.weight"], eps)
            x = x + self._attention(l, n, pos, wins[l])
            n = rmsnorm(x, w[p + "post_attention_layernorm.weight"], eps)
            if self.is_moe(l):
                delta = np.asarray(moe_fn(l, n.astype(np.float32)), dtype=np.float64)
            else:
                g = n @ w[p + "mlp.gate_proj.weight"].T
                u = n @ w[p + "mlp.up_proj.weight"].T
                delta = ((g / (1 + np.exp(-g))) * u) @ w[p + "mlp.down_proj.weight"].T
            x = x + delta
        nx = rmsnorm(x, w["model.norm.weight"], eps)
        return nx @ w["lm_head.weight"].T


def oracle_moe_fn(model: TinyModel, routing=None):
    """The routed layer computed by the CPU oracle, for TinyModel.forward."""
    from oracle import pyoracle as O

    spec = model.routing_spec()
    layers = {}

    def fn(l: int, xn: np.ndarray) -> np.ndarray:
        if l not in layers:
            mt = model.moe_tensors(l)
            layers[l] = O.OracleLayer(xn.shape[1], model.n_experts, spec["top_k"], mt["router"], mt["experts"],
                                      sigmoid=spec["sigmoid"], norm_topk=spec["norm_topk"],
                                      routed_scale=spec["routed_scale"], n_group=spec["n_group"],
                                      topk_group=spec["topk_group"], e_bias=mt["e_bias"], shared=mt["shared"])
        out, *_ = layers[l].forward(xn, routing)
        return out

    return fn


def host_tensors(name: str, quant_dt: Optional[int] = None):
    """A fixture as the whole-model paths load it: (Spec, {name: HostTensor}),
    every tensor F32 unless the pack rule (src/store.rs:418-429) stored it in
    `quant_dt`."""
    from moe_amd.model import HostTensor, Spec

    m = TinyModel(name, quant_dt=quant_dt)
    out = {}
    for k, v in m.raw.items():
        if k in m.packed:
            dt, rows, cols, q = m.packed[k]
            out[k] = HostTensor(dt, v.shape, np.ascontiguousarray(q).view(np.uint8).reshape(-1))
        else:
            out[k] = HostTensor(0, v.shape, np.ascontiguousarray(v).view(np.uint8).reshape(-1))
    spec = Spec.derive(m.cfg, {k: t.shape for k, t in out.items()})
    return m, spec, out
