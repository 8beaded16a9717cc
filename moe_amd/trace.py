"""Routing traces as JSONL files, and the counts read back from them.

`write_trace` writes what the reference's `moe run --trace PATH` writes
(`write_trace`, src/main.rs:771-799): a header object naming the model, its
layer and expert counts and its top-k, then one object per (token, routed
layer) with the experts chosen, strongest first, and the weights applied.
Objects are written as serde_json's compact writer writes a `json!` value:
keys in sorted order (the default map is a BTreeMap), no spaces, weights (f32)
widened to f64 and printed as the shortest digits that read back to the same
f64, in the notation the Rust float writers use (`1.0`, `0.00001`, `1e-6`,
`1.5e-7`, `1e16`).  Readers parse numbers, so the notation carries no meaning.

`Counts` mirrors `moe::Counts` (src/route.rs:28-177): selections per
(layer, expert) from an in-memory trace or from a JSONL file, and the
statistics the reference prints from them, computed in f32 as the reference
computes them (`logf` from the C library, which Rust's `f32::ln` calls).
"""
from __future__ import annotations

import ctypes
import ctypes.util
import json
import math
from dataclasses import dataclass, field
from typing import Iterable, Optional, Sequence

import numpy as np

f32 = np.float32


def _f64_text(v: float) -> str:
    """A finite f64 as the Rust float writers print it: the shortest
    round-trip digits D with value D * 10^k, placed by the decimal exponent
    kk = len(D) + k (10^(kk-1) <= |v| < 10^kk)."""
    if not math.isfinite(v):
        return "null"  # serde_json writes a non-finite float as null
    if v == 0.0:
        return "-0.0" if math.copysign(1.0, v) < 0 else "0.0"
    sign = "-" if v < 0 else ""
    mant, _, e = repr(abs(v)).partition("e")
    ip, _, fp = mant.partition(".")
    digits = (ip + fp).lstrip("0")
    k = (int(e) if e else 0) - len(fp)
    stripped = digits.rstrip("0")
    k += len(digits) - len(stripped)
    digits = stripped
    n = len(digits)
    kk = n + k
    if 0 <= k and kk <= 16:
        body = digits + "0" * (kk - n) + ".0"
    elif 0 < kk <= 16:
        body = digits[:kk] + "." + digits[kk:]
    elif -5 < kk <= 0:
        body = "0." + "0" * (-kk) + digits
    elif n == 1:
        body = digits + "e" + str(kk - 1)
    else:
        body = digits[0] + "." + digits[1:] + "e" + str(kk - 1)
    return sign + body


def _json_value(v) -> str:
    """One value as serde_json's compact writer prints it."""
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, (int, np.integer)):
        return str(int(v))
    if isinstance(v, (float, np.floating)):
        return _f64_text(float(v))
    if isinstance(v, str):
        # serde_json escapes '"', '\\' and the C0 controls only (short forms
        # for \b \t \n \f \r, lowercase \u00xx for the rest), as does
        # json.dumps with ensure_ascii off.
        return json.dumps(v, ensure_ascii=False)
    if isinstance(v, dict):
        return "{" + ",".join(json.dumps(str(key)) + ":" + _json_value(v[key]) for key in sorted(v)) + "}"
    if isinstance(v, (list, tuple)):
        return "[" + ",".join(_json_value(x) for x in v) + "]"
    raise TypeError(f"no JSON form for {type(v).__name__}")


def header_line(model: str, layers: int, experts: int, top_k: int) -> str:
    return _json_value({"model": model, "layers": int(layers), "experts": int(experts), "top_k": int(top_k)})


def route_line(route, tokens: Optional[Sequence[int]] = None, texts: Optional[Sequence[str]] = None) -> str:
    """One route: token is the id at route.pos when `tokens` covers it, text
    its decoded form when `texts` (one string per token id position) is
    given (src/main.rs:788-796)."""
    tok = int(tokens[route.pos]) if tokens is not None and route.pos < len(tokens) else None
    text = texts[route.pos] if (texts is not None and tok is not None) else None
    # The weight goes out as the f32 the layer applied, widened to f64.
    ex = [[int(e), float(f32(w))] for (e, w) in route.experts]
    return _json_value({"pos": int(route.pos), "layer": int(route.layer), "token": tok, "text": text, "experts": ex})


def write_trace(path: str, routes: Iterable, model: str, layers: int, experts: int, top_k: int,
                tokens: Optional[Sequence[int]] = None, texts: Optional[Sequence[str]] = None) -> int:
    """Write a trace file; returns the number of routes written."""
    n = 0
    with open(path, "w", encoding="utf-8", newline="\n") as f:
        f.write(header_line(model, layers, experts, top_k) + "\n")
        for r in routes:
            f.write(route_line(r, tokens, texts) + "\n")
            n += 1
    return n


# ------------------------------------------------------------------ counts

_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]


def _lnf(x) -> np.float32:
    return f32(_libm.logf(float(x)))


def _u32(v) -> Optional[int]:
    """serde_json's as_u64 narrowed as the reference narrows it (`as u32`):
    non-negative integers only."""
    if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v >= 1 << 64:
        return None
    return v


@dataclass
class Counts:
    """Selections per (layer, expert) (src/route.rs:28-37)."""

    model: str = ""
    experts: int = 0
    top_k: int = 0
    tokens: int = 0
    counts: dict = field(default_factory=dict)

    @staticmethod
    def from_trace(routes: Iterable, model: str, experts: int, top_k: int) -> "Counts":
        """src/route.rs:42-56."""
        c = Counts(model=model, experts=experts, top_k=top_k)
        positions = set()
        for r in routes:
            positions.add(int(r.pos))
            for (e, _) in r.experts:
                key = (int(r.layer), int(e))
                c.counts[key] = c.counts.get(key, 0) + 1
        c.tokens = len(positions)
        return c

    @staticmethod
    def read(path: str) -> "Counts":
        """A JSONL trace, header line included (src/route.rs:58-90): blank
        and unparsable lines are skipped, an object without "pos" is the
        header, missing numbers read as 0."""
        c = Counts()
        positions = set()
        with open(path, encoding="utf-8") as f:
            for line in f:
                if not line.strip():
                    continue
                try:
                    v = json.loads(line)
                except ValueError:
                    continue
                get = v.get if isinstance(v, dict) else (lambda key, d=None: d)
                # A "pos" key holding null still marks a route line.
                if not (isinstance(v, dict) and "pos" in v):
                    m = get("model")
                    c.model = m if isinstance(m, str) else ""
                    c.experts = _u32(get("experts")) or 0
                    c.top_k = _u32(get("top_k")) or 0
                    continue
                pos = (_u32(get("pos")) or 0) & 0xFFFFFFFF
                layer = (_u32(get("layer")) or 0) & 0xFFFFFFFF
                positions.add(pos)
                pairs = get("experts")
                for pair in pairs if isinstance(pairs, list) else []:
                    e = _u32(pair[0]) if isinstance(pair, list) and pair else None
                    if e is not None:
                        key = (layer, e & 0xFFFFFFFF)
                        c.counts[key] = c.counts.get(key, 0) + 1
        c.tokens = len(positions)
        if c.experts == 0:
            c.experts = max((e + 1 for (_, e) in c.counts), default=0)
        return c

    def is_empty(self) -> bool:
        return not self.counts

    def layers(self) -> list:
        return sorted({l for (l, _) in self.counts})

    def count(self, layer: int, expert: int) -> int:
        return self.counts.get((layer, expert), 0)

    def share(self, layer: int, expert: int) -> np.float32:
        return f32(self.count(layer, expert)) / f32(max(self.tokens, 1))

    def _layer_counts(self, layer: int) -> list:
        return [self.count(layer, e) for e in range(self.experts)]

    def entropy(self, layer: int) -> np.float32:
        """Normalised routing entropy (src/route.rs:112-131): the f32 sum
        folds from -0.0 in expert order."""
        c = self._layer_counts(layer)
        total = sum(c)
        if total == 0 or self.experts < 2:
            return f32(0.0)
        h = f32(-0.0)
        for n in c:
            if n > 0:
                p = f32(n) / f32(total)
                h = f32(h + f32(-p * _lnf(p)))
        return f32(h / _lnf(f32(self.experts)))

    def peak_ratio(self, layer: int) -> np.float32:
        """src/route.rs:135-144."""
        c = self._layer_counts(layer)
        total = sum(c)
        if total == 0:
            return f32(0.0)
        return f32(f32(max(c)) * f32(self.experts)) / f32(total)

    def dead(self, layer: int) -> int:
        return sum(1 for n in self._layer_counts(layer) if n == 0)

    def coverage(self) -> np.float32:
        """src/route.rs:151-160."""
        nl = len(self.layers())
        if nl == 0 or self.experts == 0:
            return f32(0.0)
        return f32(sum(1 for n in self.counts.values() if n > 0)) / f32(nl * self.experts)

    def hottest(self) -> list:
        """Every (layer, expert) touched, busiest first, then by key
        (src/route.rs:167-171)."""
        items = [(k, n) for k, n in self.counts.items() if n > 0]
        items.sort(key=lambda kv: (-kv[1], kv[0]))
        return [k for k, _ in items]
