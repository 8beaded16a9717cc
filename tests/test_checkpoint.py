"""Checkpoint containers on the host: the .moe writer and reader round trip,
GGUF tensor infos and names, and malformed files refused rather than read
out of bounds (the reference's tests/malformed.rs and src/gguf.rs tests,
restated against moe_container_open)."""
import ctypes as C
import json
import struct

import numpy as np
import pytest

from gguf_writer import GgufWriter


@pytest.fixture(scope="module")
def lib():
    from moe_amd import _lib as L

    return L.lib()


def parse(lib, data: bytes):
    """(status, recs) of moe_container_open over raw bytes; every rec that
    the parser accepted is checked to lie inside the buffer."""
    from moe_amd import _lib as L

    buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    h = C.c_void_p()
    rc = lib.moe_container_open(buf.ctypes.data_as(C.c_void_p), len(data), C.byref(h))
    if rc != 0:
        return rc, None
    recs = []
    r = L.RecC()
    for i in range(lib.moe_container_count(h)):
        assert lib.moe_container_rec(h, i, C.byref(r)) == 0
        assert r.offset + r.bytes <= len(data), f"{r.name}: accepted past the end"
        recs.append((r.name.decode(errors="replace"), r.dt, r.slabs, r.rows, r.cols, r.offset, r.bytes))
    lib.moe_container_close(h)
    return 0, recs


@pytest.fixture(scope="module")
def tiny_moe(tmp_path_factory):
    """A synthetic routed layer (hidden 512, 8 experts, Q8_0) packed as .moe."""
    from moe_amd import checkpoint, synth

    host = synth.build_host_layer(synth.scaled(synth.SHAPES["tiny_mixtral"], inter=256), 3)
    path = str(tmp_path_factory.mktemp("ckpt") / "tiny.moe")
    tensors = checkpoint.host_layer_tensors(host, layer=2)
    checkpoint.write_moe(path, tensors, config={"model_type": "mixtral", "num_local_experts": 8})
    return host, path, tensors


def test_moe_round_trip(tiny_moe):
    """Names, formats, shapes and bytes read back as written; the payload is
    unpadded (src/store.rs:439-441) and the config survives."""
    from moe_amd import _lib as L
    from moe_amd import checkpoint

    host, path, tensors = tiny_moe
    c = checkpoint.Container(path)
    try:
        assert c.kind == checkpoint.KIND_MOE
        assert c.config() == {"model_type": "mixtral", "num_local_experts": 8}
        assert set(c.recs) == {t[0] for t in tensors}
        offsets = []
        for name, dt, shape, raw in tensors:
            r = c.recs[name]
            assert r["dt"] == dt
            assert [r["slabs"], r["rows"], r["cols"]][-len(shape):] == list(shape) or \
                (len(shape) == 2 and (r["slabs"], r["rows"], r["cols"]) == (1, shape[0], shape[1]))
            assert c.bytes_of(name).tobytes() == raw
            offsets.append((r["offset"], r["bytes"]))
        offsets.sort()
        for (o1, n1), (o2, _) in zip(offsets, offsets[1:]):
            assert o1 + n1 == o2  # back to back
        assert L.DT_Q8_0 in {r["dt"] for r in c.recs.values()}
    finally:
        c.close()


def test_moe_header_names_are_the_references(tiny_moe):
    """The header is the reference's: {config, tokenizer, chat_template,
    tensors: {name: {dt: "Q8"/"F32", shape, off, len}}}."""
    _, path, _ = tiny_moe
    raw = open(path, "rb").read()
    assert raw[:4] == b"MOEF" and struct.unpack("<I", raw[4:8])[0] == 1
    hlen = struct.unpack("<Q", raw[8:16])[0]
    head = json.loads(raw[16:16 + hlen])
    assert set(head) == {"config", "tokenizer", "chat_template", "tensors"}
    dts = {v["dt"] for v in head["tensors"].values()}
    assert dts <= {"F32", "Q8"} and "Q8" in dts
    stack = head["tensors"]["model.layers.2.mlp.experts.gate_proj"]
    assert stack["shape"] == [8, 256, 512]


def _gguf(alignment=64):
    from moe_amd import _lib as L

    E, H, I = 4, 64, 32
    rng = np.random.default_rng(0)
    router = rng.standard_normal((E, H)).astype(np.float32)
    q4 = rng.integers(0, 256, E * I * (H // 32) * 18, dtype=np.uint8)
    w = GgufWriter(alignment)
    w.kv_str("general.architecture", "qwen2moe").kv_strs("tokenizer.ggml.tokens", ["a", "bb", "ccc"])
    w.kv_f32("qwen2moe.rope.freq_base", 1e6).kv_bool("general.flag", True).kv_i32s("some.ints", [1, 2, 3])
    w.tensor("blk.0.ffn_gate_inp.weight", [E, H], L.DT_F32, router.tobytes())
    w.tensor("blk.0.ffn_gate_exps.weight", [E, I, H], L.DT_Q4_0, q4.tobytes())
    w.tensor("rope_freqs.weight", [8], L.DT_F32, np.zeros(8, np.float32).tobytes())
    return w.build(), router, q4


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_tensor_infos(lib, alignment):
    """Dimensions come back outermost first, offsets land on the data
    section (general.alignment, default 32), and the bytes are the ones
    written."""
    from moe_amd import _lib as L

    data, router, q4 = _gguf(alignment)
    rc, recs = parse(lib, data)
    assert rc == 0
    by = {r[0]: r for r in recs}
    _, dt, slabs, rows, cols, off, n = by["blk.0.ffn_gate_inp.weight"]
    assert (dt, slabs, rows, cols) == (L.DT_F32, 1, 4, 64) and off % alignment == 0
    assert data[off:off + n] == router.tobytes()
    _, dt, slabs, rows, cols, off, n = by["blk.0.ffn_gate_exps.weight"]
    assert (dt, slabs, rows, cols) == (L.DT_Q4_0, 4, 32, 64)
    assert data[off:off + n] == q4.tobytes()
    assert by["rope_freqs.weight"][2:5] == (1, 1, 8)


def test_gguf_names_map_onto_the_engines_own():
    """gguf::rename's own test (src/gguf.rs:740-768)."""
    from moe_amd.checkpoint import gguf_rename

    for src, dst in [
        ("token_embd.weight", "model.embed_tokens.weight"),
        ("output.weight", "lm_head.weight"),
        ("output_norm.weight", "model.norm.weight"),
        ("blk.0.attn_norm.weight", "model.layers.0.input_layernorm.weight"),
        ("blk.7.attn_q.weight", "model.layers.7.self_attn.q_proj.weight"),
        ("blk.7.attn_q_norm.weight", "model.layers.7.self_attn.q_norm.weight"),
        ("blk.7.attn_output.weight", "model.layers.7.self_attn.o_proj.weight"),
        ("blk.1.ffn_norm.weight", "model.layers.1.post_attention_layernorm.weight"),
        ("blk.1.ffn_gate_inp.weight", "model.layers.1.mlp.gate.weight"),
        ("blk.1.ffn_gate_exps.weight", "model.layers.1.mlp.experts.gate_proj"),
        ("blk.1.ffn_down_exps.weight", "model.layers.1.mlp.experts.down_proj"),
        ("blk.1.ffn_down.weight", "model.layers.1.mlp.down_proj.weight"),
        ("blk.1.ffn_gate_shexp.weight", "model.layers.1.mlp.shared_expert.gate_proj.weight"),
        ("blk.1.ffn_gate_inp_shexp.weight", "model.layers.1.mlp.shared_expert_gate.weight"),
        ("blk.3.exp_probs_b.bias", "model.layers.3.mlp.gate.e_score_correction_bias"),
    ]:
        assert gguf_rename(src) == dst, src
    for src in ("rope_freqs.weight", "blk.0.something_else.weight", "blk.x.attn_q.weight", "blk."):
        assert gguf_rename(src) is None, src


class Rand:
    """splitmix64 byte source (tests/malformed.rs:16-45)."""

    def __init__(self, seed):
        self.s = seed

    def next(self):
        self.s = (self.s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def bytes(self, n):
        return bytes((self.next() >> 24) & 0xFF for _ in range(n))

    def mutate(self, src):
        out = bytearray(src)
        if out:
            out[self.next() % len(out)] = (self.next() >> 24) & 0xFF
        return bytes(out)


def test_arbitrary_bytes_are_refused_or_bounded(lib):
    """Noise, and noise behind each magic, never reads outside the buffer
    (tests/malformed.rs:88-105)."""
    r = Rand(0xC0FFEE)
    for n in (0, 1, 4, 8, 16, 17, 64, 300):
        for _ in range(40):
            for head in (b"", b"MOEF", b"GGUF"):
                parse(lib, head + r.bytes(n))


def test_corrupted_packed_model_is_refused_not_trusted(lib, tiny_moe):
    """Single-byte corruptions, every truncation of the header and the
    extreme header lengths (tests/malformed.rs:107-133): an error or a
    bounded index, never a read past the end."""
    _, path, _ = tiny_moe
    whole = open(path, "rb").read()
    assert parse(lib, whole)[0] == 0
    hlen = struct.unpack("<Q", whole[8:16])[0]
    r = Rand(7)
    head = whole[:16 + hlen + 64]
    for _ in range(400):
        parse(lib, r.mutate(head) + whole[len(head):])
    for cut in range(min(len(whole), 16 + hlen + 64)):
        rc, _ = parse(lib, whole[:cut])
        assert rc != 0 or cut >= 16 + hlen
    for bad_len in (0, 1, 15, 2**64 - 1, 2**64 - 17, 1 << 40, 1 << 62):
        bad = whole[:8] + struct.pack("<Q", bad_len) + whole[16:]
        parse(lib, bad)


def test_truncated_or_corrupted_gguf_is_refused(lib):
    """Every truncation of a GGUF and single-byte corruptions of its header
    (src/gguf.rs malformed_headers_are_refused)."""
    data, _, _ = _gguf()
    assert parse(lib, data)[0] == 0
    data_start = min(r[5] for r in parse(lib, data)[1])
    for cut in range(len(data)):
        rc, _ = parse(lib, data[:cut])
        if cut < data_start:
            assert rc != 0, cut
    r = Rand(11)
    for _ in range(400):
        parse(lib, r.mutate(data[:data_start]) + data[data_start:])


def _moe_with(entries: dict, payload: bytes) -> bytes:
    header = json.dumps({"config": {}, "tensors": entries}, separators=(",", ":")).encode()
    return b"MOEF" + struct.pack("<IQ", 1, len(header)) + header + payload


@pytest.mark.parametrize("dt,shape", [
    ("F32", [2**63 + 2**32 + 1, 2**63 - 2**32 + 1, 1]),   # slabs * rows * 4 wraps past 2^128 to 4 bytes
    ("F32", [1, 2**62]),                                 # cols * 4 wraps to 0 in 64 bits
    ("F32", [2**62, 2**62, 4]),
    ("Q8", [3, 2**61, 2**60]),
    ("F16", [1, 2**63]),
])
def test_wrapping_shapes_are_refused(lib, dt, shape):
    """Header shapes whose byte size overflows 64 bits (or 128) are
    refused: every size multiply saturates, as the reference's Rec::len does
    (src/store.rs:36-43), so no wrapped small size can pass the bounds check."""
    data = _moe_with({"w": {"dt": dt, "shape": shape, "off": 0, "len": 4}}, b"\0" * 64)
    rc, recs = parse(lib, data)
    assert rc != 0, f"accepted {shape} as {recs}"


def test_gguf_four_dimension_product_saturates(lib):
    """A 4-D GGUF tensor whose outer dimensions multiply past 2^64 is refused
    (the slab count saturates instead of wrapping)."""
    from moe_amd import _lib as L

    w = GgufWriter(32)
    w.tensor("x.weight", [2**40, 2**40, 1, 64], L.DT_F32, b"\0" * 256)
    data = w.build()
    rc, recs = parse(lib, data)
    assert rc != 0, f"accepted {recs}"
