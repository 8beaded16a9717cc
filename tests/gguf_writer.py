"""A minimal GGUF v3 writer for tests (the reference builds its test files the
same way: bytes in memory, src/gguf.rs tests `Builder`).

Layout: "GGUF", u32 version, u64 tensor count, u64 metadata count, the
metadata key/values, the tensor infos (name, dims fastest-first, ggml type,
offset relative to the data section), padding to `general.alignment`, data.
"""
from __future__ import annotations

import struct

T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64 = 4, 5, 6, 7, 8, 9, 10


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    def __init__(self, alignment: int = 32):
        self.meta: list[bytes] = []
        self.infos: list[tuple[str, list[int], int, bytes]] = []
        self.alignment = alignment
        if alignment != 32:
            self.kv_u32("general.alignment", alignment)

    def kv_str(self, key: str, v: str):
        self.meta.append(_str(key) + struct.pack("<I", T_STR) + _str(v))
        return self

    def kv_u32(self, key: str, v: int):
        self.meta.append(_str(key) + struct.pack("<II", T_U32, v))
        return self

    def kv_f32(self, key: str, v: float):
        self.meta.append(_str(key) + struct.pack("<If", T_F32, v))
        return self

    def kv_bool(self, key: str, v: bool):
        self.meta.append(_str(key) + struct.pack("<IB", T_BOOL, 1 if v else 0))
        return self

    def kv_strs(self, key: str, vs: list[str]):
        self.meta.append(_str(key) + struct.pack("<IIQ", T_ARR, T_STR, len(vs)) + b"".join(_str(v) for v in vs))
        return self

    def kv_i32s(self, key: str, vs: list[int]):
        self.meta.append(_str(key) + struct.pack("<IIQ", T_ARR, T_I32, len(vs)) + struct.pack(f"<{len(vs)}i", *vs))
        return self

    def tensor(self, name: str, shape_outer_first: list[int], ggml_type: int, data: bytes):
        """shape as the engine sees it (outermost first); stored reversed."""
        self.infos.append((name, list(reversed(shape_outer_first)), ggml_type, bytes(data)))
        return self

    def build(self) -> bytes:
        head = b"GGUF" + struct.pack("<IQQ", 3, len(self.infos), len(self.meta)) + b"".join(self.meta)
        data, offs = b"", []
        for _, _, _, d in self.infos:
            pad = (-len(data)) % self.alignment
            data += b"\0" * pad
            offs.append(len(data))
            data += d
        for (name, dims, t, _), off in zip(self.infos, offs):
            head += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
            head += struct.pack("<IQ", t, off)
        head += b"\0" * ((-len(head)) % self.alignment)
        return head + data
