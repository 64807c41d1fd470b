"""Minimal GGUF v3 writer for tests (the byte layout src/gguf/reader.rs
reads: header, typed key/values, tensor infos in ne order, 32-byte aligned
data).  Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR = 4, 5, 6, 7, 8, 9
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    def __init__(self, version: int = 3, magic: bytes = b"GGUF"):
        self.version = version
        self.magic = magic
        self.kv: list[bytes] = []
        self.tensors: list[tuple[str, list[int], int, bytes]] = []

    def u32(self, k: str, v: int):
        self.kv.append(_str(k) + struct.pack("<II", T_U32, v))

    def i32(self, k: str, v: int):
        self.kv.append(_str(k) + struct.pack("<Ii", T_I32, v))

    def f32(self, k: str, v: float):
        self.kv.append(_str(k) + struct.pack("<If", T_F32, v))

    def boolean(self, k: str, v: bool):
        self.kv.append(_str(k) + struct.pack("<IB", T_BOOL, 1 if v else 0))

    def str(self, k: str, v: str):
        self.kv.append(_str(k) + struct.pack("<I", T_STR) + _str(v))

    def arr_str(self, k: str, vs):
        body = b"".join(_str(s) for s in vs)
        self.kv.append(_str(k) + struct.pack("<IIQ", T_ARR, T_STR, len(vs)) + body)

    def arr_i32(self, k: str, vs):
        body = b"".join(struct.pack("<i", v) for v in vs)
        self.kv.append(_str(k) + struct.pack("<IIQ", T_ARR, T_I32, len(vs)) + body)

    def tensor(self, name: str, dims_ne, data, ggml_type: int = 0):
        """dims in ne order ([cols, rows]); data: float32 array (F32) or the
        raw block bytes of a quantized type."""
        raw = np.ascontiguousarray(data, np.float32).tobytes() if ggml_type == 0 else bytes(data)
        self.tensors.append((name, [int(d) for d in dims_ne], ggml_type, raw))

    def finish(self) -> bytes:
        out = bytearray(self.magic + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv)))
        for kv in self.kv:
            out += kv
        off = 0
        offsets = []
        for _, _, _, raw in self.tensors:
            offsets.append(off)
            off = (off + len(raw) + ALIGN - 1) // ALIGN * ALIGN
        for (name, dims, t, _), o in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", t, o)
        out += b"\0" * ((-len(out)) % ALIGN)
        start = len(out)
        for (_, _, _, raw), o in zip(self.tensors, offsets):
            out += b"\0" * (start + o - len(out))
            out += raw
        return bytes(out)


def llama_meta(g: GgufWriter, *, ctx: int, embd: int, n_layer: int, ff: int, n_head: int, n_head_kv: int,
               vocab: int, eps: float = 1e-5, theta: float = 10000.0, rope_dim: int | None = None):
    g.str("general.architecture", "llama")
    g.u32("llama.context_length", ctx)
    g.u32("llama.embedding_length", embd)
    g.u32("llama.block_count", n_layer)
    g.u32("llama.feed_forward_length", ff)
    g.u32("llama.attention.head_count", n_head)
    g.u32("llama.attention.head_count_kv", n_head_kv)
    g.f32("llama.attention.layer_norm_rms_epsilon", eps)
    g.u32("llama.rope.dimension_count", rope_dim if rope_dim is not None else embd // n_head)
    g.f32("llama.rope.freq_base", theta)
    toks = ["<unk>"] + [f"t{i}" for i in range(1, vocab)]
    g.arr_str("tokenizer.ggml.tokens", toks)
    g.arr_str("tokenizer.ggml.merges", [])
    g.u32("tokenizer.ggml.unknown_token_id", 0)
    g.u32("tokenizer.ggml.bos_token_id", 0)
    g.u32("tokenizer.ggml.eos_token_id", 0)
