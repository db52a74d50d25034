"""GGUF writer for synthetic files (test fixtures, benchmarks).

Writes the layout the engine's reader parses (GgufFile, the reference's
src/io/gguf_reader.cpp:160-241): "GGUF", u32 version, u64 tensor count,
u64 metadata count, metadata (string key, u32 type, value), the tensor
directory (string name, u32 rank, u64 dims, u32 type, u64 offset relative to
the data section), zero padding up to `align_up(end of directory,
alignment)` and the tensor bytes.  Strings are u64 length + bytes, arrays
u32 item type + u64 count + items, bools one byte.

The writer does not validate: tests use it to build malformed files too
(explicit offsets, short tensor data, any type codes).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

# metadata value type codes
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}

# tensor type codes and (elements, bytes) per block
T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 14, 30
BLOCK = {T_F32: (1, 4), T_F16: (1, 2), T_Q8_0: (32, 34), T_Q4_K: (256, 144), T_Q6_K: (256, 210), T_BF16: (1, 2)}


def tensor_nbytes(ttype: int, elements: int) -> int:
    n, b = BLOCK[ttype]
    return (elements + n - 1) // n * b


def align_up(v: int, a: int) -> int:
    """The readers' rounding: a power-of-two mask, none for 0."""
    return v if a == 0 else (v + a - 1) & ~(a - 1)


def _s(x: Union[str, bytes]) -> bytes:
    b = x.encode() if isinstance(x, str) else bytes(x)
    return struct.pack("<Q", len(b)) + b


def _scalar(t: int, v) -> bytes:
    if t == STR:
        return _s(v)
    if t == BOOL:
        return struct.pack("<B", v if isinstance(v, int) and not isinstance(v, bool) else int(bool(v)))
    return struct.pack(_FMT[t], v)


@dataclass
class Meta:
    """One metadata entry: type `t` (an array when `item` is set)."""
    key: Union[str, bytes]
    t: int
    value: object
    item: Optional[int] = None

    def pack(self) -> bytes:
        out = _s(self.key) + struct.pack("<I", self.t)
        if self.t != ARR:
            return out + _scalar(self.t, self.value)
        items = list(self.value)
        out += struct.pack("<I", self.item) + struct.pack("<Q", len(items))
        return out + b"".join(_scalar(self.item, v) for v in items)


def scalar(key, t, value) -> Meta:
    return Meta(key, t, value)


def array(key, item, values) -> Meta:
    return Meta(key, ARR, list(values), item)


@dataclass
class Tensor:
    name: Union[str, bytes]
    dims: Sequence[int]
    ttype: int
    data: bytes = b""
    offset: Optional[int] = None   # relative offset; None = next aligned slot


def build(meta: Iterable[Meta], tensors: Iterable[Tensor], version: int = 3, alignment: int = 32,
          tensor_count: Optional[int] = None, meta_count: Optional[int] = None) -> bytes:
    """The file's bytes.  `alignment` places the data section and the tensors;
    it must equal what the reader derives from the metadata (general.alignment,
    default 32) for the offsets to mean the same thing."""
    meta, tensors = list(meta), list(tensors)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors) if tensor_count is None else tensor_count,
                                 len(meta) if meta_count is None else meta_count)
    body = b"".join(m.pack() for m in meta)
    offsets, cur = [], 0
    for t in tensors:
        off = align_up(cur, alignment) if t.offset is None else t.offset
        offsets.append(off)
        if t.data:   # an entry without bytes (a test's dangling offset) adds none
            cur = max(cur, off + len(t.data))
    directory = b""
    for t, off in zip(tensors, offsets):
        directory += _s(t.name) + struct.pack("<I", len(t.dims)) + b"".join(struct.pack("<Q", d) for d in t.dims)
        directory += struct.pack("<IQ", t.ttype, off)
    pre = head + body + directory
    start = align_up(len(pre), alignment)
    data = bytearray(cur)
    for t, off in zip(tensors, offsets):
        if t.data:
            data[off:off + len(t.data)] = t.data
    return pre + b"\0" * (start - len(pre)) + bytes(data)


def write(path: str, meta: Iterable[Meta], tensors: Iterable[Tensor], **kw) -> int:
    blob = build(meta, tensors, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return len(blob)


def qwen_meta(arch: str = "qwen3", vocab: int = 512, hidden: int = 1024, blocks: int = 2, ff: int = 2048,
              heads: int = 8, kv_heads: int = 4, head_dim: Optional[int] = 128, context: int = 4096,
              eps: float = 1e-6, theta: float = 1e6, alignment: Optional[int] = None) -> List[Meta]:
    """Metadata of a Qwen3-style file (the keys QwenConfig::from_gguf reads)."""
    m = [scalar("general.architecture", STR, arch),
         array("tokenizer.ggml.tokens", STR, [f"t{i}" for i in range(vocab)]),
         scalar(f"{arch}.context_length", U32, context),
         scalar(f"{arch}.embedding_length", U32, hidden),
         scalar(f"{arch}.block_count", U32, blocks),
         scalar(f"{arch}.feed_forward_length", U32, ff),
         scalar(f"{arch}.attention.head_count", U32, heads),
         scalar(f"{arch}.attention.head_count_kv", U32, kv_heads),
         scalar(f"{arch}.attention.layer_norm_rms_epsilon", F32, eps),
         scalar(f"{arch}.rope.freq_base", F32, theta)]
    if head_dim is not None:
        m += [scalar(f"{arch}.attention.key_length", U32, head_dim),
              scalar(f"{arch}.attention.value_length", U32, head_dim)]
    if alignment is not None:
        m.append(scalar("general.alignment", U32, alignment))
    return m


def f32_bytes(a) -> bytes:
    return np.ascontiguousarray(a, dtype="<f4").tobytes()


def f16_bytes(a) -> bytes:
    return np.ascontiguousarray(a, dtype="<u2").tobytes()
