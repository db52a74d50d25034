"""CPU restatement of the reference's GGUF reader and QwenConfig::from_gguf.

TEST INFRASTRUCTURE ONLY: tests/ use it as the checker for the engine's
GgufFile / QwenConfig::from_gguf; nothing in the product imports it.

Follows, step by step:
  src/io/gguf_reader.cpp:160-241   GgufFile::load (header, metadata, tensor
                                   directory, data offset)
  src/io/gguf_reader.cpp:12-112    read_pod / read_string / read_array /
                                   read_scalar / read_array_value / read_value
  src/io/gguf_reader.cpp:115-120   align_to (power-of-two mask, 0 = none)
  src/io/gguf_reader.cpp:243-407   find_tensor, has_key and the typed getters
  src/io/gguf_reader.cpp:436-452   metadata_value_to_string (ostream <<)
  src/compute/common/dtype.cpp:28-64  gguf_tensor_nbytes (size_t arithmetic)
  src/model/qwen_config.cpp:59-151 QwenConfig::from_gguf
All size_t / uint64 arithmetic wraps modulo 2^64 as in C++.

`dump(path)` renders what a reader exposes as canonical bytes -- the same
format oracle/gguf_dump.hpp prints for a C++ GgufFile -- so the engine's
reader, the reference's (compiled into oracle/_ref) and this restatement
can be compared byte for byte.
"""
from __future__ import annotations

import struct
from typing import Dict, List, Optional, Tuple

import numpy as np

M64 = (1 << 64) - 1
MAX_ITEMS = 1 << 32

# metadata type codes (gguf_reader.h:12-26); variant alternative index =
# code for codes < 9, code - 1 above (GgufScalar / GgufArray order)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
        F64: "<d"}

# dtype.cpp:28-52: (elements per block, bytes per block); 0 for the rest
_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210)}

_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1", 10: "Q2_K",
               11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 30: "BF16"}


class GgufError(Exception):
    pass


def to_f32(x: float) -> float:
    """A double rounded to float as static_cast<float> does (round to nearest
    even; beyond the float range +-inf)."""
    with np.errstate(over="ignore"):
        return float(np.float32(x))


def tensor_nbytes(ttype: int, elements: int) -> int:
    """dtype.cpp:54-64."""
    block, nbytes = _BLOCK.get(ttype, (0, 0))
    if block == 0:
        return 0
    return ((((elements + block - 1) & M64) // block) * nbytes) & M64


def align_to(v: int, a: int) -> int:
    """gguf_reader.cpp:115-120."""
    if a == 0:
        return v
    return ((v + a - 1) & M64) & (~(a - 1) & M64)


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.o = data, 0

    def take(self, n: int) -> bytes:
        if n > len(self.d) - self.o:
            raise GgufError("read past the end")
        b = self.d[self.o:self.o + n]
        self.o += n
        return b

    def pod(self, t: int):
        fmt = _FMT[U8 if t == BOOL else t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> bytes:            # :21-32
        n = self.pod(U64)
        if n > MAX_ITEMS:
            raise GgufError("string too large")
        return self.take(n)

    def scalar(self, t: int):             # :49-65
        if t == BOOL:
            return self.pod(U8) != 0
        if t == STR:
            return self.string()
        if t in _FMT:
            return self.pod(t)
        raise GgufError("unsupported GGUF metadata scalar type")

    def array(self, item: int) -> list:   # :69-100
        n = self.pod(U64)
        if item == STR:
            if n > MAX_ITEMS:
                raise GgufError("array too large")
            return [self.string() for _ in range(n)]
        if item == BOOL:
            if n > MAX_ITEMS:
                raise GgufError("array too large")
            return [b != 0 for b in self.take(n)]
        if item in _FMT:
            if n > MAX_ITEMS:
                raise GgufError("array too large")
            size = struct.calcsize(_FMT[item])
            raw = self.take(n * size)
            return list(struct.unpack("<%d%s" % (n, _FMT[item][1]), raw)) if n else []
        raise GgufError("unsupported GGUF metadata array type")

    def value(self) -> Tuple[str, int, object]:   # :103-112
        t = self.pod(U32)
        if t == ARR:
            item = self.pod(U32)
            return ("a", item, self.array(item))
        return ("s", t, self.scalar(t))


class GgufFile:
    """The parsed header, metadata {key: (kind, type, value)} and tensors."""

    def __init__(self, data: bytes):
        r = _Reader(data)
        magic = data[:4]
        r.o = min(4, len(data))
        if magic != b"GGUF":                                    # :171-175
            raise GgufError("not a GGUF file")
        self.version = r.pod(U32)
        n_tensors = r.pod(U64)
        n_meta = r.pod(U64)
        self.metadata: Dict[bytes, Tuple[str, int, object]] = {}
        for _ in range(n_meta):                                 # :184-188
            key = r.string()
            self.metadata[key] = r.value()
        self.alignment = self.get_u64(b"general.alignment", 32)    # :197
        self.tensors: List[dict] = []
        self.index: Dict[bytes, int] = {}
        for _ in range(n_tensors):                              # :205-229
            name = r.string()
            nd = r.pod(U32)
            dims = [r.pod(U64) for _ in range(nd)]
            ttype = r.pod(U32)
            rel = r.pod(U64)
            count = 1
            for d in dims:
                count = (count * d) & M64
            nbytes = tensor_nbytes(ttype, count)
            if nbytes == 0:
                raise GgufError("unsupported GGUF tensor type for tensor: %s type=%s"
                                % (name.decode("latin-1"), _TYPE_NAMES.get(ttype, "Unknown")))
            self.index[name] = len(self.tensors)
            self.tensors.append(dict(name=name, dims=dims, type=ttype, rel=rel, nbytes=nbytes, count=count))
        self.data_offset = align_to(r.o, self.alignment)       # :232-239
        for t in self.tensors:
            t["abs"] = (self.data_offset + t["rel"]) & M64

    # ---- getters (:243-407) ------------------------------------------------
    def _scalar(self, key: bytes):
        v = self.metadata.get(key)
        return None if v is None or v[0] != "s" else (v[1], v[2])

    def get_string(self, key: bytes, fallback: bytes) -> bytes:
        s = self._scalar(key)
        return s[1] if s and s[0] == STR else fallback

    def get_u64(self, key: bytes, fallback: int) -> int:
        s = self._scalar(key)
        if not s:
            return fallback
        t, v = s
        if t in (U64, U32):
            return v
        if t in (I64, I32):
            return v & M64 if v >= 0 else fallback
        return fallback

    def get_i64(self, key: bytes, fallback: int) -> int:
        s = self._scalar(key)
        if not s:
            return fallback
        t, v = s
        if t in (I64, I32):
            return v
        if t in (U64, U32):
            return v - (1 << 64) if v >= (1 << 63) else v
        return fallback

    def get_f64(self, key: bytes, fallback: float) -> float:
        s = self._scalar(key)
        return float(s[1]) if s and s[0] in (F64, F32) else fallback

    def get_f32(self, key: bytes, fallback: float) -> float:
        """static_cast<float>(get_f64(key, fallback)) (:360-362): nearest-even,
        overflow to +-inf."""
        return to_f32(self.get_f64(key, fallback))

    def get_bool(self, key: bytes, fallback: bool) -> bool:
        s = self._scalar(key)
        return s[1] if s and s[0] == BOOL else fallback

    def _array(self, key: bytes, item: int) -> list:
        v = self.metadata.get(key)
        return v[2] if v is not None and v[0] == "a" and v[1] == item else []

    def get_string_array(self, key: bytes) -> List[bytes]:
        return self._array(key, STR)

    def get_f32_array(self, key: bytes) -> List[float]:
        return self._array(key, F32)

    def get_u32_array(self, key: bytes) -> List[int]:
        return self._array(key, U32)

    def find_tensor(self, name: bytes) -> Optional[dict]:
        i = self.index.get(name)
        return None if i is None else self.tensors[i]


def value_to_string(kind: str, t: int, v) -> bytes:
    """metadata_value_to_string (:436-452): `std::ostream << v` for a scalar
    (8-bit integers print as the character, bool as 1/0, floating point as
    %g), "array[N]" for an array."""
    if kind == "a":
        return b"array[%d]" % len(v)
    if t in (U8, I8):
        return bytes([v & 0xFF])
    if t == BOOL:
        return b"1" if v else b"0"
    if t == STR:
        return v
    if t in (F32, F64):
        return (b"%g" % v)
    return b"%d" % v


# ---- QwenConfig::from_gguf (qwen_config.cpp:59-151) ----------------------
def from_gguf(g: GgufFile) -> dict:
    def u32(arch: bytes, suffix: bytes, fallback: int = 0) -> int:
        return g.get_u64(arch + b"." + suffix, fallback) & 0xFFFFFFFF

    def f32(arch: bytes, suffix: bytes, fallback: float) -> float:
        return g.get_f32(arch + b"." + suffix, fallback)

    arch = g.get_string(b"general.architecture", b"qwen3")
    if b"qwen" not in arch:
        raise GgufError("Only Qwen/Qwen3 dense GGUF is supported in this engine")
    c = dict(arch=arch, vocab=len(g.get_string_array(b"tokenizer.ggml.tokens")) & 0xFFFFFFFF)
    c["ctx"] = u32(arch, b"context_length", 2048)
    c["emb"] = u32(arch, b"embedding_length")
    c["blocks"] = u32(arch, b"block_count")
    c["ff"] = u32(arch, b"feed_forward_length")
    c["heads"] = u32(arch, b"attention.head_count")
    c["kv"] = u32(arch, b"attention.head_count_kv", c["heads"])
    c["hd"] = u32(arch, b"attention.key_length", 0)
    c["vd"] = u32(arch, b"attention.value_length", 0)
    c["eps"] = f32(arch, b"attention.layer_norm_rms_epsilon", struct.unpack("<f", struct.pack("<f", 1e-6))[0])
    c["theta"] = f32(arch, b"rope.freq_base", 1000000.0)
    q2 = b"qwen2"
    for k, suffix in (("emb", b"embedding_length"), ("blocks", b"block_count"), ("ff", b"feed_forward_length"),
                      ("heads", b"attention.head_count")):
        if c[k] == 0:
            c[k] = u32(q2, suffix)
    if c["kv"] == 0:
        c["kv"] = u32(q2, b"attention.head_count_kv", c["heads"])
    if c["hd"] == 0:
        c["hd"] = u32(q2, b"attention.key_length", 0)
    if c["vd"] == 0:
        c["vd"] = u32(q2, b"attention.value_length", 0)
    for k, what in (("vocab", "vocab size"), ("emb", "embedding_length"), ("blocks", "block_count"),
                    ("ff", "feed_forward_length"), ("heads", "attention.head_count"),
                    ("kv", "attention.head_count_kv")):
        if c[k] == 0:
            raise GgufError("failed to read %s from GGUF" % what)
    if c["hd"] == 0:
        q = g.find_tensor(b"blk.0.attn_q.weight")
        if q is not None and len(q["dims"]) >= 2 and q["dims"][1] % c["heads"] == 0:
            c["hd"] = (q["dims"][1] // c["heads"]) & 0xFFFFFFFF
    if c["vd"] == 0:
        v = g.find_tensor(b"blk.0.attn_v.weight")
        if v is not None and len(v["dims"]) >= 2 and v["dims"][1] % c["kv"] == 0:
            c["vd"] = (v["dims"][1] // c["kv"]) & 0xFFFFFFFF
    if c["hd"] == 0:
        if c["emb"] % c["heads"] != 0:
            raise GgufError("embedding_length must be divisible by head_count when attention.key_length is absent")
        c["hd"] = c["emb"] // c["heads"]
    if c["vd"] == 0:
        c["vd"] = c["hd"]
    if c["hd"] == 0:
        raise GgufError("failed to read or derive attention.key_length/head_dim from GGUF")
    if c["vd"] != c["hd"]:
        raise GgufError("this minimal attention path currently requires attention.value_length == "
                        "attention.key_length")
    return c


# ---- canonical dump (same bytes as oracle/gguf_dump.hpp) ------------------
_PLAIN = set(range(0x21, 0x7F)) - {ord(c) for c in "\\;,[]="}
FALLBACK_U64 = 0xDEADBEEFDEADBEEF
FALLBACK_I64 = -0x123456789
FALLBACK_F64 = 0.5
FALLBACK_F32 = 0.25
FALLBACK_STR = b"\x01fallback"
ABSENT_KEY = b"no.such.key"


def esc(b: bytes) -> bytes:
    return b"".join(bytes([c]) if c in _PLAIN else b"\\x%02x" % c for c in b)


def _f64bits(v: float) -> bytes:
    return b"%016x" % struct.unpack("<Q", struct.pack("<d", v))[0]


def _f32bits(v: float) -> bytes:
    return b"%08x" % struct.unpack("<I", struct.pack("<f", v))[0]


def _getters(g: GgufFile, key: bytes) -> bytes:
    sa = g.get_string_array(key)
    fa = g.get_f32_array(key)
    ua = g.get_u32_array(key)
    return b" ".join([
        b"u64=%d" % g.get_u64(key, FALLBACK_U64),
        b"i64=%d" % g.get_i64(key, FALLBACK_I64),
        b"f64=" + _f64bits(g.get_f64(key, FALLBACK_F64)),
        b"f32=" + _f32bits(g.get_f32(key, FALLBACK_F32)),
        b"b=%d%d" % (g.get_bool(key, False), g.get_bool(key, True)),
        b"str=" + esc(g.get_string(key, FALLBACK_STR)),
        b"sarr=%d[" % len(sa) + b";".join(esc(s) for s in sa) + b"]",
        b"farr=%d[" % len(fa) + b",".join(_f32bits(f) for f in fa) + b"]",
        b"uarr=%d[" % len(ua) + b",".join(b"%d" % u for u in ua) + b"]",
    ])


def _variant_index(code: int) -> int:
    return code if code < ARR else code - 1


def dump_file(g: GgufFile) -> bytes:
    out = [b"version %d" % g.version, b"alignment %d" % g.alignment, b"tensors %d" % len(g.tensors)]
    for i, t in enumerate(g.tensors):
        found = g.index[t["name"]]
        out.append(b"T %d %s dims=%s type=%d rel=%d abs=%d nbytes=%d find=%d" % (
            i, esc(t["name"]), b",".join(b"%d" % d for d in t["dims"]), t["type"], t["rel"], t["abs"],
            t["nbytes"], found))
    out.append(b"metadata %d" % len(g.metadata))
    for key in sorted(g.metadata):
        kind, t, v = g.metadata[key]
        out.append(b"M %s kind=%s%d text=%s %s" % (esc(key), kind.encode(), _variant_index(t) if kind == "s"
                                                    else _variant_index(t), esc(value_to_string(kind, t, v)),
                                                    _getters(g, key)))
    out.append(b"A has=%d %s" % (ABSENT_KEY in g.metadata, _getters(g, ABSENT_KEY)))
    return b"\n".join(out) + b"\n"


def dump_config(g: GgufFile) -> bytes:
    try:
        c = from_gguf(g)
    except GgufError as e:
        return b"config error: " + esc(str(e).encode()) + b"\n"
    return (b"config arch=%s vocab=%d ctx=%d emb=%d blocks=%d ff=%d heads=%d kv=%d hd=%d vd=%d eps=%s theta=%s\n"
            % (esc(c["arch"]), c["vocab"], c["ctx"], c["emb"], c["blocks"], c["ff"], c["heads"], c["kv"], c["hd"],
               c["vd"], _f32bits(c["eps"]), _f32bits(c["theta"])))


def read_tensor_bytes(g: GgufFile, data: bytes, t: dict) -> bytes:
    """gguf_reader.cpp:410-423: nbytes from absolute_offset, or an error
    when they run past the end of the file."""
    if t["abs"] > len(data) or t["nbytes"] > len(data) - t["abs"]:
        raise GgufError("failed to read GGUF tensor: %s" % t["name"].decode("latin-1"))
    return data[t["abs"]:t["abs"] + t["nbytes"]]


def fnv1a64(b: bytes) -> int:
    h = 0xCBF29CE484222325
    for c in b:
        h = ((h ^ c) * 0x100000001B3) & M64
    return h


def dump_reads(g: GgufFile, data: bytes) -> bytes:
    out = []
    for i, t in enumerate(g.tensors):
        try:
            b = read_tensor_bytes(g, data, t)
            out.append(b"R %d n=%d fnv=%016x" % (i, len(b), fnv1a64(b)))
        except GgufError:
            out.append(b"R %d error" % i)
    return b"".join(x + b"\n" for x in out)


def dump(path: str) -> bytes:
    """The canonical dump of a file, or b"error: ..." when it does not load."""
    with open(path, "rb") as f:
        data = f.read()
    try:
        g = GgufFile(data)
    except GgufError as e:
        return b"error: " + esc(str(e).encode()) + b"\n"
    return dump_file(g) + dump_config(g) + dump_reads(g, data)
