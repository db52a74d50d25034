"""The GGUF fixture files (inputs only): small files that cover the format
rules of the reference's reader (src/io/gguf_reader.cpp) and
QwenConfig::from_gguf (src/model/qwen_config.cpp), valid and malformed.
make_gguf_golden.py writes them with the reference's dumps of each."""
from __future__ import annotations

import os
import struct
import sys
from typing import Callable, Dict

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "citlali-llm-engine_amd"))

from pycitlali import gguf_write as W  # noqa: E402


def _rand_bytes(seed: int, n: int) -> bytes:
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def _weights(seed: int, hidden=256, q=256, kv=128) -> list:
    """A few tensors of every type the engine stores."""
    t = [W.Tensor("token_embd.weight", [hidden, 4], W.T_Q6_K, _rand_bytes(seed, W.tensor_nbytes(W.T_Q6_K, hidden * 4))),
         W.Tensor("blk.0.attn_q.weight", [hidden, q], W.T_Q4_K, _rand_bytes(seed + 1, W.tensor_nbytes(W.T_Q4_K, hidden * q))),
         W.Tensor("blk.0.attn_v.weight", [hidden, kv], W.T_Q6_K,
                  _rand_bytes(seed + 2, W.tensor_nbytes(W.T_Q6_K, hidden * kv))),
         W.Tensor("blk.0.attn_norm.weight", [hidden], W.T_F32,
                  W.f32_bytes(np.random.default_rng(seed + 3).standard_normal(hidden))),
         W.Tensor("blk.0.f16", [64, 2], W.T_F16, _rand_bytes(seed + 4, 256)),
         W.Tensor("blk.0.bf16", [100], W.T_BF16, _rand_bytes(seed + 5, 200)),
         W.Tensor("blk.0.q8", [70], W.T_Q8_0, _rand_bytes(seed + 6, W.tensor_nbytes(W.T_Q8_0, 70)))]
    return t


def qwen3_basic() -> bytes:
    return W.build(W.qwen_meta(vocab=16, hidden=256, blocks=1, ff=1024, heads=2, kv_heads=1, head_dim=128), _weights(1))


def qwen3_derive_head_dim() -> bytes:
    # head_dim from blk.0.attn_q rows (256 / 2 heads), value_dim from attn_v (128 / 1)
    return W.build(W.qwen_meta(vocab=16, hidden=256, blocks=1, ff=1024, heads=2, kv_heads=1, head_dim=None),
                   _weights(2))


def qwen3_derive_from_embedding() -> bytes:
    # no key/value length, no blk.0.attn_q / attn_v: head_dim = 512 / 8
    ts = [t for t in _weights(3) if "attn_q" not in t.name and "attn_v" not in t.name]
    return W.build(W.qwen_meta(vocab=8, hidden=512, blocks=2, ff=1024, heads=8, kv_heads=8, head_dim=None), ts[:2])


def qwen2_keys_under_other_arch() -> bytes:
    # architecture "qwen3x": its own keys are absent, the qwen2.* ones are read
    m = [W.scalar("general.architecture", W.STR, "qwen3x"),
         W.array("tokenizer.ggml.tokens", W.STR, ["a", "b", "c"])]
    m += [x for x in W.qwen_meta("qwen2", vocab=3, hidden=256, blocks=3, ff=512, heads=2, kv_heads=1, head_dim=128)
          if not x.key.startswith("general.") and not x.key.startswith("tokenizer.")]
    m.append(W.scalar("qwen3x.attention.head_count_kv", W.I32, -1))   # negative: treated as absent
    return W.build(m, [])


def config_not_qwen() -> bytes:
    return W.build(W.qwen_meta("llama", vocab=4, hidden=256), [])


def config_default_arch_and_value_mismatch() -> bytes:
    m = [x for x in W.qwen_meta(vocab=4, hidden=256, head_dim=128) if x.key != "general.architecture"
         and x.key != "qwen3.attention.value_length"]
    m.append(W.scalar("qwen3.attention.value_length", W.U64, 64))
    return W.build(m, [])


def config_missing_vocab() -> bytes:
    return W.build([x for x in W.qwen_meta(vocab=4) if x.key != "tokenizer.ggml.tokens"], [])


def config_missing_ff() -> bytes:
    return W.build([x for x in W.qwen_meta(vocab=4) if x.key != "qwen3.feed_forward_length"], [])


def config_not_divisible() -> bytes:
    ts = []
    return W.build(W.qwen_meta(vocab=4, hidden=250, heads=3, kv_heads=3, head_dim=None), ts)


def config_eps_f64_and_theta_i32() -> bytes:
    m = [x for x in W.qwen_meta(vocab=4) if "epsilon" not in x.key and "freq_base" not in x.key]
    m += [W.scalar("qwen3.attention.layer_norm_rms_epsilon", W.F64, 1e-5),
          W.scalar("qwen3.rope.freq_base", W.I32, 10000)]          # not a float: default theta
    m.append(W.scalar("qwen3.context_length", W.U64, 1 << 33))      # u64 cut to u32
    return W.build(m, [])


def all_types() -> bytes:
    m = [W.scalar("u8.zero", W.U8, 0), W.scalar("u8.nl", W.U8, 10), W.scalar("u8.max", W.U8, 255),
         W.scalar("i8.neg", W.I8, -1), W.scalar("i8.a", W.I8, 65),
         W.scalar("u16", W.U16, 65535), W.scalar("i16", W.I16, -32768),
         W.scalar("u32.max", W.U32, 2 ** 32 - 1), W.scalar("i32.neg", W.I32, -7), W.scalar("i32.pos", W.I32, 7),
         W.scalar("u64.max", W.U64, 2 ** 64 - 1), W.scalar("u64.big", W.U64, 2 ** 63 + 5),
         W.scalar("i64.min", W.I64, -2 ** 63), W.scalar("i64.pos", W.I64, 123456789012345),
         W.scalar("f32.third", W.F32, 1.0 / 3), W.scalar("f32.negzero", W.F32, -0.0),
         W.scalar("f32.inf", W.F32, float("inf")), W.scalar("f32.neginf", W.F32, float("-inf")),
         W.scalar("f32.tiny", W.F32, 1e-45), W.scalar("f32.big", W.F32, 3.0e38),
         W.scalar("f64.big", W.F64, 1e300), W.scalar("f64.small", W.F64, 1e-310), W.scalar("f64.pi", W.F64, np.pi),
         W.scalar("f64.round", W.F64, 1.0 + 2.0 ** -30),
         W.scalar("bool.t", W.BOOL, 1), W.scalar("bool.f", W.BOOL, 0), W.scalar("bool.raw7", W.BOOL, 7),
         W.scalar("str.empty", W.STR, ""), W.scalar("str.bytes", W.STR, b"a b\n\x00\xff=;[],\\"),
         W.scalar("dup", W.U32, 1), W.scalar("dup", W.STR, "second wins"),
         W.array("a.u8", W.U8, [0, 1, 255]), W.array("a.i8", W.I8, [-128, 127]), W.array("a.u16", W.U16, [9]),
         W.array("a.i16", W.I16, [-9, 9]), W.array("a.u32", W.U32, [0, 7, 2 ** 32 - 1]),
         W.array("a.i32", W.I32, [-1, 1]), W.array("a.f32", W.F32, [1.5, -0.0, float("inf")]),
         W.array("a.bool", W.BOOL, [0, 1, 2]), W.array("a.str", W.STR, ["x", "", "y z", b"\x80"]),
         W.array("a.u64", W.U64, [2 ** 64 - 1]), W.array("a.i64", W.I64, [-5]), W.array("a.f64", W.F64, [0.1]),
         W.array("a.empty.str", W.STR, []), W.array("a.empty.f32", W.F32, []), W.array("a.empty.u32", W.U32, []),
         W.scalar("", W.U32, 3), W.scalar(b"key with space\x01", W.U32, 4)]
    ts = [W.Tensor("scalar0d", [], W.T_F32, b"\0\0\x80\x3f"), W.Tensor("ones", [1, 1, 1, 8], W.T_F16, b"\1" * 16),
          W.Tensor("dup.t", [4], W.T_F32, b"\2" * 16), W.Tensor("dup.t", [8], W.T_F32, b"\3" * 32),
          W.Tensor("partial.q8", [33], W.T_Q8_0, _rand_bytes(9, 68)),
          W.Tensor("partial.q4k", [300], W.T_Q4_K, _rand_bytes(10, 288))]
    return W.build(m, ts, version=3)


def _aligned(value_meta, alignment) -> bytes:
    m = W.qwen_meta(vocab=4, hidden=256, head_dim=128) + [value_meta]
    return W.build(m, _weights(20)[3:], alignment=alignment)


def alignment_64_u64() -> bytes:
    return _aligned(W.scalar("general.alignment", W.U64, 64), 64)


def alignment_zero() -> bytes:
    return _aligned(W.scalar("general.alignment", W.U32, 0), 0)


def alignment_negative_i32() -> bytes:
    return _aligned(W.scalar("general.alignment", W.I32, -8), 32)   # negative: default 32


def alignment_as_string() -> bytes:
    return _aligned(W.scalar("general.alignment", W.STR, "64"), 32)   # not an integer: default 32


def alignment_48() -> bytes:
    # not a power of two: both readers apply the same mask rounding
    return _aligned(W.scalar("general.alignment", W.U32, 48), 48)


def version_2() -> bytes:
    return W.build(W.qwen_meta(vocab=4, hidden=256), _weights(30)[3:], version=2)


def tensor_past_end() -> bytes:
    # the directory loads; the second tensor's bytes lie beyond the file
    t0 = _weights(31)[0]
    return W.build(W.qwen_meta(vocab=4, hidden=256), [t0, W.Tensor("far", [256], W.T_F32, b"", 1 << 40)])


def truncated_data() -> bytes:
    b = all_types()
    return b[:len(b) - 40]   # directory intact, last tensor short


def bad_magic() -> bytes:
    return b"GGUG" + all_types()[4:]


def empty_file() -> bytes:
    return b""


def truncated_in_metadata() -> bytes:
    return config_eps_f64_and_theta_i32()[:200]


def unsupported_meta_type() -> bytes:
    # value type 13 does not exist
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    return head + struct.pack("<Q", 3) + b"bad" + struct.pack("<I", 13) + b"\0" * 8


def nested_array() -> bytes:
    # an array whose item type is "array"
    return W.build([W.Meta("nest", W.ARR, [], W.ARR)], [])


def unsupported_tensor_type() -> bytes:
    return W.build(W.qwen_meta(vocab=4), [W.Tensor("q4_0", [32], 2, b"\0" * 18)])


def zero_dim_tensor() -> bytes:
    return W.build(W.qwen_meta(vocab=4), [W.Tensor("empty", [0, 4], W.T_F32, b"")])


def string_too_long() -> bytes:
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, 1)
    return head + struct.pack("<Q", (1 << 32) + 1) + b"x" * 16


def huge_tensor_count() -> bytes:
    return W.build(W.qwen_meta(vocab=4), [], tensor_count=1 << 40)


CASES: Dict[str, Callable[[], bytes]] = {f.__name__: f for f in (
    qwen3_basic, qwen3_derive_head_dim, qwen3_derive_from_embedding, qwen2_keys_under_other_arch, config_not_qwen,
    config_default_arch_and_value_mismatch, config_missing_vocab, config_missing_ff, config_not_divisible,
    config_eps_f64_and_theta_i32, all_types, alignment_64_u64, alignment_zero, alignment_negative_i32,
    alignment_as_string, alignment_48, version_2, tensor_past_end, truncated_data, bad_magic, empty_file,
    truncated_in_metadata, unsupported_meta_type, nested_array, unsupported_tensor_type, zero_dim_tensor,
    string_too_long, huge_tensor_count)}
