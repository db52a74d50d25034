"""Tokenizer: the engine's citlali::tokenizer::Tokenizer (the reference's
src/tokenizer/tokenizer.cpp:130-400) through tests/cpp/test_tokenizer,
against the reference's own tokenizer's view of the fixture files
(tests/golden/tokenizer/*.dump, written by tests/golden/make_tok_golden.py
with the reference tokenizer compiled into oracle/_ref/ref_tok_dump), byte
for byte: every piece and decode_token, encode with and without BOS,
decode(encode), the ChatML template.  Where oracle/_ref is built, also
random texts and random vocabularies against the compiled reference live.
No GPU."""
import os
import random
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "tokenizer")
BIN = os.path.join(ROOT, "tests", "cpp", "test_tokenizer")
REF = os.path.join(ROOT, "oracle", "_ref", "ref_tok_dump")
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

import tok_cases as C  # noqa: E402

TEXTS = os.path.join(GOLD, "texts.hex")
need_ref = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref/ref_tok_dump is not built "
                                                              "(the reference sources are absent)")


def run_dump(exe, texts, paths):
    out = subprocess.run([exe, *(["dump"] if exe == BIN else []), texts, *paths], capture_output=True, timeout=300)
    assert out.returncode == 0, out.stderr.decode(errors="replace")[-2000:]
    parts = out.stdout.split(b"\0\n")
    assert parts[-1] == b"" and len(parts) == len(paths) + 1
    return parts[:-1]


def engine(texts, paths):
    assert os.path.exists(BIN), "tests/cpp/test_tokenizer is not built: run __graft_entry__.build()"
    return run_dump(BIN, texts, paths)


def first_difference(a: bytes, b: bytes) -> str:
    for la, lb in zip(a.split(b"\n"), b.split(b"\n")):
        if la != lb:
            return f"engine {la[:200]!r}\nreference {lb[:200]!r}"
    return f"lengths {len(a)} vs {len(b)}"


@pytest.mark.parametrize("case", sorted(C.CASES))
def test_fixture_dump_matches_reference(case):
    path = os.path.join(GOLD, case + ".gguf")
    with open(path, "rb") as f:
        assert f.read() == C.CASES[case](), f"{case}.gguf no longer matches tok_cases.py: rerun make_tok_golden.py"
    with open(os.path.join(GOLD, case + ".dump"), "rb") as f:
        want = f.read()
    (got,) = engine(TEXTS, [path])
    assert got == want, first_difference(got, want)


def test_fixture_texts_cover_the_fallbacks():
    """The committed dumps reach what they are meant to: merges that chain,
    control tokens as one id, '<0xXX>' and raw-byte pieces, the unknown id,
    a BOS id that is out of range and one that is negative."""
    dump = {c: open(os.path.join(GOLD, c + ".dump"), "rb").read().decode("latin-1") for c in C.CASES}
    lines = {c: dict((" ".join(l.split()[:2]), l.split()[2:]) for l in d.splitlines() if l) for c, d in dump.items()}
    q = lines["qwen_like"]
    k = C.TEXTS.index(b"The quick brown fox jumps over the lazy dog.")
    assert len(q[f"enc {k}"]) < len(C.TEXTS[k]) // 3   # merged far below one id per byte
    k = C.TEXTS.index(b"<|endoftext|>")
    assert q[f"enc {k}"] == ["797"] and q[f"bos {k}"] == ["797", "797"]
    s = lines["sparse"]
    k = C.TEXTS.index(b"\x00\x01\x02\x07\x1b\x7f")
    assert "3" in s[f"enc {k}"]                         # raw-byte pieces -> unknown id 3
    assert s[f"bos {k}"][0] == "151643"                 # default BOS id, outside the vocabulary
    d = lines["dup_tokens"]
    assert d["bos 0"] == [] and dump["dup_tokens"].startswith("vocab 604 bos -7 ")
    assert dump["missing_tokens"] == "load error\n" and dump["empty_tokens"] == "load error\n"


def test_tokenizer_that_never_loaded():
    """Defaults and no vocabulary: every byte is its own piece and the
    unknown id 0, nothing decodes, the template still applies."""
    got = subprocess.run([BIN, "fresh", TEXTS], capture_output=True, check=True, timeout=60).stdout
    with open(os.path.join(GOLD, "fresh.dump"), "rb") as f:
        want = f.read()
    assert got == want, first_difference(got, want)


def test_reload_keeps_ids_the_second_file_lacks():
    a, b = os.path.join(GOLD, "qwen_like.gguf"), os.path.join(GOLD, "no_merges.gguf")
    got = subprocess.run([BIN, "reload", a, b], capture_output=True, check=True, timeout=60).stdout
    assert got == b"vocab 1024 bos 797 eos 331 pad 797\nvocab 270 bos 797 eos 257 pad 258\n"
    if os.path.exists(REF):
        assert subprocess.run([REF, "--reload", a, b], capture_output=True, check=True, timeout=60).stdout == got


def test_long_text_encodes_in_n_log_n():
    """200 kB through the heap-ordered merge loop, and back."""
    out = subprocess.run([BIN, "time", os.path.join(GOLD, "qwen_like.gguf"), "200000"], capture_output=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr.decode(errors="replace")
    ms = float(out.stdout.split()[-2])
    assert ms < 2000, out.stdout


@need_ref
def test_random_texts_against_reference():
    rng = random.Random(20261202)
    with tempfile.TemporaryDirectory() as d:
        paths = []
        for case in ("qwen_like", "sparse", "no_merges", "dup_tokens"):
            paths.append(os.path.join(GOLD, case + ".gguf"))
        vocab = C.qwen_like_parts()[0]
        texts = [C.random_text(rng, vocab, rng.randrange(0, 300)) for _ in range(400)]
        tf = os.path.join(d, "texts.hex")
        with open(tf, "w") as f:
            f.write("".join(t.hex() + "\n" for t in texts))
        for path, got, want in zip(paths, engine(tf, paths), run_dump(REF, tf, paths)):
            assert got == want, os.path.basename(path) + "\n" + first_difference(got, want)


@need_ref
def test_random_vocabularies_against_reference():
    rng = random.Random(77)
    with tempfile.TemporaryDirectory() as d:
        paths = []
        for i in range(30):
            p = os.path.join(d, f"v{i}.gguf")
            with open(p, "wb") as f:
                f.write(C.random_tokenizer(rng))
            paths.append(p)
        vocab = C.qwen_like_parts()[0]
        texts = [C.random_text(rng, vocab, rng.randrange(0, 200)) for _ in range(60)]
        tf = os.path.join(d, "texts.hex")
        with open(tf, "w") as f:
            f.write("".join(t.hex() + "\n" for t in texts))
        for path, got, want in zip(paths, engine(tf, paths), run_dump(REF, tf, paths)):
            assert got == want, os.path.basename(path) + "\n" + first_difference(got, want)
