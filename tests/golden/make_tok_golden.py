"""Writes the tokenizer fixtures under tests/golden/tokenizer/: each case of
tok_cases.py as <case>.gguf, the texts as texts.hex (one hex line each), and
the reference's own tokenizer's view of them -- src/tokenizer/tokenizer.cpp
and its GGUF reader compiled from /root/reference into
oracle/_ref/ref_tok_dump by oracle/Makefile -- as <case>.dump (the canonical
text of oracle/tok_dump.hpp), and its view of a tokenizer that never loaded
a file as fresh.dump.

    make -C oracle && python tests/golden/make_tok_golden.py
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)

from tok_cases import CASES, TEXTS  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "ref_tok_dump")
OUT = os.path.join(HERE, "tokenizer")


def main() -> None:
    if not os.path.exists(REF):
        raise SystemExit("oracle/_ref/ref_tok_dump is not built (make -C oracle)")
    os.makedirs(OUT, exist_ok=True)
    texts = os.path.join(OUT, "texts.hex")
    with open(texts, "w") as f:
        f.write("".join(t.hex() + "\n" for t in TEXTS))
    fresh = subprocess.run([REF, "--fresh", texts], capture_output=True, check=True).stdout
    with open(os.path.join(OUT, "fresh.dump"), "wb") as f:
        f.write(fresh)
    for name, make in CASES.items():
        path = os.path.join(OUT, name + ".gguf")
        with open(path, "wb") as f:
            f.write(make())
        out = subprocess.run([REF, texts, path], capture_output=True, check=True).stdout
        assert out.endswith(b"\0\n"), name
        with open(os.path.join(OUT, name + ".dump"), "wb") as f:
            f.write(out[:-2])
        print(f"{name:16s} {os.path.getsize(path):7d} B gguf, {len(out):7d} B dump: "
              f"{out.splitlines()[0][:60].decode('latin-1')}")


if __name__ == "__main__":
    main()
