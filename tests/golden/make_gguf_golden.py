"""Writes the GGUF fixtures under tests/golden/gguf/: each case of
gguf_cases.py as <case>.gguf and the reference's own view of it -- its
GgufFile and QwenConfig::from_gguf compiled from /root/reference into
oracle/_ref/ref_gguf_dump by oracle/Makefile -- as <case>.dump
(the canonical text of oracle/gguf_dump.hpp).

    make -C oracle && python tests/golden/make_gguf_golden.py
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)

from gguf_cases import CASES  # noqa: E402

REF = os.path.join(ROOT, "oracle", "_ref", "ref_gguf_dump")
OUT = os.path.join(HERE, "gguf")


def main() -> None:
    if not os.path.exists(REF):
        raise SystemExit("oracle/_ref/ref_gguf_dump is not built (make -C oracle)")
    os.makedirs(OUT, exist_ok=True)
    for name, make in CASES.items():
        path = os.path.join(OUT, name + ".gguf")
        with open(path, "wb") as f:
            f.write(make())
        out = subprocess.run([REF, path], capture_output=True, check=True).stdout
        assert out.endswith(b"\0\n"), name
        with open(os.path.join(OUT, name + ".dump"), "wb") as f:
            f.write(out[:-2])
        print(f"{name:40s} {os.path.getsize(path):7d} B  {out.splitlines()[0][:60].decode('latin-1')}")


if __name__ == "__main__":
    main()
