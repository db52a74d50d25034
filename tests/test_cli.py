"""bin/citlali_cli, the command line over InferenceSession (the reference's
src/cli/main.cpp): argument handling, --info, and --tokens (whose ids and
decoded text must equal the reference tokenizer's view in
tests/golden/tokenizer/qwen_like.dump) without a GPU; generation against an
InferenceSession run of the same prompt on the GPU."""
import os
import re
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "citlali-llm-engine_amd", "bin", "citlali_cli")
HOST = os.path.join(ROOT, "tests", "cpp", "test_host_layer")
TOK = os.path.join(ROOT, "tests", "golden", "tokenizer", "qwen_like.gguf")
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

import tok_cases as C  # noqa: E402


def cli(*args, timeout=120):
    assert os.path.exists(CLI), "citlali_cli is not built: run __graft_entry__.build()"
    return subprocess.run([CLI, *args], capture_output=True, timeout=timeout)


def unescape(s: bytes) -> bytes:
    out, i = bytearray(), 0
    while i < len(s):
        if s[i:i + 1] == b"\\":
            c = s[i + 1:i + 2]
            if c == b"x":
                out.append(int(s[i + 2:i + 4], 16))
                i += 4
                continue
            out += {b"n": b"\n", b"r": b"\r", b"t": b"\t", b'"': b'"', b"\\": b"\\"}[c]
            i += 2
        else:
            out.append(s[i])
            i += 1
    return bytes(out)


@pytest.fixture(scope="module")
def model():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "session_model.gguf")
        out = subprocess.run([HOST, "write_session_model", TOK, path], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0, out.stdout + out.stderr
        yield path


def test_usage_and_argument_errors():
    r = cli("--help")
    assert r.returncode == 0 and b"Usage:" in r.stdout
    r = cli()
    assert r.returncode == 1 and b"Usage:" in r.stdout
    for args, msg in ((("--remote", "127.0.0.1:1"), b"remote layer offload is not part of this build"),
                      (("--offload", "layer:0"), b"remote layer offload is not part of this build"),
                      (("--bogus",), b"unknown argument: --bogus"),
                      (("--max-new-tokens", "12x"), b"--max-new-tokens needs a number"),
                      # refused while parsing, before any model file is opened
                      (("--model", os.path.join(ROOT, "no_such_file.gguf"), "--decode-chunk", "0"),
                       b"--decode-chunk must be at least 1"),
                      (("--model",), b"missing value for --model")):
        r = cli(*args)
        assert r.returncode == 1 and msg in r.stderr, (args, r.stderr)
    r = cli("--model", os.path.join(ROOT, "no_such_file.gguf"), "--info")
    assert r.returncode == 1 and r.stderr.startswith(b"error: ")


def test_info(model):
    r = cli("--model", model, "--info")
    assert r.returncode == 0, r.stderr
    lines = dict(l.split(": ", 1) for l in r.stdout.decode().splitlines() if ": " in l)
    assert (lines["architecture"], lines["vocab"], lines["layers"], lines["hidden"], lines["ffn"], lines["heads"],
            lines["kv_heads"], lines["head_dim"]) == ("qwen3", "1024", "2", "1024", "2048", "8", "4", "128")
    assert lines["tensors"] == "25" and "  Q4_K: 10" in r.stdout.decode()


def reference_lines(case="qwen_like"):
    d = {}
    for l in open(os.path.join(ROOT, "tests", "golden", "tokenizer", case + ".dump"), "rb").read().splitlines():
        parts = l.split(b" ")
        if parts[0] in (b"bos", b"dec"):
            d[(parts[0], int(parts[1]))] = parts[2:]
    return d


def test_tokens_match_reference_tokenizer():
    ref = reference_lines()
    checked = 0
    for k, text in enumerate(C.TEXTS):
        if not text or b"\x00" in text:
            continue   # argv cannot carry these
        r = cli("--model", TOK, "--prompt", text, "--tokens", "--no-chat-template")
        assert r.returncode == 0, (text, r.stderr)
        rows = [l.split(b"\t") for l in r.stdout.split(b"\n") if re.match(rb"^\d+\t", l)]
        ids = [row[1] for row in rows]
        assert ids == ref[(b"bos", k)], text
        decoded = b"".join(unescape(row[3][len(b'decoded="'):-1]) for row in rows)
        assert decoded.hex().encode() == (ref[(b"dec", k)][0] if ref[(b"dec", k)] else b""), text
        checked += 1
    assert checked >= 30


def test_tokens_with_chat_template():
    r = cli("--model", TOK, "--prompt", "Hello, world!", "--tokens")
    assert r.returncode == 0
    out = r.stdout.decode()
    assert out.startswith("prompt_text: <|im_start|>user\nHello, world!<|im_end|>\n<|im_start|>assistant\n\n")
    rows = [l.split("\t") for l in out.splitlines() if re.match(r"^\d+\t", l)]
    assert int(out.split("token_count: ")[1].split("\n")[0]) == len(rows)
    assert rows[0][2] == 'piece="<|endoftext|>"' and rows[0][3] == 'decoded=""'   # BOS (add_bos_token)
    assert rows[1][2] == 'piece="<|im_start|>"'


def run_generation(model, prompt, max_new, chat, quantized, chunk=None):
    args = ["--model", model, "--prompt", prompt, "--max-new-tokens", str(max_new), "--ctx", "256"]
    if not chat:
        args.append("--no-chat-template")
    if quantized:
        args.append("--quantized")
    if chunk is not None:
        args += ["--decode-chunk", str(chunk)]
    r = cli(*args, timeout=300)
    assert r.returncode == 0, r.stderr.decode(errors="replace")
    text, sep, stats = r.stdout.rpartition(b"\n[stats] ")
    assert sep, r.stdout
    m = re.match(rb"tokens=(\d+) time=[\d.]+s speed=[\d.]+ tok/s stop=(\w+)\n$", stats)
    assert m, stats
    return text, int(m.group(1)), m.group(2).decode()


@pytest.mark.gpu
@pytest.mark.parametrize("quantized", [True, False])
def test_generation_equals_session(model, quantized):
    names = {"max_new": "max_new_tokens", "eos": "eos", "context": "context_limit"}
    for prompt, chat in (("Hello there", True), ("The quick brown fox", False)):
        text, n, stop = run_generation(model, prompt, 24, chat, quantized)
        ref = subprocess.run([HOST, "session_text", model, prompt, "24", str(int(chat)), str(int(quantized))],
                             capture_output=True, text=True, timeout=300)
        assert ref.returncode == 0, ref.stdout + ref.stderr
        m = re.search(r"tokens (\d+) stop (\w+) text ([0-9a-f]*)", ref.stdout)
        assert m, ref.stdout
        assert (n, stop, text) == (int(m.group(1)), names[m.group(2)], bytes.fromhex(m.group(3))), prompt
        assert run_generation(model, prompt, 24, chat, quantized, chunk=1)[:2] == (text, n)
