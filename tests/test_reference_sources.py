"""The reference's own callers of the model-layer API compile unchanged
against this build's headers (g++ -fsyntax-only): src/runtime/session.cpp
(QwenModel::load with its RemoteOptions argument, session.cpp:9-25) and
src/cli/main.cpp (InferenceSession::load_model(..., args.remote), the
remote::Transport / Backend options).  Needs the reference sources, which
exist only in the build container; skipped elsewhere.  Nothing is linked or
run: the point is the declarations, the behaviour is tested in
tests/cpp/test_host_layer (cpu mode, test_remote_options)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("CITLALI_REFERENCE", "/root/reference")
INCLUDES = [os.path.join(ROOT, "include"), os.path.join(ROOT, "citlali-llm-engine_amd", "csrc", "host", "include")]


@pytest.mark.parametrize("source", ["src/runtime/session.cpp", "src/cli/main.cpp"])
def test_reference_caller_compiles(source):
    path = os.path.join(REF, source)
    if not os.path.exists(path):
        pytest.skip("reference sources absent")
    cmd = ["g++", "-std=c++17", "-fsyntax-only", *[f"-I{d}" for d in INCLUDES], path]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
