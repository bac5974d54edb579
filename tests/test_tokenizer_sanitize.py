"""The tokenizer's host code (host/tokenizer.cpp) under AddressSanitizer and
UndefinedBehaviorSanitizer: tests/tokenizer_sanitize.cpp is compiled with
g++ together with the library's tokenizer source and run over a trained
byte-level vocabulary (the one test_tokenizer.py trains) and over malformed
vocab.json / merges.txt files.  A memory error, a leak or undefined
behaviour ends the run with the sanitizer's report; the driver's own checks
cover the C ABI's sizing and truncation rules and the round trip."""
import os
import shutil
import subprocess

import pytest

from test_tokenizer import trained_dir  # noqa: F401  (fixture)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cuda-llm-inference-engine_amd")


def test_tokenizer_under_asan_ubsan(trained_dir, tmp_path):  # noqa: F811
    if shutil.which("g++") is None:
        pytest.skip("g++ is not installed")
    exe = str(tmp_path / "tokenizer_sanitize")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "csrc"),
           os.path.join(ROOT, "tests", "tokenizer_sanitize.cpp"), os.path.join(PKG, "host", "tokenizer.cpp"),
           "-o", exe]
    b = subprocess.run(cmd, capture_output=True, text=True)
    if b.returncode != 0 and ("cannot find -lasan" in b.stderr or "cannot find -lubsan" in b.stderr):
        pytest.skip("g++ has no sanitizer runtimes here")
    assert b.returncode == 0, b.stderr[-4000:]
    scratch = tmp_path / "files"
    scratch.mkdir()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, trained_dir[0], str(scratch)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "tokenizer_sanitize: ok" in r.stdout, (r.returncode, r.stderr[-4000:])
