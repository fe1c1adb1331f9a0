"""The host C++ that parses untrusted input (the checkpoint header reader and
tensor layout, TransformerFactory.cpp:59-135) and builds the RoPE table,
built with AddressSanitizer and UndefinedBehaviorSanitizer and driven by a
header fuzz (tests/host/checkpoint_fuzz.cpp): truncated headers of every
version, extreme and random Config fields, garbage files.  Any sanitizer
report or layout outside the reported bytes fails the test.  CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "leap_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_checkpoint_reader_and_rope_table_under_asan_ubsan(tmp_path):
    exe = tmp_path / "checkpoint_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           os.path.join(ROOT, "tests", "host", "checkpoint_fuzz.cpp"),
           os.path.join(CSRC, "checkpoint.cpp"), os.path.join(CSRC, "rope_table.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe), str(tmp_path / "fuzz.bin")], capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert "ok: 0 failures" in r.stdout
