"""CPU checks of the host-side memory bookkeeping and copy loops under
sanitizers: csrc/device_cache.h (the caching allocator behind tt_malloc /
tt_free and the per-stream workspace cache of the attention launchers) over
a fake malloc backend with allocation-failure injection, and the staged
transfers' loops of csrc/host_copy.cpp, compiled with g++ into standalone
executables (tests/native/host_checks.cpp) with AddressSanitizer +
UndefinedBehaviorSanitizer, and with ThreadSanitizer for the multi-threaded
workspace leases.  A planted one-byte overrun shows that the ASan build
reports what it should.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pku-aiprogramming_amd", "csrc")
SRC = [os.path.join(ROOT, "tests", "native", "host_checks.cpp"), os.path.join(CSRC, "host_copy.cpp")]
BASE = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-pthread", "-I", CSRC]

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")


def _build(tmp, name, flags):
    exe = os.path.join(tmp, name)
    subprocess.run(BASE + flags + SRC + ["-o", exe], check=True, capture_output=True, text=True)
    return exe


def _run(exe, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=300, env=env)


def test_host_checks_under_asan_and_ubsan(tmp_path):
    exe = _build(str(tmp_path), "asan", ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"])
    r = _run(exe)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host checks passed" in r.stdout


def test_workspace_leases_under_tsan(tmp_path):
    exe = _build(str(tmp_path), "tsan", ["-fsanitize=thread"])
    r = _run(exe, "threads")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "WARNING: ThreadSanitizer" not in r.stderr


def test_asan_build_catches_a_planted_overrun(tmp_path):
    exe = _build(str(tmp_path), "planted", ["-fsanitize=address", "-DTT_PLANTED_OVERRUN"])
    r = _run(exe)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
