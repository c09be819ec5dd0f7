"""The oracle's C code under AddressSanitizer and UndefinedBehaviorSanitizer:
tests/oracle_sanitize.c calls every oracle function on small ragged inputs
(odd dimensions, k above n, several threads); any out-of-bounds access,
leak, signed overflow or misaligned access aborts it.  Host code only: the
HIP library's host side cannot run without a GPU, and GPU sanitizers are not
available here."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no gcc")
def test_oracle_under_asan_ubsan(tmp_path):
    exe = tmp_path / "oracle_sanitize"
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-ffp-contract=off", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "oracle"),
           os.path.join(ROOT, "tests", "oracle_sanitize.c"),
           os.path.join(ROOT, "oracle", "vsk_oracle.c"), "-lm", "-lpthread", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "oracle sanitize ok" in r.stdout
