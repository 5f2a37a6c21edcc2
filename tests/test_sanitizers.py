"""The library's host code and the oracle under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU (tests/sanitize/):

- qora_file_fuzz: the .qora v1 reader (qora-llm_amd/csrc/qora_file.cpp,
  save.rs:154-262) and writer on valid Q4 and F16 files, every truncation up
  to 512 bytes and a stride past it, 3000 seeded byte/bit corruptions and
  0xFF length runs at every header offset: valid files round-trip byte for
  byte, truncated ones are refused, a refused load releases every upload it
  made, and no sanitizer report; plus the synthetic generator (synth.cpp).
- oracle_check: every oracle function on ragged shapes, and a tiny model's
  prefill and decode in Q4 and F16, T = 1 and 3, both F16 orders.

The device upload API the reader calls is replaced by a host recorder inside
the harness (host code only: nothing here builds or runs GPU code)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def built():
    if shutil.which("g++") is None or shutil.which("gcc") is None:
        pytest.skip("no host compiler")
    subprocess.run(["make", "-j4", "-C", SAN], check=True, capture_output=True)
    return os.path.join(SAN, "_build")


def _run(cmd):
    r = subprocess.run(cmd, env=ENV, capture_output=True, text=True, timeout=600)
    report = r.stderr[-4000:]
    assert r.returncode == 0, report
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, report
    return r.stdout


def test_qora_file_reader_under_sanitizers(built, tmp_path):
    assert "all cases held" in _run([os.path.join(built, "qora_file_fuzz"), str(tmp_path)])


def test_oracle_under_sanitizers(built):
    assert "clean" in _run([os.path.join(built, "oracle_check")])
