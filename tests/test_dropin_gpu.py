"""The drop-in C++ header (include/kernel_warpper.h) used the way the
reference's call sites use it, built as plain C++ by tests/dropin/Makefile
and run as its own process; the program checks every result against the
CPU oracle and prints one line per case."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "dropin", "dropin_test")


def test_dropin_header_program():
    assert os.path.exists(BIN), "tests/dropin/dropin_test is missing: run __graft_entry__.build()"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(res.stdout, res.stderr, flush=True)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-2000:]
    assert "ALL PASS" in res.stdout
    assert res.stdout.count("[PASS]") >= 40
