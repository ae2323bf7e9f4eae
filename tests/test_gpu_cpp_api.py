"""Runs the C++ drop-in API test (tests/cpp/test_api.cpp, built by
__graft_entry__.build()) on the GPU: Cheddar's C++ entry points used the way
the reference's own tests use them, checked bit-exactly against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(__file__), "cpp", "_build", "test_api")


def test_cpp_api():
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/_build/test_api is missing: run "
                    "__graft_entry__.build() first")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASS" in r.stdout
