"""Runs tests/cpp/test_attention: the reference's attention tests
(crates/core/src/ops/attention.rs:264-394) restated in C++ against the C++
mirror of the reference interface (include/cfattn.hpp) over libcfattn.so."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_attention")


def test_reference_attention_tests_in_cpp():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: run __graft_entry__.build() first")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
