"""Runs the C++ facade tests (tests/cpp/test_facade.cpp) built by
__graft_entry__.build() (make -C tests/cpp)."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "test_facade")


def _run(args):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: build with `python -c 'import __graft_entry__ as g; g.build()'`")
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout


def test_facade_host_only():
    _run(["--cpu"])


@pytest.mark.gpu
def test_facade_on_gpu(cuda):
    _run([])
