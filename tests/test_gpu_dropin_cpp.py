"""Runs tests/cpp/build/test_dropin: the C++ drop-in (kokoro_decoder_backward.h)
driven as the reference's own test drives it (N = 1, (C, 1) affines, its
miniature shapes, seeds and finite-difference tolerances) on the GPU,
against the oracle's atoms, with the inference twins and the producer step.
The binary is built with the libraries by __graft_entry__.build()."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "build", "test_dropin")


def test_cpp_drop_in():
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
