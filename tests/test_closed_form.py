"""Closed-form special cases of the decoder's composition on the CPU oracle
(tests/cpp/closed_forms.hpp, run by tests/cpp/build/test_closed_form): the
AdainResBlk1d shortcut and /sqrt(2), the 0.2 / 0.1 / 0.01 leaky slopes, the
AdaINResBlock1 skip, the generator's 1/K resblock mean and noise-branch add,
the backbone's cat orders and the reflect pad side, each from a construction
whose output is known exactly. The same cases run through the HIP drop-in in
tests/cpp/test_dropin.cpp. Each case was checked to fail for the slip it
targets, planted in a copy of the oracle.
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")


def test_closed_forms_on_the_oracle():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-j8"], check=True)
    subprocess.run(["make", "-s", "-C", CPP, "build/test_closed_form"], check=True)
    r = subprocess.run([os.path.join(CPP, "build", "test_closed_form")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "0 failure(s)" in r.stdout
