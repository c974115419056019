"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: the
same sources built with -fsanitize=address,undefined (oracle/Makefile,
`make sanitize`), driven through a whole-decoder forward + backward with every
extension and the kink masks, plus the standalone ops, in a child process
with the ASan runtime preloaded. Any out-of-bounds access, use after free or
undefined behaviour (signed overflow, misaligned load, bad shift, ...) aborts
the child with a report.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")

CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, {tests!r})
sys.path.insert(0, {root!r})
import oracle_lib as O
from brosoundml_amd import config as C, synth

for name, T in (("TINY", 5), ("SMALL", 4)):
    cfg = getattr(C, name)
    om = O.OracleModel(cfg)
    shapes = om.param_shapes()
    params = synth.init_params(shapes)
    om.set_params(params)
    asr, F0, Nn, st, dA = synth.decoder_inputs(cfg, 1, T, "san." + name, unvoiced=0.3)
    om.zero_grad()
    a = om.forward(asr[0], F0[0], Nn[0], st[0], T)
    om.backward(dA[0])
    # the kink-mask path: the model's own leaky inputs as masks
    om.set_kinks([om.leaky_input(s) for s in range(om.kink_site_count())])
    om.forward(asr[0], F0[0], Nn[0], st[0], T)
    om.backward(dA[0])
    om.clear_kinks()
    for n, s in shapes.items():
        om.grad(n, s)
    assert np.all(np.isfinite(a))
rng = np.random.default_rng(3)
x = rng.normal(size=(3, 50)).astype(np.float32)
W = rng.normal(size=(4, 3 * 5)).astype(np.float32)
y = O.conv1d(x.ravel(), W, None, 3, 50, 4, 5, 2, 3, 2)
O.conv1d_dgrad(W, rng.normal(size=y.size).astype(np.float32), 3, 50, 4, 5, 2, 3, 2)
O.convt1d(x.ravel(), rng.normal(size=(3, 4 * 6)).astype(np.float32), None, 3, 50, 4, 6, 3, 1)
O.harmonic_source(rng.uniform(80, 300, 12).astype(np.float32), rng.normal(size=9).astype(np.float32),
                  np.zeros(1, np.float32), 8, 24000, 60, 20, 5)
print("sanitized oracle run: ok")
"""


def _runtime():
    r = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True, text=True)
    p = r.stdout.strip()
    return p if r.returncode == 0 and os.path.isabs(p) and os.path.exists(p) else None


def test_oracle_under_asan_and_ubsan():
    asan = _runtime()
    if asan is None:
        pytest.skip("no libasan runtime for the host compiler")
    subprocess.run(["make", "-s", "-C", ORACLE, "-j8", "sanitize"], check=True)
    env = dict(os.environ)
    env.update(LD_PRELOAD=asan, KDEC_ORACLE_LIB=os.path.join(ORACLE, "build", "san", "libkdec_oracle.so"),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               OMP_NUM_THREADS="2")
    code = CHILD.format(tests=os.path.join(ROOT, "tests"), root=ROOT)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "sanitized oracle run: ok" in r.stdout
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
