"""The oracle's composed decoder against an independent restatement: torch
float64 modules in the upstream Kokoro iSTFTNet order, differentiated by
autograd (tests/torch_ref.py). The oracle follows the reference's `_train`
assemblies and its hand-written backward; agreement of the waveform, every
AdaIN affine grad, d(style) and every parameter grad pins the composition
(the /sqrt(2) residual, the 1/K resblock mean, the leaky slopes, the cat
order, the left reflect pad, the nearest-2x shortcut, the AdaINResBlock1
skip) and the backward independently of the oracle's own derivation.

Both sides take the oracle's harmonic source. Bars: 1e-5 rel-L2 on the
waveform and on every grad whose norm is above float noise (the conv biases
in front of an instance norm have an exactly zero grad; their float residue
is bounded relative to the layer's weight grad instead).
"""
import numpy as np
import pytest

import oracle_lib as O
import torch_ref
from brosoundml_amd import config as C
from brosoundml_amd import synth
from model_parity import oracle_har_of, rel_l2

TOL = 1e-5


@pytest.mark.parametrize("name,T", [("TINY", 6), ("SMALL", 6), ("KOKORO", 16)])
def test_oracle_matches_torch_restatement(name, T):
    cfg = getattr(C, name)
    om = O.OracleModel(cfg)
    shapes = om.param_shapes()
    params = synth.init_params(shapes)
    om.set_params(params)
    asr, F0, Nn, st, dA = synth.decoder_inputs(cfg, 1, T, f"torchref.{name}", unvoiced=0.2)
    har = oracle_har_of(cfg, params, F0[0])
    a = om.forward(asr[0], F0[0], Nn[0], st[0], T, har=har)
    ds = om.backward(dA[0])
    ref = torch_ref.Ref(cfg, params)
    ta, tds, tg, taff = ref.run(asr, F0, Nn, st, har[None], dA)
    assert rel_l2(a, ta[0]) <= TOL
    assert rel_l2(ds, tds[0]) <= TOL
    units = om.units()
    assert sorted(n for n, _ in units) == sorted(taff)
    for i, (n, c) in enumerate(units):
        _, _, dg, db = om.affine(i, c)
        e = rel_l2(np.concatenate([dg, db]), np.concatenate([taff[n][0][0], taff[n][1][0]]))
        assert e <= TOL, (n, e)
    for n, s in shapes.items():
        if "m_source" in n:
            continue  # forward-only
        g, r = om.grad(n, s), tg[n]
        w = n[:-len(".bias")] + ".weight"
        if n.endswith(".bias") and w in tg and np.linalg.norm(r) < 1e-9 * max(np.linalg.norm(tg[w]), 1.0):
            assert np.linalg.norm(g) <= 1e-6 * np.linalg.norm(tg[w]), n  # exactly zero in exact arithmetic
            continue
        assert rel_l2(g, r) <= TOL, (n, rel_l2(g, r))
