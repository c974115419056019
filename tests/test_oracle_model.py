"""Pins the oracle's assemblies and their extensions by finite differences.

The reference verifies its backward atoms with directional finite differences
of an MSE loss (tests/test_kokoro_decoder_backward.cpp:97-125). The same check
runs here on the whole decoder - style projection, backbone, generator,
spectral head - for every parameter tensor (conv / convT / pool weights and
biases, snake alphas, the style fc) and for the style vector itself, so the
extensions the reference does not compute (wgrad, dalpha, d(style)) are pinned
by the forward alone.

The checks run on the oracle's FP64 shadow (the same source compiled with
double storage), where a central difference with step 1e-5 is accurate to
~1e-7 relative: far tighter than the reference's float tolerances (abs 4e-3,
rel 8e-3), which a whole-decoder loss with exp() and leaky-ReLU kinks cannot
meet in float. The float oracle is then pinned to its FP64 twin.
"""
import numpy as np
import pytest

import oracle_lib as O
from brosoundml_amd import config as C
from brosoundml_amd import synth

T = 4


def make_inputs(cfg, T, tag="fd"):
    L = C.lengths(cfg, T)
    asr = synth.normal(f"{tag}.asr", (cfg["asr_dim"], T))
    F0 = synth.uniform(f"{tag}.F0", (2 * T,), 80.0, 300.0)
    N = synth.normal(f"{tag}.N", (2 * T,), 0.5)
    style = synth.normal(f"{tag}.style", (cfg["style_dim"],), 0.3)
    target = synth.normal(f"{tag}.target", (L["audio"],), 0.3).astype(np.float64)
    return asr, F0, N, style, target


def loss64(m, inputs, har, style=None):
    asr, F0, N, st, target = inputs
    a = m.forward_f64(asr, F0, N, st if style is None else style, T, har)
    return 0.5 * np.sum((a - target) ** 2), a


def shared_har(cfg):
    # The harmonic source's phase channels are atan2 of near-zero STFT bins
    # wherever a bin holds no harmonic energy, so float and FP64 evaluations
    # legitimately disagree there; both models take the float oracle's har.
    m = O.OracleModel(cfg)
    m.set_params(synth.init_params(m.param_shapes()))
    m.forward(*make_inputs(cfg, T)[:4], T)
    return m.har()


def run_model(cfg, fp64):
    m = O.OracleModel(cfg, fp64=fp64)
    shapes = m.param_shapes()
    params = synth.init_params(shapes)
    m.set_params(params)
    inputs = make_inputs(cfg, T)
    har = shared_har(cfg)
    L0, audio = loss64(m, inputs, har)
    m.zero_grad()
    dstyle = m.backward((audio - inputs[4]).astype(np.float32))
    grads = {n: m.grad(n, s) for n, s in shapes.items()}
    return dict(m=m, cfg=cfg, shapes=shapes, params=params, inputs=inputs, har=har,
                grads=grads, dstyle=dstyle, L0=L0, audio=audio)


@pytest.fixture(scope="module")
def tiny64():
    return run_model(C.TINY, True)


@pytest.fixture(scope="module")
def tiny32():
    return run_model(C.TINY, False)


H = 1e-5
TOL = 2e-5


def central(fn, h=H):
    return (fn(h) - fn(-h)) / (2 * h)


def directional(r, name, seed):
    m, params = r["m"], r["params"]
    v = synth.uniform(f"dir.{name}.{seed}", params[name].shape, -1.0, 1.0).astype(np.float64)
    base = params[name].astype(np.float64)

    def loss_at(h):
        m.set_params_f64({name: base + h * v})
        return loss64(m, r["inputs"], r["har"])[0]

    fd = central(loss_at)
    m.set_params({name: params[name]})
    an = float(np.dot(r["grads"][name].astype(np.float64), v.ravel()))
    return an, fd


def test_every_param_has_a_grad_path(tiny64):
    shapes = tiny64["shapes"]
    assert "decoder.module.generator.ups.0.weight" in shapes
    assert "decoder.module.decode.1.pool.weight" in shapes
    assert "decoder.module.generator.resblocks.3.alpha2.2" in shapes
    nonzero = [n for n, g in tiny64["grads"].items() if np.any(g != 0)]
    # l_linear is the forward-only harmonic source: no grad by construction
    missing = [n for n in shapes if n not in nonzero and "m_source" not in n]
    assert not missing, missing


def test_fd_all_params(tiny64):
    fails = []
    for i, name in enumerate(sorted(tiny64["params"])):
        if "m_source" in name:
            continue
        an, fd = directional(tiny64, name, i)
        if abs(an - fd) > TOL * max(abs(an), abs(fd), 1e-2):
            fails.append((name, an, fd))
    assert not fails, fails[:10]


def test_fd_style(tiny64):
    r = tiny64
    style = r["inputs"][3].astype(np.float64)
    v = synth.uniform("dir.style", style.shape, -1.0, 1.0).astype(np.float64)
    fd = central(lambda h: loss64(r["m"], r["inputs"], r["har"], style + h * v)[0])
    an = float(np.dot(r["dstyle"].astype(np.float64), v))
    assert abs(an - fd) <= TOL * max(abs(an), abs(fd), 1e-2), (an, fd)


def test_fd_per_element_style(tiny64):
    # per-element FD on a few style components (tests/test_kokoro_decoder_backward.cpp:81-95)
    r = tiny64
    style = r["inputs"][3].astype(np.float64)
    for j in (0, 5, 11):
        e = np.zeros_like(style)
        e[j] = 1.0
        fd = central(lambda h: loss64(r["m"], r["inputs"], r["har"], style + h * e)[0])
        an = float(r["dstyle"][j])
        assert abs(an - fd) <= TOL * max(abs(an), abs(fd), 1e-2), (j, an, fd)


def test_affine_grads_are_fc_adjoint(tiny64):
    # d fc.bias == [dgamma; dbeta]: the reference's affine grads pass through
    # the style projection unchanged (decoder_lora.cpp:198-207)
    m, grads = tiny64["m"], tiny64["grads"]
    for i, (unit, Cc) in enumerate(m.units()):
        g, b, dg, db = m.affine(i, Cc)
        np.testing.assert_allclose(grads[unit + ".fc.bias"], np.concatenate([dg, db]),
                                   rtol=1e-6, atol=1e-7)


def test_reference_semantics_flags(tiny32):
    # reference semantics (no wgrad / dalpha) give the same affine grads and
    # leave every weight grad at zero
    r = tiny32
    m = r["m"]
    m.forward(*r["inputs"][:4], T, r["har"])
    m.zero_grad()
    m.backward((r["audio"] - r["inputs"][4]).astype(np.float32), wgrad=False, dalpha=False,
               dstyle=False)
    for i, (unit, Cc) in enumerate(m.units()):
        _, _, dg, db = m.affine(i, Cc)
        np.testing.assert_allclose(r["grads"][unit + ".fc.bias"], np.concatenate([dg, db]),
                                   rtol=1e-6, atol=1e-7)
    for name in ("decoder.module.generator.resblocks.0.convs1.0.weight",
                 "decoder.module.generator.noise_res.1.alpha1.0",
                 "decoder.module.encode.norm1.fc.weight"):
        assert not np.any(m.grad(name, r["shapes"][name]))


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_float_oracle_matches_fp64_shadow(tiny32, tiny64):
    # the float oracle differs from exact arithmetic only by float storage
    assert rel_l2(tiny32["audio"], tiny64["audio"]) < 1e-5
    assert rel_l2(tiny32["dstyle"], tiny64["dstyle"]) < 1e-4
    # A conv bias in front of an instance norm has an identically zero grad
    # (the mean subtraction cancels it); float leaves ~1e-8 of rounding there,
    # hence the absolute floor.
    for n, g64 in tiny64["grads"].items():
        if "m_source" in n:
            continue
        g32 = tiny32["grads"][n].astype(np.float64)
        err = np.linalg.norm(g32 - g64)
        assert err <= 1e-4 * np.linalg.norm(g64) + 1e-6 * np.sqrt(g64.size), (n, err)


def test_harmonic_source_shapes_and_unvoiced():
    cfg = C.TINY
    L = C.lengths(cfg, T)
    F0 = synth.uniform("hs.F0", (2 * T,), 80.0, 300.0)
    F0[3] = 0.0  # unvoiced frame
    lW = synth.uniform("hs.lW", (9,), -0.3, 0.3)
    lb = np.array([0.05], np.float32)
    har, frames = O.harmonic_source(F0, lW, lb, 8, 24000, C.upsample_prod(cfg) * cfg["hop"],
                                    cfg["n_fft"], cfg["hop"])
    assert frames == L["frames"]
    F = cfg["n_fft"] // 2 + 1
    mag = har[: F * frames].reshape(F, frames)
    assert np.all(mag >= 0)
    ph = har[F * frames:].reshape(F, frames)
    assert np.all(np.abs(ph) <= np.pi + 1e-6)


def test_harmonic_source_closed_form():
    # A constant F0 drives harmonic h at frequency (h+1)*F0; with a single
    # active harmonic (lW = e_0) and a small amplitude, tanh is ~linear, so the
    # STFT magnitude peaks at the bin nearest F0 * n_fft / sample_rate.
    n_fft, hop, sr = 20, 5, 24000
    f0 = 3600.0  # bin 3 exactly
    frames_in = 8
    F0 = np.full(frames_in, f0, np.float32)
    lW = np.zeros(9, np.float32)
    lW[0] = 1.0
    har, frames = O.harmonic_source(F0, lW, np.zeros(1, np.float32), 8, sr, 300, n_fft, hop)
    F = n_fft // 2 + 1
    mag = har[: F * frames].reshape(F, frames)
    mid = mag[:, frames // 4: 3 * frames // 4]
    assert np.all(np.argmax(mid, axis=0) == 3)


@pytest.fixture(scope="module")
def lora64():
    # DecoderLora adapters on every unit (rank 3, scale 0.7) with nonzero A, B
    # and gate, so every LoRA path carries signal
    cfg = C.TINY
    m = O.OracleModel(cfg, fp64=True)
    shapes = m.param_shapes()
    params = synth.init_params(shapes)
    m.set_params(params)
    rank, S = 3, cfg["style_dim"]
    m.lora_enable(rank, 0.7)
    units = m.units()
    lora = {}
    for i, (_, Cu) in enumerate(units):
        A = synth.normal(f"lora.A.{i}", (rank, S), 0.2).astype(np.float64)
        B = synth.normal(f"lora.B.{i}", (2 * Cu, rank), 0.2).astype(np.float64)
        m.lora_set(i, A, B)
        lora[i] = (A, B)
    gate = synth.normal("lora.gate", (rank,), 1.0).astype(np.float64)
    m.lora_gate(gate)
    inputs = make_inputs(cfg, T)
    har = shared_har(cfg)
    L0, audio = loss64(m, inputs, har)
    m.zero_grad()
    dstyle = m.backward((audio - inputs[4]).astype(np.float32))
    grads = {i: m.lora_grads(i, Cu) for i, (_, Cu) in enumerate(units)}
    return dict(m=m, units=units, lora=lora, gate=gate, inputs=inputs, har=har, grads=grads,
                dgate=m.lora_dgate(), dstyle=dstyle)


def test_fd_lora_adapters(lora64):
    r = lora64
    m = r["m"]
    fails = []
    for i in (0, 3, len(r["units"]) - 1):
        A, B = r["lora"][i]
        for which, base, an_grad in (("A", A, r["grads"][i][0]), ("B", B, r["grads"][i][1])):
            v = synth.uniform(f"dir.lora.{which}.{i}", base.shape, -1.0, 1.0).astype(np.float64)

            def loss_at(hh, which=which, base=base, v=v):
                m.lora_set(i, **{which: base + hh * v})
                return loss64(m, r["inputs"], r["har"])[0]

            fd = central(loss_at)
            m.lora_set(i, **{which: base})
            an = float(np.sum(an_grad.astype(np.float64) * v))
            if abs(an - fd) > TOL * max(abs(an), abs(fd), 1e-2):
                fails.append((i, which, an, fd))
    assert not fails, fails


def test_fd_lora_gate_and_style(lora64):
    r = lora64
    m = r["m"]
    v = synth.uniform("dir.lora.gate", r["gate"].shape, -1.0, 1.0).astype(np.float64)

    def loss_gate(hh):
        m.lora_gate(r["gate"] + hh * v)
        return loss64(m, r["inputs"], r["har"])[0]

    fd = central(loss_gate)
    m.lora_gate(r["gate"])
    an = float(np.dot(r["dgate"].astype(np.float64), v))
    assert abs(an - fd) <= TOL * max(abs(an), abs(fd), 1e-2), ("gate", an, fd)
    style = r["inputs"][3].astype(np.float64)
    vs = synth.uniform("dir.lora.style", style.shape, -1.0, 1.0).astype(np.float64)
    fd = central(lambda hh: loss64(m, r["inputs"], r["har"], style + hh * vs)[0])
    an = float(np.dot(r["dstyle"].astype(np.float64), vs))
    assert abs(an - fd) <= TOL * max(abs(an), abs(fd), 1e-2), ("style", an, fd)


@pytest.mark.parametrize("name", ["TINY", "SMALL", "KOKORO"])
def test_affine_rows_match_the_units(name):
    # config.affine_rows (the bench's style-projection case) against the
    # oracle model's own AdaIN units
    cfg = getattr(C, name)
    assert C.affine_rows(cfg) == 2 * sum(c for _, c in O.OracleModel(cfg).units())
