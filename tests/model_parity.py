"""Whole-decoder parity helpers shared by the GPU model tests: run the HIP
model (kdec_model through the C ABI) and the CPU oracle model on identical
parameters and inputs, utterance by utterance on the oracle side, and
compare the waveform, every parameter grad, the AdaIN affine grads the
reference returns and d(style).

Bars: waveform rel-L2 <= 1e-5; every grad rel-L2 <= 1e-4, with an absolute
floor of 1e-6 * sqrt(size) (and, for a conv bias that feeds an instance
norm, whose exact grad is zero, 1e-7 times the layer's weight-grad norm).
Each comparison's rel-L2 and max-abs error are kept in the report.

The leaky ReLUs are the decoder's only non-smooth points: an input within
rounding of zero can fall on opposite sides of the kink in two float
evaluations, and the one element's different slope moves every grad
upstream of it by about (its share of the grad norm), e.g. 2e-3 for one of
the 983 168 spectral-head inputs at T = 64. So the oracle takes every leaky
site's branch from the GPU's own inputs at that site
(kdec_model_leaky_input -> OracleModel.set_kinks): both sides are then
differentiated on the same linear piece, and the report counts the elements
whose branch this reconciled ("kink_flips"). That reconciliation is bounded:
at every element whose branch it overrode, the oracle's own input must lie
within KINK_TOL times the site's rms of zero (a rounding-level disagreement,
not a sign error upstream), each site's inputs must agree to the forward bar
(rel-L2 <= 1e-5), and at most KINK_FRAC of a site's elements may flip.

Every comparison is also appended to REPORT (what, rel-L2, max-abs, and the
flip statistics), which tests/conftest.py writes out as JSON lines when
KDEC_PARITY_REPORT names a file.
"""
from __future__ import annotations

import numpy as np

import oracle_lib as O
from brosoundml_amd import config as C
from brosoundml_amd import synth

FWD_TOL = 1e-5
GRAD_TOL = 1e-4
KINK_TOL = 1e-5   # |oracle's own input| / site rms at a reconciled element
KINK_FRAC = 1e-4  # reconciled elements per site element

REPORT = []


def record(what, rel=None, maxabs=None, **extra):
    """One parity figure for the per-config report."""
    REPORT.append(dict(what=what, rel_l2=rel, max_abs=maxabs, **extra))


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b))) if a.size else 0.0


def inputs(cfg, N, T, tag, unvoiced=0.0):
    return synth.decoder_inputs(cfg, N, T, tag, unvoiced)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def oracle_har_of(cfg, params, F0):
    """The oracle's harmonic source (HarmonicSource::forward) for one utterance."""
    g = "decoder.module.generator.m_source.l_linear."
    us = C.upsample_prod(cfg) * cfg["hop"]
    har, _ = O.harmonic_source(F0, params[g + "weight"], params[g + "bias"], cfg["harmonic_num"],
                               cfg["sample_rate"], us, cfg["n_fft"], cfg["hop"])
    return har


def run_pair(ctx, cfg, N, T, tag, wgrad=True, dalpha=True, lora=None, unvoiced=0.0, params=None,
             oracle_har=True, kinks=True, split=False):
    """Forward + backward on both sides. oracle_har: both sides take the
    oracle's harmonic-source output (the model's own is compared separately,
    since the atan2 of a near-empty STFT bin is noise in any float
    evaluation and the phase channels enter the noise convs at full
    weight). split: the model's two half-batch chains, or one (the default)."""
    import torch
    from brosoundml_amd import native
    m = native.Model(ctx, cfg)
    m.set_batch_split(split)
    shapes = m.param_shapes()
    om = O.OracleModel(cfg)
    assert shapes == om.param_shapes()
    if params is None:
        params = synth.init_params(shapes)
    m.set_params(params)
    om.set_params(params)
    asr, F0, Nn, style, dA = inputs(cfg, N, T, tag, unvoiced)
    units = om.units()
    if lora:  # DecoderLora adapters on every unit, a gate per utterance
        rank, scale = lora
        S = cfg["style_dim"]
        m.lora_enable(rank, scale)
        om.lora_enable(rank, scale)
        offs = [u[2] for u in m.units()]
        A = synth.normal(f"{tag}.loraA", (len(units) * rank, S), 0.2)
        B = synth.normal(f"{tag}.loraB", (m.affine_rows(), rank), 0.2)
        gates = synth.normal(f"{tag}.gate", (N, rank), 1.0)
        m.lora_set(A, B)
        for i, (_, c) in enumerate(units):
            om.lora_set(i, A[i * rank:(i + 1) * rank], B[offs[i]:offs[i] + 2 * c])
        ref_dA, ref_dB, ref_dG = np.zeros_like(A, np.float64), np.zeros_like(B, np.float64), []

    # the oracle's harmonic source, one utterance at a time
    ref_har = [oracle_har_of(cfg, params, F0[n]) for n in range(N)]

    # GPU first: its leaky-site inputs fix the oracle's branch at every kink
    t_asr, t_F0, t_N, t_style = dev(asr), dev(F0), dev(Nn), dev(style)
    t_har = dev(np.stack(ref_har)) if oracle_har else None
    if lora:
        t_gate = dev(gates)
        t_dG = torch.zeros_like(t_gate)
        m.lora_gate(t_gate, t_dG)
    m.zero_grad()
    audio = m.forward(t_asr, t_F0, t_N, t_style, T, har=t_har)
    pre = m.leaky_inputs() if kinks else None
    dstyle = torch.empty_like(t_style)
    t_dA = dev(dA)
    m.backward(t_dA, wgrad=wgrad, dalpha=dalpha, dstyle=dstyle)
    torch.cuda.synchronize()

    # oracle, utterance by utterance
    ref_audio, ref_dstyle, ref_aff, flips, kink_stats = [], [], [], [], []
    ref_grads = {n: np.zeros(int(np.prod(s))) for n, s in shapes.items()}
    for n in range(N):
        om.zero_grad()
        if pre is not None:
            om.set_kinks([p[n] for p in pre])
        if lora:
            om.lora_gate(gates[n])
        a = om.forward(asr[n], F0[n], Nn[n], style[n], T, har=ref_har[n] if oracle_har else None)
        flips.append(om.kink_flips())
        if pre is not None:
            kink_stats.append(kink_check([p[n] for p in pre], om))
        ref_audio.append(a)
        ref_dstyle.append(om.backward(dA[n], wgrad=wgrad, dalpha=dalpha, dstyle=True))
        for name, s in shapes.items():
            ref_grads[name] += om.grad(name, s)
        ref_aff.append([om.affine(i, c) for i, (_, c) in enumerate(units)])
        if lora:
            for i, (_, c) in enumerate(units):
                gA, gB = om.lora_grads(i, c)
                ref_dA[i * rank:(i + 1) * rank] += gA
                ref_dB[offs[i]:offs[i] + 2 * c] += gB
            ref_dG.append(om.lora_dgate())
    om.clear_kinks()
    got_grads = {n: m.grad(n, s) for n, s in shapes.items()}
    gb, dgb = m.affines(N)
    r = dict(m=m, om=om, shapes=shapes, audio=audio.cpu().numpy(), ref_audio=np.stack(ref_audio),
             ref_har=np.stack(ref_har), dstyle=dstyle.cpu().numpy(), ref_dstyle=np.stack(ref_dstyle),
             grads=got_grads, ref_grads=ref_grads, dgb=dgb, ref_aff=ref_aff, units=m.units(),
             oracle_units=om.units(), inputs=(asr, F0, Nn, style, dA), params=params, kink_flips=flips,
             kink_stats=kink_stats)
    if lora:
        gA, gB = m.lora_grads()
        r.update(lora_got=(gA, gB, t_dG.cpu().numpy()), lora_ref=(ref_dA, ref_dB, np.stack(ref_dG)))
    return r


def kink_check(gpu_pre, om):
    """Bounds the branch reconciliation at every leaky site of one utterance:
    gpu_pre are the GPU's inputs at each site, the oracle's own are read back
    after its (reconciled) forward. Returns (flips, elements, worst |x|/rms at
    a flipped element, worst site rel-L2); asserts the bars."""
    flips = elems = 0
    worst_mag = worst_rel = 0.0
    for site, g in enumerate(gpu_pre):
        o = om.leaky_input(site).astype(np.float64)
        g = np.asarray(g, np.float64).ravel()
        assert o.size == g.size, (site, o.size, g.size)
        rms = float(np.sqrt(np.mean(o * o))) or 1.0
        flipped = (o > 0) != (g > 0)
        nf = int(flipped.sum())
        mag = float(np.max(np.abs(o[flipped]))) / rms if nf else 0.0
        rel = rel_l2(g, o)
        assert rel <= FWD_TOL, f"leaky site {site}: GPU vs oracle inputs rel-L2 {rel:.3e}"
        assert mag <= KINK_TOL, f"leaky site {site}: reconciled element at {mag:.3e} x rms from zero"
        assert nf <= KINK_FRAC * o.size, f"leaky site {site}: {nf} of {o.size} elements reconciled"
        flips += nf
        elems += o.size
        worst_mag, worst_rel = max(worst_mag, mag), max(worst_rel, rel)
    return flips, elems, worst_mag, worst_rel


def grad_errors(grads, ref_grads, wgrad=True):
    """[(err/tol, name, rel-L2, max-abs, nonzero)] over every parameter grad. The bar:
    rel-L2 <= GRAD_TOL with an absolute floor of 1e-6 * sqrt(size); a bias
    in front of an instance norm, whose exact grad is zero, also gets 1e-7
    times its layer's weight-grad norm. Without weight grads only the snake
    alphas may be nonzero."""
    worst = []
    for name, ref in ref_grads.items():
        got = grads[name].astype(np.float64)
        err = np.linalg.norm(got - ref)
        tol = GRAD_TOL * np.linalg.norm(ref) + 1e-6 * np.sqrt(ref.size)
        wname = name[:-len(".bias")] + ".weight"
        if name.endswith(".bias") and wname in ref_grads:
            # a bias in front of an instance norm has an identically zero
            # grad; what remains is float rounding of a cancelling sum, which
            # scales with the layer's weight grad
            tol += 1e-7 * np.linalg.norm(ref_grads[wname])
        # (err/tol, name, rel-L2, max-abs, not identically zero)
        worst.append((err / max(tol, 1e-30), name, rel_l2(got, ref), max_abs(got, ref),
                      GRAD_TOL * np.linalg.norm(ref) > 1e-6 * np.sqrt(ref.size)))
        if not wgrad and ".alpha" not in name:
            assert not np.any(got), f"{name}: grad produced in reference semantics"
    return worst


def record_grads(name, worst):
    """Records the worst rel-L2 over the grads that are not identically zero
    (a conv bias in front of an instance norm has an exact grad of zero, so
    only its absolute error means anything: recorded apart) and the worst
    error over the bar."""
    nz = [w for w in worst if w[4]]
    zero = [w for w in worst if not w[4]]
    top = max(worst)
    extra = dict(worst_err_over_tol=top[0], worst_err_over_tol_param=top[1])
    rel = mx = None
    if nz:  # (none in the reference semantics without alpha grads)
        w = max(nz, key=lambda t: t[2])
        rel, mx = w[2], w[3]
        extra["param"] = w[1]
    if zero:
        z = max(zero, key=lambda t: t[3])
        extra.update(zero_grads=len(zero), zero_grads_worst_max_abs=z[3], zero_grads_worst_param=z[1])
    record(f"{name} parameter grads ({len(worst)}; worst rel-L2)", rel, mx, **extra)


def check_pair(r, wgrad=True, name=None):
    """Asserts the bars; returns a report {what: (rel-L2, max-abs)} with the
    worst grads. With a name, each figure goes to REPORT before its bar is
    asserted."""
    rec = record if name else (lambda *a, **k: None)
    rep = {"kink_flips": r.get("kink_flips")}
    ks = r.get("kink_stats") or []
    if ks:
        rep["kink"] = dict(flips=sum(k[0] for k in ks), elements=sum(k[1] for k in ks),
                           worst_abs_over_rms=max(k[2] for k in ks), worst_site_rel_l2=max(k[3] for k in ks))
    e = rel_l2(r["audio"], r["ref_audio"])
    rep["waveform"] = (e, max_abs(r["audio"], r["ref_audio"]))
    rec(f"{name} waveform", *rep["waveform"], **({"kink": rep["kink"]} if ks else {}))
    assert e <= FWD_TOL, f"waveform rel-L2 {e:.3e} (max-abs {rep['waveform'][1]:.3e})"
    assert [u[0] for u in r["units"]] == [u[0] for u in r["oracle_units"]]
    # affine grads (the reference semantics' outputs)
    worst_aff = (0.0, "", 0.0)
    for n, aff in enumerate(r["ref_aff"]):
        for (uname, Cc, off), (_, _, dg, db) in zip(r["units"], aff):
            got = r["dgb"][n, off:off + 2 * Cc]
            ref = np.concatenate([dg, db])
            err = np.linalg.norm(got - ref)
            tol = GRAD_TOL * np.linalg.norm(ref) + 1e-6 * np.sqrt(ref.size)
            worst_aff = max(worst_aff, (err / tol, uname, max_abs(got, ref)))
    rep["affine_grads_worst_err_over_tol"] = worst_aff
    rec(f"{name} AdaIN affine grads (worst unit err/tol)", None, worst_aff[2], err_over_tol=worst_aff[0],
        unit=worst_aff[1])
    assert worst_aff[0] <= 1.0, worst_aff
    e = rel_l2(r["dstyle"], r["ref_dstyle"])
    rep["dstyle"] = (e, max_abs(r["dstyle"], r["ref_dstyle"]))
    rec(f"{name} d(style)", *rep["dstyle"])
    assert e <= GRAD_TOL, f"d(style) rel-L2 {e:.3e}"
    worst = grad_errors(r["grads"], r["ref_grads"], wgrad)
    worst.sort(reverse=True)
    rep["grads_worst"] = worst[:3]
    if name:
        record_grads(name, worst)
    assert worst[0][0] <= 1.0, worst[:5]
    return rep


def check_har(got, ref, n_fft, what="harmonic source"):
    """Magnitude channels at rel-L2 1e-5 and max-abs reported; phase channels
    (atan2) only where the bin holds energy, as a wrapped difference."""
    F = n_fft // 2 + 1
    got = np.asarray(got, np.float64).reshape(F * 2, -1)
    ref = np.asarray(ref, np.float64).reshape(F * 2, -1)
    e = rel_l2(got[:F], ref[:F])
    assert e <= 1e-5, f"{what} magnitude rel-L2 {e:.3e} (max-abs {max_abs(got[:F], ref[:F]):.3e})"
    strong = ref[:F] > 1e-3 * ref[:F].max()
    dphi = np.angle(np.exp(1j * (got[F:][strong] - ref[F:][strong])))
    worst = float(np.max(np.abs(dphi))) if dphi.size else 0.0
    assert worst < 1e-3, f"{what} phase error {worst:.3e} on strong bins"
    return dict(mag=(e, max_abs(got[:F], ref[:F])), phase_strong_max=worst, strong_frac=float(strong.mean()))
