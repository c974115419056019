"""DecoderLora on the GPU (kdec_dlora_*, kdec_lora_gate_*, kdec_adam_step)
against the oracle: the gate kernels and Adam against oracle/decoder_lora.py,
the whole DecoderLora forward / backward against the oracle model with the
same adapters and gate (the reference's test_kokoro_decoder_backward.cpp:
499-577 checks: neutral identity at cond = 0, every LoRA and gate grad, an
exact checkpoint round trip), and the ELRA1 file against its layout."""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O
from brosoundml_amd import config as C
from brosoundml_amd import synth

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import decoder_lora as DL  # noqa: E402

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def f32(x):
    # the ABI's hyper-parameters are floats (as DecoderLora::adam_step's): the
    # oracle takes the same rounded values
    return float(np.float32(x))


@pytest.fixture(scope="module")
def ctx():
    from brosoundml_amd import native
    return native.Context(0)


def test_gate_kernels(ctx):
    from brosoundml_amd import native
    P = native.ptr
    r = np.random.default_rng(1)
    N, I, H, R = 3, 3, 16, 4
    W1, W2 = r.normal(size=(H, I)), r.normal(size=(R, H))
    v, dG = r.normal(size=(N, I)), r.normal(size=(N, R))
    tW1, tW2, tv, tdG = dev(W1), dev(W2), dev(v), dev(dG)
    act, g = torch.empty(N, H, device="cuda"), torch.empty(N, R, device="cuda")
    dW1, dW2 = torch.full((H, I), 0.5, device="cuda"), torch.full((R, H), -0.25, device="cuda")
    ctx.call("kdec_lora_gate_fwd", P(tW1), P(tW2), P(tv), I, N, I, H, R, P(act), P(g), R)
    ctx.call("kdec_lora_gate_bwd", P(tW2), P(tv), I, P(act), P(tdG), R, N, I, H, R, P(dW1), P(dW2))
    torch.cuda.synchronize()
    g_ref, act_ref = DL.gate_forward(np.float32(W1), np.float32(W2), np.float32(v))
    dW1_ref, dW2_ref = DL.gate_backward(np.float32(W2), np.float32(v), act_ref, np.float32(dG))
    assert rel_l2(g.cpu(), g_ref) <= 1e-6
    assert rel_l2(act.cpu(), act_ref) <= 1e-6
    # accumulates onto what is there
    assert rel_l2(dW1.cpu(), dW1_ref + 0.5) <= 1e-6
    assert rel_l2(dW2.cpu(), dW2_ref - 0.25) <= 1e-6
    with pytest.raises(native.KdecError):
        ctx.call("kdec_lora_gate_fwd", P(tW1), P(tW2), P(tv), 1, N, I, H, R, P(act), P(g), R)


def test_adam_kernel(ctx):
    from brosoundml_amd import native
    P = native.ptr
    r = np.random.default_rng(2)
    n = 5000
    p, m, v = r.normal(size=n), np.zeros(n), np.zeros(n)
    tp, tm, tv = dev(p), dev(m), dev(v)
    for step in range(1, 4):
        g = r.normal(size=n)
        ctx.call("kdec_adam_step", P(tp), P(dev(g)), P(tm), P(tv), n, 1e-3, 0.9, 0.999, 1e-8, step)
        p, m, v = DL.adam_step(p, np.float32(g).astype(np.float64), m, v, f32(1e-3), f32(0.9), f32(0.999),
                               f32(1e-8), step)
    torch.cuda.synchronize()
    assert rel_l2(tp.cpu(), p) <= 1e-6
    assert rel_l2(tm.cpu(), m) <= 1e-6
    assert rel_l2(tv.cpu(), v) <= 1e-6
    with pytest.raises(native.KdecError):
        ctx.call("kdec_adam_step", P(tp), P(dev(g)), P(tm), P(tv), n, 1e-3, 0.9, 0.999, 1e-8, 0)


def make_model(ctx, cfg, tag, with_params=False):
    from brosoundml_amd import native
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    params = synth.init_params(shapes)
    m.set_params(params)
    om = O.OracleModel(cfg)
    om.set_params(params)
    return (m, om, params) if with_params else (m, om)


def inputs(cfg, N, T, tag):
    S = cfg["style_dim"]
    asr = synth.normal(f"{tag}.asr", (N, cfg["asr_dim"], T))
    F0 = synth.uniform(f"{tag}.F0", (N, 2 * T), 80.0, 300.0)
    Nn = synth.normal(f"{tag}.N", (N, 2 * T), 0.5)
    ref_s = synth.normal(f"{tag}.ref_s", (N, 2 * S), 0.3)
    cond = synth.normal(f"{tag}.cond", (N, 3), 0.6)
    dA = synth.normal(f"{tag}.daudio", (N, C.lengths(cfg, T)["audio"]), 1.0)
    return asr, F0, Nn, ref_s, cond, dA


def test_neutral_identity(ctx):
    # cond = 0 closes the gate: the base decoder's waveform (g(0) = 0 exactly)
    from brosoundml_amd import native
    cfg, N, T = C.TINY, 2, 4
    m, om = make_model(ctx, cfg, "dl.id")
    d = native.DecoderLora(m, 4, 1.0, seed=123)
    d.set("W2", np.random.default_rng(4).uniform(-0.2, 0.2, (4, 16)))  # open weights, closed condition
    asr, F0, Nn, ref_s, _, _ = inputs(cfg, N, T, "dl.id")
    S = cfg["style_dim"]
    t = [dev(a) for a in (asr, F0, Nn, ref_s)]
    base = m.forward(t[0], t[1], t[2], t[3][:, :S].contiguous(), T).clone()
    import ctypes
    har = torch.empty(N, (cfg["n_fft"] + 2) * C.lengths(cfg, T)["frames"], device="cuda")
    hp = ctx.L.kdec_model_har(m.h)  # the base forward's harmonic source output
    ctx.check(ctx.L.kdec_axpby(ctx.h, 1.0, ctypes.c_void_p(hp), har.shape[1], 0.0, None, 0, native.ptr(har),
                               har.shape[1], N, har.shape[1]))
    audio = d.forward(t[0], t[1], t[2], t[3], T, torch.zeros(N, 3, device="cuda"), har=har)
    torch.cuda.synchronize()
    err = (audio - base).abs().max().item()
    assert err <= 1e-6 * base.abs().max().item(), err
    # without har the DecoderLora runs the model's harmonic source: the same bits
    audio2 = d.forward(t[0], t[1], t[2], t[3], T, torch.zeros(N, 3, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(audio, audio2)


@pytest.mark.parametrize("cfg_name,N,T", [("TINY", 1, 4), ("TINY", 2, 4), ("SMALL", 2, 6), ("KOKORO", 2, 64)])
def test_grads_against_oracle(ctx, cfg_name, N, T):
    # The GPU runs first: its leaky-site inputs (kdec_dlora_leaky_input) fix
    # the oracle's branch at every kink, bounded as in the model tests
    # (model_parity.kink_check); both sides take the oracle's harmonic source.
    from brosoundml_amd import native
    from model_parity import kink_check, oracle_har_of, record
    cfg, rank, scale = getattr(C, cfg_name), 3, 0.7
    m, om, params = make_model(ctx, cfg, "dl.g", with_params=True)
    d = native.DecoderLora(m, rank, scale, seed=77)
    W2 = np.random.default_rng(8).uniform(-0.3, 0.3, (rank, 16)).astype(np.float32)
    d.set("W2", W2)
    A, B, W1 = d.get("A"), d.get("B"), d.get("W1")
    asr, F0, Nn, ref_s, cond, dA = inputs(cfg, N, T, f"dl.g{cfg_name}{N}")
    S = cfg["style_dim"]
    units = om.units()
    offs = [u[2] for u in m.units()]
    har = [oracle_har_of(cfg, params, F0[n]) for n in range(N)]
    t = [dev(a) for a in (asr, F0, Nn, ref_s, cond)]
    d.zero_grad()
    audio = d.forward(t[0], t[1], t[2], t[3], T, t[4], har=dev(np.stack(har)))
    pre = d.leaky_inputs()
    d.backward(dev(dA))
    torch.cuda.synchronize()
    om.lora_enable(rank, scale)
    for i, (_, c) in enumerate(units):
        om.lora_set(i, A[i * rank:(i + 1) * rank], B[offs[i]:offs[i] + 2 * c])
    ref_audio, kinks = [], []
    ref_dA, ref_dB = np.zeros_like(A, np.float64), np.zeros_like(B, np.float64)
    ref_dW1, ref_dW2 = np.zeros((16, 3)), np.zeros((rank, 16))
    for n in range(N):
        g, act = DL.gate_forward(W1, W2, cond[n].astype(np.float32))
        om.lora_gate(g[0])
        om.zero_grad()
        om.set_kinks([p[n] for p in pre])
        ref_audio.append(om.forward(asr[n], F0[n], Nn[n], ref_s[n, :S], T, har=har[n]))
        kinks.append(kink_check([p[n] for p in pre], om))
        om.backward(dA[n], wgrad=False, dalpha=False, dstyle=False)
        for i, (_, c) in enumerate(units):
            gA, gB = om.lora_grads(i, c)
            ref_dA[i * rank:(i + 1) * rank] += gA
            ref_dB[offs[i]:offs[i] + 2 * c] += gB
        dW1n, dW2n = DL.gate_backward(W2, cond[n].astype(np.float32), act, om.lora_dgate())
        ref_dW1 += dW1n
        ref_dW2 += dW2n
    om.clear_kinks()
    tag = f"DecoderLora {cfg_name} N={N} T={T}"
    e = rel_l2(audio.cpu(), np.stack(ref_audio))
    record(f"{tag} waveform", e, float(np.max(np.abs(audio.cpu().numpy() - np.stack(ref_audio)))),
           kink=dict(flips=sum(k[0] for k in kinks), elements=sum(k[1] for k in kinks),
                     worst_abs_over_rms=max(k[2] for k in kinks)))
    assert e <= 1e-5, f"waveform rel-L2 {e:.3e}"
    for name, ref in (("dA", ref_dA), ("dB", ref_dB), ("dW1", ref_dW1), ("dW2", ref_dW2)):
        got = d.get(name)
        e = rel_l2(got, ref)
        record(f"{tag} {name}", e, float(np.max(np.abs(got - ref))))
        print(f"{tag} {name}: rel-L2 {e:.3e}", flush=True)
        assert e <= 1e-4, f"{name} rel-L2 {e:.3e}"

    # one Adam step over every trainable, against the oracle's on the same grads
    pre = {k: d.get(k).astype(np.float64) for k in ("A", "B", "W1", "W2")}
    grads = {k: d.get("d" + k).astype(np.float64) for k in ("A", "B", "W1", "W2")}
    d.adam_step(2e-3)
    for k in pre:
        want, _, _ = DL.adam_step(pre[k], grads[k], 0.0, 0.0, f32(2e-3), f32(0.9), f32(0.999), f32(1e-8), 1)
        assert rel_l2(d.get(k), want) <= 1e-6, k


def test_checkpoint_round_trip(ctx, tmp_path):
    from brosoundml_amd import native
    cfg, rank = C.TINY, 4
    m, _ = make_model(ctx, cfg, "dl.ck")
    d = native.DecoderLora(m, rank, 0.8, seed=123)
    d.set("W2", np.random.default_rng(9).normal(size=(rank, 16)))
    path = str(tmp_path / "decoder_lora_test.ckpt")
    d.save(path)
    # the file is the reference's ELRA1 layout
    f = DL.elra1_parse(open(path, "rb").read())
    S = cfg["style_dim"]
    units = m.units()
    A, B = d.get("A"), d.get("B")
    assert (f["rank"], f["style_dim"], f["gate_hidden"]) == (rank, S, 16)
    assert np.float32(f["scale"]) == np.float32(0.8)
    np.testing.assert_array_equal(f["W1"], d.get("W1"))
    np.testing.assert_array_equal(f["W2"], d.get("W2"))
    assert len(f["adapters"]) == len(units)
    for i, ((_, c, off), (C_, A_, B_)) in enumerate(zip(units, f["adapters"])):
        assert C_ == c
        np.testing.assert_array_equal(A_, A[i * rank:(i + 1) * rank])
        np.testing.assert_array_equal(B_, B[off:off + 2 * c])
    # a differently seeded DecoderLora restores every parameter exactly
    d2 = native.DecoderLora(m, rank, 1.0, seed=999)
    assert not np.array_equal(d2.get("A"), A)
    d2.load(path)
    for k in ("A", "B", "W1", "W2"):
        np.testing.assert_array_equal(d2.get(k), d.get(k))
    assert np.float32(d2.scale) == np.float32(0.8)
    # errors: bad magic, another rank, a missing file
    bad = str(tmp_path / "bad.ckpt")
    data = open(path, "rb").read()
    open(bad, "wb").write(b"ELRA2" + data[5:])
    with pytest.raises(native.KdecError, match="bad magic"):
        d2.load(bad)
    d3 = native.DecoderLora(m, rank + 1, 1.0, seed=5)
    with pytest.raises(native.KdecError, match="architecture mismatch"):
        d3.load(path)
    with pytest.raises(native.KdecError, match="cannot open"):
        d2.load(str(tmp_path / "missing.ckpt"))
