"""Whole-decoder GPU parity: kdec_model (the C++ drop-in atoms on gfx950)
against the CPU oracle model on identical parameters and inputs.

Checked per utterance: the waveform (rel-L2 <= 1e-5), every parameter grad
(conv / conv-transpose / pool / style-fc weights and biases, snake alphas;
rel-L2 <= 1e-4, with an absolute floor for the identically-zero grads of conv
biases that feed an instance norm), the AdaIN affine grads the reference
returns, and d(style). Both sides take the oracle's harmonic-source output so
the comparison is not exposed to the atan2 of near-empty STFT bins (the
harmonic source itself is compared in test_gpu_ops).
"""
import os

import numpy as np
import pytest

from brosoundml_amd import config as C
from brosoundml_amd import synth
from model_parity import check_pair, inputs, rel_l2, run_pair

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from brosoundml_amd import native
    return native.Context(0)


def test_tiny_full_extension(ctx):
    check_pair(run_pair(ctx, C.TINY, 2, 4, "gm.tiny"), name="TINY N=2 T=4")


def test_tiny_with_lora_adapters(ctx):
    # DecoderLora adapters (rank 3) on every AdaIN unit, one gate per utterance:
    # the waveform, every grad above, and dA, dB and the gate grad
    r = run_pair(ctx, C.TINY, 2, 4, "gm.lora", lora=(3, 0.7))
    check_pair(r)
    for name, got, ref in zip(("dA", "dB", "dG"), r["lora_got"], r["lora_ref"]):
        e = rel_l2(got, ref)
        assert e <= 1e-4, f"LoRA {name} rel-L2 {e:.3e}"


def test_small_full_extension(ctx):
    check_pair(run_pair(ctx, C.SMALL, 2, 6, "gm.small"), name="SMALL N=2 T=6")


def test_reference_semantics_single_utterance(ctx):
    r = run_pair(ctx, C.TINY, 1, 5, "gm.ref", wgrad=False, dalpha=False)
    check_pair(r, wgrad=False)


def test_backward_is_linear_in_daudio(ctx):
    # size-independent property: grads scale with the upstream grad
    from brosoundml_amd import native
    cfg = C.TINY
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    m.set_params(synth.init_params(shapes))
    asr, F0, Nn, style, dA = inputs(cfg, 2, 4, "gm.lin")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn, style)]
    m.forward(*t, 4)
    outs = []
    for scale in (1.0, 2.0):
        m.zero_grad()
        d = dev(dA * scale)
        m.backward(d, wgrad=True, dalpha=True)
        torch.cuda.synchronize()
        outs.append({n: m.grad(n, s) for n, s in shapes.items()})
    for n in shapes:
        if "m_source" in n:
            continue
        np.testing.assert_allclose(outs[1][n], 2.0 * outs[0][n], rtol=1e-5, atol=1e-6)


def test_in_model_harmonic_source_matches_op(ctx):
    # The model runs the harmonic source on a side stream joined before the
    # generator; its waveform must equal, bit for bit, a forward fed the
    # harmonic-source op's output computed on its own. T is long enough that
    # the side-stream work outlasts the (tiny) backbone, so a missing join
    # would show.
    from brosoundml_amd import native
    cfg, N, T = C.TINY, 2, 96
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    params = synth.init_params(shapes)
    m.set_params(params)
    asr, F0, Nn, style, _ = inputs(cfg, N, T, "gm.hs")
    F0[0, 5:9] = 0.0
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn, style)]
    a1 = m.forward(*t, T).clone()
    L = C.lengths(cfg, T)
    us = int(np.prod(cfg["ups_rates"][:cfg["n_ups"]])) * cfg["hop"]
    har = torch.empty(N, (cfg["n_fft"] + 2) * L["frames"], device="cuda")
    g = "decoder.module.generator.m_source.l_linear."
    lW, lb = dev(params[g + "weight"]), dev(params[g + "bias"])
    ctx.call("kdec_harmonic_source", native.ptr(t[1]), 2 * T, native.ptr(har), har.shape[1], N, 2 * T,
             native.ptr(lW), native.ptr(lb), cfg["harmonic_num"], cfg["sample_rate"], us, cfg["n_fft"], cfg["hop"])
    a2 = m.forward(*t, T, har=har)
    torch.cuda.synchronize()
    assert torch.equal(a1, a2)


def test_single_stream_equals_overlapped(ctx):
    # kdec_model_set_overlap(0) keeps every launch on one stream; with the
    # two-stream schedule (one chain for the batch) the waveform, d(style) and
    # every grad are the same bits (all reductions sum in a fixed order).
    from brosoundml_amd import native
    cfg, N, T = C.SMALL, 2, 6
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    m.set_params(synth.init_params(shapes))
    asr, F0, Nn, style, dA = inputs(cfg, N, T, "gm.ovl")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn, style)]
    d = dev(dA)
    res = []
    for on in (True, False):
        m.set_overlap(on)
        m.zero_grad()
        audio = m.forward(*t, T).clone()
        ds = torch.empty_like(t[3])
        m.backward(d, wgrad=True, dalpha=True, dstyle=ds)
        torch.cuda.synchronize()
        res.append((audio.cpu().numpy(), ds.cpu().numpy(), {n: m.grad(n, s) for n, s in shapes.items()}))
    np.testing.assert_array_equal(res[0][0], res[1][0])
    np.testing.assert_array_equal(res[0][1], res[1][1])
    for n in shapes:
        np.testing.assert_array_equal(res[0][2][n], res[1][2][n], err_msg=n)


def test_reference_semantics_three_resblock_streams(ctx):
    # without conv weight grads the generator's resblock and noise-branch
    # backwards run on three streams (K = 3 here): the affine grads and
    # d(style) the reference returns, against the oracle at the usual bars
    r = run_pair(ctx, C.SMALL, 2, 6, "gm.ref3", wgrad=False, dalpha=False)
    check_pair(r, wgrad=False)


def test_no_weight_grad_backward_single_stream_equals_overlapped(ctx):
    # the same bit-for-bit property as above for the backward without conv
    # weight grads (its resblocks on three streams), with alpha grads on and off
    from brosoundml_amd import native
    cfg, N, T = C.SMALL, 2, 6
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    m.set_params(synth.init_params(shapes))
    asr, F0, Nn, style, dA = inputs(cfg, N, T, "gm.ovl2")
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn, style)]
    d = dev(dA)
    for dalpha in (False, True):
        res = []
        for on in (True, False):
            m.set_overlap(on)
            m.zero_grad()
            m.forward(*t, T)
            ds = torch.empty_like(t[3])
            m.backward(d, wgrad=False, dalpha=dalpha, dstyle=ds)
            torch.cuda.synchronize()
            _, dgb = m.affines(N)
            res.append((ds.cpu().numpy(), np.array(dgb), {n: m.grad(n, s) for n, s in shapes.items() if "alpha" in n}))
        m.set_overlap(True)
        np.testing.assert_array_equal(res[0][0], res[1][0])
        np.testing.assert_array_equal(res[0][1], res[1][1])
        for n in res[0][2]:
            np.testing.assert_array_equal(res[0][2][n], res[1][2][n], err_msg=n)


@pytest.mark.parametrize("split", [True, False])
def test_batch_split_vs_oracle(ctx, split):
    # kdec_model_set_batch_split(1) runs a batch of N >= 2 as two half-batch
    # chains (rows [0, N - N//2) and the rest) on two streams, forwards and
    # backwards concurrent, the second half's weight grads in a second buffer
    # added at the end. With N = 3 (parts of 2 and 1 rows) and with one chain
    # for the whole batch, every output against the oracle at the usual bars
    # (the leaky kinks reconciled from the model's own site inputs, which
    # the two schedules may round to opposite sides of zero).
    r = run_pair(ctx, C.SMALL, 3, 6, "gm.split", split=split)
    report = check_pair(r)
    print(f"split={split}: " + ", ".join(f"{k}={v}" for k, v in report.items()), flush=True)


def test_inference_forwards(ctx):
    # kdec_model_infer (the training forward without caches) gives the
    # training forward's waveform bit for bit. decode_back_half runs the
    # separately composed inference forwards (DecoderBackbone / HarmonicSource
    # / Generator::forward and their building blocks), the twin the reference
    # checks its `_train` composition against at 1e-4
    # (test_kokoro_decoder_backward.cpp:516-530); here within 1e-5. A
    # backward after an inference forward is refused.
    import ctypes
    from brosoundml_amd import native
    cfg, N, T = C.SMALL, 2, 6
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    m.set_params(synth.init_params(shapes))
    asr, F0, Nn, style, dA = inputs(cfg, N, T, "gm.inf")
    F0[1, 3:7] = 0.0
    S = cfg["style_dim"]
    ref_s = np.concatenate([style, synth.normal("gm.inf.ref2", (N, S), 0.3)], axis=1)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn, style)]
    t_ref = dev(ref_s)
    a_train = m.forward(*t, T).clone()
    a_inf = torch.empty_like(a_train)
    P = native.ptr
    m._c(ctx.L.kdec_model_infer(m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(t[3]), None, P(a_inf)))
    a_dbh = torch.empty_like(a_train)
    m._c(ctx.L.kdec_model_decode_back_half(m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(t_ref), 2 * S, P(a_dbh)))
    torch.cuda.synchronize()
    assert torch.equal(a_inf, a_train)
    e = rel_l2(a_dbh.cpu().numpy(), a_train.cpu().numpy())
    assert e <= 1e-5, f"inference twin vs training forward rel-L2 {e:.3e}"
    with pytest.raises(native.KdecError, match="no training forward"):
        m.backward(dev(dA))
    # a training forward makes the backward available again
    m.forward(*t, T)
    m.backward(dev(dA))
    torch.cuda.synchronize()
    del ctypes


def test_decode_back_half_cancellation(ctx):
    # the reference's cooperative cancellation: polled before the generator
    # and before each upsample stage; a cancel leaves the audio unwritten
    import ctypes
    from brosoundml_amd import native
    cfg, N, T = C.SMALL, 1, 5
    m = native.Model(ctx, cfg)
    m.set_params(synth.init_params(m.param_shapes()))
    asr, F0, Nn, style, _ = inputs(cfg, N, T, "gm.cancel")
    S = cfg["style_dim"]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn)]
    ref_s = dev(np.concatenate([style, style], axis=1))
    L = C.lengths(cfg, T)
    P = native.ptr
    full = torch.empty(N, L["audio"], device="cuda")
    m._c(ctx.L.kdec_model_decode_back_half(m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(ref_s), 2 * S, P(full)))
    torch.cuda.synchronize()
    CB = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)
    for cancel_at in (1, 2, 3, None):  # poll 1: before the generator, 2-3: before stages 0-1
        polls = []

        def poll(_user, polls=polls, cancel_at=cancel_at):
            polls.append(1)
            return int(cancel_at is not None and len(polls) >= cancel_at)
        cb = CB(poll)
        out = torch.full((N, L["audio"]), 7.0, device="cuda")
        flag = ctypes.c_int(-1)
        m._c(ctx.L.kdec_model_decode_back_half_cancellable(
            m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(ref_s), 2 * S, P(out), ctypes.cast(cb, ctypes.c_void_p), None,
            ctypes.cast(ctypes.pointer(flag), ctypes.c_void_p)))
        torch.cuda.synchronize()
        if cancel_at is None:
            assert flag.value == 0 and len(polls) == 1 + cfg["n_ups"]
            assert torch.equal(out, full)
        else:
            assert flag.value == 1 and len(polls) == cancel_at
            assert torch.all(out == 7.0)


def test_decode_back_half_trace(ctx):
    # the reference's KokoroTrace from decode_back_half (kokoro.cpp:366,
    # 389-390, 396): "gen_in", "har" and "audio" per utterance, equal to the
    # untraced call's audio, the harmonic-source op's output and the oracle's
    # backbone output
    import ctypes
    import oracle_lib as O
    from brosoundml_amd import native
    cfg, N, T = C.SMALL, 2, 6
    m = native.Model(ctx, cfg)
    params = synth.init_params(m.param_shapes())
    m.set_params(params)
    asr, F0, Nn, style, _ = inputs(cfg, N, T, "gm.trace")
    S = cfg["style_dim"]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    t = [dev(a) for a in (asr, F0, Nn)]
    ref_s = dev(np.concatenate([style, style], axis=1))
    L = C.lengths(cfg, T)
    P = native.ptr
    plain = torch.empty(N, L["audio"], device="cuda")
    m._c(ctx.L.kdec_model_decode_back_half(m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(ref_s), 2 * S, P(plain)))
    tr = ctypes.c_void_p()
    ctx.check(ctx.L.kdec_trace_create(ctypes.byref(tr)))
    traced = torch.empty_like(plain)
    m._c(ctx.L.kdec_model_decode_back_half_traced(m.h, N, T, P(t[0]), P(t[1]), P(t[2]), P(ref_s), 2 * S,
                                                  P(traced), None, None, None, tr))
    torch.cuda.synchronize()
    assert torch.equal(plain, traced)
    stages = {}
    for i in range(ctx.L.kdec_trace_count(tr)):
        h, w = ctypes.c_int(), ctypes.c_int()
        name = ctx.L.kdec_trace_stage(tr, i, ctypes.cast(ctypes.pointer(h), ctypes.c_void_p),
                                      ctypes.cast(ctypes.pointer(w), ctypes.c_void_p)).decode()
        p = ctypes.cast(ctx.L.kdec_trace_data(tr, i), ctypes.POINTER(ctypes.c_float))
        stages[name] = np.ctypeslib.as_array(p, shape=(h.value * w.value,)).copy().reshape(h.value, w.value)
    ctx.check(ctx.L.kdec_trace_destroy(tr))
    assert list(stages) == [f"{s}.{n}" for s in ("gen_in", "har", "audio") for n in range(N)]
    om = O.OracleModel(cfg)
    om.set_params(params)
    for n in range(N):
        assert stages[f"audio.{n}"].shape == (1, L["audio"])
        np.testing.assert_array_equal(stages[f"audio.{n}"][0], plain[n].cpu().numpy())
        assert stages[f"har.{n}"].shape == (cfg["n_fft"] + 2, L["frames"])
        om.forward(asr[n], F0[n], Nn[n], style[n], T)
        assert rel_l2(stages[f"har.{n}"][: cfg["n_fft"] // 2 + 1], om.har().reshape(cfg["n_fft"] + 2, -1)[
            : cfg["n_fft"] // 2 + 1]) <= 1e-5
        gi = stages[f"gen_in.{n}"]
        assert gi.shape == (cfg["dec_out"][-1], 2 * T)
        assert rel_l2(gi.ravel(), om.gen_in()) <= 1e-5


def test_debug_stages_env():
    # BROSOUNDML_DEBUG_STAGES=1: decode_back_half prints the reference's
    # per-stage summaries (kokoro.cpp:46-90) plus the non-finite count, in a
    # child process so the environment is read fresh
    import subprocess
    import sys
    code = (
        "import sys, numpy as np, torch\n"
        "sys.path[:0] = [%r, %r]\n"
        "from brosoundml_amd import native, config as C, synth\n"
        "from model_parity import inputs\n"
        "ctx = native.Context(0); cfg = C.SMALL; N, T = 1, 5\n"
        "m = native.Model(ctx, cfg); m.set_params(synth.init_params(m.param_shapes()))\n"
        "asr, F0, Nn, st, _ = inputs(cfg, N, T, 'gm.dbg')\n"
        "d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()\n"
        "rs = d(np.concatenate([st, st], axis=1)); a = torch.empty(N, C.lengths(cfg, T)['audio'], device='cuda')\n"
        "P = native.ptr\n"
        "m._c(ctx.L.kdec_model_decode_back_half(m.h, N, T, P(d(asr)), P(d(F0)), P(d(Nn)), P(rs), 2 * cfg['style_dim'], P(a)))\n"
        "torch.cuda.synchronize()\n" % (os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                        os.path.dirname(os.path.abspath(__file__))))
    env = dict(os.environ, BROSOUNDML_DEBUG_STAGES="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stderr.splitlines() if ln.startswith("[stage]")]
    assert [ln.split()[1] for ln in lines] == ["09_gen_in", "10_har_stub", "11_audio"], r.stderr[-2000:]
    for ln in lines:
        assert "nonfinite=0" in ln and "std=" in ln, ln
