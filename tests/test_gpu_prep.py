"""The producer step (kdec_model_decode_prep, the KokoroDecodePrep of
Kokoro::prepare_decode_context after the predictor, kokoro.cpp:667-732):
asr is the per-phoneme repeat of the text features (np.repeat pins it bit for
bit), F0 / N are the predictions or the overrides, har is the model's
harmonic source on that F0 (bit for bit with the op), and the reference's
errors come back with its messages. The DecoderLoraContext view drives a
DecoderLora forward exactly as the same tensors passed directly do.
"""
import ctypes

import numpy as np
import pytest

from brosoundml_amd import config as C
from brosoundml_amd import synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CFG = C.SMALL


@pytest.fixture(scope="module")
def model():
    from brosoundml_amd import native
    ctx = native.Context(0)
    m = native.Model(ctx, CFG)
    m.set_params(synth.init_params(m.param_shapes()))
    return ctx, m


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def P(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def fptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def prep(ctx, m, t_en, dur, F0=None, Nn=None, F0_ov=None, N_ov=None, ref_s=None):
    h = ctypes.c_void_p()
    d = np.ascontiguousarray(dur, np.int32)
    f_ov = None if F0_ov is None else np.ascontiguousarray(F0_ov, np.float32)
    n_ov = None if N_ov is None else np.ascontiguousarray(N_ov, np.float32)
    m._c(ctx.L.kdec_model_decode_prep(m.h, P(t_en), d.size, fptr(d), P(F0), P(Nn), fptr(f_ov),
                                      0 if f_ov is None else f_ov.size, fptr(n_ov), 0 if n_ov is None else n_ov.size,
                                      P(ref_s), ctypes.byref(h)))
    return h


def read(ctx, h, which, n):
    out = torch.empty(n, device="cuda")
    p = ctx.L.kdec_prep_ptr(h, which)
    assert p
    ctx.check(ctx.L.kdec_axpby(ctx.h, 1.0, ctypes.c_void_p(p), n, 0.0, None, 0, P(out), n, 1, n))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def inputs(L, seed):
    r = np.random.default_rng(seed)
    dur = r.integers(0, 5, L).astype(np.int32)
    dur[0] = max(dur[0], 1)
    total = int(dur.sum())
    te = r.normal(size=(CFG["asr_dim"], L)).astype(np.float32)
    F0 = r.uniform(80, 300, 2 * total).astype(np.float32)
    F0[r.uniform(size=2 * total) < 0.2] = 0.0
    Nn = r.normal(0, 0.5, 2 * total).astype(np.float32)
    ref_s = r.normal(0, 0.3, 2 * CFG["style_dim"]).astype(np.float32)
    return dur, total, te, F0, Nn, ref_s


def test_prep_outputs(model):
    ctx, m = model
    L = 23
    dur, total, te, F0, Nn, ref_s = inputs(L, 5)
    t_te, t_F0, t_N, t_ref = dev(te), dev(F0), dev(Nn), dev(ref_s)
    h = prep(ctx, m, t_te, dur, t_F0, t_N, ref_s=t_ref)
    try:
        us = C.upsample_prod(CFG)
        frames = 2 * total * us + 1
        assert ctx.L.kdec_prep_total(h) == total and ctx.L.kdec_prep_frames(h) == frames
        asr = read(ctx, h, 0, CFG["asr_dim"] * total).reshape(CFG["asr_dim"], total)
        assert np.array_equal(asr, np.repeat(te, dur, axis=1))
        assert np.array_equal(read(ctx, h, 1, 2 * total), F0)
        assert np.array_equal(read(ctx, h, 2, 2 * total), Nn)
        assert np.array_equal(read(ctx, h, 4, 2 * CFG["style_dim"]), ref_s)
        # the harmonic source, as the op computes it on the same F0
        nh = (CFG["n_fft"] + 2) * frames
        har = torch.empty(1, nh, device="cuda")
        g = "decoder.module.generator.m_source.l_linear."
        params = synth.init_params(m.param_shapes())
        lW, lb = dev(params[g + "weight"]), dev(params[g + "bias"])
        ctx.call("kdec_harmonic_source", P(t_F0), 2 * total, P(har), nh, 1, 2 * total, P(lW), P(lb),
                 CFG["harmonic_num"], CFG["sample_rate"], us * CFG["hop"], CFG["n_fft"], CFG["hop"])
        torch.cuda.synchronize()
        assert np.array_equal(read(ctx, h, 3, nh), har.cpu().numpy()[0])
        # the context drives a DecoderLora forward as the tensors themselves do
        from brosoundml_amd import native
        dl = native.DecoderLora(m, 4, 0.5, seed=9)
        dl.set("W2", synth.normal("prep.w2", (4, 16), 0.3))
        cond = dev(np.array([[0.3, -0.2, 0.9]], np.float32))
        a_ctx = torch.empty(1, 2 * total * us * CFG["hop"], device="cuda")
        pp = [ctypes.c_void_p(ctx.L.kdec_prep_ptr(h, w)) for w in range(5)]
        m._c(ctx.L.kdec_dlora_forward(dl.h, 1, total, pp[0], pp[1], pp[2], pp[4], 2 * CFG["style_dim"], pp[3],
                                      P(cond), P(a_ctx)))
        t_asr = dev(np.repeat(te, dur, axis=1))
        a_dir = dl.forward(t_asr[None], t_F0[None], t_N[None], t_ref[None], total, cond, har=har)
        torch.cuda.synchronize()
        assert torch.equal(a_ctx, a_dir)
    finally:
        ctx.L.kdec_prep_destroy(h)


def test_prep_overrides(model):
    ctx, m = model
    dur, total, te, F0, Nn, ref_s = inputs(17, 6)
    F0_ov = np.linspace(90, 250, 2 * total).astype(np.float32)
    N_ov = np.linspace(-1, 1, 2 * total).astype(np.float32)
    h = prep(ctx, m, dev(te), dur, None, None, F0_ov, N_ov, ref_s=dev(ref_s))
    try:
        assert np.array_equal(read(ctx, h, 1, 2 * total), F0_ov)
        assert np.array_equal(read(ctx, h, 2, 2 * total), N_ov)
    finally:
        ctx.L.kdec_prep_destroy(h)


def test_prep_errors(model):
    from brosoundml_amd import native
    ctx, m = model
    dur, total, te, F0, Nn, ref_s = inputs(11, 7)
    t_te, t_ref = dev(te), dev(ref_s)
    with pytest.raises(native.KdecError, match="predicted total frame count is 0"):
        prep(ctx, m, t_te, np.zeros(11, np.int32), dev(F0), dev(Nn), ref_s=t_ref)
    with pytest.raises(native.KdecError, match=rf"F0 override size must be 2\*total \({2 * total}\)"):
        prep(ctx, m, t_te, dur, None, dev(Nn), np.zeros(2 * total - 1, np.float32), ref_s=t_ref)
    bad = dur.copy()
    bad[3] = -1
    with pytest.raises(native.KdecError, match="negative predicted duration"):
        prep(ctx, m, t_te, bad, dev(F0), dev(Nn), ref_s=t_ref)
