"""GPU parity at the real Kokoro-82M shapes.

* Config 0: the whole decoder, B = 1, T = 64 (38 400 samples), against the
  oracle: waveform, every parameter grad, the AdaIN affine grads, d(style),
  and the in-model harmonic source at full length.
* Config 1: Snake + AdaIN1d forward and backward on x [1, 256, 48000] with
  (gamma, beta) from a 128 -> 512 style projection: dX, d(alpha), d(style).
* Config 2: Conv1d 512 -> 512, k 3, dilations 1 / 3 / 5 on [4, 512, 2048]:
  forward, input grad, weight and bias grads against torch float64 on the
  CPU.
* Config 3: the two ConvTranspose1d upsamplers (ups0 on [4, 512, 512], ups1
  on [4, 256, 5120] and on [4, 256, 512]) likewise.
* Config 4: one utterance at T = 512 (307 200 samples, 20 % unvoiced F0)
  against the oracle, and the benchmark's own B = 8, T = 512 step: every
  utterance's waveform and leaky-site inputs against a B = 1 run; the
  batch's d(style) and AdaIN affine grads of utterances 0 and 7 against the
  oracle; the batch's parameter grads (every conv, conv-transpose, pool and
  fc weight and bias, every snake alpha) with dL/dwav nonzero on utterance
  n only (n = 0 and 7: the B = 8 kernels, split plans and weight-grad lane,
  with utterance n's grads alone) against the oracle's utterance n; and the
  full batch's parameter grads against the sum of the eight one-utterance
  backwards of the same forward (the fold over utterances).
* The weight-grad GEMM at production K: 8 x 61 441 positions at C = 128
  (the stage-1 instance) and 8 x 10 240 at C = 256 (stage 0).
* The reference's own semantics (conv input grads only, no weight grads,
  snake alpha grads on or off) at Kokoro shapes, N = 2, T = 64: against the
  oracle, and the overlapped schedule bit for bit against one stream.
* The inference forwards (kdec_model_infer, kdec_model_decode_back_half)
  against the oracle's forward.

Each comparison prints its rel-L2 and max-abs error and records it
(model_parity.REPORT).
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from brosoundml_amd import config as C
from brosoundml_amd import synth
from model_parity import (FWD_TOL, GRAD_TOL, check_har, check_pair, dev, grad_errors, inputs, kink_check, max_abs,
                          record, record_grads, rel_l2, run_pair)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
F = torch.nn.functional


@pytest.fixture(scope="module")
def ctx():
    from brosoundml_amd import native
    return native.Context(0)


@pytest.fixture(scope="module")
def kokoro_params():
    shapes = O.OracleModel(C.KOKORO).param_shapes()
    return synth.init_params(shapes)


def P(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def close(got, ref, tol, what):
    e, m = rel_l2(got, ref), max_abs(got, ref)
    print(f"{what}: rel-L2 {e:.3e} max-abs {m:.3e}", flush=True)
    record(what, e, m)
    assert e <= tol, f"{what}: rel-L2 {e:.3e} > {tol:.0e} (max-abs {m:.3e})"


def report(name, rep):
    print(f"{name}: " + ", ".join(f"{k}={v}" for k, v in rep.items()), flush=True)


def model_har(ctx, m, cfg, N, T, ins):
    """The model's own harmonic source for these inputs (a forward without har_in)."""
    asr, F0, Nn, style = (dev(a) for a in ins[:4])
    m.forward(asr, F0, Nn, style, T)
    torch.cuda.synchronize()
    return m.har(N, T)


# ─── config 0 ───

def test_config0_whole_decoder(ctx, kokoro_params):
    cfg, N, T = C.KOKORO, 1, 64
    r = run_pair(ctx, cfg, N, T, "cfg0", params=kokoro_params)
    report("config0 B=1 T=64", check_pair(r, name="config 0: decoder B=1 T=64"))
    har = model_har(ctx, r["m"], cfg, N, T, r["inputs"])
    report("config0 in-model harmonic source", check_har(har[0], r["ref_har"][0], cfg["n_fft"]))


# ─── config 1 ───

def test_config1_snake_adain(ctx):
    C_, L, S = 256, 48000, 128
    x = synth.normal("cfg1.x", (1, C_, L))
    alpha = synth.uniform("cfg1.alpha", (C_,), 0.5, 2.0)
    style = synth.normal("cfg1.style", (1, S), 0.3)
    bound = 1.0 / np.sqrt(S)
    W = synth.uniform("cfg1.fcW", (2 * C_, S), -bound, bound)
    b = synth.uniform("cfg1.fcb", (2 * C_,), -bound, bound)
    dY = synth.normal("cfg1.dy", (1, C_, L))
    tx, tW, tb, ts, ta, tdy = (dev(a) for a in (x, W, b, style, alpha, dY))
    gb = torch.empty(1, 2 * C_, device="cuda")
    ctx.call("kdec_style_proj_fwd", P(tW), P(tb), P(ts), S, P(gb), 2 * C_, 1, 2 * C_, S)
    st = torch.empty(C_, 2, device="cuda")
    y = torch.empty(1, C_, L, device="cuda")
    g_p, b_p = P(gb), ctypes.c_void_p(gb.data_ptr() + 4 * C_)
    ctx.call("kdec_adain_act_fwd_stats", P(tx), C_ * L, 1e-5, P(st), g_p, b_p, 2 * C_, 2, 0.0, P(ta), P(y), C_ * L,
             None, 0, 1, C_, L)
    dx = torch.empty_like(tx)
    dgb = torch.empty(1, 2 * C_, device="cuda")
    da = torch.zeros(C_, device="cuda")
    ctx.call("kdec_adain_act_bwd", P(tx), C_ * L, P(st), g_p, b_p, 2 * C_, 2, 0.0, P(ta), P(tdy), C_ * L, None, 0,
             P(dx), C_ * L, P(dgb), ctypes.c_void_p(dgb.data_ptr() + 4 * C_), 2 * C_, P(da), 1, C_, L)
    dstyle = torch.empty(1, S, device="cuda")
    dW = torch.zeros(2 * C_, S, device="cuda")
    dbias = torch.zeros(2 * C_, device="cuda")
    ctx.call("kdec_style_proj_bwd", P(tW), P(ts), S, P(dgb), 2 * C_, P(dstyle), S, 0.0, P(dW), P(dbias), 1,
             2 * C_, S)
    torch.cuda.synchronize()
    # oracle: projection in float64, AdaIN and Snake by the C restatement
    gb_ref = W.astype(np.float64) @ style[0].astype(np.float64) + b
    close(gb.cpu().numpy()[0], gb_ref, FWD_TOL, "config1 style projection")
    gam, bet = gb_ref[:C_].astype(np.float32), gb_ref[C_:].astype(np.float32)
    s = O.adain_affine(x[0], gam, bet, C_, L)
    close(y.cpu().numpy(), O.snake(s, alpha, C_, L), FWD_TOL, "config1 forward y")
    ds, rda = O.snake_bwd(s, alpha, dY[0], C_, L)
    rdx, rdg, rdb = O.adain_affine_bwd(x[0], gam, ds, C_, L)
    close(dx.cpu().numpy(), rdx, GRAD_TOL, "config1 dX")
    close(da.cpu().numpy(), rda, GRAD_TOL, "config1 d(alpha)")
    rdgb = np.concatenate([rdg, rdb]).astype(np.float64)
    close(dgb.cpu().numpy()[0], rdgb, GRAD_TOL, "config1 d(gamma, beta)")
    close(dstyle.cpu().numpy()[0], W.astype(np.float64).T @ rdgb, GRAD_TOL, "config1 d(style)")
    close(dW.cpu().numpy(), np.outer(rdgb, style[0].astype(np.float64)), GRAD_TOL, "config1 d(fc.weight)")


# ─── config 2 ───

@pytest.mark.parametrize("d", [1, 3, 5])
def test_config2_conv1d_512(ctx, d):
    N, Cc, L, k = 4, 512, 2048, 3
    bound = 1.0 / np.sqrt(Cc * k)
    x = synth.normal(f"cfg2.x{d}", (N, Cc, L))
    W = synth.uniform(f"cfg2.W{d}", (Cc, Cc * k), -bound, bound)
    b = synth.uniform(f"cfg2.b{d}", (Cc,), -bound, bound)
    dY = synth.normal(f"cfg2.dy{d}", (N, Cc, L))
    tx, tW, tb, tdy = (dev(a) for a in (x, W, b, dY))
    Y = torch.empty(N, Cc, L, device="cuda")
    ctx.call("kdec_conv1d_fwd", P(tx), Cc * L, P(tW), P(tb), P(Y), Cc * L, N, Cc, L, Cc, k, 1, d, d, None, 0, 1.0,
             0.0)
    dX = torch.empty(N, Cc, L, device="cuda")
    ctx.call("kdec_conv1d_dgrad", P(tW), P(tdy), Cc * L, P(dX), Cc * L, N, Cc, L, Cc, k, 1, d, d, 1.0, 0.0)
    dW = torch.zeros(Cc, Cc * k, device="cuda")
    db = torch.zeros(Cc, device="cuda")
    ctx.call("kdec_conv1d_wgrad", P(tx), Cc * L, P(tdy), Cc * L, P(dW), P(db), N, Cc, L, Cc, k, 1, d, d)
    torch.cuda.synchronize()
    xd, Wd, dyd = (torch.from_numpy(a).double() for a in (x, W.reshape(Cc, Cc, k), dY))
    close(Y.cpu().numpy(), F.conv1d(xd, Wd, torch.from_numpy(b).double(), padding=d, dilation=d).numpy(), FWD_TOL,
          f"config2 d={d} forward")
    close(dX.cpu().numpy(), F.conv_transpose1d(dyd, Wd, padding=d, dilation=d).numpy(), GRAD_TOL,
          f"config2 d={d} input grad")
    rW = torch.nn.grad.conv1d_weight(xd, Wd.shape, dyd, padding=d, dilation=d).reshape(Cc, Cc * k)
    close(dW.cpu().numpy(), rW.numpy(), GRAD_TOL, f"config2 d={d} weight grad")
    close(db.cpu().numpy(), dyd.sum(dim=(0, 2)).numpy(), GRAD_TOL, f"config2 d={d} bias grad")


# ─── config 3 ───

@pytest.mark.parametrize("name,Cin,Cout,L,k,s,p", [
    ("ups0", 512, 256, 512, 20, 10, 5),
    ("ups1", 256, 128, 5120, 12, 6, 3),
    ("ups1_unchained", 256, 128, 512, 12, 6, 3),
])
def test_config3_convt(ctx, name, Cin, Cout, L, k, s, p):
    N = 4
    Lo = O.convt1d_out_len(L, k, s, p, 0, 1)
    bound = 1.0 / np.sqrt(Cout * k)
    x = synth.normal(f"cfg3.{name}.x", (N, Cin, L))
    W = synth.uniform(f"cfg3.{name}.W", (Cin, Cout * k), -bound, bound)
    b = synth.uniform(f"cfg3.{name}.b", (Cout,), -bound, bound)
    dY = synth.normal(f"cfg3.{name}.dy", (N, Cout, Lo))
    tx, tW, tb, tdy = (dev(a) for a in (x, W, b, dY))
    Y = torch.empty(N, Cout, Lo, device="cuda")
    ctx.call("kdec_convt1d_fwd", P(tx), Cin * L, P(tW), P(tb), P(Y), Cout * Lo, N, Cin, L, Cout, k, s, p, 0)
    dX = torch.empty(N, Cin, L, device="cuda")
    ctx.call("kdec_convt1d_dgrad", P(tW), P(tdy), Cout * Lo, P(dX), Cin * L, N, Cin, L, Cout, k, s, p, 0)
    dW = torch.zeros(Cin, Cout * k, device="cuda")
    db = torch.zeros(Cout, device="cuda")
    ctx.call("kdec_convt1d_wgrad", P(tx), Cin * L, P(tdy), Cout * Lo, P(dW), P(db), N, Cin, L, Cout, k, s, p, 0)
    torch.cuda.synchronize()
    xd = torch.from_numpy(x).double()
    Wd = torch.from_numpy(W.reshape(Cin, Cout, k)).double().requires_grad_(True)
    dyd = torch.from_numpy(dY).double()
    y = F.conv_transpose1d(xd, Wd, torch.from_numpy(b).double(), stride=s, padding=p)
    assert y.shape[-1] == Lo
    close(Y.cpu().numpy(), y.detach().numpy(), FWD_TOL, f"config3 {name} forward")
    y.backward(dyd)
    close(dX.cpu().numpy(), F.conv1d(dyd, Wd.detach(), stride=s, padding=p).numpy(), GRAD_TOL,
          f"config3 {name} input grad")
    close(dW.cpu().numpy(), Wd.grad.reshape(Cin, Cout * k).numpy(), GRAD_TOL, f"config3 {name} weight grad")
    close(db.cpu().numpy(), dyd.sum(dim=(0, 2)).numpy(), GRAD_TOL, f"config3 {name} bias grad")


# ─── weight grads at production K ───

@pytest.mark.parametrize("Cc,L,k,d", [(128, 61441, 11, 5), (128, 61441, 3, 1), (256, 10240, 7, 3),
                                       (256, 10240, 11, 5)])
def test_wgrad_production_k(ctx, Cc, L, k, d):
    # The ResBlock1 weight grads of a B = 8, T = 512 step at K = 8 x L
    # positions (split-K over rounds of resident blocks, the in-row fast
    # staging path and the boundary chunks): stage 1 (C = 128, L = 61441;
    # C_in*k = 384 / 1408, the 128-column tile) and stage 0 (C = 256,
    # L = 10240; C_in*k = 1792 / 2816, the 256-column tile)
    N = 8
    p = d * (k - 1) // 2
    x = synth.normal(f"wgk.x{Cc}.{k}", (N, Cc, L))
    dY = synth.normal(f"wgk.dy{Cc}.{k}", (N, Cc, L))
    tx, tdy = dev(x), dev(dY)
    dW = torch.zeros(Cc, Cc * k, device="cuda")
    db = torch.zeros(Cc, device="cuda")
    ctx.call("kdec_conv1d_wgrad", P(tx), Cc * L, P(tdy), Cc * L, P(dW), P(db), N, Cc, L, Cc, k, 1, p, d)
    torch.cuda.synchronize()
    xd, dyd = torch.from_numpy(x).double(), torch.from_numpy(dY).double()
    rW = torch.nn.grad.conv1d_weight(xd, (Cc, Cc, k), dyd, padding=p, dilation=d).reshape(Cc, Cc * k)
    close(dW.cpu().numpy(), rW.numpy(), GRAD_TOL, f"wgrad N=8 C={Cc} L={L} k={k} d={d}")
    close(db.cpu().numpy(), dyd.sum(dim=(0, 2)).numpy(), GRAD_TOL, f"bias grad N=8 C={Cc} L={L} k={k}")


# ─── config 4 ───

def test_config4_one_utterance(ctx, kokoro_params):
    cfg, N, T = C.KOKORO, 1, 512
    r = run_pair(ctx, cfg, N, T, "cfg4", params=kokoro_params, unvoiced=0.2)
    report("config4 B=1 T=512", check_pair(r, name="config 4: decoder B=1 T=512"))
    har = model_har(ctx, r["m"], cfg, N, T, r["inputs"])
    report("config4 in-model harmonic source (307200 samples)", check_har(har[0], r["ref_har"][0], cfg["n_fft"]))


def test_config4_batch_of_8(ctx, kokoro_params):
    # The benchmark's workload (B = 8, T = 512, 20 % unvoiced F0, its inputs).
    from brosoundml_amd import native
    cfg, N, T = C.KOKORO, 8, 512
    m = native.Model(ctx, cfg)
    m.set_params(kokoro_params)
    shapes = m.param_shapes()
    asr, F0, Nn, style, dA = inputs(cfg, N, T, "bench", unvoiced=0.2)  # the benchmark's inputs
    m.zero_grad()
    audio = m.forward(dev(asr), dev(F0), dev(Nn), dev(style), T).cpu().numpy()
    har8 = m.har(N, T)
    pre8 = m.leaky_inputs()
    # the benchmark's backward: every output of every utterance
    dst8 = torch.empty(N, cfg["style_dim"], device="cuda")
    m.backward(dev(dA), wgrad=True, dalpha=True, dstyle=dst8)
    torch.cuda.synchronize()
    dst8 = dst8.cpu().numpy()
    _, dgb8 = m.affines(N)
    full = {name: m.grad(name, sh).astype(np.float64) for name, sh in shapes.items()}
    # the same forward differentiated one utterance at a time (dL/dwav zero
    # elsewhere): the B = 8 kernels and split plans, utterance n's grads alone
    one = {}
    total = {name: np.zeros_like(g) for name, g in full.items()}
    for n in range(N):
        dAn = np.zeros_like(dA)
        dAn[n] = dA[n]
        m.zero_grad()
        m.backward(dev(dAn), wgrad=True, dalpha=True)
        torch.cuda.synchronize()
        g = {name: m.grad(name, sh) for name, sh in shapes.items()}
        for name in total:
            total[name] += g[name]
        if n in (0, N - 1):
            one[n] = g
    # the batch's grads are the sum of its utterances' (the fold over N)
    worst = grad_errors(full, total)
    record_grads("config 4 B=8: full-batch grads vs the sum of one-utterance backwards", worst)
    assert max(worst)[0] <= 1.0, sorted(worst, reverse=True)[:5]
    # batch independence of the forward
    for n in range(N):
        sl = slice(n, n + 1)
        a1 = m.forward(dev(asr[sl]), dev(F0[sl]), dev(Nn[sl]), dev(style[sl]), T).cpu().numpy()
        assert np.array_equal(m.har(1, T)[0], har8[n]), f"utterance {n}: harmonic source depends on the batch"
        close(audio[n], a1[0], FWD_TOL, f"config 4 utterance {n} waveform, B=8 vs B=1")
        pre1 = m.leaky_inputs()
        worst_pre = max(rel_l2(p8[n], p1[0]) for p8, p1 in zip(pre8, pre1))
        assert worst_pre <= FWD_TOL, f"utterance {n}: leaky-site inputs B=8 vs B=1 rel-L2 {worst_pre:.3e}"
    # utterances 0 and 7 of the batched step against the oracle, on the batch
    # run's own linear pieces (its leaky-site inputs) and harmonic source
    om = O.OracleModel(cfg)
    om.set_params(kokoro_params)
    for n in (0, N - 1):
        om.zero_grad()
        om.set_kinks([p[n] for p in pre8])
        ra = om.forward(asr[n], F0[n], Nn[n], style[n], T, har=har8[n])
        fl, el, mag, srel = kink_check([p[n] for p in pre8], om)
        print(f"config 4 B=8 utterance {n}: {fl} of {el} leaky inputs reconciled, worst |x|/rms {mag:.2e}, "
              f"worst site rel-L2 {srel:.2e}", flush=True)
        record(f"config 4 B=8 utterance {n} leaky sites", srel, None, flips=fl, elements=el, worst_abs_over_rms=mag)
        close(audio[n], ra, FWD_TOL, f"config 4 B=8 utterance {n} waveform vs oracle")
        rds = om.backward(dA[n], wgrad=True, dalpha=True, dstyle=True)
        close(dst8[n], rds, GRAD_TOL, f"config 4 B=8 utterance {n} d(style) vs oracle")
        got = np.concatenate([dgb8[n, off:off + 2 * c] for _, c, off in m.units()])
        ref = np.concatenate([np.concatenate(om.affine(i, c)[2:]) for i, (_, c) in enumerate(om.units())])
        close(got, ref, GRAD_TOL, f"config 4 B=8 utterance {n} AdaIN affine grads vs oracle")
        ref_grads = {name: om.grad(name, sh).astype(np.float64) for name, sh in shapes.items()}
        worst = grad_errors(one[n], ref_grads)
        record_grads(f"config 4 B=8 utterance {n} (one-utterance backward) vs oracle", worst)
        top = sorted(worst, reverse=True)
        print(f"config 4 B=8 utterance {n} parameter grads: worst err/tol {top[0][0]:.3f} ({top[0][1]}), "
              f"worst rel-L2 {max(w[2] for w in worst if w[4]):.2e} (grads not identically zero)", flush=True)
        assert top[0][0] <= 1.0, top[:5]
    om.clear_kinks()


# ─── the reference's own semantics at Kokoro shapes ───

@pytest.mark.parametrize("dalpha", [False, True])
def test_reference_semantics_kokoro(ctx, kokoro_params, dalpha):
    # conv input grads only (no weight grads): the generator's resblock and
    # noise-branch backwards run on three streams; against the oracle
    r = run_pair(ctx, C.KOKORO, 2, 64, f"refsem{int(dalpha)}", wgrad=False, dalpha=dalpha, params=kokoro_params)
    report(f"reference semantics dalpha={dalpha}",
           check_pair(r, wgrad=False, name=f"reference semantics (dalpha={'on' if dalpha else 'off'}) KOKORO N=2 T=64"))


def test_reference_semantics_kokoro_single_stream_equals_overlapped(ctx, kokoro_params):
    from brosoundml_amd import native
    cfg, N, T = C.KOKORO, 2, 64
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    m.set_params(kokoro_params)
    asr, F0, Nn, style, dA = inputs(cfg, N, T, "refsem.ovl")
    t = [dev(a) for a in (asr, F0, Nn, style)]
    d = dev(dA)
    for dalpha in (False, True):
        res = []
        for on in (True, False):
            m.set_overlap(on)
            m.zero_grad()
            a = m.forward(*t, T).cpu().numpy()
            ds = torch.empty_like(t[3])
            m.backward(d, wgrad=False, dalpha=dalpha, dstyle=ds)
            torch.cuda.synchronize()
            _, dgb = m.affines(N)
            res.append((a, ds.cpu().numpy(), np.array(dgb),
                        {n: m.grad(n, s) for n, s in shapes.items() if "alpha" in n}))
        m.set_overlap(True)
        for i in range(3):
            np.testing.assert_array_equal(res[0][i], res[1][i])
        for n in res[0][3]:
            np.testing.assert_array_equal(res[0][3][n], res[1][3][n], err_msg=n)


# ─── inference forwards ───

@pytest.mark.parametrize("cfg_name,N,T", [("SMALL", 2, 6), ("KOKORO", 1, 64)])
def test_inference_forwards_vs_oracle(ctx, kokoro_params, cfg_name, N, T):
    from brosoundml_amd import native
    cfg = getattr(C, cfg_name)
    m = native.Model(ctx, cfg)
    om = O.OracleModel(cfg)
    params = kokoro_params if cfg_name == "KOKORO" else synth.init_params(m.param_shapes())
    m.set_params(params)
    om.set_params(params)
    asr, F0, Nn, style, _ = inputs(cfg, N, T, f"inf.{cfg_name}", unvoiced=0.2)
    S = cfg["style_dim"]
    ref_s = np.concatenate([style, synth.normal(f"inf.{cfg_name}.ref2", (N, S), 0.3)], axis=1)
    t = [dev(a) for a in (asr, F0, Nn, style)]
    L = C.lengths(cfg, T)
    Pn = native.ptr
    # the model's own harmonic source (the op the inference forwards run)
    us = C.upsample_prod(cfg) * cfg["hop"]
    har = torch.empty(N, (cfg["n_fft"] + 2) * L["frames"], device="cuda")
    g = "decoder.module.generator.m_source.l_linear."
    lW, lb = dev(params[g + "weight"]), dev(params[g + "bias"])
    ctx.call("kdec_harmonic_source", Pn(t[1]), 2 * T, Pn(har), har.shape[1], N, 2 * T, Pn(lW), Pn(lb),
             cfg["harmonic_num"], cfg["sample_rate"], us, cfg["n_fft"], cfg["hop"])
    a_inf = torch.empty(N, L["audio"], device="cuda")
    m._c(ctx.L.kdec_model_infer(m.h, N, T, Pn(t[0]), Pn(t[1]), Pn(t[2]), Pn(t[3]), None, Pn(a_inf)))
    a_dbh = torch.empty(N, L["audio"], device="cuda")
    t_ref = dev(ref_s)
    m._c(ctx.L.kdec_model_decode_back_half(m.h, N, T, Pn(t[0]), Pn(t[1]), Pn(t[2]), Pn(t_ref), 2 * S, Pn(a_dbh)))
    torch.cuda.synchronize()
    h_gpu = har.cpu().numpy()
    for n in range(N):
        om.forward(asr[n], F0[n], Nn[n], style[n], T)
        report(f"{cfg_name} harmonic source utt {n}", check_har(h_gpu[n], om.har(), cfg["n_fft"]))
        # the waveform's reference takes the GPU's harmonic source, so the
        # comparison covers the backbone and generator composition exactly
        ref = om.forward(asr[n], F0[n], Nn[n], style[n], T, har=h_gpu[n])
        close(a_inf[n].cpu().numpy(), ref, FWD_TOL, f"{cfg_name} kdec_model_infer utt {n} vs oracle")
        close(a_dbh[n].cpu().numpy(), ref, FWD_TOL, f"{cfg_name} decode_back_half utt {n} vs oracle")


@pytest.mark.parametrize("name,N,Cin,Cout,L,k,s,p,pad_left", [
    ("ups1", 4, 256, 128, 5120, 12, 6, 3, 1),
    ("ups1_b8", 8, 256, 128, 10240, 12, 6, 3, 1),
    ("ups0", 4, 512, 256, 512, 20, 10, 5, 0),
    ("ups1_small", 2, 256, 128, 40, 12, 6, 3, 1),
])
def test_convt_fwd_pad_source_fused(ctx, name, N, Cin, Cout, L, k, s, p, pad_left):
    # kdec_convt1d_fwd_res: the transposed conv, the one-sample left reflect
    # pad and the noise-source add in one epilogue, equal bit for bit to the
    # transposed conv followed by the pad and a float32 add (the epilogue adds
    # bias then the source, as the separate passes round), at the decoder's
    # B = 8 stage-1 shape and smaller grids (whole and split tiles)
    Lo = O.convt1d_out_len(L, k, s, p, 0, 1)
    Ly = Lo + pad_left
    bound = 1.0 / np.sqrt(Cout * k)
    x = synth.normal(f"cvtr.{name}.x", (N, Cin, L))
    W = synth.uniform(f"cvtr.{name}.W", (Cin, Cout * k), -bound, bound)
    b = synth.uniform(f"cvtr.{name}.b", (Cout,), -bound, bound)
    R = synth.normal(f"cvtr.{name}.r", (N, Cout, Ly))
    tx, tW, tb, tR = (dev(a) for a in (x, W, b, R))
    Y = torch.empty(N, Cout, Lo, device="cuda")
    ctx.call("kdec_convt1d_fwd", P(tx), Cin * L, P(tW), P(tb), P(Y), Cout * Lo, N, Cin, L, Cout, k, s, p, 0)
    Yf = torch.full((N, Cout, Ly), float("nan"), device="cuda")
    ctx.call("kdec_convt1d_fwd_res", P(tx), Cin * L, P(tW), P(tb), P(Yf), Cout * Ly, N, Cin, L, Cout, k, s, p, 0,
             P(tR), Cout * Ly, pad_left)
    torch.cuda.synchronize()
    y = Y.cpu().numpy()
    if pad_left:
        y = np.concatenate([y[:, :, 1:2], y], axis=2)
    want = (y + R).astype(np.float32)
    got = Yf.cpu().numpy()
    assert np.array_equal(got, want), f"{name}: max |diff| {np.nanmax(np.abs(got - want)):.3e}"
