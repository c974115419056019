"""Kokoro-82M iSTFTNet decoder forward + backward throughput on one MI355X.

One step is the full decoder back half for B = 8 independent utterances of
T = 512 asr frames (12.8 s of 24 kHz audio each, 102.4 audio-seconds per
step): harmonic source, style projection, DecoderBackbone, Generator,
spectral head / iSTFT forward, then the backward with every extension on
(conv / conv-transpose / pool / style-fc weight grads, Snake alpha grads and
d(style)) besides the reference's AdaIN affine grads. Inputs are synthetic
(asr ~ N(0,1), F0 ~ U(80, 300) Hz with 20% unvoiced zeros, N ~ N(0, 0.5),
style ~ N(0, 0.3), dL/dwav ~ N(0, 1)) and the weights are random-init FP32
at the real shapes; everything is resident in HBM before the timed region.

`value` / `ms_per_step` come from K steps with nothing recorded between
launches. The per-family times and the roofline come from a second pass of
the same K steps with a HIP event pair around each kernel family launch
(`profiled_ms_per_step`), and `serial` repeats both on one stream (no
weight-grad / harmonic-source lanes), where no family shares the CUs.

Prints one JSON line (rank 0). Usage: python bench.py [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA = 157.3e12   # MI355X dense FP32 matrix, FLOP/s
PEAK_HBM = 8.0e12           # MI355X HBM3E, B/s
B, T = 8, 512


def make_inputs(cfg, N, T, tag, unvoiced=0.2):
    from brosoundml_amd import synth
    return synth.decoder_inputs(cfg, N, T, tag, unvoiced)


def cpu_info():
    """Host cores this process may use and the CPU model (lscpu)."""
    import subprocess
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return {"nproc": avail, "cpu_count": os.cpu_count(), "lscpu_model": model}


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    return O


def _median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


def _progress(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_decoder_time(cfg, params, T, ext, threads, runs, warmup=0, tag="bench.cpu", verbose=False):
    """Seconds per decoder forward + backward of one utterance of T frames on
    the oracle at `threads` OpenMP threads (0: all): the median of `runs`
    timed runs after `warmup` untimed ones. ext: the extension's grads
    (conv/convT/pool weights, Snake alphas, d(style)); else the reference's
    semantics (conv dgrad only)."""
    O = _oracle()
    n = O.set_threads(threads)
    om = O.OracleModel(cfg)
    om.set_params(params)
    asr, F0, Nn, style, dA = make_inputs(cfg, 1, T, tag)
    ts = []
    for i in range(warmup + runs):
        t0 = time.perf_counter()
        om.zero_grad()
        om.forward(asr[0], F0[0], Nn[0], style[0], T)
        om.backward(dA[0], wgrad=ext, dalpha=ext, dstyle=ext)
        if i >= warmup:
            ts.append(time.perf_counter() - t0)
        if verbose:
            _progress(f"cpu: decoder T={T} ext={ext} threads={n} run {i}: {time.perf_counter() - t0:.2f} s")
    return _median(ts), n, ts


def cpu_baseline(cfg, params):
    """The oracle (CPU restatement of the reference path, OpenMP) on a bounded
    sample of the benchmarked workload: one utterance of T = 64 frames
    (1.6 s of audio, the config-0 shape) through the decoder forward +
    backward with the same extensions, on this host's cores. All cores: the
    median of 3 after a warm-up; one thread: one run of T = 16 (its cost is
    linear in T, so audio-s/s carries over). About half a minute in all.
    A reported baseline, not the target; `python bench.py --cpu-plan` runs
    the full plan (configs 0-4, both modes, both thread counts)."""
    from brosoundml_amd import config as C
    info = cpu_info()
    T_all, T_one = 64, 16
    med, n_all, ts = cpu_decoder_time(cfg, params, T_all, True, 0, 3, warmup=1)
    one, _, _ = cpu_decoder_time(cfg, params, T_one, True, 1, 1)
    a_all, a_one = C.lengths(cfg, T_all)["audio_seconds"], C.lengths(cfg, T_one)["audio_seconds"]
    _oracle().set_threads(0)
    return {"value": round(a_all / med, 5), "unit": "audio-s/s", "cores": n_all, "kind": "port",
            "seconds": round(med, 3), "runs_s": [round(t, 3) for t in ts],
            "one_thread": {"value": round(a_one / one, 5), "unit": "audio-s/s", "cores": 1, "seconds": round(one, 3),
                           "sample": f"B=1, T={T_one} ({a_one} audio-s), one run"},
            **info,
            "sample": f"B=1, T={T_all} ({a_all} audio-s) of the B={B}, T={T} workload: decoder fwd+bwd with "
                      f"wgrad/dalpha/dstyle on the CPU oracle (double-accumulating C++, OpenMP {n_all} threads), "
                      f"median of 3 after 1 warm-up"}


def cpu_plan(cfg, params, runs=3):
    """The full CPU baseline plan: configs 0-3 in full and config 4 at B = 1
    in full (all cores), at 1 thread and all cores, medians of `runs` after a
    warm-up, both semantics for the decoder. The 1-thread config-4 figure is
    config 0's (cost linear in T), labelled extrapolated, as is the B = 8
    figure (B independent utterances). Long: several minutes."""
    from brosoundml_amd import config as C
    O = _oracle()
    out = {"cpu": cpu_info(), "runs": runs}
    rng = np.random.default_rng(20260)

    def timed(fn, threads, what):
        n = O.set_threads(threads)
        ts = []
        for i in range(runs + 1):  # the first is the warm-up
            t0 = time.perf_counter()
            fn()
            dt = time.perf_counter() - t0
            _progress(f"cpu: {what} threads={n} run {i}: {dt:.2f} s")
            if i:
                ts.append(dt)
        return {"median_s": round(_median(ts), 4), "runs_s": [round(t, 4) for t in ts], "threads": n}

    # config 0 / 4: the decoder, both semantics
    dec = {}
    for name, T in (("config0_B1_T64", 64), ("config4_B1_T512", 512)):
        a = C.lengths(cfg, T)["audio_seconds"]
        for mode, ext in (("extension", True), ("reference_semantics", False)):
            for threads in ((0, 1) if T == 64 else (0,)):
                med, n, ts = cpu_decoder_time(cfg, params, T, ext, threads, runs, warmup=1, tag=f"plan.{name}",
                                              verbose=True)
                dec[f"{name}.{mode}.{'1thread' if threads == 1 else 'all'}"] = {
                    "median_s": round(med, 3), "runs_s": [round(t, 3) for t in ts], "threads": n,
                    "audio_s_per_s": round(a / med, 5)}
    for mode in ("extension", "reference_semantics"):
        c0 = dec[f"config0_B1_T64.{mode}.1thread"]
        c4 = dec[f"config4_B1_T512.{mode}.all"]
        dec[f"config4_B1_T512.{mode}.1thread"] = {"audio_s_per_s": c0["audio_s_per_s"],
                                                   "extrapolated": "config 0's 1-thread rate; cost is linear in T"}
        dec[f"config4_B8_T512.{mode}.all"] = {"audio_s_per_s": c4["audio_s_per_s"],
                                              "seconds": round(8 * c4["median_s"], 3),
                                              "extrapolated": "8 independent utterances x the B=1 time"}
    out["decoder"] = dec

    # config 1: Snake + AdaIN1d backward, x [1,256,48000], style 128 -> 2*256
    Cc, L = 256, 48000
    x = rng.normal(size=(Cc, L)).astype(np.float32)
    dy = rng.normal(size=(Cc, L)).astype(np.float32)
    alpha = rng.uniform(0.5, 2.0, Cc).astype(np.float32)
    Wfc = (rng.uniform(-1, 1, (2 * Cc, 128)) / np.sqrt(128)).astype(np.float32)
    bfc = np.zeros(2 * Cc, np.float32)
    st = rng.normal(0, 0.3, 128).astype(np.float32)

    def c1():
        gb = Wfc @ st + bfc
        s = O.adain_affine(x, gb[:Cc], gb[Cc:], Cc, L)
        ds, _ = O.snake_bwd(s, alpha, dy.ravel(), Cc, L)
        _, dg, db = O.adain_affine_bwd(x, gb[:Cc], ds, Cc, L)
        return Wfc.T @ np.concatenate([dg, db])
    out["config1_snake_adain_bwd"] = {t: timed(c1, th, "config1") for t, th in (("all", 0), ("1thread", 1))}

    # config 2: Conv1d 512->512 k3 d{1,3,5} dgrad + wgrad on [4,512,2048]
    N2, C2, L2, k = 4, 512, 2048, 3
    X2 = rng.normal(size=(N2, C2 * L2)).astype(np.float32)
    G2 = rng.normal(size=(N2, C2 * L2)).astype(np.float32)
    W2 = (rng.uniform(-1, 1, (C2, C2 * k)) / np.sqrt(C2 * k)).astype(np.float32)

    def c2():
        for d in (1, 3, 5):
            for n in range(N2):
                O.conv1d_dgrad(W2, G2[n], C2, L2, C2, k, 1, d, d)
                O.conv1d_wgrad(X2[n], G2[n], C2, L2, C2, k, 1, d, d)
    out["config2_conv1d_bwd"] = {t: timed(c2, th, "config2") for t, th in (("all", 0), ("1thread", 1))}
    out["config2_conv1d_bwd"]["gflop"] = round(3 * 2 * 2.0 * N2 * C2 * C2 * k * L2 / 1e9, 2)

    # config 3: ConvTranspose1d upsampler backwards (dgrad + wgrad)
    cases = {"ups0_512to256_k20_s10_x4x512": (512, 256, 512, 20, 10, 5),
             "ups1_256to128_k12_s6_x4x5120": (256, 128, 5120, 12, 6, 3)}
    c3 = {}
    for name, (Ci, Co, Lin, kk, ss, pp) in cases.items():
        Lo = (Lin - 1) * ss - 2 * pp + kk
        Xt = rng.normal(size=(4, Ci * Lin)).astype(np.float32)
        Gt = rng.normal(size=(4, Co * Lo)).astype(np.float32)
        Wt = (rng.uniform(-1, 1, (Ci, Co * kk)) * 0.05).astype(np.float32)

        def run(Xt=Xt, Gt=Gt, Wt=Wt, Ci=Ci, Co=Co, Lin=Lin, kk=kk, ss=ss, pp=pp):
            for n in range(4):
                O.convt1d_dgrad(Wt, Gt[n], Ci, Lin, Co, kk, ss, pp)
                O.convt1d_wgrad(Xt[n], Gt[n], Ci, Lin, Co, kk, ss, pp)
        c3[name] = {t: timed(run, th, f"config3 {name}") for t, th in (("all", 0), ("1thread", 1))}
        c3[name]["gflop"] = round(2 * 2.0 * 4 * Ci * Co * kk * Lin / 1e9, 2)
    out["config3_convt_bwd"] = c3
    O.set_threads(0)
    return out


def micro_benches(ctx, reps=50):
    """The per-kernel-class cases quoted beside the headline: Snake + AdaIN1d
    backward (x [1,256,48000]), Conv1d 512->512 k3 backward (dgrad + wgrad,
    dilations 1/3/5, X [4,512,2048]), the two ConvTranspose1d upsampler
    backwards, the iSTFT head backward and forward and the style projection
    at the benchmark's B = 8 shapes, each timed alone with HIP events on the context stream over
    `reps` back-to-back calls after 3 untimed ones (the cases take 5-450 us,
    so a shorter run would weigh the queue's start-up on them) and priced
    against its roofline (algorithmic bytes at 8 TB/s or FLOP at the
    FP32-MFMA peak). The timed calls are queued behind a ~4 ms spacer GEMM
    (torch.mm, before the first event), so that the device runs them back to
    back as it does inside a step, instead of at the rate the host issues
    them: each call is one or more ctypes calls and kernel launches, which
    take longer on the host than the few-microsecond cases take on the GPU."""
    import torch
    from brosoundml_amd import native, synth
    P = native.ptr
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    spa = torch.ones(4096, 4096, device="cuda")

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(4):
            torch.mm(spa, spa)
        s0.record()
        for _ in range(reps):
            fn()
        s1.record()
        torch.cuda.synchronize()
        return s0.elapsed_time(s1) / reps * 1e-3

    out = {}
    # Snake + AdaIN1d backward: dX, dgamma, dbeta, dalpha (12 B/elem: dY, x in; dX out)
    C, L = 256, 48000
    x = dev(synth.normal("micro.x", (1, C, L)))
    dy = dev(synth.normal("micro.dy", (1, C, L)))
    alpha = dev(synth.uniform("micro.alpha", (C,), 0.5, 2.0))
    gb = dev(synth.normal("micro.gb", (1, 2 * C), 0.3))
    stats = torch.empty(C, 2, device="cuda")
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    dgb = torch.empty(1, 2 * C, device="cuda")
    da = torch.zeros(C, device="cuda")
    ctx.call("kdec_instnorm_stats", P(x), C * L, 1, C, L, 1e-5, P(stats))
    g_ptr, b_ptr = P(gb), native.ctypes.c_void_p(gb.data_ptr() + 4 * C)
    dg_ptr, db_ptr = P(dgb), native.ctypes.c_void_p(dgb.data_ptr() + 4 * C)
    t = timed(lambda: ctx.call("kdec_adain_act_bwd", P(x), C * L, P(stats), g_ptr, b_ptr, 0, 2, 0.0, P(alpha),
                               P(dy), C * L, None, 0, P(dx), C * L, dg_ptr, db_ptr, 0, P(da), 1, C, L))
    by = 12.0 * C * L
    out["snake_adain_bwd_x1x256x48000"] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                          "frac_hbm": round(by / t / PEAK_HBM, 4),
                                          "algorithmic_bytes": by}
    # forward: statistics, affine and Snake in one pass (the training forward's entry)
    t = timed(lambda: ctx.call("kdec_adain_act_fwd_stats", P(x), C * L, 1e-5, P(stats), g_ptr, b_ptr, 0, 2, 0.0,
                               P(alpha), P(y), C * L, None, 0, 1, C, L))
    by = 8.0 * C * L
    out["snake_adain_fwd_x1x256x48000"] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                          "frac_hbm": round(by / t / PEAK_HBM, 4),
                                          "algorithmic_bytes": by}
    del x, dy, y, dx

    # Conv1d 512 -> 512, k = 3, same padding, dilations 1, 3, 5: dgrad + wgrad
    N, C, L, k = 4, 512, 2048, 3
    X = dev(synth.normal("micro.cx", (N, C, L)))
    G = dev(synth.normal("micro.cg", (N, C, L)))
    W = dev(synth.uniform("micro.cw", (C, C * k), -1 / np.sqrt(C * k), 1 / np.sqrt(C * k)))
    dX = torch.empty_like(X)
    dW = torch.zeros_like(W)
    db = torch.zeros(C, device="cuda")
    tot_t, tot_f = 0.0, 0.0
    for d in (1, 3, 5):
        def run(d=d):
            ctx.call("kdec_conv1d_dgrad", P(W), P(G), C * L, P(dX), C * L, N, C, L, C, k, 1, d, d, 1.0, 0.0)
            ctx.call("kdec_conv1d_wgrad", P(X), C * L, P(G), C * L, P(dW), P(db), N, C, L, C, k, 1, d, d)
        t = timed(run)
        tot_t += t
        tot_f += 2 * 2.0 * N * C * C * k * L
    out["conv1d_bwd_512x512_k3_d135_x4x2048"] = {"ms": round(tot_t * 1e3, 4),
                                                 "TFLOP/s": round(tot_f / tot_t / 1e12, 2),
                                                 "frac_mfma": round(tot_f / tot_t / PEAK_FP32_MFMA, 4),
                                                 "flop": tot_f}
    del X, G, W, dX, dW

    # ConvTranspose1d upsampler backwards (dgrad + wgrad)
    res = {}
    for name, (Ci, Co, Lin, kk, ss, pp) in {"ups0_512to256_k20_s10_x4x512": (512, 256, 512, 20, 10, 5),
                                          "ups1_256to128_k12_s6_x4x5120": (256, 128, 5120, 12, 6, 3)}.items():
        Lo = (Lin - 1) * ss - 2 * pp + kk
        Xt = dev(synth.normal(f"micro.{name}.x", (4, Ci, Lin)))
        Gt = dev(synth.normal(f"micro.{name}.g", (4, Co, Lo)))
        Wt = dev(synth.uniform(f"micro.{name}.w", (Ci, Co * kk), -0.05, 0.05))
        dXt = torch.empty_like(Xt)
        dWt = torch.zeros_like(Wt)
        dbt = torch.zeros(Co, device="cuda")

        def run():
            ctx.call("kdec_convt1d_dgrad", P(Wt), P(Gt), Co * Lo, P(dXt), Ci * Lin, 4, Ci, Lin, Co, kk, ss, pp, 0)
            ctx.call("kdec_convt1d_wgrad", P(Xt), Ci * Lin, P(Gt), Co * Lo, P(dWt), P(dbt), 4, Ci, Lin, Co, kk, ss,
                     pp, 0)
        t = timed(run)
        fl = 2 * 2.0 * 4 * Ci * Co * kk * Lin
        res[name] = {"ms": round(t * 1e3, 4), "TFLOP/s": round(fl / t / 1e12, 2),
                     "frac_mfma": round(fl / t / PEAK_FP32_MFMA, 4), "flop": fl}
    out["convT_bwd"] = res
    del Xt, Gt, Wt, dXt, dWt

    # iSTFT head (n_fft 20, hop 5) at the benchmark's shape, B = 8 utterances
    # of 61 441 frames: backward reads post [8, 22, 61441] and dAudio
    # [8, 307200] and writes dpost; forward reads post and writes audio
    Nb, Lf, nfft, hop = 8, 61441, 20, 5
    sig = (Lf - 1) * hop
    post = dev(synth.normal("micro.post", (Nb, nfft + 2, Lf), 0.5))
    da = dev(synth.normal("micro.daudio", (Nb, sig)))
    dpost = torch.empty_like(post)
    aud = torch.empty(Nb, sig, device="cuda")
    t = timed(lambda: ctx.call("kdec_spectral_bwd", P(post), (nfft + 2) * Lf, None, P(da), sig, P(dpost),
                               (nfft + 2) * Lf, Nb, Lf, nfft, hop))
    by = 4.0 * Nb * (2.0 * (nfft + 2) * Lf + sig)
    out["istft_bwd_x8x22x61441"] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                    "frac_hbm": round(by / t / PEAK_HBM, 4), "algorithmic_bytes": by}
    t = timed(lambda: ctx.call("kdec_spectral_fwd", P(post), (nfft + 2) * Lf, None, P(aud), sig, Nb, Lf, nfft,
                               hop))
    by = 4.0 * Nb * ((nfft + 2) * Lf + sig)
    out["istft_fwd_x8x22x61441"] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                    "frac_hbm": round(by / t / PEAK_HBM, 4), "algorithmic_bytes": by}
    del post, da, dpost, aud

    # style projection of every AdaIN unit at once (R rows of the stacked fc,
    # S = 128, B = 8): forward (gamma, beta) and d(style)
    from brosoundml_amd import config as Cfg
    R, S = Cfg.affine_rows(Cfg.KOKORO), 128
    Wf = dev(synth.uniform("micro.fcw", (R, S), -0.09, 0.09))
    bf = dev(synth.uniform("micro.fcb", (R,), -0.09, 0.09))
    st = dev(synth.normal("micro.style", (Nb, S), 0.3))
    gbv = torch.empty(Nb, R, device="cuda")
    dgbv = dev(synth.normal("micro.dgb", (Nb, R)))
    dst = torch.empty(Nb, S, device="cuda")
    t = timed(lambda: ctx.call("kdec_style_proj_fwd", P(Wf), P(bf), P(st), S, P(gbv), R, Nb, R, S))
    by = 4.0 * (R * S + R + Nb * (S + R))
    out["style_proj_fwd_R%d_x8" % R] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                        "frac_hbm": round(by / t / PEAK_HBM, 4), "algorithmic_bytes": by}
    t = timed(lambda: ctx.call("kdec_style_proj_bwd", P(Wf), P(st), S, P(dgbv), R, P(dst), S, 0.0, None, None, Nb,
                               R, S))
    by = 4.0 * (R * S + Nb * (S + R))
    out["style_proj_dstyle_R%d_x8" % R] = {"ms": round(t * 1e3, 4), "GB/s": round(by / t / 1e9, 1),
                                           "frac_hbm": round(by / t / PEAK_HBM, 4), "algorithmic_bytes": by}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ref-steps", type=int, default=3, help="steps of the reference-semantics mode")
    ap.add_argument("--no-micro", action="store_true", help="skip the per-kernel-class microbenchmarks")
    ap.add_argument("--no-serving", action="store_true",
                    help="skip the inference-forward and DecoderLora-step lines (profiles of the training step)")
    ap.add_argument("--micro-only", action="store_true",
                    help="run only the per-kernel-class microbenchmarks and print their JSON (for profiling them)")
    ap.add_argument("--serial", action="store_true",
                    help="one stream (no harmonic-source / weight-grad overlap): per-family times without sharing")
    ap.add_argument("--serial-steps", type=int, default=3,
                    help="steps of a one-stream pass after the timed region (serial family times and GEMM rate)")
    ap.add_argument("--batch-split", type=int, default=0,
                    help="1: run the batch as two half-batch chains on two streams (kdec_model_set_batch_split); "
                         "0 (default): one chain")
    ap.add_argument("--cpu-plan", action="store_true",
                    help="run only the full CPU baseline plan (configs 0-4 on the oracle, 1 thread and all cores, "
                         "medians of 3) and print its JSON; several minutes")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (3 times): the reference kernel for "
                         "scaling HBM byte counters")
    a = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the decoder path shards by utterance with no exchange, "
              "and this build runs on a single GPU; use --gpus 1.", file=sys.stderr)
        return 2

    if a.cpu_plan:
        from brosoundml_amd import config as C, synth
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        shapes = O.OracleModel(C.KOKORO).param_shapes()
        print(json.dumps({"cpu_plan": cpu_plan(C.KOKORO, synth.init_params(shapes))}), flush=True)
        return 0

    import torch
    from brosoundml_amd import config as C, native, synth

    cfg = C.KOKORO
    lens = C.lengths(cfg, T)
    if a.calib_copy_mib > 0:
        n = a.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    ctx = native.Context(0)
    if a.micro_only:
        print(json.dumps({"micro": micro_benches(ctx)}), flush=True)
        return 0
    model = native.Model(ctx, cfg)
    shapes = model.param_shapes()
    params = synth.init_params(shapes)
    model.set_params(params)
    if a.serial:
        model.set_overlap(False)
    model.set_batch_split(a.batch_split)
    asr, F0, Nn, style, dA = make_inputs(cfg, B, T, "bench")
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    t_asr, t_F0, t_N, t_style, t_dA = (dev(x) for x in (asr, F0, Nn, style, dA))
    audio = torch.empty(B, lens["audio"], device="cuda")
    dstyle = torch.empty_like(t_style)

    def step(full=True):
        model.zero_grad()
        model.forward(t_asr, t_F0, t_N, t_style, T, audio=audio)
        model.backward(t_dA, wgrad=full, dalpha=full, dstyle=dstyle if full else None)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    # timed region: K steps with nothing recorded between launches
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    if not torch.isfinite(audio).all() or not torch.isfinite(dstyle).all():
        print("non-finite output", file=sys.stderr)
        return 1
    # profiled region: the same K steps again with a HIP event pair around
    # every kernel family launch, on the stream it runs on (the per-family
    # times and the roofline); the events themselves lengthen a step by a
    # millisecond or two, which is why the throughput is timed without them
    ctx.profile(True)
    ctx.profile_reset()
    torch.cuda.synchronize()
    p0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    pdt = time.perf_counter() - p0
    prof = ctx.profile_read()
    ctx.profile(False)

    # the same step on one stream after the timed region: per-family times
    # and the conv GEMM rate without the weight-grad lane sharing the CUs
    serial = {}
    if a.serial_steps > 0 and not a.serial:
        model.set_overlap(False)
        step()
        torch.cuda.synchronize()
        s0 = time.perf_counter()
        for _ in range(a.serial_steps):
            step()
        torch.cuda.synchronize()
        sdt = (time.perf_counter() - s0) / a.serial_steps
        ctx.profile(True)
        ctx.profile_reset()
        s0 = time.perf_counter()
        for _ in range(a.serial_steps):
            step()
        torch.cuda.synchronize()
        spdt = (time.perf_counter() - s0) / a.serial_steps
        sprof = ctx.profile_read()
        ctx.profile(False)
        model.set_overlap(True)
        serial = {"ms_per_step": round(sdt * 1e3, 3), "profiled_ms_per_step": round(spdt * 1e3, 3),
                  "steps": a.serial_steps, "prof": sprof}

    # reference semantics (conv dgrad only, alpha grad dropped, no d(style))
    ref = {}
    if a.ref_steps > 0:
        step(False)
        torch.cuda.synchronize()
        r0 = time.perf_counter()
        for _ in range(a.ref_steps):
            step(False)
        torch.cuda.synchronize()
        rdt = (time.perf_counter() - r0) / a.ref_steps
        ref = {"ms_per_step": round(rdt * 1e3, 3), "value": round(B * lens["audio_seconds"] / rdt, 3)}

    ms = dt / a.steps * 1e3
    audio_per_step = B * lens["audio_seconds"]
    value = audio_per_step / (dt / a.steps)

    # dominant kernel: the conv implicit GEMM family with the most time
    GEMM_FAMS = ("conv_fwd", "conv_dgrad", "convt_fwd", "convt_dgrad")
    conv_fams = {k: v for k, v in prof.items() if k in GEMM_FAMS}
    gemm_ms = sum(v["ms"] for v in conv_fams.values())
    gemm_flops = sum(v["flops"] for v in conv_fams.values())
    gemm_bytes = sum(v["bytes"] for v in conv_fams.values())
    gemm_launches = sum(v["launches"] for v in conv_fams.values())
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if os.path.exists(tpath):  # measured HBM bytes per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE passes)
        with open(tpath) as f:
            traffic = json.load(f).get("conv_gemm", {}).get("bytes_per_launch")
    wg = prof.get("conv_wgrad", {"ms": 0, "flops": 0, "launches": 0})
    wgt = prof.get("convt_wgrad", {"ms": 0, "flops": 0, "launches": 0})
    achieved = gemm_flops / (gemm_ms * 1e-3) if gemm_ms else 0.0
    total_conv_flops = gemm_flops + wg["flops"] + wgt["flops"]
    # step roofline: every conv FLOP at the FP32-MFMA peak plus the compulsory
    # elementwise bytes (8 B/elem forward, 12 B/elem backward over the AdaIN
    # units' elements) at the HBM peak
    elems = adain_elements(cfg, T) * B
    ideal_s = (total_conv_flops / a.steps) / PEAK_FP32_MFMA + 20.0 * elems / PEAK_HBM
    out = {
        "metric": "Kokoro decoder fwd+bwd audio-sec/s (T=512,B=8); % of FP32-MFMA/HBM roofline",
        "value": round(value, 3),
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic inputs, random-init FP32 weights at Kokoro-82M shapes",
        "config": {"workload": "Kokoro-82M iSTFTNet decoder back half fwd+bwd incl. harmonic source and "
                               "iSTFT backward, with conv/convT/pool/fc weight grads, Snake alpha grads, d(style)",
                   "batch": B, "T": T, "audio_s_per_utterance": lens["audio_seconds"],
                   "audio_s_per_step": audio_per_step, "params": int(sum(np.prod(s) for s in shapes.values()))},
        "roofline": {"bound": "mfma", "kernel": "conv_gemm (conv1d fwd / dgrad, convT fwd / dgrad)",
                     "achieved": round(achieved / 1e12, 3), "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": traffic,
                     "region": "profiled pass of the same K steps (events around every family launch)",
                     "algorithmic_bytes_per_launch": round(gemm_bytes / max(gemm_launches, 1)),
                     "launches_per_step": gemm_launches // a.steps,
                     "ms_per_step": round(gemm_ms / a.steps, 3),
                     "flop_per_step": gemm_flops / a.steps},
        "wgrad_roofline": {"kernel": "wgrad_gemm", "achieved": round(
            (wg["flops"] + wgt["flops"]) / max((wg["ms"] + wgt["ms"]) * 1e-3, 1e-12) / 1e12, 3),
            "unit": "TFLOP/s", "ms_per_step": round((wg["ms"] + wgt["ms"]) / a.steps, 3)},
        "step_roofline": {"ideal_ms": round(ideal_s * 1e3, 3), "frac": round(ideal_s * 1e3 / ms, 4),
                          "conv_tflop_per_step": round(total_conv_flops / a.steps / 1e12, 4),
                          "elementwise_gb_per_step": round(20.0 * elems / 1e9, 3)},
        "profiled_ms_per_step": round(pdt / a.steps * 1e3, 3),
        "families_ms_per_step": {k: round(v["ms"] / a.steps, 3) for k, v in sorted(prof.items())},
        "reference_semantics": ref,
        "streams": 1 if a.serial else 2,
    }
    if serial:
        sp, n = serial.pop("prof"), serial["steps"]
        s_ms = sum(v["ms"] for k, v in sp.items() if k in GEMM_FAMS)
        s_fl = sum(v["flops"] for k, v in sp.items() if k in GEMM_FAMS)
        swg = [sp.get(k, {"ms": 0, "flops": 0}) for k in ("conv_wgrad", "convt_wgrad")]
        w_ms, w_fl = sum(v["ms"] for v in swg), sum(v["flops"] for v in swg)
        serial["roofline"] = {"kernel": out["roofline"]["kernel"], "achieved": round(s_fl / (s_ms * 1e-3) / 1e12, 3)
                              if s_ms else 0.0, "frac": round(s_fl / (s_ms * 1e-3) / PEAK_FP32_MFMA, 4) if s_ms else 0.0,
                              "ms_per_step": round(s_ms / n, 3)}
        serial["wgrad_roofline"] = {"achieved": round(w_fl / max(w_ms * 1e-3, 1e-12) / 1e12, 3),
                                    "frac": round(w_fl / max(w_ms * 1e-3, 1e-12) / PEAK_FP32_MFMA, 4),
                                    "ms_per_step": round(w_ms / n, 3)}
        serial["families_ms_per_step"] = {k: round(v["ms"] / n, 3) for k, v in sorted(sp.items())}
        out["serial"] = serial
        # The roofline figure is the one-stream pass's: there each conv GEMM
        # launch has the GPU to itself, so the family's launch time per step
        # stays within the step. On the default schedule up to three conv
        # GEMMs and the weight-grad GEMMs share the CUs, each launch's
        # duration also holds the others' work, and the family's summed
        # launch time exceeds the step; that figure is kept, labelled.
        rf = out["roofline"]
        rf["frac_overlapped"], rf["achieved_overlapped"] = rf["frac"], rf["achieved"]
        rf["ms_per_step_overlapped"] = rf["ms_per_step"]
        rf["achieved"], rf["frac"] = serial["roofline"]["achieved"], serial["roofline"]["frac"]
        rf["ms_per_step"] = serial["roofline"]["ms_per_step"]
        rf["region"] = ("one-stream pass of the same step after the timed region (events around every family "
                        "launch); *_overlapped: the profiled pass of the default schedule")
    out["step_roofline"]["frac_serial"] = round(ideal_s * 1e3 / serial["ms_per_step"], 4) if serial else None
    if not a.no_serving:
        out["inference"] = inference_bench(ctx, model, t_asr, t_F0, t_N, t_style, audio, audio_per_step)
        out["lora_train_step"] = lora_bench(model, t_asr, t_F0, t_N, t_style, t_dA, audio_per_step)
    if not a.no_micro:
        out["micro"] = micro_benches(ctx)
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, params)
    print(json.dumps(out))
    return 0


def inference_bench(ctx, model, asr, F0, Nn, style, audio, audio_per_step, reps=5):
    """The serving path: the decoder back half forward only (harmonic source,
    backbone, generator, iSTFT) without training caches, B utterances of T
    frames, as decode_back_half runs it."""
    import torch
    from brosoundml_amd import native
    P = native.ptr
    run = lambda: model._c(ctx.L.kdec_model_infer(model.h, B, T, P(asr), P(F0), P(Nn), P(style), None, P(audio)))
    run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    return {"ms_per_step": round(dt * 1e3, 3), "value": round(audio_per_step / dt, 2), "unit": "audio-s/s",
            "workload": f"decoder back half forward only (no caches), B={B}, T={T}"}


def lora_bench(model, asr, F0, Nn, style, dA, audio_per_step, reps=3):
    """One DecoderLora training step (decoder_lora.cpp:211-314): gate,
    forward with the adapters on every AdaIN unit, backward to the affine
    grads and through the adapters and gate (frozen decoder: no weight
    grads), Adam over A, B and the gate; rank 4, one condition per utterance."""
    import torch
    from brosoundml_amd import native
    d = native.DecoderLora(model, 4, 1.0, seed=11)
    d.set("W2", np.full((4, 16), 0.05, np.float32))
    cond = torch.full((B, 3), 0.3, device="cuda")
    ref_s = torch.cat([style, style], dim=1).contiguous()

    def step():
        d.zero_grad()
        d.forward(asr, F0, Nn, ref_s, T, cond)
        d.backward(dA)
        d.adam_step(1e-4)
    step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    del d
    return {"ms_per_step": round(dt * 1e3, 3), "value": round(audio_per_step / dt, 2), "unit": "audio-s/s",
            "workload": f"DecoderLora step (rank 4, frozen decoder), B={B}, T={T}"}


def adain_elements(cfg, T):
    """Elements passing through AdaIN(+activation) units per utterance."""
    lg = 2 * T
    e = (cfg["asr_dim"] + 2) * T + cfg["enc_dim"] * T          # encode norm1, norm2
    prev, res, Lnow = cfg["enc_dim"], True, T
    for i in range(cfg["n_decode"]):
        din = prev + cfg["asr_res_dim"] + 2 if res else prev
        up = i == cfg["dec_up_at"]
        Lout = 2 * Lnow if up else Lnow
        e += din * Lnow + cfg["dec_out"][i] * Lout
        prev, Lnow = cfg["dec_out"][i], Lout
        if up:
            res = False
    init_C = cfg["dec_out"][cfg["n_decode"] - 1]
    L = lg
    for i in range(cfg["n_ups"]):
        L = L * cfg["ups_rates"][i] + (1 if i == cfg["n_ups"] - 1 else 0)
        Cc = init_C >> (i + 1)
        e += (1 + cfg["n_kernels"]) * 6 * Cc * L
    return e


if __name__ == "__main__":
    sys.exit(main())
