"""Golden vectors (tests/golden/*.npz, written by tests/golden/make_golden.py
from PyTorch's float64 CPU ops) checked against the CPU oracle and, on a GPU,
against the HIP path through the C ABI.

The fixtures pin the semantics both implementations share (conv / conv-
transpose geometry, the AdaIN (1 + gamma) affine with eps 1e-5, the Snake and
leaky-ReLU derivatives, the exp / sin polar form and the centred iSTFT, the
reflect-padded STFT) to an implementation outside this repository. Bars:
rel-L2 <= 1e-5 for forward values, <= 1e-4 for gradients.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FWD_TOL = 1e-5
GRAD_TOL = 1e-4


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    assert a.shape == b.shape, (a.shape, b.shape)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_close(got, ref, tol, what):
    e = rel_l2(got, ref)
    mx = float(np.max(np.abs(np.asarray(got, np.float64).ravel() - np.asarray(ref, np.float64).ravel())))
    assert e <= tol, f"{what}: rel-L2 {e:.3e} > {tol:.0e} (max-abs {mx:.3e})"


CONV = load("conv")
CONVT = load("convt")
ADAIN = load("adain")
SPEC = load("spectral")
STFT = load("stft")
CONV_IDS = sorted({k.split("_")[0] for k in CONV})
CONVT_IDS = sorted({k.split("_")[0] for k in CONVT})


# ─── oracle (CPU) ────────────────────────────────────────────────────────

@pytest.mark.parametrize("cid", CONV_IDS)
def test_oracle_conv1d(cid):
    c = {k[len(cid) + 1:]: v for k, v in CONV.items() if k.startswith(cid + "_")}
    N, Ci, Co, L, k, s, p, d = (int(v) for v in c["geo"])
    Lo = O.conv1d_out_len(L, k, s, p, d)
    y = np.stack([O.conv1d(c["x"][n], c["W"], c["b"], Ci, L, Co, k, s, p, d).reshape(Co, Lo) for n in range(N)])
    assert_close(y, c["y"], FWD_TOL, f"{cid} forward")
    dx = np.stack([O.conv1d_dgrad(c["W"], c["dy"][n], Ci, L, Co, k, s, p, d).reshape(Ci, L) for n in range(N)])
    assert_close(dx, c["dx"], GRAD_TOL, f"{cid} input grad")
    dW, db = 0.0, 0.0
    for n in range(N):
        a, bb = O.conv1d_wgrad(c["x"][n], c["dy"][n], Ci, L, Co, k, s, p, d)
        dW, db = dW + a, db + bb
    assert_close(dW, c["dW"], GRAD_TOL, f"{cid} weight grad")
    assert_close(db, c["db"], GRAD_TOL, f"{cid} bias grad")


@pytest.mark.parametrize("cid", CONVT_IDS)
def test_oracle_convt1d(cid):
    c = {k[len(cid) + 1:]: v for k, v in CONVT.items() if k.startswith(cid + "_")}
    N, Ci, Co, L, k, s, p, op, grp = (int(v) for v in c["geo"])
    Lo = O.convt1d_out_len(L, k, s, p, op, 1)
    y = np.stack([O.convt1d(c["x"][n], c["W"], c["b"], Ci, L, Co, k, s, p, op, 1, grp).reshape(Co, Lo)
                  for n in range(N)])
    assert_close(y, c["y"], FWD_TOL, f"{cid} forward")
    dx = np.stack([O.convt1d_dgrad(c["W"], c["dy"][n], Ci, L, Co, k, s, p, op, 1, grp).reshape(Ci, L)
                   for n in range(N)])
    assert_close(dx, c["dx"], GRAD_TOL, f"{cid} input grad")
    dW, db = 0.0, 0.0
    for n in range(N):
        a, bb = O.convt1d_wgrad(c["x"][n], c["dy"][n], Ci, L, Co, k, s, p, op, 1, grp)
        dW, db = dW + a, db + bb
    assert_close(dW, c["dW"], GRAD_TOL, f"{cid} weight grad")
    assert_close(db, c["db"], GRAD_TOL, f"{cid} bias grad")


@pytest.mark.parametrize("act", ["none", "leaky", "snake"])
def test_oracle_adain_act(act):
    a = ADAIN
    N, C, L = (int(v) for v in a["shape"])
    slope = float(a["slope"])
    ys, dxs, dgs, dbs, das = [], [], [], [], 0.0
    for n in range(N):
        x, gm, bt = a["x"][n], a["gamma"][n], a["beta"][n]
        s = O.adain_affine(x, gm, bt, C, L)
        dy = a[f"{act}_dy"][n]
        if act == "none":
            y, ds = s, dy
        elif act == "leaky":
            y, ds = O.leaky(s, slope), O.leaky_bwd(s, dy, slope)
        else:
            y = O.snake(s, a["alpha"], C, L)
            ds, da = O.snake_bwd(s, a["alpha"], dy, C, L)
            das = das + da
        dx, dg, db = O.adain_affine_bwd(x, gm, ds, C, L)
        ys.append(y); dxs.append(dx); dgs.append(dg); dbs.append(db)
    assert_close(np.stack(ys), a[f"{act}_y"], FWD_TOL, f"adain+{act} forward")
    assert_close(np.stack(dxs), a[f"{act}_dx"], GRAD_TOL, f"adain+{act} input grad")
    assert_close(np.stack(dgs), a[f"{act}_dgamma"], GRAD_TOL, f"adain+{act} gamma grad")
    assert_close(np.stack(dbs), a[f"{act}_dbeta"], GRAD_TOL, f"adain+{act} beta grad")
    if act == "snake":
        assert_close(das, a["snake_dalpha"], GRAD_TOL, "snake alpha grad")


def test_oracle_spectral_head():
    sp = SPEC
    N, C, n_fft, hop, L, k = (int(v) for v in sp["shape"])
    audio = np.stack([O.spectral_head(sp["x"][n], C, L, sp["W"], sp["b"], k, n_fft, hop)[0] for n in range(N)])
    assert_close(audio, sp["audio"], FWD_TOL, "spectral head forward")
    dx, dW, db = [], 0.0, 0.0
    for n in range(N):
        a, w, b = O.spectral_head_bwd(sp["x"][n], C, L, sp["W"], sp["b"], k, n_fft, hop, sp["daudio"][n])
        dx.append(a); dW, db = dW + w, db + b
    assert_close(np.stack(dx), sp["dx"], GRAD_TOL, "spectral head input grad")
    assert_close(dW, sp["dW"], GRAD_TOL, "conv_post weight grad")
    assert_close(db, sp["db"], GRAD_TOL, "conv_post bias grad")


def test_oracle_stft():
    st = STFT
    n_fft, hop, length = (int(v) for v in st["shape"])
    spec, frames = O.stft(st["x"], O.hann(n_fft), n_fft, hop)
    spec = spec.reshape(frames, n_fft // 2 + 1, 2)
    assert_close(spec[..., 0], st["re"], FWD_TOL, "stft real")
    assert_close(spec[..., 1], st["im"], FWD_TOL, "stft imag")
    assert_close(np.hypot(spec[..., 0], spec[..., 1]), st["mag"], FWD_TOL, "stft magnitude")


# ─── HIP path (GPU) ──────────────────────────────────────────────────────

@pytest.fixture(scope="module")
def K():
    pytest.importorskip("torch")
    from brosoundml_amd import native
    return native.Context(0)


def _torch():
    import torch
    return torch


def dev(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch = _torch()
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def P(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@pytest.mark.gpu
@pytest.mark.parametrize("cid", CONV_IDS)
def test_gpu_conv1d(K, cid):
    torch = _torch()
    c = {k[len(cid) + 1:]: v for k, v in CONV.items() if k.startswith(cid + "_")}
    N, Ci, Co, L, k, s, p, d = (int(v) for v in c["geo"])
    Lo = O.conv1d_out_len(L, k, s, p, d)
    x, W, b, dy = dev(c["x"]), dev(c["W"]), dev(c["b"]), dev(c["dy"])
    Y = torch.empty(N, Co, Lo, device="cuda")
    K.call("kdec_conv1d_fwd", P(x), Ci * L, P(W), P(b), P(Y), Co * Lo, N, Ci, L, Co, k, s, p, d, None, 0, 1.0, 0.0)
    assert_close(host(Y), c["y"], FWD_TOL, f"{cid} forward")
    if s == 1:  # the input grad of the strided convs is not on the decoder path
        dX = torch.empty(N, Ci, L, device="cuda")
        K.call("kdec_conv1d_dgrad", P(W), P(dy), Co * Lo, P(dX), Ci * L, N, Ci, L, Co, k, s, p, d, 1.0, 0.0)
        assert_close(host(dX), c["dx"], GRAD_TOL, f"{cid} input grad")
    dW = torch.zeros(Co, Ci * k, device="cuda")
    db = torch.zeros(Co, device="cuda")
    K.call("kdec_conv1d_wgrad", P(x), Ci * L, P(dy), Co * Lo, P(dW), P(db), N, Ci, L, Co, k, s, p, d)
    assert_close(host(dW), c["dW"], GRAD_TOL, f"{cid} weight grad")
    assert_close(host(db), c["db"], GRAD_TOL, f"{cid} bias grad")


@pytest.mark.gpu
@pytest.mark.parametrize("cid", CONVT_IDS)
def test_gpu_convt1d(K, cid):
    torch = _torch()
    c = {k[len(cid) + 1:]: v for k, v in CONVT.items() if k.startswith(cid + "_")}
    N, Ci, Co, L, k, s, p, op, grp = (int(v) for v in c["geo"])
    Lo = O.convt1d_out_len(L, k, s, p, op, 1)
    x, W, b, dy = dev(c["x"]), dev(c["W"]), dev(c["b"]), dev(c["dy"])
    Y = torch.empty(N, Co, Lo, device="cuda")
    dX = torch.empty(N, Ci, L, device="cuda")
    dW = torch.zeros(*c["dW"].shape, device="cuda")
    db = torch.zeros(Co, device="cuda")
    if grp == 1:
        K.call("kdec_convt1d_fwd", P(x), Ci * L, P(W), P(b), P(Y), Co * Lo, N, Ci, L, Co, k, s, p, op)
        K.call("kdec_convt1d_dgrad", P(W), P(dy), Co * Lo, P(dX), Ci * L, N, Ci, L, Co, k, s, p, op)
        K.call("kdec_convt1d_wgrad", P(x), Ci * L, P(dy), Co * Lo, P(dW), P(db), N, Ci, L, Co, k, s, p, op)
    else:  # the depthwise k3 s2 p1 op1 pool
        assert (Ci, Co, k, s, p, op) == (grp, grp, 3, 2, 1, 1)
        K.call("kdec_pool_fwd", P(x), Ci * L, P(W), P(b), P(Y), Co * Lo, N, Ci, L)
        K.call("kdec_pool_dgrad", P(W), P(dy), Co * Lo, P(dX), Ci * L, N, Ci, L)
        K.call("kdec_pool_wgrad", P(x), Ci * L, P(dy), Co * Lo, P(dW), P(db), N, Ci, L)
    assert_close(host(Y), c["y"], FWD_TOL, f"{cid} forward")
    assert_close(host(dX), c["dx"], GRAD_TOL, f"{cid} input grad")
    assert_close(host(dW), c["dW"], GRAD_TOL, f"{cid} weight grad")
    assert_close(host(db), c["db"], GRAD_TOL, f"{cid} bias grad")


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["none", "leaky", "snake"])
def test_gpu_adain_act(K, act):
    torch = _torch()
    a = ADAIN
    N, C, L = (int(v) for v in a["shape"])
    code = {"none": 0, "leaky": 1, "snake": 2}[act]
    x = dev(a["x"])
    gb = dev(np.concatenate([a["gamma"], a["beta"]], 1))  # (N, 2C): gamma then beta
    gam, bet = P(gb), ctypes.c_void_p(gb.data_ptr() + 4 * C)
    alpha = dev(a["alpha"])
    stats = torch.empty(N * C, 2, device="cuda")
    Y = torch.empty(N, C, L, device="cuda")
    K.call("kdec_instnorm_stats", P(x), C * L, N, C, L, float(a["eps"]), P(stats))
    K.call("kdec_adain_act_fwd", P(x), C * L, P(stats), gam, bet, 2 * C, code, float(a["slope"]), P(alpha), P(Y),
           C * L, None, 0, N, C, L)
    assert_close(host(Y), a[f"{act}_y"], FWD_TOL, f"adain+{act} forward")
    dy = dev(a[f"{act}_dy"])
    dX = torch.empty(N, C, L, device="cuda")
    dgb = torch.zeros(N, 2 * C, device="cuda")
    da = torch.zeros(C, device="cuda")
    K.call("kdec_adain_act_bwd", P(x), C * L, P(stats), gam, bet, 2 * C, code, float(a["slope"]), P(alpha),
           P(dy), C * L, None, 0, P(dX), C * L, P(dgb), ctypes.c_void_p(dgb.data_ptr() + 4 * C), 2 * C,
           P(da) if act == "snake" else None, N, C, L)
    g = host(dgb)
    assert_close(host(dX), a[f"{act}_dx"], GRAD_TOL, f"adain+{act} input grad")
    assert_close(g[:, :C], a[f"{act}_dgamma"], GRAD_TOL, f"adain+{act} gamma grad")
    assert_close(g[:, C:], a[f"{act}_dbeta"], GRAD_TOL, f"adain+{act} beta grad")
    if act == "snake":
        assert_close(host(da), a["snake_dalpha"], GRAD_TOL, "snake alpha grad")


@pytest.mark.gpu
def test_gpu_spectral_head(K):
    torch = _torch()
    sp = SPEC
    N, C, n_fft, hop, L, k = (int(v) for v in sp["shape"])
    Fq2 = n_fft + 2
    x, W, b = dev(sp["x"]), dev(sp["W"]), dev(sp["b"])
    xl = torch.empty(N, C, L, device="cuda")
    K.call("kdec_leaky_fwd", P(x), C * L, P(xl), C * L, N, C * L, 0.01)
    post = torch.empty(N, Fq2, L, device="cuda")
    K.call("kdec_conv1d_fwd", P(xl), C * L, P(W), P(b), P(post), Fq2 * L, N, C, L, Fq2, k, 1, (k - 1) // 2, 1,
           None, 0, 1.0, 0.0)
    S = (L - 1) * hop
    audio = torch.empty(N, S, device="cuda")
    K.call("kdec_spectral_fwd", P(post), Fq2 * L, None, P(audio), S, N, L, n_fft, hop)
    assert_close(host(audio), sp["audio"], FWD_TOL, "spectral head forward")
    da = dev(sp["daudio"])
    dpost = torch.empty(N, Fq2, L, device="cuda")
    K.call("kdec_spectral_bwd", P(post), Fq2 * L, None, P(da), S, P(dpost), Fq2 * L, N, L, n_fft, hop)
    dxl = torch.empty(N, C, L, device="cuda")
    K.call("kdec_conv1d_dgrad", P(W), P(dpost), Fq2 * L, P(dxl), C * L, N, C, L, Fq2, k, 1, (k - 1) // 2, 1,
           1.0, 0.0)
    dx = torch.empty(N, C, L, device="cuda")
    K.call("kdec_leaky_bwd", P(x), C * L, P(dxl), C * L, P(dx), C * L, N, C * L, 0.01)
    dW = torch.zeros(Fq2, C * k, device="cuda")
    db = torch.zeros(Fq2, device="cuda")
    K.call("kdec_conv1d_wgrad", P(xl), C * L, P(dpost), Fq2 * L, P(dW), P(db), N, C, L, Fq2, k, 1, (k - 1) // 2, 1)
    assert_close(host(dx), sp["dx"], GRAD_TOL, "spectral head input grad")
    assert_close(host(dW), sp["dW"], GRAD_TOL, "conv_post weight grad")
    assert_close(host(db), sp["db"], GRAD_TOL, "conv_post bias grad")
