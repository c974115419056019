"""Pins the CPU oracle's op restatements.

Each op is checked against what fixes it independently of the oracle's own
code: PyTorch's reference implementation of the same op (a third-party library,
run here in float64), the reference's known-answer tests
(tests/test_modules.cpp:151-177, 356-386), adjoint dot-product identities and
closed forms (the periodic-Hann overlap-add constant, istft o stft = identity,
brute-force DFT). A dropped term, a wrong sign, index or transposed operand in
the oracle fails at least one of these.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

import oracle_lib as O

rng = np.random.default_rng(1234)


def rnd(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def t64(a):
    return torch.tensor(np.asarray(a, dtype=np.float64))


def close(a, b, rtol=2e-5, atol=2e-5):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    assert a.shape == b.shape
    err = np.abs(a - b).max() if a.size else 0.0
    scale = max(np.abs(b).max() if b.size else 0.0, 1.0)
    assert err <= atol + rtol * scale, f"max abs err {err} (scale {scale})"


CONV_CASES = [
    # C_in, C_out, L, k, s, p, d, g
    (3, 4, 17, 3, 1, 1, 1, 1),
    (4, 6, 20, 7, 1, 9, 3, 1),
    (5, 3, 33, 11, 1, 25, 5, 1),
    (2, 4, 31, 12, 6, 3, 1, 1),     # noise_convs-style strided
    (1, 1, 16, 3, 2, 1, 1, 1),      # F0_conv / N_conv
    (6, 6, 19, 3, 1, 1, 1, 3),      # grouped
    (8, 5, 9, 1, 1, 0, 1, 1),       # 1x1
]


@pytest.mark.parametrize("C_in,C_out,L,k,s,p,d,g", CONV_CASES)
def test_conv1d_vs_torch(C_in, C_out, L, k, s, p, d, g):
    x = rnd(C_in, L)
    W = rnd(C_out, C_in // g, k, scale=0.3)
    b = rnd(C_out)
    y = O.conv1d(x, W, b, C_in, L, C_out, k, s, p, d, g)
    xt = t64(x)[None].requires_grad_(True)
    Wt = t64(W).requires_grad_(True)
    bt = t64(b).requires_grad_(True)
    yt = Fn.conv1d(xt, Wt, bt, stride=s, padding=p, dilation=d, groups=g)
    close(y, yt.detach().numpy())
    dy = rnd(*yt.shape[1:])
    yt.backward(t64(dy)[None])
    dx = O.conv1d_dgrad(W, dy, C_in, L, C_out, k, s, p, d, g)
    close(dx, xt.grad.numpy())
    dW, db = O.conv1d_wgrad(x, dy, C_in, L, C_out, k, s, p, d, g)
    close(dW, Wt.grad.numpy())
    close(db, bt.grad.numpy())


CONVT_CASES = [
    # C_in, C_out, L, k, s, p, op, d, g
    (4, 3, 9, 20, 10, 5, 0, 1, 1),   # ups0 geometry
    (3, 2, 11, 12, 6, 3, 0, 1, 1),   # ups1 geometry
    (5, 5, 8, 3, 2, 1, 1, 1, 5),     # depthwise pool k3 s2 p1 op1
    (3, 4, 7, 5, 3, 1, 0, 1, 1),     # k not a multiple of s
    (2, 3, 6, 4, 2, 1, 0, 2, 1),     # dilated
]


@pytest.mark.parametrize("C_in,C_out,L,k,s,p,op,d,g", CONVT_CASES)
def test_convt1d_vs_torch(C_in, C_out, L, k, s, p, op, d, g):
    x = rnd(C_in, L)
    W = rnd(C_in, C_out // g, k, scale=0.3)
    b = rnd(C_out)
    y = O.convt1d(x, W, b, C_in, L, C_out, k, s, p, op, d, g)
    xt = t64(x)[None].requires_grad_(True)
    Wt = t64(W).requires_grad_(True)
    bt = t64(b).requires_grad_(True)
    yt = Fn.conv_transpose1d(xt, Wt, bt, stride=s, padding=p, output_padding=op, groups=g,
                             dilation=d)
    close(y, yt.detach().numpy())
    dy = rnd(*yt.shape[1:])
    yt.backward(t64(dy)[None])
    dx = O.convt1d_dgrad(W, dy, C_in, L, C_out, k, s, p, op, d, g)
    close(dx, xt.grad.numpy())
    dW, db = O.convt1d_wgrad(x, dy, C_in, L, C_out, k, s, p, op, d, g)
    close(dW, Wt.grad.numpy())
    close(db, bt.grad.numpy())


def test_conv_adjoint_identities():
    # <conv(x), y> == <x, dgrad(y)> and <dW, W'> == <dY, conv(X, W')>
    C_in, C_out, L, k, s, p, d = 6, 5, 40, 7, 1, 9, 3
    x, W, y = rnd(C_in, L), rnd(C_out, C_in, k), None
    Lo = O.conv1d_out_len(L, k, s, p, d)
    y = rnd(C_out, Lo)
    lhs = np.dot(O.conv1d(x, W, None, C_in, L, C_out, k, s, p, d).astype(np.float64), y.ravel())
    rhs = np.dot(x.ravel().astype(np.float64), O.conv1d_dgrad(W, y, C_in, L, C_out, k, s, p, d))
    assert abs(lhs - rhs) <= 1e-4 * max(abs(lhs), 1)
    W2 = rnd(C_out, C_in, k)
    dW, _ = O.conv1d_wgrad(x, y, C_in, L, C_out, k, s, p, d)
    lhs = np.dot(dW.astype(np.float64), W2.ravel())
    rhs = np.dot(y.ravel().astype(np.float64), O.conv1d(x, W2, None, C_in, L, C_out, k, s, p, d))
    assert abs(lhs - rhs) <= 1e-4 * max(abs(lhs), 1)
    # convT is the adjoint of the strided conv with the same weight tensor
    ci, co, Lx, kk, ss, pp = 4, 3, 12, 20, 10, 5
    Wt = rnd(ci, co, kk)
    xx = rnd(ci, Lx)
    Ly = O.convt1d_out_len(Lx, kk, ss, pp, 0, 1)
    yy = rnd(co, Ly)
    lhs = np.dot(O.convt1d(xx, Wt, None, ci, Lx, co, kk, ss, pp).astype(np.float64), yy.ravel())
    # conv1d of yy with weight viewed as (ci, co*k) is the strided correlation
    rhs = np.dot(xx.ravel().astype(np.float64),
                 O.conv1d(yy, Wt.reshape(ci, co * kk), None, co, Ly, ci, kk, ss, pp))
    assert abs(lhs - rhs) <= 1e-4 * max(abs(lhs), 1)


def test_conv1d_known_answer():
    # tests/test_modules.cpp:151-177: ones kernel over [1..5] -> [6, 9, 12]; bias adds
    x = np.array([1, 2, 3, 4, 5], np.float32)
    W = np.ones(3, np.float32)
    y = O.conv1d(x, W, np.zeros(1, np.float32), 1, 5, 1, 3)
    assert np.array_equal(y, np.array([6, 9, 12], np.float32))
    y = O.conv1d(x, W, np.array([100], np.float32), 1, 5, 1, 3)
    assert y[0] == 106.0


def test_adain_known_answer():
    # tests/test_modules.cpp:356-386: output channel mean == shift, biased var == scale^2
    x = np.array([1, 2, 3, 4, 7, 9, 11, 13], np.float32)
    scale = np.array([2.0, 3.0], np.float32)
    shift = np.array([0.5, -1.0], np.float32)
    y = O.adain_affine(x, scale - 1.0, shift, 2, 4).reshape(2, 4).astype(np.float64)
    assert np.allclose(y.mean(1), shift, atol=1e-6)
    assert np.allclose(y.var(1), scale ** 2, rtol=1e-4)


@pytest.mark.parametrize("C,L", [(3, 17), (5, 1000)])
def test_instnorm_and_adain_vs_torch(C, L):
    x = rnd(C, L, scale=2.0) + 0.7
    g = rnd(C, scale=0.5)
    b = rnd(C, scale=0.4)
    xt = t64(x)[None].requires_grad_(True)
    gt = t64(1.0 + g).requires_grad_(True)
    bt = t64(b).requires_grad_(True)
    yt = Fn.group_norm(xt, C, gt, bt, eps=1e-5)
    close(O.instnorm(x, 1.0 + g, b, C, L), yt.detach().numpy())
    close(O.adain_affine(x, g, b, C, L), yt.detach().numpy())
    dy = rnd(C, L)
    yt.backward(t64(dy)[None])
    dx, dg, db = O.instnorm_bwd(x, 1.0 + g, dy, C, L)
    close(dx, xt.grad.numpy(), rtol=1e-4)
    close(dg, gt.grad.numpy(), rtol=1e-4)
    close(db, bt.grad.numpy())
    # the AdaIN atom's dGamma is the grad w.r.t. gamma in (1 + gamma)
    dx2, dg2, db2 = O.adain_affine_bwd(x, g, dy, C, L)
    close(dx2, xt.grad.numpy(), rtol=1e-4)
    close(dg2, gt.grad.numpy(), rtol=1e-4)
    close(db2, bt.grad.numpy())


def test_snake_vs_autograd():
    C, L = 4, 257
    x = rnd(C, L, scale=2.0)
    a = rng.uniform(0.5, 2.0, C).astype(np.float32)
    xt = t64(x).requires_grad_(True)
    at = t64(a).requires_grad_(True)
    yt = xt + torch.sin(at[:, None] * xt) ** 2 / at[:, None]
    close(O.snake(x, a, C, L), yt.detach().numpy())
    dy = rnd(C, L)
    yt.backward(t64(dy))
    dx, da = O.snake_bwd(x, a, dy, C, L)
    close(dx, xt.grad.numpy())
    close(da, at.grad.numpy(), rtol=1e-5)


def test_leaky_and_pad():
    x = rnd(3, 10)
    close(O.leaky(x, 0.2), Fn.leaky_relu(t64(x), 0.2).numpy())
    dy = rnd(3, 10)
    close(O.leaky_bwd(x, dy, 0.1), np.where(x > 0, dy, 0.1 * dy))
    xt = t64(x)[None].requires_grad_(True)
    yt = Fn.pad(xt, (1, 0), mode="reflect")
    close(O.pad_reflect_left1(x, 3, 10), yt.detach().numpy())
    dy = rnd(3, 11)
    yt.backward(t64(dy)[None])
    close(O.pad_reflect_left1_bwd(dy, 3, 10), xt.grad.numpy())


def test_hann_periodic():
    for N in (8, 16, 20):
        w = O.hann(N)
        close(w, torch.hann_window(N, periodic=True, dtype=torch.float64).numpy(), atol=1e-7)
    # closed form: with hop = N/4 the squared periodic Hann overlap-adds to 1.5
    w = O.hann(20).astype(np.float64)
    env = sum(np.roll(np.pad(w ** 2, (0, 20)), 5 * i)[:40] for i in range(8))
    assert np.allclose(env[20:25], 1.5, atol=1e-6)


@pytest.mark.parametrize("n_fft,hop,frames", [(20, 5, 33), (8, 2, 17), (16, 4, 9)])
def test_istft_vs_torch(n_fft, hop, frames):
    F = n_fft // 2 + 1
    spec = rnd(frames, F, 2)
    win = O.hann(n_fft)
    sig = (frames - 1) * hop
    out = O.istft(spec, win, frames, sig, n_fft, hop)
    st = torch.complex(t64(spec[..., 0]), t64(spec[..., 1])).T.contiguous()
    st.requires_grad_(True)
    yt = torch.istft(st, n_fft, hop, n_fft, t64(win), center=True, normalized=False,
                     onesided=True, length=sig)
    close(out, yt.detach().numpy(), rtol=1e-5)
    dy = rnd(sig)
    yt.backward(t64(dy))
    g = st.grad.T.numpy()
    # torch's complex grad is conj-convention d/dre + i d/dim
    gtorch = np.stack([g.real, g.imag], -1).ravel()
    ds = O.istft_bwd(dy, win, frames, sig, n_fft, hop)
    # irfft ignores Im of DC / Nyquist; torch agrees that their grad is zero
    close(ds, gtorch, rtol=1e-5)


@pytest.mark.parametrize("n_fft,hop,length", [(20, 5, 600), (8, 2, 40)])
def test_stft_vs_torch_and_roundtrip(n_fft, hop, length):
    x = rnd(length)
    win = O.hann(n_fft)
    spec, frames = O.stft(x, win, n_fft, hop)
    st = torch.stft(t64(x), n_fft, hop, n_fft, t64(win), center=True, pad_mode="reflect",
                    normalized=False, onesided=True, return_complex=True)
    assert frames == st.shape[1] == length // hop + 1
    ref = np.stack([st.real.numpy().T, st.imag.numpy().T], -1).ravel()
    close(spec, ref, rtol=1e-5)
    # istft(stft(x)) == x (center=True recovers every sample)
    back = O.istft(spec, win, frames, (frames - 1) * hop, n_fft, hop)
    close(back, x[: (frames - 1) * hop], rtol=1e-5, atol=1e-5)


def test_istft_brute_force_dft():
    # one frame through irfft, checked against a direct complex DFT sum
    n_fft, hop = 8, 2
    F = n_fft // 2 + 1
    frames = 5
    spec = rnd(frames, F, 2)
    win = O.hann(n_fft).astype(np.float64)
    full = []
    for f in range(frames):
        X = spec[f, :, 0].astype(np.float64) + 1j * spec[f, :, 1]
        X[0] = X[0].real
        X[-1] = X[-1].real
        Xf = np.concatenate([X, np.conj(X[1:-1][::-1])])
        n = np.arange(n_fft)
        full.append(np.real(np.exp(2j * np.pi * np.outer(n, n) / n_fft) @ Xf) / n_fft)
    total = n_fft + hop * (frames - 1)
    ola, env = np.zeros(total), np.zeros(total)
    for f in range(frames):
        ola[f * hop:f * hop + n_fft] += full[f] * win
        env[f * hop:f * hop + n_fft] += win ** 2
    sig = (frames - 1) * hop
    ref = (ola / np.where(env > 1e-11, env, 1))[n_fft // 2:n_fft // 2 + sig]
    close(O.istft(spec, O.hann(n_fft), frames, sig, n_fft, hop), ref, rtol=1e-5)


def _lora_case(rows=10, rank=4, S=16):
    W, b = rnd(rows, S, scale=0.3), rnd(rows, scale=0.2)
    A, B = rnd(rank, S, scale=0.3), rnd(rows, rank, scale=0.3)
    g, s = rnd(rank), rnd(S)
    return W, b, A, B, g, s


def test_lora_closed_forms():
    # the adapter contract (decoder_lora.h:63-77): a zero gate or a zero B
    # leaves the frozen projection exactly; otherwise y = W s + b + scale B (g * A s)
    W, b, A, B, g, s = _lora_case()
    base = (W.astype(np.float64) @ s + b)
    y0, _ = O.lora_fwd(W, b, A, B, np.zeros_like(g), 0.7, s)
    close(y0, base, rtol=1e-6, atol=1e-6)
    y1, _ = O.lora_fwd(W, b, A, np.zeros_like(B), g, 0.7, s)
    close(y1, base, rtol=1e-6, atol=1e-6)
    # the LoRA term is linear in scale
    ya, _ = O.lora_fwd(W, b, A, B, g, 0.5, s)
    yb, _ = O.lora_fwd(W, b, A, B, g, 1.5, s)
    close(yb - base, 3.0 * (ya - base), rtol=1e-5, atol=1e-5)


def test_lora_adjoint_identities():
    # y is linear in each of B, A, g and s with the others fixed, so for any
    # direction D: <dy, y(X + D) - y(X)> = <dX, D> (up to float rounding).
    W, b, A, B, g, s = _lora_case()
    scale = 0.8
    y, h = O.lora_fwd(W, b, A, B, g, scale, s)
    dy = rnd(W.shape[0])
    gr = O.lora_bwd(W, A, B, g, scale, s, h, dy)

    def inner(y2):
        return float(np.dot(dy.astype(np.float64), y2.astype(np.float64) - y.astype(np.float64)))

    for name, args_fn, D in (
        ("B", lambda D: (W, b, A, B + D, g, scale, s), rnd(*B.shape)),
        ("A", lambda D: (W, b, A + D, B, g, scale, s), rnd(*A.shape)),
        ("G", lambda D: (W, b, A, B, g + D, scale, s), rnd(*g.shape)),
        ("style", lambda D: (W, b, A, B, g, scale, s + D), rnd(*s.shape)),
        ("W", lambda D: (W + D, b, A, B, g, scale, s), rnd(*W.shape)),
        ("b", lambda D: (W, b + D, A, B, g, scale, s), rnd(*b.shape)),
    ):
        lhs = inner(O.lora_fwd(*args_fn(D))[0])
        rhs = float(np.sum(gr["d" + name].astype(np.float64) * D))
        assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(rhs)), (name, lhs, rhs)
