"""Writes the golden vectors under tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

Every expected output comes from PyTorch's CPU implementation of the same op
in float64 (torch is a third-party library, independent of the reference and
of this repository's oracle), on small seeded float32 inputs that are stored
beside the outputs. Backward values are torch autograd gradients for the
stored upstream gradient. The files are data only (numpy .npz, no pickles);
tests load them with numpy.load(allow_pickle=False).

Ops and the reference call sites whose semantics they fix:
  conv.npz      Conv1d forward / input / weight / bias grads
                (kokoro_decoder_backward.cpp:152-285, 287-376, 378-458)
  convt.npz     ConvTranspose1d (upsamplers, depthwise pool) forward and grads
                (kokoro_decoder_backward.cpp:252-256, 592-737)
  adain.npz     AdaIN1d ((1 + gamma) * instance_norm(x) + beta, eps 1e-5)
                followed by none / leaky ReLU / Snake, forward and grads
                (kokoro_decoder_backward.cpp:100-150, 287-376)
  spectral.npz  spectral head: exp / sin polar form -> iSTFT (n_fft 20, hop 5,
                periodic Hann, center) and its adjoint
                (kokoro_decoder_backward.cpp:378-458)
  stft.npz      HarmonicSource's STFT magnitude / phase
                (kokoro_modules.cpp:1640-1650)
"""
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
rng = np.random.default_rng(0x60_1DE7)


def f32(*shape, scale=1.0, lo=None, hi=None):
    if lo is not None:
        return rng.uniform(lo, hi, shape).astype(np.float32)
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def t(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=grad)


def conv_cases():
    geo = [  # N, C_in, C_out, L, k, s, p, d
        (2, 5, 6, 37, 3, 1, 1, 1),
        (2, 4, 3, 50, 7, 1, 9, 3),
        (2, 3, 4, 61, 11, 1, 25, 5),
        (2, 2, 5, 41, 12, 6, 3, 1),
        (2, 6, 5, 20, 1, 1, 0, 1),
        (1, 1, 1, 16, 3, 2, 1, 1),
    ]
    out = {}
    for i, (N, Ci, Co, L, k, s, p, d) in enumerate(geo):
        x = f32(N, Ci, L)
        W = f32(Co, Ci * k, scale=0.3)
        b = f32(Co, scale=0.2)
        xt, Wt, bt = t(x, True), t(W.reshape(Co, Ci, k), True), t(b, True)
        y = F.conv1d(xt, Wt, bt, stride=s, padding=p, dilation=d)
        dy = f32(*y.shape)
        y.backward(t(dy))
        pre = f"c{i}_"
        out.update({pre + "geo": np.array([N, Ci, Co, L, k, s, p, d], np.int64), pre + "x": x, pre + "W": W,
                    pre + "b": b, pre + "dy": dy, pre + "y": y.detach().numpy(), pre + "dx": xt.grad.numpy(),
                    pre + "dW": Wt.grad.numpy().reshape(Co, Ci * k), pre + "db": bt.grad.numpy()})
    return out


def convt_cases():
    geo = [  # N, C_in, C_out, L, k, s, p, op, groups
        (2, 6, 4, 12, 20, 10, 5, 0, 1),
        (2, 4, 3, 15, 12, 6, 3, 0, 1),
        (1, 3, 3, 11, 3, 1, 1, 0, 1),
        (2, 5, 5, 13, 3, 2, 1, 1, 5),   # the depthwise 2x pool of the upsampling block
    ]
    out = {}
    for i, (N, Ci, Co, L, k, s, p, op, grp) in enumerate(geo):
        x = f32(N, Ci, L)
        W = f32(Ci, (Co // grp) * k, scale=0.3)
        b = f32(Co, scale=0.2)
        xt, Wt, bt = t(x, True), t(W.reshape(Ci, Co // grp, k), True), t(b, True)
        y = F.conv_transpose1d(xt, Wt, bt, stride=s, padding=p, output_padding=op, groups=grp)
        dy = f32(*y.shape)
        y.backward(t(dy))
        pre = f"t{i}_"
        out.update({pre + "geo": np.array([N, Ci, Co, L, k, s, p, op, grp], np.int64), pre + "x": x,
                    pre + "W": W, pre + "b": b, pre + "dy": dy, pre + "y": y.detach().numpy(),
                    pre + "dx": xt.grad.numpy(), pre + "dW": Wt.grad.numpy().reshape(Ci, (Co // grp) * k),
                    pre + "db": bt.grad.numpy()})
    return out


def adain_cases():
    N, C, L, eps = 2, 4, 300, 1e-5
    out = {"shape": np.array([N, C, L], np.int64), "eps": np.array(eps), "slope": np.array(0.2)}
    x = f32(N, C, L, scale=1.5) + 0.3
    gamma = f32(N, C, scale=0.3)
    beta = f32(N, C, scale=0.3)
    alpha = f32(C, lo=0.5, hi=2.0)
    out.update(x=x, gamma=gamma, beta=beta, alpha=alpha)
    for act in ("none", "leaky", "snake"):
        xt, gt, bt, at = t(x, True), t(gamma, True), t(beta, True), t(alpha, True)
        m = xt.mean(-1, keepdim=True)
        v = ((xt - m) ** 2).mean(-1, keepdim=True)
        s = (1.0 + gt[..., None]) * (xt - m) / torch.sqrt(v + eps) + bt[..., None]
        if act == "none":
            y = s
        elif act == "leaky":
            y = F.leaky_relu(s, 0.2)
        else:
            a = at[None, :, None]
            y = s + torch.sin(a * s) ** 2 / a
        dy = f32(N, C, L)
        y.backward(t(dy))
        out.update({f"{act}_dy": dy, f"{act}_y": y.detach().numpy(), f"{act}_dx": xt.grad.numpy(),
                    f"{act}_dgamma": gt.grad.numpy(), f"{act}_dbeta": bt.grad.numpy()})
        if act == "snake":
            out["snake_dalpha"] = at.grad.numpy()
    return out


def spectral_cases():
    # leaky_relu(0.01) -> conv_post (k 7, same padding) -> exp / sin polar -> iSTFT
    N, C, n_fft, hop, L, k = 2, 6, 20, 5, 21, 7
    Fq = n_fft // 2 + 1
    x = f32(N, C, L, scale=0.8)
    W = f32(2 * Fq, C * k, scale=0.3 / np.sqrt(C * k))
    b = f32(2 * Fq, scale=0.1)
    win = torch.hann_window(n_fft, periodic=True, dtype=torch.float64)
    xt, Wt, bt = t(x, True), t(W.reshape(2 * Fq, C, k), True), t(b, True)
    post = F.conv1d(F.leaky_relu(xt, 0.01), Wt, bt, padding=(k - 1) // 2)
    mag = torch.exp(post[:, :Fq])
    ph = torch.sin(post[:, Fq:])
    spec = torch.complex(mag * torch.cos(ph), mag * torch.sin(ph))
    S = (L - 1) * hop
    audio = torch.istft(spec, n_fft, hop, n_fft, win, center=True, normalized=False, onesided=True, length=S)
    da = f32(N, S)
    audio.backward(t(da))
    return {"shape": np.array([N, C, n_fft, hop, L, k], np.int64), "x": x, "W": W, "b": b, "daudio": da,
            "audio": audio.detach().numpy(), "dx": xt.grad.numpy(), "dW": Wt.grad.numpy().reshape(2 * Fq, C * k),
            "db": bt.grad.numpy()}


def stft_cases():
    n_fft, hop, length = 20, 5, 600
    x = f32(length)
    win = torch.hann_window(n_fft, periodic=True, dtype=torch.float64)
    st = torch.stft(t(x), n_fft, hop, n_fft, win, center=True, pad_mode="reflect", normalized=False,
                    onesided=True, return_complex=True)
    return {"shape": np.array([n_fft, hop, length], np.int64), "x": x,
            "re": st.real.numpy().T.copy(), "im": st.imag.numpy().T.copy(),
            "mag": st.abs().numpy().T.copy(), "phase": torch.angle(st).numpy().T.copy()}


def main():
    torch.manual_seed(0)
    for name, fn in (("conv", conv_cases), ("convt", convt_cases), ("adain", adain_cases),
                     ("spectral", spectral_cases), ("stft", stft_cases)):
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
