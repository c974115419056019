"""The decoder back half as a torch float64 module graph with autograd.

Test infrastructure: a second, independent restatement used to pin the
oracle's composed forward and its hand-written backward. The oracle follows
the reference's `_train` assemblies op by op (kokoro_decoder_backward.cpp)
and differentiates by hand. This file instead composes torch's own conv1d /
conv_transpose1d / instance norm / istft in the module order of the upstream
Kokoro iSTFTNet decoder, which the reference's inference forwards mirror:

* AdaIN1d: y = (1 + gamma) * instance_norm(x) + beta, (gamma, beta) =
  chunk(fc(style)) (kokoro_modules.cpp:596-620, eps 1e-5).
* AdainResBlk1d: norm1 -> leaky 0.2 -> [depthwise convT pool k3 s2 p1 op1]
  -> conv1 -> norm2 -> leaky 0.2 -> conv2, shortcut [nearest 2x] -> [1x1],
  (residual + shortcut) / sqrt(2) (kokoro_modules.cpp:651-706).
* DecoderBackbone: F0 / N convs (k3 s2), cat [asr, F0, N] -> encode,
  asr_res 1x1, decode blocks with [x, asr_res, F0, N] cat'd while no
  upsampling block has run (kokoro_modules.cpp:1087-1141).
* AdaINResBlock1: for i in 0..2: adain1 -> Snake -> convs1[i] (dilated) ->
  adain2 -> Snake -> convs2[i] -> + x (kokoro_modules.cpp:1197-1231).
* Generator: per stage leaky 0.1 -> noise_convs(har) -> noise_res; ups
  convT (+ left reflect pad by 1 on the last stage) + source; mean of the K
  resblocks; then leaky 0.01 -> conv_post -> exp / sin -> istft (n_fft, hop,
  periodic Hann, center) (kokoro_modules.cpp:1400-1552).

The harmonic source is an input here (har), as in the model parity tests.
The backward is torch autograd of sum(audio * dL/daudio): every parameter
grad, the per-unit (dgamma, dbeta) and d(style).
"""
from __future__ import annotations

import math

import numpy as np
import torch

F = torch.nn.functional
PFX = "decoder.module."


class Ref:
    def __init__(self, cfg: dict, params: dict):
        self.cfg = cfg
        self.p = {k: torch.tensor(np.asarray(v, np.float64)).requires_grad_(True) for k, v in params.items()}
        self.units = []  # (name, C) in the order the forward visits them
        self.affine = {}  # unit name -> the (2C,) fc output, kept for its grad

    # ─── building blocks ───
    def W(self, name, *shape):
        return self.p[PFX + name].reshape(*shape)

    def b(self, name):
        t = self.p.get(PFX + name)
        return None if t is None else t.reshape(-1)

    def conv(self, name, x, k, stride=1, pad=0, dil=1):
        w = self.p[PFX + name + ".weight"]
        co = w.shape[0]
        return F.conv1d(x, w.reshape(co, -1, k), self.b(name + ".bias"), stride=stride, padding=pad,
                        dilation=dil)

    def adain(self, name, x, s):
        C = x.shape[1]
        h = F.linear(s, self.p[PFX + name + ".fc.weight"], self.b(name + ".fc.bias"))  # (N, 2C)
        h.retain_grad()
        self.affine[PFX + name] = h
        self.units.append((PFX + name, C))
        gamma, beta = h[:, :C, None], h[:, C:, None]
        return (1.0 + gamma) * F.instance_norm(x, eps=1e-5) + beta

    @staticmethod
    def snake(x, a):
        a = a.reshape(1, -1, 1)
        return x + torch.sin(a * x) ** 2 / a

    def resblk(self, name, x, s, upsample):
        c_in = x.shape[1]
        r = F.leaky_relu(self.adain(name + ".norm1", x, s), 0.2)
        if upsample:
            r = F.conv_transpose1d(r, self.W(name + ".pool.weight", c_in, 1, 3), self.b(name + ".pool.bias"),
                                   stride=2, padding=1, output_padding=1, groups=c_in)
        r = self.conv(name + ".conv1", r, 3, pad=1)
        r = F.leaky_relu(self.adain(name + ".norm2", r, s), 0.2)
        r = self.conv(name + ".conv2", r, 3, pad=1)
        sc = F.interpolate(x, scale_factor=2, mode="nearest") if upsample else x
        if PFX + name + ".conv1x1.weight" in self.p:
            sc = self.conv(name + ".conv1x1", sc, 1)
        return (r + sc) / math.sqrt(2.0)

    def resblock1(self, name, x, s, k, dils):
        for i in range(3):
            xt = self.snake(self.adain(f"{name}.adain1.{i}", x, s), self.p[PFX + f"{name}.alpha1.{i}"])
            xt = self.conv(f"{name}.convs1.{i}", xt, k, pad=dils[i] * (k - 1) // 2, dil=dils[i])
            xt = self.snake(self.adain(f"{name}.adain2.{i}", xt, s), self.p[PFX + f"{name}.alpha2.{i}"])
            xt = self.conv(f"{name}.convs2.{i}", xt, k, pad=(k - 1) // 2)
            x = xt + x
        return x

    # ─── decoder ───
    def backbone(self, asr, F0, Nn, s):
        c = self.cfg
        f0 = self.conv("F0_conv", F0[:, None, :], 3, stride=2, pad=1)
        nn_ = self.conv("N_conv", Nn[:, None, :], 3, stride=2, pad=1)
        x = self.resblk("encode", torch.cat([asr, f0, nn_], dim=1), s, False)
        asr_res = self.conv("asr_res.0", asr, 1)
        res = True
        for i in range(c["n_decode"]):
            if res:
                x = torch.cat([x, asr_res, f0, nn_], dim=1)
            up = i == c["dec_up_at"]
            x = self.resblk(f"decode.{i}", x, s, up)
            if up:
                res = False
        return x

    def generator(self, x, har, s):
        c = self.cfg
        U, K = c["n_ups"], c["n_kernels"]
        for i in range(U):
            x = F.leaky_relu(x, 0.1)
            stride_f0 = int(np.prod(c["ups_rates"][i + 1:U])) if i + 1 < U else 1
            if i + 1 < U:
                src = self.conv(f"generator.noise_convs.{i}", har, 2 * stride_f0, stride=stride_f0,
                                pad=(stride_f0 + 1) // 2)
            else:
                src = self.conv(f"generator.noise_convs.{i}", har, 1)
            src = self.resblock1(f"generator.noise_res.{i}", src, s, 7 if i + 1 < U else 11, [1, 3, 5])
            u, k = c["ups_rates"][i], c["ups_kernels"][i]
            w = self.p[PFX + f"generator.ups.{i}.weight"]
            x = F.conv_transpose1d(x, w.reshape(w.shape[0], -1, k), self.b(f"generator.ups.{i}.bias"), stride=u,
                                   padding=(k - u) // 2)
            if i == U - 1:
                x = F.pad(x, (1, 0), mode="reflect")
            x = x + src
            xs = None
            for j in range(K):
                r = self.resblock1(f"generator.resblocks.{i * K + j}", x, s, c["rb_kernels"][j], c["rb_dil"][j])
                xs = r if xs is None else xs + r
            x = xs / K
        x = F.leaky_relu(x, 0.01)
        post = self.conv("generator.conv_post", x, c["conv_post_k"], pad=(c["conv_post_k"] - 1) // 2)
        nf, hop = c["n_fft"], c["hop"]
        Fq = nf // 2 + 1
        spec = torch.exp(post[:, :Fq]) * torch.exp(1j * torch.sin(post[:, Fq:]))
        win = torch.hann_window(nf, periodic=True, dtype=torch.float64)
        return torch.istft(spec, nf, hop, nf, window=win, center=True)

    def run(self, asr, F0, Nn, style, har, daudio):
        """Forward + backward for N utterances (numpy in); returns audio,
        d(style), grads {name: array} and affine grads {unit: (dgamma, dbeta)}."""
        t = lambda a: torch.tensor(np.asarray(a, np.float64))
        s = t(style).requires_grad_(True)
        self.units, self.affine = [], {}
        gen_in = self.backbone(t(asr), t(F0), t(Nn), s)
        audio = self.generator(gen_in, t(har).reshape(len(asr), self.cfg["n_fft"] + 2, -1), s)
        (audio * t(daudio)).sum().backward()
        grads = {k: (v.grad.numpy().ravel() if v.grad is not None else np.zeros(v.numel())) for k, v in self.p.items()}
        aff = {}
        for name, C in self.units:
            g = self.affine[name].grad.numpy()
            aff[name] = (g[:, :C], g[:, C:])
        return audio.detach().numpy(), s.grad.numpy(), grads, aff
