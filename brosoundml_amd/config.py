"""Decoder configurations.

``KOKORO`` is the Kokoro-82M decoder (config.json values from the reference's
tests/test_kokoro.cpp:44-63 plus the channel plan hard-coded in
DecoderBackbone::load_from, kokoro_modules.cpp:1052-1062). The miniatures keep
every structural feature (cat'd decode blocks, the 2x-upsampling block, two
upsample stages, K resblocks, the final reflect pad, the spectral head and the
harmonic source) at sizes a CPU finishes in well under a second.
"""
from __future__ import annotations

import copy

KOKORO = dict(
    asr_dim=512, asr_res_dim=64, style_dim=128, enc_dim=1024,
    n_decode=4, dec_out=[1024, 1024, 1024, 512], dec_up_at=3,
    n_ups=2, ups_rates=[10, 6], ups_kernels=[20, 12],
    n_kernels=3, rb_kernels=[3, 7, 11], rb_dil=[[1, 3, 5]] * 3,
    n_fft=20, hop=5, conv_post_k=7, sample_rate=24000, harmonic_num=8,
)

# Small but structurally complete: backbone 12 -> (16, 16 up 12) and a
# generator 12 -> 6 -> 3 with upsample rates (2, 3).
TINY = dict(
    asr_dim=12, asr_res_dim=4, style_dim=16, enc_dim=16,
    n_decode=2, dec_out=[16, 12], dec_up_at=1,
    n_ups=2, ups_rates=[2, 3], ups_kernels=[4, 5],
    n_kernels=2, rb_kernels=[3, 5], rb_dil=[[1, 2, 3], [1, 3, 5]],
    n_fft=8, hop=2, conv_post_k=7, sample_rate=24000, harmonic_num=8,
)

# Kokoro's channel plan scaled down 8x (C=64/32/16 in the generator), with the
# real upsample rates / kernels, n_fft 20, hop 5 and the resblock kernels.
SMALL = dict(
    asr_dim=64, asr_res_dim=8, style_dim=128, enc_dim=128,
    n_decode=4, dec_out=[128, 128, 128, 64], dec_up_at=3,
    n_ups=2, ups_rates=[10, 6], ups_kernels=[20, 12],
    n_kernels=3, rb_kernels=[3, 7, 11], rb_dil=[[1, 3, 5]] * 3,
    n_fft=20, hop=5, conv_post_k=7, sample_rate=24000, harmonic_num=8,
)


def normalize(cfg: dict) -> dict:
    c = copy.deepcopy(cfg)
    c["dec_out"] = list(c["dec_out"]) + [0] * (8 - len(c["dec_out"]))
    c["ups_rates"] = list(c["ups_rates"]) + [0] * (4 - len(c["ups_rates"]))
    c["ups_kernels"] = list(c["ups_kernels"]) + [0] * (4 - len(c["ups_kernels"]))
    c["rb_kernels"] = list(c["rb_kernels"]) + [0] * (4 - len(c["rb_kernels"]))
    c["rb_dil"] = [list(r) for r in c["rb_dil"]] + [[0, 0, 0]] * (4 - len(c["rb_dil"]))
    return c


def flat_ints(cfg: dict) -> list[int]:
    """The config as the flat int list both C ABIs take, in this order:
    asr_dim, asr_res_dim, style_dim, enc_dim, n_decode, dec_out[8], dec_up_at,
    n_ups, ups_rates[4], ups_kernels[4], n_kernels, rb_kernels[4],
    rb_dil[4][3], n_fft, hop, conv_post_k, sample_rate, harmonic_num."""
    c = normalize(cfg)
    v = [c["asr_dim"], c["asr_res_dim"], c["style_dim"], c["enc_dim"], c["n_decode"]]
    v += c["dec_out"] + [c["dec_up_at"], c["n_ups"]] + c["ups_rates"] + c["ups_kernels"]
    v += [c["n_kernels"]] + c["rb_kernels"]
    for r in c["rb_dil"]:
        v += r
    v += [c["n_fft"], c["hop"], c["conv_post_k"], c["sample_rate"], c["harmonic_num"]]
    return [int(x) for x in v]


def upsample_prod(cfg: dict) -> int:
    p = 1
    for r in cfg["ups_rates"][: cfg["n_ups"]]:
        p *= r
    return p


def lengths(cfg: dict, T: int) -> dict:
    """Per-utterance lengths for T asr frames (kokoro.cpp:365-373)."""
    L_gen = 2 * T
    frames = L_gen * upsample_prod(cfg) + 1
    audio = (frames - 1) * cfg["hop"]
    return dict(L_gen=L_gen, frames=frames, audio=audio,
                audio_seconds=audio / cfg["sample_rate"])


def affine_rows(cfg: dict) -> int:
    """Rows of the stacked AdaIN style projection, sum over units of 2C:
    the encode block's norms on C_in = asr_dim + 2 and enc_dim, each decode
    block's on its input (the previous output cat'd with asr_res, F0 and N
    up to and including the upsampling block) and output, and six units per
    generator ResBlock1 (the noise_res block and K resblocks of each stage,
    C = the last decode block's output / 2^(i+1) at stage i)."""
    C = [cfg["asr_dim"] + 2, cfg["enc_dim"]]
    prev, res = cfg["enc_dim"], True
    for i in range(cfg["n_decode"]):
        cin = prev + (cfg["asr_res_dim"] + 2 if res else 0)
        C += [cin, cfg["dec_out"][i]]
        prev = cfg["dec_out"][i]
        if i == cfg["dec_up_at"]:
            res = False
    for i in range(cfg["n_ups"]):
        c = cfg["dec_out"][cfg["n_decode"] - 1] // (2 ** (i + 1))
        C += [c] * 6 * (1 + cfg["n_kernels"])
    return 2 * sum(C)
