"""Deterministic synthetic inputs and random-init weights.

A fixed in-repo generator keeps fixtures portable across platforms and
libraries: SplitMix64 counter streams give uniforms, Box-Muller turns pairs of
uniforms into normals, and every tensor draws from its own named sub-seed so
adding a tensor never shifts another's values.

Weight init follows PyTorch's default Kaiming-uniform (a = sqrt(5)), i.e.
U(-1/sqrt(fan_in), 1/sqrt(fan_in)) for conv / transposed-conv / linear weights
and biases; Snake alphas are U(0.5, 2).
"""
from __future__ import annotations

import math

import numpy as np

BASE_SEED = 0x4B4F4B4F
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def sub_seed(name: str, base: int = BASE_SEED) -> int:
    z = np.array([(base ^ _fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    return int(_mix(z)[0])


def uniform01(seed: int, n: int) -> np.ndarray:
    """n doubles in [0, 1) from the SplitMix64 stream of `seed`."""
    i = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GOLDEN
    return (_mix(z) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def uniform(name: str, shape, lo: float, hi: float, base: int = BASE_SEED) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    u = uniform01(sub_seed(name, base), n)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(name: str, shape, std: float = 1.0, mean: float = 0.0, base: int = BASE_SEED) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    m = (n + 1) // 2
    u = uniform01(sub_seed(name, base), 2 * m)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log1p(-u1))
    th = 2.0 * math.pi * u2
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def init_params(shapes, base: int = BASE_SEED) -> dict:
    """Random init for every named decoder parameter.

    ``shapes`` maps name -> (rows, cols). fan_in follows PyTorch and equals
    the weight's second dimension in every layout used here: Conv1d weight
    (C_out, C_in*k) -> C_in*k; ConvTranspose1d weight (C_in, C_out*k) ->
    C_out*k (torch reads dim 1); the depthwise pool (C_in, 1*3) -> 3; Linear
    (out, in) -> in. A bias shares its weight's fan_in.
    """
    out = {}
    for name, (rows, cols) in shapes.items():
        if ".alpha" in name:
            out[name] = uniform(name, (rows, cols), 0.5, 2.0, base)
            continue
        wname = name[: -len(".bias")] + ".weight" if name.endswith(".bias") else name
        fan_in = shapes[wname][1] if wname in shapes else cols
        bound = 1.0 / math.sqrt(max(fan_in, 1))
        out[name] = uniform(name, (rows, cols), -bound, bound, base)
    return out


def decoder_inputs(cfg: dict, N: int, T: int, tag: str, unvoiced: float = 0.0):
    """Synthetic decoder inputs for N utterances of T asr frames, each tensor
    from its own named sub-seed: asr ~ N(0, 1) (N, asr_dim, T), F0 ~ U(80, 300)
    Hz (N, 2T) with a fraction `unvoiced` of frames set to 0, the N curve ~
    N(0, 0.5) (N, 2T), style ~ N(0, 0.3) (N, style_dim) and dL/dwav ~ N(0, 1)
    (N, audio_len)."""
    from .config import lengths
    asr = normal(f"{tag}.asr", (N, cfg["asr_dim"], T))
    F0 = uniform(f"{tag}.F0", (N, 2 * T), 80.0, 300.0)
    if unvoiced > 0.0:
        F0[uniform(f"{tag}.uv", (N, 2 * T), 0.0, 1.0) < unvoiced] = 0.0
    Nn = normal(f"{tag}.N", (N, 2 * T), 0.5)
    style = normal(f"{tag}.style", (N, cfg["style_dim"]), 0.3)
    dA = normal(f"{tag}.daudio", (N, lengths(cfg, T)["audio"]), 1.0)
    return asr, F0, Nn, style, dA
