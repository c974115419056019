"""CPU restatement, in numpy float64, of DecoderLora's parts that sit beside
the decoder: the conditioning gate, the Adam step and the ELRA1 checkpoint
format. Test infrastructure only: tests and the benchmark's CPU leg use it
as the checker; the product never imports it.

Follows the reference's include/brosoundml/decoder_lora.h:20-53 and
src/decoder_lora.cpp:30-80 (gate), :298-314 (Adam via bt::adam_step) and
:316-396 (checkpoint I/O). The adapters themselves (the LoRA style
projection) and the decoder live in the C++ oracle (oracle/kdec_model.cpp).

Pinning: the gate by its structural zero (g(0) = 0 for any weights, the
reference's test_decoder_lora.cpp:57-70), finite differences
(test_decoder_lora.cpp:72-100) and torch autograd; Adam by torch.optim.Adam
(bt::adam_step's source is not in the reference tree, so its exact rounding
is parity unpinned); ELRA1 by its byte layout and round trips.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = b"ELRA1\x00\x00\x00"


def gate_forward(W1, W2, v):
    """g = W2 tanh(W1 v) per condition row (ConditioningGate::forward,
    decoder_lora.cpp:56-66, no biases). v (N, in_dim) -> g (N, gate_dim),
    act (N, hidden)."""
    v = np.atleast_2d(np.asarray(v, np.float64))
    act = np.tanh(v @ np.asarray(W1, np.float64).T)
    return act @ np.asarray(W2, np.float64).T, act


def gate_backward(W2, v, act, dG):
    """(dW1, dW2) for the upstream dG (N, gate_dim) (ConditioningGate::backward,
    decoder_lora.cpp:68-80; the condition is not trainable: no dv)."""
    v = np.atleast_2d(np.asarray(v, np.float64))
    dG = np.atleast_2d(np.asarray(dG, np.float64))
    dW2 = dG.T @ act
    dpre = (dG @ np.asarray(W2, np.float64)) * (1.0 - act * act)
    return dpre.T @ v, dW2


def adam_step(p, g, m, v, lr, beta1, beta2, eps, step):
    """One Adam step with bias correction (DecoderLora::adam_step,
    decoder_lora.cpp:305-314, through bt::adam_step): returns (p, m, v)."""
    m = beta1 * m + (1.0 - beta1) * g
    v = beta2 * v + (1.0 - beta2) * g * g
    mh = m / (1.0 - beta1 ** step)
    vh = v / (1.0 - beta2 ** step)
    return p - lr * mh / (np.sqrt(vh) + eps), m, v


def _tensor(a):
    a = np.asarray(a, np.float32)
    return struct.pack("<ii", a.shape[0], a.shape[1]) + a.tobytes()


def elra1_bytes(rank, style_dim, scale, gate_hidden, W1, W2, adapters):
    """The checkpoint DecoderLora::save writes (decoder_lora.cpp:352-372):
    magic, int32 rank, int32 style_dim, float scale, int32 gate hidden, gate
    W1, W2, then per adapter int32 C, A (rank, style_dim), B (2C, rank); a
    tensor is int32 rows, int32 cols and its floats, little-endian.
    `adapters` is a list of (C, A, B)."""
    out = [MAGIC, struct.pack("<iifi", rank, style_dim, scale, gate_hidden), _tensor(W1), _tensor(W2)]
    for C, A, B in adapters:
        out += [struct.pack("<i", C), _tensor(A), _tensor(B)]
    return b"".join(out)


def elra1_parse(data: bytes):
    """Inverse of elra1_bytes (DecoderLora::load, decoder_lora.cpp:374-396)."""
    if data[:8] != MAGIC:
        raise ValueError("bad magic")
    rank, sd, scale, gh = struct.unpack_from("<iifi", data, 8)
    off = 24

    def tensor():
        nonlocal off
        r, c = struct.unpack_from("<ii", data, off)
        off += 8
        a = np.frombuffer(data, np.float32, r * c, off).reshape(r, c).copy()
        off += 4 * r * c
        return a

    W1, W2 = tensor(), tensor()
    ads = []
    while off < len(data):
        (C,) = struct.unpack_from("<i", data, off)
        off += 4
        A = tensor()
        B = tensor()
        ads.append((C, A, B))
    return dict(rank=rank, style_dim=sd, scale=scale, gate_hidden=gh, W1=W1, W2=W2, adapters=ads)
