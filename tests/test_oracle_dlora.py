"""Pins the CPU restatement of DecoderLora's gate, Adam step and ELRA1
checkpoint (oracle/decoder_lora.py): the gate's structural zero and finite
differences (the reference's test_decoder_lora.cpp:52-100), torch autograd
for the gate, torch.optim.Adam for the optimiser step, and the checkpoint
byte layout."""
import os
import struct
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import decoder_lora as DL  # noqa: E402

torch = pytest.importorskip("torch")


def rng(seed):
    return np.random.default_rng(seed)


def test_gate_structural_zero():
    # g(0) = 0 exactly for a zero W2 and for random weights alike
    r = rng(20260606)
    W1 = r.uniform(-0.7, 0.7, (16, 3))
    W2 = np.zeros((4, 16))
    g, _ = DL.gate_forward(W1, W2, np.zeros(3))
    assert np.all(g == 0.0)
    W2 = r.uniform(-0.7, 0.7, (4, 16))
    g, _ = DL.gate_forward(W1, W2, np.zeros((2, 3)))
    assert np.all(g == 0.0)
    # W2 = 0 closes the gate for any condition
    g, _ = DL.gate_forward(W1, np.zeros((4, 16)), r.normal(size=(5, 3)))
    assert np.all(g == 0.0)


def test_gate_backward_finite_differences():
    # the reference's check: loss = 0.5 |g(v) - target|^2, central differences
    r = rng(7)
    W1 = r.uniform(-0.7, 0.7, (16, 3))
    W2 = r.uniform(-0.7, 0.7, (4, 16))
    v = np.array([[0.2, -0.5, 0.7]])
    target = r.uniform(-0.5, 0.5, (1, 4))

    def loss(W1_, W2_):
        g, _ = DL.gate_forward(W1_, W2_, v)
        return 0.5 * np.sum((g - target) ** 2)

    g, act = DL.gate_forward(W1, W2, v)
    dW1, dW2 = DL.gate_backward(W2, v, act, g - target)
    h = 1e-6
    for P, D, which in ((W1, dW1, 0), (W2, dW2, 1)):
        fd = np.zeros_like(P)
        for i in np.ndindex(P.shape):
            Pp, Pm = P.copy(), P.copy()
            Pp[i] += h
            Pm[i] -= h
            lp = loss(Pp, W2) if which == 0 else loss(W1, Pp)
            lm = loss(Pm, W2) if which == 0 else loss(W1, Pm)
            fd[i] = (lp - lm) / (2 * h)
        np.testing.assert_allclose(D, fd, rtol=1e-6, atol=1e-9)


def test_gate_against_torch_autograd():
    r = rng(11)
    W1 = r.normal(size=(16, 3))
    W2 = r.normal(size=(5, 16))
    v = r.normal(size=(3, 3))
    dG = r.normal(size=(3, 5))
    tW1 = torch.tensor(W1, requires_grad=True)
    tW2 = torch.tensor(W2, requires_grad=True)
    tg = torch.tanh(torch.tensor(v) @ tW1.T) @ tW2.T
    tg.backward(torch.tensor(dG))
    g, act = DL.gate_forward(W1, W2, v)
    dW1, dW2 = DL.gate_backward(W2, v, act, dG)
    np.testing.assert_allclose(g, tg.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dW1, tW1.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dW2, tW2.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_adam_against_torch():
    r = rng(3)
    p0 = r.normal(size=(6, 7))
    grads = [r.normal(size=p0.shape) for _ in range(5)]
    tp = torch.tensor(p0.copy(), requires_grad=True)
    opt = torch.optim.Adam([tp], lr=3e-3, betas=(0.9, 0.999), eps=1e-8)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step, g in enumerate(grads, 1):
        opt.zero_grad()
        tp.grad = torch.tensor(g)
        opt.step()
        p, m, v = DL.adam_step(p, g, m, v, 3e-3, 0.9, 0.999, 1e-8, step)
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-12, atol=1e-13)


def test_elra1_layout_and_round_trip(tmp_path):
    r = rng(5)
    W1 = r.normal(size=(16, 3)).astype(np.float32)
    W2 = r.normal(size=(4, 16)).astype(np.float32)
    ads = [(C, r.normal(size=(4, 8)).astype(np.float32), r.normal(size=(2 * C, 4)).astype(np.float32))
           for C in (3, 5)]
    data = DL.elra1_bytes(4, 8, 0.75, 16, W1, W2, ads)
    # header: magic, rank, style_dim, scale, gate hidden
    assert data[:8] == b"ELRA1\x00\x00\x00"
    assert struct.unpack_from("<iifi", data, 8) == (4, 8, 0.75, 16)
    # the gate's W1 tensor header right after
    assert struct.unpack_from("<ii", data, 24) == (16, 3)
    tensor = lambda rws, cls: 8 + 4 * rws * cls
    size = 24 + tensor(16, 3) + tensor(4, 16) + sum(4 + tensor(4, 8) + tensor(2 * C, 4) for C, _, _ in ads)
    assert len(data) == size
    back = DL.elra1_parse(data)
    assert (back["rank"], back["style_dim"], back["scale"], back["gate_hidden"]) == (4, 8, 0.75, 16)
    np.testing.assert_array_equal(back["W1"], W1)
    np.testing.assert_array_equal(back["W2"], W2)
    for (C, A, B), (C2, A2, B2) in zip(ads, back["adapters"]):
        assert C == C2
        np.testing.assert_array_equal(A, A2)
        np.testing.assert_array_equal(B, B2)
    with pytest.raises(ValueError):
        DL.elra1_parse(b"ELRA2" + data[5:])
