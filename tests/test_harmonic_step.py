"""The harmonic source's phase step on the GPU is branch free:

    y = fl(ph + omega)
    s = clamp(fma(y, 2^21, -fl(2pi) * 2^21), 0, 1)
    ph' = fma(s, -fl(2pi), y)

The reference's step (kokoro_modules.cpp:1611-1616) is y = fl(ph + omega);
ph' = fl(y - 2pi) if y > 2pi else y. The two must agree bit for bit on every
state the recurrence can reach, since the phase chain runs 300k steps and a
single differing rounding shifts everything after it.

Both fmas are single float32 additions of exact operands here (y * 2^21 is a
power-of-two scaling, s * 2pi with s in {0, 1} is exact), so numpy float32
arithmetic evaluates the device step exactly. The check runs the two steps
side by side over long chains at every harmonic of voiced F0 up to 800 Hz,
and exhaustively over all floats in the last 2^16 ulps below and above
fl(2pi) for a sweep of omegas, which is where the wrap decision is made.
"""
import numpy as np

TWO_PI = np.float32(6.28318530717958647692)
S = np.float32(2.0 ** 21)
TS = np.float32(-TWO_PI * S)


def ref_step(ph, w):
    y = (ph + w).astype(np.float32)
    return np.where(y > TWO_PI, (y - TWO_PI).astype(np.float32), y)


def device_step(ph, w):
    y = (ph + w).astype(np.float32)
    s = np.clip((y * S).astype(np.float32) + TS, np.float32(0), np.float32(1)).astype(np.float32)
    return ((s * -TWO_PI).astype(np.float32) + y).astype(np.float32)


def omegas(f0):
    f0 = np.asarray(f0, np.float32)
    out = []
    for h in range(9):
        w = (TWO_PI * np.float32(h + 1)).astype(np.float32)
        w = (w * f0).astype(np.float32)
        out.append((w / np.float32(24000.0)).astype(np.float32))
    return np.concatenate(out)


def test_step_is_a_clamp_select():
    # s is exactly 0 or 1 on every reachable y
    rng = np.random.default_rng(1)
    y = rng.uniform(0, 8, 1_000_000).astype(np.float32)
    s = np.clip((y * S).astype(np.float32) + TS, 0, 1)
    assert set(np.unique(s).tolist()) <= {0.0, 1.0}
    assert np.array_equal(s == 1.0, y > TWO_PI)


def test_long_chains_agree():
    rng = np.random.default_rng(2)
    w = omegas(np.concatenate([rng.uniform(0, 800, 400), [0.0, 80.0, 300.0, 799.9]]))
    ph_r = np.zeros_like(w)
    ph_d = np.zeros_like(w)
    for t in range(20_000):
        ph_r = ref_step(ph_r, w)
        ph_d = device_step(ph_d, w)
        if t % 1000 == 0:
            assert np.array_equal(ph_r.view(np.uint32), ph_d.view(np.uint32)), f"diverged by step {t}"
    assert np.array_equal(ph_r.view(np.uint32), ph_d.view(np.uint32))


def test_edges_around_two_pi_exhaustive():
    bits = TWO_PI.view(np.uint32)
    x = np.arange(int(bits) - (1 << 16), int(bits) + (1 << 16), dtype=np.uint32).view(np.float32)
    x = x[x <= TWO_PI]  # states never exceed fl(2pi)
    for w in np.concatenate([omegas([83.0, 170.5, 299.9, 611.0]), np.float32([1e-7, 2 ** -22, 3 * 2 ** -23])]):
        assert np.array_equal(ref_step(x, w).view(np.uint32), device_step(x, w).view(np.uint32)), f"omega {w}"
    # states just after a wrap and in the low binades
    lo = np.float32(np.concatenate([np.linspace(0, 4.2, 200_001), np.float32(2.0) ** -np.arange(1, 40)]))
    for w in omegas([97.0, 251.0]):
        assert np.array_equal(ref_step(lo, w).view(np.uint32), device_step(lo, w).view(np.uint32))
