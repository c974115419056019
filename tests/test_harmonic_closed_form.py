"""Closed forms of the harmonic source (kokoro_modules.cpp:1574-1665), each a
construction whose STFT is known exactly, aimed at one constant or index of
the reference:

* the unvoiced gate (uv = F0 > 0, :1604): frames of F0 <= 0 carry no sine, so
  with a zero l_linear bias their magnitude is exactly zero;
* the l_linear bias and the tanh (:1621-1625): an all-unvoiced signal is the
  constant c = tanh(b), whose periodic-Hann STFT is c times the window's DFT:
  |X[0]| = (n_fft / 2) |c|, |X[1]| = (n_fft / 4) |c| and nothing else, in
  every frame (the reflect padding of a constant is the constant);
* sine_amp = 0.1 and the harmonic frequency (h + 1) * F0 (:1606-1614): with
  one active harmonic (lW = w e_h, w small so tanh is linear to 1e-7) and
  (h + 1) F0 on bin k of sample_rate / n_fft, an interior frame of the sine
  A sin(theta) (A = 0.1 w) holds |X[k]| = A n_fft / 4 and
  |X[k +- 1]| = A n_fft / 8 (the periodic Hann's DFT is n/2, -n/4, -n/4 at
  bins 0, +-1), and no other bin;
* the nearest-neighbour upsampling index frame = t / upsample_scale (:1602):
  an F0 step from 0 to a voiced value at input frame f makes sample
  300 f the first nonzero sample. The STFT frame j covers samples
  [5 j - 10, 5 j + 10), so frame 60 f - 2 is exactly zero and frame
  60 f - 1 equals the windowed DFT of a signal whose first 15 samples are
  zero, computed here in float64 from the sine's own definition; the index
  rule (t + 1) / 300 or (t - 1) / 300 moves the first sample by one and fails
  one of the two.

Each construction runs on the oracle (CPU) and, in the gpu-marked case at the
end, through the gfx950 kernels (kdec_harmonic_source), whose magnitudes must
also be within rel-L2 1e-5 of the oracle's.
"""
import numpy as np
import pytest

import oracle_lib as O

N_FFT, HOP, SR, US, HN = 20, 5, 24000, 300, 8
F = N_FFT // 2 + 1
BIN_HZ = SR / N_FFT  # 1200 Hz per bin


def run_oracle(F0, lW, lb):
    har, frames = O.harmonic_source(np.asarray(F0, np.float32), np.asarray(lW, np.float32),
                                    np.asarray([lb], np.float32), HN, SR, US, N_FFT, HOP)
    return har.reshape(2 * F, frames)


def unit_lw(h, w):
    lW = np.zeros(HN + 1, np.float32)
    lW[h] = w
    return lW


def check_unvoiced_zero(har, frames_sl=slice(None)):
    mag = har[:F, frames_sl]
    assert np.all(mag == 0.0), f"max magnitude {np.max(mag):.3e} on unvoiced frames"


def check_bias(har, b):
    mag = har[:F]
    want = (N_FFT / 2) * abs(np.tanh(np.float64(b)))
    np.testing.assert_allclose(mag[0], want, rtol=2e-6)
    np.testing.assert_allclose(mag[1], want / 2, rtol=2e-6)
    assert np.max(mag[2:]) <= 1e-6 * want


def check_peak(har, k, A, interior):
    mag = har[:F, interior].astype(np.float64)
    np.testing.assert_allclose(mag[k], A * N_FFT / 4, rtol=2e-5)
    # bin 0 of a bin-1 sine also takes the mirror term: |X[0]| = A n/4 |sin phi|
    for kk in (k - 1, k + 1):
        if 0 < kk < F:
            np.testing.assert_allclose(mag[kk], A * N_FFT / 8, rtol=4e-5)
    rest = [i for i in range(F) if abs(i - k) > 1]
    assert np.max(mag[rest]) <= 2e-5 * A * N_FFT / 4, np.max(mag[rest])


def step_frame_expected(A, omega):
    """|DFT| of STFT frame 60 f - 1 of a sine that starts at sample 300 f:
    window samples n = 0..19 cover t = 300 f - 15 + n, the sine is
    A sin(omega * (t - 300 f + 1)) from t = 300 f on (the phase accumulator
    adds omega before each sample and does not move while F0 = 0)."""
    n = np.arange(N_FFT)
    w = 0.5 - 0.5 * np.cos(2 * np.pi * n / N_FFT)
    tt = n - 15  # t - 300 f
    x = np.where(tt >= 0, A * np.sin(omega * (tt + 1)), 0.0)
    return np.abs(np.fft.rfft(w * x))


@pytest.mark.parametrize("f0", [0.0, -150.0])
def test_unvoiced_frames_are_silent(f0):
    har = run_oracle(np.full(6, f0), unit_lw(0, 0.7), 0.0)
    check_unvoiced_zero(har)


@pytest.mark.parametrize("b", [0.3, -0.8])
def test_bias_through_tanh(b):
    har = run_oracle(np.zeros(6), unit_lw(2, 0.5), b)
    check_bias(har, b)


@pytest.mark.parametrize("f0,h,k", [(1200.0, 0, 1), (1200.0, 1, 2), (600.0, 1, 1), (2400.0, 2, 6)])
def test_sine_amp_and_harmonic_frequency(f0, h, k):
    assert (h + 1) * f0 == k * BIN_HZ
    w = 1e-3
    har = run_oracle(np.full(4, f0), unit_lw(h, w), 0.0)
    frames = har.shape[1]
    check_peak(har, k, 0.1 * w, slice(3, frames - 3))


@pytest.mark.parametrize("f", [1, 3])
def test_f0_step_starts_at_sample_300f(f):
    f0, w = 1200.0, 1e-3
    F0 = np.zeros(5, np.float32)
    F0[f:] = f0
    har = run_oracle(F0, unit_lw(0, w), 0.0)
    j = 60 * f
    check_unvoiced_zero(har, slice(0, j - 1))
    omega = float(np.float32(2 * np.pi) * np.float32(1.0) * np.float32(f0) / np.float32(SR))
    want = step_frame_expected(0.1 * w, omega)
    got = har[:F, j - 1].astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6 * want.max())
    # a one-sample shift of the start changes that frame by O(1)
    for shift in (-1, 1):
        n = np.arange(N_FFT)
        wdw = 0.5 - 0.5 * np.cos(2 * np.pi * n / N_FFT)
        tt = n - 15 - shift
        x = np.where(tt >= 0, 0.1 * w * np.sin(omega * (tt + 1)), 0.0)
        alt = np.abs(np.fft.rfft(wdw * x))
        assert np.linalg.norm(alt - want) > 0.05 * np.linalg.norm(want)


CASES = [
    ("unvoiced0", np.full(6, 0.0), unit_lw(0, 0.7), 0.0),
    ("unvoiced_neg", np.full(6, -150.0), unit_lw(0, 0.7), 0.0),
    ("bias", np.zeros(6), unit_lw(2, 0.5), 0.3),
    ("peak_h0", np.full(4, 1200.0), unit_lw(0, 1e-3), 0.0),
    ("peak_h1", np.full(4, 1200.0), unit_lw(1, 1e-3), 0.0),
    ("peak_h2", np.full(4, 2400.0), unit_lw(2, 1e-3), 0.0),
    ("step_f3", np.array([0, 0, 0, 1200, 1200], np.float32), unit_lw(0, 1e-3), 0.0),
]


@pytest.mark.gpu
def test_gpu_harmonic_source_closed_forms():
    torch = pytest.importorskip("torch")
    from brosoundml_amd import native
    ctx = native.Context(0)
    for name, F0, lW, lb in CASES:
        F0 = np.asarray(F0, np.float32)
        ref = run_oracle(F0, lW, lb)
        frames = ref.shape[1]
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
        tF0, tW, tb = d(F0[None]), d(lW), d(np.array([lb], np.float32))
        har = torch.full((1, 2 * F * frames), float("nan"), device="cuda")
        ctx.call("kdec_harmonic_source", native.ptr(tF0), F0.size, native.ptr(har), har.shape[1], 1, F0.size,
                 native.ptr(tW), native.ptr(tb), HN, SR, US, N_FFT, HOP)
        torch.cuda.synchronize()
        got = har.cpu().numpy().reshape(2 * F, frames)
        print(f"{name}: frames {frames}", flush=True)
        den = max(np.linalg.norm(ref[:F].astype(np.float64)), 1e-30)
        e = np.linalg.norm(got[:F].astype(np.float64) - ref[:F]) / den
        assert e <= 1e-5 or not np.any(ref[:F]), f"{name}: magnitude rel-L2 {e:.3e} vs the oracle"
        if name.startswith("unvoiced"):
            check_unvoiced_zero(got)
        elif name == "bias":
            check_bias(got, lb)
        elif name.startswith("peak"):
            h = int(np.argmax(lW))
            check_peak(got, int((h + 1) * F0[0] / BIN_HZ), 0.1 * 1e-3, slice(3, frames - 3))
        else:
            check_unvoiced_zero(got, slice(0, 60 * 3 - 1))
