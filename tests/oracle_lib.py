"""ctypes binding of the CPU parity oracle (oracle/build/libkdec_oracle.so).

Test infrastructure: imported only by tests, the smoke check and the bench's
CPU-baseline leg. The oracle is the checker, never the thing measured.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
# KDEC_ORACLE_LIB selects another build of the same sources (the sanitizer
# build of test_oracle_sanitize.py)
LIB_PATH = os.environ.get("KDEC_ORACLE_LIB") or os.path.join(ORACLE_DIR, "build", "libkdec_oracle.so")

_fp = ctypes.POINTER(ctypes.c_float)
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "-j8"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.ko_last_error.restype = ctypes.c_char_p
        for pre in ("ko_", "ko64_"):
            def f(n):
                return getattr(L, pre + n)
            f("model_last_error").restype = ctypes.c_char_p
            f("model_create").restype = ctypes.c_void_p
            f("model_create").argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int]
            for fn in ("model_destroy", "model_param_count", "model_unit_count",
                       "model_zero_grad"):
                f(fn).argtypes = [ctypes.c_void_p]
            f("model_param_name").restype = ctypes.c_char_p
            f("model_param_name").argtypes = [ctypes.c_void_p, ctypes.c_int]
            f("model_unit_name").restype = ctypes.c_char_p
            f("model_unit_name").argtypes = [ctypes.c_void_p, ctypes.c_int]
            f("model_unit_channels").argtypes = [ctypes.c_void_p, ctypes.c_int]
            for fn in ("model_audio_len", "model_har_len", "model_gen_in_len"):
                f(fn).restype = ctypes.c_long
                f(fn).argtypes = [ctypes.c_void_p]
            f("model_param_shape").argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                               ctypes.POINTER(ctypes.c_int),
                                               ctypes.POINTER(ctypes.c_int)]
            f("model_set_param").argtypes = [ctypes.c_void_p, ctypes.c_char_p, _fp, ctypes.c_long]
            f("model_get_grad").argtypes = [ctypes.c_void_p, ctypes.c_char_p, _fp, ctypes.c_long]
            f("model_get_affine").argtypes = [ctypes.c_void_p, ctypes.c_int, _fp, _fp, _fp, _fp]
            f("model_forward").argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _fp, ctypes.c_int, _fp]
            f("model_backward").argtypes = [ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int, _fp]
            for fn in ("model_get_audio", "model_get_har", "model_get_gen_in"):
                f(fn).argtypes = [ctypes.c_void_p, _fp]
            _dp = ctypes.POINTER(ctypes.c_double)
            f("model_set_param_f64").argtypes = [ctypes.c_void_p, ctypes.c_char_p, _dp, ctypes.c_long]
            f("model_forward_style_f64").argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _dp, ctypes.c_int,
                                                     _fp]
            f("model_get_audio_f64").argtypes = [ctypes.c_void_p, _dp]
            f("model_lora_enable").argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float]
            f("model_lora_set").argtypes = [ctypes.c_void_p, ctypes.c_int, _dp, _dp]
            f("model_lora_get_grad").argtypes = [ctypes.c_void_p, ctypes.c_int, _fp, _fp]
            f("model_lora_gate").argtypes = [ctypes.c_void_p, _dp]
            f("model_lora_get_dgate").argtypes = [ctypes.c_void_p, _fp]
            f("model_kink_site_count").argtypes = [ctypes.c_void_p]
            f("model_set_kink").argtypes = [ctypes.c_void_p, ctypes.c_int, _fp, ctypes.c_long]
            f("model_clear_kinks").argtypes = [ctypes.c_void_p]
            f("model_kink_flips").restype = ctypes.c_long
            f("model_kink_flips").argtypes = [ctypes.c_void_p, ctypes.c_int]
            f("model_leaky_input").argtypes = [ctypes.c_void_p, ctypes.c_int, _fp, ctypes.c_long]
            f("model_leaky_size").restype = ctypes.c_long
            f("model_leaky_size").argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.ko_leaky_fwd.argtypes = [_fp, ctypes.c_float, ctypes.c_long, _fp]
        L.ko_leaky_bwd.argtypes = [_fp, _fp, ctypes.c_float, ctypes.c_long, _fp]
        for fn in ("ko_instnorm_fwd", "ko_adain_affine_fwd"):
            getattr(L, fn).argtypes = [_fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        for fn in ("ko_instnorm_bwd", "ko_adain_affine_bwd"):
            getattr(L, fn).argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_float]
        _lib = L
    return _lib


def set_threads(n: int) -> int:
    """OpenMP threads of the oracle (n <= 0: all); returns the count in effect."""
    return int(lib().ko_set_threads(int(n)))


def P(a):
    """float32 pointer for a numpy array (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_fp)


def check(rc):
    if rc < 0:
        raise RuntimeError("oracle: " + lib().ko_last_error().decode())
    return rc


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ─── op wrappers (N = 1, numpy in / numpy out) ───

def conv1d_out_len(L, k, s, p, d):
    return (L + 2 * p - d * (k - 1) - 1) // s + 1


def convt1d_out_len(L, k, s, p, op, d):
    return (L - 1) * s - 2 * p + d * (k - 1) + op + 1


def conv1d(x, W, b, C_in, L, C_out, k, s=1, p=0, d=1, g=1):
    Lo = conv1d_out_len(L, k, s, p, d)
    y = np.zeros(C_out * Lo, np.float32)
    check(lib().ko_conv1d_fwd(P(f32(x)), P(f32(W)), P(None if b is None else f32(b)), P(y),
                              C_in, L, C_out, k, s, p, d, g))
    return y


def conv1d_dgrad(W, dy, C_in, L_in, C_out, k, s=1, p=0, d=1, g=1):
    dx = np.zeros(C_in * L_in, np.float32)
    check(lib().ko_conv1d_dgrad(P(f32(W)), P(f32(dy)), P(dx), C_in, L_in, C_out, k, s, p, d, g))
    return dx


def conv1d_wgrad(x, dy, C_in, L_in, C_out, k, s=1, p=0, d=1, g=1):
    dW = np.zeros(C_out * (C_in // g) * k, np.float32)
    db = np.zeros(C_out, np.float32)
    check(lib().ko_conv1d_wgrad(P(f32(x)), P(f32(dy)), P(dW), P(db), C_in, L_in, C_out, k, s, p, d, g))
    return dW, db


def convt1d(x, W, b, C_in, L, C_out, k, s=1, p=0, op=0, d=1, g=1):
    Lo = convt1d_out_len(L, k, s, p, op, d)
    y = np.zeros(C_out * Lo, np.float32)
    check(lib().ko_convt1d_fwd(P(f32(x)), P(f32(W)), P(None if b is None else f32(b)), P(y),
                               C_in, L, C_out, k, s, p, op, d, g))
    return y


def convt1d_dgrad(W, dy, C_in, L_in, C_out, k, s=1, p=0, op=0, d=1, g=1):
    dx = np.zeros(C_in * L_in, np.float32)
    check(lib().ko_convt1d_dgrad(P(f32(W)), P(f32(dy)), P(dx), C_in, L_in, C_out, k, s, p, op, d, g))
    return dx


def convt1d_wgrad(x, dy, C_in, L_in, C_out, k, s=1, p=0, op=0, d=1, g=1):
    dW = np.zeros(C_in * (C_out // g) * k, np.float32)
    db = np.zeros(C_out, np.float32)
    check(lib().ko_convt1d_wgrad(P(f32(x)), P(f32(dy)), P(dW), P(db), C_in, L_in, C_out, k, s, p, op,
                                 d, g))
    return dW, db


def instnorm(x, gamma, beta, C, L, eps=1e-5):
    y = np.zeros(C * L, np.float32)
    check(lib().ko_instnorm_fwd(P(f32(x)), P(f32(gamma)), P(f32(beta)), P(y), C, L, eps))
    return y


def instnorm_bwd(x, gamma, dy, C, L, eps=1e-5):
    dx = np.zeros(C * L, np.float32)
    dg = np.zeros(C, np.float32)
    db = np.zeros(C, np.float32)
    check(lib().ko_instnorm_bwd(P(f32(x)), P(f32(gamma)), P(f32(dy)), P(dx), P(dg), P(db), C, L, eps))
    return dx, dg, db


def adain_affine(x, gamma, beta, C, L, eps=1e-5):
    y = np.zeros(C * L, np.float32)
    check(lib().ko_adain_affine_fwd(P(f32(x)), P(f32(gamma)), P(f32(beta)), P(y), C, L, eps))
    return y


def adain_affine_bwd(x, gamma, dy, C, L, eps=1e-5):
    dx = np.zeros(C * L, np.float32)
    dg = np.zeros(C, np.float32)
    db = np.zeros(C, np.float32)
    check(lib().ko_adain_affine_bwd(P(f32(x)), P(f32(gamma)), P(f32(dy)), P(dx), P(dg), P(db), C, L,
                                    eps))
    return dx, dg, db


def snake(x, alpha, C, L):
    y = np.zeros(C * L, np.float32)
    check(lib().ko_snake_fwd(P(f32(x)), P(f32(alpha)), P(y), C, L))
    return y


def snake_bwd(x, alpha, dy, C, L):
    dx = np.zeros(C * L, np.float32)
    da = np.zeros(C, np.float32)
    check(lib().ko_snake_bwd(P(f32(x)), P(f32(alpha)), P(f32(dy)), P(dx), P(da), C, L))
    return dx, da


def leaky(x, slope):
    x = f32(x)
    y = np.zeros_like(x)
    check(lib().ko_leaky_fwd(P(x), slope, x.size, P(y)))
    return y


def leaky_bwd(x, dy, slope):
    x = f32(x)
    dx = np.zeros_like(x)
    check(lib().ko_leaky_bwd(P(x), P(f32(dy)), slope, x.size, P(dx)))
    return dx


def pad_reflect_left1(x, C, L):
    y = np.zeros(C * (L + 1), np.float32)
    check(lib().ko_pad_reflect_left1_fwd(P(f32(x)), C, L, P(y)))
    return y


def pad_reflect_left1_bwd(dy, C, L):
    dx = np.zeros(C * L, np.float32)
    check(lib().ko_pad_reflect_left1_bwd(P(f32(dy)), C, L, P(dx)))
    return dx


def hann(N):
    w = np.zeros(N, np.float32)
    check(lib().ko_hann(P(w), N))
    return w


def istft(spec, window, frames, signal_len, n_fft, hop, win=None):
    out = np.zeros(signal_len, np.float32)
    check(lib().ko_istft(P(f32(spec)), P(f32(window)), P(out), frames, signal_len, n_fft, hop,
                         win or n_fft))
    return out


def istft_bwd(dout, window, frames, signal_len, n_fft, hop, win=None):
    F = n_fft // 2 + 1
    ds = np.zeros(frames * 2 * F, np.float32)
    check(lib().ko_istft_bwd(P(f32(dout)), P(f32(window)), P(ds), frames, signal_len, n_fft, hop,
                             win or n_fft))
    return ds


def stft(x, window, n_fft, hop, win=None):
    x = f32(x)
    F = n_fft // 2 + 1
    maxf = x.size // hop + 2
    spec = np.zeros(maxf * 2 * F, np.float32)
    frames = check(lib().ko_stft(P(x), x.size, P(f32(window)), n_fft, hop, win or n_fft, P(spec), maxf))
    return spec[: frames * 2 * F], frames


def spectral_head(x, C, L, W, b, k, n_fft, hop):
    audio = np.zeros((L - 1) * hop, np.float32)
    post = np.zeros((n_fft + 2) * L, np.float32)
    check(lib().ko_spectral_head_fwd(P(f32(x)), C, L, P(f32(W)), P(f32(b)), k, n_fft, hop, P(audio),
                                     P(post)))
    return audio, post


def spectral_head_bwd(x, C, L, W, b, k, n_fft, hop, daudio, want_wgrad=True):
    dx = np.zeros(C * L, np.float32)
    dW = np.zeros((n_fft + 2) * C * k, np.float32) if want_wgrad else None
    db = np.zeros(n_fft + 2, np.float32) if want_wgrad else None
    check(lib().ko_spectral_head_bwd(P(f32(x)), C, L, P(f32(W)), P(f32(b)), k, n_fft, hop,
                                     P(f32(daudio)), P(dx), P(dW), P(db)))
    return dx, dW, db


def lora_fwd(W, b, A, B, g, scale, s):
    """One adapter, one utterance: y = W s + b + scale * B (g * (A s)); returns (y, h)."""
    rows, S = W.shape
    rank = A.shape[0]
    y = np.zeros(rows, np.float32)
    h = np.zeros(rank, np.float32)
    check(lib().ko_lora_fwd(P(f32(W)), P(None if b is None else f32(b)), P(f32(A)), P(f32(B)), P(f32(g)),
                            ctypes.c_float(scale), P(f32(s)), rows, rank, S, P(y), P(h)))
    return y, h


def lora_bwd(W, A, B, g, scale, s, h, dy):
    """Adjoint of lora_fwd: returns dict of dstyle, dW, db, dA, dB, dG."""
    rows, S = W.shape
    rank = A.shape[0]
    out = {"dstyle": np.zeros(S, np.float32), "dW": np.zeros((rows, S), np.float32),
           "db": np.zeros(rows, np.float32), "dA": np.zeros((rank, S), np.float32),
           "dB": np.zeros((rows, rank), np.float32), "dG": np.zeros(rank, np.float32)}
    check(lib().ko_lora_bwd(P(f32(W)), P(f32(A)), P(f32(B)), P(f32(g)), ctypes.c_float(scale), P(f32(s)),
                            P(f32(h)), P(f32(dy)), rows, rank, S, P(out["dstyle"]), P(out["dW"]), P(out["db"]),
                            P(out["dA"]), P(out["dB"]), P(out["dG"])))
    return out


def harmonic_source(F0, lW, lb, harmonic_num, sample_rate, upsample_scale, n_fft, hop):
    F0 = f32(F0)
    F = n_fft // 2 + 1
    maxf = F0.size * upsample_scale // hop + 2
    har = np.zeros(2 * F * maxf, np.float32)
    frames = check(lib().ko_harmonic_source(P(F0), F0.size, P(f32(lW)), P(f32(lb)), harmonic_num,
                                            sample_rate, upsample_scale, n_fft, hop, P(har), maxf))
    return har[: 2 * F * frames], frames


# ─── model ───

class OracleModel:
    """Whole decoder on the CPU oracle, parameters addressed by state-dict name.

    fp64=True selects the FP64 shadow (same source, double storage)."""

    def __init__(self, cfg: dict, fp64: bool = False):
        from brosoundml_amd.config import flat_ints
        self.cfg = cfg
        self.pre = "ko64_" if fp64 else "ko_"
        v = flat_ints(cfg)
        arr = (ctypes.c_int * len(v))(*v)
        self.h = self._f("model_create")(arr, len(v))
        if not self.h:
            raise RuntimeError("oracle: " + self._f("model_last_error")().decode())

    def _f(self, name):
        return getattr(lib(), self.pre + name)

    def _check(self, rc):
        if rc < 0:
            raise RuntimeError("oracle: " + self._f("model_last_error")().decode())
        return rc

    def __del__(self):
        if getattr(self, "h", None):
            self._f("model_destroy")(self.h)
            self.h = None

    def param_shapes(self) -> dict:
        out = {}
        for i in range(self._f("model_param_count")(self.h)):
            name = self._f("model_param_name")(self.h, i)
            r, c = ctypes.c_int(), ctypes.c_int()
            self._check(self._f("model_param_shape")(self.h, name, ctypes.byref(r), ctypes.byref(c)))
            out[name.decode()] = (r.value, c.value)
        return out

    def units(self) -> list:
        return [(self._f("model_unit_name")(self.h, i).decode(),
                 self._f("model_unit_channels")(self.h, i))
                for i in range(self._f("model_unit_count")(self.h))]

    def set_params(self, params: dict):
        for name, v in params.items():
            v = f32(v).ravel()
            self._check(self._f("model_set_param")(self.h, name.encode(), P(v), v.size))

    def set_params_f64(self, params: dict):
        for name, v in params.items():
            v = np.ascontiguousarray(v, dtype=np.float64).ravel()
            self._check(self._f("model_set_param_f64")(
                self.h, name.encode(), v.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), v.size))

    def forward_f64(self, asr, F0, N, style, T, har=None):
        """Forward with a double-precision style; returns double audio."""
        st = np.ascontiguousarray(style, dtype=np.float64)
        self._check(self._f("model_forward_style_f64")(
            self.h, P(f32(asr)), P(f32(F0)), P(f32(N)),
            st.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), T,
            P(None if har is None else f32(har))))
        a = np.zeros(self._f("model_audio_len")(self.h), np.float64)
        self._f("model_get_audio_f64")(self.h, a.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        return a

    def grad(self, name: str, shape) -> np.ndarray:
        g = np.zeros(int(np.prod(shape)), np.float32)
        self._check(self._f("model_get_grad")(self.h, name.encode(), P(g), g.size))
        return g

    def zero_grad(self):
        self._check(self._f("model_zero_grad")(self.h))

    def forward(self, asr, F0, N, style, T, har=None):
        self._check(self._f("model_forward")(self.h, P(f32(asr)), P(f32(F0)), P(f32(N)),
                                             P(f32(style)), T,
                                             P(None if har is None else f32(har))))
        a = np.zeros(self._f("model_audio_len")(self.h), np.float32)
        self._f("model_get_audio")(self.h, P(a))
        return a

    def har(self):
        h = np.zeros(self._f("model_har_len")(self.h), np.float32)
        self._f("model_get_har")(self.h, P(h))
        return h

    def gen_in(self):
        h = np.zeros(self._f("model_gen_in_len")(self.h), np.float32)
        self._f("model_get_gen_in")(self.h, P(h))
        return h

    def backward(self, daudio, wgrad=True, dalpha=True, dstyle=True):
        ds = np.zeros(self.cfg["style_dim"], np.float32) if dstyle else None
        self._check(self._f("model_backward")(self.h, P(f32(daudio)), int(wgrad), int(dalpha),
                                              P(ds)))
        return ds

    # ─── LoRA adapters on every AdaIN unit (decoder_lora.h:63-77) ───
    def lora_enable(self, rank, scale):
        self.lora_rank = rank
        self._check(self._f("model_lora_enable")(self.h, rank, ctypes.c_float(scale)))

    def lora_set(self, i, A=None, B=None):
        dp = ctypes.POINTER(ctypes.c_double)
        a = None if A is None else np.ascontiguousarray(A, np.float64)
        b = None if B is None else np.ascontiguousarray(B, np.float64)
        self._check(self._f("model_lora_set")(self.h, i, None if a is None else a.ctypes.data_as(dp),
                                              None if b is None else b.ctypes.data_as(dp)))

    def lora_gate(self, g):
        gg = np.ascontiguousarray(g, np.float64)
        self._check(self._f("model_lora_gate")(self.h, gg.ctypes.data_as(ctypes.POINTER(ctypes.c_double))))

    def lora_grads(self, i, C):
        S, r = self.cfg["style_dim"], self.lora_rank
        dA = np.zeros((r, S), np.float32)
        dB = np.zeros((2 * C, r), np.float32)
        self._check(self._f("model_lora_get_grad")(self.h, i, P(dA), P(dB)))
        return dA, dB

    def lora_dgate(self):
        d = np.zeros(self.lora_rank, np.float32)
        self._check(self._f("model_lora_get_dgate")(self.h, P(d)))
        return d

    # ─── leaky-site masks (see KinkMasks in oracle/kdec_oracle.hpp) ───
    def kink_site_count(self):
        return self._f("model_kink_site_count")(self.h)

    def set_kinks(self, pre):
        """Take every leaky site's branch from the signs of `pre` (a list of
        per-site inputs computed by another implementation), forward and backward."""
        self._f("model_clear_kinks")(self.h)
        for site, v in enumerate(pre):
            v = f32(v).ravel()
            self._check(self._f("model_set_kink")(self.h, site, P(v), v.size))

    def leaky_input(self, site):
        """The oracle's own input at leaky site `site` after a forward."""
        n = self._check(self._f("model_leaky_size")(self.h, site))
        v = np.zeros(n, np.float32)
        self._check(self._f("model_leaky_input")(self.h, site, P(v), n))
        return v

    def clear_kinks(self):
        self._f("model_clear_kinks")(self.h)

    def kink_flips(self, site=-1):
        """Elements whose own sign the last forward overrode (site -1: all)."""
        return self._f("model_kink_flips")(self.h, site)

    def affine(self, i, C):
        g, b, dg, db = (np.zeros(C, np.float32) for _ in range(4))
        self._check(self._f("model_get_affine")(self.h, i, P(g), P(b), P(dg), P(db)))
        return g, b, dg, db
