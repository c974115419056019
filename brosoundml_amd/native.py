"""ctypes binding of libkdec.so (the gfx950 kernels, the C ABI and the C++
drop-in layer). Torch supplies device memory and the stream; every compute
call goes through the C ABI. There is no fallback: if the library is missing
or no HIP device is present, construction fails loudly."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkdec.so")

ROOT = os.path.dirname(HERE)
HEADERS = [os.path.join(ROOT, "include", "kdec.h"), os.path.join(ROOT, "include", "kdec_model.h")]


def _ctype(decl: str):
    """ctypes type for a C declaration's type part (pointer-sized for any pointer)."""
    d = decl.replace("const", " ").strip()
    if "*" in d:
        single_char = d.count("*") == 1 and d.replace("*", "").split() == ["char"]
        return ctypes.c_char_p if single_char else ctypes.c_void_p
    base = d.split()[-1] if d.split() else d
    if base.endswith("_fn"):  # a callback typedef
        return ctypes.c_void_p
    return {"int": ctypes.c_int, "long": ctypes.c_long, "float": ctypes.c_float,
            "double": ctypes.c_double, "size_t": ctypes.c_size_t, "void": None}[base]


def parse_headers(paths=HEADERS) -> dict:
    """{name: (restype, [argtypes])} for every function the C headers declare."""
    import re
    sigs = {}
    for path in paths:
        with open(path) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(kdec_\w+)\s*\(([^)]*)\)\s*;", text):
            ret, name, params = m.group(1), m.group(2), m.group(3).strip()
            args = []
            if params and params != "void":
                for prm in params.split(","):
                    prm = prm.strip()
                    mm = re.match(r"(.*?)([A-Za-z_]\w*)$", prm)
                    args.append(_ctype(mm.group(1) if mm and mm.group(1).strip() else prm))
            sigs[name] = (_ctype(ret), args)
    return sigs


_lib = None


def exported_symbols():
    return list(parse_headers())


def lib():
    """Loads libkdec.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m brosoundml_amd.build`")
        # torch ships its own libamdhip64 with the same soname as ROCm's;
        # loading torch first makes libkdec bind to that one runtime instead
        # of bringing a second HIP runtime into the process.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in parse_headers().items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(t):
    """Device (or host) address of a torch tensor, or None."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


class KdecError(RuntimeError):
    pass


class Context:
    """A kdec context bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0, stream=None):
        import torch
        if not torch.cuda.is_available():
            raise KdecError("no HIP device: the gfx950 library has no CPU path")
        self.L = lib()
        h = ctypes.c_void_p()
        rc = self.L.kdec_ctx_create(device, ctypes.byref(h))
        if rc != 0:
            raise KdecError(f"kdec_ctx_create failed ({rc})")
        self.h = h
        self.device = device
        s = stream if stream is not None else torch.cuda.current_stream(device)
        self.check(self.L.kdec_set_stream(self.h, ctypes.c_void_p(s.cuda_stream)))

    def close(self):
        if getattr(self, "h", None):
            self.L.kdec_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc):
        if rc != 0:
            raise KdecError(self.L.kdec_last_error(self.h).decode())
        return rc

    def call(self, name, *args):
        return self.check(getattr(self.L, name)(self.h, *args))

    def synchronize(self):
        self.call("kdec_synchronize")

    # profiling
    def profile(self, on=True):
        self.call("kdec_profile_enable", int(on))

    def profile_reset(self):
        self.call("kdec_profile_reset")

    def profile_read(self):
        cap = 64
        names = (ctypes.c_char_p * cap)()
        ms = (ctypes.c_double * cap)()
        launches = (ctypes.c_long * cap)()
        flops = (ctypes.c_double * cap)()
        nbytes = (ctypes.c_double * cap)()
        n = self.L.kdec_profile_read(self.h, ctypes.cast(names, ctypes.c_void_p),
                                     ctypes.cast(ms, ctypes.c_void_p),
                                     ctypes.cast(launches, ctypes.c_void_p),
                                     ctypes.cast(flops, ctypes.c_void_p),
                                     ctypes.cast(nbytes, ctypes.c_void_p), cap)
        if n < 0:
            raise KdecError(self.L.kdec_last_error(self.h).decode())
        return {names[i].decode(): dict(ms=ms[i], launches=launches[i], flops=flops[i], bytes=nbytes[i])
                for i in range(min(n, cap))}


def config_ints(cfg: dict) -> list[int]:
    from .config import flat_ints
    return flat_ints(cfg)


class Model:
    """The whole decoder (kdec_model.h) on a Context."""

    def __init__(self, ctx: Context, cfg: dict):
        self.ctx = ctx
        self.cfg = cfg
        v = config_ints(cfg)
        arr = (ctypes.c_int * len(v))(*v)
        h = ctypes.c_void_p()
        rc = ctx.L.kdec_model_create(ctx.h, ctypes.cast(arr, ctypes.c_void_p), len(v), ctypes.byref(h))
        if rc != 0:
            raise KdecError(f"kdec_model_create failed ({rc})")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            self.ctx.L.kdec_model_destroy(self.h)
            self.h = None

    def _c(self, rc):
        return self.ctx.check(rc)

    def param_shapes(self) -> dict:
        L = self.ctx.L
        out = {}
        for i in range(L.kdec_model_param_count(self.h)):
            name = L.kdec_model_param_name(self.h, i)
            r, c = ctypes.c_int(), ctypes.c_int()
            self._c(L.kdec_model_param_shape(self.h, name, ctypes.cast(ctypes.pointer(r), ctypes.c_void_p),
                                             ctypes.cast(ctypes.pointer(c), ctypes.c_void_p)))
            out[name.decode()] = (r.value, c.value)
        return out

    def units(self) -> list:
        L = self.ctx.L
        return [(L.kdec_model_unit_name(self.h, i).decode(), L.kdec_model_unit_channels(self.h, i),
                 L.kdec_model_unit_offset(self.h, i)) for i in range(L.kdec_model_unit_count(self.h))]

    def affine_rows(self) -> int:
        return self.ctx.L.kdec_model_affine_rows(self.h)

    def set_params(self, params: dict):
        import numpy as np
        for name, v in params.items():
            a = np.ascontiguousarray(v, dtype=np.float32).ravel()
            self._c(self.ctx.L.kdec_model_set_param(self.h, name.encode(), a.ctypes.data_as(ctypes.c_void_p),
                                                    a.size))

    def grad(self, name: str, shape):
        import numpy as np
        g = np.zeros(int(np.prod(shape)), np.float32)
        self._c(self.ctx.L.kdec_model_get_grad(self.h, name.encode(), g.ctypes.data_as(ctypes.c_void_p), g.size))
        return g

    def zero_grad(self):
        self._c(self.ctx.L.kdec_model_zero_grad(self.h))

    def lengths(self, T):
        a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        self._c(self.ctx.L.kdec_model_lengths(self.h, T, ctypes.cast(ctypes.pointer(a), ctypes.c_void_p),
                                              ctypes.cast(ctypes.pointer(b), ctypes.c_void_p),
                                              ctypes.cast(ctypes.pointer(c), ctypes.c_void_p)))
        return dict(L_gen=a.value, frames=b.value, audio=c.value)

    def forward(self, asr, F0, Nn, style, T, har=None, audio=None):
        import torch
        N = asr.shape[0]
        if audio is None:
            audio = torch.empty(N, self.lengths(T)["audio"], device=asr.device, dtype=torch.float32)
        self._c(self.ctx.L.kdec_model_forward(self.h, N, T, ptr(asr), ptr(F0), ptr(Nn), ptr(style), ptr(har),
                                              ptr(audio)))
        # the training caches refer to the inputs (asr, F0 and N feed the
        # backbone's input-conv weight grads): held until the next forward,
        # as the reference's cache tensors share their storage
        self._keep = (asr, F0, Nn, style, har)
        self.N_last = N
        return audio

    def backward(self, daudio, wgrad=True, dalpha=True, dstyle=None):
        self._c(self.ctx.L.kdec_model_backward(self.h, ptr(daudio), int(wgrad), int(dalpha), ptr(dstyle)))

    def set_overlap(self, on: bool):
        """True (default): harmonic source and conv weight grads on a second
        stream; False: every launch on the context's stream in program order."""
        self._c(self.ctx.L.kdec_model_set_overlap(self.h, int(on)))

    def set_batch_split(self, on: bool):
        """True: with overlap on, forwards and backwards of N >= 2 run as two
        half-batch chains on two streams; False (default): one chain."""
        self._c(self.ctx.L.kdec_model_set_batch_split(self.h, int(on)))

    # ─── DecoderLora adapters (kdec_model_lora_*) ───
    def lora_enable(self, rank: int, scale: float):
        self.lora_rank = rank
        self._c(self.ctx.L.kdec_model_lora_enable(self.h, rank, scale))

    def _lora_shape(self, which: int):
        if which % 2 == 0:
            return len(self.units()) * self.lora_rank, self.cfg["style_dim"]
        return self.affine_rows(), self.lora_rank

    def lora_set(self, A=None, B=None):
        """Copies A (units*rank, style_dim) and / or B (affine_rows, rank) into the model (device copy)."""
        import torch
        for which, v in ((0, A), (1, B)):
            if v is None:
                continue
            t = torch.as_tensor(v, dtype=torch.float32).reshape(self._lora_shape(which)).contiguous().cuda()
            dst = self.ctx.L.kdec_model_lora_ptr(self.h, which)
            if not dst:
                raise KdecError("kdec_model_lora_ptr: adapters not enabled")
            self.ctx.check(self.ctx.L.kdec_axpby(self.ctx.h, 1.0, ptr(t), 0, 0.0, None, 0, ctypes.c_void_p(dst), 0,
                                                 1, t.numel()))
            self.ctx.synchronize()

    def lora_grads(self):
        """(dA, dB) as host arrays."""
        import torch
        out = []
        for which in (2, 3):
            shape = self._lora_shape(which)
            t = torch.empty(shape, dtype=torch.float32, device="cuda")
            src = self.ctx.L.kdec_model_lora_ptr(self.h, which)
            self.ctx.check(self.ctx.L.kdec_axpby(self.ctx.h, 1.0, ctypes.c_void_p(src), 0, 0.0, None, 0, ptr(t), 0,
                                                 1, t.numel()))
            self.ctx.synchronize()
            out.append(t.cpu().numpy())
        return tuple(out)

    def lora_gate(self, g, dG=None):
        """g: torch cuda (N, rank) or (rank,) for one gate shared by every utterance."""
        g_bs = self.lora_rank if g.dim() == 2 else 0
        self._lora_keep = (g, dG)
        self._c(self.ctx.L.kdec_model_lora_gate(self.h, ptr(g), g_bs, ptr(dG)))

    def affines(self, N):
        import numpy as np
        R = self.affine_rows()
        gb = np.zeros(N * R, np.float32)
        dgb = np.zeros(N * R, np.float32)
        self._c(self.ctx.L.kdec_model_get_affines(self.h, gb.ctypes.data_as(ctypes.c_void_p),
                                                  dgb.ctypes.data_as(ctypes.c_void_p)))
        return gb.reshape(N, R), dgb.reshape(N, R)

    def har_ptr(self):
        return self.ctx.L.kdec_model_har(self.h)

    def leaky_inputs(self):
        """Host copies of every leaky-ReLU site's input of the last training
        forward (kdec_model_leaky_input), in site order: a list of (N, C*L) arrays."""
        import numpy as np
        L = self.ctx.L
        res = []
        for site in range(L.kdec_model_leaky_site_count(self.h)):
            n = L.kdec_model_leaky_size(self.h, site)
            if n < 0:
                raise KdecError(L.kdec_last_error(self.ctx.h).decode())
            a = np.empty(n, np.float32)
            self._c(L.kdec_model_leaky_input(self.h, site, a.ctypes.data_as(ctypes.c_void_p), n))
            res.append(a.reshape(self.N_last, -1))
        return res

    def har(self, N, T):
        """Host copy of the last forward's harmonic-source output (N, (n_fft+2)*frames)."""
        import torch
        n = (self.cfg["n_fft"] + 2) * self.lengths(T)["frames"]
        t = torch.empty((N, n), dtype=torch.float32, device="cuda")
        self.ctx.check(self.ctx.L.kdec_axpby(self.ctx.h, 1.0, ctypes.c_void_p(self.har_ptr()), n, 0.0, None, 0,
                                             ptr(t), n, N, n))
        self.ctx.synchronize()
        return t.cpu().numpy()


class DecoderLora:
    """DecoderLora (kdec_dlora_*) over a Model's frozen weights: the LoRA on
    every AdaIN unit's style projection with the shared conditioning gate,
    Adam state and the ELRA1 checkpoint."""

    NAMES = {"A": 0, "B": 1, "dA": 2, "dB": 3, "W1": 4, "W2": 5, "dW1": 6, "dW2": 7}

    def __init__(self, model: "Model", rank: int, scale: float, seed: int = 0):
        self.model = model
        self.ctx = model.ctx
        h = ctypes.c_void_p()
        model._c(self.ctx.L.kdec_dlora_create(model.h, rank, scale, seed, ctypes.byref(h)))
        self.h = h
        self.rank = rank

    def __del__(self):
        try:
            if getattr(self, "h", None):
                self.ctx.L.kdec_dlora_destroy(self.h)
                self.h = None
        except Exception:
            pass

    def _c(self, rc):
        return self.model._c(rc)

    def tensor(self, name):
        """(device pointer, rows, cols) of A, B, dA, dB, W1, W2, dW1 or dW2."""
        r, c = ctypes.c_int(), ctypes.c_int()
        p = self.ctx.L.kdec_dlora_ptr(self.h, self.NAMES[name], ctypes.cast(ctypes.pointer(r), ctypes.c_void_p),
                                      ctypes.cast(ctypes.pointer(c), ctypes.c_void_p))
        if not p:
            raise KdecError(f"kdec_dlora_ptr({name}) failed")
        return p, r.value, c.value

    def get(self, name):
        import torch
        p, r, c = self.tensor(name)
        torch.cuda.synchronize()
        t = torch.empty((r, c), dtype=torch.float32, device="cuda")
        self.ctx.check(self.ctx.L.kdec_axpby(self.ctx.h, 1.0, ctypes.c_void_p(p), c, 0.0, None, 0, ptr(t), c, r, c))
        return t.cpu().numpy()

    def set(self, name, value):
        import numpy as np
        import torch
        p, r, c = self.tensor(name)
        v = np.ascontiguousarray(value, np.float32).reshape(r, c)
        t = torch.from_numpy(v).cuda()
        self.ctx.check(self.ctx.L.kdec_axpby(self.ctx.h, 1.0, ptr(t), c, 0.0, None, 0, ctypes.c_void_p(p), c, r, c))
        torch.cuda.synchronize()

    def forward(self, asr, F0, Nn, ref_s, T, cond, har=None, audio=None):
        import torch
        N = asr.shape[0]
        if audio is None:
            audio = torch.empty(N, self.model.lengths(T)["audio"], device=asr.device, dtype=torch.float32)
        self._keep = (asr, F0, Nn, ref_s, cond, har)
        self._N = N
        self._c(self.ctx.L.kdec_dlora_forward(self.h, N, T, ptr(asr), ptr(F0), ptr(Nn), ptr(ref_s),
                                              ref_s.stride(0), ptr(har), ptr(cond), ptr(audio)))
        return audio

    def backward(self, daudio):
        self._c(self.ctx.L.kdec_dlora_backward(self.h, ptr(daudio)))

    def leaky_inputs(self):
        """Host copies of every leaky-ReLU site's input of the last DecoderLora
        forward (kdec_dlora_leaky_input), in site order: (N, C*L) arrays."""
        import numpy as np
        L = self.ctx.L
        res = []
        for site in range(L.kdec_model_leaky_site_count(self.model.h)):
            n = L.kdec_dlora_leaky_size(self.h, site)
            if n < 0:
                raise KdecError(L.kdec_last_error(self.ctx.h).decode())
            a = np.empty(n, np.float32)
            self._c(L.kdec_dlora_leaky_input(self.h, site, a.ctypes.data_as(ctypes.c_void_p), n))
            res.append(a.reshape(self._N, -1))
        return res

    def zero_grad(self):
        self._c(self.ctx.L.kdec_dlora_zero_grad(self.h))

    def adam_step(self, lr, beta1=0.9, beta2=0.999, eps=1e-8):
        self._c(self.ctx.L.kdec_dlora_adam_step(self.h, lr, beta1, beta2, eps))

    def save(self, path):
        self._c(self.ctx.L.kdec_dlora_save(self.h, os.fsencode(path)))

    def load(self, path):
        self._c(self.ctx.L.kdec_dlora_load(self.h, os.fsencode(path)))

    @property
    def scale(self):
        return self.ctx.L.kdec_dlora_scale(self.h)
