"""Weight loading from safetensors (kdec_model_load_safetensors, the
reference's load_from over brotensor::safetensors): the host-side index on
the CPU (well-formed and malformed files), and on the GPU the whole decoder
loaded from a file of its own parameters, in fused and in weight-norm form
(weight = g * v / |v| per output row, scripts/convert-kokoro.py:71-110),
with the reference's errors for a missing key, a non-F32 tensor and a wrong
element count."""
import ctypes
import json
import struct

import numpy as np
import pytest

from brosoundml_amd import config as C
from brosoundml_amd import native, synth

st = pytest.importorskip("safetensors.numpy")


def count(path):
    return native.lib().kdec_safetensors_count(str(path).encode())


def test_index_and_malformed_files(tmp_path):
    p = tmp_path / "ok.safetensors"
    st.save_file({"a": np.ones((2, 3), np.float32), "b.c": np.zeros(5, np.float32)}, str(p),
                 metadata={"format": "pt"})
    assert count(p) == 2
    assert count(tmp_path / "missing.safetensors") < 0
    data = p.read_bytes()
    n = struct.unpack("<Q", data[:8])[0]
    bad = {
        "short": data[:5],
        "length_past_end": struct.pack("<Q", len(data)) + data[8:],
        "not_json": data[:8] + b"{" + b" " * (n - 1) + data[8 + n:],
        "offsets_past_end": None,
    }
    hdr = json.loads(data[8:8 + n])
    hdr["a"]["data_offsets"] = [0, 10 ** 6]
    h2 = json.dumps(hdr).encode()
    bad["offsets_past_end"] = struct.pack("<Q", len(h2)) + h2 + data[8 + n:]
    for name, b in bad.items():
        q = tmp_path / f"{name}.safetensors"
        q.write_bytes(b)
        assert count(q) < 0, name


@pytest.mark.gpu
def test_load_decoder_weights(tmp_path):
    torch = pytest.importorskip("torch")
    ctx = native.Context(0)
    cfg = C.TINY
    m = native.Model(ctx, cfg)
    shapes = m.param_shapes()
    params = {k: np.asarray(v, np.float32).reshape(shapes[k]) for k, v in synth.init_params(shapes).items()}
    # fused: every key as it is
    p = tmp_path / "fused.safetensors"
    st.save_file({k: v for k, v in params.items()}, str(p))
    m2 = native.Model(ctx, cfg)
    ctx.check(ctx.L.kdec_model_load_safetensors(m2.h, str(p).encode()))
    for k, s in shapes.items():
        np.testing.assert_array_equal(get_param(ctx, m2, k, s), params[k].ravel(), err_msg=k)
    # weight-norm form for every conv weight: v = W * positive row scales, g = |W_r|
    r = np.random.default_rng(3)
    wn = {}
    for k, v in params.items():
        if k.endswith(".weight") and v.ndim == 2 and "fc" not in k and "l_linear" not in k:
            scale = r.uniform(0.5, 2.0, (v.shape[0], 1)).astype(np.float32)
            wn[k[:-7] + ".weight_v"] = (v * scale).astype(np.float32)
            wn[k[:-7] + ".weight_g"] = np.linalg.norm(v.astype(np.float64), axis=1).astype(np.float32).reshape(-1, 1, 1)
        else:
            wn[k] = v
    assert any(k.endswith(".weight_g") for k in wn)
    p = tmp_path / "wn.safetensors"
    st.save_file(wn, str(p))
    m3 = native.Model(ctx, cfg)
    ctx.check(ctx.L.kdec_model_load_safetensors(m3.h, str(p).encode()))
    for k, s in shapes.items():
        got = get_param(ctx, m3, k, s)
        np.testing.assert_allclose(got, params[k].ravel(), rtol=2e-6, atol=1e-7, err_msg=k)
    # the reference's errors
    key = next(iter(shapes))
    cases = {
        "missing safetensors key": {k: v for k, v in params.items() if k != key},
        "is not F32": {**params, key: params[key].astype(np.float16)},
        "elements; expected": {**params, key: np.zeros(params[key].size + 1, np.float32)},
    }
    for msg, d in cases.items():
        q = tmp_path / "bad.safetensors"
        st.save_file(d, str(q))
        with pytest.raises(native.KdecError, match=msg):
            ctx.check(ctx.L.kdec_model_load_safetensors(m3.h, str(q).encode()))
    del torch


def get_param(ctx, m, name, shape):
    out = np.zeros(int(np.prod(shape)), np.float32)
    ctx.check(ctx.L.kdec_model_get_param(m.h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size))
    return out
