"""CPU checks of the C ABI: the product library loads without a GPU and
exports every function include/*.h declares (no compute calls here)."""
import ctypes
import os
import re

from brosoundml_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for h in ("kdec.h", "kdec_model.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        names |= set(re.findall(r"\b(kdec_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(native.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(L, n)]
    assert not missing, missing


def test_header_parse_matches_declarations():
    sigs = native.parse_headers()
    assert set(sigs) == declared()
    ret, args = sigs["kdec_conv1d_fwd"]
    assert ret is ctypes.c_int and len(args) == 19
    assert sigs["kdec_last_error"][0] is ctypes.c_char_p
    assert sigs["kdec_model_param_ptr"][0] is ctypes.c_void_p


def test_binding_loads():
    L = native.lib()
    assert L.kdec_last_error(None) == b"brosoundml: null context"
    # a null context is rejected, not dereferenced
    assert L.kdec_synchronize(None) == -1
