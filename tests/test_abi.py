"""CPU checks of the C ABI library: it loads, exports every function include/mnn.h declares,
the Python binding covers them all, and without a GPU the product path fails loudly."""
import re
from pathlib import Path

import numpy as np
import pytest

from metalaudio_amd import _lib, workloads

HEADERS = sorted((Path(__file__).resolve().parent.parent / "include").glob("*.h"))


def header_functions():
    """Every function any header under include/ declares (mnn.h, mnn_debug.h, ...)."""
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(mnn_[a-z0-9_]+)\s*\(", text))
    names.discard("mnn_completion_fn")  # a function-pointer type, not an entry point
    return sorted(names)


def test_library_is_built():
    assert _lib.LIB_PATH.exists(), "build libmnn.so first: python -m metalaudio_amd.build"


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_header():
    assert set(_lib.SIGNATURES) == set(header_functions())


def test_status_strings_and_version():
    lib = _lib.lib()
    assert lib.mnn_version().decode().startswith("mnn ")
    for code, name in _lib.STATUS.items():
        assert lib.mnn_status_string(code)
    assert lib.mnn_status_string(0).decode() == "ok"


def test_null_handles_are_rejected():
    lib = _lib.lib()
    assert lib.mnn_tensor_destroy(None) == 0  # destroying NULL is a no-op
    rc = lib.mnn_layer_forward(None, None, None, None)
    assert rc == 12 and b"null" in lib.mnn_last_error_message()


def test_no_gpu_fails_loudly():
    """On a machine without a HIP device, creating a device raises instead of falling back."""
    import ctypes as C
    lib = _lib.lib()
    h = C.c_void_p()
    rc = lib.mnn_device_create(0, C.byref(h))
    if rc == 0:  # a GPU is present (GPU box): nothing to check here
        lib.mnn_device_destroy(h)
        pytest.skip("GPU present")
    assert rc in (6, 3), rc
    with pytest.raises(_lib.MNNError):
        _lib.check(rc)


def test_workloads_are_seeded_and_shaped():
    a, b = workloads.config1(), workloads.config1()
    np.testing.assert_array_equal(a["x"], b["x"])
    assert a["x"].shape == (1, 2, 44100) and a["conv_w"].shape == (48, 2, 8)
    c4 = workloads.config4(samples=1000)
    assert [lv["conv.weight"].shape for lv in c4["levels"]] == [
        (48, 2, 8), (96, 48, 8), (192, 96, 8), (384, 192, 8)]
    assert abs(float(c4["levels"][1]["conv.weight"].std()) - np.sqrt(2 / 384)) < 0.01
    c5 = workloads.config5(batch=1, time_len=8, freq_len=16)
    assert c5["time"].shape == (1, 8, 384) and c5["freq"].shape == (1, 16, 384)
    assert "layers.1.time.norm3.weight" in c5["params"]
    assert "layers.0.time.norm3.weight" not in c5["params"]
