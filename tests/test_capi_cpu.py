"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, reports a missing device as GpuAdapterNotFound (the condition
the reference's callers fall back to the CPU on, src/main.rs:893-904), rejects
bad arguments without touching a device, and shares the oracle's window rule."""
import ctypes as C
import re
from pathlib import Path

import pytest

import oracle as orc
from glint_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "glint_attn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(gla_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_api():
    names = declared_functions()
    assert len(names) >= 25
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(hip_lib):
    for name in declared_functions():
        assert hasattr(hip_lib, name), name


def _visible_devices():
    import subprocess, sys
    code = "import ctypes;h=ctypes.CDLL('libamdhip64.so');n=ctypes.c_int(0);r=h.hipGetDeviceCount(ctypes.byref(n));print(n.value if r==0 else 0)"
    try:
        return int(subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=60).stdout.strip() or 0)
    except Exception:
        return 0


def test_no_device_is_gpu_adapter_not_found(hip_lib):
    if _visible_devices() > 0:
        pytest.skip("a HIP device is visible here")
    from glint_amd.attn import GpuBackend
    with pytest.raises(_lib.GlaError) as ei:
        GpuBackend(0)
    assert ei.value.code == _lib.GLA_ERR_NO_DEVICE and ei.value.name == "GpuAdapterNotFound"


def test_null_arguments_are_rejected(hip_lib):
    assert hip_lib.gla_create(0, None) == _lib.GLA_ERR_INVALID
    assert "NULL" in _lib.last_error()
    assert hip_lib.gla_sync(None) == _lib.GLA_ERR_INVALID
    assert hip_lib.gla_decode(None, None) == _lib.GLA_ERR_INVALID
    assert hip_lib.gla_prefill(None, None) == _lib.GLA_ERR_INVALID
    out = C.c_void_p()
    assert hip_lib.gla_kv_cache_create(None, 0, 1, 1, 1, 1, 64, C.byref(out)) == _lib.GLA_ERR_INVALID
    assert hip_lib.gla_kv_row_id(None, 0, 0, 0) == -1
    assert hip_lib.gla_destroy(None) == _lib.GLA_OK
    assert hip_lib.gla_kv_destroy(None) == _lib.GLA_OK


def test_window_start_matches_oracle(hip_lib):
    for w in (0, 1, 7, 16, 4096):
        for alt in (0, 1):
            for layer in (0, 1, 2, 5):
                for pos in (0, 1, 6, 7, 15, 16, 100, 4095, 4096, 9000):
                    assert hip_lib.gla_window_start(pos, w, alt, layer) == orc.window_start(pos, w, bool(alt), layer)


def test_decode_args_layout_matches_header():
    """The ctypes mirror of gla_decode_args has the header's field order, ending with the
    optional host copies of kv_start / kv_len."""
    import re
    from pathlib import Path
    from glint_amd import _lib
    hdr = (Path(__file__).resolve().parents[1] / "include" / "glint_attn.h").read_text()
    body = hdr[hdr.index("typedef struct gla_decode_args"):hdr.index("} gla_decode_args;")]
    names = re.findall(r"\b(\w+);", re.sub(r"/\*.*?\*/", "", body, flags=re.S))
    assert names == [f for f, _ in _lib.DecodeArgs._fields_]
