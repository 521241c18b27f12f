"""The probes behind bench.py's measured ceilings (glint_amd/csrc/gla_probe.hip): they run,
return figures in a physically possible range for one MI355X, and refuse bad arguments
without launching. The figures themselves are reported by the bench, not asserted here."""
from __future__ import annotations

import ctypes as C
import importlib.util
import pathlib

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_probe_library_exports_every_ceiling():
    """CPU: the probe library loads and exports what bench.py binds (no call)."""
    lib = C.CDLL(str(ROOT / "glint_amd" / "libglint_probe.so"))
    for name in ("glp_stream_read", "glp_read_per_launch", "glp_mfma_peak", "glp_mfma_clock"):
        assert hasattr(lib, name), name


@pytest.mark.gpu
def test_read_and_clock_probes(backend):
    bench = _bench()
    lib = bench.probe_lib()
    nbytes = 256 << 20
    buf = backend.empty(nbytes)
    out = C.c_double()
    try:
        # bad arguments come back as -1 before anything is launched
        assert lib.glp_read_per_launch(buf.ptr, nbytes, 0, 64, 1, C.byref(out)) == -1
        assert lib.glp_read_per_launch(buf.ptr, nbytes, 24, 64, 1, C.byref(out)) == -1
        assert lib.glp_read_per_launch(buf.ptr, 16, 32, 64, 1, C.byref(out)) == -1
        # one 4 MiB chunk per launch, 64 chunks in rotation: a launch takes at least the
        # empty-launch floor and reads no faster than the HBM's 8 TB/s
        assert lib.glp_read_per_launch(buf.ptr, nbytes, 4 << 20, 512, 50, C.byref(out)) == 0
        assert 0.5 < out.value < 1000.0, out.value
        assert (4 << 20) / (out.value * 1e-6) < 8.5e12
        assert lib.glp_stream_read(buf.ptr, nbytes, 3, C.byref(out)) == 0
        assert 500.0 < out.value < 8500.0, out.value
        assert lib.glp_mfma_clock(20000, C.byref(out)) == 0
        assert 500.0 < out.value < 3000.0, out.value  # MHz; the peak engine clock is 2.4 GHz
    finally:
        buf.free()
