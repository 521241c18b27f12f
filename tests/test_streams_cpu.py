"""Stream ownership in the Python mirror, on the CPU (the HIP runtime and the library are
replaced by recording fakes): a backend holds the HipStream it runs on, and destroying a
HipStream first moves every backend that used it back to its own stream and hands the
stream's scratch back (gla_release_stream) -- so no context is left pointing at a destroyed
hipStream_t."""
from __future__ import annotations

import ctypes as C
import gc

import pytest

from glint_amd import attn


class _FakeLib:
    def __init__(self):
        self.calls = []

    def gla_set_stream(self, ctx, ptr):
        self.calls.append(("set", ptr.value if isinstance(ptr, C.c_void_p) else ptr))
        return 0

    def gla_release_stream(self, ctx, ptr):
        self.calls.append(("release", ptr.value if isinstance(ptr, C.c_void_p) else ptr))
        return 0

    def gla_destroy(self, ctx):
        self.calls.append(("destroy", None))
        return 0


class _FakeHip:
    def __init__(self):
        self.next = 0x1000
        self.destroyed = []

    def hipStreamCreateWithFlags(self, out, flags):
        out._obj.value = self.next
        self.next += 0x10
        return 0

    def hipStreamDestroy(self, ptr):
        self.destroyed.append(ptr.value)
        return 0


@pytest.fixture
def fakes(monkeypatch):
    lib, hip = _FakeLib(), _FakeHip()
    monkeypatch.setattr(attn._lib, "lib", lambda: lib)
    monkeypatch.setattr(attn, "_hip", lambda: hip)
    return lib, hip


def _backend():
    be = attn.GpuBackend.__new__(attn.GpuBackend)
    be.ctx = C.c_void_p(0xC0)
    be._stream = None
    return be


def test_backend_keeps_the_stream_alive(fakes):
    lib, hip = fakes
    be = _backend()
    be.set_stream(attn.HipStream())  # no other reference to the stream
    gc.collect()
    assert hip.destroyed == []  # still held by the backend
    s = be._stream
    be.set_stream(None)
    assert be._stream is None
    del s
    gc.collect()
    assert hip.destroyed == [0x1000]
    # the stream left the context before it was destroyed, and its scratch was handed back
    assert lib.calls == [("set", 0x1000), ("set", None), ("release", 0x1000)]


def test_destroying_a_current_stream_resets_the_backend_first(fakes):
    lib, hip = fakes
    a, b = _backend(), _backend()
    s = attn.HipStream()
    a.set_stream(s)
    b.set_stream(s)
    b.set_stream(None)
    s.destroy()
    assert a._stream is None
    assert hip.destroyed == [0x1000]
    # both backends released the stream's scratch before hipStreamDestroy; `a` also switched back
    assert ("release", 0x1000) in lib.calls and lib.calls.count(("release", 0x1000)) == 2
    assert lib.calls.index(("set", None), 3) < len(lib.calls)
    with pytest.raises(ValueError, match="destroyed"):
        a.set_stream(s)
