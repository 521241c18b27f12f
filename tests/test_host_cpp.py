"""The C++ host layer (glint_amd/host/glint.hpp) through its test program
tests/cpp/test_host.cpp: page bookkeeping of PagePool / PagedKvCache with the
cases of src/cache/paged.rs's own tests (CPU, over a host-memory page store),
then on the GPU the same cases over the HBM pool plus attention through
GpuBackend against an f64 softmax and the paged == contiguous and
fork == fresh bitwise invariants."""
from __future__ import annotations

import subprocess

import pytest

from glint_amd import build as b


def _binary():
    if not (b.HOST_TEST.exists() and b.HOST_LIB.exists()):
        if not b.HIP_LIB.exists():
            b.build_hip()
        b.build_host()
        b.build_host_tests()
    return str(b.HOST_TEST)


def _run(*args, timeout):
    proc = subprocess.run([_binary(), *args], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout)
    return proc


def test_host_layer_bookkeeping_cpu():
    proc = _run(timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "0 failed (host)" in proc.stdout


@pytest.mark.gpu
def test_host_layer_device():
    proc = _run("--device", timeout=110)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "0 failed (device)" in proc.stdout
