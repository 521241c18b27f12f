import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs on an MI355X through libglint_attn.so (the C ABI)")


@pytest.fixture(scope="session", autouse=True)
def host_libs():
    """The host helper libraries (gcc, seconds); built here only if absent."""
    from glint_amd import build

    if not build.SYNTH_LIB.exists():
        build.build_synth()
    if not build.ORACLE_LIB.exists():
        build.build_oracle()


@pytest.fixture(scope="session")
def hip_lib():
    """libglint_attn.so, built only if absent (tests never fall back to anything else)."""
    from glint_amd import _lib, build

    if not build.HIP_LIB.exists():
        build.build_hip()
    return _lib.lib()


@pytest.fixture(scope="session")
def backend(hip_lib):
    from glint_amd.attn import GpuBackend

    be = GpuBackend(0)
    yield be
    be.close()
