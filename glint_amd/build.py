"""Build recipe for the gfx950 attention library and its host helpers.

    python -m glint_amd.build            # everything
    python -m glint_amd.build --hip      # libglint_attn.so only

Outputs (in-tree, git-ignored, shipped with the tree to the GPU box):
    glint_amd/libglint_attn.so    HIP kernels + C ABI (include/glint_attn.h)
    glint_amd/libglint_synth.so   seeded synthetic inputs (host C)
    glint_amd/libglint_probe.so   achievable-peak probes for bench.py (stream read, MFMA loops)
    glint_amd/libglint_host.so    C++ host layer over the C ABI (glint_amd/host/glint.hpp)
    glint_amd/_build/test_host    its test program (tests/cpp/test_host.cpp; run by tests/test_host_cpp.py)
    oracle/liboracle.so           CPU oracle, built by oracle/Makefile (tests only)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
HIP_LIB = PKG / "libglint_attn.so"
SYNTH_LIB = PKG / "libglint_synth.so"
PROBE_LIB = PKG / "libglint_probe.so"
HOST_LIB = PKG / "libglint_host.so"
HOST_TEST = BUILD / "test_host"
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "liboracle.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in the device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the decode kernel rescales them on the VALU,
    # which otherwise costs an AGPR->VGPR->AGPR round trip per step
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{ROOT / 'include'}",
]
HIP_SOURCES = ["gla_capi.hip", "gla_kvstore.hip", "gla_decode.hip", "gla_decode_q8.hip", "gla_prefill.hip",
               "gla_ops.hip"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build_hip(jobs: int = 4) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_probe() -> Path:
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", str(tmp), str(CSRC / "gla_probe.hip")])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


HOST_FLAGS = ["-O2", "-std=c++17", "-Wall", "-Wextra", "-fPIC", f"-I{ROOT / 'include'}", f"-I{PKG / 'host'}"]


def build_host() -> Path:
    """The C++ host layer (links libglint_attn.so, found next to it at run time)."""
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run(["g++", *HOST_FLAGS, "-shared", "-o", str(tmp), str(PKG / "host" / "glint.cpp"), f"-L{PKG}",
          "-lglint_attn", "-Wl,-rpath,$ORIGIN", "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build_host_tests() -> Path:
    BUILD.mkdir(exist_ok=True)
    tmp = HOST_TEST.with_suffix(".tmp")
    _run(["g++", *HOST_FLAGS, f"-I{ROOT / 'tests' / 'cpp'}", "-o", str(tmp), str(ROOT / "tests" / "cpp" / "test_host.cpp"),
          f"-L{PKG}", "-lglint_host", "-lglint_attn", "-Wl,-rpath,$ORIGIN/..", "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, HOST_TEST)
    return HOST_TEST


def build_synth() -> Path:
    tmp = SYNTH_LIB.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-o", str(tmp), str(CSRC / "synth.c"),
          "-lm", "-pthread"])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


def build_oracle() -> Path:
    _run(["make", "-s", "-B", "-C", str(ORACLE_DIR)])
    return ORACLE_LIB


def build_all(jobs: int = 4) -> None:
    build_synth()
    build_oracle()
    build_hip(jobs)
    build_probe()
    build_host()
    build_host_tests()


if __name__ == "__main__":
    args = set(sys.argv[1:])
    if "--hip" in args:
        build_hip()
    elif "--cpp" in args:
        build_host()
        build_host_tests()
    elif "--host" in args:
        build_synth()
        build_oracle()
    else:
        build_all()
    print("built:", ", ".join(str(p.relative_to(ROOT)) for p in (HIP_LIB, SYNTH_LIB, PROBE_LIB, HOST_LIB,
                                                                      HOST_TEST, ORACLE_LIB)
                               if p.exists()))
