"""Writes the golden fixtures of tests/golden/cases.py from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture <case>.npz holds the oracle's output ("out", float32) and the
SHA-256 of the case's seeded inputs ("inputs_sha256"); q8_codec.npz holds
the Glint-format Q8_0 bytes of cases.q8_codec_rows(). Run it only when a case
is added or deliberately changed; tests/test_golden.py checks that the oracle
still reproduces every fixture bit for bit.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (str(ROOT), str(ROOT / "oracle"), str(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

import cases  # noqa: E402
import oracle as orc  # noqa: E402


def main() -> None:
    for name, make in cases.DECODE_CASES.items():
        c = make()
        np.savez_compressed(HERE / f"{name}.npz", out=cases.oracle_decode(c),
                            inputs_sha256=np.array(cases.digest(c.inputs)))
        print("wrote", name)
    for name, make in cases.PREFILL_CASES.items():
        c = make()
        np.savez_compressed(HERE / f"{name}.npz", out=cases.oracle_prefill(c),
                            inputs_sha256=np.array(cases.digest(c.inputs)))
        print("wrote", name)
    for name, make in cases.OPS_CASES.items():
        c = make()
        np.savez_compressed(HERE / f"{name}.npz", out=cases.oracle_ops(c),
                            inputs_sha256=np.array(cases.digest(c.inputs)))
        print("wrote", name)
    x = cases.q8_codec_rows()
    np.savez_compressed(HERE / "q8_codec.npz", bytes=orc.q8_quantize_rows(x),
                        inputs_sha256=np.array(cases.digest([x])))
    print("wrote q8_codec")


if __name__ == "__main__":
    main()
