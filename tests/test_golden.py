"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: every case's seeded inputs still hash to the recorded SHA-256, and the
oracle still reproduces the stored output bit for bit (a regression pin on the
oracle and on the input generator).
GPU: the kernels, through the C ABI, match the stored outputs at the fp32 bar
(max abs 1e-4 / rel 1e-3; the ops at their own bars, stated in their test);
the Q8_0 bytes written on the device equal the stored Glint-format bytes
exactly.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import cases  # noqa: E402
import oracle as orc  # noqa: E402
from gpu_util import Contig, Pool, run_decode, run_prefill  # noqa: E402
from helpers import assert_close  # noqa: E402


def _fixture(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", list(cases.DECODE_CASES))
def test_decode_fixture_oracle(name):
    c = cases.DECODE_CASES[name]()
    fx = _fixture(name)
    assert cases.digest(c.inputs) == str(fx["inputs_sha256"]), "input generator changed"
    assert np.array_equal(cases.oracle_decode(c).view(np.uint32), fx["out"].view(np.uint32))


@pytest.mark.parametrize("name", list(cases.PREFILL_CASES))
def test_prefill_fixture_oracle(name):
    c = cases.PREFILL_CASES[name]()
    fx = _fixture(name)
    assert cases.digest(c.inputs) == str(fx["inputs_sha256"]), "input generator changed"
    assert np.array_equal(cases.oracle_prefill(c).view(np.uint32), fx["out"].view(np.uint32))


@pytest.mark.parametrize("name", list(cases.OPS_CASES))
def test_ops_fixture_oracle(name):
    c = cases.OPS_CASES[name]()
    fx = _fixture(name)
    assert cases.digest(c.inputs) == str(fx["inputs_sha256"]), "input generator changed"
    assert np.array_equal(cases.oracle_ops(c).view(np.uint32), fx["out"].view(np.uint32))


def test_q8_codec_fixture_oracle():
    x = cases.q8_codec_rows()
    fx = _fixture("q8_codec")
    assert cases.digest([x]) == str(fx["inputs_sha256"])
    assert np.array_equal(orc.q8_quantize_rows(x), fx["bytes"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(cases.DECODE_CASES))
def test_decode_fixture_gpu(backend, name):
    c = cases.DECODE_CASES[name]()
    want = _fixture(name)["out"]
    B = c.q.shape[0]
    if c.paged:
        p = Pool(backend, c.kind, c.pb, c.Hkv, c.d, k=c.k, v=c.v)
        got = run_decode(backend, p.pool, c.q, c.kv_start, c.kv_len, c.H, c.scale, c.softcap, table=c.table)
    else:
        S = c.k.shape[1]
        ct = Contig(backend, c.kind, B, 1, S, c.Hkv, c.d, k=c.k.reshape(B, 1, S, -1), v=c.v.reshape(B, 1, S, -1))
        got = run_decode(backend, ct.cache, c.q, c.kv_start, c.kv_len, c.H, c.scale, c.softcap)
    assert_close(got, want, what=name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(cases.PREFILL_CASES))
def test_prefill_fixture_gpu(backend, name):
    c = cases.PREFILL_CASES[name]()
    want = _fixture(name)["out"]
    B, S = c.k.shape[0], c.k.shape[1]
    ct = Contig(backend, c.kind, B, 1, S, c.Hkv, c.d, k=c.k.reshape(B, 1, S, -1), v=c.v.reshape(B, 1, S, -1))
    got = run_prefill(backend, ct.cache, c.q, c.q_start, c.pos_offset, c.H, c.scale, c.softcap, c.window)
    assert_close(got, want, what=name)


@pytest.mark.gpu
def test_q8_codec_fixture_gpu(backend):
    x = cases.q8_codec_rows()
    want = _fixture("q8_codec")["bytes"]
    n, kv_dim = x.shape
    pool = backend.create_page_pool((n + 15) // 16, kv_dim // 64, 64, "q8")
    rows = np.arange(n, dtype=np.int64)
    pool.write_rows(rows, x, x)
    kb, vb = pool.export_rows(rows)
    assert np.array_equal(kb, want) and np.array_equal(vb, want)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(cases.OPS_CASES))
def test_ops_fixture_gpu(backend, name):
    """RoPE within 1e-5 x max|x| (the angles match the reference's; cos/sin may differ in the
    last place); the matvec within 4e-6 x sum |w x| per output of the oracle's f32 sums (both
    sides' rounding, as tests/test_gpu_ops.py bounds it against the oracle)."""
    c = cases.OPS_CASES[name]()
    want = _fixture(name)["out"]
    if c.kind == "rope":
        dx = backend.buffer(np.ascontiguousarray(c.x, np.float32))
        backend.rope(dx, c.x.shape[0], c.x.shape[1], c.head_dim, backend.buffer(c.pos), c.base, c.scaling,
                     c.rot_dim)
        backend.sync()
        got = dx.download(c.x.shape)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(c.x).max()
        return
    w = backend.create_q8_weights(c.raw, c.rows, c.cols)
    dy = backend.empty(c.x.shape[0] * c.rows * 4)
    backend.matvec_q8_0(w, backend.buffer(c.x), c.x.shape[0], dy)
    backend.sync()
    got = dy.download((c.x.shape[0], c.rows))
    w.destroy()
    blk = c.raw.reshape(c.rows, c.cols // 32, 34)
    scale = blk[:, :, :2].copy().view(np.float16).astype(np.float64)
    wd = (blk[:, :, 2:].view(np.int8).astype(np.float64) * scale).reshape(c.rows, c.cols)
    mag = np.abs(c.x.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 4e-6 * mag)
