"""gla_decode_noalloc, the decode entry point that allocates nothing (its split partials live in
the library's static per-GPU scratch array), against gla_decode through the C ABI. Both run the
same kernels, so the outputs must be equal bit for bit. Two calls in a row, the second on a
smaller input (the array still holds the first call's partials), for Q8_0 (cfg3 shape, and a
Gemma-2 shape with soft-cap and window) and f32 (cfg2 shape) storage. A call whose partials would
exceed the array is refused before anything runs, and the entry point works again after it."""
from __future__ import annotations

import numpy as np
import pytest

from glint_amd import synth
from glint_amd._lib import GLA_DECODE_NOALLOC_SCRATCH_BYTES, GLA_ERR_INVALID, GlaError
from gpu_util import Contig, Pool

pytestmark = pytest.mark.gpu


def _both(be, kv, q, kv_start, kv_len, H, scale, cap=None, table=None, layer=0, host=True):
    """(gla_decode output, gla_decode_noalloc output) of one batch, as uint32 bits."""
    B = q.shape[0]
    dq = be.buffer(np.ascontiguousarray(q, np.float32))
    ds, dl = be.buffer(np.asarray(kv_start, np.int32)), be.buffer(np.asarray(kv_len, np.int32))
    kw = {}
    if table is not None:
        kw = dict(page_table=be.buffer(np.ascontiguousarray(table, np.int32)), page_table_stride=table.shape[1])
    if host:
        kw.update(kv_start_host=np.asarray(kv_start, np.int32), kv_len_host=np.asarray(kv_len, np.int32))
    outs = []
    for noalloc in (False, True):
        out = be.empty(q.nbytes)
        be.decode(kv, dq, out, ds, dl, B, int(np.max(kv_len)), H, scale, cap, layer=layer, noalloc=noalloc, **kw)
        be.sync()
        outs.append(out.download(q.shape).view(np.uint32))
    return outs


def test_noalloc_equals_decode_q8(backend):
    H, Hkv, d, B = 32, 8, 128, 64
    ctx = synth.uniform_int(9101, 128, 8192, B)
    pb = synth.paged_batch(9102, ctx, prefix_tokens=256)
    p = Pool(backend, "q8", pb, Hkv, d, seed=9103)
    q = synth.normal(9104, (B, H, d))
    ref, got = _both(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.088, table=pb.table)
    assert np.isfinite(ref.view(np.float32)).all()
    assert np.array_equal(ref, got), "cfg3 batch"
    # second call, smaller: 9 sequences, windowed, soft-capped, without host lengths
    sub = np.arange(3, 57, 6)
    w = synth.windowed(pb, 1000)
    ref, got = _both(backend, p.pool, q[sub], w.kv_start[sub], w.kv_len[sub], H, 0.088, 30.0,
                     table=pb.table[sub], host=False)
    assert np.array_equal(ref, got), "windowed sub-batch"


def test_noalloc_equals_decode_gemma_shape(backend):
    H, Hkv, d, B = 16, 8, 256, 32
    ctx = synth.uniform_int(9201, 2048, 8192, B)
    pb = synth.paged_batch(9202, ctx)
    p = Pool(backend, "q8", pb, Hkv, d, seed=9203, k_mul=3.0)
    w = synth.windowed(pb, 4096)
    q = synth.normal(9204, (B, H, d))
    for rows in (np.arange(B), np.arange(0, B, 5)):
        ref, got = _both(backend, p.pool, q[rows], w.kv_start[rows], w.kv_len[rows], H, 1 / 16.0, 50.0,
                         table=pb.table[rows])
        assert np.array_equal(ref, got), len(rows)


def test_noalloc_equals_decode_f32(backend):
    H, Hkv, d = 32, 8, 128
    c = Contig(backend, "f32", 1, 1, 4096, Hkv, d, seed=9301)
    for n, seed in ((4096, 9302), (700, 9303)):
        q = synth.normal(seed, (1, H, d))
        ref, got = _both(backend, c.cache, q, [0], [n], H, float(1 / np.sqrt(d)))
        assert np.array_equal(ref, got), n


def test_noalloc_equals_decode_f32_mixed_windows(backend):
    """A batch mixing f32 windows merged in the split kernel (up to 65 pages: the static arrival
    counters; here 300, 500 and 700 positions) with ones merged by the combine kernel (1050 and
    2000), then a smaller batch of both kinds: bit for bit."""
    H, Hkv, d = 32, 8, 128
    starts = np.array([0, 0, 5, 0, 0, 16, 3], np.int32)
    lens = np.array([1, 17, 300, 500, 1050, 2000, 700], np.int32)
    c = Contig(backend, "f32", len(lens), 1, int((starts + lens).max()), Hkv, d, seed=9311)
    for rows in (np.arange(len(lens)), np.array([1, 3, 5])):
        q = synth.normal(9312 + len(rows), (len(rows), H, d))
        ref, got = _both(backend, c.cache, q, starts[rows], lens[rows], H, float(1 / np.sqrt(d)))
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), len(rows)


PARTIAL_BYTES = GLA_DECODE_NOALLOC_SCRATCH_BYTES


@pytest.mark.parametrize("dtype,fits", [("q8", 192), ("f32", 29)])
def test_noalloc_capacity_per_storage(backend, dtype, fits):
    """The header's capacity at Llama-3-8B heads and 8,192 positions (no host lengths, so the
    launch is sized from max_kv_len): `fits` sequences run and equal gla_decode bit for bit;
    one more needs more partials than the array holds: GLA_ERR_INVALID, nothing launched; the
    next call works. (Every table entry names page 0 of a small pool: the sizing, not the
    data, is under test.)"""
    H, Hkv, d = 32, 8, 128
    pool = backend.create_page_pool(64, Hkv, d, dtype)
    pool.write_rows(np.arange(16, dtype=np.int64), synth.normal_rows(9401, 16, Hkv * d),
                    synth.normal_rows(9402, 16, Hkv * d))
    stride = 8192 // 16 + 1
    try:
        for B in (fits + 1, fits):
            table = np.zeros((B, stride), np.int32)
            starts, lens = np.zeros(B, np.int32), np.full(B, 8192, np.int32)
            q = synth.normal(9403, (B, H, d))
            if B > fits:
                with pytest.raises(GlaError) as ei:
                    _both(backend, pool, q, starts, lens, H, 0.088, table=table, host=False)
                assert ei.value.code == GLA_ERR_INVALID
                assert "scratch" in str(ei.value) and str(PARTIAL_BYTES) in str(ei.value)
            else:
                ref, got = _both(backend, pool, q, starts, lens, H, 0.088, table=table, host=False)
                assert np.array_equal(ref, got)
    finally:
        pool.destroy()
    test_noalloc_equals_decode_f32(backend)
