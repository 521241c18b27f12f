"""Decode attention on the GPU through the C ABI, checked against the CPU oracle.

fp32 bar: max abs 1e-4 / rel 1e-3 per element (helpers.ABS_TOL / REL_TOL).
Page-table and mask indexing: bit-exact (test_indexing_is_bit_exact).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from gpu_util import Contig, Pool, run_decode
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _oracle_decode(stores, q, kv_start, kv_len, H, Hkv, d, scale, softcap=None, layer=0):
    B = q.shape[0]
    return orc.decode_batch(q.reshape(B, H * d), stores, layer, kv_start, kv_len, H, Hkv, d, scale,
                            softcap).reshape(B, H, d)


def test_cfg1_smollm_decode(backend):
    """H9/KV3, d64, B1, contiguous f32 ctx 512, query at 511, scale 1/8."""
    H, Hkv, d, ctx = 9, 3, 64, 512
    c = Contig(backend, "f32", 1, 1, ctx, Hkv, d, seed=101)
    q = synth.normal(202, (1, H, d))
    want = _oracle_decode(c.stores, q, [0], [ctx], H, Hkv, d, 0.125)
    got = run_decode(backend, c.cache, q, [0], [ctx], H, 0.125)
    assert_close(got, want, what="cfg1 gla_decode")
    # GpuBackend::attention mirror: host K/V in Glint's [pos][kv_h][d] layout
    got2 = backend.attention(q[0].reshape(-1), c.k[0, 0], c.v[0, 0], H, Hkv, d, ctx, 0.125)
    assert_close(got2.reshape(H, d), want[0], what="cfg1 attention()")
    # GpuBackend::attention_resident mirror over the device cache
    got3 = backend.attention_resident(q[0].reshape(-1), c.cache, 0, 0, ctx, H, Hkv, d, 0.125)
    assert_close(got3.reshape(H, d), want[0], what="cfg1 attention_resident()")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("d,H,Hkv", [(64, 9, 3), (64, 14, 2), (64, 8, 8), (128, 32, 8), (128, 8, 4),
                                     (128, 6, 2), (256, 16, 8), (256, 4, 1)])
def test_contiguous_batch(backend, dtype, d, H, Hkv):
    """Ragged lengths and windows over a batch of contiguous caches (incl. GQA 1..8, MQA)."""
    B, max_seq = 6, 700
    c = Contig(backend, dtype, B, 2, max_seq, Hkv, d, seed=300 + d + H)
    q = synth.normal(400 + d, (B, H, d))
    kv_start = np.array([0, 0, 5, 16, 100, 37], np.int32)
    kv_len = np.array([1, 15, 16, 17, 600, 663], np.int32)
    for layer in (0, 1):
        for cap in (None, 30.0):
            want = _oracle_decode(c.stores, q, kv_start, kv_len, H, Hkv, d, 1 / np.sqrt(d), cap, layer)
            got = run_decode(backend, c.cache, q, kv_start, kv_len, H, 1 / np.sqrt(d), cap, layer=layer)
            assert_close(got, want, what=f"{dtype} d{d} H{H}/{Hkv} layer{layer} cap{cap}")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_paged_shared_prefix_windows(backend, dtype):
    """Pool with a permuted page table, a 64-token shared prefix, windows that start mid-page."""
    H, Hkv, d = 16, 4, 128
    ctx = np.array([1, 20, 64, 65, 200, 513, 1000, 77], np.int32)
    pb = synth.paged_batch(55, ctx, prefix_tokens=64)
    p = Pool(backend, dtype, pb, Hkv, d, seed=66)
    q = synth.normal(77, (len(ctx), H, d))
    for window in (None, 50, 300):
        w = synth.windowed(pb, window)
        for cap in (None, 20.0):
            want = _oracle_decode(p.stores, q, w.kv_start, w.kv_len, H, Hkv, d, 0.088, cap)
            got = run_decode(backend, p.pool, q, w.kv_start, w.kv_len, H, 0.088, cap, table=pb.table)
            assert_close(got, want, what=f"paged {dtype} window {window} cap {cap}")


def test_seq_slot_selects_cache(backend):
    """Batch rows may read any cache sequence (the engine's slot -> cache map)."""
    H, Hkv, d = 8, 2, 64
    c = Contig(backend, "f32", 4, 1, 100, Hkv, d, seed=5)
    q = synth.normal(6, (3, H, d))
    slots = [3, 0, 3]
    want = _oracle_decode([c.stores[s] for s in slots], q, [0, 10, 50], [100, 90, 20], H, Hkv, d, 0.125)
    got = run_decode(backend, c.cache, q, [0, 10, 50], [100, 90, 20], H, 0.125, seq_slot=slots)
    assert_close(got, want, what="seq_slot")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_empty_window_gives_zero(backend, dtype):
    H, Hkv, d = 4, 1, 64
    c = Contig(backend, dtype, 2, 1, 64, Hkv, d, seed=9)
    q = synth.normal(10, (2, H, d))
    got = run_decode(backend, c.cache, q, [0, 5], [0, 3], H, 0.125)
    assert not got[0].any()
    want = _oracle_decode(c.stores, q, [0, 5], [0, 3], H, Hkv, d, 0.125)
    assert_close(got, want)


@pytest.mark.parametrize("host_lengths", [True, False])
@pytest.mark.parametrize("chunk", [None, "2", "16", "64"])
def test_q8_chunk_sizes(backend, monkeypatch, chunk, host_lengths):
    """Q8_0 decode with the default chunk size (sized from the host copies of the lengths, or
    from max_kv_len without them) and forced ones (GLA_Q8_CHUNK_PAGES): 2-page chunks (many
    partials per unit), 64-page chunks (the largest a wave holds). More than 64 sequences,
    empty windows, single-page and single-position sequences, windows starting mid-page."""
    if chunk is None:
        monkeypatch.delenv("GLA_Q8_CHUNK_PAGES", raising=False)
    else:
        monkeypatch.setenv("GLA_Q8_CHUNK_PAGES", chunk)
    H, Hkv, d = 8, 4, 64
    ctx = synth.uniform_int(811, 1, 1500, 150)
    ctx[[0, 7, 64, 65, 149]] = [0, 1, 16, 0, 2049]
    pb = synth.paged_batch(812, ctx, prefix_tokens=48)
    p = Pool(backend, "q8", pb, Hkv, d, seed=813)
    q = synth.normal(814, (len(ctx), H, d))
    w = synth.windowed(pb, 700)
    want = _oracle_decode(p.stores, q, w.kv_start, w.kv_len, H, Hkv, d, 0.125)
    got = run_decode(backend, p.pool, q, w.kv_start, w.kv_len, H, 0.125, table=pb.table,
                     host_lengths=host_lengths)
    assert not got[0].any() and not got[65].any()
    assert_close(got, want, what=f"q8 chunk {chunk}")


@pytest.mark.parametrize("host_lengths", [True, False])
def test_q8_context_beyond_64_chunks(backend, monkeypatch, host_lengths):
    """A 70,000-token window (4,376 pages, more than 64 chunks of 64 pages): chunks stay at
    most 64 pages, one page id per lane, with more workgroups per sequence instead. A
    short sequence beside it keeps the launch ragged."""
    monkeypatch.delenv("GLA_Q8_CHUNK_PAGES", raising=False)
    H, Hkv, d = 8, 2, 64
    ctx = np.array([70000, 300], np.int32)
    pb = synth.paged_batch(821, ctx)
    p = Pool(backend, "q8", pb, Hkv, d, seed=822)
    q = synth.normal(823, (len(ctx), H, d))
    want = _oracle_decode(p.stores, q, pb.kv_start, pb.kv_len, H, Hkv, d, 0.125)
    got = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.125, table=pb.table,
                     host_lengths=host_lengths)
    assert_close(got, want, what="q8 70k context")


def test_q8_host_lengths_shorter_than_device(backend, monkeypatch):
    """Host copies of the lengths that understate the device arrays break the gla_decode_args
    contract: the launch is sized from them, so the result is not the attention over the device
    windows, but every partial stays inside the slots sized for the launch (finite output, no
    error); with matching copies the same call is exact."""
    monkeypatch.setenv("GLA_Q8_CHUNK_PAGES", "2")  # many partials per unit
    H, Hkv, d = 8, 2, 64
    ctx = np.array([900, 40, 333], np.int32)
    pb = synth.paged_batch(831, ctx)
    p = Pool(backend, "q8", pb, Hkv, d, seed=832)
    q = synth.normal(833, (len(ctx), H, d))
    B = len(ctx)
    dq, dout = backend.buffer(np.ascontiguousarray(q)), backend.empty(q.nbytes)
    ds, dl = backend.buffer(pb.kv_start), backend.buffer(pb.kv_len)
    table = backend.buffer(np.ascontiguousarray(pb.table))
    short = np.minimum(pb.kv_len, 100).astype(np.int32)
    backend.decode(p.pool, dq, dout, ds, dl, B, int(pb.kv_len.max()), H, 0.125, None, page_table=table,
                   page_table_stride=pb.table.shape[1], kv_start_host=pb.kv_start, kv_len_host=short)
    backend.sync()
    assert np.all(np.isfinite(dout.download(q.shape)))
    want = _oracle_decode(p.stores, q, pb.kv_start, pb.kv_len, H, Hkv, d, 0.125)
    got = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.125, table=pb.table)
    assert_close(got, want, what="matching host lengths")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("paged", [False, True])
def test_indexing_is_bit_exact(backend, dtype, paged):
    """K = 0 gives equal weights, so out = mean of V over exactly the attended positions.
    V holds small integers (exact in f32 and in Q8_0 with scale 1), so every partial sum is
    exact and the only rounding is sum * (1/L): any wrong page, slot, head, element or window
    bound changes the bits."""
    H, Hkv, d = 8, 2, 128
    kv_dim = Hkv * d
    ctx = np.array([3, 16, 17, 250, 1029, 64, 33], np.int32)
    B = len(ctx)
    if paged:
        pb = synth.paged_batch(12, ctx, prefix_tokens=32)
        n_rows = pb.n_pages * 16
    else:
        max_seq = int(ctx.max())
        n_rows = B * max_seq
    # V[row][e] = integer in [-127, 127] that encodes (row, e); every 32-block holds a +-127
    r = np.arange(n_rows)[:, None]
    e = np.arange(kv_dim)[None, :]
    v = (((r * 131 + e * 7) % 255) - 127).astype(np.float32)
    v[:, ::32] = 127.0
    k = np.zeros_like(v)
    if paged:
        p = Pool(backend, dtype, pb, Hkv, d, k=k, v=v)
        kv, table = p.pool, pb.table
        v_of = lambda b, pos: v[pb.table[b, pos // 16] * 16 + pos % 16]
    else:
        c = Contig(backend, dtype, B, 1, max_seq, Hkv, d, k=k.reshape(B, 1, max_seq, kv_dim),
                   v=v.reshape(B, 1, max_seq, kv_dim))
        kv, table = c.cache, None
        v_of = lambda b, pos: v[b * max_seq + pos]
    q = synth.normal(3, (B, H, d))
    for window in (None, 15, 100):
        kv_start = np.array([0 if not window else max(0, n - window) for n in ctx], np.int32)
        kv_len = ctx - kv_start
        got = run_decode(backend, kv, q, kv_start, kv_len, H, 0.125, table=table)
        for b in range(B):
            rows = np.stack([v_of(b, pos) for pos in range(kv_start[b], ctx[b])]).astype(np.float64)
            s = rows.sum(0).astype(np.float32)  # exact: |sum| < 2^24
            want = s * (np.float32(1.0) / np.float32(kv_len[b]))
            for h in range(H):
                kvh = h // (H // Hkv)
                assert np.array_equal(got[b, h].view(np.uint32), want[kvh * d:(kvh + 1) * d].view(np.uint32)), \
                    (dtype, paged, window, b, h)


def test_quantize_on_write_is_bit_exact(backend):
    """Device Q8_0 rows exported in Glint's block format equal KvCacheQ8::quantize_into bytes."""
    Hkv, d = 4, 64
    kv_dim = Hkv * d
    n = 512
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((n, kv_dim)) * 10.0 ** rng.integers(-3, 3, (n, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :32] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5] + [0.0] * 25
    x[2, 5] = np.nan
    x[3, :] = 1e-30
    y = x[::-1].copy()
    pool = backend.create_page_pool(n // 16, Hkv, d, "q8")
    rows = np.arange(n, dtype=np.int64)[::-1].copy()
    pool.write_rows(rows, x, y)
    kb, vb = pool.export_rows(rows)
    assert np.array_equal(kb, orc.q8_quantize_rows(x))
    assert np.array_equal(vb, orc.q8_quantize_rows(y))


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_export_import_copy_zero(backend, dtype):
    """export_raw/import_raw bytes (snapshots), copy-on-write and recycle wipe of pages."""
    Hkv, d = 2, 64
    kv_dim = Hkv * d
    pool = backend.create_page_pool(8, Hkv, d, dtype)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, kv_dim)).astype(np.float32)
    y = rng.standard_normal((32, kv_dim)).astype(np.float32)
    rows = np.arange(16, 48, dtype=np.int64)  # pages 1 and 2
    pool.write_rows(rows, x, y)
    kb, vb = pool.export_rows(rows)
    if dtype == "f32":
        assert np.array_equal(kb.view(np.float32).reshape(32, kv_dim), x)
    else:
        assert np.array_equal(kb, orc.q8_quantize_rows(x))
    # import into page 5 and read back the same bytes
    rows5 = np.arange(80, 96, dtype=np.int64)
    pool.import_rows(rows5, kb[:16], vb[:16])
    k5, v5 = pool.export_rows(rows5)
    assert np.array_equal(k5, kb[:16]) and np.array_equal(v5, vb[:16])
    # copy page 2 -> 6, then wipe page 2
    pool.copy_page(2, 6)
    k6, v6 = pool.export_rows(np.arange(96, 112))
    assert np.array_equal(k6, kb[16:]) and np.array_equal(v6, vb[16:])
    pool.zero_page(2)
    backend.sync()
    k2, _ = pool.export_rows(np.arange(32, 48))
    if dtype == "f32":
        assert not k2.any()
    else:
        assert not k2.reshape(16, -1, 34)[:, :, 2:].any()


def test_cfg2_llama_decode_two_layers(backend):
    """BASELINE config 2 shape: H32/KV8, d128, contiguous f32 ctx 4096 (2 of the 32 layers)."""
    H, Hkv, d, ctx = 32, 8, 128, 4096
    c = Contig(backend, "f32", 1, 2, ctx, Hkv, d, seed=21)
    for layer in (0, 1):
        q = synth.normal(30 + layer, (1, H, d))
        want = _oracle_decode(c.stores, q, [0], [ctx], H, Hkv, d, 1 / np.sqrt(128), layer=layer)
        got = run_decode(backend, c.cache, q, [0], [ctx], H, 1 / np.sqrt(128), layer=layer)
        assert_close(got, want, what=f"cfg2 layer {layer}")


def test_cfg3_paged_q8_batch64_full(backend):
    """BASELINE config 3 at full size: B=64, ctx U[128, 8192], 16-token pages, permuted pool,
    256-token shared prefix, Q8_0 K/V; every sequence against the oracle."""
    H, Hkv, d = 32, 8, 128
    ctx = synth.uniform_int(3003, 128, 8192, 64)
    pb = synth.paged_batch(3004, ctx, prefix_tokens=256)
    p = Pool(backend, "q8", pb, Hkv, d, seed=3005)
    q = synth.normal(3006, (64, H, d))
    want = _oracle_decode(p.stores, q, pb.kv_start, pb.kv_len, H, Hkv, d, 1 / np.sqrt(128))
    got = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 1 / np.sqrt(128), table=pb.table)
    assert_close(got, want, what="cfg3")


def test_cfg5_gemma2_windowed_and_global(backend):
    """H16/KV8, d256, soft-cap 50, window 4096 on even layers, global on odd
    layers, B=32, ctx U[2048, 8192], paged Q8_0, K x 3."""
    H, Hkv, d = 16, 8, 256
    ctx = synth.uniform_int(5005, 2048, 8192, 32)
    pb = synth.paged_batch(5006, ctx)
    p = Pool(backend, "q8", pb, Hkv, d, seed=5007, k_mul=3.0)
    for layer in (0, 1):
        ws = np.array([orc.window_start(int(n) - 1, 4096, True, layer) for n in ctx], np.int32)
        kl = (ctx - ws).astype(np.int32)
        q = synth.normal(5008 + layer, (32, H, d))
        want = _oracle_decode(p.stores, q, ws, kl, H, Hkv, d, 1 / 16.0, 50.0)
        got = run_decode(backend, p.pool, q, ws, kl, H, 1 / 16.0, 50.0, table=pb.table)
        assert_close(got, want, what=f"cfg5 layer {layer}")


def test_q8_host_lengths_beyond_the_row_list(backend, monkeypatch):
    """Host lengths whose workgroups overflow the kernel-argument row list (1,536 entries: here
    2-page chunks, 8 pages per workgroup, 120 sequences of ~2,000 positions): the launch falls
    back to the (unit, workgroup, sequence) grid sized from the host lengths. Same bits as
    without host lengths, and the oracle's values."""
    monkeypatch.setenv("GLA_Q8_CHUNK_PAGES", "2")
    H, Hkv, d = 8, 2, 64
    ctx = synth.uniform_int(831, 1500, 2500, 120)
    pb = synth.paged_batch(832, ctx, prefix_tokens=32)
    p = Pool(backend, "q8", pb, Hkv, d, seed=833)
    q = synth.normal(834, (len(ctx), H, d))
    assert sum(-(-int(n) // 128) for n in ctx) > 1536
    want = _oracle_decode(p.stores, q, pb.kv_start, pb.kv_len, H, Hkv, d, 0.125)
    a = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.125, table=pb.table, host_lengths=True)
    b = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.125, table=pb.table, host_lengths=False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert_close(a, want, what="q8 host lengths past the row list")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_host_lengths_outside_the_storage_are_refused(backend, dtype):
    """The reference panics on a window outside the storage (src/cache/paged.rs:453-465,
    src/cache/mod.rs:167-171). With the host copies of the lengths, gla_decode refuses such a
    window on the host (GLA_ERR_INVALID) before anything runs; the out buffer is untouched and the
    next call works."""
    from glint_amd._lib import GLA_ERR_INVALID, GlaError
    H, Hkv, d = 8, 2, 64
    ctx = np.array([100, 40, 333], np.int32)
    pb = synth.paged_batch(851, ctx)
    p = Pool(backend, dtype, pb, Hkv, d, seed=852)
    q = synth.normal(853, (len(ctx), H, d))
    limit = pb.table.shape[1] * 16  # positions a row of the page table covers
    dq, dout = backend.buffer(np.ascontiguousarray(q)), backend.buffer(np.full(q.shape, 7.0, np.float32))
    table = backend.buffer(np.ascontiguousarray(pb.table))
    bad = [
        (np.array([0, 0, limit - 10], np.int32), np.array([100, 40, 11], np.int32), limit),  # past the end
        (np.array([0, -1, 0], np.int32), np.array([100, 40, 333], np.int32), 333),           # negative start
        (np.array([0, 0, 0], np.int32), np.array([100, -3, 333], np.int32), 333),            # negative length
        (np.array([0, 0, 0], np.int32), np.array([100, 40, 333], np.int32), 300),            # > max_kv_len
    ]
    for st, ln, max_len in bad:
        ds, dl = backend.buffer(st), backend.buffer(ln)
        with pytest.raises(GlaError) as ei:
            backend.decode(p.pool, dq, dout, ds, dl, len(ctx), max_len, H, 0.125, None, page_table=table,
                           page_table_stride=pb.table.shape[1], kv_start_host=st, kv_len_host=ln)
        assert ei.value.code == GLA_ERR_INVALID and "outside" in str(ei.value)
    backend.sync()
    assert np.all(dout.download(q.shape) == 7.0)  # nothing ran
    want = _oracle_decode(p.stores, q, pb.kv_start, pb.kv_len, H, Hkv, d, 0.125)
    got = run_decode(backend, p.pool, q, pb.kv_start, pb.kv_len, H, 0.125, table=pb.table)
    assert_close(got, want, what=f"{dtype} after the refusals")
