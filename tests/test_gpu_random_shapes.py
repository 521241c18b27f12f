"""A seeded sweep over shapes the hand-picked tests do not name: prefill (fp32 and bf16-input) and
decode against the oracle (src/transformer/forward.rs:927-958 prefill loop, :1468-1507 batched
decode, flash.rs:46-124 per head) with head_dim 64/128/256, GQA groups 1-8, empty and ragged
lengths, arbitrary chunk offsets and window starts, soft-cap and sliding window on or off, f32
and Q8_0 caches, contiguous and paged (permuted page tables with a shared prefix); and the Q8_0 matvec
(quantized.rs:247-346) over vector counts, row counts, widths and x alignments, and RoPE
(ops.rs:212-245) over head and rotary dimensions, bases, scalings and positions, and KV row
writes (cache/mod.rs:296-315) over shapes, scales and special values, and the host-pointer
attention entry points (backend/gpu.rs:266-397, :860-992). Every case
is drawn from its own fixed seed, so a failure names a reproducible
shape. Bars: fp32 abs 1e-4 / rel 1e-3; bf16-input prefill abs 3e-2 / rel 3e-2 against the fp32
oracle (helpers.py), and bit-identical to the per-workgroup bf16 path. GLA_TEST_SWEEP=k runs k
times as many cases of every family (the first ones are always the same; the default is 1)."""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from gpu_util import Contig, Pool, run_decode, run_prefill
from helpers import BF16_ABS_TOL, BF16_REL_TOL, assert_close

pytestmark = pytest.mark.gpu

SWEEP = max(1, int(os.environ.get("GLA_TEST_SWEEP", "1")))
N_PREFILL = 32 * SWEEP
N_DECODE = 32 * SWEEP
N_PAGED = 16 * SWEEP


def _prefill_case(i):
    rng = np.random.default_rng(91000 + i)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 3, 4, 8]))
    n_seqs = int(rng.integers(1, 4))
    lens = [int(x) for x in rng.integers(0, 261, n_seqs)]
    if sum(lens) == 0:
        lens[0] = int(rng.integers(1, 100))
    offs = [int(x) for x in rng.integers(0, 151, n_seqs)]
    window = None if rng.random() < 0.5 else int(rng.integers(1, 301))
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    dtype = str(rng.choice(["f32", "q8"]))
    precision = str(rng.choice(["f32", "bf16"]))
    # the bf16 bar is stated for unit-scale scores; the fp32 path also takes other scales
    scale = float(1.0 / np.sqrt(d)) * (1.0 if precision == "bf16" else float(rng.uniform(0.5, 2.0)))
    extra = int(rng.integers(0, 41))
    return dict(d=d, hkv=hkv, H=hkv * group, lens=lens, offs=offs, window=window, cap=cap, dtype=dtype,
                precision=precision, scale=scale, max_seq=max(o + n for o, n in zip(offs, lens)) + extra)


def _decode_case(i):
    rng = np.random.default_rng(92000 + i)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 9))
    total = [int(x) for x in rng.integers(1, 3001, B)]
    # a window start anywhere in the sequence (the length attended is what follows it); some
    # sequences attend nothing
    starts = [int(rng.integers(0, t)) if rng.random() < 0.5 else 0 for t in total]
    lens = [t - s for t, s in zip(total, starts)]
    if B > 1 and rng.random() < 0.3:
        lens[int(rng.integers(0, B))] = 0
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    dtype = str(rng.choice(["f32", "q8"]))
    scale = float(1.0 / np.sqrt(d)) * float(rng.uniform(0.5, 2.0))
    return dict(d=d, hkv=hkv, H=hkv * group, starts=starts, lens=lens, cap=cap, dtype=dtype, scale=scale,
                max_seq=max(total))


@pytest.mark.parametrize("case", range(N_PREFILL))
def test_prefill_random_shapes(backend, monkeypatch, case):
    c_ = _prefill_case(case)
    d, hkv, H = c_["d"], c_["hkv"], c_["H"]
    lens, offs = c_["lens"], c_["offs"]
    c = Contig(backend, c_["dtype"], len(lens), 1, c_["max_seq"], hkv, d, seed=93000 + case)
    q = synth.normal(94000 + case, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    monkeypatch.delenv("GLA_BF16_UNSTAGED", raising=False)
    got = run_prefill(backend, c.cache, q, q_start, offs, H, c_["scale"], c_["cap"], c_["window"],
                      precision=c_["precision"])
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if c_["precision"] == "bf16" else ()
    for b, n in enumerate(lens):
        if n == 0:
            continue
        rows = slice(q_start[b], q_start[b + 1])
        want = orc.prefill(q[rows].reshape(n, H * d), c.stores[b], 0, offs[b], H, hkv, d, c_["scale"], c_["cap"],
                           c_["window"]).reshape(n, H, d)
        assert_close(got[rows], want, *tol, what=f"case {case} {c_} seq {b}")
    if c_["precision"] == "bf16":
        monkeypatch.setenv("GLA_BF16_UNSTAGED", "1")
        unstaged = run_prefill(backend, c.cache, q, q_start, offs, H, c_["scale"], c_["cap"], c_["window"],
                               precision="bf16")
        assert np.array_equal(got.view(np.uint32), unstaged.view(np.uint32)), (case, c_)


@pytest.mark.parametrize("case", range(N_DECODE))
def test_decode_random_shapes(backend, case):
    c_ = _decode_case(case)
    d, hkv, H = c_["d"], c_["hkv"], c_["H"]
    starts = np.asarray(c_["starts"], np.int32)
    lens = np.asarray(c_["lens"], np.int32)
    B = len(lens)
    c = Contig(backend, c_["dtype"], B, 1, c_["max_seq"], hkv, d, seed=95000 + case)
    q = synth.normal(96000 + case, (B, H, d))
    want = orc.decode_batch(q.reshape(B, H * d), c.stores, 0, starts, lens, H, hkv, d, c_["scale"],
                            c_["cap"]).reshape(B, H, d)
    for host_lengths in (True, False):
        got = run_decode(backend, c.cache, q, starts, lens, H, c_["scale"], c_["cap"], host_lengths=host_lengths)
        assert_close(got, want, what=f"case {case} {c_} host lengths {host_lengths}")


def _paged_case(i):
    rng = np.random.default_rng(97000 + i)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 9))
    ctx = [int(x) for x in rng.integers(1, 2001, B)]
    prefix = int(rng.choice([0, 16, 64, 200]))
    window = None if rng.random() < 0.5 else int(rng.integers(1, 700))
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    dtype = str(rng.choice(["f32", "q8"]))
    scale = float(1.0 / np.sqrt(d)) * float(rng.uniform(0.5, 2.0))
    # prefill: each sequence prefills its last n positions (the first ones are "cached")
    n_new = [int(rng.integers(0, min(c, 200) + 1)) for c in ctx]
    precision = str(rng.choice(["f32", "bf16"]))
    return dict(d=d, hkv=hkv, H=hkv * group, ctx=ctx, prefix=prefix, window=window, cap=cap, dtype=dtype,
                scale=scale, n_new=n_new, precision=precision)


@pytest.mark.parametrize("case", range(N_PAGED))
def test_paged_random_shapes(backend, case):
    """Decode and chunked prefill over one paged pool: the sequences' tables share a prefix and
    map logical pages to a seeded permutation of physical ones."""
    c_ = _paged_case(case)
    d, hkv, H = c_["d"], c_["hkv"], c_["H"]
    ctx = np.asarray(c_["ctx"], np.int32)
    pb = synth.paged_batch(98000 + case, ctx, prefix_tokens=c_["prefix"])
    p = Pool(backend, c_["dtype"], pb, hkv, d, seed=99000 + case)
    B = len(ctx)
    # decode at position ctx - 1 over the window
    w = synth.windowed(pb, c_["window"])
    q = synth.normal(99500 + case, (B, H, d))
    want = orc.decode_batch(q.reshape(B, H * d), p.stores, 0, w.kv_start, w.kv_len, H, hkv, d, c_["scale"],
                            c_["cap"]).reshape(B, H, d)
    got = run_decode(backend, p.pool, q, w.kv_start, w.kv_len, H, c_["scale"], c_["cap"], table=pb.table)
    assert_close(got, want, what=f"case {case} {c_} decode")
    # chunked prefill of each sequence's last n_new positions
    n = np.asarray(c_["n_new"], np.int32)
    if n.sum() == 0:
        return
    scale = float(1.0 / np.sqrt(d)) if c_["precision"] == "bf16" else c_["scale"]
    offs = ctx - n
    qp = synth.normal(99700 + case, (int(n.sum()), H, d))
    q_start = np.concatenate([[0], np.cumsum(n)]).astype(np.int32)
    got = run_prefill(backend, p.pool, qp, q_start, offs, H, scale, c_["cap"], c_["window"], table=pb.table,
                      precision=c_["precision"])
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if c_["precision"] == "bf16" else ()
    for b in range(B):
        if n[b] == 0:
            continue
        rows = slice(q_start[b], q_start[b + 1])
        want = orc.prefill(qp[rows].reshape(int(n[b]), H * d), p.stores[b], 0, int(offs[b]), H, hkv, d, scale,
                           c_["cap"], c_["window"]).reshape(int(n[b]), H, d)
        assert_close(got[rows], want, *tol, what=f"case {case} {c_} prefill seq {b}")


N_MATVEC = 24 * SWEEP


def _matvec_case(i):
    rng = np.random.default_rng(99800 + i)
    rows = int(rng.integers(1, 701))
    cols = 32 * int(rng.integers(1, 601))     # past 16,384 the activation split reads each row twice
    n_vec = int(rng.integers(1, 5)) if rng.random() < 0.3 else int(rng.integers(5, 151))
    misaligned = bool(rng.random() < 0.5)       # x 4 bytes past a 16-byte boundary: scalar loads
    return dict(rows=rows, cols=cols, n_vec=n_vec, misaligned=misaligned)


class _At:
    """A device pointer `offset` bytes into a buffer (the matvec reads only `.ptr`)."""

    def __init__(self, buf, offset):
        import ctypes
        self.ptr = ctypes.c_void_p(buf.ptr.value + offset)


@pytest.mark.parametrize("case", range(N_MATVEC))
def test_matvec_random_shapes(backend, case):
    """Q8_0 matvec (src/tensor/quantized.rs:247-346, :587-610) over seeded shapes: the vector-ALU
    kernel for 1-4 vectors, the split-K MFMA kernel with 1-4 vector tiles per launch and several
    launches, row tails, odd block counts and x at any 4-byte alignment. Bar as in the ops tests:
    |got - f64| <= 2e-6 x sum_c |w x|, and the oracle within 4e-6 of the same sum."""
    c_ = _matvec_case(case)
    rows, cols, n_vec = c_["rows"], c_["cols"], c_["n_vec"]
    raw = orc.q8_quantize_rows(synth.normal_rows(99900 + case, rows, cols)).reshape(-1)
    x = synth.normal(99950 + case, (n_vec, cols))
    # the activation pieces take a scale per vector and K slice from the slice's largest |x|:
    # a few large entries in the first slice, and by case an all-zero stretch (a slice of
    # zeros) or a tail a million times smaller (its slices' scales 2^20 apart from the first's)
    x[:, : 1 + case % 5] *= 300.0
    if case % 3 == 0:
        x[:, cols // 2: cols // 2 + max(32, cols // 4)] = 0.0
    elif case % 3 == 1:
        x[:, cols // 2:] *= 1e-6
    w = backend.create_q8_weights(raw, rows, cols)
    pad = 1 if c_["misaligned"] else 0
    dx = backend.buffer(np.concatenate([np.zeros(pad, np.float32), x.reshape(-1)]))
    dy = backend.empty(n_vec * rows * 4)
    backend.matvec_q8_0(w, _At(dx, 4 * pad), n_vec, dy)
    backend.sync()
    got = dy.download((n_vec, rows))
    w.destroy()
    blk = raw.reshape(rows, cols // 32, 34)
    wd = (blk[:, :, 2:].view(np.int8).astype(np.float64) *
          blk[:, :, :2].copy().view("<f2").astype(np.float64)).reshape(rows, cols)
    exact = x.astype(np.float64) @ wd.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(got - exact) <= 2e-6 * mag), (case, c_, float(np.max(np.abs(got - exact) / mag)))
    for v in sorted({0, n_vec // 2, n_vec - 1}):
        want = orc.matvec_q8_0(raw, rows, cols, x[v])
        assert np.all(np.abs(got[v] - want) <= 4e-6 * mag[v]), (case, c_, v)


N_ROPE = 16 * SWEEP


@pytest.mark.parametrize("case", range(N_ROPE))
def test_rope_random_shapes(backend, case):
    """RoPE (src/tensor/ops.rs:212-245) over seeded head counts, head and rotary dimensions (odd
    ones included), bases, linear scalings and positions up to 2^20; the dimensions past the
    rotary part are left bit for bit. Bar: max abs 1e-5 x max|x| per row, as in the ops tests."""
    rng = np.random.default_rng(99600 + case)
    head_dim = int(rng.integers(1, 257))
    rot_dim = head_dim if rng.random() < 0.5 else int(rng.integers(0, head_dim + 1))
    n_heads = int(rng.integers(1, 41))
    n_rows = int(rng.integers(1, 65))
    base = float(rng.choice([10000.0, 500000.0, 1e6])) * float(rng.uniform(0.5, 2.0))
    scaling = float(rng.choice([1.0, 1.0, 2.0, 4.0, 8.0])) * float(rng.uniform(0.9, 1.1))
    pos = rng.integers(0, 1 << 20, n_rows).astype(np.int32)
    pos[0] = 0
    x = synth.normal(99700 + case, (n_rows, n_heads, head_dim))
    dx = backend.buffer(x)
    dp = backend.buffer(pos)
    backend.rope(dx, n_rows, n_heads, head_dim, dp, base, scaling, rot_dim)
    backend.sync()
    got = dx.download(x.shape)
    rot = min(rot_dim, head_dim) & ~1
    for r in range(n_rows):
        want = orc.rope(x[r].reshape(-1), int(pos[r]), head_dim, base, scaling, rot_dim).reshape(n_heads, head_dim)
        err = float(np.abs(got[r] - want).max())
        assert err <= 1e-5 * float(np.abs(x[r]).max()), (case, head_dim, rot_dim, int(pos[r]), err)
        assert np.array_equal(got[r][:, rot:], x[r][:, rot:]), (case, r)
    assert np.array_equal(got[0], x[0]), case   # position 0 is the identity


N_KV_WRITE = 16 * SWEEP


@pytest.mark.parametrize("case", range(N_KV_WRITE))
def test_kv_write_random_shapes(backend, case):
    """KV rows written to a page pool (KvCacheQ8::quantize_into, src/cache/mod.rs:296-315, for Q8_0;
    the f32 store's plain copy) through the host and the device entry points, over seeded KV head
    counts, head dims, row scales from 1e-12 to 1e7 (f16 block scales that flush to zero, go
    subnormal or overflow to inf), NaN and +-inf entries and exact .5 multiples of the scale,
    exported in the reference's row format and compared byte for byte with the oracle; then
    imported into other rows and exported again unchanged."""
    rng = np.random.default_rng(99400 + case)
    dtype = "q8" if case % 4 else "f32"
    hkv = int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128, 256]))
    kv_dim = hkv * d
    pages = int(rng.integers(4, 41))
    n = int(rng.integers(1, pages * 16 // 2 + 1))
    rows = rng.permutation(pages * 16)[: 2 * n].astype(np.int64)
    src, dst = rows[:n], rows[n:]
    x = (rng.standard_normal((2, n, kv_dim)) * 10.0 ** rng.uniform(-12, 7, (2, n, 1))).astype(np.float32)
    for t in range(2):
        for r in rng.choice(n, size=min(n, 6), replace=False):
            kind = int(rng.integers(0, 5))
            c = int(rng.integers(0, kv_dim))
            if kind == 0:
                x[t, r, c] = np.nan
            elif kind == 1:
                x[t, r, c] = np.inf if rng.random() < 0.5 else -np.inf
            elif kind == 2:
                x[t, r, (c // 32) * 32:(c // 32) * 32 + 32] = 0.0
            elif kind == 3:     # quants that land on .5 before rounding: 127 * (k + 0.5) / 127
                blk = slice((c // 32) * 32, (c // 32) * 32 + 32)
                x[t, r, blk] = (rng.integers(-127, 127, 32) + 0.5).astype(np.float32)
                x[t, r, (c // 32) * 32] = 127.0
            else:
                x[t, r, c] = -x[t, r, c] * 1e3
    k, v = x[0], x[1]
    pool = backend.create_page_pool(pages, hkv, d, dtype)
    half = n // 2
    pool.write_rows(src[:half], k[:half], v[:half])
    if n > half:
        pool.write_rows_device(backend.buffer(src[half:]), backend.buffer(k[half:]), backend.buffer(v[half:]), n - half)
    kb, vb = pool.export_rows(src)
    if dtype == "q8":
        assert np.array_equal(kb, orc.q8_quantize_rows(k)), case
        assert np.array_equal(vb, orc.q8_quantize_rows(v)), case
    else:
        assert np.array_equal(kb.view(np.uint32).reshape(n, kv_dim), k.view(np.uint32)), case
        assert np.array_equal(vb.view(np.uint32).reshape(n, kv_dim), v.view(np.uint32)), case
    pool.import_rows(dst, kb, vb)
    k2, v2 = pool.export_rows(dst)
    assert np.array_equal(k2, kb) and np.array_equal(v2, vb), case
    pool.destroy()


N_HOST_ATTN = 16 * SWEEP


@pytest.mark.parametrize("case", range(N_HOST_ATTN))
def test_host_attention_random_shapes(backend, case):
    """The host-pointer entry points over seeded shapes: GpuBackend::attention (host q and K/V,
    src/backend/gpu.rs:266-397) and attention_resident (host q over a device cache, a sequence
    slot, a layer and a window, gpu.rs:860-992), against the oracle's batched decode of the
    same rows at the fp32 bar."""
    rng = np.random.default_rng(99300 + case)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    H = hkv * int(rng.choice([1, 2, 3, 4, 8]))
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    scale = float(1.0 / np.sqrt(d)) * float(rng.uniform(0.5, 2.0))
    kv_dim = hkv * d
    # host K/V
    seq_len = int(rng.integers(1, 2501))
    k = synth.normal(99310 + case, (1, seq_len, kv_dim))
    v = synth.normal(99320 + case, (1, seq_len, kv_dim))
    q = synth.normal(99330 + case, (1, H * d))
    want = orc.decode_batch(q, [orc.kv_cache(k, v)], 0, [0], [seq_len], H, hkv, d, scale, cap)
    got = backend.attention(q[0], k[0], v[0], H, hkv, d, seq_len, scale, cap)
    assert_close(got.reshape(1, -1), want, what=f"case {case} attention d {d} H {H}/{hkv} len {seq_len}")
    # resident cache
    dtype = str(rng.choice(["f32", "q8"]))
    n_seqs = int(rng.integers(1, 4))
    max_seq = int(rng.integers(1, 2001))
    c = Contig(backend, dtype, n_seqs, 2, max_seq, hkv, d, seed=99340 + case)
    seq = int(rng.integers(0, n_seqs))
    layer = int(rng.integers(0, 2))
    start = int(rng.integers(0, max_seq))
    attend = int(rng.integers(1, max_seq - start + 1))
    want = orc.decode_batch(q, [c.stores[seq]], layer, [start], [attend], H, hkv, d, scale, cap)
    got = backend.attention_resident(q[0], c.cache, layer, start, attend, H, hkv, d, scale, cap, seq=seq)
    assert_close(got.reshape(1, -1), want,
                 what=f"case {case} resident {dtype} d {d} H {H}/{hkv} seq {seq} layer {layer} [{start}, +{attend})")


N_ODD_GROUPS = 12 * SWEEP


@pytest.mark.parametrize("case", range(N_ODD_GROUPS))
def test_decode_odd_groups_random(backend, case):
    """Decode with GQA groups that do not fill the kernels' 4-head wave groups (3, 5, 6, 7) or
    span several of them (12, 16), contiguous and paged, f32 and Q8_0, against the oracle."""
    rng = np.random.default_rng(99200 + case)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 3, 4]))
    group = int(rng.choice([3, 5, 6, 7, 12, 16]))
    H = hkv * group
    B = int(rng.integers(1, 7))
    ctx = np.asarray(rng.integers(1, 2501, B), np.int32)
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    dtype = str(rng.choice(["f32", "q8"]))
    scale = float(1.0 / np.sqrt(d)) * float(rng.uniform(0.5, 2.0))
    q = synth.normal(99210 + case, (B, H, d))
    if case % 2:
        pb = synth.paged_batch(99220 + case, ctx, prefix_tokens=int(rng.choice([0, 32])))
        p = Pool(backend, dtype, pb, hkv, d, seed=99230 + case)
        w = synth.windowed(pb, None)
        want = orc.decode_batch(q.reshape(B, H * d), p.stores, 0, w.kv_start, w.kv_len, H, hkv, d, scale, cap)
        got = run_decode(backend, p.pool, q, w.kv_start, w.kv_len, H, scale, cap, table=pb.table)
    else:
        c = Contig(backend, dtype, B, 1, int(ctx.max()), hkv, d, seed=99240 + case)
        starts = np.asarray([int(rng.integers(0, t)) for t in ctx], np.int32)
        lens = ctx - starts
        want = orc.decode_batch(q.reshape(B, H * d), c.stores, 0, starts, lens, H, hkv, d, scale, cap)
        got = run_decode(backend, c.cache, q, starts, lens, H, scale, cap)
    assert_close(got, want.reshape(B, H, d), what=f"case {case} d {d} H {H}/{hkv} {dtype} B {B}")


N_PREFILL_ODD = 10 * SWEEP


@pytest.mark.parametrize("case", range(N_PREFILL_ODD))
def test_prefill_odd_groups_random(backend, monkeypatch, case):
    """Prefill with GQA groups 5, 6, 7, 12 and 16 (the workgroup's heads-per-KV-head split
    part-filled or repeated), f32 and bf16-input, against the oracle; bf16 also bit-identical
    to the per-workgroup path."""
    rng = np.random.default_rng(99100 + case)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2]))
    H = hkv * int(rng.choice([5, 6, 7, 12, 16]))
    lens = [int(x) for x in rng.integers(1, 200, int(rng.integers(1, 3)))]
    offs = [int(x) for x in rng.integers(0, 100, len(lens))]
    window = None if rng.random() < 0.5 else int(rng.integers(1, 200))
    cap = None if rng.random() < 0.5 else float(rng.uniform(5.0, 60.0))
    dtype = str(rng.choice(["f32", "q8"]))
    precision = "bf16" if case % 2 else "f32"
    scale = float(1.0 / np.sqrt(d))
    c = Contig(backend, dtype, len(lens), 1, max(o + n for o, n in zip(offs, lens)), hkv, d, seed=99110 + case)
    q = synth.normal(99120 + case, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    monkeypatch.delenv("GLA_BF16_UNSTAGED", raising=False)
    got = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, precision=precision)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    for b, n in enumerate(lens):
        rows = slice(q_start[b], q_start[b + 1])
        want = orc.prefill(q[rows].reshape(n, H * d), c.stores[b], 0, offs[b], H, hkv, d, scale, cap,
                           window).reshape(n, H, d)
        assert_close(got[rows], want, *tol, what=f"case {case} d {d} H {H}/{hkv} {dtype} {precision} seq {b}")
    if precision == "bf16":
        monkeypatch.setenv("GLA_BF16_UNSTAGED", "1")
        unstaged = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, precision="bf16")
        assert np.array_equal(got.view(np.uint32), unstaged.view(np.uint32)), case
