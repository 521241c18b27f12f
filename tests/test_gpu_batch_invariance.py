"""A sequence decodes to the same bits alone as in any batch -- the reference's batched ==
single guarantee (`assert_same_logits` compares to_bits(), src/transformer/forward.rs:1946-1954;
checked at :1960-2002 and, for Q8_0, :2257-2308), on which its engine tests build (a paged
pool gives the same tokens, src/server/engine.rs:1095; a forked admission is bit-identical to a
cold one, :1836).

Every sequence of a cfg3-shaped batch (Llama-3-8B heads, B=64, ctx U[128, 8192], paged, 256-token
shared prefix) is decoded in the whole batch (with and without the host copies of the lengths,
which size the launch), in a shuffled sub-batch, and alone, for Q8_0 and f32 pools, global and
with a 4096-token window and soft-cap 50 (K x 3, so the cap bites). All outputs must be equal
bit for bit. Alone, the Q8_0 path spreads the q-heads of a KV head over more waves (the batch is
too small to fill the device otherwise), so this also checks that a head's result does not
depend on the heads that share its wave. For f32 the host-buffer entry point
(GpuBackend::attention, Glint's [pos][kv_head][d] layout) must give the same bits as well.
Prefill keeps the same property: a prompt gives the same bits alone, in a ragged batch and in a
shuffled sub-batch, on both the fp32 and the bf16-input paths.
"""
from __future__ import annotations

import numpy as np
import pytest

from glint_amd import synth
from gpu_util import run_decode, write_rows_chunked

pytestmark = pytest.mark.gpu

H, HKV, D, B = 32, 8, 128, 64
SCALE = float(1 / np.sqrt(D))


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def cfg3_batch():
    ctx = synth.uniform_int(3103, 128, 8192, B)
    pb = synth.paged_batch(3104, ctx, prefix_tokens=256)
    rows, k, v = synth.pool_rows(3105, 3106, 0, pb.n_pages, HKV * D, 3.0)
    q = synth.normal(3107, (B, H, D))
    return pb, rows, k, v, q


@pytest.mark.parametrize("dtype", ["q8", "f32"])
def test_decode_is_batch_invariant_cfg3(backend, cfg3_batch, dtype):
    pb, rows, k, v, q = cfg3_batch
    pool = backend.create_page_pool(pb.n_pages, HKV, D, dtype)
    write_rows_chunked(pool, rows, k, v)
    sub = np.random.default_rng(3108).permutation(B)[:24]
    try:
        for window, cap in ((None, None), (4096, 50.0)):
            w = synth.windowed(pb, window)
            what = f"{dtype} window {window} cap {cap}"
            full = run_decode(backend, pool, q, w.kv_start, w.kv_len, H, SCALE, cap, table=pb.table)
            assert np.isfinite(full).all(), what
            nohost = run_decode(backend, pool, q, w.kv_start, w.kv_len, H, SCALE, cap, table=pb.table,
                                host_lengths=False)
            assert np.array_equal(_bits(nohost), _bits(full)), f"{what}: launch sized without host lengths"
            part = run_decode(backend, pool, q[sub], w.kv_start[sub], w.kv_len[sub], H, SCALE, cap,
                              table=pb.table[sub])
            for i, b in enumerate(sub):
                assert np.array_equal(_bits(part[i]), _bits(full[b])), f"{what}: seq {b} in a shuffled sub-batch"
            for b in range(B):
                alone = run_decode(backend, pool, q[b:b + 1], w.kv_start[b:b + 1], w.kv_len[b:b + 1], H, SCALE,
                                   cap, table=pb.table[b:b + 1])
                assert np.array_equal(_bits(alone[0]), _bits(full[b])), f"{what}: seq {b} alone"
            if dtype == "f32" and window is None:
                for b in (int(np.argmax(pb.ctx)), int(np.argmin(pb.ctx))):
                    pos = np.arange(int(pb.ctx[b]))
                    r = pb.table[b, pos // 16].astype(np.int64) * 16 + pos % 16
                    got = backend.attention(q[b].reshape(-1), k[r], v[r], H, HKV, D, len(pos), SCALE, cap)
                    assert np.array_equal(_bits(got), _bits(full[b].reshape(-1))), f"attention() seq {b}"
    finally:
        pool.destroy()


@pytest.mark.parametrize("d,h,hkv,nb", [(64, 9, 3, 65), (128, 32, 8, 65)])
def test_f32_merge_switch_is_batch_invariant(backend, d, h, hkv, nb):
    """An f32 window of more than one split and at most nb = 65 pages (at these head shapes: 1
    or 2 merged elements per thread) merges its splits in the split kernel's last workgroup to
    arrive; longer ones in decode_combine_kernel. The choice is a rule on the window (and the model's head shape), so
    windows on both sides of it (nb and nb + 1 pages, from a page boundary and from mid-page,
    plus one-split windows) give the same bits alone, in a batch that mixes both merges, in a
    shuffled sub-batch and with the launch sized without host lengths; each matches the oracle,
    and the arrival counters are left ready for the next call (a second run repeats the bits)."""
    import oracle as orc
    from gpu_util import Contig
    from helpers import assert_close

    starts = np.array([0, 0, 0, 0, 0, 8, 8, 0, 5, 3], np.int32)
    lens = np.array([1, 16, 17, (nb - 1) * 16, nb * 16, nb * 16 - 8, nb * 16 - 7, (nb + 1) * 16, 2000, 130],
                    np.int32)
    B = len(lens)
    c = Contig(backend, "f32", B, 1, int((starts + lens).max()), hkv, d, seed=5150 + d)
    q = synth.normal(5151 + d, (B, h, d))
    scale = float(1 / np.sqrt(d))
    want = orc.decode_batch(q.reshape(B, h * d), c.stores, 0, starts, lens, h, hkv, d, scale,
                            None).reshape(B, h, d)
    full = run_decode(backend, c.cache, q, starts, lens, h, scale)
    assert_close(full, want, what=f"d{d} batch across the merge switch")
    again = run_decode(backend, c.cache, q, starts, lens, h, scale)
    assert np.array_equal(_bits(again), _bits(full)), "second call"
    nohost = run_decode(backend, c.cache, q, starts, lens, h, scale, host_lengths=False)
    assert np.array_equal(_bits(nohost), _bits(full)), "launch sized without host lengths"
    sub = np.random.default_rng(5152).permutation(B)[:6]
    part = run_decode(backend, c.cache, q[sub], starts[sub], lens[sub], h, scale, seq_slot=sub)
    for i, b in enumerate(sub):
        assert np.array_equal(_bits(part[i]), _bits(full[b])), f"seq {b} in a shuffled sub-batch"
    for b in range(B):
        alone = run_decode(backend, c.cache, q[b:b + 1], starts[b:b + 1], lens[b:b + 1], h, scale,
                           seq_slot=[b])
        assert np.array_equal(_bits(alone[0]), _bits(full[b])), f"seq {b} (start {starts[b]}, len {lens[b]}) alone"


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_prefill_is_batch_invariant(backend, dtype, precision):
    """A prompt's prefill gives the same bits alone as in a ragged batch of prompts (different
    lengths and position offsets, so the grid, the query-block count and the staged tile images
    are sized by other sequences), global and with a 48-token sliding window and soft-cap 30."""
    from gpu_util import Contig, run_prefill

    h, hkv, d = 8, 2, 64
    lens = np.array([70, 1, 129, 33], np.int32)
    offs = np.array([0, 200, 17, 300], np.int32)
    max_seq = 512
    c = Contig(backend, dtype, len(lens), 1, max_seq, hkv, d, seed=4101, k_mul=3.0)
    q = synth.normal(4102, (int(lens.sum()), h, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    for sw, cap in ((None, None), (48, 30.0)):
        whole = run_prefill(backend, c.cache, q, q_start, offs, h, 0.125, cap, sw, precision=precision)
        for b in range(len(lens)):
            rows = slice(int(q_start[b]), int(q_start[b + 1]))
            alone = run_prefill(backend, c.cache, q[rows], np.array([0, lens[b]], np.int32), offs[b:b + 1], h, 0.125,
                                cap, sw, precision=precision, seq_slot=np.array([b], np.int32))
            assert np.array_equal(_bits(alone), _bits(whole[rows])), (dtype, precision, sw, b)
        order = [2, 0, 3]  # a shuffled sub-batch
        sub_q = np.concatenate([q[int(q_start[b]):int(q_start[b + 1])] for b in order])
        sub_start = np.concatenate([[0], np.cumsum(lens[order])]).astype(np.int32)
        sub = run_prefill(backend, c.cache, sub_q, sub_start, offs[order], h, 0.125, cap, sw, precision=precision,
                          seq_slot=np.array(order, np.int32))
        for i, b in enumerate(order):
            assert np.array_equal(_bits(sub[int(sub_start[i]):int(sub_start[i + 1])]),
                                  _bits(whole[int(q_start[b]):int(q_start[b + 1])])), (dtype, precision, sw, "sub", b)


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_chunked_prefill_equals_one_pass(backend, precision):
    """A prompt prefilled in chunks (the second continuing at the first's end) gives the same
    bits as one pass: in the reference each query runs the same blocked softmax over keys
    0 .. its position whichever call it belongs to (src/transformer/forward.rs:927-958)."""
    from gpu_util import Contig, run_prefill

    h, hkv, d, n = 8, 2, 64, 150
    c = Contig(backend, "f32", 1, 1, 256, hkv, d, seed=4201)
    q = synth.normal(4202, (n, h, d))
    for sw in (None, 40):
        one = run_prefill(backend, c.cache, q, np.array([0, n], np.int32), np.array([0], np.int32), h, 0.125,
                          None, sw, precision=precision)
        for cut in (70, 97):
            a = run_prefill(backend, c.cache, q[:cut], np.array([0, cut], np.int32), np.array([0], np.int32), h,
                            0.125, None, sw, precision=precision)
            b = run_prefill(backend, c.cache, q[cut:], np.array([0, n - cut], np.int32), np.array([cut], np.int32), h,
                            0.125, None, sw, precision=precision)
            assert np.array_equal(_bits(np.concatenate([a, b])), _bits(one)), (precision, sw, cut)
