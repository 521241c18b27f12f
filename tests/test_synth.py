"""The seeded input generator: Glint's Xorshift64 (src/sampling/sampler.rs:56-69)
restated in Python, determinism, and the shapes of the paged workloads."""
import numpy as np

from glint_amd import synth


def xorshift64(seed, n):
    s = seed or 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        out.append(s)
    return out


def test_xorshift_sequence():
    for seed in (1, 42, 0xDEADBEEF, 0):
        assert list(synth.xorshift_seq(seed, 50)) == xorshift64(seed, 50)


def test_normals_are_deterministic_and_standard():
    a = synth.normal_rows(7, 300, 1000)
    b = synth.normal_rows(7, 300, 1000)
    assert np.array_equal(a, b)
    # any row can be regenerated alone
    assert np.array_equal(synth.normal_rows(7, 1, 1000, row0=123)[0], a[123])
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert not np.array_equal(a, synth.normal_rows(8, 300, 1000))


def test_uniform_and_permutation():
    u = synth.uniform_int(3, 128, 8192, 10000)
    assert u.min() >= 128 and u.max() <= 8192
    p = synth.permutation(5, 1000)
    assert sorted(p) == list(range(1000))


def test_paged_batch_shares_prefix_pages():
    ctx = np.array([100, 256, 257, 1000, 8192], np.int32)
    pb = synth.paged_batch(9, ctx, prefix_tokens=256)
    need = (ctx + 15) // 16
    assert pb.n_pages == 16 + int(np.sum(np.maximum(0, need - 16)))
    prefix = pb.table[4, :16]
    for b in range(len(ctx)):
        assert np.array_equal(pb.table[b, :min(16, need[b])], prefix[:min(16, need[b])])
    own = np.concatenate([pb.table[b, 16:need[b]] for b in range(len(ctx))])
    assert len(set(own)) == len(own) and not set(own) & set(prefix)
    assert set(np.concatenate([prefix, own])) == set(range(pb.n_pages))
    w = synth.windowed(pb, 300)
    assert list(w.kv_len) == [100, 256, 257, 300, 300]
    assert list(w.kv_start + w.kv_len) == list(ctx)
