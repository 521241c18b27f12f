"""The ops beside attention on a decode step, on the GPU through the C ABI: RoPE
(src/tensor/ops.rs:212-245) and the Q8_0 weight matvec (src/tensor/quantized.rs:247-346,
:587-610), against the oracle's restatements and an f64 product.

RoPE bar: max abs 1e-5 x max|x| (the angles are computed exactly as the reference computes
them; cos/sin differ in the last place). Matvec bar: |got - f64| <= 2e-6 x sum_c |w x|, the
size of f32 rounding over the 4,096-term sums (the fp32 attention bar's 1e-4 absolute does not
apply to dot products whose terms are O(1000)); the reference's own fixture is matched exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth

pytestmark = pytest.mark.gpu


def _rope_gpu(be, x, pos, head_dim, base, scaling, rot_dim):
    n_rows, n_heads = x.shape[0], x.shape[1]
    dx = be.buffer(np.ascontiguousarray(x, np.float32))
    dp = be.buffer(np.asarray(pos, np.int32))
    be.rope(dx, n_rows, n_heads, head_dim, dp, base, scaling, rot_dim)
    be.sync()
    return dx.download(x.shape)


def test_rope_reference_known_answers(backend):
    """ops.rs tests on the device: position 0 is the identity (full and partial rotary), and
    pos 2 with scaling 2 equals pos 1 with scaling 1, bit for bit."""
    x = np.array([[[1.0, 2.0, 3.0, 4.0]]], np.float32)
    assert np.array_equal(_rope_gpu(backend, x, [0], 4, 10000.0, 1.0, 4), x)
    assert np.array_equal(_rope_gpu(backend, x, [0], 4, 10000.0, 1.0, 2), x)
    a = _rope_gpu(backend, x, [2], 4, 10000.0, 2.0, 4)
    b = _rope_gpu(backend, x, [1], 4, 10000.0, 1.0, 4)
    assert np.array_equal(a, b)
    assert np.allclose(a.reshape(-1), orc.rope(x.reshape(-1), 1, 4, 10000.0, 1.0, 4), atol=1e-6)


@pytest.mark.parametrize("n_heads,head_dim,rot_dim,base,scaling", [
    (4, 5, 5, 10000.0, 1.0),         # odd head_dim: its last dimension is left alone, as in the reference
    (32, 128, 128, 500000.0, 1.0),   # Llama-3-8B q
    (8, 128, 128, 500000.0, 1.0),    # its k
    (9, 64, 64, 10000.0, 1.0),       # SmolLM
    (4, 96, 48, 10000.0, 4.0),       # Phi-3-style partial rotary, linear scaling
    (2, 64, 33, 10000.0, 1.0),       # odd rot_dim rounds down
    (2, 1100, 1100, 10000.0, 1.0),   # 550 pairs: three launches of at most 256 pairs
    (3, 251, 251, 10000.0, 1.0),     # glibc's powf is not correctly rounded at i = 110 here
])
def test_rope_matches_oracle(backend, n_heads, head_dim, rot_dim, base, scaling):
    pos = np.array([0, 1, 17, 511, 4095, 8191, 65535], np.int32)
    x = synth.normal(1200 + head_dim + rot_dim, (len(pos), n_heads, head_dim))
    got = _rope_gpu(backend, x, pos, head_dim, base, scaling, rot_dim)
    rot = min(rot_dim, head_dim) & ~1
    for r, p in enumerate(pos):
        want = orc.rope(x[r].reshape(-1), int(p), head_dim, base, scaling, rot_dim).reshape(n_heads, head_dim)
        err = np.abs(got[r] - want).max()
        assert err <= 1e-5 * np.abs(x[r]).max(), (int(p), err)
        assert np.array_equal(got[r][:, rot:], x[r][:, rot:])


def _q8_rows(rows, cols, seed, mul=1.0):
    w = synth.normal_rows(seed, rows, cols, mul)
    return orc.q8_quantize_rows(w).reshape(-1)


def _dequant(raw, rows, cols):
    blk = raw.reshape(rows, cols // 32, 34)
    scale = blk[:, :, :2].copy().view("<f2").astype(np.float64)
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    return (q * scale).reshape(rows, cols)


def _matvec_gpu(be, raw, rows, cols, x):
    w = be.create_q8_weights(raw, rows, cols)
    n_vec = x.shape[0]
    dx = be.buffer(np.ascontiguousarray(x, np.float32))
    dy = be.empty(n_vec * rows * 4)
    be.matvec_q8_0(w, dx, n_vec, dy)
    be.sync()
    y = dy.download((n_vec, rows))
    w.destroy()
    return y


def test_matvec_q8_0_reference_fixture(backend):
    """quantized.rs test_q8_0_matvec_matches_f32: 10416 and -20832, here exactly (integer
    products and sums below 2^24, exact in the f16 pieces and the f32 accumulation)."""
    data = np.frombuffer(orc.q8_0_block(1.0, range(32)) + orc.q8_0_block(2.0, [-i for i in range(32)]), np.uint8)
    y = _matvec_gpu(backend, data, 2, 32, np.arange(32, dtype=np.float32)[None, :])
    assert y.tolist() == [[10416.0, -20832.0]]


@pytest.mark.parametrize("rows,cols,n_vec", [
    (6144, 4096, 1),    # Llama-3-8B fused QKV projection, one token (the vector-ALU kernel)
    (6144, 4096, 4),    # four tokens: the largest vector-ALU launch
    (6144, 4096, 64),   # the same over a decode batch of 64 (MFMA)
    (96, 14336, 2),     # FFN down-projection width: x of one vector fills LDS, one launch per vector
    (40, 16416, 1),     # 513 blocks: x too wide for LDS, a single vector on the MFMA path
    (100, 96, 3),       # vector-ALU kernel on a row tail and an odd block count
    (64, 4096, 3),      # three vectors: x padded to 3 x 5632 floats, 66 KiB of LDS
    (16, 32, 2),        # one block pair: seven of the eight waves have no blocks
    (4096, 4096, 5),    # the output projection, a ragged batch
    (100, 96, 70),      # a row tail (100 = 6 x 16 + 4), an odd block count, two vector launches
    (16, 32, 17),
])
def test_matvec_q8_0_matches_oracle_and_f64(backend, rows, cols, n_vec):
    raw = _q8_rows(rows, cols, 1300 + rows + n_vec)
    x = synth.normal(1400 + cols + n_vec, (n_vec, cols))
    x[0, :7] *= 1e4     # a few large entries: the first K slice's piece scale follows the largest
    got = _matvec_gpu(backend, raw, rows, cols, x)
    wd = _dequant(raw, rows, cols)
    exact = x.astype(np.float64) @ wd.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    assert np.all(np.abs(got - exact) <= 2e-6 * mag), np.max(np.abs(got - exact) / mag)
    for v in (0, n_vec // 2, n_vec - 1):
        want = orc.matvec_q8_0(raw, rows, cols, x[v])
        assert np.all(np.abs(got[v] - want) <= 4e-6 * mag[v]), v


@pytest.mark.parametrize("n_vec", [1, 8])
def test_matvec_q8_0_nonfinite_activations_like_the_reference(backend, n_vec):
    """Infinite and NaN activations give what the reference's block loop gives
    (src/tensor/quantized.rs:587-610: each block's sum of q * x, times the block's scale): +-inf
    where the infinite terms of a row share one sign, NaN where they differ, where a zero q or
    scale meets an infinity, or where the row holds a NaN; the same inf / NaN pattern, sign for
    sign, as the oracle. One vector takes the vector-ALU kernel, eight the MFMA path, whose
    activation pieces keep an infinity exact (hi = +-inf, lo = 0) and take their scale from the
    finite entries; its finite vectors stay within the usual bar."""
    rows, cols = 64, 512
    raw = _q8_rows(rows, cols, 1500 + n_vec)
    x = synth.normal(1600 + n_vec, (n_vec, cols))
    x[0, 37] = np.inf
    x[0, 400] *= 1e3   # a large finite entry in another K slice
    if n_vec > 1:
        x[1, 100] = -np.inf
        x[1, 101] = 50.0   # beside the infinity, in its slice: must not overflow its f16 pieces
        x[2, 5] = np.nan
        x[3, 3] = np.inf
        x[3, 300] = -np.inf
    got = _matvec_gpu(backend, raw, rows, cols, x)
    wd = _dequant(raw, rows, cols)
    for v in range(n_vec):
        want = orc.matvec_q8_0(raw, rows, cols, x[v])
        np.testing.assert_array_equal(np.isnan(got[v]), np.isnan(want), err_msg=f"vector {v}")
        np.testing.assert_array_equal(np.isposinf(got[v]), np.isposinf(want), err_msg=f"vector {v}")
        np.testing.assert_array_equal(np.isneginf(got[v]), np.isneginf(want), err_msg=f"vector {v}")
        if np.all(np.isfinite(x[v])):
            mag = np.abs(x[v].astype(np.float64)) @ np.abs(wd).T
            assert np.all(np.abs(got[v] - want) <= 4e-6 * mag), v
    assert not np.all(np.isfinite(got[0]))


def test_matvec_q8_0_result_independent_of_the_batch(backend):
    """A vector's outputs do not depend on the other vectors of the call, as in the reference,
    which computes each vector alone (src/tensor/quantized.rs:247-346): on the MFMA path (5 or
    more vectors) every output's arithmetic order is fixed by the shape, and a piece scale by the
    vector's own slice, so the first vectors come out bit for bit the same in batches of 5, 17,
    64 and 70 (two launches). Batches of 1-4 take the vector-ALU kernel, whose rounding differs:
    those agree with the MFMA path within the matvec bar."""
    rows, cols = 200, 1536
    raw = _q8_rows(rows, cols, 1700)
    x = synth.normal(1701, (70, cols))
    x[1, 5] *= 1e4  # an outlier in vector 1: the other vectors' piece scales must not follow it
    base = _matvec_gpu(backend, raw, rows, cols, x[:5])
    for n in (17, 64, 70):
        got = _matvec_gpu(backend, raw, rows, cols, x[:n])
        assert np.array_equal(got[:5].view(np.uint32), base.view(np.uint32)), n
    few = _matvec_gpu(backend, raw, rows, cols, x[:3])
    mag = np.abs(x[:3].astype(np.float64)) @ np.abs(_dequant(raw, rows, cols)).T
    assert np.all(np.abs(few - base[:3]) <= 4e-6 * mag)


def test_ops_argument_errors_and_empty_calls(backend):
    """Shapes the ABI rejects come back as GLA_ERR_INVALID (the caller's CPU path), and empty
    calls are no-ops: zero vectors, zero rows, a rotary dimension of 0 or 1 (no whole pair)."""
    from glint_amd._lib import GLA_ERR_INVALID, GlaError

    raw = _q8_rows(16, 64, 7)
    with pytest.raises(GlaError) as e:
        backend.create_q8_weights(np.zeros(34 * 3, np.uint8), 1, 96 + 16)  # cols not a multiple of 32
    assert e.value.code == GLA_ERR_INVALID
    w = backend.create_q8_weights(raw, 16, 64)
    y = backend.buffer(np.full(16, 7.0, np.float32))
    backend.matvec_q8_0(w, backend.empty(64 * 4), 0, y)  # no vectors: y untouched
    backend.sync()
    assert np.all(y.download((16,)) == 7.0)
    with pytest.raises(GlaError) as e:
        backend.matvec_q8_0(w, backend.empty(64 * 4), -1, y)
    assert e.value.code == GLA_ERR_INVALID
    with pytest.raises(GlaError) as e:  # past the activation split's grid: refused before any launch
        backend.matvec_q8_0(w, backend.empty(64 * 4), 262129, y)
    assert e.value.code == GLA_ERR_INVALID and "n_vec" in str(e.value)
    backend.matvec_q8_0(w, backend.empty(64 * 4), 0, y)  # and the context still works
    backend.sync()
    w.destroy()

    x = synth.normal(3, (2, 2, 8))
    for rot in (0, 1):  # no whole pair below rot: nothing moves
        assert np.array_equal(_rope_gpu(backend, x, [5, 9], 8, 10000.0, 1.0, rot), x)
    with pytest.raises(GlaError) as e:
        _rope_gpu(backend, x, [5, 9], 0, 10000.0, 1.0, 8)  # head_dim 0
    assert e.value.code == GLA_ERR_INVALID
