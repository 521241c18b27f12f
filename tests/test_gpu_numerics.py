"""Numerics of the attention kernels where ordinary N(0,1) inputs do not reach:

* the soft-cap's saturating regime (cap 5 with q x 8 and K x 3, as the oracle is checked in
  tests/test_oracle.py: |s| / cap >> 1, where each kernel's tanh must saturate correctly);
* the reference's soft-cap known answers (src/tensor/ops.rs:457-471: 0 -> 0,
  50 -> 50 tanh(1), +-1000 -> +-50 at cap 50), each probed through a two-position softmax whose
  output is proportional to exp(cap(s_a) - cap(s_b)), against the closed form;
* outlier-heavy data: a few positions with K and V norms 100-1000x the rest and q with outlier
  dimensions, which stress the Q8_0 kernel's split of q and of p * vscale into f16 pieces scaled
  by per-head and per-chunk powers of two.

Each case runs on f32 and Q8_0 decode and on fp32 and bf16-input prefill, against the oracle at
the bars of helpers.py, and against an f64 brute force. The bf16-input prefill is compared at its
own bar with the oracle over the inputs rounded as the kernel rounds them
(helpers.bf16_prefill_inputs): with scores of tens, rounding q and K to 8 bits alone moves a
score by ~0.04 and the softmax weights by ~4%, a property of bf16 inputs, not of the kernel."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from gpu_util import Contig, run_decode, run_prefill
from helpers import BF16_ABS_TOL, BF16_REL_TOL, assert_close, attention_f64, bf16_prefill_inputs

pytestmark = pytest.mark.gpu


def _decode_oracle(c, q, kv_start, kv_len, H, Hkv, d, scale, cap):
    B = q.shape[0]
    return orc.decode_batch(q.reshape(B, H * d), c.stores, 0, kv_start, kv_len, H, Hkv, d, scale,
                            cap).reshape(B, H, d)


def _dequant(c, dtype, b, d, Hkv, n):
    """K, V rows the kernels see for sequence b: f32 as written, Q8_0 dequantised."""
    if dtype == "f32":
        return c.k[b, 0, :n].astype(np.float64), c.v[b, 0, :n].astype(np.float64)
    kv_dim = Hkv * d
    K = np.stack([np.concatenate([c.stores[b].read_k_head(0, p, h, d) for h in range(Hkv)]) for p in range(n)])
    V = np.stack([np.concatenate([c.stores[b].read_v_head(0, p, h, d) for h in range(Hkv)]) for p in range(n)])
    return K.reshape(n, kv_dim).astype(np.float64), V.reshape(n, kv_dim).astype(np.float64)


def _prefill_oracle(c, b, q, off, H, Hkv, d, scale, cap=None, window=None, precision="f32"):
    """The oracle's prefill of sequence b of a one-layer Contig; for bf16 over the inputs as the
    kernel rounds them."""
    T = q.shape[0]
    st = c.stores[b]
    if precision == "bf16":
        q, k, v = bf16_prefill_inputs(q, c.k[b], c.v[b], scale, cap)
        st = orc.kv_cache(k, v)
    return orc.prefill(q.reshape(T, H * d), st, 0, off, H, Hkv, d, scale, cap, window).reshape(T, H, d)


# ---------------------------------------------------------------- soft-cap saturation
@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("d,H,Hkv", [(64, 8, 2), (128, 32, 8), (256, 16, 8)])
def test_decode_softcap_saturates(backend, dtype, d, H, Hkv):
    """Decode with cap 5 and 50 on scores of q x 8 . K x 3 (|s| up to ~100): most scores sit
    on the flat part of tanh, where a wrong saturation shifts whole softmax weights."""
    lens = np.array([1, 31, 300, 1000, 2500], np.int32)
    c = Contig(backend, dtype, len(lens), 1, int(lens.max()), Hkv, d, seed=7100 + d, k_mul=3.0)
    q = synth.normal(7200 + d, (len(lens), H, d), 8.0)
    scale = float(1 / np.sqrt(d))
    starts = np.zeros_like(lens)
    for cap in (5.0, 50.0):
        want = _decode_oracle(c, q, starts, lens, H, Hkv, d, scale, cap)
        got = run_decode(backend, c.cache, q, starts, lens, H, scale, cap)
        assert_close(got, want, what=f"{dtype} d{d} cap {cap}")
        for b in (2, 4):  # f64 brute force on two sequences, every head
            K, V = _dequant(c, dtype, b, d, Hkv, int(lens[b]))
            for h in range(H):
                kvh = h // (H // Hkv)
                f64 = attention_f64(q[b, h], K[:, kvh * d:(kvh + 1) * d], V[:, kvh * d:(kvh + 1) * d], scale, cap)
                assert_close(got[b, h], f64, what=f"{dtype} d{d} cap {cap} seq {b} head {h} vs f64")


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("d,H,Hkv", [(64, 8, 2), (128, 8, 2), (256, 4, 2)])
def test_prefill_softcap_saturates(backend, precision, d, H, Hkv):
    """Prefill (causal, two prompts with offsets) with cap 5 on q x 8 . K x 3."""
    lens, offs = [300, 97], [0, 40]
    max_seq = max(o + n for o, n in zip(offs, lens))
    c = Contig(backend, "f32", 2, 1, max_seq, Hkv, d, seed=7300 + d, k_mul=3.0)
    q = synth.normal(7400 + d, (sum(lens), H, d), 8.0)
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    scale = float(1 / np.sqrt(d))
    for cap, window in ((5.0, None), (5.0, 64), (50.0, None)):
        got = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, precision=precision)
        for b in range(2):
            rows = slice(q_start[b], q_start[b + 1])
            want = _prefill_oracle(c, b, q[rows], offs[b], H, Hkv, d, scale, cap, window, precision)
            assert_close(got[rows], want, *tol, what=f"{precision} d{d} cap {cap} w {window} seq {b}")


# ---------------------------------------------------------------- known answers of the cap
# Pairs (s_a, s_b) of raw scores; the cap (50) maps them to the known answers of ops.rs:457-471.
# A sequence holds two positions: a with V = 0 and b with V = M * e_1, so out[1] =
# M * w_b = M / (1 + exp(cap(s_a) - cap(s_b))), and M is chosen so out[1] is O(0.1): any error
# in the capped scores moves out[1] by the same relative amount (1e-3 bar <-> 1e-3 in the
# scores), and an uncapped score makes it 0.
_PAIRS = [(1000.0, 50.0), (-50.0, -1000.0), (0.0, 5.0), (-1000.0, 1000.0)]


def _cap_pairs_case(be, dtype, d=64, Hkv=1, H=1):
    n = len(_PAIRS)
    k = np.zeros((n, 1, 2, Hkv * d), np.float32)
    v = np.zeros_like(k)
    M = np.zeros(n)
    for i, (sa, sb) in enumerate(_PAIRS):
        k[i, 0, 0, 0], k[i, 0, 1, 0] = sa, sb
        ca, cb = 50.0 * np.tanh(sa / 50.0), 50.0 * np.tanh(sb / 50.0)
        M[i] = float(min(1e4, 0.1 * (1.0 + np.exp(ca - cb))))
        v[i, 0, 1, 1] = M[i]
    c = Contig(be, dtype, n, 1, 2, Hkv, d, k=k, v=v)
    return c, M


def _closed_form(c, dtype, d, n_seqs):
    """out[1] of each pair from the stored (for Q8_0: dequantised) K and V, through the
    textbook softmax of 50 tanh(s / 50) in f64."""
    want = np.zeros((n_seqs, d))
    for b in range(n_seqs):
        K, V = _dequant(c, dtype, b, d, 1, 2)
        want[b] = attention_f64(np.eye(d)[0], K, V, 1.0, 50.0)
    return want


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_decode_softcap_known_answers(backend, dtype):
    d = 64
    c, _ = _cap_pairs_case(backend, dtype, d)
    n = len(_PAIRS)
    q = np.zeros((n, 1, d), np.float32)
    q[:, 0, 0] = 1.0
    got = run_decode(backend, c.cache, q, [0] * n, [2] * n, 1, 1.0, 50.0)
    want = _closed_form(c, dtype, d, n)
    assert_close(got[:, 0], want, what=f"{dtype} cap known answers")
    assert_close(got, _decode_oracle(c, q, [0] * n, [2] * n, 1, 1, d, 1.0, 50.0), what=f"{dtype} vs oracle")
    assert np.all(got[:, 0, 1] > 0.05), got[:, 0, 1]  # the b-position weight survived the cap


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_softcap_known_answers(backend, precision):
    """Row 1 of each two-token prompt attends both positions (causal); row 0 only itself."""
    d = 64
    c, _ = _cap_pairs_case(backend, "f32", d)
    n = len(_PAIRS)
    q = np.zeros((2 * n, 1, d), np.float32)
    q[:, 0, 0] = 1.0
    q_start = np.arange(n + 1, dtype=np.int32) * 2
    got = run_prefill(backend, c.cache, q, q_start, [0] * n, 1, 1.0, 50.0, precision=precision)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    want = _closed_form(c, "f32", d, n)
    assert_close(got[1::2, 0], want, *tol, what=f"{precision} cap known answers")
    assert np.all(got[1::2, 0, 1] > 0.05), got[1::2, 0, 1]


# ---------------------------------------------------------------- outlier-heavy data
def _outlier_data(seed, n_seqs, max_seq, Hkv, d, H):
    """N(0,1) K/V with, per sequence, a sink at position 0 and two more positions with K x 100,
    three positions with V x 1000 and one with V x 100; q with two outlier dimensions (x 30) per
    head. Every 32-element Q8_0 block of an outlier row is an outlier block."""
    rng = np.random.default_rng(seed)
    kv_dim = Hkv * d
    k = rng.standard_normal((n_seqs, 1, max_seq, kv_dim)).astype(np.float32)
    v = rng.standard_normal((n_seqs, 1, max_seq, kv_dim)).astype(np.float32)
    for s in range(n_seqs):
        pk = np.concatenate([[0], rng.choice(np.arange(1, max_seq), 2, replace=False)])
        pv = rng.choice(np.arange(max_seq), 4, replace=False)
        k[s, 0, pk] *= 100.0
        v[s, 0, pv[:3]] *= 1000.0
        v[s, 0, pv[3]] *= 100.0
    q = rng.standard_normal((n_seqs, H, d)).astype(np.float32)
    dims = rng.choice(d, 2, replace=False)
    q[:, :, dims] *= 30.0
    return k, v, q


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("d,H,Hkv", [(64, 9, 3), (128, 32, 8), (256, 16, 8)])
def test_decode_outliers(backend, dtype, d, H, Hkv):
    lens = np.array([17, 500, 2000, 3000], np.int32)
    k, v, q = _outlier_data(7500 + d, len(lens), int(lens.max()), Hkv, d, H)
    c = Contig(backend, dtype, len(lens), 1, int(lens.max()), Hkv, d, k=k, v=v)
    scale = float(1 / np.sqrt(d))
    # the temperature keeps several positions in play beside the sinks
    for s, cap in ((scale / 30.0, None), (scale, 50.0)):
        for start in (0, 7):
            st = np.full(len(lens), start, np.int32)
            ln = (lens - st).astype(np.int32)
            want = _decode_oracle(c, q, st, ln, H, Hkv, d, s, cap)
            got = run_decode(backend, c.cache, q, st, ln, H, s, cap)
            assert_close(got, want, what=f"{dtype} d{d} outliers scale {s:.4g} cap {cap} start {start}")
    b = 2
    K, V = _dequant(c, dtype, b, d, Hkv, int(lens[b]))
    got = run_decode(backend, c.cache, q, [0] * len(lens), lens, H, scale / 30.0)
    for h in range(0, H, max(1, H // 4)):
        kvh = h // (H // Hkv)
        f64 = attention_f64(q[b, h], K[:, kvh * d:(kvh + 1) * d], V[:, kvh * d:(kvh + 1) * d], scale / 30.0)
        assert_close(got[b, h], f64, what=f"{dtype} d{d} outliers head {h} vs f64")


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_outliers(backend, precision):
    H, Hkv, d = 8, 2, 128
    lens, offs = [400, 150], [0, 100]
    max_seq = max(o + n for o, n in zip(offs, lens))
    k, v, _ = _outlier_data(7600, 2, max_seq, Hkv, d, H)
    c = Contig(backend, "f32", 2, 1, max_seq, Hkv, d, k=k, v=v)
    rng = np.random.default_rng(7601)
    q = rng.standard_normal((sum(lens), H, d)).astype(np.float32)
    q[:, :, rng.choice(d, 2, replace=False)] *= 30.0
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    s = float(1 / np.sqrt(d)) / 30.0
    got = run_prefill(backend, c.cache, q, q_start, offs, H, s, precision=precision)
    for b in range(2):
        rows = slice(q_start[b], q_start[b + 1])
        want = _prefill_oracle(c, b, q[rows], offs[b], H, Hkv, d, s, precision=precision)
        if precision == "f32":
            assert_close(got[rows], want, what=f"f32 outliers seq {b}")
            continue
        # bf16 rounds each probability to 8 bits before the P.V product, so an output's error
        # scales with the magnitudes of its terms, sum_j p_j |v_j| / l, not with the output
        # itself (V rows of 1000 with weights ~1e-2 cancel to outputs ~1): the bf16 bar applies
        # to that sum, from an f64 brute force over the rounded inputs.
        qr, kr, vr = bf16_prefill_inputs(q[rows], c.k[b, 0], c.v[b, 0], s)
        for h in range(H):
            kvh = h // (H // Hkv)
            Q = qr[:, h].astype(np.float64)
            K = kr[:, kvh * d:(kvh + 1) * d].astype(np.float64)
            V = vr[:, kvh * d:(kvh + 1) * d].astype(np.float64)
            S = Q @ K.T * s
            pos = offs[b] + np.arange(lens[b])
            S[np.arange(max_seq)[None, :] > pos[:, None]] = -np.inf
            P = np.exp(S - S.max(axis=1, keepdims=True))
            P /= P.sum(axis=1, keepdims=True)
            f64, mass = P @ V, P @ np.abs(V)
            err = np.abs(got[rows][:, h] - f64)
            bound = np.maximum(BF16_ABS_TOL, BF16_REL_TOL * mass)
            assert (err <= bound).all(), (b, h, float((err / bound).max()))
            assert_close(want[:, h], f64, 1e-3, 1e-3, what=f"oracle over bf16 inputs vs f64, seq {b} head {h}")


# ---------------------------------------------------------------- a running maximum that keeps moving
@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("window", [None, 64])
def test_prefill_rising_scores(backend, precision, window):
    """Scores that climb along the keys (K = noise + (pos / 8) * u, q ~ u): every query's
    running maximum passes the kernels' lazy threshold (8 log2 units) again and again, so the
    rescale of O and of the row sums runs on most tiles of every query block, not only on a
    query's first attended tile as with N(0,1) data."""
    H, Hkv, d, T = 8, 2, 128, 320
    kv_dim = Hkv * d
    rng = np.random.default_rng(7700)
    u = np.full(d, 4.0 / np.sqrt(d), np.float32)
    pos = np.arange(T, dtype=np.float32)[:, None]
    k = 0.5 * rng.standard_normal((T, kv_dim)).astype(np.float32) + (pos / 8.0) * np.tile(u, Hkv)[None, :]
    v = rng.standard_normal((T, kv_dim)).astype(np.float32)
    c = Contig(backend, "f32", 1, 1, T, Hkv, d, k=k.reshape(1, 1, T, kv_dim), v=v.reshape(1, 1, T, kv_dim))
    q = (u[None, None, :] + 0.1 * rng.standard_normal((T, H, d))).astype(np.float32)
    s = float(1 / np.sqrt(d))
    # the scores really climb: the last key's score is tens of log2 units above the first's
    kf = k[:, :d].astype(np.float64)
    sc = (kf @ q[0, 0].astype(np.float64)) * s / np.log(2.0)
    assert sc[-1] - sc[0] > 60.0
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    got = run_prefill(backend, c.cache, q, [0, T], [0], H, s, None, window, precision=precision)
    want = _prefill_oracle(c, 0, q, 0, H, Hkv, d, s, None, window, precision)
    assert_close(got, want, *tol, what=f"rising scores {precision} window {window}")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("d,H,Hkv", [(64, 9, 3), (128, 32, 8), (256, 16, 8)])
def test_decode_rising_scores(backend, dtype, d, H, Hkv):
    """Decode over keys whose scores climb with the position (K = noise + (pos / 8) * u, q ~ u):
    the running maximum moves on nearly every step of every chunk, and the chunks of a long
    sequence merge partials whose maxima differ by hundreds of log2 units."""
    lens = np.array([40, 700, 2100], np.int32)
    T = int(lens.max())
    kv_dim = Hkv * d
    rng = np.random.default_rng(7800 + d)
    u = np.full(d, 4.0 / np.sqrt(d), np.float32)
    pos = np.arange(T, dtype=np.float32)[:, None]
    k = np.stack([0.5 * rng.standard_normal((T, kv_dim)).astype(np.float32) + (pos / 8.0) * np.tile(u, Hkv)[None, :]
                  for _ in lens])
    v = rng.standard_normal((len(lens), T, kv_dim)).astype(np.float32)
    c = Contig(backend, dtype, len(lens), 1, T, Hkv, d, k=k[:, None], v=v[:, None])
    q = (u[None, None, :] + 0.1 * rng.standard_normal((len(lens), H, d))).astype(np.float32)
    s = float(1 / np.sqrt(d))
    for st in (np.zeros(len(lens), np.int32), np.maximum(lens - 300, 0).astype(np.int32)):
        ln = (lens - st).astype(np.int32)
        want = _decode_oracle(c, q, st, ln, H, Hkv, d, s, None)
        got = run_decode(backend, c.cache, q, st, ln, H, s)
        assert_close(got, want, what=f"{dtype} d{d} rising scores start {st.tolist()}")
