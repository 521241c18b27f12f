"""Attention over non-finite data on the GPU, against the oracle's restatement of
flash_attn_1d_ext (src/tensor/flash.rs:46-124): a NaN score or value makes its head's sums
NaN, and the reference then leaves them unnormalised (flash.rs:118-123, `if l > 0`), so the
head's output is NaN, not zeros; an infinite value under a non-zero weight gives +-inf in that
dimension; an infinite q entry gives infinite or NaN scores. Every path is checked: f32 decode
through the split kernel's in-kernel merge and through the combine kernel, Q8_0 decode (whose
codec turns a block holding a NaN or an infinity into NaN or infinite values, as the reference
codec does) through one workgroup and through the combine, and fp32 and bf16-input prefill,
each with and without the soft-cap (under which an infinite score becomes +-cap).
The inf / NaN pattern must equal the oracle's element for element, sign for sign, and the
finite elements stay within the usual bars."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from gpu_util import Contig, run_decode, run_prefill
from helpers import ABS_TOL, REL_TOL

pytestmark = pytest.mark.gpu

H, HKV, D = 8, 2, 64
GROUP = H // HKV


def _plant(k, v):
    """Non-finite K/V entries, layer 0: seq 0 a NaN in K (KV head 0, position 5), seq 1 +inf
    in V (KV head 1, position 7, dim 3), seq 2 -inf in V and +inf in V of one head at two
    positions (dim 10 and 11), seq 3 clean; seqs 4, 5 (long windows) as seqs 0, 1, seq 5 with a
    second infinity."""
    k[0, 0, 5, 2] = np.nan
    v[1, 0, 7, D + 3] = np.inf
    v[2, 0, 9, 10] = -np.inf
    v[2, 0, 40, 11] = np.inf
    if k.shape[0] > 5 and k.shape[2] > 1700:
        k[4, 0, 1500, 2] = np.nan
        v[5, 0, 1700, D + 3] = np.inf
        v[5, 0, 100, D + 5] = np.inf  # in a split the f32 combine's padded entries reload


def _check(got, want, tol_abs, tol_rel, what):
    for name, f in (("NaN", np.isnan), ("+inf", np.isposinf), ("-inf", np.isneginf)):
        bad = np.argwhere(f(got) != f(want))
        assert bad.size == 0, f"{what}: {name} pattern differs at {bad[:5].tolist()}"
    fin = np.isfinite(want)
    err = np.abs(got[fin] - want[fin])
    ok = (err <= tol_abs) | (err <= tol_rel * np.abs(want[fin]))
    assert np.all(ok), f"{what}: finite elements off by up to {float(err.max())}"


@pytest.mark.parametrize("cap", [None, 30.0])
@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_decode_nonfinite_like_reference(backend, dtype, cap):
    B, max_seq = 6, 2048
    k = synth.normal_rows(71, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    v = synth.normal_rows(72, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    _plant(k, v)
    c = Contig(backend, dtype, B, 1, max_seq, HKV, D, k=k, v=v)
    q = synth.normal(73, (B, H, D))
    q[3, 5, 7] = np.inf  # seq 3: one head's q holds an infinity (every score NaN)
    q[5, 1, 9] = -np.inf  # the same in a long window: all-NaN partials through the combine
    # seqs 0-3: 200 positions (the f32 kernel merges its splits in the kernel, the Q8_0 kernel
    # covers them in one workgroup); seqs 4, 5: 2,000 (the combine kernel for both)
    kv_start = np.zeros(B, np.int32)
    kv_len = np.array([200, 200, 200, 200, 2000, 2000], np.int32)
    scale = 1 / np.sqrt(D)
    want = orc.decode_batch(q.reshape(B, H * D), c.stores, 0, kv_start, kv_len, H, HKV, D, scale,
                            cap).reshape(B, H, D)
    # (the Q8_0 codec drops a NaN, quantised to 0, and makes a block holding an infinity NaN)
    if dtype == "f32":
        assert np.isnan(want[0, :GROUP]).all() and np.isposinf(want[1, GROUP:, 3]).all()
    else:
        assert np.isfinite(want[0]).all() and np.isnan(want[1, GROUP:, :32]).all()
    # (under the soft-cap an infinite score becomes +-cap: that head's output is finite)
    assert np.isfinite(want[3, :5]).all() and (np.isfinite(want[3, 5]).all() if cap else np.isnan(want[3, 5]).all())
    got = run_decode(backend, c.cache, q, kv_start, kv_len, H, scale, cap)
    _check(got, want, ABS_TOL, REL_TOL, f"{dtype} decode, cap {cap}")


@pytest.mark.parametrize("cap", [None, 30.0])
@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_nonfinite_like_reference(backend, precision, cap):
    B, max_seq, n_q = 4, 256, 64
    k = synth.normal_rows(81, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    v = synth.normal_rows(82, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    _plant(k, v)
    c = Contig(backend, "f32", B, 1, max_seq, HKV, D, k=k, v=v)
    q = synth.normal(83, (B * n_q, H, D))
    q[3 * n_q + 20, 5, 7] = np.inf
    q_start = np.arange(B + 1, dtype=np.int32) * n_q
    pos_offset = np.full(B, 100, np.int32)  # queries at positions 100..163: all plants in range
    scale = 1 / np.sqrt(D)
    want = np.concatenate([
        orc.prefill(q[b * n_q:(b + 1) * n_q].reshape(n_q, H * D), c.stores[b], 0, 100, H, HKV, D, scale,
                    cap, None).reshape(n_q, H, D) for b in range(B)])
    got = run_prefill(backend, c.cache, q, q_start, pos_offset, H, scale, cap, precision=precision)
    tol = (ABS_TOL, REL_TOL) if precision == "f32" else (3e-2, 3e-2)
    _check(got, want, tol[0], tol[1], f"{precision} prefill, cap {cap}")


def _plant_outside(k, v, lo, hi):
    """NaN in K and +-inf / NaN in V at every KV head of positions lo-3 .. lo-1 and hi .. hi+2
    (the slots just outside a window, in the same pages and tiles as its edges)."""
    for pos in list(range(max(0, lo - 3), lo)) + list(range(hi, min(k.shape[2], hi + 3))):
        k[:, 0, pos, ::7] = np.nan
        v[:, 0, pos, ::5] = np.inf
        v[:, 0, pos, 1::5] = -np.inf
        v[:, 0, pos, 2::5] = np.nan


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_decode_ignores_nonfinite_outside_the_window(backend, dtype):
    """Slots outside [kv_start, kv_start + kv_len) are never read by the reference: non-finite
    data there, in the same pages as the window's edges, must not reach the output."""
    B, max_seq = 2, 2048
    starts = np.array([21, 37], np.int32)
    lens = np.array([150, 1900], np.int32)  # the split kernel's own merge, and the combine
    k = synth.normal_rows(91, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    v = synth.normal_rows(92, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    for b in range(B):
        kb, vb = k[b:b + 1], v[b:b + 1]
        _plant_outside(kb, vb, int(starts[b]), int(starts[b] + lens[b]))
    c = Contig(backend, dtype, B, 1, max_seq, HKV, D, k=k, v=v)
    q = synth.normal(93, (B, H, D))
    for cap in (None, 30.0):
        want = orc.decode_batch(q.reshape(B, H * D), c.stores, 0, starts, lens, H, HKV, D, 0.125,
                                cap).reshape(B, H, D)
        assert np.isfinite(want).all()
        got = run_decode(backend, c.cache, q, starts, lens, H, 0.125, cap)
        _check(got, want, ABS_TOL, REL_TOL, f"{dtype} decode outside the window, cap {cap}")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_ignores_nonfinite_outside_the_window(backend, precision, dtype):
    """Keys after a sequence's last query position, and before its sliding window, sit in the
    tiles prefill reads but are never attended: non-finite data there must not reach the output
    (a masked weight times a NaN value would still be NaN)."""
    B, max_seq, n_q, window = 2, 512, 70, 40
    k = synth.normal_rows(95, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    v = synth.normal_rows(96, B * max_seq, HKV * D).reshape(B, 1, max_seq, HKV * D)
    pos0 = 101
    # first attended key: pos0 - window + 1 with the window, 0 without; last: pos0 + n_q - 1
    _plant_outside(k, v, pos0 - window + 1, pos0 + n_q)
    c = Contig(backend, dtype, B, 1, max_seq, HKV, D, k=k, v=v)
    q = synth.normal(97, (B * n_q, H, D))
    q_start = np.arange(B + 1, dtype=np.int32) * n_q
    pos_offset = np.full(B, pos0, np.int32)
    tol = (ABS_TOL, REL_TOL) if precision == "f32" else (3e-2, 3e-2)
    for sw in (window, None):
        if sw is None:  # no window: the slots before it are attended, so only the tail stays planted
            k2, v2 = k.copy(), v.copy()
            k2[:, 0, : pos0 - window + 1] = k[:, 0, 200:200 + pos0 - window + 1]
            v2[:, 0, : pos0 - window + 1] = v[:, 0, 200:200 + pos0 - window + 1]
            c = Contig(backend, dtype, B, 1, max_seq, HKV, D, k=k2, v=v2)
        want = np.concatenate([
            orc.prefill(q[b * n_q:(b + 1) * n_q].reshape(n_q, H * D), c.stores[b], 0, pos0, H, HKV, D, 0.125,
                        None, sw).reshape(n_q, H, D) for b in range(B)])
        assert np.isfinite(want).all()
        got = run_prefill(backend, c.cache, q, q_start, pos_offset, H, 0.125, None, sw, precision=precision)
        _check(got, want, tol[0], tol[1], f"{precision} prefill over {dtype}, window {sw}")
