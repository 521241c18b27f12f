"""Test helpers: an f64 brute-force softmax attention (the textbook definition,
independent of both the oracle and the kernels) and tolerance checks."""
from __future__ import annotations

import numpy as np

# fp32 parity bar of the attention path: max abs 1e-4 and max rel 1e-3 (an
# element passes if it meets either bound, rel measured against |want|).
ABS_TOL = 1e-4
REL_TOL = 1e-3

# bf16-input prefill (Q, K, V and the probabilities rounded to bf16, 8
# significant bits; fp32 accumulation): scores carry ~sqrt(d) * 2^-8 relative
# error and each P.V term ~2^-8, so outputs of N(0,1) data move by ~1e-3 to
# 1e-2. Bar: max abs 3e-2 or rel 3e-2 per element.
BF16_ABS_TOL = 3e-2
BF16_REL_TOL = 3e-2


def attention_f64(q, K, V, scale, softcap=None):
    """q [d], K/V [L][d] -> softmax(cap(q.K*scale)).V in float64."""
    q = np.asarray(q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    if len(K) == 0:
        return np.zeros(q.shape[-1])
    s = K @ q * scale
    if softcap:
        s = softcap * np.tanh(s / softcap)
    w = np.exp(s - s.max())
    w /= w.sum()
    return w @ V


def assert_close(got, want, abs_tol=ABS_TOL, rel_tol=REL_TOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bad = err > np.maximum(abs_tol, rel_tol * np.abs(want))
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err, 0)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside abs {abs_tol} / rel {rel_tol}; "
                             f"worst at {i}: got {got[i]!r} want {want[i]!r} (abs err {err[i]:.3g})")


def max_errors(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    rel = err / np.maximum(np.abs(want), 1e-30)
    return float(err.max(initial=0.0)), float(rel.max(initial=0.0))


LOG2E_F32 = np.float32(1.4426950408889634)


def bf16_round(x):
    """f32 values rounded to bf16 (nearest, ties to even), returned as f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_prefill_inputs(q, k, v, scale, softcap=None):
    """The values a bf16-input prefill multiplies, as f32 inputs for the fp32 oracle: K and V
    rounded to bf16, and q as the kernel rounds it, bf16(q * mul) / mul with mul = scale (with a
    soft-cap) or scale * log2(e) (the kernel folds the exp2 base into q). The oracle over these
    inputs differs from the kernel only by the bf16 rounding of the probabilities and the order
    of the fp32 sums; the gap to the oracle over the raw inputs is the input rounding, which
    grows with the score magnitudes."""
    mul = np.float32(scale) if softcap else np.float32(scale) * LOG2E_F32
    qm = np.ascontiguousarray(q, np.float32) * mul
    return bf16_round(qm) / mul, bf16_round(k), bf16_round(v)
