"""Batched causal prefill on the GPU (fp32 MFMA and the bf16-input variant) through the C ABI,
against the oracle's prefill loop (src/transformer/forward.rs:927-958).
fp32 bar: max abs 1e-4 / rel 1e-3; bf16 bar: max abs 3e-2 / rel 3e-2 (helpers.BF16_*);
indexing bit-exact for both (K = 0, small-integer V: every bf16 rounding is exact)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from gpu_util import Contig, Pool, run_prefill
from helpers import BF16_ABS_TOL, BF16_REL_TOL, assert_close, max_errors

pytestmark = pytest.mark.gpu


def _oracle_prefill(store, q, pos_offset, H, Hkv, d, scale, softcap=None, window=None, layer=0):
    T = q.shape[0]
    return orc.prefill(q.reshape(T, H * d), store, layer, pos_offset, H, Hkv, d, scale, softcap,
                       window).reshape(T, H, d)


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("d,H,Hkv", [(128, 8, 2), (64, 9, 3), (256, 4, 2), (128, 4, 4), (64, 16, 2)])
def test_prefill_varlen_batch(backend, dtype, d, H, Hkv):
    """Three prompts of different lengths and offsets in one launch (chunked prefill)."""
    lens = [70, 1, 130]
    offs = [0, 40, 17]
    max_seq = max(o + n for o, n in zip(offs, lens))
    c = Contig(backend, dtype, 3, 2, max_seq, Hkv, d, seed=800 + d + H)
    q = synth.normal(900 + d, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    scale = 1 / np.sqrt(d)
    for layer, cap, window in [(0, None, None), (1, 30.0, None), (0, None, 21), (1, 15.0, 64)]:
        got = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, layer=layer)
        for b in range(3):
            rows = slice(q_start[b], q_start[b + 1])
            want = _oracle_prefill(c.stores[b], q[rows], offs[b], H, Hkv, d, scale, cap, window, layer)
            assert_close(got[rows], want, what=f"{dtype} d{d} H{H}/{Hkv} seq{b} layer{layer} cap{cap} w{window}")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_paged(backend, dtype, precision):
    """Paged pools; the table is 17 pages wide (272 positions, not a multiple of the 32-key
    tile), and the last sequence's last tile runs past it."""
    H, Hkv, d = 8, 2, 128
    ctx = np.array([100, 37, 260], np.int32)
    pb = synth.paged_batch(41, ctx, prefix_tokens=32)
    p = Pool(backend, dtype, pb, Hkv, d, seed=42)
    # each sequence prefills its last n positions (the first ones are "cached")
    n = np.array([60, 37, 200], np.int32)
    offs = ctx - n
    q = synth.normal(43, (int(n.sum()), H, d))
    q_start = np.concatenate([[0], np.cumsum(n)]).astype(np.int32)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    for window in (None, 40):
        got = run_prefill(backend, p.pool, q, q_start, offs, H, 0.09, None, window, table=pb.table,
                          precision=precision)
        for b in range(3):
            rows = slice(q_start[b], q_start[b + 1])
            want = _oracle_prefill(p.stores[b], q[rows], int(offs[b]), H, Hkv, d, 0.09, None, window)
            assert_close(got[rows], want, *tol, what=f"paged {dtype} {precision} seq {b} window {window}")


@pytest.mark.parametrize("d,H,Hkv", [(128, 8, 2), (64, 9, 3), (256, 4, 2), (64, 16, 2)])
@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_prefill_bf16_staged_equals_unstaged(backend, monkeypatch, dtype, d, H, Hkv):
    """The bf16 path with the tile images staged once per call (the default) and with each
    workgroup converting its own tiles (GLA_BF16_UNSTAGED) round the same values and feed the
    MFMAs in the same order: bit-identical outputs, windows and soft-cap included."""
    lens = [70, 1, 130]
    offs = [0, 40, 17]
    max_seq = max(o + n for o, n in zip(offs, lens))
    c = Contig(backend, dtype, 3, 1, max_seq, Hkv, d, seed=870 + d + H)
    q = synth.normal(970 + d, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    for cap, window in [(None, None), (20.0, 33)]:
        monkeypatch.delenv("GLA_BF16_UNSTAGED", raising=False)
        staged = run_prefill(backend, c.cache, q, q_start, offs, H, 0.1, cap, window, precision="bf16")
        monkeypatch.setenv("GLA_BF16_UNSTAGED", "1")
        unstaged = run_prefill(backend, c.cache, q, q_start, offs, H, 0.1, cap, window, precision="bf16")
        assert np.array_equal(staged.view(np.uint32), unstaged.view(np.uint32)), (dtype, d, cap, window)


@pytest.mark.parametrize("d,H,Hkv", [(128, 8, 2), (64, 9, 3), (256, 4, 2), (128, 4, 4), (64, 16, 2)])
@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_prefill_bf16_varlen_batch(backend, dtype, d, H, Hkv):
    """bf16-input variant over the varlen batch (chunked offsets, soft-cap, windows): within the
    bf16 bar of the fp32 oracle, and really rounded (not equal to the fp32 kernel's output)."""
    lens = [70, 1, 130]
    offs = [0, 40, 17]
    max_seq = max(o + n for o, n in zip(offs, lens))
    c = Contig(backend, dtype, 3, 2, max_seq, Hkv, d, seed=850 + d + H)
    q = synth.normal(950 + d, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    scale = 1 / np.sqrt(d)
    for layer, cap, window in [(0, None, None), (1, 30.0, None), (0, None, 21), (1, 15.0, 64)]:
        got = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, layer=layer, precision="bf16")
        f32 = run_prefill(backend, c.cache, q, q_start, offs, H, scale, cap, window, layer=layer)
        assert max_errors(got, f32)[0] > 0.0, "bf16 variant returned the fp32 result"
        for b in range(3):
            rows = slice(q_start[b], q_start[b + 1])
            want = _oracle_prefill(c.stores[b], q[rows], offs[b], H, Hkv, d, scale, cap, window, layer)
            assert_close(got[rows], want, BF16_ABS_TOL, BF16_REL_TOL,
                         what=f"bf16 {dtype} d{d} H{H}/{Hkv} seq{b} layer{layer} cap{cap} w{window}")


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_zero_length_prompts(backend, precision):
    """Prompts with no tokens between and around others in one launch (chunked prefill can hand
    a sequence an empty chunk): the others' rows are unaffected."""
    H, Hkv, d = 8, 2, 128
    lens = [0, 45, 0, 7, 0]
    offs = [5, 0, 30, 60, 0]
    max_seq = max(o + n for o, n in zip(offs, lens)) + 8
    c = Contig(backend, "f32", len(lens), 1, max_seq, Hkv, d, seed=611)
    q = synth.normal(612, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    for cap, window in [(None, None), (25.0, 20)]:
        got = run_prefill(backend, c.cache, q, q_start, offs, H, 0.088, cap, window, precision=precision)
        for b in range(len(lens)):
            if lens[b] == 0:
                continue
            rows = slice(q_start[b], q_start[b + 1])
            want = _oracle_prefill(c.stores[b], q[rows], offs[b], H, Hkv, d, 0.088, cap, window)
            assert_close(got[rows], want, *tol, what=f"{precision} seq {b} cap {cap} w {window}")


@pytest.mark.parametrize("dtype", ["f32", "q8"])
def test_prefill_bf16_d256_long_prompt(backend, monkeypatch, dtype):
    """head_dim 256 (the 4-tile ring: two tiles in flight behind the current one) over a long
    chunk: 700 queries after 100 cached positions, 25 tiles per query block at the end; with
    and without soft-cap and window, against the oracle at the bf16 bar and bit-identical to
    the per-workgroup path."""
    H, Hkv, d = 8, 4, 256
    lens, offs = [700], [100]
    c = Contig(backend, dtype, 1, 1, 800, Hkv, d, seed=2560)
    q = synth.normal(2561, (700, H, d))
    q_start = np.array([0, 700], np.int32)
    for cap, window in [(None, None), (50.0, None), (None, 300)]:
        monkeypatch.delenv("GLA_BF16_UNSTAGED", raising=False)
        got = run_prefill(backend, c.cache, q, q_start, offs, H, 0.0625, cap, window, precision="bf16")
        want = _oracle_prefill(c.stores[0], q, 100, H, Hkv, d, 0.0625, cap, window)
        assert_close(got, want, BF16_ABS_TOL, BF16_REL_TOL, what=f"{dtype} d256 cap {cap} w {window}")
        monkeypatch.setenv("GLA_BF16_UNSTAGED", "1")
        unstaged = run_prefill(backend, c.cache, q, q_start, offs, H, 0.0625, cap, window, precision="bf16")
        assert np.array_equal(got.view(np.uint32), unstaged.view(np.uint32)), (dtype, cap, window)


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_prefill_indexing_is_bit_exact(backend, precision):
    """K = 0 and small-integer V: out = mean of V over [window(pos), pos] exactly."""
    H, Hkv, d = 8, 2, 64
    kv_dim = Hkv * d
    T = 150
    r = np.arange(T)[:, None]
    e = np.arange(kv_dim)[None, :]
    v = (((r * 131 + e * 7) % 255) - 127).astype(np.float32).reshape(1, 1, T, kv_dim)
    c = Contig(backend, "f32", 1, 1, T, Hkv, d, k=np.zeros_like(v), v=v)
    q = synth.normal(4, (T, H, d))
    for window in (None, 16, 33):
        got = run_prefill(backend, c.cache, q, [0, T], [0], H, 0.125, None, window, precision=precision)
        for pos in range(T):
            lo = 0 if not window else max(0, pos - window + 1)
            s = v[0, 0, lo:pos + 1].astype(np.float64).sum(0).astype(np.float32)
            want = s * (np.float32(1.0) / np.float32(pos + 1 - lo))
            for h in range(H):
                kvh = h // (H // Hkv)
                assert np.array_equal(got[pos, h].view(np.uint32), want[kvh * d:(kvh + 1) * d].view(np.uint32)), \
                    (precision, window, pos, h)


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_cfg4_llama_prefill_4x2048(backend, precision):
    """BASELINE config 4 at full size (4 prompts x 2048, H32/KV8, d128, f32 KV cache): every
    query row of every prompt against the oracle's prefill loop (so every row residue of the
    kernels' 32- and 96-row query blocks and every causal-diagonal tile is compared)."""
    H, Hkv, d, S, B = 32, 8, 128, 2048, 4
    c = Contig(backend, "f32", B, 1, S, Hkv, d, seed=4004)
    q = synth.normal(4005, (B * S, H, d))
    q_start = np.arange(B + 1, dtype=np.int32) * S
    scale = 1 / np.sqrt(128)
    got = run_prefill(backend, c.cache, q, q_start, [0] * B, H, scale, precision=precision)
    tol = (BF16_ABS_TOL, BF16_REL_TOL) if precision == "bf16" else ()
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        want = _oracle_prefill(c.stores[b], q[rows], 0, H, Hkv, d, scale)
        assert_close(got[rows], want, *tol, what=f"cfg4 {precision} prompt {b}")
