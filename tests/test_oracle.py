"""Pins the CPU oracle (oracle/glint_oracle.c) before anything is checked against it.

Each check_* takes an oracle library handle, so the same check runs on the real
oracle (must pass) and on builds with a planted mistake (must fail):
  - the reference's own fixtures (src/tensor/flash.rs:180-232, src/cache/mod.rs:651-702,
    src/cache/paged.rs:617-707, src/tensor/dequantize.rs:717-748);
  - known answers (round half away from zero, zero-block scale 1.0, L=1, identical keys);
  - the textbook: float64 brute-force softmax attention;
  - invariants: paged == contiguous bitwise, batch == single bitwise, attend_len = min(pos+1, w);
  - numpy's IEEE float16 conversion for the f16 codec (half 2.7.1 is round-to-nearest-even).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from helpers import attention_f64

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- f16 codec
def check_f16(L):
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 5.96e-08, 2.98e-08,
                  2.99e-08, 1.0 / 127.0, 127.0 / 127.0, 1e-40], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):  # values past 65519.99 round to infinity, as they should
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([orc.f16_from_f32(float(v), L) for v in x], dtype=np.uint16)
    bad = np.nonzero(got != want)[0]
    assert len(bad) == 0, f"f16_from_f32 differs from IEEE RNE at {x[bad[:5]]}: {got[bad[:5]]} vs {want[bad[:5]]}"
    codes = np.arange(65536, dtype=np.uint16)
    back = np.array([orc.f16_to_f32(int(c), L) for c in codes], dtype=np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(back), nan)
    assert np.array_equal(back[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_matches_ieee_rne():
    check_f16(orc.lib())


# ---------------------------------------------------------------- Q8_0 codec
def check_q8_known_answers(L):
    # max 127 -> d = 1 exactly, so x * (1/d) = x and rounding is visible.
    blk = np.zeros(32, np.float32)
    blk[:9] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.4999, -126.5]
    row = orc.q8_quantize_rows(blk, L)
    assert row.shape == (34,)
    assert row[0] == 0x00 and row[1] == 0x3C, "scale must be f16(1.0)"
    q = row[2:].view(np.int8)
    assert list(q[:9]) == [127, 3, -3, 1, -1, 2, -2, 3, -127], f"round half away from zero: {list(q[:9])}"
    # all-zero block stores scale 1.0 (src/cache/mod.rs:303) and zero quants
    z = orc.q8_quantize_rows(np.zeros(32, np.float32), L)
    assert z[0] == 0x00 and z[1] == 0x3C and not z[2:].any()
    # partial last block is zero padded; NaN quantises to 0 and is skipped by the max
    x = np.arange(40, dtype=np.float32) - 20.0
    x[3] = np.nan
    r = orc.q8_quantize_rows(x, L)
    assert r.shape == (68,)
    assert r[2 + 3] == 0
    assert not r[34 + 2 + 8:].any()
    assert abs(r[2:34].view(np.int8)).max() == 127


def test_q8_known_answers():
    check_q8_known_answers(orc.lib())


def check_q8_roundtrip(L):
    # src/cache/mod.rs:651-671: head_dim 32, one block each for K and V, error < 0.12
    k = np.arange(32, dtype=np.float32) * 0.5 - 8.0
    v = np.arange(32, dtype=np.float32) * 0.3 + 1.0
    for x in (k, v):
        dq = orc.q8_dequant_range(orc.q8_quantize_rows(x, L), 0, 32, L)
        assert np.max(np.abs(dq - x)) < 0.12
    # src/cache/mod.rs:687-702: 2 heads, read head 1
    kk = np.arange(64, dtype=np.float32) * 0.1
    h1 = orc.q8_dequant_range(orc.q8_quantize_rows(kk, L), 32, 64, L)
    assert np.max(np.abs(h1 - kk[32:])) < 0.12
    # random rows: error within half a step of the f16 scale, plus the scale's own rounding
    x = RNG.standard_normal((200, 128)).astype(np.float32) * 3
    rows = orc.q8_quantize_rows(x, L)
    for r in range(0, 200, 7):
        dq = orc.q8_dequant_range(rows[r], 0, 128, L)
        for b in range(4):
            blk = x[r, 32 * b:32 * b + 32]
            d = np.abs(blk).max() / 127.0
            d16 = float(np.float32(d).astype(np.float16))
            bound = 0.5 * d16 + 127.0 * abs(d16 - d) + 1e-6
            assert np.max(np.abs(dq[32 * b:32 * b + 32] - blk)) <= bound


def test_q8_roundtrip_reference_fixtures():
    check_q8_roundtrip(orc.lib())


def test_q8_dequant_scale_two():
    # src/tensor/dequantize.rs:717-748: scale f16(2.0), quants 0, 0, 1, -1, 2, -2, ...
    quants = np.array([(i // 2) if i % 2 == 0 else -(i // 2) for i in range(32)], dtype=np.int8)
    h = orc.f16_from_f32(2.0)
    row = np.concatenate([np.array([h & 0xFF, h >> 8], np.uint8), quants.view(np.uint8)])
    out = orc.q8_dequant_range(row, 0, 32)
    assert np.array_equal(out, quants.astype(np.float32) * 2.0)


def test_q8_compression_ratio():
    # src/cache/mod.rs:673-685: 4 heads x 32 -> ratio in [3.5, 4.0]
    kv_dim = 4 * 32
    ratio = (kv_dim * 4) / orc.q8_row_bytes(kv_dim)
    assert 3.5 < ratio < 4.0


# ---------------------------------------------------------------- flash attention
def _ramp_cache(seq_len, head_dim, n_kv_heads):
    kv_dim = n_kv_heads * head_dim
    idx = np.arange(seq_len * kv_dim, dtype=np.float32).reshape(1, seq_len, kv_dim)
    k = idx * np.float32(0.1) - np.float32(0.5)
    v = idx * np.float32(0.07) + np.float32(0.1)
    return k, v


@pytest.mark.parametrize("seq_len,head_dim,n_kv", [(64, 4, 2), (50, 4, 2), (1, 4, 2), (35, 128, 1)])
def test_flash_vs_standard_reference_shapes(seq_len, head_dim, n_kv):
    """src/tensor/flash.rs:180-232, same closed-form ramp inputs, abs < 1e-4."""
    k, v = _ramp_cache(seq_len, head_dim, n_kv)
    st = orc.kv_cache(k, v)
    q = np.arange(head_dim, dtype=np.float32) * np.float32(0.05) - np.float32(0.1)
    scale = 1.0 / np.sqrt(np.float32(head_dim))
    want = orc.standard_attn(q, st, 0, 0, 0, seq_len, head_dim, scale)
    got = orc.flash_attn_1d_ext(q, st, 0, 0, 0, seq_len, head_dim, scale)
    assert np.max(np.abs(want - got)) < 1e-4


def check_flash_f64(L):
    rng = np.random.default_rng(11)
    for d, n_kv, seq, start, span in [(4, 2, 37, 0, 37), (64, 3, 200, 17, 150), (128, 2, 600, 0, 600),
                                      (256, 1, 90, 33, 40), (128, 1, 1, 0, 1)]:
        k = rng.standard_normal((1, seq, n_kv * d)).astype(np.float32)
        v = rng.standard_normal((1, seq, n_kv * d)).astype(np.float32)
        st = orc.kv_cache(k, v, L=L)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        for kv_h in range(n_kv):
            q = rng.standard_normal(d).astype(np.float32)
            got = orc.flash_attn_1d_ext(q, st, 0, kv_h, start, span, d, scale)
            K = k[0, start:start + span, kv_h * d:(kv_h + 1) * d]
            V = v[0, start:start + span, kv_h * d:(kv_h + 1) * d]
            want = attention_f64(q, K, V, scale)
            assert np.max(np.abs(got - want)) < 2e-5, (d, seq, kv_h)


def test_flash_vs_f64():
    check_flash_f64(orc.lib())


def check_softcap_f64(L):
    rng = np.random.default_rng(12)
    d, seq = 256, 300
    k = (rng.standard_normal((1, seq, d)) * 3).astype(np.float32)  # K x 3 so the cap bites (cfg 5)
    v = rng.standard_normal((1, seq, d)).astype(np.float32)
    st = orc.kv_cache(k, v, L=L)
    q = (rng.standard_normal(d) * 8).astype(np.float32)
    scale = 1.0 / 16.0
    for cap in (50.0, 5.0):
        got = orc.flash_attn_1d_ext(q, st, 0, 0, 0, seq, d, scale, softcap=cap)
        want = attention_f64(q, k[0], v[0], scale, softcap=cap)
        assert np.max(np.abs(got - want)) < 5e-5, cap
    # a cap far above every score is the uncapped result
    got = orc.flash_attn_1d_ext(q, st, 0, 0, 0, seq, d, scale, softcap=1e7)
    assert np.max(np.abs(got - attention_f64(q, k[0], v[0], scale))) < 5e-5


def test_softcap_vs_f64():
    check_softcap_f64(orc.lib())


def test_softcap_known_answers():
    """The reference's soft-cap known answers (src/tensor/ops.rs:457-471, cap 50: 0 -> 0,
    +-50 -> +-50 tanh(1), +-1000 -> +-50) through flash_attn_1d_ext: two positions a, b with
    scores s_a, s_b (q = e_0, k = s e_0, scale 1), V_a = 0 and V_b = M e_1, so out[1] =
    M / (1 + exp(cap(s_a) - cap(s_b))) with the known capped values; M makes out[1] ~0.1, so
    a capped score off by 1e-4 moves out[1] by 1e-4 relative, and an uncapped 1000 sends it to
    0. (The GPU kernels are checked on the same construction.)"""
    d = 64
    known = {0.0: 0.0, 5.0: 50.0 * np.tanh(0.1), 50.0: 50.0 * np.tanh(1.0), -50.0: -50.0 * np.tanh(1.0),
             1000.0: 50.0, -1000.0: -50.0}
    for sa, sb in [(1000.0, 50.0), (-50.0, -1000.0), (0.0, 5.0), (-1000.0, 1000.0)]:
        k = np.zeros((1, 2, d), np.float32)
        v = np.zeros_like(k)
        k[0, 0, 0], k[0, 1, 0] = sa, sb
        ratio = np.exp(known[sa] - known[sb])
        M = min(1e4, 0.1 * (1.0 + ratio))
        v[0, 1, 1] = M
        st = orc.kv_cache(k, v)
        got = orc.flash_attn_1d_ext(np.eye(d, dtype=np.float32)[0], st, 0, 0, 0, 2, d, 1.0, softcap=50.0)
        want = M / (1.0 + ratio)
        assert want > 0.05
        assert abs(got[1] - want) <= 1e-5 * want, (sa, sb, got[1], want)
        assert not np.delete(got, 1).any()


def test_flash_special_cases():
    rng = np.random.default_rng(13)
    d = 64
    k = rng.standard_normal((1, 50, d)).astype(np.float32)
    v = rng.standard_normal((1, 50, d)).astype(np.float32)
    st = orc.kv_cache(k, v)
    q = rng.standard_normal(d).astype(np.float32)
    # L = 1: out == v exactly
    for pos in (0, 17, 49):
        out = orc.flash_attn_1d_ext(q, st, 0, 0, pos, 1, d, 0.125)
        assert np.array_equal(out, v[0, pos])
    # identical keys: out == mean(V)
    k2 = np.repeat(k[:, :1], 50, axis=1)
    st2 = orc.kv_cache(k2, v)
    out = orc.flash_attn_1d_ext(q, st2, 0, 0, 0, 50, d, 0.125)
    assert np.max(np.abs(out - v[0].astype(np.float64).mean(0))) < 1e-6
    # L = 0: the pre-zeroed output stays zero
    assert not orc.flash_attn_1d_ext(q, st, 0, 0, 5, 0, d, 0.125).any()


def check_gqa_f64(L):
    rng = np.random.default_rng(14)
    H, Hkv, d, seq = 8, 2, 64, 70
    k = rng.standard_normal((1, seq, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((1, seq, Hkv * d)).astype(np.float32)
    st = orc.kv_cache(k, v, L=L)
    q = rng.standard_normal(H * d).astype(np.float32)
    out = orc.attn_heads_cpu(q, st, 0, 0, seq, H, H // Hkv, d, 0.125)
    for h in range(H):
        kvh = h // (H // Hkv)
        want = attention_f64(q[h * d:(h + 1) * d], k[0, :, kvh * d:(kvh + 1) * d], v[0, :, kvh * d:(kvh + 1) * d],
                             0.125)
        assert np.max(np.abs(out[h * d:(h + 1) * d] - want)) < 2e-5, h


def test_gqa_head_mapping_vs_f64():
    check_gqa_f64(orc.lib())


# ---------------------------------------------------------------- window rule
def check_window(L):
    for w in (1, 4, 16, 4096):
        for pos in range(0, 5000, 37):
            ws = orc.window_start(pos, w, False, 0, L)
            assert ws >= 0 and pos + 1 - ws == min(pos + 1, w), (pos, w, ws)
            # alternating (Gemma-2): odd layers are global, even layers windowed
            assert orc.window_start(pos, w, True, 1, L) == 0
            assert orc.window_start(pos, w, True, 2, L) == ws
    for pos in (0, 1, 100):
        assert orc.window_start(pos, None, False, 0, L) == 0


def test_window_rule():
    check_window(orc.lib())


# ---------------------------------------------------------------- paged storage
N_LAYERS, N_KV, HD = 2, 2, 4
KVD = N_KV * HD


def _row(tag, pos):
    """src/cache/paged.rs:617-622: tag + pos*0.25 + d*0.0625."""
    return np.array([tag + pos * 0.25 + d * 0.0625 for d in range(KVD)], np.float32)


def _paged_from_rows(k_rows, v_rows, rng):
    """Scatter per-layer rows [layer][pos][kv_dim] into randomly numbered pages."""
    n_layers, n_pos, kv_dim = k_rows.shape
    n_lp = (n_pos + 15) // 16
    perm = rng.permutation(n_layers * n_lp).astype(np.int32)
    table = perm.reshape(n_layers, n_lp)
    pk = np.zeros((n_layers * n_lp, 16, kv_dim), k_rows.dtype)
    pv = np.zeros_like(pk)
    for layer in range(n_layers):
        for pos in range(n_pos):
            pk[table[layer, pos // 16], pos % 16] = k_rows[layer, pos]
            pv[table[layer, pos // 16], pos % 16] = v_rows[layer, pos]
    return pk, pv, table


def check_paged_bitwise(L):
    rng = np.random.default_rng(15)
    seq = 37  # spans 3 pages, last one partial
    k = np.stack([np.stack([_row(float(layer), p) for p in range(seq)]) for layer in range(N_LAYERS)])
    v = np.stack([np.stack([_row(100.0 + layer, p) for p in range(seq)]) for layer in range(N_LAYERS)])
    plain = orc.kv_cache(k, v, L=L)
    pk, pv, table = _paged_from_rows(k, v, rng)
    paged = orc.paged_f32(pk, pv, table, L=L)
    q = np.arange(HD, dtype=np.float32) * np.float32(0.3) - np.float32(0.4)
    scale = float(1.0 / np.sqrt(np.float32(HD)))
    for layer in range(N_LAYERS):
        for kvh in range(N_KV):
            want = orc.flash_attn_1d_ext(q, plain, layer, kvh, 0, seq, HD, scale)
            got = orc.flash_attn_1d_ext(q, paged, layer, kvh, 0, seq, HD, scale)
            assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), (layer, kvh)
            for pos in range(seq):
                assert np.array_equal(plain.read_k_head(layer, pos, kvh, HD), paged.read_k_head(layer, pos, kvh, HD))
    # src/cache/paged.rs:687-707: window starting mid-page (13, span 21), head 1
    q2 = np.arange(HD, dtype=np.float32) * np.float32(0.1)
    want = orc.flash_attn_1d_ext(q2, plain, 0, 1, 13, 21, HD, scale)
    got = orc.flash_attn_1d_ext(q2, paged, 0, 1, 13, 21, HD, scale)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))


def test_paged_matches_contiguous_bitwise():
    check_paged_bitwise(orc.lib())


def test_paged_q8_matches_q8_bitwise():
    """The paged-Q8 composition reads exactly the KvCacheQ8 rows."""
    rng = np.random.default_rng(16)
    H, Hkv, d, seq = 8, 2, 64, 83
    kf = rng.standard_normal((1, seq, Hkv * d)).astype(np.float32)
    vf = rng.standard_normal((1, seq, Hkv * d)).astype(np.float32)
    kq = orc.q8_quantize_rows(kf)
    vq = orc.q8_quantize_rows(vf)
    plain = orc.kv_cache_q8(kq, vq, Hkv * d)
    pk, pv, table = _paged_from_rows(kq, vq, rng)
    paged = orc.paged_q8(pk, pv, Hkv * d, table)
    q = rng.standard_normal(H * d).astype(np.float32)
    for (ws, al) in [(0, seq), (21, 40), (64, 19)]:
        a = orc.attn_heads_cpu(q, plain, 0, ws, al, H, H // Hkv, d, 0.125)
        b = orc.attn_heads_cpu(q, paged, 0, ws, al, H, H // Hkv, d, 0.125)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------- batch and prefill loops
def test_batch_equals_single_bitwise():
    """src/transformer/forward.rs:1960-2002: a sequence decodes the same alone or in a batch."""
    rng = np.random.default_rng(17)
    H, Hkv, d = 4, 2, 64
    stores, lens = [], [1, 17, 64, 100]
    for n in lens:
        k = rng.standard_normal((1, n, Hkv * d)).astype(np.float32)
        v = rng.standard_normal((1, n, Hkv * d)).astype(np.float32)
        stores.append(orc.kv_cache(k, v))
    q = rng.standard_normal((len(lens), H * d)).astype(np.float32)
    ks = np.array([0, 3, 10, 0])
    kl = np.array(lens) - ks
    out = orc.decode_batch(q, stores, 0, ks, kl, H, Hkv, d, 0.125, n_threads=3)
    for s, st in enumerate(stores):
        single = orc.attn_heads_cpu(q[s], st, 0, int(ks[s]), int(kl[s]), H, H // Hkv, d, 0.125)
        assert np.array_equal(out[s].view(np.uint32), single.view(np.uint32))


def check_prefill_f64(L):
    rng = np.random.default_rng(18)
    H, Hkv, d, T, off = 4, 2, 64, 40, 9
    n = off + T
    k = rng.standard_normal((1, n, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((1, n, Hkv * d)).astype(np.float32)
    st = orc.kv_cache(k, v, L=L)
    q = rng.standard_normal((T, H * d)).astype(np.float32)
    for w in (None, 7):
        out = orc.prefill(q, st, 0, off, H, Hkv, d, 0.125, sliding_window=w, n_threads=4)
        for lp in range(T):
            pos = off + lp
            lo = 0 if not w else max(0, pos - w + 1)
            for h in range(H):
                kvh = h // (H // Hkv)
                want = attention_f64(q[lp, h * d:(h + 1) * d], k[0, lo:pos + 1, kvh * d:(kvh + 1) * d],
                                     v[0, lo:pos + 1, kvh * d:(kvh + 1) * d], 0.125)
                assert np.max(np.abs(out[lp, h * d:(h + 1) * d] - want)) < 2e-5, (w, lp, h)


def test_prefill_vs_f64():
    check_prefill_f64(orc.lib())


def test_prefill_equals_per_position_decode_bitwise():
    """forward.rs:1722-1766: prefill gives what decoding position by position gives."""
    rng = np.random.default_rng(19)
    H, Hkv, d, T = 6, 3, 64, 33
    k = rng.standard_normal((1, T, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((1, T, Hkv * d)).astype(np.float32)
    st = orc.kv_cache(k, v)
    q = rng.standard_normal((T, H * d)).astype(np.float32)
    out = orc.prefill(q, st, 0, 0, H, Hkv, d, 0.125, softcap=30.0, sliding_window=10, n_threads=4)
    for lp in range(T):
        ws = orc.window_start(lp, 10, False, 0)
        single = orc.attn_heads_cpu(q[lp], st, 0, ws, lp + 1 - ws, H, H // Hkv, d, 0.125, softcap=30.0)
        assert np.array_equal(out[lp].view(np.uint32), single.view(np.uint32))


# ---------------------------------------------------------------- planted mistakes are caught
MUTANT_CHECKS = {
    1: [check_flash_f64],                   # dropped rescale of the accumulator
    2: [check_gqa_f64, check_prefill_f64],  # GQA head map h % G
    3: [check_window],                      # window off by one
    4: [check_f16],                         # f16 truncation instead of RNE
    5: [check_q8_known_answers],            # round half to even
    6: [check_paged_bitwise],               # paged slot index shifted
    7: [check_softcap_f64],                 # soft-cap without the divide
    8: [check_q8_roundtrip],                # scale bytes read big-endian
    9: [check_prefill_f64],                 # prefill drops its own position
    10: [check_flash_f64],                  # scale applied twice
}


@pytest.mark.parametrize("mutant", sorted(MUTANT_CHECKS))
def test_planted_mistake_is_caught(mutant, tmp_path_factory):
    L = orc.build_mutant(mutant, tmp_path_factory.mktemp("mutants"))
    for check in MUTANT_CHECKS[mutant]:
        with pytest.raises(AssertionError):
            check(L)


# ---- RoPE (src/tensor/ops.rs:212-245) and Q8_0 matvec (src/tensor/quantized.rs:587-610) ----

def _rope_f64(x, pos, head_dim, base, scaling, rot_dim):
    """The rotation in float64: every head's adjacent pair (i, i+1) by (pos/scaling) * base^(-i/d)."""
    x = np.asarray(x, np.float64).reshape(-1, head_dim).copy()
    out = x.copy()
    rot = min(rot_dim, head_dim) & ~1
    for i in range(0, rot, 2):
        a = (pos / scaling) * base ** (-i / head_dim)
        c, s = np.cos(a), np.sin(a)
        out[:, i] = x[:, i] * c - x[:, i + 1] * s
        out[:, i + 1] = x[:, i] * s + x[:, i + 1] * c
    return out.reshape(-1)


def test_rope_reference_known_answers():
    """ops.rs tests: position 0 is the identity (full and partial rotary), and pos 2 with
    scaling 2 equals pos 1 with scaling 1 bit for bit (both angles are exactly 1.0 x freq)."""
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    assert np.array_equal(orc.rope(x, 0, 4, 10000.0, 1.0, 4), x)
    assert np.array_equal(orc.rope(x, 0, 4, 10000.0, 1.0, 2), x)
    assert np.array_equal(orc.rope(x, 2, 4, 10000.0, 2.0, 4), orc.rope(x, 1, 4, 10000.0, 1.0, 4))


@pytest.mark.parametrize("head_dim,rot_dim,scaling", [(64, 64, 1.0), (128, 128, 1.0), (128, 64, 1.0),
                                                      (128, 65, 1.0), (96, 96, 4.0)])
def test_rope_vs_f64(head_dim, rot_dim, scaling):
    """Against the float64 rotation at positions up to 8191 (angles up to ~8,000 rad: the f32
    angle's own rounding dominates, ~1e-3 rad there, so the bound grows with pos); dimensions
    past rot_dim (rounded down to even) are copied bit for bit; every rotated pair keeps its
    length."""
    rng = np.random.default_rng(head_dim + rot_dim)
    x = rng.standard_normal(3 * head_dim).astype(np.float32)
    rot = min(rot_dim, head_dim) & ~1
    for pos in (0, 1, 17, 511, 4095, 8191):
        got = orc.rope(x, pos, head_dim, 500000.0, scaling, rot_dim)
        want = _rope_f64(x, pos, head_dim, 500000.0, scaling, rot_dim)
        tol = 1e-5 + 4e-7 * pos / scaling
        assert np.abs(got - want).max() <= tol * np.abs(x).max() * 2, (pos, np.abs(got - want).max())
        g = got.reshape(-1, head_dim)
        xx = x.reshape(-1, head_dim)
        assert np.array_equal(g[:, rot:], xx[:, rot:])
        n_got = np.hypot(g[:, 0:rot:2], g[:, 1:rot:2])
        n_x = np.hypot(xx[:, 0:rot:2], xx[:, 1:rot:2])
        assert np.allclose(n_got, n_x, rtol=1e-6, atol=1e-6)


def test_matvec_q8_0_reference_fixture():
    """quantized.rs test_q8_0_matvec_matches_f32: rows [0..31] x scale 1 and [0..-31] x scale 2
    against vec [0..31] give sum(i^2) = 10416 and -2 * 10416 (within 0.1, the reference's bar;
    here exactly, all products and sums being integers below 2^24)."""
    data = orc.q8_0_block(1.0, range(32)) + orc.q8_0_block(2.0, [-i for i in range(32)])
    got = orc.matvec_q8_0(np.frombuffer(data, np.uint8), 2, 32, np.arange(32, dtype=np.float32))
    assert got.tolist() == [10416.0, -20832.0]


def test_matvec_q8_0_multi_block_vs_f64():
    """quantized.rs test_q8_0_simd_matches_scalar's 4 x 128 fixture (quants (r*4+b)*(j+1) as
    wrapping i8, scale 0.1*(r+1), vec i*0.01) and random 64 x 512 rows, against the float64
    product of the dequantised rows (scales as stored in f16)."""
    data = b""
    for r in range(4):
        for b in range(4):
            q = [np.int8(np.uint8(((r * 4 + b) * (j + 1)) & 0xFF).view(np.int8)) for j in range(32)]
            data += orc.q8_0_block(0.1 * (r + 1), q)
    vec = (np.arange(128) * 0.01).astype(np.float32)
    for raw, rows, cols, v in [(np.frombuffer(data, np.uint8), 4, 128, vec), _random_q8(64, 512, 5)]:
        got = orc.matvec_q8_0(raw, rows, cols, v)
        want = _q8_dequant_rows(raw, rows, cols) @ v.astype(np.float64)
        mag = np.abs(_q8_dequant_rows(raw, rows, cols)) @ np.abs(v.astype(np.float64))
        assert np.all(np.abs(got - want) <= 1e-6 * mag + 1e-6)


def _q8_dequant_rows(raw, rows, cols):
    blk = raw.reshape(rows, cols // 32, 34)
    scale = blk[:, :, :2].copy().view("<f2").astype(np.float64)
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    return (q * scale).reshape(rows, cols)


def _random_q8(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    raw = orc.q8_quantize_rows(w).reshape(-1)
    return raw, rows, cols, rng.standard_normal(cols).astype(np.float32)
