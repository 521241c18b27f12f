"""Golden cases: small seeded attention problems whose expected outputs are
committed as fixtures (tests/golden/*.npz, written by make_golden.py from the
CPU oracle). Each case rebuilds its inputs from seeds with glint_amd.synth
(deterministic Xorshift64 + Box-Muller) and records a SHA-256 of them, so a
change in the generator shows up as a checksum mismatch rather than as a
silent change of what the fixture means.

The oracle restates Glint's CPU flash path (oracle/glint_oracle.c); the
fixtures pin it against regressions and give the GPU tests a fixed target
that does not depend on rebuilding the oracle on the GPU box.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional

import numpy as np

from glint_amd import synth

PAGE = 16


def digest(arrays: List[np.ndarray]) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


@dataclass
class DecodeCase:
    """A batched decode: K/V per sequence in a contiguous cache (table None)
    or a page pool, q [B][H][d], one window per sequence."""
    name: str
    kind: str  # "f32" or "q8"
    paged: bool
    H: int
    Hkv: int
    d: int
    scale: float
    softcap: Optional[float]
    q: np.ndarray
    k: np.ndarray  # contiguous: [B][max_seq][kv_dim]; paged: [n_pages*16][kv_dim]
    v: np.ndarray
    kv_start: np.ndarray
    kv_len: np.ndarray
    table: Optional[np.ndarray] = None
    pb: Optional[synth.PagedBatch] = None
    inputs: List[np.ndarray] = field(default_factory=list)


@dataclass
class PrefillCase:
    name: str
    kind: str
    H: int
    Hkv: int
    d: int
    scale: float
    softcap: Optional[float]
    window: Optional[int]
    q: np.ndarray  # [rows][H][d]
    q_start: np.ndarray
    pos_offset: np.ndarray
    k: np.ndarray  # [B][max_seq][kv_dim]
    v: np.ndarray
    inputs: List[np.ndarray] = field(default_factory=list)


def decode_cfg1() -> DecodeCase:
    """SmolLM-135M shape, H9/KV3 d64, f32 contiguous ctx 512."""
    H, Hkv, d, ctx = 9, 3, 64, 512
    k = synth.normal_rows(0x6C01, ctx, Hkv * d).reshape(1, ctx, Hkv * d)
    v = synth.normal_rows(0x6C02, ctx, Hkv * d).reshape(1, ctx, Hkv * d)
    q = synth.normal(0x6C03, (1, H, d))
    c = DecodeCase("decode_cfg1", "f32", False, H, Hkv, d, 0.125, None, q, k, v,
                   np.array([0], np.int32), np.array([ctx], np.int32))
    c.inputs = [q, k, v]
    return c


def decode_q8_paged() -> DecodeCase:
    """Llama-3 heads (H32/KV8 d128 at batch 5) over a permuted Q8_0 page pool with a
    48-token shared prefix, a 100-token sliding window (windows start mid-page) and a
    soft-cap of 30."""
    H, Hkv, d = 32, 8, 128
    ctx = np.array([1, 47, 48, 130, 333], np.int32)
    pb = synth.windowed(synth.paged_batch(0x6C11, ctx, prefix_tokens=48), 100)
    rows, k, v = synth.pool_rows(0x6C12, 0x6C13, 0, pb.n_pages, Hkv * d)
    q = synth.normal(0x6C14, (len(ctx), H, d))
    c = DecodeCase("decode_q8_paged", "q8", True, H, Hkv, d, float(1 / np.sqrt(d)), 30.0, q, k, v,
                   pb.kv_start, pb.kv_len, pb.table, pb)
    c.inputs = [q, k, v, pb.kv_start, pb.kv_len, pb.table]
    return c


def decode_gemma_q8() -> DecodeCase:
    """Gemma-2 heads (H16/KV8 d256), K x 3, soft-cap 50, Q8_0 contiguous cache, batch 3,
    window 64 (the sliding layer of an alternating model)."""
    H, Hkv, d, S = 16, 8, 256, 200
    B = 3
    k = synth.normal_rows(0x6C21, B * S, Hkv * d, 3.0).reshape(B, S, Hkv * d)
    v = synth.normal_rows(0x6C22, B * S, Hkv * d).reshape(B, S, Hkv * d)
    q = synth.normal(0x6C23, (B, H, d))
    ctx = np.array([200, 65, 17], np.int32)
    start = np.maximum(0, ctx - 64).astype(np.int32)
    c = DecodeCase("decode_gemma_q8", "q8", False, H, Hkv, d, 1 / 16.0, 50.0, q, k, v, start,
                   (ctx - start).astype(np.int32))
    c.inputs = [q, k, v, start]
    return c


def prefill_varlen() -> PrefillCase:
    """Three prompt chunks at offsets (chunked prefill), H4/KV2 d64, f32 cache, window 21."""
    H, Hkv, d = 4, 2, 64
    lens = [33, 1, 47]
    offs = [0, 40, 17]
    S = max(o + n for o, n in zip(offs, lens))
    B = 3
    k = synth.normal_rows(0x6C31, B * S, Hkv * d).reshape(B, S, Hkv * d)
    v = synth.normal_rows(0x6C32, B * S, Hkv * d).reshape(B, S, Hkv * d)
    q = synth.normal(0x6C33, (sum(lens), H, d))
    q_start = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    c = PrefillCase("prefill_varlen", "f32", H, Hkv, d, float(1 / np.sqrt(d)), None, 21, q, q_start,
                    np.array(offs, np.int32), k, v)
    c.inputs = [q, k, v, q_start]
    return c


def q8_codec_rows() -> np.ndarray:
    """Rows exercising KvCacheQ8::quantize_into's rules: all-zero blocks (scale 1.0),
    half-way roundings, NaN, tiny and huge magnitudes."""
    rng = np.random.default_rng(0x6C41)
    x = (rng.standard_normal((24, 128)) * 10.0 ** rng.integers(-4, 4, (24, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :8] = [127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -1.5, 2.5]
    x[2, 3] = np.nan
    x[3] = 1e-30
    x[4, 40] = -65000.0
    return x


@dataclass
class OpsCase:
    """The ops beside attention: RoPE over rows of heads (src/tensor/ops.rs:212-245) and a
    Q8_0 matvec (src/tensor/quantized.rs:587-610)."""
    name: str
    kind: str  # "rope" or "matvec"
    x: np.ndarray
    pos: Optional[np.ndarray] = None  # rope: one position per row
    head_dim: int = 0
    rot_dim: int = 0
    base: float = 0.0
    scaling: float = 1.0
    raw: Optional[np.ndarray] = None  # matvec: GGML Q8_0 bytes [rows][cols/32 x 34]
    rows: int = 0
    cols: int = 0
    inputs: List[np.ndarray] = field(default_factory=list)


def ops_rope() -> OpsCase:
    """Partial rotary (24 of 32 dimensions) with linear scaling 2, positions up to 65,535."""
    x = synth.normal(0x0B01, (4, 3, 32))
    pos = np.array([0, 17, 4095, 65535], np.int32)
    c = OpsCase("ops_rope", "rope", x, pos=pos, head_dim=32, rot_dim=24, base=500000.0, scaling=2.0)
    c.inputs = [x, pos]
    return c


def ops_matvec_q8_0() -> OpsCase:
    """A 70 x 160 Q8_0 matrix (5 blocks per row: an odd block count, and a row tile of 6) times
    5 vectors (the vector-ALU path's limit is 4: this takes the MFMA path)."""
    import oracle as orc

    w = synth.normal_rows(0x0B02, 70, 160)
    raw = orc.q8_quantize_rows(w).reshape(-1)
    x = synth.normal(0x0B03, (5, 160))
    c = OpsCase("ops_matvec_q8_0", "matvec", x, raw=raw, rows=70, cols=160)
    c.inputs = [raw, x]
    return c


DECODE_CASES: Dict[str, Callable[[], DecodeCase]] = {
    "decode_cfg1": decode_cfg1,
    "decode_q8_paged": decode_q8_paged,
    "decode_gemma_q8": decode_gemma_q8,
}
PREFILL_CASES: Dict[str, Callable[[], PrefillCase]] = {
    "prefill_varlen": prefill_varlen,
}
OPS_CASES: Dict[str, Callable[[], OpsCase]] = {
    "ops_rope": ops_rope,
    "ops_matvec_q8_0": ops_matvec_q8_0,
}


# ---- the oracle's answers (what make_golden.py stores) ----------------------
def oracle_decode(c: DecodeCase) -> np.ndarray:
    import oracle as orc

    B = c.q.shape[0]
    kv_dim = c.Hkv * c.d
    if c.paged:
        pk = c.k.reshape(-1, PAGE, kv_dim)
        pv = c.v.reshape(-1, PAGE, kv_dim)
        if c.kind == "q8":
            kq, vq = orc.q8_quantize_rows(pk), orc.q8_quantize_rows(pv)
            stores = [orc.paged_q8(kq, vq, kv_dim, c.table[b:b + 1]) for b in range(B)]
        else:
            stores = [orc.paged_f32(pk, pv, c.table[b:b + 1]) for b in range(B)]
    elif c.kind == "q8":
        kq, vq = orc.q8_quantize_rows(c.k), orc.q8_quantize_rows(c.v)
        stores = [orc.kv_cache_q8(kq[b][None], vq[b][None], kv_dim) for b in range(B)]
    else:
        stores = [orc.kv_cache(c.k[b][None], c.v[b][None]) for b in range(B)]
    out = orc.decode_batch(c.q.reshape(B, -1), stores, 0, c.kv_start, c.kv_len, c.H, c.Hkv, c.d, c.scale,
                           c.softcap)
    return out.reshape(c.q.shape).astype(np.float32)


def oracle_prefill(c: PrefillCase) -> np.ndarray:
    import oracle as orc

    out = np.zeros_like(c.q)
    for b in range(len(c.pos_offset)):
        r0, r1 = int(c.q_start[b]), int(c.q_start[b + 1])
        st = orc.kv_cache(c.k[b][None], c.v[b][None])
        out[r0:r1] = orc.prefill(c.q[r0:r1].reshape(r1 - r0, -1), st, 0, int(c.pos_offset[b]), c.H, c.Hkv, c.d,
                                 c.scale, c.softcap, c.window).reshape(r1 - r0, c.H, c.d)
    return out


def oracle_ops(c: OpsCase) -> np.ndarray:
    import oracle as orc

    if c.kind == "rope":
        return np.stack([orc.rope(c.x[r].reshape(-1), int(c.pos[r]), c.head_dim, c.base, c.scaling,
                                  c.rot_dim).reshape(c.x.shape[1:]) for r in range(c.x.shape[0])]).astype(np.float32)
    return np.stack([orc.matvec_q8_0(c.raw, c.rows, c.cols, c.x[v]) for v in range(c.x.shape[0])]).astype(np.float32)
