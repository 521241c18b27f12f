"""Seeded synthetic inputs (Xorshift64 + Box-Muller, see csrc/synth.c) and the
BASELINE workload shapes built from them.

The same host arrays feed the GPU path and the CPU oracle, so both see
identical inputs.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import _lib

PAGE = _lib.GLA_PAGE_SIZE


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def normal_rows(seed: int, n_rows: int, row_len: int, mul: float = 1.0, row0: int = 0) -> np.ndarray:
    """[n_rows][row_len] float32, row r drawn from stream splitmix64(seed + row0 + r)."""
    out = np.empty((n_rows, row_len), dtype=np.float32)
    if n_rows and row_len:
        _lib.synth().gs_fill_normal_rows(seed, out.ctypes.data, n_rows, row_len, row0, mul, _threads())
    return out


def normal(seed: int, shape, mul: float = 1.0) -> np.ndarray:
    """One stream of N(0,1)*mul values in the given shape."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    if n:
        _lib.synth().gs_fill_normal(seed, out.ctypes.data, n, mul)
    return out.reshape(shape)


def uniform_int(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    if n:
        _lib.synth().gs_uniform_int(seed, lo, hi, n, out.ctypes.data)
    return out


def permutation(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    if n:
        _lib.synth().gs_permutation(seed, out.ctypes.data, n)
    return out


def xorshift_seq(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    if n:
        _lib.synth().gs_xorshift_seq(seed, n, out.ctypes.data)
    return out


def tensor_seed(base: int, config: int, layer: int, tensor: int) -> int:
    """Per-tensor seed: base xor (config, layer, tensor id) packed into one word."""
    return (base ^ ((config & 0xFF) << 48) ^ ((layer & 0xFFFF) << 16) ^ (tensor & 0xFFFF)) & 0xFFFFFFFFFFFFFFFF


@dataclass
class PagedBatch:
    """A batch of sequences over a page pool: the layout of BASELINE configs 3 and 5.

    table[b][lp] is the physical page of logical page lp of sequence b; the
    first `prefix_pages` logical pages of every sequence map to the same
    physical pages (a refcounted shared prefix, as PagedKvCache::fork_from
    produces, src/cache/paged.rs:293-310)."""

    ctx: np.ndarray            # int32[B] context length (the query sits at ctx-1)
    table: np.ndarray          # int32[B][max_pages]
    n_pages: int               # pool pages in use
    prefix_pages: int
    kv_start: np.ndarray = field(default=None)  # int32[B]
    kv_len: np.ndarray = field(default=None)    # int32[B]


def paged_batch(seed: int, ctx: np.ndarray, prefix_tokens: int = 0, page_base: int = 0) -> PagedBatch:
    """Page tables for sequences of lengths ctx; physical ids are a seeded permutation of
    page_base .. page_base + n_pages - 1."""
    ctx = np.asarray(ctx, dtype=np.int32)
    B = len(ctx)
    prefix_pages = (prefix_tokens + PAGE - 1) // PAGE
    need = [(int(c) + PAGE - 1) // PAGE for c in ctx]
    own = [max(0, n - prefix_pages) for n in need]
    n_pages = (prefix_pages if prefix_tokens else 0) + sum(own)
    perm = permutation(seed, n_pages) + page_base
    max_pages = max(need) if B else 1
    table = np.zeros((B, max(1, max_pages)), dtype=np.int32)
    cur = prefix_pages if prefix_tokens else 0
    for b in range(B):
        if prefix_tokens:
            table[b, :min(prefix_pages, need[b])] = perm[:min(prefix_pages, need[b])]
            start = prefix_pages
        else:
            start = 0
        n_own = need[b] - start
        if n_own > 0:
            table[b, start:need[b]] = perm[cur:cur + n_own]
            cur += n_own
    pb = PagedBatch(ctx=ctx, table=table, n_pages=n_pages, prefix_pages=prefix_pages if prefix_tokens else 0)
    pb.kv_start = np.zeros(B, dtype=np.int32)
    pb.kv_len = ctx.copy()
    return pb


def windowed(pb: PagedBatch, window: Optional[int]) -> PagedBatch:
    """The same batch attending a sliding window of the last `window` positions
    (src/transformer/forward.rs:574-582 with pos = ctx - 1)."""
    out = PagedBatch(ctx=pb.ctx, table=pb.table, n_pages=pb.n_pages, prefix_pages=pb.prefix_pages)
    if not window:
        out.kv_start = np.zeros_like(pb.ctx)
    else:
        out.kv_start = np.maximum(0, pb.ctx - 1 - window + 1).astype(np.int32)
    out.kv_len = (pb.ctx - out.kv_start).astype(np.int32)
    return out


def pool_rows(seed_k: int, seed_v: int, first_page: int, n_pages: int, kv_dim: int,
              k_mul: float = 1.0) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """K/V rows of pool pages [first_page, first_page + n_pages): row ids and N(0,1) data
    (K scaled by k_mul). Returns (rows int64[n], k f32[n][kv_dim], v f32[n][kv_dim])."""
    n = n_pages * PAGE
    rows = np.arange(first_page * PAGE, first_page * PAGE + n, dtype=np.int64)
    k = normal_rows(seed_k, n, kv_dim, k_mul, row0=first_page * PAGE)
    v = normal_rows(seed_v, n, kv_dim, 1.0, row0=first_page * PAGE)
    return rows, k, v
