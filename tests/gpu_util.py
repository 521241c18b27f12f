"""Builders shared by the GPU tests: the same seeded host arrays go into a device
cache/pool (through the C ABI) and into oracle stores."""
from __future__ import annotations

import numpy as np

import oracle as orc
from glint_amd import synth

PAGE = 16
CHUNK_ROWS = 1 << 16


def write_rows_chunked(kv, rows, k, v):
    for i in range(0, len(rows), CHUNK_ROWS):
        kv.write_rows(rows[i:i + CHUNK_ROWS], k[i:i + CHUNK_ROWS], v[i:i + CHUNK_ROWS])


def contig_row_ids(n_seqs, n_layers, max_seq):
    """Row ids of every (seq, layer, pos) of a contiguous cache, [n_seqs][n_layers][max_seq]."""
    ppl = (max_seq + PAGE - 1) // PAGE
    s = np.arange(n_seqs)[:, None, None]
    layer = np.arange(n_layers)[None, :, None]
    p = np.arange(max_seq)[None, None, :]
    return (((s * n_layers + layer) * ppl) * PAGE + p).astype(np.int64)


class Contig:
    """A device contiguous cache and its oracle twins, from seeded N(0,1) data."""

    def __init__(self, be, dtype, n_seqs, n_layers, max_seq, n_kv, d, seed=1, k_mul=1.0, k=None, v=None):
        kv_dim = n_kv * d
        n = n_seqs * n_layers * max_seq
        if k is None:
            k = synth.normal_rows(seed, n, kv_dim, k_mul).reshape(n_seqs, n_layers, max_seq, kv_dim)
            v = synth.normal_rows(seed + 1000003, n, kv_dim).reshape(n_seqs, n_layers, max_seq, kv_dim)
        self.k, self.v = k, v
        self.cache = be.create_kv_cache(n_layers, max_seq, n_kv, d, dtype, n_seqs)
        rows = contig_row_ids(n_seqs, n_layers, max_seq)
        assert self.cache.row_id(n_seqs - 1, n_layers - 1, max_seq - 1) == rows[-1, -1, -1]
        write_rows_chunked(self.cache, rows.reshape(-1), k.reshape(n, kv_dim), v.reshape(n, kv_dim))
        if dtype == "f32":
            self.stores = [orc.kv_cache(k[s], v[s]) for s in range(n_seqs)]
        else:
            kq = orc.q8_quantize_rows(k)
            vq = orc.q8_quantize_rows(v)
            self.stores = [orc.kv_cache_q8(kq[s], vq[s], kv_dim) for s in range(n_seqs)]


class Pool:
    """A device page pool holding a PagedBatch and per-sequence oracle stores."""

    def __init__(self, be, dtype, pb: synth.PagedBatch, n_kv, d, seed=2, k_mul=1.0, k=None, v=None):
        kv_dim = n_kv * d
        if k is None:
            rows, k, v = synth.pool_rows(seed, seed + 7777, 0, pb.n_pages, kv_dim, k_mul)
        else:
            rows = np.arange(pb.n_pages * PAGE, dtype=np.int64)
        self.k, self.v = k, v
        self.pool = be.create_page_pool(pb.n_pages, n_kv, d, dtype)
        write_rows_chunked(self.pool, rows, k, v)
        pk = k.reshape(pb.n_pages, PAGE, kv_dim)
        pv = v.reshape(pb.n_pages, PAGE, kv_dim)
        if dtype == "f32":
            self.stores = [orc.paged_f32(pk, pv, pb.table[b:b + 1]) for b in range(len(pb.ctx))]
        else:
            kq = orc.q8_quantize_rows(pk)
            vq = orc.q8_quantize_rows(pv)
            self.stores = [orc.paged_q8(kq, vq, kv_dim, pb.table[b:b + 1]) for b in range(len(pb.ctx))]


def run_decode(be, kv, q, kv_start, kv_len, n_heads, scale, softcap=None, layer=0, table=None, seq_slot=None,
               host_lengths=True):
    """gla_decode through device buffers; q [B][H][d] host -> out [B][H][d] host. host_lengths:
    also pass the host copies of kv_start / kv_len (they only size the launch)."""
    B = q.shape[0]
    dq = be.buffer(np.ascontiguousarray(q, np.float32))
    dout = be.empty(q.nbytes)
    ds = be.buffer(np.asarray(kv_start, np.int32))
    dl = be.buffer(np.asarray(kv_len, np.int32))
    kw = {}
    if table is not None:
        kw["page_table"] = be.buffer(np.ascontiguousarray(table, np.int32))
        kw["page_table_stride"] = table.shape[1]
    if seq_slot is not None:
        kw["seq_slot"] = be.buffer(np.asarray(seq_slot, np.int32))
    if host_lengths:
        kw["kv_start_host"] = np.asarray(kv_start, np.int32)
        kw["kv_len_host"] = np.asarray(kv_len, np.int32)
    be.decode(kv, dq, dout, ds, dl, B, int(np.max(kv_len)) if B else 0, n_heads, scale, softcap, layer=layer, **kw)
    be.sync()
    return dout.download(q.shape)


def run_prefill(be, kv, q, q_start, pos_offset, n_heads, scale, softcap=None, sliding_window=None, layer=0,
                table=None, seq_slot=None, precision="f32"):
    """gla_prefill through device buffers; q [rows][H][d] host -> out [rows][H][d] host."""
    dq = be.buffer(np.ascontiguousarray(q, np.float32))
    dout = be.empty(q.nbytes)
    qs = np.asarray(q_start, np.int32)
    dqs = be.buffer(qs)
    dpo = be.buffer(np.asarray(pos_offset, np.int32))
    kw = {}
    if table is not None:
        kw["page_table"] = be.buffer(np.ascontiguousarray(table, np.int32))
        kw["page_table_stride"] = table.shape[1]
    if seq_slot is not None:
        kw["seq_slot"] = be.buffer(np.asarray(seq_slot, np.int32))
    be.prefill(kv, dq, dout, dqs, dpo, len(qs) - 1, int(np.max(np.diff(qs))), n_heads, scale, softcap,
               sliding_window, layer=layer, precision=precision, **kw)
    be.sync()
    return dout.download(q.shape)
