"""One backend's work on two streams at once (gla_set_stream). Both a bf16 prefill (its tile
images) and a decode (its split partials) use device scratch; each stream has its own, so
calls that overlap on different streams give the same bits as when run one at a time. The
engine's single-context GpuBackend (src/backend/gpu.rs:30-39) would put a prefill chunk and
the batch's decode step on different streams this way."""
from __future__ import annotations

import numpy as np
import pytest

from glint_amd import synth
from glint_amd.attn import HipStream
from gpu_util import Contig, Pool

pytestmark = pytest.mark.gpu


def _bits(buf, shape):
    return buf.download(shape).view(np.uint32)


def test_prefill_and_decode_overlap_on_two_streams(backend):
    be = backend
    # cfg3-shaped paged Q8_0 decode
    H, Hkv, d, B = 32, 8, 128, 64
    ctx = synth.uniform_int(6101, 128, 8192, B)
    pb = synth.paged_batch(6102, ctx, prefix_tokens=256)
    p = Pool(be, "q8", pb, Hkv, d, seed=6103)
    dq = [be.buffer(synth.normal(6104 + i, (B, H, d))) for i in range(2)]
    ds, dl, dt = be.buffer(pb.kv_start), be.buffer(pb.kv_len), be.buffer(pb.table)
    # cfg4-shaped bf16 prefill: 4 x 2048 over an f32 cache
    S, P = 2048, 4
    c = Contig(be, "f32", P, 1, S, Hkv, d, seed=6105)
    pq = [be.buffer(synth.normal(6106 + i, (P * S, H, d))) for i in range(2)]
    qs, po = be.buffer(np.arange(P + 1, dtype=np.int32) * S), be.buffer(np.zeros(P, np.int32))

    dshape, pshape = (B, H, d), (P * S, H, d)

    def decode(i, out):
        be.decode(p.pool, dq[i], out, ds, dl, B, int(pb.kv_len.max()), H, 0.088, 50.0, page_table=dt,
                  page_table_stride=pb.table.shape[1], kv_start_host=pb.kv_start, kv_len_host=pb.kv_len)

    def prefill(i, out):
        be.prefill(c.cache, pq[i], out, qs, po, P, S, H, 0.088, precision="bf16")

    # one at a time on the backend's own stream
    want_d = [be.empty(int(np.prod(dshape)) * 4) for _ in range(2)]
    want_p = [be.empty(int(np.prod(pshape)) * 4) for _ in range(2)]
    for i in range(2):
        decode(i, want_d[i])
        be.sync()
        prefill(i, want_p[i])
        be.sync()
    wd = [_bits(x, dshape) for x in want_d]
    wp = [_bits(x, pshape) for x in want_p]

    s1, s2 = HipStream(), HipStream()
    got_d = [be.empty(int(np.prod(dshape)) * 4) for _ in range(2)]
    got_p = [be.empty(int(np.prod(pshape)) * 4) for _ in range(2)]
    try:
        for rep in range(3):
            # interleaved, nothing waited for: s1 prefill 0, s2 decode 0, s1 decode 1, s2 prefill 1
            be.set_stream(s1)
            prefill(0, got_p[0])
            be.set_stream(s2)
            decode(0, got_d[0])
            be.set_stream(s1)
            decode(1, got_d[1])
            be.set_stream(s2)
            prefill(1, got_p[1])
            s1.synchronize()
            s2.synchronize()
            for i in range(2):
                assert np.array_equal(_bits(got_d[i], dshape), wd[i]), (rep, "decode", i)
                assert np.array_equal(_bits(got_p[i], pshape), wp[i]), (rep, "prefill", i)
            be.set_stream(None)
            for g in got_d + got_p:  # clear the outputs on the backend's stream
                g.upload(np.zeros(g.nbytes // 4, np.float32))
    finally:
        be.set_stream(None)
        be.sync()
        s1.destroy()
        s2.destroy()
