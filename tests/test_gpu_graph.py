"""HIP graph capture of library calls (GpuBackend.capture): a decode step's calls -- a paged
Q8_0 batch decode, three layers of a contiguous f32 decode, a Q8_0 projection and RoPE on its
output -- captured once and replayed. Between replays new inputs are uploaded, the sequences'
device lengths grow (as they do from one decode step to the next), and the same calls run
eagerly into other buffers; every replay equals the eager calls bit for bit (the kernels are
deterministic, and the graph must read the buffers' current contents). The captured decode is
sized for the page table's capacity and passes no host lengths (the eager one passes them, as
the engine does); a capture with host lengths is refused. Before the last replays an eager call
with a much larger scratch need (a 64-token projection of 4096 columns) makes the context
allocate a larger scratch; the graph keeps the old buffer, which stays allocated."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from glint_amd import synth
from glint_amd._lib import GlaError
from gpu_util import Contig, Pool

pytestmark = pytest.mark.gpu


def test_graph_replays_equal_eager_calls(backend):
    be = backend
    # paged Q8_0 decode: 4 sequences, Llama-3 head shape, soft-capped
    H, Hkv, d = 8, 2, 128
    pb = synth.paged_batch(11, np.array([5, 40, 300, 129], np.int32), prefix_tokens=32)
    p = Pool(be, "q8", pb, Hkv, d, seed=12)
    ds, dl, dt = be.buffer(pb.kv_start), be.buffer(pb.kv_len), be.buffer(pb.table)
    # contiguous f32 decode: one sequence, 3 layers, SmolLM head shape, ctx 512
    c = Contig(be, "f32", 1, 3, 512, 3, 64, seed=13)
    dsf, dlf = be.buffer(np.array([0], np.int32)), be.buffer(np.array([512], np.int32))
    # a 48 x 96 Q8_0 projection of 2 tokens, then RoPE on its rows (3 heads of 16)
    raw = orc.q8_quantize_rows(synth.normal_rows(14, 48, 96)).reshape(-1)
    w = be.create_q8_weights(raw, 48, 96)
    dpos = be.buffer(np.array([7, 300], np.int32))

    dq8, dqf, dx = be.empty(4 * H * d * 4), be.empty(9 * 64 * 4), be.empty(2 * 96 * 4)
    o8 = [be.empty(4 * H * d * 4) for _ in range(2)]      # [eager, graph]
    of = [[be.empty(9 * 64 * 4) for _ in range(3)] for _ in range(2)]
    oy = [be.empty(2 * 48 * 4) for _ in range(2)]

    capacity = pb.table.shape[1] * 16
    lens = {"now": pb.kv_len.copy()}

    def calls(k):
        if k == 0:  # eager: sized from the host lengths
            be.decode(p.pool, dq8, o8[k], ds, dl, 4, int(lens["now"].max()), H, 0.088, 30.0,
                      page_table=dt, page_table_stride=pb.table.shape[1], kv_start_host=pb.kv_start,
                      kv_len_host=lens["now"])
        else:  # captured: sized for every length a replay may see
            be.decode(p.pool, dq8, o8[k], ds, dl, 4, capacity, H, 0.088, 30.0,
                      page_table=dt, page_table_stride=pb.table.shape[1])
        for layer in range(3):
            be.decode(c.cache, dqf, of[k][layer], dsf, dlf, 1, 512, 9, 0.125, layer=layer)
        be.matvec_q8_0(w, dx, 2, oy[k])
        be.rope(oy[k], 2, 3, 16, dpos, 10000.0, 1.0, 16)

    rng = np.random.default_rng(15)

    def new_inputs(rep):
        dq8.upload(rng.standard_normal(4 * H * d).astype(np.float32))
        dqf.upload(rng.standard_normal(9 * 64).astype(np.float32))
        dx.upload(rng.standard_normal(2 * 96).astype(np.float32))
        # the sequences grow by 3 positions a step up to their written length
        lens["now"] = np.maximum(1, pb.kv_len - 3 * (5 - rep)).astype(np.int32)
        dl.upload(lens["now"])

    # a capture that passes host lengths is refused (its replays would keep their sizing)
    with pytest.raises(GlaError, match="captured"):
        be.capture(lambda: be.decode(p.pool, dq8, o8[1], ds, dl, 4, capacity, H, 0.088, 30.0, page_table=dt,
                                     page_table_stride=pb.table.shape[1], kv_start_host=pb.kv_start,
                                     kv_len_host=pb.kv_len))
    new_inputs(0)
    calls(0)  # sizes the scratch: nothing allocates during the capture
    calls(1)
    be.sync()
    g = be.capture(lambda: calls(1))
    big = be.create_q8_weights(orc.q8_quantize_rows(synth.normal_rows(16, 512, 4096)).reshape(-1), 512, 4096)
    try:
        for rep in range(6):
            if rep == 4:  # grow the scratch after the capture: ~2 MiB of pieces and partials
                bx, by = be.buffer(rng.standard_normal(64 * 4096).astype(np.float32)), be.empty(64 * 512 * 4)
                be.matvec_q8_0(big, bx, 64, by)
                be.sync()
                assert np.isfinite(by.download((64 * 512,))).all()
            new_inputs(rep)
            calls(0)
            g.replay()
            be.sync()
            pairs = [(o8[0], o8[1], 4 * H * d), (oy[0], oy[1], 96)]
            pairs += [(of[0][layer], of[1][layer], 9 * 64) for layer in range(3)]
            for a, b, n in pairs:
                ea, eb = a.download((n,)), b.download((n,))
                assert np.isfinite(ea).all()
                assert np.array_equal(ea.view(np.uint32), eb.view(np.uint32)), rep
    finally:
        g.destroy()
        w.destroy()
        big.destroy()


def test_capture_that_would_grow_scratch_is_refused(backend):
    """A captured call whose scratch the stream has not yet sized is refused with
    GLA_ERR_INVALID (an allocation is not allowed inside a capture); the stream works after, and
    the captured 64-token matvec's replays equal eager calls on the same inputs bit for bit."""
    from glint_amd.attn import HipStream
    be = backend
    w = be.create_q8_weights(orc.q8_quantize_rows(synth.normal_rows(17, 256, 1024)).reshape(-1), 256, 1024)
    s = HipStream()
    try:
        be.set_stream(s)
        x, y = be.buffer(synth.normal_rows(18, 64, 1024)), be.empty(64 * 256 * 4)
        with pytest.raises(GlaError, match="sized before capture"):
            be.capture(lambda: be.matvec_q8_0(w, x, 64, y))
        be.matvec_q8_0(w, x, 64, y)  # eager: sizes the stream's scratch
        be.sync()
        g = be.capture(lambda: be.matvec_q8_0(w, x, 64, y))
        # replays with new inputs and eager calls between them: the split-K kernel's per-row-group
        # arrival counters must be back at zero after every run for the next to sum its K slices
        y2 = be.empty(64 * 256 * 4)
        for rep in range(4):
            x.upload(synth.normal_rows(19 + rep, 64, 1024))
            be.matvec_q8_0(w, x, 64, y2)
            g.replay()
            be.sync()
            want = y2.download((64 * 256,))
            assert np.isfinite(want).all()
            assert np.array_equal(y.download((64 * 256,)).view(np.uint32), want.view(np.uint32)), rep
        g.destroy()
    finally:
        be.set_stream(None)
        s.destroy()
        w.destroy()
