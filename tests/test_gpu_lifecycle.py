"""Handle lifetimes across the C ABI. A context owns the device memory of the caches, pools
and weights created on it: destroying the context first frees that memory and detaches the
handles, which can then still be released (freeing only the handle), and any other use of a
detached handle is refused with GLA_ERR_INVALID instead of touching freed memory. Garbage
collection can release handles in any order (a failing test's traceback, for one, keeps its
caches alive past the session's context)."""
from __future__ import annotations

import numpy as np
import pytest

from glint_amd import synth
from glint_amd._lib import GLA_ERR_INVALID, GlaError
from glint_amd.attn import GpuBackend

pytestmark = pytest.mark.gpu


def test_context_destroyed_before_its_handles(hip_lib):
    be = GpuBackend(0)
    cache = be.create_kv_cache(1, 64, 2, 64, "f32", 1)
    pool = be.create_page_pool(4, 2, 64, "q8")
    w = be.create_q8_weights(np.zeros((16, 2, 34), np.uint8), 16, 64)
    cache.write_rows([0, 1], synth.normal_rows(1, 2, 128), synth.normal_rows(2, 2, 128))
    be.close()  # frees the storage and weights above; their handles stay valid to release

    other = GpuBackend(0)
    try:
        with pytest.raises(GlaError) as ei:
            cache.backend = other
            cache.write_rows([0], np.zeros((1, 128), np.float32), np.zeros((1, 128), np.float32))
        assert ei.value.code == GLA_ERR_INVALID and "destroyed context" in str(ei.value)
        # a live handle of another context is refused too
        mine = other.create_kv_cache(1, 64, 2, 64, "f32", 1)
        third = GpuBackend(0)
        try:
            with pytest.raises(GlaError) as ei:
                mine.backend = third
                mine.write_rows([0], np.zeros((1, 128), np.float32), np.zeros((1, 128), np.float32))
            assert ei.value.code == GLA_ERR_INVALID and "another context" in str(ei.value)
        finally:
            third.close()
        mine.backend = other
        mine.destroy()
    finally:
        other.close()
    cache.destroy()  # detached: frees the handle only
    pool.destroy()
    w.destroy()
