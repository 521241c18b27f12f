"""Host-side mirror of Glint's GPU attention interface over the gfx950 library.

The Rust engine would bind include/glint_attn.h directly; this module is the
same binding in Python, shaped like the reference types so tests read like the
reference's own:

    GpuBackend          src/backend/gpu.rs:30-39  (new, attention, attention_resident,
                                                   create_kv_cache)
    GpuKvCache          src/backend/gpu.rs:1035-1058, KvStore impl src/cache/mod.rs:430-578
    DevicePagePool      PagePool, src/cache/paged.rs:100-240 (page storage; page ids and
                        reference counts stay with the caller, as in PagedKvCache)

plus the batched entry points the reference lacks on the GPU (decode over a
batch of sequences, forward.rs:1468-1502; prefill, forward.rs:927-958).
Every call goes to the HIP library; there is no CPU fallback here.
"""
from __future__ import annotations

import ctypes as C
import weakref
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import GLA_PAGE_SIZE, GlaError, check

PAGE_SIZE = GLA_PAGE_SIZE
_DTYPES = {"f32": _lib.GLA_KV_F32, "q8": _lib.GLA_KV_Q8_0, "q8_0": _lib.GLA_KV_Q8_0}


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def _cap(softcap: Optional[float]) -> float:
    return float(softcap) if softcap is not None else 0.0


def window_start(pos: int, sliding_window: Optional[int], alternating: bool, layer: int) -> int:
    """window_start rule of src/transformer/forward.rs:574-581, via the library."""
    return int(_lib.lib().gla_window_start(pos, int(sliding_window or 0), int(bool(alternating)), layer))


class DeviceBuffer:
    """A device allocation owned by a GpuBackend (gla_dev_alloc)."""

    def __init__(self, backend: "GpuBackend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(_lib.lib().gla_dev_alloc(backend.ctx, max(self.nbytes, 16), C.byref(p)))
        self.ptr = p

    @classmethod
    def from_numpy(cls, backend: "GpuBackend", a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(backend, a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(_lib.lib().gla_memcpy_htod(self.backend.ctx, self.ptr, _ptr(a), a.nbytes))

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(_lib.lib().gla_memcpy_dtoh(self.backend.ctx, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(_lib.lib().gla_dev_free(self.backend.ctx, self.ptr))
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            if self.ptr and self.backend.ctx:
                _lib.lib().gla_dev_free(self.backend.ctx, self.ptr)
        except Exception:
            pass


class _KvBase:
    def __init__(self, backend: "GpuBackend", handle: C.c_void_p, dtype: str, n_kv_heads: int, head_dim: int):
        self.backend = backend
        self.handle = handle
        self.dtype = dtype
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.kv_dim = n_kv_heads * head_dim

    @property
    def row_bytes(self) -> int:
        return int(_lib.lib().gla_kv_row_bytes(self.handle))

    def write_rows(self, rows: Sequence[int], k: np.ndarray, v: np.ndarray) -> None:
        """KvStore::write for many rows at once (quantise-on-write for Q8_0)."""
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(len(rows), self.kv_dim)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(len(rows), self.kv_dim)
        check(_lib.lib().gla_kv_write_rows_host(self.backend.ctx, self.handle, _ptr(rows), _ptr(k), _ptr(v),
                                                len(rows)))

    def write_rows_device(self, rows: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, n_rows: int) -> None:
        check(_lib.lib().gla_kv_write_rows(self.backend.ctx, self.handle, rows.ptr, k.ptr, v.ptr, n_rows))

    def export_rows(self, rows: Sequence[int]) -> tuple[np.ndarray, np.ndarray]:
        """Rows in KvStore::export_raw byte format: ([n][row_bytes], [n][row_bytes]) uint8."""
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        rb = self.row_bytes
        k = np.empty((len(rows), rb), dtype=np.uint8)
        v = np.empty((len(rows), rb), dtype=np.uint8)
        check(_lib.lib().gla_kv_export_rows_host(self.backend.ctx, self.handle, _ptr(rows), len(rows), _ptr(k),
                                                 _ptr(v)))
        return k, v

    def import_rows(self, rows: Sequence[int], k_bytes: np.ndarray, v_bytes: np.ndarray) -> None:
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        k_bytes = np.ascontiguousarray(k_bytes, dtype=np.uint8)
        v_bytes = np.ascontiguousarray(v_bytes, dtype=np.uint8)
        assert k_bytes.size == len(rows) * self.row_bytes and v_bytes.size == k_bytes.size
        check(_lib.lib().gla_kv_import_rows_host(self.backend.ctx, self.handle, _ptr(rows), len(rows),
                                                 _ptr(k_bytes), _ptr(v_bytes)))

    def destroy(self) -> None:
        if self.handle:
            _lib.lib().gla_kv_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class GpuKvCache(_KvBase):
    """Device-resident contiguous KV caches for n_seqs sequences (KvCache / KvCacheQ8 layout
    semantics, src/cache/mod.rs:117-423), the live counterpart of the reference's unused
    GpuKvCache (src/backend/gpu.rs:1060-1104)."""

    def __init__(self, backend, handle, dtype, n_seqs, n_layers, max_seq_len, n_kv_heads, head_dim):
        super().__init__(backend, handle, dtype, n_kv_heads, head_dim)
        self.n_seqs = n_seqs
        self.n_layers = n_layers
        self.max_seq_len = max_seq_len
        self.len = [0] * n_seqs

    def row_id(self, seq: int, layer: int, pos: int) -> int:
        r = int(_lib.lib().gla_kv_row_id(self.handle, seq, layer, pos))
        if r < 0:
            raise GlaError(_lib.GLA_ERR_INVALID, f"row ({seq}, {layer}, {pos}) outside the cache")
        return r

    def write(self, layer: int, pos: int, k: np.ndarray, v: np.ndarray, seq: int = 0) -> None:
        """KvStore::write (src/cache/mod.rs:166-177); panics past max_seq_len like the reference."""
        if pos >= self.max_seq_len:
            raise AssertionError(f"KV-cache overflow: pos {pos} >= {self.max_seq_len}")
        self.write_rows([self.row_id(seq, layer, pos)], k, v)

    def advance(self, seq: int = 0) -> None:
        self.len[seq] += 1

    def export_raw(self, seq: int = 0) -> tuple[list[bytes], list[bytes]]:
        """KvStore::export_raw: per-layer bytes of positions 0..len."""
        ks, vs = [], []
        for layer in range(self.n_layers):
            rows = [self.row_id(seq, layer, p) for p in range(self.len[seq])]
            k, v = self.export_rows(rows) if rows else (np.zeros((0, 0), np.uint8),) * 2
            ks.append(k.tobytes())
            vs.append(v.tobytes())
        return ks, vs

    def import_raw(self, k_layers, v_layers, token_count: int, seq: int = 0) -> None:
        """KvStore::import_raw with the reference's size check (src/cache/mod.rs:397-422)."""
        expected = token_count * self.row_bytes
        for layer, (kb, vb) in enumerate(zip(k_layers, v_layers)):
            if len(kb) != expected or len(vb) != expected:
                raise GlaError(_lib.GLA_ERR_INVALID,
                               f"SnapshotCacheSizeMismatch layer {layer}: expected {expected}, "
                               f"found {len(kb)}/{len(vb)}")
            rows = [self.row_id(seq, layer, p) for p in range(token_count)]
            if rows:
                self.import_rows(rows, np.frombuffer(kb, np.uint8), np.frombuffer(vb, np.uint8))
        self.len[seq] = token_count


class DevicePagePool(_KvBase):
    """Device page storage of a PagePool (src/cache/paged.rs:157-240): capacity_pages pages of
    PAGE_SIZE positions x kv_dim of K and V. Row id of (page, slot) = page * 16 + slot."""

    def __init__(self, backend, handle, dtype, capacity_pages, n_kv_heads, head_dim):
        super().__init__(backend, handle, dtype, n_kv_heads, head_dim)
        self.capacity = capacity_pages

    def copy_page(self, src: int, dst: int) -> None:
        """Copy-on-write body (src/cache/paged.rs:433-444)."""
        check(_lib.lib().gla_pool_copy_page(self.backend.ctx, self.handle, src, dst))

    def zero_page(self, page: int) -> None:
        """PageBuf::reset of a recycled page (src/cache/paged.rs:79-82)."""
        check(_lib.lib().gla_pool_zero_page(self.backend.ctx, self.handle, page))


class Q8Weights:
    """GGML Q8_0 weights uploaded once and repacked for the MFMA matvec (gla_q8w_create)."""

    def __init__(self, backend: "GpuBackend", handle: C.c_void_p, rows: int, cols: int):
        self.backend, self.handle, self.rows, self.cols = backend, handle, rows, cols

    def destroy(self) -> None:
        if self.handle:
            check(_lib.lib().gla_q8w_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


_HIP = None


def _hip() -> C.CDLL:
    """The HIP runtime the library is linked against (already loaded with it)."""
    global _HIP
    if _HIP is None:
        _lib.lib()
        for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _HIP = C.CDLL(name)
                break
            except OSError:
                continue
        if _HIP is None:
            raise GlaError(_lib.GLA_ERR_DEVICE, "libamdhip64.so not found")
        for fn, args in (("hipStreamBeginCapture", [C.c_void_p, C.c_int]),
                         ("hipStreamEndCapture", [C.c_void_p, C.POINTER(C.c_void_p)]),
                         ("hipGraphInstantiate", [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p,
                                                  C.c_size_t]),
                         ("hipGraphLaunch", [C.c_void_p, C.c_void_p]),
                         ("hipGraphExecDestroy", [C.c_void_p]),
                         ("hipGraphDestroy", [C.c_void_p]),
                         ("hipStreamCreateWithFlags", [C.POINTER(C.c_void_p), C.c_uint]),
                         ("hipStreamDestroy", [C.c_void_p]),
                         ("hipStreamSynchronize", [C.c_void_p])):
            f = getattr(_HIP, fn)
            f.argtypes, f.restype = args, C.c_int
    return _HIP


def _hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise GlaError(_lib.GLA_ERR_DEVICE, f"{what}: hipError {rc}")


class HipStream:
    """A HIP stream of default priority (non-blocking), for running library work on more than
    one stream of a backend (GpuBackend.set_stream)."""

    def __init__(self):
        s = C.c_void_p()
        _hip_check(_hip().hipStreamCreateWithFlags(C.byref(s), 1), "hipStreamCreateWithFlags")
        self.ptr = s
        # backends that have run work on this stream: destroy() hands their
        # scratch for it back (gla_release_stream) before the stream goes
        self._users = weakref.WeakSet()

    @property
    def handle(self) -> int:
        return int(self.ptr.value or 0)

    def synchronize(self) -> None:
        _hip_check(_hip().hipStreamSynchronize(self.ptr), "hipStreamSynchronize")

    def destroy(self) -> None:
        """Release the stream: each backend that used it goes back to its own stream if this one
        is current, and frees the scratch it kept for this stream (gla_release_stream, which
        waits for the stream first); then the stream is destroyed."""
        if self.ptr:
            for be in list(self._users):
                be._forget_stream(self)
            self._users = weakref.WeakSet()
            _hip().hipStreamDestroy(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class HipGraph:
    """Library calls captured on a backend's stream and replayed with one hipGraphLaunch.
    A replay repeats the captured launches exactly: the same buffers (whose contents may
    change between replays), shapes and host-side launch decisions -- and the same context
    scratch. A later call that needs more scratch moves to a larger buffer and keeps the old
    one allocated until the context is destroyed, so the graph's pointers stay valid. A
    captured gla_decode must be sized for the lengths of every replay: pass max_kv_len = the
    capacity and no host lengths (the library refuses host lengths during a capture)."""

    def __init__(self, backend: "GpuBackend", graph: C.c_void_p, exe: C.c_void_p):
        self.backend, self.graph, self.exe = backend, graph, exe

    def replay(self) -> None:
        """Enqueue the graph on the backend's stream (asynchronous, like the calls it holds)."""
        _hip_check(_hip().hipGraphLaunch(self.exe, C.c_void_p(self.backend.stream)), "hipGraphLaunch")

    def destroy(self) -> None:
        if self.exe:
            _hip().hipGraphExecDestroy(self.exe)
            self.exe = None
        if self.graph:
            _hip().hipGraphDestroy(self.graph)
            self.graph = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class GpuBackend:
    """One HIP device and stream (gla_ctx). Mirrors GpuBackend::new's failure mode:
    no device -> GlaError named GpuAdapterNotFound, and the caller keeps its CPU path."""

    def __init__(self, device: int = 0):
        p = C.c_void_p()
        check(_lib.lib().gla_create(device, C.byref(p)))
        self.ctx = p
        # the HipStream set with set_stream (None: the context's own): held so
        # the stream outlives its use by the context
        self._stream: Optional["HipStream"] = None

    def close(self) -> None:
        if self.ctx:
            _lib.lib().gla_destroy(self.ctx)
            self.ctx = C.c_void_p()
        self._stream = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- plumbing ---------------------------------------------------------
    def sync(self) -> None:
        check(_lib.lib().gla_sync(self.ctx))

    @property
    def stream(self) -> int:
        return int(_lib.lib().gla_get_stream(self.ctx) or 0)

    def set_stream(self, stream: Optional["HipStream"]) -> None:
        """Enqueue later calls on `stream` (None: the backend's own stream). Work on different
        streams uses different scratch buffers, so calls may overlap across streams. The backend
        keeps `stream` alive while it is set; HipStream.destroy() resets the backend first."""
        if stream is not None and not stream.ptr:
            raise ValueError("set_stream: the HipStream was destroyed")
        check(_lib.lib().gla_set_stream(self.ctx, stream.ptr if stream is not None else None))
        self._stream = stream
        if stream is not None:
            stream._users.add(self)

    def _forget_stream(self, stream: "HipStream") -> None:
        """`stream` is about to be destroyed: leave it if current, and free its scratch."""
        if not self.ctx:
            return
        if self._stream is stream:
            self.set_stream(None)
        check(_lib.lib().gla_release_stream(self.ctx, stream.ptr))

    @property
    def cu_count(self) -> int:
        return int(_lib.lib().gla_device_cu_count(self.ctx))

    def capture(self, calls) -> HipGraph:
        """Capture ``calls()`` -- device-pointer library calls on this backend, e.g. a decode
        step's layers -- into a HIP graph. Run the same calls once beforehand, so that no call
        grows its scratch (allocates) during the capture. A later call that needs more scratch
        moves to a new buffer and leaves the old one allocated until the context is destroyed,
        so the graph's pointers stay valid."""
        hip = _hip()
        stream = C.c_void_p(self.stream)
        _hip_check(hip.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")  # thread-local mode
        graph = C.c_void_p()
        try:
            calls()
        except BaseException:
            hip.hipStreamEndCapture(stream, C.byref(graph))
            if graph:
                hip.hipGraphDestroy(graph)
            raise
        rc = hip.hipStreamEndCapture(stream, C.byref(graph))
        _hip_check(rc, "hipStreamEndCapture")
        exe = C.c_void_p()
        rc = hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0)
        if rc != 0:
            hip.hipGraphDestroy(graph)
            _hip_check(rc, "hipGraphInstantiate")
        return HipGraph(self, graph, exe)

    def buffer(self, a: np.ndarray) -> DeviceBuffer:
        return DeviceBuffer.from_numpy(self, a)

    def empty(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    # -- KV storage -------------------------------------------------------
    def create_kv_cache(self, n_layers: int, max_seq_len: int, n_kv_heads: int, head_dim: int,
                        dtype: str = "f32", n_seqs: int = 1) -> GpuKvCache:
        h = C.c_void_p()
        check(_lib.lib().gla_kv_cache_create(self.ctx, _DTYPES[dtype], n_seqs, n_layers, max_seq_len, n_kv_heads,
                                             head_dim, C.byref(h)))
        return GpuKvCache(self, h, dtype, n_seqs, n_layers, max_seq_len, n_kv_heads, head_dim)

    def create_page_pool(self, capacity_pages: int, n_kv_heads: int, head_dim: int,
                         dtype: str = "f32") -> DevicePagePool:
        h = C.c_void_p()
        check(_lib.lib().gla_pool_create(self.ctx, _DTYPES[dtype], n_kv_heads, head_dim, capacity_pages,
                                         C.byref(h)))
        return DevicePagePool(self, h, dtype, capacity_pages, n_kv_heads, head_dim)

    # -- reference entry points --------------------------------------------
    def attention(self, q, k, v, n_heads: int, n_kv_heads: int, head_dim: int, seq_len: int, scale: float,
                  softcap: Optional[float] = None) -> np.ndarray:
        """GpuBackend::attention (src/backend/gpu.rs:266-397): host q [H*d], k/v [seq][Hkv*d]."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        out = np.empty(n_heads * head_dim, dtype=np.float32)
        check(_lib.lib().gla_attention(self.ctx, _ptr(q), _ptr(k), _ptr(v), n_heads, n_kv_heads, head_dim,
                                       seq_len, float(scale), _cap(softcap), _ptr(out)))
        return out

    def attention_resident(self, q, kv_buf: GpuKvCache, layer_idx: int, window_start: int, attend_len: int,
                           n_heads: int, n_kv_heads: int, head_dim: int, scale: float,
                           softcap: Optional[float] = None, seq: int = 0) -> np.ndarray:
        """GpuBackend::attention_resident (src/backend/gpu.rs:860-992)."""
        assert n_kv_heads == kv_buf.n_kv_heads and head_dim == kv_buf.head_dim
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.empty(n_heads * head_dim, dtype=np.float32)
        check(_lib.lib().gla_attention_resident(self.ctx, _ptr(q), kv_buf.handle, seq, layer_idx, window_start,
                                                attend_len, n_heads, float(scale), _cap(softcap), _ptr(out)))
        return out

    # -- batched device entry points ----------------------------------------
    def decode(self, kv: _KvBase, q: DeviceBuffer, out: DeviceBuffer, kv_start: DeviceBuffer,
               kv_len: DeviceBuffer, n_seqs: int, max_kv_len: int, n_heads: int, scale: float,
               softcap: Optional[float] = None, layer: int = 0, seq_slot: Optional[DeviceBuffer] = None,
               page_table: Optional[DeviceBuffer] = None, page_table_stride: int = 0,
               kv_start_host: Optional[np.ndarray] = None, kv_len_host: Optional[np.ndarray] = None,
               noalloc: bool = False) -> None:
        """gla_decode on device buffers (asynchronous on the backend's stream). kv_start_host /
        kv_len_host: optional host copies of the device arrays (int32[B]); they let the library
        size the launch to the real lengths. noalloc: call gla_decode_noalloc (partials in the
        library's static per-GPU scratch; nothing is allocated)."""
        a = _lib.DecodeArgs()
        a.kv = kv.handle
        a.layer = layer
        a.n_seqs = n_seqs
        a.seq_slot = seq_slot.ptr if seq_slot is not None else None
        a.page_table = page_table.ptr if page_table is not None else None
        a.page_table_stride = page_table_stride
        a.kv_start = kv_start.ptr
        a.kv_len = kv_len.ptr
        a.max_kv_len = max_kv_len
        a.n_heads = n_heads
        a.scale = scale
        a.softcap = _cap(softcap)
        a.q = q.ptr
        a.out = out.ptr
        if (kv_start_host is None) != (kv_len_host is None):
            raise ValueError("pass both kv_start_host and kv_len_host, or neither")
        if kv_start_host is not None:
            hs = np.ascontiguousarray(kv_start_host, dtype=np.int32)
            hl = np.ascontiguousarray(kv_len_host, dtype=np.int32)
            if hs.shape != (n_seqs,) or hl.shape != (n_seqs,):
                raise ValueError("kv_start_host / kv_len_host must be int32[n_seqs]")
            a.kv_start_host = hs.ctypes.data
            a.kv_len_host = hl.ctypes.data
        fn = _lib.lib().gla_decode_noalloc if noalloc else _lib.lib().gla_decode
        check(fn(self.ctx, C.byref(a)))

    def prefill(self, kv: _KvBase, q: DeviceBuffer, out: DeviceBuffer, q_start: DeviceBuffer,
                pos_offset: DeviceBuffer, n_seqs: int, max_q_len: int, n_heads: int, scale: float,
                softcap: Optional[float] = None, sliding_window: Optional[int] = None, layer: int = 0,
                seq_slot: Optional[DeviceBuffer] = None, page_table: Optional[DeviceBuffer] = None,
                page_table_stride: int = 0, precision: str = "f32") -> None:
        """gla_prefill on device buffers (asynchronous on the backend's stream)."""
        a = _lib.PrefillArgs()
        a.kv = kv.handle
        a.layer = layer
        a.n_seqs = n_seqs
        a.seq_slot = seq_slot.ptr if seq_slot is not None else None
        a.page_table = page_table.ptr if page_table is not None else None
        a.page_table_stride = page_table_stride
        a.q_start = q_start.ptr
        a.pos_offset = pos_offset.ptr
        a.max_q_len = max_q_len
        a.n_heads = n_heads
        a.scale = scale
        a.softcap = _cap(softcap)
        a.sliding_window = int(sliding_window or 0)
        a.precision = {"f32": _lib.GLA_PREC_F32, "bf16": _lib.GLA_PREC_BF16}[precision]
        a.q = q.ptr
        a.out = out.ptr
        check(_lib.lib().gla_prefill(self.ctx, C.byref(a)))

    def rope(self, x: DeviceBuffer, n_rows: int, n_heads: int, head_dim: int, pos: DeviceBuffer, freq_base: float,
             scaling_factor: float = 1.0, rot_dim: Optional[int] = None) -> None:
        """ops::rope (src/tensor/ops.rs:212-245) in place on device rows x [n_rows][n_heads][head_dim]."""
        check(_lib.lib().gla_rope(self.ctx, x.ptr, n_rows, n_heads, head_dim, pos.ptr, float(freq_base),
                                  float(scaling_factor), head_dim if rot_dim is None else rot_dim))

    def create_q8_weights(self, ggml: np.ndarray, rows: int, cols: int) -> Q8Weights:
        """Upload GGML Q8_0 bytes [rows][cols/32 x 34] (gla_q8w_create)."""
        raw = np.ascontiguousarray(ggml, dtype=np.uint8).reshape(-1)
        assert raw.size == rows * (cols // 32) * 34
        h = C.c_void_p()
        check(_lib.lib().gla_q8w_create(self.ctx, _ptr(raw), rows, cols, C.byref(h)))
        return Q8Weights(self, h, rows, cols)

    def matvec_q8_0(self, w: Q8Weights, x: DeviceBuffer, n_vec: int, y: DeviceBuffer) -> None:
        """y[v] = W x[v] for n_vec device vectors (QuantizedTensor::matvec, src/tensor/quantized.rs:247-346)."""
        check(_lib.lib().gla_matvec_q8_0(self.ctx, w.handle, x.ptr, n_vec, y.ptr))
