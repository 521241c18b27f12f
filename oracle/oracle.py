"""ctypes binding of the CPU oracle (oracle/glint_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the CPU baseline, never
as the thing measured or shipped.

Every function restates the Glint file:line cited in glint_oracle.c. The KV
stores take numpy arrays in Glint's own host layouts:
  f32 contiguous  k[layer][max_seq][kv_dim]                (KvCache, src/cache/mod.rs:117-164)
  q8  contiguous  k[layer][max_seq][ceil(kv_dim/32)*34] u8 (KvCacheQ8, src/cache/mod.rs:270-358)
  paged f32       k[page][16][kv_dim], table[layer][lp]    (PagedKvCache, src/cache/paged.rs:453-465)
  paged q8        k[page][16][row_bytes] u8, table         (paged indexing + the Q8 row codec)
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32, Q8, PAGED_F32, PAGED_Q8 = 0, 1, 2, 3

_P = C.c_void_p
_I = C.c_int
_L = C.c_long
_F = C.c_float


def _bind(path: Path) -> C.CDLL:
    h = C.CDLL(str(path))
    h.or_f16_from_f32.restype = C.c_uint16
    h.or_f16_from_f32.argtypes = [_F]
    h.or_f16_to_f32.restype = _F
    h.or_f16_to_f32.argtypes = [C.c_uint16]
    h.or_q8_quantize_row.argtypes = [_P, _I, _P]
    h.or_q8_quantize_rows.argtypes = [_P, _L, _I, _P, _I]
    h.or_q8_dequant_range.argtypes = [_P, _I, _I, _P]
    h.or_store_new.restype = _P
    h.or_store_new.argtypes = [_I, _I, _I, _I, _P, _P, _P, _I]
    h.or_store_free.argtypes = [_P]
    h.or_read_k_head.argtypes = [_P, _I, _L, _I, _I, _P]
    h.or_read_v_head.argtypes = [_P, _I, _L, _I, _I, _P]
    h.or_flash_attn_1d_ext.argtypes = [_P, _P, _I, _I, _L, _L, _I, _F, _I, _F, _P]
    h.or_standard_attn.argtypes = [_P, _P, _I, _I, _L, _L, _I, _F, _I, _F, _P]
    h.or_attn_heads_cpu.argtypes = [_P, _P, _I, _L, _L, _I, _I, _I, _F, _I, _F, _P]
    h.or_window_start.restype = _L
    h.or_window_start.argtypes = [_L, _L, _I, _I]
    h.or_decode_batch.argtypes = [_P, _P, _I, _I, _P, _P, _I, _I, _I, _F, _I, _F, _P, _I]
    h.or_prefill.argtypes = [_P, _P, _I, _L, _L, _I, _I, _I, _F, _I, _F, _L, _I, _P, _I]
    h.or_rope.argtypes = [_P, _P, _I, _L, _I, _F, _F, _I]
    h.or_matvec_q8_0.argtypes = [_P, _L, _I, _P, _P]
    return h


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        _lib = _bind(LIB_PATH)
    return _lib


def build_mutant(n: int, out_dir: Path) -> C.CDLL:
    """Compile the oracle with planted mistake number n (OR_MUTANT=n) and bind it."""
    out_dir.mkdir(parents=True, exist_ok=True)
    so = out_dir / f"liboracle_mutant{n}.so"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", f"-DOR_MUTANT={n}", "-o", str(so),
                    str(HERE / "glint_oracle.c"), "-lm", "-pthread"], check=True)
    return _bind(so)


NATIVE_FLAGS = ["-O3", "-march=native", "-ffp-contract=off", "-fno-fast-math"]


def build_native(out_dir: Path) -> C.CDLL:
    """Compile the oracle for the CPU it runs on (gcc -O3 -march=native -ffp-contract=off, no
    fast-math: the CPU-baseline build; the float operations and their order are those of the
    portable -O2 build, since gcc does not reassociate without fast-math) and bind it."""
    out_dir.mkdir(parents=True, exist_ok=True)
    so = out_dir / "liboracle_native.so"
    subprocess.run(["gcc", *NATIVE_FLAGS, "-fPIC", "-shared", "-std=c11", "-o", str(so),
                    str(HERE / "glint_oracle.c"), "-lm", "-pthread"], check=True, capture_output=True)
    return _bind(so)


def host_cores() -> int:
    """Cores this process may run on (its affinity mask; os.cpu_count() without one)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def threads() -> int:
    """Worker threads: the cores this process may use (its affinity mask, what Rust's
    available_parallelism() and so Rayon's default pool see), unless OMP_NUM_THREADS asks for
    fewer (a shared host's CPU share; the GPU boxes set it to their share)."""
    n = host_cores()
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def _p(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def f16_from_f32(x: float, L=None) -> int:
    return int((L or lib()).or_f16_from_f32(x))


def f16_to_f32(h: int, L=None) -> float:
    return float((L or lib()).or_f16_to_f32(h))


def q8_row_bytes(n: int) -> int:
    return ((n + 31) // 32) * 34


def q8_quantize_rows(x: np.ndarray, L=None) -> np.ndarray:
    """KvCacheQ8::quantize_into over the last axis (src/cache/mod.rs:296-315)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    out = np.empty(x.shape[:-1] + (q8_row_bytes(n),), dtype=np.uint8)
    (L or lib()).or_q8_quantize_rows(_p(x), rows, n, _p(out), threads())
    return out


def q8_dequant_range(row: np.ndarray, start: int, end: int, L=None) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    buf = np.empty(end - start, dtype=np.float32)
    (L or lib()).or_q8_dequant_range(_p(row), start, end, _p(buf))
    return buf


class Store:
    """An `&dyn KvStore` over numpy arrays (kept alive by this object)."""

    def __init__(self, kind: int, k: np.ndarray, v: np.ndarray, kv_dim: int, n_layers: int = 1,
                 max_seq: int = 0, table: Optional[np.ndarray] = None, L=None):
        self.L = L or lib()
        self.kind = kind
        self.k = np.ascontiguousarray(k)
        self.v = np.ascontiguousarray(v)
        self.table = None if table is None else np.ascontiguousarray(table, dtype=np.int32)
        stride = 0 if self.table is None else self.table.shape[-1]
        self.ptr = self.L.or_store_new(kind, n_layers, max_seq, kv_dim, _p(self.k), _p(self.v),
                                       None if self.table is None else _p(self.table), stride)

    def __del__(self):
        try:
            self.L.or_store_free(self.ptr)
        except Exception:
            pass

    def read_k_head(self, layer: int, pos: int, kv_h: int, d: int) -> np.ndarray:
        buf = np.empty(d, np.float32)
        self.L.or_read_k_head(self.ptr, layer, pos, kv_h, d, _p(buf))
        return buf

    def read_v_head(self, layer: int, pos: int, kv_h: int, d: int) -> np.ndarray:
        buf = np.empty(d, np.float32)
        self.L.or_read_v_head(self.ptr, layer, pos, kv_h, d, _p(buf))
        return buf


def kv_cache(k: np.ndarray, v: np.ndarray, L=None) -> Store:
    """f32 KvCache from k, v [n_layers][max_seq][kv_dim]."""
    return Store(F32, k.astype(np.float32), v.astype(np.float32), k.shape[-1], k.shape[0], k.shape[1], L=L)


def kv_cache_q8(kq: np.ndarray, vq: np.ndarray, kv_dim: int, L=None) -> Store:
    """KvCacheQ8 from quantised rows [n_layers][max_seq][row_bytes]."""
    return Store(Q8, kq, vq, kv_dim, kq.shape[0], kq.shape[1], L=L)


def paged_f32(pages_k: np.ndarray, pages_v: np.ndarray, table: np.ndarray, L=None) -> Store:
    """PagedKvCache: pages [n_pages][16][kv_dim], table [n_layers][max_pages]."""
    t = np.atleast_2d(table)
    return Store(PAGED_F32, pages_k.astype(np.float32), pages_v.astype(np.float32), pages_k.shape[-1],
                 t.shape[0], 0, t, L=L)


def paged_q8(pages_kq: np.ndarray, pages_vq: np.ndarray, kv_dim: int, table: np.ndarray, L=None) -> Store:
    t = np.atleast_2d(table)
    return Store(PAGED_Q8, pages_kq, pages_vq, kv_dim, t.shape[0], 0, t, L=L)


def _cap(softcap):
    return (1, float(softcap)) if softcap else (0, 0.0)


def flash_attn_1d_ext(q, store: Store, layer: int, kv_h: int, start_pos: int, seq_len: int, head_dim: int,
                      scale: float, softcap: Optional[float] = None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(head_dim, np.float32)
    hc, c = _cap(softcap)
    store.L.or_flash_attn_1d_ext(_p(q), store.ptr, layer, kv_h, start_pos, seq_len, head_dim, scale, hc, c,
                                 _p(out))
    return out


def standard_attn(q, store: Store, layer: int, kv_h: int, start_pos: int, seq_len: int, head_dim: int,
                  scale: float, softcap: Optional[float] = None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(head_dim, np.float32)
    hc, c = _cap(softcap)
    store.L.or_standard_attn(_p(q), store.ptr, layer, kv_h, start_pos, seq_len, head_dim, scale, hc, c, _p(out))
    return out


def attn_heads_cpu(q_all, store: Store, layer: int, window_start: int, attend_len: int, n_heads: int,
                   kv_group_size: int, head_dim: int, scale: float, softcap: Optional[float] = None) -> np.ndarray:
    q_all = np.ascontiguousarray(q_all, dtype=np.float32)
    out = np.zeros(n_heads * head_dim, np.float32)
    hc, c = _cap(softcap)
    store.L.or_attn_heads_cpu(_p(q_all), store.ptr, layer, window_start, attend_len, n_heads, kv_group_size,
                              head_dim, scale, hc, c, _p(out))
    return out


def window_start(pos: int, sliding_window: Optional[int], alternating: bool, layer: int, L=None) -> int:
    return int((L or lib()).or_window_start(pos, int(sliding_window or 0), int(alternating), layer))


def decode_batch(q: np.ndarray, stores: Sequence[Store], layer: int, kv_start, kv_len, n_heads: int,
                 n_kv_heads: int, head_dim: int, scale: float, softcap: Optional[float] = None,
                 n_threads: Optional[int] = None) -> np.ndarray:
    """forward.rs:1468-1502: q [B][H*d] -> out [B][H*d], one task per sequence."""
    B = len(stores)
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(B, n_heads * head_dim)
    out = np.zeros((B, n_heads * head_dim), np.float32)
    ptrs = (C.c_void_p * B)(*[s.ptr for s in stores])
    ks = np.ascontiguousarray(kv_start, dtype=np.int64)
    kl = np.ascontiguousarray(kv_len, dtype=np.int64)
    hc, c = _cap(softcap)
    stores[0].L.or_decode_batch(_p(q), ptrs, B, layer, _p(ks), _p(kl), n_heads, n_kv_heads, head_dim, scale, hc,
                                c, _p(out), n_threads or threads())
    return out


def prefill(q: np.ndarray, store: Store, layer: int, pos_offset: int, n_heads: int, n_kv_heads: int,
            head_dim: int, scale: float, softcap: Optional[float] = None, sliding_window: Optional[int] = None,
            alternating: bool = False, n_threads: Optional[int] = None) -> np.ndarray:
    """forward.rs:927-958: q [T][H*d] -> out [T][H*d], one task per query position."""
    T = q.shape[0]
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(T, n_heads * head_dim)
    out = np.zeros_like(q)
    hc, c = _cap(softcap)
    store.L.or_prefill(_p(q), store.ptr, layer, pos_offset, T, n_heads, n_kv_heads, head_dim, scale, hc, c,
                       int(sliding_window or 0), int(alternating), _p(out), n_threads or threads())
    return out


def rope(x: np.ndarray, pos: int, head_dim: int, freq_base: float, scaling_factor: float, rot_dim: int,
         L=None) -> np.ndarray:
    """ops.rs:212-245: rotate the adjacent pairs of every head of x (whole heads of head_dim)."""
    L = L or lib()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty_like(x)
    L.or_rope(_p(x), _p(out), x.size, int(pos), head_dim, freq_base, scaling_factor, rot_dim)
    return out


def q8_0_block(scale: float, quants) -> bytes:
    """One GGML Q8_0 block: f16 scale (little-endian) then 32 int8 (dequantize.rs test helper layout)."""
    q = np.asarray(quants, dtype=np.int8)
    assert q.size == 32
    return np.array([f16_from_f32(scale)], dtype="<u2").tobytes() + q.tobytes()


def matvec_q8_0(data: np.ndarray, rows: int, cols: int, vec: np.ndarray, L=None) -> np.ndarray:
    """quantized.rs:587-610: GGML Q8_0 rows [rows][cols/32 x 34 B] times vec [cols] -> [rows]."""
    L = L or lib()
    data = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray)
                                else data, dtype=np.uint8)
    assert data.size == rows * (cols // 32) * 34
    vec = np.ascontiguousarray(vec, dtype=np.float32)
    out = np.empty(rows, dtype=np.float32)
    L.or_matvec_q8_0(_p(data), rows, cols, _p(vec), _p(out))
    return out
