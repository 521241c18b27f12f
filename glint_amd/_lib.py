"""ctypes binding of libglint_attn.so (include/glint_attn.h).

The library must have been built (``python -m glint_amd.build``); loading
fails loudly otherwise -- there is no CPU fallback behind this module.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
HIP_LIB_PATH = PKG / "libglint_attn.so"
SYNTH_LIB_PATH = PKG / "libglint_synth.so"

GLA_OK = 0
GLA_ERR_NO_DEVICE = -1
GLA_ERR_DEVICE = -2
GLA_ERR_BUFFER = -3
GLA_ERR_KERNEL = -4
GLA_ERR_INVALID = -5
GLA_ERR_POOL_EXHAUSTED = -6

GLA_PAGE_SIZE = 16
GLA_DECODE_NOALLOC_SCRATCH_BYTES = 16 << 20
GLA_KV_F32 = 0
GLA_KV_Q8_0 = 1
GLA_PREC_F32 = 0
GLA_PREC_BF16 = 1

# GlintError variant each status code stands for (src/error.rs:41-52, :78-82).
ERROR_NAMES = {
    GLA_ERR_NO_DEVICE: "GpuAdapterNotFound",
    GLA_ERR_DEVICE: "GpuDeviceError",
    GLA_ERR_BUFFER: "GpuBufferError",
    GLA_ERR_KERNEL: "GpuShaderError",
    GLA_ERR_INVALID: "Unsupported",
    GLA_ERR_POOL_EXHAUSTED: "KvPagePoolExhausted",
}


class GlaError(RuntimeError):
    """A failed library call: ``code`` is the status, ``name`` the GlintError variant."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.name = ERROR_NAMES.get(code, f"code {code}")
        super().__init__(f"{self.name}: {message}")


class DecodeArgs(C.Structure):
    _fields_ = [
        ("kv", C.c_void_p),
        ("layer", C.c_int),
        ("n_seqs", C.c_int),
        ("seq_slot", C.c_void_p),
        ("page_table", C.c_void_p),
        ("page_table_stride", C.c_int),
        ("kv_start", C.c_void_p),
        ("kv_len", C.c_void_p),
        ("max_kv_len", C.c_int),
        ("n_heads", C.c_int),
        ("scale", C.c_float),
        ("softcap", C.c_float),
        ("q", C.c_void_p),
        ("out", C.c_void_p),
        ("kv_start_host", C.c_void_p),
        ("kv_len_host", C.c_void_p),
    ]


class PrefillArgs(C.Structure):
    _fields_ = [
        ("kv", C.c_void_p),
        ("layer", C.c_int),
        ("n_seqs", C.c_int),
        ("seq_slot", C.c_void_p),
        ("page_table", C.c_void_p),
        ("page_table_stride", C.c_int),
        ("q_start", C.c_void_p),
        ("pos_offset", C.c_void_p),
        ("max_q_len", C.c_int),
        ("n_heads", C.c_int),
        ("scale", C.c_float),
        ("softcap", C.c_float),
        ("sliding_window", C.c_int),
        ("precision", C.c_int),
        ("q", C.c_void_p),
        ("out", C.c_void_p),
    ]


# name -> (restype, argtypes); every symbol include/glint_attn.h declares.
_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_SZ = C.c_size_t
_I64 = C.c_int64
_L = C.c_long
SIGNATURES = {
    "gla_last_error": (C.c_char_p, []),
    "gla_create": (_I, [_I, C.POINTER(_P)]),
    "gla_destroy": (_I, [_P]),
    "gla_set_stream": (_I, [_P, _P]),
    "gla_get_stream": (_P, [_P]),
    "gla_sync": (_I, [_P]),
    "gla_device_cu_count": (_I, [_P]),
    "gla_release_stream": (_I, [_P, _P]),
    "gla_dev_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "gla_dev_free": (_I, [_P, _P]),
    "gla_memcpy_htod": (_I, [_P, _P, _P, _SZ]),
    "gla_memcpy_dtoh": (_I, [_P, _P, _P, _SZ]),
    "gla_kv_cache_create": (_I, [_P, _I, _I, _I, _I, _I, _I, C.POINTER(_P)]),
    "gla_pool_create": (_I, [_P, _I, _I, _I, _I, C.POINTER(_P)]),
    "gla_kv_destroy": (_I, [_P]),
    "gla_kv_row_id": (_I64, [_P, _I, _I, _I]),
    "gla_kv_write_rows": (_I, [_P, _P, _P, _P, _P, _I]),
    "gla_kv_write_rows_host": (_I, [_P, _P, _P, _P, _P, _I]),
    "gla_kv_export_rows_host": (_I, [_P, _P, _P, _I, _P, _P]),
    "gla_kv_import_rows_host": (_I, [_P, _P, _P, _I, _P, _P]),
    "gla_kv_row_bytes": (_I64, [_P]),
    "gla_pool_copy_page": (_I, [_P, _P, _I, _I]),
    "gla_pool_zero_page": (_I, [_P, _P, _I]),
    "gla_window_start": (_L, [_L, _L, _I, _I]),
    "gla_decode": (_I, [_P, C.POINTER(DecodeArgs)]),
    "gla_decode_noalloc": (_I, [_P, C.POINTER(DecodeArgs)]),
    "gla_prefill": (_I, [_P, C.POINTER(PrefillArgs)]),
    "gla_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _P]),
    "gla_attention_resident": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P]),
    "gla_rope": (_I, [_P, _P, _I, _I, _I, _P, _F, _F, _I]),
    "gla_q8w_create": (_I, [_P, _P, _I, _I, C.POINTER(_P)]),
    "gla_q8w_destroy": (_I, [_P]),
    "gla_q8w_rows": (_I, [_P]),
    "gla_q8w_cols": (_I, [_P]),
    "gla_matvec_q8_0": (_I, [_P, _P, _P, _I, _P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded HIP library (loaded once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not HIP_LIB_PATH.exists():
            raise ImportError(
                f"{HIP_LIB_PATH} is missing: build it with `python -m glint_amd.build` "
                "(the attention path has no CPU fallback)"
            )
        handle = C.CDLL(str(HIP_LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().gla_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != GLA_OK:
        raise GlaError(rc, last_error())


_synth = None


def synth() -> C.CDLL:
    """Seeded synthetic-input generator (host C library)."""
    global _synth
    if _synth is None:
        if not SYNTH_LIB_PATH.exists():
            raise ImportError(f"{SYNTH_LIB_PATH} is missing: build it with `python -m glint_amd.build`")
        h = C.CDLL(str(SYNTH_LIB_PATH))
        h.gs_fill_normal.argtypes = [C.c_uint64, _P, C.c_int64, _F]
        h.gs_fill_normal_rows.argtypes = [C.c_uint64, _P, C.c_int64, C.c_int64, C.c_int64, _F, _I]
        h.gs_uniform_int.argtypes = [C.c_uint64, C.c_int64, C.c_int64, C.c_int64, _P]
        h.gs_permutation.argtypes = [C.c_uint64, _P, C.c_int64]
        h.gs_xorshift_seq.argtypes = [C.c_uint64, C.c_int64, _P]
        h.gs_row_seed.argtypes = [C.c_uint64, C.c_uint64]
        h.gs_row_seed.restype = C.c_uint64
        _synth = h
    return _synth
