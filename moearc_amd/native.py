"""ctypes binding of ``libmoearc_attn.so`` (the C ABI in ``include/moearc_attn.h`` and
``include/moearc_kv.h``).

The library is loaded from this package's directory only. A missing library is an error, never a
fallback: there is no CPU implementation behind this package.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libmoearc_attn.so")
CODE_OBJECT = os.path.join(HERE, "moearc_attn_gfx950.co")

_c_ulong = ctypes.c_ulong
_vp = ctypes.c_void_p
_u32 = ctypes.c_uint

# (name, restype, argtypes) for every symbol the header declares.
SIGNATURES = {
    "moearc_ctx_create": (_vp, []),
    "moearc_ctx_destroy": (None, [_vp]),
    "moearc_ctx_stream": (_vp, [_vp]),
    "moearc_profile_events_enabled": (ctypes.c_int, [_vp]),
    "moearc_profile_events_reset": (ctypes.c_int, [_vp]),
    "moearc_profile_events_report": (ctypes.c_int, [_vp, ctypes.c_char_p, _c_ulong]),
    "moearc_sync": (ctypes.c_int, [_vp]),
    "moearc_zero": (ctypes.c_int, [_vp, _vp, _c_ulong]),
    "moearc_device_name": (ctypes.c_int, [_vp, ctypes.c_char_p, _c_ulong]),
    "moearc_alloc_device": (_vp, [_vp, _c_ulong]),
    "moearc_free_device": (None, [_vp, _vp]),
    "moearc_copy_h2d": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong]),
    "moearc_copy_h2d_async": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong]),
    "moearc_copy_d2h": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong]),
    "moearc_quantize_f16": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong]),
    "moearc_matvec_q": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _c_ulong, _c_ulong]),
    "moearc_matvec_q_batched": (ctypes.c_int, [_vp, _u32, _vp, _vp, _u32, _vp, _c_ulong, _c_ulong,
                                               _c_ulong]),
    "moearc_matvec_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_ulong, _c_ulong]),
    "moearc_add": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_ulong]),
    "moearc_read_floor": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong]),
    "moearc_mfma_floor": (ctypes.c_int, [_vp, _vp, _vp, _c_ulong, _c_ulong]),
    "moearc_attn_qkv": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_ulong]),
    "moearc_attn_block_chunk": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_ulong, _c_ulong, _vp, _vp, _vp]),
    "moearc_matmul_q": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _vp, _c_ulong, _c_ulong, _c_ulong]),
    "moearc_attn_out": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _vp, _c_ulong, _c_ulong]),
    "moearc_kv_append": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _c_ulong, _c_ulong,
                                        _c_ulong, _u32]),
    "moearc_kv_append_chunk": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_ulong,
                                              _c_ulong, _c_ulong, _c_ulong, _u32]),
    "moearc_attn_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_ulong, _c_ulong,
                                          _c_ulong, _c_ulong, _c_ulong, _c_ulong, ctypes.c_float,
                                          _u32]),
    "moearc_attn_decode_batched": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _c_ulong,
                                                  _vp, _vp, _vp, _c_ulong, _c_ulong, _c_ulong,
                                                  _c_ulong, _c_ulong, ctypes.c_float, _u32]),
    "moearc_attn_decode_batched_noalloc": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _c_ulong,
                                                          _vp, _vp, _vp, _c_ulong, _c_ulong, _c_ulong,
                                                          _c_ulong, _c_ulong, ctypes.c_float, _u32]),
    "moearc_attn_prefill": (ctypes.c_int, [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _c_ulong,
                                           _c_ulong, _c_ulong, _c_ulong, _c_ulong, _c_ulong,
                                           _c_ulong, ctypes.c_float, _u32]),
    "moearc_rope": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_ulong, _c_ulong, _c_ulong, _c_ulong,
                                   ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_float, ctypes.c_float, ctypes.c_int]),
    "moearc_rope_kv_append_chunk": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                   _c_ulong, _c_ulong, _c_ulong, _c_ulong,
                                                   _c_ulong, ctypes.c_float, ctypes.c_float,
                                                   ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                                   ctypes.c_float, ctypes.c_int, _u32]),
    # include/moearc_kv.h
    "moearc_kv_pool_create": (ctypes.c_int, [_u32, _u32, _u32, ctypes.POINTER(_vp)]),
    "moearc_kv_pool_destroy": (None, [_vp]),
    "moearc_kv_pool_last_error": (ctypes.c_int, [_vp, _vp, _vp]),
    "moearc_kv_pool_begin": (ctypes.c_int, [_vp, ctypes.c_uint64, _u32]),
    "moearc_kv_pool_append": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp, _vp]),
    "moearc_kv_pool_append_chunk": (ctypes.c_int, [_vp, ctypes.c_uint64, _u32, _vp, _vp]),
    "moearc_kv_pool_end": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp]),
    "moearc_kv_pool_pages": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp, _u32, _vp, _vp]),
    "moearc_kv_pool_can_admit": (ctypes.c_int, [_vp, _u32]),
    "moearc_kv_pool_usage": (ctypes.c_int, [_vp, _vp]),
    "moearc_kv_pool_block_tables": (ctypes.c_int, [_vp, _vp, _u32, _u32, _vp]),
    "moearc_kv_geometry": (ctypes.c_int, [_u32, _u32, _u32, _u32, _vp, _vp]),
    "moearc_kv_ring_table": (ctypes.c_int, [_u32, _u32, _vp]),
}

_lib = None


class NativeLibraryMissing(RuntimeError):
    """The HIP build of this package is absent; run ``python -m moearc_amd.build``."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY) or not os.path.exists(CODE_OBJECT):
        raise NativeLibraryMissing(
            f"{LIBRARY} / {CODE_OBJECT} not built; run `python -m moearc_amd.build`")
    lib = ctypes.CDLL(LIBRARY)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
