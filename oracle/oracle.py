"""ctypes wrapper over the CPU oracle (moearc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg, always as the checker or the timed CPU baseline, never as the product
path. The product library (``moearc_amd``) does not import this module.

Each wrapper names the reference function it restates (paths relative to the reference repo).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

KV_F32 = 0
KV_F16 = 1

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_sz = ctypes.c_size_t
_i32p = ctypes.POINTER(ctypes.c_int32)
_f = ctypes.c_float


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_splitmix64_next.argtypes = [_u64p]
        L.orc_splitmix64_next.restype = ctypes.c_uint64
        L.orc_rng_unit.argtypes = [_u64p]
        L.orc_rng_unit.restype = ctypes.c_float
        L.orc_rng_fill_unit.argtypes = [_u64p, _f32p, _sz]
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, _sz]
        L.orc_f16_to_f32_n.argtypes = [_u16p, _f32p, _sz]
        L.orc_kv_store_value.argtypes = [ctypes.c_float, ctypes.c_uint32]
        L.orc_kv_store_value.restype = ctypes.c_float
        L.orc_kv_index.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _sz, _sz, _sz, _sz, _sz]
        L.orc_kv_index.restype = _sz
        L.orc_kv_append.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_uint32,
                                    _sz, _sz, _sz, ctypes.c_uint32]
        L.orc_kv_append_raw.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _f32p, _f32p,
                                        ctypes.c_uint32, ctypes.c_uint32, _sz, _sz, _sz,
                                        ctypes.c_uint32]
        L.orc_attn_decode.argtypes = [_f32p, _f64p, _f32p, ctypes.c_void_p, ctypes.c_void_p, _u32p,
                                      _f32p, _sz, _sz, _sz, _sz, _sz, _sz, ctypes.c_float,
                                      ctypes.c_uint32, _f64p]
        L.orc_attn_decode.restype = ctypes.c_int
        L.orc_attn_decode_batched.argtypes = [_f32p, _f32p, ctypes.c_void_p, ctypes.c_void_p, _u32p,
                                              _sz, _u32p, _u32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                              ctypes.c_float, ctypes.c_uint32, _f64p, _sz,
                                              ctypes.c_int]
        L.orc_attn_decode_batched.restype = ctypes.c_int
        L.orc_attn_prefill.argtypes = [_f32p, _f32p, ctypes.c_void_p, ctypes.c_void_p, _u32p, _f32p,
                                       _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz,
                                       ctypes.c_float, ctypes.c_uint32, _f64p, ctypes.c_int]
        L.orc_attn_prefill.restype = ctypes.c_int
        L.orc_rope.argtypes = [_f32p, _f32p, _i32p, _sz, _sz, _sz, _sz, _f, ctypes.c_int]
        L.orc_rope_yarn.argtypes = [_f64p, _f32p, _i32p, _sz, _sz, _sz, _sz, _f, _f, _f, _f, _f, _f,
                                    ctypes.c_int]
        L.orc_rope_kv_append_chunk.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _f32p, _f32p, _i32p,
                                               _u32p, _u32p, _sz, _sz, _sz, _sz, _sz, _f, _f, _f, _f,
                                               _f, _f, ctypes.c_int, ctypes.c_uint32, _f64p, _f32p]
        L.orc_block_bytes.argtypes = [ctypes.c_uint32]
        L.orc_block_bytes.restype = _sz
        L.orc_block_elems.argtypes = [ctypes.c_uint32]
        L.orc_block_elems.restype = _sz
        L.orc_e8m0_half.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_half.restype = ctypes.c_float
        L.orc_dequant.argtypes = [ctypes.c_uint32, ctypes.c_void_p, _sz, _f32p]
        L.orc_dequant.restype = ctypes.c_int
        L.orc_matvec_q.argtypes = [ctypes.c_uint32, ctypes.c_void_p, _f32p, _sz, _sz, _f32p, _f64p,
                                   ctypes.c_int]
        L.orc_matvec_q.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


class OracleRefusal(ValueError):
    """The oracle refused the arguments (the reference's -2 / BadArgument)."""


# ---- RNG (crates/moearc-kernels/tests/common/mod.rs:11-37) -----------------------------------

class Rng:
    """SplitMix64 with the reference tests' ``unit()`` (tests/common/mod.rs:11-37)."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        return int(lib().orc_splitmix64_next(ctypes.byref(self.state)))

    def unit(self) -> float:
        return float(lib().orc_rng_unit(ctypes.byref(self.state)))

    def vec_unit(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().orc_rng_fill_unit(ctypes.byref(self.state), _p(out, _f32p), n)
        return out


# ---- f16 codecs (reference.rs:123-149, :647-691) ---------------------------------------------

def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_f16_n(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16).ravel()
    out = np.empty(bits.size, np.float32)
    lib().orc_f16_to_f32_n(_p(bits, _u16p), _p(out, _f32p), bits.size)
    return out


def kv_store_value(v: float, kv_type: int) -> float:
    return float(lib().orc_kv_store_value(ctypes.c_float(v), kv_type))


# ---- KV layout (reference.rs:767-802) ---------------------------------------------------------

def kv_index(page, slot, head, d, n_kv_heads, head_dim, page_tokens) -> int:
    return int(lib().orc_kv_index(page, slot, head, d, n_kv_heads, head_dim, page_tokens))


def kv_append(k_pages, v_pages, k, v, page, slot, n_kv_heads, head_dim, page_tokens, kv_type):
    """Host-mirror append into f32 pools (reference.rs:781-802)."""
    assert k_pages.dtype == np.float32 and k_pages.flags.c_contiguous
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    lib().orc_kv_append(_p(k_pages, _f32p), _p(v_pages, _f32p), _p(k, _f32p), _p(v, _f32p),
                        page, slot, n_kv_heads, head_dim, page_tokens, kv_type)


def kv_append_raw(k_pages, v_pages, k, v, page, slot, n_kv_heads, head_dim, page_tokens, kv_type):
    """Device-format append: pools hold stored bytes (f32 or f16 bits)."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    lib().orc_kv_append_raw(k_pages.ctypes.data, v_pages.ctypes.data, _p(k, _f32p), _p(v, _f32p),
                            page, slot, n_kv_heads, head_dim, page_tokens, kv_type)


# ---- attention (reference.rs:821-873 + sink, kernels.cpp:1864-1880) --------------------------

def _pages(p, kv_type):
    want = np.uint16 if kv_type == KV_F16 else np.float32
    p = np.ascontiguousarray(p)
    if p.dtype != want:
        raise TypeError(f"pages must be {want} for kv_type {kv_type}, got {p.dtype}")
    return p


def attn_decode(q, k_pages, v_pages, block_table, n_heads, n_kv_heads, head_dim, kv_begin, n_kv,
                page_tokens, scale, kv_type=KV_F32, sinks=None, f64=False):
    """Single-query paged attention; returns [n_heads*head_dim] (f32, or f64 if ``f64``)."""
    q = np.ascontiguousarray(q, np.float32).ravel()
    kp, vp = _pages(k_pages, kv_type), _pages(v_pages, kv_type)
    bt = np.ascontiguousarray(block_table, np.uint32)
    s = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    out = np.empty(n_heads * head_dim, np.float32)
    out_d = np.empty(n_heads * head_dim, np.float64)
    scratch = np.empty(max(1, n_kv), np.float64)
    rc = lib().orc_attn_decode(_p(out, _f32p), _p(out_d, _f64p), _p(q, _f32p), kp.ctypes.data,
                               vp.ctypes.data, _p(bt, _u32p), _p(s, _f32p), n_heads, n_kv_heads,
                               head_dim, kv_begin, n_kv, page_tokens, ctypes.c_float(scale),
                               kv_type, _p(scratch, _f64p))
    if rc != 0:
        raise OracleRefusal(f"orc_attn_decode refused its arguments (rc {rc})")
    return out_d if f64 else out


def attn_decode_batched(q, k_pages, v_pages, block_tables, kv_begin, n_kv, n_heads, n_kv_heads,
                        head_dim, page_tokens, scale, kv_type=KV_F16, sinks=None, n_threads=1):
    """n_seqs independent decode calls; q [n_seqs][n_heads][head_dim]; block_tables 2-D."""
    bts = np.ascontiguousarray(block_tables, np.uint32)
    assert bts.ndim == 2
    kb = np.ascontiguousarray(kv_begin, np.uint32)
    nk = np.ascontiguousarray(n_kv, np.uint32)
    n_seqs = kb.size
    q = np.ascontiguousarray(q, np.float32)
    kp, vp = _pages(k_pages, kv_type), _pages(v_pages, kv_type)
    s = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    max_span = int((nk.astype(np.int64) - kb.astype(np.int64)).max())
    threads = max(1, int(n_threads))
    scratch = np.empty(threads * max(1, max_span), np.float64)
    out = np.empty((n_seqs, n_heads, head_dim), np.float32)
    rc = lib().orc_attn_decode_batched(_p(out, _f32p), _p(q, _f32p), kp.ctypes.data,
                                       vp.ctypes.data, _p(bts, _u32p), bts.shape[1],
                                       _p(kb, _u32p), _p(nk, _u32p), _p(s, _f32p), n_seqs,
                                       n_heads, n_kv_heads, head_dim, page_tokens,
                                       ctypes.c_float(scale), kv_type, _p(scratch, _f64p),
                                       max_span, threads)
    if rc != 0:
        raise OracleRefusal(f"orc_attn_decode_batched refused its arguments (rc {rc})")
    return out


def attn_prefill(q, k_pages, v_pages, block_table, n_q, pos0, n_swa, n_heads, n_kv_heads,
                 head_dim, page_tokens, scale, kv_type=KV_F16, sinks=None, rows=None,
                 n_threads=1):
    """Chunked prefill as repeated decode (moe.rs:1856-1862). ``rows`` = (begin, end, step)
    computes only those rows; the others are left NaN."""
    q = np.ascontiguousarray(q, np.float32)
    kp, vp = _pages(k_pages, kv_type), _pages(v_pages, kv_type)
    bt = np.ascontiguousarray(block_table, np.uint32)
    s = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    rb, re, rs = rows if rows is not None else (0, n_q, 1)
    threads = max(1, int(n_threads))
    scratch = np.empty(threads * (pos0 + n_q), np.float64)
    out = np.full((n_q, n_heads, head_dim), np.nan, np.float32)
    rc = lib().orc_attn_prefill(_p(out, _f32p), _p(q, _f32p), kp.ctypes.data, vp.ctypes.data,
                                _p(bt, _u32p), _p(s, _f32p), n_q, pos0, n_swa, rb, re, rs,
                                n_heads, n_kv_heads, head_dim, page_tokens, ctypes.c_float(scale),
                                kv_type, _p(scratch, _f64p), threads)
    if rc != 0:
        raise OracleRefusal(f"orc_attn_prefill refused its arguments (rc {rc})")
    return out


# ---- RoPE (reference.rs:468-505; kernels.cpp:1399-1468) -------------------------------------

def rope(src, pos, n_tokens, n_heads, head_dim, n_dims, freq_base, neox=True):
    """reference::rope: iterated f32 angle table, f32 rotation; returns f32."""
    src = np.ascontiguousarray(src, np.float32).reshape(-1)
    pos = np.ascontiguousarray(pos, np.int32)
    out = np.empty_like(src)
    lib().orc_rope(_p(out, _f32p), _p(src, _f32p), _p(pos, _i32p), n_tokens, n_heads, head_dim,
                   n_dims, _f(freq_base), int(bool(neox)))
    return out


def rope_yarn(src, pos, n_tokens, n_heads, head_dim, n_dims, freq_base, freq_scale=1.0,
              ext_factor=0.0, attn_factor=1.0, corr_lo=0.0, corr_hi=0.0, neox=True):
    """The kernel's closed form with YaRN, evaluated in f64; returns f64."""
    src = np.ascontiguousarray(src, np.float32).reshape(-1)
    pos = np.ascontiguousarray(pos, np.int32)
    out = np.empty(src.shape, np.float64)
    lib().orc_rope_yarn(_p(out, _f64p), _p(src, _f32p), _p(pos, _i32p), n_tokens, n_heads, head_dim,
                        n_dims, _f(freq_base), _f(freq_scale), _f(ext_factor), _f(attn_factor),
                        _f(corr_lo), _f(corr_hi), int(bool(neox)))
    return out


def rope_kv_append_chunk(k_pages, v_pages, k, v, pos, page_ids, slots, n_tok, n_kv_heads, head_dim,
                         page_tokens, n_dims, freq_base, scaling=(1.0, 0.0, 1.0, 0.0, 0.0), neox=True,
                         kv_type=KV_F16):
    """The engine's per-token rope-then-append over a chunk, into device-format pools (in place)."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    pos = np.ascontiguousarray(pos, np.int32)
    pg = np.ascontiguousarray(page_ids, np.uint32)
    sl = np.ascontiguousarray(slots, np.uint32)
    row = n_kv_heads * head_dim
    sd, sf = np.empty(row, np.float64), np.empty(row, np.float32)
    fs, ext, att, clo, chi = (float(x) for x in scaling)
    lib().orc_rope_kv_append_chunk(k_pages.ctypes.data, v_pages.ctypes.data, _p(k, _f32p), _p(v, _f32p),
                                   _p(pos, _i32p), _p(pg, _u32p), _p(sl, _u32p), n_tok, n_kv_heads,
                                   head_dim, page_tokens, n_dims, _f(freq_base), _f(fs), _f(ext), _f(att),
                                   _f(clo), _f(chi), int(bool(neox)), kv_type, _p(sd, _f64p), _p(sf, _f32p))


# ---- GGUF block formats and matvec (crates/moearc-kernels/src/reference.rs:42-336) ---------------

def block_bytes(ty: int) -> int:
    return int(lib().orc_block_bytes(ty))


def block_elems(ty: int) -> int:
    return int(lib().orc_block_elems(ty))


def e8m0_half(x: int) -> float:
    """2^(x - 128) as reference.rs:66-70 builds it (subnormal below x = 2)."""
    return float(lib().orc_e8m0_half(x))


def dequant(ty: int, src, nblocks: int) -> np.ndarray:
    """Expand nblocks blocks to f32 (reference.rs:168-192)."""
    src = np.ascontiguousarray(np.frombuffer(bytes(src), np.uint8) if not isinstance(src, np.ndarray)
                               else src.view(np.uint8).reshape(-1))
    if src.size < nblocks * block_bytes(ty):
        raise OracleRefusal(f"{nblocks} blocks need {nblocks * block_bytes(ty)} bytes, got {src.size}")
    out = np.zeros(nblocks * max(block_elems(ty), 1), np.float32)
    if lib().orc_dequant(ty, src.ctypes.data, nblocks, _p(out, _f32p)):
        raise OracleRefusal(f"unknown type {ty}")
    return out


def matvec_q(ty: int, w, x, n_rows: int, n_cols: int, n_threads: int = 8):
    """(out f32 [n_rows], absum f64 [n_rows]) with out[r] = W[r] . x accumulated in f64 over the
    f32-dequantised row (reference.rs:305-321) and absum[r] = sum |W[r][c] x[c]|."""
    w = np.ascontiguousarray(np.asarray(w).view(np.uint8).reshape(-1))
    x = np.ascontiguousarray(x, np.float32)
    assert x.size >= n_cols
    if n_cols % max(block_elems(ty), 1) or not block_bytes(ty):
        raise OracleRefusal(f"type {ty}: {n_cols} columns")
    assert w.size >= n_rows * n_cols // block_elems(ty) * block_bytes(ty)
    out = np.zeros(n_rows, np.float32)
    absum = np.zeros(n_rows, np.float64)
    lib().orc_matvec_q(ty, w.ctypes.data, _p(x, _f32p), n_rows, n_cols, _p(out, _f32p),
                       _p(absum, _f64p), n_threads)
    return out, absum
