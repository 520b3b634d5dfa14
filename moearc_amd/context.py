"""Python mirror of the reference's safe wrapper (crates/moearc-kernels/src/lib.rs) over the C ABI.

Same names, argument meaning and error behaviour as the Rust ``Context``: a wrapper submits and
returns; a non-zero return code drains the stream before it is reported (lib.rs:198-215); ``-2``
is ``BadArgument`` and any other failure ``Failed`` (lib.rs:157-165); buffer sizes are checked
before the call (``BufferTooSmall``, lib.rs:1216-1221); ``MOEARC_SYNC_EACH=1`` waits after every
launch (lib.rs:183-195). Device memory is owned by ``DeviceBuffer`` and freed when it is dropped.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Optional

import numpy as np

from . import native


class KernelError(Exception):
    """Base of the wrapper's errors (lib.rs ``KernelError``)."""


class NoDevice(KernelError):
    pass


class OutOfMemory(KernelError):
    def __init__(self, nbytes: int):
        super().__init__(f"device allocation of {nbytes} bytes failed")
        self.nbytes = nbytes


class BadArgument(KernelError):
    pass


class Failed(KernelError):
    pass


class BufferTooSmall(KernelError):
    def __init__(self, what: str, need: int, have: int):
        super().__init__(f"{what}: need {need} bytes, have {have}")
        self.what, self.need, self.have = what, need, have


class KvType(enum.IntEnum):
    """How a KV page stores its numbers; the value is the GGUF type id (reference.rs:728-752)."""
    F32 = 0
    F16 = 1

    @property
    def elem_bytes(self) -> int:
        return 4 if self is KvType.F32 else 2


OUT_F32 = 0
OUT_F16 = 1


class RopeKind(enum.IntEnum):
    """Pairing of rotated channels (reference.rs:451-457): NORMAL (2p, 2p+1), NEOX (p, p + n_dims/2)."""
    NORMAL = 0
    NEOX = 1


class RopeScaling:
    """YaRN parameters as the RoPE kernel takes them (reference.rs:536-590)."""

    def __init__(self, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, corr_lo=0.0, corr_hi=0.0):
        self.freq_scale, self.ext_factor, self.attn_factor = freq_scale, ext_factor, attn_factor
        self.corr_lo, self.corr_hi = corr_lo, corr_hi

    @classmethod
    def yarn(cls, n_dims, n_ctx_orig, freq_base, factor, beta_fast=32.0, beta_slow=1.0):
        """From the GGUF keys and the model geometry: ggml_rope_yarn_corr_dims (reference.rs:573-590)."""
        f32 = np.float32

        def corr(beta):
            return f32(f32(n_dims) * np.log(f32(n_ctx_orig) / (f32(beta) * f32(2.0) * f32(np.pi)))
                       / (f32(2.0) * np.log(f32(freq_base))))
        return cls(float(f32(1.0) / f32(factor)), 1.0, 1.0, float(max(np.floor(corr(beta_fast)), 0.0)),
                   float(min(np.ceil(corr(beta_slow)), n_dims - 1.0)))

    def args(self):
        return (self.freq_scale, self.ext_factor, self.attn_factor, self.corr_lo, self.corr_hi)


RopeScaling.NONE = RopeScaling()


class DeviceBuffer:
    """An owned device allocation (lib.rs ``DeviceBuffer``)."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int):
        self.ctx, self.ptr, self.len = ctx, ptr, nbytes

    def require(self, what: str, need: int) -> None:
        if self.len < need:
            raise BufferTooSmall(what, need, self.len)

    def free(self) -> None:
        if self.ptr:
            self.ctx._lib.moearc_free_device(self.ctx.raw, self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            if self.ctx.raw:
                self.free()
        except Exception:
            pass


def _check(rc: int, what: str) -> None:
    if rc == 0:
        return
    if rc == -2:
        raise BadArgument(what)
    raise Failed(what)


class Context:
    """A HIP stream on the current device plus the loaded kernels (lib.rs ``Context``)."""

    def __init__(self):
        self._lib = native.load()
        self.raw = self._lib.moearc_ctx_create()
        if not self.raw:
            raise NoDevice("moearc_ctx_create returned NULL (no HIP device, or code object missing)")
        self.sync_each = os.environ.get("MOEARC_SYNC_EACH") == "1"

    # ---- lifecycle ----------------------------------------------------------------------------
    def close(self) -> None:
        if self.raw:
            self._lib.moearc_ctx_destroy(self.raw)
            self.raw = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def finish(self, rc: int, what: str) -> None:
        """Drain before reporting an error, so nothing in flight outlives the caller's buffers."""
        if rc != 0:
            self._lib.moearc_sync(self.raw)
            _check(rc, what)
        elif self.sync_each:
            self.sync()

    def sync(self) -> None:
        _check(self._lib.moearc_sync(self.raw), "stream synchronisation")

    @property
    def stream(self) -> int:
        return self._lib.moearc_ctx_stream(self.raw) or 0

    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        if self._lib.moearc_device_name(self.raw, buf, 256) != 0:
            raise Failed("querying the device name")
        return buf.value.decode(errors="replace")

    # ---- profiling ----------------------------------------------------------------------------
    def profile_events_enabled(self) -> bool:
        return bool(self._lib.moearc_profile_events_enabled(self.raw))

    def profile_events_reset(self) -> None:
        _check(self._lib.moearc_profile_events_reset(self.raw), "profile reset")

    def profile_events_report(self) -> dict:
        """{key: (nanoseconds, calls)} from ``moearc_profile_events_report``."""
        buf = ctypes.create_string_buffer(1 << 16)
        _check(self._lib.moearc_profile_events_report(self.raw, buf, 1 << 16), "profile report")
        out = {}
        for line in buf.value.decode().splitlines():
            parts = line.rsplit(" ", 2)
            if len(parts) == 3:
                out[parts[0]] = (int(parts[1]), int(parts[2]))
        return out

    # ---- memory -------------------------------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        ptr = self._lib.moearc_alloc_device(self.raw, int(nbytes))
        if not ptr:
            raise OutOfMemory(nbytes)
        return DeviceBuffer(self, ptr, int(nbytes))

    def alloc_n(self, dtype, n: int) -> DeviceBuffer:
        return self.alloc(int(n) * np.dtype(dtype).itemsize)

    def upload_slice(self, dst: DeviceBuffer, src: np.ndarray) -> None:
        src = np.ascontiguousarray(src)
        dst.require("upload destination", src.nbytes)
        _check(self._lib.moearc_copy_h2d(self.raw, dst.ptr, src.ctypes.data, src.nbytes), "upload")

    def upload(self, src: np.ndarray) -> DeviceBuffer:
        src = np.ascontiguousarray(src)
        buf = self.alloc(max(1, src.nbytes))
        self.upload_slice(buf, src)
        return buf

    def download_slice(self, dst: np.ndarray, src: DeviceBuffer) -> np.ndarray:
        assert dst.flags.c_contiguous
        src.require("download source", dst.nbytes)
        _check(self._lib.moearc_copy_d2h(self.raw, dst.ctypes.data, src.ptr, dst.nbytes), "download")
        return dst

    def download(self, src: DeviceBuffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        return self.download_slice(out, src)

    def zero(self, dst: DeviceBuffer, n: int) -> None:
        dst.require("zero destination", n * 4)
        self.finish(self._lib.moearc_zero(self.raw, dst.ptr, n), "zero")

    # ---- kernels ------------------------------------------------------------------------------
    def quantize_f16(self, dst: DeviceBuffer, src: DeviceBuffer, n: int) -> None:
        """f32 -> f16 RNE (kernels.cpp:1727-1735)."""
        src.require("f32 source", n * 4)
        dst.require("f16 destination", n * 2)
        self.finish(self._lib.moearc_quantize_f16(self.raw, dst.ptr, src.ptr, n), "f16 narrowing")

    def kv_append(self, k_pages: DeviceBuffer, v_pages: DeviceBuffer, k: DeviceBuffer,
                  v: DeviceBuffer, page_id: int, slot: int, n_kv_heads: int, head_dim: int,
                  page_tokens: int, kv: KvType) -> None:
        """One token's K and V into a page slot (lib.rs:1079-1114)."""
        kv = KvType(kv)
        row = n_kv_heads * head_dim
        k.require("key vector", row * 4)
        v.require("value vector", row * 4)
        need = (page_id * page_tokens + slot + 1) * row * kv.elem_bytes
        k_pages.require("key pages", need)
        v_pages.require("value pages", need)
        rc = self._lib.moearc_kv_append(self.raw, k_pages.ptr, v_pages.ptr, k.ptr, v.ptr, page_id,
                                        slot, n_kv_heads, head_dim, page_tokens, int(kv))
        self.finish(rc, "KV append")

    def kv_append_chunk(self, k_pages: DeviceBuffer, v_pages: DeviceBuffer, k: DeviceBuffer,
                        v: DeviceBuffer, page_ids: DeviceBuffer, slots: DeviceBuffer, n_tok: int,
                        n_kv_heads: int, head_dim: int, page_tokens: int, kv: KvType) -> None:
        """n_tok tokens' K and V at (page_ids[t], slots[t]); equal to n_tok kv_append calls."""
        row = n_kv_heads * head_dim
        k.require("key rows", n_tok * row * 4)
        v.require("value rows", n_tok * row * 4)
        page_ids.require("page ids", n_tok * 4)
        slots.require("slots", n_tok * 4)
        rc = self._lib.moearc_kv_append_chunk(self.raw, k_pages.ptr, v_pages.ptr, k.ptr, v.ptr,
                                              page_ids.ptr, slots.ptr, n_tok, n_kv_heads,
                                              head_dim, page_tokens, int(KvType(kv)))
        self.finish(rc, "KV chunk append")

    def rope(self, dst: DeviceBuffer, src: DeviceBuffer, pos: DeviceBuffer, n_tokens: int,
             n_heads: int, head_dim: int, n_dims: int, freq_base: float,
             scaling: Optional[RopeScaling] = None, kind: RopeKind = RopeKind.NEOX) -> None:
        """RoPE with optional YaRN (lib.rs:834-870): dst, src f32 [n_tokens][n_heads][head_dim]."""
        n = n_tokens * n_heads * head_dim
        src.require("rope input", n * 4)
        dst.require("rope output", n * 4)
        pos.require("rope positions", n_tokens * 4)
        sc = scaling or RopeScaling.NONE
        rc = self._lib.moearc_rope(self.raw, dst.ptr, src.ptr, pos.ptr, n_tokens, n_heads, head_dim,
                                   n_dims, freq_base, *sc.args(), int(RopeKind(kind)))
        self.finish(rc, "rope")

    def rope_kv_append_chunk(self, k_pages: DeviceBuffer, v_pages: DeviceBuffer, k: DeviceBuffer,
                             v: DeviceBuffer, pos: DeviceBuffer, page_ids: DeviceBuffer,
                             slots: DeviceBuffer, n_tok: int, n_kv_heads: int, head_dim: int,
                             page_tokens: int, n_dims: int, freq_base: float,
                             scaling: Optional[RopeScaling] = None,
                             kind: RopeKind = RopeKind.NEOX, kv: KvType = KvType.F16) -> None:
        """K rotated as rope() would, then K and V appended as kv_append_chunk() would, in one pass."""
        row = n_kv_heads * head_dim
        k.require("key rows", n_tok * row * 4)
        v.require("value rows", n_tok * row * 4)
        pos.require("rope positions", n_tok * 4)
        page_ids.require("page ids", n_tok * 4)
        slots.require("slots", n_tok * 4)
        sc = scaling or RopeScaling.NONE
        rc = self._lib.moearc_rope_kv_append_chunk(
            self.raw, k_pages.ptr, v_pages.ptr, k.ptr, v.ptr, pos.ptr, page_ids.ptr, slots.ptr,
            n_tok, n_kv_heads, head_dim, page_tokens, n_dims, freq_base, *sc.args(),
            int(RopeKind(kind)), int(KvType(kv)))
        self.finish(rc, "RoPE + KV chunk append")

    def attn_decode(self, out, q, k_pages, v_pages, block_table, n_heads, n_kv_heads, head_dim,
                    n_kv, page_tokens, scale, kv) -> None:
        """Full causal attention over every cached key (lib.rs:1135-1171)."""
        self.attn_decode_ext(out, q, k_pages, v_pages, block_table, None, n_heads, n_kv_heads,
                             head_dim, 0, n_kv, page_tokens, scale, kv)

    def attn_decode_ext(self, out: DeviceBuffer, q: DeviceBuffer, k_pages: DeviceBuffer,
                        v_pages: DeviceBuffer, block_table: DeviceBuffer,
                        sinks: Optional[DeviceBuffer], n_heads: int, n_kv_heads: int,
                        head_dim: int, kv_begin: int, n_kv: int, page_tokens: int, scale: float,
                        kv: KvType) -> None:
        """Attention with sinks and an explicit key span [kv_begin, n_kv) (lib.rs:1188-1242)."""
        if n_kv_heads == 0 or n_heads % n_kv_heads != 0:
            raise BadArgument("n_heads is not a multiple of n_kv_heads")
        if page_tokens == 0:
            raise BadArgument("page_tokens must be non-zero")
        if kv_begin >= n_kv:
            raise BadArgument("kv_begin is not before n_kv")
        q.require("query", n_heads * head_dim * 4)
        out.require("attention output", n_heads * head_dim * 4)
        block_table.require("block table", -(-n_kv // page_tokens) * 4)
        if sinks is not None:
            sinks.require("attention sinks", n_heads * 4)
        rc = self._lib.moearc_attn_decode(self.raw, out.ptr, q.ptr, k_pages.ptr, v_pages.ptr,
                                          block_table.ptr, sinks.ptr if sinks is not None else None,
                                          n_heads, n_kv_heads, head_dim, kv_begin, n_kv,
                                          page_tokens, float(scale), int(KvType(kv)))
        self.finish(rc, "paged attention")

    def attn_decode_batched(self, out: DeviceBuffer, q: DeviceBuffer, k_pages: DeviceBuffer,
                            v_pages: DeviceBuffer, block_tables: DeviceBuffer, bt_stride: int,
                            kv_begin, n_kv, sinks: Optional[DeviceBuffer], n_heads: int,
                            n_kv_heads: int, head_dim: int, page_tokens: int, scale: float,
                            kv: KvType, out_type: int = OUT_F32) -> None:
        """Ragged batch of decode calls; kv_begin/n_kv are host sequences of per-sequence ints."""
        kb = np.ascontiguousarray(kv_begin, np.uint32)
        nk = np.ascontiguousarray(n_kv, np.uint32)
        n_seqs = kb.size
        if nk.size != n_seqs:
            raise BadArgument("kv_begin and n_kv differ in length")
        out_bytes = 2 if out_type == OUT_F16 else 4
        q.require("query", n_seqs * n_heads * head_dim * 4)
        out.require("attention output", n_seqs * n_heads * head_dim * out_bytes)
        block_tables.require("block tables", n_seqs * bt_stride * 4)
        if sinks is not None:
            sinks.require("attention sinks", n_heads * 4)
        rc = self._lib.moearc_attn_decode_batched(
            self.raw, out.ptr, out_type, q.ptr, k_pages.ptr, v_pages.ptr, block_tables.ptr,
            bt_stride, kb.ctypes.data, nk.ctypes.data, sinks.ptr if sinks is not None else None,
            n_seqs, n_heads, n_kv_heads, head_dim, page_tokens, float(scale), int(KvType(kv)))
        self.finish(rc, "batched paged attention")

    def attn_prefill(self, out: DeviceBuffer, q: DeviceBuffer, k_pages: DeviceBuffer,
                     v_pages: DeviceBuffer, block_table: DeviceBuffer,
                     sinks: Optional[DeviceBuffer], n_q: int, pos0: int, n_swa: int,
                     n_heads: int, n_kv_heads: int, head_dim: int, page_tokens: int,
                     scale: float, kv: KvType = KvType.F16, out_type: int = OUT_F32) -> None:
        """Chunked prefill: row i equals decode at n_kv = pos0+i+1 (moe.rs:1856-1862)."""
        out_bytes = 2 if out_type == OUT_F16 else 4
        q.require("query (f16)", n_q * n_heads * head_dim * 2)
        out.require("attention output", n_q * n_heads * head_dim * out_bytes)
        block_table.require("block table", -(-(pos0 + n_q) // max(1, page_tokens)) * 4)
        if sinks is not None:
            sinks.require("attention sinks", n_heads * 4)
        rc = self._lib.moearc_attn_prefill(self.raw, out.ptr, out_type, q.ptr, k_pages.ptr,
                                           v_pages.ptr, block_table.ptr,
                                           sinks.ptr if sinks is not None else None, n_q, pos0,
                                           n_swa, n_heads, n_kv_heads, head_dim, page_tokens,
                                           float(scale), int(KvType(kv)))
        self.finish(rc, "chunked prefill attention")

    # ---- attention projections -------------------------------------------------------------
    def matvec_q(self, ty, out: DeviceBuffer, w: DeviceBuffer, x: DeviceBuffer, n_rows: int,
                  n_cols: int) -> None:
        """out[r] = W[r] . x against quantised weights (lib.rs matvec_q, kernels.cpp:1046-1111)."""
        ty = QuantType(ty)
        if n_cols % ty.block_elems:
            raise BadArgument(f"{ty.name}: {n_cols} columns is not a whole number of blocks")
        w.require("weights", n_rows * ty.row_bytes(n_cols))
        x.require("activation", n_cols * 4)
        out.require("output", n_rows * 4)
        self.finish(self._lib.moearc_matvec_q(self.raw, int(ty), out.ptr, w.ptr, x.ptr, n_rows, n_cols),
                    f"matvec {ty.name}")


    def matvec_q_batched(self, ty, out: DeviceBuffer, ws, x: DeviceBuffer, x_stride: int, n_rows: int,
                          n_cols: int) -> None:
        """len(ws) matrices in one launch (lib.rs matvec_q_batched, kernels.cpp:1146-1206)."""
        ty = QuantType(ty)
        if n_cols % ty.block_elems:
            raise BadArgument(f"{ty.name}: {n_cols} columns is not a whole number of blocks")
        for w in ws:
            w.require("weights", n_rows * ty.row_bytes(n_cols))
        x.require("activation", ((len(ws) - 1) * x_stride + n_cols) * 4)
        out.require("output", len(ws) * n_rows * 4)
        ptrs = _ptr_array(ws)
        self.finish(self._lib.moearc_matvec_q_batched(self.raw, int(ty), out.ptr, ptrs, len(ws), x.ptr,
                                                      x_stride, n_rows, n_cols), f"batched matvec {ty.name}")


    def matvec_f32(self, out: DeviceBuffer, w: DeviceBuffer, x: DeviceBuffer, n_rows: int,
                    n_cols: int) -> None:
        """out[r] = W[r] . x against f32 weights (kernels.cpp:1116-1135)."""
        w.require("weights", n_rows * n_cols * 4)
        x.require("activation", n_cols * 4)
        out.require("output", n_rows * 4)
        self.finish(self._lib.moearc_matvec_f32(self.raw, out.ptr, w.ptr, x.ptr, n_rows, n_cols),
                    "matvec f32")


    def read_floor(self, out: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
        """Calibration read of nbytes at src; out[g] = xor of the 32-bit words of its g-th 64 KiB."""
        src.require("source", nbytes)
        out.require("checksums", (nbytes + 65535) // 65536 * 4)
        self.finish(self._lib.moearc_read_floor(self.raw, out.ptr, src.ptr, nbytes), "read_floor")

    def mfma_floor(self, out: DeviceBuffer, src: DeviceBuffer, n_wgs: int, iters: int) -> None:
        """Calibration of the matrix cores (moearc_mfma_floor): n_wgs x 4 waves of dense f16 MFMA
        chains over the operands at src (32 KiB per work-group); out[w] = wave w's accumulator sum."""
        src.require("operands", n_wgs * 32768)
        out.require("checksums", n_wgs * 4 * 4)
        self.finish(self._lib.moearc_mfma_floor(self.raw, out.ptr, src.ptr, n_wgs, iters), "mfma_floor")

    def add(self, out: DeviceBuffer, a: DeviceBuffer, b: DeviceBuffer, n: int) -> None:
        """out = a + b, element-wise (kernels.cpp:1676-1683)."""
        for buf, what in ((out, "output"), (a, "left operand"), (b, "right operand")):
            buf.require(what, n * 4)
        self.finish(self._lib.moearc_add(self.raw, out.ptr, a.ptr, b.ptr, n), "add")


    def matmul_q(self, ty, y: DeviceBuffer, w: DeviceBuffer, x: DeviceBuffer, bias: Optional[DeviceBuffer],
                 n_tok: int, n_rows: int, n_cols: int) -> None:
        """A chunk's projection on MFMA: y[t] = W x[t] (+ bias), Q8_0 or F16 weights."""
        ty = QuantType(ty)
        w.require("weights", n_rows * ty.row_bytes(n_cols))
        x.require("activations", n_tok * n_cols * 4)
        y.require("output", n_tok * n_rows * 4)
        self.finish(self._lib.moearc_matmul_q(self.raw, int(ty), y.ptr, w.ptr, x.ptr,
                                              bias.ptr if bias is not None else None, n_tok, n_rows, n_cols),
                    f"matmul {ty.name}")

    def attn_out(self, ty, h: DeviceBuffer, w: DeviceBuffer, bias: Optional[DeviceBuffer], attn: DeviceBuffer,
                 n_rows: int, n_cols: int) -> None:
        """h += W attn (+ bias) in one launch (attn.proj and the residual add, moe.rs:2063-2071)."""
        ty = QuantType(ty)
        w.require("weights", n_rows * ty.row_bytes(n_cols))
        attn.require("attention output", n_cols * 4)
        h.require("residual", n_rows * 4)
        self.finish(self._lib.moearc_attn_out(self.raw, int(ty), h.ptr, w.ptr, bias.ptr if bias is not None else None,
                                              attn.ptr, n_rows, n_cols), f"attn out {ty.name}")

    def attn_block_chunk(self, desc: "AttnBlockDesc", h: DeviceBuffer, x: DeviceBuffer, n_tok: int,
                         pos0: int, pos: DeviceBuffer, page_ids: DeviceBuffer, slots: DeviceBuffer) -> None:
        """The attention half of one block over n_tok prompt tokens (moe.rs:1942-2071, chunked)."""
        h.require("residual", n_tok * desc.n_embd * 4)
        x.require("normed input", n_tok * desc.n_embd * 4)
        for buf, what in ((pos, "positions"), (page_ids, "page ids"), (slots, "slots")):
            buf.require(what, n_tok * 4)
        self.finish(self._lib.moearc_attn_block_chunk(self.raw, ctypes.byref(desc), h.ptr, x.ptr, n_tok, pos0,
                                                      pos.ptr, page_ids.ptr, slots.ptr), "attention block chunk")

    def attn_qkv(self, types, outs, ws, biases, rows, x: DeviceBuffer, n_cols: int) -> None:
        """The q, k, v projections plus their biases in as few launches as the types allow."""
        types = [QuantType(t) for t in types]
        for t, o, w, b, r in zip(types, outs, ws, biases, rows):
            if n_cols % t.block_elems:
                raise BadArgument(f"{t.name}: {n_cols} columns is not a whole number of blocks")
            if r:
                w.require("weights", r * t.row_bytes(n_cols))
                o.require("output", r * 4)
                if b is not None:
                    b.require("bias", r * 4)
        x.require("activation", n_cols * 4)
        tarr = (ctypes.c_uint * 3)(*[int(t) for t in types])
        rarr = (ctypes.c_ulong * 3)(*rows)
        self.finish(self._lib.moearc_attn_qkv(self.raw, tarr, _ptr_array(outs), _ptr_array(ws),
                                              _ptr_array(biases), rarr, x.ptr, n_cols), "attn qkv")


class AttnBlockDesc(ctypes.Structure):
    """``moearc_attn_block`` (include/moearc_attn.h): one block's attention weights, cache and RoPE."""
    _fields_ = [("w_type", ctypes.c_uint * 4), ("w", ctypes.c_void_p * 4), ("bias", ctypes.c_void_p * 4),
                ("sinks", ctypes.c_void_p), ("k_pages", ctypes.c_void_p), ("v_pages", ctypes.c_void_p),
                ("block_table", ctypes.c_void_p), ("n_embd", ctypes.c_ulong), ("n_head", ctypes.c_ulong),
                ("n_head_kv", ctypes.c_ulong), ("head_dim", ctypes.c_ulong), ("page_tokens", ctypes.c_ulong),
                ("n_swa", ctypes.c_ulong), ("ring_pages", ctypes.c_ulong), ("scale", ctypes.c_float), ("n_rot", ctypes.c_ulong),
                ("freq_base", ctypes.c_float), ("freq_scale", ctypes.c_float), ("ext_factor", ctypes.c_float),
                ("attn_factor", ctypes.c_float), ("corr_lo", ctypes.c_float), ("corr_hi", ctypes.c_float)]

    @staticmethod
    def make(types, ws, biases, sinks, k_pages, v_pages, block_table, n_embd, n_head, n_head_kv,
             head_dim, page_tokens, n_swa, scale, n_rot, freq_base, scaling: "RopeScaling | None" = None,
             ring_pages: int = 0):
        s = scaling or RopeScaling()
        d = AttnBlockDesc()
        for i in range(4):
            d.w_type[i] = int(types[i])
            d.w[i] = ws[i].ptr
            d.bias[i] = biases[i].ptr if biases[i] is not None else None
        d.sinks = sinks.ptr if sinks is not None else None
        d.k_pages, d.v_pages, d.block_table = k_pages.ptr, v_pages.ptr, block_table.ptr
        d.n_embd, d.n_head, d.n_head_kv, d.head_dim = n_embd, n_head, n_head_kv, head_dim
        d.page_tokens, d.n_swa, d.scale, d.n_rot, d.freq_base = page_tokens, n_swa, scale, n_rot, freq_base
        d.ring_pages = ring_pages
        d.freq_scale, d.ext_factor, d.attn_factor = s.freq_scale, s.ext_factor, s.attn_factor
        d.corr_lo, d.corr_hi = s.corr_lo, s.corr_hi
        # the descriptor holds raw device pointers: keep their buffers alive as long as it lives
        d._buffers = [b for b in (*ws, *biases, sinks, k_pages, v_pages, block_table) if b is not None]
        return d

class QuantType(enum.IntEnum):
    """GGUF weight formats the matvec kernels expand (lib.rs ``QuantType``, reference.rs:69-121)."""
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    MXFP4 = 39

    @property
    def block_bytes(self) -> int:
        return {0: 4, 1: 2, 8: 34, 12: 144, 13: 176, 14: 210, 39: 17}[int(self)]

    @property
    def block_elems(self) -> int:
        return {0: 1, 1: 1, 8: 32, 12: 256, 13: 256, 14: 256, 39: 32}[int(self)]

    def row_bytes(self, n_cols: int) -> int:
        return n_cols // self.block_elems * self.block_bytes


class DeviceView(DeviceBuffer):
    """A non-owning window into a DeviceBuffer (e.g. a tensor at an offset inside a weight blob)."""

    def __init__(self, base: DeviceBuffer, offset: int, nbytes: Optional[int] = None):
        self._base = base
        super().__init__(base.ctx, base.ptr + offset, base.len - offset if nbytes is None else nbytes)

    def free(self) -> None:
        self.ptr = 0


def _ptr_array(bufs) -> ctypes.Array:
    return (ctypes.c_void_p * len(bufs))(*[b.ptr if b is not None else None for b in bufs])
