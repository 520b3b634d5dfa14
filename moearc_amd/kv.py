"""KV page pool and cache geometry (``include/moearc_kv.h``), with the reference engine's API.

``PagedKvCache`` mirrors crates/moearc-engine/src/kv.rs:85-205 (begin / append / end / pages_of /
can_admit / usage, the same refusals as ``KvError``), plus ``append_chunk`` -- a prefill chunk's
places in one all-or-nothing call, in the form ``Context.kv_append_chunk`` and
``Context.rope_kv_append_chunk`` take -- and ``block_tables`` for ``attn_decode_batched``.
``KvGeometry`` mirrors moe.rs:716-771: pages of a full-attention layer, pages of a windowed
layer's ring, and the cyclic table that turns the ring into an ordinary block table
(moe.rs:1506-1513). Everything here is host bookkeeping; no device memory is touched.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import native

EXHAUSTED, UNKNOWN_SEQUENCE, CONTEXT_LIMIT, INVALID_GEOMETRY = -3, -4, -5, -6


class KvError(Exception):
    """A refused KV operation (kv.rs:23-34); the pool is left as it was."""


class Exhausted(KvError):
    def __init__(self, requested: int, free: int):
        super().__init__(f"KV cache exhausted: {requested} page(s) needed, {free} free")
        self.requested, self.free = requested, free


class UnknownSequence(KvError):
    def __init__(self, seq: int):
        super().__init__(f"sequence {seq} is not active")
        self.seq = seq


class ContextLimit(KvError):
    def __init__(self, seq: int, tokens: int, limit: int):
        super().__init__(f"sequence {seq} reached {tokens} tokens, past the {limit}-token limit")
        self.seq, self.tokens, self.limit = seq, tokens, limit


class InvalidGeometry(KvError):
    pass


@dataclass(frozen=True)
class KvUsage:
    """How full the pool is (kv.rs:64-82)."""
    total_pages: int
    used_pages: int
    sequences: int
    slack_tokens: int

    def free_pages(self) -> int:
        return self.total_pages - self.used_pages

    def utilisation(self) -> float:
        return 0.0 if self.total_pages == 0 else self.used_pages / self.total_pages


@dataclass(frozen=True)
class SeqPages:
    """One sequence's page table (kv.rs:55-62): token t lives in pages[t // page_tokens]."""
    pages: tuple
    tokens: int


class _Usage(ctypes.Structure):
    _fields_ = [("total_pages", ctypes.c_uint32), ("used_pages", ctypes.c_uint32),
                ("sequences", ctypes.c_uint32), ("slack_tokens", ctypes.c_uint32)]


def _u32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class PagedKvCache:
    """A pool of ``total_pages`` pages of ``page_tokens`` tokens shared by concurrent sequences."""

    def __init__(self, total_pages: int, page_tokens: int, context_limit: int):
        self._lib = native.load()
        h = ctypes.c_void_p()
        rc = self._lib.moearc_kv_pool_create(total_pages, page_tokens, context_limit, ctypes.byref(h))
        if rc == INVALID_GEOMETRY:
            raise InvalidGeometry("a pool needs at least one page" if total_pages == 0
                                  else "a page must hold at least one token")
        if rc:
            raise RuntimeError(f"moearc_kv_pool_create failed ({rc})")
        self._h = h
        self._page_tokens = page_tokens

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.moearc_kv_pool_destroy(self._h)
            self._h = None

    __del__ = close

    def page_tokens(self) -> int:
        return self._page_tokens

    def _raise(self, rc: int, seq: int):
        a, b = ctypes.c_uint32(), ctypes.c_uint32()
        self._lib.moearc_kv_pool_last_error(self._h, ctypes.byref(a), ctypes.byref(b))
        if rc == EXHAUSTED:
            raise Exhausted(a.value, b.value)
        if rc == UNKNOWN_SEQUENCE:
            raise UnknownSequence(seq)
        if rc == CONTEXT_LIMIT:
            raise ContextLimit(seq, a.value, b.value)
        raise ValueError(f"KV pool call refused ({rc}) for sequence {seq}")

    def begin(self, seq: int, prompt_tokens: int) -> SeqPages:
        """A sequence with room for ``prompt_tokens`` (kv.rs:120-138)."""
        rc = self._lib.moearc_kv_pool_begin(self._h, seq, prompt_tokens)
        if rc:
            self._raise(rc, seq)
        return self.pages_of(seq)

    def append(self, seq: int) -> tuple:
        """One more token; returns its (page, slot) (kv.rs:140-169)."""
        page, slot = ctypes.c_uint32(), ctypes.c_uint32()
        rc = self._lib.moearc_kv_pool_append(self._h, seq, ctypes.byref(page), ctypes.byref(slot))
        if rc:
            self._raise(rc, seq)
        return page.value, slot.value

    def append_chunk(self, seq: int, n: int) -> tuple:
        """``n`` more tokens, all or nothing; returns (page_ids, slots) as uint32 arrays."""
        pages, slots = np.zeros(n, np.uint32), np.zeros(n, np.uint32)
        rc = self._lib.moearc_kv_pool_append_chunk(self._h, seq, n, _u32p(pages), _u32p(slots))
        if rc:
            self._raise(rc, seq)
        return pages, slots

    def end(self, seq: int) -> int:
        """Release a sequence's pages; returns how many (kv.rs:171-180)."""
        n = ctypes.c_uint32()
        rc = self._lib.moearc_kv_pool_end(self._h, seq, ctypes.byref(n))
        if rc:
            self._raise(rc, seq)
        return n.value

    def pages_of(self, seq: int) -> SeqPages:
        n, tok = ctypes.c_uint32(), ctypes.c_uint32()
        rc = self._lib.moearc_kv_pool_pages(self._h, seq, None, 0, ctypes.byref(n), ctypes.byref(tok))
        if rc:
            raise UnknownSequence(seq)
        pages = np.zeros(max(n.value, 1), np.uint32)
        self._lib.moearc_kv_pool_pages(self._h, seq, _u32p(pages), n.value, None, None)
        return SeqPages(tuple(int(p) for p in pages[:n.value]), tok.value)

    def can_admit(self, tokens: int) -> bool:
        return bool(self._lib.moearc_kv_pool_can_admit(self._h, tokens))

    def usage(self) -> KvUsage:
        u = _Usage()
        self._lib.moearc_kv_pool_usage(self._h, ctypes.byref(u))
        return KvUsage(u.total_pages, u.used_pages, u.sequences, u.slack_tokens)

    def block_tables(self, seqs, stride: int | None = None) -> tuple:
        """Rows of the sequences' page tables (zero-padded to ``stride``, by default the longest):
        the ``block_tables`` / ``bt_stride`` pair of ``Context.attn_decode_batched``."""
        seqs = np.ascontiguousarray(seqs, np.uint64)
        if stride is None:
            stride = max([len(self.pages_of(int(s)).pages) for s in seqs] + [1])
        table = np.zeros((len(seqs), stride), np.uint32)
        rc = self._lib.moearc_kv_pool_block_tables(self._h, seqs.ctypes.data_as(ctypes.c_void_p),
                                                   len(seqs), stride, _u32p(table))
        if rc == UNKNOWN_SEQUENCE:
            raise KvError("a sequence in the batch is not active")
        if rc:
            raise ValueError(f"a sequence holds more than {stride} pages")
        return table, stride


@dataclass(frozen=True)
class KvGeometry:
    """Pages per layer for a context of ``n_ctx`` tokens (KvGeometry::plan, moe.rs:735-757).

    A windowed layer keeps a ring of ``swa_pages`` pages: a chunk of ``chunk`` tokens is appended
    before it is attended, so the ring holds ``n_swa + chunk - 1`` tokens (``chunk = 1``: token by
    token decode), rounded up to pages and capped at ``pages``."""
    pages: int
    swa_pages: int
    page_tokens: int

    @staticmethod
    def plan(n_ctx: int, page_tokens: int, n_swa: int | None = None, chunk: int = 1) -> "KvGeometry":
        lib = native.load()
        p, s = ctypes.c_uint32(), ctypes.c_uint32()
        rc = lib.moearc_kv_geometry(n_ctx, page_tokens, n_swa or 0, chunk, ctypes.byref(p), ctypes.byref(s))
        if rc:
            raise InvalidGeometry("a page must hold at least one token")
        return KvGeometry(p.value, s.value, page_tokens)

    def ring_tokens(self) -> int:
        return self.swa_pages * self.page_tokens

    def ring_table(self) -> np.ndarray:
        """The cyclic block table of a windowed layer: entry i = i % swa_pages (moe.rs:1506-1513)."""
        t = np.zeros(self.pages, np.uint32)
        native.load().moearc_kv_ring_table(self.pages, self.swa_pages, _u32p(t))
        return t
