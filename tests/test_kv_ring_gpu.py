"""Chunked prefill, then decode, of a windowed and a full-attention layer kept through this
build's KV bookkeeping (include/moearc_kv.h), on the GPU, against the oracle over a contiguous cache.

The windowed layer stores its keys in a ring of KvGeometry::swa_pages pages, indexed through the
cyclic table (moe.rs:1506-1513) -- the kernels see an ordinary block table; the full layer takes
its pages from the pool, a chunk at a time (moearc_kv_pool_append_chunk). Each chunk's K/V are
appended (moearc_kv_append_chunk) before the chunk attends, as the engine orders it. Bar: the
north star's max-abs 2e-3 on the output.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import KvType
from moearc_amd.kv import KvGeometry, PagedKvCache
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _report(label, got, want):
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
    print(f"{label}: max |gpu - oracle| = {err:.3e} (tolerance {TOL:.0e})", flush=True)
    assert err <= TOL, f"{label}: {err:.3e} > {TOL}"


@pytest.mark.parametrize("pt,chunk,n_swa", [(16, 24, 40), (32, 64, 128)])
def test_chunked_prefill_then_decode_through_ring_and_pool(ctx, pt, chunk, n_swa):
    T = 300
    c = fx.prefill_case(0x6A00 + pt + chunk, n_q=T + 1, pos0=0, pt=pt)  # token T is the decode step
    H, G, D, row = c.H, c.G, c.D, c.G * c.D
    phys = np.array([int(c.bt[x // pt]) * pt + x % pt for x in range(T + 1)])
    k_f32 = c.k_raw.reshape(-1, row)[phys].view(np.float16).astype(np.float32)  # logical order
    v_f32 = c.v_raw.reshape(-1, row)[phys].view(np.float16).astype(np.float32)
    geo = KvGeometry.plan(T + 1, pt, n_swa, chunk=chunk)
    assert geo.swa_pages < geo.pages  # the ring really wraps
    ring = geo.ring_table()
    pool = PagedKvCache(geo.pages + 5, pt, T + 1)
    pool.begin(1, 0)
    page_bytes = pt * row * 2
    rk, rv = ctx.alloc(geo.swa_pages * page_bytes), ctx.alloc(geo.swa_pages * page_bytes)
    fk, fv = ctx.alloc((geo.pages + 5) * page_bytes), ctx.alloc((geo.pages + 5) * page_bytes)
    for b in (rk, rv, fk, fv):
        ctx.zero(b, b.len // 4)
    dring = ctx.upload(ring)
    ds = ctx.upload(c.sinks)
    want_swa = oracle.attn_prefill(c.qp[:T].astype(np.float32), c.k_raw, c.v_raw, c.bt, T, 0, n_swa,
                                   H, G, D, pt, float(c.scale), sinks=c.sinks, n_threads=16)
    want_full = oracle.attn_prefill(c.qp[:T].astype(np.float32), c.k_raw, c.v_raw, c.bt, T, 0, 0, H, G,
                                    D, pt, float(c.scale), sinks=c.sinks, n_threads=16)
    got_swa = np.zeros((T, H, D), np.float32)
    got_full = np.zeros_like(got_swa)
    for p0 in range(0, T, chunk):
        n = min(chunk, T - p0)
        pos = np.arange(p0, p0 + n)
        dk, dvv = ctx.upload(k_f32[p0:p0 + n]), ctx.upload(v_f32[p0:p0 + n])
        dq = ctx.upload(np.ascontiguousarray(c.qp[p0:p0 + n]).view(np.uint16))
        out = ctx.alloc(n * H * D * 4)
        # windowed layer: ring slots through the cyclic table
        ctx.kv_append_chunk(rk, rv, dk, dvv, ctx.upload(ring[pos // pt]), ctx.upload((pos % pt).astype(np.uint32)),
                            n, G, D, pt, KvType.F16)
        ctx.attn_prefill(out, dq, rk, rv, dring, ds, n, p0, n_swa, H, G, D, pt, float(c.scale), KvType.F16)
        got_swa[p0:p0 + n] = ctx.download(out, np.float32, (n, H, D))
        # full layer: pages from the pool
        pages, slots = pool.append_chunk(1, n)
        ctx.kv_append_chunk(fk, fv, dk, dvv, ctx.upload(pages), ctx.upload(slots), n, G, D, pt, KvType.F16)
        table = np.array(pool.pages_of(1).pages, np.uint32)
        ctx.attn_prefill(out, dq, fk, fv, ctx.upload(table), ds, n, p0, 0, H, G, D, pt, float(c.scale),
                         KvType.F16)
        got_full[p0:p0 + n] = ctx.download(out, np.float32, (n, H, D))
    _report(f"ring prefill pt={pt} chunk={chunk} n_swa={n_swa}", got_swa, want_swa)
    _report(f"pool prefill pt={pt} chunk={chunk}", got_full, want_full)

    # one decode step at position T: append, then attend (the window through the ring)
    q = fx.synth.normal(0x6AFF, H * D).astype(np.float32)
    dq = ctx.upload(q)
    dk, dvv = ctx.upload(k_f32[T:T + 1]), ctx.upload(v_f32[T:T + 1])
    out = ctx.alloc(H * D * 4)
    ctx.kv_append_chunk(rk, rv, dk, dvv, ctx.upload(ring[T // pt:T // pt + 1]),
                        ctx.upload(np.array([T % pt], np.uint32)), 1, G, D, pt, KvType.F16)
    kb = max(0, T + 1 - n_swa)
    ctx.attn_decode_ext(out, dq, rk, rv, dring, ds, H, G, D, kb, T + 1, pt, float(c.scale), KvType.F16)
    want = oracle.attn_decode(q, c.k_raw, c.v_raw, c.bt, H, G, D, kb, T + 1, pt, float(c.scale),
                              kv_type=1, sinks=c.sinks)
    _report("ring decode", ctx.download(out, np.float32, H * D), want)
    page, slot = pool.append(1)
    ctx.kv_append_chunk(fk, fv, dk, dvv, ctx.upload(np.array([page], np.uint32)),
                        ctx.upload(np.array([slot], np.uint32)), 1, G, D, pt, KvType.F16)
    table = np.array(pool.pages_of(1).pages, np.uint32)
    ctx.attn_decode_ext(out, dq, fk, fv, ctx.upload(table), ds, H, G, D, 0, T + 1, pt, float(c.scale),
                        KvType.F16)
    want = oracle.attn_decode(q, c.k_raw, c.v_raw, c.bt, H, G, D, 0, T + 1, pt, float(c.scale),
                              kv_type=1, sinks=c.sinks)
    _report("pool decode", ctx.download(out, np.float32, H * D), want)
    pool.end(1)
