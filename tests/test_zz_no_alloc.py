"""The allocation-free decode entry point (moearc_attn_decode_batched_noalloc) on the GPU, through the
C ABI, against the allocating one (moearc_attn_decode_batched) on the same inputs: the same kernels,
so the outputs must be bit-identical. Two calls in a row on one context, the second smaller (the
fixed record array keeps the first call's contents), then a call too large for the array, which
must be refused with -2 before anything is enqueued."""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import Context, KvType, OUT_F16, OUT_F32

pytestmark = pytest.mark.gpu


def _call(cx, fn, out, dq, dk, dv, dbt, stride, kb, nk, ds, H, G, D, pt, out_type):
    kb = np.ascontiguousarray(kb, np.uint32)
    nk = np.ascontiguousarray(nk, np.uint32)
    return fn(cx.raw, out.ptr, out_type, dq.ptr, dk.ptr, dv.ptr, dbt.ptr, stride, kb.ctypes.data,
              nk.ctypes.data, ds.ptr if ds is not None else None, kb.size, H, G, D, pt, 0.125,
              int(KvType.F16))


def _ragged(seed, lens, pt, windows):
    """A ragged batch over one shared page pool: per sequence (case, block-table row)."""
    H, G, D = 64, 8, 64
    c = fx.north_star_case(seed, int(sum(lens)), pt=pt, extra_pages=len(lens))
    pages = [-(-n // pt) for n in lens]
    stride = max(pages)
    table = np.zeros((len(lens), stride), np.uint32)
    off = 0
    for s, p in enumerate(pages):
        table[s, :p] = c.bt_full[off:off + p]
        off += p
    kb = [max(0, n - w) if w else 0 for n, w in zip(lens, windows)]
    q = fx.synth.normal(seed + 7, len(lens) * H * D)
    return c, table, stride, np.array(kb, np.uint32), np.array(lens, np.uint32), q


@pytest.mark.parametrize("out_type", [OUT_F32, OUT_F16])
def test_noalloc_equals_allocating_entry_point(out_type):
    H, G, D = 64, 8, 64
    with Context() as cx:
        lib = cx._lib
        for label, (seed, lens, pt, windows) in (
                ("first call: 3 ragged sequences, 256-token pages", (0xA110, [20000, 7001, 32768], 256, [0, 128, 0])),
                ("second call, smaller: 1 sequence, 32-token pages", (0xA111, [3000], 32, [0]))):
            c, table, stride, kb, nk, q = _ragged(seed, lens, pt, windows)
            dk, dv, dbt = cx.upload(c.k_raw), cx.upload(c.v_raw), cx.upload(table)
            dq, ds = cx.upload(q), cx.upload(c.sinks)
            nb = 2 if out_type == OUT_F16 else 4
            want_buf, got_buf = cx.alloc(len(lens) * H * D * nb), cx.alloc(len(lens) * H * D * nb)
            rc = _call(cx, lib.moearc_attn_decode_batched, want_buf, dq, dk, dv, dbt, stride, kb, nk, ds,
                       H, G, D, pt, out_type)
            assert rc == 0
            rc = _call(cx, lib.moearc_attn_decode_batched_noalloc, got_buf, dq, dk, dv, dbt, stride, kb,
                       nk, ds, H, G, D, pt, out_type)
            assert rc == 0
            cx.sync()
            dt = np.float16 if out_type == OUT_F16 else np.float32
            want = cx.download(want_buf, dt, len(lens) * H * D)
            got = cx.download(got_buf, dt, len(lens) * H * D)
            print(f"{label}: bit-identical = {np.array_equal(got.view(np.uint16 if nb == 2 else np.uint32), want.view(np.uint16 if nb == 2 else np.uint32))}",
                  flush=True)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), label


def test_noalloc_refuses_a_call_too_large_for_the_array(monkeypatch):
    # forced 128-key splits of the one-KV-head kernel over 70000 keys: 547 work items x 64 heads x 66
    # floats > the array's 2^21 floats
    monkeypatch.setenv("MOEARC_DECODE_VARIANT", "1x4x1")
    monkeypatch.setenv("MOEARC_DECODE_SPLIT", "128")
    H, G, D, pt = 64, 8, 64, 256
    c = fx.north_star_case(0xA112, 70000, pt=pt)
    with Context() as cx:
        lib = cx._lib
        dk, dv, dbt, dq, ds = (cx.upload(c.k_raw), cx.upload(c.v_raw), cx.upload(c.bt), cx.upload(c.q),
                               cx.upload(c.sinks))
        sentinel = np.full(H * D, 7.25, np.float32)
        out = cx.upload(sentinel)
        rc = _call(cx, lib.moearc_attn_decode_batched_noalloc, out, dq, dk, dv, dbt, c.bt.size, [0], [70000],
                   ds, H, G, D, pt, OUT_F32)
        assert rc == -2
        cx.sync()
        assert np.array_equal(cx.download(out, np.float32, H * D), sentinel)  # nothing was enqueued
        # the allocating entry point takes the same call
        rc = _call(cx, lib.moearc_attn_decode_batched, out, dq, dk, dv, dbt, c.bt.size, [0], [70000], ds,
                   H, G, D, pt, OUT_F32)
        assert rc == 0
        cx.sync()
