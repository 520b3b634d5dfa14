"""Decode parity on the GPU: the HIP path through the C ABI against the oracle and golden vectors.

The first group reproduces the reference's own attention tests (forward_pass_gpu.rs), with their
fixtures regenerated bit-exactly and their tolerances; they run the general f32 kernel (f32 KV or
head_dim 128). The second group runs the gpt-oss shape (64 q heads, 8 KV heads, head_dim 64, f16
KV, sinks) on the split-K MFMA kernel at the north star's bar: max-abs error <= 2e-3 against the
oracle (the measured error is printed; it is far below the bar).
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import BadArgument, Context, KvType, OUT_F16, OUT_F32
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL_NS = 2e-3  # the north star's max-abs error bar on the output


def _report(label, got, want, tol):
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
    print(f"{label}: max |gpu - oracle| = {err:.3e} (tolerance {tol:.3e})", flush=True)
    assert err <= tol, f"{label}: {err:.3e} > {tol:.3e}"
    return err


def _upload_case(ctx, c, bt=None):
    b = {}
    b["k"] = ctx.upload(c.k_raw)
    b["v"] = ctx.upload(c.v_raw)
    b["q"] = ctx.upload(c.q.astype(np.float32))
    b["bt"] = ctx.upload(np.asarray(c.bt if bt is None else bt, np.uint32))
    b["sinks"] = ctx.upload(c.sinks.astype(np.float32)) if c.sinks is not None else None
    b["out"] = ctx.alloc(c.H * c.D * 4)
    return b


def _decode(ctx, c, b, kv_begin, sinks=True):
    ctx.attn_decode_ext(b["out"], b["q"], b["k"], b["v"], b["bt"], b["sinks"] if sinks else None,
                        c.H, c.G, c.D, kv_begin, c.n_kv, c.pt, float(c.scale), KvType(c.kv))
    return ctx.download(b["out"], np.float32, c.H * c.D)


# ---- the reference's attention tests -------------------------------------------------------------

@pytest.mark.parametrize("name", ["scattered_f32", "scattered_f16"])
def test_paged_attention_matches_across_scattered_pages(ctx, name):
    # forward_pass_gpu.rs:500-591; K/V written through the GPU append kernel, one token at a time
    c = fx.reference_case(name)
    g = fx.load_golden("ref_" + name)
    assert str(g["digest"]) == c.digest()
    row = c.G * c.D
    kv = KvType(c.kv)
    dk = ctx.alloc(c.k_raw.nbytes)
    dv = ctx.alloc(c.v_raw.nbytes)
    ctx.zero(dk, c.k_raw.nbytes // 4)
    ctx.zero(dv, c.v_raw.nbytes // 4)
    dk_tok, dv_tok = ctx.alloc(row * 4), ctx.alloc(row * 4)
    for j in range(c.n_kv):
        ctx.upload_slice(dk_tok, c.token_rows[j, 0])
        ctx.upload_slice(dv_tok, c.token_rows[j, 1])
        ctx.kv_append(dk, dv, dk_tok, dv_tok, int(c.bt[j // c.pt]), j % c.pt, c.G, c.D, c.pt, kv)
    # the appended pool equals the reference mirror byte for byte
    assert np.array_equal(ctx.download(dk, c.k_raw.dtype, c.k_raw.shape), c.k_raw)
    assert np.array_equal(ctx.download(dv, c.v_raw.dtype, c.v_raw.shape), c.v_raw)
    dq, dbt, dout = ctx.upload(c.q), ctx.upload(c.bt), ctx.alloc(c.H * c.D * 4)
    ctx.attn_decode(dout, dq, dk, dv, dbt, c.H, c.G, c.D, c.n_kv, c.pt, float(c.scale), kv)
    got = ctx.download(dout, np.float32, c.H * c.D)
    _report(f"attn_decode {name}", got, g["expected"], fx.ref_tolerance(c.D, c.n_kv))
    assert np.abs(got).max() <= np.abs(c.v_val).max() + 1e-4


def test_grouped_query_heads(ctx):
    # forward_pass_gpu.rs:594-673
    c = fx.reference_case("gqa")
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, 0)
    _report("attn_decode GQA 8/2", got, fx.load_golden("ref_gqa")["expected"],
            fx.ref_tolerance(c.D, c.n_kv))
    assert not np.array_equal(got[:c.D], got[c.D:2 * c.D])


def test_single_cached_key_returns_v_exactly(ctx):
    # forward_pass_gpu.rs:676-744
    c = fx.reference_case("single_key")
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, 0).reshape(c.H, c.D)
    v = c.v_val.reshape(-1, c.G, c.D)[int(c.bt[0]) * c.pt]
    assert np.all(np.abs(got - v) <= 1e-6 * np.maximum(np.abs(v), 1.0))


def test_windowed_span(ctx):
    # forward_pass_gpu.rs:747-871: agreement, the window moves the answer, one-key window = V
    c = fx.reference_case("window")
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, 15)
    _report("attn_decode window", got, fx.load_golden("ref_window")["expected"],
            fx.ref_tolerance(c.D, 6))
    full = _decode(ctx, c, b, 0)
    assert float(np.max(np.abs(got - full))) > 1e-3
    one = _decode(ctx, c, b, c.n_kv - 1).reshape(c.H, c.D)
    j = c.n_kv - 1
    v = c.v_val.reshape(-1, c.G, c.D)[int(c.bt[j // c.pt]) * c.pt + j % c.pt]
    want = np.repeat(v, c.H // c.G, axis=0)
    assert np.all(np.abs(one - want) <= 1e-6 * np.maximum(np.abs(want), 1.0))


def test_refusals(ctx):
    # forward_pass_gpu.rs:874-899
    buf = ctx.alloc(1 << 16)
    bt = ctx.alloc(16)
    with pytest.raises(BadArgument):
        ctx.attn_decode_ext(buf, buf, buf, buf, bt, None, 4, 4, 8, 4, 4, 4, 1.0, KvType.F32)
    with pytest.raises(BadArgument):
        ctx.attn_decode(buf, buf, buf, buf, bt, 6, 4, 8, 4, 4, 1.0, KvType.F32)
    # the raw ABI refuses in the reference's order (kernels.cpp:1842-1852)
    lib, raw = ctx._lib, ctx.raw
    args = lambda **kw: dict(dict(H=4, G=4, D=8, kb=0, n=4, pt=4, kv=0), **kw)
    call = lambda a: lib.moearc_attn_decode(raw, buf.ptr, buf.ptr, buf.ptr, buf.ptr, bt.ptr, None,
                                            a["H"], a["G"], a["D"], a["kb"], a["n"], a["pt"], 1.0,
                                            a["kv"])
    assert call(args(kv=2)) == -2
    assert call(args(n=0)) == -2
    assert call(args(pt=0)) == -2
    assert call(args(H=6)) == -2
    assert call(args(kb=4)) == -2
    assert call(args(D=2048)) == -2
    assert lib.moearc_attn_decode(raw, None, buf.ptr, buf.ptr, buf.ptr, bt.ptr, None, 4, 4, 8, 0,
                                  4, 4, 1.0, 0) == -1
    ctx.sync()


def test_kv_append_writes_exactly_the_slot(ctx):
    # forward_pass_gpu.rs:431-497
    heads, hd, pt, pages = 3, 16, 4, 5
    row = heads * hd
    pool = pages * pt * row
    r = oracle.Rng(0xC0DE)
    k, v = r.vec_unit(row), r.vec_unit(row)
    poison = np.full(pool, -7.5, np.float32)
    dk, dv = ctx.upload(poison), ctx.upload(poison)
    ctx.kv_append(dk, dv, ctx.upload(k), ctx.upload(v), 3, 2, heads, hd, pt, KvType.F32)
    got = ctx.download(dk, np.float32, pool)
    want_k, want_v = poison.copy(), poison.copy()
    oracle.kv_append(want_k, want_v, k, v, 3, 2, heads, hd, pt, oracle.KV_F32)
    assert np.array_equal(got, want_k)
    assert np.array_equal(ctx.download(dv, np.float32, pool), want_v)
    with pytest.raises(BadArgument):
        ctx.kv_append(dk, dv, ctx.upload(k), ctx.upload(v), 0, 4, heads, hd, pt, KvType.F32)


def test_kv_append_chunk_equals_token_appends(ctx):
    G, D, pt, pages, n_tok = 8, 64, 32, 6, 70
    row = G * D
    rows_k = fx.synth.normal(1, n_tok * row).reshape(n_tok, row)
    rows_v = fx.synth.normal(2, n_tok * row).reshape(n_tok, row)
    bt = fx.synth.random_block_table(3, pages)
    page_ids = np.array([bt[t // pt] for t in range(n_tok)], np.uint32)
    slots = np.array([t % pt for t in range(n_tok)], np.uint32)
    pool = pages * pt * row
    a_k, a_v = ctx.upload(np.zeros(pool, np.uint16)), ctx.upload(np.zeros(pool, np.uint16))
    b_k, b_v = ctx.upload(np.zeros(pool, np.uint16)), ctx.upload(np.zeros(pool, np.uint16))
    dk, dv = ctx.upload(rows_k), ctx.upload(rows_v)
    ctx.kv_append_chunk(a_k, a_v, dk, dv, ctx.upload(page_ids), ctx.upload(slots), n_tok, G, D, pt,
                        KvType.F16)
    tk, tv = ctx.alloc(row * 4), ctx.alloc(row * 4)
    want_k = np.zeros(pool, np.uint16)
    want_v = np.zeros(pool, np.uint16)
    for t in range(n_tok):
        ctx.upload_slice(tk, rows_k[t])
        ctx.upload_slice(tv, rows_v[t])
        ctx.kv_append(b_k, b_v, tk, tv, int(page_ids[t]), int(slots[t]), G, D, pt, KvType.F16)
        oracle.kv_append_raw(want_k, want_v, rows_k[t], rows_v[t], int(page_ids[t]), int(slots[t]),
                             G, D, pt, oracle.KV_F16)
    got_a = ctx.download(a_k, np.uint16, pool)
    assert np.array_equal(got_a, ctx.download(b_k, np.uint16, pool))
    assert np.array_equal(got_a, want_k)
    assert np.array_equal(ctx.download(a_v, np.uint16, pool), want_v)


@pytest.mark.parametrize("fused", [False, True])
def test_out_of_page_slot_is_refused_at_sync(fused):
    # The slots live on the device, so the host cannot refuse a slot outside its page when the
    # call is made; the kernel leaves that token unwritten and the next synchronisation fails. The
    # other tokens land, and the next call starts clean.
    from moearc_amd import Failed
    from moearc_amd import RopeKind
    G, D, pt, pages, n_tok = 2, 64, 16, 3, 5
    row = G * D
    rows = fx.synth.normal(9, n_tok * row).reshape(n_tok, row)
    page_ids = np.array([0, 1, 2, 1, 0], np.uint32)
    slots = np.array([3, pt, 7, 15, 0], np.uint32)  # token 1's slot lies outside the page
    with Context() as cx:
        pool = pages * pt * row
        kp, vp = cx.upload(np.zeros(pool, np.uint16)), cx.upload(np.zeros(pool, np.uint16))
        dk, dv = cx.upload(rows), cx.upload(rows)
        dpg, dsl = cx.upload(page_ids), cx.upload(slots)
        if fused:
            cx.rope_kv_append_chunk(kp, vp, dk, dv, cx.upload(np.arange(n_tok, dtype=np.int32)), dpg, dsl,
                                    n_tok, G, D, pt, D, 10000.0, kind=RopeKind.NEOX, kv=KvType.F16)
        else:
            cx.kv_append_chunk(kp, vp, dk, dv, dpg, dsl, n_tok, G, D, pt, KvType.F16)
        with pytest.raises(Failed):
            cx.sync()
        got = cx.download(vp, np.uint16, pool).reshape(pages, pt, row)
        for t in (0, 2, 3, 4):
            assert np.array_equal(got[page_ids[t], slots[t]], fx.synth.f16_bits(rows[t]))
        assert np.count_nonzero(got) == 4 * row  # nothing else written
        # a clean call afterwards synchronises without error
        good = np.array([0, 1, 2, 1, 0], np.uint32) * 0 + np.arange(n_tok, dtype=np.uint32)
        cx.kv_append_chunk(kp, vp, dk, dv, dpg, cx.upload(good), n_tok, G, D, pt, KvType.F16)
        cx.sync()


# ---- gpt-oss shape on the split-K MFMA kernel ----------------------------------------------------

@pytest.mark.parametrize("golden,kv_begin", [("ns_decode_full", 0), ("ns_decode_swa128", 172)])
def test_north_star_shape_against_golden(ctx, golden, kv_begin):
    c = fx.north_star_case(0x5EED, 300, pt=32)
    g = fx.load_golden(golden)
    assert str(g["digest"]) == c.digest()
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, kv_begin)
    _report(f"split-K decode {golden}", got, g["expected"], TOL_NS)


@pytest.mark.parametrize("n_kv,pt,kv_begin,group", [
    (4096, 256, 0, 8),      # config 1 depth
    (4096, 256, 3968, 8),   # SWA-128 at 4K
    (1000, 16, 0, 8),       # pages smaller than a tile
    (777, 64, 5, 16),       # group 16, odd span start
    (1, 32, 0, 8),          # one key
    (33, 32, 1, 4),         # tile edge
])
def test_split_k_decode_against_oracle(ctx, n_kv, pt, kv_begin, group):
    H = 8 * group
    c = fx.north_star_case(1000 + n_kv + pt, n_kv, pt=pt, H=H, G=8, D=64)
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, kv_begin)
    want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, kv_begin, n_kv, pt,
                              float(c.scale), kv_type=1, sinks=c.sinks)
    _report(f"split-K decode n_kv={n_kv} pt={pt} begin={kv_begin} group={group}", got, want, TOL_NS)
    nosink = _decode(ctx, c, b, kv_begin, sinks=False)
    want_ns = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, kv_begin, n_kv, pt,
                                 float(c.scale), kv_type=1)
    _report("  without sinks", nosink, want_ns, TOL_NS)


def test_config2_depth_32k_against_oracle(ctx):
    # B=1, 32K keys, full causal, f16 KV, per-head sinks
    c = fx.north_star_case(0xC2, 32768, pt=256)
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, 0)
    want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                              float(c.scale), kv_type=1, sinks=c.sinks)
    _report("split-K decode 32K", got, want, TOL_NS)


@pytest.mark.parametrize("n_kv,kv_begin", [(20000, 0), (20000, 19872)], ids=["full", "swa128"])
def test_f32_kv_long_context_against_oracle(ctx, n_kv, kv_begin):
    # an f32 KV cache (the reference's other KvType, reference.rs:728-752) at a long context, both
    # a full span and a 128-key window, through a random page permutation: the general kernel
    c = fx.north_star_case(0xF32, n_kv, pt=256)
    row = c.G * c.D
    kvals = np.zeros((c.k_raw.shape[0], row), np.float32)
    vvals = np.zeros_like(kvals)
    live = c.bt[np.arange(n_kv) // c.pt].astype(np.int64) * c.pt + np.arange(n_kv) % c.pt
    kvals[live] = fx.synth.normal(0xF33, n_kv * row).reshape(n_kv, row)
    vvals[live] = fx.synth.normal(0xF34, n_kv * row).reshape(n_kv, row)
    dk, dv, dq = ctx.upload(kvals), ctx.upload(vvals), ctx.upload(c.q.astype(np.float32))
    dbt, ds, out = ctx.upload(np.asarray(c.bt, np.uint32)), ctx.upload(c.sinks), ctx.alloc(c.H * c.D * 4)
    ctx.attn_decode_ext(out, dq, dk, dv, dbt, ds, c.H, c.G, c.D, kv_begin, n_kv, c.pt, float(c.scale),
                        KvType.F32)
    got = ctx.download(out, np.float32, c.H * c.D)
    want = oracle.attn_decode(c.q, kvals, vvals, c.bt, c.H, c.G, c.D, kv_begin, n_kv, c.pt,
                              float(c.scale), kv_type=0, sinks=c.sinks)
    _report(f"f32 KV decode n_kv={n_kv} begin={kv_begin}", got, want, TOL_NS)


def test_single_key_closed_form_with_sink(ctx):
    # one key: out = V * sigmoid(s - sink)
    c = fx.north_star_case(77, 1, pt=32)
    b = _upload_case(ctx, c)
    got = _decode(ctx, c, b, 0).reshape(c.H, c.D)
    K, V = fx.contiguous_kv(c, "k")[0], fx.contiguous_kv(c, "v")[0]
    for h in range(c.H):
        g = h // 8
        s = float(np.dot(c.q[h * 64:(h + 1) * 64].astype(np.float64), K[g])) * float(c.scale)
        want = V[g] / (1.0 + math.exp(float(c.sinks[h]) - s))
        assert np.max(np.abs(got[h] - want)) < 1e-5


def test_forced_splits_and_variants(monkeypatch):
    # both work-group shapes, with many splits (merged by the second launch), several chunks per
    # wave (the chunk loop), and one split (finished in place)
    c = fx.north_star_case(0xAB, 5000, pt=256, spike_frac=0.01)
    want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                              float(c.scale), kv_type=1, sinks=c.sinks)
    for variant, split in (("4x2x4", 256), ("4x2x4", 1024), ("4x2x4", 4096), ("4x2x4", 8192),
                           ("1x4x1", 128), ("1x4x1", 640), ("1x4x1", 8192)):
        monkeypatch.setenv("MOEARC_DECODE_VARIANT", variant)
        monkeypatch.setenv("MOEARC_DECODE_SPLIT", str(split))
        with Context() as cx:
            b = _upload_case(cx, c)
            for rep in range(2):
                got = _decode(cx, c, b, 0)
                _report(f"variant={variant} split={split} rep={rep}", got, want, TOL_NS)


def test_merge_over_many_rounds(monkeypatch):
    # 157 splits: each merge lane takes more than one round of records (128 per round)
    c = fx.north_star_case(0xAC, 20000, pt=64, spike_frac=0.01)
    want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                              float(c.scale), kv_type=1, sinks=c.sinks)
    monkeypatch.setenv("MOEARC_DECODE_VARIANT", "1x4x1")
    monkeypatch.setenv("MOEARC_DECODE_SPLIT", "128")
    with Context() as cx:
        b = _upload_case(cx, c)
        got = _decode(cx, c, b, 0)
        _report("variant=1x4x1 split=128 n_kv=20000", got, want, TOL_NS)


@pytest.mark.parametrize("scale", [-0.125, 0.0])
def test_non_positive_scale(ctx, scale):
    # the split-K kernel needs a positive scale; these run on the general kernel with the same result
    c = fx.north_star_case(0xAD, 3000, pt=64)
    want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                              scale, kv_type=1, sinks=c.sinks)
    b = _upload_case(ctx, c)
    ctx.attn_decode_ext(b["out"], b["q"], b["k"], b["v"], b["bt"], b["sinks"], c.H, c.G, c.D, 0,
                        c.n_kv, c.pt, scale, KvType.F16)
    got = ctx.download(b["out"], np.float32, c.H * c.D)
    _report(f"scale={scale}", got, want, TOL_NS)


def test_batched_ragged_decode(ctx):
    _batched_ragged(ctx)


@pytest.mark.parametrize("variant", ["4x2x4", "1x4x1"])
def test_batched_ragged_decode_each_variant(monkeypatch, variant):
    # the same batch with each work-group shape forced, twice per context (records reused)
    monkeypatch.setenv("MOEARC_DECODE_VARIANT", variant)
    with Context() as cx:
        _batched_ragged(cx)
        _batched_ragged(cx)


def _batched_ragged(ctx):
    # BASELINE config 3 in miniature: ragged lengths, 256-token pages in one shared pool through a
    # random page permutation, SWA-128 and full, f16 output option
    H, G, D, pt = 64, 8, 64, 256
    rng = np.random.default_rng(3)
    lens = rng.integers(100, 3000, size=9).astype(np.uint32)
    pages = [-(-int(n) // pt) for n in lens]
    total_pages = sum(pages) + 3
    perm = fx.synth.random_block_table(0xB7, total_pages)
    stride = max(pages)
    bts = np.zeros((len(lens), stride), np.uint32)
    off = 0
    for i, p in enumerate(pages):
        bts[i, :p] = perm[off:off + p]
        off += p
    row = G * D
    kp = fx.synth.f16_bits(fx.synth.normal(0xB8, total_pages * pt * row))
    vp = fx.synth.f16_bits(fx.synth.normal(0xB9, total_pages * pt * row))
    q = fx.synth.normal(0xBA, len(lens) * H * D).reshape(len(lens), H, D)
    sinks = fx.synth.normal(0xBB, H)
    dk, dv, dq, dbt, ds = (ctx.upload(kp), ctx.upload(vp), ctx.upload(q), ctx.upload(bts),
                           ctx.upload(sinks))
    for window in (0, 128):
        kb = np.maximum(lens.astype(np.int64) - window, 0).astype(np.uint32) if window else np.zeros_like(lens)
        want = oracle.attn_decode_batched(q, kp, vp, bts, kb, lens, H, G, D, pt, 0.125, sinks=sinks,
                                          n_threads=8)
        for out_type in (OUT_F32, OUT_F16):
            nb = 2 if out_type == OUT_F16 else 4
            dout = ctx.alloc(len(lens) * H * D * nb)
            ctx.attn_decode_batched(dout, dq, dk, dv, dbt, stride, kb, lens, ds, H, G, D, pt, 0.125,
                                    KvType.F16, out_type=out_type)
            got = ctx.download(dout, np.float16 if out_type == OUT_F16 else np.float32, want.shape)
            _report(f"batched window={window} out={'f16' if nb == 2 else 'f32'}", got, want, TOL_NS)
    with pytest.raises(BadArgument):  # an empty span in one sequence refuses the call
        ctx.attn_decode_batched(ctx.alloc(len(lens) * H * D * 4), dq, dk, dv, dbt, stride, lens,
                                lens, ds, H, G, D, pt, 0.125, KvType.F16)


def _shared_pool_case(seed, lens, pool_pages, spike=0.0, pt=256):
    """Full-size batched decode input: one pool of random f16 pages (K rows optionally spiked by
    8x), each sequence reading its own random permutation of the pool, so B long sequences cost one
    pool of host memory while the kernel still walks B distinct page tables."""
    H, G, D = 64, 8, 64
    row = G * D
    rng = np.random.default_rng(seed)
    n_tok = pool_pages * pt
    kp = np.empty(n_tok * row, np.uint16)
    vp = np.empty_like(kp)
    step = 1 << 16
    for s in range(0, n_tok, step):
        n = min(step, n_tok - s)
        k = rng.standard_normal((n, row), dtype=np.float32)
        if spike:
            k[rng.random(n) < spike] *= np.float32(8.0)
        kp[s * row:(s + n) * row] = k.astype(np.float16).view(np.uint16).ravel()
        vp[s * row:(s + n) * row] = rng.standard_normal(n * row, dtype=np.float32).astype(np.float16).view(np.uint16)
    pages = [-(-int(n) // pt) for n in lens]
    assert max(pages) <= pool_pages
    bts = np.stack([rng.permutation(pool_pages).astype(np.uint32) for _ in lens])
    q = rng.standard_normal((len(lens), H, D), dtype=np.float32)
    sinks = rng.standard_normal(H, dtype=np.float32)
    return H, G, D, pt, kp, vp, bts, q, sinks


def _check_batched_full_size(ctx, label, case, lens, windows, out_types):
    H, G, D, pt, kp, vp, bts, q, sinks = case
    dk, dv, dq, dbt, ds = (ctx.upload(kp), ctx.upload(vp), ctx.upload(q), ctx.upload(bts),
                           ctx.upload(sinks))
    stride = bts.shape[1]
    for window in windows:
        kb = np.maximum(lens.astype(np.int64) - window, 0).astype(np.uint32) if window else np.zeros_like(lens)
        want = oracle.attn_decode_batched(q, kp, vp, bts, kb, lens, H, G, D, pt, 0.125, sinks=sinks,
                                          n_threads=16)
        for out_type in out_types:
            nb = 2 if out_type == OUT_F16 else 4
            dout = ctx.alloc(len(lens) * H * D * nb)
            ctx.attn_decode_batched(dout, dq, dk, dv, dbt, stride, kb, lens, ds, H, G, D, pt, 0.125,
                                    KvType.F16, out_type=out_type)
            got = ctx.download(dout, np.float16 if out_type == OUT_F16 else np.float32, want.shape)
            _report(f"{label} window={window} out={'f16' if nb == 2 else 'f32'}", got, want, TOL_NS)


def test_config3_full_size(ctx):
    # B=32 ragged lengths ~U[1024, 32768], 256-token pages through random page
    # tables, SWA-128 and full
    lens = np.random.default_rng(33).integers(1024, 32769, size=32).astype(np.uint32)
    case = _shared_pool_case(0xC3, lens, pool_pages=128)
    _check_batched_full_size(ctx, "config 3", case, lens, (0, 128), (OUT_F32, OUT_F16))


def test_config5_full_size(ctx):
    # B=8 x 131072 keys, full attention, 256-token pages, 1% of K rows x8 (the
    # running maximum moves late and often); 2 GiB of K/V read per call
    lens = np.full(8, 131072, np.uint32)
    case = _shared_pool_case(0xC5, lens, pool_pages=512, spike=0.01)
    _check_batched_full_size(ctx, "config 5", case, lens, (0,), (OUT_F32,))


def test_large_q_magnitudes(ctx):
    # q beyond f16's range and far below it: the power-of-two normalisation keeps the hi/lo split exact
    c = fx.north_star_case(0x51, 700, pt=64)
    for mult in (1e5, 1e-6):
        cq = fx.Case(**dict(c.__dict__))
        cq.q = (c.q * np.float32(mult)).astype(np.float32)
        b = _upload_case(ctx, cq)
        got = _decode(ctx, cq, b, 0)
        want = oracle.attn_decode(cq.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                                  float(c.scale), kv_type=1, sinks=c.sinks)
        _report(f"q x {mult:g}", got, want, TOL_NS)


@pytest.mark.parametrize("variant,n_kv,kv_begin,pt,split", [
    ("4x2x4", 32768, 0, 256, 0), ("4x2x4", 5000, 123, 32, 0), ("1x4x1", 1500, 0, 16, 128),
    ("1x4x1", 9000, 8000, 64, 128), ("4x2x4", 70000, 1000, 16, 0)])
def test_repeated_calls_on_fresh_data(monkeypatch, variant, n_kv, kv_begin, pt, split):
    """Three calls per context, each on different data, so a record left over from an earlier
    call (the workspace is reused, never cleared) would show; pages smaller than a tile and spans
    that start mid-page exercise the per-lane block-table walk."""
    monkeypatch.setenv("MOEARC_DECODE_VARIANT", variant)
    if split:
        monkeypatch.setenv("MOEARC_DECODE_SPLIT", str(split))
    with Context() as cx:
        for rep in range(3):
            c = fx.north_star_case(0xF5E0 + 17 * rep + n_kv, n_kv, pt=pt)
            b = _upload_case(cx, c)
            got = _decode(cx, c, b, kv_begin)
            want = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, kv_begin, n_kv, pt,
                                      float(c.scale), kv_type=1, sinks=c.sinks)
            _report(f"{variant} n_kv={n_kv} begin={kv_begin} pt={pt} split={split} rep={rep}", got,
                    want, TOL_NS)
