"""The attention block over prompt chunks (moearc_attn_block_chunk) on the GPU, against the oracle
composed step by step as the reference engine runs one token at a time (moe.rs:1942-2071):
projections + biases (orc_matvec_q), NeoX RoPE (orc_rope_yarn), the f16 KV append
(orc_kv_append_raw), attention as repeated decode (orc_attn_prefill) and the output projection
added to the residual.

Bar: every attention output within the north star's 2e-3, carried through W_o: per residual
element |gpu - oracle| <= 2e-3 * sum_c |W_o[r][c]| + 1e-5. The activations are scaled (x ~
N(0, 0.01)) so that q and k come out O(1), as a normed residual gives them: with scores in the
thousands the softmax turns a one-ulp f16 difference in a rotated key (f32 angles on the GPU,
f64 in the oracle) into a different winner, which no attention tolerance covers.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import AttnBlockDesc, KvType, RopeScaling
from moearc_amd.kv import KvGeometry, PagedKvCache
from oracle import oracle

pytestmark = pytest.mark.gpu

TOY = dict(E=256, H=8, G=2, D=64, PT=16)
# gpt-oss-20b's attention block: 2880-wide residual, 64 query heads over 8 KV heads (group 8, the
# prefill_g8 kernel), head_dim 64, 256-token pages
GPT_OSS = dict(E=2880, H=64, G=8, D=64, PT=256)


class Block:
    def __init__(self, ctx, types, seed, biases=True, sinks=True, n_swa=0, n_ctx=256, chunk=64,
                 scaling=None, freq_base=10000.0, dims=TOY, x_scale=0.1):
        self.types, self.n_swa, self.scaling, self.freq_base = types, n_swa, scaling or RopeScaling(), freq_base
        self.E, self.H, self.G, self.D, self.PT = (dims[k] for k in ("E", "H", "G", "D", "PT"))
        self.x_scale = x_scale
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        shapes = [(H * D, E), (G * D, E), (G * D, E), (E, H * D)]
        self.w = [fx.synth_blocks(t, r * c // fx.QT_BLOCK[t][1], seed + i)[0] for i, (t, (r, c)) in
                  enumerate(zip(types, shapes))]
        self.shapes = shapes
        self.b = [fx.synth.unit(seed + 10 + i, r).astype(np.float32) * np.float32(0.1) if biases else None
                  for i, (r, _) in enumerate(shapes)]
        self.sinks = fx.synth.unit(seed + 20, H).astype(np.float32) if sinks else None
        geo = KvGeometry.plan(n_ctx, PT, n_swa or None, chunk=chunk)
        self.ring = n_swa > 0
        self.n_pages = geo.swa_pages if self.ring else geo.pages + 2
        self.table = geo.ring_table() if self.ring else None
        self.pool = None if self.ring else PagedKvCache(self.n_pages, PT, n_ctx)
        if self.pool is not None:
            self.pool.begin(7, 0)
        self.kp = np.zeros(self.n_pages * PT * G * D, np.uint16)  # the oracle's copy of the pages
        self.vp = np.zeros_like(self.kp)
        self.d_w = [ctx.upload(w) for w in self.w]
        self.d_b = [ctx.upload(b) if b is not None else None for b in self.b]
        self.d_s = ctx.upload(self.sinks) if sinks else None
        self.d_kp, self.d_vp = ctx.alloc(self.kp.nbytes), ctx.alloc(self.vp.nbytes)
        ctx.upload_slice(self.d_kp, self.kp)
        ctx.upload_slice(self.d_vp, self.vp)
        self.n = 0  # tokens so far

    def places(self, n):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        if self.ring:
            pos = np.arange(self.n, self.n + n)
            return self.table[pos // PT].astype(np.uint32), (pos % PT).astype(np.uint32), self.table
        pages, slots = self.pool.append_chunk(7, n)
        return pages, slots, np.array(self.pool.pages_of(7).pages, np.uint32)

    def rope(self, a, pos, heads):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        s = self.scaling
        return oracle.rope_yarn(a, pos, len(pos), heads, D, D, self.freq_base, s.freq_scale, s.ext_factor,
                                s.attn_factor, s.corr_lo, s.corr_hi).astype(np.float32)

    def oracle_chunk(self, h, x, pages, slots, table):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        n, pos0 = x.shape[0], self.n
        pos = np.arange(pos0, pos0 + n, dtype=np.int32)
        proj = []
        for i, (r, c) in enumerate(self.shapes[:3]):
            y = np.stack([oracle.matvec_q(self.types[i], self.w[i], x[t], r, c)[0] for t in range(n)])
            proj.append(y + self.b[i] if self.b[i] is not None else y)
        q, k, v = proj
        qr, kr = self.rope(q, pos, H), self.rope(k, pos, G).reshape(n, G * D)
        for t in range(n):
            oracle.kv_append_raw(self.kp, self.vp, kr[t], v[t], int(pages[t]), int(slots[t]), G, D, PT,
                                 oracle.KV_F16)
        # a chunk's q enters the prefill kernel in f16; a single token's stays f32 (the decode call)
        q16 = (qr.astype(np.float16).astype(np.float32) if n > 1 else qr).reshape(n, H, D)
        att = oracle.attn_prefill(q16, self.kp, self.vp, table, n, pos0, self.n_swa, H, G, D, PT,
                                  1.0 / np.sqrt(D), sinks=self.sinks, n_threads=8).reshape(n, H * D)
        r, c = self.shapes[3]
        o = np.stack([oracle.matvec_q(self.types[3], self.w[3], att[t], r, c)[0] for t in range(n)])
        if self.b[3] is not None:
            o = o + self.b[3]
        return (h + o).astype(np.float32)

    def desc(self, ctx, d_table):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        return AttnBlockDesc.make(self.types, self.d_w, self.d_b, self.d_s, self.d_kp, self.d_vp, d_table,
                                  E, H, G, D, PT, self.n_swa, float(np.float32(1.0 / np.sqrt(D))), D,
                                  self.freq_base, self.scaling, ring_pages=self.n_pages if self.ring else 0)

    def gpu_chunk(self, ctx, h, x, pages, slots, table):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        n = x.shape[0]
        d_h, d_x = ctx.upload(h), ctx.upload(x)
        pos = np.arange(self.n, self.n + n, dtype=np.int32)
        ctx.attn_block_chunk(self.desc(ctx, ctx.upload(table)), d_h, d_x, n, self.n, ctx.upload(pos),
                             ctx.upload(pages), ctx.upload(slots))
        return ctx.download(d_h, np.float32, (n, E))

    def bound(self):
        r, c = self.shapes[3]  # noqa: E501
        wo = oracle.dequant(self.types[3], self.w[3], r * c // fx.QT_BLOCK[self.types[3]][1]).reshape(r, c)
        return 2e-3 * np.abs(wo.astype(np.float64)).sum(axis=1) + 1e-5

    def step(self, ctx, n, seed, label):
        E, H, G, D, PT = self.E, self.H, self.G, self.D, self.PT
        x = (fx.synth.normal(seed, n * E) * self.x_scale).astype(np.float32).reshape(n, E)
        h = fx.synth.normal(seed + 1, n * E).astype(np.float32).reshape(n, E)
        pages, slots, table = self.places(n)
        got = self.gpu_chunk(ctx, h, x, pages, slots, table)
        want = self.oracle_chunk(h, x, pages, slots, table)
        self.n += n
        err = np.abs(got.astype(np.float64) - want)
        worst = float(np.max(err / self.bound()))
        print(f"{label}: {n} tokens at {self.n - n}: worst |gpu - oracle| / bound = {worst:.3f}", flush=True)
        assert worst <= 1.0, label
        return got


def test_chunks_then_decode_full_attention(ctx):
    blk = Block(ctx, (8, 8, 8, 8), 0xB10C)
    blk.step(ctx, 37, 1, "full, Q8_0, chunk 1")
    blk.step(ctx, 29, 3, "full, Q8_0, chunk 2")
    blk.step(ctx, 1, 5, "full, Q8_0, decode step")


def test_windowed_ring_mixed_types_yarn(ctx):
    # a windowed block through its ring (sized for window + chunk), sinks, YaRN, four weight types
    blk = Block(ctx, (1, 8, 12, 14), 0xB20C, n_swa=24, chunk=40,
                scaling=RopeScaling.yarn(TOY["D"], 4096, 150000.0, 32.0), freq_base=150000.0)
    blk.step(ctx, 40, 11, "SWA-24 ring, chunk 1")
    blk.step(ctx, 33, 13, "SWA-24 ring, chunk 2")
    blk.step(ctx, 1, 15, "SWA-24 ring, decode step")


@pytest.mark.parametrize("n_swa", [0, 128])
def test_gpt_oss_shape_chunks_then_decode(ctx, n_swa):
    # the block at gpt-oss-20b's shape: Q8_0 projections with biases, sinks, YaRN (factor 32 over a
    # 4096-token original context, base 150000), group-8 prefill, a full layer through pool pages and
    # a windowed (SWA-128) layer through its ring; two chunks then a decode step. Activations scaled
    # so q and k come out O(1) at 2880 columns.
    blk = Block(ctx, (8, 8, 8, 8), 0xB50C + n_swa, n_swa=n_swa, n_ctx=512, chunk=160,
                scaling=RopeScaling.yarn(64, 4096, 150000.0, 32.0), freq_base=150000.0, dims=GPT_OSS,
                x_scale=0.03)
    label = f"gpt-oss {'SWA-128 ring' if n_swa else 'full'}"
    blk.step(ctx, 160, 21, f"{label}, chunk 1")
    blk.step(ctx, 97, 23, f"{label}, chunk 2")
    blk.step(ctx, 1, 25, f"{label}, decode step")


@pytest.mark.parametrize("n_swa", [0, 128])
def test_gpt_oss_shape_long_chunk(ctx, n_swa):
    # one 1024-token chunk through the block at gpt-oss-20b's shape: eight token tiles in every
    # launch (the q/k/v product without split-K, the output projection with it, the group-8
    # prefill over 1024 rows), then a decode step
    blk = Block(ctx, (8, 8, 8, 8), 0xB70C + n_swa, n_swa=n_swa, n_ctx=1088, chunk=1024,
                scaling=RopeScaling.yarn(64, 4096, 150000.0, 32.0), freq_base=150000.0, dims=GPT_OSS,
                x_scale=0.03)
    label = f"gpt-oss {'SWA-128 ring' if n_swa else 'full'}"
    blk.step(ctx, 1024, 31, f"{label}, 1024-token chunk")
    blk.step(ctx, 1, 33, f"{label}, decode step")


def test_chunk_equals_token_by_token(ctx):
    # the chunked call against the reference's shape of work, one token per call, both on the GPU
    a, b = Block(ctx, (8, 8, 8, 8), 0xB30C, sinks=False), Block(ctx, (8, 8, 8, 8), 0xB30C, sinks=False)
    n, E = 21, a.E
    x = (fx.synth.normal(0x77, n * E) * 0.1).astype(np.float32).reshape(n, E)
    h = fx.synth.normal(0x78, n * E).astype(np.float32).reshape(n, E)
    pa, sa, ta = a.places(n)
    chunked = a.gpu_chunk(ctx, h, x, pa, sa, ta)
    rows = []
    for t in range(n):
        p1, s1, t1 = b.places(1)
        rows.append(b.gpu_chunk(ctx, h[t:t + 1], x[t:t + 1], p1, s1, t1)[0])
        b.n += 1
    err = np.abs(chunked.astype(np.float64) - np.stack(rows))
    worst = float(np.max(err / a.bound()))
    print(f"chunk of {n} vs {n} single-token calls: worst / bound = {worst:.3f}", flush=True)
    assert worst <= 1.0


@pytest.mark.parametrize("dims", ["toy", "gpt_oss", "toy_no_biases"])
def test_fused_launches_equal_separate_ones(monkeypatch, dims):
    # The block's fused steps (the default) against the launches they replace (MOEARC_BLOCK_FUSED=0):
    # the RoPE of q and the K/V append as one launch (moearc_rope_qkv_chunk64_k; after a split q/k/v
    # product moearc_rope_qkv_sums64_k, which also adds the product's k-slice sums and biases in
    # place of its reduction launch), and the prefill writing the output projection's f16 hi + lo
    # split instead of f32 rows and a split launch. The residual after a 45-token chunk (the
    # 16-token product), a 128-token one (the MFMA product) and a decode step, and both pools,
    # bit-identical.
    from moearc_amd import Context
    d = GPT_OSS if dims == "gpt_oss" else TOY
    got = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("MOEARC_BLOCK_FUSED", fused)
        with Context() as cx:
            blk = Block(cx, (8, 8, 8, 8), 0xB60C, biases=dims != "toy_no_biases", n_ctx=256, chunk=128, dims=d,
                        x_scale=0.03,
                        scaling=RopeScaling.yarn(64, 4096, 150000.0, 32.0), freq_base=150000.0)
            outs = []
            for n, seed in ((45, 31), (128, 35), (1, 33)):
                x = (fx.synth.normal(seed, n * blk.E) * blk.x_scale).astype(np.float32).reshape(n, blk.E)
                h = fx.synth.normal(seed + 1, n * blk.E).astype(np.float32).reshape(n, blk.E)
                pages, slots, table = blk.places(n)
                outs.append(blk.gpu_chunk(cx, h, x, pages, slots, table))
                blk.n += n
            outs.append(cx.download(blk.d_kp, np.uint16, blk.kp.shape))
            outs.append(cx.download(blk.d_vp, np.uint16, blk.vp.shape))
        got[fused] = outs
    for name, a, b in zip(("chunk", "chunk of 128", "decode step", "K pool", "V pool"), got["1"], got["0"]):
        print(f"fused block launches, {dims}, {name}: {int(np.sum(a.view(np.uint8) != b.view(np.uint8)))} bytes differ",
              flush=True)
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name


def test_wide_tile_products_in_the_block(monkeypatch):
    # The block's q/k/v product is one launch over three matrices (segments of row tiles); with
    # MOEARC_MM_WIDE=1 it and the output projection run on the eight-wave 128 x 256 tiles (as a
    # 2048-token chunk's q/k/v product does by default). Without split-K the block's outputs and
    # pools equal the 128 x 128 tiles' to the bit; with it, the oracle's bar.
    from moearc_amd import Context
    monkeypatch.setenv("MOEARC_MM_SPLIT_WG", "0")
    got = {}
    for wide in ("1", "0"):
        monkeypatch.setenv("MOEARC_MM_WIDE", wide)
        with Context() as cx:
            blk = Block(cx, (8, 8, 8, 8), 0xB80C, n_ctx=512, chunk=160, dims=GPT_OSS, x_scale=0.03,
                        scaling=RopeScaling.yarn(64, 4096, 150000.0, 32.0), freq_base=150000.0)
            outs = []
            for n, seed in ((160, 41), (97, 43), (1, 45)):
                x = (fx.synth.normal(seed, n * blk.E) * blk.x_scale).astype(np.float32).reshape(n, blk.E)
                h = fx.synth.normal(seed + 1, n * blk.E).astype(np.float32).reshape(n, blk.E)
                pages, slots, table = blk.places(n)
                outs.append(blk.gpu_chunk(cx, h, x, pages, slots, table))
                blk.n += n
            outs.append(cx.download(blk.d_kp, np.uint16, blk.kp.shape))
        got[wide] = outs
    for name, a, b in zip(("chunk 1", "chunk 2", "decode step", "K pool"), got["1"], got["0"]):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"wide tiles changed the block's {name}"
    monkeypatch.delenv("MOEARC_MM_SPLIT_WG")
    monkeypatch.setenv("MOEARC_MM_WIDE", "1")
    with Context() as cx:
        blk = Block(cx, (8, 8, 8, 8), 0xB90C, n_ctx=512, chunk=160, dims=GPT_OSS, x_scale=0.03,
                    scaling=RopeScaling.yarn(64, 4096, 150000.0, 32.0), freq_base=150000.0)
        blk.step(cx, 160, 51, "gpt-oss full, wide tiles with split-K, chunk 1")
        blk.step(cx, 1, 53, "gpt-oss full, wide tiles with split-K, decode step")


def test_refusals(ctx):
    blk = Block(ctx, (8, 8, 8, 8), 0xB40C)
    d = blk.desc(ctx, ctx.upload(np.arange(4, dtype=np.uint32)))
    lib = ctx._lib
    buf = ctx.alloc(4096)
    assert lib.moearc_attn_block_chunk(ctx.raw, None, buf.ptr, buf.ptr, 1, 0, buf.ptr, buf.ptr, buf.ptr) == -1
    d.w_type[3] = 2  # Q4_0: not a format the path expands
    import ctypes
    assert lib.moearc_attn_block_chunk(ctx.raw, ctypes.byref(d), buf.ptr, buf.ptr, 1, 0, buf.ptr, buf.ptr,
                                       buf.ptr) == -2
    d.w_type[3] = 8
    # a windowed block whose ring cannot hold the chunk's keys (n_tok + n_swa - 1 > ring tokens)
    d.n_swa, d.ring_pages = 24, 2  # 32 ring tokens
    assert lib.moearc_attn_block_chunk(ctx.raw, ctypes.byref(d), buf.ptr, buf.ptr, 10, 0, buf.ptr, buf.ptr,
                                       buf.ptr) == -2
    d.n_swa, d.ring_pages = 0, 0
    d.head_dim = 32
    assert lib.moearc_attn_block_chunk(ctx.raw, ctypes.byref(d), buf.ptr, buf.ptr, 1, 0, buf.ptr, buf.ptr,
                                       buf.ptr) == -2
    ctx.sync()
    assert KvType.F16 == 1
