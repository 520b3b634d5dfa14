"""RoPE and the fused RoPE-K + chunk append on the GPU, through the C ABI, against the oracle.

The first two tests are the reference's own (kernels_gpu.rs:292-398) at their tolerances: the
elementwise comparison with reference::rope at small positions, and the length invariant at long
ones. YaRN is checked at gpt-oss's parameters against the f64 closed form. The fused append must
equal moearc_rope followed by moearc_kv_append_chunk bit for bit (the same device arithmetic), and
the oracle's rope-then-append within the f16 rounding of the stored keys.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import BadArgument, Context, KvType, RopeKind, RopeScaling
from oracle import oracle

pytestmark = pytest.mark.gpu

U = 5.960464477539063e-8  # kernels_gpu.rs:33
R = fx.ROPE_REF
GPT = fx.GPT_OSS_ROPE


def _yarn(n_dims=64):
    return RopeScaling.yarn(n_dims, GPT["n_ctx_orig"], GPT["freq_base"], GPT["factor"], GPT["beta_fast"],
                            GPT["beta_slow"])


def _report(label, err, tol):
    print(f"{label}: max |gpu - oracle| = {err:.3e} (tolerance {tol:.3e})", flush=True)
    assert err <= tol, f"{label}: {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("kind", [RopeKind.NORMAL, RopeKind.NEOX])
def test_rope_matches_the_cpu_reference(ctx, kind):
    # kernels_gpu.rs:292-351
    src, pos = fx.rope_reference_inputs()
    dsrc, dpos, ddst = ctx.upload(src), ctx.upload(pos), ctx.alloc(src.nbytes)
    ctx.rope(ddst, dsrc, dpos, R["tokens"], R["heads"], R["head_dim"], R["n_dims"], R["freq_base"],
             kind=kind)
    got = ctx.download(ddst, np.float32, src.shape)
    g = fx.load_golden("ref_rope")
    want = g["expected_neox" if kind == RopeKind.NEOX else "expected_normal"]
    tol = 4.0 * (16.0 * 12.0 + 4.0) * U
    _report(f"rope {kind.name}", float(np.max(np.abs(got.astype(np.float64) - want))), tol)
    g3, s3 = got.reshape(5, 4, 80), src.reshape(5, 4, 80)
    assert np.array_equal(g3[..., 64:], s3[..., 64:]), "channels past n_dims must pass through"
    assert np.max(np.abs(g3[1, :, :64] - s3[1, :, :64])) > 1e-3, "token 1 did not move"


@pytest.mark.parametrize("kind", [RopeKind.NORMAL, RopeKind.NEOX])
def test_rope_preserves_pair_lengths(ctx, kind):
    # kernels_gpu.rs:354-398, and the same with YaRN, where lengths scale by mscale
    rng = oracle.Rng(0x1507)
    src = rng.vec_unit(3 * 2 * 64)
    pos = np.array([0, 2048, 4095], np.int32)
    dsrc, dpos, ddst = ctx.upload(src), ctx.upload(pos), ctx.alloc(src.nbytes)
    x = src.astype(np.float64).reshape(3, 2, 64)
    for scaling, msc, label in ((None, 1.0, "plain"), (_yarn(), 1.0 + 0.1 * np.log(GPT["factor"]), "yarn")):
        ctx.rope(ddst, dsrc, dpos, 3, 2, 64, 64, 10000.0, scaling=scaling, kind=kind)
        y = ctx.download(ddst, np.float32, src.shape).astype(np.float64).reshape(3, 2, 64)
        if kind == RopeKind.NEOX:
            b, a = np.hypot(x[..., :32], x[..., 32:]), np.hypot(y[..., :32], y[..., 32:])
        else:
            b, a = np.hypot(x[..., 0::2], x[..., 1::2]), np.hypot(y[..., 0::2], y[..., 1::2])
        _report(f"pair length {kind.name} {label}", float(np.max(np.abs(a - msc * b))), 32.0 * U * 1.5 * msc)


def test_yarn_matches_the_closed_form(ctx):
    # gpt-oss RoPE at small positions, where an f32 angle is exact to a few ulp
    rng = np.random.default_rng(11)
    n, H, D = 40, 8, 64
    src = rng.standard_normal(n * H * D).astype(np.float32)
    pos = np.arange(n, dtype=np.int32) * 2
    sc = _yarn()
    dsrc, dpos, ddst = ctx.upload(src), ctx.upload(pos), ctx.alloc(src.nbytes)
    ctx.rope(ddst, dsrc, dpos, n, H, D, D, GPT["freq_base"], scaling=sc, kind=RopeKind.NEOX)
    got = ctx.download(ddst, np.float32, src.shape).astype(np.float64)
    want = oracle.rope_yarn(src, pos, n, H, D, D, GPT["freq_base"], *sc.args(), neox=True)
    # angle <= 78 rad: 16 ulp of it, times |x| <= ~5, times mscale, plus the rotation's own rounding
    tol = 16.0 * 78.0 * 2 * U * 5.0 * 1.35 + 8 * U * 5.0
    _report("yarn closed form", float(np.max(np.abs(got - want))), tol)


def _chunk(n_tok, G, D, pt, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_tok, G, D)).astype(np.float32)
    v = rng.standard_normal((n_tok, G, D)).astype(np.float32)
    pos0 = 1000
    pos = (pos0 + np.arange(n_tok)).astype(np.int32)
    n_pages = -(-(pos0 + n_tok) // pt) + 2
    perm = fx.synth.random_block_table(seed, n_pages).astype(np.uint32)
    pages = perm[pos // pt].astype(np.uint32)
    slots = (pos % pt).astype(np.uint32)
    return k, v, pos, pages, slots, n_pages


# f16 pools with NeoX over all 64 channels and KV heads dividing 16 take the whole-row kernel
# (moearc_rope_kv_append_chunk64_k: 16 / G tokens per work-group, G = 1 and 16 its extremes, 300
# tokens leaving the last work-group part empty for G = 1); G = 3 and f32 pools the general one
@pytest.mark.parametrize("pt,kv,G", [(256, KvType.F16, 8), (16, KvType.F16, 8), (32, KvType.F32, 8),
                                     (16, KvType.F16, 1), (256, KvType.F16, 16), (16, KvType.F16, 3)],
                         ids=str)
def test_fused_append_equals_rope_then_append(ctx, pt, kv, G):
    n_tok, D = 300, 64
    k, v, pos, pages, slots, n_pages = _chunk(n_tok, G, D, pt, 0x40 + pt)
    el = 2 if kv == KvType.F16 else 4
    nbytes = n_pages * pt * G * D * el
    dk, dv, dpos, dpg, dsl = ctx.upload(k), ctx.upload(v), ctx.upload(pos), ctx.upload(pages), ctx.upload(slots)
    sc = _yarn()
    pools = []
    for fused in (True, False):
        kp, vp = ctx.alloc(nbytes), ctx.alloc(nbytes)
        ctx.zero(kp, nbytes // 4)
        ctx.zero(vp, nbytes // 4)
        if fused:
            ctx.rope_kv_append_chunk(kp, vp, dk, dv, dpos, dpg, dsl, n_tok, G, D, pt, D, GPT["freq_base"],
                                     scaling=sc, kind=RopeKind.NEOX, kv=kv)
        else:
            kr = ctx.alloc(k.nbytes)
            ctx.rope(kr, dk, dpos, n_tok, G, D, D, GPT["freq_base"], scaling=sc, kind=RopeKind.NEOX)
            ctx.kv_append_chunk(kp, vp, kr, dv, dpg, dsl, n_tok, G, D, pt, kv)
        dt = np.uint16 if kv == KvType.F16 else np.float32
        pools.append((ctx.download(kp, dt, nbytes // el), ctx.download(vp, dt, nbytes // el)))
    assert np.array_equal(pools[0][0], pools[1][0]), "fused K differs from rope + append"
    assert np.array_equal(pools[0][1], pools[1][1]), "fused V differs from append"
    # against the oracle's rope-then-append (f64 closed form rounded to f32, then stored)
    if kv == KvType.F16:
        ok = np.zeros(nbytes // 2, np.uint16)
        ov = np.zeros_like(ok)
        oracle.rope_kv_append_chunk(ok, ov, k, v, pos, pages, slots, n_tok, G, D, pt, D, GPT["freq_base"],
                                    sc.args(), True, 1)
        assert np.array_equal(pools[0][1], ov), "V must be stored exactly"
        gk, wk = oracle.f16_to_f32(pools[0][0]), oracle.f16_to_f32(ok)
        # positions ~1300 (angles ~1300 rad): f32 angle error ~16 ulp of the angle times |k|, plus
        # one f16 ulp of the stored key
        tol = 16.0 * 1300.0 * 2 * U * 5.0 * 1.35 + np.abs(wk) * 2.0 ** -10 + 1e-7
        err = np.abs(gk.astype(np.float64) - wk)
        print(f"fused append pt={pt}: max |gpu - oracle| = {err.max():.3e}", flush=True)
        assert np.all(err <= tol)


def test_fused_append_config4_chunk(ctx):
    # a config-4 chunk's keys and values (2048 tokens at positions 1000 .. 3047, 8 KV heads,
    # 256-token pages through a random permutation) against the oracle's rope-then-append
    n_tok, D, G, pt = 2048, 64, 8, 256
    k, v, pos, pages, slots, n_pages = _chunk(n_tok, G, D, pt, 0x4C4)
    nbytes = n_pages * pt * G * D * 2
    kp, vp = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ctx.zero(kp, nbytes // 4)
    ctx.zero(vp, nbytes // 4)
    sc = _yarn()
    ctx.rope_kv_append_chunk(kp, vp, ctx.upload(k), ctx.upload(v), ctx.upload(pos), ctx.upload(pages),
                             ctx.upload(slots), n_tok, G, D, pt, D, GPT["freq_base"], scaling=sc,
                             kind=RopeKind.NEOX, kv=KvType.F16)
    gk, gv = ctx.download(kp, np.uint16, nbytes // 2), ctx.download(vp, np.uint16, nbytes // 2)
    ok = np.zeros(nbytes // 2, np.uint16)
    ov = np.zeros_like(ok)
    oracle.rope_kv_append_chunk(ok, ov, k, v, pos, pages, slots, n_tok, G, D, pt, D, GPT["freq_base"],
                                sc.args(), True, 1)
    assert np.array_equal(gv, ov), "V must be stored exactly"
    wk = oracle.f16_to_f32(ok)
    # angles up to ~3050 rad: f32 angle error ~16 ulp of the angle times |k|, plus one f16 ulp
    tol = 16.0 * 3050.0 * 2 * U * 5.0 * 1.35 + np.abs(wk) * 2.0 ** -10 + 1e-7
    err = np.abs(oracle.f16_to_f32(gk).astype(np.float64) - wk)
    print(f"fused append, config-4 chunk: max |gpu - oracle| = {err.max():.3e}", flush=True)
    assert np.all(err <= tol)


def test_refusals(ctx):
    src, pos = fx.rope_reference_inputs()
    dsrc, dpos, ddst = ctx.upload(src), ctx.upload(pos), ctx.alloc(src.nbytes)
    for n_dims in (0, 63, 82):
        with pytest.raises(BadArgument):
            ctx.rope(ddst, dsrc, dpos, 5, 4, 80, n_dims, 10000.0)
    k = ctx.alloc(4 * 8 * 64 * 4)
    pg = ctx.upload(np.zeros(4, np.uint32))
    with pytest.raises(BadArgument):
        ctx.rope_kv_append_chunk(ctx.alloc(1024), ctx.alloc(1024), k, k, dpos, pg, pg, 4, 8, 64, 16, 65,
                                 10000.0)
    with pytest.raises(BadArgument):
        ctx.rope_kv_append_chunk(ctx.alloc(1024), ctx.alloc(1024), k, k, dpos, pg, pg, 4, 8, 64, 0, 64,
                                 10000.0)
