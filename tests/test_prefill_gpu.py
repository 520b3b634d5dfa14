"""Chunked-prefill parity on the GPU against the oracle (row i == decode at n_kv = pos0+i+1).

Golden fixtures pin a small gpt-oss-shaped chunk; the oracle covers every GQA group the kernel
supports, windowed and full layers, ragged chunk ends and page sizes, score jumps and large scores;
at BASELINE config 4's full size (2048 new tokens after 2048 cached) every output is compared with
the oracle, also with config 5's stress pattern. The bar is the north star's: max-abs error <= 2e-3
on the output.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import BadArgument, KvType, OUT_F16, OUT_F32
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _report(label, got, want, tol=TOL):
    err = float(np.nanmax(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
    print(f"{label}: max |gpu - oracle| = {err:.3e} (tolerance {tol:.3e})", flush=True)
    assert err <= tol, f"{label}: {err:.3e} > {tol:.3e}"


def _run(ctx, pc, n_swa, out_type=OUT_F32, sinks=True):
    dk, dv, dbt = ctx.upload(pc.k_raw), ctx.upload(pc.v_raw), ctx.upload(pc.bt)
    ds = ctx.upload(pc.sinks) if sinks else None
    dq = ctx.upload(np.ascontiguousarray(pc.qp).view(np.uint16))
    nb = 2 if out_type == OUT_F16 else 4
    dout = ctx.alloc(pc.n_q * pc.H * pc.D * nb)
    ctx.attn_prefill(dout, dq, dk, dv, dbt, ds, pc.n_q, pc.pos0, n_swa, pc.H, pc.G, pc.D, pc.pt,
                     float(pc.scale), KvType.F16, out_type=out_type)
    return ctx.download(dout, np.float16 if out_type == OUT_F16 else np.float32,
                        (pc.n_q, pc.H, pc.D)).astype(np.float32)


@pytest.mark.parametrize("golden,n_swa", [("ns_prefill_full", 0), ("ns_prefill_swa16", 16)])
def test_against_golden(ctx, golden, n_swa):
    pc = fx.prefill_case(0x9F11, n_q=48, pos0=80)
    g = fx.load_golden(golden)
    assert str(g["digest"]) == fx.prefill_digest(pc)
    got = _run(ctx, pc, n_swa)
    _report(f"prefill {golden}", got[g["rows"]], g["expected"])


@pytest.mark.parametrize("group,n_q,pos0,pt,n_swa", [
    (8, 100, 37, 32, 0), (8, 100, 37, 32, 128), (8, 17, 0, 16, 0), (8, 70, 300, 64, 5),
    (4, 90, 11, 32, 0), (2, 40, 64, 8, 33), (1, 150, 9, 32, 0), (1, 150, 9, 32, 64),
])
def test_shapes_against_oracle(ctx, group, n_q, pos0, pt, n_swa):
    G = 8 if group > 1 else 4
    pc = fx.prefill_case(0x700 + n_q + pos0 + group, n_q=n_q, pos0=pos0, pt=pt, H=G * group, G=G)
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, n_q, pos0, n_swa,
                               pc.H, pc.G, pc.D, pt, float(pc.scale), sinks=pc.sinks, n_threads=8)
    got = _run(ctx, pc, n_swa)
    _report(f"prefill group={group} n_q={n_q} pos0={pos0} pt={pt} n_swa={n_swa}", got, want)
    nosink = _run(ctx, pc, n_swa, sinks=False)
    want_ns = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, n_q, pos0,
                                  n_swa, pc.H, pc.G, pc.D, pt, float(pc.scale), n_threads=8)
    _report("  without sinks", nosink, want_ns)


# K rows scaled by small factors early and larger ones later: the scores jump by more than 8 in
# base-2 units (the rescale threshold) where a row first sees the scaled-up keys.
JUMPS = {
    "late": [(0, 600, 0.02), (600, 4096, 2.0)],
    "early": [(0, 32, 0.02), (32, 128, 1.8), (128, 4096, 0.3)],
    "bands": [(0, 4096, 0.02), (300, 320, 100.0), (470, 480, 100.0), (700, 716, 100.0)],
}


@pytest.mark.parametrize("group,n_q,pos0,n_swa,jumps", [
    (8, 256, 512, 0, "late"), (8, 256, 512, 0, "early"), (8, 256, 512, 0, "bands"),
    (8, 256, 512, 128, "bands"), (4, 256, 512, 0, "late"), (2, 200, 300, 100, "bands"),
    (1, 300, 200, 64, "bands"),
])
def test_score_jumps_against_oracle(ctx, group, n_q, pos0, n_swa, jumps):
    """Scores that rise far above everything a row saw first: the default kernels' lazy rescale
    (a chunk whose exponents reach the threshold moves the row's reference before its weights are
    formed) runs early in a row ("early"), late in it ("late"), and at several places ("bands")."""
    G = 8 if group > 1 else 4
    pc = fx.prefill_case(0x5C0 + n_q + group, n_q=n_q, pos0=pos0, pt=32, H=G * group, G=G,
                         boost=JUMPS[jumps])
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, n_q, pos0, n_swa,
                               pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks, n_threads=8)
    got = _run(ctx, pc, n_swa)
    assert np.isfinite(got).all()
    _report(f"prefill jumps group={group} n_q={n_q} pos0={pos0} n_swa={n_swa} {jumps}", got, want)


# Large scores: the kernels' arithmetic must not lose accuracy as |q|.|k| grows (scaling q by
# scale*log2(e) in f16 before the product, as an earlier form of the default kernels did, reaches
# 6e-3 max-abs error on "band6" and 1e-2 on "spike8"). "band6": keys 600 onward scaled by 6;
# "spike8": BASELINE config 5's stress pattern, 1% of K rows scaled by 8; "all3": every key by 3.
STRESS = {"band6": dict(boost=[(600, 1 << 20, 6.0)]), "spike8": dict(spike_frac=0.01),
          "all3": dict(boost=[(0, 1 << 20, 3.0)])}


@pytest.mark.parametrize("n_swa", [0, 128])
@pytest.mark.parametrize("stress", sorted(STRESS))
def test_large_scores_against_oracle(ctx, stress, n_swa):
    pc = fx.prefill_case(0x5D0 + len(stress), n_q=256, pos0=1792, pt=32, **STRESS[stress])
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0,
                               n_swa, pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks,
                               n_threads=16)
    got = _run(ctx, pc, n_swa)
    assert np.isfinite(got).all()
    _report(f"prefill {stress} n_q=256 pos0=1792 n_swa={n_swa}", got, want)


@pytest.mark.parametrize("precise", [False, True])
def test_long_context_small_pages(monkeypatch, precise):
    # 40,024 keys in 16-token pages: 2,502 block-table entries per row's span (the kernels read
    # block-table entries per tile, so no page-count limit applies)
    from moearc_amd import Context
    monkeypatch.setenv("MOEARC_PREFILL_PRECISE", "1" if precise else "0")
    pc = fx.prefill_case(0x5E, n_q=24, pos0=40000, pt=16)
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0, 0,
                               pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks, n_threads=16)
    with Context() as cx:
        got = _run(cx, pc, 0)
    _report(f"prefill 40024 keys, 16-token pages, precise={precise}", got, want)


@pytest.mark.parametrize("precise", [False, True])
def test_rows_equal_decode_calls(monkeypatch, precise):
    # the defining property: row i == moearc_attn_decode at n_kv = pos0 + i + 1 (f16 q widened).
    # The precise variant carries p to ~22 bits like decode; the default one p in f16.
    from moearc_amd import Context
    monkeypatch.setenv("MOEARC_PREFILL_PRECISE", "1" if precise else "0")
    ctx = Context()
    pc = fx.prefill_case(0x3D, n_q=40, pos0=200, pt=32)
    got = _run(ctx, pc, 128)
    dk, dv, dbt, ds = ctx.upload(pc.k_raw), ctx.upload(pc.v_raw), ctx.upload(pc.bt), ctx.upload(pc.sinks)
    dq, dout = ctx.alloc(pc.H * pc.D * 4), ctx.alloc(pc.H * pc.D * 4)
    for i in (0, 13, 39):
        n_kv = pc.pos0 + i + 1
        ctx.upload_slice(dq, pc.qp[i].astype(np.float32))
        ctx.attn_decode_ext(dout, dq, dk, dv, dbt, ds, pc.H, pc.G, pc.D, max(0, n_kv - 128), n_kv,
                            pc.pt, float(pc.scale), KvType.F16)
        dec = ctx.download(dout, np.float32, (pc.H, pc.D))
        _report(f"  prefill row {i} vs decode (precise={precise})", got[i], dec, 1e-5 if precise else TOL)
    ctx.close()


def test_precise_variant_against_oracle(monkeypatch):
    from moearc_amd import Context
    monkeypatch.setenv("MOEARC_PREFILL_PRECISE", "1")
    with Context() as cx:
        for n_swa in (0, 16):
            pc = fx.prefill_case(0x9F11, n_q=48, pos0=80)
            g = fx.load_golden("ns_prefill_full" if n_swa == 0 else "ns_prefill_swa16")
            got = _run(cx, pc, n_swa)
            _report(f"precise prefill n_swa={n_swa}", got[g["rows"]], g["expected"], 1e-5)


def _config4(seed, **kw):
    # 2048 new tokens after 2048 cached, 64q/8kv, d64, f16, sinks
    return fx.prefill_case(seed, n_q=2048, pos0=2048, pt=256, **kw)


@pytest.mark.parametrize("n_swa", [0, 128])
def test_config4_full_size(ctx, n_swa):
    """Every one of the 2048 x 64 x 64 outputs of config 4 against the oracle, f32 and f16 out."""
    pc = _config4(0xC4)
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0,
                               n_swa, pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks,
                               n_threads=16)
    assert np.isfinite(want).all()
    for out_type in (OUT_F32, OUT_F16):
        got = _run(ctx, pc, n_swa, out_type=out_type)
        assert np.isfinite(got).all()
        _report(f"config 4 n_swa={n_swa} out={'f16' if out_type else 'f32'} (all 2048 rows)", got, want)


@pytest.mark.parametrize("n_swa", [0, 128])
def test_config4_full_size_spikes(ctx, n_swa):
    """Config 4 with config 5's stress pattern (1% of K rows scaled by 8), every output."""
    pc = _config4(0xC45, spike_frac=0.01)
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0,
                               n_swa, pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks,
                               n_threads=16)
    got = _run(ctx, pc, n_swa)
    assert np.isfinite(got).all()
    _report(f"config 4 spikes n_swa={n_swa} (all 2048 rows)", got, want)


@pytest.mark.parametrize("n_swa", [0, 128])
@pytest.mark.parametrize("n_q,pos0", [(2048, 1001), (2000, 1001)])
def test_full_size_unaligned_chunks(ctx, n_q, pos0, n_swa):
    """Config-4 sized chunks starting off a 32-key boundary: 2048 rows (512 work-groups, so the
    pair balance runs, with every tile's key range ragged) and 2000 rows (a last tile of 16 tokens);
    every output against the oracle."""
    pc = fx.prefill_case(0xC46 + n_q, n_q=n_q, pos0=pos0, pt=256)
    want = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0,
                               n_swa, pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks,
                               n_threads=16)
    got = _run(ctx, pc, n_swa, out_type=OUT_F16)
    assert np.isfinite(got).all()
    _report(f"prefill n_q={n_q} pos0={pos0} n_swa={n_swa} (all rows)", got, want)


def test_refusals(ctx):
    buf, bt = ctx.alloc(1 << 16), ctx.alloc(64)
    with pytest.raises(BadArgument):  # head_dim 128 is not the prefill kernel's
        ctx.attn_prefill(buf, buf, buf, buf, bt, None, 4, 0, 0, 8, 8, 128, 32, 0.1, KvType.F16)
    with pytest.raises(BadArgument):  # group 3
        ctx.attn_prefill(buf, buf, buf, buf, bt, None, 4, 0, 0, 6, 2, 64, 32, 0.1, KvType.F16)
    with pytest.raises(BadArgument):  # f32 KV
        ctx.attn_prefill(buf, buf, buf, buf, bt, None, 4, 0, 0, 8, 8, 64, 32, 0.1, KvType.F32)
    ctx.sync()
