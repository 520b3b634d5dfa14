"""Repeatability of the full-size hot paths on the GPU: every kernel here is deterministic (fixed
reduction orders, no atomics), so the same call enqueued several times back to back must give
bit-identical outputs. A race -- a copy read before it lands, a store that picks up a register's
next value, LDS reused too early -- shows up here as calls that disagree, at the sizes and loads
where such races happen, without needing the oracle's tolerance to catch it.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import OUT_F16, OUT_F32, KvType, QuantType

pytestmark = pytest.mark.gpu

REPEATS = 3


def _same(label, outs):
    bits = [o.view(np.uint32) for o in outs]
    diff = [int(np.count_nonzero(bits[0] != b)) for b in bits[1:]]
    print(f"{label}: {REPEATS} calls, differing words against the first: {diff}", flush=True)
    assert all(d == 0 for d in diff), label
    assert np.all(np.isfinite(outs[0]))


def test_decode_config2_repeats(ctx):
    # B=1, 32K keys, f16 KV through a random page permutation, sinks
    c = fx.north_star_case(0xD2, 32768, pt=256)
    dk, dv, dq = ctx.upload(c.k_raw), ctx.upload(c.v_raw), ctx.upload(c.q.astype(np.float32))
    dbt, ds = ctx.upload(np.asarray(c.bt, np.uint32)), ctx.upload(c.sinks.astype(np.float32))
    outs = [ctx.alloc(c.H * c.D * 4) for _ in range(REPEATS)]
    for o in outs:  # enqueued back to back, read after
        ctx.attn_decode_ext(o, dq, dk, dv, dbt, ds, c.H, c.G, c.D, 0, c.n_kv, c.pt, float(c.scale),
                            KvType(c.kv))
    _same("decode config 2", [ctx.download(o, np.float32, c.H * c.D) for o in outs])


@pytest.mark.parametrize("n_swa", [0, 128])
@pytest.mark.parametrize("out_f16", [False, True], ids=["f32_out", "f16_out"])
def test_prefill_config4_repeats(ctx, n_swa, out_f16):
    # 2048 new tokens after 2048 cached, both layer types, both output types
    pc = fx.prefill_case(0xD4, n_q=2048, pos0=2048, pt=256)
    dk, dv, dbt = ctx.upload(pc.k_raw), ctx.upload(pc.v_raw), ctx.upload(pc.bt)
    ds, dq = ctx.upload(pc.sinks), ctx.upload(np.ascontiguousarray(pc.qp).view(np.uint16))
    nb = 2 if out_f16 else 4
    outs = [ctx.alloc(pc.n_q * pc.H * pc.D * nb) for _ in range(REPEATS)]
    for o in outs:
        ctx.attn_prefill(o, dq, dk, dv, dbt, ds, pc.n_q, pc.pos0, n_swa, pc.H, pc.G, pc.D, pc.pt,
                         float(pc.scale), KvType.F16, out_type=OUT_F16 if out_f16 else OUT_F32)
    dt = np.float16 if out_f16 else np.float32
    got = [ctx.download(o, dt, (pc.n_q, pc.H, pc.D)) for o in outs]
    _same(f"prefill config 4 n_swa={n_swa} {'f16' if out_f16 else 'f32'} out",
          [g.astype(np.float32) for g in got])


@pytest.mark.parametrize("ty,rows,cols", [
    (QuantType.Q8_0, 4096, 2880), (QuantType.F16, 4096, 2880), (QuantType.MXFP4, 4096, 2880),
    (QuantType.Q4_K, 4096, 2048), (QuantType.Q6_K, 4096, 2048)], ids=str)
def test_chunk_matmul_2048_tokens_repeats(ctx, ty, rows, cols):
    # the activation split and the product over a 2048-token chunk, called back to back
    n_tok = 2048
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0xD5)
    x = fx.synth.unit(0xD6, n_tok * cols).reshape(n_tok, cols)
    bias = fx.synth.unit(0xD7, rows)
    dw, dx, db = ctx.upload(w), ctx.upload(x), ctx.upload(bias)
    outs = [ctx.alloc(n_tok * rows * 4) for _ in range(REPEATS)]
    for o in outs:
        ctx.matmul_q(ty, o, dw, dx, db, n_tok, rows, cols)
    _same(f"matmul {ty.name} {n_tok}x{rows}x{cols}", [ctx.download(o, np.float32, (n_tok, rows)) for o in outs])
