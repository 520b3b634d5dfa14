"""Quantised matvec, batched matvec, the fused q/k/v projections and the bias add on the GPU,
through the C ABI, against the oracle (reference.rs:305-336 restated, pinned in
test_matvec_oracle.py).

Bar: the reference's own (kernels_gpu.rs:126-137): per row |gpu - oracle| <= 2 (cols/32 + 5) u
sum|w x|, u = 2^-24. Batched and fused launches are held to bit-identity with the single calls
they replace, as the reference holds its batched matvec (kernels_gpu.rs:483-533).
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import BadArgument, DeviceView, QuantType
from oracle import oracle

pytestmark = pytest.mark.gpu

ALL = [QuantType.F32, QuantType.F16, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q5_K,
       QuantType.Q6_K, QuantType.MXFP4]


def _run(ctx, ty, w, x, rows, cols, w_offset=0):
    buf = ctx.alloc(w.nbytes + w_offset + 64)
    wv = DeviceView(buf, w_offset, w.nbytes)
    ctx.upload_slice(wv, w)
    dx = ctx.upload(x)
    out = ctx.alloc(max(rows, 1) * 4)
    ctx.matvec_q(ty, out, wv, dx, rows, cols)
    return ctx.download(out, np.float32, rows)


def _check(label, got, ty, w, x, rows, cols):
    want, absum = oracle.matvec_q(int(ty), w, x, rows, cols, n_threads=16)
    tol = fx.matvec_tolerance(cols, absum)
    fin = np.isfinite(want)
    err = np.abs(got.astype(np.float64) - want)
    worst = float(np.max(np.where(fin, err / np.maximum(tol, 1e-300), 0.0))) if fin.any() else 0.0
    print(f"{label}: worst |gpu - oracle| / bound = {worst:.3f}", flush=True)
    assert np.all(err[fin] <= tol[fin]), f"{label}: over the bound"
    bad = ~fin
    if bad.any():  # rows the reference overflows: the same infinities / NaNs
        assert np.array_equal(np.isnan(got[bad]), np.isnan(want[bad]))
        assert np.array_equal(got[bad & ~np.isnan(want)], want[bad & ~np.isnan(want)])
    return want


@pytest.mark.parametrize("ty", ALL, ids=lambda t: t.name)
def test_matvec_matches_the_oracle_for_every_type(ctx, ty):
    # 37 rows x 1024 columns, drawn as kernels_gpu.rs:99-140 draws them
    rows, cols = 37, 1024
    w, x = fx.matvec_case(int(ty), rows, cols, 0x5EED ^ int(ty))
    want = _check(f"matvec {ty.name} {rows}x{cols}", _run(ctx, ty, w, x, rows, cols), ty, w, x, rows, cols)
    assert np.any(want != 0)


def test_f32_matvec_33x700(ctx):
    # kernels_gpu.rs:143-172: 700 columns, not a multiple of the 8-float piece
    rows, cols = 33, 700
    w, x = fx.matvec_case(0, rows, cols, 0x000A11CE)
    dw, dx, out = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.matvec_f32(out, dw, dx, rows, cols)
    _check("matvec_f32 33x700", ctx.download(out, np.float32, rows), QuantType.F32, w, x, rows, cols)


@pytest.mark.parametrize("ty,rows,cols", [
    (QuantType.Q8_0, 4096, 2880), (QuantType.Q8_0, 2880, 4096), (QuantType.F16, 4096, 2880),
    (QuantType.MXFP4, 4096, 2880), (QuantType.Q4_K, 4096, 2048), (QuantType.Q5_K, 512, 2048),
    (QuantType.Q6_K, 512, 2048), (QuantType.Q6_K, 2048, 4096)], ids=str)
def test_projection_shapes(ctx, ty, rows, cols):
    # gpt-oss attention (64 x 64 query, 8 x 64 KV, 2880 embedding) and Qwen3-30B-A3B (4096 / 2048)
    w, x = fx.matvec_case(int(ty), rows, cols, 0x7A11 + rows + int(ty))
    _check(f"matvec {ty.name} {rows}x{cols}", _run(ctx, ty, w, x, rows, cols), ty, w, x, rows, cols)


@pytest.mark.parametrize("ty,cols,offset", [
    (QuantType.Q8_0, 1024, 1), (QuantType.Q8_0, 2880, 2), (QuantType.Q6_K, 1024, 3),
    (QuantType.Q4_K, 512, 13), (QuantType.MXFP4, 1024, 5), (QuantType.F16, 1001, 7),
    (QuantType.F32, 7, 9), (QuantType.F16, 3, 1)], ids=str)
def test_any_weight_alignment_and_ragged_float_rows(ctx, ty, cols, offset):
    rows = 19
    w, x = fx.matvec_case(int(ty), rows, cols, 0xA1 + offset)
    _check(f"matvec {ty.name} cols={cols} +{offset}B", _run(ctx, ty, w, x, rows, cols, offset), ty, w, x,
           rows, cols)


@pytest.mark.parametrize("ty,cols", [(QuantType.Q8_0, 12288), (QuantType.F32, 5000),
                                     (QuantType.F16, 4100), (QuantType.Q4_K, 16384),
                                     (QuantType.MXFP4, 9216)], ids=str)
def test_rows_longer_than_one_slab(ctx, ty, cols):
    # more pieces than one pass of a wave holds: the row is walked in column slabs (and the widest
    # read their activation from global memory instead of LDS)
    rows = 45
    w, x = fx.matvec_case(int(ty), rows, cols, 0x51AB + cols)
    _check(f"matvec {ty.name} 45x{cols}", _run(ctx, ty, w, x, rows, cols), ty, w, x, rows, cols)


def test_mxfp4_extreme_exponents(ctx):
    # E8M0 0 and 1 give subnormal scales; from 253 up the reference's per-element products
    # overflow f32, and the kernel must overflow the same way
    rows, cols = 8, 256
    w, x = fx.matvec_case(39, rows, cols, 0xE8E0)
    blocks = w.reshape(-1, 17)
    blocks[:, 0] = np.array([0, 1, 2, 252, 253, 254, 255, 127], np.uint8)[np.arange(blocks.shape[0]) % 8]
    _check("matvec MXFP4 extreme exponents", _run(ctx, QuantType.MXFP4, w, x, rows, cols),
           QuantType.MXFP4, w, x, rows, cols)


@pytest.mark.parametrize("ty", [QuantType.Q8_0, QuantType.Q4_K, QuantType.Q5_K, QuantType.Q6_K],
                         ids=lambda t: t.name)
def test_batched_is_bit_identical_to_single_calls(ctx, ty):
    # kernels_gpu.rs:494-533
    rows, cols, mats = 37, 1024, 5
    x = fx.synth.unit(0x0BA7C4ED ^ int(ty), cols)
    dx = ctx.upload(x)
    ws, want = [], []
    for m in range(mats):
        w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0xB0 + 7 * m + int(ty))
        dw = ctx.upload(w)
        one = ctx.alloc(rows * 4)
        ctx.matvec_q(ty, one, dw, dx, rows, cols)
        want.append(ctx.download(one, np.float32, rows))
        ws.append(dw)
    out = ctx.alloc(mats * rows * 4)
    ctx.matvec_q_batched(ty, out, ws, dx, 0, rows, cols)
    got = ctx.download(out, np.float32, mats * rows)
    assert np.array_equal(got, np.concatenate(want)), "batching changed the answer"
    assert np.any(got != 0)


def test_batched_strided_activation(ctx):
    # kernels_gpu.rs:536-577: matrix m reads x + m * cols
    ty, rows, cols, mats = QuantType.Q4_K, 20, 512, 4
    xs = fx.synth.unit(0x05731DED, mats * cols)
    dxs = ctx.upload(xs)
    ws, want = [], []
    for m in range(mats):
        w, _ = fx.synth_blocks(int(ty), rows * cols // 256, 0x5700 + m)
        ws.append(ctx.upload(w))
        want.append(_run(ctx, ty, w, xs[m * cols:(m + 1) * cols], rows, cols))
    out = ctx.alloc(mats * rows * 4)
    ctx.matvec_q_batched(ty, out, ws, dxs, cols, rows, cols)
    assert np.array_equal(ctx.download(out, np.float32, mats * rows), np.concatenate(want))


def test_batched_refusals(ctx):
    # kernels_gpu.rs:580-593: more matrices than one launch carries is refused, not truncated
    ty, cols = QuantType.Q4_K, 256
    dw, dx, out = ctx.alloc(144), ctx.alloc(cols * 4), ctx.alloc(33 * 4)
    with pytest.raises(BadArgument):
        ctx.matvec_q_batched(ty, out, [dw] * 33, dx, 0, 1, cols)
    ctx.matvec_q_batched(ty, out, [], dx, 0, 1, cols)  # nothing to do
    ctx.sync()


@pytest.mark.parametrize("types", [(8, 8, 8), (12, 12, 14), (39, 1, 8)], ids=str)
def test_attn_qkv_is_bit_identical_to_matvec_then_add(ctx, types):
    # moe.rs:1942-1959: three matvecs, then the biases added in place
    cols = 2048
    rows = (512, 128, 128)
    x = fx.synth.unit(0x9C5, cols)
    dx = ctx.upload(x)
    outs, ws, biases, want = [], [], [], []
    for i, (t, r) in enumerate(zip(types, rows)):
        w, _ = fx.synth_blocks(t, r * cols // fx.QT_BLOCK[t][1], 0x9C50 + i)
        dw = ctx.upload(w)
        b = ctx.upload(fx.synth.unit(0x9C60 + i, r)) if i != 1 else None  # k without a bias
        one = ctx.alloc(r * 4)
        ctx.matvec_q(t, one, dw, dx, r, cols)
        if b is not None:
            ctx.add(one, one, b, r)
        want.append(ctx.download(one, np.float32, r))
        outs.append(ctx.alloc(r * 4))
        ws.append(dw)
        biases.append(b)
    ctx.attn_qkv(types, outs, ws, biases, rows, dx, cols)
    for i, r in enumerate(rows):
        assert np.array_equal(ctx.download(outs[i], np.float32, r), want[i]), f"projection {i}"


def test_add_is_exact_and_may_alias(ctx):
    n = 10000
    a, b = fx.synth.unit(1, n), fx.synth.unit(2, n)
    da, db, out = ctx.upload(a), ctx.upload(b), ctx.alloc(n * 4)
    ctx.add(out, da, db, n)
    assert np.array_equal(ctx.download(out, np.float32, n), a + b)
    ctx.add(da, da, db, n)  # out aliasing the left operand, as the engine calls it
    assert np.array_equal(ctx.download(da, np.float32, n), a + b)


def test_matvec_refusals_and_empty_shapes(ctx):
    dw, dx, out = ctx.alloc(1 << 16), ctx.alloc(4096), ctx.alloc(256)
    lib = ctx._lib
    assert lib.moearc_matvec_q(ctx.raw, 12, out.ptr, dw.ptr, dx.ptr, 4, 300) == -2  # ragged Q4_K
    assert lib.moearc_matvec_q(ctx.raw, 2, out.ptr, dw.ptr, dx.ptr, 4, 256) == -2   # Q4_0: unknown
    assert lib.moearc_matvec_q(ctx.raw, 8, None, dw.ptr, dx.ptr, 4, 256) == -1
    assert lib.moearc_matvec_q(ctx.raw, 8, out.ptr, dw.ptr, dx.ptr, 0, 256) == 0   # no rows
    with pytest.raises(BadArgument):
        ctx.matvec_q(QuantType.Q4_K, out, dw, dx, 4, 300)
    # zero columns: every row's sum is empty
    ctx.upload_slice(out, np.full(8, 7.0, np.float32))
    ctx.matvec_q(QuantType.Q8_0, out, dw, dx, 8, 0)
    assert np.array_equal(ctx.download(out, np.float32, 8), np.zeros(8, np.float32))
    ctx.sync()


@pytest.mark.parametrize("ty,n_tok,rows,cols", [
    (QuantType.Q8_0, 37, 200, 1024), (QuantType.Q8_0, 130, 512, 2880), (QuantType.F16, 67, 96, 512),
    (QuantType.Q8_0, 2, 4096, 2880), (QuantType.F16, 129, 2880, 4096),
    # enough work-groups for the 32-rows-per-wave kernels
    (QuantType.Q8_0, 512, 8192, 256), (QuantType.F16, 256, 16384, 128),
    # the 128 x 128-tile kernels (Q8_0 and F16 from 64 tokens): ragged tiles, k-block counts around
    # the three-deep pipeline and its six-block unroll (Q8_0 there only with an even count: its
    # weights travel in pairs of blocks; odd counts, as 224 and 96 columns, take the 16x16 kernels)
    (QuantType.Q8_0, 200, 300, 64), (QuantType.Q8_0, 64, 128, 224), (QuantType.F16, 100, 200, 32),
    (QuantType.Q8_0, 300, 129, 96), (QuantType.F16, 190, 257, 160),
    (QuantType.Q8_0, 64, 128, 128), (QuantType.Q8_0, 100, 200, 192), (QuantType.Q8_0, 70, 130, 320),
    (QuantType.Q8_0, 96, 160, 448), (QuantType.F16, 65, 136, 224), (QuantType.F16, 80, 128, 352),
    # K-quants (sub-block scales and mins) and MXFP4, both launch shapes
    (QuantType.Q4_K, 37, 200, 1024), (QuantType.Q4_K, 512, 8192, 256), (QuantType.Q5_K, 67, 96, 2048),
    (QuantType.Q5_K, 512, 8192, 256), (QuantType.MXFP4, 37, 200, 1024), (QuantType.MXFP4, 512, 8192, 96),
    (QuantType.Q6_K, 37, 200, 1024), (QuantType.Q6_K, 512, 8192, 256),
    # Q4_K on the 128 x 128 tiles (from 64 tokens): ragged tiles, super-block counts around the
    # three-deep pipeline and its six-block unroll, and a split launch (slices on super-blocks)
    (QuantType.Q4_K, 64, 128, 256), (QuantType.Q4_K, 200, 300, 512), (QuantType.Q4_K, 130, 257, 768),
    (QuantType.Q4_K, 96, 160, 1280), (QuantType.Q4_K, 128, 512, 2048),
    (QuantType.Q5_K, 64, 128, 256), (QuantType.Q5_K, 200, 300, 512), (QuantType.Q5_K, 130, 257, 1280),
    (QuantType.Q5_K, 128, 512, 2048),
    (QuantType.Q6_K, 64, 128, 256), (QuantType.Q6_K, 200, 300, 512), (QuantType.Q6_K, 130, 257, 1280),
    (QuantType.Q6_K, 128, 512, 2048),
    # MXFP4 on the 128 x 128 tiles (pairs of 17-byte blocks; odd block counts take the 16x16 kernels)
    (QuantType.MXFP4, 64, 128, 64), (QuantType.MXFP4, 200, 300, 192), (QuantType.MXFP4, 130, 257, 2880),
    (QuantType.MXFP4, 96, 160, 96), (QuantType.MXFP4, 128, 512, 2048),
    # grids of at most one work-group per CU split the reduction into k-slices (also above: every
    # case with 16 or more k-blocks and a small grid, K-quant slices on super-block bounds, a ragged
    # last slice) -- here a 128-token chunk's output projection at gpt-oss shapes (11 slices)
    (QuantType.Q8_0, 128, 2880, 4096)],
    ids=str)
def test_chunk_matmul_meets_the_matvec_bound(ctx, ty, n_tok, rows, cols):
    # the MFMA product of a chunk, token by token against the oracle's matvec. The bound is the
    # reference's model with the MFMA's 32-wide block sums added: each block sum inside the matrix
    # core may take up to 32 roundings of its terms, where the reference's lane sums take n/32
    # (this matters only for short rows: at 96 columns the two bounds are 74 u and 16 u)
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0x3A3 + rows)
    x = fx.synth.unit(0x3A4 + cols, n_tok * cols).reshape(n_tok, cols)
    bias = fx.synth.unit(0x3A5, rows)
    y = ctx.alloc(n_tok * rows * 4)
    ctx.matmul_q(ty, y, ctx.upload(w), ctx.upload(x), ctx.upload(bias), n_tok, rows, cols)
    got = ctx.download(y, np.float32, (n_tok, rows)).astype(np.float64)
    worst = 0.0
    for t in range(n_tok):
        want, absum = oracle.matvec_q(int(ty), w, x[t], rows, cols, n_threads=16)
        err = np.abs(got[t] - (want.astype(np.float64) + bias))
        # + the f32 bias add: half an ulp of the result, at most 2^-23 of it
        tol = fx.matvec_tolerance(cols, absum) + 2.0 * 32 * 2.0 ** -24 * absum + 2.0 ** -23 * np.abs(want + bias)
        worst = max(worst, float(np.max(err / tol)))
    print(f"matmul {ty.name} {n_tok}x{rows}x{cols}: worst / bound = {worst:.3f}", flush=True)
    assert worst <= 1.0


def _matmul_with(env, ty, w, x, bias, n_tok, rows, cols):
    """The chunk product in a fresh context created under the given environment (the launch-shape
    switches are read at context creation)."""
    import os
    from moearc_amd import Context
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        with Context() as c:
            y = c.alloc(n_tok * rows * 4)
            c.matmul_q(ty, y, c.upload(w), c.upload(x), c.upload(bias), n_tok, rows, cols)
            return c.download(y, np.float32, (n_tok, rows))
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _within_bound(label, got, ty, w, x, bias, rows, cols, tokens):
    worst = 0.0
    for t in tokens:
        want, absum = oracle.matvec_q(int(ty), w, x[t], rows, cols, n_threads=16)
        err = np.abs(got[t].astype(np.float64) - (want.astype(np.float64) + bias))
        tol = fx.matvec_tolerance(cols, absum) + 2.0 * 32 * 2.0 ** -24 * absum + 2.0 ** -23 * np.abs(want + bias)
        worst = max(worst, float(np.max(err / tol)))
    print(f"{label}: worst / bound = {worst:.3f}", flush=True)
    assert worst <= 1.0


@pytest.mark.parametrize("ty,n_tok,rows,cols", [
    # F16, Q8_0 and MXFP4 on eight-wave work-groups of 128 tokens x 256 rows: ragged row and token tiles,
    # k-block counts around the three-deep pipeline and its six-block unroll, a 128-token chunk's
    # output projection at gpt-oss shapes
    (QuantType.Q8_0, 200, 300, 64), (QuantType.Q8_0, 130, 513, 320), (QuantType.Q8_0, 64, 256, 448),
    (QuantType.Q8_0, 100, 260, 192), (QuantType.F16, 100, 257, 32), (QuantType.F16, 190, 600, 160),
    (QuantType.F16, 65, 136, 352), (QuantType.Q8_0, 128, 2880, 4096),
    # MXFP4 pairs of 17-byte blocks
    (QuantType.MXFP4, 200, 300, 192), (QuantType.MXFP4, 130, 513, 2880), (QuantType.MXFP4, 64, 260, 64)],
    ids=str)
def test_chunk_matmul_wide_tiles(ty, n_tok, rows, cols):
    # forced on (MOEARC_MM_WIDE=1) against forced off: without split-K both accumulate every output
    # in the same k order, so they must agree bit for bit; with the split-K the wide form's launch
    # picks, the oracle's bound
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0x3B3 + rows)
    x = fx.synth.unit(0x3B4 + cols, n_tok * cols).reshape(n_tok, cols)
    bias = fx.synth.unit(0x3B5, rows)
    narrow = _matmul_with({"MOEARC_MM_WIDE": "0", "MOEARC_MM_SPLIT_WG": "0"}, ty, w, x, bias, n_tok, rows, cols)
    wide = _matmul_with({"MOEARC_MM_WIDE": "1", "MOEARC_MM_SPLIT_WG": "0"}, ty, w, x, bias, n_tok, rows, cols)
    assert np.array_equal(wide.view(np.uint32), narrow.view(np.uint32))
    split = _matmul_with({"MOEARC_MM_WIDE": "1"}, ty, w, x, bias, n_tok, rows, cols)
    _within_bound(f"wide {ty.name} {n_tok}x{rows}x{cols}", split, ty, w, x, bias, rows, cols, range(n_tok))


@pytest.mark.parametrize("ty,rows,cols", [
    # gpt-oss's attn_q over a config-4 chunk (Q8_0 and F16 take the wide tiles there by default)
    (QuantType.Q8_0, 4096, 2880), (QuantType.F16, 4096, 2880), (QuantType.MXFP4, 4096, 2880),
    # Qwen3-30B-A3B's attn_q (K-quant rows of whole super-blocks)
    (QuantType.Q4_K, 4096, 2048), (QuantType.Q5_K, 4096, 2048), (QuantType.Q6_K, 4096, 2048)], ids=str)
def test_chunk_matmul_full_size_attn_q(ctx, ty, rows, cols):
    # a 2048-token chunk: every row of 40 tokens spread over all 16 token tiles
    n_tok = 2048
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0x3C3)
    x = fx.synth.unit(0x3C4, n_tok * cols).reshape(n_tok, cols)
    bias = fx.synth.unit(0x3C5, rows)
    y = ctx.alloc(n_tok * rows * 4)
    ctx.matmul_q(ty, y, ctx.upload(w), ctx.upload(x), ctx.upload(bias), n_tok, rows, cols)
    got = ctx.download(y, np.float32, (n_tok, rows))
    assert np.all(np.isfinite(got))
    tokens = sorted(set(range(0, n_tok, 53)) | {1, 127, 128, n_tok - 1})
    _within_bound(f"matmul {ty.name} {n_tok}x{rows}x{cols}", got, ty, w, x, bias, rows, cols, tokens)


def test_chunk_matmul_activation_alignment(ctx):
    # the activation's f16 split runs eight elements per thread from a 16-byte aligned x and one
    # element per thread otherwise: the same arithmetic, so the products agree to the bit
    ty, n_tok, rows, cols = QuantType.Q8_0, 96, 200, 320
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0x7A1)
    x = fx.synth.unit(0x7A2, n_tok * cols).reshape(n_tok, cols)
    dw = ctx.upload(w)
    outs = []
    for off in (0, 4):
        buf = ctx.alloc(x.nbytes + 16)
        xv = DeviceView(buf, off, x.nbytes)
        ctx.upload_slice(xv, x)
        y = ctx.alloc(n_tok * rows * 4)
        ctx.matmul_q(ty, y, dw, xv, None, n_tok, rows, cols)
        outs.append(ctx.download(y, np.float32, (n_tok, rows)))
    assert np.array_equal(outs[0], outs[1])
    assert np.any(outs[0] != 0)


@pytest.mark.parametrize("bias", [True, False], ids=["bias", "no_bias"])
def test_chunk_matmul_reduction_alignment(ctx, bias):
    # a split product's k-slice sums are added four elements per lane when y, the bias and every
    # row allow 16-byte accesses and one element per lane otherwise (y one float off here): the
    # same additions in the same order, so the outputs agree to the bit
    ty, n_tok, rows, cols = QuantType.Q8_0, 128, 2880, 4096  # a 128-token chunk's attn_output: 11 slices
    w, _ = fx.synth_blocks(int(ty), rows * cols // ty.block_elems, 0x7B1)
    x = fx.synth.unit(0x7B2, n_tok * cols).reshape(n_tok, cols)
    dw, dx = ctx.upload(w), ctx.upload(x)
    db = ctx.upload(fx.synth.unit(0x7B3, rows)) if bias else None
    outs = []
    for off in (0, 4):
        buf = ctx.alloc(n_tok * rows * 4 + 16)
        y = DeviceView(buf, off, n_tok * rows * 4)
        ctx.matmul_q(ty, y, dw, dx, db, n_tok, rows, cols)
        outs.append(ctx.download(y, np.float32, (n_tok, rows)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.all(np.isfinite(outs[0])) and np.any(outs[0] != 0)


def test_chunk_matmul_refusals(ctx):
    lib = ctx._lib
    buf = ctx.alloc(1 << 16)
    assert lib.moearc_matmul_q(ctx.raw, 0, buf.ptr, buf.ptr, buf.ptr, None, 4, 4, 256) == -2  # F32
    assert lib.moearc_matmul_q(ctx.raw, 12, buf.ptr, buf.ptr, buf.ptr, None, 4, 4, 128) == -2  # Q4_K 128
    assert lib.moearc_matmul_q(ctx.raw, 8, buf.ptr, buf.ptr, buf.ptr, None, 4, 4, 48) == -2   # not 32k
    assert lib.moearc_matmul_q(ctx.raw, 8, buf.ptr, buf.ptr + 1, buf.ptr, None, 4, 4, 64) == -2  # odd W
    assert lib.moearc_matmul_q(ctx.raw, 8, buf.ptr, buf.ptr, buf.ptr, None, 0, 4, 64) == 0


@pytest.mark.parametrize("ty", [QuantType.Q8_0, QuantType.MXFP4, QuantType.F16], ids=lambda t: t.name)
def test_attn_out_is_bit_identical_to_matvec_then_two_adds(ctx, ty):
    # moe.rs:2063-2071: proj = W attn; proj += bias; h += proj
    rows, cols = 2880, 4096
    w, attn = fx.matvec_case(int(ty), rows, cols, 0xA770 + int(ty))
    bias, h = fx.synth.unit(0xA771, rows), fx.synth.normal(0xA772, rows)
    dw, da, db = ctx.upload(w), ctx.upload(attn), ctx.upload(bias)
    proj, dh = ctx.alloc(rows * 4), ctx.upload(h)
    ctx.matvec_q(ty, proj, dw, da, rows, cols)
    ctx.add(proj, proj, db, rows)
    ctx.add(dh, dh, proj, rows)
    want = ctx.download(dh, np.float32, rows)
    dh2 = ctx.upload(h)
    ctx.attn_out(ty, dh2, dw, db, da, rows, cols)
    assert np.array_equal(ctx.download(dh2, np.float32, rows), want)
