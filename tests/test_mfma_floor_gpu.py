"""The matrix-core calibration (moearc_mfma_floor) that bench.py times beside the prefill: every
wave's accumulator sum against a float64 recomputation from its operands, and its refusals, through
the C ABI.

Wave w's operands: A_k, B_k (k < 4) are the 1 KiB blocks 8 KiB * w + 1 KiB * k and + 1 KiB * (4 + k)
of src, lane l holding f16 elements 8 l .. 8 l + 7 of each -- in v_mfma_f32_32x32x16_f16's layout
A[l % 32][8 (l // 32) + i] and B[8 (l // 32) + i][l % 32]. Every chain meets every (A_k, B_k)
twice per four rounds, so the sum of all accumulators is 2 iters sum_k sum_kk (sum_m A_k[m][kk])
(sum_n B_k[kk][n])."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _expected(src, n_wgs, iters):
    h = src.view(np.float16).astype(np.float64).reshape(n_wgs * 4, 8, 64, 8)  # wave, block, lane, i
    out, mag = [], []
    for w in range(n_wgs * 4):
        tot = tmag = 0.0
        for k in range(4):
            a, b = h[w, k], h[w, 4 + k]  # [lane][i]
            for g in range(2):  # kk = 8 g + i: lanes 32 g .. 32 g + 31
                ca = a[32 * g: 32 * g + 32].sum(axis=0)
                rb = b[32 * g: 32 * g + 32].sum(axis=0)
                tot += float(np.dot(ca, rb))
                tmag += float(np.dot(np.abs(a[32 * g: 32 * g + 32]).sum(axis=0),
                                     np.abs(b[32 * g: 32 * g + 32]).sum(axis=0)))
        out.append(2.0 * iters * tot)
        mag.append(2.0 * iters * tmag)
    return np.array(out), np.array(mag)


@pytest.mark.parametrize("n_wgs,iters", [(1, 4), (4, 8), (512, 64)])
def test_checksums(ctx, n_wgs, iters):
    rng = np.random.default_rng(n_wgs * 1000 + iters)
    src = rng.standard_normal(n_wgs * 16384).astype(np.float16)
    dsrc = ctx.upload(src)
    dout = ctx.alloc(n_wgs * 4 * 4)
    ctx.mfma_floor(dout, dsrc, n_wgs, iters)
    got = ctx.download(dout, np.float32, n_wgs * 4).astype(np.float64)
    want, mag = _expected(src, n_wgs, iters)
    err = np.max(np.abs(got - want) / mag)
    print(f"mfma_floor n_wgs={n_wgs} iters={iters}: max |gpu - f64| / magnitude = {err:.2e}", flush=True)
    # f32 rounding of at most ~4,300 accumulations, each bounded by the magnitude: < 3e-4
    assert err < 1e-3


def test_refusals(ctx):
    lib, raw = ctx._lib, ctx.raw
    buf = ctx.alloc(1 << 15)
    out = ctx.alloc(64)
    assert lib.moearc_mfma_floor(raw, None, buf.ptr, 1, 4) == -1
    assert lib.moearc_mfma_floor(raw, out.ptr, None, 1, 4) == -1
    assert lib.moearc_mfma_floor(raw, out.ptr, buf.ptr, 0, 4) == -2
    assert lib.moearc_mfma_floor(raw, out.ptr, buf.ptr, 1, 0) == -2
    assert lib.moearc_mfma_floor(raw, out.ptr, buf.ptr, 1, 6) == -2       # not a multiple of 4
    assert lib.moearc_mfma_floor(raw, out.ptr, buf.ptr + 8, 1, 4) == -2   # misaligned source
    ctx.sync()
