"""The f16 codec on the GPU, bit-exact against the oracle (forward_pass_gpu.rs:75-150)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu


def _narrow(ctx, x):
    x = np.ascontiguousarray(x, np.float32)
    src, dst = ctx.upload(x), ctx.alloc(x.size * 2)
    ctx.quantize_f16(dst, src, x.size)
    return ctx.download(dst, np.uint16, x.size)


def test_round_trip_over_every_bit_pattern(ctx):
    vals = oracle.f16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    vals = vals[~np.isnan(vals)]
    bits = _narrow(ctx, vals)
    assert np.array_equal(bits, oracle.f32_to_f16(vals))
    assert np.array_equal(oracle.f16_to_f32(bits).view(np.uint32), vals.view(np.uint32))


def test_narrowing_hard_cases_and_nans(ctx):
    hard = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65520.0, 65519.996, 1e-8, -1e-8,
                     6e-8, 5.9604645e-8, 1.7881393e-7, np.finfo(np.float32).tiny, 1e30, -1e30,
                     np.inf, -np.inf], np.float32)
    rng = oracle.Rng(0xF167)
    x = np.concatenate([hard, rng.vec_unit(8192) * 4, rng.vec_unit(2048) * 1e-5,
                        np.array([0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x7FA00000, 0x00000001,
                                  0x80000001], np.uint32).view(np.float32)]).astype(np.float32)
    lo = np.arange(0, 0x7BFF, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (np.arange(0, 0x7BFF, dtype=np.uint32) + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([x, mid, -mid, np.nextafter(mid, np.float32(np.inf))])
    got = _narrow(ctx, x)
    want = oracle.f32_to_f16(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first input {x[bad[0]]!r}: gpu {got[bad[0]]:#06x} oracle {want[bad[0]]:#06x}"
