"""The calibration read (moearc_read_floor) that bench.py times beside the decode: every 64 KiB
piece's xor checksum against numpy, ragged tails, and its refusals, through the C ABI."""
from __future__ import annotations


import numpy as np
import pytest


pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 65536, 65552, 3 * 65536 + 4096, 64 << 20])
def test_checksums(ctx, nbytes):
    data = np.random.default_rng(nbytes).integers(0, 2 ** 32, nbytes // 4, dtype=np.uint32)
    src = ctx.upload(data)
    words = (nbytes + 65535) // 65536
    out = ctx.alloc(words * 4)
    ctx.read_floor(out, src, nbytes)
    got = ctx.download(out, np.uint32, words)
    padded = np.zeros(words * 16384, np.uint32)
    padded[: data.size] = data
    want = np.bitwise_xor.reduce(padded.reshape(words, 16384), axis=1)
    assert np.array_equal(got, want)


def test_refusals(ctx):
    lib, raw = ctx._lib, ctx.raw
    buf = ctx.alloc(1 << 16)
    out = ctx.alloc(64)
    assert lib.moearc_read_floor(raw, None, buf.ptr, 1024) == -1
    assert lib.moearc_read_floor(raw, out.ptr, None, 1024) == -1
    assert lib.moearc_read_floor(raw, out.ptr, buf.ptr, 0) == -2
    assert lib.moearc_read_floor(raw, out.ptr, buf.ptr, 1000) == -2      # not a multiple of 16
    assert lib.moearc_read_floor(raw, out.ptr, buf.ptr + 8, 1024) == -2  # misaligned source
    ctx.sync()
