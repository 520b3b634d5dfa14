"""The oracle's GGUF block decoders and matvec, pinned on the CPU.

The decoders restate reference.rs:168-303, itself a restatement of ggml's dequantize_row_* (ggml is
a dependency the reference does not vendor; its golden dump, gguf_crosscheck.rs, needs a model
file this image does not have). They are pinned here by what the formats fix, independently of
the decoder code:
  * encoders written from the packing side of the formats (ggml's quantize_row_*_ref layouts:
    where each nibble, high bit, 6-bit scale and min lands) round-trip through the decoder, so a
    misread bit position or element order fails;
  * known answers: Q8_0 with d = 1 is the int8 payload; MXFP4 elements are the OCP E2M1 code
    points {0, .5, 1, 1.5, 2, 3, 4, 6} times 2^(e-127) (the reference's doubled table and halved
    scale must agree with that), with the reference's subnormal and top exponents;
  * the f64 matvec against numpy's float64 product of the decoded matrix.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from oracle import oracle

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4 = 0, 1, 8, 12, 13, 14, 39
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def f16b(x) -> bytes:
    return np.float16(x).tobytes()


def pack_scales_k4(sc, m) -> np.ndarray:
    """The 12 scale bytes of a Q4_K/Q5_K block from 8 six-bit scales and mins: sub-blocks 0-3 in
    the low six bits of bytes j and j+4; 4-7 as low nibbles in bytes j+4 (scale) / high nibbles
    (min) and their top two bits in the top bits of bytes j-4 (scale) and j (min)."""
    q = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            q[j] = sc[j]
            q[j + 4] = m[j]
        else:
            q[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            q[j - 4] |= (sc[j] >> 4) << 6
            q[j] |= (m[j] >> 4) << 6
    return q


def encode_q4_k(d, dmin, sc, m, L) -> bytes:
    qs = np.zeros(128, np.uint8)
    for g in range(4):  # 64 elements: the low nibbles of 32 bytes, then their high nibbles
        qs[32 * g:32 * g + 32] = L[64 * g:64 * g + 32] | (L[64 * g + 32:64 * g + 64] << 4)
    return f16b(d) + f16b(dmin) + pack_scales_k4(sc, m).tobytes() + qs.tobytes()


def encode_q5_k(d, dmin, sc, m, L) -> bytes:
    qh = np.zeros(32, np.uint8)
    qs = np.zeros(128, np.uint8)
    for g in range(4):
        lo, hi = L[64 * g:64 * g + 32], L[64 * g + 32:64 * g + 64]
        qh |= ((lo >> 4) << (2 * g)).astype(np.uint8) | ((hi >> 4) << (2 * g + 1)).astype(np.uint8)
        qs[32 * g:32 * g + 32] = (lo & 0xF) | ((hi & 0xF) << 4)
    return f16b(d) + f16b(dmin) + pack_scales_k4(sc, m).tobytes() + qh.tobytes() + qs.tobytes()


def encode_q6_k(d, sc, L) -> bytes:
    """L in 0..63 (value L - 32); sc: 16 int8 scales, one per 16 elements."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(2):
        b = L[128 * n:128 * n + 128]
        for l in range(32):
            q1, q2, q3, q4 = b[l], b[l + 32], b[l + 64], b[l + 96]
            ql[64 * n + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * n + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return ql.tobytes() + qh.tobytes() + np.asarray(sc, np.int8).tobytes() + f16b(d)


def test_block_sizes_are_the_formats():
    for ty, (bb, be) in fx.QT_BLOCK.items():
        assert (oracle.block_bytes(ty), oracle.block_elems(ty)) == (bb, be)
    assert oracle.block_bytes(2) == 0  # Q4_0: not a format this path expands


def test_q8_0_is_the_payload_times_d():
    q = np.arange(-128, 128, dtype=np.int32).astype(np.int8)
    for d in (1.0, 0.5, -2.0):
        blocks = b"".join(f16b(d) + q[32 * i:32 * i + 32].tobytes() for i in range(8))
        y = oracle.dequant(Q8_0, blocks, 8)
        assert np.array_equal(y, q.astype(np.float32) * np.float32(d))


def test_mxfp4_is_e2m1_times_two_to_the_e_minus_127():
    rng = np.random.default_rng(1)
    for e in (1, 2, 100, 127, 128, 200, 252):
        payload = rng.integers(0, 256, 16, dtype=np.uint8)
        y = oracle.dequant(MXFP4, bytes([e]) + payload.tobytes(), 1).astype(np.float64)
        want = np.concatenate([E2M1[payload & 0xF], E2M1[payload >> 4]]) * 2.0 ** (e - 127)
        assert np.array_equal(y, want), e
    # every byte value: low nibble -> element j, high nibble -> element j + 16
    for base in range(0, 256, 16):
        payload = np.arange(base, base + 16, dtype=np.uint8)
        y = oracle.dequant(MXFP4, bytes([127]) + payload.tobytes(), 1).astype(np.float64)
        assert np.array_equal(y[:16], E2M1[payload & 0xF])
        assert np.array_equal(y[16:], E2M1[payload >> 4])


def test_e8m0_half_at_its_ends():
    assert oracle.e8m0_half(0) == 2.0 ** -128 and oracle.e8m0_half(1) == 2.0 ** -127
    assert oracle.e8m0_half(2) == 2.0 ** -126 and oracle.e8m0_half(255) == 2.0 ** 127


@pytest.mark.parametrize("ty", [Q4_K, Q5_K])
def test_k4_formats_round_trip_their_encoder(ty):
    rng = np.random.default_rng(ty)
    top = 16 if ty == Q4_K else 32
    for _ in range(20):
        d, dmin = np.float32(rng.uniform(0.01, 2)), np.float32(rng.uniform(0.01, 2))
        d, dmin = np.float32(np.float16(d)), np.float32(np.float16(dmin))
        sc = rng.integers(0, 64, 8, dtype=np.uint8)
        m = rng.integers(0, 64, 8, dtype=np.uint8)
        L = rng.integers(0, top, 256, dtype=np.uint8)
        blk = (encode_q4_k if ty == Q4_K else encode_q5_k)(d, dmin, sc, m, L)
        y = oracle.dequant(ty, blk, 1)
        sub = np.arange(256) // 32
        d1 = (d * sc.astype(np.float32))[sub]
        m1 = (dmin * m.astype(np.float32))[sub]
        assert np.array_equal(y, d1 * L.astype(np.float32) - m1)


def test_q6_k_round_trips_its_encoder():
    rng = np.random.default_rng(6)
    for _ in range(20):
        d = np.float32(np.float16(rng.uniform(0.001, 1)))
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        L = rng.integers(0, 64, 256, dtype=np.uint8)
        y = oracle.dequant(Q6_K, encode_q6_k(d, sc, L), 1)
        ds = (d * sc.astype(np.float32))[np.arange(256) // 16]
        assert np.array_equal(y, ds * (L.astype(np.float32) - np.float32(32)))


def test_f16_and_f32_blocks_are_the_values():
    v = np.array([1.5, -2.25, 65504.0, 2.0 ** -24], np.float32)
    assert np.array_equal(oracle.dequant(F16, v.astype(np.float16).tobytes(), 4), v)
    assert np.array_equal(oracle.dequant(F32, v.tobytes(), 4), v)


@pytest.mark.parametrize("ty", [F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, MXFP4])
def test_matvec_is_the_float64_product_of_the_decoded_matrix(ty):
    rows, cols = 37, 1024
    w, x = fx.matvec_case(ty, rows, cols, 0x5EED ^ ty)
    got, absum = oracle.matvec_q(ty, w, x, rows, cols)
    nb = cols // fx.QT_BLOCK[ty][1]
    dense = oracle.dequant(ty, w, rows * nb).reshape(rows, cols).astype(np.float64)
    want = dense @ x.astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-30)
    assert np.allclose(absum, np.abs(dense * x.astype(np.float64)).sum(axis=1), rtol=1e-12)
    assert np.any(want != 0)


def test_unknown_types_and_ragged_rows_are_refused():
    with pytest.raises(oracle.OracleRefusal):
        oracle.dequant(2, b"\0" * 18, 1)
    with pytest.raises(oracle.OracleRefusal):
        oracle.matvec_q(Q4_K, np.zeros(144 * 4, np.uint8), np.zeros(300, np.float32), 4, 300)


def test_f16_hi_lo_split_carries_f32_to_2_pow_minus_22():
    # The chunk product's precision model (moearc_split_f16_k): hi = f16(x), lo = f16(x - hi)
    # leaves |x - hi - lo| <= 2^-22 |x| for normal values, and at most half of f16's smallest
    # subnormal (2^-25) below; every f32 below 65504 in magnitude splits without overflow.
    rng = np.random.default_rng(22)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32),
                        (rng.standard_normal(50000) * 1e3).astype(np.float32),
                        (rng.standard_normal(50000) * 1e-4).astype(np.float32),
                        np.float32([65504.0, -65504.0, 6.1e-5, 5.9e-8, 1.0 + 2.0 ** -23])])
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    assert np.all(np.isfinite(hi)) and np.all(np.isfinite(lo))
    resid = np.abs(x.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    assert np.all(resid <= 2.0 ** -22 * np.abs(x.astype(np.float64)) + 2.0 ** -25)
