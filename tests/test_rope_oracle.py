"""Pins the RoPE oracle (oracle/moearc_oracle.c: orc_rope, orc_rope_yarn) on the CPU.

orc_rope restates the reference's CPU rope (reference.rs:468-505: angle table by repeated f32
multiplication); orc_rope_yarn restates the kernel's closed form with YaRN (kernels.cpp:1441-1466)
in f64. Both are checked against an independent formulation -- complex multiplication by
mscale * e^(i theta), pairs taken by slicing -- and against what the mathematics fixes: position 0
is the identity, a rotation keeps each pair's length (times mscale), YaRN's ramp endpoints are pure
extrapolation and pure interpolation, YaRN with freq_scale 1 is plain RoPE.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

import fixtures as fx
from oracle import oracle

R = fx.ROPE_REF
GPT = fx.GPT_OSS_ROPE


def _yarn_params(n_dims=64):
    from moearc_amd import RopeScaling
    return RopeScaling.yarn(n_dims, GPT["n_ctx_orig"], GPT["freq_base"], GPT["factor"],
                            GPT["beta_fast"], GPT["beta_slow"]).args()


def test_reference_fixture():
    src, pos = fx.rope_reference_inputs()
    g = fx.load_golden("ref_rope")
    assert str(g["digest"]) == hashlib.sha256(src.tobytes()).hexdigest()
    for name, neox in (("neox", True), ("normal", False)):
        got = oracle.rope(src, pos, R["tokens"], R["heads"], R["head_dim"], R["n_dims"], R["freq_base"], neox)
        assert np.array_equal(got, g["expected_" + name])


@pytest.mark.parametrize("neox", [True, False])
def test_iterated_and_closed_forms_match_complex_rotation(neox):
    src, pos = fx.rope_reference_inputs()
    args = (src, pos, R["tokens"], R["heads"], R["head_dim"], R["n_dims"], R["freq_base"])
    ind = fx.rope_complex(*args, neox=neox)
    it = oracle.rope(*args, neox=neox).astype(np.float64)
    closed = oracle.rope_yarn(*args, neox=neox)
    assert np.max(np.abs(it - ind)) < 1e-5
    assert np.max(np.abs(closed - ind)) < 1e-12
    # the channels past n_dims pass through bit for bit
    tail = np.asarray(src).reshape(R["tokens"], R["heads"], R["head_dim"])[..., R["n_dims"]:]
    assert np.array_equal(it.reshape(tail.shape[:2] + (-1,))[..., R["n_dims"]:], tail)


@pytest.mark.parametrize("neox", [True, False])
def test_yarn_closed_form_matches_complex_rotation_at_long_positions(neox):
    rng = np.random.default_rng(5)
    src = rng.standard_normal(6 * 2 * 64).astype(np.float32)
    pos = np.array([0, 1, 4095, 4096, 65536, 131071], np.int32)
    sc = _yarn_params()
    got = oracle.rope_yarn(src, pos, 6, 2, 64, 64, GPT["freq_base"], *sc, neox=neox)
    want = fx.rope_complex(src, pos, 6, 2, 64, 64, GPT["freq_base"], scaling=sc, neox=neox)
    assert np.max(np.abs(got - want)) < 1e-9


def test_position_zero_is_the_identity():
    src = np.random.default_rng(1).standard_normal(3 * 4 * 64).astype(np.float32)
    pos = np.zeros(3, np.int32)
    assert np.array_equal(oracle.rope(src, pos, 3, 4, 64, 64, 10000.0, True), src)
    assert np.array_equal(oracle.rope_yarn(src, pos, 3, 4, 64, 64, 10000.0), src.astype(np.float64))


@pytest.mark.parametrize("neox", [True, False])
def test_rotation_keeps_pair_lengths_times_mscale(neox):
    src = np.random.default_rng(2).standard_normal(4 * 3 * 64).astype(np.float32)
    pos = np.array([0, 2048, 4095, 131000], np.int32)
    x = src.astype(np.float64).reshape(4, 3, 64)
    for sc, msc in ((None, 1.0), (_yarn_params(), 1.0 + 0.1 * np.log(GPT["factor"]))):
        args = () if sc is None else sc
        y = oracle.rope_yarn(src, pos, 4, 3, 64, 64, GPT["freq_base"], *args, neox=neox).reshape(4, 3, 64)
        if neox:
            before, after = np.hypot(x[..., :32], x[..., 32:]), np.hypot(y[..., :32], y[..., 32:])
        else:
            before, after = np.hypot(x[..., 0::2], x[..., 1::2]), np.hypot(y[..., 0::2], y[..., 1::2])
        assert np.max(np.abs(after - msc * before)) < 1e-12


def test_yarn_ramp_endpoints():
    # corr dims above every pair: the ramp is 1 everywhere -> pure extrapolation (theta_extrap);
    # below every pair: the ramp is 0 -> pure interpolation (freq_scale * theta_extrap). Both with
    # YaRN's magnitude scale.
    src = np.random.default_rng(3).standard_normal(2 * 64).astype(np.float32)
    pos = np.array([7, 3000], np.int32)
    fs = 1.0 / GPT["factor"]
    msc = 1.0 + 0.1 * np.log(GPT["factor"])
    extrap = oracle.rope_yarn(src, pos, 2, 1, 64, 64, 10000.0, fs, 1.0, 1.0, 100.0, 100.0)
    want_e = fx.rope_complex(src, pos, 2, 1, 64, 64, 10000.0, scaling=(1.0, 0.0, msc, 0.0, 0.0))
    assert np.max(np.abs(extrap - want_e)) < 1e-12
    interp = oracle.rope_yarn(src, pos, 2, 1, 64, 64, 10000.0, fs, 1.0, 1.0, -100.0, -100.0)
    want_i = fx.rope_complex(src, pos, 2, 1, 64, 64, 10000.0, scaling=(fs, 0.0, msc, 0.0, 0.0))
    assert np.max(np.abs(interp - want_i)) < 1e-12
    # and the two endpoints differ, so the ramp's direction matters
    assert np.max(np.abs(extrap - interp)) > 1e-2


def test_yarn_with_unit_freq_scale_is_plain_rope():
    src = np.random.default_rng(4).standard_normal(3 * 64).astype(np.float32)
    pos = np.array([1, 50, 900], np.int32)
    a = oracle.rope_yarn(src, pos, 3, 1, 64, 64, 10000.0, 1.0, 1.0, 1.0, 8.0, 18.0)
    b = oracle.rope_yarn(src, pos, 3, 1, 64, 64, 10000.0)
    assert np.max(np.abs(a - b)) < 1e-15


def test_checks_catch_a_wrong_convention_and_a_flipped_sign():
    # the complex check tells the pairings apart, and a rotation the wrong way round
    src, pos = fx.rope_reference_inputs()
    args = (src, pos, R["tokens"], R["heads"], R["head_dim"], R["n_dims"], R["freq_base"])
    neox = oracle.rope_yarn(*args, neox=True)
    assert np.max(np.abs(neox - fx.rope_complex(*args, neox=False))) > 1e-2
    flipped = oracle.rope_yarn(src, -pos, *args[2:], neox=True)  # e^(-i theta)
    assert np.max(np.abs(flipped - fx.rope_complex(*args, neox=True))) > 1e-2


def test_rope_kv_append_chunk_composes_rope_and_append():
    G, D, pt, n = 2, 64, 8, 5
    rng = np.random.default_rng(6)
    k = rng.standard_normal((n, G, D)).astype(np.float32)
    v = rng.standard_normal((n, G, D)).astype(np.float32)
    pos = np.array([10, 11, 12, 13, 14], np.int32)
    pages, slots = np.array([3, 3, 0, 0, 0], np.uint32), np.array([6, 7, 0, 1, 2], np.uint32)
    kp = np.zeros(4 * pt * G * D, np.uint16)
    vp = np.zeros_like(kp)
    sc = _yarn_params()
    oracle.rope_kv_append_chunk(kp, vp, k, v, pos, pages, slots, n, G, D, pt, 64, GPT["freq_base"], sc)
    rot = oracle.rope_yarn(k.reshape(-1), pos, n, G, D, 64, GPT["freq_base"], *sc).reshape(n, G, D)
    for t in range(n):
        base = ((int(pages[t]) * pt + int(slots[t])) * G) * D
        assert np.array_equal(kp[base:base + G * D], oracle.f32_to_f16(rot[t].astype(np.float32).reshape(-1)))
        assert np.array_equal(vp[base:base + G * D], oracle.f32_to_f16(v[t].reshape(-1)))
