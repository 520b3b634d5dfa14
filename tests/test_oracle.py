"""Pins the CPU oracle (CPU only, no GPU).

Each check compares the oracle with something it does not share code with: numpy's IEEE binary16
conversion, torch's float64 scaled_dot_product_attention, closed forms, brute force, and the
reference tests' own fixtures and assertions (crates/moearc-kernels/tests/forward_pass_gpu.rs).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import synth
from oracle import oracle


# ---- RNG ----------------------------------------------------------------------------------------

def test_splitmix64_matches_published_vectors():
    # SplitMix64 seeded with 0: the first outputs published with the generator.
    r = oracle.Rng(0)
    assert [r.next_u64() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                                0x06C45D188009454F]
    assert list(synth.splitmix64(0, 3)) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                            0x06C45D188009454F]


def test_vectorised_unit_draws_equal_the_sequential_generator():
    for seed in (0xA77E, 0x6A11, 0x5A11, 12345):
        r = oracle.Rng(seed)
        seq = r.vec_unit(1000)
        assert np.array_equal(seq, synth.unit(seed, 1000))
        assert np.array_equal(synth.unit(seed, 10, skip=990), seq[990:])
        assert seq.min() >= -1.0 and seq.max() < 1.0


def test_normal_generator_moments():
    z = synth.normal(7, 1 << 20)
    assert abs(float(z.mean())) < 5e-3 and abs(float(z.std()) - 1.0) < 5e-3


# ---- f16 codecs (reference.rs:123-149, :647-691) ------------------------------------------------

def test_f16_widening_equals_numpy_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # signed zeros too


def test_f16_narrowing_equals_numpy_ieee_rne():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    ok = ~np.isnan(vals)
    assert np.array_equal(oracle.f32_to_f16(vals[ok]), bits[ok])  # exact values round-trip
    hard = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65520.0, 65519.996, 1e-8, -1e-8,
                     6e-8, 5.9604645e-8, 1.7881393e-7, np.finfo(np.float32).tiny, 1e30, -1e30,
                     np.inf, -np.inf], np.float32)  # forward_pass_gpu.rs:112-131
    rng = oracle.Rng(0xF167)
    rand = np.concatenate([rng.vec_unit(8192) * 4, rng.vec_unit(2048) * 1e-5]).astype(np.float32)
    # every tie and near-tie between adjacent f16 values, over the whole range
    lo = np.arange(0, 0x7BFF, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (np.arange(0, 0x7BFF, dtype=np.uint32) + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    x = np.concatenate([hard, rand, near, -near]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x), want)


def test_f16_nan_payload_rule():
    # reference.rs:655-660: NaN keeps NaN-ness with payload 0x200 | mant >> 13
    for bits in (0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x7FA00000):
        f = np.array([bits], np.uint32).view(np.float32)
        mant = bits & 0x7FFFFF
        want = ((bits >> 16) & 0x8000) | 0x7C00 | 0x200 | (mant >> 13)
        assert int(oracle.f32_to_f16(f)[0]) == want


# ---- KV layout (reference.rs:767-802) -----------------------------------------------------------

def test_kv_append_writes_exactly_its_slot():
    # forward_pass_gpu.rs:431-497: G=3, D=16, pt=4, 5 pages poisoned with -7.5, page 3 slot 2
    heads, hd, pt, pages = 3, 16, 4, 5
    row = heads * hd
    pool = pages * pt * row
    r = oracle.Rng(0xC0DE)
    k, v = r.vec_unit(row), r.vec_unit(row)
    kp = np.full(pool, -7.5, np.float32)
    vp = np.full(pool, -7.5, np.float32)
    oracle.kv_append(kp, vp, k, v, 3, 2, heads, hd, pt, oracle.KV_F32)
    base = oracle.kv_index(3, 2, 0, 0, heads, hd, pt)
    assert base == (3 * pt + 2) * row
    assert np.array_equal(kp[base:base + row], k) and np.array_equal(vp[base:base + row], v)
    assert kp[base - 1] == -7.5 and kp[base + row] == -7.5
    assert np.count_nonzero(kp != -7.5) == np.count_nonzero(k != -7.5)
    # f16 storage: the value that lands is f16_to_f32(f32_to_f16(x)) (reference.rs:754-759)
    kp16 = np.zeros(pool, np.float32)
    vp16 = np.zeros(pool, np.float32)
    oracle.kv_append(kp16, vp16, k, v, 3, 2, heads, hd, pt, oracle.KV_F16)
    assert np.array_equal(kp16[base:base + row], k.astype(np.float16).astype(np.float32))


def test_kv_index_layout_against_numpy_reshape():
    G, D, pt = 3, 5, 4
    pool = np.arange(7 * pt * G * D).reshape(7, pt, G, D)
    for page, slot, h, d in [(0, 0, 0, 0), (6, 3, 2, 4), (2, 1, 1, 3)]:
        assert oracle.kv_index(page, slot, h, d, G, D, pt) == pool[page, slot, h, d]


# ---- attention against torch SDPA and closed forms ----------------------------------------------

@pytest.mark.parametrize("name", list(fx.REFERENCE_CASES))
def test_reference_fixtures_against_sdpa_and_golden(name):
    c = fx.reference_case(name)
    g = fx.load_golden("ref_" + name)
    assert str(g["digest"]) == c.digest(), "the regenerated reference inputs drifted"
    got = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, c.kv_begin, c.n_kv, c.pt,
                             float(c.scale), kv_type=c.kv, f64=True)
    ref = fx.sdpa_reference(c)
    assert np.max(np.abs(got - ref)) < 1e-12
    assert np.array_equal(got, g["expected"])
    # |out| <= max|V| (forward_pass_gpu.rs:586-589)
    assert np.abs(got).max() <= np.abs(c.v_val).max() + 1e-12


def test_host_mirror_equals_device_format_pools():
    c = fx.reference_case("scattered_f16")
    a = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                           float(c.scale), kv_type=1, f64=True)
    b = oracle.attn_decode(c.q, c.k_val, c.v_val, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                           float(c.scale), kv_type=0, f64=True)
    assert np.array_equal(a, b)


def test_single_key_returns_v_exactly():
    c = fx.reference_case("single_key")
    out = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 1, c.pt, 0.125)
    v = c.v_val.reshape(-1, c.G, c.D)[int(c.bt[0]) * c.pt]  # page 1 slot 0
    assert np.array_equal(out.reshape(c.H, c.D), v)


def test_window_claims():
    c = fx.reference_case("window")
    run = lambda b: oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, b, c.n_kv,
                                       c.pt, float(c.scale), f64=True)
    win, full, one = run(15), run(0), run(c.n_kv - 1)
    assert np.max(np.abs(win - full)) > 1e-3  # the window must move the answer
    j = c.n_kv - 1
    vrow = c.v_val.reshape(-1, c.G, c.D)[int(c.bt[j // c.pt]) * c.pt + j % c.pt]
    group = c.H // c.G
    assert np.array_equal(one.reshape(c.H, c.D), np.repeat(vrow, group, axis=0).astype(np.float64))


def test_refusals():
    c = fx.reference_case("gqa")
    with pytest.raises(oracle.OracleRefusal):  # empty span (forward_pass_gpu.rs:874-886)
        oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 4, 4, c.pt, 1.0)
    with pytest.raises(oracle.OracleRefusal):  # 6 % 4 (forward_pass_gpu.rs:889-899)
        oracle.attn_decode(np.zeros(48, np.float32), c.k_raw, c.v_raw, c.bt, 6, 4, 8, 0, 4, 4, 1.0)


def test_sinks_against_sdpa_with_a_zero_valued_key():
    c = fx.north_star_case(11, 200, pt=16)
    got = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, c.n_kv, c.pt,
                             float(c.scale), kv_type=1, sinks=c.sinks, f64=True)
    assert np.max(np.abs(got - fx.sdpa_reference(c, sinks=c.sinks))) < 1e-12
    g = fx.load_golden("ns_decode_full")
    c2 = fx.north_star_case(0x5EED, 300, pt=32)
    assert str(g["digest"]) == c2.digest()


def test_sink_closed_forms():
    c = fx.north_star_case(3, 1, pt=4, H=8, G=2, D=16)
    out = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 1, c.pt,
                             float(c.scale), kv_type=1, sinks=c.sinks, f64=True).reshape(c.H, c.D)
    K = fx.contiguous_kv(c, "k")[0]
    V = fx.contiguous_kv(c, "v")[0]
    for h in range(c.H):
        g = h // (c.H // c.G)
        s = float(np.dot(c.q[h * c.D:(h + 1) * c.D].astype(np.float64), K[g])) * float(c.scale)
        sig = 1.0 / (1.0 + math.exp(float(c.sinks[h]) - s))  # one key: V * sigma(s - sink)
        assert np.allclose(out[h], V[g] * sig, rtol=0, atol=1e-12)
    # identical keys: out = mean(V) * n / (n + e^(sink - s))
    n = 37
    c = fx.north_star_case(4, n, pt=8, H=4, G=1, D=8)
    k0 = c.k_raw.reshape(-1, c.G * c.D)[int(c.bt[0]) * c.pt].copy()
    kr = c.k_raw.reshape(-1, c.G * c.D)
    for j in range(n):
        kr[int(c.bt[j // c.pt]) * c.pt + j % c.pt] = k0
    out = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, n, c.pt,
                             float(c.scale), kv_type=1, sinks=c.sinks, f64=True).reshape(c.H, c.D)
    V = fx.contiguous_kv(c, "v")[:, 0]
    k0f = k0.view(np.float16).astype(np.float64)
    for h in range(c.H):
        s = float(np.dot(c.q[h * c.D:(h + 1) * c.D].astype(np.float64), k0f)) * float(c.scale)
        want = V.mean(axis=0) * n / (n + math.exp(float(c.sinks[h]) - s))
        assert np.allclose(out[h], want, rtol=0, atol=1e-12)
    # sink -> -1e30 is no sink
    c = fx.north_star_case(5, 50, pt=8, H=8, G=2, D=16)
    a = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 50, c.pt, float(c.scale),
                           kv_type=1, sinks=np.full(c.H, -1e30, np.float32), f64=True)
    b = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 50, c.pt, float(c.scale),
                           kv_type=1, f64=True)
    assert np.array_equal(a, b)


def test_batched_equals_single_calls():
    cs = [fx.north_star_case(20 + i, n, pt=16, H=16, G=4, D=64) for i, n in enumerate((5, 70, 33))]
    # one shared pool: give each sequence its own pages in a combined table
    G, D, pt = 4, 64, 16
    row = G * D
    pools_k, pools_v, tables, off = [], [], [], 0
    for c in cs:
        pools_k.append(c.k_raw.reshape(-1, row))
        pools_v.append(c.v_raw.reshape(-1, row))
        tables.append(c.bt_full + off)
        off += pools_k[-1].shape[0] // pt
    kp, vp = np.concatenate(pools_k).ravel(), np.concatenate(pools_v).ravel()
    stride = max(len(t) for t in tables)
    bts = np.zeros((3, stride), np.uint32)
    for i, t in enumerate(tables):
        bts[i, :len(t)] = t
    q = np.stack([c.q.reshape(16, 64) for c in cs])
    kb = np.array([0, 70 - 16, 3], np.uint32)
    nk = np.array([5, 70, 33], np.uint32)
    sinks = cs[0].sinks
    got = oracle.attn_decode_batched(q, kp, vp, bts, kb, nk, 16, G, D, pt, 0.125, sinks=sinks,
                                     n_threads=3)
    for i in range(3):
        want = oracle.attn_decode(q[i], kp, vp, bts[i], 16, G, D, int(kb[i]), int(nk[i]), pt, 0.125,
                                  kv_type=1, sinks=sinks)
        assert np.array_equal(got[i].ravel(), want)


def test_prefill_rows_equal_brute_force_and_golden():
    pc = fx.prefill_case(0x9F11, n_q=48, pos0=80)
    for name, n_swa in (("ns_prefill_full", 0), ("ns_prefill_swa16", 16)):
        g = fx.load_golden(name)
        assert str(g["digest"]) == fx.prefill_digest(pc)
        out = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q,
                                  pc.pos0, n_swa, pc.H, pc.G, pc.D, pc.pt, float(pc.scale),
                                  sinks=pc.sinks, n_threads=4)
        brute = fx.prefill_brute(pc, n_swa)
        assert np.max(np.abs(out - brute)) < 1e-6
        assert np.max(np.abs(out[g["rows"]] - g["expected"])) < 1e-6
    # row i is decode at n_kv = pos0 + i + 1 (moe.rs:1856-1862)
    i = 17
    dec = oracle.attn_decode(pc.qp[i].astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.H, pc.G,
                             pc.D, pc.pos0 + i + 1 - 16, pc.pos0 + i + 1, pc.pt, float(pc.scale),
                             kv_type=1, sinks=pc.sinks)
    out = oracle.attn_prefill(pc.qp.astype(np.float32), pc.k_raw, pc.v_raw, pc.bt, pc.n_q, pc.pos0,
                              16, pc.H, pc.G, pc.D, pc.pt, float(pc.scale), sinks=pc.sinks,
                              rows=(i, i + 1, 1))
    assert np.array_equal(out[i].ravel(), dec)


def test_a_planted_mistake_is_caught():
    """A dropped sink term, a wrong GQA map or a transposed page walk must fail the SDPA check."""
    c = fx.north_star_case(31, 40, pt=8, H=8, G=2, D=16)
    good = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 40, c.pt,
                              float(c.scale), kv_type=1, sinks=c.sinks, f64=True)
    ref = fx.sdpa_reference(c, sinks=c.sinks)
    assert np.max(np.abs(good - ref)) < 1e-12
    no_sink = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 40, c.pt,
                                 float(c.scale), kv_type=1, f64=True)
    assert np.max(np.abs(no_sink - ref)) > 1e-3
    # kvh = h % G instead of h / group: run head h's query against head perm[h]'s KV head
    group = c.H // c.G
    perm = np.array([(h % c.G) * group + h // c.G for h in range(c.H)])
    qp = c.q.reshape(c.H, c.D)[np.argsort(perm)].ravel()
    wrong_group = oracle.attn_decode(qp, c.k_raw, c.v_raw, c.bt, c.H, c.G, c.D, 0, 40, c.pt,
                                     float(c.scale), kv_type=1, sinks=c.sinks[np.argsort(perm)],
                                     f64=True).reshape(c.H, c.D)[perm].ravel()
    assert np.max(np.abs(wrong_group - ref)) > 1e-3
    swapped = oracle.attn_decode(c.q, c.v_raw, c.k_raw, c.bt, c.H, c.G, c.D, 0, 40, c.pt,
                                 float(c.scale), kv_type=1, sinks=c.sinks, f64=True)
    assert np.max(np.abs(swapped - ref)) > 1e-3
    # full attention is permutation-invariant over keys, so a page-walk mistake shows on a span
    ref_w = fx.sdpa_reference(c, kv_begin=21, sinks=c.sinks)
    bad_table = oracle.attn_decode(c.q, c.k_raw, c.v_raw, c.bt[::-1].copy(), c.H, c.G, c.D, 21, 40,
                                   c.pt, float(c.scale), kv_type=1, sinks=c.sinks, f64=True)
    assert np.max(np.abs(bad_table - ref_w)) > 1e-3
