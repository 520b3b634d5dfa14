"""KV page pool and geometry (include/moearc_kv.h), CPU only.

The first eleven tests restate the reference's own tests of PagedKvCache
(crates/moearc-engine/src/kv.rs:207-353) against this build's pool, scenario for scenario. The
rest cover what this build adds -- the all-or-nothing chunk append, batched block tables, the ring
sizing of a windowed layer under chunked prefill -- the last pinned with the oracle: a prefill run
through the ring equals one over a contiguous cache exactly when the ring holds window + chunk - 1
tokens, and differs when it holds one page less.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd.kv import (ContextLimit, Exhausted, InvalidGeometry, KvError, KvGeometry,
                           PagedKvCache, UnknownSequence)
from oracle import oracle


def pool():
    return PagedKvCache(16, 4, 1024)


# ---- the reference's tests (kv.rs:214-352) ------------------------------------------------------

def test_a_prompt_takes_only_the_pages_it_needs():
    kv = pool()
    s = kv.begin(1, 9)  # 9 tokens over 4-token pages = 3 pages, the last a quarter used
    assert len(s.pages) == 3
    u = kv.usage()
    assert u.used_pages == 3
    assert u.slack_tokens == 3  # 12 slots for 9 tokens


def test_appending_allocates_only_when_a_page_fills():
    kv = pool()
    kv.begin(1, 4)
    assert kv.usage().used_pages == 1
    _, slot = kv.append(1)  # must open a second page
    assert slot == 0
    assert kv.usage().used_pages == 2
    for _ in range(3):
        kv.append(1)
    assert kv.usage().used_pages == 2, "no page opened before it was needed"
    kv.append(1)
    assert kv.usage().used_pages == 3


def test_tokens_land_where_the_page_table_says():
    kv = pool()
    kv.begin(1, 0)
    seen = [kv.append(1) for _ in range(10)]
    table = kv.pages_of(1).pages
    for i, (page, slot) in enumerate(seen):
        assert page == table[i // 4], f"token {i} is in the wrong page"
        assert slot == i % 4, f"token {i} is in the wrong slot"


def test_ending_a_sequence_returns_every_page():
    kv = pool()
    kv.begin(1, 12)
    kv.begin(2, 8)
    assert kv.usage().used_pages == 5
    assert kv.end(1) == 3
    assert kv.usage().used_pages == 2
    assert kv.end(2) == 2
    assert kv.usage().used_pages == 0
    assert kv.usage().free_pages() == 16


def test_pages_are_reused_rather_than_leaked():
    kv = pool()  # cycle far more sequences than there are pages: a leak shows up as exhaustion
    for i in range(200):
        kv.begin(i, 12)
        for _ in range(5):
            kv.append(i)
        kv.end(i)
    assert kv.usage().used_pages == 0
    assert kv.usage().free_pages() == 16


def test_exhaustion_is_reported_and_leaves_state_untouched():
    kv = PagedKvCache(2, 4, 1024)
    kv.begin(1, 8)  # takes both pages
    before = kv.usage()
    with pytest.raises(Exhausted) as e:
        kv.begin(2, 4)
    assert (e.value.requested, e.value.free) == (1, 0)
    assert kv.usage() == before, "a failed begin must not consume anything"
    tokens_before = kv.pages_of(1).tokens
    with pytest.raises(Exhausted):
        kv.append(1)
    assert kv.pages_of(1).tokens == tokens_before, "sequence was half-extended"


@pytest.mark.parametrize("tokens", [0, 1, 4, 5, 60, 64, 65, 2000])
def test_can_admit_agrees_with_what_begin_actually_does(tokens):
    kv = pool()
    predicted = kv.can_admit(tokens)
    try:
        kv.begin(1, tokens)
        actual = True
    except KvError:
        actual = False
    assert predicted == actual, f"disagreement at {tokens} tokens"


def test_the_context_limit_is_enforced_at_both_entry_points():
    kv = PagedKvCache(64, 4, 8)
    with pytest.raises(ContextLimit):
        kv.begin(1, 9)
    kv.begin(2, 8)
    with pytest.raises(ContextLimit) as e:
        kv.append(2)
    assert (e.value.seq, e.value.tokens, e.value.limit) == (2, 8, 8)


def test_unknown_sequences_are_refused_rather_than_panicking():
    kv = pool()
    with pytest.raises(UnknownSequence):
        kv.append(99)
    with pytest.raises(UnknownSequence):
        kv.end(99)
    with pytest.raises(UnknownSequence):
        kv.pages_of(99)


def test_no_two_live_sequences_share_a_page():
    kv = pool()
    for i in range(4):
        kv.begin(i, 4)
    pages = [p for i in range(4) for p in kv.pages_of(i).pages]
    assert len(set(pages)) == len(pages), "a page was handed to two sequences"


def test_invalid_geometry_is_rejected():
    with pytest.raises(InvalidGeometry):
        PagedKvCache(0, 4, 16)
    with pytest.raises(InvalidGeometry):
        PagedKvCache(4, 0, 16)


# ---- this build's additions ---------------------------------------------------------------------

def test_fresh_pool_hands_out_page_zero_first_and_reuses_freed_pages_first():
    kv = pool()
    assert kv.begin(1, 8).pages == (0, 1)
    kv.end(1)
    assert kv.begin(2, 4).pages == (0,)


def test_chunk_append_equals_token_appends():
    a, b = pool(), pool()
    a.begin(1, 3)
    b.begin(1, 3)
    pages, slots = a.append_chunk(1, 11)
    want = [b.append(1) for _ in range(11)]
    assert list(zip(pages.tolist(), slots.tolist())) == want
    assert a.pages_of(1) == b.pages_of(1)
    assert a.usage() == b.usage()


def test_chunk_append_is_all_or_nothing():
    kv = PagedKvCache(3, 4, 1024)
    kv.begin(1, 2)
    before, table = kv.usage(), kv.pages_of(1)
    with pytest.raises(Exhausted) as e:
        kv.append_chunk(1, 11)  # 13 tokens need 4 pages, 1 held + 2 free
    assert (e.value.requested, e.value.free) == (3, 2)
    assert kv.usage() == before and kv.pages_of(1) == table
    lim = PagedKvCache(16, 4, 10)
    lim.begin(1, 6)
    with pytest.raises(ContextLimit) as e:
        lim.append_chunk(1, 5)
    assert (e.value.tokens, e.value.limit) == (11, 10)
    assert lim.pages_of(1).tokens == 6


def test_begin_on_an_active_sequence_is_refused():
    kv = pool()
    kv.begin(1, 5)
    with pytest.raises(ValueError):
        kv.begin(1, 5)
    assert kv.usage().used_pages == 2


def test_batched_block_tables():
    kv = pool()
    kv.begin(7, 9)
    kv.begin(3, 1)
    kv.begin(5, 16)
    table, stride = kv.block_tables([7, 3, 5])
    assert stride == 4
    for row, s in zip(table, (7, 3, 5)):
        pages = kv.pages_of(s).pages
        assert tuple(row[:len(pages)]) == pages and not row[len(pages):].any()
    with pytest.raises(ValueError):
        kv.block_tables([5], stride=3)
    with pytest.raises(KvError):
        kv.block_tables([7, 42])


def test_geometry_matches_the_reference_plan_for_token_by_token_decode():
    # KvGeometry::plan (moe.rs:735-757): pages = ceil(n_ctx/pt) >= 1, ring = ceil(n_swa/pt)
    # capped at pages
    for n_ctx, pt, w in [(32768, 256, 128), (4096, 16, 128), (100, 64, 128), (1, 256, None),
                         (0, 16, 128), (131072, 256, None)]:
        g = KvGeometry.plan(n_ctx, pt, w)
        pages = max(1, -(-n_ctx // pt))
        assert g.pages == pages
        assert g.swa_pages == (pages if w is None else min(pages, max(1, -(-w // pt))))


def test_ring_holds_window_plus_chunk():
    g = KvGeometry.plan(40960, 16, 128, chunk=2048)
    assert g.ring_tokens() >= 128 + 2048 - 1
    assert g.swa_pages == -(-(128 + 2048 - 1) // 16)
    assert KvGeometry.plan(1000, 16, 128, chunk=2048).swa_pages == 63  # capped at the full cache
    t = KvGeometry.plan(200, 8, 40, chunk=24).ring_table()
    assert t.tolist() == [i % 8 for i in range(25)]


def _ring_prefill(c, ring_pages, chunk, n_swa):
    """Chunked prefill of every token of case c through a ring of ring_pages pages (the K/V of a
    chunk written before it attends, as the engine does), on the oracle."""
    pt, row = c.pt, c.G * c.D
    T = c.n_q
    k_rows, v_rows = c.k_raw.reshape(-1, row), c.v_raw.reshape(-1, row)  # f16 bits, physical rows
    table = KvGeometry(-(-T // pt), ring_pages, pt).ring_table()
    rk = np.zeros((ring_pages * pt, row), np.uint16)
    rv = np.zeros_like(rk)
    out = np.zeros((T, c.H, c.D), np.float32)
    for p0 in range(0, T, chunk):
        n = min(chunk, T - p0)
        for x in range(p0, p0 + n):
            src = int(c.bt[x // pt]) * pt + x % pt
            dst = int(table[x // pt]) * pt + x % pt
            rk[dst], rv[dst] = k_rows[src], v_rows[src]
        out[p0:p0 + n] = oracle.attn_prefill(c.qp[p0:p0 + n].astype(np.float32), rk, rv, table, n, p0,
                                             n_swa, c.H, c.G, c.D, pt, float(c.scale), sinks=c.sinks,
                                             n_threads=8)
    return out


def test_ring_size_under_chunked_prefill_is_pinned_by_the_oracle():
    n_swa, chunk, pt = 40, 24, 8
    c = fx.prefill_case(0x41D6, n_q=200, pos0=0, pt=pt)
    want = oracle.attn_prefill(c.qp.astype(np.float32), c.k_raw, c.v_raw, c.bt, c.n_q, 0, n_swa, c.H,
                               c.G, c.D, pt, float(c.scale), sinks=c.sinks, n_threads=8)
    need = KvGeometry.plan(200, pt, n_swa, chunk=chunk).swa_pages
    assert need * pt >= n_swa + chunk - 1 and (need - 1) * pt < n_swa + chunk - 1
    exact = _ring_prefill(c, need, chunk, n_swa)
    assert np.array_equal(exact, want)
    short = _ring_prefill(c, need - 1, chunk, n_swa)  # one page short: window keys overwritten
    assert np.max(np.abs(short - want)) > 1e-3
    decode_sized = KvGeometry.plan(200, pt, n_swa).swa_pages  # the reference's ring (chunk 1)
    assert np.max(np.abs(_ring_prefill(c, decode_sized, chunk, n_swa) - want)) > 1e-3
