"""Profiling events on the GPU: the reference's key contract.

With MOEARC_PROFILE_EVENTS=1 the reference records every tracked submission once, under a key that
carries the launch geometry: "attn_decode r<n_heads> m<head_dim>" for attention, with sliding-window
and full-causal calls summed under the one key (kernels.cpp:1905-1916), and "mvq <type>",
"mvq_batched <type>" or "mv_generic" for the matvecs (kernels.cpp:1057-1111, :1168-1196). Its
consumers add every key of the report into one busy figure, so a call must appear under exactly one
key: the split and merge launches of a decode are not keys of their own unless
MOEARC_PROFILE_KERNELS=1 asks for them. Entry points the reference does not track (the KV append,
zero, add, RoPE) add no key.
"""
from __future__ import annotations

import numpy as np
import pytest

import fixtures as fx
from moearc_amd import Context, KvType

pytestmark = pytest.mark.gpu


def _decode_calls(cx, c, spans):
    dk, dv, dq = cx.upload(c.k_raw), cx.upload(c.v_raw), cx.upload(c.q)
    dbt, ds = cx.upload(c.bt), cx.upload(c.sinks)
    dout = cx.alloc(c.H * c.D * 4)
    for kv_begin in spans:
        cx.attn_decode_ext(dout, dq, dk, dv, dbt, ds, c.H, c.G, c.D, kv_begin, c.n_kv, c.pt,
                           float(c.scale), KvType.F16)
    cx.sync()


def test_decode_calls_are_one_key_summed_over_window_and_full(monkeypatch):
    monkeypatch.setenv("MOEARC_PROFILE_EVENTS", "1")
    monkeypatch.delenv("MOEARC_PROFILE_KERNELS", raising=False)
    c = fx.north_star_case(0x9E0, 20000, pt=256)
    # full-causal calls (split, merged by a second launch) and SWA-128 calls (one split each)
    spans = [0, 0, c.n_kv - 128, 0, c.n_kv - 128, c.n_kv - 128, 0]
    with Context() as cx:
        assert cx.profile_events_enabled()
        _decode_calls(cx, c, spans)
        # untracked entry points of the reference: no key
        buf = cx.alloc(4096)
        cx.zero(buf, 1024)
        cx.add(buf, buf, buf, 1024)
        cx.sync()
        rep = cx.profile_events_report()
        print("report:", rep, flush=True)
        assert set(rep) == {"attn_decode r64 m64"}
        ns, calls = rep["attn_decode r64 m64"]
        assert calls == len(spans)
        assert ns > 0
        # reset clears the totals
        cx.profile_events_reset()
        assert cx.profile_events_report() == {}


def test_general_kernel_shape_keys_by_its_geometry(monkeypatch):
    # the reference's own shape (16 q heads over 4 KV heads, head_dim 128, f32 KV) runs the general
    # kernel; the key carries that geometry
    monkeypatch.setenv("MOEARC_PROFILE_EVENTS", "1")
    monkeypatch.delenv("MOEARC_PROFILE_KERNELS", raising=False)
    c = fx.north_star_case(0x9E1, 300, H=16, G=4, D=128, pt=8)
    with Context() as cx:
        _decode_calls(cx, c, [0, 100, 299])
        rep = cx.profile_events_report()
        assert set(rep) == {"attn_decode r16 m128"}
        assert rep["attn_decode r16 m128"][1] == 3


def test_kernel_detail_only_on_request(monkeypatch):
    monkeypatch.setenv("MOEARC_PROFILE_EVENTS", "1")
    monkeypatch.setenv("MOEARC_PROFILE_KERNELS", "1")
    c = fx.north_star_case(0x9E2, 20000, pt=256)
    with Context() as cx:
        _decode_calls(cx, c, [0, 0, c.n_kv - 128])
        rep = cx.profile_events_report()
        print("report:", rep, flush=True)
        assert rep["attn_decode r64 m64"][1] == 3
        assert rep["kernel attn_decode.split r64 m64"][1] == 3
        # the two full-causal calls are split; the window fits one split and has no merge
        assert rep["kernel attn_decode.merge r64 m64"][1] == 2
        # the brackets nest: the call's time covers its kernels'
        inner = rep["kernel attn_decode.split r64 m64"][0] + rep["kernel attn_decode.merge r64 m64"][0]
        assert inner <= rep["attn_decode r64 m64"][0] * 1.02


def test_matvec_keys_name_the_weight_type(monkeypatch):
    monkeypatch.setenv("MOEARC_PROFILE_EVENTS", "1")
    monkeypatch.delenv("MOEARC_PROFILE_KERNELS", raising=False)
    rows, cols = 96, 512
    with Context() as cx:
        w8, _ = fx.synth_blocks(8, rows * cols // 32, 0x9E3)
        w16 = (np.random.default_rng(5).standard_normal(rows * cols) * 0.1).astype(np.float16)
        x = fx.synth.unit(0x9E4, cols)
        dw8, dw16, dx = cx.upload(w8), cx.upload(w16.view(np.uint8)), cx.upload(x)
        dy = cx.alloc(3 * rows * 4)
        cx.matvec_q(8, dy, dw8, dx, rows, cols)
        cx.matvec_q(8, dy, dw8, dx, rows, cols)
        cx.matvec_q(1, dy, dw16, dx, rows, cols)
        cx.matvec_q_batched(8, dy, [dw8, dw8, dw8], dx, 0, rows, cols)
        cx.matvec_f32(dy, cx.upload(np.ones(rows * cols, np.float32)), dx, rows, cols)
        cx.sync()
        rep = cx.profile_events_report()
        print("report:", rep, flush=True)
        assert rep["mvq Q8_0 r96 m1"][1] == 2
        assert rep["mv_generic r96 m1"][1] == 1
        assert rep["mvq_batched Q8_0 r96 m3"][1] == 1
        # moearc_matvec_f32 is not tracked by the reference
        assert set(rep) == {"mvq Q8_0 r96 m1", "mv_generic r96 m1", "mvq_batched Q8_0 r96 m3"}
