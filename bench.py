"""Benchmark of the attention hot path on one MI355X; prints one JSON line.

Workload (the config the metric is quoted on): single-sequence decode,
B=1, 32768 keys, 64 query heads over 8 KV heads, head_dim 64, f16 KV in 256-token pages through a
random page permutation, per-head f32 sinks, full causal, f16 output. A step is one attention layer
call. Inputs are N(0,1) from a seed (synthetic data; there is no model).

* Timed region: K steps captured in one HIP graph on the library's stream and replayed once,
  bracketed by stream synchronisations; every step reads a different one of 6 KV copies (384 MiB)
  so the 256 MB Infinity Cache cannot serve repeats. value = algorithmic bytes per step / step time.
* roofline: the dominant kernel (the split-K kernel) timed with HIP events on the library stream
  over K eager steps; achieved = algorithmic bytes per launch / its average duration, against
  8 TB/s. traffic = HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
  summary (profiles/decode_c2_pmc.md), when present.
* prefill: BASELINE config 4 (2048 new + 2048 cached tokens), full causal and SWA-128, MFMA
  utilisation = algorithmic flops / time / 2.5 PFLOP/s (dense f16).
* rope_kv_append_chunk: the fused RoPE-K + f16 K/V append of the same config-4 chunk (HBM-bound;
  bytes = f32 K/V in + f16 K/V out + position/page/slot per token).
* cpu_baseline: the CPU oracle (a C restatement of the reference's f64 CPU twin,
  reference.rs:821-873, plus the sink) timed on this host on a bounded sample of the same decode.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
H, G, D, PT = 64, 8, 64, 256
N_KV = 32768
COPIES = 6

# algorithmic bytes per C2 step: K + V (f16) + q (f32) + sinks (f32) + out (f16)
C2_BYTES = 2 * N_KV * G * D * 2 + H * D * 4 + H * 4 + H * D * 2
# config 4: 2048 new tokens after 2048 cached
PF_NQ, PF_POS0 = 2048, 2048
PF_PAIRS_FULL = sum(PF_POS0 + i + 1 for i in range(PF_NQ))
PF_FLOPS_FULL = PF_PAIRS_FULL * H * D * 4           # QK^T and PV, 2 flops per MAC
PF_FLOPS_SWA = PF_NQ * 128 * H * D * 4
PF_BYTES_SWA = PF_NQ * H * D * 2 + (PF_POS0 + PF_NQ - (PF_POS0 - 127)) * G * D * 2 * 2 + \
    PF_NQ * H * D * 2 + H * 4


class Hip:
    """The few HIP runtime calls the timing needs (graph capture and events), via ctypes."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipGetErrorString.restype = ctypes.c_char_p

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.lib.hipGetErrorString(rc).decode()}")

    def event(self):
        e = ctypes.c_void_p()
        self.ok(self.lib.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream):
        self.ok(self.lib.hipEventRecord(e, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, e0, e1):
        self.ok(self.lib.hipEventSynchronize(e1), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ok(self.lib.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def capture(self, stream, fn):
        """Capture fn()'s work on `stream` into an executable graph."""
        s = ctypes.c_void_p(stream)
        self.ok(self.lib.hipStreamBeginCapture(s, 1), "hipStreamBeginCapture")  # thread-local mode
        try:
            fn()
        finally:
            graph = ctypes.c_void_p()
            rc = self.lib.hipStreamEndCapture(s, ctypes.byref(graph))
        self.ok(rc, "hipStreamEndCapture")
        exe = ctypes.c_void_p()
        self.ok(self.lib.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)),
                "hipGraphInstantiate")
        return graph, exe

    def launch(self, exe, stream):
        self.ok(self.lib.hipGraphLaunch(exe, ctypes.c_void_p(stream)), "hipGraphLaunch")

    def destroy(self, graph, exe):
        self.lib.hipGraphExecDestroy(exe)
        self.lib.hipGraphDestroy(graph)


def decode_inputs(seed=0xC2):
    from moearc_amd import synth
    row = G * D
    pages = N_KV // PT
    k = synth.f16_bits(synth.normal(seed, N_KV * row))
    v = synth.f16_bits(synth.normal(seed + 1, N_KV * row))
    bt = synth.random_block_table(seed + 5, pages)
    # scatter logical keys into their physical pages
    kp = np.empty_like(k).reshape(pages, PT, row)
    vp = np.empty_like(v).reshape(pages, PT, row)
    kp[bt] = k.reshape(pages, PT, row)
    vp[bt] = v.reshape(pages, PT, row)
    q = synth.normal(seed + 3, H * D)
    sinks = synth.normal(seed + 4, H)
    return kp.ravel(), vp.ravel(), bt, q, sinks


def pmc_traffic(path):
    """HBM bytes per launch of the split kernel from the committed rocprofv3 summary."""
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split()[1])
    return vals or None


def run(steps, warmup, skip_cpu=False, skip_prefill=False):
    from moearc_amd import Context, KvType, OUT_F16

    hip = Hip()
    kp, vp, bt, q, sinks = decode_inputs()
    result = {}

    with Context() as ctx:
        stream = ctx.stream
        dks = [ctx.upload(kp) for _ in range(COPIES)]
        dvs = [ctx.upload(vp) for _ in range(COPIES)]
        dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
        dout = ctx.alloc(H * D * 2)
        kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)

        def step(i):
            ctx.attn_decode_batched(dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT, kb,
                                    nk, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)

        for i in range(warmup):
            step(i)
        ctx.sync()
        eager_out = ctx.download(dout, np.float16, (H, D)).astype(np.float32)
        graph, exe = hip.capture(stream, lambda: [step(i) for i in range(steps)])
        e0, e1 = hip.event(), hip.event()
        hip.launch(exe, stream)  # one untimed replay
        ctx.sync()
        ctx.sync()
        t0 = time.perf_counter()
        hip.record(e0, stream)
        hip.launch(exe, stream)
        hip.record(e1, stream)
        ctx.sync()
        t1 = time.perf_counter()
        gpu_ms = hip.elapsed_ms(e0, e1)
        hip.destroy(graph, exe)
        graph_out = ctx.download(dout, np.float16, (H, D)).astype(np.float32)
        wall_ms = (t1 - t0) * 1e3
        result["step_us_gpu"] = gpu_ms * 1e3 / steps
        result["step_us_wall"] = wall_ms * 1e3 / steps
        result["graph_equals_eager"] = bool(np.array_equal(graph_out, eager_out))
        result["out"] = graph_out
        del dks, dvs
        result["projections"] = bench_matvec(ctx, hip, steps=max(20, steps))
        result["block_chunk"] = bench_block(ctx, hip)
        result["chunk_projections"] = bench_matmul(ctx, hip)

    # per-kernel event timing (eager, profiling context)
    os.environ["MOEARC_PROFILE_EVENTS"] = "1"
    try:
        with Context() as ctx:
            dks = [ctx.upload(kp) for _ in range(COPIES)]
            dvs = [ctx.upload(vp) for _ in range(COPIES)]
            dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
            dout = ctx.alloc(H * D * 2)
            kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
            for i in range(warmup + steps):
                if i == warmup:
                    ctx.sync()
                    ctx.profile_events_reset()
                ctx.attn_decode_batched(dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT,
                                        kb, nk, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)
            ctx.sync()
            rep = ctx.profile_events_report()
            result["events"] = {k: v[0] / v[1] / 1e3 for k, v in rep.items()}

            if not skip_prefill:
                result["prefill"] = bench_prefill(ctx, steps=max(5, steps // 5), warmup=3)
    finally:
        os.environ.pop("MOEARC_PROFILE_EVENTS", None)

    if not skip_cpu:
        result["cpu"] = cpu_baseline(kp, vp, bt, q, sinks)
    return result


def bench_prefill(ctx, steps, warmup):
    import fixtures as fx  # tests/fixtures.py: the same seeded prefill inputs the parity tests use
    from moearc_amd import KvType, OUT_F16
    pc = fx.prefill_case(0xC4, n_q=PF_NQ, pos0=PF_POS0, pt=PT)
    copies = 4
    dks = [ctx.upload(pc.k_raw) for _ in range(copies)]
    dvs = [ctx.upload(pc.v_raw) for _ in range(copies)]
    dqs = [ctx.upload(np.ascontiguousarray(pc.qp).view(np.uint16)) for _ in range(copies)]
    dbt, ds = ctx.upload(pc.bt), ctx.upload(pc.sinks)
    dout = ctx.alloc(PF_NQ * H * D * 2)
    out = {}
    for name, n_swa in (("full", 0), ("swa128", 128)):
        for i in range(warmup + steps):
            if i == warmup:
                ctx.sync()
                ctx.profile_events_reset()
            ctx.attn_prefill(dout, dqs[i % copies], dks[i % copies], dvs[i % copies], dbt, ds, PF_NQ,
                             PF_POS0, n_swa, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)
        ctx.sync()
        rep = ctx.profile_events_report()
        us = rep["attn_prefill r64 m64"][0] / rep["attn_prefill r64 m64"][1] / 1e3
        flops = PF_FLOPS_FULL if n_swa == 0 else PF_FLOPS_SWA
        tflops = flops / us / 1e6
        entry = {"us": round(us, 2), "tflops": round(tflops, 1),
                 "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                 "tokens_per_s": round(PF_NQ * 1e6 / us, 0)}
        if n_swa:
            gbs = PF_BYTES_SWA / us / 1e3
            bound_us = max(PF_BYTES_SWA / (HBM_PEAK_GBS * 1e3), flops / (MFMA_F16_PEAK_TFLOPS * 1e6))
            entry.update({"hbm_gbs": round(gbs, 0), "roofline_frac": round(bound_us / us, 4)})
        out[name] = entry
    out["rope_kv_append_chunk"] = bench_rope_append(ctx, steps, warmup)
    return out


def rope_append_inputs(ctx, copies):
    """Device inputs for the fused RoPE-K + K/V append of one config-4 chunk (2048 tokens after
    2048 cached, 8 KV heads x 64, 256-token pages), in ``copies`` independent sets so that repeated
    launches stream from HBM rather than the 256 MB Infinity Cache."""
    n, row = PF_NQ, G * D
    rng = np.random.default_rng(0xA11)
    k = rng.standard_normal(n * row).astype(np.float32)
    v = rng.standard_normal(n * row).astype(np.float32)
    pos = (PF_POS0 + np.arange(n)).astype(np.int32)
    n_pages = (PF_POS0 + n) // PT
    pages, slots = (pos // PT).astype(np.uint32), (pos % PT).astype(np.uint32)
    meta = ctx.upload(pos), ctx.upload(pages), ctx.upload(slots)
    sets = [(ctx.upload(k), ctx.upload(v), ctx.alloc(n_pages * PT * row * 2),
             ctx.alloc(n_pages * PT * row * 2)) for _ in range(copies)]
    return sets, meta


def rope_append_launch(ctx, sets, meta, i):
    from moearc_amd import KvType, RopeKind, RopeScaling
    dk, dv, kp, vp = sets[i % len(sets)]
    dpos, dpg, dsl = meta
    ctx.rope_kv_append_chunk(kp, vp, dk, dv, dpos, dpg, dsl, PF_NQ, G, D, PT, D, 150000.0,
                             scaling=RopeScaling.yarn(D, 4096, 150000.0, 32.0), kind=RopeKind.NEOX,
                             kv=KvType.F16)


# algorithmic bytes of one chunk append: f32 K and V read, f16 K and V written, and the per-token
# position, page id and slot (4 bytes each)
RA_BYTES = PF_NQ * G * D * (4 + 4 + 2 + 2) + PF_NQ * 12


def bench_rope_append(ctx, steps, warmup):
    """The fused RoPE-K + f16 K/V append (HBM-bound) timed with the library's events."""
    sets, meta = rope_append_inputs(ctx, 24)
    for i in range(warmup + steps):
        if i == warmup:
            ctx.sync()
            ctx.profile_events_reset()
        rope_append_launch(ctx, sets, meta, i)
    ctx.sync()
    rep = ctx.profile_events_report()
    key = [k2 for k2 in rep if k2.startswith("rope_kv_append_chunk")][0]
    us = rep[key][0] / rep[key][1] / 1e3
    gbs = RA_BYTES / us / 1e3
    return {"us": round(us, 2), "bytes": RA_BYTES, "hbm_gbs": round(gbs, 0),
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}


# The attention projections either side of the path, at gpt-oss-20b's shapes (2880-wide residual,
# 64 x 64 query, 8 x 64 KV; moe.rs:1942-1959 and 2063-2071) and Qwen3-30B-A3B's q (4096 x 2048):
# (label, type id, rows of q / k / v or of the single matrix, columns, fused qkv with biases?)
MV_CASES = [
    ("attn.qkv Q8_0 gpt-oss (4096+512+512)x2880 +bias", 8, (4096, 512, 512), 2880, True),
    ("attn.proj Q8_0 gpt-oss 2880x4096", 8, (2880,), 4096, False),
    ("attn.qkv F16 gpt-oss (4096+512+512)x2880 +bias", 1, (4096, 512, 512), 2880, True),
    ("attn.qkv MXFP4 gpt-oss (4096+512+512)x2880 +bias", 39, (4096, 512, 512), 2880, True),
    ("attn_q Q4_K qwen3-30b 4096x2048", 12, (4096,), 2048, False),
]


def mv_inputs(ctx, ty, rows, cols, fused, copies):
    """Weight copies enough to stream from HBM (each launch reads a different copy, and all of
    them together exceed the 256 MB Infinity Cache), one activation, biases and outputs."""
    from moearc_amd import QuantType
    qt = QuantType(ty)
    rng = np.random.default_rng(0x3A7 + ty)
    x = rng.standard_normal(cols).astype(np.float32)
    mats = []
    for r in rows:
        nbytes = r * qt.row_bytes(cols)
        w = rng.integers(0, 256, nbytes, dtype=np.uint8)
        if ty in (0, 1):  # finite values, not random bit patterns
            w = (rng.standard_normal(nbytes // qt.block_bytes).astype(np.float32 if ty == 0 else np.float16)
                 .view(np.uint8))
        mats.append(w)
    per_copy = sum(m.nbytes for m in mats)
    n = max(2, min(copies, (400 << 20) // per_copy + 1))
    dws = [[ctx.upload(m) for m in mats] for _ in range(n)]
    biases = [ctx.upload(rng.standard_normal(r).astype(np.float32)) if fused else None for r in rows]
    outs = [ctx.alloc(r * 4) for r in rows]
    return ctx.upload(x), dws, biases, outs, per_copy


def mv_launch(ctx, ty, rows, cols, fused, inputs, i):
    dx, dws, biases, outs, _ = inputs
    ws = dws[i % len(dws)]
    if fused:
        ctx.attn_qkv([ty] * 3, outs, ws, biases, rows, dx, cols)
    else:
        ctx.matvec_q(ty, outs[0], ws[0], dx, rows[0], cols)


def bench_matvec(ctx, hip, steps):
    """Each projection case as a captured graph of `steps` launches (each on the next weight copy),
    replayed once untimed and once between HIP events: the per-launch time excludes host
    submission, which for kernels this short would otherwise dominate. Achieved bandwidth counts
    the algorithmic bytes (every weight byte once, the activation, biases and outputs)."""
    res = {}
    for label, ty, rows, cols, fused in MV_CASES:
        inputs = mv_inputs(ctx, ty, rows, cols, fused, 128)
        mv_launch(ctx, ty, rows, cols, fused, inputs, 0)
        ctx.sync()
        graph, exe = hip.capture(ctx.stream, lambda: [mv_launch(ctx, ty, rows, cols, fused, inputs, i)
                                                      for i in range(steps)])
        e0, e1 = hip.event(), hip.event()
        hip.launch(exe, ctx.stream)
        ctx.sync()
        hip.record(e0, ctx.stream)
        hip.launch(exe, ctx.stream)
        hip.record(e1, ctx.stream)
        ctx.sync()
        us = hip.elapsed_ms(e0, e1) * 1e3 / steps
        hip.destroy(graph, exe)
        nbytes = inputs[4] + cols * 4 + sum(rows) * 4 * (2 if fused else 1)
        gbs = nbytes / us / 1e3
        res[label] = {"us": round(us, 2), "bytes": nbytes, "hbm_gbs": round(gbs, 0),
                      "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}
        del inputs
    return res


# Chunk-form projections on MFMA (moearc_matmul_q) at a config-4 chunk of gpt-oss-20b: (label,
# type, tokens, rows, columns).
MM_CASES = [
    ("attn_q Q8_0 2048 tokens x 4096 x 2880", 8, 2048, 4096, 2880),
    ("attn.proj Q8_0 2048 tokens x 2880 x 4096", 8, 2048, 2880, 4096),
    ("attn_q F16 2048 tokens x 4096 x 2880", 1, 2048, 4096, 2880),
]


def bench_matmul(ctx, hip, steps=5):
    """Each chunk product as a captured graph of `steps` launches (the activation split included),
    replayed once untimed and once between HIP events. TFLOP/s counts 2 * tokens * rows * cols;
    the kernel issues twice that on the f16 MFMA (the activation's hi and lo halves)."""
    from moearc_amd import QuantType
    res = {}
    rng = np.random.default_rng(0x33A)
    for label, ty, n_tok, rows, cols in MM_CASES:
        qt = QuantType(ty)
        nbytes = rows * qt.row_bytes(cols)
        if ty == 1:
            w = (rng.standard_normal(nbytes // 2) * 0.05).astype(np.float16).view(np.uint8)
        else:
            w = rng.integers(0, 256, nbytes, dtype=np.uint8).reshape(-1, 34)
            w[:, 0:2] = np.frombuffer(np.full(w.shape[0], 0x1800, np.uint16).tobytes(), np.uint8).reshape(-1, 2)
        dw = ctx.upload(w)
        dx = ctx.upload(rng.standard_normal((n_tok, cols)).astype(np.float32))
        db = ctx.upload(rng.standard_normal(rows).astype(np.float32))
        dy = ctx.alloc(n_tok * rows * 4)
        ctx.matmul_q(ty, dy, dw, dx, db, n_tok, rows, cols)
        ctx.sync()
        graph, exe = hip.capture(ctx.stream, lambda: [ctx.matmul_q(ty, dy, dw, dx, db, n_tok, rows, cols)
                                                      for _ in range(steps)])
        e0, e1 = hip.event(), hip.event()
        hip.launch(exe, ctx.stream)
        ctx.sync()
        hip.record(e0, ctx.stream)
        hip.launch(exe, ctx.stream)
        hip.record(e1, ctx.stream)
        ctx.sync()
        us = hip.elapsed_ms(e0, e1) * 1e3 / steps
        hip.destroy(graph, exe)
        tflops = 2.0 * n_tok * rows * cols / us / 1e6
        res[label] = {"us": round(us, 1), "tflops": round(tflops, 1),
                      "mfma_f16_frac_issued": round(2 * tflops / MFMA_F16_PEAK_TFLOPS, 4),
                      "us_per_token": round(us / n_tok, 3)}
    return res


def bench_block(ctx, hip, n_tok=128):
    """The attention half of one gpt-oss block (Q8_0 projections with biases, sinks, YaRN RoPE,
    f16 KV in 256-token pages) over a prompt of n_tok tokens: one moearc_attn_block_chunk call
    against n_tok single-token calls (the reference engine's shape of work, session.rs:378-381).
    Both timed between HIP events on the context's stream, host submission included (that is
    the engine's cost too)."""
    from moearc_amd import AttnBlockDesc, RopeScaling
    E, Hq, Gk = 2880, H, G
    rng = np.random.default_rng(0xB10C)
    shapes = [(Hq * D, E), (Gk * D, E), (Gk * D, E), (E, Hq * D)]
    ws = []
    for r, c in shapes:
        w = rng.integers(0, 256, r * c // 32 * 34, dtype=np.uint8).reshape(-1, 34)
        w[:, 0:2] = np.frombuffer(np.full(w.shape[0], 0x1800, np.uint16).tobytes(), np.uint8).reshape(-1, 2)
        ws.append(ctx.upload(w))
    bs = [ctx.upload((rng.standard_normal(r) * 0.1).astype(np.float32)) for r, _ in shapes]
    sinks = ctx.upload(rng.standard_normal(Hq).astype(np.float32))
    pages = (n_tok + PT - 1) // PT
    kp, vp = ctx.alloc(pages * PT * Gk * D * 2), ctx.alloc(pages * PT * Gk * D * 2)
    table = ctx.upload(np.arange(pages, dtype=np.uint32))
    desc = AttnBlockDesc.make([8] * 4, ws, bs, sinks, kp, vp, table, E, Hq, Gk, D, PT, 0, 0.125, D,
                              150000.0, RopeScaling.yarn(D, 4096, 150000.0, 32.0))
    x = ctx.upload((rng.standard_normal((n_tok, E)) * 0.05).astype(np.float32))
    h = ctx.upload(rng.standard_normal((n_tok, E)).astype(np.float32))
    pos = ctx.upload(np.arange(n_tok, dtype=np.int32))
    pg = ctx.upload((np.arange(n_tok) // PT).astype(np.uint32))
    sl = ctx.upload((np.arange(n_tok) % PT).astype(np.uint32))
    from moearc_amd import DeviceView
    views = [(DeviceView(h, t * E * 4, E * 4), DeviceView(x, t * E * 4, E * 4), DeviceView(pos, 4 * t, 4),
              DeviceView(pg, 4 * t, 4), DeviceView(sl, 4 * t, 4)) for t in range(n_tok)]
    res = {}
    for label in ("chunked", "token_by_token", "chunked"):
        ctx.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, ctx.stream)
        if label == "chunked":
            ctx.attn_block_chunk(desc, h, x, n_tok, 0, pos, pg, sl)
        else:
            for t, (hv, xv, pv, gv, sv) in enumerate(views):
                ctx.attn_block_chunk(desc, hv, xv, 1, t, pv, gv, sv)
        hip.record(e1, ctx.stream)
        ctx.sync()
        res[label] = hip.elapsed_ms(e0, e1) * 1e3
    return {"tokens": n_tok, "chunked_us": round(res["chunked"], 1),
            "token_by_token_us": round(res["token_by_token"], 1),
            "chunked_us_per_token": round(res["chunked"] / n_tok, 2),
            "token_by_token_us_per_token": round(res["token_by_token"] / n_tok, 2)}


def cpu_baseline(kp, vp, bt, q, sinks):
    """The oracle (f64, two-pass, sequential heads: the reference's CPU twin) on this host."""
    from oracle import oracle
    oracle.lib()
    bt1 = np.ascontiguousarray(bt, np.uint32)
    t0 = time.perf_counter()
    n = 0
    while True:  # single thread, as the reference runs it; a bounded ~10 s sample
        oracle.attn_decode(q, kp, vp, bt1, H, G, D, 0, N_KV, PT, 0.125, kv_type=1, sinks=sinks)
        n += 1
        if time.perf_counter() - t0 > 10.0 or n >= 40:
            break
    st_s = (time.perf_counter() - t0) / n
    threads = min(16, os.cpu_count() or 1)
    qb = q.reshape(1, H, D)
    kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
    t0 = time.perf_counter()
    m = 0
    while True:
        oracle.attn_decode_batched(qb, kp, vp, bt1.reshape(1, -1), kb, nk, H, G, D, PT, 0.125,
                                   sinks=sinks, n_threads=threads)
        m += 1
        if time.perf_counter() - t0 > 5.0 or m >= 200:
            break
    mt_s = (time.perf_counter() - t0) / m
    return {"single_us": st_s * 1e6, "single_calls": n, "mt_us": mt_s * 1e6, "mt_calls": m,
            "threads": threads}


def bench_configs(steps, warmup):
    """BASELINE configs 1, 3 and 5 (decode), reported one JSON line each; config 2 is the main line.
    K/V are random finite f16 bit patterns (|x| < 2) -- timing does not depend on their values --
    in 256-token pages. Each config touches more than the 256 MB Infinity Cache per replay cycle:
    config 1 rotates 40 contiguous copies, config 3 rotates 40 random block tables over a pool of
    every sequence's pages, config 5 reads 2 GiB per call. Algorithmic bytes: K/V read
    (2 KiB per key), q (16 KiB) and f16 out (8 KiB) per sequence, sinks, block-table entries."""
    from moearc_amd import Context, KvType, OUT_F16
    hip = Hip()
    rng = np.random.default_rng(0xD5)
    row = G * D

    def pages_of(n_pages):
        bits = rng.integers(0, 1 << 16, size=n_pages * PT * row, dtype=np.uint16)
        return bits & np.uint16(0xBFFF)  # exponent below 31: finite, |x| < 2

    def timed(ctx, step):
        for i in range(warmup):
            step(i)
        ctx.sync()
        graph, exe = hip.capture(ctx.stream, lambda: [step(i) for i in range(steps)])
        hip.launch(exe, ctx.stream)  # one untimed replay
        ctx.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, ctx.stream)
        hip.launch(exe, ctx.stream)
        hip.record(e1, ctx.stream)
        ctx.sync()
        us = hip.elapsed_ms(e0, e1) * 1e3 / steps
        hip.destroy(graph, exe)
        return us

    def emit(name, us, nbytes, b):
        gbs = nbytes / us / 1e3
        print(json.dumps({"config": name, "us_per_layer": round(us, 2), "algorithmic_bytes": nbytes,
                          "gbs": round(gbs, 1), "pct_peak_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                          "tokens_per_s": round(b * 1e6 / us, 0)}), flush=True)

    seq_bytes = H * D * 4 + H * D * 2  # q f32 in, f16 out
    with Context() as ctx:
        q32 = rng.standard_normal((32, H, D), dtype=np.float32)
        dq, ds = ctx.upload(q32), ctx.upload(rng.standard_normal(H, dtype=np.float32))

        # C1: B=1, 4096 keys, contiguous pages
        n1 = 4096
        copies = 40
        dk1 = [ctx.upload(pages_of(n1 // PT)) for _ in range(copies)]
        dv1 = [ctx.upload(pages_of(n1 // PT)) for _ in range(copies)]
        dbt1 = ctx.upload(np.arange(n1 // PT, dtype=np.uint32))
        out1 = ctx.alloc(H * D * 2)
        kb1, nk1 = np.zeros(1, np.uint32), np.full(1, n1, np.uint32)
        us = timed(ctx, lambda i: ctx.attn_decode_batched(out1, dq, dk1[i % copies], dv1[i % copies], dbt1,
                                                          n1 // PT, kb1, nk1, ds, H, G, D, PT, 0.125,
                                                          KvType.F16, out_type=OUT_F16))
        emit("C1 decode B=1, 4096 keys, full, contiguous pages", us,
             n1 * 2 * row * 2 + seq_bytes + H * 4 + 4 * (n1 // PT), 1)
        del dk1, dv1

        # C3: B=32, lengths ~U[1024, 32768], random page tables, SWA-128 and full
        lens = np.random.default_rng(33).integers(1024, 32769, size=32).astype(np.uint32)
        npg = [-(-int(n) // PT) for n in lens]
        pool = sum(npg)
        dk3, dv3 = ctx.upload(pages_of(pool)), ctx.upload(pages_of(pool))
        stride = max(npg)
        bts = []
        for _ in range(copies):
            perm = rng.permutation(pool).astype(np.uint32)
            t = np.zeros((32, stride), np.uint32)
            off = 0
            for s, p in enumerate(npg):
                t[s, :p] = perm[off:off + p]
                off += p
            bts.append(ctx.upload(t))
        out3 = ctx.alloc(32 * H * D * 2)
        for window in (0, 128):
            kb = np.maximum(lens.astype(np.int64) - window, 0).astype(np.uint32) if window else np.zeros_like(lens)
            span = (lens.astype(np.int64) - kb.astype(np.int64))
            first, last = kb.astype(np.int64) // PT, (lens.astype(np.int64) - 1) // PT
            us = timed(ctx, lambda i: ctx.attn_decode_batched(out3, dq, dk3, dv3, bts[i % copies], stride, kb,
                                                              lens, ds, H, G, D, PT, 0.125, KvType.F16,
                                                              out_type=OUT_F16))
            emit(f"C3 decode B=32 ragged U[1024,32768], {'SWA-128' if window else 'full'}", us,
                 int(span.sum()) * 2 * row * 2 + 32 * seq_bytes + H * 4 + 4 * int((last - first + 1).sum()), 32)
        del dk3, dv3, bts

        # C5: B=8 x 131072 keys, full
        n5, b5 = 131072, 8
        p5 = n5 // PT
        dk5, dv5 = ctx.upload(pages_of(b5 * p5)), ctx.upload(pages_of(b5 * p5))
        dbt5 = ctx.upload(rng.permutation(b5 * p5).astype(np.uint32).reshape(b5, p5))
        out5 = ctx.alloc(b5 * H * D * 2)
        kb5, nk5 = np.zeros(b5, np.uint32), np.full(b5, n5, np.uint32)
        us = timed(ctx, lambda i: ctx.attn_decode_batched(out5, dq, dk5, dv5, dbt5, p5, kb5, nk5, ds, H, G, D,
                                                          PT, 0.125, KvType.F16, out_type=OUT_F16))
        emit("C5 decode B=8 x 131072 keys, full", us, b5 * n5 * 2 * row * 2 + b5 * seq_bytes + H * 4 + 4 * b5 * p5, b5)


def only(what, steps, warmup):
    """Runs one workload eagerly with no timing of its own, for rocprofv3 to wrap:
    decode (C2), prefill (C4 full then SWA-128), rope_append (the fused RoPE-K + K/V append of one
    C4 chunk), matvec (the projection cases of MV_CASES, in order), matmul (MM_CASES, each as
    a graph of `steps` launches, replayed twice), or copy (a 256 MiB device-to-device copy, the
    reference size for scaling FETCH_SIZE/WRITE_SIZE readings to bytes)."""
    from moearc_amd import Context, KvType, OUT_F16
    with Context() as ctx:
        if what == "decode":
            kp, vp, bt, q, sinks = decode_inputs()
            dks = [ctx.upload(kp) for _ in range(COPIES)]
            dvs = [ctx.upload(vp) for _ in range(COPIES)]
            dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
            dout = ctx.alloc(H * D * 2)
            kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
            for i in range(warmup + steps):
                ctx.attn_decode_batched(dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT,
                                        kb, nk, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)
        elif what == "prefill":
            import fixtures as fx
            pc = fx.prefill_case(0xC4, n_q=PF_NQ, pos0=PF_POS0, pt=PT)
            dk, dv, dbt, ds = ctx.upload(pc.k_raw), ctx.upload(pc.v_raw), ctx.upload(pc.bt), ctx.upload(pc.sinks)
            dq = ctx.upload(np.ascontiguousarray(pc.qp).view(np.uint16))
            dout = ctx.alloc(PF_NQ * H * D * 2)
            for n_swa in (0, 128):
                for i in range(warmup + steps):
                    ctx.attn_prefill(dout, dq, dk, dv, dbt, ds, PF_NQ, PF_POS0, n_swa, H, G, D, PT,
                                     0.125, KvType.F16, out_type=OUT_F16)
        elif what == "rope_append":
            sets, meta = rope_append_inputs(ctx, 24)
            for i in range(warmup + steps):
                rope_append_launch(ctx, sets, meta, i)
        elif what == "matvec":
            for label, ty, rows, cols, fused in MV_CASES:
                inputs = mv_inputs(ctx, ty, rows, cols, fused, 128)
                for i in range(warmup + steps):
                    mv_launch(ctx, ty, rows, cols, fused, inputs, i)
                ctx.sync()
                del inputs
        elif what == "matmul":
            hip = Hip()
            bench_matmul(ctx, hip, steps=steps)
        elif what == "copy":
            hip = Hip()
            n = 256 << 20
            src, dst = ctx.alloc(n), ctx.alloc(n)
            ctx.zero(src, n // 4)
            for i in range(warmup + steps):
                hip.ok(hip.lib.hipMemcpyDtoDAsync(ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr),
                                                  ctypes.c_size_t(n), ctypes.c_void_p(ctx.stream)),
                       "hipMemcpyDtoDAsync")
        ctx.sync()
    print(f"ran {what}: {warmup + steps} launches", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--only", choices=["decode", "prefill", "rope_append", "matvec", "matmul", "copy"],
                    help="run one workload without timing, for rocprofv3 to wrap")
    ap.add_argument("--configs", action="store_true",
                    help="time BASELINE configs 1, 3 and 5 instead (one JSON line each)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus "
              f"{args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("RANK", "0")) != 0:
        return
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    if args.only:
        only(args.only, args.steps, args.warmup)
        return
    if args.configs:
        bench_configs(args.steps, args.warmup)
        return
    r = run(args.steps, args.warmup, args.skip_cpu, args.skip_prefill)

    step_us = r["step_us_gpu"]
    gbs = C2_BYTES / step_us / 1e3
    split_us = r["events"].get("attn_decode.split r64 m64")
    ach = C2_BYTES / split_us / 1e3 if split_us else None
    # parity spot check against the oracle (f64) on the same inputs
    from oracle import oracle
    kp, vp, bt, q, sinks = decode_inputs()
    want = oracle.attn_decode(q, kp, vp, bt, H, G, D, 0, N_KV, PT, 0.125, kv_type=1, sinks=sinks)
    err = float(np.max(np.abs(r["out"].ravel() - want)))
    traffic = pmc_traffic(os.path.join(ROOT, "profiles", "decode_c2_pmc.md"))
    line = {
        "metric": "decode attn µs/layer + HBM GB/s (% peak) at B=1, 32K ctx; prefill MFMA util",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) q/K/V, f16 KV; no model)",
        "config": {
            "workload": "C2 decode: B=1, 32768 keys, 64q/8kv heads, head_dim 64, f16 KV in 256-token "
                        "pages (random permutation), per-head f32 sinks, full causal, f16 out",
            "global_batch": 1, "seq_len": N_KV, "parallelism": "single GPU",
        },
        "us_per_layer": round(step_us, 2),
        "us_per_layer_wall": round(r["step_us_wall"], 2),
        "pct_peak_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
        "tokens_per_s": round(1e6 / step_us, 0),
        "kernel_us": {k: round(v, 2) for k, v in r["events"].items()},
        "graph_replay_equals_eager": r["graph_equals_eager"],
        "parity_max_abs_err": err,
        "roofline": {
            "bound": "hbm",
            "achieved": round(ach, 1) if ach else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4) if ach else None,
            "traffic": traffic,
            "kernel": "moearc_attn_decode_f16d64 (split-K)",
            "bytes_per_launch": C2_BYTES,
        },
    }
    if "prefill" in r:
        line["prefill"] = r["prefill"]
    if "projections" in r:
        line["projections"] = r["projections"]
    if "block_chunk" in r:
        line["block_chunk"] = r["block_chunk"]
    if "chunk_projections" in r:
        line["chunk_projections"] = r["chunk_projections"]
    if "cpu" in r:
        c = r["cpu"]
        line["cpu_baseline"] = {
            "value": round(C2_BYTES / c["single_us"] / 1e3, 3),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"C2 decode, {c['single_calls']} calls of the f64 oracle, one thread "
                      f"({c['single_us'] / 1e3:.1f} ms/call)",
            "multithread": {"threads": c["threads"], "us_per_call": round(c["mt_us"], 1),
                            "value": round(C2_BYTES / c["mt_us"] / 1e3, 3)},
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
