"""Benchmark of the attention hot path on one MI355X; prints one JSON line.

Workload (the config the metric is quoted on): single-sequence decode,
B=1, 32768 keys, 64 query heads over 8 KV heads, head_dim 64, f16 KV in 256-token pages through a
random page permutation, per-head f32 sinks, full causal, f16 output. A step is one attention layer
call (the split-K launch and the merge launch). Inputs are N(0,1) from a seed (synthetic data;
there is no model).

* Timed region: K steps captured in one HIP graph on the library's stream and replayed, bracketed
  by stream synchronisations; every step reads a different one of 8 KV copies (512 MiB) so the
  256 MB Infinity Cache cannot serve repeats. The replay is repeated REPS times (the first
  discarded, bench/PROTOCOL.md:73-87); value = algorithmic bytes per step / median step time.
* roofline: the whole call (split + merge) at the replay's step time, against 8 TB/s; frac_split
  beside it from the split launch alone (HIP events on the library stream, eager, with
  MOEARC_PROFILE_KERNELS=1). traffic = HBM bytes per call from the committed rocprofv3
  FETCH_SIZE/WRITE_SIZE summary (profiles/decode_c2_pmc.md), when present.
* read_floor: a plain streaming read of the same 64 MiB (moearc_read_floor, every load of a lane
  in flight, over the same rotating copies and graph replay): what reading the call's bytes alone
  costs on this device; decode_frac_of_floor = its time over the decode call's.
* configs: BASELINE configs 1, 3 (SWA-128 and full) and 5, timed the same way.
* prefill: BASELINE config 4 (2048 new + 2048 cached tokens), full causal and SWA-128, timed as
  the decode (8 calls in one graph, replayed REPS times, the median per call); MFMA utilisation =
  algorithmic flops / time / 2.5 PFLOP/s (dense f16), SWA-128 also against max(bytes / 8 TB/s,
  flops / 2.5 PF); also as top-level keys. Beside it: per-call HIP-event timing (us_events) and
  the committed trace's kernel duration (us_trace, profiles/prefill_c4_kernel_trace.md).
* rope_kv_append_chunk: the fused RoPE-K + f16 K/V append of the same config-4 chunk, timed by
  graph replay (24 calls over 24 input sets), with event timing and the committed trace beside it.
* launch_overhead: moearc_amd/launch_overhead (examples/launch_overhead.rs:21-125 over the C ABI).
* cpu_baseline: the CPU oracle (a C restatement of the reference's f64 CPU twin,
  reference.rs:821-873, plus the sink) timed on this host on a bounded sample of the same decode,
  single thread as the reference runs it, REPS invocations after a discarded first, with the
  1-minute load average read before each, nproc and the CPU model stated; plus an OpenMP figure.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10]
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import math
import os
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA
H, G, D, PT = 64, 8, 64, 256
N_KV = 32768
COPIES = 8
REPS = 6  # timed repetitions; the first is discarded

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


def summary_value(path, key):
    """A `key value` line of a committed rocprofv3 summary under profiles/, or None."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(key + " "):
            return float(line.split()[1])
    return None


def pmc_traffic(path):
    """HBM bytes per decode call (split + merge) from the committed rocprofv3 summary."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_call"):
            return float(line.split()[1])
    return None


def rep_stats(xs):
    """mean, sd, median over the repetitions after the first (bench/PROTOCOL.md:73-87)."""
    kept = xs[1:] if len(xs) > 1 else xs
    return {"n": len(kept), "mean": round(statistics.mean(kept), 3),
            "sd": round(statistics.stdev(kept), 3) if len(kept) > 1 else 0.0,
            "median": round(statistics.median(kept), 3), "all": [round(x, 3) for x in xs]}


def graph_timed(hip, ctx, step, steps, warmup, reps=REPS):
    """Per-step microseconds of `steps` calls captured in one graph, replayed `reps` times."""
    for i in range(warmup):
        step(i)
    ctx.sync()
    graph, exe = hip.capture(ctx.stream, lambda: [step(i) for i in range(steps)])
    hip.launch(exe, ctx.stream)  # one untimed replay
    ctx.sync()
    out = []
    for _ in range(reps):
        e0, e1 = hip.event(), hip.event()
        ctx.sync()
        hip.record(e0, ctx.stream)
        hip.launch(exe, ctx.stream)
        hip.record(e1, ctx.stream)
        ctx.sync()
        out.append(hip.elapsed_ms(e0, e1) * 1e3 / steps)
    hip.destroy(graph, exe)
    return out


def run(steps, warmup, skip_cpu=False, skip_prefill=False):
    from moearc_amd import Context, KvType, OUT_F16

    hip = Hip()
    kp, vp, bt, q, sinks = decode_inputs()
    result = {}

    with Context() as ctx:
        result["device"] = ctx.device_name()
        dks = [ctx.upload(kp) for _ in range(COPIES)]
        dvs = [ctx.upload(vp) for _ in range(COPIES)]
        dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
        dout = ctx.alloc(H * D * 2)
        kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)

        def step(i):
            ctx.attn_decode_batched(dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT, kb,
                                    nk, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)

        step(0)
        ctx.sync()
        eager_out = ctx.download(dout, np.float16, (H, D)).astype(np.float32)
        t0 = time.perf_counter()
        result["step_us_reps"] = graph_timed(hip, ctx, step, steps, warmup)
        result["wall_s"] = time.perf_counter() - t0
        graph_out = ctx.download(dout, np.float16, (H, D)).astype(np.float32)
        result["graph_equals_eager"] = bool(np.array_equal(graph_out, eager_out))
        result["out"] = graph_out
        del dks, dvs
        result["read_floor"] = bench_read_floor(ctx, hip, steps, warmup)
        # the prefill before the MFMA-heavy chunk products: its full-causal kernel is power-limited,
        # and right after them it measures ~15% slower
        if not skip_prefill:
            result["prefill_graph"] = bench_prefill_graph(ctx, hip)
            result["mfma_floor"] = bench_mfma_floor(ctx, hip)
            result["rope_graph"] = bench_rope_append_graph(ctx, hip)
        result["configs"] = bench_configs(ctx, hip, steps, warmup)
        result["headline_step"] = bench_headline(ctx, hip)
        result["projections"] = bench_matvec(ctx, hip, steps=max(20, steps))
        result["block_chunk"] = bench_block(ctx, hip)
        result["chunk_projections"] = bench_matmul(ctx, hip)

    # per-kernel event timing (eager): the call under the reference's key, its launches apart
    os.environ["MOEARC_PROFILE_KERNELS"] = "1"
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
            del dks, dvs
            if not skip_prefill:
                result["prefill"] = bench_prefill(ctx, steps=max(5, steps // 5), warmup=3,
                                                  graph=result.get("prefill_graph"),
                                                  rope_graph=result.get("rope_graph"))
    finally:
        os.environ.pop("MOEARC_PROFILE_KERNELS", None)

    result["launch_overhead"] = launch_overhead()
    if not skip_cpu:
        result["cpu"] = cpu_baseline(kp, vp, bt, q, sinks)
        if not skip_prefill:
            result["cpu_prefill"] = cpu_prefill_baseline()
    return result


def read_floor_inputs(ctx, copies=COPIES):
    """COPIES buffers of C2's KV bytes (K then V of copy i), for the calibration read."""
    from moearc_amd import DeviceView
    kp, vp, _, _, _ = decode_inputs()
    nbytes = kp.nbytes + vp.nbytes
    bufs = []
    for _ in range(copies):
        b = ctx.alloc(nbytes)
        ctx.upload_slice(DeviceView(b, 0, kp.nbytes), kp)
        ctx.upload_slice(DeviceView(b, kp.nbytes, vp.nbytes), vp)
        bufs.append(b)
    out = ctx.alloc((nbytes + 65535) // 65536 * 4)
    return bufs, out, nbytes


def bench_read_floor(ctx, hip, steps, warmup):
    """The plain read of C2's 64 MiB of KV (moearc_read_floor: every load of a lane in flight, 64 KiB
    per work-group) over the same rotating copies and graph replay as the decode: what a streaming
    read of those bytes costs on this device, the floor under the decode call's time."""
    bufs, out, nbytes = read_floor_inputs(ctx)
    ctx.read_floor(out, bufs[0], nbytes)
    ctx.sync()
    got = ctx.download(out, np.uint32, (nbytes + 65535) // 65536)
    kp, vp = decode_inputs()[:2]
    host = np.concatenate([kp.view(np.uint8).ravel(), vp.view(np.uint8).ravel()]).view(np.uint32)
    want = np.bitwise_xor.reduce(host.reshape(-1, 16384), axis=1)
    reps = graph_timed(hip, ctx, lambda i: ctx.read_floor(out, bufs[i % COPIES], nbytes), steps, warmup)
    st = rep_stats(reps)
    # the same read followed by a dependent one-work-group launch (a 64-float fill), as the decode
    # call's split launch is followed by its merge; and that tiny launch alone, back to back
    tiny = ctx.alloc(64 * 4)

    def chain(i):
        ctx.read_floor(out, bufs[i % COPIES], nbytes)
        ctx.zero(tiny, 64)
    ch = rep_stats(graph_timed(hip, ctx, chain, steps, warmup))
    tl = rep_stats(graph_timed(hip, ctx, lambda i: ctx.zero(tiny, 64), steps, warmup))
    del bufs
    return {"bytes": nbytes, "us": st["median"], "us_reps": st,
            "gbs": round(nbytes / st["median"] / 1e3, 1),
            "frac_of_peak": round(nbytes / st["median"] / 1e3 / HBM_PEAK_GBS, 4),
            "checksums_match": bool(np.array_equal(got, want)),
            "with_dependent_launch_us": ch["median"], "with_dependent_launch_reps": ch,
            "dependent_launch_us": round(ch["median"] - st["median"], 3),
            "tiny_launch_alone_us": tl["median"], "tiny_launch_alone_reps": tl}


def launch_overhead():
    """The reference's launch-overhead example (examples/launch_overhead.rs) over the C ABI."""
    exe = os.path.join(ROOT, "moearc_amd", "launch_overhead")
    if not os.path.exists(exe):
        return None
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    if res.returncode != 0:
        return {"error": res.stderr.strip()[-200:]}
    return json.loads(res.stdout.strip().splitlines()[-1])


# independent config-4 input sets the prefill timings rotate over: 12 x (16 MiB q + 2 x 4 MiB K/V)
# = 288 MiB, more than the 256 MB Infinity Cache, so no call is served its inputs from that cache
PF_SETS = 12


def prefill_inputs(ctx, copies=PF_SETS):
    """Config-4 prefill inputs (tests/fixtures.py: the same seeded case the parity tests use), in
    `copies` independent sets of q, K and V."""
    import fixtures as fx
    pc = fx.prefill_case(0xC4, n_q=PF_NQ, pos0=PF_POS0, pt=PT)
    dks = [ctx.upload(pc.k_raw) for _ in range(copies)]
    dvs = [ctx.upload(pc.v_raw) for _ in range(copies)]
    dqs = [ctx.upload(np.ascontiguousarray(pc.qp).view(np.uint16)) for _ in range(copies)]
    return dks, dvs, dqs, ctx.upload(pc.bt), ctx.upload(pc.sinks), ctx.alloc(PF_NQ * H * D * 2)


def bench_prefill_graph(ctx, hip, calls=PF_SETS, warmup=3):
    """Both config-4 layers timed as the decode is: `calls` calls (each on its own input set,
    PF_SETS of them) captured in one graph and replayed REPS times; per-call µs statistics, the
    first replay discarded. Close to the kernel's own duration (one dispatch gap per call)."""
    from moearc_amd import KvType, OUT_F16
    dks, dvs, dqs, dbt, ds, dout = prefill_inputs(ctx)
    n_sets = len(dks)
    out = {}
    for name, n_swa in (("full", 0), ("swa128", 128)):
        def call(i, n_swa=n_swa):
            ctx.attn_prefill(dout, dqs[i % n_sets], dks[i % n_sets], dvs[i % n_sets], dbt, ds, PF_NQ,
                             PF_POS0, n_swa, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)
        out[name] = rep_stats(graph_timed(hip, ctx, call, calls, warmup))
    return out


# Matrix-core calibration beside the prefill: 512 work-groups of 4 waves (the prefill's grid and two
# waves per SIMD), MF_ITERS rounds of 8 v_mfma_f32_32x32x16_f16 per wave on N(0,1) f16 operands, so a
# call does about as much matrix work as the full-causal prefill and runs as long.
MF_WGS, MF_ITERS = 512, 384
MF_FLOPS = MF_WGS * 4 * MF_ITERS * 8 * 32768


def bench_mfma_floor(ctx, hip, calls=12, warmup=3):
    """moearc_mfma_floor timed as the prefill is (graph replay of `calls` calls, REPS replays, the
    first discarded): the f16 MFMA rate this device sustains on data like the prefill's, with the
    clock the power limit leaves it. Returns µs statistics and TFLOP/s."""
    rng = np.random.default_rng(0xF100)
    out = ctx.alloc(MF_WGS * 16)
    res = {}
    for name, data in (("normal", rng.standard_normal(MF_WGS * 16384).astype(np.float16)),
                       ("zeros", np.zeros(MF_WGS * 16384, np.float16))):
        src = ctx.upload(data)
        st = rep_stats(graph_timed(hip, ctx, lambda i: ctx.mfma_floor(out, src, MF_WGS, MF_ITERS), calls, warmup))
        tflops = MF_FLOPS / st["median"] / 1e6
        res[name] = {"us": round(st["median"], 2), "us_reps": st, "tflops": round(tflops, 1),
                     "frac_of_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        del src
    return {**res["normal"], "flops": MF_FLOPS, "zero_operands": res["zeros"],
            "note": "moearc_mfma_floor: dense 32x32x16 f16 MFMA chains, 512 x 4 waves (two per SIMD, the "
                    "prefill's occupancy), on N(0,1) operands (the practical MFMA ceiling for the "
                    "prefill's data) and on zero operands (the same instructions with little switching: "
                    "the gap is the power limit's clock)"}


def bench_prefill(ctx, steps, warmup, graph=None, rope_graph=None):
    """Config-4 prefill: per-call HIP-event timing (eager, under the reference's key), and -- when
    `graph` holds bench_prefill_graph's statistics -- the headline from the graph replay, with the
    committed trace's kernel duration under the same replay beside it (us_trace)."""
    from moearc_amd import KvType, OUT_F16
    dks, dvs, dqs, dbt, ds, dout = prefill_inputs(ctx)
    copies = len(dks)
    trace_path = os.path.join(ROOT, "profiles", "prefill_c4_kernel_trace.md")
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
        us_events = rep["attn_prefill r64 m64"][0] / rep["attn_prefill r64 m64"][1] / 1e3
        us = graph[name]["median"] if graph else us_events
        flops = PF_FLOPS_FULL if n_swa == 0 else PF_FLOPS_SWA
        bound_us = max(PF_BYTES_SWA / (HBM_PEAK_GBS * 1e3), flops / (MFMA_F16_PEAK_TFLOPS * 1e6))

        def fracs(t):
            f = {"mfma_util": round(flops / t / 1e6 / MFMA_F16_PEAK_TFLOPS, 4)}
            if n_swa:
                f["roofline_frac"] = round(bound_us / t, 4)
            return f
        tflops = flops / us / 1e6
        entry = {"us": round(us, 2), "timing": "graph replay, median per call" if graph else "HIP events",
                 "tflops": round(tflops, 1), **fracs(us), "tokens_per_s": round(PF_NQ * 1e6 / us, 0),
                 "us_events": round(us_events, 2)}
        if graph:
            entry["us_reps"] = graph[name]
        if n_swa:
            entry["hbm_gbs"] = round(PF_BYTES_SWA / us / 1e3, 0)
        tr = summary_value(trace_path, f"{name}_us_trace_graph")
        if tr:
            entry["us_trace"] = tr
            entry.update({k + "_trace": v for k, v in fracs(tr).items()})
        out[name] = entry
    out["rope_kv_append_chunk"] = bench_rope_append(ctx, steps, warmup, rope_graph)
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


def bench_rope_append_graph(ctx, hip):
    """The fused RoPE-K + f16 K/V append: 24 calls over 24 input sets in one graph, replayed REPS
    times; per-call µs statistics, the first replay discarded."""
    sets, meta = rope_append_inputs(ctx, 24)
    return rep_stats(graph_timed(hip, ctx, lambda i: rope_append_launch(ctx, sets, meta, i), 24, 3))


def bench_rope_append(ctx, steps, warmup, graph=None):
    """The fused RoPE-K + f16 K/V append (HBM-bound): the library's per-call event timing and, when
    `graph` holds bench_rope_append_graph's statistics, the headline from the graph replay; the
    committed trace's kernel duration beside them."""
    sets, meta = rope_append_inputs(ctx, 24)
    for i in range(warmup + steps):
        if i == warmup:
            ctx.sync()
            ctx.profile_events_reset()
        rope_append_launch(ctx, sets, meta, i)
    ctx.sync()
    rep = ctx.profile_events_report()
    key = [k2 for k2 in rep if k2.startswith("rope_kv_append_chunk")][0]
    us_events = rep[key][0] / rep[key][1] / 1e3
    out = {"bytes": RA_BYTES, "us_events": round(us_events, 2)}
    us = us_events
    if graph:
        us = graph["median"]
        out["us_reps"] = graph
    gbs = RA_BYTES / us / 1e3
    out.update({"us": round(us, 2), "timing": "graph replay, median per call" if graph else "HIP events",
                "hbm_gbs": round(gbs, 0), "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)})
    tr = summary_value(os.path.join(ROOT, "profiles", "rope_append_c4_kernel_trace.md"), "rope_append_us_trace")
    if tr:
        out["us_trace"] = tr
        out["roofline_frac_trace"] = round(RA_BYTES / tr / 1e3 / HBM_PEAK_GBS, 4)
    return out


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
    replayed REPS times (the first discarded, bench/PROTOCOL.md:73-87): the per-launch time excludes
    host submission, which for kernels this short would otherwise dominate. `us` is the median over
    the repetitions; achieved bandwidth counts the algorithmic bytes (every weight byte once, the
    activation, biases and outputs)."""
    res = {}
    for label, ty, rows, cols, fused in MV_CASES:
        inputs = mv_inputs(ctx, ty, rows, cols, fused, 128)
        st = rep_stats(graph_timed(hip, ctx, lambda i: mv_launch(ctx, ty, rows, cols, fused, inputs, i),
                                   steps, 2))
        us = st["median"]
        nbytes = inputs[4] + cols * 4 + sum(rows) * 4 * (2 if fused else 1)
        gbs = nbytes / us / 1e3
        res[label] = {"us": round(us, 2), "us_reps": st, "bytes": nbytes, "hbm_gbs": round(gbs, 0),
                      "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}
        del inputs
    return res


# Chunk-form projections on MFMA (moearc_matmul_q) at a config-4 chunk of gpt-oss-20b: (label,
# type, tokens, rows, columns).
MM_CASES = [
    ("attn_q Q8_0 2048 tokens x 4096 x 2880", 8, 2048, 4096, 2880),
    ("attn.proj Q8_0 2048 tokens x 2880 x 4096", 8, 2048, 2880, 4096),
    ("attn_q F16 2048 tokens x 4096 x 2880", 1, 2048, 4096, 2880),
    ("attn_q MXFP4 2048 tokens x 4096 x 2880", 39, 2048, 4096, 2880),
    # Qwen3-30B-A3B's attn_q (Q4_K in its Q4_K_M files) over a chunk of the same length
    ("attn_q Q4_K qwen3-30b 2048 tokens x 4096 x 2048", 12, 2048, 4096, 2048),
]


def mm_weights(rng, ty, rows, cols):
    """Synthetic weights of one format: random payload bytes, block scales set to small normal
    f16 values (so no block is inf or NaN), MXFP4 exponents near 2^0."""
    from moearc_amd import QuantType
    qt = QuantType(ty)
    nbytes = rows * qt.row_bytes(cols)
    if ty == 1:
        return (rng.standard_normal(nbytes // 2) * 0.05).astype(np.float16).view(np.uint8)
    w = rng.integers(0, 256, nbytes, dtype=np.uint8).reshape(-1, qt.block_bytes)
    f16 = lambda v: np.frombuffer(np.full(w.shape[0], v, np.uint16).tobytes(), np.uint8).reshape(-1, 2)
    if ty == 8:
        w[:, 0:2] = f16(0x1800)
    elif ty in (12, 13):
        w[:, 0:2] = f16(0x1800)
        w[:, 2:4] = f16(0x1400)
    elif ty == 14:
        w[:, 208:210] = f16(0x1800)
    elif ty == 39:
        w[:, 0] = 120
    return w.reshape(-1)


def bench_matmul(ctx, hip, steps=5):
    """Each chunk product as a captured graph of `steps` launches (the activation split included),
    replayed REPS times (the first discarded); `us` is the median per launch. TFLOP/s counts
    2 * tokens * rows * cols; the kernel issues twice that on the f16 MFMA (the activation's hi and
    lo halves)."""
    res = {}
    rng = np.random.default_rng(0x33A)
    for label, ty, n_tok, rows, cols in MM_CASES:
        dw = ctx.upload(mm_weights(rng, ty, rows, cols))
        dx = ctx.upload(rng.standard_normal((n_tok, cols)).astype(np.float32))
        db = ctx.upload(rng.standard_normal(rows).astype(np.float32))
        dy = ctx.alloc(n_tok * rows * 4)
        st = rep_stats(graph_timed(hip, ctx, lambda i: ctx.matmul_q(ty, dy, dw, dx, db, n_tok, rows, cols),
                                   steps, 1))
        us = st["median"]
        tflops = 2.0 * n_tok * rows * cols / us / 1e6
        res[label] = {"us": round(us, 1), "us_reps": st, "tflops": round(tflops, 1),
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
    res = {"chunked": [], "token_by_token": []}
    for _ in range(REPS):  # alternating, each REPS times; the first of each discarded
        for label in ("chunked", "token_by_token"):
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
            res[label].append(hip.elapsed_ms(e0, e1) * 1e3)
    ch, tbt = rep_stats(res["chunked"]), rep_stats(res["token_by_token"])
    return {"tokens": n_tok, "timing": "HIP events around the call, host submission included; "
            "median of REPS repetitions after a discarded first",
            "chunked_us": round(ch["median"], 1), "chunked_us_reps": ch,
            "token_by_token_us": round(tbt["median"], 1), "token_by_token_us_reps": tbt,
            "chunked_us_per_token": round(ch["median"] / n_tok, 2),
            "token_by_token_us_per_token": round(tbt["median"] / n_tok, 2)}


def host_info():
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": model}


def cpu_baseline(kp, vp, bt, q, sinks):
    """The oracle (f64, two-pass, sequential heads: the reference's CPU twin) on this host, after
    bench/PROTOCOL.md:50-58 and :73-87: REPS invocations of a bounded sample (the first discarded),
    the 1-minute load average read before each, mean +- sd and median reported."""
    from oracle import oracle
    oracle.lib()
    bt1 = np.ascontiguousarray(bt, np.uint32)
    calls_per_rep = 2
    single, loads = [], []
    for _ in range(REPS):  # single thread, as the reference runs it
        loads.append(os.getloadavg()[0])
        t0 = time.perf_counter()
        for _ in range(calls_per_rep):
            oracle.attn_decode(q, kp, vp, bt1, H, G, D, 0, N_KV, PT, 0.125, kv_type=1, sinks=sinks)
        single.append((time.perf_counter() - t0) / calls_per_rep * 1e6)
    threads = min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1)
    qb = q.reshape(1, H, D)
    kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
    multi = []
    for _ in range(REPS):
        t0 = time.perf_counter()
        for _ in range(4):
            oracle.attn_decode_batched(qb, kp, vp, bt1.reshape(1, -1), kb, nk, H, G, D, PT, 0.125,
                                       sinks=sinks, n_threads=threads)
        multi.append((time.perf_counter() - t0) / 4 * 1e6)
    return {"single_us": rep_stats(single), "calls_per_rep": calls_per_rep, "loadavg_1m": loads,
            "mt_us": rep_stats(multi), "threads": threads, **host_info()}


def bench_configs(ctx, hip, steps, warmup):
    """BASELINE configs 1, 3 (SWA-128 and full) and 5 (decode); config 2 is the main line.
    K/V are random finite f16 bit patterns (|x| < 2) -- timing does not depend on their values --
    in 256-token pages. Each config touches more than the 256 MB Infinity Cache per replay cycle:
    config 1 rotates 40 contiguous copies, config 3 rotates 40 random block tables over a pool of
    every sequence's pages, config 5 reads 2 GiB per call. Algorithmic bytes: K/V read
    (2 KiB per key), q (16 KiB) and f16 out (8 KiB) per sequence, sinks, block-table entries.
    Each entry: median step time over REPS graph replays (the first discarded)."""
    from moearc_amd import KvType, OUT_F16
    rng = np.random.default_rng(0xD5)
    row = G * D
    out = {}

    def pages_of(n_pages):
        bits = rng.integers(0, 1 << 16, size=n_pages * PT * row, dtype=np.uint16)
        return bits & np.uint16(0xBFFF)  # exponent below 31: finite, |x| < 2

    def emit(name, reps, nbytes, b):
        st = rep_stats(reps)
        us = st["median"]
        gbs = nbytes / us / 1e3
        out[name] = {"us_per_layer": round(us, 2), "us_reps": st, "algorithmic_bytes": nbytes,
                     "gbs": round(gbs, 1), "pct_peak_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                     "tokens_per_s": round(b * 1e6 / us, 0)}

    seq_bytes = H * D * 4 + H * D * 2  # q f32 in, f16 out
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
    reps = graph_timed(hip, ctx, lambda i: ctx.attn_decode_batched(
        out1, dq, dk1[i % copies], dv1[i % copies], dbt1, n1 // PT, kb1, nk1, ds, H, G, D, PT, 0.125,
        KvType.F16, out_type=OUT_F16), steps, warmup)
    emit("C1 decode B=1, 4096 keys, full, contiguous pages", reps,
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
        for s_, p in enumerate(npg):
            t[s_, :p] = perm[off:off + p]
            off += p
        bts.append(ctx.upload(t))
    out3 = ctx.alloc(32 * H * D * 2)
    for window in (128, 0):
        kb = np.maximum(lens.astype(np.int64) - window, 0).astype(np.uint32) if window else np.zeros_like(lens)
        span = (lens.astype(np.int64) - kb.astype(np.int64))
        first, last = kb.astype(np.int64) // PT, (lens.astype(np.int64) - 1) // PT
        reps = graph_timed(hip, ctx, lambda i: ctx.attn_decode_batched(
            out3, dq, dk3, dv3, bts[i % copies], stride, kb, lens, ds, H, G, D, PT, 0.125, KvType.F16,
            out_type=OUT_F16), steps, warmup)
        emit(f"C3 decode B=32 ragged U[1024,32768], {'SWA-128' if window else 'full'}", reps,
             int(span.sum()) * 2 * row * 2 + 32 * seq_bytes + H * 4 + 4 * int((last - first + 1).sum()), 32)
    del dk3, dv3, bts

    # C5: B=8 x 131072 keys, full
    n5, b5 = 131072, 8
    p5 = n5 // PT
    dk5, dv5 = ctx.upload(pages_of(b5 * p5)), ctx.upload(pages_of(b5 * p5))
    dbt5 = ctx.upload(rng.permutation(b5 * p5).astype(np.uint32).reshape(b5, p5))
    out5 = ctx.alloc(b5 * H * D * 2)
    kb5, nk5 = np.zeros(b5, np.uint32), np.full(b5, n5, np.uint32)
    reps = graph_timed(hip, ctx, lambda i: ctx.attn_decode_batched(
        out5, dq, dk5, dv5, dbt5, p5, kb5, nk5, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16),
        max(4, steps // 4), 2)
    emit("C5 decode B=8 x 131072 keys, full", reps, b5 * n5 * 2 * row * 2 + b5 * seq_bytes + H * 4 + 4 * b5 * p5, b5)
    del dk5, dv5
    return out


# The reference's own headline quantity for this path: `attn.attend` (the attention call of
# moe.rs:2043-2061) summed over one decode step of gpt-oss-120b's 36 blocks -- 18 with a 128-token
# sliding window, 18 full causal -- at B=1 and context depth d, measured on an Arc B580 with
# MOEARC_SYNC_EACH=1 (every call synchronised): 15.21 ms at 512 and 49.51 ms at 2048
# (bench/results/2026-09-06-moearc-sync-each.txt:17-18); 187.3 ms at 8192 is the reference's own
# extrapolation from its fit 3.77 + 0.02240 d ms (bench/baselines/gpt-oss-120b.md:626), not a
# measurement.
HEADLINE_DEPTHS = (512, 2048, 8192)
REF_ATTN_ATTEND_MS = {512: (15.21, "measured"), 2048: (49.51, "measured"),
                      8192: (187.3, "the reference's extrapolation 3.77 + 0.02240 d")}


def bench_headline(ctx, hip):
    """One decode step's 36 attention calls (blocks alternate SWA-128 and full causal, as gpt-oss
    declares its window on alternating blocks) at B=1 and depths 512, 2048 and 8192: 64 q / 8 KV
    heads, head_dim 64, f16 KV in 256-token pages, per-head sinks, f32 q and output (the engine's
    decode surface, moe.rs:2043-2061). Each full block reads its own pool through its own random
    page permutation; each windowed block its own two-page ring through the cyclic table (the
    window's 128 keys touch at most two consecutive pages). Enough independent sets of the 36
    blocks rotate for a replay cycle to touch more than 512 MiB, so the 256 MB Infinity Cache
    serves no repeats. Two protocols, each REPS repetitions with the first discarded:
    graph replay of the steps (device time per step, launches back to back) and sync-each (a
    host wall clock around every call and its stream synchronisation, summed over the step: the
    reference's MOEARC_SYNC_EACH=1 protocol, here with the Python binding's call overhead in
    it)."""
    from moearc_amd import KvType
    rng = np.random.default_rng(0x36B)
    row = G * D
    q = ctx.upload(rng.standard_normal(H * D).astype(np.float32))
    sinks = [ctx.upload(rng.standard_normal(H).astype(np.float32)) for _ in range(36)]
    out = ctx.alloc(H * D * 4)
    bits = rng.integers(0, 1 << 16, size=(8192 // PT) * PT * row, dtype=np.uint16) & np.uint16(0xBFFF)
    res = {}
    for d in HEADLINE_DEPTHS:
        n_pages = -(-d // PT)
        pool_bytes = lambda pages: pages * PT * row * 2
        per_set = 18 * 2 * pool_bytes(n_pages) + 18 * 2 * pool_bytes(2)
        n_sets = max(2, -(-(512 << 20) // per_set))
        sets = []
        for _ in range(n_sets):
            blocks = []
            for blk in range(36):
                if blk % 2 == 0:  # windowed block: ring of two pages, cyclic table
                    pages, kv_begin = 2, max(0, d - 128)
                    table = (np.arange(n_pages) % 2).astype(np.uint32)
                else:
                    pages, kv_begin = n_pages, 0
                    table = rng.permutation(n_pages).astype(np.uint32)
                kp, vp = ctx.upload(bits[:pages * PT * row]), ctx.upload(bits[:pages * PT * row])
                blocks.append((kp, vp, ctx.upload(table), sinks[blk], kv_begin))
            sets.append(blocks)

        def step(i):
            for kp, vp, table, sk, kv_begin in sets[i % n_sets]:
                ctx.attn_decode_ext(out, q, kp, vp, table, sk, H, G, D, kv_begin, d, PT, 0.125, KvType.F16)

        graph = rep_stats(graph_timed(hip, ctx, step, n_sets, 1))
        sync_each = []
        for r in range(REPS):
            total = 0.0
            for kp, vp, table, sk, kv_begin in sets[r % n_sets]:
                t0 = time.perf_counter()
                ctx.attn_decode_ext(out, q, kp, vp, table, sk, H, G, D, kv_begin, d, PT, 0.125, KvType.F16)
                ctx.sync()
                total += time.perf_counter() - t0
            sync_each.append(total * 1e3)
        se = rep_stats(sync_each)
        ref_ms, ref_kind = REF_ATTN_ATTEND_MS[d]
        full_bytes = 18 * (d * 2 * row * 2 + H * D * 8 + H * 4 + 4 * n_pages)
        swa_bytes = 18 * (min(128, d) * 2 * row * 2 + H * D * 8 + H * 4 + 8)
        res[str(d)] = {
            "us_per_step_graph": round(graph["median"], 2), "graph_reps": graph,
            "ms_per_step_sync_each": round(se["median"], 4), "sync_each_reps": se,
            "reference_ms_per_step_b580": ref_ms, "reference_kind": ref_kind,
            "speedup_vs_reference_sync_each": round(ref_ms / se["median"], 1),
            "speedup_vs_reference_graph": round(ref_ms * 1e3 / graph["median"], 1),
            "algorithmic_bytes_per_step": full_bytes + swa_bytes,
            "gbs_graph": round((full_bytes + swa_bytes) / graph["median"] / 1e3, 1),
            "sets_rotated": n_sets}
        del sets
    return res


def cpu_prefill_baseline():
    """The reference engine's prefill on the CPU: one decode call per prompt token
    (session.rs:378-381, moe.rs:1856-1862), here the oracle (the f64 CPU twin, reference.rs:821-873,
    plus the sink) on one thread, over config 4's 2048 tokens after 2048 cached, for both layer types.
    Bounded sample: evenly spaced rows of the chunk (16 of the full-causal layer, 64 of the
    SWA-128 layer), REPS passes with the first discarded; the per-key cost of the sample is
    extrapolated to all 2048 rows (full causal: the exact key count PF_PAIRS_FULL; SWA-128: 128
    keys per row). Inputs: the same seeded case as the GPU prefill (tests/fixtures.py)."""
    import fixtures as fx
    from oracle import oracle
    oracle.lib()
    pc = fx.prefill_case(0xC4, n_q=PF_NQ, pos0=PF_POS0, pt=PT)
    qf = pc.qp.astype(np.float32).reshape(PF_NQ, H * D)
    bt = np.ascontiguousarray(pc.bt, np.uint32)
    out = {}
    for name, n_swa, rows in (("full", 0, np.arange(64, PF_NQ, PF_NQ // 16)),
                              ("swa128", 128, np.arange(16, PF_NQ, PF_NQ // 64))):
        per_pass, keys_sample = [], 0
        for r in range(REPS):
            keys_sample = 0
            t0 = time.perf_counter()
            for i in rows:
                n_kv = PF_POS0 + int(i) + 1
                kv_begin = max(0, n_kv - n_swa) if n_swa else 0
                oracle.attn_decode(qf[i], pc.k_raw, pc.v_raw, bt, H, G, D, kv_begin, n_kv, PT, 0.125,
                                   kv_type=1, sinks=pc.sinks)
                keys_sample += n_kv - kv_begin
            per_pass.append(time.perf_counter() - t0)
        st = rep_stats(per_pass)
        keys_total = PF_PAIRS_FULL if n_swa == 0 else PF_NQ * n_swa
        layer_s = st["median"] / keys_sample * keys_total
        out[name] = {"seconds_per_layer_call": round(layer_s, 3),
                     "tokens_per_s": round(PF_NQ / layer_s, 1),
                     "sample": f"{len(rows)} evenly spaced rows of 2048 ({keys_sample} of {keys_total} "
                               f"row-keys), extrapolated by key count",
                     "sample_seconds": st}
    return {**out, "cores": 1, "kind": "port", **host_info()}


def only(what, steps, warmup):
    """Runs one workload eagerly with no timing of its own, for rocprofv3 to wrap:
    decode_graph (the main line's timed region: C2 steps in one graph, replayed), decode (C2), prefill (C4 full then SWA-128),
    prefill_graph (the main line's prefill timing: each layer 8 calls per graph, replayed), rope_append (the fused RoPE-K + K/V append of one
    C4 chunk), matvec (the projection cases of MV_CASES, in order), matmul (MM_CASES, each as
    a graph of `steps` launches, replayed twice), block (`steps` rounds of bench_block: the 128-token
    attention block as one chunked call and as single-token calls), read_floor (the calibration read of C2's 64 MiB of
    KV over the rotating copies), or copy (a 256 MiB device-to-device copy, the reference size for
    scaling FETCH_SIZE/WRITE_SIZE readings to bytes)."""
    from moearc_amd import Context, KvType, OUT_F16
    with Context() as ctx:
        if what == "decode_graph":
            # the timed region of the main line: C2 steps captured in one graph, replayed REPS times
            kp, vp, bt, q, sinks = decode_inputs()
            dks = [ctx.upload(kp) for _ in range(COPIES)]
            dvs = [ctx.upload(vp) for _ in range(COPIES)]
            dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
            dout = ctx.alloc(H * D * 2)
            kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
            reps = graph_timed(Hip(), ctx, lambda i: ctx.attn_decode_batched(
                dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT, kb, nk, ds, H, G, D, PT, 0.125,
                KvType.F16, out_type=OUT_F16), steps, warmup)
            print(f"graph replay: {rep_stats(reps)['median']:.2f} us per step", flush=True)
        elif what == "decode":
            kp, vp, bt, q, sinks = decode_inputs()
            dks = [ctx.upload(kp) for _ in range(COPIES)]
            dvs = [ctx.upload(vp) for _ in range(COPIES)]
            dq, dbt, ds = ctx.upload(q), ctx.upload(bt), ctx.upload(sinks)
            dout = ctx.alloc(H * D * 2)
            kb, nk = np.zeros(1, np.uint32), np.full(1, N_KV, np.uint32)
            for i in range(warmup + steps):
                ctx.attn_decode_batched(dout, dq, dks[i % COPIES], dvs[i % COPIES], dbt, N_KV // PT,
                                        kb, nk, ds, H, G, D, PT, 0.125, KvType.F16, out_type=OUT_F16)
        elif what == "prefill_graph":
            # the prefill's timed region in the main line: both layers, 8 calls per graph, replayed
            r = bench_prefill_graph(ctx, Hip())
            print("graph replay: " + ", ".join(f"{k} {v['median']:.2f} us" for k, v in r.items()), flush=True)
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
        elif what == "block":
            hip = Hip()
            for _ in range(max(1, steps)):
                bench_block(ctx, hip)
        elif what == "headline":
            r = bench_headline(ctx, Hip())
            print(json.dumps({k: (v["us_per_step_graph"], v["ms_per_step_sync_each"]) for k, v in r.items()}),
                  flush=True)
        elif what == "mfma_floor":
            r = bench_mfma_floor(ctx, Hip())
            print(f"graph replay: {r['us']:.2f} us per call, {r['tflops']:.1f} TFLOP/s; zero operands "
                  f"{r['zero_operands']['us']:.2f} us, {r['zero_operands']['tflops']:.1f} TFLOP/s", flush=True)
        elif what == "read_floor":
            bufs, out, nbytes = read_floor_inputs(ctx)
            for i in range(warmup + steps):
                ctx.read_floor(out, bufs[i % COPIES], nbytes)
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
    ap.add_argument("--only", choices=["decode", "decode_graph", "prefill", "prefill_graph", "rope_append", "matvec", "matmul",
                                       "block", "headline", "read_floor", "mfma_floor", "copy"],
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
        from moearc_amd import Context
        with Context() as ctx:
            for name, entry in bench_configs(ctx, Hip(), args.steps, args.warmup).items():
                print(json.dumps({"config": name, **entry}), flush=True)
        return
    r = run(args.steps, args.warmup, args.skip_cpu, args.skip_prefill)

    st = rep_stats(r["step_us_reps"])
    step_us = st["median"]
    gbs = C2_BYTES / step_us / 1e3
    ev = r["events"]
    split_us = ev.get("kernel attn_decode.split r64 m64")
    merge_us = ev.get("kernel attn_decode.merge r64 m64")
    # parity spot check against the oracle (f64) on the same inputs
    from oracle import oracle
    kp, vp, bt, q, sinks = decode_inputs()
    want = oracle.attn_decode(q, kp, vp, bt, H, G, D, 0, N_KV, PT, 0.125, kv_type=1, sinks=sinks)
    err = float(np.max(np.abs(r["out"].ravel() - want)))
    traffic = pmc_traffic(os.path.join(ROOT, "profiles", "decode_c2_pmc.md"))
    split_tr = summary_value(os.path.join(ROOT, "profiles", "decode_c2_kernel_trace.md"), "split_us_trace_graph")
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
        "us_per_layer_reps": st,
        "pct_peak_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
        "tokens_per_s": round(1e6 / step_us, 0),
        "graph_replay_equals_eager": r["graph_equals_eager"],
        "parity_max_abs_err": err,
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "scope": "whole decode call (split-K launch + merge launch), graph-replay step time",
            "bytes_per_call": C2_BYTES,
            "frac_split": round(C2_BYTES / split_us / 1e3 / HBM_PEAK_GBS, 4) if split_us else None,
            "frac_split_note": "split launch alone, HIP events around it in an eager run (they also "
                               "bracket the dispatch gap); frac_split_trace: the committed rocprofv3 trace "
                               "of the graph replay (profiles/decode_c2_kernel_trace.md)",
            "frac_split_trace": round(C2_BYTES / split_tr / 1e3 / HBM_PEAK_GBS, 4) if split_tr else None,
            "split_us_trace": split_tr,
            "split_us_events": round(split_us, 2) if split_us else None,
            "merge_us_events": round(merge_us, 2) if merge_us else None,
            "call_us_events": round(ev["attn_decode r64 m64"], 2) if "attn_decode r64 m64" in ev else None,
        },
        "read_floor": dict(r["read_floor"], decode_frac_of_floor=round(r["read_floor"]["us"] / step_us, 4),
                           decode_frac_of_two_launch_floor=round(
                               r["read_floor"]["with_dependent_launch_us"] / step_us, 4),
                           note="moearc_read_floor over the same 64 MiB copies and graph replay: a plain "
                                "streaming read of the call's KV bytes; decode_frac_of_floor = its time "
                                "over the decode call's; with_dependent_launch_us: the same read followed "
                                "by a dependent one-work-group launch, as the split launch is followed "
                                "by the merge (decode_frac_of_two_launch_floor = that over the call's time)"),
        "device": r.get("device"),
        "commit": git_head(),
        "source_sha16": source_sha16(),
    }
    if "prefill" in r:
        pf = r["prefill"]
        line["prefill_full_mfma_util"] = pf["full"]["mfma_util"]
        line["prefill_full_us"] = pf["full"]["us"]
        line["prefill_swa128_hbm_frac"] = pf["swa128"]["roofline_frac"]
        line["prefill_swa128_us"] = pf["swa128"]["us"]
        line["prefill"] = pf
        if "mfma_floor" in r:
            mf = r["mfma_floor"]
            line["mfma_floor"] = mf
            line["prefill_full_frac_of_mfma_floor"] = round(pf["full"]["tflops"] / mf["tflops"], 4)
    line["configs"] = r["configs"]
    line["headline_step"] = dict(
        r["headline_step"],
        what="the reference's attn.attend per decode step: 36 attention calls (18 SWA-128 + 18 full "
             "causal, B=1) at context depth d; reference figures from an Arc B580 under "
             "MOEARC_SYNC_EACH=1 (bench/results/2026-09-06-moearc-sync-each.txt:17-18, "
             "bench/baselines/gpt-oss-120b.md:626); ms_per_step_sync_each is the same protocol here")
    line["launch_overhead"] = r["launch_overhead"]
    for k in ("projections", "block_chunk", "chunk_projections"):
        if k in r:
            line[k] = r[k]
    if "cpu" in r:
        c = r["cpu"]
        us = c["single_us"]["mean"]
        line["cpu_baseline"] = {
            "value": round(C2_BYTES / us / 1e3, 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"C2 decode (the whole 32768-key call), {c['calls_per_rep']} calls per invocation x "
                      f"{c['single_us']['n']} invocations after a discarded first, of the f64 oracle on one "
                      f"thread: {us / 1e3:.1f} +- {c['single_us']['sd'] / 1e3:.1f} ms per call",
            "us_per_call": c["single_us"],
            "loadavg_1m_before_each": [round(x, 2) for x in c["loadavg_1m"]],
            "nproc": c["nproc"], "affinity_cpus": c["affinity_cpus"], "cpu_model": c["cpu_model"],
            "multithread": {"threads": c["threads"], "us_per_call": c["mt_us"],
                            "value": round(C2_BYTES / c["mt_us"]["mean"] / 1e3, 3)},
        }
    if "cpu_prefill" in r:
        cp = r["cpu_prefill"]
        line["cpu_baseline_prefill"] = {
            "what": "config 4 prefill as the reference engine runs it on the CPU: one decode call per "
                    "prompt token (session.rs:378-381), the f64 oracle on one thread; seconds per "
                    "layer call of 2048 tokens, extrapolated from an evenly spaced row sample",
            "full": cp["full"], "swa128": cp["swa128"], "cores": 1, "kind": "port",
            "gpu_speedup_full": round(cp["full"]["seconds_per_layer_call"] * 1e6 / line["prefill_full_us"], 0)
            if "prefill_full_us" in line else None,
            "gpu_speedup_swa128": round(cp["swa128"]["seconds_per_layer_call"] * 1e6 / line["prefill_swa128_us"], 0)
            if "prefill_swa128_us" in line else None}
    print(json.dumps(line), flush=True)


def git_head():
    try:
        res = subprocess.run(["git", "-C", ROOT, "rev-parse", "HEAD"], capture_output=True, text=True,
                             timeout=10)
        return res.stdout.strip() or None if res.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        return None


def source_sha16():
    """Digest of the sources this line was measured with (the device code, host runtime, headers and
    this file), so the line can be matched to a tree where git history is absent."""
    h = hashlib.sha256()
    files = [os.path.join(ROOT, "bench.py")]
    for d in ("moearc_amd/csrc", "include"):
        full = os.path.join(ROOT, d)
        files += [os.path.join(full, f) for f in sorted(os.listdir(full))
                  if f.endswith((".hip", ".cpp", ".h", ".inc", ".py"))]
    for f in files:
        h.update(os.path.relpath(f, ROOT).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()[:16]


if __name__ == "__main__":
    main()
