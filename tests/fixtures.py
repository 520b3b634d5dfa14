"""Input builders shared by the tests and tests/golden/gen_golden.py.

Reference-test fixtures are regenerated bit-exactly: SplitMix64 ``unit()`` draws in the reference's
``fill_cache`` order -- per token j, the K row then the V row, each n_kv_heads*head_dim values; the
query after all tokens (crates/moearc-kernels/tests/forward_pass_gpu.rs:383-428, :548).
North-star fixtures use N(0,1) values (moearc_amd.synth.normal) and f16 pages.
"""
from __future__ import annotations

import hashlib
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from moearc_amd import synth  # noqa: E402

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")
U = 5.960464477539063e-8  # f32 unit roundoff, 2^-24 (forward_pass_gpu.rs:17)

# The reference's attention tests (forward_pass_gpu.rs), with their seeds and shapes.
REFERENCE_CASES = {
    # :500-591, seed 0xA77E ^ type_id
    "scattered_f32": dict(seed=0xA77E ^ 0, H=16, G=16, D=128, pt=8, pages=16, n_kv=37,
                          bt=[11, 2, 15, 7, 0], kv=0, kv_begin=0),
    "scattered_f16": dict(seed=0xA77E ^ 1, H=16, G=16, D=128, pt=8, pages=16, n_kv=37,
                          bt=[11, 2, 15, 7, 0], kv=1, kv_begin=0),
    # :594-673
    "gqa": dict(seed=0x6A11, H=8, G=2, D=64, pt=4, pages=6, n_kv=10, bt=[5, 1, 3], kv=0,
                kv_begin=0),
    # :676-744 (scale 0.125 fixed by the test)
    "single_key": dict(seed=0x01E1, H=4, G=4, D=32, pt=4, pages=2, n_kv=1, bt=[1], kv=0,
                       kv_begin=0, scale=0.125),
    # :747-871, window 6 of 21 keys (begin 15)
    "window": dict(seed=0x5A11, H=8, G=2, D=64, pt=4, pages=8, n_kv=21, bt=[7, 0, 4, 2, 6, 1],
                   kv=0, kv_begin=15),
}


def ref_tolerance(D: int, n: int) -> float:
    """The reference tests' bound: 8 * ((D/32 + 5) + n + 8) * 2^-24 (forward_pass_gpu.rs:582-583)."""
    return 8.0 * ((D / 32.0 + 5.0) * U + n * U + 8.0 * U)


class Case:
    """One attention problem: pools (device format and f32 host mirror), table, q, sinks."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    def digest(self) -> str:
        h = hashlib.sha256()
        for a in (self.k_raw, self.v_raw, self.q, self.bt):
            h.update(np.ascontiguousarray(a).tobytes())
        if self.sinks is not None:
            h.update(np.ascontiguousarray(self.sinks).tobytes())
        return h.hexdigest()


def _store(x: np.ndarray, kv: int):
    """(device bytes, f32 values the cache holds) for rows x: KvType::store (reference.rs:754-759)."""
    if kv == 1:
        bits = synth.f16_bits(x)
        return bits, bits.view(np.float16).astype(np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return x.copy(), x.copy()


def reference_case(name: str) -> Case:
    p = dict(REFERENCE_CASES[name])
    H, G, D, pt, pages, n_kv, kv = p["H"], p["G"], p["D"], p["pt"], p["pages"], p["n_kv"], p["kv"]
    row = G * D
    draws = synth.unit(p["seed"], 2 * n_kv * row + H * D)
    rows = draws[: 2 * n_kv * row].reshape(n_kv, 2, row)
    q = draws[2 * n_kv * row:].copy()
    bt = np.asarray(p["bt"], np.uint32)
    pool = pages * pt * row
    dt = np.uint16 if kv == 1 else np.float32
    k_raw, v_raw = np.zeros(pool, dt), np.zeros(pool, dt)
    k_val, v_val = np.zeros(pool, np.float32), np.zeros(pool, np.float32)
    for j in range(n_kv):
        base = (int(bt[j // pt]) * pt + j % pt) * row
        kr, kf = _store(rows[j, 0], kv)
        vr, vf = _store(rows[j, 1], kv)
        k_raw[base:base + row], k_val[base:base + row] = kr, kf
        v_raw[base:base + row], v_val[base:base + row] = vr, vf
    scale = p.get("scale", 1.0 / math.sqrt(D))
    return Case(name=name, H=H, G=G, D=D, pt=pt, n_kv=n_kv, kv_begin=p["kv_begin"], kv=kv,
                scale=np.float32(scale), q=q, bt=bt, k_raw=k_raw, v_raw=v_raw, k_val=k_val,
                v_val=v_val, sinks=None, token_rows=rows)


def north_star_case(seed: int, n_kv: int, kv_begin: int = 0, H: int = 64, G: int = 8, D: int = 64,
                    pt: int = 256, sinks: bool = True, scatter: bool = True,
                    spike_frac: float = 0.0, extra_pages: int = 0, boost=None) -> Case:
    """gpt-oss-shaped decode input: q, K, V ~ N(0,1) (K/V stored f16), per-head f32 sinks ~ N(0,1),
    KV in pt-token pages through a seeded random page permutation. With spike_frac > 0 that
    fraction of K rows is scaled by 8 (stresses the running max); boost, a list of (start, stop,
    factor), scales K rows start..stop-1 by factor, in order (jumps in the scores where chosen)."""
    row = G * D
    n_pages = -(-n_kv // pt) + extra_pages
    kvals = synth.normal(seed, n_kv * row).reshape(n_kv, row)
    vvals = synth.normal(seed + 1, n_kv * row).reshape(n_kv, row)
    if spike_frac > 0:
        pick = synth.splitmix64(seed + 2, n_kv) % np.uint64(10000) < np.uint64(int(spike_frac * 10000))
        kvals[pick] *= np.float32(8.0)
    for start, stop, factor in boost or ():
        kvals[start:stop] *= np.float32(factor)
    q = synth.normal(seed + 3, H * D)
    s = synth.normal(seed + 4, H) if sinks else None
    bt = synth.random_block_table(seed + 5, n_pages) if scatter else np.arange(n_pages, dtype=np.uint32)
    pool_tokens = n_pages * pt
    k_raw = np.zeros((pool_tokens, row), np.uint16)
    v_raw = np.zeros((pool_tokens, row), np.uint16)
    j = np.arange(n_kv)
    phys = bt[j // pt].astype(np.int64) * pt + j % pt
    k_raw[phys] = synth.f16_bits(kvals)
    v_raw[phys] = synth.f16_bits(vvals)
    return Case(name=f"ns_{n_kv}", H=H, G=G, D=D, pt=pt, n_kv=n_kv, kv_begin=kv_begin, kv=1,
                scale=np.float32(1.0 / math.sqrt(D)), q=q, bt=bt[: max(1, -(-n_kv // pt))].copy(),
                bt_full=bt, k_raw=k_raw.ravel(), v_raw=v_raw.ravel(), k_val=None, v_val=None,
                sinks=s)


def contiguous_kv(case: Case, which: str) -> np.ndarray:
    """[n_kv][G][D] f64 values of the span's keys, gathered through the block table (numpy fancy
    indexing, independent of the oracle's kv_index)."""
    raw = case.k_raw if which == "k" else case.v_raw
    vals = raw.view(np.float16).astype(np.float64) if case.kv == 1 else raw.astype(np.float64)
    vals = vals.reshape(-1, case.G, case.D)
    j = np.arange(case.n_kv)
    phys = case.bt[j // case.pt].astype(np.int64) * case.pt + j % case.pt
    return vals[phys]


def sdpa_reference(case: Case, kv_begin: int | None = None, sinks=None) -> np.ndarray:
    """Independent float64 answer from torch's scaled_dot_product_attention: K/V gathered to a
    contiguous run, GQA by repeat_interleave, the span as a slice, and a sink as one extra key of
    value zero whose additive bias is the sink logit (the sink enters only the denominator)."""
    import torch
    kb = case.kv_begin if kv_begin is None else kv_begin
    K = torch.from_numpy(contiguous_kv(case, "k")[kb:])  # [n, G, D]
    V = torch.from_numpy(contiguous_kv(case, "v")[kb:])
    group = case.H // case.G
    K = K.permute(1, 0, 2).repeat_interleave(group, dim=0)  # [H, n, D]
    V = V.permute(1, 0, 2).repeat_interleave(group, dim=0)
    Q = torch.from_numpy(case.q.astype(np.float64).reshape(case.H, 1, case.D))
    scale = float(case.scale)
    if sinks is not None:
        n = K.shape[1]
        K = torch.cat([K, torch.zeros(case.H, 1, case.D, dtype=torch.float64)], dim=1)
        V = torch.cat([V, torch.zeros(case.H, 1, case.D, dtype=torch.float64)], dim=1)
        bias = torch.zeros(case.H, 1, n + 1, dtype=torch.float64)
        bias[:, 0, n] = torch.from_numpy(np.asarray(sinks, np.float64))
        out = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=bias, scale=scale)
    else:
        out = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=scale)
    return out.reshape(-1).numpy()


def prefill_case(seed, n_q, pos0, pt=32, H=64, G=8, D=64, spike_frac=0.0, boost=None):
    case = north_star_case(seed, pos0 + n_q, pt=pt, H=H, G=G, D=D, spike_frac=spike_frac, boost=boost)
    case.qp = synth.normal(seed + 7, n_q * H * D).astype(np.float16).reshape(n_q, H, D)
    case.n_q, case.pos0, case.seed = n_q, pos0, seed
    return case


def prefill_brute(case, n_swa):
    """float64 masked softmax over the whole chunk at once (rows = queries, columns = keys), with
    the sink as an extra column of value zero; independent of the oracle's per-row decode loop."""
    K = contiguous_kv(case, "k")  # [T, G, D]
    V = contiguous_kv(case, "v")
    group = case.H // case.G
    Q = case.qp.astype(np.float64)  # [n_q, H, D]
    T = case.pos0 + case.n_q
    pos = case.pos0 + np.arange(case.n_q)[:, None]
    j = np.arange(T)[None, :]
    visible = j <= pos
    if n_swa:
        visible &= j > pos - n_swa
    out = np.empty((case.n_q, case.H, case.D))
    for h in range(case.H):
        g = h // group
        s = (Q[:, h, :] @ K[:, g, :].T) * float(case.scale)
        s = np.where(visible, s, -np.inf)
        sink = np.full((case.n_q, 1), float(case.sinks[h]))
        full = np.concatenate([s, sink], axis=1)
        mx = full.max(axis=1, keepdims=True)
        e = np.exp(full - mx)
        out[:, h, :] = (e[:, :T] @ V[:, g, :]) / e.sum(axis=1, keepdims=True)
    return out


def prefill_digest(case) -> str:
    h = hashlib.sha256()
    for a in (case.qp, case.k_raw, case.v_raw, case.bt, case.sinks):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---- RoPE ------------------------------------------------------------------------------------

# crates/moearc-kernels/tests/kernels_gpu.rs:292-351: 5 tokens x 4 heads x 80 channels, 64 rotated,
# base 10000, positions 3t, inputs Rng(0xB0BE).vec_unit.
ROPE_REF = dict(seed=0xB0BE, tokens=5, heads=4, head_dim=80, n_dims=64, freq_base=10000.0)
# gpt-oss's published RoPE configuration: base 150000, YaRN factor 32 over a 4096-token original
# context, beta_fast 32, beta_slow 1 (the GGUF defaults moe.rs:582-586 falls back to).
GPT_OSS_ROPE = dict(freq_base=150000.0, factor=32.0, n_ctx_orig=4096, beta_fast=32.0, beta_slow=1.0)


def rope_reference_inputs():
    from oracle import oracle
    r = ROPE_REF
    src = oracle.Rng(r["seed"]).vec_unit(r["tokens"] * r["heads"] * r["head_dim"])
    pos = (np.arange(r["tokens"], dtype=np.int32) * 3).astype(np.int32)
    return src, pos


def host_powf(x, y):
    """The host C library's powf (what the runtime and the reference's host use for theta_scale;
    numpy's float32 power can differ from it in the last bit)."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return float(libm.powf(float(np.float32(x)), float(np.float32(y))))


def rope_complex(src, pos, n_tokens, n_heads, head_dim, n_dims, freq_base, scaling=None, neox=True):
    """An independent formulation: each rotated pair is a complex number z = x_lo + i x_hi (pairs
    taken by slicing -- the two halves for NeoX, even/odd channels otherwise) multiplied by
    mscale * e^(i theta) in complex128. theta_p = pos * theta_scale^p with theta_scale rounded to
    f32 (the host's powf); YaRN mixes the interpolated and extrapolated angles by the ramp."""
    x = np.asarray(src, np.float64).reshape(n_tokens, n_heads, head_dim).copy()
    half = n_dims // 2
    ts = host_powf(freq_base, -2.0 / n_dims)
    p = np.arange(half, dtype=np.float64)
    ext = np.asarray(pos, np.float64)[:, None] * ts ** p[None, :]  # [tokens][half]
    fs, ef, af, lo, hi = (1.0, 0.0, 1.0, 0.0, 0.0) if scaling is None else scaling
    theta, msc = fs * ext, af
    if ef != 0.0:
        y = (p - lo) / max(0.001, hi - lo)
        mix = (1.0 - np.clip(y, 0.0, 1.0)) * ef
        theta = theta * (1.0 - mix)[None, :] + ext * mix[None, :]
        msc = af * (1.0 + 0.1 * np.log(1.0 / fs))
    rot = msc * np.exp(1j * theta)[:, None, :]  # broadcast over heads
    if neox:
        z = x[..., :half] + 1j * x[..., half:n_dims]
        z = z * rot
        x[..., :half], x[..., half:n_dims] = z.real, z.imag
    else:
        z = x[..., 0:n_dims:2] + 1j * x[..., 1:n_dims:2]
        z = z * rot
        x[..., 0:n_dims:2], x[..., 1:n_dims:2] = z.real, z.imag
    return x.reshape(-1)


# ---- quantised weights (crates/moearc-kernels/tests/common/mod.rs:45-84) ---------------------

QT_BLOCK = {0: (4, 1), 1: (2, 1), 8: (34, 32), 12: (144, 256), 13: (176, 256), 14: (210, 256),
            39: (17, 32)}  # type id -> (block bytes, block elements)


def synth_blocks(ty: int, nblocks: int, seed: int):
    """The reference tests' ``synth_blocks(ty, nblocks, &mut Rng::new(seed))`` followed by
    ``rng.vec_unit`` -- returns (blocks as uint8, draws consumed) so the caller can continue the
    stream. Random payload bytes (low byte of each draw), then per block the constrained fields:
    f16 scales 0x1000 + u32 % 0x1800 (Q8_0: d; Q4_K/Q5_K: d, dmin; Q6_K: d at byte 208), an E8M0
    exponent 100 + u32 % 56 (MXFP4), a unit value (F32) or its f16 (F16)."""
    bb, _ = QT_BLOCK[ty]
    n = nblocks * bb
    v = (synth.splitmix64(seed, n) & np.uint64(0xFF)).astype(np.uint8).reshape(nblocks, bb)
    per = {8: 1, 12: 2, 13: 2, 14: 1, 39: 1, 0: 1, 1: 1}[ty]
    draws = synth.splitmix64(seed, nblocks * per, n).reshape(nblocks, per)
    lo32 = draws & np.uint64(0xFFFFFFFF)

    def scale(col):
        return (np.uint64(0x1000) + lo32[:, col] % np.uint64(0x1800)).astype(np.uint16)

    if ty in (8, 12, 13):
        v[:, 0:2] = scale(0).view(np.uint8).reshape(nblocks, 2)
        if ty != 8:
            v[:, 2:4] = scale(1).view(np.uint8).reshape(nblocks, 2)
    elif ty == 14:
        v[:, 208:210] = scale(0).view(np.uint8).reshape(nblocks, 2)
    elif ty == 39:
        v[:, 0] = (np.uint64(100) + lo32[:, 0] % np.uint64(56)).astype(np.uint8)
    else:
        u = synth.unit(seed, nblocks, n)
        if ty == 0:
            v[:, :] = u.view(np.uint8).reshape(nblocks, 4)
        else:
            v[:, :] = synth.f16_bits(u).view(np.uint8).reshape(nblocks, 2)
    return v.reshape(-1), n + nblocks * per


def matvec_case(ty: int, rows: int, cols: int, seed: int):
    """(w bytes, x f32) drawn as the reference's matvec tests draw them (kernels_gpu.rs:110-116)."""
    be = QT_BLOCK[ty][1]
    w, used = synth_blocks(ty, rows * cols // be, seed)
    x = synth.unit(seed, cols, used)
    return w, x


def matvec_tolerance(cols: int, absum: np.ndarray) -> np.ndarray:
    """The reference's bound (kernels_gpu.rs:126-137): 2 (cols/32 + 5) u sum|w x| per row."""
    return 2.0 * (cols / 32.0 + 5.0) * 2.0 ** -24 * absum
