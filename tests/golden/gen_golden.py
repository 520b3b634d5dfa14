"""Writes the golden fixtures under tests/golden/.

Inputs are never stored: each fixture names its generator (seed, shapes) and holds a SHA-256 of
the regenerated inputs, so a drift in the generator fails loudly. Stored are the expected outputs:

* ``expected``  -- the oracle (oracle/moearc_oracle.c, a restatement of reference.rs:821-873 with
  the sink of kernels.cpp:1864-1880), float64;
* ``sdpa``      -- torch's float64 scaled_dot_product_attention on the same inputs, an independent
  library computation (sinks as an extra zero-valued key with an additive bias).

The script refuses to write a fixture whose two answers differ by more than 1e-12.
The reference-test fixtures reproduce crates/moearc-kernels/tests/forward_pass_gpu.rs's inputs
bit-exactly (SplitMix64 and the fill order of fill_cache, :383-428).

The RoPE fixture (kernels_gpu.rs:292-351's inputs) stores reference::rope's outputs, checked against
an independent complex128 formulation to 1e-5.

Run: python tests/golden/gen_golden.py            (every fixture)
     python tests/golden/gen_golden.py rope       (the RoPE fixture only)
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import fixtures as fx  # noqa: E402
from oracle import oracle  # noqa: E402


def _agree(a, b, what):
    err = float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
    if not err <= 1e-12:
        raise SystemExit(f"{what}: oracle and SDPA differ by {err:.3e}")
    return err


def decode_fixture(name, case, kv_begin, sinks, **meta):
    raw_k = case.k_raw if case.kv == 1 else case.k_raw.astype(np.float32)
    raw_v = case.v_raw if case.kv == 1 else case.v_raw.astype(np.float32)
    exp = oracle.attn_decode(case.q, raw_k, raw_v, case.bt, case.H, case.G, case.D, kv_begin,
                             case.n_kv, case.pt, float(case.scale), kv_type=case.kv, sinks=sinks,
                             f64=True)
    ref = fx.sdpa_reference(case, kv_begin=kv_begin, sinks=sinks)
    err = _agree(exp, ref, name)
    np.savez(os.path.join(HERE, name + ".npz"), expected=exp, sdpa=ref,
             digest=np.array(case.digest()), kv_begin=np.array(kv_begin),
             **{k: np.array(v) for k, v in meta.items()})
    print(f"{name}: oracle vs SDPA {err:.2e}, |out|max {np.abs(exp).max():.3f}")


def prefill_fixture(name, case, n_swa):
    q32 = case.qp.astype(np.float32)
    exp = oracle.attn_prefill(q32, case.k_raw, case.v_raw, case.bt, case.n_q, case.pos0, n_swa,
                              case.H, case.G, case.D, case.pt, float(case.scale),
                              kv_type=oracle.KV_F16, sinks=case.sinks)
    ref = fx.prefill_brute(case, n_swa)
    err = float(np.max(np.abs(exp.astype(np.float64) - ref)))
    # The oracle returns f32 rows here; agreement is to f32 rounding of an O(1) result.
    if not err <= 1e-6:
        raise SystemExit(f"{name}: oracle vs brute force differ by {err:.3e}")
    dig = fx.prefill_digest(case)
    rows = np.arange(0, case.n_q, 5)  # a fifth of the rows keeps the fixture small
    np.savez(os.path.join(HERE, name + ".npz"), expected=ref[rows].astype(np.float32), rows=rows,
             digest=np.array(dig), n_swa=np.array(n_swa), seed=np.array(case.seed),
             n_q=np.array(case.n_q), pos0=np.array(case.pos0), pt=np.array(case.pt))
    print(f"{name}: oracle vs brute force {err:.2e}")


def rope_fixture():
    # kernels_gpu.rs:292-351's inputs; expected = reference::rope (iterated angle table, f32) for
    # both conventions; the complex128 closed form must agree to 1e-5 (the iterated table drifts
    # by a few ulp of the angle).
    r = fx.ROPE_REF
    src, pos = fx.rope_reference_inputs()
    out = {}
    for name, neox in (("neox", True), ("normal", False)):
        want = oracle.rope(src, pos, r["tokens"], r["heads"], r["head_dim"], r["n_dims"],
                           r["freq_base"], neox)
        ind = fx.rope_complex(src, pos, r["tokens"], r["heads"], r["head_dim"], r["n_dims"],
                              r["freq_base"], neox=neox)
        err = float(np.max(np.abs(want.astype(np.float64) - ind)))
        if not err <= 1e-5:
            raise SystemExit(f"rope {name}: oracle and complex form differ by {err:.3e}")
        out["expected_" + name] = want
    import hashlib
    np.savez(os.path.join(HERE, "ref_rope.npz"), digest=hashlib.sha256(src.tobytes()).hexdigest(),
             pos=pos, **out)


def main():
    for name in fx.REFERENCE_CASES:
        c = fx.reference_case(name)
        decode_fixture("ref_" + name, c, c.kv_begin, None)
    c = fx.reference_case("window")
    decode_fixture("ref_window_full", c, 0, None)
    decode_fixture("ref_window_one", c, c.n_kv - 1, None)
    # gpt-oss shape, small depth: full and SWA-128 spans, with sinks, scattered 32-token pages
    ns = fx.north_star_case(0x5EED, 300, pt=32)
    decode_fixture("ns_decode_full", ns, 0, ns.sinks, seed=0x5EED, n_kv=300, pt=32)
    decode_fixture("ns_decode_swa128", ns, 300 - 128, ns.sinks, seed=0x5EED, n_kv=300, pt=32)
    pc = fx.prefill_case(0x9F11, n_q=48, pos0=80)
    prefill_fixture("ns_prefill_full", pc, 0)
    prefill_fixture("ns_prefill_swa16", pc, 16)
    rope_fixture()


if __name__ == "__main__" and sys.argv[1:] == ["rope"]:
    rope_fixture()
elif __name__ == "__main__":
    main()
