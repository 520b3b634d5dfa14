"""The C ABI library loads and exports every symbol include/*.h declares (CPU only).

No compute call is made: only entry points refused on the host before any device work (a null
context returns -1, the reference's null-argument code) are called.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest

from moearc_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moearc_attn.h")
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_symbols(headers=None):
    text = "".join(open(h).read() for h in (headers or HEADERS))
    return sorted(set(re.findall(r"\b(moearc_\w+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    names = declared_symbols([HEADER])
    # the attention + lifecycle subset of crates/moearc-kernels/src/ffi.rs:20-234
    for n in ("moearc_ctx_create", "moearc_ctx_destroy", "moearc_profile_events_enabled",
              "moearc_profile_events_reset", "moearc_profile_events_report", "moearc_sync",
              "moearc_zero", "moearc_device_name", "moearc_alloc_device", "moearc_free_device",
              "moearc_copy_h2d", "moearc_copy_h2d_async", "moearc_copy_d2h",
              "moearc_quantize_f16", "moearc_kv_append", "moearc_attn_decode", "moearc_matvec_q",
              "moearc_matvec_q_batched", "moearc_matvec_f32", "moearc_add"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = native.load()
    for n in declared_symbols():
        assert hasattr(lib, n), f"{n} is declared but not exported"
        assert n in native.SIGNATURES, f"{n} has no ctypes signature"


def test_code_object_holds_every_kernel_the_runtime_loads():
    blob = open(native.CODE_OBJECT, "rb").read()
    src = open(os.path.join(ROOT, "moearc_amd", "csrc", "runtime.cpp")).read()
    kernels = set(re.findall(r'"(moearc_\w+_k|moearc_attn_decode_f16d64_k\d+w\d+t\d+|moearc_attn_decode_merge)"', src))
    kernels |= {f"moearc_attn_prefill_{v}g{g}" for v in ("", "precise_") for g in (1, 2, 4, 8)}
    kernels |= {f"moearc_matmul_{t}_r{r}_k" for t in ("q8_0", "f16", "q4_k", "q5_k", "q6_k", "mxfp4") for r in (1, 2)}
    kernels |= {"moearc_split_f16_k", "moearc_block_sums_k"}
    kernels |= {f"moearc_matvec_{t}_p{p}" for t in ("f32", "f16", "q8_0", "q4_k", "q5_k", "q6_k", "mxfp4")
                for p in (1, 2, 4)}
    assert kernels
    for k in kernels:
        assert k.encode() in blob, f"kernel {k} missing from the code object"


def test_kv_pool_header_is_bound():
    names = declared_symbols([os.path.join(ROOT, "include", "moearc_kv.h")])
    assert "moearc_kv_pool_create" in names and "moearc_kv_ring_table" in names
    lib = native.load()
    assert lib.moearc_kv_pool_begin(None, 1, 1) == -1


def test_null_context_is_refused_with_minus_one():
    lib = native.load()
    assert lib.moearc_sync(None) == -1
    assert lib.moearc_profile_events_reset(None) == -1
    assert lib.moearc_profile_events_enabled(None) == 0
    assert lib.moearc_attn_decode(None, None, None, None, None, None, None, 64, 8, 64, 0, 10, 32,
                                  ctypes.c_float(0.125), 1) == -1
    assert lib.moearc_kv_append(None, None, None, None, None, 0, 0, 8, 64, 32, 1) == -1
    assert lib.moearc_attn_prefill(None, None, 0, None, None, None, None, None, 8, 0, 0, 64, 8,
                                   64, 32, ctypes.c_float(0.125), 1) == -1
    assert lib.moearc_alloc_device(None, 16) is None
    assert lib.moearc_copy_h2d(None, None, None, 0) == -1
    assert lib.moearc_quantize_f16(None, None, None, 4) == -1
    assert lib.moearc_matvec_q(None, 8, None, None, None, 4, 32) == -1
    assert lib.moearc_matvec_q_batched(None, 8, None, None, 1, None, 0, 4, 32) == -1
    assert lib.moearc_matvec_f32(None, None, None, None, 4, 4) == -1
    assert lib.moearc_add(None, None, None, None, 4) == -1
    assert lib.moearc_attn_qkv(None, None, None, None, None, None, None, 32) == -1
    assert lib.moearc_attn_block_chunk(None, None, None, None, 1, 0, None, None, None) == -1
    assert lib.moearc_matmul_q(None, 8, None, None, None, None, 4, 4, 32) == -1
    assert lib.moearc_attn_out(None, 8, None, None, None, None, 4, 32) == -1


def test_missing_build_fails_loudly(monkeypatch):
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "LIBRARY", "/nonexistent/libmoearc_attn.so")
    with pytest.raises(native.NativeLibraryMissing):
        native.load()


def _c_arity(path):
    src = open(path).read()
    out = {}
    for m in re.finditer(r"^(?:int|void|void \*|moearc_ctx \*)\s*\*?\s*(moearc_\w+)\s*\(([^;]*?)\);", src,
                         re.M | re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("void", "") else args.count(",") + 1
    return out


def _rust_arity(path):
    src = open(path).read()
    out = {}
    for m in re.finditer(r"pub fn (moearc_\w+)\s*\((.*?)\)\s*(?:->|;)", src, re.S):
        args = m.group(2).strip().rstrip(",")
        out[m.group(1)] = 0 if not args else args.count(",") + 1
    return out


def test_rust_ffi_crate_declares_the_headers():
    # crates/moearc-hip/src/{ffi,kv_ffi}.rs are hand-written like the reference's ffi.rs: every C
    # declaration appears there once, with the same number of arguments
    c = {**_c_arity(os.path.join(ROOT, "include", "moearc_attn.h")),
         **_c_arity(os.path.join(ROOT, "include", "moearc_kv.h"))}
    rs = {**_rust_arity(os.path.join(ROOT, "crates", "moearc-hip", "src", "ffi.rs")),
          **_rust_arity(os.path.join(ROOT, "crates", "moearc-hip", "src", "kv_ffi.rs"))}
    assert c and set(c) == set(rs)
    assert {k: c[k] for k in c} == {k: rs[k] for k in c}


def test_rust_block_descriptor_matches_the_header():
    # the moearc_attn_block field order, as declared in C, in the Rust struct and in the ctypes one
    hdr = open(os.path.join(ROOT, "include", "moearc_attn.h")).read()
    body = hdr[hdr.index("typedef struct moearc_attn_block {"):hdr.index("} moearc_attn_block;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    c_fields = []
    for decl in body.split("{", 1)[1].split(";"):
        decl = decl.strip()
        if decl:
            c_fields += [re.sub(r"[\*\[\]0-9]", "", n).strip().split()[-1] for n in decl.split(",")]
    rs = open(os.path.join(ROOT, "crates", "moearc-hip", "src", "ffi.rs")).read()
    rs_body = rs[rs.index("pub struct MoearcAttnBlock {"):]
    rs_body = rs_body[:rs_body.index("}")]
    rs_fields = re.findall(r"pub (\w+):", rs_body)
    from moearc_amd.context import AttnBlockDesc
    py_fields = [f[0] for f in AttnBlockDesc._fields_]
    assert c_fields == rs_fields == py_fields
