"""Checks the compiled prefill kernels for the gfx950 hazards that hand-written asm must respect.

The key loop of the default prefill kernels is one inline-asm statement (prefill_loop.inc), so the
compiler inserts no wait states or counter waits inside it. This script compiles moearc_kernels.hip
to assembly with the build's flags and walks the control-flow graph of each kernel (branches and
calls followed, `s_setpc_b64` returns ending a path), counting wait states (one per instruction,
N + 1 for `s_nop N`):

  1. an MFMA result (its destination registers) is not read or written by any other instruction
     within MFMA_WAIT wait states of the MFMA; a later MFMA may accumulate into exactly the same
     registers (same-size back-to-back accumulation is forwarded) but not read them as A or B;
  2. a VALU result is not read by an MFMA within VALU_MFMA_WAIT wait states;
  3. no register that an asm-issued `ds_read*` or block-table `global_load_dword` writes is touched
     between the load and the `s_waitcnt` that retires it (loads counted in program order);
  4. an inline-asm statement that writes m0 (the LDS base of the DMA copies; a register the compiler
     owns, so no asm may list it as clobbered) first saves it to an SGPR and ends by restoring it
     from that SGPR, which nothing in between writes -- in every kernel of the code object;
  5. every register the key loop (prefill_loop.inc) writes is an output ("+{...}") or a clobber of
     the asm statement in prefill_fast.hip: the compiler keeps its own values in any other register
     across the statement, and in an input-only operand it may reuse the value afterwards;
  6. the VALU wait states hipcc itself inserts for gfx950 (seen in its output for plain HIP code):
     a VALU result is not read by v_readfirstlane / v_readlane within 1 wait state, a transcendental
     result (v_exp_f32 and the like) not by another VALU instruction within 1, and an SGPR written by
     v_readfirstlane / v_readlane not read by a VALU instruction within 2;
  7. the data registers of a vector-memory store of more than 8 bytes (dwordx3 / dwordx4) are not
     written within 2 wait states of it: the store reads them after issue (hipcc puts s_nop 1
     between its own such stores and a VALU write of their data on gfx950, and nothing after an
     inline-asm store -- a 16-byte asm store followed at once by a VALU write of its data stored the
     new value, and with one wait state it still did, now and then, under load) -- in every kernel
     of the code object.

Usage: python check_asm_hazards.py [kernel-name-prefix ...]   (default: moearc_attn_prefill_g)
Exit status 1 when a hazard is found.
"""
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
MFMA_WAIT = 20      # 16-pass XDL result -> VALU: 18 on gfx940, 19 on gfx950, one spare
VALU_MFMA_WAIT = 2  # VALU result -> MFMA source
FLAGS = ["--offload-arch=gfx950", "--cuda-device-only", "-S", "-O3", "-std=c++17",
         "-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
         "-mllvm", "-amdgpu-kernarg-preload-count=14",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def compile_asm():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hipcc = os.path.join(rocm, "bin", "hipcc")
    out = os.path.join(tempfile.mkdtemp(prefix="moearc_asm_"), "kernels.s")
    subprocess.run([hipcc, *FLAGS, "-I", HERE, os.path.join(HERE, "moearc_kernels.hip"), "-o", out],
                   check=True, stderr=subprocess.DEVNULL)
    return open(out).read().split("\n")


def kernel_body(lines, name):
    start = next(i for i, l in enumerate(lines) if l.split(";")[0].rstrip() == name + ":")
    ins, labels = [], {}
    for l in lines[start + 1:]:
        t = l.split(";")[0].strip()
        if t.startswith(".end_amdhsa_kernel") or t.startswith(".Lfunc_end"):
            break
        if not t:
            continue
        if t.endswith(":"):
            labels[t[:-1]] = len(ins)
        elif not t.startswith("."):
            ins.append(t)
    return ins, labels


def regs(tok):
    tok = tok.split()[0] if tok else ""
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def split_ops(t):
    parts = t.split(None, 1)
    return parts[0], ([a.strip() for a in parts[1].split(",")] if len(parts) > 1 else [])


def writes_reads(t):
    """VGPRs an instruction writes and reads."""
    op, args = split_ops(t)
    rs = [regs(a) for a in args]
    allr = set().union(*rs) if rs else set()
    if op.startswith(("v_cmp", "v_readfirstlane", "v_readlane")):
        return set(), allr
    if op.startswith(("ds_write", "global_store", "global_load_lds", "scratch_store",
                      "buffer_store", "global_atomic")):
        return set(), allr
    if op.startswith(("v_", "ds_read", "ds_bpermute", "global_load", "buffer_load", "scratch_load")):
        return (rs[0] if rs else set()), (set().union(*rs[1:]) if len(rs) > 1 else set())
    return set(), set()


def wait_states(t):
    m = re.match(r"s_nop (\d+)", t)
    return int(m.group(1)) + 1 if m else 1


def successors(ins, labels, j):
    op, args = split_ops(ins[j])
    if op == "s_branch":
        return [labels[args[0]]]
    if op.startswith("s_cbranch"):
        return [labels[args[0]], j + 1]
    if op == "s_call_b64":
        return [labels[args[1]], j + 1]
    if op in ("s_setpc_b64", "s_endpgm"):
        return []
    return [j + 1]


def walk(ins, labels, i, need, check):
    """Instructions reachable from i with fewer than `need` wait states in between, for which
    check() reports a problem."""
    found, best = [], {}
    stack = [(k, 0) for k in successors(ins, labels, i)]
    while stack:
        j, d = stack.pop()
        if j >= len(ins) or d >= need or best.get(j, 1 << 30) <= d:
            continue
        best[j] = d
        msg = check(ins[j])
        if msg:
            found.append(f"[{ins[i]}] -> [{ins[j]}] after {d} wait states: {msg}")
            continue
        stack.extend((k, d + wait_states(ins[j])) for k in successors(ins, labels, j))
    return found


def mfma_hazards(ins, labels):
    out = []
    for i, t in enumerate(ins):
        op, args = split_ops(t)
        if op.startswith("v_mfma"):
            dst = regs(args[0])

            def chk(u, dst=dst):
                uop, ua = split_ops(u)
                if uop.startswith("v_mfma"):
                    c = regs(ua[3]) if len(ua) > 3 else set()
                    if dst & (regs(ua[1]) | regs(ua[2])):
                        return "MFMA reads the result as A or B"
                    if dst & c and c != dst:
                        return "MFMA C partly overlaps the result"
                    return None
                w, r = writes_reads(u)
                return "result used" if dst & (w | r) else None
            out += walk(ins, labels, i, MFMA_WAIT, chk)
        elif op.startswith("v_"):
            w, _ = writes_reads(t)
            if not w:
                continue

            def chk2(u, w=w):
                uop, ua = split_ops(u)
                if uop.startswith("v_mfma") and w & set().union(*[regs(a) for a in ua[1:4]]):
                    return "MFMA reads a VALU result"
                return None
            out += walk(ins, labels, i, VALU_MFMA_WAIT, chk2)
    return out


TRANS = ("v_exp_", "v_log_", "v_rcp_", "v_rsq_", "v_sqrt_", "v_sin_", "v_cos_")


def sregs(tok):
    """SGPR numbers named by one operand (sN or s[a:b])."""
    tok = tok.split()[0] if tok else ""
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def valu_wait_hazards(ins, labels):
    """Check 6 over the instructions of one kernel or asm statement."""
    out = []
    for i, t in enumerate(ins):
        op, args = split_ops(t)
        if not op.startswith("v_") or op.startswith("v_mfma"):
            continue
        if op.startswith(("v_readfirstlane", "v_readlane")):
            sd = sregs(args[0]) if args else set()

            def chk_s(u, sd=sd):
                uop, ua = split_ops(u)
                if uop.startswith("v_") and any(sd & sregs(a) for a in ua[1:]):
                    return "VALU reads an SGPR that v_readfirstlane/v_readlane wrote"
                return None
            out += walk(ins, labels, i, 2, chk_s)
            continue
        w, _ = writes_reads(t)
        if not w:
            continue

        def chk_r(u, w=w):
            uop, ua = split_ops(u)
            if uop.startswith(("v_readfirstlane", "v_readlane")) and len(ua) > 1 and w & regs(ua[1]):
                return "v_readfirstlane/v_readlane reads a VALU result"
            return None
        out += walk(ins, labels, i, 1, chk_r)
        if op.startswith(TRANS):
            def chk_t(u, w=w):
                uop, ua = split_ops(u)
                if uop.startswith("v_") and not uop.startswith("v_mfma") and \
                        w & set().union(*[regs(a) for a in ua[1:]] or [set()]):
                    return "VALU reads a transcendental result"
                return None
            out += walk(ins, labels, i, 1, chk_t)
    return out


def load_hazards(ins):
    """Straight-line check of asm-issued load destinations against their retiring wait."""
    out = []
    for i, t in enumerate(ins):
        if t.startswith("ds_read"):
            kind = "lgkm"
        elif re.match(r"global_load_dword v\d+, v\[\d+:\d+\], off$", t):
            kind = "vm"
        else:
            continue
        dst = regs(t.split(",")[0].split(None, 1)[1])
        younger = 0
        for j in range(i + 1, min(len(ins), i + 3000)):
            u = ins[j]
            if u.startswith(("s_branch", "s_endpgm", "s_setpc_b64")):
                break
            m = re.match(r"s_waitcnt (.*)", u)
            if m:
                c = re.search(kind + r"cnt\((\d+)\)", m.group(1))
                if c and int(c.group(1)) <= younger:
                    break
                continue
            if (kind == "lgkm" and u.startswith(("ds_", "s_load"))) or \
               (kind == "vm" and u.startswith(("global_", "buffer_"))):
                younger += 1
            w, r = writes_reads(u)
            if dst & (w | r):
                out.append(f"[{t}] -> [{u}]: destination touched before its wait")
                break
    return out


STORE_WAIT = 2  # wait states before a VALU write of a >64-bit store's data VGPRs (gfx950)


def store_data_hazards(ins, labels):
    out = []
    for i, t in enumerate(ins):
        op, args = split_ops(t)
        if not re.match(r"(global|flat|scratch|buffer)_store_dwordx[34]$", op) or len(args) < 2:
            continue
        data = regs(args[0] if op.startswith("buffer") else args[1])

        def check(u, data=data):
            w, _ = writes_reads(u)
            return "writes the store's data" if w & data else None
        out += walk(ins, labels, i, STORE_WAIT, check)
    return out


def m0_hazards(lines):
    """Check 4 over the raw assembly: every ;;#ASMSTART .. ;;#ASMEND region that writes m0 saves
    it first (s_mov_b32 sN, m0) and restores it last (s_mov_b32 m0, sN), sN untouched between."""
    out = []
    region = None
    for l in lines + [";;#ASMSTART"]:
        t = l.split(";")[0].strip()
        if ";;#ASMSTART" in l:
            region = []
            continue
        if ";;#ASMEND" in l:
            if region is not None:
                out += _m0_region(region)
            region = None
            continue
        if region is not None and t and not t.endswith(":") and not t.startswith("."):
            region.append(t)
    return out


def _m0_region(ins):
    writes_m0 = [i for i, t in enumerate(ins) if re.match(r"s_\w+ m0\b", t)]
    if not writes_m0:
        return []
    saves = [i for i, t in enumerate(ins) if re.fullmatch(r"s_mov_b32 s\d+, m0", t)]
    if not saves or saves[0] > writes_m0[0]:
        return [f"[{ins[writes_m0[0]]}]: m0 written before it is saved"]
    reg = ins[saves[0]].split()[1].rstrip(",")
    last = writes_m0[-1]
    if ins[last] != f"s_mov_b32 m0, {reg}":
        return [f"[{ins[last]}]: the statement's last m0 write does not restore it from {reg}"]
    for t in ins[saves[0] + 1:last]:
        if re.match(rf"\S+ {reg}\b", t) or re.match(rf"\S+ s\[(\d+):(\d+)\]", t) and \
                int(re.match(rf"\S+ s\[(\d+):(\d+)\]", t).group(1)) <= int(reg[1:]) <= \
                int(re.match(rf"\S+ s\[(\d+):(\d+)\]", t).group(2)):
            return [f"[{t}]: overwrites the saved m0 in {reg}"]
    for t in ins[last + 1:]:
        if re.match(r"(global|buffer)_load\S*_lds|global_load_lds", t):
            return [f"[{t}]: an LDS copy after m0 was restored"]
    return []


_NO_SDST = ("s_cmp", "s_bitcmp", "s_cbranch", "s_branch", "s_waitcnt", "s_barrier", "s_nop",
            "s_setpc", "s_sleep", "s_endpgm", "s_dcache", "s_setprio", "s_sethalt", "s_trap")


def sgpr_regs(tok):
    tok = tok.split()[0] if tok else ""
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    if re.fullmatch(r"s\d+|vcc|exec|m0|scc", tok):
        return {tok}
    return set()


def scalar_writes(t):
    """Scalar registers (sN, vcc, exec, m0, scc) an instruction writes."""
    op, args = split_ops(t)
    out = set()
    if op.startswith("s_cmp") or op.startswith("s_bitcmp"):
        return {"scc"}
    if op.startswith("s_") and not op.startswith(_NO_SDST) and args:
        out |= sgpr_regs(args[0])
        if not op.startswith(("s_mov", "s_call", "s_getpc", "s_load", "s_memtime", "s_memrealtime",
                              "s_readfirstlane")):
            out.add("scc")
    elif op.startswith("v_cmp") and args and "_e64" in op:
        out |= sgpr_regs(args[0])
    elif op.startswith("v_cmp"):
        out.add("vcc")
    elif op.startswith(("v_readfirstlane", "v_readlane")) and args:
        out |= sgpr_regs(args[0])
    elif op.startswith("v_") and len(args) > 1 and op.startswith(("v_add_co", "v_addc_co", "v_sub_co",
                                                                    "v_subb_co", "v_mad_u64", "v_mad_i64")):
        out |= sgpr_regs(args[1])
    return out


def asm_statement_registers(hip_text):
    """Outputs, input-only operands and clobbers (register names) of the key-loop asm statement."""
    start = hip_text.index('#include "prefill_loop.inc"')
    end = hip_text.index("PFF_CLOBBERS);", start)
    body = hip_text[start:end]
    outs_txt, ins_txt = body.split("\n        : ", 2)[1:3] if body.count("\n        : ") >= 2 else (body, "")

    def names(txt, plus):
        found = set()
        for m in re.finditer(r'"(\+?)\{(v\[(\d+):(\d+)\]|v(\d+))\}"', txt):
            if bool(m.group(1)) != plus:
                continue
            if m.group(3):
                found |= {f"v{i}" for i in range(int(m.group(3)), int(m.group(4)) + 1)}
            else:
                found.add(f"v{m.group(5)}")
        return found
    outputs = names(outs_txt, True)
    inputs = names(ins_txt, False)
    mac = hip_text.index("#define PFF_CLOBBERS")
    mac_end = hip_text.index("\n\n", mac)
    clobbers = set(re.findall(r'"(v\d+|s\d+|vcc|scc|exec)"', hip_text[mac:mac_end]))
    return outputs, inputs, clobbers


def loop_instructions(inc_text):
    ins = []
    for l in inc_text.split("\n"):
        m = re.fullmatch(r'"(.*)\\n\\t"', l.strip())
        if m and not m.group(1).endswith(":"):
            ins.append(m.group(1))
    return ins


def undeclared_writes(inc_text, hip_text):
    """Check 5: instructions of the key loop that write a register the statement does not declare
    as written (m0 is covered by check 4)."""
    outputs, _, clobbers = asm_statement_registers(hip_text)
    declared = outputs | clobbers | {"m0"}
    out = []
    for t in loop_instructions(inc_text):
        w, _ = writes_reads(t)
        written = {f"v{i}" for i in w} | scalar_writes(t)
        bad = sorted(written - declared)
        if bad:
            out.append(f"[{t}]: writes {', '.join(bad)}, not an output or clobber of the statement")
    return out


def main(prefixes):
    undeclared = undeclared_writes(open(os.path.join(HERE, "prefill_loop.inc")).read(),
                                   open(os.path.join(HERE, "prefill_fast.hip")).read())
    print(f"key loop writes outside its outputs and clobbers: {len(undeclared)}")
    for p in undeclared[:10]:
        print("   ", p)
    lines = compile_asm()
    m0 = m0_hazards(lines)
    print(f"inline asm writing m0: {len(m0)} hazards")
    for p in m0[:10]:
        print("   ", p)
    heads = [l.split(";")[0].rstrip() for l in lines]
    kernels = sorted({h[:-1] for h in heads if re.match(r"^moearc_\w*_k\w*:$", h) or re.match(r"^moearc_attn_prefill_g\d+:$", h)})
    store = []
    for name in kernels:
        ins, labels = kernel_body(lines, name)
        store += [f"{name}: {p}" for p in store_data_hazards(ins, labels)]
    print(f"stores of more than 8 bytes with their data overwritten too soon, {len(kernels)} kernels: {len(store)}")
    for p in store[:10]:
        print("   ", p)
    names = sorted({h[:-1] for h in heads if re.match(r"^[A-Za-z_]\w*:$", h)
                    and any(h.startswith(p) for p in prefixes)})
    bad = 0
    for name in names:
        ins, labels = kernel_body(lines, name)
        probs = mfma_hazards(ins, labels) + load_hazards(ins) + valu_wait_hazards(ins, labels)
        print(f"{name}: {len(ins)} instructions, {len(probs)} hazards")
        for p in probs[:10]:
            print("   ", p)
        bad += len(probs)
    if not names:
        print("no kernel matches", prefixes)
        return 1
    return 1 if bad or m0 or undeclared or store else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:] or ["moearc_attn_prefill_g"]))
