"""Generates prefill_loop.inc: the key loop of the default prefill kernels (prefill_fast.hip) as one
gfx950 inline-asm statement.

Why asm: the loop keeps ~180 VGPRs of state (four 16-register O accumulators, two score tuples,
Q, K and V^T operands). Written in C++, the compiler's allocator copies whole
accumulator tuples at every join and spills; and register constraints on separate asm statements
do not pin a value between them. One asm statement over a fixed register map does.

Run `python gen_prefill_loop.py` after editing; the output is committed (the build does not run
this script).

Register map (VGPRs):
  v0-v15 v16-v31     O of block A, channel blocks 0 and 1      v128-v143  Q of block A (4 x half8)
  v32-v47 v48-v63    O of block B                              v144-v159  Q of block B
  v64-v79 v80-v95    S of blocks A and B (exponents, weights)  v160-v175  K operands of a chunk
  v96 v112           bias 7 - m of blocks A and B (per row)    v176-v191  V^T operands of a chunk
  v100-v103 v104-v107  row sums of blocks A and B (16x16x32 MFMA accumulators: register 0 of lane
                     n < 32 holds row n's sum, every other element stays 0)
  v108-v111          the selection operand of the row-sum MFMAs (v97-v99, v113-v127 are not used)
  v192-v199          P operands (one block at a time)          v200-v207  temporaries
  v208 v209          reference m of A, B                       v210 v211  unused
  v212-v215          LDS addresses of the K operand reads (buffer 0, chunk 0)
  v216-v217          LDS addresses of the V^T operand reads
  v218 v219 v220 v221  mask parameters c_A, span_A, c_B, span_B (key offset of chunk 0 relative to
                     the row's window start; row position minus window start)
  v222-v229          block-table entries of four tiles (two per tile: this lane's two copy keys;
                     tiles 0 and 1 are inputs of the statement)
  v230-v233          copy offsets within a tile, uniform path (K copy 0, 1, V copy 0, 1)
  v234-v241          per-lane 64-bit copy bases (K copy 0, 1, V copy 0, 1): pages base + chunk
  v242               this lane's first copy key within a tile (16 * wave + lane / 8)
  v243               ds_bpermute address of lane ^ 32
  v244-v247          temporaries                               v248-v249  block-table base (64-bit)
  v250-v255          unused
SGPRs s64-s85 are the loop's own (listed as clobbers); s[82:83] and s[84:85] hold the rescale tests
of blocks A and B (lanes whose chunk exponents reach the threshold %[thr]).
"""
import os

HERE = os.path.dirname(os.path.abspath(__file__))
NBUF = 4          # LDS tile buffers
BUF = 16384       # bytes per buffer: K tile (8 KiB) + V tile (8 KiB)
TILE = 8192

out = []
ool = []  # out-of-line blocks (rare paths), emitted after the main loop


def ins(s):
    out.append(s)


def ool_block(label, body, back):
    """A rare path placed after the loop: `label`, its instructions, a branch back to `back`. The
    common path reaches it by a conditional branch that is normally not taken (falls through)."""
    ool.extend([f"{label}:", *body, f"s_branch {back}"])


def mfma(d, a, b, c):
    ins(f"v_mfma_f32_32x32x16_f16 v[{d}], v[{a}], v[{b}], {c}")


K_OPS = ["160:163", "164:167", "168:171", "172:175"]


def qk_exp(sd, q0, e):
    """S_D = K . Q^T, the raw scores (4 chained MFMAs from zero), beside the 16 exponentials of the
    weights in v[e..e+15] (in place), four after each MFMA."""
    qs = [f"{q0 + 4 * t}:{q0 + 4 * t + 3}" for t in range(4)]
    for t in range(4):
        mfma(sd, K_OPS[t], qs[t], "0" if t == 0 else f"v[{sd}]")
        for i in range(4 * t, 4 * t + 4):
            ins(f"v_exp_f32 v{e + i}, v{e + i}")


def fma_ops(e, bias):
    """Exponent inputs of the raw scores v[e..e+15], in place: x = s * c + bias, c = scale * log2(e)
    in f32 (Q enters the MFMA as the caller's exact f16 values) and bias = 7 - m of the lane's row."""
    return [f"v_fma_f32 v{e + i}, v{e + i}, %[cs], v{bias}" for i in range(16)]


def max_ops(e, flag):
    """Largest exponent input of v[e..e+15] (two chains in v244, v245: free outside tile steps and
    the mask and rescale paths) compared with the rescale threshold: s[flag:flag+1] = lanes whose
    weights could leave f16's range."""
    E = list(range(e, e + 16))
    m3 = lambda d, x, y, z: f"v_max3_f32 v{d}, v{x}, v{y}, v{z}"
    return [m3(244, E[0], E[1], E[2]), m3(245, E[3], E[4], E[5]), m3(244, 244, E[6], E[7]),
            m3(245, 245, E[8], E[9]), m3(244, 244, E[10], E[11]), m3(245, 245, E[12], E[13]),
            m3(244, 244, 245, E[14]), f"v_max_f32 v244, v244, v{E[15]}",
            f"v_cmp_le_f32_e64 s[{flag}:{flag + 1}], %[thr], v244"]


def rowsum(lsum, p):
    """l += the chunk's weights of every row, on the matrix core: a 16x16x32 MFMA whose B operand is
    the block's P^T registers read as 32 keys x 16 columns (lane l then holds row l % 32's keys
    8 (l / 32) .. + 7 of the 16-key half, in column l % 16, k-slots 8 (l / 16) .. + 7) and whose A
    operand (v108-v111) has ones in row 0 over the k-slots of lanes 0-15 and 32-47 (rows 0-15) and in
    row 4 over those of lanes 16-31 and 48-63 (rows 16-31): D[0][n] is row n's sum and D[4][n] row
    n + 16's, which the accumulator layout places in register 0 of lanes n and n + 16."""
    ins(f"v_mfma_f32_16x16x32_f16 v[{lsum}], v[108:111], v[{p}], v[{lsum}]")


def pv(o0, o1, e, extra, lsum, pad=0):
    """O_0 += V^T(0, s) . P_s, O_1 += V^T(1, s) . P_s, P_s = f16 of weights v[e + 8s .. + 7], and
    the row sums l += P_s (`rowsum`, into v[lsum]), with the VALU instructions `extra` (not writing
    P or the V^T operands) spread between the MFMAs in four equal groups, one after each P.V MFMA.
    All eight P packs come first, so the first group -- the other block's exponent inputs, 16 FMAs
    on the scores of the previous region's MFMAs -- starts after the first P.V MFMA, at least 20
    wait states after those MFMAs (`pad` wait states more where the region before is short)."""
    cvt = lambda d, a, b: ins(f"v_cvt_pk_f16_f32 v{d}, v{e + a}, v{e + b}")
    extra = list(extra)
    take = lambda n: [ins(extra.pop(0)) for _ in range(min(n, len(extra)))]
    group = -(-len(extra) // 4)
    cvt(192, 0, 1); cvt(193, 2, 3); cvt(194, 4, 5); cvt(195, 6, 7)
    cvt(196, 8, 9); cvt(197, 10, 11); cvt(198, 12, 13); cvt(199, 14, 15)
    mfma(o0, "176:179", "192:195", f"v[{o0}]")
    if pad:
        ins(f"s_nop {pad - 1}")
    take(group)
    mfma(o1, "184:187", "192:195", f"v[{o1}]")
    rowsum(lsum, "192:195")
    take(group)
    mfma(o0, "180:183", "196:199", f"v[{o0}]")
    take(group)
    mfma(o1, "188:191", "196:199", f"v[{o1}]")
    rowsum(lsum, "196:199")
    take(len(extra))


def read_k(off, dst="160"):
    d = int(dst)
    for t in range(4):
        ins(f"ds_read_b128 v[{d + 4 * t}:{d + 4 * t + 3}], v{212 + t} offset:{off}")


def read_v(off):
    # operand (mb, s) at v[176 + 8mb + 4s]: low half keys 16s + 4h.., high half 16s + 8 + 4h..
    for mb in range(2):
        for e in range(4):
            r = 176 + 8 * mb + 2 * e
            ins(f"ds_read_b64_tr_b16 v[{r}:{r + 1}], v{216 + mb} offset:{off + 1024 * e}")


def pid_load(slot, tile_sgpr, label):
    """Block-table entries of tile s[tile_sgpr] (clamped to the last tile) for this lane's two copy
    keys (clamped to the last query position) into v[222 + 2 slot], v[223 + 2 slot]."""
    ins(f"s_min_u32 s79, s{tile_sgpr}, %[ntm1]")
    ins("s_lshl_b32 s79, s79, 6")
    ins("s_add_u32 s79, s79, %[kb0]")
    for i in range(2):
        ins(f"v_add3_u32 v244, s79, v242, {8 * i}")
        ins("v_min_u32 v244, %[plast], v244")
        ins("v_lshrrev_b32 v244, %[sh], v244")
        ins("v_lshlrev_b32 v244, 2, v244")
        ins("v_add_co_u32 v246, vcc, v248, v244")
        ins("v_addc_co_u32 v247, vcc, 0, v249, vcc")
        ins(f"global_load_dword v{222 + 2 * slot + i}, v[246:247], off")


def copy_tile(slot, tile_sgpr, buf, label):
    """LDS-DMA copy of tile s[tile_sgpr] (clamped) into buffer `buf` with the entries in `slot`:
    wave-uniform scalar-base form when the tile's 64 keys lie in one page (tiles start on a 32-key
    boundary, so a tile may straddle two pages) wholly below the last query position, per-lane
    addresses otherwise (out of line). Four memory operations either way."""
    ins(f"s_min_u32 s71, s{tile_sgpr}, %[ntm1]")
    ins("s_lshl_b32 s70, s71, 6")
    ins("s_add_u32 s70, s70, %[kb0]")          # first key of the tile
    ins("s_add_u32 s73, s70, 63")
    ins("s_cmp_gt_u32 s73, %[plast]")
    ins(f"s_cbranch_scc1 {label}_lane")
    ins("s_and_b32 s73, s70, %[pmask]")        # the tile's first key within its page
    ins("s_add_u32 s79, s73, 63")
    ins("s_cmp_gt_u32 s79, %[pmask]")          # last key past the page's end (always for pages < 64)
    ins(f"s_cbranch_scc1 {label}_lane")
    ins(f"v_readfirstlane_b32 s72, v{222 + 2 * slot}")
    ins("s_lshl_b32 s72, s72, %[sh]")
    ins("s_or_b32 s72, s72, s73")               # row of the tile's first key
    ins("s_mul_i32 s74, s72, %[rowb]")
    ins("s_mul_hi_u32 s75, s72, %[rowb]")       # byte offset of the row (64-bit)
    for kind, base, voff in (("k", "kp", (230, 231)), ("v", "vp", (232, 233))):
        ins(f"s_add_u32 s68, s74, %[{base}lo]")
        ins(f"s_addc_u32 s69, s75, %[{base}hi]")
        for i in range(2):
            lds_off = buf * BUF + (TILE if kind == "v" else 0) + 1024 * i
            ins(f"s_add_u32 m0, %[ldsw], {lds_off}")
            ins("s_nop 0")
            ins(f"global_load_lds_dwordx4 v{voff[i]}, s[68:69]")
    ins(f"{label}_done:")
    lane = []
    for i in range(2):
        lane.append(f"v_add3_u32 v244, s70, v242, {8 * i}")
        lane.append("v_min_u32 v244, %[plast], v244")
        lane.append("v_and_b32 v244, %[pmask], v244")
        lane.append(f"v_lshlrev_b32 v245, %[sh], v{222 + 2 * slot + i}")
        lane.append("v_or_b32 v244, v244, v245")         # row of this lane's key
        for kind, pair in (("k", 234 + 2 * i), ("v", 238 + 2 * i)):
            lane.append(f"v_mad_u64_u32 v[246:247], vcc, v244, %[rowb], v[{pair}:{pair + 1}]")
            lds_off = buf * BUF + (TILE if kind == "v" else 0) + 1024 * i
            lane.append(f"s_add_u32 m0, %[ldsw], {lds_off}")
            lane.append("s_nop 0")
            lane.append("global_load_lds_dwordx4 v[246:247], off")
    ool_block(f"{label}_lane", lane, f"{label}_done")


def tile_step(si, label):
    """Tile step t = s65: wait for this wave's copies of tile t and the entries of tile t + 2,
    meet the other waves, copy tile t + 2 into buffer (t + 2) % 4, load the entries of tile t + 4.
    Six memory operations per step, so the wait is vmcnt(6); tiles past the last are not copied,
    so the step after the last copy (t + 1 >= ntiles) waits vmcnt(2), its predecessor's two entry
    loads being the only younger operations."""
    sc = (si + 2) % NBUF
    # a pair's second work-group leaves its raised issue priority at tile %[btile]
    ins("s_cmp_eq_u32 s65, %[btile]")
    ins(f"s_cbranch_scc0 {label}_np")
    ins("s_setprio 0")
    ins(f"{label}_np:")
    if label == "pro_t0":
        ins("s_waitcnt vmcnt(6)")
    else:
        # the step before the last issued no copies (tile t + 1 past the last): its two entry loads
        # are the only younger memory operations
        ins("s_add_u32 s79, s65, 1")
        ins("s_cmp_ge_u32 s79, %[ntiles]")
        ins(f"s_cbranch_scc1 {label}_w2")
        ins("s_waitcnt vmcnt(6)")
        ins(f"{label}_wd:")
        ool_block(f"{label}_w2", ["s_waitcnt vmcnt(2)"], f"{label}_wd")
    ins("s_barrier")
    ins("s_add_u32 s80, s65, 2")
    # no copies of tiles past the last (the clamped copy would repeat the last tile into a buffer
    # nothing reads, and the loop's end would wait for it)
    ins("s_cmp_ge_u32 s80, %[ntiles]")
    ins(f"s_cbranch_scc1 {label}_cd")
    copy_tile(sc, 80, sc, f"{label}_c")
    ins(f"{label}_cd:")
    ins("s_add_u32 s80, s65, 4")
    pid_load(si, 80, f"{label}_p")


def chunk(bi, ci, label):
    """Chunk j = s64 (32 keys): R1 S_B(j) MFMAs | exponentials of A(j); R2 O_A += V(j)^T P_A(j)
    and A(j)'s row sums (MFMAs) | f16 P_A(j), exponent inputs and rescale test of S_B(j); R3
    S_A(j + 1) | exponentials of B(j); R4 O_B += V(j)^T P_B(j) and B(j)'s row sums | f16 P_B(j),
    exponent inputs and rescale test of S_A(j + 1). Each rescale test is taken at the start of the
    next region that exponentiates the block, long after its compare."""
    bn = (bi + 1) % NBUF if ci else bi
    off = bi * BUF + 4096 * ci
    offn = bn * BUF + 4096 * (ci ^ 1)
    if ci == 1:
        # chunk j + 1 opens tile t = (j + 1) / 2
        ins("s_add_u32 s65, s64, 1")
        ins("s_lshr_b32 s65, s65, 1")
        ins("s_cmp_ge_u32 s65, %[ntiles]")
        ins(f"s_cbranch_scc1 {label}_nostep")
        tile_step(bn, f"{label}_t")
        ins(f"{label}_nostep:")
    # R1: S_B(j) | weights of A(j)
    ins("s_cmp_lg_u64 s[82:83], 0")
    ins(f"s_cbranch_scc1 {label}_ra")
    ins(f"{label}_a_ok:")
    ool_block(f"{label}_ra", ["s_mov_b32 s78, s64", "s_call_b64 s[66:67], pff_rescale_a"], f"{label}_a_ok")
    qk_exp("80:95", 144, 64)
    read_k(offn)
    # R2: mask of S_B(j); O_A += V(j)^T . P_A(j), row sums of A(j) | exponent inputs and rescale test of S_B(j)
    ins("s_waitcnt lgkmcnt(4)")
    ins("s_sub_u32 s79, s64, %[jlob]")
    ins("s_cmp_ge_u32 s79, %[jnb]")
    ins(f"s_cbranch_scc1 {label}_mb")
    ins(f"{label}_mb_ok:")
    ool_block(f"{label}_mb", ["s_mov_b32 s78, s64", "s_call_b64 s[66:67], pff_mask_b"], f"{label}_mb_ok")
    pv("0:15", "16:31", 64, fma_ops(80, 112) + max_ops(80, 84), "100:103")
    # R3: S_A(j + 1) | weights of B(j)
    ins("s_cmp_lg_u64 s[84:85], 0")
    ins(f"s_cbranch_scc1 {label}_rb")
    ins(f"{label}_b_ok:")
    ool_block(f"{label}_rb", ["s_mov_b32 s78, s64", f"s_mov_b32 s76, {off}", f"s_mov_b32 s77, {offn}",
                              "s_call_b64 s[66:67], pff_rescale_b"], f"{label}_b_ok")
    ins("s_waitcnt lgkmcnt(0)")
    qk_exp("64:79", 128, 80)
    # R4: mask of S_A(j + 1); O_B += V(j)^T . P_B(j), row sums of B(j) | exponent inputs and rescale test of S_A(j + 1)
    ins("s_sub_u32 s79, s64, %[jloa1]")           # (j + 1) - jlo_A
    ins("s_cmp_ge_u32 s79, %[jna]")
    ins(f"s_cbranch_scc1 {label}_ma")
    ins(f"{label}_ma_ok:")
    ool_block(f"{label}_ma", ["s_add_u32 s78, s64, 1", "s_call_b64 s[66:67], pff_mask_a"], f"{label}_ma_ok")
    pv("32:47", "48:63", 80, fma_ops(64, 96) + max_ops(64, 82), "104:107", pad=4)
    read_v(offn)
    ins("s_add_u32 s64, s64, 1")


def mask_body(e, c_reg, span_reg):
    """Keys of chunk s78 outside each row's span -> -inf in v[e..e+15]: key offset of register i
    is 8 (i >> 2) + (i & 3); outside iff c + 32 j + k > span (unsigned)."""
    ins("s_lshl_b32 s79, s78, 5")
    ins(f"v_add_u32 v244, s79, v{c_reg}")
    ins("v_mov_b32 v245, 0xff800000")
    for i in range(16):
        k = 8 * (i >> 2) + (i & 3)
        ins(f"v_add_u32 v246, {k}, v244")
        ins(f"v_cmp_gt_u32 vcc, v246, v{span_reg}")
        ins(f"v_cndmask_b32 v{e + i}, v{e + i}, v245, vcc")


def rescale_body(sd, e, q0, o_base, bias_base, m, l, c_reg, span_reg, jlo, jn, label):
    """Raw scores of the chunk (K in v160-v175) -> v[e..], masked if the chunk needs it, the row
    maximum across lanes n and n + 32, m moved to it, O, l and the bias rescaled, and the exponent
    inputs redone with the new bias (the caller exponentiates them)."""
    E = list(range(e, e + 16))
    qs = [f"{q0 + 4 * t}:{q0 + 4 * t + 3}" for t in range(4)]
    mfma(sd, K_OPS[0], qs[0], "0")
    for t in (1, 2, 3):
        mfma(sd, K_OPS[t], qs[t], f"v[{sd}]")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")  # MFMA results -> VALU
    ins(f"s_sub_u32 s79, s78, {jlo}")
    ins(f"s_cmp_lt_u32 s79, {jn}")
    ins(f"s_cbranch_scc1 {label}_nm")
    mask_body(e, c_reg, span_reg)
    ins(f"{label}_nm:")
    for i in range(16):  # log2-domain scores (masked keys stay -inf: c > 0)
        ins(f"v_mul_f32 v{E[i]}, %[cs], v{E[i]}")
    ins(f"v_max3_f32 v200, v{E[0]}, v{E[1]}, v{E[2]}")
    for i in range(3, 15, 2):
        ins(f"v_max3_f32 v200, v200, v{E[i]}, v{E[i + 1]}")
    ins(f"v_max_f32 v200, v200, v{E[15]}")
    ins("ds_bpermute_b32 v202, v243, v200")
    ins("s_waitcnt lgkmcnt(0)")
    ins(f"v_max3_f32 v202, v202, v200, v{m}")      # m_new
    ins(f"v_sub_f32 v203, v{m}, v202")
    ins("v_exp_f32 v203, v203")                      # corr = 2^(m_old - m_new)
    ins(f"v_mov_b32 v{m}, v202")
    ins("v_sub_f32 v204, 0x40e00000, v202")          # bias = 7 - m_new
    ins(f"v_mul_f32 v{l}, v{l}, v203")
    for i in range(32):
        ins(f"v_mul_f32 v{o_base + i}, v{o_base + i}, v203")
    ins(f"v_mov_b32 v{bias_base}, v204")
    for i in range(16):
        ins(f"v_add_f32 v{E[i]}, v{E[i]}, v204")


def first_max(e, m, bias, inputs):
    """m = max(m, the row maximum of the log2-domain scores of v[e..e+15] over lanes n and n + 32),
    bias = 7 - m; with `inputs`, v[e..] become the exponent inputs (s c) + bias, as the rescale
    path leaves them."""
    E = list(range(e, e + 16))
    for i in range(16):
        ins(f"v_mul_f32 v{E[i]}, %[cs], v{E[i]}")
    ins(f"v_max3_f32 v200, v{E[0]}, v{E[1]}, v{E[2]}")
    for i in range(3, 15, 2):
        ins(f"v_max3_f32 v200, v200, v{E[i]}, v{E[i + 1]}")
    ins(f"v_max_f32 v200, v200, v{E[15]}")
    ins("ds_bpermute_b32 v202, v243, v200")
    ins("s_waitcnt lgkmcnt(0)")
    ins(f"v_max3_f32 v202, v202, v200, v{m}")
    ins(f"v_mov_b32 v{m}, v202")
    ins(f"v_sub_f32 v{bias}, 0x40e00000, v202")
    if inputs:
        for i in range(16):
            ins(f"v_add_f32 v{E[i]}, v{E[i]}, v{bias}")


def generate():
    # m0 (the LDS base of the copies) is the compiler's register: saved here, restored at the one
    # exit, so the statement leaves it as it found it and needs no m0 clobber
    ins("s_mov_b32 s86, m0")
    # ---- prologue: copies of tiles 0 and 1 (their entries arrive as inputs in v222-v225, loaded
    # beside the query rows before the statement, so the two loads share one memory round trip),
    # entries of tiles 2 and 3, step 0, both blocks' reference m from chunk 0 ----
    ins("s_mov_b32 s80, 0")
    copy_tile(0, 80, 0, "pro_c0")
    ins("s_mov_b32 s80, 2")
    pid_load(2, 80, "pro_p2")
    ins("s_mov_b32 s80, 1")
    copy_tile(1, 80, 1, "pro_c1")
    ins("s_mov_b32 s80, 3")
    pid_load(3, 80, "pro_p3")
    ins("s_mov_b32 s65, 0")
    tile_step(0, "pro_t0")
    # chunk 0's K and V^T operands, S_A(0), its mask
    read_k(0)
    read_v(0)
    ins("s_waitcnt lgkmcnt(8)")
    mfma("64:79", K_OPS[0], "128:131", "0")
    for t in (1, 2, 3):
        mfma("64:79", K_OPS[t], f"{128 + 4 * t}:{131 + 4 * t}", "v[64:79]")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_mov_b32 s64, 0")
    ins("s_mov_b32 s78, 0")
    ins("s_sub_u32 s79, 0, %[jloa]")
    ins("s_cmp_lt_u32 s79, %[jna]")
    ins("s_cbranch_scc1 pro_ma_ok")
    ins("s_call_b64 s[66:67], pff_mask_a")
    ins("pro_ma_ok:")
    # S_B(0) too (R1 of chunk 0 computes it again for the loop), masked
    mfma("80:95", K_OPS[0], "144:147", "0")
    for t in (1, 2, 3):
        mfma("80:95", K_OPS[t], f"{144 + 4 * t}:{147 + 4 * t}", "v[80:95]")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_sub_u32 s79, 0, %[jlob]")
    ins("s_cmp_lt_u32 s79, %[jnb]")
    ins("s_cbranch_scc1 pro_mb_ok")
    ins("s_call_b64 s[66:67], pff_mask_b")
    ins("pro_mb_ok:")
    # each block's reference m starts at chunk 0's row maximum (no rescale of chunk 0); A's exponent
    # inputs follow, B's are taken by the loop's first R2
    first_max(64, 208, 96, True)
    first_max(80, 209, 112, False)
    ins("s_mov_b64 s[82:83], 0")
    # ---- main loop: four tiles (eight chunks) per pass; buffers and entry slots fixed ----
    # (the chunk count may be odd: the loop can end after a tile's first chunk)
    ins("pff_loop:")
    for k in range(NBUF):
        for ci in range(2):
            chunk(k, ci, f"c{k}{ci}")
            ins("s_cmp_ge_u32 s64, %[nc]")
            ins("s_cbranch_scc1 pff_end")
    ins("s_branch pff_loop")
    out.extend(ool)
    # ---- rare paths (called with s_call_b64 s[66:67], return with s_setpc_b64) ----
    ins("pff_mask_a:")  # called soon after the MFMAs that wrote S_A
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")
    mask_body(64, 218, 219)
    ins("s_setpc_b64 s[66:67]")
    ins("pff_mask_b:")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")
    mask_body(80, 220, 221)
    ins("s_setpc_b64 s[66:67]")
    ins("pff_rescale_a:")  # K(j) is in v160-v175
    rescale_body("64:79", 64, 128, 0, 96, 208, 100, 218, 219, "%[jloa]", "%[jna]", "ra")
    ins("s_setpc_b64 s[66:67]")
    ins("pff_rescale_b:")  # K(j + 1) is in v160-v175: read K(j) (LDS offset s76), then K(j + 1) (s77)
    for t in range(4):
        ins(f"v_add_u32 v{244 + t}, s76, v{212 + t}")
    ins("s_waitcnt lgkmcnt(0)")
    for t in range(4):
        ins(f"ds_read_b128 v[{160 + 4 * t}:{163 + 4 * t}], v{244 + t}")
    ins("s_waitcnt lgkmcnt(0)")
    rescale_body("80:95", 80, 144, 32, 112, 209, 104, 220, 221, "%[jlob]", "%[jnb]", "rb")
    for t in range(4):
        ins(f"v_add_u32 v{244 + t}, s77, v{212 + t}")
    for t in range(4):
        ins(f"ds_read_b128 v[{160 + 4 * t}:{163 + 4 * t}], v{244 + t}")
    ins("s_waitcnt lgkmcnt(0)")
    ins("s_setpc_b64 s[66:67]")
    # ---- end: every copy and read has landed; the last MFMA results are readable ----
    ins("pff_end:")
    ins("s_mov_b32 m0, s86")
    ins("s_waitcnt vmcnt(0) lgkmcnt(0)")
    ins("s_nop 7")
    ins("s_nop 7")
    ins("s_nop 7")


def emit():
    import re
    generate()
    # labels get the asm statement's unique number (%=) so that several kernels can inline it
    label_defs = sorted({l[:-1] for l in out if l.endswith(":")}, key=len, reverse=True)

    def fix(line):
        for lab in label_defs:
            line = re.sub(r"\b" + re.escape(lab) + r"\b", lab + "_%=", line)
        return line

    lines = [fix(l) for l in out]
    path = os.path.join(HERE, "prefill_loop.inc")
    with open(path, "w") as f:
        f.write("// Generated by gen_prefill_loop.py: the key loop of the default prefill kernels as one\n")
        f.write("// gfx950 asm statement (register map and semantics in that script and prefill_fast.hip).\n")
        for l in lines:
            f.write('"' + l + '\\n\\t"\n')
    print(f"wrote {path}: {len(lines)} instructions and labels")


if __name__ == "__main__":
    emit()
