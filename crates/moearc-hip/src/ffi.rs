//! Hand-written declarations of include/moearc_attn.h, the C ABI of libmoearc_attn.so.
//!
//! The reference engine's declarations (crates/moearc-kernels/src/ffi.rs:19-263) with the same
//! names, argument order and types for every entry point this library exports -- the lifecycle
//! and memory calls, the f16 codec, the KV append, attention, RoPE and the attention projections
//! -- followed by this library's extensions. Every function returns `0` when the work was
//! accepted (not completed), `-1` for a device failure or a null argument, and `-2` for an
//! argument out of range, with nothing enqueued.

use std::os::raw::{c_char, c_float, c_int, c_uint, c_ulong, c_void};

#[repr(C)]
pub struct MoearcCtx {
    _private: [u8; 0],
}

/// `moearc_attn_block` (include/moearc_attn.h): one block's attention weights, cache and RoPE.
#[repr(C)]
pub struct MoearcAttnBlock {
    pub w_type: [c_uint; 4],
    pub w: [*const c_void; 4],
    pub bias: [*const c_float; 4],
    pub sinks: *const c_float,
    pub k_pages: *mut c_void,
    pub v_pages: *mut c_void,
    pub block_table: *const c_uint,
    pub n_embd: c_ulong,
    pub n_head: c_ulong,
    pub n_head_kv: c_ulong,
    pub head_dim: c_ulong,
    pub page_tokens: c_ulong,
    pub n_swa: c_ulong,
    pub ring_pages: c_ulong,
    pub scale: c_float,
    pub n_rot: c_ulong,
    pub freq_base: c_float,
    pub freq_scale: c_float,
    pub ext_factor: c_float,
    pub attn_factor: c_float,
    pub corr_lo: c_float,
    pub corr_hi: c_float,
}

pub const MOEARC_OUT_F32: c_uint = 0;
pub const MOEARC_OUT_F16: c_uint = 1;

unsafe extern "C" {
    // ---- the reference's entry points (ffi.rs:20-51, :97-103, :167-173, :188-252) ----------
    pub fn moearc_ctx_create() -> *mut MoearcCtx;
    pub fn moearc_ctx_destroy(c: *mut MoearcCtx);
    pub fn moearc_profile_events_enabled(c: *mut MoearcCtx) -> c_int;
    pub fn moearc_profile_events_reset(c: *mut MoearcCtx) -> c_int;
    pub fn moearc_profile_events_report(c: *mut MoearcCtx, out: *mut c_char, cap: c_ulong) -> c_int;
    pub fn moearc_sync(c: *mut MoearcCtx) -> c_int;
    pub fn moearc_zero(c: *mut MoearcCtx, dst: *mut c_float, n: c_ulong) -> c_int;
    pub fn moearc_device_name(c: *mut MoearcCtx, out: *mut c_char, cap: c_ulong) -> c_int;
    pub fn moearc_alloc_device(c: *mut MoearcCtx, bytes: c_ulong) -> *mut c_void;
    pub fn moearc_free_device(c: *mut MoearcCtx, p: *mut c_void);
    pub fn moearc_copy_h2d(c: *mut MoearcCtx, dst: *mut c_void, src: *const c_void, bytes: c_ulong) -> c_int;
    pub fn moearc_copy_h2d_async(
        c: *mut MoearcCtx,
        dst: *mut c_void,
        src: *const c_void,
        bytes: c_ulong,
    ) -> c_int;
    pub fn moearc_copy_d2h(c: *mut MoearcCtx, dst: *mut c_void, src: *const c_void, bytes: c_ulong) -> c_int;
    pub fn moearc_matvec_q(
        c: *mut MoearcCtx,
        type_id: c_uint,
        out: *mut c_float,
        w: *const c_void,
        x: *const c_float,
        n_rows: c_ulong,
        n_cols: c_ulong,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_matvec_q_batched(
        c: *mut MoearcCtx,
        type_id: c_uint,
        out: *mut c_float,
        w: *const *const c_void,
        n_mat: c_uint,
        x: *const c_float,
        x_stride: c_ulong,
        n_rows: c_ulong,
        n_cols: c_ulong,
    ) -> c_int;
    pub fn moearc_matvec_f32(
        c: *mut MoearcCtx,
        out: *mut c_float,
        w: *const c_float,
        x: *const c_float,
        n_rows: c_ulong,
        n_cols: c_ulong,
    ) -> c_int;
    pub fn moearc_add(c: *mut MoearcCtx, out: *mut c_float, a: *const c_float, b: *const c_float, n: c_ulong) -> c_int;
    /// Calibration read (no counterpart in the reference): out[g] = xor of the g-th 64 KiB at src.
    pub fn moearc_read_floor(c: *mut MoearcCtx, out: *mut c_uint, src: *const c_void, bytes: c_ulong) -> c_int;
    /// Matrix-core calibration (no counterpart in the reference): dense f16 MFMA chains over the
    /// operands at src; out[w] = wave w's accumulator sum.
    pub fn moearc_mfma_floor(c: *mut MoearcCtx, out: *mut c_float, src: *const c_void, n_wgs: c_ulong, iters: c_ulong) -> c_int;
    pub fn moearc_quantize_f16(c: *mut MoearcCtx, dst: *mut c_void, src: *const c_float, n: c_ulong) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_kv_append(
        c: *mut MoearcCtx,
        k_pages: *mut c_void,
        v_pages: *mut c_void,
        k: *const c_float,
        v: *const c_float,
        page_id: c_uint,
        slot: c_uint,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_decode(
        c: *mut MoearcCtx,
        out: *mut c_float,
        q: *const c_float,
        k_pages: *const c_void,
        v_pages: *const c_void,
        block_table: *const c_uint,
        sinks: *const c_float,
        n_heads: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        kv_begin: c_ulong,
        n_kv: c_ulong,
        page_tokens: c_ulong,
        scale: c_float,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_rope(
        c: *mut MoearcCtx,
        dst: *mut c_float,
        src: *const c_float,
        pos: *const c_int,
        n_tokens: c_ulong,
        n_heads: c_ulong,
        head_dim: c_ulong,
        n_dims: c_ulong,
        freq_base: c_float,
        freq_scale: c_float,
        ext_factor: c_float,
        attn_factor: c_float,
        corr_lo: c_float,
        corr_hi: c_float,
        neox: c_int,
    ) -> c_int;

    // ---- extensions (include/moearc_attn.h; same conventions) ---------------------------------
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_decode_batched(
        c: *mut MoearcCtx,
        out: *mut c_void,
        out_type: c_uint,
        q: *const c_float,
        k_pages: *const c_void,
        v_pages: *const c_void,
        block_tables: *const c_uint,
        bt_stride: c_ulong,
        kv_begin: *const c_uint,
        n_kv: *const c_uint,
        sinks: *const c_float,
        n_seqs: c_ulong,
        n_heads: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        scale: c_float,
        kv_type: c_uint,
    ) -> c_int;
    /// Allocation-free form of `moearc_attn_decode_batched` (no counterpart in the reference): for
    /// callers that cannot allocate (HIP graph capture, serving loops); partial records go to a
    /// fixed 8 MiB array of the code object, a call too large for it is refused with -2.
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_decode_batched_noalloc(
        c: *mut MoearcCtx,
        out: *mut c_void,
        out_type: c_uint,
        q: *const c_float,
        k_pages: *const c_void,
        v_pages: *const c_void,
        block_tables: *const c_uint,
        bt_stride: c_ulong,
        kv_begin: *const c_uint,
        n_kv: *const c_uint,
        sinks: *const c_float,
        n_seqs: c_ulong,
        n_heads: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        scale: c_float,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_prefill(
        c: *mut MoearcCtx,
        out: *mut c_void,
        out_type: c_uint,
        q: *const c_void,
        k_pages: *const c_void,
        v_pages: *const c_void,
        block_table: *const c_uint,
        sinks: *const c_float,
        n_q: c_ulong,
        pos0: c_ulong,
        n_swa: c_ulong,
        n_heads: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        scale: c_float,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_kv_append_chunk(
        c: *mut MoearcCtx,
        k_pages: *mut c_void,
        v_pages: *mut c_void,
        k: *const c_float,
        v: *const c_float,
        page_ids: *const c_uint,
        slots: *const c_uint,
        n_tok: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_rope_kv_append_chunk(
        c: *mut MoearcCtx,
        k_pages: *mut c_void,
        v_pages: *mut c_void,
        k: *const c_float,
        v: *const c_float,
        pos: *const c_int,
        page_ids: *const c_uint,
        slots: *const c_uint,
        n_tok: c_ulong,
        n_kv_heads: c_ulong,
        head_dim: c_ulong,
        page_tokens: c_ulong,
        n_dims: c_ulong,
        freq_base: c_float,
        freq_scale: c_float,
        ext_factor: c_float,
        attn_factor: c_float,
        corr_lo: c_float,
        corr_hi: c_float,
        neox: c_int,
        kv_type: c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_qkv(
        c: *mut MoearcCtx,
        type_ids: *const c_uint,
        out: *const *mut c_float,
        w: *const *const c_void,
        bias: *const *const c_float,
        rows: *const c_ulong,
        x: *const c_float,
        n_cols: c_ulong,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_matmul_q(
        c: *mut MoearcCtx,
        type_id: c_uint,
        y: *mut c_float,
        w: *const c_void,
        x: *const c_float,
        bias: *const c_float,
        n_tok: c_ulong,
        n_rows: c_ulong,
        n_cols: c_ulong,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_block_chunk(
        c: *mut MoearcCtx,
        b: *const MoearcAttnBlock,
        h: *mut c_float,
        x: *const c_float,
        n_tok: c_ulong,
        pos0: c_ulong,
        pos: *const c_int,
        page_ids: *const c_uint,
        slots: *const c_uint,
    ) -> c_int;
    #[allow(clippy::too_many_arguments)]
    pub fn moearc_attn_out(
        c: *mut MoearcCtx,
        type_id: c_uint,
        h: *mut c_float,
        w: *const c_void,
        bias: *const c_float,
        attn: *const c_float,
        n_rows: c_ulong,
        n_cols: c_ulong,
    ) -> c_int;
    pub fn moearc_ctx_stream(c: *mut MoearcCtx) -> *mut c_void;
}
