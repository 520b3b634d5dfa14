//! Hand-written declarations of include/moearc_kv.h: the paged KV pool (the engine's
//! PagedKvCache, crates/moearc-engine/src/kv.rs:85-205) and the cache geometry (KvGeometry,
//! moe.rs:716-771), host-side bookkeeping in the same library.
//!
//! Codes: 0 ok; -1 null argument; -2 invalid argument; -3 exhausted (a = requested pages,
//! b = free pages); -4 unknown sequence; -5 context limit (a = tokens, b = limit); -6 invalid
//! geometry. The details of the last refusal come from `moearc_kv_pool_last_error`.

use std::os::raw::c_int;

#[repr(C)]
pub struct MoearcKvPool {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct MoearcKvUsage {
    pub total_pages: u32,
    pub used_pages: u32,
    pub sequences: u32,
    pub slack_tokens: u32,
}

unsafe extern "C" {
    pub fn moearc_kv_pool_create(
        total_pages: u32,
        page_tokens: u32,
        context_limit: u32,
        out: *mut *mut MoearcKvPool,
    ) -> c_int;
    pub fn moearc_kv_pool_destroy(p: *mut MoearcKvPool);
    pub fn moearc_kv_pool_last_error(p: *const MoearcKvPool, a: *mut u32, b: *mut u32) -> c_int;
    pub fn moearc_kv_pool_begin(p: *mut MoearcKvPool, seq: u64, prompt_tokens: u32) -> c_int;
    pub fn moearc_kv_pool_append(p: *mut MoearcKvPool, seq: u64, page: *mut u32, slot: *mut u32) -> c_int;
    pub fn moearc_kv_pool_append_chunk(
        p: *mut MoearcKvPool,
        seq: u64,
        n: u32,
        pages: *mut u32,
        slots: *mut u32,
    ) -> c_int;
    pub fn moearc_kv_pool_end(p: *mut MoearcKvPool, seq: u64, n_pages: *mut u32) -> c_int;
    pub fn moearc_kv_pool_pages(
        p: *const MoearcKvPool,
        seq: u64,
        pages: *mut u32,
        cap: u32,
        n_pages: *mut u32,
        tokens: *mut u32,
    ) -> c_int;
    pub fn moearc_kv_pool_can_admit(p: *const MoearcKvPool, tokens: u32) -> c_int;
    pub fn moearc_kv_pool_usage(p: *const MoearcKvPool, out: *mut MoearcKvUsage) -> c_int;
    pub fn moearc_kv_pool_block_tables(
        p: *const MoearcKvPool,
        seqs: *const u64,
        n_seqs: u32,
        stride: u32,
        table: *mut u32,
    ) -> c_int;
    pub fn moearc_kv_geometry(
        n_ctx: u32,
        page_tokens: u32,
        n_swa: u32,
        chunk: u32,
        pages: *mut u32,
        swa_pages: *mut u32,
    ) -> c_int;
    pub fn moearc_kv_ring_table(pages: u32, swa_pages: u32, table: *mut u32) -> c_int;
}
