//! The thin FFI crate between the reference engine and the MI355X attention path.
//!
//! `ffi` declares include/moearc_attn.h -- for the reference's own entry points, exactly the
//! declarations of crates/moearc-kernels/src/ffi.rs, so the reference's safe wrapper
//! (crates/moearc-kernels/src/lib.rs: `Context`, `DeviceBuffer`, the drain-before-error rule of
//! lib.rs:198-215) binds this library unchanged for the attention path -- and `kv_ffi` the paged
//! KV pool of include/moearc_kv.h. build.rs compiles the HIP sources for gfx950 and links
//! libmoearc_attn.so by absolute soname, as the reference's build.rs links its SYCL object.

pub mod ffi;
pub mod kv_ffi;

/// Return codes of every `ffi` entry point.
pub const OK: i32 = 0;
/// A null argument, or a HIP call failed.
pub const ERR: i32 = -1;
/// An argument out of range; nothing was enqueued.
pub const ERR_ARG: i32 = -2;
