// Shared device-side definitions for the gfx950 attention kernels.
//
// Only HIP for CDNA4 (gfx950): 64-lane wavefronts, MFMA f16 matrix ops, 160 KiB of LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#include "launch_args.h"

// log2(e) in f32: exp(x) = exp2(x * log2(e)).
#define MOEARC_LOG2E 1.4426950408889634f

// A 16-byte store written through to the device-coherent level (sc1, as an agent-scope store): a
// kernel's end then has no dirty L2 lines of it to write back, which for outputs of tens of MB is
// microseconds of the dispatch. It pays for whole-line writes (the prefill's output rows); 4-byte
// pieces written this way measured slower (the chunk product's epilogue: +7%), the L2 no longer
// merging them into lines.
// The store reads its 16 data bytes after issue: no VALU instruction may overwrite them within 2
// wait states on gfx950 (hipcc puts s_nop 1 between its own 16-byte stores and such a write, but
// knows nothing of an asm one). With a single wait state the split's stores wrote, now and then
// under load, the register's next value (the f32 of hi) into the first dword of a piece.
__device__ __forceinline__ void store_through16(void *p, u32x4_t v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_through8(void *p, u32x2_t v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
