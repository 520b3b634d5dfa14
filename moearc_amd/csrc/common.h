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
