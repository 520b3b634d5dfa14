// The single translation unit of the device code object (moearc_attn_gfx950.co), loaded at
// context creation with hipModuleLoad. Each included file holds one family of kernels.
#include "kernels_misc.hip"
#include "decode_general.hip"
#include "decode_splitk.hip"
#include "prefill.hip"
#include "prefill_fast.hip"
#include "rope.hip"
#include "matvec.hip"
#include "matmul.hip"
#include "matmul2.hip"
