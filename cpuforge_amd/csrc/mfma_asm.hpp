// Scheduling fences and inline-assembly MFMA accumulation shared by the
// hand-scheduled one-wave-per-SIMD kernels (attn_dkdv.hip, attn_fwd_q64.hip).
//
// Those kernels keep their long-lived accumulators in AGPRs and everything
// the VALU reads in VGPRs.  The compiler gives every MFMA of a function one
// register form, so the accumulating MFMAs are inline assembly ("+a") and
// the score MFMAs compiler builtins built for the VGPR form
// (-mllvm -amdgpu-mfma-vgpr-form=1).  The compiler's hazard recognizer does
// not see inside the assembly: the code provides the wait states itself --
// CF_HAZARD_FENCE before an MFMA whose operands a VALU instruction just
// wrote, acc_wait8 (34 wait states, the 8 passes of a 32x32x16 MFMA plus
// the write-back) before any compiler-generated read or copy of an
// accumulator, and acc_ready8 or mfma_acc_lead after any such copy, before
// the next MFMA.
#pragma once
#include "cfattn_common.hpp"

// No instruction is scheduled across this point.
#define CF_FENCE() __builtin_amdgcn_sched_barrier(0)
// A fence with two wait states in it: the operand registers a VALU
// instruction wrote just before must not be read by an MFMA issued from
// inline assembly in the next two cycles.
#define CF_HAZARD_FENCE()                  \
    do {                                   \
        __builtin_amdgcn_sched_barrier(0); \
        asm volatile("s_nop 1");           \
        __builtin_amdgcn_sched_barrier(0); \
    } while (0)

namespace cfattn {

// acc += a * b with acc in AGPRs.  Back-to-back MFMAs accumulating into the
// same registers need no wait states.
__device__ __forceinline__ void mfma_acc(f32x16& acc, const bf16x8& a, const bf16x8& b) {
    asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same behind two wait states, for the first MFMA into an accumulator
// in a block where the compiler may have just copied the accumulator to
// the registers the MFMA reads (the wait a VALU write needs before an MFMA
// reads the register).
__device__ __forceinline__ void mfma_acc_lead(f32x16& acc, const bf16x8& a, const bf16x8& b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Keeps a value in AGPRs from here on (ties its registers to an empty asm).
__device__ __forceinline__ void agpr_pin(f32x16& acc) { asm volatile("" : "+a"(acc)); }

// 34 wait states tied to eight accumulators: the MFMAs that last wrote
// them have completed before anything after this reads them.
__device__ __forceinline__ void acc_wait8(f32x16& a0, f32x16& a1, f32x16& a2, f32x16& a3, f32x16& a4, f32x16& a5,
                                          f32x16& a6, f32x16& a7) {
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 3"
                 : "+a"(a0), "+a"(a1), "+a"(a2), "+a"(a3), "+a"(a4), "+a"(a5), "+a"(a6), "+a"(a7));
}

// Five wait states tied to eight accumulators, right before the MFMAs that
// accumulate into them: the compiler may copy the accumulators to other
// registers where control flow joins (v_accvgpr_mov), and an MFMA reading
// a register such a copy just wrote as its accumulator input needs wait
// states the compiler does not insert for inline assembly.
__device__ __forceinline__ void acc_ready8(f32x16& a0, f32x16& a1, f32x16& a2, f32x16& a3, f32x16& a4, f32x16& a5,
                                           f32x16& a6, f32x16& a7) {
    asm volatile("s_nop 4"
                 : "+a"(a0), "+a"(a1), "+a"(a2), "+a"(a3), "+a"(a4), "+a"(a5), "+a"(a6), "+a"(a7));
}

}  // namespace cfattn
