// w4a16_device.h -- device helpers shared by the gfx950 kernel files
// (w4a16_kernels.hip, w4a16_head.hip): vector types and the MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4k {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// D = A * B + D with a tied accumulator.  Issued from asm so that the
// accumulator keeps its registers for the whole K loop: left to itself the
// compiler may give an MFMA a SrcC different from its Dst and hand the freed
// SrcC registers to the next instruction while the MFMA still reads them,
// which it guards against only for writers it can see (not dequant8).
// s_nop 1 first: gfx950 needs 2 wait states between a VALU write of a VGPR
// and an MFMA read of it (A/B come from dequant8 and from zero fills).
// Back-to-back MFMAs accumulating into the same registers need none.
__device__ __forceinline__ void mfma_acc(floatx4& acc, const bf16x8& a, const bf16x8& b) {
  asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

// Wait states after the last MFMA before any VALU / memory instruction reads
// its result (the compiler does not count them after inline asm).  Needed at
// every point where compiler-generated code may touch the accumulator: after
// the K loop, and at the end of every loop body or chunk, since at control-flow
// joins the compiler may copy the accumulator to other registers with VALU
// moves that would otherwise read it before the last MFMA has written it.
template <int MT>
__device__ __forceinline__ void mfma_drain(floatx4 (&acc)[MT]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(acc[0]));
#pragma unroll
  for (int mt = 1; mt < MT; ++mt) asm volatile("" : "+v"(acc[mt]));
}

}  // namespace w4k
