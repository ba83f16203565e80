// Direct-to-LDS load helpers shared by the GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsmx_common.h"

namespace lsmx {

LSMX_DEV uint32_t lds_u32(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Direct-to-LDS loads through a buffer descriptor: lane l's bytes land at
// m0 + l*size, and a lane whose offset lies at or past the descriptor's byte
// count reads zeros (raw buffer, stride 0), so rows past the operand need no
// clamping and a load costs no 64-bit address arithmetic.  The descriptor is
// built in SGPRs from a wave-uniform base and size; dword 3 selects the
// 32-bit data format that untyped buffer loads require.
typedef int v4i_rsrc __attribute__((ext_vector_type(4)));
LSMX_DEV v4i_rsrc buf_rsrc(const void *base, uint64_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
    return v4i_rsrc{(int)__builtin_amdgcn_readfirstlane((uint32_t)p),
                    (int)(__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32)) & 0xFFFF),
                    (int)__builtin_amdgcn_readfirstlane(n), 0x00020000};
}
LSMX_DEV void dma_x4(uint32_t off, v4i_rsrc r, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(off), "s"(r),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory");
}
// dma_x4 of the lane offset off0 + i * step, formed inside the asm (i a
// compile-time constant after unrolling, step < 2^24 wave-uniform): the
// compiler cannot hoist one offset register per i out of the loop.
LSMX_DEV void dma_x4_at(uint32_t off0, int i, uint32_t step, v4i_rsrc r, uint32_t m0) {
    uint32_t off;
    asm volatile("v_mad_u32_u24 %0, %1, %2, %3\n\ts_mov_b32 m0, %5\n\tbuffer_load_dwordx4 %0, %4, 0 offen lds"
                 : "=&v"(off)
                 : "i"(i), "s"(step), "v"(off0), "s"(r), "s"(__builtin_amdgcn_readfirstlane(m0))
                 : "memory");
}
LSMX_DEV void dma_x1(uint32_t off, v4i_rsrc r, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(off), "s"(r),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory");
}

}  // namespace lsmx
