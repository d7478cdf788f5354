// Global -> LDS DMA (global_load_lds_dwordx4) and explicit vmcnt waits, shared
// by the decode and prefill kernels.
#pragma once

#include "mx_common.h"

namespace mx {

#define MX_AS_LDS __attribute__((address_space(3)))
#define MX_AS_GLB __attribute__((address_space(1)))

// one 16-byte global -> LDS copy per lane; `lds_dst` must be wave-uniform (the
// hardware writes lane i's 16 bytes at lds_dst + 16 * i)
template <int AUX = 0>
__device__ __forceinline__ void dma16(const uint8_t *src, uint8_t *lds_dst) {
    __builtin_amdgcn_global_load_lds((MX_AS_GLB void *)src, (MX_AS_LDS void *)lds_dst, 16, 0, AUX);
}
// Cache policy of copies whose bytes nothing reads again soon: non-temporal (the
// gfx950 NT bit of the instruction's cache-policy operand).  The t = 1 decode
// weight streams use it (C1 layer 41.9 -> 39.5 us); verify blocks must not:
// their repeated experts are served from L2 (C2 335 -> 353 us with it).
#ifndef MX_DMA_NT
#define MX_DMA_NT 2
#endif
constexpr int DMA_NT = MX_DMA_NT;

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..63 (expcnt / lgkmcnt not waited)
#define MX_VMW(n) \
    case n: __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14)); break;
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
        MX_VMW(0) MX_VMW(1) MX_VMW(2) MX_VMW(3) MX_VMW(4) MX_VMW(5) MX_VMW(6) MX_VMW(7)
        MX_VMW(8) MX_VMW(9) MX_VMW(10) MX_VMW(11) MX_VMW(12) MX_VMW(13) MX_VMW(14) MX_VMW(15)
        MX_VMW(16) MX_VMW(17) MX_VMW(18) MX_VMW(19) MX_VMW(20) MX_VMW(21) MX_VMW(22) MX_VMW(23)
        MX_VMW(24) MX_VMW(25) MX_VMW(26) MX_VMW(27) MX_VMW(28) MX_VMW(29) MX_VMW(30) MX_VMW(31)
        MX_VMW(32) MX_VMW(33) MX_VMW(34) MX_VMW(35) MX_VMW(36) MX_VMW(37) MX_VMW(38) MX_VMW(39)
        MX_VMW(40) MX_VMW(41) MX_VMW(42) MX_VMW(43) MX_VMW(44) MX_VMW(45) MX_VMW(46) MX_VMW(47)
        MX_VMW(48) MX_VMW(49) MX_VMW(50) MX_VMW(51) MX_VMW(52) MX_VMW(53) MX_VMW(54) MX_VMW(55)
        MX_VMW(56) MX_VMW(57) MX_VMW(58) MX_VMW(59) MX_VMW(60) MX_VMW(61) MX_VMW(62) MX_VMW(63)
        default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
    asm volatile("" ::: "memory");
}
#undef MX_VMW

// s_waitcnt lgkmcnt(0): every LDS read this wave issued has returned (before an
// LDS DMA may overwrite what they read)
__device__ __forceinline__ void wait_lgkmcnt0() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
}

}  // namespace mx
