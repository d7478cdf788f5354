// Shared device/host helpers for the maxuna_moe gfx950 kernels.
//
// Block layouts are the public GGUF/ggml formats (reference: mv.metal:55-80):
//   Q4_K 144 B: f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q5_K 176 B: f16 d | f16 dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]
//   Q6_K 210 B: u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
//   Q8_0  34 B: f16 d | i8 qs[32]
// Q6_K and Q8_0 blocks are only 2-byte aligned inside a row, so every load of
// their bytes here is either a 16-bit load or a 4-byte-aligned dword load that
// contains at least one requested byte (see load8_a2).
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/maxuna_moe.h"

namespace mx {

constexpr int kQ8_0 = MX_Q8_0;
constexpr int kQ4_K = MX_Q4_K;
constexpr int kQ5_K = MX_Q5_K;
constexpr int kQ6_K = MX_Q6_K;
constexpr int QK_K = 256;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// 16 bytes read once and not again by this kernel (streamed intermediates): a
// non-temporal load, which keeps the stream from displacing cached lines
__device__ __forceinline__ float4 ld_stream4(const float *p) {
    const float4_t q = __builtin_nontemporal_load(reinterpret_cast<const float4_t *>(p));
    return make_float4(q[0], q[1], q[2], q[3]);
}

__host__ __device__ constexpr int block_size(int dt) {
    return dt == kQ8_0 ? 32 : (dt == kQ4_K || dt == kQ5_K || dt == kQ6_K) ? 256 : -1;
}
__host__ __device__ constexpr int type_size(int dt) {
    return dt == kQ8_0 ? 34 : dt == kQ4_K ? 144 : dt == kQ5_K ? 176 : dt == kQ6_K ? 210 : -1;
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}

// 8 bytes from a 2-byte-aligned address p, using only 4-byte-aligned dword
// loads, each of which contains at least one of the 8 requested bytes (so it
// never touches a page the requested bytes do not).
__device__ __forceinline__ uint2 load8_a2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
    if ((a & 2) == 0) {
        return make_uint2(q[0], q[1]);
    }
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbit(d1, d0, 16), __builtin_amdgcn_alignbit(d2, d1, 16));
}

// Q4_K 6-bit scale/min of sub-block j (0..7) from the 12 scale bytes, held as
// three little-endian dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11).
// Restates get_scale_min_k4 (mm_id.metal:89-92).
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xFFu;  // scales[j+4]
        sc = (b8 & 0xFu) | (((s0 >> (8 * jj)) >> 6 & 3u) << 4);
        m = (b8 >> 4) | (((s1 >> (8 * jj)) >> 6 & 3u) << 4);
    }
}

// The scales and mins of sub-blocks 2i and 2i + 1 (i in 0..3, may differ per
// lane) without a branch: byte 0 of sc / m is sub-block 2i's 6-bit value, byte 1
// sub-block 2i + 1's -- the same bits as q4k_scale_min(2i) and (2i + 1).
__device__ __forceinline__ void q4k_pair_scale_min(int i, uint32_t s0, uint32_t s1, uint32_t s2,
                                                   uint32_t &sc, uint32_t &m) {
    const uint32_t b = 16u * (uint32_t)(i & 1);  // bit offset of byte (2i) mod 4
    const uint32_t a0 = __builtin_amdgcn_ubfe(s0, b, 16), a1 = __builtin_amdgcn_ubfe(s1, b, 16);
    const uint32_t a2 = __builtin_amdgcn_ubfe(s2, b, 16);
    const bool upper = i >= 2;  // sub-blocks 4..7: low nibbles in scales[8..11], top bits in scales[0..3]
    sc = upper ? (a2 & 0x0F0Fu) | ((a0 >> 2) & 0x3030u) : a0 & 0x3F3Fu;
    m = upper ? ((a2 >> 4) & 0x0F0Fu) | ((a1 >> 2) & 0x3030u) : a1 & 0x3F3Fu;
}

// The value held by this lane's partner for O in {1, 2, 4, 8, 16, 32}, exchanged
// without LDS (DPP / permlane).  The partner differs from the lane in bit log2(O)
// and possibly in lower bits, never in higher ones: lane ^ 1, ^ 2, ^ 7
// (row_half_mirror), ^ 15 (row_mirror), ^ 16, ^ 32.  Butterfly reductions that
// visit O from high to low therefore still combine every lane of the group, and
// partners are mutual, so keep/send halving stays consistent.
template <int O> __device__ __forceinline__ float lane_partner(float v) {
    const int iv = __float_as_int(v);
    if constexpr (O == 1) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
    } else if constexpr (O == 2) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
    } else if constexpr (O == 4) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false));  // row_half_mirror
    } else if constexpr (O == 8) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x140, 0xF, 0xF, false));  // row_mirror
    } else if constexpr (O == 16) {
        // odd rows of [0] and even rows of [1] hold the other row's values
        const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)iv, (uint32_t)iv, false, false);
        return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
    } else {
        static_assert(O == 32, "lane_partner: O must be a power of two <= 32");
        const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)iv, (uint32_t)iv, false, false);
        return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
    }
}

// f(std::integral_constant<int, O>) for O = o, o / 2, ..., 1 (o a wave-uniform power
// of two <= 32, or 0 for none): one dispatch for the whole chain
template <class F> __device__ __forceinline__ void for_offsets_down(int o, F &&f) {
    switch (o) {
    case 32: f(std::integral_constant<int, 32>{}); [[fallthrough]];
    case 16: f(std::integral_constant<int, 16>{}); [[fallthrough]];
    case 8: f(std::integral_constant<int, 8>{}); [[fallthrough]];
    case 4: f(std::integral_constant<int, 4>{}); [[fallthrough]];
    case 2: f(std::integral_constant<int, 2>{}); [[fallthrough]];
    case 1: f(std::integral_constant<int, 1>{}); break;
    default: break;
    }
}
// f(std::integral_constant<int, O>) for the single O = o
template <class F> __device__ __forceinline__ void at_offset(int o, F &&f) {
    switch (o) {
    case 32: f(std::integral_constant<int, 32>{}); break;
    case 16: f(std::integral_constant<int, 16>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    default: f(std::integral_constant<int, 1>{}); break;
    }
}

// A lambda that must be inlined: one not inlined gets the arrays it captures by
// reference (accumulators, register tables) passed by address, which moves them
// to scratch memory
#define MX_INLINE_LAMBDA __attribute__((always_inline))

// f(std::integral_constant<int, i>) for i = I .. N - 1: a loop whose index is a
// compile-time constant in every iteration, whatever the unroller decides (an
// array indexed by a loop variable that stays a variable is moved to scratch)
template <int I, int N, class F> __device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

__device__ __forceinline__ float warp_sum_width(float v, int width) {
    for_offsets_down(width >> 1, [&](auto c) { v += lane_partner<decltype(c)::value>(v); });
    return v;
}

}  // namespace mx

// ---- host-side status plumbing (shared by every translation unit) ---------------
namespace mx {
mx_status fail(mx_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
mx_status hip_check(hipError_t e, const char *what);
}  // namespace mx

#define MX_TRY(expr)                          \
    do {                                      \
        mx_status _s = (expr);                \
        if (_s != MX_OK) return _s;           \
    } while (0)

#define MX_HIP(expr) MX_TRY(::mx::hip_check((expr), #expr))
#define MX_LAUNCH(name) MX_TRY(::mx::hip_check(hipGetLastError(), name))
