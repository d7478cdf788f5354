// One f32 row -> f16 times a power of two (the grouped GEMM's A operand form):
// the row's maximum magnitude lands in [2^14, 2^15), so any f32 magnitude keeps
// f16's full precision; scale = 2^ex with x = y * scale.  Shared by the
// conversion kernel (mx_gemm.hip) and the fused router's x rows (mx_route.hip).
#pragma once

#include "mx_common.h"

namespace mx {

// A 256-thread block converts one row of k values (k % 4 == 0).  RPT > 0:
// k <= 1024 * RPT, the row's float4s stay in registers between the max pass and
// the conversion (all loads issued up front); RPT == 0: any k, the row is read
// twice.  s_red: 4 floats of LDS.  Every thread of the block must call it.
// PERM: each group of four values is stored in the order 0, 2, 1, 3 (the K order
// in which the Q4_K verify tiles build their weight operand).
template <int RPT, bool PERM = false>
__device__ __forceinline__ void f16_row(const float *__restrict__ x, int k, _Float16 *__restrict__ y,
                                        float *__restrict__ scale, float *s_red) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const float4 *xr = reinterpret_cast<const float4 *>(x);
    const int n4 = k / 4;
    auto amax4 = [](const float4 &v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
    float mx = 0.f;
    float4 cache[RPT > 0 ? RPT : 1];
    if constexpr (RPT > 0) {
#pragma unroll
        for (int j = 0; j < RPT; j++) {
            const int i = threadIdx.x + 256 * j;
            cache[j] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < RPT; j++) mx = fmaxf(mx, amax4(cache[j]));
    } else {
        for (int i = threadIdx.x; i < n4; i += 256) mx = fmaxf(mx, amax4(xr[i]));
    }
    mx = fmaxf(mx, lane_partner<32>(mx));
    mx = fmaxf(mx, lane_partner<16>(mx));
    mx = fmaxf(mx, lane_partner<8>(mx));
    mx = fmaxf(mx, lane_partner<4>(mx));
    mx = fmaxf(mx, lane_partner<2>(mx));
    mx = fmaxf(mx, lane_partner<1>(mx));
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    // exponent so that max * 2^-ex lies in [2^14, 2^15)
    const int ex = mx > 0.f ? ilogbf(mx) - 14 : 0;
    const float inv = ldexpf(1.0f, -ex);
    half4_t *yr = reinterpret_cast<half4_t *>(y);
    auto put = [&](int i, const float4 &v) {
        const half2_t lo = __builtin_convertvector((f2_t){v.x * inv, v.y * inv}, half2_t);
        const half2_t hi = __builtin_convertvector((f2_t){v.z * inv, v.w * inv}, half2_t);
        yr[i] = PERM ? (half4_t){lo[0], hi[0], lo[1], hi[1]} : (half4_t){lo[0], lo[1], hi[0], hi[1]};
    };
    if constexpr (RPT > 0) {
#pragma unroll
        for (int j = 0; j < RPT; j++) {
            const int i = threadIdx.x + 256 * j;
            if (i < n4) put(i, cache[j]);
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += 256) put(i, xr[i]);
    }
    if (threadIdx.x == 0) *scale = ldexpf(1.0f, ex);
}

}  // namespace mx
