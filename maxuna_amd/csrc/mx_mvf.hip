// Gather mat-vec in plain f32 for any row width: the form every shape takes
// that the LDS-ring decode kernels (mx_mv.hip) cannot hold -- rows wider than
// their DMA batch or LDS budget.  It follows the reference's semantics most
// directly (ReferenceExperts, moe.rs:173-180: dequantise, f32 dot): each lane
// dequantises whole 32-weight chunks bit-exactly (mx_deq.h) and accumulates
// chunk * x with f32 FMAs, x read as f32 straight from memory.  Any k that is
// a multiple of the block size works, as in the reference's mat-vec
// (mv.metal:181-290, which loops over any number of super-blocks).
#include "mx_launch.h"
#include "mx_deq.h"

namespace mx {

constexpr int MVF_WAVES = 4, MVF_ROWS = 1;  // rows per wave (each row a chain of dependent loads: 4 -> 1 took a hidden-7168 layer 320 -> 257 us)

template <int DT>
__global__ void __launch_bounds__(64 * MVF_WAVES) k_mv_f32(MvfArgs a) {
    const int pair = blockIdx.y;  // token * top_k + slot
    const int tok = pair / a.top_k, slot = pair % a.top_k;
    int e = 0;
    if (a.ids) {
        const uint32_t id = a.ids[pair];
        e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;  // ids are validated by mx_check_ids
    }
    const float *xrow = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    constexpr int CPB = block_size(DT) / 32, TS = type_size(DT);
    const int nchunk = a.k / 32;
    float *dst = a.dst + ((int64_t)tok * a.dst_stride + slot + a.dst_add) * a.n_out;
    for (int r = 0; r < MVF_ROWS; r++) {
        const int row = (blockIdx.x * MVF_WAVES + wave) * MVF_ROWS + r;
        if (row >= a.n_out) break;
        const uint8_t *rp = a.w + (int64_t)e * a.expert_bytes + (int64_t)row * a.row_bytes;
        float acc = 0.f;
        for (int c = lane; c < nchunk; c += 64) {
            float y[32];
            dequant_chunk<DT>(rp + (int64_t)(c / CPB) * TS, c % CPB, y);
            const float4 *xv = reinterpret_cast<const float4 *>(xrow + 32 * (int64_t)c);
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const float4 v = xv[w];
                acc = __builtin_fmaf(y[4 * w], v.x, acc);
                acc = __builtin_fmaf(y[4 * w + 1], v.y, acc);
                acc = __builtin_fmaf(y[4 * w + 2], v.z, acc);
                acc = __builtin_fmaf(y[4 * w + 3], v.w, acc);
            }
        }
        acc = warp_sum_width(acc, 64);
        if (lane == 0) dst[row] = acc;
    }
}

mx_status launch_mv_f32(int dtype, const MvfArgs &a, hipStream_t s) {
    const int rows_per_block = MVF_WAVES * MVF_ROWS;
    const dim3 grid((unsigned)((a.n_out + rows_per_block - 1) / rows_per_block), (unsigned)(a.t * a.top_k));
    if (grid.x == 0 || grid.y == 0) return MX_OK;
    switch (dtype) {
    case kQ4_K: hipLaunchKernelGGL(k_mv_f32<kQ4_K>, grid, dim3(64 * MVF_WAVES), 0, s, a); break;
    case kQ5_K: hipLaunchKernelGGL(k_mv_f32<kQ5_K>, grid, dim3(64 * MVF_WAVES), 0, s, a); break;
    case kQ6_K: hipLaunchKernelGGL(k_mv_f32<kQ6_K>, grid, dim3(64 * MVF_WAVES), 0, s, a); break;
    default: hipLaunchKernelGGL(k_mv_f32<kQ8_0>, grid, dim3(64 * MVF_WAVES), 0, s, a); break;
    }
    MX_LAUNCH("k_mv_f32");
    return MX_OK;
}

}  // namespace mx
