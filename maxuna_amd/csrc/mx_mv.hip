// Decode-time gather mat-vec over raw GGUF blocks (the mul_mv_id hot path) and
// the fused decode MoE kernels built from it.
//
// Work layout (gfx950, wave64).  A row of k weights is cut into "groups":
//   Q4_K  group = one 64-weight half of a super-block pair  (4 per block)
//   Q6_K  group = 32 weights: (half n, 8-wide l-slice j)     (8 per block)
//   Q8_0  group = one 34-byte block of 32 weights            (1 per block)
// P lanes (a power of two dividing the group count, <= 64) share a row; each
// lane owns NG = groups/P fixed groups, so the activation slice a lane needs is
// the same for every row: it is loaded into registers once and reused while
// the wave streams RW rows of weights.  Per-row partial sums are reduced across
// the P lanes with xor-shuffles.  All weight bytes are read straight from the
// GGUF layout (reference kernel this replaces: kernel_mul_mv_id_*_f32_v,
// mv.metal:680-731; dispatch geometry dispatch.rs:409-462).
#include "mx_launch.h"

namespace mx {

template <int DT> struct Grp;

// ---- Q4_K -------------------------------------------------------------------------
template <> struct Grp<kQ4_K> {
    static constexpr int GPB = 4;   // groups per block
    static constexpr int NW = 64;   // weights per group
    struct X { float v[64]; float slo, shi; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        const float4 *p = reinterpret_cast<const float4 *>(xrow + 64 * g);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 f = p[i];
            x.v[4 * i] = f.x; x.v[4 * i + 1] = f.y; x.v[4 * i + 2] = f.z; x.v[4 * i + 3] = f.w;
            if (i < 8) slo += (f.x + f.y) + (f.z + f.w);
            else shi += (f.x + f.y) + (f.z + f.w);
        }
        x.slo = slo; x.shi = shi;
    }
    __device__ static float dot(const uint8_t *__restrict__ row, int g, const X &x) {
        const uint8_t *blk = row + (g >> 2) * 144;
        const int i = g & 3;
        const uint4 h = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * i);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * i);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t lo = q[w] & 0x0F0F0F0Fu;
            const uint32_t hi = (q[w] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                slo = __builtin_fmaf((float)((lo >> (8 * bb)) & 0xFFu), x.v[4 * w + bb], slo);
                shi = __builtin_fmaf((float)((hi >> (8 * bb)) & 0xFFu), x.v[32 + 4 * w + bb], shi);
            }
        }
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * i, h.y, h.z, h.w, sc0, m0);
        q4k_scale_min(2 * i + 1, h.y, h.z, h.w, sc1, m1);
        const float d = h2f((uint16_t)(h.x & 0xFFFFu));
        const float dmin = h2f((uint16_t)(h.x >> 16));
        const float a = __builtin_fmaf((float)sc0, slo, (float)sc1 * shi);
        const float b = __builtin_fmaf((float)m0, x.slo, (float)m1 * x.shi);
        return __builtin_fmaf(d, a, -dmin * b);
    }
};

// ---- Q6_K -------------------------------------------------------------------------
template <> struct Grp<kQ6_K> {
    static constexpr int GPB = 8;
    static constexpr int NW = 32;
    struct X { float v[32]; float s[4]; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const float *base = xrow + b * 256 + 128 * n + 8 * j;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float4 f0 = *reinterpret_cast<const float4 *>(base + 32 * p);
            const float4 f1 = *reinterpret_cast<const float4 *>(base + 32 * p + 4);
            x.v[8 * p + 0] = f0.x; x.v[8 * p + 1] = f0.y; x.v[8 * p + 2] = f0.z; x.v[8 * p + 3] = f0.w;
            x.v[8 * p + 4] = f1.x; x.v[8 * p + 5] = f1.y; x.v[8 * p + 6] = f1.z; x.v[8 * p + 7] = f1.w;
            x.s[p] = ((f0.x + f0.y) + (f0.z + f0.w)) + ((f1.x + f1.y) + (f1.z + f1.w));
        }
    }
    __device__ static float dot(const uint8_t *__restrict__ row, int g, const X &x) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint8_t *blk = row + b * 210;
        const uint2 A = load8_a2(blk + 64 * n + 8 * j);        // ql[l]     : q1 lo, q3 hi
        const uint2 B = load8_a2(blk + 64 * n + 32 + 8 * j);   // ql[l+32]  : q2 lo, q4 hi
        const uint2 H = load8_a2(blk + 128 + 32 * n + 8 * j);  // qh[l]
        const int is = j >> 1;
        const uint8_t *scb = blk + 192 + 8 * n;
        float sc[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint16_t pr = ld_u16(scb + 2 * p);          // bytes 2p, 2p+1
            sc[p] = (float)(int8_t)(is ? (pr >> 8) : (pr & 0xFF));
        }
        const float d = h2f(ld_u16(blk + 208));
        const uint32_t a[2] = {A.x, A.y}, bq[2] = {B.x, B.y}, hq[2] = {H.x, H.y};
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t q1 = (a[w] & 0x0F0F0F0Fu) | ((hq[w] << 4) & 0x30303030u);
            const uint32_t q2 = (bq[w] & 0x0F0F0F0Fu) | ((hq[w] << 2) & 0x30303030u);
            const uint32_t q3 = ((a[w] >> 4) & 0x0F0F0F0Fu) | (hq[w] & 0x30303030u);
            const uint32_t q4 = ((bq[w] >> 4) & 0x0F0F0F0Fu) | ((hq[w] >> 2) & 0x30303030u);
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const int ll = 4 * w + bb;
                s[0] = __builtin_fmaf((float)((q1 >> (8 * bb)) & 0xFFu), x.v[ll], s[0]);
                s[1] = __builtin_fmaf((float)((q2 >> (8 * bb)) & 0xFFu), x.v[8 + ll], s[1]);
                s[2] = __builtin_fmaf((float)((q3 >> (8 * bb)) & 0xFFu), x.v[16 + ll], s[2]);
                s[3] = __builtin_fmaf((float)((q4 >> (8 * bb)) & 0xFFu), x.v[24 + ll], s[3]);
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int p = 0; p < 4; p++) acc = __builtin_fmaf(sc[p], __builtin_fmaf(-32.f, x.s[p], s[p]), acc);
        return d * acc;
    }
};

// ---- Q8_0 -------------------------------------------------------------------------
template <> struct Grp<kQ8_0> {
    static constexpr int GPB = 1;
    static constexpr int NW = 32;
    struct X { float v[32]; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        const float4 *p = reinterpret_cast<const float4 *>(xrow + 32 * g);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = p[i];
            x.v[4 * i] = f.x; x.v[4 * i + 1] = f.y; x.v[4 * i + 2] = f.z; x.v[4 * i + 3] = f.w;
        }
    }
    __device__ static float dot(const uint8_t *__restrict__ row, int g, const X &x) {
        const uint8_t *blk = row + g * 34;
        const float d = h2f(ld_u16(blk));
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < 16; m++) {
            const uint16_t pr = ld_u16(blk + 2 + 2 * m);
            s = __builtin_fmaf((float)(int8_t)(pr & 0xFF), x.v[2 * m], s);
            s = __builtin_fmaf((float)(int8_t)(pr >> 8), x.v[2 * m + 1], s);
        }
        return d * s;
    }
};

// Lane geometry for a row of k weights of type DT.
template <int DT> struct RowGeom {
    int P, NG, RPI;  // lanes per row, groups per lane, rows per wave iteration
    __device__ __forceinline__ RowGeom(int k) {
        const int G = (k / block_size(DT)) * Grp<DT>::GPB;
        int p = G & (-G);
        if (p > 64) p = 64;
        P = p; NG = G / p; RPI = 64 / p;
    }
};

// Accumulates acc[r] += W[row_r] . x over this lane's groups for the RW rows a
// wave covers starting at row0 (rows >= n_out are skipped), then reduces each
// acc[r] across its P lanes.  Every lane ends up holding the full row sums.
template <int DT, int RW>
__device__ __forceinline__ void wave_rows(const uint8_t *__restrict__ w, int64_t row_bytes,
                                          int n_out, int k, const float *__restrict__ xrow,
                                          int row0, float (&acc)[RW]) {
    const RowGeom<DT> geo(k);
    const int lane = threadIdx.x & 63;
    const int sub = lane & (geo.P - 1);
    const int rsub = lane / geo.P;
    const int iters = (RW + geo.RPI - 1) / geo.RPI;
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.f;
    for (int jg = 0; jg < geo.NG; jg++) {
        const int g = sub + geo.P * jg;
        typename Grp<DT>::X xs;
        Grp<DT>::load_x(xrow, g, xs);
#pragma unroll
        for (int it = 0; it < RW; it++) {
            if (it < iters) {
                const int row = row0 + rsub + geo.RPI * it;
                if (rsub + geo.RPI * it < RW && row < n_out)
                    acc[it] += Grp<DT>::dot(w + (int64_t)row * row_bytes, g, xs);
            }
        }
    }
#pragma unroll
    for (int it = 0; it < RW; it++) {
        if (it < iters) acc[it] = warp_sum_width(acc[it], geo.P);
    }
}

// Row index a lane reports for iteration `it` (valid when lane is its row's lane 0).
template <int DT>
__device__ __forceinline__ int lane_row(int k, int row0, int it, bool &writer) {
    const RowGeom<DT> geo(k);
    const int lane = threadIdx.x & 63;
    writer = (lane & (geo.P - 1)) == 0;
    return row0 + lane / geo.P + geo.RPI * it;
}

template <int DT>
__device__ __forceinline__ int lane_row_limit(int k, int RW, int it) {
    const RowGeom<DT> geo(k);
    const int lane = threadIdx.x & 63;
    const int iters = (RW + geo.RPI - 1) / geo.RPI;
    return (it < iters && lane / geo.P + geo.RPI * it < RW) ? 1 : 0;
}

// ---- mul_mv_id -----------------------------------------------------------------------
constexpr int MV_WAVES = 4;
constexpr int MV_RW = 8;  // rows per wave

template <int DT>
__global__ void __launch_bounds__(64 * MV_WAVES) k_mul_mv_id(MvArgs a) {
    const int pair = blockIdx.y;  // token * top_k + slot
    const int tok = pair / a.top_k, slot = pair % a.top_k;
    int e = 0;
    if (a.ids) {
        const uint32_t id = a.ids[pair];
        e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
    }
    const float *xrow = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
    const uint8_t *w = a.w + (int64_t)e * a.expert_bytes;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * MV_RW;
    if (row0 >= a.n_out) return;
    float acc[MV_RW];
    wave_rows<DT, MV_RW>(w, a.row_bytes, a.n_out, a.k, xrow, row0, acc);
    float *dst = a.dst + (int64_t)pair * a.n_out;
#pragma unroll
    for (int it = 0; it < MV_RW; it++) {
        bool writer;
        const int row = lane_row<DT>(a.k, row0, it, writer);
        if (writer && lane_row_limit<DT>(a.k, MV_RW, it) && row < a.n_out) dst[row] = acc[it];
    }
}

mx_status launch_mul_mv_id(int dtype, const MvArgs &a, hipStream_t s) {
    const int rows_per_block = MV_WAVES * MV_RW;
    const dim3 grid((unsigned)((a.n_out + rows_per_block - 1) / rows_per_block),
                    (unsigned)(a.t * a.top_k));
    if (grid.y == 0 || grid.x == 0) return MX_OK;
    switch (dtype) {
    case kQ4_K: hipLaunchKernelGGL(k_mul_mv_id<kQ4_K>, grid, dim3(64 * MV_WAVES), 0, s, a); break;
    case kQ6_K: hipLaunchKernelGGL(k_mul_mv_id<kQ6_K>, grid, dim3(64 * MV_WAVES), 0, s, a); break;
    default: hipLaunchKernelGGL(k_mul_mv_id<kQ8_0>, grid, dim3(64 * MV_WAVES), 0, s, a); break;
    }
    MX_LAUNCH("k_mul_mv_id");
    return MX_OK;
}

// ---- fused decode: gate/up + SwiGLU ---------------------------------------------------
// blockIdx.y = pair (t*top_k routed pairs, then t shared-expert pairs).
// act[pair_slot, :] = silu(gate . x) * (up . x), silu(g) = g / (1 + exp(-g)) and
// the product rounded separately (silu_mul.metal:57-72).
constexpr int GU_RW = 8;

template <int DT>
__device__ __forceinline__ void gate_up_rows(const uint8_t *gw, const uint8_t *uw, int64_t row_bytes,
                                             int ff, int hidden, const float *xrow, int row0,
                                             float *act_row) {
    float g[GU_RW], u[GU_RW];
    wave_rows<DT, GU_RW>(gw, row_bytes, ff, hidden, xrow, row0, g);
    wave_rows<DT, GU_RW>(uw, row_bytes, ff, hidden, xrow, row0, u);
#pragma unroll
    for (int it = 0; it < GU_RW; it++) {
        bool writer;
        const int row = lane_row<DT>(hidden, row0, it, writer);
        if (writer && lane_row_limit<DT>(hidden, GU_RW, it) && row < ff) {
            const float sg = g[it] / (1.0f + expf(-g[it]));
            act_row[row] = sg * u[it];
        }
    }
}

template <int DT, int SDT>
__global__ void __launch_bounds__(64 * MV_WAVES) k_decode_gate_up(DecodeGateUpArgs a) {
    const int pair = blockIdx.y;
    const int n_routed = a.t * a.top_k;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * GU_RW;
    if (row0 >= a.ff) return;
    const int slots = a.top_k + (a.sh_gate ? 1 : 0);
    if (pair < n_routed) {
        const int tok = pair / a.top_k, slot = pair % a.top_k;
        const uint32_t id = a.ids[pair];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        const float *xrow = a.x + (int64_t)tok * a.hidden;
        float *act_row = a.act + ((int64_t)tok * slots + slot) * a.ff;
        gate_up_rows<DT>(a.gate + (int64_t)e * a.gu_expert_bytes, a.up + (int64_t)e * a.gu_expert_bytes,
                         a.gu_row_bytes, a.ff, a.hidden, xrow, row0, act_row);
    } else {
        const int tok = pair - n_routed;
        const float *xrow = a.x + (int64_t)tok * a.hidden;
        float *act_row = a.act + ((int64_t)tok * slots + a.top_k) * a.ff;
        gate_up_rows<SDT>(a.sh_gate, a.sh_up, a.sh_row_bytes, a.ff, a.hidden, xrow, row0, act_row);
    }
}

// ---- fused decode: down + weighted combine + shared + residual -------------------------
// Each wave owns RW output rows of the hidden dimension and walks every slot of
// its token, so the combine needs no second pass:
//   out[c] = residual[c] + ( sum_k w[k] * (Wd[id_k][c] . act_k) + (Wsd[c] . act_sh) )
// with the routed sum taken in slot order (combine.metal:70-97) and the shared
// expert added afterwards (moe.rs:73-78), then the residual (model.rs:351).
constexpr int DN_RW = 4;

template <int DT, int SDT>
__global__ void __launch_bounds__(64 * MV_WAVES) k_decode_down(DecodeDownArgs a) {
    __shared__ float s_routed[MV_WAVES][DN_RW];
    __shared__ float s_shared[MV_WAVES][DN_RW];
    const int tok = blockIdx.y;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * DN_RW;
    const bool active = row0 < a.hidden;  // wave-uniform; no early return (barrier below)
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    if (active) {
        float routed[DN_RW];
#pragma unroll
        for (int r = 0; r < DN_RW; r++) routed[r] = 0.f;
        for (int slot = 0; slot < a.top_k; slot++) {
            const uint32_t id = a.ids[tok * a.top_k + slot];
            const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
            const float wt = a.w[tok * a.top_k + slot];
            float acc[DN_RW];
            wave_rows<DT, DN_RW>(a.down + (int64_t)e * a.d_expert_bytes, a.d_row_bytes, a.hidden,
                                 a.ff, a.act + ((int64_t)tok * slots + slot) * a.ff, row0, acc);
#pragma unroll
            for (int r = 0; r < DN_RW; r++) routed[r] = routed[r] + acc[r] * wt;
        }
#pragma unroll
        for (int it = 0; it < DN_RW; it++) {
            bool writer;
            const int row = lane_row<DT>(a.ff, row0, it, writer);
            if (writer && lane_row_limit<DT>(a.ff, DN_RW, it)) s_routed[wave][row - row0] = routed[it];
        }
        if (a.sh_down) {
            float sh[DN_RW];
            wave_rows<SDT, DN_RW>(a.sh_down, a.sh_row_bytes, a.hidden, a.ff,
                                  a.act + ((int64_t)tok * slots + a.top_k) * a.ff, row0, sh);
#pragma unroll
            for (int it = 0; it < DN_RW; it++) {
                bool writer;
                const int row = lane_row<SDT>(a.ff, row0, it, writer);
                if (writer && lane_row_limit<SDT>(a.ff, DN_RW, it)) s_shared[wave][row - row0] = sh[it];
            }
        }
    }
    __syncthreads();
    if (active && lane < DN_RW && row0 + lane < a.hidden) {
        float v = s_routed[wave][lane];
        if (a.sh_down) v = v + s_shared[wave][lane];
        const int64_t o = (int64_t)tok * a.hidden + row0 + lane;
        if (a.residual) v = a.residual[o] + v;
        a.out[o] = v;
    }
}

template <int DT>
static mx_status gate_up_dispatch_sdt(int sdt, const DecodeGateUpArgs &a, dim3 grid, hipStream_t s) {
    switch (sdt) {
    case kQ4_K: hipLaunchKernelGGL((k_decode_gate_up<DT, kQ4_K>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    case kQ6_K: hipLaunchKernelGGL((k_decode_gate_up<DT, kQ6_K>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    default: hipLaunchKernelGGL((k_decode_gate_up<DT, kQ8_0>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    }
    MX_LAUNCH("k_decode_gate_up");
    return MX_OK;
}

mx_status launch_decode_gate_up(int dtype, int sh_dtype, const DecodeGateUpArgs &a, hipStream_t s) {
    const int rows_per_block = MV_WAVES * GU_RW;
    const dim3 grid((unsigned)((a.ff + rows_per_block - 1) / rows_per_block),
                    (unsigned)(a.t * a.top_k + (a.sh_gate ? a.t : 0)));
    if (grid.x == 0 || grid.y == 0) return MX_OK;
    const int sdt = a.sh_gate ? sh_dtype : dtype;
    switch (dtype) {
    case kQ4_K: return gate_up_dispatch_sdt<kQ4_K>(sdt, a, grid, s);
    case kQ6_K: return gate_up_dispatch_sdt<kQ6_K>(sdt, a, grid, s);
    default: return gate_up_dispatch_sdt<kQ8_0>(sdt, a, grid, s);
    }
}

template <int DT>
static mx_status down_dispatch_sdt(int sdt, const DecodeDownArgs &a, dim3 grid, hipStream_t s) {
    switch (sdt) {
    case kQ4_K: hipLaunchKernelGGL((k_decode_down<DT, kQ4_K>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    case kQ6_K: hipLaunchKernelGGL((k_decode_down<DT, kQ6_K>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    default: hipLaunchKernelGGL((k_decode_down<DT, kQ8_0>), grid, dim3(64 * MV_WAVES), 0, s, a); break;
    }
    MX_LAUNCH("k_decode_down");
    return MX_OK;
}

mx_status launch_decode_down(int dtype, int sh_dtype, const DecodeDownArgs &a, hipStream_t s) {
    const int rows_per_block = MV_WAVES * DN_RW;
    const dim3 grid((unsigned)((a.hidden + rows_per_block - 1) / rows_per_block), (unsigned)a.t);
    if (grid.x == 0 || grid.y == 0) return MX_OK;
    const int sdt = a.sh_down ? sh_dtype : dtype;
    switch (dtype) {
    case kQ4_K: return down_dispatch_sdt<kQ4_K>(sdt, a, grid, s);
    case kQ6_K: return down_dispatch_sdt<kQ6_K>(sdt, a, grid, s);
    default: return down_dispatch_sdt<kQ8_0>(sdt, a, grid, s);
    }
}

}  // namespace mx
