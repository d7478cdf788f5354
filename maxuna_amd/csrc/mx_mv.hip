// Decode-time gather mat-vec over raw GGUF blocks (the mul_mv_id hot path) and
// the fused decode MoE kernels built from it.
//
// Work layout (gfx950, wave64).  A row of k weights is cut into "groups":
//   Q4_K  group = one 64-weight super-block pair (sub-blocks 2i, 2i+1)   (4 per block)
//   Q6_K  group = 32 weights: half n, 8-wide l-slice j of all 4 parts      (8 per block)
//   Q8_0  group = one 34-byte block of 32 weights                          (1 per block)
// P lanes share a row; lane `sub` owns groups sub, sub+P, ... (NG of them, the
// last possibly masked), so the activation slice a lane needs is the same for
// every row.  It is quantised once per wave to int16 with an exact per-group
// power-of-two scale (|x| * 2^-e < 2^14: 15 significant bits, ~2^-15 relative
// to the group maximum) and kept in registers while the wave streams its rows.
// Weight bytes are read straight from the GGUF layout, NB row-iterations per
// batch so that several rows' loads are in flight per wave.
//
// Inner product: quants are unpacked into int16 pairs with shifts and masks and
// multiplied with the int16 activations by v_dot2_i32_i16 -- exact int32
// accumulation per sub-block (bounds: 32 * 255 * 16384 < 2^31).  The super-block
// scales (d*sc, dmin*m) are applied per sub-block in f32.
//
// Reference kernels replaced: kernel_mul_mv_id_*_f32_v (mv.metal:680-731, dispatch
// geometry dispatch.rs:409-462), silu_mul.metal:57-72, combine.metal:70-97.
#include "mx_launch.h"

namespace mx {

typedef short short2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}

// 16-byte load of streamed weight bytes, marked non-temporal (read once per pass)
__device__ __forceinline__ uint4 ld_stream16(const uint8_t *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Activation quantiser for one group: xi = round(x * 2^-e) with e chosen so that
// max|x| * 2^-e lies in [2^13, 2^14).  Rounding is the f32 add of 1.5 * 2^23
// (round-to-nearest-even); the low 16 bits of the sum's bit pattern are the
// int16 two's-complement value.
struct XQ {
    float inv, scale;
    __device__ __forceinline__ explicit XQ(float mx) {
        const int e = mx > 0.f ? ilogbf(mx) - 13 : 0;
        inv = ldexpf(1.f, -e);
        scale = ldexpf(1.f, e);
    }
    __device__ __forceinline__ uint32_t pack(float a, float b) const {
        const float ra = a * inv + 12582912.0f, rb = b * inv + 12582912.0f;
        return __builtin_amdgcn_perm(__float_as_uint(rb), __float_as_uint(ra), 0x05040100u);
    }
};
constexpr uint32_t ONES = 0x00010001u;  // sdot2 with (1, 1): sum of an int16 pair

template <int DT> struct Q;

// ---- Q4_K -------------------------------------------------------------------------
template <> struct Q<kQ4_K> {
    static constexpr int GPB = 4;
    struct X {
        uint32_t lo[16], hi[16];  // qs dword w: [2w] = (x[4w], x[4w+2]), [2w+1] = (x[4w+1], x[4w+3])
        int slo, shi;
        float scale;
    };
    struct Raw { uint4 h, qa, qb; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        float v[64];
        const float4 *p = reinterpret_cast<const float4 *>(xrow + 64 * g);
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 f = p[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
        }
        const XQ qz(mx);
        x.scale = qz.scale;
        int slo = 0, shi = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            x.lo[2 * w] = qz.pack(v[4 * w], v[4 * w + 2]);
            x.lo[2 * w + 1] = qz.pack(v[4 * w + 1], v[4 * w + 3]);
            x.hi[2 * w] = qz.pack(v[32 + 4 * w], v[32 + 4 * w + 2]);
            x.hi[2 * w + 1] = qz.pack(v[32 + 4 * w + 1], v[32 + 4 * w + 3]);
            slo = sdot2(x.lo[2 * w], ONES, sdot2(x.lo[2 * w + 1], ONES, slo));
            shi = sdot2(x.hi[2 * w], ONES, sdot2(x.hi[2 * w + 1], ONES, shi));
        }
        x.slo = slo; x.shi = shi;
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const uint8_t *blk = row + (g >> 2) * 144;
        const int i = g & 3;
        Raw r;
        r.h = ld_stream16(blk);
        r.qa = ld_stream16(blk + 16 + 32 * i);
        r.qb = ld_stream16(blk + 32 + 32 * i);
        return r;
    }
    __device__ static float dot(const Raw &r, int g, const X &x) {
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        int alo = 0, ahi = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t v = q[w];
            alo = sdot2(v & 0x000F000Fu, x.lo[2 * w], alo);
            alo = sdot2((v >> 8) & 0x000F000Fu, x.lo[2 * w + 1], alo);
            ahi = sdot2((v >> 4) & 0x000F000Fu, x.hi[2 * w], ahi);
            ahi = sdot2((v >> 12) & 0x000F000Fu, x.hi[2 * w + 1], ahi);
        }
        uint32_t sc0, m0, sc1, m1;
        const int i = g & 3;
        q4k_scale_min(2 * i, r.h.y, r.h.z, r.h.w, sc0, m0);
        q4k_scale_min(2 * i + 1, r.h.y, r.h.z, r.h.w, sc1, m1);
        const float d = h2f((uint16_t)(r.h.x & 0xFFFFu));
        const float dmin = h2f((uint16_t)(r.h.x >> 16));
        const float a = __builtin_fmaf((float)sc0, (float)alo, (float)sc1 * (float)ahi);
        const float b = __builtin_fmaf((float)m0, (float)x.slo, (float)m1 * (float)x.shi);
        return __builtin_fmaf(d, a, -dmin * b) * x.scale;
    }
};

// ---- Q6_K -------------------------------------------------------------------------
template <> struct Q<kQ6_K> {
    static constexpr int GPB = 8;
    struct X {
        uint32_t v[16];  // part p, dword w: [4p+2w] = (l0, l2), [4p+2w+1] = (l1, l3)
        int s[4];
        float scale;
    };
    struct Raw { uint2 a, b, h, s; uint32_t d; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const float *base = xrow + b * 256 + 128 * n + 8 * j;
        float v[32];
        float mx = 0.f;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float4 f0 = *reinterpret_cast<const float4 *>(base + 32 * p);
            const float4 f1 = *reinterpret_cast<const float4 *>(base + 32 * p + 4);
            v[8 * p + 0] = f0.x; v[8 * p + 1] = f0.y; v[8 * p + 2] = f0.z; v[8 * p + 3] = f0.w;
            v[8 * p + 4] = f1.x; v[8 * p + 5] = f1.y; v[8 * p + 6] = f1.z; v[8 * p + 7] = f1.w;
        }
#pragma unroll
        for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(v[i]));
        const XQ qz(mx);
        x.scale = qz.scale;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            int s = 0;
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const float *q = v + 8 * p + 4 * w;
                x.v[4 * p + 2 * w] = qz.pack(q[0], q[2]);
                x.v[4 * p + 2 * w + 1] = qz.pack(q[1], q[3]);
                s = sdot2(x.v[4 * p + 2 * w], ONES, sdot2(x.v[4 * p + 2 * w + 1], ONES, s));
            }
            x.s[p] = s;
        }
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint8_t *blk = row + b * 210;
        Raw r;
        r.a = load8_a2(blk + 64 * n + 8 * j);         // ql[l]     : q1 low nibble, q3 high
        r.b = load8_a2(blk + 64 * n + 32 + 8 * j);    // ql[l+32]  : q2 low nibble, q4 high
        r.h = load8_a2(blk + 128 + 32 * n + 8 * j);   // qh[l]     : 2 bits of each of q1..q4
        r.s = load8_a2(blk + 192 + 8 * n);            // scales[8n .. 8n+7]
        r.d = ld_u16(blk + 208);
        return r;
    }
    __device__ static float dot(const Raw &r, int g, const X &x) {
        const int is = ((g & 7) & 3) >> 1;
        int acc[4] = {0, 0, 0, 0};
        const uint32_t A[2] = {r.a.x, r.a.y}, B[2] = {r.b.x, r.b.y}, H[2] = {r.h.x, r.h.y};
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t qp[4] = {
                (A[w] & 0x0F0F0F0Fu) | ((H[w] << 4) & 0x30303030u),
                (B[w] & 0x0F0F0F0Fu) | ((H[w] << 2) & 0x30303030u),
                ((A[w] >> 4) & 0x0F0F0F0Fu) | (H[w] & 0x30303030u),
                ((B[w] >> 4) & 0x0F0F0F0Fu) | ((H[w] >> 2) & 0x30303030u)};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                acc[p] = sdot2(qp[p] & 0x003F003Fu, x.v[4 * p + 2 * w], acc[p]);
                acc[p] = sdot2((qp[p] >> 8) & 0x003F003Fu, x.v[4 * p + 2 * w + 1], acc[p]);
            }
        }
        float tot = 0.f;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int byte = is + 2 * p;  // scales[8n + is + 2p]
            const uint32_t src = byte < 4 ? r.s.x : r.s.y;
            const float sc = (float)(int8_t)((src >> (8 * (byte & 3))) & 0xFFu);
            tot = __builtin_fmaf(sc, (float)(acc[p] - 32 * x.s[p]), tot);  // sum (q - 32) x, exact in int32
        }
        return h2f((uint16_t)r.d) * tot * x.scale;
    }
};

// ---- Q8_0 -------------------------------------------------------------------------
template <> struct Q<kQ8_0> {
    static constexpr int GPB = 1;
    struct X { uint32_t v[16]; int s; float scale; };
    struct Raw { uint2 q[4]; uint32_t d; };
    __device__ static void load_x(const float *__restrict__ xrow, int g, X &x) {
        float v[32];
        const float4 *p = reinterpret_cast<const float4 *>(xrow + 32 * g);
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = p[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
        }
        const XQ qz(mx);
        x.scale = qz.scale;
        int s = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            x.v[2 * w] = qz.pack(v[4 * w], v[4 * w + 2]);
            x.v[2 * w + 1] = qz.pack(v[4 * w + 1], v[4 * w + 3]);
            s = sdot2(x.v[2 * w], ONES, sdot2(x.v[2 * w + 1], ONES, s));
        }
        x.s = s;
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const uint8_t *blk = row + g * 34;
        Raw r;
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = load8_a2(blk + 2 + 8 * i);
        r.d = ld_u16(blk);
        return r;
    }
    __device__ static float dot(const Raw &r, int, const X &x) {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t u = (h ? r.q[i].y : r.q[i].x) ^ 0x80808080u;  // q + 128, unsigned
                const int w = 2 * i + h;
                acc = sdot2(u & 0x00FF00FFu, x.v[2 * w], acc);
                acc = sdot2((u >> 8) & 0x00FF00FFu, x.v[2 * w + 1], acc);
            }
        }
        return h2f((uint16_t)r.d) * (float)(acc - 128 * x.s) * x.scale;  // sum (u - 128) x
    }
};

// ---- lane geometry ----------------------------------------------------------------------
// P = largest power of two <= 64 dividing the row's group count G; if that leaves
// more than NG_MAX groups per lane, P = 64 with the tail groups masked.
constexpr int NG_MAX = 8;

template <int DT> struct Geo {
    int G, P, NG, RPI;
    __host__ __device__ explicit Geo(int k) {
        G = (k / block_size(DT)) * Q<DT>::GPB;
        int p = G & (-G);
        if (p > 64) p = 64;
        if (G / p > NG_MAX) p = 64;
        P = p;
        NG = (G + p - 1) / p;
        RPI = 64 / p;
    }
};

// the compiled groups-per-lane variants: the smallest >= NG
__host__ __device__ constexpr int ng_variant(int ng) {
    return ng <= 1 ? 1 : ng <= 2 ? 2 : ng <= 3 ? 3 : ng <= 4 ? 4 : ng <= 6 ? 6 : 8;
}

// Reduces NB tuples of NM floats over the P lanes of each row group.  While the
// tuple count allows, each xor step halves the tuples a lane keeps (the lane
// whose offset bit is set keeps the upper half), so NB tuples cost
// NB - 1 + log2(P / NB) shuffles per float instead of NB * log2(P).  On return
// v[0] holds the full sums of tuple `*which` on the lanes that must publish it
// (`*leader`).  Requires P >= NB; otherwise every tuple is reduced in place and
// published by the lane with sub == 0.
template <int NM, int NB>
__device__ __forceinline__ void reduce_tuples(float (&v)[NB][NM], int P, int sub, int &which, bool &leader) {
    which = 0;
    if (P < NB) {
#pragma unroll
        for (int ib = 0; ib < NB; ib++)
#pragma unroll
            for (int m = 0; m < NM; m++) v[ib][m] = warp_sum_width(v[ib][m], P);
        leader = sub == 0;
        return;
    }
    int o = P >> 1;
#pragma unroll
    for (int half = NB / 2; half >= 1; half /= 2) {
        const bool up = (sub & o) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const float keep = up ? v[half + i][m] : v[i][m];
                const float send = up ? v[i][m] : v[half + i][m];
                v[i][m] = keep + __shfl_xor(send, o, 64);
            }
        }
        if (up) which += half;
        o >>= 1;
    }
    for (; o >= 1; o >>= 1) {
#pragma unroll
        for (int m = 0; m < NM; m++) v[0][m] += __shfl_xor(v[0][m], o, 64);
    }
    leader = (sub & (P / NB - 1)) == 0;
}

// Streams the rows [r_begin, r_end) of NM matrices that share one activation
// through this wave, NB row-iterations (NB * RPI rows) per batch.  The first
// batch's weight loads are issued before `xload` fills `xs` (so the activation
// load and quantisation overlap them), and each batch's loads are issued before
// the previous batch is reduced and published.  sink(row, sums[NM]) runs once
// per row with the fully reduced sums.
template <int DT, int NG, int NB, int NM, class XLoad, class Sink>
__device__ __forceinline__ void stream_rows(const uint8_t *const (&w)[NM], int64_t row_bytes, const Geo<DT> &geo,
                                            typename Q<DT>::X (&xs)[NG], int r_begin, int r_end, XLoad &&xload,
                                            Sink &&sink) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & (geo.P - 1);
    const int rsub = lane / geo.P;
    const int step = NB * geo.RPI;
    typename Q<DT>::Raw raw[NM][NB][NG];
    auto issue = [&](int r0) {
#pragma unroll
        for (int ib = 0; ib < NB; ib++) {
            const int row = r0 + rsub + geo.RPI * ib;
            if (row < r_end) {
                const int64_t off = (int64_t)row * row_bytes;
#pragma unroll
                for (int jg = 0; jg < NG; jg++) {
                    const int g = sub + geo.P * jg;
#pragma unroll
                    for (int m = 0; m < NM; m++) raw[m][ib][jg] = Q<DT>::load(w[m] + off, g < geo.G ? g : 0);
                }
            }
        }
    };
    int r0 = r_begin;
    issue(r0);
    xload();
    while (true) {
        float acc[NB][NM];
#pragma unroll
        for (int ib = 0; ib < NB; ib++) {
            const bool ok = r0 + rsub + geo.RPI * ib < r_end;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                float a = 0.f;
                if (ok) {
#pragma unroll
                    for (int jg = 0; jg < NG; jg++) {
                        const int g = sub + geo.P * jg;
                        if (NG == 1 || g < geo.G) a += Q<DT>::dot(raw[m][ib][jg], g, xs[jg]);
                    }
                }
                acc[ib][m] = a;
            }
        }
        const int r_next = r0 + step;
        const bool more = r_next < r_end;
        if (more) issue(r_next);
        int which;
        bool leader;
        reduce_tuples<NM, NB>(acc, geo.P, sub, which, leader);
        if (leader) {
            if (geo.P < NB) {
#pragma unroll
                for (int ib = 0; ib < NB; ib++) {
                    const int row = r0 + rsub + geo.RPI * ib;
                    if (row < r_end) sink(row, acc[ib]);
                }
            } else {
                const int row = r0 + rsub + geo.RPI * which;
                if (row < r_end) sink(row, acc[0]);
            }
        }
        if (!more) break;
        r0 = r_next;
    }
}

template <int DT, int NG>
__device__ __forceinline__ void load_xs(const float *__restrict__ xrow, const Geo<DT> &geo,
                                        typename Q<DT>::X (&xs)[NG]) {
    const int sub = (threadIdx.x & 63) & (geo.P - 1);
#pragma unroll
    for (int jg = 0; jg < NG; jg++) {
        const int g = sub + geo.P * jg;
        Q<DT>::load_x(xrow, g < geo.G ? g : 0, xs[jg]);
    }
}

constexpr int WAVES = 4;
// rows per wave: generic mat-vec, fused gate/up (activation reused by 2 matrices),
// fused down (every projection of a down tile shares one row tiling)
constexpr int RW_MV = 16, RW_GU = 4, RW_DN = 16;

// NB (row-iterations per batch): keep ~4-8 row-loads per matrix in flight
template <int NG, int NM> struct Batch { static constexpr int NB = NG == 1 ? 4 : (NG <= 4 ? 2 : 1); };

// ---- mul_mv_id -----------------------------------------------------------------------
template <int DT, int NG>
__global__ void __launch_bounds__(64 * WAVES) k_mul_mv_id(MvArgs a) {
    const int pair = blockIdx.y;  // token * top_k + slot
    const int tok = pair / a.top_k, slot = pair % a.top_k;
    int e = 0;
    if (a.ids) {
        const uint32_t id = a.ids[pair];
        e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
    }
    const float *xrow = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
    const uint8_t *const w[1] = {a.w + (int64_t)e * a.expert_bytes};
    const int r0 = blockIdx.x * (WAVES * RW_MV) + (threadIdx.x >> 6) * RW_MV;
    if (r0 >= a.n_out) return;  // wave-uniform; no block barrier in this kernel
    const Geo<DT> geo(a.k);
    typename Q<DT>::X xs[NG];
    float *dst = a.dst + (int64_t)pair * a.n_out;
    stream_rows<DT, NG, Batch<NG, 1>::NB, 1>(
        w, a.row_bytes, geo, xs, r0, min(r0 + RW_MV, a.n_out), [&] { load_xs<DT, NG>(xrow, geo, xs); },
        [&](int row, const float (&s)[1]) { dst[row] = s[0]; });
}

#define MX_NG_SWITCH(ng, MACRO) \
    switch (ng) {               \
    case 1: MACRO(1); break;    \
    case 2: MACRO(2); break;    \
    case 3: MACRO(3); break;    \
    case 4: MACRO(4); break;    \
    case 6: MACRO(6); break;    \
    default: MACRO(8); break;   \
    }

template <int DT>
static void launch_mv_dt(const MvArgs &a, dim3 grid, hipStream_t s) {
    const int ng = ng_variant(Geo<DT>(a.k).NG);
#define MX_L(N) hipLaunchKernelGGL((k_mul_mv_id<DT, N>), grid, dim3(64 * WAVES), 0, s, a)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
}

mx_status launch_mul_mv_id(int dtype, const MvArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.n_out + WAVES * RW_MV - 1) / (WAVES * RW_MV)), (unsigned)(a.t * a.top_k));
    if (grid.y == 0 || grid.x == 0) return MX_OK;
    switch (dtype) {
    case kQ4_K: launch_mv_dt<kQ4_K>(a, grid, s); break;
    case kQ6_K: launch_mv_dt<kQ6_K>(a, grid, s); break;
    default: launch_mv_dt<kQ8_0>(a, grid, s); break;
    }
    MX_LAUNCH("k_mul_mv_id");
    return MX_OK;
}

// ---- fused decode: gate/up + SwiGLU ---------------------------------------------------
// grid (ff / 64, slots, t); slot top_k (if present) is the shared expert, which
// then has the routed experts' quant type and shape.
// act[tok, slot, r] = silu(gate_r . x) * (up_r . x), silu(g) = g / (1 + exp(-g)),
// the product rounded on its own (silu_mul.metal:57-72).
template <int DT, int NG>
__global__ void __launch_bounds__(64 * WAVES) k_decode_gate_up(DecodeGateUpArgs a) {
    const int slot = blockIdx.y, tok = blockIdx.z;
    const int r0 = blockIdx.x * (WAVES * RW_GU) + (threadIdx.x >> 6) * RW_GU;
    if (r0 >= a.ff) return;
    const int slots = a.top_k + (a.sh_gate ? 1 : 0);
    const uint8_t *gw, *uw;
    int64_t rb;
    if (slot < a.top_k) {
        const uint32_t id = a.ids[tok * a.top_k + slot];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        gw = a.gate + (int64_t)e * a.gu_expert_bytes;
        uw = a.up + (int64_t)e * a.gu_expert_bytes;
        rb = a.gu_row_bytes;
    } else {
        gw = a.sh_gate;
        uw = a.sh_up;
        rb = a.sh_row_bytes;
    }
    const uint8_t *const w[2] = {gw, uw};
    const Geo<DT> geo(a.hidden);
    typename Q<DT>::X xs[NG];
    float *act = a.act + ((int64_t)tok * slots + slot) * a.ff;
    const float *xrow = a.x + (int64_t)tok * a.hidden;
    stream_rows<DT, NG, Batch<NG, 2>::NB, 2>(w, rb, geo, xs, r0, min(r0 + RW_GU, a.ff),
                                             [&] { load_xs<DT, NG>(xrow, geo, xs); },
                                             [&](int row, const float (&s)[2]) {
                                                 const float g = s[0];
                                                 const float sg = g / (1.0f + expf(-g));
                                                 act[row] = sg * s[1];
                                             });
}

template <int DT>
static void launch_gu_dt(const DecodeGateUpArgs &a, dim3 grid, hipStream_t s) {
    const int ng = ng_variant(Geo<DT>(a.hidden).NG);
#define MX_L(N) hipLaunchKernelGGL((k_decode_gate_up<DT, N>), grid, dim3(64 * WAVES), 0, s, a)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
}

mx_status launch_decode_gate_up(int dtype, const DecodeGateUpArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.ff + WAVES * RW_GU - 1) / (WAVES * RW_GU)),
                    (unsigned)(a.top_k + (a.sh_gate ? 1 : 0)), (unsigned)a.t);
    if (grid.x == 0 || a.t == 0) return MX_OK;
    switch (dtype) {
    case kQ4_K: launch_gu_dt<kQ4_K>(a, grid, s); break;
    case kQ6_K: launch_gu_dt<kQ6_K>(a, grid, s); break;
    default: launch_gu_dt<kQ8_0>(a, grid, s); break;
    }
    MX_LAUNCH("k_decode_gate_up");
    return MX_OK;
}

// ---- fused decode: down (one slot per block) + last-block weighted combine ---------------
// grid (hidden / 64, n_slot_blocks, t).  Each block writes its slot's 64 down rows
// to part[tok, slot, :]; the last of the n_slot_blocks blocks of a (tok, row tile)
// to finish (device-scope counter) combines them in slot order:
//   out[c] = residual[c] + ( sum_k w[k] * part[k][c] + part[shared][c] )
// (combine.metal:70-97, moe.rs:73-78, model.rs:351) and resets the counter.  When
// the shared expert has another quant type than the routed experts, the host
// computes it separately and passes it as a.shared_out (a.sh_down == NULL).
template <int DT, int NG>
__global__ void __launch_bounds__(64 * WAVES) k_decode_down(DecodeDownArgs a) {
    __shared__ int s_last;
    const int slot = blockIdx.y, tok = blockIdx.z;
    constexpr int ROWS_PER_WG = WAVES * RW_DN;
    const int tile0 = blockIdx.x * ROWS_PER_WG;
    const int r0 = tile0 + (threadIdx.x >> 6) * RW_DN;
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    if (r0 < a.hidden) {  // wave-uniform; the barrier below is reached by every wave
        const uint8_t *wp;
        int64_t rb;
        if (slot < a.top_k) {
            const uint32_t id = a.ids[tok * a.top_k + slot];
            const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
            wp = a.down + (int64_t)e * a.d_expert_bytes;
            rb = a.d_row_bytes;
        } else {
            wp = a.sh_down;
            rb = a.sh_row_bytes;
        }
        const uint8_t *const w[1] = {wp};
        const Geo<DT> geo(a.ff);
        typename Q<DT>::X xs[NG];
        const float *xrow = a.act + ((int64_t)tok * slots + slot) * a.ff;
        float *part = a.part + ((int64_t)tok * slots + slot) * a.hidden;
        stream_rows<DT, NG, Batch<NG, 1>::NB, 1>(w, rb, geo, xs, r0, min(r0 + RW_DN, a.hidden),
                                                 [&] { load_xs<DT, NG>(xrow, geo, xs); },
                                                 [&](int row, const float (&s)[1]) { st_agent(part + row, s[0]); });
    }
    // publish this block's partial rows (completed agent-coherent stores), then count in
    drain_vmem();
    __syncthreads();
    unsigned *counter = a.counters + (int64_t)tok * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0) s_last = arrive_last(counter, gridDim.y);
    __syncthreads();
    if (!s_last) return;
    const float *wt = a.w + tok * a.top_k;
    for (int r = threadIdx.x; r < ROWS_PER_WG; r += blockDim.x) {
        const int c = tile0 + r;
        if (c >= a.hidden) break;
        const float *pc = a.part + (int64_t)tok * slots * a.hidden + c;
        float v = 0.f;
        for (int s = 0; s < a.top_k; s++) v = v + ld_agent(pc + (int64_t)s * a.hidden) * wt[s];
        const int64_t o = (int64_t)tok * a.hidden + c;
        if (a.sh_down) v = v + ld_agent(pc + (int64_t)a.top_k * a.hidden);
        else if (a.shared_out) v = v + a.shared_out[o];
        if (a.residual) v = a.residual[o] + v;
        a.out[o] = v;
    }
    if (threadIdx.x == 0) reset_counter(counter);
}

template <int DT>
static void launch_dn_dt(const DecodeDownArgs &a, dim3 grid, hipStream_t s) {
    const int ng = ng_variant(Geo<DT>(a.ff).NG);
#define MX_L(N) hipLaunchKernelGGL((k_decode_down<DT, N>), grid, dim3(64 * WAVES), 0, s, a)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
}

size_t decode_down_counter_words(int t, int hidden) {
    return (size_t)t * (size_t)((hidden + WAVES * RW_DN - 1) / (WAVES * RW_DN));
}

mx_status launch_decode_down(int dtype, const DecodeDownArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.hidden + WAVES * RW_DN - 1) / (WAVES * RW_DN)),
                    (unsigned)(a.top_k + (a.sh_down ? 1 : 0)), (unsigned)a.t);
    if (grid.x == 0 || a.t == 0) return MX_OK;
    switch (dtype) {
    case kQ4_K: launch_dn_dt<kQ4_K>(a, grid, s); break;
    case kQ6_K: launch_dn_dt<kQ6_K>(a, grid, s); break;
    default: launch_dn_dt<kQ8_0>(a, grid, s); break;
    }
    MX_LAUNCH("k_decode_down");
    return MX_OK;
}

}  // namespace mx
