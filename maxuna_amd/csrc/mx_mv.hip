// Decode-time gather mat-vec over raw GGUF blocks (the mul_mv_id hot path) and
// the fused decode MoE kernels built from it.
//
// Activations are consumed in the staged integer form of mx_stage.h: per
// 32-value group a power-of-two scale s_g and 24-bit integers
// x24 = 65536 * xh + 256 * xm + xl in three int8 digit planes, plus the sum of
// x24 over every 32 values.  The gate/up kernel
// reads the token rows staged once by the router kernel (global memory); the
// down kernel and the generic mat-vec stage their row into LDS per workgroup
// (activation loads issued before the weight loads).  The weight quants are unpacked to bytes with masks and shifts and contracted with all three
// digit planes on v_dot4_i32_i8, so each plane's sum of q * digit is exact in
// int32; the three plane sums are recombined in f32 (two roundings), and the
// per-sub-block scales (d*sc, dmin*m) and the group scale s_g are applied once
// per sub-block in f32 (the factored form of mv.metal:263-267).  Each activation
// value is carried to within 2^-23 * (1 + 2^-8) of its group's largest
// magnitude -- the 24-bit width of the reference's f32 y (mv.metal:227-275).
//
// Work layout (gfx950, wave64).  A row of k weights is cut into "groups":
//   Q4_K  group = one 64-weight sub-block pair (2i, 2i+1) of a super-block (4 per block)
//   Q5_K  as Q4_K, with the pair's fifth bits from qh
//   Q6_K  group = 32 weights: half n, 8-wide l-slice j of all 4 parts        (8 per block)
//   Q8_0  group = one 34-byte block of 32 weights                            (1 per block)
// P lanes share a row; lane `sub` owns groups sub, sub+P, ... (NG of them, the
// last possibly masked), so the activation slice a lane needs is the same for
// every row and is held in registers.
//
// Weight bytes never pass through the lanes' own load pattern: each wave copies
// the contiguous byte span of its next batch of rows into a private, double-
// buffered LDS ring with global_load_lds_dwordx4 (every wave instruction moves
// 1 KB of consecutive aligned 16-byte chunks -- fully coalesced, no VGPRs), and
// the lanes then read their groups from LDS.  The copy of batch i+1 is in
// flight while batch i is computed; the wave waits on its own copy with an
// explicit vmcnt.  Aligned 16-byte chunks never cross a page, so copying the
// chunks that cover a span never touches an unmapped page.
//
// Reference kernels replaced: kernel_mul_mv_id_*_f32_v (mv.metal:680-731, dispatch
// geometry dispatch.rs:409-462), silu_mul.metal:57-72, combine.metal:70-97.
#include "mx_launch.h"
#include "mx_stage.h"
#include "mx_dma.h"
#include "mx_select.h"

namespace mx {

// product of two values that fit 24-bit signed integers (v_mul_i32_i24)
__device__ __forceinline__ int mul24(int a, int b) { return ((a << 8) >> 8) * ((b << 8) >> 8); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// DMA instructions for a batch of `rows` rows of `row_bytes` of nm matrices:
// each matrix's span gets its own instructions (worst-case alignment: one extra
// chunk per span)
__host__ __device__ inline int dma_insts(int nm, int rows, int64_t row_bytes) {
    const int64_t chunks = (rows * row_bytes + 15) / 16 + 1;  // per matrix
    return nm * (int)((chunks + 63) / 64);
}
constexpr int DMA_MAX_INSTS = 15;  // per batch (vmcnt budget of the waits, up to 2 batches ahead)

__device__ __forceinline__ void lds_words(const int8_t *p, uint32_t *dst, int n16) {
    // n16 16-byte reads from a 16-byte-aligned LDS address
    const uint4 *q = reinterpret_cast<const uint4 *>(p);
    for (int i = 0; i < n16; i++) {
        const uint4 v = q[i];
        dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
}

template <int DT> struct Q;

// sum over the 4 bytes of each of two dwords times c (c = 1: the plain digit sum)
__device__ __forceinline__ int digit_sum2(uint32_t a, uint32_t b, uint32_t c) { return dot4(c, a, dot4(c, b, 0)); }

// 65536 * h + 256 * m + l in f32: the three exact int32 digit-plane sums of a
// dot product recombined with at most two roundings (m * 256 + l is formed in
// int32, exact; its conversion and the final fma each round once).
__device__ __forceinline__ float planes(int h, int m, int l) {
    return __builtin_fmaf((float)h, 65536.0f, (float)(m * 256 + l));
}

// ---- Q4_K -------------------------------------------------------------------------
template <> struct Q<kQ4_K> {
    static constexpr int GPB = 4;
    struct X {
        // [0..8): sub-block 2i positions 0..31, [8..16): sub-block 2i+1; one array per digit plane
        uint32_t h[16], m[16], l[16];
        float sa, sb, ssa, ssb;  // group scales and scale * sum(x24)
    };
    struct Raw { uint4 hd, qa, qb; };
    __device__ static void load_x(const XView &xv, int g, X &x) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            lds_words(xv.xh + 64 * g + 32 * half, x.h + 8 * half, 2);
            lds_words(xv.xm + 64 * g + 32 * half, x.m + 8 * half, 2);
            lds_words(xv.xl + 64 * g + 32 * half, x.l + 8 * half, 2);
        }
        x.sa = xv.s[2 * g];
        x.sb = xv.s[2 * g + 1];
        x.ssa = x.sa * (float)xv.S32[2 * g];
        x.ssb = x.sb * (float)xv.S32[2 * g + 1];
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const uint8_t *blk = row + (g >> 2) * 144;
        const int i = g & 3;
        Raw r;
        r.hd = *reinterpret_cast<const uint4 *>(blk);
        r.qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * i);
        r.qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * i);
        return r;
    }
    // sum_q x over a 64-weight sub-block pair (sub-block 2i: low nibbles, 2i+1: high
    // nibbles), with the pair's per-sub-block scales applied
    __device__ static float pair(const uint32_t (&q)[8], uint32_t hd0, uint32_t s0, uint32_t s1, uint32_t s2, int i,
                                 const X &x, const uint32_t *hb = nullptr) {
        int ah = 0, am = 0, al = 0, bh = 0, bm = 0, bl = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            uint32_t lo = q[w] & 0x0F0F0F0Fu;
            uint32_t hi = (q[w] >> 4) & 0x0F0F0F0Fu;
            if (hb) {  // Q5_K: the fifth bit of each weight
                const uint32_t hs = hb[w] >> (2 * i);
                lo |= (hs & 0x01010101u) << 4;
                hi |= ((hs >> 1) & 0x01010101u) << 4;
            }
            ah = dot4(lo, x.h[w], ah);
            am = dot4(lo, x.m[w], am);
            al = dot4(lo, x.l[w], al);
            bh = dot4(hi, x.h[8 + w], bh);
            bm = dot4(hi, x.m[8 + w], bm);
            bl = dot4(hi, x.l[8 + w], bl);
        }
        const float A = planes(ah, am, al), B = planes(bh, bm, bl);
        uint32_t sc, mn;
        q4k_pair_scale_min(i, s0, s1, s2, sc, mn);
        const float d = h2f((uint16_t)(hd0 & 0xFFFFu));
        const float dmin = h2f((uint16_t)(hd0 >> 16));
        const float sc0 = (float)(sc & 0xFFu), sc1 = (float)(sc >> 8), m0 = (float)(mn & 0xFFu), m1 = (float)(mn >> 8);
        // sa, sb are powers of two: sc * sa is exact
        const float p = __builtin_fmaf(sc0 * x.sa, A, sc1 * x.sb * B);
        const float m = __builtin_fmaf(m0, x.ssa, m1 * x.ssb);
        return __builtin_fmaf(d, p, -dmin * m);
    }
    __device__ static float dot(const Raw &r, int g, const X &x) {
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        return pair(q, r.hd.x, r.hd.y, r.hd.z, r.hd.w, g & 3, x);
    }
};

// ---- Q5_K -------------------------------------------------------------------------
// Q4_K's group layout (one 64-weight sub-block pair per group) plus the fifth
// bit: weight 32h + l of pair i takes bit 2i + h of qh[l] (mm_id.metal:113-134).
template <> struct Q<kQ5_K> {
    static constexpr int GPB = 4;
    using X = Q<kQ4_K>::X;
    struct Raw { uint4 hd, qa, qb, ha, hb; };
    __device__ static void load_x(const XView &xv, int g, X &x) { Q<kQ4_K>::load_x(xv, g, x); }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const uint8_t *blk = row + (g >> 2) * 176;
        const int i = g & 3;
        Raw r;
        r.hd = *reinterpret_cast<const uint4 *>(blk);
        r.ha = *reinterpret_cast<const uint4 *>(blk + 16);
        r.hb = *reinterpret_cast<const uint4 *>(blk + 32);
        r.qa = *reinterpret_cast<const uint4 *>(blk + 48 + 32 * i);
        r.qb = *reinterpret_cast<const uint4 *>(blk + 64 + 32 * i);
        return r;
    }
    __device__ static float dot(const Raw &r, int g, const X &x) {
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        const uint32_t h[8] = {r.ha.x, r.ha.y, r.ha.z, r.ha.w, r.hb.x, r.hb.y, r.hb.z, r.hb.w};
        return Q<kQ4_K>::pair(q, r.hd.x, r.hd.y, r.hd.z, r.hd.w, g & 3, x, h);
    }
};

// ---- Q6_K -------------------------------------------------------------------------
template <> struct Q<kQ6_K> {
    static constexpr int GPB = 8;
    struct X {
        uint32_t h[8], m[8], l[8];  // part p: [2p], [2p+1] = 8 activation values, one array per digit plane
        int nh[4], nml[4];          // -32 * (digit sums of the part's 8 values): h plane; 256 * m + l planes
        float s[4];                 // group scale of the part's positions
    };
    // raw dwords of the 8-byte fields (3 aligned dwords each, funnel-shifted in dot()
    // so that no arithmetic on loaded values sits between the loads and their use)
    struct Raw { uint32_t a[3], b[3], hq[3], sc[3]; uint32_t sh, d; };
    __device__ static void load_x(const XView &xv, int g, X &x) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        constexpr uint32_t M32 = 0xE0E0E0E0u;  // -32 in every byte
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int pos = 256 * b + 128 * n + 32 * p + 8 * j;
            const uint2 vh = *reinterpret_cast<const uint2 *>(xv.xh + pos);
            const uint2 vm = *reinterpret_cast<const uint2 *>(xv.xm + pos);
            const uint2 vl = *reinterpret_cast<const uint2 *>(xv.xl + pos);
            x.h[2 * p] = vh.x; x.h[2 * p + 1] = vh.y;
            x.m[2 * p] = vm.x; x.m[2 * p + 1] = vm.y;
            x.l[2 * p] = vl.x; x.l[2 * p + 1] = vl.y;
            x.nh[p] = digit_sum2(vh.x, vh.y, M32);
            x.nml[p] = 256 * digit_sum2(vm.x, vm.y, M32) + digit_sum2(vl.x, vl.y, M32);
            x.s[p] = xv.s[pos >> 5];
        }
    }
    // 3 dwords at a 4-byte aligned p: the 8 bytes of a field that starts at p or p + 2
    __device__ static void ld3(const uint8_t *p, uint32_t (&d)[3]) {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
        d[0] = q[0]; d[1] = q[1]; d[2] = q[2];
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const int b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint8_t *blk = row + b * 210;
        // Every field sits at a multiple of 8 inside the block, so all of them
        // share the block's offset mod 4 (0 or 2): one aligned base serves all.
        // Pointer arithmetic (not an integer round trip) keeps the LDS address
        // space visible.
        const uint32_t mis = (uint32_t)reinterpret_cast<uintptr_t>(blk) & 2;
        const uint8_t *ab = blk - mis;
        Raw r;
        r.sh = mis << 3;
        ld3(ab + 64 * n + 8 * j, r.a);          // ql[l]    : part 0 low nibble, part 2 high
        ld3(ab + 64 * n + 32 + 8 * j, r.b);     // ql[l+32] : part 1 low nibble, part 3 high
        ld3(ab + 128 + 32 * n + 8 * j, r.hq);   // qh[l]    : 2 bits of each part
        ld3(ab + 192 + 8 * n, r.sc);            // scales[8n .. 8n+7]
        r.d = ld_u16(blk + 208);
        return r;
    }
    // The lane group's four parts (positions 128n + 32p + 8j of a block) lie in
    // one 128-value staging block (Q6_K rows have k % 256 == 0, so they are
    // always staged with one scale per 128 values, mx_stage.h) and share its scale
    // x.s[0].  The accumulators start at -32 * (digit sums), so each part's plane
    // sums are sum (q - 32) * digit, exact; the parts' sums are weighted by their
    // int8 scales in integer arithmetic (|sc * sum| <= 128 * 32768 per part, at
    // most 2^24 over the four: exact in f32), and the three planes are
    // recombined in f32 (two roundings) and scaled once per group.
    __device__ static float dot(const Raw &r, int g, const X &x) {
        const int jh = ((g & 7) & 3) >> 1;  // scale byte is scales[8n + jh + 2p]
        int hacc[4] = {x.nh[0], x.nh[1], x.nh[2], x.nh[3]}, macc[4] = {0, 0, 0, 0},
            lacc[4] = {x.nml[0], x.nml[1], x.nml[2], x.nml[3]};
        auto fun = [&](const uint32_t (&d)[3], int w) { return __builtin_amdgcn_alignbit(d[w + 1], d[w], r.sh); };
        const uint32_t A[2] = {fun(r.a, 0), fun(r.a, 1)}, B[2] = {fun(r.b, 0), fun(r.b, 1)},
                       H[2] = {fun(r.hq, 0), fun(r.hq, 1)};
        const uint32_t SC[2] = {fun(r.sc, 0), fun(r.sc, 1)};
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t qp[4] = {
                (A[w] & 0x0F0F0F0Fu) | ((H[w] << 4) & 0x30303030u),
                (B[w] & 0x0F0F0F0Fu) | ((H[w] << 2) & 0x30303030u),
                ((A[w] >> 4) & 0x0F0F0F0Fu) | (H[w] & 0x30303030u),
                ((B[w] >> 4) & 0x0F0F0F0Fu) | ((H[w] >> 2) & 0x30303030u)};
#pragma unroll
            for (int p = 0; p < 4; p++) {
                hacc[p] = dot4(qp[p], x.h[2 * p + w], hacc[p]);
                macc[p] = dot4(qp[p], x.m[2 * p + w], macc[p]);
                lacc[p] = dot4(qp[p], x.l[2 * p + w], lacc[p]);
            }
        }
        int Hs = 0, Ms = 0, Ls = 0;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int sc = __builtin_amdgcn_sbfe((int)SC[p >> 1], 8 * (jh + 2 * (p & 1)), 8);
            Hs += mul24(sc, hacc[p]);
            Ms += mul24(sc, macc[p]);
            Ls += mul24(sc, lacc[p]);
        }
        const float v = __builtin_fmaf((float)Hs, 65536.0f, __builtin_fmaf((float)Ms, 256.0f, (float)Ls));
        return h2f((uint16_t)r.d) * (x.s[0] * v);
    }
};

// ---- Q8_0 -------------------------------------------------------------------------
template <> struct Q<kQ8_0> {
    static constexpr int GPB = 1;
    struct X { uint32_t h[8], m[8], l[8]; float s; };
    struct Raw { uint32_t q[9]; uint32_t sh, d; };
    __device__ static void load_x(const XView &xv, int g, X &x) {
        lds_words(xv.xh + 32 * g, x.h, 2);
        lds_words(xv.xm + 32 * g, x.m, 2);
        lds_words(xv.xl + 32 * g, x.l, 2);
        x.s = xv.s[g];
    }
    __device__ static Raw load(const uint8_t *__restrict__ row, int g) {
        const uint8_t *blk = row + g * 34;
        const uint8_t *qs = blk + 2;
        const uintptr_t mis = reinterpret_cast<uintptr_t>(qs) & 3;
        const uint32_t *p = reinterpret_cast<const uint32_t *>(qs - mis);
        Raw r;
        r.sh = (uint32_t)(mis & 2) << 3;
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = p[i];
        r.q[8] = p[8];  // LDS: the dword past the block is padding or the next block
        r.d = ld_u16(blk);
        return r;
    }
    __device__ static float dot(const Raw &r, int, const X &x) {
        int ah = 0, am = 0, al = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t v = __builtin_amdgcn_alignbit(r.q[w + 1], r.q[w], r.sh);
            ah = dot4(v, x.h[w], ah);
            am = dot4(v, x.m[w], am);
            al = dot4(v, x.l[w], al);
        }
        return h2f((uint16_t)r.d) * (x.s * planes(ah, am, al));
    }
};

// ---- lane geometry ----------------------------------------------------------------------
// P = largest power of two <= 64 dividing the row's group count G; if that leaves
// more than NG_MAX groups per lane, P = 64 with the tail groups masked.
#ifndef MX_NG_MAX
#define MX_NG_MAX 8
#endif
constexpr int NG_MAX = MX_NG_MAX;

// full_wave: a row whose groups fit one wave takes the whole wave (one group per
// lane, lanes past G idle) instead of P = the largest power of two dividing G;
// fewer activation registers per lane at the cost of idle lanes.
// Built on the host and passed to the kernels as an argument (so no wave spends
// scalar instructions on its divisions); lp = log2 P, lrpi = log2 RPI.
// wide: every row takes the whole wave (P = 64, the tail groups masked), so one
// row per iteration: rows whose RPI-row batches would not fit the DMA budget.
template <int DT> struct Geo {
    int G, P, NG, RPI, lp, lrpi;
    __host__ __device__ explicit Geo(int k, bool full_wave = false, bool wide = false) {
        G = (k / block_size(DT)) * Q<DT>::GPB;
        int p = G & (-G);
        if (p > 64) p = 64;
        if (G / p > NG_MAX) p = 64;
        if ((full_wave && G <= 64) || wide) p = 64;
        P = p;
        NG = (G + p - 1) / p;
        RPI = 64 / p;
        lp = 0;
        while ((1 << lp) < P) lp++;
        lrpi = 6 - lp;
    }
};

// the compiled groups-per-lane variants: the smallest >= NG
__host__ __device__ constexpr int ng_variant(int ng) {
    return ng <= 1 ? 1 : ng <= 2 ? 2 : ng <= 3 ? 3 : ng <= 4 ? 4 : ng <= 6 ? 6 : 8;
}

// Reduces NB tuples of NM floats over the P lanes of each row group.  While the
// tuple count allows, each exchange step (lane_partner) halves the tuples a lane
// keeps (the lane whose offset bit is set keeps the upper half), so NB tuples cost
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
        at_offset(o, [&](auto c) {
#pragma unroll
            for (int i = 0; i < half; i++) {
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const float keep = up ? v[half + i][m] : v[i][m];
                    const float send = up ? v[i][m] : v[half + i][m];
                    v[i][m] = keep + lane_partner<decltype(c)::value>(send);
                }
            }
        });
        if (up) which += half;
        o >>= 1;
    }
    for_offsets_down(o, [&](auto c) {
#pragma unroll
        for (int m = 0; m < NM; m++) v[0][m] += lane_partner<decltype(c)::value>(v[0][m]);
    });
    leader = (sub & (P / NB - 1)) == 0;
}

// Streams the rows [r_begin, r_end) of NM matrices that share one activation
// through this wave, NIT row-iterations (NIT * RPI rows) per batch, through the
// wave's LDS ring `ring` of RING buffers of ni KB (ni = dma_insts(NM, rows per
// batch, row_bytes)): batches i+1 .. i+RING-1 are in flight while batch i is
// computed.  A batch's image in a buffer is the NM matrices' row spans, each
// as the aligned 16-byte chunks covering it, packed back to back.  `pre`
// issues the activation loads before the first copies, `post` finishes filling
// `xs`.  sink(row, sums[NM]) runs once per row with the fully reduced sums.
// EARLY (RING == 1): a batch's weight words are read from LDS into registers
// first, then the next batch's copy is issued into the same buffer, then the
// batch is computed from registers -- the copy overlaps the compute without a
// second buffer.
template <int DT, int NG, int NIT, int NM, int RING, class XPreF, class XPostF, class Sink, bool EARLY = false>
__device__ __forceinline__ void stream_rows(const uint8_t *const (&w)[NM], int64_t row_bytes, const Geo<DT> &geo,
                                            typename Q<DT>::X (&xs)[NG], int r_begin, int r_end, uint8_t *ring,
                                            int ni, XPreF &&pre, XPostF &&post, Sink &&sink) {
    static_assert((NIT & (NIT - 1)) == 0, "NIT: a power of two");
    constexpr int LNIT = NIT == 1 ? 0 : NIT == 2 ? 1 : NIT == 4 ? 2 : NIT == 8 ? 3 : 4;
    const int lane = threadIdx.x & 63;
    const int sub = lane & (geo.P - 1);
    const int rsub = lane >> geo.lp;
    const int step = NIT << geo.lrpi;
    const int bstride = ni * 1024;
    const int nbatch = (r_end - r_begin + step - 1) >> (LNIT + geo.lrpi);
    // the chunk range [base_m, base_m + 16 * nch_m) of matrix m's span for the batch at r0
    auto span = [&](int m, int r0, uintptr_t &base, int &nch) {
        const int r1 = min(r0 + step, r_end);
        const uintptr_t S = reinterpret_cast<uintptr_t>(w[m] + (int64_t)r0 * row_bytes);
        const uintptr_t E = reinterpret_cast<uintptr_t>(w[m] + (int64_t)r1 * row_bytes);
        base = S & ~uintptr_t(15);
        nch = (int)((E + 15 - base) >> 4);
    };
    auto issue = [&](int bi) {
        const int r0 = r_begin + bi * step;
        uintptr_t base[NM];
        int nch[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) span(m, r0, base[m], nch[m]);
        uint8_t *dst = ring + (bi % RING) * bstride;
        const int per = ni / NM;  // instructions per matrix span
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const uint8_t *b = reinterpret_cast<const uint8_t *>(base[m]);
            for (int q = 0; q < per; q++) {
                const int ci = min(64 * q + lane, nch[m] - 1);  // spare lanes re-copy the last chunk
                dma16(b + (uint32_t)(16 * ci), dst + 1024 * (m * per + q));
            }
        }
    };
    auto process = [&](int bi) {
        const int r0 = r_begin + bi * step;
        // LDS offset of each matrix's row r0 in the batch's buffer (wave-uniform);
        // row r0 + i sits i * row_bytes after it
        int moff[NM];
        {
            uintptr_t base0, base1 = 0;
            int n0, n1 = 0;
            span(0, r0, base0, n0);
            moff[0] = (bi % RING) * bstride + (int)(reinterpret_cast<uintptr_t>(w[0] + (int64_t)r0 * row_bytes) - base0);
            if (NM > 1) {
                span(1, r0, base1, n1);
                moff[NM - 1] = (bi % RING) * bstride + 1024 * (ni / NM) +
                               (int)(reinterpret_cast<uintptr_t>(w[NM - 1] + (int64_t)r0 * row_bytes) - base1);
            }
        }
        const int rb32 = (int)row_bytes;
        float acc[NIT][NM];
        if constexpr (EARLY) {
            typename Q<DT>::Raw raw[NIT][NM][NG];
#pragma unroll
            for (int ib = 0; ib < NIT; ib++) {
                const int row = min(r0 + rsub + geo.RPI * ib, r_end - 1);
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const uint8_t *rl = ring + moff[m] + (row - r0) * rb32;
#pragma unroll
                    for (int jg = 0; jg < NG; jg++) {
                        const int g = sub + geo.P * jg;
                        raw[ib][m][jg] = Q<DT>::load(rl, g < geo.G ? g : 0);
                    }
                }
            }
            // the buffer's words are in registers: the next batch may overwrite it
            wait_lgkmcnt0();
            if (bi + 1 < nbatch) issue(bi + 1);
#pragma unroll
            for (int ib = 0; ib < NIT; ib++) {
                const bool ok = r0 + rsub + geo.RPI * ib < r_end;
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    float a = 0.f;
#pragma unroll
                    for (int jg = 0; jg < NG; jg++) {
                        const int g = sub + geo.P * jg;
                        if (ok && g < geo.G) a += Q<DT>::dot(raw[ib][m][jg], g, xs[jg]);
                    }
                    acc[ib][m] = a;
                }
            }
        } else
#pragma unroll
        for (int ib = 0; ib < NIT; ib++) {
            const int row = r0 + rsub + geo.RPI * ib;
            const bool ok = row < r_end;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                float a = 0.f;
                if (ok) {
                    const uint8_t *rl = ring + moff[m] + (row - r0) * rb32;
#pragma unroll
                    for (int jg = 0; jg < NG; jg++) {
                        const int g = sub + geo.P * jg;
                        if (g < geo.G) a += Q<DT>::dot(Q<DT>::load(rl, g), g, xs[jg]);
                    }
                }
                acc[ib][m] = a;
            }
        }
        int which;
        bool leader;
        reduce_tuples<NM, NIT>(acc, geo.P, sub, which, leader);
        if (leader) {
            if (geo.P < NIT) {
#pragma unroll
                for (int ib = 0; ib < NIT; ib++) {
                    const int row = r0 + rsub + geo.RPI * ib;
                    if (row < r_end) sink(row, acc[ib]);
                }
            } else {
                const int row = r0 + rsub + geo.RPI * which;
                if (row < r_end) sink(row, acc[0]);
            }
        }
    };
    if constexpr (EARLY) {
        static_assert(RING == 1, "EARLY re-issues into the one buffer");
        pre();
        if (nbatch > 0) issue(0);
        post();
        for (int bi = 0; bi < nbatch; bi++) {
            wait_vmcnt(0);
            process(bi);
        }
        return;
    }
    pre();
    for (int bi = 0; bi < RING - 1 && bi < nbatch; bi++) issue(bi);
    post();
    for (int bi = 0; bi < nbatch; bi++) {
        if (bi + RING - 1 < nbatch) issue(bi + RING - 1);
        // batch bi has landed once at most the copies of the later batches are outstanding
        wait_vmcnt(ni * min(RING - 1, nbatch - 1 - bi));
        process(bi);
    }
}

// Loads this lane's slices from the group-major staged copy (mx_stage.h):
// GM_CHUNKS 16-byte loads per group, each wave instruction 1 KB of consecutive bytes.
template <int DT, int NG>
__device__ __forceinline__ void load_xs_gm(const uint8_t *gm, int k, const Geo<DT> &geo,
                                           typename Q<DT>::X (&xs)[NG]) {
    static_assert(DT == kQ4_K || DT == kQ5_K, "group-major staging is the 64-value group layout");
    const int G = k / 64;
    const uint4 *c = reinterpret_cast<const uint4 *>(gm);
    const int sub = (threadIdx.x & 63) & (geo.P - 1);
    auto put = [](uint32_t *d, const uint4 v) { d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w; };
#pragma unroll
    for (int jg = 0; jg < NG; jg++) {
        int g = sub + geo.P * jg;
        g = g < G ? g : 0;
        typename Q<DT>::X &x = xs[jg];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            put(x.h + 4 * q, c[(size_t)q * G + g]);
            put(x.m + 4 * q, c[(size_t)(4 + q) * G + g]);
            put(x.l + 4 * q, c[(size_t)(8 + q) * G + g]);
        }
        const uint4 sc = c[(size_t)12 * G + g];
        x.sa = __uint_as_float(sc.x);
        x.sb = __uint_as_float(sc.y);
        x.ssa = __uint_as_float(sc.z);
        x.ssb = __uint_as_float(sc.w);
    }
}

// Loads this lane's slices of a staged activation row (global memory or LDS).
template <int DT, int NG>
__device__ __forceinline__ void load_xs(const uint8_t *staged, int k, const Geo<DT> &geo,
                                        typename Q<DT>::X (&xs)[NG]) {
    const XView xv(staged, k);
    const int sub = (threadIdx.x & 63) & (geo.P - 1);
#pragma unroll
    for (int jg = 0; jg < NG; jg++) {
        const int g = sub + geo.P * jg;
        Q<DT>::load_x(xv, g < geo.G ? g : 0, xs[jg]);
    }
}

#ifndef MX_WAVES
#define MX_WAVES 4
#endif
// rows per wave and LDS ring depth per kernel (tuned on MI355X for the C1 layer)
#ifndef MX_RW_GU
#define MX_RW_GU 1
#endif
#ifndef MX_RING_GU
#define MX_RING_GU 1
#endif
#ifndef MX_GU_EARLY
#define MX_GU_EARLY 0
#endif
constexpr bool GU_EARLY = MX_GU_EARLY != 0;
#ifndef MX_RW_DN
#define MX_RW_DN 16
#endif
#ifndef MX_RING_DN
#define MX_RING_DN 1
#endif
#ifndef MX_NIT1
#define MX_NIT1 1
#endif
#ifndef MX_NIT2
#define MX_NIT2 1
#endif
#ifndef MX_WAVES_DN
#define MX_WAVES_DN 4
#endif
#ifndef MX_DN_FULL
#define MX_DN_FULL 0
#endif
#ifndef MX_NIT_DN
#define MX_NIT_DN 1
#endif
constexpr int WAVES = MX_WAVES;
constexpr int WAVES_DN = MX_WAVES_DN;  // waves per block of the fused down kernel
#ifndef MX_DN_TPB
#define MX_DN_TPB 4
#endif
constexpr int DN_TPB = MX_DN_TPB;  // RW_DN-row tiles per wave of k_decode_down
constexpr int RW_MV = 16, RW_GU = MX_RW_GU, RW_DN = MX_RW_DN;
constexpr int RING_MV = 2, RING_GU = MX_RING_GU, RING_DN = MX_RING_DN;

// row-iterations per batch: NIT * RPI rows are copied per DMA batch
template <int NG> struct Batch { static constexpr int NIT = NG == 1 ? MX_NIT1 : MX_NIT2; };

// the down kernel's row layout (Geo full_wave) and row-iterations per batch
constexpr bool DN_FULL = MX_DN_FULL != 0;
template <int NG> struct BatchDn { static constexpr int NIT = NG == 1 && DN_FULL ? MX_NIT_DN : Batch<NG>::NIT; };

// DMA instructions per batch for NM matrices of row_bytes rows at k
template <int DT, int NG>
static int ring_insts(int nm, int k, int64_t row_bytes, int nit = Batch<NG>::NIT, bool full_wave = false,
                      bool wide = false) {
    return dma_insts(nm, nit * Geo<DT>(k, full_wave, wide).RPI, row_bytes);
}
__host__ __device__ inline size_t align16(size_t v) { return (v + 15) & ~size_t(15); }

// ---- mul_mv_id -----------------------------------------------------------------------
// grid (row tiles, t * top_k); one (token, slot) pair per block, its activation
// row staged into LDS by the whole block, then one LDS ring per wave.
template <int DT, int NG>
__global__ void __launch_bounds__(64 * WAVES) k_mul_mv_id(MvArgs a, int ni, Geo<DT> geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int pair = blockIdx.y;  // token * top_k + slot
    const int tok = pair / a.top_k, slot = pair % a.top_k;
    int e = 0;
    if (a.ids) {
        const uint32_t id = a.ids[pair];
        e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
    }
    const float *xrow = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
    const uint8_t *const w[1] = {a.w + (int64_t)e * a.expert_bytes};
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
    const int r0 = blockIdx.x * (WAVES * RW_MV) + wave * RW_MV;
    typename Q<DT>::X xs[NG];
    XPre xp;
    uint8_t *ring = lds + align16(xstage_bytes(a.k)) + wave * (RING_MV * ni * 1024);
    if (r0 >= a.n_out) {  // wave-uniform: take part in the staging, then leave
        stage_pre(xrow, a.k, xp);
        stage_post(xrow, a.k, xp, lds);
        return;
    }
    float *dst = a.dst + (int64_t)pair * a.n_out;
    stream_rows<DT, NG, Batch<NG>::NIT, 1, RING_MV>(
        w, a.row_bytes, geo, xs, r0, min(r0 + RW_MV, a.n_out), ring, ni, [&] { stage_pre(xrow, a.k, xp); },
        [&] {
            stage_post(xrow, a.k, xp, lds);
            load_xs<DT, NG>(lds, a.k, geo, xs);
        },
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

template <int DT, int NG>
static mx_status launch_mv_ng(const MvArgs &a, dim3 grid, hipStream_t s) {
    const int ni = ring_insts<DT, NG>(1, a.k, a.row_bytes);
    if (ni > DMA_MAX_INSTS) return fail(MX_ERR_SHAPE, "mul_mv_id: rows of %lld bytes are too long", (long long)a.row_bytes);
    const size_t lds = align16(xstage_bytes(a.k)) + (size_t)WAVES * RING_MV * ni * 1024;
    if (lds > 160 * 1024) return fail(MX_ERR_SHAPE, "mul_mv_id: k = %d needs %zu bytes of LDS", a.k, lds);
    hipLaunchKernelGGL((k_mul_mv_id<DT, NG>), grid, dim3(64 * WAVES), lds, s, a, ni, Geo<DT>(a.k));
    return MX_OK;
}

template <int DT>
static mx_status launch_mv_dt(const MvArgs &a, dim3 grid, hipStream_t s) {
    const int ng = ng_variant(Geo<DT>(a.k).NG);
#define MX_L(N) return launch_mv_ng<DT, N>(a, grid, s)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
    return MX_OK;
}

// ---- compile-time Q6_K mat-vec (plain mul_mv and mul_mv_id, e.g. the lm_head) ----------
// Q6_K rows of K = 32 * P * NG weights: P lanes per row, NG 32-weight groups per
// lane, RPI = 64 / P rows per batch.  The geometry of k_mul_mv_id, with every
// count compile-time: the row bytes, the batch's copy instructions (so every
// vmcnt wait is an immediate, no runtime wait table), the lanes' field offsets
// and 2-byte block phases (rows are 4-byte aligned: 210 * K / 256 is a multiple
// of 4), hoisted out of the row loop as in k_decode_down_q6r.  Each wave walks
// MVQ6_RPW rows of one (token, slot) pair in batches through two LDS buffers of
// its own (batch b + 1 in flight while b is contracted); the workgroup stages the
// pair's activation row once.  Same per-row arithmetic and 32-lane sum as
// k_mul_mv_id (Q<kQ6_K>::dot, reduce_tuples).  The rows per wave (nb batches) are
// chosen at launch so that the grid is one round of resident workgroups: with a
// fixed 16 rows the lm_head's 1568 workgroups ran as 2.04 rounds of 768, the last
// round almost empty.
#ifndef MX_MV_Q6
#define MX_MV_Q6 1
#endif
#ifndef MX_MVQ6_RPW
#define MX_MVQ6_RPW 16
#endif
constexpr int MVQ6_RPW = MX_MVQ6_RPW;  // the fewest rows per wave

template <int NG, int P> struct MvQ6 {
    static constexpr int K = 32 * P * NG, RB = K / 256 * 210, RPI = 64 / P;
    static constexpr int BCH = RPI * RB / 16, NI = (BCH + 63) / 64, NB = MVQ6_RPW / RPI;
    static_assert((RPI * RB) % 16 == 0 && RB % 4 == 0, "batches start 16-byte aligned, rows 4-byte aligned");
    static_assert(MVQ6_RPW % RPI == 0 && NB % 2 == 0, "whole batch pairs per wave");
};
// nb: batches per wave (even, >= MvQ6::NB)
template <int NG, int P>
__global__ void __launch_bounds__(64 * WAVES) k_mv_q6(MvArgs a, int nb) {
    using G = MvQ6<NG, P>;
    constexpr int DT = kQ6_K, RB = G::RB, RPI = G::RPI, NI = G::NI, BCH = G::BCH;
    const int nbt = a.n_out / RPI;  // batches of the matrix (whole: the launcher checks)
    __shared__ __attribute__((aligned(16))) uint8_t ring0[WAVES][NI * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[WAVES][NI * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t stg[(xstage_bytes(G::K) + 15) & ~15];
    const int pair = blockIdx.y;  // token * top_k + slot
    const int tok = pair / a.top_k, slot = pair % a.top_k;
    int e = 0;
    if (a.ids) {
        const uint32_t id = a.ids[pair];
        e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int sub = lane & (P - 1), rsub = lane / P;
    // grid-strided batches: the wave's batch bi is gw + bi * NW, so the waves of the
    // grid stream neighbouring batches together (with one contiguous run of rows per
    // wave the lm_head's copies alone took 51 us, grid-strided 46.5 us); a batch
    // past the end re-copies the matrix's last batch and stores nothing
    const int gw = blockIdx.x * WAVES + wave, NW = gridDim.x * WAVES;
    const float *xrow = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
    const uint8_t *wp = a.w + (int64_t)e * a.expert_bytes;
    uint8_t *const b0 = ring0[wave], *const b1 = ring1[wave];
    // every lane issues every copy (spare lanes repeat the batch's last chunk into
    // the buffer's unused tail): no branch around a copy, so the counts stay exact
    auto issue = [&](int bi, uint8_t *dst) {
        const uint8_t *src = wp + (int64_t)min(gw + bi * NW, nbt - 1) * (RPI * RB);
#pragma unroll
        for (int q = 0; q < NI; q++) {
            const int ci = min(64 * q + lane, BCH - 1);
            dma16(src + (uint32_t)(16 * ci), dst + 1024 * q);
        }
        asm volatile("" ::: "memory");
    };
    XPre xp;
    stage_pre(xrow, G::K, xp);
    // the activation loads have returned before the first copies are issued
    // (ordinary loads are not counted across LDS copies)
    wait_vmcnt(0);
#pragma unroll
    for (int i = 0; i < XPRE; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) asm volatile("" : "+v"(xp.v[i][j]));
    issue(0, b0);
    issue(1, b1);
    stage_post_t(xrow, G::K, xp, stg, (int)threadIdx.x, (int)blockDim.x);
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();  // (a bare barrier: __syncthreads would wait for the copies)
    asm volatile("" ::: "memory");
    typename Q<DT>::X xs[NG];
    {
        const XView xv(stg, G::K);
#pragma unroll
        for (int jg = 0; jg < NG; jg++) Q<DT>::load_x(xv, sub + P * jg, xs[jg]);
    }
    uint32_t oa[NG], ohq[NG], osc[NG], od[NG], sh[NG];
#pragma unroll
    for (int jg = 0; jg < NG; jg++) {
        const int g = sub + P * jg, b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint32_t mis = (uint32_t)(210 * b) & 2u, ab = (uint32_t)(210 * b) - mis;
        oa[jg] = ab + 64 * n + 8 * j;
        ohq[jg] = ab + 128 + 32 * n + 8 * j;
        osc[jg] = ab + 192 + 8 * n;
        od[jg] = (uint32_t)(210 * b) + 208;
        sh[jg] = mis << 3;
    }
    float *dst = a.dst + (int64_t)pair * a.n_out;
    auto batch = [&](int bi, uint8_t *buf) {
        wait_vmcnt(NI);  // batch bi has landed (bi + 1 is in flight)
        const uint8_t *rl = buf + rsub * RB;
        float acc[1][1];
        // the batch's fields into registers, then the copy of batch bi + 2 into the
        // same buffer, then the dots: the copy is in flight while they run (175
        // VGPRs, 2 waves/SIMD; forced to 3 it spills and takes 64 us instead of 54)
        typename Q<DT>::Raw r[NG];
#pragma unroll
        for (int jg = 0; jg < NG; jg++) {
            Q<DT>::ld3(rl + oa[jg], r[jg].a);
            Q<DT>::ld3(rl + oa[jg] + 32, r[jg].b);
            Q<DT>::ld3(rl + ohq[jg], r[jg].hq);
            Q<DT>::ld3(rl + osc[jg], r[jg].sc);
            r[jg].d = ld_u16(rl + od[jg]);
            r[jg].sh = sh[jg];
        }
        wait_lgkmcnt0();  // every read of the buffer returned before it is overwritten
        issue(bi + 2, buf);
        float v = 0.f;
#pragma unroll
        for (int jg = 0; jg < NG; jg++) v += Q<DT>::dot(r[jg], sub + P * jg, xs[jg]);
        acc[0][0] = v;
        int which;
        bool leader;
        reduce_tuples<1, 1>(acc, P, sub, which, leader);
        const int b = gw + bi * NW;
        if (leader && b < nbt) dst[b * RPI + rsub] = acc[0][0];
    };
#pragma unroll 1
    for (int bi = 0; bi < nb; bi += 2) {
        batch(bi, b0);
        batch(bi + 1, b1);
    }
    wait_vmcnt(0);  // no copy into this workgroup's LDS outlives it
}

// the (NG, P) variant of k_mv_q6 for this shape, or false
static bool mv_q6_pick(const MvArgs &a, int &ng, int &p) {
    auto al = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (!al(a.w) || a.expert_bytes % 16 != 0 || a.row_bytes != (int64_t)a.k / 256 * 210) return false;
    switch (a.k) {
    case 1536: ng = 3; p = 16; break;
    case 2048: ng = 2; p = 32; break;
    case 3072: ng = 3; p = 32; break;
    case 4096: ng = 4; p = 32; break;
    default: return false;
    }
    // whole batches: a batch's copy never reads past the matrix's last row
    return a.n_out % (64 / p) == 0;
}
// resident workgroups of k_mv_q6<NG, P> on the current device (0: unknown)
template <int NG, int P> static int mv_q6_resident() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cache[dev]) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_mv_q6<NG, P>, 64 * WAVES, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cache[dev] = per_cu > 0 && cus > 0 ? per_cu * cus : -1;
    }
    return cache[dev] > 0 ? cache[dev] : 0;
}
template <int NG, int P> static void launch_mv_q6_v(const MvArgs &a, hipStream_t s) {
    using G = MvQ6<NG, P>;
    const int64_t pairs = (int64_t)a.t * a.top_k;
    // batches per wave: at least G::NB, else enough that every workgroup of the grid
    // is resident at once (the rows of all pairs over the resident waves)
    const int64_t res = mv_q6_resident<NG, P>();
    int64_t nb = G::NB;
    if (res > 0) {
        const int64_t rows_per_wave = (a.n_out * pairs + res * WAVES - 1) / (res * WAVES);
        const int64_t want = (rows_per_wave + G::RPI - 1) / G::RPI;
        nb = want > nb ? (want + 1) & ~int64_t(1) : nb;
    }
    const int64_t rpw = nb * G::RPI;
    const dim3 grid((unsigned)((a.n_out + WAVES * rpw - 1) / (WAVES * rpw)), (unsigned)pairs);
    hipLaunchKernelGGL((k_mv_q6<NG, P>), grid, dim3(64 * WAVES), 0, s, a, (int)nb);
}
static mx_status launch_mv_q6(const MvArgs &a, int ng, int p, hipStream_t s) {
    if (ng == 3 && p == 16) launch_mv_q6_v<3, 16>(a, s);
    else if (ng == 2) launch_mv_q6_v<2, 32>(a, s);
    else if (ng == 3) launch_mv_q6_v<3, 32>(a, s);
    else launch_mv_q6_v<4, 32>(a, s);
    MX_LAUNCH("k_mv_q6");
    return MX_OK;
}

// ---- shape fits of the LDS-ring kernels (host) --------------------------------------
// Each kernel holds NG <= NG_MAX activation groups per lane, copies a batch of rows
// with at most DMA_MAX_INSTS wave instructions per matrix set, and needs its LDS.
template <int DT> static int64_t row_bytes_of(int k) { return (int64_t)(k / block_size(DT)) * type_size(DT); }
template <int DT> static bool geo_ok(int k, bool full_wave = false) {
    return k > 0 && k % block_size(DT) == 0 && Geo<DT>(k, full_wave).NG <= NG_MAX;
}
template <int DT> static bool mv_fits_dt(int k) {
    if (!geo_ok<DT>(k)) return false;
    const Geo<DT> g(k);
    const int nit = g.NG == 1 ? Batch<1>::NIT : Batch<2>::NIT;
    const int ni = dma_insts(1, nit * g.RPI, row_bytes_of<DT>(k));
    return ni <= DMA_MAX_INSTS && align16(xstage_bytes(k)) + (size_t)WAVES * RING_MV * ni * 1024 <= 160 * 1024;
}
template <int DT> static bool gu_geo_fits(int hidden, int64_t row_bytes, bool wide) {
    const Geo<DT> g(hidden, false, wide);
    if (!(hidden > 0 && hidden % block_size(DT) == 0 && g.NG <= NG_MAX) || row_bytes != row_bytes_of<DT>(hidden))
        return false;
    const int nit = g.NG == 1 ? Batch<1>::NIT : Batch<2>::NIT;
    const int ni = dma_insts(2, nit * g.RPI, row_bytes);
    return ni <= DMA_MAX_INSTS && (size_t)WAVES * RING_GU * ni * 1024 <= 160 * 1024;
}
// the gate/up rows take the wide geometry (hidden 7168: 112 groups, 16 lanes a row
// and 4 rows an iteration put 32 copy instructions in a gate + up batch)
template <int DT> static bool gu_wide(int hidden, int64_t row_bytes) {
    return !gu_geo_fits<DT>(hidden, row_bytes, false) && gu_geo_fits<DT>(hidden, row_bytes, true);
}
template <int DT> static bool gu_fits_dt(int hidden, int64_t row_bytes) {
    return gu_geo_fits<DT>(hidden, row_bytes, false) || gu_geo_fits<DT>(hidden, row_bytes, true);
}
template <int DT> static bool dn_fits_dt(int ff, int64_t row_bytes) {
    if (!geo_ok<DT>(ff, DN_FULL) || row_bytes != row_bytes_of<DT>(ff)) return false;
    const Geo<DT> g(ff, DN_FULL);
    const int nit = g.NG == 1 ? BatchDn<1>::NIT : BatchDn<2>::NIT;
    const int ni = dma_insts(1, nit * g.RPI, row_bytes);
    return ni <= DMA_MAX_INSTS && align16(xstage_bytes(ff)) + (size_t)WAVES_DN * RING_DN * ni * 1024 <= 160 * 1024;
}
#define MX_DT_SWITCH(dtype, EXPR)                       \
    switch (dtype) {                                    \
    case kQ4_K: { constexpr int DT = kQ4_K; return EXPR; } \
    case kQ5_K: { constexpr int DT = kQ5_K; return EXPR; } \
    case kQ6_K: { constexpr int DT = kQ6_K; return EXPR; } \
    case kQ8_0: { constexpr int DT = kQ8_0; return EXPR; } \
    default: return false;                              \
    }
bool mv_ring_fits(int dtype, int k) { MX_DT_SWITCH(dtype, mv_fits_dt<DT>(k)) }
bool decode_gate_up_fits(int dtype, int hidden, int64_t row_bytes) { MX_DT_SWITCH(dtype, gu_fits_dt<DT>(hidden, row_bytes)) }
bool decode_down_fits(int dtype, int ff, int64_t row_bytes) { MX_DT_SWITCH(dtype, dn_fits_dt<DT>(ff, row_bytes)) }
#undef MX_DT_SWITCH

mx_status launch_mul_mv_id(int dtype, const MvArgs &a, hipStream_t s) {
    const dim3 grid((unsigned)((a.n_out + WAVES * RW_MV - 1) / (WAVES * RW_MV)), (unsigned)(a.t * a.top_k));
    if (grid.y == 0 || grid.x == 0) return MX_OK;
    if (!mv_ring_fits(dtype, a.k)) {  // any other row width: the f32 mat-vec
        const MvfArgs f{a.w, a.expert_bytes, a.row_bytes, a.n_expert, a.n_out, a.k, a.x, a.x_per_row,
                        a.ids, a.t, a.top_k, a.dst, a.top_k, 0};
        return launch_mv_f32(dtype, f, s);
    }
    int ng = 0, p = 0;
    if (dtype == kQ6_K && MX_MV_Q6 && mv_q6_pick(a, ng, p)) return launch_mv_q6(a, ng, p, s);
    switch (dtype) {
    case kQ4_K: MX_TRY(launch_mv_dt<kQ4_K>(a, grid, s)); break;
    case kQ5_K: MX_TRY(launch_mv_dt<kQ5_K>(a, grid, s)); break;
    case kQ6_K: MX_TRY(launch_mv_dt<kQ6_K>(a, grid, s)); break;
    default: MX_TRY(launch_mv_dt<kQ8_0>(a, grid, s)); break;
    }
    MX_LAUNCH("k_mul_mv_id");
    return MX_OK;
}

// ---- fused decode: gate/up + SwiGLU ---------------------------------------------------
// grid (ff / (WAVES * RW_GU) row tiles, nslot slots, t tokens): slots slot0 ..
// slot0 + nslot - 1; slot top_k (if present) is the shared expert, which then has
// the routed experts' quant type and shape.
// act[tok, slot, r] = silu(gate_r . x) * (up_r . x), silu(g) = g / (1 + exp(-g)),
// the product rounded on its own (silu_mul.metal:57-72).  The token row comes
// staged from the router kernel (global memory).  Expert waves are independent.
// The routed slots read the ids the selection kernel (k_decode_select, the
// previous launch) wrote.
#ifndef MX_GU_WPE
#define MX_GU_WPE 5
#endif
// waves per SIMD the generic gate/up kernel's registers must allow: MX_GU_WPE
// for one activation group per lane; each further group holds its three digit
// planes in registers (Q4_K / Q5_K: 52 VGPRs a group), so more groups get fewer
// waves (at 5 waves per SIMD two groups spilled 200 bytes per lane to scratch,
// eight 1.6 KB)
template <int DT, int NG> constexpr int gu_wpe() {
    if (NG <= 1) return MX_GU_WPE;
    if (DT == kQ8_0) return NG <= 2 ? 5 : NG <= 4 ? 4 : 2;
    if (DT == kQ6_K) return NG <= 2 ? 4 : NG <= 3 ? 3 : NG <= 4 ? 2 : 1;
    return NG <= 2 ? 3 : NG <= 4 ? 2 : 1;
}
template <int DT, int NG, bool GM>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(gu_wpe<DT, NG>())))
k_decode_gate_up(DecodeGateUpArgs a, int ni, int slot0, Geo<DT> geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int slots = a.top_k + (a.sh_gate ? 1 : 0);
    const int tile = blockIdx.x;
    int slot = slot0 + blockIdx.y, tok = blockIdx.z;
    int pe = -1;  // the pair's expert, from the expert-ordered launch list
    if (a.perm) {  // (all slots launched: slot0 == 0)
        const int v = a.perm[blockIdx.z * slots + blockIdx.y];
        tok = (v & 0xFFFF) / slots;
        slot = (v & 0xFFFF) % slots;
        pe = v >> 16;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
    const int r0 = tile * (WAVES * RW_GU) + wave * RW_GU;
    if (r0 >= a.ff) return;  // wave-uniform; no block barrier below
    float *act = a.act + ((int64_t)tok * slots + slot) * a.ff;
    const uint8_t *gw, *uw;
    int64_t rb;
    if (slot < a.top_k) {
        const uint32_t id = pe >= 0 ? (uint32_t)pe : a.ids[tok * a.top_k + slot];
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
    typename Q<DT>::X xs[NG];
    const uint8_t *staged = a.xstage + (int64_t)tok * xstage_stride(a.hidden);
    uint8_t *ring = lds + wave * (RING_GU * ni * 1024);
    // GM: the slices come from the group-major copy (a compile-time choice: a
    // runtime branch between the two loaders measurably delays the loads)
    auto pre = [&] {
        if constexpr (GM) load_xs_gm<DT, NG>(a.xstage_gm + (int64_t)tok * xstage_gm_stride(a.hidden), a.hidden, geo, xs);
        else load_xs<DT, NG>(staged, a.hidden, geo, xs);
    };
    auto sink = [&](int row, const float (&s)[2]) {
        const float g = s[0];
        const float sg = g / (1.0f + expf(-g));
        act[row] = sg * s[1];
    };
    auto nopost = [] {};
    stream_rows<DT, NG, Batch<NG>::NIT, 2, RING_GU, decltype(pre) &, decltype(nopost) &, decltype(sink) &, GU_EARLY>(
        w, rb, geo, xs, r0, min(r0 + RW_GU, a.ff), ring, ni, pre, nopost, sink);
}

// Gate/up rows of exactly 64 groups (Q4_K / Q5_K at hidden 4096, 16-byte-aligned
// rows): the geometry is compile-time -- one group per lane, one row pair per
// iteration, no masked lanes -- and each wave takes R consecutive row pairs of its
// (slot, token).  The wave's one LDS buffer holds a gate row and an up row; as
// soon as the current pair's words are in registers the next pair's copy is
// issued into it, so the copy overlaps the dot products.  Sums and SwiGLU are the
// generic kernel's, operation for operation (the 64-lane sums in the same order).
#ifndef MX_GU64_R
#define MX_GU64_R 2
#endif
constexpr int GU64_R = MX_GU64_R;
#ifndef MX_GU64_TPB
#define MX_GU64_TPB 8
#endif
constexpr int GU64_TPB = MX_GU64_TPB;
#ifndef MX_GU64_TPB1
#define MX_GU64_TPB1 3
#endif
constexpr int GU64_TPB1 = MX_GU64_TPB1;
template <int DT> struct Row64 {
    static_assert(DT == kQ4_K || DT == kQ5_K, "64-group rows: the K-quants with 64-weight groups");
    static constexpr int RB = 16 * (DT == kQ4_K ? 144 : 176);  // row bytes (16 super-blocks)
    static constexpr int CH = RB / 16, NI = (CH + 63) / 64;     // 16-byte chunks, copy instructions
};
constexpr int GU_SEL_E = 256;  // experts of the in-block top-k
static_assert(64 * WAVES == SEL_THREADS, "the in-block top-k needs SEL_THREADS threads");
// TPB: row-pair tiles per workgroup (tiles blockIdx.x, blockIdx.x + gridDim.x, ...
// of its (slot, token)); WPE: waves per SIMD the registers must allow (the verify
// form runs at 4: C2 333 -> 324 us; t = 1 at 5); AUX: the weight copies' cache
// policy (DMA_NT at t = 1).
template <int DT, int R, int TPB, int WPE, int AUX>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(WPE)))
k_decode_gate_up64(DecodeGateUpArgs a, int slot0, Geo<DT> geo) {
    constexpr int RB = Row64<DT>::RB, CH = Row64<DT>::CH, NI = Row64<DT>::NI;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int slots = a.top_k + (a.sh_gate ? 1 : 0);
    int slot = slot0 + blockIdx.y, tok = blockIdx.z;
    int pe = -1;  // the pair's expert, from the expert-ordered launch list
    if (a.perm) {  // (all slots launched: slot0 == 0)
        const int v = a.perm[blockIdx.z * slots + blockIdx.y];
        tok = (v & 0xFFFF) / slots;
        slot = (v & 0xFFFF) % slots;
        pe = v >> 16;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // the workgroup walks its tiles loading the activation slices and the expert once
    const int rfirst = (blockIdx.x * WAVES + wave) * R;
    typename Q<DT>::X xs[1];
    if (rfirst < a.ff) load_xs_gm<DT, 1>(a.xstage_gm + (int64_t)tok * xstage_gm_stride(a.hidden), a.hidden, geo, xs);
    if (a.sel_keys && slot < a.top_k) {  // block-uniform: the whole block selects (t == 1)
        auto &sh = *reinterpret_cast<SelSharedT<GU_SEL_E> *>(lds + WAVES * 2 * RB);
        const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
        topk_from_keys<GU_SEL_E>(a.sel_keys, a.sel_probs, a.n_expert, a.top_k, a.sel_scale, a.sel_apply,
                                 a.sel_norm, writer ? a.sel_ids : nullptr, a.sel_w, sh);
        pe = sh.pick[slot];
    }
    if (rfirst >= a.ff) return;  // wave-uniform; no block barrier below
    const uint8_t *gw, *uw;
    if (slot < a.top_k) {
        const uint32_t id = pe >= 0 ? (uint32_t)pe : a.ids[tok * a.top_k + slot];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        gw = a.gate + (int64_t)e * a.gu_expert_bytes;
        uw = a.up + (int64_t)e * a.gu_expert_bytes;
    } else {
        gw = a.sh_gate;
        uw = a.sh_up;
    }
    const uint8_t *const gw0 = gw, *const uw0 = uw;
    uint8_t *buf = lds + wave * (2 * RB);
    // The wave's row pairs i = tt * R + r: row r of its slice of tile blockIdx.x +
    // tt * gridDim.x.  Valid pairs form a prefix (only the matrix's last tile is
    // partial), and the copy of pair i + 1 is issued as soon as pair i's words are
    // in registers, across tiles too: the wave never waits for a first copy after
    // its first pair.
    constexpr int NR = TPB * R;
    auto row_of = [&](int i) { return ((int)blockIdx.x + (i / R) * (int)gridDim.x) * (WAVES * R) + wave * R + i % R; };
    // row pair i of matrix m (0 gate, 1 up) into the matrix's half of the buffer;
    // every address a scalar base plus a 32-bit lane offset
    auto issue = [&](int m, int i) {
        const uint8_t *src = (m ? uw0 : gw0) + (int64_t)row_of(i) * RB;
#pragma unroll
        for (int q = 0; q < NI; q++) {
            const int ci = 64 * q + lane;
            if (q < NI - 1 || ci < CH) dma16<AUX>(src + (uint32_t)(16 * ci), buf + m * RB + 1024 * q);
        }
        asm volatile("" ::: "memory");
    };
    float res[NR];
    issue(0, 0);  // (row_of(0) < ff: checked above)
    issue(1, 0);
    // Only the copies count in vmcnt inside the loop (the act stores come after it):
    // when pair i's gate copy is waited for, at most pair i's up copy is younger; when
    // its up copy is, at most pair i + 1's gate copy.
#pragma unroll
    for (int i = 0; i < NR; i++) {
        if (i == 0 || row_of(i) < a.ff) {  // wave-uniform
            const bool more = i + 1 < NR && row_of(i + 1) < a.ff;
            float v2[2];
#pragma unroll
            for (int m = 0; m < 2; m++) {
                wait_vmcnt(m == 0 || more ? NI : 0);
                const typename Q<DT>::Raw rw = Q<DT>::load(buf + m * RB, lane);
                if (more) {
                    wait_lgkmcnt0();  // the words are in registers: the half may be overwritten
                    issue(m, i + 1);
                }
                v2[m] = Q<DT>::dot(rw, lane, xs[0]);
            }
            // 64-lane sums of g and u: lanes 0-31 keep g, 32-63 keep u after the first step
            const bool hi = (lane & 32) != 0;
            float v = (hi ? v2[1] : v2[0]) + lane_partner<32>(hi ? v2[0] : v2[1]);
            v += lane_partner<16>(v);
            v += lane_partner<8>(v);
            v += lane_partner<4>(v);
            v += lane_partner<2>(v);
            v += lane_partner<1>(v);
            const float G = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
            const float U = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
            res[i] = G / (1.0f + expf(-G)) * U;
        }
    }
    float *act = a.act + ((int64_t)tok * slots + slot) * a.ff;
#pragma unroll
    for (int i = 0; i < NR; i++)
        if ((i == 0 || row_of(i) < a.ff) && lane == i % R) act[row_of(i)] = res[i];
}

// The selection blocks alone (a launch with no expert slots): their own kernel,
// so profiles tell the top-k from the expert rows.
__global__ void __launch_bounds__(SEL_THREADS) k_decode_select(int top_k, DecodeSelArgs sel) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    SelShared &sh = *reinterpret_cast<SelShared *>(lds);
    const int64_t o = (int64_t)blockIdx.x * sel.n_expert;
    topk_from_keys(sel.keys + o, sel.probs + o, sel.n_expert, top_k, sel.scale, sel.apply_scale, sel.norm,
                   sel.ids + (int64_t)blockIdx.x * top_k, sel.w + (int64_t)blockIdx.x * top_k, sh);
}

__global__ void __launch_bounds__(PAIR_ORDER_THREADS) k_pair_order(const uint32_t *__restrict__ ids, int t,
                                                                    int top_k, int n_expert, int slots,
                                                                    int32_t *__restrict__ perm,
                                                                    int32_t *__restrict__ runs) {
    constexpr int NT = PAIR_ORDER_THREADS, PPT = PAIR_ORDER_MAX / NT;  // pairs per thread
    __shared__ int cnt[SEL_MAX_E + 2];
    __shared__ int s_scan[NT];
    const int tid = threadIdx.x, n = t * slots, ne = n_expert + 1;  // expert n_expert: the shared slot
    for (int i = tid; i < ne; i += NT) cnt[i] = 0;
    __syncthreads();
    // pair tid + NT j of this thread: its expert and its rank among the expert's pairs
    int pe[PPT], rank[PPT];
#pragma unroll
    for (int j = 0; j < PPT; j++) {
        const int v = tid + NT * j;
        pe[j] = 0;
        rank[j] = 0;
        if (v < n) {
            const int tok = v / slots, slot = v % slots;
            int e = n_expert;
            if (slot < top_k) {
                const uint32_t id = ids[tok * top_k + slot];
                e = id < (uint32_t)n_expert ? (int)id : n_expert - 1;  // as the expert kernels clamp it
            }
            pe[j] = e;
            rank[j] = atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // exclusive scan of the counts (low 16 bits) and of the 16-pair runs (high
    // 16 bits; both totals <= PAIR_ORDER_MAX < 2^16): each thread sums `per` experts
    const int per = (ne + NT - 1) / NT;
    const int e0 = min(tid * per, ne), e1 = min(e0 + per, ne);
    int sum = 0;
    for (int i = e0; i < e1; i++) sum += cnt[i] + (((cnt[i] + 15) >> 4) << 16);
    s_scan[tid] = sum;
    __syncthreads();
    for (int d = 1; d < NT; d <<= 1) {
        const int v = tid >= d ? s_scan[tid - d] : 0;
        __syncthreads();
        s_scan[tid] += v;
        __syncthreads();
    }
    const int ex = s_scan[tid] - sum;
    int run = ex & 0xFFFF, r = ex >> 16;
    for (int i = e0; i < e1; i++) {
        const int c = cnt[i];
        cnt[i] = run;
        if (runs)
            for (int j = 0; j < c; j += 16, r++) {
                runs[2 + 2 * r] = (run + j) | (min(16, c - j) << 16);
                runs[3 + 2 * r] = i;
            }
        run += c;
    }
    if (runs && tid == NT - 1) runs[0] = s_scan[tid] >> 16;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PPT; j++) {
        const int v = tid + NT * j;
        if (v < n) perm[cnt[pe[j]] + rank[j]] = v | (pe[j] << 16);  // the expert rides along: no ids load downstream
    }
}

mx_status launch_pair_order(const uint32_t *ids, int t, int top_k, int n_expert, int slots, int32_t *perm,
                            hipStream_t s, int32_t *runs) {
    if ((int64_t)t * slots > PAIR_ORDER_MAX || n_expert > SEL_MAX_E)
        return fail(MX_ERR_SHAPE, "pair order: t * slots <= %d and n_expert <= %d", PAIR_ORDER_MAX, SEL_MAX_E);
    hipLaunchKernelGGL(k_pair_order, dim3(1), dim3(PAIR_ORDER_THREADS), 0, s, ids, t, top_k, n_expert, slots, perm,
                       runs);
    MX_LAUNCH("k_pair_order");
    return MX_OK;
}

template <int DT, int NG>
static mx_status launch_gu_ng(const DecodeGateUpArgs &a, int slot0, int nslot, hipStream_t s, bool wide) {
    const unsigned tiles = (unsigned)((a.ff + WAVES * RW_GU - 1) / (WAVES * RW_GU));
    const dim3 grid(tiles, (unsigned)nslot, (unsigned)a.t);
    constexpr bool GM_OK = DT == kQ4_K || DT == kQ5_K;
    const int ni = ring_insts<DT, NG>(2, a.hidden, a.gu_row_bytes, Batch<NG>::NIT, false, wide);
    const size_t lds = (size_t)WAVES * RING_GU * ni * 1024;
    const Geo<DT> geo(a.hidden, false, wide);
    if (GM_OK && a.xstage_gm)
        hipLaunchKernelGGL((k_decode_gate_up<DT, NG, GM_OK>), grid, dim3(64 * WAVES), lds, s, a, ni, slot0, geo);
    else
        hipLaunchKernelGGL((k_decode_gate_up<DT, NG, false>), grid, dim3(64 * WAVES), lds, s, a, ni, slot0, geo);
    return MX_OK;
}

// the 64-group kernel's conditions: Q4_K / Q5_K, 64 groups per row, 16-byte-aligned
// rows and experts, and the group-major staged activation
template <int DT>
static bool gu64_ok(const DecodeGateUpArgs &a) {
    if constexpr (DT != kQ4_K) {  // (Q5_K's extra high-bit words spill at this occupancy)
        (void)a;
        return false;
    } else {
        auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        return GU64_R > 0 && Geo<DT>(a.hidden).G == 64 && a.gu_row_bytes == Row64<DT>::RB &&
               a.gu_expert_bytes % 16 == 0 && al(a.gate) && al(a.up) && a.xstage_gm &&
               (!a.sh_gate || (al(a.sh_gate) && al(a.sh_up)));
    }
}

template <int DT>
static mx_status launch_gu_dt(const DecodeGateUpArgs &a, int slot0, int nslot, hipStream_t s) {
    if constexpr (DT == kQ4_K) {  // (gu64_ok holds for Q4_K only)
        if (gu64_ok<DT>(a)) {
            const unsigned tiles = (unsigned)((a.ff + WAVES * GU64_R - 1) / (WAVES * GU64_R));
            // verify blocks (t > 1): GU64_TPB tiles per workgroup, the activation
            // slices and per-wave setup amortised over more rows (C2: 8 tiles
            // 369 -> 363 us; 16 and 24 slower); t = 1: GU64_TPB1 tiles, so the
            // in-block top-k and the activation loads run once per workgroup
            const bool verify = a.t > 1;
            const int tpb = verify ? GU64_TPB : GU64_TPB1;
            const dim3 grid((tiles + tpb - 1) / tpb, (unsigned)nslot, (unsigned)a.t);
            const size_t lds = (size_t)WAVES * 2 * Row64<DT>::RB + (a.sel_keys ? sizeof(SelSharedT<GU_SEL_E>) : 0);
            constexpr int R = GU64_R > 0 ? GU64_R : 1;
            if (verify)
                hipLaunchKernelGGL((k_decode_gate_up64<DT, R, GU64_TPB, 4, 0>), grid, dim3(64 * WAVES), lds, s, a, slot0,
                                   Geo<DT>(a.hidden));
            else
                hipLaunchKernelGGL((k_decode_gate_up64<DT, R, GU64_TPB1, MX_GU_WPE, DMA_NT>), grid, dim3(64 * WAVES), lds,
                                   s, a, slot0, Geo<DT>(a.hidden));
            return MX_OK;
        }
    }
    const bool wide = gu_wide<DT>(a.hidden, a.gu_row_bytes);
    const int ng = ng_variant(Geo<DT>(a.hidden, false, wide).NG);
#define MX_L(N) return launch_gu_ng<DT, N>(a, slot0, nslot, s, wide)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
    return MX_OK;
}

mx_status launch_decode_select(int top_k, const DecodeSelArgs &sel, hipStream_t s) {
    if (sel.n_sel == 0) return MX_OK;
    if (sel.n_expert > SEL_MAX_E || top_k > SEL_MAX_K)
        return fail(MX_ERR_SHAPE, "decode select: n_expert <= %d and top_k <= %d", SEL_MAX_E, SEL_MAX_K);
    hipLaunchKernelGGL(k_decode_select, dim3((unsigned)sel.n_sel), dim3(SEL_THREADS), sizeof(SelShared), s, top_k,
                       sel);
    MX_LAUNCH("k_decode_select");
    return MX_OK;
}

bool decode_gate_up_selects(int dtype, const DecodeGateUpArgs &a) {
    return dtype == kQ4_K && gu64_ok<kQ4_K>(a) && a.t == 1 && a.n_expert <= GU_SEL_E && a.top_k <= SEL_MAX_K &&
           !a.perm;
}

mx_status launch_decode_gate_up(int dtype, const DecodeGateUpArgs &a, int slot0, int nslot, hipStream_t s) {
    if (a.t == 0 || nslot == 0) return MX_OK;
    if ((int64_t)a.t > 65535 || nslot > 65535) return fail(MX_ERR_OVERFLOW, "decode gate/up: grid too large");
    if (a.hidden % 32) return fail(MX_ERR_BLOCK, "decode gate/up: hidden must be a multiple of 32");
    if (a.sh_gate && a.sh_row_bytes != a.gu_row_bytes)
        return fail(MX_ERR_SHAPE, "decode gate/up: shared expert rows must match the routed rows");
    if (a.perm && (slot0 != 0 || nslot != a.top_k + (a.sh_gate ? 1 : 0)))
        return fail(MX_ERR_SHAPE, "decode gate/up: an expert-ordered launch covers every slot");
    if (a.sel_keys && (!decode_gate_up_selects(dtype, a) || slot0 != 0))
        return fail(MX_ERR_SHAPE, "decode gate/up: the in-block top-k needs t == 1 and the 64-group kernel");
    switch (dtype) {
    case kQ4_K: MX_TRY(launch_gu_dt<kQ4_K>(a, slot0, nslot, s)); break;
    case kQ5_K: MX_TRY(launch_gu_dt<kQ5_K>(a, slot0, nslot, s)); break;
    case kQ6_K: MX_TRY(launch_gu_dt<kQ6_K>(a, slot0, nslot, s)); break;
    default: MX_TRY(launch_gu_dt<kQ8_0>(a, slot0, nslot, s)); break;
    }
    MX_LAUNCH("k_decode_gate_up");
    return MX_OK;
}

// ---- fused decode: down (one slot per block), then the combine kernel ---------------------
// grid (hidden / (WAVES_DN * rpw), slots, t), rpw = RW_DN * DN_TPB rows per wave (C2:
// 4 tiles per wave 362 -> 334 us, the act row staged once per workgroup for 4x the
// rows; 2 and 8 measured 343).  Each block writes its slot's down rows to part[tok, slot, :]; the
// combine kernel that follows on the stream (the kernel boundary orders the two)
// forms out[c] = residual[c] + ( sum_k w[k] * part[k][c] + shared[c] )
// (combine.metal:70-97, moe.rs:73-78, model.rs:351).  The shared expert is
// part's last slot when it has the routed quant types, else a.shared_out.
#ifndef MX_DN_WPE
#define MX_DN_WPE 1
#endif
template <int DT, int NG>
__global__ void __launch_bounds__(64 * WAVES_DN) __attribute__((amdgpu_waves_per_eu(MX_DN_WPE))) k_decode_down(DecodeDownArgs a, int ni, int rpw, Geo<DT> geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    const int tile = blockIdx.x;  // grid (row tiles, slots, t)
    int slot = blockIdx.y, tok = blockIdx.z, pe = -1;
    if (a.perm) {  // expert-ordered pairs: an expert's repeats run back to back (its rows in L2)
        const int v = a.perm[blockIdx.z * slots + blockIdx.y];
        tok = (v & 0xFFFF) / slots;
        slot = (v & 0xFFFF) % slots;
        pe = v >> 16;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
    const int r0 = (tile * WAVES_DN + wave) * rpw;  // rpw rows per wave, the act row staged once
    const float *xrow = a.act + ((int64_t)tok * slots + slot) * a.ff;
    uint8_t *ring = lds + align16(xstage_bytes(a.ff)) + wave * (RING_DN * ni * 1024);
    XPre xp;
    if (r0 >= a.hidden) {  // wave-uniform; every wave takes part in the staging barrier
        stage_pre(xrow, a.ff, xp);
        stage_post(xrow, a.ff, xp, lds);
        return;
    }
    const uint8_t *wp;
    int64_t rb;
    if (slot < a.top_k) {
        const uint32_t id = pe >= 0 ? (uint32_t)pe : a.ids[tok * a.top_k + slot];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        wp = a.down + (int64_t)e * a.d_expert_bytes;
        rb = a.d_row_bytes;
    } else {
        wp = a.sh_down;
        rb = a.sh_row_bytes;
    }
    const uint8_t *const w[1] = {wp};
    typename Q<DT>::X xs[NG];
    float *part = a.part + ((int64_t)tok * slots + slot) * a.hidden;
    stream_rows<DT, NG, BatchDn<NG>::NIT, 1, RING_DN>(w, rb, geo, xs, r0, min(r0 + rpw, a.hidden), ring, ni,
                                                     [&] { stage_pre(xrow, a.ff, xp); },
                                                     [&] {
                                                         stage_post(xrow, a.ff, xp, lds);
                                                         load_xs<DT, NG>(lds, a.ff, geo, xs);
                                                     },
                                                     [&](int row, const float (&s)[1]) { part[row] = s[0]; });
}

// ---- fused decode down, one workgroup per (token, row tile) holding every slot ---------
// grid (hidden / RW_DN, t), 64 * slots threads: wave s stages slot s's act row into
// its own LDS area and streams the slot's RW_DN down rows; the partial rows meet in
// LDS and threads 0 .. RW_DN - 1 combine them in slot order, with the arithmetic of
// k_decode_down's combine (combine.metal:70-97).  No partial rows in global
// memory, no arrival counters, no cross-block tail.
#ifndef MX_DN_SLOTS
#define MX_DN_SLOTS 1
#endif
#ifndef MX_DN_SLOTS_MAX_T
#define MX_DN_SLOTS_MAX_T 4  // above this, more and smaller blocks (k_decode_down) keep the CUs fuller
#endif
constexpr int DN_SLOTS_MAX = 12;  // 3 waves per SIMD: 168 VGPRs
// row-iterations per DMA batch (NG > 1): 2 -> 8-row batches of Q6_K at ff = 1536
#ifndef MX_NIT_DNS
#define MX_NIT_DNS 2
#endif
template <int NG> struct BatchDnSlots { static constexpr int NIT = NG == 1 ? BatchDn<1>::NIT : MX_NIT_DNS; };
// LDS per slot (wave): the staged act row, then the wave's ring in the same bytes
static_assert(RING_DN == 1, "k_decode_down_slots overlays its ring on the staged row: one batch in flight");
__host__ __device__ inline size_t dn_slot_area(int ff, int ni) {
    const size_t xs = align16(xstage_bytes(ff)), ring = (size_t)ni * 1024;
    return xs > ring ? xs : ring;
}
constexpr int XPRE_W = 4;  // act quarters per lane held in registers before the weight copies
template <int DT, int NG>
__global__ void __launch_bounds__(64 * DN_SLOTS_MAX) k_decode_down_slots(DecodeDownArgs a, int ni, Geo<DT> geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float s_part[DN_SLOTS_MAX][RW_DN];
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int tok = blockIdx.y;
    const int r0 = blockIdx.x * RW_DN, r1 = min(r0 + RW_DN, a.hidden);
    // the slot's staged row is read into registers before the first weight copy,
    // so the ring reuses its LDS (dn_slot_area)
    uint8_t *xs_lds = lds + (size_t)slot * dn_slot_area(a.ff, ni);
    uint8_t *ring = xs_lds;
    const float *xrow = a.act + ((int64_t)tok * slots + slot) * a.ff;
    XPreT<XPRE_W> xp;
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
    typename Q<DT>::X xs[NG];
    stream_rows<DT, NG, BatchDnSlots<NG>::NIT, 1, RING_DN>(w, rb, geo, xs, r0, r1, ring, ni,
                                                     [&] { stage_pre_t(xrow, a.ff, xp, lane, 64); },
                                                     [&] {
                                                         stage_post_t(xrow, a.ff, xp, xs_lds, lane, 64);
                                                         load_xs<DT, NG>(xs_lds, a.ff, geo, xs);
                                                         wait_lgkmcnt0();  // before the ring overwrites it
                                                     },
                                                     [&](int row, const float (&v)[1]) { s_part[slot][row - r0] = v[0]; });
    __syncthreads();
    const int r = threadIdx.x;
    if (r >= r1 - r0) return;
    const int c = r0 + r;
    const int64_t o = (int64_t)tok * a.hidden + c;
    const float sh = a.sh_down ? s_part[a.top_k][r] : a.shared_out ? a.shared_out[o] : 0.f;
    const float res = a.residual ? a.residual[o] : 0.f;
    const float *wt = a.w + tok * a.top_k;
    float v = 0.f;
    for (int s = 0; s < a.top_k; s++) v = v + s_part[s][r] * wt[s];
    if (a.sh_down || a.shared_out) v = v + sh;
    if (a.residual) v = res + v;
    a.out[o] = v;
}

// Q6_K down rows of the C1 shape (ff = 1536: 48 groups of 32 weights per row of
// 1260 bytes), compile-time: the slot-per-wave kernel's work and arithmetic (16
// lanes per row, 3 groups per lane), with every lane's field offsets computed
// once.  Rows are 4-byte aligned when the stacks are 16-byte aligned (1260 = 4 *
// 315), so a block's 2-byte phase is its index parity: lane constants, not
// per-row arithmetic.  Results are bit-identical to k_decode_down_slots.
// The 16-row tile runs in four 4-row batches through two LDS buffers per slot
// wave, so batch b + 1's copy is in flight while batch b is contracted (a form
// that copied 8-row batches into one buffer per wave and waited for each before
// contracting measured 17.05 against 15.4 us at C1).  The staged act row (4992
// bytes) is built in the second buffer while the first batch's copy runs, and
// read into registers before that buffer's first copy.
constexpr int DQ6_FF = 1536, DQ6_RB = 1260, DQ6_P = 16, DQ6_NG = 3, DQ6_RPI = 64 / DQ6_P;
#ifndef MX_DN_Q6
#define MX_DN_Q6 1
#endif
constexpr int DQ6R_BROWS = 4, DQ6R_CH = DQ6R_BROWS * DQ6_RB / 16, DQ6R_NI = (DQ6R_CH + 63) / 64;
static_assert(DQ6R_BROWS == DQ6_RPI, "one row per lane group per batch");
template <int AUX>  // cache policy of the weight copies (DMA_NT at t = 1)
__global__ void __launch_bounds__(64 * DN_SLOTS_MAX) k_decode_down_q6r(DecodeDownArgs a, Geo<kQ6_K> geo) {
    constexpr int DT = kQ6_K, NB = RW_DN / DQ6R_BROWS;
    // two separate LDS objects, so the compiler can tell a copy into one buffer
    // from the reads of the other
    __shared__ __attribute__((aligned(16))) uint8_t ring0[DN_SLOTS_MAX][DQ6R_NI * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[DN_SLOTS_MAX][DQ6R_NI * 1024];
    __shared__ float s_part[DN_SLOTS_MAX][RW_DN];
    static_assert((size_t)xstage_bytes(DQ6_FF) <= (size_t)DQ6R_NI * 1024, "the staged row fits one buffer");
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int sub = lane & (DQ6_P - 1), rsub = lane / DQ6_P;
    const int tok = blockIdx.y;
    const int r0 = blockIdx.x * RW_DN;
    const float *xrow = a.act + ((int64_t)tok * slots + slot) * a.ff;
    const uint8_t *wp;
    if (slot < a.top_k) {
        const uint32_t id = a.ids[tok * a.top_k + slot];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        wp = a.down + (int64_t)e * a.d_expert_bytes;
    } else {
        wp = a.sh_down;
    }
    wp += (int64_t)r0 * DQ6_RB;
    uint8_t *const b0 = ring0[slot], *const b1 = ring1[slot];
    // every lane copies (the last instruction's spare lanes repeat the batch's last
    // chunk into the buffer's unused tail): no branch around a copy, so the
    // compiler's copy counts stay exact and it adds no vmcnt(0) of its own
    auto issue = [&](int bi, uint8_t *dst) {
        const uint8_t *src = wp + bi * (DQ6R_BROWS * DQ6_RB);
#pragma unroll
        for (int q = 0; q < DQ6R_NI; q++) {
            const int ci = min(64 * q + lane, DQ6R_CH - 1);
            dma16<AUX>(src + (uint32_t)(16 * ci), dst + 1024 * q);
        }
        asm volatile("" ::: "memory");
    };
    XPreT<XPRE_W> xp;
    stage_pre_t(xrow, a.ff, xp, lane, 64);
    // the act loads have returned before the first copy is issued (ordinary loads
    // are not counted across LDS copies), so the copy overlaps the staging work
    wait_vmcnt(0);
#pragma unroll
    for (int i = 0; i < XPRE_W; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) asm volatile("" : "+v"(xp.v[i][j]));
    issue(0, b0);
    typename Q<DT>::X xs[DQ6_NG];
    stage_post_t(xrow, a.ff, xp, b1, lane, 64);
    load_xs<DT, DQ6_NG>(b1, a.ff, geo, xs);
    wait_lgkmcnt0();
    if (NB > 1) issue(1, b1);
    // this lane's field offsets inside a row (Q<kQ6_K>::load's, hoisted)
    uint32_t oa[DQ6_NG], ohq[DQ6_NG], osc[DQ6_NG], od[DQ6_NG], sh[DQ6_NG];
#pragma unroll
    for (int jg = 0; jg < DQ6_NG; jg++) {
        const int g = sub + DQ6_P * jg, b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint32_t mis = (uint32_t)(210 * b) & 2u, ab = (uint32_t)(210 * b) - mis;
        oa[jg] = ab + 64 * n + 8 * j;
        ohq[jg] = ab + 128 + 32 * n + 8 * j;
        osc[jg] = ab + 192 + 8 * n;
        od[jg] = (uint32_t)(210 * b) + 208;
        sh[jg] = mis << 3;
    }
#pragma unroll
    for (int bi = 0; bi < NB; bi++) {
        uint8_t *const buf = (bi & 1) ? b1 : b0;
        wait_vmcnt(bi + 1 < NB ? DQ6R_NI : 0);  // batch bi has landed (bi + 1 may be in flight)
        const uint8_t *rl = buf + rsub * DQ6_RB;
        float acc[1][1];
        {
            float v = 0.f;
#pragma unroll
            for (int jg = 0; jg < DQ6_NG; jg++) {
                typename Q<DT>::Raw r;
                Q<DT>::ld3(rl + oa[jg], r.a);
                Q<DT>::ld3(rl + oa[jg] + 32, r.b);
                Q<DT>::ld3(rl + ohq[jg], r.hq);
                Q<DT>::ld3(rl + osc[jg], r.sc);
                r.d = ld_u16(rl + od[jg]);
                r.sh = sh[jg];
                v += Q<DT>::dot(r, sub + DQ6_P * jg, xs[jg]);
            }
            acc[0][0] = v;
        }
        int which;
        bool leader;
        reduce_tuples<1, 1>(acc, DQ6_P, sub, which, leader);
        if (leader) s_part[slot][bi * DQ6R_BROWS + rsub] = acc[0][0];
        if (bi + 2 < NB) {
            wait_lgkmcnt0();  // every read of the buffer returned before it is overwritten
            issue(bi + 2, buf);
        }
    }
    __syncthreads();
    const int r = threadIdx.x;
    if (r >= RW_DN) return;
    const int c = r0 + r;
    const int64_t o = (int64_t)tok * a.hidden + c;
    const float shv = a.sh_down ? s_part[a.top_k][r] : a.shared_out ? a.shared_out[o] : 0.f;
    const float res = a.residual ? a.residual[o] : 0.f;
    const float *wt = a.w + tok * a.top_k;
    float vv = 0.f;
    for (int s2 = 0; s2 < a.top_k; s2++) vv = vv + s_part[s2][r] * wt[s2];
    if (a.sh_down || a.shared_out) vv = vv + shv;
    if (a.residual) vv = res + vv;
    a.out[o] = vv;
}

// Verify-block form of the compile-time Q6_K down rows (t > 4, the grid of
// k_decode_down: one workgroup per (row tile, slot, token), DQ6V_RPW rows per
// wave, the pair's act row staged once per workgroup): the field offsets of
// k_decode_down_q6r, hoisted out of the row loop, and its two-buffer ring of
// 4-row batches per wave.  Same per-row arithmetic as k_decode_down (part rows
// bit-identical).
constexpr int DQ6V_RPW = 64;
#ifndef MX_DN_Q6V
#define MX_DN_Q6V 1
#endif
__global__ void __launch_bounds__(64 * WAVES_DN) k_decode_down_q6v(DecodeDownArgs a, Geo<kQ6_K> geo) {
    constexpr int DT = kQ6_K, NB = DQ6V_RPW / DQ6R_BROWS;
    __shared__ __attribute__((aligned(16))) uint8_t ring0[WAVES_DN][DQ6R_NI * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t ring1[WAVES_DN][DQ6R_NI * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t stg[(xstage_bytes(DQ6_FF) + 15) & ~15];
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    int slot = blockIdx.y, tok = blockIdx.z, pe = -1;
    if (a.perm) {  // expert-ordered pairs (as k_decode_down)
        const int v = a.perm[blockIdx.z * slots + blockIdx.y];
        tok = (v & 0xFFFF) / slots;
        slot = (v & 0xFFFF) % slots;
        pe = v >> 16;
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int sub = lane & (DQ6_P - 1), rsub = lane / DQ6_P;
    const int r0 = (blockIdx.x * WAVES_DN + wave) * DQ6V_RPW;  // hidden % (WAVES_DN * DQ6V_RPW) == 0
    const float *xrow = a.act + ((int64_t)tok * slots + slot) * a.ff;
    const uint8_t *wp;
    if (slot < a.top_k) {
        const uint32_t id = pe >= 0 ? (uint32_t)pe : a.ids[tok * a.top_k + slot];
        const int e = id < (uint32_t)a.n_expert ? (int)id : a.n_expert - 1;
        wp = a.down + (int64_t)e * a.d_expert_bytes;
    } else {
        wp = a.sh_down;
    }
    wp += (int64_t)r0 * DQ6_RB;
    uint8_t *const b0 = ring0[wave], *const b1 = ring1[wave];
    // every lane copies every batch (spare lanes repeat the last chunk into the
    // buffer's tail; the batch after the last repeats the last batch): no branch
    // around a copy, so the compiler's counts stay exact
    auto issue = [&](int bi, uint8_t *dst) {
        const uint8_t *src = wp + min(bi, NB - 1) * (DQ6R_BROWS * DQ6_RB);
#pragma unroll
        for (int q = 0; q < DQ6R_NI; q++) {
            const int ci = min(64 * q + lane, DQ6R_CH - 1);
            dma16(src + (uint32_t)(16 * ci), dst + 1024 * q);
        }
        asm volatile("" ::: "memory");
    };
    XPre xp;
    stage_pre(xrow, a.ff, xp);
    // the act loads have returned before the first copies are issued (ordinary
    // loads are not counted across LDS copies), so the copies overlap the staging
    wait_vmcnt(0);
#pragma unroll
    for (int i = 0; i < XPRE; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) asm volatile("" : "+v"(xp.v[i][j]));
    issue(0, b0);
    issue(1, b1);
    stage_post_t(xrow, a.ff, xp, stg, (int)threadIdx.x, (int)blockDim.x);
    // a bare barrier after this wave's LDS writes: __syncthreads would also wait
    // for the weight copies just issued
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    typename Q<DT>::X xs[DQ6_NG];
    load_xs<DT, DQ6_NG>(stg, a.ff, geo, xs);
    uint32_t oa[DQ6_NG], ohq[DQ6_NG], osc[DQ6_NG], od[DQ6_NG], sh[DQ6_NG];
#pragma unroll
    for (int jg = 0; jg < DQ6_NG; jg++) {
        const int g = sub + DQ6_P * jg, b = g >> 3, gi = g & 7, n = gi >> 2, j = gi & 3;
        const uint32_t mis = (uint32_t)(210 * b) & 2u, ab = (uint32_t)(210 * b) - mis;
        oa[jg] = ab + 64 * n + 8 * j;
        ohq[jg] = ab + 128 + 32 * n + 8 * j;
        osc[jg] = ab + 192 + 8 * n;
        od[jg] = (uint32_t)(210 * b) + 208;
        sh[jg] = mis << 3;
    }
    float *part = a.part + ((int64_t)tok * slots + slot) * a.hidden + r0;
    auto batch = [&](int bi, uint8_t *buf) {
        wait_vmcnt(DQ6R_NI);  // batch bi has landed (the next copy is in flight)
        const uint8_t *rl = buf + rsub * DQ6_RB;
        float acc[1][1];
        float v = 0.f;
#pragma unroll
        for (int jg = 0; jg < DQ6_NG; jg++) {
            typename Q<DT>::Raw r;
            Q<DT>::ld3(rl + oa[jg], r.a);
            Q<DT>::ld3(rl + oa[jg] + 32, r.b);
            Q<DT>::ld3(rl + ohq[jg], r.hq);
            Q<DT>::ld3(rl + osc[jg], r.sc);
            r.d = ld_u16(rl + od[jg]);
            r.sh = sh[jg];
            v += Q<DT>::dot(r, sub + DQ6_P * jg, xs[jg]);
        }
        acc[0][0] = v;
        int which;
        bool leader;
        reduce_tuples<1, 1>(acc, DQ6_P, sub, which, leader);
        if (leader) part[bi * DQ6R_BROWS + rsub] = acc[0][0];
        wait_lgkmcnt0();  // every read of the buffer returned before it is overwritten
        issue(bi + 2, buf);
    };
#pragma unroll 1
    for (int bi = 0; bi < NB; bi += 2) {
        batch(bi, b0);
        batch(bi + 1, b1);
    }
    wait_vmcnt(0);  // no copy into this workgroup's LDS outlives it
}

static bool dn_q6_ok(const DecodeDownArgs &a) {
    if (MX_DN_Q6 == 0) return false;
    auto al = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const Geo<kQ6_K> g(DQ6_FF, DN_FULL);
    return a.ff == DQ6_FF && a.d_row_bytes == DQ6_RB && g.P == DQ6_P && g.NG == DQ6_NG && g.G == DQ6_P * DQ6_NG &&
           a.hidden % RW_DN == 0 && (size_t)xstage_bytes(DQ6_FF) <= (size_t)DQ6R_NI * 1024 &&
           a.d_expert_bytes % 16 == 0 && al(a.down) && (!a.sh_down || (a.sh_row_bytes == DQ6_RB && al(a.sh_down)));
}

// the slot waves (3 per SIMD: 168 VGPRs) hold this many activation groups without
// spilling to scratch; wider rows take k_decode_down and the combine
template <int DT> constexpr int dn_slots_max_ng() { return DT == kQ8_0 ? 4 : DT == kQ6_K ? 3 : 2; }
template <int DT, int NG>
static mx_status launch_dn_slots_ng(const DecodeDownArgs &a, hipStream_t s) {
    if constexpr (NG > dn_slots_max_ng<DT>()) {  // (not instantiated: dn_slots_fit refuses these)
        (void)a;
        (void)s;
        return fail(MX_ERR_SHAPE, "decode down: %d activation groups per lane exceed the slot kernel", NG);
    } else {
        const int ni = ring_insts<DT, NG>(1, a.ff, a.d_row_bytes, BatchDnSlots<NG>::NIT, DN_FULL);
        if (ni > DMA_MAX_INSTS) return fail(MX_ERR_SHAPE, "decode down: rows too long for the LDS ring");
        const int slots = a.top_k + (a.sh_down ? 1 : 0);
        const size_t lds = (size_t)slots * dn_slot_area(a.ff, ni);
        const dim3 grid((unsigned)((a.hidden + RW_DN - 1) / RW_DN), (unsigned)a.t);
        hipLaunchKernelGGL((k_decode_down_slots<DT, NG>), grid, dim3(64 * slots), lds, s, a, ni, Geo<DT>(a.ff, DN_FULL));
        return MX_OK;
    }
}
// LDS bytes of the slot-per-wave kernel (SIZE_MAX: its DMA batch does not fit)
template <int DT, int NG>
static size_t dn_slots_lds(const DecodeDownArgs &a) {
    const int ni = ring_insts<DT, NG>(1, a.ff, a.d_row_bytes, BatchDnSlots<NG>::NIT, DN_FULL);
    if (ni > DMA_MAX_INSTS) return SIZE_MAX;
    const int slots = a.top_k + (a.sh_down ? 1 : 0);
    return (size_t)slots * dn_slot_area(a.ff, ni);
}
// true when the slot-per-wave kernel takes this launch
template <int DT>
static bool dn_slots_fit(const DecodeDownArgs &a) {
    if (!MX_DN_SLOTS || a.t > MX_DN_SLOTS_MAX_T) return false;
    if (a.top_k + (a.sh_down ? 1 : 0) > DN_SLOTS_MAX) return false;
    const int ng = ng_variant(Geo<DT>(a.ff, DN_FULL).NG);
    if (ng > dn_slots_max_ng<DT>()) return false;
    size_t lds = SIZE_MAX;
    [&] {
#define MX_L(N) { lds = dn_slots_lds<DT, N>(a); return; }
        MX_NG_SWITCH(ng, MX_L)
#undef MX_L
    }();
    return lds <= 160 * 1024 - sizeof(float) * DN_SLOTS_MAX * RW_DN;
}
template <int DT>
static mx_status launch_dn_slots_dt(const DecodeDownArgs &a, hipStream_t s) {
    if constexpr (DT == kQ6_K) {
        if (dn_q6_ok(a)) {
            const int slots = a.top_k + (a.sh_down ? 1 : 0);
            const dim3 grid((unsigned)(a.hidden / RW_DN), (unsigned)a.t);
            if (a.t == 1)
                hipLaunchKernelGGL(k_decode_down_q6r<DMA_NT>, grid, dim3(64 * slots), 0, s, a,
                                   Geo<kQ6_K>(DQ6_FF, DN_FULL));
            else
                hipLaunchKernelGGL(k_decode_down_q6r<0>, grid, dim3(64 * slots), 0, s, a, Geo<kQ6_K>(DQ6_FF, DN_FULL));
            return MX_OK;
        }
    }
    const int ng = ng_variant(Geo<DT>(a.ff, DN_FULL).NG);
#define MX_L(N) return launch_dn_slots_ng<DT, N>(a, s)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
    return MX_OK;
}

template <int DT, int NG>
static mx_status launch_dn_ng(const DecodeDownArgs &a, dim3 grid, hipStream_t s) {
    const int ni = ring_insts<DT, NG>(1, a.ff, a.d_row_bytes, BatchDn<NG>::NIT, DN_FULL);
    if (ni > DMA_MAX_INSTS) return fail(MX_ERR_SHAPE, "decode down: rows too long for the LDS ring");
    const size_t lds = align16(xstage_bytes(a.ff)) + (size_t)WAVES_DN * RING_DN * ni * 1024;
    if (lds > 160 * 1024) return fail(MX_ERR_SHAPE, "decode down: expert_ff = %d needs %zu bytes of LDS", a.ff, lds);
    // RW_DN * DN_TPB rows per wave: each workgroup stages its act row once for that many
    const int rpw = RW_DN * DN_TPB;
    const dim3 g((unsigned)((a.hidden + WAVES_DN * rpw - 1) / (WAVES_DN * rpw)), grid.y, grid.z);
    hipLaunchKernelGGL((k_decode_down<DT, NG>), g, dim3(64 * WAVES_DN), lds, s, a, ni, rpw, Geo<DT>(a.ff, DN_FULL));
    return MX_OK;
}

template <int DT>
static mx_status launch_dn_dt(const DecodeDownArgs &a, dim3 grid, hipStream_t s) {
    const int ng = ng_variant(Geo<DT>(a.ff, DN_FULL).NG);
#define MX_L(N) return launch_dn_ng<DT, N>(a, grid, s)
    MX_NG_SWITCH(ng, MX_L)
#undef MX_L
    return MX_OK;
}

mx_status launch_decode_down(int dtype, const DecodeDownArgs &a, hipStream_t s) {
    const unsigned tiles = (unsigned)((a.hidden + WAVES_DN * RW_DN - 1) / (WAVES_DN * RW_DN));
    const unsigned slots = (unsigned)(a.top_k + (a.sh_down ? 1 : 0));
    const dim3 grid(tiles, slots, (unsigned)a.t);
    if (grid.x == 0 || a.t == 0) return MX_OK;
    if (a.ff % 32) return fail(MX_ERR_BLOCK, "decode down: expert_ff must be a multiple of 32");
    if (a.sh_down && a.sh_row_bytes != a.d_row_bytes)
        return fail(MX_ERR_SHAPE, "decode down: shared expert rows must match the routed rows");
    bool slots_kernel = false;
    switch (dtype) {
    case kQ4_K: slots_kernel = dn_slots_fit<kQ4_K>(a); break;
    case kQ5_K: slots_kernel = dn_slots_fit<kQ5_K>(a); break;
    case kQ6_K: slots_kernel = dn_slots_fit<kQ6_K>(a); break;
    default: slots_kernel = dn_slots_fit<kQ8_0>(a); break;
    }
    if (slots_kernel) {
        switch (dtype) {
        case kQ4_K: MX_TRY(launch_dn_slots_dt<kQ4_K>(a, s)); break;
        case kQ5_K: MX_TRY(launch_dn_slots_dt<kQ5_K>(a, s)); break;
        case kQ6_K: MX_TRY(launch_dn_slots_dt<kQ6_K>(a, s)); break;
        default: MX_TRY(launch_dn_slots_dt<kQ8_0>(a, s)); break;
        }
        MX_LAUNCH("k_decode_down_slots");
        return MX_OK;
    }
    if (dtype == kQ6_K && MX_DN_Q6V && dn_q6_ok(a) && a.hidden % (WAVES_DN * DQ6V_RPW) == 0) {
        const dim3 g((unsigned)(a.hidden / (WAVES_DN * DQ6V_RPW)), grid.y, grid.z);
        hipLaunchKernelGGL(k_decode_down_q6v, g, dim3(64 * WAVES_DN), 0, s, a, Geo<kQ6_K>(DQ6_FF, DN_FULL));
        MX_LAUNCH("k_decode_down_q6v");
        return launch_combine_prefill(a.part, a.w, a.residual, a.t, a.top_k, a.sh_down ? 1 : 0, a.hidden, a.out, s,
                                      a.shared_out);
    }
    switch (dtype) {
    case kQ4_K: MX_TRY(launch_dn_dt<kQ4_K>(a, grid, s)); break;
    case kQ5_K: MX_TRY(launch_dn_dt<kQ5_K>(a, grid, s)); break;
    case kQ6_K: MX_TRY(launch_dn_dt<kQ6_K>(a, grid, s)); break;
    default: MX_TRY(launch_dn_dt<kQ8_0>(a, grid, s)); break;
    }
    MX_LAUNCH("k_decode_down");
    return launch_combine_prefill(a.part, a.w, a.residual, a.t, a.top_k, a.sh_down ? 1 : 0, a.hidden, a.out, s,
                                  a.shared_out);
}

}  // namespace mx
