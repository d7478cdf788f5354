// Grouped expert GEMM of the fused prefill / verify path on MFMA.
//
// Replaces the kernel_mul_mm_id_* dispatches of the reference's prefill block
// (mm_id.metal:492-647, driven from moe.rs:242-323).  One workgroup computes a
// 128-pair x 256-column tile of one expert:
//
//  * A (activations) are f16 rows, each scaled by its own power of two so any
//    f32 magnitude lands in [2^14, 2^15) (the scale is applied back to the f32
//    result, so the only rounding is the f16 rounding of x itself).  The tile's
//    rows are gathered by pair (token = pair / top_k, or the bucket position)
//    and copied straight into LDS with global_load_lds, 128 K-values per
//    stage, double-buffered.  16-byte chunks are XOR-swizzled by row so the
//    MFMA operand reads (16 consecutive rows, same chunk) hit distinct banks.
//  * B (weights) are read from the raw GGUF blocks into registers, one stage
//    ahead, and dequantised in registers directly into the MFMA B-operand
//    layout: f32 dequantisation of the reference's formula, then one
//    round-to-nearest f16 pack (the reference dequantises into half tiles).
//    Each wave owns 64 output columns, so no weight is dequantised twice in a
//    workgroup.
//  * v_mfma_f32_32x32x16_f16, f32 accumulation: each wave holds 4 (pairs) x 2
//    (columns) 32x32 accumulators.
//
// The K order inside a 128-value stage is permuted (identically for A and B):
// MFMA step (p, h) gives lane half kh the 8 values at
// 32p + 16kh + 8h + [0, 8) of the stage, which makes every lane's weight bytes
// contiguous 16-byte pieces of the block.
//
// Epilogues: SwiGLU (wave columns = 32 gate rows and the same 32 up rows, so
// act = silu(g) * u is lane-local; act is written f32 at the pair's bucket
// position) or plain (f32 rows scattered to the pair's output row).
//
// Work items are (m-tile, n-tile) pairs, m-tile fastest; blocks are dealt to
// the 8 XCDs round-robin by the hardware, so block b takes item
// (b % 8) * per + b / 8: each XCD works through a contiguous run of items, and
// the m-tiles of one expert that share a weight slice run together on one L2.
#include "mx_launch.h"
#include "mx_dma.h"

namespace mx {

namespace {

constexpr int KS = 128;                // K per stage
constexpr int ROWB = KS * 2;           // LDS bytes per A row and stage
constexpr int STAGE_BYTES = GM_BM * ROWB;
constexpr int BN = 256;  // weight rows (output columns) per block

// Weight rows per wave = 32 * NB.  NB = 2 (4 waves per block) reuses every A
// fragment read from LDS for two MFMAs and is what the SwiGLU epilogue needs
// (32 gate + the same 32 up rows in one wave); NB = 1 (8 waves) halves the
// accumulators and weight registers per wave, which lets the Q6_K plain GEMM
// run two waves per SIMD without spilling.
#ifndef MX_GEMM_NB_PLAIN
#define MX_GEMM_NB_PLAIN 1
#endif
// waves of the NB = 2 (SwiGLU, Q4_K) tiles: 4 (256 weight rows, two workgroups
// per CU) or 8 (512 rows, one workgroup per CU at the same 2 waves per SIMD:
// each A tile is gathered once for twice the columns)
#ifndef MX_GEMM_WAVES2
#define MX_GEMM_WAVES2 8
#endif
template <int DT, bool SWIGLU> struct GemmNb {
    static constexpr int nb = (SWIGLU || DT == kQ4_K) ? 2 : MX_GEMM_NB_PLAIN;
    // (Q6_K / Q8_0 SwiGLU keep 4 waves: at 8 a workgroup caps them at 256 VGPRs)
    static constexpr int waves = nb == 2 ? ((DT == kQ4_K || DT == kQ5_K) ? MX_GEMM_WAVES2 : 4) : BN / (32 * nb);
    static constexpr int bn = waves * 32 * nb;  // weight rows per workgroup
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {  // 4-byte aligned p
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes from a 2-byte aligned address: an aligned 16-byte load plus, when p
// is not 4-byte aligned, the dword after it (funnel-shifted in `fix16`)
struct Raw16 {
    uint4 v;
    uint32_t tail;
    uint32_t sh;  // 0 or 16
};
__device__ __forceinline__ Raw16 ld16_a2(const uint8_t *p) {
    Raw16 r;
    const uintptr_t mis = reinterpret_cast<uintptr_t>(p) & 3;
    const uint8_t *q = p - mis;
    r.v = ld16(q);
    r.tail = mis ? *reinterpret_cast<const uint32_t *>(q + 16) : 0u;
    r.sh = (uint32_t)mis * 8;
    return r;
}
__device__ __forceinline__ uint4 fix16(const Raw16 &r) {
    return make_uint4(__builtin_amdgcn_alignbit(r.v.y, r.v.x, r.sh), __builtin_amdgcn_alignbit(r.v.z, r.v.y, r.sh),
                      __builtin_amdgcn_alignbit(r.v.w, r.v.z, r.sh), __builtin_amdgcn_alignbit(r.tail, r.v.w, r.sh));
}

__device__ __forceinline__ half8_t pack8(const float (&f)[8]) {
    half8_t h;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const half2_t p = __builtin_convertvector((float2_t){f[2 * i], f[2 * i + 1]}, half2_t);
        h[2 * i] = p[0];
        h[2 * i + 1] = p[1];
    }
    return h;
}

// 4 unsigned bytes of w -> floats (v_cvt_f32_ubyte0..3)
__device__ __forceinline__ void ubytes(uint32_t w, float *f) {
#pragma unroll
    for (int b = 0; b < 4; b++) f[b] = (float)((w >> (8 * b)) & 0xFFu);
}

// Packed-f16 dequantisation (MX_GEMM_PKDQ).  Bytes b < 1024 of two dwords become
// the f16 numbers 1024 + b by placing them under the exponent byte 0x64
// (v_perm_b32); the rest is v_pk_*_f16 arithmetic on small integers, exact
// except where noted:
//   K-quants with min (Q4_K, Q5_K): t = fma(1024 + q, sc, -1024 sc) = sc * q
//     (exact: |sc * q| <= 63 * 31), y = fl16(fma(t, d, -fl16(dmin * m)))
//   Q6_K: t = ((1024 + q) - 1056) * sc = sc * (q - 32) (exact while <= 2048 in
//     magnitude), y = fl16(t * d)
// d and dmin are the blocks' own f16 values, so against the f32 form (one f16
// rounding of the f32 value) only fl16(dmin * m) adds an error.  About 1.5
// VALU per weight instead of 3.
#ifndef MX_GEMM_PKDQ
#define MX_GEMM_PKDQ 1
#endif
__device__ __forceinline__ half2_t pk_bytes(uint32_t w, uint32_t sel) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, sel));
}
__device__ __forceinline__ void pk_bytes8(uint32_t w0, uint32_t w1, half2_t (&x)[4]) {
    x[0] = pk_bytes(w0, 0x04010400u);  // bytes 0, 1
    x[1] = pk_bytes(w0, 0x04030402u);  // bytes 2, 3
    x[2] = pk_bytes(w1, 0x04010400u);
    x[3] = pk_bytes(w1, 0x04030402u);
}
__device__ __forceinline__ half8_t pk_join(const half2_t (&y)[4]) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[2 * i] = y[i][0];
        r[2 * i + 1] = y[i][1];
    }
    return r;
}
// sc2 = (sc, sc), d2 = (d, d), nm2 = -fl16(dmin * m) twice
__device__ __forceinline__ half8_t dq8_kmin(uint32_t w0, uint32_t w1, half2_t sc2, half2_t d2, half2_t nm2) {
    half2_t x[4], y[4];
    pk_bytes8(w0, w1, x);
    const half2_t nb = sc2 * half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};  // exact
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = __builtin_elementwise_fma(__builtin_elementwise_fma(x[i], sc2, nb), d2, nm2);
    return pk_join(y);
}
__device__ __forceinline__ half8_t dq8_q6(uint32_t w0, uint32_t w1, half2_t sc2, half2_t d2) {
    half2_t x[4], y[4];
    pk_bytes8(w0, w1, x);
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = ((x[i] + half2_t{(_Float16)-1056.0f, (_Float16)-1056.0f}) * sc2) * d2;
    return pk_join(y);
}
__device__ __forceinline__ half2_t h2splat(float v) {
    const _Float16 h = (_Float16)v;
    return half2_t{h, h};
}
__device__ __forceinline__ half2_t h2bits(uint32_t bits16) {
    return __builtin_bit_cast(half2_t, (bits16 & 0xFFFFu) * 0x10001u);
}

// ---- per-type weight registers: one stage, one weight row, one lane half --------------
template <int DT> struct WB;

// Q4_K: stage = half `par` of super-block ks / 2; 64-value chunks i = 2 par + c.
// Lane half kh holds qs bytes [32 i + 16 kh, +16) of both chunks; step p = 2c + nib
// uses the low (nib 0) or high nibbles, sub-block 2 i + nib (mm_id.metal:95-113).
template <> struct WB<kQ4_K> {
    static constexpr int kMinLoads = 3;  // memory instructions load() always issues: header + 2 quant pieces
    uint4 h, q[2];
    __device__ __forceinline__ void load(const uint8_t *base, __amdgpu_buffer_rsrc_t rs, uint32_t row, int ks, int kh) {
        const uint8_t *blk = base + (row + (uint32_t)(ks >> 1) * 144u);
        h = ld16(blk);
        const uint8_t *qs = blk + 16 + 64 * (ks & 1) + 16 * kh;
        q[0] = ld16(qs);
        q[1] = ld16(qs + 32);
    }
#if MX_GEMM_PKDQ
    half2_t scm[4], d2;  // (sc, -fl16(dmin * m)) of each sub-block, packed
#else
    float d[4], m[4];
#endif
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
        [[maybe_unused]] const float dd = h2f((uint16_t)(h.x & 0xFFFFu));
        const float dmin = h2f((uint16_t)(h.x >> 16));
#if MX_GEMM_PKDQ
        d2 = h2bits(h.x);
#endif
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mn;
            q4k_scale_min(4 * PAR + p, h.y, h.z, h.w, sc, mn);
#if MX_GEMM_PKDQ
            scm[p] = half2_t{(_Float16)(float)sc, (_Float16)(-(dmin * (float)mn))};
#else
            d[p] = dd * (float)sc;
            m[p] = dmin * (float)mn;
#endif
        }
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &v = q[p >> 1];
        const int sh = 4 * (p & 1);
        const uint32_t w0 = ((hh ? v.z : v.x) >> sh) & 0x0F0F0F0Fu;
        const uint32_t w1 = ((hh ? v.w : v.y) >> sh) & 0x0F0F0F0Fu;
#if MX_GEMM_PKDQ
        return dq8_kmin(w0, w1, half2_t{scm[p][0], scm[p][0]}, d2, half2_t{scm[p][1], scm[p][1]});
#else
        float f[8];
        ubytes(w0, f);
        ubytes(w1, f + 4);
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = __builtin_fmaf(d[p], f[i], -m[p]);
        return pack8(f);
#endif
    }
};

// Q5_K: Q4_K's stage layout (qs at byte 48) plus lane half kh's 16 bytes of qh;
// step p of half `par` adds bit 4 par + p of qh[l] as the fifth bit (mm_id.metal:113-134).
template <> struct WB<kQ5_K> {
    static constexpr int kMinLoads = 4;  // memory instructions load() always issues: header + qh + 2 quant pieces
    uint4 h, q[2], qh;
    __device__ __forceinline__ void load(const uint8_t *base, __amdgpu_buffer_rsrc_t rs, uint32_t row, int ks, int kh) {
        const uint8_t *blk = base + (row + (uint32_t)(ks >> 1) * 176u);
        h = ld16(blk);
        qh = ld16(blk + 16 + 16 * kh);
        const uint8_t *qs = blk + 48 + 64 * (ks & 1) + 16 * kh;
        q[0] = ld16(qs);
        q[1] = ld16(qs + 32);
    }
#if MX_GEMM_PKDQ
    half2_t scm[4], d2;  // (sc, -fl16(dmin * m)) of each sub-block, packed
#else
    float d[4], m[4];
#endif
    int hsh;
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
        [[maybe_unused]] const float dd = h2f((uint16_t)(h.x & 0xFFFFu));
        const float dmin = h2f((uint16_t)(h.x >> 16));
#if MX_GEMM_PKDQ
        d2 = h2bits(h.x);
#endif
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mn;
            q4k_scale_min(4 * PAR + p, h.y, h.z, h.w, sc, mn);
#if MX_GEMM_PKDQ
            scm[p] = half2_t{(_Float16)(float)sc, (_Float16)(-(dmin * (float)mn))};
#else
            d[p] = dd * (float)sc;
            m[p] = dmin * (float)mn;
#endif
        }
        hsh = 4 * PAR;
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &v = q[p >> 1];
        const int sh = 4 * (p & 1);
        const uint32_t hb = hsh + p;
        const uint32_t w0 = (((hh ? v.z : v.x) >> sh) & 0x0F0F0F0Fu) | ((((hh ? qh.z : qh.x) >> hb) & 0x01010101u) << 4);
        const uint32_t w1 = (((hh ? v.w : v.y) >> sh) & 0x0F0F0F0Fu) | ((((hh ? qh.w : qh.y) >> hb) & 0x01010101u) << 4);
#if MX_GEMM_PKDQ
        return dq8_kmin(w0, w1, half2_t{scm[p][0], scm[p][0]}, d2, half2_t{scm[p][1], scm[p][1]});
#else
        float f[8];
        ubytes(w0, f);
        ubytes(w1, f + 4);
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = __builtin_fmaf(d[p], f[i], -m[p]);
        return pack8(f);
#endif
    }
};

// Q6_K: stage = half n = par of super-block ks / 2 (128 values).  Lane half kh
// holds ql[64n + 16kh, +16), ql[64n + 32 + 16kh, +16), qh[32n + 16kh, +16);
// step p takes the 4-bit part from the low (p even) / high (p odd) ql piece,
// nibble p / 2, and bits 2p of qh; scale 8n + 2p + kh (mm_id.metal:115-135).
template <> struct WB<kQ6_K> {
    static constexpr int kMinLoads = 11;  // buffer loads load() issues: 3 x (piece + next dword) + 3 scale words + d
    // raw bytes, realigned in place by prep(): ql low piece, ql high piece, qh
    uint4 lo, hi, qh;
    uint32_t lo_t, hi_t, qh_t;  // the dword after each piece (2-byte aligned blocks)
    uint32_t sc0, sc1, sc2w, dsh;  // 3 dwords covering scales[8n .. 8n+7]; d and the shift
    // Buffer loads through the expert's resource: every word is loaded whatever
    // the block's 4-byte phase (no branches, so exact wait counts), and the
    // words past the end of the expert's rows read 0 instead of faulting.
    __device__ __forceinline__ void load(const uint8_t *base, __amdgpu_buffer_rsrc_t rs, uint32_t row, int ks, int kh) {
        const uint32_t blk = row + (uint32_t)(ks >> 1) * 210u;  // byte offset in the expert
        const int n = ks & 1;
        auto piece = [&](uint32_t off, uint4 &v, uint32_t &t) {
            const uint32_t al = off & ~3u;
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)al, 0, 0);
            v = make_uint4(q[0], q[1], q[2], q[3]);
            t = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(al + 16), 0, 0);
        };
        piece(blk + 64 * n + 16 * kh, lo, lo_t);
        piece(blk + 64 * n + 32 + 16 * kh, hi, hi_t);
        piece(blk + 128 + 32 * n + 16 * kh, qh, qh_t);
        const uint32_t sa = (blk + 192 + 8 * n) & ~3u;
        sc0 = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)sa, 0, 0);
        sc1 = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(sa + 4), 0, 0);
        sc2w = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(sa + 8), 0, 0);
        // every field of a block shares its 4-byte phase
        const uint32_t sh = (uint32_t)((reinterpret_cast<uintptr_t>(base) + blk) & 2) * 8;
        dsh = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(blk + 208), 0, 0) | (sh << 16);
    }
#if MX_GEMM_PKDQ
    half2_t sc2[4], d2;
#else
    float ds[4];
#endif
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        const float d = h2f((uint16_t)(dsh & 0xFFFFu));
        const uint32_t sh = dsh >> 16;
#if MX_GEMM_PKDQ
        d2 = h2bits(dsh);
        (void)d;
#endif
        const uint32_t s0 = __builtin_amdgcn_alignbit(sc1, sc0, sh), s1 = __builtin_amdgcn_alignbit(sc2w, sc1, sh);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int j = 2 * p + kh;  // byte j of the stage's 8 scales
            const uint32_t word = j < 4 ? s0 : s1;
            const int8_t s8 = (int8_t)((word >> (8 * (j & 3))) & 0xFFu);
#if MX_GEMM_PKDQ
            sc2[p] = h2splat((float)s8);
#else
            ds[p] = d * (float)s8;
#endif
        }
        lo = fix16(Raw16{lo, lo_t, sh});
        hi = fix16(Raw16{hi, hi_t, sh});
        qh = fix16(Raw16{qh, qh_t, sh});
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &ql = (p & 1) ? hi : lo;
        const int shl = 4 * (p >> 1), shh = 2 * p;
        const uint32_t a0 = ((hh ? ql.z : ql.x) >> shl) & 0x0F0F0F0Fu;
        const uint32_t a1 = ((hh ? ql.w : ql.y) >> shl) & 0x0F0F0F0Fu;
        const uint32_t b0 = (((hh ? qh.z : qh.x) >> shh) & 0x03030303u) << 4;
        const uint32_t b1 = (((hh ? qh.w : qh.y) >> shh) & 0x03030303u) << 4;
#if MX_GEMM_PKDQ
        return dq8_q6(a0 | b0, a1 | b1, sc2[p], d2);
#else
        float f[8];
        ubytes(a0 | b0, f);
        ubytes(a1 | b1, f + 4);
        const float off = -32.0f * ds[p];
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = __builtin_fmaf(ds[p], f[i], off);
        return pack8(f);
#endif
    }
};

// Q8_0: stage = blocks 4 ks + p; lane half kh holds quants [16 kh, +16) of each.
template <> struct WB<kQ8_0> {
    static constexpr int kMinLoads = 8;  // memory instructions load() always issues: 4 x (piece + d)
    Raw16 q[4];
    uint16_t dh[4];
    __device__ __forceinline__ void load(const uint8_t *base, __amdgpu_buffer_rsrc_t rs, uint32_t row, int ks, int kh) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint8_t *blk = base + (row + (uint32_t)(4 * ks + p) * 34u);
            q[p] = ld16_a2(blk + 2 + 16 * kh);
            dh[p] = ld_u16(blk);
        }
    }
    float d[4];
    uint4 v[4];
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            d[p] = h2f(dh[p]);
            v[p] = fix16(q[p]);
        }
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint32_t w0 = hh ? v[p].z : v[p].x, w1 = hh ? v[p].w : v[p].y;
        float f[8];
#pragma unroll
        for (int b = 0; b < 4; b++) {
            f[b] = (float)((int32_t)(w0 << (24 - 8 * b)) >> 24);
            f[4 + b] = (float)((int32_t)(w1 << (24 - 8 * b)) >> 24);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = d[p] * f[i];
        return pack8(f);
    }
};

#ifndef MX_GEMM_PIN_W
#define MX_GEMM_PIN_W 1
#endif
// leave the next stage's weight loads outstanding across the stage barrier
#ifndef MX_GEMM_WSLACK
#define MX_GEMM_WSLACK 1
#endif

// Makes the compiler wait for every register of `v` here (an empty asm that
// reads them).  Placed before a stage's A copies, the wait then covers weight
// loads only: the compiler's counters cannot order weight loads against LDS
// copies issued after them and would otherwise wait for everything.
// The operands are in-out, so nothing computed from `v` can be hoisted above
// this point either (the compiler would otherwise start the next stage's prep
// inside this stage and wait for the loads just issued).
template <class T> __device__ __forceinline__ void touch_regs(T &v) {
    static_assert(sizeof(T) % 4 == 0, "touch_regs: whole dwords");
    uint32_t *w = reinterpret_cast<uint32_t *>(&v);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 4); i++) asm volatile("" : "+v"(w[i]));
}

struct Tile {
    int e, pos0, mrows, nt;
};

// decodes this block's work item; false: nothing to do (block-uniform)
__device__ __forceinline__ bool tile_of(const GemmArgs &a, int nt_count, Tile &t) {
    const MapLayout L(a.n_map_expert, a.t, a.top_k);
    const int n_mt = a.map[L.n_tiles];
    const int n_items = n_mt * nt_count;
    const int per = (n_items + 7) / 8;
    const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
    if (local >= per) return false;
    const int item = xcd * per + local;
    if (item >= n_items) return false;
    t.nt = item / n_mt;
    const int word = a.map[L.tiles + item % n_mt];
    t.e = word >> 16;
    const int mt = word & 0xFFFF;
    const int cnt = a.map[L.tpe + t.e];
    t.mrows = min(GM_BM, cnt - mt * GM_BM);
    t.pos0 = a.map[L.off + t.e] + mt * GM_BM;
    return true;
}

// waves per SIMD the register allocation must allow, per weight type
#ifndef MX_GEMM_WPE_Q4K
#define MX_GEMM_WPE_Q4K 2
#endif
#ifndef MX_GEMM_WPE_Q6K
#define MX_GEMM_WPE_Q6K 1
#endif
template <int DT> struct GemmWpe {
    static constexpr int v = (DT == kQ4_K || DT == kQ5_K) ? MX_GEMM_WPE_Q4K : DT == kQ6_K ? MX_GEMM_WPE_Q6K : 1;
};

template <int DT, bool SWIGLU>
__global__ void __launch_bounds__((64 * GemmNb<DT, SWIGLU>::waves))
    __attribute__((amdgpu_waves_per_eu(GemmWpe<DT>::v))) k_gemm(GemmArgs a) {
    constexpr int NB = GemmNb<DT, SWIGLU>::nb;
    constexpr int NWAVE = GemmNb<DT, SWIGLU>::waves;
    constexpr int DMA_PER_WAVE = STAGE_BYTES / 1024 / NWAVE;
    // two separate LDS objects (not one 2-D array): the compiler can then tell
    // that a copy into one buffer does not feed reads of the other, and does
    // not wait for the next stage's copies before this stage's reads
    __shared__ __attribute__((aligned(1024))) uint8_t sA0[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t sA1[STAGE_BYTES];
    __shared__ uint32_t s_src[GM_BM];  // byte offset of the A row from the tile's first row
    __shared__ float s_scale[GM_BM];
    __shared__ int s_out[GM_BM];      // output row
    constexpr int NCOL = SWIGLU ? GemmNb<DT, SWIGLU>::bn / 2 : GemmNb<DT, SWIGLU>::bn;
    const int nt_count = (a.n_out + NCOL - 1) / NCOL;
    Tile tl;
    if (!tile_of(a, nt_count, tl)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, kh = lane >> 5;
    {
        const MapLayout L(a.n_map_expert, a.t, a.top_k);
        if (tid < GM_BM) {
            const int r = min(tid, tl.mrows - 1);  // rows past the tile repeat its last row
            const int pos = tl.pos0 + r;
            const int pair = a.map[L.list + pos];
            const int64_t arow = a.a_by_token ? pair / a.top_k : pos;
            // rows ascend within a tile (tokens ascend within a bucket), so the
            // offsets from the first row stay below (t or GM_BM) * k * 2 bytes
            const int64_t arow0 = a.a_by_token ? a.map[L.list + tl.pos0] / a.top_k : tl.pos0;
            s_src[tid] = (uint32_t)((arow - arow0) * a.k * 2);
            s_scale[tid] = a.a_scale[arow];
            s_out[tid] = SWIGLU ? pos : pair / a.top_k * a.out_stride + pair % a.top_k + a.out_add;
        }
    }
    __syncthreads();

    // this lane's two weight rows (one per 32-column MFMA block)
    const bool shared = tl.e >= a.n_expert;
    const int64_t rb = shared ? a.sh_row_bytes : a.row_bytes;
    const uint8_t *wbase[NB];  // wave-uniform expert base
    __amdgpu_buffer_rsrc_t wres[NB];  // the expert's rows as a buffer (range-checked loads)
    uint32_t wrow[NB];         // this lane's row offset from it (the launcher checks it fits)
    int col[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int m = SWIGLU ? nb : 0;
        const uint8_t *base = shared ? a.w_sh[m] : a.w[m] + (int64_t)tl.e * a.expert_bytes;
        col[nb] = SWIGLU ? tl.nt * NCOL + wave * 32 + j : tl.nt * NCOL + wave * 32 * NB + nb * 32 + j;
        wbase[nb] = base;
        wres[nb] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, (int)(a.n_out * rb),
                                                     0x00020000);
        wrow[nb] = (uint32_t)(min(col[nb], a.n_out - 1) * rb);
    }

    const MapLayout L0(a.n_map_expert, a.t, a.top_k);
    const int64_t arow0 = a.a_by_token ? a.map[L0.list + tl.pos0] / a.top_k : tl.pos0;
    const uint8_t *abase = reinterpret_cast<const uint8_t *>(a.a) + arow0 * a.k * 2;  // tile's first A row
    // A stage copy: wave instruction i fills LDS rows 4 (8 wave + i) + lane / 16
    auto issue_a = [&](int ks, uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < DMA_PER_WAVE; i++) {
            const int inst = DMA_PER_WAVE * wave + i;
            const int row = 4 * inst + (lane >> 4);
            const int c = (lane & 15) ^ (row & 15);
            dma16(abase + (s_src[row] + (uint32_t)(ks * ROWB + c * 16)), buf + inst * 1024);
        }
        // keep the copies at the start of the stage: without this the compiler
        // sinks them behind the stage's LDS reads (the buffers are separate
        // objects), which leaves the copy no time to land before the barrier
        asm volatile("" ::: "memory");
    };

    // per-lane LDS offsets of the A operand for the 8 steps of a stage
    int aoff[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int c = 4 * (s >> 1) + 2 * kh + (s & 1);
        aoff[s] = j * ROWB + ((c ^ (j & 15)) << 4);
    }

    float16_t acc[4][NB];
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mb][nb][r] = 0.f;

    auto compute = [&](const uint8_t *buf, WB<DT>(&wb)[NB]) {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int p = s >> 1, hh = s & 1;
            half8_t bf[NB];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) bf[nb] = wb[nb].step(p, hh);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const half8_t af = *reinterpret_cast<const half8_t *>(buf + mb * 32 * ROWB + aoff[s]);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[nb], acc[mb][nb], 0, 0, 0);
            }
        }
    };

    WB<DT> w0[NB], w1[NB];
    const int nks = a.k / KS;  // even
    issue_a(0, sA0);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) w0[nb].load(wbase[nb], wres[nb], wrow[nb], 0, kh);
    wait_vmcnt(0);
    __syncthreads();
    // Each stage: prep the weights loaded one stage ago, issue the next
    // stage's A copy and weight loads, compute.  Stage ends wait for the A copy
    // only and use a bare s_barrier: the copies are complete (vmcnt) and LDS
    // needs no further fence between the waves of a workgroup.
    // One-column tiles (NB = 1) have the registers to hold the next stage's
    // weights through the compute: keep their loads at the stage start (the
    // compiler would sink them next to their use).  The two-column tiles
    // would spill, so their loads stay where the compiler puts them.
    auto pin_weight_loads = [] {
        if constexpr (NB == 1 && MX_GEMM_PIN_W) asm volatile("" ::: "memory");
    };
    auto stage_end = [&] {
        wait_vmcnt(MX_GEMM_WSLACK ? NB * WB<DT>::kMinLoads : 0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    for (int ks = 0; ks < nks; ks += 2) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) touch_regs(w0[nb]);
        issue_a(ks + 1, sA1);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) w1[nb].load(wbase[nb], wres[nb], wrow[nb], ks + 1, kh);
        pin_weight_loads();
#pragma unroll
        for (int nb = 0; nb < NB; nb++) w0[nb].template prep<0>(kh);
        compute(sA0, w0);
        stage_end();
#pragma unroll
        for (int nb = 0; nb < NB; nb++) touch_regs(w1[nb]);
        {
            // unconditional, clamped at the last stage (a harmless re-copy into
            // the buffer nobody reads next): no branch merge in front of the
            // next waits, so the compiler keeps exact memory counters
            const int kn = min(ks + 2, nks - 1);
            issue_a(kn, sA0);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) w0[nb].load(wbase[nb], wres[nb], wrow[nb], kn, kh);
            pin_weight_loads();
        }
#pragma unroll
        for (int nb = 0; nb < NB; nb++) w1[nb].template prep<1>(kh);
        compute(sA1, w1);
        stage_end();
    }
    __syncthreads();

    // epilogue: acc[mb][nb][r] = D[row 32 mb + 8 (r / 4) + 4 kh + r % 4][col[nb]]
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 32 * mb + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (row >= tl.mrows) continue;
            const float sc = s_scale[row];
            float *orow = a.out + (int64_t)s_out[row] * a.n_out;
            if constexpr (SWIGLU) {
                if (col[0] < a.n_out) {
                    const float g = acc[mb][0][r] * sc, u = acc[mb][1][r] * sc;
                    // silu(g) * u (silu_mul.metal:57-72) on the hardware exp2 and
                    // reciprocal (about 1 ulp each): the act row is rounded to f16
                    // for the down GEMM, far above these errors
                    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);  // exp(-g)
                    orow[col[0]] = g * __builtin_amdgcn_rcpf(1.0f + e) * u;
                }
            } else {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    if (col[nb] < a.n_out) orow[col[nb]] = acc[mb][nb][r] * sc;
            }
        }
    }
}

// ---- f32 rows -> scaled f16 rows ----------------------------------------------------
// RPT > 0: k <= 1024 * RPT; the row's float4s stay in registers between the
// max pass and the conversion (all loads issued up front).  RPT == 0: any k,
// the row is read twice.
template <int RPT>
__global__ void __launch_bounds__(256) k_to_f16_rows(const float *__restrict__ x, int k,
                                                     const int32_t *__restrict__ count,
                                                     _Float16 *__restrict__ y, float *__restrict__ scale) {
    const int64_t row = blockIdx.x;
    if (count && row >= *count) return;
    __shared__ float s_red[4];
    const float4 *xr = reinterpret_cast<const float4 *>(x + row * k);
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
    half4_t *yr = reinterpret_cast<half4_t *>(y + row * k);
    auto put = [&](int i, const float4 &v) {
        const half2_t lo = __builtin_convertvector((float2_t){v.x * inv, v.y * inv}, half2_t);
        const half2_t hi = __builtin_convertvector((float2_t){v.z * inv, v.w * inv}, half2_t);
        yr[i] = (half4_t){lo[0], lo[1], hi[0], hi[1]};
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
    if (threadIdx.x == 0) scale[row] = ldexpf(1.0f, ex);
}

__global__ void k_ids_with_shared(const uint32_t *__restrict__ ids, int t, int top_k, int n_expert,
                                  uint32_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int kk = top_k + 1;
    if (i >= (int64_t)t * kk) return;
    const int64_t tok = i / kk;
    const int s = (int)(i % kk);
    out[i] = s < top_k ? ids[tok * top_k + s] : (uint32_t)n_expert;
}

// out = residual + (sum_s w_s down_s) + shared   (moe.rs:78; combine.metal:16-40 order)
// KK > 0: compiled for kk = top_k + has_shared == KK, so every slot's load is
// issued before the first one is used; KK == 0: any kk, one slot at a time.
template <int KK>
__global__ void __launch_bounds__(256) k_combine_prefill(const float *__restrict__ down, const float *__restrict__ w,
                                                         const float *__restrict__ residual,
                                                         const float *__restrict__ shared_sep, int top_k,
                                                         int has_shared, int n, float *__restrict__ out) {
    const int64_t tok = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const int kk = KK > 0 ? KK : top_k + has_shared;
    const float *d = down + tok * kk * n + i;
    auto fma4 = [](float ws, const float4 &v, float4 &acc) {
        acc.x = __builtin_fmaf(ws, v.x, acc.x);
        acc.y = __builtin_fmaf(ws, v.y, acc.y);
        acc.z = __builtin_fmaf(ws, v.z, acc.z);
        acc.w = __builtin_fmaf(ws, v.w, acc.w);
    };
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 sh = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (KK > 0) {
        float4 v[KK];
#pragma unroll
        for (int s = 0; s < KK; s++) v[s] = *reinterpret_cast<const float4 *>(d + (int64_t)s * n);
#pragma unroll
        for (int s = 0; s < KK; s++)
            if (s < top_k) fma4(w[tok * top_k + s], v[s], acc);
        if (has_shared) sh = v[KK - 1];
    } else {
        for (int s = 0; s < top_k; s++) fma4(w[tok * top_k + s], *reinterpret_cast<const float4 *>(d + (int64_t)s * n), acc);
        if (has_shared) sh = *reinterpret_cast<const float4 *>(d + (int64_t)top_k * n);
    }
    if (shared_sep) sh = *reinterpret_cast<const float4 *>(shared_sep + tok * n + i);
    if (has_shared || shared_sep) {
        acc.x += sh.x; acc.y += sh.y; acc.z += sh.z; acc.w += sh.w;
    }
    if (residual) {
        const float4 r = *reinterpret_cast<const float4 *>(residual + tok * n + i);
        acc.x = r.x + acc.x; acc.y = r.y + acc.y; acc.z = r.z + acc.z; acc.w = r.w + acc.w;
    }
    *reinterpret_cast<float4 *>(out + tok * n + i) = acc;
}

}  // namespace

bool gemm_supported(int dtype, int k) {
    return (dtype == kQ4_K || dtype == kQ5_K || dtype == kQ6_K || dtype == kQ8_0) && k > 0 && k % 256 == 0;
}

static bool gemm_spans_fit(int64_t a_span, int k, int n_out, int64_t row_bytes) {
    return a_span * k * 2 < (INT64_C(1) << 32) && (int64_t)n_out * row_bytes < (INT64_C(1) << 31);
}

bool gemm_fits(int t, int hidden, int ff, int64_t gu_row_bytes, int64_t d_row_bytes) {
    return gemm_spans_fit(t, hidden, ff, gu_row_bytes) && gemm_spans_fit(GM_BM, ff, hidden, d_row_bytes);
}

mx_status launch_gemm(int dtype, bool swiglu, const GemmArgs &a, hipStream_t s) {
    if (a.t == 0) return MX_OK;
    const MapLayout L(a.n_map_expert, a.t, a.top_k);
    int ncol = 256;
    switch (dtype) {  // output columns per workgroup of the instantiation launched below
    case kQ4_K: ncol = swiglu ? GemmNb<kQ4_K, true>::bn / 2 : GemmNb<kQ4_K, false>::bn; break;
    case kQ5_K: ncol = swiglu ? GemmNb<kQ5_K, true>::bn / 2 : GemmNb<kQ5_K, false>::bn; break;
    case kQ6_K: ncol = swiglu ? GemmNb<kQ6_K, true>::bn / 2 : GemmNb<kQ6_K, false>::bn; break;
    default: ncol = swiglu ? GemmNb<kQ8_0, true>::bn / 2 : GemmNb<kQ8_0, false>::bn; break;
    }
    const int64_t nt = (a.n_out + ncol - 1) / ncol;
    const int64_t t_max = ((int64_t)a.t * a.top_k + GM_BM - 1) / GM_BM + a.n_map_expert;  // m-tiles of GM_BM
    // the kernel addresses a tile's A rows from its first row, and one expert's
    // weight rows from the expert, with 32-bit offsets
    const int64_t a_span = a.a_by_token ? a.t : GM_BM;
    if (!gemm_spans_fit(a_span, a.k, a.n_out, a.row_bytes > a.sh_row_bytes ? a.row_bytes : a.sh_row_bytes))
        return fail(MX_ERR_OVERFLOW, "gemm: an operand span beyond 4 GiB (t * k * 2 bytes of x); split the batch");
    const int64_t blocks = (t_max * nt + 7) / 8 * 8;
    if (blocks > INT32_MAX) return fail(MX_ERR_OVERFLOW, "gemm: too many tiles");
    const dim3 grid((unsigned)blocks);
#define MX_G(DT, SW) hipLaunchKernelGGL((k_gemm<DT, SW>), grid, dim3((64 * GemmNb<DT, SW>::waves)), 0, s, a)
    switch (dtype) {
    case kQ4_K: if (swiglu) MX_G(kQ4_K, true); else MX_G(kQ4_K, false); break;
    case kQ5_K: if (swiglu) MX_G(kQ5_K, true); else MX_G(kQ5_K, false); break;
    case kQ6_K: if (swiglu) MX_G(kQ6_K, true); else MX_G(kQ6_K, false); break;
    default: if (swiglu) MX_G(kQ8_0, true); else MX_G(kQ8_0, false); break;
    }
#undef MX_G
    (void)L;
    MX_LAUNCH("k_gemm");
    return MX_OK;
}

mx_status launch_to_f16_rows(const float *x, int64_t rows, int k, const int32_t *count, _Float16 *y, float *scale,
                             hipStream_t s) {
    if (rows == 0) return MX_OK;
    const dim3 grid((unsigned)rows);
    if (k <= 1024 * 2) hipLaunchKernelGGL(k_to_f16_rows<2>, grid, dim3(256), 0, s, x, k, count, y, scale);
    else if (k <= 1024 * 4) hipLaunchKernelGGL(k_to_f16_rows<4>, grid, dim3(256), 0, s, x, k, count, y, scale);
    else hipLaunchKernelGGL(k_to_f16_rows<0>, grid, dim3(256), 0, s, x, k, count, y, scale);
    MX_LAUNCH("k_to_f16_rows");
    return MX_OK;
}

mx_status launch_ids_with_shared(const uint32_t *ids, int t, int top_k, int n_expert, uint32_t *ids_aug,
                                 hipStream_t s) {
    const int64_t n = (int64_t)t * (top_k + 1);
    if (n == 0) return MX_OK;
    hipLaunchKernelGGL(k_ids_with_shared, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ids, t, top_k,
                       n_expert, ids_aug);
    MX_LAUNCH("k_ids_with_shared");
    return MX_OK;
}

mx_status launch_combine_prefill(const float *down, const float *w, const float *residual, int t, int top_k,
                                 int has_shared, int n, float *out, hipStream_t s, const float *shared_sep) {
    if (t == 0) return MX_OK;
    const dim3 grid((unsigned)((n / 4 + 255) / 256), (unsigned)t);
    switch (top_k + has_shared) {
#define MX_CB(K) \
    case K: hipLaunchKernelGGL(k_combine_prefill<K>, grid, dim3(256), 0, s, down, w, residual, shared_sep, top_k, has_shared, n, out); break;
        MX_CB(2) MX_CB(3) MX_CB(4) MX_CB(5) MX_CB(6) MX_CB(7) MX_CB(8) MX_CB(9) MX_CB(10) MX_CB(11) MX_CB(12)
#undef MX_CB
        default: hipLaunchKernelGGL(k_combine_prefill<0>, grid, dim3(256), 0, s, down, w, residual, shared_sep, top_k, has_shared, n, out);
    }
    MX_LAUNCH("k_combine_prefill");
    return MX_OK;
}

}  // namespace mx
