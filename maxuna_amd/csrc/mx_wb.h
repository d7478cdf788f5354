// Weight dequantisation into f16 MFMA operands, shared by the grouped GEMM
// (mx_gemm.hip) and the verify-block tiles (mx_vmm.hip): per-type staging of
// the raw GGUF bytes of a weight row in LDS and the lane registers read from it.
#pragma once

#include "mx_common.h"
#include "mx_dma.h"

namespace mx {
namespace {

typedef float float2_t __attribute__((ext_vector_type(2)));

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

// Dequantisation into the MFMA B operand: every weight is the f16 rounding of
// the reference's f32 dequantised value (mm_id.metal:75-167), rounded once.
// Bytes b < 1024 of two dwords become the f16 numbers 1024 + b by placing them
// under the exponent byte 0x64 (v_perm_b32); each weight is then one
// v_fma_mix{lo,hi}_f16, an f32 fma of that f16 input with f32 scale factors,
// rounded to f16 once:
//   K-quants with min (Q4_K, Q5_K): y = fma(1024 + q, d1, c), d1 = d * sc and
//     c = -dmin * m - 1024 * d1 in f32.  Against the reference's
//     fl(d1 * q) - fl(dmin * m) the f32 value differs by at most ~2^-13 * d1
//     (the 1024 offset's f32 roundings), far below the f16 rounding that follows
//     (|y| ~ 8 * d1, half an f16 ulp ~2^-9 * d1)
//   Q6_K: y = fma(1024 + q, d1, -1056 * d1) with d1 = d * sc: d has an 11-bit
//     significand, sc 7 bits and 1056 = 33 * 2^5 six, so d1 and -1056 * d1 are
//     exact in f32 and the fma's exact result is (q - 32) * d1 -- exactly the
//     reference's f32 value fl(d1 * (q - 32)), then rounded to f16
// One f16 rounding per weight (the packed-f16 form this replaces rounded twice:
// fl16(dmin * m), and sc * (q - 32) beyond 2048): per two weights one perm
// (shared) and two mix ops.
__device__ __forceinline__ half2_t pk_bytes(uint32_t w, uint32_t sel) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, sel));
}
__device__ __forceinline__ void pk_bytes8(uint32_t w0, uint32_t w1, half2_t (&x)[4]) {
    x[0] = pk_bytes(w0, 0x04010400u);  // bytes 0, 1
    x[1] = pk_bytes(w0, 0x04030402u);  // bytes 2, 3
    x[2] = pk_bytes(w1, 0x04010400u);
    x[3] = pk_bytes(w1, 0x04030402u);
}
// (f16 fma(x.lo, a, c), f16 fma(x.hi, a, c)), each an f32 fma rounded to f16 once
// (v_fma_mixlo_f16 / v_fma_mixhi_f16)
__device__ __forceinline__ half2_t mix2(half2_t x, float a, float c) {
    const _Float16 lo = (_Float16)__builtin_fmaf((float)x[0], a, c);
    const _Float16 hi = (_Float16)__builtin_fmaf((float)x[1], a, c);
    return half2_t{lo, hi};
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
// d1 = d * sc, c = -dmin * m - 1024 * d1 (f32)
__device__ __forceinline__ half8_t dq8_kmin(uint32_t w0, uint32_t w1, float d1, float c) {
    half2_t x[4], y[4];
    pk_bytes8(w0, w1, x);
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = mix2(x[i], d1, c);
    return pk_join(y);
}
// d1 = d * sc, c = -1056 * d1 (both exact in f32)
__device__ __forceinline__ half8_t dq8_q6(uint32_t w0, uint32_t w1, float d1, float c) {
    half2_t x[4], y[4];
    pk_bytes8(w0, w1, x);
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = mix2(x[i], d1, c);
    return pk_join(y);
}
// ---- per-type weight staging: LDS slots filled by DMA, lane registers read from them -----
// Every stage, the workgroup copies the raw bytes of its weight rows for that
// stage into LDS with buffer->LDS DMA (16-byte chunks, consecutive lanes take
// consecutive chunks of a row, so each copy instruction reads a few whole row
// spans instead of 64 scattered pieces).  Row R of the tile owns a slot of
// CPR chunks at R * SLOT; the chunks are the 16-byte-aligned pieces covering
// the fields the stage needs.  A lane then reads its own row's slot (slots are
// SLOT bytes apart, chosen so 8 consecutive rows hit distinct LDS banks) and
// dequantises in registers as before.
//   Q4_K  5 chunks: block header (d, dmin, scales) | qs[64 par, +64)
//   Q5_K  7 chunks: header | qh[0, 32) | qs[64 par, +64)
//   Q6_K 11 chunks: ql[64 n, +64) | qh[32 n, +32) | scales + d, each span from its
//        16-byte-aligned start (blocks are 2-byte aligned; m1 = the block's
//        address mod 16 locates the fields), plus one spare
//   Q8_0 11 chunks: the 4 blocks (136 bytes) of the stage from the aligned start
// The buffer resource starts at the expert's 16-byte-aligned base, so every
// chunk offset is aligned; the range ends at the 16-byte boundary after the
// expert's last byte (chunks wholly past it copy nothing and are never read).
template <int DT> struct WB;

// one 16-byte buffer -> LDS copy per lane (lane i's bytes land at lds_dst + 16 i)
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint8_t *lds_dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (MX_AS_LDS void *)lds_dst, 16, off, 0, 0, 0);
}

// Q4_K: stage = half `par` of super-block ks / 2; 64-value chunks i = 2 par + c.
// Lane half kh holds qs bytes [32 i + 16 kh, +16) of both chunks; step p = 2c + nib
// uses the low (nib 0) or high nibbles, sub-block 2 i + nib (mm_id.metal:95-113).
template <> struct WB<kQ4_K> {
    static constexpr int CPR = 5, SLOT = 80;
    // byte offset (from the block start) of chunk c of stage parity par
    __device__ static uint32_t chunk_off(int c, int par) { return c == 0 ? 0u : (uint32_t)(16 + 64 * par + 16 * (c - 1)); }
    static constexpr int BLK = 144;
    uint4 h, q[2];
    __device__ __forceinline__ void load_lds(const uint8_t *slot, int kh, uint32_t) {
        h = *reinterpret_cast<const uint4 *>(slot);
        q[0] = *reinterpret_cast<const uint4 *>(slot + 16 + 16 * kh);
        q[1] = *reinterpret_cast<const uint4 *>(slot + 48 + 16 * kh);
    }
    float d1[4], c1[4];  // d * sc and -dmin * m - 1024 * d * sc of each sub-block
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
        const float d = h2f((uint16_t)(h.x & 0xFFFFu)), dmin = h2f((uint16_t)(h.x >> 16));
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mn;
            q4k_scale_min(4 * PAR + p, h.y, h.z, h.w, sc, mn);
            d1[p] = d * (float)sc;
            c1[p] = __builtin_fmaf(-1024.0f, d1[p], -(dmin * (float)mn));
        }
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &v = q[p >> 1];
        const int sh = 4 * (p & 1);
        const uint32_t w0 = ((hh ? v.z : v.x) >> sh) & 0x0F0F0F0Fu;
        const uint32_t w1 = ((hh ? v.w : v.y) >> sh) & 0x0F0F0F0Fu;
        return dq8_kmin(w0, w1, d1[p], c1[p]);
    }
};

// Q4_K, the form the prefill GEMM uses: the same stage slot, but lane half kh
// owns the 64-value chunk kh of the half super-block -- sub-blocks 2 kh (low
// nibbles) and 2 kh + 1 (high nibbles), qs bytes [32 kh, +32) of the slot's 64 --
// so it unpacks two scale / min pairs per half instead of four; step s gives it
// the values 64 kh + 8 s + [0, 8) of the half.  Same dequantised values as
// WB<kQ4_K> (the K order of the MFMA steps differs; A follows it).
struct WB4L {
    static constexpr int CPR = WB<kQ4_K>::CPR, SLOT = WB<kQ4_K>::SLOT, BLK = WB<kQ4_K>::BLK;
    uint4 h, q[2];
    __device__ __forceinline__ void load_lds(const uint8_t *slot, int kh, uint32_t) {
        h = *reinterpret_cast<const uint4 *>(slot);
        q[0] = *reinterpret_cast<const uint4 *>(slot + 16 + 32 * kh);
        q[1] = *reinterpret_cast<const uint4 *>(slot + 32 + 32 * kh);
    }
    float d1[2], c1[2];
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        const float d = h2f((uint16_t)(h.x & 0xFFFFu)), dmin = h2f((uint16_t)(h.x >> 16));
        uint32_t sc, mn;
        q4k_pair_scale_min(2 * PAR + kh, h.y, h.z, h.w, sc, mn);  // sub-blocks 4 PAR + 2 kh, + 1
#pragma unroll
        for (int i = 0; i < 2; i++) {
            d1[i] = d * (float)((sc >> (8 * i)) & 0xFFu);
            c1[i] = __builtin_fmaf(-1024.0f, d1[i], -(dmin * (float)((mn >> (8 * i)) & 0xFFu)));
        }
    }
    __device__ __forceinline__ half8_t step(int s) const {
        const uint4 &v = q[(s & 3) >> 1];
        const int sh = 4 * (s >> 2);
        const uint32_t w0 = (((s & 1) ? v.z : v.x) >> sh) & 0x0F0F0F0Fu;
        const uint32_t w1 = (((s & 1) ? v.w : v.y) >> sh) & 0x0F0F0F0Fu;
        return dq8_kmin(w0, w1, d1[s >> 2], c1[s >> 2]);
    }
};

// Q5_K: Q4_K's stage layout (qs at byte 48) plus lane half kh's 16 bytes of qh;
// step p of half `par` adds bit 4 par + p of qh[l] as the fifth bit (mm_id.metal:113-134).
template <> struct WB<kQ5_K> {
    static constexpr int CPR = 7, SLOT = 112;
    __device__ static uint32_t chunk_off(int c, int par) {
        return c < 3 ? (uint32_t)(16 * c) : (uint32_t)(48 + 64 * par + 16 * (c - 3));
    }
    static constexpr int BLK = 176;
    uint4 h, q[2], qh;
    __device__ __forceinline__ void load_lds(const uint8_t *slot, int kh, uint32_t) {
        h = *reinterpret_cast<const uint4 *>(slot);
        qh = *reinterpret_cast<const uint4 *>(slot + 16 + 16 * kh);
        q[0] = *reinterpret_cast<const uint4 *>(slot + 48 + 16 * kh);
        q[1] = *reinterpret_cast<const uint4 *>(slot + 80 + 16 * kh);
    }
    float d1[4], c1[4];
    int hsh;
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
        const float d = h2f((uint16_t)(h.x & 0xFFFFu)), dmin = h2f((uint16_t)(h.x >> 16));
#pragma unroll
        for (int p = 0; p < 4; p++) {
            uint32_t sc, mn;
            q4k_scale_min(4 * PAR + p, h.y, h.z, h.w, sc, mn);
            d1[p] = d * (float)sc;
            c1[p] = __builtin_fmaf(-1024.0f, d1[p], -(dmin * (float)mn));
        }
        hsh = 4 * PAR;
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &v = q[p >> 1];
        const int sh = 4 * (p & 1);
        const uint32_t hb = hsh + p;
        const uint32_t w0 = (((hh ? v.z : v.x) >> sh) & 0x0F0F0F0Fu) | ((((hh ? qh.z : qh.x) >> hb) & 0x01010101u) << 4);
        const uint32_t w1 = (((hh ? v.w : v.y) >> sh) & 0x0F0F0F0Fu) | ((((hh ? qh.w : qh.y) >> hb) & 0x01010101u) << 4);
        return dq8_kmin(w0, w1, d1[p], c1[p]);
    }
};

// 16 bytes at slot + off (off even, the field's offset inside its 16-byte-aligned
// span): an aligned-down dword run, funnel-shifted by the 2-byte phase
__device__ __forceinline__ uint4 lds16_a2(const uint8_t *slot, uint32_t off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(slot + (off & ~3u));
    const uint32_t sh = (off & 2u) * 8u;
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[4];
    return make_uint4(__builtin_amdgcn_alignbit(d1, d0, sh), __builtin_amdgcn_alignbit(d2, d1, sh),
                      __builtin_amdgcn_alignbit(d3, d2, sh), __builtin_amdgcn_alignbit(d4, d3, sh));
}

// Q6_K: stage = half n = par of super-block ks / 2 (128 values).  Lane half kh
// holds ql[64n + 16kh, +16), ql[64n + 32 + 16kh, +16), qh[32n + 16kh, +16);
// step p takes the 4-bit part from the low (p even) / high (p odd) ql piece,
// nibble p / 2, and bits 2p of qh; scale 8n + 2p + kh (mm_id.metal:115-135).
template <> struct WB<kQ6_K> {
    static constexpr int CPR = 11, SLOT = 176;
    static constexpr int BLK = 210;
    // chunk c (relative to the block's 16-byte-aligned address) of stage parity n:
    // ql span 0-4, qh span 5-7, scales/d span 8-10 (10 is spare)
    __device__ static uint32_t chunk_off(int c, int n) {
        return c < 5 ? (uint32_t)(64 * n + 16 * c) : c < 8 ? (uint32_t)(128 + 32 * n + 16 * (c - 5))
                                                           : (uint32_t)(192 + 16 * (c - 8));
    }
    uint4 lo, hi, qh;
    uint32_t s0, s1;
    uint16_t dbits;
    __device__ __forceinline__ void load_lds(const uint8_t *slot, int kh, uint32_t m1, int n) {
        lo = lds16_a2(slot, m1 + 16 * kh);
        hi = lds16_a2(slot, m1 + 32 + 16 * kh);
        qh = lds16_a2(slot + 80, m1 + 16 * kh);
        // scales[8n .. 8n+7] and d: tail span at slot + 128, scales[0] at m1, d at m1 + 16
        const uint32_t so = m1 + 8 * n;
        const uint32_t *w = reinterpret_cast<const uint32_t *>(slot + 128 + (so & ~3u));
        const uint32_t sh = (so & 2u) * 8u;
        const uint32_t a0 = w[0], a1 = w[1], a2 = w[2];
        s0 = __builtin_amdgcn_alignbit(a1, a0, sh);
        s1 = __builtin_amdgcn_alignbit(a2, a1, sh);
        dbits = *reinterpret_cast<const uint16_t *>(slot + 128 + m1 + 16);
    }
    float d1[4], c1[4];  // d * sc and -1056 * d * sc, exact in f32
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        const float d = h2f(dbits);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int j = 2 * p + kh;  // byte j of the stage's 8 scales
            const uint32_t word = j < 4 ? s0 : s1;
            const int8_t s8 = (int8_t)((word >> (8 * (j & 3))) & 0xFFu);
            d1[p] = d * (float)s8;
            c1[p] = -1056.0f * d1[p];
        }
    }
    __device__ __forceinline__ half8_t step(int p, int hh) const {
        const uint4 &ql = (p & 1) ? hi : lo;
        const int shl = 4 * (p >> 1), shh = 2 * p;
        const uint32_t a0 = ((hh ? ql.z : ql.x) >> shl) & 0x0F0F0F0Fu;
        const uint32_t a1 = ((hh ? ql.w : ql.y) >> shl) & 0x0F0F0F0Fu;
        const uint32_t b0 = (((hh ? qh.z : qh.x) >> shh) & 0x03030303u) << 4;
        const uint32_t b1 = (((hh ? qh.w : qh.y) >> shh) & 0x03030303u) << 4;
        return dq8_q6(a0 | b0, a1 | b1, d1[p], c1[p]);
    }
};

// Q8_0: stage = blocks 4 ks + p (136 bytes from the aligned start); lane half kh
// holds quants [16 kh, +16) of each.
template <> struct WB<kQ8_0> {
    static constexpr int CPR = 11, SLOT = 176;
    __device__ static uint32_t chunk_off(int c, int) { return (uint32_t)(16 * c); }
    uint4 v[4];
    uint16_t dh[4];
    __device__ __forceinline__ void load_lds(const uint8_t *slot, int kh, uint32_t m1, int) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            v[p] = lds16_a2(slot, m1 + 34 * p + 2 + 16 * kh);
            dh[p] = *reinterpret_cast<const uint16_t *>(slot + m1 + 34 * p);
        }
    }
    float d[4];
    template <int PAR> __device__ __forceinline__ void prep(int kh) {
        (void)kh;
#pragma unroll
        for (int p = 0; p < 4; p++) d[p] = h2f(dh[p]);
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

// byte offset of stage ks's data inside a weight row, and whether the type's
// fields need the block's 16-byte phase (2-byte-aligned blocks)
template <int DT> __device__ __forceinline__ uint32_t stage_block_off(int ks) {
    if constexpr (DT == kQ8_0) return (uint32_t)(4 * ks) * 34u;
    else return (uint32_t)(ks >> 1) * (uint32_t)WB<DT>::BLK;
}
template <int DT> constexpr bool kPhased = DT == kQ6_K || DT == kQ8_0;
template <int DT> __device__ __forceinline__ void wb_load(WB<DT> &w, const uint8_t *slot, int kh, uint32_t m1, int par) {
    if constexpr (kPhased<DT>) w.load_lds(slot, kh, m1, par);
    else w.load_lds(slot, kh, m1);
}

}  // namespace
}  // namespace mx
