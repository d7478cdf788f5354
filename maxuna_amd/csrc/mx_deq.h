// Bit-exact dequantisation of one 32-weight chunk of a raw GGUF block, shared
// by the dequantise kernel and the f32 gather mat-vec.  Restates the GGUF
// formulas the reference dequantises with (candle QTensor::dequantize,
// moe.rs:173-175; block math mm_id.metal:75-167):
//   Q4_K  y = fl(fl(d*sc) * q) - fl(dmin*m)      (one rounding per op)
//   Q5_K  the same, q = low nibble + 16 * high bit (bit 2i + h of qh[l])
//   Q6_K  y = fl(fl(d*sc) * (q - 32))
//   Q8_0  y = fl(q * d)
// Chunk `part` of a block holds its weights 32 * part .. 32 * part + 31.
// Every including file is compiled with -ffp-contract=off, so no
// product/difference pair is fused into an FMA.
#pragma once

#include "mx_common.h"

namespace mx {

template <int DT>
__device__ __forceinline__ void dequant_chunk(const uint8_t *__restrict__ blk, int part, float (&y)[32]) {
    if constexpr (DT == kQ4_K || DT == kQ5_K) {
        const int i = part >> 1, hi = part & 1;
        const float d = h2f(ld_u16(blk)), dmin = h2f(ld_u16(blk + 2));
        const uint32_t s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8), s2 = ld_u32(blk + 12);
        uint32_t sc, m;
        q4k_scale_min(2 * i + hi, s0, s1, s2, sc, m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        constexpr int QS = DT == kQ5_K ? 48 : 16;  // Q5_K: qh[32] sits before qs
        const uint8_t *q = blk + QS + 32 * i;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t v = ld_u32(q + 4 * w);
            const uint32_t hb = DT == kQ5_K ? ld_u32(blk + 16 + 4 * w) >> (2 * i + hi) : 0u;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const uint32_t byte = (v >> (8 * bb)) & 0xFFu;
                const uint32_t qq = (hi ? (byte >> 4) : (byte & 0xFu)) | (((hb >> (8 * bb)) & 1u) << 4);
                const float p = d1 * (float)qq;
                y[4 * w + bb] = p - m1;
            }
        }
    } else if constexpr (DT == kQ6_K) {
        // part = 4*n + p: half n (0/1), quarter p (0..3) -> weights 128n + 32p + l
        const int n = part >> 2, p = part & 3;
        const float d = h2f(ld_u16(blk + 208));
        const uint8_t *ql = blk + 64 * n + ((p & 1) ? 32 : 0);
        const uint8_t *qh = blk + 128 + 32 * n;
        const int8_t *scp = reinterpret_cast<const int8_t *>(blk + 192 + 8 * n);
        const int shift_l = (p & 2) ? 4 : 0;    // q3/q4 use the high nibble
        const int shift_h = 2 * p;              // qh bits 0-1, 2-3, 4-5, 6-7
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const int ql_b = ql[l], qh_b = qh[l];
            const int q = (((ql_b >> shift_l) & 0xF) | (((qh_b >> shift_h) & 3) << 4)) - 32;
            const float s = d * (float)scp[(l >> 4) + 2 * p];
            y[l] = s * (float)q;
        }
    } else {
        (void)part;
        const float d = h2f(ld_u16(blk));
        const int8_t *qs = reinterpret_cast<const int8_t *>(blk + 2);
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = (float)qs[l] * d;
    }
}

}  // namespace mx
