// Staged activations: the integer form in which the decode kernels consume an
// activation row (x for gate/up, the SwiGLU output for down).
//
// Per scale group g of a k-vector (k % 32 == 0) -- the aligned 128-value block
// when k % 128 == 0, else the 32-value group -- with m = max|x| over g:
//   s_g = 2^e, e = frexp_exp(m) - 23 (+1 if m / 2^e > X24_MAX), e >= -149
//   x24 = rint(x / s_g), an integer in [-2^23, X24_MAX]
//   x24 = 65536 * xh + 256 * xm + xl, three signed int8 digits in [-128, 127]
// The scale is a power of two, so x / s_g is exact and s_g * x24 is the
// represented value exactly; the only error is the rint:
//   |s_g * x24 - x| <= s_g / 2 <= 2^-23 * (1 + 2^-8) * m
// i.e. every value is carried to within ~2 f32 ulps of its group's largest
// magnitude (a 24-bit grid, the width of an f32 significand).  Values whose
// magnitude is within 2^-1 of m keep their f32 value to within one ulp of
// their own; smaller values keep 24 bits below m.
// Stored as three byte planes so four consecutive values form one dword for
// v_dot4_i32_i8, plus the integer sum of x24 over every 32 values (the Q4_K
// "min" term is applied from it).
// Layout (bytes): xh[k] | xm[k] | xl[k] | s[k/32] f32 | S32[k/32] i32 (s per
// 32-value group; with 128-value scale groups the four entries of a block hold
// the same scale).
// The same layout is used in LDS (per-workgroup staging) and in global memory
// (staged once per layer by the router kernel).
#pragma once

#include "mx_common.h"

namespace mx {

// largest x24 whose three balanced digits all fit int8: 127 * (65536 + 256 + 1)
constexpr int X24_MAX = 8355711;

__host__ __device__ constexpr int xstage_bytes(int k) { return 3 * k + (k / 32) * 8; }
// distance between staged rows in a buffer of several (256-byte aligned, so
// every row can be copied with aligned 16-byte pieces)
__host__ __device__ constexpr int xstage_stride(int k) { return (xstage_bytes(k) + 255) & ~255; }

struct XView {
    const int8_t *xh, *xm, *xl;
    const float *s;
    const int *S32;
    __device__ XView(const uint8_t *base, int k)
        : xh(reinterpret_cast<const int8_t *>(base)), xm(reinterpret_cast<const int8_t *>(base) + k),
          xl(reinterpret_cast<const int8_t *>(base) + 2 * k), s(reinterpret_cast<const float *>(base + 3 * k)),
          S32(reinterpret_cast<const int *>(base + 3 * k) + k / 32) {}
};

// Group-major copy for 64-value groups (the Q4_K / Q5_K decode geometry, in
// which lane g of a row reads values 64g .. 64g+63): group g has 13 16-byte
// chunks and chunk c of every group is stored together, at byte (c * G + g) * 16
// with G = k / 64.  Chunks 0-3: xh[64g, 64g+64); 4-7: xm; 8-11: xl; 12: f32
// {s[2g], s[2g+1], s[2g] * S32[2g], s[2g+1] * S32[2g+1]}.  A wave then reads its
// slices with 13 loads of 1 KB of consecutive bytes each, instead of 16-byte
// pieces 64 bytes apart (which made every load instruction touch ~32 lines).
constexpr int GM_CHUNKS = 13;
__host__ __device__ constexpr int xstage_gm_bytes(int k) { return (k / 64) * 16 * GM_CHUNKS; }
__host__ __device__ constexpr int xstage_gm_stride(int k) { return (xstage_gm_bytes(k) + 255) & ~255; }

// Exponent e of a group's power-of-two scale for its largest magnitude m
// (m finite, > 0): m / 2^e lies in [2^22, X24_MAX].
__device__ __forceinline__ int x24_exponent(float m) {
    int e = __builtin_amdgcn_frexp_expf(m) - 23;  // m = f * 2^(e + 23), f in [0.5, 1)
    if (e < -149) e = -149;                         // below: absolute error <= 2^-150
    if (__builtin_amdgcn_ldexpf(m, -e) > (float)X24_MAX) e += 1;
    return e;
}


// The staged form of quarter-group values v (8 consecutive values of one 32-value
// group): digit words h, m, l (4 values per word), the group scale sg and the
// group's sum of x24 (s32).  The four quarters of a group must sit in four
// consecutive lanes (4m .. 4m+3) of one wave, and all four lanes must call this
// together (cross-lane max and sum); `valid` = false lanes contribute zeros.  A
// group holding Inf or NaN gets a NaN scale, so it poisons the rows that read it,
// as f32 arithmetic would.
// wide (rows with k % 128 == 0, uniform over the wave): the scale is shared by
// the 16 quarters (128 values) of an aligned block, which then sit in 16
// consecutive lanes (16m .. 16m+15): every 32-value group of the block gets the
// same s_g, so the grid is relative to the block's largest magnitude.  The four
// 32-value parts a Q6_K lane group reads lie in one such block, so their integer
// sums are scaled and added before the conversion to f32 (Q<kQ6_K>::dot).  s32
// stays per 32-value group.
__device__ __forceinline__ void quarter_digits(const float (&v)[8], bool valid, uint32_t (&h)[2], uint32_t (&m)[2],
                                               uint32_t (&l)[2], float &sg, int &s32, bool wide) {
    // max |x| as the integer order of the magnitude bits: Inf and NaN patterns
    // are above every finite one, so a group holding either ends with a
    // non-finite maximum (also across lanes: integer max never drops a NaN)
    uint32_t mb = 0;
    if (valid) {
#pragma unroll
        for (int i = 0; i < 8; i++) mb = max(mb, __float_as_uint(v[i]) & 0x7FFFFFFFu);
    }
    auto pmax = [&](auto c) {
        mb = max(mb, __float_as_uint(lane_partner<decltype(c)::value>(__uint_as_float(mb))));
    };
    pmax(std::integral_constant<int, 1>{});
    pmax(std::integral_constant<int, 2>{});
    if (wide) {
        pmax(std::integral_constant<int, 4>{});
        pmax(std::integral_constant<int, 8>{});
    }
    const float mx = __uint_as_float(mb);
    const bool finite = mb < 0x7F800000u;
    const bool nz = finite && mb != 0;
    const int e = nz ? x24_exponent(mx) : 0;
    // x24 = 65536 h + 256 m + l with balanced digits in [-128, 127]: l is the low
    // byte of x24 read as signed, r = (x24 + 128) >> 8 = 256 h + m, and
    // h = (r + 128) >> 8; each digit's byte is the low byte of x24, r and h, which
    // v_perm_b32 gathers four at a time into the plane words
    int xq[8], r[8], hh[8];
    int s8 = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        xq[i] = (valid && nz) ? (int)rintf(__builtin_amdgcn_ldexpf(v[i], -e)) : 0;
        r[i] = (xq[i] + 128) >> 8;
        hh[i] = (r[i] + 128) >> 8;
        s8 += xq[i];
    }
    // low bytes of a, b, c, d -> one word, a in byte 0 (v_perm_b32 selector byte
    // 0 = the second operand's low byte, 4 = the first operand's)
    auto gather = [](int a0, int b0, int c0, int d0) {
        const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b0, (uint32_t)a0, 0x0C0C0400u);
        const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d0, (uint32_t)c0, 0x0C0C0400u);
        return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
    };
#pragma unroll
    for (int w = 0; w < 2; w++) {
        l[w] = gather(xq[4 * w], xq[4 * w + 1], xq[4 * w + 2], xq[4 * w + 3]);
        m[w] = gather(r[4 * w], r[4 * w + 1], r[4 * w + 2], r[4 * w + 3]);
        h[w] = gather(hh[4 * w], hh[4 * w + 1], hh[4 * w + 2], hh[4 * w + 3]);
    }
    s32 = s8 + __float_as_int(lane_partner<1>(__int_as_float(s8)));
    s32 = s32 + __float_as_int(lane_partner<2>(__int_as_float(s32)));
    sg = !finite ? __builtin_nanf("") : nz ? __builtin_amdgcn_ldexpf(1.0f, e) : 0.f;
}

// Quantises quarter-group q (values 8q .. 8q+7, given in v) into the staged
// layout at `base` (and, when gm != NULL and k % 64 == 0, into the group-major
// copy at gm), under quarter_digits' lane rules; `valid` = false lanes store
// nothing.
// Rows with k % 128 == 0 take one scale per 128-value block (quarter_digits'
// wide rule: the 16 quarters of a block in 16 consecutive lanes).
__device__ __forceinline__ void stage_quarter(const float (&v)[8], int q, bool valid, uint8_t *base, int k,
                                              uint8_t *gm = nullptr) {
    uint32_t h[2], m[2], l[2];
    float sg;
    int s32;
    quarter_digits(v, valid, h, m, l, sg, s32, k % 128 == 0);
    if (valid) {
        int8_t *xh = reinterpret_cast<int8_t *>(base);
        int8_t *xm = xh + k;
        int8_t *xl = xh + 2 * k;
        float *s = reinterpret_cast<float *>(base + 3 * k);
        int *S32 = reinterpret_cast<int *>(s + k / 32);
        *reinterpret_cast<uint2 *>(xh + 8 * q) = make_uint2(h[0], h[1]);
        *reinterpret_cast<uint2 *>(xm + 8 * q) = make_uint2(m[0], m[1]);
        *reinterpret_cast<uint2 *>(xl + 8 * q) = make_uint2(l[0], l[1]);
        if ((q & 3) == 0) {
            s[q >> 2] = sg;
            S32[q >> 2] = s32;
        }
        if (gm) {
            const int G = k / 64, g = q >> 3, cq = q & 7;
            const size_t half = (size_t)(cq & 1) * 8;
            *reinterpret_cast<uint2 *>(gm + ((size_t)(cq >> 1) * G + g) * 16 + half) = make_uint2(h[0], h[1]);
            *reinterpret_cast<uint2 *>(gm + ((size_t)(4 + (cq >> 1)) * G + g) * 16 + half) = make_uint2(m[0], m[1]);
            *reinterpret_cast<uint2 *>(gm + ((size_t)(8 + (cq >> 1)) * G + g) * 16 + half) = make_uint2(l[0], l[1]);
            if ((q & 3) == 0) {
                float *sc = reinterpret_cast<float *>(gm + ((size_t)12 * G + g) * 16);
                const int par = (q >> 2) & 1;
                sc[par] = sg;
                sc[2 + par] = sg * (float)s32;
            }
        }
    }
}

// 8 consecutive floats from a 16-byte-aligned address.
__device__ __forceinline__ void load8f(const float *p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Block-cooperative staging of one row into LDS, split so the activation loads
// can be issued before a wave's weight loads: `pre` loads this thread's
// quarters (quarter tid + blockDim * i, XPRE of them in registers), `post`
// quantises them (and any beyond XPRE, loading on the fly), then a block barrier.
// Every thread of the block must call both.
constexpr int XPRE = 2;
template <int NP> struct XPreT {
    float v[NP][8];
};
using XPre = XPreT<XPRE>;
// Staging by a group of nth threads (thread tid of them): quarters tid + nth * i.
template <int NP>
__device__ __forceinline__ void stage_pre_t(const float *__restrict__ x, int k, XPreT<NP> &p, int tid, int nth) {
    const int nq = k / 8;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int q = tid + nth * i;
        if (q < nq) load8f(x + 8 * q, p.v[i]);
    }
}
// nth must be a multiple of 16 and uniform over the group; no barrier
template <int NP>
__device__ __forceinline__ void stage_post_t(const float *__restrict__ x, int k, const XPreT<NP> &p, uint8_t *lds,
                                             int tid, int nth) {
    const int nq = k / 8;
    const int iters = (nq + nth - 1) / nth;  // group-uniform
#pragma unroll
    for (int i = 0; i < NP; i++) {
        if (i < iters) {
            const int q = tid + nth * i;
            stage_quarter(p.v[i], q, q < nq, lds, k);
        }
    }
    for (int i = NP; i < iters; i++) {
        const int q = tid + nth * i;
        float v[8];
        if (q < nq) load8f(x + 8 * q, v);
        stage_quarter(v, q, q < nq, lds, k);
    }
}
__device__ __forceinline__ void stage_pre(const float *__restrict__ x, int k, XPre &p) {
    stage_pre_t(x, k, p, (int)threadIdx.x, (int)blockDim.x);
}
__device__ __forceinline__ void stage_post(const float *__restrict__ x, int k, const XPre &p, uint8_t *lds) {
    stage_post_t(x, k, p, lds, (int)threadIdx.x, (int)blockDim.x);
    __syncthreads();
}

}  // namespace mx
