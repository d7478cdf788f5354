// Staged activations: the integer form in which the decode kernels consume an
// activation row (x for gate/up, the SwiGLU output for down).
//
// Per 32-value group g of a k-vector (k % 32 == 0):
//   s_g  = max|x| / 32000                      (f32)
//   x16  = rint(x / s_g) in [-32000, 32000]    (exact integer grid)
//   x16  = 256 * xh + xl, xh and xl signed int8 (xl in [-128, 127])
// stored as two byte planes so four consecutive values form one dword for
// v_dot4_i32_i8, plus the integer sums of x16 over every 8 and every 32 values
// (the Q4_K "min" term and the Q6_K "-32" offset are applied from them).
// Layout (bytes): xh[k] | xl[k] | s[k/32] f32 | S32[k/32] i32 | S8[k/8] i32.
// The same layout is used in LDS (per-workgroup staging) and in global memory
// (staged once per layer by the router kernel).
#pragma once

#include "mx_common.h"

namespace mx {

constexpr float XQ_RANGE = 32000.0f;

__host__ __device__ constexpr int xstage_bytes(int k) { return 2 * k + (k / 32) * 8 + (k / 8) * 4; }
// distance between staged rows in a buffer of several (256-byte aligned, so
// every row can be copied with aligned 16-byte pieces)
__host__ __device__ constexpr int xstage_stride(int k) { return (xstage_bytes(k) + 255) & ~255; }

struct XView {
    const int8_t *xh, *xl;
    const float *s;
    const int *S32, *S8;
    __device__ XView(const uint8_t *base, int k)
        : xh(reinterpret_cast<const int8_t *>(base)), xl(reinterpret_cast<const int8_t *>(base) + k),
          s(reinterpret_cast<const float *>(base + 2 * k)),
          S32(reinterpret_cast<const int *>(base + 2 * k) + k / 32),
          S8(reinterpret_cast<const int *>(base + 2 * k) + 2 * (k / 32)) {}
};

// Group-major copy for 64-value groups (the Q4_K / Q5_K decode geometry, in
// which lane g of a row reads values 64g .. 64g+63): group g has 9 16-byte
// chunks and chunk c of every group is stored together, at byte (c * G + g) * 16
// with G = k / 64.  Chunks 0-3: xh[64g, 64g+64); 4-7: xl[64g, 64g+64); 8: f32
// {s[2g], s[2g+1], s[2g] * S32[2g], s[2g+1] * S32[2g+1]}.  A wave then reads its
// slices with 9 loads of 1 KB of consecutive bytes each, instead of 16-byte
// pieces 64 bytes apart (which made every load instruction touch ~32 lines).
__host__ __device__ constexpr int xstage_gm_bytes(int k) { return (k / 64) * 144; }
__host__ __device__ constexpr int xstage_gm_stride(int k) { return (xstage_gm_bytes(k) + 255) & ~255; }

// Quantises quarter-group q (values 8q .. 8q+7, given in v) into the staged
// layout at `base` (and, when gm != NULL and k % 64 == 0, into the group-major
// copy at gm).  The four quarters of a group must sit in four consecutive
// lanes (4m .. 4m+3) of one wave, and all four lanes must call this together
// (cross-lane max and sum); `valid` = false lanes contribute nothing and store
// nothing.
__device__ __forceinline__ void stage_quarter(const float (&v)[8], int q, bool valid, uint8_t *base, int k,
                                              uint8_t *gm = nullptr) {
    float mx = 0.f;
    if (valid) {
#pragma unroll
        for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(v[i]));
    }
    mx = fmaxf(mx, lane_partner<1>(mx));
    mx = fmaxf(mx, lane_partner<2>(mx));
    const float inv = mx > 0.f ? XQ_RANGE / mx : 0.f;
    uint32_t h[2], l[2];
    int s8 = 0;
#pragma unroll
    for (int w = 0; w < 2; w++) {
        uint32_t hw = 0, lw = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int xq = valid ? (int)rintf(v[4 * w + b] * inv) : 0;
            const int hd = (xq + 128) >> 8;
            const int ld = xq - (hd << 8);
            s8 += xq;
            hw |= ((uint32_t)hd & 0xFFu) << (8 * b);
            lw |= ((uint32_t)ld & 0xFFu) << (8 * b);
        }
        h[w] = hw;
        l[w] = lw;
    }
    int s32 = s8 + __float_as_int(lane_partner<1>(__int_as_float(s8)));
    s32 = s32 + __float_as_int(lane_partner<2>(__int_as_float(s32)));
    if (valid) {
        int8_t *xh = reinterpret_cast<int8_t *>(base);
        int8_t *xl = xh + k;
        float *s = reinterpret_cast<float *>(base + 2 * k);
        int *S32 = reinterpret_cast<int *>(s + k / 32);
        int *S8 = S32 + k / 32;
        *reinterpret_cast<uint2 *>(xh + 8 * q) = make_uint2(h[0], h[1]);
        *reinterpret_cast<uint2 *>(xl + 8 * q) = make_uint2(l[0], l[1]);
        S8[q] = s8;
        if ((q & 3) == 0) {
            s[q >> 2] = mx / XQ_RANGE;
            S32[q >> 2] = s32;
        }
        if (gm) {
            const int G = k / 64, g = q >> 3, cq = q & 7;
            *reinterpret_cast<uint2 *>(gm + ((size_t)(cq >> 1) * G + g) * 16 + (cq & 1) * 8) = make_uint2(h[0], h[1]);
            *reinterpret_cast<uint2 *>(gm + ((size_t)(4 + (cq >> 1)) * G + g) * 16 + (cq & 1) * 8) = make_uint2(l[0], l[1]);
            if ((q & 3) == 0) {
                float *sc = reinterpret_cast<float *>(gm + ((size_t)8 * G + g) * 16);
                const int par = (q >> 2) & 1;
                const float sg = mx / XQ_RANGE;
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
// nth must be a multiple of 4 and uniform over the group; no barrier
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
