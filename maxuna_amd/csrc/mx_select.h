// Block-wide stable top-k over expert sort keys (route_from_logits,
// src/moe.rs:94-119: stable descending order of probs + bias, ties -> lower
// expert id; weights = the unbiased probabilities of the picks, normalised by
// max(sum, 6.103515625e-5) in slot order, then scaled).
//
// Keys are distinct 64-bit values (score bits above the complemented expert
// id, see sel_key), so "rank = number of larger keys" is a total order.
// Ranking every key against every other costs n_expert^2 compares; instead:
//   1. the maximum key of each group of 8 consecutive experts;
//   2. T = the top_k-th largest group maximum (0 when there are fewer groups
//      than top_k).  top_k groups have a maximum >= T, so at least top_k keys
//      are >= T and every key of the top_k is >= T;
//   3. keys >= T are gathered (at most 8 * top_k of them) and ranked among
//      themselves.
// E = 256, k = 10: 32 + (<= 80) compares per thread instead of 256.
#pragma once

#include "mx_common.h"

namespace mx {

constexpr int SEL_THREADS = 256;
constexpr int SEL_MAX_E = 1024;
constexpr int SEL_MAX_K = 32;
constexpr int SEL_PER = SEL_MAX_E / SEL_THREADS;

// Sort key of a stable descending sort on the selection score: the score's
// bits mapped to an unsigned order (-0 folded to +0 first, so equal floats get
// equal keys) in the high word, the complemented expert id in the low word
// (equal scores -> the lower id ranks first).  Larger key = earlier position.
__device__ __forceinline__ uint64_t sel_key(float v, int e) {
    v = v + 0.0f;  // -0 -> +0
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)(~(uint32_t)e);
}

// the 64-bit value of this lane's lane_partner<O> (a DPP move of both halves)
template <int O> __device__ __forceinline__ uint64_t lane_partner_u64(uint64_t v) {
    const uint32_t lo = __float_as_uint(lane_partner<O>(__uint_as_float((uint32_t)v)));
    const uint32_t hi = __float_as_uint(lane_partner<O>(__uint_as_float((uint32_t)(v >> 32))));
    return ((uint64_t)hi << 32) | lo;
}

// LDS of one top-k for up to MAXE experts.
template <int MAXE = SEL_MAX_E> struct SelSharedT {
    static_assert(MAXE % SEL_THREADS == 0 && MAXE <= SEL_MAX_E, "MAXE: a multiple of SEL_THREADS");
    uint64_t gmax[MAXE / 8];
    uint64_t ckey[MAXE];
    float cprob[MAXE];
    float prob[SEL_MAX_K];
    int pick[SEL_MAX_K];
    uint64_t thresh;
    int ncand;
    float sum;
};
using SelShared = SelSharedT<>;

// key[j], prob[j]: expert e = threadIdx.x + SEL_THREADS * j (key 0 for e >=
// n_expert).  All SEL_THREADS threads of the block must call; blockDim.x must
// be SEL_THREADS.  Writes ids_out[0..top_k), w_out[0..top_k) (ids_out NULL: neither;
// the picks stay in sh.pick).
// MAXE: the largest n_expert the caller allows (the key arrays hold MAXE /
// SEL_THREADS entries per thread).
template <int MAXE = SEL_MAX_E>
__device__ __forceinline__ void topk_select(const uint64_t (&key)[MAXE / SEL_THREADS],
                                            const float (&prob)[MAXE / SEL_THREADS], int n_expert, int top_k,
                                            float scale, int apply_scale, int norm, uint32_t *__restrict__ ids_out,
                                            float *__restrict__ w_out, SelSharedT<MAXE> &sh) {
    constexpr int PER = MAXE / SEL_THREADS;
    const int tid = threadIdx.x;
    const int G = (n_expert + 7) >> 3;
    // 1. group maxima (8 consecutive experts = 8 consecutive lanes)
#pragma unroll
    for (int j = 0; j < PER; j++) {
        if (j * SEL_THREADS < n_expert) {  // block-uniform
            // partners lane ^ 1, lane ^ 2, then the mirror lane of the 8: the
            // maximum of all 8 lanes reaches every lane of the group
            uint64_t g = key[j];
            uint64_t o = lane_partner_u64<1>(g);
            g = o > g ? o : g;
            o = lane_partner_u64<2>(g);
            g = o > g ? o : g;
            o = lane_partner_u64<4>(g);
            g = o > g ? o : g;
            const int e = tid + SEL_THREADS * j;
            if ((tid & 7) == 0 && e < n_expert) sh.gmax[e >> 3] = g;
        }
    }
    if (tid == 0) {
        sh.ncand = 0;
        sh.thresh = 0;
    }
    __syncthreads();
    // 2. threshold: the group maximum of rank top_k - 1
    if (G >= top_k) {
        for (int g = tid; g < G; g += SEL_THREADS) {
            const uint64_t mine = sh.gmax[g];
            int rank = 0;
            for (int i = 0; i < G; i++) rank += sh.gmax[i] > mine;
            if (rank == top_k - 1) sh.thresh = mine;
        }
    }
    __syncthreads();
    // 3. candidates, ranked among themselves
    const uint64_t T = sh.thresh;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = tid + SEL_THREADS * j;
        if (e < n_expert && key[j] >= T) {
            const int c = atomicAdd(&sh.ncand, 1);
            sh.ckey[c] = key[j];
            sh.cprob[c] = prob[j];
        }
    }
    __syncthreads();
    const int nc = sh.ncand;
    for (int c = tid; c < nc; c += SEL_THREADS) {
        const uint64_t mine = sh.ckey[c];
        int rank = 0;
        for (int i = 0; i < nc; i++) rank += sh.ckey[i] > mine;
        if (rank < top_k) {
            sh.pick[rank] = (int)(~(uint32_t)mine);
            sh.prob[rank] = sh.cprob[c];
        }
    }
    __syncthreads();
    if (!ids_out) return;  // (block-uniform) the caller needs only sh.pick: no weights
    if (tid == 0) {
        float sum = 0.f;
        for (int k = 0; k < top_k; k++) sum = sum + sh.prob[k];
        sh.sum = sum < 6.103515625e-5f ? 6.103515625e-5f : sum;
    }
    __syncthreads();
    if (tid < top_k && ids_out) {  // (NULL: the caller reads sh.pick)
        float wk = sh.prob[tid];
        if (norm) wk = wk / sh.sum;
        if (apply_scale) wk = wk * scale;
        ids_out[tid] = (uint32_t)sh.pick[tid];
        w_out[tid] = wk;
    }
    __syncthreads();
}

// Top-k from keys and probabilities in global memory (written by an earlier
// kernel on the stream).
template <int MAXE = SEL_MAX_E>
__device__ __forceinline__ void topk_from_keys(const uint64_t *__restrict__ keys, const float *__restrict__ probs,
                                               int n_expert, int top_k, float scale, int apply_scale, int norm,
                                               uint32_t *__restrict__ ids_out, float *__restrict__ w_out,
                                               SelSharedT<MAXE> &sh) {
    constexpr int PER = MAXE / SEL_THREADS;
    uint64_t key[PER];
    float prob[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = threadIdx.x + SEL_THREADS * j;
        key[j] = e < n_expert ? keys[e] : 0;
        prob[j] = e < n_expert ? probs[e] : 0.f;
    }
    topk_select<MAXE>(key, prob, n_expert, top_k, scale, apply_scale, norm, ids_out, w_out, sh);
}

}  // namespace mx
