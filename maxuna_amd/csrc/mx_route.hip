// On-GPU sigmoid router with DeepSeek-style selection bias and stable top-k.
//
// Restates route_logits / route_from_logits (src/moe.rs:84-119):
//   probs = sigmoid(logits) = 1 / (exp(-v) + 1)           (f32)
//   sel   = probs + bias                                    (selection only)
//   ids   = stable descending top_k of sel (ties -> lower expert id)
//   w     = probs[ids]; if norm: w /= max(sum(w), 6.103515625e-5); if scale: w *= scale
// The weight sum is accumulated in slot order, like a sequential reduction.
#include "mx_launch.h"

namespace mx {

constexpr int RT_THREADS = 256;
constexpr int RT_MAX_E = 1024;  // experts per token handled by one block (4 per thread)
constexpr int RT_MAX_K = 32;

// Block-wide selection for one token.  `logits` may live in global or shared
// memory; the block must have RT_THREADS threads and all of them must call.
__device__ void select_token(const float *logits, const float *__restrict__ bias, int n_expert,
                             int top_k, float scale, int apply_scale, int norm,
                             uint32_t *__restrict__ ids_out, float *__restrict__ w_out) {
    __shared__ float s_val[RT_THREADS / 64];
    __shared__ int s_idx[RT_THREADS / 64];
    __shared__ int s_pick[RT_MAX_K];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float prob[RT_MAX_E / RT_THREADS], sel[RT_MAX_E / RT_THREADS];
    bool taken[RT_MAX_E / RT_THREADS];
#pragma unroll
    for (int j = 0; j < RT_MAX_E / RT_THREADS; j++) {
        const int e = tid + RT_THREADS * j;
        taken[j] = e >= n_expert;
        prob[j] = 0.f;
        sel[j] = 0.f;
        if (e < n_expert) {
            const float v = logits[e];
            const float ex = expf(-v);
            prob[j] = 1.0f / (ex + 1.0f);
            sel[j] = prob[j] + bias[e];
        }
    }
    for (int k = 0; k < top_k; k++) {
        float best = 0.f;
        int bidx = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < RT_MAX_E / RT_THREADS; j++) {
            const int e = tid + RT_THREADS * j;
            if (!taken[j] && (bidx == 0x7fffffff || sel[j] > best)) { best = sel[j]; bidx = e; }
        }
        // wave argmax: larger value wins; equal values -> lower index
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(bidx, off, 64);
            const bool take = (oi != 0x7fffffff) &&
                              (bidx == 0x7fffffff || ov > best || (ov == best && oi < bidx));
            if (take) { best = ov; bidx = oi; }
        }
        if (lane == 0) { s_val[wave] = best; s_idx[wave] = bidx; }
        __syncthreads();
        if (tid == 0) {
            float b = s_val[0];
            int bi = s_idx[0];
            for (int wv = 1; wv < RT_THREADS / 64; wv++) {
                const float ov = s_val[wv];
                const int oi = s_idx[wv];
                if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > b || (ov == b && oi < bi))) { b = ov; bi = oi; }
            }
            s_pick[k] = bi;
        }
        __syncthreads();
        const int pick = s_pick[k];
#pragma unroll
        for (int j = 0; j < RT_MAX_E / RT_THREADS; j++)
            if (tid + RT_THREADS * j == pick) taken[j] = true;
    }
    // gather unbiased probs of the picks
    __shared__ float s_prob[RT_MAX_K];
#pragma unroll
    for (int j = 0; j < RT_MAX_E / RT_THREADS; j++) {
        const int e = tid + RT_THREADS * j;
        for (int k = 0; k < top_k; k++)
            if (s_pick[k] == e) s_prob[k] = prob[j];
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.f;
        for (int k = 0; k < top_k; k++) sum = sum + s_prob[k];
        if (sum < 6.103515625e-5f) sum = 6.103515625e-5f;
        for (int k = 0; k < top_k; k++) {
            float wk = s_prob[k];
            if (norm) wk = wk / sum;
            if (apply_scale) wk = wk * scale;
            ids_out[k] = (uint32_t)s_pick[k];
            w_out[k] = wk;
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(RT_THREADS) k_route_select(const float *__restrict__ logits,
                                                             const float *__restrict__ bias,
                                                             int n_expert, int top_k, float scale,
                                                             int apply_scale, int norm,
                                                             uint32_t *__restrict__ ids,
                                                             float *__restrict__ w) {
    const int tok = blockIdx.x;
    select_token(logits + (int64_t)tok * n_expert, bias, n_expert, top_k, scale, apply_scale, norm,
                 ids + (int64_t)tok * top_k, w + (int64_t)tok * top_k);
}

mx_status launch_route_select(const float *logits, const float *bias, int t, int n_expert,
                              int top_k, float scale, int apply_scale, int norm, uint32_t *ids,
                              float *w, hipStream_t s) {
    if (t == 0) return MX_OK;
    hipLaunchKernelGGL(k_route_select, dim3(t), dim3(RT_THREADS), 0, s, logits, bias, n_expert,
                       top_k, scale, apply_scale, norm, ids, w);
    MX_LAUNCH("k_route_select");
    return MX_OK;
}

// ---- logits GEMM: [t,H] x [H,E] -> [t,E], f32 ------------------------------------------
// 64x64 output tile per block, 256 threads each computing a 4x4 micro-tile,
// K staged through LDS 32 at a time.
constexpr int LG_T = 64, LG_E = 64, LG_K = 32;

__global__ void __launch_bounds__(256) k_route_logits(const float *__restrict__ x,
                                                      const float *__restrict__ rt, int t,
                                                      int hidden, int n_expert,
                                                      float *__restrict__ logits) {
    __shared__ float sx[LG_K][LG_T + 4];
    __shared__ float sr[LG_K][LG_E];
    const int t0 = blockIdx.y * LG_T, e0 = blockIdx.x * LG_E;
    const int tid = threadIdx.x;
    const int ty = tid / 16, tx = tid % 16;  // 16x16 threads, 4x4 each
    float acc[4][4] = {};
    for (int k0 = 0; k0 < hidden; k0 += LG_K) {
        // x tile: 64 tokens x 32 k (transposed into sx[k][t])
        for (int i = tid; i < LG_T * LG_K; i += 256) {
            const int tt = i / LG_K, kk = i % LG_K;
            const int tok = t0 + tt, kg = k0 + kk;
            sx[kk][tt] = (tok < t && kg < hidden) ? x[(int64_t)tok * hidden + kg] : 0.f;
        }
        for (int i = tid; i < LG_K * LG_E; i += 256) {
            const int kk = i / LG_E, ee = i % LG_E;
            const int kg = k0 + kk, e = e0 + ee;
            sr[kk][ee] = (kg < hidden && e < n_expert) ? rt[(int64_t)kg * n_expert + e] : 0.f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < LG_K; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = sx[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = sr[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int tok = t0 + ty * 4 + i;
        if (tok >= t) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = e0 + tx * 4 + j;
            if (e < n_expert) logits[(int64_t)tok * n_expert + e] = acc[i][j];
        }
    }
}

mx_status launch_route_logits(const float *x, const float *router_t, int t, int hidden,
                              int n_expert, float *logits, hipStream_t s) {
    if (t == 0) return MX_OK;
    const dim3 grid((unsigned)((n_expert + LG_E - 1) / LG_E), (unsigned)((t + LG_T - 1) / LG_T));
    hipLaunchKernelGGL(k_route_logits, grid, dim3(256), 0, s, x, router_t, t, hidden, n_expert, logits);
    MX_LAUNCH("k_route_logits");
    return MX_OK;
}

// ---- fused decode router ------------------------------------------------------------------
// grid.x = ceil(hidden / RF_CHUNK) blocks.  Block c: (optional RMSNorm of each
// token row) -> partial logits over hidden rows [c*RF_CHUNK, +RF_CHUNK) for all
// t tokens -> ws partials.  The last block to finish (device-scope counter)
// reduces the partials in chunk order and runs the selection for every token.
constexpr int RF_CHUNK = 16;
constexpr int RF_MAX_T = 16;

size_t route_fused_ws_bytes(int t, int hidden, int n_expert) {
    const size_t chunks = (size_t)(hidden + RF_CHUNK - 1) / RF_CHUNK;
    return 256 + chunks * (size_t)t * (size_t)n_expert * sizeof(float) +
           (size_t)t * (size_t)n_expert * sizeof(float);
}

__global__ void __launch_bounds__(RT_THREADS) k_route_fused(
    const float *__restrict__ x, const float *__restrict__ rms_alpha, float rms_eps,
    float *__restrict__ x_normed, const float *__restrict__ rt, const float *__restrict__ bias, int t,
    int hidden, int n_expert, int top_k, float scale, int apply_scale, int norm,
    uint32_t *__restrict__ ids, float *__restrict__ w, uint8_t *__restrict__ ws) {
    __shared__ float s_rms[RF_MAX_T];
    __shared__ float s_x[RF_MAX_T][RF_CHUNK];
    __shared__ float s_red[RT_THREADS / 64];
    __shared__ int s_last;
    unsigned int *counter = reinterpret_cast<unsigned int *>(ws);
    float *partial = reinterpret_cast<float *>(ws + 256);
    const int nchunks = gridDim.x;
    float *logits = partial + (size_t)nchunks * t * n_expert;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x;
    const int h0 = c * RF_CHUNK;

    // 1/rms per token (recomputed by every block; the row is L2-resident)
    for (int tok = 0; tok < t; tok++) {
        if (rms_alpha) {
            const float *xr = x + (int64_t)tok * hidden;
            float ss = 0.f;
            for (int i = tid; i < hidden; i += RT_THREADS) ss = __builtin_fmaf(xr[i], xr[i], ss);
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            if (lane == 0) s_red[wave] = ss;
            __syncthreads();
            if (tid == 0) {
                float tot = 0.f;
                for (int wv = 0; wv < RT_THREADS / 64; wv++) tot += s_red[wv];
                s_rms[tok] = sqrtf(tot / (float)hidden + rms_eps);
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < t * RF_CHUNK; i += RT_THREADS) {
        const int tok = i / RF_CHUNK, hh = i % RF_CHUNK, h = h0 + hh;
        float v = 0.f;
        if (h < hidden) {
            v = x[(int64_t)tok * hidden + h];
            if (rms_alpha) v = v / s_rms[tok] * rms_alpha[h];
            if (x_normed) x_normed[(int64_t)tok * hidden + h] = v;
        }
        s_x[tok][hh] = v;
    }
    __syncthreads();
    for (int e = tid; e < n_expert; e += RT_THREADS) {
        float r[RF_CHUNK];
#pragma unroll
        for (int hh = 0; hh < RF_CHUNK; hh++)
            r[hh] = (h0 + hh < hidden) ? rt[(int64_t)(h0 + hh) * n_expert + e] : 0.f;
        for (int tok = 0; tok < t; tok++) {
            float acc = 0.f;
#pragma unroll
            for (int hh = 0; hh < RF_CHUNK; hh++) acc = __builtin_fmaf(s_x[tok][hh], r[hh], acc);
            partial[((size_t)c * t + tok) * n_expert + e] = acc;
        }
    }
    // publish partials (each wave drains and writes back its stores), then count in
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)nchunks - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;  // block-uniform
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __shared__ float s_logit[RT_MAX_E];
    for (int tok = 0; tok < t; tok++) {
        for (int e = tid; e < n_expert; e += RT_THREADS) {
            float acc = 0.f;
            for (int cc = 0; cc < nchunks; cc++) acc += partial[((size_t)cc * t + tok) * n_expert + e];
            s_logit[e] = acc;
            logits[(size_t)tok * n_expert + e] = acc;
        }
        __syncthreads();
        select_token(s_logit, bias, n_expert, top_k, scale, apply_scale, norm,
                     ids + (int64_t)tok * top_k, w + (int64_t)tok * top_k);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

mx_status launch_route_fused(const float *x, const float *rms_alpha, float rms_eps,
                             float *x_normed, const float *router_t, const float *bias, int t,
                             int hidden, int n_expert, int top_k, float scale, int apply_scale,
                             int norm, uint32_t *ids, float *w, void *ws, hipStream_t s) {
    if (t == 0) return MX_OK;
    if (t > RF_MAX_T) return fail(MX_ERR_SHAPE, "fused router handles at most %d tokens", RF_MAX_T);
    const dim3 grid((unsigned)((hidden + RF_CHUNK - 1) / RF_CHUNK));
    hipLaunchKernelGGL(k_route_fused, grid, dim3(RT_THREADS), 0, s, x, rms_alpha, rms_eps, x_normed,
                       router_t, bias, t, hidden, n_expert, top_k, scale, apply_scale, norm, ids, w,
                       reinterpret_cast<uint8_t *>(ws));
    MX_LAUNCH("k_route_fused");
    return MX_OK;
}

}  // namespace mx
