// On-GPU sigmoid router with DeepSeek-style selection bias and stable top-k.
//
// Restates route_logits / route_from_logits (src/moe.rs:84-119):
//   logits = x . router^T                                  (f32)
//   probs  = sigmoid(logits) = 1 / (exp(-v) + 1)           (f32)
//   sel    = probs + bias                                  (selection only)
//   ids    = stable descending top_k of sel (ties -> lower expert id)
//   w      = probs[ids]; if norm: w /= max(sum(w), 6.103515625e-5); if scale: w *= scale
// The weight sum is accumulated in slot order, like a sequential reduction.
//
// The router weight is taken in its GGUF layout `ffn_gate_inp` [n_expert, hidden]
// (each expert's weights contiguous), so a wave reads one expert's row with
// fully coalesced 16-byte loads; the reference transposes it at load time for
// its matmul (moe.rs:43), which this layout makes unnecessary.
#include "mx_launch.h"

namespace mx {

constexpr int RT_THREADS = 256;
constexpr int RT_MAX_E = 1024;
constexpr int RT_MAX_K = 32;

// Block-wide stable top-k for one token, by rank: expert e's rank is the number
// of experts whose selection score is larger, or equal with a lower id -- exactly
// its position in a stable descending sort.  `logits` may be in shared or global
// memory; all RT_THREADS threads must call.
__device__ void select_token(const float *logits, const float *__restrict__ bias, int n_expert, int top_k,
                             float scale, int apply_scale, int norm, uint32_t *__restrict__ ids_out,
                             float *__restrict__ w_out) {
    __shared__ float s_sel[RT_MAX_E];
    __shared__ float s_prob[RT_MAX_K];
    __shared__ int s_pick[RT_MAX_K];
    const int tid = threadIdx.x;
    float prob[RT_MAX_E / RT_THREADS];
#pragma unroll
    for (int j = 0; j < RT_MAX_E / RT_THREADS; j++) {
        const int e = tid + RT_THREADS * j;
        if (e < n_expert) {
            const float ex = expf(-logits[e]);
            prob[j] = 1.0f / (ex + 1.0f);
            s_sel[e] = prob[j] + bias[e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RT_MAX_E / RT_THREADS; j++) {
        const int e = tid + RT_THREADS * j;
        if (e < n_expert) {
            const float mine = s_sel[e];
            int rank = 0;
            for (int o = 0; o < n_expert; o++) {
                const float v = s_sel[o];
                rank += (v > mine) || (v == mine && o < e);
            }
            if (rank < top_k) {
                s_pick[rank] = e;
                s_prob[rank] = prob[j];
            }
        }
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
                                                             const float *__restrict__ bias, int n_expert,
                                                             int top_k, float scale, int apply_scale, int norm,
                                                             uint32_t *__restrict__ ids, float *__restrict__ w) {
    const int tok = blockIdx.x;
    select_token(logits + (int64_t)tok * n_expert, bias, n_expert, top_k, scale, apply_scale, norm,
                 ids + (int64_t)tok * top_k, w + (int64_t)tok * top_k);
}

mx_status launch_route_select(const float *logits, const float *bias, int t, int n_expert, int top_k, float scale,
                              int apply_scale, int norm, uint32_t *ids, float *w, hipStream_t s) {
    if (t == 0) return MX_OK;
    hipLaunchKernelGGL(k_route_select, dim3(t), dim3(RT_THREADS), 0, s, logits, bias, n_expert, top_k, scale,
                       apply_scale, norm, ids, w);
    MX_LAUNCH("k_route_select");
    return MX_OK;
}

// ---- logits GEMM: [t,H] x [E,H]^T -> [t,E], f32 ---------------------------------------
// 64x64 output tile per block, 256 threads each computing a 4x4 micro-tile,
// K staged through LDS 32 at a time (both operands are K-contiguous).
constexpr int LG_T = 64, LG_E = 64, LG_K = 32;

__global__ void __launch_bounds__(256) k_route_logits(const float *__restrict__ x, const float *__restrict__ r,
                                                      int t, int hidden, int n_expert,
                                                      float *__restrict__ logits) {
    __shared__ float sx[LG_K][LG_T + 4];
    __shared__ float sr[LG_K][LG_E + 4];
    const int t0 = blockIdx.y * LG_T, e0 = blockIdx.x * LG_E;
    const int tid = threadIdx.x;
    const int ty = tid / 16, tx = tid % 16;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < hidden; k0 += LG_K) {
        for (int i = tid; i < LG_T * LG_K; i += 256) {
            const int tt = i / LG_K, kk = i % LG_K;
            const int tok = t0 + tt, kg = k0 + kk;
            sx[kk][tt] = (tok < t && kg < hidden) ? x[(int64_t)tok * hidden + kg] : 0.f;
        }
        for (int i = tid; i < LG_E * LG_K; i += 256) {
            const int ee = i / LG_K, kk = i % LG_K;
            const int e = e0 + ee, kg = k0 + kk;
            sr[kk][ee] = (kg < hidden && e < n_expert) ? r[(int64_t)e * hidden + kg] : 0.f;
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

mx_status launch_route_logits(const float *x, const float *router, int t, int hidden, int n_expert, float *logits,
                              hipStream_t s) {
    if (t == 0) return MX_OK;
    const dim3 grid((unsigned)((n_expert + LG_E - 1) / LG_E), (unsigned)((t + LG_T - 1) / LG_T));
    hipLaunchKernelGGL(k_route_logits, grid, dim3(256), 0, s, x, router, t, hidden, n_expert, logits);
    MX_LAUNCH("k_route_logits");
    return MX_OK;
}

// ---- fused decode router (t <= RF_MAX_T) ------------------------------------------------
// One wave per expert computes that expert's full logits (its router row is
// contiguous); block b covers experts [4b, 4b+4).  Optional RMSNorm of the token
// rows is folded in (every block recomputes the row statistics; block 0 writes
// the normalised rows for the expert kernels).  The last block to finish
// (device-scope counter in `ws`, self-resetting) runs the selection.
constexpr int RF_WAVES = 4;
constexpr int RF_MAX_T = 4;
constexpr int RF_VEC = 8;  // float4 per lane per load batch

size_t route_fused_ws_bytes(int t, int hidden, int n_expert) {
    (void)hidden;
    return 256 + (size_t)t * (size_t)n_expert * sizeof(float);
}

__global__ void __launch_bounds__(64 * RF_WAVES) k_route_fused(
    const float *__restrict__ x, const float *__restrict__ rms_alpha, float rms_eps, float *__restrict__ x_normed,
    const float *__restrict__ router, const float *__restrict__ bias, int t, int hidden, int n_expert, int top_k,
    float scale, int apply_scale, int norm, uint32_t *__restrict__ ids, float *__restrict__ w,
    uint8_t *__restrict__ ws) {
    __shared__ float s_red[RF_MAX_T][RF_WAVES];
    __shared__ float s_rms[RF_MAX_T];
    __shared__ int s_last;
    unsigned *counter = reinterpret_cast<unsigned *>(ws);
    float *logits = reinterpret_cast<float *>(ws + 256);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (rms_alpha) {
        for (int tok = 0; tok < t; tok++) {
            const float *xr = x + (int64_t)tok * hidden;
            float ss = 0.f;
            for (int i = 4 * tid; i < hidden; i += 4 * 64 * RF_WAVES) {
                const float4 v = *reinterpret_cast<const float4 *>(xr + i);
                ss = __builtin_fmaf(v.x, v.x, ss);
                ss = __builtin_fmaf(v.y, v.y, ss);
                ss = __builtin_fmaf(v.z, v.z, ss);
                ss = __builtin_fmaf(v.w, v.w, ss);
            }
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
            if (lane == 0) s_red[tok][wave] = ss;
        }
        __syncthreads();
        if (tid < t) {
            float tot = 0.f;
            for (int wv = 0; wv < RF_WAVES; wv++) tot += s_red[tid][wv];
            s_rms[tid] = sqrtf(tot / (float)hidden + rms_eps);
        }
        __syncthreads();
        if (blockIdx.x == 0 && x_normed) {
            for (int i = tid; i < t * hidden; i += 64 * RF_WAVES) {
                const int tok = i / hidden, h = i % hidden;
                x_normed[i] = x[i] / s_rms[tok] * rms_alpha[h];
            }
        }
    }
    const int e = blockIdx.x * RF_WAVES + wave;
    if (e < n_expert) {
        // all loads of a chunk (RF_VEC float4 per lane of the router row, the
        // token rows and the norm weight) are issued before any arithmetic
        const float *rr = router + (int64_t)e * hidden;
        float acc[RF_MAX_T] = {};
        for (int c0 = 4 * lane; c0 < hidden; c0 += 256 * RF_VEC) {
            float4 rv[RF_VEC], xv[RF_MAX_T][RF_VEC], al[RF_VEC];
#pragma unroll
            for (int i = 0; i < RF_VEC; i++) {
                const int h = c0 + 256 * i;
                const bool ok = h < hidden;
                rv[i] = ok ? *reinterpret_cast<const float4 *>(rr + h) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int tok = 0; tok < RF_MAX_T; tok++)
                    xv[tok][i] = (ok && tok < t) ? *reinterpret_cast<const float4 *>(x + (int64_t)tok * hidden + h)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
                if (rms_alpha) al[i] = ok ? *reinterpret_cast<const float4 *>(rms_alpha + h) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int tok = 0; tok < RF_MAX_T; tok++) {
                if (tok >= t) break;
                float a = acc[tok];
#pragma unroll
                for (int i = 0; i < RF_VEC; i++) {
                    float4 v = xv[tok][i];
                    if (rms_alpha) {
                        const float m = s_rms[tok];
                        v.x = v.x / m * al[i].x; v.y = v.y / m * al[i].y;
                        v.z = v.z / m * al[i].z; v.w = v.w / m * al[i].w;
                    }
                    a = __builtin_fmaf(v.x, rv[i].x, a);
                    a = __builtin_fmaf(v.y, rv[i].y, a);
                    a = __builtin_fmaf(v.z, rv[i].z, a);
                    a = __builtin_fmaf(v.w, rv[i].w, a);
                }
                acc[tok] = a;
            }
        }
        for (int tok = 0; tok < t; tok++) {
            float v = acc[tok];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == 0) st_agent(logits + (int64_t)tok * n_expert + e, v);
        }
    }
    // publish (completed agent-coherent stores), then count this block in
    drain_vmem();
    __syncthreads();
    if (tid == 0) s_last = arrive_last(counter, gridDim.x);
    __syncthreads();
    if (!s_last) return;  // block-uniform
    __shared__ float s_logit[RT_MAX_E];
    for (int tok = 0; tok < t; tok++) {
        for (int e2 = tid; e2 < n_expert; e2 += 64 * RF_WAVES) s_logit[e2] = ld_agent(logits + (int64_t)tok * n_expert + e2);
        __syncthreads();
        select_token(s_logit, bias, n_expert, top_k, scale, apply_scale, norm, ids + (int64_t)tok * top_k,
                     w + (int64_t)tok * top_k);
    }
    if (tid == 0) reset_counter(counter);
}

int route_fused_max_t() { return RF_MAX_T; }

mx_status launch_route_fused(const float *x, const float *rms_alpha, float rms_eps, float *x_normed,
                             const float *router, const float *bias, int t, int hidden, int n_expert, int top_k,
                             float scale, int apply_scale, int norm, uint32_t *ids, float *w, void *ws,
                             hipStream_t s) {
    if (t == 0) return MX_OK;
    if (t > RF_MAX_T) return fail(MX_ERR_SHAPE, "fused router handles at most %d tokens", RF_MAX_T);
    if (hidden % 4) return fail(MX_ERR_SHAPE, "fused router needs hidden %% 4 == 0");
    const dim3 grid((unsigned)((n_expert + RF_WAVES - 1) / RF_WAVES));
    hipLaunchKernelGGL(k_route_fused, grid, dim3(64 * RF_WAVES), 0, s, x, rms_alpha, rms_eps, x_normed, router,
                       bias, t, hidden, n_expert, top_k, scale, apply_scale, norm, ids, w,
                       reinterpret_cast<uint8_t *>(ws));
    MX_LAUNCH("k_route_fused");
    return MX_OK;
}

}  // namespace mx
