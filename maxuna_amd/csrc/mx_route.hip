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
#include "mx_stage.h"
#include "mx_f16row.h"
#include "mx_select.h"
#include "mx_dma.h"

namespace mx {

constexpr int RT_THREADS = SEL_THREADS;
static_assert(SEL_MAX_E == 1024 && SEL_MAX_K == 32, "route limits: n_expert <= 1024, top_k <= 32");

// Block-wide stable top-k for one token from its logits (mx_select.h).
// `logits` may be in shared or global memory; all RT_THREADS threads must call.
__device__ void select_token(const float *logits, const float *__restrict__ bias, int n_expert, int top_k,
                             float scale, int apply_scale, int norm, uint32_t *__restrict__ ids_out,
                             float *__restrict__ w_out) {
    __shared__ SelShared sh;
    uint64_t key[SEL_PER];
    float prob[SEL_PER];
#pragma unroll
    for (int j = 0; j < SEL_PER; j++) {
        const int e = threadIdx.x + SEL_THREADS * j;
        prob[j] = 0.f;
        key[j] = 0;
        if (e < n_expert) {
            const float ex = expf(-logits[e]);
            prob[j] = 1.0f / (ex + 1.0f);  // sigmoid (moe.rs:101)
            key[j] = sel_key(prob[j] + bias[e], e);
        }
    }
    topk_select(key, prob, n_expert, top_k, scale, apply_scale, norm, ids_out, w_out, sh);
}

// parts > 1: logits holds `parts` partial sums [parts][t][n_expert] over K
// (launch_route_logits_split), added in part order into the token's row first
__global__ void __launch_bounds__(RT_THREADS) k_route_select(const float *__restrict__ logits, int parts, int t,
                                                             const float *__restrict__ bias, int n_expert,
                                                             int top_k, float scale, int apply_scale, int norm,
                                                             uint32_t *__restrict__ ids, float *__restrict__ w) {
    __shared__ float s_row[SEL_MAX_E];
    const int tok = blockIdx.x;
    const float *row = logits + (int64_t)tok * n_expert;
    if (parts > 1) {
        for (int e = threadIdx.x; e < n_expert; e += RT_THREADS) {
            float v = row[e];
            for (int z = 1; z < parts; z++) v += row[(int64_t)z * t * n_expert + e];
            s_row[e] = v;
        }
        __syncthreads();
        row = s_row;
    }
    select_token(row, bias, n_expert, top_k, scale, apply_scale, norm, ids + (int64_t)tok * top_k,
                 w + (int64_t)tok * top_k);
}

mx_status launch_route_select(const float *logits, const float *bias, int t, int n_expert, int top_k, float scale,
                              int apply_scale, int norm, uint32_t *ids, float *w, hipStream_t s, int parts) {
    if (t == 0) return MX_OK;
    hipLaunchKernelGGL(k_route_select, dim3(t), dim3(RT_THREADS), 0, s, logits, parts, t, bias, n_expert, top_k,
                       scale, apply_scale, norm, ids, w);
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

// MFMA variant (hidden % 16 == 0): v_mfma_f32_32x32x2_f32, f32 products and sums.
// Block = 32 tokens x 64 experts; its 8 waves split K in 16-wide chunks
// (chunk c goes to wave c % 8) and the 8 partial tiles are summed in LDS in
// wave order.  Inside a chunk, lane half kh holds k = 8kh .. 8kh+7 and MFMA
// step s contracts k = s and 8 + s (the same permutation for both operands).
constexpr int RL_T = 32, RL_E = 64, RL_W = 8, RL_KC = 16;

__global__ void __launch_bounds__(64 * RL_W) k_route_logits_mfma(const float *__restrict__ x,
                                                                  const float *__restrict__ r, int t, int hidden,
                                                                  int n_expert, float *__restrict__ logits) {
    __shared__ float red[RL_W][RL_T * RL_E];
    const int t0 = blockIdx.y * RL_T, e0 = blockIdx.x * RL_E;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 31, kh = lane >> 5;
    const float *xr = x + (int64_t)min(t0 + i, t - 1) * hidden + 8 * kh;
    const float *ra = r + (int64_t)min(e0 + i, n_expert - 1) * hidden + 8 * kh;
    const float *rb = r + (int64_t)min(e0 + 32 + i, n_expert - 1) * hidden + 8 * kh;
    float16_t acc0, acc1;
#pragma unroll
    for (int q = 0; q < 16; q++) acc0[q] = acc1[q] = 0.f;
    const int nch = hidden / RL_KC;
    struct Chunk {
        float4 x0, x1, a0, a1, b0, b1;
    };
    auto load = [&](int c, Chunk &v) {
        const int64_t k = (int64_t)c * RL_KC;
        v.x0 = *reinterpret_cast<const float4 *>(xr + k);
        v.x1 = *reinterpret_cast<const float4 *>(xr + k + 4);
        v.a0 = *reinterpret_cast<const float4 *>(ra + k);
        v.a1 = *reinterpret_cast<const float4 *>(ra + k + 4);
        v.b0 = *reinterpret_cast<const float4 *>(rb + k);
        v.b1 = *reinterpret_cast<const float4 *>(rb + k + 4);
    };
    auto mma = [&](const Chunk &v) {
        const float xs[8] = {v.x0.x, v.x0.y, v.x0.z, v.x0.w, v.x1.x, v.x1.y, v.x1.z, v.x1.w};
        const float as[8] = {v.a0.x, v.a0.y, v.a0.z, v.a0.w, v.a1.x, v.a1.y, v.a1.z, v.a1.w};
        const float bs[8] = {v.b0.x, v.b0.y, v.b0.z, v.b0.w, v.b1.x, v.b1.y, v.b1.z, v.b1.w};
#pragma unroll
        for (int q = 0; q < 8; q++) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[q], as[q], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[q], bs[q], acc1, 0, 0, 0);
        }
    };
    Chunk c0, c1;
    int c = wave;
    if (c < nch) load(c, c0);
    while (c < nch) {
        if (c + RL_W < nch) load(c + RL_W, c1);
        mma(c0);
        c += RL_W;
        if (c >= nch) break;
        if (c + RL_W < nch) load(c + RL_W, c0);
        mma(c1);
        c += RL_W;
    }
    // acc[q] = D[token 8 (q / 4) + 4 kh + q % 4][expert i (+ 32)]
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int row = 8 * (q >> 2) + 4 * kh + (q & 3);
        red[wave][row * RL_E + i] = acc0[q];
        red[wave][row * RL_E + 32 + i] = acc1[q];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < RL_T * RL_E; o += 64 * RL_W) {
        float v = red[0][o];
#pragma unroll
        for (int w2 = 1; w2 < RL_W; w2++) v += red[w2][o];
        const int tok = t0 + o / RL_E, e = e0 + o % RL_E;
        if (tok < t && e < n_expert) logits[(int64_t)tok * n_expert + e] = v;
    }
}

// The same contraction with its operands staged through LDS (hidden % 128 == 0).
// Per 128-wide K stage the block's 32 x rows and 64 router rows (48 KB) are
// copied into LDS by global_load_lds, each copy instruction moving two whole
// 512-byte row slices (8 cache lines, where a lane-per-row register load
// touches 32), double-buffered so stage s + 1 is in flight while stage s is
// contracted (a third buffer measured slower: 50 against 47 us at C3).  Wave w contracts the stage's 16-wide chunk w, so chunk c of K
// still goes to wave c % 8 with the lane permutation of k_route_logits_mfma:
// the sums are the same operations in the same order, bit for bit.  The 16-byte
// chunks of a row are XOR-swizzled by row (position = chunk ^ (row & 31)), so
// the 32 lanes reading one chunk of 32 rows hit distinct banks.
#ifndef MX_RL_LDS
#define MX_RL_LDS 1
#endif
constexpr int RLL_KS = 128, RLL_ROWB = RLL_KS * 4, RLL_ROWS = RL_T + RL_E;   // 96 rows of 512 bytes
constexpr int RLL_STAGE = RLL_ROWS * RLL_ROWB, RLL_NI = RLL_STAGE / 1024;       // 48 KB, 48 copies
static_assert(RLL_NI % RL_W == 0, "copies split evenly over the waves");
static_assert(2 * RLL_STAGE >= RL_W * RL_T * RL_E * 4, "the reduction fits the staging buffers");

__global__ void __launch_bounds__(64 * RL_W) k_route_logits_lds(const float *__restrict__ x,
                                                                 const float *__restrict__ r, int t, int hidden,
                                                                 int n_expert, float *__restrict__ logits) {
    // split K (gridDim.z > 1, small grids): block z sums stages [z nst / Z, (z + 1) nst / Z)
    // into partial tile z of logits ([Z][t][n_expert]); the selection adds the parts
    // two separate objects: a copy into one buffer is not ordered against reads of the other
    __shared__ __attribute__((aligned(1024))) uint8_t sb0[RLL_STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t sb1[RLL_STAGE];
    const int t0 = blockIdx.y * RL_T, e0 = blockIdx.x * RL_E;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int i = lane & 31, kh = lane >> 5;
    // copy q of a stage moves LDS bytes [1024 q, 1024 q + 1024): rows 2q and 2q + 1
    // (0..31: x rows, 32..95: router rows); lane l writes position l & 31 of row
    // 2q + (l >> 5), which holds the row's chunk (l & 31) ^ (row & 31)
    const float *src[RLL_NI / RL_W];
#pragma unroll
    for (int u = 0; u < RLL_NI / RL_W; u++) {
        const int q = wave + RL_W * u, row = 2 * q + (lane >> 5);
        const int chunk = (lane & 31) ^ (row & 31);
        const float *base = row < RL_T ? x + (int64_t)min(t0 + row, t - 1) * hidden
                                       : r + (int64_t)min(e0 + row - RL_T, n_expert - 1) * hidden;
        src[u] = base + 4 * chunk;
    }
    auto issue = [&](int st, uint8_t *buf) {
#pragma unroll
        for (int u = 0; u < RLL_NI / RL_W; u++)
            dma16(reinterpret_cast<const uint8_t *>(src[u] + (int64_t)st * RLL_KS), buf + 1024 * (wave + RL_W * u));
        asm volatile("" ::: "memory");
    };
    // this lane's operand addresses inside a stage: chunks 4w + 2kh and 4w + 2kh + 1
    // of its x row i and router rows i and 32 + i
    auto pos = [&](int row, int c) { return row * RLL_ROWB + 16 * (c ^ (row & 31)); };
    const int c0 = 4 * wave + 2 * kh;
    const int ax0 = pos(i, c0), ax1 = pos(i, c0 + 1);
    const int aa0 = pos(RL_T + i, c0), aa1 = pos(RL_T + i, c0 + 1);
    const int ab0 = pos(RL_T + 32 + i, c0), ab1 = pos(RL_T + 32 + i, c0 + 1);
    float16_t acc0, acc1;
#pragma unroll
    for (int q = 0; q < 16; q++) acc0[q] = acc1[q] = 0.f;
    const int nst = hidden / RLL_KS / (int)gridDim.z;  // stages of this block (the launcher checks divisibility)
    {
        const int64_t k0 = (int64_t)blockIdx.z * nst * RLL_KS;
#pragma unroll
        for (int u = 0; u < RLL_NI / RL_W; u++) src[u] += k0;
        logits += (int64_t)blockIdx.z * t * n_expert;
    }
    // stage st from cur while stage st + 1 is copied into nxt; the loop is unrolled
    // by two so each buffer is a compile-time object (a runtime choice between
    // them makes the compiler wait for every copy before any LDS read)
    auto step = [&](int st, const uint8_t *cur, uint8_t *nxt) {
        wait_vmcnt(0);    // this wave's copies of stage st have landed
        __syncthreads();  // every wave's copies have; every read of nxt (stage st - 1) is done
        if (st + 1 < nst) issue(st + 1, nxt);
        const float4 x0 = *reinterpret_cast<const float4 *>(cur + ax0), x1 = *reinterpret_cast<const float4 *>(cur + ax1);
        const float4 a0 = *reinterpret_cast<const float4 *>(cur + aa0), a1 = *reinterpret_cast<const float4 *>(cur + aa1);
        const float4 b0 = *reinterpret_cast<const float4 *>(cur + ab0), b1 = *reinterpret_cast<const float4 *>(cur + ab1);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float as[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int q = 0; q < 8; q++) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[q], as[q], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[q], bs[q], acc1, 0, 0, 0);
        }
    };
    issue(0, sb0);
    for (int st = 0; st < nst; st += 2) {
        step(st, sb0, sb1);
        if (st + 1 < nst) step(st + 1, sb1, sb0);
    }
    __syncthreads();  // the staging buffers now hold the wave partials
    // the wave partials [RL_W][RL_T * RL_E] over sb0 | sb1
    static_assert(RLL_STAGE % (RL_T * RL_E * 4) == 0, "wave partial tiles do not straddle the buffers");
    auto red_at = [&](int w2) -> float * {
        const int per = RLL_STAGE / (RL_T * RL_E * 4);
        return reinterpret_cast<float *>(w2 < per ? sb0 : sb1) + (w2 % per) * (RL_T * RL_E);
    };
    // acc[q] = D[token 8 (q / 4) + 4 kh + q % 4][expert i (+ 32)]
    float *mine = red_at(wave);
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const int row = 8 * (q >> 2) + 4 * kh + (q & 3);
        mine[row * RL_E + i] = acc0[q];
        mine[row * RL_E + 32 + i] = acc1[q];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < RL_T * RL_E; o += 64 * RL_W) {
        float v = red_at(0)[o];
#pragma unroll
        for (int w2 = 1; w2 < RL_W; w2++) v += red_at(w2)[o];
        const int tok = t0 + o / RL_E, e = e0 + o % RL_E;
        if (tok < t && e < n_expert) logits[(int64_t)tok * n_expert + e] = v;
    }
}

// Few tokens (t < RLR_T): one block per expert; its 256 threads split the
// expert's router row (and the same columns of the token rows), then reduce
// through DPP and LDS.  The tiled kernels give a 256-expert router at t = 1 only
// four blocks (1.5 ms at hidden 7168).
constexpr int RLR_T = 8;
__global__ void __launch_bounds__(256) k_route_logits_rows(const float *__restrict__ x, const float *__restrict__ r,
                                                           int t, int hidden, int n_expert,
                                                           float *__restrict__ logits) {
    __shared__ float s_red[RLR_T][4];
    const int e = blockIdx.x, tid = threadIdx.x;
    const float *re = r + (int64_t)e * hidden;
    float dot[RLR_T] = {};
    for (int h = 4 * tid; h < hidden; h += 4 * 256) {
        const float4 rv = *reinterpret_cast<const float4 *>(re + h);
#pragma unroll
        for (int j = 0; j < RLR_T; j++) {
            if (j < t) {  // (block-uniform)
                const float4 v = *reinterpret_cast<const float4 *>(x + (int64_t)j * hidden + h);
                dot[j] = __builtin_fmaf(v.x, rv.x, dot[j]);
                dot[j] = __builtin_fmaf(v.y, rv.y, dot[j]);
                dot[j] = __builtin_fmaf(v.z, rv.z, dot[j]);
                dot[j] = __builtin_fmaf(v.w, rv.w, dot[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < RLR_T; j++) {
        if (j < t) {
            const float a = warp_sum_width(dot[j], 64);
            if ((tid & 63) == 0) s_red[j][tid >> 6] = a;
        }
    }
    __syncthreads();
    if (tid < t) {
        const float *sr = s_red[0] + 4 * tid;  // (row tid of s_red)
        logits[(int64_t)tid * n_expert + e] = ((sr[0] + sr[1]) + sr[2]) + sr[3];
    }
}

mx_status launch_route_logits(const float *x, const float *router, int t, int hidden, int n_expert, float *logits,
                              hipStream_t s) {
    if (t == 0) return MX_OK;
    if (t < RLR_T && hidden % 4 == 0) {
        hipLaunchKernelGGL(k_route_logits_rows, dim3((unsigned)n_expert), dim3(256), 0, s, x, router, t, hidden,
                           n_expert, logits);
        MX_LAUNCH("k_route_logits_rows");
        return MX_OK;
    }
    if (MX_RL_LDS && hidden % RLL_KS == 0 && t >= 8) {
        const dim3 grid((unsigned)((n_expert + RL_E - 1) / RL_E), (unsigned)((t + RL_T - 1) / RL_T), 1u);
        hipLaunchKernelGGL(k_route_logits_lds, grid, dim3(64 * RL_W), 0, s, x, router, t, hidden, n_expert, logits);
        MX_LAUNCH("k_route_logits_lds");
        return MX_OK;
    }
    if (hidden % RL_KC == 0 && t >= 8) {
        const dim3 grid((unsigned)((n_expert + RL_E - 1) / RL_E), (unsigned)((t + RL_T - 1) / RL_T));
        hipLaunchKernelGGL(k_route_logits_mfma, grid, dim3(64 * RL_W), 0, s, x, router, t, hidden, n_expert, logits);
        MX_LAUNCH("k_route_logits_mfma");
        return MX_OK;
    }
    const dim3 grid((unsigned)((n_expert + LG_E - 1) / LG_E), (unsigned)((t + LG_T - 1) / LG_T));
    hipLaunchKernelGGL(k_route_logits, grid, dim3(256), 0, s, x, router, t, hidden, n_expert, logits);
    MX_LAUNCH("k_route_logits");
    return MX_OK;
}

#ifndef MX_RL_SPLIT
#define MX_RL_SPLIT 1
#endif
int route_logits_splits(int t, int hidden, int n_expert) {
    if (!MX_RL_SPLIT || !MX_RL_LDS || hidden % RLL_KS || t < RLR_T) return 1;
    const int64_t blocks = (int64_t)((n_expert + RL_E - 1) / RL_E) * ((t + RL_T - 1) / RL_T);
    int z = 1;
    while (z < 8 && blocks * z * 2 <= 256 && (hidden / RLL_KS) % (z * 2) == 0) z *= 2;
    return z;
}

mx_status launch_route_logits_split(const float *x, const float *router, int t, int hidden, int n_expert,
                                    float *parts, int splits, hipStream_t s) {
    if (t == 0) return MX_OK;
    if (splits == 1) return launch_route_logits(x, router, t, hidden, n_expert, parts, s);
    if (splits != route_logits_splits(t, hidden, n_expert))
        return fail(MX_ERR_SHAPE, "route logits: %d K splits do not fit this shape", splits);
    const dim3 grid((unsigned)((n_expert + RL_E - 1) / RL_E), (unsigned)((t + RL_T - 1) / RL_T), (unsigned)splits);
    hipLaunchKernelGGL(k_route_logits_lds, grid, dim3(64 * RL_W), 0, s, x, router, t, hidden, n_expert, parts);
    MX_LAUNCH("k_route_logits_lds");
    return MX_OK;
}

// ---- decode router, logits half (t <= RF_TOKENS) ----------------------------------------
// Blocks [0, n_expert): one expert each.  Its 256 threads split the expert's
// router row (contiguous in the GGUF layout) and the token rows, so every
// logit costs one memory round trip.  Optional RMSNorm is folded in: the block
// reduces sum(x^2) alongside the dot product and forms
//   logit = sum(x * alpha * r) / sqrt(mean(x^2) + eps).
// The block turns the logit into the expert's sigmoid probability and its
// stable-sort key (bias added for selection only) and stores both in `ws`;
// the top-k runs in the next kernel on the stream (k_decode_select in
// mx_mv.hip), which sees these stores at the kernel boundary.  Selecting in a
// last-arriving block instead costs a device-scope publish + atomic round trip
// per block (measured: 3.5 us more than a kernel boundary on MI355X).
// Blocks [n_expert, n_expert + n_stage): stage the (normalised) token rows for
// the expert kernels (mx_stage.h layout, one row of xstage_bytes(hidden) per
// token in `xstage`) and, if requested, write them as f32 to `x_normed`.
// Then, when x16 is given (no RMSNorm), one block per token writes its row as
// f16 times a power of two (mx_f16row.h) for the MFMA verify tiles.
constexpr int RF_MAX_T = 4;     // tokens per register pass
#ifndef MX_RF_TOKENS
#define MX_RF_TOKENS 128
#endif
// tokens per launch: up to 128 the per-expert blocks beat the MFMA logits
// kernel, whose few 32-token x 64-expert tiles leave most CUs idle at these t
// (C1-shaped layer on the verify tiles, µs: t = 40: 451 -> 428, 64: 505 -> 485,
// 96: 568 -> 550, 128: 627 -> 614; from 160 on equal)
constexpr int RF_TOKENS = MX_RF_TOKENS;
constexpr int RF_THREADS = 256;
constexpr int RF_UNROLL = 4;  // float4 loads per thread per pass

// ws: keys u64 [t][E] | probs f32 [t][E]
size_t route_fused_ws_bytes(int t, int hidden, int n_expert) {
    (void)hidden;
    return (size_t)t * (size_t)n_expert * (sizeof(uint64_t) + sizeof(float));
}

// Normalised token value block: x / m * alpha (alpha == NULL: x as is).
__device__ __forceinline__ void norm8(float (&v)[8], const float *alpha, int h0, float m) {
    if (!alpha) return;
    float a[8];
    load8f(alpha + h0, a);
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = v[i] / m * a[i];
}

// Block-wide sum of the first t partials (all threads call).  The loops run over
// all N with a block-uniform guard, so v stays in registers (a loop bounded by t
// indexes it with a variable, which puts it in scratch memory).
template <int N>
__device__ __forceinline__ void block_sums(float (&v)[N], int t, float (*s_red)[RF_THREADS / 64]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int tok = 0; tok < N; tok++) {
        if (tok < t) {
            float a = v[tok];
            a = warp_sum_width(a, 64);
            if (lane == 0) s_red[tok][wave] = a;
        }
    }
    __syncthreads();
#pragma unroll
    for (int tok = 0; tok < N; tok++) {
        if (tok < t) {
            float a = 0.f;
            for (int wv = 0; wv < RF_THREADS / 64; wv++) a += s_red[tok][wv];
            v[tok] = a;
        }
    }
    __syncthreads();
}

// v[i] for a lane-dependent i < N without indexing the array: a register array
// read at a per-lane index lives in scratch memory, and a chain of selects is
// folded back into such a read by the compiler, so the bits are masked and OR-ed
template <int N> __device__ __forceinline__ float pick(const float (&v)[N], int i) {
    uint32_t r = 0;
#pragma unroll
    for (int k = 0; k < N; k++) r |= __float_as_uint(v[k]) & (0u - (uint32_t)(i == k));
    return __uint_as_float(r);
}

// EPB: experts per expert block (1, or 4 for t > RF_MAX_T: the block's token
// rows, loaded once, serve four router rows, and a 16-token block runs 256
// expert blocks instead of 1024).  Every logit is the same sum in the same
// order for any EPB (each thread's partial over the same columns, then the same
// block reduction).
template <int EPB>
__global__ void __launch_bounds__(RF_THREADS) k_route_fused(
    const float *__restrict__ x, const float *__restrict__ rms_alpha, float rms_eps, float *__restrict__ x_normed,
    const float *__restrict__ router, const float *__restrict__ bias, int t, int hidden, int n_expert,
    uint8_t *__restrict__ ws, uint8_t *__restrict__ xstage, uint8_t *__restrict__ xstage_gm,
    _Float16 *__restrict__ x16, float *__restrict__ x16s, int n_stage) {
    __shared__ float s_red[EPB * RF_MAX_T][RF_THREADS / 64];
    uint64_t *keys = reinterpret_cast<uint64_t *>(ws);
    float *probs = reinterpret_cast<float *>(keys + (int64_t)t * n_expert);
    const int tid = threadIdx.x;
    // expert blocks: one per (EPB experts, group of RF_MAX_T tokens), each one register pass
    const int n_eg = n_expert / EPB;
    const int n_tg = (t + RF_MAX_T - 1) / RF_MAX_T, n_eb = n_eg * n_tg;
    if ((int)blockIdx.x >= n_eb + n_stage) {
        // ---- f16 row blocks: token row -> f16 times a power of two (x16 != NULL,
        // no RMSNorm), the operand of the MFMA verify tiles
        const int tok = blockIdx.x - n_eb - n_stage;
        // (in the Q4_K verify tiles' K order: the only reader)
        if (hidden <= 4096)
            f16_row<4, true>(x + (int64_t)tok * hidden, hidden, x16 + (int64_t)tok * hidden, x16s + tok, &s_red[0][0]);
        else f16_row<0, true>(x + (int64_t)tok * hidden, hidden, x16 + (int64_t)tok * hidden, x16s + tok, &s_red[0][0]);
        return;
    }
    if ((int)blockIdx.x >= n_eb) {
        // ---- staging blocks: quarter qi = 8 values of token qi / nq
        __shared__ float s_m[RF_THREADS * 8 / 32 + 2];  // the RMS of the block's tokens (hidden >= 32)
        const int nq = hidden / 8;
        const int qi0 = (blockIdx.x - n_eb) * RF_THREADS;
        const int qi = qi0 + tid;
        const int tok = qi / nq, q = qi % nq;
        const bool valid = tok < t;
        const int ta = qi0 / nq, tb = min(t - 1, (qi0 + RF_THREADS - 1) / nq);
        if (rms_alpha) {  // RMS of the tokens this block touches, RF_MAX_T at a time (block-uniform loop)
            for (int t0 = ta; t0 <= tb; t0 += RF_MAX_T) {
                const int tc = min(RF_MAX_T, tb - t0 + 1);
                float ss[RF_MAX_T] = {};
                for (int h = 4 * tid; h < hidden; h += 4 * RF_THREADS) {
#pragma unroll
                    for (int k = 0; k < RF_MAX_T; k++) {
                        if (k < tc) {  // (block-uniform; a loop bounded by tc put ss in scratch)
                            const float4 v = *reinterpret_cast<const float4 *>(x + (int64_t)(t0 + k) * hidden + h);
                            ss[k] = __builtin_fmaf(v.x, v.x, ss[k]);
                            ss[k] = __builtin_fmaf(v.y, v.y, ss[k]);
                            ss[k] = __builtin_fmaf(v.z, v.z, ss[k]);
                            ss[k] = __builtin_fmaf(v.w, v.w, ss[k]);
                        }
                    }
                }
                block_sums(ss, tc, s_red);
                if (tid < tc) s_m[t0 - ta + tid] = sqrtf(pick(ss, tid) / (float)hidden + rms_eps);
            }
            __syncthreads();
        }
        float v[8] = {};
        if (valid) {
            load8f(x + (int64_t)tok * hidden + 8 * q, v);
            if (rms_alpha) norm8(v, rms_alpha, 8 * q, s_m[tok - ta]);
            if (x_normed) {
                float4 *o = reinterpret_cast<float4 *>(x_normed + (int64_t)tok * hidden + 8 * q);
                o[0] = make_float4(v[0], v[1], v[2], v[3]);
                o[1] = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
        if (xstage)
            stage_quarter(v, q, valid, xstage + (int64_t)(valid ? tok : 0) * xstage_stride(hidden), hidden,
                          xstage_gm ? xstage_gm + (int64_t)(valid ? tok : 0) * xstage_gm_stride(hidden) : nullptr);
        return;
    }
    // ---- expert blocks: the experts' router rows against their group of RF_MAX_T
    // tokens (the groups of one expert read the row from L2 after the first)
    const int e0 = (blockIdx.x % n_eg) * EPB, tg = blockIdx.x / n_eg;
    float be[EPB];  // issued early: needed only after the reduction
#pragma unroll
    for (int k = 0; k < EPB; k++) be[k] = bias[e0 + k];
    for (int t0 = tg * RF_MAX_T; t0 < min(t, (tg + 1) * RF_MAX_T); t0 += RF_MAX_T) {
        const int tc = min(RF_MAX_T, t - t0);
        const float *xt = x + (int64_t)t0 * hidden;
        float dot[EPB * RF_MAX_T] = {}, ss[RF_MAX_T] = {};
        for (int c0 = 4 * tid; c0 < hidden; c0 += 4 * RF_THREADS * RF_UNROLL) {
            float4 rv[EPB][RF_UNROLL], av[RF_UNROLL], xv[RF_MAX_T][RF_UNROLL];
#pragma unroll
            for (int i = 0; i < RF_UNROLL; i++) {
                const int h = c0 + 4 * RF_THREADS * i;
                const bool ok = h < hidden;
                // (values selected after the loads: a select between a load's address
                // and a local's put the local in scratch memory)
#pragma unroll
                for (int k = 0; k < EPB; k++) {
                    rv[k][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (ok) rv[k][i] = *reinterpret_cast<const float4 *>(router + (int64_t)(e0 + k) * hidden + h);
                }
                av[i] = make_float4(1.f, 1.f, 1.f, 1.f);
                if (ok && rms_alpha) av[i] = *reinterpret_cast<const float4 *>(rms_alpha + h);
#pragma unroll
                for (int j = 0; j < RF_MAX_T; j++) {
                    xv[j][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (ok && j < tc) xv[j][i] = *reinterpret_cast<const float4 *>(xt + (int64_t)j * hidden + h);
                }
            }
#pragma unroll
            for (int j = 0; j < RF_MAX_T; j++) {
                if (j >= tc) continue;  // (block-uniform)
#pragma unroll
                for (int i = 0; i < RF_UNROLL; i++) {
                    const float4 v = xv[j][i];
                    ss[j] = __builtin_fmaf(v.x, v.x, ss[j]);
                    ss[j] = __builtin_fmaf(v.y, v.y, ss[j]);
                    ss[j] = __builtin_fmaf(v.z, v.z, ss[j]);
                    ss[j] = __builtin_fmaf(v.w, v.w, ss[j]);
#pragma unroll
                    for (int k = 0; k < EPB; k++) {
                        float &d = dot[k * RF_MAX_T + j];
                        d = __builtin_fmaf(v.x * av[i].x, rv[k][i].x, d);
                        d = __builtin_fmaf(v.y * av[i].y, rv[k][i].y, d);
                        d = __builtin_fmaf(v.z * av[i].z, rv[k][i].z, d);
                        d = __builtin_fmaf(v.w * av[i].w, rv[k][i].w, d);
                    }
                }
            }
        }
        block_sums(dot, EPB * RF_MAX_T, s_red);
        if (rms_alpha) block_sums(ss, tc, s_red);
        const int k = tid / RF_MAX_T, j = tid % RF_MAX_T;
        if (k < EPB && j < tc) {
            const float d = pick(dot, k * RF_MAX_T + j);
            const float lg = rms_alpha ? d / sqrtf(pick(ss, j) / (float)hidden + rms_eps) : d;
            const float p = 1.0f / (expf(-lg) + 1.0f);  // sigmoid (moe.rs:101)
            const int64_t o = (int64_t)(t0 + j) * n_expert + e0 + k;
            keys[o] = sel_key(p + pick(be, k), e0 + k);
            probs[o] = p;
        }
    }
}

int route_fused_max_t() { return RF_TOKENS; }

mx_status launch_route_fused(const float *x, const float *rms_alpha, float rms_eps, float *x_normed,
                             const float *router, const float *bias, int t, int hidden, int n_expert, void *ws,
                             uint8_t *xstage, uint8_t *xstage_gm, hipStream_t s, _Float16 *x16, float *x16s) {
    if (t == 0) return MX_OK;
    if (t > RF_TOKENS) return fail(MX_ERR_SHAPE, "fused router handles at most %d tokens", RF_TOKENS);
    if (hidden % 32) return fail(MX_ERR_SHAPE, "fused router needs hidden %% 32 == 0");
    if (xstage_gm && hidden % 64) return fail(MX_ERR_SHAPE, "group-major staging needs hidden %% 64 == 0");
    if (x16 && (rms_alpha || !x16s || hidden % 4))
        return fail(MX_ERR_SHAPE, "fused router f16 rows: no RMSNorm, a scale array and hidden %% 4 == 0");
    const int n_x16 = x16 ? t : 0;
    const int nq = t * (hidden / 8);
    const int n_stage = (xstage || x_normed) ? (nq + RF_THREADS - 1) / RF_THREADS : 0;
    const int n_tg = (t + RF_MAX_T - 1) / RF_MAX_T;
    if (t > RF_MAX_T && n_expert % 4 == 0)
        hipLaunchKernelGGL(k_route_fused<4>, dim3((unsigned)(n_expert / 4 * n_tg + n_stage + n_x16)), dim3(RF_THREADS),
                           0, s, x, rms_alpha, rms_eps, x_normed, router, bias, t, hidden, n_expert,
                           reinterpret_cast<uint8_t *>(ws), xstage, xstage_gm, x16, x16s, n_stage);
    else
        hipLaunchKernelGGL(k_route_fused<1>, dim3((unsigned)(n_expert * n_tg + n_stage + n_x16)), dim3(RF_THREADS), 0,
                           s, x, rms_alpha, rms_eps, x_normed, router, bias, t, hidden, n_expert,
                           reinterpret_cast<uint8_t *>(ws), xstage, xstage_gm, x16, x16s, n_stage);
    MX_LAUNCH("k_route_fused");
    return MX_OK;
}

// ---- activation staging for the decode expert kernels (rows of t tokens) ---------------
__global__ void __launch_bounds__(256) k_stage_rows(const float *__restrict__ x, int t, int k,
                                                    uint8_t *__restrict__ xstage, uint8_t *__restrict__ xstage_gm) {
    const int nq = k / 8;
    const int qi = blockIdx.x * 256 + threadIdx.x;
    const int tok = qi / nq, q = qi % nq;
    const bool valid = tok < t;
    float v[8] = {};
    if (valid) load8f(x + (int64_t)tok * k + 8 * q, v);
    stage_quarter(v, q, valid, xstage + (int64_t)(valid ? tok : 0) * xstage_stride(k), k,
                  xstage_gm ? xstage_gm + (int64_t)(valid ? tok : 0) * xstage_gm_stride(k) : nullptr);
}

size_t stage_row_bytes(int k) { return (size_t)xstage_stride(k); }

mx_status launch_stage_rows(const float *x, int t, int k, uint8_t *xstage, uint8_t *xstage_gm, hipStream_t s) {
    if (t == 0) return MX_OK;
    if (k % 32) return fail(MX_ERR_SHAPE, "staging needs k %% 32 == 0");
    if (xstage_gm && k % 64) return fail(MX_ERR_SHAPE, "group-major staging needs k %% 64 == 0");
    const int64_t nq = (int64_t)t * (k / 8);
    hipLaunchKernelGGL(k_stage_rows, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, x, t, k, xstage, xstage_gm);
    MX_LAUNCH("k_stage_rows");
    return MX_OK;
}

}  // namespace mx
