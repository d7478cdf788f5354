// Elementwise glue of the MoE block: SwiGLU activation, weighted combine,
// RMSNorm.  f32 throughout, each operation rounded on its own (the library is
// compiled with -ffp-contract=off).
#include "mx_launch.h"

namespace mx {

// act = silu(g) * u, silu(g) = g / (1 + exp(-g))  (silu_mul.metal:57-72)
__global__ void __launch_bounds__(256) k_silu_mul(const float *__restrict__ g,
                                                  const float *__restrict__ u, int64_t n,
                                                  float *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    const float s = gv / (1.0f + expf(-gv));
    dst[i] = s * u[i];
}

mx_status launch_silu_mul(const float *g, const float *u, int64_t n, float *dst, hipStream_t s) {
    if (n == 0) return MX_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, n, dst);
    MX_LAUNCH("k_silu_mul");
    return MX_OK;
}

// dst[s,c] = sum_k down[s,k,c] * w[s,k], k in slot order (combine.metal:70-97);
// rescale form ((down * l2) * 2^-15) * w (combine.metal:102-133).
__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ down,
                                                 const float *__restrict__ l2,
                                                 const float *__restrict__ w, int seq, int top_k,
                                                 int n_out, float *__restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)seq * n_out) return;
    const int s = (int)(i / n_out), c = (int)(i % n_out);
    float acc = 0.f;
    for (int k = 0; k < top_k; k++) {
        float d = down[((int64_t)s * top_k + k) * n_out + c];
        if (l2) {
            d = d * l2[s * top_k + k];
            d = d * (1.0f / 32768.0f);
        }
        acc = acc + d * w[s * top_k + k];
    }
    dst[i] = acc;
}

mx_status launch_combine(const float *down, const float *col_l2, const float *w, int seq,
                         int top_k, int n_out, float *dst, hipStream_t s) {
    const int64_t n = (int64_t)seq * n_out;
    if (n == 0) return MX_OK;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, down, col_l2,
                       w, seq, top_k, n_out, dst);
    MX_LAUNCH("k_combine");
    return MX_OK;
}

// dst = x / sqrt(mean(x^2) + eps) * alpha, one block per row.
__global__ void __launch_bounds__(256) k_rms_norm(const float *__restrict__ x,
                                                  const float *__restrict__ alpha, int dim,
                                                  float eps, float *__restrict__ dst) {
    __shared__ float s_red[4];
    __shared__ float s_m;
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (int64_t)row * dim;
    float ss = 0.f;
    for (int i = tid; i < dim; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if ((tid & 63) == 0) s_red[tid >> 6] = ss;
    __syncthreads();
    if (tid == 0) s_m = sqrtf((((s_red[0] + s_red[1]) + s_red[2]) + s_red[3]) / (float)dim + eps);
    __syncthreads();
    const float m = s_m;
    for (int i = tid; i < dim; i += 256) dst[(int64_t)row * dim + i] = xr[i] / m * alpha[i];
}

mx_status launch_rms_norm(const float *x, const float *alpha, int rows, int dim, float eps,
                          float *dst, hipStream_t s) {
    if (rows == 0) return MX_OK;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(256), 0, s, x, alpha, dim, eps, dst);
    MX_LAUNCH("k_rms_norm");
    return MX_OK;
}

// dst = (a + b) + c, c optional (residual + (routed + shared)).
__global__ void __launch_bounds__(256) k_add3(const float *a, const float *b, const float *c,
                                              int64_t n, float *dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = a[i] + b[i];
    if (c) v = c[i] + v;
    dst[i] = v;
}

mx_status launch_add3(const float *a, const float *b, const float *c, int64_t n, float *dst,
                      hipStream_t s) {
    if (n == 0) return MX_OK;
    hipLaunchKernelGGL(k_add3, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, b, c, n, dst);
    MX_LAUNCH("k_add3");
    return MX_OK;
}

// Routing-id validation: flags = (1 if some token repeats an id across its
// top_k slots) | (2 if some id >= n_expert).  Up to CHECK_ONE_BLOCK pairs one
// block walks every token and writes the flag word once by a plain store (no
// clearing launch, no atomics).  Larger batches: a grid of blocks, one token per
// thread, each block ORing its flags (when set) into the word that a one-thread
// launch cleared first.
constexpr int64_t CHECK_ONE_BLOCK = 1 << 16;

__device__ __forceinline__ uint32_t check_token(const uint32_t *__restrict__ r, int top_k, uint32_t n_expert) {
    uint32_t f = 0;
    for (int a = 0; a < top_k; a++) {
        const uint32_t ia = r[a];
        if (ia >= n_expert) f |= 2u;
        for (int b = a + 1; b < top_k; b++)
            if (r[b] == ia) f |= 1u;
    }
    return f;
}

// OR of f over the block, valid in thread 0
__device__ __forceinline__ uint32_t block_or(uint32_t f, uint32_t *s_f) {
    for (int off = 32; off > 0; off >>= 1) f |= (uint32_t)__shfl_xor((int)f, off, 64);
    if ((threadIdx.x & 63) == 0) s_f[threadIdx.x >> 6] = f;
    __syncthreads();
    uint32_t v = 0;
    if (threadIdx.x == 0)
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) v |= s_f[i];
    return v;
}

__global__ void __launch_bounds__(1024) k_check_ids(const uint32_t *__restrict__ ids, int64_t t, int top_k,
                                                    uint32_t n_expert, uint32_t *__restrict__ flags) {
    __shared__ uint32_t s_f[16];
    uint32_t f = 0;
    for (int64_t tok = threadIdx.x; tok < t; tok += blockDim.x) f |= check_token(ids + tok * top_k, top_k, n_expert);
    const uint32_t v = block_or(f, s_f);
    if (threadIdx.x == 0) *flags = v;
}

__global__ void k_check_ids_clear(uint32_t *flags) { *flags = 0u; }

__global__ void __launch_bounds__(256) k_check_ids_grid(const uint32_t *__restrict__ ids, int64_t t, int top_k,
                                                        uint32_t n_expert, uint32_t *__restrict__ flags) {
    __shared__ uint32_t s_f[4];
    const int64_t tok = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const uint32_t f = tok < t ? check_token(ids + tok * top_k, top_k, n_expert) : 0u;
    const uint32_t v = block_or(f, s_f);
    if (threadIdx.x == 0 && v) atomicOr(flags, v);
}

mx_status launch_check_ids(const uint32_t *ids, int64_t t, int top_k, int n_expert, uint32_t *flags,
                           hipStream_t s) {
    if (t * top_k <= CHECK_ONE_BLOCK) {
        hipLaunchKernelGGL(k_check_ids, dim3(1), dim3(1024), 0, s, ids, t, top_k, (uint32_t)n_expert, flags);
        MX_LAUNCH("k_check_ids");
        return MX_OK;
    }
    hipLaunchKernelGGL(k_check_ids_clear, dim3(1), dim3(1), 0, s, flags);
    MX_LAUNCH("k_check_ids_clear");
    hipLaunchKernelGGL(k_check_ids_grid, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, s, ids, t, top_k,
                       (uint32_t)n_expert, flags);
    MX_LAUNCH("k_check_ids_grid");
    return MX_OK;
}

// ---- plain streaming read (bench probe of the achievable HBM read rate) ---------------
// Every thread reads 16-byte words strided by the grid, four loads in flight,
// and folds them into one word that is stored only if it matches an impossible
// value (so the loads are not optimised away).  512 workgroups of 256 threads
// measured fastest for 57-512 MB reads on MI355X.
__global__ void __launch_bounds__(256) k_read_probe(const uint4 *__restrict__ p, int64_t n16,
                                                    uint32_t *__restrict__ sink) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t st = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    for (; i + 3 * st < n16; i += 4 * st) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = p[i + u * st];
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += st) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) *sink = acc;
}

mx_status launch_read_probe(const void *src, int64_t nbytes, uint32_t *sink, hipStream_t s) {
    if (nbytes <= 0) return MX_OK;
    hipLaunchKernelGGL(k_read_probe, dim3(512), dim3(256), 0, s, reinterpret_cast<const uint4 *>(src), nbytes / 16,
                       sink);
    MX_LAUNCH("k_read_probe");
    return MX_OK;
}

}  // namespace mx
