// Bit-exact dequantisation of raw GGUF blocks, and the seeded synthetic block
// generator used by tests and the benchmark.
//
// Dequantisation restates the GGUF formulas the reference dequantises with
// (candle QTensor::dequantize, moe.rs:173-175; block math mm_id.metal:75-167):
//   Q4_K  y = fl(fl(d*sc) * q) - fl(dmin*m)      (one rounding per op)
//   Q5_K  the same, q = low nibble + 16 * high bit (bit 2i + h of qh[l])
//   Q6_K  y = fl(fl(d*sc) * (q - 32))
//   Q8_0  y = fl(q * d)
// This file is compiled with -ffp-contract=off, so no product/difference pair
// is fused into an FMA.
#include "mx_launch.h"
#include "mx_deq.h"

namespace mx {

// One thread per 32 consecutive output weights of one block.
template <int DT>
__global__ void __launch_bounds__(256) k_dequantize(const uint8_t *__restrict__ blocks,
                                                    int64_t n_chunks,
                                                    float *__restrict__ out) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n_chunks) return;
    constexpr int CPB = block_size(DT) / 32;  // 32-weight chunks per block
    const int64_t b = c / CPB;
    float y[32];
    dequant_chunk<DT>(blocks + b * type_size(DT), (int)(c % CPB), y);
    float4 *o = reinterpret_cast<float4 *>(out + 32 * c);
#pragma unroll
    for (int w = 0; w < 8; w++) o[w] = make_float4(y[4 * w], y[4 * w + 1], y[4 * w + 2], y[4 * w + 3]);
}

mx_status launch_dequantize(int dtype, const uint8_t *blocks, int64_t n, float *out,
                            hipStream_t s) {
    const int64_t chunks = n / 32;
    if (chunks == 0) return MX_OK;
    const dim3 grid((unsigned)((chunks + 255) / 256));
    switch (dtype) {
    case kQ4_K: hipLaunchKernelGGL(k_dequantize<kQ4_K>, grid, dim3(256), 0, s, blocks, chunks, out); break;
    case kQ5_K: hipLaunchKernelGGL(k_dequantize<kQ5_K>, grid, dim3(256), 0, s, blocks, chunks, out); break;
    case kQ6_K: hipLaunchKernelGGL(k_dequantize<kQ6_K>, grid, dim3(256), 0, s, blocks, chunks, out); break;
    default: hipLaunchKernelGGL(k_dequantize<kQ8_0>, grid, dim3(256), 0, s, blocks, chunks, out); break;
    }
    MX_LAUNCH("k_dequantize");
    return MX_OK;
}

// ---- seeded synthetic blocks ---------------------------------------------------
// Byte j of a tensor = byte (j & 7) of mix64(key + (j/8 + 1) * GAMMA); then the
// f16 scale fields of each block are set to f16(0.001 + 0.009 u).
constexpr uint64_t GAMMA = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27; z *= 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z;
}

uint64_t tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id) {
    const uint64_t a = mix64(seed + GAMMA);
    const uint64_t b = mix64((((uint64_t)layer << 16) | tensor_id) + 2 * GAMMA);
    return mix64(a ^ b);
}

__global__ void __launch_bounds__(256) k_synth_fill(uint64_t key, uint8_t *__restrict__ dst,
                                                    int64_t nbytes) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // word index
    const int64_t j0 = i * 8;
    if (j0 >= nbytes) return;
    const uint64_t w = mix64(key + ((uint64_t)i + 1) * GAMMA);
    const uintptr_t a = reinterpret_cast<uintptr_t>(dst + j0);
    if (j0 + 8 <= nbytes && (a & 7) == 0) {
        *reinterpret_cast<uint64_t *>(dst + j0) = w;
    } else {
        for (int b = 0; b < 8 && j0 + b < nbytes; b++) dst[j0 + b] = (uint8_t)(w >> (8 * b));
    }
}

__device__ __forceinline__ uint16_t synth_scale(uint64_t h, int which) {
    const uint32_t bits24 = which == 0 ? (uint32_t)(h >> 40) : (uint32_t)((h >> 16) & 0xFFFFFFu);
    const float u = (float)bits24 * (1.0f / 16777216.0f);
    const float p = 0.009f * u;
    const float v = 0.001f + p;
    return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: round to nearest even
}

template <int DT>
__global__ void __launch_bounds__(256) k_synth_fix(uint64_t key, uint8_t *__restrict__ dst,
                                                   int64_t n_blocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint64_t h = mix64((key ^ 0xA0761D6478BD642Full) + ((uint64_t)b + 1) * GAMMA);
    uint8_t *blk = dst + b * type_size(DT);
    if constexpr (DT == kQ4_K || DT == kQ5_K) {
        *reinterpret_cast<uint16_t *>(blk) = synth_scale(h, 0);
        *reinterpret_cast<uint16_t *>(blk + 2) = synth_scale(h, 1);
    } else if constexpr (DT == kQ6_K) {
        *reinterpret_cast<uint16_t *>(blk + 208) = synth_scale(h, 0);
    } else {
        *reinterpret_cast<uint16_t *>(blk) = synth_scale(h, 0);
    }
}

mx_status launch_synth(int dtype, uint64_t key, uint8_t *dst, int64_t nbytes, hipStream_t s) {
    const int64_t words = (nbytes + 7) / 8;
    if (words == 0) return MX_OK;
    hipLaunchKernelGGL(k_synth_fill, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s, key,
                       dst, nbytes);
    MX_LAUNCH("k_synth_fill");
    const int64_t nb = nbytes / type_size(dtype);
    if (nb == 0) return MX_OK;
    const dim3 grid((unsigned)((nb + 255) / 256));
    switch (dtype) {
    case kQ4_K: hipLaunchKernelGGL(k_synth_fix<kQ4_K>, grid, dim3(256), 0, s, key, dst, nb); break;
    case kQ5_K: hipLaunchKernelGGL(k_synth_fix<kQ5_K>, grid, dim3(256), 0, s, key, dst, nb); break;
    case kQ6_K: hipLaunchKernelGGL(k_synth_fix<kQ6_K>, grid, dim3(256), 0, s, key, dst, nb); break;
    default: hipLaunchKernelGGL(k_synth_fix<kQ8_0>, grid, dim3(256), 0, s, key, dst, nb); break;
    }
    MX_LAUNCH("k_synth_fix");
    return MX_OK;
}

}  // namespace mx
