// Prefill / verify grouped expert GEMM (the mul_mm_id path).
//
// 1. Bucket pass (replaces kernel_mul_mm_id_map0, mm_id.metal:207-259): per
//    expert, the flattened (token*top_k + slot) pairs routed to it, tokens
//    ascending, compacted into one list with per-expert offsets, plus a list
//    of (expert, m-tile) work items (m-tiles of `bm` pairs; the mm_id
//    projections use GM_BM).  Built as chunked histogram -> scan -> ordered
//    fill, so no thread walks all t*top_k ids.
// 2. Fallback grouped GEMM (replaces kernel_mul_mm_id_*_t, mm_id.metal:492-647,
//    for the projections the MFMA GEMM of the prefill path does not take: K not
//    a whole number of 256-weight super-blocks, or operand spans past its 32-bit
//    offsets): one block per (half of a GM_BM work item, 64-row n-tile).
//    Each 256-wide K step dequantises the expert's 64x256 weight tile from raw GGUF blocks into LDS as f16,
//    gathers the 64 token rows of x into LDS as f16 with a per-(row, K-step)
//    power-of-two scale (so any f32 magnitude fits f16 without rounding the
//    scale), and contracts on v_mfma_f32_16x16x32_f16 with f32 accumulation;
//    the step result is rescaled into an f32 total.  Rows are scattered to
//    dst[token, slot, :].
#include "mx_launch.h"

namespace mx {

constexpr int MM_BN = 64;       // weight rows per n-tile
constexpr int MM_BK = 256;      // K per step (one K-quant super-block)
constexpr int MM_LDK = MM_BK + 8;  // padded LDS row (halves)

size_t map0_bytes(int n_expert, int t, int top_k) {
    return (size_t)MapLayout(n_expert, t, top_k).words * 4;
}

// Flags of a chunk (duplicate id within a token: 1, out-of-range id: 2) ride in
// bits 28-29 of the chunk's expert-0 count; the scan folds them into the dup word.
constexpr int BK_FLAG_SHIFT = 28;
constexpr int32_t BK_COUNT_MASK = (1 << BK_FLAG_SHIFT) - 1;

// Copies the chunk's ids into LDS (the duplicate checks then read LDS).  `ids`
// holds routed_k ids per token; a map of top_k > routed_k slots gives every
// token slots routed_k .. top_k - 1 with expert n_expert - 1 (the shared expert
// joined to the routed map as its last expert).
__device__ __forceinline__ void stage_chunk_ids(const uint32_t *__restrict__ ids, int tok0, int n, int top_k,
                                                int routed_k, int n_expert, uint32_t *s_ids) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int tt = i / top_k, sl = i % top_k;
        s_ids[i] = sl < routed_k ? ids[(int64_t)(tok0 + tt) * routed_k + sl] : (uint32_t)(n_expert - 1);
    }
}
// true when slot `slot` of row `row` is the first slot of its token with this id
__device__ __forceinline__ bool first_of_token(const uint32_t *row, int slot, uint32_t id) {
    bool first = true;
    for (int s2 = 0; s2 < slot; s2++) first = first && (row[s2] != id);
    return first;
}

// chunk histogram: cnt[c][e] = pairs of chunk c routed to e, plus the chunk's flags.
__global__ void __launch_bounds__(256) k_bucket_count(const uint32_t *__restrict__ ids, int t,
                                                      int top_k, int routed_k, int n_expert,
                                                      int32_t *__restrict__ map) {
    extern __shared__ int32_t s_hist[];  // [n_expert] counts | [BK_CHUNK * top_k] ids
    __shared__ int s_flag;
    uint32_t *s_ids = reinterpret_cast<uint32_t *>(s_hist + n_expert);
    const MapLayout L(n_expert, t, top_k);
    const int c = blockIdx.x, tid = threadIdx.x;
    const int tok0 = c * BK_CHUNK;
    const int ntok = min(BK_CHUNK, t - tok0);
    for (int e = tid; e < n_expert; e += 256) s_hist[e] = 0;
    if (tid == 0) s_flag = 0;
    stage_chunk_ids(ids, tok0, ntok * top_k, top_k, routed_k, n_expert, s_ids);
    __syncthreads();
    int flag = 0;
    for (int i = tid; i < ntok * top_k; i += 256) {
        const uint32_t id = s_ids[i];
        const bool first = first_of_token(s_ids + (i / top_k) * top_k, i % top_k, id);  // a token counts once per expert
        if (!first) flag |= 1;
        if (id >= (uint32_t)n_expert) flag |= 2;  // out-of-range id: dropped
        else if (first) atomicAdd(&s_hist[id], 1);
    }
    if (flag) atomicOr(&s_flag, flag);
    __syncthreads();
    for (int e = tid; e < n_expert; e += 256)
        map[L.chunk + (int64_t)c * n_expert + e] = s_hist[e] | (e == 0 ? s_flag << BK_FLAG_SHIFT : 0);
}

// per-expert scan over chunks, expert offsets, tile list, dup word.  One block of
// 1024; also the whole header when t == 0 (no chunks).
__global__ void __launch_bounds__(1024) k_bucket_scan(int t, int top_k, int n_expert, int bm,
                                                      int32_t *__restrict__ map) {
    __shared__ int32_t s_a[1024], s_b[1024];
    __shared__ int s_flag;
    const MapLayout L(n_expert, t, top_k);
    const int tid = threadIdx.x;
    if (tid == 0) s_flag = 0;
    __syncthreads();
    const int per = (n_expert + 1023) / 1024;
    const int e0 = min(tid * per, n_expert), e1 = min(e0 + per, n_expert);
    int sum_pairs = 0, sum_tiles = 0, flag = 0;
    constexpr int CB = 16;  // chunk counts loaded together (independent loads in flight)
    for (int e = e0; e < e1; e++) {
        int run = 0;
        int32_t *p = map + L.chunk + e;
        for (int64_t c0 = 0; c0 < L.nchunks; c0 += CB) {
            int32_t v[CB];
#pragma unroll
            for (int i = 0; i < CB; i++) v[i] = c0 + i < L.nchunks ? p[(c0 + i) * n_expert] : 0;
#pragma unroll
            for (int i = 0; i < CB; i++) {
                if (c0 + i < L.nchunks) {
                    flag |= v[i] >> BK_FLAG_SHIFT;
                    p[(c0 + i) * n_expert] = run;  // exclusive prefix within the expert
                    run += v[i] & BK_COUNT_MASK;
                }
            }
        }
        map[L.tpe + e] = run;
        sum_pairs += run;
        sum_tiles += (run + bm - 1) / bm;
    }
    if (flag) atomicOr(&s_flag, flag);
    // block exclusive scan of (pairs, tiles) over threads
    s_a[tid] = sum_pairs;
    s_b[tid] = sum_tiles;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int va = tid >= d ? s_a[tid - d] : 0, vb = tid >= d ? s_b[tid - d] : 0;
        __syncthreads();
        s_a[tid] += va;
        s_b[tid] += vb;
        __syncthreads();
    }
    int po = s_a[tid] - sum_pairs, to = s_b[tid] - sum_tiles;
    for (int e = e0; e < e1; e++) {
        const int n = map[L.tpe + e];
        map[L.off + e] = po;
        const int mt = (n + bm - 1) / bm;
        for (int m = 0; m < mt; m++) map[L.tiles + to + m] = (e << 16) | m;
        po += n;
        to += mt;
    }
    if (tid == 1023) {
        map[L.off + n_expert] = s_a[1023];
        map[L.n_tiles] = s_b[1023];
        map[L.dup] = s_flag;
    }
}

// ordered fill with its own scan: for each chunk, each expert-thread walks the
// chunk's tokens in order.  Every block reads all chunk counts of its experts
// (a few KB from L2) and forms the offsets itself -- the exclusive prefix over
// chunks within each expert and over experts -- so no scan launch sits between
// the count and fill passes; block 0 also writes the header (counts, offsets,
// tile list, flags), as k_bucket_scan does.
// s_slot[e * BK_ROW + tt]: the first slot of token tt that picked expert e (0xFF:
// none).  Each expert's thread reads its row as BK_W 16-byte words and walks the
// chunk's tokens from registers.
constexpr int BK_ROW = BK_CHUNK + 16;  // table row bytes: BK_CHUNK slots, padded to spread the rows over the banks
constexpr int BK_W = BK_CHUNK / 16;    // 16-byte words per table row
constexpr int BK_EPT = 4;    // experts per thread (n_expert <= 1024)
static_assert(BK_CHUNK % 16 == 0 && BK_ROW % 16 == 0, "table rows: whole 16-byte words");
__global__ void __launch_bounds__(256) k_bucket_fill(const uint32_t *__restrict__ ids, int t,
                                                     int top_k, int routed_k, int n_expert, int bm,
                                                     int32_t *__restrict__ map) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_slot[];
    __shared__ int32_t s_a[256], s_b[256];
    __shared__ int s_flag;
    const int table = n_expert * BK_ROW;
    uint32_t *s_ids = reinterpret_cast<uint32_t *>(s_slot + table);
    const MapLayout L(n_expert, t, top_k);
    const int c = blockIdx.x, tid = threadIdx.x;
    const int tok0 = c * BK_CHUNK;
    const int ntok = min(BK_CHUNK, t - tok0);
    uint4 *w128 = reinterpret_cast<uint4 *>(s_slot);
    for (int i = tid; i < table / 16; i += 256) w128[i] = make_uint4(~0u, ~0u, ~0u, ~0u);
    if (tid == 0) s_flag = 0;
    stage_chunk_ids(ids, tok0, ntok * top_k, top_k, routed_k, n_expert, s_ids);
    // this thread's experts [e0, e1): totals and the prefix before chunk c
    const int per = (n_expert + 255) / 256;
    const int e0 = min(tid * per, n_expert), e1 = min(e0 + per, n_expert);
    int tot[BK_EPT], before[BK_EPT];
    int sum_pairs = 0, sum_tiles = 0, flag = 0;
#pragma unroll
    for (int j = 0; j < BK_EPT; j++) {
        tot[j] = 0;
        before[j] = 0;
        const int e = e0 + j;
        if (e < e1) {
            const int32_t *p = map + L.chunk + e;
            constexpr int CB = 16;  // chunk counts loaded together (independent loads in flight)
            int run = 0;
            for (int64_t q0 = 0; q0 < L.nchunks; q0 += CB) {
                int32_t v[CB];
#pragma unroll
                for (int i = 0; i < CB; i++) v[i] = q0 + i < L.nchunks ? p[(q0 + i) * n_expert] : 0;
#pragma unroll
                for (int i = 0; i < CB; i++) {
                    if (q0 + i == c) before[j] = run;
                    flag |= v[i] >> BK_FLAG_SHIFT;
                    run += v[i] & BK_COUNT_MASK;
                }
            }
            tot[j] = run;
            sum_pairs += run;
            sum_tiles += (run + bm - 1) / bm;
        }
    }
    if (flag) atomicOr(&s_flag, flag);
    s_a[tid] = sum_pairs;
    s_b[tid] = sum_tiles;
    __syncthreads();
    for (int i = tid; i < ntok * top_k; i += 256) {
        const int slot = i % top_k;
        const uint32_t id = s_ids[i];
        // out-of-range ids are dropped (flagged by the count pass)
        const bool first = id < (uint32_t)n_expert && first_of_token(s_ids + (i / top_k) * top_k, slot, id);
        if (first) s_slot[id * BK_ROW + i / top_k] = (uint8_t)slot;  // one writer per (token, expert)
    }
    for (int d = 1; d < 256; d <<= 1) {  // inclusive scans of (pairs, tiles) over threads
        const int va = tid >= d ? s_a[tid - d] : 0, vb = tid >= d ? s_b[tid - d] : 0;
        __syncthreads();
        s_a[tid] += va;
        s_b[tid] += vb;
        __syncthreads();
    }
    int po = s_a[tid] - sum_pairs, to = s_b[tid] - sum_tiles;
    int32_t *dst = map + L.list;
#pragma unroll
    for (int j = 0; j < BK_EPT; j++) {
        const int e = e0 + j;
        if (e >= e1) continue;
        if (c == 0) {  // the header
            map[L.tpe + e] = tot[j];
            map[L.off + e] = po;
            const int mt = (tot[j] + bm - 1) / bm;
            for (int m = 0; m < mt; m++) map[L.tiles + to + m] = (e << 16) | m;
            to += mt;
        }
        int pos = po + before[j];
        po += tot[j];
        const uint4 *row = reinterpret_cast<const uint4 *>(s_slot + e * BK_ROW);
        uint32_t wd[4 * BK_W];
#pragma unroll
        for (int q = 0; q < BK_W; q++) {
            const uint4 v = row[q];
            wd[4 * q] = v.x;
            wd[4 * q + 1] = v.y;
            wd[4 * q + 2] = v.z;
            wd[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int tt = 0; tt < BK_CHUNK; tt++) {
            const uint32_t sl = (wd[tt >> 2] >> (8 * (tt & 3))) & 0xFFu;
            if (sl != 0xFFu) dst[pos++] = (tok0 + tt) * top_k + (int)sl;  // (rows past ntok stay 0xFF)
        }
    }
    if (c == 0 && tid == 255) {
        map[L.off + n_expert] = s_a[255];
        map[L.n_tiles] = s_b[255];
        map[L.dup] = s_flag;
    }
}

// The same list for expert counts whose slot table does not fit in LDS: each
// expert's thread scans the chunk's ids directly.
__global__ void __launch_bounds__(256) k_bucket_fill_scan(const uint32_t *__restrict__ ids, int t,
                                                          int top_k, int routed_k, int n_expert,
                                                          int32_t *__restrict__ map) {
    extern __shared__ uint32_t s_ids[];
    const MapLayout L(n_expert, t, top_k);
    const int c = blockIdx.x, tid = threadIdx.x;
    const int tok0 = c * BK_CHUNK;
    const int ntok = min(BK_CHUNK, t - tok0);
    stage_chunk_ids(ids, tok0, ntok * top_k, top_k, routed_k, n_expert, s_ids);
    __syncthreads();
    for (int e = tid; e < n_expert; e += 256) {
        int pos = map[L.off + e] + map[L.chunk + (int64_t)c * n_expert + e];
        for (int tt = 0; tt < ntok; tt++) {
            for (int s = 0; s < top_k; s++) {
                if (s_ids[tt * top_k + s] == (uint32_t)e) {
                    map[L.list + pos++] = (tok0 + tt) * top_k + s;
                    break;  // one slot per token (duplicates collapse, as map0 does)
                }
            }
        }
    }
}

mx_status launch_map0(const uint32_t *ids, int t, int top_k, int n_expert, int32_t *map,
                      hipStream_t s, int bm, int routed_k) {
    if (routed_k <= 0) routed_k = top_k;
    const MapLayout L(n_expert, t, top_k);
    const size_t ids_lds = (size_t)BK_CHUNK * top_k * 4;
    if (t > 0) {
        hipLaunchKernelGGL(k_bucket_count, dim3((unsigned)L.nchunks), dim3(256), n_expert * 4 + ids_lds, s, ids, t,
                           top_k, routed_k, n_expert, map);
        MX_LAUNCH("k_bucket_count");
    }
    const size_t slot_lds = (size_t)n_expert * BK_ROW + ids_lds;
    if (t > 0 && slot_lds <= 60 * 1024 && n_expert <= 256 * BK_EPT) {
        // the fill pass forms the offsets itself (and block 0 writes the header)
        hipLaunchKernelGGL(k_bucket_fill, dim3((unsigned)L.nchunks), dim3(256), slot_lds, s, ids, t, top_k,
                           routed_k, n_expert, bm, map);
        MX_LAUNCH("k_bucket_fill");
        return MX_OK;
    }
    // writes the whole header (tpe, off, n_tiles, dup), also for t == 0
    hipLaunchKernelGGL(k_bucket_scan, dim3(1), dim3(1024), 0, s, t, top_k, n_expert, bm, map);
    MX_LAUNCH("k_bucket_scan");
    if (t == 0) return MX_OK;
    {
        hipLaunchKernelGGL(k_bucket_fill_scan, dim3((unsigned)L.nchunks), dim3(256), BK_CHUNK * top_k * 4, s, ids,
                           t, top_k, routed_k, n_expert, map);
        MX_LAUNCH("k_bucket_fill_scan");
    }
    return MX_OK;
}

// ---- tile dequantisation into LDS (f16) ---------------------------------------------
// Thread (r, q): row r of the tile, quarter q (64 weights) of the 256-wide step.
template <int DT>
__device__ __forceinline__ void deq_quarter(const uint8_t *__restrict__ row, int kstep, int q,
                                            int k, _Float16 *__restrict__ out) {
    if constexpr (DT == kQ4_K || DT == kQ5_K) {
        constexpr int TS = DT == kQ5_K ? 176 : 144, QS = DT == kQ5_K ? 48 : 16;
        const uint8_t *blk = row + (int64_t)kstep * TS;
        const uint4 h = *reinterpret_cast<const uint4 *>(blk);
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * q, h.y, h.z, h.w, sc0, m0);
        q4k_scale_min(2 * q + 1, h.y, h.z, h.w, sc1, m1);
        const float d = h2f((uint16_t)(h.x & 0xFFFFu)), dmin = h2f((uint16_t)(h.x >> 16));
        const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
        const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + QS + 32 * q);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + QS + 16 + 32 * q);
        const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int w = 0; w < 8; w++) {
            half4_t lo, hi;
            // Q5_K: the fifth bits of weights 32*half + 4w .. +3 of this pair (bits 2q, 2q+1)
            const uint32_t hb = DT == kQ5_K ? *reinterpret_cast<const uint32_t *>(blk + 16 + 4 * w) >> (2 * q) : 0u;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                const uint32_t byte = (qw[w] >> (8 * bb)) & 0xFFu;
                const uint32_t h5 = (hb >> (8 * bb)) & 3u;
                lo[bb] = (_Float16)(d1 * (float)((byte & 0xFu) | ((h5 & 1u) << 4)) - mm1);
                hi[bb] = (_Float16)(d2 * (float)((byte >> 4) | ((h5 >> 1) << 4)) - mm2);
            }
            *reinterpret_cast<half4_t *>(out + 4 * w) = lo;
            *reinterpret_cast<half4_t *>(out + 32 + 4 * w) = hi;
        }
    } else if constexpr (DT == kQ6_K) {
        const uint8_t *blk = row + (int64_t)kstep * 210;
        const int n = q >> 1, p0 = 2 * (q & 1);
        const float d = h2f(ld_u16(blk + 208));
        const uint8_t *qh = blk + 128 + 32 * n;
        const int8_t *scp = reinterpret_cast<const int8_t *>(blk + 192 + 8 * n);
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const int p = p0 + pp;
            const uint8_t *ql = blk + 64 * n + ((p & 1) ? 32 : 0);
            const int shl = (p & 2) ? 4 : 0, shh = 2 * p;
            const float s0 = d * (float)scp[2 * p], s1 = d * (float)scp[2 * p + 1];
#pragma unroll 8
            for (int l = 0; l < 32; l++) {
                const int qv = (((ql[l] >> shl) & 0xF) | (((qh[l] >> shh) & 3) << 4)) - 32;
                out[32 * pp + l] = (_Float16)((l < 16 ? s0 : s1) * (float)qv);
            }
        }
    } else {
        // two 34-byte Q8_0 blocks: blocks 8*kstep + 2q, +1 (zero past k)
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int blk_i = 8 * kstep + 2 * q + bb;
            if (blk_i * 32 >= k) {
#pragma unroll
                for (int l = 0; l < 32; l++) out[32 * bb + l] = (_Float16)0.f;
                continue;
            }
            const uint8_t *blk = row + (int64_t)blk_i * 34;
            const float d = h2f(ld_u16(blk));
#pragma unroll
            for (int m = 0; m < 16; m++) {
                const uint16_t pr = ld_u16(blk + 2 + 2 * m);
                out[32 * bb + 2 * m] = (_Float16)((float)(int8_t)(pr & 0xFF) * d);
                out[32 * bb + 2 * m + 1] = (_Float16)((float)(int8_t)(pr >> 8) * d);
            }
        }
    }
}

template <int DT>
__global__ void __launch_bounds__(256) k_mul_mm_id(MmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 sA[MM_BN * MM_LDK];
    __shared__ __attribute__((aligned(16))) _Float16 sB[MM_BM * MM_LDK];
    __shared__ float s_scale[MM_BM];
    __shared__ int s_pair[MM_BM];
    const MapLayout L(a.n_expert, a.t, a.top_k);
    // the map's m-tiles hold GM_BM pairs: block pairs 2i, 2i + 1 take the halves of tile i
    const int tile = blockIdx.x >> 1;
    if (tile >= a.map[L.n_tiles]) return;  // block-uniform
    const int item = a.map[L.tiles + tile];
    const int e = item >> 16, mt = item & 0xFFFF;
    const int cnt = a.map[L.tpe + e];
    const int m0 = mt * GM_BM + (blockIdx.x & 1) * MM_BM;
    const int mrows = min(MM_BM, cnt - m0);
    if (mrows <= 0) return;
    const int n0 = blockIdx.y * MM_BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < MM_BM) s_pair[tid] = tid < mrows ? a.map[L.list + a.map[L.off + e] + m0 + tid] : -1;
    __syncthreads();

    const uint8_t *wexp = a.w + (int64_t)e * a.expert_bytes;
    const int wr = (wave >> 1) * 32;  // wave's 32 weight rows within the tile
    const int wc = (wave & 1) * 32;   // wave's 32 pairs within the tile
    float4_t tot[2][2] = {};
    const int nsteps = (a.k + MM_BK - 1) / MM_BK;
    const int r = tid >> 2, q = tid & 3;  // loader role: row/pair r, quarter q
    for (int ks = 0; ks < nsteps; ks++) {
        // A: dequantised weight rows n0 + r
        {
            _Float16 *dstA = sA + r * MM_LDK + 64 * q;
            if (n0 + r < a.n_out) {
                deq_quarter<DT>(wexp + (int64_t)(n0 + r) * a.row_bytes, ks, q, a.k, dstA);
            } else {
#pragma unroll
                for (int i = 0; i < 64; i++) dstA[i] = (_Float16)0.f;
            }
        }
        // B: x rows of the tile's pairs, scaled by 2^-e per (pair, step)
        {
            float v[64];
            const int pair = s_pair[r];
            float mx = 0.f;
            if (pair >= 0) {
                const int tok = pair / a.top_k, slot = pair % a.top_k;
                const float *xr = a.x + ((int64_t)tok * a.x_per_row + (a.x_per_row == 1 ? 0 : slot)) * a.k;
                const int kb = ks * MM_BK + 64 * q;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (kb + 4 * i < a.k) f = *reinterpret_cast<const float4 *>(xr + kb + 4 * i);
                    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
                }
#pragma unroll
                for (int i = 0; i < 64; i++) mx = fmaxf(mx, fabsf(v[i]));
            } else {
#pragma unroll
                for (int i = 0; i < 64; i++) v[i] = 0.f;
            }
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            // exponent so that max * 2^-ex lies in [2^14, 2^15)
            int ex = 0;
            if (mx > 0.f) ex = ilogbf(mx) - 14;
            const float inv = ldexpf(1.0f, -ex);
            if (q == 0) s_scale[r] = ldexpf(1.0f, ex);
            _Float16 *dstB = sB + r * MM_LDK + 64 * q;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                half4_t h;
                h[0] = (_Float16)(v[4 * i] * inv); h[1] = (_Float16)(v[4 * i + 1] * inv);
                h[2] = (_Float16)(v[4 * i + 2] * inv); h[3] = (_Float16)(v[4 * i + 3] * inv);
                *reinterpret_cast<half4_t *>(dstB + 4 * i) = h;
            }
        }
        __syncthreads();
        float4_t acc[2][2] = {};
#pragma unroll
        for (int kk = 0; kk < MM_BK; kk += 32) {
            half8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                af[i] = *reinterpret_cast<const half8_t *>(sA + (wr + 16 * i + (lane & 15)) * MM_LDK + kk + 8 * (lane >> 4));
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = *reinterpret_cast<const half8_t *>(sB + (wc + 16 * j + (lane & 15)) * MM_LDK + kk + 8 * (lane >> 4));
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float sc = s_scale[wc + 16 * j + (lane & 15)];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int v = 0; v < 4; v++) tot[i][j][v] = __builtin_fmaf(acc[i][j][v], sc, tot[i][j][v]);
        }
        __syncthreads();
    }
    // scatter: lane holds rows wr+16i+4*(lane>>4)+v of pair column wc+16j+(lane&15)
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int pair = s_pair[wc + 16 * j + (lane & 15)];
        if (pair < 0) continue;
        float *drow = a.dst + (int64_t)pair * a.n_out;
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = n0 + wr + 16 * i + 4 * (lane >> 4) + v;
                if (row < a.n_out) drow[row] = tot[i][j][v];
            }
        }
    }
}

mx_status launch_mul_mm_id(int dtype, const MmArgs &a, hipStream_t s) {
    if (a.t == 0) return MX_OK;
    static_assert(GM_BM == 2 * MM_BM, "a map tile is two fallback tiles");
    const int64_t tiles = ((int64_t)a.t * a.top_k + GM_BM - 1) / GM_BM + a.n_expert;  // m-tiles of GM_BM
    const dim3 grid((unsigned)(2 * tiles), (unsigned)((a.n_out + MM_BN - 1) / MM_BN));
    switch (dtype) {
    case kQ4_K: hipLaunchKernelGGL(k_mul_mm_id<kQ4_K>, grid, dim3(256), 0, s, a); break;
    case kQ5_K: hipLaunchKernelGGL(k_mul_mm_id<kQ5_K>, grid, dim3(256), 0, s, a); break;
    case kQ6_K: hipLaunchKernelGGL(k_mul_mm_id<kQ6_K>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(k_mul_mm_id<kQ8_0>, grid, dim3(256), 0, s, a); break;
    }
    MX_LAUNCH("k_mul_mm_id");
    return MX_OK;
}

}  // namespace mx
