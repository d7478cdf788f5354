// Grouped expert GEMM of the fused prefill / verify path on MFMA.
//
// Replaces the kernel_mul_mm_id_* dispatches of the reference's prefill block
// (mm_id.metal:492-647, driven from moe.rs:242-323).  One workgroup computes a
// 128-pair x 256-column tile of one expert:
//
//  * A (activations) are f16 rows, each scaled by its own power of two so any
//    f32 magnitude lands in [2^14, 2^15) (the scale is applied back to the f32
//    result, so the only rounding is the f16 rounding of x itself).  The tile's
//    rows are gathered by pair (token = pair / top_k, or the bucket position)
//    and copied straight into LDS with global_load_lds, 128 K-values per
//    stage, double-buffered.  16-byte chunks are XOR-swizzled by row so the
//    MFMA operand reads (16 consecutive rows, same chunk) hit distinct banks.
//  * B (weights): each stage, the raw GGUF bytes the stage needs from every
//    weight row of the tile are copied into LDS by buffer->LDS DMA (one slot
//    per row; see WB), in flight with the A copy while the previous stage
//    computes.  Each lane then reads its own row's slot and dequantises in
//    registers directly into the MFMA B-operand layout: the reference's
//    formula in packed f16 arithmetic, one rounding to f16 (the reference
//    dequantises into half tiles).  Each wave owns 64 (or 32) output
//    columns, so no weight is dequantised twice in a workgroup.
//  * v_mfma_f32_32x32x16_f16, f32 accumulation: each wave holds 4 (pairs) x 2
//    (columns) 32x32 accumulators.
//
// The K order inside a 128-value stage is permuted (identically for A and B):
// MFMA step (p, h) gives lane half kh the 8 values at
// 32p + 16kh + 8h + [0, 8) of the stage, which makes every lane's weight bytes
// contiguous 16-byte pieces of the block.
//
// Epilogues: SwiGLU (wave columns = 32 gate rows and the same 32 up rows, so
// act = silu(g) * u is lane-local; act is written f32 at the pair's bucket
// position) or plain (f32 rows scattered to the pair's output row).
//
// Work items are (m-tile, n-tile) pairs, ordered expert by expert (within an
// expert n-tile-major, m-tile fastest); blocks are dealt to the 8 XCDs
// round-robin by the hardware, so block b takes item (b % 8) * per + b / 8: each
// XCD works through a contiguous run of items, so the m-tiles of one expert that
// share a weight slice, and the n-tiles that share its A rows, run together on
// one L2.
#include "mx_launch.h"
#include "mx_dma.h"
#include "mx_wb.h"
#include "mx_f16row.h"

namespace mx {

namespace {

constexpr int KS = 128;                // K per stage
constexpr int ROWB = KS * 2;           // LDS bytes per A row and stage
constexpr int STAGE_BYTES = GM_BM * ROWB;
constexpr int BN = 256;  // weight rows (output columns) per block

// Weight rows per wave = 32 * NB.  NB = 2 (4 waves per block) reuses every A
// fragment read from LDS for two MFMAs and is what the SwiGLU epilogue needs
// (32 gate + the same 32 up rows in one wave); NB = 1 (8 waves) halves the
// accumulators and weight registers per wave, which lets the Q6_K plain GEMM
// run two waves per SIMD without spilling.
#ifndef MX_GEMM_NB_PLAIN
#define MX_GEMM_NB_PLAIN 1
#endif
// waves of the NB = 2 (SwiGLU, Q4_K) tiles: 4 (256 weight rows, two workgroups
// per CU) or 8 (512 rows, one workgroup per CU at the same 2 waves per SIMD:
// each A tile is gathered once for twice the columns)
#ifndef MX_GEMM_WAVES2
#define MX_GEMM_WAVES2 8
#endif
template <int DT, bool SWIGLU> struct GemmNb {
    static constexpr int nb = (SWIGLU || DT == kQ4_K) ? 2 : MX_GEMM_NB_PLAIN;
    // (Q6_K / Q8_0 SwiGLU keep 4 waves: at 8 a workgroup caps them at 256 VGPRs)
    static constexpr int waves = nb == 2 ? (DT == kQ4_K ? MX_GEMM_WAVES2 : 4) : BN / (32 * nb);
    static constexpr int bn = waves * 32 * nb;  // weight rows per workgroup
};


#ifndef MX_GEMM_IGLP_SWIGLU
#define MX_GEMM_IGLP_SWIGLU -1
#endif
#ifndef MX_GEMM_IGLP_PLAIN
#define MX_GEMM_IGLP_PLAIN 0
#endif
#ifndef MX_GEMM_BPAD
#define MX_GEMM_BPAD 2
#endif
#ifndef MX_GEMM_EXPERT_ORDER
#define MX_GEMM_EXPERT_ORDER 1
#endif

struct Tile {
    int e, pos0, mrows, nt;
};

// decodes this block's work item; false: nothing to do (block-uniform)
__device__ __forceinline__ bool tile_of(const GemmArgs &a, int nt_count, Tile &t) {
    const MapLayout L(a.n_map_expert, a.t, a.top_k);
    const int n_mt = a.map[L.n_tiles];
    const int n_items = n_mt * nt_count;
    const int per = (n_items + 7) / 8;
    const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
    if (local >= per) return false;
    const int item = xcd * per + local;
    if (item >= n_items) return false;
#if MX_GEMM_EXPERT_ORDER
    // expert-major items: an expert's T m-tiles x nt_count n-tiles are consecutive,
    // n-tile-major, so an XCD works through one expert's A rows and weight slices
    // together (its L2 serves the repeats).  Tiles list each expert's m-tiles in
    // order, so item / nt_count falls on one of the item's expert's tiles.
    const int j0 = item / nt_count;
    const int w0 = a.map[L.tiles + j0];
    t.e = w0 >> 16;
    const int first = j0 - (w0 & 0xFFFF);  // the expert's first tile
    const int cnt = a.map[L.tpe + t.e];
    const int T = (cnt + GM_BM - 1) / GM_BM;
    const int loc = item - first * nt_count;
    t.nt = loc / T;
    const int mt = loc - t.nt * T;
#else
    t.nt = item / n_mt;
    const int word = a.map[L.tiles + item % n_mt];
    t.e = word >> 16;
    const int mt = word & 0xFFFF;
    const int cnt = a.map[L.tpe + t.e];
#endif
    t.mrows = min(GM_BM, cnt - mt * GM_BM);
    t.pos0 = a.map[L.off + t.e] + mt * GM_BM;
    return true;
}

// waves per SIMD the register allocation must allow: the LDS of one 8-wave
// workgroup per CU holds 2 waves per SIMD; the 4-wave tiles run 1
template <int DT, bool SWIGLU> struct GemmWpe {
    static constexpr int v = GemmNb<DT, SWIGLU>::waves == 8 ? 2 : 1;
};

// B slot layout in LDS.  Row R's slot starts at byte R * SLOT, plus PAD spare
// 16-byte chunks after every 16 rows.  With SLOT = 176 (44 dwords) rows j and
// j + 16 of a wave's 32 lanes would otherwise start on the same LDS bank
// (44 * 16 = 704 = 11 * 64 dwords): a two-way conflict on every dword read of the
// 2-byte-aligned types.  Two spare chunks shift row j + 16 by 8 banks, which also
// keeps the other lane half (16 bytes further on) and the four row phases of the
// 2-byte-aligned blocks on distinct banks.  Only the plain tiles pad (a SwiGLU
// tile's copies must not straddle its two matrices).
template <int DT, bool SWIGLU> struct BSlots {
    static constexpr int CPR = WB<DT>::CPR, SLOT = WB<DT>::SLOT;
    static constexpr int PAD = (!SWIGLU && (DT == kQ6_K || DT == kQ8_0)) ? MX_GEMM_BPAD : 0;
    static constexpr int GROUP = 16 * CPR + PAD;  // positions per 16 rows
    __device__ static int row_off(int R) { return R * SLOT + 16 * PAD * (R >> 4); }
    static constexpr int bytes(int rows) { return rows * SLOT + 16 * PAD * (rows / 16); }
    static constexpr int positions(int rows) { return rows * CPR + PAD * (rows / 16); }
};

// FEW (plain tiles): compiled for m-tiles that are mostly partly filled, which
// skip the MFMAs and A reads of their empty 32-row blocks (the SwiGLU tiles
// always do)
template <int DT, bool SWIGLU, bool FEW = false>
__global__ void __launch_bounds__((64 * GemmNb<DT, SWIGLU>::waves))
    __attribute__((amdgpu_waves_per_eu(GemmWpe<DT, SWIGLU>::v))) k_gemm(GemmArgs a) {
    constexpr int NB = GemmNb<DT, SWIGLU>::nb;
    constexpr int NWAVE = GemmNb<DT, SWIGLU>::waves;
    constexpr int DMA_PER_WAVE = STAGE_BYTES / 1024 / NWAVE;
    constexpr int BROWS = GemmNb<DT, SWIGLU>::bn;           // weight rows of the tile
    using BS = BSlots<DT, SWIGLU>;
    using GW = std::conditional_t<DT == kQ4_K, WB4L, WB<DT>>;  // the lane's weight registers
    constexpr int CPR = BS::CPR;
    constexpr int B_POS = BS::positions(BROWS);
    constexpr int B_INSTS = (B_POS + 63) / 64;                 // B copy instructions per stage
    constexpr int B_PER_MAT = SWIGLU ? B_INSTS / 2 : B_INSTS; // instructions per matrix (gate / up)
    static_assert(BS::PAD ? !SWIGLU : ((BROWS * CPR) % 64 == 0 && (!SWIGLU || B_INSTS % 2 == 0)),
                  "B copies must not straddle matrices");
    static_assert(BROWS % 16 == 0, "whole 16-row slot groups");
    constexpr int B_PER_WAVE = (B_INSTS + NWAVE - 1) / NWAVE;
    // separate LDS objects per buffer: the compiler can then tell that a copy into
    // one buffer does not feed reads of the other
    __shared__ __attribute__((aligned(1024))) uint8_t sA0[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t sA1[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t sB0[BS::bytes(BROWS)];
    __shared__ __attribute__((aligned(1024))) uint8_t sB1[BS::bytes(BROWS)];
    __shared__ uint32_t s_src[GM_BM];  // byte offset of the A row from the tile's first row
    __shared__ float s_scale[GM_BM];
    __shared__ int s_out[GM_BM];      // output row
    constexpr int NCOL = SWIGLU ? BROWS / 2 : BROWS;
    const int nt_count = (a.n_out + NCOL - 1) / NCOL;
    Tile tl;
    if (!tile_of(a, nt_count, tl)) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31, kh = lane >> 5;
    {
        const MapLayout L(a.n_map_expert, a.t, a.top_k);
        if (tid < GM_BM) {
            const int r = min(tid, tl.mrows - 1);  // rows past the tile repeat its last row
            const int pos = tl.pos0 + r;
            const int pair = a.map[L.list + pos];
            const int64_t arow = a.a_div ? pair / a.a_div : pos;
            // rows ascend within a tile (tokens ascend within a bucket), so the
            // offsets from the first row stay below (A rows or GM_BM) * k * 2 bytes
            const int64_t arow0 = a.a_div ? a.map[L.list + tl.pos0] / a.a_div : tl.pos0;
            s_src[tid] = (uint32_t)((arow - arow0) * a.k * 2);
            s_scale[tid] = a.a_scale[arow];
            s_out[tid] = SWIGLU ? pos : pair / a.top_k * a.out_stride + pair % a.top_k + a.out_add;
        }
    }

    // the tile's weight matrices as buffers from their 16-byte-aligned base
    const bool shared = tl.e >= a.n_expert;
    const int64_t rb = shared ? a.sh_row_bytes : a.row_bytes;
    constexpr int NMAT = SWIGLU ? 2 : 1;
    __amdgpu_buffer_rsrc_t wres[NMAT];
    uint32_t wphase[NMAT];  // base address mod 16
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const uint8_t *base = shared ? a.w_sh[m] : a.w[m] + (int64_t)tl.e * a.expert_bytes;
        const uintptr_t ab = reinterpret_cast<uintptr_t>(base);
        wphase[m] = (uint32_t)(ab & 15);
        // the range ends at the 16-byte boundary after the matrix's last byte: the
        // chunk holding that byte is copied whole (it cannot cross a page, so its
        // spare bytes are readable); copies of whole chunks past it read nothing
        wres[m] = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<uint8_t *>(ab & ~uintptr_t(15)), (short)0,
                                                    (int)((a.n_out * rb + wphase[m] + 15) & ~int64_t(15)),
                                                    0x00020000);
    }
    // this lane's copy chunks: instruction q of the wave covers tile chunk
    // (wave + NWAVE q) * 64 + lane = row R, chunk c; the row's offset in its matrix
    uint32_t b_row[B_PER_WAVE];
    int b_c[B_PER_WAVE];
    bool b_on[B_PER_WAVE];  // false: a spare position (or past the last one), no copy
#pragma unroll
    for (int q = 0; q < B_PER_WAVE; q++) {
        const int inst = wave + NWAVE * q;
        const int ch = inst * 64 + lane;  // LDS position
        const int grp = ch / BS::GROUP, w = ch - grp * BS::GROUP;
        b_on[q] = ch < B_POS && w < 16 * CPR;
        const int R = min(16 * grp + w / CPR, BROWS - 1);
        b_c[q] = w % CPR;
        const int rm = SWIGLU ? R % (BROWS / 2) : R;
        const int colr = min(tl.nt * NCOL + rm, a.n_out - 1);
        b_row[q] = (uint32_t)(colr * rb);
    }
    auto issue_b = [&](int ks, uint8_t *buf) MX_INLINE_LAMBDA {
        const uint32_t so = stage_block_off<DT>(ks);
#pragma unroll
        for (int q = 0; q < B_PER_WAVE; q++) {
            const int inst = wave + NWAVE * q;
            if (inst < B_INSTS) {
                const int m = SWIGLU ? (inst >= B_PER_MAT ? 1 : 0) : 0;
                const uint32_t blk = wphase[m] + b_row[q] + so;  // block offset from the aligned base
                const uint32_t off = kPhased<DT> ? (blk & ~15u) + WB<DT>::chunk_off(b_c[q], ks & 1)
                                                 : blk + WB<DT>::chunk_off(b_c[q], ks & 1);
                if (!BS::PAD || b_on[q]) dma16_buf(wres[m], off, buf + inst * 1024);
            }
        }
        asm volatile("" ::: "memory");
    };

    // this lane's B rows: tile row index, and (2-byte-aligned types) the block phase
    int brow[NB];
    uint32_t rowoff[NB];
    int col[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        brow[nb] = SWIGLU ? nb * (BROWS / 2) + wave * 32 + j : wave * 32 * NB + nb * 32 + j;
        col[nb] = SWIGLU ? tl.nt * NCOL + wave * 32 + j : tl.nt * NCOL + wave * 32 * NB + nb * 32 + j;
        rowoff[nb] = wphase[SWIGLU ? nb : 0] + (uint32_t)(min(col[nb], a.n_out - 1) * rb);
    }
    __syncthreads();

    const MapLayout L0(a.n_map_expert, a.t, a.top_k);
    const int64_t arow0 = a.a_div ? a.map[L0.list + tl.pos0] / a.a_div : tl.pos0;
    const uint8_t *abase = reinterpret_cast<const uint8_t *>(a.a) + arow0 * a.k * 2;  // tile's first A row
    // A stage copy: wave instruction i fills LDS rows 4 (8 wave + i) + lane / 16
    auto issue_a = [&](int ks, uint8_t *buf) MX_INLINE_LAMBDA {
#pragma unroll
        for (int i = 0; i < DMA_PER_WAVE; i++) {
            const int inst = DMA_PER_WAVE * wave + i;
            const int row = 4 * inst + (lane >> 4);
            const int c = (lane & 15) ^ (row & 15);
            dma16(abase + (s_src[row] + (uint32_t)(ks * ROWB + c * 16)), buf + inst * 1024);
        }
        asm volatile("" ::: "memory");
    };

    // per-lane LDS offsets of the A operand for the 8 steps of a stage: the
    // 16-byte chunk (8 K values) the lane's weight operand holds at step s
    // (Q4_K, WB4L: 64 kh + 8 s; the others: 32 (s / 2) + 16 kh + 8 (s % 2))
    int aoff[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int c = DT == kQ4_K ? 8 * kh + s : 4 * (s >> 1) + 2 * kh + (s & 1);
        aoff[s] = j * ROWB + ((c ^ (j & 15)) << 4);
    }

    float16_t acc[4][NB];
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mb][nb][r] = 0.f;

    // MB: 32-row blocks of the tile that hold rows (a partly filled last m-tile of
    // an expert skips the MFMAs and A reads of its empty blocks)
    auto compute = [&](auto mbc, const uint8_t *buf, GW(&wb)[NB]) MX_INLINE_LAMBDA {
        constexpr int MB = decltype(mbc)::value;
        // the A fragments of step s + 1 are read while step s computes
        half8_t af[2][4];
#pragma unroll
        for (int mb = 0; mb < MB; mb++) af[0][mb] = *reinterpret_cast<const half8_t *>(buf + mb * 32 * ROWB + aoff[0]);
        // (a compile-time step index: with a runtime one the weight registers, indexed
        // by step, were moved to scratch in the larger instantiations)
        static_for<0, 8>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            // plain tiles: let the scheduler interleave the step's LDS reads,
            // dequantisation and MFMAs (iglp_opt(0): down GEMM 548 -> 520 us at C3);
            // the SwiGLU tiles measured slower with it (0 or 1: +2-4%)
            if constexpr (!SWIGLU && MX_GEMM_IGLP_PLAIN >= 0) __builtin_amdgcn_iglp_opt(MX_GEMM_IGLP_PLAIN);
            if constexpr (SWIGLU && MX_GEMM_IGLP_SWIGLU >= 0) __builtin_amdgcn_iglp_opt(MX_GEMM_IGLP_SWIGLU);
            constexpr int p = s >> 1, hh = s & 1, cur = s & 1;
            if constexpr (s + 1 < 8) {
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
                    af[cur ^ 1][mb] = *reinterpret_cast<const half8_t *>(buf + mb * 32 * ROWB + aoff[s + 1]);
            }
            half8_t bf[NB];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                if constexpr (DT == kQ4_K) bf[nb] = wb[nb].step(s);
                else bf[nb] = wb[nb].step(p, hh);
            }
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cur][mb], bf[nb], acc[mb][nb], 0, 0, 0);
        });
    };
    // stage ks's B registers from LDS (the block phase of the lane's row for this stage)
    GW wb[NB];
    auto load_b = [&](int ks, const uint8_t *buf) MX_INLINE_LAMBDA {
        const uint32_t so = stage_block_off<DT>(ks);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            if constexpr (DT == kQ4_K) wb[nb].load_lds(buf + BS::row_off(brow[nb]), kh, 0u);
            else wb_load<DT>(wb[nb], buf + BS::row_off(brow[nb]), kh, (rowoff[nb] + so) & 15u, ks & 1);
        }
    };

    const int nks = a.k / KS;  // even
    issue_a(0, sA0);
    issue_b(0, sB0);
    wait_vmcnt(0);
    __syncthreads();
    // Each stage: issue the next stage's A and B copies, read this stage's B rows
    // from LDS, dequantise, compute; stage ends wait for the copies and use a bare
    // s_barrier (the copies are complete (vmcnt) and LDS needs no further fence
    // between the waves of a workgroup).
    auto stage_end = [&]() MX_INLINE_LAMBDA {
        wait_vmcnt(0);
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    auto k_loop = [&](auto mbc) MX_INLINE_LAMBDA {
        for (int ks = 0; ks < nks; ks += 2) {
            issue_a(ks + 1, sA1);
            issue_b(ks + 1, sB1);
            load_b(ks, sB0);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wb[nb].template prep<0>(kh);
            compute(mbc, sA0, wb);
            stage_end();
            {
                // unconditional, clamped at the last stage (a harmless re-copy into
                // the buffer nobody reads next): no branch merge in front of the
                // next waits, so the compiler keeps exact memory counters
                const int kn = min(ks + 2, nks - 1);
                issue_a(kn, sA0);
                issue_b(kn, sB0);
            }
            load_b(ks + 1, sB1);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wb[nb].template prep<1>(kh);
            compute(mbc, sA1, wb);
            stage_end();
        }
    };
    // block-uniform: the tile's filled 32-row blocks.  The plain tiles run full
    // tiles in a loop of their own: as one more case of k_loop the compiler
    // schedules it worse (C3 down 524 -> 571 us), and next to the smaller cases
    // too (-> 541 us), so only the FEW instantiation carries those.
    if constexpr (SWIGLU) {
        if (tl.mrows > 64) k_loop(std::integral_constant<int, 4>{});
        else if (tl.mrows > 32) k_loop(std::integral_constant<int, 2>{});
        else k_loop(std::integral_constant<int, 1>{});
    } else if (FEW && tl.mrows <= 32) {
        k_loop(std::integral_constant<int, 1>{});
    } else if (FEW && tl.mrows <= 64) {
        k_loop(std::integral_constant<int, 2>{});
    } else {
        for (int ks = 0; ks < nks; ks += 2) {
            issue_a(ks + 1, sA1);
            issue_b(ks + 1, sB1);
            load_b(ks, sB0);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wb[nb].template prep<0>(kh);
            compute(std::integral_constant<int, 4>{}, sA0, wb);
            stage_end();
            {
                const int kn = min(ks + 2, nks - 1);  // clamped, unconditional (see k_loop)
                issue_a(kn, sA0);
                issue_b(kn, sB0);
            }
            load_b(ks + 1, sB1);
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wb[nb].template prep<1>(kh);
            compute(std::integral_constant<int, 4>{}, sA1, wb);
            stage_end();
        }
    }
    __syncthreads();

    // epilogue: acc[mb][nb][r] = D[row 32 mb + 8 (r / 4) + 4 kh + r % 4][col[nb]]
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = 32 * mb + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (row >= tl.mrows) continue;
            const float sc = s_scale[row];
            float *orow = a.out + (int64_t)s_out[row] * a.n_out;
            if constexpr (SWIGLU) {
                if (col[0] < a.n_out) {
                    const float g = acc[mb][0][r] * sc, u = acc[mb][1][r] * sc;
                    // silu(g) * u (silu_mul.metal:57-72) on the hardware exp2 and
                    // reciprocal (about 1 ulp each): the act row is rounded to f16
                    // for the down GEMM, far above these errors
                    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);  // exp(-g)
                    orow[col[0]] = g * __builtin_amdgcn_rcpf(1.0f + e) * u;
                }
            } else {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    if (col[nb] < a.n_out) orow[col[nb]] = acc[mb][nb][r] * sc;
            }
        }
    }
}

// ---- f32 rows -> scaled f16 rows (body in mx_f16row.h) -------------------------------
template <int RPT, bool PERM>
__global__ void __launch_bounds__(256) k_to_f16_rows(const float *__restrict__ x, int k,
                                                     const int32_t *__restrict__ count,
                                                     const int32_t *__restrict__ src,
                                                     _Float16 *__restrict__ y, float *__restrict__ scale) {
    const int64_t row = blockIdx.x;
    if (count && row >= *count) return;
    const int64_t xr = src ? src[row] : row;
    __shared__ float s_red[4];
    f16_row<RPT, PERM>(x + xr * k, k, y + row * k, scale + row, s_red);
}

// out = residual + (sum_s w_s down_s) + shared   (moe.rs:78; combine.metal:16-40 order)
// KK > 0: compiled for kk = top_k + has_shared == KK, so every slot's load is
// issued before the first one is used; KK == 0: any kk, one slot at a time.
template <int KK>
__global__ void __launch_bounds__(256) k_combine_prefill(const float *__restrict__ down, const float *__restrict__ w,
                                                         const float *__restrict__ residual,
                                                         const float *__restrict__ shared_sep, int top_k,
                                                         int has_shared, int n, float *__restrict__ out) {
    const int64_t tok = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const int kk = KK > 0 ? KK : top_k + has_shared;
    const float *d = down + tok * kk * n + i;
    auto fma4 = [](float ws, const float4 &v, float4 &acc) {
        acc.x = __builtin_fmaf(ws, v.x, acc.x);
        acc.y = __builtin_fmaf(ws, v.y, acc.y);
        acc.z = __builtin_fmaf(ws, v.z, acc.z);
        acc.w = __builtin_fmaf(ws, v.w, acc.w);
    };
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 sh = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (KK > 0) {
        float4 v[KK];
#pragma unroll
        for (int s = 0; s < KK; s++) v[s] = ld_stream4(d + (int64_t)s * n);  // (combine 75 -> 62 us at C3)
#pragma unroll
        for (int s = 0; s < KK; s++)
            if (s < top_k) fma4(w[tok * top_k + s], v[s], acc);
        if (has_shared) sh = v[KK - 1];
    } else {
        for (int s = 0; s < top_k; s++) fma4(w[tok * top_k + s], ld_stream4(d + (int64_t)s * n), acc);
        if (has_shared) sh = *reinterpret_cast<const float4 *>(d + (int64_t)top_k * n);
    }
    if (shared_sep) sh = *reinterpret_cast<const float4 *>(shared_sep + tok * n + i);
    if (has_shared || shared_sep) {
        acc.x += sh.x; acc.y += sh.y; acc.z += sh.z; acc.w += sh.w;
    }
    if (residual) {
        const float4 r = *reinterpret_cast<const float4 *>(residual + tok * n + i);
        acc.x = r.x + acc.x; acc.y = r.y + acc.y; acc.z = r.z + acc.z; acc.w = r.w + acc.w;
    }
    *reinterpret_cast<float4 *>(out + tok * n + i) = acc;
}

}  // namespace

bool gemm_supported(int dtype, int k) {
    return (dtype == kQ4_K || dtype == kQ5_K || dtype == kQ6_K || dtype == kQ8_0) && k > 0 && k % 256 == 0;
}

static bool gemm_spans_fit(int64_t a_span, int k, int n_out, int64_t row_bytes) {
    return a_span * k * 2 < (INT64_C(1) << 32) && (int64_t)n_out * row_bytes < (INT64_C(1) << 31);
}

bool gemm_fits(int t, int hidden, int ff, int64_t gu_row_bytes, int64_t d_row_bytes) {
    return gemm_spans_fit(t, hidden, ff, gu_row_bytes) && gemm_spans_fit(GM_BM, ff, hidden, d_row_bytes);
}

bool gemm_plain_fits(int64_t a_rows, int k, int n_out, int64_t row_bytes) {
    return gemm_spans_fit(a_rows, k, n_out, row_bytes);
}

mx_status launch_gemm(int dtype, bool swiglu, const GemmArgs &a, hipStream_t s) {
    if (a.t == 0) return MX_OK;
    const MapLayout L(a.n_map_expert, a.t, a.top_k);
    int ncol = 256;
    switch (dtype) {  // output columns per workgroup of the instantiation launched below
    case kQ4_K: ncol = swiglu ? GemmNb<kQ4_K, true>::bn / 2 : GemmNb<kQ4_K, false>::bn; break;
    case kQ5_K: ncol = swiglu ? GemmNb<kQ5_K, true>::bn / 2 : GemmNb<kQ5_K, false>::bn; break;
    case kQ6_K: ncol = swiglu ? GemmNb<kQ6_K, true>::bn / 2 : GemmNb<kQ6_K, false>::bn; break;
    default: ncol = swiglu ? GemmNb<kQ8_0, true>::bn / 2 : GemmNb<kQ8_0, false>::bn; break;
    }
    const int64_t nt = (a.n_out + ncol - 1) / ncol;
    const int64_t t_max = ((int64_t)a.t * a.top_k + GM_BM - 1) / GM_BM + a.n_map_expert;  // m-tiles of GM_BM
    // the kernel addresses a tile's A rows from its first row, and one expert's
    // weight rows from the expert, with 32-bit offsets
    const int64_t a_span = a.a_div ? ((int64_t)a.t * a.top_k + a.a_div - 1) / a.a_div : GM_BM;
    if (!gemm_spans_fit(a_span, a.k, a.n_out, a.row_bytes > a.sh_row_bytes ? a.row_bytes : a.sh_row_bytes))
        return fail(MX_ERR_OVERFLOW, "gemm: an operand span beyond 4 GiB (t * k * 2 bytes of x); split the batch");
    const int64_t blocks = (t_max * nt + 7) / 8 * 8;
    if (blocks > INT32_MAX) return fail(MX_ERR_OVERFLOW, "gemm: too many tiles");
    const dim3 grid((unsigned)blocks);
    // plain tiles: the FEW form when the average expert holds under 64 pairs
    // (C3's down, 88 pairs per expert with the shared one, takes the full-tile form)
    const bool few = !swiglu && (int64_t)a.t * a.top_k < (int64_t)64 * a.n_map_expert;
#define MX_G(DT, SW, F) hipLaunchKernelGGL((k_gemm<DT, SW, F>), grid, dim3((64 * GemmNb<DT, SW>::waves)), 0, s, a)
#define MX_P(DT) if (swiglu) MX_G(DT, true, false); else if (few) MX_G(DT, false, true); else MX_G(DT, false, false)
    switch (dtype) {
    case kQ4_K: MX_P(kQ4_K); break;
    case kQ5_K: MX_P(kQ5_K); break;
    case kQ6_K: MX_P(kQ6_K); break;
    default: MX_P(kQ8_0); break;
    }
#undef MX_P
#undef MX_G
    (void)L;
    MX_LAUNCH("k_gemm");
    return MX_OK;
}

template <bool PERM>
static void to_f16_rows(const float *x, int64_t rows, int k, const int32_t *count, const int32_t *src, _Float16 *y,
                        float *scale, hipStream_t s) {
    const dim3 grid((unsigned)rows);
    if (k <= 1024 * 2)
        hipLaunchKernelGGL((k_to_f16_rows<2, PERM>), grid, dim3(256), 0, s, x, k, count, src, y, scale);
    else if (k <= 1024 * 4)
        hipLaunchKernelGGL((k_to_f16_rows<4, PERM>), grid, dim3(256), 0, s, x, k, count, src, y, scale);
    else hipLaunchKernelGGL((k_to_f16_rows<0, PERM>), grid, dim3(256), 0, s, x, k, count, src, y, scale);
}

mx_status launch_to_f16_rows(const float *x, int64_t rows, int k, const int32_t *count, _Float16 *y, float *scale,
                             hipStream_t s, bool perm, const int32_t *src) {
    if (rows == 0) return MX_OK;
    if (perm) to_f16_rows<true>(x, rows, k, count, src, y, scale, s);
    else to_f16_rows<false>(x, rows, k, count, src, y, scale, s);
    MX_LAUNCH("k_to_f16_rows");
    return MX_OK;
}

mx_status launch_combine_prefill(const float *down, const float *w, const float *residual, int t, int top_k,
                                 int has_shared, int n, float *out, hipStream_t s, const float *shared_sep) {
    if (t == 0) return MX_OK;
    const dim3 grid((unsigned)((n / 4 + 255) / 256), (unsigned)t);
    switch (top_k + has_shared) {
#define MX_CB(K) \
    case K: hipLaunchKernelGGL(k_combine_prefill<K>, grid, dim3(256), 0, s, down, w, residual, shared_sep, top_k, has_shared, n, out); break;
        MX_CB(2) MX_CB(3) MX_CB(4) MX_CB(5) MX_CB(6) MX_CB(7) MX_CB(8) MX_CB(9) MX_CB(10) MX_CB(11) MX_CB(12)
#undef MX_CB
        default: hipLaunchKernelGGL(k_combine_prefill<0>, grid, dim3(256), 0, s, down, w, residual, shared_sep, top_k, has_shared, n, out);
    }
    MX_LAUNCH("k_combine_prefill");
    return MX_OK;
}

}  // namespace mx
