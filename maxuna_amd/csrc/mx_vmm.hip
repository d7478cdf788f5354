// Verify blocks on MFMA: each expert a block touches is streamed from HBM once
// and contracted with all of that expert's (token, slot) pairs as 16-pair
// tiles (v_mfma_f32_16x16x32_f16).
//
// Serves the reference's mul_mm_id role for blocks of a few to a few dozen
// tokens (moe.rs:236-240 picks the grouped expert matmul by token count; the
// kernel_mul_mm_id dispatch it replaces is mm_id.metal:492-647).  At this size
// an expert is hit by a handful of pairs, so the per-pair mat-vec kernels spend
// their time repeating the same weight work once per pair; here the
// dequantisation is done once per weight and the pairs ride along as MFMA
// rows.
//
//  * Work items are (pair run, 32-column block): a run is up to 16 pairs of one
//    expert (launch_pair_order), the column block 32 output columns -- for the
//    SwiGLU form 32 gate rows and the same 32 up rows.  The grid is persistent:
//    wave w of W takes items w, w + W, ..., and its stage sequence runs through
//    all of them, so the weight copy of the next stage is always in flight,
//    also across items.
//  * A stage is one super-block (256 K values) of every weight row of the item:
//    the rows' raw GGUF blocks are copied into the wave's own LDS buffer (two
//    buffers, one stage ahead), each lane reads the fields of its row and K
//    quarter and dequantises them into the B operand (mx_wb.h: the f16 rounding
//    of the reference's f32 dequantised value, once).
//  * A (activations) are f16 rows scaled by a power of two per row (the prefill
//    GEMM's operand form), read straight from global memory (L2) one stage
//    ahead; a run's missing rows repeat its last pair and are not stored.
//  * Lane l holds row n = l % 16 of each 16-row block and K quarter q = l / 16.
//    Q4_K: the lane owns 32-value sub-block q of each half super-block, so it
//    unpacks one scale / min per half, not four: MFMA step P gives it values
//    32 q + 8 P + [0, 8) of the half, each group of four in the order 0, 2, 1, 3
//    (the A rows are stored so; see VmQ4).  Q6_K (16-value scale groups): step P
//    gives it 32 P + 8 q + [0, 8) (the prefill GEMM's per-half layout).  The A
//    fragments follow the same K order.  Results: lane l holds D[4 q + r][n],
//    r = 0..3.
//
// Copies of the K-quants with 16-byte-aligned blocks (Q4_K) are plain global ->
// LDS copies of exactly the block's bytes; Q6_K blocks (2-byte aligned) copy
// the 16-byte-aligned span around the block through a buffer resource whose
// range ends at the 16-byte boundary after the expert's last byte, so a span
// never reads past the page that holds the expert's end (chunks wholly beyond
// it copy nothing; their slot bytes are never read).
#include "mx_launch.h"
#include "mx_dma.h"
#include "mx_wb.h"

namespace mx {

namespace {

constexpr int VM_WAVES = 4;
constexpr int VM_ROWS_M = 16;  // pairs per tile

// one super-block per stage: 16-byte chunks per row and the LDS slot of a row
template <int DT> struct VmBlk;
template <> struct VmBlk<kQ4_K> {
    static constexpr int BLK = 144, CPR = 9, SLOT = 144;  // 36 dwords: 16 rows on distinct banks
};
template <> struct VmBlk<kQ6_K> {
    static constexpr int BLK = 210, CPR = 15, SLOT = 240;  // the aligned span (phase <= 14)
};

// COLS output columns per item (16 or 32): the wave's weight rows are COLS rows
// of each matrix, slot order matrix-major
template <int DT, bool SWIGLU, int COLS> struct VmGeo {
    static_assert(COLS == 16 || COLS == 32, "16 or 32 columns per item");
    static constexpr int NMAT = SWIGLU ? 2 : 1;
    static constexpr int ROWS = COLS * NMAT;    // weight rows per wave and stage
    static constexpr int NBLK = ROWS / 16;      // 16-row MFMA column blocks
    static constexpr int CPR = VmBlk<DT>::CPR, SLOT = VmBlk<DT>::SLOT, BLK = VmBlk<DT>::BLK;
    static constexpr int POS = ROWS * CPR;      // copy positions (rows x chunks)
    static constexpr int NI = (POS + 63) / 64;  // copy instructions per stage
    static constexpr int BUF = NI * 1024;       // bytes per stage buffer (spare lanes land past POS)
    static constexpr bool kBuf = DT == kQ6_K;   // copies through a buffer resource
};

// Q6_K half super-block `par` of the lane's row from its stage slot (the whole
// block, from the 16-byte-aligned address below it; m1 = the block's phase):
// the registers WB<kQ6_K>::load_lds fills from the prefill GEMM's per-half slots.
__device__ __forceinline__ void vm_load(WB<kQ6_K> &w, const uint8_t *slot, int kh, uint32_t m1, int par) {
    w.lo = lds16_a2(slot, m1 + 64 * par + 16 * kh);       // ql[64 par + 16 kh, +16)
    w.hi = lds16_a2(slot, m1 + 64 * par + 32 + 16 * kh);  // ql[64 par + 32 + 16 kh, +16)
    w.qh = lds16_a2(slot, m1 + 128 + 32 * par + 16 * kh); // qh[32 par + 16 kh, +16)
    const uint32_t so = m1 + 192 + 8 * par;               // scales[8 par, +8)
    const uint32_t *p = reinterpret_cast<const uint32_t *>(slot + (so & ~3u));
    const uint32_t sh = (so & 2u) * 8u;
    const uint32_t a0 = p[0], a1 = p[1], a2 = p[2];
    w.s0 = __builtin_amdgcn_alignbit(a1, a0, sh);
    w.s1 = __builtin_amdgcn_alignbit(a2, a1, sh);
    w.dbits = *reinterpret_cast<const uint16_t *>(slot + m1 + 208);
}

// Q4_K half super-block `PAR` of the lane's row for the sub-block-per-lane
// order: sub-block j = 4 PAR + q (32 values, one 6-bit scale and min).  Word i of
// its 32 quant bytes holds values 4 i .. 4 i + 3 in the lane's nibble (low for
// even q, high for odd q).  One and-or against the f16 exponent 0x6400 turns a
// word into the f16 pair 1024 + q of values 4 i and 4 i + 2 (the word shifted by
// a byte: 4 i + 1 and 4 i + 3), so step P gives values 8 P + {0, 2, 1, 3, 4, 6,
// 5, 7}: the A rows are stored in that order (launch_to_f16_rows with perm).  A
// high nibble reads as 1024 + 16 q, so odd sub-blocks take d1 / 16 (exact); each
// value is the f32 fma (1024 + q) d1 + c rounded to f16 once, as in WB<kQ4_K>.
struct VmQ4 {
    uint32_t w[8];  // the quant bytes of values 4 i .. 4 i + 3 in word i
    uint32_t m;     // the lane's nibble of bytes 0 and 2: 0x000F000F or 0x00F000F0
    float d1, c1;   // d * sc (/ 16 for a high nibble) and -dmin * m - 1024 * d1
    template <int PAR> __device__ __forceinline__ void load(const uint8_t *slot, int q) {
        const uint4 h = *reinterpret_cast<const uint4 *>(slot);  // d, dmin | scales[12]
        const uint8_t *qs = slot + 16 + 64 * PAR + 32 * (q >> 1); // the sub-block pair's 32 bytes
        const uint4 a = *reinterpret_cast<const uint4 *>(qs);
        const uint4 b = *reinterpret_cast<const uint4 *>(qs + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
        m = (q & 1) ? 0x00F000F0u : 0x000F000Fu;
        // get_scale_min_k4 of sub-block j (q4k_scale_min) with j = 4 PAR + q
        const uint32_t o = 8u * (uint32_t)q;
        uint32_t sc, mn;
        if constexpr (PAR == 0) {
            sc = __builtin_amdgcn_ubfe(h.y, o, 6);
            mn = __builtin_amdgcn_ubfe(h.z, o, 6);
        } else {
            const uint32_t b8 = __builtin_amdgcn_ubfe(h.w, o, 8);
            sc = (b8 & 0xFu) | (__builtin_amdgcn_ubfe(h.y, o + 6, 2) << 4);
            mn = (b8 >> 4) | (__builtin_amdgcn_ubfe(h.z, o + 6, 2) << 4);
        }
        const float d = h2f((uint16_t)(h.x & 0xFFFFu)), dmin = h2f((uint16_t)(h.x >> 16));
        d1 = d * (float)sc * ((q & 1) ? 0.0625f : 1.0f);
        c1 = __builtin_fmaf(-1024.0f, d1, -(dmin * (float)mn));
    }
    __device__ __forceinline__ half8_t step(int P) const {
        const uint32_t r0 = w[2 * P], r1 = w[2 * P + 1];
        const half2_t x[4] = {__builtin_bit_cast(half2_t, (r0 & m) | 0x64006400u),
                              __builtin_bit_cast(half2_t, ((r0 >> 8) & m) | 0x64006400u),
                              __builtin_bit_cast(half2_t, (r1 & m) | 0x64006400u),
                              __builtin_bit_cast(half2_t, ((r1 >> 8) & m) | 0x64006400u)};
        half2_t y[4];
#pragma unroll
        for (int i = 0; i < 4; i++) y[i] = mix2(x[i], d1, c1);
        return pk_join(y);
    }
};

// One work item, as a wave sees it.  Uniform: the matrices and the run; per
// lane: the copy sources, the A row and the output rows of its accumulators.
template <int DT, bool SWIGLU, int COLS> struct VmItem {
    using G = VmGeo<DT, SWIGLU, COLS>;
    const uint8_t *base[G::NMAT];  // expert matrices (Q6_K: 16-byte-aligned base)
    __amdgpu_buffer_rsrc_t rsrc;   // Q6_K: the expert matrix as a buffer
    uint32_t src[G::NI];           // per copy instruction: chunk offset from its matrix (stage 0)
    int mat[G::NI];                // SwiGLU: the matrix of the lane's chunk
    uint32_t rowpos[G::NBLK];      // Q6_K: phase + row offset of the lane's rows (block phases)
    const _Float16 *arow;          // the lane's A row (pair n of the run, clamped)
    bool aon;                      // pair n exists (else the lane's A fragments are 0)
    int pv[4];                     // pair index of accumulator row 4 q + r, -1: none
    float ps[4];                   // its A scale
    int cb;                        // column block
};

// the run tables and A scales come in as restrict kernel arguments: nothing the
// kernel stores aliases them, so their wave-uniform loads stay scalar
struct VmTabs {
    const int32_t *__restrict__ perm;
    const int32_t *__restrict__ runs;
    const float *__restrict__ a_scale;
};

template <int DT, bool SWIGLU, int COLS>
__device__ __forceinline__ void vm_item(const VmmArgs &a, const VmTabs &tb, int item, int CB, int lane,
                                        VmItem<DT, SWIGLU, COLS> &it) {
    using G = VmGeo<DT, SWIGLU, COLS>;
    const int run = item / CB;
    const int cb = item - run * CB;
    const int w0 = tb.runs[2 + 2 * run], e = tb.runs[3 + 2 * run];
    const int start = w0 & 0xFFFF, cnt = w0 >> 16;
    const bool sh = e >= a.n_expert;
    const int64_t rb = sh ? a.sh_row_bytes : a.row_bytes;
    it.cb = cb;
    // the run's pairs (scalar loads; entries past the run are not used)
    // (16 consecutive words: one scalar load; perm is followed by the run table,
    // so the words past the last run stay inside the workspace)
    const int32_t *pp = tb.perm + start;
    int raw[VM_ROWS_M], pair[VM_ROWS_M];
#pragma unroll
    for (int m = 0; m < VM_ROWS_M; m++) raw[m] = pp[m];
#pragma unroll
    for (int m = 0; m < VM_ROWS_M; m++) pair[m] = (m < cnt ? raw[m] : raw[0]) & 0xFFFF;
    const int n = lane & 15, q = lane >> 4;
    int mine = pair[0];
#pragma unroll
    for (int m = 1; m < VM_ROWS_M; m++) mine = n == m ? pair[m] : mine;
    it.arow = a.a + (int64_t)(mine / a.a_slots) * a.k;
    it.aon = n < cnt;
    float sc[VM_ROWS_M];  // (scalar loads)
#pragma unroll
    for (int m = 0; m < VM_ROWS_M; m++) sc[m] = tb.a_scale[pair[m] / a.a_slots];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int v = pair[r];
        float f = sc[r];
#pragma unroll
        for (int qq = 1; qq < 4; qq++) {
            v = q == qq ? pair[4 * qq + r] : v;
            f = q == qq ? sc[4 * qq + r] : f;
        }
        it.pv[r] = 4 * q + r < cnt ? v : -1;
        it.ps[r] = f;
    }
    uint32_t phase = 0;
#pragma unroll
    for (int m = 0; m < G::NMAT; m++) {
        const uint8_t *b = sh ? a.w_sh[m] : a.w[m] + (int64_t)e * a.expert_bytes;
        if constexpr (G::kBuf) {
            phase = (uint32_t)(reinterpret_cast<uintptr_t>(b) & 15);
            b -= phase;
            // (to the 16-byte boundary after the matrix's last byte, as in k_gemm: a
            // chunk that holds matrix bytes is always copied whole)
            it.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(b), (short)0,
                                                        (int)((a.n_out * rb + phase + 15) & ~int64_t(15)),
                                                        0x00020000);
        }
        it.base[m] = b;
    }
#pragma unroll
    for (int i = 0; i < G::NI; i++) {
        const int p = min(64 * i + lane, G::POS - 1);  // spare lanes repeat the last chunk
        const int R = p / G::CPR, c = p - R * G::CPR;
        it.mat[i] = R / COLS;
        const uint32_t row = (uint32_t)(cb * COLS + R % COLS) * (uint32_t)rb;
        it.src[i] = G::kBuf ? phase + row : row + 16u * (uint32_t)c;
    }
#pragma unroll
    for (int nb = 0; nb < G::NBLK; nb++)
        it.rowpos[nb] = phase + (uint32_t)(cb * COLS + (16 * nb) % COLS + n) * (uint32_t)rb;
}

// stage ks's copies of the item into buf (every lane copies: no branch around a
// copy, so the copy counts the waits assume are exact)
template <int DT, bool SWIGLU, int COLS>
__device__ __forceinline__ void vm_issue_b(const VmItem<DT, SWIGLU, COLS> &it, int ks, int lane, uint8_t *buf) {
    using G = VmGeo<DT, SWIGLU, COLS>;
#pragma unroll
    for (int i = 0; i < G::NI; i++) {
        if constexpr (G::kBuf) {
            const int p = min(64 * i + lane, G::POS - 1);
            const int c = p % G::CPR;
            const uint32_t blk = it.src[i] + (uint32_t)(ks * G::BLK);
            dma16_buf(it.rsrc, (blk & ~15u) + 16u * (uint32_t)c, buf + 1024 * i);
        } else {
            const uint8_t *b = G::NMAT == 2 && it.mat[i] ? it.base[G::NMAT - 1] : it.base[0];
            dma16(b + it.src[i] + (uint32_t)(ks * G::BLK), buf + 1024 * i);
        }
    }
    asm volatile("" ::: "memory");
}

// stage ks's A fragments af[4 par + P]: the 8 values the lane's weight operand
// holds at step P of half par (Q4_K: 32 q + 8 P, Q6_K: 32 P + 8 q of the half)
// (lanes of missing pairs load nothing; lane n = 0 always loads, so every load
// instruction issues and the wait counts stay exact)
template <int DT>
__device__ __forceinline__ void vm_issue_a(const _Float16 *arow, bool on, int ks, int q, half8_t (&af)[8]) {
    const _Float16 *p = arow + ks * 256 + (DT == kQ4_K ? 32 : 8) * q;
#pragma unroll
    for (int s = 0; s < 8; s++) af[s] = half8_t{};
    if (on) {
#pragma unroll
        for (int s = 0; s < 8; s++)
            af[s] = *reinterpret_cast<const half8_t *>(p + 128 * (s >> 2) + (DT == kQ4_K ? 8 : 32) * (s & 3));
    }
}

}  // namespace

template <int DT, bool SWIGLU, int COLS, int WPE>
__global__ void __launch_bounds__(64 * VM_WAVES) __attribute__((amdgpu_waves_per_eu(WPE)))
k_vmm(VmmArgs a, const int32_t *__restrict__ perm, const int32_t *__restrict__ runs,
      const float *__restrict__ a_scale) {
    const VmTabs tb{perm, runs, a_scale};
    using G = VmGeo<DT, SWIGLU, COLS>;
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][VM_WAVES][G::BUF];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, q = lane >> 4, kh = q >> 1, hh = q & 1;
    const int gw = blockIdx.x * VM_WAVES + wave, NW = gridDim.x * VM_WAVES;
    const int CB = a.n_out / COLS;
    const int n_items = runs[0] * CB;
    if (gw >= n_items) return;  // wave-uniform; no block barrier in this kernel
    const int nks = a.k / 256;  // even
    const int total = ((n_items - 1 - gw) / NW + 1) * nks;
    uint8_t *const b0 = sB[0][wave], *const b1 = sB[1][wave];

    VmItem<DT, SWIGLU, COLS> cur, nxt;
    vm_item(a, tb, gw, CB, lane, cur);
    nxt = cur;
    half8_t a0[8], a1[8];
    float4_t acc[G::NBLK];
#pragma unroll
    for (int nb = 0; nb < G::NBLK; nb++) acc[nb] = float4_t{0.f, 0.f, 0.f, 0.f};
    vm_issue_a<DT>(cur.arow, cur.aon, 0, q, a0);
    vm_issue_b(cur, 0, lane, b0);

    // stage S from (buf, af); issues stage S + 1 (clamped: the last stage re-copies
    // itself into the other buffer) into (nbuf, naf) first
    // (stage S is stage ks of the wave's item jn; counted along, not divided out)
    int ks = 0, jn = 0;
    auto body = [&](int S, const uint8_t *__restrict__ buf, half8_t (&af)[8], uint8_t *__restrict__ nbuf,
                    half8_t (&naf)[8]) {
        const bool last = S + 1 >= total;
        const int ks1 = last ? ks : (ks + 1 == nks ? 0 : ks + 1);
        if (!last && ks1 == 0) vm_item(a, tb, gw + (jn + 1) * NW, CB, lane, nxt);  // wave-uniform
        wait_lgkmcnt0();  // this wave's reads of nbuf (stage S - 1) have returned
        vm_issue_a<DT>(nxt.arow, nxt.aon, ks1, q, naf);
        vm_issue_b(nxt, ks1, lane, nbuf);
        // stage S's copy and fragments have landed: younger are only stage S + 1's
        wait_vmcnt(8 + G::NI);
        auto half = [&](auto parc) {
            constexpr int PAR = decltype(parc)::value;
            using W = std::conditional_t<DT == kQ4_K, VmQ4, WB<DT>>;
            W wb[G::NBLK];
#pragma unroll
            for (int nb = 0; nb < G::NBLK; nb++) {
                const uint8_t *slot = buf + (16 * nb + n) * G::SLOT;
                if constexpr (DT == kQ4_K) {
                    wb[nb].template load<PAR>(slot, q);
                } else {
                    vm_load(wb[nb], slot, kh, (cur.rowpos[nb] + (uint32_t)(ks * G::BLK)) & 15u, PAR);
                    wb[nb].template prep<PAR>(kh);
                }
            }
#pragma unroll
            for (int P = 0; P < 4; P++) {
                // every column block's weight operand first, then the MFMAs: no MFMA
                // waits on the instruction just before it (hazard nops 214 -> 85 in the
                // gate/up loop; C2 278.9 -> 276.6 us)
                half8_t bf[G::NBLK];
#pragma unroll
                for (int nb = 0; nb < G::NBLK; nb++) {
                    if constexpr (DT == kQ4_K) bf[nb] = wb[nb].step(P);
                    else bf[nb] = wb[nb].step(P, hh);
                }
#pragma unroll
                for (int nb = 0; nb < G::NBLK; nb++)
                    acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[4 * PAR + P], bf[nb], acc[nb], 0, 0, 0);
            }
        };
        half(std::integral_constant<int, 0>{});
        half(std::integral_constant<int, 1>{});
        if (ks == nks - 1) {  // the item's last stage: its outputs, then the next item
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (cur.pv[r] < 0) continue;
                float *orow = a.out + (int64_t)cur.pv[r] * a.n_out + cur.cb * COLS + n;
                if constexpr (SWIGLU) {
#pragma unroll
                    for (int h = 0; h < G::NBLK / 2; h++) {
                        const float g = acc[h][r] * cur.ps[r], u = acc[G::NBLK / 2 + h][r] * cur.ps[r];
                        orow[16 * h] = g / (1.0f + expf(-g)) * u;  // silu(g) * u (silu_mul.metal:57-72)
                    }
                } else {
#pragma unroll
                    for (int nb = 0; nb < G::NBLK; nb++) orow[16 * nb] = acc[nb][r] * cur.ps[r];
                }
            }
#pragma unroll
            for (int nb = 0; nb < G::NBLK; nb++) acc[nb] = float4_t{0.f, 0.f, 0.f, 0.f};
            cur = nxt;
            jn++;
        }
        ks = ks1;
    };
    for (int S = 0; S < total; S += 2) {
        body(S, b0, a0, b1, a1);
        body(S + 1, b1, a1, b0, a0);
    }
    wait_vmcnt(0);  // the clamped re-copy has landed before the wave's LDS can be reused
}

namespace {
int vm_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = v;
    }
    return cus[dev];
}
}  // namespace

bool vmm_supported(int gate_dtype, int down_dtype, int hidden, int ff, int64_t gu_row_bytes, int64_t d_row_bytes) {
    // both contractions need an even number of super-blocks and 32-column
    // blocks; Q4_K copies read whole 16-byte-aligned blocks
    return gate_dtype == kQ4_K && (down_dtype == kQ4_K || down_dtype == kQ6_K) && hidden % 512 == 0 &&
           ff % 512 == 0 && gu_row_bytes % 16 == 0 && (down_dtype != kQ4_K || d_row_bytes % 16 == 0) &&
           (int64_t)hidden * 2 < (int64_t)1 << 31;
}

// columns per item and waves per SIMD of the SwiGLU (gate/up) and plain (down)
// kernels
#ifndef MX_VMM_GU_COLS
#define MX_VMM_GU_COLS 32
#endif
#ifndef MX_VMM_GU_WPE
#define MX_VMM_GU_WPE 2
#endif
#ifndef MX_VMM_DN_COLS
#define MX_VMM_DN_COLS 32
#endif
#ifndef MX_VMM_DN_WPE
#define MX_VMM_DN_WPE 2
#endif

namespace {
template <int DT, bool SWIGLU, int COLS, int WPE>
void vm_launch(const VmmArgs &a, int max_runs, hipStream_t s) {
    using G = VmGeo<DT, SWIGLU, COLS>;
    const int64_t items = (int64_t)max_runs * (a.n_out / COLS);
    const int64_t want = (items + VM_WAVES - 1) / VM_WAVES;
    // resident workgroups per CU: WPE by registers (4 waves each), and by LDS
    const int by_lds = (160 * 1024) / (2 * VM_WAVES * G::BUF);
    const int64_t cap = (int64_t)(WPE < by_lds ? WPE : by_lds) * vm_cus();
    const unsigned grid = (unsigned)(want < cap ? want : cap);
    hipLaunchKernelGGL((k_vmm<DT, SWIGLU, COLS, WPE>), dim3(grid), dim3(64 * VM_WAVES), 0, s, a, a.perm, a.runs,
                       a.a_scale);
}
}  // namespace

mx_status launch_vmm(int dtype, bool swiglu, const VmmArgs &a, int max_runs, hipStream_t s) {
    if (max_runs == 0) return MX_OK;
    if (dtype == kQ4_K && swiglu) vm_launch<kQ4_K, true, MX_VMM_GU_COLS, MX_VMM_GU_WPE>(a, max_runs, s);
    else if (dtype == kQ4_K) vm_launch<kQ4_K, false, MX_VMM_DN_COLS, MX_VMM_DN_WPE>(a, max_runs, s);
    else if (dtype == kQ6_K && !swiglu) vm_launch<kQ6_K, false, MX_VMM_DN_COLS, MX_VMM_DN_WPE>(a, max_runs, s);
    else return fail(MX_ERR_DTYPE, "verify tiles: unsupported weight type %d", dtype);
    MX_LAUNCH("k_vmm");
    return MX_OK;
}

}  // namespace mx
