// Internal launcher interface between the C-ABI layer (mx_api.hip) and the
// kernel translation units.  Launchers assume validated arguments.
#pragma once

#include "mx_common.h"

namespace mx {

// mx_dequant.hip
mx_status launch_dequantize(int dtype, const uint8_t *blocks, int64_t n, float *out,
                            hipStream_t s);
mx_status launch_synth(int dtype, uint64_t key, uint8_t *dst, int64_t nbytes, hipStream_t s);
uint64_t tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id);

// mx_mv.hip -- gather mat-vec.  `ids` may be NULL (plain mat-vec: expert 0).
struct MvArgs {
    const uint8_t *w;       // first block of expert 0
    int64_t expert_bytes;   // n_out * row_bytes
    int64_t row_bytes;
    int n_expert, n_out, k;
    const float *x;
    int x_per_row;
    const uint32_t *ids;    // [t, top_k] or NULL
    int t, top_k;
    float *dst;             // [t, top_k, n_out]
};
mx_status launch_mul_mv_id(int dtype, const MvArgs &a, hipStream_t s);
// true when the LDS-ring mat-vec (k_mul_mv_id) takes this shape; otherwise
// launch_mul_mv_id runs the f32 mat-vec (mx_mvf.hip)
bool mv_ring_fits(int dtype, int k);

// mx_mvf.hip -- f32 gather mat-vec for any k (a multiple of the block size).
// dst row of (token, slot): (token * dst_stride + slot + dst_add) * n_out.
struct MvfArgs {
    const uint8_t *w;
    int64_t expert_bytes, row_bytes;
    int n_expert, n_out, k;
    const float *x;
    int x_per_row;
    const uint32_t *ids;    // [t, top_k] or NULL (expert 0)
    int t, top_k;
    float *dst;
    int dst_stride, dst_add;
};
mx_status launch_mv_f32(int dtype, const MvfArgs &a, hipStream_t s);

// Fused decode layer pieces (mx_mv.hip).
struct DecodeGateUpArgs {
    const uint8_t *gate, *up;            // routed stacks (first block of expert 0)
    int64_t gu_expert_bytes, gu_row_bytes;
    const uint8_t *sh_gate, *sh_up;      // shared expert (or NULL)
    int64_t sh_row_bytes;
    int n_expert, ff, hidden;
    const uint8_t *xstage;               // [t] staged rows of x (mx_stage.h), xstage_bytes(hidden) each
    const uint32_t *ids;                 // [t, top_k]
    int t, top_k;
    float *act;                          // [t, slots, ff], slots = top_k + (sh_gate != NULL)
    const uint8_t *xstage_gm;            // NULL, or the group-major copy of xstage (Q4_K / Q5_K reads)
    // NULL, or the launch order of the (token, slot) pairs, [t * slots] of
    // (tok * slots + slot) | expert << 16 (the shared slot: n_expert), pairs of
    // one expert adjacent (launch_pair_order)
    const int32_t *perm;
    // t == 1 with the 64-group kernel: the top-k runs in every routed block from
    // the router's keys/probs [n_expert] (NULL: ids come from k_decode_select),
    // and block (0, 0) writes ids/w for the down kernel and the caller
    const uint64_t *sel_keys;
    const float *sel_probs;
    float sel_scale;
    int sel_apply, sel_norm;
    uint32_t *sel_ids;
    float *sel_w;
};
// Whether launch_decode_gate_up can run the top-k itself for these arguments
// (t == 1, the 64-group kernel, n_expert <= 256).
bool decode_gate_up_selects(int dtype, const DecodeGateUpArgs &a);
// Verify blocks (t > 1): orders the t * slots (token, slot) pairs by expert (the
// shared slot as expert n_expert) into perm, so the gate/up blocks of pairs that
// share an expert run back to back on one XCD and the repeats read its L2.
// t * slots <= PAIR_ORDER_MAX; the order within an expert is unspecified.
#ifndef MX_PAIR_ORDER_MAX
#define MX_PAIR_ORDER_MAX 4096
#endif
constexpr int PAIR_ORDER_MAX = MX_PAIR_ORDER_MAX;
constexpr int PAIR_ORDER_THREADS = 1024;  // one workgroup; each thread orders up to 4 pairs
static_assert(PAIR_ORDER_MAX % PAIR_ORDER_THREADS == 0 && PAIR_ORDER_MAX <= 4 * PAIR_ORDER_THREADS,
              "pairs per thread");
// the decode kernels take expert-ordered pairs up to this many (verify blocks)
constexpr int PAIR_ORDER_DECODE_MAX = 1024;
// runs (optional, 2 * (t * slots + 1) words): runs[0] = the number of runs, run r
// at runs[2 + 2r] = first perm position | pairs << 16 (1..16 pairs), runs[3 + 2r] =
// its expert: every expert's pairs cut into consecutive runs of at most 16.
mx_status launch_pair_order(const uint32_t *ids, int t, int top_k, int n_expert, int slots, int32_t *perm,
                            hipStream_t s, int32_t *runs = nullptr);
// Decode top-k (decode router split): block i < n_sel selects token i from
// keys/probs [n_sel, n_expert] (written by launch_route_fused) into ids/w
// [n_sel, top_k].
struct DecodeSelArgs {
    const uint64_t *keys;
    const float *probs;
    int n_expert, n_sel;
    float scale;
    int apply_scale, norm;
    uint32_t *ids;
    float *w;
};
mx_status launch_decode_select(int top_k, const DecodeSelArgs &sel, hipStream_t s);
// Slots slot0 .. slot0 + nslot - 1 of every token (slot top_k = the shared
// expert, which must have the routed experts' quant type).
mx_status launch_decode_gate_up(int dtype, const DecodeGateUpArgs &a, int slot0, int nslot, hipStream_t s);
// true when the fused decode kernels take a layer of these shapes (their DMA
// batches and LDS fit); checked before any launch of a forward
bool decode_gate_up_fits(int dtype, int hidden, int64_t row_bytes);
bool decode_down_fits(int dtype, int ff, int64_t row_bytes);

struct DecodeDownArgs {
    const uint8_t *down;
    int64_t d_expert_bytes, d_row_bytes;
    const uint8_t *sh_down;              // shared down of the routed quant type, or NULL
    int64_t sh_row_bytes;
    const float *shared_out;             // [t, hidden] precomputed shared expert, or NULL
    int n_expert, ff, hidden;
    const float *act;                    // [t, top_k + (sh_down != NULL), ff]
    const uint32_t *ids;                 // [t, top_k]
    const float *w;                      // [t, top_k]
    const float *residual;               // [t, hidden] or NULL
    int t, top_k;
    float *out;                          // [t, hidden]
    float *part;                         // [t, top_k + (sh_down != NULL), hidden] scratch
    const int32_t *perm;                 // NULL, or the expert-ordered pair list (DecodeGateUpArgs::perm)
};
mx_status launch_decode_down(int dtype, const DecodeDownArgs &a, hipStream_t s);

// mx_route.hip
// router: [n_expert, hidden] (GGUF ffn_gate_inp layout)
mx_status launch_route_logits(const float *x, const float *router, int t, int hidden,
                              int n_expert, float *logits, hipStream_t s);
// parts > 1: logits are launch_route_logits_split's partial sums, added first
mx_status launch_route_select(const float *logits, const float *bias, int t, int n_expert,
                              int top_k, float scale, int apply_scale, int norm, uint32_t *ids,
                              float *w, hipStream_t s, int parts = 1);
// K splits of the logits GEMM for this shape (1: none): grids under 256
// workgroups split K into 2, 4 or 8 parts
int route_logits_splits(int t, int hidden, int n_expert);
// the logits as `splits` partial sums parts[splits][t][n_expert] (splits ==
// route_logits_splits(...); 1: the logits themselves)
mx_status launch_route_logits_split(const float *x, const float *router, int t, int hidden, int n_expert,
                                    float *parts, int splits, hipStream_t s);
// Decode router, first half: RMSNorm (optional) + logits -> sigmoid
// probabilities and selection sort keys for t tokens (ws: keys u64 [t, E] |
// probs f32 [t, E]); also stages the (normalised) rows into `xstage`
// (mx_stage.h layout) and/or writes them to `x_normed` when non-NULL, and (no
// RMSNorm) as f16 rows times a per-row power of two, in the Q4_K verify tiles'
// K order (launch_to_f16_rows with perm), into x16 / x16s when
// non-NULL.  The top-k runs in k_decode_select (launch_decode_select).
size_t route_fused_ws_bytes(int t, int hidden, int n_expert);
int route_fused_max_t();
mx_status launch_route_fused(const float *x, const float *rms_alpha, float rms_eps,
                             float *x_normed, const float *router, const float *bias, int t,
                             int hidden, int n_expert, void *ws, uint8_t *xstage, uint8_t *xstage_gm,
                             hipStream_t s,
                             _Float16 *x16 = nullptr, float *x16s = nullptr);
// Stages t rows of k values (mx_stage.h layout, xstage_bytes(k) per row).
// xstage_gm: optional group-major copy (mx_stage.h; k % 64 == 0)
mx_status launch_stage_rows(const float *x, int t, int k, uint8_t *xstage, uint8_t *xstage_gm, hipStream_t s);
size_t stage_row_bytes(int k);

// mx_elem.hip
mx_status launch_silu_mul(const float *g, const float *u, int64_t n, float *dst, hipStream_t s);
mx_status launch_combine(const float *down, const float *col_l2, const float *w, int seq,
                         int top_k, int n_out, float *dst, hipStream_t s);
mx_status launch_rms_norm(const float *x, const float *alpha, int rows, int dim, float eps,
                          float *dst, hipStream_t s);
mx_status launch_check_ids(const uint32_t *ids, int64_t t, int top_k, int n_expert, uint32_t *flags,
                           hipStream_t s);
mx_status launch_add3(const float *a, const float *b, const float *c, int64_t n, float *dst,
                      hipStream_t s);
// plain streaming read of nbytes (a multiple of 16) from 16-byte-aligned src
mx_status launch_read_probe(const void *src, int64_t nbytes, uint32_t *sink, hipStream_t s);

// mx_mm.hip -- bucketing + grouped GEMM
//
// Bucket map (map0 scratch), int32 words:
//   tpe[E] pairs per expert | off[E+1] first list position per expert |
//   n_tiles | dup flags | tiles[t_max] (expert << 16 | m-tile) |
//   list[t*top_k] pair indices (token*top_k + slot), grouped by expert, tokens
//   ascending | chunk[nchunks][E] per-chunk counts (scratch of the build).
// Sized for the smallest m-tile (MM_BM pairs); launch_map0 cuts m-tiles of
// `bm` >= MM_BM pairs.
constexpr int MM_BM = 64;
#ifndef MX_BK_CHUNK
#define MX_BK_CHUNK 32
#endif
constexpr int BK_CHUNK = MX_BK_CHUNK;  // tokens per bucket chunk (C3 bucket pass: 16 / 32 / 48 / 64 / 128 tokens 32.4 / 29.8 / 32.3 / 32.0 / 44 us)
struct MapLayout {
    int64_t tpe, off, n_tiles, dup, tiles, list, chunk;  // word offsets
    int64_t t_max, nchunks, words;
    __host__ __device__ MapLayout(int n_expert, int t, int top_k) {
        const int64_t pairs = (int64_t)t * top_k;
        t_max = (pairs + MM_BM - 1) / MM_BM + n_expert;
        nchunks = (t + BK_CHUNK - 1) / BK_CHUNK;
        tpe = 0;
        off = n_expert;
        n_tiles = off + n_expert + 1;
        dup = n_tiles + 1;
        tiles = dup + 1;
        list = tiles + t_max;
        chunk = list + pairs;
        words = chunk + nchunks * n_expert;
    }
};
size_t map0_bytes(int n_expert, int t, int top_k);
// routed_k (0: top_k): ids per token in `ids`; slots routed_k .. top_k - 1 of
// every token go to expert n_expert - 1 (a shared expert joined to the map).
mx_status launch_map0(const uint32_t *ids, int t, int top_k, int n_expert, int32_t *scratch,
                      hipStream_t s, int bm = MM_BM, int routed_k = 0);
struct MmArgs {
    const uint8_t *w;
    int64_t expert_bytes, row_bytes;
    int n_expert, n_out, k;
    const float *x;          // [t, x_per_row, k] f32
    int x_per_row;
    int t, top_k;
    const int32_t *map;      // map0 scratch
    float *dst;              // [t, top_k, n_out]
};
mx_status launch_mul_mm_id(int dtype, const MmArgs &a, hipStream_t s);

// mx_gemm.hip -- MFMA grouped GEMM of the fused prefill path.
// A operand: f16 rows scaled by a power of two per row (x = a * a_scale).
constexpr int GM_BM = 128;   // pairs per m-tile (launch_map0 with bm = GM_BM)
struct GemmArgs {
    const uint8_t *w[2];        // routed stacks (first block of expert 0): [0] = gate / the
                                // only matrix, [1] = up (SwiGLU)
    const uint8_t *w_sh[2];     // map expert n_expert: shared expert (n_expert == 1 stacks)
    int64_t expert_bytes, row_bytes, sh_row_bytes;
    int n_expert, n_out, k;     // k % 256 == 0
    const _Float16 *a;          // [rows, k]
    const float *a_scale;       // [rows]
    int a_div;                  // > 0: A row = pair / a_div (top_k: one row per token, 1: one
                                // per pair), 0: A row = bucket position
    int t, top_k, n_map_expert; // map geometry
    const int32_t *map;         // built with bm = GM_BM
    float *out;                 // SwiGLU: act [position, n_out]; plain: rows
                                // (pair / top_k) * out_stride + pair % top_k + out_add
    int out_stride, out_add;
};
bool gemm_supported(int dtype, int k);
// the kernel's 32-bit operand offsets hold for t tokens of x [t, hidden] and
// weight rows of these byte widths
bool gemm_fits(int t, int hidden, int ff, int64_t gu_row_bytes, int64_t d_row_bytes);
// the same for one plain GEMM over a_rows A rows addressed by pair (a_div > 0)
bool gemm_plain_fits(int64_t a_rows, int k, int n_out, int64_t row_bytes);
mx_status launch_gemm(int dtype, bool swiglu, const GemmArgs &a, hipStream_t s);
// rows of x (f32, [rows, k], k % 4 == 0) -> f16 times a per-row power of two;
// rows at or beyond *count (when count != NULL) are skipped.  perm: each group of
// four values stored in the order 0, 2, 1, 3 (the K order of the Q4_K verify tiles);
// src (when not NULL): output row r holds x row src[r] (a gather, e.g. into bucket order)
mx_status launch_to_f16_rows(const float *x, int64_t rows, int k, const int32_t *count, _Float16 *y,
                             float *scale, hipStream_t s, bool perm = false, const int32_t *src = nullptr);
// out[t, n] = residual + (sum_s w[t, s] * down[t * kk + s] + shared), kk = top_k + has_shared,
// shared = down[t * kk + top_k] (has_shared), shared_sep[t] (shared_sep != NULL) or 0; n % 4 == 0
mx_status launch_combine_prefill(const float *down, const float *w, const float *residual, int t, int top_k,
                                 int has_shared, int n, float *out, hipStream_t s, const float *shared_sep = nullptr);

// mx_vmm.hip -- verify blocks on MFMA (16-pair tiles, each touched expert's
// weights streamed once).  Output row of pair v = tok * slots + slot: out[v].
struct VmmArgs {
    const uint8_t *w[2];        // routed stacks: gate, up (SwiGLU) / the only matrix
    const uint8_t *w_sh[2];     // run expert n_expert: the shared expert
    int64_t expert_bytes, row_bytes, sh_row_bytes;
    int n_expert, n_out, k;     // k % 512 == 0, n_out % 32 == 0
    const _Float16 *a;          // A rows, f16 scaled by a_scale (x = a * a_scale)
    const float *a_scale;
    int a_slots;                // A row of pair v: v / a_slots
    const int32_t *perm, *runs; // launch_pair_order
    float *out;                 // [pairs, n_out]; SwiGLU: silu(gate) * up
};
bool vmm_supported(int gate_dtype, int down_dtype, int hidden, int ff, int64_t gu_row_bytes, int64_t d_row_bytes);
// max_runs: an upper bound of runs[0] (the grid is sized from it)
mx_status launch_vmm(int dtype, bool swiglu, const VmmArgs &a, int max_runs, hipStream_t s);

}  // namespace mx
