/*
 * maxuna_moe -- MI355X (gfx950) quantized indexed-MoE hot path, C ABI.
 *
 * Plain pointers and sizes only.  Every tensor argument is a DEVICE pointer
 * (HIP global memory) unless stated otherwise; every call is enqueued on the
 * given HIP stream and returns before the work completes.  Outputs are
 * caller-allocated.  All argument validation happens on the host before any
 * launch; a non-zero status means nothing was enqueued and mx_last_error()
 * describes why (thread-local text).  No C++ exception crosses this boundary.
 *
 * Each entry point cites the reference (crate `laguna`) interface it replaces
 * as file:line into the reference tree.
 *
 * Quantised weights are raw GGUF/ggml blocks, read in place (no repacking):
 *   Q4_K (type 12): 144-byte super-blocks of 256 weights
 *   Q5_K (type 13): 176-byte super-blocks of 256 weights
 *   Q6_K (type 14): 210-byte super-blocks of 256 weights
 *   Q8_0 (type  8):  34-byte blocks of 32 weights
 * An expert stack is [n_expert, n_out, k] expert-major: row stride
 * k/block_size*type_size bytes, expert stride n_out*row_stride bytes.
 */
#ifndef MAXUNA_MOE_H
#define MAXUNA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *mx_stream_t; /* == hipStream_t; NULL = default stream */

/* ---- status codes (one per host validation class, dispatch.rs:812-847) ---- */
typedef int32_t mx_status;
#define MX_OK                 0
#define MX_ERR_NULL           1  /* a required pointer is NULL                      */
#define MX_ERR_SHAPE          2  /* dimensions disagree (k, t, top_k, n_expert ...) */
#define MX_ERR_DTYPE          3  /* quant type not supported by this entry point    */
#define MX_ERR_BLOCK          4  /* k is not a multiple of the quant block size     */
#define MX_ERR_XPR            5  /* x_per_row is neither 1 nor top_k                */
#define MX_ERR_SCRATCH        6  /* workspace too small / map0 geometry mismatch    */
#define MX_ERR_OVERFLOW       7  /* index math would overflow int32                 */
#define MX_ERR_TOPK           8  /* top_k out of range (0 < top_k <= min(E, 32))    */
#define MX_ERR_ALIGN          9  /* pointer misaligned for its element type         */
#define MX_ERR_HIP           10  /* the HIP runtime reported an error               */
#define MX_ERR_IO            11  /* a file could not be opened or read              */
#define MX_ERR_FORMAT        12  /* a GGUF file is malformed or unsupported         */
#define MX_ERR_NOT_FOUND     13  /* no tensor / metadata key of that name           */

/* GGML type ids (GgmlDType). */
#define MX_Q8_0  8
#define MX_Q4_K 12
#define MX_Q5_K 13
#define MX_Q6_K 14

/* Thread-local text for the last non-zero status returned on this thread. */
const char *mx_last_error(void);
/* Library version string. */
const char *mx_version(void);

/* Weights per block / bytes per block for a ggml type; -1 if unsupported. */
int32_t mx_block_size(int32_t dtype);
int32_t mx_type_size(int32_t dtype);

/* A stacked expert tensor in GGUF layout.  Replaces `ExpertStack`
 * (src/gguf.rs:247-276): `data` is the device allocation, `base_off` the byte
 * offset of the first block inside it (gguf.rs:264-270). */
typedef struct mx_expert_stack {
    const void *data;
    uint64_t base_off;
    int32_t dtype;
    int32_t reserved;
    int64_t n_expert;
    int64_t n_out;
    int64_t k;
} mx_expert_stack;

/* ---- dequantisation ------------------------------------------------------
 * out[0..n) = dequantised weights of the raw blocks, bit-exact with the GGUF
 * formulas (candle QTensor::dequantize as used by moe.rs:173-175; block math
 * mm_id.metal:75-167).  n % block_size == 0. */
mx_status mx_dequantize(int32_t dtype, const void *blocks, int64_t n, float *out,
                        mx_stream_t stream);

/* ---- decode gather mat-vec ------------------------------------------------
 * Replaces ops::mv_id::mul_mv_id (src/ops/mv_id.rs:37-45 -> dispatch.rs:775,
 * kernel_mul_mv_id_*_f32_v mv.metal:680-731).
 *   x   [t, x_per_row, k] f32, x_per_row in {1, top_k}
 *   ids [t, top_k] u32 (ids_t must equal t)
 *   dst [t, top_k, n_out] f32:  dst[i,s,:] = W[ids[i,s]] . x[i, x_per_row==1 ? 0 : s]
 * Supported: Q4_K, Q5_K, Q6_K, Q8_0, any k that is a multiple of the block
 * size (rows the LDS-ring kernel cannot hold take an f32 kernel).  Out-of-range
 * ids are clamped into range on the device (no fault); mx_check_ids detects
 * them. */
mx_status mx_mul_mv_id(const mx_expert_stack *stack, const float *x, int64_t t,
                       int64_t x_per_row, int64_t k, const uint32_t *ids, int64_t ids_t,
                       int64_t top_k, float *dst, mx_stream_t stream);

/* Validates routing ids on the device, the fail-closed check the reference's
 * host-side validation (dispatch.rs:812-847) cannot make on device-resident
 * ids: *flags (one device u32, written by a single store) becomes
 * (1 if some token repeats an id across its top_k slots) | (2 if some id is
 * >= n_expert).  The gather kernels clamp an out-of-range id into range (no
 * fault, wrong expert) and the bucket pass collapses repeats (mm_id.metal:
 * 243-251), so callers that take ids from outside the router check them here.
 * Ids produced by mx_route_from_logits / mx_moe_forward are always valid.
 * Cost: one 1024-thread workgroup walks every token (top_k^2 / 2 compares
 * each), so its time grows linearly with t on a single CU -- a validation
 * step for ids from outside the router, not for a serving loop's hot path. */
mx_status mx_check_ids(const uint32_t *ids, int64_t t, int64_t top_k, int64_t n_expert,
                       uint32_t *flags, mx_stream_t stream);

/* Plain quantised mat-vec.  Replaces ops::mv_id::mul_mv (mv_id.rs:54-56 ->
 * dispatch.rs:964-1057).  w: [n_out, k] raw blocks; x [t, k]; dst [t, n_out]. */
mx_status mx_mul_mv(const void *w, int32_t dtype, int64_t n_out, int64_t k, const float *x,
                    int64_t t, float *dst, mx_stream_t stream);

/* ---- prefill grouped GEMM (token bucketing + MFMA) -------------------------
 * The map0 scratch replaces dispatch::Map0Scratch (dispatch.rs:752-757).
 * Layout (int32 words, documented for tests):
 *   [0, E)                 tpe[e]       pairs routed to expert e
 *   [E, 2E+1)              off[e]       exclusive prefix of tpe (off[E] = t*top_k)
 *   [2E+1]                 n_tiles      number of (expert, m-tile) work items
 *   [2E+2, 2E+2+T_max)     tiles        expert<<16 | m_tile (m-tiles of 128 pairs),
 *                                       T_max = ceil(t*top_k/64) + E words reserved
 *   then t*top_k words     list         flattened pair ids token*top_k+slot, grouped by
 *                                       expert (ascending e), tokens ascending within e
 *   then chunk tables (internal).
 * Within a token the top_k ids must be distinct (real top-k guarantees it;
 * mm_id.metal:243-251 collapses duplicate slots).  The bucket pass checks this
 * on the device and records a duplicate (1) or an out-of-range id (2) in the
 * dup word at [2E+2]; mx_check_ids gives the same flags without a map. */
typedef struct mx_map0 {
    void *buffer;
    size_t bytes;
    int64_t n_expert;
    int64_t t;
    int64_t top_k;
} mx_map0;

size_t mx_map0_scratch_bytes(int64_t n_expert, int64_t t, int64_t top_k);

/* Replaces ops::mm_id::prepare_map0 (mm_id.rs:27-29 -> dispatch.rs:927-956). */
mx_status mx_prepare_map0(int64_t n_expert, const uint32_t *ids, int64_t t, int64_t top_k,
                          void *scratch, size_t scratch_bytes, mx_stream_t stream);

/* Replaces ops::mm_id::mul_mm_id_shared (mm_id.rs:32-39 -> dispatch.rs:789).
 * Shapes as mx_mul_mv_id; `map` must come from mx_prepare_map0 with the same
 * ids, and its geometry must match (n_expert, t, top_k), else MX_ERR_SCRATCH
 * (dispatch.rs:886-896).  Supported: Q4_K, Q5_K, Q6_K, Q8_0.
 * Up to 2560 (token, slot) pairs (Q4_K / Q6_K, K a multiple of 512, n_out of
 * 32) the projection runs the 16-pair MFMA tiles of the MoE forward's verify
 * blocks; beyond that, when K is a multiple of 256, the prefill path's MFMA
 * GEMM; both over x rounded to f16 (one power-of-two scale per x row).  Their
 * temporaries (the f16 rows, t * x_per_row * (2k + 4) bytes, and the tiles'
 * pair order) are stream-ordered memory from a library pool per device, which
 * keeps its peak size reserved.  Other K run the fallback tiles with no
 * temporary. */
mx_status mx_mul_mm_id_shared(const mx_expert_stack *stack, const float *x, int64_t t,
                              int64_t x_per_row, int64_t k, const uint32_t *ids,
                              int64_t ids_t, int64_t top_k, const mx_map0 *map,
                              float *dst, mx_stream_t stream);

/* Self-contained form (map0 + mm).  Replaces ops::mm_id::mul_mm_id
 * (mm_id.rs:16-18).  workspace >= mx_mul_mm_id_workspace_bytes(...), 256-byte
 * aligned: the map0, then (K a multiple of 256) x's f16 rows; results are
 * bitwise those of mx_mul_mm_id_shared. */
size_t mx_mul_mm_id_workspace_bytes(int64_t n_expert, int64_t t, int64_t top_k,
                                    int64_t x_per_row, int64_t k);
mx_status mx_mul_mm_id(const mx_expert_stack *stack, const float *x, int64_t t,
                       int64_t x_per_row, int64_t k, const uint32_t *ids, int64_t ids_t,
                       int64_t top_k, void *workspace, size_t workspace_bytes, float *dst,
                       mx_stream_t stream);

/* ---- elementwise / glue ----------------------------------------------------- */
/* dst = silu(gate) * up, silu(g) = g / (1 + exp(-g)), f32, each op rounded.
 * Replaces ops::silu_mul (silu_mul.rs:14-16, silu_mul.metal:57-72). */
mx_status mx_silu_mul(const float *gate, const float *up, int64_t n, float *dst,
                      mx_stream_t stream);

/* dst[s,c] = sum_k down[s,k,c] * w[s,k]; with col_l2 != NULL ([seq,top_k]):
 * dst[s,c] = sum_k ((down[s,k,c]*col_l2[s,k]) * 2^-15) * w[s,k].
 * Replaces ops::combine (combine.rs:16-18, combine.metal:70-133). */
mx_status mx_combine(const float *down, const float *col_l2, const float *w, int64_t seq,
                     int64_t top_k, int64_t n_out, float *dst, mx_stream_t stream);

/* RMSNorm: dst = x / sqrt(mean(x^2) + eps) * alpha, rows of `dim`.
 * Replaces the candle RmsNorm on the MoE input (model.rs:340-341). */
mx_status mx_rms_norm(const float *x, const float *alpha, int64_t rows, int64_t dim, float eps,
                      float *dst, mx_stream_t stream);

/* ---- routing -------------------------------------------------------------------
 * logits[t,e] = <x[t,:], router[e,:]> in f32.  Replaces route_logits
 * (src/moe.rs:84-87).  `router` is [n_expert, hidden] -- the GGUF
 * `ffn_gate_inp` tensor as stored; the reference's load-time transpose
 * (moe.rs:43) is not needed. */
mx_status mx_route_logits(const float *x, const float *router, int64_t t, int64_t hidden,
                          int64_t n_expert, float *logits, mx_stream_t stream);

/* probs = sigmoid(logits); selection = probs + bias; stable descending top_k of
 * selection (ties -> lower expert id); w = probs[ids]; if norm:
 * w /= max(sum(w), 6.103515625e-5); if scale not in {0,1}: w *= scale.
 * Replaces route_from_logits (src/moe.rs:94-119).  n_expert <= 1024,
 * top_k <= 32. */
mx_status mx_route_from_logits(const float *logits, const float *bias, int64_t t,
                               int64_t n_expert, int64_t top_k, double scale, int32_t norm,
                               uint32_t *ids, float *w, mx_stream_t stream);

/* ---- whole MoE block ----------------------------------------------------------
 * Replaces MoeBlock::forward (src/moe.rs:73-78) with the FusedExperts runner
 * (moe.rs:221-323) and SharedExpert (moe.rs:327-345):
 *   out = FusedExperts(x, route(x)) + SharedExpert(x)
 * Fewer than 16 tokens run the f32-class fused decode kernels.  From 16 tokens
 * on, the expert matmuls take f16 operands (the reference's grouped-matmul
 * precision class): 16-pair MFMA tiles while t * (top_k + shared) <= 2560, the
 * grouped GEMM beyond that for t >= mm_min_seq (moe.rs:236-240; mm_min_seq == 0
 * selects the default 32, ops/mod.rs:31), else the decode kernels.
 * mm_min_seq < 0 never uses the tiles nor the grouped GEMM (LAGUNA_NO_MM_ID,
 * ops/mod.rs:57-64).  The shared expert is optional (shared_gate.data == NULL).
 * Optionally (rms_alpha != NULL) the block first applies RMSNorm(rms_eps) to
 * `x`: out = residual + MoE(RMSNorm(x)) -- the FFN half of a decoder layer
 * (model.rs:340-351).  `residual` may equal `out` (in-place update of the
 * residual stream) but neither may overlap `x` unless it IS `x` exactly. */
typedef struct mx_moe_layer {
    const float *router;        /* [n_expert, hidden] f32, ffn_gate_inp      */
    const float *exp_probs_b;   /* [n_expert] f32 selection bias (moe.rs:44) */
    mx_expert_stack gate, up, down;           /* routed experts            */
    mx_expert_stack shared_gate, shared_up, shared_down; /* n_expert == 1  */
    int64_t hidden;
    int64_t expert_ff;
    int64_t top_k;
    double weights_scale;       /* expert_weights_scale (config.rs:128)     */
    int32_t weights_norm;       /* expert_weights_norm                      */
    int32_t mm_min_seq;         /* MM_ID_MIN_SEQ; 0 -> 32, <0 -> never mm   */
    const float *rms_alpha;     /* optional [hidden] RMSNorm weight         */
    float rms_eps;
    int32_t reserved;
} mx_moe_layer;

size_t mx_moe_workspace_bytes(const mx_moe_layer *layer, int64_t t);

/* x [t, hidden] f32 -> out [t, hidden] f32.  `residual` is NULL or
 * [t, hidden] f32 and is added to the output.  `ids_out`/`w_out` (optional,
 * [t, top_k]) receive the routing decision.  The workspace holds no state
 * between calls: every forward initialises what it reads, so any bytes will
 * do, and one workspace serves calls of any t (sized for the largest).  Calls
 * that share a workspace must be ordered on one stream.  Every shape that
 * passes validation runs: rows too wide for the fused decode kernels' LDS
 * take the f32 gather mat-vec path (chosen before the first launch). */
mx_status mx_moe_forward(const mx_moe_layer *layer, const float *x, int64_t t,
                         const float *residual, float *out, uint32_t *ids_out, float *w_out,
                         void *workspace, size_t workspace_bytes, mx_stream_t stream);

/* mx_moe_forward with no workspace argument and no allocation of any kind.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The workspace is a device array inside the library,
 * mx_moe_forward_noalloc_max_bytes() = 16 MiB per GPU, held by every GPU the
 * library runs on until the process ends.  A call whose t needs more
 * (mx_moe_workspace_bytes) fails with MX_ERR_SCRATCH before any launch; a
 * C1-shaped layer (hidden 4096, 256 experts, top-10 + shared) fits up to
 * t = 57.  Calls on one GPU share that array: calls that overlap on one GPU
 * (different streams, or different host threads) race; order them on one
 * stream.  Nothing in the array needs clearing between calls. */
size_t mx_moe_forward_noalloc_max_bytes(void);
mx_status mx_moe_forward_noalloc(const mx_moe_layer *layer, const float *x, int64_t t,
                                 const float *residual, float *out, uint32_t *ids_out, float *w_out,
                                 mx_stream_t stream);

/* ---- GGUF ingestion --------------------------------------------------------------
 * A GGUF v2/v3 file: header, typed metadata, tensor table and data section
 * (public GGUF layout).  Replaces what the reference host gets from candle's
 * gguf_file::Content plus its loaders (src/gguf.rs:554-658 expert stacks,
 * gguf.rs:676-687 bias-suffixed f32 tensors, config.rs:115-130 metadata).
 * The handle keeps the file open; tensor bytes are read on request.  Not
 * thread-safe per handle. */
typedef struct mx_gguf mx_gguf;
typedef struct mx_gguf_tensor {
    const char *name;     /* owned by the handle (valid until mx_gguf_close)     */
    int32_t ggml_type;
    int32_t n_dims;
    int64_t ne[4];        /* ggml order: ne[0] is the contiguous (row) dimension;
                             an expert stack [n_expert, n_out, k] has ne = {k, n_out, n_expert} */
    uint64_t offset;      /* absolute file offset of the first byte             */
    uint64_t nbytes;      /* 0 if the ggml type's size is unknown here           */
} mx_gguf_tensor;

mx_status mx_gguf_open(const char *path, mx_gguf **out);
void mx_gguf_close(mx_gguf *g);
uint32_t mx_gguf_version(const mx_gguf *g);
uint64_t mx_gguf_alignment(const mx_gguf *g);
uint64_t mx_gguf_data_offset(const mx_gguf *g);
int64_t mx_gguf_tensor_count(const mx_gguf *g);
mx_status mx_gguf_tensor_at(const mx_gguf *g, int64_t index, mx_gguf_tensor *out);
mx_status mx_gguf_find_tensor(const mx_gguf *g, const char *name, mx_gguf_tensor *out);
/* Metadata: the GGUF value type of `key` (-1 if absent); integers of any width
 * and bool as int64; f32/f64 (or an integer) as double; strings (owned by the
 * handle); arrays as (element type, count). */
int32_t mx_gguf_kv_type(const mx_gguf *g, const char *key);
mx_status mx_gguf_get_int(const mx_gguf *g, const char *key, int64_t *out);
mx_status mx_gguf_get_float(const mx_gguf *g, const char *key, double *out);
mx_status mx_gguf_get_string(const mx_gguf *g, const char *key, const char **out);
mx_status mx_gguf_get_array(const mx_gguf *g, const char *key, int32_t *elem_type, uint64_t *count);
/* Copies a tensor's bytes into host memory (dst_bytes >= t->nbytes). */
mx_status mx_gguf_read_host(const mx_gguf *g, const mx_gguf_tensor *t, void *dst, uint64_t dst_bytes);
/* Copies a tensor's raw bytes into device memory: the file is read in chunks
 * into two pinned host buffers while the previous chunk's DMA runs on
 * `stream`.  Returns after the copy has completed.  The zero-copy mmap view of
 * the reference (gguf.rs:616-658) becomes one upload into HBM. */
mx_status mx_gguf_read(mx_gguf *g, const mx_gguf_tensor *t, void *dst, uint64_t dst_bytes,
                       mx_stream_t stream);

/* ---- synthetic weights (bench/test utility, no reference counterpart) ----------
 * Fills nbytes of a tensor of raw blocks with the library's seeded generator:
 * byte j = byte (j&7) of splitmix64-mix(key + (j/8+1)*0x9E3779B97F4A7C15); the
 * f16 super-block scales are then set to f16(0.001 + 0.009*u). */
uint64_t mx_tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id);
mx_status mx_synth_blocks(int32_t dtype, uint64_t key, void *dst, int64_t nbytes,
                          mx_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
