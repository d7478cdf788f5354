/*
 * CPU oracle for the quantized indexed-MoE hot path -- TEST INFRASTRUCTURE.
 *
 * A plain-C restatement of the reference's `--moe-impl reference` semantics
 * (crate `laguna`, /root/reference).  It is the checker the GPU path is
 * compared against; nothing in the shipped library links or calls it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function cites the reference file:line it restates.  Dot products are
 * accumulated in double and rounded to f32 at each op boundary where the
 * reference materialises an f32 tensor (matmul output, silu, mul, combine).
 * Compile with -ffp-contract=off: dequantisation rounds each product and
 * difference separately, exactly as the GGUF formulas are written.
 */
#ifndef MAXUNA_MOE_ORACLE_H
#define MAXUNA_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type codes (GgmlDType ids in GGUF). */
enum { OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14 };

int    or_block_size(int dtype);   /* weights per block (-1 if unsupported) */
int    or_type_size(int dtype);    /* bytes per block   (-1 if unsupported) */

float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);   /* round-to-nearest-even */

/* Dequantise n weights (n % block_size == 0) of raw blocks to f32. */
int or_dequantize(int dtype, const uint8_t *blocks, int64_t n, float *out);

/* Seeded synthetic GGUF blocks: bytes [byte_off, byte_off+nbytes) of a tensor
 * of `n_blocks_total` blocks identified by `key` (see or_tensor_key). */
uint64_t or_mix64(uint64_t z);
uint64_t or_tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id);
int or_synth_blocks(int dtype, uint64_t key, int64_t byte_off, int64_t nbytes,
                    uint8_t *out);

/* Routing (moe.rs:84-119). logits [t,E]; bias [E]; ids [t,k]; w [t,k]. */
void or_route_logits(const float *x, const float *router_t, int64_t t,
                     int64_t hidden, int64_t n_expert, float *logits);
void or_route_from_logits(const float *logits, const float *bias, int64_t t,
                          int64_t n_expert, int64_t top_k, double scale,
                          int norm, uint32_t *ids, float *w);

/* Brute-force gather mat-vec (dispatch.rs:2273-2301): dst [t,top_k,n_out].
 * `experts[e]` points at expert e's raw blocks (n_out rows of k weights); an
 * entry may be NULL if no id selects it. */
int or_mul_mv_id(int dtype, const uint8_t *const *experts, int64_t n_expert,
                 int64_t n_out, int64_t k, const float *x, int64_t x_per_row,
                 const uint32_t *ids, int64_t t, int64_t top_k, float *dst);

/* Plain quantised mat-vec: dst[t,n_out] = W[n_out,k] . x[t,k]. */
int or_mul_mv(int dtype, const uint8_t *w, int64_t n_out, int64_t k,
              const float *x, int64_t t, float *dst);

/* map0 bucket (mm_id.metal:207-259): tpe[E]; hids[E*t] = token*top_k+slot. */
int or_map0(const uint32_t *ids, int64_t t, int64_t top_k, int64_t n_expert,
            int32_t *tpe, int32_t *hids);

void or_silu_mul(const float *gate, const float *up, int64_t n, float *dst);
void or_combine(const float *down, const float *col_l2, const float *w,
                int64_t seq, int64_t top_k, int64_t n_out, float *dst);
void or_rmsnorm(const float *x, const float *alpha, int64_t rows, int64_t dim,
                float eps, float *dst);

/* ReferenceExperts::forward (moe.rs:141-187).  out [t,hidden]. */
int or_reference_experts(int gate_dt, const uint8_t *const *gate,
                         int up_dt, const uint8_t *const *up,
                         int down_dt, const uint8_t *const *down,
                         int64_t n_expert, int64_t hidden, int64_t ff,
                         const float *x, const uint32_t *ids, const float *w,
                         int64_t t, int64_t top_k, float *out);

/* SharedExpert::forward / swiglu (moe.rs:342-344, 369-374). out [t,hidden]. */
int or_swiglu(int gate_dt, const uint8_t *gate, int up_dt, const uint8_t *up,
              int down_dt, const uint8_t *down, int64_t hidden, int64_t ff,
              const float *x, int64_t t, float *out);

/* Number of OpenMP threads the oracle uses (1 when built without OpenMP). */
int or_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
