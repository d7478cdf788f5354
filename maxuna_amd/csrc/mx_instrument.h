/*
 * maxuna_moe instrumentation -- bench-only entry points of libmaxuna_moe.so.
 *
 * These are NOT part of the drop-in boundary (include/maxuna_moe.h): the
 * reference's MoE interface (src/moe.rs:19-21, src/ops/ files) has no
 * counterpart, and a host binding for the reference never calls them.  They
 * exist so bench.py can time the decode stages inside a replayed graph and
 * read per-stage event times.  mx_moe_forward_repeat with times != 1 gives
 * wrong outputs by design (it skips or repeats a stage).
 */
#ifndef MX_INSTRUMENT_H
#define MX_INSTRUMENT_H

#include "../../include/maxuna_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Same as mx_moe_forward, and additionally records a HIP event after each
 * stage on `stream`, waits for the last one and returns the stage durations
 * in milliseconds.  Decode (t < mm_min_seq): router (fused router: logits,
 * sort keys and activation staging; else logits + top-k), top-k (fused router:
 * k_decode_select, and for a verify block the expert-ordered pair list; empty
 * otherwise, and at t = 1 when the 64-group gate/up kernel runs the top-k in its
 * own blocks), routed + shared gate/up + SwiGLU, down + combine.
 * Grouped path: route, map0, x -> f16, then per bucket map gate/up GEMM +
 * SwiGLU, act -> f16, down GEMM (one map when the shared expert has the
 * routed quant types, else a second map for it), then combine.  For profiling
 * and the benchmark; no reference counterpart.  Not capturable. */
mx_status mx_moe_forward_profiled(const mx_moe_layer *layer, const float *x, int64_t t,
                                  const float *residual, float *out, uint32_t *ids_out,
                                  float *w_out, void *workspace, size_t workspace_bytes,
                                  mx_stream_t stream, float *stage_ms, int32_t max_stages,
                                  int32_t *n_stages);

/* Same as mx_moe_forward, with the kernels of decode stage `stage` (0 router
 * logits + staging, 1 top-k (nothing at t = 1 when gate/up selects in its own
 * blocks), 2 routed + shared gate/up, 3 down + combine; the
 * fused-router decode path, t < mm_min_seq <= 32) launched `times` times (0..16).  times = 0 skips
 * the stage: the later stages then read what the workspace holds from the
 * previous forward of the same layer (valid inputs, stale results) -- a graph
 * of layers with one stage skipped, subtracted from the full graph, gives that
 * stage's time inside the replayed pipeline.  Every stage recomputes its
 * outputs from its inputs, so times > 1 leaves the result unchanged; `residual`
 * must not alias `out` then.  Capturable.  For profiling and the benchmark; no
 * reference counterpart. */
mx_status mx_moe_forward_repeat(const mx_moe_layer *layer, const float *x, int64_t t,
                                const float *residual, float *out, uint32_t *ids_out, float *w_out,
                                void *workspace, size_t workspace_bytes, mx_stream_t stream,
                                int32_t stage, int32_t times);

/* A plain streaming read of nbytes (multiple of 16) from src (16-byte aligned),
 * 512 x 256 threads with four 16-byte loads in flight each: the achievable HBM
 * read rate the expert kernels are compared with.  `sink` receives nothing in
 * practice.  Capturable.  For the benchmark; no reference counterpart. */
mx_status mx_probe_read(const void *src, int64_t nbytes, uint32_t *sink, mx_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
