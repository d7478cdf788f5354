// C-ABI entry points: host-side validation (every check happens before any
// launch, as dispatch.rs:812-847 does), then the launchers.  No exception or
// HIP error escapes as anything but a status code + thread-local text.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "mx_launch.h"
#include "mx_stage.h"
#include "mx_instrument.h"

// bytes of the device-resident workspace of mx_moe_forward_noalloc (per device)
#ifndef MX_NOALLOC_SCRATCH_BYTES
#define MX_NOALLOC_SCRATCH_BYTES (16u << 20)
#endif

namespace mx {

static thread_local char g_err[512] = "";

mx_status fail(mx_status code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

mx_status hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return MX_OK;
    return fail(MX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// the 16-pair MFMA tiles' upper end (MoE forward and the mm_id projections) in (token, slot) pairs: the measured crossover with the
// grouped GEMM on C1-shaped layers (11 slots; 4 layers replayed, µs, tiles vs
// GEMM): t = 200: 760 vs 826, 256: 864 vs 862, 300: 945 vs 900
#ifndef MX_VMM_MAX_PAIRS
#define MX_VMM_MAX_PAIRS 2560
#endif
constexpr int64_t kVmmMaxPairs = MX_VMM_MAX_PAIRS;
static_assert(kVmmMaxPairs <= PAIR_ORDER_MAX, "the pair order covers the tiles' range");

static bool supported(int dt) { return dt == kQ4_K || dt == kQ5_K || dt == kQ6_K || dt == kQ8_0; }
static bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
static const char *dt_name(int dt) {
    return dt == kQ4_K ? "Q4_K" : dt == kQ5_K ? "Q5_K" : dt == kQ6_K ? "Q6_K" : dt == kQ8_0 ? "Q8_0" : "unsupported";
}

// Validates a stack and returns its geometry.
struct StackGeom {
    const uint8_t *w;
    int64_t row_bytes, expert_bytes;
};

static mx_status check_stack(const mx_expert_stack *st, const char *what, StackGeom &g) {
    if (!st) return fail(MX_ERR_NULL, "%s: stack is NULL", what);
    if (!st->data) return fail(MX_ERR_NULL, "%s: stack has no device buffer", what);
    if (!supported(st->dtype))
        return fail(MX_ERR_DTYPE, "%s: no kernel for ggml type %d", what, (int)st->dtype);
    if (st->n_expert <= 0 || st->n_out <= 0 || st->k <= 0)
        return fail(MX_ERR_SHAPE, "%s: empty stack [%lld, %lld, %lld]", what, (long long)st->n_expert,
                    (long long)st->n_out, (long long)st->k);
    const int bs = block_size(st->dtype);
    if (st->k % bs)
        return fail(MX_ERR_BLOCK, "%s: k (%lld) is not a multiple of %s block size %d", what,
                    (long long)st->k, dt_name(st->dtype), bs);
    if (st->n_expert > 32767 || st->n_out > (1 << 30) || st->k > (1 << 24))
        return fail(MX_ERR_OVERFLOW, "%s: stack dimensions exceed the kernels' index range", what);
    g.w = static_cast<const uint8_t *>(st->data) + st->base_off;
    g.row_bytes = st->k / bs * type_size(st->dtype);
    g.expert_bytes = st->n_out * g.row_bytes;
    // Q4_K / Q5_K rows are read with 16-byte loads (144 and 176 are multiples of 16).  Q6_K/Q8_0 blocks are 2-byte aligned
    // inside a row; they are read with 16-bit loads or with 4-byte-aligned dwords
    // that each contain at least one byte of the block (never a byte of an
    // unmapped page), so 2-byte alignment suffices.
    const size_t need = (st->dtype == kQ4_K || st->dtype == kQ5_K) ? 16 : 2;
    if (!aligned(g.w, need))
        return fail(MX_ERR_ALIGN, "%s: first block (data + base_off) must be %zu-byte aligned", what, need);
    return MX_OK;
}

static mx_status check_f32(const float *p, const char *what) {
    if (!p) return fail(MX_ERR_NULL, "%s is NULL", what);
    if (!aligned(p, 16)) return fail(MX_ERR_ALIGN, "%s must be 16-byte aligned", what);
    return MX_OK;
}

// Shapes shared by mv_id / mm_id (dispatch.rs:812-847).
static mx_status check_id_call(const mx_expert_stack *st, const float *x, int64_t t,
                               int64_t x_per_row, int64_t k, const uint32_t *ids, int64_t ids_t,
                               int64_t top_k, float *dst, StackGeom &g) {
    MX_TRY(check_stack(st, "expert stack", g));
    if (t < 0 || top_k < 0) return fail(MX_ERR_SHAPE, "negative t (%lld) or top_k (%lld)", (long long)t, (long long)top_k);
    if (k != st->k)
        return fail(MX_ERR_SHAPE, "x k (%lld) does not match expert stack k (%lld)", (long long)k, (long long)st->k);
    if (ids_t != t)
        return fail(MX_ERR_SHAPE, "ids t (%lld) does not match x t (%lld)", (long long)ids_t, (long long)t);
    if (top_k == 0 || top_k > 64) return fail(MX_ERR_TOPK, "top_k (%lld) must be in 1..64", (long long)top_k);
    if (x_per_row != 1 && x_per_row != top_k)
        return fail(MX_ERR_XPR, "x_per_row (%lld) must be 1 (shared row) or top_k (%lld) (per-slot row)",
                    (long long)x_per_row, (long long)top_k);
    if ((k % 4) != 0) return fail(MX_ERR_SHAPE, "k must be a multiple of 4");
    if (t * top_k > (int64_t)1 << 22 || t * top_k * st->n_out > INT64_C(1) << 40)
        return fail(MX_ERR_OVERFLOW, "t*top_k=%lld exceeds the kernels' index range", (long long)(t * top_k));
    if (t == 0) return MX_OK;
    MX_TRY(check_f32(x, "x"));
    MX_TRY(check_f32(dst, "dst"));
    if (!ids) return fail(MX_ERR_NULL, "ids is NULL");
    return MX_OK;
}

}  // namespace mx

using namespace mx;

extern "C" {

const char *mx_last_error(void) { return g_err; }
const char *mx_version(void) { return "maxuna_moe 0.1.0 gfx950"; }
int32_t mx_block_size(int32_t dtype) { return supported(dtype) ? block_size(dtype) : -1; }
int32_t mx_type_size(int32_t dtype) { return supported(dtype) ? type_size(dtype) : -1; }

mx_status mx_dequantize(int32_t dtype, const void *blocks, int64_t n, float *out, mx_stream_t stream) {
    if (!supported(dtype)) return fail(MX_ERR_DTYPE, "dequantize: no kernel for ggml type %d", (int)dtype);
    if (n < 0) return fail(MX_ERR_SHAPE, "dequantize: negative n");
    if (n % block_size(dtype))
        return fail(MX_ERR_BLOCK, "dequantize: n (%lld) is not a multiple of %s block size %d", (long long)n,
                    dt_name(dtype), block_size(dtype));
    if (n == 0) return MX_OK;
    if (!blocks) return fail(MX_ERR_NULL, "dequantize: blocks is NULL");
    MX_TRY(check_f32(out, "dequantize: out"));
    if (!aligned(blocks, (dtype == kQ4_K || dtype == kQ5_K) ? 16 : 2))
        return fail(MX_ERR_ALIGN, "dequantize: blocks misaligned");
    return launch_dequantize(dtype, static_cast<const uint8_t *>(blocks), n, out, (hipStream_t)stream);
}

mx_status mx_mul_mv_id(const mx_expert_stack *stack, const float *x, int64_t t, int64_t x_per_row,
                       int64_t k, const uint32_t *ids, int64_t ids_t, int64_t top_k, float *dst,
                       mx_stream_t stream) {
    StackGeom g;
    MX_TRY(check_id_call(stack, x, t, x_per_row, k, ids, ids_t, top_k, dst, g));
    if (t == 0) return MX_OK;
    MvArgs a{g.w, g.expert_bytes, g.row_bytes, (int)stack->n_expert, (int)stack->n_out, (int)stack->k,
             x, (int)x_per_row, ids, (int)t, (int)top_k, dst};
    return launch_mul_mv_id(stack->dtype, a, (hipStream_t)stream);
}

mx_status mx_mul_mv(const void *w, int32_t dtype, int64_t n_out, int64_t k, const float *x, int64_t t,
                    float *dst, mx_stream_t stream) {
    mx_expert_stack st{w, 0, dtype, 0, 1, n_out, k};
    StackGeom g;
    MX_TRY(check_stack(&st, "mul_mv weight", g));
    if (t < 0) return fail(MX_ERR_SHAPE, "mul_mv: negative t");
    if (t == 0) return MX_OK;
    MX_TRY(check_f32(x, "x"));
    MX_TRY(check_f32(dst, "dst"));
    if (t > (1 << 22)) return fail(MX_ERR_OVERFLOW, "mul_mv: t too large");
    MvArgs a{g.w, g.expert_bytes, g.row_bytes, 1, (int)n_out, (int)k, x, 1, nullptr, (int)t, 1, dst};
    return launch_mul_mv_id(dtype, a, (hipStream_t)stream);
}

size_t mx_map0_scratch_bytes(int64_t n_expert, int64_t t, int64_t top_k) {
    if (n_expert <= 0 || t < 0 || top_k <= 0) return 0;
    return map0_bytes((int)n_expert, (int)t, (int)top_k);
}

static mx_status check_map_geom(int64_t n_expert, int64_t t, int64_t top_k) {
    if (n_expert <= 0 || n_expert > 16384) return fail(MX_ERR_SHAPE, "map0: n_expert (%lld) must be in 1..16384", (long long)n_expert);
    if (t < 0) return fail(MX_ERR_SHAPE, "map0: negative t");
    if (top_k <= 0 || top_k > 64 || top_k > n_expert) return fail(MX_ERR_TOPK, "map0: top_k (%lld) must be in 1..min(64, n_expert)", (long long)top_k);
    if (t * top_k > (int64_t)1 << 22) return fail(MX_ERR_OVERFLOW, "map0: t*top_k exceeds 4M pairs");
    return MX_OK;
}

mx_status mx_prepare_map0(int64_t n_expert, const uint32_t *ids, int64_t t, int64_t top_k, void *scratch,
                          size_t scratch_bytes, mx_stream_t stream) {
    MX_TRY(check_map_geom(n_expert, t, top_k));
    if (!scratch) return fail(MX_ERR_NULL, "map0: scratch is NULL");
    if (!aligned(scratch, 4)) return fail(MX_ERR_ALIGN, "map0: scratch must be 4-byte aligned");
    const size_t need = map0_bytes((int)n_expert, (int)t, (int)top_k);
    if (scratch_bytes < need)
        return fail(MX_ERR_SCRATCH, "map0: scratch of %zu bytes, need %zu", scratch_bytes, need);
    if (t > 0 && !ids) return fail(MX_ERR_NULL, "map0: ids is NULL");
    // m-tiles of GM_BM pairs: the tiles of the prefill GEMM, which the mm_id
    // projections run on (the fallback tiles take each as two halves)
    return launch_map0(ids, (int)t, (int)top_k, (int)n_expert, static_cast<int32_t *>(scratch),
                       (hipStream_t)stream, GM_BM);
}

}  // extern "C"

namespace {
// Stream-ordered temporaries come from one memory pool per device that keeps
// what it has reserved (release threshold: never), so a repeated call of the
// same size reuses its memory instead of mapping it again.
std::mutex g_pool_mu;
hipMemPool_t g_pool[64] = {};

mx_status pool_alloc(size_t bytes, hipStream_t s, void **out) {
    int dev = -1;
    MX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return fail(MX_ERR_SHAPE, "pool: device %d out of range", dev);
    hipMemPool_t pool;
    {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        if (!g_pool[dev]) {
            hipMemPoolProps props{};
            props.allocType = hipMemAllocationTypePinned;
            props.location.type = hipMemLocationTypeDevice;
            props.location.id = dev;
            hipMemPool_t p = nullptr;
            MX_HIP(hipMemPoolCreate(&p, &props));
            uint64_t keep = UINT64_MAX;
            MX_HIP(hipMemPoolSetAttribute(p, hipMemPoolAttrReleaseThreshold, &keep));
            g_pool[dev] = p;
        }
        pool = g_pool[dev];
    }
    MX_HIP(hipMallocFromPoolAsync(out, bytes, pool, s));
    return MX_OK;
}

// bytes of x's f16 rows and their scales for the GEMM route
size_t mm_x16_bytes(int64_t t, int64_t x_per_row, int64_t k) {
    return (((size_t)(t * x_per_row * k) * 2 + 255) & ~size_t(255)) + (size_t)(t * x_per_row) * 4;
}
// the tiles route: the pair order (perm, then its runs: the tiles read 16 words
// from a run's start, which stay inside the runs table), then x's f16 rows
size_t mm_tiles_order_bytes(int64_t pairs) { return (((size_t)pairs + 2 * ((size_t)pairs + 1)) * 4 + 255) & ~size_t(255); }
size_t mm_tiles_bytes(int64_t t, int64_t top_k, int64_t x_per_row, int64_t k) {
    return mm_tiles_order_bytes(t * top_k) + mm_x16_bytes(t, x_per_row, k);
}
// A few pairs per expert: the 16-pair MFMA tiles of the verify blocks (each
// touched expert's weights streamed once) instead of 128-pair GEMM m-tiles
bool mm_on_tiles(const mx_expert_stack *st, const StackGeom &g, int64_t t, int64_t top_k) {
    return (st->dtype == kQ4_K || st->dtype == kQ6_K) && st->k % 512 == 0 && st->n_out % 32 == 0 &&
           t * top_k <= kVmmMaxPairs && st->n_expert <= 1024 && (st->dtype != kQ4_K || g.row_bytes % 16 == 0) &&
           st->n_out * g.row_bytes < ((int64_t)1 << 31) && st->k * 2 < ((int64_t)1 << 31);
}
// pair order, x -> scaled f16 rows (the Q4_K tiles' K order), the plain tiles;
// output row of pair v = token * top_k + slot is dst row v
mx_status mm_tiles(const mx_expert_stack *st, const StackGeom &g, const float *x, int64_t t, int64_t x_per_row,
                   const uint32_t *ids, int64_t top_k, void *tmp, float *dst, hipStream_t s) {
    const int64_t np = t * top_k;
    const int k = (int)st->k;
    int32_t *perm = static_cast<int32_t *>(tmp);
    int32_t *runs = perm + np;
    uint8_t *xb = static_cast<uint8_t *>(tmp) + mm_tiles_order_bytes(np);
    _Float16 *x16 = reinterpret_cast<_Float16 *>(xb);
    float *x16s = reinterpret_cast<float *>(xb + (((size_t)(t * x_per_row * k) * 2 + 255) & ~size_t(255)));
    MX_TRY(launch_pair_order(ids, (int)t, (int)top_k, (int)st->n_expert, (int)top_k, perm, s, runs));
    MX_TRY(launch_to_f16_rows(x, t * x_per_row, k, nullptr, x16, x16s, s, st->dtype == kQ4_K));
    VmmArgs a{};
    a.w[0] = g.w;
    a.expert_bytes = g.expert_bytes; a.row_bytes = g.row_bytes; a.sh_row_bytes = g.row_bytes;
    a.n_expert = (int)st->n_expert; a.n_out = (int)st->n_out; a.k = k;
    a.a = x16; a.a_scale = x16s;
    a.a_slots = x_per_row == 1 ? (int)top_k : 1;  // A row of pair v: v / a_slots
    a.perm = perm; a.runs = runs;
    a.out = dst;
    return launch_vmm(st->dtype, false, a, (int)np, s);
}
// the grouped GEMM of the prefill path takes a projection whose K is whole
// super-blocks and whose operand spans fit its 32-bit offsets; the rest run the
// fallback tiles
bool mm_on_gemm(const mx_expert_stack *st, const StackGeom &g, int64_t t, int64_t x_per_row) {
    // A rows: x's token rows (x_per_row == 1) or a bucket-ordered tile (mm_gemm)
    return gemm_supported(st->dtype, (int)st->k) &&
           gemm_plain_fits(x_per_row == 1 ? t : GM_BM, (int)st->k, (int)st->n_out, g.row_bytes);
}
mx_status mm_fallback(const mx_expert_stack *st, const StackGeom &g, const float *x, int64_t t, int64_t x_per_row,
                      int64_t top_k, const int32_t *map, float *dst, hipStream_t s) {
    MmArgs a{g.w, g.expert_bytes, g.row_bytes, (int)st->n_expert, (int)st->n_out, (int)st->k,
             x, (int)x_per_row, (int)t, (int)top_k, map, dst};
    return launch_mul_mm_id(st->dtype, a, s);
}
// x -> scaled f16 rows in tmp (mm_x16_bytes, 256-aligned), then the plain GEMM
// with one output row per pair (row token * top_k + slot of dst)
mx_status mm_gemm(const mx_expert_stack *st, const StackGeom &g, const float *x, int64_t t, int64_t x_per_row,
                  int64_t top_k, const int32_t *map, void *tmp, float *dst, hipStream_t s) {
    const int k = (int)st->k;
    _Float16 *x16 = static_cast<_Float16 *>(tmp);
    float *x16s = reinterpret_cast<float *>(static_cast<uint8_t *>(tmp) +
                                            (((size_t)(t * x_per_row * k) * 2 + 255) & ~size_t(255)));
    // one x row per pair (x_per_row == top_k): gathered into bucket order, so a
    // tile's A rows are consecutive (rows past the map's pair count are skipped);
    // one per token: the token's row, shared by its slots
    const MapLayout L((int)st->n_expert, (int)t, (int)top_k);
    const bool by_pair = x_per_row != 1;
    if (by_pair)
        MX_TRY(launch_to_f16_rows(x, t * top_k, k, map + L.off + st->n_expert, x16, x16s, s, false, map + L.list));
    else
        MX_TRY(launch_to_f16_rows(x, t, k, nullptr, x16, x16s, s));
    GemmArgs a{};
    a.w[0] = g.w;
    a.expert_bytes = g.expert_bytes; a.row_bytes = g.row_bytes; a.sh_row_bytes = g.row_bytes;
    a.n_expert = (int)st->n_expert; a.n_out = (int)st->n_out; a.k = k;
    a.a = x16; a.a_scale = x16s;
    a.a_div = by_pair ? 0 : (int)top_k;  // bucket position / token of the pair
    a.t = (int)t; a.top_k = (int)top_k; a.n_map_expert = (int)st->n_expert; a.map = map;
    a.out = dst; a.out_stride = (int)top_k; a.out_add = 0;
    return launch_gemm(st->dtype, false, a, s);
}
}  // namespace

extern "C" {

mx_status mx_mul_mm_id_shared(const mx_expert_stack *stack, const float *x, int64_t t, int64_t x_per_row,
                              int64_t k, const uint32_t *ids, int64_t ids_t, int64_t top_k,
                              const mx_map0 *map, float *dst, mx_stream_t stream) {
    StackGeom g;
    MX_TRY(check_id_call(stack, x, t, x_per_row, k, ids, ids_t, top_k, dst, g));
    if (!map || !map->buffer) return fail(MX_ERR_NULL, "mul_mm_id_shared: map0 scratch is NULL");
    // dispatch.rs:886-896: the producer's geometry must match this projection
    if (map->n_expert != stack->n_expert || map->t != t || map->top_k != top_k)
        return fail(MX_ERR_SCRATCH,
                    "shared map0 scratch geometry (n_expert=%lld, t=%lld, top_k=%lld) does not match this "
                    "projection (n_expert=%lld, t=%lld, top_k=%lld)",
                    (long long)map->n_expert, (long long)map->t, (long long)map->top_k,
                    (long long)stack->n_expert, (long long)t, (long long)top_k);
    if (map->bytes < map0_bytes((int)map->n_expert, (int)t, (int)top_k))
        return fail(MX_ERR_SCRATCH, "shared map0 scratch too small");
    if (t == 0) return MX_OK;
    const hipStream_t s = (hipStream_t)stream;
    const int32_t *mp = static_cast<const int32_t *>(map->buffer);
    const bool tiles = mm_on_tiles(stack, g, t, top_k);
    if (!tiles && !mm_on_gemm(stack, g, t, x_per_row)) return mm_fallback(stack, g, x, t, x_per_row, top_k, mp, dst, s);
    // no workspace in this interface (mm_id.rs:32-39): x's f16 rows (and the tiles'
    // pair order) live in stream-ordered memory of the library's pool for the call
    void *tmp = nullptr;
    MX_TRY(pool_alloc(tiles ? mm_tiles_bytes(t, top_k, x_per_row, stack->k) : mm_x16_bytes(t, x_per_row, stack->k),
                      s, &tmp));
    const mx_status rc = tiles ? mm_tiles(stack, g, x, t, x_per_row, ids, top_k, tmp, dst, s)
                               : mm_gemm(stack, g, x, t, x_per_row, top_k, mp, tmp, dst, s);
    MX_HIP(hipFreeAsync(tmp, s));
    return rc;
}

size_t mx_mul_mm_id_workspace_bytes(int64_t n_expert, int64_t t, int64_t top_k, int64_t x_per_row, int64_t k) {
    // map0, then x's f16 rows and their scales (GEMM route) or the pair order and
    // the f16 rows (tiles route)
    const size_t map = (mx_map0_scratch_bytes(n_expert, t, top_k) + 255) & ~size_t(255);
    size_t extra = 0;
    if (k > 0 && k % 256 == 0) extra = mm_x16_bytes(t, x_per_row, k);
    if (k > 0 && k % 512 == 0 && t * top_k <= kVmmMaxPairs) extra = std::max(extra, mm_tiles_bytes(t, top_k, x_per_row, k));
    return map + extra;
}

mx_status mx_mul_mm_id(const mx_expert_stack *stack, const float *x, int64_t t, int64_t x_per_row, int64_t k,
                       const uint32_t *ids, int64_t ids_t, int64_t top_k, void *workspace,
                       size_t workspace_bytes, float *dst, mx_stream_t stream) {
    StackGeom g;
    MX_TRY(check_id_call(stack, x, t, x_per_row, k, ids, ids_t, top_k, dst, g));
    MX_TRY(check_map_geom(stack->n_expert, t, top_k));
    if (t == 0) return MX_OK;
    const size_t need = mx_mul_mm_id_workspace_bytes(stack->n_expert, t, top_k, x_per_row, k);
    if (!workspace) return fail(MX_ERR_NULL, "mul_mm_id: workspace is NULL");
    if (workspace_bytes < need)
        return fail(MX_ERR_SCRATCH, "mul_mm_id: workspace of %zu bytes, need %zu", workspace_bytes, need);
    const size_t map_bytes = (mx_map0_scratch_bytes(stack->n_expert, t, top_k) + 255) & ~size_t(255);
    const hipStream_t s = (hipStream_t)stream;
    const bool tiles = mm_on_tiles(stack, g, t, top_k);
    if ((tiles || mm_on_gemm(stack, g, t, x_per_row)) && !aligned(workspace, 256))
        return fail(MX_ERR_ALIGN, "mul_mm_id: workspace must be 256-byte aligned");
    uint8_t *tmp = static_cast<uint8_t *>(workspace) + map_bytes;
    if (tiles) return mm_tiles(stack, g, x, t, x_per_row, ids, top_k, tmp, dst, s);  // (no bucket map)
    MX_TRY(mx_prepare_map0(stack->n_expert, ids, t, top_k, workspace, map_bytes, stream));
    const int32_t *mp = static_cast<const int32_t *>(workspace);
    if (!mm_on_gemm(stack, g, t, x_per_row)) return mm_fallback(stack, g, x, t, x_per_row, top_k, mp, dst, s);
    return mm_gemm(stack, g, x, t, x_per_row, top_k, mp, tmp, dst, s);
}

mx_status mx_check_ids(const uint32_t *ids, int64_t t, int64_t top_k, int64_t n_expert, uint32_t *flags,
                       mx_stream_t stream) {
    if (t < 0 || top_k <= 0 || top_k > 64 || n_expert <= 0 || n_expert > INT32_MAX)
        return fail(MX_ERR_SHAPE, "check_ids: bad shape t=%lld top_k=%lld n_expert=%lld", (long long)t,
                    (long long)top_k, (long long)n_expert);
    if (t * top_k > (int64_t)1 << 22) return fail(MX_ERR_OVERFLOW, "check_ids: t*top_k exceeds 4M pairs");
    if (!flags) return fail(MX_ERR_NULL, "check_ids: flags is NULL");
    if (t > 0 && !ids) return fail(MX_ERR_NULL, "check_ids: ids is NULL");
    return launch_check_ids(ids, t, (int)top_k, (int)n_expert, flags, (hipStream_t)stream);
}

mx_status mx_silu_mul(const float *gate, const float *up, int64_t n, float *dst, mx_stream_t stream) {
    if (n < 0) return fail(MX_ERR_SHAPE, "silu_mul: negative n");
    if (n == 0) return MX_OK;
    if (!gate || !up || !dst) return fail(MX_ERR_NULL, "silu_mul: NULL operand");
    return launch_silu_mul(gate, up, n, dst, (hipStream_t)stream);
}

mx_status mx_combine(const float *down, const float *col_l2, const float *w, int64_t seq, int64_t top_k,
                     int64_t n_out, float *dst, mx_stream_t stream) {
    if (seq < 0 || top_k <= 0 || n_out <= 0)
        return fail(MX_ERR_SHAPE, "combine: bad shape seq=%lld top_k=%lld n_out=%lld", (long long)seq,
                    (long long)top_k, (long long)n_out);
    // combine.rs / dispatch.rs:1453-1462: index math must fit i32
    if (seq * top_k * n_out > INT32_MAX)
        return fail(MX_ERR_OVERFLOW, "combine index math overflows i32: seq*top_k*n_out = %lld",
                    (long long)(seq * top_k * n_out));
    if (seq == 0) return MX_OK;
    if (!down || !w || !dst) return fail(MX_ERR_NULL, "combine: NULL operand");
    return launch_combine(down, col_l2, w, (int)seq, (int)top_k, (int)n_out, dst, (hipStream_t)stream);
}

mx_status mx_rms_norm(const float *x, const float *alpha, int64_t rows, int64_t dim, float eps, float *dst,
                      mx_stream_t stream) {
    if (rows < 0 || dim <= 0 || rows > INT32_MAX) return fail(MX_ERR_SHAPE, "rms_norm: bad shape");
    if (rows == 0) return MX_OK;
    if (!x || !alpha || !dst) return fail(MX_ERR_NULL, "rms_norm: NULL operand");
    return launch_rms_norm(x, alpha, (int)rows, (int)dim, eps, dst, (hipStream_t)stream);
}

mx_status mx_route_logits(const float *x, const float *router, int64_t t, int64_t hidden, int64_t n_expert,
                          float *logits, mx_stream_t stream) {
    if (t < 0 || hidden <= 0 || n_expert <= 0 || t > INT32_MAX / 2)
        return fail(MX_ERR_SHAPE, "route_logits: bad shape");
    if (t == 0) return MX_OK;
    if (!x || !router || !logits) return fail(MX_ERR_NULL, "route_logits: NULL operand");
    return launch_route_logits(x, router, (int)t, (int)hidden, (int)n_expert, logits, (hipStream_t)stream);
}

static mx_status check_route(int64_t t, int64_t n_expert, int64_t top_k) {
    if (t < 0) return fail(MX_ERR_SHAPE, "route: negative t");
    if (n_expert <= 0 || n_expert > 1024) return fail(MX_ERR_SHAPE, "route: n_expert (%lld) must be in 1..1024", (long long)n_expert);
    if (top_k <= 0 || top_k > 32 || top_k > n_expert)
        return fail(MX_ERR_TOPK, "route: top_k (%lld) must be in 1..min(32, n_expert)", (long long)top_k);
    return MX_OK;
}

mx_status mx_route_from_logits(const float *logits, const float *bias, int64_t t, int64_t n_expert, int64_t top_k,
                               double scale, int32_t norm, uint32_t *ids, float *w, mx_stream_t stream) {
    MX_TRY(check_route(t, n_expert, top_k));
    if (t == 0) return MX_OK;
    if (!logits || !bias || !ids || !w) return fail(MX_ERR_NULL, "route_from_logits: NULL operand");
    const int apply = (scale != 0.0 && scale != 1.0) ? 1 : 0;
    return launch_route_select(logits, bias, (int)t, (int)n_expert, (int)top_k, (float)scale, apply, norm ? 1 : 0,
                               ids, w, (hipStream_t)stream);
}

}  // extern "C"

// ---- whole MoE block --------------------------------------------------------------------
namespace {

constexpr int64_t kDefaultMmMinSeq = 32;  // ops/mod.rs:31 MM_ID_MIN_SEQ
#ifndef MX_FUSE_SELECT
#define MX_FUSE_SELECT 1
#endif
constexpr bool kFuseSelect = MX_FUSE_SELECT != 0;
// Below the grouped-GEMM threshold, blocks of at least this many tokens run their
// experts as 16-pair MFMA tiles (mx_vmm.hip) instead of per-pair mat-vecs
#ifndef MX_VMM_MIN_T
#define MX_VMM_MIN_T 16
#endif
constexpr int64_t kVmmMinT = MX_VMM_MIN_T;

struct Ws {
    uint8_t *base;
    size_t off = 0;
    explicit Ws(void *b) : base(static_cast<uint8_t *>(b)) {}
    template <class T> T *take(size_t count) {
        off = (off + 255) & ~size_t(255);
        T *p = base ? reinterpret_cast<T *>(base + off) : nullptr;
        off += count * sizeof(T);
        return p;
    }
};

struct Plan {
    bool mm, fused_router, has_shared;
    bool generic;           // below the GEMM threshold, shapes the fused decode kernels cannot hold:
                            // router + f32 gather mat-vecs + SwiGLU + combine
    bool shared_in_decode;  // shared expert rides in the fused decode kernels (same quant types)
    bool vmm;               // verify block on the 16-pair MFMA tiles (after the fused router)
    int64_t min_seq;
};

int64_t stack_row_bytes(const mx_expert_stack &st) {
    return supported(st.dtype) ? st.k / block_size(st.dtype) * type_size(st.dtype) : 0;
}

// Chooses the kernels of a forward; every shape limit of the chosen kernels is
// checked here, so a validated call never fails after its first launch.
Plan plan_for(const mx_moe_layer *L, int64_t t) {
    Plan p;
    p.min_seq = L->mm_min_seq > 0 ? L->mm_min_seq : kDefaultMmMinSeq;
    // < 0: never (LAGUNA_NO_MM_ID).  The MFMA GEMM needs K % 256 == 0 for every
    // stack; other shapes stay on the gather mat-vec kernels at any t.
    bool shapes = gemm_supported(L->gate.dtype, (int)L->hidden) && gemm_supported(L->down.dtype, (int)L->expert_ff);
    if (L->shared_gate.data)
        shapes = shapes && gemm_supported(L->shared_gate.dtype, (int)L->hidden) &&
                 gemm_supported(L->shared_down.dtype, (int)L->expert_ff);
    shapes = shapes && gemm_fits((int)t, (int)L->hidden, (int)L->expert_ff, stack_row_bytes(L->gate),
                                 stack_row_bytes(L->down));
    if (L->shared_gate.data)
        shapes = shapes && gemm_fits((int)t, (int)L->hidden, (int)L->expert_ff, stack_row_bytes(L->shared_gate),
                                     stack_row_bytes(L->shared_down));
    p.has_shared = L->shared_gate.data != nullptr;
    p.shared_in_decode = p.has_shared && L->shared_gate.dtype == L->gate.dtype &&
                         L->shared_down.dtype == L->down.dtype;
    const bool decode_fits = decode_gate_up_fits(L->gate.dtype, (int)L->hidden, stack_row_bytes(L->gate)) &&
                             decode_down_fits(L->down.dtype, (int)L->expert_ff, stack_row_bytes(L->down));
    const int64_t slots = L->top_k + (p.shared_in_decode ? 1 : 0);
    const int64_t gu_rb = stack_row_bytes(L->gate), d_rb = stack_row_bytes(L->down);
    // 16-pair MFMA tiles: from kVmmMinT tokens up to kVmmMaxPairs pairs, also past
    // mm_min_seq (the grouped GEMM's tiles are mostly empty there: measured
    // 25-35% slower per C1-shaped layer from 32 to 93 tokens, 8% at 200);
    // LAGUNA_NO_MM_ID (mm_min_seq < 0) keeps every t on the mat-vec kernels
    const bool vmm_ok =
        L->mm_min_seq >= 0 && decode_fits && t >= kVmmMinT && (!p.has_shared || p.shared_in_decode) &&
        t * slots <= kVmmMaxPairs && L->gate.n_expert <= 1024 &&
        vmm_supported(L->gate.dtype, L->down.dtype, (int)L->hidden, (int)L->expert_ff, gu_rb, d_rb) &&
        L->expert_ff * gu_rb < ((int64_t)1 << 31) && L->hidden * d_rb < ((int64_t)1 << 31) &&
        (!p.has_shared || (stack_row_bytes(L->shared_gate) == gu_rb && stack_row_bytes(L->shared_down) == d_rb));
    p.mm = L->mm_min_seq >= 0 && t >= p.min_seq && shapes && !vmm_ok;
    p.generic = !p.mm && !decode_fits;
    p.fused_router = !p.mm && !p.generic && t <= route_fused_max_t();
    p.vmm = vmm_ok;
    return p;
}

// Verify blocks on the decode kernels launch their gate/up pairs in expert order.
bool pair_order_used(int64_t t, int64_t slots, int64_t n_expert) {
    return t > 1 && t * slots <= PAIR_ORDER_DECODE_MAX && n_expert <= 1024;  // the top-k kernels' limit
}

// Carves the workspace; with base == nullptr it only measures.
struct Layout {
    uint8_t *route_ws = nullptr;
    float *x_normed = nullptr, *logits = nullptr, *w = nullptr, *act = nullptr;
    uint32_t *ids = nullptr, *zero_ids = nullptr;
    int32_t *perm = nullptr;  // expert-ordered (token, slot) pairs of a verify block
    int32_t *runs = nullptr;  // their 16-pair runs (MFMA verify tiles)
    uint8_t *xstage = nullptr, *xstage_gm = nullptr;
    float *part = nullptr;
    int32_t *map = nullptr, *map_sh = nullptr;
    _Float16 *x16 = nullptr, *act16 = nullptr;
    float *x16s = nullptr, *act16s = nullptr, *down = nullptr, *act_u = nullptr;
    float *sh_g = nullptr, *sh_u = nullptr, *sh_out = nullptr;
    size_t bytes = 0;
};

Layout carve(const mx_moe_layer *L, int64_t t, const Plan &p, void *base) {
    Ws ws(base);
    Layout o;
    const int64_t H = L->hidden, FF = L->expert_ff, K = L->top_k, E = L->gate.n_expert;
    if (L->rms_alpha) o.x_normed = ws.take<float>(t * H);
    o.ids = ws.take<uint32_t>(t * K);
    o.w = ws.take<float>(t * K);
    if (p.fused_router) {
        o.route_ws = ws.take<uint8_t>(route_fused_ws_bytes((int)t, (int)H, (int)E));
    } else {
        o.logits = ws.take<float>(t * E * route_logits_splits((int)t, (int)L->hidden, (int)E));
    }
    if (p.generic) {
        const int64_t KK = K + (p.has_shared ? 1 : 0);
        o.act = ws.take<float>(t * K * FF);
        o.act_u = ws.take<float>(t * K * FF);
        if (p.has_shared) {
            o.sh_g = ws.take<float>(t * FF);
            o.sh_u = ws.take<float>(t * FF);
        }
        o.down = ws.take<float>(t * KK * H);
    } else if (p.vmm) {
        const int64_t slots = K + (p.has_shared ? 1 : 0);
        o.perm = ws.take<int32_t>(t * slots);
        o.runs = ws.take<int32_t>(2 * (t * slots + 1));
        o.x16 = ws.take<_Float16>(t * H);
        o.x16s = ws.take<float>(t);
        o.act = ws.take<float>(t * slots * FF);
        o.act16 = ws.take<_Float16>(t * slots * FF);
        o.act16s = ws.take<float>(t * slots);
        o.down = ws.take<float>(t * slots * H);
    } else if (!p.mm) {
        const int64_t slots = K + (p.shared_in_decode ? 1 : 0);
        o.xstage = ws.take<uint8_t>(t * stage_row_bytes((int)H));
        if (H % 64 == 0) o.xstage_gm = ws.take<uint8_t>(t * xstage_gm_stride((int)H));
        o.act = ws.take<float>(t * slots * FF);
        o.part = ws.take<float>(t * slots * H);
        if (pair_order_used(t, slots, E)) o.perm = ws.take<int32_t>(t * slots);
        if (p.has_shared && !p.shared_in_decode) {
            o.sh_g = ws.take<float>(t * FF);
            o.sh_u = ws.take<float>(t * FF);
            o.sh_out = ws.take<float>(t * H);
        }
    } else {
        // one bucket map over routed + shared (expert E, every token) when the shared
        // expert has the routed quant types, else a second one-expert map
        const int64_t S = p.has_shared ? 1 : 0;
        const int64_t KK = K + S;
        const int64_t EM = E + (p.shared_in_decode ? 1 : 0);
        const int64_t KM = K + (p.shared_in_decode ? 1 : 0);
        o.map = ws.take<int32_t>(map0_bytes((int)EM, (int)t, (int)KM) / 4);
        if (p.has_shared && !p.shared_in_decode) {
            o.map_sh = ws.take<int32_t>(map0_bytes(1, (int)t, 1) / 4);
            o.zero_ids = ws.take<uint32_t>(t);
        }
        o.x16 = ws.take<_Float16>(t * H);
        o.x16s = ws.take<float>(t);
        o.act = ws.take<float>(t * KK * FF);
        o.act16 = ws.take<_Float16>(t * KK * FF);
        o.act16s = ws.take<float>(t * KK);
        o.down = ws.take<float>(t * KK * H);
    }
    o.bytes = ws.off + 256;
    return o;
}

__global__ void k_fill_u32(uint32_t *p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

mx_status check_layer(const mx_moe_layer *L, int64_t t, StackGeom &gg, StackGeom &gu, StackGeom &gd,
                      StackGeom &sg, StackGeom &su, StackGeom &sd) {
    if (!L) return fail(MX_ERR_NULL, "moe: layer is NULL");
    if (t < 0) return fail(MX_ERR_SHAPE, "moe: negative t");
    MX_TRY(check_stack(&L->gate, "ffn_gate_exps", gg));
    MX_TRY(check_stack(&L->up, "ffn_up_exps", gu));
    MX_TRY(check_stack(&L->down, "ffn_down_exps", gd));
    const int64_t H = L->hidden, FF = L->expert_ff, E = L->gate.n_expert;
    // moe.rs:206-216: the three stacks must agree on n_expert
    if (L->up.n_expert != E || L->down.n_expert != E)
        return fail(MX_ERR_SHAPE, "MoE expert stacks disagree on n_expert: gate=%lld, up=%lld, down=%lld",
                    (long long)E, (long long)L->up.n_expert, (long long)L->down.n_expert);
    if (L->gate.n_out != FF || L->up.n_out != FF || L->gate.k != H || L->up.k != H || L->down.n_out != H ||
        L->down.k != FF)
        return fail(MX_ERR_SHAPE, "moe: expert stacks do not match hidden=%lld expert_ff=%lld", (long long)H,
                    (long long)FF);
    if (L->gate.dtype != L->up.dtype)
        return fail(MX_ERR_DTYPE, "moe: gate (%s) and up (%s) experts must share a quant type",
                    dt_name(L->gate.dtype), dt_name(L->up.dtype));
    MX_TRY(check_route(t, E, L->top_k));
    if (!L->router || !L->exp_probs_b) return fail(MX_ERR_NULL, "moe: router or exp_probs_b is NULL");
    if (L->shared_gate.data) {
        MX_TRY(check_stack(&L->shared_gate, "ffn_gate_shexp", sg));
        MX_TRY(check_stack(&L->shared_up, "ffn_up_shexp", su));
        MX_TRY(check_stack(&L->shared_down, "ffn_down_shexp", sd));
        if (L->shared_gate.n_expert != 1 || L->shared_up.n_expert != 1 || L->shared_down.n_expert != 1)
            return fail(MX_ERR_SHAPE, "moe: shared expert stacks must have n_expert == 1");
        if (L->shared_gate.n_out != FF || L->shared_up.n_out != FF || L->shared_gate.k != H ||
            L->shared_up.k != H || L->shared_down.n_out != H || L->shared_down.k != FF)
            return fail(MX_ERR_SHAPE, "moe: shared expert must be [%lld x %lld] / [%lld x %lld]", (long long)FF,
                        (long long)H, (long long)H, (long long)FF);
        if (L->shared_gate.dtype != L->shared_up.dtype)
            return fail(MX_ERR_DTYPE, "moe: shared gate and up must share a quant type");
    }
    if (H % 4 || FF % 4) return fail(MX_ERR_SHAPE, "moe: hidden and expert_ff must be multiples of 4");
    if (t * L->top_k > (int64_t)1 << 22) return fail(MX_ERR_OVERFLOW, "moe: t*top_k exceeds 4M pairs");
    return MX_OK;
}

}  // namespace

extern "C" {

size_t mx_moe_workspace_bytes(const mx_moe_layer *layer, int64_t t) {
    if (!layer || t < 0) return 0;
    const Plan p = plan_for(layer, t);
    return carve(layer, t, p, nullptr).bytes;
}

}  // extern "C"

namespace {
// Records a HIP event after each stage of a forward (profiling variant only).
struct StageTimer {
    hipEvent_t ev[17];
    int n = 0;
    mx_status mark(hipStream_t s) {
        if (n >= 17) return fail(MX_ERR_SHAPE, "too many stages");
        MX_HIP(hipEventCreate(&ev[n]));
        MX_HIP(hipEventRecord(ev[n], s));
        n++;
        return MX_OK;
    }
    ~StageTimer() {
        for (int i = 0; i < n; i++) (void)hipEventDestroy(ev[i]);
    }
};
#define MX_STAGE() \
    do {           \
        if (tm) MX_TRY(tm->mark(s)); \
    } while (0)

// Launch count of decode stage `stage` (profiling: one stage skipped or
// repeated, see mx_moe_forward_repeat; 1 otherwise).
struct Repeat {
    int stage = -1, times = 1;
    int operator()(int st) const { return st == stage ? times : 1; }
};

mx_status moe_forward_impl(const mx_moe_layer *L, const float *x, int64_t t, const float *residual, float *out,
                           uint32_t *ids_out, float *w_out, void *workspace, size_t workspace_bytes,
                           hipStream_t s, StageTimer *tm, Repeat rep = Repeat()) {
    StackGeom gg, gu, gd, sg{}, su{}, sd{};
    MX_TRY(check_layer(L, t, gg, gu, gd, sg, su, sd));
    if (t == 0) return MX_OK;
    MX_TRY(check_f32(x, "x"));
    MX_TRY(check_f32(out, "out"));
    if (residual) MX_TRY(check_f32(residual, "residual"));
    if (!workspace) return fail(MX_ERR_NULL, "moe: workspace is NULL");
    const Plan p = plan_for(L, t);
    const Layout o = carve(L, t, p, workspace);
    if (workspace_bytes < o.bytes)
        return fail(MX_ERR_SCRATCH, "moe: workspace of %zu bytes, need %zu", workspace_bytes, o.bytes);
    MX_STAGE();
    const int64_t H = L->hidden, FF = L->expert_ff, K = L->top_k, E = L->gate.n_expert;
    const float scale = (float)L->weights_scale;
    const int apply = (L->weights_scale != 0.0 && L->weights_scale != 1.0) ? 1 : 0;
    uint32_t *ids = ids_out ? ids_out : o.ids;
    float *w = w_out ? w_out : o.w;
    const float *xin = x;

    // routing (+ the RMSNorm of the FFN half when requested)
    // (verify tiles without RMSNorm: the router also writes the f16 x rows)
    const bool x16_in_router = p.vmm && p.fused_router && !L->rms_alpha;
    if (p.fused_router) {
        // logits -> keys/probs; the router also stages the (normalised) rows for the
        // decode expert kernels.  The top-k is its own launch (k_decode_select, below).
        for (int r = 0; r < rep(0); r++)
            MX_TRY(launch_route_fused(x, L->rms_alpha, L->rms_eps, o.x_normed, L->router, L->exp_probs_b, (int)t,
                                      (int)H, (int)E, o.route_ws, o.xstage, o.xstage_gm, s,
                                      x16_in_router ? o.x16 : nullptr, x16_in_router ? o.x16s : nullptr));
        if (L->rms_alpha) xin = o.x_normed;
    } else {
        if (L->rms_alpha) {
            MX_TRY(launch_rms_norm(x, L->rms_alpha, (int)t, (int)H, L->rms_eps, o.x_normed, s));
            xin = o.x_normed;
        }
        const int splits = route_logits_splits((int)t, (int)H, (int)E);
        MX_TRY(launch_route_logits_split(xin, L->router, (int)t, (int)H, (int)E, o.logits, splits, s));
        MX_TRY(launch_route_select(o.logits, L->exp_probs_b, (int)t, (int)E, (int)K, scale, apply,
                                   L->weights_norm, ids, w, s, splits));
        if (!p.mm && !p.generic && !p.vmm) MX_TRY(launch_stage_rows(xin, (int)t, (int)H, o.xstage, o.xstage_gm, s));

    }
    MX_STAGE();

    if (p.generic) {
        // f32 gather mat-vecs (any row width), then the prefill combine
        const int S = p.has_shared ? 1 : 0, KK = (int)K + S;
        MvfArgs m{gg.w, gg.expert_bytes, gg.row_bytes, (int)E, (int)FF, (int)H, xin, 1, ids, (int)t, (int)K,
                  o.act, (int)K, 0};
        MX_TRY(launch_mv_f32(L->gate.dtype, m, s));
        m.w = gu.w;
        m.dst = o.act_u;
        MX_TRY(launch_mv_f32(L->up.dtype, m, s));
        MX_TRY(launch_silu_mul(o.act, o.act_u, t * K * FF, o.act, s));
        MvfArgs d{gd.w, gd.expert_bytes, gd.row_bytes, (int)E, (int)H, (int)FF, o.act, (int)K, ids, (int)t,
                  (int)K, o.down, KK, 0};
        MX_TRY(launch_mv_f32(L->down.dtype, d, s));
        if (S) {
            MvfArgs sgm{sg.w, sg.expert_bytes, sg.row_bytes, 1, (int)FF, (int)H, xin, 1, nullptr, (int)t, 1,
                        o.sh_g, 1, 0};
            MX_TRY(launch_mv_f32(L->shared_gate.dtype, sgm, s));
            sgm.w = su.w;
            sgm.dst = o.sh_u;
            MX_TRY(launch_mv_f32(L->shared_up.dtype, sgm, s));
            MX_TRY(launch_silu_mul(o.sh_g, o.sh_u, t * FF, o.sh_g, s));
            MvfArgs sdm{sd.w, sd.expert_bytes, sd.row_bytes, 1, (int)H, (int)FF, o.sh_g, 1, nullptr, (int)t, 1,
                        o.down, KK, (int)K};
            MX_TRY(launch_mv_f32(L->shared_down.dtype, sdm, s));
        }
        MX_TRY(launch_combine_prefill(o.down, w, residual, (int)t, (int)K, S, (int)H, out, s));
        MX_STAGE();
        return MX_OK;
    }

    if (!p.mm) {
        const bool shf = p.shared_in_decode;
        const float *shared_out = nullptr;
        if (p.has_shared && !shf) {
            // shared expert of another quant type: its own gather mat-vecs (expert 0)
            MvArgs mg{sg.w, sg.expert_bytes, sg.row_bytes, 1, (int)FF, (int)H, xin, 1, nullptr, (int)t, 1, o.sh_g};
            MX_TRY(launch_mul_mv_id(L->shared_gate.dtype, mg, s));
            mg.w = su.w;
            mg.dst = o.sh_u;
            MX_TRY(launch_mul_mv_id(L->shared_up.dtype, mg, s));
            MX_TRY(launch_silu_mul(o.sh_g, o.sh_u, t * FF, o.sh_g, s));
            MvArgs md{sd.w, sd.expert_bytes, sd.row_bytes, 1, (int)H, (int)FF, o.sh_g, 1, nullptr, (int)t, 1, o.sh_out};
            MX_TRY(launch_mul_mv_id(L->shared_down.dtype, md, s));
            shared_out = o.sh_out;
        }
        DecodeGateUpArgs ga{gg.w, gu.w, gg.expert_bytes, gg.row_bytes, shf ? sg.w : nullptr, shf ? su.w : nullptr,
                            sg.row_bytes, (int)E, (int)FF, (int)H, o.xstage, ids, (int)t, (int)K, o.act,
                            o.xstage_gm, o.perm};
        DecodeDownArgs da{gd.w, gd.expert_bytes, gd.row_bytes, shf ? sd.w : nullptr, sd.row_bytes, shared_out,
                          (int)E, (int)FF, (int)H, o.act, ids, w, residual, (int)t, (int)K, out, o.part,
                          o.perm};
        if (p.fused_router) {
            const uint8_t *keys = static_cast<const uint8_t *>(o.route_ws);
            DecodeSelArgs sel{reinterpret_cast<const uint64_t *>(keys),
                              reinterpret_cast<const float *>(keys + (size_t)t * E * sizeof(uint64_t)), (int)E,
                              (int)t, scale, apply, L->weights_norm, ids, w};
            // one token: the gate/up blocks run the top-k themselves where they can
            // (no launch boundary between router and experts); else its own launch
            ga.sel_keys = sel.keys;
            ga.sel_probs = sel.probs;
            ga.sel_scale = scale;
            ga.sel_apply = apply;
            ga.sel_norm = L->weights_norm;
            ga.sel_ids = ids;
            ga.sel_w = w;
            if (!(kFuseSelect && decode_gate_up_selects(L->gate.dtype, ga))) {
                ga.sel_keys = nullptr;
                for (int r = 0; r < rep(1); r++) MX_TRY(launch_decode_select((int)K, sel, s));
            }
        }
        if (p.vmm) {
            // 16-pair MFMA tiles: x -> scaled f16, gate/up + SwiGLU, act -> scaled f16,
            // down into rows token * slots + slot, then the prefill combine
            const int slots = (int)K + (shf ? 1 : 0), np = (int)t * slots;
            MX_TRY(launch_pair_order(ids, (int)t, (int)K, (int)E, slots, o.perm, s, o.runs));
            MX_STAGE();
            VmmArgs g{};
            g.w[0] = gg.w;
            g.w[1] = gu.w;
            g.w_sh[0] = shf ? sg.w : nullptr;
            g.w_sh[1] = shf ? su.w : nullptr;
            g.expert_bytes = gg.expert_bytes;
            g.row_bytes = gg.row_bytes;
            g.sh_row_bytes = sg.row_bytes;
            g.n_expert = (int)E;
            g.n_out = (int)FF;
            g.k = (int)H;
            g.a = o.x16;
            g.a_scale = o.x16s;
            g.a_slots = slots;
            g.perm = o.perm;
            g.runs = o.runs;
            g.out = o.act;
            for (int r = 0; r < rep(2); r++) {
                if (!x16_in_router) MX_TRY(launch_to_f16_rows(xin, t, (int)H, nullptr, o.x16, o.x16s, s, true));
                MX_TRY(launch_vmm(L->gate.dtype, true, g, np, s));
            }
            MX_STAGE();
            VmmArgs d = g;
            d.w[0] = gd.w;
            d.w[1] = nullptr;
            d.w_sh[0] = shf ? sd.w : nullptr;
            d.w_sh[1] = nullptr;
            d.expert_bytes = gd.expert_bytes;
            d.row_bytes = gd.row_bytes;
            d.sh_row_bytes = sd.row_bytes;
            d.n_out = (int)H;
            d.k = (int)FF;
            d.a = o.act16;
            d.a_scale = o.act16s;
            d.a_slots = 1;
            d.out = o.down;
            for (int r = 0; r < rep(3); r++) {
                MX_TRY(launch_to_f16_rows(o.act, np, (int)FF, nullptr, o.act16, o.act16s, s,
                                          L->down.dtype == kQ4_K));  // (the Q4_K tiles' K order)
                MX_TRY(launch_vmm(L->down.dtype, false, d, np, s));
                MX_TRY(launch_combine_prefill(o.down, w, residual, (int)t, (int)K, shf ? 1 : 0, (int)H, out, s));
            }
            MX_STAGE();
            return MX_OK;
        }
        if (o.perm) MX_TRY(launch_pair_order(ids, (int)t, (int)K, (int)E, (int)K + (shf ? 1 : 0), o.perm, s));
        MX_STAGE();
        for (int r = 0; r < (p.fused_router ? rep(2) : 1); r++)
            MX_TRY(launch_decode_gate_up(L->gate.dtype, ga, 0, (int)K + (shf ? 1 : 0), s));
        MX_STAGE();
        for (int r = 0; r < (p.fused_router ? rep(3) : 1); r++) MX_TRY(launch_decode_down(L->down.dtype, da, s));
        MX_STAGE();
        return MX_OK;
    }

    // prefill / verify (moe.rs:242-323): bucket once, x -> scaled f16, gate+up GEMM
    // with SwiGLU, act -> scaled f16, down GEMM into rows token * KK + slot (slot K:
    // shared expert), combine with the shared expert and the residual
    const int S = p.has_shared ? 1 : 0;
    const int KK = (int)K + S;
    const bool one_map = p.shared_in_decode;  // shared joins the routed map as expert E
    const int EM = (int)E + (one_map ? 1 : 0), KM = one_map ? KK : (int)K;
    if (one_map) {
        MX_TRY(launch_map0(ids, (int)t, KM, EM, o.map, s, GM_BM, (int)K));  // slot K: expert E
    } else {
        MX_TRY(launch_map0(ids, (int)t, (int)K, (int)E, o.map, s, GM_BM));
        if (p.has_shared) {
            hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((t + 255) / 256)), dim3(256), 0, s, o.zero_ids, t, 0u);
            MX_LAUNCH("k_fill_u32");
            MX_TRY(launch_map0(o.zero_ids, (int)t, 1, 1, o.map_sh, s, GM_BM));
        }
    }
    MX_STAGE();
    MX_TRY(launch_to_f16_rows(xin, t, (int)H, nullptr, o.x16, o.x16s, s));
    MX_STAGE();
    // one bucket map's gate+up (SwiGLU, act rows at its bucket positions from act_row0 on)
    // and down (rows token * KK + slot + out_add)
    auto experts = [&](const int32_t *map, int n_map_expert, int top_k, int n_routed, const uint8_t *wg,
                       const uint8_t *wu, const uint8_t *wd, const uint8_t *shg, const uint8_t *shu,
                       const uint8_t *shd, int64_t act_row0, int out_add, int dt_gu, int dt_d,
                       const StackGeom &geo_gu, const StackGeom &geo_d, const StackGeom &geo_sgu,
                       const StackGeom &geo_sd) -> mx_status {
        const MapLayout LM(n_map_expert, (int)t, top_k);
        GemmArgs ga{};
        ga.w[0] = wg; ga.w[1] = wu;
        ga.w_sh[0] = shg; ga.w_sh[1] = shu;
        ga.expert_bytes = geo_gu.expert_bytes; ga.row_bytes = geo_gu.row_bytes; ga.sh_row_bytes = geo_sgu.row_bytes;
        ga.n_expert = n_routed; ga.n_out = (int)FF; ga.k = (int)H;
        ga.a = o.x16; ga.a_scale = o.x16s; ga.a_div = top_k;
        ga.t = (int)t; ga.top_k = top_k; ga.n_map_expert = n_map_expert; ga.map = map;
        ga.out = o.act + act_row0 * FF;
        MX_TRY(launch_gemm(dt_gu, true, ga, s));
        MX_STAGE();
        MX_TRY(launch_to_f16_rows(ga.out, t * top_k, (int)FF, map + LM.off + n_map_expert,
                                  o.act16 + act_row0 * FF, o.act16s + act_row0, s));
        MX_STAGE();
        GemmArgs da = ga;
        da.w[0] = wd; da.w[1] = nullptr;
        da.w_sh[0] = shd; da.w_sh[1] = nullptr;
        da.expert_bytes = geo_d.expert_bytes; da.row_bytes = geo_d.row_bytes; da.sh_row_bytes = geo_sd.row_bytes;
        da.n_out = (int)H; da.k = (int)FF;
        da.a = o.act16 + act_row0 * FF; da.a_scale = o.act16s + act_row0; da.a_div = 0;
        da.out = o.down; da.out_stride = KK; da.out_add = out_add;
        MX_TRY(launch_gemm(dt_d, false, da, s));
        MX_STAGE();
        return MX_OK;
    };
    if (one_map) {
        MX_TRY(experts(o.map, EM, KM, (int)E, gg.w, gu.w, gd.w, sg.w, su.w, sd.w, 0, 0, L->gate.dtype,
                       L->down.dtype, gg, gd, sg, sd));
    } else {
        MX_TRY(experts(o.map, (int)E, (int)K, (int)E, gg.w, gu.w, gd.w, nullptr, nullptr, nullptr, 0, 0,
                       L->gate.dtype, L->down.dtype, gg, gd, gg, gd));
        if (p.has_shared)
            MX_TRY(experts(o.map_sh, 1, 1, 0, nullptr, nullptr, nullptr, sg.w, su.w, sd.w, t * K, (int)K,
                           L->shared_gate.dtype, L->shared_down.dtype, sg, sd, sg, sd));
    }
    MX_TRY(launch_combine_prefill(o.down, w, residual, (int)t, (int)K, S, (int)H, out, s));
    MX_STAGE();
    return MX_OK;
}
}  // namespace

extern "C" {

mx_status mx_moe_forward(const mx_moe_layer *L, const float *x, int64_t t, const float *residual, float *out,
                         uint32_t *ids_out, float *w_out, void *workspace, size_t workspace_bytes,
                         mx_stream_t stream) {
    return moe_forward_impl(L, x, t, residual, out, ids_out, w_out, workspace, workspace_bytes,
                            (hipStream_t)stream, nullptr);
}

mx_status mx_moe_forward_profiled(const mx_moe_layer *L, const float *x, int64_t t, const float *residual,
                                  float *out, uint32_t *ids_out, float *w_out, void *workspace,
                                  size_t workspace_bytes, mx_stream_t stream, float *stage_ms,
                                  int32_t max_stages, int32_t *n_stages) {
    if (!stage_ms || !n_stages) return fail(MX_ERR_NULL, "moe_forward_profiled: NULL stage output");
    StageTimer tm;
    MX_TRY(moe_forward_impl(L, x, t, residual, out, ids_out, w_out, workspace, workspace_bytes,
                            (hipStream_t)stream, &tm));
    if (tm.n == 0) {
        *n_stages = 0;
        return MX_OK;
    }
    MX_HIP(hipEventSynchronize(tm.ev[tm.n - 1]));
    int k = 0;
    for (int i = 1; i < tm.n && k < max_stages; i++, k++)
        MX_HIP(hipEventElapsedTime(&stage_ms[k], tm.ev[i - 1], tm.ev[i]));
    *n_stages = k;
    return MX_OK;
}

mx_status mx_probe_read(const void *src, int64_t nbytes, uint32_t *sink, mx_stream_t stream) {
    if (!src || !sink) return fail(MX_ERR_NULL, "probe_read: NULL pointer");
    if (nbytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15))
        return fail(MX_ERR_ALIGN, "probe_read: 16-byte-aligned source and size");
    return launch_read_probe(src, nbytes, sink, (hipStream_t)stream);
}

mx_status mx_moe_forward_repeat(const mx_moe_layer *L, const float *x, int64_t t, const float *residual, float *out,
                                uint32_t *ids_out, float *w_out, void *workspace, size_t workspace_bytes,
                                mx_stream_t stream, int32_t stage, int32_t times) {
    if (times < 0 || times > 16) return fail(MX_ERR_SHAPE, "moe_forward_repeat: times must be in 0..16");
    if (times > 1 && residual && residual == out)
        return fail(MX_ERR_SHAPE, "moe_forward_repeat: an in-place residual would be added once per repeat");
    Repeat rep;
    rep.stage = stage;
    rep.times = times;
    return moe_forward_impl(L, x, t, residual, out, ids_out, w_out, workspace, workspace_bytes, (hipStream_t)stream,
                            nullptr, rep);
}

}  // extern "C"

// ---- the forward that allocates nothing --------------------------------------------------
// A file-scope device array serves as the workspace.  In host code its name is
// only a stand-in: the device address comes from hipGetSymbolAddress, once per
// device (each GPU holds its own copy at its own address), and only that address
// is ever passed to kernels.  The forward keeps no state in its workspace (every
// call initialises what it reads), so nothing needs clearing between calls.
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)MX_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

mx_status scratch_for_current_device(void **out) {
    int dev = -1;
    MX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(MX_ERR_SHAPE, "no-alloc forward: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        MX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(MX_ERR_HIP, "no-alloc forward: no device address for the scratch array");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MX_OK;
}
}  // namespace

extern "C" {

size_t mx_moe_forward_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

mx_status mx_moe_forward_noalloc(const mx_moe_layer *L, const float *x, int64_t t, const float *residual, float *out,
                                 uint32_t *ids_out, float *w_out, mx_stream_t stream) {
    StackGeom gg, gu, gd, sg{}, su{}, sd{};
    MX_TRY(check_layer(L, t, gg, gu, gd, sg, su, sd));
    const size_t need = mx_moe_workspace_bytes(L, t);
    if (need > kNoAllocScratchBytes)
        return fail(MX_ERR_SCRATCH,
                    "no-alloc forward: t = %lld needs %zu bytes of workspace, its scratch holds %zu "
                    "(use mx_moe_forward with a caller workspace)",
                    (long long)t, need, kNoAllocScratchBytes);
    if (t == 0) return MX_OK;
    void *ws = nullptr;
    MX_TRY(scratch_for_current_device(&ws));
    return moe_forward_impl(L, x, t, residual, out, ids_out, w_out, ws, kNoAllocScratchBytes, (hipStream_t)stream,
                            nullptr);
}

uint64_t mx_tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id) {
    return tensor_key(seed, layer, tensor_id);
}

mx_status mx_synth_blocks(int32_t dtype, uint64_t key, void *dst, int64_t nbytes, mx_stream_t stream) {
    if (!supported(dtype)) return fail(MX_ERR_DTYPE, "synth: unsupported ggml type %d", (int)dtype);
    if (nbytes < 0 || nbytes % type_size(dtype))
        return fail(MX_ERR_BLOCK, "synth: nbytes must be a multiple of the %s block size", dt_name(dtype));
    if (nbytes == 0) return MX_OK;
    if (!dst) return fail(MX_ERR_NULL, "synth: dst is NULL");
    if (!aligned(dst, 2)) return fail(MX_ERR_ALIGN, "synth: dst must be 2-byte aligned");
    return launch_synth(dtype, key, static_cast<uint8_t *>(dst), nbytes, (hipStream_t)stream);
}

}  // extern "C"
