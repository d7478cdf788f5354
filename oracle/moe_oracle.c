/*
 * CPU oracle for the quantized indexed-MoE hot path -- TEST INFRASTRUCTURE.
 * See moe_oracle.h.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * Citations are file:line into the reference tree (crate `laguna`).
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__FP_FAST_FMA) || defined(__FAST_MATH__)
#error "the oracle must be built without fast-math / FP contraction"
#endif

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---- block geometry (mv.metal:55-80; GGUF/ggml block formats) ----------- */
int or_block_size(int dtype) {
    switch (dtype) {
    case OR_Q8_0: return 32;
    case OR_Q4_K: return 256;
    case OR_Q5_K: return 256;
    case OR_Q6_K: return 256;
    default: return -1;
    }
}

int or_type_size(int dtype) {
    switch (dtype) {
    case OR_Q8_0: return 34;  /* f16 d; i8 qs[32] */
    case OR_Q4_K: return 144; /* f16 d, dmin; u8 scales[12]; u8 qs[128] */
    case OR_Q5_K: return 176; /* f16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128] */
    case OR_Q6_K: return 210; /* u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d */
    default: return -1;
    }
}

/* ---- IEEE half <-> float ------------------------------------------------- */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0));
    int32_t e = (int32_t)(absx >> 23) - 127 + 15;
    uint32_t man = absx & 0x7FFFFFu;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) { /* subnormal or zero in half */
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t q = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++; /* may carry into exp: fine */
    return (uint16_t)(sign | q);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- dequantisation (mm_id.metal:75-167; candle QTensor::dequantize,
 *      moe.rs:173-175).  Rounding order: d1=fl(d*sc), m1=fl(dmin*m),
 *      y=fl(fl(d1*q)-m1) for Q4_K and Q5_K (q = 4 low bits + 16 * high bit);
 *      y=fl(fl(d*sc)*q) for Q6_K; y=fl(d*q) Q8_0. */
static void get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    /* mm_id.metal:89-92 */
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static void deq_q4_K(const uint8_t *b, float *y) {
    const float d = or_f16_to_f32(rd16(b));
    const float dmin = or_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *q = b + 16;
    for (int i = 0; i < 4; i++) {
        uint8_t sc, m;
        get_scale_min_k4(2 * i, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        get_scale_min_k4(2 * i + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) {
            float p1 = d1 * (float)(q[32 * i + l] & 0xF);
            y[64 * i + l] = p1 - m1;
            float p2 = d2 * (float)(q[32 * i + l] >> 4);
            y[64 * i + 32 + l] = p2 - m2;
        }
    }
}

/* Q5_K (mm_id.metal:113-134 per 16-value piece; the public ggml formula per
 * block): the Q4_K header, then qh[32] and qs[128].  Pair i (weights 64i ..
 * 64i+63) uses sub-blocks 2i / 2i+1: the low / high nibble of qs[32i + l] plus
 * 16 times bit 2i / 2i+1 of qh[l].  (The reference's d/16 with the nibble left
 * in the high half is the same value: every product is exact in f32.) */
static void deq_q5_K(const uint8_t *b, float *y) {
    const float d = or_f16_to_f32(rd16(b));
    const float dmin = or_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qh = b + 16;
    const uint8_t *q = b + 48;
    for (int i = 0; i < 4; i++) {
        uint8_t sc, m;
        get_scale_min_k4(2 * i, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        get_scale_min_k4(2 * i + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) {
            const int v1 = (q[32 * i + l] & 0xF) + (((qh[l] >> (2 * i)) & 1) << 4);
            const int v2 = (q[32 * i + l] >> 4) + (((qh[l] >> (2 * i + 1)) & 1) << 4);
            float p1 = d1 * (float)v1;
            y[64 * i + l] = p1 - m1;
            float p2 = d2 * (float)v2;
            y[64 * i + 32 + l] = p2 - m2;
        }
    }
}

static void deq_q6_K(const uint8_t *b, float *y) {
    const float d = or_f16_to_f32(rd16(b + 208));
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n;
        const uint8_t *qh = b + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
        float *yy = y + 128 * n;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            float s;
            s = d * (float)sc[is + 0]; yy[l] = s * (float)q1;
            s = d * (float)sc[is + 2]; yy[l + 32] = s * (float)q2;
            s = d * (float)sc[is + 4]; yy[l + 64] = s * (float)q3;
            s = d * (float)sc[is + 6]; yy[l + 96] = s * (float)q4;
        }
    }
}

static void deq_q8_0(const uint8_t *b, float *y) {
    const float d = or_f16_to_f32(rd16(b));
    const int8_t *qs = (const int8_t *)(b + 2);
    for (int i = 0; i < 32; i++) y[i] = (float)qs[i] * d;
}

int or_dequantize(int dtype, const uint8_t *blocks, int64_t n, float *out) {
    const int bs = or_block_size(dtype), ts = or_type_size(dtype);
    if (bs <= 0 || n % bs) return -1;
    const int64_t nb = n / bs;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = blocks + i * ts;
        float *y = out + i * bs;
        if (dtype == OR_Q4_K) deq_q4_K(b, y);
        else if (dtype == OR_Q5_K) deq_q5_K(b, y);
        else if (dtype == OR_Q6_K) deq_q6_K(b, y);
        else deq_q8_0(b, y);
    }
    return 0;
}

/* ---- seeded synthetic blocks ---------------------------------------------
 * Counter-based splitmix64 stream: byte j of a tensor is byte (j & 7) of
 * mix64(key + (j/8 + 1) * GAMMA).  The f16 super-block scales are then
 * overwritten with d = f16(0.001 + 0.009 u), u uniform on [0,1) in 2^-24 steps
 * (and dmin likewise for Q4_K / Q5_K), f32 ops rounded separately, f16 by RNE.
 * The device generator in the library implements the same definition. */
#define OR_GAMMA 0x9E3779B97F4A7C15ull

uint64_t or_mix64(uint64_t z) {
    z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27; z *= 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z;
}

uint64_t or_tensor_key(uint64_t seed, uint32_t layer, uint32_t tensor_id) {
    uint64_t a = or_mix64(seed + OR_GAMMA);
    uint64_t b = or_mix64((((uint64_t)layer << 16) | tensor_id) + 2 * OR_GAMMA);
    return or_mix64(a ^ b);
}

static uint16_t synth_scale(uint64_t h, int which) {
    uint32_t bits24 = which == 0 ? (uint32_t)(h >> 40) : (uint32_t)((h >> 16) & 0xFFFFFFu);
    float u = (float)bits24 * (1.0f / 16777216.0f);
    float p = 0.009f * u;
    float v = 0.001f + p;
    return or_f32_to_f16(v);
}

int or_synth_blocks(int dtype, uint64_t key, int64_t byte_off, int64_t nbytes, uint8_t *out) {
    const int ts = or_type_size(dtype);
    if (ts <= 0) return -1;
    #pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < nbytes; j++) {
        const uint64_t g = (uint64_t)(byte_off + j);
        const uint64_t w = or_mix64(key + ((g >> 3) + 1) * OR_GAMMA);
        out[j] = (uint8_t)(w >> (8 * (g & 7)));
    }
    /* fix-up of the f16 scale fields of every block overlapping the range */
    const int64_t b0 = byte_off / ts, b1 = (byte_off + nbytes + ts - 1) / ts;
    for (int64_t b = b0; b < b1; b++) {
        const uint64_t h = or_mix64((key ^ 0xA0761D6478BD642Full) + ((uint64_t)b + 1) * OR_GAMMA);
        uint16_t f[2];
        int off[2], nf = 0;
        if (dtype == OR_Q4_K || dtype == OR_Q5_K) {
            f[0] = synth_scale(h, 0); off[0] = 0; f[1] = synth_scale(h, 1); off[1] = 2; nf = 2;
        }
        else if (dtype == OR_Q6_K) { f[0] = synth_scale(h, 0); off[0] = 208; nf = 1; }
        else { f[0] = synth_scale(h, 0); off[0] = 0; nf = 1; }
        for (int i = 0; i < nf; i++) {
            for (int k = 0; k < 2; k++) {
                const int64_t gpos = b * ts + off[i] + k;
                if (gpos >= byte_off && gpos < byte_off + nbytes)
                    out[gpos - byte_off] = (uint8_t)(f[i] >> (8 * k));
            }
        }
    }
    return 0;
}

/* ---- routing (moe.rs:84-119) --------------------------------------------- */
void or_route_logits(const float *x, const float *router_t, int64_t t, int64_t hidden,
                     int64_t n_expert, float *logits) {
    /* moe.rs:84-87: logits = x[t,H] . router_t[H,E] in f32 */
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < t * n_expert; i++) {
        const int64_t r = i / n_expert, e = i % n_expert;
        double acc = 0.0;
        for (int64_t h = 0; h < hidden; h++)
            acc += (double)x[r * hidden + h] * (double)router_t[h * n_expert + e];
        logits[i] = (float)acc;
    }
}

void or_route_from_logits(const float *logits, const float *bias, int64_t t, int64_t n_expert,
                          int64_t top_k, double scale, int norm, uint32_t *ids, float *w) {
    const float floor_ = 6.103515625e-5f; /* moe.rs:14 WEIGHTS_SUM_FLOOR */
    float *probs = (float *)malloc(sizeof(float) * n_expert);
    float *sel = (float *)malloc(sizeof(float) * n_expert);
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * n_expert);
    for (int64_t r = 0; r < t; r++) {
        for (int64_t e = 0; e < n_expert; e++) {
            /* candle sigmoid: (exp(-v) + 1)^-1, moe.rs:101 */
            const float v = logits[r * n_expert + e];
            const float ex = expf(-v);
            probs[e] = 1.0f / (ex + 1.0f);
            sel[e] = probs[e] + bias[e]; /* moe.rs:102: bias affects selection only */
            order[e] = (uint32_t)e;
        }
        /* stable descending arg-sort (moe.rs:104-106): insertion sort keeps
         * equal keys in index order, so ties resolve to the lower expert id. */
        for (int64_t i = 1; i < n_expert; i++) {
            uint32_t cur = order[i];
            int64_t j = i - 1;
            while (j >= 0 && sel[order[j]] < sel[cur]) { order[j + 1] = order[j]; j--; }
            order[j + 1] = cur;
        }
        float sum = 0.0f;
        for (int64_t k = 0; k < top_k; k++) {
            ids[r * top_k + k] = order[k];
            w[r * top_k + k] = probs[order[k]]; /* gather from UNBIASED probs */
            sum += w[r * top_k + k];
        }
        if (norm) { /* moe.rs:110-114 */
            if (sum < floor_) sum = floor_; /* clamp(floor, +inf) */
            for (int64_t k = 0; k < top_k; k++) w[r * top_k + k] = w[r * top_k + k] / sum;
        }
        if (scale != 0.0 && scale != 1.0) { /* moe.rs:115-117 */
            const float s = (float)scale;
            for (int64_t k = 0; k < top_k; k++) w[r * top_k + k] = w[r * top_k + k] * s;
        }
    }
    free(probs); free(sel); free(order);
}

/* ---- matmul helpers --------------------------------------------------------- */
static float *deq_matrix(int dtype, const uint8_t *blocks, int64_t rows, int64_t k) {
    float *m = (float *)malloc(sizeof(float) * rows * k);
    if (!m) return NULL;
    if (or_dequantize(dtype, blocks, rows * k, m) != 0) { free(m); return NULL; }
    return m;
}

/* y[m,n] = a[m,k] . W[n,k]^T, f64 accumulation rounded to f32 */
static void matmul_nt(const float *a, const float *wt, int64_t m, int64_t n, int64_t k, float *y) {
    /* y[r, c] = sum_j a[r, j] * wt[c, j], each output summed in j order in
     * double and rounded once.  Four rows share every weight load (the order of
     * each output's sum is unchanged), so large m runs at several GFLOP/s. */
    #pragma omp parallel for schedule(dynamic, 16)
    for (int64_t c = 0; c < n; c++) {
        const float *wr = wt + c * k;
        int64_t r = 0;
        for (; r + 4 <= m; r += 4) {
            const float *a0 = a + r * k, *a1 = a0 + k, *a2 = a1 + k, *a3 = a2 + k;
            double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
            for (int64_t j = 0; j < k; j++) {
                const double wj = (double)wr[j];
                s0 += (double)a0[j] * wj;
                s1 += (double)a1[j] * wj;
                s2 += (double)a2[j] * wj;
                s3 += (double)a3[j] * wj;
            }
            y[r * n + c] = (float)s0;
            y[(r + 1) * n + c] = (float)s1;
            y[(r + 2) * n + c] = (float)s2;
            y[(r + 3) * n + c] = (float)s3;
        }
        for (; r < m; r++) {
            const float *ar = a + r * k;
            double acc = 0.0;
            for (int64_t j = 0; j < k; j++) acc += (double)ar[j] * (double)wr[j];
            y[r * n + c] = (float)acc;
        }
    }
}

static inline float silu_f(float g) { return g / (1.0f + expf(-g)); } /* silu_mul.metal:70 */

int or_mul_mv_id(int dtype, const uint8_t *const *experts, int64_t n_expert, int64_t n_out,
                 int64_t k, const float *x, int64_t x_per_row, const uint32_t *ids, int64_t t,
                 int64_t top_k, float *dst) {
    /* dispatch.rs:2273-2301: per (token, slot) dot of every expert row with the
     * token's shared row (x_per_row==1) or its per-slot row (x_per_row==top_k). */
    if (x_per_row != 1 && x_per_row != top_k) return -1;
    for (int64_t tok = 0; tok < t; tok++) {
        for (int64_t s = 0; s < top_k; s++) {
            const uint32_t e = ids[tok * top_k + s];
            if (e >= n_expert || !experts[e]) return -2;
            float *wd = deq_matrix(dtype, experts[e], n_out, k);
            if (!wd) return -3;
            const float *xr = x + (tok * x_per_row + (x_per_row == 1 ? 0 : s)) * k;
            matmul_nt(xr, wd, 1, n_out, k, dst + (tok * top_k + s) * n_out);
            free(wd);
        }
    }
    return 0;
}

int or_mul_mv(int dtype, const uint8_t *w, int64_t n_out, int64_t k, const float *x, int64_t t,
              float *dst) {
    float *wd = deq_matrix(dtype, w, n_out, k);
    if (!wd) return -3;
    matmul_nt(x, wd, t, n_out, k, dst);
    free(wd);
    return 0;
}

/* ---- map0 (mm_id.metal:207-259) -------------------------------------------- */
int or_map0(const uint32_t *ids, int64_t t, int64_t top_k, int64_t n_expert, int32_t *tpe,
            int32_t *hids) {
    for (int64_t e = 0; e < n_expert; e++) {
        int32_t n = 0;
        for (int64_t tok = 0; tok < t; tok++) {
            int sel = 0;
            for (int64_t s = 0; s < top_k; s++) sel += (ids[tok * top_k + s] == (uint32_t)e) * (int)(s + 1);
            if (sel > 0) hids[e * t + n++] = (int32_t)(tok * top_k + sel - 1);
        }
        tpe[e] = n;
    }
    return 0;
}

/* ---- elementwise ------------------------------------------------------------- */
void or_silu_mul(const float *gate, const float *up, int64_t n, float *dst) {
    /* silu_mul.metal:57-72: s = g/(1+exp(-g)); dst = s*up, two roundings */
    for (int64_t i = 0; i < n; i++) {
        const float s = silu_f(gate[i]);
        dst[i] = s * up[i];
    }
}

void or_combine(const float *down, const float *col_l2, const float *w, int64_t seq,
                int64_t top_k, int64_t n_out, float *dst) {
    /* combine.metal:70-133: dst[s,c] = sum_k down[s,k,c] * w[s,k]; the rescale
     * form is ((down*l2)*2^-15)*w, each multiply rounded. */
    for (int64_t s = 0; s < seq; s++)
        for (int64_t c = 0; c < n_out; c++) {
            float acc = 0.0f;
            for (int64_t k = 0; k < top_k; k++) {
                float d = down[(s * top_k + k) * n_out + c];
                if (col_l2) { d = d * col_l2[s * top_k + k]; d = d * (1.0f / 32768.0f); }
                const float r = d * w[s * top_k + k];
                acc = acc + r;
            }
            dst[s * n_out + c] = acc;
        }
}

void or_rmsnorm(const float *x, const float *alpha, int64_t rows, int64_t dim, float eps,
                float *dst) {
    /* candle_nn RmsNorm (model.rs:340 ffn_norm): m = sqrt(sum(x^2)/dim + eps);
     * dst = x / m * alpha, f32 throughout. */
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * dim;
        float sum2 = 0.0f;
        for (int64_t i = 0; i < dim; i++) sum2 += xr[i] * xr[i];
        const float m = sqrtf(sum2 / (float)dim + eps);
        for (int64_t i = 0; i < dim; i++) dst[r * dim + i] = xr[i] / m * alpha[i];
    }
}

/* ---- ReferenceExperts::forward (moe.rs:141-187) --------------------------- */
int or_reference_experts(int gate_dt, const uint8_t *const *gate, int up_dt,
                         const uint8_t *const *up, int down_dt, const uint8_t *const *down,
                         int64_t n_expert, int64_t hidden, int64_t ff, const float *x,
                         const uint32_t *ids, const float *w, int64_t t, int64_t top_k,
                         float *out) {
    int64_t *cnt = (int64_t *)calloc((size_t)n_expert, sizeof(int64_t));
    int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * (size_t)(t * top_k));
    float *wts = (float *)malloc(sizeof(float) * (size_t)(t * top_k));
    if (!cnt || !rows || !wts) return -3;
    for (int64_t i = 0; i < t * top_k; i++) {
        if (ids[i] >= (uint64_t)n_expert) { free(cnt); free(rows); free(wts); return -2; }
        cnt[ids[i]]++;
    }
    memset(out, 0, sizeof(float) * (size_t)(t * hidden));
    int rc = 0;
    for (int64_t e = 0; e < n_expert && rc == 0; e++) {
        if (!cnt[e]) continue;
        /* moe.rs:154-162: bucket (token, weight) pairs, tokens ascending */
        int64_t m = 0;
        for (int64_t tok = 0; tok < t; tok++)
            for (int64_t s = 0; s < top_k; s++)
                if (ids[tok * top_k + s] == (uint32_t)e) { rows[m] = tok; wts[m] = w[tok * top_k + s]; m++; }
        if (!gate[e] || !up[e] || !down[e]) { rc = -2; break; }
        float *xe = (float *)malloc(sizeof(float) * m * hidden); /* index_select moe.rs:171 */
        for (int64_t j = 0; j < m; j++) memcpy(xe + j * hidden, x + rows[j] * hidden, sizeof(float) * hidden);
        float *gw = deq_matrix(gate_dt, gate[e], ff, hidden);
        float *uw = deq_matrix(up_dt, up[e], ff, hidden);
        float *dw = deq_matrix(down_dt, down[e], hidden, ff);
        float *g = (float *)malloc(sizeof(float) * m * ff);
        float *u = (float *)malloc(sizeof(float) * m * ff);
        float *d = (float *)malloc(sizeof(float) * m * hidden);
        if (!xe || !gw || !uw || !dw || !g || !u || !d) rc = -3;
        if (rc == 0) {
            matmul_nt(xe, gw, m, ff, hidden, g);                    /* moe.rs:177 */
            for (int64_t i = 0; i < m * ff; i++) g[i] = silu_f(g[i]);
            matmul_nt(xe, uw, m, ff, hidden, u);                    /* moe.rs:178 */
            for (int64_t i = 0; i < m * ff; i++) g[i] = g[i] * u[i]; /* moe.rs:179 */
            matmul_nt(g, dw, m, hidden, ff, d);                     /* moe.rs:180 */
            for (int64_t j = 0; j < m; j++)                         /* moe.rs:182-184 */
                for (int64_t c = 0; c < hidden; c++) {
                    const float v = d[j * hidden + c] * wts[j];
                    out[rows[j] * hidden + c] = out[rows[j] * hidden + c] + v;
                }
        }
        free(xe); free(gw); free(uw); free(dw); free(g); free(u); free(d);
    }
    free(cnt); free(rows); free(wts);
    return rc;
}

/* ---- SharedExpert / swiglu (moe.rs:342-344, 369-374) ----------------------- */
int or_swiglu(int gate_dt, const uint8_t *gate, int up_dt, const uint8_t *up, int down_dt,
              const uint8_t *down, int64_t hidden, int64_t ff, const float *x, int64_t t,
              float *out) {
    float *gw = deq_matrix(gate_dt, gate, ff, hidden);
    float *uw = deq_matrix(up_dt, up, ff, hidden);
    float *dw = deq_matrix(down_dt, down, hidden, ff);
    float *g = (float *)malloc(sizeof(float) * t * ff);
    float *u = (float *)malloc(sizeof(float) * t * ff);
    int rc = 0;
    if (!gw || !uw || !dw || !g || !u) rc = -3;
    if (rc == 0) {
        matmul_nt(x, gw, t, ff, hidden, g);
        for (int64_t i = 0; i < t * ff; i++) g[i] = silu_f(g[i]);
        matmul_nt(x, uw, t, ff, hidden, u);
        for (int64_t i = 0; i < t * ff; i++) g[i] = g[i] * u[i];
        matmul_nt(g, dw, t, hidden, ff, out);
    }
    free(gw); free(uw); free(dw); free(g); free(u);
    return rc;
}
