/*
 * moe_oracle.c — CPU restatement of JGalego/Moe's routed-MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed
 * CPU baseline; nothing in the product (moe_amd/) links, loads or calls it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * It restates, function by function, the reference's CPU arithmetic so that
 * a result from here is bit-identical to what the Rust engine computes on an
 * x86-64 host with AVX2+FMA and glibc:
 *
 *   f16 <-> f32 ............ src/quant.rs:131-174
 *   Dt::row_bytes .......... src/quant.rs:68-83
 *   dequant (F32/F16/BF16/Q8/Q4/Q5) src/quant.rs:177-227
 *   quantize (F32/Q8/Q4/Q5)  src/quant.rs:304-365
 *   dot_avx2 ............... src/quant.rs:386-420 (lane and reduction order)
 *   matmul ................. src/quant.rs:482-506 (one dot per (row, token))
 *   softmax ................ src/model.rs:218-228
 *   Mlp::forward (SwiGLU) .. src/model.rs:26-35
 *   feed_forward Ffn::Moe .. src/model.rs:841-971
 *   prune_groups ........... src/model.rs:999-1012
 *
 * Numerics: compile with -O2 -mavx2 -mfma -ffp-contract=off and without
 * -ffast-math, so the only fused multiply-adds are the explicit ones the
 * reference also issues (_mm256_fmadd_ps).  exp() is glibc's expf, which is
 * what Rust's f32::exp resolves to on linux-gnu.
 *
 * Sorting: Rust's sort_unstable_by is an insertion sort (stable) for slices
 * of at most 20 elements.  Above that it is ipnsort, whose order among exact
 * ties is not specified; this restatement uses the stable order (descending
 * rank, lower index first) for every length and counts the tokens on which
 * an exact tie reaches the selected prefix, so such cases are reported rather
 * than silently assumed ("parity unpinned" for ties at E > 20).
 *
 * Threading mirrors the reference's shape (row bands of
 * clamp(rows/(threads*4), 1, 64), experts in parallel) through OpenMP; every
 * output element is still produced by exactly one dot call in a fixed order,
 * so results do not depend on the thread count.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Storage formats, numbered as GGUF numbers them (src/gguf.rs:166-198). */
enum { ODT_F32 = 0, ODT_F16 = 1, ODT_Q4 = 2, ODT_Q5 = 6, ODT_Q8 = 8, ODT_BF16 = 30 };
#define BLK 32

/* ------------------------------------------------------------ f16 helpers */

/* src/quant.rs:131-147 */
static inline float f16_to_f32(uint16_t b) {
    uint32_t sign = ((uint32_t)(b >> 15)) << 31;
    uint32_t exp = (b >> 10) & 0x1f;
    uint32_t man = b & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t lz = (uint32_t)__builtin_clz(man);
        bits = sign | ((134u - lz) << 23) | ((man << (lz - 8)) & 0x7fffffu);
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/quant.rs:149-174 */
static inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    int32_t exp = (int32_t)((x >> 23) & 0xff) - 127 + 15;
    uint32_t man = x & 0x7fffff;
    if (exp >= 0x1f) return sign | 0x7c00;
    if (exp <= 0) {
        if (exp < -10) return sign;
        uint32_t m = (man | 0x800000) >> (uint32_t)(1 - exp);
        return sign | (uint16_t)((m + 0x1000) >> 13);
    }
    uint32_t rounded = man + 0x0fff + ((man >> 13) & 1);
    if (rounded & 0x800000) {
        exp += 1;
        if (exp >= 0x1f) return sign | 0x7c00;
    }
    return sign | (uint16_t)(exp << 10) | (uint16_t)((rounded & 0x7fffff) >> 13);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---------------------------------------------------------------- formats */

/* src/quant.rs:68-83 */
size_t orc_row_bytes(int dt, size_t cols) {
    switch (dt) {
    case ODT_F32: return cols * 4;
    case ODT_F16:
    case ODT_BF16: return cols * 2;
    case ODT_Q8: return cols / BLK * (2 + BLK);
    case ODT_Q4: return cols / BLK * (2 + BLK / 2);
    case ODT_Q5: return cols / BLK * (2 + BLK / 8 + BLK / 2);
    default: return 0;
    }
}

/* src/quant.rs:177-227 — one row of `cols` values. */
static void dequant_row(int dt, const uint8_t *src, size_t cols, float *out) {
    switch (dt) {
    case ODT_F32:
        memcpy(out, src, cols * 4);
        break;
    case ODT_F16:
        for (size_t i = 0; i < cols; i++) out[i] = f16_to_f32(rd16(src + 2 * i));
        break;
    case ODT_BF16:
        for (size_t i = 0; i < cols; i++) {
            uint32_t b = (uint32_t)rd16(src + 2 * i) << 16;
            memcpy(&out[i], &b, 4);
        }
        break;
    case ODT_Q8:
        for (size_t b = 0; b < cols / BLK; b++) {
            const uint8_t *blk = src + b * (2 + BLK);
            float d = f16_to_f32(rd16(blk));
            for (int i = 0; i < BLK; i++) out[b * BLK + i] = d * (float)(int8_t)blk[2 + i];
        }
        break;
    case ODT_Q4:
        for (size_t b = 0; b < cols / BLK; b++) {
            const uint8_t *blk = src + b * (2 + BLK / 2);
            float d = f16_to_f32(rd16(blk));
            for (int i = 0; i < BLK / 2; i++) {
                uint8_t v = blk[2 + i];
                out[b * BLK + i] = d * (float)((int)(v & 0x0f) - 8);
                out[b * BLK + i + BLK / 2] = d * (float)((int)(v >> 4) - 8);
            }
        }
        break;
    case ODT_Q5:
        for (size_t b = 0; b < cols / BLK; b++) {
            const uint8_t *blk = src + b * (2 + BLK / 8 + BLK / 2);
            float d = f16_to_f32(rd16(blk));
            const uint8_t *hi = blk + 2, *qs = blk + 2 + BLK / 8;
            for (int i = 0; i < BLK / 2; i++) {
                uint8_t v = qs[i];
                int b0 = (hi[i / 8] >> (i % 8)) & 1;
                int j = i + BLK / 2;
                int b1 = (hi[j / 8] >> (j % 8)) & 1;
                out[b * BLK + i] = d * (float)(((int)(v & 0x0f) | (b0 << 4)) - 16);
                out[b * BLK + j] = d * (float)(((int)(v >> 4) | (b1 << 4)) - 16);
            }
        }
        break;
    }
}

/* Rust `f32 as i32`: saturating, NaN -> 0. */
static inline int32_t sat_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}
static inline float fclamp(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline int32_t iclamp(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* Rust f32::max / f32::abs fold as used for amax. */
static inline float fmax_rs(float a, float b) { return (a != a) ? b : ((b != b) ? a : (a > b ? a : b)); }

/* src/quant.rs:304-365 — one row. */
static void quantize_row(int dt, const float *s, size_t cols, uint8_t *dst) {
    switch (dt) {
    case ODT_F32:
        memcpy(dst, s, cols * 4);
        break;
    case ODT_F16:
        for (size_t i = 0; i < cols; i++) {
            uint16_t h = f32_to_f16(s[i]);
            dst[2 * i] = (uint8_t)h;
            dst[2 * i + 1] = (uint8_t)(h >> 8);
        }
        break;
    case ODT_Q8:
        for (size_t b = 0; b < cols / BLK; b++) {
            const float *v = s + b * BLK;
            uint8_t *blk = dst + b * (2 + BLK);
            float amax = 0.0f;
            for (int i = 0; i < BLK; i++) amax = fmax_rs(amax, fabsf(v[i]));
            float d = amax / 127.0f;
            uint16_t dh = f32_to_f16(d);
            blk[0] = (uint8_t)dh;
            blk[1] = (uint8_t)(dh >> 8);
            float inv = d > 0.0f ? 1.0f / f16_to_f32(dh) : 0.0f;
            for (int i = 0; i < BLK; i++) {
                float q = fclamp(roundf(v[i] * inv), -127.0f, 127.0f);
                blk[2 + i] = (uint8_t)(int8_t)sat_i32(q);
            }
        }
        break;
    case ODT_Q4:
        for (size_t b = 0; b < cols / BLK; b++) {
            const float *v = s + b * BLK;
            uint8_t *blk = dst + b * (2 + BLK / 2);
            float amax = 0.0f;
            for (int i = 0; i < BLK; i++) amax = fmax_rs(amax, fabsf(v[i]));
            float d = amax / 7.0f;
            uint16_t dh = f32_to_f16(d);
            blk[0] = (uint8_t)dh;
            blk[1] = (uint8_t)(dh >> 8);
            float inv = d > 0.0f ? 1.0f / f16_to_f32(dh) : 0.0f;
            for (int i = 0; i < BLK / 2; i++) {
                uint8_t lo = (uint8_t)iclamp(sat_i32(roundf(v[i] * inv)) + 8, 0, 15);
                uint8_t hi = (uint8_t)iclamp(sat_i32(roundf(v[i + BLK / 2] * inv)) + 8, 0, 15);
                blk[2 + i] = (uint8_t)(lo | (hi << 4));
            }
        }
        break;
    case ODT_Q5:
        for (size_t b = 0; b < cols / BLK; b++) {
            const float *v = s + b * BLK;
            uint8_t *blk = dst + b * (2 + BLK / 8 + BLK / 2);
            float amax = 0.0f;
            for (int i = 0; i < BLK; i++) amax = fmax_rs(amax, fabsf(v[i]));
            float d = amax / 15.0f;
            uint16_t dh = f32_to_f16(d);
            blk[0] = (uint8_t)dh;
            blk[1] = (uint8_t)(dh >> 8);
            float inv = d > 0.0f ? 1.0f / f16_to_f32(dh) : 0.0f;
            memset(blk + 2, 0, BLK / 8 + BLK / 2);
            for (int i = 0; i < BLK / 2; i++) {
                uint8_t lo = (uint8_t)iclamp(sat_i32(roundf(v[i] * inv)) + 16, 0, 31);
                uint8_t hi = (uint8_t)iclamp(sat_i32(roundf(v[i + BLK / 2] * inv)) + 16, 0, 31);
                blk[2 + BLK / 8 + i] = (uint8_t)((lo & 0x0f) | ((hi & 0x0f) << 4));
                int j0 = i, j1 = i + BLK / 2;
                blk[2 + j0 / 8] |= (uint8_t)(((lo >> 4) & 1) << (j0 % 8));
                blk[2 + j1 / 8] |= (uint8_t)(((hi >> 4) & 1) << (j1 % 8));
            }
        }
        break;
    }
}

void orc_f16_to_f32(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f16_to_f32(in[i]);
}
void orc_f32_to_f16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f32_to_f16(in[i]);
}
void orc_quantize_rows(int dt, const float *src, size_t rows, size_t cols, uint8_t *dst) {
    size_t rb = orc_row_bytes(dt, cols);
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) quantize_row(dt, src + r * cols, cols, dst + r * rb);
}
void orc_dequant_rows(int dt, const uint8_t *src, size_t rows, size_t cols, float *dst) {
    size_t rb = orc_row_bytes(dt, cols);
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) dequant_row(dt, src + r * rb, cols, dst + r * cols);
}

/* ------------------------------------------------------------------- dot */

/* src/quant.rs:386-420, bit for bit: two 8-lane FMA accumulators over
 * 16-element chunks, an 8-element step into acc0, then
 * (acc0+acc1) -> hi128+lo128 -> hadd -> hadd, and a scalar tail of
 * separate multiply and add. */
__attribute__((target("avx2,fma"))) float orc_dot(const float *a, const float *b, size_t n) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
        acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), acc1);
    }
    for (; i + 8 <= n; i += 8) acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc0);
    __m256 s = _mm256_add_ps(acc0, acc1);
    __m128 q = _mm_add_ps(_mm256_extractf128_ps(s, 1), _mm256_castps256_ps128(s));
    q = _mm_hadd_ps(q, q);
    q = _mm_hadd_ps(q, q);
    float out = _mm_cvtss_f32(q);
    for (; i < n; i++) {
        float p = a[i] * b[i];
        out += p;
    }
    return out;
}

/* The same order written with scalar fmaf, as an independent check of the
 * vector version (and the form the device kernels mirror). */
float orc_dot_scalar(const float *a, const float *b, size_t n) {
    float acc[16] = {0};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    float s[8], q[4];
    for (int j = 0; j < 8; j++) s[j] = acc[j] + acc[j + 8];
    for (int j = 0; j < 4; j++) q[j] = s[j + 4] + s[j];
    float out = (q[0] + q[1]) + (q[2] + q[3]);
    for (; i < n; i++) {
        float p = a[i] * b[i];
        out += p;
    }
    return out;
}

/* ---------------------------------------------------------------- matmul */

typedef struct {
    int32_t dt, rows, cols, _pad;
    const uint8_t *data;
} orc_qt;

/* src/quant.rs:482-506: out[t][r] = dot(dequant(row r), x[t]).  Row bands of
 * clamp(rows/(threads*4), 1, 64) go to the pool; each row is dequantised once
 * and dotted with every token. */
static void matmul(const orc_qt *w, const float *x, size_t t, float *out) {
    size_t rows = (size_t)w->rows, cols = (size_t)w->cols;
    size_t rb = orc_row_bytes(w->dt, cols);
    int threads = omp_in_parallel() ? 1 : omp_get_max_threads();
    size_t band = rows / ((size_t)threads * 4);
    if (band < 1) band = 1;
    if (band > 64) band = 64;
    size_t nbands = (rows + band - 1) / band;
#pragma omp parallel for schedule(dynamic, 1) if (threads > 1)
    for (size_t bi = 0; bi < nbands; bi++) {
        float *buf = (float *)malloc(cols * sizeof(float));
        size_t r1 = (bi + 1) * band < rows ? (bi + 1) * band : rows;
        for (size_t r = bi * band; r < r1; r++) {
            dequant_row(w->dt, w->data + r * rb, cols, buf);
            for (size_t ti = 0; ti < t; ti++) out[ti * rows + r] = orc_dot(buf, x + ti * cols, cols);
        }
        free(buf);
    }
}

void orc_matmul(const orc_qt *w, const float *x, size_t t, float *out) { matmul(w, x, t, out); }

/* src/model.rs:26-35: down(silu(gate x) * up x), silu as a / (1 + exp(-a)). */
static void mlp_forward(const orc_qt *gate, const orc_qt *up, const orc_qt *down, const float *x, size_t t,
                        float *out) {
    size_t n = (size_t)gate->rows;
    float *g = (float *)malloc(t * n * sizeof(float));
    float *u = (float *)malloc(t * n * sizeof(float));
    matmul(gate, x, t, g);
    matmul(up, x, t, u);
    for (size_t i = 0; i < t * n; i++) {
        float a = g[i];
        float den = 1.0f + expf(-a);
        float q = a / den;
        g[i] = q * u[i];
    }
    matmul(down, g, t, out);
    free(g);
    free(u);
}

/* ---------------------------------------------------------------- routing */

/* Rust f32::total_cmp as an order-preserving signed key. */
static inline int32_t tkey(float v) {
    int32_t b;
    memcpy(&b, &v, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* src/model.rs:218-228 */
static void softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) m = fmax_rs(m, x[i]);
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        s += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= s;
}

/* Stable insertion sort of idx[0..n) by descending rank: Rust's
 * insertion_sort_shift_left under `rank[b].total_cmp(&rank[a])`. */
static void sort_desc(int32_t *idx, size_t n, const float *rank) {
    for (size_t i = 1; i < n; i++) {
        int32_t v = idx[i];
        int32_t kv = tkey(rank[v]);
        size_t j = i;
        while (j > 0 && kv > tkey(rank[idx[j - 1]])) {
            idx[j] = idx[j - 1];
            j--;
        }
        idx[j] = v;
    }
}

/* src/model.rs:999-1012 */
static void prune_groups(float *rank, size_t n, size_t groups, size_t keep) {
    size_t per = n / groups;
    int32_t gi[1024];
    float gs[1024];
    for (size_t g = 0; g < groups; g++) {
        /* top two of the group by total_cmp, summed from -0.0 (Rust's f32
         * Sum fold starts at -0.0). */
        int32_t k1 = INT32_MIN, k2 = INT32_MIN;
        float v1 = 0.0f, v2 = 0.0f;
        for (size_t i = 0; i < per; i++) {
            float v = rank[g * per + i];
            int32_t k = tkey(v);
            if (k > k1) {
                k2 = k1, v2 = v1;
                k1 = k, v1 = v;
            } else if (k > k2) {
                k2 = k, v2 = v;
            }
        }
        float s = -0.0f;
        if (per >= 1) s = s + v1;
        if (per >= 2) s = s + v2;
        gi[g] = (int32_t)g;
        gs[g] = s;
    }
    sort_desc(gi, groups, gs);
    for (size_t r = keep; r < groups; r++)
        for (size_t i = 0; i < per; i++) rank[(size_t)gi[r] * per + i] = -INFINITY;
}

typedef struct {
    int32_t hidden, n_experts, top_k, sigmoid, norm_topk, n_group, topk_group;
    float routed_scale;
    orc_qt router;           /* F32 [E, H] */
    const float *e_bias;     /* [E] or NULL */
    const orc_qt *experts;   /* [E * 3]: gate, up, down */
    const orc_qt *shared;    /* [3] or NULL */
    const orc_qt *shared_gate; /* [1, H] or NULL */
} orc_layer;

typedef struct {
    const int32_t *disabled;
    int32_t n_disabled;
    const int32_t *forced;
    int32_t n_forced;
    float temp;
    int32_t top_k;
} orc_routing;

/* Route one token: src/model.rs:855-897.  `sc` holds the token's logits on
 * entry and the gate scores on exit.  Writes k = min(top_k, E) experts
 * strongest first.  Returns 1 when an exact rank tie reaches the selected
 * prefix (the case where ipnsort's order is unspecified for E > 20). */
static int route_token(const orc_layer *L, const orc_routing *ovr, int top_k, float *sc, float *rank, int32_t *idx,
                       int32_t *sel, float *w) {
    size_t n = (size_t)L->n_experts;
    if (L->sigmoid) {
        for (size_t e = 0; e < n; e++) {
            float nv = -sc[e];
            float den = 1.0f + expf(nv);
            sc[e] = 1.0f / den;
        }
    } else {
        softmax(sc, n);
    }
    for (size_t e = 0; e < n; e++) rank[e] = L->e_bias ? sc[e] + L->e_bias[e] : sc[e];
    if (L->n_group > 1 && L->topk_group < L->n_group) prune_groups(rank, n, (size_t)L->n_group, (size_t)L->topk_group);
    if (ovr)
        for (int i = 0; i < ovr->n_disabled; i++)
            if (ovr->disabled[i] >= 0 && (size_t)ovr->disabled[i] < n) rank[ovr->disabled[i]] = -INFINITY;
    for (size_t e = 0; e < n; e++) idx[e] = (int32_t)e;
    sort_desc(idx, n, rank);
    size_t k = (size_t)top_k < n ? (size_t)top_k : n;
    int tie = 0;
    for (size_t i = 0; i + 1 < n && i < k; i++)
        if (tkey(rank[idx[i]]) == tkey(rank[idx[i + 1]])) tie = 1;
    if (ovr)
        for (int i = 0; i < ovr->n_forced; i++) {
            int32_t e = ovr->forced[i];
            if (e < 0 || (size_t)e >= n) continue;
            int present = 0;
            for (size_t j = 0; j < k; j++) present |= idx[j] == e;
            if (present) continue;
            if (k > 0) idx[k - 1] = e;
            else idx[k++] = e;
            sort_desc(idx, k, rank);
        }
    float z = -0.0f;
    for (size_t j = 0; j < k; j++) {
        float v = sc[idx[j]];
        w[j] = fmax_rs(v, 0.0f);
        z += w[j];
    }
    if (L->norm_topk) {
        z = fmax_rs(z, 1e-20f);
        for (size_t j = 0; j < k; j++) w[j] /= z;
    }
    for (size_t j = 0; j < k; j++) {
        w[j] *= L->routed_scale;
        sel[j] = idx[j];
    }
    return tie;
}

static size_t qt_bytes(const orc_qt *q) { return (size_t)q->rows * orc_row_bytes(q->dt, (size_t)q->cols); }

/* Router logits plus gating for `t` tokens: sel/w are [t, k].  Returns the
 * number of tokens with an exact tie in the selected prefix. */
int orc_route(const orc_layer *L, const orc_routing *ovr, const float *x, int t, int32_t *sel, float *w,
              float *logits_out) {
    size_t n = (size_t)L->n_experts;
    int top_k = (ovr && ovr->top_k > 0) ? ovr->top_k : L->top_k;
    size_t k = (size_t)top_k < n ? (size_t)top_k : n;
    float *logits = (float *)malloc((size_t)t * n * sizeof(float));
    matmul(&L->router, x, (size_t)t, logits);
    if (ovr && ovr->temp > 0.0f)
        for (size_t i = 0; i < (size_t)t * n; i++) logits[i] /= ovr->temp;
    if (logits_out) memcpy(logits_out, logits, (size_t)t * n * sizeof(float));
    float *rank = (float *)malloc(n * sizeof(float));
    int32_t *idx = (int32_t *)malloc(n * sizeof(int32_t));
    int ties = 0;
    for (int i = 0; i < t; i++)
        ties += route_token(L, ovr, top_k, logits + (size_t)i * n, rank, idx, sel + (size_t)i * k, w + (size_t)i * k);
    free(rank);
    free(idx);
    free(logits);
    return ties;
}

/* The whole routed layer, src/model.rs:841-971.
 *   out   [t, H]  overwritten with the layer's delta
 *   sel/w [t, k]  the routing table, strongest first (Route.experts)
 *   hits  [E+1]   hits[0] = count, then ascending experts with >= 1 token
 *   prev  [E+1]   the previous call's hits (same format) or NULL
 *   stats [4]     += routed, reused, expert_bytes, tie tokens
 * Returns k (experts per token) or a negative value on bad input. */
int orc_moe_forward(const orc_layer *L, const orc_routing *ovr, const float *x, int t, float *out, int32_t *sel,
                    float *w, uint32_t *hits, const uint32_t *prev, uint64_t *stats) {
    if (t <= 0 || L->n_experts <= 0) return -1;
    size_t h = (size_t)L->hidden, n = (size_t)L->n_experts;
    int top_k = (ovr && ovr->top_k > 0) ? ovr->top_k : L->top_k;
    size_t k = (size_t)top_k < n ? (size_t)top_k : n;
    memset(out, 0, (size_t)t * h * sizeof(float));
    int ties = orc_route(L, ovr, x, t, sel, w, NULL);

    /* Invert the table: tokens per expert in ascending token order. */
    size_t *cnt = (size_t *)calloc(n, sizeof(size_t));
    for (size_t i = 0; i < (size_t)t * k; i++) cnt[sel[i]]++;
    size_t *off = (size_t *)calloc(n + 1, sizeof(size_t));
    for (size_t e = 0; e < n; e++) off[e + 1] = off[e] + cnt[e];
    size_t *fill = (size_t *)calloc(n, sizeof(size_t));
    int32_t *tok = (int32_t *)malloc((size_t)t * k * sizeof(int32_t));
    float *tw = (float *)malloc((size_t)t * k * sizeof(float));
    for (size_t i = 0; i < (size_t)t; i++)
        for (size_t j = 0; j < k; j++) {
            int32_t e = sel[i * k + j];
            size_t p = off[e] + fill[e]++;
            tok[p] = (int32_t)i;
            tw[p] = w[i * k + j];
        }
    uint64_t routed = 0, reused = 0, bytes = 0;
    uint32_t nh = 0;
    for (size_t e = 0; e < n; e++) {
        if (!cnt[e]) continue;
        routed += cnt[e];
        int in_prev = 0;
        if (prev)
            for (uint32_t j = 0; j < prev[0]; j++) in_prev |= prev[1 + j] == (uint32_t)e;
        if (in_prev) reused += cnt[e];
        const orc_qt *ex = L->experts + 3 * e;
        bytes += qt_bytes(&ex[0]) + qt_bytes(&ex[1]) + qt_bytes(&ex[2]);
        if (hits) hits[1 + nh] = (uint32_t)e;
        nh++;
    }
    if (hits) hits[0] = nh;

    /* Experts over their tokens, then the combine in ascending expert order.
     * Each expert's matmuls spread their row bands over the whole pool (the
     * reference nests rayon's expert par_iter, join and bands under one
     * work-stealing pool; banding every matmul over all threads keeps every
     * core busy the same way, including at T=1 where only k experts run). */
    float *y = (float *)malloc((size_t)t * k * h * sizeof(float));
    for (size_t e = 0; e < n; e++) {
        if (!cnt[e]) continue;
        size_t ne = cnt[e];
        float *g = (float *)malloc(ne * h * sizeof(float));
        for (size_t s = 0; s < ne; s++) memcpy(g + s * h, x + (size_t)tok[off[e] + s] * h, h * sizeof(float));
        const orc_qt *ex = L->experts + 3 * e;
        mlp_forward(&ex[0], &ex[1], &ex[2], g, ne, y + off[e] * h);
        free(g);
    }
    for (size_t e = 0; e < n; e++)
        for (size_t s = 0; s < cnt[e]; s++) {
            size_t p = off[e] + s;
            float *o = out + (size_t)tok[p] * h;
            const float *yy = y + p * h;
            float wt = tw[p];
            for (size_t j = 0; j < h; j++) {
                float prod = wt * yy[j];
                o[j] += prod;
            }
        }
    free(y);

    if (L->shared) {
        float *ys = (float *)malloc((size_t)t * h * sizeof(float));
        mlp_forward(&L->shared[0], &L->shared[1], &L->shared[2], x, (size_t)t, ys);
        if (L->shared_gate) {
            float *gate = (float *)malloc((size_t)t * sizeof(float));
            matmul(L->shared_gate, x, (size_t)t, gate);
            for (size_t i = 0; i < (size_t)t; i++) {
                float den = 1.0f + expf(-gate[i]);
                float s = 1.0f / den;
                for (size_t j = 0; j < h; j++) ys[i * h + j] *= s;
            }
            free(gate);
        }
        for (size_t i = 0; i < (size_t)t * h; i++) out[i] += ys[i];
        free(ys);
    }
    if (stats) {
        stats[0] += routed;
        stats[1] += reused;
        stats[2] += bytes;
        stats[3] += (uint64_t)ties;
    }
    free(cnt);
    free(off);
    free(fill);
    free(tok);
    free(tw);
    return (int)k;
}

/* Plain SwiGLU MLP over t rows (a dense layer, src/model.rs:840, or one
 * expert on its own). */
void orc_mlp_forward(const orc_qt *gate, const orc_qt *up, const orc_qt *down, const float *x, int t, float *out) {
    mlp_forward(gate, up, down, x, (size_t)t, out);
}

float orc_expf(float x) { return expf(x); }
void orc_set_threads(int n) { omp_set_num_threads(n); }
int orc_max_threads(void) { return omp_get_max_threads(); }

/* expf over an array (host glibc), for checking the device port. */
void orc_expf_array(const float *x, float *y, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ======================================================= the model around it
 * The rest of the reference's forward (src/model.rs:646-834), restated so
 * that a whole model can run on the CPU path for the end-to-end checks:
 * RMSNorm, the rotary embedding with its context-extension schemes, and the
 * causal attention loop.  Projections reuse matmul, FFNs mlp_forward and
 * orc_moe_forward. */

/* src/model.rs:211-216: scale = 1 / sqrt(sum(v*v) / n + eps) (Rust's f32
 * Sum folds from -0.0 in order), out = v * scale * g.  `rows` rows of `n`
 * values, `xs` / `os` apart. */
void orc_rmsnorm_rows(const float *x, size_t rows, size_t n, size_t xs, const float *w, float eps, float *out,
                      size_t os) {
    for (size_t r = 0; r < rows; r++) {
        const float *v = x + r * xs;
        float *o = out + r * os;
        float ss = -0.0f;
        for (size_t i = 0; i < n; i++) {
            float sq = v[i] * v[i];
            ss += sq;
        }
        float mean = ss / (float)n;
        float den = sqrtf(mean + eps);
        float scale = 1.0f / den;
        for (size_t i = 0; i < n; i++) {
            float a = v[i] * scale;
            o[i] = a * w[i];
        }
    }
}

/* src/model.rs:324-333: rotate pairs (i, i + half) of x[0..dim) by pos * inv[i]
 * with f32 sin and cos (Rust's f32::sin_cos, glibc's sinf and cosf). */
static void rope1(float *x, size_t dim, float pos, const float *inv, size_t n_inv) {
    size_t half = dim / 2;
    for (size_t i = 0; i < n_inv && i < half; i++) {
        float ang = pos * inv[i];
        float s = sinf(ang), c = cosf(ang);
        float a = x[i], b = x[i + half];
        float ac = a * c, bs = b * s, as = a * s, bc = b * c;
        x[i] = ac - bs;
        x[i + half] = as + bc;
    }
}

/* The rotary embedding of `heads` heads (each `dim` values, `hs` apart,
 * starting `off` into the row) of `rows` rows `rs` apart; row r is at
 * position pos[r]. */
void orc_rope_rows(float *x, size_t rows, size_t rs, size_t heads, size_t hs, size_t off, size_t dim,
                   const int32_t *pos, const float *inv, size_t n_inv) {
    for (size_t r = 0; r < rows; r++)
        for (size_t h = 0; h < heads; h++) rope1(x + r * rs + h * hs + off, dim, (float)pos[r], inv, n_inv);
}

/* src/spec.rs:89-145: per-pair inverse frequencies for a head of head_dim
 * values.  kind: 0 none, 1 linear, 2 dynamic (NTK), 3 YaRN, 4 Llama 3. */
void orc_inv_freqs(int kind, float theta, float factor, size_t original_ctx, float low_freq_factor,
                   float high_freq_factor, float beta_fast, float beta_slow, size_t head_dim, float *out) {
    size_t half = head_dim / 2;
    float dim = (float)head_dim;
    float s = factor > 1e-6f ? factor : 1e-6f;
    float th = theta;
    if (kind == 2) {
        float d2 = dim - 2.0f;
        if (d2 < 1.0f) d2 = 1.0f;
        th = theta * powf(s, dim / d2);
    }
    for (size_t i = 0; i < half; i++) {
        float e = -2.0f * (float)i / dim;
        out[i] = powf(th, e);
    }
    if (kind == 1) {
        for (size_t i = 0; i < half; i++) out[i] = out[i] / s;
    } else if (kind == 4) {
        float l = (float)original_ctx;
        float lo_wave = l / low_freq_factor, hi_wave = l / high_freq_factor;
        float span = high_freq_factor - low_freq_factor;
        if (span < 1e-6f) span = 1e-6f;
        for (size_t i = 0; i < half; i++) {
            float f = out[i];
            float wave = 2.0f * 3.14159265358979323846f / f;
            if (wave > lo_wave) {
                out[i] = f / s;
            } else if (wave < hi_wave) {
                out[i] = f;
            } else {
                float t = ((l / wave) - low_freq_factor) / span;
                float a = (1.0f - t) * f / s;
                float b = t * f;
                out[i] = a + b;
            }
        }
    } else if (kind == 3) {
        float l = (float)original_ctx;
        float ln_base = logf(theta);
        if (ln_base < 1e-6f) ln_base = 1e-6f;
        float twopi = 2.0f * 3.14159265358979323846f;
        float bf = dim * logf(l / (beta_fast * twopi)) / (2.0f * ln_base);
        float bs = dim * logf(l / (beta_slow * twopi)) / (2.0f * ln_base);
        float low = floorf(bf), high = ceilf(bs);
        float span = high - low;
        if (span < 1e-3f) span = 1e-3f;
        for (size_t i = 0; i < half; i++) {
            float f = out[i];
            float ramp = ((float)i - low) / span;
            ramp = ramp < 0.0f ? 0.0f : (ramp > 1.0f ? 1.0f : ramp);
            float a = (1.0f - ramp) * (f / s);
            float b = ramp * f;
            out[i] = a + b;
        }
    }
}

/* src/spec.rs:64-70, 147-160: the attention-scale multiplier (YaRN only). */
static float yarn_mscale(float scale, float mscale) { return scale <= 1.0f ? 1.0f : 0.1f * mscale * logf(scale) + 1.0f; }
float orc_attn_scale(int kind, float factor, float mscale, float mscale_all_dim, float attn_factor) {
    if (kind != 3) return 1.0f;
    if (mscale > 0.0f || mscale_all_dim > 0.0f) {
        float num = yarn_mscale(factor, mscale), den = yarn_mscale(factor, mscale_all_dim);
        if (den < 1e-6f) den = 1e-6f;
        return num / den * attn_factor;
    }
    return yarn_mscale(factor, 1.0f) * attn_factor;
}

/* src/model.rs:797-831: causal scaled dot-product attention of t tokens at
 * positions base .. base + t - 1 against the cache (rows of kd keys and vdim
 * values per position; head h of a key is kd values [kvh * qd, +qd)).  Per
 * (token, head): scores = dot(q, k_j) * scale for j in [lo, p] (lo = p + 1 -
 * window for a windowed layer), softmax, then acc += w * v_j in position
 * order from +0.  q is [t, heads * qd], out [t, heads * vd]. */
void orc_attention(const float *q, const float *kc, const float *vc, size_t t, size_t base, size_t heads, size_t n_kv,
                   size_t qd, size_t vd, float scale, size_t window, float *out) {
    size_t kd = n_kv * qd, vdim = n_kv * vd;
    size_t rep = heads / (n_kv > 0 ? n_kv : 1);
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t idx = 0; idx < t * heads; idx++) {
        size_t i = idx / heads, hi = idx % heads, p = base + i;
        size_t lo = window ? (p + 1 > window ? p + 1 - window : 0) : 0;
        size_t kvh = rep > 1 ? hi / rep : (hi < n_kv - 1 ? hi : n_kv - 1);
        const float *qv = q + i * heads * qd + hi * qd;
        size_t n = p + 1 - lo;
        float *sc = (float *)malloc(n * sizeof(float));
        for (size_t j = lo; j <= p; j++) {
            float d = orc_dot(qv, kc + j * kd + kvh * qd, qd);
            sc[j - lo] = d * scale;
        }
        softmax(sc, n);
        float *acc = out + i * heads * vd + hi * vd;
        for (size_t c = 0; c < vd; c++) acc[c] = 0.0f;
        for (size_t k = 0; k < n; k++) {
            const float *vj = vc + (lo + k) * vdim + kvh * vd;
            float w = sc[k];
            for (size_t c = 0; c < vd; c++) {
                float prod = w * vj[c];
                acc[c] += prod;
            }
        }
        free(sc);
    }
}
