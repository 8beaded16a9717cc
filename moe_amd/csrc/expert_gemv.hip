// expert_gemv.hip — SwiGLU experts over few tokens per expert (decode).
//
// Two families:
//  * fast GEMV: weights stream from HBM once; a thread owns one 64-value
//    unit (two 32-value blocks) of a row, dequantises it in registers and
//    dots it with activations it keeps in registers.  Lanes that share a row
//    sum through shuffles; when a row is wider than one wavefront's 64 units
//    (KS = 2 or 4 waves per row) the waves' partial sums meet in LDS.  Each
//    thread issues the loads of several rows before computing any of them.
//    fp32 throughout, weights exact (d * q is exact in f32), so results
//    differ from the reference only by summation order.  For small T the down
//    projection also performs the combine (ascending expert order from +0,
//    separate multiply and add, src/model.rs:936-942), the shared expert
//    (src/model.rs:956-970) and the residual add (src/model.rs:680-683).
//  * exact GEMV: one thread per (row, token) computing the reference's dot
//    (src/quant.rs:386-420) in its exact lane and reduction order over the
//    exactly dequantised row (src/quant.rs:177-227), and SwiGLU with glibc's
//    expf (src/model.rs:31-33).  Bit-identical to the CPU path; used where a
//    shape does not fit the fast path (rows not 4-byte aligned, widths not a
//    multiple of 64, F32 experts) and for the bit-exact parity mode.
//
// Work list: task y < hits[0] is the routed expert hits[1 + y] over its
// tokens (permuted rows offsets[e] .. offsets[e] + counts[e]); task
// task_bound is the shared expert over all T tokens.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "exact_math.h"
#include "moe_internal.h"

namespace moe {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ inline float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)(bits & 0xffff))); }
__device__ inline uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t s) { return __builtin_amdgcn_alignbyte(hi, lo, s); }
__device__ inline float ub(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xffu); }

// Bits 0..3 of h moved to bit 4 of bytes 0..3.
__device__ inline uint32_t spread4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

// The group a task works on.
struct Task {
    int g;        // expert index (E = shared)
    int n;        // tokens
    int row0;     // first permuted row in h / y
    bool shared;
};
__device__ inline bool task_of(const GemvArgs &a, int y, Task &tk) {
    if (a.has_shared && y == a.task_bound) {
        tk.g = a.E, tk.n = a.T, tk.row0 = 0, tk.shared = true;
        return true;
    }
    if (y >= a.hits[0]) return false;
    const int e = a.hits[1 + y];
    tk.g = e, tk.n = a.counts[e], tk.row0 = a.offsets[e], tk.shared = false;
    return true;
}

// ---------------------------------------------------------------- fast path

// A 64-value unit: two blocks, 4-byte aligned.  Q4_0 36 bytes, Q5_0 44,
// Q8_0 68.
template <int DT>
struct Unit;
template <>
struct Unit<MOE_DT_Q4_0> {
    static constexpr int dw = 9, bytes = 36;
};
template <>
struct Unit<MOE_DT_Q5_0> {
    static constexpr int dw = 11, bytes = 44;
};
template <>
struct Unit<MOE_DT_Q8_0> {
    static constexpr int dw = 17, bytes = 68;
};

template <int DT>
__device__ inline void load_unit(const uint8_t *p, uint32_t (&d)[Unit<DT>::dw]) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p, 4));
    constexpr int N = Unit<DT>::dw;
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        u32x4 v = *reinterpret_cast<const u32x4 *>(q + i);
        d[i] = v.x, d[i + 1] = v.y, d[i + 2] = v.z, d[i + 3] = v.w;
    }
#pragma unroll
    for (int i = N & ~3; i < N; i++) d[i] = q[i];
}

// Dot of a loaded unit with NT activation vectors.  `sx` holds the per-block
// sums of the activations, which absorb the format's zero offset:
// sum((q - o) x) = sum(q x) - o sum(x) with q read unsigned.
template <int DT, int NT>
__device__ inline void dot_unit(const uint32_t (&d)[Unit<DT>::dw], const float (&xv)[NT][64],
                                const float (&sx)[NT][2], float (&acc)[NT]) {
    if constexpr (DT == MOE_DT_Q4_0) {
        // [dA qA0..15][dB qB0..15]
        const float sa = h2f(d[0]), sb = h2f(d[4] >> 16);
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qa[i] = alignb(d[i + 1], d[i], 2), qb[i] = d[5 + i];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float pa0 = 0.0f, pa1 = 0.0f, pb0 = 0.0f, pb1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t la = qa[i] & 0x0f0f0f0fu, ha = (qa[i] >> 4) & 0x0f0f0f0fu;
                const uint32_t lb = qb[i] & 0x0f0f0f0fu, hb = (qb[i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    pa0 = fmaf(ub(la, b), xv[t][4 * i + b], pa0);
                    pa1 = fmaf(ub(ha, b), xv[t][16 + 4 * i + b], pa1);
                    pb0 = fmaf(ub(lb, b), xv[t][32 + 4 * i + b], pb0);
                    pb1 = fmaf(ub(hb, b), xv[t][48 + 4 * i + b], pb1);
                }
            }
            acc[t] = fmaf(sa, (pa0 + pa1) - 8.0f * sx[t][0], acc[t]);
            acc[t] = fmaf(sb, (pb0 + pb1) - 8.0f * sx[t][1], acc[t]);
        }
    } else if constexpr (DT == MOE_DT_Q5_0) {
        // [dA hA(4) qA0..15][dB hB(4) qB0..15]
        const float sa = h2f(d[0]), sb = h2f(d[5] >> 16);
        const uint32_t ha = alignb(d[1], d[0], 2), hb = d[6];
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qa[i] = alignb(d[i + 2], d[i + 1], 2), qb[i] = d[7 + i];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float pa0 = 0.0f, pa1 = 0.0f, pb0 = 0.0f, pb1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t la = (qa[i] & 0x0f0f0f0fu) | spread4((ha >> (4 * i)) & 0xfu);
                const uint32_t xa = ((qa[i] >> 4) & 0x0f0f0f0fu) | spread4((ha >> (16 + 4 * i)) & 0xfu);
                const uint32_t lb = (qb[i] & 0x0f0f0f0fu) | spread4((hb >> (4 * i)) & 0xfu);
                const uint32_t xb = ((qb[i] >> 4) & 0x0f0f0f0fu) | spread4((hb >> (16 + 4 * i)) & 0xfu);
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    pa0 = fmaf(ub(la, b), xv[t][4 * i + b], pa0);
                    pa1 = fmaf(ub(xa, b), xv[t][16 + 4 * i + b], pa1);
                    pb0 = fmaf(ub(lb, b), xv[t][32 + 4 * i + b], pb0);
                    pb1 = fmaf(ub(xb, b), xv[t][48 + 4 * i + b], pb1);
                }
            }
            acc[t] = fmaf(sa, (pa0 + pa1) - 16.0f * sx[t][0], acc[t]);
            acc[t] = fmaf(sb, (pb0 + pb1) - 16.0f * sx[t][1], acc[t]);
        }
    } else {  // Q8_0: [dA qA0..31][dB qB0..31]
        const float sa = h2f(d[0]), sb = h2f(d[8] >> 16);
        uint32_t qa[8], qb[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // int8 -> uint8 + 128, absorbed by the block sums below.
            qa[i] = alignb(d[i + 1], d[i], 2) ^ 0x80808080u;
            qb[i] = d[9 + i] ^ 0x80808080u;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float pa0 = 0.0f, pa1 = 0.0f, pb0 = 0.0f, pb1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    pa0 = fmaf(ub(qa[i], b), xv[t][4 * i + b], pa0);
                    pa1 = fmaf(ub(qa[4 + i], b), xv[t][16 + 4 * i + b], pa1);
                    pb0 = fmaf(ub(qb[i], b), xv[t][32 + 4 * i + b], pb0);
                    pb1 = fmaf(ub(qb[4 + i], b), xv[t][48 + 4 * i + b], pb1);
                }
            }
            acc[t] = fmaf(sa, (pa0 + pa1) - 128.0f * sx[t][0], acc[t]);
            acc[t] = fmaf(sb, (pb0 + pb1) - 128.0f * sx[t][1], acc[t]);
        }
    }
}

// Thread placement for a matrix of `units` 64-value units per row: CG lanes
// of a wave share a row slice (CG >= units when KS == 1), KS waves share a
// row (KS > 1: CG = 64 and wave kw owns units kw*64 .. kw*64+63).  NS row
// slots work side by side.
struct Map {
    int cg, ks, ns, slot, kw, c, u, set;
};
__device__ inline Map map_of(int cg, int ks) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    Map m;
    m.cg = cg, m.ks = ks;
    m.kw = wv % ks;
    m.set = wv / ks;                     // which wave set (ks > 1)
    m.ns = (4 / ks) * (64 / cg);
    m.slot = m.set * (64 / cg) + lane / cg;
    m.c = lane % cg;
    m.u = m.kw * 64 + m.c;
    return m;
}
__device__ inline float sum_cg(float v, int cg) {
    for (int m = cg >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Activations of unit u for NT rows (null rows read as zero), and their
// per-block sums.
template <int NT>
__device__ inline void load_acts(const float *const (&src)[NT], int u, int units, float (&xv)[NT][64],
                                 float (&sx)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (u < units && src[t]) {
            const float4 *s4 = reinterpret_cast<const float4 *>(src[t] + 64 * u);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 v = s4[i];
                xv[t][4 * i] = v.x, xv[t][4 * i + 1] = v.y, xv[t][4 * i + 2] = v.z, xv[t][4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 64; i++) xv[t][i] = 0.0f;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) s0 += xv[t][i], s1 += xv[t][32 + i];
        sx[t][0] = s0, sx[t][1] = s1;
    }
}

// Copy n floats to LDS with the whole block (n a multiple of 4).
__device__ inline void stage_rows(const float *__restrict__ src, float *dst, int n) {
    const float4 *s4 = reinterpret_cast<const float4 *>(src);
    float4 *d4 = reinterpret_cast<float4 *>(dst);
    for (int i = threadIdx.x; i < n / 4; i += 256) d4[i] = s4[i];
}

// The activation rows of a task's token chunk [t0, t0 + NT): pointers to
// global memory, or to LDS copies when several wave sets read them.
template <int NT, bool UP>
__device__ inline void task_rows(const GemvArgs &a, const Task &tk, int t0, bool stage, float *act, int cols,
                                 const float *(&src)[NT], int (&rowid)[NT]) {
    const int Icol = tk.shared ? a.I_s : a.I;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int i = t0 + t;
        rowid[t] = i < tk.n ? tk.row0 + i : -1;
        const float *g = nullptr;
        if (rowid[t] >= 0) {
            if (UP) {
                const int tok = tk.shared ? i : a.perm_tok[rowid[t]];
                g = a.x + (size_t)tok * a.H;
            } else {
                g = (tk.shared ? a.hs : a.h) + (size_t)rowid[t] * Icol;
            }
        }
        src[t] = g;
    }
    if (stage) {
        __syncthreads();  // the previous chunk's LDS copy is no longer read
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (src[t]) stage_rows(src[t], act + (size_t)t * cols, cols);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (src[t]) src[t] = act + (size_t)t * cols;
    }
}

// gate/up + SwiGLU: h[row][r] = silu(gate_r . x) * (up_r . x) for the rows
// [blockIdx.x * rows_per_block, +rows_per_block) of one task.
template <int DT, int NT, int RPS>
__global__ __launch_bounds__(256) void gemv_up_kernel(GemvArgs a, int cg, int ks, int rows_per_block,
                                                      int shared_only) {
    extern __shared__ float act[];
    __shared__ float red[2 * RPS * NT * 2 * 4];  // [set][i][t][gate/up][kw]
    Task tk;
    if (!task_of(a, shared_only ? a.task_bound : (int)blockIdx.y, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &G = ex.m[0], &U = ex.m[1];
    const int rows = G.rows, units = G.cols / 64;
    const int r_begin = blockIdx.x * rows_per_block;
    if (r_begin >= rows) return;
    const int r_end = min(rows, r_begin + rows_per_block);
    const Map m = map_of(cg, ks);
    const int Icol = tk.shared ? a.I_s : a.I;
    float *hout = tk.shared ? a.hs : a.h;
    constexpr int DW = Unit<DT>::dw, UB = Unit<DT>::bytes;
    for (int t0 = 0; t0 < tk.n; t0 += NT) {
        const float *src[NT];
        int rowid[NT];
        task_rows<NT, true>(a, tk, t0, ks < 4, act, G.cols, src, rowid);
        float xv[NT][64], sx[NT][2];
        load_acts<NT>(src, m.u, units, xv, sx);
        for (int rb = r_begin; rb < r_end; rb += m.ns * RPS) {
            uint32_t rg[RPS][DW], ru[RPS][DW];
#pragma unroll
            for (int i = 0; i < RPS; i++) {
                const int r = rb + m.slot + i * m.ns;
                if (r < r_end && m.u < units) {
                    load_unit<DT>(G.ptr + (size_t)r * G.stride + (size_t)m.u * UB, rg[i]);
                    load_unit<DT>(U.ptr + (size_t)r * U.stride + (size_t)m.u * UB, ru[i]);
                }
            }
            float pg[RPS][NT], pu[RPS][NT];
#pragma unroll
            for (int i = 0; i < RPS; i++) {
#pragma unroll
                for (int t = 0; t < NT; t++) pg[i][t] = 0.0f, pu[i][t] = 0.0f;
                const int r = rb + m.slot + i * m.ns;
                if (r < r_end && m.u < units) {
                    dot_unit<DT, NT>(rg[i], xv, sx, pg[i]);
                    dot_unit<DT, NT>(ru[i], xv, sx, pu[i]);
                }
#pragma unroll
                for (int t = 0; t < NT; t++) pg[i][t] = sum_cg(pg[i][t], cg), pu[i][t] = sum_cg(pu[i][t], cg);
            }
            if (ks == 1) {
                if (m.c == 0) {
#pragma unroll
                    for (int i = 0; i < RPS; i++) {
                        const int r = rb + m.slot + i * m.ns;
                        if (r >= r_end) continue;
#pragma unroll
                        for (int t = 0; t < NT; t++)
                            if (rowid[t] >= 0) {
                                const float g = pg[i][t];
                                hout[(size_t)rowid[t] * Icol + r] = (g / (1.0f + __expf(-g))) * pu[i][t];
                            }
                    }
                }
            } else {
                if (m.c == 0) {
#pragma unroll
                    for (int i = 0; i < RPS; i++)
#pragma unroll
                        for (int t = 0; t < NT; t++) {
                            const int base = ((m.set * RPS + i) * NT + t) * 2;
                            red[(base + 0) * 4 + m.kw] = pg[i][t];
                            red[(base + 1) * 4 + m.kw] = pu[i][t];
                        }
                }
                __syncthreads();
                const int sets = 4 / ks;
                for (int q = threadIdx.x; q < sets * RPS * NT; q += 256) {
                    const int t = q % NT, i = (q / NT) % RPS, set = q / (NT * RPS);
                    const int r = rb + set + i * m.ns;
                    if (r >= r_end || rowid[t] < 0) continue;
                    const int base = ((set * RPS + i) * NT + t) * 2;
                    float g = 0.0f, u = 0.0f;
                    for (int w = 0; w < ks; w++) g += red[base * 4 + w], u += red[(base + 1) * 4 + w];
                    hout[(size_t)rowid[t] * Icol + r] = (g / (1.0f + __expf(-g))) * u;
                }
                __syncthreads();
            }
        }
    }
}

// down: y[row][j] = down_j . h[row] (the unfused form, for larger T).
template <int DT, int NT, int RPS>
__global__ __launch_bounds__(256) void gemv_down_kernel(GemvArgs a, int cg, int ks, int rows_per_block,
                                                        int shared_only) {
    extern __shared__ float act[];
    __shared__ float red[2 * RPS * NT * 4];
    Task tk;
    if (!task_of(a, shared_only ? a.task_bound : (int)blockIdx.y, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &D = ex.m[2];
    const int rows = D.rows, units = D.cols / 64;
    const int r_begin = blockIdx.x * rows_per_block;
    if (r_begin >= rows) return;
    const int r_end = min(rows, r_begin + rows_per_block);
    const Map m = map_of(cg, ks);
    float *yout = tk.shared ? a.ys : a.y;
    constexpr int DW = Unit<DT>::dw, UB = Unit<DT>::bytes;
    for (int t0 = 0; t0 < tk.n; t0 += NT) {
        const float *src[NT];
        int rowid[NT];
        task_rows<NT, false>(a, tk, t0, ks < 4, act, D.cols, src, rowid);
        float xv[NT][64], sx[NT][2];
        load_acts<NT>(src, m.u, units, xv, sx);
        for (int rb = r_begin; rb < r_end; rb += m.ns * RPS) {
            uint32_t rw[RPS][DW];
#pragma unroll
            for (int i = 0; i < RPS; i++) {
                const int r = rb + m.slot + i * m.ns;
                if (r < r_end && m.u < units) load_unit<DT>(D.ptr + (size_t)r * D.stride + (size_t)m.u * UB, rw[i]);
            }
            float py[RPS][NT];
#pragma unroll
            for (int i = 0; i < RPS; i++) {
#pragma unroll
                for (int t = 0; t < NT; t++) py[i][t] = 0.0f;
                const int r = rb + m.slot + i * m.ns;
                if (r < r_end && m.u < units) dot_unit<DT, NT>(rw[i], xv, sx, py[i]);
#pragma unroll
                for (int t = 0; t < NT; t++) py[i][t] = sum_cg(py[i][t], cg);
            }
            if (ks == 1) {
                if (m.c == 0) {
#pragma unroll
                    for (int i = 0; i < RPS; i++) {
                        const int r = rb + m.slot + i * m.ns;
                        if (r >= r_end) continue;
#pragma unroll
                        for (int t = 0; t < NT; t++)
                            if (rowid[t] >= 0) yout[(size_t)rowid[t] * a.H + r] = py[i][t];
                    }
                }
            } else {
                if (m.c == 0) {
#pragma unroll
                    for (int i = 0; i < RPS; i++)
#pragma unroll
                        for (int t = 0; t < NT; t++) red[((m.set * RPS + i) * NT + t) * 4 + m.kw] = py[i][t];
                }
                __syncthreads();
                const int sets = 4 / ks;
                for (int q = threadIdx.x; q < sets * RPS * NT; q += 256) {
                    const int t = q % NT, i = (q / NT) % RPS, set = q / (NT * RPS);
                    const int r = rb + set + i * m.ns;
                    if (r >= r_end || rowid[t] < 0) continue;
                    float v = 0.0f;
                    for (int w = 0; w < ks; w++) v += red[((set * RPS + i) * NT + t) * 4 + w];
                    yout[(size_t)rowid[t] * a.H + r] = v;
                }
                __syncthreads();
            }
        }
    }
}

// down + combine for T <= kFusedMaxT: a block owns output rows [j0, j0 + RPB)
// of every token and walks the tasks in order — routed experts ascending
// (mode 0), or the shared expert alone (mode 1, after mode 0) — adding
// w * y into an LDS accumulator that starts at +0 (mode 0) or at out
// (mode 1).  Each (row, token) has one writer per task, and tasks are
// separated by barriers, so every sum runs in the reference's order.
template <int DT, int NT, int RPS>
__global__ __launch_bounds__(256) void gemv_down_combine_kernel(GemvArgs a, int cg, int ks, int rows_per_block,
                                                                int mode, int finish) {
    extern __shared__ float act[];
    __shared__ float red[2 * RPS * NT * 4];
    __shared__ float accum[64 * kFusedMaxT];  // [row - j0][token]
    const int j0 = blockIdx.x * rows_per_block;
    const int H = a.H;
    if (j0 >= H) return;
    const int j1 = min(H, j0 + rows_per_block);
    const Map m = map_of(cg, ks);
    for (int q = threadIdx.x; q < (j1 - j0) * a.T; q += 256) {
        const int jr = q / a.T, t = q % a.T;
        accum[jr * kFusedMaxT + t] = mode == 0 ? 0.0f : a.out[(size_t)t * H + j0 + jr];
    }
    __syncthreads();
    const int ntasks = mode == 0 ? a.hits[0] : 1;
    constexpr int DW = Unit<DT>::dw, UB = Unit<DT>::bytes;
    for (int y = 0; y < ntasks; y++) {
        Task tk;
        task_of(a, mode == 0 ? y : a.task_bound, tk);
        const MatDev &D = a.experts[tk.g].m[2];
        const int units = D.cols / 64;
        for (int t0 = 0; t0 < tk.n; t0 += NT) {
            const float *src[NT];
            int rowid[NT];
            task_rows<NT, false>(a, tk, t0, ks < 4, act, D.cols, src, rowid);
            int tok[NT];
            float wt[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) {
                tok[t] = -1, wt[t] = 0.0f;
                if (rowid[t] >= 0) {
                    if (tk.shared) {
                        tok[t] = t0 + t;
                        wt[t] = a.shgate ? a.shgate[tok[t]] : 1.0f;
                    } else {
                        tok[t] = a.perm_tok[rowid[t]];
                        wt[t] = a.perm_w[rowid[t]];
                    }
                }
            }
            float xv[NT][64], sx[NT][2];
            load_acts<NT>(src, m.u, units, xv, sx);
            for (int rb = j0; rb < j1; rb += m.ns * RPS) {
                uint32_t rw[RPS][DW];
#pragma unroll
                for (int i = 0; i < RPS; i++) {
                    const int r = rb + m.slot + i * m.ns;
                    if (r < j1 && m.u < units) load_unit<DT>(D.ptr + (size_t)r * D.stride + (size_t)m.u * UB, rw[i]);
                }
                float py[RPS][NT];
#pragma unroll
                for (int i = 0; i < RPS; i++) {
#pragma unroll
                    for (int t = 0; t < NT; t++) py[i][t] = 0.0f;
                    const int r = rb + m.slot + i * m.ns;
                    if (r < j1 && m.u < units) dot_unit<DT, NT>(rw[i], xv, sx, py[i]);
#pragma unroll
                    for (int t = 0; t < NT; t++) py[i][t] = sum_cg(py[i][t], cg);
                }
                if (ks == 1) {
                    if (m.c == 0) {
#pragma unroll
                        for (int i = 0; i < RPS; i++) {
                            const int r = rb + m.slot + i * m.ns;
                            if (r >= j1) continue;
#pragma unroll
                            for (int t = 0; t < NT; t++)
                                if (tok[t] >= 0) {
                                    float &cell = accum[(r - j0) * kFusedMaxT + tok[t]];
                                    const float prod = wt[t] * py[i][t];
                                    cell = cell + prod;
                                }
                        }
                    }
                } else {
                    if (m.c == 0) {
#pragma unroll
                        for (int i = 0; i < RPS; i++)
#pragma unroll
                            for (int t = 0; t < NT; t++) red[((m.set * RPS + i) * NT + t) * 4 + m.kw] = py[i][t];
                    }
                    __syncthreads();
                    const int sets = 4 / ks;
                    for (int q = threadIdx.x; q < sets * RPS * NT; q += 256) {
                        const int t = q % NT, i = (q / NT) % RPS, set = q / (NT * RPS);
                        const int r = rb + set + i * m.ns;
                        if (r >= j1 || tok[t] < 0) continue;
                        float v = 0.0f;
                        for (int w = 0; w < ks; w++) v += red[((set * RPS + i) * NT + t) * 4 + w];
                        float &cell = accum[(r - j0) * kFusedMaxT + tok[t]];
                        const float prod = wt[t] * v;
                        cell = cell + prod;
                    }
                    __syncthreads();
                }
            }
        }
        __syncthreads();  // next task's adds come after this one's
    }
    for (int q = threadIdx.x; q < (j1 - j0) * a.T; q += 256) {
        const int jr = q / a.T, t = q % a.T;
        const float v = accum[jr * kFusedMaxT + t];
        a.out[(size_t)t * H + j0 + jr] = v;
        if (finish && a.residual) a.residual[(size_t)t * H + j0 + jr] = a.residual[(size_t)t * H + j0 + jr] + v;
    }
}

// --------------------------------------------------------------- exact path

__device__ inline uint32_t ld_u16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Value c of a row, exactly as dequant produces it (src/quant.rs:177-227).
__device__ inline float wval(const uint8_t *row, int dt, int c) {
    const int b = c >> 5, i = c & 31;
    switch (dt) {
    case MOE_DT_F32: {
        const uint8_t *p = row + 4 * (size_t)c;
        return __uint_as_float(ld_u16(p) | (ld_u16(p + 2) << 16));
    }
    case MOE_DT_Q8_0: {
        const uint8_t *blk = row + 34 * (size_t)b;
        return h2f(ld_u16(blk)) * (float)(int8_t)blk[2 + i];
    }
    case MOE_DT_Q4_0: {
        const uint8_t *blk = row + 18 * (size_t)b;
        const uint32_t v = blk[2 + (i & 15)];
        const int nib = i < 16 ? (int)(v & 15) : (int)(v >> 4);
        return h2f(ld_u16(blk)) * (float)(nib - 8);
    }
    default: {  // Q5_0
        const uint8_t *blk = row + 22 * (size_t)b;
        const uint32_t v = blk[6 + (i & 15)];
        const int nib = i < 16 ? (int)(v & 15) : (int)(v >> 4);
        const int hb = (blk[2 + i / 8] >> (i % 8)) & 1;
        return h2f(ld_u16(blk)) * (float)((nib | (hb << 4)) - 16);
    }
    }
}

// dot_avx2's order over a dequantised row and an f32 vector.
__device__ inline float dot_exact(const uint8_t *row, int dt, const float *xv, int n) {
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;
    int i = 0;
    for (; i + 16 <= n; i += 16)
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = fmaf(wval(row, dt, i + j), xv[i + j], acc[j]);
    for (; i + 8 <= n; i += 8)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = fmaf(wval(row, dt, i + j), xv[i + j], acc[j]);
    float s[8], q[4];
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = acc[j] + acc[j + 8];
#pragma unroll
    for (int j = 0; j < 4; j++) q[j] = s[j + 4] + s[j];
    float out = (q[0] + q[1]) + (q[2] + q[3]);
    for (; i < n; i++) {
        float p = wval(row, dt, i) * xv[i];
        out += p;
    }
    return out;
}

// Exact gate+up+SwiGLU: thread per (row r, token slot i).
__global__ __launch_bounds__(256) void gemv_up_exact_kernel(GemvArgs a) {
    Task tk;
    if (!task_of(a, blockIdx.y, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &G = ex.m[0], &U = ex.m[1];
    const int rows = G.rows;
    const int Icol = tk.shared ? a.I_s : a.I;
    float *hout = tk.shared ? a.hs : a.h;
    const long long n = (long long)rows * tk.n;
    for (long long q = (long long)blockIdx.x * 256 + threadIdx.x; q < n; q += (long long)gridDim.x * 256) {
        const int r = (int)(q % rows), i = (int)(q / rows);
        const int tok = tk.shared ? i : a.perm_tok[tk.row0 + i];
        const float *xv = a.x + (size_t)tok * a.H;
        const float g = dot_exact(G.ptr + (size_t)r * G.stride, G.dt, xv, G.cols);
        const float u = dot_exact(U.ptr + (size_t)r * U.stride, U.dt, xv, U.cols);
        const float ng = -g;
        const float den = 1.0f + expf_exact(ng);
        const float sg = g / den;
        hout[(size_t)(tk.row0 + i) * Icol + r] = sg * u;
    }
}

__global__ __launch_bounds__(256) void gemv_down_exact_kernel(GemvArgs a) {
    Task tk;
    if (!task_of(a, blockIdx.y, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &D = ex.m[2];
    const int rows = D.rows;
    const int Icol = tk.shared ? a.I_s : a.I;
    const float *hin = tk.shared ? a.hs : a.h;
    float *yout = tk.shared ? a.ys : a.y;
    const long long n = (long long)rows * tk.n;
    for (long long q = (long long)blockIdx.x * 256 + threadIdx.x; q < n; q += (long long)gridDim.x * 256) {
        const int r = (int)(q % rows), i = (int)(q / rows);
        const float *hv = hin + (size_t)(tk.row0 + i) * Icol;
        yout[(size_t)(tk.row0 + i) * a.H + r] = dot_exact(D.ptr + (size_t)r * D.stride, D.dt, hv, D.cols);
    }
}


// --------------------------------------------------------------- launchers

struct Plan {
    int cg, ks, rps_rows;  // lanes per row slice, waves per row, rows per slot per batch
};
Plan plan_for(int cols) {
    const int units = cols / 64;
    Plan p;
    if (units <= 64) {
        p.ks = 1;
        p.cg = 16;
        while (p.cg < units) p.cg <<= 1;
    } else {
        p.ks = units <= 128 ? 2 : 4;
        p.cg = 64;
    }
    p.rps_rows = 0;
    return p;
}
int slots_of(const Plan &p) { return (4 / p.ks) * (64 / p.cg); }

// Rows per slot per batch: as many weight units in flight per thread as
// the register file allows (two token columns double the activations).
template <int DT, int NT>
constexpr int rps_of() {
    return (DT == MOE_DT_Q8_0 ? 2 : 4) / NT;
}

enum Kind { kUp, kDown, kDownCombine };

template <int DT, int NT>
hipError_t launch_kind(Kind kind, dim3 grid, size_t lds, const GemvArgs &a, const Plan &p, int rpb, int x1, int x2,
                       hipStream_t s) {
    constexpr int R = rps_of<DT, NT>();
    switch (kind) {
    case kUp: hipLaunchKernelGGL((gemv_up_kernel<DT, NT, R>), grid, dim3(256), lds, s, a, p.cg, p.ks, rpb, x1); break;
    case kDown: hipLaunchKernelGGL((gemv_down_kernel<DT, NT, R>), grid, dim3(256), lds, s, a, p.cg, p.ks, rpb, x1); break;
    case kDownCombine:
        hipLaunchKernelGGL((gemv_down_combine_kernel<DT, NT, R>), grid, dim3(256), lds, s, a, p.cg, p.ks, rpb, x1, x2);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_any(int dt, bool two, Kind kind, dim3 grid, size_t lds, const GemvArgs &a, const Plan &p, int rpb,
                      int x1, int x2, hipStream_t s) {
    switch (dt) {
    case MOE_DT_Q4_0:
        return two ? launch_kind<MOE_DT_Q4_0, 2>(kind, grid, lds, a, p, rpb, x1, x2, s)
                   : launch_kind<MOE_DT_Q4_0, 1>(kind, grid, lds, a, p, rpb, x1, x2, s);
    case MOE_DT_Q5_0:
        return two ? launch_kind<MOE_DT_Q5_0, 2>(kind, grid, lds, a, p, rpb, x1, x2, s)
                   : launch_kind<MOE_DT_Q5_0, 1>(kind, grid, lds, a, p, rpb, x1, x2, s);
    case MOE_DT_Q8_0:
        return two ? launch_kind<MOE_DT_Q8_0, 2>(kind, grid, lds, a, p, rpb, x1, x2, s)
                   : launch_kind<MOE_DT_Q8_0, 1>(kind, grid, lds, a, p, rpb, x1, x2, s);
    default: return hipErrorInvalidValue;
    }
}

int rps_rows(int dt, int nt) { return (dt == MOE_DT_Q8_0 ? 2 : 4) / nt; }

// Rows per block for `tasks` tasks of `rows` rows: about two blocks per CU
// in all, a whole number of batches each.
int rows_per_block(int rows, int tasks, int batch) {
    long long want = 512;
    int rpb = batch;
    while ((long long)((rows + 2 * rpb - 1) / (2 * rpb)) * tasks >= want && 2 * rpb <= rows) rpb *= 2;
    return rpb;
}

hipError_t gemv_launch(Kind kind, const GemvArgs &a, const ExpertDev &ex, bool shared_only, hipStream_t s) {
    const MatDev &m = kind == kUp ? ex.m[0] : ex.m[2];
    const Plan p = plan_for(m.cols);
    const bool two = a.T > 1;
    const int NT = two ? 2 : 1;
    const size_t lds = p.ks < 4 ? (size_t)NT * m.cols * 4 : 0;
    const int batch = slots_of(p) * rps_rows(m.dt, NT);
    if (kind == kDownCombine) {
        // Output rows per block: about one block per CU (the block walks
        // every task, so the grid has no task dimension).
        const int rpb = std::max(4, std::min(64, a.H / 256));
        dim3 grid((a.H + rpb - 1) / rpb);
        return launch_any(m.dt, two, kind, grid, lds, a, p, rpb, shared_only ? 1 : 0,
                          (shared_only || !a.has_shared) ? 1 : 0, s);
    }
    const int tasks = shared_only ? 1 : a.task_bound;
    const int rpb = rows_per_block(m.rows, tasks, batch);
    dim3 grid((m.rows + rpb - 1) / rpb, tasks);
    return launch_any(m.dt, two, kind, grid, lds, a, p, rpb, shared_only ? 1 : 0, 0, s);
}

}  // namespace

hipError_t launch_gemv_up(const GemvArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t err = gemv_launch(kUp, a, e0, false, s);
    if (err == hipSuccess && a.has_shared && sh) err = gemv_launch(kUp, a, *sh, true, s);
    return err;
}

hipError_t launch_gemv_down(const GemvArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t err = gemv_launch(kDown, a, e0, false, s);
    if (err == hipSuccess && a.has_shared && sh) err = gemv_launch(kDown, a, *sh, true, s);
    return err;
}

hipError_t launch_gemv_down_single(const GemvArgs &a, const ExpertDev &ex, hipStream_t s) {
    return gemv_launch(kDown, a, ex, true, s);
}

hipError_t launch_gemv_down_combine(const GemvArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t err = gemv_launch(kDownCombine, a, e0, false, s);
    if (err == hipSuccess && a.has_shared && sh) err = gemv_launch(kDownCombine, a, *sh, true, s);
    return err;
}

hipError_t launch_gemv_exact(bool up, const GemvArgs &a, hipStream_t s) {
    const int tasks = a.task_bound + (a.has_shared ? 1 : 0);
    dim3 grid(64, tasks);
    if (up)
        hipLaunchKernelGGL(gemv_up_exact_kernel, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(gemv_down_exact_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace moe
