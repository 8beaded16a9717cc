// expert_gemv.hip — SwiGLU experts over few tokens per expert (decode).
//
// Two families:
//  * fast GEMV: weights stream from HBM once, each thread dequantises one
//    64-value unit (two 32-value blocks) of a row in registers and dots it
//    with activations it keeps in registers for the whole kernel; a row's
//    partial sums are reduced across the row group.  fp32 throughout, weights
//    exact (d * q is exact in f32), so results differ from the reference only
//    by summation order.
//  * exact GEMV: one thread per (row, token) computing the reference's dot
//    (src/quant.rs:386-420) in its exact lane and reduction order over the
//    exactly dequantised row (src/quant.rs:177-227), and SwiGLU with glibc's
//    expf (src/model.rs:31-33).  Bit-identical to the CPU path; used where a
//    shape does not fit the fast path (rows not 4-byte aligned, widths not a
//    multiple of 64) and for the bit-exact parity mode.
//
// Work list: blockIdx.y < hits[0] is the routed expert hits[1 + y] over its
// tokens (permuted rows offsets[e] .. offsets[e] + counts[e]); blockIdx.y ==
// task_bound is the shared expert over all T tokens.  Higher y exit at once.
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
__device__ inline bool task_of(const GemvArgs &a, Task &tk) {
    const int y = blockIdx.y;
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

// Dot of one 64-value unit at `p` (4-byte aligned) with NT activation vectors.
// `sx` holds the per-block sums of the activations, which absorb the format's
// zero offset: sum((q - o) x) = sum(q x) - o sum(x) with q read unsigned.
template <int DT, int NT>
__device__ inline void unit_dot(const uint8_t *p, const float (&xv)[NT][64], const float (&sx)[NT][2],
                                float (&acc)[NT]) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p, 4));
    if constexpr (DT == MOE_DT_F32) {
        float w[64];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
            w[4 * i + 0] = __uint_as_float(v.x);
            w[4 * i + 1] = __uint_as_float(v.y);
            w[4 * i + 2] = __uint_as_float(v.z);
            w[4 * i + 3] = __uint_as_float(v.w);
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) {
                s0 = fmaf(w[i], xv[t][i], s0);
                s1 = fmaf(w[32 + i], xv[t][32 + i], s1);
            }
            acc[t] += s0 + s1;
        }
    } else if constexpr (DT == MOE_DT_Q4_0) {
        // 36 bytes: [dA qA0..15][dB qB0..15]
        uint32_t d[9];
        u32x4 v0 = *reinterpret_cast<const u32x4 *>(q);
        u32x4 v1 = *reinterpret_cast<const u32x4 *>(q + 4);
        d[0] = v0.x, d[1] = v0.y, d[2] = v0.z, d[3] = v0.w;
        d[4] = v1.x, d[5] = v1.y, d[6] = v1.z, d[7] = v1.w;
        d[8] = q[8];
        const float sa = h2f(d[0]), sb = h2f(d[4] >> 16);
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qa[i] = alignb(d[i + 1], d[i], 2);
            qb[i] = d[5 + i];
        }
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
        // 44 bytes: [dA hA(4) qA0..15][dB hB(4) qB0..15]
        uint32_t d[11];
        u32x4 v0 = *reinterpret_cast<const u32x4 *>(q);
        u32x4 v1 = *reinterpret_cast<const u32x4 *>(q + 4);
        d[0] = v0.x, d[1] = v0.y, d[2] = v0.z, d[3] = v0.w;
        d[4] = v1.x, d[5] = v1.y, d[6] = v1.z, d[7] = v1.w;
        d[8] = q[8], d[9] = q[9], d[10] = q[10];
        const float sa = h2f(d[0]), sb = h2f(d[5] >> 16);
        const uint32_t ha = alignb(d[1], d[0], 2), hb = d[6];
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qa[i] = alignb(d[i + 2], d[i + 1], 2);
            qb[i] = d[7 + i];
        }
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
    } else {  // Q8_0, 68 bytes: [dA qA0..31][dB qB0..31]
        uint32_t d[17];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
            d[4 * i + 0] = v.x, d[4 * i + 1] = v.y, d[4 * i + 2] = v.z, d[4 * i + 3] = v.w;
        }
        d[16] = q[16];
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

// Sum over the CG threads of a row group.  CG <= 64: shuffles inside the
// wave; CG > 64: shuffles, then the row group's waves combine through LDS.
template <int CG>
__device__ inline float group_sum(float v, float *red, int slot) {
    constexpr int W = CG < 64 ? CG : 64;
#pragma unroll
    for (int m = W / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    if constexpr (CG <= 64) {
        return v;
    } else {
        constexpr int NW = CG / 64;
        const int wv = (threadIdx.x & (CG - 1)) >> 6;
        if ((threadIdx.x & 63) == 0) red[slot * NW + wv] = v;
        __syncthreads();
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++) s += red[slot * NW + i];
        __syncthreads();
        return s;
    }
}

template <int NT>
__device__ inline void load_acts(const float *const (&src)[NT], int c, int units, float (&xv)[NT][64],
                                 float (&sx)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (c < units && src[t]) {
            const float4 *s4 = reinterpret_cast<const float4 *>(src[t] + 64 * c);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float4 v = s4[i];
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

// gate+up+SwiGLU for one expert's tokens: h[row][r] = silu(gate_r . x) * (up_r . x).
template <int DT, int CG, int NT>
__global__ __launch_bounds__(256) void gemv_up_kernel(GemvArgs a, int rows_per_block) {
    __shared__ float red[2 * NT * (256 / 64)];
    Task tk;
    if (!task_of(a, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &G = ex.m[0], &U = ex.m[1];
    const int rows = G.rows;
    const int r_begin = blockIdx.x * rows_per_block;
    if (r_begin >= rows) return;
    const int r_end = min(rows, r_begin + rows_per_block);
    constexpr int RG = 256 / CG;
    const int c = threadIdx.x % CG, rg = threadIdx.x / CG;
    const int units = G.cols / 64;
    const int Icol = tk.shared ? a.I_s : a.I;
    float *hout = tk.shared ? a.hs : a.h;
    for (int t0 = 0; t0 < tk.n; t0 += NT) {
        const float *src[NT];
        int rowid[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int i = t0 + t;
            rowid[t] = i < tk.n ? tk.row0 + i : -1;
            const int tok = i < tk.n ? (tk.shared ? i : a.perm_tok[tk.row0 + i]) : -1;
            src[t] = tok >= 0 ? a.x + (size_t)tok * a.H : nullptr;
        }
        float xv[NT][64], sx[NT][2];
        load_acts<NT>(src, c, units, xv, sx);
        for (int rb = r_begin; rb < r_end; rb += RG) {
            const int r = rb + rg;
            float ag[NT], au[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) ag[t] = 0.0f, au[t] = 0.0f;
            if (r < r_end && c < units) {
                unit_dot<DT, NT>(G.ptr + (size_t)r * G.stride + (size_t)c * 2 * block_bytes(DT), xv, sx, ag);
                unit_dot<DT, NT>(U.ptr + (size_t)r * U.stride + (size_t)c * 2 * block_bytes(DT), xv, sx, au);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float g = group_sum<CG>(ag[t], red, rg * 2 * NT + 2 * t);
                const float u = group_sum<CG>(au[t], red, rg * 2 * NT + 2 * t + 1);
                if (c == 0 && r < r_end && rowid[t] >= 0) {
                    const float sg = g / (1.0f + __expf(-g));
                    hout[(size_t)rowid[t] * Icol + r] = sg * u;
                }
            }
        }
    }
}

// down: y[row][j] = down_j . h[row].
template <int DT, int CG, int NT>
__global__ __launch_bounds__(256) void gemv_down_kernel(GemvArgs a, int rows_per_block) {
    __shared__ float red[NT * (256 / 64)];
    Task tk;
    if (!task_of(a, tk)) return;
    const ExpertDev &ex = a.experts[tk.g];
    const MatDev &D = ex.m[2];
    const int rows = D.rows;  // H
    const int r_begin = blockIdx.x * rows_per_block;
    if (r_begin >= rows) return;
    const int r_end = min(rows, r_begin + rows_per_block);
    constexpr int RG = 256 / CG;
    const int c = threadIdx.x % CG, rg = threadIdx.x / CG;
    const int units = D.cols / 64;
    const int Icol = tk.shared ? a.I_s : a.I;
    const float *hin = tk.shared ? a.hs : a.h;
    float *yout = tk.shared ? a.ys : a.y;
    for (int t0 = 0; t0 < tk.n; t0 += NT) {
        const float *src[NT];
        int rowid[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int i = t0 + t;
            rowid[t] = i < tk.n ? tk.row0 + i : -1;
            src[t] = rowid[t] >= 0 ? hin + (size_t)rowid[t] * Icol : nullptr;
        }
        float xv[NT][64], sx[NT][2];
        load_acts<NT>(src, c, units, xv, sx);
        for (int rb = r_begin; rb < r_end; rb += RG) {
            const int r = rb + rg;
            float ay[NT];
#pragma unroll
            for (int t = 0; t < NT; t++) ay[t] = 0.0f;
            if (r < r_end && c < units)
                unit_dot<DT, NT>(D.ptr + (size_t)r * D.stride + (size_t)c * 2 * block_bytes(DT), xv, sx, ay);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float v = group_sum<CG>(ay[t], red, rg * NT + t);
                if (c == 0 && r < r_end && rowid[t] >= 0) yout[(size_t)rowid[t] * a.H + r] = v;
            }
        }
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
    if (!task_of(a, tk)) return;
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
    if (!task_of(a, tk)) return;
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

int pick_cg(int units) {
    int cg = 16;
    while (cg < units && cg < 256) cg <<= 1;
    return cg;
}

// Rows per block: enough blocks to cover the chip several times.
int pick_rpb(int rows, int rg, int tasks) {
    int rpb = rg;
    while (rpb < rows && (long long)((rows + rpb * 2 - 1) / (rpb * 2)) * tasks >= 2048) rpb *= 2;
    return rpb;
}

#define MOE_GEMV_DISPATCH(KERNEL, DT, CG, NT, grid, a, rpb, s)                                      \
    hipLaunchKernelGGL((KERNEL<DT, CG, NT>), grid, dim3(256), 0, s, a, rpb)

template <int CG, int NT>
hipError_t launch_up_dt(int dt, dim3 grid, const GemvArgs &a, int rpb, hipStream_t s) {
    switch (dt) {
    case MOE_DT_F32: MOE_GEMV_DISPATCH(gemv_up_kernel, MOE_DT_F32, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q8_0: MOE_GEMV_DISPATCH(gemv_up_kernel, MOE_DT_Q8_0, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q4_0: MOE_GEMV_DISPATCH(gemv_up_kernel, MOE_DT_Q4_0, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q5_0: MOE_GEMV_DISPATCH(gemv_up_kernel, MOE_DT_Q5_0, CG, NT, grid, a, rpb, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
template <int CG, int NT>
hipError_t launch_down_dt(int dt, dim3 grid, const GemvArgs &a, int rpb, hipStream_t s) {
    switch (dt) {
    case MOE_DT_F32: MOE_GEMV_DISPATCH(gemv_down_kernel, MOE_DT_F32, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q8_0: MOE_GEMV_DISPATCH(gemv_down_kernel, MOE_DT_Q8_0, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q4_0: MOE_GEMV_DISPATCH(gemv_down_kernel, MOE_DT_Q4_0, CG, NT, grid, a, rpb, s); break;
    case MOE_DT_Q5_0: MOE_GEMV_DISPATCH(gemv_down_kernel, MOE_DT_Q5_0, CG, NT, grid, a, rpb, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool UP, int NT>
hipError_t launch_cg(int cg, int dt, dim3 grid, const GemvArgs &a, int rpb, hipStream_t s) {
    switch (cg) {
    case 16: return UP ? launch_up_dt<16, NT>(dt, grid, a, rpb, s) : launch_down_dt<16, NT>(dt, grid, a, rpb, s);
    case 32: return UP ? launch_up_dt<32, NT>(dt, grid, a, rpb, s) : launch_down_dt<32, NT>(dt, grid, a, rpb, s);
    case 64: return UP ? launch_up_dt<64, NT>(dt, grid, a, rpb, s) : launch_down_dt<64, NT>(dt, grid, a, rpb, s);
    case 128: return UP ? launch_up_dt<128, NT>(dt, grid, a, rpb, s) : launch_down_dt<128, NT>(dt, grid, a, rpb, s);
    case 256: return UP ? launch_up_dt<256, NT>(dt, grid, a, rpb, s) : launch_down_dt<256, NT>(dt, grid, a, rpb, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Fast launches take the format and widths from the routed experts (all
// routed experts of a layer share them; the shared expert is launched
// separately when its format or width differs).
static hipError_t gemv_fast(bool up, const GemvArgs &a0, const ExpertDev &ex, int tasks_routed, bool shared_only,
                            hipStream_t s) {
    GemvArgs a = a0;
    const MatDev &m = up ? ex.m[0] : ex.m[2];
    const int units = m.cols / 64;
    const int cg = pick_cg(units);
    const int rg = 256 / cg;
    const int rows = m.rows;
    int tasks = tasks_routed;
    if (shared_only) {
        // Only the shared-expert task: make it task 0 of a 1-task grid.
        a.task_bound = 0;
        tasks = 1;
    } else {
        a.has_shared = 0;
    }
    const int rpb = pick_rpb(rows, rg, tasks);
    dim3 grid((rows + rpb - 1) / rpb, tasks);
    // Two token columns per pass whenever a task can carry several tokens.
    const bool two = a.T > 1;
    if (two) return up ? launch_cg<true, 2>(cg, m.dt, grid, a, rpb, s) : launch_cg<false, 2>(cg, m.dt, grid, a, rpb, s);
    return up ? launch_cg<true, 1>(cg, m.dt, grid, a, rpb, s) : launch_cg<false, 1>(cg, m.dt, grid, a, rpb, s);
}

hipError_t launch_gemv_up(const GemvArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t err = gemv_fast(true, a, e0, a.task_bound, false, s);
    if (err == hipSuccess && a.has_shared && sh) err = gemv_fast(true, a, *sh, 0, true, s);
    return err;
}

hipError_t launch_gemv_down(const GemvArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t err = gemv_fast(false, a, e0, a.task_bound, false, s);
    if (err == hipSuccess && a.has_shared && sh) err = gemv_fast(false, a, *sh, 0, true, s);
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
