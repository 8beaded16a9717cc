// expert_batch.hip — SwiGLU experts over a few tokens per expert.
//
// With up to a few dozen tokens per expert the expert products read every
// weight of the hit experts once and do little arithmetic per weight, so
// they are HBM-bound if the arithmetic per weight byte stays small.  The
// one-token kernels' scheme carries over: weights are dotted, still
// quantised, with three-level int8 activations (qact.h) by v_dot4_i32_i8, and
// a lane keeps the activation units of NT tokens in registers so that each
// weight unit it loads serves all of them (the unpacking of a unit is shared
// by the tokens; the dots are four values per operation per token).
//
//  * qenc_kernel: rows of f32 to activation units (x before gate/up, h
//    before down).
//  * batch_up_kernel: h = silu(gate . x) * (up . x) (src/model.rs:31-33,
//    925-935) for the rows of one tile (an expert and up to NT of its
//    tokens, in dispatch order) over one block of weight rows.
//  * batch_down_kernel: y = down . h for the same tiles over one block of
//    output rows and one K part; the combine kernel then sums K parts and
//    experts in the reference's order.
//
// Lanes and rows: a row of `units` 64-value units is covered by CG lanes of
// a wave (CG = 16, 32 or 64 >= units), which own units c and, for rows of
// 65..128 units, c + 64 (UPL = 2).  A wave takes 64 / CG rows per step; the
// four waves of a block interleave their steps over the block's rows, and
// every wave keeps NBUF - 1 steps of weights in flight.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "gmem.h"
#include "moe_internal.h"
#include "qact.h"
#include "qdot.h"

namespace moe {
namespace {

using namespace qd;

// A matrix descriptor from the device expert table, read through global
// loads.
__device__ inline MatDev mat_of(const MatDev *m) {
    MatDev r;
    r.ptr = gload(&m->ptr);
    r.stride = gload(&m->stride);
    r.dt = gload(&m->dt);
    r.rows = gload(&m->rows);
    r.cols = gload(&m->cols);
    return r;
}

// ------------------------------------------------------------- encoding

// One wavefront per 64-value unit (qact_wave_encode).
__global__ __launch_bounds__(256) void qenc_kernel(const float *__restrict__ src, int rows, int cols,
                                                   uint8_t *__restrict__ dst) {
    const int units = cols / 64;
    const long long n = (long long)rows * units;
    const int lane = threadIdx.x & 63;
    const long long w0 = (long long)blockIdx.x * 4 + (threadIdx.x >> 6), nw = (long long)gridDim.x * 4;
    for (long long w = w0; w < n; w += nw) {
        const long long r = w / units;
        const int u = (int)(w - r * units);
        qact_wave_encode(gload(src + r * cols + 64 * u + lane), dst + (size_t)w * kQUnitBytes, lane);
    }
}

// ------------------------------------------------------------- tiles
//
// Block (x, y) of a launch covers row block x of tile y.  The grid is walked
// in the order (expert, row block, tile of the expert), tiles fastest, and
// each XCD (linear block id mod 8) takes a contiguous range of that order:
// the tiles of an expert that read the same weight rows run side by side in
// one XCD, so the rows come from HBM once and from L2 after that.
struct BTile {
    int g;       // expert (E: the shared expert)
    int r0;      // first permuted row (routed) or first token (shared)
    int n;       // tokens, 1..NT
    int rb;      // row block
    bool shared;
};

__device__ inline bool btile_of(const BatchArgs &a, int mode, int nt, BTile &b) {
    const int gx = gridDim.x, gy = gridDim.y;
    const int total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    const int routed = mode == 1 ? 0 : gload(a.ntiles) - a.shared_tiles;
    const int valid = (mode == 1 ? a.shared_tiles : routed) * gx;
    int t = lin;
    if ((total & 7) == 0) {
        const int per = (valid + 7) >> 3;
        const int j = lin >> 3;
        if (j >= per) return false;
        t = (lin & 7) * per + j;
    }
    if (t >= valid) return false;
    int g, m0;
    if (mode == 1) {
        // The shared expert's tiles: every token in tiles of a.nt, as the
        // dispatch lists them after the routed ones, taken from the
        // arguments so that these launches need nothing the routing writes.
        const int mt = a.shared_tiles;
        b.rb = t / mt;
        g = a.E, m0 = (t % mt) * a.nt;
    } else {
        // The tiles of one expert are contiguous: t / gx lies inside t's expert.
        const int ie = t / gx;
        const int f = gload(a.tiles + 4 * ie + 2), mt = gload(a.tiles + 4 * ie + 3);
        const int local = t - f * gx;
        const int i = f + local % mt;
        b.rb = local / mt;
        g = gload(a.tiles + 4 * i), m0 = gload(a.tiles + 4 * i + 1);
    }
    b.shared = mode == 1;
    if (!b.shared && g >= a.E) return false;
    b.g = g;
    const int cnt = b.shared ? a.T : gload(a.counts + g);
    b.n = min(nt, cnt - m0);
    b.r0 = b.shared ? m0 : gload(a.offsets + g) + m0;
    return b.n > 0;
}

// --------------------------------------------------------------- gate / up

template <int DT, int NT, int UPL, int NBUF>
__global__ __launch_bounds__(256) void batch_up_kernel(BatchArgs a, int rpb, int mode) {
    BTile b;
    if (!btile_of(a, mode, NT, b)) return;
    const MatDev G = mat_of(&a.experts[b.g].m[0]);
    const MatDev U = mat_of(&a.experts[b.g].m[1]);
    const int rows = G.rows;
    const int r0 = b.rb * rpb;
    if (r0 >= rows) return;
    const int r1 = min(rows, r0 + rpb);
    const int units = a.H / 64, cg = lanes_for(units), slices = 64 / cg;
    const int lane = threadIdx.x & 63, slot = lane / cg, c = lane % cg;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool tail = c == cg - 1;
    const int n = b.n;
    constexpr int DW = WUnit<DT>::dw, UB = WUnit<DT>::bytes;
    bool live[UPL];
#pragma unroll
    for (int j = 0; j < UPL; j++) live[j] = c + 64 * j < units;

    // This tile's tokens: activation units into registers, h rows.
    uint32_t xa[UPL][NT][kQUnitDw];
    float *hrow[NT];
    const int Icol = b.shared ? a.I_s : a.I;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tt = t < n ? t : 0;
        const int tok = b.shared ? b.r0 + tt : gload(a.perm_tok + b.r0 + tt);
        hrow[t] = (b.shared ? a.hs : a.h) + (size_t)(b.r0 + tt) * Icol;
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            if (t < n && live[j])
                load_qunit<1>(a.xq + ((size_t)tok * units + c + 64 * j) * kQUnitBytes, xa[j][t]);
            else
#pragma unroll
                for (int q = 0; q < kQUnitDw; q++) xa[j][t][q] = 0u;
        }
    }

    // Step s of this wave: rows r0 + (wv + 4 s) * slices + slot.  Loads are
    // unconditional (steps, rows and units past the end re-read the last
    // ones) so that the compiler counts them exactly and waits for one step
    // at a time rather than for all of them.
    const int nsteps = (r1 - r0 - wv * slices + 4 * slices - 1) / (4 * slices);
    if (nsteps <= 0) return;
    uint32_t w[NBUF][2][UPL][DW];
    auto row_of = [&](int s) { return r0 + (wv + 4 * s) * slices + slot; };
    auto load = [&](int s, uint32_t (&wb)[2][UPL][DW]) {
        const int r = min(row_of(min(s, nsteps - 1)), r1 - 1);
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            const int u = min(c + 64 * j, units - 1);
            load_wunit<DT, DW>(G.ptr + (size_t)r * G.stride + (size_t)u * UB, wb[0][j]);
            load_wunit<DT, DW>(U.ptr + (size_t)r * U.stride + (size_t)u * UB, wb[1][j]);
        }
    };
    // Branch-free but for the stores: rows past the block re-read valid
    // rows (load), tokens past the tile have all-zero units, and lanes past
    // the row's units add nothing.
    auto compute = [&](int s, const uint32_t (&wb)[2][UPL][DW]) {
        const int r = row_of(s);
        float g[NT], u[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) g[t] = 0.0f, u[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            float pg[NT], pu[NT];
            qdot_multi<DT, DW, NT>(wb[0][j], xa[j], pg);
            qdot_multi<DT, DW, NT>(wb[1][j], xa[j], pu);
#pragma unroll
            for (int t = 0; t < NT; t++) g[t] += live[j] ? pg[t] : 0.0f, u[t] += live[j] ? pu[t] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float gs = slice_sum(g[t], cg), us = slice_sum(u[t], cg);
            if (tail && r < r1 && t < n) gstore(hrow[t] + r, silu_mul(gs, us));
        }
    };
#pragma unroll
    for (int q = 0; q + 1 < NBUF; q++) load(q, w[q]);
    for (int s = 0; s < nsteps;) {
#pragma unroll
        for (int q = 0; q < NBUF; q++) {
            load(s + NBUF - 1, w[(q + NBUF - 1) % NBUF]);
            if (s >= nsteps) break;
            compute(s, w[q]);
            s++;
        }
    }
}

// --------------------------------------------------------------- down
//
// K part p = blockIdx.z covers units [p * per, p * per + per) of each row
// (per <= 64, one unit per lane).

template <int DT, int NT, int NBUF>
__global__ __launch_bounds__(256) void batch_down_kernel(BatchArgs a, int rpb, int mode) {
    BTile b;
    if (!btile_of(a, mode, NT, b)) return;
    const MatDev D = mat_of(&a.experts[b.g].m[2]);
    const int rows = D.rows;
    const int r0 = b.rb * rpb;
    if (r0 >= rows) return;
    const int r1 = min(rows, r0 + rpb);
    const int units = D.cols / 64, ks = gridDim.z, p = blockIdx.z;
    const int per = (units + ks - 1) / ks;
    const int u0 = p * per, un = min(per, units - u0);
    const int cg = lanes_for(per), slices = 64 / cg;
    const int lane = threadIdx.x & 63, slot = lane / cg, c = lane % cg;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool tail = c == cg - 1, live = c < un;
    const int n = b.n;
    constexpr int DW = WUnit<DT>::dw, UB = WUnit<DT>::bytes;

    uint32_t xa[NT][kQUnitDw];
    float *yrow[NT];
    const uint8_t *src = b.shared ? a.hsq : a.hq;
    float *ybase = b.shared ? a.ys + (size_t)p * a.yspart : a.y + (size_t)p * a.ypart;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int row = b.r0 + (t < n ? t : 0);
        yrow[t] = ybase + (size_t)row * a.H;
        if (t < n && live)
            load_qunit<1>(src + ((size_t)row * units + u0 + c) * kQUnitBytes, xa[t]);
        else
#pragma unroll
            for (int q = 0; q < kQUnitDw; q++) xa[t][q] = 0u;
    }

    const int nsteps = (r1 - r0 - wv * slices + 4 * slices - 1) / (4 * slices);
    if (nsteps <= 0) return;
    uint32_t w[NBUF][DW];
    auto row_of = [&](int s) { return r0 + (wv + 4 * s) * slices + slot; };
    const int uload = min(u0 + c, units - 1);  // unconditional loads, as in the gate/up kernel
    auto load = [&](int s, uint32_t (&wb)[DW]) {
        const int r = min(row_of(min(s, nsteps - 1)), r1 - 1);
        load_wunit<DT, DW>(D.ptr + (size_t)r * D.stride + (size_t)uload * UB, wb);
    };
    auto compute = [&](int s, const uint32_t (&wb)[DW]) {  // branch-free as in the gate/up kernel
        const int r = row_of(s);
        float yv[NT];
        qdot_multi<DT, DW, NT>(wb, xa, yv);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float v = slice_sum(live ? yv[t] : 0.0f, cg);
            if (tail && r < r1 && t < n) gstore(yrow[t] + r, v);
        }
    };
#pragma unroll
    for (int q = 0; q + 1 < NBUF; q++) load(q, w[q]);
    for (int s = 0; s < nsteps;) {
#pragma unroll
        for (int q = 0; q < NBUF; q++) {
            load(s + NBUF - 1, w[(q + NBUF - 1) % NBUF]);
            if (s >= nsteps) break;
            compute(s, w[q]);
            s++;
        }
    }
}

// --------------------------------------------------------------- launchers

bool qfmt(int dt) { return dt == MOE_DT_Q4_0 || dt == MOE_DT_Q5_0 || dt == MOE_DT_Q8_0; }
int lanes_host(int units) { return units <= 16 ? 16 : units <= 32 ? 32 : 64; }

// Weight steps in flight per wave (2..4): the ring fits beside the
// tokens' activations in half the register file, so two waves share a SIMD.
template <int DT, int UPL>
constexpr int up_bufs() {
    constexpr int n = 110 / (2 * UPL * WUnit<DT>::dw);
    return n < 2 ? 2 : n > 4 ? 4 : n;
}
template <int DT>
constexpr int down_bufs() {
    return 4;
}

int cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

// Rows per block: a whole number of block steps (4 waves x slices rows),
// enough blocks in all for about eight per CU.
int rows_per_block(int rows, int tiles, int slices) {
    const int step = 4 * slices;
    const long long want = 8LL * cus();
    long long rpb = ((long long)rows * tiles + want - 1) / want;
    rpb = (rpb + step - 1) / step * step;
    rpb = std::max<long long>(rpb, 2 * step);
    return (int)std::min<long long>(rpb, rows);
}

// Grid width: the row blocks, rounded up to a multiple of 8 so that the
// XCD-contiguous order of btile_of applies (blocks past the rows exit).
int row_blocks(int rows, int rpb) { return ((rows + rpb - 1) / rpb + 7) / 8 * 8; }

template <int DT, int NT, int UPL>
hipError_t up_go(const BatchArgs &a, int rows, int tiles, int mode, hipStream_t s) {
    const int units = a.H / 64, slices = 64 / lanes_host(units);
    const int rpb = rows_per_block(rows, tiles, slices);
    dim3 grid(row_blocks(rows, rpb), tiles);
    hipLaunchKernelGGL((batch_up_kernel<DT, NT, UPL, up_bufs<DT, UPL>()>), grid, dim3(256), 0, s, a, rpb, mode);
    return hipGetLastError();
}

template <int DT, int NT>
hipError_t down_go(const BatchArgs &a, int K, int tiles, int mode, hipStream_t s) {
    const int per = (K / 64 + a.ksplit - 1) / a.ksplit, slices = 64 / lanes_host(per);
    const int rpb = rows_per_block(a.H, tiles * a.ksplit, slices);
    dim3 grid(row_blocks(a.H, rpb), tiles, a.ksplit);
    hipLaunchKernelGGL((batch_down_kernel<DT, NT, down_bufs<DT>()>), grid, dim3(256), 0, s, a, rpb, mode);
    return hipGetLastError();
}

hipError_t up_dt(int dt, const BatchArgs &a, int rows, int tiles, int mode, hipStream_t s) {
    // Two units per lane (rows wider than 4096) take one token per tile.
    const int v = a.H / 64 > 64 ? 0 : a.nt == 1 ? 1 : 2;
    switch (dt * 3 + v) {
    case MOE_DT_Q4_0 * 3 + 0: return up_go<MOE_DT_Q4_0, 1, 2>(a, rows, tiles, mode, s);
    case MOE_DT_Q4_0 * 3 + 1: return up_go<MOE_DT_Q4_0, 1, 1>(a, rows, tiles, mode, s);
    case MOE_DT_Q4_0 * 3 + 2: return up_go<MOE_DT_Q4_0, 2, 1>(a, rows, tiles, mode, s);
    case MOE_DT_Q5_0 * 3 + 0: return up_go<MOE_DT_Q5_0, 1, 2>(a, rows, tiles, mode, s);
    case MOE_DT_Q5_0 * 3 + 1: return up_go<MOE_DT_Q5_0, 1, 1>(a, rows, tiles, mode, s);
    case MOE_DT_Q5_0 * 3 + 2: return up_go<MOE_DT_Q5_0, 2, 1>(a, rows, tiles, mode, s);
    case MOE_DT_Q8_0 * 3 + 0: return up_go<MOE_DT_Q8_0, 1, 2>(a, rows, tiles, mode, s);
    case MOE_DT_Q8_0 * 3 + 1: return up_go<MOE_DT_Q8_0, 1, 1>(a, rows, tiles, mode, s);
    case MOE_DT_Q8_0 * 3 + 2: return up_go<MOE_DT_Q8_0, 2, 1>(a, rows, tiles, mode, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t down_dt(int dt, const BatchArgs &a, int K, int tiles, int mode, hipStream_t s) {
    const bool one = a.nt == 1;
    switch (dt) {
    case MOE_DT_Q4_0: return one ? down_go<MOE_DT_Q4_0, 1>(a, K, tiles, mode, s) : down_go<MOE_DT_Q4_0, 2>(a, K, tiles, mode, s);
    case MOE_DT_Q5_0: return one ? down_go<MOE_DT_Q5_0, 1>(a, K, tiles, mode, s) : down_go<MOE_DT_Q5_0, 2>(a, K, tiles, mode, s);
    case MOE_DT_Q8_0: return one ? down_go<MOE_DT_Q8_0, 1>(a, K, tiles, mode, s) : down_go<MOE_DT_Q8_0, 2>(a, K, tiles, mode, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool batch_supported(int H, int I, int I_s, int dt_routed, int dt_shared) {
    auto width = [](int cols, int max_units) { return cols > 0 && cols % 64 == 0 && cols / 64 <= max_units; };
    if (!width(H, 128) || !width(I, 64 * kMaxKSplit) || !qfmt(dt_routed)) return false;
    if (I_s > 0 && (!width(I_s, 64 * kMaxKSplit) || !qfmt(dt_shared))) return false;
    return true;
}

int batch_tile_tokens(int H, int t, int k, int E) { return (H / 64 > 64 || (long long)t * k <= E) ? 1 : 2; }

int batch_ksplit(int I, int I_s) {
    const int units = std::max(I, I_s) / 64;
    return (units + 63) / 64;
}

hipError_t launch_qenc(const float *src, int rows, int cols, uint8_t *dst, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (cols % 64 != 0) return hipErrorInvalidValue;
    const long long waves = (long long)rows * (cols / 64);  // one per unit
    const int grid = (int)std::min<long long>((waves + 3) / 4, 8LL * cus());
    hipLaunchKernelGGL(qenc_kernel, dim3(grid), dim3(256), 0, s, src, rows, cols, dst);
    return hipGetLastError();
}

hipError_t launch_batch_up(const BatchArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t e = up_dt(e0.m[0].dt, a, e0.m[0].rows, a.max_tiles, 0, s);
    if (e != hipSuccess || !sh || !a.shared_tiles) return e;
    return up_dt(sh->m[0].dt, a, sh->m[0].rows, a.shared_tiles, 1, s);
}

hipError_t launch_batch_down(const BatchArgs &a, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    hipError_t e = down_dt(e0.m[2].dt, a, e0.m[2].cols, a.max_tiles, 0, s);
    if (e != hipSuccess || !sh || !a.shared_tiles) return e;
    return down_dt(sh->m[2].dt, a, sh->m[2].cols, a.shared_tiles, 1, s);
}

hipError_t launch_batch_up_shared(const BatchArgs &a, const ExpertDev &sh, hipStream_t s) {
    return a.shared_tiles ? up_dt(sh.m[0].dt, a, sh.m[0].rows, a.shared_tiles, 1, s) : hipSuccess;
}

hipError_t launch_batch_down_shared(const BatchArgs &a, const ExpertDev &sh, hipStream_t s) {
    return a.shared_tiles ? down_dt(sh.m[2].dt, a, sh.m[2].cols, a.shared_tiles, 1, s) : hipSuccess;
}

}  // namespace moe
