// expert_decode.hip — the experts of one token (T = 1) on gfx950.
//
// Decoding one token reads every weight of the k selected experts once and
// does two multiply-adds per weight, so the kernels are HBM-bound only if the
// arithmetic per weight byte stays small.  They dot the quantised weights
// directly against three-level int8 activations (qact.h) with
// v_dot4_i32_i8: a Q4_0 block of 32 values costs 3 unpack operations and 6
// integer dots per 8 values plus 7 float operations per block, fewer
// operations than dequantising to fp32.  The integer sums are exact; the
// activation error is at most 2^-24 of each 32-value block's range, so the
// products carry f32 precision.
//
//  * decode_up_kernel: h = silu(gate . x) * (up . x) for every row of the
//    selected experts (and the shared expert): src/model.rs:31-33 and the
//    expert's forward at src/model.rs:925-935.  Persistent waves stream rows
//    with several rows' weights in flight; each block first encodes x into
//    LDS.
//  * decode_up_unit_kernel: the same rows, one block per 64-row unit of h,
//    which the block encodes into activation units itself; used while the
//    units fit one round of resident blocks.
//  * decode_hq_kernel: otherwise, every selected expert's h (f32) to
//    activation units, one wavefront per 64-value unit, once for all down
//    blocks.
//  * decode_down_kernel: a block owns ranges of output rows and one group of
//    waves per selected expert; each lane loads its units of the experts'
//    h, streams their down rows and combines each row in
//    LDS: out = sum over the
//    selected experts in ascending order of w * y, from +0, separate
//    multiply and add (src/model.rs:842, 936-942); plus the shared expert
//    times its sigmoid gate (src/model.rs:956-970); plus the residual add
//    (src/model.rs:680-683).
//
// Lanes and rows: a row of `units` 64-value units is covered by CG lanes of
// a wave (CG = 16, 32 or 64 >= units; lanes own units c and, for rows of
// 65..128 units, c + 64) or, for wider down rows, by 4 waves of 64 lanes.
// A lane keeps its units of the activations in registers and streams the
// same units of many rows.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "gmem.h"
#include "moe_internal.h"
#include "qact.h"
#include "qdot.h"

namespace moe {
namespace {

using namespace qd;

// Loads the 32 floats at src into registers (16-byte aligned).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ inline void load32(const float *src, float (&v)[32]) {
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const f32x4 f = gload(s4 + i);
        v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
}

// All vector loads of a wave retire in order, so a wave that waits for one
// also waits for every load issued before it.  The kernels below therefore
// read their per-task metadata once, into LDS, before the weight stream
// starts, and issue activation loads ahead of weight loads.

// ------------------------------------------------------------- gate / up
//
// Work is a flat list of steps; step s is one row of one task (routed task
// i = the i-th selected expert, then the shared expert) for each of the
// 64 / CG row slices of a wave, i.e. rows s * (64 / CG) + slot.  Waves are
// persistent: wave w takes steps w, w + W, ..., with the weights of the next
// NBUF - 1 steps in flight while it computes the current one.  A block
// first encodes x into LDS (while its first weights load); each row's
// h = silu(gate . x) * (up . x) is written as f32 by the last lane of its
// slice.
struct UpStep {
    const uint8_t *g, *u;  // this lane's first unit of its row
    float *h;              // its h value
    bool ok;
};

// Every step yields loadable pointers, so that every step issues the same
// loads: the compiler then counts them exactly and waits for one step at a
// time (loads under a condition make it wait for all of them).  A step past
// the end, or of a task without an expert, reads task 0's first rows (task 0
// always has an expert) and is not computed; lanes past the row's units
// (c >= units) read its last unit.
__device__ inline UpStep up_step(const DecodeTask *tasks, int k_bound, int s, int n_steps, int spr, int slices,
                                 int slot, int c, int units, int UB) {
    UpStep st;
    const int sc = s < n_steps ? s : n_steps - 1;
    const int t = sc < k_bound * spr ? sc / spr : k_bound;
    const DecodeTask &T = tasks[t];
    st.ok = s < n_steps && T.live;
    const int r = T.live ? (t < k_bound ? sc - t * spr : sc - k_bound * spr) * slices + slot : slot;
    const DecodeTask &L = T.live ? T : tasks[0];
    const int cl = c < units ? c : units - 1;
    st.g = L.g + (size_t)r * L.gs + (size_t)cl * UB;
    st.u = L.u + (size_t)r * L.us + (size_t)cl * UB;
    st.h = T.h + r;
    return st;
}

template <int DT, int UPL, int DW>
__device__ inline void up_load(const UpStep &st, const bool (&live)[UPL], uint32_t (&w)[2][UPL][DW]) {
    constexpr int UB = WUnit<DT>::bytes;
#pragma unroll
    for (int j = 0; j < UPL; j++) {
        const size_t off = live[j] ? (size_t)j * 64 * UB : 0;
        load_wunit<DT, DW>(st.g + off, w[0][j]);
        load_wunit<DT, DW>(st.u + off, w[1][j]);
    }
}

template <int DT, int UPL, int DW>
__device__ inline void up_compute(const UpStep &st, const bool (&live)[UPL], const uint32_t (&w)[2][UPL][DW],
                                  const uint32_t (&xa)[UPL][kQUnitDw], int cg, bool tail) {
    if (!st.ok) return;
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int j = 0; j < UPL; j++)
        if (live[j]) g += qdot<DT, DW>(w[0][j], xa[j]), u += qdot<DT, DW>(w[1][j], xa[j]);
    g = slice_sum(g, cg);
    u = slice_sum(u, cg);
    if (tail) gstore(st.h, silu_mul(g, u));
}

// Steps per routed task `spr`; the shared expert's steps follow the routed
// ones as task k_bound.
template <int DT, int UPL, int NBUF>
__global__ __launch_bounds__(256) void decode_up_kernel(DecodeArgs a, const float *__restrict__ x, int spr,
                                                        int n_steps) {
    extern __shared__ __align__(16) uint8_t xs[];  // x as units
    __shared__ DecodeTask tasks[kMaxTopK + 1];
    constexpr int DW = WUnit<DT>::dw, UB = WUnit<DT>::bytes;
    const int units = a.H / 64, cg = lanes_for(units), slices = 64 / cg;
    const int lane = threadIdx.x & 63, slot = lane / cg, c = lane % cg;
    const bool tail = c == cg - 1;
    bool live[UPL];
#pragma unroll
    for (int j = 0; j < UPL; j++) live[j] = c + 64 * j < units;
    const int waves = blockDim.x >> 6;
    const int nw = gridDim.x * waves;
    const int s0 = blockIdx.x * waves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // x block of this thread, then the task table.
    const int n_xb = a.H / 32;
    float xv[32];
    if ((int)threadIdx.x < n_xb) load32(x + (size_t)threadIdx.x * 32, xv);
    const int ntask = a.k_bound + a.n_shared;
    for (int t = threadIdx.x; t < ntask; t += blockDim.x) tasks[t] = a.tasks[t];
    __syncthreads();

    uint32_t w[NBUF][2][UPL][DW];
    UpStep st[NBUF];
#pragma unroll
    for (int b = 0; b + 1 < NBUF; b++) {
        st[b] = up_step(tasks, a.k_bound, s0 + b * nw, n_steps, spr, slices, slot, c, units, UB);
        up_load<DT, UPL, DW>(st[b], live, w[b]);
    }
    if ((int)threadIdx.x < n_xb)
        qact_block_put<3>(qact_block(xv), xs + (size_t)(threadIdx.x >> 1) * kQUnitBytes, threadIdx.x & 1);
    __syncthreads();
    uint32_t xa[UPL][kQUnitDw];
#pragma unroll
    for (int j = 0; j < UPL; j++)
        if (live[j]) load_qunit<3>(xs + (size_t)(c + 64 * j) * kQUnitBytes, xa[j]);

    for (int s = s0; s < n_steps;) {
#pragma unroll
        for (int b = 0; b < NBUF; b++) {
            const int nb = (b + NBUF - 1) % NBUF;
            st[nb] = up_step(tasks, a.k_bound, s + (NBUF - 1) * nw, n_steps, spr, slices, slot, c, units, UB);
            up_load<DT, UPL, DW>(st[nb], live, w[nb]);
            if (s >= n_steps) break;
            up_compute<DT, UPL, DW>(st[b], live, w[b], xa, cg, tail);
            s += nw;
        }
    }
}

// Unit-aligned gate/up: block b computes the 64 rows of h that form unit b
// of the activation-unit list (routed task t's units, t ascending, then
// the shared expert's), its four waves taking the unit's steps w, w + 4,
// ... with NBUF - 1 steps in flight.  Each row's h goes to LDS; after a
// barrier the first wave encodes the unit (qact_wave_encode) where the down
// kernel reads it, so no encoding launch follows.  A block of a task
// without an expert does nothing.
template <int DT, int UPL, int NBUF>
__global__ __launch_bounds__(256) void decode_up_unit_kernel(DecodeArgs a, const float *__restrict__ x) {
    extern __shared__ __align__(16) uint8_t xs[];  // x as units
    __shared__ DecodeTask task;
    __shared__ float hrow[64];
    constexpr int DW = WUnit<DT>::dw, UB = WUnit<DT>::bytes;
    const int units = a.H / 64, cg = lanes_for(units), slices = 64 / cg;
    const int lane = threadIdx.x & 63, slot = lane / cg, c = lane % cg;
    const bool tail = c == cg - 1;
    bool live[UPL];
#pragma unroll
    for (int j = 0; j < UPL; j++) live[j] = c + 64 * j < units;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int upr = a.I / 64;
    const int b = blockIdx.x;
    const bool routed = b < a.k_bound * upr;
    const int t = routed ? b / upr : a.k_bound;
    const int u = routed ? b - t * upr : b - a.k_bound * upr;
    const int n_steps = 64 / slices;

    const int n_xb = a.H / 32;
    float xv[32];
    if ((int)threadIdx.x < n_xb) load32(x + (size_t)threadIdx.x * 32, xv);
    if (threadIdx.x == 0) task = a.tasks[t];
    __syncthreads();
    if (!task.live) return;  // the whole block

    // Step j of the unit: rows 64 u + j * slices + slot of the task; steps
    // past the unit re-read its last one and are not computed.
    const int cl = c < units ? c : units - 1;
    auto step = [&](int j) {
        UpStep st;
        st.ok = j < n_steps;
        const int r = 64 * u + (st.ok ? j : n_steps - 1) * slices + slot;
        st.g = task.g + (size_t)r * task.gs + (size_t)cl * UB;
        st.u = task.u + (size_t)r * task.us + (size_t)cl * UB;
        st.h = nullptr;
        return st;
    };
    uint32_t w[NBUF][2][UPL][DW];
    UpStep st[NBUF];
    int sj[NBUF];
#pragma unroll
    for (int k = 0; k + 1 < NBUF; k++) {
        sj[k] = wave + 4 * k;
        st[k] = step(sj[k]);
        up_load<DT, UPL, DW>(st[k], live, w[k]);
    }
    if ((int)threadIdx.x < n_xb)
        qact_block_put<3>(qact_block(xv), xs + (size_t)(threadIdx.x >> 1) * kQUnitBytes, threadIdx.x & 1);
    __syncthreads();
    uint32_t xa[UPL][kQUnitDw];
#pragma unroll
    for (int j = 0; j < UPL; j++)
        if (live[j]) load_qunit<3>(xs + (size_t)(c + 64 * j) * kQUnitBytes, xa[j]);

    for (bool more = sj[0] < n_steps; more;) {
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            const int nk = (k + NBUF - 1) % NBUF;
            sj[nk] = sj[(k + NBUF - 2) % NBUF] + 4;
            st[nk] = step(sj[nk]);
            up_load<DT, UPL, DW>(st[nk], live, w[nk]);
            if (!st[k].ok) {
                more = false;
                break;
            }
            float g = 0.0f, uu = 0.0f;
#pragma unroll
            for (int j = 0; j < UPL; j++)
                if (live[j]) g += qdot<DT, DW>(w[k][0][j], xa[j]), uu += qdot<DT, DW>(w[k][1][j], xa[j]);
            g = slice_sum(g, cg);
            uu = slice_sum(uu, cg);
            if (tail) hrow[sj[k] * slices + slot] = silu_mul(g, uu);
        }
    }
    __syncthreads();
    if (wave == 0) qact_wave_encode(hrow[lane], a.hq + ((size_t)t * a.hq_units + u) * kQUnitBytes, lane);
}

// --------------------------------------------------------------- down
//
// Units of h.  Wave w of the grid encodes unit w of the list (routed task
// t's units t * I/64 .. , then the shared expert's).  With one token each
// selected expert has one permuted row, so task t's h is row t of a.h (the
// dispatch kernel points the task there); the units of a task that is not
// live encode a row nobody wrote this call and are never read.
__global__ __launch_bounds__(256) void decode_hq_kernel(DecodeArgs a) {
    const int ur = a.I / 64, us = a.n_shared ? a.I_s / 64 : 0;
    const int n = a.k_bound * ur + us;
    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= n) return;
    const bool routed = w < a.k_bound * ur;
    const int t = routed ? w / ur : a.k_bound;
    const int u = routed ? w - t * ur : w - a.k_bound * ur;
    const float *h = routed ? a.h + (size_t)t * a.I : a.hs;
    qact_wave_encode(gload(h + 64 * u + lane), a.hq + ((size_t)t * a.hq_units + u) * kQUnitBytes, lane);
}

// A block owns output row ranges r = blockIdx.x, + gridDim.x, ... of `rb`
// rows and one group of waves per task: routed task i (the i-th selected
// expert, ascending) owns waves [i * ks_r, (i + 1) * ks_r), the shared
// expert the ks_s waves after them.  Each lane first loads its units of its
// task's h; each wave then streams the task's down rows of each range,
// NBUF - 1 ranges ahead.  Row slices leave their sums in
// LDS; after a barrier the block combines each row in the reference's
// order.  Lanes own one unit (UPL = 1: CG lanes per row slice, 64 / CG slices
// per wave, or ks = 4 waves of 64 lanes for rows wider than 128 units) or
// two (UPL = 2, rows of 65..128 units).
struct DownLane {
    bool active, tail;
    int task, kw, slot, rs, cg;
    bool live[2];
    const uint8_t *w;  // this lane's first unit of the task's row 0
    uint32_t stride;
};

// Unconditional, like up_load: ranges past the end re-read the last one,
// rows past the slot's rs its last row, units past the row its last unit,
// and lanes of a task without an expert read task 0's rows (down_lane).
template <int DT, int UPL, int RS, int DW>
__device__ inline void down_load(const DownLane &L, int range, int n_ranges, int rb, uint32_t (&w)[RS][UPL][DW]) {
    constexpr int UB = WUnit<DT>::bytes;
    const int rg = range < n_ranges ? range : n_ranges - 1;
    const uint8_t *p = L.w + (size_t)(rg * rb + L.slot * L.rs) * L.stride;
#pragma unroll
    for (int i = 0; i < RS; i++) {
        const int ii = i < L.rs ? i : L.rs - 1;
#pragma unroll
        for (int j = 0; j < UPL; j++) {
            const size_t off = L.live[j] ? (size_t)j * 64 * UB : 0;
            load_wunit<DT, DW>(p + (size_t)ii * L.stride + off, w[i][j]);
        }
    }
}

template <int DT, int UPL, int RS, int DW>
__device__ inline void down_compute(const DownLane &L, const uint32_t (&w)[RS][UPL][DW],
                                    const uint32_t (&xa)[UPL][kQUnitDw], float (*part)[32][4]) {
    if (!L.active) return;
#pragma unroll
    for (int i = 0; i < RS; i++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < UPL; j++)
            if (i < L.rs && L.live[j]) acc += qdot<DT, DW>(w[i][j], xa[j]);
        acc = slice_sum(acc, L.cg);
        if (L.tail && i < L.rs) part[L.task][L.slot * L.rs + i][L.kw] = acc;
    }
}

template <int DT>
__device__ inline void down_lane(const DecodeTask *tasks, int k_bound, int wv, int ks_r, int ks_s, int rb,
                                 DownLane &L) {
    const int routed_waves = k_bound * ks_r;
    const bool shared = wv >= routed_waves;
    L.task = shared ? k_bound : wv / ks_r;
    const DecodeTask &T = tasks[L.task];
    L.active = T.live != 0;
    L.tail = false;
    L.live[0] = L.live[1] = false;
    L.rs = 1;
    L.cg = 64;
    L.kw = L.slot = 0;
    L.w = tasks[0].d;  // loaded, not computed (down_load)
    L.stride = tasks[0].ds;
    if (!L.active) return;
    const int units = T.dcols / 64, lane = threadIdx.x & 63;
    const int ks = shared ? ks_s : ks_r;
    L.kw = (shared ? wv - routed_waves : wv) % ks;
    L.cg = ks > 1 ? 64 : lanes_for(units);
    L.slot = lane / L.cg;
    L.rs = rb / (64 / L.cg);
    L.tail = lane % L.cg == L.cg - 1;
    const int u0 = L.kw * 64 + lane % L.cg;
    L.live[0] = u0 < units;
    L.live[1] = u0 + 64 < units;
    L.w = T.d + (size_t)(u0 < units ? u0 : units - 1) * WUnit<DT>::bytes;
    L.stride = T.ds;
}

// Combine `n` rows of the partial sums in part (row q of part is row
// q % rb of the range the block took at iteration it0 + q / rb).
__device__ inline void down_combine(const DecodeArgs &a, const DecodeTask *tasks, int nh, float (*part)[32][4],
                                    int it0, int n, int rb, int ks_r, int ks_s) {
    for (int q = threadIdx.x; q < n; q += blockDim.x) {
        const int range = blockIdx.x + (it0 + q / rb) * gridDim.x;
        const int j = range * rb + q % rb;
        float out = 0.0f;
        for (int t = 0; t < nh; t++) {
            float v = 0.0f;
            for (int k = 0; k < ks_r; k++) v += part[t][q][k];
            const float prod = tasks[t].w * v;
            out = out + prod;
        }
        if (a.n_shared) {
            float v = 0.0f;
            for (int k = 0; k < ks_s; k++) v += part[a.k_bound][q][k];
            if (a.has_gate) v = v * tasks[a.k_bound].w;
            out = out + v;
        }
        if (a.addend) out = out + gload(a.addend + j);
        gstore(a.out + j, out);
        if (a.residual) gstore(a.residual + j, gload(a.residual + j) + out);
    }
}

template <int DT_R, int DT_S, int UPL, int RS, int NBUF, int NTHR>
__global__ __launch_bounds__(NTHR) void decode_down_kernel(DecodeArgs a, int rb,
                                                           int ks_r, int ks_s, int n_ranges) {
    __shared__ float part[2][kDecodeMaxWaves][32][4];
    __shared__ DecodeTask tasks[kDecodeMaxWaves];
    // Wave-uniform, so the branches on `shared` are scalar branches.
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr bool one_fmt = DT_R == DT_S;
    const bool shared = !one_fmt && wv >= a.k_bound * ks_r;
    constexpr int DWR = WUnit<DT_R>::dw, DWS = WUnit<DT_S>::dw;
    constexpr int DW = DWR > DWS ? DWR : DWS;
    const int ntask = a.k_bound + a.n_shared;

    if ((int)threadIdx.x < ntask) tasks[threadIdx.x] = a.tasks[threadIdx.x];
    __syncthreads();
    DownLane L;
    if (shared)
        down_lane<DT_S>(tasks, a.k_bound, wv, ks_r, ks_s, rb, L);
    else
        down_lane<DT_R>(tasks, a.k_bound, wv, ks_r, ks_s, rb, L);
    // The lane's units of its task's h (encoded by decode_hq_kernel) load
    // first, then the first ranges' weights (loads retire in order, so
    // waiting for the units does not wait for the weights).  Unconditional:
    // lanes without a unit read task 0's first unit.
    uint32_t xa[UPL][kQUnitDw];
    const int u0 = L.kw * 64 + (threadIdx.x & 63) % L.cg;
    const uint8_t *ub = a.hq + (size_t)L.task * a.hq_units * kQUnitBytes;
#pragma unroll
    for (int j = 0; j < UPL; j++)
        qact_unit_gload((L.active && L.live[j]) ? ub + (size_t)(u0 + 64 * j) * kQUnitBytes : a.hq, xa[j]);
    uint32_t w[NBUF][RS][UPL][DW];
    auto load = [&](int it, uint32_t (&buf)[RS][UPL][DW]) {
        const int range = blockIdx.x + it * gridDim.x;
        if (shared)
            down_load<DT_S, UPL, RS, DW>(L, range, n_ranges, rb, buf);
        else
            down_load<DT_R, UPL, RS, DW>(L, range, n_ranges, rb, buf);
    };
#pragma unroll
    for (int b = 0; b + 1 < NBUF; b++) load(b, w[b]);

    // Selected experts (live routed tasks come first).
    int nh = 0;
    while (nh < a.k_bound && tasks[nh].live) nh++;
    // Row sums collect in a 32-row chunk of part; a full chunk (or the last
    // range) is combined after one barrier, while the next chunk fills the
    // other half.
    const int n_it = (n_ranges - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    int it = 0, it0 = 0, sel = 0;
    for (bool more = it < n_it; more;) {
#pragma unroll
        for (int b = 0; b < NBUF; b++) {
            load(it + NBUF - 1, w[(b + NBUF - 1) % NBUF]);
            if (it >= n_it) {
                more = false;
                break;
            }
            float(*pp)[32][4] = reinterpret_cast<float(*)[32][4]>(&part[sel][0][(it - it0) * rb][0]);
            if (shared)
                down_compute<DT_S, UPL, RS, DW>(L, w[b], xa, pp);
            else
                down_compute<DT_R, UPL, RS, DW>(L, w[b], xa, pp);
            it++;
            if ((it - it0) * rb == 32 || it == n_it) {
                __syncthreads();
                down_combine(a, tasks, nh, part[sel], it0, (it - it0) * rb, rb, ks_r, ks_s);
                it0 = it;
                sel ^= 1;
            }
        }
    }
}

// --------------------------------------------------------------- launchers

int cus_of_current_device() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Resident blocks of `kernel` per CU at `threads` threads and `lds` bytes
// of dynamic LDS (at least 1), remembered per (kernel, threads, lds); lifts
// the kernel's dynamic LDS limit to `lds` first.
int occupancy(const void *kernel, int threads, size_t lds) {
    struct Entry {
        const void *k;
        int threads;
        size_t lds;
        int n;
    };
    static std::mutex mu;
    static std::vector<Entry> seen;
    std::lock_guard<std::mutex> g(mu);
    for (const Entry &e : seen)
        if (e.k == kernel && e.threads == threads && e.lds == lds) return e.n;
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, lds) != hipSuccess || n < 1) n = 1;
    seen.push_back({kernel, threads, lds, n});
    return n;
}

bool qfmt(int dt) { return dt == MOE_DT_Q4_0 || dt == MOE_DT_Q5_0 || dt == MOE_DT_Q8_0; }
int lanes_for_host(int units) { return units <= 16 ? 16 : units <= 32 ? 32 : 64; }
int upl_of(int units) { return units > 64 && units <= 128 ? 2 : 1; }
int dw_of(int dt) { return dt == MOE_DT_Q8_0 ? 17 : dt == MOE_DT_Q5_0 ? 11 : 9; }

// Down projection: waves per row and row slices per wave group.
int down_ks(int units) { return units > 128 ? 4 : 1; }
int down_slices(int units) { return units > 64 ? 1 : 64 / lanes_for_host(units); }

constexpr int kUpBuffers = 4;
constexpr int kDownBuffers = 3;

template <int DT, int UPL>
hipError_t up_go(const DecodeArgs &a, const float *x, int n_steps, int spr, hipStream_t s) {
    auto k = decode_up_kernel<DT, UPL, kUpBuffers>;
    const size_t lds = (size_t)(a.H / 64) * kQUnitBytes;
    const int per_cu = occupancy((const void *)k, 256, lds);
    const int nb = std::max(1, std::min((n_steps + 3) / 4, cus_of_current_device() * per_cu));
    hipLaunchKernelGGL(k, dim3(nb), dim3(256), lds, s, a, x, spr, n_steps);
    return hipGetLastError();
}

// Rows per lane slice of the down kernel for a format pair: at most 2 (more
// rows per range leave a block fewer ranges to pipeline: Mixtral's down
// kernel took 22.2 µs at 4 rows and 20.0 at 2), and what fits the register
// budget beside the activations, NBUF buffers deep.
int down_rs(int dt_r, int dt_s, int upl, bool big_block) {
    const int dw = std::max(dw_of(dt_r), dw_of(dt_s));
    const int budget = big_block ? 60 : 140;  // registers for the weight ring
    int rs = 2;
    while (rs > 1 && kDownBuffers * rs * upl * dw > budget) rs /= 2;
    return rs;
}

}  // namespace

bool decode_shared_apart(int I, int I_s, int dt_routed, int dt_shared) {
    // One down launch holds both formats only as Q4_0 + Q5_0 (the kernel's
    // two-format instance), and one number of units per lane.
    const bool fmt = dt_shared == dt_routed || (dt_routed == MOE_DT_Q4_0 && dt_shared == MOE_DT_Q5_0);
    return !fmt || upl_of(I / 64) != upl_of(I_s / 64);
}

bool decode_supported(int H, int I, int I_s, int dt_routed, int dt_shared) {
    auto width = [](int cols) { return cols > 0 && cols % 64 == 0 && cols / 64 <= 256; };
    if (!width(H) || H / 64 > 128 || !width(I) || !qfmt(dt_routed)) return false;
    if (I_s > 0 && (!width(I_s) || !qfmt(dt_shared))) return false;
    return true;
}

bool decode_fits(int I, int I_s, int k, int has_shared, int dt_routed, int dt_shared) {
    const bool apart = has_shared && decode_shared_apart(I, I_s, dt_routed, dt_shared);
    const int waves = k * down_ks(I / 64) + (has_shared && !apart ? down_ks(I_s / 64) : 0);
    if (waves > kDecodeMaxWaves) return false;
    if (apart) return down_ks(I_s / 64) <= kDecodeMaxWaves;
    if (!has_shared) return true;
    // Every task's row slices must split a range evenly.
    const int lo = std::min(down_slices(I / 64), down_slices(I_s / 64));
    const int hi = std::max(down_slices(I / 64), down_slices(I_s / 64));
    return hi / lo <= down_rs(dt_routed, dt_shared, upl_of(I / 64), waves > 8);
}

template <int DT, int UPL>
hipError_t up_unit_go(const DecodeArgs &a, const float *x, int n_units, hipStream_t s) {
    auto k = decode_up_unit_kernel<DT, UPL, kUpBuffers>;
    const size_t lds = (size_t)(a.H / 64) * kQUnitBytes;
    (void)occupancy((const void *)k, 256, lds);  // lifts the LDS limit
    hipLaunchKernelGGL(k, dim3(n_units), dim3(256), lds, s, a, x);
    return hipGetLastError();
}

// Which one-token gate/up kernel runs: 0 by decode_unit_pays, 1 the strided
// kernel (and the encoding launch), 2 the unit-aligned kernel.  Set by
// moe_debug_decode_kernel, or at load by MOE_DECODE_UNIT=0 / 1.
static int decode_unit_from_env() {
    const char *e = getenv("MOE_DECODE_UNIT");
    return e && (e[0] == '0' || e[0] == '1') ? 1 + (e[0] - '0') : 0;
}
static std::atomic<int> g_decode_unit{decode_unit_from_env()};

int set_decode_kernel(int choice) { return g_decode_unit.exchange(choice); }

// The unit-aligned kernel runs one block per unit of h and saves the
// encoding launch: it pays while the units fit one round of resident
// blocks (two per CU at one unit per lane, one at two).  Measured on
// MI355X, one token: Mixtral (448 units) 60.3 -> 58.6 µs, Qwen3 (96) 34.7 ->
// 32.0, V2-Lite (176) 38.8 -> 34.9, Qwen2-MoE (176) 46.5 -> 42.2; DeepSeek-V3
// (288 units at one block per CU, two rounds) 90.5 -> 107.
static bool decode_unit_pays(int n_units, int upl, int cus) { return n_units <= cus * (upl == 1 ? 2 : 1); }

hipError_t launch_decode_up(const DecodeArgs &a, const float *x, int dt_routed, int dt_shared, bool &encoded,
                            hipStream_t s) {
    const int units = a.H / 64, upl = upl_of(units);
    const int slices = 64 / lanes_for_host(units);
    encoded = false;
    const int n_units = a.k_bound * (a.I / 64) + (a.n_shared ? a.I_s / 64 : 0);
    const int forced = g_decode_unit.load();
    const bool unit = forced ? forced == 2 : decode_unit_pays(n_units, upl, cus_of_current_device());
    if (unit && a.hq && a.I % 64 == 0 && (!a.n_shared || a.I_s % 64 == 0) && a.I / 64 <= a.hq_units &&
        (!a.n_shared || a.I_s / 64 <= a.hq_units)) {
        auto ugo = [&](int dt, const DecodeArgs &d, int nu) -> hipError_t {
            switch (dt * 4 + upl) {
            case MOE_DT_Q4_0 * 4 + 1: return up_unit_go<MOE_DT_Q4_0, 1>(d, x, nu, s);
            case MOE_DT_Q4_0 * 4 + 2: return up_unit_go<MOE_DT_Q4_0, 2>(d, x, nu, s);
            case MOE_DT_Q5_0 * 4 + 1: return up_unit_go<MOE_DT_Q5_0, 1>(d, x, nu, s);
            case MOE_DT_Q5_0 * 4 + 2: return up_unit_go<MOE_DT_Q5_0, 2>(d, x, nu, s);
            case MOE_DT_Q8_0 * 4 + 1: return up_unit_go<MOE_DT_Q8_0, 1>(d, x, nu, s);
            case MOE_DT_Q8_0 * 4 + 2: return up_unit_go<MOE_DT_Q8_0, 2>(d, x, nu, s);
            default: return hipErrorInvalidValue;
            }
        };
        hipError_t e;
        if (!a.n_shared || dt_shared == dt_routed) {
            e = ugo(dt_routed, a, n_units);
        } else {
            DecodeArgs r = a;
            r.n_shared = 0;
            e = ugo(dt_routed, r, a.k_bound * (a.I / 64));
            if (e == hipSuccess) {
                // The shared expert's units: task 0 of its own table, its
                // units after the routed tasks' in hq.
                DecodeArgs sh = a;
                sh.k_bound = 0;
                sh.tasks = a.tasks + a.k_bound;
                sh.hq = a.hq + (size_t)a.k_bound * a.hq_units * kQUnitBytes;
                e = ugo(dt_shared, sh, a.I_s / 64);
            }
        }
        encoded = e == hipSuccess;
        return e;
    }
    auto go = [&](int dt, const DecodeArgs &d, int n_steps, int spr) -> hipError_t {
        switch (dt * 4 + upl) {
        case MOE_DT_Q4_0 * 4 + 1: return up_go<MOE_DT_Q4_0, 1>(d, x, n_steps, spr, s);
        case MOE_DT_Q4_0 * 4 + 2: return up_go<MOE_DT_Q4_0, 2>(d, x, n_steps, spr, s);
        case MOE_DT_Q5_0 * 4 + 1: return up_go<MOE_DT_Q5_0, 1>(d, x, n_steps, spr, s);
        case MOE_DT_Q5_0 * 4 + 2: return up_go<MOE_DT_Q5_0, 2>(d, x, n_steps, spr, s);
        case MOE_DT_Q8_0 * 4 + 1: return up_go<MOE_DT_Q8_0, 1>(d, x, n_steps, spr, s);
        case MOE_DT_Q8_0 * 4 + 2: return up_go<MOE_DT_Q8_0, 2>(d, x, n_steps, spr, s);
        default: return hipErrorInvalidValue;
        }
    };
    if (a.I % slices != 0 || (a.n_shared && a.I_s % slices != 0)) return hipErrorInvalidValue;
    const int spr = a.I / slices;
    if (!a.n_shared || dt_shared == dt_routed) return go(dt_routed, a, a.k_bound * spr + a.n_shared * (a.I_s / slices), spr);
    // A shared expert in another format: its own launch.
    DecodeArgs r = a;
    r.n_shared = 0;
    hipError_t e = go(dt_routed, r, a.k_bound * spr, spr);
    if (e != hipSuccess) return e;
    DecodeArgs sh = a;
    sh.k_bound = 0;
    sh.tasks = a.tasks + a.k_bound;  // the shared expert's entry
    return go(dt_shared, sh, a.I_s / slices, 1);
}

hipError_t launch_decode_encode(const DecodeArgs &a, hipStream_t s) {
    if (!a.hq || a.I % 64 || (a.n_shared && a.I_s % 64) || a.I / 64 > a.hq_units ||
        (a.n_shared && a.I_s / 64 > a.hq_units))
        return hipErrorInvalidValue;
    const int n = a.k_bound * (a.I / 64) + (a.n_shared ? a.I_s / 64 : 0);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(decode_hq_kernel, dim3((n + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_decode_down(const DecodeArgs &a, int dt_routed, int dt_shared, hipStream_t s) {
    if (a.n_shared && decode_shared_apart(a.I, a.I_s, dt_routed, dt_shared)) {
        // The shared expert alone first, its gated output into a.ys; then
        // the routed experts, adding it after their sum (the order of the
        // one-launch combine).
        if (!a.ys) return hipErrorInvalidValue;
        DecodeArgs sh = a;
        sh.k_bound = 0;
        sh.tasks = a.tasks + a.k_bound;
        sh.hq = a.hq + (size_t)a.k_bound * a.hq_units * kQUnitBytes;
        sh.I = a.I_s;
        sh.out = a.ys;
        sh.residual = nullptr;
        sh.addend = nullptr;
        hipError_t e = launch_decode_down(sh, dt_shared, dt_shared, s);
        if (e != hipSuccess) return e;
        DecodeArgs rt = a;
        rt.n_shared = 0;
        rt.addend = a.ys;
        return launch_decode_down(rt, dt_routed, dt_routed, s);
    }
    const int ur = a.I / 64, us = a.n_shared ? a.I_s / 64 : ur;
    const int upl = upl_of(ur);
    const int ks_r = down_ks(ur), ks_s = a.n_shared ? down_ks(us) : 1;
    const int waves = a.k_bound * ks_r + a.n_shared * ks_s;
    if (waves > kDecodeMaxWaves || (a.n_shared && upl_of(us) != upl)) return hipErrorInvalidValue;
    const bool big = waves > 8;
    const int ns_r = down_slices(ur), ns_s = a.n_shared ? down_slices(us) : ns_r;
    const int lo = std::min(ns_r, ns_s), hi = std::max(ns_r, ns_s);
    const int ds = a.n_shared ? dt_shared : dt_routed;
    const int RS = down_rs(dt_routed, ds, upl, big);
    if (hi / lo > RS) return hipErrorInvalidValue;
    const int rb = RS * lo;  // every task's slices get rb / ns <= RS rows
    if (rb > 32 || a.H % rb != 0) return hipErrorInvalidValue;
    const int n_ranges = a.H / rb;
    const int threads = 64 * waves;
    auto launch = [&](auto kern) -> hipError_t {
        const int per_cu = occupancy((const void *)kern, threads, 0);
        const int nb = std::max(1, std::min(n_ranges, cus_of_current_device() * per_cu));
        hipLaunchKernelGGL(kern, dim3(nb), dim3(threads), 0, s, a, rb, ks_r, ks_s, n_ranges);
        return hipGetLastError();
    };
#define MOE_DOWN_RS(R, S, U, N)                                                                                        \
    switch (RS) {                                                                                                      \
    case 1: return launch(decode_down_kernel<R, S, U, 1, kDownBuffers, N>);                                           \
    case 2: return launch(decode_down_kernel<R, S, U, 2, kDownBuffers, N>);                                           \
    default: return launch(decode_down_kernel<R, S, U, 4, kDownBuffers, N>);                                          \
    }
#define MOE_DOWN(R, S)                                                                                                 \
    if (upl == 2) {                                                                                                    \
        if (big) { MOE_DOWN_RS(R, S, 2, 1024) } else { MOE_DOWN_RS(R, S, 2, 512) }                                    \
    } else {                                                                                                           \
        if (big) { MOE_DOWN_RS(R, S, 1, 1024) } else { MOE_DOWN_RS(R, S, 1, 512) }                                    \
    }
    if (dt_routed == MOE_DT_Q4_0 && ds == MOE_DT_Q4_0) {
        MOE_DOWN(MOE_DT_Q4_0, MOE_DT_Q4_0)
    } else if (dt_routed == MOE_DT_Q4_0 && ds == MOE_DT_Q5_0) {
        MOE_DOWN(MOE_DT_Q4_0, MOE_DT_Q5_0)
    } else if (dt_routed == MOE_DT_Q5_0 && ds == MOE_DT_Q5_0) {
        MOE_DOWN(MOE_DT_Q5_0, MOE_DT_Q5_0)
    } else if (dt_routed == MOE_DT_Q8_0 && ds == MOE_DT_Q8_0) {
        MOE_DOWN(MOE_DT_Q8_0, MOE_DT_Q8_0)
    }
#undef MOE_DOWN
#undef MOE_DOWN_RS
    return hipErrorInvalidValue;
}

}  // namespace moe
