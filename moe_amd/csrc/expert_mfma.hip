// expert_mfma.hip — grouped SwiGLU expert GEMMs on gfx950 matrix cores.
//
// One block computes a 128-token x 128-column tile of one expert:
//   up   : 64 gate rows and the same 64 up rows of the expert, K = H; the
//          epilogue forms h = silu(G) * U and stores it as f16.
//   down : 128 rows of W_down, K = I (optionally split in two halves, each
//          half writing its own output buffer); output y in f32.
// Four waves each own all 128 tokens x 32 columns, so every weight value is
// dequantised exactly once per block and goes straight into MFMA operand
// registers: raw weight blocks are staged in LDS (one 4-byte-aligned record
// per 32-value block: scale dword, then code dwords) and each lane turns its
// eight codes of a block into f16 (d * q rounded once).  Activations are
// staged in LDS with K permuted inside each 32-value block so that a lane's
// eight K positions are {4q..4q+3, 16+4q..16+4q+3}, the values whose codes
// share one dword of a Q4_0/Q5_0 block.  Both LDS stages are double
// buffered; the next K step's global loads are issued before the current
// step's MFMAs (V_MFMA_F32_16X16X32_F16, f32 accumulation).  16-row
// sub-tiles past the expert's last token are skipped.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gmem.h"
#include "moe_internal.h"

namespace moe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));

constexpr int BM = 128;        // tokens per tile
constexpr int BW = 256;        // weight rows per tile (up: 128 gate + 128 up rows)
constexpr int BK = 64;         // K values per step (two 32-value blocks)
constexpr int LDA = BK + 8;    // A row stride in halves (144 bytes)

__device__ inline uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t s) { return __builtin_amdgcn_alignbyte(hi, lo, s); }
__device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }
__device__ inline __half2 as_h2(uint32_t v) {
    __half2 h;
    __builtin_memcpy(&h, &v, 4);
    return h;
}
__device__ inline uint32_t h2_bits(__half2 h) {
    uint32_t v;
    __builtin_memcpy(&v, &h, 4);
    return v;
}
__device__ inline uint32_t spread4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

// Codes b0..b3 (bytes of v, each < 256), minus `off2`, times `d2`, as f16
// pairs (b0, b1) and (b2, b3).  0x64 in the high byte makes each f16 exactly
// 1024 + b, so the subtraction is exact and the product rounds once.
__device__ inline void codes4(uint32_t v, __half2 off2, __half2 d2, uint32_t &w01, uint32_t &w23) {
    w01 = h2_bits(__hmul2(__hsub2(as_h2(perm(0x64646464u, v, 0x04010400u)), off2), d2));
    w23 = h2_bits(__hmul2(__hsub2(as_h2(perm(0x64646464u, v, 0x04030402u)), off2), d2));
}

// Per-format layout of one 32-value block: bytes in the checkpoint, dwords
// fetched from a 4-byte-aligned address, dwords of the LDS record.
template <int DT>
struct Fmt;
template <>
struct Fmt<MOE_DT_Q4_0> {
    static constexpr int bytes = 18, fetch = 5, rec = 5;
};
template <>
struct Fmt<MOE_DT_Q5_0> {
    static constexpr int bytes = 22, fetch = 6, rec = 6;
};
template <>
struct Fmt<MOE_DT_Q8_0> {
    static constexpr int bytes = 34, fetch = 9, rec = 9;
};

// The dwords covering block b of a 4-byte-aligned row, as loaded (global
// loads; nothing waits for them here).
template <int DT>
__device__ inline void fetch_raw(const uint8_t *row, int b, uint32_t (&d)[Fmt<DT>::fetch]) {
    const uint32_t *q =
        reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(row, 4)) + ((b * Fmt<DT>::bytes) >> 2);
#pragma unroll
    for (int i = 0; i < Fmt<DT>::fetch; i++) d[i] = gload(q + i);
}

// Normalise fetched dwords to the block's LDS record: rec[0] = scale (low 16
// bits), rec[1..] = the bytes after the scale.  `odd`: the block starts 2
// bytes into its first dword (an odd block index in every format).
template <int DT>
__device__ inline void normalise(const uint32_t (&d)[Fmt<DT>::fetch], bool odd, uint32_t (&rec)[Fmt<DT>::rec]) {
    constexpr int N = Fmt<DT>::fetch;
    uint32_t s[N];  // the block starting at byte 0
#pragma unroll
    for (int i = 0; i < N - 1; i++) s[i] = odd ? alignb(d[i + 1], d[i], 2) : d[i];
    s[N - 1] = odd ? (d[N - 1] >> 16) : d[N - 1];
    rec[0] = s[0] & 0xffffu;
#pragma unroll
    for (int i = 1; i < Fmt<DT>::rec; i++) rec[i] = alignb(s[i], s[i - 1], 2);
}

// Lane group q's eight values of a block record, as one MFMA operand:
// slots 0..3 = elements 4q..4q+3, slots 4..7 = elements 16+4q..16+4q+3.
// rec_codes reads the record dwords that hold them; dequant_codes turns them
// into f16 (d * q rounded once).
template <int DT>
struct Codes;
template <>
struct Codes<MOE_DT_Q4_0> {
    static constexpr int n = 1;  // the code dword
};
template <>
struct Codes<MOE_DT_Q5_0> {
    static constexpr int n = 2;  // high-bit dword, code dword
};
template <>
struct Codes<MOE_DT_Q8_0> {
    static constexpr int n = 2;  // low-half and high-half code dwords
};
template <int DT>
__device__ inline void rec_codes(const uint32_t *rec, int q, uint32_t (&c)[Codes<DT>::n]) {
    if constexpr (DT == MOE_DT_Q4_0) {
        c[0] = rec[1 + q];
    } else if constexpr (DT == MOE_DT_Q5_0) {
        c[0] = rec[1], c[1] = rec[2 + q];
    } else {
        c[0] = rec[1 + q], c[1] = rec[5 + q];
    }
}
template <int DT>
__device__ inline half8 dequant_codes(uint32_t scale, const uint32_t (&c)[Codes<DT>::n], int q) {
    const __half2 d2 = as_h2((scale & 0xffffu) * 0x10001u);
    uint32_t o[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        codes4(c[0] & 0x0f0f0f0fu, off2, d2, o[0], o[1]);
        codes4((c[0] >> 4) & 0x0f0f0f0fu, off2, d2, o[2], o[3]);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const uint32_t hb = c[0];
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        codes4((c[1] & 0x0f0f0f0fu) | spread4((hb >> (4 * q)) & 0xfu), off2, d2, o[0], o[1]);
        codes4(((c[1] >> 4) & 0x0f0f0f0fu) | spread4((hb >> (16 + 4 * q)) & 0xfu), off2, d2, o[2], o[3]);
    } else {  // Q8_0: int8 codes, read as uint8 + 128
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
        codes4(c[0] ^ 0x80808080u, off2, d2, o[0], o[1]);
        codes4(c[1] ^ 0x80808080u, off2, d2, o[2], o[3]);
    }
    half8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

// Tile coordinates.  mode 0: routed tiles from the dispatch list; mode 1: the
// shared expert over all T tokens.  The grid is walked in the order
// (expert, N tile, M tile), M fastest, and each XCD (linear block id mod 8)
// takes a contiguous range of that order: an expert's weight tile is read
// from HBM once and met in L2 by the expert's other M tiles, and the
// expert's activations stay in that XCD's L2 while its N tiles go by.
struct TileInfo {
    int g, m0, n, row0, ntile, ksplit;
    bool shared;
};
__device__ inline bool tile_of(const MfmaArgs &a, int mode, int gx, TileInfo &ti) {
    const int gy = gridDim.y, gz = gridDim.z;
    const int total = gx * gy;
    const int lin = blockIdx.x + gx * blockIdx.y;
    ti.ksplit = gz > 1 ? (int)blockIdx.z : 0;
    const int mt_sh = (a.T + BM - 1) / BM;
    const int valid = mode == 1 ? mt_sh * gy : a.ntiles[0] * gy;  // <= total
    // XCD x (= lin mod 8) takes t in [x * per, (x + 1) * per) in order.
    int t = lin;
    if ((total & 7) == 0) {
        const int per = (valid + 7) >> 3;
        const int j = lin >> 3;
        if (j >= per) return false;
        t = (lin & 7) * per + j;
    }
    if (t >= valid) return false;
    if (mode == 1) {
        ti.ntile = t / mt_sh;
        ti.g = a.E, ti.m0 = (t % mt_sh) * BM, ti.n = a.T, ti.row0 = 0, ti.shared = true;
        return true;
    }
    // Tiles of one group are contiguous: t / gy lies inside t's group.
    const int ie = t / gy;
    const int f = a.tiles[4 * ie + 2], mt = a.tiles[4 * ie + 3];
    const int local = t - f * gy;
    const int i = f + local % mt;
    ti.ntile = local / mt;
    const int g = a.tiles[4 * i];
    if (g >= a.E) return false;
    ti.g = g, ti.m0 = a.tiles[4 * i + 1], ti.n = a.counts[g], ti.row0 = a.offsets[g], ti.shared = false;
    return true;
}

template <int DT, bool UP>
__global__ __launch_bounds__(256, 2) void mfma_kernel(MfmaArgs a, int mode, int gx, int ksplit) {
    constexpr int REC = Fmt<DT>::rec;
    constexpr int BREC = 2 * REC + 1;  // dwords per weight row per step (+1 spreads banks)
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDA];
    __shared__ __attribute__((aligned(16))) uint32_t Bs[2][BW * BREC];
    __shared__ int src_row[BM];
    __shared__ int dst_row[BM];

    TileInfo ti;
    if (!tile_of(a, mode, gx, ti)) return;
    const ExpertDev &ex = a.experts[ti.g];
    const MatDev &W0 = UP ? ex.m[0] : ex.m[2];
    const MatDev &W1 = UP ? ex.m[1] : ex.m[2];
    const int n0 = ti.ntile * (UP ? BW / 2 : BW);  // first gate row (up) or output column (down)
    if (n0 >= W0.rows) return;
    const int Ktot = W0.cols;
    const int kspan = Ktot / ksplit;  // a multiple of BK (checked on the host)
    const int kbeg = ti.ksplit * kspan, kend = kbeg + kspan;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int Icol = ti.shared ? a.I_s : a.I;
    const int valid = min(BM, ti.n - ti.m0);

    if (tid < BM) {
        int s = -1, d = -1;
        if (tid < valid) {
            d = ti.row0 + ti.m0 + tid;
            s = UP ? (ti.shared ? ti.m0 + tid : a.perm_tok[d]) : d;
        }
        src_row[tid] = s;
        dst_row[tid] = d;
    }
    __syncthreads();

    // ---- staging: thread -> A row am, 32-value block ab of the step; weight
    //      row bn (LDS row; up: gate rows 0..127, up rows 128..255), both
    //      blocks of the step.  Every thread issues the same loads on every
    //      step (rows past the end read row 0 and are zeroed when stored), so
    //      each wait for a step's data counts exactly the loads after it.
    const int am = tid >> 1, ab = tid & 1;
    const int arow = src_row[am];
    const bool avalid = arow >= 0;
    const uint16_t *abase = UP ? a.xh + (size_t)(avalid ? arow : src_row[0]) * a.H
                               : (ti.shared ? a.hs : a.h) + (size_t)(avalid ? arow : src_row[0]) * Icol;
    const int bn = tid;
    const MatDev &WB = (UP && bn >= BW / 2) ? W1 : W0;
    const int brow = UP ? n0 + (bn & (BW / 2 - 1)) : n0 + bn;
    const bool bvalid = brow < WB.rows;
    const uint8_t *browp = WB.ptr + (size_t)(bvalid ? brow : 0) * WB.stride;

    // Global loads are held as raw dwords and normalised when stored to LDS.
    constexpr int FD = Fmt<DT>::fetch;
    constexpr int FQ = Codes<DT>::n;
    u32x4a areg[4];
    uint32_t braw[2][FD];
    auto load_step = [&](int k0, u32x4a (&ar)[4], uint32_t (&br)[2][FD]) {
        const int kc = k0 < kend ? k0 : kbeg;  // past the end: a harmless reload
        const u32x4a *src = reinterpret_cast<const u32x4a *>(abase + kc + 32 * ab);
#pragma unroll
        for (int i = 0; i < 4; i++) ar[i] = gload(src + i);
#pragma unroll
        for (int bb = 0; bb < 2; bb++) fetch_raw<DT>(browp, kc / 32 + bb, br[bb]);
    };
    // Chunk c of a 32-value block holds elements 8c..8c+7; its two halves go
    // to the K-permuted slots 16 (c & 1) + 4 (c >> 1) and that + 8.  Block bb
    // of a step has parity bb (k0 / 32 is even), so it starts 2 bytes into
    // its first dword exactly when bb == 1.
    auto store_step = [&](int buf, const u32x4a (&ar)[4], const uint32_t (&br)[2][FD]) {
        _Float16 *arow_lds = &As[buf][am * LDA + 32 * ab];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int p0 = 16 * (c & 1) + 4 * (c >> 1);
            const u32x4a v = avalid ? ar[c] : u32x4a{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x2a *>(arow_lds + p0) = u32x2a{v.x, v.y};
            *reinterpret_cast<u32x2a *>(arow_lds + p0 + 8) = u32x2a{v.z, v.w};
        }
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            uint32_t rec[REC];
            normalise<DT>(br[bb], bb == 1, rec);
            if (!bvalid) rec[0] = 0u;  // scale 0: a zero weight row
            uint32_t *brow_lds = &Bs[buf][bn * BREC + bb * REC];
#pragma unroll
            for (int i = 0; i < REC; i++) brow_lds[i] = rec[i];
        }
    };

    // Wave wv owns all 128 tokens and two 32-column tiles j: up -> gate rows
    // 32 wv .. +32 (j = 0) and the same up rows (j = 1); down -> output
    // columns 64 wv + 32 j .. +32.  Each V_MFMA_F32_32X32X16_F16 takes A lane
    // l = row l % 32, K slots 8 (l / 32) .. +8 and B lane l = column l % 32,
    // the same K slots; D lane l element v = row 8 (v / 4) + 4 (l / 32) + v % 4,
    // column l % 32.  Within a 32-value block, MFMA m covers permuted slots
    // 16 m .. 16 m + 15, so lane half h reads slot group q = 2 m + h: the
    // eight codes of dword q.  An activation fragment feeds two MFMAs (j), a
    // dequantised weight fragment the MT 32-token tiles.
    floatx16 acc[4][2];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[t][j] = floatx16{};
    const int l32 = lane & 31, hf = lane >> 5;
    int bcol[2];
#pragma unroll
    for (int j = 0; j < 2; j++) bcol[j] = UP ? (128 * j + 32 * wv + l32) : (64 * wv + 32 * j + l32);

    // The K loop for MT live 32-token tiles (chosen once per block).
    auto run = [&](auto mt_c) {
        constexpr int MT = decltype(mt_c)::value;
        // A step is four fragment groups g = (kb, m): group g + 1's
        // activation fragments and weight codes are read from LDS while group
        // g's MFMAs run.
        auto compute = [&](int buf) {
            half8 af[2][MT];
            uint32_t bsc[2][2], bq[2][2][FQ];
            auto read_group = [&](int g, half8 (&A)[MT], uint32_t (&sc)[2], uint32_t (&bqv)[2][FQ]) {
                const int kb = g >> 1, q = 2 * (g & 1) + hf;
#pragma unroll
                for (int t = 0; t < MT; t++)
                    A[t] = *reinterpret_cast<const half8 *>(&As[buf][(32 * t + l32) * LDA + 32 * kb + 8 * q]);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t *rec = &Bs[buf][bcol[j] * BREC + kb * REC];
                    sc[j] = rec[0];
                    rec_codes<DT>(rec, q, bqv[j]);
                }
            };
            read_group(0, af[0], bsc[0], bq[0]);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int c = g & 1;
                if (g + 1 < 4) read_group(g + 1, af[c ^ 1], bsc[c ^ 1], bq[c ^ 1]);
                // keep those reads ahead of this group's MFMAs
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const half8 bf = dequant_codes<DT>(bsc[c][j], bq[c][j], 2 * (g & 1) + hf);
#pragma unroll
                    for (int t = 0; t < MT; t++)
                        acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][t], bf, acc[t][j], 0, 0, 0);
                }
            }
        };
        // Double buffering: step s + 1's loads are issued before step s's
        // MFMAs and stored to the other LDS buffer after them.
        load_step(kbeg, areg, braw);
        store_step(0, areg, braw);
        __syncthreads();
        const int nsteps = (kend - kbeg) / BK;
        for (int st = 0; st + 1 < nsteps; st++) {
            load_step(kbeg + (st + 1) * BK, areg, braw);
            compute(st & 1);
            store_step((st + 1) & 1, areg, braw);
            __syncthreads();
        }
        compute((nsteps - 1) & 1);
    };
    const int mt = (valid + 31) / 32;
    switch (mt) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 4>{}); break;
    }

    // ---- epilogue: lane holds C[32 t + 8 (v / 4) + 4 hf + v % 4][bcol[j]].
    if (UP) {
        uint16_t *hout = ti.shared ? a.hs : a.h;
        const int col = n0 + 32 * wv + l32;
        if (col < W0.rows) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t >= mt) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int d = dst_row[32 * t + 8 * (v / 4) + 4 * hf + (v % 4)];
                    if (d < 0) continue;
                    const float g = acc[t][0][v], u = acc[t][1][v];
                    const float hv = (g / (1.0f + __expf(-g))) * u;
                    hout[(size_t)d * Icol + col] = __half_as_ushort(__float2half_rn(hv));
                }
            }
        }
    } else {
        float *yout = ti.shared ? a.ys + ti.ksplit * a.yspart : a.y + ti.ksplit * a.ypart;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + 64 * wv + 32 * j + l32;
            if (col >= W0.rows) continue;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t >= mt) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int d = dst_row[32 * t + 8 * (v / 4) + 4 * hf + (v % 4)];
                    if (d >= 0) yout[(size_t)d * a.H + col] = acc[t][j][v];
                }
            }
        }
    }
}

template <bool UP>
hipError_t launch_dt(int dt, dim3 grid, const MfmaArgs &a, int mode, int ksplit, hipStream_t s) {
    const int gx = (int)grid.x;
    switch (dt) {
    case MOE_DT_Q8_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q8_0, UP>), grid, dim3(256), 0, s, a, mode, gx, ksplit); break;
    case MOE_DT_Q4_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q4_0, UP>), grid, dim3(256), 0, s, a, mode, gx, ksplit); break;
    case MOE_DT_Q5_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q5_0, UP>), grid, dim3(256), 0, s, a, mode, gx, ksplit); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

int mfma_tile_m() { return BM; }

bool mfma_format_ok(int dt) { return dt == MOE_DT_Q4_0 || dt == MOE_DT_Q5_0 || dt == MOE_DT_Q8_0; }

// Split K of the down projection (2 or 4 parts) when its grid would leave
// CUs idle: the fewest parts that give about two blocks per CU.
int mfma_down_ksplit(int m_tiles, int n_rows, int K, int K_shared) {
    const long long blocks = (long long)m_tiles * ((n_rows + BW - 1) / BW);
    int ks = 1;
    while (ks < kMaxKSplit && blocks * ks < 512) ks *= 2;
    while (ks > 1 && (K % (ks * BK) != 0 || (K_shared > 0 && K_shared % (ks * BK) != 0))) ks /= 2;
    return ks;
}

hipError_t launch_mfma(bool up, const MfmaArgs &a, int /*bm*/, const ExpertDev &e0, const ExpertDev *sh,
                       hipStream_t s) {
    const MatDev &m = up ? e0.m[0] : e0.m[2];
    const int cols = up ? BW / 2 : BW;
    const int ks = up ? 1 : a.ksplit;
    dim3 grid(a.max_tiles, (m.rows + cols - 1) / cols, ks);
    hipError_t err = up ? launch_dt<true>(m.dt, grid, a, 0, ks, s) : launch_dt<false>(m.dt, grid, a, 0, ks, s);
    if (err != hipSuccess || !sh) return err;
    const MatDev &ms = up ? sh->m[0] : sh->m[2];
    dim3 gs((a.T + BM - 1) / BM, (ms.rows + cols - 1) / cols, ks);
    return up ? launch_dt<true>(ms.dt, gs, a, 1, ks, s) : launch_dt<false>(ms.dt, gs, a, 1, ks, s);
}

}  // namespace moe
