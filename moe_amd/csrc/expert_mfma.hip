// expert_mfma.hip — grouped SwiGLU expert GEMMs on gfx950 matrix cores.
//
// One block computes a tile of up to 160 tokens x 256 weight rows of one
// expert:
//   up   : 128 gate rows and the same 128 up rows of the expert, K = H; the
//          epilogue forms h = silu(G) * U and stores it as f16.
//   down : 256 rows of W_down, K = I (optionally split into 2 or 4 K parts,
//          each written to its own part of y); output y in f32.
// Four waves, one per SIMD.  Wave w owns every token row of the tile and 64
// weight rows, so each weight value is dequantised exactly once per tile, in
// the registers of the wave that multiplies it (f16, d * q rounded once), and
// the 160 x 64 f32 accumulators live in the wave's AGPRs
// (V_MFMA_F32_32X32X16_F16).  An expert's tokens normally fit one tile, so a
// weight row is dequantised once per expert.  160 tokens (not more) leaves
// LDS room for a deep ring: a step multiplies in ~0.4 us while a weight load
// from HBM takes ~2 us under load, so loads run several steps ahead.
//
// Operands reach LDS by DMA (global_load_lds), never through VGPRs:
//   activations  16-byte chunks of each token row; the chunk index is XORed
//                with the row's low three bits, so the 16-byte fragment reads
//                of eight consecutive rows hit eight different bank groups;
//   weights      the raw bytes of two quantised blocks per row per K step, in
//                per-wave regions (32 rows each) that only the owning wave
//                reads.
// An NS-stage ring (5 stages for Q4_0, 4 for Q5_0/Q8_0: as many as LDS
// holds) keeps the loads of NS - 1 K steps in flight behind the step being
// multiplied.  The DMAs are issued from inline assembly, because the
// compiler makes every LDS read that follows an LDS DMA wait for all
// outstanding loads; the kernel instead waits with exact vmcnt counts: in the
// middle of step s a wave waits for its own loads of step s + 1 and
// dequantises that step's first block ahead of time, and one barrier per step
// publishes the other waves' activation chunks.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gmem.h"
#include "moe_internal.h"

namespace moe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 160;              // tokens per tile
constexpr int MTMAX = BM / 32;       // 32-token MFMA tiles per block tile
constexpr int BW = 256;              // weight rows per tile (up: 128 gate + 128 up rows)
constexpr int BK = 64;               // K values per step (two 32-value blocks)
constexpr int A_STAGE = BM * BK * 2;  // bytes of activations per stage

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
__device__ inline half8 pack8(const uint32_t (&o)[4]) {
    half8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

// Bytes of one 32-value block, and dwords per weight row per K step (two
// blocks; a row's step always starts 4-byte aligned since K % 64 == 0).
template <int DT>
struct Fmt;
template <>
struct Fmt<MOE_DT_Q4_0> {
    static constexpr int bytes = 18, rd = 9;
};
template <>
struct Fmt<MOE_DT_Q5_0> {
    static constexpr int bytes = 22, rd = 11;
};
template <>
struct Fmt<MOE_DT_Q8_0> {
    static constexpr int bytes = 34, rd = 17;
};
// Weight DMA.  A row's step (rd dwords) is split into nx4 16-byte lanes
// (dwords 0 .. 4 nx4 - 1) and nd dword lanes (the rest).  One 32-row region
// is laid out as
//   X part  lane q = 32 x + r  (x < nx4) at 16 q: dwords 4x .. 4x+3 of row r
//   D part  lane q = 32 e + r  (e < nd)  at X + 4 q: dword 4 nx4 + e of row r
// and filled by nx4 / 2 dwordx4 DMAs plus ceil(nd / 2) dword DMAs (lanes
// past nd load row 0 into the padding at the region's end).  Dword d of row
// r of the region therefore sits at loc(d, r) below.
template <int DT>
struct BLay {
    static constexpr int rd = Fmt<DT>::rd;
    static constexpr int nx4 = rd / 4;             // 2, 2, 4 (even)
    static constexpr int nd = rd - 4 * nx4;        // 1, 3, 1
    static constexpr int ix = nx4 / 2;             // dwordx4 DMAs per region
    static constexpr int id = (nd + 1) / 2;        // dword DMAs per region
    static constexpr int inst = ix + id;
    static constexpr int xbytes = 512 * nx4;
    static constexpr int region = xbytes + 256 * id;  // bytes
    static constexpr int stage = 8 * region;
    static_assert(nx4 % 2 == 0, "whole dwordx4 DMAs per region");
    __device__ static constexpr uint32_t loc(int d, int r) {
        return d < 4 * nx4 ? (uint32_t)(512 * (d >> 2) + 16 * r + 4 * (d & 3))
                           : (uint32_t)(xbytes + 128 * (d - 4 * nx4) + 4 * r);
    }
};
// Ring stages per format: as many as fit in the 160 KiB of LDS.
template <int DT>
constexpr int ring_stages() {
    return (160 * 1024 - 2 * BM * 4) / (A_STAGE + BLay<DT>::stage);
}
template <int DT>
constexpr int lds_bytes() {
    return ring_stages<DT>() * (A_STAGE + BLay<DT>::stage) + 2 * BM * 4;
}
static_assert(ring_stages<MOE_DT_Q4_0>() == 5 && ring_stages<MOE_DT_Q5_0>() == 4 &&
                  ring_stages<MOE_DT_Q8_0>() == 4,
              "ring depth per format");
static_assert(lds_bytes<MOE_DT_Q4_0>() <= 160 * 1024 && lds_bytes<MOE_DT_Q5_0>() <= 160 * 1024 &&
                  lds_bytes<MOE_DT_Q8_0>() <= 160 * 1024,
              "LDS budget");

// ---- LDS DMA and exact waits ------------------------------------------------
// global_load_lds writes lane l's 16 (or 4) bytes to LDS address m0 + 16 l
// (4 l); lanes with EXEC clear write nothing.  Addresses are an SGPR base
// plus a 32-bit VGPR offset; the base and the LDS address are wave-uniform
// (readfirstlane states that to the compiler, which may not prove it).
//
// The compiler cannot see that the assembly below is a vector memory load
// that reads an SGPR base and M0, so it would not insert the wait states the
// hardware needs between a VALU write of an SGPR (v_readfirstlane) and a
// vector memory instruction reading it (5), or between an M0 write and an
// LDS DMA (1).  The assembly therefore copies the base with s_mov_b64 (a
// scalar read, which the hardware interlocks) into SGPRs that nothing but
// scalar instructions ever wrote, and pads one wait state after the copy.
__device__ inline const void *uniform_ptr(const void *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const void *>(lo | (hi << 32));
}
__device__ inline void dma16(const void *base, uint32_t off, uint32_t lds) {
    uint64_t sb;
    asm volatile(
        "s_mov_b64 %0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %0"
        : "=&s"(sb)
        : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane((int)lds))
        : "memory");
}
__device__ inline void dma4(const void *base, uint32_t off, uint32_t lds) {
    uint64_t sb;
    asm volatile(
        "s_mov_b64 %0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, %0"
        : "=&s"(sb)
        : "v"(off), "s"(uniform_ptr(base)), "{m0}"(__builtin_amdgcn_readfirstlane((int)lds))
        : "memory");
}
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Wait for all but the newest N of this wave's loads and for its LDS reads,
// then meet the other waves.
template <int N>
__device__ inline void wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
typedef const __attribute__((address_space(3))) uint8_t *lds_p;
typedef uint32_t u32x4l __attribute__((ext_vector_type(4)));
__device__ inline uint32_t lds_u32(lds_p p) { return *(const __attribute__((address_space(3))) uint32_t *)p; }
__device__ inline half8 lds_h8(lds_p p) { return *(const __attribute__((address_space(3))) half8 *)p; }

// ---- weight fragments -----------------------------------------------------
// Lane (l32, h) of a wave reads row l32 of a 32-row region.  For K group
// (block kb, MFMA m) the MFMA takes elements 16 m + 8 h .. + 7 of block kb in
// natural order; both MFMAs of a block use the same eight code bytes
// 8 h .. 8 h + 7 of the block's code array (Q4_0/Q5_0: low nibbles for m = 0,
// high nibbles for m = 1), Q8_0 bytes 16 m + 8 h .. + 7.  Slots<DT> lists the
// row dwords a lane reads for block kb: dword base + 2 h * hm; their LDS
// offsets are computed once per lane.  dequant turns the dwords (v, in slot
// order) into the block's two MFMA operands.
template <int DT>
struct Slots;
template <>
struct Slots<MOE_DT_Q4_0> {  // kb 0: bytes 0..17 (scale, codes 2..17); kb 1: bytes 18..35
    static constexpr int n[2] = {4, 3};
    static constexpr int base[2][7] = {{0, 0, 1, 2}, {4, 5, 6}};
    static constexpr int hm[2][7] = {{0, 1, 1, 1}, {0, 1, 1}};
};
template <>
struct Slots<MOE_DT_Q5_0> {  // kb 0: scale 0..1, qh 2..5, codes 6..21; kb 1: scale 22..23, qh 24..27, codes 28..43
    static constexpr int n[2] = {5, 4};
    static constexpr int base[2][7] = {{0, 1, 1, 2, 3}, {5, 6, 7, 8}};
    static constexpr int hm[2][7] = {{0, 0, 1, 1, 1}, {0, 0, 1, 1}};
};
template <>
struct Slots<MOE_DT_Q8_0> {  // kb 0: scale 0..1, codes 2..33; kb 1: scale 34..35, codes 36..67
    static constexpr int n[2] = {7, 5};
    static constexpr int base[2][7] = {{0, 0, 1, 2, 4, 5, 6}, {8, 9, 10, 13, 14}};
    static constexpr int hm[2][7] = {{0, 1, 1, 1, 1, 1, 1}, {0, 1, 1, 1, 1}};
};

template <int DT, int KB>
__device__ inline void dequant(const uint32_t *v, half8 (&b)[2], int h) {
    const uint32_t s = KB == 0 ? (v[0] & 0xffffu) : (v[0] >> 16);
    const __half2 d2 = as_h2(s * 0x10001u);
    uint32_t o[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        const uint32_t w0 = KB == 0 ? alignb(v[2], v[1], 2) : v[1];
        const uint32_t w1 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        codes4(w0 & 0x0f0f0f0fu, off2, d2, o[0], o[1]);
        codes4(w1 & 0x0f0f0f0fu, off2, d2, o[2], o[3]);
        b[0] = pack8(o);
        codes4((w0 >> 4) & 0x0f0f0f0fu, off2, d2, o[0], o[1]);
        codes4((w1 >> 4) & 0x0f0f0f0fu, off2, d2, o[2], o[3]);
        b[1] = pack8(o);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        const uint32_t qh = KB == 0 ? alignb(v[1], v[0], 2) : v[1];
        const uint32_t w0 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        const uint32_t w1 = KB == 0 ? alignb(v[4], v[3], 2) : v[3];
        const uint32_t hb = qh >> (8 * h);  // bit i: element 8 h + i; bit 16 + i: element 16 + 8 h + i
        codes4((w0 & 0x0f0f0f0fu) | spread4(hb & 0xfu), off2, d2, o[0], o[1]);
        codes4((w1 & 0x0f0f0f0fu) | spread4((hb >> 4) & 0xfu), off2, d2, o[2], o[3]);
        b[0] = pack8(o);
        codes4(((w0 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 16) & 0xfu), off2, d2, o[0], o[1]);
        codes4(((w1 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 20) & 0xfu), off2, d2, o[2], o[3]);
        b[1] = pack8(o);
    } else {  // Q8_0: int8 codes, read as uint8 + 128
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const uint32_t *c = v + 1 + (KB == 0 ? 3 : 2) * m;
            const uint32_t w0 = KB == 0 ? alignb(c[1], c[0], 2) : c[0];
            const uint32_t w1 = KB == 0 ? alignb(c[2], c[1], 2) : c[1];
            codes4(w0 ^ 0x80808080u, off2, d2, o[0], o[1]);
            codes4(w1 ^ 0x80808080u, off2, d2, o[2], o[3]);
            b[m] = pack8(o);
        }
    }
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
    // Routed tiles come first in the tile list, the shared expert's last; a
    // launch walks only its own (at most gx of them, so valid <= total).
    const int valid = mode == 1 ? mt_sh * gy : (a.ntiles[0] - a.shared_tiles) * gy;
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
__global__ __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void mfma_kernel(MfmaArgs a, int mode, int gx, int ksplit) {
    using BL = BLay<DT>;
    constexpr int NS = ring_stages<DT>();
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int *src_row = reinterpret_cast<int *>(smem + NS * (A_STAGE + BL::stage));
    int *dst_row = src_row + BM;

    TileInfo ti;
    if (!tile_of(a, mode, gx, ti)) return;
    const ExpertDev &ex = a.experts[ti.g];
    const MatDev &W0 = UP ? ex.m[0] : ex.m[2];
    const MatDev &W1 = UP ? ex.m[1] : ex.m[2];
    const int n0 = ti.ntile * (UP ? BW / 2 : BW);  // first gate row (up) or output column (down)
    if (n0 >= W0.rows) return;
    const int Ktot = W0.cols;
    const int kspan = Ktot / ksplit;  // a multiple of BK (checked on the host)
    const int kbeg = ti.ksplit * kspan;
    const int nsteps = kspan / BK;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int Icol = ti.shared ? a.I_s : a.I;
    const int valid = min(BM, ti.n - ti.m0);
    const int mt = (valid + 31) / 32;

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

    const uint32_t lds0 = lds_addr(smem);
    const uint32_t ldsB = lds0 + NS * A_STAGE;
    const lds_p sm = (lds_p)smem;
    const int l32 = lane & 31, hf = lane >> 5;

    // Activation DMA: instruction u of wave wv covers rows 8 i .. 8 i + 7,
    // i = wv + 4 u; lane l takes row r = 8 i + l / 8 and stores slot l % 8 of
    // that row's 128 bytes, which holds logical chunk (l % 8) ^ ((r / 2) % 8).
    // Rows past the tile's tokens repeat token row 0 (their outputs are never
    // stored).
    const uint8_t *abase = reinterpret_cast<const uint8_t *>(UP ? a.xh : (ti.shared ? a.hs : a.h));
    const uint32_t arow_bytes = (uint32_t)(UP ? a.H : Icol) * 2;
    // Weight DMA: region j of wave wv holds 32 weight rows.  woff: per DMA
    // (the region's dwordx4 DMAs, then its dword DMAs) the lane's byte offset
    // in the weight matrix, without the step's K offset.
    const uint8_t *wbase[2];
    uint32_t woff[2][BL::inst];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const MatDev &W = (UP && j == 1) ? W1 : W0;
        wbase[j] = W.ptr;
        const int row0 = UP ? n0 + 32 * wv : n0 + 64 * wv + 32 * j;
        int row = row0 + (lane & 31);
        if (row >= W.rows) row = 0;
#pragma unroll
        for (int i = 0; i < BL::inst; i++) {
            const int q = 64 * (i < BL::ix ? i : i - BL::ix) + lane;  // lane within the part
            uint32_t off;
            if (i < BL::ix) {
                off = (uint32_t)row * W.stride + 16u * (uint32_t)(q >> 5);
            } else {
                const int e = q >> 5;
                off = e < BL::nd ? (uint32_t)row * W.stride + (uint32_t)(16 * BL::nx4 + 4 * e) : 0u;
            }
            woff[j][i] = off;
        }
    }

    // Per-lane LDS offsets of the compute side.
    uint32_t aoff[4];  // group g = 2 kb + m: row l32, logical chunk 2 g + hf
#pragma unroll
    for (int g = 0; g < 4; g++) aoff[g] = (uint32_t)l32 * 128u + ((uint32_t)((2 * g + hf) ^ ((l32 >> 1) & 7)) << 4);
    using SL = Slots<DT>;
    const uint32_t brow_x = 16u * l32;                 // row l32's X part within a region
    const uint32_t brow_d = BL::xbytes + 4u * l32;     // and its D part

    floatx16 acc[MTMAX][2];
#pragma unroll
    for (int t = 0; t < MTMAX; t++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[t][j] = floatx16{};

    auto run = [&](auto mt_c) {
        constexpr int MT = decltype(mt_c)::value;
        constexpr int NB = 2 * BL::inst;  // weight DMAs per wave per step
        constexpr int ND = MT + NB;       // DMAs per wave per step
        uint32_t aoffg[MT];               // activation source offsets (step 0)
#pragma unroll
        for (int u = 0; u < MT; u++) {
            const int r = 8 * (wv + 4 * u) + (lane >> 3);
            const int sr = src_row[r < valid ? r : 0];
            aoffg[u] = (uint32_t)sr * arow_bytes + (uint32_t)kbeg * 2u +
                       (uint32_t)(((lane & 7) ^ ((r >> 1) & 7)) << 4);
        }
        // DMA d of step `step` into ring stage `st`: d < MT activations, then
        // the weight regions.  Steps past the end reload the last step into a
        // stage nobody reads any more, so every step issues the same DMAs.
        auto dma = [&](auto d_c, int step, int st) {
            constexpr int d = decltype(d_c)::value;
            const int sc = step < nsteps ? step : nsteps - 1;
            if constexpr (d < MT) {
                dma16(abase + (size_t)sc * (BK * 2), aoffg[d],
                      lds0 + (uint32_t)st * A_STAGE + (uint32_t)(wv + 4 * d) * 1024u);
            } else {
                constexpr int j = (d - MT) / BL::inst, i = (d - MT) % BL::inst;
                const uint8_t *wb = wbase[j] + (size_t)(kbeg / 32 + 2 * sc) * Fmt<DT>::bytes;
                const uint32_t lr = ldsB + (uint32_t)st * BL::stage + (uint32_t)(2 * wv + j) * BL::region;
                if constexpr (i < BL::ix)
                    dma16(wb, woff[j][i], lr + 1024u * i);
                else
                    dma4(wb, woff[j][i], lr + BL::xbytes + 256u * (i - BL::ix));
            }
        };
        auto dma_from = [&](auto lo_c, auto hi_c, int step, int st, auto self) {
            constexpr int lo = decltype(lo_c)::value, hi = decltype(hi_c)::value;
            if constexpr (lo < hi) {
                dma(std::integral_constant<int, lo>{}, step, st);
                self(std::integral_constant<int, lo + 1>{}, hi_c, step, st, self);
            }
        };
        auto dma_range = [&](auto lo_c, auto hi_c, int step, int st) { dma_from(lo_c, hi_c, step, st, dma_from); };

        // Row l32's whole step (rd dwords) of both regions, read with 16-byte
        // LDS reads (both lane halves read the same row, which the LDS
        // broadcasts); each lane then picks its dwords (Slots: base, or
        // base + 2 for the upper lane half).
        half8 bq[2][2][2];  // [kb][j][m]
        half8 af[4][MT];    // one per group, read two groups ahead
        uint32_t rowv[2][BL::rd];
        auto read_rows = [&](lds_p stage_b) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t reg = (uint32_t)(2 * wv + j) * BL::region;
#pragma unroll
                for (int x = 0; x < BL::nx4; x++) {
                    const u32x4l v =
                        *(const __attribute__((address_space(3))) u32x4l *)(stage_b + reg + brow_x + 512 * x);
                    rowv[j][4 * x] = v.x, rowv[j][4 * x + 1] = v.y, rowv[j][4 * x + 2] = v.z, rowv[j][4 * x + 3] = v.w;
                }
#pragma unroll
                for (int e = 0; e < BL::nd; e++)
                    rowv[j][4 * BL::nx4 + e] = lds_u32(stage_b + reg + brow_d + 128 * e);
            }
        };
        auto dequant_raw = [&](auto kb_c, half8 (&B)[2][2]) {
            constexpr int kb = decltype(kb_c)::value;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                uint32_t v[7];
#pragma unroll
                for (int k = 0; k < SL::n[kb]; k++) {
                    const int b = SL::base[kb][k];
                    v[k] = SL::hm[kb][k] ? (hf ? rowv[j][b + 2] : rowv[j][b]) : rowv[j][b];
                }
                dequant<DT, kb>(v, B[j], hf);
            }
        };
        auto read_a = [&](lds_p sa, int g, half8 (&A)[MT]) {
            const lds_p p = sa + aoff[g];
#pragma unroll
            for (int t = 0; t < MT; t++) A[t] = lds_h8(p + 4096 * t);
        };
        auto mfma = [&](const half8 (&A)[MT], const half8 (&B)[2][2], int m, int i) {
            const int t = i >> 1, j = i & 1;
            acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[t], B[j][m], acc[t][j], 0, 0, 0);
        };
        // One group's 2 MT MFMAs with DMAs [LO, HI) of step `step` spread
        // between them: a DMA that the memory pipeline cannot take yet stalls
        // this wave, not the MFMAs already queued.
        auto mfmas_dma = [&](const half8 (&A)[MT], const half8 (&B)[2][2], int m, auto lo_c, auto hi_c, int step,
                             int st) {
            constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
            auto body = [&](auto i_c, auto self) {
                constexpr int i = decltype(i_c)::value;
                if constexpr (i < 2 * MT) {
                    mfma(A, B, m, i);
                    dma_range(std::integral_constant<int, LO + i * (HI - LO) / (2 * MT)>{},
                              std::integral_constant<int, LO + (i + 1) * (HI - LO) / (2 * MT)>{}, step, st);
                    self(std::integral_constant<int, i + 1>{}, self);
                }
            };
            body(std::integral_constant<int, 0>{}, body);
        };
        auto mfmas = [&](const half8 (&A)[MT], const half8 (&B)[2][2], int m) {
#pragma unroll
            for (int i = 0; i < 2 * MT; i++) mfma(A, B, m, i);
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        constexpr int MA = MT / 2;  // activation DMAs in group 0; the rest in group 1

        const lds_p smB = sm + NS * A_STAGE;
        // Prologue: steps 0 .. NS - 2 into stages 0 .. NS - 2, then wait for
        // step 0.
        for (int p = 0; p < NS - 1; p++) dma_range(I0{}, std::integral_constant<int, ND>{}, p, p);
        wait_vm_barrier<(NS - 2) * ND>();
        read_a(sm, 0, af[0]);
        read_a(sm, 1, af[1]);
        read_rows(smB);
        dequant_raw(I0{}, bq[0]);
        int st = 0;
        // Per step, this wave's loads of step s + NS - 1 go out in order: the
        // activation DMAs in groups 0 and 1, the weight DMAs in group 3, into
        // the stage step s - 1 used.  At the wait in group 2 this wave's
        // outstanding loads are those of steps s + 1 .. s + NS - 2 (ND each)
        // and the MT activation DMAs of step s + NS - 1; leaving all but step
        // s + 1's outstanding completes step s + 1.
        constexpr int WAIT = (NS - 3) * ND + MT;
        static_assert((NS - 1) * ND < 64 && WAIT >= 0, "vmcnt range");
        for (int s = 0; s < nsteps; s++) {
            const lds_p sa = sm + st * A_STAGE;
            const int st1 = st + 1 == NS ? 0 : st + 1, stn = st == 0 ? NS - 1 : st - 1;
            const int sn = s + NS - 1;
            // g = 0 (kb 0, m 0): group 2's activations first.
            read_a(sa, 2, af[2]);
            __builtin_amdgcn_sched_barrier(0);
            mfmas_dma(af[0], bq[0], 0, I0{}, std::integral_constant<int, MA>{}, sn, stn);
            // g = 1 (kb 0, m 1): dequantise block 1, read group 3.
            dequant_raw(I1{}, bq[1]);
            read_a(sa, 3, af[3]);
            mfmas_dma(af[1], bq[0], 1, std::integral_constant<int, MA>{}, std::integral_constant<int, MT>{}, sn, stn);
            __builtin_amdgcn_sched_barrier(0);
            // g = 2 (kb 1, m 0); then wait for this wave's loads of step
            // s + 1 and meet the other waves, after which step s + 1's stage
            // is complete and nobody reads stage s any more.
            mfmas(af[2], bq[1], 0);
            __builtin_amdgcn_sched_barrier(0);
            wait_vm_barrier<WAIT>();
            __builtin_amdgcn_sched_barrier(0);
            // g = 3 (kb 1, m 1): step s + 1's groups 0 and 1 and weight
            // rows; step s + NS - 1's weight DMAs.
            const lds_p sa1 = sm + st1 * A_STAGE;
            read_a(sa1, 0, af[0]);
            read_a(sa1, 1, af[1]);
            read_rows(smB + st1 * BL::stage);
            __builtin_amdgcn_sched_barrier(0);
            mfmas_dma(af[3], bq[1], 1, std::integral_constant<int, MT>{}, std::integral_constant<int, ND>{}, sn, stn);
            dequant_raw(I0{}, bq[0]);
            __builtin_amdgcn_sched_barrier(0);
            st = st1;
        }
    };
    static_assert(MTMAX == 5, "one case per 32-token tile count");
    switch (mt) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    case 4: run(std::integral_constant<int, 4>{}); break;
    default: run(std::integral_constant<int, 5>{}); break;
    }
    wait_vm<0>();

    // ---- epilogue: lane holds C[32 t + 8 (v / 4) + 4 hf + v % 4][column l32 of set j].
    if (UP) {
        uint16_t *hout = ti.shared ? a.hs : a.h;
        const int col = n0 + 32 * wv + l32;
        if (col < W0.rows) {
#pragma unroll
            for (int t = 0; t < MTMAX; t++) {
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
            for (int t = 0; t < MTMAX; t++) {
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

template <int DT, bool UP>
hipError_t launch_one(dim3 grid, const MfmaArgs &a, int mode, int ksplit, hipStream_t s) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_kernel<DT, UP>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes<DT>());
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((mfma_kernel<DT, UP>), grid, dim3(256), lds_bytes<DT>(), s, a, mode, (int)grid.x, ksplit);
    return hipGetLastError();
}

template <bool UP>
hipError_t launch_dt(int dt, dim3 grid, const MfmaArgs &a, int mode, int ksplit, hipStream_t s) {
    switch (dt) {
    case MOE_DT_Q8_0: return launch_one<MOE_DT_Q8_0, UP>(grid, a, mode, ksplit, s);
    case MOE_DT_Q4_0: return launch_one<MOE_DT_Q4_0, UP>(grid, a, mode, ksplit, s);
    case MOE_DT_Q5_0: return launch_one<MOE_DT_Q5_0, UP>(grid, a, mode, ksplit, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

int mfma_tile_m() { return BM; }

bool mfma_format_ok(int dt) { return dt == MOE_DT_Q4_0 || dt == MOE_DT_Q5_0 || dt == MOE_DT_Q8_0; }

// The kernels address activations and weight rows with 32-bit offsets.
bool mfma_fits(size_t t, size_t k, size_t H, size_t I, size_t I_s) {
    const size_t lim = (size_t)1 << 32;
    return t * H * 2 < lim && t * k * I * 2 < lim && t * I_s * 2 < lim;
}

// Split K of the down projection (2 or 4 parts) when its grid would leave
// CUs idle: the fewest parts that give every CU a block (one block fits per
// CU: the ring takes most of the LDS).  Each part is written separately and
// summed by the combine, so fewer parts also mean less traffic there.
int mfma_down_ksplit(int m_tiles, int n_rows, int K, int K_shared) {
    const long long blocks = (long long)m_tiles * ((n_rows + BW - 1) / BW);
    int ks = 1;
    while (ks < kMaxKSplit && blocks * ks < 256) ks *= 2;
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
