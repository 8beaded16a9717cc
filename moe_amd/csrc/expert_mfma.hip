// expert_mfma.hip — grouped SwiGLU expert GEMMs on gfx950 matrix cores, in
// f32 precision.
//
// One block computes a tile of up to BM tokens (160, or 128 when a Q8_0
// matrix needs the LDS) x 256 weight rows of one expert:
//   up   : 128 gate rows and the same 128 up rows of the expert, K = H; the
//          epilogue forms h = silu(G) * U in f32 (src/model.rs:31-33).
//   down : 256 rows of W_down, K = I (optionally split into 2 or 4 K parts,
//          each written to its own part of y); output y in f32.
// Four waves, one per SIMD (or eight, two per SIMD: SPLIT below).  Wave w
// owns every token row of the tile and 64 weight rows, so each weight value
// is decoded once per tile (per wave of a pair), in the registers of the
// wave that multiplies it, and the f32 accumulators of its tiles live in
// registers (V_MFMA_F32_32X32X16_F16).
//
// Precision.  The reference multiplies f32 activations by exactly
// dequantised f32 weights d q (src/quant.rs:482-506).  The default
// (two-pass) kernels carry the activations as two f16 pieces (below) and
// the weights as their codes q, exact in f16: per 32-value block, four
// MFMAs accumulate (hi + lo) q of both 16-value halves in f32 from zero,
// and the block's d (f32) adds that sum into the tile with one fma; the
// products are exact, so the activations' 22 bits bound the error.  The
// three-pass kernels (kept for measurement) carry both operands as two f16
// pieces and three MFMAs accumulate hi.hi + hi.lo + lo.hi in f32:
//   weights      d q has at most 18 significant bits (11 of d, 7 of q), so
//                hi = f16(d q) and lo = d q - hi (one fma, exact) hold it
//                exactly; d is first multiplied by 2^wexp (exact), the
//                matrix's power of two that puts its largest |d q| in
//                [2^14, 2^15), so lo stays in f16's normal range;
//   activations  split_rows_kernel writes hi + lo of v 2^ex, ex per row
//                putting the row's largest |v| in [2^14, 2^15): 22
//                significant bits (the dropped lo.lo term and the rounding
//                of lo are ~2^-22 of a product);
// the epilogue multiplies by 2^-(ex + wexp) (two-pass: 2^-ex), which is
// exact.  SwiGLU's
// sigmoid uses the hardware exp (v_exp_f32, about 1 ulp), as the other
// fast paths do; only routing needs glibc's expf bit for bit.
//
// Operands reach LDS by DMA (global_load_lds), never through VGPRs:
//   activations  16-byte chunks of each token row, for hi and lo alike; the
//                chunk index is XORed with the row's low three bits, so the
//                16-byte fragment reads of eight consecutive rows hit eight
//                different bank groups;
//   weights      the raw bytes of two quantised blocks per row per K step, in
//                per-wave regions (32 rows each) that only the owning wave
//                reads.
// A three-stage ring holds K steps s, s + 1 and s + 2; the loads of step
// s + 3 go out during step s, as soon as every wave is past its last read of
// step s's stage, so each load has about two steps (~2.5 us) to arrive.  The
// DMAs are issued from inline assembly, because the compiler makes every
// LDS read that follows an LDS DMA wait for all outstanding loads; the
// kernel instead waits with exact vmcnt counts, and one barrier per step
// publishes the other waves' activation chunks.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "gmem.h"
#include "lds_dma.h"
#include "mfma_tiles.h"
#include "moe_internal.h"

namespace moe {
namespace {

using namespace lds;
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BW = 256;  // weight rows per tile (up: 128 gate + 128 up rows)
constexpr int BK = 64;   // K values per step (two 32-value blocks)
// Bytes of one activation piece (hi or lo) of one ring stage.
template <int BM>
constexpr int a_stage() {
    return BM * BK * 2;
}

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

// Codes b0..b3 (bytes of v, each < 256) minus `off2`, times `d2`: the
// products as exact f16 pieces, hi (pairs (b0, b1), (b2, b3)) and lo.  0x64
// in the high byte makes each f16 exactly 1024 + b, so q = b - off is exact;
// hi = f16(q d) and lo = fma(q, d, -hi), which is exact because q d - hi fits
// in f16's 11 bits.
__device__ inline void codes4(uint32_t v, __half2 off2, __half2 d2, uint32_t &h01, uint32_t &h23, uint32_t &l01,
                              uint32_t &l23) {
    const __half2 q01 = __hsub2(as_h2(perm(0x64646464u, v, 0x04010400u)), off2);
    const __half2 q23 = __hsub2(as_h2(perm(0x64646464u, v, 0x04030402u)), off2);
    const __half2 p01 = __hmul2(q01, d2), p23 = __hmul2(q23, d2);
    h01 = h2_bits(p01), h23 = h2_bits(p23);
    l01 = h2_bits(__hfma2(q01, d2, __hneg2(p01)));
    l23 = h2_bits(__hfma2(q23, d2, __hneg2(p23)));
}
__device__ inline half8 pack8(const uint32_t (&o)[4]) {
    half8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

// Ring stages per format and token tile: as many as fit in the 160 KiB of
// LDS beside three per-row arrays.
template <int DT, int BM>
constexpr int ring_stages() {
    return (160 * 1024 - 3 * BM * 4) / (2 * a_stage<BM>() + BLay<DT>::stage);
}
template <int DT, int BM>
constexpr int lds_bytes() {
    return ring_stages<DT, BM>() * (2 * a_stage<BM>() + BLay<DT>::stage) + 3 * BM * 4;
}
static_assert(ring_stages<MOE_DT_Q4_0, 160>() == 3 && ring_stages<MOE_DT_Q5_0, 160>() == 3 &&
                  ring_stages<MOE_DT_Q8_0, 128>() == 3 && ring_stages<MOE_DT_Q4_0, 128>() == 3 &&
                  ring_stages<MOE_DT_Q5_0, 128>() == 3,
              "three-stage ring for every instantiated format and tile");
static_assert(ring_stages<MOE_DT_Q8_0, 160>() < 3, "Q8_0 takes 128-token tiles");


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

// Block kb's two MFMA operands (m = 0, 1) as hi and lo pieces; `wexp`
// scales the block's d by 2^wexp first (exact: a power of two).
template <int DT, int KB>
__device__ inline void dequant(const uint32_t *v, half8 (&bh)[2], half8 (&bl)[2], int h, int wexp) {
    const uint32_t s = KB == 0 ? (v[0] & 0xffffu) : (v[0] >> 16);
    const __half ds = __float2half_rn(ldexpf(__half2float(__ushort_as_half((unsigned short)s)), wexp));
    const __half2 d2 = __halves2half2(ds, ds);
    uint32_t oh[4], ol[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        const uint32_t w0 = KB == 0 ? alignb(v[2], v[1], 2) : v[1];
        const uint32_t w1 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        codes4(w0 & 0x0f0f0f0fu, off2, d2, oh[0], oh[1], ol[0], ol[1]);
        codes4(w1 & 0x0f0f0f0fu, off2, d2, oh[2], oh[3], ol[2], ol[3]);
        bh[0] = pack8(oh), bl[0] = pack8(ol);
        codes4((w0 >> 4) & 0x0f0f0f0fu, off2, d2, oh[0], oh[1], ol[0], ol[1]);
        codes4((w1 >> 4) & 0x0f0f0f0fu, off2, d2, oh[2], oh[3], ol[2], ol[3]);
        bh[1] = pack8(oh), bl[1] = pack8(ol);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        const uint32_t qh = KB == 0 ? alignb(v[1], v[0], 2) : v[1];
        const uint32_t w0 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        const uint32_t w1 = KB == 0 ? alignb(v[4], v[3], 2) : v[3];
        const uint32_t hb = qh >> (8 * h);  // bit i: element 8 h + i; bit 16 + i: element 16 + 8 h + i
        codes4((w0 & 0x0f0f0f0fu) | spread4(hb & 0xfu), off2, d2, oh[0], oh[1], ol[0], ol[1]);
        codes4((w1 & 0x0f0f0f0fu) | spread4((hb >> 4) & 0xfu), off2, d2, oh[2], oh[3], ol[2], ol[3]);
        bh[0] = pack8(oh), bl[0] = pack8(ol);
        codes4(((w0 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 16) & 0xfu), off2, d2, oh[0], oh[1], ol[0], ol[1]);
        codes4(((w1 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 20) & 0xfu), off2, d2, oh[2], oh[3], ol[2], ol[3]);
        bh[1] = pack8(oh), bl[1] = pack8(ol);
    } else {  // Q8_0: int8 codes, read as uint8 + 128
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const uint32_t *c = v + 1 + (KB == 0 ? 3 : 2) * m;
            const uint32_t w0 = KB == 0 ? alignb(c[1], c[0], 2) : c[0];
            const uint32_t w1 = KB == 0 ? alignb(c[2], c[1], 2) : c[1];
            codes4(w0 ^ 0x80808080u, off2, d2, oh[0], oh[1], ol[0], ol[1]);
            codes4(w1 ^ 0x80808080u, off2, d2, oh[2], oh[3], ol[2], ol[3]);
            bh[m] = pack8(oh), bl[m] = pack8(ol);
        }
    }
}

// The codes of block kb as f16 (exact: |q| <= 128) for the two-pass
// kernels, and the block's scale d: the MFMAs multiply the activations'
// pieces by q, and d multiplies the block's f32 sums afterwards.
__device__ inline void codesq4(uint32_t v, __half2 off2, uint32_t &q01, uint32_t &q23) {
    q01 = h2_bits(__hsub2(as_h2(perm(0x64646464u, v, 0x04010400u)), off2));
    q23 = h2_bits(__hsub2(as_h2(perm(0x64646464u, v, 0x04030402u)), off2));
}
template <int DT, int KB>
__device__ inline void decode_codes(const uint32_t *v, half8 (&bq)[2], float &d, int h) {
    const uint32_t s = KB == 0 ? (v[0] & 0xffffu) : (v[0] >> 16);
    d = __half2float(__ushort_as_half((unsigned short)s));
    uint32_t o[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        const uint32_t w0 = KB == 0 ? alignb(v[2], v[1], 2) : v[1];
        const uint32_t w1 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        codesq4(w0 & 0x0f0f0f0fu, off2, o[0], o[1]);
        codesq4(w1 & 0x0f0f0f0fu, off2, o[2], o[3]);
        bq[0] = pack8(o);
        codesq4((w0 >> 4) & 0x0f0f0f0fu, off2, o[0], o[1]);
        codesq4((w1 >> 4) & 0x0f0f0f0fu, off2, o[2], o[3]);
        bq[1] = pack8(o);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        const uint32_t qh = KB == 0 ? alignb(v[1], v[0], 2) : v[1];
        const uint32_t w0 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        const uint32_t w1 = KB == 0 ? alignb(v[4], v[3], 2) : v[3];
        const uint32_t hb = qh >> (8 * h);
        codesq4((w0 & 0x0f0f0f0fu) | spread4(hb & 0xfu), off2, o[0], o[1]);
        codesq4((w1 & 0x0f0f0f0fu) | spread4((hb >> 4) & 0xfu), off2, o[2], o[3]);
        bq[0] = pack8(o);
        codesq4(((w0 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 16) & 0xfu), off2, o[0], o[1]);
        codesq4(((w1 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 20) & 0xfu), off2, o[2], o[3]);
        bq[1] = pack8(o);
    } else {
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const uint32_t *c = v + 1 + (KB == 0 ? 3 : 2) * m;
            const uint32_t w0 = KB == 0 ? alignb(c[1], c[0], 2) : c[0];
            const uint32_t w1 = KB == 0 ? alignb(c[2], c[1], 2) : c[1];
            codesq4(w0 ^ 0x80808080u, off2, o[0], o[1]);
            codesq4(w1 ^ 0x80808080u, off2, o[2], o[3]);
            bq[m] = pack8(o);
        }
    }
}

// Waves per SIMD of the MFMA kernels: 0 chooses per launch (below);
// MOE_MFMA_SPLIT=1 or 2 forces one (for measurements).
int mfma_split_forced() {
    const char *e = getenv("MOE_MFMA_SPLIT");
    return e && (e[0] == '1' || e[0] == '2') ? e[0] - '0' : 0;
}
const int g_mfma_split = mfma_split_forced();

// Three-pass kernels: two waves per SIMD pay once a tile holds two or more
// 32-token MFMA tiles (each wave of a pair then multiplies at least one):
// measured on MI355X, -4% at 128 tokens per expert (Mixtral T=512) and -12%
// at 128 (Qwen3 T=2048) in gate/up time, +3% at 8 tokens per expert
// (Mixtral T=32), where the second wave of each pair has no tile and only
// loads.
// The two-pass kernels (launch split 3) run by default: measured on MI355X
// against the three-pass ones, Mixtral T=512 1.106 -> 0.947 ms per layer
// (gate/up 713 -> 612 µs, down 341 -> 282), Qwen3 T=2048 0.784 -> 0.724,
// Mixtral T=32 0.404 -> 0.389, Qwen3 T=128 and V2-Lite T=256 within 1.5%.
// MOE_MFMA_Q2=0 at load, or moe_debug_mfma_kernel(1), selects the
// three-pass kernels (for measurements and tests).
int mfma_q2_off() {
    const char *e = getenv("MOE_MFMA_Q2");
    return e && e[0] == '0';
}
std::atomic<int> g_mfma_q2_off{mfma_q2_off()};

int mfma_split_for(double tokens_per_group) {
    if (!g_mfma_q2_off.load()) return 3;
    if (g_mfma_split) return g_mfma_split;
    return tokens_per_group >= 48.0 ? 2 : 1;
}

// SPLIT = 1: four waves, one per SIMD; wave w owns weight regions 2 w and
// 2 w + 1 and every token tile.  SPLIT = 2: eight waves, two per SIMD; the
// pair (w, w + 4) shares regions 2 w and 2 w + 1 (each wave loads one of
// them) and splits the token tiles, wave w taking the first ceil(MT / 2)
// and wave w + 4 the rest.  Both waves of a pair dequantise the same weight
// step, which costs VALU time but no LDS traffic, and whenever one of them
// waits for LDS, for the barrier or for its dequantisation, the other can
// issue MFMAs.
//
// Q2 (two passes; SPLIT = 2 only): the weights enter the MFMAs as their
// codes q (exact in f16) and each product is (hi + lo) q in two MFMAs; the
// four MFMAs of a 32-value block accumulate the block's sum P from zero,
// and the block's scale d then adds it into the tile: acc = fma(d, P, acc),
// in f32.  Against the three passes of d q split into pieces this drops a
// third of the MFMAs and most of the dequantisation; it adds 16 fmas per
// lane per tile and block.  The ring, DMAs, waits and epilogue are shared.
template <int DT, bool UP, int BM, int SPLIT, bool Q2>
__global__ __launch_bounds__(256 * SPLIT, 1) __attribute__((amdgpu_waves_per_eu(SPLIT, SPLIT))) void mfma_kernel(MfmaArgs a, int mode, int gx, int ksplit) {
    using BL = BLay<DT>;
    constexpr int NS = ring_stages<DT, BM>();
    constexpr int MTMAX = BM / 32;        // 32-token MFMA tiles per block tile
    constexpr int MWMAX = (MTMAX + SPLIT - 1) / SPLIT;  // tiles of one wave
    constexpr int AS = a_stage<BM>();     // bytes of one activation piece per stage
    constexpr int RS = 2 * AS + BL::stage;  // bytes of one ring stage
    constexpr int NJ = 2 / SPLIT;         // weight regions one wave loads
    static_assert(NS == 3, "the step loop below assumes three stages");
    static_assert(SPLIT == 1 || SPLIT == 2, "one or two waves per SIMD");
    static_assert(!Q2 || SPLIT == 2, "two-pass tiles keep their sums in VGPRs: two waves per SIMD");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int *src_row = reinterpret_cast<int *>(smem + NS * RS);
    int *dst_row = src_row + BM;
    int *ex_row = dst_row + BM;

    TileInfo ti;
    if (!tile_of<BM, 32>(a, mode, gx, ti)) return;
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
    const int sw = wv & 3;                     // the SIMD's weight regions 2 sw, 2 sw + 1
    const int half = SPLIT == 2 ? wv >> 2 : 0;  // which token tiles (SPLIT 2)
    const int Icol = ti.shared ? a.I_s : a.I;
    const int valid = min(BM, ti.n - ti.m0);
    const int mt = (valid + 31) / 32;
    const int wexp0 = Q2 ? 0 : W0.wexp, wexp1 = Q2 ? 0 : W1.wexp;

    // Activation pieces and their row exponents.
    const uint16_t *ahi = UP ? a.xhi : (ti.shared ? a.hshi : a.hhi);
    const uint16_t *alo = UP ? a.xlo : (ti.shared ? a.hslo : a.hlo);
    const int32_t *aex = UP ? a.xex : (ti.shared ? a.hsex : a.hex);
    if (tid < BM) {
        int s = -1, d = -1, e = 0;
        if (tid < valid) {
            d = ti.row0 + ti.m0 + tid;
            s = UP ? (ti.shared ? ti.m0 + tid : a.perm_tok[d]) : d;
            e = aex[s];
        }
        src_row[tid] = s;
        dst_row[tid] = d;
        ex_row[tid] = e;
    }
    __syncthreads();

    const uint32_t lds0 = lds_addr(smem);
    const uint32_t ldsB = lds0 + NS * 2 * AS;
    const lds_p sm = (lds_p)smem;
    const int l32 = lane & 31, hf = lane >> 5;

    // Activation DMA: the tile's rows come in groups of eight (group i =
    // rows 8 i .. 8 i + 7, 1 KiB per piece at offset 1024 i of the stage);
    // instruction u of wave wv loads group wv + 4 SPLIT u (modulo the tile's
    // groups: a group loaded twice is written twice with the same bytes,
    // before the barrier that publishes it).  Lane l takes row r = 8 i + l / 8
    // and stores slot l % 8 of that row's 128 bytes, which holds logical
    // chunk (l % 8) ^ ((r / 2) % 8).  Rows past the tile's tokens repeat
    // token row 0 (their outputs are never stored).  The lo piece uses the
    // same offsets in its own array.
    const uint32_t arow_bytes = (uint32_t)(UP ? a.H : Icol) * 2;
    // Weight DMA: region 2 sw + j holds 32 weight rows; this wave loads the
    // regions j of jj < NJ (SPLIT 1: both, SPLIT 2: j = half).  woff: per DMA
    // (the region's dwordx4 DMAs, then its dword DMAs) the lane's byte offset
    // in the weight matrix, without the step's K offset.
    const uint8_t *wbase[NJ];
    uint32_t woff[NJ][BL::inst];
    uint32_t wreg[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) {
        const int j = SPLIT == 2 ? half : jj;
        const MatDev &W = (UP && j == 1) ? W1 : W0;
        wbase[jj] = W.ptr;
        wreg[jj] = (uint32_t)(2 * sw + j);
        const int row0 = UP ? n0 + 32 * sw : n0 + 64 * sw + 32 * j;
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
            woff[jj][i] = off;
        }
    }
    // The dequantisation's scale exponent of region j (gate, up: the two
    // matrices of the up projection; down: one matrix).
    const int wx[2] = {wexp0, UP ? wexp1 : wexp0};

    // Per-lane LDS offsets of the compute side.
    uint32_t aoff[4];  // group g = 2 kb + m: row l32, logical chunk 2 g + hf
#pragma unroll
    for (int g = 0; g < 4; g++) aoff[g] = (uint32_t)l32 * 128u + ((uint32_t)((2 * g + hf) ^ ((l32 >> 1) & 7)) << 4);
    using SL = Slots<DT>;
    const uint32_t brow_x = 16u * l32;                 // row l32's X part within a region
    const uint32_t brow_d = BL::xbytes + 4u * l32;     // and its D part

    floatx16 acc[MWMAX][2];
#pragma unroll
    for (int t = 0; t < MWMAX; t++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[t][j] = floatx16{};

    // The step loop for a tile of MT 32-token tiles; this wave multiplies
    // tiles T0 .. T0 + MW - 1 (MW may be 0: the wave then only loads).
    auto run = [&](auto mt_c, auto mw_c, auto t0_c) {
        constexpr int MT = decltype(mt_c)::value;
        constexpr int MW = decltype(mw_c)::value, T0 = decltype(t0_c)::value;
        constexpr int MWR = MW > 0 ? MW : 1;  // array extent
        constexpr int NG = 4 * MT;             // activation row groups per piece
        constexpr int UA = (NG + 4 * SPLIT - 1) / (4 * SPLIT);  // of this wave
        constexpr int NA = 2 * UA;             // activation DMAs per wave per step (hi, then lo)
        constexpr int NB = NJ * BL::inst;      // weight DMAs per wave per step
        constexpr int ND = NA + NB;            // DMAs per wave per step
        uint32_t aoffg[UA], agrp[UA];          // source offsets (step 0) and LDS groups
#pragma unroll
        for (int u = 0; u < UA; u++) {
            const int i = (wv + 4 * SPLIT * u) % NG;
            const int r = 8 * i + (lane >> 3);
            const int sr = src_row[r < valid ? r : 0];
            aoffg[u] = (uint32_t)sr * arow_bytes + (uint32_t)kbeg * 2u +
                       (uint32_t)(((lane & 7) ^ ((r >> 1) & 7)) << 4);
            agrp[u] = (uint32_t)i * 1024u;
        }
        // DMA d of step `step` into ring stage `st`: d < NA activations
        // (hi pieces, then lo), then the weight regions.  Steps past the end
        // reload the last step into a stage nobody reads any more, so every
        // step issues the same DMAs.
        auto dma = [&](auto d_c, int step, int st) {
            constexpr int d = decltype(d_c)::value;
            const int sc = step < nsteps ? step : nsteps - 1;
            if constexpr (d < NA) {
                constexpr int p = d / UA, u = d % UA;
                const uint16_t *src = p == 0 ? ahi : alo;
                dma16(reinterpret_cast<const uint8_t *>(src) + (size_t)sc * (BK * 2), aoffg[u],
                      lds0 + (uint32_t)st * 2 * AS + (uint32_t)p * AS + agrp[u]);
            } else {
                constexpr int jj = (d - NA) / BL::inst, i = (d - NA) % BL::inst;
                const uint8_t *wb = wbase[jj] + (size_t)(kbeg / 32 + 2 * sc) * Fmt<DT>::bytes;
                const uint32_t lr = ldsB + (uint32_t)st * BL::stage + wreg[jj] * BL::region;
                if constexpr (i < BL::ix)
                    dma16(wb, woff[jj][i], lr + 1024u * i);
                else
                    dma4(wb, woff[jj][i], lr + BL::xbytes + 256u * (i - BL::ix));
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
        half8 bh[2][2][2], bl[2][2][2];  // [kb][j][m] hi and lo pieces
        half8 ah[2][MWR], al[2][MWR];    // activation pieces of two groups
        uint32_t rowv[2][BL::rd];
        auto read_rows = [&](lds_p stage_b) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t reg = (uint32_t)(2 * sw + j) * BL::region;
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
        auto dequant_raw = [&](auto kb_c) {
            constexpr int kb = decltype(kb_c)::value;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                uint32_t v[7];
#pragma unroll
                for (int k = 0; k < SL::n[kb]; k++) {
                    const int b = SL::base[kb][k];
                    v[k] = SL::hm[kb][k] ? (hf ? rowv[j][b + 2] : rowv[j][b]) : rowv[j][b];
                }
                dequant<DT, kb>(v, bh[kb][j], bl[kb][j], hf, wx[j]);
            }
        };
        auto read_a = [&](lds_p sa, int g, int slot) {
            const lds_p p = sa + aoff[g];
#pragma unroll
            for (int t = 0; t < MW; t++)
                ah[slot][t] = lds_h8(p + 4096 * (T0 + t)), al[slot][t] = lds_h8(p + AS + 4096 * (T0 + t));
        };
        // MFMA pass q of tile i = 2 t + j for group (kb, m): q 0 = hi.lo,
        // 1 = lo.hi, 2 = hi.hi.  A group runs pass 0 over all its tiles, then
        // pass 1, then pass 2, so consecutive MFMAs never share an
        // accumulator (with one tile, the pair of regions still alternates).
        auto mfma = [&](int slot, int kb, int m, int q, int i) {
            const int t = i >> 1, j = i & 1;
            const half8 &A = q == 1 ? al[slot][t] : ah[slot][t];
            const half8 &B = q == 0 ? bl[kb][j][m] : bh[kb][j][m];
            acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, acc[t][j], 0, 0, 0);
        };
        // One group's 6 MW MFMAs with DMAs [LO, HI) of step `step` spread
        // between them: a DMA that the memory pipeline cannot take yet stalls
        // this wave, not the MFMAs already queued.
        auto mfmas_dma = [&](int slot, int kb, int m, auto lo_c, auto hi_c, int step, int st) {
            constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
            constexpr int N = 6 * MW;
            if constexpr (N == 0) {
                dma_range(lo_c, hi_c, step, st);
            } else {
                auto body = [&](auto i_c, auto self) {
                    constexpr int i = decltype(i_c)::value;
                    if constexpr (i < N) {
                        mfma(slot, kb, m, i / (2 * MW), i % (2 * MW));
                        dma_range(std::integral_constant<int, LO + i * (HI - LO) / N>{},
                                  std::integral_constant<int, LO + (i + 1) * (HI - LO) / N>{}, step, st);
                        self(std::integral_constant<int, i + 1>{}, self);
                    }
                };
                body(std::integral_constant<int, 0>{}, body);
            }
        };
        auto mfmas = [&](int slot, int kb, int m) {
#pragma unroll
            for (int q = 0; q < 3; q++)
#pragma unroll
                for (int i = 0; i < 2 * MW; i++) mfma(slot, kb, m, q, i);
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        constexpr bool work = MW > 0;

        const lds_p smB = sm + NS * 2 * AS;
        constexpr int WAIT = (NS - 2) * ND;
        static_assert(NS * ND < 64, "vmcnt range");
        if constexpr (!Q2) {
            // Prologue: steps 0 .. NS - 1 into stages 0 .. NS - 1, then wait for
            // step 0.
            for (int p = 0; p < NS; p++) dma_range(I0{}, std::integral_constant<int, ND>{}, p, p);
            wait_vm_barrier<(NS - 1) * ND>();
            if constexpr (work) {
                read_a(sm, 0, 0);
                read_rows(smB);
                dequant_raw(I0{});
            }
            int st = 0;
            // At the wait in group 2 of step s this wave's outstanding loads are
            // those of steps s + 1 .. s + NS - 1 (ND each, in order); leaving the
            // newest (NS - 2) ND outstanding completes step s + 1.  After the
            // barrier that follows, no wave reads stage s again (its last reads,
            // group 3's activations, come before the barrier), so group 3 sends
            // step s + NS's loads into it.
            for (int s = 0; s < nsteps; s++) {
                const lds_p sa = sm + st * 2 * AS;
                const int st1 = st + 1 == NS ? 0 : st + 1;
                if constexpr (work) {
                    // g = 0 (kb 0, m 0); read group 1.
                    read_a(sa, 1, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    mfmas(0, 0, 0);
                    // g = 1 (kb 0, m 1): dequantise block 1, read group 2.
                    dequant_raw(I1{});
                    read_a(sa, 2, 0);
                    mfmas(1, 0, 1);
                    __builtin_amdgcn_sched_barrier(0);
                    // g = 2 (kb 1, m 0): read group 3; then wait for this wave's
                    // loads of step s + 1 and meet the other waves.
                    read_a(sa, 3, 1);
                    mfmas(0, 1, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
                wait_vm_barrier<WAIT>();
                __builtin_amdgcn_sched_barrier(0);
                // g = 3 (kb 1, m 1): step s + 1's group 0 and weight rows; step
                // s + NS's DMAs into this step's stage.
                if constexpr (work) {
                    read_a(sm + st1 * 2 * AS, 0, 0);
                    read_rows(smB + st1 * BL::stage);
                }
                __builtin_amdgcn_sched_barrier(0);
                mfmas_dma(1, 1, 1, I0{}, std::integral_constant<int, ND>{}, s + NS, st);
                if constexpr (work) dequant_raw(I0{});
                __builtin_amdgcn_sched_barrier(0);
                st = st1;
            }
        } else {
            // Two passes.  Unit u (< 2 MW) of a step is tile T0 + u % MW of
            // block u / MW: its activations (hi and lo of both 16-value
            // groups) sit in buffer u % 2, read one unit ahead.  Its eight
            // MFMAs (the two regions' chains alternating: back-to-back
            // MFMAs on one accumulator stall) leave the block sums in
            // ps[u % 2]; the fmas that add them into the tiles follow the
            // next unit's MFMAs, so the matrix cores need not wait for them.
            // One block's codes are held at a time: block 1's are decoded
            // once block 0's last unit has issued its MFMAs.
            half8 bq[1][2][2];  // [j][m] codes of the block in progress
            float dq[2][2];     // [kb][j] scale of the lane's row
            half8 A[2][4];      // hi m0, lo m0, hi m1, lo m1
            const floatx16 zero = {};
            auto decode = [&](auto kb_c) {
                constexpr int kb = decltype(kb_c)::value;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    uint32_t v[7];
#pragma unroll
                    for (int k = 0; k < SL::n[kb]; k++) {
                        const int b = SL::base[kb][k];
                        v[k] = SL::hm[kb][k] ? (hf ? rowv[j][b + 2] : rowv[j][b]) : rowv[j][b];
                    }
                    decode_codes<DT, kb>(v, bq[0][j], dq[kb][j], hf);
                }
            };
            auto read_unit = [&](lds_p sa, int u, half8(&Ab)[4]) {
                const int kb = u / MWR, t = u % MWR;
                const lds_p p0 = sa + aoff[2 * kb] + 4096 * (T0 + t);
                const lds_p p1 = sa + aoff[2 * kb + 1] + 4096 * (T0 + t);
                Ab[0] = lds_h8(p0), Ab[1] = lds_h8(p0 + AS), Ab[2] = lds_h8(p1), Ab[3] = lds_h8(p1 + AS);
            };
            floatx16 ps[2][2];  // [unit parity][j]
            auto unit_mfma = [&](auto u_c, auto lo_c, auto hi_c, int step, int stg) {
                constexpr int u = decltype(u_c)::value, b = u % 2;
                constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
                auto mf = [&](auto i_c) {
                    constexpr int i = decltype(i_c)::value, j = i & 1, q = i >> 1;
                    ps[b][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[b][q], bq[0][j][q >> 1], i < 2 ? zero : ps[b][j],
                                                                      0, 0, 0);
                    dma_range(std::integral_constant<int, LO + i * (HI - LO) / 8>{},
                              std::integral_constant<int, LO + (i + 1) * (HI - LO) / 8>{}, step, stg);
                };
                mf(std::integral_constant<int, 0>{});
                mf(std::integral_constant<int, 1>{});
                mf(std::integral_constant<int, 2>{});
                mf(std::integral_constant<int, 3>{});
                mf(std::integral_constant<int, 4>{});
                mf(std::integral_constant<int, 5>{});
                mf(std::integral_constant<int, 6>{});
                mf(std::integral_constant<int, 7>{});
            };
            auto unit_fma = [&](auto u_c) {
                constexpr int u = decltype(u_c)::value, kb = u / MWR, t = u % MWR, b = u % 2;
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[t][j][v] = fmaf(dq[kb][j], ps[b][j][v], acc[t][j][v]);
            };
            auto units_to = [&](auto u_c, auto self, const lds_p sa) {
                constexpr int u = decltype(u_c)::value;
                if constexpr (u + 1 < 2 * MW) {
                    read_unit(sa, u + 1, A[(u + 1) % 2]);
                    unit_mfma(u_c, I0{}, I0{}, 0, 0);
                    if constexpr (u > 0) unit_fma(std::integral_constant<int, u - 1>{});
                    if constexpr (u == MW - 1) decode(I1{});
                    __builtin_amdgcn_sched_barrier(0);
                    self(std::integral_constant<int, u + 1>{}, self, sa);
                }
            };
            for (int p = 0; p < NS; p++) dma_range(I0{}, std::integral_constant<int, ND>{}, p, p);
            wait_vm_barrier<(NS - 1) * ND>();
            if constexpr (work) {
                read_rows(smB);
                decode(I0{});
                read_unit(sm, 0, A[0]);
            }
            int st = 0;
            for (int s = 0; s < nsteps; s++) {
                const lds_p sa = sm + st * 2 * AS;
                const int st1 = st + 1 == NS ? 0 : st + 1;
                // Units 0 .. 2 MW - 2; the last unit's activations are read
                // during the one before it.
                if constexpr (work) units_to(I0{}, units_to, sa);
                // Every read of this stage is done: wait for this wave's
                // loads of step s + 1 and meet the other waves.
                wait_vm_barrier<WAIT>();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (work) {
                    // The next step's first unit and weight rows, then this
                    // step's last unit with step s + NS's DMAs between its
                    // MFMAs, then the next step's block-0 codes.
                    read_unit(sm + st1 * 2 * AS, 0, A[0]);
                    read_rows(smB + st1 * BL::stage);
                    __builtin_amdgcn_sched_barrier(0);
                    unit_mfma(std::integral_constant<int, 2 * MWR - 1>{}, I0{}, std::integral_constant<int, ND>{},
                              s + NS, st);
                    unit_fma(std::integral_constant<int, 2 * MWR - 2>{});
                    unit_fma(std::integral_constant<int, 2 * MWR - 1>{});
                    decode(I0{});
                } else {
                    dma_range(I0{}, std::integral_constant<int, ND>{}, s + NS, st);
                }
                __builtin_amdgcn_sched_barrier(0);
                st = st1;
            }
        }
    };
    static_assert(MTMAX == 5 || MTMAX == 4, "one case per 32-token tile count");
    // Tiles of this wave: SPLIT 1 all MT; SPLIT 2 the first ceil(MT / 2)
    // (half 0) or the rest (half 1).
    auto run_mt = [&](auto mt_c) {
        constexpr int MT = decltype(mt_c)::value;
        if constexpr (SPLIT == 1) {
            run(mt_c, mt_c, std::integral_constant<int, 0>{});
        } else {
            constexpr int MA = (MT + 1) / 2;
            if (half == 0)
                run(mt_c, std::integral_constant<int, MA>{}, std::integral_constant<int, 0>{});
            else
                run(mt_c, std::integral_constant<int, MT - MA>{}, std::integral_constant<int, MA>{});
        }
    };
    switch (mt) {
    case 1: run_mt(std::integral_constant<int, 1>{}); break;
    case 2: run_mt(std::integral_constant<int, 2>{}); break;
    case 3: run_mt(std::integral_constant<int, 3>{}); break;
    case 4: run_mt(std::integral_constant<int, 4>{}); break;
    default:
        if constexpr (MTMAX == 5) run_mt(std::integral_constant<int, MTMAX>{});
        break;
    }
    wait_vm<0>();

    // This wave's tiles: t0 .. t0 + mw - 1.
    const int ma = SPLIT == 2 ? (mt + 1) / 2 : mt;
    const int t0 = half ? ma : 0, mw = half ? mt - ma : ma;

    // ---- epilogue: lane holds C[32 t + 8 (v / 4) + 4 hf + v % 4][column l32 of set j],
    // scaled by 2^(ex_row + wexp).
    if (UP) {
        float *hout = ti.shared ? a.hs : a.h;
        const int col = n0 + 32 * sw + l32;
        if (col < W0.rows) {
#pragma unroll
            for (int t = 0; t < MWMAX; t++) {
                if (t >= mw) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int r = 32 * (t0 + t) + 8 * (v / 4) + 4 * hf + (v % 4);
                    const int d = dst_row[r];
                    if (d < 0) continue;
                    const int e = ex_row[r];
                    const float g = ldexpf(acc[t][0][v], -(e + wexp0)), u = ldexpf(acc[t][1][v], -(e + wexp1));
                    hout[(size_t)d * Icol + col] = (g / (1.0f + __expf(-g))) * u;
                }
            }
        }
    } else {
        float *yout = ti.shared ? a.ys + ti.ksplit * a.yspart : a.y + ti.ksplit * a.ypart;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + 64 * sw + 32 * j + l32;
            if (col >= W0.rows) continue;
#pragma unroll
            for (int t = 0; t < MWMAX; t++) {
                if (t >= mw) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int r = 32 * (t0 + t) + 8 * (v / 4) + 4 * hf + (v % 4);
                    const int d = dst_row[r];
                    if (d >= 0) yout[(size_t)d * a.H + col] = ldexpf(acc[t][j][v], -(ex_row[r] + wexp0));
                }
            }
        }
    }
}

template <int DT, bool UP, int BM, int SPLIT, bool Q2>
hipError_t launch_split(dim3 grid, const MfmaArgs &a, int mode, int ksplit, hipStream_t s) {
    constexpr int lds = lds_bytes<DT, BM>();
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&mfma_kernel<DT, UP, BM, SPLIT, Q2>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((mfma_kernel<DT, UP, BM, SPLIT, Q2>), grid, dim3(256 * SPLIT), lds, s, a, mode, (int)grid.x,
                       ksplit);
    return hipGetLastError();
}
// split 3: the two-pass kernel (two waves per SIMD).
template <int DT, bool UP, int BM>
hipError_t launch_one(dim3 grid, const MfmaArgs &a, int mode, int ksplit, int split, hipStream_t s) {
    if (split == 3) return launch_split<DT, UP, BM, 2, true>(grid, a, mode, ksplit, s);
    return split == 2 ? launch_split<DT, UP, BM, 2, false>(grid, a, mode, ksplit, s)
                      : launch_split<DT, UP, BM, 1, false>(grid, a, mode, ksplit, s);
}

template <bool UP>
hipError_t launch_dt(int dt, int bm, dim3 grid, const MfmaArgs &a, int mode, int ksplit, int split,
                     hipStream_t s) {
    if (bm == 160) {
        switch (dt) {
        case MOE_DT_Q4_0: return launch_one<MOE_DT_Q4_0, UP, 160>(grid, a, mode, ksplit, split, s);
        case MOE_DT_Q5_0: return launch_one<MOE_DT_Q5_0, UP, 160>(grid, a, mode, ksplit, split, s);
        default: return hipErrorInvalidValue;
        }
    }
    if (bm != 128) return hipErrorInvalidValue;
    switch (dt) {
    case MOE_DT_Q8_0: return launch_one<MOE_DT_Q8_0, UP, 128>(grid, a, mode, ksplit, split, s);
    case MOE_DT_Q4_0: return launch_one<MOE_DT_Q4_0, UP, 128>(grid, a, mode, ksplit, split, s);
    case MOE_DT_Q5_0: return launch_one<MOE_DT_Q5_0, UP, 128>(grid, a, mode, ksplit, split, s);
    default: return hipErrorInvalidValue;
    }
}

// ---- activation pieces ------------------------------------------------------
// One block per row: the row's largest magnitude (a max over the block),
// then every value's scaled hi and lo pieces.  Rows of up to 16384 values
// stay in registers between the two (one read of the row); wider rows are
// read twice.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
constexpr int kSplitCached4 = 16;  // float4 per thread kept in registers

__device__ inline int split_exponent(float m) {
    int e = 0;
    if (m > 0.0f && m <= 3.402823466e38f) {
        int fe;
        (void)frexpf(m, &fe);  // m in [2^(fe-1), 2^fe)
        e = 15 - fe;
    }
    return e;
}
__device__ inline void split_store(const f32x4 &v, int e, u16x4 *h4, u16x4 *l4) {
    u16x4 ho, lw;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float x = ldexpf(v[c], e);
        const __half h = __float2half_rn(x);
        ho[c] = __half_as_ushort(h);
        lw[c] = __half_as_ushort(__float2half_rn(x - __half2float(h)));
    }
    gstore(h4, ho);
    gstore(l4, lw);
}
__device__ inline float block_max256(float m, float *part) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    return fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
}
template <bool CACHED>
__global__ __launch_bounds__(256) void split_rows_kernel(const float *__restrict__ src, int cols,
                                                         uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                         int32_t *__restrict__ ex) {
    __shared__ float part[4];
    const size_t row = blockIdx.x;
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src + row * cols);
    u16x4 *h4 = reinterpret_cast<u16x4 *>(hi + row * cols);
    u16x4 *l4 = reinterpret_cast<u16x4 *>(lo + row * cols);
    const int n4 = cols / 4;
    float m = 0.0f;
    if constexpr (CACHED) {
        f32x4 v[kSplitCached4];
#pragma unroll
        for (int u = 0; u < kSplitCached4; u++) {
            const int i = threadIdx.x + 256 * u;
            v[u] = i < n4 ? gload(s4 + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
        }
        const int e = split_exponent(block_max256(m, part));
        if (threadIdx.x == 0) ex[row] = e;
#pragma unroll
        for (int u = 0; u < kSplitCached4; u++) {
            const int i = threadIdx.x + 256 * u;
            if (i < n4) split_store(v[u], e, h4 + i, l4 + i);
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += 256) {
            const f32x4 v = gload(s4 + i);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        const int e = split_exponent(block_max256(m, part));
        if (threadIdx.x == 0) ex[row] = e;
        for (int i = threadIdx.x; i < n4; i += 256) split_store(gload(s4 + i), e, h4 + i, l4 + i);
    }
}

// Rows of at most 64 kSplitWave4 float4s: one wavefront per row (four rows
// per block), the row's largest |v| from lane shuffles; the same pieces and
// exponent as split_rows_kernel.
constexpr int kSplitWave4 = 8;
__global__ __launch_bounds__(256) void split_rows_wave_kernel(const float *__restrict__ src, int rows, int cols,
                                                              uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                              int32_t *__restrict__ ex) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f32x4 *s4 = reinterpret_cast<const f32x4 *>(src + (size_t)row * cols);
    u16x4 *h4 = reinterpret_cast<u16x4 *>(hi + (size_t)row * cols);
    u16x4 *l4 = reinterpret_cast<u16x4 *>(lo + (size_t)row * cols);
    const int n4 = cols / 4;
    f32x4 v[kSplitWave4];
    float m = 0.0f;
#pragma unroll
    for (int u = 0; u < kSplitWave4; u++) {
        const int i = lane + 64 * u;
        v[u] = i < n4 ? gload(s4 + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const int e = split_exponent(m);
    if (lane == 0) ex[row] = e;
#pragma unroll
    for (int u = 0; u < kSplitWave4; u++) {
        const int i = lane + 64 * u;
        if (i < n4) split_store(v[u], e, h4 + i, l4 + i);
    }
}

// ---- weight scales -------------------------------------------------------------
// Block (g, m, z): slice z of matrix m of expert g; every 32-value block's
// scale (the first two bytes of the block), as |d| in f16 bits.
__global__ __launch_bounds__(256) void scale_max_kernel(const ExpertDev *__restrict__ experts,
                                                        unsigned *__restrict__ out) {
    const MatDev m = experts[blockIdx.x].m[blockIdx.y];
    const int bb = block_bytes(m.dt);
    unsigned best = 0;
    if (m.dt == MOE_DT_Q4_0 || m.dt == MOE_DT_Q5_0 || m.dt == MOE_DT_Q8_0) {
        const long long per_row = m.cols / 32, n = (long long)m.rows * per_row;
        for (long long i = (long long)blockIdx.z * 256 + threadIdx.x; i < n; i += (long long)gridDim.z * 256) {
            const long long r = i / per_row, b = i - r * per_row;
            const uint8_t *p = m.ptr + (size_t)r * m.stride + (size_t)b * bb;
            const unsigned bits = ((unsigned)gload(p) | ((unsigned)gload(p + 1) << 8)) & 0x7fffu;
            best = bits > best && bits < 0x7c00u ? bits : best;  // skip inf / nan scales
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) best = max(best, (unsigned)__shfl_xor((int)best, o, 64));
    if ((threadIdx.x & 63) == 0 && best) atomicMax(out + 3 * blockIdx.x + blockIdx.y, best);
}

}  // namespace

int mfma_tile_m(const int *dts, int n) {
    for (int i = 0; i < n; i++)
        if (dts[i] == MOE_DT_Q8_0) return 128;
    return 160;
}

// The token tile of one routed call.  A layer whose formats allow 160-token
// tiles takes 128 when it has many experts (their token counts spread, and
// a full 128-token tile splits two and two between the waves of a SIMD
// where a 160-token one splits three and two) or when its experts hold at
// most 32 tokens on average.  Measured on MI355X (ms per layer, 160 against
// 128): DeepSeek-V3 Zipf T=4096 8.79 -> 8.65, DeepSeek-V3 T=64 1.258 ->
// 1.222, Mixtral T=32 0.421 -> 0.414 and 0.412 -> 0.408; Mixtral T=512,
// whose 8 experts hold about 128 tokens each, 0.909 -> 1.03 (experts just
// over 128 tokens take a second, nearly empty tile), so it keeps 160.
int mfma_call_tile(int layer_bm, int t, int k, int E) {
    if (layer_bm != 160) return layer_bm;
    return (E >= 64 || (long long)t * k <= 32LL * E) ? 128 : 160;
}

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

int device_cus() {
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
int split_cus(double tokens_per_tile, double min_tokens) {
    return tokens_per_tile >= min_tokens ? device_cus() / 8 : 0;
}
// Down launches keep their plain grid's order (order = false): with many
// token tiles per expert (skewed routing) the XCD order re-reads each tile's
// activations for every N tile, where the plain order keeps a token tile on
// one XCD.  Gate/up launches take it (an expert's activations meet every N
// tile in one L2).
dim3 tile_grid(int tiles, int rows, int cols, int ks, int xcd_cus, bool order) {
    const int gy = (rows + cols - 1) / cols;
    if (xcd_cus <= 0 || ks != 1) return dim3(tiles, gy, ks);
    if (!order && ((long long)tiles * gy) % 8 != 0) return dim3(tiles, gy, ks);
    const long long need = (long long)tiles * gy + 8LL * (xcd_cus / 2);
    int gx = (int)((need + gy - 1) / gy);
    while (((long long)gx * gy) & 7) gx++;
    return dim3(gx, gy, ks);
}

hipError_t launch_mfma(bool up, const MfmaArgs &a0, int bm, const ExpertDev &e0, const ExpertDev *sh,
                       hipStream_t s) {
    MfmaArgs a = a0;
    a.xcd_cus = split_cus(a.E > 0 ? (double)a.T * a.k / a.E : 0.0, 48.0);
    const MatDev &m = up ? e0.m[0] : e0.m[2];
    const int cols = up ? BW / 2 : BW;
    const int ks = up ? 1 : a.ksplit;
    const dim3 grid = tile_grid(a.max_tiles, m.rows, cols, ks, a.xcd_cus, up);
    const int sp = mfma_split_for(a.E > 0 ? (double)a.T * a.k / a.E : 0.0);
    hipError_t err = up ? launch_dt<true>(m.dt, bm, grid, a, 0, ks, sp, s)
                        : launch_dt<false>(m.dt, bm, grid, a, 0, ks, sp, s);
    if (err != hipSuccess || !sh) return err;
    return launch_mfma_single(up, a, bm, *sh, s);
}

hipError_t launch_mfma_single(bool up, const MfmaArgs &a0, int bm, const ExpertDev &ex, hipStream_t s) {
    MfmaArgs a = a0;
    a.xcd_cus = split_cus((double)(a.T < bm ? a.T : bm), 48.0);
    const MatDev &m = up ? ex.m[0] : ex.m[2];
    const int cols = up ? BW / 2 : BW;
    const int ks = up ? 1 : a.ksplit;
    const dim3 gs = tile_grid((a.T + bm - 1) / bm, m.rows, cols, ks, a.xcd_cus, up);
    const int sp = mfma_split_for((double)a.T);
    return up ? launch_dt<true>(m.dt, bm, gs, a, 1, ks, sp, s) : launch_dt<false>(m.dt, bm, gs, a, 1, ks, sp, s);
}

hipError_t launch_split_rows(const float *src, int rows, int cols, uint16_t *hi, uint16_t *lo, int32_t *ex,
                             hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (cols % 4 != 0) return hipErrorInvalidValue;
    if (cols / 4 <= 64 * kSplitWave4)
        hipLaunchKernelGGL(split_rows_wave_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, src, rows, cols, hi, lo, ex);
    else if (cols / 4 <= 256 * kSplitCached4)
        hipLaunchKernelGGL(split_rows_kernel<true>, dim3(rows), dim3(256), 0, s, src, cols, hi, lo, ex);
    else
        hipLaunchKernelGGL(split_rows_kernel<false>, dim3(rows), dim3(256), 0, s, src, cols, hi, lo, ex);
    return hipGetLastError();
}

hipError_t launch_scale_max(const ExpertDev *experts, int n, unsigned *out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(scale_max_kernel, dim3(n, 3, 16), dim3(256), 0, s, experts, out);
    return hipGetLastError();
}

int set_mfma_kernel(int choice) { return g_mfma_q2_off.exchange(choice == 1 ? 1 : 0); }

}  // namespace moe
