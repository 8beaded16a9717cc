// expert_stream.hip — grouped SwiGLU expert products on gfx950 matrix cores,
// weight rows streamed through a deep LDS ring (mode 6 of the layer).
//
// A block computes a tile of up to BM = 32 S tokens x 256 weight rows of one
// expert:
//   up   : 128 gate rows and the same 128 up rows of the expert, K = H; the
//          epilogue forms h = silu(G) * U in f32 (src/model.rs:31-33);
//   down : 256 rows of W_down, K = I (or one K part of it); y in f32.
// Eight waves, two per SIMD.  The SIMD's pair (w, w + 4) owns 64 weight rows
// as two 32-row regions (up: gate rows 32 w .. 32 w + 31 and the same up
// rows, so one lane holds a token's gate and up sums for one row; down:
// rows 64 w .. 64 w + 63) and every token of the tile as S 32-token
// subtiles; the two waves take the two 32-value blocks of every 64-value
// ring step, so each decodes only its own block, and whenever one waits
// (for LDS, its fmas or the barrier) the other issues MFMAs.  Accumulators,
// S x 2 tiles of V_MFMA_F32_32X32X16_F16 per wave, stay in registers for the
// whole K loop; at the end the two halves of each sum meet in LDS.
//
// Precision, the same arithmetic as expert_mfma.hip.  The reference
// multiplies f32 activations by exactly dequantised f32 weights d q
// (src/quant.rs:482-506).  Here split_rows writes each activation row as
// hi + lo f16 pieces of v 2^ex (ex per row putting its largest |v| in
// [2^14, 2^15): 22 significant bits), and the weights enter the MFMAs as
// their codes q, exact in f16.  The four MFMAs of a 32-value block
// ((hi + lo) q over two 16-value halves) accumulate the block's sum P from
// zero, and the block's scale adds it into the tile, acc = fma(d, P, acc),
// in f32; the epilogue multiplies by 2^-ex, which is exact.  SwiGLU's
// sigmoid uses the hardware exp and reciprocal (v_exp_f32, v_rcp_f32, about
// 1 ulp each).
//
// Operands reach LDS by DMA (global_load_lds): the activations' 16-byte
// chunks (the chunk index XORed with bits 1..3 of the token row, so the
// fragment reads of 16 consecutive rows hit 16 different bank groups) and
// the raw quantised bytes of each wave's own region.  A ring of NS stages
// (as many as fit in the LDS, up to 12) keeps NS - 1 K steps in flight with
// exact vmcnt waits, the DMAs of a step spread over its subtiles so that no
// wave stalls on a burst of issues; one barrier per step publishes the
// stage, and the next step's codes are decoded while the current MFMAs run.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

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

// f(integral_constant<I>) for I = B .. E - 1, in order.
template <int B, int E, typename F>
__device__ inline void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr int SW = 256;  // weight rows per tile
constexpr int SK = 64;   // K values per ring step (two blocks)

// Bytes of one activation piece of one ring stage: 32 S token rows of SK
// f16 values.
template <int S>
constexpr int s_act() {
    return 32 * S * SK * 2;
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
__device__ inline half8 pack8(const uint32_t (&o)[4]) {
    half8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

// ---- weight slots -------------------------------------------------------------
// Lane (l32, h) multiplies row l32 of a region.  MFMA m of block kb takes
// the block's values 16 m + 8 h .. + 7 in natural order; both MFMAs use the
// same eight code bytes 8 h .. 8 h + 7 (Q4_0 / Q5_0: low nibbles for m = 0,
// high nibbles for m = 1; Q8_0: bytes 16 m + 8 h ..).  Slot k of block kb is
// dword base[k] + 2 h hm[k] of the row's ring step (rd dwords: block 0 at
// byte 0, block 1 right after it):
//   Q4_0 kb 0: d at bytes 0-1, codes 2..17   -> dw 0, then dw 2h, 2h + 1, 2h + 2 (codes shifted by 2)
//        kb 1: d 18-19, codes 20..35         -> dw 4 (d in the high half), dw 5 + 2h, 6 + 2h
//   Q5_0 kb 0: d 0-1, qh 2-5, codes 6..21    -> dw 0, 1 (d, qh shifted by 2), dw 1 + 2h .. 3 + 2h
//        kb 1: d 22-23, qh 24-27, codes 28.. -> dw 5, 6, dw 7 + 2h, 8 + 2h
//   Q8_0 kb 0: d 0-1, codes 2..33            -> dw 0, dw 2h .. 2h + 2, dw 4 + 2h .. 6 + 2h
//        kb 1: d 34-35, codes 36..67         -> dw 8, dw 9 + 2h, 10 + 2h, 13 + 2h, 14 + 2h
template <int DT, int KB>
struct Slots;
template <>
struct Slots<MOE_DT_Q4_0, 0> {
    static constexpr int n = 4;
    static constexpr int base[n] = {0, 0, 1, 2}, hm[n] = {0, 1, 1, 1};
};
template <>
struct Slots<MOE_DT_Q4_0, 1> {
    static constexpr int n = 3;
    static constexpr int base[n] = {4, 5, 6}, hm[n] = {0, 1, 1};
};
template <>
struct Slots<MOE_DT_Q5_0, 0> {
    static constexpr int n = 5;
    static constexpr int base[n] = {0, 1, 1, 2, 3}, hm[n] = {0, 0, 1, 1, 1};
};
template <>
struct Slots<MOE_DT_Q5_0, 1> {
    static constexpr int n = 4;
    static constexpr int base[n] = {5, 6, 7, 8}, hm[n] = {0, 0, 1, 1};
};
template <>
struct Slots<MOE_DT_Q8_0, 0> {
    static constexpr int n = 7;
    static constexpr int base[n] = {0, 0, 1, 2, 4, 5, 6}, hm[n] = {0, 1, 1, 1, 1, 1, 1};
};
template <>
struct Slots<MOE_DT_Q8_0, 1> {
    static constexpr int n = 5;
    static constexpr int base[n] = {8, 9, 10, 13, 14}, hm[n] = {0, 1, 1, 1, 1};
};
constexpr int kMaxSlots = 7;

// Four codes b0..b3 (bytes of c) as f16 pairs (b0, b1), (b2, b3) minus the
// code offset: 0x64 in each high byte makes the f16 exactly 1024 + b.
__device__ inline void codes_q(uint32_t c, __half2 off2, uint32_t (&o)[4], int i) {
    o[i] = h2_bits(__hsub2(as_h2(perm(0x64646464u, c, 0x04010400u)), off2));
    o[i + 1] = h2_bits(__hsub2(as_h2(perm(0x64646464u, c, 0x04030402u)), off2));
}
// Block KB's codes (m = 0, 1) and its scale d, from the slot dwords v.
template <int DT, int KB>
__device__ inline void decode2(const uint32_t *v, int h, half8 (&bq)[2], float &d) {
    const uint32_t s = KB == 0 ? (v[0] & 0xffffu) : (v[0] >> 16);
    d = __half2float(__ushort_as_half((unsigned short)s));
    uint32_t o[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        const uint32_t w0 = KB == 0 ? alignb(v[2], v[1], 2) : v[1];
        const uint32_t w1 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        codes_q(w0 & 0x0f0f0f0fu, off2, o, 0);
        codes_q(w1 & 0x0f0f0f0fu, off2, o, 2);
        bq[0] = pack8(o);
        codes_q((w0 >> 4) & 0x0f0f0f0fu, off2, o, 0);
        codes_q((w1 >> 4) & 0x0f0f0f0fu, off2, o, 2);
        bq[1] = pack8(o);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        const uint32_t qh = KB == 0 ? alignb(v[1], v[0], 2) : v[1];
        const uint32_t w0 = KB == 0 ? alignb(v[3], v[2], 2) : v[2];
        const uint32_t w1 = KB == 0 ? alignb(v[4], v[3], 2) : v[3];
        const uint32_t hb = qh >> (8 * h);
        codes_q((w0 & 0x0f0f0f0fu) | spread4(hb & 0xfu), off2, o, 0);
        codes_q((w1 & 0x0f0f0f0fu) | spread4((hb >> 4) & 0xfu), off2, o, 2);
        bq[0] = pack8(o);
        codes_q(((w0 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 16) & 0xfu), off2, o, 0);
        codes_q(((w1 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 20) & 0xfu), off2, o, 2);
        bq[1] = pack8(o);
    } else {
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const uint32_t *c = v + 1 + (KB == 0 ? 3 : 2) * m;
            const uint32_t w0 = KB == 0 ? alignb(c[1], c[0], 2) : c[0];
            const uint32_t w1 = KB == 0 ? alignb(c[2], c[1], 2) : c[1];
            codes_q(w0 ^ 0x80808080u, off2, o, 0);
            codes_q(w1 ^ 0x80808080u, off2, o, 2);
            bq[m] = pack8(o);
        }
    }
}

// DMAs per wave per step: one 32-row weight region (each wave of a SIMD
// loads one of the SIMD's two), and S of the 8 S activation DMAs.
template <int DT, int S>
constexpr int s2_nd() {
    return BLay<DT>::inst + S;
}
template <int DT, int S>
constexpr int s2_stages() {
    constexpr int per = 2 * s_act<S>() + BLay<DT>::stage;
    constexpr int by_lds = (160 * 1024 - 3 * 32 * S * 4) / per;
    constexpr int by_vm = 1 + 63 / s2_nd<DT, S>();
    constexpr int n = by_lds < by_vm ? by_lds : by_vm;
    return n > 12 ? 12 : n;
}
template <int DT, int S>
constexpr int s2_lds() {
    return s2_stages<DT, S>() * (2 * s_act<S>() + BLay<DT>::stage) + 3 * 32 * S * 4;
}

template <int DT, bool UP, int S>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void stream2_kernel(MfmaArgs a,
                                                                                                      int mode, int gx,
                                                                                                      int ksplit) {
    using BL = BLay<DT>;
    constexpr int BM = 32 * S;
    constexpr int NS = s2_stages<DT, S>();
    constexpr int AS = s_act<S>();
    constexpr int RS = 2 * AS + BL::stage;
    constexpr int NB = BL::inst;  // weight DMAs per wave per step
    static_assert(NS >= 3, "at least two steps in flight");
    static_assert(NS * RS >= 4 * 8192, "the accumulator exchange fits in the ring");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int *src_row = reinterpret_cast<int *>(smem + NS * RS);
    int *dst_row = src_row + BM;
    int *ex_row = dst_row + BM;

    TileInfo ti;
    if (!tile_of<BM, 32>(a, mode, gx, ti)) return;
    const ExpertDev &ex = a.experts[ti.g];
    const MatDev &W0 = UP ? ex.m[0] : ex.m[2];
    const MatDev &W1 = UP ? ex.m[1] : ex.m[2];
    const int n0 = ti.ntile * (UP ? SW / 2 : SW);
    if (n0 >= W0.rows) return;
    const int kspan = W0.cols / ksplit;
    const int kbeg = ti.ksplit * kspan;
    const int nsteps = kspan / SK;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sd = wv & 3, kh = wv >> 2;  // the wave's SIMD (its rows) and block of each step
    const int l32 = lane & 31, hf = lane >> 5;
    const int Icol = ti.shared ? a.I_s : a.I;
    const int valid = min(BM, ti.n - ti.m0);
    const int mt = (valid + 31) / 32;

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
    const lds_p sm = (lds_p)smem;
    const uint32_t arow_bytes = (uint32_t)(UP ? a.H : Icol) * 2;

    // Weight DMA: region kh of the SIMD's two (LDS region 2 sd + kh): up:
    // gate (kh 0) or up (kh 1) rows n0 + 32 sd ..; down: rows
    // n0 + 64 sd + 32 kh ..
    const MatDev &Wd = (UP && kh == 1) ? W1 : W0;
    const uint8_t *wbase = Wd.ptr;
    uint32_t woff[BL::inst];
    {
        const int row0 = UP ? n0 + 32 * sd : n0 + 64 * sd + 32 * kh;
        int row = row0 + l32;
        if (row >= Wd.rows) row = 0;
#pragma unroll
        for (int i = 0; i < BL::inst; i++) {
            const int qq = 64 * (i < BL::ix ? i : i - BL::ix) + lane;
            uint32_t off;
            if (i < BL::ix) {
                off = (uint32_t)row * Wd.stride + 16u * (uint32_t)(qq >> 5);
            } else {
                const int e = qq >> 5;
                off = e < BL::nd ? (uint32_t)row * Wd.stride + (uint32_t)(16 * BL::nx4 + 4 * e) : 0u;
            }
            woff[i] = off;
        }
    }
    // PK: one subtile of at most 16 tokens, whose hi and lo pieces share
    // the MFMAs' 32 rows (rows 16 + r carry token r's lo piece): half the
    // MFMAs and activation DMAs, and the two halves of each sum meet in the
    // fmas (C rows r and 16 + r sit in one lane, at v and v + 8).
    auto run = [&](auto mt_c, auto kh_c, auto pk_c) {
        constexpr int MT = decltype(mt_c)::value;
        constexpr int KH = decltype(kh_c)::value;  // == kh
        constexpr bool PK = decltype(pk_c)::value;
        static_assert(!PK || MT == 1, "packed pieces: one 16-token subtile");
        constexpr int NP = PK ? 1 : 2;  // MFMAs per 16-value half (one per piece unless packed)
        constexpr int NM = 4 * NP;      // MFMAs per subtile (two regions, two halves)
        constexpr int NV = PK ? 8 : 16; // accumulator values that hold tokens
        // Activations of subtile t, this wave's block KH, MFMA m (piece p at
        // + p AS; packed: lane l32 reads piece l32 / 16, row l32 % 16).
        uint32_t aoff[2];
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const int r = PK ? (l32 & 15) : l32;
            aoff[m] = (uint32_t)r * 128u + ((uint32_t)((4 * KH + 2 * m + hf) ^ ((r >> 1) & 7)) << 4) +
                      (PK ? (uint32_t)(l32 >> 4) * AS : 0u);
        }
        // Activation DMAs per wave per step: the step's 8 MT (packed: 4, from
        // the waves of block 0).
        constexpr int NA = PK ? (KH == 0 ? 1 : 0) : MT;
        constexpr int GA = PK ? 2 : 4 * MT;  // 8-row groups per piece
        constexpr int ND = NB + NA;
        static_assert((NS - 1) * ND <= 63, "vmcnt range");
        floatx16 acc[MT][2];
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[t][j] = floatx16{};
        // Activation DMA u of this wave: instruction q = wv + 8 u of the
        // step's 2 GA (piece q / GA, 8-row group q % GA).
        constexpr int NA1 = NA > 0 ? NA : 1;
        uint32_t aoffg[NA1], adst[NA1];
        const uint16_t *asrc[NA1];
#pragma unroll
        for (int u = 0; u < NA; u++) {
            const int qd = wv + 8 * u, p = qd / GA, i = qd % GA;
            const int r = 8 * i + (lane >> 3);
            const int sr = src_row[r < valid ? r : 0];
            aoffg[u] = (uint32_t)sr * arow_bytes + (uint32_t)kbeg * 2u + (uint32_t)(((lane & 7) ^ ((r >> 1) & 7)) << 4);
            adst[u] = (uint32_t)p * AS + (uint32_t)i * 1024u;
            asrc[u] = p == 0 ? ahi : alo;
        }
        auto dma = [&](auto d_c, int step, int st) {
            constexpr int d = decltype(d_c)::value;
            const int sc = step < nsteps ? step : nsteps - 1;
            const uint32_t sb = lds0 + (uint32_t)st * RS;
            if constexpr (d < NB) {
                const uint8_t *wb = wbase + (size_t)(kbeg / 32 + 2 * sc) * Fmt<DT>::bytes;
                const uint32_t lr = sb + 2 * AS + (uint32_t)(2 * sd + kh) * BL::region;
                if constexpr (d < BL::ix)
                    dma16(wb, woff[d], lr + 1024u * d);
                else
                    dma4(wb, woff[d], lr + BL::xbytes + 256u * (d - BL::ix));
            } else {
                constexpr int u = d - NB;
                dma16(reinterpret_cast<const uint8_t *>(asrc[u]) + (size_t)sc * (SK * 2), aoffg[u], sb + adst[u]);
            }
        };
        auto dma_all = [&](int step, int st) {
            static_for<0, ND>([&](auto d_c) { dma(d_c, step, st); });
        };
        // A step's DMAs go out spread over the subtiles after the barrier
        // that frees their stage: the weights between the MFMAs of the
        // step's last subtile, the activations Q per subtile of the next
        // step (all between the last subtile's MFMAs when there is only
        // one).  Issued together, the eight waves' DMAs would queue in the
        // CU's memory pipeline and stall their waves and the barrier that
        // follows; between MFMAs a wave's stall leaves the matrix pipe busy.
        constexpr int K0 = MT == 1 ? ND : NB;
        constexpr int Q = MT == 1 ? 0 : (ND - K0 + MT - 2) / (MT - 1);
        auto dma_part = [&](auto t_c, int step, int st) {
            constexpr int t = decltype(t_c)::value;
            static_for<(K0 + t * Q < ND ? K0 + t * Q : ND), (K0 + (t + 1) * Q < ND ? K0 + (t + 1) * Q : ND)>(
                [&](auto d_c) { dma(d_c, step, st); });
        };

        // Activation fragments (hi m0, lo m0, hi m1, lo m1) of one subtile;
        // with room in the registers (tiles of at most 128 tokens) the next
        // subtile's are read while this one's MFMAs run.
        constexpr int NAB = S <= 4 ? 2 : 1;
        half8 Ab[NAB][4];
        half8 B[2][2];   // [region][m] codes of this wave's block
        float dsc[2];    // [region] its scale
        uint32_t raw[1][kMaxSlots];
        auto read_a = [&](int st, int t, half8(&A)[4]) {
            const lds_p p = sm + st * RS + 4096 * t;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                if constexpr (PK) {
                    A[m] = lds_h8(p + aoff[m]);
                } else {
                    A[2 * m] = lds_h8(p + aoff[m]);
                    A[2 * m + 1] = lds_h8(p + AS + aoff[m]);
                }
            }
        };
        auto decode_block = [&](int st) {
            using SL = Slots<DT, KH>;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const lds_p rb = sm + st * RS + 2 * AS + (2 * sd + j) * BL::region;
#pragma unroll
                for (int k = 0; k < SL::n; k++) raw[0][k] = lds_u32(rb + BL::loc(SL::base[k] + 2 * hf * SL::hm[k], l32));
                decode2<DT, KH>(raw[0], hf, B[j], dsc[j]);
            }
        };
        // Subtile t: the block's sums P of both regions, NM / 2 MFMAs
        // each, then acc += d P.  Region 1's MFMAs go out before region 0's
        // fmas (which wait for region 0's sums), and region 1's fmas follow
        // the next subtile's region-0 MFMAs, so each wave's fmas run beside
        // its own MFMAs as well as its partner's.  MFMA i: region i / (2 NP),
        // half m, piece p.
        floatx16 ps[2];
        auto mm = [&](auto i_c, const half8(&A)[4]) {
            constexpr int i = decltype(i_c)::value;
            constexpr int j = i / (2 * NP), m = (i % (2 * NP)) / NP, p = i % NP;
            ps[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[NP * m + p], B[j][m],
                                                           (i % (2 * NP)) ? ps[j] : floatx16{}, 0, 0, 0);
        };
        auto scale_add = [&](int t, int j) {
            if constexpr (PK) {
#pragma unroll
                for (int v = 0; v < 8; v++) acc[t][j][v] = fmaf(dsc[j], ps[j][v] + ps[j][v + 8], acc[t][j][v]);
            } else {
#pragma unroll
                for (int v = 0; v < 16; v++) acc[t][j][v] = fmaf(dsc[j], ps[j][v], acc[t][j][v]);
            }
        };
        constexpr int WAIT_STEP = (NS - 2) * ND;  // step s + 1 complete

        for (int p = 0; p < NS - 1; p++) dma_all(p, p);
        wait_vm_barrier<WAIT_STEP>();
        static_for<0, K0>([&](auto d_c) { dma(d_c, NS - 1, NS - 1); });
        decode_block(0);

        // Across steps too when the step has an even number of subtiles
        // (the last one then uses buffer 1); otherwise each step reads its
        // first subtile's fragments itself.
        constexpr bool XS = NAB == 2 && MT % 2 == 0;
        int st = 0;
        if constexpr (XS) read_a(0, 0, Ab[0]);
        for (int s = 0; s < nsteps; s++) {
            const int st1 = st + 1 == NS ? 0 : st + 1;
            const int st0 = st == 0 ? NS - 1 : st - 1;  // the stage step s + NS - 1's DMAs fill
            static_for<0, MT>([&](auto t_c) {
                constexpr int t = decltype(t_c)::value;
                constexpr int ab = NAB == 2 ? t & 1 : 0;  // this subtile's buffer
                if constexpr (NAB == 1 || (t == 0 && !XS)) read_a(st, t, Ab[0]);
                if constexpr (NAB == 2 && t + 1 < MT) read_a(st, t + 1, Ab[ab ^ 1]);
                if constexpr (t == MT - 1) {
                    // Every read of this stage is done (the weights were
                    // decoded at the end of the previous step): wait for
                    // step s + 1, meet the other waves, start refilling this
                    // stage.
                    wait_vm_barrier<WAIT_STEP>();
                    // (two buffers: the next step's first subtile, from the
                    // stage the barrier completed)
                    if constexpr (XS) read_a(st1, 0, Ab[0]);
                } else {
                    dma_part(t_c, s + NS - 1, st0);
                }
                static_for<0, NM>([&](auto i_c) {
                    constexpr int i = decltype(i_c)::value;
                    mm(i_c, Ab[ab]);
                    if constexpr (i == NM / 2 - 1 && t > 0) scale_add(t - 1, 1);
                    if constexpr (t == MT - 1) {
                        // The refill of this stage: DMAs d0 .. d1 - 1 of
                        // the K0 after MFMA i.
                        constexpr int d0 = (K0 * i + NM - 1) / NM, d1 = (K0 * (i + 1) + NM - 1) / NM;
                        if constexpr (d1 > d0) {
                            __builtin_amdgcn_sched_barrier(0);
                            static_for<d0, d1>([&](auto d_c) { dma(d_c, s + NS, st); });
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                });
                scale_add(t, 0);
                __builtin_amdgcn_sched_barrier(0);
            });
            // The last subtile's region-1 fmas, then the next step's codes
            // and scales (its weights are complete and, after the barrier,
            // visible from both waves of the SIMD).
            scale_add(MT - 1, 1);
            decode_block(st1);
            st = st1;
        }
        wait_vm<0>();
        __syncthreads();

        // ---- epilogue: the two halves of each subtile meet in LDS (the
        // ring is free): the wave that does not own subtile t (owner: the
        // wave of block t & 1) writes its sums, the owner adds them and
        // stores.  Lane holds C[32 t + 8 (v / 4) + 4 hf + v % 4][row l32 of
        // region j], scaled by 2^ex_row.
        float *xb = reinterpret_cast<float *>(smem) + sd * 2048;
#pragma unroll
        for (int t = 0; t < MT; t++) {
            if (KH != (t & 1)) {
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int v = 0; v < NV; v++) xb[(j * 16 + v) * 64 + lane] = acc[t][j][v];
            }
            __syncthreads();
            if (KH == (t & 1)) {
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[t][j][v] += xb[(j * 16 + v) * 64 + lane];
                if (UP) {
                    float *hout = ti.shared ? a.hs : a.h;
                    const int col = n0 + 32 * sd + l32;
                    if (col < W0.rows) {
#pragma unroll
                        for (int v = 0; v < NV; v++) {
                            const int row = 32 * t + 8 * (v / 4) + 4 * hf + (v % 4);
                            const int d = dst_row[row];
                            if (d < 0) continue;
                            const int e = ex_row[row];
                            const float g = ldexpf(acc[t][0][v], -e), u = ldexpf(acc[t][1][v], -e);
                            hout[(size_t)d * Icol + col] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                        }
                    }
                } else {
                    float *yout = ti.shared ? a.ys + ti.ksplit * a.yspart : a.y + ti.ksplit * a.ypart;
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int col = n0 + 64 * sd + 32 * j + l32;
                        if (col >= W0.rows) continue;
#pragma unroll
                        for (int v = 0; v < NV; v++) {
                            const int row = 32 * t + 8 * (v / 4) + 4 * hf + (v % 4);
                            const int d = dst_row[row];
                            if (d >= 0) yout[(size_t)d * a.H + col] = ldexpf(acc[t][j][v], -ex_row[row]);
                        }
                    }
                }
            }
            __syncthreads();
        }
    };
    auto run_kh = [&](auto mt_c, auto pk_c) {
        if (kh == 0)
            run(mt_c, std::integral_constant<int, 0>{}, pk_c);
        else
            run(mt_c, std::integral_constant<int, 1>{}, pk_c);
    };
    using NoPk = std::false_type;
    switch (mt) {
    case 1:
        if (valid <= 16)
            run_kh(std::integral_constant<int, 1>{}, std::true_type{});
        else
            run_kh(std::integral_constant<int, 1>{}, NoPk{});
        break;
    case 2: if constexpr (S >= 2) run_kh(std::integral_constant<int, 2>{}, NoPk{}); break;
    case 3: if constexpr (S >= 3) run_kh(std::integral_constant<int, 3>{}, NoPk{}); break;
    case 4: if constexpr (S >= 4) run_kh(std::integral_constant<int, 4>{}, NoPk{}); break;
    default: if constexpr (S >= 5) run_kh(std::integral_constant<int, 5>{}, NoPk{}); break;
    }
}

// ---- the tiled layout and its one-subtile kernel ------------------------------
// Tiles of at most 32 tokens (about 4 to 20 per expert) carry too few
// products per weight byte for the LDS ring: their time is the weight
// stream's.  Read row-major, a 32-row region's ring step is a gather of 32
// rows 36 bytes apart in 32 cache lines, which the CU serves at about a
// third of HBM speed.  The tiled copy lays each 32-row region's steps out
// contiguously, and inside a row's step puts the bytes each MFMA lane needs
// next to each other:
//   region r, step s at ((r * steps + s) * 32 + l) * RB bytes for row l of
//   the region (rows past the matrix's are zero), RB = two blocks' bytes;
//   Q4_0 (36): d0 d1 | codes0[0:8] codes1[0:8] | codes0[8:16] codes1[8:16]
//   Q5_0 (44): d0 d1 | qh0 | qh1 | codes0[0:8] codes1[0:8] | codes0[8:16] codes1[8:16]
//   Q8_0 (68): d0 d1 | c0[0:8] c0[16:24] c1[0:8] c1[16:24] | c0[8:16] c0[24:32] c1[8:16] c1[24:32]
// so lane (l32, hf) loads the head (scales, and Q5_0's high bits) and its
// own half's 16 (Q8_0: 32) code bytes, and a wave's loads of a step cover
// 32 RB contiguous bytes.  Each of the eight waves owns one region for the
// whole K (SIMD sd: regions 2 sd and 2 sd + 1 of the tile; up: gate (j = 0)
// and up (j = 1) rows n0 + 32 sd ..; down: rows n0 + 64 sd + 32 j ..) and
// keeps P steps of it in flight in registers; the activations go through
// LDS in groups of G steps, double-buffered, filled by plain loads (issued
// P steps ahead, written G steps ahead) and published by one barrier per
// group.  Tiles of
// at most 16 tokens pack their hi and lo pieces into the MFMAs' 32 rows, and
// tiles of at most 8 skip the fmas of the rows that hold no token.
template <int DT>
struct Tiled;
template <>
struct Tiled<MOE_DT_Q4_0> {
    static constexpr int rb = 36, head = 1, half = 4, nd = head + half;
    // source byte (of the row's two blocks) of each tiled byte
    static constexpr unsigned char src[rb] = {0,  1,  18, 19, 2,  3,  4,  5,  6,  7,  8,  9,
                                              20, 21, 22, 23, 24, 25, 26, 27, 10, 11, 12, 13,
                                              14, 15, 16, 17, 28, 29, 30, 31, 32, 33, 34, 35};
};
template <>
struct Tiled<MOE_DT_Q5_0> {
    static constexpr int rb = 44, head = 3, half = 4, nd = head + half;
    static constexpr unsigned char src[rb] = {0,  1,  22, 23, 2,  3,  4,  5,  24, 25, 26, 27, 6,  7,  8,
                                              9,  10, 11, 12, 13, 28, 29, 30, 31, 32, 33, 34, 35, 14, 15,
                                              16, 17, 18, 19, 20, 21, 36, 37, 38, 39, 40, 41, 42, 43};
};
template <>
struct Tiled<MOE_DT_Q8_0> {
    static constexpr int rb = 68, head = 1, half = 8, nd = head + half;
    static constexpr unsigned char src[rb] = {
        0,  1,  34, 35,                                  // d0 d1
        2,  3,  4,  5,  6,  7,  8,  9,  18, 19, 20, 21, 22, 23, 24, 25,   // c0[0:8] c0[16:24]
        36, 37, 38, 39, 40, 41, 42, 43, 52, 53, 54, 55, 56, 57, 58, 59,   // c1[0:8] c1[16:24]
        10, 11, 12, 13, 14, 15, 16, 17, 26, 27, 28, 29, 30, 31, 32, 33,   // c0[8:16] c0[24:32]
        44, 45, 46, 47, 48, 49, 50, 51, 60, 61, 62, 63, 64, 65, 66, 67};  // c1[8:16] c1[24:32]
};
template <int DT>
struct TiledStep {
    static constexpr int rb = Tiled<DT>::rb, step_bytes = 32 * rb;
};
// Steps of weights in flight per wave.
template <int DT>
constexpr int tiled_ring() {
    return DT == MOE_DT_Q4_0 ? 8 : 6;
}
typedef uint32_t u32x2_dw __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3_dw __attribute__((ext_vector_type(3), aligned(4)));
// Lane hf's dwords of one row step at p: the head, then its half.
template <int DT>
__device__ inline void tiled_load(const uint8_t *p, int hf, uint32_t (&v)[Tiled<DT>::nd]) {
    using TL = Tiled<DT>;
    const gptr<uint32_t> q = (gptr<uint32_t>)p;
    if constexpr (TL::head == 1) {
        v[0] = *q;
    } else {
        const u32x3_dw h = *(gptr<u32x3_dw>)q;
        v[0] = h.x, v[1] = h.y, v[2] = h.z;
    }
#pragma unroll
    for (int i = 0; i < TL::half / 4; i++) {
        const u32x4_dw c = *(gptr<u32x4_dw>)(q + TL::head + TL::half * hf + 4 * i);
        v[TL::head + 4 * i] = c.x, v[TL::head + 4 * i + 1] = c.y, v[TL::head + 4 * i + 2] = c.z,
                       v[TL::head + 4 * i + 3] = c.w;
    }
}
// Block KB's codes (m = 0, 1) and scale from a lane's tiled dwords (the
// same values as decode2 gives from the row-major slots).
template <int DT, int KB>
__device__ inline void tiled_decode(const uint32_t *v, int h, half8 (&bq)[2], float &d) {
    const uint32_t s = KB == 0 ? (v[0] & 0xffffu) : (v[0] >> 16);
    d = __half2float(__ushort_as_half((unsigned short)s));
    uint32_t o[4];
    if constexpr (DT == MOE_DT_Q4_0) {
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        const uint32_t w0 = v[1 + 2 * KB], w1 = v[2 + 2 * KB];
        codes_q(w0 & 0x0f0f0f0fu, off2, o, 0);
        codes_q(w1 & 0x0f0f0f0fu, off2, o, 2);
        bq[0] = pack8(o);
        codes_q((w0 >> 4) & 0x0f0f0f0fu, off2, o, 0);
        codes_q((w1 >> 4) & 0x0f0f0f0fu, off2, o, 2);
        bq[1] = pack8(o);
    } else if constexpr (DT == MOE_DT_Q5_0) {
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        const uint32_t w0 = v[3 + 2 * KB], w1 = v[4 + 2 * KB];
        const uint32_t hb = v[1 + KB] >> (8 * h);
        codes_q((w0 & 0x0f0f0f0fu) | spread4(hb & 0xfu), off2, o, 0);
        codes_q((w1 & 0x0f0f0f0fu) | spread4((hb >> 4) & 0xfu), off2, o, 2);
        bq[0] = pack8(o);
        codes_q(((w0 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 16) & 0xfu), off2, o, 0);
        codes_q(((w1 >> 4) & 0x0f0f0f0fu) | spread4((hb >> 20) & 0xfu), off2, o, 2);
        bq[1] = pack8(o);
    } else {
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
#pragma unroll
        for (int m = 0; m < 2; m++) {
            codes_q(v[1 + 4 * KB + 2 * m] ^ 0x80808080u, off2, o, 0);
            codes_q(v[2 + 4 * KB + 2 * m] ^ 0x80808080u, off2, o, 2);
            bq[m] = pack8(o);
        }
    }
}

// One thread per (region, step, row): the row's step, permuted.
template <int DT>
__global__ __launch_bounds__(256) void tile_kernel(MatDev m, uint8_t *__restrict__ dst, size_t n) {
    using TL = Tiled<DT>;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int steps = m.cols / SK;
    const int l = (int)(i & 31);
    const size_t rs = i >> 5;
    const int s = (int)(rs % steps);
    const int row = (int)(rs / steps) * 32 + l;
    uint32_t in[TL::rb / 4], out[TL::rb / 4];
    if (row < m.rows) {
        const uint32_t *p = reinterpret_cast<const uint32_t *>(m.ptr + (size_t)row * m.stride + (size_t)s * TL::rb);
#pragma unroll
        for (int k = 0; k < TL::rb / 4; k++) in[k] = gload(p + k);
    } else {
#pragma unroll
        for (int k = 0; k < TL::rb / 4; k++) in[k] = 0;
    }
#pragma unroll
    for (int k = 0; k < TL::rb / 4; k++) {
        uint32_t w = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int sb = TL::src[4 * k + b];
            w |= ((in[sb >> 2] >> (8 * (sb & 3))) & 0xffu) << (8 * b);
        }
        out[k] = w;
    }
    uint32_t *q = reinterpret_cast<uint32_t *>(dst + i * TL::rb);
#pragma unroll
    for (int k = 0; k < TL::rb / 4; k++) gstore(q + k, out[k]);
}

template <int DT, bool UP>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void tiled_kernel(MfmaArgs a,
                                                                                                    int mode, int gx,
                                                                                                    int ksplit) {
    using TL = Tiled<DT>;
    using TS = TiledStep<DT>;
    constexpr int ND = TL::nd;
    constexpr int P = tiled_ring<DT>();
    constexpr int G = 2;  // steps of activations per LDS group (one barrier per group)
    static_assert(P % G == 0, "ring rounds hold whole groups");
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * G * 8192];
    __shared__ int src_row[32], dst_row[32], ex_row[32];

    TileInfo ti;
    if (!tile_of<32, 32, UP>(a, mode, gx, ti)) return;
    const ExpertDev &ex = a.experts[ti.g];
    const MatDev &W0 = UP ? ex.m[0] : ex.m[2];
    const MatDev &W1 = UP ? ex.m[1] : ex.m[2];
    const int n0 = ti.ntile * (UP ? SW / 2 : SW);
    if (n0 >= W0.rows) return;
    const int kspan = W0.cols / ksplit;
    int kbeg = ti.ksplit * kspan;
    int nsteps = kspan / SK;
    // A tile of the launch's last round split along K (gate/up): half 0
    // takes the first nsteps / 2 steps, half 1 the rest.
    const bool khalf = UP && ti.khalf >= 0;
    if (khalf) {
        const int h0 = nsteps / 2;
        kbeg += ti.khalf ? h0 * SK : 0;
        nsteps = ti.khalf ? nsteps - h0 : h0;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sd = wv & 3, j = wv >> 2;  // the wave's SIMD and region
    const int l32 = lane & 31, hf = lane >> 5;
    const int Icol = ti.shared ? a.I_s : a.I;
    const int valid = min(32, ti.n - ti.m0);

    const uint16_t *ahi = UP ? a.xhi : (ti.shared ? a.hshi : a.hhi);
    const uint16_t *alo = UP ? a.xlo : (ti.shared ? a.hslo : a.hlo);
    const int32_t *aex = UP ? a.xex : (ti.shared ? a.hsex : a.hex);
    if (tid < 32) {
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

    // The wave's region of the tiled copy (a region past the matrix's rows,
    // whose sums no one stores, reads region 0), lane l32's row in it.
    const MatDev &Wd = (UP && j == 1) ? W1 : W0;
    const int row0 = UP ? n0 + 32 * sd : n0 + 64 * sd + 32 * j;
    const size_t region = row0 < Wd.rows ? (size_t)(row0 / 32) : 0;
    const uint8_t *wp = Wd.tiled + (region * (size_t)(Wd.cols / SK) + (size_t)(kbeg / SK)) * TS::step_bytes +
                        (size_t)l32 * TL::rb;
    const size_t arow_bytes = (size_t)(UP ? a.H : Icol) * 2;
    const lds_p sm = (lds_p)smem;

    // NV: accumulator values that hold tokens (C rows 8 (v / 4) + 4 hf + v % 4
    // for v < NV): 16 unpacked, 8 packed, 4 for at most 8 tokens.
    auto run = [&](auto pk_c, auto nv_c) {
        constexpr bool PK = decltype(pk_c)::value;
        constexpr int NP = PK ? 1 : 2;    // pieces per MFMA operand set
        constexpr int NV = decltype(nv_c)::value;
        constexpr int AST = PK ? 4096 : 8192;  // activation bytes per step
        // Activation staging: thread tid moves AB bytes of each step.
        //   unpacked: piece tid / 256, token row (tid / 8) % 32, 16-byte chunk tid % 8
        //   packed:   MFMA row tid / 16 (piece row / 16, token row % 16), 8-byte unit tid % 16
        constexpr int AB = PK ? 8 : 16;
        const int arow = PK ? (tid >> 4) : ((tid >> 3) & 31);      // MFMA row in the stage
        const int apiece = PK ? (arow >> 4) : (tid >> 8);
        const int atok = PK ? (arow & 15) : arow;
        const int achunk = PK ? ((tid & 15) >> 1) : (tid & 7);
        const int sr = src_row[atok < valid ? atok : 0];
        const uint8_t *asrc = reinterpret_cast<const uint8_t *>(apiece ? alo : ahi) + (size_t)sr * arow_bytes +
                              (size_t)kbeg * 2 + (size_t)(PK ? 8 * (tid & 15) : 16 * (tid & 7));
        const uint32_t adst = (uint32_t)(PK ? 0 : apiece * 4096) + (uint32_t)arow * 128u +
                              ((uint32_t)(achunk ^ ((arow >> 1) & 7)) << 4) + (PK ? 8u * (tid & 1) : 0u);
        typedef uint32_t areg_t __attribute__((ext_vector_type(AB / 4)));
        auto aload = [&](int step) {
            const int sc = step < nsteps ? step : nsteps - 1;
            return *(gptr<areg_t>)(asrc + (size_t)sc * (SK * 2));
        };
        // Step q's activations: stage (group q / G's buffer, q % G of it).
        auto stage_of = [&](int q) { return ((q / G) & 1) * G + q % G; };
        auto awrite = [&](int q, areg_t v) { *(lptr<areg_t>)(smem + stage_of(q) * 8192 + adst) = v; };
        // A fragments of step stage `stage`: block kb, half m, piece p.
        uint32_t aoff[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int m = 0; m < 2; m++)
                aoff[kb][m] = (uint32_t)l32 * 128u + ((uint32_t)((4 * kb + 2 * m + hf) ^ ((l32 >> 1) & 7)) << 4);

        floatx16 acc = floatx16{};
        uint32_t raw[P][ND];
        areg_t areg[P];
        // Prologue: group 0's activations into its stages, then the loads
        // of steps G .. G + P - 1 (activations) and 0 .. P - 1 (weights) in
        // the order the loop issues them, so that the loop's waits find the
        // same number of loads in flight on its first round as on the
        // others.
        {
            areg_t a0[G];
#pragma unroll
            for (int g = 0; g < G; g++) a0[g] = aload(g);
#pragma unroll
            for (int i = 0; i < P; i++) {
                areg[(i + G) % P] = aload(i + G);
                tiled_load<DT>(wp + (size_t)(i < nsteps ? i : nsteps - 1) * TS::step_bytes, hf, raw[i]);
            }
#pragma unroll
            for (int g = 0; g < G; g++) awrite(g, a0[g]);
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

        // Step s with ring slot i = s % P, software-pipelined over three
        // steps: step s's MFMAs go out, then step s - 1's fmas (its sums
        // long done), then step s + 1's codes are decoded, so no wave waits
        // on its own MFMAs.  The codes, scales and sums of a step live in the
        // register set of its parity (P is even, so i & 1 is s's parity).
        static_assert(P % 2 == 0, "ring slots keep the steps' parity");
        half8 Bq[2][2][2];  // [parity][block][m]
        float dq[2][2];     // [parity][block]
        floatx16 pq[2][2];  // [parity][block]
        auto decode = [&](int slot_dummy, const uint32_t(&v)[ND], int q) {
            (void)slot_dummy;
            tiled_decode<DT, 0>(v, hf, Bq[q][0], dq[q][0]);
            tiled_decode<DT, 1>(v, hf, Bq[q][1], dq[q][1]);
        };
        auto scale_add = [&](int q) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int v = 0; v < NV; v++)
                    acc[v] = fmaf(dq[q][kb], PK ? pq[q][kb][v] + pq[q][kb][v + 8] : pq[q][kb][v], acc[v]);
            }
        };
        decode(0, raw[0], 0);
        pq[1][0] = pq[1][1] = floatx16{};
        dq[1][0] = dq[1][1] = 0.0f;
        auto step = [&](auto i_c, int s) {
            constexpr int i = decltype(i_c)::value, i1 = (i + 1) % P, q = i & 1, ia = (i + G) % P;
            // Step s + G's activations into the next group's buffer (last
            // read before the previous group's barrier), then the loads of
            // step s + G + P into the freed registers.
            awrite(s + G, areg[ia]);
            areg[ia] = aload(s + G + P);
            const lds_p st = sm + stage_of(s) * 8192;
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int m = 0; m < 2; m++) {
#pragma unroll
                    for (int p = 0; p < NP; p++) {
                        const half8 A = lds_h8(st + p * 4096 + aoff[kb][m]);
                        pq[q][kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, Bq[q][kb][m],
                                                                           (m | p) ? pq[q][kb] : floatx16{}, 0, 0, 0);
                    }
                }
            }
            scale_add(q ^ 1);  // step s - 1 (zero sums before the first step)
            decode(i1, raw[i1], q ^ 1);
            // The codes and scales exist in registers of their own before
            // the slot's next load is issued: the compiler would otherwise
            // keep reading the loaded registers, hold them across the load
            // and copy them at the loop's end, waiting for loads in flight.
            asm volatile("" : "+v"(dq[q ^ 1][0]), "+v"(dq[q ^ 1][1]), "+v"(Bq[q ^ 1][0][0]), "+v"(Bq[q ^ 1][0][1]),
                         "+v"(Bq[q ^ 1][1][0]), "+v"(Bq[q ^ 1][1][1]));
            tiled_load<DT>(wp + (size_t)(s + P < nsteps ? s + P : nsteps - 1) * TS::step_bytes, hf, raw[i]);
            // The group's last step: publish the next group, free this one.
            if constexpr ((i + 1) % G == 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);  // each step's code stays in its step
        };
        // Whole rounds of the ring without guards (a guard per step would
        // merge each slot's registers with their reloaded values and copy
        // them, waiting for loads just issued), then the rest.
        int s0 = 0;
        for (; s0 + P <= nsteps; s0 += P) static_for<0, P>([&](auto i_c) { step(i_c, s0 + decltype(i_c)::value); });
        static_for<0, P>([&](auto i_c) {
            if (s0 + decltype(i_c)::value < nsteps) step(i_c, s0 + decltype(i_c)::value);
        });
        if ((nsteps - 1) & 1)  // the last step's fmas
            scale_add(1);
        else
            scale_add(0);
        // Every wave's last reads of the stages are done before the epilogue
        // reuses their memory (a last group of fewer than G steps ends
        // without a barrier).
        __syncthreads();

        // A K half: both blocks write their sums to the tile's slot; the one
        // that counts second adds the other's and goes on, the first is done
        // (no block waits for another).  Sums of either half are added in
        // the same order whichever finishes first (a + b = b + a).
        if (khalf) {
            float *part = a.tail_part + (size_t)ti.slot * (2 * 8 * 16 * 64);
#pragma unroll
            for (int v = 0; v < NV; v++) part[((ti.khalf * 8 + wv) * 16 + v) * 64 + lane] = acc[v];
            __syncthreads();
            __shared__ int s_second;
            if (tid == 0) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
                const bool second = atomicAdd(&a.tail_cnt[ti.slot], 1u) == 1u;
                if (second) {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    a.tail_cnt[ti.slot] = 0u;  // zero for the next call
                }
                s_second = second;
            }
            __syncthreads();
            if (!s_second) return;
#pragma unroll
            for (int v = 0; v < NV; v++) acc[v] += part[(((1 - ti.khalf) * 8 + wv) * 16 + v) * 64 + lane];
            __syncthreads();
        }

        // ---- epilogue.  Lane holds C[8 (v / 4) + 4 hf + v % 4][row l32 of
        // its region], scaled by 2^ex_row.
        if (UP) {
            // The up wave (j = 1) hands its sums to the gate wave of its SIMD.
            float *xb = reinterpret_cast<float *>(smem) + sd * 1024;
            if (j == 1) {
#pragma unroll
                for (int v = 0; v < NV; v++) xb[v * 64 + lane] = acc[v];
            }
            __syncthreads();
            if (j == 0) {
                float *hout = ti.shared ? a.hs : a.h;
                const int col = n0 + 32 * sd + l32;
                if (col < W0.rows) {
#pragma unroll
                    for (int v = 0; v < NV; v++) {
                        const int row = 8 * (v / 4) + 4 * hf + (v % 4);
                        const int d = dst_row[row];
                        if (d < 0) continue;
                        const int e = ex_row[row];
                        const float g = ldexpf(acc[v], -e), u = ldexpf(xb[v * 64 + lane], -e);
                        hout[(size_t)d * Icol + col] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    }
                }
            }
        } else {
            float *yout = ti.shared ? a.ys + ti.ksplit * a.yspart : a.y + ti.ksplit * a.ypart;
            const int col = n0 + 64 * sd + 32 * j + l32;
            if (col < W0.rows) {
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const int row = 8 * (v / 4) + 4 * hf + (v % 4);
                    const int d = dst_row[row];
                    if (d >= 0) yout[(size_t)d * a.H + col] = ldexpf(acc[v], -ex_row[row]);
                }
            }
        }
    };
    if (valid <= 8)
        run(std::true_type{}, std::integral_constant<int, 4>{});
    else if (valid <= 16)
        run(std::true_type{}, std::integral_constant<int, 8>{});
    else
        run(std::false_type{}, std::integral_constant<int, 16>{});
}

template <int DT, bool UP, int S>
hipError_t launch_s(dim3 grid, const MfmaArgs &a, int mode, int ksplit, bool tiled, hipStream_t s) {
    // One-subtile tiles stream the tiled copies; wider tiles read the
    // row-major matrices, which every layer keeps.
    if constexpr (S == 1) {
        if (tiled) {
            hipLaunchKernelGGL((tiled_kernel<DT, UP>), grid, dim3(512), 0, s, a, mode, (int)grid.x, ksplit);
            return hipGetLastError();
        }
    }
    constexpr int lds = s2_lds<DT, S>();
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&stream2_kernel<DT, UP, S>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((stream2_kernel<DT, UP, S>), grid, dim3(512), lds, s, a, mode, (int)grid.x, ksplit);
    return hipGetLastError();
}

template <int DT, bool UP>
hipError_t launch_fmt(int bm, dim3 grid, const MfmaArgs &a, int mode, int ksplit, bool tiled, hipStream_t s) {
    switch (bm) {
    case 32: return launch_s<DT, UP, 1>(grid, a, mode, ksplit, tiled, s);
    case 64: return launch_s<DT, UP, 2>(grid, a, mode, ksplit, tiled, s);
    case 128: return launch_s<DT, UP, 4>(grid, a, mode, ksplit, tiled, s);
    case 160:
        if constexpr (DT != MOE_DT_Q8_0) return launch_s<DT, UP, 5>(grid, a, mode, ksplit, tiled, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

template <bool UP>
hipError_t launch_dt(int dt, int bm, dim3 grid, const MfmaArgs &a, int mode, int ksplit, bool tiled, hipStream_t s) {
    switch (dt) {
    case MOE_DT_Q4_0: return launch_fmt<MOE_DT_Q4_0, UP>(bm, grid, a, mode, ksplit, tiled, s);
    case MOE_DT_Q5_0: return launch_fmt<MOE_DT_Q5_0, UP>(bm, grid, a, mode, ksplit, tiled, s);
    case MOE_DT_Q8_0: return launch_fmt<MOE_DT_Q8_0, UP>(bm, grid, a, mode, ksplit, tiled, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Token tile for a launch whose tiles average `tokens` tokens: the smallest
// of 32, 64, 128 and 160 that holds them with room for the spread of the
// experts' counts (160 only where no matrix is Q8_0, whose ring needs the
// LDS).
int stream_tile(double tokens, bool q8) {
    const double need = tokens * 1.15 + 8.0;
    for (int b : {32, 64, 128})
        if (b >= need) return b;
    return q8 ? 128 : 160;
}

size_t tiled_bytes(const MatDev &m) {
    if (m.cols <= 0 || m.cols % SK || m.rows <= 0) return 0;
    size_t rb = 0;
    switch (m.dt) {
    case MOE_DT_Q4_0: rb = Tiled<MOE_DT_Q4_0>::rb; break;
    case MOE_DT_Q5_0: rb = Tiled<MOE_DT_Q5_0>::rb; break;
    case MOE_DT_Q8_0: rb = Tiled<MOE_DT_Q8_0>::rb; break;
    default: return 0;
    }
    return (size_t)((m.rows + 31) / 32) * (m.cols / SK) * 32 * rb;
}

hipError_t tile_matrix(const MatDev &m, uint8_t *dst, hipStream_t s) {
    const size_t bytes = tiled_bytes(m);
    if (!bytes || !dst) return hipErrorInvalidValue;
    const size_t n = (size_t)((m.rows + 31) / 32) * (m.cols / SK) * 32;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (m.dt) {
    case MOE_DT_Q4_0: hipLaunchKernelGGL(tile_kernel<MOE_DT_Q4_0>, grid, dim3(256), 0, s, m, dst, n); break;
    case MOE_DT_Q5_0: hipLaunchKernelGGL(tile_kernel<MOE_DT_Q5_0>, grid, dim3(256), 0, s, m, dst, n); break;
    default: hipLaunchKernelGGL(tile_kernel<MOE_DT_Q8_0>, grid, dim3(256), 0, s, m, dst, n); break;
    }
    return hipGetLastError();
}

int stream_tile_exact(int tokens, bool q8) { return tokens <= 32 ? 32 : stream_tile((double)tokens, q8); }

hipError_t launch_stream(bool up, const MfmaArgs &a0, int bm, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    MfmaArgs a = a0;
    const double per = a.E > 0 ? (double)a.T * a.k / a.E : 0.0;
    const MatDev &m = up ? e0.m[0] : e0.m[2];
    // Tiled copies exist for every routed expert or for none.
    const bool tiled = m.tiled && (!up || e0.m[1].tiled);
    // One-subtile gate/up tiles split the last round's tiles along K (their
    // tokens cannot be halved usefully); other launches along tokens, when
    // the tiles hold enough of them.
    const bool ktail = up && tiled && bm == 32 && a.tail_part && a.tail_cnt && device_cus() / 8 <= 2 * kTailPerXcd;
    a.xcd_cus = ktail ? device_cus() / 8 : split_cus(per < bm ? per : bm, 48.0);
    if (!ktail) a.tail_part = nullptr, a.tail_cnt = nullptr;
    const int cols = up ? SW / 2 : SW;
    const int ks = up ? 1 : a.ksplit;
    const dim3 grid = tile_grid(a.max_tiles, m.rows, cols, ks, a.xcd_cus, up);
    hipError_t err = up ? launch_dt<true>(m.dt, bm, grid, a, 0, ks, tiled, s)
                        : launch_dt<false>(m.dt, bm, grid, a, 0, ks, tiled, s);
    if (err != hipSuccess || !sh) return err;
    // The shared expert takes every token: its own tile for T tokens.
    const bool q8 = m.dt == MOE_DT_Q8_0 || sh->m[0].dt == MOE_DT_Q8_0 || sh->m[2].dt == MOE_DT_Q8_0;
    return launch_stream_single(up, a, stream_tile_exact(a.T, q8), *sh, s);
}

hipError_t launch_stream_single(bool up, const MfmaArgs &a0, int bm, const ExpertDev &ex, hipStream_t s) {
    MfmaArgs a = a0;
    a.tail_part = nullptr, a.tail_cnt = nullptr;  // the shared expert's tiles split along tokens only
    a.xcd_cus = split_cus((double)(a.T < bm ? a.T : bm), 48.0);
    const MatDev &m = up ? ex.m[0] : ex.m[2];
    const int cols = up ? SW / 2 : SW;
    const int ks = up ? 1 : a.ksplit;
    const dim3 gs = tile_grid((a.T + bm - 1) / bm, m.rows, cols, ks, a.xcd_cus, up);
    const bool tiled = m.tiled && (!up || ex.m[1].tiled);
    return up ? launch_dt<true>(m.dt, bm, gs, a, 1, ks, tiled, s) : launch_dt<false>(m.dt, bm, gs, a, 1, ks, tiled, s);
}

}  // namespace moe
