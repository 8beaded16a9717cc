// expert_mfma.hip — grouped SwiGLU expert GEMMs on gfx950 matrix cores.
//
// One block computes a BM-token x 64-row tile of one expert:
//   up   : G = X W_gate^T, U = X W_up^T over K = H, h = silu(G) * U -> f16
//   down : Y = h W_down^T over K = I -> f32
// X rows are gathered through the expert's permuted token list, so no
// permuted copy of the activations is materialised.  Weights stay in their
// checkpoint format in HBM; each K step (128 values = four 32-value blocks
// per row) a block reads its 64 rows' raw blocks once, dequantises them to
// f16 (d * q rounded once, the only weight rounding) into LDS, and four
// waves run V_MFMA_F32_16X16X32_F16 over them with f32 accumulation.
// Tiles come from the dispatch kernel's (expert, m0) list; blocks past the
// list's end exit at once.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "moe_internal.h"

namespace moe {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));

constexpr int BN = 64;         // weight rows per tile
constexpr int BK = 128;        // K values per step
constexpr int LDK = BK + 8;    // LDS row stride in halves (pads banks)

__device__ inline uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t s) { return __builtin_amdgcn_alignbyte(hi, lo, s); }
__device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// Two f16 lanes from a packed pair of 16-bit words.
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

// Unsigned bytes b0..b3 of `v` (each < 256) -> two words of f16 (1024 + b):
// lo word holds (b0, b1), hi word (b2, b3).
__device__ inline void bytes_to_magic(uint32_t v, uint32_t &w01, uint32_t &w23) {
    w01 = perm(0x64646464u, v, 0x04010400u);
    w23 = perm(0x64646464u, v, 0x04030402u);
}

// Dequantise one 32-value block given as 16 bytes of codes in `c` (byte i =
// element pairing of the format) into out[0..16) (16 words = 32 halves).
// `off` is 1024 + the format's zero offset; scale applied in f16.
__device__ inline void codes_to_f16(const uint32_t (&lo)[4], const uint32_t (&hi)[4], __half2 off2, __half2 d2,
                                    uint32_t (&out)[16]) {
    // lo[i]: bytes are elements 4i..4i+3; hi[i]: elements 16+4i..16+4i+3.
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t a, b;
        bytes_to_magic(lo[i], a, b);
        out[2 * i] = h2_bits(__hmul2(__hsub2(as_h2(a), off2), d2));
        out[2 * i + 1] = h2_bits(__hmul2(__hsub2(as_h2(b), off2), d2));
        bytes_to_magic(hi[i], a, b);
        out[8 + 2 * i] = h2_bits(__hmul2(__hsub2(as_h2(a), off2), d2));
        out[8 + 2 * i + 1] = h2_bits(__hmul2(__hsub2(as_h2(b), off2), d2));
    }
}

__device__ inline uint32_t spread4(uint32_t h) { return ((h * 0x00204081u) & 0x01010101u) << 4; }

// One 64-value unit (two blocks) of a row at `p` (4-byte aligned) -> 32
// words of f16 in natural element order.
template <int DT>
__device__ inline void dequant_unit(const uint8_t *p, uint32_t (&out)[32]) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p, 4));
    if constexpr (DT == MOE_DT_F32) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
            __half2 a = __floats2half2_rn(__uint_as_float(v.x), __uint_as_float(v.y));
            __half2 b = __floats2half2_rn(__uint_as_float(v.z), __uint_as_float(v.w));
            out[2 * i] = h2_bits(a);
            out[2 * i + 1] = h2_bits(b);
        }
    } else if constexpr (DT == MOE_DT_Q4_0) {
        uint32_t d[9];
        u32x4 v0 = *reinterpret_cast<const u32x4 *>(q);
        u32x4 v1 = *reinterpret_cast<const u32x4 *>(q + 4);
        d[0] = v0.x, d[1] = v0.y, d[2] = v0.z, d[3] = v0.w, d[4] = v1.x, d[5] = v1.y, d[6] = v1.z, d[7] = v1.w;
        d[8] = q[8];
        const __half2 off2 = __floats2half2_rn(1032.0f, 1032.0f);
        uint32_t lo[4], hi[4], o[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t c = alignb(d[i + 1], d[i], 2);
            lo[i] = c & 0x0f0f0f0fu, hi[i] = (c >> 4) & 0x0f0f0f0fu;
        }
        codes_to_f16(lo, hi, off2, as_h2((d[0] & 0xffffu) * 0x10001u), o);
#pragma unroll
        for (int i = 0; i < 16; i++) out[i] = o[i];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t c = d[5 + i];
            lo[i] = c & 0x0f0f0f0fu, hi[i] = (c >> 4) & 0x0f0f0f0fu;
        }
        codes_to_f16(lo, hi, off2, as_h2((d[4] >> 16) * 0x10001u), o);
#pragma unroll
        for (int i = 0; i < 16; i++) out[16 + i] = o[i];
    } else if constexpr (DT == MOE_DT_Q5_0) {
        uint32_t d[11];
        u32x4 v0 = *reinterpret_cast<const u32x4 *>(q);
        u32x4 v1 = *reinterpret_cast<const u32x4 *>(q + 4);
        d[0] = v0.x, d[1] = v0.y, d[2] = v0.z, d[3] = v0.w, d[4] = v1.x, d[5] = v1.y, d[6] = v1.z, d[7] = v1.w;
        d[8] = q[8], d[9] = q[9], d[10] = q[10];
        const __half2 off2 = __floats2half2_rn(1040.0f, 1040.0f);
        uint32_t lo[4], hi[4], o[16];
        const uint32_t ha = alignb(d[1], d[0], 2), hb = d[6];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t c = alignb(d[i + 2], d[i + 1], 2);
            lo[i] = (c & 0x0f0f0f0fu) | spread4((ha >> (4 * i)) & 0xfu);
            hi[i] = ((c >> 4) & 0x0f0f0f0fu) | spread4((ha >> (16 + 4 * i)) & 0xfu);
        }
        codes_to_f16(lo, hi, off2, as_h2((d[0] & 0xffffu) * 0x10001u), o);
#pragma unroll
        for (int i = 0; i < 16; i++) out[i] = o[i];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t c = d[7 + i];
            lo[i] = (c & 0x0f0f0f0fu) | spread4((hb >> (4 * i)) & 0xfu);
            hi[i] = ((c >> 4) & 0x0f0f0f0fu) | spread4((hb >> (16 + 4 * i)) & 0xfu);
        }
        codes_to_f16(lo, hi, off2, as_h2((d[5] >> 16) * 0x10001u), o);
#pragma unroll
        for (int i = 0; i < 16; i++) out[16 + i] = o[i];
    } else {  // Q8_0
        uint32_t d[17];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
            d[4 * i] = v.x, d[4 * i + 1] = v.y, d[4 * i + 2] = v.z, d[4 * i + 3] = v.w;
        }
        d[16] = q[16];
        const __half2 off2 = __floats2half2_rn(1152.0f, 1152.0f);
        const __half2 da = as_h2((d[0] & 0xffffu) * 0x10001u), db = as_h2((d[8] >> 16) * 0x10001u);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t ca = alignb(d[i + 1], d[i], 2) ^ 0x80808080u;
            const uint32_t cb = d[9 + i] ^ 0x80808080u;
            uint32_t a, b;
            bytes_to_magic(ca, a, b);
            out[2 * i] = h2_bits(__hmul2(__hsub2(as_h2(a), off2), da));
            out[2 * i + 1] = h2_bits(__hmul2(__hsub2(as_h2(b), off2), da));
            bytes_to_magic(cb, a, b);
            out[16 + 2 * i] = h2_bits(__hmul2(__hsub2(as_h2(a), off2), db));
            out[16 + 2 * i + 1] = h2_bits(__hmul2(__hsub2(as_h2(b), off2), db));
        }
    }
}

template <int DT>
constexpr int unit_bytes() {
    return DT == MOE_DT_F32 ? 256 : DT == MOE_DT_Q4_0 ? 36 : DT == MOE_DT_Q5_0 ? 44 : 68;
}

// Tile coordinates for this block.  mode 0: routed tiles from the list;
// mode 1: the shared expert, tile m0 = blockIdx.x * BM over all T tokens.
struct TileInfo {
    int g, m0, n, row0;
    bool shared;
};
template <int BM>
__device__ inline bool tile_of(const MfmaArgs &a, int mode, TileInfo &ti) {
    if (mode == 1) {
        ti.g = a.E, ti.m0 = blockIdx.x * BM, ti.n = a.T, ti.row0 = 0, ti.shared = true;
        return ti.m0 < a.T;
    }
    const int b = blockIdx.x;
    if (b >= a.ntiles[0]) return false;
    const int g = a.tiles[2 * b];
    if (g >= a.E) return false;
    ti.g = g, ti.m0 = a.tiles[2 * b + 1], ti.n = a.counts[g], ti.row0 = a.offsets[g], ti.shared = false;
    return true;
}

template <int DT, int BM, bool UP>
__global__ __launch_bounds__(256) void mfma_kernel(MfmaArgs a, int mode) {
    constexpr int NB = UP ? 2 : 1;   // weight matrices per tile
    constexpr int MT = BM / 16;      // 16-row MFMA tiles along M
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[NB * BN * LDK];
    __shared__ int rows_perm[BM];

    TileInfo ti;
    if (!tile_of<BM>(a, mode, ti)) return;
    const ExpertDev &ex = a.experts[ti.g];
    const MatDev &W0 = UP ? ex.m[0] : ex.m[2];
    const MatDev &W1 = UP ? ex.m[1] : ex.m[2];
    const int n0 = blockIdx.y * BN;
    if (n0 >= W0.rows) return;
    const int K = W0.cols;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    // Permuted row (h / y row) and source row for each of the BM token slots.
    const int Icol = ti.shared ? a.I_s : a.I;
    if (tid < BM) {
        const int i = ti.m0 + tid;
        rows_perm[tid] = i < ti.n ? ti.row0 + i : -1;
    }
    __syncthreads();

    floatx4 acc[NB][MT];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[b][m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // A source pointer for this thread's load slots.
    constexpr int A_CHUNKS = BM * (BK / 8);  // 16-byte chunks per K step
    for (int k0 = 0; k0 < K; k0 += BK) {
        // ---- A: BM rows x 128 halves, 16 B per chunk.
#pragma unroll
        for (int c = tid; c < A_CHUNKS; c += 256) {
            const int r = c / (BK / 8), cc = c % (BK / 8);
            const int pr = rows_perm[r];
            u32x4a v = u32x4a{0u, 0u, 0u, 0u};
            if (pr >= 0) {
                const uint16_t *src;
                if (UP) {
                    const int tok = ti.shared ? pr : a.perm_tok[pr];
                    src = a.xh + (size_t)tok * a.H + k0 + cc * 8;
                } else {
                    src = (ti.shared ? a.hs : a.h) + (size_t)pr * Icol + k0 + cc * 8;
                }
                v = *reinterpret_cast<const u32x4a *>(src);
            }
            *reinterpret_cast<u32x4a *>(&As[r * LDK + cc * 8]) = v;
        }
        // ---- B: NB x 64 rows x 2 units, one unit per thread.
        if (tid < NB * BN * 2) {
            const int b = tid / (BN * 2), rem = tid % (BN * 2);
            const int r = rem >> 1, u = rem & 1;
            const MatDev &W = b == 0 ? W0 : W1;
            uint32_t o[32];
            const int row = n0 + r;
            if (row < W.rows) {
                const uint8_t *p = W.ptr + (size_t)row * W.stride + (size_t)(k0 / 64 + u) * unit_bytes<DT>();
                dequant_unit<DT>(p, o);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) o[i] = 0u;
            }
            u32x4a *dst = reinterpret_cast<u32x4a *>(&Bs[(b * BN + r) * LDK + u * 64]);
#pragma unroll
            for (int i = 0; i < 8; i++) dst[i] = u32x4a{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        }
        __syncthreads();
        // ---- MFMA: wave wv owns weight rows [16 wv, 16 wv + 16) of the tile.
#pragma unroll
        for (int kk = 0; kk < BK / 32; kk++) {
            const int kofs = kk * 32 + 8 * (lane >> 4);
            half8 bf[NB];
#pragma unroll
            for (int b = 0; b < NB; b++)
                bf[b] = *reinterpret_cast<const half8 *>(&Bs[(b * BN + 16 * wv + (lane & 15)) * LDK + kofs]);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const half8 af = *reinterpret_cast<const half8 *>(&As[(16 * m + (lane & 15)) * LDK + kofs]);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    acc[b][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[b][m], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // ---- epilogue: lane holds C[16 m + 4 (lane/16) + v][16 wv + lane%16].
    const int col = n0 + 16 * wv + (lane & 15);
    if (col >= W0.rows) return;
#pragma unroll
    for (int m = 0; m < MT; m++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int r = 16 * m + 4 * (lane >> 4) + v;
            const int pr = rows_perm[r];
            if (pr < 0) continue;
            if (UP) {
                const float g = acc[0][m][v], u = acc[NB - 1][m][v];
                const float hv = (g / (1.0f + __expf(-g))) * u;
                uint16_t *dst = (ti.shared ? a.hs : a.h) + (size_t)pr * Icol + col;
                *dst = __half_as_ushort(__float2half_rn(hv));
            } else {
                float *dst = (ti.shared ? a.ys : a.y) + (size_t)pr * a.H + col;
                *dst = acc[0][m][v];
            }
        }
    }
}

template <bool UP, int BM>
hipError_t launch_bm(int dt, dim3 grid, const MfmaArgs &a, int mode, hipStream_t s) {
    switch (dt) {
    case MOE_DT_F32: hipLaunchKernelGGL((mfma_kernel<MOE_DT_F32, BM, UP>), grid, dim3(256), 0, s, a, mode); break;
    case MOE_DT_Q8_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q8_0, BM, UP>), grid, dim3(256), 0, s, a, mode); break;
    case MOE_DT_Q4_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q4_0, BM, UP>), grid, dim3(256), 0, s, a, mode); break;
    case MOE_DT_Q5_0: hipLaunchKernelGGL((mfma_kernel<MOE_DT_Q5_0, BM, UP>), grid, dim3(256), 0, s, a, mode); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool UP>
hipError_t launch_mode(int bm, int dt, dim3 grid, const MfmaArgs &a, int mode, hipStream_t s) {
    switch (bm) {
    case 16: return launch_bm<UP, 16>(dt, grid, a, mode, s);
    case 32: return launch_bm<UP, 32>(dt, grid, a, mode, s);
    case 64: return launch_bm<UP, 64>(dt, grid, a, mode, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_mfma(bool up, const MfmaArgs &a, int bm, const ExpertDev &e0, const ExpertDev *sh, hipStream_t s) {
    const MatDev &m = up ? e0.m[0] : e0.m[2];
    dim3 grid(a.max_tiles, (m.rows + BN - 1) / BN);
    hipError_t err = up ? launch_mode<true>(bm, m.dt, grid, a, 0, s) : launch_mode<false>(bm, m.dt, grid, a, 0, s);
    if (err != hipSuccess || !sh) return err;
    const MatDev &ms = up ? sh->m[0] : sh->m[2];
    dim3 gs((a.T + bm - 1) / bm, (ms.rows + BN - 1) / BN);
    return up ? launch_mode<true>(bm, ms.dt, gs, a, 1, s) : launch_mode<false>(bm, ms.dt, gs, a, 1, s);
}

}  // namespace moe
