// route.hip — router logits, gating and token->expert dispatch for gfx950.
//
// Everything here is bit-exact to the reference's CPU path, because expert
// selection must be: the logits follow dot_avx2's lane and reduction order
// (src/quant.rs:386-420), the gates use a port of glibc's expf, and every
// sum the reference folds sequentially is folded sequentially here too.
// This file is compiled with -ffp-contract=off so that no multiply and add
// are fused except where fmaf() says so.
#include <hip/hip_fp16.h>
#include <cmath>
#include <algorithm>
#include <hip/hip_runtime.h>

#include "exact_math.h"
#include "moe_internal.h"

namespace moe {
namespace {

constexpr int kSmallRouterTokens = 4;

// Rust f32::total_cmp as a signed integer key.
__device__ inline int32_t tkey(float v) {
    int32_t b = __float_as_int(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// Rust f32::max: NaN loses to a number.
__device__ inline float fmax_rs(float a, float b) { return (a != a) ? b : ((b != b) ? a : (a > b ? a : b)); }

// Reduce the 16 per-lane chains of one dot product in dot_avx2's order:
// s[j] = acc0[j] + acc1[j]; q[j] = s[j+4] + s[j]; (q0+q1) + (q2+q3).
// `acc` is lane j's chain (j = lane & 15); the result is valid in j == 0.
__device__ inline float reduce16_avx2(float acc) {
    float s = acc + __shfl_down(acc, 8, 16);
    float q = __shfl_down(s, 4, 16) + s;
    float a = q + __shfl_down(q, 1, 16);   // lane 0: q0+q1, lane 2: q2+q3
    return a + __shfl_down(a, 2, 16);      // lane 0: (q0+q1)+(q2+q3)
}

// Scalar tail of dot_avx2 (elements past the last full 8): out += a*b.
__device__ inline float dot_tail(float out, const float *a, const float *b, int from, int n) {
    for (int i = from; i < n; i++) {
        float p = a[i] * b[i];
        out += p;
    }
    return out;
}

// Copy n floats from global memory to LDS with every thread of the block,
// eight 16-byte loads in flight per thread before any store.  Loads and
// stores are unconditional (indices past the end re-read and re-write the
// last vector with its own value), so the compiler cannot sink a load into a
// branch and serialise the copy.
__device__ inline void stage_to_lds(const float *__restrict__ src, float *__restrict__ dst, int n) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if ((n & 3) == 0 && (((uintptr_t)src) & 15) == 0) {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        float4 *d4 = reinterpret_cast<float4 *>(dst);
        const int n4 = n >> 2;
        if (n4 == 0) return;
        for (int base = 0; base < n4; base += 8 * nt) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = base + u * nt + tid;
                v[u] = s4[i < n4 ? i : n4 - 1];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = base + u * nt + tid;
                d4[i < n4 ? i : n4 - 1] = v[u];
            }
        }
    } else {
        for (int i = tid; i < n; i += nt) dst[i] = src[i];
    }
}

// Copy na floats from a and nb floats from b (16-byte aligned, positive
// multiples of 4) from global memory to LDS, issuing all of a thread's loads
// (up to U float4 from each source) before its first store: one memory
// round trip per U * blockDim.x float4 of each source.  The sources are rows
// of len4 float4; in LDS consecutive rows start stride4 float4 apart.
// Indices past the end re-read and re-write the last vector, so no access is
// conditional.
template <int U>
__device__ inline void stage2_to_lds(const float *__restrict__ a, float *__restrict__ da, int na,
                                     const float *__restrict__ b, float *__restrict__ db, int nb, int len4,
                                     int stride4) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    const int na4 = na >> 2, nb4 = nb >> 2;
    const int n4 = na4 > nb4 ? na4 : nb4;
    auto dst = [&](int i) { return (i / len4) * stride4 + i % len4; };
    for (int base = 0; base < n4; base += U * nt) {
        float4 va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * nt + tid;
            va[u] = a4[i < na4 ? i : na4 - 1];
            vb[u] = b4[i < nb4 ? i : nb4 - 1];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * nt + tid;
            reinterpret_cast<float4 *>(da)[dst(i < na4 ? i : na4 - 1)] = va[u];
            reinterpret_cast<float4 *>(db)[dst(i < nb4 ? i : nb4 - 1)] = vb[u];
        }
    }
}

__host__ __device__ inline int router_lds_stride(int H) { return (H % 64 == 0) ? H + 16 : H; }

// Latency-bound router: a block stages RB router rows and TB token rows in
// LDS (the whole of H), then thread (g, j) runs lane j of dot_avx2 for the
// (row, token) pairs g, g + 16, ..., PPT of them (RB TB <= 16 PPT), their
// chains interleaved and read eight steps at a time.  Each chain keeps its
// order, so PPT changes no bit; it puts more pairs on each staged row.
template <int PPT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void router_lds_kernel(const float *__restrict__ W, const float *__restrict__ x,
                                                         int T, int n_rows, int E, int H, int RB, int TB, float temp,
                                                         float *__restrict__ logits) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int r0 = blockIdx.x * RB, t0 = blockIdx.y * TB;
    const int nr = min(RB, n_rows - r0), nt = min(TB, T - t0);
    // Rows sit LS floats apart: when H % 64 == 0 the extra 16 floats put
    // the four rows a wavefront reads at once in different bank groups.
    const int LS = router_lds_stride(H);
    float *wl = lds;
    float *xl = lds + (size_t)RB * LS;
    const bool vec = (H & 3) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0;
    if (vec) {
        stage2_to_lds<16>(W + (size_t)r0 * H, wl, nr * H, x + (size_t)t0 * H, xl, nt * H, H >> 2, LS >> 2);
    } else {
        for (int r = 0; r < nr; r++) stage_to_lds(W + (size_t)(r0 + r) * H, wl + (size_t)r * LS, H);
        for (int r = 0; r < nt; r++) stage_to_lds(x + (size_t)(t0 + r) * H, xl + (size_t)r * LS, H);
    }
    __syncthreads();
    const int tid = threadIdx.x, j = tid & 15, g = tid >> 4;
    const int np = nr * nt;
    if (g >= np) return;  // whole 16-lane groups leave together
    // Pairs past np repeat the group's first pair (never stored).
    const float *a[PPT], *b[PPT];
#pragma unroll
    for (int q = 0; q < PPT; q++) {
        const int p = g + 16 * q < np ? g + 16 * q : g;
        a[q] = wl + (size_t)(p / nt) * LS;
        b[q] = xl + (size_t)(p % nt) * LS;
    }
    const int n16 = H / 16;
    const bool has8 = (H % 16) >= 8;
    float acc[PPT];
#pragma unroll
    for (int q = 0; q < PPT; q++) acc[q] = 0.0f;
    int c = 0;
    for (; c + 8 <= n16; c += 8) {
        float av[PPT][8], bv[PPT][8];
#pragma unroll
        for (int q = 0; q < PPT; q++)
#pragma unroll
            for (int u = 0; u < 8; u++) {
                av[q][u] = a[q][16 * (c + u) + j];
                bv[q][u] = b[q][16 * (c + u) + j];
            }
#pragma unroll
        for (int u = 0; u < 8; u++)
#pragma unroll
            for (int q = 0; q < PPT; q++) acc[q] = fmaf(av[q][u], bv[q][u], acc[q]);
    }
    for (; c < n16; c++)
#pragma unroll
        for (int q = 0; q < PPT; q++) acc[q] = fmaf(a[q][16 * c + j], b[q][16 * c + j], acc[q]);
#pragma unroll
    for (int q = 0; q < PPT; q++) {
        if (has8 && j < 8) acc[q] = fmaf(a[q][16 * n16 + j], b[q][16 * n16 + j], acc[q]);
        float v = reduce16_avx2(acc[q]);
        const int p = g + 16 * q;
        if (j == 0 && p < np) {
            v = dot_tail(v, a[q], b[q], 16 * n16 + (has8 ? 8 : 0), H);
            const int r = r0 + p / nt;
            if (temp > 0.0f && r < E) v = v / temp;
            logits[(size_t)(t0 + p % nt) * n_rows + r] = v;
        }
    }
}

// Tiled router for larger T: a 32-row x 32-token tile per block, K staged
// through LDS 64 values at a time.  Thread (j, g) owns lane j of the chains
// of 8 rows x 8 tokens.  Chunks past the last full 16 are zero-padded, and
// fma(0, 0, acc) == acc for every acc a chain can hold (chains start at +0
// and never reach -0), so padding does not change a single bit.
constexpr int kRT = 32;   // rows per tile
constexpr int kKC = 64;   // K chunk
template <int TPT, bool VEC>
__global__ __launch_bounds__(256) void router_tiled_kernel(const float *__restrict__ W, const float *__restrict__ x,
                                                           int T, int n_rows, int E, int H, float temp,
                                                           float *__restrict__ logits) {
    // A chunk row holds its 64 values transposed, value 16 s + j at 4 j + s,
    // so that chain lane j reads its four values of the chunk (s = 0..3) with
    // one 16-byte read; eight lanes then read 128 contiguous bytes.
    constexpr int kLS = kKC;
    __shared__ __attribute__((aligned(16))) float wt[kRT][kLS];
    constexpr int kTTv = 4 * TPT;  // tokens per tile: TPT per thread
    __shared__ __attribute__((aligned(16))) float xt[kTTv][kLS];
    const int tid = threadIdx.x, j = tid & 15, g = tid >> 4;
    const int rg = g & 3, tg = g >> 2;
    const int r0 = blockIdx.x * kRT, t0 = blockIdx.y * kTTv;
    const int n16 = H / 16;
    const int kfull = n16 * 16;  // elements covered by full 16-chunks
    float acc[8][TPT];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int u = 0; u < TPT; u++) acc[i][u] = 0.0f;
    // Each thread moves 2 float4 of W (32 rows x 16 float4) and up to 2 of x
    // (kTTv tokens) per chunk, through two register buffers: the loads of
    // chunk c + 2 are issued before chunk c's FMAs.  VEC (H % 4 == 0): every
    // thread issues the same loads in every chunk, from addresses clamped
    // into the matrices, so that the compiler counts the loads in flight
    // exactly (a load under a condition, or a select of its value, makes it
    // wait for all of them, and a chunk then waited for the next chunk's
    // loads: one chunk in flight instead of two).  Rows past the router's
    // and tokens past T then hold copies of valid ones, which only feed
    // their own chains, never stored; the values past kfull are zeroed
    // where the last, partial chunk is stored to LDS.  Threads without a
    // token row of their own load one of the tile's (lines another thread
    // loads too), and the loads past the last chunk fill a buffer that is
    // never read.  VEC needs H >= 16 (addresses clamped into the last full
    // 16-value chunk).
    auto load_chunk = [&](int k0, float4(&pw)[2], float4(&px)[2]) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int q = tid + 256 * u, rr = q >> 4, kk = (q & 15) * 4;
            const int gk = k0 + kk, gr = r0 + rr, gt = t0 + rr;
            float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f), x4 = w4;
            if constexpr (VEC) {
                const int ck = min(gk, kfull - 4);
                const int xt_row = min(t0 + min(rr, kTTv - 1), T - 1);
                w4 = *reinterpret_cast<const float4 *>(W + (size_t)min(gr, n_rows - 1) * H + ck);
                x4 = *reinterpret_cast<const float4 *>(x + (size_t)xt_row * H + ck);
            } else {
                float *wp = &w4.x, *xp = &x4.x;
                for (int e = 0; e < 4; e++) {
                    if (gr < n_rows && gk + e < kfull) wp[e] = W[(size_t)gr * H + gk + e];
                    if (rr < kTTv && gt < T && gk + e < kfull) xp[e] = x[(size_t)gt * H + gk + e];
                }
            }
            pw[u] = w4, px[u] = x4;
        }
    };
    float4 pwa[2], pxa[2], pwb[2], pxb[2];
    const int nch = (kfull + kKC - 1) / kKC;  // chunks, the last possibly partial
    if (VEC || nch > 0) load_chunk(0, pwa, pxa);
    if (VEC || nch > 1) load_chunk(kKC, pwb, pxb);
    // Chunk k0 from register buffer (pw, px), which then takes chunk
    // k0 + 2 kKC.
    auto chunk = [&](int k0, float4(&pw)[2], float4(&px)[2]) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int q = tid + 256 * u, rr = q >> 4, kk = (q & 15) * 4;
            // Values kk..kk+3 are (s, j) = (kk / 16, kk % 16 + e).
            const int s0 = kk >> 4, j0 = kk & 15;
            if (VEC && k0 + kKC > kfull && k0 + kk >= kfull)
                pw[u] = px[u] = make_float4(0.f, 0.f, 0.f, 0.f);  // past the last full 16-value chunk
            float *wr = &wt[rr][0];
            wr[4 * (j0 + 0) + s0] = pw[u].x, wr[4 * (j0 + 1) + s0] = pw[u].y;
            wr[4 * (j0 + 2) + s0] = pw[u].z, wr[4 * (j0 + 3) + s0] = pw[u].w;
            if (rr < kTTv) {
                float *xr = &xt[rr][0];
                xr[4 * (j0 + 0) + s0] = px[u].x, xr[4 * (j0 + 1) + s0] = px[u].y;
                xr[4 * (j0 + 2) + s0] = px[u].z, xr[4 * (j0 + 3) + s0] = px[u].w;
            }
        }
        __syncthreads();
        if (VEC || k0 + 2 * kKC < kfull) load_chunk(k0 + 2 * kKC, pw, px);
        static_assert(kKC == 64, "four 16-value steps per chunk");
        float4 wq[8], xq[TPT];
#pragma unroll
        for (int i = 0; i < 8; i++) wq[i] = *reinterpret_cast<const float4 *>(&wt[rg * 8 + i][4 * j]);
#pragma unroll
        for (int u = 0; u < TPT; u++) xq[u] = *reinterpret_cast<const float4 *>(&xt[tg * TPT + u][4 * j]);
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float wv = s == 0 ? wq[i].x : s == 1 ? wq[i].y : s == 2 ? wq[i].z : wq[i].w;
#pragma unroll
                for (int u = 0; u < TPT; u++) {
                    const float xv = s == 0 ? xq[u].x : s == 1 ? xq[u].y : s == 2 ? xq[u].z : xq[u].w;
                    acc[i][u] = fmaf(wv, xv, acc[i][u]);
                }
            }
        }
        __syncthreads();
    };
    int c = 0;
    for (; c + 2 <= nch; c += 2) {
        chunk(c * kKC, pwa, pxa);
        chunk((c + 1) * kKC, pwb, pxb);
    }
    if (c < nch) chunk(c * kKC, pwa, pxa);
    const bool has8 = (H % 16) >= 8;
    const int tail = kfull + (has8 ? 8 : 0);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = r0 + rg * 8 + i;
#pragma unroll
        for (int u = 0; u < TPT; u++) {
            const int t = t0 + tg * TPT + u;
            float a = acc[i][u];
            const bool valid = r < n_rows && t < T;
            if (has8 && j < 8 && valid) a = fmaf(W[(size_t)r * H + kfull + j], x[(size_t)t * H + kfull + j], a);
            float v = reduce16_avx2(a);
            if (j == 0 && valid) {
                v = dot_tail(v, W + (size_t)r * H, x + (size_t)t * H, tail, H);
                if (temp > 0.0f && r < E) v = v / temp;
                logits[(size_t)t * n_rows + r] = v;
            }
        }
    }
}

// ------------------------------------------------------------------ gating

__device__ inline float wave_max_rs(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmax_rs(v, __shfl_xor(v, m, 64));
    return v;
}
// Wave-wide max of an int32, every lane receiving it: DPP steps within rows
// of 16 lanes, row broadcasts to lane 63, then a read of lane 63.
__device__ inline int32_t dpp_max_step(int32_t v, int ctrl) {
    int o;
    switch (ctrl) {
    case 0: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0xb1, 0xf, 0xf, false); break;   // quad [1,0,3,2]
    case 1: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x4e, 0xf, 0xf, false); break;   // quad [2,3,0,1]
    case 2: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x141, 0xf, 0xf, false); break;  // half-row mirror
    case 3: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x140, 0xf, 0xf, false); break;  // row mirror
    case 4: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x142, 0xa, 0xf, false); break;  // row bcast 15
    default: o = __builtin_amdgcn_update_dpp(INT32_MIN, v, 0x143, 0xc, 0xf, false); break; // row bcast 31
    }
    return o > v ? o : v;
}
__device__ inline int32_t wave_max_i32(int32_t v) {
#pragma unroll
    for (int c = 0; c < 6; c++) v = dpp_max_step(v, c);
    return __builtin_amdgcn_readlane(v, 63);
}

// LDS scratch of one gating wavefront.
template <int EPL>
struct GateScratch {
    float sc[EPL * 64];
    float rank[EPL * 64];
    float gs[64];
    int idx[kMaxTopK];
    float w[kMaxTopK];          // the selected experts' weights
    int32_t key[64];            // rank keys (EPL == 1)
    int32_t bypos[kMaxTopK + 1];  // key at each sorted position <= k (EPL == 1)
    float bcast;
    float shg;                  // the shared expert's sigmoid gate (has_shared_gate)
};

// Orders this wavefront's LDS writes before its later LDS reads (the
// gating scratch is private to one wavefront, so no block barrier is needed).
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// The inputs of gate_token that are fixed for the layer, fetched by the
// wavefront ahead of the logits: expf_exact's table (one entry per lane,
// expf_exact_w) and the score-correction biases of the lane's experts.
template <int EPL>
struct GateConst {
    uint64_t tab;
    float bias[EPL];
};

template <int EPL>
__device__ inline GateConst<EPL> gate_const(const GateParams &p) {
    GateConst<EPL> G;
    const int lane = threadIdx.x & 63;
    G.tab = exp2_lane_entry();
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane * EPL + i;
        G.bias[i] = (p.e_bias && e < p.n_experts) ? p.e_bias[e] : 0.0f;
    }
    return G;
}

// Gating for token t by one wavefront, experts e = lane*EPL + i.  Restates
// src/model.rs:855-897: gate, rank = score + bias, prune_groups, disabled,
// stable descending sort truncated to k (ties: lower index first), forced
// experts, weights = max(score, 0), renormalise, scale.  `lg` is the token's
// logits row (temperature already applied; entry E is the shared-expert gate
// logit when the layer has one).  Every lane of the wavefront calls it
// together.  STORE = false leaves the selection (S.idx, S.w) and the shared
// gate (S.shg) in LDS only.
template <int EPL, bool STORE = true>
__device__ void gate_token(const float *__restrict__ lg, int t, const GateParams &p, const GateConst<EPL> &G,
                           GateScratch<EPL> &S, int32_t *__restrict__ sel, float *__restrict__ wsel,
                           float *__restrict__ shgate, unsigned long long *__restrict__ stats) {
    const int lane = threadIdx.x & 63;
    const int E = p.n_experts;
    float sc[EPL], rank[EPL], bias[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {  // the logits and the shared gate's logit requested together
        const int e = lane * EPL + i;
        sc[i] = e < E ? lg[e] : 0.0f;
        bias[i] = G.bias[i];
    }
    const float lg_shared = (p.has_shared_gate && lane == 0) ? lg[E] : 0.0f;
    if (p.sigmoid) {
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            float nv = -sc[i];
            float den = 1.0f + expf_exact_w(nv, G.tab);
            sc[i] = 1.0f / den;
        }
    } else {
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (lane * EPL + i < E) m = fmax_rs(m, sc[i]);
        m = wave_max_rs(m);
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            sc[i] = expf_exact_w(sc[i] - m, G.tab);
            if (lane * EPL + i < E) S.sc[lane * EPL + i] = sc[i];
        }
        wave_sync();
        if (lane == 0) {
            // Sequential sum (e ascending); reads issued 16 at a time.
            float s = 0.0f;
            int e = 0;
            for (; e + 16 <= E; e += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = S.sc[e + u];
#pragma unroll
                for (int u = 0; u < 16; u++) s += v[u];
            }
            for (; e < E; e++) s += S.sc[e];
            S.bcast = s;
        }
        wave_sync();
        const float s = S.bcast;
#pragma unroll
        for (int i = 0; i < EPL; i++) sc[i] = sc[i] / s;
    }
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane * EPL + i;
        rank[i] = (p.e_bias && e < E) ? sc[i] + bias[i] : sc[i];
    }
    const int per_g = p.n_group > 0 ? E / p.n_group : 0, lpg = per_g / EPL;
    if (p.n_group > 1 && p.topk_group < p.n_group && per_g * p.n_group == E && per_g % EPL == 0 &&
        (lpg & (lpg - 1)) == 0 && lpg <= 64) {
        // Groups of lpg whole lanes: each lane takes the top two keys of its
        // EPL experts, the group's lanes merge theirs by shuffles (the two
        // largest keys, hence values, do not depend on the merge order), and
        // the group sum is formed as below: -0.0 + first + second.
        // Same insertion as the sequential form below: keys equal to
        // INT32_MIN never enter and leave their slot's value at 0.
        int32_t k1 = INT32_MIN, k2 = INT32_MIN;
        auto put = [&](int32_t k) {
            if (k > k1) {
                k2 = k1;
                k1 = k;
            } else if (k > k2) {
                k2 = k;
            }
        };
#pragma unroll
        for (int i = 0; i < EPL; i++) put(tkey(rank[i]));
        for (int m = 1; m < lpg; m <<= 1) {
            const int32_t o1 = __shfl_xor(k1, m, 64), o2 = __shfl_xor(k2, m, 64);
            put(o1);
            put(o2);
        }
        auto val = [](int32_t k) {
            return k == INT32_MIN ? 0.0f : __int_as_float(k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1));
        };
        float gsum = -0.0f;
        if (per_g >= 1) gsum = gsum + val(k1);
        if (per_g >= 2) gsum = gsum + val(k2);
        const int g = lane / lpg;
        if (lane % lpg == 0) S.gs[g] = gsum;
        wave_sync();
        const int32_t kg = tkey(gsum);
        int position = 0;
        int g2 = 0;
        for (; g2 + 8 <= p.n_group; g2 += 8) {  // reads issued 8 at a time
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = S.gs[g2 + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int32_t kk = tkey(v[u]);
                position += (kk > kg) || (kk == kg && g2 + u < g);
            }
        }
        for (; g2 < p.n_group; g2++) {
            const int32_t kk = tkey(S.gs[g2]);
            position += (kk > kg) || (kk == kg && g2 < g);
        }
        if (position >= p.topk_group)
#pragma unroll
            for (int i = 0; i < EPL; i++) rank[i] = -INFINITY;
    } else if (p.n_group > 1 && p.topk_group < p.n_group) {
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (lane * EPL + i < E) S.rank[lane * EPL + i] = rank[i];
        wave_sync();
        const int per = E / p.n_group;
        if (lane < p.n_group) {
            int32_t k1 = INT32_MIN, k2 = INT32_MIN;
            float v1 = 0.0f, v2 = 0.0f;
            auto take = [&](float v) {
                const int32_t k = tkey(v);
                if (k > k1) {
                    k2 = k1, v2 = v1;
                    k1 = k, v1 = v;
                } else if (k > k2) {
                    k2 = k, v2 = v;
                }
            };
            int i = 0;
            for (; i + 8 <= per; i += 8) {  // reads issued 8 at a time, taken in order
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = S.rank[lane * per + i + u];
#pragma unroll
                for (int u = 0; u < 8; u++) take(v[u]);
            }
            for (; i < per; i++) take(S.rank[lane * per + i]);
            float gsum = -0.0f;
            if (per >= 1) gsum = gsum + v1;
            if (per >= 2) gsum = gsum + v2;
            S.gs[lane] = gsum;
        }
        wave_sync();
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane * EPL + i;
            const int g = per > 0 ? e / per : p.n_group;
            if (e < E && g < p.n_group) {
                const int32_t kg = tkey(S.gs[g]);
                int position = 0;
                for (int g2 = 0; g2 < p.n_group; g2++) {
                    const int32_t k2 = tkey(S.gs[g2]);
                    position += (k2 > kg) || (k2 == kg && g2 < g);
                }
                if (position >= p.topk_group) rank[i] = -INFINITY;
            }
        }
    }
    if (p.any_disabled) {
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane * EPL + i;
            if (e < E && ((p.disabled[e >> 5] >> (e & 31)) & 1u)) rank[i] = -INFINITY;
        }
    }
    wave_sync();
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane * EPL + i;
        if (e < E) {
            S.sc[e] = sc[i];
            S.rank[e] = rank[i];
        }
    }
    // Selection in the stable descending order (key desc, index asc); the
    // tie check compares neighbours among the first min(k + 1, E).
    const int k = p.top_k;
    int tie = 0;
    if constexpr (EPL == 1) {
        // One expert per lane: its sorted position is the number of experts
        // ahead of it.
        const int32_t my = tkey(rank[0]);
        if (lane < E) S.key[lane] = my;
        wave_sync();
        int pos = 0;
        if (lane < E) {
            int e2 = 0;
            for (; e2 + 8 <= E; e2 += 8) {
                int32_t kv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) kv[u] = S.key[e2 + u];
#pragma unroll
                for (int u = 0; u < 8; u++) pos += (kv[u] > my) || (kv[u] == my && e2 + u < lane);
            }
            for (; e2 < E; e2++) {
                const int32_t k2 = S.key[e2];
                pos += (k2 > my) || (k2 == my && e2 < lane);
            }
        }
        if (lane < E && pos < k) S.idx[pos] = lane;
        if (lane < E && pos <= k) S.bypos[pos] = my;
        wave_sync();
        const int last = k < E ? k : E - 1;
        if (lane >= 1 && lane <= last && S.bypos[lane] == S.bypos[lane - 1]) tie = 1;
        tie = __any(tie) ? 1 : 0;
    } else {
        // k + 1 rounds of argmax; the extra round finds the best unselected
        // rank for the tie check.  A round takes the wave's largest key, then
        // the lowest expert holding it: experts ascend with the lane and,
        // within a lane, with i, so that is the lowest lane whose best
        // (lowest i among its largest keys) has the key.
        int32_t ckey[EPL];
        bool cfree[EPL];
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            ckey[i] = tkey(rank[i]);
            cfree[i] = lane * EPL + i < E;
        }
        int32_t prev_key = 0;
        const int rounds = k < E ? k + 1 : k;
        for (int r = 0; r < rounds; r++) {
            int bi = -1;
            int32_t bk = INT32_MIN;
#pragma unroll
            for (int i = 0; i < EPL; i++)
                if (cfree[i] && (bi < 0 || ckey[i] > bk)) bk = ckey[i], bi = i;
            const int32_t key = wave_max_i32(bi >= 0 ? bk : INT32_MIN);
            const unsigned long long at = __ballot(bi >= 0 && bk == key);
            const int wl = __builtin_ctzll(at);
            const int e = wl * EPL + __builtin_amdgcn_readlane(bi, wl);
            if (r > 0 && key == prev_key) tie = 1;
            prev_key = key;
            if (r < k) {
                if (lane == 0) S.idx[r] = e;
#pragma unroll
                for (int i = 0; i < EPL; i++)
                    if (lane * EPL + i == e) cfree[i] = false;
            }
        }
    }
    wave_sync();
    if (lane == 0) {
        int *idx = S.idx;
        const float *rk = S.rank;
        for (int f = 0; f < p.n_forced; f++) {
            const int e = p.forced[f];
            if (e < 0 || e >= E) continue;
            bool present = false;
            for (int j = 0; j < k; j++) present |= idx[j] == e;
            if (present) continue;
            idx[k - 1] = e;
            // Stable insertion sort of the k picks by descending rank.
            for (int a = 1; a < k; a++) {
                const int v = idx[a];
                const int32_t kv = tkey(rk[v]);
                int b = a;
                while (b > 0 && kv > tkey(rk[idx[b - 1]])) {
                    idx[b] = idx[b - 1];
                    b--;
                }
                idx[b] = v;
            }
        }
    }
    wave_sync();
    // Weights: lane j < k holds pick j's max(score, 0); the normaliser sums
    // them in pick order from -0.0 (read lane by lane), then each lane
    // finishes its own weight.
    int ij = 0;
    float vj = 0.0f;
    if (lane < k) {
        ij = S.idx[lane];
        vj = fmax_rs(S.sc[ij], 0.0f);
    }
    float z = -0.0f;
    for (int j = 0; j < k; j++) z += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vj), j));
    if (p.norm_topk) z = fmax_rs(z, 1e-20f);
    if (lane < k) {
        float wv = vj;
        if (p.norm_topk) wv = wv / z;
        wv = wv * p.routed_scale;
        if (STORE) {
            sel[(size_t)t * k + lane] = ij;
            wsel[(size_t)t * k + lane] = wv;
        }
        S.w[lane] = wv;
    }
    const float sh_exp = expf_exact_w(-lg_shared, G.tab);  // every lane; lane 0's is the gate's
    if (lane == 0) {
        if (p.has_shared_gate) {
            float den = 1.0f + sh_exp;
            const float g = 1.0f / den;
            S.shg = g;
            if (STORE) shgate[t] = g;
        }
        if (tie && stats) atomicAdd(stats + 3, 1ull);
    }
}

// One wavefront per token.
template <int EPL>
__global__ __launch_bounds__(256) void gating_kernel(const float *__restrict__ logits, int ld, int T, GateParams p,
                                                     int32_t *__restrict__ sel, float *__restrict__ wsel,
                                                     float *__restrict__ shgate,
                                                     unsigned long long *__restrict__ stats) {
    __shared__ GateScratch<EPL> S[4];
    const int w = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + w;
    if (t >= T) return;
    const GateConst<EPL> G = gate_const<EPL>(p);
    gate_token<EPL>(logits + (size_t)t * ld, t, p, G, S[w], sel, wsel, shgate, stats);
}

// ---------------------------------------------------------------- dispatch

constexpr int kDispatchThreads = 512;
constexpr int kDispatchWaves = kDispatchThreads / 64;
// Tokens per chunk of the many-token dispatch (count and place kernels run
// one block of this many threads per chunk): 128 up to kSmallChunkMaxT
// tokens, kDispatchThreads beyond (the scan walks every chunk per expert).
// Measured on MI355X, dispatch at 128-token chunks against 512: Qwen3
// T=4096 27.1 -> 22.2 us, DeepSeek-V3 T=4096 27.9 -> 24.0; V2-Lite T=8192
// 25.1 -> 26.6, so 512 beyond 4096 tokens.
constexpr int kChunkTokens = 128;
constexpr int kSmallChunkMaxT = 4096;

// Exclusive scan of one int per thread across the block; returns the
// exclusive prefix and writes the block total to *total.
__device__ inline int block_scan_excl(int v, int *wave_sums, int *total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wave_sums[wv] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int i = 0; i < kDispatchWaves; i++) {
        before += i < wv ? wave_sums[i] : 0;
        all += wave_sums[i];
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

// One block: histogram, scan, stats, hit list, tile list and the stable
// per-expert token order (src/model.rs:902-924).  Positions come from
// per-wave 64-bit ballots, so tokens keep ascending order within an expert
// without relying on atomic ordering.
// Offsets, hit list, counters, one-token task table and MFMA tile list from
// the per-expert counts (one expert per thread, E <= kMaxExperts); returns
// this thread's expert's first permuted row.  Every thread of the block
// calls it.
__device__ int dispatch_tables(const DispatchArgs &a, int c, int *wave_sums, unsigned long long *s_reused,
                               unsigned long long *s_bytes) {
    const int tid = threadIdx.x;
    const int E = a.E, T = a.T, k = a.k;
    const int e = tid;
    int total;
    const int o = block_scan_excl(c, wave_sums, &total);
    if (e < E) {
        a.counts[e] = c;
        a.offsets[e] = o;
    }
    if (tid == 0) {
        a.offsets[E] = total;
        a.offsets[E + 1] = total + (a.has_shared ? T : 0);
        a.counts[E] = a.has_shared ? T : 0;
    }
    // The previous call's hit list as a bit set, loaded in parallel.
    __shared__ unsigned long long prev_bits[kMaxExperts / 64];
    if (a.prev) {
        for (int x = tid; x < kMaxExperts / 64; x += kDispatchThreads) prev_bits[x] = 0ull;
        __syncthreads();
        const uint32_t np = a.prev[0];
        for (uint32_t j = tid; j < np; j += kDispatchThreads) {
            const uint32_t v = a.prev[1 + j];
            if (v < (uint32_t)E) atomicOr(&prev_bits[v >> 6], 1ull << (v & 63));
        }
    }
    int nh;
    const int hp = block_scan_excl(c > 0 ? 1 : 0, wave_sums, &nh);  // its barrier publishes prev_bits
    if (c > 0) {
        a.hits[1 + hp] = e;
        if (a.hits_out) a.hits_out[1 + hp] = (uint32_t)e;
        atomicAdd(s_bytes, a.expert_bytes[e]);
        if (a.prev && ((prev_bits[e >> 6] >> (e & 63)) & 1ull)) atomicAdd(s_reused, (unsigned long long)c);
    }
    if (tid == 0) {
        a.hits[0] = nh;
        if (a.hits_out) a.hits_out[0] = (uint32_t)nh;
    }
    if (a.dtasks) {
        // One token: selected expert number hp in ascending order is task hp,
        // with its permuted row o and the weight of the slot that chose it.
        if (c > 0 && hp < a.dk_bound) {
            DecodeTask d{};
            const ExpertDev &x = a.experts[e];
            d.g = x.m[0].ptr, d.u = x.m[1].ptr, d.d = x.m[2].ptr;
            d.gs = x.m[0].stride, d.us = x.m[1].stride, d.ds = x.m[2].stride;
            d.dcols = x.m[2].cols;
            d.h = a.h + (size_t)o * a.I;
            for (int s = 0; s < k; s++)
                if (a.sel[s] == e) d.w = a.wsel[s];
            d.live = 1;
            a.dtasks[hp] = d;
        }
        for (int t = nh + tid; t < a.dk_bound; t += kDispatchThreads) a.dtasks[t] = DecodeTask{};
        if (tid == 0 && a.has_shared) {
            DecodeTask d{};
            const ExpertDev &x = a.experts[E];
            d.g = x.m[0].ptr, d.u = x.m[1].ptr, d.d = x.m[2].ptr;
            d.gs = x.m[0].stride, d.us = x.m[1].stride, d.ds = x.m[2].stride;
            d.dcols = x.m[2].cols;
            d.h = a.hs;
            d.w = a.shgate ? a.shgate[0] : 1.0f;
            d.live = 1;
            a.dtasks[a.dk_bound] = d;
        }
    }
    if (a.bm > 0) {
        const int nt = (c + a.bm - 1) / a.bm;
        int tt;
        const int tb = block_scan_excl(nt, wave_sums, &tt);
        for (int i = 0; i < nt; i++) {
            a.tiles[4 * (tb + i)] = e;
            a.tiles[4 * (tb + i) + 1] = i * a.bm;
            a.tiles[4 * (tb + i) + 2] = tb;
            a.tiles[4 * (tb + i) + 3] = nt;
        }
        if (tid == 0) {
            int ntot = tt;
            if (a.has_shared) {
                const int ns = (T + a.bm - 1) / a.bm;
                for (int i = 0; i < ns; i++) {
                    a.tiles[4 * (tt + i)] = E;
                    a.tiles[4 * (tt + i) + 1] = i * a.bm;
                    a.tiles[4 * (tt + i) + 2] = tt;
                    a.tiles[4 * (tt + i) + 3] = ns;
                }
                ntot += ns;
            }
            a.ntiles[0] = ntot;
        }
    }
    return o;
}

// Stable permuted rows of tokens t0 .. t0 + NT - 1 (one per thread of an
// NT-thread block): within an expert, lower token first.  run[e] enters as
// the expert's next free row and leaves advanced past these tokens.  bm and
// wb are LDS scratch of NT / 64 rows.
template <int NT>
__device__ void dispatch_place(const DispatchArgs &a, int t0, int *run, unsigned long long (*bm)[kMaxExperts],
                               int (*wb)[kMaxExperts]) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = a.E, T = a.T, k = a.k;
    const int t = t0 + tid;
    for (int x = lane; x < E; x += 64) bm[wv][x] = 0ull;
    __syncthreads();
    if (t < T)
        for (int s = 0; s < k; s++) atomicOr(&bm[wv][a.sel[(size_t)t * k + s]], 1ull << lane);
    __syncthreads();
    for (int x = tid; x < E; x += NT) {
        int r = run[x];
        for (int w2 = 0; w2 < NW; w2++) {
            wb[w2][x] = r;
            r += __popcll(bm[w2][x]);
        }
        run[x] = r;
    }
    __syncthreads();
    if (t < T) {
        const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        for (int s = 0; s < k; s++) {
            const int ex = a.sel[(size_t)t * k + s];
            const float wt = a.wsel[(size_t)t * k + s];
            const int pp = wb[wv][ex] + __popcll(bm[wv][ex] & below);
            a.perm_tok[pp] = t;
            a.perm_w[pp] = wt;
            a.pos[(size_t)t * k + s] = pp;
            if (a.routes) {
                a.routes[(size_t)t * k + s].expert = (uint32_t)ex;
                a.routes[(size_t)t * k + s].weight = wt;
            }
        }
    }
    __syncthreads();
}

// Counts of the selections of tokens t0 .. t0 + len - 1 into cnt (LDS,
// zeroed by the caller), by an NT-thread block.
template <int NT>
__device__ inline void dispatch_count(const DispatchArgs &a, int t0, int len, int *cnt) {
    const int E = a.E, k = a.k;
    const int n = len * k;
    for (int i = threadIdx.x; i < n; i += NT) {
        const int e = a.sel[(size_t)t0 * k + i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
}

__device__ void dispatch_block(const DispatchArgs &a) {
    __shared__ int cnt[kMaxExperts];
    __shared__ int run[kMaxExperts];
    __shared__ unsigned long long bm[kDispatchWaves][kMaxExperts];
    __shared__ int wb[kDispatchWaves][kMaxExperts];
    __shared__ int wave_sums[kDispatchWaves];
    __shared__ unsigned long long s_reused, s_bytes;
    const int tid = threadIdx.x;
    const int E = a.E, T = a.T;
    for (int e = tid; e < E; e += kDispatchThreads) cnt[e] = 0;
    if (tid == 0) s_reused = 0, s_bytes = 0;
    __syncthreads();
    dispatch_count<kDispatchThreads>(a, 0, T, cnt);
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    const int o = dispatch_tables(a, c, wave_sums, &s_reused, &s_bytes);
    if (tid < E) run[tid] = o;
    __syncthreads();
    if (tid == 0) {
        a.stats[0] += (unsigned long long)T * a.k;
        a.stats[1] += s_reused;
        a.stats[2] += s_bytes;
    }
    // Stable positions, kDispatchThreads tokens per pass.
    for (int t0 = 0; t0 < T; t0 += kDispatchThreads) dispatch_place<kDispatchThreads>(a, t0, run, bm, wb);
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_kernel(DispatchArgs a) { dispatch_block(a); }

// Many tokens: chunks of dispatch_chunk_tokens(T) tokens.  Pass 1 counts each
// chunk's selections per expert; pass 2 (one block) sums them into the
// tables and gives every (chunk, expert) its first row; pass 3 places each
// chunk's tokens from there.  The rows are the same as dispatch_block's.
template <int NT>
__global__ __launch_bounds__(NT) void dispatch_count_kernel(DispatchArgs a, int32_t *chunk_cnt) {
    __shared__ int cnt[kMaxExperts];
    const int t0 = blockIdx.x * NT;
    for (int e = threadIdx.x; e < a.E; e += NT) cnt[e] = 0;
    __syncthreads();
    dispatch_count<NT>(a, t0, min(NT, a.T - t0), cnt);
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += NT) chunk_cnt[(size_t)blockIdx.x * a.E + e] = cnt[e];
}

__global__ __launch_bounds__(kDispatchThreads) void dispatch_scan_kernel(DispatchArgs a, int32_t *chunk_cnt,
                                                                         int n_chunks) {
    __shared__ int wave_sums[kDispatchWaves];
    __shared__ unsigned long long s_reused, s_bytes;
    const int tid = threadIdx.x;
    if (tid == 0) s_reused = 0, s_bytes = 0;
    __syncthreads();
    // Chunk counts are read kScanBatch at a time, all in flight together
    // (one dependent load per chunk cost a memory round trip each); the
    // first batch stays in registers for the second pass.
    constexpr int kScanBatch = 16;
    int cb[kScanBatch];
    int c = 0;
    if (tid < a.E)
        for (int ch0 = 0; ch0 < n_chunks; ch0 += kScanBatch) {
            int v[kScanBatch];
#pragma unroll
            for (int u = 0; u < kScanBatch; u++)
                v[u] = ch0 + u < n_chunks ? chunk_cnt[(size_t)(ch0 + u) * a.E + tid] : 0;
#pragma unroll
            for (int u = 0; u < kScanBatch; u++) {
                c += v[u];
                if (ch0 == 0) cb[u] = v[u];
            }
        }
    int o = dispatch_tables(a, c, wave_sums, &s_reused, &s_bytes);
    // Each chunk's first row per expert, in place of its count.
    if (tid < a.E)
        for (int ch0 = 0; ch0 < n_chunks; ch0 += kScanBatch) {
            int v[kScanBatch];
#pragma unroll
            for (int u = 0; u < kScanBatch; u++)
                v[u] = ch0 == 0 ? cb[u] : ch0 + u < n_chunks ? chunk_cnt[(size_t)(ch0 + u) * a.E + tid] : 0;
#pragma unroll
            for (int u = 0; u < kScanBatch; u++) {
                if (ch0 + u < n_chunks) chunk_cnt[(size_t)(ch0 + u) * a.E + tid] = o;
                o += v[u];
            }
        }
    __syncthreads();
    if (tid == 0) {
        a.stats[0] += (unsigned long long)a.T * a.k;
        a.stats[1] += s_reused;
        a.stats[2] += s_bytes;
    }
}

template <int NT>
__global__ __launch_bounds__(NT) void dispatch_place_kernel(DispatchArgs a, const int32_t *chunk_base) {
    __shared__ int run[kMaxExperts];
    __shared__ unsigned long long bm[NT / 64][kMaxExperts];
    __shared__ int wb[NT / 64][kMaxExperts];
    for (int e = threadIdx.x; e < a.E; e += NT) run[e] = chunk_base[(size_t)blockIdx.x * a.E + e];
    __syncthreads();
    dispatch_place<NT>(a, blockIdx.x * NT, run, bm, wb);
}

// The previous call's hit list (DispatchArgs::prev) as a wavefront holds
// it: n and entries 1 + lane + 64 m.
struct PrevLanes {
    uint32_t n;
    uint32_t v[kMaxExperts / 64];
};

__device__ inline PrevLanes prev_lanes(const DispatchArgs &a) {
    PrevLanes P;
    const int lane = threadIdx.x & 63;
    P.n = a.prev ? a.prev[0] : 0u;
#pragma unroll
    for (int m = 0; m < kMaxExperts / 64; m++) {
        const int j = lane + 64 * m;
        P.v[m] = (a.prev && j < a.E) ? a.prev[1 + j] : 0xffffffffu;
    }
    return P;
}

// An expert's entry of the one-token task table, without its h row and
// weight: what the table holds for it.
__device__ inline DecodeTask task_entry(const ExpertDev &xe) {
    DecodeTask dt{};
    dt.g = xe.m[0].ptr, dt.u = xe.m[1].ptr, dt.d = xe.m[2].ptr;
    dt.gs = xe.m[0].stride, dt.us = xe.m[1].stride, dt.ds = xe.m[2].stride;
    dt.dcols = xe.m[2].cols;
    return dt;
}

// The dispatch of a single token by one wavefront: the same outputs as
// dispatch_block for T = 1, plus the token's selection (sel, wsel) and
// shared gate, which the one-token kernel's gating leaves in LDS.  idx/w
// are the token's k selections (distinct experts) in slot order, `shg` the
// shared expert's gate (has_gate), `bits` LDS scratch for two E-bit sets.
// Its inputs come from LDS and registers, fetched before the kernel's
// acquire: `tasks` [E + 1] the experts' task_entry (a.dtasks only),
// `bytes` [E] a.expert_bytes, `P` the previous hits.  It only stores.
__device__ void dispatch_one(const DispatchArgs &a, const int *idx, const float *w, float shg, bool has_gate,
                             unsigned long long *bits, const DecodeTask *tasks, const unsigned long long *bytes_of,
                             const PrevLanes &P) {
    const int lane = threadIdx.x & 63;
    const int E = a.E, k = a.k;
    const int nw = (E + 63) / 64;
    unsigned long long *pbits = bits + kMaxExperts / 64;
    constexpr int PM = kMaxExperts / 64;

    const bool pick = lane < k;
    const int e = pick ? idx[lane] : 0;
    const float we = pick ? w[lane] : 0.0f;
    const unsigned long long eb = pick ? bytes_of[e] : 0ull;
    const bool task = pick && a.dtasks != nullptr;
    const bool stask = lane == 0 && a.dtasks != nullptr && a.has_shared;
    const uint32_t n_prev = P.n;
    // Task q of the table: expert x's entry with its h row and weight.
    auto put_task = [&](int q, int x, float *h, float wt) {
        const DecodeTask &src = tasks[x];
        DecodeTask dt;
        dt.g = src.g, dt.u = src.u, dt.d = src.d;
        dt.h = h;
        dt.gs = src.gs, dt.us = src.us, dt.ds = src.ds;
        dt.dcols = src.dcols;
        dt.w = wt;
        dt.live = 1;
        dt._pad[0] = dt._pad[1] = 0;
        a.dtasks[q] = dt;
    };

    // The selected set and the previous call's set, as bits in LDS.
    if (lane < nw) bits[lane] = pbits[lane] = 0ull;
    wave_sync();
    if (pick) atomicOr(&bits[e >> 6], 1ull << (e & 63));
#pragma unroll
    for (int m = 0; m < PM; m++) {
        const int j = lane + 64 * m;
        if (j < E && (uint32_t)j < n_prev && P.v[m] < (uint32_t)E) atomicOr(&pbits[P.v[m] >> 6], 1ull << (P.v[m] & 63));
    }
    wave_sync();
    // Selected experts before x (ascending): its permuted row, and hit slot.
    auto below = [&](int x) {
        int n = 0;
        for (int q = 0; q < (x >> 6); q++) n += __popcll(bits[q]);
        const unsigned long long msk = (x & 63) ? ((1ull << (x & 63)) - 1) : 0ull;
        return n + __popcll(bits[x >> 6] & msk);
    };
    int nsel = 0, reused = 0;
    for (int q = 0; q < nw; q++) {
        nsel += __popcll(bits[q]);
        reused += __popcll(bits[q] & pbits[q]);
    }

    // Stores.
    for (int x = lane; x < E; x += 64) {
        a.counts[x] = (int)((bits[x >> 6] >> (x & 63)) & 1ull);
        a.offsets[x] = below(x);
    }
    if (pick) {
        const int o = below(e);
        a.hits[1 + o] = e;
        if (a.hits_out) a.hits_out[1 + o] = (uint32_t)e;
        if (a.bm > 0) {
            a.tiles[4 * o] = e;
            a.tiles[4 * o + 1] = 0;
            a.tiles[4 * o + 2] = o;
            a.tiles[4 * o + 3] = 1;
        }
        if (task && o < a.dk_bound) put_task(o, e, a.h + (size_t)o * a.I, we);
        a.perm_tok[o] = 0;
        a.perm_w[o] = we;
        a.pos[lane] = o;
        const_cast<int32_t *>(a.sel)[lane] = e;
        const_cast<float *>(a.wsel)[lane] = we;
        if (a.routes) {
            a.routes[lane].expert = (uint32_t)e;
            a.routes[lane].weight = we;
        }
    }
    if (a.dtasks)
        for (int t = nsel + lane; t < a.dk_bound; t += 64) a.dtasks[t] = DecodeTask{};
    // Wave sum of the byte count.
    unsigned long long bytes = eb;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) bytes += __shfl_xor(bytes, m, 64);
    if (lane == 0) {
        a.offsets[E] = nsel;
        a.offsets[E + 1] = nsel + (a.has_shared ? 1 : 0);
        a.counts[E] = a.has_shared ? 1 : 0;
        a.hits[0] = nsel;
        if (a.hits_out) a.hits_out[0] = (uint32_t)nsel;
        if (a.bm > 0) {
            int nt = nsel;
            if (a.has_shared) {
                a.tiles[4 * nt] = E;
                a.tiles[4 * nt + 1] = 0;
                a.tiles[4 * nt + 2] = nt;
                a.tiles[4 * nt + 3] = 1;
                nt++;
            }
            a.ntiles[0] = nt;
        }
        if (has_gate && a.shgate_out) a.shgate_out[0] = shg;
        atomicAdd(a.stats + 0, (unsigned long long)k);
        atomicAdd(a.stats + 1, (unsigned long long)reused);
        atomicAdd(a.stats + 2, bytes);
        if (stask) put_task(a.dk_bound, E, a.hs, a.shgate ? shg : 1.0f);
    }
}

// ------------------------------------------------------------ one token
//
// Router, gating and dispatch of a single token in one launch.  Block r
// computes logit r: dot_avx2's 16 lane chains (chain j sums elements j,
// j + 16, ... with fma, in order), then its lane reduction and scalar tail.
// The block stages its router row and x into LDS transposed: chain j's
// elements contiguous in row j, rows one_pitch(H) floats apart (= 4 mod 64,
// so the 16 chains' 16-byte reads, and the staging writes, fall in distinct
// banks); the elements past the last full 16 follow both arrays as they
// are.  Each chain then reads four steps per LDS access, one batch ahead.
// The last block to finish, counted with one device atomic after a release
// fence, gates the token and dispatches it.  The counter is returned to zero
// by that block, and no block waits on another.
//
// The acquire that follows the count invalidates the caches, so every load
// after it comes from memory, one dependent round trip at a time.  Every
// block therefore fetches what the gating and dispatch read besides the
// logits before its count, together with its operands: wave 0 the gating
// constants and the previous hits (registers), thread e expert e's task
// entry and byte count (LDS, after the operands).
__host__ __device__ inline int one_pitch(int H) {
    const int n16 = H >> 4;
    return n16 <= 4 ? 4 : 4 + 64 * ((n16 - 4 + 63) / 64);
}
inline size_t one_lds_bytes(int H, int E, bool tasks) {
    return ((size_t)32 * one_pitch(H) + 32) * sizeof(float) + (tasks ? (size_t)(E + 1) * sizeof(DecodeTask) : 0) +
           (size_t)E * sizeof(unsigned long long);
}

// Element i of an operand into the transposed layout.
__device__ inline void one_put(float *t, float *tail, int P, int n16, int i, float v) {
    if (i < 16 * n16)
        t[(i & 15) * P + (i >> 4)] = v;
    else
        tail[i - 16 * n16] = v;
}

template <int EPL>
__global__ __launch_bounds__(kDispatchThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void route_one_kernel(const float *__restrict__ W,
                                                                     const float *__restrict__ x, int n_rows, int E,
                                                                     int H, float temp, float *__restrict__ logits,
                                                                     GateParams p, DispatchArgs d,
                                                                     unsigned *__restrict__ counter) {
    // [16][P] row, [16][P] x, 16 + 16 tail, [E + 1] task entries (d.dtasks), [E] byte counts
    extern __shared__ __align__(16) float lds[];
    __shared__ GateScratch<EPL> S;
    __shared__ int s_last;
    const int r = blockIdx.x;
    const int n16 = H >> 4, P = one_pitch(H);
    float *ta = lds, *tb = lds + 16 * P, *tail_a = lds + 32 * P, *tail_b = tail_a + 16;
    DecodeTask *ltask = reinterpret_cast<DecodeTask *>(lds + 32 * P + 32);
    unsigned long long *lbytes = reinterpret_cast<unsigned long long *>(d.dtasks ? ltask + E + 1 : ltask);
    const float *wr = W + (size_t)r * H;
    const int tid = threadIdx.x, nt = blockDim.x;
    // The layer's constants for the last block (requested before the
    // operands, stored after them).
    GateConst<EPL> G{};
    PrevLanes Pv{};
    if (tid < 64) {
        G = gate_const<EPL>(p);
        Pv = prev_lanes(d);
    }
    auto has_task = [&](int e) { return d.dtasks != nullptr && (e < E || (e == E && d.has_shared)); };
    DecodeTask te{};
    unsigned long long tbytes = 0;
    if (tid < E) tbytes = d.expert_bytes[tid];
    if (has_task(tid)) te = task_entry(d.experts[tid]);
    if ((H & 3) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0) {
        // Four float4 of each operand in flight per thread before its stores;
        // indices past the end re-read the last vector and store nothing.
        const float4 *a4 = reinterpret_cast<const float4 *>(wr), *b4 = reinterpret_cast<const float4 *>(x);
        const int n4 = H >> 2;
        for (int base = 0; base < n4; base += 4 * nt) {
            float4 va[4], vb[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = base + u * nt + tid, ic = i < n4 ? i : n4 - 1;
                va[u] = a4[ic];
                vb[u] = b4[ic];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = base + u * nt + tid;
                if (i < n4) {
                    one_put(ta, tail_a, P, n16, 4 * i, va[u].x);
                    one_put(ta, tail_a, P, n16, 4 * i + 1, va[u].y);
                    one_put(ta, tail_a, P, n16, 4 * i + 2, va[u].z);
                    one_put(ta, tail_a, P, n16, 4 * i + 3, va[u].w);
                    one_put(tb, tail_b, P, n16, 4 * i, vb[u].x);
                    one_put(tb, tail_b, P, n16, 4 * i + 1, vb[u].y);
                    one_put(tb, tail_b, P, n16, 4 * i + 2, vb[u].z);
                    one_put(tb, tail_b, P, n16, 4 * i + 3, vb[u].w);
                }
            }
        }
    } else {
        for (int i = tid; i < H; i += nt) {
            const float va = wr[i], vb = x[i];
            one_put(ta, tail_a, P, n16, i, va);
            one_put(tb, tail_b, P, n16, i, vb);
        }
    }
    if (tid < E) lbytes[tid] = tbytes;
    if (has_task(tid)) ltask[tid] = te;
    for (int e = tid + nt; e <= E; e += nt) {  // E + 1 > blockDim.x
        if (e < E) lbytes[e] = d.expert_bytes[e];
        if (has_task(e)) ltask[e] = task_entry(d.experts[e]);
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int j = threadIdx.x;
        const float4 *pa = reinterpret_cast<const float4 *>(ta + j * P);
        const float4 *pb = reinterpret_cast<const float4 *>(tb + j * P);
        const int nq = n16 >> 2;  // full quads of steps
        float acc = 0.0f;
        if (nq > 0) {
            // Batches of four quads; the next batch's reads are issued before
            // this batch's fmas.  Reads past the last quad re-read it.
            float4 a0[4], b0[4], a1[4], b1[4];
            auto ld = [&](int q, float4(&av)[4], float4(&bv)[4]) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int qi = q + u < nq ? q + u : nq - 1;
                    av[u] = pa[qi];
                    bv[u] = pb[qi];
                }
            };
            auto mac = [&](int q, const float4(&av)[4], const float4(&bv)[4]) {
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (q + u < nq) {
                        acc = fmaf(av[u].x, bv[u].x, acc);
                        acc = fmaf(av[u].y, bv[u].y, acc);
                        acc = fmaf(av[u].z, bv[u].z, acc);
                        acc = fmaf(av[u].w, bv[u].w, acc);
                    }
            };
            ld(0, a0, b0);
            for (int q = 0; q < nq; q += 8) {
                ld(q + 4, a1, b1);
                mac(q, a0, b0);
                ld(q + 8, a0, b0);
                mac(q + 4, a1, b1);
            }
        }
        for (int c = 4 * nq; c < n16; c++) acc = fmaf(ta[j * P + c], tb[j * P + c], acc);
        const int rem = H - 16 * n16;
        if (rem >= 8 && j < 8) acc = fmaf(tail_a[j], tail_b[j], acc);
        float v = reduce16_avx2(acc);
        if (j == 0) {
            v = dot_tail(v, tail_a, tail_b, rem >= 8 ? 8 : 0, rem);
            if (temp > 0.0f && r < E) v = v / temp;
            logits[r] = v;
        }
    }
    // Thread 0 wrote the logit: it releases it with the count, and in the
    // last block acquires the others' before the barrier hands them on.
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last = atomicAdd(counter, 1u) == (unsigned)(gridDim.x - 1);
        if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        s_last = last;
    }
    __syncthreads();
    if (!s_last || threadIdx.x >= 64) return;
    // The last block's first wavefront gates and dispatches the token; the
    // selection's stores wait for the dispatch's loads (dispatch_one).
    __shared__ unsigned long long bits[2 * (kMaxExperts / 64)];
    gate_token<EPL, false>(logits, 0, p, G, S, nullptr, nullptr, nullptr, d.stats);
    wave_sync();
    dispatch_one(d, S.idx, S.w, S.shg, p.has_shared_gate != 0, bits, ltask, lbytes, Pv);
    if (threadIdx.x == 0) *counter = 0u;
}

__global__ void expf_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) y[i] = expf_exact(x[i]);
}

}  // namespace

hipError_t launch_router(const float *W, const float *x, int T, int n_rows, int E, int H, float temp, float *logits,
                         hipStream_t s) {
    const double budget = 160.0 * 1024;
    const double clk_us = 2400.0;  // cycles per microsecond
    // Cost model (microseconds) of the row-staging kernel for an RB x TB
    // tile: per round of resident blocks, one memory round trip (~1 us) per
    // 16 float4 per thread, the staged bytes through each CU at ~64 B per
    // cycle, and the H/16-step chain at ~10 cycles per step.
    // PPT pairs per thread (RB TB <= 16 PPT): interleaved chains, assumed
    // to cost (1 + (PPT - 1) / 2) times one chain.
    int best_rb = 0, best_tb = 0, best_ppt = 1;
    double best = 1e30;
    for (int ppt = 1; ppt <= 4; ppt *= 2)
        for (int RB = 1; RB <= 16 * ppt && RB < 2 * n_rows; RB *= 2)
            for (int TB = 1; RB * TB <= 16 * ppt && TB < 2 * T; TB *= 2) {
                if (ppt > 1 && RB * TB <= 8 * ppt) continue;  // fits fewer pairs per thread
                const double lds = (RB + TB) * (double)router_lds_stride(H) * 4;
                if (lds > budget) continue;
                const long long blocks = (long long)((n_rows + RB - 1) / RB) * ((T + TB - 1) / TB);
                int per_cu = (int)(budget / lds);
                if (per_cu > 8) per_cu = 8;
                const double rounds = std::ceil((double)blocks / (256.0 * per_cu));
                const double trips = std::ceil((double)std::max(RB, TB) * H / 4 / (16 * 256));
                const double chain = (H / 16) * 10.0 / clk_us * (1.0 + 0.5 * (ppt - 1));
                const double t = rounds * (trips + per_cu * lds / 64.0 / clk_us + chain);
                if (t < best) best = t, best_rb = RB, best_tb = TB, best_ppt = ppt;
            }
    // The tiled kernel: 32 rows x 4 TPT tokens, TPT = 8 unless that leaves
    // fewer than three blocks per CU (latency then shows: 32 x 32 tiles at
    // one block per CU ran 4.5x slower than their FMA count); ~1150 cycles
    // per 64-value K chunk at TPT = 8.
    auto tiles_of = [&](int tpt) { return (double)((n_rows + kRT - 1) / kRT) * ((T + 4 * tpt - 1) / (4 * tpt)); };
    const int tpt = tiles_of(8) >= 3 * 256 ? 8 : tiles_of(4) >= 3 * 256 ? 4 : tiles_of(2) >= 3 * 256 ? 2 : 1;
    const double tiled = std::ceil(tiles_of(8) / (256.0 * 3)) * (H / 64.0) * 1150.0 / clk_us;
    if (best_rb > 0 && best <= tiled) {
        const int RB = best_rb, TB = best_tb;
        dim3 grid((n_rows + RB - 1) / RB, (T + TB - 1) / TB);
        const size_t lds = (size_t)(RB + TB) * router_lds_stride(H) * 4;
        static bool raised = false;
        if (!raised) {
            (void)hipFuncSetAttribute((const void *)router_lds_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      160 * 1024);
            (void)hipFuncSetAttribute((const void *)router_lds_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      160 * 1024);
            (void)hipFuncSetAttribute((const void *)router_lds_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      160 * 1024);
            raised = true;
        }
        if (best_ppt == 4)
            hipLaunchKernelGGL(router_lds_kernel<4>, grid, dim3(256), lds, s, W, x, T, n_rows, E, H, RB, TB, temp, logits);
        else if (best_ppt == 2)
            hipLaunchKernelGGL(router_lds_kernel<2>, grid, dim3(256), lds, s, W, x, T, n_rows, E, H, RB, TB, temp, logits);
        else
            hipLaunchKernelGGL(router_lds_kernel<1>, grid, dim3(256), lds, s, W, x, T, n_rows, E, H, RB, TB, temp, logits);
    } else {
        dim3 grid((n_rows + kRT - 1) / kRT, (T + 4 * tpt - 1) / (4 * tpt));
        if ((H & 3) != 0 || H < 16) {
            // Rows of a length that is not a multiple of 4, or shorter than
            // 16: scalar loads.
            dim3 g1((n_rows + kRT - 1) / kRT, (T + 3) / 4);
            hipLaunchKernelGGL((router_tiled_kernel<1, false>), g1, dim3(256), 0, s, W, x, T, n_rows, E, H, temp, logits);
        } else if (tpt == 8) {
            hipLaunchKernelGGL((router_tiled_kernel<8, true>), grid, dim3(256), 0, s, W, x, T, n_rows, E, H, temp, logits);
        } else if (tpt == 4) {
            hipLaunchKernelGGL((router_tiled_kernel<4, true>), grid, dim3(256), 0, s, W, x, T, n_rows, E, H, temp, logits);
        } else if (tpt == 2) {
            hipLaunchKernelGGL((router_tiled_kernel<2, true>), grid, dim3(256), 0, s, W, x, T, n_rows, E, H, temp, logits);
        } else {
            hipLaunchKernelGGL((router_tiled_kernel<1, true>), grid, dim3(256), 0, s, W, x, T, n_rows, E, H, temp, logits);
        }
    }
    return hipGetLastError();
}

hipError_t launch_gating(const float *logits, int ld, int T, const GateParams &p, int32_t *sel, float *wsel,
                         float *shgate, unsigned long long *stats, hipStream_t s) {
    dim3 grid((T + 3) / 4);
    if (p.n_experts <= 64)
        hipLaunchKernelGGL(gating_kernel<1>, grid, dim3(256), 0, s, logits, ld, T, p, sel, wsel, shgate, stats);
    else if (p.n_experts <= 128)
        hipLaunchKernelGGL(gating_kernel<2>, grid, dim3(256), 0, s, logits, ld, T, p, sel, wsel, shgate, stats);
    else if (p.n_experts <= 256)
        hipLaunchKernelGGL(gating_kernel<4>, grid, dim3(256), 0, s, logits, ld, T, p, sel, wsel, shgate, stats);
    else
        hipLaunchKernelGGL(gating_kernel<8>, grid, dim3(256), 0, s, logits, ld, T, p, sel, wsel, shgate, stats);
    return hipGetLastError();
}

// The transposed operands and the prefetched tables take one_lds_bytes:
// 76 KiB at H = 7168, E = 256.  Up to 64 KiB needs no attribute; beyond,
// the launch raises the kernel's limit (the block's static LDS is under
// 16 KiB of the CU's 160 KiB).
bool route_one_ok(int H, int E) { return H > 0 && E > 0 && one_lds_bytes(H, E, true) <= 144 * 1024; }

hipError_t launch_route_one(const float *W, const float *x, int n_rows, int E, int H, float temp, float *logits,
                            const GateParams &p, const DispatchArgs &d, unsigned *counter, hipStream_t s) {
    if (!route_one_ok(H, E)) return hipErrorInvalidValue;
    const size_t lds = one_lds_bytes(H, E, d.dtasks != nullptr);
    auto go = [&](auto kern) {
        if (lds > 64 * 1024) {
            const hipError_t e =
                hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3(n_rows), dim3(kDispatchThreads), lds, s, W, x, n_rows, E, H, temp, logits, p,
                           d, counter);
        return hipGetLastError();
    };
    if (p.n_experts <= 64) return go(route_one_kernel<1>);
    if (p.n_experts <= 128) return go(route_one_kernel<2>);
    if (p.n_experts <= 256) return go(route_one_kernel<4>);
    return go(route_one_kernel<8>);
}

int dispatch_chunk_tokens(int T) { return T <= kSmallChunkMaxT ? kChunkTokens : kDispatchThreads; }
int dispatch_chunks(int T) {
    const int c = dispatch_chunk_tokens(T);
    return T > kDispatchThreads ? (T + c - 1) / c : 0;
}

int dispatch_chunks_upto(int T) {
    return std::max(dispatch_chunks(std::min(T, kSmallChunkMaxT)), dispatch_chunks(T));
}

hipError_t launch_dispatch(const DispatchArgs &a, int32_t *chunk_scratch, size_t chunk_cap, hipStream_t s) {
    const int nc = dispatch_chunks(a.T);
    if (nc > 0 && chunk_scratch && (size_t)nc * a.E > chunk_cap) return hipErrorInvalidValue;
    if (nc == 0 || !chunk_scratch) {
        hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(kDispatchThreads), 0, s, a);
        return hipGetLastError();
    }
    if (dispatch_chunk_tokens(a.T) == kChunkTokens) {
        hipLaunchKernelGGL(dispatch_count_kernel<kChunkTokens>, dim3(nc), dim3(kChunkTokens), 0, s, a, chunk_scratch);
        hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(kDispatchThreads), 0, s, a, chunk_scratch, nc);
        hipLaunchKernelGGL(dispatch_place_kernel<kChunkTokens>, dim3(nc), dim3(kChunkTokens), 0, s, a, chunk_scratch);
    } else {
        hipLaunchKernelGGL(dispatch_count_kernel<kDispatchThreads>, dim3(nc), dim3(kDispatchThreads), 0, s, a,
                           chunk_scratch);
        hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(kDispatchThreads), 0, s, a, chunk_scratch, nc);
        hipLaunchKernelGGL(dispatch_place_kernel<kDispatchThreads>, dim3(nc), dim3(kDispatchThreads), 0, s, a,
                           chunk_scratch);
    }
    return hipGetLastError();
}

hipError_t launch_expf(const float *x, float *y, size_t n, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(expf_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

}  // namespace moe
